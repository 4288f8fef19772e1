// Inject path: re-RoPE of staged pre-RoPE cold-tier keys back to their
// original positions, fused with the held-slot replacement in the hot buffer.
//
// Replaces _rotate_k_with_pos / _rope_cos_sin_for_positions
// (src/hotcold_kv/patch.py:76-102), which build cos/sin through the model's
// rotary module and apply HF apply_rotary_pos_emb, and the held-slot update
// plus torch.cat of patch.py:241-270.  The staged fp32 rows are read once,
// converted to the cache dtype, rotated and written straight into rows
// 0..R-1 of the fixed-capacity hot buffer (no per-step concatenation).
//
// Arithmetic follows the reference's per-op rounding:
//   f   = fp32(fp32(pos) * inv_freq[i])          (inv_freq @ pos, K = 1)
//   c,s = dtype(fp32(cos/sin(f)) * fp32(scaling))
//   k'  = dtype(dtype(k*c) + dtype(rotate_half(k)*s))   in fp32 then rounded
// cos/sin of the fp32 angle are evaluated in fp64 and rounded to fp32.
#include "hc_common.h"

namespace hc {

template <typename T>
__global__ void inject_rerope_kernel(const float* __restrict__ kp, int64_t kp_sb, int64_t kp_sh, int64_t kp_ss,
                                     const float* __restrict__ vp, int64_t vp_sb, int64_t vp_sh, int64_t vp_ss,
                                     const int64_t* __restrict__ pos, int64_t pos_sb, int64_t pos_sh,
                                     const float* __restrict__ inv_freq, float scaling, int D,
                                     T* __restrict__ kd, int64_t kd_sb, int64_t kd_sh, int64_t kd_ss,
                                     T* __restrict__ vd, int64_t vd_sb, int64_t vd_sh, int64_t vd_ss) {
#pragma clang fp contract(off)
  const int r = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int half = D / 2;
  const float* krow = kp + b * kp_sb + h * kp_sh + (int64_t)r * kp_ss;
  const float* vrow = vp + b * vp_sb + h * vp_sh + (int64_t)r * vp_ss;
  T* kout = kd + b * kd_sb + h * kd_sh + (int64_t)r * kd_ss;
  T* vout = vd + b * vd_sb + h * vd_sh + (int64_t)r * vd_ss;
  const float fpos = (float)pos[b * pos_sb + h * pos_sh + r];
  for (int i = threadIdx.x; i < half; i += blockDim.x) {
    const float f = fpos * inv_freq[i];
    double sd, cd;
    sincos((double)f, &sd, &cd);  // one shared argument reduction
    const float cf = (float)cd * scaling;
    const float sf = (float)sd * scaling;
    const float c = to_f32(from_f32<T>(cf));
    const float s = to_f32(from_f32<T>(sf));
    const float ka = to_f32(from_f32<T>(krow[i]));
    const float kb = to_f32(from_f32<T>(krow[i + half]));
    const float a1 = to_f32(from_f32<T>(ka * c));
    const float a2 = to_f32(from_f32<T>((-kb) * s));
    const float b1 = to_f32(from_f32<T>(kb * c));
    const float b2 = to_f32(from_f32<T>(ka * s));
    kout[i] = from_f32<T>(a1 + a2);
    kout[i + half] = from_f32<T>(b1 + b2);
    vout[i] = from_f32<T>(vrow[i]);
    vout[i + half] = from_f32<T>(vrow[i + half]);
  }
}

// Vector form with cos/sin supplied (the model's rotary tables at the held
// positions, already rounded to the cache dtype, as apply_rotary_pos_emb
// receives them): every element is then the reference's bits.  A thread
// takes four dims of each half of one row -- 4-wide loads of the staged K
// and V (fp32, or already in the cache dtype), one 4-wide load of cos and of
// sin -- so D/8 threads cover a row and a 256-thread workgroup 2048/D rows.
// Rows run (b, h, r) with r fastest; a table shared by the KV heads of a
// batch row has cs_sh = 0.
struct InjectTab {
  const void* kp;
  int64_t kp_sb, kp_sh, kp_ss;
  const void* vp;
  int64_t vp_sb, vp_sh, vp_ss;
  const void* cs_cos;
  const void* cs_sin;
  int64_t cs_sb, cs_sh, cs_ss;
  void* kd;
  int64_t kd_sb, kd_sh, kd_ss;
  void* vd;
  int64_t vd_sb, vd_sh, vd_ss;
  int64_t rows;
  int Hk, R, D;
};

template <typename T>
struct Vec4;
template <>
struct Vec4<float> {
  typedef floatx4 type;
  __device__ static floatx4 load(const float* p) { return *reinterpret_cast<const floatx4*>(p); }
  __device__ static float get(const floatx4& x, int j) { return x[j]; }
  __device__ static void store(float* p, const float (&x)[4]) {
    *reinterpret_cast<floatx4*>(p) = floatx4{x[0], x[1], x[2], x[3]};
  }
};
template <typename T>
struct Vec4 {  // 2-byte types: four values in 8 bytes
  typedef u32x2 type;
  __device__ static u32x2 load(const T* p) { return *reinterpret_cast<const u32x2*>(p); }
  __device__ static float get(const u32x2& x, int j) {
    const uint32_t w = x[j >> 1];
    return to_f32(__builtin_bit_cast(T, (uint16_t)((j & 1) ? (w >> 16) : (w & 0xffffu))));
  }
  __device__ static void store(T* p, const float (&x)[4]) {
    uint32_t w[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
      w[j] = (uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(x[2 * j])) |
             ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(x[2 * j + 1])) << 16);
    *reinterpret_cast<u32x2*>(p) = u32x2{w[0], w[1]};
  }
};

// T: the cache dtype; KT: the staged rows' type (float, or T itself -- the
// keys are rounded to T before the rotation either way).
template <typename T, typename KT>
__global__ __launch_bounds__(256) void inject_rerope_tab_kernel(InjectTab a) {
#pragma clang fp contract(off)
  const int half = a.D / 2;
  const int tpr = half / 4;  // threads per row
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = t / tpr;
  if (row >= a.rows) return;
  const int i = (int)(t - row * tpr) * 4;
  const int r = (int)(row % a.R);
  const int64_t bh = row / a.R;
  const int h = (int)(bh % a.Hk);
  const int b = (int)(bh / a.Hk);
  const KT* krow = reinterpret_cast<const KT*>(a.kp) + b * a.kp_sb + h * a.kp_sh + (int64_t)r * a.kp_ss;
  const KT* vrow = reinterpret_cast<const KT*>(a.vp) + b * a.vp_sb + h * a.vp_sh + (int64_t)r * a.vp_ss;
  const int64_t cso = b * a.cs_sb + h * a.cs_sh + (int64_t)r * a.cs_ss + i;
  const typename Vec4<KT>::type k0 = Vec4<KT>::load(krow + i), k1 = Vec4<KT>::load(krow + half + i);
  const typename Vec4<KT>::type v0 = Vec4<KT>::load(vrow + i), v1 = Vec4<KT>::load(vrow + half + i);
  const typename Vec4<T>::type cv = Vec4<T>::load(reinterpret_cast<const T*>(a.cs_cos) + cso);
  const typename Vec4<T>::type sv = Vec4<T>::load(reinterpret_cast<const T*>(a.cs_sin) + cso);
  float o0[4], o1[4], w0[4], w1[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float c = Vec4<T>::get(cv, j), s = Vec4<T>::get(sv, j);
    const float ka = to_f32(from_f32<T>(Vec4<KT>::get(k0, j))), kb = to_f32(from_f32<T>(Vec4<KT>::get(k1, j)));
    // (k * cos) + (rotate_half(k) * sin), each op rounded to T
    const float a1 = to_f32(from_f32<T>(ka * c));
    const float a2 = to_f32(from_f32<T>((-kb) * s));
    const float b1 = to_f32(from_f32<T>(kb * c));
    const float b2 = to_f32(from_f32<T>(ka * s));
    o0[j] = a1 + a2;
    o1[j] = b1 + b2;
    w0[j] = Vec4<KT>::get(v0, j);
    w1[j] = Vec4<KT>::get(v1, j);
  }
  T* kout = reinterpret_cast<T*>(a.kd) + b * a.kd_sb + h * a.kd_sh + (int64_t)r * a.kd_ss;
  T* vout = reinterpret_cast<T*>(a.vd) + b * a.vd_sb + h * a.vd_sh + (int64_t)r * a.vd_ss;
  Vec4<T>::store(kout + i, o0);
  Vec4<T>::store(kout + half + i, o1);
  Vec4<T>::store(vout + i, w0);
  Vec4<T>::store(vout + half + i, w1);
}

// Pooled retrieval query: out[b][vh][d] = (sum over the window's T query
// tensors, then over the heads of KV head vh's group -- or over all Hq heads
// when there is one vector per batch row -- of q[b][h][d]) / (T * heads), in
// fp32 with the additions in that fixed order.  Up to kMaxPoolRows window
// rows (hc_retrieval_query_max_rows; the host pools longer windows itself).
constexpr int kMaxPoolRows = 64;
struct PoolQueryArgs {
  const void* q[kMaxPoolRows];
  int64_t sb[kMaxPoolRows];
  int64_t sh[kMaxPoolRows];
  int T, Hq, G, D, per_head;
  float* out;
};

template <typename T>
__global__ void pool_query_kernel(PoolQueryArgs a) {
#pragma clang fp contract(off)
  const int b = blockIdx.x, vh = blockIdx.y, nvh = gridDim.y;
  const int h0 = a.per_head ? vh * a.G : 0, nh = a.per_head ? a.G : a.Hq;
  const float inv = 1.0f / (float)(a.T * nh);
  for (int d = threadIdx.x; d < a.D; d += blockDim.x) {
    float acc = 0.0f;
    // the window rows by constant index (a runtime index into the argument
    // arrays would copy them to scratch); 8 head loads in flight per batch,
    // then their adds in order
#pragma unroll
    for (int t = 0; t < kMaxPoolRows; ++t) {
      if (t < a.T) {
        const T* q = reinterpret_cast<const T*>(a.q[t]) + b * a.sb[t] + d;
        const int64_t sh = a.sh[t];
        for (int hb = 0; hb < nh; hb += 8) {
          float v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) v[u] = hb + u < nh ? to_f32(q[(int64_t)(h0 + min(hb + u, nh - 1)) * sh]) : 0.0f;
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (hb + u < nh) acc += v[u];
        }
      }
    }
    a.out[((int64_t)b * nvh + vh) * a.D + d] = acc * inv;
  }
}

}  // namespace hc

using namespace hc;

extern "C" int64_t hc_retrieval_query_max_rows(void) { return kMaxPoolRows; }

extern "C" int hc_retrieval_query(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t T,
                                  const void* const* q, const int64_t* q_sb, const int64_t* q_sh, int per_head,
                                  float* dev_out, float* host_out, void* event, void* stream) {
  HC_REQUIRE(dtype == HC_DTYPE_F32 || dtype == HC_DTYPE_F16 || dtype == HC_DTYPE_BF16, "retrieval_query: bad dtype");
  HC_REQUIRE(B > 0 && Hq > 0 && Hk > 0 && D > 0 && T > 0 && Hq % Hk == 0, "retrieval_query: bad shape");
  HC_REQUIRE(T <= kMaxPoolRows, "retrieval_query: at most %d window rows", kMaxPoolRows);
  HC_REQUIRE(B <= 65535 && Hk <= 65535, "retrieval_query: B or Hk too large for the grid");
  HC_REQUIRE(q && q_sb && q_sh && dev_out, "retrieval_query: null pointer");
  PoolQueryArgs a{};
  for (int64_t t = 0; t < T; ++t) {
    HC_REQUIRE(q[t] != nullptr, "retrieval_query: null query row %lld", (long long)t);
    a.q[t] = q[t];
    a.sb[t] = q_sb[t];
    a.sh[t] = q_sh[t];
  }
  a.T = (int)T; a.Hq = (int)Hq; a.G = (int)(Hq / Hk); a.D = (int)D; a.per_head = per_head ? 1 : 0;
  a.out = dev_out;
  const int nvh = per_head ? (int)Hk : 1;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)B, (unsigned)nvh);
  const int threads = D >= 256 ? 256 : (D >= 128 ? 128 : 64);
  if (dtype == HC_DTYPE_F16) hipLaunchKernelGGL(pool_query_kernel<half_t>, grid, dim3(threads), 0, st, a);
  else if (dtype == HC_DTYPE_BF16) hipLaunchKernelGGL(pool_query_kernel<bf16_t>, grid, dim3(threads), 0, st, a);
  else hipLaunchKernelGGL(pool_query_kernel<float>, grid, dim3(threads), 0, st, a);
  int rc = check_launch("pool_query");
  if (rc != HC_OK) return rc;
  if (host_out) {
    const hipError_t e = hipMemcpyAsync(host_out, dev_out, sizeof(float) * B * nvh * D, hipMemcpyDeviceToHost, st);
    if (e != hipSuccess) return set_error(HC_ERR_HIP, "retrieval_query: hipMemcpyAsync: %s", hipGetErrorString(e));
  }
  if (event) {
    const hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(event), st);
    if (e != hipSuccess) return set_error(HC_ERR_HIP, "retrieval_query: hipEventRecord: %s", hipGetErrorString(e));
  }
  return HC_OK;
}

extern "C" int hc_inject_rerope_tab(int dtype, int64_t B, int64_t Hk, int64_t R, int64_t D, int kv_dtype,
                                    const void* k_pre, int64_t kp_sb, int64_t kp_sh, int64_t kp_ss, const void* v,
                                    int64_t vp_sb, int64_t vp_sh, int64_t vp_ss, const void* cos_t, const void* sin_t,
                                    int64_t cs_sb, int64_t cs_sh, int64_t cs_ss, void* k_dst, int64_t kd_sb,
                                    int64_t kd_sh, int64_t kd_ss, void* v_dst, int64_t vd_sb, int64_t vd_sh,
                                    int64_t vd_ss, void* stream) {
  HC_REQUIRE(dtype == HC_DTYPE_F32 || dtype == HC_DTYPE_F16 || dtype == HC_DTYPE_BF16, "inject_tab: bad dtype %d",
             dtype);
  HC_REQUIRE(kv_dtype == HC_DTYPE_F32 || kv_dtype == dtype,
             "inject_tab: staged k_pre / v must be fp32 or the cache dtype (%d, cache %d)", kv_dtype, dtype);
  HC_REQUIRE(B > 0 && Hk > 0 && R >= 0 && D > 0, "inject_tab: bad shape");
  HC_REQUIRE(D % 8 == 0, "inject_tab: head_dim %lld must be a multiple of 8", (long long)D);
  if (R == 0) return HC_OK;
  HC_REQUIRE(k_pre && v && cos_t && sin_t && k_dst && v_dst, "inject_tab: null pointer");
  const int es = dtype_size(dtype), kes = dtype_size(kv_dtype);
  const auto al = [](const void* p, int n) { return ((uintptr_t)p % n) == 0; };
  // 4-element pieces of the staged rows, the tables and the outputs
  HC_REQUIRE(al(k_pre, 4 * kes) && al(v, 4 * kes) && kp_sb % 4 == 0 && kp_sh % 4 == 0 && kp_ss % 4 == 0 &&
                 vp_sb % 4 == 0 && vp_sh % 4 == 0 && vp_ss % 4 == 0,
             "inject_tab: staged k_pre / v rows must be aligned to 4 elements");
  HC_REQUIRE(al(cos_t, 4 * es) && al(sin_t, 4 * es) && cs_sb % 4 == 0 && cs_sh % 4 == 0 && cs_ss % 4 == 0 &&
                 al(k_dst, 4 * es) && al(v_dst, 4 * es) && kd_sb % 4 == 0 && kd_sh % 4 == 0 && kd_ss % 4 == 0 &&
                 vd_sb % 4 == 0 && vd_sh % 4 == 0 && vd_ss % 4 == 0,
             "inject_tab: cos/sin tables and destination rows must be aligned to 4 elements");
  InjectTab a;
  a.kp = k_pre; a.kp_sb = kp_sb; a.kp_sh = kp_sh; a.kp_ss = kp_ss;
  a.vp = v; a.vp_sb = vp_sb; a.vp_sh = vp_sh; a.vp_ss = vp_ss;
  a.cs_cos = cos_t; a.cs_sin = sin_t; a.cs_sb = cs_sb; a.cs_sh = cs_sh; a.cs_ss = cs_ss;
  a.kd = k_dst; a.kd_sb = kd_sb; a.kd_sh = kd_sh; a.kd_ss = kd_ss;
  a.vd = v_dst; a.vd_sb = vd_sb; a.vd_sh = vd_sh; a.vd_ss = vd_ss;
  a.rows = B * Hk * R;
  a.Hk = (int)Hk; a.R = (int)R; a.D = (int)D;
  const int64_t threads = a.rows * (D / 8);
  HC_REQUIRE(cdiv(threads, (int64_t)256) <= 0x7fffffff, "inject_tab: grid too large");
  const dim3 grid((unsigned)cdiv(threads, (int64_t)256));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool f32 = kv_dtype == HC_DTYPE_F32;
  if (dtype == HC_DTYPE_F16) {
    if (f32) hipLaunchKernelGGL((inject_rerope_tab_kernel<half_t, float>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((inject_rerope_tab_kernel<half_t, half_t>), grid, dim3(256), 0, st, a);
  } else if (dtype == HC_DTYPE_BF16) {
    if (f32) hipLaunchKernelGGL((inject_rerope_tab_kernel<bf16_t, float>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((inject_rerope_tab_kernel<bf16_t, bf16_t>), grid, dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL((inject_rerope_tab_kernel<float, float>), grid, dim3(256), 0, st, a);
  }
  return check_launch("inject_rerope_tab");
}

extern "C" int hc_inject_rerope(int dtype, int64_t B, int64_t Hk, int64_t R, int64_t D, const float* k_pre,
                                int64_t kp_sb, int64_t kp_sh, int64_t kp_ss, const float* v, int64_t vp_sb,
                                int64_t vp_sh, int64_t vp_ss, const int64_t* pos, int64_t pos_sb, int64_t pos_sh,
                                const float* inv_freq, double attention_scaling, void* k_dst, int64_t kd_sb,
                                int64_t kd_sh, int64_t kd_ss, void* v_dst, int64_t vd_sb, int64_t vd_sh, int64_t vd_ss,
                                void* stream) {
  HC_REQUIRE(dtype == HC_DTYPE_F32 || dtype == HC_DTYPE_F16 || dtype == HC_DTYPE_BF16, "inject: bad dtype %d", dtype);
  HC_REQUIRE(B > 0 && Hk > 0 && R >= 0 && D > 0, "inject: bad shape");
  HC_REQUIRE(D % 2 == 0, "inject: head_dim must be even");
  HC_REQUIRE(B <= 65535 && Hk <= 65535 && R <= 0x7fffffff, "inject: grid too large");
  if (R == 0) return HC_OK;
  HC_REQUIRE(k_pre && v && pos && inv_freq && k_dst && v_dst, "inject: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)R, (unsigned)Hk, (unsigned)B);
  const int threads = (int)(D / 2 < 64 ? 64 : (D / 2 > 256 ? 256 : D / 2));
  const float sc = (float)attention_scaling;
  if (dtype == HC_DTYPE_F16)
    hipLaunchKernelGGL(inject_rerope_kernel<half_t>, grid, dim3(threads), 0, st, k_pre, kp_sb, kp_sh, kp_ss, v, vp_sb,
                       vp_sh, vp_ss, pos, pos_sb, pos_sh, inv_freq, sc, (int)D, (half_t*)k_dst, kd_sb, kd_sh, kd_ss,
                       (half_t*)v_dst, vd_sb, vd_sh, vd_ss);
  else if (dtype == HC_DTYPE_BF16)
    hipLaunchKernelGGL(inject_rerope_kernel<bf16_t>, grid, dim3(threads), 0, st, k_pre, kp_sb, kp_sh, kp_ss, v, vp_sb,
                       vp_sh, vp_ss, pos, pos_sb, pos_sh, inv_freq, sc, (int)D, (bf16_t*)k_dst, kd_sb, kd_sh, kd_ss,
                       (bf16_t*)v_dst, vd_sb, vd_sh, vd_ss);
  else
    hipLaunchKernelGGL(inject_rerope_kernel<float>, grid, dim3(threads), 0, st, k_pre, kp_sb, kp_sh, kp_ss, v, vp_sb,
                       vp_sh, vp_ss, pos, pos_sb, pos_sh, inv_freq, sc, (int)D, (float*)k_dst, kd_sb, kd_sh, kd_ss,
                       (float*)v_dst, vd_sb, vd_sh, vd_ss);
  return check_launch("inject_rerope");
}
