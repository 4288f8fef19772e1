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

}  // namespace hc

using namespace hc;

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
