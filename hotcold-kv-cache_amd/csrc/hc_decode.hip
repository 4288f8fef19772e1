// GQA decode attention over the hot buffer (+ held retrieved slot), split-K.
//
// Replaces evict_fwd_kernel / triton_evict_attention_forward
// (src/hotcold_kv/kernels.py:9-137).  The reference launches one program per
// QUERY head (grid (B, Hq), kernels.py:114) and reads each KV head's K/V G
// times, with an unstabilised exp (kernels.py:57).  Here one workgroup owns
// (batch, KV head, key split) and serves all G query heads of the group from
// a single K/V read:
//   * Q.K^T on MFMA: v_mfma_f32_16x16x32_{f16,bf16} with the 16 key rows of a
//     tile as the A operand and the G (<=16) query heads as the B operand;
//     fp32 inputs use v_mfma_f32_16x16x4f32.
//   * online max-stabilised softmax in the log2 domain (exp2), fp32;
//   * P.V on the VALU: 16 lanes cover one 2*D-byte V row (128-bit loads),
//     4 rows per wave instruction, fp32 accumulators;
//   * split partials (m, l, acc) combined by the last-arriving workgroup of
//     each (b, kv-head) through an atomic ticket (no second launch).
#include "hc_common.h"

namespace hc {

struct DecodeArgs {
  const void* q;
  int64_t q_sb, q_sh;
  const void* k;
  int64_t k_sb, k_sh, k_ss;
  const void* v;
  int64_t v_sb, v_sh, v_ss;
  const uint8_t* mask;
  int64_t mask_sb;
  const int64_t* held_pos;
  int64_t hp_sb, hp_sh;
  const uint8_t* held_valid;
  int64_t hv_sb, hv_sh;
  const int64_t* cur_pos;
  int64_t held_len;
  void* out;
  int64_t o_sb, o_sh;
  float* part;         // [units][splits][G*D + 2*G] split partials (splits > 1)
  float* scores;       // optional [B][Hq][S] log2-domain logits (eviction score)
  float* ml;           // optional [B][Hq][2] final (max, sum)
  int B, Hq, Hk, G, S, splits, keys_per_split;
  float scale_log2;
};

// ---------------------------------------------------------------------------
// Per-lane registers of one 16-key tile, loaded one tile ahead of use.
//   K (MFMA A operand): lane l holds key row tile + l%16, 16-byte pieces at
//     dims 32t + 8*(l/16) (f16/bf16) or 16t + 4*(l/16) (f32).
//   V (P.V layout): lane l holds rows tile + 4*(l/16) + i, i = 0..3, dims
//     (l%16)*DPL .. +DPL.
// ---------------------------------------------------------------------------
template <typename T, int D>
struct TileRegs {
  static constexpr int KW = (sizeof(T) == 4) ? D / 16 : (D + 31) / 32;  // 16-byte K pieces
  static constexpr int DPL = D / 16;
  static constexpr int VB = DPL * (int)sizeof(T);                        // V bytes per row per lane
  static constexpr int VWORDS = VB >= 4 ? VB / 4 : 1;
  u32x4 k[KW];
  uint32_t v[4][VWORDS];
  uint32_t keep;  // bit i: key tile + 4*(l/16) + i is attended
};

template <typename T, int D>
__device__ __forceinline__ void load_tile(TileRegs<T, D>& r, const T* kbase, const T* vbase, int64_t k_ss,
                                          int64_t v_ss, int tile, int key_end, int col, int grp,
                                          const DecodeArgs& a, int b, int hk, int64_t cur, const uint8_t* mrow) {
  using R = TileRegs<T, D>;
  // Key mask of this lane's four rows, evaluated here (one tile ahead) so
  // that the MFMA, the reads of its result and the score selects of
  // process_tile form one straight-line block.
  uint32_t keep = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = tile + 4 * grp + i;
    bool kp = key < key_end;
    if (kp && mrow) kp = mrow[key] != 0;
    if (kp && key < a.held_len)
      kp = a.held_valid[b * a.hv_sb + hk * a.hv_sh + key] != 0 && a.held_pos[b * a.hp_sb + hk * a.hp_sh + key] <= cur;
    keep |= (kp ? 1u : 0u) << i;
  }
  r.keep = keep;
  const int arow = tile + col;
  const bool kok = arow < key_end;
  const T* krow = kbase + (int64_t)arow * k_ss;
#pragma unroll
  for (int t = 0; t < R::KW; ++t) {
    const int d0 = (sizeof(T) == 4) ? 16 * t + 4 * grp : 32 * t + 8 * grp;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (kok && d0 < D) w = ld16(krow + d0);
    r.k[t] = w;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = tile + 4 * grp + i;
    const char* p = reinterpret_cast<const char*>(vbase + (int64_t)key * v_ss + col * R::DPL);
    if (key < key_end) {
      if constexpr (R::VB >= 16) {
#pragma unroll
        for (int c = 0; c < R::VB / 16; ++c) {
          const u32x4 x = ld16(p + 16 * c);
          r.v[i][4 * c + 0] = x[0];
          r.v[i][4 * c + 1] = x[1];
          r.v[i][4 * c + 2] = x[2];
          r.v[i][4 * c + 3] = x[3];
        }
      } else if constexpr (R::VB == 8) {
        const u32x2 x = *reinterpret_cast<const u32x2*>(p);
        r.v[i][0] = x[0];
        r.v[i][1] = x[1];
      } else if constexpr (R::VB == 4) {
        r.v[i][0] = *reinterpret_cast<const uint32_t*>(p);
      } else {
        r.v[i][0] = (uint32_t)(*reinterpret_cast<const uint16_t*>(p));
      }
    } else {
#pragma unroll
      for (int c = 0; c < R::VWORDS; ++c) r.v[i][c] = 0u;
    }
  }
}

// Q.K^T of one tile.  Output lane layout of every 16x16 fp32 MFMA block:
// lane l holds C[4*(l/16)+i][l%16], i = 0..3  (row = key, column = head).
template <typename T, int D>
struct QFrag;

template <int D>
struct QFrag<half_t, D> {
  static constexpr int NK = (D + 31) / 32;
  half8 qb[NK];
  // B operand: lane l supplies q[head l%16][32t + 8*(l/16) + j].
  __device__ void load(const half_t* q0, int64_t q_sh, int col, int grp, int G) {
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      const int d0 = 32 * t + 8 * grp;
      u32x4 w = {0u, 0u, 0u, 0u};
      if (col < G && d0 < D) w = ld16(q0 + col * q_sh + d0);
      qb[t] = __builtin_bit_cast(half8, w);
    }
  }
  __device__ floatx4 dot(const TileRegs<half_t, D>& r) const {
    floatx4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NK; ++t)
      c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, r.k[t]), qb[t], c, 0, 0, 0);
    return c;
  }
};

template <int D>
struct QFrag<bf16_t, D> {
  static constexpr int NK = (D + 31) / 32;
  bf16x8 qb[NK];
  __device__ void load(const bf16_t* q0, int64_t q_sh, int col, int grp, int G) {
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      const int d0 = 32 * t + 8 * grp;
      u32x4 w = {0u, 0u, 0u, 0u};
      if (col < G && d0 < D) w = ld16(q0 + col * q_sh + d0);
      qb[t] = __builtin_bit_cast(bf16x8, w);
    }
  }
  __device__ floatx4 dot(const TileRegs<bf16_t, D>& r) const {
    floatx4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NK; ++t)
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.k[t]), qb[t], c, 0, 0, 0);
    return c;
  }
};

template <int D>
struct QFrag<float, D> {
  // v_mfma_f32_16x16x4f32: lane l supplies A[l%16][l/16] and B[l/16][l%16].
  // One 16-byte piece per lane covers four MFMA steps: step j of block t uses
  // dim 16t + 4*(l/16) + j (a permutation of the block's 16 dims).
  static constexpr int NB = D / 16;
  float qb[NB][4];
  __device__ void load(const float* q0, int64_t q_sh, int col, int grp, int G) {
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (col < G) w = ld16(q0 + col * q_sh + 16 * t + 4 * grp);
      // Whole-vector bit cast, then element reads: a bit cast of a single
      // vector element miscompiles to element 0 with this toolchain.
      const floatx4 f = __builtin_bit_cast(floatx4, w);
      qb[t][0] = f[0];
      qb[t][1] = f[1];
      qb[t][2] = f[2];
      qb[t][3] = f[3];
    }
  }
  __device__ floatx4 dot(const TileRegs<float, D>& r) const {
    floatx4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const floatx4 f = __builtin_bit_cast(floatx4, r.k[t]);
      const float a0 = f[0];
      const float a1 = f[1];
      const float a2 = f[2];
      const float a3 = f[3];
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, qb[t][0], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, qb[t][1], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(a2, qb[t][2], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(a3, qb[t][3], c, 0, 0, 0);
    }
    return c;
  }
};

// Online-softmax state of one lane: running max / partial sum of head `col`
// and the P.V accumulators of the lane's dim slice for every head.
template <int GM, int DPL>
struct SoftmaxState {
  float m_run;
  float l_run;
  float acc[GM][DPL];
};

template <typename T, int D, int GM>
__device__ __forceinline__ void process_tile(const TileRegs<T, D>& r, const QFrag<T, D>& qf,
                                             SoftmaxState<GM, D / 16>& st, const DecodeArgs& a, int b, int hk,
                                             int tile, int key_end, int col, int grp, int64_t cur,
                                             const uint8_t* mrow, float* srow) {
  constexpr int DPL = D / 16;
  const int G = a.G;
  const floatx4 c = qf.dot(r);
  const float c4[4] = {c[0], c[1], c[2], c[3]};
  const uint32_t keep = (col < G) ? r.keep : 0u;
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = ((keep >> i) & 1u) ? c4[i] * a.scale_log2 : -INFINITY;
  if (srow && col < G) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = tile + 4 * grp + i;
      if (key < key_end) srow[key] = s[i];
    }
  }
  float tm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  tm = fmaxf(tm, __shfl_xor(tm, 16, 64));
  tm = fmaxf(tm, __shfl_xor(tm, 32, 64));
  const float m_new = fmaxf(st.m_run, tm);
  const bool dead = (m_new == -INFINITY);
  const float alpha = dead ? 1.f : exp2f(st.m_run - m_new);
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = dead ? 0.f : exp2f(s[i] - m_new);
  st.l_run = st.l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
  st.m_run = m_new;

  // P.V: lane (grp, col) handles keys tile + 4*grp + i, dims col*DPL ..
  const int src = 16 * grp;
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      if (g < G) {
        const float ag = __shfl(alpha, src + g, 64);
#pragma unroll
        for (int j = 0; j < DPL; ++j) st.acc[g][j] *= ag;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float vv[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) vv[j] = Unpack<T>::get(r.v[i], j);
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      if (g < G) {
        const float pg = __shfl(p[i], src + g, 64);
#pragma unroll
        for (int j = 0; j < DPL; ++j) st.acc[g][j] = fmaf(pg, vv[j], st.acc[g][j]);
      }
    }
  }
}

// grid (splits, Hk, B), block 256 (4 waves).  Each wave takes every fourth
// 16-key tile of the workgroup's key range, with the next tile's K/V loads in
// flight while the current one is processed.
template <typename T, int D, int GM>
__global__ __launch_bounds__(256) void decode_attn_kernel(DecodeArgs a) {
  constexpr int DPL = D / 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int split = blockIdx.x;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const int G = a.G;
  const int key_begin = split * a.keys_per_split;
  const int key_end = min(a.S, key_begin + a.keys_per_split);

  const T* kbase = reinterpret_cast<const T*>(a.k) + b * a.k_sb + hk * a.k_sh;
  const T* vbase = reinterpret_cast<const T*>(a.v) + b * a.v_sb + hk * a.v_sh;

  QFrag<T, D> qf;
  qf.load(reinterpret_cast<const T*>(a.q) + b * a.q_sb + (int64_t)(hk * G) * a.q_sh, a.q_sh, col, grp, G);

  const int64_t cur = a.cur_pos ? *a.cur_pos : INT64_MAX;
  const uint8_t* mrow = a.mask ? a.mask + b * a.mask_sb : nullptr;
  float* srow = a.scores ? a.scores + ((int64_t)b * a.Hq + hk * G + col) * a.S : nullptr;

  SoftmaxState<GM, DPL> st;
  st.m_run = -INFINITY;
  st.l_run = 0.f;
#pragma unroll
  for (int g = 0; g < GM; ++g)
#pragma unroll
    for (int j = 0; j < DPL; ++j) st.acc[g][j] = 0.f;

  TileRegs<T, D> ra, rb;
  int tile = key_begin + wave * 16;
  if (tile < key_end) load_tile<T, D>(ra, kbase, vbase, a.k_ss, a.v_ss, tile, key_end, col, grp, a, b, hk, cur, mrow);
  while (tile < key_end) {
    if (tile + 64 < key_end) load_tile<T, D>(rb, kbase, vbase, a.k_ss, a.v_ss, tile + 64, key_end, col, grp, a, b, hk, cur, mrow);
    process_tile<T, D, GM>(ra, qf, st, a, b, hk, tile, key_end, col, grp, cur, mrow, srow);
    tile += 64;
    if (tile >= key_end) break;
    if (tile + 64 < key_end) load_tile<T, D>(ra, kbase, vbase, a.k_ss, a.v_ss, tile + 64, key_end, col, grp, a, b, hk, cur, mrow);
    process_tile<T, D, GM>(rb, qf, st, a, b, hk, tile, key_end, col, grp, cur, mrow, srow);
    tile += 64;
  }

  // ---- reduce the four row groups of the wave (they share m_run) ----
  float l_run = st.l_run;
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
#pragma unroll
  for (int g = 0; g < GM; ++g)
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      float x = st.acc[g][j];
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      st.acc[g][j] = x;
    }

  __shared__ float sm_m[4][GM];
  __shared__ float sm_l[4][GM];
  __shared__ float sm_acc[4][GM][D];
  if (grp == 0) {
    if (col < GM) {
      sm_m[wave][col] = st.m_run;
      sm_l[wave][col] = l_run;
    }
#pragma unroll
    for (int g = 0; g < GM; ++g)
#pragma unroll
      for (int j = 0; j < DPL; ++j) sm_acc[wave][g][col * DPL + j] = st.acc[g][j];
  }
  __syncthreads();

  const int unit = b * a.Hk + hk;
  const int stride_part = G * D + 2 * G;
  T* obase = reinterpret_cast<T*>(a.out) + b * a.o_sb + (int64_t)(hk * G) * a.o_sh;
  for (int e = threadIdx.x; e < G * D; e += 256) {
    const int g = e / D, d = e - g * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm_m[w][g]);
    float A = 0.f, L = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float sc = exp2f(sm_m[w][g] - M);
        A = fmaf(sm_acc[w][g][d], sc, A);
        L = fmaf(sm_l[w][g], sc, L);
      }
    }
    if (a.splits == 1) {
      obase[g * a.o_sh + d] = from_f32<T>(A / L);
      if (a.ml && d == 0) {
        a.ml[((int64_t)b * a.Hq + hk * G + g) * 2 + 0] = M;
        a.ml[((int64_t)b * a.Hq + hk * G + g) * 2 + 1] = L;
      }
    } else {
      float* pp = a.part + ((int64_t)unit * a.splits + split) * stride_part;
      pp[e] = A;
      if (d == 0) {
        pp[G * D + g] = M;
        pp[G * D + G + g] = L;
      }
    }
  }
}

// Merge the split partials of every (b, kv head).  grid (Hk, B), block 256.
template <typename T>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeArgs a, int D) {
  const int hk = blockIdx.x, b = blockIdx.y;
  const int G = a.G;
  const int unit = b * a.Hk + hk;
  const int stride_part = G * D + 2 * G;
  const float* pu = a.part + (int64_t)unit * a.splits * stride_part;
  T* obase = reinterpret_cast<T*>(a.out) + b * a.o_sb + (int64_t)(hk * G) * a.o_sh;
  for (int e = threadIdx.x; e < G * D; e += blockDim.x) {
    const int g = e / D, d = e - g * D;
    float M = -INFINITY;
    for (int s = 0; s < a.splits; ++s) M = fmaxf(M, pu[s * stride_part + G * D + g]);
    float A = 0.f, L = 0.f;
    if (M != -INFINITY) {
      for (int s = 0; s < a.splits; ++s) {
        const float* ps = pu + s * stride_part;
        const float sc = exp2f(ps[G * D + g] - M);
        A = fmaf(ps[e], sc, A);
        L = fmaf(ps[G * D + G + g], sc, L);
      }
    }
    obase[g * a.o_sh + d] = from_f32<T>(A / L);
    if (a.ml && d == 0) {
      a.ml[((int64_t)b * a.Hq + hk * G + g) * 2 + 0] = M;
      a.ml[((int64_t)b * a.Hq + hk * G + g) * 2 + 1] = L;
    }
  }
}

// Per-token eviction score of the reference kernel (kernels.py:66-67, 134-136):
//   loss[b,s] = dtype( mean_h( p[b,h,s] / l[b,h] * mean_d |v[b,hk(h),s,d]| ) )
// with p = exp(logit - max) (the max cancels), and evict_idx[b] = first argmin.
template <typename T>
__global__ __launch_bounds__(256) void evict_score_kernel(const float* scores, const float* ml,
                                                          const T* v, int64_t v_sb, int64_t v_sh,
                                                          int64_t v_ss, int Hq, int G, int S, int D,
                                                          float* loss, int64_t* idx) {
  const int b = blockIdx.x;
  float best = INFINITY;
  int best_i = 0x7fffffff;
  for (int s = threadIdx.x; s < S; s += blockDim.x) {
    float tot = 0.f;
    for (int hk = 0; hk < Hq / G; ++hk) {
      const T* vr = v + b * v_sb + hk * v_sh + (int64_t)s * v_ss;
      float av = 0.f;
      for (int d = 0; d < D; ++d) av += fabsf(to_f32(vr[d]));
      av /= (float)D;
      for (int g = 0; g < G; ++g) {
        const int h = hk * G + g;
        const float M = ml[((int64_t)b * Hq + h) * 2 + 0];
        const float L = ml[((int64_t)b * Hq + h) * 2 + 1];
        const float sc = scores[((int64_t)b * Hq + h) * S + s];
        const float pn = (sc == -INFINITY) ? 0.f : exp2f(sc - M) / L;
        tot += pn * av;
      }
    }
    const float lv = to_f32(from_f32<T>(tot / (float)Hq));
    loss[(int64_t)b * S + s] = lv;
    if (lv < best || (lv != lv && best == best)) {  // NaN ranks lowest (torch.argmin)
      best = lv;
      best_i = s;
    }
  }
  __shared__ float sb[256];
  __shared__ int si[256];
  sb[threadIdx.x] = best;
  si[threadIdx.x] = best_i;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      const float x = sb[threadIdx.x + o];
      const int xi = si[threadIdx.x + o];
      const float y = sb[threadIdx.x];
      const int yi = si[threadIdx.x];
      const bool xnan = (x != x), ynan = (y != y);
      bool take;
      if (xnan || ynan) take = xnan && (!ynan || xi < yi);
      else take = (x < y) || (x == y && xi < yi);
      if (take) {
        sb[threadIdx.x] = x;
        si[threadIdx.x] = xi;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) idx[b] = si[0];
}

static int pick_splits(int64_t units, int64_t S, int64_t requested) {
  int64_t splits = requested;
  if (splits <= 0) {
    // Enough workgroups to cover the 256 CUs about twice; a split smaller
    // than 64 keys leaves waves of the workgroup idle.
    const int64_t target_blocks = 512;
    splits = cdiv(target_blocks, units);
  }
  const int64_t max_splits = cdiv(S, 64);
  if (splits > max_splits) splits = max_splits;
  if (splits < 1) splits = 1;
  const int64_t kps = cdiv(cdiv(S, splits), 64) * 64;
  return (int)cdiv(S, kps);
}

static int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

struct DecodeLayout {
  int64_t part_off, scores_off, ml_off, total;
};

static DecodeLayout decode_layout(int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
                                  int64_t splits, int with_evict) {
  DecodeLayout L;
  const int64_t units = B * Hk;
  const int64_t G = Hq / (Hk > 0 ? Hk : 1);
  L.part_off = 0;
  const int64_t part_bytes = splits > 1 ? units * splits * (G * D + 2 * G) * 4 : 0;
  L.scores_off = align256(L.part_off + part_bytes);
  const int64_t scores_bytes = with_evict ? B * Hq * S * 4 : 0;
  L.ml_off = align256(L.scores_off + scores_bytes);
  const int64_t ml_bytes = with_evict ? B * Hq * 2 * 4 : 0;
  L.total = align256(L.ml_off + ml_bytes);
  return L;
}

template <typename T, int D, int GM>
static void launch_decode(const DecodeArgs& a, hipStream_t st) {
  dim3 grid(a.splits, a.Hk, a.B);
  hipLaunchKernelGGL((decode_attn_kernel<T, D, GM>), grid, dim3(256), 0, st, a);
  if (a.splits > 1)
    hipLaunchKernelGGL(decode_combine_kernel<T>, dim3(a.Hk, a.B), dim3(256), 0, st, a, D);
}

template <typename T, int D>
static int dispatch_g(const DecodeArgs& a, hipStream_t st) {
  if (a.G <= 4) {
    launch_decode<T, D, 4>(a, st);
  } else if (a.G <= 8) {
    launch_decode<T, D, 8>(a, st);
  } else {
    if constexpr (D <= 128) {
      if (a.G <= 16) {
        launch_decode<T, D, 16>(a, st);
        return HC_OK;
      }
    }
    return set_error(HC_ERR_UNSUPPORTED, "decode: group size %d unsupported for D=%d", a.G, D);
  }
  return HC_OK;
}

template <typename T>
static int dispatch_d(int64_t D, const DecodeArgs& a, hipStream_t st) {
  switch (D) {
    case 16: return dispatch_g<T, 16>(a, st);
    case 32: return dispatch_g<T, 32>(a, st);
    case 64: return dispatch_g<T, 64>(a, st);
    case 128: return dispatch_g<T, 128>(a, st);
    case 256: return dispatch_g<T, 256>(a, st);
    default: return set_error(HC_ERR_UNSUPPORTED, "decode: head_dim %lld unsupported (16/32/64/128/256)", (long long)D);
  }
}

}  // namespace hc

using namespace hc;

extern "C" int64_t hc_decode_attn_workspace_size(int64_t B, int64_t Hq, int64_t Hk, int64_t D,
                                                 int64_t S, int64_t num_splits, int with_evict) {
  if (B <= 0 || Hq <= 0 || Hk <= 0 || D <= 0 || S <= 0) return 256;
  const int splits = pick_splits(B * Hk, S, num_splits);
  return decode_layout(B, Hq, Hk, D, S, splits, with_evict).total;
}

extern "C" int hc_decode_attn(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
                              const void* q, int64_t q_sb, int64_t q_sh,
                              const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                              const void* v, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                              const uint8_t* mask, int64_t mask_sb,
                              int64_t held_len,
                              const int64_t* held_pos, int64_t hp_sb, int64_t hp_sh,
                              const uint8_t* held_valid, int64_t hv_sb, int64_t hv_sh,
                              const int64_t* cur_pos,
                              double scaling, double dropout,
                              void* out, int64_t o_sb, int64_t o_sh,
                              float* evict_loss, int64_t* evict_idx,
                              void* workspace, int64_t workspace_bytes, int64_t num_splits,
                              void* stream) {
  if (dropout != 0.0) return set_error(HC_ERR_DROPOUT, "dropout must be 0.0 , because we are not in training");
  HC_REQUIRE(dtype == HC_DTYPE_F32 || dtype == HC_DTYPE_F16 || dtype == HC_DTYPE_BF16, "decode: bad dtype %d", dtype);
  HC_REQUIRE(B > 0 && Hq > 0 && Hk > 0 && D > 0 && S > 0, "decode: empty shape B=%lld Hq=%lld Hk=%lld D=%lld S=%lld",
             (long long)B, (long long)Hq, (long long)Hk, (long long)D, (long long)S);
  if (Hq % Hk != 0) return set_error(HC_ERR_GROUP, "Hq(%lld)//N_REP must equal Hk(%lld)", (long long)Hq, (long long)Hk);
  HC_REQUIRE(B <= 65535 && Hk <= 65535, "decode: B or Hk too large for the grid");
  HC_REQUIRE(S <= (int64_t)1 << 30, "decode: S too large");
  HC_REQUIRE(q && k && v && out, "decode: null tensor pointer");
  HC_REQUIRE(held_len >= 0 && held_len <= S, "decode: held_len %lld out of [0, S]", (long long)held_len);
  HC_REQUIRE(held_len == 0 || (held_pos && held_valid), "decode: held slot needs held_pos and held_valid");
  const int es = dtype_size(dtype);
  // 16-byte alignment of every row start used by the vector loads.
  const int64_t rowb = D * es;
  HC_REQUIRE(((uintptr_t)q % 16 == 0) && ((uintptr_t)k % 16 == 0) && ((uintptr_t)v % 16 == 0),
             "decode: q/k/v must be 16-byte aligned");
  HC_REQUIRE((q_sb * es) % 16 == 0 && (q_sh * es) % 16 == 0 && (k_sb * es) % 16 == 0 && (k_sh * es) % 16 == 0 &&
                 (k_ss * es) % 16 == 0 && (v_sb * es) % 16 == 0 && (v_sh * es) % 16 == 0 && (v_ss * es) % 16 == 0,
             "decode: q/k/v strides must be multiples of 16 bytes (row bytes %lld)", (long long)rowb);
  const int G = (int)(Hq / Hk);
  const int splits = pick_splits(B * Hk, S, num_splits);
  const int with_evict = (evict_loss != nullptr || evict_idx != nullptr);
  const DecodeLayout lay = decode_layout(B, Hq, Hk, D, S, splits, with_evict);
  if (!workspace || workspace_bytes < lay.total)
    return set_error(HC_ERR_WORKSPACE, "decode: workspace of %lld bytes needed, got %lld", (long long)lay.total,
                     (long long)workspace_bytes);
  HC_REQUIRE(((uintptr_t)workspace % 256) == 0, "decode: workspace must be 256-byte aligned");
  HC_REQUIRE(!with_evict || (evict_loss && evict_idx), "decode: evict_loss and evict_idx go together");

  DecodeArgs a;
  a.q = q; a.q_sb = q_sb; a.q_sh = q_sh;
  a.k = k; a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss;
  a.v = v; a.v_sb = v_sb; a.v_sh = v_sh; a.v_ss = v_ss;
  a.mask = mask; a.mask_sb = mask_sb;
  a.held_pos = held_pos; a.hp_sb = hp_sb; a.hp_sh = hp_sh;
  a.held_valid = held_valid; a.hv_sb = hv_sb; a.hv_sh = hv_sh;
  a.cur_pos = cur_pos; a.held_len = held_len;
  a.out = out; a.o_sb = o_sb; a.o_sh = o_sh;
  char* ws = reinterpret_cast<char*>(workspace);
  a.part = reinterpret_cast<float*>(ws + lay.part_off);
  a.scores = with_evict ? reinterpret_cast<float*>(ws + lay.scores_off) : nullptr;
  a.ml = with_evict ? reinterpret_cast<float*>(ws + lay.ml_off) : nullptr;
  a.B = (int)B; a.Hq = (int)Hq; a.Hk = (int)Hk; a.G = G; a.S = (int)S;
  a.splits = splits;
  a.keys_per_split = (int)(cdiv(cdiv(S, splits), 64) * 64);
  a.scale_log2 = (float)(scaling * 1.4426950408889634);

  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int rc;
  if (dtype == HC_DTYPE_F16) rc = dispatch_d<half_t>(D, a, st);
  else if (dtype == HC_DTYPE_BF16) rc = dispatch_d<bf16_t>(D, a, st);
  else rc = dispatch_d<float>(D, a, st);
  if (rc != HC_OK) return rc;
  if ((rc = check_launch("decode_attn")) != HC_OK) return rc;

  if (with_evict) {
    if (dtype == HC_DTYPE_F16)
      hipLaunchKernelGGL(evict_score_kernel<half_t>, dim3((unsigned)B), dim3(256), 0, st, a.scores, a.ml,
                         (const half_t*)v, v_sb, v_sh, v_ss, (int)Hq, G, (int)S, (int)D, evict_loss, evict_idx);
    else if (dtype == HC_DTYPE_BF16)
      hipLaunchKernelGGL(evict_score_kernel<bf16_t>, dim3((unsigned)B), dim3(256), 0, st, a.scores, a.ml,
                         (const bf16_t*)v, v_sb, v_sh, v_ss, (int)Hq, G, (int)S, (int)D, evict_loss, evict_idx);
    else
      hipLaunchKernelGGL(evict_score_kernel<float>, dim3((unsigned)B), dim3(256), 0, st, a.scores, a.ml,
                         (const float*)v, v_sb, v_sh, v_ss, (int)Hq, G, (int)S, (int)D, evict_loss, evict_idx);
    if ((rc = check_launch("evict_score")) != HC_OK) return rc;
  }
  return HC_OK;
}
