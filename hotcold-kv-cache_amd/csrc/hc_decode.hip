// GQA decode attention over the hot buffer (+ held retrieved slot), split-K.
//
// Replaces evict_fwd_kernel / triton_evict_attention_forward
// (src/hotcold_kv/kernels.py:9-137).  The reference launches one program per
// QUERY head (grid (B, Hq), kernels.py:114) and reads each KV head's K/V G
// times, with an unstabilised exp (kernels.py:57).  Here one workgroup owns
// (batch, KV head, key split) and serves all G query heads of the group from
// a single K/V read:
//   * K/V stream through a per-wave ring of register tiles filled by raw
//     buffer loads (128-bit per lane).  Rows outside the workgroup's key range
//     are addressed past the buffer's end, so the hardware returns zeros
//     without touching memory; every load is unconditional, which lets the
//     compiler keep the whole ring in flight (exact vmcnt waits);
//   * Q.K^T on MFMA: v_mfma_f32_16x16x32_{f16,bf16} with the 16 key rows of a
//     tile as the A operand and the G (<=16) query heads as the B operand;
//     fp32 inputs use v_mfma_f32_16x16x4f32;
//   * online max-stabilised softmax in the log2 domain (exp2), fp32;
//   * P.V on MFMA for f16/bf16 (v_mfma_f32_16x16x16_{f16,bf16}): the Q.K^T
//     output leaves lane (r, c) holding p for keys 4r..4r+3 of head c, which
//     is exactly its B-operand share, and its four V rows give the A operand
//     (a byte permute per register), so no lane exchanges data; P is rounded
//     to the input type and the softmax sum uses the same rounded values.
//     fp32 inputs use the VALU (16 lanes per V row, fp32 FMAs);
//   * the attention mask and the held slot's valid & (pos <= cur) test are
//     evaluated once per workgroup into an LDS bitmap;
//   * split partials (m, l, acc) are merged by a second, one-pass kernel.
#include "hc_common.h"
#include <stddef.h>
#include <algorithm>
#include <mutex>

namespace hc {

struct DecodeArgs {
  // Fields the kernel's prologue reads come first: they fit the first 128
  // bytes, two scalar loads issued together, so the first K/V loads wait on
  // one round trip to the argument memory.
  const void* q;
  int64_t q_sb, q_sh;
  const void* k;
  int64_t k_sb, k_sh, k_ss;
  const void* v;
  int64_t v_sb, v_sh, v_ss;
  uint32_t k_bytes, v_bytes, q_bytes;  // buffer extents of one (b, kv head)
  int G;
  int keys_per_split;
  int S_cache;  // rows read from k/v: S, or S-1 with a fused append
  float scale_log2;
  int splits, S, Hq;
  int B, Hk;
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
  // Fused append (hc_decode_attn_append): the token at row S-1 comes from
  // k_new / v_new ([B][Hk][D]); the last split's workgroup attends it and
  // writes it (and optionally its pre-RoPE key and position) into row S-1.
  // Last in the struct: only the append kernels read these.
  const void* k_new;
  int64_t kn_sb, kn_sh;
  const void* v_new;
  int64_t vn_sb, vn_sh;
  const void* p_new;
  int64_t pn_sb, pn_sh;
  void* p_dst;
  int64_t pd_sb, pd_sh, pd_ss;
  const int64_t* pos_new;
  int64_t posn_sb;
  int64_t* pos_dst;
  int64_t posd_sb;
};
static_assert(offsetof(DecodeArgs, Hq) + sizeof(int) <= 128, "prologue fields must fit the first 128 bytes");

// Keys of one split when the keep bitmap is needed (mask or held slot).
constexpr int kMaxBitmapKeys = 16384;
// ---------------------------------------------------------------------------
// Per-lane registers of one 16-key tile.
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

// Keep bit of key `key` in the split's bitmap (bit key - key_begin).
__device__ __forceinline__ uint32_t bitmap_bit(const uint32_t* bits, int key, int key_begin) {
  const int rel = min(key - key_begin, kMaxBitmapKeys - 1);
  return (bits[rel >> 5] >> (rel & 31)) & 1u;
}

// Keep bits (bit i: key tile + 4*grp + i) of a tile from the bitmap.
__device__ __forceinline__ uint32_t tile_keep_bits(int tile, int key_begin, int grp, const uint32_t* bits) {
  uint32_t keep = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) keep |= bitmap_bit(bits, tile + 4 * grp + i, key_begin) << i;
  return keep;
}

// Issue the loads of one tile (all unconditional) and read its keep bits.
template <typename T, int D>
__device__ __forceinline__ void load_tile(TileRegs<T, D>& r, __amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                          uint32_t k_rowb, uint32_t v_rowb, int tile, int key_begin, int key_end,
                                          int col, int grp, const uint32_t* bits) {
  using R = TileRegs<T, D>;
  const int arow = tile + col;
  const bool kok = arow < key_end;
#pragma unroll
  for (int t = 0; t < R::KW; ++t) {
    const int d0 = (sizeof(T) == 4) ? 16 * t + 4 * grp : 32 * t + 8 * grp;
    const uint32_t off = (kok && d0 < D) ? (uint32_t)arow * k_rowb + (uint32_t)(d0 * sizeof(T)) : kOob;
    uint32_t w[4];
    bload<16>(krs, off, w);
    r.k[t] = u32x4{w[0], w[1], w[2], w[3]};
  }
  uint32_t keep = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = tile + 4 * grp + i;
    const bool ok = key < key_end;
    const uint32_t off = ok ? (uint32_t)key * v_rowb + (uint32_t)(col * R::DPL * sizeof(T)) : kOob;
    bload<(R::VB >= 16 ? 16 : R::VB)>(vrs, off, r.v[i]);
    if constexpr (R::VB > 16) {
#pragma unroll
      for (int c = 1; c < R::VB / 16; ++c) bload<16>(vrs, off == kOob ? kOob : off + 16 * c, &r.v[i][4 * c]);
    }
    const bool kp = ok && (!bits || bitmap_bit(bits, key, key_begin));
    keep |= (kp ? 1u : 0u) << i;
  }
  r.keep = keep;
}

// Q.K^T of one tile.  Output lane layout of every 16x16 fp32 MFMA block:
// lane l holds C[4*(l/16)+i][l%16], i = 0..3  (row = key, column = head).
// The appended token as a one-key tile: key row 0 of the K (MFMA A operand)
// and V (P.V) layouts, read from k_new / v_new; every other row is zero and
// not attended.  Resources of extent 0 (waves that do not own the token)
// make every load return zeros without a memory access.
template <typename T, int D>
__device__ __forceinline__ void load_token(TileRegs<T, D>& r, __amdgpu_buffer_rsrc_t knrs,
                                           __amdgpu_buffer_rsrc_t vnrs, int col, int grp, bool tok) {
  using R = TileRegs<T, D>;
#pragma unroll
  for (int t = 0; t < R::KW; ++t) {
    const int d0 = (sizeof(T) == 4) ? 16 * t + 4 * grp : 32 * t + 8 * grp;
    const uint32_t off = (col == 0 && d0 < D) ? (uint32_t)(d0 * sizeof(T)) : kOob;
    uint32_t w[4];
    bload<16>(knrs, off, w);
    r.k[t] = u32x4{w[0], w[1], w[2], w[3]};
  }
  const uint32_t off = (grp == 0) ? (uint32_t)(col * R::DPL * sizeof(T)) : kOob;
  bload<(R::VB >= 16 ? 16 : R::VB)>(vnrs, off, r.v[0]);
  if constexpr (R::VB > 16) {
#pragma unroll
    for (int c = 1; c < R::VB / 16; ++c) bload<16>(vnrs, off == kOob ? kOob : off + 16 * c, &r.v[0][4 * c]);
  }
#pragma unroll
  for (int i = 1; i < 4; ++i)
#pragma unroll
    for (int w = 0; w < R::VWORDS; ++w) r.v[i][w] = 0u;
  r.keep = (tok && grp == 0) ? 1u : 0u;
}

// Write the token tile's K and V rows at byte offsets k_row / v_row of the
// hot buffer (dropped unless tok).
template <typename T, int D>
__device__ __forceinline__ void store_token(const TileRegs<T, D>& r, __amdgpu_buffer_rsrc_t krs,
                                            __amdgpu_buffer_rsrc_t vrs, uint32_t k_row, uint32_t v_row, int col,
                                            int grp, bool tok) {
  using R = TileRegs<T, D>;
#pragma unroll
  for (int t = 0; t < R::KW; ++t) {
    const int d0 = (sizeof(T) == 4) ? 16 * t + 4 * grp : 32 * t + 8 * grp;
    const uint32_t off = (tok && col == 0 && d0 < D) ? k_row + (uint32_t)(d0 * sizeof(T)) : kOob;
    const u32x4 x = r.k[t];
    const uint32_t w[4] = {x[0], x[1], x[2], x[3]};
    bstore<16>(krs, off, w);
  }
  const uint32_t off = (tok && grp == 0) ? v_row + (uint32_t)(col * R::DPL * sizeof(T)) : kOob;
  bstore<(R::VB >= 16 ? 16 : R::VB)>(vrs, off, r.v[0]);
  if constexpr (R::VB > 16) {
#pragma unroll
    for (int c = 1; c < R::VB / 16; ++c) bstore<16>(vrs, off == kOob ? kOob : off + 16 * c, &r.v[0][4 * c]);
  }
}

template <typename T, int D>
struct QFrag;

template <int D>
struct QFrag<half_t, D> {
  static constexpr int NK = (D + 31) / 32;
  half8 qb[NK];
  // B operand: lane l supplies q[head l%16][32t + 8*(l/16) + j].
  __device__ void load(__amdgpu_buffer_rsrc_t qrs, uint32_t q_rowb, int col, int grp, int G) {
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      const int d0 = 32 * t + 8 * grp;
      const uint32_t off = (col < G && d0 < D) ? (uint32_t)col * q_rowb + (uint32_t)(d0 * 2) : kOob;
      uint32_t w[4];
      bload<16>(qrs, off, w);
      qb[t] = __builtin_bit_cast(half8, u32x4{w[0], w[1], w[2], w[3]});
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
  __device__ void load(__amdgpu_buffer_rsrc_t qrs, uint32_t q_rowb, int col, int grp, int G) {
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      const int d0 = 32 * t + 8 * grp;
      const uint32_t off = (col < G && d0 < D) ? (uint32_t)col * q_rowb + (uint32_t)(d0 * 2) : kOob;
      uint32_t w[4];
      bload<16>(qrs, off, w);
      qb[t] = __builtin_bit_cast(bf16x8, u32x4{w[0], w[1], w[2], w[3]});
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
  __device__ void load(__amdgpu_buffer_rsrc_t qrs, uint32_t q_rowb, int col, int grp, int G) {
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const uint32_t off = (col < G) ? (uint32_t)col * q_rowb + (uint32_t)((16 * t + 4 * grp) * 4) : kOob;
      uint32_t w[4];
      bload<16>(qrs, off, w);
      // Whole-vector bit cast, then element reads: a bit cast of a single
      // vector element miscompiles to element 0 with this toolchain.
      const floatx4 f = __builtin_bit_cast(floatx4, u32x4{w[0], w[1], w[2], w[3]});
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

template <typename T, int D, int GM, bool EVICT>
__device__ __forceinline__ void process_tile(const TileRegs<T, D>& r, const QFrag<T, D>& qf,
                                             SoftmaxState<GM, D / 16>& st, int G, float scale_log2, int tile,
                                             int key_end, int col, int grp, float* srow) {
  constexpr int DPL = D / 16;
  const floatx4 c = qf.dot(r);
  const float c4[4] = {c[0], c[1], c[2], c[3]};
  const uint32_t keep = (col < G) ? r.keep : 0u;
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = ((keep >> i) & 1u) ? c4[i] * scale_log2 : -INFINITY;
  if constexpr (EVICT) {
    if (col < G) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = tile + 4 * grp + i;
        if (key < key_end) srow[key] = s[i];
      }
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

// P.V on MFMA (2-byte types).  Accumulator block j holds, in lane (r, c),
// out[dim (4r + i) * (D/16) + j][head c] for i = 0..3.
template <int D>
struct MxState {
  float m_run;
  float l_run;
  floatx4 acc[D / 16];
};

template <typename T>
struct MxOps;

template <>
struct MxOps<half_t> {
  typedef _Float16 vec4 __attribute__((ext_vector_type(4)));
  __device__ static floatx4 mma(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(vec4, u32x2{a0, a1}),
                                                __builtin_bit_cast(vec4, u32x2{b0, b1}), c, 0, 0, 0);
  }
  // Round two probabilities to f16; return the packed pair and the rounded values.
  __device__ static uint32_t pack2(float x, float y, float& rx, float& ry) {
    const half_t hx = (half_t)x, hy = (half_t)y;
    rx = (float)hx;
    ry = (float)hy;
    return (uint32_t)__builtin_bit_cast(uint16_t, hx) | ((uint32_t)__builtin_bit_cast(uint16_t, hy) << 16);
  }
};

template <>
struct MxOps<bf16_t> {
  typedef short vec4 __attribute__((ext_vector_type(4)));
  __device__ static floatx4 mma(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(vec4, u32x2{a0, a1}),
                                                    __builtin_bit_cast(vec4, u32x2{b0, b1}), c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float x, float y, float& rx, float& ry) {
    const bf16_t hx = (bf16_t)x, hy = (bf16_t)y;
    rx = (float)hx;
    ry = (float)hy;
    return (uint32_t)__builtin_bit_cast(uint16_t, hx) | ((uint32_t)__builtin_bit_cast(uint16_t, hy) << 16);
  }
};

template <typename T, int D, bool EVICT>
__device__ __forceinline__ void process_tile_mx(const TileRegs<T, D>& r, const QFrag<T, D>& qf, MxState<D>& st,
                                                int G, float scale_log2, int tile, int key_end, int col, int grp,
                                                float* srow) {
  constexpr int DPL = D / 16;
  const floatx4 c = qf.dot(r);
  const float c4[4] = {c[0], c[1], c[2], c[3]};
  const uint32_t keep = (col < G) ? r.keep : 0u;
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = ((keep >> i) & 1u) ? c4[i] * scale_log2 : -INFINITY;
  if constexpr (EVICT) {
    if (col < G) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = tile + 4 * grp + i;
        if (key < key_end) srow[key] = s[i];
      }
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
  float pr[4];
  const uint32_t b0 = MxOps<T>::pack2(p[0], p[1], pr[0], pr[1]);
  const uint32_t b1 = MxOps<T>::pack2(p[2], p[3], pr[2], pr[3]);
  st.l_run = st.l_run * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
  st.m_run = m_new;
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int j = 0; j < DPL; ++j) st.acc[j] *= alpha;
  }
  // A operand of block j: the lane's four V rows at dim col*DPL + j.
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
    const int w = j >> 1;
    const uint32_t a0 = __builtin_amdgcn_perm(r.v[1][w], r.v[0][w], sel);
    const uint32_t a1 = __builtin_amdgcn_perm(r.v[3][w], r.v[2][w], sel);
    st.acc[j] = MxOps<T>::mma(a0, a1, b0, b1, st.acc[j]);
  }
}

template <typename T, int D, int GM>
struct DecodeState {
  typedef SoftmaxState<GM, D / 16> type;
};
template <int D, int GM>
struct DecodeState<half_t, D, GM> {
  typedef MxState<D> type;
};
template <int D, int GM>
struct DecodeState<bf16_t, D, GM> {
  typedef MxState<D> type;
};

// grid (splits, Hk, B), block 64*NW (NW waves).  Wave w streams a
// contiguous key range through a ring of NBUF register tiles.
// Mode bits: kEvict keeps every head's log2 logits (eviction score, H2O);
// kAppend attends and writes this step's token from k_new / v_new.
enum DecodeMode { kPlain = 0, kEvict = 1, kAppend = 2, kAppendEvict = 3 };

template <typename T, int D, int GM, int NW, int NBUF, int MINW, int MODE>
__global__ __launch_bounds__(64 * NW, MINW) void decode_attn_kernel(DecodeArgs a) {
  constexpr bool EVICT = (MODE & kEvict) != 0;
  constexpr bool APPEND = (MODE & kAppend) != 0;
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
  const int key_end = min(a.S_cache, key_begin + a.keys_per_split);

  const T* kbase = reinterpret_cast<const T*>(a.k) + b * a.k_sb + hk * a.k_sh;
  const T* vbase = reinterpret_cast<const T*>(a.v) + b * a.v_sb + hk * a.v_sh;
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(kbase, a.k_bytes);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vbase, a.v_bytes);
  const uint32_t k_rowb = (uint32_t)(a.k_ss * (int64_t)sizeof(T));
  const uint32_t v_rowb = (uint32_t)(a.v_ss * (int64_t)sizeof(T));


  constexpr bool MX = sizeof(T) == 2;
  typename DecodeState<T, D, GM>::type st;
  st.m_run = -INFINITY;
  st.l_run = 0.f;
  if constexpr (MX) {
#pragma unroll
    for (int j = 0; j < DPL; ++j) st.acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  } else {
#pragma unroll
    for (int g = 0; g < GM; ++g)
#pragma unroll
      for (int j = 0; j < DPL; ++j) st.acc[g][j] = 0.f;
  }

  // Wave w takes the 16-key tiles w, w + NW, w + 2 NW, ... of the split's
  // range, so the waves of a workgroup read neighbouring tiles at any
  // moment.  Contiguous per-wave ranges measured 13% slower at 72 MB per
  // launch (16.9 against 14.7 us): the last waves to receive their rows held
  // the workgroup at its final barrier.  Tile counts differ by at most one.
  const int first = key_begin + wave * 16;
  const int wend = key_end;
  const int nt = first < key_end ? (key_end - first + 16 * NW - 1) / (16 * NW) : 0;
  {
    QFrag<T, D> qf;
    const T* q0 = reinterpret_cast<const T*>(a.q) + b * a.q_sb + (int64_t)(hk * G) * a.q_sh;
    qf.load(make_rsrc(q0, a.q_bytes), (uint32_t)(a.q_sh * (int64_t)sizeof(T)), col, grp, G);

    // The ring's first NBUF-1 tiles are issued before the keep bitmap is
    // built, so the bitmap's own loads overlap them; their keep bits are
    // applied once the bitmap is complete.
    TileRegs<T, D> r[NBUF];
#pragma unroll
    for (int i = 0; i < NBUF - 1; ++i)
      load_tile<T, D>(r[i], krs, vrs, k_rowb, v_rowb, first + i * 16 * NW, key_begin, wend, col, grp, nullptr);

    // Fused append: the last wave of the last split attends the new token as
    // a one-key tile and copies the token's K/V (and pre-RoPE key and
    // position) into row S-1.  Its loads are issued right after the ring's
    // first tiles and it is processed after the wave's first NBUF tiles, by
    // when they have landed, so it adds no wait; the copies are stored after
    // the last tile.  Every wave runs
    // this code with resources of extent 0 where it does not own the token:
    // no branch around memory operations, so the compiler's load counting
    // stays exact.
    TileRegs<T, D> rn;
    uint32_t pw[TileRegs<T, D>::KW][4];
    uint32_t pos_w[2];
    bool tok = false;
    if constexpr (APPEND) {
      tok = split == a.splits - 1 && __builtin_amdgcn_readfirstlane(wave) == NW - 1;
      constexpr uint32_t rowb = D * sizeof(T);
      const T* kn = tok ? reinterpret_cast<const T*>(a.k_new) + b * a.kn_sb + hk * a.kn_sh : kbase;
      const T* vn = tok ? reinterpret_cast<const T*>(a.v_new) + b * a.vn_sb + hk * a.vn_sh : vbase;
      load_token<T, D>(rn, make_rsrc(kn, tok ? rowb : 0u), make_rsrc(vn, tok ? rowb : 0u), col, grp, tok);
      const bool tp = tok && a.p_new != nullptr;
      const T* pn = tp ? reinterpret_cast<const T*>(a.p_new) + b * a.pn_sb + hk * a.pn_sh : kbase;
      const __amdgpu_buffer_rsrc_t pnrs = make_rsrc(pn, tp ? rowb : 0u);
#pragma unroll
      for (int t = 0; t < TileRegs<T, D>::KW; ++t) {
        const int d0 = (sizeof(T) == 4) ? 16 * t + 4 * grp : 32 * t + 8 * grp;
        bload<16>(pnrs, (col == 0 && d0 < D) ? (uint32_t)(d0 * sizeof(T)) : kOob, pw[t]);
      }
      const bool tq = tok && a.pos_new != nullptr && hk == 0;
      const int64_t* psrc = tq ? a.pos_new + b * a.posn_sb : reinterpret_cast<const int64_t*>(kbase);
      bload<8>(make_rsrc(psrc, tq ? 8u : 0u), lane == 0 ? 0u : kOob, pos_w);
    }

    // Keep bitmap of the split's keys (attention mask and held-slot test
    // valid & pos <= cur), one key per thread, packed by wave ballots.
    __shared__ uint32_t sm_bits[kMaxBitmapKeys / 32];
    const bool use_bits = (a.mask != nullptr) || (a.held_len > key_begin);
    if (use_bits) {
      const int64_t cur = a.cur_pos ? *a.cur_pos : INT64_MAX;
      const uint8_t* mrow = a.mask ? a.mask + b * a.mask_sb : nullptr;
      const int nkeys = key_end - key_begin;
      for (int base = 0; base < nkeys; base += 64 * NW) {
        const int rel = base + (int)threadIdx.x;
        const int key = key_begin + rel;
        bool kp = rel < nkeys;
        if (kp && mrow) kp = mrow[key] != 0;
        if (kp && key < a.held_len)
          kp = a.held_valid[b * a.hv_sb + hk * a.hv_sh + key] != 0 &&
               a.held_pos[b * a.hp_sb + hk * a.hp_sh + key] <= cur;
        const unsigned long long m = __ballot(kp);
        if (lane < 2) sm_bits[((base + 64 * wave) >> 5) + lane] = lane ? (uint32_t)(m >> 32) : (uint32_t)m;
      }
      // LDS-only fences: the barrier does not wait for the ring's K/V loads.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#pragma unroll
      for (int i = 0; i < NBUF - 1; ++i) r[i].keep &= tile_keep_bits(first + i * 16 * NW, key_begin, grp, sm_bits);
    }
    const uint32_t* bits = use_bits ? sm_bits : nullptr;
    float* srow = EVICT ? a.scores + ((int64_t)b * a.Hq + hk * G + min(col, G - 1)) * a.S : nullptr;

    // Step t issues the loads of tile t + NBUF - 1 (past the range: no memory
    // traffic) and then processes tile t, so NBUF-1 tiles stay in flight.
#define HC_RING_GROUP(g0)                                                                                  \
  _Pragma("unroll") for (int j = 0; j < NBUF; ++j) {                                                       \
    const int t = (g0) + j;                                                                                \
    load_tile<T, D>(r[(j + NBUF - 1) % NBUF], krs, vrs, k_rowb, v_rowb, first + (t + NBUF - 1) * 16 * NW,  \
                    key_begin, wend, col, grp, bits);                                                      \
    if (t < nt) {                                                                                          \
      if constexpr (MX)                                                                                    \
        process_tile_mx<T, D, EVICT>(r[j], qf, st, G, a.scale_log2, first + t * 16 * NW, wend, col, grp, srow); \
      else                                                                                                 \
        process_tile<T, D, GM, EVICT>(r[j], qf, st, G, a.scale_log2, first + t * 16 * NW, wend, col, grp, srow); \
    }                                                                                                      \
  }
    int g_start = 0;
    if constexpr (APPEND) {
      HC_RING_GROUP(0)
      g_start = NBUF;
      // the token is key S-1; with EVICT its logit is kept like every key's
      // (only the owning wave's row 0 falls inside [S-1, key_end))
      if constexpr (MX)
        process_tile_mx<T, D, EVICT>(rn, qf, st, G, a.scale_log2, a.S - 1, tok ? a.S : 0, col, grp, srow);
      else
        process_tile<T, D, GM, EVICT>(rn, qf, st, G, a.scale_log2, a.S - 1, tok ? a.S : 0, col, grp, srow);
    }
    for (int g0 = g_start; g0 < nt; g0 += NBUF) {
      HC_RING_GROUP(g0)
    }
#undef HC_RING_GROUP
    if constexpr (APPEND) {
      // The token's rows.  Stored after the last tile: issued before the
      // loop instead, they measured slower.
      const uint32_t row = (uint32_t)(a.S - 1);
      store_token<T, D>(rn, krs, vrs, row * k_rowb, row * v_rowb, col, grp, tok);
      const bool tp = tok && a.p_new != nullptr;
      T* pd = tp ? reinterpret_cast<T*>(a.p_dst) + b * a.pd_sb + hk * a.pd_sh + (int64_t)row * a.pd_ss
                 : const_cast<T*>(kbase);
      const __amdgpu_buffer_rsrc_t pdrs = make_rsrc(pd, tp ? (uint32_t)(D * sizeof(T)) : 0u);
#pragma unroll
      for (int t = 0; t < TileRegs<T, D>::KW; ++t) {
        const int d0 = (sizeof(T) == 4) ? 16 * t + 4 * grp : 32 * t + 8 * grp;
        bstore<16>(pdrs, (col == 0 && d0 < D) ? (uint32_t)(d0 * sizeof(T)) : kOob, pw[t]);
      }
      const bool tq = tok && a.pos_new != nullptr && hk == 0;
      int64_t* pdst = tq ? a.pos_dst + b * a.posd_sb + row : reinterpret_cast<int64_t*>(const_cast<T*>(kbase));
      bstore<8>(make_rsrc(pdst, tq ? 8u : 0u), lane == 0 ? 0u : kOob, pos_w);
    }
  }

  // ---- reduce the four row groups of the wave (they share m_run) ----
  float l_run = st.l_run;
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  // Partials in LDS, one padding float per 32 (bank-conflict-free writes of
  // the MFMA layout, where the four row groups sit 32 floats apart).
  constexpr int RS = D + D / 32 + 1;
  __shared__ float sm_m[NW][GM];
  __shared__ float sm_l[NW][GM];
  __shared__ float sm_acc[NW][GM][RS];
  if (grp == 0 && col < GM) {
    sm_m[wave][col] = st.m_run;
    sm_l[wave][col] = l_run;
  }
  if constexpr (MX) {
    // lane (grp, col) holds dims (4*grp + i) * DPL + j of head col
    if (col < G) {
#pragma unroll
      for (int j = 0; j < DPL; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = (4 * grp + i) * DPL + j;
          sm_acc[wave][col][d + (d >> 5)] = st.acc[j][i];
        }
    }
  } else {
#pragma unroll
    for (int g = 0; g < GM; ++g)
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        float x = st.acc[g][j];
        x += __shfl_xor(x, 16, 64);
        x += __shfl_xor(x, 32, 64);
        st.acc[g][j] = x;
      }
    if (grp == 0) {
#pragma unroll
      for (int g = 0; g < GM; ++g)
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const int d = col * DPL + j;
          sm_acc[wave][g][d + (d >> 5)] = st.acc[g][j];
        }
    }
  }
  __syncthreads();

  const int unit = b * a.Hk + hk;
  const int stride_part = G * D + 2 * G;
  T* obase = reinterpret_cast<T*>(a.out) + b * a.o_sb + (int64_t)(hk * G) * a.o_sh;

  for (int e = threadIdx.x; e < G * D; e += 64 * NW) {
    const int g = e / D, d = e - g * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm_m[w][g]);
    float A = 0.f, L = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float sc = exp2f(sm_m[w][g] - M);
        A = fmaf(sm_acc[w][g][d + (d >> 5)], sc, A);
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

// Merge the split partials of every (b, kv head) in one pass over the splits
// (online rescaling, loads independent of the running values).
// grid (Hk, B), block 256.
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
    float M = -INFINITY, A = 0.f, L = 0.f;
#pragma unroll 8
    for (int s = 0; s < a.splits; ++s) {
      const float* ps = pu + s * stride_part;
      const float ms = ps[G * D + g];
      const float as = ps[e];
      const float ls = ps[G * D + G + g];
      const float Mn = fmaxf(M, ms);
      if (Mn != -INFINITY) {
        const float c0 = exp2f(M - Mn), c1 = exp2f(ms - Mn);
        A = A * c0 + as * c1;
        L = L * c0 + ls * c1;
        M = Mn;
      }
    }
    obase[g * a.o_sh + d] = from_f32<T>(A / L);
    if (a.ml && d == 0) {
      a.ml[((int64_t)b * a.Hq + hk * G + g) * 2 + 0] = M;
      a.ml[((int64_t)b * a.Hq + hk * G + g) * 2 + 1] = L;
    }
  }
}

// H2O accumulated attention (layer_state.py:55-65, 102-114): for every key
// s of (b, kv head hk), the attention probability averaged over the G query
// heads of the group (_reduce_probs_to_kv, scoring.py:29-37),
//   col = (1/G) sum_g exp2(score[h][s] - M[h]) / L[h],   h = hk*G + g,
// is added to acc[b][hk][s]; key S-1 (the token appended this step) starts
// from zero (the torch.cat of a zero column, layer_state.py:108-111).
// The one expression both H2O kernels use, so the fused eviction writes the
// same bits as accumulation followed by a separate selection.
__device__ __forceinline__ float h2o_updated(const float* scores, const float* ml, int Hq, int G, int S, int b,
                                             int hk, int s, const float* acc_row) {
  float col = 0.f;
  for (int g = 0; g < G; ++g) {
    const int h = hk * G + g;
    const float M = ml[((int64_t)b * Hq + h) * 2 + 0];
    const float L = ml[((int64_t)b * Hq + h) * 2 + 1];
    const float sc = scores[((int64_t)b * Hq + h) * S + s];
    col += (sc == -INFINITY) ? 0.f : exp2f(sc - M) / L;
  }
  col /= (float)G;
  return (s == S - 1 ? 0.f : acc_row[s]) + col;
}

// grid (cdiv(S, 256), Hk, B), block 256.
__global__ __launch_bounds__(256) void h2o_accum_kernel(const float* scores, const float* ml, int Hq, int G, int S,
                                                        float* acc, int64_t a_sb, int64_t a_sh) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  const int hk = blockIdx.y, b = blockIdx.z;
  if (s >= S) return;
  float* a = acc + b * a_sb + hk * a_sh;
  a[s] = h2o_updated(scores, ml, Hq, G, S, b, hk, s, a);
}

// H2O re-eviction of a cache one token over its budget, fused with the
// accumulation above (layer_state.py:102-114 then _compress, :68-79).  With
// keep_prefix = prefix - 1, keep_index (scoring.py:110-132) drops exactly one
// prefix row: the last in (score desc, index asc) order, i.e. the lowest
// order key and, among equal keys, the highest index.  Every other row keeps
// its order, so row r goes to r - (r > e).  K, V and the updated scores are
// written out of place into the destination buffers (S-1 rows).
//
// Every workgroup recomputes the updated scores of all S keys into LDS and
// finds e itself (a few KB of logits from L2), so the row copy needs no
// second launch; its own rows' loads are issued first and overlap that work.
// grid (cdiv(S, rows_per_wg), Hk, B), block 256; rows are rowb bytes
// (a multiple of 16), rows_per_wg <= 256 and rows_per_wg * rowb / 16 <= 2 * 256.
constexpr int kEvictMaxKeys = 8192;
struct H2OEvictArgs {
  const char* k;
  int64_t k_sb, k_sh, k_ss;  // byte strides
  const char* v;
  int64_t v_sb, v_sh, v_ss;
  char* kd;
  int64_t kd_sb, kd_sh, kd_ss;
  char* vd;
  int64_t vd_sb, vd_sh, vd_ss;
  float* acc_dst;
  int64_t ad_sb, ad_sh;
  int prefix, rowb, rows_per_wg;
};

__global__ __launch_bounds__(256) void h2o_evict_one_kernel(const float* scores, const float* ml, int Hq, int G,
                                                            int S, const float* acc, int64_t a_sb, int64_t a_sh,
                                                            H2OEvictArgs e) {
  __shared__ float sm_sc[kEvictMaxKeys];
  __shared__ uint32_t sm_best[2][4];
  const int hk = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r0 = blockIdx.x * e.rows_per_wg;
  const int cpr = e.rowb >> 4;
  const char* ks = e.k + b * e.k_sb + hk * e.k_sh;
  const char* vs = e.v + b * e.v_sb + hk * e.v_sh;

  u32x4 kr[2], vr[2];
  int row[2], part[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + 256 * i;
    row[i] = r0 + c / cpr;
    part[i] = c - (c / cpr) * cpr;
    if (c >= e.rows_per_wg * cpr || row[i] >= S) row[i] = -1;
    if (row[i] >= 0) {
      kr[i] = ld16(ks + row[i] * e.k_ss + part[i] * 16);
      vr[i] = ld16(vs + row[i] * e.v_ss + part[i] * 16);
    }
  }

  const float* arow = acc + b * a_sb + hk * a_sh;
  for (int s = tid; s < S; s += 256) sm_sc[s] = h2o_updated(scores, ml, Hq, G, S, b, hk, s, arow);
  __syncthreads();

  // lowest (order key, ~index) over the prefix
  uint32_t bk = 0xffffffffu, bi = 0xffffffffu;
  for (int s = tid; s < e.prefix; s += 256) {
    const uint32_t key = order_key(sm_sc[s]), inv = ~(uint32_t)s;
    if (key < bk || (key == bk && inv < bi)) { bk = key; bi = inv; }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t ok = __shfl_xor(bk, off, 64), oi = __shfl_xor(bi, off, 64);
    if (ok < bk || (ok == bk && oi < bi)) { bk = ok; bi = oi; }
  }
  if (lane == 0) { sm_best[0][wave] = bk; sm_best[1][wave] = bi; }
  __syncthreads();
  bk = sm_best[0][0]; bi = sm_best[1][0];
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    const uint32_t ok = sm_best[0][w], oi = sm_best[1][w];
    if (ok < bk || (ok == bk && oi < bi)) { bk = ok; bi = oi; }
  }
  const int ev = (int)~bi;

  char* kd = e.kd + b * e.kd_sb + hk * e.kd_sh;
  char* vd = e.vd + b * e.vd_sb + hk * e.vd_sh;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (row[i] >= 0 && row[i] != ev) {
      const int d = row[i] - (row[i] > ev);
      st16(kd + d * e.kd_ss + part[i] * 16, kr[i]);
      st16(vd + d * e.vd_ss + part[i] * 16, vr[i]);
    }
  }
  const int r = r0 + tid;
  if (tid < e.rows_per_wg && r < S && r != ev)
    e.acc_dst[b * e.ad_sb + hk * e.ad_sh + (r - (r > ev))] = sm_sc[r];
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

// Launch shape of one (element size, head_dim, group bucket) instance:
//   nbuf  depth of the per-wave K/V register ring (tiles in flight + 1);
//   minw  waves per SIMD the register budget is sized for (2: <= 256 VGPRs,
//         1: up to 512 with the accumulation registers);
//   nw    waves per workgroup (8 needs minw 2 and an epilogue of at most
//         32 KB LDS, nw*gm*D floats).
// Chosen so that no instance spills (checked with the compiler's
// kernel-resource-usage report).
struct DecodeCfg {
  int nbuf, minw, nw;
};

constexpr DecodeCfg decode_cfg(int es, int D, int gm) {
  int nbuf = 2, minw = 1;
  if (es == 2) {
    // MFMA P.V: the accumulators do not grow with the group.  One tile in
    // flight per wave measured fastest (deeper rings add VGPRs, no speed).
    if (D <= 128) { nbuf = 2; minw = 2; }
  } else if (D <= 32) {
    nbuf = 4; minw = 2;
  } else if (D == 64) {
    nbuf = gm >= 16 ? 2 : 4; minw = 2;
  }
  const int nw = (minw == 2 && gm * D <= 1024) ? 8 : 4;
  return DecodeCfg{nbuf, minw, nw};
}

static int group_bucket(int64_t G) { return G <= 4 ? 4 : (G <= 8 ? 8 : 16); }

// Key splits per (batch, kv head).  Every split beyond one costs a second
// (merge) launch, a few microseconds of latency, so few units with short key
// ranges (up to 512 KB of K and V per unit, e.g. one layer at batch 1) run
// unsplit.  Otherwise: enough workgroups to give every CU one 8-wave (or two
// 4-wave) workgroups, no split shorter than one tile per wave, and, when the
// keep bitmap is used (mask or held slot), no split longer than the bitmap.
static int pick_splits(int64_t units, int64_t S, int64_t requested, int nw, bool bitmap, int64_t row_bytes) {
  int64_t splits = requested;
  if (splits <= 0) {
    splits = cdiv((int64_t)256 * 8 / nw, units);
    if (units < 128 && S * 2 * row_bytes <= ((int64_t)512 << 10)) splits = 1;
  }
  const int64_t step = 16 * nw;
  const int64_t max_splits = cdiv(S, step);
  if (splits > max_splits) splits = max_splits;
  if (bitmap && splits < cdiv(S, kMaxBitmapKeys)) splits = cdiv(S, kMaxBitmapKeys);
  if (splits < 1) splits = 1;
  const int64_t kps = cdiv(cdiv(S, splits), step) * step;
  return (int)cdiv(S, kps);
}

static int64_t keys_per_split(int64_t S, int splits, int nw) {
  const int64_t step = 16 * nw;
  return cdiv(cdiv(S, splits), step) * step;
}

static int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

// Split count of one launch (the choice decode_impl makes).
static int decode_splits(int es, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S_cache, int64_t num_splits,
                         bool bitmap) {
  const int nw = decode_cfg(es, (int)D, group_bucket(Hq / Hk)).nw;
  return pick_splits(B * Hk, S_cache > 0 ? S_cache : 1, num_splits, nw, bitmap, D * es);
}

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

template <typename T, int D, int GM, int NW, int NBUF, int MINW>
static void launch_decode(const DecodeArgs& a, hipStream_t st) {
  dim3 grid(a.splits, a.Hk, a.B);
  if (a.scores && a.k_new)
    hipLaunchKernelGGL((decode_attn_kernel<T, D, GM, NW, NBUF, MINW, kAppendEvict>), grid, dim3(64 * NW), 0, st, a);
  else if (a.scores)
    hipLaunchKernelGGL((decode_attn_kernel<T, D, GM, NW, NBUF, MINW, kEvict>), grid, dim3(64 * NW), 0, st, a);
  else if (a.k_new)
    hipLaunchKernelGGL((decode_attn_kernel<T, D, GM, NW, NBUF, MINW, kAppend>), grid, dim3(64 * NW), 0, st, a);
  else
    hipLaunchKernelGGL((decode_attn_kernel<T, D, GM, NW, NBUF, MINW, kPlain>), grid, dim3(64 * NW), 0, st, a);
  if (a.splits > 1)
    hipLaunchKernelGGL(decode_combine_kernel<T>, dim3(a.Hk, a.B), dim3(256), 0, st, a, D);
}

template <typename T, int D, int GM>
static void launch_nw(const DecodeArgs& a, int nw, hipStream_t st) {
  constexpr DecodeCfg c = decode_cfg((int)sizeof(T), D, GM);
  (void)nw;  // equals c.nw: the host picked the splits for it
  launch_decode<T, D, GM, c.nw, c.nbuf, c.minw>(a, st);
}

template <typename T, int D>
static int dispatch_g(const DecodeArgs& a, int nw, hipStream_t st) {
  if (a.G <= 4) {
    launch_nw<T, D, 4>(a, nw, st);
  } else if (a.G <= 8) {
    launch_nw<T, D, 8>(a, nw, st);
  } else {
    if constexpr (D <= 128) {
      if (a.G <= 16) {
        launch_nw<T, D, 16>(a, nw, st);
        return HC_OK;
      }
    }
    return set_error(HC_ERR_UNSUPPORTED, "decode: group size %d unsupported for D=%d", a.G, D);
  }
  return HC_OK;
}

template <typename T>
static int dispatch_d(int64_t D, const DecodeArgs& a, int nw, hipStream_t st) {
  switch (D) {
    case 16: return dispatch_g<T, 16>(a, nw, st);
    case 32: return dispatch_g<T, 32>(a, nw, st);
    case 64: return dispatch_g<T, 64>(a, nw, st);
    case 128: return dispatch_g<T, 128>(a, nw, st);
    case 256: return dispatch_g<T, 256>(a, nw, st);
    default: return set_error(HC_ERR_UNSUPPORTED, "decode: head_dim %lld unsupported (16/32/64/128/256)", (long long)D);
  }
}

}  // namespace hc

using namespace hc;

extern "C" int64_t hc_decode_attn_workspace_size(int64_t B, int64_t Hq, int64_t Hk, int64_t D,
                                                 int64_t S, int64_t num_splits, int with_evict) {
  if (B <= 0 || Hq <= 0 || Hk <= 0 || D <= 0 || S <= 0) return 256;
  // The element size is not an argument: size for every launch shape.
  int64_t need = 0;
  for (int es : {2, 4})
    for (int nw : {4, 8})
      for (bool bitmap : {false, true})
        for (int64_t Sc : {S, S > 1 ? S - 1 : S}) {
        const int splits = pick_splits(B * Hk, Sc, num_splits, nw, bitmap, D * es);
        const int64_t t = decode_layout(B, Hq, Hk, D, S, splits, with_evict).total;
        if (t > need) need = t;
        }
  return need;
}

static int decode_impl(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
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
                              void* stream, const DecodeArgs* ap, float* h2o_acc = nullptr,
                              int64_t h2o_sb = 0, int64_t h2o_sh = 0, const H2OEvictArgs* h2o_ev = nullptr) {
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
  const int nw = decode_cfg(es, (int)D, group_bucket(G)).nw;
  const bool bitmap = mask != nullptr || held_len > 0;
  const int64_t S_cache = ap ? S - 1 : S;  // a fused append's token is not read from k/v
  HC_REQUIRE(held_len <= S_cache, "decode: held_len %lld beyond the cached rows", (long long)held_len);
  const int splits = decode_splits(es, B, Hq, Hk, D, S_cache, num_splits, bitmap);
  // Buffer extents of one (b, kv head) must fit the 31-bit load offsets.
  const int64_t k_bytes = ((S - 1) * k_ss + D) * es, v_bytes = ((S - 1) * v_ss + D) * es;
  const int64_t q_bytes = ((Hq / Hk - 1) * q_sh + D) * es;
  HC_REQUIRE(k_ss >= D && v_ss >= D && k_bytes < ((int64_t)1 << 31) && v_bytes < ((int64_t)1 << 31) &&
                 q_bytes < ((int64_t)1 << 31),
             "decode: one (batch, kv head) K/V/Q extent must be below 2 GiB with row stride >= D");
  if (ap) {
    const auto al16 = [](const void* p) { return ((uintptr_t)p % 16) == 0; };
    HC_REQUIRE(al16(ap->k_new) && al16(ap->v_new) && (ap->kn_sb * es) % 16 == 0 && (ap->kn_sh * es) % 16 == 0 &&
                   (ap->vn_sb * es) % 16 == 0 && (ap->vn_sh * es) % 16 == 0,
               "decode_append: k_new / v_new rows must be 16-byte aligned");
    HC_REQUIRE(!ap->p_new || (al16(ap->p_new) && al16(ap->p_dst) && (ap->pn_sb * es) % 16 == 0 &&
                              (ap->pn_sh * es) % 16 == 0 && (ap->pd_sb * es) % 16 == 0 &&
                              (ap->pd_sh * es) % 16 == 0 && (ap->pd_ss * es) % 16 == 0 && ap->pd_ss >= D),
               "decode_append: p_new / p_dst rows must be 16-byte aligned with row stride >= D");
  }
  // per-head logits and (max, sum) are kept for the eviction score or H2O
  const int with_evict = (evict_loss != nullptr || evict_idx != nullptr || h2o_acc != nullptr);
  const DecodeLayout lay = decode_layout(B, Hq, Hk, D, S, splits, with_evict);
  if (!workspace || workspace_bytes < lay.total)
    return set_error(HC_ERR_WORKSPACE, "decode: workspace of %lld bytes needed, got %lld", (long long)lay.total,
                     (long long)workspace_bytes);
  HC_REQUIRE(((uintptr_t)workspace % 256) == 0, "decode: workspace must be 256-byte aligned");
  HC_REQUIRE((evict_loss == nullptr) == (evict_idx == nullptr), "decode: evict_loss and evict_idx go together");
  HC_REQUIRE(!(h2o_acc && evict_loss), "decode: H2O accumulation and the eviction score are exclusive");
  HC_REQUIRE(!(evict_loss && ap), "decode: the eviction score is not computed with a fused append");

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
  a.keys_per_split = (int)keys_per_split(S_cache > 0 ? S_cache : 1, splits, nw);
  a.S_cache = (int)S_cache;
  if (ap) {
    a.k_new = ap->k_new; a.kn_sb = ap->kn_sb; a.kn_sh = ap->kn_sh;
    a.v_new = ap->v_new; a.vn_sb = ap->vn_sb; a.vn_sh = ap->vn_sh;
    a.p_new = ap->p_new; a.pn_sb = ap->pn_sb; a.pn_sh = ap->pn_sh;
    a.p_dst = ap->p_dst; a.pd_sb = ap->pd_sb; a.pd_sh = ap->pd_sh; a.pd_ss = ap->pd_ss;
    a.pos_new = ap->pos_new; a.posn_sb = ap->posn_sb; a.pos_dst = ap->pos_dst; a.posd_sb = ap->posd_sb;
  } else {
    a.k_new = a.v_new = a.p_new = nullptr;
    a.p_dst = nullptr;
    a.pos_new = nullptr;
    a.pos_dst = nullptr;
  }
  a.scale_log2 = (float)(scaling * 1.4426950408889634);
  a.k_bytes = (uint32_t)k_bytes;
  a.v_bytes = (uint32_t)v_bytes;
  a.q_bytes = (uint32_t)q_bytes;

  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int rc;
  if (dtype == HC_DTYPE_F16) rc = dispatch_d<half_t>(D, a, nw, st);
  else if (dtype == HC_DTYPE_BF16) rc = dispatch_d<bf16_t>(D, a, nw, st);
  else rc = dispatch_d<float>(D, a, nw, st);
  if (rc != HC_OK) return rc;
  if ((rc = check_launch("decode_attn")) != HC_OK) return rc;

  if (h2o_acc && h2o_ev) {
    const dim3 grid((unsigned)cdiv(S, h2o_ev->rows_per_wg), (unsigned)Hk, (unsigned)B);
    hipLaunchKernelGGL(h2o_evict_one_kernel, grid, dim3(256), 0, st, a.scores, a.ml, (int)Hq, G, (int)S, h2o_acc,
                       h2o_sb, h2o_sh, *h2o_ev);
    if ((rc = check_launch("h2o_evict_one")) != HC_OK) return rc;
  } else if (h2o_acc) {
    const dim3 grid((unsigned)cdiv(S, 256), (unsigned)Hk, (unsigned)B);
    hipLaunchKernelGGL(h2o_accum_kernel, grid, dim3(256), 0, st, a.scores, a.ml, (int)Hq, G, (int)S, h2o_acc,
                       h2o_sb, h2o_sh);
    if ((rc = check_launch("h2o_accum")) != HC_OK) return rc;
  } else if (with_evict) {
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
  return decode_impl(dtype, B, Hq, Hk, D, S, q, q_sb, q_sh, k, k_sb, k_sh, k_ss, v, v_sb, v_sh, v_ss, mask, mask_sb,
                     held_len, held_pos, hp_sb, hp_sh, held_valid, hv_sb, hv_sh, cur_pos, scaling, dropout, out, o_sb,
                     o_sh, evict_loss, evict_idx, workspace, workspace_bytes, num_splits, stream, nullptr);
}

extern "C" int hc_decode_attn_append(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
                                     const void* q, int64_t q_sb, int64_t q_sh,
                                     void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                                     void* v, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                                     const void* k_new, int64_t kn_sb, int64_t kn_sh,
                                     const void* v_new, int64_t vn_sb, int64_t vn_sh,
                                     const void* p_new, int64_t pn_sb, int64_t pn_sh,
                                     void* p_dst, int64_t pd_sb, int64_t pd_sh, int64_t pd_ss,
                                     const int64_t* pos_new, int64_t posn_sb, int64_t* pos_dst, int64_t posd_sb,
                                     const uint8_t* mask, int64_t mask_sb,
                                     int64_t held_len,
                                     const int64_t* held_pos, int64_t hp_sb, int64_t hp_sh,
                                     const uint8_t* held_valid, int64_t hv_sb, int64_t hv_sh,
                                     const int64_t* cur_pos,
                                     double scaling,
                                     void* out, int64_t o_sb, int64_t o_sh,
                                     void* workspace, int64_t workspace_bytes, int64_t num_splits,
                                     void* stream) {
  HC_REQUIRE(k_new && v_new, "decode_append: k_new and v_new are required");
  HC_REQUIRE((p_new == nullptr) == (p_dst == nullptr), "decode_append: p_new and p_dst go together");
  HC_REQUIRE((pos_new == nullptr) == (pos_dst == nullptr), "decode_append: pos_new and pos_dst go together");
  DecodeArgs ap{};
  ap.k_new = k_new; ap.kn_sb = kn_sb; ap.kn_sh = kn_sh;
  ap.v_new = v_new; ap.vn_sb = vn_sb; ap.vn_sh = vn_sh;
  ap.p_new = p_new; ap.pn_sb = pn_sb; ap.pn_sh = pn_sh;
  ap.p_dst = p_dst; ap.pd_sb = pd_sb; ap.pd_sh = pd_sh; ap.pd_ss = pd_ss;
  ap.pos_new = pos_new; ap.posn_sb = posn_sb; ap.pos_dst = pos_dst; ap.posd_sb = posd_sb;
  return decode_impl(dtype, B, Hq, Hk, D, S, q, q_sb, q_sh, k, k_sb, k_sh, k_ss, v, v_sb, v_sh, v_ss, mask, mask_sb,
                     held_len, held_pos, hp_sb, hp_sh, held_valid, hv_sb, hv_sh, cur_pos, scaling, 0.0, out, o_sb,
                     o_sh, nullptr, nullptr, workspace, workspace_bytes, num_splits, stream, &ap);
}

extern "C" int hc_decode_attn_h2o(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
                                  const void* q, int64_t q_sb, int64_t q_sh,
                                  const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                                  const void* v, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                                  double scaling,
                                  void* out, int64_t o_sb, int64_t o_sh,
                                  float* acc, int64_t a_sb, int64_t a_sh,
                                  void* workspace, int64_t workspace_bytes, int64_t num_splits, void* stream) {
  HC_REQUIRE(acc != nullptr, "decode_h2o: acc is required");
  return decode_impl(dtype, B, Hq, Hk, D, S, q, q_sb, q_sh, k, k_sb, k_sh, k_ss, v, v_sb, v_sh, v_ss, nullptr, 0, 0,
                     nullptr, 0, 0, nullptr, 0, 0, nullptr, scaling, 0.0, out, o_sb, o_sh, nullptr, nullptr, workspace,
                     workspace_bytes, num_splits, stream, nullptr, acc, a_sb, a_sh);
}

extern "C" int hc_decode_attn_h2o_evict(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
                                        const void* q, int64_t q_sb, int64_t q_sh,
                                        const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                                        const void* v, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                                        const void* k_new, int64_t kn_sb, int64_t kn_sh,
                                        const void* v_new, int64_t vn_sb, int64_t vn_sh,
                                        double scaling,
                                        void* out, int64_t o_sb, int64_t o_sh,
                                        const float* acc, int64_t a_sb, int64_t a_sh,
                                        int64_t window, int64_t budget,
                                        void* k_dst, int64_t kd_sb, int64_t kd_sh, int64_t kd_ss,
                                        void* v_dst, int64_t vd_sb, int64_t vd_sh, int64_t vd_ss,
                                        float* acc_dst, int64_t ad_sb, int64_t ad_sh,
                                        void* workspace, int64_t workspace_bytes, int64_t num_splits,
                                        void* stream) {
  HC_REQUIRE(acc != nullptr && acc_dst != nullptr && k_dst != nullptr && v_dst != nullptr,
             "decode_h2o_evict: acc, acc_dst, k_dst and v_dst are required");
  HC_REQUIRE(dtype == HC_DTYPE_F32 || dtype == HC_DTYPE_F16 || dtype == HC_DTYPE_BF16,
             "decode_h2o_evict: bad dtype %d", dtype);
  HC_REQUIRE(window >= 0 && budget >= 0, "decode_h2o_evict: negative window or budget");
  // keep_index's counts (scoring.py:118-120): exactly one prefix row goes.
  const int64_t win = window < S ? window : S;
  const int64_t prefix = S - win;
  int64_t kp = budget - win < prefix ? budget - win : prefix;
  if (kp < 0) kp = 0;
  HC_REQUIRE(prefix - kp == 1, "decode_h2o_evict: S=%lld, window=%lld, budget=%lld drop %lld rows, not one",
             (long long)S, (long long)window, (long long)budget, (long long)(prefix - kp));
  HC_REQUIRE(S <= kEvictMaxKeys, "decode_h2o_evict: S=%lld above %d", (long long)S, kEvictMaxKeys);
  HC_REQUIRE(acc != acc_dst && k != k_dst && v != v_dst, "decode_h2o_evict: destinations must not alias sources");
  const int es = dtype_size(dtype);
  const int64_t rowb = D * es;
  HC_REQUIRE(rowb % 16 == 0 && rowb <= 8192, "decode_h2o_evict: row bytes %lld must be a multiple of 16, <= 8192",
             (long long)rowb);
  HC_REQUIRE(((uintptr_t)k_dst % 16 == 0) && ((uintptr_t)v_dst % 16 == 0) && (kd_sb * es) % 16 == 0 &&
                 (kd_sh * es) % 16 == 0 && (kd_ss * es) % 16 == 0 && (vd_sb * es) % 16 == 0 &&
                 (vd_sh * es) % 16 == 0 && (vd_ss * es) % 16 == 0 && kd_ss >= D && vd_ss >= D,
             "decode_h2o_evict: k_dst / v_dst rows must be 16-byte aligned with row stride >= D");
  H2OEvictArgs ev;
  ev.k = reinterpret_cast<const char*>(k); ev.k_sb = k_sb * es; ev.k_sh = k_sh * es; ev.k_ss = k_ss * es;
  ev.v = reinterpret_cast<const char*>(v); ev.v_sb = v_sb * es; ev.v_sh = v_sh * es; ev.v_ss = v_ss * es;
  ev.kd = reinterpret_cast<char*>(k_dst); ev.kd_sb = kd_sb * es; ev.kd_sh = kd_sh * es; ev.kd_ss = kd_ss * es;
  ev.vd = reinterpret_cast<char*>(v_dst); ev.vd_sb = vd_sb * es; ev.vd_sh = vd_sh * es; ev.vd_ss = vd_ss * es;
  ev.acc_dst = acc_dst; ev.ad_sb = ad_sb; ev.ad_sh = ad_sh;
  ev.prefix = (int)prefix;
  ev.rowb = (int)rowb;
  ev.rows_per_wg = (int)std::min<int64_t>(256, 512 / (rowb / 16));
  HC_REQUIRE((k_new == nullptr) == (v_new == nullptr), "decode_h2o_evict: k_new and v_new go together");
  DecodeArgs ap{};
  ap.k_new = k_new; ap.kn_sb = kn_sb; ap.kn_sh = kn_sh;
  ap.v_new = v_new; ap.vn_sb = vn_sb; ap.vn_sh = vn_sh;
  return decode_impl(dtype, B, Hq, Hk, D, S, q, q_sb, q_sh, k, k_sb, k_sh, k_ss, v, v_sb, v_sh, v_ss, nullptr, 0, 0,
                     nullptr, 0, 0, nullptr, 0, 0, nullptr, scaling, 0.0, out, o_sb, o_sh, nullptr, nullptr, workspace,
                     workspace_bytes, num_splits, stream, k_new ? &ap : nullptr, const_cast<float*>(acc), a_sb, a_sh,
                     &ev);
}

// ---------------------------------------------------------------------------
// Allocation-free fused append + decode, for callers that cannot allocate
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  It is hc_decode_attn_append with the split partials kept in a
// static device array instead of a caller-owned workspace:
//   * the array (kNoAllocScratchBytes) lives in the library's code object, so
//     every GPU the library runs on holds its own copy until the process ends;
//   * its device address is taken once per device with hipGetSymbolAddress
//     (on the first call on that device, with that device current) and only
//     that address is passed to the kernels -- the array's name in host code
//     is a host-side stand-in, not device memory;
//   * every call on one GPU shares that GPU's array and leaves its contents
//     behind: the split partials are fully written before they are read, so
//     nothing is cleared, and two calls that may overlap on one GPU (two
//     streams) race on it;
//   * a call whose partials would not fit is refused (HC_ERR_WORKSPACE), and
//     no call allocates or frees memory.
// ---------------------------------------------------------------------------
namespace hc {
constexpr int64_t kNoAllocScratchBytes = (int64_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxScratchDevices = 64;
static void* g_scratch_ptr[kMaxScratchDevices];
static std::mutex g_scratch_mu;

// Device address of the current device's scratch array, taken on first use.
static int scratch_address(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(HC_ERR_HIP, "decode_append_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  HC_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, "decode_append_noalloc: device %d out of range", dev);
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess)
      return set_error(HC_ERR_HIP, "decode_append_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
    HC_REQUIRE(sdev == dev, "decode_append_noalloc: the stream belongs to device %d, the current device is %d",
               (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(HC_ERR_HIP, "decode_append_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return HC_OK;
}
}  // namespace hc

extern "C" int hc_decode_attn_append_noalloc(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
                                             const void* q, int64_t q_sb, int64_t q_sh,
                                             void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                                             void* v, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                                             const void* k_new, int64_t kn_sb, int64_t kn_sh,
                                             const void* v_new, int64_t vn_sb, int64_t vn_sh,
                                             const void* p_new, int64_t pn_sb, int64_t pn_sh,
                                             void* p_dst, int64_t pd_sb, int64_t pd_sh, int64_t pd_ss,
                                             const int64_t* pos_new, int64_t posn_sb, int64_t* pos_dst,
                                             int64_t posd_sb,
                                             const uint8_t* mask, int64_t mask_sb,
                                             int64_t held_len,
                                             const int64_t* held_pos, int64_t hp_sb, int64_t hp_sh,
                                             const uint8_t* held_valid, int64_t hv_sb, int64_t hv_sh,
                                             const int64_t* cur_pos,
                                             double scaling,
                                             void* out, int64_t o_sb, int64_t o_sh,
                                             int64_t num_splits, void* stream) {
  HC_REQUIRE(dtype == HC_DTYPE_F32 || dtype == HC_DTYPE_F16 || dtype == HC_DTYPE_BF16,
             "decode_append_noalloc: bad dtype %d", dtype);
  HC_REQUIRE(B > 0 && Hq > 0 && Hk > 0 && D > 0 && S > 0 && Hq % Hk == 0,
             "decode_append_noalloc: bad shape B=%lld Hq=%lld Hk=%lld D=%lld S=%lld", (long long)B, (long long)Hq,
             (long long)Hk, (long long)D, (long long)S);
  // The partials this launch needs, against the array's fixed size.
  const bool bitmap = mask != nullptr || held_len > 0;
  const int splits = decode_splits(dtype_size(dtype), B, Hq, Hk, D, S - 1, num_splits, bitmap);
  const int64_t need = decode_layout(B, Hq, Hk, D, S, splits, 0).total;
  if (need > kNoAllocScratchBytes)
    return set_error(HC_ERR_WORKSPACE,
                     "decode_append_noalloc: %d key splits over %lld (batch, kv head) units need %lld bytes of "
                     "scratch, above the static maximum of %lld bytes; use fewer splits or hc_decode_attn_append",
                     splits, (long long)(B * Hk), (long long)need, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  int rc = scratch_address(stream, &ws);
  if (rc != HC_OK) return rc;
  return hc_decode_attn_append(dtype, B, Hq, Hk, D, S, q, q_sb, q_sh, k, k_sb, k_sh, k_ss, v, v_sb, v_sh, v_ss,
                               k_new, kn_sb, kn_sh, v_new, vn_sb, vn_sh, p_new, pn_sb, pn_sh, p_dst, pd_sb, pd_sh,
                               pd_ss, pos_new, posn_sb, pos_dst, posd_sb, mask, mask_sb, held_len, held_pos, hp_sb,
                               hp_sh, held_valid, hv_sb, hv_sh, cur_pos, scaling, out, o_sb, o_sh, ws,
                               kNoAllocScratchBytes, num_splits, stream);
}
