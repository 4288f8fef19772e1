// Device side of the GQA decode attention (hc_decode.hip holds the host
// side and the C ABI).  The kernel templates are instantiated once per
// element type in hc_decode_{f16,bf16,f32}.hip, so the three compile in
// parallel.
//
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
//     without touching memory; every ring load is unconditional, which lets
//     the compiler keep the whole ring in flight (exact vmcnt waits).  The
//     split's rows are dealt out evenly over the waves (whole tiles, then
//     one partial tile each), so the waves finish together;
//   * Q.K^T on MFMA: v_mfma_f32_16x16x32_{f16,bf16} with the 16 key rows of a
//     tile as the A operand and the G (<=16) query heads as the B operand;
//     fp32 inputs use v_mfma_f32_16x16x4f32;
//   * online softmax in the log2 domain (exp2), fp32, with a lazy
//     reference max: the accumulators are rescaled only when a tile's max
//     exceeds the reference by more than 8 in the log2 domain (a factor of
//     2^8);
//   * P.V on MFMA for f16/bf16 (v_mfma_f32_16x16x16_{f16,bf16}): the Q.K^T
//     output leaves lane (r, c) holding p for keys 4r..4r+3 of head c, which
//     is exactly its B-operand share, and its four V rows give the A operand
//     (a byte permute per register), so no lane exchanges data; for bf16, P
//     enters as a high and a low part (two MFMAs per block, a 16-bit
//     mantissa), for f16 rounded once; the softmax sum uses the same values.
//     fp32 inputs use the VALU (16 lanes per V row, fp32 FMAs);
//   * the attention mask and the held slot's valid & (pos <= cur) test are
//     evaluated once per workgroup into an LDS bitmap;
//   * split partials (m, l, acc) are merged by the last workgroup of each
//     (batch, kv head) to finish, through device-coherent stores, an arrival
//     counter and device-coherent loads issued together; launches with many
//     workgroups merge them in a second, one-pass kernel instead;
//   * the fused append's token is loaded, attended and stored by the one
//     wave that owns it, so no other wave spends load slots or registers on
//     it.
#pragma once
#include "hc_common.h"
#include <stddef.h>
#include <algorithm>
#include <type_traits>


namespace hc {

struct DecodeArgs {
  // Bytes 0-127 (one 128-byte line of the argument memory): what the first
  // K/V tile's and q's loads need, so both leave after one batch of scalar
  // loads.  Bytes 128-255: the rest of the prologue's fields (the fused
  // append's token rows, the keep bitmap's mask and held length), one more
  // line.
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
  // Fused append (hc_decode_attn_append): the token at row S-1 comes from
  // k_new / v_new ([B][Hk][D]); the last split's workgroup attends it and
  // writes it (and optionally its pre-RoPE key and position) into row S-1.
  const void* k_new;
  int64_t kn_sb, kn_sh;
  const void* v_new;
  int64_t vn_sb, vn_sh;
  const void* p_new;
  int64_t pn_sb, pn_sh;
  const int64_t* pos_new;
  int64_t posn_sb;
  const uint8_t* mask;
  int64_t mask_sb;
  int64_t held_len;
  const int64_t* cur_pos;
  // Read after the first tile's loads have left.
  const int64_t* held_pos;
  int64_t hp_sb, hp_sh;
  const uint8_t* held_valid;
  int64_t hv_sb, hv_sh;
  void* out;
  int64_t o_sb, o_sh;
  float* part;         // [units][splits][G*D + 2*G] split partials (splits > 1)
  float* scores;       // optional [B][Hq][S] log2-domain logits (eviction score)
  float* ml;           // optional [B][Hq][2] final (max, sum)
  void* p_dst;         // fused append: the pre-RoPE key's and position's destinations
  int64_t pd_sb, pd_sh, pd_ss;
  int64_t* pos_dst;
  int64_t posd_sb;
  // In-kernel merge of the split partials (splits > 1): one arrival word
  // per (b, kv head), [launch tag : 32 | done : 1 | arrivals : 31], any
  // initial contents; NULL = a second merge kernel.  epoch is this launch's
  // tag, prev_epoch the tag the words were left under by the workspace's
  // previous launch (epoch itself if not known).
  unsigned long long* counters;
  uint32_t epoch, prev_epoch;
};
static_assert(offsetof(DecodeArgs, Hq) + sizeof(int) <= 128, "the first loads' fields must fit bytes 0-127");
static_assert(offsetof(DecodeArgs, B) == 128 && offsetof(DecodeArgs, cur_pos) + sizeof(void*) <= 256,
              "the prologue's other fields must fit bytes 128-255");

// Keys of one split when the keep bitmap is needed (mask or held slot).
constexpr int kMaxBitmapKeys = 16384;

// Online softmax with a lazy reference: a tile moves the reference (and
// rescales the accumulators) only when its max exceeds the reference by more
// than this many log2 units, so the probabilities stay below 2^8 -- well
// inside the f16/bf16 range of the rounded P -- and most tiles skip the
// rescale.  The (m, l, acc) partials are exact for whatever reference they
// carry, so every merge below is unchanged.
constexpr float kLazyLog2 = 8.0f;

// exp2 on the hardware instruction: every argument here is <= 8 (a logit
// minus a reference at most 8 below it), where v_exp_f32 needs none of
// exp2f's range scaling; -inf gives 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Reductions over the four 16-lane rows of a wave (lanes c, c+16, c+32,
// c+48), on gfx950's row-swap permutes instead of LDS-routed shuffles.  With
// both operands equal, v_permlane16_swap leaves rows (0,1) of the pair
// holding (r0, r1) and rows (2,3) holding (r2, r3); v_permlane32_swap then
// pairs the two halves.  Every lane ends with the same value, combined in
// the same order.
__device__ __forceinline__ float rows_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}
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
  const float tm = rows_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
  const bool bump = tm > st.m_run + kLazyLog2;  // false for an all-masked tile
  const float m_new = bump ? tm : st.m_run;
  const bool dead = (m_new == -INFINITY);
  const float alpha = bump ? fast_exp2(st.m_run - m_new) : 1.f;
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = dead ? 0.f : fast_exp2(s[i] - m_new);
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
  __device__ static uint32_t bits(float x, float& r) {
    const half_t h = (half_t)x;
    r = (float)h;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
  }
};

template <>
struct MxOps<bf16_t> {
  typedef short vec4 __attribute__((ext_vector_type(4)));
  __device__ static floatx4 mma(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(vec4, u32x2{a0, a1}),
                                                    __builtin_bit_cast(vec4, u32x2{b0, b1}), c, 0, 0, 0);
  }
  __device__ static uint32_t bits(float x, float& r) {
    const bf16_t h = (bf16_t)x;
    r = (float)h;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
  }
};

// Probabilities for the P.V MFMA's B operand, packed in pairs.  For bf16
// (8-bit mantissa) each p enters as a high and a low part, hi = T(p) and
// lo = T(p - hi), and V.hi + V.lo (two MFMAs, fp32 accumulation) carry p
// with a 16-bit mantissa: the output's mean error is then the bf16 rounding
// of the exact result, where rounding p itself had made it 1.2-1.5 times
// that.  f16 (11-bit mantissa) rounds p once: its error stays well inside
// its tolerance, and the second MFMA would cost the 32-layer launch about
// 2%.  r returns the value each product uses (hi + lo, or the rounded p),
// for the softmax sum.
template <typename T>
struct PSplit {
  static constexpr bool kTwo = std::is_same<T, bf16_t>::value;
};
template <typename T>
__device__ __forceinline__ void split2(float x, float y, uint32_t& hi, uint32_t& lo, float& rx, float& ry) {
  float hx, hy;
  const uint32_t bx = MxOps<T>::bits(x, hx), by = MxOps<T>::bits(y, hy);
  hi = bx | (by << 16);
  if constexpr (PSplit<T>::kTwo) {
    float lx, ly;
    const uint32_t cx = MxOps<T>::bits(x - hx, lx), cy = MxOps<T>::bits(y - hy, ly);
    lo = cx | (cy << 16);
    rx = hx + lx;
    ry = hy + ly;
  } else {
    lo = 0u;
    rx = hx;
    ry = hy;
  }
}

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
  const float tm = rows_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
  const bool bump = tm > st.m_run + kLazyLog2;  // false for an all-masked tile
  const float m_new = bump ? tm : st.m_run;
  const bool dead = (m_new == -INFINITY);
  const float alpha = bump ? fast_exp2(st.m_run - m_new) : 1.f;
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = dead ? 0.f : fast_exp2(s[i] - m_new);
  float pr[4];
  uint32_t b0, b1, e0, e1;
  split2<T>(p[0], p[1], b0, e0, pr[0], pr[1]);
  split2<T>(p[2], p[3], b1, e1, pr[2], pr[3]);
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
    if constexpr (PSplit<T>::kTwo) st.acc[j] = MxOps<T>::mma(a0, a1, e0, e1, st.acc[j]);
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

// Device-coherent (agent-scope) accesses of the split partials merged in
// the decode kernel itself: they bypass the per-XCD caches' incoherence.
__device__ __forceinline__ void store_agent(float* p, float x) {
  __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merge the split partials (m, l, acc) of unit (b, hk) and write the output
// rows, plus the final (max, sum) when a.ml is set.  The partials of up to
// eight splits are loaded before any is used, so their loads are in flight
// together (loaded and used one split at a time, each load had waited for
// the one before: 1.2 us more per launch at five splits); they are then
// combined by online rescaling.  Threads tid, tid + nthreads, ... take the
// unit's G*D output elements.
template <typename T, bool AGENT>
__device__ __forceinline__ void merge_partials(const DecodeArgs& a, int b, int hk, int D, int tid, int nthreads) {
  constexpr int kChunk = 8;
  const int G = a.G;
  const int unit = b * a.Hk + hk;
  const int stride_part = G * D + 2 * G;
  const float* pu = a.part + (int64_t)unit * a.splits * stride_part;
  T* obase = reinterpret_cast<T*>(a.out) + b * a.o_sb + (int64_t)(hk * G) * a.o_sh;
  for (int e = tid; e < G * D; e += nthreads) {
    const int g = e / D, d = e - g * D;
    float M = -INFINITY, A = 0.f, L = 0.f;
    for (int s0 = 0; s0 < a.splits; s0 += kChunk) {
      float ms[kChunk], as[kChunk], ls[kChunk];
#pragma unroll
      for (int j = 0; j < kChunk; ++j) {
        const float* ps = pu + min(s0 + j, a.splits - 1) * stride_part;
        ms[j] = AGENT ? load_agent(ps + G * D + g) : ps[G * D + g];
        as[j] = AGENT ? load_agent(ps + e) : ps[e];
        ls[j] = AGENT ? load_agent(ps + G * D + G + g) : ps[G * D + G + g];
      }
#pragma unroll
      for (int j = 0; j < kChunk; ++j) {
        const float Mn = fmaxf(M, ms[j]);
        if (s0 + j < a.splits && Mn != -INFINITY) {
          const float c0 = fast_exp2(M - Mn), c1 = fast_exp2(ms[j] - Mn);
          A = A * c0 + as[j] * c1;
          L = L * c0 + ls[j] * c1;
          M = Mn;
        }
      }
    }
    obase[g * a.o_sh + d] = from_f32<T>(A / L);
    if (a.ml && d == 0) {
      a.ml[((int64_t)b * a.Hq + hk * G + g) * 2 + 0] = M;
      a.ml[((int64_t)b * a.Hq + hk * G + g) * 2 + 1] = L;
    }
  }
}

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

  // Tile schedule of the split's keys [key_begin, key_end): full rounds of
  // NW 16-key tiles, wave w taking the w-th tile of each round (so the waves
  // of a workgroup read neighbouring rows at any moment), then the keys left
  // over spread evenly over the waves, one partial tile each.  Every wave
  // thus reads about the same number of rows: with whole tiles in the last
  // round, half the waves of a 36-tile unit had a tile more to wait for and
  // held the workgroup at its final barrier.  Tile t of the wave covers rows
  // [tlo(t), thi(t)); past the wave's last tile the range is empty, so the
  // ring's extra loads touch no memory.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int nkeys = max(0, key_end - key_begin);
  const int full = nkeys / (16 * NW);
  const int rem = nkeys - full * 16 * NW;
  const int cw = (rem + NW - 1) / NW;
  const bool part = wv * cw < rem;
  const int nt = full + (part ? 1 : 0);
  const int tail_lo = key_begin + full * 16 * NW + wv * cw;
  const int tail_hi = min(tail_lo + cw, key_end);
  auto tlo = [&](int t) { return t < full ? key_begin + (t * NW + wv) * 16 : (t == full && part ? tail_lo : key_end); };
  auto thi = [&](int t) {
    return t < full ? key_begin + (t * NW + wv) * 16 + 16 : (t == full && part ? tail_hi : key_end);
  };
  {
    // The ring's first tiles (NBUF-1 of them; the one tile of a depth-1
    // ring) are issued first, so their HBM round trip overlaps everything
    // else the prologue loads; the keep bitmap's bits are applied to them
    // once it is complete.
    constexpr int PRE = NBUF > 1 ? NBUF - 1 : 1;
    TileRegs<T, D> r[NBUF];
#pragma unroll
    for (int i = 0; i < PRE; ++i)
      load_tile<T, D>(r[i], krs, vrs, k_rowb, v_rowb, tlo(i), key_begin, thi(i), col, grp, nullptr);

    // q next: its fields share the tile's first argument loads, so its
    // loads leave in the same round trip (placed after the token's, they
    // had waited for a second batch of argument loads).
    QFrag<T, D> qf;
    const T* q0 = reinterpret_cast<const T*>(a.q) + b * a.q_sb + (int64_t)(hk * G) * a.q_sh;
    qf.load(make_rsrc(q0, a.q_bytes), (uint32_t)(a.q_sh * (int64_t)sizeof(T)), col, grp, G);

    // Fused append: the last wave of the last split attends the new token
    // (key S-1) as a one-key tile and copies its K/V (and pre-RoPE key and
    // position) into row S-1.  Only that wave loads it, in a wave-uniform
    // branch ahead of every load the ring waits on, so the other waves issue
    // nothing for it and the ring's load counting stays exact.  With a ring
    // of depth 2 or more the token is processed and stored before the ring,
    // which frees its registers.  With a ring of depth 1 (splits of one tile
    // per wave) it is processed after the wave's tile, whose loads (and q's)
    // leave first, and the token's stores are acknowledged together with the
    // split's partial stores.  Processed first, the token had held back the
    // tile's load until after its stores, whose acknowledgement the tile's
    // wait then included: two round trips for that wave of the last split.
    bool tok = false;
    if constexpr (APPEND) tok = split == a.splits - 1 && wv == NW - 1;
    TileRegs<T, D> rn;
    uint32_t pw[TileRegs<T, D>::KW][4];
    uint32_t pos_w[2];
    if (APPEND && tok) {
      constexpr uint32_t rowb = D * sizeof(T);
      const T* kn = reinterpret_cast<const T*>(a.k_new) + b * a.kn_sb + hk * a.kn_sh;
      const T* vn = reinterpret_cast<const T*>(a.v_new) + b * a.vn_sb + hk * a.vn_sh;
      load_token<T, D>(rn, make_rsrc(kn, rowb), make_rsrc(vn, rowb), col, grp, true);
      const bool tp = a.p_new != nullptr;
      const T* pn = tp ? reinterpret_cast<const T*>(a.p_new) + b * a.pn_sb + hk * a.pn_sh : kbase;
      const __amdgpu_buffer_rsrc_t pnrs = make_rsrc(pn, tp ? rowb : 0u);
#pragma unroll
      for (int t = 0; t < TileRegs<T, D>::KW; ++t) {
        const int d0 = (sizeof(T) == 4) ? 16 * t + 4 * grp : 32 * t + 8 * grp;
        bload<16>(pnrs, (col == 0 && d0 < D) ? (uint32_t)(d0 * sizeof(T)) : kOob, pw[t]);
      }
      const bool tq = a.pos_new != nullptr && hk == 0;
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
      for (int base = 0; base < nkeys; base += 64 * NW) {
        const int rel = base + (int)threadIdx.x;
        const int key = key_begin + rel;
        const bool in = rel < nkeys;
        const bool held = in && key < a.held_len;
        // The mask byte and the held slot's valid byte and position are
        // each loaded only where they are read, and all of them before any
        // is tested: one round trip.  (Tested as loaded, the position's load
        // had waited for the valid byte's.)
        uint32_t mv = 1, hvv = 1;
        int64_t hpv = 0;
        if (in && mrow) mv = mrow[key];
        if (held) {
          hvv = a.held_valid[b * a.hv_sb + hk * a.hv_sh + key];
          hpv = a.held_pos[b * a.hp_sb + hk * a.hp_sh + key];
        }
        const bool kp = in && mv != 0 && (!held || (hvv != 0 && hpv <= cur));
        const unsigned long long m = __ballot(kp);
        if (lane < 2) sm_bits[((base + 64 * wave) >> 5) + lane] = lane ? (uint32_t)(m >> 32) : (uint32_t)m;
      }
      // LDS-only fences: the barrier does not wait for the ring's K/V loads.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#pragma unroll
      for (int i = 0; i < PRE; ++i) r[i].keep &= tile_keep_bits(tlo(i), key_begin, grp, sm_bits);
    }
    float* srow = EVICT ? a.scores + ((int64_t)b * a.Hq + hk * G + min(col, G - 1)) * a.S : nullptr;

    auto attend_token = [&]() {
      // with EVICT the token's logit is kept like every key's
      if constexpr (MX)
        process_tile_mx<T, D, EVICT>(rn, qf, st, G, a.scale_log2, a.S - 1, a.S, col, grp, srow);
      else
        process_tile<T, D, GM, EVICT>(rn, qf, st, G, a.scale_log2, a.S - 1, a.S, col, grp, srow);
      const uint32_t row = (uint32_t)(a.S - 1);
      store_token<T, D>(rn, krs, vrs, row * k_rowb, row * v_rowb, col, grp, true);
      const bool tp = a.p_new != nullptr;
      T* pd = tp ? reinterpret_cast<T*>(a.p_dst) + b * a.pd_sb + hk * a.pd_sh + (int64_t)row * a.pd_ss
                 : const_cast<T*>(kbase);
      const __amdgpu_buffer_rsrc_t pdrs = make_rsrc(pd, tp ? (uint32_t)(D * sizeof(T)) : 0u);
#pragma unroll
      for (int t = 0; t < TileRegs<T, D>::KW; ++t) {
        const int d0 = (sizeof(T) == 4) ? 16 * t + 4 * grp : 32 * t + 8 * grp;
        bstore<16>(pdrs, (col == 0 && d0 < D) ? (uint32_t)(d0 * sizeof(T)) : kOob, pw[t]);
      }
      const bool tq = a.pos_new != nullptr && hk == 0;
      int64_t* pdst = tq ? a.pos_dst + b * a.posd_sb + row : reinterpret_cast<int64_t*>(const_cast<T*>(kbase));
      bstore<8>(make_rsrc(pdst, tq ? 8u : 0u), lane == 0 ? 0u : kOob, pos_w);
    };
    if constexpr (NBUF > 1)
      if (APPEND && tok) attend_token();

    // Step t issues the loads of tile t + NBUF - 1 (an empty range past the
    // wave's tiles: no memory traffic) and then processes tile t, so NBUF-1
    // tiles stay in flight.  A ring of depth 1 issued tile 0 in the prologue
    // and loads tile t at step t > 0.  The loop is compiled twice, with and
    // without the keep bitmap, so launches without one carry no bitmap test
    // per key.
    auto ring = [&](auto with_bits) {
      constexpr bool WB = decltype(with_bits)::value;
      const uint32_t* bits = WB ? sm_bits : nullptr;
      for (int g0 = 0; g0 < nt; g0 += NBUF) {
#pragma unroll
        for (int j = 0; j < NBUF; ++j) {
          const int t = g0 + j;
          if constexpr (NBUF == 1) {
            if (t > 0)
              load_tile<T, D>(r[0], krs, vrs, k_rowb, v_rowb, tlo(t), key_begin, thi(t), col, grp, bits);
          } else {
            load_tile<T, D>(r[(j + NBUF - 1) % NBUF], krs, vrs, k_rowb, v_rowb, tlo(t + NBUF - 1), key_begin,
                            thi(t + NBUF - 1), col, grp, bits);
          }
          if (t < nt) {
            if constexpr (MX)
              process_tile_mx<T, D, EVICT>(r[j], qf, st, G, a.scale_log2, tlo(t), thi(t), col, grp, srow);
            else
              process_tile<T, D, GM, EVICT>(r[j], qf, st, G, a.scale_log2, tlo(t), thi(t), col, grp, srow);
          }
        }
      }
    };
    if (use_bits)
      ring(std::true_type{});
    else
      ring(std::false_type{});
    if constexpr (NBUF == 1)
      if (APPEND && tok) attend_token();
  }

  // ---- reduce the four row groups of the wave (they share m_run) ----
  const float l_run = rows_sum(st.l_run);
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
        st.acc[g][j] = rows_sum(st.acc[g][j]);
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

  const bool in_kernel_merge = a.splits > 1 && a.counters != nullptr;
  float* pp = a.part + ((int64_t)unit * a.splits + split) * stride_part;
  for (int e = threadIdx.x; e < G * D; e += 64 * NW) {
    const int g = e / D, d = e - g * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm_m[w][g]);
    float A = 0.f, L = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float sc = fast_exp2(sm_m[w][g] - M);
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
    } else if (in_kernel_merge) {
      store_agent(pp + e, A);
      if (d == 0) {
        store_agent(pp + G * D + g, M);
        store_agent(pp + G * D + G + g, L);
      }
    } else {
      pp[e] = A;
      if (d == 0) {
        pp[G * D + g] = M;
        pp[G * D + G + g] = L;
      }
    }
  }
  if (in_kernel_merge) {
    // The last workgroup of the unit to arrive merges every split's partial.
    // Partials are written and read with agent-scope (device-coherent)
    // accesses, so no L2 write-back or invalidation is needed: each thread
    // waits until its stores have completed, the workgroup's arrival is
    // counted after that, and the merging workgroup reads only after it has
    // seen every other arrival.  The ordering between the partials and the
    // count rests on those completed stores, not on release/acquire, so it
    // is outside the HIP memory model's guarantees: it relies on gfx950's
    // agent-scope stores having reached the device-coherent level once the
    // vmcnt wait returns, and on agent-scope loads reading that level.  A
    // release on the count (it writes back the XCD's whole L2) with an
    // acquire in the merger gives the same outputs and costs 1.5 us per
    // launch of one 8k layer (7.75 against 9.3 us cold, replayed graph).
    //
    // Arrival words.  A merging workgroup leaves its unit's word as
    // (tag, done, 0).  The next launch on the workspace passes that tag as
    // prev_epoch, and its arrivals count on the word as it is: one atomic
    // add each.  Counts are this launch's only in a word under prev_epoch
    // with the done bit (what a finished launch left), under this launch's
    // own tag with the done bit (left by this same launch, replayed from a
    // captured graph), or under its own tag without it (registered by this
    // launch, below).  An arrival that finds anything else (garbage, a
    // count an unfinished launch left behind, a tag the host no longer
    // knows) re-registers the word with a compare-and-swap as (tag, 1), so
    // no stale count can make a workgroup merge early.  Every failed swap
    // means another workgroup of the unit changed the word (at most twice
    // each), so the loop is bounded by 2 * splits + 1 rounds.
    __shared__ uint32_t sm_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    unsigned long long* word = a.counters + unit;
    constexpr unsigned long long kHi = 0xffffffff00000000ull, kDone = 0x80000000ull;
    const unsigned long long tag = (unsigned long long)a.epoch << 32;
    const unsigned long long prev = (unsigned long long)a.prev_epoch << 32;
    if (threadIdx.x == 0) {
      const auto counting = [&](unsigned long long w) {
        return (w & kDone) ? ((w & kHi) == prev || (w & kHi) == tag) : ((w & kHi) == tag);
      };
      const unsigned long long old = __hip_atomic_fetch_add(word, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      unsigned long long mine = old + 1;
      if (!counting(old)) {
        mine = 0;
        unsigned long long cur = old + 1;
        for (int round = 0; round <= 2 * a.splits; ++round) {
          const unsigned long long want = counting(cur) ? cur + 1 : (tag | 1ull);
          if (__hip_atomic_compare_exchange_strong(word, &cur, want, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT)) {
            mine = want;
            break;
          }
        }
      }
      sm_last = (uint32_t)(mine & 0x7fffffffull) == (uint32_t)a.splits;
    }
    __syncthreads();
    if (sm_last) {
      merge_partials<T, true>(a, b, hk, D, threadIdx.x, 64 * NW);
      if (threadIdx.x == 0) __hip_atomic_store(word, tag | kDone, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// grid (Hk, B), block 256: the split partials merged by a second kernel
// (launches whose units have no arrival counter).
template <typename T>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeArgs a, int D) {
  merge_partials<T, false>(a, blockIdx.y, blockIdx.x, D, threadIdx.x, blockDim.x);
}

// Launch shape of one (element size, head_dim, group bucket) instance:
//   nbuf  depth of the per-wave K/V register ring (tiles in flight + 1);
//   minw  waves per SIMD the register budget is sized for (2: <= 256 VGPRs,
//         1: up to 512 with the accumulation registers);
//   nw    waves per workgroup (8 needs minw 2 and an epilogue of at most
//         32 KB LDS, nw*gm*D floats).
// Chosen so that no f16/bf16 instance spills (checked with the compiler's
// kernel-resource-usage report).  The fp32 instances keep P.V on the VALU,
// GM * D / 16 accumulators per lane, and from D = 64 on (D = 128 with
// groups of 16) they spill 48-968 bytes per lane to scratch; fp32 caches
// are a correctness path, not a speed one.
struct DecodeCfg {
  int nbuf, minw, nw;
};

constexpr DecodeCfg decode_cfg(int es, int D, int gm) {
  int nbuf = 2, minw = 1;
  if (es == 2) {
    // MFMA P.V: the accumulators do not grow with the group.  A ring of
    // depth 1 (each wave's next tile loaded when its last is done; the
    // workgroup's other waves overlap the loads), with the first tile issued
    // ahead of q and the token, measured fastest at every launch shape: the
    // 32-layer 8k launch 15.3 against 15.9 us with depth 2, and 0.6-3% at
    // the 16k, 32k x 16 and 64k x 4 launches.
    if (D <= 128) { nbuf = 1; minw = 2; }
  } else if (D <= 32) {
    nbuf = 4; minw = 2;
  } else if (D == 64) {
    nbuf = gm >= 16 ? 2 : 4; minw = 2;
  }
  const int nw = (minw == 2 && gm * D <= 1024) ? 8 : 4;
  return DecodeCfg{nbuf, minw, nw};
}

static int group_bucket(int64_t G) { return G <= 4 ? 4 : (G <= 8 ? 8 : 16); }

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
  if (a.splits > 1 && a.counters == nullptr)
    hipLaunchKernelGGL(decode_combine_kernel<T>, dim3(a.Hk, a.B), dim3(256), 0, st, a, D);
}

template <typename T, int D, int GM>
static void launch_nw(const DecodeArgs& a, int nw, hipStream_t st) {
  constexpr DecodeCfg c = decode_cfg((int)sizeof(T), D, GM);
  (void)nw;  // equals c.nw: the host picked the shape for it
  // Splits of at most one tile per wave (latency-bound launches of a few
  // units, e.g. one layer at batch 1) run with a ring of depth 1 at every
  // element type: nothing follows the tile.
  if constexpr (c.nbuf > 1) {
    if (a.keys_per_split <= 16 * c.nw) {
      launch_decode<T, D, GM, c.nw, 1, c.minw>(a, st);
      return;
    }
  }
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

// One instantiation per element type (hc_decode_<type>.hip).
int decode_dispatch_f16(int64_t D, const DecodeArgs& a, int nw, hipStream_t st);
int decode_dispatch_bf16(int64_t D, const DecodeArgs& a, int nw, hipStream_t st);
int decode_dispatch_f32(int64_t D, const DecodeArgs& a, int nw, hipStream_t st);

}  // namespace hc
