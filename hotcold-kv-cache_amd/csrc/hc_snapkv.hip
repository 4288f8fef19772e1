// SnapKV window scoring: GQA query mean, window logits, softmax over keys,
// sum over the window, 1-D pooling.  Replaces snapkv_importance
// (src/hotcold_kv/baselines/scoring.py:50-79) with _group_query_to_kv
// (scoring.py:17-26) and pool1d (scoring.py:40-47), and the raw-logit scoring
// of HotColdLayer._compress_if_needed (src/hotcold_kv/cache.py:55-69).
//
// The scores are defined bit-for-bit so that kept indices are reproducible:
//   qf[w][d]  = (sum_g (double)q_g[w][d]) / G                  (fp64, g ascending)
//   dot[w][s] = fma chain over d ascending of qf[w][d]*(double)k[s][d] from 0.0
//   L[w][s]   = (float)(dot * scaling)     SNAPKV, -inf where s > S-W+w
//             = (float)(dot / sqrt(D))     RAWSUM (cache.py:68)
//   SNAPKV:  m_w = max_s L;  e = det_exp((double)L - (double)m_w)
//            l_w = 2^-44 * sum_s round(e * 2^44)   (exact uint64 sum)
//            imp[s] = (float)(fma chain over w ascending of e * (1/l_w))
//   RAWSUM:  imp[s] = (float)(sum over w ascending of (double)L)
//   pooled[s] = max (or fp64 sum / k) of imp over [s-k/2, s+k/2] within [0,S)
// The integer normaliser makes the softmax sum independent of how keys are
// split over workgroups, so the GPU needs no fixed reduction tree.
//
// Kernels (one stream, in order):
//   qmean   -> qf (fp64 [B][Hk][Wpad][D], rows >= W zeroed)
//   logits  -> L (fp32 [B][Hk][W][S]) + row max (atomicMax on order keys)
//   rowsum  -> l_w (uint64, 64-bit atomics)            [SNAPKV only]
//   imp     -> pooled fp32 scores [B][Hk][S]
#include "hc_common.h"

namespace hc {

constexpr int kChunkM = 128;  // keys per logits workgroup (4 waves x 32 keys)
constexpr int kRowBlk = 32;   // window rows per logits workgroup up to a window of 32
constexpr int kRowBlkWide = 64;  // ... and for longer windows

// Window rows per logits workgroup: a window of up to 32 rows in one block
// of 32; longer windows in blocks of 64, so each key slice is loaded and
// converted once for twice the matrix work (with blocks of 32 a window of 64
// read every key twice: 2.4 GB of fetch for 1.07 GB of keys at 32k x 16).
static int64_t row_block(int64_t W) { return W > kRowBlk ? kRowBlkWide : kRowBlk; }
constexpr int kMaxPool = 32;  // max half-width of the pooling window

struct ScoreLayout {
  int64_t wpad, nchunk_m, qf_off, logits_off, rmax_off, rstat_off, total;
};

// Per window row, for the importance pass: the row max and 1/l_w in fp64.
// Rows are padded to a multiple of kStatPad per (b, h); the padding rows hold
// {+inf, 0}, so they add an exact zero to the importance chain.
struct RowStat {
  double m, inv;
};
constexpr int kStatPad = 16;

static int64_t al256(int64_t x) { return (x + 255) & ~(int64_t)255; }

static ScoreLayout score_layout(int64_t B, int64_t Hk, int64_t S, int64_t D, int64_t W) {
  ScoreLayout L;
  L.wpad = cdiv(W, row_block(W)) * row_block(W);
  L.nchunk_m = cdiv(S, kChunkM);
  L.qf_off = 0;
  L.logits_off = al256(L.qf_off + B * Hk * L.wpad * D * 8);
  L.rmax_off = al256(L.logits_off + B * Hk * W * S * 4);
  L.rstat_off = al256(L.rmax_off + B * Hk * W * 4);
  L.total = al256(L.rstat_off + B * Hk * cdiv(W, kStatPad) * kStatPad * (int64_t)sizeof(RowStat));
  return L;
}

// qf[b][h][w][d] for w < wpad (zero rows past W).  grid (wpad, Hk, B), block D.
// Also resets the row-max keys (to the key of -inf) that the logits kernel
// accumulates into, and writes the padding rows of the row statistics.
// q_rows (may be NULL): row b's queries start at q_rows[b] instead of q + b*q_sb.
template <typename T>
__global__ void qmean_kernel(const T* __restrict__ q, const T* const* __restrict__ q_rows, int64_t q_sb,
                             int64_t q_sh, int64_t q_ss, int64_t q_row0, int Hq, int Hk, int W, int wpad, int D,
                             double* __restrict__ qf, uint32_t* __restrict__ rmax, RowStat* __restrict__ rstat) {
  const int w = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int d = threadIdx.x;
  const int wst = (int)cdiv(W, kStatPad) * kStatPad;  // wst <= wpad
  if (d == 0 && w < W) rmax[((int64_t)b * Hk + h) * W + w] = order_key(-INFINITY);
  if (d == 0 && w >= W && w < wst) rstat[((int64_t)b * Hk + h) * wst + w] = RowStat{INFINITY, 0.0};
  if (d >= D) return;
  double* dst = qf + (((int64_t)b * Hk + h) * wpad + w) * D + d;
  if (w >= W) {
    *dst = 0.0;
    return;
  }
  int g0, G;
  if (Hq % Hk == 0) {
    G = Hq / Hk;
    g0 = h * G;
  } else {  // scoring.py:26: mean over every query head, shared by all KV heads
    G = Hq;
    g0 = 0;
  }
  const T* src = (q_rows ? q_rows[b] : q + b * q_sb) + (q_row0 + w) * q_ss + d;
  double sum = to_f64(src[(int64_t)g0 * q_sh]);
  for (int g = 1; g < G; ++g) sum = sum + to_f64(src[(int64_t)(g0 + g) * q_sh]);
  *dst = sum / (double)G;
}

typedef double doublex4 __attribute__((ext_vector_type(4)));

// K operand of the fp64 MFMA.  Lane (kk, col) needs, for k-step t, the key
// element at dim 4t + kk.  2-byte types: a 16-byte load brings dims d0..d0+7
// of the lane's key row, and one byte permute with a per-lane selector
// extracts dim d0 + kk (dwords 0,1) or d0 + 4 + kk (dwords 2,3): no lane
// exchange, no dynamic register indexing.  fp32: a 4-byte load per k-step.
template <typename T>
struct KOperand;

template <>
struct KOperand<half_t> {
  static constexpr int DSTEP = 8;  // dims per load
  uint32_t w[4];
  __device__ static uint32_t sel(int kk) { return 0x0c0c0000u | ((uint32_t)(2 * kk + 1) << 8) | (uint32_t)(2 * kk); }
  // The dim offset is the load's scalar offset: no select and no add per load
  // (kOob stays past the extent, and a valid row's 16 bytes stay in the row).
  __device__ void load(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int d0, int kk) {
    (void)kk;
    bload_so<16>(r, row_off, (uint32_t)(d0 * 2), w);
  }
  __device__ double elem(int half, uint32_t sl) const {
    const uint32_t bits = half ? __builtin_amdgcn_perm(w[3], w[2], sl) : __builtin_amdgcn_perm(w[1], w[0], sl);
    return (double)(float)__builtin_bit_cast(half_t, (uint16_t)bits);
  }
};

template <>
struct KOperand<bf16_t> {
  static constexpr int DSTEP = 8;
  uint32_t w[4];
  // the element's two bytes land in the high half: the fp32 of the bf16
  __device__ static uint32_t sel(int kk) { return ((uint32_t)(2 * kk + 1) << 24) | ((uint32_t)(2 * kk) << 16) | 0x0c0cu; }
  // The dim offset is the load's scalar offset: no select and no add per load
  // (kOob stays past the extent, and a valid row's 16 bytes stay in the row).
  __device__ void load(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int d0, int kk) {
    (void)kk;
    bload_so<16>(r, row_off, (uint32_t)(d0 * 2), w);
  }
  __device__ double elem(int half, uint32_t sl) const {
    const uint32_t bits = half ? __builtin_amdgcn_perm(w[3], w[2], sl) : __builtin_amdgcn_perm(w[1], w[0], sl);
    return (double)__uint_as_float(bits);
  }
};

template <>
struct KOperand<float> {
  static constexpr int DSTEP = 4;
  uint32_t w[1];
  __device__ static uint32_t sel(int) { return 0u; }
  __device__ void load(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int d0, int kk) {
    bload<4>(r, row_off == kOob ? kOob : row_off + (uint32_t)((d0 + kk) * 4), w);
  }
  __device__ double elem(int, uint32_t) const { return (double)__uint_as_float(w[0]); }
};

// Window logits on the fp64 matrix cores.  v_mfma_f64_16x16x4f64 computes
// every output as a sequential IEEE fma chain over its four k terms in
// ascending k, so chaining the k-steps over d = 4t + k reproduces exactly the
// fma chain over ascending d that defines the scores.
//   A (16 rows x 4): lane l supplies qf[w0 + 16*nb + l%16][4t + l/16]
//   B (4 x 16 keys): lane l supplies k[key0 + 16*mb + l%16][4t + l/16]
//   D: lane l holds rows w0 + 16*nb + l/16 + 4i, key key0 + 16*mb + l%16
// grid (ceil(S / (128*cpw)), Hk * nrb, B), block 256.  The ROWS x D
// fp64 query block (ROWS = 32 or 64 window rows, 16 * NRB) is staged in LDS
// once and reused for cpw chunks of 128 keys; per chunk each wave covers 32
// keys (two 16-key blocks) x ROWS window rows (NRB 16-row blocks).  K loads are unconditional buffer loads
// ahead of use (rows past S read zeros).  With the head dim known at compile
// time (DC > 0) the dim loop is unrolled over a register ring of kKRing
// slices, kKRing - 1 of them in flight while one is multiplied, and the ring
// runs on into the next chunk; for any other head dim (DC == 0) it is a
// two-slot ping-pong over a runtime loop.  Logits are stored straight from
// the accumulators with unconditional buffer stores (masked lanes address
// kOob), so the compiler's vmcnt waits for the ring never have to drain the
// stores.  The LDS q block (33 KB at D = 128) allows four workgroups per CU;
// the occupancy ceiling of 4 tells the scheduler not to trade the ring's
// registers for occupancy it cannot get.  The host sets the chunks per
// workgroup (cpw, up to kLogitChunks) to leave about four workgroups per CU:
// 16 at the 8k, 32-layer batch (one round of 1024 workgroups), 1 for one
// 8k layer.
constexpr int kLogitChunks = 16;
constexpr int kNeverRead = 512;  // > the 256 (rowsum) and 270 (imp_pool) read margins
constexpr int kLogitTargetWg = 1024;
constexpr int kKRing = 4;

template <typename T, int MODE, int DC, int NRB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, NRB == 2 ? 4 : 2))) void logits_kernel(
    const T* __restrict__ k, const T* const* __restrict__ k_rows, int64_t k_sb, int64_t k_sh, int64_t k_ss,
    uint32_t k_bytes, const double* __restrict__ qf, int Hk, int S, int Drt, int W, int wpad, double scaling,
    int cpw, float* __restrict__ logits, uint32_t* __restrict__ rmax) {
  constexpr int ROWS = 16 * NRB;  // window rows of the workgroup: NRB 16-row MFMA blocks
  const int D = DC > 0 ? DC : Drt;
  extern __shared__ double sq[];  // [ROWS][D + 1] window-row block of qf
  __shared__ float red[4][ROWS];
  const int nrb = wpad / ROWS;
  // Workgroup -> (row block, key range, head), row block fastest.  The
  // hardware hands consecutive workgroups to the eight XCDs in turn; with a
  // window as long as the prompt, a key range's work grows with the row
  // block (the causal skip), so a key range fixed per XCD (key range
  // fastest) loads the XCDs unevenly -- 6.6x between the first and the last
  // of four ranges at an 8k prompt.  Row blocks in turn spread every range
  // over all XCDs.  Heavy workgroups go first (last row block, last key
  // range) so the last round is not all heavy ones.
  const int nx = (int)gridDim.x;
  const int f = (int)blockIdx.x + nx * (int)blockIdx.y;
  const int rb = nrb - 1 - f % nrb;
  const int xr = nx - 1 - (f / nrb) % nx;
  const int h = f / (nrb * nx);
  const int b = blockIdx.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, kk = lane >> 4;
  const int w0 = rb * ROWS;
  const int nw = min(ROWS, W - w0);
  const int64_t bh = (int64_t)b * Hk + h;
  const int ld = D + 1;
  // k_rows (may be NULL): row b's keys start at k_rows[b] instead of k + b*k_sb
  const T* krow = k_rows ? k_rows[b] : k + b * k_sb;
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(krow + h * k_sh, k_bytes);
  const uint32_t rowb = (uint32_t)(k_ss * (int64_t)sizeof(T));
  constexpr int DS = KOperand<T>::DSTEP;
  const int qpos0 = S - W + w0;
  const uint32_t sl = KOperand<T>::sel(kk);
  const double* qrow = sq + col * ld + kk;  // row 16 i + col of the block at qrow + 16 i ld
  // this (b, h)'s W x S logits; W * S * 4 < 2^31 is checked by the host
  const __amdgpu_buffer_rsrc_t lrs = make_rsrc(logits + bh * W * S, (uint32_t)((int64_t)W * S * 4));
  float mrow[4 * NRB];
#pragma unroll
  for (int j = 0; j < 4 * NRB; ++j) mrow[j] = -INFINITY;

  constexpr int NS = DC / DS;  // dim slices per key chunk (compile-time D)
  // the ring runs on into the next chunk: slice s of every chunk must land in
  // slot s % kKRing, so the slices per chunk are a multiple of the ring
  static_assert(DC == 0 || (DC % (2 * DS) == 0 && NS % kKRing == 0), "ring must tile the slices of a chunk");
  // Logits more than kNeverRead keys past their row's position are never read
  // (rowsum reads row w up to key S - W + w + 256, imp_pool reads key s from
  // rows whose position is at least s - 270): a workgroup wholly past that
  // line has nothing to do, and one wholly past its rows' positions has
  // nothing to multiply (no q block to stage).
  const int wg_key0 = xr * (kChunkM * cpw);
  if constexpr (MODE == HC_SCORE_SNAPKV)
    if (wg_key0 > qpos0 + nw - 1 + kNeverRead) return;  // workgroup-uniform
  const bool stage = MODE != HC_SCORE_SNAPKV || wg_key0 <= qpos0 + nw - 1;
  KOperand<T> ka[kKRing], kb[kKRing];
  int key0 = wg_key0 + wave * 32;
  uint32_t off0 = key0 + col < S ? (uint32_t)(key0 + col) * rowb : kOob;
  uint32_t off1 = key0 + 16 + col < S ? (uint32_t)(key0 + 16 + col) * rowb : kOob;
  // first K slices in flight before the q block is staged
  if constexpr (DC > 0) {
#pragma unroll
    for (int j = 0; j < kKRing - 1; ++j) {
      ka[j].load(krs, off0, j * DS, kk);
      kb[j].load(krs, off1, j * DS, kk);
    }
  } else {
    ka[0].load(krs, off0, 0, kk);
    kb[0].load(krs, off1, 0, kk);
  }
  const double* qsrc = qf + (bh * wpad + w0) * D;
  if (stage)
    for (int i = threadIdx.x; i < ROWS * D; i += 256) sq[(i / D) * ld + (i % D)] = qsrc[i];
  __syncthreads();

  // wave-uniform chunk count: short prompts stop at their last chunk
  const int nch = key0 < S ? min(cpw, (S - key0 + kChunkM - 1) / kChunkM) : 0;
  // Chunks whose 32 keys all lie after every row's position are wholly masked
  // (a window as long as the prompt, H2O); keys only grow, so they are the
  // last nch - nmul chunks: stored as -inf below, no MFMA.
  int nmul = nch;
  if constexpr (MODE == HC_SCORE_SNAPKV) {
    const int last = qpos0 + nw - 1;  // the last row's position
    nmul = key0 > last ? 0 : min(nch, (last - key0) / kChunkM + 1);
  }
  for (int c = 0; c < nmul; ++c) {
    // the q reads repeat for every chunk; keep them inside the loop (hoisted,
    // all D/2 of them would hold 2*D registers for the kernel's lifetime)
    __asm__ volatile("" ::: "memory");
    // acc[i][m]: rows 16 i .. of the block against key block m
    doublex4 acc[NRB][2];
#pragma unroll
    for (int i = 0; i < NRB; ++i) acc[i][0] = acc[i][1] = doublex4{0.0, 0.0, 0.0, 0.0};
    auto steps = [&](const KOperand<T>& xa, const KOperand<T>& xb, int d0) {
#pragma unroll
      for (int hf = 0; hf < DS / 4; ++hf) {  // k-steps t = d0/4 + hf
        const int d = d0 + 4 * hf;
        const double b0 = xa.elem(hf, sl);
        const double b1 = xb.elem(hf, sl);
#pragma unroll
        for (int i = 0; i < NRB; ++i) {
          const double ai = qrow[16 * i * ld + d];
          acc[i][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(ai, b0, acc[i][0], 0, 0, 0);
          acc[i][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(ai, b1, acc[i][1], 0, 0, 0);
        }
      }
    };
    // ping-pong over pairs of dim chunks (D % 16 == 0); the final pair of
    // loads targets dim 0 of this wave's rows in the next chunk
    const int nkey0 = key0 + kChunkM;
    const uint32_t noff0 = nkey0 + col < S ? (uint32_t)(nkey0 + col) * rowb : kOob;
    const uint32_t noff1 = nkey0 + 16 + col < S ? (uint32_t)(nkey0 + 16 + col) * rowb : kOob;
    if constexpr (DC > 0) {
      // slice j is multiplied while slices j+1 .. j+kKRing-1 are in flight;
      // the loads past the last slice start the next chunk's rows
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const int jl = j + kKRing - 1;
        if (jl < NS) {
          ka[jl % kKRing].load(krs, off0, jl * DS, kk);
          kb[jl % kKRing].load(krs, off1, jl * DS, kk);
        } else {
          ka[jl % kKRing].load(krs, noff0, (jl - NS) * DS, kk);
          kb[jl % kKRing].load(krs, noff1, (jl - NS) * DS, kk);
        }
        steps(ka[j % kKRing], kb[j % kKRing], j * DS);
      }
    } else {
      for (int d0 = 0; d0 < D; d0 += 2 * DS) {
        ka[1].load(krs, off0, d0 + DS, kk);
        kb[1].load(krs, off1, d0 + DS, kk);
        steps(ka[0], kb[0], d0);
        const bool last = d0 + 2 * DS >= D;
        ka[0].load(krs, last ? noff0 : off0, last ? 0 : d0 + 2 * DS, kk);
        kb[0].load(krs, last ? noff1 : off1, last ? 0 : d0 + 2 * DS, kk);
        steps(ka[1], kb[1], d0 + DS);
      }
    }

    // Epilogue: lane holds rows 16*nbk + kk + 4i for keys 16*mb + col.  The
    // 16 lanes of one row store 64 contiguous bytes and the two key blocks
    // complete the row's 128-byte segment; masked lanes store to kOob.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int nbk = 0; nbk < NRB; ++nbk) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          const double v = acc[nbk][mb][i];
          const int w = 16 * nbk + kk + 4 * i;
          const int key = key0 + 16 * mb + col;
          float L;
          if constexpr (MODE == HC_SCORE_SNAPKV) L = (key > qpos0 + w) ? -INFINITY : (float)(v * scaling);
          else L = (float)(v / scaling);
          const bool ok = key < S && w < nw;
          const uint32_t bits = __float_as_uint(L);
          bstore<4>(lrs, ok ? (uint32_t)((w0 + w) * S + key) * 4u : kOob, &bits);
          if constexpr (MODE == HC_SCORE_SNAPKV) mrow[4 * nbk + i] = fmaxf(mrow[4 * nbk + i], ok ? L : -INFINITY);
        }
      }
    }
    key0 = nkey0;
    off0 = noff0;
    off1 = noff1;
  }

  if constexpr (MODE != HC_SCORE_SNAPKV) return;
  for (int c = nmul; c < nch && key0 <= qpos0 + nw - 1 + kNeverRead; ++c) {  // wholly masked chunks
    const uint32_t ninf = __float_as_uint(-INFINITY);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int nbk = 0; nbk < NRB; ++nbk) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          const int w = 16 * nbk + kk + 4 * i;
          const int key = key0 + 16 * mb + col;
          bstore<4>(lrs, (key < S && w < nw) ? (uint32_t)((w0 + w) * S + key) * 4u : kOob, &ninf);
        }
      }
    }
    key0 += kChunkM;
  }
#pragma unroll
  for (int j = 0; j < 4 * NRB; ++j) {  // row 16*(j/4) + kk + 4*(j%4), max over the 16 key lanes
    float m = mrow[j];
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    m = fmaxf(m, __shfl_xor(m, 8, 64));
    if (col == 0) red[wave][16 * (j >> 2) + kk + 4 * (j & 3)] = m;
  }
  __syncthreads();
  if (threadIdx.x < nw) {
    const int w = threadIdx.x;
    const float m = fmaxf(fmaxf(red[0][w], red[1][w]), fmaxf(red[2][w], red[3][w]));
    atomicMax(&rmax[bh * W + w0 + w], order_key(m));
  }
}

// Inverse of order_key for non-NaN keys.
__device__ __forceinline__ float key_to_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Exact fixed-point softmax denominators.  grid (ceil(W / (4 / nsplit)), Hk,
// B), block 256: the workgroup's 4 waves cover 4 / nsplit window rows, nsplit
// waves per row, each streaming its split of the row's logits (4 keys per
// lane per step, kSumRing steps in flight) and summing rint(e * 2^44)
// exactly in uint64.  The splits of a row combine in LDS (integer addition:
// the total does not depend on the order), and the row's first wave writes
// its max and 1/l_w, l_w = (double)sum * 2^-44.  nsplit > 1 serves grids with
// too few rows to fill the GPU (one layer at batch 1).
constexpr int kSumRing = 4;
constexpr int kSumTargetWaves = 2048;

template <bool VEC>
__global__ __launch_bounds__(256) void rowsum_kernel(const float* __restrict__ logits,
                                                     const uint32_t* __restrict__ rmax, int Hk, int S, int W,
                                                     int nsplit, RowStat* __restrict__ rstat) {
  __shared__ uint64_t sm_part[4];
  // the wave index through readfirstlane: the row's buffer resource is then
  // known to be wave-uniform and lives in SGPRs (no waterfall per load)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sp = wave % nsplit;
  const int w = blockIdx.x * (4 / nsplit) + wave / nsplit;
  const bool live = w < W;  // wave-uniform; every wave reaches the barrier
  const int wr = live ? w : W - 1;
  const int64_t bh = (int64_t)blockIdx.z * Hk + blockIdx.y;
  const double md = (double)key_to_float(rmax[bh * W + wr]);
  const DetExp dexp = DetExp::load();
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(logits + (bh * W + wr) * S, (uint32_t)S * 4u);
  // this split's steps [st0, st0 + nstep) and keys [st0 * 256, kend); a wave
  // past W streams nothing (kend = 0).  The row attends keys up to its own
  // position S - W + w; later keys are -inf and add only the bias, so the
  // row's steps stop there (half the keys when the window is the prompt).
  const int nstep_all = (min(S, S - W + wr + 1) + 255) / 256;
  const int sps = (nstep_all + nsplit - 1) / nsplit;
  const int st0 = min(nstep_all, sp * sps);
  const int nstep = live ? min(nstep_all, st0 + sps) - st0 : 0;
  const int kend = min(S, (st0 + nstep) * 256);
  uint64_t acc[4] = {0, 0, 0, 0};
  uint32_t x[kSumRing][4];
  auto load = [&](uint32_t (&dst)[4], int step) {
    const int key = (st0 + step) * 256 + lane * 4;
    if constexpr (VEC) {
      bload<16>(rs, key < kend ? (uint32_t)key * 4u : kOob, dst);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) bload<4>(rs, key + e < kend ? (uint32_t)(key + e) * 4u : kOob, &dst[e]);
    }
  };
#pragma unroll
  for (int i = 0; i < kSumRing - 1; ++i) load(x[i], i);
  // each term is added with its 2^52 bias left in (keys past kend add the
  // bias alone); the 4 * nadd biases come off once, in wrapping uint64
  const int nadd = (nstep + kSumRing - 1) / kSumRing * kSumRing;
  for (int s0 = 0; s0 < nstep; s0 += kSumRing) {
#pragma unroll
    for (int j = 0; j < kSumRing; ++j) {
      load(x[(j + kSumRing - 1) % kSumRing], s0 + j + kSumRing - 1);
      const int key = (st0 + s0 + j) * 256 + lane * 4;
      if constexpr (VEC) {
        // S % 4 == 0 and kend % 4 == 0: the lane's four keys are all in range
        // or all past kend; past it the max becomes +inf, so x = -inf and the
        // term is the bias
        const double mk = key < kend ? md : INFINITY;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += dexp.fixed_biased((double)__uint_as_float(x[j][e]) - mk);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float L = key + e < kend ? __uint_as_float(x[j][e]) : -INFINITY;
          acc[e] += dexp.fixed_biased((double)L - md);
        }
      }
    }
  }
  uint64_t t = (acc[0] + acc[1]) + (acc[2] + acc[3]) - (uint64_t)(4 * nadd) * HC_FIX_BIAS;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t rl = __shfl_xor((uint32_t)t, o, 64);
    const uint32_t rh = __shfl_xor((uint32_t)(t >> 32), o, 64);
    t += ((uint64_t)rh << 32) | rl;
  }
  RowStat* out = rstat + bh * (cdiv(W, kStatPad) * kStatPad) + w;
  if (nsplit == 1) {  // uniform: no barrier
    if (live && lane == 0) *out = RowStat{md, 1.0 / ((double)t * 0x1p-44)};
    return;
  }
  if (lane == 0) sm_part[wave] = t;
  __syncthreads();
  if (live && sp == 0 && lane == 0) {
    uint64_t tot = 0;
    for (int j = 0; j < nsplit; ++j) tot += sm_part[wave + j];
    *out = RowStat{md, 1.0 / ((double)tot * 0x1p-44)};
  }
}

// Importance and pooling.  grid (ceil(S / (256 - 2P)), Hk, B), block 256:
// thread t computes imp for key c0 - P + t as the fma chain over the window
// rows in ascending order (rows streamed 8 at a time, the next 8 in flight),
// then the inner 256 - 2P threads pool over their neighbours in LDS.  Each
// row's max and 1/l_w are wave-uniform: they come through scalar loads into
// SGPRs, with no LDS staging and no per-row branch.
constexpr int kImpRows = 8;
// Windows from this many rows on take the mirrored-pair importance kernel
// when there is no pooling (chain lengths then differ by up to W rows).
constexpr int kMirrorMinW = 1024;

// One key's importance: the fma chain over rows [wbeg, W) of the logits
// column at byte offset `base` (kOob for a lane without a key).  Rows are
// streamed kImpRows at a time with the next group in flight; a group's
// logits and (scalar) row statistics are issued one group ahead.  Groups
// start at multiples of kImpRows and the statistics are padded to kStatPad
// (a multiple of 2 * kImpRows) rows.
template <int MODE>
__device__ __forceinline__ double imp_chain(__amdgpu_buffer_rsrc_t rs, uint32_t base, uint32_t rowb,
                                            const RowStat* st, int wst, int W, int wbeg, const DetExp& dexp) {
  static_assert(kStatPad % (2 * kImpRows) == 0, "statistics padding covers whole row pairs");
  auto load = [&](uint32_t (&dst)[kImpRows], RowStat (&sdst)[kImpRows], int w0) {
#pragma unroll
    for (int r = 0; r < kImpRows; ++r) {
      const int w = w0 + r;
      bload<4>(rs, base + (w < W ? (uint32_t)w * rowb : kOob), &dst[r]);
    }
    if constexpr (MODE == HC_SCORE_SNAPKV) {
      // the look-ahead past the last group re-reads the last group (unused)
      const RowStat* g = st + min(w0, wst - kImpRows);
#pragma unroll
      for (int r = 0; r < kImpRows; ++r) sdst[r] = g[r];
    }
  };
  double acc = 0.0;
  // rows [w0, w0 + kImpRows); rows past W add an exact zero: their padding
  // statistics are {+inf, 0}, so x = -inf, e = 0 and fma(0, 0, acc) = acc
  // (acc >= +0)
  auto chain = [&](const uint32_t (&x)[kImpRows], const RowStat (&sx)[kImpRows], int w0) {
#pragma unroll
    for (int r = 0; r < kImpRows; ++r) {
      const int w = w0 + r;
      const float L = __uint_as_float(x[r]);
      if constexpr (MODE == HC_SCORE_SNAPKV) {
        acc = __builtin_fma(dexp((double)L - sx[r].m), sx[r].inv, acc);
      } else {
        acc = acc + (w < W ? (double)L : 0.0);
      }
    }
  };
  uint32_t xa[kImpRows], xb[kImpRows];
  RowStat sa[kImpRows], sb[kImpRows];
  load(xa, sa, wbeg);
  for (int w0 = wbeg; w0 < W; w0 += 2 * kImpRows) {
    load(xb, sb, w0 + kImpRows);
    chain(xa, sa, w0);
    load(xa, sa, w0 + 2 * kImpRows);
    chain(xb, sb, w0 + kImpRows);
  }
  return acc;
}

// First row a chain over keys from kmin on must start at: key s is masked in
// the rows w < s - (S - W) (their position precedes s), which add exact zeros
// to acc (starting at +0), so the chain starts at the first row kmin attends,
// rounded down to a row pair.  The logits it then reads lie at most
// 255 + 2 * kImpRows - 1 = 270 keys past a row's position for a workgroup's
// 256 keys, inside what the logits kernel writes.
__device__ __forceinline__ int imp_first_row(int kmin, int S, int W) {
  return max(0, kmin - (S - W)) / (2 * kImpRows) * (2 * kImpRows);
}

template <int MODE>
__global__ __launch_bounds__(256) void imp_pool_kernel(const float* __restrict__ logits,
                                                       const RowStat* __restrict__ rstat, int Hk, int S, int W,
                                                       int P, int pooling, int ksize,
                                                       float* __restrict__ scores) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * Hk + h;
  const int out_per_block = 256 - 2 * P;
  const int c0 = blockIdx.x * out_per_block;
  __shared__ float sm_imp[256];
  const int s = c0 - P + (int)threadIdx.x;
  const bool sv = s >= 0 && s < S;
  // W * S * 4 < 2^31 (checked by the host), so every in-range offset is below
  // 2^31.  A lane outside [0, S) starts at kOob = 2^31: plus a row offset
  // (< 2^31) it stays out of range; rows past W use the row offset kOob, out
  // of range for in-range lanes (and wrapping to offset 0, a harmless read, for
  // the others, whose result is discarded).
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(logits + bh * W * S, (uint32_t)((int64_t)W * S * 4));
  const uint32_t base = sv ? (uint32_t)s * 4u : kOob;
  const int wst = (int)cdiv(W, kStatPad) * kStatPad;
  const DetExp dexp = DetExp::load();
  const int wbeg = MODE == HC_SCORE_SNAPKV ? imp_first_row(c0 - P, S, W) : 0;
  const double acc = imp_chain<MODE>(rs, base, (uint32_t)S * 4u, rstat + bh * wst, wst, W, wbeg, dexp);
  sm_imp[threadIdx.x] = sv ? (float)acc : 0.f;
  __syncthreads();
  const int t = threadIdx.x;
  if (t < P || t >= 256 - P || s >= S) return;
  float out;
  if (P == 0) {
    out = sm_imp[t];
  } else if (pooling == HC_POOL_MAX) {
    out = -INFINITY;
    for (int j = -P; j <= P; ++j) {
      const int sj = s + j;
      if (sj >= 0 && sj < S) out = fmaxf(out, sm_imp[t + j]);
    }
  } else {
    double sum = 0.0;
    for (int j = -P; j <= P; ++j) {
      const int sj = s + j;
      if (sj >= 0 && sj < S) sum = sum + (double)sm_imp[t + j];
    }
    out = (float)(sum / (double)ksize);
  }
  scores[bh * S + s] = out;
}

// Importance without pooling for long windows, keys in mirrored pairs.
// With a window as long as the prompt (H2O) key s's chain covers the S - s
// rows at or after its position, so one thread per key leaves the first
// keys' threads with thousands of rows and the last keys' with a few, and
// every chain must stay in one thread (its order is part of the scores).
// Here thread t of workgroup x owns keys a = 256x + t and S - 1 - a: every
// thread's two chains together cover about S + 1 rows.  The chains and the
// fp32 result are those of imp_pool_kernel with P = 0, bit for bit.
// grid (ceil(ceil(S / 2) / 256), Hk, B), block 256.
__global__ __launch_bounds__(256) void imp_mirror_kernel(const float* __restrict__ logits,
                                                         const RowStat* __restrict__ rstat, int Hk, int S, int W,
                                                         float* __restrict__ scores) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * Hk + h;
  const int c0 = blockIdx.x * 256;
  const int a = c0 + (int)threadIdx.x;
  const int m = S - 1 - a;                 // the mirrored key
  const bool av = a <= m, mv = a < m;      // the middle key of an odd S once
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(logits + bh * W * S, (uint32_t)((int64_t)W * S * 4));
  const uint32_t rowb = (uint32_t)S * 4u;
  const int wst = (int)cdiv(W, kStatPad) * kStatPad;
  const RowStat* st = rstat + bh * wst;
  const DetExp dexp = DetExp::load();
  const double acc_a = imp_chain<HC_SCORE_SNAPKV>(rs, av ? (uint32_t)a * 4u : kOob, rowb, st, wst, W,
                                                  imp_first_row(c0, S, W), dexp);
  // the workgroup's mirrored keys are S - 1 - c0 - 255 .. S - 1 - c0
  const double acc_m = imp_chain<HC_SCORE_SNAPKV>(rs, mv ? (uint32_t)m * 4u : kOob, rowb, st, wst, W,
                                                  imp_first_row(max(0, S - 1 - c0 - 255), S, W), dexp);
  float* out = scores + bh * S;
  if (av) out[a] = (float)acc_a;
  if (mv) out[m] = (float)acc_m;
}

// out[b][s] = (float)((sum_h (double)x[b][h][s]) / H), h ascending.
__global__ void head_mean_kernel(const float* __restrict__ x, int H, int S, float* __restrict__ out) {
  const int b = blockIdx.y;
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= S) return;
  double acc = 0.0;
  for (int h = 0; h < H; ++h) acc = acc + (double)x[((int64_t)b * H + h) * S + s];
  out[(int64_t)b * S + s] = (float)(acc / (double)H);
}

template <typename T>
static void launch_score(const ScoreLayout& lay, char* ws, int mode, int64_t B, int64_t Hq, int64_t Hk, int64_t S,
                         int64_t D, int64_t W, const void* q, const void* const* q_rows, int64_t q_sb, int64_t q_sh,
                         int64_t q_ss, int64_t q_row0, const void* k, const void* const* k_rows, int64_t k_sb,
                         int64_t k_sh, int64_t k_ss, double scal, int P, int pooling, int ksize, float* scores,
                         hipStream_t st) {
  double* qf = reinterpret_cast<double*>(ws + lay.qf_off);
  float* logits = reinterpret_cast<float*>(ws + lay.logits_off);
  uint32_t* rmax = reinterpret_cast<uint32_t*>(ws + lay.rmax_off);
  RowStat* rstat = reinterpret_cast<RowStat*>(ws + lay.rstat_off);
  const int rows = (int)row_block(W);
  const int nrb = (int)(lay.wpad / rows);
  hipLaunchKernelGGL(qmean_kernel<T>, dim3((unsigned)lay.wpad, (unsigned)Hk, (unsigned)B),
                     dim3((unsigned)(D < 64 ? 64 : D)), 0, st, (const T*)q, (const T* const*)q_rows, q_sb, q_sh,
                     q_ss, q_row0, (int)Hq,
                     (int)Hk, (int)W, (int)lay.wpad, (int)D, qf, rmax, rstat);
  const size_t lds = (size_t)(rows * (D + 1) * 8);
  const uint32_t k_bytes = (uint32_t)(((S - 1) * k_ss + D) * (int64_t)sizeof(T));
  const int64_t wg1 = cdiv(S, (int64_t)kChunkM) * Hk * nrb * B;  // workgroups at one chunk each
  const int cpw = (int)std::max<int64_t>(1, std::min<int64_t>(kLogitChunks, wg1 / kLogitTargetWg));
  const dim3 grid((unsigned)cdiv(S, (int64_t)kChunkM * cpw), (unsigned)(Hk * nrb), (unsigned)B);
  auto launch = [&](auto kern) {
    if (lds > 48 * 1024)
      (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(kern, grid, dim3(256), lds, st, (const T*)k, (const T* const*)k_rows, k_sb, k_sh, k_ss,
                       k_bytes, (const double*)qf,
                       (int)Hk, (int)S, (int)D, (int)W, (int)lay.wpad, scal, cpw, logits, rmax);
  };
  if (mode == HC_SCORE_SNAPKV) {
    if (rows == kRowBlk) {
      if (D == 128) launch(logits_kernel<T, HC_SCORE_SNAPKV, 128, 2>);
      else if (D == 64) launch(logits_kernel<T, HC_SCORE_SNAPKV, 64, 2>);
      else launch(logits_kernel<T, HC_SCORE_SNAPKV, 0, 2>);
    } else {
      if (D == 128) launch(logits_kernel<T, HC_SCORE_SNAPKV, 128, 4>);
      else if (D == 64) launch(logits_kernel<T, HC_SCORE_SNAPKV, 64, 4>);
      else launch(logits_kernel<T, HC_SCORE_SNAPKV, 0, 4>);
    }
  } else {
    // the raw sums' fp64 divides leave no registers for the unrolled ring
    if (rows == kRowBlk) launch(logits_kernel<T, HC_SCORE_RAWSUM, 0, 2>);
    else launch(logits_kernel<T, HC_SCORE_RAWSUM, 0, 4>);
  }
  if (mode == HC_SCORE_SNAPKV) {
    // rows split across the waves of a workgroup (1, 2 or 4 per row) when
    // there are too few rows to fill the GPU (about kSumTargetWaves waves)
    const int64_t rows = W * Hk * B;
    int nsplit = 1;
    while (nsplit < 4 && rows * nsplit * 2 <= kSumTargetWaves && cdiv(S, 256) >= 2 * nsplit) nsplit *= 2;
    const dim3 g((unsigned)cdiv(W, 4 / nsplit), (unsigned)Hk, (unsigned)B);
    if (S % 4 == 0)
      hipLaunchKernelGGL(rowsum_kernel<true>, g, dim3(256), 0, st, (const float*)logits, (const uint32_t*)rmax,
                         (int)Hk, (int)S, (int)W, nsplit, rstat);
    else
      hipLaunchKernelGGL(rowsum_kernel<false>, g, dim3(256), 0, st, (const float*)logits, (const uint32_t*)rmax,
                         (int)Hk, (int)S, (int)W, nsplit, rstat);
  }
  if (mode == HC_SCORE_SNAPKV && P == 0 && W >= kMirrorMinW) {
    const dim3 gm((unsigned)cdiv(cdiv(S, 2), 256), (unsigned)Hk, (unsigned)B);
    hipLaunchKernelGGL(imp_mirror_kernel, gm, dim3(256), 0, st, (const float*)logits, (const RowStat*)rstat,
                       (int)Hk, (int)S, (int)W, scores);
    return;
  }
  const dim3 gi((unsigned)cdiv(S, 256 - 2 * P), (unsigned)Hk, (unsigned)B);
  if (mode == HC_SCORE_SNAPKV)
    hipLaunchKernelGGL(imp_pool_kernel<HC_SCORE_SNAPKV>, gi, dim3(256), 0, st, (const float*)logits,
                       (const RowStat*)rstat, (int)Hk, (int)S, (int)W, P, pooling, ksize,
                       scores);
  else
    hipLaunchKernelGGL(imp_pool_kernel<HC_SCORE_RAWSUM>, gi, dim3(256), 0, st, (const float*)logits,
                       (const RowStat*)rstat, (int)Hk, (int)S, (int)W, P, pooling, ksize,
                       scores);
}

}  // namespace hc

using namespace hc;

extern "C" int64_t hc_snapkv_score_workspace_size(int64_t B, int64_t Hk, int64_t S, int64_t D, int64_t W) {
  if (B <= 0 || Hk <= 0 || S <= 0 || D <= 0 || W <= 0) return 256;
  if (W > S) W = S;
  return score_layout(B, Hk, S, D, W).total;
}

static int score_impl(int dtype, int mode, int64_t B, int64_t Hq, int64_t Hk, int64_t S, int64_t D, int64_t W,
                      const void* q, const void* const* q_rows, int64_t q_sb, int64_t q_sh, int64_t q_ss,
                      int64_t q_row0, const void* k, const void* const* k_rows, int64_t k_sb, int64_t k_sh,
                      int64_t k_ss, double scaling, int64_t kernel_size, int pooling, float* scores, void* workspace,
                      int64_t workspace_bytes, void* stream) {
  HC_REQUIRE(dtype == HC_DTYPE_F32 || dtype == HC_DTYPE_F16 || dtype == HC_DTYPE_BF16, "score: bad dtype %d", dtype);
  HC_REQUIRE(mode == HC_SCORE_SNAPKV || mode == HC_SCORE_RAWSUM, "score: bad mode %d", mode);
  HC_REQUIRE(B > 0 && Hq > 0 && Hk > 0 && S > 0 && D > 0 && W > 0, "score: empty shape");
  HC_REQUIRE(W <= S, "score: window %lld exceeds S %lld", (long long)W, (long long)S);
  HC_REQUIRE(W * S * 4 < ((int64_t)1 << 31), "score: window x keys (%lld x %lld) logits above 2 GiB per head",
             (long long)W, (long long)S);
  HC_REQUIRE(D % 16 == 0 && D <= 512, "score: head_dim %lld must be a multiple of 16 and <= 512", (long long)D);
  HC_REQUIRE(S <= ((int64_t)1 << 19), "score: S %lld above 2^19 (fixed-point normaliser range)", (long long)S);
  HC_REQUIRE(B <= 65535 && Hk * cdiv(W, row_block(W)) <= 65535, "score: grid too large");
  HC_REQUIRE(q_row0 >= 0, "score: negative q_row0");
  HC_REQUIRE((q || q_rows) && (k || k_rows) && scores, "score: null pointer");
  const int es = dtype_size(dtype);
  HC_REQUIRE(k_ss >= D && ((S - 1) * k_ss + D) * es < ((int64_t)1 << 31),
             "score: one (batch, kv head) key extent must be below 2 GiB with row stride >= D");
  HC_REQUIRE((uintptr_t)k % 16 == 0 && (k_sb * es) % 16 == 0 && (k_sh * es) % 16 == 0 && (k_ss * es) % 16 == 0,
             "score: keys must be 16-byte aligned rows");
  int P = 0;
  if (kernel_size > 1) {
    HC_REQUIRE(kernel_size % 2 == 1, "score: pooling kernel_size %lld must be odd", (long long)kernel_size);
    P = (int)(kernel_size / 2);
    HC_REQUIRE(P <= kMaxPool, "score: pooling kernel_size %lld too large", (long long)kernel_size);
    HC_REQUIRE(pooling == HC_POOL_MAX || pooling == HC_POOL_AVG, "score: bad pooling %d", pooling);
  }
  const ScoreLayout lay = score_layout(B, Hk, S, D, W);
  if (!workspace || workspace_bytes < lay.total)
    return set_error(HC_ERR_WORKSPACE, "score: workspace of %lld bytes needed, got %lld", (long long)lay.total,
                     (long long)workspace_bytes);
  HC_REQUIRE((uintptr_t)workspace % 256 == 0, "score: workspace must be 256-byte aligned");
  // RAWSUM divides by sqrt(D) like cache.py:68; the host square root is the
  // correctly rounded IEEE value.
  const double scal = (mode == HC_SCORE_SNAPKV) ? scaling : sqrt((double)D);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = reinterpret_cast<char*>(workspace);
  if (dtype == HC_DTYPE_F16)
    launch_score<half_t>(lay, ws, mode, B, Hq, Hk, S, D, W, q, q_rows, q_sb, q_sh, q_ss, q_row0, k, k_rows, k_sb,
                         k_sh, k_ss, scal, P, pooling, (int)kernel_size, scores, st);
  else if (dtype == HC_DTYPE_BF16)
    launch_score<bf16_t>(lay, ws, mode, B, Hq, Hk, S, D, W, q, q_rows, q_sb, q_sh, q_ss, q_row0, k, k_rows, k_sb,
                         k_sh, k_ss, scal, P, pooling, (int)kernel_size, scores, st);
  else
    launch_score<float>(lay, ws, mode, B, Hq, Hk, S, D, W, q, q_rows, q_sb, q_sh, q_ss, q_row0, k, k_rows, k_sb,
                        k_sh, k_ss, scal, P, pooling, (int)kernel_size, scores, st);
  return check_launch("snapkv_score");
}

extern "C" int hc_snapkv_score(int dtype, int mode, int64_t B, int64_t Hq, int64_t Hk, int64_t S, int64_t D,
                               int64_t W, const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_row0,
                               const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss, double scaling,
                               int64_t kernel_size, int pooling, float* scores, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  HC_REQUIRE(q && k, "score: null pointer");
  return score_impl(dtype, mode, B, Hq, Hk, S, D, W, q, nullptr, q_sb, q_sh, q_ss, q_row0, k, nullptr, k_sb, k_sh,
                    k_ss, scaling, kernel_size, pooling, scores, workspace, workspace_bytes, stream);
}

extern "C" int hc_snapkv_score_rows(int dtype, int mode, int64_t R, int64_t Hq, int64_t Hk, int64_t S, int64_t D,
                                    int64_t W, const void* const* q_rows, int64_t q_sh, int64_t q_ss,
                                    int64_t q_row0, const void* const* k_rows, int64_t k_sh, int64_t k_ss,
                                    double scaling, int64_t kernel_size, int pooling, float* scores,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
  HC_REQUIRE(q_rows && k_rows, "score_rows: null row table");
  return score_impl(dtype, mode, R, Hq, Hk, S, D, W, nullptr, q_rows, 0, q_sh, q_ss, q_row0, nullptr, k_rows, 0,
                    k_sh, k_ss, scaling, kernel_size, pooling, scores, workspace, workspace_bytes, stream);
}

extern "C" int hc_head_mean(int64_t B, int64_t H, int64_t S, const float* scores, float* out, void* stream) {
  HC_REQUIRE(B > 0 && H > 0 && S > 0 && scores && out, "head_mean: bad arguments");
  HC_REQUIRE(B <= 65535, "head_mean: B too large");
  hipLaunchKernelGGL(head_mean_kernel, dim3((unsigned)cdiv(S, 256), (unsigned)B), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), scores, (int)H, (int)S, out);
  return check_launch("head_mean");
}
