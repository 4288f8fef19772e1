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
constexpr int kRowBlk = 32;   // window rows per logits workgroup (fp64 accumulators)
constexpr int kSumChunk = 512;  // keys per rowsum workgroup (two per lane)
constexpr int kMaxW = 256;
constexpr int kMaxPool = 32;  // max half-width of the pooling window

struct ScoreLayout {
  int64_t wpad, nchunk_m, qf_off, logits_off, rmax_off, lsum_off, total;
};

static int64_t al256(int64_t x) { return (x + 255) & ~(int64_t)255; }

static ScoreLayout score_layout(int64_t B, int64_t Hk, int64_t S, int64_t D, int64_t W) {
  ScoreLayout L;
  L.wpad = cdiv(W, kRowBlk) * kRowBlk;
  L.nchunk_m = cdiv(S, kChunkM);
  L.qf_off = 0;
  L.logits_off = al256(L.qf_off + B * Hk * L.wpad * D * 8);
  L.rmax_off = al256(L.logits_off + B * Hk * W * S * 4);
  L.lsum_off = al256(L.rmax_off + B * Hk * W * 4);
  L.total = al256(L.lsum_off + B * Hk * W * 8);
  return L;
}

// qf[b][h][w][d] for w < wpad (zero rows past W).  grid (wpad, Hk, B), block D.
// Also resets the row-max keys (to the key of -inf) and the fixed-point
// row sums that the following kernels accumulate into.
template <typename T>
__global__ void qmean_kernel(const T* __restrict__ q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_row0,
                             int Hq, int Hk, int W, int wpad, int D, double* __restrict__ qf,
                             uint32_t* __restrict__ rmax, uint64_t* __restrict__ lsum) {
  const int w = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int d = threadIdx.x;
  if (d == 0 && w < W) {
    rmax[((int64_t)b * Hk + h) * W + w] = order_key(-INFINITY);
    lsum[((int64_t)b * Hk + h) * W + w] = 0ull;
  }
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
  const T* src = q + b * q_sb + (q_row0 + w) * q_ss + d;
  double sum = to_f64(src[(int64_t)g0 * q_sh]);
  for (int g = 1; g < G; ++g) sum = sum + to_f64(src[(int64_t)(g0 + g) * q_sh]);
  *dst = sum / (double)G;
}

// Raw 16-byte pieces of one 8-dim chunk of a key row (16-bit types: one
// piece; fp32: two).
template <typename T>
struct KChunk {
  static constexpr int N = (sizeof(T) == 4) ? 2 : 1;
  uint32_t w[4 * N];
};

template <typename T>
__device__ __forceinline__ void load_kchunk(KChunk<T>& c, const T* p, bool ok) {
#pragma unroll
  for (int i = 0; i < KChunk<T>::N; ++i) {
    u32x4 x = {0u, 0u, 0u, 0u};
    if (ok) x = ld16(reinterpret_cast<const char*>(p) + 16 * i);
    c.w[4 * i + 0] = x[0];
    c.w[4 * i + 1] = x[1];
    c.w[4 * i + 2] = x[2];
    c.w[4 * i + 3] = x[3];
  }
}

// Element j (0..7) of the chunk as an exact double, j chosen per lane.
template <typename T>
__device__ __forceinline__ double kchunk_elem(const KChunk<T>& c, int j);
template <>
__device__ __forceinline__ double kchunk_elem<half_t>(const KChunk<half_t>& c, int j) {
  const uint32_t word = (j & 4) ? ((j & 2) ? c.w[3] : c.w[2]) : ((j & 2) ? c.w[1] : c.w[0]);
  const uint16_t bits = (uint16_t)((j & 1) ? (word >> 16) : (word & 0xffffu));
  return (double)(float)__builtin_bit_cast(half_t, bits);
}
template <>
__device__ __forceinline__ double kchunk_elem<bf16_t>(const KChunk<bf16_t>& c, int j) {
  const uint32_t word = (j & 4) ? ((j & 2) ? c.w[3] : c.w[2]) : ((j & 2) ? c.w[1] : c.w[0]);
  const uint32_t bits = (j & 1) ? (word & 0xffff0000u) : (word << 16);
  return (double)__uint_as_float(bits);
}
template <>
__device__ __forceinline__ double kchunk_elem<float>(const KChunk<float>& c, int j) {
  const uint32_t lo = (j & 2) ? ((j & 1) ? c.w[3] : c.w[2]) : ((j & 1) ? c.w[1] : c.w[0]);
  const uint32_t hi = (j & 2) ? ((j & 1) ? c.w[7] : c.w[6]) : ((j & 1) ? c.w[5] : c.w[4]);
  return (double)__uint_as_float((j & 4) ? hi : lo);
}

typedef double doublex4 __attribute__((ext_vector_type(4)));

// Window logits on the fp64 matrix cores.  v_mfma_f64_16x16x4f64 computes
// every output as a sequential IEEE fma chain over its four k terms in
// ascending k, so chaining the k-steps over d = 4t + k reproduces exactly the
// fma chain over ascending d that defines the scores.
//   A (16 rows x 4): lane l supplies qf[w0 + 16*nb + l%16][4t + l/16]
//   B (4 x 16 keys): lane l supplies k[key0 + 16*mb + l%16][4t + l/16]
//   D: lane l holds rows w0 + 16*nb + l/16 + 4i, key key0 + 16*mb + l%16
// grid (ceil(S/128), Hk * nrb, B), block 256: each wave covers 32 keys
// (two 16-key blocks) x 32 window rows (two 16-row blocks).
template <typename T>
__global__ __launch_bounds__(256) void logits_kernel(const T* __restrict__ k, int64_t k_sb, int64_t k_sh,
                                                     int64_t k_ss, const double* __restrict__ qf, int Hk, int S,
                                                     int D, int W, int wpad, int mode, double scaling,
                                                     float* __restrict__ logits, uint32_t* __restrict__ rmax) {
  extern __shared__ double sq[];  // [32][D + 1] window-row block of qf
  const int nrb = wpad / kRowBlk;
  const int rb = blockIdx.y % nrb;
  const int h = blockIdx.y / nrb;
  const int b = blockIdx.z;
  const int chunk = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, kk = lane >> 4;
  const int w0 = rb * kRowBlk;
  const int nw = min(kRowBlk, W - w0);
  const int64_t bh = (int64_t)b * Hk + h;
  const int ld = D + 1;
  const double* qsrc = qf + (bh * wpad + w0) * D;
  for (int i = threadIdx.x; i < kRowBlk * D; i += 256) sq[(i / D) * ld + (i % D)] = qsrc[i];
  __syncthreads();

  const int key0 = chunk * kChunkM + wave * 32;
  const T* kb = k + b * k_sb + h * k_sh;
  const int r0 = key0 + col, r1 = key0 + 16 + col;
  const T* kr0 = kb + (int64_t)min(r0, S - 1) * k_ss;
  const T* kr1 = kb + (int64_t)min(r1, S - 1) * k_ss;
  const bool ok0 = r0 < S, ok1 = r1 < S;
  const double* q0 = sq + col * ld + kk;         // rows 0..15 of the block
  const double* q1 = sq + (16 + col) * ld + kk;  // rows 16..31

  doublex4 acc00 = {0.0, 0.0, 0.0, 0.0}, acc01 = acc00, acc10 = acc00, acc11 = acc00;
  KChunk<T> ca, cb;
  load_kchunk<T>(ca, kr0, ok0);
  load_kchunk<T>(cb, kr1, ok1);
  for (int d0 = 0; d0 < D; d0 += 8) {
    KChunk<T> na, nb;
    const bool more = d0 + 8 < D;
    if (more) {
      load_kchunk<T>(na, kr0 + d0 + 8, ok0);
      load_kchunk<T>(nb, kr1 + d0 + 8, ok1);
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {  // k-steps t = d0/4 + half
      const int d = d0 + 4 * half;
      const double a0 = q0[d], a1 = q1[d];
      const double b0 = kchunk_elem<T>(ca, 4 * half + kk);
      const double b1 = kchunk_elem<T>(cb, 4 * half + kk);
      acc00 = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b0, acc00, 0, 0, 0);
      acc01 = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b0, acc01, 0, 0, 0);
      acc10 = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b1, acc10, 0, 0, 0);
      acc11 = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b1, acc11, 0, 0, 0);
    }
    if (more) {
      ca = na;
      cb = nb;
    }
  }

  // Epilogue: lane holds rows w0 + 16*nb + kk + 4i for key key0 + 16*mb + col.
  const double r00[4] = {acc00[0], acc00[1], acc00[2], acc00[3]};
  const double r01[4] = {acc01[0], acc01[1], acc01[2], acc01[3]};
  const double r10[4] = {acc10[0], acc10[1], acc10[2], acc10[3]};
  const double r11[4] = {acc11[0], acc11[1], acc11[2], acc11[3]};
  __shared__ float red[4][kRowBlk];
  const int qpos0 = S - W + w0;
#pragma unroll
  for (int nbk = 0; nbk < 2; ++nbk) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int w = 16 * nbk + kk + 4 * i;  // row within the block
      float m = -INFINITY;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const double v = nbk == 0 ? (mb == 0 ? r00[i] : r10[i]) : (mb == 0 ? r01[i] : r11[i]);
        const int key = key0 + 16 * mb + col;
        float L;
        if (mode == HC_SCORE_SNAPKV) {
          L = (key > qpos0 + w) ? -INFINITY : (float)(v * scaling);
        } else {
          L = (float)(v / scaling);
        }
        if (key < S && w < nw) {
          logits[(bh * W + w0 + w) * S + key] = L;
          m = fmaxf(m, L);
        }
      }
      if (mode == HC_SCORE_SNAPKV) {
        // max over the 16 lanes that share this row (same kk)
        m = fmaxf(m, __shfl_xor(m, 1, 64));
        m = fmaxf(m, __shfl_xor(m, 2, 64));
        m = fmaxf(m, __shfl_xor(m, 4, 64));
        m = fmaxf(m, __shfl_xor(m, 8, 64));
        if (col == 0) red[wave][w] = m;
      }
    }
  }
  if (mode != HC_SCORE_SNAPKV) return;
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

// grid (ceil(S/kSumChunk), Hk, B), block 256: exact fixed-point softmax
// denominators.  Each lane accumulates its keys for 16 rows at a time; a
// butterfly reduce-scatter then leaves the wave sum of row (lane >> 2) in
// lanes 4r .. 4r+3 (16 exchanges per row block instead of a full reduction
// per row).
constexpr int kSumRows = 16;
__global__ __launch_bounds__(256) void rowsum_kernel(const float* __restrict__ logits,
                                                     const uint32_t* __restrict__ rmax, int Hk, int S, int W,
                                                     uint64_t* __restrict__ lsum) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * Hk + h;
  __shared__ float sm_m[kMaxW];
  __shared__ uint64_t sm_red[4][kSumRows];
  for (int w = threadIdx.x; w < W; w += blockDim.x) sm_m[w] = key_to_float(rmax[bh * W + w]);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int s0 = blockIdx.x * kSumChunk + threadIdx.x;
  for (int w0 = 0; w0 < W; w0 += kSumRows) {
    const int nw = min(kSumRows, W - w0);
    uint64_t acc[kSumRows];
#pragma unroll
    for (int w = 0; w < kSumRows; ++w) acc[w] = 0;
#pragma unroll 1
    for (int i = 0; i < kSumChunk / 256; ++i) {
      const int s = s0 + 256 * i;
      if (s < S) {
        float L[kSumRows];
        const float* pr = logits + (bh * W + w0) * S + s;
#pragma unroll
        for (int w = 0; w < kSumRows; ++w) {
          L[w] = (w < nw) ? *pr : -INFINITY;
          pr += S;
        }
#pragma unroll
        for (int w = 0; w < kSumRows; ++w)
          if (w < nw) acc[w] += det_fix(det_exp_nonpos((double)L[w] - (double)sm_m[w0 + w]));
      }
    }
    // reduce-scatter over lanes: 16 -> 8 -> 4 -> 2 -> 1 rows per lane
#pragma unroll
    for (int n = kSumRows / 2, o = 32; n >= 1; n >>= 1, o >>= 1) {
      const bool up = (lane & o) != 0;
#pragma unroll
      for (int i = 0; i < n; ++i) {
        const uint64_t lo = acc[i], hi = acc[i + n];
        const uint64_t send = up ? lo : hi;
        const uint64_t keep = up ? hi : lo;
        const uint32_t rl = __shfl_xor((uint32_t)send, o, 64);
        const uint32_t rh = __shfl_xor((uint32_t)(send >> 32), o, 64);
        acc[i] = keep + (((uint64_t)rh << 32) | rl);
      }
    }
#pragma unroll
    for (int o = 2; o >= 1; o >>= 1) {
      const uint32_t rl = __shfl_xor((uint32_t)acc[0], o, 64);
      const uint32_t rh = __shfl_xor((uint32_t)(acc[0] >> 32), o, 64);
      acc[0] += ((uint64_t)rh << 32) | rl;
    }
    // step o kept the half of the rows selected by lane bit o, so lanes
    // 4r .. 4r+3 now hold the wave sum of row r
    if ((lane & 3) == 0) sm_red[wave][lane >> 2] = acc[0];
    __syncthreads();
    if (threadIdx.x < nw) {
      const int w = threadIdx.x;
      const uint64_t tot = sm_red[0][w] + sm_red[1][w] + sm_red[2][w] + sm_red[3][w];
      if (tot) atomicAdd((unsigned long long*)&lsum[bh * W + w0 + w], (unsigned long long)tot);
    }
    __syncthreads();
  }
}

// grid (ceil(S / (256 - 2P)), Hk, B), block 256: thread t computes the
// importance of key c0 - P + t; threads P .. 255-P pool and write keys
// c0 .. c0 + 255 - 2P.
__global__ __launch_bounds__(256) void imp_pool_kernel(const float* __restrict__ logits,
                                                       const uint32_t* __restrict__ rmax,
                                                       const uint64_t* __restrict__ lsum, int Hk, int S,
                                                       int W, int mode, int P, int pooling, int ksize,
                                                       float* __restrict__ scores) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * Hk + h;
  const int out_per_block = 256 - 2 * P;
  const int c0 = blockIdx.x * out_per_block;
  __shared__ float sm_m[kMaxW];
  __shared__ double sm_inv[kMaxW];
  __shared__ float sm_imp[256];
  if (mode == HC_SCORE_SNAPKV) {
    for (int w = threadIdx.x; w < W; w += blockDim.x) {
      sm_m[w] = key_to_float(rmax[bh * W + w]);
      const double l = (double)lsum[bh * W + w] * 0x1p-44;
      sm_inv[w] = 1.0 / l;
    }
  }
  __syncthreads();
  const int s = c0 - P + (int)threadIdx.x;
  float v = 0.f;
  if (s >= 0 && s < S) {
    double acc = 0.0;
    for (int w0 = 0; w0 < W; w0 += kSumRows) {
      const int nw = min(kSumRows, W - w0);
      float L[kSumRows];
      const float* pr = logits + (bh * W + w0) * S + s;
#pragma unroll
      for (int w = 0; w < kSumRows; ++w) {
        L[w] = (w < nw) ? *pr : 0.f;
        pr += S;
      }
      if (mode == HC_SCORE_SNAPKV) {
#pragma unroll
        for (int w = 0; w < kSumRows; ++w)
          if (w < nw) acc = __builtin_fma(det_exp_nonpos((double)L[w] - (double)sm_m[w0 + w]), sm_inv[w0 + w], acc);
      } else {
#pragma unroll
        for (int w = 0; w < kSumRows; ++w)
          if (w < nw) acc = acc + (double)L[w];
      }
    }
    v = (float)acc;
  }
  sm_imp[threadIdx.x] = v;
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
                         int64_t D, int64_t W, const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss,
                         int64_t q_row0, const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss, double scal,
                         int P, int pooling, int ksize, float* scores, hipStream_t st) {
  double* qf = reinterpret_cast<double*>(ws + lay.qf_off);
  float* logits = reinterpret_cast<float*>(ws + lay.logits_off);
  uint32_t* rmax = reinterpret_cast<uint32_t*>(ws + lay.rmax_off);
  uint64_t* lsum = reinterpret_cast<uint64_t*>(ws + lay.lsum_off);
  const int nrb = (int)(lay.wpad / kRowBlk);
  hipLaunchKernelGGL(qmean_kernel<T>, dim3((unsigned)lay.wpad, (unsigned)Hk, (unsigned)B),
                     dim3((unsigned)(D < 64 ? 64 : D)), 0, st, (const T*)q, q_sb, q_sh, q_ss, q_row0, (int)Hq,
                     (int)Hk, (int)W, (int)lay.wpad, (int)D, qf, rmax, lsum);
  const size_t lds = (size_t)(kRowBlk * (D + 1) * 8);
  if (lds > 65536)
    (void)hipFuncSetAttribute((const void*)logits_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL(logits_kernel<T>, dim3((unsigned)lay.nchunk_m, (unsigned)(Hk * nrb), (unsigned)B), dim3(256),
                     lds, st, (const T*)k, k_sb, k_sh, k_ss, (const double*)qf, (int)Hk, (int)S, (int)D, (int)W,
                     (int)lay.wpad, mode, scal, logits, rmax);
  if (mode == HC_SCORE_SNAPKV)
    hipLaunchKernelGGL(rowsum_kernel, dim3((unsigned)cdiv(S, kSumChunk), (unsigned)Hk, (unsigned)B), dim3(256), 0,
                       st, (const float*)logits, (const uint32_t*)rmax, (int)Hk, (int)S, (int)W, lsum);
  hipLaunchKernelGGL(imp_pool_kernel, dim3((unsigned)cdiv(S, 256 - 2 * P), (unsigned)Hk, (unsigned)B), dim3(256), 0,
                     st, (const float*)logits, (const uint32_t*)rmax, (const uint64_t*)lsum, (int)Hk, (int)S, (int)W,
                     mode, P, pooling, ksize, scores);
}

}  // namespace hc

using namespace hc;

extern "C" int64_t hc_snapkv_score_workspace_size(int64_t B, int64_t Hk, int64_t S, int64_t D, int64_t W) {
  if (B <= 0 || Hk <= 0 || S <= 0 || D <= 0 || W <= 0) return 256;
  if (W > S) W = S;
  return score_layout(B, Hk, S, D, W).total;
}

extern "C" int hc_snapkv_score(int dtype, int mode, int64_t B, int64_t Hq, int64_t Hk, int64_t S, int64_t D,
                               int64_t W, const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_row0,
                               const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss, double scaling,
                               int64_t kernel_size, int pooling, float* scores, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  HC_REQUIRE(dtype == HC_DTYPE_F32 || dtype == HC_DTYPE_F16 || dtype == HC_DTYPE_BF16, "score: bad dtype %d", dtype);
  HC_REQUIRE(mode == HC_SCORE_SNAPKV || mode == HC_SCORE_RAWSUM, "score: bad mode %d", mode);
  HC_REQUIRE(B > 0 && Hq > 0 && Hk > 0 && S > 0 && D > 0 && W > 0, "score: empty shape");
  HC_REQUIRE(W <= S, "score: window %lld exceeds S %lld", (long long)W, (long long)S);
  HC_REQUIRE(W <= kMaxW, "score: window %lld above the supported %d rows", (long long)W, kMaxW);
  HC_REQUIRE(D % 8 == 0 && D <= 512, "score: head_dim %lld must be a multiple of 8 and <= 512", (long long)D);
  HC_REQUIRE(S <= ((int64_t)1 << 19), "score: S %lld above 2^19 (fixed-point normaliser range)", (long long)S);
  HC_REQUIRE(B <= 65535 && Hk * cdiv(W, kRowBlk) <= 65535, "score: grid too large");
  HC_REQUIRE(q_row0 >= 0, "score: negative q_row0");
  HC_REQUIRE(q && k && scores, "score: null pointer");
  const int es = dtype_size(dtype);
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
    launch_score<half_t>(lay, ws, mode, B, Hq, Hk, S, D, W, q, q_sb, q_sh, q_ss, q_row0, k, k_sb, k_sh, k_ss, scal,
                         P, pooling, (int)kernel_size, scores, st);
  else if (dtype == HC_DTYPE_BF16)
    launch_score<bf16_t>(lay, ws, mode, B, Hq, Hk, S, D, W, q, q_sb, q_sh, q_ss, q_row0, k, k_sb, k_sh, k_ss, scal,
                         P, pooling, (int)kernel_size, scores, st);
  else
    launch_score<float>(lay, ws, mode, B, Hq, Hk, S, D, W, q, q_sb, q_sh, q_ss, q_row0, k, k_sb, k_sh, k_ss, scal,
                        P, pooling, (int)kernel_size, scores, st);
  return check_launch("snapkv_score");
}

extern "C" int hc_head_mean(int64_t B, int64_t H, int64_t S, const float* scores, float* out, void* stream) {
  HC_REQUIRE(B > 0 && H > 0 && S > 0 && scores && out, "head_mean: bad arguments");
  HC_REQUIRE(B <= 65535, "head_mean: B too large");
  hipLaunchKernelGGL(head_mean_kernel, dim3((unsigned)cdiv(S, 256), (unsigned)B), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), scores, (int)H, (int)S, out);
  return check_launch("head_mean");
}
