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
//   logits  -> L (fp32 [B][Hk][W][S]) + per-256-key-chunk row max
//   rowsum  -> l_w (uint64, 64-bit atomics)            [SNAPKV only]
//   imp     -> pooled fp32 scores [B][Hk][S]
#include "hc_common.h"

namespace hc {

constexpr int kChunk = 256;   // keys per logits/imp workgroup (one per lane)
constexpr int kRowBlk = 32;   // window rows per logits workgroup (fp64 accumulators)
constexpr int kSumChunk = 512;  // keys per rowsum workgroup
constexpr int kMaxW = 256;
constexpr int kMaxPool = 64;  // max half-width of the pooling window

struct ScoreLayout {
  int64_t wpad, nchunk, qf_off, logits_off, cmax_off, lsum_off, total;
};

static int64_t al256(int64_t x) { return (x + 255) & ~(int64_t)255; }

static ScoreLayout score_layout(int64_t B, int64_t Hk, int64_t S, int64_t D, int64_t W) {
  ScoreLayout L;
  L.wpad = cdiv(W, kRowBlk) * kRowBlk;
  L.nchunk = cdiv(S, kChunk);
  L.qf_off = 0;
  L.logits_off = al256(L.qf_off + B * Hk * L.wpad * D * 8);
  L.cmax_off = al256(L.logits_off + B * Hk * W * S * 4);
  L.lsum_off = al256(L.cmax_off + B * Hk * L.nchunk * W * 4);
  L.total = al256(L.lsum_off + B * Hk * W * 8);
  return L;
}

// qf[b][h][w][d] for w < wpad (zero rows past W).  grid (wpad, Hk, B), block D.
template <typename T>
__global__ void qmean_kernel(const T* __restrict__ q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_row0,
                             int Hq, int Hk, int W, int wpad, int D, double* __restrict__ qf) {
  const int w = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int d = threadIdx.x;
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

// Load 8 contiguous elements (d0..d0+7) of a key row as doubles.
template <typename T>
__device__ __forceinline__ void load8_f64(const T* p, double (&kd)[8]);
template <>
__device__ __forceinline__ void load8_f64<half_t>(const half_t* p, double (&kd)[8]) {
  const u32x4 w = ld16(p);
  const uint32_t ww[4] = {w[0], w[1], w[2], w[3]};
#pragma unroll
  for (int j = 0; j < 8; ++j) kd[j] = (double)Unpack<half_t>::get(ww, j);
}
template <>
__device__ __forceinline__ void load8_f64<bf16_t>(const bf16_t* p, double (&kd)[8]) {
  const u32x4 w = ld16(p);
  const uint32_t ww[4] = {w[0], w[1], w[2], w[3]};
#pragma unroll
  for (int j = 0; j < 8; ++j) kd[j] = (double)Unpack<bf16_t>::get(ww, j);
}
template <>
__device__ __forceinline__ void load8_f64<float>(const float* p, double (&kd)[8]) {
  const u32x4 w0 = ld16(p);
  const u32x4 w1 = ld16(p + 4);
  const uint32_t ww[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
#pragma unroll
  for (int j = 0; j < 8; ++j) kd[j] = (double)__builtin_bit_cast(float, ww[j]);
}

// grid (nchunk, Hk * nrb, B), block 256: one key per lane, 32 window rows per
// workgroup held as fp64 accumulators; qf is wave-uniform (scalar loads).
template <typename T>
__global__ __launch_bounds__(256) void logits_kernel(const T* __restrict__ k, int64_t k_sb, int64_t k_sh,
                                                     int64_t k_ss, const double* __restrict__ qf, int Hk,
                                                     int S, int D, int W, int wpad, int mode, double scaling,
                                                     float* __restrict__ logits, float* __restrict__ cmax,
                                                     uint64_t* __restrict__ lsum) {
  const int nrb = wpad / kRowBlk;
  const int rb = blockIdx.y % nrb;
  const int h = blockIdx.y / nrb;
  const int b = blockIdx.z;
  const int chunk = blockIdx.x;
  const int s = chunk * kChunk + threadIdx.x;
  const int w0 = rb * kRowBlk;
  const int nw = min(kRowBlk, W - w0);
  const int64_t bh = (int64_t)b * Hk + h;
  const double* qrow = qf + (bh * wpad + w0) * D;

  double acc[kRowBlk];
#pragma unroll
  for (int w = 0; w < kRowBlk; ++w) acc[w] = 0.0;

  if (s < S) {
    const T* krow = k + b * k_sb + h * k_sh + (int64_t)s * k_ss;
    for (int d0 = 0; d0 < D; d0 += 8) {
      double kd[8];
      load8_f64<T>(krow + d0, kd);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int w = 0; w < kRowBlk; ++w) acc[w] = __builtin_fma(qrow[w * D + d0 + j], kd[j], acc[w]);
      }
    }
  }

  __shared__ float red[4][kRowBlk];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int qpos0 = S - W + w0;  // absolute position of window row w0
#pragma unroll
  for (int w = 0; w < kRowBlk; ++w) {
    if (w < nw) {
      float L = -INFINITY;
      if (s < S) {
        if (mode == HC_SCORE_SNAPKV) {
          L = (float)(acc[w] * scaling);
          if (s > qpos0 + w) L = -INFINITY;
        } else {
          L = (float)(acc[w] / scaling);
        }
        logits[(bh * W + w0 + w) * S + s] = L;
      }
      if (mode == HC_SCORE_SNAPKV) {
        const float m = wave_max(L);
        if (lane == 0) red[wave][w] = m;
      }
    }
  }
  if (mode != HC_SCORE_SNAPKV) return;
  __syncthreads();
  if (threadIdx.x < nw) {
    const int w = threadIdx.x;
    const float m = fmaxf(fmaxf(red[0][w], red[1][w]), fmaxf(red[2][w], red[3][w]));
    cmax[(bh * gridDim.x + chunk) * W + w0 + w] = m;
    if (chunk == 0) lsum[bh * W + w0 + w] = 0ull;
  }
}

// Row maxima from the per-chunk maxima.  m[w] for w < W into shared memory.
__device__ __forceinline__ void load_row_max(const float* cmax, int64_t bh, int nchunk, int W, float* sm_m) {
  for (int w = threadIdx.x; w < W; w += blockDim.x) {
    float m = -INFINITY;
    for (int c = 0; c < nchunk; ++c) m = fmaxf(m, cmax[(bh * nchunk + c) * W + w]);
    sm_m[w] = m;
  }
}

// grid (ceil(S/512), Hk, B), block 256: exact fixed-point softmax denominators.
__global__ __launch_bounds__(256) void rowsum_kernel(const float* __restrict__ logits,
                                                     const float* __restrict__ cmax, int Hk, int S, int W,
                                                     int nchunk, uint64_t* __restrict__ lsum) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * Hk + h;
  __shared__ float sm_m[kMaxW];
  load_row_max(cmax, bh, nchunk, W, sm_m);
  __syncthreads();
  const int s0 = blockIdx.x * kSumChunk + threadIdx.x;
  const int lane = threadIdx.x & 63;
  for (int w = 0; w < W; ++w) {
    const double m = (double)sm_m[w];
    const float* row = logits + (bh * W + w) * S;
    uint64_t part = 0;
#pragma unroll
    for (int i = 0; i < kSumChunk / 256; ++i) {
      const int s = s0 + 256 * i;
      if (s < S) part += det_fix(det_exp_nonpos((double)row[s] - m));
    }
    part = wave_sum_u64(part);
    if (lane == 0 && part) atomicAdd((unsigned long long*)&lsum[bh * W + w], (unsigned long long)part);
  }
}

// grid (nchunk, Hk, B), block 256: importance of keys [c0-P, c0+256+P), then
// pooling of keys [c0, c0+256).
__global__ __launch_bounds__(256) void imp_pool_kernel(const float* __restrict__ logits,
                                                       const float* __restrict__ cmax,
                                                       const uint64_t* __restrict__ lsum, int Hk, int S,
                                                       int W, int nchunk, int mode, int P, int pooling,
                                                       int ksize, float* __restrict__ scores) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * Hk + h;
  const int c0 = blockIdx.x * kChunk;
  __shared__ float sm_m[kMaxW];
  __shared__ double sm_inv[kMaxW];
  __shared__ float sm_imp[kChunk + 2 * kMaxPool];
  if (mode == HC_SCORE_SNAPKV) {
    load_row_max(cmax, bh, nchunk, W, sm_m);
    for (int w = threadIdx.x; w < W; w += blockDim.x) {
      const double l = (double)lsum[bh * W + w] * 0x1p-44;
      sm_inv[w] = 1.0 / l;
    }
  }
  __syncthreads();
  const int span = kChunk + 2 * P;
  for (int t = threadIdx.x; t < span; t += blockDim.x) {
    const int s = c0 - P + t;
    float v = 0.f;
    if (s >= 0 && s < S) {
      double acc = 0.0;
      if (mode == HC_SCORE_SNAPKV) {
        for (int w = 0; w < W; ++w) {
          const double e = det_exp_nonpos((double)logits[(bh * W + w) * S + s] - (double)sm_m[w]);
          acc = __builtin_fma(e, sm_inv[w], acc);
        }
      } else {
        for (int w = 0; w < W; ++w) acc = acc + (double)logits[(bh * W + w) * S + s];
      }
      v = (float)acc;
    }
    sm_imp[t] = v;
  }
  __syncthreads();
  const int s = c0 + threadIdx.x;
  if (s >= S) return;
  float out;
  if (P == 0) {
    out = sm_imp[threadIdx.x];
  } else if (pooling == HC_POOL_MAX) {
    out = -INFINITY;
    for (int j = -P; j <= P; ++j) {
      const int sj = s + j;
      if (sj >= 0 && sj < S) out = fmaxf(out, sm_imp[threadIdx.x + P + j]);
    }
  } else {
    double sum = 0.0;
    for (int j = -P; j <= P; ++j) {
      const int sj = s + j;
      if (sj >= 0 && sj < S) sum = sum + (double)sm_imp[threadIdx.x + P + j];
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
  float* cmax = reinterpret_cast<float*>(ws + lay.cmax_off);
  uint64_t* lsum = reinterpret_cast<uint64_t*>(ws + lay.lsum_off);
  const int nrb = (int)(lay.wpad / kRowBlk);
  hipLaunchKernelGGL(qmean_kernel<T>, dim3((unsigned)lay.wpad, (unsigned)Hk, (unsigned)B),
                     dim3((unsigned)(D < 64 ? 64 : D)), 0, st, (const T*)q, q_sb, q_sh, q_ss, q_row0, (int)Hq,
                     (int)Hk, (int)W, (int)lay.wpad, (int)D, qf);
  hipLaunchKernelGGL(logits_kernel<T>, dim3((unsigned)lay.nchunk, (unsigned)(Hk * nrb), (unsigned)B), dim3(256),
                     0, st, (const T*)k, k_sb, k_sh, k_ss, (const double*)qf, (int)Hk, (int)S, (int)D, (int)W,
                     (int)lay.wpad, mode, scal, logits, cmax, lsum);
  if (mode == HC_SCORE_SNAPKV)
    hipLaunchKernelGGL(rowsum_kernel, dim3((unsigned)cdiv(S, kSumChunk), (unsigned)Hk, (unsigned)B), dim3(256), 0,
                       st, (const float*)logits, (const float*)cmax, (int)Hk, (int)S, (int)W, (int)lay.nchunk,
                       lsum);
  hipLaunchKernelGGL(imp_pool_kernel, dim3((unsigned)lay.nchunk, (unsigned)Hk, (unsigned)B), dim3(256), 0, st,
                     (const float*)logits, (const float*)cmax, (const uint64_t*)lsum, (int)Hk, (int)S, (int)W,
                     (int)lay.nchunk, mode, P, pooling, ksize, scores);
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
  HC_REQUIRE(D % 8 == 0 && D <= 1024, "score: head_dim %lld must be a multiple of 8 and <= 1024", (long long)D);
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
