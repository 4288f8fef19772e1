// Kept-index selection and row movement into the hot buffer.
//
// hc_topk_keep replaces keep_index (src/hotcold_kv/baselines/scoring.py:110-132)
// and the top-k of HotColdLayer._compress_if_needed (src/hotcold_kv/cache.py:47-95).
// One workgroup per (batch, head): an MSB-first radix select over 32-bit
// order keys (three passes: 11, 11, 10 bits) finds the threshold key T of
// the keep_prefix-th largest prefix
// score, then one ordered pass emits every index with key > T plus the
// lowest-index ties with key == T.  Emitting in index order gives the
// ascending sort of scoring.py:130 for free, and the result is the exact
// "value descending, ties to the lower index" set (no nth_element ambiguity).
// hc_topk_keep_ws makes the same selection for grids of few rows longer than
// the LDS key cache, each row spread over chunks of 8192 keys (topk_*_kernel).
//
// hc_gather_rows / hc_append_rows replace gather_kv (scoring.py:135-139),
// the gathers of cache.py:79-84 and the torch.cat appends of cache.py:145-148
// and layer_state.py:99-100: 16-byte vector copies of whole rows into the
// fixed-capacity hot buffer, no re-copy of the resident cache.
#include "hc_common.h"

namespace hc {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / 64;
constexpr int kTopkCache = 32768;  // prefix keys cached in LDS (128 KiB)
constexpr int kTopkU = 8;          // keys loaded together per thread (one wait per batch)

// Block-wide exclusive prefix sum of v in thread order (wave scans plus one
// pass over the wave totals); writes the block total to *total.
__device__ __forceinline__ int block_excl_scan(int v, int* sm_wave, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) sm_wave[wave] = incl;
  __syncthreads();
  int before = 0, tot = 0;
  for (int w = 0; w < kTopkWaves; ++w) {
    const int c = sm_wave[w];
    if (w < wave) before += c;
    tot += c;
  }
  __syncthreads();
  *total = tot;
  return before + incl - v;
}

// Digit search of one radix pass over kDigitBins bins: the largest digit d
// with count(digits > d) < krem <= count(digits >= d).  Thread t holds the
// bin pair kDigitBins-1-2t, kDigitBins-2-2t, so thread order is descending
// digit order and one block scan finds d.
constexpr int kDigitBins = 2048;
static_assert(kDigitBins == 2 * kTopkThreads, "two bins per thread");
__device__ __forceinline__ void find_digit(const uint32_t* hist, uint32_t krem, uint32_t* sm_scan,
                                           uint32_t* sm_digit, uint32_t* sm_krem) {
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const uint32_t c0 = hist[kDigitBins - 1 - 2 * t], c1 = hist[kDigitBins - 2 - 2 * t];
  const uint32_t v = c0 + c1;
  uint32_t incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) sm_scan[wave] = incl;
  __syncthreads();
  // all wave totals read at once (a loop bounded by `wave` issues its LDS
  // reads one after another)
  uint32_t before = 0;
#pragma unroll
  for (int w = 0; w < kTopkWaves; ++w) before += w < wave ? sm_scan[w] : 0u;
  incl += before;
  const uint32_t excl = incl - v;
  if (excl < krem && excl + c0 >= krem) {
    *sm_digit = (uint32_t)(kDigitBins - 1 - 2 * t);
    *sm_krem = krem - excl;
  } else if (excl + c0 < krem && incl >= krem) {
    *sm_digit = (uint32_t)(kDigitBins - 2 - 2 * t);
    *sm_krem = krem - excl - c0;
  }
  __syncthreads();
}

// One workgroup per (batch, head).  The prefix's order keys are cached in
// LDS when they fit (prefix <= kTopkCache), otherwise re-read from global.
__global__ __launch_bounds__(kTopkThreads) void topk_keep_kernel(const float* __restrict__ scores, int64_t s_sb,
                                                                 int64_t s_sh, int H, int prefix, int keep_prefix,
                                                                 int window, int64_t* __restrict__ keep,
                                                                 int64_t* __restrict__ evicted) {
  extern __shared__ uint32_t skey[];
  const int h = blockIdx.x, b = blockIdx.y;
  const float* sc = scores + b * s_sb + h * s_sh;
  const int n_keep = keep_prefix + window;
  int64_t* out = keep + ((int64_t)b * H + h) * n_keep;
  const int n_ev = prefix - keep_prefix;
  int64_t* ev = evicted ? evicted + ((int64_t)b * H + h) * n_ev : nullptr;
  const bool cached = prefix <= kTopkCache;

  __shared__ uint32_t hist[kDigitBins];
  __shared__ uint32_t sm_scan[kTopkWaves];
  __shared__ uint32_t sm_digit, sm_krem;
  __shared__ int sm_wave[kTopkWaves];

  // Global reads go kTopkU at a time with clamped (in-range) indices, so a
  // batch costs one memory round trip instead of one per key.
  // kTopkU order keys at idx(u), from LDS or (one batch of loads) global
  auto keys_of = [&](uint32_t (&ks)[kTopkU], auto idx) {
    if (cached) {
#pragma unroll
      for (int u = 0; u < kTopkU; ++u) ks[u] = skey[idx(u)];
    } else {
      float v[kTopkU];
#pragma unroll
      for (int u = 0; u < kTopkU; ++u) v[u] = sc[idx(u)];
#pragma unroll
      for (int u = 0; u < kTopkU; ++u) ks[u] = order_key(v[u]);
    }
  };
  if (cached && keep_prefix > 0) {
    for (int base = 0; base < prefix; base += kTopkThreads * kTopkU) {
      float v[kTopkU];
#pragma unroll
      for (int u = 0; u < kTopkU; ++u) v[u] = sc[min(base + u * kTopkThreads + (int)threadIdx.x, prefix - 1)];
#pragma unroll
      for (int u = 0; u < kTopkU; ++u) {
        const int i = base + u * kTopkThreads + (int)threadIdx.x;
        if (i < prefix) skey[i] = order_key(v[u]);
      }
    }
    __syncthreads();
  }

  uint32_t tkey = 0;
  int need_eq = 0;
  if (keep_prefix > 0) {
    uint32_t pbits = 0, pmask = 0;
    uint32_t krem = (uint32_t)keep_prefix;
    // three passes of 11, 11 and 10 bits: scores crowd a few exponents, and
    // wide digits spread them over many bins (LDS atomics to one address
    // serialise)
    for (int ps = 0; ps < 3; ++ps) {
      const int shift = ps == 0 ? 21 : ps == 1 ? 10 : 0;
      const uint32_t dmask = ps == 2 ? 1023u : 2047u;
      for (int i = threadIdx.x; i < kDigitBins; i += kTopkThreads) hist[i] = 0;
      __syncthreads();
      for (int base = 0; base < prefix; base += kTopkThreads * kTopkU) {
        uint32_t ks[kTopkU];
        keys_of(ks, [&](int u) { return min(base + u * kTopkThreads + (int)threadIdx.x, prefix - 1); });
#pragma unroll
        for (int u = 0; u < kTopkU; ++u) {
          const int i = base + u * kTopkThreads + (int)threadIdx.x;
          hist_add(hist, (ks[u] >> shift) & dmask, i < prefix && (ks[u] & pmask) == pbits);
        }
      }
      __syncthreads();
      find_digit(hist, krem, sm_scan, &sm_digit, &sm_krem);
      pbits |= sm_digit << shift;
      pmask |= dmask << shift;
      krem = sm_krem;
      __syncthreads();
    }
    tkey = pbits;
    need_eq = (int)krem;
  }

  // Each thread owns a contiguous run of the prefix; two block scans give
  // every run its first output slot, so the kept indices come out ascending.
  const int run = (prefix + kTopkThreads - 1) / kTopkThreads;
  const int i0 = min(prefix, (int)threadIdx.x * run);
  const int i1 = min(prefix, i0 + run);
  int n_gt = 0, n_eq = 0;
  if (keep_prefix > 0) {
    for (int c = i0; c < i1; c += kTopkU) {
      uint32_t ks[kTopkU];
      keys_of(ks, [&](int u) { return min(c + u, i1 - 1); });
#pragma unroll
      for (int u = 0; u < kTopkU; ++u) {
        if (c + u < i1) {
          n_gt += ks[u] > tkey;
          n_eq += ks[u] == tkey;
        }
      }
    }
  }
  int tot;
  const int eq_before = block_excl_scan(n_eq, sm_wave, &tot);
  const int take_eq = max(0, min(need_eq - eq_before, n_eq));
  const int sel_before = block_excl_scan(n_gt + take_eq, sm_wave, &tot);
  int pos = sel_before;
  int epos = i0 - sel_before;
  int eq_seen = 0;
  for (int c = i0; c < i1; c += kTopkU) {
    uint32_t ks[kTopkU] = {};
    if (keep_prefix > 0) keys_of(ks, [&](int u) { return min(c + u, i1 - 1); });
#pragma unroll
    for (int u = 0; u < kTopkU; ++u) {
      const int i = c + u;
      if (i >= i1) break;
      bool sel = false;
      if (keep_prefix > 0) {
        if (ks[u] > tkey) {
          sel = true;
        } else if (ks[u] == tkey) {
          sel = eq_seen < take_eq;
          ++eq_seen;
        }
      }
      if (sel) out[pos++] = i;
      else if (ev) ev[epos++] = i;
    }
  }
  for (int j = threadIdx.x; j < window; j += kTopkThreads) out[keep_prefix + j] = prefix + j;
}

// The same selection with each (batch, head) row spread over chunks of
// kTopkChunk keys, for grids of few long rows (one workgroup per row would
// leave most CUs idle, each scanning its whole row several times).  A chain
// of launches on one stream, whose boundaries order the steps:
//   topk_init   per row: zero the histogram, state = (0, 0, keep_prefix)
//   3 x topk_hist   per chunk: LDS histogram of the pass's digit over the
//                   keys that match the row's prefix, added to the row's
//                   global histogram
//       topk_digit  per row: the digit of the pass (find_digit), folded into
//                   the row's prefix; the histogram is left zeroed
//   topk_count  per chunk: keys above the threshold and equal to it
//   topk_emit   per chunk: the kept and evicted indices of the chunk, at the
//               offsets the earlier chunks' counts give
// The threshold key, the number of ties kept and every output position are
// those of topk_keep_kernel: the ties kept are still the lowest-index ones.
constexpr int kTopkChunk = kTopkThreads * kTopkU;  // keys per workgroup
constexpr int kTopkState = 4;                      // (prefix bits, prefix mask, keys still to take, 0)

__device__ __forceinline__ int pass_shift(int pass) { return pass == 0 ? 21 : pass == 1 ? 10 : 0; }
__device__ __forceinline__ uint32_t pass_mask(int pass) { return pass == 2 ? 1023u : 2047u; }

__global__ __launch_bounds__(256) void topk_init_kernel(int H, uint32_t keep_prefix, uint32_t* __restrict__ ghist,
                                                        uint32_t* __restrict__ state) {
  const int64_t row = (int64_t)blockIdx.y * H + blockIdx.x;
  for (int i = threadIdx.x; i < kDigitBins; i += 256) ghist[row * kDigitBins + i] = 0;
  if (threadIdx.x < kTopkState) state[row * kTopkState + threadIdx.x] = threadIdx.x == 2 ? keep_prefix : 0u;
}

// The order keys of chunk c of a row: kTopkU per thread, loaded together
// (indices clamped into [k0, k1); the lanes past k1 are masked by the caller).
__device__ __forceinline__ void chunk_keys(const float* sc, int k0, int k1, uint32_t (&ks)[kTopkU]) {
  float v[kTopkU];
#pragma unroll
  for (int u = 0; u < kTopkU; ++u) v[u] = sc[min(k0 + u * kTopkThreads + (int)threadIdx.x, k1 - 1)];
#pragma unroll
  for (int u = 0; u < kTopkU; ++u) ks[u] = order_key(v[u]);
}

__global__ __launch_bounds__(kTopkThreads) void topk_hist_kernel(const float* __restrict__ scores, int64_t s_sb,
                                                                 int64_t s_sh, int H, int prefix, int pass,
                                                                 uint32_t* __restrict__ ghist,
                                                                 const uint32_t* __restrict__ state) {
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t row = (int64_t)b * H + h;
  const float* sc = scores + b * s_sb + h * s_sh;
  const int k0 = c * kTopkChunk, k1 = min(prefix, k0 + kTopkChunk);
  const int shift = pass_shift(pass);
  const uint32_t dmask = pass_mask(pass);
  const uint32_t pbits = state[row * kTopkState + 0], pmask = state[row * kTopkState + 1];
  __shared__ uint32_t hist[kDigitBins];
  for (int i = threadIdx.x; i < kDigitBins; i += kTopkThreads) hist[i] = 0;
  __syncthreads();
  uint32_t ks[kTopkU];
  chunk_keys(sc, k0, k1, ks);
#pragma unroll
  for (int u = 0; u < kTopkU; ++u) {
    const int i = k0 + u * kTopkThreads + (int)threadIdx.x;
    hist_add(hist, (ks[u] >> shift) & dmask, i < k1 && (ks[u] & pmask) == pbits);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kDigitBins; i += kTopkThreads) {
    const uint32_t n = hist[i];
    if (n) atomicAdd(&ghist[row * kDigitBins + i], n);
  }
}

__global__ __launch_bounds__(kTopkThreads) void topk_digit_kernel(int H, int pass, uint32_t* __restrict__ ghist,
                                                                  uint32_t* __restrict__ state) {
  const int64_t row = (int64_t)blockIdx.y * H + blockIdx.x;
  __shared__ uint32_t hist[kDigitBins];
  __shared__ uint32_t sm_scan[kTopkWaves];
  __shared__ uint32_t sm_digit, sm_krem;
  uint32_t* g = ghist + row * kDigitBins;
  for (int i = threadIdx.x; i < kDigitBins; i += kTopkThreads) {
    hist[i] = g[i];
    g[i] = 0;
  }
  const uint32_t krem = state[row * kTopkState + 2];
  __syncthreads();
  find_digit(hist, krem, sm_scan, &sm_digit, &sm_krem);
  if (threadIdx.x == 0) {
    const int shift = pass_shift(pass);
    state[row * kTopkState + 0] |= sm_digit << shift;
    state[row * kTopkState + 1] |= pass_mask(pass) << shift;
    state[row * kTopkState + 2] = sm_krem;
  }
}

__global__ __launch_bounds__(kTopkThreads) void topk_count_kernel(const float* __restrict__ scores, int64_t s_sb,
                                                                  int64_t s_sh, int H, int prefix, int nchunk,
                                                                  const uint32_t* __restrict__ state,
                                                                  int* __restrict__ counts) {
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t row = (int64_t)b * H + h;
  const float* sc = scores + b * s_sb + h * s_sh;
  const int k0 = c * kTopkChunk, k1 = min(prefix, k0 + kTopkChunk);
  const uint32_t tkey = state[row * kTopkState + 0];
  __shared__ int sm_wave[kTopkWaves];
  uint32_t ks[kTopkU];
  chunk_keys(sc, k0, k1, ks);
  int n_gt = 0, n_eq = 0;
#pragma unroll
  for (int u = 0; u < kTopkU; ++u) {
    if (k0 + u * kTopkThreads + (int)threadIdx.x < k1) {
      n_gt += ks[u] > tkey;
      n_eq += ks[u] == tkey;
    }
  }
  int tot_gt, tot_eq;
  block_excl_scan(n_gt, sm_wave, &tot_gt);
  block_excl_scan(n_eq, sm_wave, &tot_eq);
  if (threadIdx.x == 0) {
    counts[(row * nchunk + c) * 2 + 0] = tot_gt;
    counts[(row * nchunk + c) * 2 + 1] = tot_eq;
  }
}

__global__ __launch_bounds__(kTopkThreads) void topk_emit_kernel(const float* __restrict__ scores, int64_t s_sb,
                                                                 int64_t s_sh, int H, int prefix, int nchunk,
                                                                 int keep_prefix, int window,
                                                                 const uint32_t* __restrict__ state,
                                                                 const int* __restrict__ counts,
                                                                 int64_t* __restrict__ keep,
                                                                 int64_t* __restrict__ evicted) {
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t row = (int64_t)b * H + h;
  const float* sc = scores + b * s_sb + h * s_sh;
  const int k0 = c * kTopkChunk, k1 = min(prefix, k0 + kTopkChunk);
  const int n_keep = keep_prefix + window;
  int64_t* out = keep + row * n_keep;
  int64_t* ev = evicted ? evicted + row * (prefix - keep_prefix) : nullptr;
  const uint32_t tkey = state[row * kTopkState + 0];
  const int need_eq = (int)state[row * kTopkState + 2];
  __shared__ int sm_wave[kTopkWaves];
  // the earlier chunks: keys above the threshold, and ties
  int gt_c = 0, eq_c = 0;
  for (int cc = 0; cc < c; ++cc) {
    gt_c += counts[(row * nchunk + cc) * 2 + 0];
    eq_c += counts[(row * nchunk + cc) * 2 + 1];
  }
  // each thread owns a contiguous run of the chunk, as in topk_keep_kernel
  const int len = k1 - k0;
  const int run = (len + kTopkThreads - 1) / kTopkThreads;
  const int i0 = k0 + min(len, (int)threadIdx.x * run);
  const int i1 = k0 + min(len, (int)threadIdx.x * run + run);
  // a run is at most kTopkU keys (a chunk is kTopkThreads * kTopkU): loaded
  // once, for the counts and the emit (an empty run, i0 == i1 == k1, reads
  // key k1 - 1 and uses none)
  static_assert(kTopkChunk == kTopkThreads * kTopkU, "one load batch per run");
  uint32_t ks[kTopkU];
#pragma unroll
  for (int u = 0; u < kTopkU; ++u) ks[u] = order_key(sc[min(i0 + u, i1 - 1 < i0 ? k1 - 1 : i1 - 1)]);
  int n_gt = 0, n_eq = 0;
#pragma unroll
  for (int u = 0; u < kTopkU; ++u) {
    if (i0 + u < i1) {
      n_gt += ks[u] > tkey;
      n_eq += ks[u] == tkey;
    }
  }
  int tot;
  // ties before this thread's run over the whole row; the ties it keeps
  const int eq_before = eq_c + block_excl_scan(n_eq, sm_wave, &tot);
  const int take_eq = max(0, min(need_eq - eq_before, n_eq));
  // indices kept before the run: every key above the threshold, and
  // min(ties before, need_eq) ties
  const int sel_before = gt_c + min(eq_c, need_eq) + block_excl_scan(n_gt + take_eq, sm_wave, &tot);
  int pos = sel_before;
  int epos = i0 - sel_before;
  int eq_seen = 0;
#pragma unroll
  for (int u = 0; u < kTopkU; ++u) {
    const int j = i0 + u;
    if (j >= i1) break;
    bool sel = false;
    if (ks[u] > tkey) {
      sel = true;
    } else if (ks[u] == tkey) {
      sel = eq_seen < take_eq;
      ++eq_seen;
    }
    if (sel) out[pos++] = j;
    else if (ev) ev[epos++] = j;
  }
  if (c == 0)
    for (int j = threadIdx.x; j < window; j += kTopkThreads) out[keep_prefix + j] = prefix + j;
}

// Row copy: thread copies one VW-byte vector of one row of each tensor.
struct RowCopy {
  const char* src[3];
  char* dst[3];
  // Optional per-row tables (row b of tensor t starts at src_tab[t][b] /
  // dst_tab[t][b]; the b strides are then unused): rows that live in
  // separate allocations, e.g. the layers of a model.
  const char* const* src_tab[3];
  char* const* dst_tab[3];
  int64_t s_sb[3], s_sh[3], s_ss[3];
  int64_t d_sb[3], d_sh[3], d_ss[3];
  int ntensor;
  const int64_t* idx;
  int64_t i_sb, i_sh;
  int64_t src_rows, src_row0, dst_row0;
  const int64_t* pos_src;
  int64_t ps_sb;
  int64_t* pos_dst;
  int64_t pd_sb;
  int B, H, n;
  int row_bytes, elem_bytes;
};

template <int VW>
__global__ __launch_bounds__(256) void row_copy_kernel(RowCopy c) {
  const int vpr = c.row_bytes / VW;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)c.B * c.H * c.n * vpr;
  if (gid >= total) return;
  const int v = (int)(gid % vpr);
  const int64_t row = gid / vpr;
  const int j = (int)(row % c.n);
  const int64_t bh = row / c.n;
  const int h = (int)(bh % c.H);
  const int b = (int)(bh / c.H);
  int64_t si;
  if (c.idx) {
    si = c.idx[b * c.i_sb + h * c.i_sh + j];
    if (si < 0 || si >= c.src_rows) return;
  } else {
    si = c.src_row0 + j;
  }
  const int64_t di = c.dst_row0 + j;
  const int eb = c.elem_bytes;
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    if (t < c.ntensor && (c.src[t] || c.src_tab[t])) {
      const char* sb = c.src_tab[t] ? c.src_tab[t][b] : c.src[t] + b * c.s_sb[t] * eb;
      char* db = c.dst_tab[t] ? c.dst_tab[t][b] : c.dst[t] + b * c.d_sb[t] * eb;
      const char* sp = sb + (h * c.s_sh[t] + si * c.s_ss[t]) * eb + (int64_t)v * VW;
      char* dp = db + (h * c.d_sh[t] + di * c.d_ss[t]) * eb + (int64_t)v * VW;
      if constexpr (VW == 16) {
        st16(dp, ld16(sp));
      } else if constexpr (VW == 8) {
        *reinterpret_cast<uint64_t*>(dp) = *reinterpret_cast<const uint64_t*>(sp);
      } else if constexpr (VW == 4) {
        *reinterpret_cast<uint32_t*>(dp) = *reinterpret_cast<const uint32_t*>(sp);
      } else {
        *reinterpret_cast<uint16_t*>(dp) = *reinterpret_cast<const uint16_t*>(sp);
      }
    }
  }
  if (c.pos_dst && h == 0 && v == 0) c.pos_dst[b * c.pd_sb + di] = c.pos_src[b * c.ps_sb + si];
}

static int pick_vw(const RowCopy& c) {
  for (int vw = 16; vw >= 2; vw >>= 1) {
    if (c.row_bytes % vw) continue;
    bool ok = true;
    for (int t = 0; t < c.ntensor; ++t) {
      if (!c.src[t] && !c.src_tab[t]) continue;
      const int64_t eb = c.elem_bytes;
      // table rows: the caller guarantees 16-byte aligned row starts
      if (((uintptr_t)c.src[t] % vw) || ((uintptr_t)c.dst[t] % vw)) ok = false;
      if ((c.s_sb[t] * eb) % vw || (c.s_sh[t] * eb) % vw || (c.s_ss[t] * eb) % vw) ok = false;
      if ((c.d_sb[t] * eb) % vw || (c.d_sh[t] * eb) % vw || (c.d_ss[t] * eb) % vw) ok = false;
    }
    if (ok) return vw;
  }
  return 0;
}

static int launch_row_copy(RowCopy& c, hipStream_t st, const char* what) {
  const int vw = pick_vw(c);
  if (vw == 0) return set_error(HC_ERR_INVALID, "%s: rows are not 2-byte aligned", what);
  const int64_t total = (int64_t)c.B * c.H * c.n * (c.row_bytes / vw);
  if (total == 0) return HC_OK;
  const dim3 grid((unsigned)cdiv(total, 256));
  switch (vw) {
    case 16: hipLaunchKernelGGL(row_copy_kernel<16>, grid, dim3(256), 0, st, c); break;
    case 8: hipLaunchKernelGGL(row_copy_kernel<8>, grid, dim3(256), 0, st, c); break;
    case 4: hipLaunchKernelGGL(row_copy_kernel<4>, grid, dim3(256), 0, st, c); break;
    default: hipLaunchKernelGGL(row_copy_kernel<2>, grid, dim3(256), 0, st, c); break;
  }
  return check_launch(what);
}

// Eviction gather with upcast (cache.py:86-125).  Output block:
//   [k fp32 B][H][te][D] | [v fp32 B][H][te][D] | [pos int64 B][te]
// Thread g < 2*B*H*te*D/4 converts four elements of one (tensor, b, h, j)
// row; the next B*te threads copy the positions.  An index outside
// [0, src_rows) writes a zero row and position -1.
struct EvictGather {
  const void* k;
  const void* v;
  int64_t k_sb, k_sh, k_ss, v_sb, v_sh, v_ss;
  const int64_t* idx;
  int64_t i_sb;
  const int64_t* pos;
  int64_t ps_sb;
  float* out;
  int64_t src_rows;
  int B, H, te, D;
};

template <typename T>
__global__ __launch_bounds__(256) void gather_evict_kernel(EvictGather a) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int q = a.D / 4;
  const int64_t per = (int64_t)a.B * a.H * a.te * q;
  if (g < 2 * per) {
    const int t = g >= per;
    const int64_t r = g - t * per;
    const int c = (int)(r % q);
    const int64_t row = r / q;
    const int j = (int)(row % a.te);
    const int64_t bh = row / a.te;
    const int h = (int)(bh % a.H);
    const int b = (int)(bh / a.H);
    const int64_t si = a.idx[b * a.i_sb + j];
    floatx4 f = {0.f, 0.f, 0.f, 0.f};
    if (si >= 0 && si < a.src_rows) {
      const T* src = reinterpret_cast<const T*>(t ? a.v : a.k) +
                     b * (t ? a.v_sb : a.k_sb) + h * (t ? a.v_sh : a.k_sh) + si * (t ? a.v_ss : a.k_ss) + 4 * c;
      if constexpr (sizeof(T) == 4) {
        f = *reinterpret_cast<const floatx4*>(src);
      } else {
        const u32x2 w = *reinterpret_cast<const u32x2*>(src);
        const uint32_t ww[2] = {w[0], w[1]};
        f = floatx4{Unpack<T>::get(ww, 0), Unpack<T>::get(ww, 1), Unpack<T>::get(ww, 2), Unpack<T>::get(ww, 3)};
      }
    }
    *reinterpret_cast<floatx4*>(a.out + t * per * 4 + row * a.D + 4 * c) = f;
  } else if (g < 2 * per + (int64_t)a.B * a.te) {
    const int64_t r = g - 2 * per;
    const int j = (int)(r % a.te), b = (int)(r / a.te);
    const int64_t si = a.idx[b * a.i_sb + j];
    int64_t* pos_out = reinterpret_cast<int64_t*>(a.out + 2 * per * 4);
    pos_out[r] = (si >= 0 && si < a.src_rows) ? a.pos[b * a.ps_sb + si] : -1;
  }
}

}  // namespace hc

using namespace hc;

extern "C" int hc_topk_keep(int64_t B, int64_t H, int64_t S, const float* scores, int64_t s_sb, int64_t s_sh,
                            int64_t window, int64_t budget, int64_t* keep, int64_t* evicted, void* stream) {
  HC_REQUIRE(B > 0 && H > 0 && S > 0, "topk: empty shape");
  HC_REQUIRE(window >= 0 && budget >= 0, "topk: negative window/budget");
  HC_REQUIRE(S < ((int64_t)1 << 31), "topk: S too large");
  HC_REQUIRE(B <= 65535 && H <= 65535, "topk: grid too large");
  HC_REQUIRE(scores && keep, "topk: null pointer");
  const int64_t win = window < S ? window : S;
  const int64_t prefix = S - win;
  int64_t kp = budget - win;
  if (kp > prefix) kp = prefix;
  if (kp < 0) kp = 0;
  const size_t lds = (kp > 0 && prefix <= kTopkCache) ? (size_t)prefix * 4 : 0;
  // set on every call: the attribute is per device, and a process may drive several
  if (lds > 65536 && hipFuncSetAttribute((const void*)topk_keep_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         kTopkCache * 4) != hipSuccess)
    return set_error(HC_ERR_HIP, "topk: cannot raise the dynamic LDS limit to %d bytes", kTopkCache * 4);
  hipLaunchKernelGGL(topk_keep_kernel, dim3((unsigned)H, (unsigned)B), dim3(kTopkThreads), lds,
                     reinterpret_cast<hipStream_t>(stream), scores, s_sb, s_sh, (int)H, (int)prefix, (int)kp,
                     (int)win, keep, evicted);
  return check_launch("topk_keep");
}

namespace {

// The chunked selection pays for its chain of launches (about 35 us) where
// one workgroup per row is slow: rows longer than the kTopkCache keys that
// workgroup keeps in LDS (it then re-reads them from memory on every pass),
// in grids of fewer rows than CUs.  At 64k keys x 32 rows the selection took
// 110 us in one workgroup per row and 51 us chunked; at 32k keys x 128 rows,
// LDS-cached, 59 us against 64.
bool topk_chunked(int64_t rows, int64_t prefix, int64_t kp) {
  return kp > 0 && rows < 256 && prefix > kTopkCache;
}

struct TopkWs {
  int64_t state_off, counts_off, total;
};

TopkWs topk_ws_layout(int64_t rows, int64_t nchunk) {
  const auto al = [](int64_t x) { return (x + 255) & ~(int64_t)255; };
  TopkWs w;
  w.state_off = al(rows * kDigitBins * 4);
  w.counts_off = w.state_off + al(rows * kTopkState * 4);
  w.total = w.counts_off + al(rows * nchunk * 2 * 4);
  return w;
}

void topk_counts(int64_t S, int64_t window, int64_t budget, int64_t* win, int64_t* prefix, int64_t* kp) {
  *win = window < S ? window : S;
  *prefix = S - *win;
  *kp = budget - *win;
  if (*kp > *prefix) *kp = *prefix;
  if (*kp < 0) *kp = 0;
}

}  // namespace

extern "C" int64_t hc_topk_keep_workspace_size(int64_t B, int64_t H, int64_t S, int64_t window, int64_t budget) {
  if (B <= 0 || H <= 0 || S <= 0 || window < 0 || budget < 0) return 0;
  int64_t win, prefix, kp;
  topk_counts(S, window, budget, &win, &prefix, &kp);
  if (!topk_chunked(B * H, prefix, kp)) return 0;
  return topk_ws_layout(B * H, cdiv(prefix, (int64_t)kTopkChunk)).total;
}

extern "C" int hc_topk_keep_ws(int64_t B, int64_t H, int64_t S, const float* scores, int64_t s_sb, int64_t s_sh,
                               int64_t window, int64_t budget, int64_t* keep, int64_t* evicted, void* ws,
                               int64_t ws_bytes, void* stream) {
  HC_REQUIRE(B > 0 && H > 0 && S > 0, "topk: empty shape");
  HC_REQUIRE(window >= 0 && budget >= 0, "topk: negative window/budget");
  HC_REQUIRE(S < ((int64_t)1 << 31), "topk: S too large");
  HC_REQUIRE(B <= 65535 && H <= 65535, "topk: grid too large");
  HC_REQUIRE(scores && keep, "topk: null pointer");
  int64_t win, prefix, kp;
  topk_counts(S, window, budget, &win, &prefix, &kp);
  if (ws == nullptr || !topk_chunked(B * H, prefix, kp))
    return hc_topk_keep(B, H, S, scores, s_sb, s_sh, window, budget, keep, evicted, stream);
  const int64_t nchunk = cdiv(prefix, (int64_t)kTopkChunk);
  const TopkWs lay = topk_ws_layout(B * H, nchunk);
  HC_REQUIRE(ws_bytes >= lay.total, "topk: workspace of %lld bytes given, %lld needed", (long long)ws_bytes,
             (long long)lay.total);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  uint32_t* ghist = static_cast<uint32_t*>(ws);
  uint32_t* state = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + lay.state_off);
  int* counts = reinterpret_cast<int*>(static_cast<char*>(ws) + lay.counts_off);
  const dim3 rows((unsigned)H, (unsigned)B), chunks((unsigned)nchunk, (unsigned)H, (unsigned)B);
  hipLaunchKernelGGL(topk_init_kernel, rows, dim3(256), 0, st, (int)H, (uint32_t)kp, ghist, state);
  for (int pass = 0; pass < 3; ++pass) {
    hipLaunchKernelGGL(topk_hist_kernel, chunks, dim3(kTopkThreads), 0, st, scores, s_sb, s_sh, (int)H, (int)prefix,
                       pass, ghist, (const uint32_t*)state);
    hipLaunchKernelGGL(topk_digit_kernel, rows, dim3(kTopkThreads), 0, st, (int)H, pass, ghist, state);
  }
  hipLaunchKernelGGL(topk_count_kernel, chunks, dim3(kTopkThreads), 0, st, scores, s_sb, s_sh, (int)H,
                     (int)prefix, (int)nchunk, (const uint32_t*)state, counts);
  hipLaunchKernelGGL(topk_emit_kernel, chunks, dim3(kTopkThreads), 0, st, scores, s_sb, s_sh, (int)H, (int)prefix,
                     (int)nchunk, (int)kp, (int)win, (const uint32_t*)state, (const int*)counts, keep, evicted);
  return check_launch("topk_keep_ws");
}

extern "C" int hc_gather_rows(int64_t B, int64_t H, int64_t n, int64_t D, int64_t elem_bytes, const int64_t* idx,
                              int64_t i_sb, int64_t i_sh, int64_t src_rows, int64_t dst_row0, const void* src1,
                              int64_t s1_sb, int64_t s1_sh, int64_t s1_ss, void* dst1, int64_t d1_sb, int64_t d1_sh,
                              int64_t d1_ss, const void* src2, int64_t s2_sb, int64_t s2_sh, int64_t s2_ss,
                              void* dst2, int64_t d2_sb, int64_t d2_sh, int64_t d2_ss, const void* src3,
                              int64_t s3_sb, int64_t s3_sh, int64_t s3_ss, void* dst3, int64_t d3_sb, int64_t d3_sh,
                              int64_t d3_ss, const int64_t* pos_src, int64_t ps_sb, int64_t* pos_dst, int64_t pd_sb,
                              void* stream) {
  HC_REQUIRE(B > 0 && H > 0 && n >= 0 && D > 0, "gather: bad shape");
  HC_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8, "gather: bad elem_bytes");
  HC_REQUIRE(idx != nullptr, "gather: null index");
  HC_REQUIRE(src1 && dst1, "gather: first tensor required");
  HC_REQUIRE((src2 == nullptr) == (dst2 == nullptr) && (src3 == nullptr) == (dst3 == nullptr),
             "gather: src/dst pairs must both be set");
  HC_REQUIRE((pos_src == nullptr) == (pos_dst == nullptr), "gather: pos_src/pos_dst must both be set");
  HC_REQUIRE(D * elem_bytes % 2 == 0, "gather: odd row size");
  if (n == 0) return HC_OK;
  RowCopy c{};
  c.src[0] = (const char*)src1; c.dst[0] = (char*)dst1;
  c.src[1] = (const char*)src2; c.dst[1] = (char*)dst2;
  c.src[2] = (const char*)src3; c.dst[2] = (char*)dst3;
  c.s_sb[0] = s1_sb; c.s_sh[0] = s1_sh; c.s_ss[0] = s1_ss; c.d_sb[0] = d1_sb; c.d_sh[0] = d1_sh; c.d_ss[0] = d1_ss;
  c.s_sb[1] = s2_sb; c.s_sh[1] = s2_sh; c.s_ss[1] = s2_ss; c.d_sb[1] = d2_sb; c.d_sh[1] = d2_sh; c.d_ss[1] = d2_ss;
  c.s_sb[2] = s3_sb; c.s_sh[2] = s3_sh; c.s_ss[2] = s3_ss; c.d_sb[2] = d3_sb; c.d_sh[2] = d3_sh; c.d_ss[2] = d3_ss;
  c.ntensor = 3;
  c.idx = idx; c.i_sb = i_sb; c.i_sh = i_sh;
  c.src_rows = src_rows; c.src_row0 = 0; c.dst_row0 = dst_row0;
  c.pos_src = pos_src; c.ps_sb = ps_sb; c.pos_dst = pos_dst; c.pd_sb = pd_sb;
  c.B = (int)B; c.H = (int)H; c.n = (int)n;
  c.row_bytes = (int)(D * elem_bytes);
  c.elem_bytes = (int)elem_bytes;
  return launch_row_copy(c, reinterpret_cast<hipStream_t>(stream), "gather_rows");
}

extern "C" int hc_gather_rows_tab(int64_t R, int64_t H, int64_t n, int64_t D, int64_t elem_bytes,
                                  const int64_t* idx, int64_t i_sb, int64_t i_sh, int64_t src_rows, int64_t dst_row0,
                                  const void* const* src1_rows, int64_t s1_sh, int64_t s1_ss,
                                  void* const* dst1_rows, int64_t d1_sh, int64_t d1_ss,
                                  const void* const* src2_rows, int64_t s2_sh, int64_t s2_ss,
                                  void* const* dst2_rows, int64_t d2_sh, int64_t d2_ss, void* stream) {
  HC_REQUIRE(R > 0 && H > 0 && n >= 0 && D > 0, "gather_tab: bad shape");
  HC_REQUIRE(R <= 65535, "gather_tab: too many rows");
  HC_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8, "gather_tab: bad elem_bytes");
  HC_REQUIRE(idx != nullptr, "gather_tab: null index");
  HC_REQUIRE(src1_rows && dst1_rows, "gather_tab: first tensor tables required");
  HC_REQUIRE((src2_rows == nullptr) == (dst2_rows == nullptr), "gather_tab: src/dst tables must both be set");
  HC_REQUIRE(D * elem_bytes % 2 == 0, "gather_tab: odd row size");
  if (n == 0) return HC_OK;
  RowCopy c{};
  c.src_tab[0] = reinterpret_cast<const char* const*>(src1_rows);
  c.dst_tab[0] = reinterpret_cast<char* const*>(dst1_rows);
  c.src_tab[1] = reinterpret_cast<const char* const*>(src2_rows);
  c.dst_tab[1] = reinterpret_cast<char* const*>(dst2_rows);
  c.s_sh[0] = s1_sh; c.s_ss[0] = s1_ss; c.d_sh[0] = d1_sh; c.d_ss[0] = d1_ss;
  c.s_sh[1] = s2_sh; c.s_ss[1] = s2_ss; c.d_sh[1] = d2_sh; c.d_ss[1] = d2_ss;
  c.ntensor = 2;
  c.idx = idx; c.i_sb = i_sb; c.i_sh = i_sh;
  c.src_rows = src_rows; c.src_row0 = 0; c.dst_row0 = dst_row0;
  c.B = (int)R; c.H = (int)H; c.n = (int)n;
  c.row_bytes = (int)(D * elem_bytes);
  c.elem_bytes = (int)elem_bytes;
  return launch_row_copy(c, reinterpret_cast<hipStream_t>(stream), "gather_rows_tab");
}

extern "C" int hc_append_rows(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, int64_t row, const void* k_src,
                              int64_t ks_sb, int64_t ks_sh, int64_t ks_ss, void* k_dst, int64_t kd_sb, int64_t kd_sh,
                              int64_t kd_ss, const void* v_src, int64_t vs_sb, int64_t vs_sh, int64_t vs_ss,
                              void* v_dst, int64_t vd_sb, int64_t vd_sh, int64_t vd_ss, const void* p_src,
                              int64_t ps_sb, int64_t ps_sh, int64_t ps_ss, void* p_dst, int64_t pd_sb, int64_t pd_sh,
                              int64_t pd_ss, const int64_t* pos_src, int64_t pos_s_sb, int64_t* pos_dst,
                              int64_t pos_d_sb, void* stream) {
  const int es = dtype_size(dtype);
  HC_REQUIRE(es > 0, "append: bad dtype %d", dtype);
  HC_REQUIRE(B > 0 && H > 0 && T >= 0 && D > 0 && row >= 0, "append: bad shape");
  HC_REQUIRE(k_src && k_dst, "append: key tensors required");
  HC_REQUIRE((v_src == nullptr) == (v_dst == nullptr) && (p_src == nullptr) == (p_dst == nullptr),
             "append: src/dst pairs must both be set");
  HC_REQUIRE((pos_src == nullptr) == (pos_dst == nullptr), "append: pos_src/pos_dst must both be set");
  if (T == 0) return HC_OK;
  RowCopy c{};
  c.src[0] = (const char*)k_src; c.dst[0] = (char*)k_dst;
  c.src[1] = (const char*)v_src; c.dst[1] = (char*)v_dst;
  c.src[2] = (const char*)p_src; c.dst[2] = (char*)p_dst;
  c.s_sb[0] = ks_sb; c.s_sh[0] = ks_sh; c.s_ss[0] = ks_ss; c.d_sb[0] = kd_sb; c.d_sh[0] = kd_sh; c.d_ss[0] = kd_ss;
  c.s_sb[1] = vs_sb; c.s_sh[1] = vs_sh; c.s_ss[1] = vs_ss; c.d_sb[1] = vd_sb; c.d_sh[1] = vd_sh; c.d_ss[1] = vd_ss;
  c.s_sb[2] = ps_sb; c.s_sh[2] = ps_sh; c.s_ss[2] = ps_ss; c.d_sb[2] = pd_sb; c.d_sh[2] = pd_sh; c.d_ss[2] = pd_ss;
  c.ntensor = 3;
  c.idx = nullptr; c.src_rows = T; c.src_row0 = 0; c.dst_row0 = row;
  c.pos_src = pos_src; c.ps_sb = pos_s_sb; c.pos_dst = pos_dst; c.pd_sb = pos_d_sb;
  c.B = (int)B; c.H = (int)H; c.n = (int)T;
  c.row_bytes = (int)(D * es);
  c.elem_bytes = es;
  return launch_row_copy(c, reinterpret_cast<hipStream_t>(stream), "append_rows");
}

extern "C" int64_t hc_gather_evict_bytes(int64_t B, int64_t H, int64_t te, int64_t D) {
  if (B <= 0 || H <= 0 || te < 0 || D <= 0) return 0;
  return 2 * B * H * te * D * (int64_t)sizeof(float) + B * te * (int64_t)sizeof(int64_t);
}

extern "C" int hc_gather_evict(int dtype, int64_t B, int64_t H, int64_t te, int64_t D, const int64_t* idx,
                               int64_t i_sb, int64_t src_rows, const void* k_src, int64_t k_sb, int64_t k_sh,
                               int64_t k_ss, const void* v_src, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                               const int64_t* pos_src, int64_t ps_sb, void* dev_out, void* host_out,
                               void* stream) {
  HC_REQUIRE(dtype == HC_DTYPE_F32 || dtype == HC_DTYPE_F16 || dtype == HC_DTYPE_BF16, "gather_evict: bad dtype %d",
             dtype);
  HC_REQUIRE(B > 0 && H > 0 && te >= 0 && D > 0 && D % 4 == 0, "gather_evict: bad shape (D %% 4 == 0)");
  HC_REQUIRE(B * H * te * (D / 4) < ((int64_t)1 << 38), "gather_evict: too large for one launch");
  HC_REQUIRE(idx && k_src && v_src && pos_src && dev_out, "gather_evict: null pointer");
  const int es = dtype_size(dtype);
  const int64_t al = 4 * es;  // four elements per load
  HC_REQUIRE((uintptr_t)k_src % al == 0 && (uintptr_t)v_src % al == 0 && (k_sb * es) % al == 0 &&
                 (k_sh * es) % al == 0 && (k_ss * es) % al == 0 && (v_sb * es) % al == 0 && (v_sh * es) % al == 0 &&
                 (v_ss * es) % al == 0 && (uintptr_t)dev_out % 16 == 0,
             "gather_evict: rows must be %lld-byte aligned", (long long)al);
  if (te == 0) return HC_OK;
  EvictGather a{};
  a.k = k_src; a.v = v_src;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss; a.v_sb = v_sb; a.v_sh = v_sh; a.v_ss = v_ss;
  a.idx = idx; a.i_sb = i_sb; a.pos = pos_src; a.ps_sb = ps_sb;
  a.out = reinterpret_cast<float*>(dev_out);
  a.src_rows = src_rows;
  a.B = (int)B; a.H = (int)H; a.te = (int)te; a.D = (int)D;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t threads = 2 * B * H * te * (D / 4) + B * te;
  const dim3 grid((unsigned)cdiv(threads, 256));
  if (dtype == HC_DTYPE_F16) hipLaunchKernelGGL(gather_evict_kernel<half_t>, grid, dim3(256), 0, st, a);
  else if (dtype == HC_DTYPE_BF16) hipLaunchKernelGGL(gather_evict_kernel<bf16_t>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(gather_evict_kernel<float>, grid, dim3(256), 0, st, a);
  int rc = check_launch("gather_evict");
  if (rc != HC_OK) return rc;
  if (host_out) {
    const hipError_t e = hipMemcpyAsync(host_out, dev_out, (size_t)hc_gather_evict_bytes(B, H, te, D),
                                        hipMemcpyDeviceToHost, st);
    if (e != hipSuccess) return set_error(HC_ERR_HIP, "gather_evict: hipMemcpyAsync: %s", hipGetErrorString(e));
  }
  return HC_OK;
}
