// Device search index of the cold store: the search vectors of every
// (batch row, vector head) kept in HBM, scanned and ranked on the GPU.
//
// The reference searches its CPU faiss.IndexFlatIP per (layer, batch row)
// (controller.py:223-232, 274-293).  The host store (hc_cold.cpp) reproduces
// that search exactly, but a scan of every stored vector per search is bound
// by host memory: at 16 batch rows of 30 720 evicted tokens and 8 KV heads a
// layer's search reads 2 GB, which host threads cannot finish within a
// retrieval window of a fast decode loop.  Here the same vectors live in HBM
// in tiles of 64 slots, [B][VH][capT/64][VD][64] fp32: a wave scores one tile,
// reading one dimension of its 64 slots per load, and a tile's dimensions are
// one contiguous run.  The same arithmetic as the host runs on the GPU:
//   * vectors: the head mean (fp64, heads in order) or one head's pre-RoPE key,
//     cropped or zero-padded to VD, divided by max(||x||, 1e-12) with the
//     squares summed in fp64 in dimension order, rounded to fp32
//     (hc_cold.cpp ColdStore::set_vec);
//   * inner products: fp64, dimension order (fp32 x fp32 products are exact in
//     fp64, so an fma chain and the host's multiply-then-add agree);
//   * ranking: inner product descending, ties to the older token (smaller
//     logical index), the top R in rank order (ColdStore::select).
// So the hits equal the host store's bit for bit.  The key/value rows stay in
// the host store; only the hits' logical indices go back to the host.
#include "hc_common.h"

namespace hc {

constexpr int kIdxMaxB = 64;      // batch rows per search launch
constexpr int kIdxMaxVD = 1024;   // vector width (query staged in LDS)
constexpr int kIdxMaxR = 1024;    // hits per (row, head)
constexpr int kIdxThreads = 1024;

struct IndexAddArgs {
  const float* kpre;  // token t, head h of row b at kpre + b*k_sb + h*k_sh + t*k_st
  int64_t k_sb, k_sh, k_st;
  const int32_t* slot_of;  // [B][te]: physical slot of token t, or -1 (not stored)
  float* vec;              // [B][VH][capT/64][VD][64]
  int64_t capT;
  int B, H, D, VH, VD, te, normalize;
};

// Offset of slot s, dimension d in a (row, head) plane [capT/64][VD][64].
__device__ __forceinline__ int64_t vec_at(int64_t s, int d, int VD) {
  return (s >> 6) * (int64_t)VD * 64 + (int64_t)d * 64 + (s & 63);
}

// Grid (cdiv(te, kAddTok), VH, B), block kAddThreads: kAddTok tokens of one
// (row, vector head) per workgroup, their values staged in LDS kAddChunk
// dimensions at a time with coalesced loads (the head mean summed in fp64,
// heads in order, then divided by H).  One thread per token runs the norm's
// fp64 chain over the dimensions in order; then every dimension is divided
// and written, a wave covering consecutive slots of one dimension.  A token's
// values are recomputed for the second pass when they span several chunks
// (the same operations, so the same values).
constexpr int kAddThreads = 256;
constexpr int kAddTok = 32;
constexpr int kAddChunk = 128;

__global__ __launch_bounds__(kAddThreads) void index_add_kernel(IndexAddArgs a) {
#pragma clang fp contract(off)
  __shared__ double xs[kAddTok][kAddChunk + 1];
  __shared__ double den_s[kAddTok];
  __shared__ int slot_s[kAddTok];
  const int t0 = blockIdx.x * kAddTok, vh = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int n = min(a.D, a.VD);
  const int nchunks = (a.VD + kAddChunk - 1) / kAddChunk;
  if (tid < kAddTok) {
    const int t = t0 + tid;
    const int slot = t < a.te ? a.slot_of[(int64_t)b * a.te + t] : -1;
    slot_s[tid] = (slot < 0 || slot >= a.capT) ? -1 : slot;
  }
  const float* kb = a.kpre + b * a.k_sb;
  auto fill = [&](int c0) {
    for (int i = tid; i < kAddTok * kAddChunk; i += kAddThreads) {
      const int tl = i / kAddChunk, dd = i % kAddChunk, d = c0 + dd, t = t0 + tl;
      double x = 0.0;
      if (t < a.te && d < n) {
        const float* kp = kb + (int64_t)t * a.k_st + d;
        if (a.VH == 1) {
          double s = 0.0;
          for (int h = 0; h < a.H; ++h) s += (double)kp[h * a.k_sh];
          x = s / (double)a.H;
        } else {
          x = (double)kp[vh * a.k_sh];
        }
      }
      xs[tl][dd] = x;
    }
  };
  double ss = 0.0;
  for (int c = 0; c < nchunks; ++c) {
    if (a.normalize || c == 0) {
      __syncthreads();
      fill(c * kAddChunk);
      __syncthreads();
    }
    if (a.normalize && tid < kAddTok) {
      const int w = min(kAddChunk, a.VD - c * kAddChunk);
      for (int dd = 0; dd < w; ++dd) {
        const double x = xs[tid][dd];
        ss += x * x;
      }
    }
  }
  if (tid < kAddTok) den_s[tid] = a.normalize ? fmax(sqrt(ss), 1e-12) : 1.0;
  float* o = a.vec + (int64_t)(b * a.VH + vh) * a.VD * a.capT;
  for (int c = 0; c < nchunks; ++c) {
    if (c > 0 || (a.normalize && nchunks > 1)) {
      __syncthreads();
      fill(c * kAddChunk);
    }
    __syncthreads();
    const int w = min(kAddChunk, a.VD - c * kAddChunk);
    for (int i = tid; i < kAddTok * w; i += kAddThreads) {
      const int dd = i / kAddTok, tl = i % kAddTok, slot = slot_s[tl];
      if (slot >= 0) o[vec_at(slot, c * kAddChunk + dd, a.VD)] = (float)(xs[tl][dd] / den_s[tl]);
    }
  }
}

struct IndexSearchArgs {
  const float* q;  // query of (row b, head vh) at q + b*q_sb + vh*q_sh, q_dim floats
  int64_t q_sb, q_sh;
  const float* vec;
  int64_t capT;
  uint64_t* keys;  // scratch [B][VH][capT]
  int64_t* hits;   // [B][VH][R]: logical indices in rank order, -1 past the hits
  int64_t* hits_mapped;  // the same, into pinned host memory through its device mapping (or null)
  int B, VH, VD, R, cap, q_dim, normalize_q;
  int size[kIdxMaxB], head[kIdxMaxB];  // ring state of each row's store
};

// A double's bits as an unsigned key that orders like the value (-0 as +0).
__device__ __forceinline__ uint64_t ordered_key(double x) {
  if (x == 0.0) x = 0.0;
  const uint64_t u = __double_as_longlong(x);
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

// Scoring: grid (cdiv(max size, kScoreSlots), VH, B), block kScoreThreads.
// Each thread scores kScorePer slots of one (row, head), one per 64-slot tile
// of its wave: the fp64 inner product in dimension order, stored as an order
// key.  A wave reads one dimension of its tile per load, so the grid streams
// the vectors at full width whatever B and VH are.
constexpr int kScoreThreads = 256;
constexpr int kScorePer = 2;
constexpr int kScoreSlots = kScoreThreads * kScorePer;

__global__ __launch_bounds__(kScoreThreads) void index_score_kernel(IndexSearchArgs a) {
#pragma clang fp contract(off)
  __shared__ float qv[kIdxMaxVD];
  __shared__ double den_s;
  const int vh = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int size = a.size[b];
  const int p0 = blockIdx.x * kScoreSlots + tid;
  if (blockIdx.x * kScoreSlots >= size) return;  // uniform per workgroup
  const float* qs = a.q + b * a.q_sb + vh * a.q_sh;
  // the query: cropped or zero-padded to VD; its norm is one fp64 chain in
  // dimension order (thread 0), each dimension divided by its own thread
  if (tid == 0) {
    double den = 1.0;
    if (a.normalize_q) {
      double ss = 0.0;
      for (int d = 0; d < a.VD; ++d) {
        const double x = d < a.q_dim ? (double)qs[d] : 0.0;
        ss += x * x;
      }
      den = fmax(sqrt(ss), 1e-12);
    }
    den_s = den;
  }
  __syncthreads();
  for (int d = tid; d < a.VD; d += kScoreThreads)
    qv[d] = d < a.q_dim ? (a.normalize_q ? (float)((double)qs[d] / den_s) : qs[d]) : 0.0f;
  __syncthreads();
  const float* vb = a.vec + (int64_t)(b * a.VH + vh) * a.VD * a.capT;
  uint64_t* kb = a.keys + (int64_t)(b * a.VH + vh) * a.capT;
  double acc[kScorePer];
#pragma unroll
  for (int j = 0; j < kScorePer; ++j) acc[j] = 0.0;
  // slots past the size are scored from the allocation's tail (clamped below
  // capT) and not stored
  const float* tile[kScorePer];
#pragma unroll
  for (int j = 0; j < kScorePer; ++j) {
    const int p = min(p0 + j * kScoreThreads, (int)a.capT - 1);
    tile[j] = vb + vec_at(p, 0, a.VD);
  }
#pragma unroll 8
  for (int d = 0; d < a.VD; ++d) {
    const double qd = (double)qv[d];
#pragma unroll
    for (int j = 0; j < kScorePer; ++j) acc[j] += qd * (double)tile[j][d * 64];
  }
#pragma unroll
  for (int j = 0; j < kScorePer; ++j) {
    const int p = p0 + j * kScoreThreads;
    if (p < size) kb[p] = ordered_key(acc[j]);
  }
}

// Selection: grid (VH, B), block kIdxThreads, one (row, head) per workgroup.
// The m-th largest key T by radix select over 8-bit digits (most significant
// first).  Once the keys sharing the selected prefix fit kCand, they are
// copied to LDS and the remaining digits are selected there, so the scored
// keys are read from memory only a few times.  Then one pass collects the
// keys above T and the logical indices of the keys equal to T, of which the
// `remaining` oldest are taken; a bitonic sort puts the m hits in rank order.
constexpr int kCand = 4096;
constexpr int kEqCap = 1024;
constexpr int kKeyBatch = 8;  // keys loaded per thread before any is used

// f(p, key) for every p < size, thread tid taking p = tid (mod kIdxThreads),
// its loads issued kKeyBatch at a time.
template <typename F>
__device__ __forceinline__ void for_keys(const uint64_t* kb, int size, int tid, F&& f) {
  for (int base = 0; base < size; base += kIdxThreads * kKeyBatch) {
    uint64_t k[kKeyBatch];
#pragma unroll
    for (int j = 0; j < kKeyBatch; ++j) {
      const int p = base + j * kIdxThreads + tid;
      k[j] = p < size ? kb[p] : 0;
    }
#pragma unroll
    for (int j = 0; j < kKeyBatch; ++j) {
      const int p = base + j * kIdxThreads + tid;
      if (p < size) f(p, k[j]);
    }
  }
}

__global__ __launch_bounds__(kIdxThreads) void index_select_kernel(IndexSearchArgs a) {
  __shared__ uint32_t hist[256];
  __shared__ uint64_t ck[kCand];
  __shared__ uint64_t wk[kIdxMaxR];
  __shared__ int32_t wl[kIdxMaxR];
  __shared__ int32_t eql[kEqCap];
  __shared__ int32_t scan[kIdxThreads];
  __shared__ int sel_digit, sel_above, sel_count, n_cand, n_above, n_eq;
  __shared__ int wave_tot[4];
  const int vh = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int size = a.size[b], head = a.head[b];
  const bool full = size >= a.cap;
  int64_t* out = a.hits + (int64_t)(b * a.VH + vh) * a.R;
  const uint64_t* kb = a.keys + (int64_t)(b * a.VH + vh) * a.capT;
  const int m = min(a.R, size);
  if (m == 0) {  // uniform per workgroup
    for (int j = tid; j < a.R; j += kIdxThreads) {
      out[j] = -1;
      if (a.hits_mapped) a.hits_mapped[(int64_t)(b * a.VH + vh) * a.R + j] = -1;
    }
    return;
  }
  auto logical = [&](int p) { return full ? (p - head + a.cap) % a.cap : p; };

  uint64_t prefix = 0;
  int remaining = m;
  bool in_lds = false;
  int nc = 0;
  for (int shift = 56; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    const uint64_t high = shift == 56 ? 0ull : ~((1ull << (shift + 8)) - 1);
    if (in_lds) {
      for (int i = tid; i < nc; i += kIdxThreads) {
        const uint64_t k = ck[i];
        if ((k & high) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
      }
    } else {
      for_keys(kb, size, tid, [&](int, uint64_t k) {
        if ((k & high) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
      });
    }
    __syncthreads();
    // the digit holding the remaining-th largest key: counts summed in
    // descending digit order (thread i holds digit 255 - i), wave scans, then
    // the four waves' totals
    int v = 0, incl = 0;
    if (tid < 256) {
      const int lane = tid & 63;
      v = (int)hist[255 - tid];
      incl = v;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int u = __shfl_up(incl, off, 64);
        if (lane >= off) incl += u;
      }
      if (lane == 63) wave_tot[tid >> 6] = incl;
    }
    __syncthreads();
    if (tid < 256) {
      const int dg = 255 - tid;
      for (int i = 0; i < (tid >> 6); ++i) incl += wave_tot[i];
      const int excl = incl - v;
      if (excl < remaining && incl >= remaining) {
        sel_digit = dg;
        sel_above = excl;
        sel_count = v;
      }
    }
    __syncthreads();
    prefix |= (uint64_t)sel_digit << shift;
    remaining -= sel_above;
    if (!in_lds && shift > 0 && sel_count <= kCand) {
      // the keys sharing the prefix so far, into LDS for the lower digits
      const uint64_t hi_new = ~((1ull << shift) - 1);
      if (tid == 0) n_cand = 0;
      __syncthreads();
      for_keys(kb, size, tid, [&](int, uint64_t k) {
        if ((k & hi_new) == prefix) ck[atomicAdd(&n_cand, 1)] = k;
      });
      __syncthreads();
      nc = n_cand;
      in_lds = true;
    }
    __syncthreads();
  }
  const uint64_t T = prefix;  // the m-th largest key; `remaining` keys equal to it are taken

  // keys above T (any order; sorted below) and the logical indices of keys equal to T
  if (tid == 0) {
    n_above = 0;
    n_eq = 0;
  }
  __syncthreads();
  for_keys(kb, size, tid, [&](int p, uint64_t k) {
    if (k > T) {
      const int i = atomicAdd(&n_above, 1);
      wk[i] = k;
      wl[i] = logical(p);
    } else if (k == T) {
      const int j = atomicAdd(&n_eq, 1);
      if (j < kEqCap) eql[j] = logical(p);
    }
  });
  __syncthreads();
  const int above = n_above, neq = n_eq;
  if (neq <= kEqCap) {
    // the `remaining` smallest logical indices among the ties (all distinct)
    for (int j = tid; j < neq; j += kIdxThreads) {
      const int l = eql[j];
      int rank = 0;
      if (neq > remaining)
        for (int i = 0; i < neq; ++i) rank += eql[i] < l;
      else
        rank = j;
      if (rank < remaining) {
        wk[above + rank] = T;
        wl[above + rank] = l;
      }
    }
  } else {
    // more ties than the buffer holds: a prefix sum over per-thread runs of
    // logical indices finds the `remaining` oldest
    const int chunk = (size + kIdxThreads - 1) / kIdxThreads;
    const int l0 = min(size, tid * chunk), l1 = min(size, l0 + chunk);
    int cnt = 0;
    for (int l = l0; l < l1; ++l) cnt += kb[full ? (head + l) % a.cap : l] == T;
    scan[tid] = cnt;
    __syncthreads();
    for (int off = 1; off < kIdxThreads; off <<= 1) {  // inclusive scan
      const int v = tid >= off ? scan[tid - off] : 0;
      __syncthreads();
      scan[tid] += v;
      __syncthreads();
    }
    int rank = scan[tid] - cnt;
    for (int l = l0; l < l1 && rank < remaining; ++l)
      if (kb[full ? (head + l) % a.cap : l] == T) {
        wk[above + rank] = T;
        wl[above + rank] = l;
        ++rank;
      }
  }
  __syncthreads();

  // the m hits in rank order: key descending, logical index ascending
  int P = 1;
  while (P < m) P <<= 1;
  if (tid < P && tid >= m) {
    wk[tid] = 0;
    wl[tid] = 0x7fffffff;
  }
  __syncthreads();
  for (int k = 2; k <= P; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      const int i = tid, o = i ^ j;
      if (i < P && o > i) {
        const bool desc_block = (i & k) == 0;  // this block sorts into rank order
        const uint64_t ki = wk[i], ko = wk[o];
        const int li = wl[i], lo = wl[o];
        const bool o_first = ko > ki || (ko == ki && lo < li);  // o ranks before i
        if (o_first == desc_block) {
          wk[i] = ko;
          wk[o] = ki;
          wl[i] = lo;
          wl[o] = li;
        }
      }
      __syncthreads();
    }
  for (int j = tid; j < a.R; j += kIdxThreads) {
    const int64_t h = j < m ? (int64_t)wl[j] : -1;
    out[j] = h;
    if (a.hits_mapped) a.hits_mapped[(int64_t)(b * a.VH + vh) * a.R + j] = h;
  }
}

}  // namespace hc

using namespace hc;

extern "C" int hc_index_add(int64_t B, int64_t H, int64_t D, int64_t VH, int64_t VD, int normalize,
                            const float* kpre, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t te,
                            const int32_t* slot_of, float* vec, int64_t capT, void* stream) {
  HC_REQUIRE(B > 0 && H > 0 && D > 0 && VD > 0 && te >= 0 && (VH == 1 || VH == H) && capT > 0 && capT % 64 == 0,
             "index_add: bad shape (B=%lld H=%lld D=%lld VH=%lld VD=%lld te=%lld)", (long long)B, (long long)H,
             (long long)D, (long long)VH, (long long)VD, (long long)te);
  HC_REQUIRE(kpre && slot_of && vec, "index_add: null pointer");
  HC_REQUIRE(B * te * VH < ((int64_t)1 << 40), "index_add: too many tokens");
  if (te == 0) return HC_OK;
  IndexAddArgs a{kpre, k_sb, k_sh, k_st, slot_of, vec, capT, (int)B, (int)H, (int)D, (int)VH, (int)VD, (int)te,
                 normalize};
  HC_REQUIRE(B <= 65535 && VH <= 65535, "index_add: grid too large");
  hipLaunchKernelGGL(index_add_kernel, dim3((unsigned)cdiv(te, kAddTok), (unsigned)VH, (unsigned)B),
                     dim3(kAddThreads), 0, reinterpret_cast<hipStream_t>(stream), a);
  return check_launch("index_add");
}

extern "C" int hc_index_search(int64_t B, int64_t VH, int64_t VD, int64_t cap, const float* q, int64_t q_sb,
                               int64_t q_sh, int64_t q_dim, int normalize_q, const float* vec, int64_t capT,
                               const int64_t* sizes, const int64_t* heads, int64_t R, uint64_t* keys, int64_t* hits,
                               int64_t* hits_host, void* wait_event, void* done_event, void* stream) {
  HC_REQUIRE(B > 0 && B <= kIdxMaxB, "index_search: batch rows %lld outside 1..%d", (long long)B, kIdxMaxB);
  HC_REQUIRE(VH > 0 && VD > 0 && VD <= kIdxMaxVD && q_dim > 0, "index_search: vector width %lld outside 1..%d",
             (long long)VD, kIdxMaxVD);
  HC_REQUIRE(R > 0 && R <= kIdxMaxR, "index_search: R=%lld outside 1..%d", (long long)R, kIdxMaxR);
  HC_REQUIRE(cap > 0 && capT >= cap && capT % 64 == 0 && capT < (1ll << 31), "index_search: bad capacity");
  HC_REQUIRE(q && vec && sizes && heads && keys && hits, "index_search: null pointer");
  IndexSearchArgs a{};
  a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.vec = vec; a.capT = capT; a.keys = keys; a.hits = hits;
  a.B = (int)B; a.VH = (int)VH; a.VD = (int)VD; a.R = (int)R; a.cap = (int)cap; a.q_dim = (int)q_dim;
  a.normalize_q = normalize_q;
  for (int64_t b = 0; b < B; ++b) {
    HC_REQUIRE(sizes[b] >= 0 && sizes[b] <= cap && heads[b] >= 0 && heads[b] < cap,
               "index_search: row %lld ring state (size %lld, head %lld) outside the capacity %lld", (long long)b,
               (long long)sizes[b], (long long)heads[b], (long long)cap);
    a.size[b] = (int)sizes[b];
    a.head[b] = (int)heads[b];
  }
  int max_size = 0;
  for (int64_t b = 0; b < B; ++b) max_size = max(max_size, a.size[b]);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (hits_host) {
    // the kernel writes the host copy itself through the pinned buffer's
    // device mapping: no copy to issue, and the hits are on the host when the
    // kernel is done
    void* mapped = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&mapped, hits_host, 0);
    if (e != hipSuccess || mapped == nullptr) {
      (void)hipGetLastError();
      return set_error(HC_ERR_INVALID, "index_search: hits_host is not pinned host memory");
    }
    a.hits_mapped = reinterpret_cast<int64_t*>(mapped);
  }
  if (wait_event) {
    const hipError_t e = hipStreamWaitEvent(st, reinterpret_cast<hipEvent_t>(wait_event), 0);
    if (e != hipSuccess) return set_error(HC_ERR_HIP, "index_search: hipStreamWaitEvent: %s", hipGetErrorString(e));
  }
  if (max_size > 0)
    hipLaunchKernelGGL(index_score_kernel, dim3((unsigned)cdiv(max_size, kScoreSlots), (unsigned)VH, (unsigned)B),
                       dim3(kScoreThreads), 0, st, a);
  hipLaunchKernelGGL(index_select_kernel, dim3((unsigned)VH, (unsigned)B), dim3(kIdxThreads), 0, st, a);
  const int rc = check_launch("index_search");
  if (rc != HC_OK) return rc;
  if (done_event) {
    const hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(done_event), st);
    if (e != hipSuccess) return set_error(HC_ERR_HIP, "index_search: hipEventRecord: %s", hipGetErrorString(e));
  }
  return HC_OK;
}
