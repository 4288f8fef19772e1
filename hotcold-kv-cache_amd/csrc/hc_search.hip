// Device search index of the cold store: the search vectors of every
// (batch row, vector head) kept in HBM, scanned and ranked on the GPU.
//
// The reference searches its CPU faiss.IndexFlatIP per (layer, batch row)
// (controller.py:223-232, 274-293).  The host store (hc_cold.cpp) reproduces
// that search exactly, but a scan of every stored vector per search is bound
// by host memory: at 16 batch rows of 30 720 evicted tokens and 8 KV heads a
// layer's search reads 2 GB, which host threads cannot finish within a
// retrieval window of a fast decode loop.  Here the same vectors live in HBM
// in tiles of 64 slots, [B][VH][capT/64][VD/4][64][4] fp32: a wave scores one
// tile, each lane reading 4 dimensions of its slot per 16-byte load, and a
// tile is one contiguous run.  The same arithmetic as the host runs on the GPU:
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
//
// With unit vectors, a copy rounded to fp16 halves the scan: its fp32 scores
// are within a proven bound delta of the exact ones, so only the slots whose
// fp16-pass score is within 2*delta of the R-th best can be in the exact top
// R; those are scored exactly and ranked as above (index_score16_kernel,
// index_select16_kernel).  The hits are the same.
#include <cmath>

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
  float* vec;              // [B][VH][capT/64][VD/4][64][4]
  half_t* vec16;           // [B][VH][capT/64][VD/8][64][8]: the same rounded to fp16 (or null)
  int64_t capT;
  int B, H, D, VH, VD, te, normalize;
};

// Offset of slot s, dimension d in a (row, head) plane [capT/64][VD/4][64][4]
// (VD a multiple of 4).
__device__ __forceinline__ int64_t vec_at(int64_t s, int d, int VD) {
  return ((s >> 6) * (int64_t)(VD / 4) + (d >> 2)) * 256 + (s & 63) * 4 + (d & 3);
}

// Offset of slot s, dims 8g..8g+7 in a (row, head) plane of vec16,
// [capT/64][VD/8][64][8]: a lane's 16-byte load covers 8 dimensions of its slot.
__device__ __forceinline__ int64_t vec16_at(int64_t s, int g, int VD) {
  return ((s >> 6) * (int64_t)(VD / 8) + g) * 512 + (s & 63) * 8;
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
  half_t* o16 = a.vec16 ? a.vec16 + (int64_t)(b * a.VH + vh) * a.VD * a.capT : nullptr;
  for (int c = 0; c < nchunks; ++c) {
    if (c > 0 || (a.normalize && nchunks > 1)) {
      __syncthreads();
      fill(c * kAddChunk);
    }
    __syncthreads();
    const int w = min(kAddChunk, a.VD - c * kAddChunk);
    for (int i = tid; i < kAddTok * w; i += kAddThreads) {
      const int dd = i / kAddTok, tl = i % kAddTok, slot = slot_s[tl];
      if (slot >= 0) {
        const int d = c * kAddChunk + dd;
        const float x = (float)(xs[tl][dd] / den_s[tl]);
        o[vec_at(slot, d, a.VD)] = x;
        if (o16) o16[vec16_at(slot, d >> 3, a.VD) + (d & 7)] = (half_t)x;
      }
    }
  }
}

struct IndexSearchArgs {
  const float* q;  // query of (row b, head vh) at q + b*q_sb + vh*q_sh, q_dim floats
  int64_t q_sb, q_sh;
  const float* vec;         // [B][VH][capT/64][VD/4][64][4] fp32
  const half_t* vec16;      // [B][VH][capT/64][VD/8][64][8]: the same vectors rounded to fp16 (or null)
  int64_t capT;
  uint64_t* keys;           // scratch [B][VH][capT]: exact order keys
  uint32_t* keys32;         // scratch [B][VH][capT]: fp16-pass order keys (with vec16)
  int64_t* hits;            // [B][VH][R]: logical indices in rank order, -1 past the hits
  int64_t* hits_mapped;     // the same, into pinned host memory through its device mapping (or null)
  double delta;             // bound on |exact score - fp16-pass score| (with vec16)
  int B, VH, VD, R, cap, q_dim, normalize_q;
  int size[kIdxMaxB], head[kIdxMaxB];  // ring state of each row's store
};

// A double's bits as an unsigned key that orders like the value (-0 as +0).
__device__ __forceinline__ uint64_t ordered_key(double x) {
  if (x == 0.0) x = 0.0;
  const uint64_t u = __double_as_longlong(x);
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}
// The fp16 pass's key: its score s (within about 1 of 0 for unit vectors)
// as fixed point, floor((s + 2) * 2^29), clamped; non-decreasing in s, and
// the leading digits spread the scores evenly, so the radix select's first
// digit already separates the top of the ranking.  Key k holds the scores in
// [k, k + 1) / 2^29 - 2.
constexpr double kFixScale = 536870912.0;  // 2^29
__device__ __forceinline__ uint32_t fixed_key32(float s) {
  const double x = ((double)s + 2.0) * kFixScale;
  return x <= 0.0 ? 0u : (x >= 4294967295.0 ? 0xffffffffu : (uint32_t)x);
}
__device__ __forceinline__ double fixed_key_low(uint32_t k) { return (double)k / kFixScale - 2.0; }
__device__ __forceinline__ double fixed_key_high(uint32_t k) { return ((double)k + 1.0) / kFixScale - 2.0; }

// The query of (row b, head vh), cropped or zero-padded to VD and (with
// normalize_q) divided by its norm, as the stored vectors are: the raw values
// are staged in LDS by all threads, the norm is one fp64 chain over them in
// dimension order (thread 0), and each dimension is divided by its own thread.
// Ends with a barrier.
__device__ void stage_query(const IndexSearchArgs& a, int b, int vh, int tid, int nthreads, float* qv,
                            double* den_s) {
#pragma clang fp contract(off)
  const float* qs = a.q + b * a.q_sb + vh * a.q_sh;
  for (int d = tid; d < a.VD; d += nthreads) qv[d] = d < a.q_dim ? qs[d] : 0.0f;
  __syncthreads();
  if (tid == 0) {
    double den = 1.0;
    if (a.normalize_q) {
      double ss = 0.0;
      for (int d = 0; d < a.VD; ++d) {
        const double x = (double)qv[d];
        ss += x * x;
      }
      den = fmax(sqrt(ss), 1e-12);
    }
    *den_s = den;
  }
  __syncthreads();
  if (a.normalize_q)
    for (int d = tid; d < a.VD; d += nthreads) qv[d] = (float)((double)qv[d] / *den_s);
  __syncthreads();
}

// The exact score of slot p: fp64 inner product in dimension order.  The
// slot's 4-dimension groups lie 1 KB apart; 8 of them (32 dimensions) are
// loaded, unconditionally (groups past VD/4 clamped), before any is used.
__device__ __forceinline__ double exact_score(const float* vb, const float* qv, int p, int VD) {
#pragma clang fp contract(off)
  const float* t = vb + vec_at(p, 0, VD);
  const int G = VD / 4;
  double acc = 0.0;
  for (int g0 = 0; g0 < G; g0 += 8) {
    floatx4 x[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = *reinterpret_cast<const floatx4*>(t + min(g0 + k, G - 1) * 256);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (g0 + k < G) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc += (double)qv[(g0 + k) * 4 + e] * (double)x[k][e];
      }
  }
  return acc;
}

// Scoring: grid (cdiv(max size, kScoreSlots), VH, B), block kScoreThreads.
// Each thread scores kScorePer slots of one (row, head), one per 64-slot tile
// of its wave: the fp64 inner product in dimension order, stored as an order
// key.  A lane reads 4 dimensions of its slot per 16-byte load (a wave 1 KB
// of its tile), so the grid streams the vectors at full width whatever B and
// VH are.
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
  stage_query(a, b, vh, tid, kScoreThreads, qv, &den_s);
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
  const int G = a.VD / 4;
#pragma unroll 4
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int j = 0; j < kScorePer; ++j) {
      const floatx4 x = *reinterpret_cast<const floatx4*>(tile[j] + g * 256);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[j] += (double)qv[g * 4 + e] * (double)x[e];
    }
  }
#pragma unroll
  for (int j = 0; j < kScorePer; ++j) {
    const int p = p0 + j * kScoreThreads;
    if (p < size) kb[p] = ordered_key(acc[j]);
  }
}

// The fp16 pass: the same grid, fp32 FMA scores of the fp16 vectors (one
// 16-byte load per lane covers 8 dimensions of its slot), as fixed-point
// keys.  |exact - this| <= delta (hc_index_search derives the bound), so the
// exact top R lies among the slots within 2*delta of this pass's R-th score.
__global__ __launch_bounds__(kScoreThreads) void index_score16_kernel(IndexSearchArgs a) {
  __shared__ float qv[kIdxMaxVD];
  __shared__ double den_s;
  const int vh = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int size = a.size[b];
  const int p0 = blockIdx.x * kScoreSlots + tid;
  if (blockIdx.x * kScoreSlots >= size) return;  // uniform per workgroup
  stage_query(a, b, vh, tid, kScoreThreads, qv, &den_s);
  const half_t* vb = a.vec16 + (int64_t)(b * a.VH + vh) * a.VD * a.capT;
  uint32_t* kb = a.keys32 + (int64_t)(b * a.VH + vh) * a.capT;
  float acc[kScorePer];
  const half_t* tile[kScorePer];
#pragma unroll
  for (int j = 0; j < kScorePer; ++j) {
    acc[j] = 0.0f;
    tile[j] = vb + vec16_at(min(p0 + j * kScoreThreads, (int)a.capT - 1), 0, a.VD);
  }
  const int G = a.VD / 8;
#pragma unroll 4
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int j = 0; j < kScorePer; ++j) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(tile[j] + g * 512);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint16_t h = (uint16_t)((k & 1) ? (w[k >> 1] >> 16) : (w[k >> 1] & 0xffffu));
        acc[j] = fmaf(qv[g * 8 + k], (float)__builtin_bit_cast(half_t, h), acc[j]);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kScorePer; ++j) {
    const int p = p0 + j * kScoreThreads;
    if (p < size) kb[p] = fixed_key32(acc[j]);
  }
}

// Selection: grid (VH, B), block kIdxThreads, one (row, head) per workgroup.
constexpr int kCand = 4096;    // keys sharing a radix prefix kept in LDS
constexpr int kEqCap = 1024;   // ties at the R-th key ranked in LDS
constexpr int kCandX = 2048;   // fp16-pass candidates re-scored exactly
constexpr int kKeyBatch = 8;   // keys loaded per thread before any is used

// f(p, key) for every p < size, thread tid taking p = tid (mod kIdxThreads),
// its loads issued kKeyBatch at a time.  The loads are unconditional (indices
// past the end are clamped to the last key): a conditional load makes the
// compiler wait for each one before the next.
template <typename K, typename F>
__device__ __forceinline__ void for_keys(const K* kb, int size, int tid, F&& f) {
  for (int base = 0; base < size; base += kIdxThreads * kKeyBatch) {
    K k[kKeyBatch];
#pragma unroll
    for (int j = 0; j < kKeyBatch; ++j) k[j] = kb[min(base + j * kIdxThreads + tid, size - 1)];
#pragma unroll
    for (int j = 0; j < kKeyBatch; ++j) {
      const int p = base + j * kIdxThreads + tid;
      if (p < size) f(p, k[j]);
    }
  }
}

struct RadixShared {
  uint32_t hist[256];
  int sel_digit, sel_above, sel_count, n_cand;
  int wave_tot[4];
};

// The m-th largest of the keys kb[0..size) by radix select over 8-bit digits,
// most significant first; `remaining` of the keys equal to it are within the
// top m.  Once the keys sharing the selected prefix fit kcap, they are copied
// to ck (LDS) and the remaining digits are selected there, so the keys are
// read from memory only a few times.  The digit holding the remaining-th key
// comes from wave scans of the histogram in descending digit order.
template <typename K>
__device__ K radix_select(const K* kb, int size, int m, int tid, K* ck, int kcap, RadixShared& rs, int& remaining) {
  constexpr int kBits = (int)sizeof(K) * 8;
  K prefix = 0;
  remaining = m;
  bool in_lds = false;
  int nc = 0;
  for (int shift = kBits - 8; shift >= 0; shift -= 8) {
    if (tid < 256) rs.hist[tid] = 0;
    __syncthreads();
    const K high = shift == kBits - 8 ? (K)0 : (K)~(((K)1 << (shift + 8)) - 1);
    if (in_lds) {
      for (int i = tid; i < nc; i += kIdxThreads) {
        const K k = ck[i];
        hist_add(rs.hist, (uint32_t)(k >> shift) & 255u, (k & high) == prefix);
      }
    } else {
      for_keys(kb, size, tid, [&](int, K k) {
        hist_add(rs.hist, (uint32_t)(k >> shift) & 255u, (k & high) == prefix);
      });
    }
    __syncthreads();
    int v = 0, incl = 0;
    if (tid < 256) {
      const int lane = tid & 63;
      v = (int)rs.hist[255 - tid];
      incl = v;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int u = __shfl_up(incl, off, 64);
        if (lane >= off) incl += u;
      }
      if (lane == 63) rs.wave_tot[tid >> 6] = incl;
    }
    __syncthreads();
    if (tid < 256) {
      for (int i = 0; i < (tid >> 6); ++i) incl += rs.wave_tot[i];
      const int excl = incl - v;
      if (excl < remaining && incl >= remaining) {
        rs.sel_digit = 255 - tid;
        rs.sel_above = excl;
        rs.sel_count = v;
      }
    }
    __syncthreads();
    prefix |= (K)rs.sel_digit << shift;
    remaining -= rs.sel_above;
    if (!in_lds && shift > 0 && rs.sel_count <= kcap) {
      const K hi_new = (K)~(((K)1 << shift) - 1);
      if (tid == 0) rs.n_cand = 0;
      __syncthreads();
      for_keys(kb, size, tid, [&](int, K k) {
        const int i = append_slot(&rs.n_cand, (k & hi_new) == prefix);
        if (i >= 0) ck[i] = k;
      });
      __syncthreads();
      nc = rs.n_cand;
      in_lds = true;
    }
    __syncthreads();
  }
  return prefix;
}

// Bitonic sort of wk/wl[0..P) (P a power of two <= 2 * kIdxThreads) into
// rank order: key descending, logical index ascending.
template <int kMax>
__device__ void sort_ranked(uint64_t* wk, int32_t* wl, int P, int tid) {
  for (int k = 2; k <= P; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < P && i < kMax; i += kIdxThreads) {
        const int o = i ^ j;
        if (o > i) {
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
      }
      __syncthreads();
    }
}

__device__ __forceinline__ void write_hits(const IndexSearchArgs& a, int b, int vh, int m, const int32_t* wl, int tid) {
  int64_t* out = a.hits + (int64_t)(b * a.VH + vh) * a.R;
  for (int j = tid; j < a.R; j += kIdxThreads) {
    const int64_t h = j < m ? (int64_t)wl[j] : -1;
    out[j] = h;
    if (a.hits_mapped) a.hits_mapped[(int64_t)(b * a.VH + vh) * a.R + j] = h;
  }
}

// LDS of the exact selection and of the fp16 pass's selection (one workgroup
// uses one or, when it falls back, the other).
struct ExactSmem {
  RadixShared rs;
  uint64_t ck[kCand];
  uint64_t wk[kIdxMaxR];
  int32_t wl[kIdxMaxR];
  int32_t eql[kEqCap];
  int32_t scan[kIdxThreads];
  int n_above, n_eq;
};
struct Pass16Smem {
  RadixShared rs;
  uint32_t ck[kCand];
  int32_t cp[kCandX];
  uint64_t ckey[kCandX];
  int32_t cl[kCandX];
  int n_c;
};
union SelectSmem {
  ExactSmem x;
  Pass16Smem y;
};

// The exact selection over the exact keys kb[0..size): the m-th largest key
// T (radix_select), then one pass collects the keys above T and the logical
// indices of the keys equal to T, of which the `remaining` oldest are taken
// (by rank within kEqCap, else by an ordered prefix scan); a bitonic sort puts
// the m hits in rank order.
__device__ void select_exact(const IndexSearchArgs& a, int b, int vh, const uint64_t* kb, int m, int tid,
                             ExactSmem& sm) {
  const int size = a.size[b], head = a.head[b];
  const bool full = size >= a.cap;
  auto logical = [&](int p) { return full ? (p - head + a.cap) % a.cap : p; };
  int remaining;
  const uint64_t T = radix_select<uint64_t>(kb, size, m, tid, sm.ck, kCand, sm.rs, remaining);

  if (tid == 0) {
    sm.n_above = 0;
    sm.n_eq = 0;
  }
  __syncthreads();
  for_keys(kb, size, tid, [&](int p, uint64_t k) {
    const int i = append_slot(&sm.n_above, k > T);
    if (i >= 0) {
      sm.wk[i] = k;
      sm.wl[i] = logical(p);
    }
    const int j = append_slot(&sm.n_eq, k == T);
    if (j >= 0 && j < kEqCap) sm.eql[j] = logical(p);
  });
  __syncthreads();
  const int above = sm.n_above, neq = sm.n_eq;
  if (neq <= kEqCap) {
    // the `remaining` smallest logical indices among the ties (all distinct)
    for (int j = tid; j < neq; j += kIdxThreads) {
      const int l = sm.eql[j];
      int rank = 0;
      if (neq > remaining)
        for (int i = 0; i < neq; ++i) rank += sm.eql[i] < l;
      else
        rank = j;
      if (rank < remaining) {
        sm.wk[above + rank] = T;
        sm.wl[above + rank] = l;
      }
    }
  } else {
    // more ties than the buffer holds: a prefix sum over per-thread runs of
    // logical indices finds the `remaining` oldest
    const int chunk = (size + kIdxThreads - 1) / kIdxThreads;
    const int l0 = min(size, tid * chunk), l1 = min(size, l0 + chunk);
    int cnt = 0;
    for (int l = l0; l < l1; ++l) cnt += kb[full ? (head + l) % a.cap : l] == T;
    sm.scan[tid] = cnt;
    __syncthreads();
    for (int off = 1; off < kIdxThreads; off <<= 1) {  // inclusive scan
      const int v = tid >= off ? sm.scan[tid - off] : 0;
      __syncthreads();
      sm.scan[tid] += v;
      __syncthreads();
    }
    int rank = sm.scan[tid] - cnt;
    for (int l = l0; l < l1 && rank < remaining; ++l)
      if (kb[full ? (head + l) % a.cap : l] == T) {
        sm.wk[above + rank] = T;
        sm.wl[above + rank] = l;
        ++rank;
      }
  }
  __syncthreads();
  int P = 1;
  while (P < m) P <<= 1;
  if (tid < P && tid >= m) {
    sm.wk[tid] = 0;
    sm.wl[tid] = 0x7fffffff;
  }
  __syncthreads();
  sort_ranked<kIdxMaxR>(sm.wk, sm.wl, P, tid);
  write_hits(a, b, vh, m, sm.wl, tid);
}

__global__ __launch_bounds__(kIdxThreads) void index_select_kernel(IndexSearchArgs a) {
  __shared__ SelectSmem sm;
  const int vh = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int m = min(a.R, a.size[b]);
  if (m == 0) {  // uniform per workgroup
    write_hits(a, b, vh, 0, nullptr, tid);
    return;
  }
  const uint64_t* kb = a.keys + (int64_t)(b * a.VH + vh) * a.capT;
  select_exact(a, b, vh, kb, m, tid, sm.x);
}

// Selection after the fp16 pass: T' = the key of the m-th largest fp16-pass
// score (radix select on the fixed-point keys); the candidates are the slots
// whose fp16-pass score can be at least the low end of T' minus 2*delta, a
// superset of the exact top m with every tie at the m-th exact score.  Their exact fp64 scores, sorted by (score
// descending, logical index ascending), give the exact hits.  More than
// kCandX candidates (many near-ties): the workgroup scores every slot exactly
// and runs the exact selection instead.
__global__ __launch_bounds__(kIdxThreads) void index_select16_kernel(IndexSearchArgs a) {
  __shared__ SelectSmem sm;
  __shared__ float qv[kIdxMaxVD];
  __shared__ double den_s;
  const int vh = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int size = a.size[b], head = a.head[b];
  const bool full = size >= a.cap;
  const int m = min(a.R, size);
  if (m == 0) {  // uniform per workgroup
    write_hits(a, b, vh, 0, nullptr, tid);
    return;
  }
  auto logical = [&](int p) { return full ? (p - head + a.cap) % a.cap : p; };
  const int64_t plane = (int64_t)(b * a.VH + vh) * a.capT;
  const uint32_t* kb32 = a.keys32 + plane;
  const float* vb = a.vec + plane * a.VD;
  Pass16Smem& y = sm.y;
  int remaining;
  const uint32_t T = radix_select<uint32_t>(kb32, size, m, tid, y.ck, kCand, y.rs, remaining);
  // every score with key T is at least fixed_key_low(T); a slot is kept if
  // its score can reach T's lower end minus 2 * delta (less 2^-40 for the
  // rounding of this difference)
  const double thr = fixed_key_low(T) - 2.0 * a.delta - 0x1p-40;
  if (tid == 0) y.n_c = 0;
  __syncthreads();
  for_keys(kb32, size, tid, [&](int p, uint32_t k) {
    const int i = append_slot(&y.n_c, fixed_key_high(k) >= thr);
    if (i >= 0 && i < kCandX) y.cp[i] = p;
  });
  stage_query(a, b, vh, tid, kIdxThreads, qv, &den_s);
  const int nc = y.n_c;
  if (nc > kCandX) {
    uint64_t* kb = a.keys + plane;
    for (int p = tid; p < size; p += kIdxThreads) kb[p] = ordered_key(exact_score(vb, qv, p, a.VD));
    __syncthreads();
    select_exact(a, b, vh, kb, m, tid, sm.x);
    return;
  }
  for (int i = tid; i < nc; i += kIdxThreads) {
    const int p = y.cp[i];
    y.ckey[i] = ordered_key(exact_score(vb, qv, p, a.VD));
    y.cl[i] = logical(p);
  }
  int P = 1;
  while (P < nc) P <<= 1;
  for (int i = nc + tid; i < P; i += kIdxThreads) {
    y.ckey[i] = 0;
    y.cl[i] = 0x7fffffff;
  }
  __syncthreads();
  sort_ranked<kCandX>(y.ckey, y.cl, P, tid);
  write_hits(a, b, vh, m, y.cl, tid);
}

}  // namespace hc

using namespace hc;

extern "C" int hc_index_add(int64_t B, int64_t H, int64_t D, int64_t VH, int64_t VD, int normalize,
                            const float* kpre, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t te,
                            const int32_t* slot_of, float* vec, void* vec16, int64_t capT, void* stream) {
  HC_REQUIRE(B > 0 && H > 0 && D > 0 && VD > 0 && te >= 0 && (VH == 1 || VH == H) && capT > 0 && capT % 64 == 0,
             "index_add: bad shape (B=%lld H=%lld D=%lld VH=%lld VD=%lld te=%lld)", (long long)B, (long long)H,
             (long long)D, (long long)VH, (long long)VD, (long long)te);
  HC_REQUIRE(kpre && slot_of && vec, "index_add: null pointer");
  HC_REQUIRE(B * te * VH < ((int64_t)1 << 40), "index_add: too many tokens");
  if (te == 0) return HC_OK;
  HC_REQUIRE(VD % 4 == 0, "index_add: vector width %lld must be a multiple of 4", (long long)VD);
  HC_REQUIRE(!vec16 || VD % 8 == 0, "index_add: an fp16 copy needs a vector width that is a multiple of 8");
  IndexAddArgs a{kpre, k_sb, k_sh, k_st, slot_of, vec, static_cast<half_t*>(vec16), capT, (int)B, (int)H, (int)D,
                 (int)VH, (int)VD, (int)te, normalize};
  HC_REQUIRE(B <= 65535 && VH <= 65535, "index_add: grid too large");
  hipLaunchKernelGGL(index_add_kernel, dim3((unsigned)cdiv(te, kAddTok), (unsigned)VH, (unsigned)B),
                     dim3(kAddThreads), 0, reinterpret_cast<hipStream_t>(stream), a);
  return check_launch("index_add");
}

extern "C" int hc_index_search(int64_t B, int64_t VH, int64_t VD, int64_t cap, const float* q, int64_t q_sb,
                               int64_t q_sh, int64_t q_dim, int normalize_q, const float* vec, const void* vec16,
                               int vec_normalized, int64_t capT, const int64_t* sizes, const int64_t* heads,
                               int64_t R, uint64_t* keys, uint32_t* keys32, int64_t* hits, int64_t* hits_host,
                               void* wait_event, void* done_event, void* stream) {
  HC_REQUIRE(B > 0 && B <= kIdxMaxB, "index_search: batch rows %lld outside 1..%d", (long long)B, kIdxMaxB);
  HC_REQUIRE(VH > 0 && VD > 0 && VD <= kIdxMaxVD && VD % 4 == 0 && q_dim > 0,
             "index_search: vector width %lld must be a multiple of 4 in 4..%d", (long long)VD, kIdxMaxVD);
  HC_REQUIRE(R > 0 && R <= kIdxMaxR, "index_search: R=%lld outside 1..%d", (long long)R, kIdxMaxR);
  HC_REQUIRE(cap > 0 && capT >= cap && capT % 64 == 0 && capT < (1ll << 31), "index_search: bad capacity");
  HC_REQUIRE(q && vec && sizes && heads && keys && hits, "index_search: null pointer");
  IndexSearchArgs a{};
  a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.vec = vec; a.capT = capT; a.keys = keys; a.hits = hits;
  a.B = (int)B; a.VH = (int)VH; a.VD = (int)VD; a.R = (int)R; a.cap = (int)cap; a.q_dim = (int)q_dim;
  a.normalize_q = normalize_q;
  // The fp16 pass needs unit vectors on both sides (its error bound is relative
  // to the norms) and whole 8-dimension groups.  Bound on |exact - fp16 pass|
  // for unit q and v (norms <= 1 + 2^-23 after rounding to fp32):
  //   fp16 rounding of v: |v - v'| <= 2^-11 |v| + 2^-25 per element, so
  //     sum |q||v - v'| <= 2^-11 |q||v| + 2^-25 sqrt(VD) |q|;
  //   the fp32 FMA chain: <= gamma_VD * sum |q v'| with gamma_n = n u/(1 - n u),
  //     u = 2^-24, sum |q v'| <= 1.01;
  //   the fp64 exact sum: < 2^-40.
  const bool pass16 = vec16 && keys32 && normalize_q && vec_normalized && VD % 8 == 0;
  if (pass16) {
    const double u = std::ldexp(1.0, -24), n = (double)VD;
    a.vec16 = static_cast<const half_t*>(vec16);
    a.keys32 = keys32;
    a.delta = std::ldexp(1.0, -11) * (1.0 + std::ldexp(1.0, -20)) +
              std::ldexp(1.0, -25) * std::sqrt(n) * (1.0 + std::ldexp(1.0, -20)) + 1.01 * n * u / (1.0 - n * u) +
              std::ldexp(1.0, -40);
  }
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
  const dim3 sgrid((unsigned)cdiv(max_size, kScoreSlots), (unsigned)VH, (unsigned)B);
  if (pass16) {
    if (max_size > 0) hipLaunchKernelGGL(index_score16_kernel, sgrid, dim3(kScoreThreads), 0, st, a);
    hipLaunchKernelGGL(index_select16_kernel, dim3((unsigned)VH, (unsigned)B), dim3(kIdxThreads), 0, st, a);
  } else {
    if (max_size > 0) hipLaunchKernelGGL(index_score_kernel, sgrid, dim3(kScoreThreads), 0, st, a);
    hipLaunchKernelGGL(index_select_kernel, dim3((unsigned)VH, (unsigned)B), dim3(kIdxThreads), 0, st, a);
  }
  const int rc = check_launch("index_search");
  if (rc != HC_OK) return rc;
  if (done_event) {
    const hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(done_event), st);
    if (e != hipSuccess) return set_error(HC_ERR_HIP, "index_search: hipEventRecord: %s", hipGetErrorString(e));
  }
  return HC_OK;
}
