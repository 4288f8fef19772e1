// Device search index of the cold store: the search vectors of every
// (batch row, vector head) kept in HBM, scanned and ranked on the GPU.
//
// The reference searches its CPU faiss.IndexFlatIP per (layer, batch row)
// (controller.py:223-232, 274-293).  The host store (hc_cold.cpp) reproduces
// that search exactly, but a scan of every stored vector per search is bound
// by host memory: at 16 batch rows of 30 720 evicted tokens and 8 KV heads a
// layer's search reads 2 GB, which host threads cannot finish within a
// retrieval window of a fast decode loop.  Here the same vectors live in HBM,
// [B][VH][VD][capT] fp32 (each dimension's slots contiguous, so a wave reads
// one dimension of 64 slots at once), and the same arithmetic runs on the GPU:
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
  float* vec;              // [B][VH][VD][capT]
  int64_t capT;
  int B, H, D, VH, VD, te, normalize;
};

// One thread per (row, token, vector head): the vector's norm is one fp64
// chain over the dimensions in order, then each dimension is recomputed and
// divided (the recomputation repeats the same operations, so it gives the
// same values as keeping them).
__global__ __launch_bounds__(256) void index_add_kernel(IndexAddArgs a) {
#pragma clang fp contract(off)
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int64_t)a.B * a.te * a.VH) return;
  const int vh = (int)(gid % a.VH);
  const int64_t bt = gid / a.VH;
  const int t = (int)(bt % a.te), b = (int)(bt / a.te);
  const int slot = a.slot_of[(int64_t)b * a.te + t];
  if (slot < 0 || slot >= a.capT) return;
  const float* kp = a.kpre + b * a.k_sb + (int64_t)t * a.k_st;
  const int n = min(a.D, a.VD);
  auto xval = [&](int d) -> double {
    if (d >= n) return 0.0;
    if (a.VH == 1) {
      double s = 0.0;
      for (int h = 0; h < a.H; ++h) s += (double)kp[h * a.k_sh + d];
      return s / (double)a.H;
    }
    return (double)kp[vh * a.k_sh + d];
  };
  double den = 1.0;
  if (a.normalize) {
    double ss = 0.0;
    for (int d = 0; d < a.VD; ++d) {
      const double x = xval(d);
      ss += x * x;
    }
    den = fmax(sqrt(ss), 1e-12);
  }
  float* o = a.vec + (int64_t)(b * a.VH + vh) * a.VD * a.capT + slot;
  for (int d = 0; d < a.VD; ++d) o[(int64_t)d * a.capT] = (float)(xval(d) / den);
}

struct IndexSearchArgs {
  const float* q;  // query of (row b, head vh) at q + b*q_sb + vh*q_sh, q_dim floats
  int64_t q_sb, q_sh;
  const float* vec;
  int64_t capT;
  uint64_t* keys;  // scratch [B][VH][capT]
  int64_t* hits;   // [B][VH][R]: logical indices in rank order, -1 past the hits
  int B, VH, VD, R, cap, q_dim, normalize_q;
  int size[kIdxMaxB], head[kIdxMaxB];  // ring state of each row's store
};

// A double's bits as an unsigned key that orders like the value (-0 as +0).
__device__ __forceinline__ uint64_t ordered_key(double x) {
  if (x == 0.0) x = 0.0;
  const uint64_t u = __double_as_longlong(x);
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

// grid (VH, B), block 1024: one (row, head) per workgroup.
__global__ __launch_bounds__(kIdxThreads) void index_search_kernel(IndexSearchArgs a) {
#pragma clang fp contract(off)
  __shared__ float qv[kIdxMaxVD];
  __shared__ uint32_t hist[256];
  __shared__ uint64_t wk[kIdxMaxR];
  __shared__ int32_t wl[kIdxMaxR];
  __shared__ int32_t scan[kIdxThreads];
  __shared__ int sel_digit, sel_above, n_above;
  const int vh = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int size = a.size[b], head = a.head[b];
  const bool full = size >= a.cap;
  int64_t* out = a.hits + (int64_t)(b * a.VH + vh) * a.R;

  // the query: cropped or zero-padded to VD, normalised as the vectors are
  if (tid == 0) {
    const float* qs = a.q + b * a.q_sb + vh * a.q_sh;
    double den = 1.0;
    if (a.normalize_q) {
      double ss = 0.0;
      for (int d = 0; d < a.VD; ++d) {
        const double x = d < a.q_dim ? (double)qs[d] : 0.0;
        ss += x * x;
      }
      den = fmax(sqrt(ss), 1e-12);
    }
    for (int d = 0; d < a.VD; ++d)
      qv[d] = d < a.q_dim ? (a.normalize_q ? (float)((double)qs[d] / den) : qs[d]) : 0.0f;
  }
  __syncthreads();

  // inner products of the stored slots, as order keys
  const float* vb = a.vec + (int64_t)(b * a.VH + vh) * a.VD * a.capT;
  uint64_t* kb = a.keys + (int64_t)(b * a.VH + vh) * a.capT;
  for (int p = tid; p < size; p += kIdxThreads) {
    double acc = 0.0;
    for (int d = 0; d < a.VD; ++d) acc += (double)qv[d] * (double)vb[(int64_t)d * a.capT + p];
    kb[p] = ordered_key(acc);
  }
  __syncthreads();

  const int m = min(a.R, size);
  // the m-th largest key: radix select over 8-bit digits, most significant first
  uint64_t prefix = 0;
  int remaining = m;
  if (m > 0) {
    for (int shift = 56; shift >= 0; shift -= 8) {
      if (tid < 256) hist[tid] = 0;
      __syncthreads();
      const uint64_t high = shift == 56 ? 0ull : ~((1ull << (shift + 8)) - 1);
      for (int p = tid; p < size; p += kIdxThreads) {
        const uint64_t k = kb[p];
        if ((k & high) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        int cum = 0;
        for (int dg = 255; dg >= 0; --dg) {
          if (cum + (int)hist[dg] >= remaining) {
            sel_digit = dg;
            sel_above = cum;
            break;
          }
          cum += (int)hist[dg];
        }
      }
      __syncthreads();
      prefix |= (uint64_t)sel_digit << shift;
      remaining -= sel_above;
      __syncthreads();
    }
  }
  const uint64_t T = prefix;  // the m-th largest key; `remaining` keys equal to it are taken

  // keys above T (any order; sorted below)
  if (tid == 0) n_above = 0;
  __syncthreads();
  if (m > 0)
    for (int p = tid; p < size; p += kIdxThreads) {
      const uint64_t k = kb[p];
      if (k > T) {
        const int i = atomicAdd(&n_above, 1);
        wk[i] = k;
        wl[i] = full ? (p - head + a.cap) % a.cap : p;
      }
    }
  __syncthreads();
  // keys equal to T: the `remaining` oldest (smallest logical index), by a
  // prefix sum over per-thread runs of logical indices
  const int above = n_above;
  const int chunk = (size + kIdxThreads - 1) / kIdxThreads;
  const int l0 = min(size, tid * chunk), l1 = min(size, l0 + chunk);
  int cnt = 0;
  if (m > 0)
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
  if (m > 0)
    for (int l = l0; l < l1 && rank < remaining; ++l)
      if (kb[full ? (head + l) % a.cap : l] == T) {
        wk[above + rank] = T;
        wl[above + rank] = l;
        ++rank;
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
  for (int j = tid; j < a.R; j += kIdxThreads) out[j] = j < m ? (int64_t)wl[j] : -1;
}

}  // namespace hc

using namespace hc;

extern "C" int hc_index_add(int64_t B, int64_t H, int64_t D, int64_t VH, int64_t VD, int normalize,
                            const float* kpre, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t te,
                            const int32_t* slot_of, float* vec, int64_t capT, void* stream) {
  HC_REQUIRE(B > 0 && H > 0 && D > 0 && VD > 0 && te >= 0 && (VH == 1 || VH == H) && capT > 0,
             "index_add: bad shape (B=%lld H=%lld D=%lld VH=%lld VD=%lld te=%lld)", (long long)B, (long long)H,
             (long long)D, (long long)VH, (long long)VD, (long long)te);
  HC_REQUIRE(kpre && slot_of && vec, "index_add: null pointer");
  HC_REQUIRE(B * te * VH < ((int64_t)1 << 40), "index_add: too many tokens");
  if (te == 0) return HC_OK;
  IndexAddArgs a{kpre, k_sb, k_sh, k_st, slot_of, vec, capT, (int)B, (int)H, (int)D, (int)VH, (int)VD, (int)te,
                 normalize};
  const int64_t total = B * te * VH;
  hipLaunchKernelGGL(index_add_kernel, dim3((unsigned)cdiv(total, 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return check_launch("index_add");
}

extern "C" int hc_index_search(int64_t B, int64_t VH, int64_t VD, int64_t cap, const float* q, int64_t q_sb,
                               int64_t q_sh, int64_t q_dim, int normalize_q, const float* vec, int64_t capT,
                               const int64_t* sizes, const int64_t* heads, int64_t R, uint64_t* keys, int64_t* hits,
                               void* stream) {
  HC_REQUIRE(B > 0 && B <= kIdxMaxB, "index_search: batch rows %lld outside 1..%d", (long long)B, kIdxMaxB);
  HC_REQUIRE(VH > 0 && VD > 0 && VD <= kIdxMaxVD && q_dim > 0, "index_search: vector width %lld outside 1..%d",
             (long long)VD, kIdxMaxVD);
  HC_REQUIRE(R > 0 && R <= kIdxMaxR, "index_search: R=%lld outside 1..%d", (long long)R, kIdxMaxR);
  HC_REQUIRE(cap > 0 && capT >= cap && cap < (1ll << 31), "index_search: bad capacity");
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
  hipLaunchKernelGGL(index_search_kernel, dim3((unsigned)VH, (unsigned)B), dim3(kIdxThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return check_launch("index_search");
}
