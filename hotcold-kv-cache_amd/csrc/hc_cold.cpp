// Host cold store: one ring of evicted tokens per (layer, batch row) with an
// exact inner-product search (src/hotcold_kv/controller.py:166-293, which
// keeps Python deques of tensors and a faiss.IndexFlatIP per ring).
//
// Contract (the oracle in oracle/reference.py restates it):
//   * A token carries its pre-RoPE key and value ([heads][head_dim] fp32),
//     its absolute position, and vec_heads search vectors of vec_dim fp32:
//     the mean over the heads of the pre-RoPE key (vec_heads == 1,
//     controller.py:190-194) or each head's key (vec_heads == heads), padded
//     with zeros or cropped to vec_dim, then divided by max(||x||, 1e-12).
//     The mean and the norm accumulate in fp64 in index order; the quotient
//     is rounded to fp32.
//   * Inner products accumulate in fp64 in dimension order.  fp32 x fp32
//     products are exact in fp64, so every implementation that adds them in
//     that order gets the same bits.
//   * Ranking: larger inner product first, ties to the older token (lower
//     logical index; logical index 0 is the oldest live token).
//   * A full ring overwrites its oldest token; a batch larger than the ring
//     keeps its last `capacity` tokens (controller.py:219-232).
//
// Storage is one uninitialised allocation per array at full capacity, so host
// pages are touched only as tokens arrive and never copied on growth.  Search
// vectors are kept in 16-slot tiles ([vec_head][slot/16][dim][16]), so a
// tile's sums stay in registers while its dimensions stream past
// contiguously.  Large adds fill
// their (distinct) slots on host threads.  Each store has a reader/writer
// lock: adds exclude searches, searches run concurrently.

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <shared_mutex>
#include <thread>
#include <vector>

#include "hotcold_hip.h"

namespace hc {
int set_error(int code, const char* fmt, ...);
}

namespace {

// Uninitialised host array: pages are touched only when tokens land in them.
template <typename T>
struct RawArray {
  T* p = nullptr;
  void reset(size_t n) {
    free(p);
    p = static_cast<T*>(malloc(n * sizeof(T)));
  }
  ~RawArray() { free(p); }
  T& operator[](size_t i) { return p[i]; }
  const T& operator[](size_t i) const { return p[i]; }
};

struct ColdStore {
  int64_t cap, H, D, VD, VH;
  bool normalize;
  int64_t size = 0;  // live tokens
  int64_t head = 0;  // physical slot of the next write once full
  RawArray<float> kpre, v;  // [slot][H][D]
  RawArray<int64_t> pos;    // [slot]
  RawArray<float> vec;      // [VH][cap/16][VD][16]: 16-slot tiles, each dimension's 16 values together
  int64_t capT = 0;         // cap rounded up to a whole tile
  // Deferred search vectors: while defer_vecs, adds store keys, values and
  // positions only (the caller searches elsewhere, e.g. a device index);
  // the first host search computes every live token's vectors
  // (materialize_vecs) and ends the deferral.
  bool defer_vecs = false;
  bool vecs_missing = false;

  size_t vidx(int64_t vh, int64_t d, int64_t slot) const {
    return (size_t)vh * VD * capT + (size_t)(slot >> 4) * VD * 16 + (size_t)d * 16 + (slot & 15);
  }
  mutable std::shared_mutex mu;
  // Search jobs submitted but not finished that read this store; destroying
  // the store waits for them.
  mutable std::mutex jobs_mu;
  mutable std::condition_variable jobs_cv;
  mutable int64_t jobs_in_flight = 0;

  void pin() const {
    std::lock_guard<std::mutex> lk(jobs_mu);
    ++jobs_in_flight;
  }
  void unpin() const {
    std::lock_guard<std::mutex> lk(jobs_mu);
    if (--jobs_in_flight == 0) jobs_cv.notify_all();
  }
  void wait_unpinned() const {
    std::unique_lock<std::mutex> lk(jobs_mu);
    jobs_cv.wait(lk, [&] { return jobs_in_flight == 0; });
  }
  // Asynchronous adds take a ticket when submitted and are applied in ticket
  // order.  add_served counts the applied ones.  A reader waits for the adds
  // submitted before it: wait_adds(ticket) returns once every add with a
  // smaller ticket has been applied.
  mutable int64_t add_next = 0, add_served = 0;
  int64_t take_ticket() const {
    std::lock_guard<std::mutex> lk(jobs_mu);
    return add_next++;
  }
  int64_t tickets() const {
    std::lock_guard<std::mutex> lk(jobs_mu);
    return add_next;
  }
  void wait_adds(int64_t ticket) const {
    std::unique_lock<std::mutex> lk(jobs_mu);
    jobs_cv.wait(lk, [&] { return add_served >= ticket; });
  }
  void serve_ticket() const {
    std::lock_guard<std::mutex> lk(jobs_mu);
    ++add_served;
    jobs_cv.notify_all();
  }
  // every add submitted so far has been applied
  void wait_all_adds() const { wait_adds(tickets()); }

  bool allocate() {
    kpre.reset((size_t)cap * H * D);
    v.reset((size_t)cap * H * D);
    pos.reset((size_t)cap);
    capT = (cap + 15) / 16 * 16;
    vec.reset((size_t)VH * VD * capT);
    return kpre.p && v.p && pos.p && vec.p;
  }

  int64_t physical(int64_t logical) const {
    return size < cap ? logical : (head + logical) % cap;
  }

  // Search vector(s) of the token in `slot` (its key already stored).
  void set_vec(int64_t slot) {
    const float* kp = &kpre[(size_t)slot * H * D];
    const int64_t n = std::min(D, VD);
    double x[4096];
    for (int64_t vh = 0; vh < VH; ++vh) {
      if (VH == 1) {
        // head mean: fp64, heads added in order (vectorised across dims)
        for (int64_t d = 0; d < n; ++d) x[d] = 0.0;
        for (int64_t h = 0; h < H; ++h)
          for (int64_t d = 0; d < n; ++d) x[d] += (double)kp[h * D + d];
        for (int64_t d = 0; d < n; ++d) x[d] = x[d] / (double)H;
      } else {
        for (int64_t d = 0; d < n; ++d) x[d] = (double)kp[vh * D + d];
      }
      for (int64_t d = n; d < VD; ++d) x[d] = 0.0;
      double den = 1.0;
      if (normalize) {
        double ss = 0.0;
        for (int64_t d = 0; d < VD; ++d) ss += x[d] * x[d];
        den = std::max(std::sqrt(ss), 1e-12);
      }
      for (int64_t d = 0; d < VD; ++d) vec[vidx(vh, d, slot)] = (float)(x[d] / den);
    }
  }

  void copy_in(int64_t slot, const float* kp, int64_t k_sh, const float* vv, int64_t v_sh, int64_t p) {
    float* kd = &kpre[(size_t)slot * H * D];
    float* vd = &v[(size_t)slot * H * D];
    for (int64_t h = 0; h < H; ++h) {
      memcpy(kd + h * D, kp + h * k_sh, sizeof(float) * D);
      memcpy(vd + h * D, vv + h * v_sh, sizeof(float) * D);
    }
    pos[slot] = p;
    if (defer_vecs) vecs_missing = true;
    else set_vec(slot);
  }

  // The vectors of every live token, if adds deferred them; later adds
  // compute theirs again.  Takes the write lock: call without holding it.
  void materialize_vecs(int64_t nthreads);

  // Slot for the next token (advances the ring).
  int64_t next_slot() {
    if (size < cap) return size++;
    const int64_t s = head;
    head = (head + 1) % cap;
    return s;
  }

  // Inner products of query q with the vectors of head vh over physical
  // slots [s0, s1): fp64, dimensions in order.  A whole 16-slot tile (its
  // 16 x VD floats contiguous) keeps its sums in four AVX2 registers across
  // all dimensions; every sum still adds its exact fp32 x fp32 products in
  // dimension order, so the bits are those of a scalar loop.
  void scan(const float* q, int64_t vh, int64_t s0, int64_t s1, double* ip) const {
    double qd[4096];
    for (int64_t d = 0; d < VD; ++d) qd[d] = (double)q[d];
    int64_t s = s0;
    for (; s < s1 && (s & 15); ++s) ip[s] = scan_one(qd, vh, s);
    for (; s + 16 <= s1; s += 16) {
      __m256d a0 = _mm256_setzero_pd(), a1 = _mm256_setzero_pd(), a2 = _mm256_setzero_pd(),
              a3 = _mm256_setzero_pd();
      const float* col = &vec[vidx(vh, 0, s)];
      for (int64_t d = 0; d < VD; ++d, col += 16) {
        const __m256d x = _mm256_set1_pd(qd[d]);
        a0 = _mm256_add_pd(a0, _mm256_mul_pd(_mm256_cvtps_pd(_mm_loadu_ps(col)), x));
        a1 = _mm256_add_pd(a1, _mm256_mul_pd(_mm256_cvtps_pd(_mm_loadu_ps(col + 4)), x));
        a2 = _mm256_add_pd(a2, _mm256_mul_pd(_mm256_cvtps_pd(_mm_loadu_ps(col + 8)), x));
        a3 = _mm256_add_pd(a3, _mm256_mul_pd(_mm256_cvtps_pd(_mm_loadu_ps(col + 12)), x));
      }
      _mm256_storeu_pd(ip + s, a0);
      _mm256_storeu_pd(ip + s + 4, a1);
      _mm256_storeu_pd(ip + s + 8, a2);
      _mm256_storeu_pd(ip + s + 12, a3);
    }
    for (; s < s1; ++s) ip[s] = scan_one(qd, vh, s);
  }

  double scan_one(const double* qd, int64_t vh, int64_t slot) const {
    double acc = 0.0;
    for (int64_t d = 0; d < VD; ++d) acc += (double)vec[vidx(vh, d, slot)] * qd[d];
    return acc;
  }

  // Top-r logical indices by (ip desc, logical asc).  One pass in logical
  // order keeps the r best in a heap whose top is the worst kept; a token
  // replaces it only if strictly better, so among equal inner products the
  // older token stays.  The kept tokens are then sorted best first.
  int64_t select(const double* ip, int64_t r, int64_t* out) const {
    const int64_t n = size;
    r = std::min(r, n);
    if (r <= 0) return 0;
    struct Cand {
      double v;
      int64_t i;
    };
    // a before b: a is better (larger value, then older)
    const auto better = [](const Cand& a, const Cand& b) { return a.v > b.v || (a.v == b.v && a.i < b.i); };
    std::vector<Cand> heap;
    heap.reserve((size_t)r);
    const int64_t start = size < cap ? 0 : head;  // physical slot of logical 0
    int64_t logical = 0;
    const auto visit = [&](int64_t p0, int64_t p1) {
      for (int64_t p = p0; p < p1; ++p, ++logical) {
        const Cand c{ip[p], logical};
        if ((int64_t)heap.size() < r) {
          heap.push_back(c);
          std::push_heap(heap.begin(), heap.end(), better);  // top: the worst kept
        } else if (better(c, heap.front())) {
          std::pop_heap(heap.begin(), heap.end(), better);
          heap.back() = c;
          std::push_heap(heap.begin(), heap.end(), better);
        }
      }
    };
    visit(start, std::min(start + n, cap));
    if (start + n > cap) visit(0, start + n - cap);
    std::sort(heap.begin(), heap.end(), better);
    for (int64_t j = 0; j < r; ++j) out[j] = heap[(size_t)j].i;
    return r;
  }
};

ColdStore* as_store(void* p) { return reinterpret_cast<ColdStore*>(p); }

int threads_for(int64_t requested, int64_t tasks) {
  int64_t hw = (int64_t)std::thread::hardware_concurrency();
  if (hw <= 0) hw = 1;
  int64_t n = requested > 0 ? requested : std::min<int64_t>(hw, 16);
  return (int)std::max<int64_t>(1, std::min(n, tasks));
}

// Run f(i) for i in [0, n) on up to `nthreads` threads.
template <typename F>
void parallel_for(int64_t n, int nthreads, F f) {
  if (nthreads <= 1 || n <= 1) {
    for (int64_t i = 0; i < n; ++i) f(i);
    return;
  }
  std::atomic<int64_t> next{0};
  std::vector<std::thread> pool;
  pool.reserve(nthreads - 1);
  const auto work = [&]() {
    for (int64_t i = next.fetch_add(1); i < n; i = next.fetch_add(1)) f(i);
  };
  for (int t = 1; t < nthreads; ++t) pool.emplace_back(work);
  work();
  for (auto& th : pool) th.join();
}

void ColdStore::materialize_vecs(int64_t nthreads) {
  std::unique_lock<std::shared_mutex> lk(mu);
  defer_vecs = false;
  if (!vecs_missing) return;
  constexpr int64_t kChunk = 256;
  const int64_t nchunks = (size + kChunk - 1) / kChunk;
  parallel_for(nchunks, threads_for(nthreads, nchunks), [&](int64_t c) {
    const int64_t i1 = std::min(size, (c + 1) * kChunk);
    for (int64_t i = c * kChunk; i < i1; ++i) set_vec(i);  // the live slots are 0..size-1
  });
  vecs_missing = false;
}

}  // namespace

using hc::set_error;

extern "C" void* hc_cold_create(int64_t capacity, int64_t heads, int64_t head_dim, int64_t vec_dim,
                                int64_t vec_heads, int normalize) {
  if (capacity <= 0 || heads <= 0 || head_dim <= 0 || vec_dim <= 0 || (vec_heads != 1 && vec_heads != heads)) {
    set_error(HC_ERR_INVALID, "cold_create: bad sizes capacity=%lld heads=%lld head_dim=%lld vec_dim=%lld "
              "vec_heads=%lld", (long long)capacity, (long long)heads, (long long)head_dim, (long long)vec_dim,
              (long long)vec_heads);
    return nullptr;
  }
  if (vec_dim > 4096) {
    set_error(HC_ERR_INVALID, "cold_create: vec_dim %lld above 4096", (long long)vec_dim);
    return nullptr;
  }
  ColdStore* s = new ColdStore();
  s->cap = capacity;
  s->H = heads;
  s->D = head_dim;
  s->VD = vec_dim;
  s->VH = vec_heads;
  s->normalize = normalize != 0;
  if (!s->allocate()) {
    delete s;
    set_error(HC_ERR_INVALID, "cold_create: out of host memory for %lld tokens", (long long)capacity);
    return nullptr;
  }
  return s;
}

extern "C" void hc_cold_destroy(void* store) {
  ColdStore* s = as_store(store);
  if (!s) return;
  s->wait_unpinned();  // a search job still reading the store finishes first
  delete s;
}

extern "C" int hc_cold_defer_vectors(void* store, int defer) {
  ColdStore* s = as_store(store);
  if (!s) return set_error(HC_ERR_INVALID, "cold_defer_vectors: null store");
  s->wait_all_adds();
  if (defer) {
    std::unique_lock<std::shared_mutex> lk(s->mu);
    s->defer_vecs = true;
  } else {
    s->materialize_vecs(0);
  }
  return HC_OK;
}

extern "C" int64_t hc_cold_size(const void* store) {
  const ColdStore* s = reinterpret_cast<const ColdStore*>(store);
  if (!s) return 0;
  s->wait_all_adds();
  std::shared_lock<std::shared_mutex> lk(s->mu);
  return s->size;
}

namespace {

// The add itself (arguments checked by the caller, earlier adds applied).
int add_impl(ColdStore* s, int64_t te, const float* kpre, int64_t k_sh, int64_t k_st, const float* v, int64_t v_sh,
             int64_t v_st, const int64_t* pos, const int64_t* evicted_idx, int64_t nthreads) {
  // tokens kept: evicted_idx[t] >= 0 (datatypes.py:58-63 pads with -1)
  std::vector<int64_t> sel;
  sel.reserve((size_t)te);
  for (int64_t t = 0; t < te; ++t)
    if (!evicted_idx || evicted_idx[t] >= 0) sel.push_back(t);
  const int64_t m = (int64_t)sel.size();
  const int64_t first = m > s->cap ? m - s->cap : 0;  // only the last cap tokens survive
  std::unique_lock<std::shared_mutex> lk(s->mu);
  std::vector<int64_t> slot((size_t)(m - first));
  for (int64_t i = first; i < m; ++i) slot[i - first] = s->next_slot();
  // distinct slots: the copies and search vectors run on host threads
  constexpr int64_t kChunk = 256;
  const int64_t nchunks = (m - first + kChunk - 1) / kChunk;
  parallel_for(nchunks, threads_for(nthreads, nchunks), [&](int64_t c) {
    const int64_t i1 = std::min(m, first + (c + 1) * kChunk);
    for (int64_t i = first + c * kChunk; i < i1; ++i) {
      const int64_t t = sel[i];
      s->copy_in(slot[i - first], kpre + t * k_st, k_sh, v + t * v_st, v_sh, pos[t]);
    }
  });
  return HC_OK;
}

}  // namespace

extern "C" int hc_cold_add(void* store, int64_t te, const float* kpre, int64_t k_sh, int64_t k_st,
                           const float* v, int64_t v_sh, int64_t v_st, const int64_t* pos,
                           const int64_t* evicted_idx) {
  ColdStore* s = as_store(store);
  if (!s) return set_error(HC_ERR_INVALID, "cold_add: null store");
  if (te < 0 || (te > 0 && (!kpre || !v || !pos))) return set_error(HC_ERR_INVALID, "cold_add: bad arguments");
  s->wait_all_adds();  // after the asynchronous adds submitted before it
  return add_impl(s, te, kpre, k_sh, k_st, v, v_sh, v_st, pos, evicted_idx, 0);
}

extern "C" int hc_cold_search(const void* store, const float* q, int64_t r, int64_t head, int64_t* out,
                              int64_t* n_out) {
  const ColdStore* s = reinterpret_cast<const ColdStore*>(store);
  if (!s || !q || !out || !n_out) return set_error(HC_ERR_INVALID, "cold_search: null argument");
  if (head < 0 || head >= s->VH) return set_error(HC_ERR_INVALID, "cold_search: head %lld out of range", (long long)head);
  s->wait_all_adds();
  as_store(const_cast<void*>(store))->materialize_vecs(0);
  std::shared_lock<std::shared_mutex> lk(s->mu);
  std::vector<double> ip((size_t)std::max<int64_t>(s->size, 1));
  s->scan(q, head, 0, s->size, ip.data());
  *n_out = s->select(ip.data(), r, out);
  return HC_OK;
}

extern "C" int hc_cold_export(const void* store, float* kpre, float* v, int64_t* pos, float* vec) {
  const ColdStore* s = reinterpret_cast<const ColdStore*>(store);
  if (!s) return set_error(HC_ERR_INVALID, "cold_export: null store");
  s->wait_all_adds();
  if (vec) as_store(const_cast<void*>(store))->materialize_vecs(0);
  std::shared_lock<std::shared_mutex> lk(s->mu);
  const int64_t HD = s->H * s->D;
  for (int64_t i = 0; i < s->size; ++i) {
    const int64_t p = s->physical(i);
    if (kpre) memcpy(kpre + i * HD, &s->kpre[(size_t)p * HD], sizeof(float) * HD);
    if (v) memcpy(v + i * HD, &s->v[(size_t)p * HD], sizeof(float) * HD);
    if (pos) pos[i] = s->pos[p];
    if (vec)
      for (int64_t h = 0; h < s->VH; ++h)
        for (int64_t d = 0; d < s->VD; ++d)
          vec[(i * s->VH + h) * s->VD + d] = s->vec[s->vidx(h, d, p)];
  }
  return HC_OK;
}

namespace {

// fp32 -> bf16, round to nearest even (NaN stays a quiet NaN): the device's
// and torch's conversion.
inline uint16_t bf16_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// n fp32 values to the retrieval's element type (HC_DTYPE_*): fp32 copies;
// fp16 rounds to nearest even with F16C (subnormal results kept), as the
// device's and torch's conversions do; bf16 as bf16_bits.
void convert_row(const float* src, void* dst, int64_t n, int dtype) {
  if (dtype == HC_DTYPE_F32) {
    memcpy(dst, src, sizeof(float) * n);
  } else if (dtype == HC_DTYPE_F16) {
    uint16_t* o = static_cast<uint16_t*>(dst);
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
      _mm_storeu_si128(reinterpret_cast<__m128i*>(o + i),
                       _mm256_cvtps_ph(_mm256_loadu_ps(src + i), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
    for (; i < n; ++i)
      o[i] = (uint16_t)_mm_extract_epi16(_mm_cvtps_ph(_mm_set_ss(src[i]), _MM_FROUND_TO_NEAREST_INT), 0);
  } else {
    // bf16_bits eight at a time (AVX2): equal to it on every fp32 bit pattern
    uint16_t* o = static_cast<uint16_t*>(dst);
    const __m256i one = _mm256_set1_epi32(1), half = _mm256_set1_epi32(0x7fff), quiet = _mm256_set1_epi32(0x40);
    const __m256i absm = _mm256_set1_epi32(0x7fffffff), inf = _mm256_set1_epi32(0x7f800000);
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) {
      const __m256i u = _mm256_castps_si256(_mm256_loadu_ps(src + i));
      const __m256i hi = _mm256_srli_epi32(u, 16);
      const __m256i rnd = _mm256_srli_epi32(_mm256_add_epi32(u, _mm256_add_epi32(half, _mm256_and_si256(hi, one))), 16);
      const __m256i nan = _mm256_cmpgt_epi32(_mm256_and_si256(u, absm), inf);
      const __m256i r = _mm256_blendv_epi8(rnd, _mm256_or_si256(hi, quiet), nan);
      const __m256i pk = _mm256_permute4x64_epi64(_mm256_packus_epi32(r, r), 0xD8);
      _mm_storeu_si128(reinterpret_cast<__m128i*>(o + i), _mm256_castsi256_si128(pk));
    }
    for (; i < n; ++i) o[i] = bf16_bits(src[i]);
  }
}

inline int64_t kv_elem_bytes(int dtype) { return dtype == HC_DTYPE_F32 ? 4 : 2; }

// A retrieval's K/V output: [B][H][R][D] of the element type `dtype`.
struct KvOut {
  int dtype;
  void* k;
  void* v;
  void* row(void* base, int64_t i, int64_t D) const {
    return static_cast<char*>(base) + i * D * kv_elem_bytes(dtype);
  }
};

// Copy the rows of hits[0..m) (logical indices of store s, rank order) into
// output row (b, h) of a retrieval: kpre/v [B][H][R][D] (one head, or every
// head with a head-mean vector) in out.dtype, pos/valid [B][VH][R].  The
// caller holds the store's read lock; zero_tail fills rows [m, R).
void emit_hits(const ColdStore* s, int64_t b, int64_t h, int per_head, int64_t R, const int64_t* hits, int64_t m,
               const KvOut& out, int64_t* pos_out, uint8_t* valid_out) {
  const int64_t H = s->H, D = s->D, VH = per_head ? H : 1;
  for (int64_t j = 0; j < m; ++j) {
    const int64_t p = s->physical(hits[j]);
    const float* kp = &s->kpre[(size_t)p * H * D];
    const float* vp = &s->v[(size_t)p * H * D];
    const int64_t h0 = per_head ? h : 0, h1 = per_head ? h + 1 : H;
    for (int64_t hh = h0; hh < h1; ++hh) {
      convert_row(kp + hh * D, out.row(out.k, (b * H + hh) * R + j, D), D, out.dtype);
      convert_row(vp + hh * D, out.row(out.v, (b * H + hh) * R + j, D), D, out.dtype);
    }
    pos_out[(b * VH + h) * R + j] = s->pos[p];
    valid_out[(b * VH + h) * R + j] = 1;
  }
}

// Zero rows [from, R) of output row (b, h), the rows emit_hits leaves past
// the hits.  Each task zeroes only its own rows, on its own thread: zeroing
// all of the outputs up front was a single-threaded pass over as many bytes
// as the copies write (8 MB per search at batch 16, 8 KV heads, 128 rows).
void zero_tail(int64_t b, int64_t h, int per_head, int64_t H, int64_t R, int64_t D, int64_t from, const KvOut& out,
               int64_t* pos_out, uint8_t* valid_out) {
  if (from >= R) return;
  const int64_t VH = per_head ? H : 1;
  const int64_t h0 = per_head ? h : 0, h1 = per_head ? h + 1 : H;
  const size_t bytes = (size_t)((R - from) * D * kv_elem_bytes(out.dtype));
  for (int64_t hh = h0; hh < h1; ++hh) {
    memset(out.row(out.k, (b * H + hh) * R + from, D), 0, bytes);
    memset(out.row(out.v, (b * H + hh) * R + from, D), 0, bytes);
  }
  memset(pos_out + (b * VH + h) * R + from, 0, sizeof(int64_t) * (size_t)(R - from));
  memset(valid_out + (b * VH + h) * R + from, 0, (size_t)(R - from));
}

// Rows of the caller's table (one per position) at the retrieved positions of
// output row (b, h); rows past the hits take position 0.
void emit_tab(int64_t b, int64_t h, int64_t VH, int64_t R, const int64_t* pos_out, const uint8_t* tab,
              int64_t tab_rows, int64_t tab_row_bytes, uint8_t* tab_out, std::atomic<int64_t>& missing) {
  for (int64_t j = 0; j < R; ++j) {
    const int64_t p = pos_out[(b * VH + h) * R + j];
    uint8_t* dst = tab_out + ((b * VH + h) * R + j) * tab_row_bytes;
    if (p >= 0 && p < tab_rows) memcpy(dst, tab + p * tab_row_bytes, (size_t)tab_row_bytes);
    else { memset(dst, 0, (size_t)tab_row_bytes); missing.fetch_add(1); }
  }
}

// The search itself (every add the caller must see already applied).
int retrieve_impl(void* const* stores, int64_t B, const float* q, int64_t q_sb, int64_t q_sh, int64_t q_dim,
                  int normalize_q, int64_t R, int per_head, int kv_dtype, void* kpre_out, void* v_out,
                  int64_t* pos_out, uint8_t* valid_out, const uint8_t* tab, int64_t tab_rows, int64_t tab_row_bytes,
                  uint8_t* tab_out, int64_t* tab_missing, int64_t nthreads) {
  if (B <= 0 || R <= 0 || q_dim <= 0 || !stores || !q || !kpre_out || !v_out || !pos_out || !valid_out)
    return set_error(HC_ERR_INVALID, "cold_retrieve: bad arguments");
  if (kv_dtype != HC_DTYPE_F32 && kv_dtype != HC_DTYPE_F16 && kv_dtype != HC_DTYPE_BF16)
    return set_error(HC_ERR_INVALID, "cold_retrieve: bad output dtype %d", kv_dtype);
  const KvOut out{kv_dtype, kpre_out, v_out};
  if (tab && (tab_rows <= 0 || tab_row_bytes <= 0 || !tab_out))
    return set_error(HC_ERR_INVALID, "cold_retrieve: table rows need a size and an output");
  const ColdStore* s0 = reinterpret_cast<const ColdStore*>(stores[0]);
  if (!s0) return set_error(HC_ERR_INVALID, "cold_retrieve: null store");
  const int64_t H = s0->H, D = s0->D, VD = s0->VD;
  for (int64_t b = 0; b < B; ++b) {
    const ColdStore* s = reinterpret_cast<const ColdStore*>(stores[b]);
    if (!s || s->H != H || s->D != D || s->VD != VD || s->VH != (per_head ? H : 1))
      return set_error(HC_ERR_INVALID, "cold_retrieve: store %lld does not match (per_head=%d)", (long long)b,
                       per_head);
  }
  for (int64_t b = 0; b < B; ++b) as_store(stores[b])->materialize_vecs(nthreads);
  const int64_t VH = per_head ? H : 1;
  // outputs: kpre/v [B][H][R][D]; pos/valid [B][R] or [B][H][R]; rows past
  // the hits zero-filled
  std::atomic<int64_t> missing{0};
  const int64_t tasks = B * VH;
  parallel_for(tasks, threads_for(nthreads, tasks), [&](int64_t task) {
    const int64_t b = task / VH, h = task % VH;
    const ColdStore* s = reinterpret_cast<const ColdStore*>(stores[b]);
    // the query: cropped or zero-padded to the vector width, then (normalize_q)
    // divided by max(||x||, 1e-12) with the squares summed in dimension order
    // in fp64 and the quotient rounded to fp32, as the stored vectors are
    std::vector<float> qv((size_t)VD, 0.0f);
    const float* qs = q + b * q_sb + h * q_sh;
    double den = 1.0;
    if (normalize_q) {
      double ss = 0.0;
      for (int64_t d = 0; d < VD; ++d) {
        const double x = d < q_dim ? (double)qs[d] : 0.0;
        ss += x * x;
      }
      den = std::max(std::sqrt(ss), 1e-12);
    }
    for (int64_t d = 0; d < std::min(VD, q_dim); ++d) qv[d] = normalize_q ? (float)((double)qs[d] / den) : qs[d];
    int64_t m = 0;
    std::vector<int64_t> hits((size_t)R);
    {
      std::shared_lock<std::shared_mutex> lk(s->mu);
      if (s->size > 0) {
        std::vector<double> ip((size_t)s->size);
        s->scan(qv.data(), h, 0, s->size, ip.data());
        m = s->select(ip.data(), R, hits.data());
        emit_hits(s, b, h, per_head, R, hits.data(), m, out, pos_out, valid_out);
      }
    }
    zero_tail(b, h, per_head, H, R, D, m, out, pos_out, valid_out);
    if (tab) emit_tab(b, h, VH, R, pos_out, tab, tab_rows, tab_row_bytes, tab_out, missing);
  });
  if (tab_missing) *tab_missing = missing.load();
  return HC_OK;
}

// The rows of hits found elsewhere (the device search index): hits [B][VH][R]
// logical indices in rank order, -1 past the hits.
int gather_impl(void* const* stores, int64_t B, int per_head, int64_t R, const int64_t* hits, int kv_dtype,
                void* kpre_out, void* v_out, int64_t* pos_out, uint8_t* valid_out, const uint8_t* tab,
                int64_t tab_rows, int64_t tab_row_bytes, uint8_t* tab_out, int64_t* tab_missing, int64_t nthreads) {
  if (B <= 0 || R <= 0 || !stores || !hits || !kpre_out || !v_out || !pos_out || !valid_out)
    return set_error(HC_ERR_INVALID, "cold_gather: bad arguments");
  if (kv_dtype != HC_DTYPE_F32 && kv_dtype != HC_DTYPE_F16 && kv_dtype != HC_DTYPE_BF16)
    return set_error(HC_ERR_INVALID, "cold_gather: bad output dtype %d", kv_dtype);
  const KvOut out{kv_dtype, kpre_out, v_out};
  if (tab && (tab_rows <= 0 || tab_row_bytes <= 0 || !tab_out))
    return set_error(HC_ERR_INVALID, "cold_gather: table rows need a size and an output");
  const ColdStore* s0 = reinterpret_cast<const ColdStore*>(stores[0]);
  if (!s0) return set_error(HC_ERR_INVALID, "cold_gather: null store");
  const int64_t H = s0->H, D = s0->D;
  for (int64_t b = 0; b < B; ++b) {
    const ColdStore* s = reinterpret_cast<const ColdStore*>(stores[b]);
    if (!s || s->H != H || s->D != D)
      return set_error(HC_ERR_INVALID, "cold_gather: store %lld does not match", (long long)b);
  }
  const int64_t VH = per_head ? H : 1;
  std::atomic<int64_t> missing{0};
  std::atomic<int> bad{0};
  const int64_t tasks = B * VH;
  parallel_for(tasks, threads_for(nthreads, tasks), [&](int64_t task) {
    const int64_t b = task / VH, h = task % VH;
    const ColdStore* s = reinterpret_cast<const ColdStore*>(stores[b]);
    const int64_t* hs = hits + (b * VH + h) * R;
    {
      std::shared_lock<std::shared_mutex> lk(s->mu);
      int64_t m = 0;
      while (m < R && hs[m] >= 0) ++m;
      for (int64_t j = 0; j < m; ++j)
        if (hs[j] >= s->size) bad.store(1);
      int64_t filled = 0;
      if (!bad.load()) {
        emit_hits(s, b, h, per_head, R, hs, m, out, pos_out, valid_out);
        filled = m;
      }
      zero_tail(b, h, per_head, H, R, D, filled, out, pos_out, valid_out);
    }
    if (tab) emit_tab(b, h, VH, R, pos_out, tab, tab_rows, tab_row_bytes, tab_out, missing);
  });
  if (bad.load()) return set_error(HC_ERR_INVALID, "cold_gather: a hit beyond its store's tokens");
  if (tab_missing) *tab_missing = missing.load();
  return HC_OK;
}

}  // namespace

extern "C" int hc_cold_gather(void* const* stores, int64_t B, int per_head, int64_t R, const int64_t* hits,
                              int kv_dtype, void* kpre_out, void* v_out, int64_t* pos_out, uint8_t* valid_out,
                              const uint8_t* tab, int64_t tab_rows, int64_t tab_row_bytes, uint8_t* tab_out,
                              int64_t* tab_missing, int64_t nthreads) {
  if (B > 0 && stores)
    for (int64_t b = 0; b < B; ++b)
      if (stores[b]) as_store(stores[b])->wait_all_adds();
  return gather_impl(stores, B, per_head, R, hits, kv_dtype, kpre_out, v_out, pos_out, valid_out, tab, tab_rows,
                     tab_row_bytes, tab_out, tab_missing, nthreads);
}

extern "C" int hc_cold_retrieve(void* const* stores, int64_t B, const float* q, int64_t q_sb, int64_t q_sh,
                                int64_t q_dim, int normalize_q, int64_t R, int per_head, int kv_dtype,
                                void* kpre_out, void* v_out, int64_t* pos_out, uint8_t* valid_out, const uint8_t* tab,
                                int64_t tab_rows, int64_t tab_row_bytes, uint8_t* tab_out, int64_t* tab_missing,
                                int64_t nthreads) {
  if (B > 0 && stores)
    for (int64_t b = 0; b < B; ++b)
      if (stores[b]) as_store(stores[b])->wait_all_adds();  // after the adds submitted before it
  return retrieve_impl(stores, B, q, q_sb, q_sh, q_dim, normalize_q, R, per_head, kv_dtype, kpre_out, v_out, pos_out,
                       valid_out, tab, tab_rows, tab_row_bytes, tab_out, tab_missing, nthreads);
}

// ---------------------------------------------------------------------------
// Retrievals as jobs on the library's own worker threads.  The decode thread
// submits a job and later polls it; a worker waits for the job's event (the
// pooled query's device-to-host copy), runs hc_cold_retrieve, counts the
// valid rows, and marks the job done.  No Python runs on the workers, so a
// search never contends for the interpreter lock with the decode loop.
// ---------------------------------------------------------------------------
namespace {

struct RetrieveJob {
  bool is_add = false;           // an asynchronous add instead of a search
  const int64_t* hits = nullptr; // a gather of these hits instead of a search
  std::vector<void*> stores;
  std::vector<int64_t> tickets;  // per store: the adds submitted before this search
  // add arguments (is_add)
  int64_t add_te = 0, add_k_sh = 0, add_k_st = 0, add_v_sh = 0, add_v_st = 0, add_ticket = 0, add_threads = 0;
  const float* add_kpre = nullptr;
  const float* add_v = nullptr;
  const int64_t* add_pos = nullptr;
  const int64_t* add_idx = nullptr;
  int64_t B = 0, q_sb = 0, q_sh = 0, q_dim = 0, R = 0, tab_rows = 0, tab_row_bytes = 0, nthreads = 0;
  int64_t n_flags = 0;  // valid_out entries: B * R, or B * heads * R per KV head
  int normalize_q = 0, per_head = 0;
  const float* q = nullptr;
  int kv_dtype = HC_DTYPE_F32;
  void* kpre_out = nullptr;
  void* v_out = nullptr;
  int64_t* pos_out = nullptr;
  uint8_t* valid_out = nullptr;
  const uint8_t* tab = nullptr;
  uint8_t* tab_out = nullptr;
  void* wait_event = nullptr;
  std::mutex mu;
  std::condition_variable cv;
  bool done = false;
  int rc = HC_OK;
  int64_t n_valid = 0, tab_missing = 0;
  char msg[512] = "";
};

class JobQueue {
 public:
  void push(RetrieveJob* j, int64_t workers) {
    std::lock_guard<std::mutex> lk(mu_);
    const int64_t want = std::max<int64_t>(1, std::min<int64_t>(workers, 16));
    while ((int64_t)started_ < want) {
      std::thread(&JobQueue::run, this).detach();  // lives until the process ends
      ++started_;
    }
    jobs_.push_back(j);
    cv_.notify_one();
  }

 private:
  void run() {
    for (;;) {
      RetrieveJob* j;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return !jobs_.empty(); });
        j = jobs_.front();
        jobs_.pop_front();
      }
      execute(j);
    }
  }

  // Waits for a device event by polling it, asleep between polls: a worker
  // blocked in the runtime's own wait spins there and slows the launches the
  // decode thread issues meanwhile.  Retrievals take milliseconds, so the
  // polling granularity is immaterial.
  static int wait_device_event(void* ev) {
    for (;;) {
      const int r = hc_event_query(ev);
      if (r != 0) return r < 0 ? r : HC_OK;
      std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
  }

  static void execute(RetrieveJob* j) {
    int rc = HC_OK;
    if (j->wait_event) rc = wait_device_event(j->wait_event);
    int64_t missing = 0, nv = 0;
    if (j->is_add) {
      // after the store's earlier adds (the queue hands jobs out in order, so
      // those are running or done); the ticket is served even on failure
      ColdStore* s = as_store(j->stores[0]);
      s->wait_adds(j->add_ticket);
      if (rc == HC_OK)
        rc = add_impl(s, j->add_te, j->add_kpre, j->add_k_sh, j->add_k_st, j->add_v, j->add_v_sh, j->add_v_st,
                      j->add_pos, j->add_idx, j->add_threads);
      s->serve_ticket();
    } else {
      for (size_t b = 0; b < j->stores.size(); ++b) as_store(j->stores[b])->wait_adds(j->tickets[b]);
      if (rc == HC_OK && j->hits)
        rc = gather_impl(j->stores.data(), j->B, j->per_head, j->R, j->hits, j->kv_dtype, j->kpre_out, j->v_out,
                         j->pos_out,
                         j->valid_out, j->tab, j->tab_rows, j->tab_row_bytes, j->tab_out, &missing, j->nthreads);
      else if (rc == HC_OK)
        rc = retrieve_impl(j->stores.data(), j->B, j->q, j->q_sb, j->q_sh, j->q_dim, j->normalize_q, j->R,
                           j->per_head, j->kv_dtype, j->kpre_out, j->v_out, j->pos_out, j->valid_out, j->tab, j->tab_rows,
                           j->tab_row_bytes, j->tab_out, &missing, j->nthreads);
      if (rc == HC_OK)
        for (int64_t i = 0; i < j->n_flags; ++i) nv += j->valid_out[i] != 0;
    }
    for (void* st : j->stores) as_store(st)->unpin();
    std::lock_guard<std::mutex> lk(j->mu);
    if (rc != HC_OK) snprintf(j->msg, sizeof(j->msg), "%s", hc_last_error());
    j->rc = rc;
    j->n_valid = nv;
    j->tab_missing = missing;
    j->done = true;
    j->cv.notify_all();
  }

  std::mutex mu_;
  std::condition_variable cv_;
  std::deque<RetrieveJob*> jobs_;
  int started_ = 0;
};

JobQueue& job_queue() {
  static JobQueue* q = new JobQueue();  // never destroyed: its threads outlive static destruction
  return *q;
}

}  // namespace

extern "C" void* hc_cold_retrieve_async(void* const* stores, int64_t B, const float* q, int64_t q_sb, int64_t q_sh,
                                        int64_t q_dim, int normalize_q, int64_t R, int per_head, int kv_dtype,
                                        void* kpre_out, void* v_out, int64_t* pos_out, uint8_t* valid_out,
                                        const uint8_t* tab, int64_t tab_rows, int64_t tab_row_bytes, uint8_t* tab_out,
                                        int64_t nthreads, void* wait_event, int64_t workers) {
  if (B <= 0 || R <= 0 || q_dim <= 0 || !stores || !q || !kpre_out || !v_out || !pos_out || !valid_out ||
      (kv_dtype != HC_DTYPE_F32 && kv_dtype != HC_DTYPE_F16 && kv_dtype != HC_DTYPE_BF16)) {
    set_error(HC_ERR_INVALID, "cold_retrieve_async: bad arguments");
    return nullptr;
  }
  if (tab && (tab_rows <= 0 || tab_row_bytes <= 0 || !tab_out)) {
    set_error(HC_ERR_INVALID, "cold_retrieve_async: table rows need a size and an output");
    return nullptr;
  }
  for (int64_t b = 0; b < B; ++b)
    if (!stores[b]) {
      set_error(HC_ERR_INVALID, "cold_retrieve_async: null store %lld", (long long)b);
      return nullptr;
    }
  RetrieveJob* j = new (std::nothrow) RetrieveJob();
  if (!j) {
    set_error(HC_ERR_INVALID, "cold_retrieve_async: out of host memory");
    return nullptr;
  }
  const ColdStore* s0 = as_store(stores[0]);
  j->stores.assign(stores, stores + B);
  j->B = B; j->q = q; j->q_sb = q_sb; j->q_sh = q_sh; j->q_dim = q_dim; j->normalize_q = normalize_q;
  j->R = R; j->per_head = per_head; j->kv_dtype = kv_dtype; j->kpre_out = kpre_out; j->v_out = v_out;
  j->pos_out = pos_out; j->valid_out = valid_out; j->tab = tab; j->tab_rows = tab_rows;
  j->tab_row_bytes = tab_row_bytes; j->tab_out = tab_out; j->nthreads = nthreads; j->wait_event = wait_event;
  j->n_flags = B * R * (per_head ? s0->H : 1);
  for (int64_t b = 0; b < B; ++b) {
    as_store(stores[b])->pin();
    j->tickets.push_back(as_store(stores[b])->tickets());
  }
  job_queue().push(j, workers);
  return j;
}

extern "C" void* hc_cold_gather_async(void* const* stores, int64_t B, int per_head, int64_t R, const int64_t* hits,
                                      int kv_dtype, void* kpre_out, void* v_out, int64_t* pos_out,
                                      uint8_t* valid_out, const uint8_t* tab, int64_t tab_rows, int64_t tab_row_bytes,
                                      uint8_t* tab_out, int64_t nthreads, void* wait_event, int64_t workers) {
  if (B <= 0 || R <= 0 || !stores || !hits || !kpre_out || !v_out || !pos_out || !valid_out ||
      (kv_dtype != HC_DTYPE_F32 && kv_dtype != HC_DTYPE_F16 && kv_dtype != HC_DTYPE_BF16)) {
    set_error(HC_ERR_INVALID, "cold_gather_async: bad arguments");
    return nullptr;
  }
  if (tab && (tab_rows <= 0 || tab_row_bytes <= 0 || !tab_out)) {
    set_error(HC_ERR_INVALID, "cold_gather_async: table rows need a size and an output");
    return nullptr;
  }
  for (int64_t b = 0; b < B; ++b)
    if (!stores[b]) {
      set_error(HC_ERR_INVALID, "cold_gather_async: null store %lld", (long long)b);
      return nullptr;
    }
  RetrieveJob* j = new (std::nothrow) RetrieveJob();
  if (!j) {
    set_error(HC_ERR_INVALID, "cold_gather_async: out of host memory");
    return nullptr;
  }
  const ColdStore* s0 = as_store(stores[0]);
  j->stores.assign(stores, stores + B);
  j->hits = hits;
  j->B = B; j->R = R; j->per_head = per_head; j->kv_dtype = kv_dtype; j->kpre_out = kpre_out; j->v_out = v_out;
  j->pos_out = pos_out; j->valid_out = valid_out; j->tab = tab; j->tab_rows = tab_rows;
  j->tab_row_bytes = tab_row_bytes;
  j->tab_out = tab_out; j->nthreads = nthreads; j->wait_event = wait_event;
  j->n_flags = B * R * (per_head ? s0->H : 1);
  for (int64_t b = 0; b < B; ++b) {
    as_store(stores[b])->pin();
    j->tickets.push_back(as_store(stores[b])->tickets());
  }
  job_queue().push(j, workers);
  return j;
}

extern "C" void* hc_cold_add_async(void* store, int64_t te, const float* kpre, int64_t k_sh, int64_t k_st,
                                   const float* v, int64_t v_sh, int64_t v_st, const int64_t* pos,
                                   const int64_t* evicted_idx, void* wait_event, int64_t nthreads,
                                   int64_t workers) {
  ColdStore* s = as_store(store);
  if (!s || te < 0 || (te > 0 && (!kpre || !v || !pos))) {
    set_error(HC_ERR_INVALID, "cold_add_async: bad arguments");
    return nullptr;
  }
  RetrieveJob* j = new (std::nothrow) RetrieveJob();
  if (!j) {
    set_error(HC_ERR_INVALID, "cold_add_async: out of host memory");
    return nullptr;
  }
  j->is_add = true;
  j->stores.assign(1, store);
  j->add_te = te; j->add_kpre = kpre; j->add_k_sh = k_sh; j->add_k_st = k_st; j->add_v = v; j->add_v_sh = v_sh;
  j->add_v_st = v_st; j->add_pos = pos; j->add_idx = evicted_idx; j->wait_event = wait_event;
  j->add_threads = nthreads;
  s->pin();
  j->add_ticket = s->take_ticket();
  job_queue().push(j, workers);
  return j;
}

extern "C" int hc_cold_job_poll(void* job, int wait, int64_t* n_valid, int64_t* tab_missing) {
  RetrieveJob* j = reinterpret_cast<RetrieveJob*>(job);
  if (!j) return set_error(HC_ERR_INVALID, "cold_job_poll: null job");
  std::unique_lock<std::mutex> lk(j->mu);
  if (wait) j->cv.wait(lk, [&] { return j->done; });
  if (!j->done) return 0;
  if (n_valid) *n_valid = j->n_valid;
  if (tab_missing) *tab_missing = j->tab_missing;
  if (j->rc != HC_OK) return set_error(j->rc, "cold_retrieve (worker): %s", j->msg);
  return 1;
}

extern "C" void hc_cold_job_free(void* job) {
  RetrieveJob* j = reinterpret_cast<RetrieveJob*>(job);
  if (!j) return;
  {
    std::unique_lock<std::mutex> lk(j->mu);
    j->cv.wait(lk, [&] { return j->done; });  // never free a job a worker still holds
  }
  delete j;
}
