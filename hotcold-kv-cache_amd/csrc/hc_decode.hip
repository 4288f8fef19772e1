// GQA decode attention: host side and C ABI (kernels in hc_decode_kernels.h).
//
// Replaces evict_fwd_kernel / triton_evict_attention_forward
// (src/hotcold_kv/kernels.py:9-137); the H2O score kernels and the
// reference's per-token eviction score run here after the attention.
#include "hc_decode_kernels.h"
#include <algorithm>
#include <atomic>
#include <mutex>

namespace hc {

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
constexpr int kH2OMaxG = 8;    // query heads per KV head with the batched score loads
                               // (kernels for groups of up to 4 and up to 8)
constexpr int kH2OBatch = 4;   // keys per thread whose scores are loaded together
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

template <int GM>
__global__ __launch_bounds__(256) void h2o_evict_one_kernel(const float* scores, const float* ml, int Hq, int G,
                                                            int S, const float* acc, int64_t a_sb, int64_t a_sh,
                                                            H2OEvictArgs e) {
  static_assert(GM >= 1 && GM <= kH2OMaxG, "group bound of the batched score loads");
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
  if (G <= GM) {
    // h2o_updated with the group's (max, sum) pairs loaded once and the score
    // loads of kH2OBatch keys issued before any is used (the same operations
    // in the same order, so the same bits)
    // (register arrays indexed only by unrolled constants; heads past G, up to
    // the kernel's bound GM, are loaded from head G-1 and not used, so every
    // load is unconditional)
    float Mg[GM], Lg[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      const int h = hk * G + min(g, G - 1);
      Mg[g] = ml[((int64_t)b * Hq + h) * 2 + 0];
      Lg[g] = ml[((int64_t)b * Hq + h) * 2 + 1];
    }
    for (int s0 = tid; s0 < S; s0 += 256 * kH2OBatch) {
      float sc[kH2OBatch][GM], av[kH2OBatch];
#pragma unroll
      for (int j = 0; j < kH2OBatch; ++j) {
        const int s = min(s0 + 256 * j, S - 1);
        // the new token (s = S-1) has no accumulated score: its column is
        // never read, so the load is clamped to the last existing one
        av[j] = S >= 2 ? arow[min(s, S - 2)] : 0.f;
#pragma unroll
        for (int g = 0; g < GM; ++g) sc[j][g] = scores[((int64_t)b * Hq + hk * G + min(g, G - 1)) * S + s];
      }
#pragma unroll
      for (int j = 0; j < kH2OBatch; ++j) {
        const int s = s0 + 256 * j;
        if (s < S) {
          float col = 0.f;
#pragma unroll
          for (int g = 0; g < GM; ++g)
            if (g < G) col += (sc[j][g] == -INFINITY) ? 0.f : exp2f(sc[j][g] - Mg[g]) / Lg[g];
          col /= (float)G;
          sm_sc[s] = (s == S - 1 ? 0.f : av[j]) + col;
        }
      }
    }
  } else {
    for (int s = tid; s < S; s += 256) sm_sc[s] = h2o_updated(scores, ml, Hq, G, S, b, hk, s, arow);
  }
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

// The first kCounterBytes of a decode workspace hold the in-kernel merge's
// arrival words, one 64-bit [launch tag | done bit, arrivals] per (batch,
// kv head).  They need no initialisation: every launch counts under a tag
// of its own (kernel comment at the arrival).
constexpr int64_t kCounterBytes = 16384;
constexpr int64_t kMaxMergeUnits = kCounterBytes / 8;

// Launch tags of the in-kernel merge: consecutive launches get different
// tags (a 32-bit counter, wrapping after 2^32 launches).
static std::atomic<uint32_t> g_launch_tag{0};

// The tag a workspace's arrival words were last left under: a launch that
// passes it counts on the words as they are, with one atomic per
// workgroup; words under any other tag cost its first arrivals a
// compare-and-swap each.  A direct-mapped table of recent workspaces: a
// workspace whose entry another one took only costs its next launch those
// swaps.
namespace {
constexpr int kTagSlots = 256;
struct TagSlot {
  uintptr_t ws;
  uint32_t tag;
};
TagSlot g_tag_slots[kTagSlots];
std::mutex g_tag_mu;

// Records tag as the workspace's latest and returns the one before it (or
// tag itself for a workspace not in the table).
uint32_t exchange_workspace_tag(const void* ws, uint32_t tag) {
  const uintptr_t p = reinterpret_cast<uintptr_t>(ws);
  TagSlot& slot = g_tag_slots[((p >> 8) ^ (p >> 20)) % kTagSlots];
  std::lock_guard<std::mutex> lk(g_tag_mu);
  const uint32_t prev = slot.ws == p ? slot.tag : tag;
  slot.ws = p;
  slot.tag = tag;
  return prev;
}
}  // namespace
// The in-kernel merge is used up to this many workgroups.  Its chain (the
// partial's device-coherent stores, the arrival count, the last workgroup's
// loads) costs a few memory round trips on the last workgroup of each unit,
// less than a second kernel for a small grid (one layer at batch 1: 8.8 us
// against 13.1 us at 5 splits); on large grids the second kernel is cheaper.
constexpr int64_t kMaxMergeWorkgroups = 512;

// Launch shape of one decode call: waves per workgroup, key splits per
// (batch, kv head) and keys per split (a multiple of 16 * nw).
struct DecodeShape {
  int nw;
  int splits;
  int64_t kps;
  bool merge_in_kernel;
};

// requested > 0: that many splits (tests and callers that pin the shape).
// Otherwise:
//   * few units with short key ranges (up to 512 KB of K and V per unit, e.g.
//     one layer at batch 1): one 16-key tile per wave, up to 256 workgroups.
//     One workgroup per unit reads at a small fraction of what the chip can
//     (about 32 GB/s per CU), so the unit's keys are spread over several CUs
//     and merged in the kernel;
//   * otherwise enough workgroups to give every CU one 8-wave (or two 4-wave)
//     workgroups, and no split shorter than one tile per wave.
// With the keep bitmap (mask or held slot) no split is longer than the bitmap.
static DecodeShape decode_shape(int es, int64_t D, int64_t G, int64_t units, int64_t S, int64_t requested,
                                bool bitmap) {
  const int nw = decode_cfg(es, (int)D, group_bucket(G)).nw;
  const int64_t step = 16 * nw;
  int64_t splits = requested;
  if (splits <= 0) {
    if (units < 128 && S * 2 * D * es <= ((int64_t)512 << 10))
      splits = std::min<int64_t>(cdiv(S, step), std::max<int64_t>(1, 256 / units));
    else
      splits = cdiv((int64_t)256 * 8 / nw, units);
  }
  const int64_t max_splits = cdiv(S, step);
  if (splits > max_splits) splits = max_splits;
  if (bitmap && splits < cdiv(S, kMaxBitmapKeys)) splits = cdiv(S, kMaxBitmapKeys);
  if (splits < 1) splits = 1;
  const int64_t kps = cdiv(cdiv(S, splits), step) * step;
  const int out_splits = (int)cdiv(S, kps);
  const bool mk = out_splits > 1 && units <= kMaxMergeUnits && units * out_splits <= kMaxMergeWorkgroups;
  return DecodeShape{nw, out_splits, kps, mk};
}

static int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

// Launch shape of one call over S_cache cached rows (the choice decode_impl makes).
static DecodeShape decode_call_shape(int es, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S_cache,
                                     int64_t num_splits, bool bitmap) {
  return decode_shape(es, D, Hq / Hk, B * Hk, S_cache > 0 ? S_cache : 1, num_splits, bitmap);
}

struct DecodeLayout {
  int64_t part_off, scores_off, ml_off, total;
};

// [counters (kCounterBytes)][split partials][eviction logits][(max, sum)]
static DecodeLayout decode_layout(int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
                                  int64_t splits, int with_evict) {
  DecodeLayout L;
  const int64_t units = B * Hk;
  const int64_t G = Hq / (Hk > 0 ? Hk : 1);
  L.part_off = kCounterBytes;
  const int64_t part_bytes = splits > 1 ? units * splits * (G * D + 2 * G) * 4 : 0;
  L.scores_off = align256(L.part_off + part_bytes);
  const int64_t scores_bytes = with_evict ? B * Hq * S * 4 : 0;
  L.ml_off = align256(L.scores_off + scores_bytes);
  const int64_t ml_bytes = with_evict ? B * Hq * 2 * 4 : 0;
  L.total = align256(L.ml_off + ml_bytes);
  return L;
}

}  // namespace hc

using namespace hc;

extern "C" int64_t hc_decode_attn_workspace_size(int64_t B, int64_t Hq, int64_t Hk, int64_t D,
                                                 int64_t S, int64_t num_splits, int with_evict) {
  if (B <= 0 || Hq <= 0 || Hk <= 0 || D <= 0 || S <= 0 || Hq % Hk != 0) return align256(kCounterBytes);
  // The element size is not an argument: size for every launch shape.
  int64_t need = 0;
  for (int es : {2, 4})
    for (bool bitmap : {false, true})
      for (int64_t Sc : {S, S > 1 ? S - 1 : S}) {
        const DecodeShape sh = decode_call_shape(es, B, Hq, Hk, D, Sc, num_splits, bitmap);
        const int64_t t = decode_layout(B, Hq, Hk, D, S, sh.splits, with_evict).total;
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
  const bool bitmap = mask != nullptr || held_len > 0;
  const int64_t S_cache = ap ? S - 1 : S;  // a fused append's token is not read from k/v
  HC_REQUIRE(held_len <= S_cache, "decode: held_len %lld beyond the cached rows", (long long)held_len);
  const DecodeShape shape = decode_call_shape(es, B, Hq, Hk, D, S_cache, num_splits, bitmap);
  const int splits = shape.splits;
  const int nw = shape.nw;
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
  a.keys_per_split = (int)shape.kps;
  a.S_cache = (int)S_cache;
  a.counters = shape.merge_in_kernel ? reinterpret_cast<unsigned long long*>(ws) : nullptr;
  a.epoch = g_launch_tag.fetch_add(1, std::memory_order_relaxed) + 1;
  a.prev_epoch = a.counters ? exchange_workspace_tag(ws, a.epoch) : a.epoch;
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
  if (dtype == HC_DTYPE_F16) rc = decode_dispatch_f16(D, a, nw, st);
  else if (dtype == HC_DTYPE_BF16) rc = decode_dispatch_bf16(D, a, nw, st);
  else rc = decode_dispatch_f32(D, a, nw, st);
  if (rc != HC_OK) return rc;
  if ((rc = check_launch("decode_attn")) != HC_OK) return rc;

  if (h2o_acc && h2o_ev) {
    const dim3 grid((unsigned)cdiv(S, h2o_ev->rows_per_wg), (unsigned)Hk, (unsigned)B);
    // a group of up to 4 (e.g. 32 query / 8 KV heads) loads only its own
    // heads' scores; larger groups take the bound-8 kernel (key by key past 8)
    if (G <= 4)
      hipLaunchKernelGGL(h2o_evict_one_kernel<4>, grid, dim3(256), 0, st, a.scores, a.ml, (int)Hq, G, (int)S,
                         h2o_acc, h2o_sb, h2o_sh, *h2o_ev);
    else
      hipLaunchKernelGGL(h2o_evict_one_kernel<kH2OMaxG>, grid, dim3(256), 0, st, a.scores, a.ml, (int)Hq, G,
                         (int)S, h2o_acc, h2o_sb, h2o_sh, *h2o_ev);
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

extern "C" int hc_decode_attn_append_packed(const hc_decode_append_args* a, void* stream) {
  HC_REQUIRE(a != nullptr, "decode_append_packed: null argument struct");
  HC_REQUIRE(a->dtype >= INT32_MIN && a->dtype <= INT32_MAX, "decode_append_packed: bad dtype");
  return hc_decode_attn_append((int)a->dtype, a->B, a->Hq, a->Hk, a->D, a->S, a->q, a->q_sb, a->q_sh, a->k, a->k_sb,
                               a->k_sh, a->k_ss, a->v, a->v_sb, a->v_sh, a->v_ss, a->k_new, a->kn_sb, a->kn_sh,
                               a->v_new, a->vn_sb, a->vn_sh, a->p_new, a->pn_sb, a->pn_sh, a->p_dst, a->pd_sb,
                               a->pd_sh, a->pd_ss, a->pos_new, a->posn_sb, a->pos_dst, a->posd_sb, a->mask,
                               a->mask_sb, a->held_len, a->held_pos, a->hp_sb, a->hp_sh, a->held_valid, a->hv_sb,
                               a->hv_sh, a->cur_pos, a->scaling, a->out, a->o_sb, a->o_sh, a->workspace,
                               a->workspace_bytes, a->num_splits, stream);
}

extern "C" int64_t hc_decode_append_args_size(void) { return (int64_t)sizeof(hc_decode_append_args); }

static_assert(sizeof(hc_decode_append_args) == 51 * 8, "hc_decode_append_args: every field is 8 bytes, no padding");

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

extern "C" int hc_decode_attn_h2o_evict_packed(const hc_decode_h2o_evict_args* a, void* stream) {
  HC_REQUIRE(a != nullptr, "decode_h2o_evict_packed: null argument struct");
  HC_REQUIRE(a->dtype >= INT32_MIN && a->dtype <= INT32_MAX, "decode_h2o_evict_packed: bad dtype");
  return hc_decode_attn_h2o_evict((int)a->dtype, a->B, a->Hq, a->Hk, a->D, a->S, a->q, a->q_sb, a->q_sh, a->k,
                                  a->k_sb, a->k_sh, a->k_ss, a->v, a->v_sb, a->v_sh, a->v_ss, a->k_new, a->kn_sb,
                                  a->kn_sh, a->v_new, a->vn_sb, a->vn_sh, a->scaling, a->out, a->o_sb, a->o_sh, a->acc,
                                  a->a_sb, a->a_sh, a->window, a->budget, a->k_dst, a->kd_sb, a->kd_sh, a->kd_ss,
                                  a->v_dst, a->vd_sb, a->vd_sh, a->vd_ss, a->acc_dst, a->ad_sb, a->ad_sh, a->workspace,
                                  a->workspace_bytes, a->num_splits, stream);
}

extern "C" int64_t hc_decode_h2o_evict_args_size(void) { return (int64_t)sizeof(hc_decode_h2o_evict_args); }

static_assert(sizeof(hc_decode_h2o_evict_args) == 46 * 8,
              "hc_decode_h2o_evict_args: every field is 8 bytes, no padding");

// ---------------------------------------------------------------------------
// Allocation-free fused append + decode, for callers that cannot allocate
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  It is hc_decode_attn_append with the split partials and merge
// words kept in a static device array instead of a caller-owned workspace:
//   * the array (kNoAllocSlots regions of kNoAllocSlotBytes) lives in the
//     library's code object, so every GPU the library runs on holds its own
//     copy until the process ends;
//   * its device address is taken once per device with hipGetSymbolAddress
//     (on the first call on that device, with that device current) and only
//     that address is passed to the kernels -- the array's name in host code
//     is a host-side stand-in, not device memory;
//   * each region serves one stream: the first call from a stream binds it a
//     free region for the rest of the process, so calls from different
//     streams never share partials, and calls from one stream are ordered by
//     that stream; a call from a stream beyond the regions is refused
//     (HC_ERR_INVALID).  The partials are fully written before they are read
//     and the merge words count under per-launch tags, so nothing is cleared;
//   * a call whose partials would not fit a region is refused
//     (HC_ERR_WORKSPACE), and no call allocates or frees memory.
// ---------------------------------------------------------------------------
namespace hc {
constexpr int kNoAllocSlots = 4;
constexpr int64_t kNoAllocSlotBytes = (int64_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocSlots * kNoAllocSlotBytes];
constexpr int kMaxScratchDevices = 64;
static void* g_scratch_ptr[kMaxScratchDevices];
static void* g_slot_stream[kMaxScratchDevices][kNoAllocSlots];
static bool g_slot_bound[kMaxScratchDevices][kNoAllocSlots];
static std::mutex g_scratch_mu;

// Device address of the calling stream's region of the current device's
// scratch array: the array's address is taken on the device's first call,
// and the stream is bound a free region on its first call.
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
  int slot = -1;
  for (int i = 0; i < kNoAllocSlots && slot < 0; ++i)
    if (g_slot_bound[dev][i] && g_slot_stream[dev][i] == stream) slot = i;
  for (int i = 0; i < kNoAllocSlots && slot < 0; ++i)
    if (!g_slot_bound[dev][i]) {
      g_slot_bound[dev][i] = true;
      g_slot_stream[dev][i] = stream;
      slot = i;
    }
  if (slot < 0)
    return set_error(HC_ERR_INVALID,
                     "decode_append_noalloc: the static scratch of device %d serves %d streams and all are bound to "
                     "other streams (calls from more streams would share partials); use hc_decode_attn_append",
                     dev, kNoAllocSlots);
  *out = static_cast<char*>(g_scratch_ptr[dev]) + (int64_t)slot * kNoAllocSlotBytes;
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
  const int splits = decode_call_shape(dtype_size(dtype), B, Hq, Hk, D, S - 1, num_splits, bitmap).splits;
  const int64_t need = decode_layout(B, Hq, Hk, D, S, splits, 0).total;
  if (need > kNoAllocSlotBytes)
    return set_error(HC_ERR_WORKSPACE,
                     "decode_append_noalloc: %d key splits over %lld (batch, kv head) units need %lld bytes of "
                     "scratch, above the static maximum of %lld bytes; use fewer splits or hc_decode_attn_append",
                     splits, (long long)(B * Hk), (long long)need, (long long)kNoAllocSlotBytes);
  void* ws = nullptr;
  int rc = scratch_address(stream, &ws);
  if (rc != HC_OK) return rc;
  return hc_decode_attn_append(dtype, B, Hq, Hk, D, S, q, q_sb, q_sh, k, k_sb, k_sh, k_ss, v, v_sb, v_sh, v_ss,
                               k_new, kn_sb, kn_sh, v_new, vn_sb, vn_sh, p_new, pn_sb, pn_sh, p_dst, pd_sb, pd_sh,
                               pd_ss, pos_new, posn_sb, pos_dst, posd_sb, mask, mask_sb, held_len, held_pos, hp_sb,
                               hp_sh, held_valid, hv_sb, hv_sh, cur_pos, scaling, out, o_sb, o_sh, ws,
                               kNoAllocSlotBytes, num_splits, stream);
}
