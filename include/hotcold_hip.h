/*
 * hotcold_hip.h -- C ABI of the MI355X (gfx950) hot tier of hotcold-kv-cache.
 *
 * Every entry point takes plain device pointers, int64 sizes and element
 * strides, a dtype code and a hipStream_t (passed as void*), and returns an
 * int status: HC_OK (0) or a negative HC_ERR_* code.  hc_last_error() returns
 * a message for the last failure on the calling thread.  Nothing here
 * allocates device memory: scratch space is a caller-owned workspace whose
 * size the matching *_workspace_size() function reports (the one exception,
 * hc_decode_attn_append_noalloc, uses a static device array instead).
 *
 * Strides are in ELEMENTS of the tensor they describe.  The innermost (head
 * dimension) stride is always 1.  A stride of 0 broadcasts (for example one
 * index set shared by every KV head).
 *
 * Citations name the reference interface (tarun931/hotcold-kv-cache,
 * src/hotcold_kv/...) each entry point replaces.
 */
#ifndef HOTCOLD_HIP_H
#define HOTCOLD_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HC_OK 0
#define HC_ERR_INVALID (-1)     /* bad argument (shape, stride, dtype, size) */
#define HC_ERR_HIP (-2)         /* a HIP runtime call failed */
#define HC_ERR_UNSUPPORTED (-3) /* valid but unsupported configuration */
#define HC_ERR_WORKSPACE (-4)   /* workspace missing or too small */
#define HC_ERR_GROUP (-5)       /* Hq / n_rep != Hk (kernels.py:99-100) */
#define HC_ERR_DROPOUT (-6)     /* dropout != 0 (kernels.py:88-89) */

#define HC_DTYPE_F32 0
#define HC_DTYPE_F16 1
#define HC_DTYPE_BF16 2

#define HC_POOL_MAX 0 /* F.max_pool1d, scoring.py:47 */
#define HC_POOL_AVG 1 /* F.avg_pool1d(count_include_pad=True), scoring.py:45-46 */

/* Score modes for hc_snapkv_score. */
#define HC_SCORE_SNAPKV 0 /* causal-masked softmax over keys, summed over the window (scoring.py:50-79) */
#define HC_SCORE_RAWSUM 1 /* raw q.k / sqrt(D) summed over the window, no mask (cache.py:68-69) */

/* Library identity and errors. */
int hc_abi_version(void);
const char* hc_last_error(void);

/* Calibration read (no counterpart in the reference): stream `bytes` (a
 * multiple of 16) from the 16-byte aligned device pointer p once, with
 * 16-byte loads over up to 1024 workgroups, writing nothing (sink may be
 * NULL).  The benchmark times it on the decode's byte count as the plain-read
 * floor the decode kernel is compared with. */
int hc_read_bytes(const void* p, int64_t bytes, uint32_t* sink, void* stream);

/*
 * GQA decode attention over the hot buffer (+ held retrieved slot), split-K.
 * Replaces evict_fwd_kernel + triton_evict_attention_forward
 * (kernels.py:9-74, 77-137) and the call site at patch.py:295-305.
 *
 *   q    [B][Hq][D]       q[b*q_sb + h*q_sh + d]
 *   k, v [B][Hk][S][D]    k[b*k_sb + h*k_sh + s*k_ss + d]
 *   mask [B][S] uint8 (1 = attend) or NULL; kernels.py:53-55, patch.py:280-291
 *   held_len > 0 masks the first held_len rows of every (b,hk) with
 *     held_valid[b*hv_sb + hk*hv_sh + r] && held_pos[b*hp_sb + hk*hp_sh + r] <= *cur_pos
 *     (patch.py:288; cur_pos may be NULL = no position test).
 *   out  [B][Hq][D] in dtype: out[b*o_sb + h*o_sh + d]
 *   evict_loss / evict_idx (may be NULL): the per-token eviction score
 *     mean_h(mean_d|p v| / l) rounded to dtype, [B][S] float, and its
 *     first-index argmin [B] int64 (kernels.py:66-67, 134-136).
 *   num_splits <= 0 picks the launch shape (few short units are spread over
 *     many workgroups); with more than one split the partial results are
 *     merged inside the launch by the last workgroup of each (b, kv head) to
 *     finish (by a second kernel when the launch has more than 512
 *     workgroups or more than 2048 units).  The workspace must hold
 *     hc_decode_attn_workspace_size(B, Hq, Hk, D, S, num_splits, with_evict)
 *     bytes.  It needs no initialisation: its first 16384 bytes hold the
 *     merge's arrival words, counted under a tag of each launch's own, so
 *     whatever a workspace holds cannot trigger an early merge.  Words the
 *     workspace's previous launch left are counted on directly; others
 *     (a new workspace, one used by another caller in between) cost the
 *     launch's first arrivals one compare-and-swap each.  One workspace
 *     must not be used by two launches that may overlap.
 *   dropout must be 0.0.
 */
int64_t hc_decode_attn_workspace_size(int64_t B, int64_t Hq, int64_t Hk, int64_t D,
                                      int64_t S, int64_t num_splits, int with_evict);
int hc_decode_attn(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
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
                   void* stream);

/*
 * Append one token per (b, kv head) and attend, in one launch.  Replaces the
 * torch.cat append of cache.py:145-148 / layer_state.py:96-100 followed by
 * the decode attention of kernels.py:77-137 (call site patch.py:295-305).
 *
 *   k, v [B][Hk][S][D]: rows 0..S-2 are the cache; row S-1 receives the new
 *     token.  k_new / v_new [B][Hk][D] are the token's key and value,
 *     attended as key S-1 and written into row S-1 by the launch.
 *   p_new / p_dst (may both be NULL): the token's pre-RoPE key, written into
 *     row S-1 of p_dst [B][Hk][*][D] (cache.py:145-148 keeps pre-RoPE keys).
 *   pos_new [B] (stride posn_sb) / pos_dst [B][*] (may both be NULL): its
 *     absolute position, written at pos_dst[b][S-1].
 *   mask / held_* apply to the cached rows (held_len <= S-1) exactly as in
 *     hc_decode_attn; the new token is always attended.  No eviction score.
 *   The workspace is sized by hc_decode_attn_workspace_size(.., S, .., 0).
 */
int hc_decode_attn_append(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
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
                          void* stream);

/*
 * The pooled retrieval query on the device: the mean of the window's T query
 * tensors q[t] [B][Hq][D] (element strides q_sb[t], q_sh[t];
 * T <= hc_retrieval_query_max_rows()) over
 * the rows and over the heads -- of each KV head's group (per_head: out
 * [B][Hk][D]) or of all Hq heads (out [B][1][D]) -- in fp32, added in
 * window-then-head order.  Replaces the torch.cat + means of _pooled_query_np
 * / _q_to_vecs_np (controller.py:240-248, which pool in the cache dtype).
 * The result goes to dev_out; then, on the same stream, to host_out (pinned,
 * may be NULL) by hipMemcpyAsync, and `event` (may be NULL) is recorded
 * behind the copy, for a search thread to wait on.
 */
/* The largest window (T) hc_retrieval_query accepts: 64.  No counterpart in
 * the reference; callers pool longer windows themselves. */
int64_t hc_retrieval_query_max_rows(void);

int hc_retrieval_query(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t T, const void* const* q,
                       const int64_t* q_sb, const int64_t* q_sh, int per_head, float* dev_out, float* host_out,
                       void* event, void* stream);

/*
 * hc_decode_attn_append with its arguments in one struct: the same launch,
 * checks and results; a per-layer decode loop keeps one struct per hot
 * buffer and rewrites only the fields that change from step to step (q, the
 * token's rows, S, the held slot, out), which saves the host the marshalling
 * of 48 scalar arguments per call.  Replaces the same reference interface as
 * hc_decode_attn_append (kernels.py:77-137, call site patch.py:295-305).
 * Every field is 8 bytes wide (sizes, strides and the dtype code as int64,
 * pointers, scaling as double), so the layout has no padding;
 * hc_decode_append_args_size() returns sizeof for a binding to check.
 */
typedef struct hc_decode_append_args {
  int64_t dtype, B, Hq, Hk, D, S;
  const void* q; int64_t q_sb, q_sh;
  void* k; int64_t k_sb, k_sh, k_ss;
  void* v; int64_t v_sb, v_sh, v_ss;
  const void* k_new; int64_t kn_sb, kn_sh;
  const void* v_new; int64_t vn_sb, vn_sh;
  const void* p_new; int64_t pn_sb, pn_sh;
  void* p_dst; int64_t pd_sb, pd_sh, pd_ss;
  const int64_t* pos_new; int64_t posn_sb;
  int64_t* pos_dst; int64_t posd_sb;
  const uint8_t* mask; int64_t mask_sb;
  int64_t held_len;
  const int64_t* held_pos; int64_t hp_sb, hp_sh;
  const uint8_t* held_valid; int64_t hv_sb, hv_sh;
  const int64_t* cur_pos;
  double scaling;
  void* out; int64_t o_sb, o_sh;
  void* workspace; int64_t workspace_bytes, num_splits;
} hc_decode_append_args;

int hc_decode_attn_append_packed(const hc_decode_append_args* args, void* stream);
int64_t hc_decode_append_args_size(void);

/*
 * hc_decode_attn_append without a workspace: no counterpart in the reference.
 * It is for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The arguments and results
 * are hc_decode_attn_append's, minus (workspace, workspace_bytes); the split
 * partials and merge words live in a static 32 MiB device array that each
 * GPU holds until the process ends: four 8 MiB regions, one per stream.  The
 * array's address is taken once per device on the first call (the current
 * device must be the stream's device), and a stream's first call binds it a
 * free region for the rest of the process, so calls on different streams
 * never share partials.  A call from a fifth stream of one device returns
 * HC_ERR_INVALID; a call whose partials need more than 8 MiB returns
 * HC_ERR_WORKSPACE (fewer splits fit).  Nothing is allocated or freed.
 */
int hc_decode_attn_append_noalloc(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
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
                                  int64_t num_splits, void* stream);

/*
 * Decode attention that also accumulates H2O scores (layer_state.py:55-65,
 * 102-114): after attending (as hc_decode_attn, no mask), for every key s the
 * attention probability averaged over the G query heads of each KV head
 * (_reduce_probs_to_kv, scoring.py:29-37) is added to acc[b*a_sb + hk*a_sh + s]
 * (fp32).  Key S-1 is the token appended this step: its score starts from zero
 * (the zero column of layer_state.py:108-111).  The workspace is
 * hc_decode_attn_workspace_size(.., S, .., with_evict = 1).
 */
int hc_decode_attn_h2o(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
                       const void* q, int64_t q_sb, int64_t q_sh,
                       const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                       const void* v, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                       double scaling,
                       void* out, int64_t o_sb, int64_t o_sh,
                       float* acc, int64_t a_sb, int64_t a_sh,
                       void* workspace, int64_t workspace_bytes, int64_t num_splits, void* stream);

/*
 * H2O decode step with the re-eviction fused (layer_state.py:102-114 followed
 * by _compress, :68-79, when the append put the cache one row over budget).
 * Attends as hc_decode_attn_h2o, forms the updated scores
 * acc'[s] = acc[s] + (G-mean probability of key s) (key S-1 from zero), and
 * drops the one prefix row keep_index(acc', window, budget) (scoring.py:110-132)
 * leaves out: the lowest score, the highest index among equal scores.  The
 * S-1 surviving rows of K, V and acc', in their order, are written to
 * k_dst / v_dst ([B][Hk][>=S-1][D], dtype) and acc_dst ([B][Hk][>=S-1] fp32);
 * acc is not modified.  Equals hc_decode_attn_h2o + hc_topk_keep +
 * hc_gather_rows bit for bit.  Requires keep_index to drop exactly one row
 * (S - min(window, S) - max(0, min(budget - min(window, S), prefix)) == 1),
 * S <= 8192, destinations distinct from the sources, D * elem_bytes a
 * multiple of 16.  The workspace is that of hc_decode_attn_h2o.
 * With k_new / v_new ([B][Hk][D], 16-byte aligned rows) the step's token is
 * appended in the same launch, as hc_decode_attn_append does: it is attended
 * from k_new / v_new and written into row S-1 of k / v (which must then be
 * writable) before the eviction copies the rows; NULL means row S-1 already
 * holds it.  Both forms give the same bits.
 */
int hc_decode_attn_h2o_evict(int dtype, int64_t B, int64_t Hq, int64_t Hk, int64_t D, int64_t S,
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
                             void* workspace, int64_t workspace_bytes, int64_t num_splits, void* stream);

/*
 * hc_decode_attn_h2o_evict with its arguments in one struct: the same launch
 * and results (layer_state.py:102-114 then _compress, :68-79), for callers
 * that run it every decode step.  A caller fills the fields that stay fixed
 * (shape, the source and destination rows, the score buffers, window, budget,
 * workspace) once per pair of storages and rewrites only q, the token's rows,
 * S and out per step.  Every field is 8 bytes (int64 / pointer / double), so
 * the layout has no padding; hc_decode_h2o_evict_args_size() returns sizeof
 * for a binding to check.
 */
typedef struct hc_decode_h2o_evict_args {
  int64_t dtype, B, Hq, Hk, D, S;
  const void* q; int64_t q_sb, q_sh;
  const void* k; int64_t k_sb, k_sh, k_ss;
  const void* v; int64_t v_sb, v_sh, v_ss;
  const void* k_new; int64_t kn_sb, kn_sh;
  const void* v_new; int64_t vn_sb, vn_sh;
  double scaling;
  void* out; int64_t o_sb, o_sh;
  const float* acc; int64_t a_sb, a_sh;
  int64_t window, budget;
  void* k_dst; int64_t kd_sb, kd_sh, kd_ss;
  void* v_dst; int64_t vd_sb, vd_sh, vd_ss;
  float* acc_dst; int64_t ad_sb, ad_sh;
  void* workspace; int64_t workspace_bytes, num_splits;
} hc_decode_h2o_evict_args;

int hc_decode_attn_h2o_evict_packed(const hc_decode_h2o_evict_args* args, void* stream);
int64_t hc_decode_h2o_evict_args_size(void);

/*
 * Window importance scores per KV head, fp32 [B][Hk][S] (row stride S).
 * Replaces snapkv_importance (scoring.py:50-79) with _group_query_to_kv
 * (scoring.py:17-26) and pool1d (scoring.py:40-47) in HC_SCORE_SNAPKV mode,
 * and the scoring of HotColdLayer._compress_if_needed (cache.py:55-69) in
 * HC_SCORE_RAWSUM mode (pooling off; the head mean is hc_head_mean).
 *
 *   q [B][Hq][*][D]: the W window query rows are q rows q_row0 .. q_row0+W-1
 *     (q[b*q_sb + h*q_sh + (q_row0+w)*q_ss + d]); in SNAPKV mode window row w
 *     sits at absolute position S-W+w for the causal mask.
 *   k [B][Hk][S][D].
 *   kernel_size <= 1 disables pooling; otherwise it must be odd.
 * Scores are defined bit-for-bit (fp64 exact-product dot chains, integer
 * fixed-point softmax normaliser, fixed-order window sum, fp32 result) so the
 * selected indices are reproducible on any conforming implementation.
 */
int64_t hc_snapkv_score_workspace_size(int64_t B, int64_t Hk, int64_t S, int64_t D, int64_t W);
int hc_snapkv_score(int dtype, int mode, int64_t B, int64_t Hq, int64_t Hk, int64_t S,
                    int64_t D, int64_t W,
                    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_row0,
                    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                    double scaling, int64_t kernel_size, int pooling,
                    float* scores,
                    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * hc_snapkv_score over R rows whose queries and keys live in separate
 * allocations -- the layers of a model, compacted together once the prompt
 * has passed every layer (layer_state.py:82-94 runs once per layer; the kept
 * indices do not depend on when it runs).  Row r's queries start at
 * q_rows[r] and its keys at k_rows[r] (device arrays of R pointers, each
 * 16-byte aligned); the head and row strides are shared by all rows.  The
 * scores [R][Hk][S] and the workspace (hc_snapkv_score_workspace_size(R, ..))
 * are as in hc_snapkv_score with B = R, and so are the bits of every score.
 */
int hc_snapkv_score_rows(int dtype, int mode, int64_t R, int64_t Hq, int64_t Hk, int64_t S,
                         int64_t D, int64_t W,
                         const void* const* q_rows, int64_t q_sh, int64_t q_ss, int64_t q_row0,
                         const void* const* k_rows, int64_t k_sh, int64_t k_ss,
                         double scaling, int64_t kernel_size, int pooling,
                         float* scores,
                         void* workspace, int64_t workspace_bytes, void* stream);

/* Mean over KV heads of fp32 scores [B][H][S] -> [B][S] (cache.py:69 ".mean(dim=1)"). */
int hc_head_mean(int64_t B, int64_t H, int64_t S, const float* scores, float* out, void* stream);

/*
 * Kept-index selection: the keep_prefix highest-scoring prefix positions
 * (value descending, ties to the lower index), ascending, followed by the
 * recent window.  Replaces keep_index (scoring.py:110-132) and the top-k of
 * cache.py:47-76 (window = recent, budget = topk + recent).
 *   window_eff = min(window, S); prefix = S - window_eff;
 *   keep_prefix = max(0, min(budget - window_eff, prefix)); n_keep = keep_prefix + window_eff
 *   scores [B][H][S] fp32 (s[b*s_sb + h*s_sh + s]) -> keep [B][H][n_keep] int64
 *   evicted [B][H][prefix-keep_prefix] int64 (prefix positions not kept,
 *   ascending), or NULL (cache.py:86-95).
 */
int hc_topk_keep(int64_t B, int64_t H, int64_t S, const float* scores, int64_t s_sb, int64_t s_sh,
                 int64_t window, int64_t budget, int64_t* keep, int64_t* evicted, void* stream);

/*
 * hc_topk_keep with a caller-provided device workspace, for the same
 * replacement of keep_index (scoring.py:110-132) and the top-k of
 * cache.py:47-95.  Grids of fewer than 256 (batch, head) rows whose prefix
 * is longer than 32768 keys take a chunked selection that spreads each row
 * over workgroups of 8192 keys (a chain of launches on `stream`); the
 * outputs are those of hc_topk_keep, bit for bit.
 * hc_topk_keep_workspace_size returns the workspace the call needs (0: none, the
 * call runs hc_topk_keep).  ws == NULL also runs hc_topk_keep; a non-NULL ws
 * of fewer bytes than needed is HC_ERR_INVALID.  The workspace needs no
 * clearing and is in use until the stream reaches the end of the call.
 */
int64_t hc_topk_keep_workspace_size(int64_t B, int64_t H, int64_t S, int64_t window, int64_t budget);
int hc_topk_keep_ws(int64_t B, int64_t H, int64_t S, const float* scores, int64_t s_sb, int64_t s_sh,
                    int64_t window, int64_t budget, int64_t* keep, int64_t* evicted, void* ws, int64_t ws_bytes,
                    void* stream);

/*
 * Row gather into the hot buffer: dst_i[b][h][j] = src_i[b][h][idx[b][h][j]] for
 * j < n, for up to three tensors that share the index set (K, V, pre-RoPE K).
 * Replaces gather_kv (scoring.py:135-139), _compress (layer_state.py:76-77) and
 * the gathers of cache.py:79-84.  idx[b*i_sb + h*i_sh + j] (i_sh = 0 shares one
 * set across heads); an index outside [0, src_rows) leaves its destination row
 * untouched.  Rows are D elements of elem_bytes bytes; dst row j is written at
 * row dst_row0 + j.  src2/dst2 and src3/dst3 may be NULL.  pos_src [B][*] /
 * pos_dst [B][*] int64 positions (cache.py:84) may be NULL.
 */
int hc_gather_rows(int64_t B, int64_t H, int64_t n, int64_t D, int64_t elem_bytes,
                   const int64_t* idx, int64_t i_sb, int64_t i_sh, int64_t src_rows,
                   int64_t dst_row0,
                   const void* src1, int64_t s1_sb, int64_t s1_sh, int64_t s1_ss,
                   void* dst1, int64_t d1_sb, int64_t d1_sh, int64_t d1_ss,
                   const void* src2, int64_t s2_sb, int64_t s2_sh, int64_t s2_ss,
                   void* dst2, int64_t d2_sb, int64_t d2_sh, int64_t d2_ss,
                   const void* src3, int64_t s3_sb, int64_t s3_sh, int64_t s3_ss,
                   void* dst3, int64_t d3_sb, int64_t d3_sh, int64_t d3_ss,
                   const int64_t* pos_src, int64_t ps_sb, int64_t* pos_dst, int64_t pd_sb,
                   void* stream);

/*
 * hc_gather_rows of two tensors (K and V) over R rows that live in separate
 * allocations: row r of tensor t is read from src<t>_rows[r] and written to
 * dst<t>_rows[r] (device arrays of R pointers, each 16-byte aligned), with
 * the head and row strides shared by all rows.  It gathers the kept rows of
 * every layer of a model into each layer's own hot buffer in one launch
 * (gather_kv, scoring.py:135-139, run for all layers at once).
 */
int hc_gather_rows_tab(int64_t R, int64_t H, int64_t n, int64_t D, int64_t elem_bytes,
                       const int64_t* idx, int64_t i_sb, int64_t i_sh, int64_t src_rows,
                       int64_t dst_row0,
                       const void* const* src1_rows, int64_t s1_sh, int64_t s1_ss,
                       void* const* dst1_rows, int64_t d1_sh, int64_t d1_ss,
                       const void* const* src2_rows, int64_t s2_sh, int64_t s2_ss,
                       void* const* dst2_rows, int64_t d2_sh, int64_t d2_ss,
                       void* stream);

/*
 * Eviction gather with fp32 upcast (replaces the per-batch gather, .float()
 * and pinned copies of cache.py:86-125).  For the te evicted token indices
 * idx[b*i_sb + j] (one set shared by the heads) the pre-RoPE keys and values
 * [B][H][*][D] (dtype, element strides) and positions pos_src[b*ps_sb + i]
 * are written into one packed device block dev_out of
 * hc_gather_evict_bytes(B, H, te, D) bytes (16-byte aligned):
 *   [k fp32 B][H][te][D] | [v fp32 B][H][te][D] | [pos int64 B][te]
 * An index outside [0, src_rows) gives a zero row and position -1.  With
 * host_out (pinned, same size) the block is then copied to it by one
 * hipMemcpyAsync on the stream.  D % 4 == 0; K/V rows aligned to 4 elements.
 */
int64_t hc_gather_evict_bytes(int64_t B, int64_t H, int64_t te, int64_t D);
int hc_gather_evict(int dtype, int64_t B, int64_t H, int64_t te, int64_t D, const int64_t* idx, int64_t i_sb,
                    int64_t src_rows, const void* k_src, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                    const void* v_src, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                    const int64_t* pos_src, int64_t ps_sb, void* dev_out, void* host_out, void* stream);

/*
 * Append T new token rows at row `row` of the hot buffer (replaces the torch.cat
 * appends of cache.py:145-148 and layer_state.py:99-100).  src rows
 * [B][H][T][D]; k_pre/pos may be NULL.  pos_src [B][T] int64 -> pos_dst[b][row+t].
 */
int hc_append_rows(int dtype, int64_t B, int64_t H, int64_t T, int64_t D, int64_t row,
                   const void* k_src, int64_t ks_sb, int64_t ks_sh, int64_t ks_ss,
                   void* k_dst, int64_t kd_sb, int64_t kd_sh, int64_t kd_ss,
                   const void* v_src, int64_t vs_sb, int64_t vs_sh, int64_t vs_ss,
                   void* v_dst, int64_t vd_sb, int64_t vd_sh, int64_t vd_ss,
                   const void* p_src, int64_t ps_sb, int64_t ps_sh, int64_t ps_ss,
                   void* p_dst, int64_t pd_sb, int64_t pd_sh, int64_t pd_ss,
                   const int64_t* pos_src, int64_t pos_s_sb, int64_t* pos_dst, int64_t pos_d_sb,
                   void* stream);

/*
 * Inject: re-RoPE staged pre-RoPE keys to their original positions and write
 * them, with their values, into the held slot (rows 0..R-1) of the hot buffer.
 * Replaces _rotate_k_with_pos / _rope_cos_sin_for_positions (patch.py:76-102)
 * and the held-slot replacement of patch.py:241-270.
 *   k_pre, v: staged fp32 [B][Hk][R][D] (element strides kp_*, vp_*)
 *   pos [B][Hk?][R] int64 with strides (pos_sh = 0: one position set per batch)
 *   inv_freq fp32 [D/2] on the device; attention_scaling as in the rotary module.
 *   k_dst/v_dst rows r of [B][Hk][*][D] in dtype.
 * The rotation follows the model's per-op rounding in dtype:
 *   k*cos + rotate_half(k)*sin with cos/sin = dtype(fp32(cos(fp32(pos*inv_freq)))*scaling).
 */
int hc_inject_rerope(int dtype, int64_t B, int64_t Hk, int64_t R, int64_t D,
                     const float* k_pre, int64_t kp_sb, int64_t kp_sh, int64_t kp_ss,
                     const float* v, int64_t vp_sb, int64_t vp_sh, int64_t vp_ss,
                     const int64_t* pos, int64_t pos_sb, int64_t pos_sh,
                     const float* inv_freq, double attention_scaling,
                     void* k_dst, int64_t kd_sb, int64_t kd_sh, int64_t kd_ss,
                     void* v_dst, int64_t vd_sb, int64_t vd_sh, int64_t vd_ss,
                     void* stream);

/*
 * hc_inject_rerope with the rotary tables supplied: cos_t / sin_t hold
 * dtype(fp32(cos/sin(angle)) * scaling) -- what the model's rotary module
 * returns for the held positions (_rope_cos_sin_for_positions,
 * patch.py:76-91) -- for the first D/2 dims (the second half repeats them),
 * as [B][Hk or 1][R][D/2] in dtype with element strides (cs_sb, cs_sh, cs_ss);
 * cs_sh = 0 shares one table across the KV heads of a batch row.  With the
 * tables given, every written key is apply_rotary_pos_emb's bits
 * (patch.py:94-102).  The staged k_pre / v are kv_dtype: HC_DTYPE_F32, or the
 * cache dtype itself (the reference moves them to the model dtype before the
 * rotation, controller.py:368-369; the keys are rounded to it either way).
 * Staged rows aligned to 4 elements, D a multiple of 8.
 */
int hc_inject_rerope_tab(int dtype, int64_t B, int64_t Hk, int64_t R, int64_t D, int kv_dtype,
                         const void* k_pre, int64_t kp_sb, int64_t kp_sh, int64_t kp_ss,
                         const void* v, int64_t vp_sb, int64_t vp_sh, int64_t vp_ss,
                         const void* cos_t, const void* sin_t, int64_t cs_sb, int64_t cs_sh, int64_t cs_ss,
                         void* k_dst, int64_t kd_sb, int64_t kd_sh, int64_t kd_ss,
                         void* v_dst, int64_t vd_sb, int64_t vd_sh, int64_t vd_ss,
                         void* stream);

/*
 * Staging primitives for the inject feed (controller.py:344-442): a library
 * side stream created hipStreamNonBlocking at default priority, pinned
 * host->device copies on it, and events that the consumer polls (never waits
 * on) before ordering its stream after the copy.
 */
int hc_stream_create(void** stream_out);
int hc_stream_destroy(void* stream);
int hc_event_create(void** event_out, int timing);
int hc_event_destroy(void* event);
int hc_event_record(void* event, void* stream);
int hc_event_query(void* event);            /* 1 = complete, 0 = pending, <0 = error */
/* Block the calling host thread until the event completes (the retrieval
 * worker waits for its query vector; the decode thread never calls it). */
int hc_event_synchronize(void* event);
int hc_event_elapsed_ms(void* start, void* end, float* ms_out);
int hc_stream_wait_event(void* stream, void* event);
int hc_memcpy_h2d_async(void* dst, const void* src, int64_t bytes, void* stream);
int hc_memcpy_d2h_async(void* dst, const void* src, int64_t bytes, void* stream);

/*
 * Host cold store (host memory, host threads; no device calls).  One store
 * per (layer, batch row) replaces the reference's ring of token tensors plus
 * faiss.IndexFlatIP (controller.py:121-293):
 *   - hc_cold_add        add_evicted_to_cold_store (controller.py:199-238)
 *   - hc_cold_retrieve   one layer's retrieval over B stores (_retrieval_worker,
 *                        controller.py:250-293), run on host threads
 *   - hc_cold_search     index.search for one query (controller.py:274)
 *   - hc_cold_size       len(cpu_kpre_ring[l][b]) == index.ntotal
 *   - hc_cold_export     the ring in logical order (oldest first), for checks
 * Tokens hold fp32 pre-RoPE key and value [heads][head_dim], an int64
 * position, and vec_heads search vectors of vec_dim floats: the head mean
 * (vec_heads == 1) or each head's key (vec_heads == heads), padded/cropped to
 * vec_dim and divided by max(||x||, 1e-12) (normalize != 0), accumulated in
 * fp64 in index order.  Inner products accumulate in fp64 in dimension order;
 * ranking is descending, ties to the older token.  A full store overwrites its
 * oldest token; an add larger than the store keeps its last tokens.  Adds
 * exclude searches; searches run concurrently.  Returns 0 / HC_ERR_INVALID.
 */
void* hc_cold_create(int64_t capacity, int64_t heads, int64_t head_dim, int64_t vec_dim, int64_t vec_heads,
                     int normalize);
/* Frees a store, first waiting for any submitted job (search or add) that
 * uses it. */
void hc_cold_destroy(void* store);
/* Tokens held, after every add submitted to the store so far. */
int64_t hc_cold_size(const void* store);
/* Tokens t < te with evicted_idx[t] >= 0 (evicted_idx may be NULL: all), from
 * kpre/v [heads][te][head_dim] with element strides (k_sh, k_st), (v_sh, v_st)
 * and pos[te] -- one batch row of EvictedKV (datatypes.py:58-63). */
int hc_cold_add(void* store, int64_t te, const float* kpre, int64_t k_sh, int64_t k_st,
                const float* v, int64_t v_sh, int64_t v_st, const int64_t* pos, const int64_t* evicted_idx);
/* hc_cold_add as a job on the library's worker threads (the reference adds
 * the evicted tokens to its index inline, controller.py:178-188): the
 * prefill's eviction returns while the store is filled.  Adds to one store are
 * applied in submission order; a synchronous call on the store (add, size,
 * search, export, retrieve) first waits for the adds submitted before it, and
 * a search job waits for the adds submitted before the search was.  The
 * worker first synchronises on wait_event (may be NULL).  nthreads <= 0 picks
 * min(cores, 16) for the copy.  The caller keeps kpre, v, pos and evicted_idx
 * alive until the job is done (hc_cold_job_poll / hc_cold_job_free, as for a
 * search job).  Returns the job, or NULL on a bad argument (hc_last_error). */
void* hc_cold_add_async(void* store, int64_t te, const float* kpre, int64_t k_sh, int64_t k_st,
                        const float* v, int64_t v_sh, int64_t v_st, const int64_t* pos, const int64_t* evicted_idx,
                        void* wait_event, int64_t nthreads, int64_t workers);
/* defer != 0: later adds store keys, values and positions but not the
 * search vectors (the caller ranks elsewhere, e.g. a device search index);
 * the next host search, retrieval or vector export computes every live
 * token's vectors first and ends the deferral, so results never change.
 * defer = 0: compute them now and stop deferring.  Waits for earlier adds. */
int hc_cold_defer_vectors(void* store, int defer);
/* Top-r logical indices for query q [vec_dim] against search vector `head`;
 * *n_out = min(r, size). */
int hc_cold_search(const void* store, const float* q, int64_t r, int64_t head, int64_t* out, int64_t* n_out);
/* Logical-order copies: kpre/v [size][heads][head_dim], pos [size],
 * vec [size][vec_heads][vec_dim]; any pointer may be NULL. */
int hc_cold_export(const void* store, float* kpre, float* v, int64_t* pos, float* vec);
/* Retrieval of R tokens per batch row (per_head = 0: query q[b] of store b's
 * head-mean vectors; outputs pos/valid [B][R]) or per (batch row, head)
 * (per_head = 1: q[b][h]; pos/valid [B][heads][R]).  kpre/v out are
 * [B][heads][R][head_dim] of kv_dtype (HC_DTYPE_F32, or HC_DTYPE_F16 /
 * HC_DTYPE_BF16: the stored fp32 values rounded to nearest even, as the
 * reference's kpre_cpu.to(device, dtype) rounds them, controller.py:368-369);
 * rows past the hits are zero with valid = 0.  q has
 * q_dim floats per query, element strides (q_sb, q_sh); it is cropped or
 * zero-padded to vec_dim and, with normalize_q, divided by max(||q||, 1e-12)
 * as the stored vectors are (squares summed in fp64 in dimension order,
 * quotient rounded to fp32).  tab (may be NULL): a table of tab_rows rows of
 * tab_row_bytes bytes indexed by position; the row of every retrieved
 * position (position 0 past the hits) is copied to tab_out, laid out like
 * pos_out, and *tab_missing (may be NULL) counts positions beyond the table
 * (their rows are zero).  This carries the rotary tables of the retrieved
 * positions (controller.py:365-373 re-rotates them).  nthreads <= 0 picks
 * min(cores, 16). */
int hc_cold_retrieve(void* const* stores, int64_t B, const float* q, int64_t q_sb, int64_t q_sh, int64_t q_dim,
                     int normalize_q, int64_t R, int per_head, int kv_dtype, void* kpre_out, void* v_out,
                     int64_t* pos_out, uint8_t* valid_out, const uint8_t* tab, int64_t tab_rows,
                     int64_t tab_row_bytes, uint8_t* tab_out, int64_t* tab_missing, int64_t nthreads);
/* hc_cold_retrieve as a job on the library's own worker threads, in place of
 * the reference's threading.Thread per search (controller.py:336-342).  Up to
 * `workers` threads (at most 16) are started on first use and kept until the
 * process ends.  The worker first synchronises on wait_event (may be NULL),
 * the event behind the pooled query's copy, then runs the retrieval and
 * counts the valid rows.  The caller keeps every buffer alive until the job
 * is done.  Returns the job, or NULL on a bad argument (hc_last_error). */
void* hc_cold_retrieve_async(void* const* stores, int64_t B, const float* q, int64_t q_sb, int64_t q_sh,
                             int64_t q_dim, int normalize_q, int64_t R, int per_head, int kv_dtype, void* kpre_out,
                             void* v_out, int64_t* pos_out, uint8_t* valid_out, const uint8_t* tab,
                             int64_t tab_rows, int64_t tab_row_bytes, uint8_t* tab_out, int64_t nthreads,
                             void* wait_event, int64_t workers);
/* The rows of hits found by the device search index (hc_index_search): hits
 * [B][VH][R] (host) holds logical indices of each row's store in rank order,
 * -1 past the hits.  Writes the outputs as hc_cold_retrieve does for the same
 * hits (kpre/v, pos/valid, table rows), after the adds submitted before it.
 * A hit beyond its store's tokens is HC_ERR_INVALID. */
int hc_cold_gather(void* const* stores, int64_t B, int per_head, int64_t R, const int64_t* hits, int kv_dtype,
                   void* kpre_out, void* v_out, int64_t* pos_out, uint8_t* valid_out, const uint8_t* tab,
                   int64_t tab_rows, int64_t tab_row_bytes, uint8_t* tab_out, int64_t* tab_missing,
                   int64_t nthreads);
/* hc_cold_gather as a job on the worker threads: the worker first waits for
 * wait_event (the event behind the search that wrote the hits) and for the
 * adds submitted before the job.  Polled and freed like a search job. */
void* hc_cold_gather_async(void* const* stores, int64_t B, int per_head, int64_t R, const int64_t* hits,
                           int kv_dtype, void* kpre_out, void* v_out, int64_t* pos_out, uint8_t* valid_out,
                           const uint8_t* tab, int64_t tab_rows, int64_t tab_row_bytes, uint8_t* tab_out,
                           int64_t nthreads, void* wait_event, int64_t workers);
/* 0 while the job runs (wait = 0); 1 when it is done, with the number of
 * valid rows and of positions past the table (0 for an add); a negative
 * HC_ERR_* code if the job failed (its message in hc_last_error on the
 * calling thread).
 * wait != 0 blocks until the job is done. */
int hc_cold_job_poll(void* job, int wait, int64_t* n_valid, int64_t* tab_missing);
/* Frees a job, first waiting for it if a worker still runs it. */
void hc_cold_job_free(void* job);

/*
 * Device search index of the cold stores of one layer: the search vectors of
 * B stores kept in HBM as vec [B][VH][capT/64][VD/4][64][4] fp32 (tiles of 64
 * slots, VD a multiple of 4; capT >= the stores' capacity, a multiple of 64),
 * with the same
 * arithmetic as hc_cold_add / hc_cold_search, so the
 * hits are the host store's, bit for bit.  It replaces the reference's CPU
 * faiss.IndexFlatIP scan (controller.py:223-232, 274-293) where a host scan
 * cannot keep up (a layer of 16 rows x 8 heads x 30 720 tokens is 2 GB of
 * vectors).  The key/value rows stay in the host store.
 *
 * hc_index_add: the vectors of tokens t < te of kpre (fp32 on the device; row
 * b, head h, token t at kpre[b*k_sb + h*k_sh + t*k_st], head_dim D elements)
 * into the physical slots slot_of[b][t] (int32 on the device; < 0: not
 * stored), as hc_cold_add would place them: the head mean (VH = 1) or each
 * head (VH = H), cropped or zero-padded to VD, normalised when normalize.
 * vec16 (may be NULL; VD a multiple of 8): the same vectors rounded to fp16,
 * [B][VH][capT/64][VD/8][64][8], for the search's fp16 pass.
 */
int hc_index_add(int64_t B, int64_t H, int64_t D, int64_t VH, int64_t VD, int normalize,
                 const float* kpre, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t te,
                 const int32_t* slot_of, float* vec, void* vec16, int64_t capT, void* stream);
/*
 * hc_index_search: for every row b < B (B <= 64) and head h < VH, the query
 * q[b*q_sb + h*q_sh .. + q_dim) (fp32 on the device; cropped or zero-padded to
 * VD <= 1024 and, with normalize_q, normalised as hc_cold_retrieve does) against
 * the row's sizes[b] stored vectors (ring of capacity cap whose oldest token is
 * in slot heads[b] once full; sizes and heads are host arrays).  Writes the
 * top R <= 1024 logical indices (oldest token = 0) in rank order -- inner
 * product descending, ties to the older token -- to hits [B][VH][R] (int64 on
 * the device), -1 past min(R, size).  keys: device scratch of B*VH*capT
 * uint64.  With vec16 and keys32 (B*VH*capT uint32 scratch) given, unit
 * vectors (vec_normalized) and a normalised query, the search first scores
 * the fp16 copy in fp32, then scores exactly only the slots within twice the
 * bound of the two scores' difference of that pass's R-th score (a superset
 * of the exact top R, ties included): the same hits, about half the bytes.  On `stream`, optionally (NULL skips each): first wait for
 * wait_event (the query's producer); write the hits to hits_host as well
 * (pinned host memory, B*VH*R int64, written by the kernel through its device
 * mapping, so they are on the host once the kernel is done; anything else is
 * HC_ERR_INVALID); record done_event behind the kernels.
 */
int hc_index_search(int64_t B, int64_t VH, int64_t VD, int64_t cap, const float* q, int64_t q_sb, int64_t q_sh,
                    int64_t q_dim, int normalize_q, const float* vec, const void* vec16, int vec_normalized,
                    int64_t capT, const int64_t* sizes, const int64_t* heads, int64_t R, uint64_t* keys,
                    uint32_t* keys32, int64_t* hits, int64_t* hits_host, void* wait_event, void* done_event,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HOTCOLD_HIP_H */
