"""CPU restatement of the reference hot-tier algorithms -- TEST INFRASTRUCTURE.

Used only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
as the checker (never as the product path).  Every function cites the
reference file:line it follows (tarun931/hotcold-kv-cache, src/hotcold_kv/...).

Parity pins (what checks each function; see tests/test_oracle.py):
  window_scores (C, bit-defined contract)   -- fp64 closed-form softmax, the
      literal fp32 torch restatement below, brute force on tiny shapes, golden
      fixtures, exp_det vs libm
  snapkv_importance_torch (literal fp32)    -- fp64 closed form
  keep_index                                -- brute force over all subsets on
      tiny S, test_baselines.py:89-100 invariants, hand-made tie cases
  gather_kv                                 -- identity / permutation checks
  decode_attention                          -- closed forms (single key, equal
      keys), torch SDPA fp32
  evict_scores                              -- closed form on a hand-made case
  rerope                                    -- HF apply_rotary_pos_emb on CPU;
      orthogonality (norm) and rot(p) then rot(-p) = identity in fp64
  hotcold_compress                          -- cache.py invariants (kept count,
      recent window, evicted = complement)
  ColdStore                                 -- test_cold_store.py self-retrieval
      and ring-wrap cases
"""

import ctypes
import math
import os
import subprocess
import threading

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libhc_oracle.so")
_lib = None
_lib_lock = threading.Lock()


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _clib():
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:                     # tests call the oracle from several threads
        if _lib is not None:
            return _lib
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        i64, vp, dbl = ctypes.c_int64, ctypes.c_void_p, ctypes.c_double
        lib.hco_exp_det.restype = dbl
        lib.hco_exp_det.argtypes = [dbl]
        lib.hco_window_scores.restype = ctypes.c_int
        lib.hco_window_scores.argtypes = [ctypes.c_int, i64, i64, i64, i64, i64, i64,
                                          vp, i64, i64, i64, i64,
                                          vp, i64, i64, i64, dbl, i64, ctypes.c_int, vp]
        lib.hco_head_mean.restype = None
        lib.hco_head_mean.argtypes = [i64, i64, i64, vp, vp]
        _lib = lib
    return _lib


def exp_det(x):
    return _clib().hco_exp_det(float(x))


def _f64(t):
    """Exact fp64 numpy copy of a CPU/GPU tensor of any float dtype."""
    return np.ascontiguousarray(t.detach().to("cpu", torch.float64).numpy())


# ---------------------------------------------------------------------------
# Window scores: the bit-defined contract (C)
# ---------------------------------------------------------------------------
def window_scores(q, k, window, scaling, kernel_size=7, pooling="maxpool", mode="snapkv", q_is_window=False):
    """Importance (B,Hk,S) float32 under the bit-defined contract.

    mode "snapkv" follows snapkv_importance (scoring.py:50-79): window rows are
    the last min(window,S) rows of q (T == S; with q_is_window, q holds only
    those rows).  mode "rawsum" follows cache.py:55-69 before the head mean:
    the last min(window,T) rows of q, no mask, no softmax, no pooling.
    """
    qn, kn = _f64(q), _f64(k)
    B, Hq, T, D = qn.shape
    _, Hk, S, _ = kn.shape
    if mode == "snapkv":
        W = min(int(window), S)
        q_row0 = S - W
        if q_is_window:
            if T != W:
                raise ValueError("q_is_window: q must hold exactly the last min(window, S) rows")
            q_row0 = 0
        m = 0
    else:
        W = min(int(window), T)
        q_row0 = T - W
        m = 1
        kernel_size = 1
    out = np.empty((B, Hk, S), dtype=np.float32)
    rc = _clib().hco_window_scores(
        m, B, Hq, Hk, S, D, W,
        qn.ctypes.data, Hq * T * D, T * D, D, q_row0,
        kn.ctypes.data, Hk * S * D, S * D, D,
        float(scaling), int(kernel_size or 1), 1 if pooling == "avgpool" else 0,
        out.ctypes.data)
    if rc != 0:
        raise ValueError("hco_window_scores: bad arguments")
    return torch.from_numpy(out)


def head_mean(x):
    xn = np.ascontiguousarray(x.detach().cpu().float().numpy())
    B, H, S = xn.shape
    out = np.empty((B, S), dtype=np.float32)
    _clib().hco_head_mean(B, H, S, xn.ctypes.data, out.ctypes.data)
    return torch.from_numpy(out)


# ---------------------------------------------------------------------------
# H2O (scoring.py:82-107, layer_state.py:55-65, 102-114)
# ---------------------------------------------------------------------------
def h2o_prefill_scores(q, k, scaling):
    """H2O prefill scores (B,Hk,S) float32 under the bit-defined contract: the
    window score of every query head with the window covering the whole
    prompt (causal rows 0..S-1, exact-sum softmax, fp64 row sum, no pooling)
    against its own KV head's keys, then the head mean over each group."""
    B, Hq, S, D = q.shape
    Hk = k.shape[1]
    G = Hq // Hk
    per_q = window_scores(q, repeat_kv(k, G), S, scaling, 1, "maxpool")        # (B,Hq,S)
    return head_mean(per_q.reshape(B * Hk, G, S)).reshape(B, Hk, S)


def h2o_prefill_scores_f64(q, k, scaling):
    """The same quantity in plain fp64 (closed form, no rounding contract)."""
    qd, kd = q.double(), k.double()
    B, Hq, S, D = qd.shape
    G = Hq // k.shape[1]
    logits = torch.matmul(qd, repeat_kv(kd, G).transpose(2, 3)) * scaling
    causal = torch.ones(S, S, dtype=torch.bool).triu(1)
    probs = torch.softmax(logits.masked_fill(causal, float("-inf")), dim=-1)
    acc = probs.sum(dim=2)                                                    # (B,Hq,S)
    return acc.view(B, Hq // G, G, S).mean(dim=2)


def h2o_decode_probs(q, k, scaling):
    """Attention probabilities of one query token (B,Hq,1,D) over k (B,Hk,S,D),
    fp64, averaged over the query heads of each KV head -> (B,Hk,S)
    (_attn_with_probs + _reduce_probs_to_kv, layer_state.py:55-65,
    scoring.py:29-37)."""
    qd, kd = q.double(), k.double()
    B, Hq = qd.shape[:2]
    G = Hq // kd.shape[1]
    logits = torch.matmul(qd, repeat_kv(kd, G).transpose(2, 3)) * scaling     # (B,Hq,1,S)
    probs = torch.softmax(logits, dim=-1)[:, :, 0]
    return probs.view(B, Hq // G, G, -1).mean(dim=2)


# ---------------------------------------------------------------------------
# Literal fp32 restatements of the reference scoring (scoring.py)
# ---------------------------------------------------------------------------
def repeat_kv(x, n_rep):
    """scoring.py:9-14."""
    if n_rep == 1:
        return x
    B, Hk, S, D = x.shape
    return x[:, :, None].expand(B, Hk, n_rep, S, D).reshape(B, Hk * n_rep, S, D)


def group_query_to_kv(q, Hk):
    """scoring.py:17-26: mean of each GQA group (or of all heads)."""
    B, Hq, T, D = q.shape
    if Hq == Hk:
        return q
    if Hq % Hk == 0:
        return q.view(B, Hk, Hq // Hk, T, D).mean(dim=2)
    return q.mean(dim=1, keepdim=True).expand(B, Hk, T, D)


def pool1d(x, kernel_size, pooling):
    """scoring.py:40-47."""
    if kernel_size is None or kernel_size <= 1:
        return x
    pad = kernel_size // 2
    if pooling == "avgpool":
        return torch.nn.functional.avg_pool1d(x, kernel_size=kernel_size, stride=1, padding=pad)
    return torch.nn.functional.max_pool1d(x, kernel_size=kernel_size, stride=1, padding=pad)


def snapkv_importance_torch(q_post, keys, window_size, scaling, kernel_size, pooling, dtype=torch.float32,
                            q_is_window=False):
    """scoring.py:50-79 on CPU with inputs upcast to `dtype` (the reference's
    own op sequence: GQA mean, matmul, causal masked_fill, fp32 softmax, sum
    over the window, pooling).  q_is_window: q_post holds only the last
    min(window, S) query rows."""
    q_post = q_post.detach().cpu().to(dtype)
    keys = keys.detach().cpu().to(dtype)
    B, Hq, _, D = q_post.shape
    S = keys.shape[2]
    Hk = keys.shape[1]
    W = min(window_size, S)
    q_for = group_query_to_kv(q_post if q_is_window else q_post[:, :, S - W:, :], Hk)
    logits = torch.matmul(q_for, keys.transpose(2, 3)) * scaling
    qpos = torch.arange(S - W, S).view(1, 1, W, 1)
    kpos = torch.arange(S).view(1, 1, 1, S)
    logits = logits.masked_fill(kpos > qpos, float("-inf"))
    probs = torch.softmax(logits.float(), dim=-1)
    imp = probs.sum(dim=2)
    return pool1d(imp, kernel_size, pooling)


def snapkv_importance_f64(q_post, keys, window_size, scaling, kernel_size, pooling):
    """Closed-form fp64 version of scoring.py:50-79 (numpy)."""
    qn, kn = _f64(q_post), _f64(keys)
    B, Hq, S, D = qn.shape
    Hk = kn.shape[1]
    W = min(window_size, S)
    qt = qn[:, :, S - W:, :]
    if Hq % Hk == 0:
        qf = qt.reshape(B, Hk, Hq // Hk, W, D).mean(axis=2)
    else:
        qf = np.broadcast_to(qt.mean(axis=1, keepdims=True), (B, Hk, W, D))
    logits = np.einsum("bhwd,bhsd->bhws", qf, kn) * scaling
    qpos = np.arange(S - W, S).reshape(1, 1, W, 1)
    kpos = np.arange(S).reshape(1, 1, 1, S)
    logits = np.where(kpos > qpos, -np.inf, logits)
    m = logits.max(axis=-1, keepdims=True)
    e = np.exp(logits - m)
    probs = e / e.sum(axis=-1, keepdims=True)
    imp = probs.sum(axis=2)
    if kernel_size and kernel_size > 1:
        P = kernel_size // 2
        padv = -np.inf if pooling != "avgpool" else 0.0
        padded = np.pad(imp, ((0, 0), (0, 0), (P, P)), constant_values=padv)
        win = np.lib.stride_tricks.sliding_window_view(padded, kernel_size, axis=-1)
        imp = win.max(axis=-1) if pooling != "avgpool" else win.sum(axis=-1) / kernel_size
    return imp


# ---------------------------------------------------------------------------
# Selection and gather (scoring.py:110-139)
# ---------------------------------------------------------------------------
def keep_counts(S, window_size, budget):
    """scoring.py:118-120."""
    window = min(window_size, S)
    prefix = S - window
    keep_prefix = max(0, min(budget - window, prefix))
    return window, prefix, keep_prefix


def keep_index(scores, window_size, budget, return_evicted=False):
    """scoring.py:110-132 with the deterministic tie rule: the keep_prefix
    prefix positions of highest score, ties to the lower index (a stable sort
    on -score), sorted ascending, then arange(prefix, S).  NaN ranks above
    every number, +inf included, as in torch.topk; NaNs tie with each other,
    and -0 with +0."""
    sc = scores.detach().cpu().float().numpy()
    squeeze = sc.ndim == 2
    if squeeze:
        sc = sc[:, None, :]
    B, H, S = sc.shape
    window, prefix, kp = keep_counts(S, window_size, budget)
    keep = np.empty((B, H, kp + window), dtype=np.int64)
    ev = np.empty((B, H, prefix - kp), dtype=np.int64)
    recent = np.arange(prefix, S, dtype=np.int64)
    for b in range(B):
        for h in range(H):
            pre = sc[b, h, :prefix].astype(np.float64)
            nan = np.isnan(pre)
            # stable: NaN first, then descending value (lexsort's last key is the primary)
            order = np.lexsort((np.where(nan, 0.0, -pre), ~nan))
            top = np.sort(order[:kp])
            keep[b, h, :kp] = top
            keep[b, h, kp:] = recent
            mask = np.ones(prefix, dtype=bool)
            mask[top] = False
            ev[b, h] = np.nonzero(mask)[0]
    keep_t = torch.from_numpy(keep)
    ev_t = torch.from_numpy(ev)
    if squeeze:
        keep_t, ev_t = keep_t[:, 0], ev_t[:, 0]
    return (keep_t, ev_t) if return_evicted else keep_t


def gather_kv(t, keep):
    """scoring.py:135-139."""
    t = t.detach().cpu()
    keep = keep.detach().cpu()
    if keep.dim() == 2:
        keep = keep.unsqueeze(1).expand(t.shape[0], t.shape[1], keep.shape[-1])
    B, H, S, D = t.shape
    return t.gather(2, keep.unsqueeze(-1).expand(B, H, keep.shape[-1], D))


# ---------------------------------------------------------------------------
# Decode attention (kernels.py:9-137, patch.py:280-305)
# ---------------------------------------------------------------------------
def decode_attention(q, k, v, scaling, mask=None):
    """softmax(q.K^T * scaling, masked) . V per query head in fp64, with the GQA
    map kv = h // (Hq/Hk) (kernels.py:35).  q (B,Hq,D) or (B,Hq,1,D); returns
    (B,Hq,D) float64 numpy.  Rows with every key masked give NaN, as the
    reference's 0/0 does."""
    qn = _f64(q)
    if qn.ndim == 4:
        qn = qn[:, :, 0, :]
    kn, vn = _f64(k), _f64(v)
    B, Hq, D = qn.shape
    Hk = kn.shape[1]
    G = Hq // Hk
    kr = np.repeat(kn, G, axis=1)
    vr = np.repeat(vn, G, axis=1)
    s = np.einsum("bhd,bhsd->bhs", qn, kr) * scaling
    if mask is not None:
        mk = mask.detach().cpu().numpy().astype(bool)
        s = np.where(mk[:, None, :], s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    with np.errstate(invalid="ignore", divide="ignore"):
        e = np.where(np.isfinite(m), np.exp(s - m), 0.0)
        out = np.einsum("bhs,bhsd->bhd", e, vr) / e.sum(axis=-1)[..., None]
    return out


def evict_scores(q, k, v, scaling, mask=None):
    """Eviction score of kernels.py:66-67 and 134-136 in fp64:
    final_loss[b,s] = mean_h( p[b,h,s]/l[b,h] * mean_d|v[b,kv(h),s,d]| ).
    Returns (final_loss (B,S) float64, argmin (B,) over the loss rounded to
    q's dtype, first index on ties)."""
    qn = _f64(q)
    if qn.ndim == 4:
        qn = qn[:, :, 0, :]
    kn, vn = _f64(k), _f64(v)
    B, Hq, D = qn.shape
    Hk = kn.shape[1]
    G = Hq // Hk
    s = np.einsum("bhd,bhsd->bhs", qn, np.repeat(kn, G, axis=1)) * scaling
    if mask is not None:
        mk = mask.detach().cpu().numpy().astype(bool)
        s = np.where(mk[:, None, :], s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    p = p / p.sum(axis=-1, keepdims=True)
    av = np.abs(np.repeat(vn, G, axis=1)).mean(axis=-1)
    loss = (p * av).mean(axis=1)
    rounded = torch.from_numpy(loss).to(q.dtype).float().numpy()
    return loss, np.argmin(rounded, axis=-1)


# ---------------------------------------------------------------------------
# Re-RoPE (patch.py:76-102; transformers LlamaRotaryEmbedding.forward and
# apply_rotary_pos_emb of the installed modeling_llama.py)
# ---------------------------------------------------------------------------
def default_inv_freq(head_dim, theta):
    """compute_default_rope_parameters: 1 / theta^(arange(0, D, 2) / D), fp32."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))


def rotary_cos_sin(inv_freq, attention_scaling, pos, dtype):
    """LlamaRotaryEmbedding.forward on CPU: cos/sin (B,S,D) in `dtype`."""
    pos = pos.detach().cpu().long()
    if pos.dim() == 1:
        pos = pos.unsqueeze(0)
    inv = inv_freq.detach().cpu().float()
    inv_exp = inv[None, :, None].expand(pos.shape[0], -1, 1)
    freqs = (inv_exp @ pos[:, None, :].float()).transpose(1, 2)
    emb = torch.cat((freqs, freqs), dim=-1)
    cos = emb.cos() * attention_scaling
    sin = emb.sin() * attention_scaling
    return cos.to(dtype), sin.to(dtype)


def rotate_half(x):
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def rerope(k_pre, pos, inv_freq, attention_scaling, dtype):
    """_rotate_k_with_pos (patch.py:94-102): staged k_pre (B,Hk,R,D) fp32 cast
    to the cache dtype (controller.py:365-373), rotated to positions pos (B,R)
    (one set per batch) or (B,Hk,R) (one per KV head) with the model's per-op
    rounding k*cos + rotate_half(k)*sin."""
    k16 = k_pre.detach().cpu().to(dtype)
    B, Hk, R, D = k16.shape
    pos = pos.detach().cpu().long()
    if pos.dim() == 2:
        cos, sin = rotary_cos_sin(inv_freq, attention_scaling, pos, dtype)   # (B,R,D)
        cos, sin = cos[:, None], sin[:, None]
    else:
        cos, sin = rotary_cos_sin(inv_freq, attention_scaling, pos.reshape(B * Hk, R), dtype)
        cos, sin = cos.view(B, Hk, R, D), sin.view(B, Hk, R, D)
    return (k16 * cos) + (rotate_half(k16) * sin)


# ---------------------------------------------------------------------------
# Hot/cold compression (cache.py:37-128)
# ---------------------------------------------------------------------------
def hotcold_compress(keys, values, pre_keys, positions, q_last, max_capacity, recent_size, topk_ratio):
    """HotColdLayer._compress_if_needed with contract scoring.  Returns None if
    no compression happens, else dict(keep (B,n), keys, values, pre_keys,
    positions, evicted_idx (B,Te) ascending)."""
    B, Hk, S, D = keys.shape
    if S <= max_capacity:
        return None
    recent = min(recent_size, max_capacity, S)
    prefix = S - recent
    if prefix <= 0:
        return None
    topk = max(1, min(int(max_capacity * topk_ratio), prefix))
    tq = min(recent, q_last.shape[2])
    per_head = window_scores(q_last, keys, tq, 1.0, kernel_size=1, mode="rawsum")
    scores = head_mean(per_head)                       # (B,S)
    keep, ev = keep_index(scores, recent, topk + recent, return_evicted=True)
    return dict(keep=keep, evicted_idx=ev,
                keys=gather_kv(keys, keep), values=gather_kv(values, keep),
                pre_keys=gather_kv(pre_keys, keep),
                positions=positions.detach().cpu().gather(1, keep))


# ---------------------------------------------------------------------------
# Cold store (controller.py:166-293), exact inner-product search
# ---------------------------------------------------------------------------
class ColdStore:
    """Ring of evicted tokens of one (layer, batch row) with exact inner-product
    search (controller.py:166-188, 190-238, 250-293; the reference indexes the
    vectors in a faiss.IndexFlatIP, whose last-bit arithmetic and tie order are
    not pinned).  The contract the native store follows:
      vector  head mean of the pre-RoPE key (or each head's key with
              per_head=True), fp64 accumulated in head order, padded/cropped
              to `dim`, divided by max(norm, 1e-12) with the norm's squares
              accumulated in dimension order; rounded to fp32
      search  inner product of the fp32 vector and fp32 query, fp64,
              accumulated in dimension order; larger first, ties to the older
              token; a full ring drops its oldest token."""

    def __init__(self, capacity, dim, normalize=True, per_head=False):
        self.capacity, self.dim, self.normalize, self.per_head = capacity, dim, normalize, per_head
        self.kpre, self.v, self.pos, self.vec = [], [], [], []

    def token_vecs(self, kp):
        """(H,D) fp32 pre-RoPE key -> (vec_heads, dim) fp32 search vectors."""
        kp = np.asarray(kp, dtype=np.float32)
        H = kp.shape[0]
        if self.per_head:
            rows = [kp[h].astype(np.float64) for h in range(H)]
        else:
            acc = np.zeros(kp.shape[1], dtype=np.float64)
            for h in range(H):
                acc = acc + kp[h].astype(np.float64)
            rows = [acc / float(H)]
        out = []
        for x in rows:
            if x.shape[0] > self.dim:
                x = x[: self.dim]
            elif x.shape[0] < self.dim:
                x = np.concatenate([x, np.zeros(self.dim - x.shape[0])])
            den = 1.0
            if self.normalize:
                ss = 0.0
                for t in x.tolist():
                    ss += t * t
                den = max(math.sqrt(ss), 1e-12)
            out.append((x / den).astype(np.float32))
        return np.stack(out)

    def add(self, kpre_tokens, v_tokens, positions, evicted_idx=None):
        """Tokens (n,H,D); those with evicted_idx < 0 are padding and skipped."""
        for t, (kp, vv, p) in enumerate(zip(kpre_tokens, v_tokens, positions)):
            if evicted_idx is not None and int(evicted_idx[t]) < 0:
                continue
            self.kpre.append(np.asarray(kp, dtype=np.float32))
            self.v.append(np.asarray(vv, dtype=np.float32))
            self.pos.append(int(p))
            self.vec.append(self.token_vecs(kp))
        over = len(self.kpre) - self.capacity
        if over > 0:
            del self.kpre[:over], self.v[:over], self.pos[:over], self.vec[:over]

    def inner_products(self, q_vec, head=0):
        n = len(self.kpre)
        keys = np.stack([v[head] for v in self.vec]).astype(np.float64) if n else np.zeros((0, self.dim))
        q = np.asarray(q_vec, dtype=np.float32).astype(np.float64)
        ip = np.zeros(n)
        for d in range(self.dim):
            ip = ip + keys[:, d] * q[d]
        return ip

    def search(self, q_vec, r, head=0):
        n = len(self.kpre)
        if n == 0 or r <= 0:
            return []
        ip = self.inner_products(q_vec, head)
        order = np.argsort(-ip, kind="stable")[: min(r, n)]
        return [int(i) for i in order]


def cold_topk(kpre, q_vec, r, head=0, per_head=False, dim=None, normalize=True):
    """ColdStore's search over a whole store at once: kpre (n,H,D) fp32 in
    logical order (oldest first), q_vec (dim,) fp32 -> logical indices of the
    top-r inner products (controller.py:190-238, 250-293 under ColdStore's
    contract).  The same per-token arithmetic as ColdStore.token_vecs and
    ColdStore.inner_products -- fp64 head sums in head order, squares and
    products accumulated in dimension order, one rounding to fp32 per vector
    -- applied to all tokens as arrays, for stores of workload size."""
    kp = np.asarray(kpre, dtype=np.float32)
    n, H, D = kp.shape
    dim = D if dim is None else int(dim)
    if n == 0 or r <= 0:
        return np.zeros((0,), dtype=np.int64)
    if per_head:
        x = kp[:, head, :].astype(np.float64)
    else:
        x = np.zeros((n, D), dtype=np.float64)
        for h in range(H):
            x = x + kp[:, h, :].astype(np.float64)
        x = x / float(H)
    if D > dim:
        x = x[:, :dim]
    elif D < dim:
        x = np.concatenate([x, np.zeros((n, dim - D))], axis=1)
    den = np.ones((n,), dtype=np.float64)
    if normalize:
        ss = np.zeros((n,), dtype=np.float64)
        for d in range(dim):
            ss = ss + x[:, d] * x[:, d]
        den = np.maximum(np.sqrt(ss), 1e-12)
    vec = (x / den[:, None]).astype(np.float32).astype(np.float64)
    q = np.asarray(q_vec, dtype=np.float32).astype(np.float64)
    ip = np.zeros((n,), dtype=np.float64)
    for d in range(dim):
        ip = ip + vec[:, d] * q[d]
    return np.argsort(-ip, kind="stable")[: min(int(r), n)].astype(np.int64)


# ---------------------------------------------------------------------------
# Literal torch-CPU reference path, timed as the CPU baseline by bench.py
# ---------------------------------------------------------------------------
def keep_index_torch(scores, window_size, budget):
    """scoring.py:110-132 verbatim in torch (topk + sort + cat)."""
    B, Hk, S = scores.shape
    window = min(window_size, S)
    prefix_len = S - window
    keep_prefix = max(0, min(budget - window, prefix_len))
    recent = torch.arange(prefix_len, S).view(1, 1, window).expand(B, Hk, window)
    if keep_prefix <= 0:
        return recent.contiguous()
    top = torch.topk(scores[:, :, :prefix_len], k=keep_prefix, dim=-1).indices
    top, _ = torch.sort(top, dim=-1)
    return torch.cat([top, recent], dim=-1)


def press_compress_torch(q_post, keys, values, window_size, budget, scaling, kernel_size=7, pooling="maxpool",
                         q_is_window=False):
    """PressLayerState._compress after prefill scoring (layer_state.py:68-94)
    on the CPU: snapkv_importance -> keep_index -> gather_kv x2."""
    imp = snapkv_importance_torch(q_post, keys, window_size, scaling, kernel_size, pooling, dtype=keys.dtype,
                                  q_is_window=q_is_window)
    keep = keep_index_torch(imp, window_size, budget)
    B, H, _, D = keys.shape
    idx = keep.unsqueeze(-1).expand(B, H, keep.shape[-1], D)
    return keys.gather(2, idx).contiguous(), values.gather(2, idx).contiguous()


def press_decode_torch(q_post, keys, values, k_new, v_new, scaling):
    """PressLayerState.decode for SnapKV (layer_state.py:96-100, 115-116, 49-53):
    cat the new token, repeat_kv, SDPA."""
    keys = torch.cat([keys, k_new], dim=2)
    values = torch.cat([values, v_new], dim=2)
    n_rep = q_post.shape[1] // keys.shape[1]
    out = torch.nn.functional.scaled_dot_product_attention(
        q_post, repeat_kv(keys, n_rep), repeat_kv(values, n_rep), is_causal=False, scale=scaling)
    return out.to(q_post.dtype), keys, values
