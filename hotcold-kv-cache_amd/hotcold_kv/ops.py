"""Torch-tensor front end of the gfx950 hot-tier kernels.

Every function here launches HIP kernels from libhotcold_hip.so on the current
torch stream of the tensors' device.  Tensors must live on a ROCm device;
there is no CPU path.  Workspaces are cached per (device, stream) and grown on
demand; torch's caching allocator owns all memory.
"""

import ctypes
import math
import threading

import torch

from . import _native as N

_ws_lock = threading.Lock()
_ws_cache = {}


def _require_device(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "hotcold_kv: the hot-tier kernels run on ROCm device tensors only "
                f"(got a tensor on {t.device})")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device):
    """The raw handle of torch's current stream on `device` (hipStream_t as an int)."""
    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


_stream_handle = stream_handle


def _ptr(t):
    return None if t is None else t.data_ptr()


# Leading bytes of a decode workspace that hold the in-kernel split merge's
# arrival words.  They need no initialisation (each launch counts under its
# own tag), so nothing clears them: a workspace first allocated while a
# graph is being captured puts no fill kernel into the graph.
DECODE_COUNTER_BYTES = 16384


def _workspace(kind, device, nbytes):
    """A uint8 workspace of at least nbytes for this stream, allocated once and
    grown geometrically."""
    key = (kind, device.index if device.index is not None else torch.cuda.current_device(),
           _stream_handle(device))
    with _ws_lock:
        ws = _ws_cache.get(key)
        if ws is None or ws.numel() < nbytes:
            size = max(nbytes, 256)
            if ws is not None:
                size = max(size, int(ws.numel() * 1.5))
            ws = torch.empty(size, dtype=torch.uint8, device=device)
            _ws_cache[key] = ws
        return ws


def _rows4(x, name):
    if x.dim() != 4:
        raise RuntimeError(f"{name} must be 4D (B,H,S,D); got {tuple(x.shape)}")
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x


# ---------------------------------------------------------------------------
# Decode attention
# ---------------------------------------------------------------------------
def _held_mask_args(B, Hk, S, mask, held_len, held_pos, held_valid, cur_pos, what):
    """Validate / normalise the mask and held-slot arguments over S cached rows."""
    if mask is not None:
        if mask.dim() != 2 or mask.shape[0] != B or mask.shape[1] < S:
            raise RuntimeError(f"{what}: mask must be (B,S)=({B},{S}); got {tuple(mask.shape)}")
        if mask.dtype == torch.bool:
            mask = mask.view(torch.uint8) if mask.is_contiguous() else mask.contiguous().view(torch.uint8)
        elif mask.dtype != torch.uint8:
            mask = (mask != 0).to(torch.uint8)
        if mask.stride(1) != 1:
            mask = mask.contiguous()
    hp_sb = hp_sh = hv_sb = hv_sh = 0
    if held_len:
        if held_pos is None or held_valid is None:
            raise RuntimeError(f"{what}: held_len needs held_pos and held_valid")
        if held_valid.dtype == torch.bool:
            held_valid = held_valid.contiguous().view(torch.uint8)
        held_pos = held_pos.contiguous()
        held_valid = held_valid.contiguous()
        for t, name in ((held_pos, "held_pos"), (held_valid, "held_valid")):
            if t.dim() not in (2, 3) or t.shape[0] != B or t.shape[-1] < held_len or held_len > S \
                    or (t.dim() == 3 and t.shape[1] != Hk):
                raise RuntimeError(f"{what}: {name} {tuple(t.shape)} does not cover {held_len} "
                                   f"held rows of (B,Hk)=({B},{Hk})")
        if held_pos.dtype != torch.int64:
            raise RuntimeError(f"{what}: held_pos must be int64")
        hp_sb, hp_sh = (held_pos.stride(0), 0) if held_pos.dim() == 2 else (held_pos.stride(0), held_pos.stride(1))
        hv_sb, hv_sh = (held_valid.stride(0), 0) if held_valid.dim() == 2 else \
            (held_valid.stride(0), held_valid.stride(1))
    if cur_pos is not None and (cur_pos.dtype != torch.int64 or cur_pos.numel() < 1):
        raise RuntimeError(f"{what}: cur_pos must be a non-empty int64 tensor")
    return mask, hp_sb, hp_sh, hv_sb, hv_sh, held_pos, held_valid


def decode_attention(q, k, v, scaling, mask=None, held_len=0, held_pos=None, held_valid=None,
                     cur_pos=None, out=None, num_splits=0, with_evict=False, dropout=0.0):
    """Single-token GQA attention of q (B,Hq,D) or (B,Hq,1,D) over k/v (B,Hk,S,D).

    mask: optional (B,S) bool/uint8, True = attend.  held_len > 0 additionally
    masks the first held_len rows with held_valid & (held_pos <= cur_pos);
    held_pos/held_valid are (B,R) or (B,Hk,R), cur_pos a 1-element int64 device
    tensor (or None).  Returns out (B,Hq,D) in q's dtype, plus
    (evict_loss (B,S) float32, evict_idx (B,) int64) when with_evict.
    """
    _require_device(q, k, v, mask, held_pos, held_valid, cur_pos)
    lib = N.lib()
    if q.dim() == 4:
        if q.shape[2] != 1:
            raise RuntimeError(f"decode_attention: expected one query token, got q {tuple(q.shape)}")
        q3 = q[:, :, 0, :]
    else:
        q3 = q
    if q3.stride(-1) != 1:
        q3 = q3.contiguous()
    k = _rows4(k, "key")
    v = _rows4(v, "value")
    B, Hq, D = q3.shape
    Bk, Hk, S, Dk = k.shape
    if Bk != B or Dk != D or tuple(v.shape) != tuple(k.shape):
        raise RuntimeError(f"decode_attention: shape mismatch q {tuple(q3.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    if k.dtype != q3.dtype or v.dtype != q3.dtype:
        raise RuntimeError("decode_attention: q, k, v must share a dtype")
    mask, hp_sb, hp_sh, hv_sb, hv_sh, held_pos, held_valid = _held_mask_args(
        B, Hk, S, mask, held_len, held_pos, held_valid, cur_pos, "decode_attention")
    if out is None:
        out = torch.empty((B, Hq, D), dtype=q3.dtype, device=q3.device)
    if out.stride(-1) != 1:
        raise RuntimeError("decode_attention: out must have a unit last stride")
    ev_loss = ev_idx = None
    if with_evict:
        ev_loss = torch.empty((B, S), dtype=torch.float32, device=q3.device)
        ev_idx = torch.empty((B,), dtype=torch.int64, device=q3.device)
    nbytes = lib.hc_decode_attn_workspace_size(B, Hq, Hk, D, S, num_splits, int(with_evict))
    ws = _workspace("decode", q3.device, nbytes)
    rc = lib.hc_decode_attn(
        N.dtype_code(q3.dtype), B, Hq, Hk, D, S,
        _ptr(q3), q3.stride(0), q3.stride(1),
        _ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _ptr(v), v.stride(0), v.stride(1), v.stride(2),
        _ptr(mask), mask.stride(0) if mask is not None else 0,
        int(held_len),
        _ptr(held_pos), hp_sb, hp_sh,
        _ptr(held_valid), hv_sb, hv_sh,
        _ptr(cur_pos),
        float(scaling), float(dropout),
        _ptr(out), out.stride(0), out.stride(1),
        _ptr(ev_loss), _ptr(ev_idx),
        _ptr(ws), ws.numel(), int(num_splits),
        _stream_handle(q3.device))
    N.check(rc, "hc_decode_attn")
    if with_evict:
        return out, ev_loss, ev_idx
    return out


def decode_attention_append(q, k, v, k_new, v_new, scaling, pre=None, pos=None, mask=None, held_len=0,
                            held_pos=None, held_valid=None, cur_pos=None, out=None, num_splits=0):
    """Append one token and attend, in one launch.

    k, v are (B,Hk,S,D) views of the hot buffer whose last row S-1 is the
    free row for the new token; k_new, v_new (B,Hk,D) or (B,Hk,1,D) are the
    token's key and value.  The kernel attends over rows 0..S-2 of k/v plus
    the new token and writes k_new/v_new into row S-1 -- the torch.cat append
    followed by attention of cache.py:145-148 / layer_state.py:96-100 and
    kernels.py:77-137.  pre = (p_new, p_dst) and pos = (pos_new (B,1),
    pos_dst (B,>=S)) optionally write the pre-RoPE key row and the position as
    well.  mask / held_* apply to the cached rows as in decode_attention; the
    new token is always attended.  Returns out (B,Hq,D).
    """
    _require_device(q, k, v, k_new, v_new, mask, held_pos, held_valid, cur_pos)
    lib = N.lib()
    if q.dim() == 4 and q.shape[2] != 1:
        raise RuntimeError(f"decode_attention_append: expected one query token, got q {tuple(q.shape)}")
    q3 = q[:, :, 0, :] if q.dim() == 4 else q
    if q3.stride(-1) != 1:
        q3 = q3.contiguous()
    if k.dim() != 4 or v.dim() != 4 or k.stride(-1) != 1 or v.stride(-1) != 1:
        raise RuntimeError("decode_attention_append: k, v must be 4D views with a unit last stride "
                           "(they are written in place)")
    kn = k_new[:, :, 0, :] if k_new.dim() == 4 else k_new
    vn = v_new[:, :, 0, :] if v_new.dim() == 4 else v_new
    B, Hq, D = q3.shape
    Bk, Hk, S, Dk = k.shape
    if Bk != B or Dk != D or S < 1 or tuple(kn.shape) != (B, Hk, D) or tuple(vn.shape) != (B, Hk, D) \
            or tuple(v.shape) != tuple(k.shape):
        raise RuntimeError(f"decode_attention_append: shape mismatch k {tuple(k.shape)} k_new {tuple(k_new.shape)} "
                           f"v_new {tuple(v_new.shape)}")
    if kn.stride(-1) != 1:
        kn = kn.contiguous()
    if vn.stride(-1) != 1:
        vn = vn.contiguous()
    for t in (k, v, kn, vn):
        if t.dtype != q3.dtype:
            raise RuntimeError("decode_attention_append: q, k, v, k_new, v_new must share a dtype")
    pn = pd = None
    if pre is not None:
        pn, pd = pre
        pn = pn[:, :, 0, :] if pn.dim() == 4 else pn
        if pn.stride(-1) != 1:
            pn = pn.contiguous()
        if tuple(pn.shape) != (B, Hk, D) or pd.dim() != 4 or pd.shape[2] < S or pd.stride(-1) != 1 \
                or pd.dtype != q3.dtype or pn.dtype != q3.dtype:
            raise RuntimeError("decode_attention_append: pre=(p_new (B,Hk,D), p_dst (B,Hk,>=S,D)) in q's dtype")
    posn = posd = None
    if pos is not None:
        posn, posd = pos
        if posn.dtype != torch.int64 or posd.dtype != torch.int64 or posn.shape[0] != B or posd.shape[0] != B \
                or posd.dim() != 2 or posd.shape[1] < S or posd.stride(1) != 1:
            raise RuntimeError("decode_attention_append: pos=(pos_new (B,1) int64, pos_dst (B,>=S) int64)")
        posn = posn.reshape(B, -1)
    mask, hp_sb, hp_sh, hv_sb, hv_sh, held_pos, held_valid = _held_mask_args(
        B, Hk, S - 1, mask, held_len, held_pos, held_valid, cur_pos, "decode_attention_append")
    if out is None:
        out = torch.empty((B, Hq, D), dtype=q3.dtype, device=q3.device)
    if out.stride(-1) != 1:
        raise RuntimeError("decode_attention_append: out must have a unit last stride")
    nbytes = lib.hc_decode_attn_workspace_size(B, Hq, Hk, D, S, num_splits, 0)
    ws = _workspace("decode", q3.device, nbytes)
    rc = lib.hc_decode_attn_append(
        N.dtype_code(q3.dtype), B, Hq, Hk, D, S,
        _ptr(q3), q3.stride(0), q3.stride(1),
        _ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _ptr(v), v.stride(0), v.stride(1), v.stride(2),
        _ptr(kn), kn.stride(0), kn.stride(1),
        _ptr(vn), vn.stride(0), vn.stride(1),
        _ptr(pn), pn.stride(0) if pn is not None else 0, pn.stride(1) if pn is not None else 0,
        _ptr(pd), *(pd.stride()[:3] if pd is not None else (0, 0, 0)),
        _ptr(posn), posn.stride(0) if posn is not None else 0,
        _ptr(posd), posd.stride(0) if posd is not None else 0,
        _ptr(mask), mask.stride(0) if mask is not None else 0,
        int(held_len),
        _ptr(held_pos), hp_sb, hp_sh,
        _ptr(held_valid), hv_sb, hv_sh,
        _ptr(cur_pos),
        float(scaling),
        _ptr(out), out.stride(0), out.stride(1),
        _ptr(ws), ws.numel(), int(num_splits),
        _stream_handle(q3.device))
    N.check(rc, "hc_decode_attn_append")
    return out


class _AppendPlan:
    """hc_decode_attn_append_packed arguments of one hot-buffer storage (a
    `st` dict): the shape, the buffers' base pointers and strides, the dtype
    and the stream's workspace are filled in once; a call validates its
    inputs and rewrites only the per-step fields.

    The per-call host work is kept to attribute reads and field writes: the
    (B,H,1,D) rows are addressed through their data pointer and first two
    strides (no views), dtypes compare by identity, and a held slot's
    tensors are validated once per (pos, valid, R) triple, which stays the
    same between injections."""

    def __init__(self, st, Hq):
        k, v = st["k"], st["v"]
        if k.dim() != 4 or v.shape != k.shape or v.dtype != k.dtype or k.stride(-1) != 1 or v.stride(-1) != 1 \
                or not k.is_cuda:
            raise RuntimeError("decode_append_rows: hot-buffer K/V storage must be matching 4D device tensors")
        B, Hk, cap, D = k.shape
        self.tensors = (k, v, st.get("p"), st.get("pos"))     # the storage the pointers below belong to
        self.B, self.Hq, self.Hk, self.cap, self.D = B, int(Hq), Hk, cap, D
        self.dtype, self.dev, self.es = k.dtype, k.device, k.element_size()
        self.devidx = k.get_device()
        self.qshapes = ((B, self.Hq, D), (B, self.Hq, 1, D))
        self.tshapes = ((B, Hk, D), (B, Hk, 1, D))
        a = self.a = N.DecodeAppendArgs()
        a.dtype, a.B, a.Hq, a.Hk, a.D = N.dtype_code(k.dtype), B, self.Hq, Hk, D
        ks, vs = k.stride(), v.stride()
        a.k_sb, a.k_sh, a.k_ss = ks[0], ks[1], ks[2]
        a.v_sb, a.v_sh, a.v_ss = vs[0], vs[1], vs[2]
        self.k0, self.v0, self.krow, self.vrow = k.data_ptr(), v.data_ptr(), ks[2] * self.es, vs[2] * self.es
        self.p = st.get("p")
        if self.p is not None:
            ps = self.p.stride()
            a.pd_sb, a.pd_sh, a.pd_ss = ps[0], ps[1], ps[2]
            self.p0, self.prow = self.p.data_ptr(), ps[2] * self.es
        self.pos = st.get("pos")
        if self.pos is not None:
            a.posd_sb = self.pos.stride(0)
            self.pos0 = self.pos.data_ptr()
        a.o_sb, a.o_sh = self.Hq * D, D
        self.stream, self.ws = None, None
        self.lo = None                  # the row offset the k / v / p_dst / pos_dst pointers are set for
        self.held_key = None            # (pos, valid, R) the held fields are set for
        self.scaling = None
        self.lib = N.lib()
        self.fn = self.lib.hc_decode_attn_append_packed
        self.bind = N.step_bind()
        self.addr = ctypes.addressof(a)

    def _bind_stream(self, stream, S):
        need = self.lib.hc_decode_attn_workspace_size(self.B, self.Hq, self.Hk, self.D, max(S, self.cap), 0, 0)
        self.ws = _workspace("decode", self.dev, need)
        self.a.workspace, self.a.workspace_bytes = self.ws.data_ptr(), self.ws.numel()
        self.stream = stream

    def _row(self, t, shapes, what):
        """data_ptr and (batch, head) strides of a (B,H,D) / (B,H,1,D) row
        tensor on the buffer's device, in its dtype, with a unit last stride."""
        sh = t.shape
        if (sh != shapes[0] and sh != shapes[1]) or t.dtype is not self.dtype or t.get_device() != self.devidx:
            raise RuntimeError(f"decode_append_rows: {what} must be {shapes[0]} or {shapes[1]} device rows in the "
                               f"buffer's dtype {self.dtype}; got {tuple(sh)} {t.dtype} on {t.device}")
        st = t.stride()
        if st[-1] != 1:
            raise RuntimeError(f"decode_append_rows: {what} needs a unit last stride")
        return t.data_ptr(), st[0], st[1]

    def _set_held(self, held, cur_pos, S):
        hp, hv, R = held
        R = int(R)
        if hv.dtype == torch.bool:
            hv = hv.view(torch.uint8)
        B, Hk = self.B, self.Hk
        if hp.dtype != torch.int64 or R > S - 1 or hp.shape[0] != B or hv.shape[0] != B \
                or hp.shape[-1] < R or hv.shape[-1] < R or hp.stride(-1) != 1 or hv.stride(-1) != 1 \
                or (hp.dim() == 3 and hp.shape[1] != Hk) or (hv.dim() == 3 and hv.shape[1] != Hk) \
                or hp.get_device() != self.devidx or hv.get_device() != self.devidx:
            raise RuntimeError("decode_append_rows: held = (pos (B,R)|(B,Hk,R) int64, valid, R <= S-1)")
        a = self.a
        a.held_len = R
        a.held_pos, a.hp_sb, a.hp_sh = hp.data_ptr(), hp.stride(0), hp.stride(1) if hp.dim() == 3 else 0
        a.held_valid, a.hv_sb, a.hv_sh = hv.data_ptr(), hv.stride(0), hv.stride(1) if hv.dim() == 3 else 0

    def run(self, q, lo, S, k_new, v_new, scaling, p_new, pos_new, held, cur_pos, keepdim):
        a = self.a
        if lo < 0 or S < 1 or lo + S > self.cap:
            raise RuntimeError(f"decode_append_rows: rows {lo}..{lo + S - 1} outside the buffer's {self.cap}")
        bind = self.bind
        if bind is None:
            a.q, a.q_sb, a.q_sh = self._row(q, self.qshapes, "q")
            a.k_new, a.kn_sb, a.kn_sh = self._row(k_new, self.tshapes, "k_new")
            a.v_new, a.vn_sb, a.vn_sh = self._row(v_new, self.tshapes, "v_new")
        a.S = S
        if lo != self.lo:
            a.k, a.v = self.k0 + lo * self.krow, self.v0 + lo * self.vrow
            if self.p is not None:
                self.p_dst = self.p0 + lo * self.prow
            if self.pos is not None:
                self.pos_dst = self.pos0 + lo * 8
            self.lo = lo
        # the native step (bind) checks and addresses q, the token's rows,
        # p_new and pos_new itself, and clears p_dst / pos_dst without them
        if p_new is not None:
            if self.p is None:
                raise RuntimeError("decode_append_rows: p_new given but the buffer keeps no pre-RoPE keys")
            if bind is None:
                a.p_new, a.pn_sb, a.pn_sh = self._row(p_new, self.tshapes, "p_new")
            a.p_dst = self.p_dst
        elif bind is None:
            a.p_new = a.p_dst = None
        if pos_new is not None:
            if self.pos is None:
                raise RuntimeError("decode_append_rows: pos_new given but the buffer keeps no positions")
            if bind is None:
                if pos_new.dtype is not torch.int64 or pos_new.shape[0] != self.B \
                        or pos_new.get_device() != self.devidx:
                    raise RuntimeError("decode_append_rows: pos_new must be (B,1) int64")
                a.pos_new, a.posn_sb = pos_new.data_ptr(), pos_new.stride(0)
            a.pos_dst = self.pos_dst
        elif bind is None:
            a.pos_new = a.pos_dst = None
        if held is not None and held[2] > 0:
            if cur_pos is not None and (cur_pos.dtype is not torch.int64 or cur_pos.get_device() != self.devidx):
                raise RuntimeError("decode_append_rows: held = (pos (B,R)|(B,Hk,R) int64, valid, R <= S-1)")
            key = self.held_key
            if key is None or held[0] is not key[0] or held[1] is not key[1] or held[2] != key[2] or held[2] > S - 1:
                self._set_held(held, cur_pos, S)
                self.held_key = (held[0], held[1], held[2])
            a.cur_pos = None if cur_pos is None else cur_pos.data_ptr()
        elif self.held_key is not None:
            a.held_len, a.held_pos, a.held_valid, a.cur_pos = 0, None, None, None
            self.held_key = None
        if scaling != self.scaling:
            a.scaling = self.scaling = scaling
        stream = _raw_stream(self.devidx) if _raw_stream is not None else stream_handle(self.dev)
        if stream != self.stream:
            self._bind_stream(stream, S)
        if bind is not None:
            out, rc = bind.decode_append_step(self.addr, q, k_new, v_new, p_new, pos_new, keepdim, stream,
                                              self.devidx)
            if rc:                              # not HC_OK (0)
                if rc == N.HC_ERR_WORKSPACE:
                    self._bind_stream(stream, S)    # a longer buffer than the one the workspace was sized for
                    out, rc = bind.decode_append_step(self.addr, q, k_new, v_new, p_new, pos_new, keepdim, stream,
                                                      self.devidx)
                N.check(rc, "hc_decode_attn_append")
            return out
        # sizes as separate arguments: 0.4 us less per call than a tuple
        out = (torch.empty(self.B, self.Hq, 1, self.D, dtype=self.dtype, device=self.dev) if keepdim
               else torch.empty(self.B, self.Hq, self.D, dtype=self.dtype, device=self.dev))
        a.out = out.data_ptr()
        rc = self.fn(self.addr, stream)
        if rc == N.HC_ERR_WORKSPACE:
            self._bind_stream(stream, S)        # a longer buffer than the one the workspace was sized for
            rc = self.fn(self.addr, stream)
        N.check(rc, "hc_decode_attn_append")
        return out


def decode_append_rows(q, st, lo, S, k_new, v_new, scaling, p_new=None, pos_new=None, held=None, cur_pos=None,
                       keepdim=False):
    """decode_attention_append over rows lo .. lo+S-1 of a hot buffer's
    storage, addressed by offset instead of through tensor views (the
    per-layer decode call of the drop-in; same launch, less host work: the
    storage's packed argument struct is kept in st and only the per-step
    fields are rewritten).

    st: {"k", "v"[, "p", "pos"]} -- (B,Hk,cap,D) K/V/pre-RoPE rows and
    (B,cap) int64 positions.  Row lo+S-1 receives k_new / v_new (and p_new,
    pos_new (B,1)).  held = (pos, valid, R): the first R attended rows are the
    held slot, masked with valid & (pos <= cur_pos).  Returns out (B,Hq,D),
    or (B,Hq,1,D) with keepdim."""
    Hq = q.shape[1]
    plan = st.get("_plan")
    if plan is None or plan.Hq != Hq or plan.tensors[0] is not st["k"] or plan.tensors[1] is not st["v"] \
            or plan.tensors[2] is not st.get("p") or plan.tensors[3] is not st.get("pos"):
        plan = st["_plan"] = _AppendPlan(st, Hq)
    return plan.run(q, int(lo), int(S), k_new, v_new, float(scaling), p_new, pos_new, held, cur_pos, keepdim)


class _H2OEvictPlan:
    """hc_decode_attn_h2o_evict_packed arguments of one (source storage,
    destination storage, scores, destination scores) quadruple: everything
    but q, the token's rows, S and out is filled in once.  An H2O layer at
    budget alternates between two such plans (its storages swap every step)."""

    def __init__(self, st, Hq, acc, dst, acc_dst, dst_lo, window, budget):
        k, v, kd, vd = st["k"], st["v"], dst["k"], dst["v"]
        for t in (v, kd, vd):
            if t.dim() != 4 or t.shape[0] != k.shape[0] or t.shape[1] != k.shape[1] or t.shape[3] != k.shape[3] \
                    or t.dtype != k.dtype or t.stride(-1) != 1 or t.get_device() != k.get_device():
                raise RuntimeError("decode_h2o_evict_rows: source and destination K/V storages must be matching "
                                   "(B,Hk,cap,D) device tensors")
        if k.dim() != 4 or k.stride(-1) != 1 or not k.is_cuda:
            raise RuntimeError("decode_h2o_evict_rows: hot-buffer K/V storage must be 4D device tensors")
        B, Hk, cap, D = k.shape
        for name, t in (("acc", acc), ("acc_dst", acc_dst)):
            if t.dtype != torch.float32 or t.dim() != 3 or tuple(t.shape[:2]) != (B, Hk) or t.stride(2) != 1 \
                    or t.get_device() != k.get_device():
                raise RuntimeError(f"decode_h2o_evict_rows: {name} must be (B,Hk,n) fp32 with unit last stride")
        self.tensors = (k, v, kd, vd, acc, acc_dst)
        self.Hq, self.dst_lo, self.window, self.budget = int(Hq), int(dst_lo), int(window), int(budget)
        self.B, self.Hk, self.cap, self.D = B, Hk, cap, D
        self.acc_cap, self.acc_dst_cap, self.dst_cap = acc.shape[2], acc_dst.shape[2], kd.shape[2] - int(dst_lo)
        self.dtype, self.dev, self.devidx, self.es = k.dtype, k.device, k.get_device(), k.element_size()
        self.qshapes = ((B, self.Hq, D), (B, self.Hq, 1, D))
        self.tshapes = ((B, Hk, D), (B, Hk, 1, D))
        a = self.a = N.DecodeH2OEvictArgs()
        a.dtype, a.B, a.Hq, a.Hk, a.D = N.dtype_code(k.dtype), B, self.Hq, Hk, D
        ks, vs, kds, vds = k.stride(), v.stride(), kd.stride(), vd.stride()
        a.k_sb, a.k_sh, a.k_ss = ks[0], ks[1], ks[2]
        a.v_sb, a.v_sh, a.v_ss = vs[0], vs[1], vs[2]
        a.kd_sb, a.kd_sh, a.kd_ss = kds[0], kds[1], kds[2]
        a.vd_sb, a.vd_sh, a.vd_ss = vds[0], vds[1], vds[2]
        a.k_dst = kd.data_ptr() + self.dst_lo * kds[2] * self.es
        a.v_dst = vd.data_ptr() + self.dst_lo * vds[2] * self.es
        self.k0, self.v0, self.krow, self.vrow = k.data_ptr(), v.data_ptr(), ks[2] * self.es, vs[2] * self.es
        acs, ads = acc.stride(), acc_dst.stride()
        a.acc, a.a_sb, a.a_sh = acc.data_ptr(), acs[0], acs[1]
        a.acc_dst, a.ad_sb, a.ad_sh = acc_dst.data_ptr(), ads[0], ads[1]
        a.window, a.budget = self.window, self.budget
        a.o_sb, a.o_sh = self.Hq * D, D
        self.stream, self.ws, self.lo, self.scaling = None, None, None, None
        self.lib = N.lib()
        self.fn = self.lib.hc_decode_attn_h2o_evict_packed
        self.addr = ctypes.addressof(a)

    def matches(self, st, Hq, acc, dst, acc_dst, dst_lo, window, budget):
        t = self.tensors
        return (t[0] is st["k"] and t[1] is st["v"] and t[2] is dst["k"] and t[3] is dst["v"] and t[4] is acc
                and t[5] is acc_dst and self.Hq == Hq and self.dst_lo == dst_lo and self.window == window
                and self.budget == budget)

    def _bind_stream(self, stream, S):
        need = self.lib.hc_decode_attn_workspace_size(self.B, self.Hq, self.Hk, self.D, max(S, self.cap), 0, 1)
        self.ws = _workspace("decode", self.dev, need)
        self.a.workspace, self.a.workspace_bytes = self.ws.data_ptr(), self.ws.numel()
        self.stream = stream

    def run(self, q, lo, S, k_new, v_new, scaling):
        a = self.a
        if lo < 0 or S < 2 or lo + S > self.cap or S > self.acc_cap or S - 1 > self.dst_cap \
                or S - 1 > self.acc_dst_cap:
            raise RuntimeError(f"decode_h2o_evict_rows: rows {lo}..{lo + S - 1} (kept {S - 1}) outside the "
                               f"buffers ({self.cap} rows, scores {self.acc_cap}, destination {self.dst_cap})")
        a.q, a.q_sb, a.q_sh = _row_args(q, self.qshapes, self.dtype, self.devidx, "q")
        a.k_new, a.kn_sb, a.kn_sh = _row_args(k_new, self.tshapes, self.dtype, self.devidx, "k_new")
        a.v_new, a.vn_sb, a.vn_sh = _row_args(v_new, self.tshapes, self.dtype, self.devidx, "v_new")
        a.S = S
        if lo != self.lo:
            a.k, a.v = self.k0 + lo * self.krow, self.v0 + lo * self.vrow
            self.lo = lo
        if scaling != self.scaling:
            a.scaling = self.scaling = scaling
        out = torch.empty(self.B, self.Hq, 1, self.D, dtype=self.dtype, device=self.dev)
        a.out = out.data_ptr()
        stream = _raw_stream(self.devidx) if _raw_stream is not None else stream_handle(self.dev)
        if stream != self.stream:
            self._bind_stream(stream, S)
        rc = self.fn(self.addr, stream)
        if rc == N.HC_ERR_WORKSPACE:
            self._bind_stream(stream, S)
            rc = self.fn(self.addr, stream)
        N.check(rc, "hc_decode_attn_h2o_evict")
        return out


def _row_args(t, shapes, dtype, devidx, what):
    """data_ptr and (batch, head) strides of a (B,H,D) / (B,H,1,D) row tensor
    on device devidx, in dtype, with a unit last stride (no view is made)."""
    sh = t.shape
    if (sh != shapes[0] and sh != shapes[1]) or t.dtype is not dtype or t.get_device() != devidx:
        raise RuntimeError(f"decode_h2o_evict_rows: {what} must be {shapes[0]} or {shapes[1]} device rows in "
                           f"{dtype}; got {tuple(sh)} {t.dtype} on {t.device}")
    st = t.stride()
    if st[-1] != 1:
        raise RuntimeError(f"decode_h2o_evict_rows: {what} needs a unit last stride")
    return t.data_ptr(), st[0], st[1]


def decode_h2o_evict_rows(q, st, lo, S, k_new, v_new, scaling, acc, window_size, budget, dst, acc_dst, dst_lo=0):
    """decode_attention_h2o_evict over rows lo .. lo+S-1 of a hot buffer's
    storage st ({"k", "v"} (B,Hk,cap,D)), addressed by offset instead of
    through views (the H2O decode step of the drop-in at budget; same launch,
    less host work): row lo+S-1 receives k_new / v_new, acc (B,Hk,>=S) fp32
    holds the scores of rows lo.. (column i: row lo+i), and the S-1 kept rows
    and their updated scores go to rows dst_lo.. of the storage dst and to
    acc_dst (B,Hk,>=S-1).  The packed argument struct of the quadruple is kept in st.
    Returns out (B,Hq,1,D)."""
    Hq = q.shape[1]
    plan = st.get("_h2o_plan")
    if plan is None or not plan.matches(st, Hq, acc, dst, acc_dst, dst_lo, window_size, budget):
        plan = st["_h2o_plan"] = _H2OEvictPlan(st, Hq, acc, dst, acc_dst, dst_lo, window_size, budget)
    return plan.run(q, int(lo), int(S), k_new, v_new, float(scaling))


def decode_attention_h2o(q, k, v, scaling, acc, out=None, num_splits=0):
    """Decode attention of q (B,Hq,D) or (B,Hq,1,D) over k/v (B,Hk,S,D) that
    adds each key's attention probability, averaged over the query heads of
    its KV head, to acc (B,Hk,>=S) fp32; key S-1 (this step's token) starts
    from zero -- H2O's accumulated attention (layer_state.py:102-114).
    Returns out (B,Hq,D)."""
    _require_device(q, k, v, acc)
    lib = N.lib()
    if q.dim() == 4:
        if q.shape[2] != 1:
            raise RuntimeError(f"decode_attention_h2o: expected one query token, got q {tuple(q.shape)}")
        q = q[:, :, 0, :]
    if q.stride(-1) != 1:
        q = q.contiguous()
    k = _rows4(k, "key")
    v = _rows4(v, "value")
    B, Hq, D = q.shape
    _, Hk, S, _ = k.shape
    if tuple(v.shape) != tuple(k.shape) or k.shape[0] != B or k.shape[3] != D or k.dtype != q.dtype \
            or v.dtype != q.dtype:
        raise RuntimeError("decode_attention_h2o: q, k, v shapes / dtypes do not match")
    if acc.dtype != torch.float32 or acc.dim() != 3 or tuple(acc.shape[:2]) != (B, Hk) or acc.shape[2] < S \
            or acc.stride(2) != 1:
        raise RuntimeError(f"decode_attention_h2o: acc must be (B,Hk,>=S) fp32 with unit last stride; "
                           f"got {tuple(acc.shape)} {acc.dtype}")
    if out is None:
        out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    nbytes = lib.hc_decode_attn_workspace_size(B, Hq, Hk, D, S, num_splits, 1)
    ws = _workspace("decode", q.device, nbytes)
    rc = lib.hc_decode_attn_h2o(
        N.dtype_code(q.dtype), B, Hq, Hk, D, S,
        _ptr(q), q.stride(0), q.stride(1),
        _ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _ptr(v), v.stride(0), v.stride(1), v.stride(2),
        float(scaling),
        _ptr(out), out.stride(0), out.stride(1),
        _ptr(acc), acc.stride(0), acc.stride(1),
        _ptr(ws), ws.numel(), int(num_splits),
        _stream_handle(q.device))
    N.check(rc, "hc_decode_attn_h2o")
    return out


H2O_EVICT_MAX_KEYS = 8192


def h2o_evicts_one(S, window_size, budget):
    """True when keep_index(scores of S keys, window_size, budget) drops
    exactly one row and S fits the fused eviction (S <= 8192)."""
    _, prefix, kp = keep_counts(S, window_size, budget)
    return prefix - kp == 1 and S <= H2O_EVICT_MAX_KEYS


def decode_attention_h2o_evict(q, k, v, scaling, acc, window_size, budget, k_dst, v_dst, acc_dst, out=None,
                               num_splits=0, k_new=None, v_new=None):
    """One H2O decode step whose append put the cache one row over budget
    (layer_state.py:102-114 then _compress, :68-79): attends q over k/v
    (B,Hk,S,D), forms the updated scores acc + this step's G-mean
    probabilities (key S-1 from zero), and writes the S-1 rows that
    keep_index(updated, window_size, budget) keeps -- all but the lowest
    prefix score, the highest index among equal ones -- in order into k_dst,
    v_dst (B,Hk,>=S-1,D) and acc_dst (B,Hk,>=S-1) fp32.  acc is only read.
    Equals decode_attention_h2o + keep_index + gather_rows bit for bit.
    With k_new, v_new (B,Hk,D) or (B,Hk,1,D) the step's token is appended in
    the same launch (decode_attention_append): row S-1 of k/v is the free row
    it is written into.  Returns out (B,Hq,D).  Called every decode step:
    shapes and strides are read once per tensor."""
    _require_device(q, k, v, acc, k_dst, v_dst, acc_dst, k_new, v_new)
    lib = N.lib()
    if q.dim() == 4:
        if q.shape[2] != 1:
            raise RuntimeError(f"decode_attention_h2o_evict: expected one query token, got q {tuple(q.shape)}")
        q = q[:, :, 0, :]
    if q.stride(-1) != 1:
        q = q.contiguous()
    k = _rows4(k, "key")
    v = _rows4(v, "value")
    B, Hq, D = q.shape
    ks, vs = tuple(k.shape), tuple(v.shape)
    _, Hk, S, _ = ks
    dt = q.dtype
    if vs != ks or ks[0] != B or ks[3] != D or k.dtype != dt or v.dtype != dt:
        raise RuntimeError("decode_attention_h2o_evict: q, k, v shapes / dtypes do not match")
    st = {}
    for name, t, rows in (("acc", acc, S), ("acc_dst", acc_dst, S - 1)):
        sh, sd = tuple(t.shape), t.stride()
        if t.dtype != torch.float32 or len(sh) != 3 or sh[:2] != (B, Hk) or sh[2] < rows or sd[2] != 1:
            raise RuntimeError(f"decode_attention_h2o_evict: {name} must be (B,Hk,>={rows}) fp32 with unit last "
                               f"stride; got {sh} {t.dtype}")
        st[name] = sd
    for name, t in (("k_dst", k_dst), ("v_dst", v_dst)):
        sh, sd = tuple(t.shape), t.stride()
        if len(sh) != 4 or sh[:2] != (B, Hk) or sh[2] < S - 1 or sh[3] != D or t.dtype != dt or sd[3] != 1:
            raise RuntimeError(f"decode_attention_h2o_evict: {name} must be (B,Hk,>={S - 1},D) {dt} rows; "
                               f"got {sh} {t.dtype}")
        st[name] = sd
    if not h2o_evicts_one(S, window_size, budget):
        raise RuntimeError(f"decode_attention_h2o_evict: S={S}, window {window_size}, budget {budget} does not "
                           f"drop exactly one row (or S > {H2O_EVICT_MAX_KEYS})")
    if (k_new is None) != (v_new is None):
        raise RuntimeError("decode_attention_h2o_evict: k_new and v_new go together")
    if k_new is not None:
        k_new, v_new = (x[:, :, 0, :] if x.dim() == 4 else x for x in (k_new, v_new))
        for name, t in (("k_new", k_new), ("v_new", v_new)):
            if tuple(t.shape) != (B, Hk, D) or t.dtype != dt:
                raise RuntimeError(f"decode_attention_h2o_evict: {name} must be (B,Hk,D)=({B},{Hk},{D}) {dt}; "
                                   f"got {tuple(t.shape)} {t.dtype}")
        k_new = k_new if k_new.stride(-1) == 1 else k_new.contiguous()
        v_new = v_new if v_new.stride(-1) == 1 else v_new.contiguous()
        kns, vns = k_new.stride(), v_new.stride()
    else:
        kns = vns = (0, 0)
    if out is None:
        out = torch.empty((B, Hq, D), dtype=dt, device=q.device)
    nbytes = lib.hc_decode_attn_workspace_size(B, Hq, Hk, D, S, num_splits, 1)
    ws = _workspace("decode", q.device, nbytes)
    qs, kss, vss, os_ = q.stride(), k.stride(), v.stride(), out.stride()
    sa, sad, skd, svd = st["acc"], st["acc_dst"], st["k_dst"], st["v_dst"]
    rc = lib.hc_decode_attn_h2o_evict(
        N.dtype_code(dt), B, Hq, Hk, D, S,
        _ptr(q), qs[0], qs[1],
        _ptr(k), kss[0], kss[1], kss[2],
        _ptr(v), vss[0], vss[1], vss[2],
        _ptr(k_new), kns[0], kns[1],
        _ptr(v_new), vns[0], vns[1],
        float(scaling),
        _ptr(out), os_[0], os_[1],
        _ptr(acc), sa[0], sa[1],
        int(window_size), int(budget),
        _ptr(k_dst), skd[0], skd[1], skd[2],
        _ptr(v_dst), svd[0], svd[1], svd[2],
        _ptr(acc_dst), sad[0], sad[1],
        _ptr(ws), ws.numel(), int(num_splits),
        _stream_handle(q.device))
    N.check(rc, "hc_decode_attn_h2o_evict")
    return out


# ---------------------------------------------------------------------------
# SnapKV compaction
# ---------------------------------------------------------------------------
def snapkv_scores(q_post, keys, window_size, scaling, kernel_size=7, pooling="maxpool",
                  mode="snapkv", q_rows=None):
    """Per-KV-head importance (B,Hk,S) float32.

    mode "snapkv": scoring.py:50-79 (window = last min(window_size,S) rows of
    q_post, causal mask, softmax, window sum, pooling).  mode "rawsum":
    cache.py:55-69 before the head mean (q_post holds the stashed queries; the
    last `window_size` of its rows are used; no mask, no softmax, no pooling).
    """
    _require_device(q_post, keys)
    lib = N.lib()
    keys = _rows4(keys, "keys")
    if q_post.dim() != 4:
        raise RuntimeError(f"q_post must be 4D (B,Hq,T,D); got {tuple(q_post.shape)}")
    if q_post.stride(-1) != 1:
        q_post = q_post.contiguous()
    B, Hq, T, D = q_post.shape
    _, Hk, S, _ = keys.shape
    if keys.dtype != q_post.dtype:
        raise RuntimeError("snapkv_scores: q and keys must share a dtype")
    if mode == "snapkv":
        W = min(int(window_size), S)
        if T != S:
            raise RuntimeError("snapkv_scores: q_post must cover the whole prompt (T == S)")
        q_row0 = S - W
        mcode = N.HC_SCORE_SNAPKV
    elif mode == "rawsum":
        W = min(int(window_size), T)
        q_row0 = T - W
        mcode = N.HC_SCORE_RAWSUM
        kernel_size = 1
    else:
        raise ValueError(f"unknown score mode {mode}")
    if kernel_size is None:
        kernel_size = 1
    pool = N.HC_POOL_AVG if pooling == "avgpool" else N.HC_POOL_MAX
    scores = torch.empty((B, Hk, S), dtype=torch.float32, device=keys.device)
    nbytes = lib.hc_snapkv_score_workspace_size(B, Hk, S, D, W)
    ws = _workspace("score", keys.device, nbytes)
    rc = lib.hc_snapkv_score(
        N.dtype_code(keys.dtype), mcode, B, Hq, Hk, S, D, W,
        _ptr(q_post), q_post.stride(0), q_post.stride(1), q_post.stride(2), q_row0,
        _ptr(keys), keys.stride(0), keys.stride(1), keys.stride(2),
        float(scaling), int(kernel_size), pool,
        _ptr(scores), _ptr(ws), ws.numel(), _stream_handle(keys.device))
    N.check(rc, "hc_snapkv_score")
    return scores


def row_addresses(tensors):
    """Base address of every batch row of every tensor, in order (tensor 0
    rows 0..B-1, tensor 1 rows 0..B-1, ...)."""
    ptrs = []
    for t in tensors:
        base, step = t.data_ptr(), t.stride(0) * t.element_size()
        ptrs.extend(base + b * step for b in range(t.shape[0]))
    return ptrs


def device_tables(*lists, device=None):
    """One device int64 array per list of addresses, all sent with a single
    copy from pinned host memory (to `device`, default the current one)."""
    flat = [p for x in lists for p in x]
    dev = device if device is not None else torch.cuda.current_device()
    tab = torch.tensor(flat, dtype=torch.int64, pin_memory=True).to(dev, non_blocking=True)
    out, o = [], 0
    for x in lists:
        out.append(tab[o:o + len(x)])
        o += len(x)
    return out


def _same_layout(tensors, what):
    t0 = tensors[0]
    for t in tensors[1:]:
        if t.shape != t0.shape or t.stride()[1:] != t0.stride()[1:] or t.dtype != t0.dtype or t.device != t0.device:
            raise RuntimeError(f"{what}: every tensor must share shape, dtype, device and head/row strides")


def snapkv_scores_rows(q_list, k_list, window_size, scaling, kernel_size=7, pooling="maxpool", tables=None):
    """snapkv_scores for several (queries, keys) pairs at once -- the layers of
    a model, each in its own allocation -- in one launch set.

    q_list[i] (B,Hq,T,D) holds at least the window (its last min(window, S)
    rows are the window queries, at prompt positions S-W..S-1); k_list[i]
    (B,Hk,S,D).  Returns (len * B, Hk, S) float32: the rows of pair i are
    i*B .. i*B+B-1, each bit-equal to snapkv_scores on that pair.  tables:
    optional device (q, k) row-address tables already built for the lists.
    """
    if not q_list or len(q_list) != len(k_list):
        raise ValueError("snapkv_scores_rows: one query tensor per key tensor, at least one")
    _require_device(*q_list, *k_list)
    _same_layout(q_list, "snapkv_scores_rows (queries)")
    _same_layout(k_list, "snapkv_scores_rows (keys)")
    q0, k0 = q_list[0], k_list[0]
    if q0.dim() != 4 or k0.dim() != 4 or q0.stride(-1) != 1 or k0.stride(-1) != 1:
        raise RuntimeError("snapkv_scores_rows: 4D tensors with contiguous rows required")
    if k0.dtype != q0.dtype:
        raise RuntimeError("snapkv_scores_rows: q and keys must share a dtype")
    B, Hq, T, D = q0.shape
    _, Hk, S, _ = k0.shape
    W = min(int(window_size), S)
    if T < W:
        raise RuntimeError(f"snapkv_scores_rows: {T} query rows hold less than the window {W}")
    R = len(k_list) * B
    pool = N.HC_POOL_AVG if pooling == "avgpool" else N.HC_POOL_MAX
    qt, kt = tables if tables is not None else device_tables(row_addresses(q_list), row_addresses(k_list),
                                                             device=k0.device)
    scores = torch.empty((R, Hk, S), dtype=torch.float32, device=k0.device)
    lib = N.lib()
    ws = _workspace("score", k0.device, lib.hc_snapkv_score_workspace_size(R, Hk, S, D, W))
    rc = lib.hc_snapkv_score_rows(
        N.dtype_code(k0.dtype), N.HC_SCORE_SNAPKV, R, Hq, Hk, S, D, W,
        _ptr(qt), q0.stride(1), q0.stride(2), T - W,
        _ptr(kt), k0.stride(1), k0.stride(2),
        float(scaling), int(kernel_size or 1), pool,
        _ptr(scores), _ptr(ws), ws.numel(), _stream_handle(k0.device))
    N.check(rc, "hc_snapkv_score_rows")
    return scores


def gather_rows_tab(idx, k_src, v_src, k_dst, v_dst, dst_row0=0, tables=None):
    """gather_rows of K and V for several tensors at once (the layers of a
    model): k_dst[i][b,h,dst_row0+j] = k_src[i][b,h,idx[i*B+b,h,j]], same for
    V, in one launch.  idx is (len * B, H, n) int64.  tables: optional device
    row-address tables of (k_src, v_src, k_dst, v_dst) already built."""
    lists = (k_src, v_src, k_dst, v_dst)
    if not k_src or any(len(x) != len(k_src) for x in lists):
        raise ValueError("gather_rows_tab: four lists of equal, non-zero length")
    for x in lists:
        _same_layout(x, "gather_rows_tab")
    _require_device(idx, *k_src, *v_src, *k_dst, *v_dst)
    s0, d0 = k_src[0], k_dst[0]
    B, H, S, D = s0.shape
    R = len(k_src) * B
    if idx.dim() != 3 or idx.shape[0] != R or idx.shape[1] != H or idx.stride(-1) != 1:
        raise RuntimeError(f"gather_rows_tab: index {tuple(idx.shape)} must be ({R},{H},n) with unit last stride")
    n = idx.shape[2]
    for s, d in ((k_src[0], k_dst[0]), (v_src[0], v_dst[0])):
        if s.dtype != s0.dtype or d.dtype != s0.dtype or s.shape[:2] != (B, H) or d.shape[:2] != (B, H) \
                or s.shape[3] != D or d.shape[3] != D or s.stride(-1) != 1 or d.stride(-1) != 1:
            raise RuntimeError("gather_rows_tab: K/V sources and destinations do not match")
        if d.shape[2] < dst_row0 + n:
            raise RuntimeError(f"gather_rows_tab: destination holds {d.shape[2]} rows, needs {dst_row0 + n}")
    dev = s0.device
    tabs = tables if tables is not None else device_tables(*[row_addresses(x) for x in lists], device=dev)
    vs, vd = v_src[0], v_dst[0]
    rc = N.lib().hc_gather_rows_tab(
        R, H, n, D, s0.element_size(), _ptr(idx), idx.stride(0), idx.stride(1), S, int(dst_row0),
        _ptr(tabs[0]), s0.stride(1), s0.stride(2), _ptr(tabs[2]), d0.stride(1), d0.stride(2),
        _ptr(tabs[1]), vs.stride(1), vs.stride(2), _ptr(tabs[3]), vd.stride(1), vd.stride(2),
        _stream_handle(dev))
    N.check(rc, "hc_gather_rows_tab")


def h2o_prefill_scores(q_post, keys, scaling, max_workspace_bytes=10 << 30):
    """H2O accumulated attention of the whole prompt per KV head, fp32
    (B,Hk,S) (scoring.py:82-107): for every key, the causal softmax
    probabilities of all query rows summed, per query head, then averaged over
    the query heads of its KV head.  It is the window score with the window
    covering the prompt, one query head per "KV head" and no pooling, so it
    runs on the exact window-score kernels (bit-defined like SnapKV's) over
    keys repeated per query head, followed by the group mean.  Query heads go
    in chunks whose logits workspace fits max_workspace_bytes (the 32 heads of
    an 8k prompt fit one: the importance kernel needs their keys together to
    fill the GPU, one chain per key)."""
    _require_device(q_post, keys)
    B, Hq, S, D = q_post.shape
    Hk = keys.shape[1]
    if Hq % Hk != 0:
        raise ValueError(f"h2o_prefill_scores: Hq ({Hq}) must be a multiple of Hk ({Hk})")
    G = Hq // Hk
    per_group = G * int(N.lib().hc_snapkv_score_workspace_size(B, 1, S, D, S))
    groups = max(1, min(Hk, max_workspace_bytes // max(per_group, 1)))     # KV groups per chunk
    per_q = torch.empty((B, Hq, S), dtype=torch.float32, device=keys.device)
    for g0 in range(0, Hk, groups):
        g1 = min(Hk, g0 + groups)
        k_rep = keys[:, g0:g1].repeat_interleave(G, dim=1).contiguous()   # one key head per query head
        per_q[:, g0 * G:g1 * G] = snapkv_scores(q_post[:, g0 * G:g1 * G], k_rep, S, scaling, 1, "maxpool")
    return head_mean(per_q.view(B * Hk, G, S)).view(B, Hk, S)


def head_mean(scores):
    """(B,H,S) float32 -> (B,S): mean over heads in fp64, rounded to fp32."""
    _require_device(scores)
    scores = scores.contiguous()
    B, H, S = scores.shape
    out = torch.empty((B, S), dtype=torch.float32, device=scores.device)
    N.check(N.lib().hc_head_mean(B, H, S, _ptr(scores), _ptr(out), _stream_handle(scores.device)), "hc_head_mean")
    return out


def keep_counts(S, window_size, budget):
    window = min(int(window_size), int(S))
    prefix = int(S) - window
    keep_prefix = max(0, min(int(budget) - window, prefix))
    return window, prefix, keep_prefix


def keep_index(scores, window_size, budget, return_evicted=False):
    """scoring.py:110-132 on the device: (B,H,S) float32 -> (B,H,keep) int64.

    Top keep_prefix prefix positions by (score desc, index asc), ascending,
    then the recent window.  With return_evicted also the ascending prefix
    positions not kept, (B,H,prefix-keep_prefix).
    """
    _require_device(scores)
    squeeze = False
    if scores.dim() == 2:
        scores = scores.unsqueeze(1)
        squeeze = True
    if scores.dtype != torch.float32:
        scores = scores.float()
    if scores.stride(-1) != 1:
        scores = scores.contiguous()
    B, H, S = scores.shape
    window, prefix, kp = keep_counts(S, window_size, budget)
    keep = torch.empty((B, H, kp + window), dtype=torch.int64, device=scores.device)
    ev = torch.empty((B, H, prefix - kp), dtype=torch.int64, device=scores.device) if return_evicted else None
    # few long rows: the chunked selection, in a workspace the library sizes
    ws_bytes = N.lib().hc_topk_keep_workspace_size(B, H, S, int(window_size), int(budget))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=scores.device) if ws_bytes > 0 else None
    rc = N.lib().hc_topk_keep_ws(B, H, S, _ptr(scores), scores.stride(0), scores.stride(1), int(window_size),
                                 int(budget), _ptr(keep), _ptr(ev), _ptr(ws), ws_bytes, _stream_handle(scores.device))
    N.check(rc, "hc_topk_keep_ws")
    if squeeze:
        keep = keep[:, 0]
        ev = ev[:, 0] if ev is not None else None
    return (keep, ev) if return_evicted else keep


def _strides3(t):
    """(sb, sh, ss) element strides of a (B,H,S,D) tensor."""
    return t.stride(0), t.stride(1), t.stride(2)


def gather_rows(idx, pairs, dst_row0=0, pos_src=None, pos_dst=None, src_rows=None):
    """dst[b,h,dst_row0+j] = src[b,h,idx[b,h,j]] for up to three (src, dst) pairs.

    idx is (B,H,n) or (B,n) (one set shared by all heads).  pos_src (B,S) and
    pos_dst (B,*) gather int64 positions with the head-0 index set.
    """
    if not 1 <= len(pairs) <= 3:
        raise ValueError("gather_rows takes one to three (src, dst) pairs")
    src0, dst0 = pairs[0]
    _require_device(idx, src0, dst0, pos_src, pos_dst)
    B, H, S, D = src0.shape
    if idx.dim() == 2:
        i_sb, i_sh, n = idx.stride(0), 0, idx.shape[1]
    else:
        i_sb, i_sh, n = idx.stride(0), idx.stride(1), idx.shape[2]
    if idx.stride(-1) != 1:
        idx = idx.contiguous()
        return gather_rows(idx, pairs, dst_row0, pos_src, pos_dst, src_rows)
    es = src0.element_size()
    args = []
    for i in range(3):
        if i < len(pairs):
            s, d = pairs[i]
            if s.dtype != src0.dtype or d.dtype != src0.dtype:
                raise RuntimeError("gather_rows: all tensors must share a dtype")
            if s.dim() != 4 or d.dim() != 4 or s.shape[0] != B or d.shape[0] != B or s.shape[1] != H \
                    or d.shape[1] != H or s.shape[3] != D or d.shape[3] != D or s.shape[2] < S:
                raise RuntimeError(f"gather_rows: shape mismatch src {tuple(s.shape)} dst {tuple(d.shape)}")
            if d.shape[2] < dst_row0 + n:
                raise RuntimeError(f"gather_rows: destination holds {d.shape[2]} rows, needs {dst_row0 + n}")
            if s.stride(-1) != 1 or d.stride(-1) != 1:
                raise RuntimeError("gather_rows: rows must be contiguous")
            args += [_ptr(s), *_strides3(s), _ptr(d), *_strides3(d)]
        else:
            args += [None, 0, 0, 0, None, 0, 0, 0]
    if idx.shape[0] != B or (idx.dim() == 3 and idx.shape[1] != H):
        raise RuntimeError(f"gather_rows: index shape {tuple(idx.shape)} does not match (B,H)=({B},{H})")
    if pos_src is not None:
        if pos_src.dim() != 2 or pos_src.shape[0] != B or pos_src.shape[1] < S or pos_dst.dim() != 2 \
                or pos_dst.shape[0] != B or pos_dst.shape[1] < dst_row0 + n or pos_src.stride(1) != 1 \
                or pos_dst.stride(1) != 1:
            raise RuntimeError("gather_rows: bad position tensors")
    rc = N.lib().hc_gather_rows(
        B, H, n, D, es, _ptr(idx), i_sb, i_sh, int(src_rows if src_rows is not None else S), int(dst_row0),
        *args,
        _ptr(pos_src), pos_src.stride(0) if pos_src is not None else 0,
        _ptr(pos_dst), pos_dst.stride(0) if pos_dst is not None else 0,
        _stream_handle(src0.device))
    N.check(rc, "hc_gather_rows")


def gather_kv(t, keep):
    """scoring.py:135-139: gather (B,H,S,D) along S with per-head keep (B,H,k)."""
    B, H, S, D = t.shape
    n = keep.shape[-1]
    out = torch.empty((B, H, n, D), dtype=t.dtype, device=t.device)
    gather_rows(keep, [(t, out)])
    return out


def gather_evict(idx, k, v, pos, dev_out=None, host_out=None):
    """Evicted rows idx (B,te) (shared by the heads) of k/v (B,H,S,D) upcast
    to fp32 plus their positions from pos (B,S), in one packed block
    (cache.py:86-125).  dev_out / host_out are uint8 tensors of at least
    gather_evict_bytes() bytes (host_out pinned: one hipMemcpyAsync D2H on the
    current stream; the caller synchronises before reading it).  Returns
    (k (B,H,te,D) f32, v, pos (B,te) int64) views of host_out if given, else
    of dev_out."""
    _require_device(idx, k, v, pos)
    B, H, S, D = k.shape
    te = int(idx.shape[-1])
    if idx.dim() != 2 or idx.shape[0] != B or idx.dtype != torch.int64 or tuple(v.shape) != tuple(k.shape) \
            or v.dtype != k.dtype or pos.dim() != 2 or pos.shape[0] != B or pos.dtype != torch.int64:
        raise RuntimeError("gather_evict: idx (B,te) int64, k/v (B,H,S,D) of one dtype, pos (B,S) int64")
    if idx.stride(1) != 1:
        idx = idx.contiguous()
    if pos.stride(1) != 1:
        pos = pos.contiguous()
    nbytes = int(N.lib().hc_gather_evict_bytes(B, H, te, D))
    if dev_out is None:
        dev_out = torch.empty((nbytes,), dtype=torch.uint8, device=k.device)
    if dev_out.numel() < nbytes or (host_out is not None and host_out.numel() < nbytes):
        raise RuntimeError(f"gather_evict: staging buffers need {nbytes} bytes")
    rc = N.lib().hc_gather_evict(
        N.dtype_code(k.dtype), B, H, te, D, _ptr(idx), idx.stride(0), S,
        _ptr(k), *k.stride()[:3], _ptr(v), *v.stride()[:3], _ptr(pos), pos.stride(0),
        _ptr(dev_out), _ptr(host_out), _stream_handle(k.device))
    N.check(rc, "hc_gather_evict")
    blk = host_out if host_out is not None else dev_out
    kv_elems = B * H * te * D
    f = blk[: 8 * kv_elems].view(torch.float32)
    kk = f[:kv_elems].view(B, H, te, D)
    vv = f[kv_elems:].view(B, H, te, D)
    pp = blk[8 * kv_elems: nbytes].view(torch.int64).view(B, te)
    return kk, vv, pp


def append_rows(row, k_src, k_dst, v_src=None, v_dst=None, p_src=None, p_dst=None, pos_src=None, pos_dst=None):
    """Write T new rows (B,H,T,D) at row `row` of the hot buffers."""
    _require_device(k_src, k_dst, v_src, v_dst, p_src, p_dst, pos_src, pos_dst)
    B, H, T, D = k_src.shape
    args = []
    for s, d in ((k_src, k_dst), (v_src, v_dst), (p_src, p_dst)):
        if s is None:
            args += [None, 0, 0, 0, None, 0, 0, 0]
        else:
            if tuple(s.shape) != (B, H, T, D) or d.dim() != 4 or tuple(d.shape[:2]) != (B, H) \
                    or d.shape[3] != D or d.shape[2] < row + T or d.dtype != s.dtype or d.stride(-1) != 1:
                raise RuntimeError(f"append_rows: bad shapes src {tuple(s.shape)} dst {tuple(d.shape)} row {row}")
            if s.stride(-1) != 1:
                s = s.contiguous()
            args += [_ptr(s), *_strides3(s), _ptr(d), *_strides3(d)]
    if pos_src is not None:
        if pos_src.stride(-1) != 1:
            pos_src = pos_src.contiguous()
        if pos_src.shape != (B, T) or pos_dst.dim() != 2 or pos_dst.shape[0] != B \
                or pos_dst.shape[1] < row + T or pos_dst.stride(1) != 1:
            raise RuntimeError("append_rows: bad position tensors")
    rc = N.lib().hc_append_rows(
        N.dtype_code(k_src.dtype), B, H, T, D, int(row), *args,
        _ptr(pos_src), pos_src.stride(0) if pos_src is not None else 0,
        _ptr(pos_dst), pos_dst.stride(0) if pos_dst is not None else 0,
        _stream_handle(k_src.device))
    N.check(rc, "hc_append_rows")


def inject_rerope(k_pre_f32, v_f32, pos, inv_freq, attention_scaling, k_dst, v_dst):
    """Re-RoPE staged fp32 pre-RoPE keys (B,Hk,R,D) to positions pos (B,R) or
    (B,Hk,R) and write them with their values into rows 0..R-1 of k_dst/v_dst
    (B,Hk,cap,D) in the cache dtype."""
    _require_device(k_pre_f32, v_f32, pos, inv_freq, k_dst, v_dst)
    B, Hk, R, D = k_pre_f32.shape
    if k_pre_f32.dtype != torch.float32 or v_f32.dtype != torch.float32:
        raise RuntimeError("inject_rerope: staged k_pre/v must be float32")
    if pos.dtype != torch.int64:
        raise RuntimeError("inject_rerope: positions must be int64")
    if inv_freq.dtype != torch.float32 or inv_freq.numel() != D // 2:
        raise RuntimeError("inject_rerope: inv_freq must be float32 of length D/2")
    inv_freq = inv_freq.contiguous()
    for d, name in ((k_dst, "k_dst"), (v_dst, "v_dst")):
        if d.dim() != 4 or d.shape[0] != B or d.shape[1] != Hk or d.shape[2] < R or d.shape[3] != D \
                or d.stride(-1) != 1:
            raise RuntimeError(f"inject_rerope: {name} {tuple(d.shape)} cannot hold {R} rows of ({B},{Hk},*,{D})")
    if tuple(v_f32.shape) != (B, Hk, R, D) or k_pre_f32.stride(-1) != 1 or v_f32.stride(-1) != 1:
        raise RuntimeError("inject_rerope: staged k_pre/v must be (B,Hk,R,D) with unit last stride")
    if not ((pos.dim() == 2 and tuple(pos.shape) == (B, R)) or (pos.dim() == 3 and tuple(pos.shape) == (B, Hk, R))):
        raise RuntimeError(f"inject_rerope: positions {tuple(pos.shape)} must be (B,R) or (B,Hk,R)")
    if pos.stride(-1) != 1:
        pos = pos.contiguous()
    if pos.dim() == 2:
        pos_sb, pos_sh = pos.stride(0), 0
    else:
        pos_sb, pos_sh = pos.stride(0), pos.stride(1)
    rc = N.lib().hc_inject_rerope(
        N.dtype_code(k_dst.dtype), B, Hk, R, D,
        _ptr(k_pre_f32), *_strides3(k_pre_f32),
        _ptr(v_f32), *_strides3(v_f32),
        _ptr(pos), pos_sb, pos_sh,
        _ptr(inv_freq), float(attention_scaling),
        _ptr(k_dst), *_strides3(k_dst),
        _ptr(v_dst), *_strides3(v_dst),
        _stream_handle(k_dst.device))
    N.check(rc, "hc_inject_rerope")


def rope_tables(pos, inv_freq, attention_scaling, dtype):
    """The rotary tables of LlamaRotaryEmbedding.forward at positions pos
    (N,R) int64, computed as it does (inv_freq @ pos in fp32, cos/sin of the
    duplicated frequencies, times attention_scaling, rounded to dtype) on the
    tensors' device; returns the first halves (N,R,D/2) of cos and sin."""
    pos = pos.long()
    inv = inv_freq.float()
    inv_exp = inv[None, :, None].expand(pos.shape[0], -1, 1)
    freqs = (inv_exp @ pos[:, None, :].float()).transpose(1, 2)
    emb = torch.cat((freqs, freqs), dim=-1)
    half = inv.numel()
    cos = (emb.cos() * attention_scaling).to(dtype)
    sin = (emb.sin() * attention_scaling).to(dtype)
    return cos[..., :half], sin[..., :half]


def inject_rerope_tab(k_pre, v_staged, cos_t, sin_t, k_dst, v_dst):
    """inject_rerope with the rotary tables supplied: cos_t / sin_t (B,R,D/2)
    (one table per batch row) or (B,Hk,R,D/2), in k_dst's dtype (rope_tables).
    The staged k_pre / v (B,Hk,R,D) are float32 or already in k_dst's dtype
    (the reference moves them to the model dtype before rotating,
    controller.py:368-369).  Writes the rotated keys and the values into rows
    0..R-1 of k_dst / v_dst (B,Hk,cap,D); the keys are apply_rotary_pos_emb's
    bits."""
    _require_device(k_pre, v_staged, cos_t, sin_t, k_dst, v_dst)
    B, Hk, R, D = k_pre.shape
    k_pre_f32, v_f32 = k_pre, v_staged
    if k_pre.dtype != v_staged.dtype or k_pre.dtype not in (torch.float32, k_dst.dtype):
        raise RuntimeError("inject_rerope_tab: staged k_pre/v must both be float32 or the cache dtype")
    if cos_t.dtype != k_dst.dtype or sin_t.dtype != k_dst.dtype or cos_t.shape != sin_t.shape \
            or cos_t.stride() != sin_t.stride():
        raise RuntimeError("inject_rerope_tab: cos/sin tables must share shape, strides and the cache dtype")
    if cos_t.dim() == 3 and tuple(cos_t.shape) == (B, R, D // 2):
        cs_sb, cs_sh, cs_ss = cos_t.stride(0), 0, cos_t.stride(1)
    elif cos_t.dim() == 4 and tuple(cos_t.shape) == (B, Hk, R, D // 2):
        cs_sb, cs_sh, cs_ss = cos_t.stride(0), cos_t.stride(1), cos_t.stride(2)
    else:
        raise RuntimeError(f"inject_rerope_tab: tables {tuple(cos_t.shape)} must be (B,R,D/2) or (B,Hk,R,D/2)")
    if cos_t.stride(-1) != 1:
        raise RuntimeError("inject_rerope_tab: tables need a unit last stride")
    for d, name in ((k_dst, "k_dst"), (v_dst, "v_dst")):
        if d.dim() != 4 or d.shape[0] != B or d.shape[1] != Hk or d.shape[2] < R or d.shape[3] != D \
                or d.stride(-1) != 1:
            raise RuntimeError(f"inject_rerope_tab: {name} {tuple(d.shape)} cannot hold {R} rows of ({B},{Hk},*,{D})")
    if tuple(v_f32.shape) != (B, Hk, R, D) or k_pre_f32.stride(-1) != 1 or v_f32.stride(-1) != 1:
        raise RuntimeError("inject_rerope_tab: staged k_pre/v must be (B,Hk,R,D) with unit last stride")
    rc = N.lib().hc_inject_rerope_tab(
        N.dtype_code(k_dst.dtype), B, Hk, R, D, N.dtype_code(k_pre.dtype),
        _ptr(k_pre_f32), *_strides3(k_pre_f32),
        _ptr(v_f32), *_strides3(v_f32),
        _ptr(cos_t), _ptr(sin_t), cs_sb, cs_sh, cs_ss,
        _ptr(k_dst), *_strides3(k_dst),
        _ptr(v_dst), *_strides3(v_dst),
        stream_handle(k_dst.device))
    N.check(rc, "hc_inject_rerope_tab")


def default_scaling(head_dim):
    return 1.0 / math.sqrt(head_dim)
