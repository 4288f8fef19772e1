"""KVController: cold store, look-ahead retrieval scheduling and the staged
host-to-device feed of the inject path (src/hotcold_kv/controller.py).

Cold store (controller.py:121-293).  One native store per (layer, batch
row) of cpu_buffer_size evicted tokens (pre-RoPE keys and values in fp32,
absolute positions) with an exact inner-product search over the head-mean,
pad/crop-to-faiss_dim, L2-normalised pre-RoPE key -- the same vectors the
reference puts in a faiss.IndexFlatIP.  The store, its search and the
retrieval gather are host C++ in the library (hc_cold_*): adds and searches
run without the GIL, a retrieval runs all batch rows (and heads) on host
threads.  Logical order is oldest first; the search ranks by inner product
(fp64, accumulated in dimension order), ties to the older token.  With
per_head_retrieval=True the search runs per KV head (one vector per token
and head) and positions become (B,Hk,R).

Staging (controller.py:344-442).  A retrieval result lives in pinned host
buffers; maybe_prefetch_to_gpu copies them with hipMemcpyAsync on a
library-owned non-blocking side stream (default priority) and records an
event; poll_staged_gpu queries the event without blocking, and once it has
completed orders the caller's stream after it (hipStreamWaitEvent) before
handing the device buffers to the inject kernel.  Host buffers stay
referenced until their copy is known complete.
"""

import ctypes
import math
import threading
from collections import deque

import numpy as np
import torch

from . import _native as N
from .datatypes import EvictedKV, RetrievedKV, _canon_br_2d, _canon_kv_4d


class _Ring:
    """Native cold store of one (layer, batch row) (hc_cold_*)."""

    def __init__(self, capacity, heads, head_dim, vec_dim, vec_heads, normalize=True):
        self.cap, self.H, self.D = int(capacity), int(heads), int(head_dim)
        self.vec_dim, self.vec_heads = int(vec_dim), int(vec_heads)
        self._lib = N.lib()
        self.handle = self._lib.hc_cold_create(self.cap, self.H, self.D, self.vec_dim, self.vec_heads,
                                               int(bool(normalize)))
        if not self.handle:
            N.check(N.HC_ERR_INVALID, "hc_cold_create")

    def __del__(self):
        h, self.handle = getattr(self, "handle", None), None
        if h:
            self._lib.hc_cold_destroy(h)

    def __len__(self):
        return int(self._lib.hc_cold_size(self.handle))

    @property
    def ntotal(self):
        """Vectors in the search index (faiss.Index.ntotal of the reference)."""
        return len(self)

    def add(self, kpre, v, pos, evicted_idx=None):
        """Tokens t with evicted_idx[t] >= 0 of kpre/v (H,Te,D) fp32, pos (Te,)."""
        kpre = np.ascontiguousarray(kpre, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        pos = np.ascontiguousarray(pos, dtype=np.int64)
        te = int(kpre.shape[1])
        idx = None if evicted_idx is None else np.ascontiguousarray(evicted_idx, dtype=np.int64)
        rc = self._lib.hc_cold_add(self.handle, te, kpre.ctypes.data, te * self.D, self.D,
                                   v.ctypes.data, te * self.D, self.D, pos.ctypes.data,
                                   None if idx is None else idx.ctypes.data)
        N.check(rc, "hc_cold_add")

    def search(self, q, r, head=0):
        """Logical indices of the top-r inner products with q (descending,
        ties to the older token)."""
        q = np.ascontiguousarray(q, dtype=np.float32)
        out = np.zeros((max(int(r), 0),), dtype=np.int64)
        n = ctypes.c_int64()
        N.check(self._lib.hc_cold_search(self.handle, q.ctypes.data, int(r), int(head), out.ctypes.data,
                                         ctypes.byref(n)), "hc_cold_search")
        return out[: n.value]

    def export(self):
        """The store in logical order (oldest first): kpre/v (n,H,D), pos (n,),
        vec (n,vec_heads,vec_dim)."""
        n = len(self)
        d = {"kpre": np.zeros((n, self.H, self.D), np.float32), "v": np.zeros((n, self.H, self.D), np.float32),
             "pos": np.zeros((n,), np.int64), "vec": np.zeros((n, self.vec_heads, self.vec_dim), np.float32)}
        N.check(self._lib.hc_cold_export(self.handle, d["kpre"].ctypes.data, d["v"].ctypes.data,
                                         d["pos"].ctypes.data, d["vec"].ctypes.data), "hc_cold_export")
        return d


class KVController:
    def __init__(
        self,
        max_capacity_prompt: int = 128,
        topk_ratio: float = 0.15,
        recent_size: int = 32,
        cpu_buffer_size: int = 8192,
        faiss_dim: int = 64,
        normalize_for_ip: bool = True,
        window_size: int = 16,
        query_pool_size: int = 4,
        lookahead_k: int = 32,
        hold_retrieved: bool = False,
        retrieve_after_prefill: bool = False,
        enable_asserts: bool = True,
        profile_overlap: bool = True,
        force_wait_for_prefetch_diagnostic: bool = False,
        per_head_retrieval: bool = False,
    ):
        self.max_capacity_prompt = int(max_capacity_prompt)
        self.topk_ratio = float(topk_ratio)
        self.recent_size = int(recent_size)
        self.cpu_buffer_size = int(cpu_buffer_size)
        self.faiss_dim = int(faiss_dim)
        self.normalize_for_ip = bool(normalize_for_ip)
        # retrieval period in decode steps (not the SnapKV observation window)
        self.window_size = int(window_size)
        self.query_pool_size = int(query_pool_size)
        self.lookahead_k = int(lookahead_k)
        # False: retrieved tokens are attended at the one step their copy lands;
        # True: they stay in attention until the next retrieval replaces them.
        self.hold_retrieved = bool(hold_retrieved)
        # True: one synchronous retrieval at the end of prefill.
        self.retrieve_after_prefill = bool(retrieve_after_prefill)
        self.enable_asserts = bool(enable_asserts)
        self.profile_overlap = bool(profile_overlap)
        self.force_wait_for_prefetch_diagnostic = bool(force_wait_for_prefetch_diagnostic)
        self.per_head_retrieval = bool(per_head_retrieval)

        self._inited = False
        self.B = self.Hk = self.D = self.n_layers = None
        self.rings = []
        self.step_count = []
        self.query_window = []
        self._retrieval_thread = []
        self._retrieval_lock = []
        self._retrieval_ready_cpu = []
        self._stage_lock = []
        self._staged = []
        self._stream = None
        self._evict_dev = None
        self._evict_host = None
        self.last_injected_len = 0
        self.held_mem = []

        self.dbg = {
            "compress_calls": 0,
            "evicted_tokens": 0,
            "faiss_add": 0,
            "retrieval_launched": 0,
            "retrieval_launched_prefill": 0,
            "retrieval_ready_cpu": 0,
            "retrieval_skipped_no_cold": 0,
            "retrieval_ready_empty": 0,
            "prefetch_launched": 0,
            "prefetch_ready": 0,
            "prefetch_skipped_empty": 0,
            "injection_used": 0,
            "injection_new": 0,
            "injection_skipped_no_valid": 0,
            "prefetch_copy_ms_sum": 0.0,
            "prefetch_copy_ms_count": 0,
            "prefetch_not_ready_checks": 0,
            "main_waited_for_prefetch": 0,
            "triton_decode_calls": 0,
            "triton_prefill_fallback": 0,
        }

    # -- setup ----------------------------------------------------------------------
    def _lazy_init(self, k_pre, n_layers):
        if self._inited:
            return
        B, Hk, _, D = k_pre.shape
        self.B, self.Hk, self.D = int(B), int(Hk), int(D)
        self.n_layers = L = int(n_layers)
        vec_heads = self.Hk if self.per_head_retrieval else 1
        self.rings = [[_Ring(self.cpu_buffer_size, self.Hk, self.D, self.faiss_dim, vec_heads,
                             self.normalize_for_ip) for _ in range(B)] for _ in range(L)]
        self.step_count = [0] * L
        self.query_window = [deque(maxlen=self.query_pool_size) for _ in range(L)]
        self._retrieval_thread = [None] * L
        self._retrieval_lock = [threading.Lock() for _ in range(L)]
        self._retrieval_ready_cpu = [None] * L
        self._stage_lock = [threading.Lock() for _ in range(L)]
        self._staged = [None] * L
        self.held_mem = [None] * L
        if k_pre.is_cuda:
            stream = ctypes.c_void_p()
            N.check(N.lib().hc_stream_create(ctypes.byref(stream)), "hc_stream_create")
            self._stream = stream.value
        self._inited = True

    def __del__(self):
        try:
            if self._stream is not None:
                N.lib().hc_stream_destroy(self._stream)
        except Exception:
            pass

    def evict_staging(self, device, B, H, te, D):
        """Device and pinned host staging blocks of at least
        hc_gather_evict_bytes(B, H, te, D) bytes for one eviction; grown on
        demand and reused (evictions run one at a time on the main thread)."""
        nbytes = int(N.lib().hc_gather_evict_bytes(B, H, te, D))
        if self._evict_dev is None or self._evict_dev.numel() < nbytes or self._evict_dev.device != device:
            size = max(nbytes, 2 * (self._evict_dev.numel() if self._evict_dev is not None else 0))
            self._evict_dev = torch.empty((size,), dtype=torch.uint8, device=device)
            self._evict_host = torch.empty((size,), dtype=torch.uint8, pin_memory=True)
        return self._evict_dev, self._evict_host

    @property
    def cpu_kpre_ring(self):
        """[layer][batch] rings (the reference keeps ring and index apart,
        controller.py:121-160; here one object is both)."""
        return self.rings

    @property
    def index(self):
        return self.rings

    def cold_size(self, layer_idx):
        if not self._inited:
            return 0
        return sum(len(r) for r in self.rings[int(layer_idx)])

    # -- search vectors (controller.py:166-188) -----------------------------------------
    def _pad_or_crop(self, x):
        d = x.shape[-1]
        if d > self.faiss_dim:
            return x[..., : self.faiss_dim]
        if d < self.faiss_dim:
            pad = np.zeros(x.shape[:-1] + (self.faiss_dim - d,), dtype=x.dtype)
            return np.concatenate([x, pad], axis=-1)
        return x

    def _normalize(self, x):
        if not self.normalize_for_ip:
            return x
        n = np.sqrt((x.astype(np.float64) ** 2).sum(axis=-1, keepdims=True))
        return (x / np.maximum(n, 1e-12)).astype(np.float32)

    def _k_token_to_vec_np(self, kpre_token):
        """(Hk,D) pre-RoPE key of one token -> its search vector(s), computed
        as the native store computes them: head mean (or each head) in fp64
        accumulated in head order, pad/crop, norm accumulated in dimension
        order, quotient rounded to fp32 -- bit-equal to the stored vector."""
        k = np.asarray(kpre_token.detach().cpu().float() if isinstance(kpre_token, torch.Tensor) else kpre_token,
                       dtype=np.float32)
        if self.per_head_retrieval:
            rows = [k[h].astype(np.float64) for h in range(k.shape[0])]
        else:
            acc = np.zeros(k.shape[-1], dtype=np.float64)
            for h in range(k.shape[0]):
                acc = acc + k[h].astype(np.float64)
            rows = [acc / float(k.shape[0])]
        out = []
        for x in rows:
            x = self._pad_or_crop(x)
            den = 1.0
            if self.normalize_for_ip:
                ss = 0.0
                for t in x.tolist():
                    ss += t * t
                den = max(math.sqrt(ss), 1e-12)
            out.append((x / den).astype(np.float32))
        return out[0] if not self.per_head_retrieval else np.stack(out)

    def _q_to_vecs_np(self, q_pre):
        """(B,Hq,T,D) pre-RoPE queries -> (B,faiss_dim), or (B,Hk,faiss_dim)
        per KV head: mean over heads (of the group) and rows, pad/crop, L2."""
        q = q_pre.detach()
        if self.per_head_retrieval:
            B, Hq, T, D = q.shape
            q = q.float().view(B, self.Hk, Hq // self.Hk, T, D).mean(dim=(2, 3))
        else:
            q = q.mean(dim=1).mean(dim=1)
        qn = q.float().cpu().numpy().astype(np.float32)
        return self._normalize(self._pad_or_crop(qn))

    # -- cold store -------------------------------------------------------------------------
    def add_evicted_to_cold_store(self, layer_idx, ev: EvictedKV):
        if not self._inited:
            raise RuntimeError("KVController not initialized")
        li = int(layer_idx)
        kpre = ev.k_pre_cpu.detach().cpu().float().contiguous().numpy()      # (B,Hk,Te,D)
        vv = ev.v_cpu.detach().cpu().float().contiguous().numpy()
        pos = ev.pos_cpu.detach().cpu().contiguous().numpy().astype(np.int64)
        idx = ev.evicted_idx.detach().cpu().contiguous().numpy().astype(np.int64)
        for b in range(kpre.shape[0]):
            kept = int((idx[b] >= 0).sum())
            if kept == 0:
                continue
            self.rings[li][b].add(kpre[b], vv[b], pos[b], idx[b])
            self.dbg["faiss_add"] += min(kept, self.cpu_buffer_size)
            if self.enable_asserts:
                assert len(self.rings[li][b]) <= self.cpu_buffer_size

    # -- query pooling / retrieval -----------------------------------------------------
    def update_query_window(self, layer_idx, q_pre):
        self.query_window[int(layer_idx)].append(q_pre.detach())

    def _pooled_query_np(self, layer_idx):
        qwin = self.query_window[int(layer_idx)]
        if len(qwin) == 0:
            return None
        return self._q_to_vecs_np(torch.cat(list(qwin), dim=2))

    def _retrieval_worker(self, layer_idx, q_vecs):
        """Top-lookahead_k tokens per batch row (or per KV head) into pinned
        host buffers (controller.py:250-293), one native call over all rows."""
        li = int(layer_idx)
        if not self._inited:
            return
        B, Hk, D, R = self.B, self.Hk, self.D, self.lookahead_k
        pin = torch.cuda.is_available()
        kpre = torch.empty((B, Hk, R, D), dtype=torch.float32, pin_memory=pin)
        vv = torch.empty((B, Hk, R, D), dtype=torch.float32, pin_memory=pin)
        pshape = (B, Hk, R) if self.per_head_retrieval else (B, R)
        pos = torch.empty(pshape, dtype=torch.int64, pin_memory=pin)
        valid = torch.empty(pshape, dtype=torch.bool, pin_memory=pin)
        q = np.ascontiguousarray(q_vecs, dtype=np.float32).reshape(B, -1, self.faiss_dim)
        stores = (ctypes.c_void_p * B)(*[self.rings[li][b].handle for b in range(B)])
        N.check(N.lib().hc_cold_retrieve(stores, B, q.ctypes.data, q.shape[1] * self.faiss_dim, self.faiss_dim, R,
                                         int(self.per_head_retrieval), kpre.data_ptr(), vv.data_ptr(),
                                         pos.data_ptr(), valid.data_ptr(), 0), "hc_cold_retrieve")
        with self._retrieval_lock[li]:
            if not bool(valid.any()):
                self._retrieval_ready_cpu[li] = None
                self.dbg["retrieval_ready_empty"] += 1
                return
            self._retrieval_ready_cpu[li] = (kpre, vv, pos, valid)
            self.dbg["retrieval_ready_cpu"] += 1

    def launch_retrieval_now(self, layer_idx, q_pre):
        """One synchronous retrieval outside the schedule (controller.py:295-312)."""
        if self.lookahead_k <= 0 or not self._inited:
            return
        li = int(layer_idx)
        if self.cold_size(li) == 0:
            self.dbg["retrieval_skipped_no_cold"] += 1
            return
        self._retrieval_worker(li, self._q_to_vecs_np(q_pre))
        self.dbg["retrieval_launched"] += 1
        self.dbg["retrieval_launched_prefill"] += 1

    def maybe_launch_async_retrieval(self, layer_idx):
        """Every window_size calls, start a background search with the pooled
        recent queries (controller.py:314-342)."""
        if self.lookahead_k <= 0:
            return
        li = int(layer_idx)
        self.step_count[li] += 1
        if self.step_count[li] % self.window_size != 0:
            return
        if not self._inited:
            return
        if self.cold_size(li) == 0:
            self.dbg["retrieval_skipped_no_cold"] += 1
            return
        q_vecs = self._pooled_query_np(li)
        if q_vecs is None:
            return
        with self._retrieval_lock[li]:
            th = self._retrieval_thread[li]
            if th is not None and th.is_alive():
                return
            th = threading.Thread(target=self._retrieval_worker, args=(li, q_vecs), daemon=True)
            self._retrieval_thread[li] = th
            th.start()
            self.dbg["retrieval_launched"] += 1

    def wait_for_retrieval(self, layer_idx, timeout=None):
        """Join the layer's background search, if any (test and shutdown helper)."""
        th = self._retrieval_thread[int(layer_idx)] if self._inited else None
        if th is not None:
            th.join(timeout)

    # -- staging ------------------------------------------------------------------------------
    def _event(self, timing):
        ev = ctypes.c_void_p()
        N.check(N.lib().hc_event_create(ctypes.byref(ev), int(timing)), "hc_event_create")
        return ev.value

    def maybe_prefetch_to_gpu(self, layer_idx, device, dtype=None):
        """Start the host-to-device copy of a finished retrieval on the side
        stream (controller.py:344-380).  dtype is accepted for compatibility:
        staged buffers stay fp32 and the inject kernel converts."""
        li = int(layer_idx)
        device = torch.device(device)
        if device.type != "cuda" or self._stream is None:
            return
        with self._retrieval_lock[li]:
            pack = self._retrieval_ready_cpu[li]
            self._retrieval_ready_cpu[li] = None
        if pack is None:
            return
        kpre, vv, pos, valid = pack
        lib = N.lib()
        dev = [torch.empty(t.shape, dtype=t.dtype, device=device) for t in pack]
        t0 = self._event(1) if self.profile_overlap else None
        t1 = self._event(1) if self.profile_overlap else None
        ready = self._event(0)
        if t0 is not None:
            N.check(lib.hc_event_record(t0, self._stream), "hc_event_record")
        for d, h in zip(dev, pack):
            N.check(lib.hc_memcpy_h2d_async(d.data_ptr(), h.data_ptr(), h.numel() * h.element_size(), self._stream),
                    "hc_memcpy_h2d_async")
        if t1 is not None:
            N.check(lib.hc_event_record(t1, self._stream), "hc_event_record")
        N.check(lib.hc_event_record(ready, self._stream), "hc_event_record")
        with self._stage_lock[li]:
            old = self._staged[li]
            self._staged[li] = dict(dev=dev, host=pack, ready=ready, t0=t0, t1=t1)
            self.dbg["prefetch_launched"] += 1
        if old is not None:
            self._release(old, wait=True)

    def _release(self, st, wait=False):
        lib = N.lib()
        if wait:
            while lib.hc_event_query(st["ready"]) == 0:
                pass
        for key in ("ready", "t0", "t1"):
            if st.get(key) is not None:
                lib.hc_event_destroy(st[key])
                st[key] = None

    def poll_staged_gpu(self, layer_idx) -> RetrievedKV:
        """Non-blocking check for a staged retrieval (controller.py:382-442)."""
        li = int(layer_idx)
        empty = RetrievedKV(k_pre=torch.empty(0), v=torch.empty(0), pos=torch.empty(0, dtype=torch.long),
                            valid=torch.empty(0, dtype=torch.bool), ready=False)
        if not self._inited or self._stream is None:
            return empty
        lib = N.lib()
        with self._stage_lock[li]:
            st = self._staged[li]
            if st is None:
                return empty
            done = lib.hc_event_query(st["ready"])
            if done < 0:
                N.check(done, "hc_event_query")
            if done == 0:
                self.dbg["prefetch_not_ready_checks"] += 1
                if not self.force_wait_for_prefetch_diagnostic:
                    return empty
                self.dbg["main_waited_for_prefetch"] += 1
                while lib.hc_event_query(st["ready"]) == 0:
                    pass
            self._staged[li] = None
            self.dbg["prefetch_ready"] += 1
        # the copy has completed; order the consumer stream after it anyway
        cur = torch.cuda.current_stream(st["dev"][0].device).cuda_stream
        N.check(lib.hc_stream_wait_event(cur, st["ready"]), "hc_stream_wait_event")
        if self.profile_overlap and st["t0"] is not None:
            ms = ctypes.c_float()
            if lib.hc_event_elapsed_ms(st["t0"], st["t1"], ctypes.byref(ms)) == 0:
                self.dbg["prefetch_copy_ms_sum"] += float(ms.value)
                self.dbg["prefetch_copy_ms_count"] += 1
        self._release(st)
        kpre, vv, pos, valid = st["dev"]
        valid = valid.view(torch.bool)
        kpre = _canon_kv_4d(kpre, "staged.k_pre")
        vv = _canon_kv_4d(vv, "staged.v")
        if not self.per_head_retrieval:
            pos = _canon_br_2d(pos, "staged.pos")
            valid = _canon_br_2d(valid, "staged.valid")
        return RetrievedKV(k_pre=kpre, v=vv, pos=pos, valid=valid, ready=True)
