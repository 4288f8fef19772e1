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

Staging (controller.py:344-442).  Each layer owns a few reusable staging
slots (pinned host buffers, device buffers and events, allocated once): the
retrieval worker fills a free slot's host buffers; maybe_prefetch_to_gpu
copies them with hipMemcpyAsync on a library-owned non-blocking side stream
(default priority) and records the slot's event; poll_staged_gpu queries the
event without blocking, and once it has completed orders the caller's stream
after it (hipStreamWaitEvent) before the inject kernel reads the slot.  A
slot whose data the held slot still uses is not refilled: when a newer
retrieval is injected, an event recorded on the consumer stream marks the
old slot free, and the side stream waits for it before copying into it
again.  A staging superseded before it was polled is recycled once its copy
is known complete; nothing waits on the host.
"""

import ctypes
import math
import os
import threading
from collections import deque

import numpy as np
import torch

from . import _native as N
from .datatypes import EvictedKV, RetrievedKV, _canon_br_2d, _canon_kv_4d
from .device_index import DeviceIndex
from .ops import rope_tables as ops_rope_tables
from .ops import stream_handle as ops_stream


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

    def add_async(self, kpre, v, pos, evicted_idx=None, nthreads=0, workers=4):
        """add() as a job on the library's worker threads (hc_cold_add_async):
        returns a _Job once submitted.  Adds apply in submission order, and
        size, searches and later adds wait for the ones submitted before them.
        The job keeps the arrays it reads alive until it is collected."""
        kpre = np.ascontiguousarray(kpre, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        pos = np.ascontiguousarray(pos, dtype=np.int64)
        te = int(kpre.shape[1])
        idx = None if evicted_idx is None else np.ascontiguousarray(evicted_idx, dtype=np.int64)
        h = self._lib.hc_cold_add_async(self.handle, te, kpre.ctypes.data, te * self.D, self.D,
                                        v.ctypes.data, te * self.D, self.D, pos.ctypes.data,
                                        None if idx is None else idx.ctypes.data, None, int(nthreads), int(workers))
        if not h:
            N.check(N.HC_ERR_INVALID, "hc_cold_add_async")
        return _Job(h, None, False, (kpre, v, pos, idx))

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


def _block_layout(specs, align=256):
    """Byte offsets of tensors of the given (shape, dtype) packed into one
    block, each start aligned to `align`; returns (offsets, ends): the byte
    just past each tensor."""
    offs, off = [], 0
    ends = []
    for shape, dt in specs:
        off = (off + align - 1) // align * align
        offs.append(off)
        off += int(np.prod(shape)) * torch.empty((), dtype=dt).element_size()
        ends.append(off)
    return offs, ends


def _carve(block, specs):
    """Views of the given (shape, dtype) into a uint8 block laid out by
    _block_layout."""
    offs, _ = _block_layout(specs)
    out = []
    for (shape, dt), off in zip(specs, offs):
        n = int(np.prod(shape)) * torch.empty((), dtype=dt).element_size()
        out.append(block[off:off + n].view(dt).view(shape))
    return tuple(out)


class _Slot:
    """One reusable staging slot of a layer: pinned host buffers (k_pre, v,
    pos, valid, and the rotary tables: per row cos then sin), all views of
    one pinned block so that a retrieval goes over in one copy; its device
    twin block; the events of its copy."""

    FREE, FILLING, RETRIEVED, COPYING, STAGED, HELD = range(6)

    def __init__(self, host, tab=None, block=None, nbytes=(0, 0), qhost=None, hits_host=None):
        self.host = host            # (kpre, v, pos, valid) pinned host tensors
        self.tab = tab              # pinned rotary tables at pos, (B,Hc,R,2,D/2) cache dtype: [..., 0, :] cos, 1 sin
        self.tab_host = None if tab is None else (tab[..., 0, :], tab[..., 1, :])
        self.block = block          # the one pinned allocation host and tab_host are views of
        self.nbytes = nbytes        # bytes of the block without / with the tables
        self.tab_dev = None
        self.has_tab = False        # the tables were computed for this retrieval
        self.qhost = qhost          # pinned pooled query of the search it serves, (B,VH,D) fp32
        self.qdev = None            # its device twin, written by the pooling kernel
        self.q_ready = None         # event behind the query's copy
        self.hits_host = hits_host  # pinned hits of a device search, (B,VH,R) int64 logical indices
        self.hits_dev = None        # their device twin, written by the search kernel
        self.hits_ready = None      # event behind the hits' device-to-host copy
        self.dev = None             # device twins, allocated on the first copy
        self.dev_block = None       # the device allocation they are views of
        self.state = _Slot.FREE
        self.ready = None           # event recorded behind the copy
        self.copied = False         # ready has been recorded (a copy was issued)
        self.t0 = self.t1 = None    # timing events (profile_overlap)
        self.free_after = None      # consumer-stream event: the slot's last reader is done
        self.released = False       # free_after has been recorded


class _Job:
    """A search running on the library's native worker threads
    (hc_cold_retrieve_async): the handle the reference keeps as a
    threading.Thread.  It holds the buffers the search reads and writes until
    the decode thread collects it."""

    def __init__(self, handle, slot, has_tab, keep, by_hits=False):
        self.handle, self.slot, self.has_tab, self.keep = handle, slot, has_tab, keep
        self.by_hits = by_hits      # a gather of device-ranked hits (hc_cold_gather_async)
        self._lib = N.lib()         # held: __del__ may run after module teardown
        self.result = None          # (n_valid, positions past the table) once done
        self.error = None           # (status, message) if the search failed

    def poll(self, wait=False):
        """True once the search is done (or failed: see error)."""
        if self.result is None:
            nv, miss = ctypes.c_int64(0), ctypes.c_int64(0)
            lib = self._lib
            rc = lib.hc_cold_job_poll(self.handle, int(wait), ctypes.byref(nv), ctypes.byref(miss))
            if rc == 0:
                return False
            if rc < 0:
                self.error = (rc, lib.hc_last_error().decode(errors="replace"))
            lib.hc_cold_job_free(self.handle)
            self.handle = None
            self.result = (nv.value, miss.value)
        return True

    def is_alive(self):
        return not self.poll()

    def join(self, timeout=None):
        self.poll(wait=True)

    def __del__(self):
        h, self.handle = getattr(self, "handle", None), None
        if h:
            self._lib.hc_cold_job_free(h)     # waits for the worker to finish with the buffers


_NOT_READY = RetrievedKV(k_pre=torch.empty(0), v=torch.empty(0), pos=torch.empty(0, dtype=torch.long),
                         valid=torch.empty(0, dtype=torch.bool), ready=False)


class _EvictStage:
    """One eviction's device and pinned host staging blocks, and the cold-store
    add jobs still reading the host block."""

    def __init__(self, dev, host):
        self.dev, self.host, self.jobs = dev, host, []

    def done(self, wait=False):
        """True once no add reads the host block; a failed add raises here."""
        pending, err = [], None
        for j in self.jobs:
            if not j.poll(wait=wait):
                pending.append(j)
            elif j.error is not None and err is None:
                err = j.error
        self.jobs = pending
        if err is not None:
            raise N.HotColdError(f"hc_cold_add (worker): {err[1]} (status {err[0]})")
        return not pending


class KVController:
    # staging slots per layer: one held, one in copy, one retrieved, one filling
    MAX_SLOTS = 4
    # Eviction staging blocks: the prefill's cold-store adds run as native jobs
    # while the next layer proceeds; a third eviction waits for the oldest.
    MAX_EVICT_STAGES = 2
    ADD_THREADS = 8
    # Scheduled searches run as jobs on the library's native worker threads
    # (no Python, no thread per search), each on SEARCH_THREADS host threads:
    # every layer searches in the same decode step, and together they keep to
    # about half of the cores (at most 12 threads, within a 16-core share), so
    # the decode thread is not starved of CPU.  With 4 workers a 32-layer 16k
    # loop at 0.6 ms per step skipped 1-8 of 256 searches whose predecessor
    # was still running; with 6, 0-3.
    SEARCH_THREADS = 2
    MAX_SEARCH_WORKERS = 6
    # The device search indexes are made only when they take at most this
    # share of the device's free memory (the model's activations need the
    # rest); otherwise the host stores search.
    DEVICE_INDEX_MAX_FREE_FRACTION = 0.5

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
        device_search: bool = True,
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
        # True: with the hot tier on a GPU, each layer's search vectors are
        # also kept in HBM (DeviceIndex) and the scheduled searches rank them
        # there; the host stores then only gather the hits' rows.  A layer
        # whose index cannot follow its store (an add without a staging stage)
        # goes back to the host search.
        self.device_search = bool(device_search)

        self._inited = False
        self.B = self.Hk = self.D = self.n_layers = None
        self.dtype = None
        self._device = None         # the device of the hot tier (from the first k_pre)
        self._rope = None           # (inv_freq fp32 CPU, attention_scaling) of the model's rotary module
        self._rope_tab = None       # byte rows [position][cos | sin] of the rotary tables (_rope_rows)
        self._max_pos = 0           # largest position in any cold store
        self.rings = []
        self.step_count = []
        self.query_window = []
        self._retrieval_thread = []
        self._retrieval_lock = []
        self._retrieval_ready_cpu = []
        self._stage_lock = []
        self._staged = []
        self._slots = []
        self._held_slot = []
        self._stream = None
        self._evict_stages = []
        self._dindex = []           # per layer: DeviceIndex, or None (host search)
        self._search_stream = None  # side stream of the device searches
        self._search_done = []      # per layer: event behind its last device search
        self._pending_search = []   # (layer, slot, index) of device searches scheduled this step
        self._flush_event = None    # decode-stream event the step's device searches wait for
        self.last_injected_len = 0
        self.held_mem = []

        self.dbg = {
            "compress_calls": 0,
            "evicted_tokens": 0,
            "faiss_add": 0,
            "retrieval_launched": 0,
            "retrieval_launched_prefill": 0,
            "retrieval_device": 0,
            "device_index_dropped": 0,
            "device_index_too_large": 0,
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
            "rope_rows_direct": 0,
            "prefetch_not_ready_checks": 0,
            "retrieval_skipped_no_slot": 0,
            "prefetch_superseded": 0,
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
        self.dtype = k_pre.dtype
        self._device = k_pre.device
        self.n_layers = L = int(n_layers)
        vec_heads = self.Hk if self.per_head_retrieval else 1
        self.rings = [[_Ring(self.cpu_buffer_size, self.Hk, self.D, self.faiss_dim, vec_heads,
                             self.normalize_for_ip) for _ in range(B)] for _ in range(L)]
        self._store_ptrs = [(ctypes.c_void_p * B)(*[r.handle for r in rings]) for rings in self.rings]
        self.step_count = [0] * L
        self.query_window = [deque(maxlen=self.query_pool_size) for _ in range(L)]
        self._retrieval_thread = [None] * L
        self._retrieval_lock = [threading.Lock() for _ in range(L)]
        self._retrieval_ready_cpu = [None] * L
        self._stage_lock = [threading.Lock() for _ in range(L)]
        self._staged = [None] * L
        self._slots = [[] for _ in range(L)]
        self._held_slot = [None] * L
        self.held_mem = [None] * L
        self._dindex = [None] * L
        self._search_done = [None] * L
        if k_pre.is_cuda:
            stream = ctypes.c_void_p()
            N.check(N.lib().hc_stream_create(ctypes.byref(stream)), "hc_stream_create")
            self._stream = stream.value
            if self.device_search and self.lookahead_k > 0:
                self._create_device_indexes()
        self._inited = True
        if k_pre.is_cuda:
            self._preallocate_slots()

    def _create_device_indexes(self):
        """One DeviceIndex per layer (vectors of every row's store, capacity
        cpu_buffer_size, fp32 and an fp16 copy: 6 bytes per dimension per
        slot) with one key scratch for all (12 bytes per slot), and the
        search stream; or none at all when they do not fit the device's
        memory or the search kernels' limits."""
        vh = self.Hk if self.per_head_retrieval else 1
        if self.B > 64 or self.faiss_dim > 1024 or self.faiss_dim % 4 or self.lookahead_k > 1024:
            return
        capT = (self.cpu_buffer_size + 63) // 64 * 64
        need = self.n_layers * self.B * vh * capT * (6 * self.faiss_dim) + self.B * vh * capT * 12
        free = torch.cuda.mem_get_info(self._device)[0]
        if need > self.DEVICE_INDEX_MAX_FREE_FRACTION * free:
            self.dbg["device_index_too_large"] = 1
            return
        try:
            # every search runs on the one search stream, so the layers share
            # one key scratch
            scratch = DeviceIndex.scratch_for(self.B, vh, capT, self._device)
            self._dindex = [DeviceIndex(self.B, self.Hk, self.D, self.faiss_dim, vh, self.cpu_buffer_size,
                                        self._device, self.normalize_for_ip, scratch=scratch)
                            for _ in range(self.n_layers)]
        except torch.OutOfMemoryError:
            self._dindex = [None] * self.n_layers
            return
        stream = ctypes.c_void_p()
        N.check(N.lib().hc_stream_create(ctypes.byref(stream)), "hc_stream_create")
        self._search_stream = stream.value
        # the host stores need no search vectors while the device ranks; a
        # host search (after an index is dropped) computes them first
        for rings in self.rings:
            for r in rings:
                N.check(N.lib().hc_cold_defer_vectors(r.handle, 1), "hc_cold_defer_vectors")

    def _drop_device_index(self, li):
        """The layer goes back to the host search (its store took an add the
        device index did not see)."""
        if self._dindex and self._dindex[li] is not None:
            self._dindex[li] = None
            self.dbg["device_index_dropped"] += 1

    def _preallocate_slots(self, n=2):
        """n staging slots per layer up front (one held, one in flight):
        pinned allocations are slow and would otherwise land in decode steps."""
        if self.lookahead_k <= 0:
            return
        for li in range(self.n_layers):
            with self._retrieval_lock[li]:
                for sl in [self._take_slot(li) for _ in range(n - len(self._slots[li]))]:
                    sl.state = _Slot.FREE

    def __del__(self):
        try:
            for th in self._retrieval_thread:
                if isinstance(th, _Job):
                    th.join()                   # a search still writing into a slot's buffers
            for st in getattr(self, "_evict_stages", ()):
                for j in st.jobs:
                    j.join()                    # an add still reading a stage's host block
            lib = N.lib()
            for slots in self._slots:
                for sl in slots:
                    for ev in (sl.ready, sl.t0, sl.t1, sl.free_after, sl.q_ready, sl.hits_ready):
                        if ev is not None:
                            lib.hc_event_destroy(ev)
            if self._flush_event is not None:
                lib.hc_event_destroy(self._flush_event)
            for s in (self._stream, self._search_stream):
                if s is not None:
                    lib.hc_stream_destroy(s)
        except Exception:
            pass

    def set_rope(self, inv_freq, attention_scaling):
        """The model's rotary parameters (LlamaRotaryEmbedding.inv_freq and
        attention_scaling): with them every retrieval carries the rotary
        tables of its positions, computed on the search thread, and the inject
        writes apply_rotary_pos_emb's exact bits."""
        self._rope = (inv_freq.detach().float().cpu().contiguous(), float(attention_scaling))
        self._rope_tab = None

    def _rope_rows(self):
        """The rotary tables of every position up to the largest one in the
        cold store, as byte rows [position][cos | sin] (D/2 values each, the
        cache dtype), or None without set_rope.  Computed on the calling
        (decode) thread as LlamaRotaryEmbedding.forward computes them, and
        regrown by doubling when the store reaches past them; the search
        threads only gather rows."""
        if self._rope is None or self.dtype is None:
            return None
        need = self._max_pos + 1
        if self._rope_tab is None or self._rope_tab.shape[0] < need:
            rows = max(4096, 2 * (self._rope_tab.shape[0] if self._rope_tab is not None else 0))
            while rows < need:
                rows *= 2
            cos, sin = ops_rope_tables(torch.arange(rows, dtype=torch.int64).view(1, rows), self._rope[0],
                                       self._rope[1], self.dtype)
            tab = torch.stack([cos[0], sin[0]], dim=1).contiguous()                 # (rows, 2, D/2)
            self._rope_tab_t = tab                                                  # owns the bytes below
            self._rope_tab = tab.view(torch.uint8).numpy().reshape(rows, -1)
        return self._rope_tab

    def evict_stage(self, device, B, H, te, D):
        """A staging stage (device and pinned host blocks of at least
        hc_gather_evict_bytes(B, H, te, D) bytes) that no cold-store add is
        reading: a free one, a new one while there are fewer than
        MAX_EVICT_STAGES, else the least recently handed out once its adds are
        done (grown if needed)."""
        nbytes = int(N.lib().hc_gather_evict_bytes(B, H, te, D))
        device = torch.device(device)
        for st in self._evict_stages:
            if st.dev.device == device and st.dev.numel() >= nbytes and st.done():
                self._evict_stages.remove(st)
                self._evict_stages.append(st)
                return st
        if len(self._evict_stages) < self.MAX_EVICT_STAGES:
            st = _EvictStage(*self._stage_blocks(device, nbytes))
        else:
            st = self._evict_stages.pop(0)
            st.done(wait=True)
            if st.dev.device != device or st.dev.numel() < nbytes:
                st.dev, st.host = self._stage_blocks(device, max(nbytes, 2 * st.dev.numel()))
        self._evict_stages.append(st)
        return st

    def _stage_blocks(self, device, nbytes):
        """A device block and a pinned host block of nbytes each."""
        return (torch.empty((nbytes,), dtype=torch.uint8, device=device),
                torch.empty((nbytes,), dtype=torch.uint8, pin_memory=True))

    def evict_staging(self, device, B, H, te, D):
        """(device, pinned host) blocks of a free staging stage (evict_stage)."""
        st = self.evict_stage(device, B, H, te, D)
        return st.dev, st.host

    def wait_cold_adds(self):
        """Wait for every cold-store add still running (raises a failed one's error)."""
        for st in self._evict_stages:
            st.done(wait=True)

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
        """x / max(||x||, 1e-12) over the last axis, the squares summed in
        fp64 in dimension order and the quotient rounded to fp32: the
        arithmetic of the stored vectors and of hc_cold_retrieve's query
        normalisation."""
        if not self.normalize_for_ip:
            return x
        x64 = np.asarray(x, dtype=np.float64)
        ss = np.zeros(x64.shape[:-1], dtype=np.float64)
        for d in range(x64.shape[-1]):
            ss = ss + x64[..., d] * x64[..., d]
        return (x64 / np.maximum(np.sqrt(ss), 1e-12)[..., None]).astype(np.float32)

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
    def add_evicted_to_cold_store(self, layer_idx, ev: EvictedKV, stage=None):
        """Add one eviction's tokens to the layer's cold stores
        (controller.py:178-188).  With stage (the _EvictStage whose host block
        ev's tensors view) the adds run as native jobs and the stage stays
        busy until they are done; without, they complete before returning."""
        if not self._inited:
            raise RuntimeError("KVController not initialized")
        li = int(layer_idx)
        kpre = ev.k_pre_cpu.detach().cpu().float().contiguous().numpy()      # (B,Hk,Te,D)
        vv = ev.v_cpu.detach().cpu().float().contiguous().numpy()
        pos = ev.pos_cpu.detach().cpu().contiguous().numpy().astype(np.int64)
        idx = ev.evicted_idx.detach().cpu().contiguous().numpy().astype(np.int64)
        if pos.size:
            self._max_pos = max(self._max_pos, int(pos.max()))
            if self._rope is not None:
                self._rope_rows()       # extend the rotary tables now (prefill), not in a decode step
        if self._dindex and self._dindex[li] is not None:
            self._index_add(li, ev, stage, idx)
        for b in range(kpre.shape[0]):
            kept = int((idx[b] >= 0).sum())
            if kept == 0:
                continue
            if stage is None:
                self.rings[li][b].add(kpre[b], vv[b], pos[b], idx[b])
            else:
                stage.jobs.append(self.rings[li][b].add_async(kpre[b], vv[b], pos[b], idx[b],
                                                              nthreads=self.ADD_THREADS,
                                                              workers=self._search_workers()))
            self.dbg["faiss_add"] += min(kept, self.cpu_buffer_size)
            if self.enable_asserts:
                assert len(self.rings[li][b]) <= self.cpu_buffer_size

    def _index_add(self, li, ev, stage, idx):
        """The eviction's search vectors into the layer's device index, from
        the stage's device block (the twin of the host block ev's tensors
        view), on the current stream after the layer's last device search
        (which may still read the ring slots this add overwrites).  First the
        layer's device search is settled: its gather addresses the host
        stores by the logical indices ranked before this add.  Without such a
        block the layer goes back to the host search."""
        self._settle_search(li)
        B, H, te, D = ev.k_pre_cpu.shape
        if stage is None or stage.dev.device.type != "cuda" or ev.k_pre_cpu.data_ptr() != stage.host.data_ptr() \
                or stage.dev.numel() < 4 * B * H * te * D:
            self._drop_device_index(li)
            return
        kdev = stage.dev[:4 * B * H * te * D].view(torch.float32).view(B, H, te, D)
        stream = ops_stream(kdev.device)
        if self._search_done[li] is not None:
            N.check(N.lib().hc_stream_wait_event(stream, self._search_done[li]), "hc_stream_wait_event")
        self._dindex[li].add(kdev, idx, stream=stream)

    # -- query pooling / retrieval -----------------------------------------------------
    def update_query_window(self, layer_idx, q_pre):
        self.query_window[int(layer_idx)].append(q_pre.detach() if q_pre.requires_grad else q_pre)

    def _pooled_query_dev(self, layer_idx):
        """The pooled recent pre-RoPE query on the device, fp32: (B,D), or
        (B,Hk,D) per KV head (the means of _q_to_vecs_np before pad/crop and
        normalisation)."""
        q = torch.cat(list(self.query_window[int(layer_idx)]), dim=2)
        if self.per_head_retrieval:
            B, Hq, T, D = q.shape
            return q.float().view(B, self.Hk, Hq // self.Hk, T, D).mean(dim=(2, 3))
        return q.mean(dim=1).mean(dim=1).float()

    def _stage_query(self, layer_idx, slot, to_host=True):
        """Pool the window's queries on the device into the slot's query
        buffer (hc_retrieval_query: the pooling kernel, on the current
        stream, no host wait); to_host: also copy it to the slot's pinned
        buffer and record the slot's event behind the copy.  Windows of more
        query rows than the kernel takes (hc_retrieval_query_max_rows), or of
        mixed dtypes, are pooled by torch (_pooled_query_dev) instead."""
        win = list(self.query_window[int(layer_idx)])
        q0 = win[0]
        B, Hq, _, D = q0.shape
        if slot.qdev is None:
            self._alloc_dev(slot, q0.device)
        if slot.q_ready is None and to_host:
            slot.q_ready = self._event(0)
        stream = ops_stream(q0.device)
        rows = [(t, r) for t in win for r in range(t.shape[2])]
        if len(rows) <= N.lib().hc_retrieval_query_max_rows() and all(
                t.dtype == q0.dtype and t.shape[:2] == q0.shape[:2] and t.shape[3] == D and t.stride(3) == 1
                and t.is_cuda for t in win):
            es = q0.element_size()
            n = len(rows)
            ptrs = (ctypes.c_void_p * n)(*[t.data_ptr() + r * t.stride(2) * es for t, r in rows])
            sb = (ctypes.c_int64 * n)(*[t.stride(0) for t, _ in rows])
            sh = (ctypes.c_int64 * n)(*[t.stride(1) for t, _ in rows])
            N.check(N.lib().hc_retrieval_query(N.dtype_code(q0.dtype), B, Hq, self.Hk, D, n, ptrs, sb, sh,
                                               int(self.per_head_retrieval), slot.qdev.data_ptr(),
                                               slot.qhost.data_ptr() if to_host else None,
                                               slot.q_ready if to_host else None, stream), "hc_retrieval_query")
            return
        vh = self.Hk if self.per_head_retrieval else 1
        slot.qdev.copy_(self._pooled_query_dev(layer_idx).reshape(B, vh, D))
        if to_host:
            slot.qhost.copy_(slot.qdev, non_blocking=True)
            N.check(N.lib().hc_event_record(slot.q_ready, stream), "hc_event_record")

    def _wait_event(self, ev):
        N.check(N.lib().hc_event_synchronize(ev), "hc_event_synchronize")

    def _pooled_query_np(self, layer_idx):
        qwin = self.query_window[int(layer_idx)]
        if len(qwin) == 0:
            return None
        return self._q_to_vecs_np(torch.cat(list(qwin), dim=2))

    # -- staging slots ------------------------------------------------------------------
    def _slot_specs(self):
        """(shape, dtype) of a slot's k_pre, v, pos, valid, rotary tables,
        pooled query and device-search hits: the order of their views in the
        slot's one block.  A retrieval copies a prefix of the block: through
        the flags without tables, through the tables with them; the pooled
        query and the hits, last, only travel device to host."""
        B, Hk, D, R = self.B, self.Hk, self.D, self.lookahead_k
        vh = Hk if self.per_head_retrieval else 1
        pshape = (B, Hk, R) if self.per_head_retrieval else (B, R)
        tshape = (B, vh, R, 2, D // 2)
        kv = self._kv_dtype()
        return (((B, Hk, R, D), kv), ((B, Hk, R, D), kv), (pshape, torch.int64),
                (pshape, torch.bool), (tshape, self.dtype), ((B, vh, D), torch.float32), ((B, vh, R), torch.int64))

    def _kv_dtype(self):
        """Element type of the staged k_pre / v: the cache dtype when it is
        fp16 or bf16 (the reference moves retrieved rows to the model dtype
        on their copy, controller.py:368-369; the native retrieval rounds
        them the same way, so the copy carries half the bytes), else fp32."""
        return self.dtype if self.dtype in (torch.float16, torch.bfloat16) else torch.float32

    def _take_slot(self, li):
        """A free slot of layer li whose last copy has completed (its host
        buffers may be overwritten), marked FILLING; None if all are busy.
        Called with the layer's retrieval lock held."""
        for sl in self._slots[li]:
            if sl.state == _Slot.FREE and (not sl.copied or self._event_done(sl.ready)):
                sl.state = _Slot.FILLING
                return sl
        if len(self._slots[li]) >= self.MAX_SLOTS:
            return None
        specs = self._slot_specs()
        ends = _block_layout(specs)[1]
        block = torch.empty(ends[-1], dtype=torch.uint8, pin_memory=torch.cuda.is_available())
        views = _carve(block, specs)
        sl = _Slot(views[:4], views[4], block, (ends[3], ends[4]), views[5], views[6])
        if self._device is not None and self._device.type == "cuda":
            self._alloc_dev(sl, self._device)
        sl.state = _Slot.FILLING
        self._slots[li].append(sl)
        return sl

    def _retrieval_worker(self, layer_idx, q_vecs, slot=None, nthreads=0, table=None):
        """Top-lookahead_k tokens per batch row (or per KV head) into a slot's
        pinned host buffers (controller.py:250-293), one native call over all
        rows, on the calling thread.  q_vecs None: the slot's pooled query is
        still being copied to the host; wait for it here, and normalise it in
        the native call.  table: the rotary tables by position (_rope_rows),
        gathered into the slot for the inject.  Returns False when no search
        ran (no free slot, not initialised)."""
        li = int(layer_idx)
        if not self._inited:
            return False
        if slot is None:
            with self._retrieval_lock[li]:
                slot = self._take_slot(li)
            if slot is None:
                self.dbg["retrieval_skipped_no_slot"] += 1
                return False
        dindex = self._dindex[li] if self._dindex else None
        if q_vecs is not None and dindex is not None:
            return self._device_retrieval_now(li, slot, dindex, q_vecs, table, nthreads)
        if q_vecs is None:
            self._wait_event(slot.q_ready)
        args, keep, tab = self._search_args(li, slot, q_vecs, table, nthreads)
        missing = ctypes.c_int64(0)
        N.check(N.lib().hc_cold_retrieve(*args[:-1], ctypes.byref(missing), args[-1]), "hc_cold_retrieve")
        self._finish_retrieval(li, slot, tab, int(slot.host[3].sum()), missing.value)
        return True

    def _device_retrieval_now(self, li, slot, dindex, q_vecs, table, nthreads):
        """_retrieval_worker on the layer's device index: the host query
        vectors (already in search form) ranked by the exact device scan, then
        the hits' rows gathered from the host stores on the calling thread
        (hc_cold_gather) -- the rows hc_cold_retrieve would write, and the
        host stores keep deferring their vectors.  The scan runs on the
        search stream (the layers share its key scratch), after the current
        stream's work, and is waited for."""
        self._settle_search(li)
        q = torch.from_numpy(np.ascontiguousarray(q_vecs, dtype=np.float32).reshape(self.B, -1, self.faiss_dim))
        q = q.to(self._device)
        if self._flush_event is None:
            self._flush_event = self._event(0)
        if slot.hits_ready is None:
            slot.hits_ready = self._event(0)
        N.check(N.lib().hc_event_record(self._flush_event, ops_stream(self._device)), "hc_event_record")
        dindex.search(q, self.lookahead_k, slot.hits_dev, normalize_q=False, stream=self._search_stream,
                      hits_host=slot.hits_host, wait_event=self._flush_event, done_event=slot.hits_ready)
        self._wait_event(slot.hits_ready)
        self._search_done[li] = slot.hits_ready
        kpre, vv, pos, valid = slot.host
        tab = table is not None and self._rope is not None
        missing = ctypes.c_int64(0)
        N.check(N.lib().hc_cold_gather(
            self._store_ptrs[li], self.B, int(self.per_head_retrieval), self.lookahead_k, slot.hits_host.data_ptr(),
            N.dtype_code(kpre.dtype), kpre.data_ptr(), vv.data_ptr(), pos.data_ptr(), valid.data_ptr(),
            table.ctypes.data if tab else None, table.shape[0] if tab else 0, table.shape[1] if tab else 0,
            slot.tab.data_ptr() if tab else None, ctypes.byref(missing), int(nthreads)), "hc_cold_gather")
        self.dbg["retrieval_device"] += 1
        self._finish_retrieval(li, slot, tab, int(valid.sum()), missing.value)
        return True

    def _search_args(self, li, slot, q_vecs, table, nthreads):
        """hc_cold_retrieve's arguments for a search of layer li into `slot`
        (without tab_missing), the arrays they point into, and whether the
        rotary rows are gathered.  q_vecs None: the slot's pooled query, raw
        (B,VH,D) fp32, cropped or padded and normalised inside the native
        call; else host vectors already in search form."""
        B, R = self.B, self.lookahead_k
        kpre, vv, pos, valid = slot.host
        if q_vecs is None:
            q = slot.qhost
            q_ptr, q_dim, norm = q.data_ptr(), q.shape[-1], int(self.normalize_for_ip)
            q_sb, q_sh = q.stride(0), (q.stride(1) if q.dim() == 3 else 0)
        else:
            q = np.ascontiguousarray(q_vecs, dtype=np.float32).reshape(B, -1, self.faiss_dim)
            q_ptr, q_dim, norm = q.ctypes.data, self.faiss_dim, 0
            q_sb, q_sh = q.shape[1] * self.faiss_dim, self.faiss_dim
        # the rows of LlamaRotaryEmbedding.forward's tables at the retrieved
        # positions (rows past the hits hold position 0 and stay masked),
        # gathered in the same native call from the table the decode thread
        # computed
        tab = table is not None and self._rope is not None
        args = (self._store_ptrs[li], B, q_ptr, q_sb, q_sh, q_dim, norm, R, int(self.per_head_retrieval),
                N.dtype_code(kpre.dtype), kpre.data_ptr(), vv.data_ptr(), pos.data_ptr(), valid.data_ptr(),
                table.ctypes.data if tab else None, table.shape[0] if tab else 0, table.shape[1] if tab else 0,
                slot.tab.data_ptr() if tab else None, int(nthreads))
        return args, (q, table), tab

    def _finish_retrieval(self, li, slot, has_tab, n_valid, missing):
        """A search into `slot` is done: hand the slot on for its copy, or
        free it when nothing valid was found."""
        slot.has_tab = has_tab
        if has_tab and missing:
            # a token evicted after the search was scheduled lies past the
            # table: compute this retrieval's rows directly
            R = self.lookahead_k
            cos, sin = ops_rope_tables(slot.host[2].reshape(-1, R), self._rope[0], self._rope[1], self.dtype)
            slot.tab_host[0].view(-1, R, self.D // 2).copy_(cos)
            slot.tab_host[1].view(-1, R, self.D // 2).copy_(sin)
            self.dbg["rope_rows_direct"] += 1
        with self._retrieval_lock[li]:
            if n_valid == 0:
                slot.state = _Slot.FREE
                self.dbg["retrieval_ready_empty"] += 1
                return
            old = self._retrieval_ready_cpu[li]
            if old is not None:        # a newer result replaces one never copied
                old.state = _Slot.FREE
            self._retrieval_ready_cpu[li] = slot
            slot.state = _Slot.RETRIEVED
            self.dbg["retrieval_ready_cpu"] += 1

    def _collect(self, li):
        """Take in the layer's finished native search, if any (decode thread)."""
        job = self._retrieval_thread[li]
        if isinstance(job, _Job) and job.poll():
            self._retrieval_thread[li] = None
            if job.error is not None:
                with self._retrieval_lock[li]:
                    job.slot.state = _Slot.FREE
                raise N.HotColdError(f"hc_cold_retrieve (search thread): {job.error[1]} (status {job.error[0]})")
            self._finish_retrieval(li, job.slot, job.has_tab, *job.result)

    def launch_retrieval_now(self, layer_idx, q_pre):
        """One synchronous retrieval outside the schedule (controller.py:295-312)."""
        if self.lookahead_k <= 0 or not self._inited:
            return
        li = int(layer_idx)
        if self.cold_size(li) == 0:
            self.dbg["retrieval_skipped_no_cold"] += 1
            return
        if self._retrieval_worker(li, self._q_to_vecs_np(q_pre), table=self._rope_rows()):
            self.dbg["retrieval_launched"] += 1
            self.dbg["retrieval_launched_prefill"] += 1

    def maybe_launch_async_retrieval(self, layer_idx):
        """Every window_size calls, start a background search with the pooled
        recent queries (controller.py:314-342).  Skipped while the layer's
        previous search still runs (controller.py:333-335) or when every
        staging slot is in use.  Device searches scheduled in one decode step
        are launched together after the last layer's call (_flush_searches)."""
        li = int(layer_idx)
        if self._pending_search and li <= self._pending_search[-1][0]:
            self._flush_searches()          # a new step began before the last layer's call
        self._maybe_launch(li)
        if self._pending_search and li == self.n_layers - 1:
            self._flush_searches()

    def _maybe_launch(self, li):
        if self.lookahead_k <= 0:
            return
        self.step_count[li] += 1
        if self.step_count[li] % self.window_size != 0:
            return
        if not self._inited:
            return
        dindex = self._dindex[li] if self._dindex and self.query_window[li] \
            and self.query_window[li][0].is_cuda else None
        # the device index knows its rows' sizes without waiting for the
        # host stores' adds
        if (dindex is not None and not dindex.size.any()) or (dindex is None and self.cold_size(li) == 0):
            self.dbg["retrieval_skipped_no_cold"] += 1
            return
        if len(self.query_window[li]) == 0:
            return
        self._collect(li)
        with self._retrieval_lock[li]:
            th = self._retrieval_thread[li]
            if th is not None and th.is_alive():
                return
            slot = self._take_slot(li)
            if slot is None:
                self.dbg["retrieval_skipped_no_slot"] += 1
                return
        if dindex is not None:
            # pooled on the device now; ranked on the search stream with the
            # step's other device searches
            self._stage_query(li, slot, to_host=False)
            self._pending_search.append((li, slot, dindex))
            self.dbg["retrieval_launched"] += 1
            return
        if self._stream is not None and self.query_window[li][0].is_cuda:
            # pooled on the device; the search thread waits for the host
            # copy, the decode thread does not
            self._stage_query(li, slot)
            q_vecs, event = None, slot.q_ready
        else:
            q_vecs, event = self._pooled_query_np(li), None
        args, keep, tab = self._search_args(li, slot, q_vecs, self._rope_rows(), self.SEARCH_THREADS)
        handle = N.lib().hc_cold_retrieve_async(*args, event, self._search_workers())
        if not handle:
            with self._retrieval_lock[li]:
                slot.state = _Slot.FREE
            N.check(N.HC_ERR_INVALID, "hc_cold_retrieve_async")
        with self._retrieval_lock[li]:
            self._retrieval_thread[li] = _Job(handle, slot, tab, keep)
            self.dbg["retrieval_launched"] += 1

    def _flush_searches(self):
        """Launch the pending device searches on the search stream, behind one
        event recorded now on the decode stream (after every pooled query).
        If a launch fails, the searches not launched yet give their slots back
        (the failing one frees its own) before the error propagates, so their
        layers can schedule again."""
        pending, self._pending_search = self._pending_search, []
        if not pending:
            return
        launched = 0
        try:
            self._record_flush_event()
            for i, (li, slot, dindex) in enumerate(pending):
                self._launch_device_search(li, slot, dindex, self._flush_event if i == 0 else None)
                launched = i + 1
        except BaseException:
            for li, slot, _ in pending[launched:]:
                with self._retrieval_lock[li]:
                    if slot.state == _Slot.FILLING:
                        slot.state = _Slot.FREE
            raise

    def _record_flush_event(self):
        """Record the event the step's device searches wait on, on the decode stream."""
        if self._flush_event is None:
            self._flush_event = self._event(0)
        N.check(N.lib().hc_event_record(self._flush_event, ops_stream(self._device)), "hc_event_record")

    def _settle_search(self, li):
        """Before the layer's store takes new tokens: its pending device search
        is launched, and its gather job (which addresses the store by the
        logical indices the device ranked) is waited for."""
        if any(p[0] == li for p in self._pending_search):
            self._flush_searches()
        job = self._retrieval_thread[li] if self._retrieval_thread else None
        if isinstance(job, _Job) and job.by_hits:
            job.join()

    def _launch_device_search(self, li, slot, dindex, wait_event):
        """A scheduled search on the device index: on the search stream, after
        wait_event, the ranking kernels write the slot's hits (also into its
        pinned buffer) and its event is recorded; a native job then waits for
        that event (and for the adds submitted before it) and gathers the
        hits' rows from the host stores into the slot, as the host search
        would have (hc_cold_gather).  The decode thread waits for none of it."""
        lib = N.lib()
        ss = self._search_stream
        if slot.hits_ready is None:
            slot.hits_ready = self._event(0)
        R = self.lookahead_k
        try:
            dindex.search(slot.qdev, R, slot.hits_dev, normalize_q=self.normalize_for_ip, stream=ss,
                          hits_host=slot.hits_host, wait_event=wait_event, done_event=slot.hits_ready)
        except Exception:
            with self._retrieval_lock[li]:
                slot.state = _Slot.FREE
            raise
        self._search_done[li] = slot.hits_ready
        table = self._rope_rows()
        tab = table is not None and self._rope is not None
        kpre, vv, pos, valid = slot.host
        handle = lib.hc_cold_gather_async(
            self._store_ptrs[li], self.B, int(self.per_head_retrieval), R, slot.hits_host.data_ptr(),
            N.dtype_code(kpre.dtype), kpre.data_ptr(), vv.data_ptr(), pos.data_ptr(), valid.data_ptr(),
            table.ctypes.data if tab else None, table.shape[0] if tab else 0, table.shape[1] if tab else 0,
            slot.tab.data_ptr() if tab else None, self.SEARCH_THREADS, slot.hits_ready, self._search_workers())
        if not handle:
            with self._retrieval_lock[li]:
                slot.state = _Slot.FREE
            N.check(N.HC_ERR_INVALID, "hc_cold_gather_async")
        with self._retrieval_lock[li]:
            self._retrieval_thread[li] = _Job(handle, slot, tab, (slot.hits_host, table), by_hits=True)
            self.dbg["retrieval_device"] += 1

    def _search_workers(self):
        """Native search threads: about half of this process's cores, at most
        MAX_SEARCH_WORKERS searches at once."""
        cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 4)
        return max(1, min(self.MAX_SEARCH_WORKERS, cores // (2 * self.SEARCH_THREADS)))

    def wait_for_retrieval(self, layer_idx, timeout=None):
        """Join the layer's background search, if any (test and shutdown helper)."""
        if any(p[0] == int(layer_idx) for p in self._pending_search):
            self._flush_searches()
        th = self._retrieval_thread[int(layer_idx)] if self._inited else None
        if th is not None:
            th.join(timeout)
            self._collect(int(layer_idx))

    # -- staging ------------------------------------------------------------------------------
    # The device-side primitives are methods so that tests can run the
    # staging state machine without a GPU.
    def _event(self, timing):
        ev = ctypes.c_void_p()
        N.check(N.lib().hc_event_create(ctypes.byref(ev), int(timing)), "hc_event_create")
        return ev.value

    def _event_done(self, ev):
        done = N.lib().hc_event_query(ev)
        if done < 0:
            N.check(done, "hc_event_query")
        return done == 1

    def _alloc_dev(self, slot, device):
        slot.dev_block = torch.empty(slot.block.numel(), dtype=torch.uint8, device=device)
        views = _carve(slot.dev_block, self._slot_specs())
        slot.dev, slot.tab_dev = views[:4], (views[4][..., 0, :], views[4][..., 1, :])
        slot.qdev, slot.hits_dev = views[5], views[6]

    def _copy_to_device(self, slot):
        """The slot's host-to-device copies on the side stream, after the
        consumer stream has released the slot's previous contents; its ready
        event recorded behind them."""
        lib = N.lib()
        if slot.ready is None:
            slot.ready = self._event(0)
            if self.profile_overlap:
                slot.t0, slot.t1 = self._event(1), self._event(1)
        if slot.released:
            N.check(lib.hc_stream_wait_event(self._stream, slot.free_after), "hc_stream_wait_event")
        if slot.t0 is not None:
            N.check(lib.hc_event_record(slot.t0, self._stream), "hc_event_record")
        nbytes = slot.nbytes[1] if slot.has_tab else slot.nbytes[0]
        N.check(lib.hc_memcpy_h2d_async(slot.dev_block.data_ptr(), slot.block.data_ptr(), nbytes, self._stream),
                "hc_memcpy_h2d_async")
        if slot.t1 is not None:
            N.check(lib.hc_event_record(slot.t1, self._stream), "hc_event_record")
        N.check(lib.hc_event_record(slot.ready, self._stream), "hc_event_record")
        slot.copied = True

    def _order_after(self, slot):
        """Order the consumer stream after the slot's copy."""
        N.check(N.lib().hc_stream_wait_event(ops_stream(slot.dev[0].device), slot.ready), "hc_stream_wait_event")

    def _mark_released(self, slot):
        """Record on the consumer stream that the slot's last reader has been
        issued; its next copy waits for this point."""
        lib = N.lib()
        if slot.free_after is None:
            slot.free_after = self._event(0)
        N.check(lib.hc_event_record(slot.free_after, ops_stream(slot.dev[0].device)), "hc_event_record")
        slot.released = True

    def _copy_ms(self, slot):
        ms = ctypes.c_float()
        if N.lib().hc_event_elapsed_ms(slot.t0, slot.t1, ctypes.byref(ms)) == 0:
            return float(ms.value)
        return None

    # -- staging state machine (controller.py:344-442) ------------------------------------------
    def maybe_prefetch_to_gpu(self, layer_idx, device, dtype=None):
        """Start the host-to-device copy of a finished retrieval on the side
        stream (controller.py:344-380).  dtype is accepted for compatibility:
        staged buffers stay fp32 and the inject kernel converts."""
        li = int(layer_idx)
        if self._stream is None or not self._inited:
            return
        if self._retrieval_thread[li] is not None:
            self._collect(li)
        if self._retrieval_ready_cpu[li] is None:
            return                       # nothing retrieved (a search finishing now is taken next step)
        device = torch.device(device)
        if device.type != "cuda":
            return
        with self._retrieval_lock[li]:
            slot = self._retrieval_ready_cpu[li]
            self._retrieval_ready_cpu[li] = None
            if slot is None:
                return
            slot.state = _Slot.COPYING
        if slot.dev is None:
            self._alloc_dev(slot, device)
        self._copy_to_device(slot)
        with self._stage_lock[li]:
            old = self._staged[li]
            self._staged[li] = slot
            self.dbg["prefetch_launched"] += 1
        if old is not None:
            # superseded before it was polled: free once its copy completes
            # (_take_slot checks the event), no wait here
            with self._retrieval_lock[li]:
                old.state = _Slot.FREE
            self.dbg["prefetch_superseded"] += 1

    def poll_staged_gpu(self, layer_idx) -> RetrievedKV:
        """Non-blocking check for a staged retrieval (controller.py:382-442)."""
        li = int(layer_idx)
        if not self._inited or self._stream is None or self._staged[li] is None:
            return _NOT_READY
        with self._stage_lock[li]:
            slot = self._staged[li]
            if slot is None:
                return _NOT_READY
            if not self._event_done(slot.ready):
                self.dbg["prefetch_not_ready_checks"] += 1
                if not self.force_wait_for_prefetch_diagnostic:
                    return _NOT_READY
                self.dbg["main_waited_for_prefetch"] += 1
                while not self._event_done(slot.ready):
                    pass
            self._staged[li] = None
            slot.state = _Slot.STAGED
            self.dbg["prefetch_ready"] += 1
        # the copy has completed; order the consumer stream after it anyway
        self._order_after(slot)
        if self.profile_overlap and slot.t0 is not None:
            ms = self._copy_ms(slot)
            if ms is not None:
                self.dbg["prefetch_copy_ms_sum"] += ms
                self.dbg["prefetch_copy_ms_count"] += 1
        kpre, vv, pos, valid = slot.dev
        kpre = _canon_kv_4d(kpre, "staged.k_pre")
        vv = _canon_kv_4d(vv, "staged.v")
        cos = sin = None
        if slot.has_tab:
            cos, sin = slot.tab_dev
            if not self.per_head_retrieval:
                cos, sin = cos[:, 0], sin[:, 0]
        if not self.per_head_retrieval:
            pos = _canon_br_2d(pos, "staged.pos")
            valid = _canon_br_2d(valid, "staged.valid")
        return RetrievedKV(k_pre=kpre, v=vv, pos=pos, valid=valid, ready=True, cos=cos, sin=sin)

    def staged_consumed(self, layer_idx):
        """The staging just returned by poll_staged_gpu has been injected on
        the consumer stream: it becomes the layer's held slot (its positions
        and valid flags stay in use), and the previous held slot is released
        behind this point of the consumer stream."""
        li = int(layer_idx)
        with self._retrieval_lock[li]:
            new = next((sl for sl in self._slots[li] if sl.state == _Slot.STAGED), None)
            if new is None:
                return
            old, self._held_slot[li] = self._held_slot[li], new
            new.state = _Slot.HELD
            if old is not None and old is not new:
                self._mark_released(old)
                old.state = _Slot.FREE

    def resolve_held(self, layer_idx, injected):
        """The held slot this step attends (patch.py:241-291): the retrieval
        injected this step, else (hold_retrieved) the last one injected --
        a copy not ready yet leaves it in place -- else none."""
        li = int(layer_idx)
        if injected is not None:
            if self.hold_retrieved:
                self.held_mem[li] = injected
                self.dbg["injection_new"] += 1
            held = injected
        else:
            held = self.held_mem[li] if self.hold_retrieved else None
        if held is not None:
            self.last_injected_len = held[2]
            self.dbg["injection_used"] += 1
        return held
