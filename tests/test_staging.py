"""CPU tests of the retrieval feed's degrade paths and staging-slot reuse.

The reference degrades without failing when a copy is late (no inject; the
held slot stays, controller.py:401-412), when the previous search still runs
(no launch, controller.py:333-335) and when the cold store is empty (no
search, controller.py:324-326, 307-309).  KVController's device primitives
(event query, host-to-device copy, stream ordering, device buffers) are
replaced here by host stand-ins, so the state machine runs without a GPU and
a copy can be held "not ready" for as long as a test wants.
"""

import pytest
import torch

from hotcold_kv import ops
from hotcold_kv.controller import KVController, _Slot, _block_layout
from hotcold_kv.datatypes import EvictedKV

HK, D = 2, 16


class _Event:
    """Completes after `polls` queries (never when polls is None)."""

    def __init__(self, polls=0):
        self.polls = polls

    def done(self):
        if self.polls is None:
            return False
        if self.polls > 0:
            self.polls -= 1
            return False
        return True


class HostCtrl(KVController):
    """KVController with host stand-ins for its device primitives."""

    def __init__(self, **kw):
        kw.setdefault("profile_overlap", False)
        super().__init__(**kw)
        self.copy_polls = 0          # queries each new copy needs before it completes
        self.log = []

    def _event_done(self, ev):
        return ev.done()

    def _alloc_dev(self, slot, device):
        slot.dev = tuple(t.clone() for t in slot.host)

    def _copy_to_device(self, slot):
        if slot.released:
            self.log.append(("wait_free", id(slot)))
        for d, h in zip(slot.dev, slot.host):
            d.copy_(h)
        slot.ready = _Event(self.copy_polls)
        slot.copied = True
        self.log.append(("copy", id(slot)))

    def _order_after(self, slot):
        self.log.append(("order", id(slot)))

    def _mark_released(self, slot):
        slot.free_after = _Event(0)
        slot.released = True
        self.log.append(("released", id(slot)))

    def _stage_blocks(self, device, nbytes):
        return torch.empty((nbytes,), dtype=torch.uint8), torch.empty((nbytes,), dtype=torch.uint8)


def _ctrl(**kw):
    args = dict(cpu_buffer_size=64, faiss_dim=D, lookahead_k=4, window_size=4, hold_retrieved=True)
    args.update(kw)
    ctrl = HostCtrl(**args)
    ctrl._lazy_init(torch.zeros(1, HK, 1, D), n_layers=1)
    ctrl._stream = "side"            # a stream handle: enables the staging path
    return ctrl


def _fill(ctrl, n=12, seed=0):
    g = torch.Generator().manual_seed(seed)
    keys = torch.randn(n, HK, D, generator=g)
    ctrl.add_evicted_to_cold_store(0, EvictedKV(
        k_pre_cpu=keys.permute(1, 0, 2).unsqueeze(0).contiguous(),
        v_cpu=(-keys).permute(1, 0, 2).unsqueeze(0).contiguous(),
        pos_cpu=torch.arange(100, 100 + n, dtype=torch.long).unsqueeze(0),
        evicted_idx=torch.arange(n, dtype=torch.long).unsqueeze(0)))


def _window(ctrl):
    """Run one retrieval period (window_size scheduled calls); the search
    runs synchronously."""
    ctrl.update_query_window(0, torch.randn(1, 4, 1, D))
    for _ in range(ctrl.window_size):
        ctrl.maybe_launch_async_retrieval(0)
        ctrl.wait_for_retrieval(0)


def _step(ctrl):
    """One decode step of the patched attention's feed: copy a finished
    retrieval, poll, inject (here: nothing to write), resolve the held slot."""
    ctrl.maybe_prefetch_to_gpu(0, "cuda")
    rr = ctrl.poll_staged_gpu(0)
    injected = None
    if rr.ready:
        ctrl.staged_consumed(0)
        injected = (rr.pos, rr.valid, int(rr.k_pre.shape[2]))
    return rr, ctrl.resolve_held(0, injected)


def test_empty_store_skips_retrieval():
    ctrl = _ctrl()
    _window(ctrl)
    assert ctrl.dbg["retrieval_skipped_no_cold"] == 1
    assert ctrl.dbg["retrieval_launched"] == 0
    rr, held = _step(ctrl)
    assert not rr.ready and held is None
    ctrl.launch_retrieval_now(0, torch.randn(1, 4, 1, D))     # the prefill-time search too
    assert ctrl.dbg["retrieval_skipped_no_cold"] == 2


def test_live_worker_skips_launch():
    ctrl = _ctrl()
    _fill(ctrl)

    class Alive:
        def is_alive(self):
            return True

        def join(self, timeout=None):
            pass

    ctrl._retrieval_thread[0] = Alive()
    _window(ctrl)
    assert ctrl.dbg["retrieval_launched"] == 0          # the running search is not doubled
    ctrl._retrieval_thread[0] = None
    _window(ctrl)
    assert ctrl.dbg["retrieval_launched"] == 1
    assert ctrl._retrieval_ready_cpu[0] is not None


def test_late_copy_keeps_the_previous_held_slot():
    ctrl = _ctrl()
    _fill(ctrl)
    _window(ctrl)
    rr, held = _step(ctrl)                    # first retrieval lands at once
    assert rr.ready and held is not None
    first = held
    assert ctrl.held_mem[0] is first and ctrl.last_injected_len == 4

    ctrl.copy_polls = None                    # the next copy never completes
    _window(ctrl)
    for i in range(3):
        rr, held = _step(ctrl)
        assert not rr.ready
        assert held is first                  # decode keeps attending the previous slot
        assert ctrl.dbg["prefetch_not_ready_checks"] == i + 1
    assert ctrl.dbg["injection_new"] == 1
    assert ctrl.dbg["injection_used"] == 4


def test_no_hold_attends_a_retrieval_only_when_it_lands():
    ctrl = _ctrl(hold_retrieved=False)
    _fill(ctrl)
    _window(ctrl)
    rr, held = _step(ctrl)
    assert rr.ready and held is not None
    rr, held = _step(ctrl)
    assert not rr.ready and held is None


def test_superseded_copy_is_recycled_without_waiting():
    ctrl = _ctrl()
    _fill(ctrl)
    ctrl.copy_polls = None                    # copies never complete
    _window(ctrl)
    ctrl.maybe_prefetch_to_gpu(0, "cuda")
    first = ctrl._staged[0]
    _window(ctrl)
    ctrl.maybe_prefetch_to_gpu(0, "cuda")     # supersedes the first, which was never polled
    assert ctrl.dbg["prefetch_superseded"] == 1
    assert ctrl._staged[0] is not first and first.state == _Slot.FREE
    # its copy is still running: a new search must not take its host buffers
    with ctrl._retrieval_lock[0]:
        taken = ctrl._take_slot(0)
    assert taken is not first
    taken.state = _Slot.FREE
    first.ready = _Event(0)                   # now the old copy completes
    with ctrl._retrieval_lock[0]:
        assert ctrl._take_slot(0) is first


def test_slots_are_reused_and_a_held_slot_is_released_before_its_next_copy():
    ctrl = _ctrl()
    _fill(ctrl)
    seen = set()
    for period in range(6):
        _window(ctrl)
        rr, held = _step(ctrl)
        assert rr.ready
        seen.add(id(ctrl._held_slot[0]))
    assert len(ctrl._slots[0]) <= 2           # held + the one in flight, allocated once
    assert len(seen) == 2
    # every copy into a slot that was held before waited for its release
    released = set()
    for kind, sid in ctrl.log:
        if kind == "released":
            released.add(sid)
        if kind == "copy" and sid in released:
            assert ("wait_free", sid) in ctrl.log


def test_busy_slots_skip_the_search():
    ctrl = _ctrl()
    _fill(ctrl)
    ctrl.copy_polls = None
    for sl in range(KVController.MAX_SLOTS):
        _window(ctrl)
        ctrl.maybe_prefetch_to_gpu(0, "cuda")
    before = ctrl.dbg["retrieval_launched"]
    _window(ctrl)                             # every slot has a copy in flight
    assert ctrl.dbg["retrieval_skipped_no_slot"] == 1
    assert ctrl.dbg["retrieval_launched"] == before


def test_two_slots_per_layer_are_preallocated():
    ctrl = _ctrl()
    ctrl._preallocate_slots()
    slots = ctrl._slots[0]
    assert len(slots) == 2 and slots[0] is not slots[1]
    assert all(sl.state == _Slot.FREE for sl in slots)
    ctrl._preallocate_slots()                 # idempotent
    assert len(ctrl._slots[0]) == 2


def test_slot_buffers_are_views_of_one_block():
    """k_pre, v, pos, valid, the rotary tables, the pooled query and the
    device-search hits carved from one block in that order, 256-byte aligned
    and disjoint; one copy of nbytes[0] carries a retrieval without tables,
    nbytes[1] one with them, and the pooled query and hits lie past both;
    cos and sin are the two halves of each table row."""
    ctrl = _ctrl(per_head_retrieval=True)
    with ctrl._retrieval_lock[0]:
        sl = ctrl._take_slot(0)
    views = list(sl.host) + [sl.tab, sl.qhost, sl.hits_host]
    base = sl.block.data_ptr()
    offs, ends = _block_layout(ctrl._slot_specs())
    spans = []
    for t, off, (shape, dt) in zip(views, offs, ctrl._slot_specs()):
        assert t.data_ptr() - base == off and off % 256 == 0
        assert tuple(t.shape) == tuple(shape) and t.dtype == dt and t.is_contiguous()
        spans.append((off, off + t.numel() * t.element_size()))
    for (a0, a1), (b0, b1) in zip(spans, spans[1:]):
        assert a1 <= b0
    assert [e for _, e in spans] == ends
    assert sl.nbytes == (spans[3][1], spans[4][1])
    assert sl.block.numel() == spans[6][1] and tuple(sl.qhost.shape) == (1, HK, D)
    assert tuple(sl.hits_host.shape) == (1, HK, 4) and sl.hits_host.dtype == torch.int64
    cos, sin = sl.tab_host
    assert cos.data_ptr() == sl.tab.data_ptr() and sin.data_ptr() == cos.data_ptr() + (D // 2) * cos.element_size()
    assert cos.stride() == sin.stride() and cos.shape == (1, HK, 4, D // 2)
    # writes through the views land in the block
    sl.host[2].fill_(7)
    assert sl.block[offs[2]:offs[2] + 8].view(torch.int64).item() == 7


def _rope_ctrl(dtype=torch.float16):
    ctrl = HostCtrl(cpu_buffer_size=64, faiss_dim=D, lookahead_k=4, window_size=4, hold_retrieved=True,
                    per_head_retrieval=True)
    ctrl._lazy_init(torch.zeros(1, HK, 1, D, dtype=dtype), n_layers=1)
    ctrl._stream = "side"
    inv = 1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ctrl.set_rope(inv, 1.0)
    return ctrl, inv


def test_retrieval_carries_the_rotary_rows_of_its_positions():
    """The search thread gathers the rows of the table computed on the decode
    thread: equal to the rotary module's tables at the retrieved positions."""
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        ctrl, inv = _rope_ctrl(dtype)
        _fill(ctrl)
        _window(ctrl)
        sl = ctrl._retrieval_ready_cpu[0]
        assert sl.has_tab and ctrl.dbg["rope_rows_direct"] == 0
        pos = sl.host[2]
        cos, sin = ops.rope_tables(pos.reshape(-1, 4), inv, 1.0, dtype)
        assert torch.equal(sl.tab_host[0].reshape(cos.shape), cos)
        assert torch.equal(sl.tab_host[1].reshape(sin.shape), sin)
        assert ctrl._rope_tab.shape[0] >= 112


def test_positions_past_the_table_are_computed_directly():
    ctrl, inv = _rope_ctrl()
    _fill(ctrl)
    small = ctrl._rope_rows()[:50]               # a table from before the evictions reached position 100
    ctrl._rope_rows = lambda: small
    _window(ctrl)
    sl = ctrl._retrieval_ready_cpu[0]
    assert sl.has_tab and ctrl.dbg["rope_rows_direct"] == 1
    cos, sin = ops.rope_tables(sl.host[2].reshape(-1, 4), inv, 1.0, torch.float16)
    assert torch.equal(sl.tab_host[0].reshape(cos.shape), cos)
    assert torch.equal(sl.tab_host[1].reshape(sin.shape), sin)


def test_native_query_normalisation_equals_the_host_one():
    """A query pooled on the device reaches the native call raw and is
    cropped / padded and normalised there; a host-pooled one is normalised
    by _normalize first.  Both retrieve the same tokens, and _normalize is
    the dimension-order fp64 formula."""
    import math

    import numpy as np
    for dim in (D, 12, 20):                        # as is, cropped, padded
        ctrl = _ctrl(per_head_retrieval=True, faiss_dim=dim)
        ctrl._wait_event = lambda ev: None
        _fill(ctrl, n=40)
        g = torch.Generator().manual_seed(dim)
        for trial in range(4):
            raw = torch.randn(1, HK, D, generator=g)
            got = []
            for host_side in (True, False):
                with ctrl._retrieval_lock[0]:
                    sl = ctrl._take_slot(0)
                if host_side:
                    assert ctrl._retrieval_worker(0, ctrl._normalize(ctrl._pad_or_crop(raw.numpy())), slot=sl)
                else:
                    sl.qhost = raw.clone()
                    assert ctrl._retrieval_worker(0, None, slot=sl)
                got.append((sl.host[2].clone(), sl.host[0].clone()))
                ctrl._retrieval_ready_cpu[0] = None
                sl.state = _Slot.FREE
            assert torch.equal(got[0][0], got[1][0]) and torch.equal(got[0][1], got[1][1]), (dim, trial)
        x = ctrl._pad_or_crop(raw.numpy())[0, 1].astype(np.float64)
        ss = 0.0
        for t in x.tolist():
            ss += t * t
        want = (x / max(math.sqrt(ss), 1e-12)).astype(np.float32)
        assert np.array_equal(ctrl._normalize(ctrl._pad_or_crop(raw.numpy()))[0, 1], want)


def test_native_search_jobs_equal_the_synchronous_search():
    """Searches scheduled on the library's worker threads (several layers at
    once) write what the synchronous call writes: positions, keys, values,
    valid flags and rotary rows."""
    L = 3
    ctrl = HostCtrl(cpu_buffer_size=64, faiss_dim=D, lookahead_k=4, window_size=1, hold_retrieved=True,
                    per_head_retrieval=True)
    ctrl._lazy_init(torch.zeros(1, HK, 1, D, dtype=torch.float16), n_layers=L)
    ctrl._stream = "side"
    ctrl.set_rope(1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D)), 1.0)
    g = torch.Generator().manual_seed(5)
    for li in range(L):
        keys = torch.randn(30, HK, D, generator=g)
        ctrl.add_evicted_to_cold_store(li, EvictedKV(
            k_pre_cpu=keys.permute(1, 0, 2).unsqueeze(0).contiguous(),
            v_cpu=(2 * keys).permute(1, 0, 2).unsqueeze(0).contiguous(),
            pos_cpu=torch.arange(50 * li, 50 * li + 30, dtype=torch.long).unsqueeze(0),
            evicted_idx=torch.arange(30, dtype=torch.long).unsqueeze(0)))
    qs = [torch.randn(1, 4, 1, D, generator=g) for _ in range(L)]
    for li in range(L):                         # all layers' searches in flight together
        ctrl.update_query_window(li, qs[li])
        ctrl.maybe_launch_async_retrieval(li)
    assert ctrl.dbg["retrieval_launched"] == L
    got = []
    for li in range(L):
        ctrl.wait_for_retrieval(li)
        sl = ctrl._retrieval_ready_cpu[li]
        assert sl is not None and sl.has_tab and ctrl._retrieval_thread[li] is None
        got.append([t.clone() for t in sl.host] + [sl.tab.clone()])
        ctrl._retrieval_ready_cpu[li] = None
        sl.state = _Slot.FREE
    for li in range(L):
        with ctrl._retrieval_lock[li]:
            sl = ctrl._take_slot(li)
        assert ctrl._retrieval_worker(li, ctrl._q_to_vecs_np(qs[li]), slot=sl, table=ctrl._rope_rows())
        for a, b in zip(got[li], list(sl.host) + [sl.tab]):
            assert torch.equal(a, b), li
        assert int(got[li][2].min()) >= 50 * li


def test_a_refused_native_search_raises_on_the_decode_thread():
    """Arguments the library refuses at submission raise on the decode thread
    (here: a zero batch); the slot is not left in flight."""
    ctrl = _ctrl()
    _fill(ctrl)
    real = ctrl._search_args

    def bad(*a, **k):
        args, keep, tab = real(*a, **k)
        return (args[0], 0) + args[2:], keep, tab

    ctrl._search_args = bad
    with pytest.raises(RuntimeError, match="cold_retrieve_async"):
        _window(ctrl)
    assert ctrl._retrieval_thread[0] is None
    assert all(sl.state == _Slot.FREE for sl in ctrl._slots[0])


def test_a_search_failing_on_its_worker_raises_once_and_frees_its_slot():
    """A retrieval that fails on the worker thread (here: the per-head flag
    does not match the store) is reported by the next collection on the
    decode thread; the slot is freed and the next search runs."""
    ctrl = _ctrl()
    _fill(ctrl)
    real = ctrl._search_args

    def mismatched(*a, **k):
        args, keep, tab = real(*a, **k)
        return args[:8] + (1,) + args[9:], keep, tab

    ctrl._search_args = mismatched
    with pytest.raises(RuntimeError, match="does not match"):
        _window(ctrl)
    assert ctrl._retrieval_thread[0] is None
    assert all(sl.state == _Slot.FREE for sl in ctrl._slots[0])
    ctrl._search_args = real
    _window(ctrl)
    assert ctrl._retrieval_ready_cpu[0] is not None


def test_a_failed_device_search_launch_frees_the_searches_after_it():
    """When one of a step's device searches fails to launch, the searches
    queued after it give their slots back (the failing one frees its own,
    the ones already launched stay with their gather jobs) and the error
    propagates; the layer can schedule again afterwards."""
    ctrl = _ctrl()
    _fill(ctrl)
    slots = [ctrl._take_slot(0) for _ in range(3)]
    assert all(sl is not None and sl.state == _Slot.FILLING for sl in slots)
    ctrl._pending_search = [(0, sl, object()) for sl in slots]
    calls = []

    def launch(li, slot, dindex, wait_event):
        calls.append(slot)
        if len(calls) == 2:
            raise RuntimeError("launch refused")

    ctrl._launch_device_search = launch
    ctrl._record_flush_event = lambda: None
    with pytest.raises(RuntimeError, match="launch refused"):
        ctrl._flush_searches()
    assert calls == slots[:2]
    assert slots[0].state == _Slot.FILLING                    # launched: its job owns it
    assert slots[1].state == _Slot.FREE and slots[2].state == _Slot.FREE
    assert ctrl._pending_search == []
    slots[0].state = _Slot.FREE
    assert ctrl._take_slot(0) is not None


def test_destroying_a_store_waits_for_its_search():
    """A store freed while a search job reads it (a controller collected with
    a search in flight) is freed only after the job has finished."""
    from hotcold_kv import _native as N
    ctrl = HostCtrl(cpu_buffer_size=20000, faiss_dim=D, lookahead_k=4, window_size=1, hold_retrieved=True)
    ctrl._lazy_init(torch.zeros(1, HK, 1, D), n_layers=1)
    ctrl._stream = "side"
    g = torch.Generator().manual_seed(9)
    keys = torch.randn(20000, HK, D, generator=g)
    ctrl.add_evicted_to_cold_store(0, EvictedKV(
        k_pre_cpu=keys.permute(1, 0, 2).unsqueeze(0).contiguous(), v_cpu=keys.permute(1, 0, 2).unsqueeze(0).contiguous(),
        pos_cpu=torch.arange(20000, dtype=torch.long).unsqueeze(0),
        evicted_idx=torch.arange(20000, dtype=torch.long).unsqueeze(0)))
    ctrl.update_query_window(0, torch.randn(1, 4, 1, D, generator=g))
    ctrl.maybe_launch_async_retrieval(0)
    job = ctrl._retrieval_thread[0]
    ring = ctrl.rings[0][0]
    handle, ring.handle = ring.handle, None
    N.lib().hc_cold_destroy(handle)                 # returns once the search no longer reads the store
    assert job.poll(wait=True) and job.error is None and job.result[0] == 4


# ---------------------------------------------------------------------------
# Cold-store adds as native jobs (the prefill's eviction returns while the
# store is filled)
# ---------------------------------------------------------------------------
def _tokens(rng, te, i):
    import numpy as np
    kpre = rng.standard_normal((HK, te, D), dtype=np.float32)
    v = rng.standard_normal((HK, te, D), dtype=np.float32)
    pos = np.arange(1000 * i, 1000 * i + te, dtype=np.int64)
    idx = np.arange(te, dtype=np.int64)
    idx[::5] = -1                                   # padding rows are skipped
    return kpre, v, pos, idx


@pytest.mark.parametrize("vec_heads", [1, HK])
def test_async_adds_equal_synchronous_adds(vec_heads):
    """Adds submitted as jobs apply in submission order, over a ring that
    wraps several times: size, searches and the store's contents equal those
    of synchronous adds, bit for bit.  Size and search, called right after the
    submissions, wait for the adds submitted before them."""
    import numpy as np
    from hotcold_kv.controller import _Ring
    a, b = _Ring(40, HK, D, D, vec_heads), _Ring(40, HK, D, D, vec_heads)
    rng = np.random.default_rng(3)
    jobs = []
    for i in range(7):
        kpre, v, pos, idx = _tokens(rng, 17 + 3 * i, i)
        a.add(kpre, v, pos, idx)
        jobs.append(b.add_async(kpre, v, pos, idx, nthreads=2, workers=4))
    assert len(b) == len(a) == 40
    q = rng.standard_normal(D).astype(np.float32)
    for h in range(vec_heads):
        assert np.array_equal(a.search(q, 9, head=h), b.search(q, 9, head=h))
    for j in jobs:
        assert j.poll(wait=True) and j.error is None
    ea, eb = a.export(), b.export()
    for k in ("kpre", "v", "pos", "vec"):
        assert np.array_equal(ea[k], eb[k]), k


def test_a_search_job_waits_for_the_adds_submitted_before_it():
    """A search job submitted right after async adds sees them: its result
    equals the synchronous retrieval over the synchronously filled store."""
    import numpy as np
    L = 2
    ctrls = []
    for mode in ("sync", "async"):
        ctrl = HostCtrl(cpu_buffer_size=64, faiss_dim=D, lookahead_k=4, window_size=1, hold_retrieved=True,
                        per_head_retrieval=True)
        ctrl._lazy_init(torch.zeros(1, HK, 1, D), n_layers=L)
        ctrl._stream = "side"
        g = torch.Generator().manual_seed(8)
        for li in range(L):
            keys = torch.randn(50, HK, D, generator=g)
            ev = EvictedKV(k_pre_cpu=keys.permute(1, 0, 2).unsqueeze(0).contiguous(),
                           v_cpu=(3 * keys).permute(1, 0, 2).unsqueeze(0).contiguous(),
                           pos_cpu=torch.arange(100 * li, 100 * li + 50, dtype=torch.long).unsqueeze(0),
                           evicted_idx=torch.arange(50, dtype=torch.long).unsqueeze(0))
            if mode == "sync":
                ctrl.add_evicted_to_cold_store(li, ev)
            else:
                st = ctrl.evict_stage("cpu", 1, HK, 50, D)
                ctrl.add_evicted_to_cold_store(li, ev, stage=st)
                assert ctrl.dbg["faiss_add"] == 50 * (li + 1)
        qs = [torch.randn(1, 4, 1, D, generator=g) for _ in range(L)]
        for li in range(L):
            ctrl.update_query_window(li, qs[li])
            ctrl.maybe_launch_async_retrieval(li)
        got = []
        for li in range(L):
            ctrl.wait_for_retrieval(li)
            sl = ctrl._retrieval_ready_cpu[li]
            got.append([t.clone() for t in sl.host])
        ctrl.wait_cold_adds()
        ctrls.append(got)
    for li in range(L):
        for x, y in zip(ctrls[0][li], ctrls[1][li]):
            assert torch.equal(x, y), li


def test_eviction_stages_are_reused_only_after_their_adds():
    """Two staging stages: a third eviction reuses the least recently handed
    out one after its adds are done, never one an add still reads."""
    ctrl = _ctrl()

    class _Pending:                 # a job that finishes after `polls` polls
        def __init__(self, polls):
            self.polls, self.error, self.waited = polls, None, False

        def poll(self, wait=False):
            if wait:
                self.waited, self.polls = True, 0
            if self.polls > 0:
                self.polls -= 1
                return False
            return True

    j1, j2 = _Pending(10 ** 9), _Pending(10 ** 9)
    s1 = ctrl.evict_stage("cpu", 1, HK, 8, D)
    assert ctrl.evict_stage("cpu", 1, HK, 8, D) is s1  # free: handed out again
    s1.jobs.append(j1)
    s2 = ctrl.evict_stage("cpu", 1, HK, 8, D)       # s1 busy: a second stage
    assert s2 is not s1
    s2.jobs.append(j2)
    s3 = ctrl.evict_stage("cpu", 1, HK, 8, D)       # both busy: the oldest, after waiting for it
    assert s3 is s1 and j1.waited and not j2.waited and not s3.jobs
    s2.jobs.clear()
    assert ctrl.evict_stage("cpu", 1, HK, 8, D) is s2  # free: reused without waiting
    big = ctrl.evict_stage("cpu", 1, HK, 4000, D)    # larger: the oldest, grown
    assert big.host.numel() >= ops.N.lib().hc_gather_evict_bytes(1, HK, 4000, D)


def test_destroying_a_store_waits_for_its_adds():
    """A store freed while adds run on the worker threads is freed only after
    them (they read the caller's buffers and write the store)."""
    import numpy as np
    from hotcold_kv import _native as N
    from hotcold_kv.controller import _Ring
    r = _Ring(20000, HK, D, D, HK)
    rng = np.random.default_rng(4)
    jobs = [r.add_async(*_tokens(rng, 6000, i), nthreads=1, workers=2) for i in range(3)]
    handle, r.handle = r.handle, None
    N.lib().hc_cold_destroy(handle)
    for j in jobs:
        assert j.poll(wait=True) and j.error is None


@pytest.mark.parametrize("per_head", [False, True])
def test_gathering_given_hits_equals_the_native_retrieval(per_head):
    """hc_cold_gather (the rows of hits found by the device search index)
    writes what hc_cold_retrieve writes when given the hits its own search
    finds: keys, values, positions, valid flags and rotary-table rows, with
    short rows (fewer tokens than R) padded the same way; and a search job
    queued behind async adds sees them (hc_cold_gather_async)."""
    import ctypes
    import numpy as np
    from hotcold_kv import _native as N
    from hotcold_kv.controller import _Ring
    lib = N.lib()
    B, H, Dd, R, cap = 3, HK, D, 8, 50
    VH = H if per_head else 1
    rng = np.random.default_rng(21)
    rings = [_Ring(cap, H, Dd, Dd, VH) for _ in range(B)]
    for b, n in enumerate((70, 5, 30)):                       # wrapped, short, partial
        kp = rng.standard_normal((H, n, Dd), dtype=np.float32)
        rings[b].add(kp, rng.standard_normal((H, n, Dd), dtype=np.float32), np.arange(7 * b, 7 * b + n) * 3)
    stores = (ctypes.c_void_p * B)(*[r.handle for r in rings])
    q = rng.standard_normal((B, VH, Dd), dtype=np.float32)
    tab = rng.integers(0, 255, size=(400, 12), dtype=np.uint8)

    def outputs():
        # garbage, as reused staging buffers hold: every row must be written
        return (np.full((B, H, R, Dd), 7.0, np.float32), np.full((B, H, R, Dd), -3.0, np.float32),
                np.full((B, VH, R), 123, np.int64), np.full((B, VH, R), 9, np.uint8),
                np.full((B, VH, R, 12), 77, np.uint8))

    want, got = outputs(), outputs()
    miss_w, miss_g = ctypes.c_int64(), ctypes.c_int64()
    N.check(lib.hc_cold_retrieve(stores, B, q.ctypes.data, VH * Dd, Dd, Dd, 1, R, int(per_head), N.HC_DTYPE_F32,
                                 *[x.ctypes.data for x in want[:4]], tab.ctypes.data, 400, 12, want[4].ctypes.data,
                                 ctypes.byref(miss_w), 2), "hc_cold_retrieve")
    hits = np.full((B, VH, R), -1, np.int64)
    for b in range(B):
        for h in range(VH):
            x = q[b, h].astype(np.float64)
            ss = 0.0
            for e in x:
                ss += e * e
            found = rings[b].search((x / max(ss ** 0.5, 1e-12)).astype(np.float32), R, head=h)
            hits[b, h, :len(found)] = found
    N.check(lib.hc_cold_gather(stores, B, int(per_head), R, hits.ctypes.data, N.HC_DTYPE_F32,
                               *[x.ctypes.data for x in got[:4]], tab.ctypes.data, 400, 12, got[4].ctypes.data,
                               ctypes.byref(miss_g), 2), "hc_cold_gather")
    for a, b_ in zip(want, got):
        assert np.array_equal(a, b_)
    assert miss_w.value == miss_g.value
    # rows past the hits: zero keys, values and positions, invalid (store 1
    # holds 5 tokens, fewer than R)
    for b in range(B):
        for h in range(VH):
            m = int((hits[b, h] >= 0).sum())
            assert got[3][b, h, :m].all() and not got[3][b, h, m:].any()
            assert (got[2][b, h, m:] == 0).all()
            heads = [h] if per_head else range(H)
            for hh in heads:
                assert not got[0][b, hh, m:].any() and not got[1][b, hh, m:].any()
    assert int((hits[1] >= 0).sum(axis=-1).min()) == 5
    # a hit beyond a store's tokens is refused
    bad = hits.copy()
    bad[1, 0, 0] = 40
    assert lib.hc_cold_gather(stores, B, int(per_head), R, bad.ctypes.data, N.HC_DTYPE_F32,
                              *[x.ctypes.data for x in got[:4]], None, 0, 0, None, None, 1) == N.HC_ERR_INVALID
    # the job form after async adds: it waits for them
    more = rng.standard_normal((H, 20, Dd), dtype=np.float32)
    adds = [rings[1].add_async(more, more, np.arange(20), nthreads=1, workers=2)]
    hits2 = hits.copy()
    hits2[1, :, :] = np.arange(R)                             # store 1 now holds 25 tokens
    job = lib.hc_cold_gather_async(stores, B, int(per_head), R, hits2.ctypes.data, N.HC_DTYPE_F32,
                                   *[x.ctypes.data for x in got[:4]], None, 0, 0, None, 1, None, 2)
    nv = ctypes.c_int64()
    assert lib.hc_cold_job_poll(job, 1, ctypes.byref(nv), None) == 1
    lib.hc_cold_job_free(job)
    assert got[3][1].all() and nv.value == int((hits2 >= 0).sum()) * 1
    for j in adds:
        assert j.poll(wait=True) and j.error is None


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_retrieved_rows_in_the_cache_dtype_round_as_torch_does(dtype):
    """A retrieval written in fp16 / bf16 (the staged rows the copy carries)
    equals torch's conversion of the same rows written in fp32 -- the
    reference's kpre_cpu.to(device, dtype) (controller.py:368-369): round to
    nearest even at exact midpoints, subnormal results, overflow to inf,
    signed zeros and infinities."""
    import ctypes

    import numpy as np

    from hotcold_kv import _native as N
    from hotcold_kv.controller import _Ring
    Dd, H, n = 16, 2, 24
    rng = np.random.default_rng(3)
    vals = [1 + 2 ** -11, 1 + 3 * 2 ** -11, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -11), 3e-6, 1e-7, 6.1e-5,
            65519.0, 65520.0, 70000.0, 3.39e38, 3.4e38, -0.0, float("inf"), float("-inf"), 2 ** -126, 1e-40]
    kpre = (rng.standard_normal((H, n, Dd)) * 10.0 ** rng.integers(-9, 6, (H, n, Dd))).astype(np.float32)
    kpre.reshape(-1)[:len(vals)] = np.array(vals, dtype=np.float32)
    v = (rng.standard_normal((H, n, Dd)) * 1e3).astype(np.float32)
    ring = _Ring(32, H, Dd, Dd, H)
    ring.add(kpre, v, np.arange(n, dtype=np.int64), np.arange(n, dtype=np.int64))
    stores = (ctypes.c_void_p * 1)(ring.handle)
    hits = np.tile(np.arange(n, dtype=np.int64), (1, H, 1))
    lib = N.lib()

    def gather(code, np_dtype):
        k = np.zeros((1, H, n, Dd), np_dtype)
        vv = np.zeros((1, H, n, Dd), np_dtype)
        pos, valid = np.zeros((1, H, n), np.int64), np.zeros((1, H, n), np.uint8)
        N.check(lib.hc_cold_gather(stores, 1, 1, n, hits.ctypes.data, code, k.ctypes.data, vv.ctypes.data,
                                   pos.ctypes.data, valid.ctypes.data, None, 0, 0, None, None, 1), "hc_cold_gather")
        return k, vv

    k32, v32 = gather(N.HC_DTYPE_F32, np.float32)
    k16, v16 = gather(N.dtype_code(dtype), np.uint16)
    for w32, w16 in ((k32, k16), (v32, v16)):
        want = torch.from_numpy(w32).to(dtype).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(w16, want)


def test_device_index_ring_mirrors_the_host_store():
    """DeviceIndex's slot assignment (host bookkeeping, no kernel): after adds
    that wrap the ring, rows with padding and a row that skips an add, the
    token at logical index l of each row sits in physical slot
    physical(b, l), and the sizes equal the host stores'.  The key scratch
    can be shared between indexes and is checked for size."""
    import numpy as np

    from hotcold_kv.controller import _Ring
    from hotcold_kv.device_index import DeviceIndex
    B, H, D, cap = 3, 2, 8, 50
    dix = DeviceIndex(B, H, D, D, H, cap, "cpu")
    assert dix.capT == 64 and dix.vec16 is not None and dix.keys.numel() == B * H * 64
    rings = [_Ring(cap, H, D, D, H) for _ in range(B)]
    where = [dict() for _ in range(B)]            # token id -> physical slot
    order = [[] for _ in range(B)]                # token ids, oldest first
    tok = 0
    rng = np.random.default_rng(1)
    for te in (20, 45, 7, 60, 33):
        idx = np.tile(np.arange(te, dtype=np.int64), (B, 1))
        idx[0, ::4] = -1
        if te == 7:
            idx[2, :] = -1
        slot_of = dix._slots(idx)
        for b in range(B):
            kept = np.nonzero(idx[b] >= 0)[0]
            k = rng.standard_normal((H, te, D), dtype=np.float32)
            rings[b].add(k, k, np.arange(te, dtype=np.int64), idx[b])
            for j in kept[-cap:]:
                where[b][tok + j] = int(slot_of[b, j])
                order[b].append(tok + j)
            order[b] = order[b][-cap:]
            assert (slot_of[b][idx[b] < 0] == -1).all()
        tok += te
    for b in range(B):
        assert int(dix.size[b]) == len(rings[b]) == len(order[b])
        for l, t in enumerate(order[b]):
            assert dix.physical(b, l) == where[b][t], (b, l)
    other = DeviceIndex(B, H, D, D, H, cap, "cpu", scratch=(dix.keys, dix.keys32))
    assert other.keys.data_ptr() == dix.keys.data_ptr()
    with pytest.raises(ValueError):
        DeviceIndex(B, H, D, D, H, 2 * cap, "cpu", scratch=(dix.keys, dix.keys32))


@pytest.mark.parametrize("vec_heads", [1, 2])
def test_deferred_search_vectors_give_the_same_results(vec_heads):
    """A store whose adds defer the search vectors (hc_cold_defer_vectors, set
    while a device index ranks) answers searches, retrievals and vector
    exports exactly as a store that computed them at every add, over adds
    that wrap the ring, before and after its first host search (which
    computes the missing vectors and ends the deferral)."""
    import ctypes

    import numpy as np

    from hotcold_kv import _native as N
    from hotcold_kv.controller import _Ring
    H, Dd, cap = 2, 16, 40
    rng = np.random.default_rng(vec_heads)
    a, b = _Ring(cap, H, Dd, Dd, vec_heads), _Ring(cap, H, Dd, Dd, vec_heads)
    assert N.lib().hc_cold_defer_vectors(b.handle, 1) == 0

    def add(te):
        k = rng.standard_normal((H, te, Dd), dtype=np.float32)
        v = rng.standard_normal((H, te, Dd), dtype=np.float32)
        p = rng.integers(0, 10 ** 6, te).astype(np.int64)
        for r in (a, b):
            r.add_async(k, v, p, nthreads=2, workers=2).join()

    def same():
        for h in range(vec_heads):
            q = rng.standard_normal(Dd).astype(np.float32)
            q /= np.linalg.norm(q)
            assert np.array_equal(a.search(q, 12, head=h), b.search(q, 12, head=h))

    add(25)
    add(30)                                   # wraps
    same()                                    # b computes its vectors here
    add(17)                                   # b computes them at the add again
    same()
    ea, eb = a.export(), b.export()
    for key in ("kpre", "v", "pos", "vec"):
        assert np.array_equal(ea[key], eb[key]), key
    # a retrieval on a deferring store
    a2, c = _Ring(cap, H, Dd, Dd, vec_heads), _Ring(cap, H, Dd, Dd, vec_heads)
    N.lib().hc_cold_defer_vectors(c.handle, 1)
    k = rng.standard_normal((H, 53, Dd), dtype=np.float32)
    for r in (a2, c):
        r.add(k, k, np.arange(53, dtype=np.int64))
    q = rng.standard_normal((1, vec_heads, Dd)).astype(np.float32)
    outs = []
    for r in (a2, c):
        st = (ctypes.c_void_p * 1)(r.handle)
        kp, vv = np.zeros((1, H, 8, Dd), np.float32), np.zeros((1, H, 8, Dd), np.float32)
        pos, valid = np.zeros((1, vec_heads, 8), np.int64), np.zeros((1, vec_heads, 8), np.uint8)
        N.check(N.lib().hc_cold_retrieve(st, 1, q.ctypes.data, vec_heads * Dd, Dd, Dd, 1, 8, int(vec_heads > 1),
                                         N.HC_DTYPE_F32, kp.ctypes.data, vv.ctypes.data, pos.ctypes.data,
                                         valid.ctypes.data, None, 0, 0, None, None, 1), "hc_cold_retrieve")
        outs.append((kp, vv, pos, valid))
    for x, y in zip(*outs):
        assert np.array_equal(x, y)
