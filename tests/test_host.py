"""CPU tests of the host side: the C-ABI library's exports and argument
checks, the Python operator layer's refusal to run without the device
library, the cold store (tests/test_cold_store.py cases of the reference),
the baseline knobs (tests/test_baselines.py) and the shape canonicalisers.
No kernel is launched here.
"""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hotcold_hip.h")

from hotcold_kv import _native as N  # noqa: E402
from oracle import reference as ref  # noqa: E402
from hotcold_kv import ops  # noqa: E402
from hotcold_kv.baselines import PressConfig, PressLayerState, pyramid_layer_budget  # noqa: E402
from hotcold_kv.baselines import scoring  # noqa: E402
from hotcold_kv.controller import KVController  # noqa: E402
from hotcold_kv.datatypes import EvictedKV, _canon_br_2d, _canon_kv_4d  # noqa: E402


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(hc_[a-z0-9_]+)\s*\(", text)))


def test_header_lists_the_entry_points():
    names = _header_functions()
    for required in ("hc_decode_attn", "hc_snapkv_score", "hc_topk_keep", "hc_gather_rows", "hc_append_rows",
                     "hc_inject_rerope", "hc_last_error"):
        assert required in names


def test_library_exports_every_header_symbol():
    lib = N.lib()
    names = _header_functions()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding types exactly the header's functions
    assert sorted(N.SIGNATURES) == names
    assert lib.hc_abi_version() == 1


@pytest.mark.parametrize("struct,mirror,size_fn", [
    ("hc_decode_append_args", "DecodeAppendArgs", "hc_decode_append_args_size"),
    ("hc_decode_h2o_evict_args", "DecodeH2OEvictArgs", "hc_decode_h2o_evict_args_size"),
])
def test_packed_decode_args_mirror_the_header_struct(struct, mirror, size_fn):
    """The ctypes mirrors of the packed argument structs: the header's field
    names in order, 8 bytes each, and the library's sizeof."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (struct, struct), text, re.S).group(1)
    names = [n.strip().lstrip("*") for decl in body.split(";") if decl.strip()
             for n in re.sub(r"^\s*(const\s+)?\w+\s*\**", "", decl.strip()).split(",")]
    cls = getattr(N, mirror)
    fields = [f[0] for f in cls._fields_]
    assert fields == names
    for i, f in enumerate(fields):
        assert getattr(cls, f).offset == 8 * i, f
    assert getattr(N.lib(), size_fn)() == ctypes.sizeof(cls) == 8 * len(fields)


def test_packed_decode_rejects_a_null_struct():
    assert N.lib().hc_decode_attn_append_packed(None, None) == N.HC_ERR_INVALID
    assert N.lib().hc_decode_attn_h2o_evict_packed(None, None) == N.HC_ERR_INVALID


def test_abi_constants_match_header():
    text = open(HEADER).read()
    for name in ("HC_OK", "HC_ERR_INVALID", "HC_ERR_HIP", "HC_ERR_UNSUPPORTED", "HC_ERR_WORKSPACE", "HC_ERR_GROUP",
                 "HC_ERR_DROPOUT", "HC_DTYPE_F32", "HC_DTYPE_F16", "HC_DTYPE_BF16", "HC_POOL_MAX", "HC_POOL_AVG",
                 "HC_SCORE_SNAPKV", "HC_SCORE_RAWSUM"):
        m = re.search(r"#define\s+%s\s+\(?(-?\d+)\)?" % name, text)
        assert m, name
        assert int(m.group(1)) == getattr(N, name), name


def _decode_call(**over):
    """hc_decode_attn with null device pointers: only the argument checks run."""
    a = dict(dtype=N.HC_DTYPE_F16, B=1, Hq=8, Hk=2, D=64, S=100, dropout=0.0)
    a.update(over)
    lib = N.lib()
    return lib.hc_decode_attn(a["dtype"], a["B"], a["Hq"], a["Hk"], a["D"], a["S"],
                              None, 0, 0, None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, None, 0, 0, None, 0, 0, None,
                              0.125, a["dropout"], None, 0, 0, None, None, None, 0, 0, None)


def test_decode_argument_errors_match_reference():
    lib = N.lib()
    # kernels.py:88-89 and :99-100 raise ValueError with these messages
    assert _decode_call(dropout=0.1) == N.HC_ERR_DROPOUT
    assert lib.hc_last_error().decode() == "dropout must be 0.0 , because we are not in training"
    assert _decode_call(Hq=6, Hk=4) == N.HC_ERR_GROUP
    assert lib.hc_last_error().decode() == "Hq(6)//N_REP must equal Hk(4)"
    with pytest.raises(ValueError):
        N.check(N.HC_ERR_GROUP, "x")
    assert _decode_call(dtype=9) == N.HC_ERR_INVALID
    assert _decode_call(S=0) == N.HC_ERR_INVALID
    assert _decode_call() == N.HC_ERR_INVALID          # null tensors are refused, not dereferenced
    with pytest.raises(N.HotColdError):
        N.check(N.HC_ERR_INVALID, "hc_decode_attn")


def test_workspace_sizes():
    lib = N.lib()
    small = lib.hc_decode_attn_workspace_size(1, 32, 8, 128, 575, 0, 0)
    big = lib.hc_decode_attn_workspace_size(16, 32, 8, 128, 2431, 0, 1)
    assert 0 <= small <= big
    s1 = lib.hc_snapkv_score_workspace_size(1, 8, 8192, 128, 32)
    s2 = lib.hc_snapkv_score_workspace_size(1, 8, 16384, 128, 32)
    assert 0 < s1 < s2
    # the fp32 window logits dominate: W*S*4 bytes per KV head
    assert s1 >= 8 * 32 * 8192 * 4
    # the chunked top-k: only grids of fewer than 256 rows whose prefix passes
    # the 32768 keys the one-workgroup kernel caches; per row a 2048-bin
    # histogram, the state and two counts per 8192-key chunk, each part
    # 256-byte aligned
    assert lib.hc_topk_keep_workspace_size(4, 8, 65536, 64, 4096) == \
        32 * 2048 * 4 + 512 + ((32 * 8 * 2 * 4 + 255) // 256) * 256
    assert lib.hc_topk_keep_workspace_size(32, 8, 8192, 32, 512) == 0       # rows >= 256
    assert lib.hc_topk_keep_workspace_size(16, 8, 32768, 64, 2048) == 0     # prefix 32704 fits the cache
    assert lib.hc_topk_keep_workspace_size(1, 1, 40000, 0, 0) == 0          # nothing kept
    assert lib.hc_topk_keep_workspace_size(1, 1, 32769, 0, 10) > 0


def test_ops_refuse_host_tensors():
    q = torch.randn(1, 8, 1, 64, dtype=torch.float16)
    k = torch.randn(1, 2, 10, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError):
        ops.decode_attention(q, k, k, 0.125)
    with pytest.raises(RuntimeError):
        ops.snapkv_scores(torch.randn(1, 8, 10, 64), torch.randn(1, 2, 10, 64), 4, 0.125)
    with pytest.raises(RuntimeError):
        ops.keep_index(torch.randn(1, 2, 10), 4, 6)


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(N, "_lib", None)
    monkeypatch.setattr(N, "_LIB_PATH", os.path.join(ROOT, "does-not-exist.so"))
    with pytest.raises(RuntimeError, match="not built"):
        N.lib()


# ---------------------------------------------------------------------------
# Cold store: tests/test_cold_store.py of the reference, on this controller
# ---------------------------------------------------------------------------
HK, D = 2, 16


def _controller(cap, lookahead=4, per_head=False):
    ctrl = KVController(cpu_buffer_size=cap, faiss_dim=D, lookahead_k=lookahead, enable_asserts=True,
                        profile_overlap=False, per_head_retrieval=per_head)
    ctrl._lazy_init(torch.zeros(1, HK, 1, D), n_layers=1)
    return ctrl


def _tokens(n, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, HK, D, generator=g)


def _evict(ctrl, keys, positions, idx=None):
    te = keys.shape[0]
    ctrl.add_evicted_to_cold_store(0, EvictedKV(
        k_pre_cpu=keys.permute(1, 0, 2).unsqueeze(0).contiguous(),
        v_cpu=(-keys).permute(1, 0, 2).unsqueeze(0).contiguous(),
        pos_cpu=torch.tensor(positions, dtype=torch.long).unsqueeze(0),
        evicted_idx=(torch.arange(te, dtype=torch.long) if idx is None else idx).unsqueeze(0),
    ))


def _top1(ctrl, key):
    q = ctrl._k_token_to_vec_np(key)[None, :]
    ctrl._retrieval_worker(0, q)
    kpre, v, pos, valid = ctrl._retrieval_ready_cpu[0].host
    assert bool(valid[0, 0])
    return int(pos[0, 0]), kpre[0, :, 0, :], v[0, :, 0, :], pos[0][valid[0]].tolist()


def test_cold_store_no_wrap_returns_queried_token():
    ctrl = _controller(cap=64)
    keys = _tokens(20)
    _evict(ctrl, keys, list(range(100, 120)))
    for t in (0, 7, 19):
        pos, kpre, v, _ = _top1(ctrl, keys[t])
        assert pos == 100 + t
        assert torch.equal(kpre, keys[t]) and torch.equal(v, -keys[t])


def test_cold_store_wrap_keeps_ids_aligned():
    cap = 8
    ctrl = _controller(cap)
    keys = _tokens(15, seed=1)
    for lo in (0, 5, 10):
        _evict(ctrl, keys[lo:lo + 5], list(range(lo, lo + 5)))
    assert len(ctrl.cpu_kpre_ring[0][0]) == cap and ctrl.index[0][0].ntotal == cap
    live = range(15 - cap, 15)
    for t in live:
        pos, kpre, v, _ = _top1(ctrl, keys[t])
        assert pos == t
        assert torch.equal(kpre, keys[t]) and torch.equal(v, -keys[t])
    for t in range(15 - cap):
        _, _, _, hits = _top1(ctrl, keys[t])
        assert all(h in live for h in hits)


def test_cold_store_batch_larger_than_ring():
    cap = 8
    ctrl = _controller(cap)
    keys = _tokens(20, seed=2)
    _evict(ctrl, keys, list(range(20)))
    assert len(ctrl.cpu_kpre_ring[0][0]) == cap
    for t in range(20 - cap, 20):
        pos, kpre, _, _ = _top1(ctrl, keys[t])
        assert pos == t and torch.equal(kpre, keys[t])


def test_cold_store_skips_padding_and_ranks_by_inner_product():
    ctrl = _controller(cap=32, lookahead=3)
    keys = _tokens(6, seed=3)
    idx = torch.tensor([0, 1, -1, 3, -1, 5])          # -1 marks padding (datatypes.py:58-63)
    _evict(ctrl, keys, list(range(6)), idx=idx)
    assert ctrl.cold_size(0) == 4
    q = ctrl._k_token_to_vec_np(keys[3])
    ctrl._retrieval_worker(0, q[None, :])
    _, _, pos, valid = ctrl._retrieval_ready_cpu[0].host
    got = pos[0][valid[0]].tolist()
    snap = ctrl.rings[0][0].export()
    ip = np.zeros(len(snap["pos"]))
    for d in range(D):                       # fp64, accumulated in dimension order
        ip = ip + snap["vec"][:, 0, d].astype(np.float64) * float(q[d])
    want_order = [int(snap["pos"][i]) for i in np.argsort(-ip, kind="stable")[:3]]
    assert got == want_order and got[0] == 3


def test_cold_store_ties_go_to_the_older_token():
    ctrl = _controller(cap=16, lookahead=2)
    k = _tokens(1, seed=4)
    _evict(ctrl, torch.cat([k, k, k]), [10, 11, 12])
    q = ctrl._k_token_to_vec_np(k[0])
    ctrl._retrieval_worker(0, q[None, :])
    _, _, pos, valid = ctrl._retrieval_ready_cpu[0].host
    assert pos[0].tolist() == [10, 11] and valid.all()


def test_cold_store_per_head_retrieval():
    ctrl = _controller(cap=32, lookahead=2, per_head=True)
    keys = _tokens(10, seed=5)
    _evict(ctrl, keys, list(range(50, 60)))
    # head 0 queries token 2's key, head 1 token 7's
    q = np.stack([ctrl._normalize(ctrl._pad_or_crop(keys[2, 0].numpy())),
                  ctrl._normalize(ctrl._pad_or_crop(keys[7, 1].numpy()))])[None]
    ctrl._retrieval_worker(0, q)
    kpre, v, pos, valid = ctrl._retrieval_ready_cpu[0].host
    assert pos.shape == (1, HK, 2) and valid.dtype == torch.bool
    assert int(pos[0, 0, 0]) == 52 and int(pos[0, 1, 0]) == 57
    assert torch.equal(kpre[0, 0, 0], keys[2, 0]) and torch.equal(kpre[0, 1, 0], keys[7, 1])


def _native_store(cap, H, Dm, dim, per_head):
    from hotcold_kv.controller import _Ring
    return _Ring(cap, H, Dm, dim, H if per_head else 1)


@pytest.mark.parametrize("per_head", [False, True])
@pytest.mark.parametrize("dim", [24, 32, 48])
def test_native_cold_store_bit_exact_against_oracle(per_head, dim):
    """Vectors, search order and ring wrap of the native store equal the
    oracle's bit for bit: random tokens, padding indices, exact ties from
    power-of-two multiples, near-ties from one-ulp perturbations, and adds
    that wrap the ring and overflow it."""
    H, Dm, cap = 4, 32, 40
    g = torch.Generator().manual_seed(7 + dim + per_head)
    nat = _native_store(cap, H, Dm, dim, per_head)
    orc = ref.ColdStore(capacity=cap, dim=dim, per_head=per_head)
    pos0 = 0
    for n in (13, 25, 7, 61):
        k = torch.randn(n, H, Dm, generator=g)
        k[3] = 2 * k[1]                                   # exact tie with token 1
        k[5] = torch.nextafter(k[4], torch.full_like(k[4], 1e9))   # near tie with token 4
        v = torch.randn(n, H, Dm, generator=g)
        idx = torch.arange(n)
        idx[torch.randperm(n, generator=g)[: n // 5]] = -1        # padding
        pos = torch.arange(pos0, pos0 + n)
        pos0 += n
        nat.add(k.permute(1, 0, 2).numpy(), v.permute(1, 0, 2).numpy(), pos.numpy(), idx.numpy())
        orc.add(k.numpy(), v.numpy(), pos.numpy(), idx.numpy())
        snap = nat.export()
        assert snap["pos"].tolist() == orc.pos
        assert np.array_equal(snap["kpre"], np.stack(orc.kpre)) and np.array_equal(snap["v"], np.stack(orc.v))
        assert np.array_equal(snap["vec"], np.stack(orc.vec))             # bit-equal vectors
        for trial in range(6):
            head = trial % (H if per_head else 1)
            if trial < 3:   # a stored token's own vector: itself and its exact tie lead
                q = snap["vec"][int(torch.randint(len(orc.pos), (1,), generator=g))][head]
            else:
                q = orc.token_vecs(torch.randn(H, Dm, generator=g).numpy())[head]
            for r in (1, 5, 64):
                assert nat.search(q, r, head).tolist() == orc.search(q, r, head)


@pytest.mark.parametrize("per_head", [False, True])
def test_native_retrieve_matches_per_row_search(per_head):
    """hc_cold_retrieve over B stores equals per-store oracle searches and
    gathers; rows past the hits are zero and invalid."""
    B, H, Dm, dim, cap, R = 3, 4, 16, 16, 32, 6
    g = torch.Generator().manual_seed(11)
    ctrl = KVController(cpu_buffer_size=cap, faiss_dim=dim, lookahead_k=R, enable_asserts=True,
                        profile_overlap=False, per_head_retrieval=per_head)
    ctrl._lazy_init(torch.zeros(B, H, 1, Dm), n_layers=1)
    orcs = [ref.ColdStore(capacity=cap, dim=dim, per_head=per_head) for _ in range(B)]
    counts = (20, 3, 0)                                  # batch row 2 stays empty
    te = max(counts)
    k = torch.randn(B, H, te, Dm, generator=g)
    v = torch.randn(B, H, te, Dm, generator=g)
    pos = torch.arange(B * te).view(B, te) + 100
    idx = torch.stack([torch.where(torch.arange(te) < c, torch.arange(te), torch.full((te,), -1)) for c in counts])
    ctrl.add_evicted_to_cold_store(0, EvictedKV(k_pre_cpu=k, v_cpu=v, pos_cpu=pos, evicted_idx=idx))
    for b in range(B):
        orcs[b].add(k[b].permute(1, 0, 2).numpy(), v[b].permute(1, 0, 2).numpy(), pos[b].numpy(), idx[b].numpy())
    vh = H if per_head else 1
    q = np.stack([np.stack([orcs[0].token_vecs(torch.randn(H, Dm, generator=g).numpy())[h % vh]
                            for h in range(vh)]) for _ in range(B)])
    ctrl._retrieval_worker(0, q if per_head else q[:, 0])
    kpre, vv, p, valid = ctrl._retrieval_ready_cpu[0].host
    for b in range(B):
        for h in range(vh):
            hits = orcs[b].search(q[b, h], R, h)
            pv = p[b, h] if per_head else p[b]
            ok = valid[b, h] if per_head else valid[b]
            assert ok.tolist() == [True] * len(hits) + [False] * (R - len(hits))
            assert pv[: len(hits)].tolist() == [orcs[b].pos[i] for i in hits]
            assert (pv[len(hits):] == 0).all()
            heads = [h] if per_head else range(H)
            for hh in heads:
                want_k = np.zeros((R, Dm), np.float32)
                want_v = np.zeros((R, Dm), np.float32)
                for j, i in enumerate(hits):
                    want_k[j], want_v[j] = orcs[b].kpre[i][hh], orcs[b].v[i][hh]
                assert np.array_equal(kpre[b, hh].numpy(), want_k) and np.array_equal(vv[b, hh].numpy(), want_v)


def test_query_pooling_matches_reference_definition():
    ctrl = _controller(cap=8)
    g = torch.Generator().manual_seed(6)
    qs = [torch.randn(1, 8, 1, D, generator=g) for _ in range(4)]
    for q in qs:
        ctrl.update_query_window(0, q)
    got = ctrl._pooled_query_np(0)
    m = torch.cat(qs, dim=2).mean(dim=1).mean(dim=1)[0].double()
    want = (m / m.norm()).numpy()
    assert np.allclose(got[0], want, atol=1e-6)


def test_retrieval_schedule_every_window_steps():
    ctrl = _controller(cap=8)
    ctrl.window_size = 4
    _evict(ctrl, _tokens(4, seed=7), [0, 1, 2, 3])
    ctrl.update_query_window(0, torch.randn(1, 8, 1, D))
    for step in range(1, 9):
        ctrl.maybe_launch_async_retrieval(0)
        ctrl.wait_for_retrieval(0)
    assert ctrl.dbg["retrieval_launched"] == 2
    assert ctrl._retrieval_ready_cpu[0] is not None


# ---------------------------------------------------------------------------
# Baseline knobs (tests/test_baselines.py)
# ---------------------------------------------------------------------------
def test_pyramid_budget_monotone_decreasing():
    n = 16
    budgets = [pyramid_layer_budget(i, n, 512, 20) for i in range(n)]
    assert budgets[0] > budgets[-1]
    assert all(budgets[i] >= budgets[i + 1] for i in range(n - 1))
    assert 300 < sum(budgets) / n < 720
    assert budgets[0] == 2 * 512 - 512 // 20 and budgets[-1] == 512 // 20


def test_press_config_checks():
    PressConfig(method="pyramidkv", pooling="avgpool")
    with pytest.raises(AssertionError):
        PressConfig(method="streaming")
    with pytest.raises(AssertionError):
        PressConfig(window_size=512, max_capacity=512)
    PressConfig(method="h2o")
    st = PressLayerState("h2o", 64, 16, 7, "maxpool")
    assert st.scores is None and st.get_seq_length() == 0
    with pytest.raises(ValueError):
        PressLayerState("streaming", 64, 16, 7, "maxpool")


def test_h2o_fused_eviction_applies_exactly_when_one_row_goes():
    """The fused H2O step runs only where keep_index drops exactly one row:
    the step after the cache reaches the budget, with the window inside it."""
    for S, window, budget in [(513, 32, 512), (65, 16, 64), (2, 1, 1), (8192, 64, 8191)]:
        assert ops.h2o_evicts_one(S, window, budget)
        w, prefix, kp = ref.keep_counts(S, window, budget)
        assert prefix - kp == 1 and kp + w == S - 1
    for S, window, budget in [(512, 32, 512), (514, 32, 512), (513, 513, 512), (100, 200, 99),
                              (8193, 64, 8192), (40, 8, 0)]:
        assert not ops.h2o_evicts_one(S, window, budget), (S, window, budget)


def test_gqa_reduction_shapes():
    q = torch.randn(1, 8, 5, 16)
    assert scoring._group_query_to_kv(q, 2).shape == (1, 2, 5, 16)
    assert scoring._reduce_probs_to_kv(torch.randn(1, 8, 1, 50), 2).shape == (1, 2, 1, 50)


def test_pool_preserves_length_odd_kernel():
    x = torch.randn(2, 3, 57)
    for pooling in ("maxpool", "avgpool"):
        assert scoring.pool1d(x, 7, pooling).shape == x.shape


# ---------------------------------------------------------------------------
# Shape canonicalisers (datatypes.py:8-44)
# ---------------------------------------------------------------------------
def test_canon_shapes():
    assert _canon_kv_4d(torch.zeros(1, 1, 2, 3, 4), "k").shape == (1, 2, 3, 4)
    assert _canon_kv_4d(torch.zeros(1, 2, 3, 4), "k").shape == (1, 2, 3, 4)
    assert _canon_br_2d(torch.zeros(1, 1, 5), "pos").shape == (1, 5)
    assert _canon_br_2d(torch.zeros(3, 1, 5), "pos").shape == (3, 5)
    with pytest.raises(RuntimeError):
        _canon_kv_4d(torch.zeros(2, 3, 4), "k")
    with pytest.raises(RuntimeError):
        _canon_br_2d(torch.zeros(2, 3, 4), "pos")
    with pytest.raises(RuntimeError):
        _canon_br_2d([1, 2], "pos")


# ---------------------------------------------------------------------------
# Rotary tables shipped with a retrieval (the inject's cos/sin)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_rope_tables_are_the_rotary_modules_tables(dtype):
    """ops.rope_tables (run on the search thread) gives the first halves of
    LlamaRotaryEmbedding.forward's cos/sin (the oracle restates it), llama3
    frequencies and an attention scaling included."""
    g = torch.Generator().manual_seed(5)
    pos = torch.randint(0, 1 << 17, (6, 40), generator=g)
    for inv, scale in ((ref.default_inv_freq(128, 500000.0), 1.0),
                       (ref.default_inv_freq(64, 10000.0) * 0.25, 1.0625)):
        cos, sin = ops.rope_tables(pos, inv, scale, dtype)
        wc, ws = ref.rotary_cos_sin(inv, scale, pos, dtype)
        half = inv.numel()
        assert torch.equal(cos, wc[..., :half]) and torch.equal(sin, ws[..., :half])
        assert torch.equal(wc[..., :half], wc[..., half:])      # the second half repeats the first


def test_device_index_entries_refuse_bad_arguments_before_any_launch():
    """hc_index_add / hc_index_search check their arguments on the host and
    return HC_ERR_INVALID without touching the device: batch rows past 64, a
    vector width that is not a multiple of 4 (or past 1024), R past 1024, a
    capacity that is not a multiple of 64, ring states outside the capacity,
    null pointers, and an fp16 copy with a width not a multiple of 8."""
    lib = N.lib()
    fake = ctypes.c_void_p(0x1000)        # never dereferenced: every call below fails its checks first
    sizes = np.zeros(2, dtype=np.int64)
    heads = np.zeros(2, dtype=np.int64)

    def search(B=2, VH=1, VD=64, cap=128, R=8, capT=128, sz=sizes, hd=heads, vec=fake, keys=fake):
        return lib.hc_index_search(B, VH, VD, cap, fake, VD, VD, VD, 1, vec, None, 1, capT, sz.ctypes.data,
                                   hd.ctypes.data, R, keys, None, fake, None, None, None, None)

    def add(VD=64, vec16=None, capT=128):
        return lib.hc_index_add(2, 2, 64, 1, VD, 1, fake, 128, 64, 64, 4, fake, fake, vec16, capT, None)

    assert search(B=65) == N.HC_ERR_INVALID
    assert search(B=0) == N.HC_ERR_INVALID
    assert search(VD=6) == N.HC_ERR_INVALID
    assert search(VD=2048) == N.HC_ERR_INVALID
    assert search(R=1025) == N.HC_ERR_INVALID
    assert search(capT=100) == N.HC_ERR_INVALID
    assert search(cap=200) == N.HC_ERR_INVALID                 # capT below the capacity
    assert search(sz=np.array([0, 129], dtype=np.int64)) == N.HC_ERR_INVALID
    assert search(hd=np.array([0, 128], dtype=np.int64)) == N.HC_ERR_INVALID
    assert search(vec=None) == N.HC_ERR_INVALID
    assert search(keys=None) == N.HC_ERR_INVALID
    assert "index_search" in lib.hc_last_error().decode()
    assert add(VD=6) == N.HC_ERR_INVALID
    assert add(VD=12, vec16=fake) == N.HC_ERR_INVALID
    assert add(capT=100) == N.HC_ERR_INVALID
    assert "index_add" in lib.hc_last_error().decode()
