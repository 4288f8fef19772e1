"""GPU tests of the drop-in package: the reference's parity checks
(tests/test_parity.py) on a small random-init Llama, the compression state
machines (tests/test_baselines.py) on the device, and the hot/cold layer's
compression, eviction and retrieval/inject flow against the oracle.

The reference's parity test loads Llama-3.1-8B by name; without network the
model here is a seeded random-init LlamaForCausalLM of the same architecture
family (GQA 4:2 heads, head_dim 64, RoPE theta 500000), with initializer
range 0.1 so that attention is far from uniform.
"""

import math

import numpy as np

import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM
from transformers.cache_utils import DynamicCache

import hotcold_kv as hk
from hotcold_kv.baselines import (PressConfig, PressLayerState, build_press_cache, install_press_patch,
                                  set_active_press_cache, uninstall_press_patch)
from hotcold_kv.cache import HotColdLayer
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
N_LAYERS = 2
# logits differences allowed against stock transformers (test_parity.py:71-73
# allows 0.5 / 1.0 on Llama-3.1-8B logits of +-30; these logits are +-5)
TOL = {torch.float32: 2e-3, torch.float16: 5e-2}


def _model(dtype):
    cfg = LlamaConfig(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=N_LAYERS,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=8192,
                      rope_theta=500000.0, initializer_range=0.1)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).to(DEV, dtype).eval()


def _ids(n, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 1000, (1, n), generator=g).to(DEV)


def decode_trace(model, ids, cache, n_steps, forced=None):
    """Prefill, then n_steps single-token steps with explicit positions
    (test_parity.py:76-101); forced tokens give teacher forcing."""
    out = model(input_ids=ids, use_cache=True, past_key_values=cache)
    prefill = out.logits[:, -1, :].float().cpu()
    past = out.past_key_values
    nxt = int(out.logits[0, -1].argmax())
    T = int(ids.shape[1])
    logits, fed = [], []
    for i in range(n_steps):
        tok = forced[i] if forced is not None else nxt
        fed.append(tok)
        cur = torch.tensor([[tok]], device=DEV, dtype=torch.long)
        cp = torch.tensor([T + i], device=DEV, dtype=torch.long)
        out = model(input_ids=cur, cache_position=cp, past_key_values=past, use_cache=True)
        lg = out.logits[:, -1, :].float()
        logits.append(lg.cpu())
        nxt = int(lg[0].argmax())
        past = out.past_key_values
    return prefill, logits, fed


def make_kvctrl(budget=10 ** 9, **kw):
    args = dict(max_capacity_prompt=budget, topk_ratio=0.15, recent_size=min(128, max(budget // 2, 1)),
                cpu_buffer_size=4096, faiss_dim=64, window_size=16, query_pool_size=4, lookahead_k=0,
                enable_asserts=True, profile_overlap=False, force_wait_for_prefetch_diagnostic=False)
    args.update(kw)
    return hk.KVController(**args)


class _HotCold:
    def __init__(self, model):
        self.model = model

    def __enter__(self):
        hk.set_active_rotary_emb(self.model.model.rotary_emb)
        hk.uninstall_monkeypatch()
        hk.install_monkeypatch(enable_debug=False)
        return self

    def __exit__(self, *exc):
        hk.uninstall_monkeypatch()
        hk.set_active_kvctrl(None)


@pytest.fixture(scope="module", params=[torch.float32, torch.float16], ids=["fp32", "fp16"])
def model_and_ref(request):
    dtype = request.param
    model = _model(dtype)
    ids = _ids(200)
    with torch.inference_mode():
        ref_trace = decode_trace(model, ids, DynamicCache(), 12)
    return model, ids, ref_trace, dtype


def test_hotcold_prefill_is_causal(model_and_ref):
    model, ids, _, dtype = model_and_ref
    k = int(ids.shape[1]) // 2
    with _HotCold(model), torch.inference_mode():
        hk.set_active_kvctrl(make_kvctrl())
        full_k = model(input_ids=ids, use_cache=False).logits[0, k].float().cpu()
        hk.set_active_kvctrl(make_kvctrl())
        trunc_k = model(input_ids=ids[:, :k + 1], use_cache=False).logits[0, -1].float().cpu()
    assert (full_k - trunc_k).abs().max().item() < TOL[dtype]


def test_hotcold_matches_stock_without_compression(model_and_ref):
    model, ids, (ref_prefill, ref_logits, fed), dtype = model_and_ref
    kv = make_kvctrl()
    with _HotCold(model), torch.inference_mode():
        hk.set_active_kvctrl(kv)
        cache = hk.build_hotcold_cache(model, kv)
        got_prefill, got_logits, _ = decode_trace(model, ids, cache, len(fed), forced=fed)
    assert (ref_prefill - got_prefill).abs().max().item() < TOL[dtype]
    d = max((a - b).abs().max().item() for a, b in zip(ref_logits, got_logits))
    agree = sum(int(a.argmax() == b.argmax()) for a, b in zip(ref_logits, got_logits))
    assert d < TOL[dtype] and agree >= len(fed) - 1, (d, agree)
    # nothing compressed, nothing retrieved (test_parity.py:180-186)
    assert kv.dbg["evicted_tokens"] == 0 and kv.dbg["injection_used"] == 0
    assert sum(kv.cold_size(i) for i in range(N_LAYERS)) == 0
    assert kv.dbg["triton_decode_calls"] == N_LAYERS * len(fed)
    assert cache.layers[0].hot_length() == ids.shape[1] + len(fed)


def test_hotcold_compression_keeps_prompt_attention(model_and_ref):
    model, ids, (ref_prefill, _, fed), dtype = model_and_ref
    small = 50
    kv = make_kvctrl(budget=small)
    with _HotCold(model), torch.inference_mode():
        hk.set_active_kvctrl(kv)
        cache = hk.build_hotcold_cache(model, kv)
        prefill, logits, _ = decode_trace(model, ids, cache, 4, forced=fed[:4])
    assert (prefill - ref_prefill).abs().max().item() < TOL[dtype]
    S = int(ids.shape[1])
    recent = min(128, small // 2)
    kept = int(small * 0.15) + recent
    assert kv.dbg["evicted_tokens"] >= S - kept
    for li in range(N_LAYERS):
        assert kv.cold_size(li) >= S - kept
        assert cache.layers[li].hot_length() <= small
    assert all(torch.isfinite(lg).all() for lg in logits)


def test_hotcold_retrieval_injects_rerotated_keys():
    dtype = torch.float16
    model = _model(dtype)
    ids = _ids(160, seed=3)
    R = 8
    kv = make_kvctrl(budget=40, lookahead_k=R, hold_retrieved=True, retrieve_after_prefill=True,
                     force_wait_for_prefetch_diagnostic=True)
    with _HotCold(model), torch.inference_mode():
        hk.set_active_kvctrl(kv)
        cache = hk.build_hotcold_cache(model, kv)
        _, logits, _ = decode_trace(model, ids, cache, 3, forced=[5, 6, 7])
        torch.cuda.synchronize()
    assert kv.dbg["retrieval_launched_prefill"] == N_LAYERS
    assert kv.dbg["injection_new"] >= N_LAYERS and kv.dbg["injection_used"] >= 3 * N_LAYERS
    assert kv.last_injected_len == R
    assert all(torch.isfinite(lg).all() for lg in logits)
    rot = model.model.rotary_emb
    for li in range(N_LAYERS):
        layer = cache.layers[li]
        pos, valid, r = kv.held_mem[li]
        assert r == R and bool(valid.all())
        pos_cpu = pos.cpu()
        snap = kv.rings[li][0].export()
        ring_pos = snap["pos"]
        ring_k = snap["kpre"]                                              # (n,Hk,D) fp32
        rows = [int((ring_pos == p).nonzero()[0][0]) for p in pos_cpu[0].tolist()]
        k_pre = torch.from_numpy(ring_k[rows]).permute(1, 0, 2).unsqueeze(0)  # (1,Hk,R,D)
        want = ref.rerope(k_pre, pos_cpu, rot.inv_freq.float().cpu(), float(rot.attention_scaling), dtype)
        kbuf, vbuf = layer.buf.held_storage()
        got = kbuf[:, :, layer.buf.held - R:layer.buf.held].cpu()
        assert torch.equal(got, want)      # rotary tables shipped with the retrieval: exact keys
        ring_v = torch.from_numpy(snap["v"][rows]).permute(1, 0, 2).unsqueeze(0)
        assert torch.equal(vbuf[:, :, layer.buf.held - R:layer.buf.held].cpu(), ring_v.to(dtype))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_hotcold_layer_compression_matches_oracle(dtype):
    B, Hq, Hk, S, D = 2, 8, 2, 300, 64
    g = torch.Generator().manual_seed(11)
    keys = torch.randn((B, Hk, S, D), generator=g).to(dtype)
    values = torch.randn((B, Hk, S, D), generator=g).to(dtype)
    pre = torch.randn((B, Hk, S, D), generator=g).to(dtype)
    pos = (torch.arange(S) + 7).view(1, S).expand(B, S).contiguous()
    q = torch.randn((B, Hq, 16, D), generator=g).to(dtype)
    kv = make_kvctrl(budget=128, recent_size=32, lookahead_k=0)
    kv._lazy_init(pre.to(DEV), n_layers=1)
    layer = HotColdLayer(kv)
    layer.set_last_query_post(q.to(DEV))
    layer.update(key_states=keys.to(DEV), value_states=values.to(DEV), layer_idx=0,
                 cache_kwargs={"pre_key_states": pre.to(DEV), "positions": pos.to(DEV)})
    torch.cuda.synchronize()
    want = ref.hotcold_compress(keys, values, pre, pos, q, max_capacity=128, recent_size=32, topk_ratio=0.15)
    keep = want["keep"]                                                    # (B,kept) shared over heads
    n = keep.shape[-1]
    assert layer.hot_length() == n and layer.get_seq_length() == S
    for b in range(B):
        assert torch.equal(layer.keys[b].cpu(), keys[b][:, keep[b]])
        assert torch.equal(layer.values[b].cpu(), values[b][:, keep[b]])
        assert torch.equal(layer.pre_keys[b].cpu(), pre[b][:, keep[b]])
        assert torch.equal(layer.positions[b].cpu(), pos[b, keep[b]])
        # the evicted complement went to the cold store in index order
        ev = want["evicted_idx"][b]
        ring = kv.rings[0][b]
        assert len(ring) == ev.numel()
        snap = ring.export()
        assert snap["pos"].tolist() == pos[b, ev].tolist()
        assert torch.equal(torch.from_numpy(snap["kpre"]), pre[b][:, ev].permute(1, 0, 2).float())
    assert kv.dbg["compress_calls"] == 1


def _press_cycle(method, dtype, B=2, Hq=8, Hk=2, S=200, D=16, budget=64, window=16, steps=40):
    """tests/test_baselines.py:44-67 on the device, with values checked
    against the oracle: kept rows bit-exact, decode within tolerance."""
    torch.manual_seed(0)
    n_rep = Hq // Hk
    scaling = 1.0 / math.sqrt(D)
    st = PressLayerState(method=method, budget=budget, window_size=window, kernel_size=7, pooling="maxpool")
    q = torch.randn(B, Hq, S, D).to(dtype)
    k = torch.randn(B, Hk, S, D).to(dtype)
    v = torch.randn(B, Hk, S, D).to(dtype)
    out = st.prefill(q.to(DEV), k.to(DEV), v.to(DEV), n_rep, scaling)
    assert out.shape == (B, Hq, S, D) and torch.isfinite(out).all()
    assert st.get_seq_length() == budget
    keep = ref.keep_index(ref.window_scores(q, k, window, scaling, 7, "maxpool"), window, budget)
    kk, vv = ref.gather_kv(k, keep), ref.gather_kv(v, keep)
    assert torch.equal(st.keys.cpu(), kk) and torch.equal(st.values.cpu(), vv)
    tol = 2e-3 if dtype == torch.float16 else 1e-5
    for _ in range(steps):
        q1, k1, v1 = (torch.randn(B, h, 1, D).to(dtype) for h in (Hq, Hk, Hk))
        out1 = st.decode(q1.to(DEV), k1.to(DEV), v1.to(DEV), n_rep, scaling)
        assert out1.shape == (B, Hq, 1, D) and torch.isfinite(out1).all()
        kk, vv = torch.cat([kk, k1], 2), torch.cat([vv, v1], 2)
        want = ref.decode_attention(q1, kk, vv, scaling)
        assert (out1[:, :, 0].double().cpu().numpy() - want).__abs__().max() < tol
    # the fused append left the token rows in the buffer
    assert torch.equal(st.keys.cpu(), kk) and torch.equal(st.values.cpu(), vv)
    return st


def _rows_to_index(buf, full):
    """Per (b, head) indices into full (B,H,n,D) of the rows of buf (B,H,m,D)."""
    B, H, m, _ = buf.shape
    idx = torch.empty((B, H, m), dtype=torch.long)
    for b in range(B):
        for h in range(H):
            eq = (buf[b, h][:, None, :] == full[b, h][None, :, :]).all(-1)     # (m, n)
            assert (eq.sum(1) == 1).all()
            idx[b, h] = eq.float().argmax(1)
    return idx


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_h2o_cycle_holds_budget_and_tracks_oracle(dtype):
    """tests/test_baselines.py:82-87 (the length stays at the budget, scores
    are (B,Hk,budget)) with every step checked against the oracle: prefill
    keeps and scores bit-exact; then each decode step's output within the
    dtype tolerance, the accumulated scores within a few fp32/fp16 rounding
    steps, and the kept set equal to the oracle's except at near-ties (where
    the oracle follows the kernel's choice)."""
    B, Hq, Hk, S, D, budget, window, steps = 2, 8, 2, 200, 16, 64, 16, 60
    n_rep, scaling = Hq // Hk, 1.0 / math.sqrt(D)
    g = torch.Generator().manual_seed(51)
    st = PressLayerState(method="h2o", budget=budget, window_size=window, kernel_size=7, pooling="maxpool")
    q, k, v = (torch.randn(B, h, S, D, generator=g).to(dtype) for h in (Hq, Hk, Hk))
    st.prefill(q.to(DEV), k.to(DEV), v.to(DEV), n_rep, scaling)
    sc = ref.h2o_prefill_scores(q, k, scaling)
    keep = ref.keep_index(sc, window, budget)
    kk, vv = ref.gather_kv(k, keep), ref.gather_kv(v, keep)
    assert torch.equal(st.keys.cpu(), kk) and torch.equal(st.values.cpu(), vv)
    assert torch.equal(st.scores.cpu(), sc.gather(2, keep))
    sc = sc.gather(2, keep).double()
    tol_out = 2e-3 if dtype == torch.float16 else 1e-5
    tol_sc = 3e-3 if dtype == torch.float16 else 2e-5
    for t in range(steps):
        q1, k1, v1 = (torch.randn(B, h, 1, D, generator=g).to(dtype) for h in (Hq, Hk, Hk))
        out1 = st.decode(q1.to(DEV), k1.to(DEV), v1.to(DEV), n_rep, scaling)
        kk, vv = torch.cat([kk, k1], 2), torch.cat([vv, v1], 2)
        want = ref.decode_attention(q1, kk, vv, scaling)
        assert np.abs(out1[:, :, 0].float().cpu().numpy() - want).max() <= tol_out, t
        sc = torch.cat([sc, torch.zeros(B, Hk, 1, dtype=torch.float64)], 2) + ref.h2o_decode_probs(q1, kk, scaling)
        assert st.get_seq_length() == budget and st.scores.shape == (B, Hk, budget)
        got_keep = _rows_to_index(st.keys.cpu(), kk)
        want_keep = ref.keep_index(sc.float(), window, budget)
        for b in range(B):
            for h in range(Hk):
                a, w_ = set(got_keep[b, h].tolist()), set(want_keep[b, h].tolist())
                if a != w_:   # only near-ties may differ
                    n = sc.shape[2]       # the recent window is always kept: ties are among the prefix
                    kth = sc[b, h, :n - window].sort(descending=True).values[budget - window - 1]
                    for i in a ^ w_:
                        assert abs(float(sc[b, h, i]) - float(kth)) <= 4 * tol_sc * max(1.0, float(kth)), (t, b, h)
        kk, vv, sc = ref.gather_kv(kk, got_keep), ref.gather_kv(vv, got_keep), sc.gather(2, got_keep)
        assert torch.allclose(st.scores.cpu().double(), sc, rtol=tol_sc, atol=tol_sc * 1e-2), t


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_snapkv_cycle(dtype):
    st = _press_cycle("snapkv", dtype, budget=64, steps=40)
    assert st.get_seq_length() == 64 + 40


def test_pyramidkv_cycle():
    _press_cycle("pyramidkv", torch.float16, budget=80, steps=20)


@pytest.mark.parametrize("method", ["snapkv", "pyramidkv", "h2o"])
def test_press_patch_matches_stock_without_compression(model_and_ref, method):
    model, ids, (ref_prefill, ref_logits, fed), dtype = model_and_ref
    install_press_patch()
    try:
        cache = build_press_cache(model, PressConfig(method=method, max_capacity=10 ** 9))
        set_active_press_cache(cache)
        with torch.inference_mode():
            b_prefill, b_logits, _ = decode_trace(model, ids, cache, len(fed), forced=fed)
    finally:
        uninstall_press_patch()
        set_active_press_cache(None)
    assert (ref_prefill - b_prefill).abs().max().item() < TOL[dtype]
    d = max((a - b).abs().max().item() for a, b in zip(ref_logits, b_logits))
    agree = sum(int(a.argmax() == b.argmax()) for a, b in zip(ref_logits, b_logits))
    assert d < TOL[dtype] and agree >= len(fed) - 1, (d, agree)


@pytest.mark.parametrize("method", ["snapkv", "pyramidkv"])
def test_press_patch_deferred_compaction_equals_per_layer(model_and_ref, method):
    """All layers compacted together after the last prefill (the default)
    store exactly the rows of one compaction per layer, and decode gives the
    same logits bit for bit."""
    model, ids, (_, _, fed), dtype = model_and_ref
    runs = []
    for defer in (True, False):
        install_press_patch()
        try:
            cache = build_press_cache(model, PressConfig(method=method, max_capacity=64, window_size=16,
                                                         defer_compaction=defer))
            set_active_press_cache(cache)
            with torch.inference_mode():
                prefill, logits, _ = decode_trace(model, ids, cache, 4, forced=fed[:4])
        finally:
            uninstall_press_patch()
            set_active_press_cache(None)
        runs.append((prefill, logits, [(l.state.keys.clone(), l.state.values.clone()) for l in cache.layers]))
    (p1, l1, kv1), (p2, l2, kv2) = runs
    assert torch.equal(p1, p2)
    assert all(torch.equal(a, b) for a, b in zip(l1, l2))
    for (k1, v1), (k2, v2) in zip(kv1, kv2):
        assert torch.equal(k1, k2) and torch.equal(v1, v2)


def test_press_patch_compresses_to_budget(model_and_ref):
    model, ids, (ref_prefill, _, fed), dtype = model_and_ref
    install_press_patch()
    try:
        cache = build_press_cache(model, PressConfig(method="snapkv", max_capacity=64, window_size=16))
        set_active_press_cache(cache)
        with torch.inference_mode():
            prefill, logits, _ = decode_trace(model, ids, cache, 5, forced=fed[:5])
    finally:
        uninstall_press_patch()
        set_active_press_cache(None)
    # compression changes what is stored, never the prompt's own attention
    assert (prefill - ref_prefill).abs().max().item() < TOL[dtype]
    for layer in cache.layers:
        assert layer.state.get_seq_length() == 64 + 5
        assert layer.get_seq_length() == ids.shape[1] + 5
    assert all(torch.isfinite(lg).all() for lg in logits)


def test_press_patch_h2o_holds_budget_in_the_model(model_and_ref):
    """H2O inside the patched model: prompt compressed to the budget, then
    re-evicted every decode step (test_baselines.py:82-87 at model level)."""
    model, ids, (ref_prefill, _, fed), dtype = model_and_ref
    install_press_patch()
    try:
        cache = build_press_cache(model, PressConfig(method="h2o", max_capacity=64, window_size=16))
        set_active_press_cache(cache)
        with torch.inference_mode():
            prefill, logits, _ = decode_trace(model, ids, cache, 5, forced=fed[:5])
    finally:
        uninstall_press_patch()
        set_active_press_cache(None)
    assert (prefill - ref_prefill).abs().max().item() < TOL[dtype]
    for layer in cache.layers:
        assert layer.state.get_seq_length() == 64
        assert layer.state.scores.shape[-1] == 64
        assert layer.get_seq_length() == ids.shape[1] + 5
    assert all(torch.isfinite(lg).all() for lg in logits)
