"""GPU parity at the sizes of the larger workloads: 16k/32k/64k prompts,
windows of 64, bf16 keys with heavy-tailed channels, held retrieval slots of
64/128/256 rows with per-KV-head positions, and batched hot buffers.

One layer (and, for the batched cases, the full batch) of each workload is
checked against the oracle: kept indices and gathered rows bit-exact,
attention within the dtype tolerance, re-rotated keys within a few rounding
steps of the model's rotation.
"""

import concurrent.futures
import math
import os

import numpy as np
import pytest
import torch

from hotcold_kv import ops, synthetic
from oracle import reference as ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2, torch.float32: 1e-4}


@pytest.mark.parametrize("name,layer", [
    ("llama8b_16k_b1024_held64", 5),
    ("b16_32k_b2048_held128", 7),
    ("bf16_b4_64k_b4096_held256", 11),
])
def test_compaction_bit_exact_one_layer(name, layer):
    """Scores, kept indices and compacted K/V of one sequence of one layer."""
    w = synthetic.WORKLOADS[name]
    p = synthetic.make_prompt(w, layer=layer, seed=0, device="cpu", batch=1)
    q, k, v = p["q_post"], p["k_post"], p["v"]
    got = ops.snapkv_scores(q.to(DEV), k.to(DEV), w.window, w.scaling, w.pool, "maxpool")
    want = ref.window_scores(q, k, w.window, w.scaling, w.pool, "maxpool")
    assert torch.equal(got.cpu(), want)
    keep = ops.keep_index(got, w.window, w.budget)
    want_keep = ref.keep_index(want, w.window, w.budget)
    assert torch.equal(keep.cpu(), want_keep)
    if not w.outliers:
        # planted needles are kept; with x20 outlier channels random keys can
        # outscore them, so the check is for the plain workloads only
        for h in range(w.hk):
            assert set(p["needles"][0, h].tolist()) <= set(want_keep[0, h].tolist())
    assert torch.equal(ops.gather_kv(k.to(DEV), keep).cpu(), ref.gather_kv(k, want_keep))
    assert torch.equal(ops.gather_kv(v.to(DEV), keep).cpu(), ref.gather_kv(v, want_keep))


def _per_sequence(fn, n):
    """[fn(b) for b in range(n)] on host threads: the oracle's C calls
    release the GIL, so sequences are checked side by side."""
    workers = max(1, min(16, os.cpu_count() or 1, n))
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        return list(ex.map(fn, range(n)))


def test_compaction_bit_exact_all_sequences_32k():
    """The 32k workload's batched compaction of one sampled layer, all 16
    sequences (independent seeds) in one launch set: scores, kept indices,
    planted needles and the compacted K/V rows against the oracle."""
    w = synthetic.WORKLOADS["b16_32k_b2048_held128"]
    print(f"[case] {w.name} layer 19, batch {w.batch}", flush=True)
    p = synthetic.make_prompt(w, layer=19, seed=0, device=DEV)
    W = min(w.window, w.seq_len)
    k, v = p["k_post"], p["v"]
    scores = ops.snapkv_scores(p["q_post"], k, w.window, w.scaling, w.pool, "maxpool")
    keep = ops.keep_index(scores, w.window, w.budget)
    kk, vv = ops.gather_kv(k, keep).cpu(), ops.gather_kv(v, keep).cpu()
    q_tail = p["q_post"][:, :, -W:].contiguous().cpu()
    needles = p["needles"].cpu()
    del p
    k_cpu, v_cpu = k.cpu(), v.cpu()
    scores, keep = scores.cpu(), keep.cpu()

    def oracle(b):
        sc = ref.window_scores(q_tail[b:b + 1], k_cpu[b:b + 1], w.window, w.scaling, w.pool, "maxpool",
                               q_is_window=True)
        return sc, ref.keep_index(sc, w.window, w.budget)

    res = _per_sequence(oracle, w.batch)
    for b, (sc, kp) in enumerate(res):
        assert torch.equal(scores[b:b + 1], sc), b
        assert torch.equal(keep[b:b + 1], kp), b
        for h in range(w.hk):
            assert set(needles[b, h].tolist()) <= set(kp[0, h].tolist()), (b, h)
    want_keep = torch.cat([kp for _, kp in res])
    assert torch.equal(kk, ref.gather_kv(k_cpu, want_keep))
    assert torch.equal(vv, ref.gather_kv(v_cpu, want_keep))


def test_prefill_retrieval_to_held_decode_at_64k():
    """The 64k bf16 workload (batch 4, budget 4096, window 64, heavy-tailed
    keys), one layer through the hot/cold engine: the prompt is compressed
    to the budget and the rest evicted to the cold store; the prefill-time
    synchronous retrieval (controller.py:295-312, ranked on the layer's device
    index) fetches the top-256 tokens
    per KV head; the first decode step (hotcold_attention) injects them into
    the held slot and attends [held | hot rows | token] in the fused launch.
    Checked: the kept rows (oracle compression), the store's contents, each
    (sequence, KV head)'s retrieved positions (oracle search over the store),
    the held keys bit for bit (the model's rotation of the stored pre-RoPE
    keys), and the attention output within the bf16 tolerance."""
    from hotcold_kv import KVController
    from hotcold_kv import patch as hp
    from hotcold_kv.cache import HotColdLayer

    w = synthetic.WORKLOADS["bf16_b4_64k_b4096_held256"]
    B, Hk, G, D, R = w.batch, w.hk, w.group, w.head_dim, w.prefill_retrieval
    print(f"[case] {w.name} layer 3, batch {B}, retrieval {R}", flush=True)
    cap = w.budget + w.decode_steps
    topk = w.budget - w.window
    ratio = (topk + 0.5) / cap
    ctrl = KVController(max_capacity_prompt=cap, topk_ratio=ratio, recent_size=w.window, cpu_buffer_size=w.seq_len,
                        faiss_dim=D, window_size=w.retrieve_every, query_pool_size=4, lookahead_k=R,
                        hold_retrieved=True, per_head_retrieval=True, retrieve_after_prefill=True,
                        force_wait_for_prefetch_diagnostic=True, profile_overlap=False, enable_asserts=True)
    p = synthetic.make_prompt(w, layer=3, seed=0, device=DEV)
    inv = synthetic.inv_freq(D, w.theta)
    ctrl._lazy_init(p["k_pre"], n_layers=1)
    ctrl.set_rope(inv, 1.0)
    layer = HotColdLayer(ctrl)
    q_last = p["q_post"][:, :, -w.window:, :].contiguous()
    qwin = p["q_pre"][:, :, -ctrl.query_pool_size:, :].contiguous()
    k_post, v, k_pre, positions = p["k_post"].cpu(), p["v"].cpu(), p["k_pre"].cpu(), p["positions"].cpu()
    # prefill (patch.py:152-172 without the prompt's own attention)
    layer.set_last_query_post(q_last)
    layer.update(key_states=p["k_post"], value_states=p["v"], layer_idx=0,
                 cache_kwargs={"pre_key_states": p["k_pre"], "positions": p["positions"]})
    del p
    ctrl.launch_retrieval_now(0, qwin)
    ctrl.maybe_prefetch_to_gpu(0, device=DEV)
    assert ctrl.dbg["retrieval_launched_prefill"] == 1
    assert ctrl.dbg["retrieval_device"] == 1          # ranked on the layer's device index
    # first decode step
    tok = synthetic.make_decode_token(w, 3, 0, seed=0, device=DEV)
    out = hp.hotcold_attention(ctrl, layer, 0, tok["q_pre"], tok["k_pre"], tok["v"], tok["q_post"], tok["k_post"],
                               tok["position"], G, w.scaling)
    torch.cuda.synchronize()
    assert ctrl.dbg["injection_new"] == 1 and ctrl.dbg["prefetch_ready"] == 1
    n = w.budget + 1

    # kept rows: the oracle's compression, sequence by sequence
    q_last_cpu = q_last.cpu()
    res = _per_sequence(lambda b: ref.hotcold_compress(k_post[b:b + 1], v[b:b + 1], k_pre[b:b + 1],
                                                       positions[b:b + 1], q_last_cpu[b:b + 1], cap, w.window,
                                                       ratio), B)
    hot_k, hot_v, hot_pos = layer.keys.cpu(), layer.values.cpu(), layer.positions.cpu()
    assert hot_k.shape[2] == n
    for b, want in enumerate(res):
        assert torch.equal(hot_pos[b, :w.budget], want["positions"][0]), b
        assert torch.equal(hot_k[b:b + 1, :, :w.budget], want["keys"]), b
        assert torch.equal(hot_v[b:b + 1, :, :w.budget], want["values"]), b

    # the store holds exactly the evicted tokens, oldest first
    qvec = ctrl._q_to_vecs_np(qwin)                                      # (B,Hk,D) the search's queries
    qf = qwin.double().cpu().view(B, Hk, G, -1, D).mean(dim=(2, 3))
    qf = qf / qf.norm(dim=-1, keepdim=True)
    assert np.abs(qvec - qf.numpy()).max() < 1e-6
    held_pos, held_valid, r = ctrl.held_mem[0]
    assert r == R and bool(held_valid.all())
    held_pos = held_pos.cpu()
    kbuf, vbuf = layer.buf.held_storage()
    lo = layer.buf.held - R
    got_k, got_v = kbuf[:, :, lo:layer.buf.held].cpu(), vbuf[:, :, lo:layer.buf.held].cpu()
    want_k = torch.empty((B, Hk, R, D), dtype=torch.float32)
    want_v = torch.empty((B, Hk, R, D), dtype=torch.float32)
    for b in range(B):
        ev = res[b]["evicted_idx"][0]
        snap = ctrl.rings[0][b].export()
        assert snap["pos"].tolist() == positions[b, ev].tolist(), b
        assert torch.equal(torch.from_numpy(snap["kpre"]), k_pre[b][:, ev].permute(1, 0, 2).float()), b
        for h in range(Hk):
            idx = ref.cold_topk(snap["kpre"], qvec[b, h], R, head=h, per_head=True, dim=D)
            assert held_pos[b, h].tolist() == snap["pos"][idx].tolist(), (b, h)
            want_k[b, h] = torch.from_numpy(snap["kpre"][idx, h])
            want_v[b, h] = torch.from_numpy(snap["v"][idx, h])
    assert torch.equal(got_k, ref.rerope(want_k, held_pos, inv, 1.0, w.dtype))
    assert torch.equal(got_v, want_v.to(w.dtype))

    # the decode over [held | hot rows | token]
    cur = tok["position"][0, -1:].cpu()
    K = torch.cat([got_k, hot_k], 2)
    V = torch.cat([got_v, hot_v], 2)
    q1 = tok["q_post"].cpu()
    o = out[:, :, 0].float().cpu().numpy()
    for h in range(Hk):
        m = torch.cat([held_valid[:, h].cpu() & (held_pos[:, h] <= cur), torch.ones((B, n), dtype=torch.bool)], 1)
        want = ref.decode_attention(q1[:, h * G:(h + 1) * G], K[:, h:h + 1], V[:, h:h + 1], w.scaling, m)
        assert np.abs(o[:, h * G:(h + 1) * G] - want).max() <= TOL[w.dtype], h


@pytest.mark.parametrize("name,batch,pool", [
    ("llama8b_16k_b1024_held64", 1, 4),
    ("llama8b_16k_b1024_held64", 1, 32),
    ("b16_32k_b2048_held128", 2, 4),
])
def test_scheduled_retrieval_windows(name, batch, pool):
    """The every-window_size-steps retrieval (controller.py:314-342) at a
    workload's size: one layer through hotcold_attention for two windows.
    The prompt is compressed to the budget and the rest evicted to the cold
    store; every retrieve_every steps the last `pool` pre-RoPE queries are
    pooled per KV head (pool 32 exceeds the old 16-row kernel bound), the
    top-R tokens are ranked on the layer's device index, copied on the side
    stream and re-rotated into the held slot, which later steps attend with
    valid & pos <= cur (patch.py:241-305).  The test waits for each search
    after its step, so the next step injects it.  Checked at every
    injection: each (sequence, KV head)'s positions against the oracle search
    over the store, the held keys bit for bit (the model's rotation of the
    stored pre-RoPE keys) and the values; at every step: the output within
    the dtype tolerance of the fp64 oracle over [held | hot rows | token]."""
    from hotcold_kv import KVController
    from hotcold_kv import patch as hp
    from hotcold_kv.cache import HotColdLayer

    w = synthetic.WORKLOADS[name]
    B, Hk, G, D, R, E = batch, w.hk, w.group, w.head_dim, w.held, w.retrieve_every
    lid = 2
    print(f"[case] {w.name} layer {lid}, batch {B}, pool {pool}, held {R}, every {E}", flush=True)
    steps = 2 * E + 2
    cap = w.budget + steps
    ratio = (w.budget - w.window + 0.5) / cap
    ctrl = KVController(max_capacity_prompt=cap, topk_ratio=ratio, recent_size=w.window, cpu_buffer_size=w.seq_len,
                        faiss_dim=D, window_size=E, query_pool_size=pool, lookahead_k=R, hold_retrieved=True,
                        per_head_retrieval=True, force_wait_for_prefetch_diagnostic=True, profile_overlap=False,
                        enable_asserts=True)
    p = synthetic.make_prompt(w, layer=lid, seed=0, device=DEV, batch=B)
    inv = synthetic.inv_freq(D, w.theta)
    ctrl._lazy_init(p["k_pre"], n_layers=1)
    ctrl.set_rope(inv, 1.0)
    layer = HotColdLayer(ctrl)
    layer.set_last_query_post(p["q_post"][:, :, -w.window:, :].contiguous())
    layer.update(key_states=p["k_post"], value_states=p["v"], layer_idx=0,
                 cache_kwargs={"pre_key_states": p["k_pre"], "positions": p["positions"]})
    del p
    ctrl.wait_cold_adds()
    # decode appends without re-compression, so the store stays as filled
    snaps = [ctrl.rings[0][b].export() for b in range(B)]
    assert all(len(s["pos"]) == w.seq_len - w.budget for s in snaps)

    q_hist, launched, windows = [], None, 0
    for t in range(steps):
        tok = synthetic.make_decode_token(w, lid, t, seed=0, device=DEV, batch=B)
        q_hist.append(tok["q_pre"])
        n_new = ctrl.dbg["injection_new"]
        out = hp.hotcold_attention(ctrl, layer, 0, tok["q_pre"], tok["k_pre"], tok["v"], tok["q_post"],
                                   tok["k_post"], tok["position"], G, w.scaling)
        torch.cuda.synchronize()
        kbuf, vbuf = layer.buf.held_storage()
        if ctrl.dbg["injection_new"] != n_new:
            # a new held slot: the search launched at the end of the last window
            assert launched is not None and t % E == 0, t
            windows += 1
            qvec = ctrl._q_to_vecs_np(launched)                        # (B,Hk,D) the search's queries
            T = launched.shape[2]
            qf = launched.double().cpu().view(B, Hk, G, T, D).mean(dim=(2, 3))
            qf = qf / qf.norm(dim=-1, keepdim=True)
            assert np.abs(qvec - qf.numpy()).max() < 1e-6
            held_pos, held_valid, r = ctrl.held_mem[0]
            assert r == R and bool(held_valid.all())
            hp_cpu = held_pos.cpu()
            want_k = torch.empty((B, Hk, R, D), dtype=torch.float32)
            want_v = torch.empty((B, Hk, R, D), dtype=torch.float32)
            for b in range(B):
                for h in range(Hk):
                    idx = ref.cold_topk(snaps[b]["kpre"], qvec[b, h], R, head=h, per_head=True, dim=D)
                    assert hp_cpu[b, h].tolist() == snaps[b]["pos"][idx].tolist(), (t, b, h)
                    want_k[b, h] = torch.from_numpy(snaps[b]["kpre"][idx, h])
                    want_v[b, h] = torch.from_numpy(snaps[b]["v"][idx, h])
            lo = layer.buf.held - R
            assert torch.equal(kbuf[:, :, lo:layer.buf.held].cpu(), ref.rerope(want_k, hp_cpu, inv, 1.0, w.dtype))
            assert torch.equal(vbuf[:, :, lo:layer.buf.held].cpu(), want_v.to(w.dtype))
        if (t + 1) % E == 0:
            launched = torch.cat(q_hist[-pool:], dim=2)              # the layer's query window
            ctrl.wait_for_retrieval(0)                                 # the next step copies and injects it
        # this step's output: [held | hot rows (the appended token last)]
        hot_k, hot_v = layer.keys.cpu(), layer.values.cpu()
        n = hot_k.shape[2]
        cur = tok["position"][0, -1:].cpu()
        held = ctrl.held_mem[0]
        q1 = tok["q_post"].cpu()
        o = out[:, :, 0].float().cpu().numpy()
        for h in range(Hk):
            if held is not None:
                lo = layer.buf.held - R
                K = torch.cat([kbuf[:, h:h + 1, lo:layer.buf.held].cpu(), hot_k[:, h:h + 1]], 2)
                V = torch.cat([vbuf[:, h:h + 1, lo:layer.buf.held].cpu(), hot_v[:, h:h + 1]], 2)
                pos_h, valid_h = held[0][:, h].cpu(), held[1][:, h].cpu()
                m = torch.cat([valid_h & (pos_h <= cur), torch.ones((B, n), dtype=torch.bool)], 1)
            else:
                K, V, m = hot_k[:, h:h + 1], hot_v[:, h:h + 1], None
            want = ref.decode_attention(q1[:, h * G:(h + 1) * G], K, V, w.scaling, m)
            assert np.abs(o[:, h * G:(h + 1) * G] - want).max() <= TOL[w.dtype], (t, h)
    assert windows == 2 and ctrl.dbg["retrieval_device"] == 2
    assert ctrl.dbg["retrieval_skipped_no_slot"] == 0


def test_retrieval_searched_without_rotary_tables_injects_exact_keys():
    """A retrieval searched before the rotary parameters were known carries
    no rotary tables; the inject then builds them from the staged positions
    (as the rotary module computes them), so the held keys are still the
    model's rotation bit for bit (patch.py:76-102 rotates with the module's
    own cos/sin)."""
    import types

    from hotcold_kv import KVController
    from hotcold_kv import patch as hp
    from hotcold_kv.cache import HotColdLayer

    w = synthetic.WORKLOADS["llama8b_16k_b1024_held64"]
    B, Hk, G, D, R = 1, w.hk, w.group, w.head_dim, w.held
    cap = w.budget + 4
    ratio = (w.budget - w.window + 0.5) / cap
    ctrl = KVController(max_capacity_prompt=cap, topk_ratio=ratio, recent_size=w.window, cpu_buffer_size=w.seq_len,
                        faiss_dim=D, window_size=w.retrieve_every, query_pool_size=4, lookahead_k=R,
                        hold_retrieved=True, per_head_retrieval=True, force_wait_for_prefetch_diagnostic=True,
                        profile_overlap=False, enable_asserts=True)
    p = synthetic.make_prompt(w, layer=4, seed=0, device=DEV, batch=B)
    inv = synthetic.inv_freq(D, w.theta)
    ctrl._lazy_init(p["k_pre"], n_layers=1)
    layer = HotColdLayer(ctrl)
    layer.set_last_query_post(p["q_post"][:, :, -w.window:, :].contiguous())
    layer.update(key_states=p["k_post"], value_states=p["v"], layer_idx=0,
                 cache_kwargs={"pre_key_states": p["k_pre"], "positions": p["positions"]})
    qwin = p["q_pre"][:, :, -4:, :].contiguous()
    del p
    ctrl.wait_cold_adds()
    assert ctrl._rope is None
    ctrl.launch_retrieval_now(0, qwin)                 # no set_rope yet: no tables travel
    ctrl.maybe_prefetch_to_gpu(0, device=DEV)
    assert ctrl.dbg["rope_rows_direct"] == 0
    hp.set_active_rotary_emb(types.SimpleNamespace(inv_freq=inv.to(DEV), attention_scaling=1.0))
    try:
        tok = synthetic.make_decode_token(w, 4, 0, seed=0, device=DEV, batch=B)
        hp.hotcold_attention(ctrl, layer, 0, tok["q_pre"], tok["k_pre"], tok["v"], tok["q_post"], tok["k_post"],
                             tok["position"], G, w.scaling)
        torch.cuda.synchronize()
    finally:
        hp.set_active_rotary_emb(None)
    assert ctrl.dbg["injection_new"] == 1 and ctrl.dbg["rope_rows_direct"] == 1
    held_pos, held_valid, r = ctrl.held_mem[0]
    assert r == R and bool(held_valid.all())
    hp_cpu = held_pos.cpu()
    snap = ctrl.rings[0][0].export()
    qvec = ctrl._q_to_vecs_np(qwin)
    want_k = torch.empty((B, Hk, R, D), dtype=torch.float32)
    for h in range(Hk):
        idx = ref.cold_topk(snap["kpre"], qvec[0, h], R, head=h, per_head=True, dim=D)
        assert hp_cpu[0, h].tolist() == snap["pos"][idx].tolist(), h
        want_k[0, h] = torch.from_numpy(snap["kpre"][idx, h])
    kbuf, _ = layer.buf.held_storage()
    got = kbuf[:, :, layer.buf.held - R:layer.buf.held].cpu()
    assert torch.equal(got, ref.rerope(want_k, hp_cpu, inv, 1.0, w.dtype))


def test_compaction_full_8k_job_layers_batched():
    """The bench's batched launch (layers stacked along the batch axis) keeps
    exactly what the per-layer oracle keeps, for the first and last layer."""
    w = synthetic.WORKLOADS["llama8b_8k_b512"]
    layers = [0, 31]
    ps = [synthetic.make_prompt(w, layer=l, seed=0, device="cpu") for l in layers]
    q = torch.cat([p["q_post"] for p in ps]).to(DEV)
    k = torch.cat([p["k_post"] for p in ps]).to(DEV)
    keep = ops.keep_index(ops.snapkv_scores(q, k, w.window, w.scaling, w.pool, "maxpool"), w.window, w.budget)
    for i, p in enumerate(ps):
        want = ref.keep_index(ref.window_scores(p["q_post"], p["k_post"], w.window, w.scaling, w.pool, "maxpool"),
                              w.window, w.budget)
        assert torch.equal(keep[i:i + 1].cpu(), want)


@pytest.mark.parametrize("name,batch,per_head", [
    ("llama8b_16k_b1024_held64", 1, False),
    ("b16_32k_b2048_held128", 16, True),
    ("bf16_b4_64k_b4096_held256", 4, True),
])
def test_decode_with_held_slot_at_workload_size(name, batch, per_head):
    """Hot buffer = held slot (R rows) + budget + decode steps, the held rows
    masked by valid & pos <= cur (per batch row or per KV head)."""
    w = synthetic.WORKLOADS[name]
    R, n = w.held, w.budget + w.decode_steps
    S, D = R + n, w.head_dim
    g = torch.Generator().manual_seed(17 * len(name) + R)
    dt = w.dtype
    q = torch.randn((batch, w.hq, 1, D), generator=g).to(dt)
    k = torch.randn((batch, w.hk, S, D), generator=g).to(dt)
    v = torch.randn((batch, w.hk, S, D), generator=g).to(dt)
    shape = (batch, w.hk, R) if per_head else (batch, R)
    valid = torch.rand(shape, generator=g) < 0.8
    pos = torch.randint(0, w.seq_len + w.decode_steps, shape, generator=g)
    cur = torch.tensor([w.seq_len + w.decode_steps // 2], dtype=torch.int64)
    sc = w.scaling
    out = ops.decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), sc, held_len=R, held_pos=pos.to(DEV),
                               held_valid=valid.to(DEV), cur_pos=cur.to(DEV)).float().cpu().numpy()
    G = w.hq // w.hk
    for h in range(w.hk):
        vh = valid[:, h] if per_head else valid
        ph = pos[:, h] if per_head else pos
        m = torch.cat([vh & (ph <= cur), torch.ones((batch, n), dtype=torch.bool)], 1)
        want = ref.decode_attention(q[:, h * G:(h + 1) * G], k[:, h:h + 1], v[:, h:h + 1], sc, m)
        assert np.abs(out[:, h * G:(h + 1) * G] - want).max() <= TOL[dt], h


@pytest.mark.parametrize("name", ["llama8b_16k_b1024_held64", "b16_32k_b2048_held128", "bf16_b4_64k_b4096_held256"])
def test_inject_full_held_slot(name):
    """Re-RoPE of a full held slot at the workload's size and dtype, per KV
    head positions, into the slot rows of a hot buffer: the rotary tables as
    the search thread computes them, every key bit-exact."""
    w = synthetic.WORKLOADS[name]
    B, Hk, R, D = w.batch, w.hk, w.held, w.head_dim
    g = torch.Generator().manual_seed(R)
    k_pre = torch.randn((B, Hk, R, D), generator=g)
    if w.outliers:
        k_pre[..., torch.randperm(D, generator=g)[:w.outliers]] *= 20.0
    v = torch.randn((B, Hk, R, D), generator=g)
    pos = torch.randint(0, w.seq_len, (B, Hk, R), generator=g)
    inv = synthetic.inv_freq(D, w.theta)
    cap = R + w.budget
    kd = torch.zeros((B, Hk, cap, D), dtype=w.dtype, device=DEV)
    vd = torch.zeros_like(kd)
    cos, sin = ops.rope_tables(pos.reshape(-1, R), inv, 1.0, w.dtype)
    cos, sin = cos.reshape(B, Hk, R, D // 2).to(DEV), sin.reshape(B, Hk, R, D // 2).to(DEV)
    ops.inject_rerope_tab(k_pre.to(DEV), v.to(DEV), cos, sin, kd, vd)
    want = ref.rerope(k_pre, pos, inv, 1.0, w.dtype)
    assert torch.equal(kd[:, :, :R].cpu(), want)
    assert torch.equal(vd[:, :, :R].cpu(), v.to(w.dtype))
    assert torch.count_nonzero(kd[:, :, R:]) == 0


def test_pipeline_16k_compaction_then_decode_matches_oracle():
    """End to end at 16k: kernel compaction -> gather -> decode of fresh
    tokens equals the oracle pipeline (same kept rows, attention within the
    fp16 tolerance)."""
    w = synthetic.WORKLOADS["llama8b_16k_b1024_held64"]
    p = synthetic.make_prompt(w, layer=0, seed=1, device="cpu", batch=1)
    k, v = p["k_post"], p["v"]
    scores = ops.snapkv_scores(p["q_post"].to(DEV), k.to(DEV), w.window, w.scaling, w.pool, "maxpool")
    keep = ops.keep_index(scores, w.window, w.budget)
    kk, vv = ops.gather_kv(k.to(DEV), keep), ops.gather_kv(v.to(DEV), keep)
    want_keep = ref.keep_index(ref.window_scores(p["q_post"], k, w.window, w.scaling, w.pool, "maxpool"),
                               w.window, w.budget)
    rk, rv = ref.gather_kv(k, want_keep), ref.gather_kv(v, want_keep)
    for t in range(3):
        tok = synthetic.make_decode_token(w, 0, t, seed=1, device="cpu", batch=1)
        out = ops.decode_attention(tok["q_post"].to(DEV), kk, vv, w.scaling).float().cpu().numpy()
        want = ref.decode_attention(tok["q_post"], rk, rv, w.scaling)
        assert np.abs(out - want).max() <= TOL[w.dtype], t


def test_device_search_at_32k_x16_equals_the_host_store():
    """The device search index at the 32k x 16 workload's size: 16 stores of
    30 720 evicted tokens, one 128-float vector per KV head, top-128 per
    (sequence, KV head).  The hits of three sequences are compared with their
    host stores' exact search (itself pinned by the oracle) for the
    workload's pooled-query-like queries: a stored key's direction, and
    random ones."""
    from hotcold_kv.controller import _Ring
    from hotcold_kv.device_index import DeviceIndex

    w = synthetic.WORKLOADS["b16_32k_b2048_held128"]
    B, Hk, D, R = w.batch, w.hk, w.head_dim, w.held
    n = w.seq_len - w.budget
    print(f"[case] {w.name}: device index {B} x {Hk} x {n}, top-{R}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(17)
    kpre = torch.randn((B, Hk, n, D), generator=g, device=DEV, dtype=torch.float32)
    dix = DeviceIndex(B, Hk, D, D, Hk, w.seq_len, DEV)
    dix.add(kpre, np.tile(np.arange(n, dtype=np.int64), (B, 1)))
    rows = (0, 7, 15)
    rings = {}
    for b in rows:
        k_b = kpre[b].cpu().numpy()
        rings[b] = _Ring(w.seq_len, Hk, D, D, Hk)
        rings[b].add(k_b, k_b, np.arange(n, dtype=np.int64), np.arange(n, dtype=np.int64))
    hits = torch.empty((B, Hk, R), dtype=torch.int64, device=DEV)
    for trial in range(3):
        q = torch.randn((B, Hk, D), generator=g, device=DEV, dtype=torch.float32)
        if trial == 0:
            q = kpre[:, :, 1234].clone()            # a stored key's direction ranks it first
        dix.search(q, R, hits)
        got = hits.cpu().numpy()
        qc = q.cpu().numpy()
        for b in rows:
            for h in range(Hk):
                x = qc[b, h].astype(np.float64)
                ss = 0.0
                for e in x:
                    ss += e * e
                want = rings[b].search((x / max(math.sqrt(ss), 1e-12)).astype(np.float32), R, head=h)
                assert np.array_equal(got[b, h], want), (trial, b, h)
                if trial == 0:
                    assert want[0] == 1234
