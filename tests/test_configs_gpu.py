"""GPU parity at the sizes of the larger workloads: 16k/32k/64k prompts,
windows of 64, bf16 keys with heavy-tailed channels, held retrieval slots of
64/128/256 rows with per-KV-head positions, and batched hot buffers.

One layer (and, for the batched cases, the full batch) of each workload is
checked against the oracle: kept indices and gathered rows bit-exact,
attention within the dtype tolerance, re-rotated keys within a few rounding
steps of the model's rotation.
"""

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
