"""GPU parity of each hot-tier kernel against the CPU oracle (same seeded inputs).

Bars: kept indices and gathered rows bit-exact; window scores bit-exact under
the bit-defined contract; attention outputs within max-abs 2e-3 (fp16),
1e-2 (bf16), 1e-4 (fp32) of the fp64 oracle; re-RoPE keys within one ulp of
the model's own rotation (and equal in at least 99.9% of elements).
"""

import contextlib
import math

import numpy as np
import pytest
import torch

from hotcold_kv import ops, synthetic
from hotcold_kv.hot_buffer import kv_rows
from oracle import reference as ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2, torch.float32: 1e-4}


def _randn(shape, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


# ---------------------------------------------------------------------------
# Decode attention
# ---------------------------------------------------------------------------
DECODE_CASES = [
    # B, Hq, Hk, S, D, dtype
    (2, 8, 2, 200, 16, torch.float32),      # reference test geometry (test_baselines.py:46)
    (2, 8, 2, 200, 16, torch.float16),
    (1, 32, 8, 574, 128, torch.float16),    # 8k/budget-512 hot buffer after 62 appends
    (1, 32, 8, 574, 128, torch.bfloat16),
    (1, 32, 8, 544, 128, torch.float32),
    (3, 16, 4, 1, 64, torch.float16),       # a single key
    (2, 8, 8, 37, 32, torch.bfloat16),      # no grouping, ragged length
    (4, 32, 8, 2431, 128, torch.float16),   # batched long hot buffer
    (1, 64, 8, 300, 128, torch.float16),    # group of 8
    (1, 8, 1, 1000, 256, torch.bfloat16),   # one KV head, wide head_dim
    (1, 32, 2, 333, 128, torch.float16),    # group of 16
    # several 16-key tiles per wave at the smaller head dims
    (2, 16, 4, 3000, 64, torch.float16),
    (1, 8, 2, 2600, 32, torch.bfloat16),
    (1, 8, 2, 4100, 16, torch.float16),
]


def test_decode_unsupported_group_raises():
    q = torch.zeros((1, 16, 1, 256), dtype=torch.float16, device=DEV)
    k = torch.zeros((1, 1, 8, 256), dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="group size 16"):
        ops.decode_attention(q, k, k, 0.1)
    with pytest.raises(ValueError, match="dropout"):
        ops.decode_attention(q, k, k, 0.1, dropout=0.1)


@pytest.mark.parametrize("B,Hq,Hk,S,D,dtype", DECODE_CASES)
@pytest.mark.parametrize("splits", [0, 1])
def test_decode_matches_oracle(B, Hq, Hk, S, D, dtype, splits):
    q = _randn((B, Hq, 1, D), 1, dtype)
    k = _randn((B, Hk, S, D), 2, dtype)
    v = _randn((B, Hk, S, D), 3, dtype)
    sc = 1.0 / math.sqrt(D)
    out = ops.decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), sc, num_splits=splits)
    want = ref.decode_attention(q, k, v, sc)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    assert np.abs(got - want).max() <= TOL[dtype], np.abs(got - want).max()


@pytest.mark.parametrize("B,S,splits", [
    (1, 2431, 16),    # 128 workgroups: merged in the kernel by the last split to finish
    (2, 575, 0),      # one layer at a small batch: the default spreads it over many workgroups
    (16, 2431, 8),    # 1024 workgroups: merged by a second kernel
])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_split_merge_paths(B, S, splits, dtype):
    Hq, Hk, D = 32, 8, 128
    q = _randn((B, Hq, 1, D), 21, dtype)
    k = _randn((B, Hk, S, D), 22, dtype)
    v = _randn((B, Hk, S, D), 23, dtype)
    sc = 1.0 / math.sqrt(D)
    want = ref.decode_attention(q, k, v, sc)
    for rep in range(3):    # repeated launches on one workspace: each counts under its own tag
        out = ops.decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), sc, num_splits=splits)
        assert np.abs(out.float().cpu().numpy() - want).max() <= TOL[dtype], rep
    # the fused append through the same shapes: rows 0..S-2 cached, the token attended as key S-1
    kd, vd = k.to(DEV).clone(), v.to(DEV).clone()
    out = ops.decode_attention_append(q.to(DEV), kd, vd, k[:, :, S - 1].to(DEV), v[:, :, S - 1].to(DEV), sc,
                                      num_splits=splits)
    assert np.abs(out.float().cpu().numpy() - want).max() <= TOL[dtype]
    torch.cuda.synchronize()
    if B * Hk * max(splits, 1) <= 512:
        # merged in the kernel: every merge leaves its unit's arrival word at
        # (tag, done, 0 arrivals)
        words = ops._workspace("decode", torch.device(DEV), 1)[:ops.DECODE_COUNTER_BYTES].view(torch.int64)
        assert int((words[:B * Hk] & 0x7fffffff).count_nonzero()) == 0
        assert int(((words[:B * Hk] >> 31) & 1).sum()) == B * Hk


@pytest.mark.parametrize("S", [300, 575, 1200, 2431, 129])
def test_decode_split_merge_as_the_shape_changes(S):
    """Launches of different lengths on one workspace, issued back to back
    (the split count and the partials' addresses change with S; decode of a
    growing cache crosses such steps): each merges only its own launch's
    partials."""
    B, Hq, Hk, D = 1, 32, 8, 128
    dtype = torch.float16
    q = _randn((B, Hq, 1, D), 40 + S, dtype)
    k = _randn((B, Hk, S, D), 41 + S, dtype)
    v = _randn((B, Hk, S, D), 42 + S, dtype)
    sc = 1.0 / math.sqrt(D)
    want = ref.decode_attention(q, k, v, sc)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    outs = [ops.decode_attention(qd, kd, vd, sc, num_splits=n) for n in (0, 3, 0, 7)]
    torch.cuda.synchronize()
    for out in outs:
        assert np.abs(out.float().cpu().numpy() - want).max() <= TOL[dtype]
    assert torch.equal(outs[0], outs[2])


def test_decode_split_merge_in_a_replayed_graph():
    """One layer's append+decode (8 KV heads, 545 keys: five splits merged
    inside the launch) captured in a graph and replayed with new queries
    and tokens each time: every replay's output equals an eager launch on
    the same inputs, bit for bit, so no replay merges partials an earlier
    replay left (a replay repeats the launch's tag: every workgroup's
    partial has landed before it counts in)."""
    B, Hq, Hk, D, S = 1, 32, 8, 128, 545
    dtype = torch.float16
    dev = torch.device(DEV)
    g = torch.Generator(device=dev).manual_seed(50)
    k, v = kv_rows((B, Hk), S + 7, D, dtype, dev)
    k.copy_(torch.randn((B, Hk, S + 7, D), generator=g, device=dev, dtype=dtype))
    v.copy_(torch.randn((B, Hk, S + 7, D), generator=g, device=dev, dtype=dtype))
    q = torch.randn((B, Hq, D), generator=g, device=dev, dtype=dtype)
    kn = torch.randn((B, Hk, 1, D), generator=g, device=dev, dtype=dtype)
    vn = torch.randn((B, Hk, 1, D), generator=g, device=dev, dtype=dtype)
    out = torch.empty((B, Hq, D), device=dev, dtype=dtype)
    sc = 1.0 / math.sqrt(D)
    st = torch.cuda.Stream(dev)
    with torch.cuda.stream(st):
        ops.decode_attention_append(q, k[:, :, :S], v[:, :, :S], kn, vn, sc, out=out)   # the stream's workspace
    st.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        ops.decode_attention_append(q, k[:, :, :S], v[:, :, :S], kn, vn, sc, out=out)
    for rep in range(6):
        with torch.cuda.stream(st):
            q.copy_(torch.randn((B, Hq, D), generator=g, device=dev, dtype=dtype))
            kn.copy_(torch.randn((B, Hk, 1, D), generator=g, device=dev, dtype=dtype))
            vn.copy_(torch.randn((B, Hk, 1, D), generator=g, device=dev, dtype=dtype))
        st.synchronize()
        graph.replay()
        st.synchronize()
        got = out.clone()
        with torch.cuda.stream(st):
            want = ops.decode_attention_append(q, k[:, :, :S], v[:, :, :S], kn, vn, sc)
        st.synchronize()
        assert torch.equal(got, want), rep
        kk = torch.cat([k[:, :, :S - 1], kn], 2).cpu()
        vv = torch.cat([v[:, :, :S - 1], vn], 2).cpu()
        oracle = ref.decode_attention(q[:, :, None].cpu(), kk, vv, sc)
        assert np.abs(got.float().cpu().numpy().reshape(oracle.shape) - oracle).max() <= TOL[dtype], rep
    del graph


@pytest.mark.parametrize("S,splits", [(2431, 0), (2431, 5), (545, 0)])
def test_decode_bf16_error_is_the_output_rounding(S, splits):
    """bf16 P.V carries each probability as a high and a low bf16 part, so the
    output's mean error against the fp64 oracle is the bf16 rounding of the
    exact result itself (rounding p to bf16 alone had made it 1.3-1.5 times
    that); V is scaled x3 so that the rounding is well above fp32 noise."""
    B, Hq, Hk, D = 1, 32, 8, 128
    dt = torch.bfloat16
    q, k = _randn((B, Hq, 1, D), 60, dt), _randn((B, Hk, S, D), 61, dt)
    v = _randn((B, Hk, S, D), 62, dt, scale=3.0)
    sc = 1.0 / math.sqrt(D)
    out = ops.decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), sc, num_splits=splits).double().cpu().numpy()
    want = ref.decode_attention(q, k, v, sc)
    rounding = np.abs(torch.from_numpy(want).to(dt).double().numpy() - want).mean()
    assert np.abs(out - want).mean() <= 1.05 * rounding


def _word(tag, low):
    """An arrival word [tag : 32 | low : 32] as a signed int64."""
    w = (tag << 32) | low
    return w - (1 << 64) if w >= 1 << 63 else w


@pytest.mark.parametrize("fill", ["random", "ones", "counts_left_behind", "finished_under_another_tag"])
def test_decode_split_merge_ignores_stale_counter_words(fill):
    """The in-kernel merge's arrival words may hold anything before a launch
    (a launch cut short, a caller's uninitialised workspace): each launch
    counts only on words left by the workspace's previous launch, so the
    output is the same bits as on a zeroed block, and a second launch on
    the words the first one left is the same again."""
    B, Hq, Hk, S, D, splits = 1, 32, 8, 2431, 128, 16
    dtype = torch.float16
    q = _randn((B, Hq, 1, D), 31, dtype).to(DEV)
    k = _randn((B, Hk, S, D), 32, dtype).to(DEV)
    v = _randn((B, Hk, S, D), 33, dtype).to(DEV)
    sc = 1.0 / math.sqrt(D)
    ws = ops._workspace("decode", torch.device(DEV), 1)     # the stream's decode workspace
    ws[:ops.DECODE_COUNTER_BYTES].zero_()
    clean = ops.decode_attention(q, k, v, sc, num_splits=splits).clone()
    torch.cuda.synchronize()
    ws = ops._workspace("decode", torch.device(DEV), 1)
    words = ws[:ops.DECODE_COUNTER_BYTES].view(torch.int64)
    g = torch.Generator().manual_seed(34)
    if fill == "random":
        # arrival words, generations and the split partials' room alike
        words.copy_(torch.randint(-(1 << 62), 1 << 62, words.shape, generator=g))
        ws[ops.DECODE_COUNTER_BYTES:].copy_(torch.randint(0, 256, (ws.numel() - ops.DECODE_COUNTER_BYTES,),
                                                          generator=g, dtype=torch.uint8))
    elif fill == "ones":
        words.fill_(-1)
    elif fill == "counts_left_behind":
        # another launch's tag with splits-1 arrivals: a plain counter would
        # let this launch's first arrival merge alone
        words.fill_(_word(0xfffffffe, splits - 1))
    else:
        # the done bit, as a finished launch leaves it, but under a tag that
        # is not the workspace's last one, and with splits-1 arrivals
        words.fill_(_word(0xfffffffe, 0x80000000 | (splits - 1)))
    torch.cuda.synchronize()
    out = ops.decode_attention(q, k, v, sc, num_splits=splits)
    again = ops.decode_attention(q, k, v, sc, num_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(out, clean), fill
    assert torch.equal(again, clean), fill
    assert np.abs(out.float().cpu().numpy() - ref.decode_attention(q.cpu(), k.cpu(), v.cpu(), sc)).max() <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_decode_mask_and_held_slot(dtype):
    B, Hq, Hk, R, n, D = 2, 32, 8, 64, 300, 128
    S = R + n
    q = _randn((B, Hq, 1, D), 4, dtype)
    k = _randn((B, Hk, S, D), 5, dtype)
    v = _randn((B, Hk, S, D), 6, dtype)
    g = torch.Generator().manual_seed(7)
    valid = torch.rand((B, R), generator=g) < 0.7
    pos = torch.randint(0, 2000, (B, R), generator=g)
    cur = torch.tensor([1500], dtype=torch.int64)
    keep_mem = valid & (pos <= cur)
    mask = torch.cat([keep_mem, torch.ones((B, n), dtype=torch.bool)], dim=1)
    sc = 1.0 / math.sqrt(D)
    want = ref.decode_attention(q, k, v, sc, mask)
    # explicit (B,S) mask, as triton_evict_attention_forward takes it
    out1 = ops.decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), sc, mask=mask.to(DEV))
    # held-slot form: the kernel evaluates valid & pos <= cur_pos itself
    out2 = ops.decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), sc, held_len=R, held_pos=pos.to(DEV),
                                held_valid=valid.to(DEV), cur_pos=cur.to(DEV))
    for out in (out1, out2):
        assert np.abs(out.float().cpu().numpy() - want).max() <= TOL[dtype]


def test_decode_per_head_held_positions():
    B, Hq, Hk, R, n, D = 1, 32, 8, 16, 100, 128
    S = R + n
    dtype = torch.float16
    q, k, v = _randn((B, Hq, 1, D), 8, dtype), _randn((B, Hk, S, D), 9, dtype), _randn((B, Hk, S, D), 10, dtype)
    g = torch.Generator().manual_seed(11)
    valid = torch.rand((B, Hk, R), generator=g) < 0.5
    pos = torch.randint(0, 100, (B, Hk, R), generator=g)
    cur = torch.tensor([60], dtype=torch.int64)
    out = ops.decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), 0.1, held_len=R, held_pos=pos.to(DEV),
                               held_valid=valid.to(DEV), cur_pos=cur.to(DEV)).float().cpu().numpy()
    for h in range(Hk):
        m = torch.cat([valid[:, h] & (pos[:, h] <= 60), torch.ones((B, n), dtype=torch.bool)], 1)
        want = ref.decode_attention(q[:, h * 4:(h + 1) * 4], k[:, h:h + 1], v[:, h:h + 1], 0.1, m)
        assert np.abs(out[:, h * 4:(h + 1) * 4] - want).max() <= 2e-3


def test_decode_all_masked_is_nan_like_reference():
    # kernels.py:55-69: every score -1e35 -> l = 0 -> 0/0.
    B, Hq, Hk, S, D = 1, 4, 1, 10, 16
    q, k, v = _randn((B, Hq, 1, D), 1, torch.float16), _randn((B, Hk, S, D), 2, torch.float16), \
        _randn((B, Hk, S, D), 3, torch.float16)
    mask = torch.zeros((B, S), dtype=torch.bool)
    out = ops.decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), 0.25, mask=mask.to(DEV))
    assert torch.isnan(out.float()).all()


def test_decode_single_unmasked_key_returns_its_value():
    B, Hq, Hk, S, D = 1, 8, 2, 77, 128
    q, k, v = _randn((B, Hq, 1, D), 1, torch.float16), _randn((B, Hk, S, D), 2, torch.float16), \
        _randn((B, Hk, S, D), 3, torch.float16)
    mask = torch.zeros((B, S), dtype=torch.bool)
    mask[0, 41] = True
    out = ops.decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), 0.1, mask=mask.to(DEV)).cpu()
    for h in range(Hq):
        assert torch.equal(out[0, h], v[0, h // 4, 41])


def test_decode_strided_views_and_evict_score():
    # hot buffer view: (B,Hk,cap,D) storage, attended prefix of n rows
    B, Hq, Hk, cap, n, D = 2, 32, 8, 700, 531, 128
    dtype = torch.float16
    kbuf, vbuf = _randn((B, Hk, cap, D), 12, dtype), _randn((B, Hk, cap, D), 13, dtype)
    q = _randn((B, Hq, 1, D), 14, dtype)
    k, v = kbuf[:, :, :n], vbuf[:, :, :n]
    out, loss, idx = ops.decode_attention(q.to(DEV), kbuf.to(DEV)[:, :, :n], vbuf.to(DEV)[:, :, :n], 0.088,
                                          with_evict=True)
    want = ref.decode_attention(q, k, v, 0.088)
    assert np.abs(out.float().cpu().numpy() - want).max() <= 2e-3
    want_loss, _ = ref.evict_scores(q, k, v, 0.088)
    got_loss = loss.cpu().numpy()
    assert np.allclose(got_loss, want_loss, rtol=2e-3, atol=1e-6)
    for b in range(B):
        # the chosen index is a minimiser of the oracle loss up to fp16 rounding
        assert want_loss[b, int(idx[b])] <= want_loss[b].min() * (1 + 2e-3) + 1e-7


APPEND_CASES = [
    # B, Hq, Hk, cap, n (cached rows), D, dtype, splits
    (1, 32, 8, 700, 573, 128, torch.float16, 0),    # 8k/budget-512 hot buffer, mid-decode
    (1, 32, 8, 700, 573, 128, torch.bfloat16, 0),
    (1, 32, 8, 600, 543, 128, torch.float32, 0),
    (2, 8, 2, 300, 199, 16, torch.float32, 0),      # reference test geometry
    (4, 32, 8, 2500, 2430, 128, torch.float16, 0),  # batched, several splits
    (1, 32, 8, 700, 573, 128, torch.float16, 1),    # forced single split
    (1, 32, 8, 700, 573, 128, torch.float16, 7),    # forced ragged splits
    (3, 16, 4, 8, 0, 64, torch.float16, 0),         # empty cache: the new token alone
    (1, 64, 8, 300, 250, 128, torch.float16, 0),    # group of 8
    (1, 8, 1, 1000, 900, 256, torch.bfloat16, 0),   # one KV head, wide head_dim
    (2, 16, 4, 3100, 3000, 64, torch.bfloat16, 0),  # several tiles per wave, head_dim 64
]


@pytest.mark.parametrize("B,Hq,Hk,cap,n,D,dtype,splits", APPEND_CASES)
def test_decode_append_matches_append_then_decode(B, Hq, Hk, cap, n, D, dtype, splits):
    """The fused launch writes the token into row n of the hot buffer and
    attends over rows 0..n: same buffer as append_rows, same output as the
    oracle on the concatenated cache."""
    kbuf, vbuf = _randn((B, Hk, cap, D), 21, dtype), _randn((B, Hk, cap, D), 22, dtype)
    q = _randn((B, Hq, 1, D), 23, dtype)
    kn, vn = _randn((B, Hk, 1, D), 24, dtype), _randn((B, Hk, 1, D), 25, dtype)
    sc = 1.0 / math.sqrt(D)
    kd, vd = kbuf.to(DEV), vbuf.to(DEV)
    out = ops.decode_attention_append(q.to(DEV), kd[:, :, :n + 1], vd[:, :, :n + 1], kn.to(DEV), vn.to(DEV), sc,
                                      num_splits=splits)
    kw, vw = kbuf.clone(), vbuf.clone()
    kw[:, :, n:n + 1], vw[:, :, n:n + 1] = kn, vn
    assert torch.equal(kd.cpu(), kw) and torch.equal(vd.cpu(), vw)
    want = ref.decode_attention(q, kw[:, :, :n + 1], vw[:, :, :n + 1], sc)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    assert np.abs(got - want).max() <= TOL[dtype], np.abs(got - want).max()
    # the two-launch path on a second copy of the buffer agrees within the tolerance
    k2, v2 = kbuf.to(DEV), vbuf.to(DEV)
    ops.append_rows(n, kn.to(DEV), k2, vn.to(DEV), v2)
    out2 = ops.decode_attention(q.to(DEV), k2[:, :, :n + 1], v2[:, :, :n + 1], sc, num_splits=splits)
    assert np.abs(out2.float().cpu().numpy() - got).max() <= TOL[dtype]
    if n == 0:
        for h in range(Hq):
            assert torch.equal(out[:, h].cpu(), vn[:, h // (Hq // Hk), 0])


@pytest.mark.parametrize("per_head", [False, True])
def test_decode_append_held_slot_mask_pre_and_pos(per_head):
    """Held-slot masking and an explicit mask apply to the cached rows; the
    new token is always attended; its pre-RoPE key and position land in row n."""
    B, Hq, Hk, R, n0, cap, D = 2, 32, 8, 64, 400, 600, 128
    n = R + n0
    dtype = torch.float16
    kbuf, vbuf, pbuf = (_randn((B, Hk, cap, D), s, dtype) for s in (31, 32, 33))
    posbuf = torch.randint(0, 5000, (B, cap), generator=torch.Generator().manual_seed(34))
    q = _randn((B, Hq, 1, D), 35, dtype)
    kn, vn, pn = (_randn((B, Hk, 1, D), s, dtype) for s in (36, 37, 38))
    posn = torch.tensor([[4321], [4322]], dtype=torch.int64)
    g = torch.Generator().manual_seed(39)
    shape = (B, Hk, R) if per_head else (B, R)
    valid = torch.rand(shape, generator=g) < 0.7
    hpos = torch.randint(0, 2000, shape, generator=g)
    cur = torch.tensor([1500], dtype=torch.int64)
    mask = torch.rand((B, n), generator=g) < 0.9
    kd, vd, pd, posd = kbuf.to(DEV), vbuf.to(DEV), pbuf.to(DEV), posbuf.to(DEV)
    out = ops.decode_attention_append(q.to(DEV), kd[:, :, :n + 1], vd[:, :, :n + 1], kn.to(DEV), vn.to(DEV), 0.088,
                                      pre=(pn.to(DEV), pd), pos=(posn.to(DEV), posd), mask=mask.to(DEV),
                                      held_len=R, held_pos=hpos.to(DEV), held_valid=valid.to(DEV),
                                      cur_pos=cur.to(DEV)).float().cpu().numpy()
    kw, vw, pw, posw = kbuf.clone(), vbuf.clone(), pbuf.clone(), posbuf.clone()
    kw[:, :, n:n + 1], vw[:, :, n:n + 1], pw[:, :, n:n + 1] = kn, vn, pn
    posw[:, n] = posn[:, 0]
    for got, want in ((kd, kw), (vd, vw), (pd, pw), (posd, posw)):
        assert torch.equal(got.cpu(), want)
    G = Hq // Hk
    for h in range(Hk):
        vh = valid[:, h] if per_head else valid
        ph = hpos[:, h] if per_head else hpos
        held = torch.cat([vh & (ph <= cur), torch.ones((B, n0), dtype=torch.bool)], 1)
        m = torch.cat([held & mask, torch.ones((B, 1), dtype=torch.bool)], 1)
        want = ref.decode_attention(q[:, h * G:(h + 1) * G], kw[:, h:h + 1, :n + 1], vw[:, h:h + 1, :n + 1], 0.088, m)
        assert np.abs(out[:, h * G:(h + 1) * G] - want).max() <= 2e-3, h


def test_packed_append_rows_equal_the_scalar_entry():
    """decode_append_rows (hc_decode_attn_append_packed over a reused argument
    struct) and decode_attention_append (hc_decode_attn_append) on twin
    buffers: identical outputs and rows, step after step, across a held slot
    with per-head positions, growth of the buffer (a new storage, so a new
    struct), a stream switch (the workspace follows the stream) and a second
    query-head count on the same storage."""
    from hotcold_kv.hot_buffer import HotBuffer
    B, Hq, Hk, D, R, n0 = 2, 32, 8, 128, 16, 300
    dtype = torch.float16
    g = torch.Generator().manual_seed(7)
    bufs = [HotBuffer(B, Hk, D, dtype, DEV, n0 + 8, held=R, with_pre=True, with_pos=True) for _ in range(2)]
    k0, v0, p0 = (torch.randn((B, Hk, n0, D), generator=g).to(dtype).to(DEV) for _ in range(3))
    pos0 = torch.arange(n0, device=DEV).view(1, -1).expand(B, -1).contiguous()
    hk, hv = torch.randn((B, Hk, R, D), generator=g).to(dtype), torch.randn((B, Hk, R, D), generator=g).to(dtype)
    for b in bufs:
        b.append(k0, v0, p0, pos0)
        kb, vb = b.held_storage()
        kb[:, :, :R], vb[:, :, :R] = hk.to(DEV), hv.to(DEV)
    hpos = torch.randint(0, n0 + 40, (B, Hk, R), generator=g).to(DEV)
    hval = (torch.rand((B, Hk, R), generator=g) < 0.8).to(DEV)
    # a second held slot (new tensors, as an injection makes) from step 12 on,
    # and a shorter one from step 18 on: the struct's held fields follow
    hpos2 = torch.randint(0, n0 + 40, (B, Hk, R), generator=g).to(DEV)
    hval2 = (torch.rand((B, Hk, R), generator=g) < 0.5).to(DEV)
    side = torch.cuda.Stream(device=DEV)
    for step in range(24):                                   # grows past n0 + 8 on step 8
        q = torch.randn((B, Hq, 1, D), generator=g).to(dtype).to(DEV)
        kn, vn, pn = (torch.randn((B, Hk, 1, D), generator=g).to(dtype).to(DEV) for _ in range(3))
        posn = torch.full((B, 1), n0 + step, dtype=torch.int64, device=DEV)
        hp_, hv_, R_ = (hpos, hval, R) if step < 12 else ((hpos2, hval2, R) if step < 18 else (hpos2, hval2, R // 2))
        held = (hp_, hv_, R_) if step % 3 else None
        on_side = step in (5, 6, 15)
        if on_side:
            side.wait_stream(torch.cuda.current_stream(DEV))
        with torch.cuda.stream(side) if on_side else contextlib.nullcontext():
            outs = []
            for i, b in enumerate(bufs):
                b.ensure(b.n + 1)
                r = R_ if held else 0
                lo, S = b.held - r, r + b.n + 1
                if i == 0:
                    o = ops.decode_append_rows(q, b.st, lo, S, kn, vn, 0.088, p_new=pn, pos_new=posn, held=held,
                                               cur_pos=posn if held else None, keepdim=True)
                else:
                    st = b.st
                    o = ops.decode_attention_append(
                        q, st["k"][:, :, lo:lo + S], st["v"][:, :, lo:lo + S], kn, vn, 0.088,
                        pre=(pn, st["p"][:, :, lo:]), pos=(posn, st["pos"][:, lo:]), held_len=r,
                        held_pos=hp_ if held else None, held_valid=hv_ if held else None,
                        cur_pos=posn[0] if held else None).unsqueeze(2)
                b.n += 1
                outs.append(o)
        torch.cuda.current_stream(DEV).wait_stream(side)
        assert torch.equal(outs[0], outs[1]), step
    torch.cuda.synchronize()
    rows = bufs[0].held + bufs[0].n
    assert bufs[1].held + bufs[1].n == rows and bufs[0].cap > n0 + 8
    for name in ("k", "v", "p"):
        assert torch.equal(bufs[0].st[name][:, :, :rows], bufs[1].st[name][:, :, :rows]), name
    assert torch.equal(bufs[0].st["pos"][:, :rows], bufs[1].st["pos"][:, :rows])
    # a second query-head count on the same storage gets its own struct
    q8 = torch.randn((B, 8, 1, D), generator=g).to(dtype).to(DEV)
    kn, vn = (torch.randn((B, Hk, 1, D), generator=g).to(dtype).to(DEV) for _ in range(2))
    b0 = bufs[0]
    b0.ensure(b0.n + 1)
    o8 = ops.decode_append_rows(q8, b0.st, b0.held, b0.n + 1, kn, vn, 0.088)
    want = ref.decode_attention(q8.cpu(), b0.st["k"][:, :, b0.held:b0.held + b0.n + 1].cpu(),
                                b0.st["v"][:, :, b0.held:b0.held + b0.n + 1].cpu(), 0.088)
    assert np.abs(o8.float().cpu().numpy() - want).max() <= 2e-3


def test_packed_append_rows_argument_errors():
    """decode_append_rows rejects, before any launch, rows of the wrong shape,
    dtype or device, a held slot that reaches the token's row, and pre-RoPE /
    position rows for a buffer that keeps none."""
    from hotcold_kv.hot_buffer import HotBuffer
    B, Hq, Hk, D = 1, 8, 2, 64
    b = HotBuffer(B, Hk, D, torch.float16, DEV, 32, held=4)
    b.append(*(torch.zeros((B, Hk, 8, D), dtype=torch.float16, device=DEV) for _ in range(2)))
    q = torch.zeros((B, Hq, 1, D), dtype=torch.float16, device=DEV)
    kn = torch.zeros((B, Hk, 1, D), dtype=torch.float16, device=DEV)
    lo, S = b.held, b.n + 1
    ops.decode_append_rows(q, b.st, lo, S, kn, kn, 0.1)      # the valid call
    with pytest.raises(RuntimeError, match="q must be"):
        ops.decode_append_rows(torch.zeros((B, Hq, 2, D), dtype=torch.float16, device=DEV), b.st, lo, S, kn, kn, 0.1)
    with pytest.raises(RuntimeError, match="k_new must be"):
        ops.decode_append_rows(q, b.st, lo, S, kn.float(), kn, 0.1)
    with pytest.raises(RuntimeError, match="v_new must be"):
        ops.decode_append_rows(q, b.st, lo, S, kn, kn.cpu(), 0.1)
    with pytest.raises(RuntimeError, match="unit last stride"):
        ops.decode_append_rows(q, b.st, lo, S, kn, torch.zeros((B, Hk, 1, 2 * D), dtype=torch.float16,
                                                                device=DEV)[..., ::2], 0.1)
    with pytest.raises(RuntimeError, match="outside the buffer"):
        ops.decode_append_rows(q, b.st, lo, 10 ** 6, kn, kn, 0.1)
    with pytest.raises(RuntimeError, match="pre-RoPE"):
        ops.decode_append_rows(q, b.st, lo, S, kn, kn, 0.1, p_new=kn)
    hp = torch.zeros((B, Hk, 4), dtype=torch.int64, device=DEV)
    hv = torch.ones((B, Hk, 4), dtype=torch.bool, device=DEV)
    with pytest.raises(RuntimeError, match="held"):
        ops.decode_append_rows(q, b.st, 0, 4, kn, kn, 0.1, held=(hp, hv, 4), cur_pos=hp[0, 0, :1])
    o = ops.decode_append_rows(q, b.st, 0, 4 + S, kn, kn, 0.1, held=(hp, hv, 4), cur_pos=hp[0, 0, :1])
    assert o.shape == (B, Hq, D) and torch.isfinite(o.float()).all()


def test_decode_append_argument_errors():
    q = torch.zeros((1, 8, 1, 64), dtype=torch.float16, device=DEV)
    k = torch.zeros((1, 2, 10, 64), dtype=torch.float16, device=DEV)
    kn = torch.zeros((1, 2, 64), dtype=torch.float16, device=DEV)
    hp = torch.zeros((1, 10), dtype=torch.int64, device=DEV)
    hv = torch.ones((1, 10), dtype=torch.bool, device=DEV)
    # the held slot may not reach the row the token is written to
    with pytest.raises(RuntimeError, match="held"):
        ops.decode_attention_append(q, k, k.clone(), kn, kn, 0.1, held_len=10, held_pos=hp, held_valid=hv)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        ops.decode_attention_append(q, k, k.clone(), kn[:, :1], kn, 0.1)


# ---------------------------------------------------------------------------
# SnapKV compaction
# ---------------------------------------------------------------------------
SCORE_CASES = [
    # B, Hq, Hk, S, D, W, dtype, pool, pooling
    (2, 8, 2, 200, 16, 16, torch.float32, 7, "maxpool"),   # test_baselines.py geometry
    (2, 8, 2, 200, 16, 16, torch.float32, 7, "avgpool"),
    (1, 32, 8, 2048, 128, 32, torch.float32, 7, "maxpool"),  # plumbing config
    (1, 32, 8, 1000, 128, 32, torch.float16, 7, "maxpool"),
    (1, 32, 8, 1000, 128, 64, torch.bfloat16, 7, "maxpool"),
    (2, 12, 4, 333, 64, 40, torch.float16, 5, "maxpool"),    # ragged window row block
    (1, 6, 4, 150, 32, 8, torch.float16, 1, "maxpool"),      # Hq % Hk != 0, no pooling
    (1, 4, 4, 20, 16, 32, torch.float32, 7, "maxpool"),      # window longer than the prompt
    # few rows: each row sum split across 4 waves, S not a multiple of 256
    (1, 8, 2, 3000, 64, 7, torch.float16, 7, "maxpool"),     # S % 4 == 0 (vector row loads)
    (1, 8, 2, 3001, 128, 7, torch.bfloat16, 5, "avgpool"),   # S % 4 != 0 (scalar row loads)
    # enough rows and keys for several 128-key chunks per logits workgroup
    (8, 32, 8, 4160, 128, 32, torch.float16, 7, "maxpool"),
    # a long window without pooling: importance over mirrored key pairs
    (1, 4, 2, 2500, 64, 1100, torch.float16, 1, "maxpool"),
    (2, 2, 2, 1301, 32, 1301, torch.float32, 1, "maxpool"),
]


@pytest.mark.parametrize("B,Hq,Hk,S,D,W,dtype,pool,pooling", SCORE_CASES)
def test_snapkv_scores_bit_exact(B, Hq, Hk, S, D, W, dtype, pool, pooling):
    q = _randn((B, Hq, S, D), 21, dtype)
    k = _randn((B, Hk, S, D), 22, dtype)
    sc = 1.0 / math.sqrt(D)
    got = ops.snapkv_scores(q.to(DEV), k.to(DEV), W, sc, pool, pooling).cpu()
    want = ref.window_scores(q, k, W, sc, pool, pooling)
    assert torch.equal(got, want), (got - want).abs().max()


def test_snapkv_scores_and_keep_llama8b_8k_layer():
    """One layer of the 8k fp16 workload with needles: scores, kept indices
    and the compacted K/V are bit-exact."""
    w = synthetic.WORKLOADS["llama8b_8k_b512"]
    p = synthetic.make_prompt(w, layer=3, seed=0, device="cpu")
    qd, kd, vd = p["q_post"].to(DEV), p["k_post"].to(DEV), p["v"].to(DEV)
    got = ops.snapkv_scores(qd, kd, w.window, w.scaling, w.pool, "maxpool")
    want = ref.window_scores(p["q_post"], p["k_post"], w.window, w.scaling, w.pool, "maxpool")
    assert torch.equal(got.cpu(), want)
    keep = ops.keep_index(got, w.window, w.budget)
    want_keep = ref.keep_index(want, w.window, w.budget)
    assert torch.equal(keep.cpu(), want_keep)
    # the needles are selected
    needles = p["needles"][0]
    for h in range(w.hk):
        assert set(needles[h].tolist()) <= set(want_keep[0, h].tolist())
    kk = ops.gather_kv(kd, keep)
    vv = ops.gather_kv(vd, keep)
    assert torch.equal(kk.cpu(), ref.gather_kv(p["k_post"], want_keep))
    assert torch.equal(vv.cpu(), ref.gather_kv(p["v"], want_keep))


def test_snapkv_scores_and_keep_golden_fixtures():
    """Kernels reproduce the committed fixtures (tests/golden) bit for bit."""
    from test_oracle import load_golden

    for case, (q, k, W, pool, budget, sc, want_scores, want_keep) in load_golden().items():
        scores = ops.snapkv_scores(q.to(DEV), k.to(DEV), W, sc, pool, "maxpool")
        assert torch.equal(scores.cpu(), want_scores), case
        assert torch.equal(ops.keep_index(scores, W, budget).cpu(), want_keep), case


def test_rawsum_scores_and_head_mean():
    B, Hq, Hk, S, T, D = 2, 32, 8, 700, 40, 128
    q = _randn((B, Hq, T, D), 31, torch.float16)
    k = _randn((B, Hk, S, D), 32, torch.float16)
    got = ops.snapkv_scores(q.to(DEV), k.to(DEV), 32, 0.0, mode="rawsum")
    want = ref.window_scores(q, k, 32, 0.0, mode="rawsum")
    assert torch.equal(got.cpu(), want)
    assert torch.equal(ops.head_mean(got).cpu(), ref.head_mean(want))


@pytest.mark.parametrize("S,window,budget", [(200, 16, 64), (100, 8, 30), (50, 32, 20), (10, 32, 512),
                                             (8192, 32, 512), (5000, 64, 5000), (4097, 1, 2)])
def test_keep_index_matches_oracle(S, window, budget):
    B, H = 2, 3
    g = torch.Generator().manual_seed(S)
    # coarse values: many exact ties, like max-pool plateaus
    sc = torch.randint(0, 50, (B, H, S), generator=g).float() / 7.0
    got, gev = ops.keep_index(sc.to(DEV), window, budget, return_evicted=True)
    want, wev = ref.keep_index(sc, window, budget, return_evicted=True)
    assert torch.equal(got.cpu(), want)
    assert torch.equal(gev.cpu(), wev)


def test_keep_index_special_values():
    sc = torch.tensor([[[0.0, -0.0, 1.0, float("inf"), -float("inf"), 0.5, -0.0, 0.0, 2.0, 2.0, 0.1, 0.2]]])
    for budget in range(1, 12):
        got = ops.keep_index(sc.to(DEV), 2, budget).cpu()
        assert torch.equal(got, ref.keep_index(sc, 2, budget)), budget
    # NaN ranks above +inf (torch.topk's order), NaNs tie with each other
    sc = torch.tensor([[[float("inf"), float("nan"), 1.0, float("inf"), float("nan"), -0.0, 0.0, float("nan"),
                         -float("inf"), 2.0, 0.5, 0.25]]])
    for budget in range(1, 12):
        got, gev = ops.keep_index(sc.to(DEV), 2, budget, return_evicted=True)
        want, wev = ref.keep_index(sc, 2, budget, return_evicted=True)
        assert torch.equal(got.cpu(), want) and torch.equal(gev.cpu(), wev), budget


def _chunk_scores(B, H, S, kind, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "coarse":     # many exact ties, like max-pool plateaus
        return torch.randint(0, 50, (B, H, S), generator=g).float() / 7.0
    if kind == "equal":
        return torch.full((B, H, S), 1.5)
    sc = torch.randn((B, H, S), generator=g)
    if kind == "special":    # NaN, +-inf and +-0 sprinkled over the row
        u = torch.rand((B, H, S), generator=g)
        sc[u < 0.002] = float("nan")
        sc[(u >= 0.002) & (u < 0.004)] = float("inf")
        sc[(u >= 0.004) & (u < 0.006)] = -float("inf")
        sc[(u >= 0.006) & (u < 0.02)] = -0.0
        sc[(u >= 0.02) & (u < 0.03)] = 0.0
    return sc


# rows < 256 and prefixes longer than 32768 keys: the chunked selection
@pytest.mark.parametrize("B,H,S,window,budget,kind", [
    (1, 8, 32768 + 65, 64, 1024, "coarse"),      # a last chunk of one key
    (2, 4, 40000, 64, 4096, "coarse"),            # a partial last chunk
    (4, 8, 65536, 64, 4096, "normal"),            # the 64k x 4 layer's rows
    (1, 1, 40000, 0, 39999, "coarse"),            # all but one key kept
    (1, 3, 50000, 32, 40, "special"),             # few kept, NaN / inf among them
    (3, 5, 33000, 7, 32990, "equal"),             # one tie class over the whole row
    (2, 2, 40960, 0, 1, "special"),               # one key kept, five whole chunks
])
def test_keep_index_chunked_matches_oracle(B, H, S, window, budget, kind):
    from hotcold_kv import _native as N
    assert N.lib().hc_topk_keep_workspace_size(B, H, S, window, budget) > 0    # the chunked path runs
    sc = _chunk_scores(B, H, S, kind, S + budget)
    scd = sc.to(DEV)
    got, gev = ops.keep_index(scd, window, budget, return_evicted=True)
    want, wev = ref.keep_index(sc, window, budget, return_evicted=True)
    assert torch.equal(got.cpu(), want)
    assert torch.equal(gev.cpu(), wev)
    # the one-workgroup-per-row kernel, called directly, gives the same outputs
    one, oev = torch.empty_like(got), torch.empty_like(gev)
    N.check(N.lib().hc_topk_keep(B, H, S, scd.data_ptr(), scd.stride(0), scd.stride(1), window, budget,
                                 one.data_ptr(), oev.data_ptr(), ops._stream_handle(scd.device)), "hc_topk_keep")
    assert torch.equal(one, got) and torch.equal(oev, gev)


def test_keep_index_chunked_workspace_reuse_and_size_check():
    from hotcold_kv import _native as N
    B, H, S, window, budget = 2, 4, 40000, 16, 500
    need = N.lib().hc_topk_keep_workspace_size(B, H, S, window, budget)
    assert need > 0
    ws = torch.full((need,), 0xA5, dtype=torch.uint8, device=DEV)    # garbage: the call needs no clearing
    for seed in (1, 2):                                               # the same workspace twice in a row
        sc = _chunk_scores(B, H, S, "coarse", seed).to(DEV)
        keep = torch.empty((B, H, budget), dtype=torch.int64, device=DEV)
        N.check(N.lib().hc_topk_keep_ws(B, H, S, sc.data_ptr(), sc.stride(0), sc.stride(1), window, budget,
                                        keep.data_ptr(), None, ws.data_ptr(), need,
                                        ops._stream_handle(sc.device)), "hc_topk_keep_ws")
        assert torch.equal(keep.cpu(), ref.keep_index(sc.cpu(), window, budget))
    rc = N.lib().hc_topk_keep_ws(B, H, S, sc.data_ptr(), sc.stride(0), sc.stride(1), window, budget,
                                 keep.data_ptr(), None, ws.data_ptr(), need - 1, ops._stream_handle(sc.device))
    assert rc == N.HC_ERR_INVALID


def test_keep_index_chunked_in_a_replayed_graph():
    """The chunked selection captured in a graph and replayed over new scores:
    its workspace, allocated at capture and never cleared by the host, is set
    up by the chain's own first kernel on every replay (no memset node)."""
    from hotcold_kv import _native as N
    B, H, S, window, budget = 2, 4, 40000, 16, 500
    assert N.lib().hc_topk_keep_workspace_size(B, H, S, window, budget) > 0
    dev = torch.device(DEV)
    sc = _chunk_scores(B, H, S, "coarse", 1).to(dev)
    st = torch.cuda.Stream(dev)
    with torch.cuda.stream(st):
        ops.keep_index(sc, window, budget, return_evicted=True)     # outside the capture first
    st.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        keep, ev = ops.keep_index(sc, window, budget, return_evicted=True)
    for rep, kind in enumerate(("coarse", "special", "normal", "coarse", "equal")):
        new = _chunk_scores(B, H, S, kind, 10 + rep)
        with torch.cuda.stream(st):
            sc.copy_(new.to(dev))
        st.synchronize()
        graph.replay()
        st.synchronize()
        want, wev = ref.keep_index(new, window, budget, return_evicted=True)
        assert torch.equal(keep.cpu(), want), rep
        assert torch.equal(ev.cpu(), wev), rep
        with torch.cuda.stream(st):                                  # the program's own work between replays
            ops.keep_index(sc, window, budget)
        st.synchronize()
    del graph


def test_gather_shared_index_with_positions():
    B, Hk, S, D, n = 2, 8, 300, 128, 77
    dtype = torch.float16
    k, v, kp = (_randn((B, Hk, S, D), s, dtype) for s in (41, 42, 43))
    pos = torch.arange(S).unsqueeze(0).expand(B, S) * 3 + 5
    g = torch.Generator().manual_seed(44)
    idx = torch.stack([torch.sort(torch.randperm(S, generator=g)[:n]).values for _ in range(B)])
    cap = 128
    dk, dv, dp = (torch.zeros((B, Hk, cap, D), dtype=dtype, device=DEV) for _ in range(3))
    dpos = torch.zeros((B, cap), dtype=torch.int64, device=DEV)
    ops.gather_rows(idx.to(DEV), [(k.to(DEV), dk), (v.to(DEV), dv), (kp.to(DEV), dp)], dst_row0=10,
                    pos_src=pos.contiguous().to(DEV), pos_dst=dpos)
    for src, dst in ((k, dk), (v, dv), (kp, dp)):
        assert torch.equal(dst[:, :, 10:10 + n].cpu(), ref.gather_kv(src, idx))
        assert torch.count_nonzero(dst[:, :, :10]) == 0 and torch.count_nonzero(dst[:, :, 10 + n:]) == 0
    assert torch.equal(dpos[:, 10:10 + n].cpu(), pos.gather(1, idx))


def test_append_rows():
    B, Hk, D, cap = 2, 8, 128, 40
    dtype = torch.bfloat16
    dk = torch.zeros((B, Hk, cap, D), dtype=dtype, device=DEV)
    dv = torch.zeros_like(dk)
    dpos = torch.zeros((B, cap), dtype=torch.int64, device=DEV)
    k1, v1 = _randn((B, Hk, 1, D), 51, dtype), _randn((B, Hk, 1, D), 52, dtype)
    ops.append_rows(17, k1.to(DEV), dk, v1.to(DEV), dv, pos_src=torch.full((B, 1), 999).to(DEV), pos_dst=dpos)
    assert torch.equal(dk[:, :, 17:18].cpu(), k1) and torch.equal(dv[:, :, 17:18].cpu(), v1)
    assert int(dpos[0, 17]) == 999 and torch.count_nonzero(dk[:, :, :17]) == 0


# ---------------------------------------------------------------------------
# Inject (re-RoPE into the held slot)
# ---------------------------------------------------------------------------
H2O_CASES = [
    # B, Hq, Hk, S, D, dtype
    (2, 8, 2, 200, 16, torch.float32),      # reference test geometry (test_baselines.py:46)
    (2, 8, 2, 200, 16, torch.float16),
    (1, 32, 8, 333, 64, torch.float16),
    (1, 8, 8, 97, 128, torch.bfloat16),
    # windows of 1024 rows or more: importance over mirrored key pairs
    (1, 4, 2, 1500, 64, torch.float16),
    (1, 2, 1, 2049, 32, torch.bfloat16),     # odd S: the middle key once
]


def test_h2o_prefill_scores_8k_properties():
    """The full 8k prompt (too long for the oracle): every causal row's
    probabilities sum to one, so each KV head's scores (group means) sum to
    S; key 0 is all of row 0's mass, so its score is at least 1; scores are
    non-negative; and equal keys give the harmonic tail sum_{i>=j} 1/(i+1)
    exactly up to fp32 rounding."""
    S, D = 8192, 128
    q, k = _randn((1, 8, S, D), 47, torch.float16), _randn((1, 2, S, D), 48, torch.float16)
    sc = ops.h2o_prefill_scores(q.to(DEV), k.to(DEV), D ** -0.5).double().cpu()
    assert sc.shape == (1, 2, S) and bool((sc >= 0).all())
    assert torch.allclose(sc.sum(-1), torch.full((1, 2), float(S), dtype=torch.float64), rtol=1e-5)
    assert bool((sc[..., 0] >= 1.0 - 1e-6).all())
    # equal keys: row i spreads 1/(i+1) over keys 0..i, so key j gets sum_{i>=j} 1/(i+1)
    keq = torch.ones((1, 1, S, D), dtype=torch.float16)
    sce = ops.h2o_prefill_scores(q[:, :4].to(DEV), keq.to(DEV), D ** -0.5).double().cpu()[0, 0]
    tail = torch.flip(torch.cumsum(torch.flip(1.0 / torch.arange(1, S + 1, dtype=torch.float64), [0]), 0), [0])
    assert torch.allclose(sce, tail, rtol=2e-5, atol=1e-6)


def test_h2o_prefill_scores_bit_exact_at_8k():
    """One KV group of the full 8k prompt (2 query heads, fp16): the H2O
    prefill scores equal the oracle's bit for bit.  The oracle's fp64
    contract takes about 20 s per query head on one core, so the two heads
    run on two threads (the oracle's C call releases the GIL)."""
    from concurrent.futures import ThreadPoolExecutor
    S, D, Hq = 8192, 128, 2
    q, k = _randn((1, Hq, S, D), 49, torch.float16), _randn((1, 1, S, D), 50, torch.float16)
    sc = D ** -0.5
    got = ops.h2o_prefill_scores(q.to(DEV), k.to(DEV), sc).cpu()
    with ThreadPoolExecutor(Hq) as pool:
        per_q = list(pool.map(lambda h: ref.window_scores(q[:, h:h + 1], k, S, sc, 1, "maxpool"), range(Hq)))
    want = ref.head_mean(torch.cat(per_q, 1)).reshape(1, 1, S)
    assert torch.equal(got, want)


@pytest.mark.parametrize("B,Hq,Hk,S,D,dtype", H2O_CASES)
def test_h2o_prefill_scores_bit_exact(B, Hq, Hk, S, D, dtype):
    q, k = _randn((B, Hq, S, D), 41, dtype), _randn((B, Hk, S, D), 42, dtype)
    want = ref.h2o_prefill_scores(q, k, 0.125)
    got = ops.h2o_prefill_scores(q.to(DEV), k.to(DEV), 0.125)
    assert torch.equal(got.cpu(), want)
    # query heads in chunks of one KV group: the same bits
    small = ops.h2o_prefill_scores(q.to(DEV), k.to(DEV), 0.125, max_workspace_bytes=1)
    assert torch.equal(small.cpu(), want)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("splits", [0, 1, 5])
def test_decode_attention_h2o_accumulates_group_mean_probs(dtype, splits):
    """out as decode attention; acc[:S-1] += mean-over-group probabilities,
    acc[S-1] = its probability (this step's token starts from zero)."""
    B, Hq, Hk, S, D, cap = 2, 32, 8, 430, 128, 500
    q, k, v = _randn((B, Hq, 1, D), 43, dtype), _randn((B, Hk, S, D), 44, dtype), _randn((B, Hk, S, D), 45, dtype)
    acc0 = torch.rand((B, Hk, cap), generator=torch.Generator().manual_seed(46)) * 10
    acc = acc0.to(DEV)
    out = ops.decode_attention_h2o(q.to(DEV), k.to(DEV), v.to(DEV), 0.088, acc[:, :, :S], num_splits=splits)
    want_out = ref.decode_attention(q, k, v, 0.088)
    assert np.abs(out.float().cpu().numpy() - want_out).max() <= TOL[dtype]
    probs = ref.h2o_decode_probs(q, k, 0.088)
    want = acc0.double().clone()
    want[:, :, S - 1] = 0
    want[:, :, :S] += probs
    got = acc.cpu().double()
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    assert torch.allclose(got[:, :, :S], want[:, :, :S], rtol=tol, atol=tol * 1e-2)
    assert torch.equal(got[:, :, S:], acc0[:, :, S:].double())   # rows past S untouched


H2O_EVICT_CASES = [
    # B, Hq, Hk, S, D, window, dtype, splits, tie
    (1, 32, 8, 513, 128, 32, torch.float16, 0, None),      # 8k/budget-512 layer, one step past the budget
    (2, 32, 8, 513, 128, 32, torch.bfloat16, 5, "low"),
    (2, 8, 2, 65, 16, 16, torch.float32, 1, "high"),       # reference test geometry (test_baselines.py:46)
    (1, 16, 4, 700, 64, 64, torch.float16, 0, "zero"),
    (3, 8, 8, 100, 256, 1, torch.bfloat16, 0, "nan"),
    (1, 32, 8, 4097, 128, 64, torch.float16, 0, "low"),    # budget 4096
    (1, 4, 1, 2, 32, 1, torch.float32, 0, None),           # one prefix key, one window key
    (1, 64, 8, 300, 128, 16, torch.float16, 0, "low"),     # group of 8: the batched score loads' widest group
    (1, 32, 2, 333, 128, 16, torch.bfloat16, 0, "high"),   # group of 16: scores loaded key by key
]


@pytest.mark.parametrize("B,Hq,Hk,S,D,window,dtype,splits,tie", H2O_EVICT_CASES)
def test_decode_attention_h2o_evict_equals_unfused(B, Hq, Hk, S, D, window, dtype, splits, tie):
    """The fused step (attend, update scores, drop one row) against
    decode_attention_h2o + keep_index + gather_rows: output, K, V and scores
    bit for bit into strided destination views, acc unchanged, rows past S-1
    untouched; the dropped row is the oracle's keep_index complement.  Tie
    cases plant equal keys with equal old scores so the updated scores tie
    exactly at the minimum (the highest index must go), at index 0 or the
    prefix end, or NaN scores (never dropped)."""
    budget = S - 1
    prefix = S - min(window, S)
    q, k, v = _randn((B, Hq, 1, D), 61, dtype), _randn((B, Hk, S, D), 62, dtype), _randn((B, Hk, S, D), 63, dtype)
    acc0 = torch.rand((B, Hk, S + 3), generator=torch.Generator().manual_seed(64)) * 10
    if tie is not None:
        rows = {"low": [2, 7, prefix // 2, prefix - 1], "high": [0, 3, 5], "zero": [0, prefix // 3],
                "nan": [1, 4]}[tie]
        rows = sorted(set(r for r in rows if r < prefix))
        k[:, :, rows] = k[:, :, rows[:1]]
        acc0[:, :, rows] = -5.0 if tie != "nan" else float("nan")
    kd, vd = (torch.full((B, Hk, S + 4, D + 8), 7.0, dtype=dtype, device=DEV) for _ in range(2))
    ad = torch.full((B, Hk, S + 5), 3.0, device=DEV)
    k_dst, v_dst, a_dst = kd[:, :, 1:S, :D], vd[:, :, 2:S + 1, 8:], ad[:, :, :S - 1]

    qd, kdv, vdv = q.to(DEV), k.to(DEV), v.to(DEV)
    acc_a = acc0.to(DEV)
    out_a = ops.decode_attention_h2o(qd, kdv, vdv, 0.09, acc_a[:, :, :S], num_splits=splits)
    keep = ops.keep_index(acc_a[:, :, :S], window, budget)
    assert torch.equal(keep.cpu(), ref.keep_index(acc_a[:, :, :S].cpu(), window, budget))
    acc_b = acc0.to(DEV)
    out_b = ops.decode_attention_h2o_evict(qd, kdv, vdv, 0.09, acc_b[:, :, :S], window, budget,
                                           k_dst, v_dst, a_dst, num_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(out_a.cpu(), out_b.cpu())
    assert torch.equal(acc_b.cpu().view(torch.int32), acc0.view(torch.int32))
    kc = keep.cpu()
    assert torch.equal(k_dst.cpu(), ref.gather_kv(k, kc))
    assert torch.equal(v_dst.cpu(), ref.gather_kv(v, kc))
    want_sc = acc_a[:, :, :S].cpu().gather(2, kc)
    assert torch.equal(a_dst.cpu().contiguous().view(torch.int32), want_sc.view(torch.int32))
    # nothing outside the S-1 destination rows is written
    assert bool((kd[:, :, 0] == 7).all() and (kd[:, :, S:] == 7).all() and (kd[..., D:] == 7).all())
    assert bool((vd[:, :, :2] == 7).all() and (vd[:, :, S + 1:] == 7).all() and (vd[..., :8] == 7).all())
    assert bool((ad[:, :, S - 1:] == 3).all())
    if tie in ("low", "high", "zero"):
        dropped = set(range(S)) - set(kc[0, 0].tolist())
        assert dropped == {rows[-1]}


@pytest.mark.parametrize("dtype,splits", [(torch.float16, 0), (torch.bfloat16, 3), (torch.float32, 1)])
def test_decode_attention_h2o_evict_with_fused_append(dtype, splits):
    """The token appended inside the fused step (attended from k_new / v_new,
    written into row S-1, its logit kept as key S-1's): the token row lands in
    place; the output and the kept rows' updated scores are within the
    tolerances of the fp64 oracle (acc + group-mean probabilities); the
    dropped row is a prefix minimiser of the oracle's updated scores up to
    that tolerance; and K, V are the bit-exact gather of every other row."""
    B, Hq, Hk, S, D, window = 2, 32, 8, 513, 128, 32
    budget, prefix = S - 1, S - window
    q = _randn((B, Hq, 1, D), 71, dtype)
    k, v = _randn((B, Hk, S, D), 72, dtype), _randn((B, Hk, S, D), 73, dtype)
    acc0 = torch.rand((B, Hk, S), generator=torch.Generator().manual_seed(76)) * 10
    acc0[:, :, S - 1] = 0
    kd, vd = k.to(DEV), v.to(DEV)
    kd[:, :, S - 1] = 0
    vd[:, :, S - 1] = 0
    k_dst, v_dst = torch.empty_like(kd), torch.empty_like(vd)
    a_dst = torch.empty((B, Hk, S), device=DEV)
    out = ops.decode_attention_h2o_evict(q.to(DEV), kd, vd, 0.09, acc0.to(DEV), window, budget, k_dst, v_dst, a_dst,
                                         num_splits=splits, k_new=k[:, :, S - 1:].to(DEV),
                                         v_new=v[:, :, S - 1:].to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu(), k) and torch.equal(vd.cpu(), v)          # the token row written in place
    assert np.abs(out.float().cpu().numpy() - ref.decode_attention(q, k, v, 0.09)).max() <= TOL[dtype]
    want = acc0.double() + ref.h2o_decode_probs(q, k, 0.09)
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    got_k = k_dst[:, :, :S - 1].cpu()
    for b in range(B):
        for h in range(Hk):
            kept = [i for i in range(S) if i != _dropped_row(got_k[b, h], k[b, h])]
            assert len(kept) == S - 1
            e = (set(range(S)) - set(kept)).pop()
            assert e < prefix
            assert float(want[b, h, e]) <= float(want[b, h, :prefix].min()) + tol * 10, (b, h, e)
            assert torch.equal(got_k[b, h], k[b, h, kept]) and torch.equal(v_dst[b, h, :S - 1].cpu(), v[b, h, kept])
            assert torch.allclose(a_dst[b, h, :S - 1].cpu().double(), want[b, h, kept], rtol=tol, atol=tol * 1e-2)


def _dropped_row(kept_rows, rows):
    """Index of the one row of rows (S,D) missing from kept_rows (S-1,D), kept in order."""
    n = kept_rows.shape[0]
    for i in range(n):
        if not torch.equal(kept_rows[i], rows[i]):
            return i
    return n


def test_decode_attention_h2o_evict_argument_errors():
    B, Hq, Hk, S, D = 1, 8, 2, 40, 64
    q, k, v = (torch.zeros(s, dtype=torch.float16, device=DEV) for s in ((B, Hq, D), (B, Hk, S, D), (B, Hk, S, D)))
    acc = torch.zeros(B, Hk, S, device=DEV)
    kd, vd, ad = torch.empty_like(k), torch.empty_like(v), torch.empty_like(acc)
    with pytest.raises(RuntimeError, match="exactly one row"):
        ops.decode_attention_h2o_evict(q, k, v, 0.1, acc, 8, S - 2, kd, vd, ad)   # two rows over budget
    with pytest.raises(RuntimeError, match="exactly one row"):
        ops.decode_attention_h2o_evict(q, k, v, 0.1, acc, 8, S, kd, vd, ad)       # within budget
    with pytest.raises(RuntimeError, match="exactly one row"):
        ops.decode_attention_h2o_evict(q, k, v, 0.1, acc, S, S - 1, kd, vd, ad)   # window covers the cache
    with pytest.raises(RuntimeError, match="acc_dst"):
        ops.decode_attention_h2o_evict(q, k, v, 0.1, acc, 8, S - 1, kd, vd, ad[:, :, :S - 2])
    lib = ops.N.lib()
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=DEV)
    ptr = ops._ptr
    rc = lib.hc_decode_attn_h2o_evict(
        ops.N.dtype_code(q.dtype), B, Hq, Hk, D, S, ptr(q), q.stride(0), q.stride(1),
        ptr(k), k.stride(0), k.stride(1), k.stride(2), ptr(v), v.stride(0), v.stride(1), v.stride(2),
        None, 0, 0, None, 0, 0, 0.1,
        ptr(q), q.stride(0), q.stride(1), ptr(acc), acc.stride(0), acc.stride(1), 8, S - 1,
        ptr(k), k.stride(0), k.stride(1), k.stride(2), ptr(vd), vd.stride(0), vd.stride(1), vd.stride(2),
        ptr(ad), ad.stride(0), ad.stride(1), ptr(ws), ws.numel(), 0, ops._stream_handle(q.device))
    assert rc != 0 and "alias" in lib.hc_last_error().decode()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_packed_h2o_evict_rows_equal_the_scalar_entry(dtype):
    """decode_h2o_evict_rows (hc_decode_attn_h2o_evict_packed over argument
    structs kept per storage pair) and decode_attention_h2o_evict
    (hc_decode_attn_h2o_evict) on twin buffers at budget: identical outputs,
    kept rows and scores step after step, while the two storages and score
    buffers swap every step and a few steps run on a side stream."""
    from hotcold_kv.hot_buffer import HotBuffer
    B, Hq, Hk, D, budget, W = 2, 32, 8, 128, 300, 32
    g = torch.Generator().manual_seed(11)
    cap = budget + 16
    bufs = [HotBuffer(B, Hk, D, dtype, DEV, cap) for _ in range(2)]
    k0, v0 = (torch.randn((B, Hk, budget, D), generator=g).to(dtype).to(DEV) for _ in range(2))
    acc0 = torch.rand((B, Hk, budget), generator=g).to(DEV)
    accs = []
    for b in bufs:
        b.append(k0, v0)
        a = torch.zeros((B, Hk, cap), device=DEV)
        a[:, :, :budget] = acc0
        accs.append([a, torch.empty_like(a)])
    side = torch.cuda.Stream(device=DEV)
    for step in range(40):
        q = torch.randn((B, Hq, 1, D), generator=g).to(dtype).to(DEV)
        kn, vn = (torch.randn((B, Hk, 1, D), generator=g).to(dtype).to(DEV) for _ in range(2))
        on_side = step in (7, 8, 21)
        if on_side:
            side.wait_stream(torch.cuda.current_stream(DEV))
        with torch.cuda.stream(side) if on_side else contextlib.nullcontext():
            outs = []
            for i, b in enumerate(bufs):
                n = b.n + 1
                b.ensure(n)
                acc, acc_sp = accs[i]
                if i == 0:
                    o = ops.decode_h2o_evict_rows(q, b.st, b.held, n, kn, vn, 0.088, acc, W, budget, b.spare(),
                                                  acc_sp, b.held)
                else:
                    o = ops.decode_attention_h2o_evict(q, b.st["k"][:, :, :n], b.st["v"][:, :, :n], 0.088,
                                                       acc[:, :, :n], W, budget, b.spare_rows("k"),
                                                       b.spare_rows("v"), acc_sp, k_new=kn, v_new=vn).unsqueeze(2)
                b.adopt_spare(n - 1)
                accs[i] = [acc_sp, acc]
                outs.append(o)
        torch.cuda.current_stream(DEV).wait_stream(side)
        assert torch.equal(outs[0], outs[1]), step
    torch.cuda.synchronize()
    for name in ("k", "v"):
        assert torch.equal(bufs[0].st[name][:, :, :budget], bufs[1].st[name][:, :, :budget]), name
    assert torch.equal(accs[0][0][:, :, :budget], accs[1][0][:, :, :budget])
    # argument errors, before any launch (rows, shapes) and from the library (not one row over budget)
    b, (acc, acc_sp) = bufs[0], accs[0]
    q = torch.zeros((B, Hq, 1, D), dtype=dtype, device=DEV)
    kn = torch.zeros((B, Hk, 1, D), dtype=dtype, device=DEV)
    with pytest.raises(RuntimeError, match="outside the buffers"):
        ops.decode_h2o_evict_rows(q, b.st, 0, cap + 1, kn, kn, 0.088, acc, W, budget, b.spare(), acc_sp)
    with pytest.raises(RuntimeError, match="q must be"):
        ops.decode_h2o_evict_rows(q[..., :64], b.st, 0, budget + 1, kn, kn, 0.088, acc, W, budget, b.spare(), acc_sp)
    with pytest.raises(RuntimeError, match="not one"):
        ops.decode_h2o_evict_rows(q, b.st, 0, budget, kn, kn, 0.088, acc, W, budget, b.spare(), acc_sp)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("to_host", [False, True])
def test_gather_evict_upcast_and_stage(dtype, to_host):
    """Evicted rows of strided hot-buffer views (held slot in front) upcast to
    fp32, with positions, in one packed block; out-of-range indices give zero
    rows and position -1; the pinned copy equals the device block."""
    B, H, held, cap, D = 2, 4, 8, 300, 128
    g = torch.Generator().manual_seed(21)
    kbuf = _randn((B, H, held + cap, D), 22, dtype).to(DEV)
    vbuf = _randn((B, H, held + cap, D), 23, dtype).to(DEV)
    posbuf = torch.randint(0, 10 ** 6, (B, held + cap), generator=g).to(DEV)
    S = 250
    k, v, pos = kbuf[:, :, held:held + S], vbuf[:, :, held:held + S], posbuf[:, held:held + S]
    te = 97
    idx = torch.stack([torch.randperm(S, generator=g)[:te] for _ in range(B)])
    idx[1, 5], idx[0, 9] = -1, S + 3
    dev_out = torch.empty((ops_bytes := 2 * B * H * te * D * 4 + B * te * 8,), dtype=torch.uint8, device=DEV)
    host_out = torch.empty((ops_bytes,), dtype=torch.uint8, pin_memory=True) if to_host else None
    kk, vv, pp = ops.gather_evict(idx.to(DEV), k, v, pos, dev_out=dev_out, host_out=host_out)
    torch.cuda.synchronize()
    kc, vc, pc = k.float().cpu(), v.float().cpu(), pos.cpu()
    for b in range(B):
        for j in range(te):
            i = int(idx[b, j])
            if 0 <= i < S:
                assert torch.equal(kk[b, :, j].cpu(), kc[b, :, i]) and torch.equal(vv[b, :, j].cpu(), vc[b, :, i])
                assert int(pp[b, j]) == int(pc[b, i])
            else:
                assert not kk[b, :, j].cpu().any() and not vv[b, :, j].cpu().any() and int(pp[b, j]) == -1
    if to_host:
        assert not kk.is_cuda and torch.equal(host_out, dev_out.cpu())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("per_head", [False, True])
def test_inject_rerope_tab_is_bit_exact(dtype, per_head):
    """With the rotary tables computed as the model's rotary module computes
    them (ops.rope_tables), the inject writes apply_rotary_pos_emb's bits."""
    B, Hk, R, D, cap = 2, 8, 64, 128, 100
    k_pre = _randn((B, Hk, R, D), 71, torch.float32, scale=3.0)
    v = _randn((B, Hk, R, D), 72, torch.float32)
    g = torch.Generator().manual_seed(73)
    pos = torch.randint(0, 1 << 17, (B, Hk, R) if per_head else (B, R), generator=g)
    inv = ref.default_inv_freq(D, 500000.0)
    cos, sin = ops.rope_tables(pos.reshape(-1, R), inv, 1.0, dtype)       # on the host, like the search thread
    shape = (B, Hk, R, D // 2) if per_head else (B, R, D // 2)
    kd = torch.zeros((B, Hk, cap, D), dtype=dtype, device=DEV)
    vd = torch.zeros_like(kd)
    ops.inject_rerope_tab(k_pre.to(DEV), v.to(DEV), cos.reshape(shape).to(DEV), sin.reshape(shape).to(DEV), kd, vd)
    assert torch.equal(kd[:, :, :R].cpu(), ref.rerope(k_pre, pos, inv, 1.0, dtype))
    assert torch.equal(vd[:, :, :R].cpu(), v.to(dtype))
    assert torch.count_nonzero(kd[:, :, R:]) == 0 and torch.count_nonzero(vd[:, :, R:]) == 0
    if dtype != torch.float32:
        # rows staged in the cache dtype (as the reference's copy converts them) give the same bits
        kd2, vd2 = torch.zeros_like(kd), torch.zeros_like(vd)
        ops.inject_rerope_tab(k_pre.to(dtype).to(DEV), v.to(dtype).to(DEV), cos.reshape(shape).to(DEV),
                              sin.reshape(shape).to(DEV), kd2, vd2)
        assert torch.equal(kd2, kd) and torch.equal(vd2, vd)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("per_head", [False, True])
def test_inject_rerope_matches_model_rotation(dtype, per_head):
    B, Hk, R, D, cap = 2, 8, 64, 128, 100
    k_pre = _randn((B, Hk, R, D), 61, torch.float32)
    v = _randn((B, Hk, R, D), 62, torch.float32)
    g = torch.Generator().manual_seed(63)
    pos = torch.randint(0, 65536, (B, Hk, R) if per_head else (B, R), generator=g)
    inv = ref.default_inv_freq(D, 500000.0)
    kd = torch.zeros((B, Hk, cap, D), dtype=dtype, device=DEV)
    vd = torch.zeros_like(kd)
    ops.inject_rerope(k_pre.to(DEV), v.to(DEV), pos.to(DEV), inv.to(DEV), 1.0, kd, vd)
    want = ref.rerope(k_pre, pos, inv, 1.0, dtype)
    got = kd[:, :, :R].cpu()
    assert torch.equal(vd[:, :, :R].cpu(), v.to(dtype))
    exact = (got == want).float().mean().item()
    # fp16/bf16 rounding absorbs the last-bit differences between the device's
    # cos/sin of the fp32 angle and torch's CPU cos/sin; fp32 output shows them.
    assert exact >= (0.999 if dtype != torch.float32 else 0.9), exact
    # any difference is a few rounding steps of the two rotated terms
    # |k_i cos| + |k_(i+-D/2) sin| (the result itself may cancel)
    k16 = k_pre.to(dtype).float()
    partner = torch.cat((k16[..., D // 2:], k16[..., : D // 2]), dim=-1)
    bound = 4 * torch.finfo(dtype).eps * (k16.abs() + partner.abs())
    diff = (got.float() - want.float()).abs()
    assert (diff <= bound).all(), (diff - bound).max()


# ---------------------------------------------------------------------------
# Several layers' compaction in one launch set (row tables)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,pooling", [(torch.float16, "maxpool"), (torch.bfloat16, "avgpool"),
                                           (torch.float32, "maxpool")])
def test_scores_and_gather_over_row_tables_equal_per_layer(dtype, pooling):
    """snapkv_scores_rows / gather_rows_tab over separately allocated layers
    give exactly the bits of one snapkv_scores / gather_rows call per layer;
    the keys use the model's (B,S,H,D)-transposed layout."""
    L, B, Hq, Hk, S, D, W, budget = 3, 2, 8, 2, 700, 64, 16, 96
    qs, ks, vs = [], [], []
    for l in range(L):
        qs.append(_randn((B, Hq, S, D), 100 + l, dtype).to(DEV))
        ks.append(_randn((B, S, Hk, D), 200 + l, dtype).to(DEV).transpose(1, 2))   # strided rows
        vs.append(_randn((B, S, Hk, D), 300 + l, dtype).to(DEV).transpose(1, 2))
    sc = 1.0 / math.sqrt(D)
    q_win = [q[:, :, S - W:].contiguous() for q in qs]
    rows = ops.snapkv_scores_rows(q_win, ks, W, sc, 7, pooling)
    keep_all = ops.keep_index(rows, W, budget)
    n = keep_all.shape[-1]
    kd = [torch.full((B, Hk, n + 5, D), float("nan"), dtype=dtype, device=DEV) for _ in range(L)]
    vd = [torch.full((B, Hk, n + 5, D), float("nan"), dtype=dtype, device=DEV) for _ in range(L)]
    ops.gather_rows_tab(keep_all, ks, vs, kd, vd, dst_row0=2)
    for l in range(L):
        one = ops.snapkv_scores(qs[l], ks[l], W, sc, 7, pooling)
        assert torch.equal(rows[l * B:(l + 1) * B], one), l
        keep = ops.keep_index(one, W, budget)
        assert torch.equal(keep_all[l * B:(l + 1) * B], keep), l
        assert torch.equal(keep.cpu(), ref.keep_index(ref.window_scores(qs[l].cpu(), ks[l].cpu(), W, sc, 7, pooling),
                                                      W, budget)), l
        assert torch.equal(kd[l][:, :, 2:2 + n], ops.gather_kv(ks[l], keep)), l
        assert torch.equal(vd[l][:, :, 2:2 + n], ops.gather_kv(vs[l], keep)), l


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("per_head", [False, True])
def test_retrieval_query_pooling(dtype, per_head):
    """hc_retrieval_query: the window's query rows (strided views, as the
    model's projections hand them over) summed in fp32 in window-then-head
    order and divided by the count -- equal to that sum computed on the
    CPU -- copied to pinned memory behind the event."""
    import ctypes

    from hotcold_kv import _native as N
    B, Hq, Hk, D, T = 2, 32, 8, 128, 4
    g = torch.Generator().manual_seed(3 + per_head)
    rows = [torch.randn((B, 1, Hq, D), generator=g).to(dtype) for _ in range(T)]
    qs = [r.to(DEV).transpose(1, 2) for r in rows]                 # (B,Hq,1,D) views, head stride D
    vh = Hk if per_head else 1
    nh = Hq // Hk if per_head else Hq
    dev = torch.empty((B, vh, D), dtype=torch.float32, device=DEV)
    host = torch.empty((B, vh, D), dtype=torch.float32, pin_memory=True)
    lib = N.lib()
    ev = ctypes.c_void_p()
    N.check(lib.hc_event_create(ctypes.byref(ev), 0), "hc_event_create")
    ptrs = (ctypes.c_void_p * T)(*[q.data_ptr() for q in qs])
    sb = (ctypes.c_int64 * T)(*[q.stride(0) for q in qs])
    sh = (ctypes.c_int64 * T)(*[q.stride(1) for q in qs])
    N.check(lib.hc_retrieval_query(N.dtype_code(dtype), B, Hq, Hk, D, T, ptrs, sb, sh, int(per_head),
                                   dev.data_ptr(), host.data_ptr(), ev.value,
                                   torch.cuda.current_stream().cuda_stream), "hc_retrieval_query")
    N.check(lib.hc_event_synchronize(ev.value), "hc_event_synchronize")
    lib.hc_event_destroy(ev.value)
    x = torch.stack([r[:, 0].float() for r in rows])               # (T,B,Hq,D)
    want = torch.empty((B, vh, D), dtype=torch.float32)
    inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(float(T * nh), dtype=torch.float32)
    for v in range(vh):
        acc = torch.zeros((B, D), dtype=torch.float32)
        for t in range(T):
            for h in range(v * nh, (v + 1) * nh):
                acc = acc + x[t, :, h]
        want[:, v] = acc * inv
    assert torch.equal(host, want)
    assert torch.equal(dev.cpu(), want)
    ref_mean = x.permute(1, 2, 0, 3).reshape(B, vh, nh * T, D).double().mean(dim=2)
    assert (host.double() - ref_mean).abs().max() < 1e-5


# ---------------------------------------------------------------------------
# Device search index of the cold stores
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("vec_heads,VD", [(1, 128), (4, 128), (4, 96), (1, 160)])
def test_device_index_equals_the_host_store(vec_heads, VD):
    """DeviceIndex (hc_index_add / hc_index_search) against the host stores
    filled with the same tokens: the same search vectors slot for slot, and the
    same top-R logical indices in the same order for random queries, planted
    exact ties (duplicate tokens) included, over rings that wrap and rows in
    different fill states."""
    from hotcold_kv.controller import _Ring
    from hotcold_kv.device_index import DeviceIndex
    B, H, D, cap = 3, 4, 128, 300
    rng = np.random.default_rng(12)
    rings = [_Ring(cap, H, D, VD, vec_heads) for _ in range(B)]
    dix = DeviceIndex(B, H, D, VD, vec_heads, cap, DEV)
    for i, te in enumerate((120, 250, 90, 400)):
        kpre = rng.standard_normal((B, H, te, D), dtype=np.float32)
        kpre[:, :, 5] = kpre[:, :, 7]                      # exact ties: a token repeated
        v = rng.standard_normal((B, H, te, D), dtype=np.float32)
        pos = np.arange(1000 * i, 1000 * i + te, dtype=np.int64)
        idx = np.tile(np.arange(te, dtype=np.int64), (B, 1))
        idx[0, ::3] = -1                                   # padding rows of row 0
        if i == 1:
            idx[2, :] = -1                                 # row 2 skips this eviction
        for b in range(B):
            rings[b].add(kpre[b], v[b], pos, idx[b])
        dix.add(torch.from_numpy(kpre).to(DEV), idx)
    torch.cuda.synchronize()
    for b in range(B):
        assert len(rings[b]) == int(dix.size[b])
        ex = rings[b].export()
        slots = [dix.physical(b, l) for l in range(len(rings[b]))]
        got = dix.vectors(b)[:, :, slots].permute(2, 0, 1).cpu().numpy()     # (n, VH, VD)
        assert np.array_equal(got, ex["vec"]), b
    R = 64
    hits = torch.empty((B, vec_heads, R), dtype=torch.int64, device=DEV)
    for trial in range(6):
        q = rng.standard_normal((B, vec_heads, D), dtype=np.float32)
        if trial == 0:
            q[:, :] = ex["kpre"][5, :vec_heads] if vec_heads > 1 else ex["kpre"][5].mean(0)  # hits a tie
        dix.search(torch.from_numpy(q).to(DEV), R, hits)
        h_dev = hits.cpu().numpy()
        for b in range(B):
            for h in range(vec_heads):
                qq = np.zeros(VD, np.float32)
                qq[:min(D, VD)] = q[b, h, :min(D, VD)]
                ss = 0.0
                for x in qq.astype(np.float64):                   # squares summed in dimension order
                    ss += x * x
                nrm = max(math.sqrt(ss), 1e-12)
                want = rings[b].search((qq.astype(np.float64) / nrm).astype(np.float32), R, head=h)
                got = h_dev[b, h]
                assert np.array_equal(got[:len(want)], want), (trial, b, h)
                assert (got[len(want):] == -1).all()



def _host_query(q, VD):
    """q cropped or padded to VD and normalised as the host store does it
    (squares summed in fp64 in dimension order)."""
    qq = np.zeros(VD, np.float32)
    n = min(len(q), VD)
    qq[:n] = q[:n]
    ss = 0.0
    for x in qq.astype(np.float64):
        ss += x * x
    return (qq.astype(np.float64) / max(math.sqrt(ss), 1e-12)).astype(np.float32)


@pytest.mark.parametrize("copies,R", [(0, 64), (500, 64), (500, 1024), (1200, 64), (1200, 1024), (5000, 256)])
def test_device_index_selection_with_many_ties(copies, R):
    """The selection's paths against the host store: candidate sets that fit
    in LDS or never do (every vector equal), ties at the R-th key fewer than
    its tie buffer or more (then taken oldest first by the ordered scan), R up
    to 1024; rings of 5000 slots after 6000 adds, so the oldest token is
    mid-ring.  The query is the repeated vector, so its copies are the top
    keys."""
    from hotcold_kv.controller import _Ring
    from hotcold_kv.device_index import DeviceIndex
    B, H, D, cap, te = 2, 2, 16, 5000, 6000
    rng = np.random.default_rng(copies + R)
    rings = [_Ring(cap, H, D, D, 1) for _ in range(B)]
    dix = DeviceIndex(B, H, D, D, 1, cap, DEV)
    kpre = rng.standard_normal((B, H, te, D), dtype=np.float32)
    u = rng.standard_normal((H, D), dtype=np.float32)
    for b in range(B):
        at = rng.choice(np.arange(1000, te), size=min(copies, te - 1000), replace=False)
        kpre[b][:, at] = u[:, None, :]
    v = rng.standard_normal((B, H, te, D), dtype=np.float32)
    pos = np.arange(te, dtype=np.int64)
    idx = np.tile(np.arange(te, dtype=np.int64), (B, 1))
    for half in (slice(0, 3500), slice(3500, te)):
        for b in range(B):
            rings[b].add(kpre[b][:, half], v[b][:, half], pos[half], idx[b, half] - half.start)
        dix.add(torch.from_numpy(np.ascontiguousarray(kpre[:, :, half])).to(DEV), idx[:, half] - half.start)
    torch.cuda.synchronize()
    hits = torch.empty((B, 1, R), dtype=torch.int64, device=DEV)
    for q in (u.mean(0), rng.standard_normal(D).astype(np.float32)):
        dix.search(torch.from_numpy(np.tile(q, (B, 1, 1))).to(DEV), R, hits)
        got = hits.cpu().numpy()
        for b in range(B):
            want = rings[b].search(_host_query(q, D), R)
            assert np.array_equal(got[b, 0, :len(want)], want), b
            assert (got[b, 0, len(want):] == -1).all()

@pytest.mark.parametrize("R", [16, 64, 512])
def test_device_index_fp16_pass_equals_the_exact_scan(R):
    """The fp16 pass (fp32 scores of the fp16 copy, then exact scores of the
    slots within twice the error bound of its R-th score) returns the exact
    scan's hits, also where the top of the ranking is crowded with
    near-duplicates closer than fp16 can tell apart (relative differences of
    1e-6), where ties are exact, and where more candidates than the pass
    re-scores survive (then the exact selection runs)."""
    from hotcold_kv.device_index import DeviceIndex
    B, H, D, cap, te = 2, 4, 128, 3000, 3500
    rng = np.random.default_rng(R)
    kpre = rng.standard_normal((B, H, te, D), dtype=np.float32)
    base = rng.standard_normal((B, H, D), dtype=np.float32)
    near = rng.choice(np.arange(600, te), size=300, replace=False)
    kpre[:, :, near] = base[:, :, None, :] * (1 + 1e-6 * rng.standard_normal((B, H, 300, D))).astype(np.float32)
    dup = rng.choice(np.setdiff1d(np.arange(600, te), near), size=2500 if R == 512 else 40, replace=False)
    kpre[1, :, dup] = kpre[1, :, dup[:1]]                     # exact duplicates in row 1
    dix = DeviceIndex(B, H, D, D, H, cap, DEV)
    assert dix.vec16 is not None
    dix.add(torch.from_numpy(kpre).to(DEV), np.tile(np.arange(te, dtype=np.int64), (B, 1)))
    h16 = torch.empty((B, H, R), dtype=torch.int64, device=DEV)
    h64 = torch.empty_like(h16)
    queries = [base, kpre[:, :, dup[0]], rng.standard_normal((B, H, D), dtype=np.float32)]
    for i, q in enumerate(queries):
        qd = torch.from_numpy(np.ascontiguousarray(q)).to(DEV)
        dix.search(qd, R, h16)
        dix.search(qd, R, h64, pass16=False)
        assert torch.equal(h16, h64), i

@pytest.mark.parametrize("per_head,faiss_dim,normalize", [(False, 32, True), (True, 64, True), (True, 96, True),
                                                         (True, 64, False)])
def test_scheduled_device_search_equals_the_host_search(per_head, faiss_dim, normalize):
    """Two controllers fed the same staged evictions (gather_evict into an
    eviction stage, as the cache evicts) and the same decode queries: one
    ranks on its device index and gathers the hits natively
    (hc_index_search + hc_cold_gather_async), the other searches the host
    stores (hc_cold_retrieve_async).  Every scheduled retrieval stages the
    same k_pre, v, positions, valid flags and rotary-table rows, over rings
    that wrap and planted exact ties; after an add the device index cannot
    follow (no stage) that layer goes back to the host search, still equal."""
    from hotcold_kv import KVController
    from hotcold_kv.datatypes import EvictedKV
    B, Hk, G, D, S, te, R = 2, 2, 2, 64, 400, 120, 16
    rng = torch.Generator().manual_seed(5)
    args = dict(max_capacity_prompt=128, cpu_buffer_size=300, faiss_dim=faiss_dim, window_size=1,
                query_pool_size=2, lookahead_k=R, hold_retrieved=True, per_head_retrieval=per_head,
                profile_overlap=False, normalize_for_ip=normalize)
    ctrls = [KVController(device_search=True, **args), KVController(device_search=False, **args)]
    inv = synthetic.inv_freq(D, 10000.0)
    for c in ctrls:
        c._lazy_init(torch.empty((B, Hk, 1, D), dtype=torch.bfloat16, device=DEV), n_layers=1)
        c.set_rope(inv, 1.0)
    assert ctrls[0]._dindex[0] is not None and ctrls[1]._dindex[0] is None
    print(f"[case] per_head {per_head} faiss_dim {faiss_dim} normalize {normalize}", flush=True)
    assert (ctrls[0]._dindex[0].vec16 is not None) == normalize       # the fp16 pass needs unit vectors
    n_dev = 0
    for rnd in range(6):
        k = torch.randn((B, Hk, S, D), generator=rng).to(torch.bfloat16)
        k[:, :, 1::2] = k[:, :, 0::2]                       # exact ties: every token twice
        v = torch.randn((B, Hk, S, D), generator=rng).to(torch.bfloat16)
        pos = (torch.arange(S, dtype=torch.int64) + 500 * rnd).repeat(B, 1)
        idx = torch.stack([torch.randperm(S, generator=rng)[:te].sort().values for _ in range(B)])
        staged = rnd != 3                                   # the fourth eviction: a synchronous add
        for c in ctrls:
            kd, vd, pd, id_ = k.to(DEV), v.to(DEV), pos.to(DEV), idx.to(DEV)
            if staged:
                st = c.evict_stage(kd.device, B, Hk, te, D)
                kp, vv, pp = ops.gather_evict(id_, kd, vd, pd, dev_out=st.dev, host_out=st.host)
                torch.cuda.synchronize()
                c.add_evicted_to_cold_store(0, EvictedKV(k_pre_cpu=kp, v_cpu=vv, pos_cpu=pp, evicted_idx=idx),
                                            stage=st)
            else:
                st = None
                kp = k.float().gather(2, idx.view(B, 1, te, 1).expand(B, Hk, te, D))
                vv = v.float().gather(2, idx.view(B, 1, te, 1).expand(B, Hk, te, D))
                c.add_evicted_to_cold_store(0, EvictedKV(k_pre_cpu=kp, v_cpu=vv, pos_cpu=pos.gather(1, idx),
                                                         evicted_idx=idx))
        for step in range(3):
            q = torch.randn((B, Hk * G, 1, D), generator=rng).to(torch.bfloat16)
            if step == 0:
                q[:, :] = k[:, :1, 2 * rnd:2 * rnd + 1].repeat_interleave(Hk * G, 1)   # aims at a tie
            slots = []
            for c in ctrls:
                c.update_query_window(0, q.to(DEV))
                c.maybe_launch_async_retrieval(0)
                c.wait_for_retrieval(0)
                slots.append(c._retrieval_ready_cpu[0])
            a, b = slots
            assert a is not None and b is not None and a is not b
            for x, y, what in zip(a.host, b.host, ("k_pre", "v", "pos", "valid")):
                assert torch.equal(x, y), (rnd, step, what)
            assert a.has_tab and b.has_tab and torch.equal(a.tab, b.tab), (rnd, step)
            assert bool(a.host[3].any())
        n_dev = ctrls[0].dbg["retrieval_device"]
        assert n_dev == (3 * (rnd + 1) if rnd < 3 else 9), rnd
        assert ctrls[1].dbg["retrieval_device"] == 0
    assert ctrls[0].dbg["device_index_dropped"] == 1 and ctrls[0]._dindex[0] is None
    for c in ctrls:
        c.wait_cold_adds()


def test_device_searches_of_a_step_launch_together_and_settle_before_adds():
    """Three layers: the device searches scheduled in a decode step wait
    until the last layer's call and are then launched together; an eviction
    into a layer whose search is still pending launches it first and waits for
    its gather, so the staged rows are those of the store the device ranked.
    Every layer's staged retrieval equals the host search's."""
    from hotcold_kv import KVController
    from hotcold_kv.datatypes import EvictedKV
    B, Hk, G, D, S, te, R, L = 2, 2, 2, 64, 300, 100, 8, 3
    rng = torch.Generator().manual_seed(9)
    args = dict(max_capacity_prompt=128, cpu_buffer_size=150, faiss_dim=D, window_size=1, query_pool_size=1,
                lookahead_k=R, hold_retrieved=True, per_head_retrieval=True, profile_overlap=False)
    ctrls = [KVController(device_search=True, **args), KVController(device_search=False, **args)]
    for c in ctrls:
        c._lazy_init(torch.empty((B, Hk, 1, D), dtype=torch.float16, device=DEV), n_layers=L)

    def evict(c, li, rnd):
        g = torch.Generator().manual_seed(100 * rnd + li)
        k = torch.randn((B, Hk, S, D), generator=g).to(torch.float16).to(DEV)
        v = torch.randn((B, Hk, S, D), generator=g).to(torch.float16).to(DEV)
        pos = (torch.arange(S, dtype=torch.int64) + 1000 * rnd).repeat(B, 1).to(DEV)
        idx = torch.stack([torch.randperm(S, generator=g)[:te].sort().values for _ in range(B)])
        st = c.evict_stage(k.device, B, Hk, te, D)
        kp, vv, pp = ops.gather_evict(idx.to(DEV), k, v, pos, dev_out=st.dev, host_out=st.host)
        torch.cuda.synchronize()
        c.add_evicted_to_cold_store(li, EvictedKV(k_pre_cpu=kp, v_cpu=vv, pos_cpu=pp, evicted_idx=idx), stage=st)

    for c in ctrls:
        for li in range(L):
            evict(c, li, 0)
    for step in range(4):
        qs = [torch.randn((B, Hk * G, 1, D), generator=rng).to(torch.float16).to(DEV) for _ in range(L)]
        for c in ctrls:
            dev = c.device_search
            for li in range(L):
                c.update_query_window(li, qs[li])
                c.maybe_launch_async_retrieval(li)
                if dev and li < L - 1 and not (step == 2 and li == 1):
                    assert [p[0] for p in c._pending_search] == list(range(li + 1))
                    assert c._retrieval_thread[li] is None
                if step == 2 and li == 1:
                    # layer 0's device search is still pending; the host search
                    # is joined first, so both rank the store before the add
                    if not dev:
                        c.wait_for_retrieval(0)
                    evict(c, 0, 1 + step)
                    if dev:                     # the pending searches were launched first
                        assert not c._pending_search and c._retrieval_thread[1] is not None
            if dev:
                assert not c._pending_search
            for li in range(L):
                c.wait_for_retrieval(li)
        for li in range(L):
            a, b = ctrls[0]._retrieval_ready_cpu[li], ctrls[1]._retrieval_ready_cpu[li]
            for x, y, what in zip(a.host, b.host, ("k_pre", "v", "pos", "valid")):
                assert torch.equal(x, y), (step, li, what)
    assert ctrls[0].dbg["retrieval_device"] == 4 * L and ctrls[1].dbg["retrieval_device"] == 0
    for c in ctrls:
        c.wait_cold_adds()


def test_device_index_is_not_made_past_its_memory_share():
    """With the device indexes' share of free memory set to zero the
    controller makes none, says so in dbg, and its searches run on the host
    stores."""
    from hotcold_kv import KVController
    c = KVController(cpu_buffer_size=64, faiss_dim=16, lookahead_k=4, window_size=1, per_head_retrieval=True)
    c.DEVICE_INDEX_MAX_FREE_FRACTION = 0.0
    c._lazy_init(torch.empty((1, 2, 1, 16), dtype=torch.float16, device=DEV), n_layers=2)
    assert c._dindex == [None, None] and c.dbg["device_index_too_large"] == 1
    d = KVController(cpu_buffer_size=64, faiss_dim=16, lookahead_k=4, window_size=1, per_head_retrieval=True)
    d._lazy_init(torch.empty((1, 2, 1, 16), dtype=torch.float16, device=DEV), n_layers=2)
    assert all(x is not None for x in d._dindex) and d._dindex[0].keys is d._dindex[1].keys
