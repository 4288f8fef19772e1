"""Pins of the CPU oracle (oracle/): each restated function is checked against
something that does not share its code -- closed forms, brute force on tiny
inputs, the literal fp32 torch restatement of the reference op sequence, the
invariants of the reference's own tests, and committed golden fixtures.
"""

import itertools
import math
import os

import numpy as np
import pytest
import torch

from oracle import reference as ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _randn(shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


# ---------------------------------------------------------------------------
# exp_det (Cody-Waite + Taylor-12) against libm
# ---------------------------------------------------------------------------
def test_exp_det_accuracy_and_range():
    rng = np.random.default_rng(0)
    xs = np.concatenate([-rng.random(20000) * 700.0, -rng.random(5000) * 1e-6, [0.0, -0.5, -1.0, -708.0]])
    worst = 0.0
    for x in xs:
        e = ref.exp_det(float(x))
        t = math.exp(float(x))
        worst = max(worst, abs(e - t) / t)
    assert worst < 4 * 2.0 ** -52, worst
    assert ref.exp_det(0.0) == 1.0
    assert ref.exp_det(-709.0) == 0.0 and ref.exp_det(float("-inf")) == 0.0


# ---------------------------------------------------------------------------
# Window scores: contract vs closed form / literal torch / brute force
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B,Hq,Hk,S,D,W,pool,pooling", [
    (2, 8, 2, 200, 16, 16, 7, "maxpool"),
    (2, 8, 2, 200, 16, 16, 7, "avgpool"),
    (1, 32, 8, 600, 128, 32, 7, "maxpool"),
    (1, 6, 4, 90, 32, 8, 5, "maxpool"),       # Hq % Hk != 0 -> mean over all heads
    (1, 4, 4, 20, 16, 32, 3, "maxpool"),      # window longer than the prompt
])
def test_window_scores_match_closed_form(B, Hq, Hk, S, D, W, pool, pooling):
    q = _randn((B, Hq, S, D), 1)
    k = _randn((B, Hk, S, D), 2)
    sc = 1.0 / math.sqrt(D)
    got = ref.window_scores(q, k, W, sc, pool, pooling).double().numpy()
    want = ref.snapkv_importance_f64(q, k, W, sc, pool, pooling)
    assert np.allclose(got, want, rtol=2e-7, atol=1e-9), np.abs(got - want).max()
    lit = ref.snapkv_importance_torch(q, k, W, sc, pool, pooling).double().numpy()
    assert np.allclose(lit, want, rtol=1e-5, atol=1e-7)


def test_window_scores_fp16_inputs_exact_upcast():
    # fp16 tensors are scored on their exact values (fp32 scores of the fp16 data)
    q = _randn((1, 8, 300, 64), 3, torch.float16)
    k = _randn((1, 2, 300, 64), 4, torch.float16)
    a = ref.window_scores(q, k, 16, 0.125, 7, "maxpool")
    b = ref.window_scores(q.float(), k.float(), 16, 0.125, 7, "maxpool")
    assert torch.equal(a, b)


def test_window_scores_brute_force_tiny():
    # pure-python fp64 loops of scoring.py:50-79 on a tiny case
    B, Hq, Hk, S, D, W = 1, 4, 2, 9, 4, 3
    q = _randn((B, Hq, S, D), 5)
    k = _randn((B, Hk, S, D), 6)
    sc = 0.5
    got = ref.window_scores(q, k, W, sc, 1, "maxpool")
    qq, kk = q.double().tolist(), k.double().tolist()
    for h in range(Hk):
        imp = [0.0] * S
        for w in range(W):
            qpos = S - W + w
            qf = [sum(qq[0][h * 2 + g][qpos][d] for g in range(2)) / 2 for d in range(D)]
            logits = [sum(qf[d] * kk[0][h][s][d] for d in range(D)) * sc if s <= qpos else -math.inf
                      for s in range(S)]
            m = max(logits)
            e = [math.exp(x - m) if x != -math.inf else 0.0 for x in logits]
            tot = sum(e)
            for s in range(S):
                imp[s] += e[s] / tot
        assert np.allclose(got[0, h].double().numpy(), imp, rtol=1e-6, atol=1e-9)


def test_window_scores_from_the_window_rows_only():
    """q_is_window: the last W query rows alone give the same scores."""
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 8, 300, 32, generator=g)
    k = torch.randn(2, 2, 300, 32, generator=g)
    full = ref.window_scores(q, k, 16, 0.2, 7, "maxpool")
    tail = ref.window_scores(q[:, :, -16:].contiguous(), k, 16, 0.2, 7, "maxpool", q_is_window=True)
    assert torch.equal(full, tail)
    with pytest.raises(ValueError):
        ref.window_scores(q[:, :, -8:].contiguous(), k, 16, 0.2, 7, "maxpool", q_is_window=True)


def test_torch_importance_from_the_window_rows_only():
    g = torch.Generator().manual_seed(6)
    q = torch.randn(1, 8, 200, 16, generator=g)
    k = torch.randn(1, 2, 200, 16, generator=g)
    full = ref.snapkv_importance_torch(q, k, 24, 0.25, 7, "maxpool")
    tail = ref.snapkv_importance_torch(q[:, :, -24:].contiguous(), k, 24, 0.25, 7, "maxpool", q_is_window=True)
    assert torch.equal(full, tail)


def test_window_scores_causal_mask():
    # a key after a window row's own position must get no weight from that row:
    # make the last key dominate; only the last window row may see it
    B, Hq, Hk, S, D, W = 1, 1, 1, 16, 8, 4
    q = torch.ones((B, Hq, S, D))
    k = torch.zeros((B, Hk, S, D))
    k[0, 0, S - 1] = 10.0
    imp = ref.window_scores(q, k, W, 1.0, 1, "maxpool")[0, 0]
    # rows S-4..S-2 never see key S-1; row S-1 puts ~all its mass there
    assert abs(float(imp[S - 1]) - 1.0) < 1e-6
    # each of the first three rows spreads one unit uniformly over its visible keys
    want = sum(1.0 / (S - W + w + 1) for w in range(W - 1))
    assert abs(float(imp[0]) - want) < 1e-6


def test_pool_definitions():
    # maxpool pads with -inf (edges see fewer values); avgpool divides by k
    x = torch.tensor([[[1.0, 5.0, 2.0, 0.0, 0.0, 3.0]]])
    mp = ref.pool1d(x, 3, "maxpool")
    assert mp.tolist() == [[[5.0, 5.0, 5.0, 2.0, 3.0, 3.0]]]
    ap = ref.pool1d(x, 3, "avgpool")
    assert torch.allclose(ap, torch.tensor([[[2.0, 8 / 3, 7 / 3, 2 / 3, 1.0, 1.0]]]))
    assert ref.pool1d(x, 1, "maxpool") is x


def test_rawsum_scores_closed_form():
    B, Hq, Hk, S, T, D = 2, 8, 2, 50, 6, 16
    q = _randn((B, Hq, T, D), 7)
    k = _randn((B, Hk, S, D), 8)
    got = ref.window_scores(q, k, 4, 0.0, mode="rawsum").double().numpy()
    qf = q.double().view(B, Hk, 4, T, D).mean(2)[:, :, -4:]
    want = (torch.matmul(qf, k.double().transpose(2, 3)) / math.sqrt(D)).sum(2).numpy()
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)
    hm = ref.head_mean(torch.from_numpy(got.astype(np.float32))).numpy()
    assert np.allclose(hm, got.mean(axis=1), rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------
# keep_index
# ---------------------------------------------------------------------------
def _rank(x):
    # torch.topk's order: NaN above every number; NaNs equal to each other
    return (1, 0.0) if math.isnan(x) else (0, x)


def _brute_keep(vals, window, budget):
    S = len(vals)
    win = min(window, S)
    prefix = S - win
    kp = max(0, min(budget - win, prefix))
    r = [_rank(x) for x in vals]
    best = None
    for comb in itertools.combinations(range(prefix), kp):
        chosen = set(comb)
        ok = all(r[i] > r[j] or (r[i] == r[j] and i < j)
                 for i in chosen for j in range(prefix) if j not in chosen)
        if ok:
            assert best is None, "selection must be unique"
            best = sorted(comb)
    return best + list(range(prefix, S))


@pytest.mark.parametrize("seed", range(6))
def test_keep_index_brute_force(seed):
    g = torch.Generator().manual_seed(seed)
    S, window, budget = 11, 3, 7
    vals = (torch.randint(0, 4, (1, 1, S), generator=g).float() / 2)  # many ties
    got = ref.keep_index(vals, window, budget)[0, 0].tolist()
    assert got == _brute_keep(vals[0, 0].tolist(), window, budget)


@pytest.mark.parametrize("seed", range(6))
def test_keep_index_brute_force_special_values(seed):
    # NaN, +-inf and +-0 among ties: NaN ranks above +inf, -0 ties with +0
    g = torch.Generator().manual_seed(100 + seed)
    S, window, budget = 11, 2, 6
    pool = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0, 1.0])
    vals = pool[torch.randint(0, len(pool), (1, 1, S), generator=g)]
    got = ref.keep_index(vals, window, budget)[0, 0].tolist()
    assert got == _brute_keep(vals[0, 0].tolist(), window, budget)
    # a keep boundary inside the NaN / +inf group
    row = [float("inf"), float("nan"), float("inf"), float("nan"), 0.0, -0.0, 1.0, 0.5]
    for budget in range(1, 7):
        got = ref.keep_index(torch.tensor([[row]]), 2, budget)[0, 0].tolist()
        assert got == _brute_keep(row, 2, budget), budget


def test_keep_index_nan_above_inf_like_torch_topk():
    # one NaN and one +inf among distinct values: a unique selection, which
    # torch.topk makes too (NaN first)
    s = _randn((1, 2, 300), 13)
    s[0, 0, 200], s[0, 0, 17] = float("inf"), float("nan")
    s[0, 1, 5], s[0, 1, 250] = float("inf"), float("nan")
    for budget in (1, 2, 3, 40):
        got = ref.keep_index(s, 8, budget + 8)
        assert torch.equal(got, ref.keep_index_torch(s, 8, budget + 8)), budget
    assert ref.keep_index(s, 8, 9)[0, 0].tolist()[0] == 17


def test_keep_index_reference_invariants():
    # tests/test_baselines.py:89-100
    B, Hk, S = 2, 3, 100
    budget, window = 30, 8
    scores = _randn((B, Hk, S), 9)
    keep = ref.keep_index(scores, window, budget)
    assert keep.shape == (B, Hk, budget)
    recent = set(range(S - window, S))
    for b in range(B):
        for h in range(Hk):
            row = keep[b, h].tolist()
            assert recent.issubset(row) and row == sorted(row) and len(set(row)) == budget


def test_keep_index_edge_budgets():
    s = _randn((1, 1, 10), 10)
    assert ref.keep_index(s, 32, 512)[0, 0].tolist() == list(range(10))      # window >= S
    assert ref.keep_index(s, 4, 2)[0, 0].tolist() == [6, 7, 8, 9]            # budget < window
    k, e = ref.keep_index(s, 4, 7, return_evicted=True)
    assert sorted(k[0, 0].tolist()[:3] + e[0, 0].tolist()) == list(range(6))


def test_keep_index_matches_torch_topk_without_ties():
    s = _randn((2, 4, 500), 11)   # continuous values: no ties, any top-k agrees
    got = ref.keep_index(s, 16, 100)
    want = ref.keep_index_torch(s, 16, 100)
    assert torch.equal(got, want)


def test_gather_kv_identity_and_permutation():
    t = _randn((2, 3, 20, 8), 12)
    idx = torch.arange(20).view(1, 1, 20).expand(2, 3, 20)
    assert torch.equal(ref.gather_kv(t, idx), t)
    perm = torch.stack([torch.randperm(20, generator=torch.Generator().manual_seed(i)) for i in range(6)]).view(2, 3, 20)
    out = ref.gather_kv(t, perm)
    for b in range(2):
        for h in range(3):
            assert torch.equal(out[b, h], t[b, h, perm[b, h]])


# ---------------------------------------------------------------------------
# Decode attention / eviction score
# ---------------------------------------------------------------------------
def test_decode_attention_closed_forms():
    B, Hq, Hk, S, D = 1, 4, 2, 7, 8
    q = _randn((B, Hq, 1, D), 13)
    v = _randn((B, Hk, S, D), 14)
    k_equal = torch.zeros((B, Hk, S, D))
    out = ref.decode_attention(q, k_equal, v, 0.3)
    for h in range(Hq):
        assert np.allclose(out[0, h], v[0, h // 2].double().mean(0).numpy())
    mask = torch.zeros((B, S), dtype=torch.bool)
    mask[0, 3] = True
    out = ref.decode_attention(q, _randn((B, Hk, S, D), 15), v, 0.3, mask)
    for h in range(Hq):
        assert np.allclose(out[0, h], v[0, h // 2, 3].double().numpy())
    assert np.isnan(ref.decode_attention(q, k_equal, v, 0.3, torch.zeros((B, S), dtype=torch.bool))).all()


def test_decode_attention_matches_sdpa():
    B, Hq, Hk, S, D = 2, 8, 2, 50, 16
    q, k, v = _randn((B, Hq, 1, D), 16), _randn((B, Hk, S, D), 17), _randn((B, Hk, S, D), 18)
    want = torch.nn.functional.scaled_dot_product_attention(
        q.double(), ref.repeat_kv(k.double(), 4), ref.repeat_kv(v.double(), 4), scale=0.25)[:, :, 0]
    assert np.allclose(ref.decode_attention(q, k, v, 0.25), want.numpy(), atol=1e-12)


def test_evict_scores_closed_form():
    # two keys, equal logits -> p = 1/2 each; loss = mean_d |v| / 2
    q = torch.zeros((1, 2, 1, 4))
    k = torch.zeros((1, 1, 2, 4))
    v = torch.tensor([[[[1.0, -1.0, 2.0, 0.0], [0.5, 0.5, 0.5, 0.5]]]])
    loss, idx = ref.evict_scores(q, k, v, 1.0)
    assert np.allclose(loss[0], [0.5 * 1.0, 0.5 * 0.5])
    assert idx[0] == 1


# ---------------------------------------------------------------------------
# Re-RoPE
# ---------------------------------------------------------------------------
def test_rerope_matches_transformers_rotation():
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding, apply_rotary_pos_emb
    from transformers import LlamaConfig

    cfg = LlamaConfig(hidden_size=512, num_attention_heads=4, num_key_value_heads=2, rope_theta=500000.0,
                      max_position_embeddings=131072)
    rot = LlamaRotaryEmbedding(cfg)
    D = 128
    pos = torch.tensor([[3, 1000, 65000, 7]])
    k = _randn((1, 2, 4, D), 19)
    for dtype in (torch.float16, torch.float32):
        cos, sin = rot(torch.empty(1, 1, dtype=dtype), pos)
        _, want = apply_rotary_pos_emb(torch.zeros_like(k.to(dtype)), k.to(dtype), cos, sin)
        got = ref.rerope(k, pos, rot.inv_freq, rot.attention_scaling, dtype)
        assert torch.equal(got, want)


def test_rerope_is_a_rotation():
    D = 64
    inv = ref.default_inv_freq(D, 10000.0)
    k = _randn((1, 1, 5, D), 20, torch.float64)
    pos = torch.tensor([[0, 1, 17, 300, 4000]])
    rk = ref.rerope(k, pos, inv, 1.0, torch.float64)
    assert torch.allclose(rk.norm(dim=-1), k.norm(dim=-1), rtol=1e-6)
    back = ref.rerope(rk, -pos, inv, 1.0, torch.float64)
    assert torch.allclose(back, k, atol=1e-5)
    assert torch.allclose(ref.rerope(k, torch.zeros_like(pos), inv, 1.0, torch.float64), k)


# ---------------------------------------------------------------------------
# Hot/cold compression and cold store
# ---------------------------------------------------------------------------
def test_hotcold_compress_invariants():
    B, Hq, Hk, S, D = 1, 8, 2, 300, 16
    keys, values, pre = _randn((B, Hk, S, D), 21), _randn((B, Hk, S, D), 22), _randn((B, Hk, S, D), 23)
    pos = torch.arange(S).view(1, S) + 100
    q = _randn((B, Hq, 5, D), 24)
    r = ref.hotcold_compress(keys, values, pre, pos, q, max_capacity=128, recent_size=32, topk_ratio=0.5)
    keep, ev = r["keep"][0].tolist(), r["evicted_idx"][0].tolist()
    assert len(keep) == 64 + 32 and keep[-32:] == list(range(S - 32, S))
    assert sorted(keep[:64] + ev) == list(range(S - 32))
    assert torch.equal(r["positions"][0], pos[0, keep])
    assert ref.hotcold_compress(keys[:, :, :100], values[:, :, :100], pre[:, :, :100], pos[:, :100], q,
                                128, 32, 0.5) is None


def test_cold_store_self_retrieval_and_wrap():
    # tests/test_cold_store.py:73-109: a token's own key retrieves it, also
    # after the ring wrapped; dropped tokens never come back
    g = torch.Generator().manual_seed(1)
    store = ref.ColdStore(capacity=8, dim=16)
    keys = torch.randn(15, 2, 16, generator=g)
    for lo in (0, 5, 10):
        store.add(keys[lo:lo + 5].numpy(), (-keys[lo:lo + 5]).numpy(), range(lo, lo + 5))
    assert len(store.pos) == 8
    for t in range(7, 15):
        hit = store.search(keys[t].mean(0).numpy(), 1)[0]
        assert store.pos[hit] == t and np.array_equal(store.kpre[hit], keys[t].numpy())


def test_cold_store_vectors_are_unit_head_means():
    # the search vector is the L2-normalised head mean (controller.py:190-194),
    # or each head's key per KV head; padded / cropped to the index width
    g = torch.Generator().manual_seed(3)
    k = torch.randn(8, 128, generator=g)
    for dim in (64, 128, 160):
        store = ref.ColdStore(capacity=4, dim=dim)
        vec = store.token_vecs(k.numpy())[0].astype(np.float64)
        m = k.double().mean(0)
        m = torch.nn.functional.pad(m, (0, max(0, dim - 128)))[:dim]
        assert abs(np.linalg.norm(vec) - 1.0) < 1e-6
        assert np.allclose(vec, (m / m.norm()).numpy(), atol=1e-7)
    per = ref.ColdStore(capacity=4, dim=64, per_head=True).token_vecs(k.numpy())
    for h in range(8):
        want = k[h, :64].double() / k[h, :64].double().norm()
        assert np.allclose(per[h], want.numpy(), atol=1e-7)


def test_cold_store_search_ranks_like_a_float64_matmul():
    # with clear gaps the order is the one of an ordinary fp64 inner product
    g = torch.Generator().manual_seed(4)
    store = ref.ColdStore(capacity=300, dim=32)
    keys = torch.randn(300, 2, 32, generator=g)
    store.add(keys.numpy(), keys.numpy(), range(300))
    q = store.token_vecs(torch.randn(2, 32, generator=g).numpy())[0]
    ip = np.stack([v[0] for v in store.vec]).astype(np.float64) @ q.astype(np.float64)
    want = np.argsort(-ip, kind="stable")[:20]
    gaps = np.diff(np.sort(ip)[::-1][:21])
    assert (np.abs(gaps) > 1e-9).all()
    assert store.search(q, 20) == [int(i) for i in want]


def test_cold_store_exact_ties_go_to_the_older_token():
    # power-of-two multiples normalise to the same bits: exact ties
    g = torch.Generator().manual_seed(5)
    k = torch.randn(2, 16, generator=g)
    store = ref.ColdStore(capacity=8, dim=16)
    store.add(torch.stack([4 * k, k, 2 * k, -k]).numpy(), np.zeros((4, 2, 16)), [40, 10, 20, 30])
    assert np.array_equal(store.vec[0], store.vec[1]) and np.array_equal(store.vec[1], store.vec[2])
    assert store.search(store.vec[1][0], 4) == [0, 1, 2, 3]


# ---------------------------------------------------------------------------
# Golden fixtures (tests/golden/make_golden.py)
# ---------------------------------------------------------------------------
def load_golden():
    """{case: (q (B,Hq,S,D), k, window, pool, budget, scaling, scores, keep)} with
    q's non-window rows zero-filled, in the case's dtype."""
    data = np.load(os.path.join(GOLDEN, "window_scores.npz"))
    cases = {}
    for case in sorted({k.split("__")[0] for k in data.files}):
        dtype = getattr(torch, str(data[f"{case}__dtype"]))
        qw = torch.from_numpy(data[f"{case}__q"]).to(dtype)
        k = torch.from_numpy(data[f"{case}__k"]).to(dtype)
        W, pool, budget = (int(x) for x in data[f"{case}__meta"])
        B, Hq, _, D = qw.shape
        S = k.shape[2]
        q = torch.zeros((B, Hq, S, D), dtype=dtype)
        q[:, :, S - W:] = qw
        cases[case] = (q, k, W, pool, budget, float(data[f"{case}__scaling"]),
                       torch.from_numpy(data[f"{case}__scores"]), torch.from_numpy(data[f"{case}__keep"]))
    return cases


@pytest.mark.parametrize("per_head,dim,normalize", [(False, 16, True), (True, 16, True), (False, 24, True),
                                                    (True, 8, True), (False, 16, False)])
def test_cold_topk_equals_cold_store_search(per_head, dim, normalize):
    """The array form ranks exactly like ColdStore.search, including exact
    ties (duplicated tokens), a wrapped ring, padding and cropping."""
    g = np.random.default_rng(dim + 3 * per_head + 7 * normalize)
    H, D = 3, 16
    store = ref.ColdStore(capacity=50, dim=dim, normalize=normalize, per_head=per_head)
    k = g.standard_normal((70, H, D)).astype(np.float32)
    k[40:45] = k[10:15]                        # duplicates: exact ties
    store.add(k, -k, np.arange(70))            # drops the 20 oldest
    kept = np.stack(store.kpre)
    for head in range(H if per_head else 1):
        for trial in range(3):
            q = g.standard_normal(dim).astype(np.float32)
            q /= np.linalg.norm(q)
            want = store.search(q, 17, head=head)
            got = ref.cold_topk(kept, q, 17, head=head, per_head=per_head, dim=dim, normalize=normalize)
            assert got.tolist() == want
    if normalize:
        # unit vectors: a stored vector used as the query ranks its own token
        # first (Cauchy-Schwarz; the kept store holds no duplicate of it)
        vec = store.vec[30][0]
        assert int(ref.cold_topk(kept, vec, 1, per_head=per_head, dim=dim)[0]) == 30


def test_golden_fixtures_reproduce():
    cases = load_golden()
    assert len(cases) >= 4
    for case, (q, k, W, pool, budget, sc, want_scores, want_keep) in cases.items():
        scores = ref.window_scores(q, k, W, sc, pool, "maxpool")
        assert torch.equal(scores, want_scores), case
        assert torch.equal(ref.keep_index(scores, W, budget), want_keep), case
        # the frozen vectors also satisfy the closed form they were pinned by
        f64 = ref.snapkv_importance_f64(q, k, W, sc, pool, "maxpool")
        assert np.allclose(want_scores.double().numpy(), f64, rtol=2e-7, atol=1e-9), case


# ---------------------------------------------------------------------------
# H2O scores (scoring.py:82-107)
# ---------------------------------------------------------------------------
def test_h2o_prefill_scores_against_fp64_closed_form():
    g = torch.Generator().manual_seed(31)
    q = torch.randn(2, 8, 40, 16, generator=g)
    k = torch.randn(2, 2, 40, 16, generator=g)
    got = ref.h2o_prefill_scores(q, k, 0.25)
    want = ref.h2o_prefill_scores_f64(q, k, 0.25)
    assert got.dtype == torch.float32 and got.shape == (2, 2, 40)
    assert torch.allclose(got.double(), want, rtol=1e-6, atol=1e-7)
    # every causal row's probabilities sum to one: the scores of a head sum to S
    assert torch.allclose(got.double().sum(-1), torch.full((2, 2), 40.0, dtype=torch.float64), rtol=1e-6)
    # key 0 is the only key row 0 sees
    assert (got[..., 0] >= 1.0 - 1e-6).all()


def test_h2o_prefill_scores_equal_keys_harmonic_tail():
    # equal keys: row i spreads 1/(i+1) over keys 0..i, so key j scores
    # sum_{i>=j} 1/(i+1) in every head
    S = 24
    q = torch.randn(1, 4, S, 8, generator=torch.Generator().manual_seed(32))
    k = torch.ones(1, 1, S, 8).mul(0.5)
    got = ref.h2o_prefill_scores(q, k, 0.3)[0, 0].double()
    want = torch.tensor([sum(1.0 / (i + 1) for i in range(j, S)) for j in range(S)], dtype=torch.float64)
    assert torch.allclose(got, want, rtol=1e-6)


def test_h2o_decode_probs_sum_to_one_and_match_attention():
    g = torch.Generator().manual_seed(33)
    q, k = torch.randn(2, 8, 1, 16, generator=g), torch.randn(2, 2, 30, 16, generator=g)
    p = ref.h2o_decode_probs(q, k, 0.25)
    assert torch.allclose(p.sum(-1), torch.ones(2, 2, dtype=torch.float64))
    v = torch.randn(2, 2, 30, 16, generator=g)
    out = ref.decode_attention(q, k, v, 0.25)                 # (B,Hq,D) fp64 numpy
    probs = torch.softmax(torch.matmul(q.double(), ref.repeat_kv(k, 4).double().transpose(2, 3)) * 0.25, -1)
    assert np.allclose(out, torch.matmul(probs, ref.repeat_kv(v, 4).double())[:, :, 0].numpy(), atol=1e-12)
