"""GPU test of the allocation-free fused append + decode entry point.

hc_decode_attn_append_noalloc keeps its split partials in a static device
array instead of a caller-owned workspace.  It must give exactly the bits of
hc_decode_attn_append (the same kernels, the same split choice) on the same
inputs: the output and the appended rows.  Two calls run back to back, the
second on a smaller input, so the second reads a scratch array that still
holds the first call's partials; a call whose partials would exceed the
array is refused.  Each stream of a device gets a region of its own, so a
call on a second stream gives the same bits; a fifth stream is refused.
"""

import pytest
import torch

from hotcold_kv import _native as N

pytestmark = pytest.mark.gpu

def _noalloc():
    return N.lib().hc_decode_attn_append_noalloc


def test_noalloc_signature_is_the_append_one_without_workspace():
    args = list(N.SIGNATURES["hc_decode_attn_append"][1])
    assert N.SIGNATURES["hc_decode_attn_append_noalloc"][1] == args[:-4] + args[-2:]


def _case(B, Hq, Hk, D, S, dtype, held, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    dev = "cuda"
    t = dict(
        q=torch.randn(B, Hq, D, generator=g).to(dtype).to(dev),
        k=torch.randn(B, Hk, S + 3, D, generator=g).to(dtype).to(dev),
        v=torch.randn(B, Hk, S + 3, D, generator=g).to(dtype).to(dev),
        kn=torch.randn(B, Hk, D, generator=g).to(dtype).to(dev),
        vn=torch.randn(B, Hk, D, generator=g).to(dtype).to(dev),
        pn=torch.randn(B, Hk, D, generator=g).to(dtype).to(dev),
        pd=torch.zeros(B, Hk, S + 3, D, dtype=dtype, device=dev),
        posn=torch.randint(0, 1 << 20, (B, 1), generator=g).to(dev),
        posd=torch.zeros(B, S + 3, dtype=torch.int64, device=dev),
        hpos=torch.randint(0, 4000, (B, Hk, max(held, 1)), generator=g).to(dev),
        hval=(torch.rand(B, Hk, max(held, 1), generator=g) < 0.8).to(torch.uint8).to(dev),
        cur=torch.tensor([3000], dtype=torch.int64, device=dev),
    )
    t["held"] = held
    t["S"] = S
    return t


def _args(t, out):
    q, k, v, kn, vn, pn, pd = t["q"], t["k"], t["v"], t["kn"], t["vn"], t["pn"], t["pd"]
    B, Hq, D = q.shape
    Hk = k.shape[1]
    S = t["S"]
    held = t["held"]
    return [N.dtype_code(q.dtype), B, Hq, Hk, D, S,
            q.data_ptr(), q.stride(0), q.stride(1),
            k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
            v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
            kn.data_ptr(), kn.stride(0), kn.stride(1),
            vn.data_ptr(), vn.stride(0), vn.stride(1),
            pn.data_ptr(), pn.stride(0), pn.stride(1),
            pd.data_ptr(), pd.stride(0), pd.stride(1), pd.stride(2),
            t["posn"].data_ptr(), t["posn"].stride(0), t["posd"].data_ptr(), t["posd"].stride(0),
            None, 0,
            held,
            t["hpos"].data_ptr() if held else None, t["hpos"].stride(0), t["hpos"].stride(1),
            t["hval"].data_ptr() if held else None, t["hval"].stride(0), t["hval"].stride(1),
            t["cur"].data_ptr(),
            1.0 / D ** 0.5,
            out.data_ptr(), out.stride(0), out.stride(1)]


def _run_pair(t, num_splits):
    """(out, k, v, pre, pos) of hc_decode_attn_append and of the no-alloc
    entry point, each on its own copy of the buffers it writes."""
    lib = N.lib()
    stream = torch.cuda.current_stream().cuda_stream
    B, Hq, D = t["q"].shape
    Hk = t["k"].shape[1]
    results = []
    for which in ("workspace", "noalloc"):
        c = dict(t)
        for name in ("k", "v", "pd", "posd"):
            c[name] = t[name].clone()
        out = torch.full((B, Hq, D), float("nan"), dtype=t["q"].dtype, device="cuda")
        a = _args(c, out)
        if which == "workspace":
            nbytes = lib.hc_decode_attn_workspace_size(B, Hq, Hk, D, t["S"], num_splits, 0)
            ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device="cuda")  # counter block zero
            rc = lib.hc_decode_attn_append(*a, ws.data_ptr(), ws.numel(), num_splits, stream)
            N.check(rc, "hc_decode_attn_append")
        else:
            rc = _noalloc()(*a, num_splits, stream)
            N.check(rc, "hc_decode_attn_append_noalloc")
        torch.cuda.synchronize()
        results.append((out, c["k"], c["v"], c["pd"], c["posd"]))
    return results


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_point(dtype):
    # first call: many units, forced splits (the scratch holds every partial);
    # second call: a smaller input that reads the array the first one left.
    for (B, S, held, splits) in ((4, 1500, 64, 6), (1, 300, 16, 3)):
        t = _case(B, 32, 8, 128, S, dtype, held, seed=B * 1000 + S)
        (o1, k1, v1, p1, s1), (o2, k2, v2, p2, s2) = _run_pair(t, splits)
        assert not torch.isnan(o1.float()).any()
        assert torch.equal(o1, o2), (B, S, dtype)
        assert torch.equal(k1, k2) and torch.equal(v1, v2) and torch.equal(p1, p2) and torch.equal(s1, s2)
        # the token went into row S-1
        assert torch.equal(k2[:, :, S - 1], t["kn"]) and torch.equal(s2[:, S - 1], t["posn"][:, 0])


def test_noalloc_auto_splits_and_group_8():
    # default split choice (num_splits = 0), a group of 8 query heads per KV head
    for (B, S) in ((16, 2431), (2, 700)):
        t = _case(B, 64, 8, 128, S, torch.float16, 0, seed=S)
        (o1, k1, v1, _, _), (o2, k2, v2, _, _) = _run_pair(t, 0)
        assert torch.equal(o1, o2) and torch.equal(k1, k2) and torch.equal(v1, v2)


def test_noalloc_refuses_oversized_partials():
    # 512 units x 64 splits of 128-dim partials are far above the array: the
    # call is refused before any launch (zero strides keep the tensors small)
    D, S = 128, 8192
    q = torch.zeros(1, 32, D, dtype=torch.float16, device="cuda")
    k = torch.zeros(1, 1, S, D, dtype=torch.float16, device="cuda")
    kn = torch.zeros(1, 1, D, dtype=torch.float16, device="cuda")
    out = torch.zeros(1, 32, D, dtype=torch.float16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = _noalloc()(N.HC_DTYPE_F16, 64, 32, 8, D, S,
                    q.data_ptr(), 0, D, k.data_ptr(), 0, 0, D, k.data_ptr(), 0, 0, D,
                    kn.data_ptr(), 0, 0, kn.data_ptr(), 0, 0, None, 0, 0, None, 0, 0, 0, None, 0, None, 0,
                    None, 0, 0, None, 0, 0, None, 0, 0, None, 0.088, out.data_ptr(), 0, D, 64, stream)
    assert rc == N.HC_ERR_WORKSPACE
    assert "static maximum" in N.lib().hc_last_error().decode()


def test_noalloc_streams_get_own_regions_and_a_fifth_is_refused():
    """Calls on other streams use regions of their own (the same bits as the
    workspace entry point); once four streams of the device are bound, a
    call from a fifth is refused.  torch's current stream, which the tests
    above bound, stays bound, so noalloc calls on it still work after this."""
    lib = N.lib()
    t = _case(2, 32, 8, 128, 700, torch.float16, 16, seed=77)
    (o_ws, k_ws, _, _, _), _ = _run_pair(t, 5)
    cur = torch.cuda.current_stream()
    others = [torch.cuda.Stream() for _ in range(4)]
    results = []
    refused = None
    for s in [cur] + others:
        c = dict(t)
        for name in ("k", "v", "pd", "posd"):
            c[name] = t[name].clone()
        out = torch.full_like(o_ws, float("nan"))
        torch.cuda.synchronize()
        rc = _noalloc()(*_args(c, out), 5, s.cuda_stream)
        torch.cuda.synchronize()
        if rc != N.HC_OK:
            refused = (s, rc, lib.hc_last_error().decode())
            break
        results.append((out, c["k"]))
    # the current stream plus three more fit; the fourth new stream does not
    assert len(results) == 4, refused
    assert refused is not None and refused[0] is others[-1] and refused[1] == N.HC_ERR_INVALID
    assert "streams" in refused[2]
    for out, kk in results:
        assert torch.equal(out, o_ws) and torch.equal(kk, k_ws)
    # the bound streams keep working
    c = dict(t)
    for name in ("k", "v", "pd", "posd"):
        c[name] = t[name].clone()
    out = torch.full_like(o_ws, float("nan"))
    N.check(_noalloc()(*_args(c, out), 5, others[0].cuda_stream), "hc_decode_attn_append_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(out, o_ws)
