"""Kept-set agreement between the bit-defined scoring contract and the
reference's literal path (scoring.py:67-79, 129: matmul in the input dtype,
softmax, window sum, pooling, then torch.topk), on layers of the 8k -> 512
workload (Llama-3.1-8B heads, 16 needles).

Informational, as the contract replaces the literal path's implementation-
defined last bits and tie order: the test prints, per literal variant, the
Jaccard index of the kept prefix sets and the largest gap between a
disagreeing token's score and the selection threshold (both in the fp64
closed form), and asserts only what the contract promises -- the fp32
literal path differs at near-ties only, and the fp16 path keeps nearly the
same set.
"""

import numpy as np
import pytest
import torch

from hotcold_kv import synthetic
from oracle import reference as ref


def _prefix_sets(keep, prefix):
    return [[set(int(i) for i in keep[b, h].tolist() if i < prefix) for h in range(keep.shape[1])]
            for b in range(keep.shape[0])]


@pytest.mark.parametrize("layer", [0, 7])
def test_contract_and_literal_reference_keep_nearly_the_same_tokens(layer):
    w = synthetic.WORKLOADS["llama8b_8k_b512"]
    p = synthetic.make_prompt(w, layer=layer, seed=0, device="cpu")
    q, k = p["q_post"], p["k_post"]                                    # fp16, as the model hands them
    S, W, budget = w.seq_len, w.window, w.budget
    prefix = S - W
    exact = ref.snapkv_importance_f64(q, k, W, w.scaling, w.pool, "maxpool")   # (B,Hk,S) fp64 closed form
    contract = ref.keep_index(ref.window_scores(q, k, W, w.scaling, w.pool, "maxpool"), W, budget)
    want = _prefix_sets(contract, prefix)
    lines = []
    for name, dtype in (("fp32 upcast", torch.float32), ("fp16 literal", torch.float16)):
        lit = ref.keep_index_torch(ref.snapkv_importance_torch(q, k, W, w.scaling, w.pool, "maxpool", dtype=dtype),
                                   W, budget)
        got = _prefix_sets(lit, prefix)
        jac, gaps = [], []
        for b in range(len(want)):
            for h in range(len(want[b])):
                a, c = want[b][h], got[b][h]
                jac.append(len(a & c) / len(a | c))
                if a != c:
                    sc = exact[b, h, :prefix]
                    thr = np.sort(sc)[::-1][budget - W - 1]               # the contract's k-th kept score
                    gaps.extend(abs(float(sc[i]) - float(thr)) / max(abs(float(thr)), 1e-30) for i in a ^ c)
        lines.append(f"layer {layer} {name}: Jaccard mean {np.mean(jac):.5f} min {np.min(jac):.5f}; "
                     f"{len(gaps)} disagreeing tokens, max relative score gap to the threshold "
                     f"{max(gaps) if gaps else 0.0:.3e}")
        if dtype == torch.float32:
            assert min(jac) >= 0.98, lines[-1]
            assert not gaps or max(gaps) <= 1e-4, lines[-1]              # near-ties only
        else:
            assert np.mean(jac) >= 0.9, lines[-1]
    print("\n" + "\n".join(lines))
