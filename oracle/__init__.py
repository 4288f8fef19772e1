"""CPU oracle of the hot-tier path -- TEST INFRASTRUCTURE, not product code.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or the timed CPU baseline).  The
product (hotcold_kv) never imports it and has no CPU fallback.

Contents:
  hc_oracle.c   plain-C restatement of the bit-defined window-scoring contract
  reference.py  numpy/torch restatements of the reference algorithms
                (scoring.py, layer_state.py, kernels.py, patch.py RoPE,
                cache.py compression, controller.py cold store), each citing
                the reference file:line it follows

Parity status of each function is listed in reference.py's module docstring.
"""
