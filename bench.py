#!/usr/bin/env python3
"""Hot-tier benchmark on one MI355X.

Workload (default): the 32-layer Llama-3.1-8B KV geometry (32 query / 8 KV
heads, head_dim 128), fp16, batch 1, 8192-token synthetic prompt with 16
needles; SnapKV compaction (window 32, max-pool 7, budget 512) of all 32
layers, then 63 decode steps, each appending one token per layer and running
GQA decode attention over the hot buffer.  Inputs are generated on the device
before the timed region.

One step = one such job.  The 32 layers are independent in this synthetic
workload, so each kernel covers all of them in one launch (layer l is batch
row l): compaction is one launch set (scores, kept indices, gather into the
hot buffer), recorded once as a HIP graph and replayed, and each decode step
is one fused launch over the 32 layers' hot buffers (72 MB) that writes the
new token's K/V row and attends over the buffer plus that token.

Before each decode launch a read sweep over 512 MiB evicts the 256 MB Infinity
Cache (in a model, the weights streamed between two visits of a layer do
that), so decode reads its K/V from HBM; the sweep's own time is measured
separately and subtracted.  It only reads, so no dirty lines are left for
decode to write back.

Reported:
  value              decode us per layer-step: median append+decode launch
                     time of the timed steps / 32, timed with HIP events on the
                     launch stream as [sweep; decode] minus [sweep] alone
                     (run_steps explains; the event-bracketed time is also
                     reported)
  compact_ms_32_layers  compaction of all 32 layers per step, ms (the 32
                     layers stacked along the batch axis, one launch set;
                     compact_ms_32_layers_per_layer_launches is the same work
                     as one launch set per layer, as a model's prefill runs it)
  roofline           decode launch: algorithmic bytes / mean launch time
  roofline_compaction (fp64 MFMA: the window logits' flop over the whole
  compaction time, with the HBM rate beside it), a per-layer-launch variant (one
  decode launch per layer, as a model's layer loop issues them), warm-cache
  figures, the reference's torch-CPU path on a bounded sample, and
  other_workloads: decode / compaction / inject figures of the 16k, 32k and
  64k workloads, and h2o: H2O prefill scores and decode steps on one layer
  (secondary; --no-other-configs skips them).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
                    [--no-cpu-baseline] [--no-other-configs] [--h2o-only]
"""

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "hotcold-kv-cache_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode µs/layer & SnapKV compact ms (8k→512); % of HBM peak GB/s on 1 MI355X"
HBM_PEAK_GBS = 8000.0
FP64_MFMA_PEAK_TFLOPS = 78.6
FLUSH_BYTES = 512 << 20
# Layers of the hot/cold loop at the larger held-slot shapes: the host cold
# store holds fp32 pre-RoPE keys and values for every prompt position (1 KB
# per token and KV head), 4.3 GB per layer at 32k x 16 and 2.1 GB at 64k x 4,
# and half as much again once a host search computes its vectors; these
# counts keep each run near 70 GB of host memory (105 GB with the vectors).
PIPELINE_LAYERS = {"b16_32k_b2048_held128": 16, "bf16_b4_64k_b4096_held256": 32}


class CacheSweep:
    """Evicts the Infinity Cache by reading FLUSH_BYTES (a max reduction)."""

    def __init__(self, dev):
        import torch
        self.buf = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)

    def __call__(self):
        import torch
        torch.amax(self.buf)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def elem_size(dtype):
    import torch
    return torch.tensor([], dtype=dtype).element_size()


def decode_bytes(w, rows, n_keys):
    """Algorithmic HBM bytes of one append+decode launch over `rows` (layer,
    batch) rows attending n_keys keys: the n_keys - 1 cached K and V rows
    read once, the new token's K and V read and written into the hot
    buffer, q read, output written."""
    es = elem_size(w.dtype)
    return rows * (2 * w.hk * (n_keys + 1) * w.head_dim + 2 * w.hq * w.head_dim) * es


def compaction_bytes(w, rows):
    """Algorithmic HBM bytes of one compaction over `rows` layer rows: the
    window queries and every key read once, fp32 scores written and read,
    kept K and V rows read and written."""
    es = elem_size(w.dtype)
    S, D, W = w.seq_len, w.head_dim, min(w.window, w.seq_len)
    q = w.hq * W * D * es
    k = w.hk * S * D * es
    scores = 2 * w.hk * S * 4
    gather = 2 * 2 * w.hk * w.budget * D * es
    return rows * (q + k + scores + gather)


class Setup:
    """Device-resident inputs, hot buffers and captured graphs of one
    workload (all layers stacked along the batch axis)."""

    def __init__(self, w, dev):
        import torch
        from hotcold_kv import synthetic
        from hotcold_kv.hot_buffer import kv_rows

        self.w = w
        L, B, S, D = w.layers, w.batch, w.seq_len, w.head_dim
        self.LB = LB = L * B
        dt = w.dtype
        self.q_post = torch.empty((LB, w.hq, S, D), dtype=dt, device=dev)
        self.k_post = torch.empty((LB, w.hk, S, D), dtype=dt, device=dev)
        self.v = torch.empty((LB, w.hk, S, D), dtype=dt, device=dev)
        for l in range(L):
            p = synthetic.make_prompt(w, layer=l, seed=0, device=dev)
            sl = slice(l * B, (l + 1) * B)
            self.q_post[sl] = p["q_post"]
            self.k_post[sl] = p["k_post"]
            self.v[sl] = p["v"]
            del p
        self.cap = w.budget + w.decode_steps
        # the hot tier's own layout (hot_buffer.kv_rows): each row's key and
        # value adjacent, K and V as (LB,Hk,cap,D) views of row stride 2*D
        self.k_hot, self.v_hot = kv_rows((LB, w.hk), self.cap, D, dt, dev)
        self.k_hot.zero_()
        self.v_hot.zero_()
        self.q_new, self.k_new, self.v_new = [], [], []
        for t in range(w.decode_steps):
            qs, ks, vs = [], [], []
            for l in range(L):
                tok = synthetic.make_decode_token(w, l, t, seed=0, device=dev)
                qs.append(tok["q_post"]), ks.append(tok["k_post"]), vs.append(tok["v"])
            self.q_new.append(torch.cat(qs, 0))
            self.k_new.append(torch.cat(ks, 0))
            self.v_new.append(torch.cat(vs, 0))
        self.out = torch.empty((LB, w.hq, D), dtype=dt, device=dev)
        self.stream = torch.cuda.Stream(dev)
        self.g_comp = None
        self.g_pl = None

    # -- eager launch sets -----------------------------------------------------------
    def compaction(self):
        from hotcold_kv import ops
        w = self.w
        scores = ops.snapkv_scores(self.q_post, self.k_post, w.window, w.scaling, w.pool, "maxpool")
        keep = ops.keep_index(scores, w.window, w.budget)
        ops.gather_rows(keep, [(self.k_post, self.k_hot), (self.v, self.v_hot)])
        return keep

    def compaction_per_layer(self):
        """The same compaction as one launch set per layer, as a model's
        prefill issues it (each layer compacts after its attention)."""
        from hotcold_kv import ops
        w, B = self.w, self.w.batch
        for l in range(w.layers):
            sl = slice(l * B, (l + 1) * B)
            scores = ops.snapkv_scores(self.q_post[sl], self.k_post[sl], w.window, w.scaling, w.pool, "maxpool")
            keep = ops.keep_index(scores, w.window, w.budget)
            ops.gather_rows(keep, [(self.k_post[sl], self.k_hot[sl]), (self.v[sl], self.v_hot[sl])])

    def decode(self, t, num_splits=0):
        """Decode step t: append token t into row budget+t of every layer's
        hot buffer and attend over rows 0..budget+t, one fused launch."""
        from hotcold_kv import ops
        n = self.w.budget + t + 1
        ops.decode_attention_append(self.q_new[t], self.k_hot[:, :, :n], self.v_hot[:, :, :n], self.k_new[t],
                                    self.v_new[t], self.w.scaling, out=self.out, num_splits=num_splits)

    def decode_per_layer(self, t):
        """One append+decode launch per layer, as a model's layer loop issues them."""
        from hotcold_kv import ops
        B, n = self.w.batch, self.w.budget + t + 1
        for l in range(self.w.layers):
            sl = slice(l * B, (l + 1) * B)
            ops.decode_attention_append(self.q_new[t][sl], self.k_hot[sl, :, :n], self.v_hot[sl, :, :n],
                                        self.k_new[t][sl], self.v_new[t][sl], self.w.scaling, out=self.out[sl])

    # -- graphs --------------------------------------------------------------------------
    def capture(self):
        """Record compaction and the per-layer decode loop as HIP graphs on a
        side stream (warmed up eagerly on that stream first)."""
        import torch
        w = self.w
        s = self.stream
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.compaction()
            self.compaction_per_layer()
            for t in range(w.decode_steps):
                self.decode(t)
            self.decode_per_layer(w.decode_steps - 1)
        s.synchronize()

        def cap(fn):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                fn()
            return g

        self.g_comp = cap(self.compaction)
        self.g_cpl = cap(self.compaction_per_layer)
        self.g_pl = cap(lambda: self.decode_per_layer(w.decode_steps - 1))
        # 20 back-to-back launches of the last step's decode (warm-cache rate)
        self.g_dec20 = cap(lambda: [self.decode(w.decode_steps - 1) for _ in range(20)])
        torch.cuda.synchronize()


def dropin_compaction(s, flush, reps=5):
    """The 32-layer compaction through the drop-in's PressLayerState objects
    (compact_prompt, the compression half of prefill), on the workload's
    per-layer prompt tensors:
      deferred   every layer joins one DeferredCompaction, which runs them
                 together after the last layer (PressCache's default): one
                 scoring launch set over per-layer row tables, one top-k, one
                 gather into every layer's hot buffer;
      per_layer  each layer compacted as its prefill returns.
    Two figures per path, medians over reps:
      gpu   events around the sequence on the launch stream, with the host
            enqueueing it while the GPU is still busy with cache sweeps (as
            the last layer's own work keeps it busy in a model's prefill):
            the GPU time of the compaction alone;
      wall  host time from an idle GPU until the stream is done (Python,
            launches and buffer allocation included)."""
    import torch
    from hotcold_kv.baselines.layer_state import DeferredCompaction, PressLayerState

    w, B = s.w, s.w.batch
    layers = [(s.q_post[l * B:(l + 1) * B], s.k_post[l * B:(l + 1) * B], s.v[l * B:(l + 1) * B])
              for l in range(w.layers)]

    states = [PressLayerState("snapkv", w.budget, w.window, w.pool, "maxpool") for _ in layers]

    def run(deferred):
        dc = DeferredCompaction() if deferred else None
        for st, (q, k, v) in zip(states, layers):
            st.compact_prompt(q, k, v, w.scaling, dc)
        if dc is not None:
            dc.flush()
        return states

    out = {}
    with torch.cuda.stream(s.stream):
        for name, deferred in (("deferred", True), ("per_layer", False)):
            run(deferred)
            gpu, wall = [], []
            for _ in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.stream.synchronize()
                for _ in range(40):     # ~6 ms of GPU work queued ahead of the timed sequence
                    flush()
                e0.record(s.stream)
                states = run(deferred)
                e1.record(s.stream)
                s.stream.synchronize()
                gpu.append(e0.elapsed_time(e1))
                flush()
                s.stream.synchronize()
                t0 = time.perf_counter()
                states = run(deferred)
                s.stream.synchronize()
                wall.append((time.perf_counter() - t0) * 1e3)
            out[name] = (statistics.median(gpu), statistics.median(wall))
            out[name + "_rows"] = states[0].get_seq_length()
    out["states"] = states
    return out


def dropin_decode(s, states, reps=3):
    """The decode steps through the drop-in's PressLayerState.decode, one
    call per layer per step, issued eagerly from Python as a model's layer
    loop issues them (no graph): the workload's decode tokens over the
    compacted caches `states` leaves behind.  Host time from an idle GPU
    until the stream is done, per layer-step (median over reps of the whole
    job; each rep restarts from the compacted caches)."""
    import torch

    w, B, G = s.w, s.w.batch, s.w.group
    toks = [[(s.q_new[t][l * B:(l + 1) * B], s.k_new[t][l * B:(l + 1) * B], s.v_new[t][l * B:(l + 1) * B])
             for l in range(w.layers)] for t in range(w.decode_steps)]
    n0 = [st.get_seq_length() for st in states]
    walls = []
    with torch.cuda.stream(s.stream):
        for _ in range(reps + 1):
            for st, n in zip(states, n0):
                st.buf.n = n                      # back to the compacted prompt
            s.stream.synchronize()
            t0 = time.perf_counter()
            for t in range(w.decode_steps):
                for st, (q, k, v) in zip(states, toks[t]):
                    st.decode(q, k, v, G, w.scaling)
            s.stream.synchronize()
            walls.append((time.perf_counter() - t0) * 1e6 / (w.decode_steps * w.layers))
    return statistics.median(walls[1:])


def run_steps(s, steps, flush):
    """Run `steps` whole jobs; return (wall ms/step, compaction ms list,
    decode ms (differential), decode ms (event-bracketed)).

    Compaction replays its graph between two events.  Each decode step t is
    timed two ways, both after a cache sweep (medians over the timed steps):
      differential  events around [sweep; decode] minus events around
                    [sweep] alone: the decode kernel plus the ordinary gap
                    between two dependent kernels, as in a model's stream;
      bracketed     events directly around the decode launch: this adds the
                    3-4 us an event marker between two kernels costs here.
    The fused launch is idempotent (it rewrites row budget+t with the same
    token), so running step t twice leaves the same buffer."""
    import torch
    w = s.w
    st = s.stream

    def ev():
        return torch.cuda.Event(enable_timing=True)

    comp_ev, sweep_ev, pair_ev, br_ev = [], [], [], []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(st):
        for _ in range(steps):
            c0, c1 = ev(), ev()
            c0.record(st)
            s.g_comp.replay()
            c1.record(st)
            comp_ev.append((c0, c1))
            for t in range(w.decode_steps):
                a0, a1, b0, b1, e0, e1 = ev(), ev(), ev(), ev(), ev(), ev()
                a0.record(st)
                flush()
                a1.record(st)
                b0.record(st)
                flush()
                s.decode(t)
                b1.record(st)
                flush()
                e0.record(st)
                s.decode(t)
                e1.record(st)
                sweep_ev.append((a0, a1))
                pair_ev.append((b0, b1))
                br_ev.append((e0, e1))
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / max(1, steps)

    def ms(evs):
        return [a.elapsed_time(b) for a, b in evs]

    if not steps:  # warm-up with --warmup 0: nothing timed
        return 0.0, [], float("nan"), float("nan")
    comp = ms(comp_ev)
    dec_diff = statistics.median(ms(pair_ev)) - statistics.median(ms(sweep_ev))
    dec_br = statistics.median(ms(br_ev))
    return wall_ms, comp, dec_diff, dec_br


def time_graph(g, st, iters, flush=None):
    """Mean ms of replays of g on st, events around each replay; the optional
    flush runs before each start event."""
    import torch
    evs = []
    with torch.cuda.stream(st):
        for i in range(iters):
            if flush is not None:
                flush()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(st)
            g.replay()
            e1.record(st)
            evs.append((e0, e1))
    torch.cuda.synchronize()
    return statistics.mean(a.elapsed_time(b) for a, b in evs)


def stream_rates(dev, nbytes=1 << 30, iters=10):
    """Measured device bandwidth for context: a read sweep (max reduction)
    over nbytes and a device copy of nbytes/2 -> nbytes/2.  The copy is also
    the known-size kernel the FETCH_SIZE / WRITE_SIZE counters are scaled by."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    half = src.numel() // 2
    dst = torch.empty(half, dtype=torch.float32, device=dev)
    torch.amax(src)
    dst.copy_(src[:half])
    torch.cuda.synchronize()
    e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    e[0].record()
    for _ in range(iters):
        torch.amax(src)
    e[1].record()
    for _ in range(iters):
        dst.copy_(src[:half])
    e[2].record()
    torch.cuda.synchronize()
    read = nbytes * iters / (e[0].elapsed_time(e[1]) * 1e-3) / 1e9
    copy = 2 * half * 4 * iters / (e[1].elapsed_time(e[2]) * 1e-3) / 1e9
    del src, dst
    return {"read_GBps": round(read, 1), "copy_GBps": round(copy, 1), "copy_bytes_each_way": half * 4}


def profiled_launch_us(workload):
    """The decode launch's average kernel duration (us) over the launches
    right after the cache sweep, from the committed rocprofv3 kernel-trace
    summary of this workload, or None if there is none."""
    import re
    path = os.path.join(ROOT, "profiles", f"decode_attn_compaction_{workload}_kernel_trace.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"^decode_launch_avg_us_after_sweep:\s*([0-9.]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


def profiled_traffic(workload):
    """HBM bytes per decode launch from the committed FETCH_SIZE / WRITE_SIZE
    summary of this workload (rocprofv3 --pmc runs, scaled by a known-size
    copy), or None if there is none."""
    import re
    path = os.path.join(ROOT, "profiles", f"decode_attn_compaction_{workload}_pmc_traffic.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", open(path).read(), re.M)
    return int(m.group(1)) if m else None


def read_floor_ms(dev, nbytes, st, flush, reps=24):
    """ms of a plain streaming read of nbytes (hc_read_bytes: 16-byte loads
    over 1024 workgroups) after the same cache sweep, differential timing:
    what a kernel that only reads the decode's bytes takes here."""
    import torch
    from hotcold_kv import _native as N
    nbytes = (int(nbytes) + 15) // 16 * 16
    buf = torch.ones(nbytes // 2, dtype=torch.float16, device=dev)
    lib = N.lib()

    def read(i):
        N.check(lib.hc_read_bytes(buf.data_ptr(), nbytes, None, torch.cuda.current_stream(dev).cuda_stream),
                "hc_read_bytes")

    with torch.cuda.stream(st):
        read(0)
    ms = differential_ms(st, flush, read, reps)
    del buf
    return ms


def differential_ms(st, flush, fn, reps, warmup=3):
    """ms of fn() measured as events around [sweep; fn] minus events around
    [sweep] alone (see run_steps), as the difference of the two medians
    after `warmup` discarded rounds."""
    import torch

    def ev():
        return torch.cuda.Event(enable_timing=True)

    sw, pr = [], []
    with torch.cuda.stream(st):
        for i in range(warmup + reps):
            a0, a1, b0, b1 = ev(), ev(), ev(), ev()
            a0.record(st)
            flush()
            a1.record(st)
            b0.record(st)
            flush()
            fn(i)
            b1.record(st)
            if i >= warmup:
                sw.append((a0, a1))
                pr.append((b0, b1))
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in pr) - statistics.median(a.elapsed_time(b) for a, b in sw)


def measure_config(w, dev, flush, reps=24, cpu=False):
    """Secondary figures of a larger workload (not the headline): the fused
    append+decode over all layers' hot buffers with the held slot active, one
    layer's compaction at the full batch, and the inject path (re-RoPE of a
    full held slot, its pinned H2D copy, and decode with that copy running
    concurrently on a side stream).  Inputs are N(0,1) of the workload's
    shapes, generated on the device.  cpu: also time the reference's
    torch-CPU path on one layer of the same inputs (cpu_baseline_config)."""
    import torch
    from hotcold_kv import ops, synthetic
    from hotcold_kv.hot_buffer import kv_rows

    g = torch.Generator(device=dev).manual_seed(5)
    dt, D, Hk, Hq = w.dtype, w.head_dim, w.hk, w.hq
    es = elem_size(dt)
    LB = w.layers * w.batch
    R = w.held
    cap = w.hot_capacity
    st = torch.cuda.Stream(dev)
    out = {"workload": w.name, "layers": w.layers, "batch": w.batch, "seq_len": w.seq_len, "budget": w.budget,
           "held": R, "dtype": {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}[dt]}

    # -- decode: hot buffers of every layer, held slot in rows 0..R-1 ------------------------
    k_hot, v_hot = kv_rows((LB, Hk), cap, D, dt, dev)
    k_hot.copy_(torch.randn((LB, Hk, cap, D), generator=g, device=dev, dtype=dt))
    v_hot.copy_(torch.randn((LB, Hk, cap, D), generator=g, device=dev, dtype=dt))
    q = torch.randn((LB, Hq, D), generator=g, device=dev, dtype=dt)
    k_new = torch.randn((LB, Hk, 1, D), generator=g, device=dev, dtype=dt)
    v_new = torch.randn((LB, Hk, 1, D), generator=g, device=dev, dtype=dt)
    held_pos = torch.randint(0, w.seq_len, (LB, Hk, R), generator=g, device=dev)
    held_valid = torch.rand((LB, Hk, R), generator=g, device=dev) < 0.9
    cur = torch.tensor([w.seq_len], dtype=torch.int64, device=dev)
    o = torch.empty((LB, Hq, D), dtype=dt, device=dev)
    steps = [int(x) for x in torch.linspace(0, w.decode_steps - 1, reps)]

    def decode(i):
        n = R + w.budget + steps[i % len(steps)] + 1
        ops.decode_attention_append(q, k_hot[:, :, :n], v_hot[:, :, :n], k_new, v_new, w.scaling, held_len=R,
                                    held_pos=held_pos, held_valid=held_valid, cur_pos=cur, out=o)

    with torch.cuda.stream(st):
        decode(0)
    dec_ms = differential_ms(st, flush, decode, reps)
    mean_keys = R + w.budget + (w.decode_steps + 1) / 2.0
    nbytes = decode_bytes(w, LB, mean_keys)
    gbps = nbytes / (dec_ms * 1e-3) / 1e9
    out["decode"] = {"us_per_layer_step": round(dec_ms * 1e3 / w.layers, 3), "launch_us": round(dec_ms * 1e3, 2),
                     "bytes_per_launch": int(nbytes), "achieved_GBps": round(gbps, 1),
                     "frac": round(gbps / HBM_PEAK_GBS, 4), "layers_per_launch": w.layers}

    # -- inject: staged held slot of every layer -> re-RoPE into the hot buffers --------------
    # (K/V staged in the cache dtype and the rotary tables at the held
    # positions, as a retrieval ships them)
    inv = synthetic.inv_freq(D, w.theta)
    kv_dt = dt if dt in (torch.float16, torch.bfloat16) else torch.float32
    kes = elem_size(kv_dt)
    kp_host = torch.randn((LB, Hk, R, D), dtype=torch.float32).to(kv_dt).pin_memory()
    vp_host = torch.randn((LB, Hk, R, D), dtype=torch.float32).to(kv_dt).pin_memory()
    kp_dev = torch.empty_like(kp_host, device=dev)
    vp_dev = torch.empty_like(vp_host, device=dev)
    kp_dev.copy_(kp_host)
    vp_dev.copy_(vp_host)
    cos_t, sin_t = ops.rope_tables(held_pos.cpu().reshape(-1, R), inv, 1.0, dt)
    cos_t = cos_t.reshape(LB, Hk, R, D // 2).to(dev)
    sin_t = sin_t.reshape(LB, Hk, R, D // 2).to(dev)

    def inject(i):
        ops.inject_rerope_tab(kp_dev, vp_dev, cos_t, sin_t, k_hot, v_hot)

    with torch.cuda.stream(st):
        inject(0)
    inj_ms = differential_ms(st, flush, inject, reps)
    # staged K and V read, both tables read, K and V written in the cache dtype
    inj_bytes = 2 * LB * Hk * R * D * kes + LB * Hk * R * D * es + 2 * LB * Hk * R * D * es
    side = torch.cuda.Stream(dev)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(side):
        e0.record(side)
        kp_dev.copy_(kp_host, non_blocking=True)
        vp_dev.copy_(vp_host, non_blocking=True)
        e1.record(side)
    torch.cuda.synchronize()
    h2d_ms = e0.elapsed_time(e1)
    h2d_bytes = 2 * LB * Hk * R * D * kes

    # decode while the side stream copies the staged slot (the inject feed's overlap)
    def decode_overlapped(i):
        with torch.cuda.stream(side):
            kp_dev.copy_(kp_host, non_blocking=True)
            vp_dev.copy_(vp_host, non_blocking=True)
        decode(i)

    ov_ms = differential_ms(st, flush, decode_overlapped, reps)
    torch.cuda.synchronize()
    out["inject"] = {"rerope_us_all_layers": round(inj_ms * 1e3, 2), "rerope_bytes": int(inj_bytes),
                     "rerope_GBps": round(inj_bytes / (inj_ms * 1e-3) / 1e9, 1),
                     "rerope_frac": round(inj_bytes / (inj_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "h2d_us_all_layers": round(h2d_ms * 1e3, 1), "h2d_bytes": int(h2d_bytes),
                     "h2d_GBps": round(h2d_bytes / (h2d_ms * 1e-3) / 1e9, 1),
                     "decode_launch_us_with_concurrent_h2d": round(ov_ms * 1e3, 2)}
    del k_hot, v_hot, kp_dev, vp_dev

    # -- compaction of one layer at the full batch ------------------------------------------
    B, S, W = w.batch, w.seq_len, min(w.window, w.seq_len)
    q_post = torch.randn((B, Hq, S, D), generator=g, device=dev, dtype=dt)
    k_post = torch.randn((B, Hk, S, D), generator=g, device=dev, dtype=dt)
    v = torch.randn((B, Hk, S, D), generator=g, device=dev, dtype=dt)
    kb = torch.empty((B, Hk, w.budget, D), dtype=dt, device=dev)
    vb = torch.empty_like(kb)

    def compact(i):
        sc = ops.snapkv_scores(q_post, k_post, W, w.scaling, w.pool, "maxpool")
        keep = ops.keep_index(sc, W, w.budget)
        ops.gather_rows(keep, [(k_post, kb), (v, vb)])

    with torch.cuda.stream(st):
        compact(0)
    comp_ms = differential_ms(st, flush, compact, 6)
    cbytes = compaction_bytes(w, B)
    cg = cbytes / (comp_ms * 1e-3) / 1e9
    sflops = 2.0 * B * Hk * W * S * D      # fp64 window logits (the exact-score contract)
    out["compaction"] = {"ms_per_layer": round(comp_ms, 4), "ms_32_layers": round(comp_ms * w.layers, 3),
                         "bytes_per_layer": int(cbytes), "achieved_GBps": round(cg, 1),
                         "frac": round(cg / HBM_PEAK_GBS, 4),
                         "scoring_tflops_fp64": round(sflops / (comp_ms * 1e-3) / 1e12, 2),
                         "scoring_mfma_frac": round(sflops / (comp_ms * 1e-3) / 1e12 / FP64_MFMA_PEAK_TFLOPS, 4)}
    if cpu:
        out["cpu_baseline"] = cpu_baseline_config(w, q_post[:, :, S - W:].cpu(), k_post.cpu(), v.cpu())
    del q_post, k_post, v, kb, vb
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    out["device_search"] = measure_device_search(w, dev, st, flush, g)
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


DECODE_LAYOUTS = ("separate", "kv_adjacent", "head_interleaved", "kv_adjacent_head_interleaved")


def decode_layout_views(kind, LB, Hk, rows, D, dtype, dev):
    """(k, v) views (LB, Hk, rows, D) of hot rows in one of four HBM layouts:
      separate                      K and V each [LB][Hk][rows][D]
      kv_adjacent                   one [LB][Hk][rows][2][D] (the hot buffer's)
      head_interleaved              K and V each [LB][rows][Hk][D]
      kv_adjacent_head_interleaved  one [LB][rows][Hk][2][D]
    The decode kernel takes row and head strides, so the same launch reads
    all four."""
    import torch
    if kind == "separate":
        return (torch.empty((LB, Hk, rows, D), dtype=dtype, device=dev),
                torch.empty((LB, Hk, rows, D), dtype=dtype, device=dev))
    if kind == "kv_adjacent":
        kv = torch.empty((LB, Hk, rows, 2, D), dtype=dtype, device=dev)
        return kv[:, :, :, 0], kv[:, :, :, 1]
    if kind == "head_interleaved":
        return (torch.empty((LB, rows, Hk, D), dtype=dtype, device=dev).permute(0, 2, 1, 3),
                torch.empty((LB, rows, Hk, D), dtype=dtype, device=dev).permute(0, 2, 1, 3))
    if kind == "kv_adjacent_head_interleaved":
        kv = torch.empty((LB, rows, Hk, 2, D), dtype=dtype, device=dev)
        return kv[:, :, :, 0].permute(0, 2, 1, 3), kv[:, :, :, 1].permute(0, 2, 1, 3)
    raise ValueError(f"unknown layout {kind!r}; one of {DECODE_LAYOUTS}")


def measure_decode_layouts(dev, kinds=DECODE_LAYOUTS, launches=("stacked", "layer"), reps=40):
    """The fused append+decode of the 32-layer 8k->512 hot tier (fp16, 543
    cached rows + the appended token per (layer, KV head), 71.96 MB per
    32-layer launch) over each hot-row layout, beside the plain read of the
    same byte count (hc_read_bytes).  Launches: "stacked" (all 32 layers in
    one launch) and "layer" (one layer's launch, layers in turn).  Timed
    differentially after the cache sweep, the layouts round-robin within
    each repetition, starting one layout later in each repetition, after a
    discarded launch over buffers of their own (so no layout follows a
    launch over its own rows; with one layout, no such launch, so that a
    kernel trace holds that layout's launches only); medians over reps.  Each layout's output is
    checked against an fp32 torch attention first."""
    import torch
    from hotcold_kv import ops, synthetic

    w = synthetic.WORKLOADS["llama8b_8k_b512"]
    LB, Hk, Hq, D, dt = w.layers * w.batch, w.hk, w.hq, w.head_dim, w.dtype
    n = w.budget + 32                       # rows per view: 543 cached + the appended token's row
    g = torch.Generator(device=dev).manual_seed(21)
    st = torch.cuda.Stream(dev)
    flush = CacheSweep(dev)
    q = torch.randn((LB, Hq, D), generator=g, device=dev, dtype=dt)
    k_new = torch.randn((LB, Hk, 1, D), generator=g, device=dev, dtype=dt)
    v_new = torch.randn((LB, Hk, 1, D), generator=g, device=dev, dtype=dt)
    o = torch.empty((LB, Hq, D), dtype=dt, device=dev)
    src_k = torch.randn((LB, Hk, n, D), generator=g, device=dev, dtype=dt)
    src_v = torch.randn((LB, Hk, n, D), generator=g, device=dev, dtype=dt)
    views, out = {}, {}
    for kind in kinds:
        k, v = decode_layout_views(kind, LB, Hk, n + 8, D, dt, dev)
        k[:, :, :n].copy_(src_k)
        v[:, :, :n].copy_(src_v)
        views[kind] = (k, v)
        ops.decode_attention_append(q, k[:, :, :n], v[:, :, :n], k_new, v_new, w.scaling, out=o)
        kk = torch.cat([src_k[:, :, :n - 1], k_new], 2).float()
        vv = torch.cat([src_v[:, :, :n - 1], v_new], 2).float()
        qq = q.float().view(LB, Hk, Hq // Hk, D)
        ref_o = torch.matmul(torch.softmax(torch.matmul(qq, kk.transpose(2, 3).contiguous()) * w.scaling, -1), vv)
        err = float((o.float() - ref_o.reshape(LB, Hq, D)).abs().max())
        if not err < 1e-2:
            raise RuntimeError(f"decode over layout {kind}: max abs error {err} against fp32 torch")
        out[kind] = {"k_strides": list(k.stride()), "v_strides": list(v.stride()), "max_abs_err_vs_fp32": err}
    del src_k, src_v
    views["_dummy"] = decode_layout_views("separate", LB, Hk, n + 8, D, dt, dev)
    for t in views["_dummy"]:
        t.zero_()
    bytes_stacked = decode_bytes(w, LB, n)
    bytes_layer = decode_bytes(w, w.batch, n)

    def ev():
        return torch.cuda.Event(enable_timing=True)

    for launch in launches:
        sw = {kind: [] for kind in kinds}
        pr = {kind: [] for kind in kinds}
        with torch.cuda.stream(st):
            for r in range(3 + reps):
                l = r % LB
                order = ["_dummy"] * (len(kinds) > 1) + [kinds[(r + i) % len(kinds)] for i in range(len(kinds))]
                for kind in order:
                    k, v = views[kind]
                    a0, a1, b0, b1 = ev(), ev(), ev(), ev()
                    a0.record(st)
                    flush()
                    a1.record(st)
                    b0.record(st)
                    flush()
                    if launch == "stacked":
                        ops.decode_attention_append(q, k[:, :, :n], v[:, :, :n], k_new, v_new, w.scaling, out=o)
                    else:
                        ops.decode_attention_append(q[l:l + 1], k[l:l + 1, :, :n], v[l:l + 1, :, :n],
                                                    k_new[l:l + 1], v_new[l:l + 1], w.scaling, out=o[l:l + 1])
                    b1.record(st)
                    if r >= 3 and kind != "_dummy":
                        sw[kind].append((a0, a1))
                        pr[kind].append((b0, b1))
        torch.cuda.synchronize()
        nb = bytes_stacked if launch == "stacked" else bytes_layer
        for kind in kinds:
            ms = (statistics.median(a.elapsed_time(b) for a, b in pr[kind])
                  - statistics.median(a.elapsed_time(b) for a, b in sw[kind]))
            out[kind][f"{launch}_us"] = round(ms * 1e3, 3)
            out[kind][f"{launch}_frac"] = round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    res = {"workload": w.name, "keys_attended": n, "layouts": out}
    if "stacked" in launches:
        res["bytes_stacked"] = int(bytes_stacked)
        res["read_floor_stacked_us"] = round(read_floor_ms(dev, bytes_stacked, st, flush) * 1e3, 3)
    if "layer" in launches:
        res["bytes_layer"] = int(bytes_layer)
        res["read_floor_layer_us"] = round(read_floor_ms(dev, bytes_layer, st, flush) * 1e3, 3)
    return res


def measure_compaction_layer(w, dev, reps=12):
    """One layer's SnapKV compaction of a workload at its full batch (window
    scores, kept indices, gather of K and V into the budget), N(0,1) inputs,
    timed differentially after the cache sweep, median of `reps`.  Printed
    alone by --compaction-only, for per-kernel profiles of the larger
    windows."""
    import torch
    from hotcold_kv import ops
    g = torch.Generator(device=dev).manual_seed(11)
    dt, D, Hk, Hq = w.dtype, w.head_dim, w.hk, w.hq
    B, S, W = w.batch, w.seq_len, min(w.window, w.seq_len)
    q_post = torch.randn((B, Hq, S, D), generator=g, device=dev, dtype=dt)
    k_post = torch.randn((B, Hk, S, D), generator=g, device=dev, dtype=dt)
    v = torch.randn((B, Hk, S, D), generator=g, device=dev, dtype=dt)
    kb = torch.empty((B, Hk, w.budget, D), dtype=dt, device=dev)
    vb = torch.empty_like(kb)
    st, flush = torch.cuda.Stream(dev), CacheSweep(dev)

    def compact(i):
        sc = ops.snapkv_scores(q_post, k_post, W, w.scaling, w.pool, "maxpool")
        keep = ops.keep_index(sc, W, w.budget)
        ops.gather_rows(keep, [(k_post, kb), (v, vb)])

    with torch.cuda.stream(st):
        compact(0)
    ms = differential_ms(st, flush, compact, reps)
    # one plain read of the keys (a known byte count: the calibration of the
    # FETCH_SIZE counter in the same run)
    from hotcold_kv import _native as N
    kbytes = k_post.numel() * k_post.element_size()
    N.check(N.lib().hc_read_bytes(k_post.data_ptr(), kbytes, None, torch.cuda.current_stream(dev).cuda_stream),
            "hc_read_bytes")
    torch.cuda.synchronize()
    sflops = 2.0 * B * Hk * W * S * D
    out = {"workload": w.name, "batch": B, "seq_len": S, "window": W, "budget": w.budget,
           "calibration_read_bytes": int(kbytes),
           "ms_per_layer": round(ms, 4), "scoring_flop_per_layer": int(sflops),
           "scoring_tflops_fp64": round(sflops / (ms * 1e-3) / 1e12, 2),
           "scoring_mfma_frac": round(sflops / (ms * 1e-3) / 1e12 / FP64_MFMA_PEAK_TFLOPS, 4),
           "fp64_floor_ms": round(sflops / (FP64_MFMA_PEAK_TFLOPS * 1e12) * 1e3, 4),
           "bytes_per_layer": int(compaction_bytes(w, B))}
    del q_post, k_post, v, kb, vb
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def measure_device_search(w, dev, st, flush, g, reps=12):
    """One layer's device search index at the workload's cold-store size:
    every sequence's evicted prompt tokens (seq_len - budget of them, N(0,1)
    pre-RoPE keys) added per KV head, then the top-held search per (sequence,
    KV head) timed differentially (hc_index_search), both ways it runs:
      search_us        the fp16 pass (fp16 copy scored in fp32, then the
                       candidates it cannot rule out scored exactly); bytes:
                       the fp16 vectors read once, 4-byte keys written and
                       read once (the candidates' exact reads are ~R rows);
      search_exact_us  the exact fp64 scan alone; bytes: the fp32 vectors
                       read once, 8-byte keys written and read once.
    Both give the same hits (tests/test_kernels_gpu.py)."""
    import numpy as np
    import torch
    from hotcold_kv.device_index import DeviceIndex

    B, Hk, D, R = w.batch, w.hk, w.head_dim, w.held
    n = w.seq_len - w.budget
    dix = DeviceIndex(B, Hk, D, D, Hk, w.seq_len, dev)
    with torch.cuda.stream(st):
        kpre = torch.randn((B, Hk, n, D), generator=g, device=dev, dtype=torch.float32)
        dix.add(kpre, np.tile(np.arange(n, dtype=np.int64), (B, 1)), stream=st.cuda_stream)
        q = torch.randn((B, Hk, D), generator=g, device=dev, dtype=torch.float32)
        hits = torch.empty((B, Hk, R), dtype=torch.int64, device=dev)
    del kpre
    ms = differential_ms(st, flush, lambda i: dix.search(q, R, hits, stream=st.cuda_stream), reps)
    ms_exact = differential_ms(st, flush, lambda i: dix.search(q, R, hits, stream=st.cuda_stream, pass16=False),
                               reps)
    fp16 = dix.vec16 is not None
    nbytes = B * Hk * n * ((2 * D + 8) if fp16 else (4 * D + 16))
    nbytes_exact = B * Hk * n * (4 * D + 16)
    gbs = nbytes / (ms * 1e-3) / 1e9
    gbs_exact = nbytes_exact / (ms_exact * 1e-3) / 1e9
    return {"tokens_per_store": n, "stores": B, "vector_heads": Hk, "vector_dim": D, "top": R,
            "path": "fp16 pass + exact re-score" if fp16 else "exact scan",
            "search_us": round(ms * 1e3, 1), "bytes": int(nbytes), "achieved_GBps": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "search_exact_us": round(ms_exact * 1e3, 1), "bytes_exact": int(nbytes_exact),
            "frac_exact": round(gbs_exact / HBM_PEAK_GBS, 4)}


def cpu_baseline_config(w, q_win, k, v, decode_sample=8, max_batch=16):
    """The reference's torch-CPU path on one layer of a larger workload, in
    the workload's dtype (fp16/bf16 CPU matmul, as scoring.py:70 runs it):
    the compaction of the layer's prompt (snapkv_importance -> keep_index ->
    gather_kv) and decode_sample decode steps (append + SDPA) over the held
    slot and the kept rows.  One layer of at most max_batch sequences is
    timed; the figures are scaled to the full batch and to all layers (the
    work is linear in both), as `sample` states."""
    import torch
    from oracle import reference as ref

    threads = max(1, min(16, os.cpu_count() or 1))
    torch.set_num_threads(threads)
    B_full = k.shape[0]
    if B_full > max_batch:
        q_win, k, v = q_win[:max_batch], k[:max_batch], v[:max_batch]
    scale = B_full / k.shape[0]
    B, Hk, S, D = k.shape
    t0 = time.perf_counter()
    keys, vals = ref.press_compress_torch(q_win, k, v, w.window, w.budget, w.scaling, w.pool, q_is_window=True)
    comp_ms = (time.perf_counter() - t0) * 1e3 * scale
    g = torch.Generator().manual_seed(0)
    if w.held:
        keys = torch.cat([torch.randn((B, Hk, w.held, D), generator=g).to(k.dtype), keys], 2)
        vals = torch.cat([torch.randn((B, Hk, w.held, D), generator=g).to(k.dtype), vals], 2)
    dec = []
    for _ in range(decode_sample + 1):
        qt = torch.randn((B, w.hq, 1, D), generator=g).to(k.dtype)
        kt, vt = (torch.randn((B, Hk, 1, D), generator=g).to(k.dtype) for _ in range(2))
        t0 = time.perf_counter()
        _, keys, vals = ref.press_decode_torch(qt, keys, vals, kt, vt, w.scaling)
        dec.append((time.perf_counter() - t0) * 1e6)
    dec_us = statistics.median(dec[1:]) * scale
    name = str(k.dtype).replace("torch.", "")
    part = f"{B} of its {B_full} sequences, scaled x{scale:g}; " if scale != 1 else ""
    return {"dtype": name, "threads": threads, "kind": "port",
            "compact_ms_per_layer": round(comp_ms, 2),
            "compact_ms_32_layers": round(comp_ms * w.layers, 1),
            "decode_us_per_layer_step": round(dec_us, 1),
            "sample": (f"one layer timed ({part}x{w.layers} for all layers): one compaction of a {S}-token "
                       f"prompt to {w.budget} rows, then {decode_sample} decode steps (median) over {w.held} held "
                       f"+ {w.budget} kept rows, torch CPU in {name}, {threads} threads")}


def measure_h2o(w, dev, reps=5, steps=96):
    """H2O (secondary, not the headline) on one layer of the workload's
    geometry: the prefill scores (the whole prompt as the window under the
    fp64 exact-score contract, causal half only) and decode steps at the
    budget through PressLayerState (append, then attention, score update and
    the one-row eviction in one call; one layer per step, so the step is
    bound by its two calls from Python).  Inputs are N(0,1), generated on the
    device."""
    import torch
    from hotcold_kv import ops
    from hotcold_kv.baselines.layer_state import PressLayerState

    g = torch.Generator(device=dev).manual_seed(9)
    dt, D, Hk, Hq, S = w.dtype, w.head_dim, w.hk, w.hq, w.seq_len
    q = torch.randn((1, Hq, S, D), generator=g, device=dev, dtype=dt)
    k = torch.randn((1, Hk, S, D), generator=g, device=dev, dtype=dt)
    v = torch.randn((1, Hk, S, D), generator=g, device=dev, dtype=dt)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ops.h2o_prefill_scores(q, k, w.scaling)
    ts = []
    for _ in range(reps):
        e0.record()
        ops.h2o_prefill_scores(q, k, w.scaling)
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    pre_ms = statistics.median(ts)
    flops = 2.0 * Hq * D * S * (S + 1) / 2        # causal (row, key) pairs of every query head
    st = PressLayerState("h2o", budget=w.budget, window_size=w.window, kernel_size=w.pool, pooling="maxpool")
    st.prefill(q, k, v, Hq // Hk, w.scaling)
    del q, k, v
    qs = torch.randn((steps, 1, Hq, 1, D), generator=g, device=dev, dtype=dt)
    ks = torch.randn((steps, 1, Hk, 1, D), generator=g, device=dev, dtype=dt)
    vs = torch.randn((steps, 1, Hk, 1, D), generator=g, device=dev, dtype=dt)
    for t in range(8):
        st.decode(qs[t], ks[t], vs[t], Hq // Hk, w.scaling)
    torch.cuda.synchronize()
    e0.record()
    for t in range(steps):
        st.decode(qs[t], ks[t], vs[t], Hq // Hk, w.scaling)
    e1.record()
    torch.cuda.synchronize()
    step_us = e0.elapsed_time(e1) * 1e3 / steps
    out = {"workload": f"one layer of {w.name}: {Hq} query / {Hk} KV heads, {S} tokens, budget {w.budget}, "
                       f"window {w.window}",
           "prefill_scores_ms": round(pre_ms, 3),
           "prefill_scores_tflops_fp64": round(flops / (pre_ms * 1e-3) / 1e12, 2),
           "decode_step_us": round(step_us, 2), "decode_steps": steps,
           "decode_hot_rows": st.get_seq_length()}
    del st, qs, ks, vs
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


class _Rotary:
    """The rotary module the inject path reads (default RoPE, no scaling)."""

    def __init__(self, w, dev):
        from hotcold_kv import synthetic
        self.inv_freq = synthetic.inv_freq(w.head_dim, w.theta, dev)
        self.attention_scaling = 1.0


def _mean_us(ms):
    """Mean of a list of millisecond times in us (None if empty)."""
    return round(statistics.fmean(ms) * 1e3, 1) if ms else None


def hotcold_pipeline(w, dev, profile_steps=None, device_search=True, layers=None, step_sync=False):
    """The hot/cold engine's own loop at a held-slot workload, through
    hotcold_attention (the patched attention's body between RoPE and o_proj):
      prefill  every layer's prompt appended to its HotColdLayer and
               compressed to the budget (cache.py:37-128: raw-logit scores of
               the recent queries, KV-head mean, top-k + recent window); the
               evicted prompt tokens go to the native cold store;
      decode   w.decode_steps steps over all layers: per-KV-head retrieval of
               w.held tokens every w.retrieve_every steps (ranked on the
               layer's device index, rows gathered from the host store on the
               library's worker threads; device_search=False: searched on the
               host store),
               the pinned copy on the side stream, re-RoPE inject into the
               held slot, and the fused append + held decode.
    Knobs: max_capacity_prompt = budget + decode steps and topk_ratio giving
    budget - window prefix tokens, so the prompt is cut to the budget once and
    decode appends without re-compression.  The prompt's own attention (torch
    SDPA in the patch) is not run: it is not part of the hot tier.  Inputs are
    the workload's synthetic tokens, generated on the device beforehand.
    layers: how many of the model's layers to run (default all); where the
    prompts of all of them would take more than a quarter of device memory,
    each layer's prompt is generated just before its update and freed after
    it, and the prefill time is the sum of the updates alone.
    step_sync: end every step by waiting for the decode stream, as a generate
    loop does when it reads the step's sampled token back to the host; without
    it the issuing thread runs ahead of the GPU by as many steps as the queue
    holds, and a search issued in one window may not have run by the next."""
    import torch
    from hotcold_kv import KVController, synthetic
    from hotcold_kv import patch as hp
    from hotcold_kv.cache import HotColdLayer

    L, B, G = int(layers or w.layers), w.batch, w.group
    cap = w.budget + w.decode_steps
    topk = w.budget - w.window
    ctrl = KVController(max_capacity_prompt=cap, topk_ratio=(topk + 0.5) / cap, recent_size=w.window,
                        cpu_buffer_size=w.seq_len, faiss_dim=w.head_dim, window_size=w.retrieve_every,
                        query_pool_size=4, lookahead_k=w.held, hold_retrieved=True, per_head_retrieval=True,
                        profile_overlap=True, enable_asserts=False, device_search=device_search)
    rot = _Rotary(w, dev)
    hp.set_active_rotary_emb(rot)
    ctrl.set_rope(rot.inv_freq, rot.attention_scaling)     # as the patched prefill does before its update
    layers = [HotColdLayer(ctrl) for _ in range(L)]
    steps = w.decode_steps if profile_steps is None else profile_steps
    toks = [[synthetic.make_decode_token(w, l, t, seed=0, device=dev) for l in range(L)] for t in range(steps)]
    esize = torch.empty((), dtype=w.dtype).element_size()
    prompt_bytes = B * w.seq_len * w.head_dim * esize * (2 * w.hq + 3 * w.hk)
    lazy = L * prompt_bytes > torch.cuda.get_device_properties(dev).total_memory // 4

    def prompt(l):
        p = synthetic.make_prompt(w, layer=l, seed=0, device=dev)
        return p, p["q_post"][:, :, -w.window:, :].contiguous()

    # inputs, not timed; lazily, only layer 0's prompt exists before the loop
    prompts = [prompt(l) for l in range(1 if lazy else L)]
    ctrl._lazy_init(prompts[0][0]["k_pre"], n_layers=L)
    prefill_s = 0.0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for l in range(L):
        if lazy:
            p, win = prompts.pop() if l == 0 else prompt(l)
            torch.cuda.synchronize()
            tl = time.perf_counter()
        else:
            p, win = prompts[l]
        layers[l].set_last_query_post(win)
        layers[l].update(key_states=p["k_post"], value_states=p["v"], layer_idx=l,
                         cache_kwargs={"pre_key_states": p["k_pre"], "positions": p["positions"]})
        if lazy:
            torch.cuda.synchronize()
            prefill_s += time.perf_counter() - tl
            del p, win
    torch.cuda.synchronize()
    if not lazy:
        prefill_s = time.perf_counter() - t0
    ctrl.wait_cold_adds()
    prefill_store_s = time.perf_counter() - t0
    del prompts
    step_ms = []
    torch.cuda.synchronize()
    t_all = time.perf_counter()
    for t in range(steps):
        ts = time.perf_counter()
        for l in range(L):
            k = toks[t][l]
            hp.hotcold_attention(ctrl, layers[l], l, k["q_pre"], k["k_pre"], k["v"], k["q_post"], k["k_post"],
                                 k["position"], G, w.scaling)
        if step_sync:
            torch.cuda.current_stream().synchronize()
        step_ms.append((time.perf_counter() - ts) * 1e3)
    t_issue = time.perf_counter()
    torch.cuda.synchronize()
    total_ms = (time.perf_counter() - t_all) * 1e3
    drain_ms = (time.perf_counter() - t_issue) * 1e3
    for l in range(L):
        ctrl.wait_for_retrieval(l)
    d = ctrl.dbg
    sl = ctrl._slots[0][0]
    retr_steps = [t for t in range(steps) if (t + 1) % w.retrieve_every in (0, 1)]
    other = [step_ms[t] for t in range(steps) if t not in retr_steps]
    out = {
        "workload": w.name, "layers": L, "batch": B, "prompt": w.seq_len, "budget": w.budget, "held": w.held,
        "retrieve_every": w.retrieve_every, "decode_steps": steps, "step_sync": step_sync,
        "prefill_compress_evict_s": round(prefill_s, 3),
        "prefill_cold_store_filled_s": round(prefill_store_s, 3),
        "prefill_timing": (f"{L} layers' compaction + eviction through HotColdLayer.update, decode thread's "
                           "wall time (cold-store adds still running on the library's workers), then until every "
                           "add is applied; prompt generation not timed"
                           + ("; prompts generated per layer, so the first figure sums the updates and the "
                              "second includes the generation" if lazy else "")),
        "cold_tokens_per_layer": ctrl.cold_size(0),
        "hot_rows_per_layer_end": layers[0].hot_length(),
        "step_times": ("step_us_wall_mean: the loop's wall time over the steps; the others: each step on the "
                       "issuing thread" + (", including its wait for the decode stream" if step_sync else "")),
        "step_us_wall_mean": round(total_ms * 1e3 / steps, 1),
        "step_us_wall_median": round(statistics.median(step_ms) * 1e3, 1),
        "step_us_issue_mean": round(statistics.fmean(step_ms) * 1e3, 1),
        "step_us_issue_first": round(step_ms[0] * 1e3, 1),
        "step_us_issue_mean_after_first": round(statistics.fmean(step_ms[1:]) * 1e3, 1) if steps > 1 else None,
        "step_us_issue_p90": round(sorted(step_ms)[(9 * len(step_ms)) // 10] * 1e3, 1),
        # the step whose layers start their searches, and the step after it
        # (the searches' copies start; the previous copies are injected)
        "step_us_issue_search_steps_mean": _mean_us([step_ms[t] for t in retr_steps if (t + 1) % w.retrieve_every == 0]),
        "step_us_issue_copy_steps_mean": _mean_us([step_ms[t] for t in retr_steps
                                                   if (t + 1) % w.retrieve_every == 1 and t > 0]),
        "gpu_drain_ms_after_loop": round(drain_ms, 2),
        "step_us_wall_without_retrieval_median": round(statistics.median(other) * 1e3, 1) if other else None,
        "layer_us_wall_mean": round(total_ms * 1e3 / steps / L, 2),
        "retrievals": d["retrieval_launched"],
        "retrievals_on_device_index": d["retrieval_device"],
        "retrievals_scheduled": L * (steps // w.retrieve_every),
        "retrievals_skipped_search_running": L * (steps // w.retrieve_every) - d["retrieval_launched"]
        - d["retrieval_skipped_no_slot"] - d["retrieval_skipped_no_cold"],
        "prefetch_launched": d["prefetch_launched"],
        "prefetch_ready": d["prefetch_ready"],
        "ready_rate": round(d["prefetch_ready"] / max(1, d["prefetch_launched"]), 4),
        "prefetch_not_ready_checks": d["prefetch_not_ready_checks"],
        "injections": d["injection_new"], "held_decodes": d["injection_used"],
        "copy_ms_mean": round(d["prefetch_copy_ms_sum"] / max(1, d["prefetch_copy_ms_count"]), 4),
        "h2d_bytes_per_copy": sl.nbytes[1] if sl.has_tab else sl.nbytes[0],
        "h2d_copy": "one hipMemcpyAsync per retrieval from the slot's pinned block: k_pre and v in the cache dtype, "
                    "int64 positions, valid flags, the rotary tables at the positions",
    }
    del layers, ctrl, toks
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def cpu_model():
    """The host CPU's model string (/proc/cpuinfo), or the platform's name."""
    import platform
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(w, sample_seconds, n_layers=4):
    """The reference's torch-CPU path (snapkv_importance -> keep_index ->
    gather_kv, then per decode step cat + repeat_kv + SDPA) on a bounded
    sample of the same workload: whole single-layer jobs (compaction of the
    prompt + the decode steps) over the first n_layers layers' inputs,
    repeated until the variant's share of sample_seconds has been spent.
    Two variants, as the reference's path could run on the CPU: the
    workload's own dtype (fp16/bf16 CPU matmul, scoring.py:70 as written)
    and the fp32 upcast.  `value` is the first.

    Threads: os.cpu_count() is recorded, and at most 16 are used -- the
    host share of one GPU on a shared multi-GPU node."""
    import torch
    from hotcold_kv import synthetic
    from oracle import reference as ref

    threads = max(1, min(16, os.cpu_count() or 1))
    torch.set_num_threads(threads)
    raw = []
    for l in range(min(n_layers, w.layers)):
        p = synthetic.make_prompt(w, layer=l, seed=0, device="cpu")
        toks = [synthetic.make_decode_token(w, l, t, seed=0, device="cpu") for t in range(w.decode_steps)]
        raw.append((p, toks))

    def run(dtype, seconds):
        layers = [(p["q_post"].to(dtype), p["k_post"].to(dtype), p["v"].to(dtype),
                   [(t["q_post"].to(dtype), t["k_post"].to(dtype), t["v"].to(dtype)) for t in toks])
                  for p, toks in raw]
        q, k, v, _ = layers[0]
        ref.press_compress_torch(q, k, v, w.window, w.budget, w.scaling, w.pool)  # warm-up
        comp, dec = [], []
        jobs = 0
        t_end = time.perf_counter() + seconds
        while jobs < 2 or time.perf_counter() < t_end:
            q, k, v, toks = layers[jobs % len(layers)]
            t0 = time.perf_counter()
            keys, vals = ref.press_compress_torch(q, k, v, w.window, w.budget, w.scaling, w.pool)
            comp.append(time.perf_counter() - t0)
            for qt, kt, vt in toks:
                t0 = time.perf_counter()
                _, keys, vals = ref.press_decode_torch(qt, keys, vals, kt, vt, w.scaling)
                dec.append(time.perf_counter() - t0)
            jobs += 1
        comp_ms = statistics.median(comp) * 1e3
        return {"decode_us_per_layer_step": round(statistics.median(dec) * 1e6, 2),
                "compact_ms_per_layer": round(comp_ms, 3),
                "compact_ms_32_layers": round(comp_ms * w.layers, 2),
                "jobs": jobs, "cpu_seconds": round(sum(comp) + sum(dec), 1)}

    lit_name = str(w.dtype).replace("torch.", "")
    lit = run(w.dtype, sample_seconds / 2)
    up = run(torch.float32, sample_seconds / 2)
    return {
        "value": lit["decode_us_per_layer_step"],
        "unit": "us/layer-step",
        "cores": threads,
        "kind": "port",
        "sample": (f"single-layer jobs of {w.name} cycling over layers 0-{len(raw) - 1}: each an "
                   f"{w.seq_len}-token SnapKV compaction and {w.decode_steps} decode steps (append + SDPA); "
                   f"median per decode step, {lit_name} torch CPU as the workload's dtype "
                   f"({lit['jobs']} jobs, {lit['cpu_seconds']} s); compaction x{w.layers} layers "
                   f"= {lit['compact_ms_32_layers']} ms; the fp32 upcast under variants"),
        "compact_ms_32_layers": lit["compact_ms_32_layers"],
        "variants": {f"{lit_name} (workload dtype)": lit, "fp32 upcast": up},
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
        "threads": threads,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="llama8b_8k_b512")
    ap.add_argument("--cpu-sample-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the secondary figures of the 16k/32k/64k workloads and H2O")
    ap.add_argument("--h2o-only", action="store_true",
                    help="only the H2O figures of one layer (one JSON object; for profiling)")
    ap.add_argument("--pipeline-only", nargs="?", const="llama8b_16k_b1024_held64", metavar="WORKLOAD",
                    help="only the hot/cold pipeline of a held-slot workload, by default the 16k one "
                         "(one JSON object)")
    ap.add_argument("--decode-layouts", nargs="?", const=",".join(DECODE_LAYOUTS), metavar="LAYOUTS",
                    help="only the 32-layer 8k decode over hot-row layouts (comma-separated, default all four), "
                         "beside the plain read of its bytes (one JSON object)")
    ap.add_argument("--layout-launch", choices=("stacked", "layer", "both"), default="both",
                    help="--decode-layouts: time the 32-layer launch, one layer's launch, or both")
    ap.add_argument("--pipeline-layers", type=int, default=None,
                    help="layers of the --pipeline-only run (default: the workload's larger-loop layer count)")
    ap.add_argument("--pipeline-step-sync", action="store_true",
                    help="--pipeline-only: wait for the decode stream at the end of every step")
    ap.add_argument("--device-search-only", action="store_true",
                    help="only the device search index figures of the 16k/32k/64k workloads (one JSON object)")
    ap.add_argument("--compaction-only", metavar="WORKLOAD",
                    help="only one layer's compaction of WORKLOAD at its full batch (one JSON object; for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only; the hot tier shards by batch and KV head "
              "across GPUs with no exchange inside the path, and no multi-GPU figure is produced. "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be at least 1 and --warmup at least 0", file=sys.stderr)
        sys.exit(2)

    import torch
    from hotcold_kv import synthetic

    w = synthetic.WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.h2o_only:
        print(json.dumps({"h2o": measure_h2o(w, dev)}), flush=True)
        return
    if args.device_search_only:
        st, g = torch.cuda.Stream(dev), torch.Generator(device=dev).manual_seed(5)
        flush = CacheSweep(dev)
        print(json.dumps({"device_search": {name: measure_device_search(synthetic.WORKLOADS[name], dev, st, flush, g)
                                             for name in ("llama8b_16k_b1024_held64", "b16_32k_b2048_held128",
                                                          "bf16_b4_64k_b4096_held256")}}), flush=True)
        return
    if args.compaction_only:
        print(json.dumps({"compaction_layer": measure_compaction_layer(synthetic.WORKLOADS[args.compaction_only],
                                                                       dev)}), flush=True)
        return
    if args.decode_layouts:
        launches = ("stacked", "layer") if args.layout_launch == "both" else (args.layout_launch,)
        print(json.dumps({"decode_layouts": measure_decode_layouts(dev, tuple(args.decode_layouts.split(",")),
                                                                   launches)}), flush=True)
        return
    if args.pipeline_only:
        pl = args.pipeline_layers or PIPELINE_LAYERS.get(args.pipeline_only)
        print(json.dumps({"hotcold_pipeline": hotcold_pipeline(synthetic.WORKLOADS[args.pipeline_only], dev,
                                                               layers=pl, step_sync=args.pipeline_step_sync)}),
              flush=True)
        return
    log(f"workload {w.name}: generating inputs on {torch.cuda.get_device_name(dev)}")
    stream = stream_rates(dev)
    log(f"device read sweep {stream['read_GBps']:.0f} GB/s, copy {stream['copy_GBps']:.0f} GB/s")
    s = Setup(w, dev)
    flush = CacheSweep(dev)
    torch.cuda.synchronize()
    s.capture()
    log("captured the compaction and per-layer decode graphs")

    run_steps(s, args.warmup, flush)
    log(f"warmup done ({args.warmup} steps)")
    wall_ms, comp, dec_ms, dec_br_ms = run_steps(s, args.steps, flush)
    comp_ms = statistics.mean(comp)
    dec_us_layer = dec_ms * 1e3 / w.layers            # one append+decode launch covers all layers
    log(f"timed {args.steps} steps: {wall_ms:.3f} ms/step wall (incl. cache sweeps), compaction "
        f"{comp_ms:.3f} ms, append+decode launch {dec_ms * 1e3:.2f} us (differential; "
        f"event-bracketed {dec_br_ms * 1e3:.2f} us) = {dec_us_layer:.3f} us/layer-step")

    # algorithmic rates
    mean_keys = w.budget + (w.decode_steps + 1) / 2.0
    nbytes = decode_bytes(w, s.LB, mean_keys)
    achieved = nbytes / (dec_ms * 1e-3) / 1e9
    cbytes = compaction_bytes(w, s.LB)
    c_achieved = cbytes / (comp_ms * 1e-3) / 1e9
    sflops = 2.0 * s.LB * w.hk * min(w.window, w.seq_len) * w.seq_len * w.head_dim
    log(f"decode {nbytes / 1e6:.1f} MB/launch -> {achieved:.0f} GB/s; compaction {cbytes / 1e6:.0f} MB -> "
        f"{c_achieved:.0f} GB/s, scoring {sflops / (comp_ms * 1e-3) / 1e12:.2f} TFLOP/s fp64")

    floor_ms = read_floor_ms(dev, nbytes, s.stream, flush)
    log(f"plain read of the same {nbytes / 1e6:.1f} MB after the same sweep: {floor_ms * 1e3:.2f} us "
        f"({nbytes / (floor_ms * 1e-3) / 1e9:.0f} GB/s); decode at {floor_ms / dec_ms:.3f} of it")

    # warm-cache decode and the per-layer-launch schedule (last decode step)
    warm_dec_ms = time_graph(s.g_dec20, s.stream, 5) / 20
    pl_cold_ms = time_graph(s.g_pl, s.stream, 20, flush)
    pl_warm_ms = time_graph(s.g_pl, s.stream, 20)
    n_last = w.budget + w.decode_steps
    log(f"last-step decode launch warm {warm_dec_ms * 1e3:.2f} us; per-layer launches cold "
        f"{pl_cold_ms * 1e3 / w.layers:.2f} us/layer, warm {pl_warm_ms * 1e3 / w.layers:.2f} us/layer")
    cpl_ms = time_graph(s.g_cpl, s.stream, 10, flush)
    log(f"compaction as one launch set per layer: {cpl_ms:.3f} ms for {w.layers} layers")
    dro = dropin_compaction(s, flush)
    log(f"drop-in compaction (PressLayerState.compact_prompt, {w.layers} layers): deferred "
        f"{dro['deferred'][0]:.3f} ms GPU / {dro['deferred'][1]:.3f} ms wall, one layer at a time "
        f"{dro['per_layer'][0]:.3f} ms GPU / {dro['per_layer'][1]:.3f} ms wall")
    eager_us = dropin_decode(s, dro.pop("states"))
    log(f"drop-in decode (PressLayerState.decode per layer, eager from Python): {eager_us:.2f} us/layer-step wall")
    del flush

    others = []
    if not args.no_other_configs and args.workload == "llama8b_8k_b512":
        flush = CacheSweep(dev)
        for name in ("llama8b_16k_b1024_held64", "b16_32k_b2048_held128", "bf16_b4_64k_b4096_held256"):
            log(f"secondary figures: {name} ...")
            r = measure_config(synthetic.WORKLOADS[name], dev, flush, cpu=not args.no_cpu_baseline)
            log(f"  decode {r['decode']['us_per_layer_step']} us/layer-step ({r['decode']['frac'] * 100:.1f}% of "
                f"HBM peak), compaction {r['compaction']['ms_per_layer']} ms/layer, re-RoPE "
                f"{r['inject']['rerope_us_all_layers']} us, H2D {r['inject']['h2d_GBps']} GB/s, device search "
                f"{r['device_search']['search_us']} us ({r['device_search']['frac'] * 100:.1f}% of HBM peak)")
            if "cpu_baseline" in r:
                c = r["cpu_baseline"]
                log(f"  cpu baseline ({c['dtype']}, {c['threads']} threads): compaction {c['compact_ms_per_layer']} "
                    f"ms/layer, decode {c['decode_us_per_layer_step']} us/layer-step")
            others.append(r)
        del flush

    pipe = pipe_larger = None
    if not args.no_other_configs and args.workload == "llama8b_8k_b512":
        pw = synthetic.WORKLOADS["llama8b_16k_b1024_held64"]
        log(f"hot/cold pipeline: {pw.name} ...")
        pipe = hotcold_pipeline(pw, dev)
        log(f"  step {pipe['step_us_wall_mean']} us wall ({pipe['layer_us_wall_mean']} us/layer), ready_rate "
            f"{pipe['ready_rate']}, {pipe['retrievals']} retrievals, copy {pipe['copy_ms_mean']} ms")
        pipe_larger = []
        for name, pl in PIPELINE_LAYERS.items():
            for sync in (True, False):
                log(f"hot/cold pipeline: {name}, {pl} layers, "
                    f"{'each step synchronized' if sync else 'steps issued ahead'} ...")
                r = hotcold_pipeline(synthetic.WORKLOADS[name], dev, layers=pl, step_sync=sync)
                log(f"  step {r['step_us_wall_mean']} us wall (median {r['step_us_wall_median']}), searches "
                    f"{r['retrievals']} run of {r['retrievals_scheduled']} scheduled "
                    f"({r['retrievals_skipped_search_running']} skipped: search still running), ready_rate "
                    f"{r['ready_rate']}")
                pipe_larger.append(r)

    h2o = None
    if not args.no_other_configs and args.workload == "llama8b_8k_b512":
        log("H2O on one layer ...")
        h2o = measure_h2o(w, dev)
        log(f"  prefill scores {h2o['prefill_scores_ms']} ms ({h2o['prefill_scores_tflops_fp64']} TFLOP/s fp64), "
            f"decode step {h2o['decode_step_us']} us at {h2o['decode_hot_rows']} hot rows")

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        cpu = cpu_baseline(w, args.cpu_sample_seconds)
        for name, v in cpu["variants"].items():
            log(f"cpu baseline {name}: {v['decode_us_per_layer_step']} us/layer-step, compaction "
                f"{v['compact_ms_32_layers']} ms ({cpu['threads']} threads of {cpu['os_cpu_count']}, {cpu['cpu_model']})")

    result = {
        "metric": METRIC,
        "value": round(dec_us_layer, 4),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}[w.dtype],
        "data": "synthetic",
        "config": {"workload": w.name, "layers": w.layers, "batch": w.batch, "seq_len": w.seq_len,
                   "budget": w.budget, "window": w.window, "pool": w.pool, "decode_steps": w.decode_steps,
                   "q_heads": w.hq, "kv_heads": w.hk, "head_dim": w.head_dim,
                   "schedule": "32 layers per launch, fused append+decode, compaction as a HIP graph, "
                               "Infinity Cache flushed before decode"},
        "compact_ms_32_layers": round(comp_ms, 4),
        "compact_ms_32_layers_per_layer_launches": round(cpl_ms, 4),
        "compact_ms_32_layers_dropin": {
            "deferred_gpu_ms": round(dro["deferred"][0], 4), "deferred_wall_ms": round(dro["deferred"][1], 4),
            "per_layer_gpu_ms": round(dro["per_layer"][0], 4), "per_layer_wall_ms": round(dro["per_layer"][1], 4),
            "hot_rows_per_layer": dro["deferred_rows"],
            "path": "PressLayerState.compact_prompt on every layer; deferred = one DeferredCompaction "
                    "(PressCache default), per_layer = compacted as each prefill returns"},
        "decode_us_per_layer_step": round(dec_us_layer, 4),
        "decode_launch_us_differential": round(dec_ms * 1e3, 3),
        "decode_launch_us_event_bracketed": round(dec_br_ms * 1e3, 3),
        "decode_us_per_layer_launch_cold": round(pl_cold_ms * 1e3 / w.layers, 3),
        "decode_us_per_layer_dropin_eager_wall": round(eager_us, 2),
        "decode_us_per_layer_launch_warm": round(pl_warm_ms * 1e3 / w.layers, 3),
        "decode_launch_us_warm_last_step": round(warm_dec_ms * 1e3, 3),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(w.name),
                     "profiled_launch_us": profiled_launch_us(w.name),
                     "profiled_launch": "rocprofv3 average kernel duration of the launches right after the sweep "
                                        "(committed kernel-trace summary); launch_us exceeds it by the gap between "
                                        "two dependent kernels",
                     "kernel": "decode_attn_kernel (fused append; unsplit at this size, so no merge kernel)",
                     "bytes_per_launch": int(nbytes), "launch_us": round(dec_ms * 1e3, 3),
                     "launch_timing": "events around [cache sweep; decode] minus events around [cache sweep]",
                     "read_floor_us": round(floor_ms * 1e3, 3),
                     "read_floor_frac": round(nbytes / (floor_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "frac_of_read_floor": round(floor_ms / dec_ms, 4),
                     "read_floor": "hc_read_bytes over the same byte count after the same sweep, same timing"},
        # the exact-score contract computes the window logits in fp64 on the
        # matrix cores: compaction is bound by the fp64 MFMA rate, not by HBM
        "roofline_compaction": {"bound": "mfma", "dtype": "f64",
                                "achieved": round(sflops / (comp_ms * 1e-3) / 1e12, 3),
                                "peak": FP64_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                "frac": round(sflops / (comp_ms * 1e-3) / 1e12 / FP64_MFMA_PEAK_TFLOPS, 4),
                                "flop_per_job": int(sflops),
                                "hbm_GBps": round(c_achieved, 1), "hbm_frac": round(c_achieved / HBM_PEAK_GBS, 4),
                                "bytes_per_job": int(cbytes)},
        "device_stream": stream,
        "other_workloads": others,
        "hotcold_pipeline": pipe,
        "hotcold_pipeline_larger": pipe_larger,
        "h2o": h2o,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
