#!/usr/bin/env python3
"""Benchmark: decode GEMV HBM GB/s (% of peak) + prefill GEMM TFLOP/s on one MI355X.

Headline (``value``): the cb4 codebook GEMV of the decode path, M=1, K=2048,
N=6144, cb4-g64 weights (4-bit indices, a 16-entry fp16 codebook per
64-group), bf16 activations, f32 output -- algorithmic bytes (weights +
activations + outputs, each once) per second over the timed steps.

A "step" is one GEMV launch over one of ``copies`` distinct device-resident
weight copies (together > 2x the 256 MB Infinity Cache), so every step reads
its weights from HBM.  Steps are captured once in a HIP graph and replayed;
the timed region is one replay of ``--steps`` launches, waited for on both
sides (stream synchronize).  A hipEvent pair recorded on the launch
stream around the replay gives the per-launch GPU time used for ``roofline``.

Other configurations are reported under ``"secondary"`` (Q8 GEMV config 0,
the Q8 small-M sweep, prefill GEMM, decode stack).  ``cpu_baseline`` times the
C restatement of the reference CPU GEMV (oracle/) on the host cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0       # dense bf16 / fp16 MFMA
MALL_BYTES = 256 << 20          # Infinity Cache
METRIC = "decode GEMV HBM GB/s (% of peak) + prefill GEMM TFLOP/s, 1×MI355X"
EAGER = False   # --eager: plain launches instead of graph replays, for profilers

# HBM bytes per launch of the headline kernel, from two rocprofv3 --pmc runs
# (FETCH_SIZE, WRITE_SIZE) scaled by what the same counters read for a
# device-to-device copy of known size; see profiles/gemv_g64_config1.md.
MEASURED_TRAFFIC_BYTES = {"config1": 12688655}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def bench_attn_step(eng, seq: int, n_head: int, n_kv: int, hd: int, batch: int = 1, calls: int = 100,
                    seed: int = 7, eager: bool = False):
    """The whole attention step (``vxt_hip_attn_step_q8_dev``: gated q, q / k
    RMSNorm, RoPE over half of each head, K / V into the cache, attention) of
    ``batch`` tokens at positions seq - batch .. seq - 1 over a filled cache,
    timed as a captured graph of ``calls`` calls."""
    import numpy as np
    from vxg_amd import engine as E
    rng = np.random.default_rng(seed)
    cache = eng.kv_q8_cache(seq, n_kv, hd)
    per = n_kv * hd
    cache.k_qs.upload(rng.integers(-127, 128, size=seq * per, dtype=np.int8))
    cache.v_qs.upload(rng.integers(-127, 128, size=seq * per, dtype=np.int8))
    d = np.float16(rng.uniform(0.002, 0.02, size=seq * per // 32)).view(np.uint16)
    cache.k_d.upload(d)
    cache.v_d.upload(d)
    q_rows = 2 * n_head * hd
    bufs = [eng.to_device(a) for a in (rng.standard_normal(batch * q_rows).astype(np.float32),
                                       rng.standard_normal(batch * per).astype(np.float32),
                                       rng.standard_normal(batch * per).astype(np.float32),
                                       (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32),
                                       (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))]
    qd, kd, vd, qn, kn = bufs
    out = eng.alloc(batch * n_head * hd * 4)
    p = E.GqaParams(qn.ptr, kn.ptr, 0, 0, 0, n_head, 1, hd // 2, 1, 1e6, 1e-6)
    pos = seq - batch

    def one(s):
        cache.step(p, qd.ptr, kd.ptr, vd.ptr, pos, pos, out.ptr, batch_m=batch, q_stride=q_rows, kv_stride=per,
                   stream=s)

    one(eng.stream)                     # sizes the workspace
    eng.synchronize()
    if eager:   # plain launches (for profilers that do not follow graph replays)
        t0 = time.perf_counter()
        for _ in range(calls):
            one(eng.stream)
        eng.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / calls
    else:
        g = eng.capture(lambda s: [one(s) for _ in range(calls)])
        g.launch(1)
        ms = g.launch(1) / calls
        g.free()
    for b in bufs + [out]:
        b.free()
    cache.free()
    return {"us": ms * 1e3, "us_per_token": ms * 1e3 / batch}


# --------------------------------------------------------------------------
# algorithmic bytes per call
# --------------------------------------------------------------------------

def weight_bytes(m) -> int:
    k = m.kind
    if k == "g64":
        return m.rows * m.padded_cols // 2 + m.rows * (m.padded_cols // 64) * 32
    if k == "q8":
        return m.rows * m.blocks_per_row * 34
    if k == "q4_0":
        return m.rows * m.blocks_per_row * 18
    return (m.rows * m.padded_cols // 2 + m.rows * (m.padded_cols // 128) * 2
            + (m.rows + 1) * 4 + m.outliers_packed.size * 4)


def call_bytes(m, M: int, x_elem: int, y_elem: int) -> int:
    return weight_bytes(m) + M * m.cols * x_elem + M * m.rows * y_elem


# --------------------------------------------------------------------------
# GPU timing
# --------------------------------------------------------------------------

def time_graph(eng, enqueue, steps: int, warmup: int, n_copies: int = 1):
    """Capture `steps` launches into one HIP graph (launch i uses weight copy
    i % n_copies); time one replay.

    Before the timed replay, one pass over all copies in order (its own
    graph) pushes the timed steps' copies out of the Infinity Cache: copy i
    was last touched n_copies - 1 launches before the timed launch that
    reads it, whatever `steps` is.

    Returns (wall seconds, GPU ms from the hipEvent pair on the launch stream).
    """
    if EAGER:
        return time_eager(eng, enqueue, steps, warmup, n_copies)
    s = eng.stream
    for i in range(max(warmup, 1)):                   # eager warm-up
        enqueue(i, s)
    eng.synchronize()
    g = eng.capture(lambda st: [enqueue(i, st) for i in range(steps)])
    g.launch(1)                                       # warm replay
    flush = None
    if n_copies > 1:
        flush = eng.capture(lambda st: [enqueue(i, st) for i in range(n_copies)])
        flush.launch(1)
    eng.synchronize()
    t0 = time.perf_counter()
    ev_ms = g.launch(1)                               # records events, waits
    t1 = time.perf_counter()
    g.free()
    if flush is not None:
        flush.free()
    return (t1 - t0), ev_ms


def bench_gemv(eng, m, M: int, x_dtype: str, y_dtype: str, steps: int, warmup: int,
               seed: int = 0):
    """GB/s of y = W x over rotating weight copies. Returns a result dict."""
    from vxg_amd import engine, synth
    wb = weight_bytes(m)
    n_copies = max(2, math.ceil(2.5 * MALL_BYTES / wb))
    base = eng.upload_packed(m)
    copies = [base] + [base.clone() for _ in range(n_copies - 1)]
    if x_dtype == "bf16":
        xd = eng.to_device(synth.make_x_bf16(M, m.cols, seed=seed))
        xdt, xel = engine.DTYPE_BF16, 2
    else:
        xd = eng.to_device(synth.make_x_f32(M, m.cols, seed=seed))
        xdt, xel = engine.DTYPE_F32, 4
    if y_dtype == "bf16":
        ydt, yel = engine.DTYPE_BF16, 2
    else:
        ydt, yel = engine.DTYPE_F32, 4
    yd = eng.alloc(M * m.rows * yel)

    def enqueue(i, stream):
        eng.matmul_dev(copies[i % n_copies], xd.ptr, xdt, M, yd.ptr, ydt, stream)

    wall_s, ev_ms = time_graph(eng, enqueue, steps, warmup, n_copies)
    nbytes = call_bytes(m, M, xel, yel)
    for c in copies:
        c.free()
    xd.free()
    yd.free()
    kern_ms = ev_ms / steps
    return {
        "bytes_per_call": nbytes, "weight_copies": n_copies, "steps": steps,
        "reuse_distance_mb": round((n_copies - 1) * wb / 2**20, 1),
        "wall_ms_per_step": wall_s * 1e3 / steps, "kernel_ms": kern_ms,
        "GBps": nbytes * steps / wall_s / 1e9, "kernel_GBps": nbytes / (kern_ms * 1e-3) / 1e9,
        "flops_per_call": 2 * M * m.rows * m.cols,
    }


def bench_floor(eng, nbytes: int, steps: int, warmup: int):
    """The HBM floor of one launch that reads `nbytes` (vxt_hip_read_probe_dev:
    the GEMV's access pattern, no arithmetic), over rotating buffers as the
    GEMV lines rotate weight copies."""
    nbytes = (nbytes + 15) // 16 * 16
    n_copies = max(2, math.ceil(2.5 * MALL_BYTES / nbytes))
    bufs = [eng.alloc(nbytes) for _ in range(n_copies)]
    for b in bufs:
        b.upload(np.full(nbytes // 4, 0x3c003c00, np.uint32))

    def enqueue(i, stream):   # one repeated word: every lane's xor fold is 0, never the key 1
        eng.read_probe_dev(bufs[i % n_copies].ptr, nbytes, 1, stream)

    wall_s, ev_ms = time_graph(eng, enqueue, steps, warmup, n_copies)
    for b in bufs:
        b.free()
    kern_ms = ev_ms / steps
    return {"bytes": nbytes, "kernel_ms": kern_ms, "GBps": nbytes / (kern_ms * 1e-3) / 1e9}


def time_eager(eng, enqueue, steps: int, warmup: int, n_copies: int = 1):
    """time_graph's protocol with plain launches (for profilers that do not
    follow graph replays): wall seconds for both returns."""
    s = eng.stream
    for i in range(max(warmup, 1)):
        enqueue(i, s)
    for i in range(n_copies):
        enqueue(i, s)
    eng.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        enqueue(i, s)
    eng.synchronize()
    t1 = time.perf_counter()
    return (t1 - t0), (t1 - t0) * 1e3


def bench_gemm(eng, m, M: int, steps: int, warmup: int, seed: int = 0):
    """TFLOP/s of the prefill dequant+GEMM (bf16 x, bf16 out) over weight copies."""
    from vxg_amd import engine, synth
    wb = weight_bytes(m)
    n_copies = max(2, math.ceil(2.5 * MALL_BYTES / wb))
    base = eng.upload_packed(m)
    copies = [base] + [base.clone() for _ in range(n_copies - 1)]
    xd = eng.to_device(synth.make_x_bf16(M, m.cols, seed=seed))
    yd = eng.alloc(M * m.rows * 2)

    def enqueue(i, stream):
        eng.matmul_dev(copies[i % n_copies], xd.ptr, engine.DTYPE_BF16, M, yd.ptr, engine.DTYPE_BF16, stream)

    wall_s, ev_ms = time_graph(eng, enqueue, steps, warmup, n_copies)
    for c in copies:
        c.free()
    xd.free()
    yd.free()
    flops = 2.0 * M * m.rows * m.cols
    kern_ms = ev_ms / steps
    return {"kernel_ms": kern_ms, "TFLOPs": flops / (kern_ms * 1e-3) / 1e12,
            "wall_TFLOPs": flops * steps / wall_s / 1e12,
            "bytes_per_call": call_bytes(m, M, 2, 2)}


def _stack_layers(eng, kind: str, layers: int, hidden: int, ffn: int, seed: int):
    """Per layer [q;k;v] (3 x hidden rows), o, [gate;up] (2 x ffn rows), down;
    every layer's weights drawn separately.  Returns (layers, weight bytes)."""
    from vxg_amd import stack, synth
    # cb4: centred centroid tables keep a 24-layer chain with no norms in range
    gen = {"g64": synth.make_g64, "cb4": lambda r, c, seed: synth.make_cb4(r, c, seed=seed, centred=True)}[kind]
    lw, nbytes = [], 0
    for li in range(layers):
        s = seed + 10 * li
        qkv = [gen(hidden, hidden, seed=s + i) for i in range(3)]
        o = gen(hidden, hidden, seed=s + 3)
        gu = [gen(ffn, hidden, seed=s + 4), gen(ffn, hidden, seed=s + 5)]
        dn = gen(hidden, ffn, seed=s + 6)
        nbytes += sum(weight_bytes(m) for m in qkv + [o] + gu + [dn])
        lw.append(stack.LayerWeights(eng.upload_concat(qkv), eng.upload_packed(o),
                                     eng.upload_concat(gu), eng.upload_packed(dn)))
    return lw, nbytes


def _free_layers(lw):
    for L in lw:
        for t in (L.qkv, L.o, L.gate_up, L.down):
            t.free()


def bench_stack(eng, kind: str, head_m, tokens: int, layers: int = 24, hidden: int = 2048,
                ffn: int = 6144, seed: int = 40):
    """Config 4: tokens/s of the decode-step linear stack (matmul-only path).

    The layers of ``_stack_layers`` then the Q8 LM head.  One token is
    captured as a HIP graph; ``tokens`` replays are timed.
    """
    from vxg_amd import stack, synth
    lw, nbytes = _stack_layers(eng, kind, layers, hidden, ffn, seed)
    nbytes += weight_bytes(head_m)
    head = eng.upload_packed(head_m)
    st = stack.DecodeStack(eng, lw, head)
    st.set_input(synth.make_x_bf16(1, hidden, seed=4)[0])
    # activations read and written per token (bf16 between layers, f32 logits)
    # qkv: h in, 3h out; o: h, h; gate/up: h, 2 ffn; down: ffn, h
    act = layers * 2 * (8 * hidden + 3 * ffn) + 2 * hidden + 4 * head_m.rows
    nbytes += act
    for _ in range(3):
        st.enqueue()
    eng.synchronize()
    runner = st.capture()
    runner.launch(3)
    t0 = time.perf_counter()
    ev_ms = runner.launch(tokens)
    wall = time.perf_counter() - t0
    runner.free()
    st.free()
    _free_layers(lw)
    head.free()
    ms_tok = ev_ms / tokens
    return {"tokens_per_s": tokens / (ev_ms * 1e-3), "wall_tokens_per_s": tokens / wall,
            "ms_per_token": ms_tok, "bytes_per_token": nbytes, "launches_per_token": st.launches,
            "GBps": nbytes / (ms_tok * 1e-3) / 1e9}


def bench_step(eng, kind: str, head_m, tokens: int, layers: int = 24, hidden: int = 2048,
               ffn: int = 6144, seed: int = 40, fuse_norm: bool = True, eager: bool = False):
    """The whole decode step (``stack.DecodeStep``) on config 4's weights:
    embedding gather (tied Q8 head), per layer RMSNorm, [q;k;v], o,
    add + RMSNorm, fused [gate;up] + SwiGLU, down; final norm, LM head,
    greedy.  Attention stands in as a slice, as in the matmul-only stack.
    Captured once; each replay is one token, the id fed back on the device.
    ``fuse_norm``: each RMSNorm built inside the projection that reads it."""
    import numpy as np
    from vxg_amd import stack
    lw, nbytes = _stack_layers(eng, kind, layers, hidden, ffn, seed)
    nbytes += weight_bytes(head_m)
    head = eng.upload_packed(head_m)
    rng = np.random.default_rng(seed)
    bufs = [eng.to_device((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32))
            for _ in range(2 * layers + 1)]
    norms = [stack.LayerNorms(bufs[2 * i], bufs[2 * i + 1]) for i in range(layers)]
    st = stack.DecodeStep(eng, lw, norms, bufs[-1], head, head, fuse_norm=fuse_norm)
    st.set_token(1)
    for _ in range(3):
        st.enqueue()
    eng.synchronize()
    if eager:   # plain launches (for profilers that do not follow graph replays)
        t0 = time.perf_counter()
        for _ in range(tokens):
            st.enqueue()
        eng.synchronize()
        wall = time.perf_counter() - t0
        ev_ms = wall * 1e3
    else:
        g = st.capture()
        g.launch(3)
        t0 = time.perf_counter()
        ev_ms = g.launch(tokens)
        wall = time.perf_counter() - t0
        g.free()
    tok, bad = st.read_token()
    launches = st.launches
    st.free()
    for b in bufs:
        b.free()
    _free_layers(lw)
    head.free()
    ms_tok = ev_ms / tokens
    return {"tokens_per_s": tokens / (ev_ms * 1e-3), "wall_tokens_per_s": tokens / wall,
            "ms_per_token": ms_tok, "launches_per_token": launches, "last_token": tok, "nonfinite": bad}


def bench_runner(eng, kind: str, head_m, prompt: int, tokens: int, layers: int = 24, hidden: int = 2048,
                 ffn: int = 6144, n_head: int = 16, hd: int = 128, seed: int = 40):
    """The C-level decode-step runner (``vxt_hip_runner_*``) on config 4's
    weights with real attention: per layer RMSNorm, [q;k;v] (16 heads x 128,
    16 kv heads), q / k RMSNorm + RoPE + K/V into the layer's Q8_0 cache +
    attention, o, add + RMSNorm, [gate;up] + SwiGLU, down; final norm, tied Q8
    LM head, greedy.  A ``prompt``-token prefill (one batched step), then
    ``tokens`` greedy decode steps on the device (one graph launch each),
    timed host-side around each call."""
    import numpy as np
    from vxg_amd import engine
    lw, _ = _stack_layers(eng, kind, layers, hidden, ffn, seed)
    head = eng.upload_packed(head_m)
    rng = np.random.default_rng(seed)
    bufs = [eng.to_device((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32))
            for _ in range(2 * layers + 1)]
    qk = [eng.to_device((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)) for _ in range(2)]
    rl = [engine.RunnerLayer(L.qkv.handle, L.o.handle, L.gate_up.handle, L.down.handle, bufs[2 * i].ptr,
                             bufs[2 * i + 1].ptr, qk[0].ptr, qk[1].ptr) for i, L in enumerate(lw)]
    cfg = engine.RunnerConfig(layers, hidden, n_head, n_head, hd, ffn, head_m.rows, 0, hd, 1, engine.ACT_SILU,
                              prompt + tokens + 8, prompt, 1e6, 1e-6, 1.0)
    r = eng.runner(cfg, rl, bufs[-1].ptr, head, head)
    ids = rng.integers(0, head_m.rows, size=prompt).astype(np.uint32)
    r.step(ids, 0)                       # warm: the batched path's workspace
    r.generate(1, prompt, 4)
    t0 = time.perf_counter()
    logits = r.step(ids, 0)
    t_prefill = time.perf_counter() - t0
    t0 = time.perf_counter()
    out, flags = r.generate(int(np.argmax(logits)), prompt, tokens)
    t_decode = time.perf_counter() - t0
    r.free()
    for b in bufs + qk:
        b.free()
    _free_layers(lw)
    head.free()
    return {"prefill_tokens_per_s": prompt / t_prefill, "prefill_ms": t_prefill * 1e3,
            "decode_tokens_per_s": tokens / t_decode, "ms_per_token": t_decode * 1e3 / tokens,
            "nonfinite_steps": int(flags.sum())}


def bench_attn(eng, seq: int, n_head: int, n_kv: int, hd: int, calls: int = 200, seed: int = 6,
               eager: bool = False):
    """Decode attention over a Q8_0 KV cache of ``seq`` positions: one
    ``vxt_hip_attn_q8_dev`` call per step, timed as a captured graph of
    ``calls`` calls.  Bytes: the cache's K and V values and scales."""
    import numpy as np
    rng = np.random.default_rng(seed)
    cache = eng.kv_q8_cache(seq, n_kv, hd)
    per = n_kv * hd
    # fill the cache: values and scales straight into the planes
    cache.k_qs.upload(rng.integers(-127, 128, size=seq * per, dtype=np.int8))
    cache.v_qs.upload(rng.integers(-127, 128, size=seq * per, dtype=np.int8))
    d = np.float16(rng.uniform(0.002, 0.02, size=seq * per // 32)).view(np.uint16)
    cache.k_d.upload(d)
    cache.v_d.upload(d)
    q = eng.to_device(rng.standard_normal(n_head * hd).astype(np.float32))
    out = eng.alloc(n_head * hd * 4)
    cache.attend(q.ptr, n_head, seq, out.ptr, 0, eng.stream)      # sizes the workspace
    eng.synchronize()
    if eager:   # plain launches (for profilers that do not follow graph replays)
        t0 = time.perf_counter()
        for _ in range(calls):
            cache.attend(q.ptr, n_head, seq, out.ptr, 0, eng.stream)
        eng.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / calls
    else:
        g = eng.capture(lambda s: [cache.attend(q.ptr, n_head, seq, out.ptr, 0, s) for _ in range(calls)])
        g.launch(1)
        ms = g.launch(1) / calls
        g.free()
    q.free()
    out.free()
    cache.free()
    nbytes = 2 * seq * per * (1 + 2 / 32)
    return {"us": ms * 1e3, "bytes": nbytes, "GBps": nbytes / (ms * 1e-3) / 1e9}


# --------------------------------------------------------------------------
# CPU baseline (reference CPU path, C restatement in oracle/)
# --------------------------------------------------------------------------

def cpu_baseline(m, budget_s: float = 10.0):
    import oracle
    from vxg_amd import synth
    threads = oracle.hardware_threads()
    xh = synth.make_x_bf16(1, m.cols, seed=0)
    from vxg_amd.formats import bf16_bits_to_f32
    x = bf16_bits_to_f32(xh)[0]
    oracle.gemv(m, x, threads)                 # warm call (bench.rs:317-318)
    n = 0
    t0 = time.perf_counter()
    while True:
        oracle.gemv(m, x, threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    per_call = el / n
    return {
        "value": call_bytes(m, 1, 2, 4) / per_call / 1e9, "unit": "GB/s", "cores": threads,
        "kind": "port", "ms_per_call": per_call * 1e3,
        "sample": f"{n} calls of the g64 GEMV (M=1, K={m.cols}, N={m.rows}) in {el:.1f} s, "
                  f"one warm call first, threads spawned per call (codebook.rs:357-369)",
    }


# --------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline only, no secondary configs")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--configs", default="f,0,r,q,g,2,3,4,s,t,a",
                    help="secondary configurations to run (f: HBM streaming floor at the configs' sizes, "
                         "s: whole decode step on config 4's weights, t: the decode-step runner with KV-cache "
                         "attention on config 4's weights, a: KV-Q8 decode attention, "
                         "c: config 3's cb4 lines on the pinned decode-in-loop tile kernel, q: Q4_0 GEMV at config 1's shape)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--eager", action="store_true",
                    help="time with plain launches instead of graph replays (for profilers: rocprofv3's kernel "
                         "tracer has crashed inside hipGraphLaunch on this image, a cause not shown to be in this "
                         "library; `value` is then not the graph-timed number)")
    args = ap.parse_args()

    global EAGER
    EAGER = args.eager
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs on a single MI355X and has no "
              f"multi-GPU path (asked for --gpus {args.gpus}); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    from vxg_amd import engine, synth

    eng = engine.HipEngine()
    log(f"device {eng.device_name}")

    # headline: config 1
    m = synth.make_g64(6144, 2048, seed=1)
    log("config 1: cb4-g64 GEMV M=1 K=2048 N=6144")
    r = bench_gemv(eng, m, 1, "bf16", "f32", args.steps, args.warmup, seed=0)
    assert r["reuse_distance_mb"] * 2**20 >= 2 * MALL_BYTES, "weight rotation must exceed 2x the MALL"
    log(f"  {r['GBps']:.1f} GB/s wall, kernel {r['kernel_ms']*1e3:.2f} us "
        f"({r['kernel_GBps']:.1f} GB/s)")

    secondary = []
    run = set() if args.quick else {c.strip() for c in args.configs.split(",")}
    if "f" in run:
        # the streaming floor at the headline's and other configs' sizes
        for label, nb in (("config 1 (g64 6144x2048)", 12611584), ("config 1 cb4-ref", 6905860),
                          ("config 0 (Q8 4096x4096)", 17858560), ("config 2 Q8 2048x2048", 4456448),
                          ("config 2 Q8 2048x6144", 13369344), ("50 MB", 50331648),
                          ("config 2 LM head", 330612736)):
            rf = bench_floor(eng, nb, max(20, min(args.steps, int(3e9 / nb))), min(args.warmup, 5))
            secondary.append({"config": f"streaming floor (read-only probe) at {label}: {rf['bytes']} B",
                              "kernel_us": round(rf["kernel_ms"] * 1e3, 3), "GBps": round(rf["GBps"], 1),
                              "frac_hbm": round(rf["GBps"] / HBM_PEAK_GBS, 4)})
            log(f"  floor {label}: {rf['kernel_ms']*1e3:.2f} us ({rf['GBps']:.1f} GB/s)")
    if "0" in run:
        m0 = synth.make_q8(4096, 4096, seed=0)
        log("config 0: Q8 GEMV M=1 K=N=4096 x f32")
        r0 = bench_gemv(eng, m0, 1, "f32", "f32", args.steps, args.warmup, seed=0)
        secondary.append({"config": "0: q8 gemv M=1 K=4096 N=4096 x=f32 y=f32",
                          "GBps": round(r0["GBps"], 1), "kernel_us": round(r0["kernel_ms"] * 1e3, 3),
                          "kernel_GBps": round(r0["kernel_GBps"], 1),
                          "frac_hbm": round(r0["kernel_GBps"] / HBM_PEAK_GBS, 4)})
        log(f"  {r0['GBps']:.1f} GB/s wall, kernel {r0['kernel_ms']*1e3:.2f} us")
    if "r" in run:
        # config 1's shape on the reference cb4 layout (128-column groups, f16
        # scales, one f32 centroid table, ~0.74 % CSR outliers)
        mr = synth.make_cb4(6144, 2048, seed=1)
        rr = bench_gemv(eng, mr, 1, "bf16", "f32", args.steps, args.warmup, seed=0)
        secondary.append({"config": f"1 on the reference cb4 layout: cb4-ref gemv M=1 K=2048 N=6144 "
                                    f"({mr.outliers_packed.size} outliers)",
                          "GBps": round(rr["GBps"], 1), "kernel_us": round(rr["kernel_ms"] * 1e3, 3),
                          "kernel_GBps": round(rr["kernel_GBps"], 1),
                          "frac_hbm": round(rr["kernel_GBps"] / HBM_PEAK_GBS, 4)})
        log(f"  cb4-ref GEMV M=1 K=2048 N=6144: {rr['kernel_GBps']:.1f} GB/s kernel "
            f"({rr['kernel_ms']*1e3:.2f} us)")
        del mr
    if "q" in run:
        # config 1's shape in Q4_0 (4.5 bits per weight streamed from the
        # resident nibble plane, q4_0.rs:109-147 / vxt_gemv.metal:461-520)
        m4 = synth.make_q40(6144, 2048, seed=3)
        r4 = bench_gemv(eng, m4, 1, "bf16", "f32", args.steps, args.warmup, seed=0)
        secondary.append({"config": "Q4_0 gemv M=1 K=2048 N=6144 (4.5 bits per weight)",
                          "GBps": round(r4["GBps"], 1), "kernel_us": round(r4["kernel_ms"] * 1e3, 3),
                          "kernel_GBps": round(r4["kernel_GBps"], 1),
                          "frac_hbm": round(r4["kernel_GBps"] / HBM_PEAK_GBS, 4)})
        log(f"  Q4_0 GEMV M=1 K=2048 N=6144: {r4['kernel_GBps']:.1f} GB/s kernel "
            f"({r4['kernel_ms']*1e3:.2f} us)")
        del m4
    if "g" in run:
        # the headline kernel at larger shapes: how much of config 1's gap to
        # the HBM roofline is the fixed cost of a 12.6 MB launch
        for (K, N) in [(2048, 24576), (8192, 6144), (2048, 151936)]:
            mg = synth.make_g64(N, K, seed=4)
            st = max(20, min(args.steps, int(2e9 / weight_bytes(mg))))
            rg = bench_gemv(eng, mg, 1, "bf16", "f32", st, min(args.warmup, 5), seed=0)
            secondary.append({"config": f"1 at larger shapes: g64 gemv M=1 K={K} N={N}",
                              "GBps": round(rg["GBps"], 1), "kernel_us": round(rg["kernel_ms"] * 1e3, 3),
                              "kernel_GBps": round(rg["kernel_GBps"], 1),
                              "frac_hbm": round(rg["kernel_GBps"] / HBM_PEAK_GBS, 4)})
            log(f"  g64 GEMV M=1 K={K} N={N}: {rg['kernel_GBps']:.1f} GB/s kernel "
                f"({rg['kernel_ms']*1e3:.2f} us)")
            del mg
    if "2" in run:
        for (K, N) in [(2048, 2048), (2048, 6144), (6144, 2048), (2048, 151936)]:
            mq = synth.make_q8(N, K, seed=2)
            for M in (1, 2, 4, 8):
                st = max(20, min(args.steps, int(2e9 / weight_bytes(mq))))
                rq = bench_gemv(eng, mq, M, "bf16", "f32", st, min(args.warmup, 5), seed=M)
                secondary.append({"config": f"2: q8 gemv M={M} K={K} N={N}",
                                  "GBps": round(rq["GBps"], 1),
                                  "kernel_us": round(rq["kernel_ms"] * 1e3, 3),
                                  "kernel_GBps": round(rq["kernel_GBps"], 1),
                                  "frac_hbm": round(rq["kernel_GBps"] / HBM_PEAK_GBS, 4)})
                log(f"  config 2 M={M} K={K} N={N}: {rq['kernel_GBps']:.1f} GB/s kernel")
            del mq
    if "3" in run:
        for kind in ("g64", "q8", "cb4"):
            for (K, N) in [(2048, 6144), (6144, 2048)]:
                mk = {"g64": synth.make_g64, "q8": synth.make_q8, "cb4": synth.make_cb4}[kind](N, K, seed=3)
                for M in (128, 512, 2048):
                    st = max(10, min(100, int(4e12 / (2.0 * M * N * K))))
                    rg = bench_gemm(eng, mk, M, st, 3, seed=M)
                    secondary.append({"config": f"3: {kind} gemm M={M} K={K} N={N} bf16->bf16",
                                      "TFLOPs": round(rg["TFLOPs"], 1),
                                      "kernel_us": round(rg["kernel_ms"] * 1e3, 2),
                                      "frac_mfma": round(rg["TFLOPs"] / BF16_PEAK_TFLOPS, 4)})
                    log(f"  config 3 {kind} M={M} K={K} N={N}: {rg['TFLOPs']:.1f} TFLOP/s")
    if "c" in run:   # config 3's cb4 lines on the decode-in-loop tile kernel (pinned FUSED path)
        eng.set_gemm_path(engine.GEMM_FUSED)
        try:
            for (K, N) in [(2048, 6144), (6144, 2048)]:
                mk = synth.make_cb4(N, K, seed=3)
                for M in (128, 512, 2048):
                    st = max(10, min(100, int(4e12 / (2.0 * M * N * K))))
                    rg = bench_gemm(eng, mk, M, st, 3, seed=M)
                    secondary.append({"config": f"3 on the cb4 decode-in-loop tile kernel (pinned): cb4 gemm M={M} "
                                                f"K={K} N={N} bf16->bf16",
                                      "TFLOPs": round(rg["TFLOPs"], 1),
                                      "kernel_us": round(rg["kernel_ms"] * 1e3, 2),
                                      "frac_mfma": round(rg["TFLOPs"] / BF16_PEAK_TFLOPS, 4)})
                    log(f"  config 3 cb4 (tile kernel) M={M} K={K} N={N}: {rg['TFLOPs']:.1f} TFLOP/s")
        finally:
            eng.set_gemm_path(engine.GEMM_AUTO)
    if "4" in run:
        head_m = synth.make_q8(151936, 2048, seed=5)
        for kind in ("g64", "cb4"):
            how = "HIP graph of 97 launches per token"
            log(f"config 4: decode stack, 24 layers {kind} + Q8 LM head, {how}")
            rs = bench_stack(eng, kind, head_m, tokens=max(20, min(200, args.steps // 2)))
            secondary.append({"config": f"4: decode stack 24x{{[q;k;v],o,[gate;up],down}} {kind} + q8 head, M=1, "
                                        f"{how}",
                              "tokens_per_s": round(rs["tokens_per_s"], 1),
                              "ms_per_token": round(rs["ms_per_token"], 4),
                              "bytes_per_token": rs["bytes_per_token"],
                              "launches_per_token": rs["launches_per_token"],
                              "GBps": round(rs["GBps"], 1),
                              "frac_hbm": round(rs["GBps"] / HBM_PEAK_GBS, 4)})
            log(f"  {rs['tokens_per_s']:.1f} tok/s ({rs['GBps']:.1f} GB/s, "
                f"{rs['ms_per_token']*1e3:.1f} us/token)")
        del head_m

    if "s" in run:
        head_m = synth.make_q8(151936, 2048, seed=5)
        for kind, fuse in (("cb4", False), ("cb4", True)):
            how = "norms inside the projections" if fuse else "separate norm launches"
            log(f"config 4 (whole step): 24 layers {kind} + norms, fused SwiGLU, Q8 head, greedy, embedding; {how}")
            rw = bench_step(eng, kind, head_m, tokens=max(20, min(200, args.steps // 2)), fuse_norm=fuse,
                            eager=args.eager)
            secondary.append({"config": f"4 (whole decode step): embed + 24x{{norm,[q;k;v],o,add+norm,"
                                        f"[gate;up]+swiglu,down}} {kind} + norm + q8 head + greedy, M=1, "
                                        f"{how}, HIP graph of {rw['launches_per_token']} launches per token",
                              "tokens_per_s": round(rw["tokens_per_s"], 1),
                              "ms_per_token": round(rw["ms_per_token"], 4),
                              "launches_per_token": rw["launches_per_token"]})
            log(f"  {rw['tokens_per_s']:.1f} tok/s ({rw['ms_per_token']*1e3:.1f} us/token, "
                f"{rw['launches_per_token']} launches)")
        del head_m
    if "t" in run:
        head_m = synth.make_q8(151936, 2048, seed=5)
        prompt, gen = 512, max(32, min(256, args.steps // 2))
        log(f"runner: 24 layers g64 with Q8_0-cache attention (16 heads x 128), tied Q8 head; prefill {prompt}, "
            f"then {gen} greedy steps")
        rr = bench_runner(eng, "g64", head_m, prompt, gen)
        secondary.append({"config": f"decode-step runner (vxt_hip_runner_*): 24 x {{norm,[q;k;v],q/k norm+RoPE+"
                                    f"Q8_0 KV cache+attention,o,add+norm,[gate;up]+swiglu,down}} g64 + norm + tied "
                                    f"q8 head + greedy; {prompt}-token prefill, then {gen} greedy steps at "
                                    f"positions {prompt}..{prompt + gen - 1}",
                          "prefill_tokens_per_s": round(rr["prefill_tokens_per_s"], 1),
                          "prefill_ms": round(rr["prefill_ms"], 2),
                          "decode_tokens_per_s": round(rr["decode_tokens_per_s"], 1),
                          "ms_per_token": round(rr["ms_per_token"], 4),
                          "nonfinite_steps": rr["nonfinite_steps"]})
        log(f"  prefill {rr['prefill_tokens_per_s']:.0f} tok/s ({rr['prefill_ms']:.1f} ms), decode "
            f"{rr['decode_tokens_per_s']:.1f} tok/s ({rr['ms_per_token']*1e3:.1f} us/token)")
        del head_m
    if "a" in run:
        for seq, nh, nkv in ((4096, 16, 16), (32768, 16, 16), (32768, 16, 4), (131072, 16, 4)):
            ra = bench_attn(eng, seq, nh, nkv, 128, eager=args.eager)
            secondary.append({"config": f"attention over a Q8_0 KV cache: {nh} heads / {nkv} kv heads x 128, "
                                        f"{seq} positions, one decode step",
                              "kernel_us": round(ra["us"], 2), "bytes": int(ra["bytes"]),
                              "GBps": round(ra["GBps"], 1), "frac_hbm": round(ra["GBps"] / HBM_PEAK_GBS, 4)})
            log(f"  attention seq={seq} heads={nh}/{nkv}: {ra['us']:.2f} us, {ra['GBps']:.1f} GB/s")
        for seq, nh, nkv, batch, calls in ((4096, 16, 16, 1, 200), (32768, 16, 4, 1, 200), (2048, 16, 4, 2048, 5),
                                           (8192, 16, 4, 512, 5)):
            rs = bench_attn_step(eng, seq, nh, nkv, 128, batch=batch, calls=calls, eager=args.eager)
            secondary.append({"config": f"attention step (gated q, q/k RMSNorm, RoPE, K/V append, attention): "
                                        f"{nh} heads / {nkv} kv heads x 128, {batch} token(s) ending at position "
                                        f"{seq}",
                              "us_per_call": round(rs["us"], 2), "us_per_token": round(rs["us_per_token"], 3)})
            log(f"  attention step seq={seq} heads={nh}/{nkv} batch={batch}: {rs['us']:.2f} us per call, "
                f"{rs['us_per_token']:.3f} us per token")

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (oracle g64 GEMV)")
        cpu = cpu_baseline(m, args.cpu_seconds)
        log(f"  {cpu['value']:.2f} GB/s on {cpu['cores']} threads")

    achieved = r["kernel_GBps"]
    out = {
        "metric": METRIC,
        "value": round(r["GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["wall_ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 idx + f16 codebook -> f32 acc (bf16 x)",
        "data": "synthetic: seeded cb4-g64 weights (uniform 4-bit indices, sorted N(0,0.02) "
                "fp16 codebooks), bf16 N(0,1) activations",
        "config": {"workload": "config 1: cb4-g64 decode GEMV", "M": 1, "K": 2048, "N": 6144,
                   "x_dtype": "bf16", "y_dtype": "f32", "weight_copies": r["weight_copies"],
                   "mall_defeat": "rotate weight copies totalling > 2x 256 MB MALL; a pass over all copies "
                                  "precedes the timed replay, so each timed launch reads a copy last touched "
                                  f"{r['reuse_distance_mb']} MB of weights earlier",
                   "mb_touched_per_timed_replay": round(r["bytes_per_call"] * args.steps / 2**20, 1),
                   "reuse_distance_mb": r["reuse_distance_mb"],
                   "timing": "HIP graph of `steps` launches, one replay"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": MEASURED_TRAFFIC_BYTES["config1"],
                     "kernel": "vxt::gv::gemv_g64_m1_kernel<1, 4, 1> (g64, M=1)",
                     "bytes_per_launch": r["bytes_per_call"],
                     "kernel_us": round(r["kernel_ms"] * 1e3, 3)},
        "cpu_baseline": None if cpu is None else {k: (round(v, 4) if isinstance(v, float) else v)
                                                  for k, v in cpu.items() if k != "ms_per_call"},
        "secondary": secondary,
    }
    eng.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
