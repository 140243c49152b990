"""Benchmark of the gfx950 Lunelette forward path on one MI355X.

Workload (the one the headline metric is quoted on): the full random-init
26-layer Ministral-3B-shaped FP8 model (hidden 3072, 32/8 heads, FFN 9216,
tied BF16 131072-token head), context capacity 4352, block 256. A seeded
512-token prompt is prefilled in two 256-token chunks (prefill + append), then
greedy decode runs for --steps tokens; a step is one decode call (all layers,
the head, the 512 KiB of logits reaching host memory and host greedy
selection). value = decode tokens/s; prefill tokens/s (the median of 5 timed
512-token prefills from an empty cache) is reported beside it.
After the timed calls the fixture's workload (1024 calls) runs untimed on the
bit-exact path (precise prefill, then the same decode kernels) and, in
lockstep with it and fed the same ids, on the matrix-core path: the bit-exact
ids are compared with the oracle's token fixture (tokens_match_fixture = how
many lead in agreement), and mps_vs_precise_logits gives the matrix-core
path's logit error per call as a fraction of the logit range;
tokens_match_fixture_mps_prefill compares the timed stream, whose matrix-core
prefill leaves a KV cache equal to the oracle's up to rounding. Then decode at
the metric's context: a 4352 - steps token prompt, then --steps timed decode
calls ending at position 4351 (decode_near_capacity).

Also measured, with HIP events on the stream the kernels run on:
- each fused decode operator at position 4351 launched over 26 distinct layer
  weight/KV copies (3.0 GB + 0.9 GB, far beyond the 256 MB Infinity Cache),
  giving the FP8 matvec HBM bandwidth; `roofline` reports the dominant kernel
  (norm + gate/up + SiLU), back to back and, as `in_layer_sequence`, its
  marginal time inside the layer's operator sequence (o before it, down after);
- decode attention at 550, 4352 and 16000 cached positions;
- one FP8 linear 9216x3072 and one prefill layer (256 tokens after 4096);
- the long-context prefix-reuse workload at capacity 17920 (16384-token
  prompt, 8 turns of restore + append 64 + decode 128), with its ids compared
  with the oracle's long fixture;
- the CPU baseline: the oracle's reference-literal schedule on the host cores
  over a bounded decode sample, with the host share of threads and with one,
  and bounded samples of the other configurations (cpu_baseline.configs).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
       [--no-operators] [--no-long] [--no-streams]
"""
import argparse
import ctypes
import hashlib
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
# Timed repetitions of the 512-token prefill (median reported).
PREFILL_TRIALS = 5
# Every DEVICE_SAMPLE-th timed decode step reports its device time.
DEVICE_SAMPLE = 8
METRIC = "decode tok/s + 256-chunk prefill tok/s @4352 ctx; FP8 matvec % HBM peak"

# FP8 weight elements per layer and projection.
FP8_WEIGHTS = {"qkv": 6144 * 3072, "o": 3072 * 4096, "gate_up": 2 * 9216 * 3072,
               "down": 3072 * 9216}
# Matrix-core prefill: activation planes per projection and their format
# (exact hi/mid/lo BF16 split, or two FP16 planes with a power-of-two scale,
# about 22 significant bits); FP8 weights convert exactly; FP32 accumulation.
PREFILL_PLANES = {"qkv": (3, "3 x bf16 (exact split of fp32)"),
                  "o": (2, "2 x fp16 + per-(token, kv head) power-of-two scale (~22 bits)"),
                  "gate_up": (2, "2 x fp16 + per-token power-of-two scale (~22 bits)"),
                  "down": (2, "2 x fp16 + per-(token, K split) power-of-two scale (~22 bits)")}
# Matrix-core prefill attention: operand formats of its two products.
PREFILL_ATTENTION = {
    "attention_qk": "Q and K as 2 x fp16 planes (power of two per (token, head) for Q, per "
                    "position for K, ~22 bits); products ql.kh + qh.kl + qh.kh; fp32 accumulation",
    "attention_pv": "P and V as 2 x bf16 planes truncated (16 bits); products pm.vh + ph.vm + "
                    "ph.vh; fp32 accumulation"}
# Algorithmic bytes per decode-step launch (weights + activations read/written).
FP8_BYTES = {"qkv_rope": 6144 * 3072, "o_residual": 3072 * 4096,
             "gateup_silu": 2 * 9216 * 3072, "down_residual": 3072 * 9216}
ACT_BYTES = {"qkv_rope": (3072 + 3072 + 4096 + 2048) * 4,
             "o_residual": (4096 + 2 * 3072) * 4,
             "gateup_silu": (3072 + 3072 + 9216) * 4,
             "down_residual": (9216 + 2 * 3072) * 4}


def pmc_traffic():
    """HBM bytes per k_gateup_silu launch from the committed PMC summary
    (FETCH_SIZE and WRITE_SIZE runs, calibrated against a kernel of known
    traffic); None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "gateup_silu_decode_pmc_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1023)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--seed", type=int, default=20251201)
    p.add_argument("--prefill", choices=["mps", "custom"], default="mps")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-operators", action="store_true")
    p.add_argument("--op-repeats", type=int, default=4)
    p.add_argument("--no-long", action="store_true",
                   help="skip the long-context prefix-reuse workload (about 10 s)")
    p.add_argument("--no-streams", action="store_true",
                   help="skip the untimed token-stream checks (the bit-exact and matrix-core "
                        "paths in lockstep over the fixture's 1024 calls) and the decode near "
                        "capacity, for profiler runs of the timed workload")
    return p.parse_args()


def time_operators(lh, syn, seed, repeats):
    """Per-operator device time at decode position 4351 (one layer, 4352 cached positions)."""
    lib = lh.lib()
    copies = 26
    capacity, length = 4352, 4351
    host = syn.layer(seed, 0)
    qkv = np.concatenate([host["q"], host["k"], host["v"]], axis=0)
    mats = [("qkv", qkv), ("o", host["o"]), ("gate", host["gate"]), ("up", host["up"]),
            ("down", host["down"])]
    per_layer = sum(m.nbytes for _, m in mats)
    weights = lh.DeviceBuffer(per_layer * copies)
    offset = 0
    first = {}
    for name, m in mats:
        first[name] = weights.ptr + offset
        lh.check(lib.lh_memcpy_htod(weights.ptr + offset, m.ctypes.data, m.nbytes))
        offset += m.nbytes
    for i in range(1, copies):
        lh.check(lib.lh_memcpy_dtod(weights.ptr + i * per_layer, weights.ptr, per_layer))
    norms = lh.DeviceBuffer.from_array(np.concatenate(
        [syn.bf16_to_f32(host["input_norm"]), syn.bf16_to_f32(host["post_norm"])]))
    kv_elems = 8 * capacity * 128
    kv = lh.DeviceBuffer(2 * copies * kv_elems * 4)
    fill = syn.normal_f32(seed, 9002, kv_elems)
    for i in range(2 * copies):
        lh.check(lib.lh_memcpy_htod(kv.ptr + i * kv_elems * 4, fill.ctypes.data, fill.nbytes))
    x = lh.DeviceBuffer.from_array(syn.normal_f32(seed, 9001, 3072))
    layers = []
    for i in range(copies):
        w = lh.LayerWeights()
        base = i * per_layer
        w.qkv, w.o, w.gate, w.up, w.down = (first[n] + base for n in
                                             ("qkv", "o", "gate", "up", "down"))
        for j, n in enumerate(("q", "k", "v", "o", "gate", "up", "down")):
            w.scale[j] = host["scale_" + n]
        w.input_norm = norms.ptr
        w.post_norm = norms.ptr + 3072 * 4
        layers.append(w)
    stream = lib.lh_stream_create()
    # Calibration launch of known traffic for the HBM counters: an elementwise
    # add over 16 Mi floats reads 128 MiB and writes 64 MiB (k_element).
    cal_n = 16 << 20
    cal = lh.DeviceBuffer(3 * cal_n * 4)
    lh.check(lib.lh_memset_device(cal.ptr, 0, 3 * cal_n * 4))
    for _ in range(2):
        lh.check(lib.lh_element(0, cal.ptr, cal.ptr + cal_n * 4, cal.ptr + 2 * cal_n * 4, cal_n,
                                stream))
    ws = lib.lh_workspace_create(capacity, 1)
    ids = np.array([7], np.int64)
    lh.check(lib.lh_workspace_set_tokens(ws, ids.ctypes.data_as(lh.c_int64_p), length, 1, stream))
    start, stop = lib.lh_event_create(), lib.lh_event_create()
    ops = [("qkv_rope", lh.OP_QKV_ROPE), ("attention", lh.OP_ATTENTION),
           ("o_residual", lh.OP_O_RESIDUAL), ("gateup_silu", lh.OP_GATEUP_SILU),
           ("down_residual", lh.OP_DOWN_RESIDUAL)]
    result = {}
    for name, op in ops:
        def launch(i):
            keys = kv.ptr + (2 * (i % copies)) * kv_elems * 4
            values = keys + kv_elems * 4
            lh.check(lib.lh_layer_operator(op, ctypes.byref(layers[i % copies]), x.ptr, keys,
                                           values, ws, stream), name)
        for i in range(copies):
            launch(i)
        n = copies * repeats
        lh.check(lib.lh_event_record(start, stream))
        for i in range(n):
            launch(i)
        lh.check(lib.lh_event_record(stop, stream))
        ms = ctypes.c_float()
        lh.check(lib.lh_event_elapsed_ms(start, stop, ctypes.byref(ms)))
        result[name] = ms.value * 1e3 / n  # microseconds per launch
    # Gate/up inside a layer's operator sequence (q|k|v, attention, o, gate/up,
    # down; each pass on the next weight and KV copy), where o runs before it
    # and down after it as in a decode step: its marginal device time is the
    # sequence's less that of the same sequence without it.
    def sequence(names):
        chosen = [op for name, op in ops if name in names]
        def one(i):
            keys = kv.ptr + (2 * (i % copies)) * kv_elems * 4
            for op in chosen:
                lh.check(lib.lh_layer_operator(op, ctypes.byref(layers[i % copies]), x.ptr,
                                               keys, keys + kv_elems * 4, ws, stream), "sequence")
        for i in range(copies):
            one(i)
        n = copies * repeats
        lh.check(lib.lh_event_record(start, stream))
        for i in range(n):
            one(i)
        lh.check(lib.lh_event_record(stop, stream))
        ms = ctypes.c_float()
        lh.check(lib.lh_event_elapsed_ms(start, stop, ctypes.byref(ms)))
        return ms.value * 1e3 / n
    everything = [name for name, _ in ops]
    full = sequence(everything)
    without = sequence([name for name in everything if name != "gateup_silu"])
    in_sequence = {"layer_us": round(full, 3), "layer_without_gateup_us": round(without, 3),
                   "gateup_silu_us": round(full - without, 3)}
    # Pure-read floors: the same weight bytes (q|k|v, o, gate and up together,
    # down) streamed by lh_read_floor from the same rotating copies, the best
    # grid and loads-in-flight that divide the size.
    spans = {"qkv_rope": (first["qkv"], qkv.nbytes), "o_residual": (first["o"], host["o"].nbytes),
             "gateup_silu": (first["gate"], host["gate"].nbytes + host["up"].nbytes),
             "down_residual": (first["down"], host["down"].nbytes)}
    assert first["up"] == first["gate"] + host["gate"].nbytes
    sink = lh.DeviceBuffer(16384 * 4)
    floors = {}
    for name, (base, nbytes) in spans.items():
        best = None
        for grid in (256, 384, 512, 576, 768, 1024, 1152, 1536, 1728, 2048, 2304, 3072):
            for unroll in (1, 2, 4, 8):
                if nbytes % (grid * 4 * 64 * 16 * unroll):
                    continue
                def launch(i):
                    lh.check(lib.lh_read_floor(base + (i % copies) * per_layer, nbytes, grid,
                                               unroll, sink.ptr, stream), "read floor")
                for i in range(copies):
                    launch(i)
                n = copies * repeats
                lh.check(lib.lh_event_record(start, stream))
                for i in range(n):
                    launch(i)
                lh.check(lib.lh_event_record(stop, stream))
                ms = ctypes.c_float()
                lh.check(lib.lh_event_elapsed_ms(start, stop, ctypes.byref(ms)))
                us = ms.value * 1e3 / n
                if best is None or us < best[0]:
                    best = (us, grid, unroll)
        floors[name] = {"floor_us": round(best[0], 3), "grid": best[1], "unroll": best[2],
                        "kernel_us": round(result[name], 3),
                        "ratio": round(result[name] / best[0], 3)}
    lib.lh_event_destroy(start)
    lib.lh_event_destroy(stop)
    lib.lh_workspace_destroy(ws)
    lib.lh_stream_destroy(stream)
    return result, floors, in_sequence


def time_attention(lh, syn, seed, lengths=(550, 4352, 16000), copies=16, repeats=4):
    """Decode attention (one query token, all 32 heads) over L cached
    positions, L = length + 1, at capacity 16448, rotating `copies` distinct
    KV caches (2.2 GB): HIP-event time per call and K+V read GB/s (8192 B per
    position)."""
    lib = lh.lib()
    capacity = 16448
    kv_elems = 8 * capacity * 128
    kv = lh.DeviceBuffer(2 * copies * kv_elems * 4)
    fill = syn.normal_f32(seed, 9300, kv_elems)
    for i in range(2 * copies):
        lh.check(lib.lh_memcpy_htod(kv.ptr + i * kv_elems * 4, fill.ctypes.data, fill.nbytes))
    q = lh.DeviceBuffer.from_array(syn.normal_f32(seed, 9301, 4096))
    out = lh.DeviceBuffer(4096 * 4)
    stream = lib.lh_stream_create()
    ws = lib.lh_workspace_create(capacity, 1)
    start, stop = lib.lh_event_create(), lib.lh_event_create()
    result = {}
    for L in lengths:
        ids = np.array([7], np.int64)
        lh.check(lib.lh_workspace_set_tokens(ws, ids.ctypes.data_as(lh.c_int64_p), L - 1, 1,
                                             stream))

        def launch(i):
            keys = kv.ptr + 2 * (i % copies) * kv_elems * 4
            lh.check(lib.lh_attention(q.ptr, keys, keys + kv_elems * 4, ws, out.ptr, stream),
                     "attention")
        for i in range(copies):
            launch(i)
        n = copies * repeats
        lh.check(lib.lh_event_record(start, stream))
        for i in range(n):
            launch(i)
        lh.check(lib.lh_event_record(stop, stream))
        ms = ctypes.c_float()
        lh.check(lib.lh_event_elapsed_ms(start, stop, ctypes.byref(ms)))
        us = ms.value * 1e3 / n
        result["L%d" % L] = {"us": round(us, 3),
                             "GBps": round(8192 * L / (us * 1e-6) / 1e9, 1)}
    for e in (start, stop):
        lib.lh_event_destroy(e)
    lib.lh_workspace_destroy(ws)
    lib.lh_stream_destroy(stream)
    return result


def fp8_linear(lh, syn, seed, copies=16, repeats=8):
    """One FP8 linear y = s*(W.x), W 9216x3072 (28.3 MB), s = 0.0125, x ~ N(0,1),
    over `copies` distinct weight copies (453 MB, beyond the 256 MB Infinity
    Cache): HIP-event time per launch and HBM GB/s."""
    lib = lh.lib()
    rows, cols = 9216, 3072
    w = syn.fp8(seed, 500, rows, cols)
    weights = lh.DeviceBuffer(w.nbytes * copies)
    lh.check(lib.lh_memcpy_htod(weights.ptr, w.ctypes.data, w.nbytes))
    for i in range(1, copies):
        lh.check(lib.lh_memcpy_dtod(weights.ptr + i * w.nbytes, weights.ptr, w.nbytes))
    x = lh.DeviceBuffer.from_array(syn.normal_f32(seed, 501, cols))
    y = lh.DeviceBuffer(rows * 4)
    stream = lib.lh_stream_create()
    start, stop = lib.lh_event_create(), lib.lh_event_create()
    for i in range(copies):
        lh.check(lib.lh_fp8_matvec(weights.ptr + i * w.nbytes, 0.0125, x.ptr, y.ptr, rows, cols,
                                   1, 0, stream))
    n = copies * repeats
    lh.check(lib.lh_event_record(start, stream))
    for i in range(n):
        lh.check(lib.lh_fp8_matvec(weights.ptr + (i % copies) * w.nbytes, 0.0125, x.ptr, y.ptr,
                                   rows, cols, 1, 0, stream))
    lh.check(lib.lh_event_record(stop, stream))
    ms = ctypes.c_float()
    lh.check(lib.lh_event_elapsed_ms(start, stop, ctypes.byref(ms)))
    us = ms.value * 1e3 / n
    nbytes = rows * cols + 4 * (cols + rows)
    for e in (start, stop):
        lib.lh_event_destroy(e)
    lib.lh_stream_destroy(stream)
    return {"shape": [rows, cols], "us": round(us, 3), "bytes": nbytes,
            "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}


def prefill_layer(lh, syn, seed, repeats=8):
    """One decoder layer in chunked-prefill mode on the matrix-core path: 256
    tokens after a 4096-token prefix (KV N(0,1)), capacity 4352. HIP-event time
    per layer. Algorithmic work: GEMM 59.59 GFLOP and attention 17.72 GFLOP.
    The MFMA units run each projection once per activation plane
    (PREFILL_PLANES), so the GEMMs issue 128.8 GFLOP of MFMA work."""
    lib = lh.lib()
    capacity, length, count = 4352, 4096, 256
    host = syn.layer(seed, 0)
    qkv = np.concatenate([host["q"], host["k"], host["v"]], axis=0)
    keep = []
    w = lh.LayerWeights()
    for name, m in (("qkv", qkv), ("o", host["o"]), ("gate", host["gate"]), ("up", host["up"]),
                    ("down", host["down"])):
        buf = lh.DeviceBuffer.from_array(m)
        keep.append(buf)
        setattr(w, name, buf.ptr)
    for j, n in enumerate(("q", "k", "v", "o", "gate", "up", "down")):
        w.scale[j] = host["scale_" + n]
    for n in ("input_norm", "post_norm"):
        buf = lh.DeviceBuffer.from_array(syn.bf16_to_f32(host[n]))
        keep.append(buf)
        setattr(w, n, buf.ptr)
    kv_elems = 8 * capacity * 128
    keys = lh.DeviceBuffer.from_array(syn.normal_f32(seed, 9200, kv_elems))
    values = lh.DeviceBuffer.from_array(syn.normal_f32(seed, 9201, kv_elems))
    x0 = lh.DeviceBuffer.from_array(syn.normal_f32(seed, 9202, count * 3072))
    x = lh.DeviceBuffer(count * 3072 * 4)
    stream = lib.lh_stream_create()
    ws = lib.lh_workspace_create(capacity, count)
    ids = np.arange(count, dtype=np.int64)
    lh.check(lib.lh_workspace_set_tokens(ws, ids.ctypes.data_as(lh.c_int64_p), length, count,
                                         stream))
    start, stop = lib.lh_event_create(), lib.lh_event_create()
    total = 0.0
    for rep in range(repeats + 2):
        lh.check(lib.lh_memcpy_dtod(x.ptr, x0.ptr, count * 3072 * 4))
        lh.check(lib.lh_event_record(start, stream))
        lh.check(lib.lh_layer_forward(ctypes.byref(w), x.ptr, keys.ptr, values.ptr, ws,
                                      lh.PATH_MFMA, stream))
        lh.check(lib.lh_event_record(stop, stream))
        ms = ctypes.c_float()
        lh.check(lib.lh_event_elapsed_ms(start, stop, ctypes.byref(ms)))
        if rep >= 2:
            total += ms.value
    us = total * 1e3 / repeats
    gemm, attn = 59.59e9, 17.72e9
    mfma_gemm = 2 * count * sum(n * PREFILL_PLANES[k][0] for k, n in FP8_WEIGHTS.items())
    for e in (start, stop):
        lib.lh_event_destroy(e)
    lib.lh_workspace_destroy(ws)
    lib.lh_stream_destroy(stream)
    return {"tokens": count, "prefix": length, "us": round(us, 1),
            "algorithmic_TFLOPs": round((gemm + attn) / (us * 1e-6) / 1e12, 1),
            "gemm_mfma_GFLOP": round(mfma_gemm / 1e9, 2),
            "gemm_mfma_util_lower_bound": round(mfma_gemm / (us * 1e-6) / 2.5e15, 4)}


def decode_loop(rt, token, steps, sample):
    """The timed greedy decode from `token`: each step is lunelette_metal_decode
    (every layer, the head, the logits in host memory, the finite check) and
    lunelette_select_greedy over the borrowed logits, called straight through
    the C ABI as a C caller would (the Runtime methods add interpreter work
    per step that is not the library's). The device time of every
    `sample`-th step is kept in rt.sampled_device_ms. Returns the tokens."""
    lib = rt._lib
    decode, select, device = (lib.lunelette_metal_decode, lib.lunelette_select_greedy,
                              lib.lunelette_metal_last_device_ms)
    handle, err, logits = rt.handle, rt._err, rt._logits
    logits_ref = ctypes.byref(logits)
    tok = ctypes.c_int64(token)
    tok_ref = ctypes.byref(tok)
    ms = ctypes.c_float()
    ms_ref = ctypes.byref(ms)
    rt.sampled_device_ms = []
    out = []
    for i in range(steps):
        if decode(handle, tok.value, logits_ref, err, 512) or select(logits, tok_ref, err, 512):
            raise RuntimeError(err.value.decode())
        if i % sample == 0:
            device(handle, ms_ref)
            rt.sampled_device_ms.append(ms.value)
        out.append(tok.value)
    return out


def agreement(got, want):
    """Number of leading ids of `got` equal to `want`."""
    n = min(len(got), len(want))
    return next((i for i in range(n) if got[i] != want[i]), n)


def lockstep_streams(lh, Runtime, seed, prompt, steps):
    """The bench workload on the bit-exact path (the 512-token prompt
    prefilled in two 256-token chunks by PREFILL_CUSTOM, the decode kernels
    with a token dimension, then steps - 1 decodes) and, in lockstep with it,
    on the matrix-core path fed the same ids. Returns the bit-exact path's
    greedy ids and, over every call, the matrix-core path's largest logit
    error as a fraction of the precise logits' range, its median, and the
    calls whose greedy id differs (with the precise top-2 gap there as a
    fraction of the range). Untimed."""
    exact = Runtime(seed=seed, layers=26, context=4352, block=256, prefill=lh.PREFILL_CUSTOM,
                    strategy=lh.COMPACT_FP8_ARITHMETIC)
    mps = Runtime(seed=seed, layers=26, context=4352, block=256, prefill=lh.PREFILL_MPS,
                  strategy=lh.COMPACT_FP8_ARITHMETIC)
    try:
        errors, flips = [], []

        def compare(a, b, call):
            span = float(a.max() - a.min())
            errors.append(float(np.max(np.abs(b - a))) / span)
            if exact.greedy() != mps.greedy():
                top = np.partition(a, -2)[-2:]
                flips.append({"call": call, "gap_over_range": float(top[1] - top[0]) / span})

        exact.prefill(prompt[:256], copy=False)
        mps.prefill(prompt[:256], copy=False)
        compare(exact.append(prompt[256:]), mps.append(prompt[256:]), 0)
        tokens = [exact.greedy()]
        for call in range(1, steps):
            a = exact.decode(tokens[-1])
            compare(a, mps.decode(tokens[-1]), call)
            tokens.append(exact.greedy())
        worst = int(np.argmax(errors))
        return tokens, {"calls": len(errors), "max_err_over_range": max(errors),
                        "worst_call": worst,
                        "median_err_over_range": float(np.median(errors)),
                        "calls_over_1e-3": int(np.sum(np.array(errors) > 1e-3)),
                        "greedy_differs": flips}
    finally:
        exact.close()
        mps.close()


def decode_near_capacity(lh, Runtime, seed, steps, prefill_mode):
    """Decode at the metric's context: a seeded prompt of 4352 - steps tokens
    prefilled in 256-token chunks (untimed), then `steps` greedy decode calls,
    timed like `value`, whose positions end at 4351 (the last attends 4352
    positions)."""
    from lunelette_amd import synthetic as syn
    length = 4352 - steps
    prompt = syn.tokens(seed, 4, length)
    rt = Runtime(seed=seed, layers=26, context=4352, block=256, prefill=prefill_mode,
                 strategy=lh.COMPACT_FP8_ARITHMETIC)
    try:
        for begin in range(0, length, 256):
            ids = prompt[begin:begin + 256]
            if begin == 0:
                rt.prefill(ids, copy=False)
            else:
                rt.append(ids, copy=False)
        token = rt.greedy()
        lh.check(lh.lib().lh_device_synchronize())
        t = time.perf_counter()
        decode_loop(rt, token, steps, DEVICE_SAMPLE)
        lh.check(lh.lib().lh_device_synchronize())
        wall = time.perf_counter() - t
        return {"decode_tok_s": round(steps / wall, 2),
                "ms_per_step": round(wall * 1e3 / steps, 4),
                "device_ms_per_step": round(statistics.mean(rt.sampled_device_ms), 4),
                "positions": [length, 4351], "prompt": length}
    finally:
        rt.close()


def fixture_tokens(name):
    """Selected ids of a committed oracle token fixture, or None."""
    path = os.path.join(ROOT, "tests", "golden", name)
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def long_context(lh, syn, Runtime, seed, prefill_mode):
    """Prefix-reuse workload at the 17920 profile: a 16384-token seeded prompt
    prefilled in 256-token chunks (checkpoint after 15872 tokens), then 8
    turns that restore the 15872-token prefix, append 64 new random tokens
    and greedily decode 128 tokens (KV length 15937..16064). The selected ids
    are compared with the oracle's (tests/golden/long_c17920_26layer.json)
    after the timed calls."""
    rt = Runtime(seed=seed, layers=26, context=17920, block=256, prefill=prefill_mode,
                 strategy=lh.COMPACT_FP8_ARITHMETIC)
    try:
        prompt = syn.tokens(seed, 2, 16384)
        keep, chunk = 15872, 256
        lh.check(lh.lib().lh_device_synchronize())
        t = time.perf_counter()
        device = 0.0
        checkpoint = None
        for begin in range(0, len(prompt), chunk):
            ids = prompt[begin:begin + chunk]
            if begin == 0:
                rt.prefill(ids, copy=False)
            else:
                rt.append(ids, copy=False)
            device += rt.last_device_ms()
            if begin + chunk == keep:
                checkpoint = rt.checkpoint()
        lh.check(lh.lib().lh_device_synchronize())
        prefill_s = time.perf_counter() - t
        turns, append_s, decode_s, decode_device = 8, 0.0, 0.0, 0.0
        decoded = 0
        tokens = []
        for turn in range(turns):
            rt.restore(checkpoint, copy=False)
            t = time.perf_counter()
            rt.append(syn.tokens(seed, 100 + turn, 64), copy=False)
            append_s += time.perf_counter() - t
            token = rt.greedy()
            tokens.append(token)
            t = time.perf_counter()
            tokens += decode_loop(rt, token, 128, DEVICE_SAMPLE)
            decode_s += time.perf_counter() - t
            decode_device += statistics.mean(rt.sampled_device_ms) * 128
            decoded += 128
        rt.destroy_checkpoint(checkpoint)
        fx = fixture_tokens("long_c17920_26layer.json")
        match = None
        if fx is not None and fx["seed"] == seed:
            want = [t for turn in fx["turns"] for t in turn["tokens"]]
            match = next((i for i in range(len(want)) if tokens[i] != want[i]), len(want))
        return {"workload": "16384-token prompt in 256-token chunks at context 17920; 8 turns "
                            "restore a 15872-token prefix, append 64 tokens, decode 128",
                "prefill_tok_s": round(len(prompt) / prefill_s, 1),
                "prefill_device_ms": round(device, 2),
                "turn_append_ms": round(append_s * 1e3 / turns, 3),
                "decode_tok_s": round(decoded / decode_s, 2),
                "decode_device_ms_per_step": round(decode_device / decoded, 4),
                "kv_length": [keep + 65, keep + 64 + 128],
                "tokens_sha256": hashlib.sha256(np.array(tokens, np.int64).tobytes()
                                                ).hexdigest()[:16],
                "tokens_match_fixture": match, "tokens": len(tokens)}
    finally:
        rt.close()


# The host threads this process may use, read before the GPU runtime starts
# (it can narrow the main thread's affinity later).
START_AFFINITY = len(os.sched_getaffinity(0))


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(syn, seed, budget_s=10.0):
    """Oracle reference-literal decode of the full model on the host cores
    (the reference's own arithmetic, restated in C, since the reference has no
    CPU forward pass): with all of this process's host share of threads
    (OMP_NUM_THREADS, else the affinity set) and with one thread, each over at
    most `budget_s` seconds of steps."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib
    o = oracle_lib.load()
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or START_AFFINITY
    t0 = time.time()
    layers = [syn.layer(seed, i) for i in range(26)]
    model = oracle_lib.HostModel(syn.embedding(seed).reshape(-1), syn.final_norm(seed), layers,
                                 4352)
    prefix = 512
    fill_k = syn.normal_f32(seed, 9100, 26 * 8 * 4352 * 128)
    model.keys[:] = fill_k
    model.values[:] = fill_k[::-1]
    log("cpu baseline: model ready in %.1fs" % (time.time() - t0))

    def run(threads, max_steps):
        o.orc_set_threads(threads)
        steps, elapsed, token = 0, 0.0, 7
        while elapsed < budget_s and steps < max_steps:
            t = time.time()
            logits = model.forward(oracle_lib.REF, [token], prefix + steps)
            elapsed += time.time() - t
            token = int(np.argmax(logits))
            steps += 1
        return steps, steps / elapsed

    steps, many = run(share, 16)
    steps1, one = run(1, 4)
    configs = cpu_configs(syn, seed, o, oracle_lib, layers, model, share)
    configs["seconds_total"] = round(time.time() - t0, 1)
    return {"value": many, "unit": "tok/s", "cores": share,
            "kind": "port",
            "sample": "%d greedy decode steps of the 26-layer model at L=%d..%d on %d threads "
                      "(OMP_PROC_BIND=%s), oracle reference-literal schedule (Kahan per 32 "
                      "lanes), KV prefix seeded N(0,1); %d steps on 1 thread" % (
                          steps, prefix + 1, prefix + steps, share,
                          os.environ.get("OMP_PROC_BIND"), steps1),
            "value_1thread": one, "host_cpus": START_AFFINITY, "online_cpus": os.cpu_count(),
            "cpu_model": cpu_model(), "configs": configs}


def cpu_configs(syn, seed, o, oracle_lib, layers, model, share, budget_s=1.0):
    """The oracle's reference-literal schedule on the other workloads,
    each bounded to about budget_s of repeats: the FP8 linear 9216x3072 (1
    thread and the host share), one decode layer at position 4351, one
    256-token prefill layer after a 4096-token prefix, and one decode step of
    the 26-layer model at L = 16001 (capacity 17920, KV prefix seeded)."""
    def repeat(fn):
        n, t = 0, time.time()
        while n == 0 or time.time() - t < budget_s:
            fn()
            n += 1
        return (time.time() - t) / n, n

    out = {}
    w = syn.fp8(seed, 500, 9216, 3072)
    x = syn.normal_f32(seed, 501, 3072)
    nbytes = 9216 * 3072 + 4 * (3072 + 9216)
    lin = {}
    for threads in (1, share):
        o.orc_set_threads(threads)
        sec, n = repeat(lambda: oracle_lib.matvec(oracle_lib.REF, 0, w, 0.0125, x, 9216, 3072))
        lin["us_%dthreads" % threads] = round(sec * 1e6, 1)
        lin["GBps_%dthreads" % threads] = round(nbytes / sec / 1e9, 2)
    out["fp8_linear_9216x3072"] = lin
    o.orc_set_threads(share)
    one = oracle_lib.HostModel(np.zeros(1, np.uint16), np.zeros(1, np.uint16), [layers[0]], 4352)
    one.keys[:] = model.keys[:one.keys.size]
    one.values[:] = model.values[:one.values.size]
    xd = syn.normal_f32(seed, 9001, 3072)
    sec, n = repeat(lambda: one.layer_forward(oracle_lib.REF, 0, xd.copy(), 4351, 1))
    out["decode_layer_pos4351"] = {"us": round(sec * 1e6, 1), "repeats": n,
                                   "threads": share}
    xp = syn.normal_f32(seed, 9202, 256 * 3072)
    t = time.time()
    one.layer_forward(oracle_lib.REF, 0, xp.copy(), 4096, 256)
    sec = time.time() - t
    out["prefill_layer_256_after_4096"] = {"s": round(sec, 3), "tok_s": round(256 / sec, 1),
                                           "threads": share}
    long = oracle_lib.HostModel(syn.embedding(seed).reshape(-1), syn.final_norm(seed), layers,
                                17920)
    per_layer = 8 * 17920 * 128
    block = syn.normal_f32(seed, 9400, per_layer)
    for i in range(26):
        long.keys[i * per_layer:(i + 1) * per_layer] = block
        long.values[i * per_layer:(i + 1) * per_layer] = block[::-1]
    t = time.time()
    long.forward(oracle_lib.REF, [7], 16000)
    sec = time.time() - t
    out["long_decode_L16001"] = {"tok_s": round(1 / sec, 3), "steps": 1, "threads": share}
    del long
    return out


def main():
    args = parse()
    # Thread placement for the CPU baseline's OpenMP runtime (read when the
    # oracle library loads).
    os.environ.setdefault("OMP_PROC_BIND", "close")
    if args.gpus != 1:
        print("bench.py measures one MI355X: the library has no multi-GPU path "
              "(--gpus %d requested)" % args.gpus, file=sys.stderr)
        sys.exit(2)
    import lunelette_amd as lh
    from lunelette_amd import synthetic as syn
    from lunelette_amd.runtime import Runtime
    lh.require_gpu()
    prefill_mode = lh.PREFILL_MPS if args.prefill == "mps" else lh.PREFILL_CUSTOM
    t0 = time.time()
    rt = Runtime(seed=args.seed, layers=26, context=4352, block=256, prefill=prefill_mode,
                 strategy=lh.COMPACT_FP8_ARITHMETIC)
    log("model resident in %.1fs: %s" % (time.time() - t0, rt.memory()))
    prompt = syn.tokens(args.seed, 1, 512)

    # Warmup on a throwaway sequence.
    rt.prefill(prompt[:256], copy=False)
    token = rt.greedy()
    for _ in range(args.warmup):
        rt.decode(token, copy=False)
        token = rt.greedy()
    rt.reset()

    # The 512-token prefill, timed PREFILL_TRIALS times from an empty cache
    # (median reported); the decode below continues the last one.
    walls, chunks1, chunks2 = [], [], []
    for trial in range(PREFILL_TRIALS):
        if trial:
            rt.reset()
        lh.check(lh.lib().lh_device_synchronize())
        t = time.perf_counter()
        rt.prefill(prompt[:256], copy=False)
        chunks1.append(rt.last_device_ms())
        rt.append(prompt[256:], copy=False)
        chunks2.append(rt.last_device_ms())
        lh.check(lh.lib().lh_device_synchronize())
        walls.append(time.perf_counter() - t)
    prefill_s = statistics.median(walls)
    chunk1_ms, chunk2_ms = statistics.median(chunks1), statistics.median(chunks2)
    token = rt.greedy()
    tokens = [token]
    log("prefill 512 tokens: %.1f ms (device %.1f + %.1f ms), median of %d" % (
        prefill_s * 1e3, chunk1_ms, chunk2_ms, PREFILL_TRIALS))

    lh.check(lh.lib().lh_device_synchronize())
    t = time.perf_counter()
    tokens += decode_loop(rt, token, args.steps, DEVICE_SAMPLE)
    lh.check(lh.lib().lh_device_synchronize())
    decode_s = time.perf_counter() - t
    device_ms = statistics.mean(rt.sampled_device_ms) * args.steps
    rt.close()
    decode_tok_s = args.steps / decode_s
    log("decode %d steps: %.3f ms/step (device %.3f ms/step)" % (
        args.steps, decode_s * 1e3 / args.steps, device_ms / args.steps))

    out = {
        "metric": METRIC,
        "value": round(decode_tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(decode_s * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "26-layer Ministral-3B-shaped random-init FP8 E4M3 model, "
                               "512-token seeded prompt prefilled in 2x256 chunks, greedy "
                               "decode at context capacity 4352",
                   "weights": "fp8_e4m3 per-tensor scale; bf16 tied head",
                   "context": 4352, "block": 256, "prompt": 512,
                   "decode_positions": [512, 512 + args.steps - 1],
                   "prefill_mode": args.prefill, "strategy": "compact-fp8-arithmetic"},
        "decode_tok_s": round(decode_tok_s, 2),
        "decode_device_ms_per_step": round(device_ms / args.steps, 4),
        "prefill_tok_s": round(512 / prefill_s, 1),
        "prefill_device_ms_per_chunk": [round(chunk1_ms, 3), round(chunk2_ms, 3)],
        "prefill_trials": PREFILL_TRIALS,
        "tokens_sha256": hashlib.sha256(np.array(tokens, np.int64).tobytes()).hexdigest()[:16],
        "first_tokens": tokens[:8],
    }
    fx = fixture_tokens("stream_c4352_26layer.json")
    if fx is not None and fx["seed"] == args.seed and args.prefill == "mps" and not args.no_streams:
        # Token identity, after the timed region: the bit-exact path (precise
        # prefill, then the same decode kernels) against the oracle's stream,
        # and the timed stream itself, whose matrix-core prefill leaves a KV
        # cache equal to the oracle's up to rounding (a near-tie can flip).
        want = fx["tokens_mirror"]
        n = min(len(tokens), len(want))
        exact, lockstep = lockstep_streams(lh, Runtime, args.seed, prompt, len(want))
        out["tokens_match_fixture"] = agreement(exact, want)
        out["tokens_match_fixture_mps_prefill"] = agreement(tokens, want)
        out["tokens_compared"] = n
        out["tokens_compared_precise"] = len(want)
        out["mps_vs_precise_logits"] = lockstep
        log("token stream: precise prefill %d/%d equal the oracle's, matrix-core prefill %d/%d"
            % (out["tokens_match_fixture"], len(want), out["tokens_match_fixture_mps_prefill"], n))
        log("matrix-core vs precise logits over %d calls: max %.3g, median %.3g of the range, "
            "%d greedy differences" % (lockstep["calls"], lockstep["max_err_over_range"],
                                       lockstep["median_err_over_range"],
                                       len(lockstep["greedy_differs"])))
    if args.steps < 4352 and not args.no_streams:
        out["decode_near_capacity"] = decode_near_capacity(lh, Runtime, args.seed, args.steps,
                                                           prefill_mode)
        log("decode near capacity: %s" % out["decode_near_capacity"])
    out["config"]["prefill_activations"] = dict({k: v[1] for k, v in PREFILL_PLANES.items()},
                                                **PREFILL_ATTENTION)
    if not args.no_operators:
        ops, floors, in_sequence = time_operators(lh, syn, args.seed, args.op_repeats)
        fp8_us = sum(ops[k] for k in FP8_BYTES)
        fp8_gbps = sum(FP8_BYTES.values()) / (fp8_us * 1e-6) / 1e9
        dom = "gateup_silu"
        dom_bytes = FP8_BYTES[dom] + ACT_BYTES[dom]
        achieved = dom_bytes / (ops[dom] * 1e-6) / 1e9
        out["operators_us_at_pos4351"] = {k: round(v, 3) for k, v in ops.items()}
        out["fp8_matvec"] = {"GBps": round(fp8_gbps, 1), "frac_hbm": round(fp8_gbps / HBM_PEAK_GBPS, 4),
                             "bytes_per_layer": sum(FP8_BYTES.values()),
                             "read_floors": floors}
        out["roofline"] = {"bound": "hbm", "kernel": "k_gateup_silu (RMSNorm + gate/up FP8 "
                           "row dots + SiLU*up)", "achieved": round(achieved, 1),
                           "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                           "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": pmc_traffic(),
                           "bytes_per_launch": dom_bytes, "avg_us": round(ops[dom], 3),
                           "in_layer_sequence": dict(in_sequence, frac=round(
                               dom_bytes / (in_sequence["gateup_silu_us"] * 1e-6) / 1e9
                               / HBM_PEAK_GBPS, 4))}
        log("operators (us): %s" % out["operators_us_at_pos4351"])
        log("read floors: %s" % floors)
        out["decode_attention"] = time_attention(lh, syn, args.seed)
        log("decode attention: %s" % out["decode_attention"])
        out["fp8_linear_9216x3072"] = fp8_linear(lh, syn, args.seed)
        out["prefill_layer_256_after_4096"] = prefill_layer(lh, syn, args.seed)
        log("fp8 linear: %s" % out["fp8_linear_9216x3072"])
        log("prefill layer: %s" % out["prefill_layer_256_after_4096"])
    if not args.no_long:
        out["long_context"] = long_context(lh, syn, Runtime, args.seed, prefill_mode)
        log("long context: %s" % out["long_context"])
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(syn, args.seed)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
