"""How far two FP32 schedules of the same model lie apart: the oracle's
reference-literal schedule (ORC_REF: the arithmetic of
src/metal_kernels.metal, per-lane Kahan sums, two-pass softmax) against its
device-mirror schedule (ORC_MIRROR), run in lockstep on the 26-layer decode
workload at context 4352.

Workload: the seeded 26-layer synthetic model, context 4352, the 512-token
prompt (synthetic.tokens(seed, 1, 512)) prefilled in two 256-token chunks,
then --decode - 1 decode calls, both schedules fed the mirror's greedy ids
(tests/golden/stream_c4352_26layer.json holds the same ids). For every call:
max |ref - mirror| over the 131072 logits as a fraction of the mirror logits'
range, and the mirror's top-2 gap as the same fraction.

Both schedules are exact FP32 restatements that differ only in summation order
and rounding placement, so this envelope is what reordering alone does to the
logits of this model; the matrix-core path's error is compared with it.

Usage: python tests/golden/make_schedule_envelope.py [--decode 1024]
Runtime on 8 host threads: about 15 minutes.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from lunelette_amd import synthetic as syn  # noqa: E402
import oracle_lib  # noqa: E402


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--seed", type=int, default=20251201)
    p.add_argument("--decode", type=int, default=1024)
    p.add_argument("--threads", type=int, default=min(8, os.cpu_count() or 1))
    p.add_argument("--out", default=os.path.join(HERE, "schedule_envelope_c4352_26layer.json"))
    args = p.parse_args()
    o = oracle_lib.load()
    o.orc_set_threads(args.threads)
    t0 = time.time()
    layers = [syn.layer(args.seed, i) for i in range(26)]
    embedding, final_norm = syn.embedding(args.seed).reshape(-1), syn.final_norm(args.seed)
    mirror = oracle_lib.HostModel(embedding, final_norm, layers, 4352)
    ref = oracle_lib.HostModel(embedding, final_norm, layers, 4352)
    prompt = syn.tokens(args.seed, 1, 512)
    errors, gaps, tokens = [], [], []

    def record(a, b):
        span = float(a.max() - a.min())
        errors.append(float(np.max(np.abs(b - a))) / span)
        top = np.partition(a, -2)[-2:]
        gaps.append(float(top[1] - top[0]) / span)
        token = ctypes.c_int64(-1)
        if o.orc_select_greedy(a.ctypes.data, a.size, ctypes.byref(token)):
            raise RuntimeError("greedy selection rejected the logits")
        tokens.append(int(token.value))

    mirror.forward(oracle_lib.MIRROR, prompt[:256], 0)
    ref.forward(oracle_lib.REF, prompt[:256], 0)
    record(mirror.forward(oracle_lib.MIRROR, prompt[256:], 256),
           ref.forward(oracle_lib.REF, prompt[256:], 256))
    for call in range(1, args.decode):
        length = 511 + call
        record(mirror.forward(oracle_lib.MIRROR, [tokens[-1]], length),
               ref.forward(oracle_lib.REF, [tokens[-1]], length))
        if call % 64 == 0:
            print("  %d calls, %.0f s, worst so far %.3g" % (call, time.time() - t0, max(errors)),
                  file=sys.stderr, flush=True)
    result = {"seed": args.seed, "layers": 26, "context": 4352, "prompt": 512, "chunk": 256,
              "calls": len(errors), "tokens_mirror_first": tokens[:8],
              "max_err_over_range": max(errors), "worst_call": int(np.argmax(errors)),
              "median_err_over_range": float(np.median(errors)),
              "calls_over_1e-3": int(np.sum(np.array(errors) > 1e-3)),
              "err_over_range": errors, "gap_over_range": gaps}
    with open(args.out, "w") as f:
        json.dump(result, f)
    print("wrote %s in %.0f s: max %.3g (call %d), median %.3g" % (
        args.out, time.time() - t0, result["max_err_over_range"], result["worst_call"],
        result["median_err_over_range"]), file=sys.stderr)


if __name__ == "__main__":
    main()
