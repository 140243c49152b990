"""Greedy token streams of the full synthetic model from the CPU oracle.

Workload: the random-init 26-layer Ministral-3B-shaped FP8 model built from
seed --seed (lunelette_amd.synthetic), context 4352, a --prompt-token seeded
prompt (synthetic.tokens(seed, 1, prompt)) prefilled in --chunk-token chunks,
then --decode greedy tokens (the first one selected from the prefill logits),
each selected with orc_select_greedy (src/generation.c:8-34 tie rule).

Both oracle schedules are run: ORC_MIRROR (the device schedule, which the
precise GPU path matches bit for bit) and ORC_REF (the reference-literal
arithmetic of src/metal_kernels.metal). The fixture holds the token ids, the
argmax logit of every step of each stream, and the first step at which the
two streams differ (the model amplifies ulp-level differences through
near-ties of its one-hot softmax).

Usage: python tests/golden/make_stream_golden.py [--decode 1024] [--out PATH]
Runtime: a few minutes per schedule on 16 host threads.
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


def stream(model, schedule, prompt, chunk, decode, log):
    o = oracle_lib.load()
    model.keys[:] = 0
    model.values[:] = 0
    length = 0
    logits = None
    for begin in range(0, len(prompt), chunk):
        ids = prompt[begin:begin + chunk]
        logits = model.forward(schedule, ids, length)
        length += len(ids)
    tokens, maxima = [], []
    token = ctypes.c_int64(-1)
    t0 = time.time()
    for step in range(decode):
        if o.orc_select_greedy(logits.ctypes.data, logits.size, ctypes.byref(token)):
            raise RuntimeError("greedy selection failed at step %d" % step)
        tokens.append(int(token.value))
        maxima.append(float(logits[token.value]))
        if step + 1 == decode:
            break
        logits = model.forward(schedule, [token.value], length)
        length += 1
        if step % 64 == 63:
            log("  schedule %d: %d tokens, %.1f s" % (schedule, step + 1, time.time() - t0))
    return tokens, maxima


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--seed", type=int, default=20251201)
    p.add_argument("--layers", type=int, default=26)
    p.add_argument("--prompt", type=int, default=512)
    p.add_argument("--chunk", type=int, default=256)
    p.add_argument("--decode", type=int, default=1024)
    p.add_argument("--context", type=int, default=4352)
    p.add_argument("--out", default=os.path.join(HERE, "stream_c4352_26layer.json"))
    args = p.parse_args()

    def log(msg):
        print(msg, file=sys.stderr, flush=True)

    o = oracle_lib.load()
    o.orc_set_threads(min(16, os.cpu_count() or 1))
    t0 = time.time()
    layers = [syn.layer(args.seed, i) for i in range(args.layers)]
    model = oracle_lib.HostModel(syn.embedding(args.seed).reshape(-1), syn.final_norm(args.seed),
                                 layers, args.context)
    prompt = syn.tokens(args.seed, 1, args.prompt)
    log("model ready in %.1f s" % (time.time() - t0))
    result = {"seed": args.seed, "layers": args.layers, "context": args.context,
              "prompt": args.prompt, "chunk": args.chunk, "decode": args.decode,
              "prompt_sha_first": [int(t) for t in prompt[:8]]}
    for name, schedule in (("mirror", oracle_lib.MIRROR), ("ref", oracle_lib.REF)):
        t = time.time()
        tokens, maxima = stream(model, schedule, prompt, args.chunk, args.decode, log)
        result["tokens_" + name] = tokens
        result["max_logit_" + name] = maxima
        log("%s: %d tokens in %.1f s" % (name, len(tokens), time.time() - t))
    a, b = result["tokens_mirror"], result["tokens_ref"]
    result["first_divergence"] = next((i for i in range(len(a)) if a[i] != b[i]), None)
    with open(args.out, "w") as f:
        json.dump(result, f)
    log("wrote %s (first divergence: %s)" % (args.out, result["first_divergence"]))


if __name__ == "__main__":
    main()
