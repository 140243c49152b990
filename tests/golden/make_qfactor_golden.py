"""Query-factor fixture from the CPU oracle (device-mirror schedule).

The query factor 1 + 0.1 ln(1 + floor(p / 16384)) multiplies Q (never K) and
differs from 1 only at positions p >= 16384 (src/metal_kernels.metal:72-76,
src/metal_encode.m:137-140). This workload crosses that boundary with decode
calls and with an append, on the seeded 2-layer synthetic model at the 17920
capacity profile (block 256):
- a 16300-token prompt (synthetic.tokens(seed, 3, 16300)) in 256-token chunks,
  the last one 172 tokens, with a checkpoint at 16300;
- 148 greedy decode calls, positions 16300..16447 (the factor turns on at the
  85th);
- restore to 16300, append 200 ids (synthetic.tokens(seed, 200, 200),
  positions 16300..16499, straddling 16384), then 4 greedy decodes.
For every call: the SHA-256 of its 131072 logits' bytes, the selected id
(orc_select_greedy), the logit range and the top-2 gap.

The fixture also records how far two planted oracle variants move the logits
of the same calls (orc_model.c built with -DORC_PLANT=3, the factor on K
instead of Q, and -DORC_PLANT=8, the factor dropped): both share the prompt's
KV cache (every prompt position is below 16384) and are fed the mirror's ids.
tests/test_query_factor.py asserts from these that every call with a position
at or past 16384 separates the plants from the fixture, bitwise and beyond the
matrix-core path's tolerance, so the GPU tests that compare against the
fixture cannot pass with either mistake.

Usage: python tests/golden/make_qfactor_golden.py
Runtime on 8 host threads: about 4 minutes.
"""
import argparse
import ctypes
import hashlib
import json
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from lunelette_amd import synthetic as syn  # noqa: E402
import oracle_lib  # noqa: E402

CONTEXT, CHUNK, PROMPT, DECODE, APPEND, TAIL = 17920, 256, 16300, 148, 200, 4
PLANTS = (3, 8)


def select(logits):
    token = ctypes.c_int64(-1)
    if oracle_lib.load().orc_select_greedy(logits.ctypes.data, logits.size, ctypes.byref(token)):
        raise RuntimeError("greedy selection rejected the logits")
    return int(token.value)


def record(logits):
    top = np.partition(logits, -2)[-2:]
    return {"sha256": hashlib.sha256(logits.tobytes()).hexdigest(), "token": select(logits),
            "min": float(logits.min()), "max": float(logits.max()),
            "gap": float(top[1] - top[0])}


def turns(model, seed, schedule, first_token, forced=None):
    """Yields (kind, length before the call, logits) for the decode run, the
    restore and the straddling append with its decodes; from a model whose KV
    holds the prompt. Decodes feed the previous greedy id, or the forced ids."""
    length, token, k = PROMPT, first_token, 0
    for _ in range(DECODE):
        if forced is not None:
            token = forced[k]
        k += 1
        logits = model.forward(schedule, [token], length)
        yield "decode", length, logits
        length += 1
        token = select(logits)
    length = PROMPT
    yield "restore", length, None
    ids = syn.tokens(seed, 200, APPEND)
    logits = model.forward(schedule, ids, length)
    yield "append", length, logits
    length += APPEND
    token = select(logits)
    for _ in range(TAIL):
        if forced is not None:
            token = forced[k]
        k += 1
        logits = model.forward(schedule, [token], length)
        yield "decode", length, logits
        length += 1
        token = select(logits)


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--seed", type=int, default=20251201)
    p.add_argument("--layers", type=int, default=2)
    p.add_argument("--threads", type=int, default=min(8, os.cpu_count() or 1))
    p.add_argument("--out", default=os.path.join(HERE, "qfactor_c17920_2layer.json"))
    args = p.parse_args()

    def log(msg):
        print(msg, file=sys.stderr, flush=True)

    t0 = time.time()
    oracle_lib.load().orc_set_threads(args.threads)
    layers = [syn.layer(args.seed, i) for i in range(args.layers)]
    embedding, final_norm = syn.embedding(args.seed).reshape(-1), syn.final_norm(args.seed)
    model = oracle_lib.HostModel(embedding, final_norm, layers, CONTEXT)
    prompt = syn.tokens(args.seed, 3, PROMPT)
    calls = []
    length = 0
    while length < PROMPT:
        n = min(CHUNK, PROMPT - length)
        logits = model.forward(oracle_lib.MIRROR, prompt[length:length + n], length)
        calls.append(dict(kind="prefill" if length == 0 else "append", length=length,
                          count=n, **record(logits)))
        length += n
    checkpoint = logits.copy()
    keys, values = model.keys.copy(), model.values.copy()
    log("prompt of %d tokens in %.0f s" % (PROMPT, time.time() - t0))

    mirror_turns = []
    for kind, at, logits in turns(model, args.seed, oracle_lib.MIRROR, calls[-1]["token"]):
        if kind == "restore":
            logits = checkpoint
        count = APPEND if kind == "append" else 1 if kind == "decode" else 0
        mirror_turns.append((kind, at, logits))
        calls.append(dict(kind=kind, length=at, count=count, **record(logits)))
    log("turns in %.0f s" % (time.time() - t0))

    # Each decode's input is the id selected by the call before it.
    decode_inputs = []
    for before, call in zip(calls[-len(mirror_turns) - 1:-1], calls[-len(mirror_turns):]):
        if call["kind"] == "decode":
            decode_inputs.append(before["token"])

    plants = {}
    with tempfile.TemporaryDirectory() as tmp:
        libs = oracle_lib.build_planted(PLANTS, tmp)
        for n, lib in libs.items():
            lib.orc_set_threads(args.threads)
            planted = oracle_lib.HostModel(embedding, final_norm, layers, CONTEXT, lib=lib)
            planted.keys[:] = keys
            planted.values[:] = values
            same, err = [], []
            for (kind, at, want), (_, _, got) in zip(
                    mirror_turns, turns(planted, args.seed, oracle_lib.MIRROR, None,
                                        decode_inputs)):
                if kind == "restore":
                    got = checkpoint
                span = float(want.max() - want.min())
                same.append(bool(np.array_equal(got.view(np.uint32), want.view(np.uint32))))
                err.append(float(np.max(np.abs(got - want)) / span))
            plants[str(n)] = {"name": oracle_lib.PLANTS[n], "bitwise_equal": same,
                              "max_err_over_range": err}
            log("plant %d in %.0f s" % (n, time.time() - t0))

    result = {"seed": args.seed, "layers": args.layers, "context": CONTEXT, "block": CHUNK,
              "prompt": PROMPT, "prompt_first": [int(t) for t in prompt[:8]],
              "decode": DECODE, "append": APPEND, "tail": TAIL,
              "append_first": [int(t) for t in syn.tokens(args.seed, 200, APPEND)[:4]],
              "schedule": "mirror", "calls": calls, "plants": plants}
    with open(args.out, "w") as f:
        json.dump(result, f)
    log("wrote %s in %.0f s" % (args.out, time.time() - t0))


if __name__ == "__main__":
    main()
