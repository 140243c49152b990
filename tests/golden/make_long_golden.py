"""Long-context prefix-reuse fixtures from the CPU oracle (device-mirror schedule).

Workload (capacity profile 17920, block 256): the seeded synthetic model, a
16384-token prompt (synthetic.tokens(seed, 2, 16384)) prefilled in 256-token
chunks, with a checkpoint taken when the length reaches 15872. Then `turns`
turns each restore the checkpoint (length back to 15872, logits back to the
checkpoint's), append 64 new ids (synthetic.tokens(seed, 100 + turn, 64)) and
run `decode` greedy decode calls, each on the token selected from the previous
logits (orc_select_greedy, the tie rule of src/generation.c:8-34). Positions
stay below 16384, so the query factor is 1 throughout the turns; the prompt
itself crosses 16384 at its last chunk.

--layers 2 --turns 1 --decode 8 writes the call-by-call fixture
(long_c17920_2layer.json): for every call the SHA-256 of its 131072 logits'
bytes, the selected id and the logit range, so the GPU's precise path can be
checked bit for bit and the matrix-core path against it.
--layers 26 --turns 8 --decode 128 writes the token-stream fixture of the
benchmark's long workload (long_c17920_26layer.json): every selected id of
every turn with its top-2 logit gap.

Usage: python tests/golden/make_long_golden.py --layers 2 --turns 1 --decode 8
       python tests/golden/make_long_golden.py --layers 26 --turns 8 --decode 128
Runtime on 8 host threads: about 3 minutes (2 layers) and 40 minutes (26).
"""
import argparse
import ctypes
import hashlib
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

CONTEXT, PROMPT, CHUNK, KEEP, APPEND = 17920, 16384, 256, 15872, 64


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


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--seed", type=int, default=20251201)
    p.add_argument("--layers", type=int, default=2)
    p.add_argument("--turns", type=int, default=1)
    p.add_argument("--decode", type=int, default=8)
    p.add_argument("--threads", type=int, default=min(8, os.cpu_count() or 1))
    p.add_argument("--out")
    args = p.parse_args()
    out = args.out or os.path.join(HERE, "long_c17920_%dlayer.json" % args.layers)

    def log(msg):
        print(msg, file=sys.stderr, flush=True)

    oracle_lib.load().orc_set_threads(args.threads)
    t0 = time.time()
    layers = [syn.layer(args.seed, i) for i in range(args.layers)]
    model = oracle_lib.HostModel(syn.embedding(args.seed).reshape(-1), syn.final_norm(args.seed),
                                 layers, CONTEXT)
    prompt = syn.tokens(args.seed, 2, PROMPT)
    log("model ready in %.1f s" % (time.time() - t0))
    calls = []
    length, checkpoint = 0, None
    for begin in range(0, PROMPT, CHUNK):
        logits = model.forward(oracle_lib.MIRROR, prompt[begin:begin + CHUNK], length)
        length += CHUNK
        calls.append(dict(kind="prefill" if begin == 0 else "append", length=length,
                          **record(logits)))
        if length == KEEP:
            checkpoint = logits.copy()
        log("  prompt %d/%d (%.0f s)" % (length, PROMPT, time.time() - t0))
    turns = []
    for turn in range(args.turns):
        length = KEEP
        logits = checkpoint
        calls.append(dict(kind="restore", length=length, **record(logits)))
        ids = syn.tokens(args.seed, 100 + turn, APPEND)
        logits = model.forward(oracle_lib.MIRROR, ids, length)
        length += APPEND
        calls.append(dict(kind="append", length=length, **record(logits)))
        tokens, gaps = [calls[-1]["token"]], [calls[-1]["gap"]]
        for _ in range(args.decode):
            logits = model.forward(oracle_lib.MIRROR, [tokens[-1]], length)
            length += 1
            r = record(logits)
            calls.append(dict(kind="decode", length=length, **r))
            tokens.append(r["token"])
            gaps.append(r["gap"])
        turns.append({"append_ids_first": [int(t) for t in ids[:4]], "tokens": tokens,
                      "gaps": gaps})
        log("  turn %d: %d tokens (%.0f s)" % (turn, len(tokens), time.time() - t0))
    result = {"seed": args.seed, "layers": args.layers, "context": CONTEXT, "block": CHUNK,
              "prompt": PROMPT, "prompt_first": [int(t) for t in prompt[:8]], "keep": KEEP,
              "append": APPEND, "decode": args.decode, "schedule": "mirror", "turns": turns}
    if args.layers <= 4:
        result["calls"] = calls
    with open(out, "w") as f:
        json.dump(result, f)
    log("wrote %s in %.0f s" % (out, time.time() - t0))


if __name__ == "__main__":
    main()
