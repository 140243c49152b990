"""Seeded random call sequences against the include/metal.h state machine.

A host model of the context (the tokens it holds, the valid flag, the
endpoint-logits flag, the active checkpoint and its epoch) predicts, for every
call, whether it is accepted (src/metal_runtime.m:349-432 for execution,
:494-564 for checkpoints, :333-347 for reset) and what it leaves behind. Each
accepted prefill, append or decode must return bitwise the logits of a fresh
context given the same tokens in one prefill call, on the bit-exact path
(PREFILL_CUSTOM; prefill == decode chain == append is pinned in
test_gpu_runtime.py); each restore the logits saved at checkpoint time. On the
matrix-core path (PREFILL_MPS) a multi-token call's rounding depends on how the
tokens were chunked, so there the logits must agree with the fresh context
within 1e-3 of its logit range (and restores stay bitwise). Every
rejected call must leave the state as it was, which the next calls check.
The sequences mix in the reference's argument errors: decode or append on an
empty context, prefill on a non-empty one, token ids out of range, counts over
the block or the remaining context, and restores of checkpoints that are no
longer active.
"""
import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd.runtime import Runtime, RuntimeError_

pytestmark = pytest.mark.gpu

SEED = 424242
LAYERS = 2
CONTEXT = 256
BLOCK = 256
VOCAB = 131072


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


class Model:
    """What the context should hold after each call."""

    def __init__(self):
        self.tokens = []
        self.valid = True
        self.endpoint = False
        self.active = None        # handle of the active checkpoint
        self.saved = {}           # handle -> (tokens, logits)


def expect_reject(call):
    with pytest.raises(RuntimeError_):
        call()


MPS_TOL = 1e-3


@pytest.fixture(scope="module", params=[lh.PREFILL_CUSTOM, lh.PREFILL_MPS],
                ids=["precise", "mps"])
def runtimes(gpu, request):
    subject = Runtime(seed=SEED, layers=LAYERS, context=CONTEXT, block=BLOCK,
                      prefill=request.param)
    replay = Runtime(seed=SEED, layers=LAYERS, context=CONTEXT, block=BLOCK,
                     prefill=request.param)
    yield subject, replay, request.param == lh.PREFILL_CUSTOM
    subject.close()
    replay.close()


def agree(got, want, exact):
    if exact:
        return np.array_equal(bits(got), bits(want))
    return float(np.max(np.abs(got - want))) <= MPS_TOL * float(np.ptp(want))


def fresh_logits(replay, tokens, cache):
    key = tuple(tokens)
    if key not in cache:
        replay.reset()
        cache[key] = replay.prefill(np.array(tokens, np.int64))
    return cache[key]


@pytest.mark.parametrize("seed", [1, 2, 3, 4, 5])
def test_random_call_sequences(runtimes, seed):
    rt, replay, exact = runtimes
    rng = np.random.default_rng(seed)
    cache = {}
    m = Model()
    rt.reset()
    counts = {"accepted": 0, "rejected": 0, "restored": 0}
    last = None
    for step in range(120):
        op = rng.choice(["prefill", "append", "decode", "checkpoint", "restore", "destroy",
                         "reset", "bad_id", "too_long"],
                        p=[0.14, 0.18, 0.26, 0.1, 0.1, 0.04, 0.06, 0.06, 0.06])
        room = CONTEXT - len(m.tokens)
        where = (seed, step, op, len(m.tokens))
        if op == "reset":
            rt.reset()
            m.tokens, m.valid, m.endpoint, m.active = [], True, False, None
            last = None
            continue
        if op in ("prefill", "append", "decode"):
            n = 1 if op == "decode" else int(rng.integers(1, 33))
            ids = [int(v) for v in rng.integers(0, VOCAB, size=n)]
            ok = m.valid and n <= room and (len(m.tokens) == 0) == (op == "prefill")
            call = {"prefill": lambda: rt.prefill(np.array(ids, np.int64)),
                    "append": lambda: rt.append(np.array(ids, np.int64)),
                    "decode": lambda: rt.decode(ids[0])}[op]
            if not ok:
                expect_reject(call)
                counts["rejected"] += 1
                continue
            got = call()
            last = got
            m.tokens += ids
            m.endpoint = True
            assert agree(got, fresh_logits(replay, m.tokens, cache), exact), where
            counts["accepted"] += 1
        elif op == "bad_id":
            bad = int(rng.choice([-1, VOCAB, VOCAB + 7, -(1 << 40)]))
            if len(m.tokens) == 0:
                expect_reject(lambda: rt.prefill(np.array([3, bad], np.int64)))
            else:
                expect_reject(lambda: rt.decode(bad))
            counts["rejected"] += 1
        elif op == "too_long":
            n = room + 1 if room < BLOCK else BLOCK + 1
            ids = np.zeros(n, np.int64)
            if len(m.tokens) == 0:
                expect_reject(lambda: rt.prefill(ids))
            else:
                expect_reject(lambda: rt.append(ids))
            counts["rejected"] += 1
        elif op == "checkpoint":
            ok = m.valid and m.endpoint and len(m.tokens) > 0
            if not ok:
                expect_reject(rt.checkpoint)
                counts["rejected"] += 1
                continue
            handle = rt.checkpoint()
            m.active = handle
            # The checkpoint keeps the endpoint logits the context returned.
            m.saved[handle] = (list(m.tokens), last)
        elif op == "restore":
            if not m.saved:
                continue
            handle = list(m.saved)[int(rng.integers(0, len(m.saved)))]
            saved_tokens, saved_logits = m.saved[handle]
            ok = (handle == m.active and m.valid and len(saved_tokens) <= len(m.tokens))
            if not ok:
                expect_reject(lambda: rt.restore(handle))
                counts["rejected"] += 1
                continue
            got = rt.restore(handle)
            last = got
            assert np.array_equal(bits(got), bits(saved_logits)), where
            m.tokens = list(saved_tokens)
            m.endpoint = True
            counts["restored"] += 1
        elif op == "destroy":
            if not m.saved:
                continue
            handle = list(m.saved)[int(rng.integers(0, len(m.saved)))]
            rt.destroy_checkpoint(handle)
            del m.saved[handle]
            if m.active == handle:
                m.active = None
    # The context still extends from whatever the sequence left.
    if m.valid and m.tokens and len(m.tokens) < CONTEXT:
        got = rt.decode(5)
        m.tokens.append(5)
        assert agree(got, fresh_logits(replay, m.tokens, cache), exact)
    for handle in list(m.saved):
        rt.destroy_checkpoint(handle)
    assert counts["accepted"] >= 10 and counts["rejected"] >= 5, counts
