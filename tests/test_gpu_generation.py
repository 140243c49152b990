"""The generation loop (lunelette_generate_with_logits) driving the gfx950
runtime, with the callback the reference's CLI uses (src/main.c:43-67): the
first call prefills the whole prompt, every later call decodes the last id of
the prefix it is handed. On a seeded 2-layer model at C256 (precise and
matrix-core prefill) the generated ids equal a direct prefill + greedy decode
driver's, and the loop stops for the budget, for EOS (an id the direct stream
produces) and for the 256-token context, each with the reference's precedence
and without a callback past the stop.
"""
import ctypes

import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import synthetic as syn
from lunelette_amd.runtime import Runtime

pytestmark = pytest.mark.gpu
SEED = 77001


class RuntimeCallback:
    def __init__(self, rt):
        self.rt, self.started, self.calls = rt, False, 0
        lib, handle = rt._lib, rt.handle
        logits = lh.c_float_p()

        def next_logits(_ctx, ids, count, output, error, capacity):
            self.calls += 1
            if not self.started:
                rc = lib.lunelette_metal_prefill(handle, ids, count, ctypes.byref(logits),
                                                 error, capacity)
            else:
                rc = lib.lunelette_metal_decode(handle, ids[count - 1], ctypes.byref(logits),
                                                error, capacity)
            if rc:
                return -1
            self.started = True
            ctypes.memmove(output, logits, 131072 * 4)
            return 0

        self.fn = lh.LOGITS_FN(next_logits)


def generate(rt, prompt, budget, eos):
    rt.reset()
    callback = RuntimeCallback(rt)
    cfg = lh.GenerationConfig(budget, eos)
    result = lh.GenerationResult()
    err = ctypes.create_string_buffer(256)
    ids = (ctypes.c_int64 * len(prompt))(*[int(t) for t in prompt])
    rc = rt._lib.lunelette_generate_with_logits(callback.fn, None, ids, len(prompt),
                                                ctypes.byref(cfg), ctypes.byref(result), err,
                                                256)
    assert rc == 0, err.value
    return list(result.tokens[:result.count]), result.stop, callback.calls


def direct(rt, prompt, n):
    rt.reset()
    rt.prefill(prompt)
    tokens = [rt.greedy()]
    while len(tokens) < n:
        rt.decode(tokens[-1])
        tokens.append(rt.greedy())
    return tokens


@pytest.mark.parametrize("mode", [lh.PREFILL_CUSTOM, lh.PREFILL_MPS], ids=["precise", "mps"])
def test_generation_loop_over_runtime(gpu, mode):
    with Runtime(seed=SEED, layers=2, context=256, block=256, prefill=mode) as rt:
        prompt = syn.tokens(SEED, 1, 20)
        want = direct(rt, prompt, 12)
        eos_free = max(set(range(131072)) - set(want[:12]))
        tokens, stop, calls = generate(rt, prompt, 12, eos_free)
        assert tokens == want and stop == 0 and calls == 12          # budget
        eos = want[4]
        first = want.index(eos)
        tokens, stop, calls = generate(rt, prompt, 12, eos)
        assert tokens == want[:first + 1] and stop == 1 and calls == first + 1   # EOS
        long_prompt = syn.tokens(SEED, 2, 250)
        want_long = direct(rt, long_prompt, 6)
        tokens, stop, calls = generate(rt, long_prompt, 12, eos_free)
        assert tokens == want_long and stop == 2 and calls == 6      # context 256
        tokens, stop, calls = generate(rt, long_prompt, 6, eos_free)
        assert tokens == want_long and stop == 0 and calls == 6      # budget beats context
