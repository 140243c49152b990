"""Native logit regression (LUN2) over the gfx950 runtime.

The reference's runner (tests/compare_native.c:348-450) captures, for prompts
of 6, 24, 150 and 248 ids, the logits after the prefill and after seven
teacher-forced decodes, and checks them later in two reset cycles with the
strict rule (finite, bitwise, same top-1/5/20/64). Its prompt fixtures are
external, so seeded ids stand in. Checked here on a 4-layer synthetic model
at C256/B256:
- capture then check on the same context and on a second context: accepted,
  all 16 checked vectors exact;
- the resident FP32 and compact arithmetic strategies capture bitwise equal
  vectors (the reference's cross-strategy invariant), and each artifact
  names its own strategy;
- a capture of the precise prefill (custom) checked on an MPS context fails
  at step 0, where the matrix-core prefill rounds differently.
"""
import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import artifacts as art
from lunelette_amd import synthetic as syn
from lunelette_amd.runtime import Runtime

pytestmark = pytest.mark.gpu
SEED = 20251203
COUNTS = (6, 24, 150, 248)


def trajectories(strategy, mode):
    out = []
    for k, count in enumerate(COUNTS):
        prompt = syn.tokens(SEED, 10 + k, count).tolist()
        forced = [1000 + int(t) % (lh.VOCAB - 1000) for t in syn.tokens(SEED, 20 + k, 8)]
        out.append(art.trajectory(prompt, forced, strategy, mode))
    return out


def runtime(strategy, prefill):
    return Runtime(seed=SEED, layers=4, context=256, block=256, prefill=prefill, strategy=strategy)


@pytest.mark.parametrize("prefill", [lh.PREFILL_CUSTOM, lh.PREFILL_MPS])
def test_capture_then_check(gpu, tmp_path, prefill):
    strategy = lh.COMPACT_FP8_ARITHMETIC
    paths = [tmp_path / ("prefill%d.bin" % c) for c in COUNTS]
    with runtime(strategy, prefill) as rt:
        for path, t in zip(paths, trajectories(strategy, prefill)):
            ok, _, error = art.run(rt, path, t, check=False)
            assert ok, error
            ok, metrics, error = art.run(rt, path, t, check=True)
            assert ok, error
            assert all(m["exact"] and m["top64"] == 64 for m in metrics)
            ok, _, error = art.run(rt, path, t, check=False)
            assert not ok                                    # never overwrites
    with runtime(strategy, prefill) as second:
        for path, t in zip(paths, trajectories(strategy, prefill)):
            ok, _, error = art.run(second, path, t, check=True)
            assert ok, error
            accepted, _, error = art.compare_files(path, path, prefill, t.count, strategy)
            assert accepted, error


def test_strategies_capture_equal_vectors(gpu, tmp_path):
    vectors = {}
    for strategy in (lh.RESIDENT_FP32, lh.COMPACT_FP8_ARITHMETIC):
        t = trajectories(strategy, lh.PREFILL_CUSTOM)[1]
        path = tmp_path / ("s%d.bin" % strategy)
        with runtime(strategy, lh.PREFILL_CUSTOM) as rt:
            ok, _, error = art.run(rt, path, t, check=False)
            assert ok, error
            wrong = trajectories(1 - strategy, lh.PREFILL_CUSTOM)[1]
            ok, _, error = art.run(rt, tmp_path / "other.bin", wrong, check=False)
            assert not ok and "strategy" in error             # the runtime's own strategy
        vectors[strategy] = art.read(path, t)
    assert np.array_equal(vectors[0].view(np.uint32), vectors[1].view(np.uint32))
    accepted, _, _ = art.compare_files(tmp_path / "s0.bin", tmp_path / "s1.bin",
                                       lh.PREFILL_CUSTOM, COUNTS[1], lh.RESIDENT_FP32)
    assert not accepted                                       # strategies never cross-accept


def test_precise_capture_fails_on_mps_context(gpu, tmp_path):
    strategy = lh.COMPACT_FP8_ARITHMETIC
    t = trajectories(strategy, lh.PREFILL_CUSTOM)[2]
    path = tmp_path / "custom.bin"
    with runtime(strategy, lh.PREFILL_CUSTOM) as rt:
        ok, _, error = art.run(rt, path, t, check=False)
        assert ok, error
    with runtime(strategy, lh.PREFILL_MPS) as mps:
        ok, metrics, error = art.run(mps, path, t, check=True)
        assert not ok and "cycle 0 step 0 differs" in error
        m = metrics[0]
        assert not m["exact"] and m["max_abs"] > 0
