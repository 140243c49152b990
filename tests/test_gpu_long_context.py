"""Long-context prefix reuse at the 17920 capacity profile on the GPU.

The workload of the benchmark's long line: a 16384-token seeded prompt
prefilled in 256-token chunks with a checkpoint at 15872, then turns that
restore the 15872-token prefix, append 64 ids and decode greedily. The
reference's own planner stops at 4352 (src/metal_plan.h:39-41) and its long
schedules at 4352 (tests/long_context/long/schedule.py:11-47), so this profile
is pinned by the oracle alone, through fixtures written offline by
tests/golden/make_long_golden.py (device-mirror schedule):
- matrix-core attention against the oracle at 8192- and 16128-token prefixes
  with 64 and 256 query rows (the KV-split launches of 16 and 4 splits), to
  the 2e-4 tolerance of the shorter cases;
- a 2-layer model through every call of the workload (64 prompt chunks,
  restore, append 64, 8 decodes): the precise path's logits equal the
  fixture's bit for bit (SHA-256 per call); the matrix-core path's logits stay
  within 1e-3 of each call's logit range of them and select the same ids;
- the 26-layer benchmark workload (8 turns of append 64 + 128 decodes): the
  precise path selects the fixture's 8 x 129 ids. The matrix-core path runs
  the same workload in lockstep with the precise path, both fed the fixture's
  ids (so one near-tie cannot change every later context): its logits stay
  within MPS_TOL (5e-3) of each call's logit range of the precise path's, the
  median over the calls within MPS_MEDIAN_TOL (5e-4), and it selects the
  fixture's id wherever the precise top-2 gap exceeds twice its largest logit
  error there (no id can flip otherwise). Over the 1104 calls the largest
  error measured on MI355X is 2.7e-3 of the range and the median about
  1.2e-4, with no id flipped (builds with another prefill summation order
  flipped two of the 1032, both at gaps below twice the error). The bound is
  looser than the 1e-3 of the 2-layer and 4352-context workloads because after a
  16K-token matrix-core prefill the 26-layer stack amplifies the prefill's
  rounding through near-tie softmax rows; those errors move no selected id.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import synthetic as syn
from lunelette_amd.runtime import Runtime

import gpu_util
import oracle_lib
from oracle_lib import MIRROR

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CONTEXT = 17920


def fixture(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.skip("fixture %s not generated (tests/golden/make_long_golden.py)" % name)
    with open(path) as f:
        return json.load(f)


@pytest.mark.parametrize("length,count", [(8192, 64), (8192, 256), (16128, 64), (16128, 256)])
def test_attention_mfma_long_prefix(gpu, length, count):
    rng = np.random.default_rng(length + count)
    total = length + count
    q = (rng.normal(size=count * 4096) * 3).astype(np.float32)
    kpm = rng.normal(size=(total, 1024)).astype(np.float32)
    vpm = rng.normal(size=(total, 1024)).astype(np.float32)
    got = gpu_util.attention_on_device(gpu, gpu.lh_attention_mfma, q, kpm, vpm, length, count,
                                       CONTEXT)
    want = oracle_lib.attention(MIRROR, q, kpm.reshape(-1), vpm.reshape(-1), 128, 1024, length,
                                count)
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - want)) < 2e-4


MPS_TOL = 5e-3
MPS_MEDIAN_TOL = 5e-4


def run_workload(fx, prefill_mode, turns, forced=None):
    """Yields (kind, logits, runtime) for every call of the fixture's
    workload. Decodes feed the previous greedy id, or with forced (one id list
    per turn) the turn's listed ids in order."""
    rt = Runtime(seed=fx["seed"], layers=fx["layers"], context=fx["context"], block=fx["block"],
                 prefill=prefill_mode)
    try:
        prompt = syn.tokens(fx["seed"], 2, fx["prompt"])
        assert [int(t) for t in prompt[:8]] == fx["prompt_first"]
        checkpoint = None
        for begin in range(0, fx["prompt"], fx["block"]):
            ids = prompt[begin:begin + fx["block"]]
            logits = rt.prefill(ids) if begin == 0 else rt.append(ids)
            yield ("prefill" if begin == 0 else "append"), logits, rt
            if begin + fx["block"] == fx["keep"]:
                checkpoint = rt.checkpoint()
        for turn in range(turns):
            yield "restore", rt.restore(checkpoint), rt
            ids = syn.tokens(fx["seed"], 100 + turn, fx["append"])
            yield "append", rt.append(ids), rt
            for k in range(fx["decode"]):
                token = rt.greedy() if forced is None else forced[turn][k]
                yield "decode", rt.decode(token), rt
        rt.destroy_checkpoint(checkpoint)
    finally:
        rt.close()


def test_long_reuse_2layer_calls(gpu):
    fx = fixture("long_c17920_2layer.json")
    calls = fx["calls"]
    precise = []
    for i, (kind, logits, rt) in enumerate(run_workload(fx, lh.PREFILL_CUSTOM, 1)):
        assert kind == calls[i]["kind"]
        digest = hashlib.sha256(logits.tobytes()).hexdigest()
        assert digest == calls[i]["sha256"], "precise path differs from the oracle at call %d" % i
        assert rt.greedy() == calls[i]["token"]
        precise.append(logits)
    assert len(precise) == len(calls)
    for i, (kind, logits, rt) in enumerate(run_workload(fx, lh.PREFILL_MPS, 1)):
        want = precise[i]
        span = float(want.max() - want.min())
        assert np.max(np.abs(logits - want)) <= 1e-3 * span, "call %d (%s)" % (i, kind)
        assert rt.greedy() == calls[i]["token"], "call %d (%s)" % (i, kind)


def expected_stream(fx):
    """Every id selected in the turns: the append's, then each decode's."""
    return [t for turn in fx["turns"] for t in turn["tokens"]]


def test_long_reuse_26layer_stream(gpu):
    fx = fixture("long_c17920_26layer.json")
    got = []
    in_turns = False
    for kind, _, rt in run_workload(fx, lh.PREFILL_CUSTOM, len(fx["turns"])):
        in_turns = in_turns or kind == "restore"
        if in_turns and kind in ("append", "decode"):
            got.append(rt.greedy())
    want = expected_stream(fx)
    first = next((i for i in range(len(want)) if i >= len(got) or got[i] != want[i]), None)
    print("long stream: %d/%d ids equal the oracle's" % (
        len(want) if first is None else first, len(want)))
    assert first is None, "first differing id at %d (top-2 gap there %.4g)" % (
        first, [g for turn in fx["turns"] for g in turn["gaps"]][first])


def test_long_reuse_26layer_mps_lockstep(gpu):
    fx = fixture("long_c17920_26layer.json")
    forced = [turn["tokens"] for turn in fx["turns"]]
    want = expected_stream(fx)
    turns = len(fx["turns"])
    worst, flips, selected, in_turns = 0.0, [], 0, False
    by_kind = {}
    for call, ((kind, ref, rt_p), (kind_m, logits, rt_m)) in enumerate(zip(
            run_workload(fx, lh.PREFILL_CUSTOM, turns, forced),
            run_workload(fx, lh.PREFILL_MPS, turns, forced))):
        assert kind == kind_m
        span = float(ref.max() - ref.min())
        err = float(np.max(np.abs(logits - ref)))
        worst = max(worst, err / span)
        by_kind.setdefault(kind, []).append(err / span)
        assert err <= MPS_TOL * span, "call %d (%s): error %.3g of range %.3g" % (
            call, kind, err, span)
        in_turns = in_turns or kind == "restore"
        if in_turns and kind in ("append", "decode"):
            assert rt_p.greedy() == want[selected]
            top2 = np.partition(ref, -2)[-2:]
            gap = float(top2[1] - top2[0])
            if rt_m.greedy() != want[selected]:
                flips.append(selected)
                assert 2 * err >= gap, "id %d flipped at gap %.4g, error %.4g" % (
                    selected, gap, err)
            selected += 1
    assert selected == len(want)
    errors = [e for v in by_kind.values() for e in v]
    print("mps lockstep: %d calls, largest error %.3g of the logit range (median %.3g), "
          "%d near-tie flips %s" % (call + 1, worst, float(np.median(errors)), len(flips), flips))
    assert float(np.median(errors)) <= MPS_MEDIAN_TOL
    print("mps lockstep errors by kind:", {k: (max(v), float(np.median(v))) for k, v in by_kind.items()})
