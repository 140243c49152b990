"""Greedy token streams of the full 26-layer model on the GPU.

Workload: the random-init 26-layer Ministral-3B-shaped FP8 model, context
4352, a 512-token seeded prompt prefilled in two 256-token chunks, then greedy
decode (the bench workload). The fixture tests/golden/stream_c4352_26layer.json
holds the CPU oracle's streams (tests/golden/make_stream_golden.py):
- the precise path (PREFILL_CUSTOM + decode) must reproduce the oracle's
  device-mirror stream token for token (it is bit-exact per step);
- the precise stream must also agree with the reference-literal stream up to
  the fixture's first divergence between the two oracle schedules (None: the
  two schedules select the same 1024 tokens for this seed, so the GPU stream
  equals the reference-literal one throughout);
- the MPS path (matrix-core prefill, tolerance-equal logits, then the
  bit-exact decode kernels over the KV cache it wrote) must select the same
  tokens up to the first step where the oracle's own top-2 logit gap is within
  twice the MPS path's logit error there: its KV cache differs from the
  oracle's by rounding, which can flip a near-tie and no other step. At a
  divergence the two paths rerun in lockstep, both fed the fixture's ids,
  which checks every step up to it: the MPS logits within 1e-3 of the logit
  range of the precise path's, and the flip at a gap below twice that error.
  (For this seed step 172 is such a near-tie: the oracle's top-2 gap there is
  4.0e-5 of the logit range, 3.7e-4 absolute; the summation order of the
  matrix-core prefill decides which side of it the MPS stream lands on.)
- over all 1024 calls in lockstep (both paths fed the fixture's ids), the MPS
  path's largest logit error stays within twice what a different exact FP32
  summation order does on the same calls (the oracle's reference-literal
  schedule against its mirror schedule,
  tests/golden/schedule_envelope_c4352_26layer.json, written by
  tests/golden/make_schedule_envelope.py) and within MPS_TOL (5e-3) of each
  call's logit range, its median within MPS_MEDIAN_TOL (5e-4), and the two
  paths select the same id wherever the precise top-2 gap exceeds twice the
  MPS error there. This model's near-one-hot softmax turns rounding-level
  differences into logit errors of a few 1e-3 of the range at a handful of
  calls whichever exact schedule is used, so 1e-3 bounds the typical call,
  not every call.
"""
import json
import os

import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import synthetic as syn
from lunelette_amd.runtime import Runtime

pytestmark = pytest.mark.gpu
FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                       "stream_c4352_26layer.json")
ENVELOPE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                        "schedule_envelope_c4352_26layer.json")
MPS_TOL = 5e-3
MPS_MEDIAN_TOL = 5e-4


def fixture():
    if not os.path.exists(FIXTURE):
        pytest.skip("stream fixture not generated (tests/golden/make_stream_golden.py)")
    with open(FIXTURE) as f:
        return json.load(f)


def run_stream(fx, prefill_mode):
    rt = Runtime(seed=fx["seed"], layers=fx["layers"], context=fx["context"], block=256,
                 prefill=prefill_mode)
    try:
        prompt = syn.tokens(fx["seed"], 1, fx["prompt"])
        assert [int(t) for t in prompt[:8]] == fx["prompt_sha_first"]
        chunk = fx["chunk"]
        rt.prefill(prompt[:chunk], copy=False)
        for begin in range(chunk, fx["prompt"], chunk):
            rt.append(prompt[begin:begin + chunk], copy=False)
        tokens = [rt.greedy()]
        for _ in range(fx["decode"] - 1):
            rt.decode(tokens[-1], copy=False)
            tokens.append(rt.greedy())
        return tokens
    finally:
        rt.close()


def agreement(a, b):
    return next((i for i in range(min(len(a), len(b))) if a[i] != b[i]), min(len(a), len(b)))


def test_precise_stream_matches_oracle_mirror(gpu):
    fx = fixture()
    tokens = run_stream(fx, lh.PREFILL_CUSTOM)
    assert tokens == fx["tokens_mirror"], "first mismatch at %d" % agreement(
        tokens, fx["tokens_mirror"])
    ref_agree = agreement(tokens, fx["tokens_ref"])
    expected = fx["first_divergence"]
    assert ref_agree == (len(tokens) if expected is None else expected)
    print("precise stream: %d/%d tokens equal the mirror oracle; %d equal the "
          "reference-literal oracle" % (len(tokens), len(tokens), ref_agree))


def lockstep_logits(fx, prefill_mode, steps):
    """Logits of the prompt's last chunk and of `steps` - 1 decodes fed the
    fixture's ids, one call at a time."""
    rt = Runtime(seed=fx["seed"], layers=fx["layers"], context=fx["context"], block=256,
                 prefill=prefill_mode)
    try:
        prompt = syn.tokens(fx["seed"], 1, fx["prompt"])
        chunk = fx["chunk"]
        logits = rt.prefill(prompt[:chunk])
        for begin in range(chunk, fx["prompt"], chunk):
            logits = rt.append(prompt[begin:begin + chunk])
        yield logits
        for i in range(steps - 1):
            yield rt.decode(fx["tokens_mirror"][i])
    finally:
        rt.close()


def test_mps_stream_matches_oracle(gpu):
    fx = fixture()
    want = fx["tokens_mirror"]
    tokens = run_stream(fx, lh.PREFILL_MPS)
    n = agreement(tokens, want)
    print("MPS stream: first %d/%d tokens equal the mirror oracle" % (n, len(tokens)))
    assert len(tokens) == len(want)
    if n == len(want):
        return
    worst = 0.0
    for i, (ref, got) in enumerate(zip(lockstep_logits(fx, lh.PREFILL_CUSTOM, n + 1),
                                       lockstep_logits(fx, lh.PREFILL_MPS, n + 1))):
        span = float(ref.max() - ref.min())
        err = float(np.max(np.abs(got - ref)))
        worst = max(worst, err / span)
        assert err <= 1e-3 * span, "step %d: MPS logit error %.3g of range %.3g" % (i, err, span)
        assert int(np.argmax(ref)) == want[i], "precise path left the fixture at %d" % i
        if i == n:
            top2 = np.partition(ref, -2)[-2:]
            gap = float(top2[1] - top2[0])
            print("MPS stream: step %d is a near-tie: top-2 gap %.3g (%.3g of the range), "
                  "MPS logit error %.3g; largest error over steps 0..%d: %.3g of the range"
                  % (n, gap, gap / span, err, n, worst))
            assert 2 * err >= gap, "step %d flipped at gap %.4g, error %.4g" % (n, gap, err)


def test_mps_lockstep_within_schedule_envelope(gpu):
    fx = fixture()
    with open(ENVELOPE) as f:
        envelope = json.load(f)
    assert envelope["seed"] == fx["seed"] and envelope["calls"] == fx["decode"]
    want = fx["tokens_mirror"]
    errors = []
    for i, (ref, got) in enumerate(zip(lockstep_logits(fx, lh.PREFILL_CUSTOM, fx["decode"]),
                                       lockstep_logits(fx, lh.PREFILL_MPS, fx["decode"]))):
        span = float(ref.max() - ref.min())
        err = float(np.max(np.abs(got - ref)))
        errors.append(err / span)
        assert int(np.argmax(ref)) == want[i], "precise path left the fixture at %d" % i
        if int(np.argmax(got)) != want[i]:
            top2 = np.partition(ref, -2)[-2:]
            assert 2 * err >= float(top2[1] - top2[0]), "call %d flipped" % i
    worst, median = max(errors), float(np.median(errors))
    print("MPS lockstep over %d calls: largest %.3g (call %d), median %.3g of the logit range; "
          "two exact FP32 schedules differ by up to %.3g (median %.3g)" % (
              len(errors), worst, int(np.argmax(errors)), median,
              envelope["max_err_over_range"], envelope["median_err_over_range"]))
    assert len(errors) == fx["decode"]
    assert worst <= min(MPS_TOL, 2 * envelope["max_err_over_range"])
    assert median <= MPS_MEDIAN_TOL
