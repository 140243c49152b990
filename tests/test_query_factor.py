"""The query factor at positions >= 16384 through the shipped kernels.

src/metal_kernels.metal:72-76 and src/metal_encode.m:137-140 multiply the
rotated Q (never K) by 1 + 0.1 ln(1 + floor(p / 16384)), which is exactly 1
below 16384 and 1 + 0.1 ln 2 from 16384 to 32767. The 17920 capacity profile
admits positions up to 17919, so every path that forms Q must apply it there:
- the fused decode epilogue of k_qkv_rope (PATH_FUSED, PATH_LOOKUP,
  PATH_RESIDENT) and the unfused rope-append (PATH_UNFUSED): one decode token
  at positions 16383, 16384, 16385 and 17919; layer output and the appended K
  and V rows bit for bit equal to the oracle's mirror schedule, the
  reference-literal schedule within the layer tolerance;
- the matrix-core epilogue (PATH_MFMA): a 128-token chunk at 16320 (straddling
  16384) and a 256-token chunk at 17664 (up to 17919), within the tolerance
  of the matrix-core layer after a 4096-token prefix;
- the runtime: a 2-layer model decoding from 16300 to 16448, then an append
  of 200 tokens at 16300 and 4 decodes (tests/golden/make_qfactor_golden.py):
  precise logits bit for bit equal to the oracle fixture per call, the
  matrix-core path within 1e-3 of each call's logit range.

In the layer cases the q and k scales are 2^-12 instead of the synthetic
[0.01, 0.02], so that scores have a standard deviation near 1.4 and the softmax
is soft: with the synthetic scales the scores' deviation is near 7e3, the
softmax is one-hot and scaling Q by 1.07 rarely changes a head's output.
The CPU tests below show that each layer case separates the oracle from two
planted variants (orc_model.c with -DORC_PLANT=3, the factor on K instead of
Q, and -DORC_PLANT=8, the factor dropped) at and past 16384, bitwise and by
more than ten times the matrix-core tolerance, and that the variants agree
with it at 16383; and that both variants move most of the runtime fixture's
calls past 16384 bit for bit, the largest by more than twice the matrix-core
tolerance. So the GPU tests cannot pass with either mistake.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import synthetic as syn
from lunelette_amd.runtime import Runtime

import oracle_lib
from oracle_lib import MIRROR, REF

SEED = 20251201
CAPACITY = 17920
DECODE_LENGTHS = (16383, 16384, 16385, 17919)
CHUNKS = ((16320, 128), (17664, 256))
MFMA_TOL = 1e-3
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "qfactor_c17920_2layer.json")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def soft_host():
    host = dict(syn.layer(SEED, 0))
    host["scale_q"] = host["scale_k"] = 2.0 ** -12
    return host


def inputs(length, count):
    x = syn.normal_f32(SEED, 9201, count * 3072)
    kpm = syn.normal_f32(SEED, 9202, length * 1024).reshape(length, 1024)
    vpm = syn.normal_f32(SEED, 9203, length * 1024).reshape(length, 1024)
    return x, kpm, vpm


def oracle_case(host, length, count, schedule=MIRROR, lib=None):
    """(x out, appended K rows, appended V rows) of one layer on the oracle."""
    x, kpm, vpm = inputs(length, count)
    model = oracle_lib.HostModel(np.zeros(1, np.uint16), np.zeros(1, np.uint16), [host],
                                 CAPACITY, lib=lib)
    kv = model.keys.reshape(8, CAPACITY, 128)
    kv[:, :length] = kpm.reshape(length, 8, 128).transpose(1, 0, 2)
    vv = model.values.reshape(8, CAPACITY, 128)
    vv[:, :length] = vpm.reshape(length, 8, 128).transpose(1, 0, 2)
    xo = np.array(x, np.float32)
    model.layer_forward(schedule, 0, xo, length, count)
    return xo, model.kv(0, 0, length, count), model.kv(0, 1, length, count)


def rel_rowmax(got, want, width):
    g, w = got.reshape(-1, width), want.reshape(-1, width)
    return float(np.max(np.abs(g - w) / np.max(np.abs(w), axis=1, keepdims=True)))


# ---- CPU: the cases separate the planted mistakes -------------------------

@pytest.fixture(scope="module")
def planted(tmp_path_factory):
    return oracle_lib.build_planted((3, 8), tmp_path_factory.mktemp("qfactor_plants"))


def test_query_factor_closed_form():
    o = oracle_lib.load()
    for p in (0, 16383):
        assert o.orc_query_factor(p) == 1.0
    want = np.float32(1.0 + 0.1 * np.log(2.0))
    for p in (16384, 16385, 17919, 32767):
        assert abs(o.orc_query_factor(p) - want) <= 1e-7


@pytest.mark.parametrize("length", DECODE_LENGTHS)
def test_decode_cases_separate_plants(soft_host, planted, length):
    want = oracle_case(soft_host, length, 1)
    for n, lib in planted.items():
        got = oracle_case(soft_host, length, 1, lib=lib)
        same = all(np.array_equal(bits(a), bits(b)) for a, b in zip(got, want))
        if length < 16384:
            assert same, "plant %d changed a result at %d, where the factor is 1" % (n, length)
        else:
            assert not np.array_equal(bits(got[0]), bits(want[0])), (n, length)
            assert rel_rowmax(got[0], want[0], 3072) > 10 * MFMA_TOL, (n, length)
    # The factor on K changes the appended K row itself.
    k3 = oracle_case(soft_host, length, 1, lib=planted[3])[1]
    assert np.array_equal(bits(k3), bits(want[1])) == (length < 16384)


@pytest.mark.parametrize("length,count", CHUNKS)
def test_chunk_cases_separate_plants(soft_host, planted, length, count):
    want = oracle_case(soft_host, length, count)
    for n, lib in planted.items():
        got = oracle_case(soft_host, length, count, lib=lib)
        assert rel_rowmax(got[0], want[0], 3072) > 10 * MFMA_TOL, n


def test_runtime_fixture_separates_plants():
    """The synthetic model's scales make most softmax rows one-hot, where
    scaling Q by 1.07 changes nothing; the factor still moves the logits of
    most calls past 16384. Measured: 49 (factor on K) and 46 (factor dropped)
    of the 69 calls differ bit for bit, by up to 0.28 and 3.4e-3 of the logit
    range; no call before 16384 differs."""
    with open(GOLDEN) as f:
        fx = json.load(f)
    calls = fx["calls"][-(fx["decode"] + 2 + fx["tail"]):]
    past = [c["length"] + c["count"] > 16384 for c in calls]
    assert sum(past) == fx["decode"] - (16384 - fx["prompt"]) + 1 + fx["tail"]
    for n, plant in fx["plants"].items():
        for i, c in enumerate(calls):
            if not past[i]:
                assert plant["bitwise_equal"][i], (n, i)
        moved = sum(1 for i, p in enumerate(past) if p and not plant["bitwise_equal"][i])
        assert moved > sum(past) // 2, (n, moved)
        worst = max(e for e, p in zip(plant["max_err_over_range"], past) if p)
        assert worst > 2 * MFMA_TOL, (n, worst)


# ---- GPU: the shipped kernels ---------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("length", DECODE_LENGTHS)
def test_decode_layer_all_paths(gpu, soft_host, length):
    from test_gpu_layer import run_layer
    x, kpm, vpm = inputs(length, 1)
    mirror = oracle_case(soft_host, length, 1)
    for path in (lh.PATH_FUSED, lh.PATH_LOOKUP, lh.PATH_UNFUSED, lh.PATH_RESIDENT):
        got = run_layer(gpu, soft_host, x, kpm, vpm, length, 1, CAPACITY, path,
                        resident=path == lh.PATH_RESIDENT)
        for g, w, name in zip(got, mirror, ("x", "k", "v")):
            assert np.array_equal(bits(g), bits(w)), (path, length, name)
    ref = oracle_case(soft_host, length, 1, REF)
    assert rel_rowmax(got[0], ref[0], 3072) < 1e-3


@pytest.mark.gpu
def test_decode_layer_synthetic_scales(gpu):
    """The synthetic scales at the last admitted position, fused path."""
    from test_gpu_layer import run_layer
    host = syn.layer(SEED, 1)
    length = CAPACITY - 1
    x, kpm, vpm = inputs(length, 1)
    got = run_layer(gpu, host, x, kpm, vpm, length, 1, CAPACITY, lh.PATH_FUSED)
    for g, w, name in zip(got, oracle_case(host, length, 1), ("x", "k", "v")):
        assert np.array_equal(bits(g), bits(w)), name


@pytest.mark.gpu
@pytest.mark.parametrize("length,count", CHUNKS)
def test_mfma_chunk_across_16384(gpu, soft_host, length, count):
    from test_gpu_layer import run_layer
    x, kpm, vpm = inputs(length, count)
    got = run_layer(gpu, soft_host, x, kpm, vpm, length, count, CAPACITY, lh.PATH_MFMA)
    want = oracle_case(soft_host, length, count)
    err = rel_rowmax(got[0], want[0], 3072)
    print("mfma chunk %d+%d: layer output within %.3g of the row max" % (length, count, err))
    assert err < MFMA_TOL
    for g, w in zip(got[1:], want[1:]):
        assert rel_rowmax(g, w, 1024) < 1e-5
    # The precise path on the same chunk is the mirror bit for bit.
    got = run_layer(gpu, soft_host, x, kpm, vpm, length, count, CAPACITY, lh.PATH_FUSED)
    for g, w in zip(got, want):
        assert np.array_equal(bits(g), bits(w))


def run_fixture_workload(fx, prefill_mode, forced=None):
    """Yields (call index, logits, runtime) over the fixture's calls. Decodes
    feed the previous greedy id, or with forced the fixture's ids."""
    calls = fx["calls"]
    rt = Runtime(seed=fx["seed"], layers=fx["layers"], context=fx["context"], block=fx["block"],
                 prefill=prefill_mode)
    try:
        prompt = syn.tokens(fx["seed"], 3, fx["prompt"])
        assert [int(t) for t in prompt[:8]] == fx["prompt_first"]
        ids_append = syn.tokens(fx["seed"], 200, fx["append"])
        assert [int(t) for t in ids_append[:4]] == fx["append_first"]
        checkpoint = None
        for i, c in enumerate(calls):
            at, n = c["length"], c["count"]
            if c["kind"] == "prefill":
                logits = rt.prefill(prompt[at:at + n])
            elif c["kind"] == "append" and at < fx["prompt"]:
                logits = rt.append(prompt[at:at + n])
            elif c["kind"] == "append":
                logits = rt.append(ids_append)
            elif c["kind"] == "restore":
                logits = rt.restore(checkpoint)
            else:
                token = calls[i - 1]["token"] if forced else rt.greedy()
                logits = rt.decode(token)
            yield i, logits, rt
            if at + n == fx["prompt"] and checkpoint is None:
                checkpoint = rt.checkpoint()
        rt.destroy_checkpoint(checkpoint)
    finally:
        rt.close()


@pytest.mark.gpu
def test_runtime_decode_across_16384(gpu):
    with open(GOLDEN) as f:
        fx = json.load(f)
    calls = fx["calls"]
    precise = []
    for i, logits, rt in run_fixture_workload(fx, lh.PREFILL_CUSTOM):
        digest = hashlib.sha256(logits.tobytes()).hexdigest()
        assert digest == calls[i]["sha256"], "precise path differs from the oracle at call %d " \
            "(%s at %d)" % (i, calls[i]["kind"], calls[i]["length"])
        assert rt.greedy() == calls[i]["token"]
        precise.append(logits)
    assert len(precise) == len(calls)
    worst = 0.0
    for i, logits, rt in run_fixture_workload(fx, lh.PREFILL_MPS, forced=True):
        want = precise[i]
        err = float(np.max(np.abs(logits - want))) / float(want.max() - want.min())
        worst = max(worst, err)
        assert err <= MFMA_TOL, "call %d (%s at %d): %.3g" % (i, calls[i]["kind"],
                                                              calls[i]["length"], err)
        if calls[i]["gap"] > 2 * err * float(want.max() - want.min()):
            assert rt.greedy() == calls[i]["token"], "call %d" % i
    print("matrix-core path across 16384: worst logit error %.3g of the range" % worst)
