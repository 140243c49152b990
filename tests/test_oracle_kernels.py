"""Pins the oracle's kernels (both schedules) against double-precision brute
force and the reference's closed forms, the way the reference's own GPU
tests do:
- projection: 7x67x3 vs double, |err| < 1e-6 (tests/test_metal.m:169-198);
  all-ones inputs give exactly K (tests/test_metal_reference.m:124-129).
- RMSNorm / element: width 67, 2e-6 (tests/test_metal.m:490-530).
- attention: 2 rows over a 3-prefix vs double softmax, 2e-6
  (tests/test_metal.m:532-578); 4352-position causal sentinel 1.0 and
  8703/4352 with masked score 0 (tests/test_metal.m:956-999).
- RoPE: formula with the query factor, 2e-6 (tests/test_metal.m:605-626).
Planted-mistake checks show the comparisons catch a transposed operand or a
dropped term.
"""
import math

import numpy as np
import pytest

import oracle_lib
from oracle_lib import MIRROR, REF, W_BF16, W_F32, W_FP8

SCHEDULES = (REF, MIRROR)


def brute_dot(w, x):
    return (w.astype(np.float64) @ x.astype(np.float64))


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_projection_small_vs_double(schedule):
    rows, cols, tokens = 7, 67, 3
    w = np.array([((i % 19) - 9) * 0.03125 for i in range(rows * cols)], np.float32)
    x = np.array([((i % 13) - 6) * 0.0625 for i in range(tokens * cols)], np.float32)
    y = oracle_lib.matvec(schedule, W_F32, w, 1.0, x, rows, cols, tokens).reshape(tokens, rows)
    for t in range(tokens):
        expected = brute_dot(w.reshape(rows, cols), x[t * cols:(t + 1) * cols])
        assert np.max(np.abs(y[t] - expected)) < 1e-6


@pytest.mark.parametrize("schedule", SCHEDULES)
@pytest.mark.parametrize("cols", [1, 7, 31, 32, 33, 63, 65, 1023, 1024, 1025, 3072])
def test_all_ones_dot_is_exactly_k(schedule, cols):
    w = np.ones(cols, np.float32)
    x = np.ones(cols, np.float32)
    assert oracle_lib.matvec(schedule, W_F32, w, 1.0, x, 1, cols)[0] == cols
    # FP8 code 0x38 is 1.0; BF16 0x3f80 is 1.0.
    assert oracle_lib.matvec(schedule, W_FP8, np.full(cols, 0x38, np.uint8), 1.0, x, 1,
                             cols)[0] == cols
    assert oracle_lib.matvec(schedule, W_BF16, np.full(cols, 0x3f80, np.uint16), 1.0, x, 1,
                             cols)[0] == cols


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_fp8_matvec_vs_double_9216x3072(schedule, product):
    import lunelette_amd.synthetic as syn
    rows, cols, scale = 9216, 3072, 0.0125
    w = syn.fp8(11, 500, rows, cols)
    x = syn.normal_f32(11, 501, cols)
    dec = np.array([oracle_lib.load().orc_fp8_decode(c) for c in range(256)], np.float32)
    wf = (dec[w] * np.float32(scale)).astype(np.float32)
    y = oracle_lib.matvec(schedule, W_FP8, w, scale, x, rows, cols)
    expected = wf.astype(np.float64) @ x.astype(np.float64)
    magnitude = np.abs(wf).astype(np.float64) @ np.abs(x).astype(np.float64)
    assert np.all(np.abs(y - expected) <= 1e-6 * magnitude)
    # A transposed-index mistake would not survive this comparison.
    assert np.max(np.abs(y[::-1] - expected) / magnitude) > 1e-3


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_rmsnorm_vs_double(schedule):
    width, tokens = 67, 2
    gamma = np.array([0.5 + i * 0.001 for i in range(width)], np.float32)
    x = np.array([((i % 17) - 8) * 0.125 for i in range(width * tokens)], np.float32)
    out = oracle_lib.rmsnorm(schedule, gamma, x, width, tokens).reshape(tokens, width)
    xx = x.reshape(tokens, width).astype(np.float64)
    expected = gamma * xx / np.sqrt((xx * xx).sum(1, keepdims=True) / width + 1e-5)
    assert np.max(np.abs(out - expected)) < 2e-6
    # Planted mistake: dropping the epsilon term is visible at this size.
    wrong = gamma * xx / np.sqrt((xx * xx).sum(1, keepdims=True) / width)
    assert np.max(np.abs(wrong - expected)) > 2e-6


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_silu_mul_vs_double(schedule, oracle):
    n = 134
    g = np.array([((i % 17) - 8) * 0.125 for i in range(n)], np.float32)
    u = np.array([((i % 11) - 5) * 0.25 for i in range(n)], np.float32)
    out = np.empty(n, np.float32)
    oracle.orc_silu_mul(schedule, g.ctypes.data, u.ctypes.data, out.ctypes.data, n)
    gd = g.astype(np.float64)
    expected = gd / (1 + np.exp(-gd)) * u
    assert np.max(np.abs(out - expected)) < 2e-6


def test_rope_formula_with_query_factor(oracle):
    positions = [0, 1, 16383, 16384, 16385]
    width = 128
    x = np.array([((i % 23) - 11) * 0.125 for i in range(len(positions) * width)], np.float32)
    cos = np.empty((len(positions), 128), np.float32)
    sin = np.empty_like(cos)
    for t, p in enumerate(positions):
        rc, c, s = oracle_lib.yarn(p)
        cos[t], sin[t] = c, s
    factor = np.array([oracle.orc_query_factor(p) for p in positions], np.float32)
    for query in (False, True):
        out = np.empty_like(x)
        oracle.orc_rope(x.ctypes.data, cos.ctypes.data, sin.ctypes.data,
                        factor.ctypes.data if query else None, out.ctypes.data, width,
                        len(positions))
        for t, p in enumerate(positions):
            row = x[t * width:(t + 1) * width].astype(np.float64)
            rot = np.concatenate([-row[64:], row[:64]])
            expected = row * cos[t] + rot * sin[t]
            if query:
                expected *= 1 + 0.1 * math.log(1 + p // 16384)
            assert np.max(np.abs(out[t * width:(t + 1) * width] - expected)) < 2e-6


def double_attention(q, k, v, prefix, count):
    out = np.zeros((count, 32, 128))
    for t in range(count):
        n = prefix + t + 1
        for h in range(32):
            qh = q[t, h * 128:(h + 1) * 128].astype(np.float64)
            kh = k[:n, (h // 4) * 128:(h // 4 + 1) * 128].astype(np.float64)
            vh = v[:n, (h // 4) * 128:(h // 4 + 1) * 128].astype(np.float64)
            s = kh @ qh / math.sqrt(128)
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ vh
    return out.reshape(count, 4096)


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_attention_small_vs_double(schedule):
    count, prefix = 2, 3
    total = prefix + count
    q = np.array([((i % 11) - 5) * 0.03125 for i in range(count * 4096)], np.float32)
    k = np.array([((i % 17) - 8) * 0.03125 for i in range(total * 1024)], np.float32)
    v = np.array([((i % 23) - 11) * 0.0625 for i in range(total * 1024)], np.float32)
    out = oracle_lib.attention(schedule, q, k, v, 128, 1024, prefix, count)
    expected = double_attention(q.reshape(count, 4096), k.reshape(total, 1024),
                                v.reshape(total, 1024), prefix, count)
    assert np.max(np.abs(out - expected.reshape(-1))) < 2e-6


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_attention_long_causal_sentinel(schedule):
    total, count = 4352, 2
    q = np.zeros(count * 4096, np.float32)
    k = np.zeros(total * 1024, np.float32)
    v = np.ones(total * 1024, np.float32)
    v[(total - 1) * 1024:] = 4352.0
    out = oracle_lib.attention(schedule, q, k, v, 128, 1024, total - count, count)
    assert np.max(np.abs(out[:4096] - 1.0)) < 2e-4
    assert np.max(np.abs(out[4096:] - 8703.0 / 4352)) < 2e-4


def test_attention_layouts_agree():
    """Position-major (reference) and head-major (device) KV layouts give the
    same bits for both schedules."""
    rng = np.random.default_rng(5)
    count, prefix, cap = 3, 130, 256
    total = prefix + count
    q = rng.normal(size=count * 4096).astype(np.float32)
    kpm = rng.normal(size=(total, 1024)).astype(np.float32)
    vpm = rng.normal(size=(total, 1024)).astype(np.float32)
    khm = np.zeros((8, cap, 128), np.float32)
    vhm = np.zeros((8, cap, 128), np.float32)
    khm[:, :total] = kpm.reshape(total, 8, 128).transpose(1, 0, 2)
    vhm[:, :total] = vpm.reshape(total, 8, 128).transpose(1, 0, 2)
    for schedule in SCHEDULES:
        a = oracle_lib.attention(schedule, q, kpm.reshape(-1), vpm.reshape(-1), 128, 1024,
                                 prefix, count)
        b = oracle_lib.attention(schedule, q, khm.reshape(-1), vhm.reshape(-1), cap * 128, 128,
                                 prefix, count)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_schedules_agree_within_fp32_tolerance():
    rng = np.random.default_rng(9)
    count, prefix = 4, 300
    total = prefix + count
    q = rng.normal(size=count * 4096).astype(np.float32)
    k = rng.normal(size=total * 1024).astype(np.float32)
    v = rng.normal(size=total * 1024).astype(np.float32)
    a = oracle_lib.attention(REF, q, k, v, 128, 1024, prefix, count)
    b = oracle_lib.attention(MIRROR, q, k, v, 128, 1024, prefix, count)
    expected = double_attention(q.reshape(count, 4096), k.reshape(total, 1024),
                                v.reshape(total, 1024), prefix, count).reshape(-1)
    assert np.max(np.abs(a - expected)) < 1e-5
    assert np.max(np.abs(b - expected)) < 1e-5
