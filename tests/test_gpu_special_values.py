"""Special-value inputs through the row-dot and RMSNorm kernels, restating the
reference's frozen regression (tests/test_metal_reference.m:60-130) on the
gfx950 kernels against the oracle's device-mirror schedule:
- inputs: all ones (pattern 0), every element one special value (+-0,
  +-smallest subnormal, largest subnormal, smallest normal, +-Inf, a NaN
  payload: patterns 1..9), 2^24 cancellation (+2^24, 0.25, -2^24, 0.25:
  pattern 10), and mixed values (pattern 11);
- weights: ones for pattern 0, otherwise a mixed FP32 pattern (FP32 row dot),
  finite E4M3FN codes (FP8), BF16 of the mixed pattern (BF16), or norm gains
  that include 0, negatives and unequal magnitudes;
- sizes K in {1, 7, 31, 32, 33, 63, 65, 3072}, 1 or 3 rows, 1..3 tokens;
- checks: every non-NaN output bit-identical to the mirror and NaN exactly
  where the mirror has NaN; four canary words before and after the output
  untouched; inputs unchanged; all-ones dots equal K exactly.
"""
import ctypes

import numpy as np
import pytest

import lunelette_amd as lh
import oracle_lib
from oracle_lib import MIRROR, W_BF16, W_F32, W_FP8

pytestmark = pytest.mark.gpu
CANARY = 0x7f24d13b
SPECIAL = [0x00000000, 0x80000000, 0x00000001, 0x80000001, 0x007fffff, 0x00800000, 0x7f800000,
           0xff800000, 0x7fc00125]
SIZES = [1, 7, 31, 32, 33, 63, 65, 3072]
NORM_GAINS = np.array([0, -2, 0.125, 3, -0.5, 8, -4], np.float32)


def pattern_values(pattern, n):
    i = np.arange(n)
    if pattern == 0:
        return np.ones(n, np.float32)
    if pattern <= 9:
        return np.full(n, SPECIAL[pattern - 1], np.uint32).view(np.float32)
    if pattern == 10:
        return np.where(i % 4 == 0, 2.0 ** 24, np.where(i % 4 == 2, -2.0 ** 24, 0.25)
                        ).astype(np.float32)
    return (((i * 7919 + 313) % 257).astype(np.int64) - 128).astype(np.float32) / 64


def guarded_run(gpu, n_out, launch):
    """Runs launch(d_out) on an output with 4 canary words either side."""
    out = lh.DeviceBuffer((n_out + 8) * 4)
    out.upload(np.full(n_out + 8, CANARY, np.uint32))
    lh.check(launch(out.ptr + 16))
    lh.check(gpu.lh_device_synchronize())
    raw = out.download(np.uint32)
    assert np.all(raw[:4] == CANARY) and np.all(raw[-4:] == CANARY), "canary overwritten"
    return raw[4:-4]


def same_bits(got, want):
    want = np.ascontiguousarray(want, np.float32).view(np.uint32)
    got_nan = (got & 0x7fffffff) > 0x7f800000
    want_nan = (want & 0x7fffffff) > 0x7f800000
    assert np.array_equal(got_nan, want_nan), "NaN class differs"
    assert np.array_equal(got[~got_nan], want[~want_nan])


CASES = [(s, p) for s in range(len(SIZES)) for p in range(12)]


@pytest.mark.parametrize("kind", ["f32", "fp8", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=["K%d-p%d" % (SIZES[s], p) for s, p in CASES])
def test_row_dot_special_values(gpu, kind, case):
    s, pattern = case
    k, rows, tokens = SIZES[s], 3 if s % 2 else 1, s % 3 + 1
    x = pattern_values(pattern, k * tokens)
    if kind == "f32":
        w = np.ones(k * rows, np.float32) if pattern == 0 else pattern_values(11, k * rows)
        scale, oracle_kind = 1.0, W_F32
    elif kind == "fp8":
        codes = (np.arange(k * rows) * 37 + 5) % 254
        w = (np.full(k * rows, 0x38) if pattern == 0 else codes + (codes >= 127)).astype(np.uint8)
        scale, oracle_kind = (1.0 if pattern == 0 else 0.0146484375), W_FP8
    else:
        values = np.ones(k * rows, np.float32) if pattern == 0 else pattern_values(11, k * rows)
        w = (values.view(np.uint32) >> 16).astype(np.uint16)
        scale, oracle_kind = 1.0, W_BF16
    d_w, d_x = lh.DeviceBuffer.from_array(w), lh.DeviceBuffer.from_array(x)
    if kind == "f32":
        run = lambda out: gpu.lh_f32_matvec(d_w.ptr, d_x.ptr, out, rows, k, tokens, None)
    elif kind == "fp8":
        run = lambda out: gpu.lh_fp8_matvec(d_w.ptr, scale, d_x.ptr, out, rows, k, tokens, 0,
                                            None)
    else:
        run = lambda out: gpu.lh_bf16_matvec(d_w.ptr, d_x.ptr, out, rows, k, tokens, None)
    got = guarded_run(gpu, rows * tokens, run)
    want = oracle_lib.matvec(MIRROR, oracle_kind, w, scale, x, rows, k, tokens)
    same_bits(got, want)
    assert np.array_equal(d_w.download(w.dtype), w) and np.array_equal(
        d_x.download(np.float32).view(np.uint32), x.view(np.uint32))
    if pattern == 0:
        assert np.all(got.view(np.float32) == k)


@pytest.mark.parametrize("case", CASES, ids=["K%d-p%d" % (SIZES[s], p) for s, p in CASES])
def test_rmsnorm_special_values(gpu, case):
    s, pattern = case
    k, tokens = SIZES[s], s % 3 + 1
    x = pattern_values(pattern, k * tokens)
    gamma = (np.ones(k, np.float32) if pattern == 0 else
             NORM_GAINS[(np.arange(k) + pattern) % 7])
    d_g, d_x = lh.DeviceBuffer.from_array(gamma), lh.DeviceBuffer.from_array(x)
    got = guarded_run(gpu, k * tokens,
                      lambda out: gpu.lh_rmsnorm(d_g.ptr, d_x.ptr, out, k, tokens, None))
    want = oracle_lib.rmsnorm(MIRROR, gamma, x, k, tokens)
    same_bits(got, want)
    assert np.array_equal(d_x.download(np.float32).view(np.uint32), x.view(np.uint32))
