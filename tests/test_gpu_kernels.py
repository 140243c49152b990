"""GPU parity of single kernels through the C-ABI (include/lunelette_kernels.h).

Bit-exact against the oracle's device-mirror schedule; within fp32 tolerance
of the reference-literal schedule. Shapes and scales follow the reference's
own tests (tests/test_metal_compact.m:46-145) and the single FP8 linear
9216x3072 (scale 0.0125, x ~ N(0,1)).
"""
import ctypes
import json
import math
import os

import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import synthetic as syn

import oracle_lib
from oracle_lib import MIRROR, REF, W_BF16, W_F32, W_FP8

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_fp8_hardware_decode_all_codes(gpu):
    golden = np.array(json.load(open(os.path.join(GOLDEN, "fp8_golden.json")))["bits"], np.uint32)
    codes = lh.DeviceBuffer.from_array(np.arange(256, dtype=np.uint8))
    out = lh.DeviceBuffer(256 * 4)
    lh.check(gpu.lh_fp8_decode(codes.ptr, out.ptr, 256, None))
    lh.check(gpu.lh_device_synchronize())
    got = out.download(np.float32)
    for code in range(256):
        if (code & 127) == 127:
            assert math.isnan(got[code]), code
        else:
            assert bits(got[code:code + 1])[0] == golden[code], hex(code)


def test_expf_bitwise_vs_oracle(gpu, oracle):
    xs = np.concatenate([np.linspace(-90, 90, 200001, dtype=np.float32),
                         np.float32([0.0, -0.0, np.inf, -np.inf, 1e-30, -1e-30])])
    d_x = lh.DeviceBuffer.from_array(xs)
    d_y = lh.DeviceBuffer(xs.nbytes)
    lh.check(gpu.lh_expf(d_x.ptr, d_y.ptr, xs.size, None))
    got = d_y.download(np.float32)
    want = np.array([oracle.orc_expf(float(x)) for x in xs], np.float32)
    assert np.array_equal(bits(got), bits(want))


def test_element_modes_bitwise(gpu, oracle):
    n = 100003
    rng = np.random.default_rng(1)
    a = (rng.normal(size=n) * 40).astype(np.float32)
    b = rng.normal(size=n).astype(np.float32)
    d_a, d_b = lh.DeviceBuffer.from_array(a), lh.DeviceBuffer.from_array(b)
    d_o = lh.DeviceBuffer(a.nbytes)
    expected = {0: a + b, 2: a * b,
                1: np.array([oracle.orc_silu_mirror(float(v)) for v in a], np.float32)}
    for mode in (0, 1, 2):
        lh.check(gpu.lh_element(mode, d_a.ptr, d_b.ptr, d_o.ptr, n, None))
        assert np.array_equal(bits(d_o.download(np.float32)), bits(expected[mode])), mode


def run_fp8(gpu, w, scale, x, rows, cols, tokens=1, lookup=0, guard=4):
    d_w = lh.DeviceBuffer.from_array(w)
    d_x = lh.DeviceBuffer.from_array(x)
    d_y = lh.DeviceBuffer((tokens * rows + guard) * 4)
    lh.check(gpu.lh_memset_device(d_y.ptr, 0x5a, d_y.nbytes))
    lh.check(gpu.lh_fp8_matvec(d_w.ptr, scale, d_x.ptr, d_y.ptr, rows, cols, tokens, lookup, None))
    out = d_y.download(np.uint8)
    assert np.all(out[tokens * rows * 4:] == 0x5a), "wrote past the output"
    return out[:tokens * rows * 4].view(np.float32)


def test_fp8_matvec_9216x3072_bitwise_mirror(gpu):
    rows, cols, scale = 9216, 3072, 0.0125
    w = syn.fp8(11, 500, rows, cols)
    x = syn.normal_f32(11, 501, cols)
    got = run_fp8(gpu, w, scale, x, rows, cols)
    mirror = oracle_lib.matvec(MIRROR, W_FP8, w, scale, x, rows, cols)
    assert np.array_equal(bits(got), bits(mirror))
    ref = oracle_lib.matvec(REF, W_FP8, w, scale, x, rows, cols)
    dec = oracle_lib.load()
    table = np.array([dec.orc_fp8_decode(c) for c in range(256)], np.float32) * np.float32(scale)
    magnitude = np.abs(table[w]).astype(np.float64) @ np.abs(x).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= 1e-6 * magnitude)
    lookup = run_fp8(gpu, w, scale, x, rows, cols, lookup=1)
    assert np.array_equal(bits(lookup), bits(got))


def test_fp8_matvec_reference_shapes_and_scales(gpu):
    """tests/test_metal_compact.m:97-145: columns {1,7,31,33,257}, 259 rows,
    every finite code in row and column positions, extreme scales; lookup and
    arithmetic bitwise equal (and equal to the mirror)."""
    scales = [1.0, float.fromhex("0x1.f6p-12"), float.fromhex("0x1.02p+5"),
              float.fromhex("0x1p-110"), float.fromhex("0x1p+100")]
    for cols in (1, 7, 31, 33, 257, 1040, 3072):
        rows = 259
        k = np.arange(rows * cols) % 254
        w = (k + (k >= 127)).astype(np.uint8)
        x = np.array([((i % 17) - 8) / 16.0 for i in range(cols)], np.float32)
        for scale in scales:
            a = run_fp8(gpu, w, scale, x, rows, cols, lookup=0)
            b = run_fp8(gpu, w, scale, x, rows, cols, lookup=1)
            m = oracle_lib.matvec(MIRROR, W_FP8, w, scale, x, rows, cols)
            assert np.array_equal(bits(a), bits(b)), (cols, scale)
            assert np.array_equal(bits(a), bits(m)), (cols, scale)


def test_fp8_matvec_multitoken_and_resident_equivalence(gpu):
    rows, cols, tokens, scale = 1024, 4096, 5, 0.015625
    w = syn.fp8(3, 77, rows, cols)
    x = syn.normal_f32(3, 78, tokens * cols)
    got = run_fp8(gpu, w, scale, x, rows, cols, tokens)
    mirror = oracle_lib.matvec(MIRROR, W_FP8, w, scale, x, rows, cols, tokens)
    assert np.array_equal(bits(got), bits(mirror))
    # Resident FP32 weights hold the exact decode; the per-tensor scale
    # multiplies the row total, so FP32 * scale equals the FP8 path bitwise.
    table = np.array([oracle_lib.load().orc_fp8_decode(c) for c in range(256)], np.float32)
    d_w = lh.DeviceBuffer.from_array(table[w])
    d_x = lh.DeviceBuffer.from_array(x)
    d_y = lh.DeviceBuffer(tokens * rows * 4)
    lh.check(gpu.lh_f32_matvec(d_w.ptr, d_x.ptr, d_y.ptr, rows, cols, tokens, None))
    resident = d_y.download(np.float32) * np.float32(scale)
    assert np.array_equal(bits(resident), bits(got))


def test_bf16_matvec_bitwise_mirror(gpu):
    rows, cols = 4099, 3072
    w = syn.normal_bf16(5, 0, rows * cols, 0.0, 0.02)
    x = syn.normal_f32(5, 9, cols)
    d_w, d_x = lh.DeviceBuffer.from_array(w), lh.DeviceBuffer.from_array(x)
    d_y = lh.DeviceBuffer(rows * 4)
    lh.check(gpu.lh_bf16_matvec(d_w.ptr, d_x.ptr, d_y.ptr, rows, cols, 1, None))
    mirror = oracle_lib.matvec(MIRROR, W_BF16, w, 1.0, x, rows, cols)
    assert np.array_equal(bits(d_y.download(np.float32)), bits(mirror))


@pytest.mark.parametrize("width,tokens", [(3072, 3), (67, 2), (9216, 2)])
def test_rmsnorm_bitwise_mirror(gpu, width, tokens):
    rng = np.random.default_rng(width)
    x = (rng.normal(size=width * tokens) * 1000).astype(np.float32)
    gamma = (1 + rng.normal(size=width) * 0.02).astype(np.float32)
    d_g, d_x = lh.DeviceBuffer.from_array(gamma), lh.DeviceBuffer.from_array(x)
    d_o = lh.DeviceBuffer(x.nbytes)
    lh.check(gpu.lh_rmsnorm(d_g.ptr, d_x.ptr, d_o.ptr, width, tokens, None))
    mirror = oracle_lib.rmsnorm(MIRROR, gamma, x, width, tokens)
    assert np.array_equal(bits(d_o.download(np.float32)), bits(mirror))


def test_rope_bitwise_oracle(gpu, oracle):
    positions = [0, 1, 4351, 16383, 16384, 16385]
    width = 4096
    rng = np.random.default_rng(4)
    x = rng.normal(size=len(positions) * width).astype(np.float32)
    cos = np.empty((len(positions), 128), np.float32)
    sin = np.empty_like(cos)
    for t, p in enumerate(positions):
        rc, c, s = oracle_lib.yarn(p)
        cos[t], sin[t] = c, s
    factor = np.array([oracle.orc_query_factor(p) for p in positions], np.float32)
    d = {k: lh.DeviceBuffer.from_array(v) for k, v in
         {"x": x, "c": cos, "s": sin, "f": factor}.items()}
    out = lh.DeviceBuffer(x.nbytes)
    expected = np.empty_like(x)
    oracle.orc_rope(x.ctypes.data, cos.ctypes.data, sin.ctypes.data, factor.ctypes.data,
                    expected.ctypes.data, width, len(positions))
    lh.check(gpu.lh_rope(d["x"].ptr, d["c"].ptr, d["s"].ptr, d["f"].ptr, out.ptr, width,
                         len(positions), None))
    assert np.array_equal(bits(out.download(np.float32)), bits(expected))


def test_head_nonfinite_flag(gpu):
    """The runtime's head step flags Inf/NaN logits on the device (in place of
    the host finite scan, src/metal_runtime.m:418-424): the logits equal the
    plain head's bitwise, the flag stays clear on finite output and is set
    when one row of the tied embedding makes its logit Inf or NaN."""
    vocab, width = lh.VOCAB, lh.HIDDEN
    gamma = lh.DeviceBuffer.from_array(np.ones(width, np.float32))
    xrow = lh.DeviceBuffer.from_array(syn.normal_f32(7, 1, width))
    table = np.zeros((vocab, width), np.uint16)
    table[::977] = 0x3F80                                # 1.0 on some rows
    cases = [("finite", None, 0), ("inf", 0x7F80, 1), ("nan", 0x7FC1, 1)]
    for name, bad, want in cases:
        if bad is not None:
            table[4242, 17] = bad
        emb = lh.DeviceBuffer.from_array(table)
        plain = lh.DeviceBuffer(vocab * 4)
        checked = lh.DeviceBuffer(vocab * 4)
        flag = lh.DeviceBuffer.from_array(np.zeros(16, np.uint32))
        lh.check(gpu.lh_head_forward(emb.ptr, gamma.ptr, xrow.ptr, plain.ptr, None), "head")
        lh.check(gpu.lh_head_forward_checked(emb.ptr, gamma.ptr, xrow.ptr, checked.ptr, flag.ptr,
                                             None), "head checked")
        lh.check(gpu.lh_device_synchronize(), "sync")
        a, b = plain.download(np.float32), checked.download(np.float32)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), name
        assert int(flag.download(np.uint32)[0]) == want, name
        assert np.isfinite(b).all() == (want == 0), name
        del emb


def test_read_floor_runs_and_validates(gpu):
    """The streaming-read measurement kernel bench.py times as the decode
    kernels' floor: it accepts sizes that the grid and loads-in-flight divide,
    refuses others, and leaves its sink alone for ordinary data."""
    nbytes = 256 * 4 * 64 * 16 * 8 * 3
    src = lh.DeviceBuffer.from_array(np.zeros(nbytes // 4, np.float32))
    sink = lh.DeviceBuffer.from_array(np.zeros(16384, np.uint32))
    for grid, unroll in ((256, 1), (256, 8), (768, 2), (1536, 4)):
        lh.check(gpu.lh_read_floor(src.ptr, nbytes, grid, unroll, sink.ptr, None))
    lh.check(gpu.lh_device_synchronize())
    assert not sink.download(np.uint32).any()
    for grid, unroll, size in ((256, 3, nbytes), (0, 1, nbytes), (256, 1, nbytes - 16),
                               (4096, 8, nbytes)):
        assert gpu.lh_read_floor(src.ptr, size, grid, unroll, sink.ptr, None) == -1
