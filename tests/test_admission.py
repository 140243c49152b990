"""FP8 admission (lh_fp8_admit, the check the runtime's upload applies to every
FP8 tensor) against the reference's own C, built from source into
oracle/_ref/libref.so:
- the compact strategies against lunelette_metal_weights_load_raw
  (src/metal_weights.c:174-231), RESIDENT_FP32 against st_load_fp8
  (src/safetensors.c:521-548), on every one of the 256 codes under scale
  patterns: the bad BF16 scales of tests/test_metal_weights.c:25-110 (0, -0,
  -1, NaN, Inf, subnormals 0x0001 and 0x007f, the smallest normals 0x0080 and
  0x0100, 0x04ff whose products go subnormal, 0x7f00 whose products overflow),
  good ones (0x39fb, 0x7f7f, 1.0), and FP32 scales no checkpoint can carry
  (1.00001, 0.0125, an FP32 subnormal, 1.5 * 2^-126);
- the reference test's whole-tensor cases: the 254 finite codes at 0x39fb, a
  NaN code at byte 65537 of a 65538-byte tensor (the same byte is named), and
  65538 signed zeros.
The reference handle is built the way tests/test_metal_weights.c:25-45 builds
it: a one-tensor file and a hand-set scale, so FP32 scales reach the checks.
"""
import ctypes
import math
import os
import struct
import tempfile

import numpy as np
import pytest

import lunelette_amd as lh
import oracle_lib

RESIDENT, COMPACT, LOOKUP = 0, 1, 2


class RefTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("dtype", ctypes.c_int),
                ("rank", ctypes.c_size_t), ("shape", ctypes.c_uint64 * 8),
                ("begin", ctypes.c_uint64), ("end", ctypes.c_uint64)]


class RefFile(ctypes.Structure):
    _fields_ = [("file", ctypes.c_void_p), ("base", ctypes.c_uint64),
                ("count", ctypes.c_size_t), ("tensors", ctypes.POINTER(RefTensor))]


class RefSlot(ctypes.Structure):
    _fields_ = [("scale", ctypes.c_float), ("tensor", ctypes.POINTER(RefTensor)),
                ("elements", ctypes.c_size_t)]


class RefWeights(ctypes.Structure):
    _fields_ = [("file", RefFile), ("weights", RefSlot * (2 + 26 * 9)), ("bytes", ctypes.c_uint64)]


def bf16(bits):
    return struct.unpack("<f", struct.pack("<I", bits << 16))[0]


def f32(bits):
    return struct.unpack("<f", struct.pack("<I", bits))[0]


BAD_BF16 = [0x0000, 0x8000, 0xbf80, 0x7fc0, 0x7f80, 0x0001, 0x007f, 0x0080, 0x0100, 0x04ff,
            0x7f00]
GOOD_BF16 = [0x39fb, 0x7f7f, 0x3f80]
SCALES = ([("bf16 0x%04x" % b, bf16(b)) for b in BAD_BF16 + GOOD_BF16] +
          [("1.00001", 1.00001), ("0.0125", 0.0125), ("fp32 subnormal", f32(1)),
           ("1.5 * 2^-126", f32(0x00c00000))])


class Reference:
    """lunelette_metal_weights_load_raw and st_load_fp8 over bytes in a
    temporary file, one tensor at a time."""

    def __init__(self, ref, data):
        libc = ctypes.CDLL(None)
        libc.fopen.restype = ctypes.c_void_p
        libc.fopen.argtypes = [ctypes.c_char_p, ctypes.c_char_p]
        libc.fclose.argtypes = [ctypes.c_void_p]
        self.libc, self.ref = libc, ref
        fd, self.path = tempfile.mkstemp(suffix=".bin")
        with os.fdopen(fd, "wb") as f:
            f.write(bytes(data))
        self.handle = libc.fopen(self.path.encode(), b"rb")
        assert self.handle
        self.tensor = RefTensor()
        self.tensor.name = b"synthetic.compact"
        self.tensor.dtype = 1
        self.w = RefWeights()
        self.w.file.file = self.handle
        self.w.file.count = 1
        self.w.file.tensors = ctypes.pointer(self.tensor)
        self.w.weights[3].tensor = ctypes.pointer(self.tensor)

    def close(self):
        self.libc.fclose(self.handle)
        os.unlink(self.path)

    def select(self, begin, end, scale):
        self.tensor.begin, self.tensor.end = begin, end
        self.w.weights[3].elements = end - begin
        self.w.weights[3].scale = scale

    def compact(self, begin, end, scale):
        self.select(begin, end, scale)
        out = (ctypes.c_ubyte * (end - begin))()
        err = ctypes.create_string_buffer(512)
        rc = self.ref.lunelette_metal_weights_load_raw(ctypes.byref(self.w), 3, out, end - begin,
                                                       err, 512)
        return rc == 0, err.value.decode()

    def resident(self, begin, end, scale):
        self.select(begin, end, scale)
        out = (ctypes.c_float * (end - begin))()
        rc = self.ref.st_load_fp8(ctypes.byref(self.w.file), ctypes.byref(self.tensor), scale,
                                  out, end - begin)
        return rc == 0


@pytest.fixture(scope="module")
def ref():
    r = oracle_lib.load_ref()
    if r is None:
        pytest.skip("oracle/_ref not built (needs the reference sources)")
    r.lunelette_metal_weights_load_raw.restype = ctypes.c_int
    r.lunelette_metal_weights_load_raw.argtypes = [ctypes.c_void_p, ctypes.c_size_t,
                                                   ctypes.c_void_p, ctypes.c_size_t,
                                                   ctypes.c_char_p, ctypes.c_size_t]
    r.st_load_fp8.restype = ctypes.c_int
    r.st_load_fp8.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p,
                              ctypes.c_size_t]
    return r


def admit(product, codes, scale, strategy):
    codes = np.ascontiguousarray(codes, np.uint8)
    err = ctypes.create_string_buffer(256)
    rc = product.lh_fp8_admit(codes.ctypes.data, codes.size, scale, strategy, err, 256)
    if rc:
        assert err.value, "refusal without a diagnostic"
    return rc == 0, err.value.decode()


@pytest.mark.parametrize("name,scale", SCALES, ids=[n for n, _ in SCALES])
def test_every_code_matches_reference(ref, product, name, scale):
    reference = Reference(ref, range(256))
    try:
        for code in range(256):
            want_compact, _ = reference.compact(code, code + 1, scale)
            want_resident = reference.resident(code, code + 1, scale)
            for strategy in (COMPACT, LOOKUP):
                assert admit(product, [code], scale, strategy)[0] == want_compact, (name, code)
            assert admit(product, [code], scale, RESIDENT)[0] == want_resident, (name, code)
    finally:
        reference.close()


def test_scale_patterns_reach_both_outcomes(ref, product):
    # The patterns above are not vacuous: somewhere each strategy admits a code
    # the other refuses, and NaN codes are refused everywhere.
    split = 0
    for _, scale in SCALES:
        for code in range(256):
            c = admit(product, [code], scale, COMPACT)[0]
            r = admit(product, [code], scale, RESIDENT)[0]
            split += r and not c
            assert not c or r   # compact admits a subset of resident
            if code in (0x7f, 0xff):
                assert not c and not r
    assert split > 100


def test_reference_whole_tensor_cases(ref, product):
    finite = [c for c in range(256) if c not in (0x7f, 0xff)]
    reference = Reference(ref, finite)
    try:
        scale = bf16(0x39fb)
        assert reference.compact(0, 254, scale)[0]
        assert admit(product, finite, scale, COMPACT)[0]
        assert reference.resident(0, 254, scale) and admit(product, finite, scale, RESIDENT)[0]
        # A subnormal scale times a large code gives a normal product: the
        # compact check still refuses the scale itself.
        tiny = bf16(0x007f)
        assert not reference.compact(0, 254, tiny)[0]
        ok, why = admit(product, finite, tiny, COMPACT)
        assert not ok and "scale" in why
    finally:
        reference.close()
    for bad in (0x7f, 0xff):
        data = [0] * 65537 + [bad]
        reference = Reference(ref, data)
        try:
            ok, why = reference.compact(0, len(data), bf16(0x39fb))
            assert not ok and "byte 65537" in why
            ok, mine = admit(product, data, bf16(0x39fb), COMPACT)
            assert not ok and "byte 65537" in mine
            assert not reference.resident(0, len(data), bf16(0x39fb))
            assert not admit(product, data, bf16(0x39fb), RESIDENT)[0]
        finally:
            reference.close()
    zeros = [0x00, 0x80] * 32769
    reference = Reference(ref, zeros)
    try:
        for scale in (bf16(0x39fb), bf16(0x7f7f)):
            assert reference.compact(0, len(zeros), scale)[0]
            assert admit(product, zeros, scale, COMPACT)[0]
        assert not reference.compact(0, len(zeros), 1.00001)[0]
        assert not admit(product, zeros, 1.00001, COMPACT)[0]
    finally:
        reference.close()


def test_admit_rejects_bad_arguments(product):
    err = ctypes.create_string_buffer(64)
    codes = np.zeros(4, np.uint8)
    assert product.lh_fp8_admit(None, 4, 1.0, COMPACT, err, 64) == -1
    assert product.lh_fp8_admit(codes.ctypes.data, 4, 1.0, 7, err, 64) == -1
    assert product.lh_fp8_admit(codes.ctypes.data, 0, 1.0, COMPACT, None, 0) == 0
    assert math.isnan(bf16(0x7fc0))
