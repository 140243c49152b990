"""Checkpoint files on the host (no GPU): the safetensors container reader and
the FP8 checkpoint tensor contract of the product library, against the
reference's own C built from its sources (oracle/_ref: src/safetensors.c and
src/metal_weights.c).

- Container: accept/reject and the parsed tensor list are compared with the
  reference's st_open on the behaviours its tests/test_safetensors.c pins
  (grammar, escapes, limits, offsets and tiling) and on seeded random
  mutations of valid headers.
- Contract: a sparse full-size checkpoint (the header plus the scalar
  payloads) is accepted by both, its scales read back exactly; mutations
  that keep the container valid but break the contract (renamed tensor,
  wrong dtype or shape, companion rank or value, unknown text tensor) are
  rejected by both; non-text tensors are ignored by both.
- create(path) rejects a missing file and a non-checkpoint container before
  any device work.
"""
import ctypes
import json
import os
import random
import struct

import numpy as np
import pytest

import lunelette_amd as lh
import oracle_lib
from checkpoint_files import (model_entries, slot_tensors, write_container,
                              write_sparse_model, bf16_bits)


class RefTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("dtype", ctypes.c_int),
                ("rank", ctypes.c_size_t), ("shape", ctypes.c_uint64 * 8),
                ("begin", ctypes.c_uint64), ("end", ctypes.c_uint64)]


class RefFile(ctypes.Structure):
    _fields_ = [("file", ctypes.c_void_p), ("base", ctypes.c_uint64),
                ("count", ctypes.c_size_t), ("tensors", ctypes.POINTER(RefTensor))]


REF_DTYPE = {1: "F8_E4M3", 2: "BF16", 4: "F32", 8: "I64"}


@pytest.fixture(scope="module")
def ref():
    r = oracle_lib.load_ref()
    if r is None:
        pytest.skip("oracle/_ref not built (needs the reference sources)")
    r.st_open.restype = ctypes.c_int
    r.st_open.argtypes = [ctypes.POINTER(RefFile), ctypes.c_char_p, ctypes.c_char_p,
                          ctypes.c_size_t]
    r.st_close.restype = None
    r.st_close.argtypes = [ctypes.POINTER(RefFile)]
    r.lunelette_metal_weights_open.restype = ctypes.c_int
    r.lunelette_metal_weights_open.argtypes = [ctypes.c_void_p, ctypes.c_char_p,
                                               ctypes.c_char_p, ctypes.c_size_t]
    r.lunelette_metal_weights_close.restype = None
    r.lunelette_metal_weights_close.argtypes = [ctypes.c_void_p]
    return r


@pytest.fixture(scope="module")
def product():
    return lh.lib()


def ref_listing(ref, path):
    f = RefFile()
    err = ctypes.create_string_buffer(256)
    if ref.st_open(ctypes.byref(f), path.encode(), err, 256):
        return None
    lines = []
    for i in range(f.count):
        t = f.tensors[i]
        dims = ",".join(str(t.shape[k]) for k in range(t.rank))
        lines.append("%s|%s|%d|%s|%d|%d\n" % (t.name.decode("latin-1"), REF_DTYPE[t.dtype],
                                              t.rank, dims, t.begin, t.end))
    ref.st_close(ctypes.byref(f))
    return "".join(lines)


def our_listing(product, path):
    cap = 1 << 22
    buf = ctypes.create_string_buffer(cap)
    err = ctypes.create_string_buffer(256)
    if product.lh_st_inspect(path.encode(), buf, cap, err, 256):
        assert err.value, "rejection without a diagnostic"
        return None
    return buf.value.decode("latin-1")


def agree(ref, product, path):
    mine, theirs = our_listing(product, path), ref_listing(ref, path)
    assert mine == theirs, (open(path, "rb").read()[:200], mine, theirs)
    return mine is not None


def T(name, dtype, shape, begin, end):
    return '"%s":{"dtype":"%s","shape":[%s],"data_offsets":[%d,%d]}' % (
        name, dtype, ",".join(str(d) for d in shape), begin, end)


# (header, data bytes, accepted) covering the reference test's behaviours.
CASES = [
    ("{}", 0, True), ("{}", 1, False), ("{", 0, False), ("{}junk", 0, False),
    (" {}", 0, False), ("{}  \n\t\r", 0, True), ('{"" : {}}', 0, False),
    ("{" + T("w", "BF16", [2, 2], 0, 8) + "," + T("f", "F32", [], 8, 12) + "," +
     T("i", "I64", [1], 12, 20) + "}", 20, True),
    ('{"x":{"dtype":"BF16","shape":[1]}}', 2, False),
    ('{"x":{"dtype":"BF16","shape":[1.0],"data_offsets":[0,2]}}', 2, False),
    ("{" + T("x", "BF16", [1], 0, 2) + ",}", 2, False),
    ("{" + T("x", "BF16", [1], 0, 2) + "," + T("\\u0078", "BF16", [1], 2, 4) + "}", 4, False),
    ("{" + T("x", "F16", [1], 0, 2) + "}", 2, False),
    ('{"x":{"dtype":"BF16","shape":[-1],"data_offsets":[0,2]}}', 2, False),
    ('{"x":{"dtype":"BF16","shape":[01],"data_offsets":[0,2]}}', 2, False),
    ('{"x":{"dtype":"BF16","shape":[0],"data_offsets":[0,0]}}', 0, True),
    ('{"x":{"dtype":"BF16","shape":[9223372036854775807,3],"data_offsets":[0,2]}}', 2, False),
    ('{"x":{"dtype":"BF16","shape":[9223372036854775808],"data_offsets":[0,2]}}', 2, False),
    ('{"x":{"dtype":"BF16","shape":[18446744073709551616],"data_offsets":[0,2]}}', 2, False),
    ("{" + T("x", "BF16", [1], 2, 0) + "}", 2, False),
    ("{" + T("x", "BF16", [1], 1, 3) + "}", 3, False),
    ("{" + T("x", "BF16", [1], 0, 2) + "}", 1, False),
    ("{" + T("x", "BF16", [1], 0, 2) + "}", 3, False),
    ('{"x":{"dtype":"BF16","dtype":"BF16","shape":[1],"data_offsets":[0,2]}}', 2, False),
    ('{"x":{},"x":{}}', 0, False),
    ("{" + T("x", "BF16", [1] * 8, 0, 2) + "}", 2, True),
    ("{" + T("x", "BF16", [1] * 9, 0, 2) + "}", 2, False),
    ("{" + T("x", "BF16", [1], 0, 2) + "," + T("y", "BF16", [1], 0, 2) + "}", 2, False),
    ('{"__metadata__":{"key":"value"}}', 0, True),
    ('{"__metadata__":{}}', 0, True),
    ('{"__metadata__":{},"__metadata__":{}}', 0, False),
    ('{"__metadata__":{"k":"v","k":"w"}}', 0, False),
    ('{"__metadata__":{"k":1}}', 0, False),
    ('{"__metadata__":[]}', 0, False),
    ('{"a\\"\\\\\\/\\u0041":{"dtype":"BF16","shape":[0],"data_offsets":[0,0]}}', 0, True),
    ('{"__metadata__":{"k":"\\n"}}', 0, False),
    ('{"__metadata__":{"k":"\\u001f"}}', 0, False),
    ('{"__metadata__":{"k":"\\u0080"}}', 0, False),
    ('{"__metadata__":{"k":"\\u00xz"}}', 0, False),
    ('{"__metadata__":{"k":"\\u007e"}}', 0, True),
    ('{"k\xc3\xa9":{"dtype":"BF16","shape":[0],"data_offsets":[0,0]}}', 0, False),
    ("{" + T("b", "BF16", [1], 2, 4) + "," + T("a", "BF16", [1], 0, 2) + "}", 4, True),
    ("{" + T("f", "F8_E4M3", [], 0, 1) + "}", 1, True),
    ('{"f":{"dtype":"F8_E4M3FN","shape":[1],"data_offsets":[0,1]}}', 1, False),
    ("{" + T("f", "F8_E4M3", [2], 0, 1) + "}", 1, False),
    ('{"e":{"dtype":"BF16","shape":[0,2],"data_offsets":[0,0]}}', 0, True),
    ('{"x":{"shape":[1],"data_offsets":[0,2],"dtype":"BF16"}}', 2, True),
    ('{"x":{"dtype":"BF16","shape":[1],"data_offsets":[0,2],"extra":1}}', 2, False),
    ('{"x":{"dtype":"BF16","shape":[1],"data_offsets":[0,2,4]}}', 2, False),
    ('{"x" : { "dtype" : "BF16" , "shape" : [ 1 ] , "data_offsets" : [ 0 , 2 ] } }', 2, True),
] + [
    ("{" + T("a", "BF16", [1], 0, 2) + "," + T("b", "BF16", [1], 2, 4) + "," +
     T("e", "BF16", [0], k, k) + "}", 4, k % 2 == 0) for k in range(5)
]


def test_container_cases_match_reference(ref, product, tmp_path):
    path = str(tmp_path / "case.safetensors")
    for header, data, accepted in CASES:
        write_container(path, header, b"\0" * data)
        assert agree(ref, product, path) == accepted, header


def test_container_limits_match_reference(ref, product, tmp_path):
    path = str(tmp_path / "limits.safetensors")
    empty = '"%s":{"dtype":"BF16","shape":[0],"data_offsets":[0,0]}'
    for count in (4096, 4097):
        write_container(path, "{" + ",".join(empty % ("t%d" % i) for i in range(count)) + "}")
        assert agree(ref, product, path) == (count == 4096)
    for length in (255, 256):
        write_container(path, "{" + empty % ("a" * length) + "}")
        assert agree(ref, product, path) == (length == 255)
        write_container(path, '{"__metadata__":{"%s":"v"}}' % ("k" * length))
        assert agree(ref, product, path) == (length == 255)
    for count in (64, 65):
        items = ",".join('"k%d":"v"' % i for i in range(count))
        write_container(path, '{"__metadata__":{%s}}' % items)
        assert agree(ref, product, path) == (count == 64)
    for length in (4095, 4096):
        write_container(path, '{"__metadata__":{"k":"%s"}}' % ("v" * length))
        assert agree(ref, product, path) == (length == 4095)
    for pad in ((1 << 20) - 2, (1 << 20) - 1):
        write_container(path, "{}" + " " * pad)
        assert agree(ref, product, path) == (pad == (1 << 20) - 2)


def test_container_truncations_match_reference(ref, product, tmp_path):
    path = str(tmp_path / "trunc.safetensors")
    header = ("{" + T("w", "BF16", [2, 2], 0, 8) + "," + T("f", "F32", [], 8, 12) + "}")
    full = struct.pack("<Q", len(header)) + header.encode() + bytes(range(12))
    for n in range(len(full)):
        with open(path, "wb") as f:
            f.write(full[:n])
        assert not agree(ref, product, path)
    with open(path, "wb") as f:
        f.write(b"\xff" * 8)
    assert not agree(ref, product, path)


def test_container_mutations_match_reference(ref, product, tmp_path):
    """Seeded random edits of valid headers: both readers agree on every one."""
    path = str(tmp_path / "fuzz.safetensors")
    seeds = [
        ("{" + T("w", "BF16", [2, 2], 0, 8) + "," + T("f", "F32", [], 8, 12) + "," +
         T("i", "I64", [1], 12, 20) + "}", 20),
        ('{"__metadata__":{"format":"pt","k\\u0041":"v"},' + T("z", "F8_E4M3", [3, 1], 0, 3) +
         "," + T("e", "BF16", [0], 3, 3) + "}", 3),
        ("{" + T("b", "BF16", [1], 2, 4) + "," + T("a", "BF16", [1], 0, 2) + "}", 4),
    ]
    alphabet = '{}[]:,"\\ 0123456789uxFBI_.-e\n'
    rng = random.Random(20251201)
    accepted = 0
    for i in range(1500):
        header, data = seeds[i % len(seeds)]
        text = list(header)
        for _ in range(rng.randint(1, 3)):
            op, at = rng.randrange(3), rng.randrange(len(text))
            if op == 0:
                del text[at]
            elif op == 1:
                text.insert(at, rng.choice(alphabet))
            else:
                text[at] = rng.choice(alphabet)
        size = data + rng.choice((0, 0, 0, 1, -1 if data else 0))
        write_container(path, "".join(text), b"\x3c" * size)
        accepted += agree(ref, product, path)
    assert 10 <= accepted <= 1490   # the edits reach both outcomes


def test_bounded_reads(product, tmp_path):
    path = str(tmp_path / "read.safetensors")
    header = "{" + T("w", "BF16", [2, 2], 0, 8) + "," + T("f", "F32", [], 8, 12) + "}"
    write_container(path, header, bytes(range(12)))
    out = (ctypes.c_uint8 * 16)()
    err = ctypes.create_string_buffer(128)
    assert product.lh_st_read_tensor(path.encode(), b"w", 0, out, 8, err, 128) == 0
    assert bytes(out[:8]) == bytes(range(8))
    assert product.lh_st_read_tensor(path.encode(), b"f", 2, out, 2, err, 128) == 0
    assert bytes(out[:2]) == bytes([10, 11])
    assert product.lh_st_read_tensor(path.encode(), b"w", 7, out, 2, err, 128) != 0
    assert product.lh_st_read_tensor(path.encode(), b"w", (1 << 64) - 1, out, 1, err, 128) != 0
    assert product.lh_st_read_tensor(path.encode(), b"missing", 0, out, 1, err, 128) != 0


# ---- checkpoint contract ----

def base_scales():
    rng = np.random.default_rng(7)
    scales = {}
    for slot, _n, dtype, _s in slot_tensors():
        if dtype == "F8_E4M3":
            scales[slot] = (bf16_bits(float(rng.uniform(0.01, 0.02))), bf16_bits(0.5))
    return scales


def ref_weights_open(ref, path):
    handle = ctypes.create_string_buffer(1 << 16)
    err = ctypes.create_string_buffer(512)
    rc = ref.lunelette_metal_weights_open(handle, path.encode(), err, 512)
    if rc == 0:
        ref.lunelette_metal_weights_close(handle)
    return rc == 0


def our_weights_open(product, path):
    scales = np.zeros(2 + 26 * 9, np.float32)
    err = ctypes.create_string_buffer(512)
    rc = product.lh_checkpoint_check(path.encode(), scales.ctypes.data_as(lh.c_float_p), err, 512)
    if rc:
        assert err.value
    return rc == 0, scales


def contract_agree(ref, product, path):
    mine, scales = our_weights_open(product, path)
    assert mine == ref_weights_open(ref, path)
    return mine, scales


def test_contract_accepts_full_checkpoint_and_reads_scales(ref, product, tmp_path):
    path = str(tmp_path / "model.safetensors")
    scales = base_scales()
    write_sparse_model(path, model_entries(scales))
    ok, read = contract_agree(ref, product, path)
    assert ok
    for slot, _n, dtype, _s in slot_tensors():
        expect = 1.0
        if dtype == "F8_E4M3":
            expect = np.array([scales[slot][0] << 16], np.uint32).view(np.float32)[0]
        assert read[slot] == expect


def mutated(entries, index, **change):
    out = [list(e) for e in entries]
    for key, value in change.items():
        out[index][{"name": 0, "dtype": 1, "shape": 2, "payload": 3}[key]] = value
    return out


def test_contract_rejections_match_reference(ref, product, tmp_path):
    path = str(tmp_path / "model.safetensors")
    scales = base_scales()
    entries = model_entries(scales)
    index = {e[0]: i for i, e in enumerate(entries)}
    q7 = "language_model.model.layers.7.self_attn.q_proj."
    cases = [
        # renamed expected tensor (container stays valid)
        (mutated(entries, index["language_model.model.layers.3.mlp.up_proj.weight"],
                 name="language_model.model.layers.3.mlp.upp_proj.weight"), False),
        # norm stored as F32 of the same byte size
        (mutated(entries, index["language_model.model.norm.weight"], dtype="F32",
                 shape=[1536]), False),
        # transposed q shape, same bytes
        (mutated(entries, index[q7 + "weight"], shape=[3072, 4096]), False),
        # embedding as F8 of the same bytes
        (mutated(entries, index["language_model.model.embed_tokens.weight"], dtype="F8_E4M3",
                 shape=[131072, 6144]), False),
        # companion rank 1
        (mutated(entries, index[q7 + "weight_scale_inv"], shape=[1]), False),
        # companion moved out of the text namespace (missing)
        (mutated(entries, index[q7 + "activation_scale"], name="vision.q7_activation_scale"),
         False),
        # unknown text tensor (the companion renamed inside the namespace)
        (mutated(entries, index[q7 + "activation_scale"],
                 name="language_model.model.layers.7.extra"), False),
        # scale values
        (mutated(entries, index[q7 + "weight_scale_inv"], payload=struct.pack("<H", 0)), False),
        (mutated(entries, index[q7 + "weight_scale_inv"], payload=struct.pack("<H", 0xbc00)),
         False),
        (mutated(entries, index[q7 + "activation_scale"], payload=struct.pack("<H", 0x7f80)),
         False),
        (mutated(entries, index[q7 + "activation_scale"], payload=struct.pack("<H", 0x7fc1)),
         False),
        (mutated(entries, index[q7 + "weight_scale_inv"], payload=struct.pack("<H", 0x0001)),
         True),   # positive subnormal: accepted here, refused later by compact admission
    ]
    extra = [list(e) for e in entries] + [["vision_tower.patch.weight", "BF16", [3], b"\0" * 6,
                                           None]]
    cases.append((extra, True))
    for case, accepted in cases:
        write_sparse_model(path, case)
        assert contract_agree(ref, product, path)[0] == accepted


def test_create_from_path_rejects_before_device_work(product, tmp_path):
    err = ctypes.create_string_buffer(512)
    missing = str(tmp_path / "absent.safetensors")
    assert not product.lunelette_metal_create(missing.encode(), err, 512)
    assert b"safetensors" in err.value
    other = str(tmp_path / "other.safetensors")
    write_container(other, "{" + T("x", "BF16", [1], 0, 2) + "}", b"\0\0")
    assert not product.lunelette_metal_create(other.encode(), err, 512)
    assert b"embed_tokens" in err.value
