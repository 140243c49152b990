"""Product host logic on the CPU (no device needed):
- the C-ABI library loads and exports every function declared in include/*.h;
- lh_yarn / lh_query_factor equal the oracle bit for bit;
- greedy selection and the generation loop follow tests/test_generation.c;
- constructors reject invalid options/profiles/paths before any device work
  (tests/test_metal.m option cases, tests/test_metal_options.c);
- the synthetic generator is deterministic, slice-consistent, and draws only
  finite E4M3FN codes with BF16-exact scales in [0.01, 0.02].
"""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import synthetic as syn

import oracle_lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for header in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(header).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b((?:lunelette|lh)_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names - {"lunelette_logits_fn"}


def test_library_exports_every_declared_function(product):
    names = declared_functions()
    assert len(names) > 50
    missing = [n for n in sorted(names) if not hasattr(product, n)]
    assert not missing, missing


def exported(path):
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", path], stdout=subprocess.PIPE,
                         text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.split()[1:2] == ["T"]}


def test_shipped_library_exports_exactly_the_abi(product):
    """The shipped library exports the functions of include/*.h and nothing
    else: no internal launcher and no test seam. The test build exports the
    same plus the seams of lunelette_amd/csrc/lh_test_seams.h."""
    abi = declared_functions()
    assert exported(lh.LIBRARY) == abi
    seams = {n for n in exported(lh.TEST_LIBRARY) - abi}
    assert seams and all(n.startswith("lunelette_metal_test_") for n in seams), seams
    assert "lunelette_metal_test_inject" in seams


def test_yarn_and_query_factor_match_oracle(product, oracle):
    fp = ctypes.POINTER(ctypes.c_float)
    c = np.empty(128, np.float32)
    s = np.empty(128, np.float32)
    for position in list(range(0, 64)) + [4351, 16383, 16384, 17919, 32768, 262143]:
        assert product.lh_yarn(position, c.ctypes.data_as(fp), s.ctypes.data_as(fp)) == 0
        rc, oc, os_ = oracle_lib.yarn(position)
        assert np.array_equal(c.view(np.uint32), oc.view(np.uint32))
        assert np.array_equal(s.view(np.uint32), os_.view(np.uint32))
        assert product.lh_query_factor(position) == oracle.orc_query_factor(position)
    assert product.lh_yarn(262144, c.ctypes.data_as(fp), s.ctypes.data_as(fp)) != 0


def select(product, logits):
    token = ctypes.c_int64(-7)
    err = ctypes.create_string_buffer(128)
    rc = product.lunelette_select_greedy(logits.ctypes.data_as(lh.c_float_p),
                                         ctypes.byref(token), err, 128)
    return rc, token.value, err.value


def test_select_greedy_cases(product):
    z = np.zeros(131072, np.float32)
    z[0] = -0.0
    assert select(product, z)[:2] == (0, 0)
    z[0], z[1] = 0.0, -0.0
    assert select(product, z)[:2] == (0, 0)
    a = np.full(131072, -10, np.float32)
    a[42] = a[43] = -1
    assert select(product, a)[:2] == (0, 42)
    for bad in (np.nan, np.inf, -np.inf):
        b = np.zeros(131072, np.float32)
        b[131071] = bad
        rc, tok, err = select(product, b)
        assert rc == -1 and tok == -7 and err
    rc, tok, err = select(product, np.zeros(131072, np.float32))
    assert rc == 0 and err == b""


class FakeLogits:
    """tests/test_generation.c:10-41: ids 42/43 tie at -1 (lowest wins);
    mode 1 fails the 2nd call, 2 makes EOS (2) win the 2nd call, 3/4/5 put
    NaN/+Inf/-Inf in the last logit."""

    def __init__(self, initial, mode=0):
        self.calls, self.initial, self.mode = 0, initial, mode

        def cb(_ctx, ids, count, logits, _err, _cap):
            assert count == self.initial + self.calls
            if self.calls:
                assert ids[count - 1] == 42
            self.calls += 1
            if self.mode == 1 and self.calls == 2:
                return -1
            arr = np.ctypeslib.as_array(logits, shape=(131072,))
            arr[:] = -10
            arr[42] = arr[43] = -1
            if self.mode == 2 and self.calls == 2:
                arr[2] = 0
            if self.mode >= 3:
                arr[131071] = {3: np.nan, 4: np.inf, 5: -np.inf}[self.mode]
            return 0

        self.fn = lh.LOGITS_FN(cb)


def generate(product, fake, ids, n, budget, eos=2, context=None):
    cfg = lh.GenerationConfig(budget, eos)
    result = lh.GenerationResult()
    ctypes.memset(ctypes.byref(result), 0x55, ctypes.sizeof(result))
    before = bytes(result)
    err = ctypes.create_string_buffer(256)
    arr = (ctypes.c_int64 * max(len(ids), 1))(*ids)
    if context is None:
        rc = product.lunelette_generate_with_logits(fake.fn, None, arr, n, ctypes.byref(cfg),
                                                    ctypes.byref(result), err, 256)
    else:
        rc = product.lunelette_generate_with_logits_capacity(fake.fn, None, arr, n, context,
                                                             ctypes.byref(cfg),
                                                             ctypes.byref(result), err, 256)
    return rc, result, bytes(result) == before


def test_generation_loop_contract(product):
    ids = [2] + [0] * 4351  # prompt EOS is not a stop condition
    rc, r, _ = generate(product, FakeLogits(1), ids, 1, 3)
    assert rc == 0 and r.count == 3 and r.tokens[0] == 42 and r.stop == 0
    rc, r, _ = generate(product, FakeLogits(1, 2), ids, 1, 3)
    assert rc == 0 and r.count == 2 and r.tokens[1] == 2 and r.stop == 1
    rc, r, _ = generate(product, FakeLogits(254, 2), ids, 254, 2)
    assert rc == 0 and r.stop == 1 and r.count == 2  # EOS beats budget and context
    fake = FakeLogits(255)
    rc, r, _ = generate(product, fake, ids, 255, 3)
    assert rc == 0 and r.count == 1 and r.stop == 2 and fake.calls == 1
    fake = FakeLogits(256)
    rc, r, _ = generate(product, fake, ids, 256, 3)
    assert rc == 0 and r.count == 0 and fake.calls == 0 and r.stop == 2
    rc, r, unchanged = generate(product, FakeLogits(1), ids, 257, 3)
    assert rc == -1 and unchanged
    assert generate(product, FakeLogits(1), ids, 0, 3)[0] == -1
    for mode in (1, 3, 4, 5):
        rc, r, unchanged = generate(product, FakeLogits(1, mode), ids, 1, 3)
        assert rc == -1 and unchanged, mode
    fake = FakeLogits(1)
    rc, r, _ = generate(product, fake, ids, 1, 256)
    assert rc == 0 and r.count == 255 and fake.calls == 255 and r.stop == 2
    assert generate(product, FakeLogits(1), ids, 1, 257)[0] == -1
    fake = FakeLogits(1)
    rc, r, _ = generate(product, fake, ids, 1, 0)
    assert rc == 0 and r.count == 0 and fake.calls == 0 and r.stop == 0
    for bad_prompt in ([-1], [131072]):
        assert generate(product, FakeLogits(1), bad_prompt, 1, 1)[0] == -1
    for eos in (-1, 131072):
        assert generate(product, FakeLogits(1), ids, 1, 1, eos=eos)[0] == -1
    rc, r, _ = generate(product, FakeLogits(1), ids, 1, 1, eos=42)
    assert rc == 0 and r.count == 1 and r.stop == 1
    # Capacity-aware variant (tests/test_generation.c long cases).
    long_ids = [0] * 4352
    fake = FakeLogits(4096)
    rc, r, _ = generate(product, fake, long_ids, 4096, 256, context=4352)
    assert rc == 0 and r.count == 256 and r.stop == 0
    rc, r, _ = generate(product, FakeLogits(4351), long_ids, 4351, 3, context=4352)
    assert rc == 0 and r.count == 1 and r.stop == 2
    rc, r, _ = generate(product, FakeLogits(4350, 2), long_ids, 4350, 3, context=4352)
    assert rc == 0 and r.count == 2 and r.stop == 1
    for n, context in ((4353, 4352), (1, 257), (257, 256)):
        assert generate(product, FakeLogits(n), long_ids, n, 3, context=context)[0] == -1


def test_constructors_reject_before_device_work(product):
    err = ctypes.create_string_buffer(512)
    bad = lh.Options(7, lh.COMPACT_FP8_ARITHMETIC)
    assert not product.lunelette_metal_create_with_options(b"/nonexistent", ctypes.byref(bad),
                                                           err, 512)
    assert b"invalid prefill option" in err.value
    bad = lh.Options(lh.PREFILL_MPS, 9)
    assert not product.lunelette_metal_create_with_options(b"/nonexistent", ctypes.byref(bad),
                                                           err, 512)
    assert b"invalid strategy" in err.value
    assert not product.lunelette_metal_create_with_options(None, None, err, 512)
    assert b"path" in err.value
    assert not product.lunelette_metal_create(None, None, 0)
    for context, block in ((257, 256), (4352, 64), (4096, 256), (0, 0)):
        lim = lh.Limits(context, block)
        assert not product.lunelette_metal_create_configured(b"x", None, ctypes.byref(lim),
                                                             err, 512)
        assert b"profile" in err.value
    cfg = lh.SyntheticConfig(1, 0)
    assert not product.lunelette_metal_create_synthetic(ctypes.byref(cfg), None, None, err, 512)
    assert product.lunelette_metal_reset(None, None, 0) == -1
    product.lunelette_metal_destroy(None)
    product.lunelette_metal_checkpoint_destroy(None)
    assert product.lunelette_metal_get_limits(None, None) == -1
    assert product.lunelette_metal_get_memory(None, None) == -1


def test_synthetic_model_needs_a_device_here(product):
    if product.lh_device_count() > 0:
        pytest.skip("a device is visible")
    err = ctypes.create_string_buffer(512)
    cfg = lh.SyntheticConfig(1, 2)
    assert not product.lunelette_metal_create_synthetic(ctypes.byref(cfg), None, None, err, 512)
    assert b"no HIP device" in err.value


def test_synthetic_generator_properties(product):
    codes = syn.fp8(5, 3, 1000, 1000).reshape(-1)
    assert codes.max() <= 254 and not np.any((codes & 127) == 127)
    counts = np.bincount(codes, minlength=256)
    assert counts[127] == 0 and counts[255] == 0
    finite = counts[[c for c in range(256) if (c & 127) != 127]]
    assert finite.min() > 3000 and finite.max() < 5000  # ~3937 each
    # Slices are reproducible from any offset.
    whole = syn.fp8(5, 3, 1, 5000).reshape(-1)
    part = syn.fp8(5, 3, 1, 1000, offset=2000).reshape(-1)
    assert np.array_equal(whole[2000:3000], part)
    x = syn.normal_f32(5, 4, 1 << 20)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    g = syn.bf16_to_f32(syn.normal_bf16(5, 6, 1 << 16, 1.0, 0.02))
    assert abs(g.mean() - 1) < 1e-3 and abs(g.std() - 0.02) < 1e-3
    for tensor in range(2, 240):
        s = np.float32(syn.scale(9, tensor))
        assert 0.01 <= s <= 0.02 and (s.view(np.uint32) & 0xffff) == 0
    t = syn.tokens(5, 1, 100000)
    assert t.min() >= 0 and t.max() < 131072 and 68000 < len(np.unique(t)) < 72000
    assert np.array_equal(syn.tokens(5, 1, 10), syn.tokens(5, 1, 10))
