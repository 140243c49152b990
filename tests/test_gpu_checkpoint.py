"""Checkpoint loading on the GPU: the seeded synthetic 26-layer model written
as an FP8 safetensors checkpoint (tests/checkpoint_files.py: the same bytes
lunelette_metal_create_synthetic uploads, per-tensor BF16 weight_scale_inv)
and loaded through lunelette_metal_create_configured(path) must behave
bitwise like the synthetic context: a 300-token prefill in two chunks (both
prefill modes, compact arithmetic and resident FP32 strategies) and 8 greedy
decode steps give identical logits. The memory report counts the same bytes.
The file is 3.83 GB, written under the pytest temporary directory.
"""
import os
import shutil

import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import synthetic as syn
from lunelette_amd.runtime import Runtime, RuntimeError_
from checkpoint_files import write_synthetic_model

pytestmark = pytest.mark.gpu
SEED = 20251201


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory, gpu):
    folder = tmp_path_factory.mktemp("checkpoint")
    if shutil.disk_usage(str(folder)).free < (6 << 30):
        pytest.skip("less than 6 GiB free for the 3.8 GB checkpoint file")
    path = str(folder / "synthetic.safetensors")
    size = write_synthetic_model(path, lh, SEED)
    print("checkpoint file: %.2f GB" % (size / 1e9), flush=True)
    yield path
    os.remove(path)


def run(rt, prompt, steps):
    out = [rt.prefill(prompt[:256]), rt.append(prompt[256:])]
    token = int(np.argmax(out[-1]))
    for _ in range(steps):
        out.append(rt.decode(token))
        token = int(np.argmax(out[-1]))
    return out


@pytest.mark.parametrize("prefill,strategy", [
    (lh.PREFILL_MPS, lh.COMPACT_FP8_ARITHMETIC),
    (lh.PREFILL_CUSTOM, lh.COMPACT_FP8_ARITHMETIC),
    (lh.PREFILL_CUSTOM, lh.RESIDENT_FP32),
])
def test_checkpoint_equals_synthetic(checkpoint, prefill, strategy):
    prompt = syn.tokens(SEED, 3, 300)
    with Runtime(path=checkpoint, context=4352, block=256, prefill=prefill,
                 strategy=strategy) as loaded:
        got = run(loaded, prompt, 8)
        memory_loaded = loaded.memory()
    with Runtime(seed=SEED, layers=26, context=4352, block=256, prefill=prefill,
                 strategy=strategy) as synthetic:
        want = run(synthetic, prompt, 8)
        memory_synthetic = synthetic.memory()
    for a, b in zip(got, want):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert memory_loaded == memory_synthetic


def sparse_checkpoint(path, slot_scale=None, payload=None):
    """A full-size checkpoint that is all holes (zero codes, zero BF16) except
    the scale companions and `payload` = (slot, bytes) at the start of one
    FP8 tensor. slot_scale = (slot, BF16 bits) overrides one scale."""
    from checkpoint_files import bf16_bits, model_entries, slot_tensors, write_sparse_model
    scales = {slot: (0x3c00, bf16_bits(1.0)) for slot, _, dtype, _ in slot_tensors()
              if dtype == "F8_E4M3"}
    if slot_scale:
        scales[slot_scale[0]] = (slot_scale[1], bf16_bits(1.0))
    entries = model_entries(scales)
    if payload:
        for entry in entries:
            if entry[4] == payload[0]:
                entry[3] = payload[1]
    write_sparse_model(path, entries)


@pytest.mark.parametrize("code", [0x7f, 0xff])
def test_nan_code_checkpoint_refused_for_every_strategy(gpu, tmp_path, code):
    """A NaN code in layer 0's q_proj: every strategy refuses the checkpoint
    while uploading (src/metal_weights.c:174-231, st_load_fp8), and create
    returns no context."""
    path = str(tmp_path / "nan.safetensors")
    sparse_checkpoint(path, payload=(3, bytes([0x38] * 5 + [code])))
    for strategy in (lh.COMPACT_FP8_ARITHMETIC, lh.COMPACT_FP8_LOOKUP, lh.RESIDENT_FP32):
        with pytest.raises(RuntimeError_, match="byte 5 code 0x%02x" % code):
            Runtime(path=path, context=256, block=256, strategy=strategy)
    os.remove(path)


def test_subnormal_products_load_resident_only(gpu, tmp_path):
    """Scale 2^-126 on layer 0's q_proj with code 0x01 (2^-9): the product is
    subnormal. The compact strategies refuse it (normal products only); the
    resident strategy accepts it as st_load_fp8 does and runs."""
    path = str(tmp_path / "subnormal.safetensors")
    sparse_checkpoint(path, slot_scale=(3, 0x0080), payload=(3, bytes([0x01, 0x81, 0x38])))
    for strategy in (lh.COMPACT_FP8_ARITHMETIC, lh.COMPACT_FP8_LOOKUP):
        with pytest.raises(RuntimeError_, match="byte 0 code 0x01"):
            Runtime(path=path, context=256, block=256, strategy=strategy)
    with Runtime(path=path, context=256, block=256, strategy=lh.RESIDENT_FP32) as rt:
        logits = rt.prefill([1, 2, 3])
        assert np.all(np.isfinite(logits))
    os.remove(path)
