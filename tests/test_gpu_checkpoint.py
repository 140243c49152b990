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
from lunelette_amd.runtime import Runtime
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
