"""lh_attention_noalloc (the entry point that allocates nothing) against
lh_attention (workspace scratch) through the C-ABI: bitwise equal outputs on
two calls in a row, the second smaller than the first (the static scratch
keeps the first call's partials), across decode and multi-token shapes; sizes
beyond the static scratch are refused before any device work."""
import ctypes

import numpy as np
import pytest

import lunelette_amd as lh
import gpu_util

pytestmark = pytest.mark.gpu


def run_noalloc(gpu, q, kpm, vpm, length, count, capacity):
    d_q = lh.DeviceBuffer.from_array(q)
    keys = lh.DeviceBuffer.from_array(gpu_util.keys_to_device(kpm, capacity))
    values = lh.DeviceBuffer.from_array(gpu_util.kv_to_device_layout(vpm, capacity))
    out = lh.DeviceBuffer(count * 4096 * 4 + 16)
    lh.check(gpu.lh_memset_device(out.ptr, 0x5a, out.nbytes))
    lh.check(gpu.lh_attention_noalloc(d_q.ptr, keys.ptr, values.ptr, length, count, capacity,
                                      out.ptr, None), "attention_noalloc")
    lh.check(gpu.lh_device_synchronize())
    raw = out.download(np.uint8)
    assert np.all(raw[count * 4096 * 4:] == 0x5a), "wrote past the output"
    return raw[:count * 4096 * 4].view(np.float32)


def case(seed, length, count):
    rng = np.random.default_rng(seed)
    total = length + count
    q = (rng.normal(size=count * 4096) * 3).astype(np.float32)
    return q, rng.normal(size=(total, 1024)).astype(np.float32), rng.normal(
        size=(total, 1024)).astype(np.float32)


@pytest.mark.parametrize("first,second", [((4351, 1, 4352), (550, 1, 4352)),
                                          ((16000, 4, 16384), (63, 2, 256)),
                                          ((1000, 17, 2048), (64, 1, 128))])
def test_noalloc_attention_equals_workspace_attention(gpu, first, second):
    for seed, (length, count, capacity) in enumerate((first, second)):
        q, kpm, vpm = case(seed + length, length, count)
        want = gpu_util.attention_on_device(gpu, gpu.lh_attention, q, kpm, vpm, length, count,
                                            capacity)
        got = run_noalloc(gpu, q, kpm, vpm, length, count, capacity)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (length, count)


def test_noalloc_attention_refuses_oversize(gpu):
    d = lh.DeviceBuffer(1 << 20)
    assert gpu.lh_attention_noalloc(d.ptr, d.ptr, d.ptr, 0, 5, 16384, d.ptr, None) == -1
    assert "static scratch" in lh.last_error()
    assert gpu.lh_attention_noalloc(d.ptr, d.ptr, d.ptr, 10, 1, 100, d.ptr, None) == -1
    assert gpu.lh_attention_noalloc(d.ptr, d.ptr, d.ptr, 128, 1, 128, d.ptr, None) == -1
