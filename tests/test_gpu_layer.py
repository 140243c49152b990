"""GPU parity of one decoder layer through the kernel-level C-ABI
lh_layer_forward.

Decode: one token at position 4351 over a 4351-entry N(0,1) FP32
KV cache, seeded FP8 weights with per-tensor scales in [0.01, 0.02].
Prefill (precise path): a 256-token chunk appended after a 4096-token prefix
with causal masking inside the chunk.
The fused, lookup, unfused and resident-FP32 paths must give identical bits,
equal to the oracle's device-mirror schedule; the reference-literal schedule
agrees within the stated activation tolerance, 1e-3 of the row's max-abs
(a near-tie in an effectively one-hot softmax can move one head's output by a
few units), with the median element within 1e-6 relative. Appended K/V rows
are checked too.
"""
import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import synthetic as syn

import gpu_util
import oracle_lib
from oracle_lib import MIRROR, REF

pytestmark = pytest.mark.gpu

SEED = 20251201


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def layer_host():
    return syn.layer(SEED, 0)


def run_layer(gpu, host, x, kv_prefix_k, kv_prefix_v, length, count, capacity, path,
              resident=False):
    dev = gpu_util.DeviceLayer(host, resident=resident)
    keys = lh.DeviceBuffer.from_array(gpu_util.keys_to_device(kv_prefix_k, capacity))
    values = lh.DeviceBuffer.from_array(gpu_util.kv_to_device_layout(kv_prefix_v, capacity))
    d_x = lh.DeviceBuffer.from_array(x)
    ws = gpu.lh_workspace_create(capacity, max(count, 1))
    assert ws, lh.last_error()
    try:
        ids = np.zeros(count, np.int64)
        lh.check(gpu.lh_workspace_set_tokens(ws, ids.ctypes.data_as(lh.c_int64_p), length, count,
                                             None), "set_tokens")
        lh.check(gpu.lh_layer_forward(dev.weights, d_x.ptr, keys.ptr, values.ptr, ws, path, None),
                 "layer_forward")
        lh.check(gpu.lh_device_synchronize())
        out = d_x.download(np.float32)
        k = gpu_util.k_untile(keys.download(np.float32).reshape(8, capacity, 128))
        v = values.download(np.float32).reshape(8, capacity, 128)
    finally:
        gpu.lh_workspace_destroy(ws)
    return out, gpu_util.kv_from_device_layout(k, length, count), \
        gpu_util.kv_from_device_layout(v, length, count)


def oracle_layer(host, x, kpm, vpm, length, count, capacity, schedule):
    model = oracle_lib.HostModel(np.zeros(1, np.uint16), np.zeros(1, np.uint16), [host], capacity)
    model.keys[:] = gpu_util.kv_to_device_layout(kpm, capacity).reshape(-1)
    model.values[:] = gpu_util.kv_to_device_layout(vpm, capacity).reshape(-1)
    xo = np.array(x, np.float32)
    model.layer_forward(schedule, 0, xo, length, count)
    return xo, model.kv(0, 0, length, count), model.kv(0, 1, length, count)


def check_layer(gpu, host, length, count, capacity, paths):
    x = syn.normal_f32(SEED, 9001, count * 3072)
    kpm = syn.normal_f32(SEED, 9002, length * 1024).reshape(length, 1024)
    vpm = syn.normal_f32(SEED, 9003, length * 1024).reshape(length, 1024)
    mirror = oracle_layer(host, x, kpm, vpm, length, count, capacity, MIRROR)
    results = {}
    for path in paths:
        resident = path == lh.PATH_RESIDENT
        results[path] = run_layer(gpu, host, x, kpm, vpm, length, count, capacity, path, resident)
        for got, want, name in zip(results[path], mirror, ("x", "k", "v")):
            assert np.array_equal(bits(got), bits(want)), (path, name)
    ref = oracle_layer(host, x, kpm, vpm, length, count, capacity, REF)
    got = results[paths[0]][0].reshape(count, 3072)
    want = ref[0].reshape(count, 3072)
    scale = np.max(np.abs(want), axis=1, keepdims=True)
    assert np.max(np.abs(got - want) / scale) < 1e-3
    assert np.median(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) < 1e-6


def test_decode_layer_pos4351_all_paths(gpu, layer_host):
    check_layer(gpu, layer_host, 4351, 1, 4352,
                [lh.PATH_FUSED, lh.PATH_LOOKUP, lh.PATH_UNFUSED, lh.PATH_RESIDENT])


def test_decode_layer_short_prefix(gpu, layer_host):
    for length in (0, 1, 63, 64, 65, 255, 256, 257):
        check_layer(gpu, layer_host, length, 1, 4352, [lh.PATH_FUSED])


def test_decode_layer_one_launch_boundaries(gpu, layer_host):
    """A decode token's q|k|v projection and attention blocks share one
    launch; its blocks combine in that launch up to 16 blocks and through
    k_attn_combine past it: both sides, both FP8 strategies, bitwise."""
    for length in (1023, 1024, 2047):
        check_layer(gpu, layer_host, length, 1, 4352, [lh.PATH_FUSED, lh.PATH_LOOKUP])


def test_prefill_chunk_256_after_4096_precise_path(gpu, layer_host):
    check_layer(gpu, layer_host, 4096, 256, 4352, [lh.PATH_FUSED])


def test_prefill_chunk_small(gpu, layer_host):
    check_layer(gpu, layer_host, 3, 5, 256, [lh.PATH_FUSED, lh.PATH_UNFUSED])


def attention_on_device(gpu, q, kpm, vpm, length, count, capacity):
    ws = gpu.lh_workspace_create(capacity, count)
    assert ws, lh.last_error()
    try:
        ids = np.zeros(count, np.int64)
        lh.check(gpu.lh_workspace_set_tokens(ws, ids.ctypes.data_as(lh.c_int64_p), length, count,
                                             None))
        d_q = lh.DeviceBuffer.from_array(q)
        keys = lh.DeviceBuffer.from_array(gpu_util.keys_to_device(kpm, capacity))
        values = lh.DeviceBuffer.from_array(gpu_util.kv_to_device_layout(vpm, capacity))
        out = lh.DeviceBuffer(count * 4096 * 4 + 16)
        lh.check(gpu.lh_memset_device(out.ptr, 0x5a, out.nbytes))
        lh.check(gpu.lh_attention(d_q.ptr, keys.ptr, values.ptr, ws, out.ptr, None))
        raw = out.download(np.uint8)
        assert np.all(raw[count * 4096 * 4:] == 0x5a)
        return raw[:count * 4096 * 4].view(np.float32)
    finally:
        gpu.lh_workspace_destroy(ws)


def test_attention_repeated_launches_one_workspace(gpu):
    """The per-(token, kv head) arrival counters return to zero after every
    launch: successive calls with different lengths and counts in one
    workspace stay bitwise equal to the mirror."""
    rng = np.random.default_rng(21)
    capacity, block = 4352, 8
    total = 3000
    kpm = rng.normal(size=(total, 1024)).astype(np.float32)
    vpm = rng.normal(size=(total, 1024)).astype(np.float32)
    keys = lh.DeviceBuffer.from_array(gpu_util.keys_to_device(kpm, capacity))
    values = lh.DeviceBuffer.from_array(gpu_util.kv_to_device_layout(vpm, capacity))
    ws = gpu.lh_workspace_create(capacity, block)
    assert ws, lh.last_error()
    try:
        for length, count in ((2991, 8), (100, 1), (2999, 1), (64, 5), (2047, 2)):
            q = (rng.normal(size=count * 4096) * 2).astype(np.float32)
            ids = np.zeros(count, np.int64)
            lh.check(gpu.lh_workspace_set_tokens(ws, ids.ctypes.data_as(lh.c_int64_p), length,
                                                 count, None))
            d_q = lh.DeviceBuffer.from_array(q)
            out = lh.DeviceBuffer(count * 4096 * 4)
            lh.check(gpu.lh_attention(d_q.ptr, keys.ptr, values.ptr, ws, out.ptr, None))
            got = out.download(np.float32)
            mirror = oracle_lib.attention(MIRROR, q, kpm[:length + count].reshape(-1),
                                          vpm[:length + count].reshape(-1), 128, 1024,
                                          length, count)
            assert np.array_equal(bits(got), bits(mirror)), (length, count)
    finally:
        gpu.lh_workspace_destroy(ws)


def test_attention_fused_combine_boundary(gpu):
    """Block grids of up to 16 blocks run as one launch whose last-arriving
    workgroup per (token, kv head) combines (from its XCD's L2); 17 and more
    as blocks + combine. Both sides of the boundary, single and multi-token
    steps (one arrival word per token), bitwise the mirror."""
    rng = np.random.default_rng(33)
    capacity = 2048
    for length, count in ((0, 1), (63, 1), (64, 1), (511, 1), (1023, 1), (1024, 1),
                          (1000, 24), (1001, 24), (990, 32), (2000, 3)):
        total = length + count
        q = (rng.normal(size=count * 4096) * 3).astype(np.float32)
        kpm = rng.normal(size=(total, 1024)).astype(np.float32)
        vpm = rng.normal(size=(total, 1024)).astype(np.float32)
        got = attention_on_device(gpu, q, kpm, vpm, length, count, capacity)
        mirror = oracle_lib.attention(MIRROR, q, kpm.reshape(-1), vpm.reshape(-1), 128, 1024,
                                      length, count)
        assert np.array_equal(bits(got), bits(mirror)), (length, count)


def test_long_causal_sentinel_through_kernels(gpu):
    """tests/test_metal.m:956-999: zero q and K, V rows of 1 except a 4352
    sentinel in the last row; query row 0 must mask it (1.0), row 1 must
    include it with total stride C (8703/4352)."""
    capacity, count = 4352, 2
    length = capacity - count
    q = np.zeros(count * 4096, np.float32)
    kpm = np.zeros((capacity, 1024), np.float32)
    vpm = np.ones((capacity, 1024), np.float32)
    vpm[capacity - 1] = 4352.0
    got = attention_on_device(gpu, q, kpm, vpm, length, count, capacity)
    assert np.max(np.abs(got[:4096] - 1.0)) < 2e-4
    assert np.max(np.abs(got[4096:] - 8703.0 / 4352)) < 2e-4
    mirror = oracle_lib.attention(MIRROR, q, kpm.reshape(-1), vpm.reshape(-1), 128, 1024,
                                  length, count)
    assert np.array_equal(bits(got), bits(mirror))


def test_attention_random_bitwise_and_tolerance(gpu):
    rng = np.random.default_rng(12)
    # Block counts 1, 4, 68 (three combine windows), 32 and 33 (window edge),
    # 17-token causal chunks, and the 16K-prefix decode shape.
    for length, count, capacity in ((0, 1, 256), (200, 3, 256), (4351, 1, 4352),
                                    (1000, 17, 4352), (2047, 1, 2048), (2047, 3, 4352),
                                    (16383, 1, 17920)):
        total = length + count
        q = (rng.normal(size=count * 4096) * 3).astype(np.float32)
        kpm = rng.normal(size=(total, 1024)).astype(np.float32)
        vpm = rng.normal(size=(total, 1024)).astype(np.float32)
        got = attention_on_device(gpu, q, kpm, vpm, length, count, capacity)
        mirror = oracle_lib.attention(MIRROR, q, kpm.reshape(-1), vpm.reshape(-1), 128, 1024,
                                      length, count)
        assert np.array_equal(bits(got), bits(mirror)), (length, count)
        ref = oracle_lib.attention(REF, q, kpm.reshape(-1), vpm.reshape(-1), 128, 1024,
                                   length, count)
        assert np.max(np.abs(got - ref)) < 1e-4


def test_attention_seeded_lengths_bitwise(gpu):
    """Seeded random decode and small-chunk shapes across the whole 17920
    capacity: partial last blocks at every offset, one to three combine
    rounds (256 blocks each), bitwise the mirror schedule."""
    rng = np.random.default_rng(20251202)
    capacity = 17920
    cases = [(int(rng.integers(0, capacity - 8)), int(rng.choice([1, 1, 1, 2, 5])))
             for _ in range(20)]
    cases += [(16383, 2), (16447, 1), (17900, 3)]
    for length, count in cases:
        total = length + count
        q = (rng.normal(size=count * 4096) * 3).astype(np.float32)
        kpm = rng.normal(size=(total, 1024)).astype(np.float32)
        vpm = rng.normal(size=(total, 1024)).astype(np.float32)
        got = attention_on_device(gpu, q, kpm, vpm, length, count, capacity)
        mirror = oracle_lib.attention(MIRROR, q, kpm.reshape(-1), vpm.reshape(-1), 128, 1024,
                                      length, count)
        assert np.array_equal(bits(got), bits(mirror)), (length, count)


def test_decode_layer_seeded_lengths(gpu, layer_host):
    """Seeded random positions across the 17920 capacity (the query factor
    above 16384 included), fused and lookup paths bitwise the mirror."""
    rng = np.random.default_rng(20251205)
    for length in [int(v) for v in rng.integers(0, 17919, size=8)]:
        check_layer(gpu, layer_host, length, 1, 17920, [lh.PATH_FUSED, lh.PATH_LOOKUP])
