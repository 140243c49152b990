"""MFMA block-projection path (PREFILL_MPS) on the GPU.

The reference's own MPS path is pinned only by tolerance (tests/test_metal.m:
200-259: |err| <= 2e-4 + 1e-4|ref| vs double); this path is held tighter:
- lh_fp8_gemm vs double: |err| <= 2e-6 * sum_c |w x| (exact BF16 operands,
  FP32 accumulation), output guard untouched;
- one decoder layer of 256 tokens after a 4096-token prefix vs the
  oracle: activations within 1e-3 of the row max-abs (median relative
  <= 1e-5), appended K/V rows within 1e-5 of the row max-abs;
- runtime prefill of a 2-layer model in MPS mode: logits within 1e-3 of the
  logit range of the precise oracle and the same greedy token, continuing
  into decode;
- matrix-core attention (FP32 MFMA, online softmax) vs the oracle's
  reference-literal and mirror schedules: |err| <= 2e-4 for unit-scale
  values over 1..69 blocks, ragged token tiles and the causal sentinel of
  tests/test_metal.m:956-999.
"""
import math

import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import synthetic as syn
from lunelette_amd.runtime import Runtime

import gpu_util
import oracle_lib
from oracle_lib import MIRROR, REF

pytestmark = pytest.mark.gpu
SEED = 99173


def run_gemm(gpu, w, scale, x, rows, cols, tokens, block=256):
    ws = gpu.lh_workspace_create(4352, block)
    assert ws, lh.last_error()
    try:
        d_w = lh.DeviceBuffer.from_array(w)
        d_x = lh.DeviceBuffer.from_array(x)
        d_y = lh.DeviceBuffer(tokens * rows * 4 + 64)
        lh.check(gpu.lh_memset_device(d_y.ptr, 0x5a, d_y.nbytes))
        lh.check(gpu.lh_fp8_gemm(ws, d_w.ptr, scale, d_x.ptr, d_y.ptr, rows, cols, tokens, None),
                 "fp8_gemm")
        raw = d_y.download(np.uint8)
        assert np.all(raw[tokens * rows * 4:] == 0x5a)
        return raw[:tokens * rows * 4].view(np.float32).reshape(tokens, rows)
    finally:
        gpu.lh_workspace_destroy(ws)


@pytest.mark.parametrize("rows,cols,tokens,block", [(3072, 3072, 256, 256), (1024, 4096, 37, 256),
                                                    (512, 9216, 5, 5), (3072, 9216, 256, 256),
                                                    (2048, 256, 100, 128)])
def test_fp8_gemm_vs_double(gpu, rows, cols, tokens, block):
    w = syn.fp8(SEED, 700 + rows, rows, cols)
    x = (syn.normal_f32(SEED, 701, tokens * cols) * 3).astype(np.float32)
    scale = 0.0146484375
    got = run_gemm(gpu, w, scale, x, rows, cols, tokens, block)
    table = gpu_util.decode_table() * np.float32(scale)
    wf = table[w].astype(np.float64)
    xx = x.reshape(tokens, cols).astype(np.float64)
    expected = xx @ wf.T
    magnitude = np.abs(xx) @ np.abs(wf).T
    assert np.all(np.abs(got - expected) <= 2e-6 * magnitude)


def test_rejects_unsupported_gemm_shapes(gpu):
    ws = gpu.lh_workspace_create(256, 16)
    try:
        d = lh.DeviceBuffer(1 << 20)
        for rows, cols, tokens in ((100, 3072, 1), (3072, 100, 1), (512, 256, 17), (4096, 256, 1)):
            assert gpu.lh_fp8_gemm(ws, d.ptr, 1.0, d.ptr, d.ptr, rows, cols, tokens, None) == -1
    finally:
        gpu.lh_workspace_destroy(ws)


def test_mfma_layer_256_after_4096(gpu):
    from test_gpu_layer import oracle_layer, run_layer
    host = syn.layer(SEED, 0)
    length, count, capacity = 4096, 256, 4352
    x = syn.normal_f32(SEED, 9001, count * 3072)
    kpm = syn.normal_f32(SEED, 9002, length * 1024).reshape(length, 1024)
    vpm = syn.normal_f32(SEED, 9003, length * 1024).reshape(length, 1024)
    got = run_layer(gpu, host, x, kpm, vpm, length, count, capacity, lh.PATH_MFMA)
    for schedule in (MIRROR, REF):
        want = oracle_layer(host, x, kpm, vpm, length, count, capacity, schedule)
        gx, wx = got[0].reshape(count, 3072), want[0].reshape(count, 3072)
        rowmax = np.max(np.abs(wx), axis=1, keepdims=True)
        assert np.max(np.abs(gx - wx) / rowmax) < 1e-3
        assert np.median(np.abs(gx - wx) / np.maximum(np.abs(wx), 1e-30)) < 1e-5
        for g, w_ in zip(got[1:], want[1:]):
            assert np.max(np.abs(g - w_) / np.max(np.abs(w_), axis=1, keepdims=True)) < 1e-5


@pytest.mark.parametrize("length,count", [(3, 5), (40, 100), (7, 130)])
def test_mfma_layer_small_odd_block(gpu, length, count):
    """One, two and three 64-token tiles, the last partial (the gate|up
    stream-K partition takes 36, 30 and 21 groups per XCD there)."""
    from test_gpu_layer import oracle_layer, run_layer
    host = syn.layer(SEED, 1)
    capacity = 256
    x = syn.normal_f32(SEED, 9101, count * 3072)
    kpm = syn.normal_f32(SEED, 9102, length * 1024).reshape(length, 1024)
    vpm = syn.normal_f32(SEED, 9103, length * 1024).reshape(length, 1024)
    got = run_layer(gpu, host, x, kpm, vpm, length, count, capacity, lh.PATH_MFMA)
    want = oracle_layer(host, x, kpm, vpm, length, count, capacity, MIRROR)
    gx, wx = got[0].reshape(count, 3072), want[0].reshape(count, 3072)
    assert np.max(np.abs(gx - wx) / np.max(np.abs(wx), axis=1, keepdims=True)) < 1e-3


@pytest.mark.parametrize("prompt", [64, 200])
def test_runtime_mps_prefill_then_decode(gpu, prompt):
    """Chained layers (each layer's last kernel splits the next layer's
    input); 200 tokens end in a partial 64-token GEMM tile."""
    from test_gpu_runtime import LAYERS, SEED as RSEED, oracle_model
    embedding = syn.embedding(RSEED)
    host = (embedding, syn.final_norm(RSEED), [syn.layer(RSEED, i) for i in range(LAYERS)])
    model = oracle_model(host)
    ids = syn.tokens(RSEED, 11, prompt)
    with Runtime(seed=RSEED, layers=LAYERS, context=256, block=256,
                 prefill=lh.PREFILL_MPS) as rt:
        got = rt.prefill(ids)
        want = model.forward(MIRROR, ids, 0)
        span = float(want.max() - want.min())
        assert np.max(np.abs(got - want)) <= 1e-3 * span
        token = rt.greedy()
        assert token == int(np.argmax(want))
        length = len(ids)
        for _ in range(4):
            got = rt.decode(token)
            want = model.forward(MIRROR, [token], length)
            assert np.max(np.abs(got - want)) <= 1e-3 * float(want.max() - want.min())
            assert rt.greedy() == int(np.argmax(want))
            token = rt.greedy()
            length += 1


@pytest.mark.parametrize("length,count,capacity", [(0, 5, 256), (60, 3, 256), (0, 256, 256),
                                                   (256, 256, 4352), (1000, 17, 4352),
                                                   (4096, 256, 4352), (2048, 128, 4352),
                                                   (2048, 130, 4352), (3001, 211, 4352),
                                                   (2000, 20, 4352)])
def test_attention_mfma_vs_oracle(gpu, length, count, capacity):
    """From a 2048-token prefix and 128 tokens on, the wide kernel runs (64
    tokens per workgroup); 130 and 211 tokens leave subtiles past the last
    token, and 2048 + 128 is the smallest such launch. The merge runs with
    4 (256 tokens), 8 (the wide kernel at 256), 10 and 16 (1000 + 17) and 32
    (2000 + 20) KV splits."""
    rng = np.random.default_rng(length + 7 * count)
    total = length + count
    q = (rng.normal(size=count * 4096) * 3).astype(np.float32)
    kpm = rng.normal(size=(total, 1024)).astype(np.float32)
    vpm = rng.normal(size=(total, 1024)).astype(np.float32)
    got = gpu_util.attention_on_device(gpu, gpu.lh_attention_mfma, q, kpm, vpm, length, count,
                                       capacity)
    mirror = oracle_lib.attention(MIRROR, q, kpm.reshape(-1), vpm.reshape(-1), 128, 1024,
                                  length, count)
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - mirror)) < 2e-4, (length, count)
    if total <= 1024:
        ref = oracle_lib.attention(REF, q, kpm.reshape(-1), vpm.reshape(-1), 128, 1024,
                                   length, count)
        assert np.max(np.abs(got - ref)) < 2e-4, (length, count)


def test_attention_mfma_causal_sentinel(gpu):
    """tests/test_metal.m:956-999 through the matrix-core kernel: zero q and K,
    V rows of 1 except 4352 in the last row; row 0 masks it (1.0), row 1
    includes it (8703/4352)."""
    capacity, count = 4352, 2
    length = capacity - count
    q = np.zeros(count * 4096, np.float32)
    kpm = np.zeros((capacity, 1024), np.float32)
    vpm = np.ones((capacity, 1024), np.float32)
    vpm[capacity - 1] = 4352.0
    got = gpu_util.attention_on_device(gpu, gpu.lh_attention_mfma, q, kpm, vpm, length, count,
                                       capacity)
    assert np.max(np.abs(got[:4096] - 1.0)) < 2e-4
    assert np.max(np.abs(got[4096:] - 8703.0 / 4352)) < 2e-4


@pytest.mark.parametrize("shift", [14, -14])
def test_mfma_layer_down_input_range(gpu, shift):
    """gate and up scales times 2^shift put SiLU(gate)*up up to about 1e13
    (far past FP16's 65504) or below about 1e-4 (mostly FP16 subnormals):
    the down projection's two FP16 planes carry a power-of-two scale per token
    and K split, so the layer stays within the matrix-core layer tolerance
    of the oracle."""
    from test_gpu_layer import oracle_layer, run_layer
    host = dict(syn.layer(SEED, 2))
    for name in ("scale_gate", "scale_up"):
        host[name] = math.ldexp(host[name], shift)   # exact: still BF16-exact and normal
    length, count, capacity = 64, 128, 256
    x = syn.normal_f32(SEED, 9201, count * 3072)
    kpm = syn.normal_f32(SEED, 9202, length * 1024).reshape(length, 1024)
    vpm = syn.normal_f32(SEED, 9203, length * 1024).reshape(length, 1024)
    got = run_layer(gpu, host, x, kpm, vpm, length, count, capacity, lh.PATH_MFMA)
    want = oracle_layer(host, x, kpm, vpm, length, count, capacity, MIRROR)
    gx, wx = got[0].reshape(count, 3072), want[0].reshape(count, 3072)
    assert np.isfinite(gx).all()
    rowmax = np.max(np.abs(wx), axis=1, keepdims=True)
    assert np.max(np.abs(gx - wx) / rowmax) < 1e-3
    assert np.median(np.abs(gx - wx) / np.maximum(np.abs(wx), 1e-30)) < 1e-5


def test_mfma_layer_down_granule_gap(gpu):
    """Adjacent 576-column granules of the down input whose largest values
    lie more than 2^100 apart: every gate row of granules 5 and 11 is the code
    -1.0 and the MLP input is positive, so those gates sit near -80 and
    SiLU(gate) * up near 2^-100 there, against about 2^17 in the granules
    before them. A stream-K segment that crosses such a boundary must not
    carry its accumulator over by the ratio of the granules' scales (it would
    overflow FP32); the layer stays finite and within the matrix-core layer
    tolerance of the oracle."""
    from test_gpu_layer import oracle_layer, run_layer
    host = dict(syn.layer(SEED, 3))
    length, count, capacity = 64, 192, 256
    rng = np.random.default_rng(77)
    x = (np.abs(rng.normal(size=count * 3072)) + 0.5).astype(np.float32)
    # o's output 2^-40 of its usual size: the MLP input stays x (positive).
    host["scale_o"] = math.ldexp(1.0, -46)
    gate = np.array(host["gate"])
    tiny = np.r_[5 * 576:6 * 576, 11 * 576:12 * 576]
    gate[tiny] = 0xB8
    host["gate"] = gate
    xx = x.reshape(count, 3072).astype(np.float64)
    gamma = syn.bf16_to_f32(host["post_norm"]).astype(np.float64)
    xn = xx / np.sqrt(np.mean(xx * xx, axis=1, keepdims=True) + 1e-5) * gamma
    host["scale_gate"] = float(np.float32(80.0 / np.median(xn.sum(axis=1))))
    dec = gpu_util.decode_table().astype(np.float64)
    g = host["scale_gate"] * (xn @ dec[gate].T)
    u = host["scale_up"] * (xn @ dec[host["up"]].T)
    silu = g * np.exp(-np.logaddexp(0.0, -g))
    y = np.abs(silu * u).reshape(count, 16, 576).max(axis=2)
    assert np.all(np.log2(y[:, 4] / y[:, 5]) > 100) and np.all(np.log2(y[:, 10] / y[:, 11]) > 100)
    kpm = syn.normal_f32(SEED, 9302, length * 1024).reshape(length, 1024)
    vpm = syn.normal_f32(SEED, 9303, length * 1024).reshape(length, 1024)
    got = run_layer(gpu, host, x, kpm, vpm, length, count, capacity, lh.PATH_MFMA)
    want = oracle_layer(host, x, kpm, vpm, length, count, capacity, MIRROR)
    gx, wx = got[0].reshape(count, 3072), want[0].reshape(count, 3072)
    assert np.isfinite(gx).all()
    rowmax = np.max(np.abs(wx), axis=1, keepdims=True)
    assert np.max(np.abs(gx - wx) / rowmax) < 1e-3
    assert np.median(np.abs(gx - wx) / np.maximum(np.abs(wx), 1e-30)) < 1e-5


@pytest.mark.parametrize("tail", [np.inf, np.nan], ids=["inf", "nan"])
@pytest.mark.parametrize("length,count,capacity", [(60, 3, 256), (256, 37, 4352),
                                                   (4000, 256, 4352)])
def test_attention_ignores_stale_cache_rows(gpu, tail, length, count, capacity):
    """Cache rows past length+count hold what an earlier sequence or a failed
    step left there (reset only rewinds the length). Both attention kernels
    must give the same result as over a clean cache: the precise kernel
    bitwise, the matrix-core kernel within its tolerance of the oracle (a
    masked weight of 0 times a stale Inf would be NaN)."""
    rng = np.random.default_rng(length + 3 * count)
    total = length + count
    q = (rng.normal(size=count * 4096) * 3).astype(np.float32)
    kpm = rng.normal(size=(total, 1024)).astype(np.float32)
    vpm = rng.normal(size=(total, 1024)).astype(np.float32)
    clean = gpu_util.attention_on_device(gpu, gpu.lh_attention, q, kpm, vpm, length, count,
                                         capacity)
    stale = gpu_util.attention_on_device(gpu, gpu.lh_attention, q, kpm, vpm, length, count,
                                         capacity, tail=tail)
    assert np.array_equal(clean.view(np.uint32), stale.view(np.uint32))
    got = gpu_util.attention_on_device(gpu, gpu.lh_attention_mfma, q, kpm, vpm, length, count,
                                       capacity, tail=tail)
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - clean)) < 2e-4


def test_attention_mfma_seeded_shapes(gpu):
    """Seeded random (prefix, chunk) shapes: both kernels (32-token tiles, and
    64-token tiles from a 2048-token prefix and 128 tokens on), 1 to 32 KV
    splits with ragged last splits, ragged token tiles; within 2e-4 of the
    mirror."""
    rng = np.random.default_rng(20251203)
    capacity = 4352
    for i in range(16):
        if i % 2:   # the wide kernel's range
            count = int(rng.integers(128, 161))
            length = int(rng.integers(2048, capacity - count + 1))
        else:
            count = int(rng.integers(1, 161))
            length = int(rng.integers(0, capacity - count + 1))
        total = length + count
        q = (rng.normal(size=count * 4096) * 3).astype(np.float32)
        kpm = rng.normal(size=(total, 1024)).astype(np.float32)
        vpm = rng.normal(size=(total, 1024)).astype(np.float32)
        got = gpu_util.attention_on_device(gpu, gpu.lh_attention_mfma, q, kpm, vpm, length, count,
                                           capacity)
        mirror = oracle_lib.attention(MIRROR, q, kpm.reshape(-1), vpm.reshape(-1), 128, 1024,
                                      length, count)
        assert np.all(np.isfinite(got)), (length, count)
        assert np.max(np.abs(got - mirror)) < 2e-4, (length, count)


def test_mfma_layer_seeded_shapes(gpu):
    """Seeded random prefixes and chunk sizes through the whole matrix-core
    layer (ragged 64-token tiles, every stream-K partition of gate|up and
    down that those counts produce, short and long prefixes), within 1e-3 of
    each row's largest magnitude of the mirror schedule."""
    from test_gpu_layer import oracle_layer, run_layer
    host = syn.layer(SEED, 2)
    rng = np.random.default_rng(20251204)
    capacity = 4352
    for i in range(12):
        count = int(rng.integers(2, 257))
        length = int(rng.integers(0, capacity - count + 1))
        x = syn.normal_f32(SEED, 9200 + i, count * 3072)
        kpm = rng.normal(size=(length, 1024)).astype(np.float32)
        vpm = rng.normal(size=(length, 1024)).astype(np.float32)
        got = run_layer(gpu, host, x, kpm, vpm, length, count, capacity, lh.PATH_MFMA)
        want = oracle_layer(host, x, kpm, vpm, length, count, capacity, MIRROR)
        gx, wx = got[0].reshape(count, 3072), want[0].reshape(count, 3072)
        err = np.max(np.abs(gx - wx) / np.max(np.abs(wx), axis=1, keepdims=True))
        assert err < 1e-3, (length, count, err)
