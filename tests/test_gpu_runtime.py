"""Runtime C-ABI on the GPU: model parity and the include/metal.h state machine.

Parity: a seeded 2-layer synthetic model (full 131072-token tied head) at
C256/B256; prefill and greedy decode logits are bit-identical to the oracle's
device-mirror schedule, and greedy tokens match.
Invariants from the reference's tests:
- compact arithmetic == compact lookup == resident FP32, bitwise
  (tests/test_metal_compact.m:97-235);
- restore + append == fresh replay, bitwise (tests/long_context/long/schedule.py:33-44);
- argument errors leave state untouched; execution/nonfinite failures
  invalidate until reset; checkpoint epochs/identity (tests/test_metal.m:629-860);
- KV prefix, suffix and tail bytes after restore/rebranch (tests/test_metal.m);
- a step that fails after some layers wrote their KV rows invalidates the
  sequence; after reset the same calls give bitwise the logits of a fresh
  context (tests/test_metal.m:629-860, encoder failures at every index);
- the N-th device or pinned allocation of create failing, for every N, returns
  NULL with a diagnostic and frees everything it had allocated
  (tests/test_metal.m:888-954);
- checkpoint epoch exhaustion refuses a new handle and keeps the active one
  (tests/test_metal.m:812-828).
The failure cases run on the test build of the library
(liblunelette_hip_test.so: the same objects plus the seams of
lunelette_amd/csrc/lh_test_seams.h); every fault is forced from the host.
"""
import math
import time

import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import synthetic as syn
from lunelette_amd.runtime import Runtime, RuntimeError_

import oracle_lib
from oracle_lib import MIRROR

pytestmark = pytest.mark.gpu

SEED = 424242
LAYERS = 2


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def host_model():
    embedding = syn.embedding(SEED)
    final = syn.final_norm(SEED)
    layers = [syn.layer(SEED, i) for i in range(LAYERS)]
    return embedding, final, layers


@pytest.fixture(scope="module")
def rt(gpu):
    r = Runtime(seed=SEED, layers=LAYERS, context=256, block=256, prefill=lh.PREFILL_CUSTOM)
    yield r
    r.close()


@pytest.fixture(scope="module")
def rts(gpu):
    """The same model on the test build, for host-forced failures."""
    r = Runtime(seed=SEED, layers=LAYERS, context=256, block=256, prefill=lh.PREFILL_CUSTOM,
                seams=True)
    yield r
    r.close()


def oracle_model(host_model, capacity=256):
    embedding, final, layers = host_model
    return oracle_lib.HostModel(embedding.reshape(-1), final, layers, capacity)


def test_prefill_and_decode_bitwise_vs_oracle(rt, host_model):
    ids = syn.tokens(SEED, 1, 7)
    model = oracle_model(host_model)
    rt.reset()
    got = rt.prefill(ids)
    want = model.forward(MIRROR, ids, 0)
    assert np.array_equal(bits(got), bits(want))
    token = rt.greedy()
    assert token == int(np.argmax(want))
    length = len(ids)
    for _ in range(3):
        got = rt.decode(token)
        want = model.forward(MIRROR, [token], length)
        assert np.array_equal(bits(got), bits(want))
        length += 1
        token = rt.greedy()
        assert token == int(np.argmax(want))
    # KV rows written by the device equal the oracle's, in the reference layout.
    for layer in range(LAYERS):
        for kind in (0, 1):
            assert np.array_equal(bits(rt.read_kv(layer, kind, 0, length)),
                                  bits(model.kv(layer, kind, 0, length)))


def test_prefill_equals_decode_chain_and_append(rt):
    ids = syn.tokens(SEED, 2, 9)
    rt.reset()
    whole = rt.prefill(ids)
    rt.reset()
    rt.prefill(ids[:1])
    for t in ids[1:]:
        chain = rt.decode(int(t))
    assert np.array_equal(bits(whole), bits(chain))
    rt.reset()
    rt.prefill(ids[:4])
    appended = rt.append(ids[4:])
    assert np.array_equal(bits(whole), bits(appended))


@pytest.mark.parametrize("strategy", [lh.COMPACT_FP8_LOOKUP, lh.RESIDENT_FP32])
def test_strategies_bitwise_equal(gpu, rt, strategy):
    ids = syn.tokens(SEED, 3, 5)
    rt.reset()
    base = rt.prefill(ids)
    base_next = rt.decode(17)
    with Runtime(seed=SEED, layers=LAYERS, context=256, block=256, prefill=lh.PREFILL_CUSTOM,
                 strategy=strategy) as other:
        assert np.array_equal(bits(other.prefill(ids)), bits(base))
        assert np.array_equal(bits(other.decode(17)), bits(base_next))
        mem = other.memory()
        assert mem["strategy"] == strategy


def test_restore_append_equals_fresh_replay(rt):
    prefix = syn.tokens(SEED, 4, 6)
    branches = [syn.tokens(SEED, 5, 3), syn.tokens(SEED, 6, 3)]
    rt.reset()
    rt.prefill(prefix)
    saved = rt.checkpoint()
    try:
        results = []
        for branch in branches:
            rt.restore(saved)
            results.append(rt.append(branch))
        for branch, got in zip(branches, results):
            rt.reset()
            rt.prefill(prefix)
            assert np.array_equal(bits(rt.append(branch)), bits(got))
    finally:
        rt.destroy_checkpoint(saved)


def test_argument_errors_leave_state(rt):
    rt.reset()
    with pytest.raises(RuntimeError_):
        rt.prefill(np.zeros(0, np.int64))
    with pytest.raises(RuntimeError_):
        rt.prefill(np.zeros(257, np.int64))
    for bad in (-1, 131072):
        with pytest.raises(RuntimeError_):
            rt.prefill([bad])
    with pytest.raises(RuntimeError_):
        rt.decode(0)  # empty sequence
    logits = rt.prefill([5])
    for bad in (-1, 131072):
        with pytest.raises(RuntimeError_):
            rt.decode(bad)
    with pytest.raises(RuntimeError_):
        rt.prefill([5])  # prefill needs an empty sequence
    # Still valid with length 1: a decode succeeds and equals a fresh chain.
    after = rt.decode(9)
    rt.reset()
    rt.prefill([5])
    assert np.array_equal(bits(rt.decode(9)), bits(after))
    assert np.all(np.isfinite(logits))


def test_execution_failure_invalidates_until_reset(rts):
    rt = rts
    rt.reset()
    rt.prefill([1, 2])
    rt.inject(1)
    with pytest.raises(RuntimeError_, match="reset required"):
        rt.decode(3)
    with pytest.raises(RuntimeError_):
        rt.decode(3)
    rt.reset()
    rt.inject(2)
    with pytest.raises(RuntimeError_, match="nonfinite"):
        rt.prefill([1])
    with pytest.raises(RuntimeError_):
        rt.append([2])
    rt.reset()
    rt.prefill([1])


def test_checkpoint_semantics(rts):
    rt = rts
    rt.reset()
    with pytest.raises(RuntimeError_):
        rt.checkpoint()  # no endpoint
    rt.prefill([3, 4, 5])
    rt.set_logit(0, -0.0)
    rt.set_logit(131071, 17.25)
    first = rt.checkpoint()
    saved = rt.restore(first)
    assert math.copysign(1, saved[0]) < 0 and saved[131071] == 17.25
    rt.append([6, 7])
    rt.decode(8)
    again = rt.restore(first)  # append/decode preserve the checkpoint
    assert np.array_equal(bits(again), bits(saved))
    second = rt.checkpoint()
    with pytest.raises(RuntimeError_):
        rt.restore(first)  # replaced handle is stale
    rt.inject(3)
    with pytest.raises(RuntimeError_):
        rt.checkpoint()  # allocation failure keeps the active handle
    assert np.array_equal(bits(rt.restore(second)), bits(saved))
    rt.set_logit(131071, float("nan"))
    with pytest.raises(RuntimeError_):
        rt.checkpoint()  # nonfinite endpoint invalidates sequence and checkpoint
    with pytest.raises(RuntimeError_):
        rt.restore(second)
    rt.reset()
    rt.prefill([3])
    third = rt.checkpoint()
    rt.reset()
    with pytest.raises(RuntimeError_):
        rt.restore(third)  # reset invalidates
    rt.prefill([3])
    rt.inject(1)
    fourth = rt.checkpoint()
    with pytest.raises(RuntimeError_):
        rt.append([4])
    with pytest.raises(RuntimeError_):
        rt.restore(fourth)  # execution failure invalidates
    for h in (first, second, third, fourth):
        rt.destroy_checkpoint(h)
    rt.reset()


def test_capacity_limits(rt):
    rt.reset()
    rt.prefill(np.arange(200, dtype=np.int64))
    rt.append(np.arange(54, dtype=np.int64))
    rt.decode(1)  # length 255
    rt.decode(2)  # length 256 == C
    with pytest.raises(RuntimeError_):
        rt.decode(3)
    rt.reset()
    rt.prefill(np.arange(255, dtype=np.int64))
    with pytest.raises(RuntimeError_):
        rt.append([1, 2])
    rt.append([1])


def test_kv_prefix_suffix_tail_after_rebranch(rt):
    rt.reset()
    rt.prefill([11, 12, 13])
    base = [rt.read_kv(l, k, 0, 3) for l in range(LAYERS) for k in (0, 1)]
    saved = rt.checkpoint()
    try:
        rt.append([14, 15, 16, 17])
        tail_a = [rt.read_kv(l, k, 3, 4) for l in range(LAYERS) for k in (0, 1)]
        rt.restore(saved)
        rt.append([21, 22])
        now = [rt.read_kv(l, k, 0, 7) for l in range(LAYERS) for k in (0, 1)]
        for b, a, n in zip(base, tail_a, now):
            assert np.array_equal(bits(n[:3]), bits(b))        # prefix kept
            assert not np.array_equal(bits(n[3:5]), bits(a[:2]))  # suffix rewritten
            assert np.array_equal(bits(n[5:7]), bits(a[2:4]))  # stale tail untouched
    finally:
        rt.destroy_checkpoint(saved)


def test_memory_and_limits(rt):
    assert rt.limits() == (256, 256)
    mem = rt.memory()
    assert mem["kv_bytes"] == 2 * LAYERS * 8 * 256 * 128 * 4
    fp8 = (6144 * 3072 + 3072 * 4096 + 2 * 9216 * 3072 + 3072 * 9216) * LAYERS
    assert mem["weight_bytes"] == fp8 + 131072 * 3072 * 2 + (2 * LAYERS + 1) * 3072 * 4
    assert mem["conversion_stage_bytes"] == 0
    assert mem["total_bytes"] == mem["weight_bytes"] + mem["scratch_bytes"] + mem["kv_bytes"]


@pytest.mark.parametrize("mode", [lh.PREFILL_CUSTOM, lh.PREFILL_MPS], ids=["precise", "mps"])
def test_failure_after_layer_then_reset_replays_bitwise(gpu, mode):
    """Each layer writes its K/V rows before the next runs; a step failing after
    layer 0 has written layer 0's rows for it. The sequence is invalid until
    reset, a checkpoint taken before is dead, and after reset the same calls
    give the logits of a fresh context bit for bit (the rows the failed step
    wrote are rewritten before any read)."""
    prompt = syn.tokens(SEED, 20, 40)
    with Runtime(seed=SEED, layers=LAYERS, context=256, block=256, prefill=mode) as fresh:
        want = [fresh.prefill(prompt), fresh.decode(7), fresh.append([8, 9, 10])]
    with Runtime(seed=SEED, layers=LAYERS, context=256, block=256, prefill=mode,
                 seams=True) as rt:
        rt.fail_after_layer(0)
        with pytest.raises(RuntimeError_, match="reset required"):
            rt.prefill(prompt)
        with pytest.raises(RuntimeError_):
            rt.decode(7)  # invalid until reset
        rt.reset()
        assert np.array_equal(bits(rt.prefill(prompt)), bits(want[0]))
        saved = rt.checkpoint()
        rt.fail_after_layer(LAYERS - 1)
        with pytest.raises(RuntimeError_, match="layer 1"):
            rt.decode(7)
        with pytest.raises(RuntimeError_):
            rt.restore(saved)  # the failure invalidated the checkpoint
        rt.destroy_checkpoint(saved)
        rt.reset()
        assert np.array_equal(bits(rt.prefill(prompt)), bits(want[0]))
        rt.fail_after_layer(0)
        with pytest.raises(RuntimeError_):
            rt.append([8, 9, 10])
        rt.reset()
        assert np.array_equal(bits(rt.prefill(prompt)), bits(want[0]))
        assert np.array_equal(bits(rt.decode(7)), bits(want[1]))
        assert np.array_equal(bits(rt.append([8, 9, 10])), bits(want[2]))
        with pytest.raises(RuntimeError_):
            rt.fail_after_layer(LAYERS)  # no such layer


def test_one_launch_attention_gives_up_then_reset_replays_bitwise(gpu):
    """A decode step's attention blocks share a launch with the q|k|v
    projection and wait, bounded, for its flags. The test build makes every
    such block of one step wait for flags that never come: each gives up
    after 64 polls and writes NaN partials, so the step reports a nonfinite
    logit and invalidates the sequence, and every kernel still ends. After
    reset (the arrival words and flags cleared) the same calls give the
    logits of a fresh context bit for bit."""
    prompt = syn.tokens(SEED, 21, 40)
    with Runtime(seed=SEED, layers=LAYERS, context=256, block=256,
                 prefill=lh.PREFILL_CUSTOM) as fresh:
        want = [fresh.prefill(prompt), fresh.decode(7), fresh.decode(8)]
    with Runtime(seed=SEED, layers=LAYERS, context=256, block=256, prefill=lh.PREFILL_CUSTOM,
                 seams=True) as rt:
        if not lh.test_lib().lunelette_metal_test_chained(len(prompt)):
            pytest.skip("this device runs the attention blocks in launches of their own")
        assert np.array_equal(bits(rt.prefill(prompt)), bits(want[0]))
        rt.inject(6)
        started = time.perf_counter()
        with pytest.raises(RuntimeError_, match="nonfinite"):
            rt.decode(7)
        assert time.perf_counter() - started < 10.0
        with pytest.raises(RuntimeError_):
            rt.decode(7)  # invalid until reset
        rt.reset()
        assert np.array_equal(bits(rt.prefill(prompt)), bits(want[0]))
        assert np.array_equal(bits(rt.decode(7)), bits(want[1]))
        assert np.array_equal(bits(rt.decode(8)), bits(want[2]))


@pytest.mark.parametrize("what,prompt_length,context", [
    (6, 1100, 4352),    # 18 blocks in the q|k|v launch: its blocks give up
    (7, 1100, 4352),    # 18 blocks in the q|k|v launch: its combiners give up
    (7, 4700, 17920),   # 74 blocks in the attention's own launch: its combiners give up
])
def test_flag_combiners_give_up_then_reset_replays_bitwise(gpu, what, prompt_length, context):
    """Past 16 blocks a decode token's attention is combined in the same
    launch by 128 combiner workgroups that wait, bounded, for every block's
    flag. The test build forces one bounded wait of one step to give up: the
    blocks' wait for the q|k|v producers (their NaN partials then reach the
    combiners) or the combiners' own wait for the block flags. The step
    reports a nonfinite logit and invalidates the sequence, every kernel still
    ends, and after reset the same calls give the logits of a fresh context
    bit for bit."""
    seams = lh.test_lib()
    if not seams.lunelette_metal_test_chained(64):
        pytest.skip("this device runs the attention blocks and combine in launches of their own")
    assert bool(seams.lunelette_metal_test_chained(prompt_length)) == (prompt_length < 72 * 64)
    prompt = syn.tokens(SEED, 23, prompt_length)

    def ingest(r):   # the prompt in 256-token calls
        for begin in range(0, prompt_length, 256):
            ids = prompt[begin:begin + 256]
            logits = r.prefill(ids) if begin == 0 else r.append(ids)
        return logits

    with Runtime(seed=SEED, layers=LAYERS, context=context, block=256,
                 prefill=lh.PREFILL_MPS) as fresh:
        want = [ingest(fresh), fresh.decode(7), fresh.decode(8)]
    with Runtime(seed=SEED, layers=LAYERS, context=context, block=256, prefill=lh.PREFILL_MPS,
                 seams=True) as rt:
        assert np.array_equal(bits(ingest(rt)), bits(want[0]))
        rt.inject(what)
        started = time.perf_counter()
        with pytest.raises(RuntimeError_, match="nonfinite"):
            rt.decode(7)
        assert time.perf_counter() - started < 10.0
        with pytest.raises(RuntimeError_):
            rt.decode(7)  # invalid until reset
        rt.reset()
        assert np.array_equal(bits(ingest(rt)), bits(want[0]))
        assert np.array_equal(bits(rt.decode(7)), bits(want[1]))
        assert np.array_equal(bits(rt.decode(8)), bits(want[2]))


@pytest.mark.parametrize("context,block", [(256, 256), (4352, 128)])
def test_allocation_failure_at_every_index(gpu, context, block):
    """The N-th device or pinned-host allocation of create fails, for every N
    create makes: create returns NULL with a diagnostic, and every allocation
    it had made is freed."""
    seams = lh.test_lib()
    seams.lunelette_metal_test_fail_allocation(0)
    live = seams.lunelette_metal_test_live_allocations()
    with Runtime(seed=SEED, layers=1, context=context, block=block, seams=True) as ok:
        total = seams.lunelette_metal_test_allocations()
        ok.prefill([1, 2])
    assert seams.lunelette_metal_test_live_allocations() == live
    assert total >= 20
    try:
        for n in range(1, total + 1):
            seams.lunelette_metal_test_fail_allocation(n)
            with pytest.raises(RuntimeError_, match="create failed: .+"):
                Runtime(seed=SEED, layers=1, context=context, block=block, seams=True)
            assert seams.lunelette_metal_test_allocations() == n
            assert seams.lunelette_metal_test_live_allocations() == live, n
    finally:
        seams.lunelette_metal_test_fail_allocation(0)
    with Runtime(seed=SEED, layers=1, context=context, block=block, seams=True) as again:
        again.prefill([1, 2])


def test_checkpoint_epoch_exhaustion(gpu):
    with Runtime(seed=SEED, layers=1, context=256, block=256, prefill=lh.PREFILL_CUSTOM,
                 seams=True) as rt:
        rt.prefill([1, 2, 3])
        first = rt.checkpoint()   # epoch 1
        saved = rt.restore(first)
        rt.decode(4)
        rt.set_epoch(2 ** 64 - 1)
        with pytest.raises(RuntimeError_, match="epoch"):
            rt.checkpoint()
        rt.set_epoch(1)
        assert np.array_equal(bits(rt.restore(first)), bits(saved))  # still the active one
        second = rt.checkpoint()
        with pytest.raises(RuntimeError_):
            rt.restore(first)
        rt.destroy_checkpoint(first)
        rt.destroy_checkpoint(second)
