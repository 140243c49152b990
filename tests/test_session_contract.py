"""Session adapter contract on the CPU.

lunelette_amd/csrc/session.c is linked with a CPU stand-in for the runtime
(tests/support/stub_runtime.c) into a test library, so the state machine runs
without a GPU. The scenarios restate the reference's adapter tests with their
expected call counts and receipts: tests/test_service_native.c:33-143
(reuse on/off), :147-273 (open, select, pending token, EOS turn, failure,
strategies and accounting) and tests/test_service_long_native.c:5-158
(block-by-block ingestion at context 4352 for every policy and block size).
The framing and detokenization steps of those tests belong to the tokenizer
and are replaced by fixed token lists.
"""
import ctypes
import json
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import artifacts
from lunelette_amd.session import LEGACY, MORE, REUSE_OFF, REUSE_ON, Session

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "lunelette_amd", "csrc")
SOURCES = [os.path.join(CSRC, "session.c"), os.path.join(CSRC, "generation.c"),
           os.path.join(CSRC, "host_alloc.c"), os.path.join(ROOT, "tests", "support", "stub_runtime.c")]
VOCAB = lh.VOCAB
GREEDY = 22177   # the stub's tied maximum: the lower id wins


@pytest.fixture(scope="module")
def stub_build(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("session") / "libsession_stub.so")
    sanitize = []
    if os.environ.get("LH_SANITIZED_LIBRARY"):
        from support import host_sanitize
        sanitize = host_sanitize.FLAGS
    subprocess.run(["gcc", "-std=c11", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", "-Werror",
                    "-I" + os.path.join(ROOT, "include"), "-I" + CSRC] + sanitize + SOURCES +
                   ["-o", out], check=True)
    return out


class Stub:
    """A private instance of the stub library (fresh counters per test)."""

    def __init__(self, path):
        self.l = ctypes.CDLL(path)
        lh.declare_session(self.l)
        self.l.stub_count.restype = ctypes.c_uint
        self.l.stub_count.argtypes = [ctypes.c_void_p]
        self.l.stub_ids.restype = ctypes.POINTER(ctypes.c_int64)
        self.l.stub_ids.argtypes = [ctypes.c_void_p]
        self.logits = np.ctypeslib.as_array((ctypes.c_float * VOCAB).in_dll(self.l, "stub_logits"))

    def __getattr__(self, name):
        return ctypes.c_uint.in_dll(self.l, "stub_" + name).value

    def set(self, name, value):
        ctypes.c_int.in_dll(self.l, "stub_" + name).value = value

    def runtime_ids(self):
        runtime = ctypes.c_void_p.in_dll(self.l, "stub_last_runtime").value
        count = self.l.stub_count(runtime)
        return list(np.ctypeslib.as_array(self.l.stub_ids(runtime), shape=(4352,))[:count])

    def open(self, context=256, block=256, prefix_reuse=LEGACY, prefill=lh.PREFILL_CUSTOM,
             strategy=lh.RESIDENT_FP32, replay_path=None):
        return Session.open("model.safetensors", context=context, block=block,
                            prefix_reuse=prefix_reuse, prefill=prefill, strategy=strategy,
                            replay_path=replay_path, library=self.l)


@pytest.fixture
def stub(stub_build, tmp_path):
    private = str(tmp_path / "libsession_stub.so")
    shutil.copy(stub_build, private)
    return Stub(private)


def test_options_rejected_before_any_runtime(stub):
    for bad in [dict(context=512), dict(context=256, block=128), dict(context=4352, block=64),
                dict(prefix_reuse=3), dict(context=17920)]:
        with pytest.raises(RuntimeError):
            stub.open(**bad)
    assert stub.creates == 0


def test_select_pending_eos_and_failure(stub):
    """tests/test_service_native.c:147-220."""
    s = stub.open()
    assert stub.creates == 1
    info = s.info
    assert info["model_load_count"] == 1 and info["generator"] == "native_greedy"
    assert info["context_capacity"] == 256 and info["prefill_chunk_size"] == 256
    ids = [1, 1001, 37133, 1002]           # a framed one-turn prompt
    assert s.materialize(ids) == 1
    assert (stub.prefills, stub.decodes) == (1, 0)
    assert s.next() == GREEDY
    assert s.next() == -1                  # a token is already pending
    assert s.materialize(ids) == 0         # the pending token must come next
    ids.append(GREEDY)
    assert s.materialize(ids) == 1
    assert (stub.prefills, stub.decodes) == (1, 1)
    assert s.materialize(ids) == 1         # nothing to run
    assert stub.decodes == 1
    changed = list(ids)
    changed[2] += 1
    assert s.materialize(changed) == 0
    # A generated EOS stays pending until the next user turn arrives with it.
    stub.logits[2] = 2
    assert s.next() == 2
    ids += [2, 1003, 1004, 1005]
    assert s.materialize(ids) == 1
    assert (stub.prefills, stub.decodes) == (2, 1)   # legacy rebuilds after EOS
    assert s.next() == GREEDY
    ids.append(GREEDY)
    stub.set("fail", 1)
    assert s.materialize(ids) == 0
    assert s.next() == -1                  # the failure left no logits
    stub.set("fail", 0)
    s.reset()
    ids = ids[:4]
    assert s.materialize(ids) == 1
    assert s.next() == GREEDY
    ids.append(GREEDY)
    assert s.materialize(ids) == 1
    stub.logits[VOCAB - 1] = np.nan        # the whole vocabulary is checked
    assert s.next() == -1
    s.reset()
    s.close()
    assert (stub.creates, stub.destroys, stub.prefills) == (1, 1, 3)
    assert stub.resets >= 4
    assert stub.violations == 0


def test_strategies_accounting_and_open_failures(stub):
    """tests/test_service_native.c:221-273."""
    s = stub.open(strategy=lh.COMPACT_FP8_ARITHMETIC)
    info = json.loads(s.info_text)
    assert info["execution_strategy"] == "compact-fp8-arithmetic"
    assert info["named_conversion_stage_bytes"] == 113246208
    assert info["named_buffer_total_bytes"] == 4893045760
    assert info["prefill"] == "custom"
    assert len(s.info_text) + 256 < 4096
    s.close()
    assert (stub.creates, stub.destroys) == (1, 1)
    s = stub.open(strategy=lh.COMPACT_FP8_ARITHMETIC, prefill=lh.PREFILL_MPS)
    assert s.info["prefill"] == "mps"
    assert ctypes.c_int.in_dll(stub.l, "stub_last_prefill").value == lh.PREFILL_MPS
    s.close()
    stub.set("fail_memory", 1)
    with pytest.raises(RuntimeError):
        stub.open()
    assert (stub.creates, stub.destroys) == (3, 3)   # the runtime is closed again
    stub.set("fail_memory", 0)
    stub.set("wrong_strategy", 1)
    with pytest.raises(RuntimeError, match="strategy"):
        stub.open(strategy=lh.COMPACT_FP8_ARITHMETIC)   # no silent fallback
    assert (stub.creates, stub.destroys) == (4, 4)
    stub.set("wrong_strategy", 0)
    s = stub.open(strategy=lh.COMPACT_FP8_LOOKUP)
    assert s.info["execution_strategy"] == "compact-fp8-lookup"
    assert s.info["named_conversion_stage_bytes"] == 113246208
    s.close()
    assert stub.violations == 0


@pytest.mark.parametrize("policy", [REUSE_ON, REUSE_OFF])
def test_reuse_policy(stub, policy):
    """tests/test_service_native.c:33-143."""
    on = policy == REUSE_ON
    s = stub.open(strategy=lh.COMPACT_FP8_ARITHMETIC, prefix_reuse=policy)
    assert s.prefix_reuse == policy
    assert s.info["prefix_reuse"] == ("on" if on else "off") and s.info["checkpoints"]
    ids = [42] * 100
    s.begin()
    assert s.materialize(ids) == 1
    w = s.work()
    assert w["full_committed"] == 100 and w["prefill_calls"] == 1
    assert s.save() == 1
    appends, prefills, decodes = stub.appends, stub.prefills, stub.decodes
    ids += [43] * 12
    s.begin()
    assert s.materialize(ids) == 1
    w = s.work()
    assert w["full_committed"] == (0 if on else 112)
    assert w["suffix_committed"] == (12 if on else 0)
    assert stub.appends == appends + on and stub.prefills == prefills + (not on)
    assert s.next() == GREEDY
    ids.append(GREEDY)
    assert s.materialize(ids) == 1
    w = s.work()
    assert w["decode_calls"] == 1 and w["pending_committed"] == 1 and w["decode_committed"] == 1
    assert stub.decodes == decodes + 1        # off does not recompute every decode
    for _ in range(3):
        prefills, decodes = stub.prefills, stub.decodes
        assert s.restore() == 1
        assert s.work()["logit_restores"] == on
        ids = ids[:100]
        assert (stub.prefills, stub.decodes) == (prefills, decodes)
        s.begin()
        assert s.materialize(ids) == 1
        w = s.work()
        assert w["full_committed"] == (0 if on else 100) and w["decode_calls"] == 0
        assert s.next() == GREEDY
        ids.append(GREEDY)
        assert s.materialize(ids) == 1
    prefills, decodes = stub.prefills, stub.decodes
    s.begin()
    assert s.materialize(ids) == 1
    w = s.work()
    assert w["full_committed"] == (0 if on else len(ids))
    assert stub.prefills == prefills + (not on) and stub.decodes == decodes
    ids[0] += 1
    assert s.materialize(ids) == 0
    ids[0] -= 1
    # An ordinary new turn reconciles the pending EOS and the user suffix together.
    stub.logits[2] = 2
    assert s.next() == 2
    ids += [2, 42, 43]
    s.begin()
    assert s.materialize(ids) == 1
    w = s.work()
    assert w["pending_committed"] == 1
    assert w["append_calls"] == on and w["suffix_committed"] == (3 if on else 0)
    # A pending EOS is materialized once, also with no user suffix.
    stub.logits[2] = 2
    assert s.next() == 2
    ids.append(2)
    assert s.materialize(ids) == 1
    w = s.work()
    assert w["pending_committed"] == 1 and w["decode_calls"] == 1
    assert s.save() == 1
    assert s.restore() == 1
    assert s.materialize(ids)
    # A failed replacement keeps the previous checkpoint.
    stub.set("fail_snapshot", 1)
    assert s.save() == 0
    stub.set("fail_snapshot", 0)
    assert s.restore() == 1
    assert s.materialize(ids)
    assert s.next() == GREEDY
    ids.append(GREEDY)
    stub.set("fail", 1)
    assert s.materialize(ids) == 0
    w = s.work()
    assert w["decode_calls"] == 1 and w["decode_attempted"] == 1 and not w["decode_committed"]
    assert w["pending_attempted"] == 1 and not w["pending_committed"]
    stub.set("fail", 0)
    if on:
        assert s.restore() == 0               # the failed execution dropped the handle
    s.reset()
    assert s.restore() == 0
    s.close()
    assert stub.snapshots >= 2 and stub.violations == 0


def ingest(stub, s, ids):
    """tests/test_service_long_native.c:5-33: materialize_step to READY, checking
    after every block that the runtime holds exactly the committed prefix."""
    total = {}
    while True:
        state, cursor = s.materialize_step(ids)
        assert state in (1, MORE)
        assert stub.runtime_ids() == list(ids[:cursor])
        w = s.work()
        assert w["full_committed"] + w["suffix_committed"] + w["decode_committed"] <= \
            s.block_capacity
        for k, v in w.items():
            total[k] = total.get(k, 0) + v
        if state == 1:
            assert cursor == len(ids)
            return total


@pytest.mark.parametrize("block", [128, 256])
@pytest.mark.parametrize("policy", [LEGACY, REUSE_ON, REUSE_OFF])
def test_long_context_ingestion(stub, block, policy):
    """tests/test_service_long_native.c:35-158 (context 4352)."""
    s = stub.open(context=4352, block=block, prefix_reuse=policy)
    assert (s.context_capacity, s.block_capacity) == (4352, block)
    ids = [1000 + (37 * i) % 8000 for i in range(4353)]
    for length in (block, block + 1, 4096, 4352):
        s.reset()
        resets = stub.resets
        s.begin()
        w = ingest(stub, s, ids[:length])
        assert stub.resets == resets + 1
        assert w["prefill_calls"] == 1 and w["full_committed"] == block
        assert w["append_calls"] == (length - 1) // block
        assert w["full_committed"] + w["suffix_committed"] == length
        assert w["recompute_committed"] == 0
        assert s.save() == 1
    assert s.materialize_step(ids[:4353])[0] == 0
    for eos in (0, 1):
        s.reset()
        s.begin()
        ingest(stub, s, ids[:4096])
        if eos:
            stub.logits[2] = 2
        token = s.next()
        assert token == (2 if eos else GREEDY)
        ids[4096] = token
        w = ingest(stub, s, ids[:4097])
        assert w["pending_committed"] == 1
        assert w["full_committed"] + w["suffix_committed"] + w["decode_committed"] == \
            (4097 if policy == LEGACY and eos else 1)
        assert s.save() == 1
        assert s.restore() == 1
        if policy == REUSE_OFF:
            ingest(stub, s, ids[:4097])
        assert s.next() == GREEDY
        ids[4097] = GREEDY
        ingest(stub, s, ids[:4098])
        assert s.restore() == 1
        ids[4097] = 43
        s.begin()
        w = ingest(stub, s, ids[:4098])
        assert w["full_committed"] + w["suffix_committed"] == (1 if policy == REUSE_ON else 4098)
        assert s.next() == GREEDY
        ids[4098] = GREEDY
        stub.set("fail", 1)
        assert s.materialize_step(ids[:4099])[0] == 0
        w = s.work()
        assert w["decode_attempted"] == 1 and w["decode_committed"] == 0
        stub.set("fail", 0)
    for eos in (0, 1):
        s.reset()
        ids = [1000 + (37 * i) % 8000 for i in range(4353)]
        s.begin()
        ingest(stub, s, ids[:4351])
        if eos:
            stub.logits[2] = 2
        ids[4351] = s.next()
        assert ids[4351] == (2 if eos else GREEDY)
        w = ingest(stub, s, ids[:4352])
        assert w["pending_committed"] == 1
        assert s.save() == 1
        assert s.restore() == 1
        if policy == REUSE_OFF:
            w = ingest(stub, s, ids[:4352])
            assert w["recompute_committed"] == 4352
        assert s.next() == -1                 # a full context has no room: never selects
    s.reset()
    s.begin()
    assert s.materialize_step(ids[:257]) == (MORE, block)
    s.work()
    stub.set("fail", 1)
    assert s.materialize_step(ids[:257]) == (0, block)
    w = s.work()
    assert w["append_calls"] == 1 and w["suffix_attempted"] == min(257 - block, block)
    assert not w["suffix_committed"] and not w["prefill_calls"]
    stub.set("fail", 0)
    s.close()
    assert stub.violations == 0


def test_recompute_accounting(stub):
    """service/native.c:185-188, 229-232: a rebuild counts the previously
    committed prefix (under off after a restore: the restored one) as
    recomputation, block by block; a pending token followed by a user suffix
    rebuilds under legacy."""
    s = stub.open(context=4352, block=128)
    ids = list(range(1000, 1300))
    w = ingest(stub, s, ids)
    assert w["recompute_committed"] == 0 and w["append_calls"] == 2
    assert s.next() == GREEDY
    ids += [GREEDY, 1500, 1501]
    prefills = stub.prefills
    w = ingest(stub, s, ids)
    assert stub.prefills == prefills + 1
    assert w["recompute_committed"] == 300 and w["pending_committed"] == 1
    assert w["full_committed"] + w["suffix_committed"] == 303
    s.close()
    s = stub.open(context=4352, block=128, prefix_reuse=REUSE_OFF)
    ids = list(range(1000, 1100))
    s.begin()
    ingest(stub, s, ids)
    assert s.save() == 1
    ids += [1200] * 12
    s.begin()
    w = ingest(stub, s, ids)
    assert w["recompute_committed"] == 100 and w["full_committed"] == 112
    assert s.restore() == 1
    ids = ids[:100] + [2000] * 40
    w = ingest(stub, s, ids)
    assert w["recompute_committed"] == 100 and w["full_committed"] == 128
    assert w["suffix_committed"] == 12
    s.close()
    assert stub.violations == 0


def read_capture(path):
    """LNRPLY1 records as (index, prefix, forced, greedy, logits)."""
    data = open(path, "rb").read()
    assert data[:8] == b"LNRPLY1\0"
    assert struct.unpack_from("<II", data, 8) == (VOCAB, 16)
    records, at = [], 16
    while at < len(data):
        index, length, forced, greedy = struct.unpack_from("<IIII", data, at)
        at += 16
        prefix = list(struct.unpack_from("<%dI" % length, data, at))
        at += 4 * length
        logits = np.frombuffer(data, "<f4", VOCAB, at)
        at += 4 * VOCAB
        records.append((index, prefix, forced, greedy, logits))
    assert at == len(data)
    return records


def test_replay_capture(stub, tmp_path):
    """service/native.c:336-416 and the capture layout of
    docs/development/replay.md:23-28: every forced selection appends one
    record of the actual prefix, the forced and the greedy id and all logits;
    the forced id becomes the pending token."""
    path = str(tmp_path / "replay.bin")
    s = stub.open(context=4352, block=256, prefix_reuse=REUSE_ON, replay_path=path)
    assert s.info["generator"] == "native_controlled_replay"
    assert s.info["evaluation_mode"] == "controlled_replay"
    with pytest.raises(RuntimeError):
        stub.open(context=4352, replay_path=path)      # the capture file is never reused
    plain = stub.open(context=4352)
    assert plain.materialize([1, 1000]) == 1
    assert plain.replay_next(53156) == -1               # replay needs the evaluation mode
    plain.close()
    ids = [1, 1000, 1001]
    assert s.materialize(ids) == 1
    for forced in (3, 999, VOCAB, 1 << 31):
        assert s.replay_next(forced) == -1              # ordinary ids 1000.. or EOS 2 only
    assert s.replay_next(53156) == 53156
    assert s.materialize(ids + [GREEDY]) == 0           # the forced id is authoritative
    assert s.materialize(ids + [53156]) == 1
    ids.append(53156)
    for k in range(15):
        forced = 2 if k == 14 else 2000 + k
        assert s.replay_next(forced) == forced
        ids.append(forced)
        assert s.materialize(ids) == 1
    assert s.replay_next(3000) == -1                    # sixteen records at most
    s.close()
    records = read_capture(path)
    assert len(records) == 16
    # The replay tool's reader accepts the capture and correlates it with the
    # authoritative trajectory.
    forced_ids = [int(t) for t in ids[3:]]
    steps = [dict(replay_tokens=forced_ids, actual_ids=forced_ids,
                  before_prefix_ids=[int(t) for t in ids[:3]])]
    assert artifacts.verify_replay(path, steps)["verified_records"] == 16
    for k, (index, prefix, forced, greedy, logits) in enumerate(records):
        assert index == k and prefix == ids[:3 + k] and forced == ids[3 + k]
        assert greedy == GREEDY
        want = np.zeros(VOCAB, np.float32)
        want[[GREEDY, GREEDY + 1]] = 1
        assert np.array_equal(logits, want)
    assert stub.violations == 0
