"""Session adapter over the gfx950 runtime.

- Precise prefill (CUSTOM): any chunking of a sequence gives bitwise equal
  logits, so a conversation driven through the adapter must select the same
  tokens from bitwise equal logits under all three reuse policies (on
  extends the cache and restores checkpoints, off recomputes the whole
  prefix at each boundary and after a restore, legacy rebuilds at each turn),
  and those logits equal a fresh prefill of the same prefix on a second
  context.
- MFMA prefill (MPS): the adapter issues exactly the runtime calls a direct
  driver would (prefill of the first block, append of the rest, decode of
  each selected token), so its logits equal that driver's bitwise.
- Controlled replay: the LNRPLY1 records hold the prefix, forced id, greedy
  id and the logits the adapter selected from.
"""
import struct

import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import synthetic as syn
from lunelette_amd.runtime import Runtime
from lunelette_amd.session import LEGACY, REUSE_OFF, REUSE_ON, Session

pytestmark = pytest.mark.gpu
SEED = 20251201
LAYERS = 4


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def ingest(session, ids):
    result, receipts = session.ingest(ids)
    assert result == 1, session.error
    return receipts


def converse(session, prompt, users, steps, checkpoints=True):
    """Turn 1, save, turn 2, restore, turn 2' (without the checkpoint steps
    for the legacy policy, whose rebuilds reset the context and with it the
    checkpoint handle). Returns [(prefix, token, logits)] at every selection."""
    seen = []

    def turn(ids):
        session.begin()
        ingest(session, ids)
        for _ in range(steps):
            token = session.next()
            assert token >= 0, session.error
            seen.append((list(ids), token, session.logits()))
            ids.append(token)
            assert session.materialize(ids) == 1, session.error

    ids = list(prompt)
    turn(ids)
    if checkpoints:
        assert session.save() == 1
    saved = list(ids)
    turn(ids + users[0])
    if checkpoints:
        assert session.restore() == 1
        turn(saved + users[1])
    return seen


@pytest.mark.parametrize("block", [256, 128])
def test_policies_select_identically_precise(gpu, block):
    prompt = syn.tokens(SEED, 1, 300).tolist()
    users = [syn.tokens(SEED, 2, 40).tolist(), syn.tokens(SEED, 3, 70).tolist()]
    runs = {}
    for policy in (REUSE_ON, REUSE_OFF, LEGACY):
        rt = Runtime(seed=SEED, layers=LAYERS, context=4352, block=block,
                     prefill=lh.PREFILL_CUSTOM)
        with Session.adopt(rt, prefix_reuse=policy) as session:
            runs[policy] = converse(session, prompt, users, 5, policy != LEGACY)
    base = runs[REUSE_ON]
    assert len(base) == 15 and len(runs[REUSE_OFF]) == 15 and len(runs[LEGACY]) == 10
    for policy in (REUSE_OFF, LEGACY):
        for (p0, t0, l0), (p1, t1, l1) in zip(base, runs[policy]):
            assert p0 == p1 and t0 == t1
            assert np.array_equal(bits(l0), bits(l1))
    with Runtime(seed=SEED, layers=LAYERS, context=4352, block=block,
                 prefill=lh.PREFILL_CUSTOM) as fresh:
        for prefix, token, logits in base[::3]:
            fresh.reset()
            got = fresh.prefill(prefix[:block])
            for at in range(block, len(prefix), block):
                got = fresh.append(prefix[at:at + block])
            assert np.array_equal(bits(got), bits(logits))
            assert token == int(np.argmax(logits))


def test_adapter_calls_equal_direct_driver_mps(gpu):
    prompt = syn.tokens(SEED, 4, 300).tolist()
    rt = Runtime(seed=SEED, layers=LAYERS, context=4352, block=256, prefill=lh.PREFILL_MPS)
    with Session.adopt(rt, prefix_reuse=REUSE_ON) as session:
        receipts = ingest(session, prompt)
        assert [r["prefill_calls"] for r in receipts] == [1, 0]
        assert [r["suffix_committed"] for r in receipts] == [0, 44]
        ids, got = list(prompt), [session.logits()]
        for _ in range(6):
            token = session.next()
            ids.append(token)
            assert session.materialize(ids) == 1
            assert session.work()["decode_committed"] == 1
            got.append(session.logits())
    with Runtime(seed=SEED, layers=LAYERS, context=4352, block=256,
                 prefill=lh.PREFILL_MPS) as direct:
        direct.prefill(prompt[:256])
        want = [direct.append(prompt[256:])]
        for token in ids[300:]:
            assert token == int(np.argmax(want[-1]))
            want.append(direct.decode(token))
    for a, b in zip(got, want):
        assert np.array_equal(bits(a), bits(b))


def test_replay_capture_records(gpu, tmp_path):
    path = str(tmp_path / "replay-logits.bin")
    prompt = syn.tokens(SEED, 5, 130).tolist()
    rt = Runtime(seed=SEED, layers=LAYERS, context=4352, block=128, prefill=lh.PREFILL_CUSTOM)
    forced = [53156, 1000, 2]
    seen = []
    with Session.adopt(rt, prefix_reuse=REUSE_ON, replay_path=path) as session:
        assert session.info["evaluation_mode"] == "controlled_replay"
        ids = list(prompt)
        ingest(session, ids)
        for token in forced:
            seen.append((list(ids), session.logits()))
            assert session.replay_next(token) == token
            ids.append(token)
            assert session.materialize(ids) == 1
    data = open(path, "rb").read()
    assert data[:8] == b"LNRPLY1\0" and struct.unpack_from("<II", data, 8) == (lh.VOCAB, 16)
    at = 16
    for k, (prefix, logits) in enumerate(seen):
        index, length, got_forced, greedy = struct.unpack_from("<IIII", data, at)
        at += 16
        assert (index, length, got_forced) == (k, len(prefix), forced[k])
        assert list(struct.unpack_from("<%dI" % length, data, at)) == prefix
        at += 4 * length
        record = np.frombuffer(data, "<f4", lh.VOCAB, at)
        at += 4 * lh.VOCAB
        assert np.array_equal(bits(record), bits(logits))
        assert greedy == int(np.argmax(logits))
    assert at == len(data)
