"""The reference's frozen LONG schedules on the gfx950 runtime.

tests/long_context/long/schedule.py:11-47 drives a 4352-token context with
block 256 or 128 through resets, chunked prefills and appends, a checkpoint
after a 4096-token (block 128: 257-token) prefix, single-token appends after
it, restores, and independent fresh replays of the same chunk schedule, and
names the snapshot pairs that must be bitwise equal. The schedule is restated
here (ids 1000 + 37 i mod 8000) and run on a 4-layer synthetic model in the
matrix-core prefill mode; every named pair must match bit for bit, and the
boundary and capacity runs must complete.
"""
import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd.runtime import Runtime

pytestmark = pytest.mark.gpu


def schedule(block):
    """(operations, pairs): operations are (api, start, ids, snapshot name)."""
    ops, pairs = [], []

    def tokens(n):
        return [1000 + (37 * i) % 8000 for i in range(n)]

    def fresh(ids, name):
        ops.append(("reset", 0, [], None))
        for p in range(0, len(ids), block):
            ops.append(("prefill" if p == 0 else "append", p, ids[p:p + block], None))
        ops.append(("snapshot", 0, [], name))

    for n in (block - 1, block, block + 1):
        fresh(tokens(n), "boundary%d" % n)
    if block == 256:
        fresh(tokens(513), "tail513")
    prefix = 4096 if block == 256 else 257
    base = tokens(prefix)
    fresh(base, "prefix")
    ops.append(("save", 0, [], None))
    for label, token in (("a", 9101), ("b", 9102)):
        ops.append(("append", prefix, [token], None))
        ops.append(("snapshot", 0, [], label))
        ops.append(("restore", 0, [], None))
        ops.append(("snapshot", 0, [], "restore_" + label))
        pairs.append(("restore_" + label, "prefix"))
    for label, token in (("a", 9101), ("b", 9102)):
        fresh(base, "replay_prefix_" + label)
        pairs.append(("replay_prefix_" + label, "prefix"))
        ops.append(("append", prefix, [token], None))
        ops.append(("snapshot", 0, [], "replay_" + label))
        pairs.append((label, "replay_" + label))
    fresh(tokens(4352 if block == 256 else 513), "capacity" if block == 256 else "tail513")
    return ops, pairs


@pytest.mark.parametrize("block", [256, 128])
def test_long_schedule_pairs_bitwise(gpu, block):
    ops, pairs = schedule(block)
    snapshots = {}
    with Runtime(seed=20251204, layers=4, context=4352, block=block,
                 prefill=lh.PREFILL_MPS) as rt:
        checkpoint, last = None, None
        for api, start, ids, name in ops:
            if api == "reset":
                rt.reset()
            elif api == "prefill":
                last = rt.prefill(ids)
            elif api == "append":
                last = rt.append(ids)
            elif api == "save":
                if checkpoint is not None:
                    rt.destroy_checkpoint(checkpoint)
                checkpoint = rt.checkpoint()
            elif api == "restore":
                last = rt.restore(checkpoint)
            elif api == "snapshot":
                assert np.isfinite(last).all()
                snapshots[name] = last.copy()
        if checkpoint is not None:
            rt.destroy_checkpoint(checkpoint)
    assert pairs
    for a, b in pairs:
        assert np.array_equal(snapshots[a].view(np.uint32), snapshots[b].view(np.uint32)), (a, b)
    # A single appended token changes the step's logits.
    assert not np.array_equal(snapshots["a"], snapshots["b"])
