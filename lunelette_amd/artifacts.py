"""Native evaluation artifacts.

- LUN1/LUN2 native logit regression (include/lunelette_artifacts.h): thin
  ctypes views of the C writer, reader, strict comparison and capture/check
  runs.
- LNRPLY1 replay captures written by the session adapter in controlled-replay
  mode: parse, verify against the authoritative trajectory and compare two
  captures, with the rules of the reference's tools/replay_logits.py:15-113,
  vectorized with numpy.
"""
import ctypes
import struct

import numpy as np

from . import (LogitMetrics, NativeTrajectory, RESIDENT_FP32, VOCAB, c_float_p, lib)

LUN1, LUN2 = 0x314E554C, 0x324E554C
STEPS = 8

REPLAY_LIMIT = 16
REPLAY_CONTEXT = 4352
REPLAY_HEADER = b"LNRPLY1\0" + struct.pack("<II", VOCAB, REPLAY_LIMIT)
REPLAY_MAX_BYTES = 16 + REPLAY_LIMIT * (16 + 4 * REPLAY_CONTEXT + 4 * VOCAB)


def _metrics(m):
    return {name: getattr(m, name) for name, _ in LogitMetrics._fields_}


def trajectory(ids, forced, strategy=RESIDENT_FP32, mode=0, magic=LUN2):
    """A lunelette_native_trajectory for prompt `ids` (1..248) and 8 forced ids."""
    t = NativeTrajectory()
    t.magic, t.strategy, t.mode, t.count = magic, strategy, mode, len(ids)
    for i, v in enumerate(ids):
        t.ids[i] = int(v)
    for i, v in enumerate(forced):
        t.forced[i] = int(v)
    return t


def _floats(array):
    array = np.ascontiguousarray(array, dtype=np.float32)
    return array, array.ctypes.data_as(c_float_p)


def top64(values):
    array, ptr = _floats(values)
    ids = (ctypes.c_size_t * 64)()
    lib().lunelette_logits_top64(ptr, array.size, ids)
    return list(ids)


def compare(a, b):
    """(accepted, metrics) under the strict native rule."""
    aa, pa = _floats(a)
    bb, pb = _floats(b)
    m = LogitMetrics()
    rc = lib().lunelette_logits_compare(pa, pb, aa.size, ctypes.byref(m))
    return rc == 0, _metrics(m)


def write(path, traj, logits):
    err = ctypes.create_string_buffer(512)
    array, ptr = _floats(logits)
    if array.size != STEPS * VOCAB:
        raise ValueError("need 8 x 131072 logits")
    if lib().lunelette_native_write(str(path).encode(), ctypes.byref(traj), ptr, err, 512):
        raise ValueError(err.value.decode())


def read(path, traj):
    err = ctypes.create_string_buffer(512)
    out = np.empty((STEPS, VOCAB), np.float32)
    if lib().lunelette_native_read(str(path).encode(), ctypes.byref(traj),
                                   out.ctypes.data_as(c_float_p), err, 512):
        raise ValueError(err.value.decode())
    return out


def compare_files(left, right, mode, count, strategy=RESIDENT_FP32):
    """(accepted, per-step metrics, diagnostic) of the offline file check."""
    err = ctypes.create_string_buffer(512)
    m = (LogitMetrics * STEPS)()
    rc = lib().lunelette_native_compare_files(str(left).encode(), str(right).encode(), mode,
                                              count, strategy, m, err, 512)
    return rc == 0, [_metrics(x) for x in m], err.value.decode()


def run(runtime, path, traj, check):
    """Capture (check=False) or check (True) one artifact on a runtime.Runtime
    (or a raw context handle). Returns (ok, metrics of the 16 checked steps,
    diagnostic)."""
    err = ctypes.create_string_buffer(512)
    m = (LogitMetrics * (2 * STEPS))()
    handle = getattr(runtime, "handle", runtime)
    rc = lib().lunelette_native_run(handle, str(path).encode(), ctypes.byref(traj), int(check),
                                    m, err, 512)
    return rc == 0, [_metrics(x) for x in m], err.value.decode()


# ---- LNRPLY1 replay captures ----

def replay_tokens(tokens):
    """1..16 forced ids: ordinary ids 1000..131071, EOS 2 only last."""
    if (not isinstance(tokens, list) or not 1 <= len(tokens) <= REPLAY_LIMIT or
            any(type(t) is not int or not (1000 <= t < VOCAB or (t == 2 and i == len(tokens) - 1))
                for i, t in enumerate(tokens))):
        raise ValueError("invalid replay tokens")
    return tokens


def parse_replay(path):
    """Records of a bounded version-1 capture; each vector must be finite and
    its greedy id must be the first index of its maximum."""
    with open(path, "rb") as source:
        size = source.seek(0, 2)
        if not 16 <= size <= REPLAY_MAX_BYTES:
            raise ValueError("capture size outside bound")
        source.seek(0)
        data = source.read(REPLAY_MAX_BYTES + 1)
    if len(data) > REPLAY_MAX_BYTES or data[:16] != REPLAY_HEADER:
        raise ValueError("invalid capture header/size")
    records, offset = [], 16
    while offset < len(data):
        if len(records) == REPLAY_LIMIT or len(data) - offset < 16:
            raise ValueError("record limit/trailing bytes")
        index, count, forced, greedy = struct.unpack_from("<IIII", data, offset)
        offset += 16
        if (index != len(records) or not 1 <= count <= REPLAY_CONTEXT or
                not (forced == 2 or 1000 <= forced < VOCAB) or not 0 <= greedy < VOCAB):
            raise ValueError("invalid record fields")
        if len(data) - offset < 4 * (count + VOCAB):
            raise ValueError("truncated capture")
        prefix = np.frombuffer(data, "<u4", count, offset)
        if np.any(prefix >= VOCAB):
            raise ValueError("invalid prefix token")
        offset += 4 * count
        raw = data[offset:offset + 4 * VOCAB]
        logits = np.frombuffer(raw, "<f4")
        offset += 4 * VOCAB
        if not np.all(np.isfinite(logits)):
            raise ValueError("nonfinite logits")
        if greedy != int(np.argmax(logits)):
            raise ValueError("incorrect first-tie greedy argmax")
        records.append(dict(index=index, prefix=prefix.tolist(), forced_token=forced,
                            greedy_token=greedy, logits=logits, raw=raw))
    return records


def verify_replay(path, steps):
    """Correlates a capture with completed steps: each step's forced ids must
    equal its actual ids, and record k must hold the prefix before the k-th
    forced id."""
    records = parse_replay(path)
    expected = []
    for step in steps:
        tokens = replay_tokens(step["replay_tokens"])
        actual = step["actual_ids"]
        if (not isinstance(actual, list) or any(type(t) is not int for t in actual) or
                actual != tokens):
            raise ValueError("incomplete replay trajectory")
        prefix = step["before_prefix_ids"]
        if (not isinstance(prefix, list) or not 1 <= len(prefix) <= REPLAY_CONTEXT or
                any(type(t) is not int or not 0 <= t < VOCAB for t in prefix)):
            raise ValueError("invalid authoritative prefix")
        prefix = list(prefix)
        for token in actual:
            expected.append((list(prefix), token))
            prefix.append(token)
    if not expected or len(records) != len(expected):
        raise ValueError("capture record count mismatch")
    for record, (prefix, forced) in zip(records, expected):
        if record["prefix"] != prefix or record["forced_token"] != forced:
            raise ValueError("capture context/target mismatch")
    return {"verified_records": len(records), "independent_numerical_oracle": False}


def compare_replay(reference, candidate, changed_partition=False):
    """Bitwise comparison of two captures of the same trajectory, or, for a
    changed prefill partition, |a - b| <= 2e-4 + 1e-4 |a| per logit."""
    left, right = parse_replay(reference), parse_replay(candidate)
    if not left or not right or len(left) != len(right):
        raise ValueError("record count mismatch")
    mismatches = 0
    max_absolute = max_relative = 0.0
    relative_undefined = False
    for a, b in zip(left, right):
        if a["prefix"] != b["prefix"] or a["forced_token"] != b["forced_token"]:
            raise ValueError("context/forced target mismatch")
        x = a["logits"].astype(np.float64)
        y = b["logits"].astype(np.float64)
        error = np.abs(x - y)
        max_absolute = max(max_absolute, float(error.max()))
        nonzero = x != 0
        if np.any(nonzero):
            max_relative = max(max_relative, float((error[nonzero] / np.abs(x[nonzero])).max()))
        relative_undefined |= bool(np.any(error[~nonzero] != 0))
        if changed_partition:
            matches = error <= 2e-4 + 1e-4 * np.abs(x)
        else:
            matches = np.frombuffer(a["raw"], "<u4") == np.frombuffer(b["raw"], "<u4")
        mismatches += int(np.count_nonzero(~matches))
    return dict(match=mismatches == 0, mismatch_count=mismatches,
                max_absolute_error=max_absolute,
                max_relative_error=None if relative_undefined else max_relative,
                relative_error_undefined_at_zero=relative_undefined,
                records=len(left), independent_numerical_oracle=False)

