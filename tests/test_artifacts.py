"""Native artifacts on the CPU.

LUN1/LUN2 (lunelette_amd/csrc/artifacts.c):
- the format and metric cases of the reference's own self-test,
  tests/compare_native.c:196-345 (strategy identity, LUN1 as resident only,
  strict acceptance, top-k intersections against a double rank oracle with
  ties, header and vector corruptions);
- differential against the reference's comparator compiled from
  tests/compare_native.c (oracle/_ref/compare_native_offline, --files mode):
  the same accept/reject verdict on identical, mutated and mixed-format file
  pairs, and the same printed metrics digit for digit.
LNRPLY1 (lunelette_amd/artifacts.py): the cases of the reference's
tests/test_replay_logits.py:11-82 (parse/compare/verify, signed zero and
undefined relative error, rejections, the size bound).
"""
import os
import re
import shutil
import struct
import subprocess

import numpy as np
import pytest

import lunelette_amd as lh
from lunelette_amd import artifacts as art

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REFBIN = os.path.join(ROOT, "oracle", "_ref", "compare_native_offline")
V = lh.VOCAB
NAMES = ["resident-fp32", "compact-fp8-arithmetic", "compact-fp8-lookup"]


@pytest.fixture(scope="module", autouse=True)
def library(product):
    return product


def logits(seed, steps=8):
    rng = np.random.default_rng(seed)
    out = rng.standard_normal((steps, V)).astype(np.float32)
    out[:, ::97] = np.round(out[:, ::97], 1)       # plenty of exact ties
    return out


def patch_u32(path, offset, value):
    with open(path, "r+b") as f:
        f.seek(offset)
        f.write(struct.pack("<I", value))


def patch_f32(path, offset, value):
    with open(path, "r+b") as f:
        f.seek(offset)
        f.write(struct.pack("<f", value))


def test_strategy_identity(tmp_path):
    """tests/compare_native.c:203-226."""
    zeros = np.zeros((8, V), np.float32)
    for strategy in range(3):
        t = art.trajectory([1], [0] * 8, strategy)
        path = tmp_path / ("s%d.bin" % strategy)
        art.write(path, t, zeros)
        art.read(path, t)
        with pytest.raises(ValueError):
            art.read(path, art.trajectory([1], [0] * 8, (strategy + 1) % 3))
        bad = tmp_path / ("s%d_word.bin" % strategy)
        shutil.copy(path, bad)
        patch_u32(bad, 4, 3)
        with pytest.raises(ValueError):
            art.read(bad, t)
    with pytest.raises(ValueError):
        art.write(tmp_path / "s0.bin", art.trajectory([1], [0] * 8), zeros)   # never overwrites


def test_lun1_is_resident_only(tmp_path):
    """tests/compare_native.c:227-255: the LUN1 layout has no strategy word."""
    old = [art.LUN1, 0, 256, 1, 8, V, 1] + [0] * 8
    path = tmp_path / "old.bin"
    with open(path, "wb") as f:
        f.write(struct.pack("<%dI" % len(old), *old))
        f.write(np.zeros((8, V), np.float32).tobytes())
    for strategy in range(3):
        t = art.trajectory([1], [0] * 8, strategy)
        if strategy == 0:
            art.read(path, t)
        else:
            with pytest.raises(ValueError):
                art.read(path, t)
    written = tmp_path / "written.bin"
    art.write(written, art.trajectory([1], [0] * 8, 0, magic=art.LUN1),
              np.zeros((8, V), np.float32))
    assert written.read_bytes()[:4 * len(old)] == struct.pack("<%dI" % len(old), *old)
    with pytest.raises(ValueError):
        art.write(tmp_path / "compact.bin", art.trajectory([1], [0] * 8, 1, magic=art.LUN1),
                  np.zeros((8, V), np.float32))


def test_strict_acceptance_and_topk():
    """tests/compare_native.c:256-291."""
    a = (127 - np.arange(128)).astype(np.float32)
    b = a.copy()
    assert art.compare(a, b)[0]
    b[127] += 0.25                   # same argmax and top-64: still rejected
    ok, m = art.compare(a, b)
    assert not ok and m["top1_a"] == m["top1_b"] and m["top64"] == 64 and not m["exact"]
    for bad in (np.nan, np.inf):
        b = a.copy()
        b[0] = bad
        ok, m = art.compare(a, b)
        assert not ok and m["finite_b"] == 127
    b = a.copy()
    b[0], b[1] = a[1], a[0]
    assert art.top64(a)[0] == 0 and art.top64(b)[0] == 1
    ok, m = art.compare(a, b)
    assert not ok and m["top5"] == 5
    b = a.copy()
    b[64] = 200
    ok, m = art.compare(a, b)
    assert (m["top5"], m["top20"], m["top64"]) == (4, 19, 63)
    # Independent double rank oracle with ties (lower id first).
    c = np.array([(i * 17) % 13 for i in range(128)], np.float32)
    top = art.top64(c)
    for i in range(128):
        rank = sum(1 for j in range(128) if float(c[j]) > float(c[i]) or (c[j] == c[i] and j < i))
        assert rank >= 64 or top[rank] == i


def test_header_and_vector_corruptions(tmp_path):
    """tests/compare_native.c:292-343."""
    prompt, forced = [1, 2, 3, 4, 5, 6], [7, 8, 9, 10, 11, 12, 13, 14]
    t = art.trajectory(prompt, forced)
    path = tmp_path / "a.bin"
    art.write(path, t, logits(1))
    art.read(path, t)
    with pytest.raises(ValueError):
        art.read(path, art.trajectory(prompt, forced, mode=1))
    with pytest.raises(ValueError):
        art.read(path, art.trajectory([2] + prompt[1:], forced))
    for offset, value in ((0, art.LUN2 + 1), (12, 257), (20, 9), (24, V + 1)):
        bad = tmp_path / ("h%d.bin" % offset)
        shutil.copy(path, bad)
        patch_u32(bad, offset, value)
        with pytest.raises(ValueError):
            art.read(bad, t)
    data = path.read_bytes()
    (tmp_path / "short.bin").write_bytes(data[:-4 * V])        # a missing step
    (tmp_path / "long.bin").write_bytes(data + b"\0")
    for name in ("short.bin", "long.bin"):
        with pytest.raises(ValueError):
            art.read(tmp_path / name, t)
    header = 4 * (7 + 6 + 8)
    for value in (float("nan"), float("inf")):
        bad = tmp_path / "nonfinite.bin"
        shutil.copy(path, bad)
        patch_f32(bad, header + 4 * (3 * V + 100), value)
        with pytest.raises(ValueError):
            art.read(bad, t)
        os.remove(bad)
        vectors = logits(2)
        vectors[5, 9] = value
        with pytest.raises(ValueError):
            art.write(tmp_path / ("refused%s.bin" % value), t, vectors)


METRIC_LINE = re.compile(
    r"finite=(\d+)/\d+ reference_finite=(\d+)/\d+ exact=(\d) top1=(\d+)/(\d+) top5=(\d+) "
    r"top20=(\d+) top64=(\d+) maxabs=(\S+) RMS=(\S+) cosine=(\S+)")


def reference_files(a, b, mode, count, strategy):
    proc = subprocess.run([REFBIN, "--files", str(a), str(b), ("mps", "custom")[mode], str(count),
                           "--strategy=" + NAMES[strategy]], capture_output=True, text=True)
    return proc.returncode, [METRIC_LINE.search(line).groups()
                             for line in proc.stdout.splitlines() if METRIC_LINE.search(line)]


def mutations(tmp_path, path, t, count):
    """(name, file) pairs built from a valid artifact."""
    header = 4 * (7 + count + 8)
    vectors = art.read(path, t)
    out = [("identical", path)]

    def variant(name, edit):
        target = tmp_path / (name + ".bin")
        shutil.copy(path, target)
        edit(target)
        out.append((name, target))
    variant("tail", lambda p: patch_f32(p, header + 4 * (3 * V - 1), vectors[2, V - 1] - 0.5))
    variant("nan", lambda p: patch_f32(p, header + 4 * (6 * V + 7), float("nan")))
    variant("inf", lambda p: patch_f32(p, header + 4 * 77, float("-inf")))
    variant("mode", lambda p: patch_u32(p, 8, 1 - t.mode))
    variant("token", lambda p: patch_u32(p, 28, (t.ids[0] + 1) % V))
    variant("strategy", lambda p: patch_u32(p, 4, (t.strategy + 1) % 3))
    variant("truncated", lambda p: os.truncate(p, os.path.getsize(p) - 4))
    variant("extended", lambda p: open(p, "ab").write(b"\0\0\0\0"))
    # Exchange the step-4 maximum with the next distinct value: a top-1 swap.
    order = np.argsort(-vectors[4], kind="stable")
    second = next(i for i in order[1:] if vectors[4, i] != vectors[4, order[0]])
    swapped = vectors.copy()
    swapped[4, order[0]], swapped[4, second] = vectors[4, second], vectors[4, order[0]]
    target = tmp_path / "swap.bin"
    art.write(target, t, swapped)
    out.append(("swap", target))
    if t.strategy == 0:
        lun1 = tmp_path / "lun1.bin"
        t1 = art.trajectory(list(t.ids[:count]), list(t.forced), 0, t.mode, art.LUN1)
        art.write(lun1, t1, vectors)
        out.append(("lun1", lun1))
    return out


@pytest.mark.skipif(not os.path.exists(REFBIN), reason="reference comparator not built")
def test_reference_self_test_builds_and_passes():
    assert subprocess.run([REFBIN, "--self-test"], capture_output=True).returncode == 0


@pytest.mark.skipif(not os.path.exists(REFBIN), reason="reference comparator not built")
@pytest.mark.parametrize("count,mode,strategy", [(6, 0, 0), (24, 1, 1), (150, 0, 2)])
def test_files_match_reference_comparator(tmp_path, count, mode, strategy):
    rng = np.random.default_rng(count)
    prompt = rng.integers(0, V, count).tolist()
    forced = rng.integers(1000, V, 8).tolist()
    t = art.trajectory(prompt, forced, strategy, mode)
    path = tmp_path / "reference.bin"
    art.write(path, t, logits(count))
    for name, other in mutations(tmp_path, path, t, count):
        ok, metrics, _ = art.compare_files(path, other, mode, count, strategy)
        rc, printed = reference_files(path, other, mode, count, strategy)
        assert ok == (rc == 0), name
        assert ok == (name in ("identical", "lun1")), name
        for step, fields in enumerate(printed):
            m = metrics[step]
            assert [int(x) for x in fields[:8]] == [
                m["finite_a"], m["finite_b"], m["exact"], m["top1_a"], m["top1_b"], m["top5"],
                m["top20"], m["top64"]], (name, step)
            assert [float(x) for x in fields[8:]] == [m["max_abs"], m["rms"], m["cosine"]], \
                (name, step)


def replay_capture(prefix=(1, 1000), forced=53156, greedy=0, value=1.0):
    vec = [0.0] * V
    vec[greedy] = value
    return (b"LNRPLY1\0" + struct.pack("<II", V, 16)
            + struct.pack("<IIII", 0, len(prefix), forced, greedy)
            + struct.pack("<%dI" % len(prefix), *prefix)
            + struct.pack("<%df" % V, *vec))


def test_replay_parse_compare_verify(tmp_path):
    """tests/test_replay_logits.py:20-38."""
    a, b = tmp_path / "a", tmp_path / "b"
    a.write_bytes(replay_capture())
    b.write_bytes(replay_capture())
    assert art.compare_replay(a, b)["match"]
    steps = [dict(replay_tokens=[53156], actual_ids=[53156], before_prefix_ids=[1, 1000])]
    assert art.verify_replay(a, steps)["verified_records"] == 1
    b.write_bytes(replay_capture(value=1.00001))
    assert not art.compare_replay(a, b)["match"]
    assert art.compare_replay(a, b, True)["match"]
    b.write_bytes(replay_capture(value=2))
    assert not art.compare_replay(a, b, True)["match"]
    b.write_bytes(replay_capture(prefix=(1, 1001)))
    with pytest.raises(ValueError):
        art.compare_replay(a, b)
    with pytest.raises(ValueError):
        art.verify_replay(a, [dict(replay_tokens=[1000], actual_ids=[1000],
                                   before_prefix_ids=[1, 1000])])


def test_replay_empty_and_signed_zero(tmp_path):
    """tests/test_replay_logits.py:40-61."""
    a, b = tmp_path / "a", tmp_path / "b"
    a.write_bytes(replay_capture()[:16])
    b.write_bytes(replay_capture()[:16])
    with pytest.raises(ValueError):
        art.compare_replay(a, b)
    with pytest.raises(ValueError):
        art.verify_replay(a, [])
    a.write_bytes(replay_capture())
    data = bytearray(replay_capture())
    offset = 16 + 16 + 2 * 4 + 4                      # the second logit, zero in a
    struct.pack_into("<f", data, offset, -0.0)
    b.write_bytes(bytes(data))
    assert not art.compare_replay(a, b)["match"]
    assert art.compare_replay(a, b, True)["match"]
    struct.pack_into("<f", data, offset, 0.00001)
    b.write_bytes(bytes(data))
    result = art.compare_replay(a, b, True)
    assert result["max_relative_error"] is None and result["relative_error_undefined_at_zero"]


def test_replay_rejections(tmp_path):
    """tests/test_replay_logits.py:63-82."""
    good = replay_capture()
    cases = [good[:-1], good + b"x", b"BADMAGIC" + good[8:],
             replay_capture(value=float("nan")), replay_capture(value=float("inf")),
             replay_capture(prefix=(V,)), replay_capture(forced=3),
             replay_capture(greedy=1, value=0)]
    for k, data in enumerate(cases):
        path = tmp_path / ("capture%d" % k)
        path.write_bytes(data)
        with pytest.raises(ValueError):
            art.parse_replay(path)
    large = tmp_path / "large"
    with open(large, "wb") as f:
        f.truncate(art.REPLAY_MAX_BYTES + 1)
    with pytest.raises(ValueError):
        art.parse_replay(large)
