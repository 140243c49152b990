"""bench.py's command-line contract and its timed decode loop, on the CPU.

The loop is exercised against a stand-in library whose decode and greedy
calls record what they were given, so the token hand-off between steps and
the device-time sampling are checked without a GPU.
"""
import ctypes
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                          stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=120)
    assert proc.returncode == 2
    assert proc.stdout == ""
    assert "one MI355X" in proc.stderr and "--gpus 2" in proc.stderr


class _StandIn:
    """The three C entry points decode_loop calls, in Python."""

    def __init__(self, fail_at=None):
        self.decoded, self.selected, self.device_calls = [], 0, 0
        self.fail_at = fail_at

    def lunelette_metal_decode(self, handle, token, logits_ref, err, capacity):
        assert handle == "ctx" and capacity == 512
        self.decoded.append(token)
        if self.fail_at is not None and len(self.decoded) == self.fail_at:
            err.value = b"planted failure"
            return -1
        return 0

    def lunelette_select_greedy(self, logits, token_ref, err, capacity):
        # The next token is a function of the one just decoded.
        token = token_ref._obj
        token.value = (token.value * 7 + 3) % 131072
        self.selected += 1
        return 0

    def lunelette_metal_last_device_ms(self, handle, ms_ref):
        self.device_calls += 1
        ms_ref._obj.value = 1.0 + self.device_calls
        return 0


class _Runtime:
    def __init__(self, lib):
        self._lib, self.handle = lib, "ctx"
        self._err = ctypes.create_string_buffer(512)
        self._logits = ctypes.POINTER(ctypes.c_float)()


def test_decode_loop_hands_each_token_to_the_next_step():
    lib = _StandIn()
    rt = _Runtime(lib)
    tokens = bench.decode_loop(rt, 11, 20, 8)
    want, t = [], 11
    for _ in range(20):
        t = (t * 7 + 3) % 131072
        want.append(t)
    assert tokens == want
    assert lib.decoded == [11] + want[:-1]
    assert lib.selected == 20
    # Steps 0, 8 and 16 report their device time.
    assert lib.device_calls == 3
    assert rt.sampled_device_ms == [2.0, 3.0, 4.0]


def test_decode_loop_stops_at_a_failed_call():
    lib = _StandIn(fail_at=4)
    rt = _Runtime(lib)
    try:
        bench.decode_loop(rt, 5, 10, 1)
    except RuntimeError as e:
        assert "planted failure" in str(e)
    else:
        raise AssertionError("a failed decode call must raise")
    assert len(lib.decoded) == 4 and lib.selected == 3
