"""The host C under AddressSanitizer and UndefinedBehaviorSanitizer.

The reference runs its host C under ASan and UBSan (Makefile:92-93,
docs/development/testing.md:41-52). Here the host sources that parse
untrusted input or own heap memory (checkpoint container and tensor contract,
tokenizer and its JSON reader, LUN1/LUN2 and LNRPLY1 artifacts, session
adapter, generation loop, runtime host code) are rebuilt by gcc with both
sanitizers (tests/support/host_sanitize.py), and the CPU suites that drive
them run again in a child process against that build with gcc's runtimes
preloaded: the checkpoint header mutations and truncations, the tokenizer's
defective files, JSON grammar and random texts, the LUN2 mutations, the
session contract (its stub build sanitized too), the generation differential
and the allocation-failure cases. Any sanitizer report aborts the child
(-fno-sanitize-recover=all). A planted heap overflow and a planted signed
overflow, built and loaded the same way, must be reported, so the runtimes are
known to be live in such a process.
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SUITES = ["tests/test_checkpoint_format.py", "tests/test_tokenizer.py", "tests/test_artifacts.py",
          "tests/test_session_contract.py", "tests/test_generation_diff.py",
          "tests/test_admission.py"]

PLANTED = r"""
#include <limits.h>
#include <stdlib.h>
#include <string.h>
int planted_overflow(int n)
{
    char *p = malloc(16);
    memset(p, 1, 16);
    int v = p[n];
    free(p);
    return v;
}
int planted_signed(int n)
{
    return INT_MAX - 1 + n;
}
"""


@pytest.fixture(scope="module")
def sanitized(tmp_path_factory):
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from support import host_sanitize
    out = tmp_path_factory.mktemp("sanitized")
    return host_sanitize, host_sanitize.library(str(out)), out


def child_env(host_sanitize, library):
    env = dict(os.environ)
    env.update(LH_SANITIZED_LIBRARY=library, LD_PRELOAD=host_sanitize.preload(),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    return env


@pytest.mark.parametrize("sanitizer,call,report", [
    ("address", "planted_overflow(16)", "heap-buffer-overflow"),
    ("undefined", "planted_signed(2)", "signed integer overflow")])
def test_instrumentation_reports_planted_mistakes(sanitized, sanitizer, call, report):
    """Each runtime reports its planted mistake in a process set up like the
    suites' (the in-bounds call before it returns normally)."""
    host_sanitize, library, out = sanitized
    src, lib = out / "planted.c", out / ("libplanted_%s.so" % sanitizer)
    src.write_text(PLANTED)
    subprocess.run(["gcc", "-O1", "-fPIC", "-shared", "-fsanitize=" + sanitizer,
                    "-fno-sanitize-recover=all", str(src), "-o", str(lib)], check=True)
    code = ("import ctypes; l = ctypes.CDLL(%r); print(l.planted_overflow(3), l.planted_signed(1), "
            "flush=True); l.%s" % (str(lib), call))
    proc = subprocess.run([sys.executable, "-c", code], env=child_env(host_sanitize, library),
                          stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
    assert proc.stdout.split() == ["1", str(2 ** 31 - 1)]
    assert proc.returncode != 0 and report in proc.stderr, proc.stderr[-2000:]


def test_host_suites_pass_under_sanitizers(sanitized):
    host_sanitize, library, out = sanitized
    proc = subprocess.run(
        [sys.executable, "-m", "pytest", "-x", "-q", "-m", "not gpu", "-p", "no:cacheprovider",
         "--basetemp", str(out / "tmp")] + SUITES,
        cwd=ROOT, env=child_env(host_sanitize, library), stdout=subprocess.PIPE,
        stderr=subprocess.STDOUT, text=True)
    tail = proc.stdout[-6000:]
    assert proc.returncode == 0, tail
    assert "AddressSanitizer" not in proc.stdout and "runtime error:" not in proc.stdout, tail
    assert " passed" in tail and "failed" not in tail, tail
