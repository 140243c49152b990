"""The reference's own callers build against this library unchanged: its CLI
(src/main.c) and its native logit comparator (tests/compare_native.c) are
compiled from the reference checkout with include/compat/ (forwarding
headers named as the reference's: metal.h, generation.h, tokenizer.h, chat.h,
metal_weights.h) ahead of the reference's include/, and linked against
lunelette_amd/liblunelette_hip.so. The comparator also links the reference's
portable container reader src/safetensors.c, which is not one of the files
this library replaces. Compile and link only: nothing is run. Skipped where
the reference checkout is absent.
"""
import os
import shutil
import subprocess

import pytest

import lunelette_amd as lh

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"


def build(sources, out):
    if not os.path.isdir(REF):
        pytest.skip("the reference checkout is not present")
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    cmd = ["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror=implicit-function-declaration",
           "-I" + os.path.join(ROOT, "include", "compat"), "-I" + os.path.join(ROOT, "include"),
           "-I" + os.path.join(REF, "include"), "-I" + os.path.join(REF, "tests")]
    cmd += sources + ["-L" + os.path.dirname(lh.LIBRARY), "-llunelette_hip",
                      "-Wl,--no-undefined", "-lm", "-o", out]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert proc.returncode == 0, proc.stdout
    assert os.path.getsize(out) > 0


def test_cli_main_links(tmp_path):
    build([os.path.join(REF, "src", "main.c")], str(tmp_path / "lunelette"))


def test_native_comparator_links(tmp_path):
    build([os.path.join(REF, "tests", "compare_native.c"), os.path.join(REF, "src",
                                                                        "safetensors.c")],
          str(tmp_path / "compare_native"))
