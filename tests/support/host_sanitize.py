"""The library with its host C under AddressSanitizer and
UndefinedBehaviorSanitizer, for CPU test runs (test infrastructure).

The host sources (lunelette_amd/csrc/*.c: checkpoint reader, tokenizer,
artifacts, session adapter, generation loop, runtime host code and the test
seams) are compiled by gcc with the sanitizers, as the reference builds its
host C (Makefile:92-93); the GPU objects are those of the shipped build
(lunelette_amd/_build/*.hip.o), not instrumented. A process that loads the
result must preload gcc's ASan and UBSan runtimes (preload())."""
import concurrent.futures
import glob
import os
import subprocess

from lunelette_amd import build

FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all",
         "-fno-omit-frame-pointer", "-g"]


def library(out_dir):
    """Builds the sanitized library into out_dir; returns its path."""
    os.makedirs(out_dir, exist_ok=True)
    if not glob.glob(os.path.join(build.OBJ, "*.hip.o")):
        build.build_library()
    inc = ["-I" + os.path.join(build.ROOT, "include"), "-I" + build.CSRC]

    def compile_host(src):
        obj = os.path.join(out_dir, os.path.basename(src) + ".o")
        build._run(["gcc"] + build.C_FLAGS + FLAGS + inc + ["-c", src, "-o", obj])
        return obj

    sources = sorted(glob.glob(os.path.join(build.CSRC, "*.c")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=8) as pool:
        host = list(pool.map(compile_host, sources))
    gpu = sorted(glob.glob(os.path.join(build.OBJ, "*.hip.o")))
    out = os.path.join(out_dir, "liblunelette_hip_sanitized.so")
    names = build.declared_functions(glob.glob(os.path.join(build.ROOT, "include", "*.h")) +
                                     [os.path.join(build.CSRC, "lh_test_seams.h")])
    build._link(out, host + gpu, names, os.path.join(out_dir, "exports.map"))
    return out


def preload():
    """LD_PRELOAD value with gcc's ASan and UBSan runtimes."""
    return ":".join(subprocess.run(["gcc", "-print-file-name=lib%s.so" % n],
                                   stdout=subprocess.PIPE, text=True, check=True).stdout.strip()
                    for n in ("asan", "ubsan"))
