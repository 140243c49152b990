"""Builds the gfx950 library lunelette_amd/liblunelette_hip.so in-tree.

HIP sources are compiled by hipcc for gfx950 only; the C host runtime by gcc
against the ROCm headers; everything links into one shared library whose C-ABI
is declared in include/*.h. Also builds the CPU oracle (test infrastructure)
and, when the reference checkout is present, oracle/_ref.
"""
import concurrent.futures
import glob
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "lunelette_amd")
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "liblunelette_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    # Packed FP32 instructions stay off (the compiler would otherwise form them).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-parameter",
]
C_FLAGS = [
    "-std=c11", "-O2", "-fPIC", "-ffp-contract=off", "-pthread", "-Wall", "-Wextra",
    "-D__HIP_PLATFORM_AMD__", "-I" + os.path.join(ROCM, "include"),
]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError("command failed: %s\n%s" % (" ".join(cmd), out))
    return out


def _compile(src):
    base = os.path.basename(src)
    obj = os.path.join(OBJ, base + ".o")
    inc = ["-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
    if src.endswith(".hip"):
        cmd = [HIPCC] + HIP_FLAGS + inc + ["-c", src, "-o", obj]
    else:
        cmd = ["gcc"] + C_FLAGS + inc + ["-c", src, "-o", obj]
    _run(cmd)
    return obj


def kernel_resources(src):
    """Per-kernel resources of one HIP source as compiled for gfx950:
    [(name, vgpr, agpr, lds_bytes, scratch_bytes)], from the code-object
    metadata of a device-only assembly build with the library's flags."""
    import re
    import tempfile
    inc = ["-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
    with tempfile.TemporaryDirectory() as tmp:
        out = os.path.join(tmp, "k.s")
        _run([HIPCC] + HIP_FLAGS + inc + ["--cuda-device-only", "-S", src, "-o", out])
        text = open(out).read()
    kernels = []
    for block in text.split("  - .agpr_count:")[1:]:
        def field(key):
            m = re.search(r"\." + key + r":\s+(\S+)", block)
            return m.group(1) if m else None
        kernels.append((field("name"), int(field("vgpr_count")), int(block.split()[0]),
                        int(field("group_segment_fixed_size")),
                        int(field("private_segment_fixed_size"))))
    return kernels


def build_library(jobs=8):
    os.makedirs(OBJ, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.c")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objects +
         ["-lpthread", "-lm"])
    os.replace(tmp, LIB)
    return LIB


def build_oracle():
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")])
    ref = "/root/reference"
    if os.path.isdir(ref):
        _run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "-f", "Makefile.ref",
              "REF=" + ref])


def build_all():
    build_library()
    build_oracle()


if __name__ == "__main__":
    build_all()
    print(LIB, file=sys.stderr)
