"""Builds the gfx950 library lunelette_amd/liblunelette_hip.so in-tree.

HIP sources are compiled by hipcc for gfx950 only; the C host runtime by gcc
against the ROCm headers; everything links into one shared library that
exports exactly the C-ABI declared in include/*.h (a linker version script
keeps every internal symbol local). The same objects plus test_seams.c link
into liblunelette_hip_test.so, which also exports the host-forced failure
seams of csrc/lh_test_seams.h for the runtime's state-machine tests. Also
builds the CPU oracle (test infrastructure) and, when the reference checkout
is present, oracle/_ref.
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
TEST_LIB = os.path.join(PKG, "liblunelette_hip_test.so")
TEST_ONLY = ("test_seams.c",)
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


def declared_functions(headers):
    """Function names (lunelette_* / lh_*) declared in the given C headers."""
    import re
    names = set()
    for header in headers:
        with open(header) as f:
            text = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
        for m in re.finditer(r"\b((?:lunelette|lh)_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names - {"lunelette_logits_fn"})


def _version_script(path, names):
    with open(path, "w") as f:
        f.write("{\n  global:\n")
        for name in names:
            f.write("    %s;\n" % name)
        f.write("  local: *;\n};\n")


def _link(out, objects, names, script):
    _version_script(script, names)
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objects +
         ["-Wl,--version-script=" + script, "-lpthread", "-lm"])
    os.replace(tmp, out)


def build_library(jobs=8):
    os.makedirs(OBJ, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.c")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(_compile, sources))
    shipped = [o for o, src in zip(objects, sources) if os.path.basename(src) not in TEST_ONLY]
    abi = declared_functions(glob.glob(os.path.join(ROOT, "include", "*.h")))
    _link(LIB, shipped, abi, os.path.join(OBJ, "exports.map"))
    seams = declared_functions([os.path.join(CSRC, "lh_test_seams.h")])
    _link(TEST_LIB, objects, abi + seams, os.path.join(OBJ, "exports_test.map"))
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
