"""Resource budget of every shipped gfx950 kernel (CPU: hipcc cross-compiles).

No kernel may use scratch memory: a private array the compiler cannot keep in
registers (a struct copied through memory, an array indexed by a runtime
value) either spills to scratch or is promoted into LDS, and both cost these
bandwidth-bound kernels tens of percent. LDS per workgroup stays within the
160 KiB of a gfx950 CU, and the unified register file (VGPR + AGPR) within 512.
"""
import glob
import os

import pytest

from lunelette_amd import build

SOURCES = sorted(glob.glob(os.path.join(build.CSRC, "*.hip")))


@pytest.mark.parametrize("src", SOURCES, ids=[os.path.basename(s) for s in SOURCES])
def test_kernels_use_no_scratch_and_fit_a_cu(src):
    if not os.path.exists(build.HIPCC):
        pytest.skip("hipcc not available")
    kernels = build.kernel_resources(src)
    assert kernels, "no kernels found in %s" % src
    for name, vgpr, agpr, lds, scratch in kernels:
        assert scratch == 0, "%s uses %d bytes of scratch" % (name, scratch)
        assert lds <= 160 * 1024, "%s uses %d bytes of LDS" % (name, lds)
        assert vgpr + agpr <= 512, "%s uses %d registers" % (name, vgpr + agpr)


def test_residual_prefetch_registers_untouched_until_waited():
    """The o and down row-dot kernels request their residual values with
    inline-assembly loads right after staging the input row (the compiler would
    sink an ordinary load to its use after the dots). The compiler does not
    know those registers are pending, so nothing may read or copy them before
    the explicit full wait that precedes their use: checked on every k_rows
    instantiation with a residual, in the gfx950 assembly of matvec.hip."""
    import re
    import subprocess
    import tempfile
    if not os.path.exists(build.HIPCC):
        pytest.skip("hipcc not available")
    src = os.path.join(build.CSRC, "matvec.hip")
    inc = ["-I" + os.path.join(build.ROOT, "include"), "-I" + build.CSRC]
    with tempfile.TemporaryDirectory() as tmp:
        out = os.path.join(tmp, "matvec.s")
        subprocess.run([build.HIPCC] + build.HIP_FLAGS + inc +
                       ["--cuda-device-only", "-S", src, "-o", out], check=True,
                       stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
        text = open(out).read()
    checked = 0
    for body in re.split(r"\n(?=_ZN2lh[^\n]*:)", text):
        name = body.split(":")[0]
        if not re.match(r"_ZN2lh6k_rowsI.*Lb1EEEv", name):
            continue
        lines = body.split("\n")
        loads = [i for i, l in enumerate(lines)
                 if re.match(r"\s+global_load_dword v\d+, v\[\d+:\d+\], off$", l)]
        assert loads, name
        for i in loads:
            reg = re.match(r"\s+global_load_dword (v\d+)", lines[i]).group(1)
            for line in lines[i + 1:]:
                if re.match(r"\s+s_waitcnt vmcnt\(0\)$", line):
                    break
                assert not re.search(r"\b%s\b" % reg, line), (name, reg, line)
            checked += 1
    assert checked >= 18
