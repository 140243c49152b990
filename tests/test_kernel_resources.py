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
