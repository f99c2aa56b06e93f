"""tqf::ref_expf (turboqwenfare_amd/csrc/tqf_expf.h), the exponential of the
device's reference-exact sampler, against the host C library's expf -- the
f32::exp of the reference's softmax (sampling/mod.rs:166-190) -- on every
binary32 input that softmax can reach: all 2^31 - 2^23 + 1 patterns from -0
to -inf, +0 and NaNs.  The header's __host__ __device__ function is compiled
for the host with hipcc and swept on the CPU.  A copy of the evaluation with
one plausible slip (the reduction's r formed from a rounded product) runs as
a negative control and must differ somewhere."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def sweep(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc is needed to compile the __host__ __device__ header")
    exe = tmp_path_factory.mktemp("expf") / "expf_sweep"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O2", "-std=c++17",
                    "-I", str(ROOT / "turboqwenfare_amd" / "csrc"),
                    str(ROOT / "tests" / "native" / "expf_sweep.cpp"), "-o", str(exe), "-lpthread"],
                   check=True, capture_output=True)
    return exe


def test_ref_expf_equals_libm_expf_on_the_softmax_domain(sweep):
    out = subprocess.run([str(sweep), "control"], check=True, capture_output=True, text=True).stdout
    last = out.strip().splitlines()[-1].split()
    n, mism, ctl = int(last[1]), int(last[3]), int(last[5])
    assert n == (0xff800000 - 0x80000000 + 1) + 6
    assert mism == 0, out
    assert ctl > 0, "the negative control matched everywhere: the sweep would not see the slip"
