"""The exact parallel f32 fold of the reference-exact sampler (the grid rule
of turboqwenfare_amd/csrc/tqf_fold.h, and the wavefront procedure of
tqf_sample.hip's fold_chunks / fold_row / fold_chunk_terms emulated lane by
lane) against the plain sequential f32 sum on the CPU: bit-identical sums and
the same inverse-CDF stopping index on the sampler's own terms (token order
and sorted), subnormal exponentials, exact ties at both parities, sums landing
on binade tops, multi-binade jumps, random bit patterns and NaN / +inf /
negative terms.  Two negative controls (the tie check removed; the binade-top
check removed) must each disagree somewhere."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def fold_check(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc is needed to compile the __host__ __device__ header")
    exe = tmp_path_factory.mktemp("fold") / "fold_check"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O2", "-std=c++17",
                    "-I", str(ROOT / "turboqwenfare_amd" / "csrc"),
                    str(ROOT / "tests" / "native" / "fold_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True)
    return exe


@pytest.mark.parametrize("seed", [1, 2])
def test_parallel_fold_equals_the_sequential_sum(fold_check, seed):
    out = subprocess.run([str(fold_check), str(seed)], check=True, capture_output=True, text=True).stdout
    last = out.strip().splitlines()[-1].split()
    rows, mism, ctl_tie, ctl_top = int(last[1]), int(last[3]), int(last[5]), int(last[7])
    assert rows > 300
    assert mism == 0, out
    assert ctl_tie > 0 and ctl_top > 0, "a negative control matched everywhere"
