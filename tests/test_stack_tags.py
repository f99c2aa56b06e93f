"""The persistent stack kernel's partial-word tags over mixed-depth launch
sequences (CPU): the tag definitions of turboqwenfare_amd/csrc/tqf_tags.h,
compiled with g++, must never let a layer read a stale word that already
carries its tag -- across the 2^31 wrap too.  The earlier launch-count
definition is run as a negative control, started just before one of its
known collisions (a 1-layer draft stack after the 40-layer target)."""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "tests" / "native" / "stack_tags_check.cpp"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("tags") / "stack_tags_check"
    subprocess.run(["g++", "-std=c++17", "-O2", "-I", str(ROOT / "turboqwenfare_amd" / "csrc"),
                    str(SRC), "-o", str(exe)], check=True)
    return exe


def run(exe, scheme, start, launches, seed):
    r = subprocess.run([str(exe), str(scheme), str(start), str(launches), str(seed)],
                       capture_output=True, text=True)
    return r.returncode, r.stdout.strip()


@pytest.mark.parametrize("start", [0, 0x7FFFFFFF - 40, 0x7FFFFFFF - 1, 0x7FFFFFFF])
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_layer_step_tags_never_collide(checker, start, seed):
    rc, out = run(checker, 0, start, 200000, seed)
    assert rc == 0, out


def test_layer_step_tags_cross_the_wrap(checker):
    # starting one layer step below the wrap, the first launches straddle it
    rc, out = run(checker, 0, 0x7FFFFFFF, 10, 7)
    assert rc == 0, out


# the launch-count tags' first collisions: a 1-layer draft stack at seq s right
# after the 40-layer target (39 s = 1 mod 2^31), and the target at seq s
# right after the draft (39 s = -1 mod 2^31)
DRAFT_AFTER_TARGET = pow(39, -1, 2**31)       # 385,445,783
TARGET_AFTER_DRAFT = 2**31 - DRAFT_AFTER_TARGET  # 1,762,037,865


# alternating launches start with the target: the target at s - 3 puts the
# draft at s - 2 and s; the target at s - 2 puts the target at s
@pytest.mark.parametrize("start", [DRAFT_AFTER_TARGET - 3, TARGET_AFTER_DRAFT - 2])
def test_launch_count_tags_collide_for_mixed_depths(checker, start):
    # negative control: alternating target / draft launches from just before
    # a collision point; the check must see it
    rc, out = run(checker, 1, start, 10, 0)
    assert rc == 1 and out.startswith("collision"), out


@pytest.mark.parametrize("start", [DRAFT_AFTER_TARGET * 40 % 2**31, TARGET_AFTER_DRAFT * 40 % 2**31,
                                   2**31 - 41])
def test_layer_step_tags_alternating_depths(checker, start):
    rc, out = run(checker, 0, start, 100000, 0)
    assert rc == 0, out
