"""Builds the gfx950 HIP backend (``libtqf_hip.so``) in-tree with hipcc.

The library is plain C ABI (``include/tqf_hip.h``); no torch extension is
involved.  Flags:
  --offload-arch=gfx950                    MI355X (CDNA4) only
  -fno-gpu-flush-denormals-to-zero         IEEE denormals, so the acceptance
                                           arithmetic matches the CPU bit for bit
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                           no packed-FP32 instructions
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "libtqf_hip.so"
SOURCES = ["tqf_q4.hip", "tqf_q4k.hip", "tqf_q6k.hip", "tqf_stack.hip", "tqf_grouped.hip",
           "tqf_accept.hip", "tqf_sample.hip", "tqf_experts.hip", "tqf_synth.hip", "tqf_loop.hip",
           "tqf_api.hip"]
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]
# Per-source additions.  The grouped GEMM keeps MFMA results in VGPRs (the
# per-block fp32 scaling reads every result; accumulators in AGPRs would cost
# a v_accvgpr_read per value).
EXTRA_FLAGS = {"tqf_grouped.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the HIP backend)")


def build(verbose: bool = False) -> Path:
    """Compiles every HIP source and links libtqf_hip.so next to this file."""
    hipcc = hipcc_path()
    build_dir = PKG_DIR / "_build"
    build_dir.mkdir(exist_ok=True)
    objs = []
    procs = []
    for src in SOURCES:
        obj = build_dir / (Path(src).stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(obj)]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        objs.append(obj)
    failed = []
    for cmd, p in procs:
        out, _ = p.communicate()
        text = "\n".join(
            line for line in out.decode(errors="replace").splitlines()
            if "packed-fp32-ops' is not a recognized feature" not in line
        )
        if p.returncode != 0:
            failed.append((cmd, text))
        elif verbose and text.strip():
            print(text, file=sys.stderr)
    if failed:
        msg = "\n\n".join(" ".join(c) + "\n" + t for c, t in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout.decode(errors="replace"))
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
