#!/usr/bin/env python3
"""Writes the committed golden fixtures under tests/golden/ (run here, where
/root/reference, hipcc and the oracle build exist; the fixtures travel, the
sources they come from do not).

  philox_vectors.txt   Philox4x32-10 known answers from ROCm's open-source
                       rocRAND header (philox_rocrand.cpp, built and run here).
  route_trace_ids.npy  uint8 [steps, 40, 8]: the expert ids of the reference's
                       committed real router trace
                       (docs/research/qualification/raw-a-128-route-trace.json),
                       the data of mtp.rs:310-343's union-bandwidth test.
  oracle_vectors.npz   CPU-oracle outputs on seeded inputs (config-1 GEMV,
                       a small MoE layer at M = 1 and 4, acceptance outcomes for
                       seeds 0..63 in greedy and stochastic modes).

Usage: python tests/golden/make_golden.py [--reference /root/reference]
"""
from __future__ import annotations

import argparse
import json
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(HERE))

from golden_inputs import (ACCEPT_K, SMALL, accept_inputs, gemv_inputs,  # noqa: E402
                           small_layer_inputs)

def philox_vectors() -> None:
    with tempfile.TemporaryDirectory() as td:
        exe = Path(td) / "philox_rocrand"
        subprocess.run(["/opt/rocm/bin/hipcc", "-O1", "-I/opt/rocm/include", "-o", str(exe),
                        str(HERE / "philox_rocrand.cpp")], check=True,
                       stderr=subprocess.DEVNULL)
        out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    (HERE / "philox_vectors.txt").write_text(out)


def route_trace(reference: Path) -> None:
    path = reference / "docs/research/qualification/raw-a-128-route-trace.json"
    trace = json.loads(path.read_text())
    steps = trace["steps"]
    n_layers = len(steps[0]["layers"])
    ids = np.zeros((len(steps), n_layers, 8), dtype=np.uint8)
    for s, step in enumerate(steps):
        for layer in step["layers"]:
            ids[s, layer["layer"]] = layer["expert_ids"]
    np.save(HERE / "route_trace_ids.npy", ids)


def oracle_vectors() -> None:
    import cpu_oracle as orc

    out = {}
    w1, x1 = gemv_inputs()
    out["gemv_y"] = orc.q4_0_matvec(w1, 512, 2048, x1)

    router, gate, x, mats = small_layer_inputs()
    E, H, F = SMALL["experts"], SMALL["hidden"], SMALL["width"]
    host = orc.MoeLayerHost(router, gate, *mats[E], [m[0] for m in mats[:E]],
                            [m[1] for m in mats[:E]], [m[2] for m in mats[:E]],
                            hidden=H, width=F)
    for m in (1, 4):
        y, ids, w = host.forward_batch(x[:m])
        out[f"moe_y{m}"], out[f"moe_ids{m}"], out[f"moe_w{m}"] = y, ids, w

    acc_len, acc_tok = [], []
    for greedy in (True, False):
        for seed in range(64):
            target, draft, dtok, u, ur = accept_inputs(seed)
            a, toks = orc.accept(target, draft, dtok, 0.7, greedy, u, ur)
            acc_len.append(a)
            acc_tok.append(toks + [-1] * (ACCEPT_K + 1 - len(toks)))
    out["accept_len"] = np.array(acc_len, dtype=np.int32).reshape(2, 64)
    out["accept_tokens"] = np.array(acc_tok, dtype=np.int32).reshape(2, 64, ACCEPT_K + 1)
    np.savez_compressed(HERE / "oracle_vectors.npz", **out)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    philox_vectors()
    route_trace(Path(args.reference))
    oracle_vectors()
    for p in sorted(HERE.iterdir()):
        print(f"{p.name:28s} {p.stat().st_size:9d} B")


if __name__ == "__main__":
    main()
