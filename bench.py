#!/usr/bin/env python3
"""MTP k=3 verify-step benchmark on one MI355X.

One step = the full-depth verify pass over the k+1 = 4 verify rows: 40
stacked MoE FFN layers h <- h + MoE_l(rmsnorm_l(h)) (model/qwen36/runtime.rs:
777-802), each with its own seeded Q4_0 experts resident in HBM (256 routed +
1 shared per layer, 18.2 GB), router softmax top-8 + gated shared expert +
SwiGLU experts, followed by acceptance sampling over fp32 logits [4, 151936]
at T = 0.7 with Philox uniforms.  Inputs are resident in HBM before timing.

The headline experts use the zero-mean nibble recipe (q - 8 symmetric on
[-7, 7]), under which the four rows keep routing apart (expert union ~30 per
layer, the i.i.d. expectation).  The literal recipe (nibbles uniform on
0..15, E[q - 8] = -0.5) gives every matrix a common-mode component that
collapses the rows onto one direction within a few layers (union ~10); its
figure is reported beside the headline as a side key.

Prints ONE JSON line (progress goes to stderr).  `value` is verify steps/s.
The roofline object is for the dominant kernel (the persistent stack kernel,
one cooperative launch per step) timed with HIP events on the library's
stream; `cpu_baseline` is the
reference's scalar path (the C restatement in oracle/) timed on this host's
cores on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
E, H, F, V, K = 256, 2048, 512, 151936, 3
M = K + 1
TEMPERATURE = 0.7


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_model(be, n_layers: int, seed: int, recipe: str):
    """Seeded synthetic n_layers-layer weight set generated directly in HBM."""
    from turboqwenfare_amd.workloads import SyntheticStack

    return SyntheticStack(be, n_layers, seed, recipe, log=lambda m: log("bench: " + m))


def verify_inputs(seed: int):
    from turboqwenfare_amd import synth

    rng = np.random.default_rng(seed)
    target = (rng.standard_normal((M, V)) * 3.0).astype(np.float32)
    draft = (rng.standard_normal((K, V)) * 3.0).astype(np.float32)
    dtok = np.argmax(draft, axis=1).astype(np.int32)
    u = synth.philox_uniforms(seed, 0, K)
    ur = synth.philox_uniforms(seed, 1, K + 1)
    h0 = synth.normal((M, H), seed=seed + 1)
    return target, draft, dtok, u, ur, h0


def host_cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(model, inputs, budget_s: float):
    """The reference's portable scalar path (C restatement, -O3
    -ffp-contract=off) on this host: MoE layers at M = 4 plus the acceptance
    at V = 151936, timed on a bounded sample of layers and scaled to 40."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import cpu_oracle as orc  # the baseline being timed (not the GPU path)

    target, draft, dtok, u, ur, h0 = inputs
    threads = int(os.environ.get("OMP_NUM_THREADS") or len(os.sched_getaffinity(0)))
    n_sample = min(4, model.n_layers)
    hosts, norm_host = [], []
    for l in range(n_sample):
        router, gate, norm = model.host_f32[l]
        ex = [model.expert_q4_0(l, e) for e in range(E + 1)]
        hosts.append(orc.MoeLayerHost(router, gate, *ex[E], [x[0] for x in ex[:E]],
                                      [x[1] for x in ex[:E]], [x[2] for x in ex[:E]]))
        norm_host.append(norm)

    def run_layers(nthreads):
        h = h0.copy()
        for Lh, nw in zip(hosts, norm_host):
            xn = np.stack([orc.qwen_rmsnorm(h[t], nw) for t in range(M)])
            y, _, _ = Lh.forward_batch(xn, nthreads=nthreads)
            h = h + y

    def timed(fn, min_s):
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t0
            if el >= min_s or reps >= 50:
                return el / reps

    res = {}
    t_acc = timed(lambda: orc.accept(target, draft, dtok, TEMPERATURE, False, u, ur), 0.5)
    for nt in sorted({1, threads}):
        per_sample = timed(lambda: run_layers(nt), budget_s / 2)
        per_step = per_sample / n_sample * model.n_layers + t_acc
        res[nt] = 1.0 / per_step
        log(f"bench: cpu {nt} thread(s): {per_sample / n_sample * 1e3:.1f} ms/layer, "
            f"{per_step * 1e3:.1f} ms/step")
    return res, threads, n_sample


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix-core peak
GROUPED_TOKENS = 512


def grouped_gemm_bench(be, layer, seed: int, iters: int = 20, cases=("zipf", "dense8")):
    """Config 5 on one resident layer: 512 bf16 tokens with Zipf(1.1)
    Gumbel-top-k routes (seed 0), timed per kernel with HIP events; plus the
    same pair count routed to 8 experts only (every expert M = 512), which
    isolates the matrix-core rate of the two GEMM kernels."""
    from turboqwenfare_amd import _lib, mtp, synth

    T = GROUPED_TOKENS
    x = synth.bf16_round(synth.normal((T, H), seed=seed + 50))
    zipf_ids, zipf_w = synth.zipf_routes(T, E, 8, 1.1, 0)
    dense_ids = np.tile(np.arange(8, dtype=np.uint16), (T, 1))
    dx, dy = be.to_device(x), be.alloc(T * H * 4)
    flops = 6.0 * H * F * T * 8  # gate + up (2 H F each) + down (2 H F) per pair
    out = {"tokens": T, "pairs": T * 8, "algorithmic_gflop": flops / 1e9}
    for name, ids, w in (("zipf", zipf_ids, zipf_w), ("dense8", dense_ids, zipf_w)):
        if name not in cases:
            continue
        dids, dw = be.to_device(ids), be.to_device(w)
        for _ in range(3):
            be.grouped_gemm_device(layer, dx, T, dids, dw, dy)
        be.profile_enable(True)
        for _ in range(iters):
            be.grouped_gemm_device(layer, dx, T, dids, dw, dy)
        per = {}
        for kind, nm in ((_lib.KERNEL_GROUPED_GATE_UP, "gate_up"),
                         (_lib.KERNEL_GROUPED_DOWN, "down"), (_lib.KERNEL_GROUPED_AUX, "aux")):
            n, ms, _ = be.profile_read(kind)
            per[nm] = ms / iters * 1e3  # us per call (aux: plan + combine)
        be.profile_enable(False)
        distinct = len(np.unique(ids))
        weight_bytes = distinct * mtp.expert_bytes_q4_0()
        algo_bytes = weight_bytes + T * H * 2 + T * 8 * 6 + T * H * 4
        total_us = per["gate_up"] + per["down"] + per["aux"]
        gemm_us = per["gate_up"] + per["down"]
        out[name] = {
            "distinct_experts": distinct,
            "head_expert_pairs": int(np.bincount(ids.reshape(-1).astype(np.int64)).max()),
            "us": total_us, "kernel_us": per,
            "algorithmic_bytes": algo_bytes,
            "hbm_gbs": algo_bytes / (total_us * 1e-6) / 1e9,
            "hbm_frac": algo_bytes / (total_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "gemm_tflops": flops / (gemm_us * 1e-6) / 1e12,
            "mfma_util": flops / (gemm_us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        }
        be.free(dids)
        be.free(dw)
    be.free(dx)
    be.free(dy)
    return out


def q4k_pool_bench(be, pool_size: int, seed: int, iters: int = 10):
    """Canonical Q4_K GEMVs at the config-1 shape (512 x 2048, m = 1) over a
    rotating pool of distinct device matrices (one launch reads every one):
    the fp32-semantics GEMV (backend::reference::q4k_gemv) and the Q8_K
    integer matvec (matvec_payload / q4_k_dot_pre).  Every pool matrix is a
    device copy of one seeded Q4_K matrix with f16 d, dmin in [0.002, 0.05)."""
    from turboqwenfare_amd import _lib, synth

    rng = np.random.default_rng(seed)
    n = 512 * (2048 // 256)
    blk = rng.integers(0, 256, size=(n, 144), dtype=np.uint8)
    blk[:, 0:2] = rng.uniform(0.002, 0.05, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    blk[:, 2:4] = rng.uniform(0.002, 0.05, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    host = blk.reshape(-1)
    pool = [be.upload_q4_k(host, 512, 2048) for _ in range(pool_size)]
    dx = be.to_device(synth.normal((2048,), seed=seed))
    dy = be.alloc(pool_size * 512 * 4)
    out = {}
    for name, fn, kind in (("gemv_fp32", be.q4k_gemv_batched_device, _lib.KERNEL_Q4K_GEMV),
                           ("matvec_q8k", be.q4k_matvec_batched_device, _lib.KERNEL_Q4K_MATVEC)):
        fn(pool, dx, dy)
        be.profile_enable(True)
        for _ in range(iters):
            fn(pool, dx, dy)
        n_l, ms, by = be.profile_read(kind)
        be.profile_enable(False)
        r = dict(matrices=pool_size, bytes_per_launch=by / n_l, avg_us=ms / n_l * 1e3,
                 gbs=by / (ms * 1e-3) / 1e9)
        r["frac"] = r["gbs"] / HBM_PEAK_GBS
        out[name] = r
    for w in pool:
        be.free_weights(w)
    be.free(dx)
    be.free(dy)
    return out


def q4k_verify_bench(be, n_layers: int, seed: int, inputs, steps: int = 50, warmup: int = 5):
    """Config 4 with the canonical checkpoint's expert format: the same
    n_layers verify step (RMSNorm, route, experts, residual per layer, then
    the acceptance) with Q4_K experts, every expert matvec on the Q8_K
    integer path (bit-identical per matvec to q4_k_dot_pre).  The experts are
    device repacks of 8 seeded centred GGML Q4_K matrices per shape, each at
    its own HBM address."""
    from turboqwenfare_amd import _lib, mtp
    from turboqwenfare_amd.workloads import SyntheticQ4KStack

    target, draft, dtok, u, ur, h0 = inputs
    model = SyntheticQ4KStack(be, n_layers, seed)
    st = model.stack
    d = {k: be.to_device(v) for k, v in dict(t=target, d=draft, dt=dtok, u=u, ur=ur, h0=h0,
                                              h=h0).items()}
    d_acc, d_tok = be.alloc(4), be.alloc(4 * M)

    def step():
        be.verify_step_device(st, d["h0"], d["h"], M, d["t"], d["d"], d["dt"], V, TEMPERATURE,
                              False, d["u"], d["ur"], d_acc, d_tok)

    for _ in range(warmup):
        step()
    be.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    be.synchronize()
    elapsed = (time.perf_counter() - t0) / steps
    be.profile_enable(True)
    for _ in range(5):
        step()
    be.synchronize()
    prof = {}
    for kind, nm in ((_lib.KERNEL_ROUTE, "route"), (_lib.KERNEL_Q4K_MATVEC, "q4k_matvec"),
                     (_lib.KERNEL_ACCEPT, "accept")):
        n, ms, by = be.profile_read(kind)
        if n:
            prof[nm] = dict(launches=n, avg_us=ms / n * 1e3)
    be.profile_enable(False)
    # algorithmic bytes of one stack pass: each layer's router, norm and the
    # GGML bytes of its (union + shared) experts
    d_ids = be.alloc(n_layers * M * 8 * 2)
    d_tmp = be.alloc(M * H * 4)
    be.stack_forward_device(st, d_tmp, M, d_ids, d_h_in=d["h0"])
    ids = be.read(d_ids, np.uint16, (n_layers, M, 8))
    unions = [len(mtp.routes_union(ids[l])) for l in range(n_layers)]
    stack_bytes = sum((un + 1) * 3 * F * (H // 256) * 144 + (E + 1) * H * 4 + H * 4
                      for un in unions) + 2 * M * H * 4
    out = dict(layers=n_layers, m=M, format="q4_k", steps_per_s=1.0 / elapsed,
               ms_per_step=elapsed * 1e3, expert_union_mean=float(np.mean(unions)),
               stack_bytes_per_step=stack_bytes, kernels=prof)
    for b in list(d.values()) + [d_acc, d_tok, d_ids, d_tmp]:
        be.free(b)
    model.free()
    return out


def gemv_pool_bench(be, n_mats: int, seed: int):
    """Config-1 GEMV bandwidth: one token against a rotating pool of distinct
    512 x 2048 Q4_0 matrices (far beyond the 256 MB Infinity Cache), one launch
    per call: HIP events around the GEMV kernel (avg_us, gbs, frac), and the
    host clock around whole calls, which add the x-record prep kernel and its
    launch gap (call_us, call_gbs, call_frac)."""
    from turboqwenfare_amd import _lib, synth

    pool = [be.synth_q4_0(512, 2048, 900_000 + i, seed) for i in range(n_mats)]
    dx = be.to_device(synth.normal((2048,), seed=seed))
    dy = be.alloc(n_mats * 512 * 4)
    be.q4_gemv_batched_device(pool, dx, dy)
    be.profile_enable(True)
    for _ in range(10):
        be.q4_gemv_batched_device(pool, dx, dy)
    n, ms, by = be.profile_read(_lib.KERNEL_GEMV)
    be.profile_enable(False)
    gemv = dict(matrices=n_mats, bytes_per_launch=by / n, avg_us=ms / n * 1e3, gbs=by / (ms * 1e-3) / 1e9)
    gemv["frac"] = gemv["gbs"] / HBM_PEAK_GBS
    # the whole call: the x-record prep kernel, the GEMV and the gap between
    # them (stream-ordered calls, host clock around 20 of them)
    be.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        be.q4_gemv_batched_device(pool, dx, dy)
    be.synchronize()
    call_s = (time.perf_counter() - t0) / 20
    gemv.update(call_us=call_s * 1e6, call_gbs=gemv["bytes_per_launch"] / call_s / 1e9)
    gemv["call_frac"] = gemv["call_gbs"] / HBM_PEAK_GBS
    for w in pool:
        be.free_weights(w)
    be.free(dx)
    be.free(dy)
    return gemv


def lm_head_bench(be, seed: int, iters: int = 20):
    """The LM head at the configs' vocabulary: Q6_K [151,936 x 2048] (255 MB,
    the canonical checkpoint's lm_head format) against the M = 4 verify rows,
    bit-exact Q8_K logits plus the fused top-4 candidates per row."""
    from turboqwenfare_amd import _lib, synth

    rng = np.random.default_rng(seed)
    n = V * (H // 256)
    blk = rng.integers(0, 256, size=(n, 210), dtype=np.uint8)
    blk[:, 208:210] = rng.uniform(0.001, 0.05, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    w = be.upload_q6_k(blk.reshape(-1), V, H)
    del blk
    out = {"vocab": V, "hidden": H, "format": "q6_k", "bytes_weights": V * (H // 256) * 210}
    for m in (1, M):
        dx = be.to_device(synth.normal((m, H), seed=seed + m))
        dy, dt, dl = be.alloc(m * V * 4), be.alloc(m * 16), be.alloc(m * 16)
        be.lm_head_logits_device(w, dx, m, dy, dt, dl)
        be.synchronize()
        be.profile_enable(True)
        t0 = time.perf_counter()
        for _ in range(iters):
            be.lm_head_logits_device(w, dx, m, dy, dt, dl)
        be.synchronize()
        call_us = (time.perf_counter() - t0) / iters * 1e6
        n_l, ms, by = be.profile_read(_lib.KERNEL_Q6K_MATVEC)
        be.profile_enable(False)
        r = dict(m=m, kernel_us=ms / n_l * 1e3, call_us=call_us, bytes_per_launch=by / n_l,
                 gbs=by / (ms * 1e-3) / 1e9)
        r["frac"] = r["gbs"] / HBM_PEAK_GBS
        out[f"m{m}"] = r
        for b in (dx, dy, dt, dl):
            be.free(b)
    be.free_weights(w)
    return out


def sampler_bench(be, seed: int, iters: int = 20):
    """One token from one row of V = 151,936 logits: the acceptance's draw at
    k = 0 (exact fixed-point sums, the loop's default pick) beside the
    reference-exact Sampler::select (sequential f32 sums, a sort), on the
    bench's N(0, 9) logits at T = 0.7 (about 38k and 28k terms in the two
    sums) and on flat N(0, 0.01) logits at T = 1 (every term in both).
    Host wall time per synchronised call, and the select's kernels by HIP
    events."""
    from turboqwenfare_amd import _lib

    out = {}
    d_acc, d_tok, d_u = be.alloc(4), be.alloc(4), be.to_device(np.array([0.37], np.float32))
    for name, scale, T in (("peaked", 3.0, TEMPERATURE), ("flat", 0.1, 1.0)):
        lg = (np.random.default_rng(seed).standard_normal(V) * scale).astype(np.float32)
        d = be.to_device(lg)
        r = {}
        for path in ("accept_draw", "sampler_select"):
            def call():
                if path == "accept_draw":
                    be.accept_device(d, d, d_tok, 0, V, T, False, d_u, d_u, d_acc, d_tok)
                else:
                    be.sampler_select_device(d, 1, V, T, d_u, d_tok)
            call()
            be.synchronize()
            be.profile_enable(True)
            t0 = time.perf_counter()
            for _ in range(iters):
                call()
                be.synchronize()
            r[f"{path}_call_us"] = (time.perf_counter() - t0) / iters * 1e6
            kind = _lib.KERNEL_ACCEPT if path == "accept_draw" else _lib.KERNEL_SAMPLE
            n, ms, _ = be.profile_read(kind)
            be.profile_enable(False)
            r[f"{path}_gpu_us"] = ms / n * 1e3 if n else None
        out[name] = r
        be.free(d)
    for b in (d_acc, d_tok, d_u):
        be.free(b)
    return out


def verify_bench(be, model, inputs, steps: int, warmup: int, greedy: bool, distribution=True):
    """Config 4 on a resident model: verify steps/s (stream-ordered), the
    per-step distribution, HIP-event kernel times of eager launches, and the
    algorithmic bytes of the dominant kernel from the routes of the same input."""
    from turboqwenfare_amd import _lib, mtp

    target, draft, dtok, u, ur, h0 = inputs
    d = {k: be.to_device(v) for k, v in dict(t=target, d=draft, dt=dtok, u=u, ur=ur, h0=h0,
                                              h=h0).items()}
    d_acc, d_tok = be.alloc(4), be.alloc(4 * M)
    d_st = be.to_device(np.zeros(1, np.int32))
    st = model.stack

    def step():
        be.verify_step_device(st, d["h0"], d["h"], M, d["t"], None if greedy else d["d"],
                              d["dt"], V, TEMPERATURE, greedy, d["u"], d["ur"], d_acc, d_tok, d_st)

    for _ in range(warmup):
        step()
    be.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    be.synchronize()
    elapsed = time.perf_counter() - t0
    status = int(be.read(d_st, np.int32, (1,))[0])
    if status != 0:
        raise RuntimeError(f"verify step reported device status {status}")
    out = dict(steps_per_s=steps / elapsed, ms_per_step=elapsed / steps * 1e3)
    if distribution:
        # each step synchronised on its own (so each sample also holds one
        # launch + synchronise round trip)
        per_step = []
        for _ in range(steps):
            t1 = time.perf_counter()
            step()
            be.synchronize()
            per_step.append((time.perf_counter() - t1) * 1e3)
        q10, q50, q90 = (float(v) for v in np.percentile(per_step, [10, 50, 90]))
        out["synchronised_step_ms"] = {"p10": q10, "median": q50, "p90": q90}
    # kernel timing with HIP events on the library stream (eager launches)
    be.profile_enable(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    be.synchronize()
    out["eager_profiled_ms_per_step"] = (time.perf_counter() - t0) / steps * 1e3
    prof = {}
    for kind, nm in ((_lib.KERNEL_STACK, "stack"), (_lib.KERNEL_ROUTE, "route"),
                     (_lib.KERNEL_GATE_UP, "gate_up"), (_lib.KERNEL_DOWN, "down"),
                     (_lib.KERNEL_ACCEPT, "accept")):
        n, ms, by = be.profile_read(kind)
        if n:
            prof[nm] = dict(launches=n, avg_us=ms / n * 1e3, bytes_per_launch=by / n,
                            gbs=by / (ms * 1e-3) / 1e9 if ms > 0 else 0.0)
    be.profile_enable(False)
    # algorithmic HBM bytes of one stack pass: every layer's router (f32
    # [E+1 x H] incl. the shared input gate), RMSNorm weight and the Q4_0
    # bytes of its (union + shared) experts, from the routes of the same input
    n_layers = model.n_layers
    d_ids = be.alloc(n_layers * M * 8 * 2)
    d_tmp = be.alloc(M * H * 4)
    be.stack_forward_device(st, d_tmp, M, d_ids, d_h_in=d["h0"])
    ids = be.read(d_ids, np.uint16, (n_layers, M, 8))
    unions = [len(mtp.routes_union(ids[l])) for l in range(n_layers)]
    stack_bytes = sum((un + 1) * mtp.expert_bytes_q4_0() + (E + 1) * H * 4 + H * 4
                      for un in unions) + 2 * M * H * 4
    accept_bytes = (2 * K + 1) * V * 4 if not greedy else (K + 1) * V * 4
    if "stack" in prof:
        prof["stack"]["bytes_per_launch"] = stack_bytes
        prof["stack"]["gbs"] = stack_bytes / (prof["stack"]["avg_us"] * 1e-6) / 1e9
    if "accept" in prof:
        prof["accept"]["bytes_per_launch"] = accept_bytes
        prof["accept"]["gbs"] = accept_bytes / (prof["accept"]["avg_us"] * 1e-6) / 1e9
    out["kernels"] = prof
    out["expert_union"] = {"mean": float(np.mean(unions)), "min": int(min(unions)),
                           "max": int(max(unions))}
    out["stack_algorithmic_bytes"] = stack_bytes
    for b in list(d.values()) + [d_acc, d_tok, d_st, d_ids, d_tmp]:
        be.free(b)
    return out


def stack_m1_bench(be, model, seed: int, iters: int = 20):
    """The 40-layer stack at M = 1 (decode): HIP-event time of the stack
    kernel per launch and per layer, with its algorithmic bytes."""
    from turboqwenfare_amd import _lib, mtp, synth

    h0 = synth.normal((1, H), seed=seed + 1)
    dh0, dh = be.to_device(h0), be.alloc(H * 4)
    be.stack_forward_device(model.stack, dh, 1, d_h_in=dh0)
    be.profile_enable(True)
    for _ in range(iters):
        be.stack_forward_device(model.stack, dh, 1, d_h_in=dh0)
    n, ms, _ = be.profile_read(_lib.KERNEL_STACK)
    if not n:  # a device without the persistent path: the per-layer kernels
        n, ms = iters, sum(be.profile_read(k)[1] for k in (_lib.KERNEL_ROUTE, _lib.KERNEL_GATE_UP,
                                                           _lib.KERNEL_DOWN))
    be.profile_enable(False)
    nb = model.n_layers * (9 * mtp.expert_bytes_q4_0() + (E + 1) * H * 4 + H * 4) + 2 * H * 4
    us = ms / n * 1e3
    be.free(dh0)
    be.free(dh)
    return dict(m=1, layers=model.n_layers, avg_us=us, per_layer_us=us / model.n_layers,
                algorithmic_bytes=nb, gbs=nb / (us * 1e-6) / 1e9,
                frac=nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS)


def layer_bench(be, model, inputs, m: int, with_accept: bool, seed: int, iters: int = 50):
    """Configs 2 and 3: one MoE layer (layer 0 of the resident model) through
    tqf_hip_moe_layer_device at M = m with x ~ N(0, 1), plus (config 3) the
    stochastic acceptance over the [4, V] logits; HIP-event kernel times and
    the algorithmic bytes of the layer's own routes."""
    from turboqwenfare_amd import _lib, mtp, synth

    target, draft, dtok, u, ur, _ = inputs
    x = synth.normal((m, H), seed=seed + 200 + m)
    dx, dy = be.to_device(x), be.alloc(m * H * 4)
    dids, dw = be.alloc(m * 8 * 2), be.alloc(m * 8 * 4)
    acc = {k: be.to_device(v) for k, v in dict(t=target, d=draft, dt=dtok, u=u, ur=ur).items()}
    d_acc, d_tok = be.alloc(4), be.alloc(4 * M)
    layer = model.layers[0]

    def call():
        be.moe_layer_device(layer, dx, m, dy, dids, dw)
        if with_accept:
            be.accept_device(acc["t"], acc["d"], acc["dt"], K, V, TEMPERATURE, False, acc["u"],
                             acc["ur"], d_acc, d_tok)

    for _ in range(3):
        call()
    be.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        call()
    be.synchronize()
    wall_us = (time.perf_counter() - t0) / iters * 1e6
    be.profile_enable(True)
    for _ in range(iters):
        call()
    per = {}
    for kind, nm in ((_lib.KERNEL_ROUTE, "route"), (_lib.KERNEL_GATE_UP, "gate_up"),
                     (_lib.KERNEL_DOWN, "down"), (_lib.KERNEL_Q4K_MATVEC, "q4k_matvec"),
                     (_lib.KERNEL_ACCEPT, "accept")):
        n, ms, _ = be.profile_read(kind)
        if n:
            per[nm] = ms / iters * 1e3
    be.profile_enable(False)
    ids = be.read(dids, np.uint16, (m, 8))
    union = len(mtp.routes_union(ids))
    layer_bytes = (union + 1) * mtp.expert_bytes_q4_0() + (E + 1) * H * 4 + 2 * m * H * 4
    accept_bytes = (2 * K + 1) * V * 4 if with_accept else 0
    kernel_us = sum(per.values())
    total = layer_bytes + accept_bytes
    out = dict(m=m, expert_union=union, kernel_us=per, total_kernel_us=kernel_us,
               wall_us_per_call=wall_us, layer_algorithmic_bytes=layer_bytes,
               accept_algorithmic_bytes=accept_bytes, gbs=total / (kernel_us * 1e-6) / 1e9,
               frac=total / (kernel_us * 1e-6) / 1e9 / HBM_PEAK_GBS)
    for b in [dx, dy, dids, dw, d_acc, d_tok] + list(acc.values()):
        be.free(b)
    return out


def mtp_loop_bench(be, layers: int, seed: int, recipe: str, steps: int = 40, warmup: int = 4):
    """The MTP decode loop (turboqwenfare_amd/mtp_loop.py) at full depth: the
    40-layer target stack, the draft head's MoE layer, a Q4_0 embedding and
    the Q6_K LM head over V = 151,936, stochastic at T = 0.7, k = 3.  Two
    draft sources: the synthetic draft head (unrelated weights: its drafts
    are rejected) and self-drafting (the target drafts for itself: drafts
    accepted).  Wall time per step from the host, Python call overhead
    included; the controller's policy as in MtpLoop."""
    from turboqwenfare_amd.mtp_loop import DeviceEngine, MtpLoop, MtpModel

    model = MtpModel(be, layers, V, seed=seed, recipe=recipe, log=log)
    out = {}
    try:
        for name, self_draft in (("draft_head", False), ("self_draft", True)):
            eng = DeviceEngine(be, model, k=K, temperature=TEMPERATURE, greedy=False, seed=seed,
                               self_draft=self_draft)
            loop = MtpLoop(eng, k=K, window=8)
            try:
                loop.run(1234, warmup)
                be.synchronize()
                t0 = time.perf_counter()
                recs = [loop.step() for _ in range(steps)]
                be.synchronize()
                dt = time.perf_counter() - t0
            finally:
                eng.free()
            spec = [r for r in recs if r.speculative]
            emitted = sum(len(r.emitted) for r in recs)
            out[name] = dict(steps=steps, ms_per_step=dt / steps * 1e3, tokens=emitted,
                             tokens_per_s=emitted / dt, speculative_steps=len(spec),
                             mean_accepted=(float(np.mean([r.accepted for r in spec])) if spec else None),
                             controller_enabled=loop.controller.enabled)
    finally:
        model.free()
    return out


def kernel_source_digest() -> str:
    """sha256 of the dominant kernel's sources: a committed traffic profile
    counts for this build only when it was taken on the same sources."""
    import hashlib

    hsh = hashlib.sha256()
    for f in ("tqf_stack.hip", "tqf_device.h", "tqf_internal.h"):
        hsh.update((ROOT / "turboqwenfare_amd" / "csrc" / f).read_bytes())
    return hsh.hexdigest()[:16]


def committed_traffic(recipe: str):
    """HBM bytes per stack launch from the committed rocprofv3 FETCH/WRITE
    profile, if it was taken on these kernel sources and this workload."""
    tfile = ROOT / "profiles" / "stack_verify_traffic.json"
    if not tfile.exists():
        return None, "no committed traffic profile"
    t = json.loads(tfile.read_text())
    if t.get("source_digest") != kernel_source_digest():
        return None, "committed traffic profile was taken on other kernel sources"
    if t.get("recipe") != recipe:
        return None, f"committed traffic profile is for recipe {t.get('recipe')}"
    return t.get("hbm_bytes_per_launch"), t.get("source", "")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--recipe", choices=("zero_mean", "uniform"), default="zero_mean",
                    help="nibble recipe of the headline model's experts (zero_mean: q - 8 "
                         "symmetric on [-7, 7]; uniform: the literal nibbles 0..15)")
    ap.add_argument("--greedy", action="store_true", help="greedy instead of stochastic acceptance")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--verify-only", action="store_true",
                    help="only the headline verify step (the command its rocprofv3 profiles are "
                         "taken with); prints the bench line without the other sections")
    ap.add_argument("--gemv-pool", type=int, default=2048,
                    help="distinct 512x2048 matrices in the config-1 GEMV bandwidth pool")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device copies of MIB MiB (torch) and exit: the "
                         "known-size kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--grouped-only", choices=("zipf", "dense8", "both"), default=None,
                    help="only run the config-5 grouped expert GEMM on one resident layer "
                         "(the command its rocprofv3 profiles are taken with) and exit")
    ap.add_argument("--grouped-iters", type=int, default=20)
    ap.add_argument("--layer-only", action="store_true",
                    help="only configs 2 and 3 (one MoE layer at M = 1, and at M = 4 plus the "
                         "acceptance) on a one-layer model, and exit")
    ap.add_argument("--lm-head-only", action="store_true",
                    help="only run the Q6_K LM head (the command its rocprofv3 profiles are "
                         "taken with) and exit")
    ap.add_argument("--q4k-verify-only", action="store_true",
                    help="only the verify step with Q4_K expert layers")
    ap.add_argument("--mtp-loop-only", action="store_true",
                    help="only the MTP decode loop at full depth (draft head and self-drafting)")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only run the Q4_0 config-1 GEMV pool (the command its rocprofv3 profile "
                         "is taken with) and exit")
    ap.add_argument("--sampler-only", action="store_true",
                    help="only the one-row draw: acceptance k = 0 against the reference-exact "
                         "Sampler::select, and exit")
    ap.add_argument("--q4k-only", action="store_true",
                    help="only run the Q4_K config-1 GEMV pools (the command their rocprofv3 "
                         "profiles are taken with) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch

        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"bench: copied {args.copy_calibration} MiB x 5 (read + write per copy)")
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); multi-GPU sharding is design-only.", file=sys.stderr)
        sys.exit(2)

    from turboqwenfare_amd import mtp
    from turboqwenfare_amd.backend import HipBackend

    be = HipBackend(0)
    if args.q4k_verify_only:
        r = q4k_verify_bench(be, args.layers, args.seed, verify_inputs(args.seed),
                             steps=min(args.steps, 100))
        log("bench: Q4_K verify step " + json.dumps(r))
        be.close()
        return
    if args.mtp_loop_only:
        log("bench: MTP loop " + json.dumps(mtp_loop_bench(be, args.layers, args.seed, args.recipe,
                                                           steps=min(args.steps, 40))))
        be.close()
        return
    if args.lm_head_only:
        log("bench: LM head " + json.dumps(lm_head_bench(be, args.seed)))
        be.close()
        return
    if args.sampler_only:
        log("bench: one-row draw " + json.dumps(sampler_bench(be, args.seed)))
        be.close()
        return
    if args.gemv_only:
        log("bench: config-1 GEMV pool " + json.dumps(gemv_pool_bench(be, args.gemv_pool, args.seed)))
        be.close()
        return
    if args.q4k_only:
        log("bench: Q4_K config-1 pools " + json.dumps(q4k_pool_bench(be, args.gemv_pool,
                                                                      args.seed)))
        be.close()
        return
    if args.grouped_only or args.layer_only:
        model = build_model(be, 1, args.seed, args.recipe)
        if args.layer_only:
            inputs = verify_inputs(args.seed)
            for name, m, acc in (("config2_layer_m1", 1, False), ("config3_layer_m4_accept", M, True)):
                log(f"bench: {name} " + json.dumps(layer_bench(be, model, inputs, m, acc, args.seed)))
        else:
            cases = ("zipf", "dense8") if args.grouped_only == "both" else (args.grouped_only,)
            grouped = grouped_gemm_bench(be, model.layers[0], args.seed, args.grouped_iters, cases)
            log("bench: config-5 grouped GEMM " + json.dumps(grouped))
        be.close()
        return

    name, cus = be.device_info()
    log(f"bench: device {name}, {cus} CUs")
    t0 = time.perf_counter()
    model = build_model(be, args.layers, args.seed, args.recipe)
    log(f"bench: {args.recipe} model resident in {time.perf_counter() - t0:.1f} s")
    inputs = verify_inputs(args.seed)
    head = verify_bench(be, model, inputs, args.steps, args.warmup, args.greedy)
    steps_per_s = head["steps_per_s"]
    log(f"bench: verify step {head['ms_per_step']:.3f} ms; mean expert union "
        f"{head['expert_union']['mean']:.2f}")
    log("bench: kernel profile " + json.dumps(head["kernels"]))

    extras = {}
    if not args.verify_only:
        inputs_layer = inputs
        extras["config2_layer_m1"] = layer_bench(be, model, inputs_layer, 1, False, args.seed)
        log("bench: config 2 " + json.dumps(extras["config2_layer_m1"]))
        extras["config3_layer_m4_accept"] = layer_bench(be, model, inputs_layer, M, True, args.seed)
        log("bench: config 3 " + json.dumps(extras["config3_layer_m4_accept"]))
        extras["stack_m1"] = stack_m1_bench(be, model, args.seed)
        log("bench: 40-layer stack at M=1 " + json.dumps(extras["stack_m1"]))
        other = "uniform" if args.recipe == "zero_mean" else "zero_mean"
        side = build_model(be, args.layers, args.seed, other)
        r = verify_bench(be, side, inputs, min(args.steps, 50), 3, args.greedy, distribution=False)
        side.free()
        extras[f"{other}_recipe"] = {k: r[k] for k in ("steps_per_s", "ms_per_step", "expert_union",
                                                       "stack_algorithmic_bytes")}
        extras[f"{other}_recipe"]["stack_us"] = r["kernels"].get("stack", {}).get("avg_us")
        log(f"bench: {other} recipe " + json.dumps(extras[f"{other}_recipe"]))

        gemv = gemv_pool_bench(be, args.gemv_pool, args.seed)
        extras["gemv_config1"] = gemv
        log("bench: config-1 GEMV pool " + json.dumps(gemv))
        extras["q4k_config1"] = q4k_pool_bench(be, args.gemv_pool, args.seed)
        log("bench: Q4_K config-1 pools " + json.dumps(extras["q4k_config1"]))
        extras["lm_head_q6k"] = lm_head_bench(be, args.seed)
        log("bench: LM head " + json.dumps(extras["lm_head_q6k"]))
        extras["sampler_select"] = sampler_bench(be, args.seed)
        log("bench: one-row draw " + json.dumps(extras["sampler_select"]))
        extras["grouped_gemm_config5"] = grouped_gemm_bench(be, model.layers[0], args.seed)
        log("bench: config-5 grouped GEMM " + json.dumps(extras["grouped_gemm_config5"]))
        extras["q4k_verify"] = q4k_verify_bench(be, args.layers, args.seed, inputs,
                                                steps=min(args.steps, 100))
        log("bench: Q4_K verify step " + json.dumps(extras["q4k_verify"]))

    cpu = None
    if not args.no_cpu_baseline and not args.verify_only:
        res, threads, n_sample = cpu_baseline(model, inputs, args.cpu_budget)
        cpu = dict(value=res[threads], unit="verify steps/s", cores=threads, kind="port",
                   host_cpu=host_cpu_model(), host_nproc=os.cpu_count(),
                   sample=f"{n_sample} of {args.layers} MoE layers at M=4 plus one acceptance at "
                          f"V={V}, scaled to {args.layers} layers; oracle/tqf_oracle.c -O3 "
                          f"-ffp-contract=off, OpenMP over output rows",
                   single_thread_value=res[1])

    traffic, traffic_src = committed_traffic(args.recipe)
    prof = head["kernels"]
    dom = prof.get("stack") or prof.get("gate_up")
    acc_word = "greedy" if args.greedy else "stochastic"
    line = {
        "metric": "MTP k=3 verify steps/sec + Q4 expert GEMV HBM GB/s (% of peak), 1 GPU",
        "value": steps_per_s,
        "unit": "verify steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights; activations as block fixed point (each value a 22-bit integer "
                 "times its 32-element block's power-of-two scale, i.e. rounded to 2^-23 of the "
                 "block maximum), exact int4 digit dots into int32, fp32 accumulate",
        "data": f"synthetic (seeded Philox Q4_0 experts, nibble recipe {args.recipe}, N(0,1) "
                f"activations, N(0,9) logits)",
        "config": {"workload": f"config 4: full-depth MTP verify step, 40 MoE layers at M=4 (k=3) "
                               f"+ {acc_word} acceptance",
                   "expert_recipe": args.recipe,
                   "layers": args.layers, "hidden": H, "experts": E, "top_k": 8,
                   "expert_width": F, "vocab": V, "temperature": TEMPERATURE,
                   "resident_weight_gb": round(args.layers * (E + 1) * 3 * 589824 / 1e9, 2)},
        "effective_tokens_per_s": {str(a): steps_per_s * mtp.expected_tokens_per_step(a, K)
                                   for a in (0.6, 0.8)},
        "roofline": {"bound": "hbm", "achieved": dom["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dom["gbs"] / HBM_PEAK_GBS, "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": "stack_kernel (persistent 40-layer MoE stack: router, union-expert "
                               "gate/up + SwiGLU, down + combine)",
                     "avg_us": dom["avg_us"], "algorithmic_bytes_per_launch": dom["bytes_per_launch"],
                     "source_digest": kernel_source_digest()},
        "expert_union": head["expert_union"],
        "kernels": prof,
        "eager_profiled_ms_per_step": head["eager_profiled_ms_per_step"],
        "synchronised_step_ms": head.get("synchronised_step_ms"),
        **extras,
        "cpu_baseline": cpu,
    }
    if cpu:
        line["speedup_vs_cpu"] = steps_per_s / cpu["value"]
    print(json.dumps(line), flush=True)
    model.free()
    be.close()


if __name__ == "__main__":
    main()
