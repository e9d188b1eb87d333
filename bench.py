#!/usr/bin/env python3
"""Headline benchmark: MXFP4 GEMV HBM GB/s on one MI355X.

Workload (one "step"): the M = 1 decode projections of one Qwen3-8B token --
36 layers x {q 4096->4096, k 4096->1024, v 4096->1024, o 4096->4096,
gate 4096->12288, up 4096->12288, down 12288->4096} plus lm_head 4096->151936,
253 GEMVs over 4,029,425,152 algorithmic bytes. Every projection has its own
resident weight (4.03 GB in HBM, far beyond the 256 MB Infinity Cache), made on
the GPU by the weight recipe (bf16 N(0, 0.02), MXFP4 by the reference rule;
tensor j uses seed 1000 + j). Activations are bf16 N(0, 1) from seed 1, already
in HBM; outputs are f32. Projections that read the same activations in the
model share a launch, as a decode step allows: q|k|v and gate|up, so a layer
is 4 launches (qkv, o, gate|up, down) and the step 145. A step is replayed as
one recorded pass (HIP graph) unless --eager is given; --separate launches all
253 GEMVs one by one.

Algorithmic bytes of one GEMV: N*K/2 (nibbles) + N*K/32 (scales) + M*K*2 (bf16
x) + M*N*4 (f32 y). value = bytes per step / wall time per step.

extra.dropin_per_call times the per-call drop-in (qwen_hip_matmul: host f32 x
and y, synchronous) on layer 0 and the lm_head: the PCIe-inclusive rate.

cpu_baseline: the CPU oracle (a restatement of engine/src/lib.rs:240-266) on
the box's host, one thread, over a bounded sample with the step's shape mix:
all 7 projections of the first 9 layers plus the matching 9/36 of lm_head's
rows. extra.cpu_all_cores runs the same sample on every host thread (the
oracle parallelises over output elements; each element keeps its order).

extra also carries the other M = 1 workloads: the Qwen3-1.7B decode step (28
layers x {q 2048->2048, k/v 2048->1024, o 2048->2048, gate/up 2048->6144,
down 6144->2048} + lm_head 2048->151936, tensor j from seed 2000 + j, grouped
and recorded like the 8B step) with its per-shape figures, and the single
6144 x 2048 GEMV of the weight from seed 0 and x from seed 1.
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
sys.path.insert(0, str(ROOT / "jalapenos-at-home_amd"))

import mx4hip  # noqa: E402

LAYER = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
         ("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
LM_HEAD = ("lm_head", 151936, 4096)
LAYERS = 36
HBM_PEAK_GBS = 8000.0
LAYER_1P7B = [("q", 2048, 2048), ("k", 1024, 2048), ("v", 1024, 2048), ("o", 2048, 2048),
              ("gate", 6144, 2048), ("up", 6144, 2048), ("down", 2048, 6144)]
LM_HEAD_1P7B = ("lm_head", 151936, 2048)
LAYERS_1P7B = 28


def gemv_bytes(m: int, n: int, k: int, x_bytes: int = 2) -> int:
    return n * k // 2 + n * k // 32 + m * k * x_bytes + m * n * 4


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def build_step(ctx: mx4hip.Context, layer=LAYER, lm_head=LM_HEAD, layers=LAYERS, seed0=1000):
    """Distinct resident weights for every projection of the step."""
    weights = []
    seed = seed0
    for _ in range(layers):
        for name, n, k in layer:
            weights.append((name, n, k, ctx.synth_weight(seed, n, k, 0.02)))
            seed += 1
    name, n, k = lm_head
    weights.append((name, n, k, ctx.synth_weight(seed, n, k, 0.02)))
    ctx.synchronize()
    return weights


def enqueue_grouped_step(ctx, weights, xs, yq, layer=LAYER, layers=LAYERS):
    """One decode step as the model issues it: per layer q|k|v (one grouped
    launch on the shared x), o, gate|up (grouped), down; then lm_head."""
    hidden = layer[0][2]
    inter = layer[-1][2]
    per = len(layer)
    for li in range(layers):
        lw = {name: w for (name, _, _, w) in weights[li * per:(li + 1) * per]}
        ctx.matmul_group(xs[hidden].ptr, mx4hip.BF16, 1, [lw["q"], lw["k"], lw["v"]],
                         [yq["q"].ptr, yq["k"].ptr, yq["v"].ptr])
        ctx.matmul_ptr(xs[hidden].ptr, mx4hip.BF16, 1, lw["o"], yq["o"].ptr)
        ctx.matmul_group(xs[hidden].ptr, mx4hip.BF16, 1, [lw["gate"], lw["up"]], [yq["gate"].ptr, yq["up"].ptr])
        ctx.matmul_ptr(xs[inter].ptr, mx4hip.BF16, 1, lw["down"], yq["down"].ptr)
    _, n, k, w = weights[-1]
    ctx.matmul_ptr(xs[k].ptr, mx4hip.BF16, 1, w, yq["lm_head"].ptr)


MIN_COPIES = 4


def copies_by_name(ctx, weights, seed0: int = 9000):
    """The weights grouped by projection name, each with at least MIN_COPIES
    distinct copies: a shape with a single weight (lm_head) gets extra copies
    from the same recipe, so that its per-launch time is taken over several
    cold launches in one recorded pass, as for the per-layer shapes. Returns
    the groups and the extra weights (to release afterwards)."""
    by, extra = {}, []
    for (nm, n, k, w) in weights:
        by.setdefault(nm, []).append((n, k, w))
    for nm, lst in by.items():
        n, k, _ = lst[0]
        while len(lst) < MIN_COPIES:
            w = ctx.synth_weight(seed0 + len(extra), n, k, 0.02)
            extra.append(w)
            lst.append((n, k, w))
    ctx.synchronize()
    return by, extra


def release(ctx, extra) -> None:
    ctx.synchronize()
    for w in extra:
        w.release()


def time_shapes(ctx, weights, xs, ys, reps: int = 3, layer=LAYER):
    """Per-launch GPU time of each projection shape and of the grouped launches:
    the distinct copies of each (one per layer; lm_head in four copies) back to
    back, cold, in a recorded pass, timed with events on the context stream."""
    by, extra = copies_by_name(ctx, weights)
    plans = [(name, [name]) for name, _, _ in layer] + [("qkv", ["q", "k", "v"]), ("gate_up", ["gate", "up"]),
                                                         ("lm_head", ["lm_head"])]
    table = {}
    for label, members in plans:
        copies = len(by[members[0]])
        k = by[members[0]][0][1]
        ybufs = [ys[by[m][0][0]] for m in members]
        if len(members) > 1:
            yext = [ctx.buffer(by[m][0][0] * 4) for m in members]
            ybufs = yext

        def enqueue():
            for c in range(copies):
                ws = [by[m][c][2] for m in members]
                if len(ws) == 1:
                    ctx.matmul_ptr(xs[k].ptr, mx4hip.BF16, 1, ws[0], ybufs[0].ptr)
                else:
                    ctx.matmul_group(xs[k].ptr, mx4hip.BF16, 1, ws, [y.ptr for y in ybufs])

        p = ctx.record(enqueue)
        p.launch()
        best = None
        for _ in range(reps):
            ctx.synchronize()
            ctx.timer_begin()
            p.launch()
            ms = ctx.timer_end() / copies
            best = ms if best is None else min(best, ms)
        p.release()
        b = sum(gemv_bytes(1, by[m][0][0], k) for m in members)
        n = sum(by[m][0][0] for m in members)
        table[label] = {"k": k, "n": n, "bytes": b, "us": round(best * 1e3, 3),
                        "GBps": round(b / (best * 1e-3) / 1e9, 1),
                        "frac": round(b / (best * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    release(ctx, extra)
    return table


def time_skinny(ctx, weights, ms=(1, 2, 4, 8, 16, 32), reps: int = 3):
    """Speculative-verify shapes: each 8B projection at M token rows (exact path:
    GEMV for M = 1, skinny bf16-MFMA kernel above), 36 cold copies (lm_head: 4)
    in a recorded pass, per-call latency and effective GB/s (bytes with
    M*K*2 + M*N*4)."""
    by, extra = copies_by_name(ctx, weights)
    out = {}
    for name, n, k in LAYER + [LM_HEAD]:
        ws = [w for (_, _, w) in by[name]]
        row = {}
        for m in ms:
            xb = ctx.buffer(m * k * 2)
            ctx.synth_bf16(2, 1.0, m * k, xb)
            yb = ctx.buffer(m * n * 4)

            def enqueue():
                for w in ws:
                    ctx.matmul_ptr(xb.ptr, mx4hip.BF16, m, w, yb.ptr)

            p = ctx.record(enqueue)
            p.launch()
            best = None
            for _ in range(reps):
                ctx.synchronize()
                ctx.timer_begin()
                p.launch()
                t = ctx.timer_end() / len(ws)
                best = t if best is None else min(best, t)
            p.release()
            b = gemv_bytes(m, n, k)
            row[f"M{m}"] = {"us": round(best * 1e3, 3), "GBps": round(b / (best * 1e-3) / 1e9, 1)}
        out[name] = row
    release(ctx, extra)
    return out


def time_lm_head_argmax(ctx, weights, xs, reps: int = 5):
    """Greedy pick after the lm_head (engine/src/model.rs:228-238, :288-296) at
    M = 1: the projection followed by a separate argmax over the 151936 logits,
    against the fused epilogue with and without writing the logits. 8 calls
    per recorded pass; per-call GPU time."""
    _, n, k, w = weights[-1]
    y = ctx.buffer(n * 4)
    idx = ctx.buffer(4)
    x = xs[k]
    forms = (("projection", lambda: ctx.matmul_ptr(x.ptr, mx4hip.BF16, 1, w, y.ptr)),
             ("projection+argmax_rows", lambda: (ctx.matmul_ptr(x.ptr, mx4hip.BF16, 1, w, y.ptr),
                                                 ctx.argmax_rows(y, 1, n, idx))),
             ("fused, logits written", lambda: ctx.matmul_argmax(x, mx4hip.BF16, w, y, idx)),
             ("fused, no logits", lambda: ctx.matmul_argmax(x, mx4hip.BF16, w, None, idx)))
    out = {}
    for label, fn in forms:
        p = ctx.record(lambda: [fn() for _ in range(8)])
        p.launch()
        best = None
        for _ in range(reps):
            ctx.synchronize()
            ctx.timer_begin()
            p.launch()
            t = ctx.timer_end() / 8
            best = t if best is None else min(best, t)
        p.release()
        out[label] = round(best * 1e3, 2)
    return {"n": n, "k": k, "us": out}


def time_prefill(ctx, weights, m: int = 512, reps: int = 5):
    """Prefill on block-scaled MFMA: each 8B q/o/gate/up/down shape at M = 512,
    activations bf16 N(0, 1) requantized per 32 along K (MXFP4, and MX-FP8).
    Reports the GEMM kernel alone (activations requantized beforehand, as when
    q|k|v or gate|up share them) and requant + GEMM, as TFLOP/s of 2*M*N*K."""
    by = {}
    for (nm, n, k, w) in weights:
        by.setdefault(nm, (n, k, w))
    peaks = {"mxfp4": 10.1e15, "mxfp8": 5.0e15}
    ctx.reserve_prefill(m, max(k for (_, k, _) in by.values()))
    out = {}
    for name in ("q", "o", "gate", "up", "down"):
        n, k, w = by[name]
        xb = ctx.buffer(m * k * 2)
        ctx.synth_bf16(3, 1.0, m * k, xb)
        yb = ctx.buffer(m * n * 4)
        row = {}
        w.prepare_prefill()  # the matrix-core copy of the weight is built outside the timed passes
        for act, code in (("mxfp4", mx4hip.ACT_MXFP4), ("mxfp8", mx4hip.ACT_MXFP8)):
            xq, xs = ctx.prefill_act_buffers(m, k, code)
            ctx.prefill_quantize(xb, mx4hip.BF16, m, k, code, xq, xs)
            flops = 2.0 * m * n * k
            res = {}
            for label, fn in (("gemm", lambda: ctx.prefill_matmul(xq, xs, code, m, w, yb)),
                              ("requant+gemm", lambda: ctx.matmul_prefill(xb, mx4hip.BF16, m, w, code, yb))):
                p = ctx.record(lambda: [fn() for _ in range(8)])
                p.launch()
                best = None
                for _ in range(reps):
                    ctx.synchronize()
                    ctx.timer_begin()
                    p.launch()
                    t = ctx.timer_end() / 8
                    best = t if best is None else min(best, t)
                p.release()
                tf = flops / (best * 1e-3)
                res[label] = {"us": round(best * 1e3, 2), "TFLOPs": round(tf / 1e12, 1),
                              "frac": round(tf / peaks[act], 4)}
            row[act] = res
        out[name] = {"m": m, "n": n, "k": k, **row}
    return out


def time_dropin(ctx, weights, x_host: dict, reps: int = 5) -> dict:
    """The per-call drop-in (qwen_hip_matmul, the qwen_metal_matmul contract):
    host f32 x in, host f32 y out, synchronous, weights cached by host address
    after the first call. Layer 0's seven projections and the lm_head, called
    from Python through ctypes; the PCIe-inclusive rate, never `value`."""
    sample = weights[:len(LAYER)] + [weights[-1]]
    host = [(n, k, *ctx.download_weight(w)) for (_, n, k, w) in sample]
    hip = mx4hip.Hip()
    for n, k, packed, scales in host:  # uploads and caches the weights
        hip.matmul(x_host[k], packed, scales)
    best = None
    for _ in range(reps):
        t0 = time.perf_counter()
        for n, k, packed, scales in host:
            hip.matmul(x_host[k], packed, scales)
        t = time.perf_counter() - t0
        best = t if best is None else min(best, t)
    hip.close()
    b = sum(gemv_bytes(1, n, k, 4) for (n, k, _, _) in host)
    return {"calls": len(host), "us_per_call": round(best / len(host) * 1e6, 2),
            "GBps": round(b / best / 1e9, 1), "bytes": b,
            "sample": "layer 0 (q, k, v, o, gate, up, down) + lm_head, f32 x, host buffers, one call each"}


def time_model_1p7b(ctx, steps: int, warmup: int, reps: int = 3) -> dict:
    """The Qwen3-1.7B decode step at M = 1 (28 layers, 0.92 GB of distinct
    resident weights), grouped and recorded like the 8B step, plus its
    per-shape figures. The weights are released afterwards."""
    weights = build_step(ctx, LAYER_1P7B, LM_HEAD_1P7B, LAYERS_1P7B, seed0=2000)
    xs = {}
    for k in sorted({k for (_, _, k, _) in weights}):
        xs[k] = ctx.buffer(k * 2)
        ctx.synth_bf16(1, 1.0, k, xs[k])
    ys = {n: ctx.buffer(n * 4) for n in sorted({n for (_, n, _, _) in weights})}
    yq = {name: ctx.buffer(n * 4) for name, n, _ in LAYER_1P7B + [LM_HEAD_1P7B]}
    step_bytes = sum(gemv_bytes(1, n, k) for (_, n, k, _) in weights)
    p = ctx.record(lambda: enqueue_grouped_step(ctx, weights, xs, yq, LAYER_1P7B, LAYERS_1P7B))
    for _ in range(warmup):
        p.launch()
    ctx.synchronize()
    best = None
    for _ in range(reps):
        ctx.synchronize()
        ctx.timer_begin()
        for _ in range(steps):
            p.launch()
        ms = ctx.timer_end() / steps
        best = ms if best is None else min(best, ms)
    p.release()
    gbps = step_bytes / (best * 1e-3) / 1e9
    out = {"workload": "qwen3-1.7b decode step, M=1: 28 layers x 7 projections + lm_head (197 GEMVs, "
                       f"{LAYERS_1P7B * 4 + 1} launches)",
           "bytes_per_step": step_bytes, "ms_per_step": round(best, 4), "GBps": round(gbps, 1),
           "frac": round(gbps / HBM_PEAK_GBS, 4),
           "shapes": time_shapes(ctx, weights, xs, ys, layer=LAYER_1P7B)}
    ctx.synchronize()
    for (_, _, _, w) in weights:
        w.release()
    return out


def time_config1(ctx, reps: int = 5) -> dict:
    """The single GEMV of the CPU reference case: W 6144 x 2048 from seed 0,
    x bf16 [1, 2048] from seed 1, y f32 [1, 6144]; 8 calls per recorded pass
    on the same (warm) weight."""
    n, k = 6144, 2048
    w = ctx.synth_weight(0, n, k, 0.02)
    x = ctx.buffer(k * 2)
    ctx.synth_bf16(1, 1.0, k, x)
    y = ctx.buffer(n * 4)
    p = ctx.record(lambda: [ctx.matmul_ptr(x.ptr, mx4hip.BF16, 1, w, y.ptr) for _ in range(8)])
    p.launch()
    best = None
    for _ in range(reps):
        ctx.synchronize()
        ctx.timer_begin()
        p.launch()
        t = ctx.timer_end() / 8
        best = t if best is None else min(best, t)
    p.release()
    ctx.synchronize()
    w.release()
    b = gemv_bytes(1, n, k)
    return {"n": n, "k": k, "bytes": b, "us": round(best * 1e3, 3), "GBps": round(b / (best * 1e-3) / 1e9, 1)}


def time_prefill_layer(ctx, weights, m: int = 512, reps: int = 5) -> dict:
    """All seven projections of one 8B layer at M = 512 as a model issues them:
    q|k|v as one grouped launch on one requantization, o, gate|up grouped, and
    down (4 requantizations + 4 GEMMs), against the seven projections launched
    one by one (7 + 7). Layer 0's weights; 8 layers per recorded pass."""
    lw = {name: w for (name, _, _, w) in weights[:len(LAYER)]}
    for w in lw.values():
        w.prepare_prefill()
    dims = {name: (n, k) for name, n, k in LAYER}
    ctx.reserve_prefill(m, max(k for (_, k) in dims.values()))
    xb = {k: ctx.buffer(m * k * 2) for k in {k for (_, k) in dims.values()}}
    for k, b in xb.items():
        ctx.synth_bf16(3, 1.0, m * k, b)
    ys = {name: ctx.buffer(m * n * 4) for name, (n, _) in dims.items()}
    flops = sum(2.0 * m * n * k for (n, k) in dims.values())
    peaks = {"mxfp4": 10.1e15, "mxfp8": 5.0e15}
    out = {"m": m, "flops": flops}
    for act, code in (("mxfp4", mx4hip.ACT_MXFP4), ("mxfp8", mx4hip.ACT_MXFP8)):
        def grouped():
            ctx.matmul_prefill_group(xb[4096], mx4hip.BF16, m, [lw["q"], lw["k"], lw["v"]], code,
                                     [ys["q"], ys["k"], ys["v"]])
            ctx.matmul_prefill(xb[4096], mx4hip.BF16, m, lw["o"], code, ys["o"])
            ctx.matmul_prefill_group(xb[4096], mx4hip.BF16, m, [lw["gate"], lw["up"]], code, [ys["gate"], ys["up"]])
            ctx.matmul_prefill(xb[12288], mx4hip.BF16, m, lw["down"], code, ys["down"])

        def separate():
            for name, (_, k) in dims.items():
                ctx.matmul_prefill(xb[k], mx4hip.BF16, m, lw[name], code, ys[name])

        res = {}
        for label, fn in (("grouped", grouped), ("separate", separate)):
            p = ctx.record(lambda: [fn() for _ in range(8)])
            p.launch()
            best = None
            for _ in range(reps):
                ctx.synchronize()
                ctx.timer_begin()
                p.launch()
                t = ctx.timer_end() / 8
                best = t if best is None else min(best, t)
            p.release()
            tf = flops / (best * 1e-3)
            res[label] = {"us": round(best * 1e3, 2), "TFLOPs": round(tf / 1e12, 1), "frac": round(tf / peaks[act], 4)}
        out[act] = res
    return out


def cpu_baseline(ctx, weights, x_host: dict, layers: int = 9, threads: int = 1) -> dict:
    """The oracle on the host: `threads` threads, `layers` layers + the matching share of lm_head."""
    from oracle import mx4_oracle as oracle

    if not oracle.LIB_PATH.exists():
        oracle.build()
    jobs = []
    for name, n, k, w in weights[: layers * len(LAYER)]:
        jobs.append((n, k, w, n))
    name, n, k, w = weights[-1]
    jobs.append((n, k, w, -(-n * layers // LAYERS)))
    total_bytes, total_s = 0, 0.0
    for n, k, w, rows in jobs:
        packed, scales = ctx.download_weight(w)
        x = x_host[k]
        t0 = time.perf_counter()
        oracle.matmul_rows(x, packed.reshape(-1), scales.reshape(-1), 0, rows, threads=threads)
        total_s += time.perf_counter() - t0
        total_bytes += gemv_bytes(1, rows, k)
    how = "single-threaded" if threads == 1 else f"{threads}-thread"
    return {"value": round(total_bytes / total_s / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"first {layers} of 36 layers (all 7 projections) + {layers}/36 of lm_head rows, "
                      f"{total_bytes} B in {total_s:.1f} s, {how} C restatement of "
                      "engine/src/lib.rs:240-266"}


def host_threads() -> int:
    """Threads this process may use: the scheduler's CPU set, capped by OMP_NUM_THREADS when set."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(env))) if env.isdigit() else n


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--eager", action="store_true", help="enqueue each step from the host instead of replaying a recorded pass")
    ap.add_argument("--separate", action="store_true", help="one launch per projection (253) instead of q|k|v and gate|up groups")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-shapes", action="store_true")
    ap.add_argument("--no-skinny", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-1p7b", action="store_true", help="skip the Qwen3-1.7B step and the single config-1 GEMV")
    ap.add_argument("--profile-traffic", action="store_true",
                    help="for counter runs: 2 eager grouped steps, then a 1 GiB device copy as the byte calibration")
    ap.add_argument("--profile-prefill", action="store_true",
                    help="for profiler runs: only the M=512 prefill (q, o, gate, up, down; MXFP4 and MX-FP8 "
                         "activations): 5 GEMMs on requantized activations, then 5 requantize + GEMM calls")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (the GEMV would shard "
              "column-wise with an all-gather of y; see the design notes). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    if mx4hip.device_count() < 1:
        print("no gfx950 device visible", file=sys.stderr)
        return 1

    ctx = mx4hip.Context(0)
    log("synthesizing 253 resident MXFP4 weights (4.03 GB) on the GPU")
    weights = build_step(ctx)

    ks = sorted({k for (_, _, k, _) in weights})
    x_host = {}
    xs = {}
    for k in ks:
        xs[k] = ctx.buffer(k * 2)
        ctx.synth_bf16(1, 1.0, k, xs[k])
        bits = xs[k].download(np.uint16)
        x_host[k] = (bits.astype(np.uint32) << 16).view(np.float32).reshape(1, k)
    ys = {n: ctx.buffer(n * 4) for n in sorted({n for (_, n, _, _) in weights})}

    ops = ctx.make_ops([(xs[k].ptr, mx4hip.BF16, 1, w, ys[n].ptr) for (_, n, k, w) in weights])
    step_bytes = sum(gemv_bytes(1, n, k) for (_, n, k, _) in weights)
    # per layer: q|k|v share x, gate|up share x (distinct y buffers for each)
    yq = {name: ctx.buffer(n * 4) for name, n, _ in LAYER + [LM_HEAD]}

    def enqueue_grouped():
        enqueue_grouped_step(ctx, weights, xs, yq)

    if args.separate:
        enqueue = lambda: ctx.matmul_batch(ops)  # noqa: E731
        launches = len(weights)
    else:
        enqueue = enqueue_grouped
        launches = LAYERS * 4 + 1
    if args.profile_prefill:
        m = 512
        by = {}
        for (nm, n, k, w) in weights:
            by.setdefault(nm, (n, k, w))
        for name in ("q", "o", "gate", "up", "down"):
            n, k, w = by[name]
            w.prepare_prefill()
            xb = ctx.buffer(m * k * 2)
            ctx.synth_bf16(3, 1.0, m * k, xb)
            yb = ctx.buffer(m * n * 4)
            for code in (mx4hip.ACT_MXFP4, mx4hip.ACT_MXFP8):
                xq, xsc = ctx.prefill_act_buffers(m, k, code)
                ctx.prefill_quantize(xb, mx4hip.BF16, m, k, code, xq, xsc)
                for _ in range(5):
                    ctx.prefill_matmul(xq, xsc, code, m, w, yb)
                for _ in range(5):
                    ctx.matmul_prefill(xb, mx4hip.BF16, m, w, code, yb)
            ctx.synchronize()
        print(json.dumps({"profile_prefill": True, "m": m, "gemm_launches_per_shape_and_format": 10,
                          "requant_launches_per_shape_and_format": 6}), flush=True)
        ctx.close()
        return 0

    if args.profile_traffic:
        for _ in range(2):
            enqueue()
        ctx.synchronize()
        src, dst = ctx.buffer(1 << 30), ctx.buffer(1 << 30)
        mx4hip.check(mx4hip.lib().mx4_copy(ctx.handle, dst.ptr, src.ptr, 1 << 30))
        ctx.synchronize()
        print(json.dumps({"profile_traffic": True, "steps": 2, "launches_per_step": launches,
                          "bytes_per_step": step_bytes, "calibration_copy_bytes": 1 << 30}), flush=True)
        ctx.close()
        return 0

    if args.eager:
        step = enqueue
        launch = f"eager, {launches} launches per step"
    else:
        pss = ctx.record(enqueue)
        step = pss.launch
        launch = f"recorded pass (HIP graph), {launches} launches per step"

    for _ in range(args.warmup):
        step()
    ctx.synchronize()
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    ctx.timer_begin()
    for _ in range(args.steps):
        step()
    gpu_ms = ctx.timer_end()
    ctx.synchronize()
    wall_s = time.perf_counter() - t0
    ms_per_step = wall_s / args.steps * 1e3
    gpu_ms_per_step = gpu_ms / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = step_bytes / (gpu_ms_per_step * 1e-3) / 1e9

    extra = {"gpu_ms_per_step": round(gpu_ms_per_step, 4), "launch": launch}
    if not args.no_shapes:
        log("per-shape timing")
        extra["shapes"] = time_shapes(ctx, weights, xs, ys)

        log("lm_head + greedy argmax timing")
        extra["lm_head_argmax"] = time_lm_head_argmax(ctx, weights, xs)

    if not args.no_skinny:
        log("skinny (speculative verify) timing")
        extra["skinny"] = time_skinny(ctx, weights)

    if not args.no_prefill:
        log("prefill (M=512, block-scaled MFMA) timing")
        extra["prefill"] = time_prefill(ctx, weights)
        extra["prefill_layer"] = time_prefill_layer(ctx, weights)

    if not args.no_1p7b:
        log("qwen3-1.7b decode step and the config-1 GEMV")
        extra["qwen3_1p7b"] = time_model_1p7b(ctx, max(5, args.steps // 2), max(1, args.warmup))
        extra["single_gemv_6144x2048"] = time_config1(ctx)
        log("per-call drop-in (host buffers)")
        extra["dropin_per_call"] = time_dropin(ctx, weights, x_host)

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle, 1 thread)")
        cpu = cpu_baseline(ctx, weights, x_host)
        nt = host_threads()
        if nt > 1:
            log(f"cpu baseline (oracle, {nt} threads)")
            extra["cpu_all_cores"] = cpu_baseline(ctx, weights, x_host, threads=nt)

    # HBM bytes per step from the committed FETCH_SIZE + WRITE_SIZE counter runs
    traffic = None
    tf = ROOT / "profiles" / "gemv_qwen3_8b_m1_step_traffic.md"
    if tf.exists() and not args.separate:
        for line in tf.read_text().splitlines():
            if line.startswith("hbm_bytes_per_step:"):
                traffic = int(line.split(":")[1])

    out = {
        "metric": "MXFP4 GEMV HBM GB/s + % peak, Qwen3-8B M=1; M=512 prefill TFLOP/s",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4 x bf16 -> f32",
        "data": "synthetic: weights bf16 N(0,0.02) quantized by the reference MXFP4 rule, x bf16 N(0,1)",
        "config": {"workload": "qwen3-8b decode step, M=1: 36 layers x 7 projections + lm_head (253 GEMVs)",
                   "bytes_per_step": step_bytes, "x_dtype": "bf16", "y_dtype": "f32",
                   "distinct_weights_bytes": sum(w.nbytes for (_, _, _, w) in weights),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "M=1 GEMV (gemv_m1_head_kernel, gemv_m1_one_kernel: all launches of the step)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "basis": "algorithmic bytes of one decode step / GPU event time of one step"},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
