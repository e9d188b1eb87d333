#!/usr/bin/env python3
"""Headline benchmark: MXFP4 GEMV HBM GB/s on one MI355X.

Workload (one "step"): the M = 1 decode projections of one Qwen3-8B token --
36 layers x {q 4096->4096, k 4096->1024, v 4096->1024, o 4096->4096,
gate 4096->12288, up 4096->12288, down 12288->4096} plus lm_head 4096->151936,
253 GEMVs over 4,029,425,152 algorithmic bytes. Every projection has its own
resident weight (4.03 GB in HBM, far beyond the 256 MB Infinity Cache), made on
the GPU by the weight recipe (bf16 N(0, 0.02), MXFP4 by the reference rule;
tensor j uses seed 1000 + j) in one device allocation, each weight on its own
2 MiB-aligned slice. Activations are bf16 N(0, 1) from seed 1, already in HBM;
outputs are f32. Projections that read the same activations in the model share
a launch, as a decode step allows: q|k|v and gate|up, so a layer is 4 launches
(qkv, o, gate|up, down) and the step 145. A step is replayed as one recorded
pass (HIP graph) unless --eager is given; --separate launches all 253 GEMVs
one by one.

Algorithmic bytes of one GEMV: N*K/2 (nibbles) + N*K/32 (scales) + M*K*2 (bf16
x) + M*N*4 (f32 y). value = bytes per step / wall time per step.

Timing protocol of every figure in `extra` (engine/src/model.rs:259-264,
engine/src/main.rs:70): a recorded pass of distinct weight copies totalling at
least 512 MiB per shape (cold: twice the Infinity Cache), 2 untimed launches,
then the median of 15 timed launches; per-call time = pass time / calls.

extra also carries the other workloads: the Qwen3-1.7B decode step (28 layers,
tensor j from seed 2000 + j) with its per-shape figures, the single 6144 x 2048
GEMV that the reference runs on its CPU path (weight seed 0, x seed 1; cold over copies, and warm on one
weight, labelled), speculative verify (8B shapes at M = 1..32), prefill at
M = 512 (block-scaled MFMA; exact bf16-MFMA AUTO path) with the matrix-core
ceiling it is read against (scaled FP4 MFMAs back to back, random and constant
codes, and the shader clock held under that load), the per-call drop-in
(PCIe-inclusive), and the CPU legs below.

cpu_baseline: the CPU oracle (a restatement of engine/src/lib.rs:240-266) on
the box's host, one thread, over a bounded sample with the step's shape mix:
all 7 projections of the first 9 layers plus the matching 9/36 of lm_head's
rows. extra.cpu holds the same sample on every host thread, the verify and
prefill shapes (row subsets, extrapolated to the full shapes, as stated in each entry), and
the host CPU model and core counts.

Profile modes (for rocprofv3; see profiles/): --profile-step, --profile-traffic,
--profile-prefill run only the work their summaries cover and print a stamp
(library sha256); --summarize KIND DIR [DIR] turns rocprofv3 CSV output into
the committed summaries. roofline.traffic is taken from
profiles/gemv_qwen3_8b_m1_step_traffic.md only when its stamp matches the
library this run loaded, and is null otherwise.
"""
from __future__ import annotations

import argparse
import csv
import ctypes
import hashlib
import json
import os
import subprocess
import sys
import time
from collections import defaultdict
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
PEAK_TFLOPS = {"mxfp4": 10100.0, "mxfp8": 5000.0, "bf16": 2500.0}
LAYER_1P7B = [("q", 2048, 2048), ("k", 1024, 2048), ("v", 1024, 2048), ("o", 2048, 2048),
              ("gate", 6144, 2048), ("up", 6144, 2048), ("down", 2048, 6144)]
LM_HEAD_1P7B = ("lm_head", 151936, 2048)
LAYERS_1P7B = 28
ROTATION_BYTES = 512 << 20   # distinct weight bytes per timed shape (2 x the Infinity Cache)
REPS, WARM = 15, 2           # timed launches (median) and untimed ones before them
VERIFY_REPS = 4              # enqueues of each verify block under --profile-verify
MIN_COPIES = 8               # launches per timed pass at least (weights rotated)
ARENA_ALIGN = 2 << 20
TRAFFIC_PROFILE = ROOT / "profiles" / "gemv_qwen3_8b_m1_step_traffic.md"
PREFILL_PROFILE = ROOT / "profiles" / "prefill_qwen3_8b_m512.md"


def gemv_bytes(m: int, n: int, k: int, x_bytes: int = 2) -> int:
    return n * k // 2 + n * k // 32 + m * k * x_bytes + m * n * 4


def weight_bytes(n: int, k: int) -> int:
    return n * k // 2 + n * k // 32


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def library_sha256() -> str:
    return hashlib.sha256(mx4hip.LIB_PATH.read_bytes()).hexdigest()


# ---------------------------------------------------------------- weights

class Arena:
    """Synthesized MXFP4 weights in one device allocation, each on its own
    2 MiB-aligned slice (packed bytes, then its scales), wrapped as resident
    weights. specs: (rows, cols, seed)."""

    def __init__(self, ctx: mx4hip.Context, specs):
        L = mx4hip.lib()
        self.ctx = ctx
        offs, total = [], 0
        for (n, k, _) in specs:
            total = (total + ARENA_ALIGN - 1) // ARENA_ALIGN * ARENA_ALIGN
            po = total
            so = (po + n * k // 2 + 255) // 256 * 256
            offs.append((po, so))
            total = so + n * k // 32
        base = ctypes.c_void_p()
        mx4hip.check(L.mx4_malloc(ctx.handle, max(total, 1), ctypes.byref(base)))
        self.base = base.value
        self.nbytes = total
        self.weights = []
        for (n, k, seed), (po, so) in zip(specs, offs):
            p, s = ctypes.c_void_p(self.base + po), ctypes.c_void_p(self.base + so)
            mx4hip.check(L.mx4_synth_weight(ctx.handle, seed, ctypes.c_double(0.02), n, k, p, s))
            h = ctypes.c_void_p()
            mx4hip.check(L.mx4_weight_wrap(ctx.handle, p, s, n, k, ctypes.byref(h)))
            self.weights.append(ctx._track(mx4hip.Weight(ctx, h.value, n, k)))
        ctx.synchronize()

    def release(self) -> None:
        self.ctx.synchronize()
        for w in self.weights:
            w.release()
        self.weights = []
        if self.base:
            mx4hip.check(mx4hip.lib().mx4_free(self.ctx.handle, ctypes.c_void_p(self.base)))
            self.base = None


def build_step(ctx, layer=LAYER, lm_head=LM_HEAD, layers=LAYERS, seed0=1000):
    """Distinct resident weights for every projection of the step, one arena."""
    specs, names = [], []
    seed = seed0
    for _ in range(layers):
        for name, n, k in layer:
            specs.append((n, k, seed))
            names.append(name)
            seed += 1
    name, n, k = lm_head
    specs.append((n, k, seed))
    names.append(name)
    arena = Arena(ctx, specs)
    weights = [(nm, n, k, w) for nm, (n, k, _), w in zip(names, specs, arena.weights)]
    return weights, arena


def enqueue_grouped_step(ctx, weights, xs, yq, layer=LAYER, layers=LAYERS, m: int = 1):
    """One decode step as the model issues it: per layer q|k|v (one grouped
    launch on the shared x), o, gate|up (grouped), down; then lm_head. With
    m > 1, a speculative verify step over m token rows (xs and yq sized for
    them)."""
    hidden = layer[0][2]
    inter = layer[-1][2]
    per = len(layer)
    for li in range(layers):
        lw = {name: w for (name, _, _, w) in weights[li * per:(li + 1) * per]}
        ctx.matmul_group(xs[hidden].ptr, mx4hip.BF16, m, [lw["q"], lw["k"], lw["v"]],
                         [yq["q"].ptr, yq["k"].ptr, yq["v"].ptr])
        ctx.matmul_ptr(xs[hidden].ptr, mx4hip.BF16, m, lw["o"], yq["o"].ptr)
        ctx.matmul_group(xs[hidden].ptr, mx4hip.BF16, m, [lw["gate"], lw["up"]], [yq["gate"].ptr, yq["up"].ptr])
        ctx.matmul_ptr(xs[inter].ptr, mx4hip.BF16, m, lw["down"], yq["down"].ptr)
    _, n, k, w = weights[-1]
    ctx.matmul_ptr(xs[k].ptr, mx4hip.BF16, m, w, yq["lm_head"].ptr)


def time_verify_step(ctx, weights, ms=(2, 4, 8, 16), steps: int = 10) -> dict:
    """The whole 8B step at m token rows (a speculative verify step: 36 layers
    of q|k|v and gate|up grouped, o, down, then the lm_head) recorded as one
    pass over the decode step's resident weights; at 8 tokens also with one
    launch per projection. GPU ms per step and GB/s over the weight bytes plus
    activations and outputs."""
    out = {}
    for m in ms:
        xs = {}
        for k in sorted({k for (_, _, k, _) in weights}):
            xs[k] = ctx.buffer(m * k * 2)
            ctx.synth_bf16(3, 1.0, m * k, xs[k])
        yq = {name: ctx.buffer(m * n * 4) for name, n, _ in LAYER + [LM_HEAD]}
        nbytes = sum(gemv_bytes(m, n, k) for (_, n, k, _) in weights)
        p = ctx.record(lambda: enqueue_grouped_step(ctx, weights, xs, yq, m=m))
        ms_g = time_step(ctx, p, steps)
        p.release()
        row = {"gpu_ms_per_step": round(ms_g, 4), "GBps": round(nbytes / (ms_g * 1e-3) / 1e9, 1)}
        if m == 8:
            ys = {n: ctx.buffer(m * n * 4) for n in sorted({n for (_, n, _, _) in weights})}
            ops = ctx.make_ops([(xs[k].ptr, mx4hip.BF16, m, w, ys[n].ptr) for (_, n, k, w) in weights])
            p = ctx.record(lambda: ctx.matmul_batch(ops))
            row["one_launch_per_projection_ms"] = round(time_step(ctx, p, steps), 4)
            p.release()
            for y in ys.values():
                y.free()
        out[f"M{m}"] = row
        for b in list(xs.values()) + list(yq.values()):
            b.free()
    return out


def rotation(ctx, members, seed0: int, min_bytes: int = ROTATION_BYTES) -> tuple[Arena, list]:
    """Copies of a shape (one member) or of a group of shapes read together
    (q|k|v, gate|up): as many distinct copies as make up min_bytes of
    weights. members: [(rows, cols)]. Returns the arena and the copies, each a
    list of weights (one per member)."""
    per = sum(weight_bytes(n, k) for n, k in members)
    # at least MIN_COPIES launches per pass: the pass's own start-up (tens of
    # microseconds for a pass of one launch) is then a small share of each call
    copies = max(MIN_COPIES, -(-min_bytes // per))
    specs = [(n, k, seed0 + c * len(members) + i) for c in range(copies) for i, (n, k) in enumerate(members)]
    arena = Arena(ctx, specs)
    ws = arena.weights
    return arena, [ws[c * len(members):(c + 1) * len(members)] for c in range(copies)]


# ---------------------------------------------------------------- timing

def time_pass(ctx, enqueue, calls: int, reps: int = REPS, warm: int = WARM) -> dict:
    """Record `enqueue` as a pass, launch it `warm` times untimed, then `reps`
    timed launches; per-call median and minimum in microseconds."""
    p = ctx.record(enqueue)
    for _ in range(warm):
        p.launch()
    ctx.synchronize()
    ts = []
    for _ in range(reps):
        ctx.timer_begin()
        p.launch()
        ts.append(ctx.timer_end() / calls * 1e3)
    p.release()
    return {"us": round(float(np.median(ts)), 3), "us_min": round(float(np.min(ts)), 3)}


def hbm_entry(t: dict, nbytes: int, extra: dict | None = None) -> dict:
    gbps = nbytes / (t["us"] * 1e-6) / 1e9
    out = dict(extra or {})
    out.update({"bytes": nbytes, "us": t["us"], "us_min": t["us_min"], "GBps": round(gbps, 1),
                "frac": round(gbps / HBM_PEAK_GBS, 4)})
    return out


def time_shapes(ctx, xs, layer=LAYER, lm_head=LM_HEAD, seed0=20000) -> dict:
    """Per-launch time of each projection shape and of the grouped launches
    (q|k|v, gate|up), each over >= 512 MiB of distinct cold copies."""
    dims = {name: (n, k) for name, n, k in layer + [lm_head]}
    plans = [(name, [name]) for name, _, _ in layer] + [("qkv", ["q", "k", "v"]), ("gate_up", ["gate", "up"]),
                                                        (lm_head[0], [lm_head[0]])]
    table = {}
    for i, (label, members) in enumerate(plans):
        mdims = [dims[m] for m in members]
        k = mdims[0][1]
        arena, copies = rotation(ctx, mdims, seed0 + 1000 * i)
        ys = [ctx.buffer(n * 4) for n, _ in mdims]

        def enqueue():
            for ws in copies:
                if len(ws) == 1:
                    ctx.matmul_ptr(xs[k].ptr, mx4hip.BF16, 1, ws[0], ys[0].ptr)
                else:
                    ctx.matmul_group(xs[k].ptr, mx4hip.BF16, 1, ws, [y.ptr for y in ys])

        t = time_pass(ctx, enqueue, len(copies))
        b = sum(gemv_bytes(1, n, k) for n, _ in mdims)
        table[label] = hbm_entry(t, b, {"k": k, "n": sum(n for n, _ in mdims), "copies": len(copies)})
        arena.release()
    return table


def time_lm_head_argmax(ctx, xs) -> dict:
    """Greedy pick after the lm_head (engine/src/model.rs:228-238, :288-296) at
    M = 1 over two cold copies (662 MB): the projection alone, followed by a
    separate argmax over the 151936 logits, and the fused epilogue with and
    without writing the logits."""
    _, n, k = LM_HEAD
    arena, copies = rotation(ctx, [(n, k)], 30000)
    y = ctx.buffer(n * 4)
    idx = ctx.buffer(4)
    x = xs[k]
    forms = (("projection", lambda w: ctx.matmul_ptr(x.ptr, mx4hip.BF16, 1, w, y.ptr)),
             ("projection+argmax_rows", lambda w: (ctx.matmul_ptr(x.ptr, mx4hip.BF16, 1, w, y.ptr),
                                                   ctx.argmax_rows(y, 1, n, idx))),
             ("fused, logits written", lambda w: ctx.matmul_argmax(x, mx4hip.BF16, w, y, idx)),
             ("fused, no logits", lambda w: ctx.matmul_argmax(x, mx4hip.BF16, w, None, idx)))
    out = {}
    for label, fn in forms:
        out[label] = time_pass(ctx, lambda: [fn(ws[0]) for ws in copies], len(copies))["us"]
    arena.release()
    return {"n": n, "k": k, "copies": len(copies), "us": out}


def time_skinny(ctx, ms=(1, 2, 4, 8, 16, 32)) -> dict:
    """Speculative-verify shapes: each 8B projection at M token rows
    through AUTO (GEMV at M = 1, few-token GEMV or skinny bf16-MFMA kernel
    above), over >= 512 MiB of cold copies per shape; per-call latency and
    effective GB/s (bytes with M*K*2 + M*N*4)."""
    out = {}
    for i, (name, n, k) in enumerate(LAYER + [LM_HEAD]):
        arena, copies = rotation(ctx, [(n, k)], 40000 + 1000 * i)
        row = {}
        for m in ms:
            xb = ctx.buffer(m * k * 2)
            ctx.synth_bf16(2, 1.0, m * k, xb)
            yb = ctx.buffer(m * n * 4)
            t = time_pass(ctx, lambda: [ctx.matmul_ptr(xb.ptr, mx4hip.BF16, m, ws[0], yb.ptr) for ws in copies],
                          len(copies))
            b = gemv_bytes(m, n, k)
            row[f"M{m}"] = {"us": t["us"], "GBps": round(b / (t["us"] * 1e-6) / 1e9, 1)}
        out[name] = row
        arena.release()
    return out


def time_skinny_groups(ctx, ms=(2, 4, 8, 16, 32), separate: dict | None = None) -> dict:
    """The verify step's grouped launches: q|k|v and gate|up at M token rows
    through mx4_matmul_group (one launch of the few-token GEMV or the skinny
    kernel over every weight's rows), over >= 512 MiB of cold copies; per-call
    latency, effective GB/s, and the sum of the members' separate calls from
    time_skinny (`separate`) when given."""
    dims = {name: (n, k) for name, n, k in LAYER}
    out = {}
    for gi, (label, members) in enumerate((("qkv", ["q", "k", "v"]), ("gate_up", ["gate", "up"]))):
        shapes = [dims[nm] for nm in members]
        k = shapes[0][1]
        arena, copies = rotation(ctx, shapes, 45000 + 1000 * gi)
        row = {}
        for m in ms:
            xb = ctx.buffer(m * k * 2)
            ctx.synth_bf16(2, 1.0, m * k, xb)
            ys = [ctx.buffer(m * n * 4) for n, _ in shapes]
            t = time_pass(ctx, lambda: [ctx.matmul_group(xb.ptr, mx4hip.BF16, m, ws, [y.ptr for y in ys])
                                        for ws in copies], len(copies))
            b = sum(gemv_bytes(m, n, k) for n, _ in shapes) - (len(shapes) - 1) * m * k * 2  # x read once
            e = {"us": t["us"], "GBps": round(b / (t["us"] * 1e-6) / 1e9, 1)}
            if separate and all(f"M{m}" in separate.get(nm, {}) for nm in members):
                e["separate_us"] = round(sum(separate[nm][f"M{m}"]["us"] for nm in members), 3)
            row[f"M{m}"] = e
            for y in ys:
                y.free()
            xb.free()
        out[label] = row
        arena.release()
    return out


def time_mfma_ceiling(ctx) -> dict:
    """What the matrix cores sustain on the prefill GEMM's instruction:
    scaled FP4 MFMAs back to back on every SIMD (mx4_mfma_ceiling), on random
    and on constant E2M1 codes, with the shader clock the waves held. The
    published 10.1 PFLOP/s assumes 2.4 GHz; under this load the part lowers
    its clock, further with random codes, so the random-code 32x32x64 rate
    (the prefill kernels' instruction and operand statistics) is the
    clock-derived ceiling the MXFP4 prefill figures are also read against;
    likewise the FP8 x FP4 instruction for the MX-FP8 prefill and the bf16
    32x32x16 for the exact GEMM."""
    out = {}
    for shape, label, peak in ((0, "32x32x64", "mxfp4"), (1, "16x16x128", "mxfp4"), (2, "fp8xfp4_32x32x64", "mxfp8"),
                               (3, "bf16_32x32x16", "bf16")):
        row = {}
        for codes, rnd in (("random", True), ("constant", False)):
            runs = [ctx.mfma_ceiling(shape, rnd) for _ in range(3)]
            pf = float(np.median([r[0] for r in runs]))
            ghz = float(np.median([r[1] for r in runs]))
            row[codes] = {"TFLOPs": round(pf * 1000, 1), "clock_GHz": round(ghz, 3),
                          "frac_of_published": round(pf * 1000 / PEAK_TFLOPS[peak], 4)}
        out[label] = row
    out["method"] = ("two waves per SIMD, one workgroup of eight per CU, independent accumulators, about 0.3 ms per "
                     "run after a warm-up; median of 3 runs; clock = shader clock counter over the constant-rate "
                     "counter, median over waves")
    return out


def _err(y: np.ndarray, r: np.ndarray) -> dict:
    """max_i |y - r| / max_i |r| and ||y - r||_2 / ||r||_2
    (python/src/jalapenos_reference/compare.py:19-22, engine/tests/mxfp4.rs:76-84)."""
    y, r = y.astype(np.float64), r.astype(np.float64)
    d = y - r
    return {"max_rel": float(f"{np.max(np.abs(d)) / max(np.max(np.abs(r)), 1e-300):.3e}"),
            "rel_l2": float(f"{np.sqrt(np.sum(d * d)) / max(np.sqrt(np.sum(r * r)), 1e-300):.3e}")}


def prefill_error(ctx, w, xb, x_host: np.ndarray, m: int, rng) -> dict:
    """What requantizing the activations costs (information, not a parity
    gate): the M = 512 outputs of requant + block-scaled MFMA (MXFP4 and
    MX-FP8 activations) and of the exact AUTO path (bf16 MFMA, no
    requantization) on sampled token rows x weight rows, against the oracle on
    the unquantized bf16 x (engine/src/lib.rs:240-266); and, for the
    requantized paths, against the oracle on dequant(requant(x)), the parity
    bar of the tests."""
    oracle = _oracle()
    n, k = w.rows, w.cols
    packed, scales = ctx.download_weight(w)
    rows = np.unique(np.concatenate([[0, m - 1], rng.choice(m, 14, replace=False)]))
    cols = np.unique(np.concatenate([[0, n - 1], rng.choice(n, 62, replace=False)]))

    def ref(xs):
        return np.concatenate([oracle.matmul_rows(xs, packed.reshape(-1), scales.reshape(-1), int(c), int(c) + 1)
                               for c in cols], axis=1)

    exact = ref(x_host[rows])
    yb = ctx.buffer(m * n * 4)
    out = {}
    for act, code in (("mxfp4", mx4hip.ACT_MXFP4), ("mxfp8", mx4hip.ACT_MXFP8)):
        ctx.matmul_prefill(xb, mx4hip.BF16, m, w, code, yb)
        y = yb.download(np.float32).reshape(m, n)[np.ix_(rows, cols)]
        xd = oracle.dequantize(*oracle.quantize(x_host[rows])) if act == "mxfp4" else \
            oracle.dequantize_fp8(*oracle.quantize_fp8(x_host[rows]))
        e = _err(y, exact)
        e["vs_requantized_oracle"] = _err(y, ref(xd))
        out[act] = e
    ctx.matmul_ptr(xb.ptr, mx4hip.BF16, m, w, yb.ptr)
    out["exact_auto"] = _err(yb.download(np.float32).reshape(m, n)[np.ix_(rows, cols)], exact)
    out["sample"] = f"{len(rows)} token rows x {len(cols)} weight rows"
    return out


def time_prefill(ctx, m: int = 512, ceiling: dict | None = None) -> dict:
    """Prefill at M = 512 on block-scaled MFMA: each 8B q/o/gate/up/down shape
    at M = 512, activations bf16 N(0, 1) requantized per 32 along K (MXFP4 and
    MX-FP8), over >= 512 MiB of cold weight copies. The GEMM kernel alone
    (activations requantized beforehand, as when q|k|v or gate|up share them)
    and requant + GEMM, as TFLOP/s of 2*M*N*K; also as a fraction of the
    measured matrix-core ceiling of each activation format (`ceiling`,
    TFLOP/s by format) when given."""
    out = {}
    dims = {name: (n, k) for name, n, k in LAYER}
    ctx.reserve_prefill(m, 12288)
    rng = np.random.default_rng(512)
    for i, name in enumerate(("q", "o", "gate", "up", "down")):
        n, k = dims[name]
        arena, copies = rotation(ctx, [(n, k)], 50000 + 1000 * i)
        for ws in copies:
            ws[0].prepare_prefill()  # the matrix-core copy of each weight, outside the timed passes
        xb = ctx.buffer(m * k * 2)
        ctx.synth_bf16(3, 1.0, m * k, xb)
        x_host = (xb.download(np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(m, k)
        yb = ctx.buffer(m * n * 4)
        flops = 2.0 * m * n * k
        row = {"m": m, "n": n, "k": k, "copies": len(copies)}
        for act, code in (("mxfp4", mx4hip.ACT_MXFP4), ("mxfp8", mx4hip.ACT_MXFP8)):
            xq, xsc = ctx.prefill_act_buffers(m, k, code)
            ctx.prefill_quantize(xb, mx4hip.BF16, m, k, code, xq, xsc)
            res = {}
            for label, fn in (("gemm", lambda w: ctx.prefill_matmul(xq, xsc, code, m, w, yb)),
                              ("requant+gemm", lambda w: ctx.matmul_prefill(xb, mx4hip.BF16, m, w, code, yb))):
                t = time_pass(ctx, lambda: [fn(ws[0]) for ws in copies], len(copies))
                tf = flops / (t["us"] * 1e-6) / 1e12
                res[label] = {"us": t["us"], "TFLOPs": round(tf, 1), "frac": round(tf / PEAK_TFLOPS[act], 4)}
                if ceiling and act in ceiling:
                    res[label]["frac_of_measured_ceiling"] = round(tf / ceiling[act], 4)
            row[act] = res
        row["requant_error"] = prefill_error(ctx, copies[0][0], xb, x_host, m, rng)
        out[name] = row
        arena.release()
    return out


def time_prefill_rows(ctx, ms=(128, 1024)) -> dict:
    """Prefill away from M = 512 (where the default instance is the tile whose
    workgroups come nearest one round of the CUs): the 8B q, gate and down
    shapes at `ms` token rows, MXFP4 and MX-FP8 activations requantized
    beforehand, the GEMM alone through the default instance, over >= 512 MiB
    of cold weight copies. [us, TFLOP/s] per shape, format and M."""
    out = {}
    dims = {name: (n, k) for name, n, k in LAYER}
    ctx.reserve_prefill(max(ms), 12288)
    for i, name in enumerate(("q", "gate", "down")):
        n, k = dims[name]
        arena, copies = rotation(ctx, [(n, k)], 57000 + 1000 * i)
        for ws in copies:
            ws[0].prepare_prefill()
        row = {}
        for act, code in (("mxfp4", mx4hip.ACT_MXFP4), ("mxfp8", mx4hip.ACT_MXFP8)):
            res = {}
            for m in ms:
                xb = ctx.buffer(m * k * 2)
                ctx.synth_bf16(3, 1.0, m * k, xb)
                yb = ctx.buffer(m * n * 4)
                xq, xsc = ctx.prefill_act_buffers(m, k, code)
                ctx.prefill_quantize(xb, mx4hip.BF16, m, k, code, xq, xsc)
                t = time_pass(ctx, lambda: [ctx.prefill_matmul(xq, xsc, code, m, ws[0], yb) for ws in copies],
                              len(copies))
                res[f"M{m}"] = [t["us"], round(2.0 * m * n * k / (t["us"] * 1e-6) / 1e12, 1)]
                for b_ in (xb, yb, xq, xsc):
                    b_.free()
            row[act] = res
        out[name] = row
        arena.release()
    out["cols"] = ["us", "TFLOPs"]
    return out


def prefill_counters() -> dict:
    """MFMA operation and busy counters of the M = 512 prefill dispatches
    from the committed profile summary, when its stamp names the library this
    process loaded (otherwise only the reason)."""
    f = PREFILL_PROFILE
    if not f.exists():
        return {"note": "no prefill profile"}
    sha = library_sha256()
    text = f.read_text().splitlines()
    stamp = next((ln.split(":", 1)[1].strip() for ln in text if ln.startswith("library_sha256:")), "missing")
    if stamp != sha:
        return {"note": f"profile stamp {stamp[:12]} != loaded library {sha[:12]}"}
    out = {}
    for ln in text:
        cells = [c.strip() for c in ln.strip().strip("|").split("|")]
        if len(cells) != 9 or not cells[0]:
            continue
        key = f"{cells[0].split()[0]} {cells[1]}"
        if key not in ("gate mxfp4", "down mxfp4", "gate mxfp8"):
            continue
        out[key] = [cells[2].replace(" ", ""), float(cells[4]), float(cells[7].split("(")[1].split()[0]),
                    round(float(cells[8].rstrip("%")) / 100, 3)]
    out["cols"] = ["instance", "warm_us", "MOPSx512/2MNK", "busy@2.4GHz"]
    out["stamp"] = sha[:12]
    return out


def prefill_summary(pf: dict, layer: dict, ceiling: dict) -> dict:
    """The M = 512 half of the headline metric, compact: per 8B shape and
    activation format [GEMM us, TFLOP/s, of peak, of the measured ceiling,
    requant + GEMM us, TFLOP/s, of peak]; the grouped layer; the largest
    requantization error against the unquantized oracle; counters of the
    dominant instances from the stamped profile."""
    out = {"m": 512, "peak_TFLOPs": {"mxfp4": PEAK_TFLOPS["mxfp4"], "mxfp8": PEAK_TFLOPS["mxfp8"]},
           "measured_ceiling_TFLOPs": {a: round(ceiling[a], 1) for a in ("mxfp4", "mxfp8")},
           "cols": ["gemm_us", "gemm_TF", "gemm_of_peak", "gemm_of_ceiling", "rq_gemm_us", "rq_gemm_TF",
                    "rq_gemm_of_peak"], "rq": "requantization of the bf16 activations included"}
    for act in ("mxfp4", "mxfp8"):
        out[act] = {}
        for name, row in pf.items():
            g, r = row[act]["gemm"], row[act]["requant+gemm"]
            out[act][name] = [g["us"], round(g["TFLOPs"]), g["frac"], g.get("frac_of_measured_ceiling"),
                              r["us"], round(r["TFLOPs"]), r["frac"]]
    out["layer_grouped"] = {a: [layer[a]["grouped"]["us"], layer[a]["grouped"]["frac"]] for a in ("mxfp4", "mxfp8")}
    out["layer_cols"] = ["us, 7 projections with rq", "of_peak"]
    out["requant_error_vs_unquantized"] = {
        a: {"max_rel": max(row["requant_error"][a]["max_rel"] for row in pf.values()),
            "rel_l2": max(row["requant_error"][a]["rel_l2"] for row in pf.values())}
        for a in ("mxfp4", "mxfp8", "exact_auto")}
    out["counters"] = prefill_counters()
    return out


def time_prefill_layer(ctx, weights, m: int = 512) -> dict:
    """All seven projections of an 8B layer at M = 512 as a model issues them:
    q|k|v as one grouped launch on one requantization, o, gate|up grouped, and
    down (4 requantizations + 4 GEMMs), against the seven projections launched
    one by one (7 + 7). Eight distinct layers of the step per pass (0.82 GB of
    weights, cold)."""
    per = len(LAYER)
    layers = [{name: w for (name, _, _, w) in weights[li * per:(li + 1) * per]} for li in range(8)]
    for lw in layers:
        for w in lw.values():
            w.prepare_prefill()
    dims = {name: (n, k) for name, n, k in LAYER}
    ctx.reserve_prefill(m, 12288)
    xb = {k: ctx.buffer(m * k * 2) for k in {k for (_, k) in dims.values()}}
    for k, b in xb.items():
        ctx.synth_bf16(3, 1.0, m * k, b)
    ys = {name: ctx.buffer(m * n * 4) for name, (n, _) in dims.items()}
    flops = sum(2.0 * m * n * k for (n, k) in dims.values())
    out = {"m": m, "flops": flops, "layers_per_pass": len(layers)}
    for act, code in (("mxfp4", mx4hip.ACT_MXFP4), ("mxfp8", mx4hip.ACT_MXFP8)):
        def grouped():
            for lw in layers:
                ctx.matmul_prefill_group(xb[4096], mx4hip.BF16, m, [lw["q"], lw["k"], lw["v"]], code,
                                         [ys["q"], ys["k"], ys["v"]])
                ctx.matmul_prefill(xb[4096], mx4hip.BF16, m, lw["o"], code, ys["o"])
                ctx.matmul_prefill_group(xb[4096], mx4hip.BF16, m, [lw["gate"], lw["up"]], code,
                                         [ys["gate"], ys["up"]])
                ctx.matmul_prefill(xb[12288], mx4hip.BF16, m, lw["down"], code, ys["down"])

        def separate():
            for lw in layers:
                for name, (_, k) in dims.items():
                    ctx.matmul_prefill(xb[k], mx4hip.BF16, m, lw[name], code, ys[name])

        res = {}
        for label, fn in (("grouped", grouped), ("separate", separate)):
            t = time_pass(ctx, fn, len(layers))
            tf = flops / (t["us"] * 1e-6) / 1e12
            res[label] = {"us": t["us"], "TFLOPs": round(tf, 1), "frac": round(tf / PEAK_TFLOPS[act], 4)}
        out[act] = res
    return out


def time_prefill_exact(ctx, ms=(33, 128, 512), ceiling: float | None = None) -> dict:
    """The exact path a drop-in call takes for M > 32 (AUTO: bf16 x, no
    requantization, f32 accumulation of exact products) on the 8B q/gate/down
    shapes, over >= 512 MiB of cold copies; TFLOP/s against the dense bf16 MFMA
    peak (2.5 PFLOP/s) and, when given, the measured bf16 ceiling (TFLOP/s)."""
    out = {}
    dims = {name: (n, k) for name, n, k in LAYER}
    for i, name in enumerate(("q", "gate", "down")):
        n, k = dims[name]
        arena, copies = rotation(ctx, [(n, k)], 60000 + 1000 * i)
        row = {"n": n, "k": k, "copies": len(copies)}
        for m in ms:
            xb = ctx.buffer(m * k * 2)
            ctx.synth_bf16(4, 1.0, m * k, xb)
            yb = ctx.buffer(m * n * 4)
            t = time_pass(ctx, lambda: [ctx.matmul_ptr(xb.ptr, mx4hip.BF16, m, ws[0], yb.ptr) for ws in copies],
                          len(copies))
            tf = 2.0 * m * n * k / (t["us"] * 1e-6) / 1e12
            row[f"M{m}"] = {"us": t["us"], "TFLOPs": round(tf, 1), "frac_bf16": round(tf / PEAK_TFLOPS["bf16"], 4)}
            if ceiling:
                row[f"M{m}"]["frac_of_measured_ceiling"] = round(tf / ceiling, 4)
            yb.free()
            xb.free()
        # f32 activations, as a drop-in call passes them (each split into three
        # bf16 terms: three MFMAs per k-step)
        for m in (128, 512):
            xb = ctx.buffer(m * k * 4)
            xb.upload(np.random.default_rng(m).standard_normal(m * k).astype(np.float32))
            yb = ctx.buffer(m * n * 4)
            t = time_pass(ctx, lambda: [ctx.matmul_ptr(xb.ptr, mx4hip.F32, m, ws[0], yb.ptr) for ws in copies],
                          len(copies))
            tf = 2.0 * m * n * k / (t["us"] * 1e-6) / 1e12
            row[f"M{m}_f32"] = {"us": t["us"], "TFLOPs": round(tf, 1)}
            yb.free()
            xb.free()
        out[name] = row
        arena.release()
    # the grouped launches of an exact prefill (mx4_matmul_group: one exact
    # GEMM over q|k|v's or gate|up's column tiles), with the members' separate
    # calls in the same pass form for comparison
    for gi, (label, members) in enumerate((("qkv_group", ["q", "k", "v"]), ("gate_up_group", ["gate", "up"]))):
        shapes = [dims[nm] for nm in members]
        k = shapes[0][1]
        arena, copies = rotation(ctx, shapes, 63000 + 1000 * gi)
        row = {"n": sum(n for n, _ in shapes), "k": k, "copies": len(copies)}
        for m in ms:
            xb = ctx.buffer(m * k * 2)
            ctx.synth_bf16(4, 1.0, m * k, xb)
            ys = [ctx.buffer(m * n * 4) for n, _ in shapes]
            t = time_pass(ctx, lambda: [ctx.matmul_group(xb.ptr, mx4hip.BF16, m, ws, [y.ptr for y in ys])
                                        for ws in copies], len(copies))
            sep = time_pass(ctx, lambda: [ctx.matmul_ptr(xb.ptr, mx4hip.BF16, m, w, y.ptr)
                                          for ws in copies for w, y in zip(ws, ys)], len(copies))
            tf = 2.0 * m * row["n"] * k / (t["us"] * 1e-6) / 1e12
            row[f"M{m}"] = {"us": t["us"], "separate_us": sep["us"], "TFLOPs": round(tf, 1),
                            "frac_bf16": round(tf / PEAK_TFLOPS["bf16"], 4)}
            for y in ys:
                y.free()
            xb.free()
        out[label] = row
        arena.release()
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
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        for n, k, packed, scales in host:
            hip.matmul(x_host[k], packed, scales)
        ts.append(time.perf_counter() - t0)
    hip.close()
    t = float(np.median(ts))
    b = sum(gemv_bytes(1, n, k, 4) for (n, k, _, _) in host)
    return {"calls": len(host), "us_per_call": round(t / len(host) * 1e6, 2),
            "GBps": round(b / t / 1e9, 1), "bytes": b,
            "sample": "layer 0 (q, k, v, o, gate, up, down) + lm_head, f32 x, host buffers, one call each, "
                      f"median of {reps}"}


def time_bf16_weights(ctx, ms=(1, 4)) -> dict:
    """bf16 (non-quantized) weights, the scales == NULL arm of the drop-in
    (engine/src/lib.rs:255, metal.rs:45-50): 8B q, gate and down at M = 1 and
    4 (bf16 x), over >= 512 MiB of distinct device copies per shape (the same
    N(0, 0.02) bf16 values uploaded to each). Bytes: N*K*2 + M*K*2 + M*N*4."""
    out = {}
    rng = np.random.default_rng(5)
    for name, n, k in (LAYER[0], LAYER[4], LAYER[6]):
        vals = (rng.standard_normal(n * k, dtype=np.float32) * 0.02).view(np.uint32)
        bits = ((vals + 0x7FFF + ((vals >> 16) & 1)) >> 16).astype(np.uint16).reshape(n, k)
        copies = [ctx.upload_weight_bf16(bits, n, k) for _ in range(max(MIN_COPIES, -(-ROTATION_BYTES // (n * k * 2))))]
        row = {"n": n, "k": k, "copies": len(copies)}
        for m in ms:
            xb = ctx.buffer(m * k * 2)
            ctx.synth_bf16(2, 1.0, m * k, xb)
            yb = ctx.buffer(m * n * 4)
            t = time_pass(ctx, lambda: [ctx.matmul_ptr(xb.ptr, mx4hip.BF16, m, w, yb.ptr) for w in copies],
                          len(copies))
            b = n * k * 2 + m * k * 2 + m * n * 4
            row[f"M{m}"] = {"us": t["us"], "GBps": round(b / (t["us"] * 1e-6) / 1e9, 1),
                            "frac": round(b / (t["us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        for w in copies:
            w.release()
        out[name] = row
    return out


def time_embed_quantize(ctx, weights) -> dict:
    """The data formats either side of the projection. Embedding
    (engine/src/lib.rs:213-234): 512 and 1 token ids into the 8B table (the tied
    lm_head weight, 151936 x 4096), decoded to bf16 rows; bytes = the rows'
    packed + scale bytes read and their bf16 written. Quantization
    (python/quantize_mxfp4.py:18-39 on device, the checkpoint converter's rule):
    a bf16 12288 x 4096 matrix to packed + scales, synchronous calls on the
    host clock; bytes = input + output."""
    out = {}
    _, n, k, table = weights[-1]
    rng = np.random.default_rng(9)
    for count in (1, 512):
        ids = ctx.to_device(rng.integers(0, n, count, dtype=np.uint32))
        ob = ctx.buffer(count * k * 2)
        # ten calls per pass: a pass of one small launch times the pass's own launch
        t = time_pass(ctx, lambda: [ctx.embed(table, ids, count, ob) for _ in range(10)], 10)
        b = count * (k // 2 + k // 32) + count * k * 2
        out[f"embed_{count}_ids"] = {"us": t["us"], "GBps": round(b / (t["us"] * 1e-6) / 1e9, 1)}
    rows, cols = 12288, 4096
    xb = ctx.buffer(rows * cols * 2)
    ctx.synth_bf16(7, 0.02, rows * cols, xb)
    packed, scales = ctx.buffer(rows * cols // 2), ctx.buffer(rows * cols // 32)
    # mx4_quantize is synchronous (it reads back the non-finite flag and fails
    # on one), so it is timed per call on the host clock, the read-back included
    ts = []
    for i in range(WARM + REPS):
        t0 = time.perf_counter()
        ctx.quantize(xb, mx4hip.BF16, rows, cols, packed, scales)
        if i >= WARM:
            ts.append((time.perf_counter() - t0) * 1e6)
    us = float(np.median(ts))
    b = rows * cols * 2 + rows * cols // 2 + rows * cols // 32
    out["quantize_bf16_12288x4096"] = {"us_per_synchronous_call": round(us, 2),
                                       "GBps": round(b / (us * 1e-6) / 1e9, 1),
                                       "frac": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    return out


def time_step(ctx, p, steps: int, reps: int = REPS, warm: int = WARM) -> float:
    """Median GPU milliseconds per step over `reps` runs of `steps` replays."""
    for _ in range(warm):
        p.launch()
    ctx.synchronize()
    ts = []
    for _ in range(reps):
        ctx.timer_begin()
        for _ in range(steps):
            p.launch()
        ts.append(ctx.timer_end() / steps)
    return float(np.median(ts))


def time_model_1p7b(ctx, steps: int) -> dict:
    """The Qwen3-1.7B decode step at M = 1 (28 layers, 0.92 GB of distinct
    resident weights, cold), grouped and recorded like the 8B step, plus its
    per-shape figures over cold copies."""
    weights, arena = build_step(ctx, LAYER_1P7B, LM_HEAD_1P7B, LAYERS_1P7B, seed0=2000)
    xs = {}
    for k in sorted({k for (_, _, k, _) in weights}):
        xs[k] = ctx.buffer(k * 2)
        ctx.synth_bf16(1, 1.0, k, xs[k])
    yq = {name: ctx.buffer(n * 4) for name, n, _ in LAYER_1P7B + [LM_HEAD_1P7B]}
    step_bytes = sum(gemv_bytes(1, n, k) for (_, n, k, _) in weights)
    p = ctx.record(lambda: enqueue_grouped_step(ctx, weights, xs, yq, LAYER_1P7B, LAYERS_1P7B))
    ms = time_step(ctx, p, steps)
    p.release()
    ys = {n: ctx.buffer(n * 4) for n in sorted({n for (_, n, _, _) in weights})}
    ops = ctx.make_ops([(xs[k].ptr, mx4hip.BF16, 1, w, ys[n].ptr) for (_, n, k, w) in weights])
    p = ctx.record(lambda: ctx.matmul_batch(ops))
    ms_sep = time_step(ctx, p, steps)
    p.release()
    arena.release()
    gbps = step_bytes / (ms * 1e-3) / 1e9
    return {"workload": "qwen3-1.7b decode step, M=1: 28 layers x 7 projections + lm_head (197 GEMVs, "
                        f"{LAYERS_1P7B * 4 + 1} launches)",
            "bytes_per_step": step_bytes, "ms_per_step": round(ms, 4), "GBps": round(gbps, 1),
            "frac": round(gbps / HBM_PEAK_GBS, 4),
            "one_launch_per_projection": {"launches": len(weights), "ms_per_step": round(ms_sep, 4),
                                          "GBps": round(step_bytes / (ms_sep * 1e-3) / 1e9, 1)},
            "shapes": time_shapes(ctx, xs, LAYER_1P7B, LM_HEAD_1P7B, seed0=70000)}


def time_single_gemv(ctx) -> dict:
    """The single GEMV of the CPU reference case: W 6144 x 2048 (seed 0; the
    cold figure also uses copies of the same recipe), x bf16 [1, 2048] from
    seed 1, y f32 [1, 6144]. Cold: over >= 512 MiB of distinct copies. Warm:
    the seed-0 weight called repeatedly (served from the Infinity Cache after
    the first call; not an HBM figure)."""
    n, k = 6144, 2048
    x = ctx.buffer(k * 2)
    ctx.synth_bf16(1, 1.0, k, x)
    y = ctx.buffer(n * 4)
    arena, copies = rotation(ctx, [(n, k)], 80000)
    cold = time_pass(ctx, lambda: [ctx.matmul_ptr(x.ptr, mx4hip.BF16, 1, ws[0], y.ptr) for ws in copies],
                     len(copies))
    arena.release()
    w = ctx.synth_weight(0, n, k, 0.02)
    warm = time_pass(ctx, lambda: [ctx.matmul_ptr(x.ptr, mx4hip.BF16, 1, w, y.ptr) for _ in range(16)], 16)
    ctx.synchronize()
    w.release()
    b = gemv_bytes(1, n, k)
    return {"n": n, "k": k, "cold": hbm_entry(cold, b, {"copies": len(copies)}),
            "warm_infinity_cache": {"us": warm["us"], "GBps": round(b / (warm["us"] * 1e-6) / 1e9, 1)}}


# ---------------------------------------------------------------- CPU legs

def host_threads() -> int:
    """Threads this process may use: the scheduler's CPU set, capped by OMP_NUM_THREADS when set."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(env))) if env.isdigit() else n


def host_cpu() -> dict:
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"model": model, "box_logical_cpus": os.cpu_count(),
            "lease_cpus": len(os.sched_getaffinity(0)), "threads_used_all": host_threads()}


def _oracle():
    from oracle import mx4_oracle as oracle

    if not oracle.LIB_PATH.exists():
        oracle.build()
    return oracle


def cpu_baseline(ctx, weights, x_host: dict, layers: int = 9, threads: int = 1) -> dict:
    """The oracle on the host: `threads` threads, `layers` layers + the matching share of lm_head."""
    oracle = _oracle()
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


def _time_full(fn, reps: int = 3) -> float:
    """Median seconds of `reps` timed calls after one untimed one
    (engine/src/model.rs:259-264: warm-ups dropped, median kept)."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_full_shapes(ctx, thread_counts) -> dict:
    """Whole shapes on the host, no sampling: the single 6144 x 2048 GEMV of
    the CPU reference case (weight seed 0, x seed 1, y f32 [1, 6144]) and
    every Qwen3-1.7B projection at M = 1 (the 1.7B step's first-layer weights,
    seeds 2000..2006, and its lm_head, seed 2196; x bf16 N(0, 1) from seed 1),
    each timed in full, 1 thread and every thread of the lease; the 1.7B step
    is 28 x the layer's seven projections + lm_head. us per call and GB/s of
    algorithmic bytes (bf16 x as the GPU reads it; the oracle takes it as f32,
    as the reference's CPU path does)."""
    oracle = _oracle()
    jobs = [("config1_6144x2048", 6144, 2048, 0)]
    jobs += [(f"1p7b_{name}", n, k, 2000 + j) for j, (name, n, k) in enumerate(LAYER_1P7B)]
    jobs.append(("1p7b_lm_head", LM_HEAD_1P7B[1], LM_HEAD_1P7B[2], 2000 + LAYERS_1P7B * len(LAYER_1P7B)))
    xs = {k: oracle.bf16_to_f32(oracle.synth_bf16(1, 1.0, k)).reshape(1, k) for k in {k for _, _, k, _ in jobs}}
    out = {f"threads_{t}": {} for t in thread_counts}
    for label, n, k, seed in jobs:
        w = ctx.synth_weight(seed, n, k, 0.02)
        packed, scales = ctx.download_weight(w)
        w.release()
        p, sc = packed.reshape(-1), scales.reshape(-1)
        for t in thread_counts:
            sec = _time_full(lambda: oracle.matmul_rows(xs[k], p, sc, 0, n, threads=t))
            out[f"threads_{t}"][label] = [round(sec * 1e6, 1), round(gemv_bytes(1, n, k) / sec / 1e9, 3)]
    step_bytes = LAYERS_1P7B * sum(gemv_bytes(1, n, k) for _, n, k in LAYER_1P7B) + \
        gemv_bytes(1, LM_HEAD_1P7B[1], LM_HEAD_1P7B[2])
    for t in thread_counts:
        row = out[f"threads_{t}"]
        us = LAYERS_1P7B * sum(row[f"1p7b_{name}"][0] for name, _, _ in LAYER_1P7B) + row["1p7b_lm_head"][0]
        row["1p7b_step_28_layers"] = [round(us, 1), round(step_bytes / (us * 1e-6) / 1e9, 3)]
    out["cols"] = ["us per call (median of 3 after 1 untimed)", "GB/s"]
    return out


def _rows_for(work_macs: float, per_row_macs: int, n: int) -> int:
    return int(min(n, max(16, -(-int(work_macs) // per_row_macs))))


def cpu_verify(ctx, weights, threads: int) -> dict:
    """Speculative verify on the host: each 8B shape at M = 2, 4, 8, 16 (bf16 N(0, 1) rows,
    seed 2), the oracle over the first R weight rows (about 5e6 multiply-adds
    per thread), extrapolated to all N rows: us per call = t * N / R."""
    oracle = _oracle()
    first = {name: w for (name, _, _, w) in weights}
    out = {}
    for name, n, k in LAYER + [LM_HEAD]:
        packed, scales = ctx.download_weight(first[name])
        row = {}
        for m in (2, 4, 8, 16):
            x = oracle.bf16_to_f32(oracle.synth_bf16(2, 1.0, m * k)).reshape(m, k)
            r = _rows_for(5e6 * threads, m * k, n)
            t0 = time.perf_counter()
            oracle.matmul_rows(x, packed.reshape(-1), scales.reshape(-1), 0, r, threads=threads)
            t = time.perf_counter() - t0
            us = t * n / r * 1e6
            row[f"M{m}"] = [r, round(us, 1), round(gemv_bytes(m, n, k) / (us * 1e-6) / 1e9, 4)]
        out[name] = row
    return {"threads": threads, "shapes": out, "cols": ["rows R", "us_per_call", "GBps"],
            "method": "oracle over the first R of N weight rows (all M token rows), us_per_call = time * N / R"}


def cpu_prefill(ctx, weights, threads: int) -> dict:
    """Prefill at M = 512 on the host: each 8B q/o/gate/up/down shape at M = 512, the
    oracle (no requantization: engine/src/lib.rs:240-266 on the bf16 rows) over
    8 of the 512 token rows and the first R weight rows (about 5e6
    multiply-adds per thread), extrapolated: seconds per call = t * (512 / 8)
    * (N / R)."""
    oracle = _oracle()
    first = {name: w for (name, _, _, w) in weights}
    out = {}
    m, mt = 512, 8
    for name, n, k in LAYER:
        if name in ("k", "v"):
            continue
        packed, scales = ctx.download_weight(first[name])
        x = oracle.bf16_to_f32(oracle.synth_bf16(3, 1.0, mt * k)).reshape(mt, k)
        r = _rows_for(5e6 * threads, mt * k, n)
        t0 = time.perf_counter()
        oracle.matmul_rows(x, packed.reshape(-1), scales.reshape(-1), 0, r, threads=threads)
        t = time.perf_counter() - t0
        s = t * (m / mt) * (n / r)
        out[name] = {"rows": r, "token_rows": mt, "s_per_call": round(s, 3),
                     "GFLOPs": round(2.0 * m * n * k / s / 1e9, 3)}
    return {"threads": threads, "m": m, "shapes": out,
            "method": "oracle over 8 of 512 token rows and the first R of N weight rows, "
                      "s_per_call = time * 64 * N / R"}


# ---------------------------------------------------------------- profiles

def traffic_from_profile() -> tuple[int | None, str]:
    """HBM bytes per step from the committed counter summary, when its stamp
    names the library this process loaded."""
    if not TRAFFIC_PROFILE.exists():
        return None, "no traffic profile"
    fields = {}
    for line in TRAFFIC_PROFILE.read_text().splitlines():
        if ":" in line and not line.startswith(("|", " ", "#")):
            key, val = line.split(":", 1)
            fields[key.strip()] = val.strip()
    sha = library_sha256()
    if fields.get("library_sha256") != sha:
        return None, f"profile stamp {fields.get('library_sha256', 'missing')[:12]} != loaded library {sha[:12]}"
    return int(fields["hbm_bytes_per_step"]), f"profile stamp matches the loaded library ({sha[:12]})"


def write_stamp(path: str | None, info: dict) -> None:
    info = dict(info)
    info["library_sha256"] = library_sha256()
    print(json.dumps(info), flush=True)
    if path:
        Path(path).parent.mkdir(parents=True, exist_ok=True)
        Path(path).write_text(json.dumps(info) + "\n")


def _read_csv(d: Path, suffix: str) -> list[dict]:
    files = sorted(d.glob(f"*{suffix}"))
    if not files:
        raise SystemExit(f"no *{suffix} under {d}")
    with open(files[0], newline="") as f:
        return list(csv.DictReader(f))


def _short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "")
    return name.split("(")[0] if not name.startswith("void ") else name[5:].split("(")[0]


def _stamp_of(d: Path) -> dict:
    f = d / "stamp.json"
    return json.loads(f.read_text()) if f.exists() else {}


def _git_head() -> str:
    try:
        return subprocess.run(["git", "-C", str(ROOT), "rev-parse", "--short=12", "HEAD"], capture_output=True,
                              text=True, check=True).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        return "unknown"


def summarize(kind: str, dirs: list[str]) -> None:
    """Markdown summaries of rocprofv3 CSV output (run here, on the pulled-back
    files): `trace DIR` (kernel stats of --profile-step), `traffic FETCH_DIR
    WRITE_DIR` (FETCH_SIZE / WRITE_SIZE of --profile-traffic, calibrated by the
    1 GiB copy), `step-pmc DIR` (per-launch averages of any counters of
    --profile-traffic), `verify-trace DIR` (--profile-verify), `prefill-trace DIR`
    and `prefill-pmc DIR` (--profile-prefill), `prefill-shapes TRACE_DIR
    PMC_DIR` (--profile-prefill: each shape's GEMM dispatches, in the order the
    mode issues them, with their traced durations and MFMA counters),
    `prefill-compare DIR` (--profile-prefill-compare)."""
    d0 = Path(dirs[0])
    st = _stamp_of(d0)
    print(f"commit: {_git_head()}")
    print(f"library_sha256: {st.get('library_sha256', 'unknown')}")
    if kind == "trace":
        rows = _read_csv(d0, "kernel_stats.csv")
        steps = st.get("steps", 0) + st.get("warmup", 0)
        print(f"steps_traced: {steps}\n")
        print("| kernel | calls | calls per step | average us | min us | max us |")
        print("|---|---|---|---|---|---|")
        step_us = 0.0
        for r in rows:
            nm = _short(r["Name"])
            calls = int(r["Calls"])
            avg = float(r["AverageNs"]) / 1e3
            per = calls / steps if steps else 0
            if nm.startswith("mx4::gemv"):
                step_us += avg * per
            print(f"| {nm} | {calls} | {per:.0f} | {avg:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                  f"{float(r['MaxNs']) / 1e3:.2f} |")
        print(f"\nsum of GEMV kernel durations per step: {step_us:.1f} us")
    elif kind == "traffic":
        cal = st.get("calibration_copy_bytes", 1 << 30)
        steps = st.get("steps", 2)
        out = {}
        for d, counter in ((Path(dirs[0]), "FETCH_SIZE"), (Path(dirs[1]), "WRITE_SIZE")):
            rows = _read_csv(d, "counter_collection.csv")
            per = defaultdict(lambda: [0, 0.0])
            copy_kib = 0.0
            for r in rows:
                if r["Counter_Name"] != counter:
                    continue
                nm = _short(r["Kernel_Name"])
                v = float(r["Counter_Value"])
                if "copyBuffer" in nm or "copy" in nm.lower() and not nm.startswith("mx4::"):
                    copy_kib += v
                elif nm.startswith("mx4::gemv"):
                    per[nm][0] += 1
                    per[nm][1] += v
            factor = cal / (copy_kib * 1024) if counter == "FETCH_SIZE" else (cal / (copy_kib * 1024))
            out[counter] = (per, factor, copy_kib)
        fper, ff, fcopy = out["FETCH_SIZE"]
        wper, wf, wcopy = out["WRITE_SIZE"]
        print(f"calibration: {cal} B device copy read {fcopy:.1f} KiB FETCH_SIZE and wrote {wcopy:.1f} KiB "
              f"WRITE_SIZE -> factors {ff:.4f}, {wf:.4f}\n")
        print("| kernel | launches per step | HBM fetch MB per step | HBM write MB per step |")
        print("|---|---|---|---|")
        tf = tw = 0.0
        for nm in sorted(fper):
            n, fk = fper[nm]
            wk = wper.get(nm, [0, 0.0])[1]
            fb, wb = fk * 1024 * ff / steps, wk * 1024 * wf / steps
            tf += fb
            tw += wb
            print(f"| {nm} | {n / steps:.0f} | {fb / 1e6:.2f} | {wb / 1e6:.3f} |")
        alg = st.get("bytes_per_step", 0)
        print(f"\nper step: HBM fetch {tf:.6g} B, write {tw:.6g} B, total {tf + tw:.6g} B; algorithmic {alg} B; "
              f"ratio {(tf + tw) / alg if alg else 0:.4f}\n")
        print(f"hbm_bytes_per_step: {int(round(tf + tw))}")
    elif kind == "verify-trace":
        rows = _read_csv(d0, "kernel_trace.csv")
        rows.sort(key=lambda r: int(r["Start_Timestamp"]))
        blocks = []
        for r in rows:
            nm = _short(r["Kernel_Name"])
            if nm == "mx4::synth_bf16_kernel":
                blocks.append([])
            elif blocks and (nm.startswith("mx4::gemv") or nm.startswith("mx4::skinny")):
                blocks[-1].append(r)
        plan = st["plan"]
        if len(blocks) != len(plan):
            raise SystemExit(f"{len(blocks)} blocks in the trace, {len(plan)} in the stamp")
        print("\n| projection | M | kernels per call: instance, workgroups x threads | us per call | GB/s |")
        print("|---|---|---|---|---|")
        for (name, m, n, k, copies, reps), blk in zip(plan, blocks):
            calls = copies * reps
            if len(blk) % calls:
                raise SystemExit(f"{name} M={m}: {len(blk)} kernels for {calls} calls")
            per = len(blk) // calls
            kinds = []
            for r in blk[:per]:
                g = int(r.get("Grid_Size_X") or r.get("Grid_Size"))
                wg = int(r.get("Workgroup_Size_X") or r.get("Workgroup_Size"))
                kinds.append(f"{_short(r['Kernel_Name'])[5:]}, {g // wg} x {wg}")
            us = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in blk) / calls / 1e3
            print(f"| {name} | {m} | {' + '.join(kinds)} | {us:.2f} | {gemv_bytes(m, n, k) / (us * 1e-6) / 1e9:.0f} |")
    elif kind == "prefill-compare":
        rows = _read_csv(d0, "counter_collection.csv")
        per = defaultdict(lambda: defaultdict(float))
        for r in rows:
            if _short(r["Kernel_Name"]).startswith("mx4::prefill"):
                per[int(r["Dispatch_Id"])][r["Counter_Name"]] += float(r["Counter_Value"])
        ids = sorted(per)
        plan, calls = st["plan"], st["calls_per_instance"]
        if len(ids) != len(plan) * calls:
            raise SystemExit(f"{len(ids)} prefill dispatches, {len(plan) * calls} expected")
        names = sorted({cn for c in per.values() for cn in c})
        print("\n| shape | kernel | " + " | ".join(names) + " |")
        print("|---|---|" + "---|" * len(names))
        for i, (shape, desc, _) in enumerate(plan):
            grp = [per[d] for d in ids[i * calls:(i + 1) * calls]]
            avg = [sum(c.get(cn, 0.0) for c in grp) / calls for cn in names]
            print(f"| {shape} | {desc} | " + " | ".join(f"{v:.4g}" for v in avg) + " |")
    elif kind == "prefill-shapes":
        # --profile-prefill issues, per shape (q, o, gate, up, down) and
        # activation format (MXFP4, MX-FP8), 5 GEMMs on requantized activations
        # and 5 requantize + GEMM calls, then, for q, gate and down, 5 exact
        # GEMMs: the GEMM dispatches of the trace and of the counter run follow
        # that order
        m = int(st.get("m", 512))
        calls = int(st.get("gemm_launches_per_shape_and_format", 10))
        exact = int(st.get("exact_gemm_launches_per_shape", 5))
        dims = {name: (n, k) for name, n, k in LAYER}
        seq = []
        for name in ("q", "o", "gate", "up", "down"):
            seq += [(name, "mxfp4")] * calls + [(name, "mxfp8")] * calls
            if name in ("q", "gate", "down"):
                seq += [(name, "exact bf16")] * exact
        gemm = ("mx4::prefill_kernel", "mx4::prefill_lds_kernel", "mx4::gemm_exact")
        trace = sorted((r for r in _read_csv(d0, "kernel_trace.csv") if _short(r["Kernel_Name"]).startswith(gemm)),
                       key=lambda r: int(r["Dispatch_Id"]))
        pmc = defaultdict(lambda: defaultdict(float))
        for r in _read_csv(Path(dirs[1]), "counter_collection.csv"):
            if _short(r["Kernel_Name"]).startswith(gemm):
                pmc[int(r["Dispatch_Id"])][r["Counter_Name"]] += float(r["Counter_Value"])
        pids = sorted(pmc)
        if len(trace) != len(seq) or len(pids) != len(seq):
            raise SystemExit(f"{len(trace)} traced / {len(pids)} counted GEMM dispatches, {len(seq)} expected")
        peak = {"mxfp4": PEAK_TFLOPS["mxfp4"], "mxfp8": PEAK_TFLOPS["mxfp8"], "exact bf16": PEAK_TFLOPS["bf16"]}
        print("\n| shape | act | kernel instance | dispatches | us | TFLOP/s | of peak | MOPS x 512 | MFMA busy |")
        print("|---|---|---|---|---|---|---|---|---|")
        i = 0
        while i < len(seq):
            j = i
            while j < len(seq) and seq[j] == seq[i]:
                j += 1
            name, act = seq[i]
            n, k = dims[name]
            us = float(np.median([(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in trace[i:j]]))
            grp = [pmc[d] for d in pids[i:j]]
            mops = float(np.mean([c.get("SQ_INSTS_VALU_MFMA_MOPS_F6F4", 0) + c.get("SQ_INSTS_VALU_MFMA_MOPS_F8", 0) +
                                  c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0) for c in grp])) * 512
            busy = float(np.mean([c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) for c in grp])) / (us * 1e-6 * 2.4e9 * 1024)
            flops = 2.0 * m * n * k
            tf = flops / (us * 1e-6) / 1e12
            inst = _short(trace[i]["Kernel_Name"]).replace("mx4::", "")
            print(f"| {name} {m}x{k}->{n} | {act} | {inst} | {j - i} | {us:.2f} | {tf:.0f} | "
                  f"{tf / peak[act]:.1%} | {mops:.4g} ({mops / flops:.3f} x 2MNK) | {busy:.1%} |")
            i = j
    elif kind == "prefill-trace":
        rows = _read_csv(d0, "kernel_trace.csv")
        per = defaultdict(list)
        for r in rows:
            nm = _short(r["Kernel_Name"])
            if nm.startswith(("mx4::prefill", "mx4::quantize_fragments", "mx4::gemm_exact")):
                grid = r.get("Grid_Size") or r.get("Grid_Size_X")
                per[(nm, grid)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        print("\n| kernel | grid | dispatches | median us | min us |")
        print("|---|---|---|---|---|")
        for (nm, g), ts in sorted(per.items()):
            print(f"| {nm} | {g} | {len(ts)} | {np.median(ts):.2f} | {min(ts):.2f} |")
    elif kind in ("prefill-pmc", "step-pmc"):
        prefix = ("mx4::prefill", "mx4::gemm_exact") if kind == "prefill-pmc" else ("mx4::gemv",)
        rows = _read_csv(d0, "counter_collection.csv")
        per = defaultdict(lambda: defaultdict(float))
        meta = {}
        for r in rows:
            nm = _short(r["Kernel_Name"])
            if not nm.startswith(prefix):
                continue
            did = r["Dispatch_Id"]
            per[did][r["Counter_Name"]] += float(r["Counter_Value"])
            meta[did] = (nm, r["Grid_Size"])
        groups = defaultdict(list)
        for did, c in per.items():
            groups[meta[did]].append(c)
        names = sorted({cn for c in per.values() for cn in c})
        print("\n| kernel | grid | dispatches | " + " | ".join(names) + " |")
        print("|---|---|---|" + "---|" * len(names))
        for (nm, g), lst in sorted(groups.items()):
            avg = [sum(c.get(cn, 0.0) for c in lst) / len(lst) for cn in names]
            print(f"| {nm} | {g} | {len(lst)} | " + " | ".join(f"{v:.4g}" for v in avg) + " |")
    else:
        raise SystemExit(f"unknown summary kind {kind}")


# ---------------------------------------------------------------- main

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
    ap.add_argument("--no-1p7b", action="store_true", help="skip the Qwen3-1.7B step and the single 6144 x 2048 GEMV")
    ap.add_argument("--profile-step", action="store_true",
                    help="for kernel traces: only the recorded decode step (warmup + steps replays)")
    ap.add_argument("--profile-traffic", action="store_true",
                    help="for counter runs: 2 eager grouped steps, then a 1 GiB device copy as the byte calibration")
    ap.add_argument("--profile-prefill", action="store_true",
                    help="for profiler runs: only the M=512 prefill (q, o, gate, up, down; MXFP4 and MX-FP8 "
                         "activations): 5 GEMMs on requantized activations, then 5 requantize + GEMM calls; "
                         "and 5 exact GEMMs (AUTO, bf16 x) for q, gate and down")
    ap.add_argument("--profile-prefill-compare", action="store_true",
                    help="for counter runs: gate and q at M=512 (MXFP4), 5 calls each of the register-direct and "
                         "the workgroup-shared prefill kernel (for q also with K in halves of their own waves)")
    ap.add_argument("--profile-verify", action="store_true",
                    help="for kernel traces: only the speculative-verify shapes (each 8B projection and the lm_head "
                         "at M = 1..32 through AUTO over cold copies, enqueued 4 times)")
    ap.add_argument("--stamp", help="profile modes: also write the stamp (library sha256, workload) to this file")
    ap.add_argument("--summarize", nargs="+", metavar=("KIND", "DIR"),
                    help="print the markdown summary of rocprofv3 CSV output: trace DIR | traffic FETCH_DIR "
                         "WRITE_DIR | step-pmc DIR | verify-trace DIR | prefill-trace DIR | prefill-pmc DIR | "
                         "prefill-shapes TRACE_DIR PMC_DIR | prefill-compare DIR")
    args = ap.parse_args()

    if args.summarize:
        summarize(args.summarize[0], args.summarize[1:])
        return 0

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (the GEMV would shard "
              "column-wise with an all-gather of y; see the design notes). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    if mx4hip.device_count() < 1:
        print("no gfx950 device visible", file=sys.stderr)
        return 1

    ctx = mx4hip.Context(0)
    if args.profile_verify:
        # Each 8B projection and the lm_head at M = 1..32 token rows through
        # AUTO over the cold copies time_skinny uses, enqueued eagerly
        # VERIFY_REPS times (kernel durations do not depend on how the launch
        # was enqueued). A synth_bf16 launch (the block's input) opens every
        # (projection, M) block, so the summary can split the trace.
        plan = []
        for i, (name, n, k) in enumerate(LAYER + [LM_HEAD]):
            arena, copies = rotation(ctx, [(n, k)], 40000 + 1000 * i)
            for m in (1, 2, 4, 8, 16, 32):
                xb = ctx.buffer(m * k * 2)
                ctx.synth_bf16(2, 1.0, m * k, xb)
                yb = ctx.buffer(m * n * 4)
                for _ in range(VERIFY_REPS):
                    for ws in copies:
                        ctx.matmul_ptr(xb.ptr, mx4hip.BF16, m, ws[0], yb.ptr)
                ctx.synchronize()
                plan.append([name, m, n, k, len(copies), VERIFY_REPS])
            arena.release()
        # the grouped launches of a verify step (mx4_matmul_group): n is the
        # group's rows, whose bytes per call are one x read and every output
        dims = {name: (n, k) for name, n, k in LAYER}
        for gi, (label, members) in enumerate((("q|k|v", ["q", "k", "v"]), ("gate|up", ["gate", "up"]))):
            shapes = [dims[nm] for nm in members]
            k = shapes[0][1]
            arena, copies = rotation(ctx, shapes, 45000 + 1000 * gi)
            for m in (2, 4, 8, 16, 32):
                xb = ctx.buffer(m * k * 2)
                ctx.synth_bf16(2, 1.0, m * k, xb)
                ys = [ctx.buffer(m * n * 4) for n, _ in shapes]
                for _ in range(VERIFY_REPS):
                    for ws in copies:
                        ctx.matmul_group(xb.ptr, mx4hip.BF16, m, ws, [y.ptr for y in ys])
                ctx.synchronize()
                plan.append([label, m, sum(n for n, _ in shapes), k, len(copies), VERIFY_REPS])
            arena.release()
        write_stamp(args.stamp, {"profile_verify": True, "plan": plan})
        ctx.close()
        return 0
    log("synthesizing 253 resident MXFP4 weights (4.03 GB, one arena) on the GPU")
    weights, arena = build_step(ctx)

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
        ctx.reserve_prefill(m, 12288)
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
            # the exact matrix-core GEMM that AUTO runs above 32 token rows (bf16 x)
            if name in ("q", "gate", "down"):
                for _ in range(5):
                    ctx.matmul_ptr(xb.ptr, mx4hip.BF16, m, w, yb.ptr)
            ctx.synchronize()
        write_stamp(args.stamp, {"profile_prefill": True, "m": m, "gemm_launches_per_shape_and_format": 10,
                                 "requant_launches_per_shape_and_format": 6,
                                 "exact_gemm_launches_per_shape": 5})
        ctx.close()
        return 0

    if args.profile_prefill_compare:
        # counters of the two prefill kernels on the same shapes (MXFP4, M = 512,
        # warm weights): 5 eager calls of each instance, in this order
        m = 512
        by = {}
        for (nm, n, k, w) in weights:
            by.setdefault(nm, (n, k, w))
        ctx.reserve_prefill(m, 12288)
        plan = [("gate", "register-direct 4x3 tiles, K halves", (128, 192, 2)),
                ("gate", "workgroup-shared 128x192, U=2, D=3, K halves", (128, 192, 128 + 16 * 2 + 3)),
                ("gate", "the same in ping-pong (default)", (128, 192, 384 + 16 * 2 + 3)),
                ("q", "register-direct 2x2 tiles, K halves", (64, 128, 2)),
                ("q", "workgroup-shared 128x64, U=2, D=4, one ring", (128, 64, 16 * 2 + 4)),
                ("q", "workgroup-shared 128x64, U=2, D=4, K halves", (128, 64, 128 + 16 * 2 + 4)),
                ("q", "the same in ping-pong", (128, 64, 384 + 16 * 2 + 4))]
        for name, _, inst in plan:
            n, k, w = by[name]
            w.prepare_prefill()
            xb = ctx.buffer(m * k * 2)
            ctx.synth_bf16(3, 1.0, m * k, xb)
            yb = ctx.buffer(m * n * 4)
            xq, xsc = ctx.prefill_act_buffers(m, k, mx4hip.ACT_MXFP4)
            ctx.prefill_quantize(xb, mx4hip.BF16, m, k, mx4hip.ACT_MXFP4, xq, xsc)
            for _ in range(5):
                mx4hip.check(ctx.prefill_config(xq, xsc, mx4hip.ACT_MXFP4, m, w, yb, *inst))
            ctx.synchronize()
        write_stamp(args.stamp, {"profile_prefill_compare": True, "m": m, "calls_per_instance": 5,
                                 "plan": [[nm, desc, list(inst)] for nm, desc, inst in plan]})
        ctx.close()
        return 0

    if args.profile_traffic:
        for _ in range(2):
            enqueue()
        ctx.synchronize()
        src, dst = ctx.buffer(1 << 30), ctx.buffer(1 << 30)
        mx4hip.check(mx4hip.lib().mx4_copy(ctx.handle, dst.ptr, src.ptr, 1 << 30))
        ctx.synchronize()
        write_stamp(args.stamp, {"profile_traffic": True, "steps": 2, "launches_per_step": launches,
                                 "bytes_per_step": step_bytes, "calibration_copy_bytes": 1 << 30})
        ctx.close()
        return 0

    if args.eager:
        step = enqueue
        launch = f"eager, {launches} launches per step"
        pss = None
    else:
        pss = ctx.record(enqueue)
        step = pss.launch
        launch = f"recorded pass (HIP graph), {launches} launches per step"

    if args.profile_step:
        for _ in range(args.warmup + args.steps):
            step()
        ctx.synchronize()
        write_stamp(args.stamp, {"profile_step": True, "steps": args.steps, "warmup": args.warmup,
                                 "launches_per_step": launches, "bytes_per_step": step_bytes})
        ctx.close()
        return 0

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

    extra = {"gpu_ms_per_step": round(gpu_ms_per_step, 4), "launch": launch,
             "weights": "one device allocation, each weight on its own 2 MiB-aligned slice"}
    if pss is not None:
        extra["gpu_ms_per_step_median"] = round(time_step(ctx, pss, max(5, args.steps // 2)), 4)
        extra["gpu_ms_per_step_median_protocol"] = f"median of {REPS} runs of {max(5, args.steps // 2)} replays"
    if pss is not None:
        # the same grouped step enqueued from the host launch by launch
        for _ in range(2):
            enqueue()
        ctx.synchronize()
        te = []
        for _ in range(REPS):
            ctx.timer_begin()
            for _ in range(max(5, args.steps // 2)):
                enqueue()
            te.append(ctx.timer_end() / max(5, args.steps // 2))
        extra["gpu_ms_per_step_eager_median"] = round(float(np.median(te)), 4)
    if not args.separate:
        # the same step with one launch per projection (253), as the reference
        # dispatches it: what grouping q|k|v and gate|up saves
        p_sep = ctx.record(lambda: ctx.matmul_batch(ops))
        ms_sep = time_step(ctx, p_sep, max(5, args.steps // 2))
        p_sep.release()
        extra["one_launch_per_projection"] = {"launches": len(weights), "gpu_ms_per_step": round(ms_sep, 4),
                                              "GBps": round(step_bytes / (ms_sep * 1e-3) / 1e9, 1)}
    if not args.no_shapes:
        log("per-shape timing (>= 512 MiB of cold copies per shape)")
        extra["shapes"] = time_shapes(ctx, xs)
        log("lm_head + greedy argmax timing")
        extra["lm_head_argmax"] = time_lm_head_argmax(ctx, xs)

    if not args.no_skinny:
        log("skinny (speculative verify) timing")
        extra["skinny"] = time_skinny(ctx)
        log("grouped verify launches (q|k|v, gate|up) timing")
        extra["skinny_group"] = time_skinny_groups(ctx, separate=extra["skinny"])
        log("verify step timing (the whole 8B step at 2-16 token rows)")
        extra["verify_step"] = time_verify_step(ctx, weights)

    prefill_top = None
    if not args.no_prefill:
        log("matrix-core ceiling (scaled FP4 MFMAs back to back) and prefill (M=512, block-scaled MFMA) timing")
        extra["mfma_ceiling"] = time_mfma_ceiling(ctx)
        ceil = {act: extra["mfma_ceiling"][key]["random"]["TFLOPs"]
                for act, key in (("mxfp4", "32x32x64"), ("mxfp8", "fp8xfp4_32x32x64"), ("bf16", "bf16_32x32x16"))}
        extra["prefill"] = time_prefill(ctx, ceiling=ceil)
        extra["prefill_layer"] = time_prefill_layer(ctx, weights)
        log("prefill at 128 and 1024 token rows")
        extra["prefill_rows"] = time_prefill_rows(ctx)
        prefill_top = prefill_summary(extra["prefill"], extra["prefill_layer"], ceil)
        log("exact matrix-core path for M > 32 (AUTO)")
        extra["prefill_exact_auto"] = time_prefill_exact(ctx, ceiling=ceil["bf16"])

    if not args.no_1p7b:
        log("qwen3-1.7b decode step and the single 6144 x 2048 GEMV")
        extra["qwen3_1p7b"] = time_model_1p7b(ctx, max(5, args.steps // 2))
        extra["single_gemv_6144x2048"] = time_single_gemv(ctx)
        log("per-call drop-in (host buffers)")
        extra["dropin_per_call"] = time_dropin(ctx, weights, x_host)
        log("bf16 weights (the unquantized arm)")
        extra["bf16_weights"] = time_bf16_weights(ctx)
        log("embedding and quantization")
        extra["embed_quantize"] = time_embed_quantize(ctx, weights)

    cpu = None
    if not args.no_cpu_baseline:
        nt = host_threads()
        cpu_extra = {"host": host_cpu()}
        log("cpu baseline (oracle, 1 thread)")
        cpu = cpu_baseline(ctx, weights, x_host)
        if nt > 1:
            log(f"cpu baseline (oracle, {nt} threads)")
            cpu_extra["step_sample_all_threads"] = cpu_baseline(ctx, weights, x_host, threads=nt)
        log("cpu legs: verify (M = 2..16) and prefill (M = 512)")
        cpu_extra["verify_1_thread"] = cpu_verify(ctx, weights, 1)
        cpu_extra["prefill_1_thread"] = cpu_prefill(ctx, weights, 1)
        if nt > 1:
            cpu_extra["verify_all_threads"] = cpu_verify(ctx, weights, nt)
            cpu_extra["prefill_all_threads"] = cpu_prefill(ctx, weights, nt)
        log("cpu legs: whole shapes (the single 6144 x 2048 GEMV, every Qwen3-1.7B M = 1 projection)")
        # last in the line, so that the end of the printed line carries it whole
        cpu_extra["full_shapes"] = cpu_full_shapes(ctx, [1] + ([nt] if nt > 1 else []))
        extra["cpu"] = cpu_extra

    traffic, traffic_note = (None, "--separate launches differ from the profiled step") if args.separate \
        else traffic_from_profile()

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
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_note": traffic_note,
                     "basis": "algorithmic bytes of one decode step / GPU event time of one step"},
        "cpu_baseline": cpu,
        "prefill": prefill_top,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)
    ctx.synchronize()
    arena.release()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
