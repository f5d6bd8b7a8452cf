#!/usr/bin/env python3
"""Benchmark of the MI355X SageAttention quantized path (one JSON line on stdout).

Workload (BASELINE.json metric): ``sageattn`` at B=1, H=32, S=16384, D=128,
bf16, HND, causal, smooth_k=False.  A step is one full ``sageattn`` call (V
layout + INT8 quant of K + fused attention that quantises Q itself and runs
INT8-QK^T / fp16-PV) on inputs already resident in HBM; ``value`` is effective
TOPS of the whole step: 4*B*H*D*S(S+1)/2 / step time.

``roofline`` is that attention kernel alone, timed with HIP events on the
stream it is launched on (torch's current stream): achieved = the same ops /
average launch time, against the published dense INT8 MFMA peak of MI355X
(5.0 POP/s).  ``cpu_baseline`` is the CPU oracle (numpy, all host cores its
BLAS uses) on one head of the same workload, scaled to effective TOPS.
``reference_shapes`` times whole ``sageattn`` calls at the reference's own
benchmark shapes (non-causal SDXL / Anima / VAE lines), with and without the
key splits the library plans for grids that leave CUs idle.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NS|C2|C3|C4|C5]
       python bench.py --reference-shapes all|NAME[,NAME...]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "sageattention-rdna3_amd"))

METRIC = "effective attn TOPS + % gfx950 MFMA peak, D=128 S=16k causal bf16"
PEAK_INT8_TOPS = 5000.0  # MI355X dense INT8 MFMA (published)
PEAK_F16_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA (published)
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    # name: (B, Hq, Hkv, S, D, dtype, layout, causal, smooth_k)
    "NS": (1, 32, 32, 16384, 128, "bf16", "HND", True, False),
    "C2": (1, 10, 10, 4096, 64, "fp16", "HND", False, False),
    "C3": (2, 32, 32, 8192, 128, "bf16", "HND", True, True),
    "C4": (1, 32, 8, 16384, 128, "fp16", "NHD", True, False),
    "C5": (1, 40, 40, 32891, 128, "bf16", "HND", False, True),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def attn_ops(B, H, Sq, Sk, D, causal):
    if causal:
        n = min(Sq, Sk)
        pairs = n * (n + 1) // 2 + max(0, Sq - Sk) * Sk
    else:
        pairs = Sq * Sk
    return 4 * B * H * D * pairs


def make_inputs(cfg, device):
    import torch

    B, Hq, Hkv, S, D, dt, layout, causal, smooth = cfg
    dtype = torch.bfloat16 if dt == "bf16" else torch.float16
    g = torch.Generator(device=device).manual_seed(0)

    def shp(h):
        return (B, h, S, D) if layout == "HND" else (B, S, h, D)

    q = torch.randn(shp(Hq), generator=g, device=device, dtype=torch.float32).to(dtype)
    k = torch.randn(shp(Hkv), generator=g, device=device, dtype=torch.float32).to(dtype)
    v = torch.randn(shp(Hkv), generator=g, device=device, dtype=torch.float32).to(dtype)
    return q, k, v


def cpu_baseline(cfg, budget_s):
    """Time the CPU oracle on one (b, h) head of the workload: quant + V layout +
    attention of that head; returns the cpu_baseline object."""
    import numpy as np

    sys.path.insert(0, REPO)
    from oracle import sage_oracle as orc

    try:
        from threadpoolctl import threadpool_info

        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # noqa: BLE001
        threads = len(os.sched_getaffinity(0))
    B, Hq, Hkv, S, D, dt, layout, causal, smooth = cfg
    rng = np.random.default_rng(0)
    shp = (1, 1, S, D)
    q, k, v = (orc.from_f32(rng.standard_normal(shp).astype(np.float32), dt) for _ in range(3))
    t0 = time.perf_counter()
    mean = orc.k_mean(k, dt, "HND") if smooth else None
    q8, qs, k8, ks = orc.quant_qk_int8(q, k, dt, "HND", D ** -0.5, k_mean=mean)
    vt = orc.v_layout(v, dt, "HND")
    t_pro = time.perf_counter() - t0
    # attention rows in 512-row blocks, from the last (heaviest for causal) down,
    # until the whole head is done or the time budget is used
    done_pairs, rows_done, t_attn = 0, 0, 0.0
    for r1 in range(S, 0, -512):
        rows = np.arange(max(0, r1 - 512), r1)
        t1 = time.perf_counter()
        orc.attn_i8_rows(q8, k8, vt, qs, ks, 0, 0, rows, causal)
        t_attn += time.perf_counter() - t1
        done_pairs += orc.pairs_for_rows(rows, S, causal)
        rows_done += rows.size
        if t_attn + t_pro > budget_s:
            break
    ops = 4 * D * done_pairs
    # scale the prologue time to the rows done (it is computed for the whole head)
    t_total = t_attn + t_pro * rows_done / S
    return {
        "value": ops / t_total / 1e12,
        "unit": "TOPS",
        "cores": int(threads),
        "kind": "port",
        "sample": (f"CPU oracle (numpy) on head 0 of 1x{Hq} heads: quant+V layout of the head "
                   f"(pro-rated) + attention of {rows_done}/{S} query rows "
                   f"({'causal ' if causal else ''}{done_pairs} key pairs), {t_total:.1f} s"),
    }


def kernels_only(cfg, q, k, v, n):
    """Each kernel of the path n times, then a plain copy of 1 GiB n times (a
    kernel of known traffic: FETCH_SIZE and WRITE_SIZE should read 1 GiB each)."""
    import torch

    from sageattention import ops

    B, Hq, Hkv, S, D, dt, layout, causal, smooth = cfg
    lay = ops.HND if layout == "HND" else ops.NHD
    for _ in range(n):
        mean = ops.mean_seq(k, lay) if smooth else torch.empty(0, device=q.device, dtype=q.dtype)
        k8, ks, vt = ops.prep_kv_int8(k, v, mean, lay)
        o = torch.empty_like(q)
        ops.qk_int8_sv_bf16_attn_qfused_t(q, k8, vt, o, ks, lay, int(causal), D ** -0.5)
    src = torch.empty(1 << 30, dtype=torch.uint8, device=q.device)
    dst = torch.empty_like(src)
    for _ in range(n):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] kernels-only: {n} x path kernels + {n} x 1 GiB copy done")


# direct (unquantised) kernel: the largest D=128 self-attention shape the reference's dispatch sends to it
DIRECT_CFG = (1, 32, 32, 2048, 128, "bf16", "HND", True, False)


def direct_probe(dev, n):
    """The direct fp16/bf16 kernel alone (HIP events on its launch stream) at DIRECT_CFG, against the
    dense bf16 MFMA peak, and a whole ``sageattn`` call at that shape through either path (the
    direct path, and the INT8 path with the direct thresholds switched off)."""
    import torch

    from sageattention import ops, sageattn

    B, Hq, Hkv, S, D, dt, layout, causal, smooth = DIRECT_CFG
    q, k, v = make_inputs(DIRECT_CFG, dev)
    lay = ops.HND if layout == "HND" else ops.NHD
    vt = torch.empty(B, Hkv, D, (S + 63) // 64 * 64, device=dev, dtype=torch.float16)
    ops.v_transpose(v, vt, lay)
    o = torch.empty_like(q)
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        for _ in range(3):
            fn()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / n

    ms_kernel = timed(lambda: ops.bf16_attn_t(q, k, vt, o, lay, int(causal), D ** -0.5, 0))
    ms_direct = timed(lambda: sageattn(q, k, v, tensor_layout=layout, is_causal=causal))
    names = ["SAGEATTN_DIRECT_THRESHOLD_D128", "SAGEATTN_DIRECT_THRESHOLD_D128_CROSS"]
    saved = {x: os.environ.get(x) for x in names}
    try:
        for x in names:
            os.environ[x] = "-1"
        ms_int8 = timed(lambda: sageattn(q, k, v, tensor_layout=layout, is_causal=causal))
    finally:
        for x, val in saved.items():
            if val is None:
                os.environ.pop(x, None)
            else:
                os.environ[x] = val
    flops = attn_ops(B, Hq, S, S, D, causal)
    achieved = flops / (ms_kernel * 1e-3) / 1e12
    log(f"[bench] direct kernel {ms_kernel:.4f} ms = {achieved:.1f} TFLOP/s "
        f"({100 * achieved / PEAK_F16_TFLOPS:.1f}% bf16 peak); sageattn at this shape: direct {ms_direct:.4f} ms, "
        f"int8 path {ms_int8:.4f} ms")
    return {
        "workload": f"bf16_attn_t B{B} Hq{Hq} S{S} D{D} {dt} {layout} {'causal' if causal else 'non-causal'}",
        "kernel": "attn_fwd_kernel (bf16 QK)",
        "kernel_ms": round(ms_kernel, 5),
        "achieved": round(achieved, 2),
        "peak": PEAK_F16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_F16_TFLOPS, 4),
        "sageattn_direct_ms": round(ms_direct, 5),
        "sageattn_int8_ms": round(ms_int8, 5),
    }


# the reference's own benchmark shapes (benchmark_attn/benchmark_attn.py:143-174, results in
# benchmark_attn-result-native.txt; all non-causal HND, h_q == h_kv): name, B, H, Sq, Sk, D, dtype.  The
# long self-attention shapes take the INT8 path, the short and cross-attention ones (kv 77, 154, 512,
# self-attention up to 2304) the direct path, as the reference dispatches them.
REFERENCE_SHAPES = [
    ("SDXL01", 1, 10, 4096, 4096, 64, "fp16"), ("SDXL02", 1, 10, 4096, 77, 64, "fp16"),
    ("SDXL03", 1, 10, 4096, 154, 64, "fp16"), ("SDXL04", 1, 20, 1024, 1024, 64, "fp16"),
    ("SDXL05", 1, 20, 1024, 77, 64, "fp16"), ("SDXL06", 1, 20, 1024, 154, 64, "fp16"),
    ("SDXLVAE01", 1, 4, 16384, 16384, 128, "fp16"), ("SDXL07", 1, 10, 6144, 6144, 64, "fp16"),
    ("SDXL08", 1, 10, 6144, 77, 64, "fp16"), ("SDXL09", 1, 10, 6144, 154, 64, "fp16"),
    ("SDXL10", 1, 20, 1536, 1536, 64, "fp16"), ("SDXL11", 1, 20, 1536, 77, 64, "fp16"),
    ("SDXL12", 1, 20, 1536, 154, 64, "fp16"), ("SDXLVAE02", 1, 4, 24576, 24576, 128, "fp16"),
    ("SDXL13", 1, 10, 9216, 9216, 64, "fp16"), ("SDXL14", 1, 10, 9216, 77, 64, "fp16"),
    ("SDXL15", 1, 10, 9216, 154, 64, "fp16"), ("SDXL16", 1, 20, 2304, 2304, 64, "fp16"),
    ("SDXL17", 1, 20, 2304, 77, 64, "fp16"), ("SDXL18", 1, 20, 2304, 154, 64, "fp16"),
    ("Anima01", 1, 16, 4096, 4096, 128, "bf16"), ("Anima02", 1, 16, 4096, 512, 128, "bf16"),
    ("AnimaVAE01", 1, 3, 16384, 16384, 128, "bf16"), ("Anima03", 1, 16, 6144, 6144, 128, "bf16"),
    ("Anima04", 1, 16, 6144, 512, 128, "bf16"), ("AnimaVAE02", 1, 3, 24576, 24576, 128, "bf16"),
    ("Anima05", 1, 16, 9216, 9216, 128, "bf16"), ("Anima06", 1, 16, 9216, 512, 128, "bf16"),
]


def reference_shapes_probe(dev, n, names=None, modes=("auto", "1")):
    """Whole ``sageattn`` calls (the reference's dispatch: quantisation, V layout and INT8 attention, or
    V layout and the direct kernel) at the reference's benchmark shapes (``names``: a subset), back to
    back on one stream, with the library's key-split plan and with splitting switched off
    (SAGEATTN_KV_SPLITS=1).  ``ms`` is the time per call as a caller sees it: for the smallest
    shapes the host's issue time per call, when it exceeds the GPU's."""
    import torch

    from sageattention import _capi, sageattn
    from sageattention.core import use_direct_path

    out = []
    saved = os.environ.get("SAGEATTN_KV_SPLITS")
    try:
        for name, B, H, Sq, Sk, D, dt in REFERENCE_SHAPES:
            if names is not None and name not in names:
                continue
            dtype = torch.bfloat16 if dt == "bf16" else torch.float16
            g = torch.Generator(device=dev).manual_seed(0)
            q = torch.randn((B, H, Sq, D), generator=g, device=dev, dtype=torch.float32).to(dtype)
            k = torch.randn((B, H, Sk, D), generator=g, device=dev, dtype=torch.float32).to(dtype)
            v = torch.randn((B, H, Sk, D), generator=g, device=dev, dtype=torch.float32).to(dtype)
            direct = use_direct_path(D, Sq, Sk, False, "HND")
            calls = n if Sq * Sk >= 1 << 24 else max(n, 200)  # enough calls to time the short shapes
            # the modes alternate over three rounds and each reports its median round, so that clock drift
            # during the probe does not favour the mode measured first
            times = {mode: [] for mode in modes}
            for _round in range(3):
                for mode in modes:
                    if mode == "auto":
                        os.environ.pop("SAGEATTN_KV_SPLITS", None)
                    else:
                        os.environ["SAGEATTN_KV_SPLITS"] = mode
                    for _ in range(3):
                        sageattn(q, k, v, tensor_layout="HND", is_causal=False)
                    torch.cuda.synchronize()
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(calls):
                        sageattn(q, k, v, tensor_layout="HND", is_causal=False)
                    e1.record()
                    e1.synchronize()
                    times[mode].append(e0.elapsed_time(e1) / calls)
            res = {mode: sorted(t)[1] for mode, t in times.items()}
            whole, splits = _capi.split_plan(not direct, B, H, Sq, Sk, D, False, 0)
            flops = attn_ops(B, H, Sq, Sk, D, False)
            row = {"shape": name, "B": B, "H": H, "Sq": Sq, "Sk": Sk, "D": D, "dtype": dt,
                   "path": "direct" if direct else "int8", "plan": {"whole_qblocks": whole, "splits": splits}}
            if "auto" in res:
                row.update(ms=round(res["auto"], 4), tops=round(flops / (res["auto"] * 1e-3) / 1e12, 1))
            if "1" in res:
                row.update(ms_unsplit=round(res["1"], 4))
            out.append(row)
            log(f"[bench] {name} ({row['path']}): " +
                ", ".join(f"{'sageattn' if m == 'auto' else 'unsplit'} {t:.4f} ms" for m, t in res.items()) +
                f", plan {whole} whole + splits of {splits}")
            del q, k, v
    finally:
        if saved is None:
            os.environ.pop("SAGEATTN_KV_SPLITS", None)
        else:
            os.environ["SAGEATTN_KV_SPLITS"] = saved
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="NS", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU oracle work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-probes", action="store_true",
                    help="skip the direct-kernel and reference-shape probes (kernel traces of the NS workload alone)")
    ap.add_argument("--reference-shapes", default=None, metavar="NAMES",
                    help="only time sageattn at these reference benchmark shapes (comma list, or 'all'), "
                         "print them as one JSON line and exit; for rocprofv3 runs of the split path")
    ap.add_argument("--reference-modes", default="auto,1", metavar="MODES",
                    help="with --reference-shapes: 'auto' (the library's key-split plan) and/or '1' (unsplit)")
    ap.add_argument("--kernels-only", action="store_true",
                    help="launch each path kernel --steps times plus a 1 GiB device copy (the HBM-counter "
                         "calibration) and exit; for rocprofv3 --pmc runs")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the path shards by (batch, head) "
              "with no communication, so N GPUs run N independent copies of this single-GPU line.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from sageattention import ops, sageattn

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = CONFIGS[args.config]
    B, Hq, Hkv, S, D, dt, layout, causal, smooth = cfg
    props = torch.cuda.get_device_properties(dev)
    log(f"[bench] device {props.name} CUs={props.multi_processor_count} config={args.config} {cfg}")

    if args.reference_shapes:
        names = None if args.reference_shapes == "all" else set(args.reference_shapes.split(","))
        unknown = (names or set()) - {x[0] for x in REFERENCE_SHAPES}
        if unknown:
            sys.exit(f"unknown reference shapes: {sorted(unknown)}")
        modes = tuple(m for m in args.reference_modes.split(",") if m)
        if not modes or any(m not in ("auto", "1") for m in modes):
            sys.exit("--reference-modes takes 'auto' and/or '1'")
        print(json.dumps({"reference_shapes": reference_shapes_probe(dev, max(args.steps, 10), names, modes)}),
              flush=True)
        return

    q, k, v = make_inputs(cfg, dev)
    torch.cuda.synchronize()
    if args.kernels_only:
        kernels_only(cfg, q, k, v, args.steps)
        return

    def step():
        return sageattn(q, k, v, tensor_layout=layout, is_causal=causal, smooth_k=smooth)

    for i in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"[bench] warmup {args.warmup} done")

    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps
    ops_step = attn_ops(B, Hq, S, S, D, causal)
    value = ops_step / (ms_step * 1e-3) / 1e12
    log(f"[bench] {args.steps} steps: {ms_step:.4f} ms/step, {value:.1f} effective TOPS")

    # ---- per-kernel timing with HIP events on the launch stream
    lay = ops.HND if layout == "HND" else ops.NHD
    stream = torch.cuda.current_stream(dev)
    mean = ops.mean_seq(k, lay) if smooth else torch.empty(0, device=dev, dtype=q.dtype)
    q8, qs, k8, ks = ops.quant_qk_int8(q, k, mean, lay, D ** -0.5)
    vt = torch.empty(B, Hkv, D, (S + 63) // 64 * 64, device=dev, dtype=torch.float16)
    ops.v_transpose(v, vt, lay)
    o = torch.empty_like(q)

    def timed(fn, n):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        for _ in range(3):
            fn()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / n

    n_k = max(args.steps, 10)
    ms_attn = timed(lambda: ops.qk_int8_sv_bf16_attn_qfused_t(q, k8, vt, o, ks, lay, int(causal), D ** -0.5), n_k)
    ms_attn_unfused = timed(lambda: ops.qk_int8_sv_bf16_attn_t(q8, k8, vt, o, qs, ks, lay, int(causal), D ** -0.5),
                            n_k)
    # The prologue kernels stream HBM: back to back on the same tensors, part of their traffic would hit the
    # L2 / Infinity Cache (256 MB), so each launch gets its own input set out of NROT (together well past the
    # caches), and the output of a set is written while the next set is read.
    NROT = 3
    qr = [q] + [q.clone() for _ in range(NROT - 1)]
    kr = [k] + [k.clone() for _ in range(NROT - 1)]
    vr = [v] + [v.clone() for _ in range(NROT - 1)]
    vtr = [vt] + [torch.empty_like(vt) for _ in range(NROT - 1)]
    rot = [0]

    def rotated(fn):
        def call():
            i = rot[0] % NROT
            rot[0] += 1
            fn(i)
        return call

    # quant allocates its outputs per call (as the reference op does); holding each set's last outputs until
    # the set comes round again keeps NROT + 1 output blocks in rotation instead of one reused block
    qouts = [None] * NROT
    ms_quant = timed(rotated(lambda i: qouts.__setitem__(i, ops.quant_qk_int8(qr[i], kr[i], mean, lay, D ** -0.5))),
                     n_k)
    ms_kquant = timed(rotated(lambda i: qouts.__setitem__(i, ops.quant_k_int8(kr[i], mean, lay))), n_k)
    ms_prep = timed(rotated(lambda i: qouts.__setitem__(i, ops.prep_kv_int8(kr[i], vr[i], mean, lay))), n_k)
    ms_vl = timed(rotated(lambda i: ops.v_transpose(vr[i], vtr[i], lay)), n_k)
    ms_mean = timed(rotated(lambda i: ops.mean_seq(kr[i], lay)), n_k) if smooth else 0.0
    del qr, kr, vr, vtr, qouts
    torch.cuda.synchronize()
    achieved = ops_step / (ms_attn * 1e-3) / 1e12
    nq, nk = B * Hq * S * D, B * Hkv * S * D
    quant_bytes = 2 * (nq + nk) + (nq + nk) + 4 * (B * Hq * ((S + 31) // 32) + B * Hkv * ((S + 15) // 16))
    kquant_bytes = 2 * nk + nk + 4 * B * Hkv * ((S + 15) // 16)
    vl_bytes = 2 * nk + 2 * B * Hkv * D * ((S + 63) // 64 * 64)
    mean_bytes = 2 * nk + 2 * B * Hkv * D
    mixed = 2.0 / (1.0 / PEAK_INT8_TOPS + 1.0 / PEAK_F16_TFLOPS)
    log(f"[bench] attn kernel {ms_attn:.4f} ms = {achieved:.1f} TOPS ({100 * achieved / PEAK_INT8_TOPS:.1f}% INT8 peak); "
        f"(two-kernel path {ms_attn_unfused:.4f} ms); quant Q+K {ms_quant * 1e3:.1f} us = "
        f"{quant_bytes / ms_quant / 1e6:.0f} GB/s, K only {ms_kquant * 1e3:.1f} us; "
        f"v_layout {ms_vl * 1e3:.1f} us = {vl_bytes / ms_vl / 1e6:.0f} GB/s; K quant + V layout in one launch "
        f"{ms_prep * 1e3:.1f} us = {(kquant_bytes + vl_bytes) / ms_prep / 1e6:.0f} GB/s")

    direct = None if args.no_probes else direct_probe(dev, n_k)
    ref_shapes = None if args.no_probes else reference_shapes_probe(dev, n_k)

    traffic = None
    tfile = os.path.join(REPO, "profiles", f"hbm_traffic_{args.config}.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            traffic = json.load(f).get("attn_bytes_per_launch")

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU oracle baseline ...")
        cpu = cpu_baseline(cfg, args.cpu_budget)
        log(f"[bench] cpu {cpu['value']:.4g} TOPS on {cpu['cores']} threads")

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic N(0,1) inputs generated on the GPU from seed 0",
        "config": {
            "workload": f"{args.config}: sageattn B{B} Hq{Hq} Hkv{Hkv} S{S} D{D} {dt} {layout} "
                        f"{'causal' if causal else 'non-causal'} smooth_k={smooth}",
            "B": B, "Hq": Hq, "Hkv": Hkv, "S": S, "D": D, "io_dtype": dt, "layout": layout,
            "causal": causal, "smooth_k": smooth, "qk": "int8 MFMA", "pv": "fp16 MFMA",
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_INT8_TOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_INT8_TOPS, 4),
            "traffic": traffic,
            "kernel": "attn_fwd_kernel (int8 QK, Q quantised in the kernel)",
            "kernel_ms": round(ms_attn, 5),
            "two_kernel_path_attn_ms": round(ms_attn_unfused, 5),
            "frac_of_mixed_int8_fp16_ceiling": round(achieved / mixed, 4),
        },
        "prologue": {
            "quant_us": round(ms_quant * 1e3, 2),
            "quant_GBps": round(quant_bytes / ms_quant / 1e6, 1),
            "quant_frac_hbm": round(quant_bytes / ms_quant / 1e6 / PEAK_HBM_GBS, 4),
            "k_quant_us": round(ms_kquant * 1e3, 2),
            "k_quant_GBps": round(kquant_bytes / ms_kquant / 1e6, 1),
            "prep_kv_us": round(ms_prep * 1e3, 2),
            "prep_kv_GBps": round((kquant_bytes + vl_bytes) / ms_prep / 1e6, 1),
            "prep_kv_frac_hbm": round((kquant_bytes + vl_bytes) / ms_prep / 1e6 / PEAK_HBM_GBS, 4),
            "v_layout_us": round(ms_vl * 1e3, 2),
            "v_layout_GBps": round(vl_bytes / ms_vl / 1e6, 1),
            "k_mean_us": round(ms_mean * 1e3, 2) if smooth else None,
            "k_mean_GBps": round(mean_bytes / ms_mean / 1e6, 1) if smooth else None,
        },
        "direct": direct,
        "reference_shapes": ref_shapes,
        "device": {"name": props.name, "cus": props.multi_processor_count},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
