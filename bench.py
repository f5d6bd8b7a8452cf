#!/usr/bin/env python3
"""Benchmark of the MI355X SageAttention quantized path (one JSON line on stdout).

Workload (BASELINE.json metric): ``sageattn`` at B=1, H=32, S=16384, D=128,
bf16, HND, causal, smooth_k=False.  A step is one full ``sageattn`` call (V
layout + INT8 quant of K + fused attention that quantises Q itself and runs
INT8-QK^T / fp16-PV) on inputs already resident in HBM; ``value`` is effective
TOPS of the whole step: 4*B*H*D*S(S+1)/2 / step time.  Order: the inputs are
generated on the CPU and copied over, the per-kernel probes of the same
tensors run (each settled first: the GPU clock ramps up over its first ~50 ms
of work after an idle period), then W warmup steps and the K timed steps.

``roofline`` is that attention kernel alone, timed with HIP events on the
stream it is launched on (torch's current stream): achieved = the same ops /
average launch time, against the published dense INT8 MFMA peak of MI355X
(5.0 POP/s).  ``configs`` times the other BASELINE configs (C2-C5) the same way
in the same run: the whole step, the attention kernel and the prologue kernels
with their HBM fractions.  ``cpu_baseline`` is the PyTorch CPU implementation of
the same quantized math (oracle/torch_cpu.py) on the host cores, on a fixed
subset of heads scaled to the whole workload.  ``reference_shapes`` times whole
``sageattn`` calls at the reference's own benchmark shapes, called as its
benchmark calls them (NHD, non-causal), with MaxErr / MSE / CosSim against fp32
attention as in its benchmark.

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


# BASELINE.json input distributions beyond N(0,1): C3's per-channel K offset (std 2, shared across tokens) and
# C5's x20 outlier channels (1% of D) in Q and K
K_OFFSET_STD = {"C3": 2.0}
OUTLIER_FRAC = {"C5": 0.01}


def make_inputs(cfg, device, name=None):
    """q, k, v of the config, generated on the CPU in fp32 from torch.Generator().manual_seed(0) (q, k, v in
    that order, then C3's K offset and C5's outlier channels), cast to the config's dtype and copied to
    ``device`` before any timing: the same bits as the parity tests' inputs for that seed."""
    import torch

    B, Hq, Hkv, S, D, dt, layout, causal, smooth = cfg
    dtype = torch.bfloat16 if dt == "bf16" else torch.float16
    g = torch.Generator().manual_seed(0)

    def shp(h):
        return (B, h, S, D) if layout == "HND" else (B, S, h, D)

    q = torch.randn(shp(Hq), generator=g)
    k = torch.randn(shp(Hkv), generator=g)
    v = torch.randn(shp(Hkv), generator=g)
    if name in K_OFFSET_STD:
        off = torch.randn((B, Hkv, 1, D), generator=g) * K_OFFSET_STD[name]
        k += off if layout == "HND" else off.transpose(1, 2)
    if name in OUTLIER_FRAC:
        n_out = max(1, round(OUTLIER_FRAC[name] * D))
        chans = torch.randperm(D, generator=g)[:n_out]
        q[..., chans] *= 20.0
        k[..., chans] *= 20.0
    return tuple(t.to(dtype).to(device) for t in (q, k, v))


class SclkSampler:
    """Samples the GPU's current shader clock as the driver reports it in sysfs (hwmon freq1_input, else the
    starred line of pp_dpm_sclk, "S: <MHz>" on MI355X) in a background thread while a timed loop runs; the card
    is the one whose PCI address is the device's.  Each read queries the SMU (~5 ms), and its value averages
    over a window that includes the gaps between launches, so it reads lower than the clock inside a kernel
    (measured with s_memtime / s_memrealtime stamps: ~1.85 GHz under the NS attention kernel).  Reports the
    median sample in MHz, or None where the files are not readable."""

    def __init__(self, dev):
        import glob
        import torch

        self.path, self.kind, self.samples = None, None, []
        props = torch.cuda.get_device_properties(dev)
        want = f"{props.pci_domain_id:04x}:{props.pci_bus_id:02x}:{props.pci_device_id:02x}"
        for card in sorted(glob.glob("/sys/class/drm/card*/device")):
            try:
                with open(os.path.join(card, "uevent")) as f:
                    slot = next((ln.split("=", 1)[1].strip() for ln in f if ln.startswith("PCI_SLOT_NAME=")), "")
            except OSError:
                continue
            if not slot.lower().startswith(want):
                continue
            hw = sorted(glob.glob(os.path.join(card, "hwmon", "hwmon*", "freq1_input")))
            if hw:
                self.path, self.kind = hw[0], "hwmon"
            elif os.path.exists(os.path.join(card, "pp_dpm_sclk")):
                self.path, self.kind = os.path.join(card, "pp_dpm_sclk"), "dpm"
            break

    def _read(self):
        try:
            with open(self.path) as f:
                text = f.read()
        except OSError:
            return None
        if self.kind == "hwmon":
            return int(text.strip()) / 1e6
        for ln in text.splitlines():
            if ln.strip().endswith("*"):
                return float(ln.split(":")[1].strip().rstrip("*").strip().lower().rstrip("mhz"))
        return None

    def __enter__(self):
        import threading

        self._stop = threading.Event()

        def run():
            while not self._stop.wait(0.005):
                v = self._read()
                if v is not None:
                    self.samples.append(v)

        if self.path:
            self._t = threading.Thread(target=run, daemon=True)
            self._t.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        if self.path:
            self._t.join()

    def mhz(self):
        if not self.samples:
            return None
        v = sorted(self.samples)
        return round(v[len(v) // 2], 1)


def queue_ahead(dev):
    """Occupy the GPU for about 2 ms (a fill of 12 GiB, HBM-bound, not MFMA: a matmul here lowers the clock
    for the next ~20 ms of MFMA work) so that the host can enqueue a whole timed loop while it runs: the
    events then bracket back-to-back launches, not the host's per-call overhead, which at the shortest
    kernels here (under 10 us) would otherwise be part of every launch's time."""
    import torch

    if dev not in _BUSY:
        _BUSY[dev] = torch.empty(12 << 30, device=dev, dtype=torch.uint8)
    _BUSY[dev].fill_(0)


_BUSY = {}


SETTLE_MS = 60.0


def settle(fn, ms=SETTLE_MS, label=None):
    """Call fn (at least 3 times) until the GPU has run it for ``ms`` milliseconds of wall time, and return the
    number of calls.  After an idle period (the CPU input generation) the GPU's clock ramps up over its first
    ~50 ms of work: NS steps measured 1.83 ms averaged over the first 10 after a 2 s idle, 1.64 ms over the
    next 10 and 1.607 ms from the 30th on (C3: 1.10, 0.98, then 0.915), so a probe timed straight after an
    idle period reads the ramp, not the kernel."""
    import torch

    t0 = time.perf_counter()
    calls, batch = 0, 1
    while True:
        for _ in range(batch):
            fn()
        torch.cuda.synchronize()
        calls += batch
        if calls >= 3 and (time.perf_counter() - t0) * 1e3 >= ms:
            if label:
                log(f"[bench] {label}: settled over {calls} calls")
            return calls
        batch = min(2 * batch, 256)


def timed_launches(fn, n, stream, dev, queue=True, label=None):
    """Average time of one call of fn over n back-to-back calls, with HIP events on the launch stream (settled
    first; with queue, the GPU kept busy while the n calls are enqueued -- for kernels shorter than the host's
    per-call time)."""
    import torch

    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    settle(fn, label=label)
    if queue:
        torch.cuda.synchronize(dev)
        queue_ahead(dev)
    e0.record(stream)
    for _ in range(n):
        fn()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / n


def step_breakdown(cfg, q, k, v, n, stream, queue=False, label=None):
    """The launches of one ``sageattn`` INT8 step -- the K prologue (smooth_k: the K mean's chunk sums, then K
    quantisation finishing the mean + V layout; else K quantisation + V layout in one launch), then the
    attention kernel that quantises Q (and the key-split merge when its plan splits) -- issued through the ops
    layer in the same order on the same tensors, n steps back to back with HIP events on the launch stream
    between them: each part's GPU time inside the step, and the GPU's idle time between steps.  With ``queue``
    (steps shorter than the ops layer's host time per step, which is longer than ``sageattn``'s compiled host
    layer: C2) the steps are queued behind an HBM fill, so that host time is not part of them; long steps are
    issued as ``sageattn``'s are (a fill before them measured the NS attention 3% slower).  ``ms_per_step`` minus
    the parts' sum is the host time a ``sageattn`` step adds."""
    import torch

    from sageattention import ops

    B, Hq, Hkv, S, D, dt, layout, causal, smooth = cfg
    lay = ops.HND if layout == "HND" else ops.NHD
    empty = torch.empty(0, device=q.device, dtype=q.dtype)

    def one(ev):
        if ev is not None:
            ev[0].record(stream)
        if smooth:
            k8, ks, vt = ops.prep_kv_int8_smooth(k, v, lay)
        else:
            k8, ks, vt = ops.prep_kv_int8(k, v, empty, lay)
        if ev is not None:
            ev[1].record(stream)
        o = torch.empty_like(q)
        ops.qk_int8_sv_bf16_attn_qfused_t(q, k8, vt, o, ks, lay, int(causal), D ** -0.5)
        if ev is not None:
            ev[2].record(stream)
        return o

    settle(lambda: one(None), label=label)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(n)]
    if queue:
        queue_ahead(q.device)
    for e in evs:
        one(e)
    torch.cuda.synchronize()
    prep = sum(e[0].elapsed_time(e[1]) for e in evs) / n
    attn = sum(e[1].elapsed_time(e[2]) for e in evs) / n
    gap = sum(evs[i][2].elapsed_time(evs[i + 1][0]) for i in range(n - 1)) / max(1, n - 1)
    return {"steps": n, "queued_behind_fill": queue, "prologue_us": round(prep * 1e3, 2), "attention_ms": round(attn, 5),
            "gap_between_steps_us": round(gap * 1e3, 2), "sum_ms": round(prep + attn + gap, 5)}


def cpu_baseline(cfg, budget_s):
    """The PyTorch CPU implementation of the same quantized math (oracle/torch_cpu.py: per-block INT8 Q/K
    quantisation with fp32 scales, K mean for smooth_k, fp16 V, exact integer QK^T, fp32 online softmax over
    key blocks with P rounded to fp16 before P.V), timed on the host cores: all of them
    (torch.set_num_threads(len(os.sched_getaffinity(0)))), wall clock, 1 warm-up then the median of 3 runs,
    on a fixed subset of query heads (as many as fit about a third of the time budget per run, at least one)
    and scaled linearly by Hq.  Inputs are generated on the CPU from seed 0."""
    import torch

    sys.path.insert(0, REPO)
    from oracle import torch_cpu

    B, Hq, Hkv, S, D, dt, layout, causal, smooth = cfg
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    dtype = torch.bfloat16 if dt == "bf16" else torch.float16
    g = torch.Generator().manual_seed(0)
    G = Hq // Hkv

    def run(nh):
        hk = max(1, -(-nh // G))
        q = torch.randn((1, nh, S, D), generator=g).to(dtype)
        k = torch.randn((1, hk, S, D), generator=g).to(dtype)
        v = torch.randn((1, hk, S, D), generator=g).to(dtype)
        t0 = time.perf_counter()
        torch_cpu.sageattn_heads(q, k, v, causal, D ** -0.5, smooth_k=smooth)
        return time.perf_counter() - t0

    t_warm = run(1)  # warm-up (one head), also sizes the sample
    nh = int(max(1, min(Hq, budget_s / 3.0 // max(t_warm, 1e-3))))
    times = sorted(run(nh) for _ in range(3))
    t_med = times[1]
    ops = attn_ops(B, Hq, S, S, D, causal)
    t_all = t_med * (B * Hq) / nh
    info = torch.__config__.parallel_info().strip().splitlines()
    return {
        "value": round(ops / t_all / 1e12, 5),
        "unit": "TOPS",
        "cores": cores,
        "kind": "port",
        "sample": (f"PyTorch CPU implementation of the quantized path (oracle/torch_cpu.py) on {nh} of {B * Hq} "
                   f"query heads (all {S} rows, {'causal' if causal else 'non-causal'}), median of 3 runs after "
                   f"1 warm-up: {t_med:.2f} s, scaled x{B * Hq / nh:.3g} to the workload"),
        "threads": torch.get_num_threads(),
        "parallel_info": [ln.strip() for ln in info if ln.strip()][:8],
    }


def kernels_only(cfg, q, k, v, n):
    """Each kernel of the path n times, the direct kernel at DIRECT_CFG n times, then a plain copy of 1 GiB n
    times (a kernel of known traffic: FETCH_SIZE and WRITE_SIZE should read 1 GiB each)."""
    import torch

    from sageattention import ops

    B, Hq, Hkv, S, D, dt, layout, causal, smooth = cfg
    lay = ops.HND if layout == "HND" else ops.NHD
    for _ in range(n):
        if smooth:
            k8, ks, vt = ops.prep_kv_int8_smooth(k, v, lay)
        else:
            k8, ks, vt = ops.prep_kv_int8(k, v, torch.empty(0, device=q.device, dtype=q.dtype), lay)
        o = torch.empty_like(q)
        ops.qk_int8_sv_bf16_attn_qfused_t(q, k8, vt, o, ks, lay, int(causal), D ** -0.5)
    dq, dk, dv = make_inputs(DIRECT_CFG, q.device)
    dB, dH, _, dS, dD = DIRECT_CFG[:5]
    dvt = torch.empty(dB, dH, dD, (dS + 63) // 64 * 64, device=q.device, dtype=torch.float16)
    ops.v_transpose(dv, dvt, ops.HND)
    do = torch.empty_like(dq)
    for _ in range(n):
        ops.bf16_attn_t(dq, dk, dvt, do, ops.HND, int(DIRECT_CFG[7]), dD ** -0.5, 0)
    del dq, dk, dv, dvt, do
    src = torch.empty(1 << 30, dtype=torch.uint8, device=q.device)
    dst = torch.empty_like(src)
    for _ in range(n):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] kernels-only: {n} x path kernels + {n} x 1 GiB copy done")


def under_profiler():
    """True when this process itself runs under rocprofv3 (its tool library is preloaded)."""
    return "rocprofiler" in os.environ.get("LD_PRELOAD", "") or any(k.startswith("ROCPROF") for k in os.environ)


def _counter_means(csv_path, counter):
    """{short kernel name: mean over dispatches of the counter (summed over its dimensions)} of a rocprofv3
    counter_collection.csv; the 1 GiB device copy is named "copy_1GiB"."""
    import csv
    import collections

    per = collections.defaultdict(float)
    names = {}
    with open(csv_path) as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") != counter:
                continue
            name = r["Kernel_Name"]
            if "sage::" in name and "(anonymous namespace)::" in name:
                short = name.split("(anonymous namespace)::")[1].split("(sage")[0]
            elif "copyBuffer" in name:
                short = "copy_1GiB"
            else:
                continue
            per[r["Dispatch_Id"]] += float(r["Counter_Value"])
            names[r["Dispatch_Id"]] = short
    acc = collections.defaultdict(list)
    for d, v in per.items():
        acc[names[d]].append(v)
    return {k: sum(v) / len(v) for k, v in acc.items()}


def measure_traffic(config, D, steps=3):
    """HBM bytes per launch of the fused-Q attention kernel, measured now: two rocprofv3 --pmc runs (FETCH_SIZE,
    then WRITE_SIZE, one counter each) of this script's --kernels-only mode for the same config, each in a child
    process while this one waits, each counter's KiB per dispatch scaled by what it reads for the 1 GiB device
    copy that mode ends with (FETCH_SIZE reads the copy as 0.5 GiB, WRITE_SIZE as 1 GiB).  None when rocprofv3
    is not installed or a run gives no figure."""
    import glob
    import shutil
    import subprocess
    import tempfile

    exe = shutil.which("rocprofv3")
    if exe is None:
        return None
    res = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="sage_pmc_", dir="/tmp")
        cmd = ["timeout", "-s", "KILL", "150", exe, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "p",
               "--", sys.executable, os.path.abspath(__file__), "--config", config, "--kernels-only",
               "--steps", str(steps)]
        log(f"[bench] traffic: rocprofv3 --pmc {counter} of bench.py --config {config} --kernels-only ...")
        env = dict(os.environ, TMPDIR="/tmp")
        with open(os.path.join(d, "run.log"), "w") as out:
            rc = subprocess.run(cmd, cwd="/tmp", env=env, stdout=out, stderr=subprocess.STDOUT).returncode
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        means = _counter_means(files[0], counter) if files else {}
        attn = [v for k, v in means.items() if k.replace(" ", "").startswith(f"attn_fwd_kernel<{D},3,")]
        # rocprofv3 can end with a fault of its own after the program and its results are complete (rc 139);
        # the figure is used whenever the results hold both kernels
        if not attn or not means.get("copy_1GiB"):
            log(f"[bench] traffic: no {counter} figure (rc {rc}; log in {d})")
            return None
        res[counter] = attn[0] * 1024.0 * ((1 << 30) / (means["copy_1GiB"] * 1024.0))
        shutil.rmtree(d, ignore_errors=True)
    return {"fetch_bytes": res["FETCH_SIZE"], "write_bytes": res["WRITE_SIZE"],
            "bytes": res["FETCH_SIZE"] + res["WRITE_SIZE"]}


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
        settle(fn)
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / n

    ms_kernel = timed_launches(lambda: ops.bf16_attn_t(q, k, vt, o, lay, int(causal), D ** -0.5, 0), n, stream, dev,
                               queue=False)
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
# benchmark_attn-result-native.txt; non-causal, h_q == h_kv, called with [b, s, h, d] tensors and
# tensor_layout="NHD", :213-215,271): name, B, H, Sq, Sk, D, dtype.  The reference's NHD dispatch sends the
# long self-attention shapes to the INT8 path and the short self-attention and cross-attention ones (kv 77,
# 154, 512; self-attention up to 3072 at D = 64, 2048 at D = 128) to the direct path.
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


def fp32_reference_nhd(q, k, v):
    """The reference benchmark's accuracy baseline (benchmark_attn.py:50-66): softmax attention in fp32 on
    [b, s, h, d] inputs, cast to the output dtype.  Computed per head in row blocks from contiguous fp32
    operands (plain matmuls, no half-precision batched products)."""
    import torch

    B, Sq, H, D = q.shape
    out = torch.empty_like(q)
    scale = D ** -0.5
    for b in range(B):
        for h in range(H):
            kh = k[b, :, h].float().contiguous()
            vh = v[b, :, h].float().contiguous()
            kt = kh.t().contiguous()
            for r0 in range(0, Sq, 4096):
                qh = q[b, r0:r0 + 4096, h].float().contiguous()
                p = torch.softmax((qh @ kt) * scale, dim=-1)
                out[b, r0:r0 + 4096, h] = (p @ vh).to(q.dtype)
    return out


def reference_shapes_probe(dev, n, names=None, modes=("auto", "1")):
    """Whole ``sageattn`` calls at the reference's benchmark shapes (``names``: a subset), called as its
    benchmark calls them: [b, s, h, d] tensors, tensor_layout="NHD", non-causal, so the reference's NHD
    dispatch picks the INT8 or the direct path.  Back to back on one stream, with the library's key-split
    plan and with splitting switched off (SAGEATTN_KV_SPLITS=1), the two modes alternating over three rounds
    (each reports its median round).  ``ms`` is the time per call as a caller sees it: for the smallest
    shapes the host's issue time per call, when it exceeds the GPU's.  MaxErr, MSE and CosSim are the
    reference benchmark's (benchmark_attn.py:50-66), over the whole output against fp32 attention cast to
    the output dtype; ``status`` is its FAIL rule (MaxErr > 0.05)."""
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
            g = torch.Generator().manual_seed(0)
            q = torch.randn((B, Sq, H, D), generator=g).to(dtype).to(dev)
            k = torch.randn((B, Sk, H, D), generator=g).to(dtype).to(dev)
            v = torch.randn((B, Sk, H, D), generator=g).to(dtype).to(dev)
            direct = use_direct_path(D, Sq, Sk, False, "NHD")
            calls = n if Sq * Sk >= 1 << 24 else max(n, 200)  # enough calls to time the short shapes
            times = {mode: [] for mode in modes}
            for _round in range(3):
                for mode in modes:
                    if mode == "auto":
                        os.environ.pop("SAGEATTN_KV_SPLITS", None)
                    else:
                        os.environ["SAGEATTN_KV_SPLITS"] = mode
                    settle(lambda: sageattn(q, k, v, tensor_layout="NHD", is_causal=False), SETTLE_MS / 3)
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(calls):
                        sageattn(q, k, v, tensor_layout="NHD", is_causal=False)
                    e1.record()
                    e1.synchronize()
                    times[mode].append(e0.elapsed_time(e1) / calls)
            res = {mode: sorted(t)[1] for mode, t in times.items()}
            os.environ.pop("SAGEATTN_KV_SPLITS", None)
            o = sageattn(q, k, v, tensor_layout="NHD", is_causal=False).float()
            ref = fp32_reference_nhd(q, k, v).float()
            max_err = (o - ref).abs().max().item()
            mse = ((o - ref) ** 2).mean().item()
            cos = torch.nn.functional.cosine_similarity(o.flatten(), ref.flatten(), dim=0).item()
            whole, splits = _capi.split_plan(not direct, B, H, Sq, Sk, D, False, 0)
            flops = attn_ops(B, H, Sq, Sk, D, False)
            row = {"shape": name, "B": B, "H": H, "Sq": Sq, "Sk": Sk, "D": D, "dtype": dt, "layout": "NHD",
                   "path": "direct" if direct else "int8", "plan": {"whole_qblocks": whole, "splits": splits},
                   "max_err": round(max_err, 6), "mse": float(f"{mse:.3e}"), "cos": round(cos, 6),
                   "status": "FAIL" if max_err > 0.05 else "OK"}
            if "auto" in res:
                row.update(ms=round(res["auto"], 4), tops=round(flops / (res["auto"] * 1e-3) / 1e12, 1))
            if "1" in res:
                row.update(ms_unsplit=round(res["1"], 4))
            out.append(row)
            log(f"[bench] {name} ({row['path']}): " +
                ", ".join(f"{'sageattn' if m == 'auto' else 'unsplit'} {t:.4f} ms" for m, t in res.items()) +
                f", plan {whole} whole + splits of {splits}; MaxErr {max_err:.6f} CosSim {cos:.6f}")
            del q, k, v, o, ref
    finally:
        if saved is None:
            os.environ.pop("SAGEATTN_KV_SPLITS", None)
        else:
            os.environ["SAGEATTN_KV_SPLITS"] = saved
    return out


def config_probe(name, dev, n):
    """One BASELINE config in the same run as the headline: the whole ``sageattn`` step, the attention kernel
    alone (Q quantised in the kernel, what ``sageattn`` launches) against the INT8 peak, and the prologue
    kernels (K quantisation + V layout in one launch, the K mean for smooth_k, the K-only quantisation)
    against HBM, each on its own rotating input set so that no launch finds its operands in the caches.
    A device copy of prep_kv's byte count (half read, half written) gives the copy ceiling at that size."""
    import torch

    from sageattention import ops, sageattn

    cfg = CONFIGS[name]
    B, Hq, Hkv, S, D, dt, layout, causal, smooth = cfg
    q, k, v = make_inputs(cfg, dev, name)
    lay = ops.HND if layout == "HND" else ops.NHD
    stream = torch.cuda.current_stream(dev)

    def timed(fn, calls, queue=True):
        return timed_launches(fn, calls, stream, dev, queue)

    ms_step = timed(lambda: sageattn(q, k, v, tensor_layout=layout, is_causal=causal, smooth_k=smooth), n,
                    queue=False)
    bd = step_breakdown(cfg, q, k, v, n, stream, queue=ms_step < 0.25)
    mean = ops.mean_seq(k, lay) if smooth else torch.empty(0, device=dev, dtype=q.dtype)
    k8, ks, vt = ops.prep_kv_int8(k, v, mean, lay)
    o = torch.empty_like(q)
    ms_attn = timed(lambda: ops.qk_int8_sv_bf16_attn_qfused_t(q, k8, vt, o, ks, lay, int(causal), D ** -0.5), n,
                    queue=D < 128)
    NROT = 3
    kr = [k] + [k.clone() for _ in range(NROT - 1)]
    vr = [v] + [v.clone() for _ in range(NROT - 1)]
    outs = [None] * NROT
    rot = [0]

    def rotated(fn):
        def call():
            i = rot[0] % NROT
            rot[0] += 1
            fn(i)
        return call

    ms_prep = timed(rotated(lambda i: outs.__setitem__(i, ops.prep_kv_int8(kr[i], vr[i], mean, lay))), n)
    ms_kq = timed(rotated(lambda i: outs.__setitem__(i, ops.quant_k_int8(kr[i], mean, lay))), n)
    ms_mean = timed(rotated(lambda i: ops.mean_seq(kr[i], lay)), n) if smooth else None
    ms_smooth = timed(rotated(lambda i: outs.__setitem__(i, ops.prep_kv_int8_smooth(kr[i], vr[i], lay))), n) \
        if smooth else None
    del kr, vr, outs
    ops_step = attn_ops(B, Hq, S, S, D, causal)
    nk = B * Hkv * S * D
    kq_bytes = 2 * nk + nk + 4 * B * Hkv * ((S + 15) // 16)
    vl_bytes = 2 * nk + 2 * B * Hkv * D * ((S + 63) // 64 * 64)
    mean_bytes = 2 * nk + 2 * B * Hkv * D
    # the copy ceiling at prep_kv's size: a device copy that reads and writes half of prep_kv's bytes each
    half = (kq_bytes + vl_bytes) // 2 // 16 * 16
    srcs = [torch.empty(half, device=dev, dtype=torch.uint8).fill_(1) for _ in range(NROT)]
    dsts = [torch.empty_like(x) for x in srcs]
    ms_copy = timed(rotated(lambda i: dsts[i].copy_(srcs[i])), n)
    del srcs, dsts
    ach = ops_step / (ms_attn * 1e-3) / 1e12
    r = {
        "workload": f"{name}: sageattn B{B} Hq{Hq} Hkv{Hkv} S{S} D{D} {dt} {layout} "
                    f"{'causal' if causal else 'non-causal'} smooth_k={smooth}",
        "step_ms": round(ms_step, 5),
        "effective_tops": round(ops_step / (ms_step * 1e-3) / 1e12, 2),
        "attn_kernel_ms": round(ms_attn, 5),
        "attn_frac_int8_peak": round(ach / PEAK_INT8_TOPS, 4),
        "prep_kv_us": round(ms_prep * 1e3, 2),
        "prep_kv_GBps": round((kq_bytes + vl_bytes) / ms_prep / 1e6, 1),
        "prep_kv_frac_hbm": round((kq_bytes + vl_bytes) / ms_prep / 1e6 / PEAK_HBM_GBS, 4),
        "copy_same_bytes_us": round(ms_copy * 1e3, 2),
        "copy_same_bytes_GBps": round(2 * half / ms_copy / 1e6, 1),
        "prep_kv_frac_of_copy": round(ms_copy / ms_prep, 4),
        "k_quant_us": round(ms_kq * 1e3, 2),
        "k_quant_GBps": round(kq_bytes / ms_kq / 1e6, 1),
        "k_quant_frac_hbm": round(kq_bytes / ms_kq / 1e6 / PEAK_HBM_GBS, 4),
        "k_mean_us": round(ms_mean * 1e3, 2) if smooth else None,
        "k_mean_GBps": round(mean_bytes / ms_mean / 1e6, 1) if smooth else None,
        "k_mean_frac_hbm": round(mean_bytes / ms_mean / 1e6 / PEAK_HBM_GBS, 4) if smooth else None,
        # smooth_k: the prologue sageattn runs (K mean's chunk sums, then K quantisation finishing the mean + V
        # layout), against the HBM bytes of the K mean read plus prep_kv's
        "prep_kv_smooth_us": round(ms_smooth * 1e3, 2) if smooth else None,
        "prep_kv_smooth_frac_hbm": round((mean_bytes + kq_bytes + vl_bytes) / ms_smooth / 1e6 / PEAK_HBM_GBS, 4)
        if smooth else None,
        "step_breakdown": dict(bd, unaccounted_us=round((ms_step - bd["sum_ms"]) * 1e3, 2)),
    }
    log(f"[bench] {name}: step {ms_step:.4f} ms ({r['effective_tops']} TOPS), attention {ms_attn:.4f} ms "
        f"({100 * r['attn_frac_int8_peak']:.1f}% INT8 peak), prep_kv {r['prep_kv_us']} us "
        f"({100 * r['prep_kv_frac_hbm']:.1f}% HBM; a copy of the same bytes {r['copy_same_bytes_us']} us = "
        f"{r['copy_same_bytes_GBps']} GB/s), K quant {r['k_quant_us']} us, K mean {r['k_mean_us']} us, smooth_k "
        f"prologue {r['prep_kv_smooth_us']} us; in-step prologue {bd['prologue_us']} us + attention "
        f"{bd['attention_ms']:.4f} ms + gap {bd['gap_between_steps_us']} us")
    del q, k, v, o, k8, ks, vt
    torch.cuda.empty_cache()
    return r


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="NS", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU oracle work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-traffic", action="store_true",
                    help="take roofline.traffic from the committed profile instead of two rocprofv3 --pmc child runs "
                         "(also skipped with --no-probes and when this process runs under rocprofv3)")
    ap.add_argument("--no-probes", action="store_true",
                    help="skip the direct-kernel, reference-shape and per-config probes (kernel traces of the NS "
                         "workload alone)")
    ap.add_argument("--configs", default="C2,C3,C4,C5", metavar="NAMES",
                    help="BASELINE configs timed after the headline (comma list, '' for none)")
    ap.add_argument("--skip", default="", metavar="PROBES",
                    help="comma list of probes to leave out: direct, reference (the reference benchmark shapes)")
    ap.add_argument("--reference-shapes", default=None, metavar="NAMES",
                    help="only time sageattn at these reference benchmark shapes (comma list, or 'all'), "
                         "print them as one JSON line and exit; for rocprofv3 runs of the split path")
    ap.add_argument("--reference-modes", default="auto,1", metavar="MODES",
                    help="with --reference-shapes: 'auto' (the library's key-split plan) and/or '1' (unsplit)")
    ap.add_argument("--kernels-only", action="store_true",
                    help="launch each path kernel and the direct kernel --steps times plus a 1 GiB device copy (the HBM-counter "
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

    q, k, v = make_inputs(cfg, dev, args.config)
    torch.cuda.synchronize()
    if args.kernels_only:
        kernels_only(cfg, q, k, v, args.steps)
        return

    lay = ops.HND if layout == "HND" else ops.NHD
    stream = torch.cuda.current_stream(dev)
    # ---- per-kernel timing with HIP events on the launch stream, back to back.  These probes run before
    # the headline steps: after the idle of the CPU input generation the GPU clock ramps up over its first
    # ~50 ms of work, which a short warm-up (the driver's W) does not cover; each probe settles first.
    mean = ops.mean_seq(k, lay) if smooth else torch.empty(0, device=dev, dtype=q.dtype)
    q8, qs, k8, ks = ops.quant_qk_int8(q, k, mean, lay, D ** -0.5)
    vt = torch.empty(B, Hkv, D, (S + 63) // 64 * 64, device=dev, dtype=torch.float16)
    ops.v_transpose(v, vt, lay)
    o = torch.empty_like(q)

    def timed(fn, n, queue=True, label=None):
        return timed_launches(fn, n, stream, dev, queue, label)

    n_k = max(args.steps, 10)
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
    ms_prep_smooth = (timed(rotated(lambda i: qouts.__setitem__(i, ops.prep_kv_int8_smooth(kr[i], vr[i], lay))), n_k)
                      if smooth else None)
    del qr, kr, vr, vtr, qouts
    # the attention kernel alone, last, so that the headline steps follow the same MFMA-bound work
    ms_attn_unfused = timed(lambda: ops.qk_int8_sv_bf16_attn_t(q8, k8, vt, o, qs, ks, lay, int(causal), D ** -0.5),
                            n_k, queue=False)
    ms_attn = timed(lambda: ops.qk_int8_sv_bf16_attn_qfused_t(q, k8, vt, o, ks, lay, int(causal), D ** -0.5), n_k,
                    queue=False, label="attention back-to-back loop")
    torch.cuda.synchronize()

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
    # the shader clock as sysfs reports it, over as many untimed steps right after: each read queries the SMU,
    # so no read runs beside the timed steps (kernel traces: the attention calls of steps timed beside the
    # sampler ran 1.7% slower than those of the in-step loop that followed, twice; without it 1.0%, once)
    sampler = SclkSampler(dev)
    with sampler:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    log(f"[bench] {args.steps} steps: {ms_step:.4f} ms/step, {value:.1f} effective TOPS; shader clock over as many "
        f"untimed steps after them (sysfs) {sampler.mhz()} MHz ({sampler.kind or 'not readable'}, "
        f"{len(sampler.samples)} samples)")

    # ---- the same steps' launches with HIP events between them (in-step kernel times)
    bd = step_breakdown(cfg, q, k, v, args.steps, stream, queue=ms_step < 0.25, label="in-step loop")
    bd["ms_per_step"] = round(ms_step, 5)
    bd["unaccounted_us"] = round((ms_step - bd["sum_ms"]) * 1e3, 2)
    log(f"[bench] in-step: prologue {bd['prologue_us']} us + attention {bd['attention_ms']:.4f} ms + gap "
        f"{bd['gap_between_steps_us']} us = {bd['sum_ms']:.4f} ms of GPU time; sageattn steps {ms_step:.4f} ms")

    # the roofline's kernel time: the attention kernel inside the steps (what ms_per_step contains)
    achieved = ops_step / (bd["attention_ms"] * 1e-3) / 1e12
    achieved_b2b = ops_step / (ms_attn * 1e-3) / 1e12
    nq, nk = B * Hq * S * D, B * Hkv * S * D
    quant_bytes = 2 * (nq + nk) + (nq + nk) + 4 * (B * Hq * ((S + 31) // 32) + B * Hkv * ((S + 15) // 16))
    kquant_bytes = 2 * nk + nk + 4 * B * Hkv * ((S + 15) // 16)
    vl_bytes = 2 * nk + 2 * B * Hkv * D * ((S + 63) // 64 * 64)
    mean_bytes = 2 * nk + 2 * B * Hkv * D
    mixed = 2.0 / (1.0 / PEAK_INT8_TOPS + 1.0 / PEAK_F16_TFLOPS)
    log(f"[bench] attn kernel in the steps {bd['attention_ms']:.4f} ms = {achieved:.1f} TOPS "
        f"({100 * achieved / PEAK_INT8_TOPS:.1f}% INT8 peak), back to back {ms_attn:.4f} ms; "
        f"(two-kernel path {ms_attn_unfused:.4f} ms); quant Q+K {ms_quant * 1e3:.1f} us = "
        f"{quant_bytes / ms_quant / 1e6:.0f} GB/s, K only {ms_kquant * 1e3:.1f} us; "
        f"v_layout {ms_vl * 1e3:.1f} us = {vl_bytes / ms_vl / 1e6:.0f} GB/s; K quant + V layout in one launch "
        f"{ms_prep * 1e3:.1f} us = {(kquant_bytes + vl_bytes) / ms_prep / 1e6:.0f} GB/s")

    del q8, qs, k8, ks, vt, o
    torch.cuda.empty_cache()
    skip = set(args.skip.split(",")) if args.skip else set()
    direct = None if args.no_probes or "direct" in skip else direct_probe(dev, n_k)
    configs = None
    if not args.no_probes and args.configs:
        configs = {name: config_probe(name, dev, n_k) for name in args.configs.split(",") if name}
    ref_shapes = None if args.no_probes or "reference" in skip else reference_shapes_probe(dev, n_k)

    # HBM bytes per attention launch, measured now by two rocprofv3 --pmc child runs (counters need runs of their
    # own); else the committed profile's figure of this workload, labelled as such
    alg_bytes = (2 * nq + nk + 2 * B * Hkv * D * ((S + 63) // 64 * 64) + 2 * nq
                 + 4 * B * Hkv * ((S + 15) // 16))  # bf16 Q, int8 K, fp16 V_T and k scales read, O written
    meas = None
    if not (args.no_traffic or args.no_probes or under_profiler()):
        meas = measure_traffic(args.config, D)
    traffic = None
    traffic_source = None
    traffic_parts = None
    if meas is not None:
        traffic = round(meas["bytes"])
        traffic_parts = {"fetch_bytes": round(meas["fetch_bytes"]), "write_bytes": round(meas["write_bytes"])}
        traffic_source = ("measured in this run: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (one run each) of bench.py "
                          "--kernels-only in a child process, each scaled by the same counter on a 1 GiB device copy")
        log(f"[bench] traffic: {traffic / 1e6:.1f} MB per attention launch ({traffic / alg_bytes:.2f}x the "
            f"{alg_bytes / 1e6:.1f} MB it must move)")
    else:
        tfile = os.path.join(REPO, "profiles", f"hbm_traffic_{args.config}.json")
        if os.path.exists(tfile):
            with open(tfile) as f:
                traffic = json.load(f).get("attn_bytes_per_launch")
            traffic_source = (f"profiles/hbm_traffic_{args.config}.json: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE "
                              f"of bench.py --kernels-only, each scaled by the same counter on a 1 GiB device copy "
                              f"(committed profile, not measured in this run)")

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (PyTorch CPU implementation) ...")
        cpu = cpu_baseline(cfg, args.cpu_budget)
        log(f"[bench] cpu {cpu['value']:.4g} TOPS on {cpu['cores']} threads")

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "before_warmup": "the per-kernel probes of the same tensors (prologue kernels, then the attention kernel, "
                         f"each run for {SETTLE_MS:.0f} ms before its timed launches): the W warmup steps follow "
                         "GPU work, not the idle of the CPU input generation, after which the clock ramps up over "
                         "~50 ms of work",
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic N(0,1) inputs generated on the CPU from torch.Generator().manual_seed(0) in fp32, cast "
                "and copied to the GPU before timing (C3: K plus a per-channel offset of std 2; C5: 1% of the "
                "channels of Q and K x20)",
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
            "traffic_source": traffic_source,
            "traffic_parts": traffic_parts,
            "algorithmic_bytes": alg_bytes,
            "traffic_over_algorithmic": round(traffic / alg_bytes, 3) if traffic else None,
            "kernel": "attn_fwd_kernel (int8 QK, Q quantised in the kernel)",
            "kernel_ms": bd["attention_ms"],
            "kernel_ms_source": "HIP events around the attention launch inside the steps (step_breakdown)",
            "kernel_ms_back_to_back": round(ms_attn, 5),
            "frac_back_to_back": round(achieved_b2b / PEAK_INT8_TOPS, 4),
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
            "prep_kv_smooth_us": round(ms_prep_smooth * 1e3, 2) if smooth else None,
        },
        "step_breakdown": bd,
        "direct": direct,
        "configs": configs,
        "reference_shapes": ref_shapes,
        "device": {"name": props.name, "cus": props.multi_processor_count,
                   "sclk_mhz_sysfs_untimed_steps": sampler.mhz(), "sclk_source": sampler.kind,
                   "peak_clock_assumed_mhz": 2400},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
