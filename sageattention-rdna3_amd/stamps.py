"""Per-wave cycle stamps of the attention kernel (the library built with ``build.py --stamps``).

Usage (GPU): ``python sageattention-rdna3_amd/stamps.py NS [C3 C4 C5 C2 ...]``.  For each BASELINE config
of ``bench.py`` (same synthetic inputs) it runs the fused-Q INT8 attention that ``sageattn`` launches
(``qk_int8_sv_bf16_attn_qfused_t``) three times, clears the stamps, runs it once more and prints one JSON
line of per-wave averages, in s_memtime cycles (the shader clock: divide by the clock for time):

* ``fast_step`` / ``masked_step``: cycles from one step's start to the next (two waves share a SIMD, so
  a SIMD runs two such steps in that time); ``*_wait``: the part spent in the step's load wait and
  block barrier; ``fast_wait_by_wave``: the barrier wait of each wave index of a block;
* ``prologue`` (item start to its first step; ``prologue_loads``, ``_quant``, ``_scan``, ``_barrier``
  are its parts up to the prologue barrier, and ``prologue_q_issue`` / ``_tile_issue`` the parts of
  ``prologue_loads`` that issue the Q loads and the tile and k-scale loads), ``epilogue`` (last step
  to item end, including ``last_wait``), per item;
* ``share``: fractions of the waves' kernel time in unmasked steps, masked steps, prologues and
  epilogues; ``redo_per_wave``: tiles redone after the lazy-max sum test fired.
"""
from __future__ import annotations

import ctypes
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
STAMPS_LIB = os.path.join(HERE, "_build_stamps", "libsage_mi355x_stamps.so")
FIELDS = ["items", "fast", "masked", "fast_cycles", "fast_wait", "masked_cycles", "masked_wait", "prologue",
          "epilogue", "start", "end", "redo", "last_wait", "pro_loads", "pro_quant", "pro_scan", "pro_barrier",
          "pro_q_issue", "pro_tile_issue"]
STRIDE = 32       # uint64 fields per wave record (kStampStride)
RECORDS = 2048 * 8


def main(names):
    if not os.path.exists(STAMPS_LIB):
        raise SystemExit(f"{STAMPS_LIB} not built: python sageattention-rdna3_amd/build.py --stamps")
    os.environ["SAGEATTN_MI355X_LIB"] = STAMPS_LIB
    sys.path[:0] = [REPO, HERE]
    import numpy as np
    import torch

    import bench
    from sageattention import ops

    lib = ctypes.CDLL(STAMPS_LIB)
    dev = torch.device("cuda:0")
    for name in names:
        B, Hq, Hkv, S, D, dt, layout, causal, smooth = cfg = bench.CONFIGS[name]
        q, k, v = bench.make_inputs(cfg, dev, name)
        lay = ops.HND if layout == "HND" else ops.NHD
        mean = ops.mean_seq(k, lay) if smooth else torch.empty(0, device=dev, dtype=q.dtype)
        k8, ks, vt = ops.prep_kv_int8(k, v, mean, lay)
        o = torch.empty_like(q)

        def run():
            ops.qk_int8_sv_bf16_attn_qfused_t(q, k8, vt, o, ks, lay, int(causal), D ** -0.5)

        for _ in range(3):
            run()
        torch.cuda.synchronize()
        assert lib.sage_stamps_clear() == 0
        run()
        torch.cuda.synchronize()
        buf = np.zeros(RECORDS * STRIDE, dtype=np.uint64)
        assert lib.sage_stamps_read(buf.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(buf.nbytes)) == 0
        rec = buf.reshape(RECORDS, STRIDE)[:, :len(FIELDS)].astype(np.float64)
        waves_per_block = 4 if (D == 64 and not causal) else 8
        live = np.nonzero(rec[:, 0] > 0)[0]
        r = {f: rec[live, i] for i, f in enumerate(FIELDS)}
        wave_time = r["end"] - r["start"]
        per = lambda a, b: round(float(a.sum() / max(b.sum(), 1.0)), 1)
        items = r["items"]
        widx = live % 8
        out = {
            "config": name, "waves": int(len(live)),
            "fast_step": per(r["fast_cycles"], r["fast"]), "fast_wait": per(r["fast_wait"], r["fast"]),
            "masked_step": per(r["masked_cycles"], r["masked"]), "masked_wait": per(r["masked_wait"], r["masked"]),
            "fast_steps_per_wave": round(float(r["fast"].mean()), 1),
            "masked_steps_per_wave": round(float(r["masked"].mean()), 1),
            "items_per_wave": round(float(items.mean()), 2),
            "prologue": per(r["prologue"], items), "prologue_loads": per(r["pro_loads"], items),
            "prologue_quant": per(r["pro_quant"], items), "prologue_scan": per(r["pro_scan"], items),
            "prologue_barrier": per(r["pro_barrier"], items),
            "prologue_q_issue": per(r["pro_q_issue"], items), "prologue_tile_issue": per(r["pro_tile_issue"], items),
            "epilogue": per(r["epilogue"], items), "last_wait": per(r["last_wait"], items),
            "redo_per_wave": round(float(r["redo"].mean()), 2),
            "wave_cycles_mean": round(float(wave_time.mean())),
            "share": {k_: round(float(r[k_].sum() / wave_time.sum()), 4)
                      for k_ in ("fast_cycles", "masked_cycles", "prologue", "epilogue")},
        }
        if waves_per_block == 8:
            out["fast_wait_by_wave"] = [per(r["fast_wait"][widx == w], r["fast"][widx == w]) for w in range(8)]
        print(json.dumps(out), flush=True)
        del q, k, v, k8, ks, vt, o


if __name__ == "__main__":
    main(sys.argv[1:] or ["NS"])
