"""A seeded sweep of random shapes through ``sageattn``, the product entry, which chooses the path
(direct or INT8), the prologue, the launch plan and the block shape by itself, against the CPU oracle.

The shapes are drawn once from a fixed seed, so the sweep is the same on every run. They reach the
launch plans a fixed list reaches only by chance:
- odd lengths (tails of the 16/32-row scale groups and of the 64-key tiles);
- fewer or more queries than keys;
- grouped heads, batches, both layouts and both dtypes, smooth_k;
- causal launches of every size class (128-row blocks, the paired persistent schedule, whole rounds);
- non-causal launches with and without key splits.

Half of the cases switch the direct path off through the reference's threshold variables, so that the
INT8 path runs at short lengths too. Each case checks the following:
- the output has q's shape and dtype and holds no NaN or inf;
- the first and last head of the first and last batch, on sampled rows, agree with the oracle's rows of
  the path the reference's dispatch picks, in the parity tests' tolerance
  (|gpu - oracle| <= ATOL + RTOL |oracle|, cos >= 0.99999);
- the LSE of those rows agrees within 2e-4 + 2e-6 |oracle|.
"""
import numpy as np
import pytest
import torch

from oracle import sage_oracle as orc
from _helpers import Config, cos_sim, make_inputs, np_to_f32, sample_rows, to_np

pytestmark = pytest.mark.gpu

TOL = {"fp16": (2e-3, 4e-3), "bf16": (4e-3, 1.6e-2)}
DIRECT_ENV = ["SAGEATTN_DIRECT_THRESHOLD_D64", "SAGEATTN_DIRECT_THRESHOLD_D64_CAUSAL",
              "SAGEATTN_DIRECT_THRESHOLD_D64_CROSS", "SAGEATTN_DIRECT_THRESHOLD_D128",
              "SAGEATTN_DIRECT_THRESHOLD_D128_CROSS"]
# B * Hq * the longer length: keeps the oracle's CPU quantisation of each case to about a second
BUDGET = 96_000


def draw_cases(n=40, seed=20261202):
    """(Config, forced INT8 path) pairs from a fixed seed."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = int(rng.choice([64, 128]))
        dtype = str(rng.choice(["fp16", "bf16"]))
        layout = str(rng.choice(["HND", "NHD"]))
        causal = bool(rng.random() < 0.5)
        smooth = bool(rng.random() < 0.3)
        B = int(rng.choice([1, 1, 1, 2, 3]))
        Hkv = int(rng.choice([1, 2, 4, 8]))
        Hq = Hkv * int(rng.choice([1, 1, 2, 4]))
        S = int(rng.integers(1, 5000))
        Sq = S if rng.random() < 0.6 else int(rng.integers(1, 5000))
        while B * Hq * max(S, Sq) > BUDGET:
            if Hq > Hkv:
                Hq //= 2
            elif Hkv > 1:
                Hkv //= 2
                Hq = Hkv
            elif B > 1:
                B -= 1
            else:
                S, Sq = max(1, S // 2), max(1, Sq // 2)
        force_i8 = bool(rng.random() < 0.5)
        name = (f"r{i:02d}_B{B}H{Hq}k{Hkv}q{Sq}kv{S}D{D}_{dtype}_{layout}{'_c' if causal else ''}"
                f"{'_sm' if smooth else ''}{'_i8' if force_i8 else ''}")
        cases.append((Config(name, B, Hq, Hkv, S, D, dtype, layout, causal, smooth,
                             Sq=None if Sq == S else Sq), force_i8))
    return cases


CASES = draw_cases()


@pytest.mark.parametrize("cfg,force_i8", CASES, ids=[c.name for c, _ in CASES])
def test_random_shape_through_sageattn(cfg, force_i8, monkeypatch):
    from sageattention import _capi, sageattn

    for name in DIRECT_ENV:
        if force_i8:
            monkeypatch.setenv(name, "-1")
        else:
            monkeypatch.delenv(name, raising=False)
    direct = orc.use_direct_path(cfg.D, cfg.q_len, cfg.S, cfg.causal, cfg.layout)
    plan = _capi.split_plan(not direct, cfg.B, cfg.Hq, cfg.q_len, cfg.S, cfg.D, cfg.causal, 0)
    print(f"[random] {cfg.name} path={'direct' if direct else 'int8'} plan={plan}", flush=True)

    idx = int(cfg.name[1:3])
    q, k, v = make_inputs(cfg, seed=100 + idx)
    o, lse = sageattn(q.cuda(), k.cuda(), v.cuda(), tensor_layout=cfg.layout, is_causal=cfg.causal,
                      return_lse=True, smooth_k=cfg.smooth_k)
    torch.cuda.synchronize()
    assert o.shape == q.shape and o.dtype == q.dtype
    assert bool(torch.isfinite(o).all()) and bool(torch.isfinite(lse).all())

    dt, sm = cfg.dtype, cfg.D ** -0.5
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    vt = orc.v_layout(vn, dt, cfg.layout)
    if direct:
        q32 = orc.to_f32(orc.to_hnd(qn, cfg.layout), dt)
        k32 = orc.to_f32(orc.to_hnd(kn, cfg.layout), dt)

        def ref_rows(b, h, rows):
            return orc.attn_direct_rows(q32, k32, vt, sm, b, h, rows, cfg.causal)

        def ref_lse(b, h, rows):
            return orc.attn_direct_lse_rows(q32, k32, sm, b, h, rows, cfg.causal)
    else:
        mean = orc.k_mean(kn, dt, cfg.layout) if cfg.smooth_k else None
        q8, qs, k8, ks = orc.quant_qk_int8(qn, kn, dt, cfg.layout, sm, k_mean=mean)

        def ref_rows(b, h, rows):
            return orc.attn_i8_rows(q8, k8, vt, qs, ks, b, h, rows, cfg.causal)

        def ref_lse(b, h, rows):
            return orc.attn_i8_lse_rows(q8, k8, qs, ks, b, h, rows, cfg.causal)

    og = orc.to_hnd(np_to_f32(to_np(o), dt), cfg.layout)
    lg = to_np(lse).astype(np.float64)
    rows = sample_rows(cfg.q_len, 8, np.random.default_rng(idx))
    atol, rtol = TOL[dt]
    for b in sorted({0, cfg.B - 1}):
        for h in sorted({0, cfg.Hq - 1}):
            ref = np_to_f32(orc.from_f32(ref_rows(b, h, rows).astype(np.float32), dt), dt)
            got = og[b, h, rows]
            err = np.abs(got.astype(np.float64) - ref)
            lim = atol + rtol * np.abs(ref)
            if not np.all(err <= lim):
                i = np.unravel_index(np.argmax(err - lim), err.shape)
                raise AssertionError(f"b={b} h={h} row={rows[i[0]]} d={i[1]}: gpu={got[i]} oracle={ref[i]}")
            assert cos_sim(got, ref) >= 0.99999
            want = ref_lse(b, h, rows)
            lerr = np.abs(lg[b, h, rows] - want)
            assert np.all(lerr <= 2e-4 + 2e-6 * np.abs(want)), f"b={b} h={h}: LSE worst {lerr.max():.3g}"
