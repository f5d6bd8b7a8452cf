"""The fused-Q INT8 attention and the direct fp16 kernel with V read in place (sage_attn_i8_fwd_qfused_vrows,
sage_attn_direct_fwd_vrows; fp16 only) against the V_T paths they replace (v_transpose followed by
sage_attn_i8_fwd_qfused or sage_attn_direct_fwd, reference core.py:141-164,173-179,190-197): the P.V MFMAs see
the same fp16 V values in the same key order, so output and LSE must match bit for bit -- at the BASELINE fp16
configs (C2, C4 at full size), the reference's cross-attention lengths (77, 154, 512 keys), ragged and cross
lengths, GQA, both layouts, a strided V view, causal and non-causal, unsplit and key-split plans.  Every output
element starts as NaN (all must be written).  The V_T paths themselves are tied to the oracle by
test_gpu_parity, test_gpu_direct and test_gpu_product, and the in-place-V outputs are also held to the oracle's
rows directly (test_vrows_rows_match_oracle, test_direct_vrows_rows_match_oracle): within
    |gpu - oracle| <= ATOL + RTOL * |oracle|,  cos >= 0.99999   (fp16 out: ATOL 2e-3, RTOL 4e-3)
on the oracle's quantisation (INT8 kernel: the same q_int8 / k_int8 and scales bit for bit) and V_T."""
import numpy as np
import pytest
import torch

from oracle import sage_oracle as orc
from _helpers import C2, C4, Config, cos_sim, make_inputs, np_to_f32, sample_rows, to_np

pytestmark = pytest.mark.gpu

CASES = [
    C2,
    C4,
    Config("ragged1000_d128_causal_hnd", 1, 4, 2, 1000, 128, "fp16", "HND", True, False),
    Config("ragged300_d64_nhd", 2, 3, 3, 300, 64, "fp16", "NHD", False, False),
    Config("ragged1000_d64_causal_nhd", 1, 4, 4, 1000, 64, "fp16", "NHD", True, False),
    Config("cross_q300_kv1000_d128", 1, 4, 4, 1000, 128, "fp16", "HND", False, False, Sq=300),
    Config("cross_q1000_kv77_d64", 1, 2, 2, 77, 64, "fp16", "NHD", False, False, Sq=1000),
    Config("gqa_d64_nhd_2304", 1, 20, 5, 2304, 64, "fp16", "NHD", False, False),
    Config("persistent_causal_d128", 1, 8, 8, 9000, 128, "fp16", "HND", True, False),
]


def _say(*a):
    print(*a, flush=True)


def _run(cfg, q, k, v, splits, v_strided=False):
    from sageattention import ops

    lay = ops.HND if cfg.layout == "HND" else ops.NHD
    k8, ks = ops.quant_k_int8(k, torch.empty(0, device="cuda", dtype=k.dtype), lay)
    vt = torch.empty(cfg.B, cfg.Hkv, cfg.D, (cfg.S + 63) // 64 * 64, device="cuda", dtype=torch.float16)
    ops.v_transpose(v, vt, lay)
    nan = float("nan")
    o_ref = torch.full_like(q, nan)
    lse_ref = torch.full((cfg.B, cfg.Hq, cfg.q_len), nan, device="cuda", dtype=torch.float32)
    ops.qk_int8_sv_bf16_attn_qfused_t(q, k8, vt, o_ref, ks, lay, int(cfg.causal), cfg.D ** -0.5, lse=lse_ref,
                                      num_splits=splits)
    if v_strided:
        # the same V values in a wider buffer: rows 2*D apart (HND) / heads 2*D apart (NHD)
        wide = torch.zeros(v.shape[:-1] + (2 * cfg.D,), device="cuda", dtype=v.dtype)
        wide[..., cfg.D // 2: cfg.D // 2 + cfg.D] = v
        v = wide[..., cfg.D // 2: cfg.D // 2 + cfg.D]
        assert not v.is_contiguous()
    o = torch.full_like(q, nan)
    lse = torch.full((cfg.B, cfg.Hq, cfg.q_len), nan, device="cuda", dtype=torch.float32)
    ops.qk_int8_sv_f16_attn_qfused_vrows(q, k8, v, o, ks, lay, int(cfg.causal), cfg.D ** -0.5, lse=lse,
                                         num_splits=splits)
    torch.cuda.synchronize()
    return o_ref, lse_ref, o, lse


@pytest.mark.parametrize("cfg", CASES, ids=lambda c: c.name)
@pytest.mark.parametrize("splits", [0, 1, 3])
def test_vrows_equals_vt_path(cfg, splits):
    if cfg.S >= 16384 and splits == 3:
        pytest.skip("causal full-size config: num_splits is ignored (covered by splits 0 and 1)")
    _say(f"[vrows] {cfg} splits={splits}")
    q, k, v = (t.cuda() for t in make_inputs(cfg, seed=5))
    o_ref, lse_ref, o, lse = _run(cfg, q, k, v, splits)
    assert not bool(torch.isnan(o).any()), f"{int(torch.isnan(o).sum())} output elements unwritten"
    assert bool(torch.isfinite(lse).all()), "LSE element left unwritten"
    assert torch.equal(o, o_ref), f"max diff {(o.float() - o_ref.float()).abs().max().item()}"
    assert torch.equal(lse, lse_ref)


ATOL, RTOL = 2e-3, 4e-3  # fp16 output


def _hold_rows(cfg, o_gpu, ref_fn, rows):
    og = orc.to_hnd(np_to_f32(to_np(o_gpu), "fp16"), cfg.layout)
    worst = 0.0
    for b in range(cfg.B):
        for h in range(cfg.Hq):
            ref = np_to_f32(orc.from_f32(ref_fn(b, h).astype(np.float32), "fp16"), "fp16")
            got = og[b, h, rows]
            err = np.abs(got.astype(np.float64) - ref)
            lim = ATOL + RTOL * np.abs(ref)
            if not np.all(err <= lim):
                i = np.unravel_index(np.argmax(err - lim), err.shape)
                raise AssertionError(f"b={b} h={h} row={rows[i[0]]} d={i[1]}: gpu={got[i]} oracle={ref[i]}")
            assert cos_sim(got, ref) >= 0.99999
            worst = max(worst, float(err.max()))
    return worst


@pytest.mark.parametrize("cfg", [CASES[0], CASES[2], CASES[5], CASES[7]], ids=lambda c: c.name)
def test_vrows_rows_match_oracle(cfg):
    """sage_attn_i8_fwd_qfused_vrows held to the oracle's INT8 attention rows (oracle quantisation of Q and K,
    oracle V_T), with the library's key-split plan."""
    _say(f"[vrows vs oracle] {cfg}")
    q, k, v = make_inputs(cfg, seed=5)
    _, _, o, _ = _run(cfg, q.cuda(), k.cuda(), v.cuda(), 0)
    q8, qs, k8, ks = orc.quant_qk_int8(to_np(q), to_np(k), "fp16", cfg.layout, cfg.D ** -0.5)
    vt = orc.v_layout(to_np(v), "fp16", cfg.layout)
    rows = sample_rows(cfg.q_len, 48, np.random.default_rng(3))
    worst = _hold_rows(cfg, o, lambda b, h: orc.attn_i8_rows(q8, k8, vt, qs, ks, b, h, rows, cfg.causal), rows)
    _say(f"  worst |gpu-oracle| = {worst:.3g}")


@pytest.mark.parametrize("cfg", [CASES[2], CASES[3]], ids=lambda c: c.name)
def test_vrows_strided_value(cfg):
    _say(f"[vrows strided V] {cfg}")
    q, k, v = (t.cuda() for t in make_inputs(cfg, seed=6))
    o_ref, lse_ref, o, lse = _run(cfg, q, k, v, 0, v_strided=True)
    assert torch.equal(o, o_ref)
    assert torch.equal(lse, lse_ref)


# ------------------------------------------------------------------ the direct (fp16) kernel with V in place
DIRECT_CASES = [
    Config("dv_cross_q1000_kv77_d64_nhd", 1, 10, 10, 77, 64, "fp16", "NHD", False, False, Sq=1000),
    Config("dv_cross_q700_kv154_d64", 1, 4, 4, 154, 64, "fp16", "HND", False, False, Sq=700),
    Config("dv_2304_d64_nhd", 1, 20, 20, 2304, 64, "fp16", "NHD", False, False),
    Config("dv_ragged1000_d128_causal_gqa", 1, 4, 2, 1000, 128, "fp16", "HND", True, False),
    Config("dv_ragged300_d128_nhd_gqa", 2, 6, 3, 300, 128, "fp16", "NHD", False, False),
    Config("dv_cross_q300_kv512_d128_nhd", 1, 16, 16, 512, 128, "fp16", "NHD", False, False, Sq=300),
    Config("dv_persistent_causal_d64", 1, 8, 8, 9000, 64, "fp16", "HND", True, False),
]


def _run_direct(cfg, q, k, v, splits, v_strided=False):
    from sageattention import ops

    lay = ops.HND if cfg.layout == "HND" else ops.NHD
    vt = torch.empty(cfg.B, cfg.Hkv, cfg.D, (cfg.S + 63) // 64 * 64, device="cuda", dtype=torch.float16)
    ops.v_transpose(v, vt, lay)
    nan = float("nan")
    o_ref = torch.full_like(q, nan)
    lse_ref = torch.full((cfg.B, cfg.Hq, cfg.q_len), nan, device="cuda", dtype=torch.float32)
    ops.fp16_attn_t(q, k, vt, o_ref, lay, int(cfg.causal), cfg.D ** -0.5, 0, lse=lse_ref, num_splits=splits)
    if v_strided:
        wide = torch.zeros(v.shape[:-1] + (2 * cfg.D,), device="cuda", dtype=v.dtype)
        wide[..., cfg.D // 2: cfg.D // 2 + cfg.D] = v
        v = wide[..., cfg.D // 2: cfg.D // 2 + cfg.D]
        assert not v.is_contiguous()
    o = torch.full_like(q, nan)
    lse = torch.full((cfg.B, cfg.Hq, cfg.q_len), nan, device="cuda", dtype=torch.float32)
    ops.fp16_attn_vrows(q, k, v, o, lay, int(cfg.causal), cfg.D ** -0.5, lse=lse, num_splits=splits)
    torch.cuda.synchronize()
    return o_ref, lse_ref, o, lse


@pytest.mark.parametrize("cfg", DIRECT_CASES, ids=lambda c: c.name)
@pytest.mark.parametrize("splits", [0, 1, 3])
def test_direct_vrows_equals_vt_path(cfg, splits):
    """sage_attn_direct_fwd_vrows against v_transpose + sage_attn_direct_fwd (reference core.py:141-164):
    output and LSE bit for bit, every element written."""
    _say(f"[direct vrows] {cfg} splits={splits}")
    q, k, v = (t.cuda() for t in make_inputs(cfg, seed=7))
    o_ref, lse_ref, o, lse = _run_direct(cfg, q, k, v, splits)
    assert not bool(torch.isnan(o).any()), f"{int(torch.isnan(o).sum())} output elements unwritten"
    assert bool(torch.isfinite(lse).all()), "LSE element left unwritten"
    assert torch.equal(o, o_ref), f"max diff {(o.float() - o_ref.float()).abs().max().item()}"
    assert torch.equal(lse, lse_ref)


@pytest.mark.parametrize("cfg", [DIRECT_CASES[0], DIRECT_CASES[3], DIRECT_CASES[5]], ids=lambda c: c.name)
def test_direct_vrows_rows_match_oracle(cfg):
    """sage_attn_direct_fwd_vrows held to the oracle's direct attention rows (fp16 Q/K in place, oracle V_T)."""
    _say(f"[direct vrows vs oracle] {cfg}")
    q, k, v = make_inputs(cfg, seed=7)
    _, _, o, _ = _run_direct(cfg, q.cuda(), k.cuda(), v.cuda(), 0)
    q32 = orc.to_f32(orc.to_hnd(to_np(q), cfg.layout), "fp16")
    k32 = orc.to_f32(orc.to_hnd(to_np(k), cfg.layout), "fp16")
    vt = orc.v_layout(to_np(v), "fp16", cfg.layout)
    rows = sample_rows(cfg.q_len, 48, np.random.default_rng(4))
    worst = _hold_rows(cfg, o, lambda b, h: orc.attn_direct_rows(q32, k32, vt, cfg.D ** -0.5, b, h, rows, cfg.causal),
                       rows)
    _say(f"  worst |gpu-oracle| = {worst:.3g}")


@pytest.mark.parametrize("cfg", [DIRECT_CASES[0], DIRECT_CASES[3]], ids=lambda c: c.name)
def test_direct_vrows_strided_value(cfg):
    _say(f"[direct vrows strided V] {cfg}")
    q, k, v = (t.cuda() for t in make_inputs(cfg, seed=8))
    o_ref, lse_ref, o, lse = _run_direct(cfg, q, k, v, 0, v_strided=True)
    assert torch.equal(o, o_ref)
    assert torch.equal(lse, lse_ref)
