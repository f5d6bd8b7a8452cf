"""GPU parity of the direct (unquantised) fp16/bf16 attention kernel against the CPU oracle, through
the ops layer and the C ABI (``sage_attn_direct_fwd``).

The direct kernel reads Q and K in place (fp16 or bf16, any 16-byte-aligned strides) and the fp16
V_T of ``v_transpose``.  Its output is compared with ``oracle.attn_direct_rows`` on the same inputs
within the parity bar of the INT8 kernel,
    |gpu - oracle| <= ATOL + RTOL * |oracle|,  cos >= 0.99999
(fp16 out: ATOL 2e-3, RTOL 4e-3; bf16 out: ATOL 4e-3, RTOL 1.6e-2), and, being unquantised, with
fp32 SDPA within cos >= 0.99999.  The LSE is held to 2e-4 + 2e-6 |oracle|.
"""
import numpy as np
import pytest
import torch

from oracle import sage_oracle as orc
from _helpers import Config, cos_sim, make_inputs, max_abs, np_to_f32, sample_rows, sdpa_rows_fp32, to_np

pytestmark = pytest.mark.gpu

TOL = {"fp16": (2e-3, 4e-3), "bf16": (4e-3, 1.6e-2)}


def _say(*a):
    print(*a, flush=True)


def gpu_direct(cfg: Config, q, k, v, sm_scale=None, with_lse=False):
    """Direct attention on device copies of q, k, v (layout of cfg) -> (out, lse or None)."""
    from sageattention import ops

    lay = ops.HND if cfg.layout == "HND" else ops.NHD
    qd, kd, vd = (t.cuda() if not t.is_cuda else t for t in (q, k, v))
    B = qd.shape[0]
    Hkv = kd.shape[1] if cfg.layout == "HND" else kd.shape[2]
    Sk = kd.shape[2] if cfg.layout == "HND" else kd.shape[1]
    NP = (Sk + 63) // 64 * 64
    vt = torch.empty(B, Hkv, cfg.D, NP, device="cuda", dtype=torch.float16)
    ops.v_transpose(vd, vt, lay)
    o = torch.empty(qd.shape, device="cuda", dtype=qd.dtype)
    Hq = qd.shape[1] if cfg.layout == "HND" else qd.shape[2]
    Sq = qd.shape[2] if cfg.layout == "HND" else qd.shape[1]
    lse = torch.empty((B, Hq, Sq), device="cuda", dtype=torch.float32) if with_lse else None
    fn = ops.bf16_attn_t if qd.dtype == torch.bfloat16 else ops.fp16_attn_t
    sm = cfg.D ** -0.5 if sm_scale is None else sm_scale
    fn(qd, kd, vt, o, lay, int(cfg.causal), sm, 0, lse=lse)
    torch.cuda.synchronize()
    return o, lse, vt


def check_direct_rows(cfg, q, k, vt, o_gpu, heads, rows, sm_scale):
    dt = cfg.dtype
    q32 = orc.to_f32(orc.to_hnd(to_np(q), cfg.layout), dt)
    k32 = orc.to_f32(orc.to_hnd(to_np(k), cfg.layout), dt)
    vtn = to_np(vt)
    og = orc.to_hnd(np_to_f32(to_np(o_gpu), dt), cfg.layout)
    atol, rtol = TOL[dt]
    worst = 0.0
    for b in range(q32.shape[0]):
        for h in heads:
            ref = orc.attn_direct_rows(q32, k32, vtn, sm_scale, b, h, rows, cfg.causal)
            ref = np_to_f32(orc.from_f32(ref.astype(np.float32), dt), dt)
            got = og[b, h, rows]
            err = np.abs(got.astype(np.float64) - ref)
            lim = atol + rtol * np.abs(ref)
            if not np.all(err <= lim):
                i = np.unravel_index(np.argmax(err - lim), err.shape)
                raise AssertionError(f"b={b} h={h} row={rows[i[0]]} d={i[1]}: gpu={got[i]} oracle={ref[i]}")
            assert cos_sim(got, ref) >= 0.99999
            worst = max(worst, float(err.max()))
    return worst


DIRECT_SMALL = [
    Config("d64_fp16", 1, 2, 2, 256, 64, "fp16", "HND", False, False),
    Config("d128_bf16_causal", 2, 4, 4, 300, 128, "bf16", "HND", True, False),
    Config("d64_nhd_gqa", 1, 8, 2, 1057, 64, "fp16", "NHD", False, False),
    Config("d128_nhd_gqa_causal", 1, 4, 1, 129, 128, "bf16", "NHD", True, False),
    Config("d64_tiny", 1, 3, 3, 1, 64, "fp16", "HND", False, False),
    Config("d128_17", 1, 2, 2, 17, 128, "fp16", "HND", True, False),
    Config("d64_33_causal_bf16", 2, 2, 1, 33, 64, "bf16", "HND", True, False),
    Config("d128_255_nhd", 1, 2, 2, 255, 128, "fp16", "NHD", False, False),
    Config("cross_q40_kv150", 1, 2, 2, 150, 64, "fp16", "HND", False, False, Sq=40),
    Config("cross_q300_kv77_causal", 1, 2, 2, 77, 128, "bf16", "HND", True, False, Sq=300),
    Config("d128_koffset", 1, 2, 2, 513, 128, "bf16", "HND", False, False, k_offset_std=2.0),
]


@pytest.mark.parametrize("cfg", DIRECT_SMALL, ids=lambda c: c.name)
def test_direct_small_full_parity(cfg):
    _say(f"[direct small] {cfg}")
    q, k, v = make_inputs(cfg, seed=11)
    o, _, vt = gpu_direct(cfg, q, k, v)
    worst = check_direct_rows(cfg, q, k, vt, o, range(cfg.Hq), np.arange(cfg.q_len), cfg.D ** -0.5)
    _say(f"  worst |gpu-oracle| = {worst:.3g}")


@pytest.mark.parametrize("sm_scale", [0.5, -0.125, 0.0])
def test_direct_sm_scale_values(sm_scale):
    """Any fp32 scale, including a negative one (applied through Q's sign bits) and zero (uniform
    weights over the live keys)."""
    cfg = Config("scale", 1, 2, 2, 200, 64, "fp16", "HND", True, False)
    _say(f"[direct scale {sm_scale}] {cfg}")
    q, k, v = make_inputs(cfg, seed=12)
    o, _, vt = gpu_direct(cfg, q, k, v, sm_scale=sm_scale)
    check_direct_rows(cfg, q, k, vt, o, range(cfg.Hq), np.arange(cfg.q_len), sm_scale)


def test_direct_strided_views_of_packed_qkv():
    """Q, K, V as views of one packed [B, S, 3, H, D] tensor (NHD, token stride 3*H*D), and HND
    views with a padded token stride: read in place, same result as contiguous copies."""
    B, S, H, D = 2, 333, 4, 128
    g = torch.Generator().manual_seed(13)
    qkv = torch.randn(B, S, 3, H, D, generator=g).to(torch.bfloat16).cuda()
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    cfg = Config("packed", B, H, H, S, D, "bf16", "NHD", True, False)
    o, _, vt = gpu_direct(cfg, q, k, v)
    oc, _, _ = gpu_direct(cfg, q.contiguous(), k.contiguous(), v.contiguous())
    assert torch.equal(o, oc)
    check_direct_rows(cfg, q, k, vt, o, range(H), np.arange(S), D ** -0.5)
    # HND with token stride D + 64 (rows padded), K only
    big = torch.randn(1, 2, 100, 192, generator=g).to(torch.float16).cuda()
    kp = big[..., :128]
    qc = torch.randn(1, 2, 100, 128, generator=g).to(torch.float16).cuda()
    vc = torch.randn(1, 2, 100, 128, generator=g).to(torch.float16).cuda()
    cfg2 = Config("padK", 1, 2, 2, 100, 128, "fp16", "HND", False, False)
    o1, _, _ = gpu_direct(cfg2, qc, kp, vc)
    o2, _, _ = gpu_direct(cfg2, qc, kp.contiguous(), vc)
    assert torch.equal(o1, o2)


@pytest.mark.parametrize("cfg", [
    Config("d128_2048_causal", 1, 8, 8, 2048, 128, "bf16", "HND", True, False),
    Config("d64_6144_causal_nhd", 1, 4, 4, 6144, 64, "fp16", "NHD", True, False),
    Config("d128_cross_q1024_kv4096", 1, 4, 2, 4096, 128, "fp16", "HND", False, False, Sq=1024),
], ids=lambda c: c.name)
def test_direct_dispatch_range_sampled_rows(cfg):
    """The largest shapes the reference's dispatch sends to the direct kernel: sampled rows against
    the oracle, and every sampled row against fp32 SDPA."""
    _say(f"[direct range] {cfg}")
    q, k, v = make_inputs(cfg, seed=14)
    o, _, vt = gpu_direct(cfg, q, k, v)
    rng = np.random.default_rng(0)
    rows = sample_rows(cfg.q_len, 48, rng)
    heads = sorted({0, cfg.Hq - 1})
    worst = check_direct_rows(cfg, q, k, vt, o, heads, rows, cfg.D ** -0.5)
    qh, kh, vh = (orc.to_hnd(np_to_f32(to_np(t), cfg.dtype), cfg.layout) for t in (q, k, v))
    og = orc.to_hnd(np_to_f32(to_np(o), cfg.dtype), cfg.layout)
    G = cfg.Hq // cfg.Hkv
    for h in heads:
        ref = sdpa_rows_fp32(qh[0, h], kh[0, h // G], vh[0, h // G], rows, cfg.causal, cfg.D ** -0.5)
        assert cos_sim(og[0, h, rows], ref) >= 0.99999
        assert max_abs(og[0, h, rows], ref) <= (1e-2 if cfg.dtype == "bf16" else 3e-3)
    _say(f"  worst |gpu-oracle| = {worst:.3g}")


@pytest.mark.parametrize("cfg", [
    Config("paired_b1h32_s2048", 1, 32, 32, 2048, 128, "bf16", "HND", True, False),
    Config("paired_b2h16_s2048_nhd_gqa", 2, 16, 4, 2048, 128, "fp16", "NHD", True, False),
    Config("paired_d64_b1h32_s2048", 1, 32, 32, 2048, 64, "fp16", "HND", True, False),
    Config("paired_cross_q2048_kv4096", 1, 32, 32, 4096, 128, "bf16", "HND", True, False, Sq=2048),
], ids=lambda c: c.name)
def test_direct_causal_paired_schedule(cfg):
    """Causal direct launches whose 256-row q-blocks fill one round run 128-row q-blocks as a persistent
    grid of one block per CU, each block a heavy and a light q-block in turn: every output
    element and LSE written (NaN canaries), sampled rows of every head against the oracle, and the LSE
    of those rows."""
    from sageattention import _capi, ops

    _say(f"[direct paired] {cfg}")
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        want = cfg.B * cfg.Hq * ((cfg.q_len + 127) // 128)
        assert _capi.split_plan(False, cfg.B, cfg.Hq, cfg.q_len, cfg.S, cfg.D, True, 0) == (want, 1)
    q, k, v = make_inputs(cfg, seed=16)
    lay = ops.HND if cfg.layout == "HND" else ops.NHD
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    vt = torch.empty(cfg.B, cfg.Hkv, cfg.D, cfg.S, device="cuda", dtype=torch.float16)
    ops.v_transpose(vd, vt, lay)
    o = torch.full(qd.shape, float("nan"), device="cuda", dtype=qd.dtype)
    lse = torch.full((cfg.B, cfg.Hq, cfg.q_len), float("nan"), device="cuda", dtype=torch.float32)
    fn = ops.bf16_attn_t if cfg.dtype == "bf16" else ops.fp16_attn_t
    fn(qd, kd, vt, o, lay, 1, cfg.D ** -0.5, 0, lse=lse)
    torch.cuda.synchronize()
    assert not bool(torch.isnan(o).any()) and bool(torch.isfinite(lse).all())
    rows = sample_rows(cfg.q_len, 24, np.random.default_rng(1))
    worst = check_direct_rows(cfg, q, k, vt, o, range(cfg.Hq), rows, cfg.D ** -0.5)
    q32 = orc.to_f32(orc.to_hnd(to_np(q), cfg.layout), cfg.dtype)
    k32 = orc.to_f32(orc.to_hnd(to_np(k), cfg.layout), cfg.dtype)
    got = to_np(lse).astype(np.float64)
    for b in range(cfg.B):
        for h in (0, cfg.Hq - 1):
            ref = orc.attn_direct_lse_rows(q32, k32, cfg.D ** -0.5, b, h, rows, True)
            assert np.all(np.abs(got[b, h, rows] - ref) <= 2e-4 + 2e-6 * np.abs(ref))
    _say(f"  worst |gpu-oracle| = {worst:.3g}")


@pytest.mark.parametrize("cfg", [DIRECT_SMALL[1], DIRECT_SMALL[2], DIRECT_SMALL[4], DIRECT_SMALL[9]],
                         ids=lambda c: c.name)
def test_direct_lse_vs_oracle(cfg):
    _say(f"[direct lse] {cfg}")
    q, k, v = make_inputs(cfg, seed=15)
    o, lse, _ = gpu_direct(cfg, q, k, v, with_lse=True)
    o_plain, _, _ = gpu_direct(cfg, q, k, v)
    assert torch.equal(o, o_plain)
    dt = cfg.dtype
    q32 = orc.to_f32(orc.to_hnd(to_np(q), cfg.layout), dt)
    k32 = orc.to_f32(orc.to_hnd(to_np(k), cfg.layout), dt)
    got = to_np(lse).astype(np.float64)
    for b in range(cfg.B):
        for h in range(cfg.Hq):
            ref = orc.attn_direct_lse_rows(q32, k32, cfg.D ** -0.5, b, h, np.arange(cfg.q_len), cfg.causal)
            err = np.abs(got[b, h] - ref)
            assert np.all(err <= 2e-4 + 2e-6 * np.abs(ref)), f"b={b} h={h} worst {err.max():.3g}"


DIRECT_GROWING = [
    Config("dgrow_d128_causal", 1, 4, 2, 1000, 128, "bf16", "HND", True, False),
    Config("dgrow_d128_nhd", 1, 4, 4, 777, 128, "fp16", "NHD", False, False),
    Config("dgrow_d64", 1, 4, 4, 1100, 64, "fp16", "HND", False, False),
]


@pytest.mark.parametrize("cfg", DIRECT_GROWING, ids=lambda c: c.name)
def test_direct_growing_scores_move_the_reference_max(cfg):
    """Keys whose magnitude grows 4x per 64-key tile over the first six tiles (then keys of one tile
    repeat four rows): every row's max jumps by far more than 2^8 (in p) from tile to tile, so the
    unmasked loop's tile-sum test fails and the tile is redone with the reference max moved (S from
    global K).  Every row against the oracle's direct attention."""
    _say(f"[direct growing] {cfg}")
    q, k, v = (t.float() for t in make_inputs(cfg, seed=11))
    kh = orc.to_hnd(k.numpy(), cfg.layout).copy()
    n = np.arange(cfg.S)
    kh *= (4.0 ** np.minimum(n // 64, 5))[None, None, :, None]
    rep = (n >= 384) & (n % 4 != 0)
    kh[:, :, rep] = kh[:, :, n[rep] // 4 * 4]
    k = torch.from_numpy(kh if cfg.layout == "HND" else kh.transpose(0, 2, 1, 3).copy())
    q, k, v = (t.to(torch.bfloat16 if cfg.dtype == "bf16" else torch.float16) for t in (q, k, v))
    o, _, vt = gpu_direct(cfg, q, k, v)
    worst = check_direct_rows(cfg, q, k, vt, o, range(cfg.Hq), np.arange(cfg.q_len), cfg.D ** -0.5)
    _say(f"  worst |gpu-oracle| = {worst:.3g}")


def test_direct_empty_kv_and_zero_rows():
    """kv_len = 0: zero output and -inf LSE (no key); q_len = 0 is a no-op."""
    from sageattention import ops

    q = torch.randn(1, 2, 5, 64, device="cuda", dtype=torch.float16)
    k = torch.empty(1, 2, 0, 64, device="cuda", dtype=torch.float16)
    vt = torch.empty(1, 2, 64, 0, device="cuda", dtype=torch.float16)
    o = torch.full_like(q, 7.0)
    lse = torch.zeros(1, 2, 5, device="cuda", dtype=torch.float32)
    ops.fp16_attn_t(q, k, vt, o, ops.HND, 0, 0.125, 0, lse=lse)
    torch.cuda.synchronize()
    assert torch.all(o == 0) and torch.all(torch.isneginf(lse))
    q0 = torch.empty(1, 2, 0, 64, device="cuda", dtype=torch.float16)
    ops.fp16_attn_t(q0, q, torch.zeros(1, 2, 64, 64, device="cuda", dtype=torch.float16), torch.empty_like(q0),
                    ops.HND, 1, 0.125, 0)
    torch.cuda.synchronize()
