"""GPU parity of the key-split path of the non-causal attention entry points
(``sage_attn_i8_fwd_qfused`` and ``sage_attn_direct_fwd`` with ``num_splits``):
each q-block's key range is cut into n parts whose fp32 partial outputs and LSEs
a second kernel merges.  The split result is the unsplit attention up to
rounding, so it is held to the same oracle bar as the unsplit kernels,
    |gpu - oracle| <= ATOL + RTOL * |oracle|,  cos >= 0.99999
(fp16 out: ATOL 2e-3, RTOL 4e-3; bf16 out: ATOL 4e-3, RTOL 1.6e-2), its LSE to
2e-4 + 2e-6 |oracle|, and to the same bar against the unsplit launch.
"""
import numpy as np
import pytest
import torch

from oracle import sage_oracle as orc
from _helpers import Config, cos_sim, make_inputs, np_to_f32, sample_rows, to_np
from test_gpu_direct import check_direct_rows
from test_gpu_parity import check_rows_vs_oracle, gpu_prologue

pytestmark = pytest.mark.gpu

TOL = {"fp16": (2e-3, 4e-3), "bf16": (4e-3, 1.6e-2)}


def _say(*a):
    print(*a, flush=True)


def _lay(cfg):
    from sageattention import ops

    return ops.HND if cfg.layout == "HND" else ops.NHD


def fused_split(cfg, qd, k8, ks, vt, n):
    """The INT8 path (Q quantised in the kernel) with n key splits -> (out, lse)."""
    from sageattention import ops

    o = torch.empty_like(qd)
    lse = torch.empty((cfg.B, cfg.Hq, cfg.q_len), device="cuda", dtype=torch.float32)
    ops.qk_int8_sv_bf16_attn_qfused_t(qd, k8, vt, o, ks, _lay(cfg), int(cfg.causal), cfg.D ** -0.5, lse=lse,
                                      num_splits=n)
    torch.cuda.synchronize()
    return o, lse


def direct_split(cfg, qd, kd, vt, n, sm_scale=None):
    from sageattention import ops

    o = torch.empty_like(qd)
    lse = torch.empty((cfg.B, cfg.Hq, cfg.q_len), device="cuda", dtype=torch.float32)
    fn = ops.bf16_attn_t if qd.dtype == torch.bfloat16 else ops.fp16_attn_t
    fn(qd, kd, vt, o, _lay(cfg), int(cfg.causal), cfg.D ** -0.5 if sm_scale is None else sm_scale, 0, lse=lse,
       num_splits=n)
    torch.cuda.synchronize()
    return o, lse


def assert_close_to(cfg, got, want):
    """Split vs unsplit launch: the oracle bar, element-wise."""
    atol, rtol = TOL[cfg.dtype]
    g, w = (orc.to_hnd(np_to_f32(to_np(t), cfg.dtype), cfg.layout).astype(np.float64) for t in (got, want))
    err = np.abs(g - w)
    assert np.all(err <= atol + rtol * np.abs(w)), f"worst |split - unsplit| {err.max():.3g}"
    assert cos_sim(g, w) >= 0.99999
    return float(err.max())


def assert_lse(got, ref):
    got = to_np(got).astype(np.float64)
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    err = np.abs(got[fin] - ref[fin])
    assert np.all(err <= 2e-4 + 2e-6 * np.abs(ref[fin])), f"worst lse err {err.max():.3g}"


SPLIT_CASES = [
    (Config("d128_fp16", 1, 4, 2, 1000, 128, "fp16", "HND", False, False), 3),
    (Config("d64_nhd_gqa_smooth", 1, 8, 2, 1057, 64, "fp16", "NHD", False, True), 5),
    (Config("d128_bf16_cross", 2, 2, 2, 777, 128, "bf16", "HND", False, False, Sq=300), 2),
    (Config("d64_bf16_ragged_16", 1, 3, 3, 4097, 64, "bf16", "HND", False, False, Sq=513), 16),
    # 5 key tiles and 7 requested splits: one tile per split, the last one partial
    (Config("one_tile_per_split", 1, 2, 2, 300, 128, "fp16", "NHD", False, False), 7),
    (Config("d128_koffset_smooth", 1, 2, 2, 2049, 128, "bf16", "HND", False, True, k_offset_std=2.0), 4),
    # D = 64 non-causal (128-row blocks of 4 waves): 9000 keys put more than 128 k-scale groups in each wave's
    # share of the block's scale scan
    (Config("d64_long_keys", 1, 2, 2, 9000, 64, "fp16", "HND", False, False, Sq=300), 2),
]


@pytest.mark.parametrize("cfg,n", SPLIT_CASES, ids=lambda c: c.name if isinstance(c, Config) else str(c))
def test_int8_split_vs_oracle_and_unsplit(cfg, n):
    _say(f"[int8 split {n}] {cfg}")
    q, k, v = make_inputs(cfg, seed=21)
    pro = gpu_prologue(cfg, q, k, v)
    qd = q.cuda()
    o, lse = fused_split(cfg, qd, pro["k8"], pro["k_scale"], pro["v_t"], n)
    o1, lse1 = fused_split(cfg, qd, pro["k8"], pro["k_scale"], pro["v_t"], 1)
    worst = check_rows_vs_oracle(cfg, pro, o, range(cfg.Hq), np.arange(cfg.q_len), cfg.dtype)
    d = assert_close_to(cfg, o, o1)
    q8, qs, k8, ks = (to_np(pro[x]) for x in ("q8", "q_scale", "k8", "k_scale"))
    assert_lse(lse, orc.attn_i8_lse(q8, k8, qs, ks, cfg.causal))
    _say(f"  worst |gpu-oracle| = {worst:.3g}, |split-unsplit| = {d:.3g}")


@pytest.mark.parametrize("cfg,n", SPLIT_CASES, ids=lambda c: c.name if isinstance(c, Config) else str(c))
def test_direct_split_vs_oracle_and_unsplit(cfg, n):
    from sageattention import ops

    _say(f"[direct split {n}] {cfg}")
    q, k, v = make_inputs(cfg, seed=22)
    qd, kd, vd = (t.cuda() for t in (q, k, v))
    NP = (cfg.S + 63) // 64 * 64
    vt = torch.empty(cfg.B, cfg.Hkv, cfg.D, NP, device="cuda", dtype=torch.float16)
    ops.v_transpose(vd, vt, _lay(cfg))
    o, lse = direct_split(cfg, qd, kd, vt, n)
    o1, _ = direct_split(cfg, qd, kd, vt, 1)
    worst = check_direct_rows(cfg, q, k, vt, o, range(cfg.Hq), np.arange(cfg.q_len), cfg.D ** -0.5)
    d = assert_close_to(cfg, o, o1)
    q32 = orc.to_f32(orc.to_hnd(to_np(q), cfg.layout), cfg.dtype)
    k32 = orc.to_f32(orc.to_hnd(to_np(k), cfg.layout), cfg.dtype)
    ref = np.stack([np.stack([orc.attn_direct_lse_rows(q32, k32, cfg.D ** -0.5, b, h, np.arange(cfg.q_len),
                                                       cfg.causal) for h in range(cfg.Hq)]) for b in range(cfg.B)])
    assert_lse(lse, ref)
    _say(f"  worst |gpu-oracle| = {worst:.3g}, |split-unsplit| = {d:.3g}")


def test_split_with_large_scales_and_negative_scale():
    """Splits whose tiles leave the conversion-free softmax (q_scale * k_scale > 0.49 in one split
    only) next to splits that keep it; and a negative sm_scale on the direct path."""
    from sageattention import ops

    cfg = Config("large_split", 1, 4, 2, 1000, 128, "fp16", "HND", False, False)
    q, k, v = (t.float() for t in make_inputs(cfg, seed=7))
    k[0, 0, 600:620, 7] = 300.0
    q[0, 0, 800:840, 7] = 300.0
    q, k, v = (t.to(torch.float16) for t in (q, k, v))
    pro = gpu_prologue(cfg, q, k, v)
    assert float(pro["q_scale"].max()) * float(pro["k_scale"].max()) > 0.6
    o, _ = fused_split(cfg, q.cuda(), pro["k8"], pro["k_scale"], pro["v_t"], 3)
    check_rows_vs_oracle(cfg, pro, o, range(cfg.Hq), np.arange(cfg.q_len), cfg.dtype)
    qd, kd = q.cuda(), k.cuda()
    vt = pro["v_t"]
    o, _ = direct_split(cfg, qd, kd, vt, 4, sm_scale=-0.07)
    check_direct_rows(cfg, q, k, vt, o, range(cfg.Hq), np.arange(cfg.q_len), -0.07)
    _ = ops  # the ops layer is exercised through the helpers


def _with_env_splits(value, fn):
    import os

    saved = os.environ.get("SAGEATTN_KV_SPLITS")
    try:
        if value is None:
            os.environ.pop("SAGEATTN_KV_SPLITS", None)
        else:
            os.environ["SAGEATTN_KV_SPLITS"] = value
        return fn()
    finally:
        if saved is None:
            os.environ.pop("SAGEATTN_KV_SPLITS", None)
        else:
            os.environ["SAGEATTN_KV_SPLITS"] = saved


def test_auto_split_of_a_small_grid():
    """B1 H10 S2048 D128 fp16 (80 q-blocks for 256 CUs): the library's own plan splits every q-block,
    and sageattn's result (direct path) matches the unsplit one and the oracle."""
    from sageattention import _capi, sageattn

    cfg = Config("small_grid", 1, 10, 10, 2048, 128, "fp16", "HND", False, False)
    whole, n = _capi.split_plan(False, 1, 10, 2048, 2048, 128, False, 0)
    _say(f"[auto split] plan: {whole} whole q-blocks, {n} splits")
    assert whole == 0 and n > 1
    q, k, v = make_inputs(cfg, seed=23)
    qd, kd, vd = (t.cuda() for t in (q, k, v))
    o_auto = _with_env_splits(None, lambda: sageattn(qd, kd, vd, tensor_layout="HND", is_causal=False))
    o_one = _with_env_splits("1", lambda: sageattn(qd, kd, vd, tensor_layout="HND", is_causal=False))
    torch.cuda.synchronize()
    assert_close_to(cfg, o_auto, o_one)
    from sageattention import ops

    vt = torch.empty(1, 10, 128, 2048, device="cuda", dtype=torch.float16)
    ops.v_transpose(vd, vt, ops.HND)
    rows = sample_rows(cfg.q_len, 64, np.random.default_rng(0))
    check_direct_rows(cfg, q, k, vt, o_auto, [0, 9], rows, cfg.D ** -0.5)


def test_auto_tail_split_of_128_row_blocks():
    """B1 H10 S4096 D64 fp16, INT8 path: 320 q-blocks of 128 rows (D = 64 non-causal runs two blocks
    per CU); the plan runs 256 whole and splits the other 64; sageattn matches the unsplit launch."""
    from sageattention import _capi, sageattn

    cfg = Config("w4_tail", 1, 10, 10, 4096, 64, "fp16", "HND", False, False)
    whole, n = _capi.split_plan(True, 1, 10, 4096, 4096, 64, False, 0)
    _say(f"[128-row tail split] plan: {whole} whole q-blocks, {n} splits")
    assert 0 < whole < 320 and n > 1
    q, k, v = make_inputs(cfg, seed=29)
    qd, kd, vd = (t.cuda() for t in (q, k, v))
    o_auto = _with_env_splits(None, lambda: sageattn(qd, kd, vd, tensor_layout="HND", is_causal=False))
    o_one = _with_env_splits("1", lambda: sageattn(qd, kd, vd, tensor_layout="HND", is_causal=False))
    torch.cuda.synchronize()
    assert_close_to(cfg, o_auto, o_one)


def test_auto_tail_split_of_a_round_and_a_bit():
    """B2 H144, 256 queries x 4096 keys, D128 (288 q-blocks = one round of 256 CUs + 32): the plan runs
    the first 256 q-blocks whole and splits only the last 32 (the last round).  Every q-block, whole
    or split, matches the unsplit launch; sampled rows of both kinds match the oracle."""
    from sageattention import _capi

    cfg = Config("tail", 2, 144, 144, 4096, 128, "bf16", "HND", False, False, Sq=256)
    whole, n = _capi.split_plan(True, 2, 144, 256, 4096, 128, False, 0)
    _say(f"[tail split] plan: {whole} whole q-blocks, {n} splits")
    assert 0 < whole < 288 and n > 1
    q, k, v = make_inputs(cfg, seed=25)
    pro = gpu_prologue(cfg, q, k, v)
    qd = q.cuda()
    o, lse = fused_split(cfg, qd, pro["k8"], pro["k_scale"], pro["v_t"], 0)
    o1, lse1 = fused_split(cfg, qd, pro["k8"], pro["k_scale"], pro["v_t"], 1)
    assert_close_to(cfg, o, o1)
    fin = torch.isfinite(lse1)
    assert torch.max(torch.abs(lse - lse1)[fin]).item() < 1e-4
    # q-block id = b * 144 + h (one q-block per head): heads 0 and 100 of batch 1 run whole (ids 144,
    # 244), heads 120 and 143 of batch 1 are split (ids 264, 287)
    rows = np.arange(0, 256, 5)
    q8, qs, k8, ks, vt = (to_np(pro[x]) for x in ("q8", "q_scale", "k8", "k_scale", "v_t"))
    og = np_to_f32(to_np(o), "bf16")
    atol, rtol = TOL["bf16"]
    for h in (0, 100, 120, 143):
        ref = orc.attn_i8_rows(q8, k8, vt, qs, ks, 1, h, rows, False)
        ref = np_to_f32(orc.from_f32(ref.astype(np.float32), "bf16"), "bf16")
        err = np.abs(og[1, h, rows].astype(np.float64) - ref)
        assert np.all(err <= atol + rtol * np.abs(ref)), f"h={h} worst {err.max():.3g}"


def test_split_repeat_is_deterministic_and_causal_ignores_splits():
    cfg = Config("rep", 1, 4, 4, 2000, 128, "bf16", "HND", False, False)
    q, k, v = make_inputs(cfg, seed=24)
    pro = gpu_prologue(cfg, q, k, v)
    qd = q.cuda()
    a, la = fused_split(cfg, qd, pro["k8"], pro["k_scale"], pro["v_t"], 6)
    b, lb = fused_split(cfg, qd, pro["k8"], pro["k_scale"], pro["v_t"], 6)
    assert torch.equal(a, b) and torch.equal(la, lb)
    ccfg = Config("rep_c", 1, 4, 4, 2000, 128, "bf16", "HND", True, False)
    c1, l1 = fused_split(ccfg, qd, pro["k8"], pro["k_scale"], pro["v_t"], 1)
    c6, l6 = fused_split(ccfg, qd, pro["k8"], pro["k_scale"], pro["v_t"], 6)
    assert torch.equal(c1, c6) and torch.equal(l1, l6)


# ------------------------------------------------------------------ persistent grid (more items than CUs)
PERSISTENT = [
    # 300 / 600 q-blocks of one 256-row block each: a persistent grid with 1-3 items per block
    Config("p_causal_h300", 1, 300, 300, 256, 64, "fp16", "HND", True, False),
    Config("p_noncausal_gqa_h600", 1, 600, 150, 200, 128, "bf16", "NHD", False, False),
    Config("p_cross_causal_2x160", 2, 160, 40, 130, 64, "bf16", "HND", True, False, Sq=300),
    Config("p_smooth_b3", 3, 100, 100, 333, 128, "fp16", "HND", False, True),
    # D = 64 non-causal runs 128-row q-blocks, two blocks per CU: 800 q-blocks over 512 slots
    Config("p_noncausal_d64_h400", 1, 400, 400, 200, 64, "fp16", "HND", False, False),
]


@pytest.mark.parametrize("cfg", PERSISTENT, ids=lambda c: c.name)
def test_persistent_grid_all_rows_vs_oracle(cfg):
    """Launches with more q-blocks than CUs run a persistent grid (static snake schedule over the XCDs);
    every row of the fused-Q INT8 kernel and of the direct kernel is held to the oracle bar, and the
    INT8 output equals the two-kernel path bit for bit (each item is computed the same way in any
    schedule)."""
    from sageattention import ops

    _say(f"[persistent] {cfg}")
    q, k, v = make_inputs(cfg, seed=31)
    pro = gpu_prologue(cfg, q, k, v)
    qd = q.cuda()
    o, _ = fused_split(cfg, qd, pro["k8"], pro["k_scale"], pro["v_t"], 1)
    check_rows_vs_oracle(cfg, pro, o, range(cfg.Hq), np.arange(cfg.q_len), cfg.dtype)
    o2 = torch.empty_like(qd)
    ops.qk_int8_sv_bf16_attn_t(pro["q8"], pro["k8"], pro["v_t"], o2, pro["q_scale"], pro["k_scale"], _lay(cfg),
                               int(cfg.causal), cfg.D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(o, o2)
    od, _ = direct_split(cfg, qd, k.cuda(), pro["v_t"], 1)
    check_direct_rows(cfg, q, k, pro["v_t"], od, range(cfg.Hq), np.arange(cfg.q_len), cfg.D ** -0.5)
