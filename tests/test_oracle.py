"""Pins the CPU oracle (oracle/sage_oracle.py) before it is trusted as the checker.

Checks are chosen so that plausible mistakes fail: known answers of the
rounding rule, a scalar brute force of the quantiser (fp32 emulated through
Python doubles + struct rounding, which is exact for single +,-,*,/ because
53 >= 2*24+2), invariants (|q8| <= 127, the group argmax hits 127, dequant
error <= scale/2, group boundaries), closed forms of the K mean, a brute-force
index check of the V layout, and for the attention: the fp64 dequantised
softmax, GQA == repeat_interleave, NHD == HND, S = 1 and fp32 SDPA agreement.
"""
import math
import struct

import numpy as np
import pytest
import torch

from oracle import sage_oracle as orc
from _helpers import C1, Config, cos_sim, make_inputs, max_abs, to_np


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


# ------------------------------------------------------------------ rounding
@pytest.mark.parametrize(
    "x,expect",
    [
        (0.0, 0), (-0.0, 0), (0.3, 0), (0.5, 1), (0.7, 1), (1.5, 2), (2.5, 3), (126.5, 127),
        (-0.3, 0), (-0.5, -1), (-1.5, -2), (-2.5, -3), (-127.5, -128),
        (127.0, 127), (127.4, 127), (127.6, 127), (200.0, 127), (-128.6, -128), (-300.0, -128),
        # fp32 add of 0.5 rounds 0.49999997 + 0.5 up to 1.0 before truncation
        (0.49999997, 1), (-0.49999997, -1), (0.49999994, 0),
        (float("nan"), 0), (float("inf"), 127), (float("-inf"), -128),
    ],
)
def test_round_half_away_known_answers(x, expect):
    got = int(orc.round_half_away_i8(np.array([x], np.float32))[0])
    assert got == expect


def test_round_is_not_bankers_rounding():
    # np.round(2.5) == 2 would be the plausible mistake
    t = np.array([0.5, 1.5, 2.5, 3.5, -2.5], np.float32)
    assert orc.round_half_away_i8(t).tolist() == [1, 2, 3, 4, -3]


def test_sm_scale_log2e_single_rounding():
    for d in (64, 128):
        s = d ** -0.5
        expect = f32(f32(s) * f32(1.4426950408889634))
        assert float(orc.sm_scale_log2e(s)) == expect
        assert abs(expect - s * math.log2(math.e)) < 1e-7


# ------------------------------------------------------------------ quant
def brute_quant(x, group, s, mean=None):
    """Scalar restatement of csrc/attn_gfx11.cu:182-316 with emulated fp32."""
    S, D = len(x), len(x[0]) if x else 0
    G = -(-S // group)
    out = [[0] * D for _ in range(S)]
    scales = []
    for g in range(G):
        rows = range(g * group, min(S, (g + 1) * group))
        am = f32(1e-7)
        for r in rows:
            for d in range(D):
                v = x[r][d] if mean is None else f32(x[r][d] - mean[d])
                am = max(am, abs(f32(v * (s if s is not None else 1.0))))
        scales.append(f32(am / 127.0))
        inv = f32(127.0 / am)
        isc = f32(inv * (s if s is not None else 1.0))
        for r in rows:
            for d in range(D):
                v = x[r][d] if mean is None else f32(x[r][d] - mean[d])
                t = f32(v * isc)
                u = f32(t + (0.5 if t >= 0 else -0.5))
                out[r][d] = max(-128, min(127, int(u)))
    return out, scales


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("S,D", [(37, 64), (50, 128), (16, 64), (1, 128)])
def test_quant_matches_scalar_brute_force(dtype, S, D):
    rng = np.random.default_rng(S * D)
    x = rng.standard_normal((1, 2, S, D)).astype(np.float32) * 3
    x[0, 1, S // 2, 3] = 40.0  # outlier in one group
    xd = orc.from_f32(x, dtype)
    x32 = orc.to_f32(xd, dtype)
    s = orc.sm_scale_log2e(D ** -0.5)
    mean = orc.from_f32(x32.mean(axis=2) + 0.25, dtype)
    mean32 = orc.to_f32(mean, dtype)
    q8, qs, k8, ks = orc.quant_qk_int8(xd, xd, dtype, "HND", D ** -0.5, k_mean=mean)
    for h in range(2):
        rows = x32[0, h].tolist()
        bq, bqs = brute_quant(rows, 32, float(s))
        bk, bks = brute_quant(rows, 16, None, mean32[0, h].tolist())
        assert q8[0, h].tolist() == bq
        assert qs[0, h].tolist() == bqs
        assert k8[0, h].tolist() == bk
        assert ks[0, h].tolist() == bks


def test_quant_invariants():
    rng = np.random.default_rng(1)
    S, D = 200, 128
    x = (rng.standard_normal((2, 3, S, D)) * rng.uniform(0.01, 5, (2, 3, 1, 1))).astype(np.float32)
    s = orc.sm_scale_log2e(D ** -0.5)
    for group, pre in ((32, s), (16, None)):
        q8, sc = orc.quant_per_block(x, group, pre)
        assert q8.dtype == np.int8 and sc.dtype == np.float32
        assert sc.shape == (2, 3, -(-S // group))
        assert np.all(np.abs(q8.astype(np.int32)) <= 127)
        xs = x * (np.float64(pre) if pre is not None else 1.0)
        for g in range(sc.shape[2]):
            blk = xs[:, :, g * group:(g + 1) * group]
            qb = q8[:, :, g * group:(g + 1) * group].astype(np.int32)
            amax = np.abs(blk).reshape(2, 3, -1).max(-1)
            # scale = amax/127 in fp32 (one rounding)
            assert np.allclose(sc[:, :, g], amax / 127, rtol=2e-7, atol=0)
            # the group's absmax element lands on +-127
            assert np.all(np.abs(qb).reshape(2, 3, -1).max(-1) == 127)
            # dequantisation error is at most half a step (plus fp32 slack)
            err = np.abs(qb * sc[:, :, g][..., None, None].astype(np.float64) - blk)
            assert np.all(err <= 0.5 * sc[:, :, g][..., None, None] * (1 + 1e-5) + 1e-12)


def test_quant_zero_group_and_tail():
    S, D = 40, 64
    x = np.zeros((1, 1, S, D), np.float32)
    x[0, 0, 35, 7] = 1.0  # only in the second (tail) Q group
    q8, sc = orc.quant_per_block(x, 32, np.float32(1.0))
    assert sc[0, 0, 0] == np.float32(np.float32(1e-7) / np.float32(127))
    assert np.all(q8[0, 0, :32] == 0)
    assert q8[0, 0, 35, 7] == 127
    assert sc[0, 0, 1] == np.float32(1.0 / 127)


def test_quant_group_boundaries():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 1, 64, 64)).astype(np.float32)
    _, base = orc.quant_per_block(x, 16, None)
    y = x.copy()
    y[0, 0, 17, 0] = 100.0  # row 17 belongs to K group 1 only
    _, sc = orc.quant_per_block(y, 16, None)
    assert sc[0, 0, 1] == np.float32(np.float32(100) / np.float32(127))
    assert np.array_equal(np.delete(sc[0, 0], 1), np.delete(base[0, 0], 1))


def test_quant_sm_scale_folding():
    """q8 * q_scale reproduces x * sm_scale * log2(e) (csrc/attn_gfx11.cu:179-180)."""
    rng = np.random.default_rng(3)
    D = 128
    x = rng.standard_normal((1, 2, 64, D)).astype(np.float16)
    q8, qs, _, _ = orc.quant_qk_int8(x, x, "fp16", "HND", 0.3)
    deq = q8.astype(np.float64) * np.repeat(qs, 32, axis=2)[..., None]
    ref = x.astype(np.float64) * 0.3 * math.log2(math.e)
    assert np.max(np.abs(deq - ref)) <= 0.5 * qs.max() * 1.001


def test_quant_nhd_equals_hnd():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 70, 64)).astype(np.float16)  # HND
    a = orc.quant_qk_int8(x, x, "fp16", "HND", 0.125)
    b = orc.quant_qk_int8(np.ascontiguousarray(x.transpose(0, 2, 1, 3)),
                          np.ascontiguousarray(x.transpose(0, 2, 1, 3)), "fp16", "NHD", 0.125)
    for u, w in zip(a, b):
        assert np.array_equal(u, w)


# ------------------------------------------------------------------ K mean
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_k_mean_constant_is_exact(dtype):
    x = np.full((1, 2, 1000, 128), 0.75, np.float32)
    m = orc.k_mean(orc.from_f32(x, dtype), dtype, "HND")
    assert np.all(orc.to_f32(m, dtype) == 0.75)


def test_k_mean_dyadic_exact():
    rng = np.random.default_rng(5)
    S = 512  # power of two: sums of small integers are exact, so is /S
    x = rng.integers(-8, 9, size=(1, 3, S, 64)).astype(np.float32)
    m = orc.k_mean(x.astype(np.float16), "fp16", "HND")
    exact = x.astype(np.float64).sum(axis=2) / S
    assert np.array_equal(m.astype(np.float64), exact.astype(np.float16).astype(np.float64))


@pytest.mark.parametrize("S", [1, 255, 256, 257, 1000, 4099])
@pytest.mark.parametrize("D", [64, 128])
def test_k_mean_close_to_fp64(S, D):
    rng = np.random.default_rng(S + D)
    x = (rng.standard_normal((1, 2, S, D)) + 3).astype(np.float16)
    m = orc.k_mean(x, "fp16", "HND").astype(np.float64)
    ref = x.astype(np.float64).mean(axis=2)
    # fp32 accumulation error is far below one fp16 ulp; the cast adds <= 1/2 ulp
    assert np.all(np.abs(m - ref) <= np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64) * 0.5 + 1e-6)


def test_k_mean_layouts_agree():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, 3, 300, 64)).astype(np.float16)
    a = orc.k_mean(x, "fp16", "HND")
    b = orc.k_mean(np.ascontiguousarray(x.transpose(0, 2, 1, 3)), "fp16", "NHD")
    assert np.array_equal(a, b)


# ------------------------------------------------------------------ V layout
@pytest.mark.parametrize("S", [1, 63, 64, 65, 130])
def test_v_layout_index_brute_force(S):
    D = 64
    n = np.arange(S)[:, None]
    d = np.arange(D)[None, :]
    val = ((n % 512) * 4 + d % 4).astype(np.float16)  # exact in fp16, encodes (n, d)
    x = np.broadcast_to(val, (1, 2, S, D)).copy()
    x[0, 1] += 1
    vt = orc.v_layout(x, "fp16", "HND")
    NP = -(-S // 64) * 64
    assert vt.shape == (1, 2, D, NP) and vt.dtype == np.float16
    for h in range(2):
        for nn in range(NP):
            for dd in range(0, D, 7):
                want = x[0, h, nn, dd] if nn < S else 0
                assert vt[0, h, dd, nn] == want


def test_v_layout_bf16_to_fp16_rounding():
    # bf16 values: exact fp16, halfway between fp16 neighbours (ties to even), overflow, tiny
    vals = np.array([1.0, -2.5, 1.0 + 2 ** -7, 1.0 + 2 ** -11 + 2 ** -12, 70000.0, 1e-8, -3e-5, 65504.0], np.float32)
    bits = orc.f32_to_bf16(vals)
    src = orc.bf16_to_f32(bits)
    x = np.zeros((1, 1, 8, 64), np.uint16)
    x[0, 0, :, 0] = bits
    vt = orc.v_layout(x, "bf16", "HND")
    got = vt[0, 0, 0, :8]
    want = src.astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    assert np.isinf(got[4]) and got[0] == 1.0


def test_bf16_rne_known_answers():
    u = np.array([0x3F808000, 0x3F818000, 0x3F80C000, 0x7F7FFFFF], np.uint32).view(np.float32)
    # tie -> even (down), tie -> even (up), above half -> up, overflow -> inf
    assert orc.f32_to_bf16(u).tolist() == [0x3F80, 0x3F82, 0x3F81, 0x7F80]


# ------------------------------------------------------------------ attention
def _dequant_attention_f64(q8, qs, k8, ks, vt, causal, Sk):
    """Independent fp64 dequantised softmax(Q K^T) V without the fp16 P rounding."""
    qd = q8.astype(np.float64) * np.repeat(qs, 32, axis=-1)[..., : q8.shape[-2], None]
    kd = k8.astype(np.float64) * np.repeat(ks, 16, axis=-1)[..., : k8.shape[-2], None]
    G = q8.shape[1] // k8.shape[1]
    kd = np.repeat(kd, G, axis=1)
    v = np.repeat(vt[..., :Sk].astype(np.float64).transpose(0, 1, 3, 2), G, axis=1)
    s = qd @ kd.transpose(0, 1, 3, 2)
    if causal:
        Sq = q8.shape[2]
        s = np.where(np.arange(Sk)[None, :] <= np.arange(Sq)[:, None], s, -np.inf)
    p = np.exp2(s - s.max(-1, keepdims=True))
    return (p @ v) / p.sum(-1, keepdims=True)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_matches_fp64_dequant_softmax(causal):
    rng = np.random.default_rng(7)
    B, Hq, Hkv, S, D = 1, 4, 2, 150, 64
    q = rng.standard_normal((B, Hq, S, D)).astype(np.float16)
    k = rng.standard_normal((B, Hkv, S, D)).astype(np.float16)
    v = rng.standard_normal((B, Hkv, S, D)).astype(np.float16)
    q8, qs, k8, ks = orc.quant_qk_int8(q, k, "fp16", "HND", D ** -0.5)
    vt = orc.v_layout(v, "fp16", "HND")
    o = orc.attn_i8(q8, k8, vt, qs, ks, causal, "fp32")
    ref = _dequant_attention_f64(q8, qs, k8, ks, vt, causal, S)
    # only the fp16 rounding of P separates them (relative 2^-11 per weight)
    assert max_abs(o, ref) < 2e-3
    assert cos_sim(o, ref) > 0.99999


PATHS = ["int8", "direct"]


@pytest.mark.parametrize("path", PATHS)
def test_attention_gqa_equals_repeated_heads(path):
    rng = np.random.default_rng(8)
    q = rng.standard_normal((1, 4, 70, 64)).astype(np.float16)
    k = rng.standard_normal((1, 2, 70, 64)).astype(np.float16)
    v = rng.standard_normal((1, 2, 70, 64)).astype(np.float16)
    o1 = orc.sageattn(q, k, v, "fp16", "HND", True, path=path)
    o2 = orc.sageattn(q, np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1), "fp16", "HND", True, path=path)
    assert np.array_equal(o1, o2)


@pytest.mark.parametrize("path", PATHS)
def test_attention_nhd_equals_hnd(path):
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((2, 3, 90, 128)).astype(np.float16) for _ in range(3))
    o1 = orc.sageattn(q, k, v, "fp16", "HND", True, smooth_k=True, path=path)
    t = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3))  # noqa: E731
    o2 = orc.sageattn(t(q), t(k), t(v), "fp16", "NHD", True, smooth_k=True, path=path)
    assert np.array_equal(o1, t(o2))


@pytest.mark.parametrize("path", PATHS)
def test_attention_single_key_and_first_causal_row(path):
    rng = np.random.default_rng(10)
    q, k, v = (rng.standard_normal((1, 2, 1, 64)).astype(np.float16) for _ in range(3))
    o = orc.sageattn(q, k, v, "fp16", "HND", False, path=path)
    assert np.array_equal(o, v)
    q, k, v = (rng.standard_normal((1, 2, 40, 64)).astype(np.float16) for _ in range(3))
    o = orc.sageattn(q, k, v, "fp16", "HND", True, path=path)
    assert np.array_equal(o[:, :, 0], v[:, :, 0])


@pytest.mark.parametrize("path", PATHS)
def test_attention_constant_v_normalises(path):
    rng = np.random.default_rng(11)
    q, k = (rng.standard_normal((1, 2, 100, 64)).astype(np.float16) for _ in range(2))
    v = np.full((1, 2, 100, 64), 0.5, np.float16)
    o = orc.sageattn(q, k, v, "fp16", "HND", False, path=path).astype(np.float64)
    assert np.all(np.abs(o - 0.5) < 2e-3)


@pytest.mark.parametrize("causal", [False, True])
def test_lse_matches_scipy_logsumexp_of_fp64_dequant_scores(causal):
    """The oracle's LSE (this build's real return_lse) against scipy's logsumexp over independently
    dequantised fp64 scores in natural-log units (the log2-domain scores times ln 2)."""
    from scipy.special import logsumexp

    rng = np.random.default_rng(17)
    B, Hq, Hkv, S, D = 1, 4, 2, 130, 64
    q = rng.standard_normal((B, Hq, S, D)).astype(np.float16)
    k = rng.standard_normal((B, Hkv, S, D)).astype(np.float16)
    q8, qs, k8, ks = orc.quant_qk_int8(q, k, "fp16", "HND", D ** -0.5)
    lse = orc.attn_i8_lse(q8, k8, qs, ks, causal)
    qd = q8.astype(np.float64) * np.repeat(qs, 32, axis=-1)[..., :S, None]
    kd = np.repeat(k8.astype(np.float64) * np.repeat(ks, 16, axis=-1)[..., :S, None], Hq // Hkv, axis=1)
    sn = (qd @ kd.transpose(0, 1, 3, 2)) * math.log(2.0)
    if causal:
        sn = np.where(np.arange(S)[None, :] <= np.arange(S)[:, None], sn, -np.inf)
    ref = logsumexp(sn, axis=-1)
    # only the fp32 rounding of qs*ks and of acc*(qs*ks) separates the two
    assert np.max(np.abs(lse - ref) / np.maximum(1.0, np.abs(ref))) < 1e-6


def test_lse_closed_forms():
    # all-zero Q: every live score is 0, so lse = ln(#live keys): ln(Sk), causal row i -> ln(i + 1)
    q8 = np.zeros((1, 1, 40, 64), np.int8)
    k8 = np.random.default_rng(18).integers(-127, 128, (1, 1, 40, 64)).astype(np.int8)
    qs, ks = np.full((1, 1, 2), 0.01, np.float32), np.full((1, 1, 3), 0.02, np.float32)
    assert np.allclose(orc.attn_i8_lse(q8, k8, qs, ks, False), math.log(40), rtol=0, atol=1e-12)
    assert np.allclose(orc.attn_i8_lse(q8, k8, qs, ks, True)[0, 0], np.log(np.arange(1, 41)), rtol=0, atol=1e-12)
    # one key: lse = s * ln 2 exactly as the score; no key: -inf
    q8 = np.full((1, 1, 1, 64), 3, np.int8)
    k8 = np.full((1, 1, 1, 64), -2, np.int8)
    s = np.float32(np.float32(3 * -2 * 64) * np.float32(np.float32(0.01) * np.float32(0.02)))
    assert orc.attn_i8_lse(q8, k8, qs[..., :1], ks[..., :1], False)[0, 0, 0] == float(s) * math.log(2.0)
    empty = orc.attn_i8_lse(q8, np.zeros((1, 1, 0, 64), np.int8), qs[..., :1], np.zeros((1, 1, 0), np.float32), False)
    assert np.all(np.isneginf(empty))


def test_attention_empty_kv_gives_zero():
    q8 = np.ones((1, 1, 5, 64), np.int8)
    k8 = np.zeros((1, 1, 0, 64), np.int8)
    o = orc.attn_i8(q8, k8, np.zeros((1, 1, 64, 0), np.float16), np.ones((1, 1, 1), np.float32),
                    np.zeros((1, 1, 0), np.float32), False, "fp16")
    assert np.all(o == 0)


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("path", PATHS)
def test_oracle_vs_fp32_sdpa(dtype, causal, path):
    """Error budget of each algorithm itself against fp32 SDPA (C1 shape): INT8 quantisation, or
    for the direct path only the fp16 rounding of P and of the output (much tighter)."""
    cfg = Config("t", 1, 2, 2, 256, 64, dtype, "HND", causal, False)
    q, k, v = make_inputs(cfg, seed=3)
    o = orc.sageattn(to_np(q), to_np(k), to_np(v), dtype, "HND", causal, path=path)
    o32 = orc.to_f32(o, "fp16" if dtype == "fp32" else dtype) if dtype != "fp32" else o
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=causal)
    if path == "int8":
        assert cos_sim(o32, ref.numpy()) > 0.999
        assert max_abs(o32, ref.numpy()) < 0.05
    else:
        assert cos_sim(o32, ref.numpy()) > 0.99999
        assert max_abs(o32, ref.numpy()) < (1e-2 if dtype == "bf16" else 2e-3)


def test_smooth_k_shift_invariance():
    rng = np.random.default_rng(12)
    q, k, v = (rng.standard_normal((1, 2, 256, 64)).astype(np.float32) for _ in range(3))
    shift = rng.standard_normal((1, 2, 1, 64)).astype(np.float32) * 4
    o1 = orc.sageattn(q.astype(np.float16), k.astype(np.float16), v.astype(np.float16), "fp16", "HND", False,
                      smooth_k=True, path="int8")
    o2 = orc.sageattn(q.astype(np.float16), (k + shift).astype(np.float16), v.astype(np.float16), "fp16", "HND", False,
                      smooth_k=True, path="int8")
    assert cos_sim(o1, o2) > 0.9999


# ------------------------------------------------------------------ direct (unquantised) path
def _textbook_attention_f64(q, k, v_hnd, dtype, layout, sm_scale, causal):
    """Independent fp64 softmax(sm_scale * Q K^T) V with natural exp, GQA by repeat, plus the fp64
    log-sum-exp (scipy); q, k in ``layout``/``dtype``, v_hnd the HND values of V as the kernel reads
    them (fp16).  No fp16 rounding of P anywhere."""
    from scipy.special import logsumexp

    qh, kh = (orc.to_f32(orc.to_hnd(t, layout), dtype).astype(np.float64) for t in (q, k))
    G = qh.shape[1] // kh.shape[1]
    kh, vh = np.repeat(kh, G, axis=1), np.repeat(v_hnd.astype(np.float64), G, axis=1)
    s = (qh @ kh.transpose(0, 1, 3, 2)) * sm_scale
    if causal:
        Sq, Sk = qh.shape[2], kh.shape[2]
        s = np.where(np.arange(Sk)[None, :] <= np.arange(Sq)[:, None], s, -np.inf)
    lse = logsumexp(s, axis=-1)
    return np.exp(s - lse[..., None]) @ vh, lse


DIRECT_CASES = [
    # B, Hq, Hkv, Sq, Sk, D, dtype, layout, causal, sm_scale
    (1, 4, 2, 150, 150, 64, "fp16", "HND", True, None),
    (2, 2, 2, 70, 130, 128, "bf16", "NHD", False, None),
    (1, 3, 1, 90, 40, 128, "fp16", "HND", True, 0.3),
    (1, 2, 2, 33, 33, 64, "bf16", "HND", False, -0.125),
]


@pytest.mark.parametrize("case", DIRECT_CASES, ids=lambda c: f"{c[6]}_{c[7]}_c{int(c[8])}_sq{c[3]}_sk{c[4]}")
def test_direct_matches_textbook_fp64_softmax(case):
    """The direct restatement against an independent fp64 softmax attention: only the fp32 rounding
    of the scores and the fp16 rounding of P (relative 2^-11 per weight) separate them; a dropped
    log2 e, a wrong mask, a transposed operand or a wrong GQA head map would not fit."""
    B, Hq, Hkv, Sq, Sk, D, dtype, layout, causal, sm = case
    sm_scale = D ** -0.5 if sm is None else sm
    rng = np.random.default_rng(21)

    def mk(H, S):
        x = rng.standard_normal((B, H, S, D)).astype(np.float32)
        x = x if layout == "HND" else np.ascontiguousarray(x.transpose(0, 2, 1, 3))
        return x.astype(np.float16) if dtype == "fp16" else orc.f32_to_bf16(x)

    q, k, v = mk(Hq, Sq), mk(Hkv, Sk), mk(Hkv, Sk)
    vt = orc.v_layout(v, dtype, layout)
    o, lse = orc.attn_direct(q, k, vt, dtype, layout, sm_scale, causal, lse=True)
    o = orc.to_f32(o, dtype).astype(np.float64)
    v_vals = orc.to_f32(vt[..., :Sk], "fp16").transpose(0, 1, 3, 2)  # V as fp16, as the kernel reads it
    ref, ref_lse = _textbook_attention_f64(q, k, v_vals, dtype, layout, sm_scale, causal)
    tol = 4e-3 if dtype == "bf16" else 2e-3  # output rounding (bf16 has 8 bits) + P rounding
    assert max_abs(o, ref) < tol
    assert cos_sim(o, ref) > 0.99999
    assert np.max(np.abs(lse - ref_lse) / np.maximum(1.0, np.abs(ref_lse))) < 2e-6


def test_direct_closed_forms():
    # zero Q: uniform weights over the live keys -> mean of V's rows; lse = ln(#live)
    B, H, S, D = 1, 1, 24, 64
    q = np.zeros((B, H, S, D), np.float16)
    rng = np.random.default_rng(22)
    k = rng.standard_normal((B, H, S, D)).astype(np.float16)
    v = (rng.integers(-4, 5, (B, H, S, D)) * 0.25).astype(np.float16)
    vt = orc.v_layout(v, "fp16", "HND")
    o, lse = orc.attn_direct(q, k, vt, "fp16", "HND", 0.125, True, lse=True)
    want = np.cumsum(v[0, 0].astype(np.float64), axis=0) / np.arange(1, S + 1)[:, None]
    assert np.max(np.abs(o[0, 0].astype(np.float64) - want)) <= 2.0 ** -10 * np.abs(want).max() + 1e-7
    assert np.allclose(lse[0, 0], np.log(np.arange(1, S + 1)), rtol=0, atol=1e-12)
    # one key: output == v exactly, lse == the natural-log score
    q1 = np.full((1, 1, 1, 64), 0.5, np.float16)
    k1 = np.full((1, 1, 1, 64), -0.25, np.float16)
    v1 = rng.standard_normal((1, 1, 1, 64)).astype(np.float16)
    o1, l1 = orc.attn_direct(q1, k1, orc.v_layout(v1, "fp16", "HND"), "fp16", "HND", 0.125, False, lse=True)
    assert np.array_equal(o1, v1)
    s = np.float32(np.float32(-8.0) * orc.sm_scale_log2e(0.125))
    assert l1[0, 0, 0] == float(s) * math.log(2.0)


def test_direct_dispatch_known_answers(monkeypatch):
    """sageattention/core.py:113-139: the thresholds at their edges, and the env overrides."""
    for k in [k for k in list(__import__("os").environ) if k.startswith("SAGEATTN_DIRECT_THRESHOLD")]:
        monkeypatch.delenv(k)
    u = orc.use_direct_path
    assert u(64, 2048, 2048, False, "HND") and not u(64, 2049, 2049, False, "HND")
    assert u(64, 3072, 3072, False, "NHD") and not u(64, 3073, 3073, False, "NHD")
    assert u(64, 6144, 6144, True, "HND") and not u(64, 6145, 6145, True, "NHD")
    assert u(64, 100, 6144, False, "HND") and not u(64, 100, 6145, False, "HND")
    assert u(128, 2048, 2048, True, "HND") and not u(128, 2049, 2049, False, "NHD")
    assert u(128, 2047, 4096, False, "HND") and not u(128, 2048, 4096, False, "HND")
    assert not u(128, 100, 4097, True, "HND")
    monkeypatch.setenv("SAGEATTN_DIRECT_THRESHOLD_D128", "-1")
    assert not u(128, 1, 1, False, "HND")
    monkeypatch.setenv("SAGEATTN_DIRECT_THRESHOLD_D64_CAUSAL", "10000")
    assert u(64, 9000, 9000, True, "HND")


def test_product_dispatch_matches_oracle(monkeypatch):
    """The package's dispatch (host logic, no GPU) agrees with the oracle's restatement."""
    from sageattention.core import use_direct_path

    for k in [k for k in list(__import__("os").environ) if k.startswith("SAGEATTN_DIRECT_THRESHOLD")]:
        monkeypatch.delenv(k)
    for D in (64, 128):
        for causal in (False, True):
            for lay in ("HND", "NHD"):
                for sq in (1, 100, 1024, 2047, 2048, 2049, 3072, 6144, 8192):
                    for sk in (1, 100, 2048, 2049, 3072, 3073, 4096, 4097, 6144, 6145):
                        assert use_direct_path(D, sq, sk, causal, lay) == orc.use_direct_path(D, sq, sk, causal, lay)


def test_attn_ops_closed_form():
    assert orc.attn_ops(1, 32, 16384, 16384, 128, True) == 4 * 32 * 128 * (16384 * 16385 // 2)
    assert orc.attn_ops(1, 10, 4096, 4096, 64, False) == 4 * 10 * 64 * 4096 * 4096
    assert orc.pairs_for_rows(np.arange(10), 10, True) == 55


# ------------------------------------------------------------------ the CPU baseline (oracle/torch_cpu.py)
@pytest.mark.parametrize("cfg", [
    Config("tc_bf16_causal", 1, 4, 2, 300, 128, "bf16", "HND", True, False),
    Config("tc_fp16_ragged", 2, 3, 3, 97, 64, "fp16", "HND", False, False),
], ids=lambda c: c.name)
def test_torch_cpu_baseline_matches_oracle(cfg):
    """bench.py's CPU baseline computes the same quantized math: its INT8 Q/K and scales equal the oracle's
    bit for bit, and its attention rows (blockwise online softmax in fp32, small blocks so that several
    key blocks and the causal diagonal are crossed) agree with the oracle's fp64 rows within the fp16
    rounding of P (a running max that is not yet the row max rounds P at a different scale)."""
    from oracle import torch_cpu as tc

    q, k, v = make_inputs(cfg, seed=3)
    sm = cfg.D ** -0.5
    q8o, qso, k8o, kso = orc.quant_qk_int8(to_np(q), to_np(k), cfg.dtype, "HND", sm)
    q8, qs, k8, ks, _ = tc.quant_qk(q, k, sm)
    for got, want in ((q8, q8o), (qs, qso), (k8, k8o), (ks, kso)):
        assert np.array_equal(got.numpy(), want)
    vt = orc.v_layout(to_np(v), cfg.dtype, "HND")
    out = tc.sageattn_heads(q, k, v, cfg.causal, sm, block=64)
    rows = np.arange(cfg.S)
    for h in range(cfg.Hq):
        ref = orc.attn_i8_rows(q8o, k8o, vt, qso, kso, 0, h, rows, cfg.causal)
        assert max_abs(out[h].numpy(), ref) < 1e-3
        assert cos_sim(out[h].numpy(), ref) > 0.99999
