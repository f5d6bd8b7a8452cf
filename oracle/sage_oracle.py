"""CPU oracle for the SageAttention quantized path (numpy restatement).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or, for the baseline, as the thing timed on the host cores).  The
product path (``sageattention.sageattn`` and the C-ABI library) never calls it.

What it restates (all citations are paths in LuXuxue/sageattention-rdna3):

* ``round_half_away_i8``   -- ``csrc/attn_gfx11.cu:85-92`` (``float_to_int8``)
* ``sm_scale_log2e``       -- ``csrc/attn_gfx11.cu:34,1995``
* ``quant_per_block``      -- ``csrc/attn_gfx11.cu:147-321`` (pass1 absmax with the
                              1e-7 floor ``:192``, ``scale=amax/127`` ``:245``,
                              ``iscale=(127/amax)*extra`` ``:252,296``)
* ``quant_qk_int8``        -- ``csrc/attn_gfx11.cu:1974-2067`` (Q groups of 32
                              tokens, K groups of 16, outputs [B,H,N,D])
* ``k_mean``               -- ``csrc/attn_gfx11.cu:94-145`` (fp32 accumulation,
                              ``sum/S``, cast to the input dtype); the fp32
                              summation ORDER is this build's own (see below)
* ``v_layout``             -- ``csrc/attn_gfx11.cu:323-407,1889-1935`` and
                              ``sageattention/core.py:173-179`` (V -> fp16
                              [B,H,D,ceil64(N)], zero padded, bf16->fp16 RNE)
* ``attn_i8``              -- ``csrc/attn_gfx11.cu:409-825`` (dequant
                              ``acc*(qs*ks)`` ``:618-627``, masks ``:628-631``,
                              exp2-domain softmax ``:656-689``, P rounded to
                              fp16 before PV ``csrc/mma_gfx11.h:97-106``, row sum
                              from unrounded p ``:689``, ``out*(1/l)`` ``:771``)
* ``attn_i8_lse``          -- this build's real ``return_lse`` (the reference
                              returns zeros, ``sageattention/core.py:203-211``):
                              ln sum_j exp of the same scores, ln 2 * (m + log2 l)
* ``attn_direct``          -- ``csrc/attn_gfx11.cu:1465-1885,2275-2472`` (direct
                              fp16/bf16 kernels: ``fl32(dot)*fl32(sm_scale*log2 e)``
                              ``:1675``, masks ``:1676-1679``, the same softmax,
                              fp16 P and ``out*(1/l)`` as the INT8 kernel)
* ``use_direct_path``      -- ``sageattention/core.py:113-139`` (direct/INT8
                              dispatch thresholds and their env overrides)
* ``sageattn``             -- ``sageattention/core.py:40-213`` (dispatch, both
                              branches, fp32 -> fp16 ``:78-83``, default
                              ``sm_scale`` ``:65-66``, ``smooth_k`` default False
                              ``:186``)

Bit-exactness contract: quantised Q/K, their scales, the K mean and the V
layout are defined here exactly (IEEE fp32, no contraction) and the HIP kernels
must reproduce them bit for bit.  The attention output is a floating-point
reduction with hardware exp2; it is compared within a stated tolerance.

The K-mean summation order (parity pinned only through closed forms and fp64
bounds, since the reference's own order is not reproducible: it was compiled
with -ffast-math, ``setup.py:183``):
    rows are cut into chunks of 1024; inside a chunk, lane slot r (0..R-1,
    R = 256 / (D/8)) sums rows r, r+R, r+2R, ... in increasing order; the R slot
    sums are added in increasing r; the chunk sums are added in increasing
    chunk order; the total is divided by fp32(S) and rounded to the dtype.

Array conventions: fp16 data is ``np.float16``; bf16 data is ``np.uint16``
holding the bit patterns (numpy has no bfloat16).  ``layout`` is "HND"
([B,H,N,D]) or "NHD" ([B,N,H,D]).
"""
from __future__ import annotations

import numpy as np

F16 = "fp16"
BF16 = "bf16"
F32 = "fp32"

LOG2E_F32 = np.float32(1.4426950408889634)  # csrc/attn_gfx11.cu:34
Q_GROUP = 32  # csrc/attn_gfx11.cu:46 (MIN_BLK_Q)
K_GROUP = 16  # csrc/attn_gfx11.cu:47 (MIN_BLK_K)
AMAX_FLOOR = np.float32(1e-7)  # csrc/attn_gfx11.cu:192
VT_ALIGN = 64  # sageattention/core.py:174 (ceil64 padding of V_T)
MEAN_CHUNK = 1024  # this build's K-mean chunk (rows per partial sum)

_f32 = np.float32


# --------------------------------------------------------------------------
# dtype helpers
# --------------------------------------------------------------------------
def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 (exact)."""
    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (NaN kept quiet)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    r = ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, ((u >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16), r)
    return r


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """float32 -> float16 round to nearest even (numpy's conversion is RNE)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def to_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == BF16:
        return bf16_to_f32(x)
    return np.asarray(x).astype(np.float32)


def from_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == BF16:
        return f32_to_bf16(x)
    if dtype == F16:
        return f32_to_f16(x)
    return np.asarray(x, dtype=np.float32)


def to_hnd(x: np.ndarray, layout: str) -> np.ndarray:
    """View an NHD [B,N,H,D] array as HND [B,H,N,D] (no copy)."""
    if layout == "HND":
        return x
    if layout == "NHD":
        return x.transpose(0, 2, 1, 3)
    raise ValueError(f"unknown tensor_layout {layout!r}")


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


# --------------------------------------------------------------------------
# quantisation
# --------------------------------------------------------------------------
def round_half_away_i8(t: np.ndarray) -> np.ndarray:
    """``float_to_int8`` of csrc/attn_gfx11.cu:85-92.

    u = fl32(t + (t >= 0 ? 0.5 : -0.5)); then v_cvt_i32_f32 (truncation toward
    zero, NaN -> 0); then clamp to [-128, 127].  Because the +-0.5 is an fp32
    add, values just below .5 can round up (0.49999997 -> 1), exactly as the
    reference does.
    """
    t = np.asarray(t, dtype=np.float32)
    half = np.where(t >= 0, _f32(0.5), _f32(-0.5)).astype(np.float32)
    u = (t + half).astype(np.float32)
    r = np.trunc(u)
    r = np.where(np.isnan(u), 0.0, r)
    r = np.clip(r, -128.0, 127.0)
    return r.astype(np.int8)


def sm_scale_log2e(sm_scale: float) -> np.float32:
    """fp32(sm_scale) * fp32(log2 e), csrc/attn_gfx11.cu:1995."""
    return _f32(_f32(sm_scale) * LOG2E_F32)


def quant_per_block(x32: np.ndarray, group: int, pre_scale, mean32=None):
    """Per-block INT8 quantisation of one tensor, HND view [B,H,S,D] fp32.

    Q (``pre_scale`` = sm_scale*log2e, ``mean32`` None), csrc/attn_gfx11.cu:179-252,296:
        amax = max(1e-7, max|fl(x*s)|), scale = fl(amax/127),
        q8 = rnd(fl(x * fl(fl(127/amax) * s)))
    K (``pre_scale`` None, optional ``mean32`` [B,H,D]), csrc/attn_gfx11.cu:209-219,277-296:
        v = fl(x - mean) (or x), amax = max(1e-7, max|v|), scale = fl(amax/127),
        q8 = rnd(fl(v * fl(127/amax)))
    Returns (int8 [B,H,S,D] contiguous, float32 scales [B,H,ceil(S/group)]).
    """
    B, H, S, D = x32.shape
    G = cdiv(S, group)
    v = np.asarray(x32, dtype=np.float32)
    if mean32 is not None:
        v = (v - mean32[:, :, None, :].astype(np.float32)).astype(np.float32)
    if pre_scale is not None:
        a = np.abs((v * _f32(pre_scale)).astype(np.float32))
    else:
        a = np.abs(v)
    pad = G * group - S
    if pad:
        a = np.concatenate([a, np.zeros((B, H, pad, D), np.float32)], axis=2)
    # fmax ignores NaN like the device fmaxf (csrc/attn_gfx11.cu:213)
    amax = np.fmax.reduce(a.reshape(B, H, G, group * D), axis=-1) if G else np.zeros((B, H, 0), np.float32)
    amax = np.maximum(amax, AMAX_FLOOR).astype(np.float32)
    scale = (amax / _f32(127.0)).astype(np.float32)
    inv = (_f32(127.0) / amax).astype(np.float32)
    if pre_scale is not None:
        iscale = (inv * _f32(pre_scale)).astype(np.float32)
    else:
        iscale = inv
    row_iscale = np.repeat(iscale, group, axis=2)[:, :, :S]
    t = (v * row_iscale[..., None]).astype(np.float32)
    return np.ascontiguousarray(round_half_away_i8(t)), scale


def quant_qk_int8(q, k, dtype, layout, sm_scale, k_mean=None):
    """``quant_qk_int8_gfx11`` (csrc/attn_gfx11.cu:1974-2067).

    q, k: arrays in ``layout`` of ``dtype``; k_mean: [B,Hkv,D] of ``dtype`` or None.
    Returns q8 [B,Hq,Sq,D], q_scale [B,Hq,ceil(Sq/32)], k8 [B,Hkv,Sk,D],
    k_scale [B,Hkv,ceil(Sk/16)].
    """
    q32 = to_f32(to_hnd(q, layout), dtype)
    k32 = to_f32(to_hnd(k, layout), dtype)
    mean32 = None if k_mean is None else to_f32(k_mean, dtype)
    q8, qs = quant_per_block(q32, Q_GROUP, sm_scale_log2e(sm_scale))
    k8, ks = quant_per_block(k32, K_GROUP, None, mean32)
    return q8, qs, k8, ks


# --------------------------------------------------------------------------
# K mean (smooth_k)
# --------------------------------------------------------------------------
def mean_slots(head_dim: int) -> int:
    """Number of row slots of a chunk (one per 16-byte column piece of 256 threads): 256 / (head_dim / 8)."""
    return 256 // (head_dim // 8)


def k_mean(k, dtype, layout):
    """Per-(b,h,d) mean over the sequence, csrc/attn_gfx11.cu:94-145.

    fp32 accumulation in this build's fixed order (module docstring), fp32
    division by S, round to ``dtype``.  Returns [B,H,D] of ``dtype``.
    """
    x = to_f32(to_hnd(k, layout), dtype)
    B, H, S, D = x.shape
    R = mean_slots(D)
    passes = MEAN_CHUNK // R
    nch = cdiv(S, MEAN_CHUNK)
    pad = nch * MEAN_CHUNK - S
    if pad:
        x = np.concatenate([x, np.zeros((B, H, pad, D), np.float32)], axis=2)
    x = x.reshape(B, H, nch, passes, R, D)
    slot = np.zeros((B, H, nch, R, D), np.float32)
    for j in range(passes):
        slot += x[:, :, :, j]
    part = np.zeros((B, H, nch, D), np.float32)
    for r in range(R):
        part += slot[:, :, :, r]
    tot = np.zeros((B, H, D), np.float32)
    for c in range(nch):
        tot += part[:, :, c]
    mean = (tot / _f32(S)).astype(np.float32) if S > 0 else np.full((B, H, D), np.nan, np.float32)
    return from_f32(mean, dtype)


# --------------------------------------------------------------------------
# V layout
# --------------------------------------------------------------------------
def v_layout(v, dtype, layout):
    """V -> fp16 V_T [B,H,D,ceil64(N)], zero padded (csrc/attn_gfx11.cu:323-407)."""
    x = to_f32(to_hnd(v, layout), dtype)
    B, H, S, D = x.shape
    NP = cdiv(S, VT_ALIGN) * VT_ALIGN
    vt = np.zeros((B, H, D, NP), np.float16)
    vt[:, :, :, :S] = f32_to_f16(x).transpose(0, 1, 3, 2)
    return vt


# --------------------------------------------------------------------------
# fused attention
# --------------------------------------------------------------------------
def _scores_rows(q8, k8, q_scale, k_scale, b, hq, rows, is_causal):
    """log2-domain scores s_ij = fl32(fl32(acc_ij) * fl32(qs[i//32] * ks[j//16])) as float64, masked
    entries (j > i when causal, top-left) at -inf; GQA head map hkv = hq // (Hq/Hkv)
    (csrc/attn_gfx11.cu:464,618-631)."""
    Hq = q8.shape[1]
    Hkv = k8.shape[1]
    Sk = k8.shape[2]
    hk = hq // (Hq // Hkv)
    kf = k8[b, hk].astype(np.float32)
    ks_col = k_scale[b, hk][np.arange(Sk) // K_GROUP].astype(np.float32)
    acc = q8[b, hq, rows].astype(np.float32) @ kf.T
    sc = (q_scale[b, hq][rows // Q_GROUP][:, None] * ks_col[None, :]).astype(np.float32)
    s = (acc * sc).astype(np.float32).astype(np.float64)
    if is_causal:
        cols = np.arange(Sk)
        s = np.where(cols[None, :] <= rows[:, None], s, -np.inf)
    return s, hk


def _softmax_pv(s, v_t, b, hk):
    """Output rows (float64) from log2-domain scores s [rows, Sk] (masked = -inf), shared by both
    kernels (INT8 csrc/attn_gfx11.cu:656-771, direct :1683-1805):
        p_ij = exp2(s_ij - max_j s_ij), l_i = sum_j p_ij (unrounded)
        o_i  = sum_j fp16(p_ij) * V_T[:, j] / l_i   (l_i == 0 -> 0)
    """
    Sk = s.shape[1]
    vf = v_t[b, hk, :, :Sk].astype(np.float64).T
    m = s.max(axis=1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp2(s - m)
    l = p.sum(axis=1, keepdims=True)
    p16 = p.astype(np.float16).astype(np.float64)
    o = p16 @ vf
    with np.errstate(invalid="ignore", divide="ignore"):
        o = np.where(l > 0, o / np.where(l > 0, l, 1.0), 0.0)
    return o


def _lse_from_scores(s):
    """ln sum_j exp(s_ij * ln 2) = ln 2 * (m + log2 sum_j exp2(s_ij - m)) per row, -inf without a
    live key."""
    m = s.max(axis=1)
    mf = np.where(np.isfinite(m), m, 0.0)
    l = np.exp2(s - mf[:, None]).sum(axis=1)
    with np.errstate(divide="ignore"):
        return np.where(l > 0, (mf + np.log2(np.where(l > 0, l, 1.0))) * np.log(2.0), -np.inf)


def attn_i8_rows(q8, k8, v_t, q_scale, k_scale, b, hq, rows, is_causal, n_kv_heads=None):
    """Attention output (float64, before the output cast) for selected rows of one head.

    Row i of head hq (GQA head map hkv = hq // (Hq/Hkv), csrc/attn_gfx11.cu:464):
        s_ij = fl32(fl32(acc_ij) * fl32(qs[i//32] * ks[j//16]))   (acc = exact int dot)
        masked (j > i when causal, top-left; j >= Sk) -> p = 0
        p_ij = exp2(s_ij - max_j s_ij), l_i = sum_j p_ij (unrounded)
        o_i  = sum_j fp16(p_ij) * V_ij / l_i   (l_i == 0 -> 0)
    """
    Sk = k8.shape[2]
    rows = np.asarray(rows, dtype=np.int64)
    D = q8.shape[3]
    if Sk == 0 or rows.size == 0:
        return np.zeros((rows.size, D), np.float64)
    s, hk = _scores_rows(q8, k8, q_scale, k_scale, b, hq, rows, is_causal)
    return _softmax_pv(s, v_t, b, hk)


def attn_i8_lse_rows(q8, k8, q_scale, k_scale, b, hq, rows, is_causal):
    """Log-sum-exp (float64) of selected rows: ln sum_j exp(s_ij * ln 2) over the natural-log scores
    (s_ij as in ``attn_i8_rows``, masked keys excluded), -inf for a row without a live key.

    Not in the reference: its ``return_lse`` returns zeros (sageattention/core.py:203-211).  This is
    the quantity that placeholder stands for, restated from the same scores the output uses.
    """
    Sk = k8.shape[2]
    rows = np.asarray(rows, dtype=np.int64)
    if Sk == 0 or rows.size == 0:
        return np.full(rows.size, -np.inf)
    s, _ = _scores_rows(q8, k8, q_scale, k_scale, b, hq, rows, is_causal)
    return _lse_from_scores(s)


def attn_i8_lse(q8, k8, q_scale, k_scale, is_causal, row_block=512):
    """``attn_i8_lse_rows`` over every row: [B,Hq,Sq] float64."""
    B, Hq, Sq, _ = q8.shape
    out = np.zeros((B, Hq, Sq), np.float64)
    for b in range(B):
        for h in range(Hq):
            for r0 in range(0, Sq, row_block):
                rows = np.arange(r0, min(Sq, r0 + row_block))
                out[b, h, rows] = attn_i8_lse_rows(q8, k8, q_scale, k_scale, b, h, rows, is_causal)
    return out


def attn_i8(q8, k8, v_t, q_scale, k_scale, is_causal, out_dtype, row_block=512):
    """Full fused-attention restatement; returns HND [B,Hq,Sq,D] in ``out_dtype``."""
    B, Hq, Sq, D = q8.shape
    out = np.zeros((B, Hq, Sq, D), np.float32)
    for b in range(B):
        for h in range(Hq):
            for r0 in range(0, Sq, row_block):
                rows = np.arange(r0, min(Sq, r0 + row_block))
                out[b, h, rows] = attn_i8_rows(q8, k8, v_t, q_scale, k_scale, b, h, rows, is_causal)
    return from_f32(out, out_dtype)


# --------------------------------------------------------------------------
# direct (unquantised) attention
# --------------------------------------------------------------------------
def _direct_scores_rows(q32, k32, sm_scale, b, hq, rows, is_causal):
    """log2-domain scores of the direct kernel (csrc/attn_gfx11.cu:1655-1680) for selected rows of
    one head, float64, masked entries (j > i when causal, top-left) at -inf:
        s_ij = fl32(fl32(q_i . k_j) * fl32(fl32(sm_scale) * log2 e))
    q32/k32 are HND fp32 copies of the fp16/bf16 inputs (exact).  The dot product is accumulated
    exactly (float64 over fp16/bf16 products) and rounded once to fp32; the kernels accumulate in
    fp32 in a hardware order, a difference inside the tests' tolerance.  The reference masks with
    -FLT_MAX/2 (:1677-1679): every masked p is 0 either way, because key 0 is live in every row.
    GQA head map hkv = hq // (Hq/Hkv)."""
    Hq = q32.shape[1]
    Hkv = k32.shape[1]
    Sk = k32.shape[2]
    hk = hq // (Hq // Hkv)
    acc = (q32[b, hq, rows].astype(np.float64) @ k32[b, hk].astype(np.float64).T).astype(np.float32)
    s = (acc * sm_scale_log2e(sm_scale)).astype(np.float32).astype(np.float64)
    if is_causal:
        cols = np.arange(Sk)
        s = np.where(cols[None, :] <= rows[:, None], s, -np.inf)
    return s, hk


def attn_direct_rows(q32, k32, v_t, sm_scale, b, hq, rows, is_causal):
    """Direct-kernel output (float64, before the output cast) for selected rows of one head: the
    scores of ``_direct_scores_rows`` through ``_softmax_pv`` (P fp16 for fp16 and bf16 inputs,
    V_T fp16, csrc/attn_gfx11.cu:1465-1467,1683-1805)."""
    Sk = k32.shape[2]
    rows = np.asarray(rows, dtype=np.int64)
    if Sk == 0 or rows.size == 0:
        return np.zeros((rows.size, q32.shape[3]), np.float64)
    s, hk = _direct_scores_rows(q32, k32, sm_scale, b, hq, rows, is_causal)
    return _softmax_pv(s, v_t, b, hk)


def attn_direct_lse_rows(q32, k32, sm_scale, b, hq, rows, is_causal):
    """Log-sum-exp (float64, natural log) of the direct kernel's scores, as ``attn_i8_lse_rows``."""
    Sk = k32.shape[2]
    rows = np.asarray(rows, dtype=np.int64)
    if Sk == 0 or rows.size == 0:
        return np.full(rows.size, -np.inf)
    s, _ = _direct_scores_rows(q32, k32, sm_scale, b, hq, rows, is_causal)
    return _lse_from_scores(s)


def attn_direct(q, k, v_t, dtype, layout, sm_scale, is_causal, row_block=512, lse=False):
    """Full direct-kernel restatement (fp16_attn_t / bf16_attn_t, csrc/attn_gfx11.cu:2275-2472):
    q, k in ``layout`` and ``dtype``, v_t from ``v_layout``; returns HND [B,Hq,Sq,D] in ``dtype``
    (and the [B,Hq,Sq] float64 log-sum-exp when ``lse``)."""
    q32 = to_f32(to_hnd(q, layout), dtype)
    k32 = to_f32(to_hnd(k, layout), dtype)
    B, Hq, Sq, D = q32.shape
    out = np.zeros((B, Hq, Sq, D), np.float32)
    lse_out = np.zeros((B, Hq, Sq), np.float64)
    for b in range(B):
        for h in range(Hq):
            for r0 in range(0, Sq, row_block):
                rows = np.arange(r0, min(Sq, r0 + row_block))
                out[b, h, rows] = attn_direct_rows(q32, k32, v_t, sm_scale, b, h, rows, is_causal)
                if lse:
                    lse_out[b, h, rows] = attn_direct_lse_rows(q32, k32, sm_scale, b, h, rows, is_causal)
    o = from_f32(out, dtype)
    return (o, lse_out) if lse else o


# --------------------------------------------------------------------------
# whole path
# --------------------------------------------------------------------------
def use_direct_path(head_dim, q_len, kv_len, is_causal, tensor_layout, env=None):
    """The reference's direct/INT8 dispatch (sageattention/core.py:113-139), thresholds overridable
    through the same environment variables (``env`` defaults to ``os.environ``)."""
    import os

    env = os.environ if env is None else env

    def thr(name, default):
        return int(env.get(name, str(default)) or default)

    if head_dim == 64:
        if is_causal:
            return kv_len <= thr("SAGEATTN_DIRECT_THRESHOLD_D64_CAUSAL", 6144)
        if q_len < kv_len:
            return kv_len <= thr("SAGEATTN_DIRECT_THRESHOLD_D64_CROSS", 6144)
        return kv_len <= thr("SAGEATTN_DIRECT_THRESHOLD_D64", 2048 if tensor_layout == "HND" else 3072)
    if q_len * 2 < kv_len:
        return kv_len <= thr("SAGEATTN_DIRECT_THRESHOLD_D128_CROSS", 4096)
    return kv_len <= thr("SAGEATTN_DIRECT_THRESHOLD_D128", 2048)


def sageattn(q, k, v, dtype, tensor_layout="HND", is_causal=False, sm_scale=None,
             smooth_k=False, intermediates=False, path="auto", lse=False):
    """``sageattention.core.sageattn`` (core.py:40-213): the direct branch or the INT8 branch.

    ``path``: "auto" (the reference's dispatch, ``use_direct_path``), "int8" or "direct".
    Returns the output in the input layout and dtype (fp32 inputs go through fp16,
    core.py:78-83,200-201), then the [B,Hq,Sq] log-sum-exp when ``lse``, then the intermediates
    dict when ``intermediates`` (its "path" names the branch taken).
    """
    D = q.shape[-1]
    if sm_scale is None:
        sm_scale = D ** -0.5
    in_dtype = dtype
    if dtype == F32:
        q, k, v = (np.asarray(t, np.float32).astype(np.float16) for t in (q, k, v))
        dtype = F16
    sq_axis = 2 if tensor_layout == "HND" else 1
    Sq, Sk = q.shape[sq_axis], k.shape[sq_axis]
    if path == "auto":
        path = "direct" if use_direct_path(D, Sq, Sk, is_causal, tensor_layout) else "int8"
    vt = v_layout(v, dtype, tensor_layout)
    if path == "direct":
        o, lse_v = attn_direct(q, k, vt, dtype, tensor_layout, sm_scale, is_causal, lse=True)
        inter = dict(path="direct", v_t=vt)
    else:
        mean = k_mean(k, dtype, tensor_layout) if smooth_k else None
        q8, qs, k8, ks = quant_qk_int8(q, k, dtype, tensor_layout, sm_scale, mean)
        o = attn_i8(q8, k8, vt, qs, ks, is_causal, dtype)
        lse_v = attn_i8_lse(q8, k8, qs, ks, is_causal) if lse else None
        inter = dict(path="int8", mean=mean, q8=q8, q_scale=qs, k8=k8, k_scale=ks, v_t=vt)
    if tensor_layout == "NHD":
        o = o.transpose(0, 2, 1, 3)
    o = np.ascontiguousarray(o)
    if in_dtype == F32:
        o = o.astype(np.float32)
    res = (o,)
    if lse:
        res += (lse_v,)
    if intermediates:
        res += (inter,)
    return res[0] if len(res) == 1 else res


def attn_ops(B, Hq, Sq, Sk, D, is_causal):
    """Effective ops 4*B*Hq*D*pairs; causal pairs = sum_i min(i+1, Sk) (top-left)."""
    if is_causal:
        n = min(Sq, Sk)
        pairs = n * (n + 1) // 2 + max(0, Sq - Sk) * Sk
    else:
        pairs = Sq * Sk
    return 4 * B * Hq * D * pairs


def pairs_for_rows(rows, Sk, is_causal):
    rows = np.asarray(rows, dtype=np.int64)
    if is_causal:
        return int(np.minimum(rows + 1, Sk).sum())
    return int(rows.size * Sk)

