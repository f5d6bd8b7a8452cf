"""Drop-in ``sageattn`` for MI355X on gfx950 kernels.

Mirrors ``sageattention/core.py:40-233`` of the reference (same signature,
defaults, assertion messages, fp32 handling, ``smooth_k`` default False, the
upstream alias and the direct/INT8 dispatch with its thresholds and
``SAGEATTN_DIRECT_THRESHOLD_*`` environment overrides, core.py:113-139);
``return_lse`` returns the real log-sum-exp where the reference returns a zero
placeholder.  The reference's Triton backend and ``SAGEATTN_BACKEND`` switch
(core.py:8,68-76) do not exist here.  Non-causal launches whose grid leaves
compute units idle may split each q-block's key range (``SAGEATTN_KV_SPLITS``:
unset or 0 = the library's choice, 1 = never split, n = n splits).
"""
from __future__ import annotations

import os
from typing import Any, Optional, Tuple, Union

import torch

from . import _capi, ops


def _vector_ready(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` or a copy that satisfies the 16-byte access contract
    (base aligned to 16 bytes, batch/head/token strides multiples of 8)."""
    st = t.stride()
    if t.data_ptr() % 16 == 0 and st[0] % 8 == 0 and st[1] % 8 == 0 and st[2] % 8 == 0:
        return t
    return t.contiguous() if not t.is_contiguous() else t.clone()


def _env_int(name: str, default: int) -> int:
    return int(os.getenv(name, str(default)) or default)


def use_direct_path(head_dim: int, q_len: int, kv_len: int, is_causal: bool, tensor_layout: str) -> bool:
    """The reference's choice between the direct fp16/bf16 kernel (no
    quantisation prologue) and the INT8 path (sageattention/core.py:113-139):
    short key ranges go direct.  Defaults, per head_dim and shape:
      D=64:  causal kv <= 6144; cross (q < kv) kv <= 6144; self kv <= 2048
             (HND) or 3072 (NHD);
      D=128: q * 2 < kv -> kv <= 4096; otherwise kv <= 2048.
    Each threshold can be overridden by its environment variable
    (SAGEATTN_DIRECT_THRESHOLD_D64[_CAUSAL|_CROSS], ..._D128[_CROSS]); a
    negative value disables the direct path for that case."""
    if head_dim == 64:
        d64_default = 2048 if tensor_layout == "HND" else 3072
        if is_causal:
            return kv_len <= _env_int("SAGEATTN_DIRECT_THRESHOLD_D64_CAUSAL", 6144)
        if q_len < kv_len:
            return kv_len <= _env_int("SAGEATTN_DIRECT_THRESHOLD_D64_CROSS", 6144)
        return kv_len <= _env_int("SAGEATTN_DIRECT_THRESHOLD_D64", d64_default)
    if q_len * 2 < kv_len:
        return kv_len <= _env_int("SAGEATTN_DIRECT_THRESHOLD_D128_CROSS", 4096)
    return kv_len <= _env_int("SAGEATTN_DIRECT_THRESHOLD_D128", 2048)


def sageattn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    tensor_layout: str = "HND",
    is_causal: bool = False,
    sm_scale: Optional[float] = None,
    return_lse: bool = False,
    **kwargs: Any,
) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """SageAttention: per-block INT8 Q/K (optional K-mean smoothing with
    ``smooth_k=True``), fp16 V, fused INT8-QK^T / fp16-PV flash attention; for
    short key ranges (:func:`use_direct_path`) the direct kernel on the fp16 /
    bf16 Q and K instead.

    q: [B,Hq,Sq,D] (HND) or [B,Sq,Hq,D] (NHD); k, v with Hkv heads (Hq % Hkv == 0).
    Returns o with q's shape, layout and dtype (and, when ``return_lse``, the
    rows' log-sum-exp [B,Hq,Sq] fp32: ln sum_j exp(sm_scale * q_i.k_j) after
    quantisation, -inf for a row with no key; the reference returns zeros).
    ``bm_sel`` (the reference's experimental direct-kernel tile override) is
    accepted and ignored; other unknown kwargs are ignored too.
    """
    dtype = q.dtype
    assert q.is_cuda, "Input tensors must be on CUDA/HIP device."
    assert dtype in [torch.float16, torch.bfloat16, torch.float32], (
        "Input tensors must be fp16, bf16, or fp32."
    )
    assert q.device == k.device == v.device, "All tensors must be on the same device."
    assert q.dtype == k.dtype == v.dtype, "All tensors must have the same dtype."

    headdim = q.size(-1)
    assert headdim in [64, 128], f"head_dim must be 64 or 128, got {headdim}."

    assert q.stride(-1) == 1 and k.stride(-1) == 1 and v.stride(-1) == 1, (
        "Last dim of qkv must be contiguous."
    )

    if sm_scale is None:
        sm_scale = headdim ** -0.5

    input_dtype = dtype
    if dtype == torch.float32:
        v = v.to(torch.float16)
        q = q.to(torch.float16)
        k = k.to(torch.float16)
        dtype = torch.float16

    _capi.load()

    assert q.stride(0) % 8 == 0 and q.stride(1) % 8 == 0 and q.stride(2) % 8 == 0, (
        "native backend requires q strides that are multiples of 8 halfs "
        "(16B aligned write-back). "
        f"Got strides={q.stride()}. Use contiguous tensors."
    )

    layout_code = ops.HND if tensor_layout == "HND" else ops.NHD
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k and v must be 4-D tensors")
    q = _vector_ready(q)
    k = _vector_ready(k)
    v = _vector_ready(v)
    (B, Hq, Sq, D), qst = ops._bhnd(q, layout_code)
    (Bk, Hkv, Sk, Dk), kst = ops._bhnd(k, layout_code)
    if tuple(k.shape) != tuple(v.shape) or Bk != B or Dk != D:
        raise ValueError(f"incompatible shapes q={tuple(q.shape)} k={tuple(k.shape)} v={tuple(v.shape)}")
    if Hq % Hkv != 0:
        raise ValueError(f"number of query heads ({Hq}) must be a multiple of kv heads ({Hkv})")
    vst = ops._bhnd(v, layout_code)[1]
    o = torch.empty_like(q)
    ost = ops._bhnd(o, layout_code)[1]
    dev = q.device

    lse = torch.empty((B, Hq, Sq), dtype=torch.float32, device=dev) if return_lse else None
    num_splits = _env_int("SAGEATTN_KV_SPLITS", 0)

    # the ops' launch helpers directly: the shapes, dtypes and layouts above already satisfy the
    # checks the public ops make (and the library checks every launch again)
    with ops._on_device(dev):
        stream = ops._stream(q)
        if use_direct_path(D, Sq, Sk, bool(is_causal), tensor_layout):
            # V transform: fp16 V_T [B,Hkv,D,ceil64(Sk)] zero padded (core.py:145-152,171-180)
            v_t = torch.empty(B, Hkv, D, (Sk + 63) // 64 * 64, device=dev, dtype=torch.float16)
            ops._v_layout_launch(v, v_t, B, Hkv, Sk, D, vst, stream)
            # direct kernel reads Q and K in place (core.py:141-164); K rows must not overlap
            if kst[2] < D:
                k = k.contiguous()
                kst = ops._bhnd(k, layout_code)[1]
            # fp16_attn_t / bf16_attn_t (core.py:153-164)
            ops._direct_launch(q, k, v_t, o, lse, B, Hq, Hkv, Sq, Sk, D, qst, kst, ost, is_causal, sm_scale,
                               num_splits, stream)
        else:
            smooth_k = kwargs.get("smooth_k", False)
            k_mean = ops.mean_seq(k, layout_code) if smooth_k and Sk > 0 else None
            # K quantisation and the V transform in one launch; Q is quantised inside the attention
            # kernel (the same q_int8 and q_scale as quant_qk_int8 would produce, so the same output,
            # without the int8 Q round trip)
            k_int8, k_scale, v_t = ops._prep_kv_launch(k, v, k_mean, B, Hkv, Sk, D, kst, vst, stream)
            # return_lse: the reference returns a zero placeholder (core.py:203-211); the fused kernel
            # writes the real log-sum-exp of each row (natural log, scaled scores; -inf for a row
            # without keys)
            ops._qfused_launch(q, k_int8, v_t, o, lse, k_scale, B, Hq, Hkv, Sq, Sk, D, qst, ost, is_causal,
                               sm_scale, num_splits, stream)

    if input_dtype == torch.float32:
        o = o.to(torch.float32)

    if return_lse:
        return o, lse

    return o


def sageattn_qk_int8_pv_fp16_cuda(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    tensor_layout: str = "HND",
    is_causal: bool = False,
    sm_scale: Optional[float] = None,
    return_lse: bool = False,
    **kwargs: Any,
) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """Upstream SageAttention name for the same kernel (core.py:216-233)."""
    return sageattn(
        q, k, v,
        tensor_layout=tensor_layout,
        is_causal=is_causal,
        sm_scale=sm_scale,
        return_lse=return_lse,
        **kwargs,
    )
