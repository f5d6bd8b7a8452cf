"""Drop-in ``sageattn`` for MI355X: the INT8 quantized path on gfx950 kernels.

Mirrors ``sageattention/core.py:40-233`` of the reference (same signature,
defaults, assertion messages, fp32 handling, ``smooth_k`` default False and
the upstream alias); ``return_lse`` returns the real log-sum-exp where the
reference returns a zero placeholder.  Every call takes the
INT8 path; the reference's Triton backend, ``SAGEATTN_BACKEND`` switch and the
direct fp16/bf16 branch (core.py:8,68-76,113-164) do not exist here.
"""
from __future__ import annotations

from typing import Any, Optional, Tuple, Union

import torch

from . import _capi, ops


def _vector_ready(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` or a copy that satisfies the 16-byte access contract
    (base aligned to 16 bytes, batch/head/token strides multiples of 8)."""
    if t.data_ptr() % 16 == 0 and all(s % 8 == 0 for s in t.stride()[:-1]):
        return t
    return t.contiguous() if not t.is_contiguous() else t.clone()


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
    """Quantized attention: per-block INT8 Q/K (optional K-mean smoothing with
    ``smooth_k=True``), fp16 V, fused INT8-QK^T / fp16-PV flash attention.

    q: [B,Hq,Sq,D] (HND) or [B,Sq,Hq,D] (NHD); k, v with Hkv heads (Hq % Hkv == 0).
    Returns o with q's shape, layout and dtype (and, when ``return_lse``, the
    rows' log-sum-exp [B,Hq,Sq] fp32: ln sum_j exp(sm_scale * q_i.k_j) after
    quantisation, -inf for a row with no key; the reference returns zeros).
    Unknown kwargs are ignored.
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
    (B, Hq, Sq, D), _ = ops._bhnd(q, layout_code)
    (Bk, Hkv, Sk, Dk), _ = ops._bhnd(k, layout_code)
    if tuple(k.shape) != tuple(v.shape) or Bk != B or Dk != D:
        raise ValueError(f"incompatible shapes q={tuple(q.shape)} k={tuple(k.shape)} v={tuple(v.shape)}")
    if Hq % Hkv != 0:
        raise ValueError(f"number of query heads ({Hq}) must be a multiple of kv heads ({Hkv})")

    q = _vector_ready(q)
    k = _vector_ready(k)
    v = _vector_ready(v)
    o = torch.empty_like(q)

    # V transform: fp16 V_T [B,Hkv,D,ceil64(Sk)] zero padded (core.py:171-180)
    padded_n = (Sk + 63) // 64 * 64
    v_t = torch.empty(B, Hkv, D, padded_n, device=q.device, dtype=torch.float16)
    ops.v_transpose(v, v_t, layout_code)

    smooth_k = kwargs.get("smooth_k", False)
    if smooth_k and Sk > 0:
        k_mean = ops.mean_seq(k, layout_code)
    else:
        k_mean = torch.empty(0, device=q.device, dtype=q.dtype)
    q_int8, q_scale, k_int8, k_scale = ops.quant_qk_int8(q, k, k_mean, layout_code, sm_scale)
    # return_lse: the reference returns a zero placeholder (core.py:203-211); the fused kernel writes
    # the real log-sum-exp of each row (natural log, scaled scores; -inf for a row without keys)
    lse = torch.empty((B, Hq, Sq), dtype=torch.float32, device=q.device) if return_lse else None
    ops.qk_int8_sv_bf16_attn_t(q_int8, k_int8, v_t, o, q_scale, k_scale,
                               layout_code, int(is_causal), sm_scale, lse=lse)

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
