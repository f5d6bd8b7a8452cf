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


_host_mod = None


def _host():
    """The compiled host layer (``_sage_host.so``, built beside the library); no fallback."""
    global _host_mod
    if _host_mod is None:
        _capi.load()  # the library (and its ABI check) first; the module links against it
        try:
            from . import _sage_host
        except ImportError as e:
            raise RuntimeError(
                "sageattention host module (_sage_host.so) is not available. Build it with:\n"
                "  python sageattention-rdna3_amd/build.py\n"
                f"Original error: {e}"
            ) from e
        if _sage_host.abi_version() != _capi.ABI_VERSION:
            raise RuntimeError(f"_sage_host links ABI {_sage_host.abi_version()}, expected {_capi.ABI_VERSION}")
        _sage_host.set_error_type(_capi.SageError)
        _host_mod = _sage_host
    return _host_mod


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
    seq = 2 if layout_code == ops.HND else 1
    direct = use_direct_path(headdim, q.shape[seq], k.shape[seq], bool(is_causal), tensor_layout)

    # the rest of the call (shapes, allocations, the launches of the direct or the INT8 path) in one
    # compiled call over the C ABI (csrc/host_ops.cpp): direct = V transform + fp16_attn_t /
    # bf16_attn_t (core.py:141-164), or for fp16 inputs up to a measured key length one launch that reads V
    # in place (the same output bit for bit); INT8 = [K mean] + K quantisation and V transform in one launch +
    # the attention kernel that quantises Q itself (the q_int8 and q_scale of quant_qk_int8, so the same
    # output).  return_lse: the reference returns a zero placeholder (core.py:203-211); both kernels
    # write the real log-sum-exp of each row (natural log of the scaled scores; -inf without keys).
    with ops._on_device(q.device):
        res = _host().sageattn_fwd(q, k, v, layout_code, bool(is_causal), float(sm_scale), bool(return_lse),
                                   bool(kwargs.get("smooth_k", False)), direct,
                                   _env_int("SAGEATTN_KV_SPLITS", 0), ops._stream(q))
    o, lse = res if return_lse else (res, None)

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
