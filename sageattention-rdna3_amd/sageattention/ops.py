"""Op-level API mirroring the reference's ``torch.ops.sageattention`` ops.

Same names, argument meaning and output shapes as the reference op layer
(csrc/pybind_gfx11.cpp:18-38, csrc/attn_gfx11.h:10-51); each op runs the gfx950
kernel behind the matching C-ABI entry point on the tensors' current HIP
stream.  ``tensor_layout`` is the reference's integer code: 1 = HND
([B,H,N,D]), 0 = NHD ([B,N,H,D]) (csrc/attn_gfx11.cu:32-33).
"""
from __future__ import annotations

import contextlib
import ctypes
import functools
from typing import List, Optional

import torch

from . import _capi

HND = 1
NHD = 0

_DTYPES = {torch.float16: _capi.DTYPE_F16, torch.bfloat16: _capi.DTYPE_BF16}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"expected fp16 or bf16 tensor, got {t.dtype}") from None


def _bhnd(t: torch.Tensor, tensor_layout: int):
    """(B, H, N, D) sizes and (stride_b, stride_h, stride_n) of a 4-D tensor."""
    if t.dim() != 4:
        raise ValueError(f"expected a 4-D tensor, got shape {tuple(t.shape)}")
    n, st = t.shape, t.stride()
    if tensor_layout == HND:
        return (n[0], n[1], n[2], n[3]), (st[0], st[1], st[2])
    return (n[0], n[2], n[1], n[3]), (st[0], st[2], st[1])


# the raw handle of a device's current stream; the public torch.cuda.current_stream(device) builds a
# Stream object first (~1.7 us a call, against ~0.1 us)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    """Handle of the current HIP stream on ``t``'s device (the stream every launch is ordered on)."""
    idx = t.device.index
    if idx is None:
        idx = torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(t.device).cuda_stream


def _on_device(dev: torch.device):
    """``torch.cuda.device(dev)``, or nothing when ``dev`` is already current (the common case; the
    context manager costs ~1 us per use).  The library reads the current device for its CU count."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(dev)


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


_NULL = None  # a null pointer argument


def mean_seq(input: torch.Tensor, tensor_layout: int) -> torch.Tensor:
    """K mean over the sequence -> [B,H,D] of input's dtype (reference mean_seq,
    csrc/attn_gfx11.cu:1937-1972)."""
    (B, H, S, D), (sb, sh, sn) = _bhnd(input, tensor_layout)
    out = torch.empty((B, H, D), dtype=input.dtype, device=input.device)
    lib = _capi.load()
    ws_bytes = lib.sage_k_mean_workspace_bytes(B, H, S, D)
    ws = torch.empty((max(ws_bytes, 4) + 3) // 4, dtype=torch.float32, device=input.device)
    with _on_device(input.device):
        _capi.call("sage_k_mean", _ptr(input), _ptr(out), _ptr(ws), _dtype_code(input),
                   B, H, S, D, sb, sh, sn, _stream(input))
    return out


def quant_qk_int8(query: torch.Tensor, key: torch.Tensor, key_mean: torch.Tensor,
                  tensor_layout: int, sm_scale: float) -> List[torch.Tensor]:
    """Per-block INT8 quantisation -> [q_int8, q_scale, k_int8, k_scale] (reference
    quant_qk_int8, csrc/attn_gfx11.cu:1974-2067).  ``key_mean`` empty -> no
    smoothing (csrc/attn_gfx11.cu:1996)."""
    (B, Hq, Sq, D), (qsb, qsh, qsn) = _bhnd(query, tensor_layout)
    (Bk, Hkv, Sk, Dk), (ksb, ksh, ksn) = _bhnd(key, tensor_layout)
    if Bk != B or Dk != D:
        raise ValueError(f"query {tuple(query.shape)} and key {tuple(key.shape)} disagree")
    if query.dtype != key.dtype:
        raise ValueError("query and key must have the same dtype")
    dev = query.device
    q8 = torch.empty((B, Hq, Sq, D), dtype=torch.int8, device=dev)
    k8 = torch.empty((B, Hkv, Sk, D), dtype=torch.int8, device=dev)
    qs = torch.empty((B, Hq, (Sq + 31) // 32), dtype=torch.float32, device=dev)
    ks = torch.empty((B, Hkv, (Sk + 15) // 16), dtype=torch.float32, device=dev)
    has_mean = key_mean is not None and key_mean.numel() > 0
    if has_mean:
        if tuple(key_mean.shape) != (B, Hkv, D) or key_mean.dtype != key.dtype:
            raise ValueError(f"key_mean must be [{B},{Hkv},{D}] of {key.dtype}")
        key_mean = key_mean.contiguous()
    mean_ptr = _ptr(key_mean) if has_mean else _NULL
    with _on_device(dev):
        _capi.call("sage_quant_qk_i8", _ptr(query), _ptr(key), mean_ptr,
                   _ptr(q8), _ptr(qs), _ptr(k8), _ptr(ks), _dtype_code(query),
                   B, Hq, Hkv, Sq, Sk, D, qsb, qsh, qsn, ksb, ksh, ksn,
                   float(sm_scale), _stream(query))
    return [q8, qs, k8, ks]


def quant_k_int8(key: torch.Tensor, key_mean: torch.Tensor, tensor_layout: int) -> List[torch.Tensor]:
    """The K half of :func:`quant_qk_int8` -> [k_int8, k_scale] (this build's split of the reference
    op, for the fused-Q attention :func:`qk_int8_sv_bf16_attn_qfused_t`)."""
    (B, Hkv, Sk, D), (ksb, ksh, ksn) = _bhnd(key, tensor_layout)
    dev = key.device
    k8 = torch.empty((B, Hkv, Sk, D), dtype=torch.int8, device=dev)
    ks = torch.empty((B, Hkv, (Sk + 15) // 16), dtype=torch.float32, device=dev)
    has_mean = key_mean is not None and key_mean.numel() > 0
    if has_mean:
        if tuple(key_mean.shape) != (B, Hkv, D) or key_mean.dtype != key.dtype:
            raise ValueError(f"key_mean must be [{B},{Hkv},{D}] of {key.dtype}")
        key_mean = key_mean.contiguous()
    mean_ptr = _ptr(key_mean) if has_mean else _NULL
    null = _NULL
    with _on_device(dev):
        _capi.call("sage_quant_qk_i8", null, _ptr(key), mean_ptr, null, null, _ptr(k8), _ptr(ks),
                   _dtype_code(key), B, Hkv, Hkv, 0, Sk, D, 0, 0, 0, ksb, ksh, ksn, 1.0, _stream(key))
    return [k8, ks]


def prep_kv_int8(key: torch.Tensor, value: torch.Tensor, key_mean: torch.Tensor,
                 tensor_layout: int) -> List[torch.Tensor]:
    """:func:`quant_k_int8` and :func:`v_transpose` in one launch -> [k_int8, k_scale, value_t], the
    same tensors bit for bit (this build's fusion of the K half of the reference's quant_qk_int8 with
    its v_transpose, for :func:`qk_int8_sv_bf16_attn_qfused_t`)."""
    (B, Hkv, Sk, D), kst = _bhnd(key, tensor_layout)
    (Bv, Hv, Sv, Dv), vst = _bhnd(value, tensor_layout)
    if (Bv, Hv, Sv, Dv) != (B, Hkv, Sk, D) or value.dtype != key.dtype:
        raise ValueError("key and value must have the same shape and dtype")
    has_mean = key_mean is not None and key_mean.numel() > 0
    if has_mean:
        if tuple(key_mean.shape) != (B, Hkv, D) or key_mean.dtype != key.dtype:
            raise ValueError(f"key_mean must be [{B},{Hkv},{D}] of {key.dtype}")
        key_mean = key_mean.contiguous()
    with _on_device(key.device):
        return _prep_kv_launch(key, value, key_mean if has_mean else None, B, Hkv, Sk, D, kst, vst, _stream(key))


def _prep_kv_launch(key, value, key_mean, B, Hkv, Sk, D, kst, vst, stream) -> List[torch.Tensor]:
    """Allocate [k_int8, k_scale, value_t] and launch sage_prep_kv_i8 (arguments already checked)."""
    dev = key.device
    k8 = torch.empty((B, Hkv, Sk, D), dtype=torch.int8, device=dev)
    ks = torch.empty((B, Hkv, (Sk + 15) // 16), dtype=torch.float32, device=dev)
    vt = torch.empty((B, Hkv, D, (Sk + 63) // 64 * 64), dtype=torch.float16, device=dev)
    _capi.call("sage_prep_kv_i8", key.data_ptr(), value.data_ptr(),
               key_mean.data_ptr() if key_mean is not None else _NULL, k8.data_ptr(), ks.data_ptr(),
               vt.data_ptr(), _dtype_code(key), B, Hkv, Sk, D, *kst, *vst, stream)
    return [k8, ks, vt]


def prep_kv_int8_smooth(key: torch.Tensor, value: torch.Tensor, tensor_layout: int,
                        return_mean: bool = False) -> List[torch.Tensor]:
    """:func:`mean_seq` + :func:`prep_kv_int8` (K smoothed by its mean) in two launches instead of
    three -> [k_int8, k_scale, value_t] (+ key_mean with ``return_mean``), the same tensors bit for
    bit (this build's fusion of the reference's mean_seq, csrc/attn_gfx11.cu:1937-1972, with the K
    half of quant_qk_int8 and v_transpose; sageattention/core.py:186-193)."""
    (B, Hkv, Sk, D), kst = _bhnd(key, tensor_layout)
    (Bv, Hv, Sv, Dv), vst = _bhnd(value, tensor_layout)
    if (Bv, Hv, Sv, Dv) != (B, Hkv, Sk, D) or value.dtype != key.dtype:
        raise ValueError("key and value must have the same shape and dtype")
    dev = key.device
    k8 = torch.empty((B, Hkv, Sk, D), dtype=torch.int8, device=dev)
    ks = torch.empty((B, Hkv, (Sk + 15) // 16), dtype=torch.float32, device=dev)
    vt = torch.empty((B, Hkv, D, (Sk + 63) // 64 * 64), dtype=torch.float16, device=dev)
    mean = torch.empty((B, Hkv, D), dtype=key.dtype, device=dev) if return_mean else None
    lib = _capi.load()
    ws_bytes = lib.sage_k_mean_workspace_bytes(B, Hkv, Sk, D)
    ws = torch.empty((max(ws_bytes, 4) + 3) // 4, dtype=torch.float32, device=dev)
    with _on_device(dev):
        _capi.call("sage_prep_kv_i8_smooth", key.data_ptr(), value.data_ptr(),
                   mean.data_ptr() if mean is not None else _NULL, ws.data_ptr(), k8.data_ptr(), ks.data_ptr(),
                   vt.data_ptr(), _dtype_code(key), B, Hkv, Sk, D, *kst, *vst, _stream(key))
    return [k8, ks, vt, mean] if return_mean else [k8, ks, vt]


def v_transpose(value: torch.Tensor, value_t: torch.Tensor, tensor_layout: int) -> torch.Tensor:
    """V -> fp16 V_T [B,H,D,ceil64(N)] written into ``value_t`` (reference
    v_transpose, csrc/attn_gfx11.cu:1889-1935)."""
    (B, H, S, D), vst = _bhnd(value, tensor_layout)
    NP = (S + 63) // 64 * 64
    if (tuple(value_t.shape) != (B, H, D, NP) or value_t.dtype != torch.float16
            or not value_t.is_contiguous()):
        raise ValueError(f"value_t must be contiguous fp16 [{B},{H},{D},{NP}]")
    with _on_device(value.device):
        _v_layout_launch(value, value_t, B, H, S, D, vst, _stream(value))
    return value_t


def _v_layout_launch(value, value_t, B, H, S, D, vst, stream) -> None:
    _capi.call("sage_v_layout", value.data_ptr(), value_t.data_ptr(), _dtype_code(value), B, H, S, D, *vst,
               stream)


def qk_int8_sv_bf16_attn_t(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                           output: torch.Tensor, q_scale: torch.Tensor, k_scale: torch.Tensor,
                           tensor_layout: int, is_causal: int, sm_scale: float,
                           lse: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused attention over quantised Q/K and V_T into ``output`` (reference
    qk_int8_sv_bf16_attn_t, csrc/attn_gfx11.cu:2069-2273).  ``sm_scale`` is
    unused: it is already folded into ``q_scale`` (as in the reference).
    ``lse`` (this build's addition; contiguous fp32 [B,Hq,Sq]) receives each
    row's natural-log log-sum-exp of the scaled scores."""
    B, Hq, Sq, D = query.shape
    Bk, Hkv, Sk, Dk = key.shape
    if Bk != B or Dk != D:
        raise ValueError("query/key int8 tensors disagree")
    for name, t in (("query", query), ("key", key)):
        if t.dtype != torch.int8 or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous int8 [B,H,N,D]")
    NP = (Sk + 63) // 64 * 64
    if tuple(value.shape) != (B, Hkv, D, NP) or value.dtype != torch.float16 or not value.is_contiguous():
        raise ValueError(f"value must be contiguous fp16 V_T [{B},{Hkv},{D},{NP}]")
    if (tuple(q_scale.shape) != (B, Hq, (Sq + 31) // 32) or tuple(k_scale.shape) != (B, Hkv, (Sk + 15) // 16)
            or q_scale.dtype != torch.float32 or k_scale.dtype != torch.float32
            or not q_scale.is_contiguous() or not k_scale.is_contiguous()):
        raise ValueError("q_scale/k_scale must be contiguous fp32 [B,H,ceil(N/32)] / [B,H,ceil(N/16)]")
    (Bo, Ho, So, Do), (osb, osh, osn) = _bhnd(output, tensor_layout)
    if (Bo, Ho, So, Do) != (B, Hq, Sq, D) or output.stride(-1) != 1:
        raise ValueError("output shape does not match the query")
    if lse is not None:
        if tuple(lse.shape) != (B, Hq, Sq) or lse.dtype != torch.float32 or not lse.is_contiguous():
            raise ValueError(f"lse must be contiguous fp32 [{B},{Hq},{Sq}]")
        with _on_device(query.device):
            _capi.call("sage_attn_i8_fwd_lse", _ptr(query), _ptr(key), _ptr(value), _ptr(output), _ptr(lse),
                       _ptr(q_scale), _ptr(k_scale), _dtype_code(output),
                       B, Hq, Hkv, Sq, Sk, D, osb, osh, osn, int(bool(is_causal)), _stream(query))
        return output
    with _on_device(query.device):
        _capi.call("sage_attn_i8_fwd", _ptr(query), _ptr(key), _ptr(value), _ptr(output),
                   _ptr(q_scale), _ptr(k_scale), _dtype_code(output),
                   B, Hq, Hkv, Sq, Sk, D, osb, osh, osn, int(bool(is_causal)), _stream(query))
    return output


@functools.lru_cache(maxsize=256)
def _workspace_bytes(quantized: int, B: int, Hq: int, Sq: int, Sk: int, D: int, is_causal: int, num_splits: int,
                     device_index: int) -> int:
    # the plan depends on the shape and on the device (its CU count) only
    return _capi.query("sage_attn_workspace_bytes", quantized, B, Hq, Sq, Sk, D, is_causal, num_splits)


def _split_workspace(quantized: bool, B: int, Hq: int, Sq: int, Sk: int, D: int, is_causal: int,
                     num_splits: int, device: torch.device):
    """Workspace for the key-split path of a non-causal launch (None when it runs unsplit).  Called
    with ``device`` current: the library's split choice depends on its CU count."""
    if not 0 <= int(num_splits) <= _capi.MAX_KV_SPLITS:
        raise ValueError(f"num_splits must be in [0, {_capi.MAX_KV_SPLITS}], got {num_splits}")
    if is_causal:
        return None, _NULL, 0  # causal launches never split
    nbytes = _workspace_bytes(int(quantized), B, Hq, Sq, Sk, D, 0, int(num_splits),
                              device.index if device.index is not None else torch.cuda.current_device())
    if nbytes == 0:
        return None, _NULL, 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    return ws, ws.data_ptr(), nbytes


def _direct_attn_t(op: str, want: torch.dtype, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                   output: torch.Tensor, tensor_layout: int, is_causal: int, sm_scale: float,
                   lse: Optional[torch.Tensor], num_splits: int = 0) -> torch.Tensor:
    for name, t in (("query", query), ("key", key), ("output", output)):
        if t.dtype != want:
            raise ValueError(f"{op}: {name} must be {want}, got {t.dtype}")
        if t.dim() != 4 or t.stride(-1) != 1:
            raise ValueError(f"{op}: {name} must be 4-D with a contiguous head_dim axis")
    (B, Hq, Sq, D), qst = _bhnd(query, tensor_layout)
    (Bk, Hkv, Sk, Dk), kst = _bhnd(key, tensor_layout)
    if Bk != B or Dk != D:
        raise ValueError(f"{op}: query {tuple(query.shape)} and key {tuple(key.shape)} disagree")
    NP = (Sk + 63) // 64 * 64
    if tuple(value.shape) != (B, Hkv, D, NP) or value.dtype != torch.float16 or not value.is_contiguous():
        raise ValueError(f"{op}: value must be contiguous fp16 V_T [{B},{Hkv},{D},{NP}]")
    (Bo, Ho, So, Do), ost = _bhnd(output, tensor_layout)
    if (Bo, Ho, So, Do) != (B, Hq, Sq, D):
        raise ValueError(f"{op}: output shape does not match the query")
    if lse is not None:
        if tuple(lse.shape) != (B, Hq, Sq) or lse.dtype != torch.float32 or not lse.is_contiguous():
            raise ValueError(f"{op}: lse must be contiguous fp32 [{B},{Hq},{Sq}]")
    with _on_device(query.device):
        _direct_launch(query, key, value, output, lse, B, Hq, Hkv, Sq, Sk, D, qst, kst, ost, is_causal,
                       sm_scale, num_splits, _stream(query))
    return output


def _direct_launch(query, key, value_t, output, lse, B, Hq, Hkv, Sq, Sk, D, qst, kst, ost, is_causal, sm_scale,
                   num_splits, stream) -> None:
    """sage_attn_direct_fwd on checked arguments, with the key-split workspace when the plan needs one
    (the device must be current)."""
    ws, ws_ptr, ws_bytes = _split_workspace(False, B, Hq, Sq, Sk, D, is_causal, num_splits, query.device)
    _capi.call("sage_attn_direct_fwd", query.data_ptr(), key.data_ptr(), value_t.data_ptr(), output.data_ptr(),
               lse.data_ptr() if lse is not None else _NULL, _dtype_code(query), B, Hq, Hkv, Sq, Sk, D,
               *qst, *kst, *ost, int(bool(is_causal)), float(sm_scale), int(num_splits), ws_ptr, ws_bytes, stream)
    del ws  # stream-ordered: the caching allocator hands it out again only behind this launch


def fp16_attn_t(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, output: torch.Tensor,
                tensor_layout: int, is_causal: int, sm_scale: float, bm_sel: int = 0,
                lse: Optional[torch.Tensor] = None, num_splits: int = 0) -> torch.Tensor:
    """Direct attention on fp16 Q/K (no quantisation) and the fp16 V_T of
    :func:`v_transpose` into fp16 ``output`` (reference fp16_attn_t,
    csrc/attn_gfx11.cu:2275-2374).  ``bm_sel`` (the reference's experimental
    tile override) is accepted and ignored: gfx950 uses one tile shape.
    ``lse`` as in :func:`qk_int8_sv_bf16_attn_t`.  ``num_splits`` (this
    build's): key splits of a non-causal launch, 0 = the library's choice for
    the device, 1 = unsplit, n = n (the workspace is allocated here)."""
    return _direct_attn_t("fp16_attn_t", torch.float16, query, key, value, output, tensor_layout, is_causal,
                          sm_scale, lse, num_splits)


def bf16_attn_t(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, output: torch.Tensor,
                tensor_layout: int, is_causal: int, sm_scale: float, bm_sel: int = 0,
                lse: Optional[torch.Tensor] = None, num_splits: int = 0) -> torch.Tensor:
    """bf16 counterpart of :func:`fp16_attn_t`: bf16 Q/K/output, fp16 V_T and
    P (reference bf16_attn_t, csrc/attn_gfx11.cu:2376-2472)."""
    return _direct_attn_t("bf16_attn_t", torch.bfloat16, query, key, value, output, tensor_layout, is_causal,
                          sm_scale, lse, num_splits)


def fp16_attn_vrows(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, output: torch.Tensor,
                    tensor_layout: int, is_causal: int, sm_scale: float,
                    lse: Optional[torch.Tensor] = None, num_splits: int = 0) -> torch.Tensor:
    """:func:`fp16_attn_t` with ``value`` the caller's fp16 V itself (``[B, Hkv, Sk, D]`` in
    ``tensor_layout``, read through its strides) instead of a V_T from :func:`v_transpose`: the kernel
    transposes V tiles in LDS, so the short-sequence branch is one launch.  Same result bit for bit as
    ``v_transpose`` followed by :func:`fp16_attn_t`.  This build's fusion; it replaces the reference's
    v_transpose + fp16_attn_t pair (core.py:141-164) for fp16 inputs."""
    op = "fp16_attn_vrows"
    for name, t in (("query", query), ("key", key), ("value", value), ("output", output)):
        if t.dtype != torch.float16:
            raise ValueError(f"{op}: {name} must be torch.float16, got {t.dtype}")
        if t.dim() != 4 or t.stride(-1) != 1:
            raise ValueError(f"{op}: {name} must be 4-D with a contiguous head_dim axis")
    (B, Hq, Sq, D), qst = _bhnd(query, tensor_layout)
    (Bk, Hkv, Sk, Dk), kst = _bhnd(key, tensor_layout)
    if Bk != B or Dk != D:
        raise ValueError(f"{op}: query {tuple(query.shape)} and key {tuple(key.shape)} disagree")
    (Bv, Hv, Sv, Dv), vst = _bhnd(value, tensor_layout)
    if (Bv, Hv, Sv, Dv) != (B, Hkv, Sk, D):
        raise ValueError(f"{op}: value must be [{B},{Hkv},{Sk},{D}] in the tensor layout")
    (Bo, Ho, So, Do), ost = _bhnd(output, tensor_layout)
    if (Bo, Ho, So, Do) != (B, Hq, Sq, D):
        raise ValueError(f"{op}: output shape does not match the query")
    if lse is not None:
        if tuple(lse.shape) != (B, Hq, Sq) or lse.dtype != torch.float32 or not lse.is_contiguous():
            raise ValueError(f"{op}: lse must be contiguous fp32 [{B},{Hq},{Sq}]")
    with _on_device(query.device):
        ws, ws_ptr, ws_bytes = _split_workspace(False, B, Hq, Sq, Sk, D, is_causal, num_splits, query.device)
        _capi.call("sage_attn_direct_fwd_vrows", query.data_ptr(), key.data_ptr(), value.data_ptr(),
                   output.data_ptr(), lse.data_ptr() if lse is not None else _NULL, _dtype_code(query), B, Hq, Hkv,
                   Sq, Sk, D, *qst, *kst, *vst, *ost, int(bool(is_causal)), float(sm_scale), int(num_splits),
                   ws_ptr, ws_bytes, _stream(query))
        del ws  # stream-ordered reuse, as in _direct_launch
    return output


def qk_int8_sv_bf16_attn_qfused_t(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                                  output: torch.Tensor, k_scale: torch.Tensor, tensor_layout: int,
                                  is_causal: int, sm_scale: float,
                                  lse: Optional[torch.Tensor] = None, num_splits: int = 0) -> torch.Tensor:
    """:func:`quant_qk_int8` (Q half) + :func:`qk_int8_sv_bf16_attn_t` in one kernel: ``query`` is
    the fp16/bf16 Q in ``tensor_layout``, quantised inside the attention kernel exactly as the quant
    op would (same q_int8 and q_scale, so the same output bit for bit); ``key``/``k_scale`` come
    from :func:`quant_k_int8`, ``value`` is the fp16 V_T.  ``num_splits`` as in :func:`fp16_attn_t`
    (the bit-identity with the two-kernel path holds for unsplit launches).  This build's fusion; no
    single reference op."""
    (B, Hq, Sq, D), qst = _bhnd(query, tensor_layout)
    if query.stride(-1) != 1 or output.dtype != query.dtype:
        raise ValueError("query needs a contiguous head_dim axis and the output's dtype")
    Bk, Hkv, Sk, Dk = key.shape
    if Bk != B or Dk != D or key.dtype != torch.int8 or not key.is_contiguous():
        raise ValueError("key must be contiguous int8 [B,Hkv,Sk,D]")
    NP = (Sk + 63) // 64 * 64
    if tuple(value.shape) != (B, Hkv, D, NP) or value.dtype != torch.float16 or not value.is_contiguous():
        raise ValueError(f"value must be contiguous fp16 V_T [{B},{Hkv},{D},{NP}]")
    if (tuple(k_scale.shape) != (B, Hkv, (Sk + 15) // 16) or k_scale.dtype != torch.float32
            or not k_scale.is_contiguous()):
        raise ValueError("k_scale must be contiguous fp32 [B,Hkv,ceil(Sk/16)]")
    (Bo, Ho, So, Do), ost = _bhnd(output, tensor_layout)
    if (Bo, Ho, So, Do) != (B, Hq, Sq, D) or output.stride(-1) != 1:
        raise ValueError("output shape does not match the query")
    if lse is not None:
        if tuple(lse.shape) != (B, Hq, Sq) or lse.dtype != torch.float32 or not lse.is_contiguous():
            raise ValueError(f"lse must be contiguous fp32 [{B},{Hq},{Sq}]")
    with _on_device(query.device):
        _qfused_launch(query, key, value, output, lse, k_scale, B, Hq, Hkv, Sq, Sk, D, qst, ost, is_causal,
                       sm_scale, num_splits, _stream(query))
    return output


def _qfused_launch(query, key, value_t, output, lse, k_scale, B, Hq, Hkv, Sq, Sk, D, qst, ost, is_causal,
                   sm_scale, num_splits, stream) -> None:
    """sage_attn_i8_fwd_qfused on checked arguments, with the key-split workspace when the plan needs
    one (the device must be current)."""
    ws, ws_ptr, ws_bytes = _split_workspace(True, B, Hq, Sq, Sk, D, is_causal, num_splits, query.device)
    _capi.call("sage_attn_i8_fwd_qfused", query.data_ptr(), key.data_ptr(), value_t.data_ptr(),
               output.data_ptr(), lse.data_ptr() if lse is not None else _NULL, k_scale.data_ptr(),
               _dtype_code(query), B, Hq, Hkv, Sq, Sk, D, *qst, *ost, int(bool(is_causal)), float(sm_scale),
               int(num_splits), ws_ptr, ws_bytes, stream)
    del ws  # stream-ordered: the caching allocator hands it out again only behind this launch


def qk_int8_sv_f16_attn_qfused_vrows(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                                     output: torch.Tensor, k_scale: torch.Tensor, tensor_layout: int,
                                     is_causal: int, sm_scale: float,
                                     lse: Optional[torch.Tensor] = None, num_splits: int = 0) -> torch.Tensor:
    """:func:`qk_int8_sv_bf16_attn_qfused_t` for fp16 inputs with ``value`` the caller's fp16 V itself
    (``[B, Hkv, Sk, D]`` in ``tensor_layout``, read through its strides) instead of a V_T from
    :func:`v_transpose`: the kernel transposes V tiles in LDS, so the V layout pass is skipped.  Same
    result bit for bit as ``v_transpose`` followed by :func:`qk_int8_sv_bf16_attn_qfused_t`.  This build's
    fusion; it replaces the reference's v_transpose + INT8 attention pair (core.py:173-179,190-197) for
    fp16 V."""
    (B, Hq, Sq, D), qst = _bhnd(query, tensor_layout)
    if query.dtype != torch.float16 or output.dtype != torch.float16 or value.dtype != torch.float16:
        raise ValueError("query, value and output must be fp16 (V is read as fp16 in place)")
    if query.stride(-1) != 1:
        raise ValueError("query needs a contiguous head_dim axis")
    Bk, Hkv, Sk, Dk = key.shape
    if Bk != B or Dk != D or key.dtype != torch.int8 or not key.is_contiguous():
        raise ValueError("key must be contiguous int8 [B,Hkv,Sk,D]")
    (Bv, Hv, Sv, Dv), vst = _bhnd(value, tensor_layout)
    if (Bv, Hv, Sv, Dv) != (B, Hkv, Sk, D) or value.stride(-1) != 1:
        raise ValueError(f"value must be fp16 [{B},{Hkv},{Sk},{D}] in the tensor layout with a contiguous head_dim")
    if (tuple(k_scale.shape) != (B, Hkv, (Sk + 15) // 16) or k_scale.dtype != torch.float32
            or not k_scale.is_contiguous()):
        raise ValueError("k_scale must be contiguous fp32 [B,Hkv,ceil(Sk/16)]")
    (Bo, Ho, So, Do), ost = _bhnd(output, tensor_layout)
    if (Bo, Ho, So, Do) != (B, Hq, Sq, D) or output.stride(-1) != 1:
        raise ValueError("output shape does not match the query")
    if lse is not None:
        if tuple(lse.shape) != (B, Hq, Sq) or lse.dtype != torch.float32 or not lse.is_contiguous():
            raise ValueError(f"lse must be contiguous fp32 [{B},{Hq},{Sq}]")
    with _on_device(query.device):
        ws, ws_ptr, ws_bytes = _split_workspace(True, B, Hq, Sq, Sk, D, is_causal, num_splits, query.device)
        _capi.call("sage_attn_i8_fwd_qfused_vrows", query.data_ptr(), key.data_ptr(), value.data_ptr(),
                   output.data_ptr(), lse.data_ptr() if lse is not None else _NULL, k_scale.data_ptr(),
                   _dtype_code(query), B, Hq, Hkv, Sq, Sk, D, *qst, *vst, *ost, int(bool(is_causal)),
                   float(sm_scale), int(num_splits), ws_ptr, ws_bytes, _stream(query))
        del ws  # stream-ordered reuse, as in _qfused_launch
    return output


# ---- torch.ops.sageattention: the reference's op namespace with its schemas (csrc/pybind_gfx11.cpp:18-47),
# backed by the functions above (their extra keyword arguments keep their defaults), for callers that use the
# op namespace directly.  Nothing is registered when the namespace is already taken (for instance by the
# reference's own extension loaded into the same process).
_SCHEMAS = {
    "qk_int8_sv_bf16_attn_t": "qk_int8_sv_bf16_attn_t(Tensor query, Tensor key, Tensor value, Tensor(a!) output, "
                              "Tensor q_scale, Tensor k_scale, int tensor_layout, int is_causal, float sm_scale"
                              ") -> Tensor",
    "fp16_attn_t": "fp16_attn_t(Tensor query, Tensor key, Tensor value, Tensor(a!) output, int tensor_layout, "
                   "int is_causal, float sm_scale, int bm_sel) -> Tensor",
    "bf16_attn_t": "bf16_attn_t(Tensor query, Tensor key, Tensor value, Tensor(a!) output, int tensor_layout, "
                   "int is_causal, float sm_scale, int bm_sel) -> Tensor",
    "quant_qk_int8": "quant_qk_int8(Tensor query, Tensor key, Tensor key_mean, int tensor_layout, float sm_scale"
                     ") -> Tensor[]",
    "mean_seq": "mean_seq(Tensor input, int tensor_layout) -> Tensor",
    "v_transpose": "v_transpose(Tensor value, Tensor(a!) value_t, int tensor_layout) -> Tensor",
}


def _register_torch_ops():
    try:
        lib = torch.library.Library("sageattention", "DEF")
    except RuntimeError:
        return None
    impls = {"qk_int8_sv_bf16_attn_t": qk_int8_sv_bf16_attn_t, "fp16_attn_t": fp16_attn_t,
             "bf16_attn_t": bf16_attn_t, "quant_qk_int8": quant_qk_int8, "mean_seq": mean_seq,
             "v_transpose": v_transpose}
    for name, schema in _SCHEMAS.items():
        lib.define(schema)
        lib.impl(name, impls[name], "CUDA")
    return lib


_TORCH_LIBRARY = _register_torch_ops()
