"""PyTorch CPU implementation of the quantized attention math: the CPU baseline that ``bench.py`` times.

Test infrastructure like the rest of ``oracle/``: only ``bench.py``'s ``cpu_baseline`` leg and ``tests/`` use
it, and no product path imports it.  The reference has no CPU path (``sageattention/core.py:51`` requires a GPU
tensor), so the baseline is this restatement of the same algorithm in torch fp32 on the host cores:

* per-block INT8 quantisation (csrc/attn_gfx11.cu:85-92,147-321 of the reference): Q in 32-token groups with
  the pre-scale fl(fl(sm_scale) * log2 e), K in 16-token groups (minus the K mean for smooth_k),
  amax = max(1e-7, max|x|), scale = amax / 127, q8 = round-half-away(x * (127 / amax) [* pre]) -- the same fp32
  operations, in the same order, as ``sage_oracle.quant_per_block`` (bit-identical on finite inputs;
  ``tests/test_oracle.py`` checks it);
* the V layout: V -> fp16 (csrc/attn_gfx11.cu:323-407);
* attention (csrc/attn_gfx11.cu:409-825): exact integer QK^T (an fp32 GEMM of int8 values is exact below
  2^24), s = fl(acc * fl(qs * ks)) in the log2 domain, an online softmax over key blocks with exp2, the row sum
  from unrounded p, P rounded to fp16 before P.V, fp32 accumulation, O / l.  Blockwise over keys, so no S x S
  matrix exists; causal query blocks stop at their diagonal key block.
"""
from __future__ import annotations

import math

import torch

Q_GROUP = 32
K_GROUP = 16
AMAX_FLOOR = 1e-7
LOG2E = 1.4426950408889634


def _f32(x: float) -> torch.Tensor:
    return torch.tensor(x, dtype=torch.float32)


def quant_per_block(x: torch.Tensor, group: int, pre: float | None = None, mean: torch.Tensor | None = None):
    """x fp32 [B,H,S,D] -> (int8 [B,H,S,D], fp32 scales [B,H,ceil(S/group)])."""
    B, H, S, D = x.shape
    G = -(-S // group)
    v = x if mean is None else x - mean[:, :, None, :]
    pre_t = None if pre is None else _f32(pre)
    a = (v * pre_t).abs() if pre_t is not None else v.abs()
    pad = G * group - S
    if pad:
        a = torch.cat([a, a.new_zeros(B, H, pad, D)], dim=2)
    amax = a.reshape(B, H, G, group * D).amax(dim=-1).clamp_min(AMAX_FLOOR)
    scale = amax / _f32(127.0)
    inv = _f32(127.0) / amax
    iscale = inv * pre_t if pre_t is not None else inv
    t = v * iscale.repeat_interleave(group, dim=2)[:, :, :S, None]
    u = t + torch.where(t >= 0, _f32(0.5), _f32(-0.5))
    return u.trunc().clamp(-128, 127).to(torch.int8), scale


def quant_qk(q: torch.Tensor, k: torch.Tensor, sm_scale: float, smooth_k: bool = False):
    """q, k fp16/bf16 [B,H,S,D] (HND) -> q8, q_scale, k8, k_scale (and the K mean used, or None)."""
    pre = float(_f32(sm_scale) * _f32(LOG2E))
    q32, k32 = q.float(), k.float()
    mean = None
    if smooth_k:
        mean = (k32.sum(dim=2) / _f32(k.shape[2])).to(k.dtype).float()
    q8, qs = quant_per_block(q32, Q_GROUP, pre=pre)
    k8, ks = quant_per_block(k32, K_GROUP, mean=mean)
    return q8, qs, k8, ks, mean


def attn_i8_head(q8: torch.Tensor, k8: torch.Tensor, v16: torch.Tensor, qs: torch.Tensor, ks: torch.Tensor,
                 causal: bool, block: int = 512) -> torch.Tensor:
    """One head: q8 [Sq,D], k8 [Sk,D] int8, v16 [Sk,D] fp16, qs [ceil(Sq/32)], ks [ceil(Sk/16)] -> fp32
    [Sq,D] (before the output cast)."""
    Sq, D = q8.shape
    Sk = k8.shape[0]
    out = torch.zeros(Sq, D, dtype=torch.float32)
    kf = k8.float()
    vf = v16.float()
    ks_col = ks.repeat_interleave(K_GROUP)[:Sk]
    for r0 in range(0, Sq, block):
        r1 = min(Sq, r0 + block)
        qf = q8[r0:r1].float()
        qs_row = qs.repeat_interleave(Q_GROUP)[r0:r1]
        m = torch.full((r1 - r0, 1), -math.inf)
        l = torch.zeros(r1 - r0, 1)
        o = torch.zeros(r1 - r0, D)
        kend = min(Sk, r1) if causal else Sk
        for c0 in range(0, kend, block):
            c1 = min(kend, c0 + block)
            s = (qf @ kf[c0:c1].T) * (qs_row[:, None] * ks_col[None, c0:c1])
            if causal and c1 > r0:
                rows = torch.arange(r0, r1)[:, None]
                cols = torch.arange(c0, c1)[None, :]
                s = s.masked_fill(cols > rows, -math.inf)
            m_new = torch.maximum(m, s.amax(dim=1, keepdim=True))
            m_use = torch.where(torch.isfinite(m_new), m_new, torch.zeros_like(m_new))
            alpha = torch.exp2(m - m_use)
            p = torch.exp2(s - m_use)
            l = l * alpha + p.sum(dim=1, keepdim=True)
            o = o * alpha + p.half().float() @ vf[c0:c1]
            m = m_new
        out[r0:r1] = torch.where(l > 0, o / torch.where(l > 0, l, torch.ones_like(l)), torch.zeros_like(o))
    return out


def sageattn_heads(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, sm_scale: float,
                   smooth_k: bool = False, heads=None, block: int = 512) -> torch.Tensor:
    """The whole quantized path for the listed query heads of batch 0 (HND inputs): quantisation of those
    heads' Q and their K/V heads, the V layout, attention.  Returns fp32 [len(heads), Sq, D]."""
    B, Hq, Sq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    heads = list(range(Hq)) if heads is None else list(heads)
    kv_heads = sorted({h // G for h in heads})
    pre = float(_f32(sm_scale) * _f32(LOG2E))
    q8, qs = quant_per_block(q[:1, heads].float(), Q_GROUP, pre=pre)
    k32 = k[:1, kv_heads].float()
    mean = (k32.sum(dim=2) / _f32(k.shape[2])).to(k.dtype).float() if smooth_k else None
    k8, ks = quant_per_block(k32, K_GROUP, mean=mean)
    v16 = v[0, kv_heads].to(torch.float16)
    out = torch.empty(len(heads), Sq, D)
    for i, h in enumerate(heads):
        j = kv_heads.index(h // G)
        out[i] = attn_i8_head(q8[0, i], k8[0, j], v16[j], qs[0, i], ks[0, j], causal, block)
    return out
