"""Shared helpers of the test suite: configs, seeded inputs, conversions, metrics."""
from __future__ import annotations

import dataclasses
import math
from typing import Optional

import numpy as np
import torch

from oracle import sage_oracle as orc


@dataclasses.dataclass(frozen=True)
class Config:
    name: str
    B: int
    Hq: int
    Hkv: int
    S: int
    D: int
    dtype: str  # "fp16" | "bf16" | "fp32"
    layout: str  # "HND" | "NHD"
    causal: bool
    smooth_k: bool
    k_offset_std: float = 0.0  # per-(b,h,d) DC offset of K
    outlier_frac: float = 0.0  # fraction of channels scaled x20 in Q and K (config 5)
    Sq: Optional[int] = None  # cross-attention query length (default S)

    @property
    def q_len(self) -> int:
        return self.S if self.Sq is None else self.Sq


# BASELINE.json configs (C1 is the CPU plumbing case) and the north-star shape.
C1 = Config("C1", 1, 2, 2, 256, 64, "fp16", "HND", False, False)
C2 = Config("C2", 1, 10, 10, 4096, 64, "fp16", "HND", False, False)
C3 = Config("C3", 2, 32, 32, 8192, 128, "bf16", "HND", True, True, k_offset_std=2.0)
C4 = Config("C4", 1, 32, 8, 16384, 128, "fp16", "NHD", True, False)
C5 = Config("C5", 1, 40, 40, 32891, 128, "bf16", "HND", False, True, outlier_frac=0.01)
NS = Config("NS", 1, 32, 32, 16384, 128, "bf16", "HND", True, False)
BASELINE_CONFIGS = [C1, C2, C3, C4, C5, NS]

TORCH_DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


def shape_of(cfg: Config, heads: int, seq: int):
    if cfg.layout == "HND":
        return (cfg.B, heads, seq, cfg.D)
    return (cfg.B, seq, heads, cfg.D)


def make_inputs(cfg: Config, seed: int = 0):
    """q, k, v as CPU torch tensors of cfg.dtype, generated in fp32 from a seeded
    CPU generator and then cast (identical bits for the oracle and the GPU)."""
    g = torch.Generator().manual_seed(seed)
    dt = TORCH_DTYPES[cfg.dtype]
    q = torch.randn(shape_of(cfg, cfg.Hq, cfg.q_len), generator=g)
    k = torch.randn(shape_of(cfg, cfg.Hkv, cfg.S), generator=g)
    v = torch.randn(shape_of(cfg, cfg.Hkv, cfg.S), generator=g)
    if cfg.k_offset_std:
        off = torch.randn((cfg.B, cfg.Hkv, 1, cfg.D), generator=g) * cfg.k_offset_std
        if cfg.layout == "NHD":
            off = off.transpose(1, 2)
        k = k + off
    if cfg.outlier_frac:
        n_out = max(1, round(cfg.outlier_frac * cfg.D))
        chans = torch.randperm(cfg.D, generator=g)[:n_out]
        q[..., chans] *= 20.0
        k[..., chans] *= 20.0
    return q.to(dt), k.to(dt), v.to(dt)


def to_np(t: torch.Tensor) -> np.ndarray:
    """CPU numpy view; bf16 becomes uint16 bit patterns (oracle convention)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def np_to_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    return orc.to_f32(a, dtype)


def cos_sim(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = math.sqrt(float(a @ a) * float(b @ b))
    return float(a @ b) / den if den > 0 else 1.0


def max_abs(a: np.ndarray, b: np.ndarray) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)))) if np.size(a) else 0.0


def sdpa_rows_fp32(q32: np.ndarray, k32: np.ndarray, v32: np.ndarray, rows, causal: bool, sm_scale: float):
    """fp32 softmax attention of selected rows of one head (HND slices [S,D])."""
    qt = torch.from_numpy(np.ascontiguousarray(q32[rows], np.float32))
    kt = torch.from_numpy(np.ascontiguousarray(k32, np.float32))
    vt = torch.from_numpy(np.ascontiguousarray(v32, np.float32))
    s = (qt @ kt.T) * sm_scale
    if causal:
        r = torch.as_tensor(np.asarray(rows))[:, None]
        c = torch.arange(kt.shape[0])[None, :]
        s = s.masked_fill(c > r, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return (p @ vt).numpy()


def sample_rows(S: int, n: int, rng: np.random.Generator):
    """Row sample that always includes the ends and group/tile boundaries."""
    fixed = [0, 1, 15, 16, 31, 32, 63, 64, 127, 128, S // 2, S - 65, S - 64, S - 33, S - 32, S - 2, S - 1]
    extra = rng.integers(0, S, size=n) if S > 0 else []
    rows = sorted({int(r) for r in list(fixed) + list(extra) if 0 <= r < S})
    return np.asarray(rows, np.int64)
