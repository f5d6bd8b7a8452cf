"""The allocation-free entry point sage_attn_i8_fwd_qfused_noalloc (its key splits' partials live in a scratch
array the library holds per GPU) against sage_attn_i8_fwd_qfused with a caller workspace, through the C ABI:
identical outputs and LSEs for the same split count, on two calls in a row (the second smaller, so the
scratch holds the first call's data when it starts), and every element written.  The refusal of split
counts beyond the scratch is checked on the CPU (tests/test_capi_cpu.py), where it cannot reach a launch."""
import ctypes

import numpy as np
import pytest
import torch

from _helpers import Config, make_inputs

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p
SCRATCH = 64 << 20


def _say(*a):
    print(*a, flush=True)


def _prep(cfg, seed):
    from sageattention import ops

    lay = ops.HND if cfg.layout == "HND" else ops.NHD
    q, k, v = (t.cuda() for t in make_inputs(cfg, seed=seed))
    k8, ks, vt = ops.prep_kv_int8(k, v, torch.empty(0, device="cuda", dtype=k.dtype), lay)
    return q, k8, ks, vt


def _args(cfg, q, k8, ks, vt, o, lse):
    from sageattention import ops

    qb, qh, qn = ops._bhnd(q, ops.HND if cfg.layout == "HND" else ops.NHD)[1]
    ob, oh, on = ops._bhnd(o, ops.HND if cfg.layout == "HND" else ops.NHD)[1]
    dt = 1 if cfg.dtype == "bf16" else 0
    return [P(q.data_ptr()), P(k8.data_ptr()), P(vt.data_ptr()), P(o.data_ptr()), P(lse.data_ptr()),
            P(ks.data_ptr()), dt, cfg.B, cfg.Hq, cfg.Hkv, cfg.q_len, cfg.S, cfg.D, qb, qh, qn, ob, oh, on,
            int(cfg.causal), cfg.D ** -0.5]


def _run_pair(lib, cfg, n, seed):
    from sageattention import ops

    q, k8, ks, vt = _prep(cfg, seed)
    stream = P(torch.cuda.current_stream().cuda_stream)
    nan = float("nan")
    o_ref = torch.full_like(q, nan)
    lse_ref = torch.full((cfg.B, cfg.Hq, cfg.q_len), nan, device="cuda", dtype=torch.float32)
    o = torch.full_like(q, nan)
    lse = torch.full_like(lse_ref, nan)
    base = _args(cfg, q, k8, ks, vt, o_ref, lse_ref)
    wsb = lib.sage_attn_workspace_bytes(1, cfg.B, cfg.Hq, cfg.q_len, cfg.S, cfg.D, int(cfg.causal), n)
    assert 0 <= wsb <= SCRATCH, wsb
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device="cuda")
    rc = lib.sage_attn_i8_fwd_qfused(*base, n, P(ws.data_ptr() if wsb else 0), wsb, stream)
    assert rc == 0, lib.sage_last_error()
    rc = lib.sage_attn_i8_fwd_qfused_noalloc(*_args(cfg, q, k8, ks, vt, o, lse), n, stream)
    assert rc == 0, lib.sage_last_error()
    torch.cuda.synchronize()
    assert not bool(torch.isnan(o).any()) and bool(torch.isfinite(lse).all())
    assert torch.equal(o, o_ref), f"max diff {(o.float() - o_ref.float()).abs().max().item()}"
    assert torch.equal(lse, lse_ref)
    whole, splits = ctypes.c_int64(0), ctypes.c_int(0)
    assert lib.sage_attn_split_plan(1, cfg.B, cfg.Hq, cfg.q_len, cfg.S, cfg.D, int(cfg.causal), n,
                                    ctypes.byref(whole), ctypes.byref(splits)) == 0
    return whole.value, splits.value


BIG = Config("noalloc_big", 1, 4, 4, 3000, 128, "bf16", "HND", False, False)
SMALL = Config("noalloc_small", 2, 3, 3, 700, 64, "fp16", "NHD", False, False)


@pytest.mark.parametrize("n", [3, 0])
def test_noalloc_equals_workspace_entry_point(n):
    """Two calls in a row, the second smaller (its launch starts with the first call's partials in the
    scratch): each equals sage_attn_i8_fwd_qfused with a workspace of its own, bit for bit."""
    from sageattention import _capi

    lib = _capi.load()
    for cfg, seed in ((BIG, 1), (SMALL, 2)):
        plan = _run_pair(lib, cfg, n, seed)
        _say(f"[noalloc] {cfg.name} num_splits={n}: plan (whole {plan[0]}, splits {plan[1]}) identical")
        if n == 3:
            assert plan[1] == 3


def test_noalloc_causal_and_unsplit_launches():
    from sageattention import _capi

    lib = _capi.load()
    cfg = Config("noalloc_causal", 1, 4, 2, 1000, 128, "bf16", "HND", True, False)
    _run_pair(lib, cfg, 0, 3)
    cfg = Config("noalloc_unsplit", 1, 4, 4, 1000, 64, "fp16", "HND", False, False)
    _run_pair(lib, cfg, 1, 4)

