"""The C-ABI library loads, exports every symbol of include/*.h, and its
argument validation answers with the documented status codes.  No call here
reaches the GPU: every case fails validation or has zero work."""
import ctypes
import glob
import os
import re

import pytest
import torch

from sageattention import _capi

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(REPO, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(sage_\w+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    return _capi.load()


def test_header_declares_the_entry_points():
    assert declared_symbols() == sorted(_capi.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    assert lib.sage_abi_version() == _capi.ABI_VERSION == 1


def test_size_helpers(lib):
    assert lib.sage_v_layout_padded_len(0) == 0
    assert lib.sage_v_layout_padded_len(1) == 64
    assert lib.sage_v_layout_padded_len(64) == 64
    assert lib.sage_v_layout_padded_len(32891) == 32896
    assert lib.sage_k_mean_workspace_bytes(2, 32, 8192, 128) == 2 * 32 * 32 * 128 * 4
    assert lib.sage_k_mean_workspace_bytes(1, 40, 32891, 128) == 40 * 129 * 128 * 4
    assert lib.sage_k_mean_workspace_bytes(0, 1, 1, 64) == 0


FAKE = ctypes.c_void_p(0x10000)  # never dereferenced: every case below fails validation first
ODD = ctypes.c_void_p(0x10001)
NULL = ctypes.c_void_p(0)


def quant(lib, **kw):
    a = dict(q=FAKE, k=FAKE, mean=NULL, q8=FAKE, qs=FAKE, k8=FAKE, ks=FAKE, dtype=0, B=1, Hq=2, Hkv=2,
             Sq=64, Sk=64, D=128, qsb=2 * 64 * 128, qsh=64 * 128, qsn=128, ksb=2 * 64 * 128, ksh=64 * 128,
             ksn=128, scale=0.1, stream=NULL)
    a.update(kw)
    return lib.sage_quant_qk_i8(*a.values())


def attn(lib, **kw):
    a = dict(q8=FAKE, k8=FAKE, vt=FAKE, o=FAKE, qs=FAKE, ks=FAKE, dtype=0, B=1, Hq=4, Hkv=2, Sq=64, Sk=64, D=128,
             osb=4 * 64 * 128, osh=64 * 128, osn=128, causal=0, stream=NULL)
    a.update(kw)
    return lib.sage_attn_i8_fwd(*a.values())


@pytest.mark.parametrize(
    "kw,code,msg",
    [
        (dict(dtype=7), _capi.ERR_INVALID_ARG, "dtype"),
        (dict(D=96), _capi.ERR_UNSUPPORTED, "head_dim"),
        (dict(Hq=0), _capi.ERR_INVALID_ARG, "size"),
        (dict(q=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(k8=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(q=ODD), _capi.ERR_ALIGNMENT, "query"),
        (dict(qsn=132), _capi.ERR_ALIGNMENT, "strides"),
        (dict(ksh=100), _capi.ERR_ALIGNMENT, "strides"),
        (dict(Sq=2 ** 31), _capi.ERR_UNSUPPORTED, "32-bit"),
    ],
)
def test_quant_validation(lib, kw, code, msg):
    assert quant(lib, **kw) == code
    assert msg in lib.sage_last_error().decode()


def test_quant_zero_work_is_ok(lib):
    assert quant(lib, B=0) == _capi.OK
    assert quant(lib, Sq=0, Sk=0, q=NULL, k=NULL) == _capi.OK
    assert lib.sage_last_error() == b""


@pytest.mark.parametrize(
    "kw,code,msg",
    [
        (dict(dtype=2), _capi.ERR_INVALID_ARG, "out_dtype"),
        (dict(D=32), _capi.ERR_UNSUPPORTED, "head_dim"),
        (dict(Hq=6, Hkv=4), _capi.ERR_INVALID_ARG, "multiple"),
        (dict(vt=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(q8=ODD), _capi.ERR_ALIGNMENT, "aligned"),
        (dict(osn=130), _capi.ERR_ALIGNMENT, "strides"),
    ],
)
def test_attn_validation(lib, kw, code, msg):
    assert attn(lib, **kw) == code
    assert msg in lib.sage_last_error().decode()


def test_attn_zero_work_is_ok(lib):
    assert attn(lib, Sq=0) == _capi.OK
    assert attn(lib, B=0) == _capi.OK


def attn_lse(lib, **kw):
    a = dict(q8=FAKE, k8=FAKE, vt=FAKE, o=FAKE, lse=FAKE, qs=FAKE, ks=FAKE, dtype=0, B=1, Hq=4, Hkv=2, Sq=64,
             Sk=64, D=128, osb=4 * 64 * 128, osh=64 * 128, osn=128, causal=0, stream=NULL)
    a.update(kw)
    return lib.sage_attn_i8_fwd_lse(*a.values())


@pytest.mark.parametrize(
    "kw,code,msg",
    [
        (dict(dtype=2), _capi.ERR_INVALID_ARG, "out_dtype"),
        (dict(vt=NULL), _capi.ERR_INVALID_ARG, "sage_attn_i8_fwd_lse: null"),
        (dict(lse=ODD), _capi.ERR_ALIGNMENT, "lse must be 4-byte aligned"),
        (dict(Sq=2 ** 31), _capi.ERR_UNSUPPORTED, "32-bit"),
    ],
)
def test_attn_lse_validation(lib, kw, code, msg):
    assert attn_lse(lib, **kw) == code
    assert msg in lib.sage_last_error().decode()


def test_attn_lse_zero_work_is_ok(lib):
    assert attn_lse(lib, Sq=0) == _capi.OK
    assert attn_lse(lib, B=0, lse=NULL) == _capi.OK


def direct(lib, **kw):
    a = dict(q=FAKE, k=FAKE, vt=FAKE, o=FAKE, lse=NULL, dtype=1, B=1, Hq=4, Hkv=2, Sq=64, Sk=64, D=128,
             qsb=4 * 64 * 128, qsh=64 * 128, qsn=128, ksb=2 * 64 * 128, ksh=64 * 128, ksn=128,
             osb=4 * 64 * 128, osh=64 * 128, osn=128, causal=1, scale=0.125, stream=NULL)
    a.update(kw)
    return lib.sage_attn_direct_fwd(*a.values())


@pytest.mark.parametrize(
    "kw,code,msg",
    [
        (dict(dtype=2), _capi.ERR_INVALID_ARG, "sage_attn_direct_fwd: dtype"),
        (dict(D=256), _capi.ERR_UNSUPPORTED, "head_dim"),
        (dict(Hq=3), _capi.ERR_INVALID_ARG, "multiple"),
        (dict(Sk=-1), _capi.ERR_INVALID_ARG, "negative"),
        (dict(k=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(o=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(q=ODD), _capi.ERR_ALIGNMENT, "aligned"),
        (dict(vt=ODD), _capi.ERR_ALIGNMENT, "aligned"),
        (dict(qsn=132), _capi.ERR_ALIGNMENT, "16 bytes"),
        (dict(ksh=100), _capi.ERR_ALIGNMENT, "16 bytes"),
        (dict(ksn=64), _capi.ERR_INVALID_ARG, "overlap"),
        (dict(qsb=-8), _capi.ERR_INVALID_ARG, "non-negative"),
        (dict(osn=130), _capi.ERR_ALIGNMENT, "strides"),
        (dict(lse=ODD), _capi.ERR_ALIGNMENT, "lse"),
        (dict(Sk=2 ** 24, ksn=2 ** 10), _capi.ERR_UNSUPPORTED, "32-bit"),
    ],
)
def test_direct_validation(lib, kw, code, msg):
    assert direct(lib, **kw) == code
    assert msg in lib.sage_last_error().decode()


def test_direct_zero_work_is_ok(lib):
    assert direct(lib, Sq=0) == _capi.OK
    assert direct(lib, B=0, q=NULL) == _capi.OK
    assert lib.sage_last_error() == b""


def qfused(lib, **kw):
    a = dict(q=FAKE, k8=FAKE, vt=FAKE, o=FAKE, lse=NULL, ks=FAKE, dtype=1, B=1, Hq=4, Hkv=2, Sq=64, Sk=64, D=128,
             qsb=4 * 64 * 128, qsh=64 * 128, qsn=128, osb=4 * 64 * 128, osh=64 * 128, osn=128, causal=1,
             scale=0.125, stream=NULL)
    a.update(kw)
    return lib.sage_attn_i8_fwd_qfused(*a.values())


@pytest.mark.parametrize(
    "kw,code,msg",
    [
        (dict(dtype=5), _capi.ERR_INVALID_ARG, "dtype"),
        (dict(D=96), _capi.ERR_UNSUPPORTED, "head_dim"),
        (dict(ks=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(q=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(q=ODD), _capi.ERR_ALIGNMENT, "aligned"),
        (dict(qsn=132), _capi.ERR_ALIGNMENT, "16 bytes"),
        (dict(osh=130), _capi.ERR_ALIGNMENT, "strides"),
        (dict(lse=ODD), _capi.ERR_ALIGNMENT, "lse"),
        (dict(Hq=5), _capi.ERR_INVALID_ARG, "multiple"),
    ],
)
def test_qfused_validation(lib, kw, code, msg):
    assert qfused(lib, **kw) == code
    assert msg in lib.sage_last_error().decode()


def test_qfused_zero_work_is_ok(lib):
    assert qfused(lib, Sq=0) == _capi.OK
    assert qfused(lib, B=0, q=NULL) == _capi.OK


def test_v_layout_and_mean_validation(lib):
    assert lib.sage_v_layout(FAKE, FAKE, 0, 1, 2, 100, 80, 0, 0, 0, NULL) == _capi.ERR_UNSUPPORTED
    assert lib.sage_v_layout(ODD, FAKE, 0, 1, 2, 100, 64, 0, 6400, 64, NULL) == _capi.ERR_ALIGNMENT
    assert lib.sage_v_layout(FAKE, FAKE, 0, 1, 2, 0, 64, 0, 0, 64, NULL) == _capi.OK
    assert lib.sage_k_mean(FAKE, FAKE, NULL, 1, 1, 2, 100, 64, 12800, 6400, 64, NULL) == _capi.ERR_INVALID_ARG
    assert lib.sage_k_mean(FAKE, FAKE, FAKE, 1, 1, 2, 0, 64, 0, 0, 64, NULL) == _capi.ERR_INVALID_ARG
    assert "empty" in lib.sage_last_error().decode()


def test_errors_raise_sage_error(lib):
    with pytest.raises(_capi.SageError, match="SAGE_ERR_UNSUPPORTED"):
        _capi.call("sage_v_layout", FAKE, FAKE, 0, 1, 2, 100, 80, 0, 0, 0, NULL)


def test_missing_library_raises_runtime_error(monkeypatch, tmp_path):
    monkeypatch.setattr(_capi, "_lib", None)
    monkeypatch.setenv("SAGEATTN_MI355X_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(RuntimeError, match="not available"):
        _capi.load()


def test_sageattn_rejects_cpu_tensors():
    from sageattention import sageattn

    q = torch.zeros(1, 2, 64, 64, dtype=torch.float16)
    with pytest.raises(AssertionError, match="CUDA/HIP device"):
        sageattn(q, q, q)


def test_package_surface():
    import sageattention

    assert sageattention.__version__ == "0.1.0"
    assert set(sageattention.__all__) == {"sageattn", "sageattn_qk_int8_pv_fp16_cuda"}
