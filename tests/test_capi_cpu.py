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
    assert lib.sage_abi_version() == _capi.ABI_VERSION == 2


def test_size_helpers(lib):
    assert lib.sage_v_layout_padded_len(0) == 0
    assert lib.sage_v_layout_padded_len(1) == 64
    assert lib.sage_v_layout_padded_len(64) == 64
    assert lib.sage_v_layout_padded_len(32891) == 32896
    # one fp32 partial row per 1024-key chunk
    assert lib.sage_k_mean_workspace_bytes(2, 32, 8192, 128) == 2 * 32 * 8 * 128 * 4
    assert lib.sage_k_mean_workspace_bytes(1, 40, 32891, 128) == 40 * 33 * 128 * 4
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
             osb=4 * 64 * 128, osh=64 * 128, osn=128, causal=1, scale=0.125, nsplit=0, ws=NULL, wsb=0,
             stream=NULL)
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
        (dict(nsplit=-1), _capi.ERR_INVALID_ARG, "num_splits"),
        (dict(nsplit=17), _capi.ERR_INVALID_ARG, "num_splits"),
        (dict(wsb=-16), _capi.ERR_INVALID_ARG, "workspace_bytes"),
        # 4 key splits of 4 q-blocks: 16 items x 256 rows x (128 + 1) fp32
        (dict(causal=0, Sk=1024, nsplit=4), _capi.ERR_INVALID_ARG, "need a workspace of 2113536 bytes (got 0)"),
        (dict(causal=0, Sk=1024, nsplit=4, ws=FAKE, wsb=2113535), _capi.ERR_INVALID_ARG, "2113536"),
        (dict(causal=0, Sk=1024, nsplit=4, ws=ODD, wsb=2113536), _capi.ERR_ALIGNMENT, "workspace"),
    ],
)
def test_direct_validation(lib, kw, code, msg):
    assert direct(lib, **kw) == code
    assert msg in lib.sage_last_error().decode()


@pytest.mark.parametrize("which", ["osb", "osh", "osn"])
def test_negative_out_strides_are_rejected(lib, which):
    for call in (attn, direct):
        assert call(lib, **{which: -8}) == _capi.ERR_INVALID_ARG
        assert "out strides must be non-negative" in lib.sage_last_error().decode()


# The attention kernels address a head's K rows and V_T rows with 32-bit buffer offsets: the per-head
# V_T span D * ceil64(Sk) * 2 bytes and the K span (Sk + 5 tiles) * k_stride_n * elem must stay within
# UINT32_MAX.  Shapes one past either edge are refused before any launch.
UINT32_MAX = 2 ** 32 - 1


def test_32bit_limits_at_the_edge(lib):
    # V_T: D = 128, np = 16777152 keeps 128 * np * 2 = 4294950912 <= UINT32_MAX; Sk one more pads to
    # np = 16777216, i.e. 2^32 bytes
    assert 128 * 16777152 * 2 <= UINT32_MAX < 128 * 16777216 * 2
    for call in (attn, direct, qfused):
        assert call(lib, Sk=16777153, causal=1) == _capi.ERR_UNSUPPORTED
        assert "32-bit" in lib.sage_last_error().decode()
    # K (direct kind, fp16, a strided K): (Sk + 320) * ksn * 2 bytes; Sk = 64, ksn one step (8) past
    # the largest multiple of 8 that fits
    ksn_max = UINT32_MAX // ((64 + 320) * 2) // 8 * 8
    assert (64 + 320) * (ksn_max + 8) * 2 > UINT32_MAX >= (64 + 320) * ksn_max * 2
    assert direct(lib, Sk=64, ksn=ksn_max + 8, ksh=ksn_max + 8, ksb=ksn_max + 8) == _capi.ERR_UNSUPPORTED
    assert "32-bit" in lib.sage_last_error().decode()
    # query lengths: q_len + one q-block must stay an int32
    assert direct(lib, Sq=2 ** 31 - 256 + 1) == _capi.ERR_UNSUPPORTED


def test_direct_zero_work_is_ok(lib):
    assert direct(lib, Sq=0) == _capi.OK
    assert direct(lib, B=0, q=NULL) == _capi.OK
    assert lib.sage_last_error() == b""


def qfused(lib, **kw):
    a = dict(q=FAKE, k8=FAKE, vt=FAKE, o=FAKE, lse=NULL, ks=FAKE, dtype=1, B=1, Hq=4, Hkv=2, Sq=64, Sk=64, D=128,
             qsb=4 * 64 * 128, qsh=64 * 128, qsn=128, osb=4 * 64 * 128, osh=64 * 128, osn=128, causal=1,
             scale=0.125, nsplit=0, ws=NULL, wsb=0, stream=NULL)
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
        (dict(nsplit=99), _capi.ERR_INVALID_ARG, "num_splits"),
        (dict(causal=0, Sk=4096, Sq=300, nsplit=3), _capi.ERR_INVALID_ARG,
         f"need a workspace of {2 * 4 * 3 * 256 * 129 * 4} bytes"),
    ],
)
def test_qfused_validation(lib, kw, code, msg):
    assert qfused(lib, **kw) == code
    assert msg in lib.sage_last_error().decode()


def qfused_vrows(lib, **kw):
    a = dict(q=FAKE, k8=FAKE, v=FAKE, o=FAKE, lse=NULL, ks=FAKE, dtype=0, B=1, Hq=4, Hkv=2, Sq=64, Sk=64, D=128,
             qsb=4 * 64 * 128, qsh=64 * 128, qsn=128, vsb=2 * 64 * 128, vsh=64 * 128, vsn=128,
             osb=4 * 64 * 128, osh=64 * 128, osn=128, causal=1, scale=0.125, nsplit=0, ws=NULL, wsb=0, stream=NULL)
    a.update(kw)
    return lib.sage_attn_i8_fwd_qfused_vrows(*a.values())


@pytest.mark.parametrize(
    "kw,code,msg",
    [
        (dict(dtype=1), _capi.ERR_UNSUPPORTED, "SAGE_DTYPE_F16"),
        (dict(D=96), _capi.ERR_UNSUPPORTED, "head_dim"),
        (dict(v=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(v=ODD), _capi.ERR_ALIGNMENT, "q/k/value must be 16-byte aligned"),
        (dict(vsn=120), _capi.ERR_INVALID_ARG, "V rows must not overlap"),
        (dict(vsh=-128), _capi.ERR_INVALID_ARG, "value strides"),
        (dict(vsn=132), _capi.ERR_ALIGNMENT, "value strides must be multiples of 16 bytes"),
        (dict(vsb=8 * 64 * 128 + 4), _capi.ERR_ALIGNMENT, "value strides"),
        # per-head V rows addressed with 32-bit offsets: (kv_len + 5 tiles) * row pitch < 4 GiB
        (dict(Sk=1 << 20, vsn=2048, vsh=2048 * (1 << 20), vsb=2 * 2048 * (1 << 20)), _capi.ERR_UNSUPPORTED,
         "32-bit"),
        (dict(qsn=132), _capi.ERR_ALIGNMENT, "16 bytes"),
        (dict(nsplit=99), _capi.ERR_INVALID_ARG, "num_splits"),
    ],
)
def test_qfused_vrows_validation(lib, kw, code, msg):
    assert qfused_vrows(lib, **kw) == code
    assert msg in lib.sage_last_error().decode()


def test_qfused_vrows_zero_work_is_ok(lib):
    assert qfused_vrows(lib, B=0) == _capi.OK
    assert qfused_vrows(lib, Sq=0) == _capi.OK


def direct_vrows(lib, **kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, o=FAKE, lse=NULL, dtype=0, B=1, Hq=4, Hkv=2, Sq=64, Sk=64, D=64,
             qsb=4 * 64 * 64, qsh=64 * 64, qsn=64, ksb=2 * 64 * 64, ksh=64 * 64, ksn=64,
             vsb=2 * 64 * 64, vsh=64 * 64, vsn=64, osb=4 * 64 * 64, osh=64 * 64, osn=64, causal=0, scale=0.125,
             nsplit=1, ws=NULL, wsb=0, stream=NULL)
    a.update(kw)
    return lib.sage_attn_direct_fwd_vrows(*a.values())


@pytest.mark.parametrize(
    "kw,code,msg",
    [
        (dict(dtype=1), _capi.ERR_UNSUPPORTED, "SAGE_DTYPE_F16"),
        (dict(dtype=7), _capi.ERR_INVALID_ARG, "sage_attn_direct_fwd_vrows: dtype"),
        (dict(D=96), _capi.ERR_UNSUPPORTED, "head_dim"),
        (dict(v=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(k=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(v=ODD), _capi.ERR_ALIGNMENT, "q/k/value must be 16-byte aligned"),
        (dict(vsn=60), _capi.ERR_INVALID_ARG, "V rows must not overlap"),
        (dict(vsh=-64), _capi.ERR_INVALID_ARG, "value strides"),
        (dict(vsn=68), _capi.ERR_ALIGNMENT, "value strides must be multiples of 16 bytes"),
        (dict(ksn=60), _capi.ERR_INVALID_ARG, "overlap"),
        (dict(Hq=3), _capi.ERR_INVALID_ARG, "multiple"),
        (dict(nsplit=99), _capi.ERR_INVALID_ARG, "num_splits"),
        # 3 key splits of 4 q-blocks (one per head, 128 rows at D = 64): 12 x 128 x 65 fp32
        (dict(nsplit=3, Sk=1024, ksb=2 * 1024 * 64, ksh=1024 * 64, vsb=2 * 1024 * 64, vsh=1024 * 64),
         _capi.ERR_INVALID_ARG, f"need a workspace of {4 * 3 * 128 * 65 * 4} bytes (got 0)"),
    ],
)
def test_direct_vrows_validation(lib, kw, code, msg):
    assert direct_vrows(lib, **kw) == code
    assert msg in lib.sage_last_error().decode()


def test_direct_vrows_zero_work_is_ok(lib):
    assert direct_vrows(lib, B=0) == _capi.OK
    assert direct_vrows(lib, Sq=0) == _capi.OK
    assert lib.sage_last_error() == b""


def test_qfused_zero_work_is_ok(lib):
    assert qfused(lib, Sq=0) == _capi.OK
    assert qfused(lib, B=0, q=NULL) == _capi.OK


def prep(lib, **kw):
    a = dict(k=FAKE, v=FAKE, mean=NULL, k8=FAKE, ks=FAKE, vt=FAKE, dtype=0, B=1, H=2, S=100, D=128,
             ksb=2 * 100 * 128, ksh=100 * 128, ksn=128, vsb=2 * 100 * 128, vsh=100 * 128, vsn=128, stream=NULL)
    a.update(kw)
    return lib.sage_prep_kv_i8(*a.values())


@pytest.mark.parametrize(
    "kw,code,msg",
    [
        (dict(dtype=3), _capi.ERR_INVALID_ARG, "dtype"),
        (dict(D=80), _capi.ERR_UNSUPPORTED, "head_dim"),
        (dict(H=0), _capi.ERR_INVALID_ARG, "negative or zero"),
        (dict(v=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(ks=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(k=ODD), _capi.ERR_ALIGNMENT, "key"),
        (dict(vsn=132), _capi.ERR_ALIGNMENT, "value"),
        (dict(mean=ODD), _capi.ERR_ALIGNMENT, "key_mean"),
        (dict(vt=ctypes.c_void_p(0x10008)), _capi.ERR_ALIGNMENT, "value_t"),
    ],
)
def test_prep_kv_validation(lib, kw, code, msg):
    assert prep(lib, **kw) == code
    assert msg in lib.sage_last_error().decode()


def test_prep_kv_zero_work_is_ok(lib):
    assert prep(lib, S=0) == _capi.OK
    assert prep(lib, B=0, k=NULL) == _capi.OK


def prep_smooth(lib, **kw):
    a = dict(k=FAKE, v=FAKE, mean=NULL, ws=FAKE, k8=FAKE, ks=FAKE, vt=FAKE, dtype=1, B=1, H=2, S=100, D=128,
             ksb=2 * 100 * 128, ksh=100 * 128, ksn=128, vsb=2 * 100 * 128, vsh=100 * 128, vsn=128, stream=NULL)
    a.update(kw)
    return lib.sage_prep_kv_i8_smooth(*a.values())


@pytest.mark.parametrize(
    "kw,code,msg",
    [
        (dict(dtype=2), _capi.ERR_INVALID_ARG, "dtype"),
        (dict(D=96), _capi.ERR_UNSUPPORTED, "head_dim"),
        (dict(B=-1), _capi.ERR_INVALID_ARG, "negative or zero"),
        (dict(ws=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(k8=NULL), _capi.ERR_INVALID_ARG, "null"),
        (dict(v=ODD), _capi.ERR_ALIGNMENT, "value"),
        (dict(ksh=100 * 128 + 4), _capi.ERR_ALIGNMENT, "key"),
        (dict(ws=ctypes.c_void_p(0x10002)), _capi.ERR_ALIGNMENT, "workspace"),
        (dict(mean=ODD), _capi.ERR_ALIGNMENT, "key_mean"),
        (dict(k8=ctypes.c_void_p(0x10004)), _capi.ERR_ALIGNMENT, "k_i8"),
        (dict(S=1 << 31), _capi.ERR_UNSUPPORTED, "grid limits"),
    ],
)
def test_prep_kv_smooth_validation(lib, kw, code, msg):
    assert prep_smooth(lib, **kw) == code
    assert msg in lib.sage_last_error().decode()


def test_prep_kv_smooth_zero_work_is_ok(lib):
    assert prep_smooth(lib, S=0) == _capi.OK
    assert prep_smooth(lib, B=0, k=NULL, ws=NULL) == _capi.OK


def test_split_workspace_bytes(lib):
    ws = lib.sage_attn_workspace_bytes
    # forced counts: items (B*Hq*ceil(Sq/256)) x splits x 256 rows x (D + 1) fp32; D = 64 non-causal
    # launches run 128-row q-blocks (two blocks per CU): B*Hq*ceil(Sq/128) x splits x 128 rows
    assert ws(1, 1, 4, 64, 1024, 128, 0, 4) == 4 * 4 * 256 * 129 * 4
    assert ws(0, 2, 3, 257, 5000, 64, 0, 16) == 2 * 3 * 3 * 16 * 128 * 65 * 4
    assert ws(1, 1, 4, 64, 128, 128, 0, 4) == 4 * 2 * 256 * 129 * 4  # at most one split per 64 keys
    assert ws(1, 1, 4, 64, 1024, 128, 0, 1) == 0
    assert ws(1, 1, 4, 64, 1024, 128, 1, 4) == 0  # causal: never split
    assert ws(1, 1, 4, 64, 0, 128, 0, 4) == 0
    assert ws(1, 0, 4, 64, 1024, 128, 0, 4) == 0
    # the library's own choice: never for a grid of whole rounds
    assert ws(1, 8, 64, 16384, 16384, 128, 0, 0) == 0
    assert ws(1, 1, 4, 64, 1024, 128, 0, 17) == _capi.ERR_INVALID_ARG
    assert ws(1, 1, 4, 64, 1024, 96, 0, 0) == _capi.ERR_UNSUPPORTED
    assert ws(1, -1, 4, 64, 1024, 128, 0, 0) == _capi.ERR_INVALID_ARG
    with pytest.raises(_capi.SageError, match="SAGE_ERR_INVALID_ARG"):
        _capi.query("sage_attn_workspace_bytes", 1, 1, 4, 64, 1024, 128, 0, -1)


def test_split_plan(lib):
    plan = _capi.split_plan
    assert plan(True, 1, 4, 64, 1024, 128, False, 4) == (0, 4)      # forced: every q-block
    assert plan(False, 1, 4, 600, 128, 64, False, 9) == (0, 2)      # at most one split per key tile
    # causal: whole; 12 q-blocks of 256 rows fill at most half the CUs, so 20 of 128 rows run instead
    assert plan(True, 1, 4, 600, 4096, 128, True, 4) == (20, 1)
    assert plan(False, 1, 4, 600, 4096, 128, True, 4) == (20, 1)    # the D = 128 direct kernel too
    assert plan(True, 1, 64, 600, 4096, 128, True, 0) == (192, 1)   # 192 q-blocks of 256 rows: more than half
    assert plan(True, 1, 4, 600, 4096, 128, False, 1) == (12, 1)
    assert plan(True, 1, 4, 600, 0, 128, False, 0) == (12, 1)       # no keys
    assert plan(True, 0, 4, 600, 4096, 128, False, 0) == (0, 1)
    with pytest.raises(_capi.SageError, match="null output"):
        _capi.call("sage_attn_split_plan", 1, 1, 4, 64, 1024, 128, 0, 0, NULL, NULL)


@pytest.mark.skipif(torch.cuda.is_available(), reason="automatic plans depend on the device's CU count")
def test_automatic_plans_for_256_cus(lib):
    """Without a device the planner assumes MI355X's 256 CUs.  Grids of whole rounds stay whole; small
    grids split every q-block when that promises 1.2x or more; grids over a whole round split only the
    last round's q-blocks."""
    plan = _capi.split_plan
    assert plan(True, 1, 32, 16384, 16384, 128, False, 0) == (2048, 1)   # 8 whole rounds
    assert plan(True, 1, 16, 4096, 4096, 128, False, 0) == (256, 1)      # exactly one round
    assert plan(True, 1, 3, 16384, 16384, 128, False, 0) == (192, 1)     # 192 q-blocks: estimated gain < 1.2x
    assert plan(True, 1, 10, 9216, 9216, 64, False, 0) == (720, 1)       # 720 128-row q-blocks: whole
    assert plan(True, 1, 3, 24576, 24576, 128, False, 0) == (256, 8)     # 288 = 256 + 32
    assert plan(False, 1, 10, 2048, 2048, 128, False, 0) == (0, 3)       # 80 q-blocks
    assert plan(True, 1, 10, 4096, 4096, 64, False, 0) == (256, 4)       # 320 128-row q-blocks = 256 + 64
    # 128-row q-blocks that fit one dispatch at two blocks per CU: a tail of up to half a round is split,
    # a longer one runs whole beside the others
    assert plan(True, 1, 12, 4096, 4096, 64, False, 0) == (256, 2)       # 384 = 256 + 128
    assert plan(True, 1, 5, 11264, 11264, 64, False, 0) == (440, 1)      # 440 = 256 + 184
    assert plan(True, 2, 144, 256, 4096, 128, False, 0) == (256, 8)
    # causal D = 128 launches whose 256-row q-blocks fill one round: 128-row q-blocks on a persistent grid (one
    # block per CU, a heavy and a light q-block each) where the causal cost model rates them faster
    assert plan(False, 1, 32, 2048, 2048, 128, True, 0) == (512, 1)
    assert plan(False, 2, 16, 2048, 2048, 128, True, 0) == (512, 1)
    assert plan(False, 1, 16, 4096, 4096, 128, True, 0) == (512, 1)
    assert plan(False, 1, 32, 1536, 1536, 128, True, 0) == (192, 1)   # a block would get two heavy q-blocks
    assert plan(True, 1, 32, 2048, 2048, 128, True, 0) == (512, 1)    # the INT8 kernels too
    assert plan(True, 1, 16, 4096, 4096, 128, True, 0) == (512, 1)
    assert plan(True, 1, 12, 4096, 4096, 128, True, 0) == (384, 1)
    assert plan(True, 1, 32, 1536, 1536, 128, True, 0) == (192, 1)
    assert plan(False, 1, 32, 4096, 4096, 128, True, 0) == (512, 1)   # two rounds of 256-row q-blocks
    assert plan(True, 1, 32, 16384, 16384, 128, True, 0) == (2048, 1)  # NS: eight rounds, 256-row q-blocks
    assert plan(False, 1, 32, 2048, 2048, 64, True, 0) == (512, 1)     # head_dim 64 too
    assert plan(True, 1, 16, 4096, 4096, 64, True, 0) == (512, 1)
    # a workspace-size query agrees with the plan: (q-blocks - whole) * splits * 256 rows * (D + 1) fp32
    assert lib.sage_attn_workspace_bytes(1, 1, 3, 24576, 24576, 128, 0, 0) == 32 * 8 * 256 * 129 * 4


def test_noalloc_refuses_splits_beyond_the_scratch(lib):
    """sage_attn_i8_fwd_qfused_noalloc: a forced split count whose partials exceed the library's 64 MiB
    scratch is refused before any launch (the pointers are never dereferenced)."""
    need = lib.sage_attn_workspace_bytes(1, 1, 64, 4096, 4096, 128, 0, 16)
    assert need > 64 << 20
    rc = lib.sage_attn_i8_fwd_qfused_noalloc(FAKE, FAKE, FAKE, FAKE, NULL, FAKE, 1, 1, 64, 64, 4096, 4096, 128,
                                             64 * 4096 * 128, 4096 * 128, 128, 64 * 4096 * 128, 4096 * 128, 128,
                                             0, 0.088, 16, NULL)
    assert rc == _capi.ERR_UNSUPPORTED
    assert "scratch" in lib.sage_last_error().decode()
    # a count that fits passes this check (and would launch): not called here
    assert lib.sage_attn_workspace_bytes(1, 1, 4, 3000, 3000, 128, 0, 3) <= 64 << 20


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


def test_host_module_loads_and_checks_shapes():
    """The compiled host layer of sageattn loads, links the same ABI, and raises the Python side's
    ValueErrors and SageError before any launch (CPU tensors; no kernel is reached)."""
    from sageattention import core

    host = core._host()
    assert host.abi_version() == _capi.ABI_VERSION
    q = torch.zeros(1, 4, 64, 64, dtype=torch.float16)
    k3 = torch.zeros(1, 3, 64, 64, dtype=torch.float16)
    args = (1, False, 0.125, False, False, True, 0, 0)
    with pytest.raises(ValueError, match="4-D"):
        host.sageattn_fwd(q[0], q, q, *args)
    with pytest.raises(ValueError, match="multiple of kv heads"):
        host.sageattn_fwd(q, k3, k3, *args)
    with pytest.raises(ValueError, match="incompatible shapes"):
        host.sageattn_fwd(q, q, q[:, :, :32], *args)
    with pytest.raises(ValueError, match="num_splits"):
        host.sageattn_fwd(q, q, q, 1, False, 0.125, False, False, True, 17, 0)
    # head_dim 96: the library's V-layout entry rejects it before launching anything
    q96 = torch.zeros(1, 4, 64, 96, dtype=torch.float16)
    with pytest.raises(_capi.SageError, match="SAGE_ERR_UNSUPPORTED"):
        host.sageattn_fwd(q96, q96, q96, *args)


def test_torch_ops_namespace_schemas():
    """torch.ops.sageattention carries the reference's six ops with their schemas
    (csrc/pybind_gfx11.cpp:18-38) and has no CPU kernel (the ops fail loudly off the GPU)."""
    from sageattention import ops  # noqa: F401  (registers the namespace)

    want = {
        "qk_int8_sv_bf16_attn_t": "(Tensor query, Tensor key, Tensor value, Tensor(a!) output, Tensor q_scale, "
                                  "Tensor k_scale, int tensor_layout, int is_causal, float sm_scale) -> Tensor",
        "fp16_attn_t": "(Tensor query, Tensor key, Tensor value, Tensor(a!) output, int tensor_layout, "
                       "int is_causal, float sm_scale, int bm_sel) -> Tensor",
        "bf16_attn_t": "(Tensor query, Tensor key, Tensor value, Tensor(a!) output, int tensor_layout, "
                       "int is_causal, float sm_scale, int bm_sel) -> Tensor",
        "quant_qk_int8": "(Tensor query, Tensor key, Tensor key_mean, int tensor_layout, float sm_scale) -> Tensor[]",
        "mean_seq": "(Tensor input, int tensor_layout) -> Tensor",
        "v_transpose": "(Tensor value, Tensor(a!) value_t, int tensor_layout) -> Tensor",
    }
    for name, sig in want.items():
        assert str(getattr(torch.ops.sageattention, name).default._schema) == f"sageattention::{name}{sig}"
    with pytest.raises(NotImplementedError):
        torch.ops.sageattention.mean_seq(torch.zeros(1, 2, 16, 64, dtype=torch.float16), 1)
