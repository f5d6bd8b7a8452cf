"""The reference's end-to-end test matrix (test_sageattn_rdna3.py:80-287, 36 cases),
run through this build's ``sageattn`` and compared with fp32 SDPA
(F.scaled_dot_product_attention on float32 copies) and with the CPU oracle of
the same math.  Every case runs twice: with the reference's direct/INT8
dispatch ("auto": most of these short shapes take the direct kernel) and with
the direct path switched off through its environment thresholds ("int8").

Tolerances: the reference's own bands (cos > 0.99 fp16 / 0.98 bf16, max-abs <
0.35, test_sageattn_rdna3.py:39-53) are kept as the outer bound and tightened
to what the INT8 algorithm reaches on these inputs: cos >= 0.999 vs fp32 SDPA
and the oracle bound of the parity tests (cos >= 0.99999).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import sage_oracle as orc
from _helpers import cos_sim, max_abs, np_to_f32, to_np

pytestmark = pytest.mark.gpu


DIRECT_ENV = ["SAGEATTN_DIRECT_THRESHOLD_D64", "SAGEATTN_DIRECT_THRESHOLD_D64_CAUSAL",
              "SAGEATTN_DIRECT_THRESHOLD_D64_CROSS", "SAGEATTN_DIRECT_THRESHOLD_D128",
              "SAGEATTN_DIRECT_THRESHOLD_D128_CROSS"]


@pytest.fixture(autouse=True)
def seed_random():
    torch.manual_seed(0)


@pytest.fixture(autouse=True, params=["auto", "int8"])
def dispatch(request, monkeypatch):
    """"auto": the reference's default thresholds; "int8": every threshold -1 (no direct path).
    The product and the oracle read the same environment."""
    for name in DIRECT_ENV:
        if request.param == "int8":
            monkeypatch.setenv(name, "-1")
        else:
            monkeypatch.delenv(name, raising=False)
    return request.param


@pytest.fixture
def sageattn():
    from sageattention import sageattn

    return sageattn


def reference_attention(q, k, v, is_causal=False, sm_scale=None):
    """fp32 SDPA on HND tensors (float32 math; returned as float32)."""
    return F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=is_causal, scale=sm_scale)


def oracle_attention(q, k, v, layout, is_causal, sm_scale=None, smooth_k=False):
    dt = {torch.float16: "fp16", torch.bfloat16: "bf16", torch.float32: "fp32"}[q.dtype]
    o = orc.sageattn(to_np(q), to_np(k), to_np(v), dt, layout, is_causal, sm_scale, smooth_k)
    return np_to_f32(o, dt) if dt != "fp32" else o


def assert_close(out, ref, dtype, oracle=None):
    o = out.float().cpu().numpy()
    r = ref.float().cpu().numpy()
    cos = cos_sim(o, r)
    mae = max_abs(o, r)
    assert cos > (0.98 if dtype == torch.bfloat16 else 0.99), f"cosine similarity {cos} too low"
    assert mae < 0.35, f"Max abs error {mae} too high"
    assert cos >= 0.999, f"cos {cos} vs fp32 SDPA below 0.999"
    if oracle is not None:
        assert cos_sim(o, oracle) >= 0.99999
    return cos, mae


def randn(*shape, dtype=torch.float16):
    return torch.randn(*shape, dtype=dtype, device="cuda")


class TestSageAttnBasic:
    @pytest.mark.parametrize("head_dim", [64, 128])
    @pytest.mark.parametrize("seq_len", [128, 256, 512, 1024])
    def test_hnd_fp16(self, sageattn, head_dim, seq_len):
        q, k, v = (randn(2, 8, seq_len, head_dim) for _ in range(3))
        out = sageattn(q, k, v, tensor_layout="HND", is_causal=False)
        assert_close(out, reference_attention(q, k, v), torch.float16, oracle_attention(q, k, v, "HND", False))

    @pytest.mark.parametrize("head_dim", [64, 128])
    def test_hnd_fp16_int8_path(self, sageattn, head_dim):
        seq_len = 2048 if head_dim == 64 else 1024
        q, k, v = (randn(1, 4, seq_len, head_dim) for _ in range(3))
        out = sageattn(q, k, v, tensor_layout="HND", is_causal=False)
        assert_close(out, reference_attention(q, k, v), torch.float16)

    @pytest.mark.parametrize("head_dim", [64, 128])
    @pytest.mark.parametrize("seq_len", [128, 256])
    def test_nhd_fp16(self, sageattn, head_dim, seq_len):
        q, k, v = (randn(2, seq_len, 8, head_dim) for _ in range(3))
        out = sageattn(q, k, v, tensor_layout="NHD", is_causal=False)
        ref = reference_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)).transpose(1, 2)
        assert_close(out, ref, torch.float16, oracle_attention(q, k, v, "NHD", False))

    @pytest.mark.parametrize("head_dim", [64, 128])
    def test_bf16(self, sageattn, head_dim):
        q, k, v = (randn(2, 8, 256, head_dim, dtype=torch.bfloat16) for _ in range(3))
        out = sageattn(q, k, v, tensor_layout="HND", is_causal=False)
        assert out.dtype == torch.bfloat16
        assert_close(out, reference_attention(q, k, v), torch.bfloat16, oracle_attention(q, k, v, "HND", False))

    def test_sm_scale(self, sageattn):
        q, k, v = (randn(1, 4, 256, 64) for _ in range(3))
        out = sageattn(q, k, v, tensor_layout="HND", is_causal=False, sm_scale=0.5)
        assert_close(out, reference_attention(q, k, v, sm_scale=0.5), torch.float16,
                     oracle_attention(q, k, v, "HND", False, 0.5))


class TestSageAttnCrossAttn:
    @pytest.mark.parametrize("head_dim", [64, 128])
    def test_cross_attn(self, sageattn, head_dim):
        q = randn(1, 4, 1024, head_dim)
        k, v = randn(1, 4, 128, head_dim), randn(1, 4, 128, head_dim)
        out = sageattn(q, k, v, tensor_layout="HND", is_causal=False)
        assert_close(out, reference_attention(q, k, v), torch.float16, oracle_attention(q, k, v, "HND", False))

    def test_cross_attn_int8(self, sageattn):
        q = randn(1, 4, 512, 64)
        k, v = randn(1, 4, 2048, 64), randn(1, 4, 2048, 64)
        out = sageattn(q, k, v, tensor_layout="HND", is_causal=False)
        assert_close(out, reference_attention(q, k, v), torch.float16, oracle_attention(q, k, v, "HND", False))


class TestSageAttnCausal:
    @pytest.mark.parametrize("head_dim", [64, 128])
    @pytest.mark.parametrize("seq_len", [128, 256, 512])
    def test_causal(self, sageattn, head_dim, seq_len):
        q, k, v = (randn(2, 8, seq_len, head_dim) for _ in range(3))
        out = sageattn(q, k, v, tensor_layout="HND", is_causal=True)
        assert_close(out, reference_attention(q, k, v, is_causal=True), torch.float16,
                     oracle_attention(q, k, v, "HND", True))

    def test_causal_int8(self, sageattn):
        q, k, v = (randn(1, 4, 2048, 64) for _ in range(3))
        out = sageattn(q, k, v, tensor_layout="HND", is_causal=True)
        assert_close(out, reference_attention(q, k, v, is_causal=True), torch.float16,
                     oracle_attention(q, k, v, "HND", True))


class TestSageAttnGQA:
    @pytest.mark.parametrize("head_dim", [64, 128])
    @pytest.mark.parametrize("num_kv_groups", [2, 4])
    def test_gqa(self, sageattn, head_dim, num_kv_groups):
        q = randn(2, 8, 256, head_dim)
        k = randn(2, 8 // num_kv_groups, 256, head_dim)
        v = randn(2, 8 // num_kv_groups, 256, head_dim)
        out = sageattn(q, k, v, tensor_layout="HND", is_causal=False)
        ref = reference_attention(q, k.repeat_interleave(num_kv_groups, dim=1), v.repeat_interleave(num_kv_groups, dim=1))
        assert_close(out, ref, torch.float16, oracle_attention(q, k, v, "HND", False))


class TestSageAttnSmoothK:
    @pytest.mark.parametrize("smooth_k", [True, False])
    def test_smooth_k_effect(self, sageattn, smooth_k):
        q, k, v = (randn(2, 8, 2048, 64) for _ in range(3))
        out = sageattn(q, k, v, tensor_layout="HND", smooth_k=smooth_k)
        assert_close(out, reference_attention(q, k, v), torch.float16)


class TestSageAttnEdgeCases:
    def test_short_seq(self, sageattn):
        q, k, v = (randn(1, 4, 32, 64) for _ in range(3))
        out = sageattn(q, k, v, tensor_layout="HND")
        assert_close(out, reference_attention(q, k, v), torch.float16, oracle_attention(q, k, v, "HND", False))

    def test_non_aligned_seq(self, sageattn):
        for seq_len in [33, 65, 100, 127, 129, 255, 1057]:
            q, k, v = (randn(1, 4, seq_len, 64) for _ in range(3))
            out = sageattn(q, k, v, tensor_layout="HND")
            cos = cos_sim(out.float().cpu().numpy(), reference_attention(q, k, v).cpu().numpy())
            assert cos > 0.999, f"Non-aligned seq_len={seq_len} cosine similarity {cos} too low"
            assert cos_sim(out.float().cpu().numpy(), oracle_attention(q, k, v, "HND", False)) >= 0.99999

    def test_single_head(self, sageattn):
        q, k, v = (randn(1, 1, 256, 64) for _ in range(3))
        out = sageattn(q, k, v, tensor_layout="HND")
        assert_close(out, reference_attention(q, k, v), torch.float16, oracle_attention(q, k, v, "HND", False))


class TestApiContract:
    """Behaviour the reference's core.py defines beyond the numerics."""

    def test_fp32_inputs_round_trip(self, sageattn):
        q, k, v = (randn(1, 2, 200, 64, dtype=torch.float32) for _ in range(3))
        out = sageattn(q, k, v)
        assert out.dtype == torch.float32
        assert_close(out, reference_attention(q, k, v), torch.float16, oracle_attention(q, k, v, "HND", False))

    def test_return_lse(self, sageattn):
        # the reference returns a zero placeholder (core.py:203-211); this build returns the real
        # log-sum-exp of each row, checked against the oracle's on the same quantised inputs
        q, k, v = (randn(2, 3, 100, 128) for _ in range(3))
        o, lse = sageattn(q, k, v, return_lse=True, is_causal=True)
        assert lse.shape == (2, 3, 100) and lse.dtype == torch.float32
        assert torch.equal(o, sageattn(q, k, v, is_causal=True))
        _, ref = orc.sageattn(*(to_np(t) for t in (q, k, v)), "fp16", "HND", True, lse=True)
        assert np.max(np.abs(to_np(lse).astype(np.float64) - ref)) < 2e-4
        qn = q.transpose(1, 2).contiguous()
        o2, lse2 = sageattn(qn, k.transpose(1, 2), v.transpose(1, 2), tensor_layout="NHD", return_lse=True,
                            is_causal=True)
        assert lse2.shape == (2, 3, 100) and torch.equal(lse2, lse)

    def test_alias_and_unknown_kwargs(self, sageattn):
        from sageattention import sageattn_qk_int8_pv_fp16_cuda

        q, k, v = (randn(1, 2, 128, 64) for _ in range(3))
        a = sageattn(q, k, v, bm_sel=2, whatever=1)
        b = sageattn_qk_int8_pv_fp16_cuda(q, k, v)
        assert torch.equal(a, b)

    def test_validation_messages(self, sageattn):
        q = randn(1, 2, 64, 96)
        with pytest.raises(AssertionError, match="head_dim must be 64 or 128"):
            sageattn(q, q, q)
        q = randn(1, 2, 64, 64)
        with pytest.raises(AssertionError, match="same dtype"):
            sageattn(q, q.bfloat16(), q)
        with pytest.raises(AssertionError, match="Last dim"):
            sageattn(q.transpose(2, 3), q, q)
        with pytest.raises(ValueError, match="multiple of kv heads"):
            sageattn(randn(1, 3, 64, 64), q, q)

    def test_strided_and_unaligned_inputs(self, sageattn):
        base = randn(1, 4, 300, 64)
        q = base[:, :, 1:257]  # strided view with a 2-byte-offset-free but sliced base
        k = base[:, :, 3:259].clone()
        v = randn(1, 4, 512, 64)[:, :, ::2]  # token stride 128 elements
        out = sageattn(q, k, v)
        assert_close(out, reference_attention(q, k, v), torch.float16)

    def test_empty_batch_and_queries(self, sageattn):
        q = randn(0, 2, 64, 64)
        assert sageattn(q, q, q).shape == q.shape
        q = randn(1, 2, 0, 64)
        k = randn(1, 2, 64, 64)
        assert sageattn(q, k, k).shape == q.shape

    @pytest.mark.parametrize("smooth_k", [False, True])
    @pytest.mark.parametrize("heads,seq_len,causal", [(4, 1000, False), (32, 2048, True)])
    def test_hip_graph_capture_and_replay(self, sageattn, smooth_k, heads, seq_len, causal):
        # the launches of a call allocate from the caller's torch allocator and never memset or synchronise,
        # so a call captured in a HIP graph replays to the eager result.  H4 S1000: the plan splits the keys
        # (16 q-blocks on a full device), so the graph also holds the workspace and the merge launch, and with
        # smooth_k the K mean's chunk-sum launch and its workspace.  H32 S2048 causal: 512 128-row q-blocks
        # on the persistent grid, heavy and light paired.
        q, k, v = (randn(1, heads, seq_len, 128) for _ in range(3))
        k = k + 3.0  # a K offset that smooth_k removes
        ref = sageattn(q, k, v, is_causal=causal, smooth_k=smooth_k)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            sageattn(q, k, v, is_causal=causal, smooth_k=smooth_k)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = sageattn(q, k, v, is_causal=causal, smooth_k=smooth_k)
        for _ in range(3):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
            # eager work between the replays
            assert torch.equal(sageattn(q, k, v, is_causal=causal, smooth_k=smooth_k), ref)

    def test_empty_keys(self, sageattn):
        # no key at all: every row's output is 0 and its log-sum-exp -inf (the oracle's convention)
        q = randn(1, 2, 300, 128)
        k = randn(1, 2, 0, 128)
        o, lse = sageattn(q, k, k, return_lse=True)
        assert o.shape == q.shape and not o.any()
        assert lse.shape == (1, 2, 300) and bool(torch.all(lse == float("-inf")))
        o, lse = sageattn(q.transpose(1, 2), k.transpose(1, 2), k.transpose(1, 2), tensor_layout="NHD",
                          is_causal=True, return_lse=True, smooth_k=True)
        assert not o.any() and bool(torch.all(lse == float("-inf")))
