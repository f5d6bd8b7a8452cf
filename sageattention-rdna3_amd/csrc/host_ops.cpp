// Compiled host layer of `sageattn` (the reference's sageattention/core.py:40-213
// after its assertions): shapes and strides, the output / LSE / intermediate
// allocations from the caller's torch allocator, and the launches through the
// C ABI of libsage_mi355x.so, in one Python call.  The Python function keeps
// the reference's assertions, its fp32 handling and the direct/INT8 dispatch
// (with its environment overrides); everything after them runs here, because
// for the short and cross-attention shapes the GPU work of a call (~12 us)
// is smaller than what the same steps cost as Python (~10 us on top of the
// launches).
//
// The module calls no HIP API itself: every launch goes through the C ABI on
// the stream handle the caller passes (the current stream of the tensors'
// device), and torch allocates on that same stream, so temporaries released
// here return to the caching allocator in stream order.
#include <torch/extension.h>

#include <cstdint>
#include <sstream>
#include <string>

#include "sageattn_mi355x.h"

namespace py = pybind11;

namespace {

// A negative status of the C ABI, raised in Python as the exception type the
// package registers (sageattention._capi.SageError: function, status, message).
struct SageStatus {
  const char* fn;
  int code;
  std::string msg;
};

// set by set_error_type(); RuntimeError until then.  A plain reference that is
// never released: a py::object here would be decremented by a static
// destructor after the interpreter has finalised.
PyObject* g_error_type = nullptr;

void check(const char* fn, int rc) {
  if (rc != SAGE_OK) {
    const char* m = sage_last_error();
    throw SageStatus{fn, rc, m != nullptr ? m : ""};
  }
}

// (B, H, N, D) sizes and (b, h, n) strides in elements of a 4-D tensor;
// layout 1 = HND [B,H,N,D], 0 = NHD [B,N,H,D] (reference csrc/attn_gfx11.cu:32-33)
struct Dims {
  int64_t b, h, n, d;
  int64_t sb, sh, sn;
};

Dims bhnd(const at::Tensor& t, int64_t layout) {
  const auto s = t.sizes();
  const auto st = t.strides();
  if (layout == 1) return {s[0], s[1], s[2], s[3], st[0], st[1], st[2]};
  return {s[0], s[2], s[1], s[3], st[0], st[2], st[1]};
}

// t, or a copy that meets the 16-byte access contract (16-byte aligned base,
// batch/head/token strides multiples of 8 elements)
at::Tensor vector_ready(const at::Tensor& t) {
  const auto st = t.strides();
  if (reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0 && st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0)
    return t;
  return t.is_contiguous() ? t.clone() : t.contiguous();
}

std::string shape_str(const at::Tensor& t) {
  std::ostringstream s;
  s << "(";
  for (int64_t i = 0; i < t.dim(); ++i) s << (i ? ", " : "") << t.size(i);
  s << ")";
  return s.str();
}

// The key-split workspace of a non-causal launch (undefined when it runs
// unsplit); num_splits is already within [0, SAGE_MAX_KV_SPLITS].
at::Tensor split_workspace(bool quantized, const Dims& q, int64_t kv_len, bool causal, int64_t num_splits,
                           const at::Tensor& like, int64_t* bytes) {
  *bytes = 0;
  if (causal) return at::Tensor();
  const int64_t n = sage_attn_workspace_bytes(quantized ? 1 : 0, q.b, q.h, q.n, kv_len, q.d, 0,
                                              static_cast<int>(num_splits));
  if (n < 0) check("sage_attn_workspace_bytes", static_cast<int>(n));
  if (n == 0) return at::Tensor();
  *bytes = n;
  return at::empty({n}, like.options().dtype(at::kByte));
}

void* ptr(const at::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

// Direct path, fp16 inputs: V is read in place (sage_attn_direct_fwd_vrows)
// instead of through a V_T pass wherever that measured faster on MI355X
// (whole direct call, launches queued): every D = 128 length of the direct
// range (kv 77 -16%, 1024 -4% to -15%, 2048 -2.5% to -7%) and D = 64 up to
// this many keys (kv 77 -10% to -19%, 1024 -4%, 1280 -2%; 1536 +5%, 3072 causal
// +9%: the in-place V operand takes twice the LDS reads per P.V MFMA).
constexpr int64_t kVRowsMaxKeysD64 = 1280;

py::object sageattn_fwd(at::Tensor q, at::Tensor k, at::Tensor v, int64_t layout, bool is_causal, double sm_scale,
                        bool return_lse, bool smooth_k, bool direct, int64_t num_splits, int64_t stream_handle) {
  if (q.dim() != 4 || k.dim() != 4 || v.dim() != 4) throw py::value_error("q, k and v must be 4-D tensors");
  if (num_splits < 0 || num_splits > SAGE_MAX_KV_SPLITS) {
    std::ostringstream s;
    s << "num_splits must be in [0, " << SAGE_MAX_KV_SPLITS << "], got " << num_splits;
    throw py::value_error(s.str());
  }
  q = vector_ready(q);
  k = vector_ready(k);
  v = vector_ready(v);
  const Dims qd = bhnd(q, layout);
  Dims kd = bhnd(k, layout);
  if (k.sizes() != v.sizes() || kd.b != qd.b || kd.d != qd.d)
    throw py::value_error("incompatible shapes q=" + shape_str(q) + " k=" + shape_str(k) + " v=" + shape_str(v));
  if (qd.h % kd.h != 0)
    throw py::value_error("number of query heads (" + std::to_string(qd.h) + ") must be a multiple of kv heads (" +
                          std::to_string(kd.h) + ")");
  const Dims vd = bhnd(v, layout);
  const int dtype = q.scalar_type() == at::kBFloat16 ? SAGE_DTYPE_BF16 : SAGE_DTYPE_F16;
  void* stream = reinterpret_cast<void*>(stream_handle);
  const int64_t B = qd.b, Hq = qd.h, Sq = qd.n, D = qd.d, Hkv = kd.h, Sk = kd.n;
  const int64_t np = sage_v_layout_padded_len(Sk);

  at::Tensor o = at::empty_like(q);
  const Dims od = bhnd(o, layout);
  at::Tensor lse;
  if (return_lse) lse = at::empty({B, Hq, Sq}, q.options().dtype(at::kFloat));

  if (direct) {
    // the direct kernel reads Q and K in place (core.py:141-164); K rows must not overlap
    if (kd.sn < D) {
      k = k.contiguous();
      kd = bhnd(k, layout);
    }
    int64_t ws_bytes = 0;
    at::Tensor ws = split_workspace(false, qd, Sk, is_causal, num_splits, q, &ws_bytes);
    if (dtype == SAGE_DTYPE_F16 && vd.sn >= D && (D == 128 || Sk <= kVRowsMaxKeysD64)) {
      // fp16 V read in place: one launch, the same output bit for bit as the V_T path below
      check("sage_attn_direct_fwd_vrows",
            sage_attn_direct_fwd_vrows(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                       static_cast<float*>(ptr(lse)), dtype, B, Hq, Hkv, Sq, Sk, D, qd.sb, qd.sh,
                                       qd.sn, kd.sb, kd.sh, kd.sn, vd.sb, vd.sh, vd.sn, od.sb, od.sh, od.sn,
                                       is_causal ? 1 : 0, sm_scale, static_cast<int>(num_splits), ptr(ws), ws_bytes,
                                       stream));
    } else {
      // V transform: fp16 V_T [B,Hkv,D,ceil64(Sk)] zero padded (reference core.py:145-152,171-180)
      at::Tensor vt = at::empty({B, Hkv, D, np}, q.options().dtype(at::kHalf));
      check("sage_v_layout",
            sage_v_layout(v.data_ptr(), vt.data_ptr(), dtype, B, Hkv, Sk, D, vd.sb, vd.sh, vd.sn, stream));
      check("sage_attn_direct_fwd",
            sage_attn_direct_fwd(q.data_ptr(), k.data_ptr(), vt.data_ptr(), o.data_ptr(),
                                 static_cast<float*>(ptr(lse)), dtype, B, Hq, Hkv, Sq, Sk, D, qd.sb, qd.sh, qd.sn,
                                 kd.sb, kd.sh, kd.sn, od.sb, od.sh, od.sn, is_causal ? 1 : 0, sm_scale,
                                 static_cast<int>(num_splits), ptr(ws), ws_bytes, stream));
    }
  } else {
    // K quantisation and the V transform in one launch; Q is quantised inside
    // the attention kernel (the q_int8 and q_scale of quant_qk_int8, so the
    // same output, without the int8 Q round trip).  smooth_k: K minus its mean
    // (reference mean_seq, csrc/attn_gfx11.cu:1937-1972), the mean's chunk
    // sums in a launch before, finished by the quantisation blocks
    at::Tensor k8 = at::empty({B, Hkv, Sk, D}, q.options().dtype(at::kChar));
    at::Tensor ks = at::empty({B, Hkv, (Sk + SAGE_K_GROUP - 1) / SAGE_K_GROUP}, q.options().dtype(at::kFloat));
    at::Tensor vt = at::empty({B, Hkv, D, np}, q.options().dtype(at::kHalf));
    if (smooth_k && Sk > 0) {
      const int64_t mb = sage_k_mean_workspace_bytes(B, Hkv, Sk, D);
      if (mb < 0) check("sage_k_mean_workspace_bytes", static_cast<int>(mb));
      at::Tensor mws = at::empty({(std::max<int64_t>(mb, 4) + 3) / 4}, q.options().dtype(at::kFloat));
      check("sage_prep_kv_i8_smooth",
            sage_prep_kv_i8_smooth(k.data_ptr(), v.data_ptr(), nullptr, mws.data_ptr(),
                                   static_cast<int8_t*>(k8.data_ptr()), static_cast<float*>(ks.data_ptr()),
                                   vt.data_ptr(), dtype, B, Hkv, Sk, D, kd.sb, kd.sh, kd.sn, vd.sb, vd.sh, vd.sn,
                                   stream));
    } else {
      check("sage_prep_kv_i8",
            sage_prep_kv_i8(k.data_ptr(), v.data_ptr(), nullptr, static_cast<int8_t*>(k8.data_ptr()),
                            static_cast<float*>(ks.data_ptr()), vt.data_ptr(), dtype, B, Hkv, Sk, D, kd.sb, kd.sh,
                            kd.sn, vd.sb, vd.sh, vd.sn, stream));
    }
    // return_lse: the reference returns a zero placeholder (core.py:203-211);
    // the fused kernel writes the real log-sum-exp of each row
    int64_t ws_bytes = 0;
    at::Tensor ws = split_workspace(true, qd, Sk, is_causal, num_splits, q, &ws_bytes);
    check("sage_attn_i8_fwd_qfused",
          sage_attn_i8_fwd_qfused(q.data_ptr(), static_cast<const int8_t*>(k8.data_ptr()), vt.data_ptr(),
                                  o.data_ptr(), static_cast<float*>(ptr(lse)), static_cast<const float*>(ks.data_ptr()),
                                  dtype, B, Hq, Hkv, Sq, Sk, D, qd.sb, qd.sh, qd.sn, od.sb, od.sh, od.sn,
                                  is_causal ? 1 : 0, sm_scale, static_cast<int>(num_splits), ptr(ws), ws_bytes,
                                  stream));
  }
  if (return_lse) return py::make_tuple(o, lse);
  return py::cast(o);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Compiled host layer of sageattn over the libsage_mi355x C ABI";
  m.def("abi_version", []() { return sage_abi_version(); });
  m.def("set_error_type", [](py::object t) {
    PyObject* old = g_error_type;
    g_error_type = t.inc_ref().ptr();
    Py_XDECREF(old);
  });
  m.def("sageattn_fwd", &sageattn_fwd, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("tensor_layout"),
        py::arg("is_causal"), py::arg("sm_scale"), py::arg("return_lse"), py::arg("smooth_k"), py::arg("direct"),
        py::arg("num_splits"), py::arg("stream"));
  py::register_exception_translator([](std::exception_ptr p) {
    try {
      if (p) std::rethrow_exception(p);
    } catch (const SageStatus& e) {
      if (g_error_type != nullptr && g_error_type != Py_None) {
        py::object type = py::reinterpret_borrow<py::object>(g_error_type);
        py::object err = type(e.fn, e.code, e.msg);
        PyErr_SetObject(g_error_type, err.ptr());
      } else {
        PyErr_SetString(PyExc_RuntimeError, (std::string(e.fn) + ": " + e.msg).c_str());
      }
    }
  });
}
