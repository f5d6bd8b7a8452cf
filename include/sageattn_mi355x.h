/*
 * sageattn_mi355x.h -- C ABI of the MI355X (gfx950) SageAttention quantized path.
 *
 * Every entry point is asynchronous on the given HIP stream (a hipStream_t
 * passed as void*; NULL = the legacy default stream), never synchronises the
 * host, and allocates nothing: the caller owns every buffer (inputs, outputs,
 * workspaces).  Entry points validate their arguments before touching the GPU
 * and return SAGE_OK (0) or a negative status; the message of the last failure
 * on the calling thread is returned by sage_last_error().
 *
 * Strides are in ELEMENTS.  Tensor "layout" (HND [B,H,N,D] or NHD [B,N,H,D])
 * is expressed only through (stride_b, stride_h, stride_n); the head_dim axis
 * must be contiguous.  16-byte vector accesses require base pointers aligned
 * to 16 bytes and batch/head/token strides that are multiples of 8 elements.
 *
 * Reference interfaces replaced (LuXuxue/sageattention-rdna3):
 *   torch.ops.sageattention.{mean_seq, quant_qk_int8, v_transpose,
 *   qk_int8_sv_bf16_attn_t, fp16_attn_t, bf16_attn_t}, declared at
 *   csrc/pybind_gfx11.cpp:18-38 and csrc/attn_gfx11.h:10-51, implemented at
 *   csrc/attn_gfx11.cu:1889-2472.
 */
#ifndef SAGEATTN_MI355X_H
#define SAGEATTN_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SAGE_ABI_VERSION 2

/* element types of the fp inputs / outputs */
#define SAGE_DTYPE_F16 0
#define SAGE_DTYPE_BF16 1

/* status codes */
#define SAGE_OK 0
#define SAGE_ERR_INVALID_ARG (-1) /* null pointer, negative size, bad dtype, Hq % Hkv != 0 */
#define SAGE_ERR_UNSUPPORTED (-2) /* head_dim not in {64, 128}, size beyond 32-bit grid limits */
#define SAGE_ERR_ALIGNMENT (-3)   /* pointer or stride breaks the 16-byte access contract */
#define SAGE_ERR_HIP (-4)         /* the HIP runtime rejected a launch */

/* Quantisation granularity (tokens per fp32 scale), csrc/attn_gfx11.cu:46-47. */
#define SAGE_Q_GROUP 32
#define SAGE_K_GROUP 16
/* V_T token padding, sageattention/core.py:174. */
#define SAGE_VT_ALIGN 64
/* Largest key-split count of the non-causal attention entry points. */
#define SAGE_MAX_KV_SPLITS 16

/* ABI version of the loaded library (== SAGE_ABI_VERSION it was built with).
 * No reference counterpart (the reference binds through the torch dispatcher). */
int sage_abi_version(void);

/* Message of the last failed call on this thread ("" if none).
 * No reference counterpart (reference: Python asserts, sageattention/core.py:50-63,91-95). */
const char* sage_last_error(void);

/* Bytes of fp32 workspace sage_k_mean needs for this shape. */
int64_t sage_k_mean_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim);

/*
 * K mean over the sequence for smooth_k: mean_out[b,h,d] = dtype(sum_s fp32(key[b,s,h,d]) / S).
 * mean_out is contiguous [B,H,D] of `dtype`; workspace holds
 * sage_k_mean_workspace_bytes() bytes (no initialisation needed).
 * Replaces mean_seq (csrc/pybind_gfx11.cpp:36, csrc/attn_gfx11.h:48,
 * csrc/attn_gfx11.cu:1937-1972; kernel :94-145).
 */
int sage_k_mean(const void* key, void* mean_out, void* workspace, int dtype,
                int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                int64_t stride_b, int64_t stride_h, int64_t stride_n, void* stream);

/*
 * Per-block INT8 quantisation of Q (pre-scaled by fp32(sm_scale)*log2(e),
 * groups of SAGE_Q_GROUP tokens) and K (minus key_mean when non-NULL, groups
 * of SAGE_K_GROUP tokens), in one launch.
 * Outputs (contiguous): q_i8 [B,Hq,Sq,D] int8, q_scale [B,Hq,ceil(Sq/32)] fp32,
 * k_i8 [B,Hkv,Sk,D] int8, k_scale [B,Hkv,ceil(Sk/16)] fp32.  key_mean is
 * contiguous [B,Hkv,D] of `dtype`.
 * Replaces quant_qk_int8 (csrc/pybind_gfx11.cpp:32-35, csrc/attn_gfx11.h:41-46,
 * csrc/attn_gfx11.cu:1974-2067; kernel :147-321), except that the caller
 * allocates the four outputs.
 */
int sage_quant_qk_i8(const void* query, const void* key, const void* key_mean,
                     int8_t* q_i8, float* q_scale, int8_t* k_i8, float* k_scale, int dtype,
                     int64_t batch, int64_t q_heads, int64_t kv_heads,
                     int64_t q_len, int64_t kv_len, int64_t head_dim,
                     int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_n,
                     int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_n,
                     double sm_scale, void* stream);

/* Token length of V_T rows: ceil(seq_len / SAGE_VT_ALIGN) * SAGE_VT_ALIGN. */
int64_t sage_v_layout_padded_len(int64_t seq_len);

/*
 * V -> V_T fp16 [B,H,D,padded_len] contiguous, tokens contiguous, zero padded
 * past seq_len, bf16 converted to fp16 with round-to-nearest-even.
 * Replaces v_transpose (csrc/pybind_gfx11.cpp:37, csrc/attn_gfx11.h:51,
 * csrc/attn_gfx11.cu:1889-1935; kernel :323-407).
 */
int sage_v_layout(const void* value, void* value_t, int dtype,
                  int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                  int64_t stride_b, int64_t stride_h, int64_t stride_n, void* stream);

/*
 * The K half of sage_quant_qk_i8 (K minus key_mean when non-NULL, groups of
 * SAGE_K_GROUP tokens) and sage_v_layout in one launch, with the same outputs
 * bit for bit: k_i8 [B,Hkv,Sk,D] int8 and k_scale [B,Hkv,ceil(Sk/16)] fp32
 * (contiguous), value_t [B,Hkv,D,padded_len] fp16.  key and value share
 * `dtype`, each with its own strides.  What sageattn runs before
 * sage_attn_i8_fwd_qfused (which quantises Q itself).
 * No single reference counterpart: the K half of quant_qk_int8
 * (csrc/attn_gfx11.cu:1974-2067) plus v_transpose (:1889-1935).
 */
int sage_prep_kv_i8(const void* key, const void* value, const void* key_mean, int8_t* k_i8, float* k_scale,
                    void* value_t, int dtype, int64_t batch, int64_t kv_heads, int64_t kv_len, int64_t head_dim,
                    int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_n,
                    int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_n, void* stream);

/*
 * sage_k_mean followed by sage_prep_kv_i8 with that mean (smooth_k), in two
 * launches instead of three: the K mean's chunk sums (into `workspace`, which
 * holds sage_k_mean_workspace_bytes() bytes, no initialisation), then one
 * launch in which the K-quantisation blocks finish the mean themselves (the
 * same additions in the same order as sage_k_mean, so the same mean bit for
 * bit) and quantise K minus it, beside the V layout blocks.  Outputs equal
 * sage_k_mean + sage_prep_kv_i8 bit for bit: k_i8, k_scale, value_t as there,
 * and key_mean [B,Hkv,D] contiguous of `dtype` (2-byte aligned; NULL = not
 * written).  Calls sharing one workspace on different streams race.
 * No single reference counterpart: mean_seq (csrc/attn_gfx11.cu:1937-1972,
 * kernel :94-145) and the K half of quant_qk_int8 (:1974-2067) with
 * v_transpose (:1889-1935), as sageattention/core.py:173-193 calls them.
 */
int sage_prep_kv_i8_smooth(const void* key, const void* value, void* key_mean, void* workspace, int8_t* k_i8,
                           float* k_scale, void* value_t, int dtype, int64_t batch, int64_t kv_heads,
                           int64_t kv_len, int64_t head_dim, int64_t k_stride_b, int64_t k_stride_h,
                           int64_t k_stride_n, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_n,
                           void* stream);

/*
 * Fused attention: S = (q_i8 . k_i8) * q_scale * k_scale (log2 domain), causal
 * mask top-left (key j > query i masked), online softmax with exp2, P rounded
 * to fp16, O = P . V_T (fp32 accumulation), out = O / rowsum cast to out_dtype.
 * Inputs are the outputs of sage_quant_qk_i8 and sage_v_layout; GQA maps query
 * head hq to kv head hq / (q_heads / kv_heads).  `out` is [B,Sq,Hq,D] or
 * [B,Hq,Sq,D] by its strides (multiples of 8 elements, 16-byte aligned base,
 * as the reference's 16-byte output stores need, csrc/attn_gfx11.cu:766-824).
 * Replaces qk_int8_sv_bf16_attn_t (csrc/pybind_gfx11.cpp:19-23,
 * csrc/attn_gfx11.h:10-19, csrc/attn_gfx11.cu:2069-2273; kernel :409-1243).
 */
int sage_attn_i8_fwd(const int8_t* q_i8, const int8_t* k_i8, const void* value_t, void* out,
                     const float* q_scale, const float* k_scale, int out_dtype,
                     int64_t batch, int64_t q_heads, int64_t kv_heads,
                     int64_t q_len, int64_t kv_len, int64_t head_dim,
                     int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                     int is_causal, void* stream);

/*
 * sage_attn_i8_fwd plus each row's log-sum-exp: lse [B,Hq,Sq] fp32
 * contiguous (4-byte aligned; NULL = not written) receives
 * ln(sum_j exp(s_ij)) over the natural-log scores s_ij = q_i.k_j * sm_scale
 * after dequantisation (the log2-domain score times ln 2), -inf for a row with
 * no live key.  The reference's return_lse returns a zero placeholder instead
 * (sageattention/core.py:203-211); this is the value that placeholder stands
 * for, usable to merge partial attentions over split key ranges.
 */
int sage_attn_i8_fwd_lse(const int8_t* q_i8, const int8_t* k_i8, const void* value_t, void* out,
                         float* lse, const float* q_scale, const float* k_scale, int out_dtype,
                         int64_t batch, int64_t q_heads, int64_t kv_heads,
                         int64_t q_len, int64_t kv_len, int64_t head_dim,
                         int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                         int is_causal, void* stream);

/*
 * Key splits of the two entry points below (non-causal launches only).  A
 * launch has B*Hq*ceil(q_len/R) q-blocks, R = 128 query rows for head_dim 64
 * non-causal launches, for causal launches (every kind) whose 256-row
 * q-blocks would fill at most half the CUs, and for causal launches whose
 * 256-row q-blocks fill at most one round when a cost model of the schedule
 * rates 128-row q-blocks faster; R = 256 otherwise (one block per CU).
 * Non-causal 128-row blocks run two per CU, causal ones one per CU (more of
 * them than CUs run as a persistent grid, a heavy and a light q-block per
 * block); for a non-causal
 * launch that leaves compute units idle
 * (fewer blocks than CUs, or a last round partly filled) the key range of
 * some or all blocks can be split into parts whose fp32 partial outputs and
 * log-sum-exps a second launch merges exactly
 * (o = sum_s e^{lse_s - lse} o_s, lse = ln sum_s e^{lse_s}); the result
 * differs from the unsplit one only by rounding.
 *   num_splits 0: the library chooses (a cost model over the device's CU
 *                 count), using only counts whose workspace fits in
 *                 workspace_bytes (workspace NULL: unsplit);
 *   num_splits 1: unsplit;
 *   num_splits n in [2, SAGE_MAX_KV_SPLITS]: n splits (at most one per 64
 *                 keys); the workspace must hold sage_attn_workspace_bytes().
 * Causal launches ignore num_splits.  The workspace (16-byte aligned, no
 * initialisation) is overwritten by the call and may be reused once the call
 * has completed on its stream; calls sharing one workspace on different
 * streams race.
 * Returns the bytes the given launch needs (0: it runs unsplit), or a
 * negative status.  `quantized` selects sage_attn_i8_fwd_qfused (1) or
 * sage_attn_direct_fwd (0); with num_splits 0 the answer depends on the
 * current device.
 * No reference counterpart (the reference launches one block per q-tile).
 */
int64_t sage_attn_workspace_bytes(int quantized, int64_t batch, int64_t q_heads, int64_t q_len, int64_t kv_len,
                                  int64_t head_dim, int is_causal, int num_splits);

/*
 * The split plan such a launch runs: q-blocks (R query rows of one head as
 * above, numbered head-major) [0, *whole_qblocks) run whole, and every later one in
 * *splits key ranges (*splits == 1: nothing is split).  num_splits 0 may
 * choose to split only the q-blocks of the last, partly filled round of the
 * device; a forced n > 1 splits every q-block.  Same arguments and
 * device dependence as sage_attn_workspace_bytes.
 * No reference counterpart.
 */
int sage_attn_split_plan(int quantized, int64_t batch, int64_t q_heads, int64_t q_len, int64_t kv_len,
                         int64_t head_dim, int is_causal, int num_splits, int64_t* whole_qblocks, int* splits);

/*
 * sage_attn_i8_fwd_lse with the Q quantisation done by the attention kernel
 * itself: `query` is the caller's fp16/bf16 Q (any 16-byte-aligned strides,
 * HND or NHD, `dtype` = its type and the output's), quantised per 32-token
 * group exactly as sage_quant_qk_i8 does (scale fl(sm_scale)*log2(e), same
 * rounding), so the unsplit result equals sage_quant_qk_i8 followed by
 * sage_attn_i8_fwd_lse bit for bit, without the int8 Q round trip through
 * HBM.  K comes from sage_quant_qk_i8 (called with q_len = 0), V_T from
 * sage_v_layout; lse may be NULL.  num_splits / workspace: see
 * sage_attn_workspace_bytes.
 * No single reference counterpart: it fuses the Q half of quant_qk_int8
 * (csrc/attn_gfx11.cu:1974-2067) into qk_int8_sv_bf16_attn_t (:2069-2273).
 */
int sage_attn_i8_fwd_qfused(const void* query, const int8_t* k_i8, const void* value_t, void* out,
                            float* lse, const float* k_scale, int dtype,
                            int64_t batch, int64_t q_heads, int64_t kv_heads,
                            int64_t q_len, int64_t kv_len, int64_t head_dim,
                            int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_n,
                            int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                            int is_causal, double sm_scale, int num_splits, void* workspace,
                            int64_t workspace_bytes, void* stream);

/*
 * sage_attn_i8_fwd_qfused for fp16 inputs with V read in place: `value` is
 * the caller's fp16 V [B,Hkv,Sk,D] through its strides (HND or NHD; 16-byte
 * aligned base, strides multiples of 8 elements, rows not overlapping) instead
 * of a V_T from sage_v_layout, so the V layout pass and its HBM round trip
 * are skipped (the kernel transposes V tiles in LDS with ds_read_b64_tr_b16).
 * dtype must be SAGE_DTYPE_F16 (Q, V and out); K from sage_quant_qk_i8 as for
 * sage_attn_i8_fwd_qfused.  The MFMAs see the same V values in the same
 * order, so results equal sage_v_layout + sage_attn_i8_fwd_qfused bit for
 * bit.  No single reference counterpart: it replaces v_transpose
 * (csrc/attn_gfx11.cu:1889-1935, kernel :323-407; sageattention/core.py:173-179)
 * followed by the INT8 attention (:2069-2273) for fp16 V.
 */
int sage_attn_i8_fwd_qfused_vrows(const void* query, const int8_t* k_i8, const void* value, void* out,
                                  float* lse, const float* k_scale, int dtype,
                                  int64_t batch, int64_t q_heads, int64_t kv_heads,
                                  int64_t q_len, int64_t kv_len, int64_t head_dim,
                                  int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_n,
                                  int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_n,
                                  int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                                  int is_causal, double sm_scale, int num_splits, void* workspace,
                                  int64_t workspace_bytes, void* stream);

/*
 * sage_attn_i8_fwd_qfused without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The key
 * splits' partial outputs go to a scratch array of 64 MiB that the library
 * holds in each GPU's memory until the process ends; the call allocates
 * nothing.  A forced n > 1 whose partials would not fit fails with
 * SAGE_ERR_UNSUPPORTED.  num_splits 0 runs the plan sage_attn_i8_fwd_qfused
 * would choose (sage_attn_split_plan) when its partials fit the scratch, and
 * otherwise the best plan that fits, whose result differs by rounding only.
 * Every call on one GPU shares that GPU's scratch: calls that overlap on one
 * GPU (different streams, or host threads) race on it; calls ordered on one
 * stream do not.  The first call that may split, per device, looks the
 * scratch's address up (with that device current).  Results equal those of
 * sage_attn_i8_fwd_qfused with the same num_splits whenever the plans agree.
 */
int sage_attn_i8_fwd_qfused_noalloc(const void* query, const int8_t* k_i8, const void* value_t, void* out,
                                    float* lse, const float* k_scale, int dtype,
                                    int64_t batch, int64_t q_heads, int64_t kv_heads,
                                    int64_t q_len, int64_t kv_len, int64_t head_dim,
                                    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_n,
                                    int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                                    int is_causal, double sm_scale, int num_splits, void* stream);

/*
 * Direct attention without quantisation (the reference's short-sequence
 * branch): S = fp32(q . k) * fl(fl(sm_scale) * log2 e) from fp16/bf16 Q and K
 * (fp32 accumulation), the same masks and online softmax as sage_attn_i8_fwd,
 * P rounded to fp16, O = P . V_T with V_T from sage_v_layout, out = O / rowsum
 * cast to `dtype` (the type of query, key and out).  query/key are read in
 * place through their strides (HND or NHD; multiples of 8 elements, 16-byte
 * aligned bases, key rows must not overlap); lse as in sage_attn_i8_fwd_lse
 * (NULL = not written); num_splits / workspace: see sage_attn_workspace_bytes.
 * Replaces fp16_attn_t / bf16_attn_t (csrc/pybind_gfx11.cpp:24-31,
 * csrc/attn_gfx11.h:21-39, csrc/attn_gfx11.cu:2275-2472; kernels :1465-1885);
 * their bm_sel tile override has no counterpart (one tile shape on gfx950).
 */
int sage_attn_direct_fwd(const void* query, const void* key, const void* value_t, void* out, float* lse,
                         int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                         int64_t q_len, int64_t kv_len, int64_t head_dim,
                         int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_n,
                         int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_n,
                         int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                         int is_causal, double sm_scale, int num_splits, void* workspace,
                         int64_t workspace_bytes, void* stream);

/*
 * sage_attn_direct_fwd for fp16 inputs with V read in place: `value` is the
 * caller's fp16 V [B,Hkv,Sk,D] through its strides (HND or NHD; 16-byte
 * aligned base, strides multiples of 8 elements, rows not overlapping) instead
 * of a V_T from sage_v_layout, so the short-sequence branch is one launch
 * (the kernel transposes V tiles in LDS with ds_read_b64_tr_b16).  dtype must
 * be SAGE_DTYPE_F16 (Q, K, V and out).  The MFMAs see the same V values in the
 * same order, so results equal sage_v_layout + sage_attn_direct_fwd bit for
 * bit.  No single reference counterpart: it replaces v_transpose
 * (csrc/attn_gfx11.cu:1889-1935, kernel :323-407; sageattention/core.py:153-164)
 * followed by fp16_attn_t (csrc/pybind_gfx11.cpp:24-31, csrc/attn_gfx11.cu:2275-2472).
 */
int sage_attn_direct_fwd_vrows(const void* query, const void* key, const void* value, void* out, float* lse,
                               int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                               int64_t q_len, int64_t kv_len, int64_t head_dim,
                               int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_n,
                               int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_n,
                               int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_n,
                               int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                               int is_causal, double sm_scale, int num_splits, void* workspace,
                               int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SAGEATTN_MI355X_H */
