// Fused flash attention for gfx950 (CDNA4, wave64 MFMA): the INT8 quantized
// path and the direct fp16/bf16 path, one kernel template.  The kernels and
// their host code live in attn_body.inc, compiled here in two block shapes;
// this file holds the C entry points, which pick the shape per launch.  The
// mapping below describes the 256-row shape (8 waves); the 128-row shape has
// 4 waves and two blocks per CU.
//
// Math (csrc/attn_gfx11.cu of the reference):
//   INT8   (:409-825)   s_ij = float(sum_d q8[i,d] * k8[j,d]) * (q_scale[i/32] * k_scale[j/16])
//   direct (:1465-1885) s_ij = fp32(sum_d q[i,d] * k[j,d]) * fl(sm_scale * log2 e)  (fp16 or bf16 Q/K)
// in the log2 domain (INT8: Q was pre-scaled by sm_scale*log2 e), causal mask
// j > i (top-left) and j >= Sk, online softmax with exp2, P rounded to fp16
// (RNE), O += P.V_T with fp32 accumulation (V_T fp16 in both paths), out =
// O * (1/l) cast to fp16/bf16.
//
// Mapping onto CDNA4:
//   * block = 8 waves x 32 query rows (BM = 256), one block per CU, two waves
//     per SIMD; KV tiles of BN = 64 keys shared by all 8 waves through LDS;
//   * S^T = K . Q^T: A = K rows from LDS, B = the wave's Q^T fragment held in
//     registers for the whole kernel (v_mfma_i32_32x32x32_i8, or
//     v_mfma_f32_32x32x16_f16/bf16 for the direct path: both take 32 bytes of
//     each row per MFMA).  The 32x32 accumulator puts one query per lane
//     column (lane & 31), so the row softmax is 32 in-lane values plus one
//     permlane32 swap;
//   * O^T = V^T . P^T with v_mfma_f32_32x32x16_f16: B = P^T taken straight
//     from the S^T accumulators (no LDS round trip), A = V_T rows from LDS.
//     K rows sit in LDS with bits 2 and 3 of the key index swapped, which
//     makes accumulator register r of lane half h hold key 16(r/8) + 8h + r%8:
//     exactly the 8 consecutive keys the PV operand wants from that lane;
//   * software pipeline inside every wave: step j runs the softmax of tile j
//     (VALU) interleaved with the MFMAs of P_{j-1}.V_{j-1} and S_{j+1} =
//     K_{j+1}.Q^T, so each wave keeps the matrix core and the VALU busy at
//     once and the two waves of a SIMD fill each other's gaps.  A single wave
//     issues VALU at half the SIMD's rate, so both waves of a SIMD carry
//     softmax work all the time (no MFMA-only / VALU-only roles).  S and P are
//     rewritten in place: the chunk order reads each before overwriting it;
//   * online softmax with a lazy reference max: the max moves only when a row
//     max grows by more than 2^8; O is then rescaled at the top of the next
//     step, after the P.V MFMAs that still used the old max.  The unmasked
//     loop tests each lane's tile sum of p against 2^8 after the exponentials
//     instead of taking the max first, and redoes the rare tile that fails
//     with the max moved (TileSoftmaxSum);
//   * K/V tiles stream into a 3-stage LDS ring with buffer_load ... lds
//     (no staging registers), issued two steps ahead; loads past the block's
//     last key read as zero through the descriptor's record count.  The
//     direct path reads K (and Q) straight from the caller's strided tensors;
//   * causal: the KV loop stops at the block's last row, masks only on tail /
//     diagonal tiles;
//   * work items (a q-block, or a key range of one for split launches) go to
//     XCDs in contiguous ranges (consecutive q-blocks of a head share an XCD's
//     L2 for K/V), heaviest causal blocks first; with more items than CUs a
//     persistent grid of one block per CU walks a static snake schedule
//     instead of relying on the hardware dispatcher (see attn_fwd_kernel);
//   * the epilogue stages each wave's output rows in LDS and writes whole
//     rows; non-causal launches that leave CUs idle can split key ranges,
//     merged by attn_merge_kernel with the partial LSEs.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <type_traits>
#include <utility>

#include "sage_common.h"

namespace sage {
namespace {

// Compute units of the current device, read once per device (256, the
// MI355X count, if the runtime cannot tell).
int device_cus() {
  constexpr int kDevs = 64;
  static std::atomic<int> cache[kDevs];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    (void)hipGetLastError();
    return 256;
  }
  if (dev < kDevs) {
    const int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) {
    (void)hipGetLastError();
    v = 256;
  }
  if (dev < kDevs) cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

}  // namespace

// The kernels and their host code in two block shapes (attn_body.inc):
//   * w8: 8 waves x 32 query rows = 256-row q-blocks, one block per CU;
//   * w4: 4 waves x 32 query rows = 128-row q-blocks, two blocks per CU, whose
//     waves do not share barriers, so one block's prologue, epilogue and
//     barrier waits overlap the other's key loop; each block loads its own K/V
//     tiles (twice the L2->LDS traffic of w8).
// w4 runs the D = 64 non-causal launches (direct and INT8) and the causal
// launches with few q-blocks (small_blocks), w8 all others.  Same-box timings
// against w8 (identical outputs): D = 64 non-causal -7% to -27% (the direct
// kernel at B1 H20 S1024: 21.3 -> 15.6 us; INT8 at B1 H10 S4096: 65.9 -> 56.2
// us); causal launches of one or more full rounds +2% to +6% and D = 128
// non-causal launches with key splits +3% to +4% (the doubled tile traffic),
// so those stay on w8.  The D = 128 direct kernel's 98 KB of LDS fits once per
// CU: its w4 launches (causal, few q-blocks) run one block per CU.
// The stamps build (build.py --stamps, SAGE_STAMPS=1) adds per-wave cycle
// stamps to the attention kernels (attn_body.inc, StampField) and the two
// functions below that read them; the default build has neither.
#ifndef SAGE_STAMPS
#define SAGE_STAMPS 0
#endif
#if SAGE_STAMPS
constexpr int kStampBlocks = 2048;  // blocks whose waves record (8 waves each at most)
constexpr int kStampStride = 32;    // uint64 fields per wave record
__device__ uint64_t g_stamps[kStampBlocks * 8 * kStampStride];
#endif

namespace w8 {
constexpr int kBM = 256;
constexpr int kWaves = 8;
constexpr int kBlocksPerCu = 1;
constexpr bool kSmallShape = false;
#include "attn_body.inc"
}  // namespace w8

namespace w4 {
constexpr int kBM = 128;
constexpr int kWaves = 4;
constexpr int kBlocksPerCu = 2;
constexpr bool kSmallShape = true;
#include "attn_body.inc"
}  // namespace w4

// A lone 128-row block on a CU takes this fraction of a 256-row block's time
// per key tile step (MI355X, B1 H32 S2048 causal: the D = 128 direct kernel
// 0.97 against 1.38 us; fitted to the Q-fused INT8 kernel's paired launches at
// B1 H16 S4096 and B1 H32 S2048: 0.77).
constexpr double kLoneHalfBlockTileDirect = 0.70;
constexpr double kLoneHalfBlockTileI8 = 0.77;

// The shape a launch runs: w4 for D = 64 non-causal launches, and for causal
// launches whose 256-row q-blocks would fill at most half the CUs (their
// 128-row q-blocks then fill twice as many, one block per CU; B1 H8 S4096
// D128 INT8: -27%; the D = 128 direct kernel, whose 98 KB of LDS fits once per
// CU, at B1 H8/H16 S1024-2048: -27% to -32%); w8 for the rest (a causal launch
// of 2048 +4% in w4).  A causal launch also runs w4 when its 256-row
// q-blocks fill one round and the causal cost model rates the 128-row q-blocks
// faster: with one block resident per CU they run as a persistent grid in
// which the snake schedule gives each block a heavy and a light q-block.
// D = 128 direct kernel: B1 H32 S2048, B2 H16 S2048 -17%, B1 H24 S2048 -15%,
// B1 H16 S4096 -21%; Q-fused INT8 kernel: B1 H16 S4096, B2 H8 S4096 -15%,
// B1 H12 S4096 -19%, B1 H32 S2048 -10%; D = 64: direct B1 H32 S2048 -16%,
// B1 H20 S3072 -5%, INT8 B1 H16 S4096 -16%, B1 H32 S2048 -9%.  The model
// keeps B1 H32 S1536 D128 direct in w8, where a block would get two heavy
// q-blocks (+15% in w4).
bool small_blocks(int64_t head_dim, int is_causal, int64_t batch, int64_t q_heads, int64_t q_len, int64_t kv_len,
                  bool direct) {
  if (is_causal == 0) return head_dim == 64;
  const int64_t qblocks = batch * q_heads * ((q_len + 255) / 256);
  if (qblocks <= 0) return false;
  if (qblocks * 2 <= device_cus()) return true;
  if (qblocks > device_cus()) return false;
  const double f = direct ? kLoneHalfBlockTileDirect : kLoneHalfBlockTileI8;
  if (head_dim == 64)
    return f * w4::causal_blocks_cost<64, w4::kQkBf16>(batch * q_heads, q_len, kv_len) <
           w8::causal_blocks_cost<64, w8::kQkBf16>(batch * q_heads, q_len, kv_len);
  return f * w4::causal_blocks_cost<128, w4::kQkBf16>(batch * q_heads, q_len, kv_len) <
         w8::causal_blocks_cost<128, w8::kQkBf16>(batch * q_heads, q_len, kv_len);
}

}  // namespace sage


using namespace sage;

// Scratch of sage_attn_i8_fwd_qfused_noalloc (the key splits' partial outputs
// and LSEs): device memory the library holds until the process ends, one copy
// per GPU.  The name is a host-side stand-in for host code; kernels get the
// device address that hipGetSymbolAddress returns for the current device.
// 64 MiB holds the automatic plans of about 95% of shapes (a sweep of B 1-4,
// H 1-64, S 256-40k, D 64/128 on 256 CUs: 4.5% need more, up to 161 MiB),
// among them every 256-piece plan of 256-row D = 128 q-blocks (33.8 MB).
constexpr int64_t kScratchBytes = int64_t{64} << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {
// The current device's address of `scratch`, looked up once per device (with
// that device current) and kept; null with the error recorded if the runtime
// cannot give it.
void* scratch_address(const char* fn) {
  constexpr int kDevs = 64;
  static std::atomic<void*> cache[kDevs];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kDevs) {
    (void)hipGetLastError();
    set_error(SAGE_ERR_HIP, "%s: no current device (%s)", fn, e != hipSuccess ? hipGetErrorString(e) : "out of range");
    return nullptr;
  }
  void* ptr = cache[dev].load(std::memory_order_acquire);
  if (ptr != nullptr) return ptr;
  e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr) {
    (void)hipGetLastError();
    set_error(SAGE_ERR_HIP, "%s: hipGetSymbolAddress(scratch) failed: %s", fn, hipGetErrorString(e));
    return nullptr;
  }
  cache[dev].store(ptr, std::memory_order_release);
  return ptr;
}

// attn_fwd of the block shape the launch runs (the arguments include head_dim and is_causal again)
template <typename... Args>
int run_attn(int64_t head_dim, int is_causal, int64_t batch, int64_t q_heads, int64_t q_len, int64_t kv_len, int qk,
             Args... args) {
  const bool direct = qk == w8::kQkF16 || qk == w8::kQkBf16 || qk == w8::kQkF16V;
  return small_blocks(head_dim, is_causal, batch, q_heads, q_len, kv_len, direct) ? w4::attn_fwd(qk, args...)
                                                                                  : w8::attn_fwd(qk, args...);
}

// The plan of the shape the launch runs and its workspace bytes (or a negative status).
int64_t split_plan(bool quantized, int64_t batch, int64_t q_heads, int64_t q_len, int64_t kv_len, int64_t head_dim,
                   int is_causal, int num_splits, int64_t* whole, int* splits) {
  int64_t r;
  if (small_blocks(head_dim, is_causal, batch, q_heads, q_len, kv_len, !quantized)) {
    w4::SplitPlan sp;
    r = w4::attn_split_plan(quantized, batch, q_heads, q_len, kv_len, head_dim, is_causal, num_splits, &sp);
    *whole = sp.nfull;
    *splits = static_cast<int>(sp.nsplit);
  } else {
    w8::SplitPlan sp;
    r = w8::attn_split_plan(quantized, batch, q_heads, q_len, kv_len, head_dim, is_causal, num_splits, &sp);
    *whole = sp.nfull;
    *splits = static_cast<int>(sp.nsplit);
  }
  return r;
}
}  // namespace

extern "C" int sage_attn_i8_fwd(const int8_t* q_i8, const int8_t* k_i8, const void* value_t, void* out,
                                const float* q_scale, const float* k_scale, int out_dtype,
                                int64_t batch, int64_t q_heads, int64_t kv_heads,
                                int64_t q_len, int64_t kv_len, int64_t head_dim,
                                int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                                int is_causal, void* stream) {
  clear_error();
  return run_attn(head_dim, is_causal, batch, q_heads, q_len, kv_len, w8::kQkI8, q_i8, k_i8, value_t, out, nullptr,
                  q_scale, k_scale, out_dtype, batch, q_heads, kv_heads, q_len, kv_len, head_dim,
                  q_heads * q_len * head_dim, q_len * head_dim, head_dim, kv_heads * kv_len * head_dim,
                  kv_len * head_dim, head_dim, 0, 0, 0, o_stride_b, o_stride_h, o_stride_n, is_causal, 0.0, 1, nullptr,
                  0, stream, "sage_attn_i8_fwd");
}

extern "C" int sage_attn_i8_fwd_lse(const int8_t* q_i8, const int8_t* k_i8, const void* value_t, void* out,
                                    float* lse, const float* q_scale, const float* k_scale, int out_dtype,
                                    int64_t batch, int64_t q_heads, int64_t kv_heads,
                                    int64_t q_len, int64_t kv_len, int64_t head_dim,
                                    int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                                    int is_causal, void* stream) {
  clear_error();
  return run_attn(head_dim, is_causal, batch, q_heads, q_len, kv_len, w8::kQkI8, q_i8, k_i8, value_t, out, lse, q_scale,
                  k_scale, out_dtype, batch, q_heads, kv_heads, q_len, kv_len, head_dim, q_heads * q_len * head_dim,
                  q_len * head_dim, head_dim, kv_heads * kv_len * head_dim, kv_len * head_dim, head_dim, 0, 0, 0,
                  o_stride_b, o_stride_h, o_stride_n, is_causal, 0.0, 1, nullptr, 0, stream, "sage_attn_i8_fwd_lse");
}

extern "C" int sage_attn_direct_fwd(const void* query, const void* key, const void* value_t, void* out, float* lse,
                                    int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                    int64_t q_len, int64_t kv_len, int64_t head_dim,
                                    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_n,
                                    int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_n,
                                    int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                                    int is_causal, double sm_scale, int num_splits, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  clear_error();
  return run_attn(head_dim, is_causal, batch, q_heads, q_len, kv_len,
                  dtype == SAGE_DTYPE_BF16 ? w8::kQkBf16 : w8::kQkF16, query, key, value_t, out, lse, nullptr, nullptr,
                  dtype, batch, q_heads, kv_heads, q_len, kv_len, head_dim, q_stride_b, q_stride_h, q_stride_n,
                  k_stride_b, k_stride_h, k_stride_n, 0, 0, 0, o_stride_b, o_stride_h, o_stride_n, is_causal, sm_scale,
                  num_splits, workspace, workspace_bytes, stream, "sage_attn_direct_fwd");
}

extern "C" int sage_attn_direct_fwd_vrows(const void* query, const void* key, const void* value, void* out,
                                          float* lse, int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                          int64_t q_len, int64_t kv_len, int64_t head_dim,
                                          int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_n,
                                          int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_n,
                                          int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_n,
                                          int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                                          int is_causal, double sm_scale, int num_splits, void* workspace,
                                          int64_t workspace_bytes, void* stream) {
  clear_error();
  return run_attn(head_dim, is_causal, batch, q_heads, q_len, kv_len, w8::kQkF16V, query, key, value, out, lse, nullptr,
                  nullptr, dtype, batch, q_heads, kv_heads, q_len, kv_len, head_dim, q_stride_b, q_stride_h,
                  q_stride_n, k_stride_b, k_stride_h, k_stride_n, v_stride_b, v_stride_h, v_stride_n, o_stride_b,
                  o_stride_h, o_stride_n, is_causal, sm_scale, num_splits, workspace, workspace_bytes, stream,
                  "sage_attn_direct_fwd_vrows");
}

extern "C" int sage_attn_i8_fwd_qfused(const void* query, const int8_t* k_i8, const void* value_t, void* out,
                                       float* lse, const float* k_scale, int dtype,
                                       int64_t batch, int64_t q_heads, int64_t kv_heads,
                                       int64_t q_len, int64_t kv_len, int64_t head_dim,
                                       int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_n,
                                       int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                                       int is_causal, double sm_scale, int num_splits, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  clear_error();
  return run_attn(head_dim, is_causal, batch, q_heads, q_len, kv_len, w8::kQkI8F, query, k_i8, value_t, out, lse,
                  nullptr, k_scale, dtype, batch, q_heads, kv_heads, q_len, kv_len, head_dim, q_stride_b, q_stride_h,
                  q_stride_n, kv_heads * kv_len * head_dim, kv_len * head_dim, head_dim, 0, 0, 0, o_stride_b,
                  o_stride_h, o_stride_n, is_causal, sm_scale, num_splits, workspace, workspace_bytes, stream,
                  "sage_attn_i8_fwd_qfused");
}

extern "C" int sage_attn_i8_fwd_qfused_vrows(const void* query, const int8_t* k_i8, const void* value, void* out,
                                             float* lse, const float* k_scale, int dtype,
                                             int64_t batch, int64_t q_heads, int64_t kv_heads,
                                             int64_t q_len, int64_t kv_len, int64_t head_dim,
                                             int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_n,
                                             int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_n,
                                             int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                                             int is_causal, double sm_scale, int num_splits, void* workspace,
                                             int64_t workspace_bytes, void* stream) {
  clear_error();
  return run_attn(head_dim, is_causal, batch, q_heads, q_len, kv_len, w8::kQkI8FV, query, k_i8, value, out, lse,
                  nullptr, k_scale, dtype, batch, q_heads, kv_heads, q_len, kv_len, head_dim, q_stride_b, q_stride_h,
                  q_stride_n, kv_heads * kv_len * head_dim, kv_len * head_dim, head_dim, v_stride_b, v_stride_h,
                  v_stride_n, o_stride_b, o_stride_h, o_stride_n, is_causal, sm_scale, num_splits, workspace,
                  workspace_bytes, stream, "sage_attn_i8_fwd_qfused_vrows");
}

extern "C" int sage_attn_i8_fwd_qfused_noalloc(const void* query, const int8_t* k_i8, const void* value_t, void* out,
                                               float* lse, const float* k_scale, int dtype,
                                               int64_t batch, int64_t q_heads, int64_t kv_heads,
                                               int64_t q_len, int64_t kv_len, int64_t head_dim,
                                               int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_n,
                                               int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                                               int is_causal, double sm_scale, int num_splits, void* stream) {
  static const char* const fn = "sage_attn_i8_fwd_qfused_noalloc";
  clear_error();
  // a forced split count must fit the scratch (an automatic plan is chosen within it)
  if (num_splits > 1 && is_causal == 0) {
    int64_t whole = 0;
    int splits = 0;
    const int64_t need = split_plan(true, batch, q_heads, q_len, kv_len, head_dim, 0, num_splits, &whole, &splits);
    if (need < 0) return static_cast<int>(need);
    if (need > kScratchBytes)
      return set_error(SAGE_ERR_UNSUPPORTED, "%s: %d key splits need %lld bytes of scratch, beyond its %lld", fn,
                       num_splits, static_cast<long long>(need), static_cast<long long>(kScratchBytes));
  }
  // only a launch that may split touches the scratch (causal launches, unsplit
  // ones and empty ones never do)
  void* ws = nullptr;
  if (is_causal == 0 && num_splits != 1 && batch > 0 && q_len > 0 && kv_len > 0) {
    ws = scratch_address(fn);
    if (ws == nullptr) return SAGE_ERR_HIP;
  }
  return run_attn(head_dim, is_causal, batch, q_heads, q_len, kv_len, w8::kQkI8F, query, k_i8, value_t, out, lse,
                  nullptr, k_scale, dtype, batch, q_heads, kv_heads, q_len, kv_len, head_dim, q_stride_b, q_stride_h,
                  q_stride_n, kv_heads * kv_len * head_dim, kv_len * head_dim, head_dim, 0, 0, 0, o_stride_b,
                  o_stride_h, o_stride_n, is_causal, sm_scale, num_splits, ws, ws != nullptr ? kScratchBytes : 0,
                  stream, fn);
}

extern "C" int64_t sage_attn_workspace_bytes(int quantized, int64_t batch, int64_t q_heads, int64_t q_len,
                                             int64_t kv_len, int64_t head_dim, int is_causal, int num_splits) {
  clear_error();
  int64_t whole = 0;
  int splits = 0;
  return split_plan(quantized != 0, batch, q_heads, q_len, kv_len, head_dim, is_causal, num_splits, &whole, &splits);
}

extern "C" int sage_attn_split_plan(int quantized, int64_t batch, int64_t q_heads, int64_t q_len, int64_t kv_len,
                                    int64_t head_dim, int is_causal, int num_splits, int64_t* whole_qblocks,
                                    int* splits) {
  clear_error();
  if (whole_qblocks == nullptr || splits == nullptr)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_attn_split_plan: null output pointer");
  const int64_t r =
      split_plan(quantized != 0, batch, q_heads, q_len, kv_len, head_dim, is_causal, num_splits, whole_qblocks, splits);
  return r < 0 ? static_cast<int>(r) : SAGE_OK;
}

#if SAGE_STAMPS
// Stamps build only: copy `bytes` of the wave records (kStampStride uint64
// fields per wave, block-major) to host memory / clear them.
extern "C" int sage_stamps_read(void* host, size_t bytes) {
  if (bytes > sizeof(sage::g_stamps)) return SAGE_ERR_INVALID_ARG;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(sage::g_stamps), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess
             ? SAGE_OK
             : SAGE_ERR_HIP;
}
extern "C" int sage_stamps_clear(void) {
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(sage::g_stamps)) != hipSuccess) return SAGE_ERR_HIP;
  return hipMemset(ptr, 0, sizeof(sage::g_stamps)) == hipSuccess ? SAGE_OK : SAGE_ERR_HIP;
}
#endif
