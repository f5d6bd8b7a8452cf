// Fused flash attention for gfx950 (CDNA4, wave64 MFMA): the INT8 quantized
// path and the direct fp16/bf16 path, one kernel template.
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
//     step, after the P.V MFMAs that still used the old max;
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
#include <atomic>
#include <cmath>
#include <type_traits>
#include <utility>

#include "sage_common.h"

namespace sage {
namespace {

constexpr int kBM = 256;
constexpr int kBN = 64;
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kXcds = 8;                   // MI355X: workgroups are dealt round-robin to 8 XCDs
constexpr float kRescale = 8.0f;           // lazy-rescale threshold of the running max (log2 units)
constexpr int kBufferWord3 = 0x00020000;   // gfx9 buffer descriptor word 3 (raw dword access)
// INT8 S accumulators start from the bit pattern of kBias = 1.5 * 2^23 instead
// of 0: for |acc| < 2^22 (D <= 128 int8 products stay below 2^21) the int32
// result kBiasBits + acc is the bit pattern of the float kBias + acc, so the
// softmax reads the scores as floats without an int->float conversion
constexpr int kBiasBits = 0x4B400000;
constexpr float kBias = 12582912.0f;
// tiles whose scales qs*ks stay below this take the conversion-free softmax
// (its exactness argument needs kBias * sc < 2^23, i.e. sc < 2/3)
constexpr float kFastScaleLimit = 0.49f;

// Q/K operand kinds
constexpr int kQkI8 = 0;    // INT8 Q/K (quantized path), per-block scales
constexpr int kQkF16 = 1;   // fp16 Q/K (direct path)
constexpr int kQkBf16 = 2;  // bf16 Q/K (direct path)
constexpr int kQkI8F = 3;   // INT8 Q/K, Q quantised by the kernel itself from fp16/bf16
constexpr bool is_i8(int qk) { return qk == kQkI8 || qk == kQkI8F; }

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

struct AttnParams {
  const void* q;         // [B,Hq,Sq,D] (INT8: contiguous int8; direct: strided fp16/bf16)
  const void* k;         // [B,Hkv,Sk,D] likewise
  const uint16_t* vt;    // fp16 [B,Hkv,D,np]
  void* out;
  float* lse;            // [B,Hq,Sq] or null
  const float* q_scale;  // [B,Hq,ceil(Sq/32)] (INT8 only)
  const float* k_scale;  // [B,Hkv,ceil(Sk/16)] (INT8 only)
  int64_t q_sb, q_sh, q_sn;  // Q/K strides in elements
  int64_t k_sb, k_sh, k_sn;
  int64_t o_sb, o_sh, o_sn;
  int64_t np;
  float sc;              // direct path: |fl(sm_scale * log2 e)|
  float qpre;            // fused Q quantisation: fl(fl(sm_scale) * log2 e)
  uint32_t q_xor;        // direct path: 0x80008000 negates Q (sm_scale < 0), else 0
  int32_t hq, hkv, sq, sk;
  int32_t group;         // Hq / Hkv
  int32_t nqb;           // query blocks per head
  int32_t q_groups, k_groups;
  int32_t work;          // work items: nfull + (B * Hq * nqb - nfull) * nsplit
  int32_t nfull;         // q-blocks [0, nfull) run whole (all of them unless the launch splits)
  int32_t nsplit;        // key-range splits of each later q-block (non-causal only)
  float* part;           // split items: [items][kBM][D] fp32 partial outputs, each normalised by its own row sum
  float* part_lse;       // split items: [items][kBM] natural-log LSE of each partial row
};

template <int D, int QK>
struct Cfg {
  static constexpr int kElem = is_i8(QK) ? 1 : 2;            // bytes per K element in LDS
  static constexpr int kStages = 3;                          // LDS ring depth (K and V)
  static constexpr int kKRow = D * kElem;                    // bytes per K row in LDS (unpadded)
  static constexpr int kVRow = kBN * 2;                      // bytes per V_T row in LDS (unpadded)
  static constexpr int kKStage = kBN * kKRow;                // bytes of one K stage
  static constexpr int kVStage = D * kVRow;                  // bytes of one V stage
  static constexpr int kKBase = kStages * kVStage;           // K stages follow the V stages
  static constexpr int kSmem = kStages * (kKStage + kVStage);
  static constexpr int kKLoads = kKStage / 1024;             // 1 KB LDS-direct loads per K tile
  static constexpr int kVLoads = kVStage / 1024;             // ... per V tile
  static constexpr int kKPerWave = kKLoads >= kWaves ? kKLoads / kWaves : 1;  // waves < kKLoads only if fewer
  static constexpr int kVPerWave = kVLoads / kWaves;
  // loads every wave issues per step (when a K tile has fewer 1 KB pieces than
  // there are waves, waves 0..kKLoads-1 issue one more); waiting until at most
  // this many are in flight retires everything issued a step earlier
  static constexpr int kStepLoads = kVPerWave + (kKLoads >= kWaves ? kKPerWave : 0);
  static constexpr int kDS = kKRow / 32;                     // k-steps of the QK MFMA (32 bytes of a row each)
  static constexpr int kDB = D / 32;                         // 32-row d blocks of O^T
  using SAcc = std::conditional_t<is_i8(QK), int16_t_, float16_t_>;  // S^T accumulator block
  static_assert(kVLoads % kWaves == 0, "V tile must split evenly over the waves");
  static_assert(kKLoads < kWaves || kKLoads % kWaves == 0, "K tile must split evenly over the waves");
};

// LDS tiles are unpadded rows of 16-byte chunks; chunk c of row r is stored at
// chunk position c ^ swz(r).  gfx950's LDS serves 256 bytes (64 banks) per
// cycle, i.e. 16 lanes of a ds_read_b128; the 16 lanes of an MFMA operand read
// take one chunk each from 16 consecutive rows.  Rows r and r + 256/ROW_BYTES
// share banks, so the XOR key is the row's index among those: every 16-lane
// group then covers all 64 banks once.  The XOR is its own inverse, so the
// same function maps position -> chunk for the loads.
template <int ROW_BYTES>
__device__ __forceinline__ int swz(int row) {
  static_assert(ROW_BYTES == 256 || ROW_BYTES == 128 || ROW_BYTES == 64, "rows of 4, 8 or 16 chunks");
  constexpr int kRowsPerWindow = 256 / ROW_BYTES;
  constexpr int kChunks = ROW_BYTES / 16;
  return (row / kRowsPerWindow) & (kChunks - 1);
}

// LDS row r of a K stage holds key kperm(r) of the tile (bits 2 and 3 swapped;
// an involution).
__device__ __forceinline__ int kperm(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max(x[lane], x[lane ^ 32]) / sum via v_permlane32_swap
__device__ __forceinline__ float xhalf_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Uniform 64-bit pointer (the compiler cannot always prove it).
template <typename T>
__device__ __forceinline__ const T* uniform_ptr(const T* ptr) {
  const uint64_t v = reinterpret_cast<uint64_t>(ptr);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Buffer descriptor over [base, base + bytes); reads past the end return 0.
// Both fields are made explicitly wave-uniform: a descriptor in VGPRs would
// turn every load into a waterfall loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(uniform_ptr(base)), static_cast<short>(0),
                                           static_cast<int>(__builtin_amdgcn_readfirstlane(bytes)), kBufferWord3);
}

// One 16-byte-per-lane buffer load straight into LDS (buffer_load_dwordx4
// ... lds): the wave's 64 lanes fill 1 KB at `lds_dst` + lane*16 from byte
// voffset + soffset of the buffer; lanes past the descriptor's end write
// zeros.  The builtin takes an LDS-address-space pointer, which only the
// device pass of this single-source file can form; in the host pass (which
// compiles no device code but would otherwise drop the kernels' launch stubs)
// the body is empty.
__device__ __forceinline__ void lds_direct_load16(__amdgpu_buffer_rsrc_t rsrc, char* lds_dst, uint32_t voffset,
                                                  uint32_t soffset) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef __attribute__((address_space(3))) void* lds_ptr;
  // the low 32 bits of a generic LDS address are the LDS offset
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, reinterpret_cast<lds_ptr>(reinterpret_cast<uintptr_t>(lds_dst)), 16,
                                           voffset, soffset, 0, 0);
#endif
}

// Tile loads straight from global memory into LDS.  Each wave instruction
// fills 1 KB of LDS at M0 + lane*16, so a lane's source offset picks the
// chunk that belongs at its LDS position (inverse swizzle; K rows also go
// through kperm).  One descriptor per head and tensor, the tile's position in
// the scalar offset: K ends just after the block's last key row (kv_end), so
// tiles and rows past it read as zero without touching memory; V_T ends at its
// padded row end (tiles past kv_end are loaded but never used).
template <int D, int QK>
struct TileLoader {
  using C = Cfg<D, QK>;
  uint32_t k_goff[C::kKPerWave];   // this lane's byte offsets in the K tile (row pitch k_pitch)
  uint32_t v_goff[C::kVPerWave];   // ... in the V_T tile (row pitch np)
  bool k_wave;                     // this wave loads K pieces
  int k_pitch;                     // bytes between K rows in global memory

  __device__ __forceinline__ TileLoader(int wave, int lane, int np, int k_pitch_) : k_pitch(k_pitch_) {
    k_wave = C::kKLoads >= kWaves || wave < C::kKLoads;
#pragma unroll
    for (int i = 0; i < C::kKPerWave; ++i) {
      const int byte = (wave * C::kKPerWave + i) * 1024 + lane * 16;  // LDS byte in the K stage
      const int row = byte / C::kKRow;
      const int c = ((byte % C::kKRow) / 16) ^ swz<C::kKRow>(row);
      k_goff[i] = static_cast<uint32_t>(kperm(row) * k_pitch + c * 16);
    }
#pragma unroll
    for (int i = 0; i < C::kVPerWave; ++i) {
      const int byte = (wave * C::kVPerWave + i) * 1024 + lane * 16;
      const int row = byte / C::kVRow;
      const int c = ((byte % C::kVRow) / 16) ^ swz<C::kVRow>(row);
      v_goff[i] = static_cast<uint32_t>(row * np * 2 + c * 16);
    }
  }

  // K rows kt.. through the head's K descriptor rk into the K stage at kstage.
  __device__ __forceinline__ void issue_k(__amdgpu_buffer_rsrc_t rk, char* kstage, int kt, int wave) const {
    if (k_wave) {
#pragma unroll
      for (int i = 0; i < C::kKPerWave; ++i)
        lds_direct_load16(rk, kstage + (wave * C::kKPerWave + i) * 1024, k_goff[i],
                          static_cast<uint32_t>(kt * k_pitch));
    }
  }
  // V_T tokens kt.. through the head's V_T descriptor rv into the V stage at vstage.
  __device__ __forceinline__ void issue_v(__amdgpu_buffer_rsrc_t rv, char* vstage, int kt, int wave) const {
#pragma unroll
    for (int i = 0; i < C::kVPerWave; ++i)
      lds_direct_load16(rv, vstage + (wave * C::kVPerWave + i) * 1024, v_goff[i], static_cast<uint32_t>(kt * 2));
  }
};

// Wait until at most N LDS-direct loads of this wave are in flight, then a
// workgroup barrier.  One asm statement: the compiler neither moves LDS
// accesses across it nor adds its own vmcnt(0) (which __syncthreads would).
template <int N>
__device__ __forceinline__ void wait_loads_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// The same, after the wave's LDS stores (and scalar loads) completed too, so
// that what the waves wrote to LDS before it is visible to all after it.
template <int N>
__device__ __forceinline__ void wait_loads_lds_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// The tile's 4 key-group scales (INT8 path), read through the constant address
// space so they land in SGPRs (the address is wave-uniform and nothing writes
// the scales during the kernel); groups past the end repeat the last one and
// only meet masked keys.  The direct path's scale is one constant.
typedef const __attribute__((address_space(4))) float* const_f32_ptr;
template <int QK>
__device__ __forceinline__ void load_ks(const AttnParams& p, const float* ksp, int kt, float (&ks)[4]) {
  if constexpr (is_i8(QK)) {
    const_f32_ptr kc = (const_f32_ptr)(reinterpret_cast<uint64_t>(uniform_ptr(ksp)));
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int gi = kt / 16 + g;
      ks[g] = kc[gi < p.k_groups ? gi : p.k_groups - 1];
    }
  } else {
#pragma unroll
    for (int g = 0; g < 4; ++g) ks[g] = 1.0f;
  }
}

// Per-lane LDS byte offsets of the MFMA operand reads: lane (m, hh) reads
// 16-byte chunk 2x+hh (x = k-step) of row m; blocks of 32 more rows keep the
// same swizzle (32 is a multiple of the swizzle period).  The K offsets carry
// the K ring's base, so that stage and block offsets (< 64 KB) fold into the
// ds_read immediate.
template <int D, int QK>
struct OperandMap {
  using C = Cfg<D, QK>;
  uint32_t k_off[C::kDS];
  uint32_t v_off[4];
  __device__ __forceinline__ OperandMap(int m, int hh) {
#pragma unroll
    for (int x = 0; x < C::kDS; ++x)
      k_off[x] = C::kKBase + m * C::kKRow + (((2 * x + hh) ^ swz<C::kKRow>(m)) * 16);
#pragma unroll
    for (int x = 0; x < 4; ++x) v_off[x] = m * C::kVRow + (((2 * x + hh) ^ swz<C::kVRow>(m)) * 16);
  }
};

// One QK MFMA: S^T block += K rows (a) . Q^T fragment (b), 32 bytes of each row.
// The first k-step accumulates onto `init` (INT8: the kBias bit pattern).
template <int QK>
__device__ __forceinline__ typename Cfg<64, QK>::SAcc qk_mfma(int4_t a, int4_t b, const typename Cfg<64, QK>::SAcc& c,
                                                              bool first, const typename Cfg<64, QK>::SAcc& init) {
  if constexpr (is_i8(QK)) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, first ? init : c, 0, 0, 0);
  } else if constexpr (QK == kQkF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b),
                                                  first ? float16_t_{} : c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   first ? float16_t_{} : c, 0, 0, 0);
  }
}

// Softmax of one tile for one wave, cut into pieces that the pipelined step
// spreads between its MFMAs: S (accumulators, read only) -> P (fp16
// fragments), running max and sum.  O is not touched: when the reference max
// moves (need), alpha = exp2(m_old - m_new) is left for the caller to apply to
// O before the next P.V.  On masked tiles the dead keys (j >= Sk, causal
// j > i) are re-derived where they are used instead of being written into a
// copy of S (register budget).  The 32 probabilities go in 16 pairs i (16-key
// step t = i/4, registers 8(t%2) + 2(i%4) .. +1 of block t/2), each in three
// stages that the step places in consecutive chunks, so the exp latency of one
// pair hides behind the work of its neighbours:
//   pieces 0-3     max of key group g, scaled (group g = step g)
//   piece  4       row max, lazy reference max, alpha
//   pieces 5-20    A(i): y = acc*sc - m_run (dequant and max in one FMA)
//   pieces 21-36   B(i): e = exp2(y)
//   pieces 37-52   C(i): fp16 RNE pair into the P^T fragment, partial sums
//   piece  53      l = l*alpha + sums
// Scales: INT8 fl(q_scale * k_scale) per 16-key group with its 3 lowest
// mantissa bits cleared (sc'; relative change < 2^-21); direct fl(sm_scale *
// log2 e) for all keys.  x -> x*sc is monotonic for sc > 0, so the group max
// can be taken on the raw accumulators: as int32 for INT8 (biased by
// kBiasBits; dead keys count as INT32_MIN, which no biased dot product
// reaches), as fp32 for the direct path (dead keys -inf).
// INT8 scores: the accumulator holds F = kBias + acc as a float, and
//   y = acc*sc' - m = fma(F, sc', -(kBias*sc' + m))
// with one rounding.  kBias*sc' is exact (3*sc' fits 24 bits), and so is
// kBias*sc' + m for an integer reference max m while kBias*sc' < 2^23 and
// |m| <= kBias*sc' (else the constant rounds by at most |m|*2^-24): FAST uses
// this form, the other paths fma(float(F - kBias)...) with the same result.
// The reference max m is kept an integer for INT8 (so alpha is a power of 2).
template <int D, int QK, bool CAUSAL, bool MASK, bool FAST = false>
struct TileSoftmax {
  static constexpr int kPieces = 54;
  using SAcc = typename Cfg<D, QK>::SAcc;
  const AttnParams& p;
  const SAcc (&acc)[2];
  const float (&ks)[4];
  float qs;
  int kt, qrow, hh;
  float sc[4];
  float bsc[4];   // INT8: kBias * sc (exact)
  float cg[4];    // INT8 FAST: -(kBias * sc + m_run)
  float gv[4];
  float y[16][2];
  float e[16][2];
  float lsum[2];
  uint32_t w[4][4];

  __device__ __forceinline__ TileSoftmax(const AttnParams& p_, const SAcc (&acc_)[2], const float (&ks_)[4], float qs_,
                                         int kt_, int qrow_, int hh_)
      : p(p_), acc(acc_), ks(ks_), qs(qs_), kt(kt_), qrow(qrow_), hh(hh_) {
    lsum[0] = lsum[1] = 0.0f;
  }

  // register r of block nb holds key kt + 32 nb + 16 (r/8) + 8 hh + r%8
  __device__ __forceinline__ bool dead(int nb, int r) const {
    const int n = kt + nb * 32 + 16 * (r >> 3) + 8 * hh + (r & 7);
    return (n >= p.sk) || (CAUSAL && n > qrow);
  }

  template <int K>
  __device__ __forceinline__ void piece(float& m_run, float& l_run, float& alpha, bool& need, half8_t (&pf)[4]) {
    if constexpr (K < 4) {
      constexpr int g = K, nb = g >> 1;
      if constexpr (is_i8(QK)) {
        sc[g] = __uint_as_float(__float_as_uint(qs * ks[g]) & ~7u);
        bsc[g] = kBias * sc[g];
        int gm = INT32_MIN;
#pragma unroll
        for (int r = (g & 1) * 8; r < (g & 1) * 8 + 8; ++r) {
          int a = acc[nb][r];
          if constexpr (MASK) a = dead(nb, r) ? INT32_MIN : a;
          gm = max(gm, a);
        }
        gv[g] = __builtin_fmaf(__int_as_float(gm), sc[g], -bsc[g]);
        if constexpr (MASK) gv[g] = (gm == INT32_MIN) ? -INFINITY : gv[g];
      } else {
        sc[g] = p.sc;
        float gm = -INFINITY;
#pragma unroll
        for (int r = (g & 1) * 8; r < (g & 1) * 8 + 8; ++r) {
          float a = acc[nb][r];
          if constexpr (MASK) a = dead(nb, r) ? -INFINITY : a;
          gm = __builtin_fmaxf(gm, a);
        }
        gv[g] = gm * sc[g];
        // a group without a live key stays -inf (also for a zero scale)
        if constexpr (MASK) gv[g] = (gm == -INFINITY) ? -INFINITY : gv[g];
      }
    } else if constexpr (K == 4) {
      // lazy reference max: it moves only when some row's max grew by more
      // than kRescale (log2 units), so p = exp2(s - m_run) stays below
      // 2^kRescale (no fp16 overflow).  A row with no live key yet keeps -inf
      // unless the wave moves, and then takes 0 (alpha = 0; its O and l are 0).
      const float mx = xhalf_max(__builtin_fmaxf(__builtin_fmaxf(gv[0], gv[1]), __builtin_fmaxf(gv[2], gv[3])));
      need = __builtin_amdgcn_ballot_w64(mx > m_run + kRescale) != 0;
      float m_new = __builtin_fmaxf(m_run, mx);
      if constexpr (is_i8(QK)) m_new = __builtin_ceilf(m_new);
      m_new = (m_new == -INFINITY) ? 0.0f : m_new;
      m_new = need ? m_new : m_run;
      alpha = need ? fast_exp2(m_run - m_new) : 1.0f;
      m_run = m_new;
      if constexpr (is_i8(QK) && FAST) {
#pragma unroll
        for (int g = 0; g < 4; ++g) cg[g] = -(bsc[g] + m_run);
      }
    } else if constexpr (K < 21) {
      constexpr int i = K - 5, t = i >> 2, nb = t >> 1, r0 = (t & 1) * 8 + 2 * (i & 3);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if constexpr (is_i8(QK) && FAST) {
          y[i][u] = __builtin_fmaf(__int_as_float(acc[nb][r0 + u]), sc[t], cg[t]);
        } else if constexpr (is_i8(QK)) {
          // F - kBias is exact (same binade)
          y[i][u] = __builtin_fmaf(__int_as_float(acc[nb][r0 + u]) - kBias, sc[t], -m_run);
        } else {
          y[i][u] = __builtin_fmaf(acc[nb][r0 + u], sc[t], -m_run);
        }
      }
    } else if constexpr (K < 37) {
      constexpr int i = K - 21, t = i >> 2, nb = t >> 1, r0 = (t & 1) * 8 + 2 * (i & 3);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        e[i][u] = fast_exp2(y[i][u]);
        if constexpr (MASK) e[i][u] = dead(nb, r0 + u) ? 0.0f : e[i][u];
      }
    } else if constexpr (K < 53) {
      constexpr int i = K - 37, t = i >> 2, j = i & 3;
      lsum[0] += e[i][0];
      lsum[1] += e[i][1];
      w[t][j] = pack_f16x2(e[i][0], e[i][1]);
      if constexpr (j == 3) pf[t] = __builtin_bit_cast(half8_t, make_uint4(w[t][0], w[t][1], w[t][2], w[t][3]));
    } else if constexpr (K == 53) {
      l_run = __builtin_fmaf(l_run, alpha, lsum[0] + lsum[1]);
    }
  }
};

// The MFMAs of one pipelined step in issue order: the P.V MFMAs of the
// previous tile (16-key step t major, the d blocks' accumulation chains
// alternate; lane half h supplies keys 16t + 8h .. 16t + 8h + 7), then the
// QK MFMAs of the next tile, key block 0 before key block 1.  MFMA i reads its
// A operand (16 bytes per lane) from LDS kAhead MFMAs earlier.
template <int D, int QK>
struct StepMfma {
  using C = Cfg<D, QK>;
  static constexpr int kPV = 4 * C::kDB;
  static constexpr int kQK = 2 * C::kDS;
  static constexpr int kN = kPV + kQK;
  static constexpr int kAhead = 2;
  const char* vst;
  const char* kst;
  const OperandMap<D, QK>& om;
  const typename C::SAcc& init;
  int4_t ring[kAhead + 1];

  __device__ __forceinline__ StepMfma(const char* vst_, const char* kst_, const OperandMap<D, QK>& om_,
                                      const typename C::SAcc& init_)
      : vst(vst_), kst(kst_), om(om_), init(init_) {}

  // the operand reads of the first kAhead MFMAs
  template <int... I>
  __device__ __forceinline__ void read_ahead(std::integer_sequence<int, I...>) {
    (read<I>(), ...);
  }
  template <int I>
  __device__ __forceinline__ void read() {
    if constexpr (I < kPV) {
      constexpr int t = I / C::kDB, db = I % C::kDB;
      ring[I % (kAhead + 1)] = *reinterpret_cast<const int4_t*>(vst + db * 32 * C::kVRow + om.v_off[t]);
    } else if constexpr (I < kN) {
      constexpr int q = I - kPV, nb = q / C::kDS, ds = q % C::kDS;
      ring[I % (kAhead + 1)] = *reinterpret_cast<const int4_t*>(kst + nb * 32 * C::kKRow + om.k_off[ds]);
    }
  }
  template <int I>
  __device__ __forceinline__ void mfma(const half8_t (&pf)[4], float16_t_ (&o)[C::kDB], const int4_t (&qf)[C::kDS],
                                       typename C::SAcc (&acc)[2]) {
    if constexpr (I < kPV) {
      constexpr int t = I / C::kDB, db = I % C::kDB;
      o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, ring[I % (kAhead + 1)]), pf[t], o[db],
                                                     0, 0, 0);
    } else {
      constexpr int q = I - kPV, nb = q / C::kDS, ds = q % C::kDS;
      acc[nb] = qk_mfma<QK>(ring[I % (kAhead + 1)], qf[ds], acc[nb], ds == 0, init);
    }
  }
};

// Softmax pieces of chunk c of a step (k-th of at most kMaxPieces; -1 =
// none).  S and P are updated in place, so the order must respect: P^T
// fragment t is rewritten (stage C of pairs 4t..4t+3) only after the P.V MFMAs
// that read it, and key block nb of S is read (group maxima, stage A) for the
// last time before the first QK MFMA that overwrites it.  Stage A of pair i
// needs the reference max of piece 4 (one chunk of slack for its ballot).
// The QK MFMAs of key block 1 start at chunk 20 or later in every kind
// (INT8 D=128: 16 P.V + 4 + 4; fp16/bf16 D=128: 16 + 8 + 8).
constexpr int kMaxPieces = 6;
template <int D>
constexpr int chunk_piece(int c, int k) {
  int list[kMaxPieces] = {-1, -1, -1, -1, -1, -1};
  int n = 0;
  if constexpr (D == 128) {
    // P.V step t at 4t..4t+3; pair i: A in chunk i+4, B in i+5, C in i+6
    if (c == 0) { list[n++] = 0; list[n++] = 1; }
    if (c == 1) { list[n++] = 2; list[n++] = 3; }
    if (c == 2) list[n++] = 4;
    if (c - 6 >= 0 && c - 6 < 16) list[n++] = 37 + c - 6;
    if (c - 5 >= 0 && c - 5 < 16) list[n++] = 21 + c - 5;
    if (c - 4 >= 0 && c - 4 < 16) list[n++] = 5 + c - 4;
    if (c == 22) list[n++] = 53;
  } else {
    // P.V step t at 2t, 2t+1; QK block 0 from chunk 8, block 1 from chunk 10
    // (INT8: 8 + 2 + 2) or 12 (fp16/bf16: 8 + 4 + 4); pairs 2q, 2q+1: A in
    // chunk q+2, B in q+3, C in q+4
    if (c == 0) { list[n++] = 0; list[n++] = 1; list[n++] = 2; list[n++] = 3; }
    if (c == 1) list[n++] = 4;
    for (int u = 0; u < 2; ++u) {
      if (c - 4 >= 0 && c - 4 < 8) list[n++] = 37 + 2 * (c - 4) + u;
      if (c - 3 >= 0 && c - 3 < 8) list[n++] = 21 + 2 * (c - 3) + u;
      if (c - 2 >= 0 && c - 2 < 8) list[n++] = 5 + 2 * (c - 2) + u;
    }
    if (c == 11) list[n++] = 53;
  }
  return k < n ? list[k] : -1;
}

template <typename SM, int... K>
__device__ __forceinline__ void run_all_pieces(SM& sm, std::integer_sequence<int, K...>, float& m_run, float& l_run,
                                               float& alpha, bool& need, half8_t (&pf)[4]) {
  (sm.template piece<K>(m_run, l_run, alpha, need, pf), ...);
}
template <typename SM, int K>
__device__ __forceinline__ void run_piece(SM& sm, float& m_run, float& l_run, float& alpha, bool& need,
                                          half8_t (&pf)[4]) {
  if constexpr (K >= 0) sm.template piece<K>(m_run, l_run, alpha, need, pf);
}

// One pipelined step: MFMA i, the operand read of MFMA i + kAhead and the
// softmax pieces of chunk i, one chunk per MFMA; sched_barrier keeps the
// chunks in this order, so the wave issues VALU work while each MFMA runs.
template <int D, int QK, typename SM, int I>
__device__ __forceinline__ void step_chunk(StepMfma<D, QK>& mf, SM& sm, const half8_t (&p_prv)[4],
                                           float16_t_ (&o)[Cfg<D, QK>::kDB], const int4_t (&qf)[Cfg<D, QK>::kDS],
                                           typename Cfg<D, QK>::SAcc (&s_nxt)[2], float& m_run, float& l_run,
                                           float& alpha, bool& need, half8_t (&p_cur)[4]) {
  mf.template read<I + StepMfma<D, QK>::kAhead>();
  mf.template mfma<I>(p_prv, o, qf, s_nxt);
  run_piece<SM, chunk_piece<D>(I, 0)>(sm, m_run, l_run, alpha, need, p_cur);
  run_piece<SM, chunk_piece<D>(I, 1)>(sm, m_run, l_run, alpha, need, p_cur);
  run_piece<SM, chunk_piece<D>(I, 2)>(sm, m_run, l_run, alpha, need, p_cur);
  run_piece<SM, chunk_piece<D>(I, 3)>(sm, m_run, l_run, alpha, need, p_cur);
  run_piece<SM, chunk_piece<D>(I, 4)>(sm, m_run, l_run, alpha, need, p_cur);
  run_piece<SM, chunk_piece<D>(I, 5)>(sm, m_run, l_run, alpha, need, p_cur);
  __builtin_amdgcn_sched_barrier(0);
}
template <int D, int QK, typename SM, int... I>
__device__ __forceinline__ void step_chunks(std::integer_sequence<int, I...>, StepMfma<D, QK>& mf, SM& sm,
                                            const half8_t (&p_prv)[4], float16_t_ (&o)[Cfg<D, QK>::kDB],
                                            const int4_t (&qf)[Cfg<D, QK>::kDS],
                                            typename Cfg<D, QK>::SAcc (&s_nxt)[2], float& m_run, float& l_run,
                                            float& alpha, bool& need, half8_t (&p_cur)[4]) {
  (step_chunk<D, QK, SM, I>(mf, sm, p_prv, o, qf, s_nxt, m_run, l_run, alpha, need, p_cur), ...);
}

// S^T of one 64-key tile for the wave's 32 queries (prologue and masked steps).
template <int D, int QK>
__device__ __forceinline__ void qk_tile(const char* kstage, const OperandMap<D, QK>& om,
                                        const int4_t (&qf)[Cfg<D, QK>::kDS], typename Cfg<D, QK>::SAcc (&acc)[2],
                                        const typename Cfg<D, QK>::SAcc& init) {
  using C = Cfg<D, QK>;
#pragma unroll
  for (int ds = 0; ds < C::kDS; ++ds) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int4_t a = *reinterpret_cast<const int4_t*>(kstage + nb * 32 * C::kKRow + om.k_off[ds]);
      acc[nb] = qk_mfma<QK>(a, qf[ds], acc[nb], ds == 0, init);
    }
  }
}

// O^T += V^T . P^T for one 64-key tile (the last tile and masked steps).
template <int D, int QK>
__device__ __forceinline__ void pv_tile(const char* vstage, const OperandMap<D, QK>& om, const half8_t (&pf)[4],
                                        float16_t_ (&o)[Cfg<D, QK>::kDB]) {
  using C = Cfg<D, QK>;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int db = 0; db < C::kDB; ++db) {
      const half8_t a = *reinterpret_cast<const half8_t*>(vstage + db * 32 * C::kVRow + om.v_off[t]);
      o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[t], o[db], 0, 0, 0);
    }
  }
}

// Largest value over the 64 lanes, without LDS: DPP butterflies inside each
// 16-lane row, then the row and half-wave swaps.
__device__ __forceinline__ float wave_max64(float v) {
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false)));
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false)));
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false)));
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false)));
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  return xhalf_max(v);
}

// Fused Q quantisation, part 1: lane (m, hh) loads the 16 fp16/bf16 elements
// 32x + 16hh .. of row wrow0 + m for k-step x, exactly the bytes its Q^T
// fragment will hold; rows past Sq load as zero (they neither raise the absmax
// nor reach the output).  Issued first, consumed after the K/V ring loads.
template <int D>
__device__ __forceinline__ void load_q_raw(const AttnParams& p, int b, int hq, int qrow, int hh,
                                           uint32_t (&w)[D / 32][8]) {
  const uint16_t* qp = static_cast<const uint16_t*>(p.q) + static_cast<int64_t>(b) * p.q_sb +
                       static_cast<int64_t>(hq) * p.q_sh + static_cast<int64_t>(qrow) * p.q_sn + hh * 16;
#pragma unroll
  for (int ds = 0; ds < D / 32; ++ds) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (qrow < p.sq) v = *reinterpret_cast<const uint4*>(qp + ds * 32 + h * 8);
      w[ds][4 * h + 0] = v.x;
      w[ds][4 * h + 1] = v.y;
      w[ds][4 * h + 2] = v.z;
      w[ds][4 * h + 3] = v.w;
    }
  }
}

// Fused Q quantisation, part 2: the wave's 32 query rows are exactly one Q
// scale group (32 tokens), quantised with the arithmetic of quant_qk_i8_kernel
// (csrc/attn_gfx11.cu:179-321 of the reference), so q8 and the returned scale
// equal the quantisation kernel's bit for bit.
template <int D, bool BF16>
__device__ __forceinline__ float quant_q_raw(const AttnParams& p, int wrow0, const uint32_t (&w)[D / 32][8],
                                             int4_t (&qf)[D / 32]) {
#pragma clang fp contract(off)
  constexpr int kDS = D / 32;
  const float pre = p.qpre;
  // max |fl(x * pre)| = fl(max |x| * |pre|): rounding is monotonic and
  // symmetric in sign, so the scaled absmax needs one multiply per group;
  // fmax ignores NaN elements as the quantisation kernel does
  float xmax = 0.0f;
#pragma unroll
  for (int ds = 0; ds < kDS; ++ds) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float2_t f = unpack2<BF16>(w[ds][k]);
      xmax = __builtin_fmaxf(xmax, __builtin_fmaxf(__builtin_fabsf(f.x), __builtin_fabsf(f.y)));
    }
  }
  xmax = wave_max64(xmax);
  const float amax = __builtin_fmaxf(kAmaxFloor, xmax * __builtin_fabsf(pre));
  const float scale = amax / 127.0f;
  const float inv = 127.0f / amax;
  const float iscale = inv * pre;
#pragma unroll
  for (int ds = 0; ds < kDS; ++ds) {
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float2_t f0 = unpack2<BF16>(w[ds][2 * k]);
      const float2_t f1 = unpack2<BF16>(w[ds][2 * k + 1]);
      o[k] = pack_i8x4(round_half_away_i8(f0.x * iscale), round_half_away_i8(f0.y * iscale),
                       round_half_away_i8(f1.x * iscale), round_half_away_i8(f1.y * iscale));
    }
    qf[ds] = int4_t{static_cast<int>(o[0]), static_cast<int>(o[1]), static_cast<int>(o[2]), static_cast<int>(o[3])};
  }
  return wrow0 < p.sq ? scale : 0.0f;
}

// One work item of a block: q-block id = bh * nqb + (nqb - 1 - qb) (heaviest
// causal blocks first); whole items run q-block w_idx, split items piece
// w_idx of the split range (q-block nfull + w_idx / nsplit, key range
// w_idx % nsplit).
template <int D, int QK, bool CAUSAL, bool OUT_BF16>
__device__ __forceinline__ void attn_item(const AttnParams& p, char* smem, float* ks_part, bool whole, int w_idx) {
  using C = Cfg<D, QK>;
  using SAcc = typename C::SAcc;
  const int nsplit = whole ? 1 : p.nsplit;
  const int split = whole ? 0 : w_idx % nsplit;
  const int wq = whole ? w_idx : p.nfull + w_idx / nsplit;
  const int bh = wq / p.nqb;
  const int qb = p.nqb - 1 - (wq - bh * p.nqb);
  const int b = bh / p.hq;
  const int hq = bh - b * p.hq;
  const int hk = hq / p.group;
  const int q0 = qb * kBM;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int m = lane & 31;
  const int hh = lane >> 5;
  const int wrow0 = q0 + wave * 32;
  const int qrow = wrow0 + m;

  // ---- Q^T fragments (lane (m, hh): bytes 32x + 16hh of row qrow for k-step
  // x) and the wave's q scale
  int4_t qf[C::kDS];
  float qs = 1.0f;
  uint32_t qraw[QK == kQkI8F ? C::kDS : 1][8];  // fused kind: Q as loaded, quantised in the prologue
  if constexpr (QK == kQkI8F) {
    load_q_raw<D>(p, b, hq, qrow, hh, qraw);
  } else {
    const char* qp = static_cast<const char*>(p.q) + hh * 16 +
                     (QK == kQkI8 ? (static_cast<int64_t>(bh) * p.sq + qrow) * D
                                  : (static_cast<int64_t>(b) * p.q_sb + static_cast<int64_t>(hq) * p.q_sh +
                                     static_cast<int64_t>(qrow) * p.q_sn) * C::kElem);
#pragma unroll
    for (int ds = 0; ds < C::kDS; ++ds) {
      if (qrow < p.sq) {
        qf[ds] = *reinterpret_cast<const int4_t*>(qp + ds * 32);
      } else {
        qf[ds] = int4_t{0, 0, 0, 0};
      }
      // a negative scale goes into Q's sign bits (exact), so the scale the
      // softmax sees is positive and max commutes with it
      if constexpr (!is_i8(QK)) qf[ds] ^= static_cast<int>(p.q_xor);
    }
    if constexpr (QK == kQkI8)
      qs = (wrow0 < p.sq) ? p.q_scale[static_cast<int64_t>(bh) * p.q_groups + wrow0 / 32] : 0.0f;
  }

  const int64_t bhk = static_cast<int64_t>(b) * p.hkv + hk;
  const char* kbase = static_cast<const char*>(p.k) + (is_i8(QK) ? bhk * p.sk * D
                                                                    : (static_cast<int64_t>(b) * p.k_sb + hk * p.k_sh) * C::kElem);
  const uint16_t* vbase = p.vt + bhk * D * p.np;
  const float* ksp = is_i8(QK) ? p.k_scale + bhk * p.k_groups : nullptr;
  // INT8 K is the contiguous quant output: its row pitch is a constant
  const int k_pitch = is_i8(QK) ? D : static_cast<int>(p.k_sn) * C::kElem;

  // key tiles of this item: [t0, t0 + ntiles) (non-causal splits take an
  // even share of the head's tiles; causal blocks end at their last row)
  const int head_tiles = (p.sk + kBN - 1) / kBN;
  const int t0 = CAUSAL ? 0 : split * head_tiles / nsplit;
  const int t1 = CAUSAL ? 0 : (split + 1) * head_tiles / nsplit;
  const int kv0 = t0 * kBN;
  const int kv_end = CAUSAL ? min(q0 + kBM, p.sk) : min(t1 * kBN, p.sk);
  const int ntiles = CAUSAL ? (kv_end + kBN - 1) / kBN : t1 - t0;
  // tiles [0, n_main) of the item need no mask for any wave of the block
  // (inside the key range and, causal, left of the block's first row)
  const int n_main = CAUSAL ? min(min(q0, p.sk) / kBN, ntiles) : (t1 * kBN <= p.sk ? ntiles : ntiles - 1);

  float16_t_ o[C::kDB];
#pragma unroll
  for (int db = 0; db < C::kDB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
  }
  float m_run = -INFINITY;
  float l_run = 0.0f;
  float alpha = 1.0f;
  bool need = false;
  SAcc s[2];         // S of the tile the next softmax reads
  half8_t pf[4];     // P^T fragments of the tile the next P.V reads
#pragma unroll
  for (int t = 0; t < 4; ++t) pf[t] = half8_t{};
  float ks[4];
  // accumulator the first QK k-step starts from (INT8: the kBias bit pattern;
  // made opaque so that its 16 registers are built once and kept, instead of
  // being rebuilt from scalars before every first k-step)
  SAcc sinit;
  if constexpr (is_i8(QK)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) sinit[r] = kBiasBits;
    asm volatile("" : "+v"(sinit));
  } else {
    sinit = SAcc{};
  }
  // INT8: the unmasked loop uses the conversion-free softmax when every k
  // scale of the block's unmasked tiles is below kFastScaleLimit / qs; the
  // largest one is found by the block's waves together (each scans an eighth
  // of the groups, the partial maxima meet in LDS at the prologue barrier).
  // Otherwise (extreme inputs only) every tile runs in the sequential loop.
  const TileLoader<D, QK> tl(wave, lane, static_cast<int>(p.np), k_pitch);
  // K: rows [0, kv_end) of the head; V_T: the head's padded rows
  const auto rk = make_rsrc(kbase, kv_end > 0 ? static_cast<uint32_t>((kv_end - 1) * k_pitch + D * C::kElem) : 0u);
  const auto rv = make_rsrc(vbase, static_cast<uint32_t>(D * static_cast<int>(p.np) * 2));
  const OperandMap<D, QK> om(m, hh);
  char* const vring = smem;                // V stages, then K stages
  char* const kring = smem + C::kKBase;    // K stage base for the loads
  const char* const kread = smem;          // ... for operand reads (offsets carry kKBase)

  auto rescale_o = [&]() __attribute__((always_inline)) {
    if (need) {
      // keeps the block a real branch: without it the multiplies of O are
      // speculated onto every step
      asm volatile("" ::: "memory");
#pragma unroll
      for (int db = 0; db < C::kDB; ++db) {
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      }
    }
  };

  if (ntiles > 0) {
    // ---- prologue: K_0, K_1 and a zero V_{-1} (read by step 0's P.V with
    // P = 0), then K_2 and V_0 (what every step issues: K_{j+3}, V_{j+1})
    tl.issue_k(rk, kring + 0 * C::kKStage, kv0, wave);
    tl.issue_k(rk, kring + 1 * C::kKStage, kv0 + kBN, wave);
    tl.issue_v(make_rsrc(vbase, 0u), vring + 2 * C::kVStage, 0, wave);
    // the first 128 k scales of this wave's share of the scan (up to 16384
    // keys a block), loaded before the fused quantisation so that their latency
    // overlaps it
    const int g0 = t0 * (kBN / SAGE_K_GROUP), ng = n_main * (kBN / SAGE_K_GROUP);
    const int lo = g0 + wave * ng / kWaves, hi = g0 + (wave + 1) * ng / kWaves;
    float ks_a = 0.0f, ks_b = 0.0f;
    if constexpr (is_i8(QK)) {
      if (lo + lane < hi) ks_a = ksp[lo + lane];
      if (lo + lane + 64 < hi) ks_b = ksp[lo + lane + 64];
    }
    // K_2 and V_0 are the wave's last kStepLoads loads before the prologue
    // barrier, which leaves them in flight (V_0 is waited for at step 1), so
    // they are issued as early as the ring allows
    tl.issue_k(rk, kring + 2 * C::kKStage, kv0 + 2 * kBN, wave);
    tl.issue_v(rv, vring + 0 * C::kVStage, kv0, wave);
    // fused kind: quantise Q while the tiles and the k scales are in flight
    if constexpr (QK == kQkI8F) qs = quant_q_raw<D, OUT_BF16>(p, wrow0, qraw, qf);
    if constexpr (is_i8(QK)) {
      float mx = __builtin_fmaxf(ks_a, ks_b);
      for (int g = lo + lane + 128; g < hi; g += 64) mx = __builtin_fmaxf(mx, ksp[g]);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, off));
      if (lane == 0) ks_part[wave] = mx;
    }
    // K_0, K_1, V_{-1} landed (everything but K_2 and V_0); ks_part published
    wait_loads_lds_barrier<C::kStepLoads>();
    bool fast_block = true;
    if constexpr (is_i8(QK)) {
      float kmax = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) kmax = __builtin_fmaxf(kmax, ks_part[w]);
      fast_block = qs * kmax < kFastScaleLimit;
    }
    load_ks<QK>(p, ksp, kv0, ks);
    qk_tile<D, QK>(kread, om, qf, s, sinit);

    // Step j (stage index st = j % 3): wait for K_{j+1} and V_{j-1} (issued at
    // step j-2), apply the pending O rescale, issue K_{j+3} into stage j%3 and
    // V_{j+1} into stage (j+1)%3 (their previous tiles were last read in step
    // j-1, which every wave has left at the barrier), then P_{j-1}.V_{j-1},
    // the softmax of S_j and S_{j+1}, interleaved; S and P are rewritten in
    // place (see chunk_piece).
    // ST (0..2) is the compile-time stage of the unrolled unmasked loop, so
    // every LDS operand address is a lane offset plus an immediate; ST = -1
    // (masked loop) takes the stage at run time.
    // causal: a tile whose first key lies past the wave's last row is masked
    // for all of the wave's rows; its softmax would leave m, l and O as they
    // are (P = 0), so the wave skips the tile's QK, softmax and P.V while the
    // loads and barriers stay with the block.  Such tiles are the block's last
    // (the condition grows with the tile), so a skipped softmax is followed only
    // by skipped P.Vs and never feeds its stale P fragments to an MFMA.
    auto dead_tile = [&](int t) __attribute__((always_inline)) { return CAUSAL && kv0 + t * kBN > wrow0 + 31; };
    auto step = [&](int j, int st_rt, auto mask_tag, auto st_tag) __attribute__((always_inline)) {
      constexpr bool MASKED = decltype(mask_tag)::value;
      constexpr int ST = decltype(st_tag)::value;
      const int st = ST >= 0 ? ST : st_rt;
      const int st1 = st == 2 ? 0 : st + 1;
      const int st2 = st == 0 ? 2 : st - 1;
      wait_loads_barrier<C::kStepLoads>();
      rescale_o();
      tl.issue_k(rk, kring + st * C::kKStage, kv0 + (j + 3) * kBN, wave);
      tl.issue_v(rv, vring + st1 * C::kVStage, kv0 + (j + 1) * kBN, wave);
      // tail / diagonal tiles (a few per block), and INT8 tiles after one with
      // scales too large for the conversion-free softmax: the same work in
      // plain order, P.V (reads P) -> softmax (reads S, writes P) -> QK (writes S)
      auto sequential = [&]() __attribute__((always_inline)) {
        if (!dead_tile(j - 1)) pv_tile<D, QK>(vring + st2 * C::kVStage, om, pf, o);
        auto softmax = [&](auto smask_tag) __attribute__((always_inline)) {
          using SM = TileSoftmax<D, QK, CAUSAL, decltype(smask_tag)::value>;
          SM sm(p, s, ks, qs, kv0 + j * kBN, qrow, hh);
          run_all_pieces(sm, std::make_integer_sequence<int, SM::kPieces>{}, m_run, l_run, alpha, need, pf);
        };
        // this wave's keys of tile j are all live: inside the key range and,
        // causal, left of the wave's first row
        if (dead_tile(j)) {
          need = false;  // no softmax: m, l and O stay as they are
        } else if (kv0 + j * kBN + kBN - 1 <= (CAUSAL ? min(wrow0, p.sk - 1) : p.sk - 1)) {
          softmax(std::false_type{});
        } else {
          softmax(std::true_type{});
        }
        if (!dead_tile(j + 1)) qk_tile<D, QK>(kread + st1 * C::kKStage, om, qf, s, sinit);
      };
      if constexpr (!MASKED) {
        using SM = TileSoftmax<D, QK, CAUSAL, false, true>;
        SM sm(p, s, ks, qs, kv0 + j * kBN, qrow, hh);
        StepMfma<D, QK> mf(vring + st2 * C::kVStage, kread + st1 * C::kKStage, om, sinit);
        mf.read_ahead(std::make_integer_sequence<int, StepMfma<D, QK>::kAhead>{});
        step_chunks<D, QK, SM>(std::make_integer_sequence<int, StepMfma<D, QK>::kN>{}, mf, sm, pf, o, qf, s, m_run,
                               l_run, alpha, need, pf);
      } else {
        sequential();
      }
      // P_j and the row statistics are consumed a step later; pinning them
      // here keeps their computation in this step (otherwise it sinks past
      // the next barrier and the step loses its VALU half)
      asm volatile("" ::"v"(pf[0]), "v"(pf[1]), "v"(pf[2]), "v"(pf[3]), "v"(l_run), "v"(alpha));
      // k scales of the next tile: issued here, after the step's last LDS
      // read, because a pending scalar load makes every later LDS wait a full
      // lgkmcnt(0) (scalar loads return out of order)
      load_ks<QK>(p, ksp, kv0 + (j + 1) * kBN, ks);
    };
    int j = 0, st = 0;
    if (fast_block) {
      for (; j + 3 <= n_main; j += 3) {
        step(j, 0, std::false_type{}, std::integral_constant<int, 0>{});
        step(j + 1, 1, std::false_type{}, std::integral_constant<int, 1>{});
        step(j + 2, 2, std::false_type{}, std::integral_constant<int, 2>{});
      }
    }
    for (; j < ntiles; ++j) {
      step(j, st, std::true_type{}, std::integral_constant<int, -1>{});
      st = st == 2 ? 0 : st + 1;
    }
    // last P.V: V_{ntiles-1} sits in stage (ntiles-1) % 3
    wait_loads_barrier<C::kStepLoads>();
    rescale_o();
    if (!dead_tile(ntiles - 1)) pv_tile<D, QK>(vring + (st == 0 ? 2 : st - 1) * C::kVStage, om, pf, o);
    // loads of tiles past the end may still be in flight into this block's LDS
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }

  // ---- epilogue: 1/l, cast, 8-byte stores (4 consecutive d per store); LSE =
  // ln(sum_j e^{s_j}) over the natural-log scores s_j = ln2 * (log2-domain
  // score) = ln2 * (m + log2 l), -inf for a row without a live key
  const float l_tot = xhalf_sum(l_run);
  if (!CAUSAL && nsplit > 1) {
    // partial result of a key split: O / l in fp32 and its LSE, merged by attn_merge_kernel
    if (qrow < p.sq) {
      const int64_t prow = static_cast<int64_t>(w_idx) * kBM + wave * 32 + m;
      if (hh == 0)
        p.part_lse[prow] = (l_tot > 0.0f) ? (m_run + __builtin_amdgcn_logf(l_tot)) * 0.6931471805599453f : -INFINITY;
      const float inv = (l_tot > 0.0f) ? 1.0f / l_tot : 0.0f;
      float* pp = p.part + prow * D;
#pragma unroll
      for (int db = 0; db < C::kDB; ++db) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int d = db * 32 + 8 * r4 + 4 * hh;
          *reinterpret_cast<float4*>(pp + d) = make_float4(o[db][4 * r4 + 0] * inv, o[db][4 * r4 + 1] * inv,
                                                           o[db][4 * r4 + 2] * inv, o[db][4 * r4 + 3] * inv);
        }
      }
    }
    return;
  }
  if (p.lse != nullptr && qrow < p.sq && hh == 0) {
    p.lse[static_cast<int64_t>(bh) * p.sq + qrow] =
        (l_tot > 0.0f) ? (m_run + __builtin_amdgcn_logf(l_tot)) * 0.6931471805599453f : -INFINITY;
  }
  // Output rows: lane (m, hh) holds 4 consecutive d of row m per (d block,
  // r4), so stores straight from registers put 16-byte pieces of 32 rows in
  // every instruction.  Instead the wave stages its 32 rows (cast, 2D bytes
  // each, rows padded by 16 bytes so that the 32 rows of one write start in
  // different banks) in its part of the LDS ring, which is free once every
  // wave's last P.V has read it, and writes whole rows: each store
  // instruction then covers 64 lanes x 16 bytes of 4 (D=128) or 8 (D=64)
  // consecutive rows.
  {
    constexpr int kRowB = D * 2;
    constexpr int kPitch = kRowB + 16;
    constexpr int kChunks = kRowB / 16;
    constexpr int kRowsPerStore = 64 / kChunks;
    static_assert(kWaves * 32 * kPitch <= C::kSmem, "output staging exceeds the LDS ring");
    const float inv = (l_tot > 0.0f) ? 1.0f / l_tot : 0.0f;
    char* const ost = smem + wave * (32 * kPitch);
    __syncthreads();  // every wave's last P.V has read the ring
    char* const wbase = ost + m * kPitch + 8 * hh;
#pragma unroll
    for (int db = 0; db < C::kDB; ++db) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const float v0 = o[db][4 * r4 + 0] * inv, v1 = o[db][4 * r4 + 1] * inv;
        const float v2 = o[db][4 * r4 + 2] * inv, v3 = o[db][4 * r4 + 3] * inv;
        uint2 w;
        if constexpr (OUT_BF16) {
          w = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
        } else {
          w = make_uint2(pack_f16x2(v0, v1), pack_f16x2(v2, v3));
        }
        // d = 32 db + 8 r4 + 4 hh: byte 64 db + 16 r4 + 8 hh of the row
        *reinterpret_cast<uint2*>(wbase + 64 * db + 16 * r4) = w;
      }
    }
    const int lr = lane / kChunks, lc = lane % kChunks;
    const char* const rbase = ost + lr * kPitch + lc * 16;
    uint16_t* const obase = static_cast<uint16_t*>(p.out) + static_cast<int64_t>(b) * p.o_sb +
                            static_cast<int64_t>(hq) * p.o_sh + static_cast<int64_t>(wrow0 + lr) * p.o_sn + lc * 8;
#pragma unroll
    for (int i = 0; i < 32 / kRowsPerStore; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(rbase + i * kRowsPerStore * kPitch);
      if (wrow0 + lr + i * kRowsPerStore < p.sq)
        *reinterpret_cast<uint4*>(obase + static_cast<int64_t>(i * kRowsPerStore) * p.o_sn) = v;
    }
  }
}

// Grid: one block per item when there are at most as many items as CUs;
// otherwise a persistent grid of one block per CU (a multiple of the XCD
// count, block L on XCD L % 8) walks a static schedule.  The hardware
// dispatcher refills a CU only in order, and with causal blocks of unequal
// length that left CUs idle for 11 us on average between blocks at
// B1 H32 S16384 (3 us between equal blocks); the static schedule has no such
// gaps.  Items are dealt in XCD-contiguous ranges (the q-blocks of a head and
// the splits of a q-block share an XCD's L2, and the blocks of one round
// stream the same K/V tiles); within a range the blocks of the XCD take
// consecutive items in rounds, in snake order for causal items (reversed in
// odd rounds).  A head's causal q-blocks come heaviest first, so a forward
// round and the reversed one after it give every block the same number of key
// tiles whenever a head's q-blocks fill a whole number of round pairs or two
// rounds cover whole heads (B1 H32 S16384: 64 q-blocks per head, 32 blocks
// per XCD).  Whole items precede split items.
// Item k of block L (false past its last).  One item per block (grid ==
// work): blocks [0, nfull) whole items, then the split items, each range
// XCD-contiguous (nfull is a multiple of the XCD count).  Persistent grid:
// range 0 (whole) then range 1 (split); block (xcd, slot) takes, in rounds r,
// index r * nb + slot of its XCD's share of the range (snake order for causal
// items: nb - 1 - slot in odd rounds).
template <bool CAUSAL>
__device__ __forceinline__ bool next_item(const AttnParams& p, int L, int k, bool& whole, int& w_idx) {
  if (static_cast<int>(gridDim.x) == p.work) {
    if (k > 0) return false;
    whole = L < p.nfull;
    const int base = whole ? 0 : p.nfull;
    const int cnt = whole ? p.nfull : p.work - p.nfull;
    const int xcd = (L - base) % kXcds;
    const int slot = (L - base) / kXcds;
    const int per = cnt / kXcds;
    const int rem = cnt % kXcds;
    w_idx = xcd * per + (xcd < rem ? xcd : rem) + slot;
    return true;
  }
  const int xcd = L % kXcds;
  const int slot = L / kXcds;
  const int nb = static_cast<int>(gridDim.x) / kXcds;  // blocks per XCD
#pragma unroll
  for (int range = 0; range < 2; ++range) {
    whole = range == 0;
    const int cnt = whole ? p.nfull : p.work - p.nfull;
    const int per = cnt / kXcds;
    const int rem = cnt % kXcds;
    const int first = xcd * per + (xcd < rem ? xcd : rem);
    const int n_x = per + (xcd < rem ? 1 : 0);
    // this block's items in the range: the full rounds plus maybe one
    const int rounds = n_x / nb;
    const int pos_last = (CAUSAL && (rounds & 1)) ? nb - 1 - slot : slot;
    const int mine = rounds + (pos_last < n_x - rounds * nb ? 1 : 0);
    if (k < mine) {
      w_idx = first + k * nb + ((CAUSAL && (k & 1)) ? nb - 1 - slot : slot);
      return true;
    }
    k -= mine;
  }
  return false;
}

// Grid: one block per item when there are at most as many items as CUs;
// otherwise a persistent grid of one block per CU (a multiple of the XCD
// count, block L on XCD L % 8) walks a static schedule.  The hardware
// dispatcher refills a CU only in order, and with causal blocks of unequal
// length that left CUs idle for 11 us on average between blocks at
// B1 H32 S16384 (3 us between equal blocks); the static schedule has no such
// gaps.  Items are dealt in XCD-contiguous ranges (the q-blocks of a head and
// the splits of a q-block share an XCD's L2); within a range the blocks of
// the XCD take items in rounds, causal items heaviest first (over the heads
// of the range) and in snake order, so every block's total of key tiles is
// the same whenever the range is whole heads and an even number of rounds.
// Whole items precede split items.
template <int D, int QK, bool CAUSAL, bool OUT_BF16>
__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(AttnParams p) {
  using C = Cfg<D, QK>;
  __shared__ __align__(16) char smem[C::kSmem];
  __shared__ float ks_part[kWaves];
  bool whole;
  int w_idx;
  for (int k = 0; next_item<CAUSAL>(p, blockIdx.x, k, whole, w_idx); ++k) {
    if (k > 0) __syncthreads();  // the item reuses the LDS ring and ks_part
    attn_item<D, QK, CAUSAL, OUT_BF16>(p, smem, ks_part, whole, w_idx);
  }
}

// ---- merge of key splits: per query row, the partial outputs o_s (each
// normalised by its own row sum) and their LSEs lse_s combine exactly as
//   M = max_s lse_s,  w_s = e^{lse_s - M},  o = sum_s w_s o_s / sum_s w_s,
//   lse = M + ln sum_s w_s
// (the softmax over the union of the key ranges).  D/4 lanes per row, one
// float4 of every partial each, so a row's reads are one contiguous run.
struct MergeParams {
  const float* part;
  const float* part_lse;
  void* out;
  float* lse;  // [B,Hq,Sq] or null
  int64_t o_sb, o_sh, o_sn;
  int64_t rows;  // (split q-blocks) * kBM
  int32_t hq, sq, nqb, nfull, nsplit;
};

template <int D, bool OUT_BF16>
__global__ __launch_bounds__(256) void attn_merge_kernel(MergeParams p) {
  constexpr int kLanesPerRow = D / 4;
  constexpr int kRowsPerBlock = 256 / kLanesPerRow;
  const int64_t gr = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / kLanesPerRow;
  if (gr >= p.rows) return;
  const int c = threadIdx.x % kLanesPerRow;
  // row r of split q-block id = nfull + gr / kBM (the attention kernel's ids)
  const int64_t sid = gr / kBM;
  const int r = static_cast<int>(gr - sid * kBM);
  const int64_t id = p.nfull + sid;
  const int64_t bh = id / p.nqb;
  const int qb = p.nqb - 1 - static_cast<int>(id - bh * p.nqb);
  const int qrow = qb * kBM + r;
  if (qrow >= p.sq) return;
  const int64_t item0 = sid * p.nsplit;  // its first split item
  const float* lp = p.part_lse + item0 * kBM + r;
  float mx = -INFINITY;
  for (int s = 0; s < p.nsplit; ++s) mx = fmaxf(mx, lp[s * kBM]);
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float wsum = 0.0f;
  if (mx > -INFINITY) {
    const float* op = p.part + (item0 * kBM + r) * D + 4 * c;
    for (int s = 0; s < p.nsplit; ++s) {
      const float w = expf(lp[s * kBM] - mx);  // 0 for a split without a live key
      const float4 v = *reinterpret_cast<const float4*>(op + static_cast<int64_t>(s) * kBM * D);
      wsum += w;
      acc.x += w * v.x;
      acc.y += w * v.y;
      acc.z += w * v.z;
      acc.w += w * v.w;
    }
  }
  const float inv = wsum > 0.0f ? 1.0f / wsum : 0.0f;
  const int64_t b = bh / p.hq;
  const int64_t hq = bh - b * p.hq;
  uint16_t* dst = static_cast<uint16_t*>(p.out) + b * p.o_sb + hq * p.o_sh + static_cast<int64_t>(qrow) * p.o_sn + 4 * c;
  uint2 w;
  if constexpr (OUT_BF16) {
    w = make_uint2(pack_bf16x2(acc.x * inv, acc.y * inv), pack_bf16x2(acc.z * inv, acc.w * inv));
  } else {
    w = make_uint2(pack_f16x2(acc.x * inv, acc.y * inv), pack_f16x2(acc.z * inv, acc.w * inv));
  }
  *reinterpret_cast<uint2*>(dst) = w;
  if (c == 0 && p.lse != nullptr) p.lse[bh * p.sq + qrow] = wsum > 0.0f ? mx + logf(wsum) : -INFINITY;
}

int device_cus();

template <int D, int QK, bool CAUSAL>
void launch(const AttnParams& p, bool out_bf16, hipStream_t st) {
  // persistent grid (one block per CU, a multiple of the XCD count) when the
  // items outnumber the CUs
  const int round = (device_cus() / kXcds) * kXcds;
  const int blocks = (round >= kXcds && p.work > round) ? round : p.work;
  const dim3 grid(static_cast<uint32_t>(blocks)), block(kThreads);
  if (out_bf16) {
    attn_fwd_kernel<D, QK, CAUSAL, true><<<grid, block, 0, st>>>(p);
  } else {
    attn_fwd_kernel<D, QK, CAUSAL, false><<<grid, block, 0, st>>>(p);
  }
}

template <int QK>
void launch_kind(const AttnParams& p, int64_t head_dim, bool causal, bool out_bf16, hipStream_t st) {
  if (head_dim == 128) {
    if (causal) launch<128, QK, true>(p, out_bf16, st);
    else launch<128, QK, false>(p, out_bf16, st);
  } else {
    if (causal) launch<64, QK, true>(p, out_bf16, st);
    else launch<64, QK, false>(p, out_bf16, st);
  }
}

template <int D>
void launch_merge(const MergeParams& mp, bool out_bf16, hipStream_t st) {
  constexpr int kRowsPerBlock = 256 / (D / 4);
  const dim3 grid(static_cast<uint32_t>(cdiv(mp.rows, kRowsPerBlock))), block(256);
  if (out_bf16) {
    attn_merge_kernel<D, true><<<grid, block, 0, st>>>(mp);
  } else {
    attn_merge_kernel<D, false><<<grid, block, 0, st>>>(mp);
  }
}

// ---- key splits (non-causal only).  A launch of W = B*Hq*ceil(Sq/256)
// equal blocks runs in ceil(W / CUs) rounds, the last one partly idle (W = 160
// or 288 on 256 CUs: 38% or 44% of the CU time lost).  A plan (nfull, n) runs
// q-blocks [0, nfull) whole (nfull: a number of full rounds) and cuts the key
// range of each remaining q-block into n parts of ceil(T/n) tiles
// (T = ceil(Sk/64)), whose fp32 partial outputs a merge launch combines:
//   * nfull = 0: every q-block split (grids smaller than the device);
//   * nfull = whole rounds: only the last, partial round split.
// The host picks the plan of least estimated time, with a model fitted to
// MI355X measurements of this kernel (non-causal, 5 shapes x up to 6 split
// counts, within ~10%):
//   item time = (tiles + kItemTiles) * t_tile * (1 + kBusySlowdown * busy)
// where busy is the fraction of an XCD's CUs running in that round (the chip
// is power-limited: a tile step takes ~1.5x longer on a full chip than on a
// lone CU), and merge = kMergeLaunchUs + partial bytes / kMergeBytesPerUs.
constexpr int kMaxSplits = SAGE_MAX_KV_SPLITS;
constexpr int kMinSplitTiles = 4;        // keys per split >= 256 (automatic plans)
constexpr double kItemTiles = 5.3;       // prologue (Q, first K/V tiles) + epilogue, in tile steps
constexpr double kBusySlowdown = 0.48;
constexpr double kMergeLaunchUs = 3.0;
constexpr double kMergeBytesPerUs = 5.5e6;
// least estimated gain for a plan: the model predicts last-round splits within
// ~7% but overrates splitting every q-block of a small grid (measured 1.0-1.2x
// where it predicts 1.1-1.4x)
constexpr double kMinGainTail = 0.95;    // t_plan < 0.95 t_whole
constexpr double kMinGainAll = 0.83;     // t_plan < 0.83 t_whole (a 1.2x estimated speed-up)

struct SplitPlan {
  int64_t nfull;   // q-blocks run whole
  int64_t nsplit;  // splits of each of the others (1: none)
};

// Workspace of a plan: fp32 partial rows [items][256][D], then their LSEs [items][256].
int64_t split_workspace_bytes(int64_t qblocks, const SplitPlan& sp, int64_t head_dim) {
  return sp.nsplit > 1 ? (qblocks - sp.nfull) * sp.nsplit * kBM * (head_dim + 1) * 4 : 0;
}

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

// Time of one 256x64 tile step on a lone CU (us), fitted on MI355X.
double tile_us(int64_t head_dim, bool quantized) {
  if (head_dim == 128) return quantized ? 1.06 : 1.3;
  return quantized ? 0.81 : 0.94;
}

// `items` equal items of `tiles` tile steps, dealt round-robin over the XCDs.
double rounds_us(int64_t items, int64_t tiles, double t_tile, int cus) {
  if (items <= 0) return 0.0;
  const int64_t per_xcd = cus / kXcds > 0 ? cus / kXcds : 1;
  const int64_t on_xcd = cdiv(items, kXcds);  // items of the busiest XCD
  const int64_t full = on_xcd / per_xcd;
  const int64_t last = on_xcd - full * per_xcd;
  const double item = (static_cast<double>(tiles) + kItemTiles) * t_tile;
  double t = static_cast<double>(full) * item * (1.0 + kBusySlowdown);
  if (last > 0) t += item * (1.0 + kBusySlowdown * static_cast<double>(last) / static_cast<double>(per_xcd));
  return t;
}

double plan_us(int64_t qblocks, int64_t tiles, const SplitPlan& sp, int64_t head_dim, bool quantized, int cus) {
  const double tt = tile_us(head_dim, quantized);
  if (sp.nsplit <= 1) return rounds_us(qblocks, tiles, tt, cus);
  const int64_t pieces = (qblocks - sp.nfull) * sp.nsplit;
  return rounds_us(sp.nfull, tiles, tt, cus) + rounds_us(pieces, cdiv(tiles, sp.nsplit), tt, cus) +
         kMergeLaunchUs + static_cast<double>(split_workspace_bytes(qblocks, sp, head_dim)) / kMergeBytesPerUs;
}

// Plan of a launch: num_splits 0 = the least estimated time among the plans
// whose workspace fits in ws_bytes; 1 = unsplit; n > 1 = every q-block in n
// splits (at most one per key tile).  Causal launches and empty key ranges
// are never split.
SplitPlan plan_splits(bool quantized, int64_t qblocks, int64_t kv_len, int64_t head_dim, bool causal,
                      int num_splits, int64_t ws_bytes) {
  const SplitPlan whole{qblocks, 1};
  if (causal || kv_len <= 0 || num_splits == 1) return whole;
  const int64_t tiles = cdiv(kv_len, kBN);
  if (num_splits > 1) {
    const int64_t n = num_splits < tiles ? num_splits : tiles;
    return n > 1 ? SplitPlan{0, n} : whole;
  }
  const int cus = device_cus();
  const int64_t round = (cus / kXcds) * kXcds;  // blocks of one full round, a multiple of the XCD count
  const int64_t tail_full = round > 0 ? (qblocks / round) * round : 0;
  SplitPlan best = whole;
  const double base_t = plan_us(qblocks, tiles, whole, head_dim, quantized, cus);
  double best_score = 1.0;  // estimated time / bar, relative to the whole launch
  for (int64_t nfull : {int64_t{0}, tail_full}) {
    if (nfull >= qblocks) continue;
    const double bar = nfull > 0 ? kMinGainTail : kMinGainAll;
    for (int64_t n = 2; n <= kMaxSplits && n * kMinSplitTiles <= tiles; ++n) {
      const SplitPlan sp{nfull, n};
      if (split_workspace_bytes(qblocks, sp, head_dim) > ws_bytes) break;
      const double score = plan_us(qblocks, tiles, sp, head_dim, quantized, cus) / (bar * base_t);
      if (score < best_score) {
        best_score = score;
        best = sp;
      }
    }
    if (tail_full == 0) break;
  }
  return best;
}

// Validation and launch shared by the entry points.  Q/K strides are in
// elements (INT8: the contiguous [B,H,N,D] of the quant outputs).
int attn_fwd(int qk, const void* q, const void* k, const void* value_t, void* out, float* lse, const float* q_scale,
             const float* k_scale, int out_dtype, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t q_len,
             int64_t kv_len, int64_t head_dim, int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb, int64_t k_sh,
             int64_t k_sn, int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n, int is_causal, double sm_scale,
             int num_splits, void* workspace, int64_t workspace_bytes, void* stream, const char* fn) {
  if (out_dtype != SAGE_DTYPE_F16 && out_dtype != SAGE_DTYPE_BF16)
    return set_error(SAGE_ERR_INVALID_ARG, "%s: %s must be SAGE_DTYPE_F16 or SAGE_DTYPE_BF16, got %d", fn,
                     qk == kQkI8 ? "out_dtype" : "dtype", out_dtype);
  if (head_dim != 64 && head_dim != 128)
    return set_error(SAGE_ERR_UNSUPPORTED, "head_dim must be 64 or 128, got %lld", static_cast<long long>(head_dim));
  if (batch < 0 || q_heads <= 0 || kv_heads <= 0 || q_len < 0 || kv_len < 0)
    return set_error(SAGE_ERR_INVALID_ARG, "%s: negative or zero size", fn);
  if (q_heads % kv_heads != 0)
    return set_error(SAGE_ERR_INVALID_ARG, "q_heads (%lld) must be a multiple of kv_heads (%lld)",
                     static_cast<long long>(q_heads), static_cast<long long>(kv_heads));
  if (num_splits < 0 || num_splits > kMaxSplits || workspace_bytes < 0)
    return set_error(SAGE_ERR_INVALID_ARG, "%s: num_splits must be in [0, %d] (got %d), workspace_bytes >= 0", fn,
                     kMaxSplits, num_splits);
  if (batch == 0 || q_len == 0) return SAGE_OK;
  const bool i8 = is_i8(qk);
  if (!out || !q || (qk == kQkI8 && !q_scale) || (kv_len > 0 && (!k || !value_t || (i8 && !k_scale))))
    return set_error(SAGE_ERR_INVALID_ARG, "%s: null pointer argument", fn);
  const int64_t q_elem = qk == kQkI8 ? 1 : 2;
  const int64_t elem = i8 ? 1 : 2;  // K
  if (!aligned(q, 16) || (kv_len > 0 && (!aligned(k, 16) || !aligned(value_t, 16))))
    return set_error(SAGE_ERR_ALIGNMENT, "%s: q/k/value_t must be 16-byte aligned", fn);
  if (q_sb < 0 || q_sh < 0 || q_sn < 0 || k_sb < 0 || k_sh < 0 || k_sn < head_dim)
    return set_error(SAGE_ERR_INVALID_ARG, "%s: q/k strides must be non-negative and K rows must not overlap", fn);
  if (((q_sb * q_elem) % 16) || ((q_sh * q_elem) % 16) || ((q_sn * q_elem) % 16) || ((k_sb * elem) % 16) ||
      ((k_sh * elem) % 16) || ((k_sn * elem) % 16))
    return set_error(SAGE_ERR_ALIGNMENT, "%s: q/k strides must be multiples of 16 bytes", fn);
  if (!aligned(out, 16) || (o_stride_b % 8) || (o_stride_h % 8) || (o_stride_n % 8))
    return set_error(SAGE_ERR_ALIGNMENT, "%s: out needs a 16-byte aligned base and strides that are multiples of 8",
                     fn);
  if (lse != nullptr && !aligned(lse, 4))
    return set_error(SAGE_ERR_ALIGNMENT, "%s: lse must be 4-byte aligned", fn);
  const int64_t nqb = cdiv(q_len, kBM);
  const int64_t items1 = batch * q_heads * nqb;
  const int64_t np = cdiv(kv_len, SAGE_VT_ALIGN) * SAGE_VT_ALIGN;
  // per-head K and V_T are addressed through 32-bit buffer offsets (K tiles
  // are fetched up to three tiles past the last one)
  if (q_len > INT32_MAX - kBM || kv_len > INT32_MAX - kBN || items1 > INT32_MAX / kMaxSplits ||
      head_dim * np * 2 > UINT32_MAX || (kv_len + kBN * 5) * k_sn * elem > UINT32_MAX)
    return set_error(SAGE_ERR_UNSUPPORTED, "%s: sizes beyond 32-bit limits", fn);
  const SplitPlan sp = plan_splits(i8, items1, kv_len, head_dim, is_causal != 0, num_splits,
                                   workspace != nullptr ? workspace_bytes : 0);
  const int64_t ws_need = split_workspace_bytes(items1, sp, head_dim);
  if (sp.nsplit > 1) {
    if (workspace == nullptr || workspace_bytes < ws_need)
      return set_error(SAGE_ERR_INVALID_ARG, "%s: %lld key splits need a workspace of %lld bytes (got %lld)", fn,
                       static_cast<long long>(sp.nsplit), static_cast<long long>(ws_need),
                       static_cast<long long>(workspace != nullptr ? workspace_bytes : 0));
    if (!aligned(workspace, 16)) return set_error(SAGE_ERR_ALIGNMENT, "%s: workspace must be 16-byte aligned", fn);
    if ((items1 - sp.nfull) * kBM / (256 / (head_dim / 4)) > INT32_MAX)
      return set_error(SAGE_ERR_UNSUPPORTED, "%s: sizes beyond 32-bit limits", fn);
  }
  const int64_t work = sp.nfull + (items1 - sp.nfull) * sp.nsplit;

  AttnParams p;
  p.q = q;
  p.k = k;
  p.vt = static_cast<const uint16_t*>(value_t);
  p.out = out;
  p.lse = lse;
  p.q_scale = q_scale;
  p.k_scale = k_scale;
  p.q_sb = q_sb;
  p.q_sh = q_sh;
  p.q_sn = q_sn;
  p.k_sb = k_sb;
  p.k_sh = k_sh;
  p.k_sn = k_sn;
  p.o_sb = o_stride_b;
  p.o_sh = o_stride_h;
  p.o_sn = o_stride_n;
  p.np = np;
  // as the reference: fl(fl(sm_scale) * log2 e); its sign moves into Q
  const float sc = static_cast<float>(sm_scale) * 1.4426950408889634f;
  p.sc = std::fabs(sc);
  p.q_xor = std::signbit(sc) ? 0x80008000u : 0u;
  p.qpre = sc;  // the quantisation kernel's pre-scale of Q (sign included)
  p.hq = static_cast<int32_t>(q_heads);
  p.hkv = static_cast<int32_t>(kv_heads);
  p.sq = static_cast<int32_t>(q_len);
  p.sk = static_cast<int32_t>(kv_len);
  p.group = static_cast<int32_t>(q_heads / kv_heads);
  p.nqb = static_cast<int32_t>(nqb);
  p.q_groups = static_cast<int32_t>(cdiv(q_len, SAGE_Q_GROUP));
  p.k_groups = static_cast<int32_t>(cdiv(kv_len, SAGE_K_GROUP));
  p.work = static_cast<int32_t>(work);
  p.nfull = static_cast<int32_t>(sp.nfull);
  p.nsplit = static_cast<int32_t>(sp.nsplit);
  const int64_t pieces = (items1 - sp.nfull) * sp.nsplit;
  p.part = sp.nsplit > 1 ? static_cast<float*>(workspace) : nullptr;
  p.part_lse = sp.nsplit > 1 ? static_cast<float*>(workspace) + pieces * kBM * head_dim : nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bf16 = out_dtype == SAGE_DTYPE_BF16;
  if (qk == kQkI8) launch_kind<kQkI8>(p, head_dim, is_causal != 0, bf16, st);
  else if (qk == kQkI8F) launch_kind<kQkI8F>(p, head_dim, is_causal != 0, bf16, st);
  else if (qk == kQkF16) launch_kind<kQkF16>(p, head_dim, is_causal != 0, bf16, st);
  else launch_kind<kQkBf16>(p, head_dim, is_causal != 0, bf16, st);
  if (sp.nsplit > 1) {
    MergeParams mp;
    mp.part = p.part;
    mp.part_lse = p.part_lse;
    mp.out = out;
    mp.lse = lse;
    mp.o_sb = o_stride_b;
    mp.o_sh = o_stride_h;
    mp.o_sn = o_stride_n;
    mp.rows = (items1 - sp.nfull) * kBM;
    mp.hq = p.hq;
    mp.sq = p.sq;
    mp.nqb = p.nqb;
    mp.nfull = p.nfull;
    mp.nsplit = p.nsplit;
    if (head_dim == 128) launch_merge<128>(mp, bf16, st);
    else launch_merge<64>(mp, bf16, st);
  }
  return check_launch(fn);
}

// The plan a launch of this shape will run and the workspace it needs (0: unsplit).
int64_t attn_split_plan(bool quantized, int64_t batch, int64_t q_heads, int64_t q_len, int64_t kv_len,
                        int64_t head_dim, int is_causal, int num_splits, SplitPlan* plan_out) {
  if (head_dim != 64 && head_dim != 128)
    return set_error(SAGE_ERR_UNSUPPORTED, "head_dim must be 64 or 128, got %lld", static_cast<long long>(head_dim));
  if (batch < 0 || q_heads <= 0 || q_len < 0 || kv_len < 0 || num_splits < 0 || num_splits > kMaxSplits)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_attn_workspace_bytes: negative size or num_splits outside [0, %d]",
                     kMaxSplits);
  const int64_t items1 = batch * q_heads * cdiv(q_len, kBM);
  *plan_out = SplitPlan{items1, 1};
  if (batch == 0 || q_len == 0) return 0;
  if (items1 > INT32_MAX / kMaxSplits)
    return set_error(SAGE_ERR_UNSUPPORTED, "sage_attn_workspace_bytes: sizes beyond 32-bit limits");
  *plan_out = plan_splits(quantized, items1, kv_len, head_dim, is_causal != 0, num_splits, INT64_MAX);
  return split_workspace_bytes(items1, *plan_out, head_dim);
}

}  // namespace
}  // namespace sage

using namespace sage;

extern "C" int sage_attn_i8_fwd(const int8_t* q_i8, const int8_t* k_i8, const void* value_t, void* out,
                                const float* q_scale, const float* k_scale, int out_dtype,
                                int64_t batch, int64_t q_heads, int64_t kv_heads,
                                int64_t q_len, int64_t kv_len, int64_t head_dim,
                                int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                                int is_causal, void* stream) {
  clear_error();
  return attn_fwd(kQkI8, q_i8, k_i8, value_t, out, nullptr, q_scale, k_scale, out_dtype, batch, q_heads, kv_heads,
                  q_len, kv_len, head_dim, q_heads * q_len * head_dim, q_len * head_dim, head_dim,
                  kv_heads * kv_len * head_dim, kv_len * head_dim, head_dim, o_stride_b, o_stride_h, o_stride_n,
                  is_causal, 0.0, 1, nullptr, 0, stream, "sage_attn_i8_fwd");
}

extern "C" int sage_attn_i8_fwd_lse(const int8_t* q_i8, const int8_t* k_i8, const void* value_t, void* out,
                                    float* lse, const float* q_scale, const float* k_scale, int out_dtype,
                                    int64_t batch, int64_t q_heads, int64_t kv_heads,
                                    int64_t q_len, int64_t kv_len, int64_t head_dim,
                                    int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_n,
                                    int is_causal, void* stream) {
  clear_error();
  return attn_fwd(kQkI8, q_i8, k_i8, value_t, out, lse, q_scale, k_scale, out_dtype, batch, q_heads, kv_heads,
                  q_len, kv_len, head_dim, q_heads * q_len * head_dim, q_len * head_dim, head_dim,
                  kv_heads * kv_len * head_dim, kv_len * head_dim, head_dim, o_stride_b, o_stride_h, o_stride_n,
                  is_causal, 0.0, 1, nullptr, 0, stream, "sage_attn_i8_fwd_lse");
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
  return attn_fwd(dtype == SAGE_DTYPE_BF16 ? kQkBf16 : kQkF16, query, key, value_t, out, lse, nullptr, nullptr, dtype,
                  batch, q_heads, kv_heads, q_len, kv_len, head_dim, q_stride_b, q_stride_h, q_stride_n, k_stride_b,
                  k_stride_h, k_stride_n, o_stride_b, o_stride_h, o_stride_n, is_causal, sm_scale, num_splits,
                  workspace, workspace_bytes, stream, "sage_attn_direct_fwd");
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
  return attn_fwd(kQkI8F, query, k_i8, value_t, out, lse, nullptr, k_scale, dtype, batch, q_heads, kv_heads, q_len,
                  kv_len, head_dim, q_stride_b, q_stride_h, q_stride_n, kv_heads * kv_len * head_dim,
                  kv_len * head_dim, head_dim, o_stride_b, o_stride_h, o_stride_n, is_causal, sm_scale, num_splits,
                  workspace, workspace_bytes, stream, "sage_attn_i8_fwd_qfused");
}

extern "C" int64_t sage_attn_workspace_bytes(int quantized, int64_t batch, int64_t q_heads, int64_t q_len,
                                             int64_t kv_len, int64_t head_dim, int is_causal, int num_splits) {
  clear_error();
  SplitPlan sp;
  return attn_split_plan(quantized != 0, batch, q_heads, q_len, kv_len, head_dim, is_causal, num_splits, &sp);
}

extern "C" int sage_attn_split_plan(int quantized, int64_t batch, int64_t q_heads, int64_t q_len, int64_t kv_len,
                                    int64_t head_dim, int is_causal, int num_splits, int64_t* whole_qblocks,
                                    int* splits) {
  clear_error();
  if (whole_qblocks == nullptr || splits == nullptr)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_attn_split_plan: null output pointer");
  SplitPlan sp;
  const int64_t r =
      attn_split_plan(quantized != 0, batch, q_heads, q_len, kv_len, head_dim, is_causal, num_splits, &sp);
  if (r < 0) return static_cast<int>(r);
  *whole_qblocks = sp.nfull;
  *splits = static_cast<int>(sp.nsplit);
  return SAGE_OK;
}
