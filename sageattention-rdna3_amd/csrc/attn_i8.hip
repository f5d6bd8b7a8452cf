// Fused INT8-QK^T / fp16-PV flash attention for gfx950 (CDNA4, wave64 MFMA).
//
// Math (csrc/attn_gfx11.cu:409-825 of the reference): for query row i and key j
//   s_ij = float(sum_d q8[i,d] * k8[j,d]) * (q_scale[i/32] * k_scale[j/16])
// (log2 domain: Q was pre-scaled by sm_scale*log2 e), causal mask j > i
// (top-left) and j >= Sk, online softmax with exp2, P rounded to fp16 (RNE),
// O += P.V with fp32 accumulation, out = O * (1/l) cast to fp16/bf16.
//
// Mapping onto CDNA4:
//   * block = 4 waves x 32 query rows (BM = 128); KV tiles of BN = 64 keys;
//   * S^T = K . Q^T with v_mfma_i32_32x32x32_i8: A = K rows from LDS, B = the
//     wave's Q^T fragment held in registers for the whole kernel.  The 32x32
//     accumulator puts one query per lane column (lane & 31), so the row
//     softmax is 32 in-lane values plus one permlane32 swap;
//   * O^T = V^T . P^T with v_mfma_f32_32x32x16_f16: B = P^T taken straight
//     from the S^T accumulators (no LDS round trip), A = V_T rows from LDS.
//     The k-order of P inside each 16-key step is (4h..4h+3, 8+4h..8+4h+3)
//     for lane half h; V_T tiles are stored in LDS with bits 2 and 3 of the
//     key index swapped so each lane reads its 8 keys as one 16-byte load;
//   * K/V tiles are double buffered in LDS with register prefetch (one
//     barrier per tile);
//   * causal: KV loop stops at the block's last row, fully masked waves skip
//     the tile, masks are evaluated only on tail / diagonal tiles;
//   * block -> work remap keeps consecutive q-blocks of a head on one XCD
//     (shared L2 for K/V) and issues the heaviest causal blocks first.
#include <cmath>

#include "sage_common.h"

namespace sage {
namespace {

constexpr int kBM = 128;
constexpr int kBN = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kXcds = 8;  // MI355X: workgroups are dealt round-robin to 8 XCDs
constexpr float kRescale = 8.0f;  // lazy-rescale threshold of the running max (log2 units)

struct AttnParams {
  const int8_t* q8;      // [B,Hq,Sq,D]
  const int8_t* k8;      // [B,Hkv,Sk,D]
  const uint16_t* vt;    // fp16 [B,Hkv,D,np]
  void* out;
  const float* q_scale;  // [B,Hq,ceil(Sq/32)]
  const float* k_scale;  // [B,Hkv,ceil(Sk/16)]
  int64_t o_sb, o_sh, o_sn;
  int64_t np;
  int32_t hq, hkv, sq, sk;
  int32_t group;         // Hq / Hkv
  int32_t nqb;           // query blocks per head
  int32_t q_groups, k_groups;
  int32_t work;          // B * Hq * nqb
};

template <int D>
struct Cfg {
  static constexpr int kKStride = D + 16;          // bytes per K row in LDS
  static constexpr int kVStride = kBN + 8;         // halves per V_T row in LDS
  static constexpr int kKBytes = kBN * kKStride;
  static constexpr int kVBytes = D * kVStride * 2;
  static constexpr int kStage = kKBytes + kVBytes;
  static constexpr int kKChunks = kBN * D / 16 / kThreads;  // 16-byte K chunks per thread
  static constexpr int kVChunks = D * kBN / 8 / kThreads;   // 16-byte V chunks per thread
  static constexpr int kDS = D / 32;                        // k-steps of the QK MFMA
  static constexpr int kDB = D / 32;                        // 32-row d blocks of O^T
};

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

template <int D>
__device__ __forceinline__ void load_tile_regs(const AttnParams& p, const int8_t* kbase,
                                               const uint16_t* vbase, const float* ksp, int kt, int tid,
                                               uint4 (&kr)[Cfg<D>::kKChunks],
                                               uint4 (&vr)[Cfg<D>::kVChunks], float (&ks)[4]) {
  using C = Cfg<D>;
  // the tile's 4 key-group scales (same address in every lane: one broadcast);
  // groups past the end repeat the last one and only meet masked keys
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int gi = kt / 16 + g;
    ks[g] = ksp[gi < p.k_groups ? gi : p.k_groups - 1];
  }
#pragma unroll
  for (int i = 0; i < C::kKChunks; ++i) {
    const int c = tid + i * kThreads;
    const int row = c / (D / 16);
    const int c16 = c % (D / 16);
    if (kt + row < p.sk) {
      kr[i] = *reinterpret_cast<const uint4*>(kbase + static_cast<int64_t>(kt + row) * D + c16 * 16);
    } else {
      kr[i] = make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < C::kVChunks; ++i) {
    const int c = tid + i * kThreads;
    const int d = c / (kBN / 8);
    const int n8 = c % (kBN / 8);
    vr[i] = *reinterpret_cast<const uint4*>(vbase + static_cast<int64_t>(d) * p.np + kt + n8 * 8);
  }
}

template <int D>
__device__ __forceinline__ void store_tile_lds(char* stage, int tid, const uint4 (&kr)[Cfg<D>::kKChunks],
                                               const uint4 (&vr)[Cfg<D>::kVChunks]) {
  using C = Cfg<D>;
#pragma unroll
  for (int i = 0; i < C::kKChunks; ++i) {
    const int c = tid + i * kThreads;
    const int row = c / (D / 16);
    const int c16 = c % (D / 16);
    *reinterpret_cast<uint4*>(stage + row * C::kKStride + c16 * 16) = kr[i];
  }
  uint16_t* vs = reinterpret_cast<uint16_t*>(stage + C::kKBytes);
#pragma unroll
  for (int i = 0; i < C::kVChunks; ++i) {
    const int c = tid + i * kThreads;
    const int d = c / (kBN / 8);
    const int n8 = c % (kBN / 8);
    // keys n8*8 .. n8*8+7 of this row: within their 16-key group, keys with
    // bit3 = n8&1 and bit2 = 0 / 1 go to positions (n8&1)*4 / 8 + (n8&1)*4
    uint16_t* dst = vs + d * C::kVStride + (n8 >> 1) * 16 + (n8 & 1) * 4;
    *reinterpret_cast<uint2*>(dst) = make_uint2(vr[i].x, vr[i].y);
    *reinterpret_cast<uint2*>(dst + 8) = make_uint2(vr[i].z, vr[i].w);
  }
}

// One 64-key tile of one wave: S^T = K.Q^T (int8 MFMA), dequant, optional
// mask, online softmax, O^T += V^T.P^T (fp16 MFMA).  MASK selects the tail /
// diagonal version; the steady-state tiles run the unmasked one.
template <int D, bool CAUSAL, bool MASK>
__device__ __forceinline__ void attn_tile(const AttnParams& p, const char* stage, const int4_t (&qf)[Cfg<D>::kDS],
                                          const float (&ks)[4], float qs, int kt, int qrow, int m, int hh,
                                          float16_t_ (&o)[Cfg<D>::kDB], float& m_run, float& l_run) {
  using C = Cfg<D>;
  // ---- S^T = K . Q^T  (2 blocks of 32 keys)
  int16_t_ acc[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[nb][r] = 0;
    const char* krow = stage + (nb * 32 + m) * C::kKStride + hh * 16;
#pragma unroll
    for (int ds = 0; ds < C::kDS; ++ds) {
      const int4_t a = *reinterpret_cast<const int4_t*>(krow + ds * 32);
      acc[nb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, qf[ds], acc[nb], 0, 0, 0);
    }
  }
  // ---- dequant scales of the 4 key groups: fl(q_scale * k_scale)
  float sc[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) sc[g] = qs * ks[g];
  // ---- mask: dead entries become INT32_MIN, which no real dot product
  // reaches (|acc| <= 128*128*D < 2^22)
  if constexpr (MASK) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = kt + nb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
        const bool dead = (n >= p.sk) || (CAUSAL && n > qrow);
        acc[nb][r] = dead ? INT32_MIN : acc[nb][r];
      }
    }
  }
  // ---- row max: integer max inside each 16-key group, then one scale per
  // group (x -> x*sc is monotonic for sc > 0, so this is max_j fl(acc*sc))
  float mx = -INFINITY;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    int gm = acc[g >> 1][(g & 1) * 8];
#pragma unroll
    for (int r = 1; r < 8; ++r) gm = max(gm, acc[g >> 1][(g & 1) * 8 + r]);
    float gv = static_cast<float>(gm) * sc[g];
    if constexpr (MASK) gv = (gm == INT32_MIN) ? -INFINITY : gv;
    mx = __builtin_fmaxf(mx, gv);
  }
  mx = xhalf_max(mx);
  // ---- lazy rescale: the reference max only moves when some row's max grew
  // by more than kRescale (log2 units), so p = exp2(s - m_run) stays below
  // 2^kRescale (no fp16 overflow) and O is rescaled only on those tiles.
  if (__builtin_amdgcn_ballot_w64(mx > m_run + kRescale) != 0) {
    // keeps the block a real branch: without it the 64 multiplies of O are
    // speculated onto every tile (they are only 4 vector ops in the IR)
    asm volatile("" ::: "memory");
    float m_new = __builtin_fmaxf(m_run, mx);
    m_new = (m_new == -INFINITY) ? 0.0f : m_new;
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int db = 0; db < C::kDB; ++db) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
    }
  }
  // ---- p = exp2(acc*sc - m_run): dequant and max subtraction in one FMA
  float s[2][16];
  float lsum = 0.0f;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float e = fast_exp2(__builtin_fmaf(static_cast<float>(acc[nb][r]), sc[nb * 2 + (r >> 3)], -m_run));
      if constexpr (MASK) e = (acc[nb][r] == INT32_MIN) ? 0.0f : e;
      s[nb][r] = e;
      lsum += e;
    }
  }
  l_run += lsum;
  // ---- P^T fragments (fp16 RNE) straight from the accumulators
  half8_t pf[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float* sv = &s[t >> 1][(t & 1) * 8];
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = pack_f16x2(sv[2 * j], sv[2 * j + 1]);
    pf[t] = __builtin_bit_cast(half8_t, make_uint4(w[0], w[1], w[2], w[3]));
  }
  // ---- O^T += V^T . P^T
  const uint16_t* vs = reinterpret_cast<const uint16_t*>(stage + C::kKBytes);
#pragma unroll
  for (int db = 0; db < C::kDB; ++db) {
    const uint16_t* vrow = vs + (db * 32 + m) * C::kVStride + hh * 8;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const half8_t a = *reinterpret_cast<const half8_t*>(vrow + t * 16);
      o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[t], o[db], 0, 0, 0);
    }
  }
}

template <int D, bool CAUSAL, bool OUT_BF16>
__global__ __launch_bounds__(kThreads) void attn_i8_fwd_kernel(AttnParams p) {
  using C = Cfg<D>;
  __shared__ __align__(16) char smem[2 * C::kStage];

  // ---- work decode: XCD-contiguous ranges, heaviest causal blocks first
  const int L = blockIdx.x;
  const int xcd = L % kXcds;
  const int slot = L / kXcds;
  const int per = p.work / kXcds;
  const int rem = p.work % kXcds;
  const int w_idx = xcd * per + (xcd < rem ? xcd : rem) + slot;
  const int bh = w_idx / p.nqb;
  const int qb = p.nqb - 1 - (w_idx - bh * p.nqb);
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

  // ---- Q^T fragments and the wave's q scale
  int4_t qf[C::kDS];
  {
    const int8_t* qp = p.q8 + (static_cast<int64_t>(bh) * p.sq + qrow) * D + hh * 16;
#pragma unroll
    for (int ds = 0; ds < C::kDS; ++ds) {
      if (qrow < p.sq) {
        qf[ds] = *reinterpret_cast<const int4_t*>(qp + ds * 32);
      } else {
        qf[ds] = int4_t{0, 0, 0, 0};
      }
    }
  }
  const float qs = (wrow0 < p.sq) ? p.q_scale[static_cast<int64_t>(bh) * p.q_groups + wrow0 / 32] : 0.0f;

  const int64_t bhk = static_cast<int64_t>(b) * p.hkv + hk;
  const int8_t* kbase = p.k8 + bhk * p.sk * D;
  const uint16_t* vbase = p.vt + bhk * D * p.np;
  const float* ksp = p.k_scale + bhk * p.k_groups;

  const int kv_end = CAUSAL ? min(q0 + kBM, p.sk) : p.sk;

  float16_t_ o[C::kDB];
#pragma unroll
  for (int db = 0; db < C::kDB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
  }
  float m_run = -INFINITY;
  float l_run = 0.0f;

  uint4 kr[C::kKChunks];
  uint4 vr[C::kVChunks];
  float ks[4], ks_next[4];
  if (kv_end > 0) {
    load_tile_regs<D>(p, kbase, vbase, ksp, 0, tid, kr, vr, ks);
    store_tile_lds<D>(smem, tid, kr, vr);
  }
  __syncthreads();

  // tiles [0, main_end) need no mask for any wave of the block: fully inside
  // the key range and (causal) entirely at or left of the block's first row
  const int main_end = CAUSAL ? min(q0, p.sk / kBN * kBN) : p.sk / kBN * kBN;
  int it = 0;
  int kt = 0;
  for (; kt < main_end; kt += kBN, ++it) {
    const bool has_next = kt + kBN < kv_end;
    if (has_next) load_tile_regs<D>(p, kbase, vbase, ksp, kt + kBN, tid, kr, vr, ks_next);
    attn_tile<D, CAUSAL, false>(p, smem + (it & 1) * C::kStage, qf, ks, qs, kt, qrow, m, hh, o, m_run, l_run);
    if (has_next) {
      store_tile_lds<D>(smem + ((it + 1) & 1) * C::kStage, tid, kr, vr);
#pragma unroll
      for (int g = 0; g < 4; ++g) ks[g] = ks_next[g];
    }
    __syncthreads();
  }
  for (; kt < kv_end; kt += kBN, ++it) {
    const bool has_next = kt + kBN < kv_end;
    if (has_next) load_tile_regs<D>(p, kbase, vbase, ksp, kt + kBN, tid, kr, vr, ks_next);
    if (!CAUSAL || kt <= wrow0 + 31) {  // a wave whose rows all precede kt skips the tile
      attn_tile<D, CAUSAL, true>(p, smem + (it & 1) * C::kStage, qf, ks, qs, kt, qrow, m, hh, o, m_run, l_run);
    }
    if (has_next) {
      store_tile_lds<D>(smem + ((it + 1) & 1) * C::kStage, tid, kr, vr);
#pragma unroll
      for (int g = 0; g < 4; ++g) ks[g] = ks_next[g];
    }
    __syncthreads();
  }

  // ---- epilogue: 1/l, cast, 8-byte stores (4 consecutive d per store)
  const float l_tot = xhalf_sum(l_run);
  if (qrow < p.sq) {
    const float inv = (l_tot > 0.0f) ? 1.0f / l_tot : 0.0f;
    uint16_t* op = static_cast<uint16_t*>(p.out) + static_cast<int64_t>(b) * p.o_sb +
                   static_cast<int64_t>(qrow) * p.o_sn + static_cast<int64_t>(hq) * p.o_sh;
#pragma unroll
    for (int db = 0; db < C::kDB; ++db) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = db * 32 + 8 * r4 + 4 * hh;
        const float v0 = o[db][4 * r4 + 0] * inv, v1 = o[db][4 * r4 + 1] * inv;
        const float v2 = o[db][4 * r4 + 2] * inv, v3 = o[db][4 * r4 + 3] * inv;
        uint2 w;
        if constexpr (OUT_BF16) {
          w = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
        } else {
          w = make_uint2(pack_f16x2(v0, v1), pack_f16x2(v2, v3));
        }
        *reinterpret_cast<uint2*>(op + d) = w;
      }
    }
  }
}

template <int D, bool CAUSAL>
void launch(const AttnParams& p, bool out_bf16, hipStream_t st) {
  const dim3 grid(static_cast<uint32_t>(p.work)), block(kThreads);
  if (out_bf16) {
    attn_i8_fwd_kernel<D, CAUSAL, true><<<grid, block, 0, st>>>(p);
  } else {
    attn_i8_fwd_kernel<D, CAUSAL, false><<<grid, block, 0, st>>>(p);
  }
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
  if (out_dtype != SAGE_DTYPE_F16 && out_dtype != SAGE_DTYPE_BF16)
    return set_error(SAGE_ERR_INVALID_ARG, "out_dtype must be SAGE_DTYPE_F16 or SAGE_DTYPE_BF16, got %d", out_dtype);
  if (head_dim != 64 && head_dim != 128)
    return set_error(SAGE_ERR_UNSUPPORTED, "head_dim must be 64 or 128, got %lld", static_cast<long long>(head_dim));
  if (batch < 0 || q_heads <= 0 || kv_heads <= 0 || q_len < 0 || kv_len < 0)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_attn_i8_fwd: negative or zero size");
  if (q_heads % kv_heads != 0)
    return set_error(SAGE_ERR_INVALID_ARG, "q_heads (%lld) must be a multiple of kv_heads (%lld)",
                     static_cast<long long>(q_heads), static_cast<long long>(kv_heads));
  if (batch == 0 || q_len == 0) return SAGE_OK;
  if (!out || !q_i8 || !q_scale || (kv_len > 0 && (!k_i8 || !k_scale || !value_t)))
    return set_error(SAGE_ERR_INVALID_ARG, "sage_attn_i8_fwd: null pointer argument");
  if (!aligned(q_i8, 16) || (kv_len > 0 && (!aligned(k_i8, 16) || !aligned(value_t, 16))))
    return set_error(SAGE_ERR_ALIGNMENT, "sage_attn_i8_fwd: q_i8/k_i8/value_t must be 16-byte aligned");
  if (!aligned(out, 8) || (o_stride_b % 4) || (o_stride_h % 4) || (o_stride_n % 4))
    return set_error(SAGE_ERR_ALIGNMENT, "sage_attn_i8_fwd: out needs an 8-byte aligned base and strides that are multiples of 4");
  const int64_t nqb = cdiv(q_len, kBM);
  const int64_t work = batch * q_heads * nqb;
  if (q_len > INT32_MAX - kBM || kv_len > INT32_MAX - kBN || work > INT32_MAX)
    return set_error(SAGE_ERR_UNSUPPORTED, "sage_attn_i8_fwd: sizes beyond 32-bit limits");

  AttnParams p;
  p.q8 = q_i8;
  p.k8 = k_i8;
  p.vt = static_cast<const uint16_t*>(value_t);
  p.out = out;
  p.q_scale = q_scale;
  p.k_scale = k_scale;
  p.o_sb = o_stride_b;
  p.o_sh = o_stride_h;
  p.o_sn = o_stride_n;
  p.np = cdiv(kv_len, SAGE_VT_ALIGN) * SAGE_VT_ALIGN;
  p.hq = static_cast<int32_t>(q_heads);
  p.hkv = static_cast<int32_t>(kv_heads);
  p.sq = static_cast<int32_t>(q_len);
  p.sk = static_cast<int32_t>(kv_len);
  p.group = static_cast<int32_t>(q_heads / kv_heads);
  p.nqb = static_cast<int32_t>(nqb);
  p.q_groups = static_cast<int32_t>(cdiv(q_len, SAGE_Q_GROUP));
  p.k_groups = static_cast<int32_t>(cdiv(kv_len, SAGE_K_GROUP));
  p.work = static_cast<int32_t>(work);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bf16 = out_dtype == SAGE_DTYPE_BF16;
  if (head_dim == 128) {
    if (is_causal) launch<128, true>(p, bf16, st);
    else launch<128, false>(p, bf16, st);
  } else {
    if (is_causal) launch<64, true>(p, bf16, st);
    else launch<64, false>(p, bf16, st);
  }
  return check_launch("sage_attn_i8_fwd");
}
