// Fused INT8-QK^T / fp16-PV flash attention for gfx950 (CDNA4, wave64 MFMA).
//
// Math (csrc/attn_gfx11.cu:409-825 of the reference): for query row i and key j
//   s_ij = float(sum_d q8[i,d] * k8[j,d]) * (q_scale[i/32] * k_scale[j/16])
// (log2 domain: Q was pre-scaled by sm_scale*log2 e), causal mask j > i
// (top-left) and j >= Sk, online softmax with exp2, P rounded to fp16 (RNE),
// O += P.V with fp32 accumulation, out = O * (1/l) cast to fp16/bf16.
//
// Mapping onto CDNA4:
//   * block = 8 waves x 32 query rows (BM = 256), one block per CU, two waves
//     per SIMD; KV tiles of BN = 64 keys shared by all 8 waves through LDS;
//   * S^T = K . Q^T with v_mfma_i32_32x32x32_i8: A = K rows from LDS, B = the
//     wave's Q^T fragment held in registers for the whole kernel.  The 32x32
//     accumulator puts one query per lane column (lane & 31), so the row
//     softmax is 32 in-lane values plus one permlane32 swap;
//   * O^T = V^T . P^T with v_mfma_f32_32x32x16_f16: B = P^T taken straight
//     from the S^T accumulators (no LDS round trip), A = V_T rows from LDS.
//     The k-order of P inside each 16-key step is (4h..4h+3, 8+4h..8+4h+3)
//     for lane half h; V_T tiles are stored in LDS with bits 2 and 3 of the
//     key index swapped so each lane reads its 8 keys as one 16-byte load;
//   * ping-pong: waves 0-3 and 4-7 (one of each per SIMD) run a phase apart.
//     Each tile takes two barrier-separated phases; in every phase one wave
//     of a SIMD issues only MFMAs (S of tile j and P.V of tile j-1) while the
//     other runs only the VALU softmax of its tile, so the matrix cores and
//     the VALU of each SIMD stay busy at the same time;
//   * online softmax with a lazy reference max: O and l are rescaled only when
//     a row max grows by more than 2^8, so most tiles touch O only in MFMAs;
//   * K/V tiles are double buffered in LDS; global loads go through buffer
//     descriptors (tail rows of K read as zero) one phase ahead of the store;
//   * causal: the KV loop stops at the block's last row, waves skip tiles
//     left of their rows' reach, masks only on tail / diagonal tiles;
//   * block -> work remap keeps consecutive q-blocks of a head on one XCD
//     (shared L2 for K/V) and issues the heaviest causal blocks first.
#include <cmath>
#include <type_traits>

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
  static constexpr int kKStride = D + 16;                    // bytes per K row in LDS
  static constexpr int kVStride = kBN + 8;                   // halves per V_T row in LDS
  static constexpr int kKStage = kBN * kKStride;             // bytes of one K stage
  static constexpr int kVStage = D * kVStride * 2;           // bytes of one V stage
  static constexpr int kVBase = 2 * kKStage;                 // V stages follow the two K stages
  static constexpr int kSmem = 2 * kKStage + 2 * kVStage;
  static constexpr int kKTasks = kBN * D / 16;               // 16-byte K chunks per tile
  static constexpr int kVTasks = D * kBN / 8;                // 16-byte V_T chunks per tile
  static constexpr int kKChunks = (kKTasks + kThreads - 1) / kThreads;
  static constexpr int kVChunks = (kVTasks + kThreads - 1) / kThreads;
  static constexpr int kDS = D / 32;                         // k-steps of the QK MFMA
  static constexpr int kDB = D / 32;                         // 32-row d blocks of O^T
};

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

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

// Tile copy global -> registers -> LDS, shared by all threads of the block.
// Chunk i of a thread lies i passes after chunk 0 (a pass = kThreads chunks),
// so only chunk 0's offsets live in registers: later chunks add a
// compile-time LDS delta and a uniform global delta.
template <int D>
struct TileCopy {
  using C = Cfg<D>;
  static constexpr int kKRowsPerPass = kThreads / (D / 16);   // K rows per pass
  static constexpr int kVRowsPerPass = kThreads / (kBN / 8);  // V_T d-rows per pass
  uint32_t k_goff, k_loff, v_goff, v_loff;
  uint4 kr[C::kKChunks];
  uint4 vr[C::kVChunks];

  __device__ __forceinline__ TileCopy(int tid, int np) {
    const int row = tid / (D / 16);
    const int c16 = tid % (D / 16);
    k_goff = row * D + c16 * 16;
    k_loff = row * C::kKStride + c16 * 16;
    const int d = tid / (kBN / 8);
    const int n8 = tid % (kBN / 8);
    v_goff = static_cast<uint32_t>((d * np + n8 * 8) * 2);
    // keys n8*8 .. n8*8+7 of row d: within their 16-key group, keys with
    // bit3 = n8&1 and bit2 = 0 / 1 go to positions (n8&1)*4 / 8 + (n8&1)*4
    v_loff = (d * C::kVStride + (n8 >> 1) * 16 + (n8 & 1) * 4) * 2;
  }

  // K rows kt.. (rows >= sk read as zero) and V_T tokens kt.. (always inside
  // the padded row) into registers.
  __device__ __forceinline__ void load(const AttnParams& p, const int8_t* kbase, const uint16_t* vbase, int kt,
                                       bool do_k, bool do_v, int tid) {
    if (do_k) {
      const int rows = min(p.sk - kt, kBN);
      const auto rk = make_rsrc(kbase + static_cast<int64_t>(kt) * D, static_cast<uint32_t>(max(rows, 0) * D));
#pragma unroll
      for (int i = 0; i < C::kKChunks; ++i) {
        if (C::kKTasks % kThreads == 0 || tid + i * kThreads < C::kKTasks) {
          const u32x4_t w = __builtin_amdgcn_raw_buffer_load_b128(rk, k_goff + i * kKRowsPerPass * D, 0, 0);
          kr[i] = make_uint4(w.x, w.y, w.z, w.w);
        }
      }
    }
    if (do_v) {
      const auto rv = make_rsrc(vbase + kt, static_cast<uint32_t>((D * static_cast<int>(p.np) - kt) * 2));
      const int pass = __builtin_amdgcn_readfirstlane(kVRowsPerPass * static_cast<int>(p.np) * 2);
#pragma unroll
      for (int i = 0; i < C::kVChunks; ++i) {
        if (C::kVTasks % kThreads == 0 || tid + i * kThreads < C::kVTasks) {
          const u32x4_t w = __builtin_amdgcn_raw_buffer_load_b128(rv, v_goff, i * pass, 0);
          vr[i] = make_uint4(w.x, w.y, w.z, w.w);
        }
      }
    }
  }

  __device__ __forceinline__ void store(char* smem, int stage, bool do_k, bool do_v, int tid) {
    if (do_k) {
      char* kb = smem + stage * C::kKStage + k_loff;
#pragma unroll
      for (int i = 0; i < C::kKChunks; ++i) {
        if (C::kKTasks % kThreads == 0 || tid + i * kThreads < C::kKTasks)
          *reinterpret_cast<uint4*>(kb + i * kKRowsPerPass * C::kKStride) = kr[i];
      }
    }
    if (do_v) {
      char* vb = smem + C::kVBase + stage * C::kVStage + v_loff;
#pragma unroll
      for (int i = 0; i < C::kVChunks; ++i) {
        if (C::kVTasks % kThreads == 0 || tid + i * kThreads < C::kVTasks) {
          char* dst = vb + i * kVRowsPerPass * C::kVStride * 2;
          *reinterpret_cast<uint2*>(dst) = make_uint2(vr[i].x, vr[i].y);
          *reinterpret_cast<uint2*>(dst + 16) = make_uint2(vr[i].z, vr[i].w);
        }
      }
    }
  }
};

// The tile's 4 key-group scales, read through the constant address space so
// they land in SGPRs (the address is wave-uniform and nothing writes the
// scales during the kernel); groups past the end repeat the last one and only
// meet masked keys.
typedef const __attribute__((address_space(4))) float* const_f32_ptr;
__device__ __forceinline__ void load_ks(const AttnParams& p, const float* ksp, int kt, float (&ks)[4]) {
  const_f32_ptr kc = (const_f32_ptr)(reinterpret_cast<uint64_t>(uniform_ptr(ksp)));
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int gi = kt / 16 + g;
    ks[g] = kc[gi < p.k_groups ? gi : p.k_groups - 1];
  }
}

// S^T of one 64-key tile for the wave's 32 queries: two 32x32 int32 blocks.
template <int D>
__device__ __forceinline__ void qk_tile(const char* kstage, const int4_t (&qf)[Cfg<D>::kDS], int m, int hh,
                                        int16_t_ (&acc)[2]) {
  using C = Cfg<D>;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const char* krow = kstage + (nb * 32 + m) * C::kKStride + hh * 16;
#pragma unroll
    for (int ds = 0; ds < C::kDS; ++ds) {
      const int4_t a = *reinterpret_cast<const int4_t*>(krow + ds * 32);
      acc[nb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, qf[ds], ds == 0 ? int16_t_{} : acc[nb], 0, 0, 0);
    }
  }
  __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
  for (int i = 0; i < 2 * C::kDS - 2; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
}

// O^T += V^T . P^T for one 64-key tile.
template <int D>
__device__ __forceinline__ void pv_tile(const char* vstage, const half8_t (&pf)[4], int m, int hh,
                                        float16_t_ (&o)[Cfg<D>::kDB]) {
  using C = Cfg<D>;
  const uint16_t* vs = reinterpret_cast<const uint16_t*>(vstage);
#pragma unroll
  for (int db = 0; db < C::kDB; ++db) {
    const uint16_t* vrow = vs + (db * 32 + m) * C::kVStride + hh * 8;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const half8_t a = *reinterpret_cast<const half8_t*>(vrow + t * 16);
      o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[t], o[db], 0, 0, 0);
    }
  }
  // operands read two MFMAs ahead of use, not all at once (register budget)
  __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
  for (int i = 0; i < 4 * C::kDB - 2; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
}

// Softmax of one tile for one wave: S (int32 in `acc`, read only) -> P (fp16
// fragments in `pf`), updating the running max / sum and, rarely, rescaling O.
// On masked tiles the dead keys (j >= Sk, causal j > i) are re-derived where
// they are used instead of being written into a copy of S (register budget).
template <int D, bool CAUSAL, bool MASK>
__device__ __forceinline__ void softmax_tile(const AttnParams& p, const int16_t_ (&acc)[2], const float (&ks)[4],
                                             float qs, int kt, int qrow, int hh, half8_t (&pf)[4],
                                             float16_t_ (&o)[Cfg<D>::kDB], float& m_run, float& l_run) {
  using C = Cfg<D>;
  auto dead = [&](int nb, int r) {
    const int n = kt + nb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
    return (n >= p.sk) || (CAUSAL && n > qrow);
  };
  // ---- dequant scales of the 4 key groups: fl(q_scale * k_scale)
  float sc[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) sc[g] = qs * ks[g];
  // ---- row max: integer max inside each 16-key group, then one scale per
  // group (x -> x*sc is monotonic for sc > 0, so this is max_j fl(acc*sc));
  // dead keys count as INT32_MIN, which no real dot product reaches
  // (|acc| <= 128*128*D < 2^22)
  float mx = -INFINITY;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int nb = g >> 1;
    int gm = INT32_MIN;
#pragma unroll
    for (int r = (g & 1) * 8; r < (g & 1) * 8 + 8; ++r) {
      int a = acc[nb][r];
      if constexpr (MASK) a = dead(nb, r) ? INT32_MIN : a;
      gm = max(gm, a);
    }
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
  // ---- p = exp2(acc*sc - m_run): dequant and max subtraction in one FMA;
  // P^T fragments (fp16 RNE) straight from the accumulator layout
  float lsum = 0.0f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float e2[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int nb = t >> 1;
        const int r = (t & 1) * 8 + 2 * j + u;
        float e = fast_exp2(__builtin_fmaf(static_cast<float>(acc[nb][r]), sc[t], -m_run));
        if constexpr (MASK) e = dead(nb, r) ? 0.0f : e;
        lsum += e;
        e2[u] = e;
      }
      w[j] = pack_f16x2(e2[0], e2[1]);
    }
    pf[t] = __builtin_bit_cast(half8_t, make_uint4(w[0], w[1], w[2], w[3]));
  }
  l_run += lsum;
}

template <int D, bool CAUSAL, bool OUT_BF16>
__global__ __launch_bounds__(kThreads) void attn_i8_fwd_kernel(AttnParams p) {
  using C = Cfg<D>;
  __shared__ __align__(16) char smem[C::kSmem];

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
  const int role = wave >> 2;  // 0: MFMA phase first; 1: a phase behind
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
  const int ntiles = (kv_end + kBN - 1) / kBN;
  // tiles [0, w_main) need no mask for this wave (inside the key range and,
  // causal, left of the wave's first row)
  const int w_main = CAUSAL ? min(wrow0 + 1, p.sk) / kBN : p.sk / kBN;

  float16_t_ o[C::kDB];
#pragma unroll
  for (int db = 0; db < C::kDB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
  }
  float m_run = -INFINITY;
  float l_run = 0.0f;
  int16_t_ acc[2];
  half8_t pf[4];
  float ks[4];

  TileCopy<D> tc(tid, static_cast<int>(p.np));
  // ---- prologue: K_0 into stage 0
  if (ntiles > 0) {
    tc.load(p, kbase, vbase, 0, true, false, tid);
    tc.store(smem, 0, true, false, tid);
  }
  __syncthreads();


  // Step j has two barrier-separated phases.  Stage j&1 holds K_j and
  // V_{j-1} during both; K_{j+1} and V_j go to stage (j+1)&1 (free since step
  // j-1 ended): loaded into registers at the start of step j and stored at
  // its end, two phases later.  MFMA phase of step j: S_j = K_j . Q^T and
  // O += P_{j-1} . V_{j-1}; softmax phase: S_j -> P_j.  Role 0 runs (MFMA,
  // softmax) of step j, role 1 runs (softmax of j-1, MFMA of j).  Each role
  // has its own copy of the loop (same barrier sequence), so neither carries
  // the other's register assignment.  Tiles a wave cannot see go through the
  // masked softmax (P = 0), so the MFMA work is unconditional.
  auto softmax_phase = [&](int j) __attribute__((always_inline)) {
    if (j < w_main) {
      softmax_tile<D, CAUSAL, false>(p, acc, ks, qs, j * kBN, qrow, hh, pf, o, m_run, l_run);
    } else {
      softmax_tile<D, CAUSAL, true>(p, acc, ks, qs, j * kBN, qrow, hh, pf, o, m_run, l_run);
    }
  };
  auto mfma_phase = [&](int j, bool with_pv) __attribute__((always_inline)) {
    load_ks(p, ksp, j * kBN, ks);
    qk_tile<D>(smem + (j & 1) * C::kKStage, qf, m, hh, acc);
    if (with_pv) pv_tile<D>(smem + C::kVBase + (j & 1) * C::kVStage, pf, m, hh, o);
  };
  // tiles [0, n_main) need no mask for any wave of the block; they run in a
  // loop with only the unmasked softmax (one register assignment for O), the
  // rest (tail / diagonal, at most a few) in a loop that picks per wave
  const int n_main = min(CAUSAL ? min(q0, p.sk) / kBN : p.sk / kBN, ntiles);
  auto run = [&](auto role_tag) __attribute__((always_inline)) {
    constexpr int ROLE = decltype(role_tag)::value;
    auto step = [&](int j, auto masked_tag) __attribute__((always_inline)) {
      constexpr bool GENERIC = decltype(masked_tag)::value;
      const bool ld_k = j + 1 < ntiles;
      tc.load(p, kbase, vbase, j * kBN + kBN, ld_k, false, tid);
      tc.load(p, kbase, vbase, j * kBN, false, true, tid);
      const int js = ROLE == 0 ? j : j - 1;  // the tile this wave's softmax phase handles
      auto smax = [&]() __attribute__((always_inline)) {
        if constexpr (GENERIC) {
          softmax_phase(js);
        } else {
          softmax_tile<D, CAUSAL, false>(p, acc, ks, qs, js * kBN, qrow, hh, pf, o, m_run, l_run);
        }
      };
      if constexpr (ROLE == 0) {
        mfma_phase(j, j > 0);
      } else {
        if (j > 0) smax();
      }
      __syncthreads();
      if constexpr (ROLE == 0) {
        smax();
      } else {
        mfma_phase(j, j > 0);
      }
      tc.store(smem, (j + 1) & 1, ld_k, true, tid);
      __syncthreads();
    };
    int j = 0;
    for (; j < n_main; ++j) step(j, std::false_type{});
    for (; j < ntiles; ++j) step(j, std::true_type{});
    // last step: only P.V of the last tile (V_{ntiles-1} in stage ntiles&1)
    const char* v_last = smem + C::kVBase + (ntiles & 1) * C::kVStage;
    if constexpr (ROLE == 0) {
      pv_tile<D>(v_last, pf, m, hh, o);
    } else {
      softmax_phase(ntiles - 1);
    }
    __syncthreads();
    if constexpr (ROLE == 1) pv_tile<D>(v_last, pf, m, hh, o);
  };
  if (ntiles > 0) {
    if (role == 0) run(std::integral_constant<int, 0>{});
    else run(std::integral_constant<int, 1>{});
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
