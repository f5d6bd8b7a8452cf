// Prologue kernels of the quantized attention path on gfx950:
//   * per-block INT8 quantisation of Q and K (one launch for both),
//   * the K mean for smooth_k (two small launches, deterministic order),
//   * the V -> fp16 V_T layout transform,
//   * K quantisation + V layout in one launch, and for smooth_k the K mean's
//     chunk sums followed by one launch that finishes the mean inside its K
//     quantisation blocks (what sageattn runs before the attention kernel).
// All are HBM-bound byte shuffles: one 16-byte load per lane per row
// piece, wave64 reductions, 8/16-byte coalesced stores, no MFMA.
//
// Bit-exactness: the quantiser's arithmetic follows the reference order
// (csrc/attn_gfx11.cu:179-321) in IEEE fp32 with contraction disabled in this
// file (the build also passes -ffp-contract=off), true division for
// amax/127 and 127/amax, and the reference rounding rule (:85-92).
#pragma clang fp contract(off)

#include "sage_common.h"

namespace sage {
namespace {

constexpr int kWave = 64;
constexpr int kQGroup = SAGE_Q_GROUP;  // tokens per Q scale
constexpr int kKGroup = SAGE_K_GROUP;  // tokens per K scale
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float wave_max_xor(float v, int width_log2) {
  // butterfly over lanes xor 1..2^(width_log2-1); max is order independent
  for (int m = 1; m < (1 << width_log2); m <<= 1) v = __builtin_fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// ------------------------------------------------------------------ quant
struct QuantParams {
  const void* q;
  const void* k;
  const void* k_mean;  // [B,Hkv,D] or null
  int8_t* q8;
  float* q_scale;
  int8_t* k8;
  float* k_scale;
  int64_t q_sb, q_sh, q_sn;
  int64_t k_sb, k_sh, k_sn;
  int64_t n_q_units;      // B*Hq*ceil(Sq/32)
  int64_t n_units;        // n_q_units + B*Hkv*ceil(Sk/32)
  int32_t hq, hkv, sq, sk;
  int32_t q_units, k_units;  // 32-token units per head
  int32_t q_groups, k_groups;
  float s;  // fp32(sm_scale) * fp32(log2 e)
};

// One wave64 per 32-token unit.  Q unit = one 32-token scale group over all 64
// lanes; K unit = two 16-token groups, one per half wave.  Lane l of half h
// owns 16-byte column chunk `cc` of rows h*16 + rsub + i*RPI (i < ITER), so
// every load instruction covers whole rows and every store is coalesced.
// load() issues the unit's row loads; quantise() waits for them and writes
// q8/k8 and the scale(s), given the lane's 8 mean values (K with smooth_k).
template <bool BF16, int D>
struct QuantUnit {
  static constexpr int CPR = D / 8;       // 16-byte chunks per row
  static constexpr int RPI = 32 / CPR;    // rows per iteration per half wave
  static constexpr int ITER = 16 / RPI;   // iterations per lane
  const QuantParams* pp;  // the launch's parameters
  bool valid, is_q;
  int64_t bh;
  int ub, S, half, li, cc, row0;
  uint4 raw[ITER];

  __device__ __forceinline__ QuantUnit(const QuantParams& p_, int64_t unit, int lane) : pp(&p_) {
    valid = unit < pp->n_units;
    is_q = unit < pp->n_q_units;
    const int64_t u = is_q ? unit : unit - pp->n_q_units;
    const int upb = is_q ? pp->q_units : pp->k_units;
    S = is_q ? pp->sq : pp->sk;
    bh = u / upb;
    ub = static_cast<int>(u - bh * upb);
    half = lane >> 5;
    li = lane & 31;
    cc = li % CPR;
    row0 = ub * 32 + half * 16 + li / CPR;
  }

  __device__ __forceinline__ void load() {
    const int H = is_q ? pp->hq : pp->hkv;
    const int64_t b = bh / H;
    const int64_t h = bh - b * H;
    const uint16_t* src = static_cast<const uint16_t*>(is_q ? pp->q : pp->k);
    const int64_t sb = is_q ? pp->q_sb : pp->k_sb;
    const int64_t sh = is_q ? pp->q_sh : pp->k_sh;
    const int64_t sn = is_q ? pp->q_sn : pp->k_sn;
    const uint16_t* base = src + b * sb + h * sh + cc * 8;
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      const int row = row0 + i * RPI;
      if (valid && row < S) {
        // streaming: each input byte is read once (non-temporal, no cache residency)
        const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(base + static_cast<int64_t>(row) * sn));
        raw[i] = make_uint4(t.x, t.y, t.z, t.w);
      } else {
        raw[i] = make_uint4(0, 0, 0, 0);
      }
    }
  }

  // the lane's 8 columns of K's mean from the [B,Hkv,D] tensor pp->k_mean
  __device__ __forceinline__ void global_mean(float (&mean)[8]) const {
    const uint4 mr = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(pp->k_mean) + bh * D + cc * 8);
    const uint32_t mw[4] = {mr.x, mr.y, mr.z, mr.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float2_t f = unpack2<BF16>(mw[j]);
      mean[2 * j] = f.x;
      mean[2 * j + 1] = f.y;
    }
  }

  __device__ __forceinline__ void quantise(const float (&mean)[8], bool has_mean, int lane) {
    if (!valid) return;
    const float pre = is_q ? pp->s : 1.0f;
    // pass 1: absmax of fl(x*s) (Q) or |fl(x - mean)| (K), floor 1e-7
    float amax = kAmaxFloor;
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      if (row0 + i * RPI < S) {
        const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float2_t f = unpack2<BF16>(w[j]);
          float v0 = f.x, v1 = f.y;
          if (has_mean) {
            v0 = v0 - mean[2 * j];
            v1 = v1 - mean[2 * j + 1];
          }
          amax = __builtin_fmaxf(amax, __builtin_fabsf(v0 * pre));
          amax = __builtin_fmaxf(amax, __builtin_fabsf(v1 * pre));
        }
      }
    }
    amax = wave_max_xor(amax, 5);  // within the half wave (one K group)
    if (is_q) amax = __builtin_fmaxf(amax, __shfl_xor(amax, 32, kWave));  // whole wave (Q group)

    const float scale = amax / 127.0f;
    const float inv = 127.0f / amax;
    const float iscale = inv * pre;
    if (is_q) {
      if (lane == 0) pp->q_scale[bh * pp->q_groups + ub] = scale;
    } else if (li == 0) {
      const int g = ub * 2 + half;
      if (g * kKGroup < S) pp->k_scale[bh * pp->k_groups + g] = scale;
    }

    // pass 2: quantise and store 8 bytes per chunk
    int8_t* dst = (is_q ? pp->q8 : pp->k8) + bh * static_cast<int64_t>(S) * D + cc * 8;
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      const int row = row0 + i * RPI;
      if (row < S) {
        const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
        int r8[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float2_t f = unpack2<BF16>(w[j]);
          float v0 = f.x, v1 = f.y;
          if (has_mean) {
            v0 = v0 - mean[2 * j];
            v1 = v1 - mean[2 * j + 1];
          }
          r8[2 * j] = round_half_away_i8(v0 * iscale);
          r8[2 * j + 1] = round_half_away_i8(v1 * iscale);
        }
        uint2 o;
        o.x = pack_i8x4(r8[0], r8[1], r8[2], r8[3]);
        o.y = pack_i8x4(r8[4], r8[5], r8[6], r8[7]);
        const u32x2_t ov = {o.x, o.y};
        __builtin_nontemporal_store(ov, reinterpret_cast<u32x2_t*>(dst + static_cast<int64_t>(row) * D));
      }
    }
  }
};

template <bool BF16, int D>
__device__ __forceinline__ void quant_unit(const QuantParams& p, int64_t unit, int lane) {
  QuantUnit<BF16, D> u(p, unit, lane);
  if (!u.valid) return;
  u.load();
  float mean[8];
  const bool has_mean = (!u.is_q) && (p.k_mean != nullptr);
#pragma unroll
  for (int j = 0; j < 8; ++j) mean[j] = 0.0f;
  if (has_mean) u.global_mean(mean);
  u.quantise(mean, has_mean, lane);
}

template <bool BF16, int D>
__global__ __launch_bounds__(256) void quant_qk_i8_kernel(QuantParams p) {
  quant_unit<BF16, D>(p, static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6), threadIdx.x & (kWave - 1));
}

// ------------------------------------------------------------------ K mean
// rows per stage-1 block.  1024 rather than 256: a quarter of the chunk sums
// for the stage that adds them (which prep_kv_mean_kernel's K blocks each
// repeat), and on MI355X the two-launch smooth_k prologue then ties the
// three-launch one (C3 107.0 / 106.7 us, C5 256.7 / 256.1 us) where with 256
// it lost 5% at C5 (270 / 257 us); the three-launch path itself gained ~1% at C5
// and held at C3 (2048: C3 +2%, its 256 blocks fill one round).
constexpr int kMeanChunk = 1024;

struct MeanParams {
  const void* k;
  void* mean;
  float* ws;  // [B*H, nchunks, D]
  int64_t sb, sh, sn;
  int32_t h, s, nchunks;
};

// Stage 1: block (chunk, h, b) sums its kMeanChunk rows per column.  Thread t
// owns column chunk t % CPR and row slot t / CPR (rows slot, slot + SLOTS,
// ... in order); slot sums are combined in slot order through LDS.  The order
// is fixed so the result is reproducible.
template <bool BF16, int D>
__device__ __forceinline__ void k_mean_partial_block(const MeanParams& p, int64_t blk) {
  constexpr int CPR = D / 8;
  constexpr int SLOTS = 256 / CPR;
  constexpr int PASSES = kMeanChunk / SLOTS;
  constexpr int BATCH = PASSES < 16 ? PASSES : 16;  // row loads in flight per thread
  __shared__ float red[SLOTS][D];
  const int t = threadIdx.x;
  const int cc = t % CPR;
  const int slot = t / CPR;
  const int64_t bh = blk / p.nchunks;
  const int64_t chunk = blk - bh * p.nchunks;
  const int64_t b = bh / p.h;
  const int64_t h = bh - b * p.h;
  const uint16_t* base = static_cast<const uint16_t*>(p.k) + b * p.sb + h * p.sh + cc * 8;
  const int row0 = static_cast<int>(chunk) * kMeanChunk + slot;

  float acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
  for (int j0 = 0; j0 < PASSES; j0 += BATCH) {
    uint4 raw[BATCH];
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const int row = row0 + (j0 + j) * SLOTS;
      raw[j] = make_uint4(0, 0, 0, 0);
      if (row < p.s) {
        // streaming: K is read again by the quantisation, but not by this launch
        // (read through the caches, so that the second read might hit the
        // Infinity Cache, it measured 10% slower for both smooth_k prologues)
        const u32x4_t v =
            __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(base + static_cast<int64_t>(row) * p.sn));
        raw[j] = make_uint4(v.x, v.y, v.z, v.w);
      }
    }
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const uint32_t w[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float2_t f = unpack2<BF16>(w[q]);
        acc[2 * q] = acc[2 * q] + f.x;
        acc[2 * q + 1] = acc[2 * q + 1] + f.y;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) red[slot][cc * 8 + c] = acc[c];
  __syncthreads();
  if (t < D) {
    float sum = 0.0f;
#pragma unroll 8
    for (int r = 0; r < SLOTS; ++r) sum = sum + red[r][t];
    p.ws[(bh * p.nchunks + chunk) * D + t] = sum;
  }
}

template <bool BF16, int D>
__global__ __launch_bounds__(256) void k_mean_partial_kernel(MeanParams p) {
  k_mean_partial_block<BF16, D>(p, blockIdx.x);
}

// Stage 2: per (b, h) and 32-column group, the block stages the chunk sums in
// LDS (up to 256 chunks at a time, their loads issued together, so the launch
// waits about one memory latency per 256 chunks) and 32 threads add them in
// chunk order, one column each.  (One thread per (b, h, d) loading batches of
// 16 chunk sums waited one latency per batch: 6.4 us at S = 32891, 40 heads,
// against 4.7 us here.)
constexpr int kMeanCols = 32;
constexpr int kMeanStage = 256;

template <bool BF16, int D>
__global__ __launch_bounds__(256) void k_mean_final_kernel(MeanParams p) {
  constexpr int kGroups = D / kMeanCols;
  constexpr int kPerThread = kMeanStage * kMeanCols / 256;
  __shared__ float stage[kMeanStage * kMeanCols];
  const int t = threadIdx.x;
  const int64_t bh = blockIdx.x / kGroups;
  const int cgrp = static_cast<int>(blockIdx.x - bh * kGroups);
  const float* w = p.ws + bh * p.nchunks * D + cgrp * kMeanCols;
  float sum = 0.0f;
  for (int c0 = 0; c0 < p.nchunks; c0 += kMeanStage) {
    const int n = min(kMeanStage, p.nchunks - c0);
    float v[kPerThread];
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int e = t + i * 256;  // element (chunk e / 32, column e % 32) of this piece
      v[i] = (e < n * kMeanCols) ? w[static_cast<int64_t>(c0 + e / kMeanCols) * D + e % kMeanCols] : 0.0f;
    }
    __syncthreads();  // the previous piece has been summed
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) stage[t + i * 256] = v[i];
    __syncthreads();
    if (t < kMeanCols) {
      for (int c = 0; c < n; ++c) sum = sum + stage[c * kMeanCols + t];
    }
  }
  if (t < kMeanCols) {
    const float m = sum / static_cast<float>(p.s);
    uint16_t out;
    if constexpr (BF16) {
      out = static_cast<uint16_t>(pack_bf16x2(m, 0.0f) & 0xffffu);
    } else {
      out = static_cast<uint16_t>(pack_f16x2(m, 0.0f) & 0xffffu);
    }
    static_cast<uint16_t*>(p.mean)[bh * D + cgrp * kMeanCols + t] = out;
  }
}

// ------------------------------------------------------------------ V layout
constexpr int kVTile = 64;  // tokens per block (== SAGE_VT_ALIGN)

struct VLayoutParams {
  const void* v;
  uint16_t* vt;  // fp16 [B,H,D,NP]
  int64_t sb, sh, sn;
  int64_t np;
  int32_t h, s, ntiles;
};

// Block = (64-token tile, b*h).  Thread loads two consecutive tokens x 8
// channels (two 16-byte loads, whole rows per wave), interleaves them into
// token-pair dwords in LDS [D][32 pairs], then stores 8 consecutive tokens
// (16 bytes) per channel row of V_T.  bf16 -> fp16 conversion is fused.
template <bool BF16, int D>
__device__ __forceinline__ void v_layout_tile(const VLayoutParams& p, int64_t blk) {
  constexpr int CPR = D / 8;                        // chunks per token row
  constexpr int PAIRS = kVTile / 2;                 // token pairs per tile
  constexpr int LOAD_TASKS = PAIRS * CPR;           // (pair, chunk) tasks
  constexpr int LOADS = LOAD_TASKS / 256;
  constexpr int STORE_TASKS = D * (kVTile / 8);     // (channel, 8-token) tasks
  constexpr int STORES = STORE_TASKS / 256;
  // tile[channel][pair]: 32 dwords per channel row, the pair index XORed with
  // pswz(channel) (a multiple of 4, so each row's 16-byte groups stay whole
  // for the ds_read_b128 of the store phase).  A load-phase write instruction
  // covers channels 8cc + const of 16 chunks cc and 4 pairs: with pswz
  // keyed on cc % 8 they land on 32 distinct banks (2-way; an unswizzled row
  // pitch of 36 dwords put the 16 chunks on 2 banks, 8-way).
  constexpr int LSTRIDE = PAIRS;
  __shared__ __align__(16) uint32_t tile[D * LSTRIDE];
  auto pswz = [](int ch) { return ((ch >> 3) & 7) << 2; };

  const int t = threadIdx.x;
  const int64_t bh = blk / p.ntiles;
  const int tile_n = static_cast<int>(blk - bh * p.ntiles);
  const int64_t b = bh / p.h;
  const int64_t h = bh - b * p.h;
  const int n0 = tile_n * kVTile;
  const uint16_t* base = static_cast<const uint16_t*>(p.v) + b * p.sb + h * p.sh;

#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int task = t + i * 256;
    const int cc = task % CPR;
    const int pr = task / CPR;
    const int n = n0 + 2 * pr;
    uint4 a = make_uint4(0, 0, 0, 0), c = make_uint4(0, 0, 0, 0);
    // streaming: each V byte is read once (non-temporal)
    if (n < p.s) {
      const u32x4_t t0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(base + static_cast<int64_t>(n) * p.sn + cc * 8));
      a = make_uint4(t0.x, t0.y, t0.z, t0.w);
    }
    if (n + 1 < p.s) {
      const u32x4_t t1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(base + static_cast<int64_t>(n + 1) * p.sn + cc * 8));
      c = make_uint4(t1.x, t1.y, t1.z, t1.w);
    }
    const uint32_t wa[4] = {a.x, a.y, a.z, a.w};
    const uint32_t wc[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t lo, hi;  // lo: channels 2q of tokens (n, n+1); hi: channel 2q+1
      if constexpr (BF16) {
        const float2_t fa = unpack2<true>(wa[q]);
        const float2_t fc = unpack2<true>(wc[q]);
        lo = pack_f16x2(fa.x, fc.x);
        hi = pack_f16x2(fa.y, fc.y);
      } else {
        lo = (wa[q] & 0xffffu) | (wc[q] << 16);
        hi = (wa[q] >> 16) | (wc[q] & 0xffff0000u);
      }
      const int c0 = cc * 8 + 2 * q, c1 = c0 + 1;
      tile[c0 * LSTRIDE + (pr ^ pswz(c0))] = lo;
      tile[c1 * LSTRIDE + (pr ^ pswz(c1))] = hi;
    }
  }
  __syncthreads();
  uint16_t* out = p.vt + bh * D * p.np + n0;
#pragma unroll
  for (int i = 0; i < STORES; ++i) {
    const int task = t + i * 256;
    const int n8 = task % (kVTile / 8);
    const int d = task / (kVTile / 8);
    const uint4 w = *reinterpret_cast<const uint4*>(&tile[d * LSTRIDE + ((n8 * 4) ^ pswz(d))]);
    *reinterpret_cast<uint4*>(out + static_cast<int64_t>(d) * p.np + n8 * 8) = w;
  }
}

template <bool BF16, int D>
__global__ __launch_bounds__(256) void v_layout_kernel(VLayoutParams p) {
  v_layout_tile<BF16, D>(p, blockIdx.x);
}

// K quantisation and the V layout in one launch (the attention kernel
// quantises Q itself): blocks [0, quant_blocks) quantise four 32-token K units
// each, the others transform one 64-token V tile each.  Both halves are
// HBM-bound; one launch saves a launch and lets the two tails overlap.
template <bool BF16, int D>
__global__ __launch_bounds__(256) void prep_kv_kernel(QuantParams qp, VLayoutParams vp, int32_t quant_blocks) {
  if (static_cast<int32_t>(blockIdx.x) < quant_blocks) {
    quant_unit<BF16, D>(qp, static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6), threadIdx.x & (kWave - 1));
  } else {
    v_layout_tile<BF16, D>(vp, static_cast<int64_t>(blockIdx.x) - quant_blocks);
  }
}

// K mean, K quantisation and the V layout in two launches (smooth_k): the
// chunk sums of k_mean_partial_kernel, then prep_kv_mean_kernel, whose K
// blocks finish the mean themselves instead of a k_mean_final_kernel launch
// between the two.  A K block quantises four consecutive 32-token units of one
// head, one per wave, as prep_kv_kernel does.  Its first D threads add the
// head's chunk sums in chunk order, the additions of k_mean_final_kernel in the
// same order, so the block holds the same mean bit for bit (rounded to the
// input dtype), which it then subtracts in the quantisation.  The wave's K rows
// are loaded before that sum, so their latency overlaps it.  K blocks are
// spread evenly among the V-layout blocks (block i is K block j = floor(i *
// k_blocks / grid) when i is the first block of that j), so the sums' L2
// latency overlaps the V tiles' streaming.  Every K block of a head repeats
// the sum (nchunks * D * 4 bytes from L2 per 32 * D * 2 * 4 bytes of K: an
// eighth of them at S = 8192 with 1024-row chunks).  Measured on MI355X against
// the three launches (K mean's two, then prep_kv_kernel), rotating inputs: C3
// (B2 H32 S8192 D128) 107.0 / 106.7 us, C5 (B1 H40 S32891 D128) 256.7 / 256.1 us;
// eight units per K block (two per wave, so a twelfth of the sums) took 110.8 and
// 266 us, sixteen K-first 110 and 273 us, and the chunk sums with the V layout in
// the first launch and the K blocks alone in the second 116 and 298 us.
template <bool BF16, int D>
__device__ __forceinline__ void mean_k_block(const QuantParams& qp, const MeanParams& mp, int64_t kb,
                                             int32_t kb_per_head, float* smean) {
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & (kWave - 1);
  const int64_t bh = kb / kb_per_head;
  const int u = static_cast<int>(kb - bh * kb_per_head) * 4 + wave;
  // the wave's unit (n_units, i.e. none, past the head's last)
  QuantUnit<BF16, D> unit(qp, u < qp.k_units ? bh * qp.k_units + u : qp.n_units, lane);
  unit.load();
  if (t < D) {
    const float* w = mp.ws + bh * mp.nchunks * D + t;
    float sum = 0.0f;
    for (int c0 = 0; c0 < mp.nchunks; c0 += 32) {
      float v[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) v[i] = (c0 + i < mp.nchunks) ? w[static_cast<int64_t>(c0 + i) * D] : 0.0f;
      // past the last chunk v is +0, which leaves the sum's bits unchanged
      // (no chunk sum is -0: each starts from +0)
#pragma unroll
      for (int i = 0; i < 32; ++i) sum = sum + v[i];
    }
    const float m = sum / static_cast<float>(mp.s);
    const uint32_t bits = (BF16 ? pack_bf16x2(m, 0.0f) : pack_f16x2(m, 0.0f)) & 0xffffu;
    if (mp.mean != nullptr && kb - bh * kb_per_head == 0)
      static_cast<uint16_t*>(mp.mean)[bh * D + t] = static_cast<uint16_t>(bits);
    smean[t] = unpack2<BF16>(bits).x;
  }
  __syncthreads();
  float mean[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) mean[j] = smean[unit.cc * 8 + j];
  unit.quantise(mean, true, lane);
}

template <bool BF16, int D>
__global__ __launch_bounds__(256) void prep_kv_mean_kernel(QuantParams qp, MeanParams mp, VLayoutParams vp,
                                                           int32_t k_blocks, int32_t kb_per_head) {
  __shared__ float smean[D];
  const int64_t i = blockIdx.x;
  const int64_t total = gridDim.x;
  const int64_t j = i * k_blocks / total;
  if (i == (j * total + k_blocks - 1) / k_blocks) {
    mean_k_block<BF16, D>(qp, mp, j, kb_per_head, smean);
  } else {
    v_layout_tile<BF16, D>(vp, i - (j + 1));
  }
}

// ------------------------------------------------------------------ checks
int check_dtype(int dtype) {
  if (dtype != SAGE_DTYPE_F16 && dtype != SAGE_DTYPE_BF16)
    return set_error(SAGE_ERR_INVALID_ARG, "dtype must be SAGE_DTYPE_F16 or SAGE_DTYPE_BF16, got %d", dtype);
  return SAGE_OK;
}

int check_head_dim(int64_t d) {
  if (d != 64 && d != 128)
    return set_error(SAGE_ERR_UNSUPPORTED, "head_dim must be 64 or 128, got %lld", static_cast<long long>(d));
  return SAGE_OK;
}

int check_strides(const char* name, const void* ptr, int64_t sb, int64_t sh, int64_t sn) {
  if (!aligned(ptr, 16))
    return set_error(SAGE_ERR_ALIGNMENT, "%s: base pointer must be 16-byte aligned", name);
  if ((sb % 8) || (sh % 8) || (sn % 8))
    return set_error(SAGE_ERR_ALIGNMENT, "%s: strides (b=%lld, h=%lld, n=%lld) must be multiples of 8 elements",
                     name, static_cast<long long>(sb), static_cast<long long>(sh), static_cast<long long>(sn));
  return SAGE_OK;
}

}  // namespace
}  // namespace sage

using namespace sage;

extern "C" int sage_quant_qk_i8(const void* query, const void* key, const void* key_mean,
                                int8_t* q_i8, float* q_scale, int8_t* k_i8, float* k_scale, int dtype,
                                int64_t batch, int64_t q_heads, int64_t kv_heads,
                                int64_t q_len, int64_t kv_len, int64_t head_dim,
                                int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_n,
                                int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_n,
                                double sm_scale, void* stream) {
  clear_error();
  int rc;
  if ((rc = check_dtype(dtype)) || (rc = check_head_dim(head_dim))) return rc;
  if (batch < 0 || q_heads <= 0 || kv_heads <= 0 || q_len < 0 || kv_len < 0)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_quant_qk_i8: negative or zero size");
  if (q_len > INT32_MAX || kv_len > INT32_MAX || q_heads > INT32_MAX || kv_heads > INT32_MAX)
    return set_error(SAGE_ERR_UNSUPPORTED, "sage_quant_qk_i8: sizes beyond 32-bit limits");
  const bool do_q = batch > 0 && q_len > 0;
  const bool do_k = batch > 0 && kv_len > 0;
  if (do_q && (!query || !q_i8 || !q_scale))
    return set_error(SAGE_ERR_INVALID_ARG, "sage_quant_qk_i8: null query/q_i8/q_scale");
  if (do_k && (!key || !k_i8 || !k_scale))
    return set_error(SAGE_ERR_INVALID_ARG, "sage_quant_qk_i8: null key/k_i8/k_scale");
  if (do_q && ((rc = check_strides("query", query, q_stride_b, q_stride_h, q_stride_n)))) return rc;
  if (do_k && ((rc = check_strides("key", key, k_stride_b, k_stride_h, k_stride_n)))) return rc;
  if (do_k && key_mean && !aligned(key_mean, 16))
    return set_error(SAGE_ERR_ALIGNMENT, "key_mean: base pointer must be 16-byte aligned");
  if ((do_q && !aligned(q_i8, 8)) || (do_k && !aligned(k_i8, 8)) || (do_q && !aligned(q_scale, 4)) ||
      (do_k && !aligned(k_scale, 4)))
    return set_error(SAGE_ERR_ALIGNMENT, "sage_quant_qk_i8: int8 outputs need 8-byte, scales 4-byte alignment");

  QuantParams p;
  p.q = query;
  p.k = key;
  p.k_mean = key_mean;
  p.q8 = q_i8;
  p.q_scale = q_scale;
  p.k8 = k_i8;
  p.k_scale = k_scale;
  p.q_sb = q_stride_b;
  p.q_sh = q_stride_h;
  p.q_sn = q_stride_n;
  p.k_sb = k_stride_b;
  p.k_sh = k_stride_h;
  p.k_sn = k_stride_n;
  p.hq = static_cast<int32_t>(q_heads);
  p.hkv = static_cast<int32_t>(kv_heads);
  p.sq = static_cast<int32_t>(q_len);
  p.sk = static_cast<int32_t>(kv_len);
  p.q_units = static_cast<int32_t>(cdiv(q_len, 32));
  p.k_units = static_cast<int32_t>(cdiv(kv_len, 32));
  p.q_groups = static_cast<int32_t>(cdiv(q_len, kQGroup));
  p.k_groups = static_cast<int32_t>(cdiv(kv_len, kKGroup));
  p.n_q_units = do_q ? batch * q_heads * p.q_units : 0;
  p.n_units = p.n_q_units + (do_k ? batch * kv_heads * p.k_units : 0);
  p.s = static_cast<float>(sm_scale) * kLog2e;
  if (p.n_units == 0) return SAGE_OK;
  const int64_t blocks = cdiv(p.n_units, 4);
  if (blocks > INT32_MAX) return set_error(SAGE_ERR_UNSUPPORTED, "sage_quant_qk_i8: grid too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(blocks)), block(256);
  if (dtype == SAGE_DTYPE_BF16) {
    if (head_dim == 128) quant_qk_i8_kernel<true, 128><<<grid, block, 0, st>>>(p);
    else quant_qk_i8_kernel<true, 64><<<grid, block, 0, st>>>(p);
  } else {
    if (head_dim == 128) quant_qk_i8_kernel<false, 128><<<grid, block, 0, st>>>(p);
    else quant_qk_i8_kernel<false, 64><<<grid, block, 0, st>>>(p);
  }
  return check_launch("sage_quant_qk_i8");
}

extern "C" int64_t sage_k_mean_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim) {
  if (batch <= 0 || heads <= 0 || seq_len <= 0 || head_dim <= 0) return 0;
  return batch * heads * cdiv(seq_len, kMeanChunk) * head_dim * static_cast<int64_t>(sizeof(float));
}

extern "C" int sage_k_mean(const void* key, void* mean_out, void* workspace, int dtype,
                           int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                           int64_t stride_b, int64_t stride_h, int64_t stride_n, void* stream) {
  clear_error();
  int rc;
  if ((rc = check_dtype(dtype)) || (rc = check_head_dim(head_dim))) return rc;
  if (batch < 0 || heads <= 0 || seq_len < 0)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_k_mean: negative or zero size");
  if (batch == 0) return SAGE_OK;
  if (seq_len == 0)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_k_mean: mean over an empty sequence");
  if (seq_len > INT32_MAX || heads > INT32_MAX ||
      batch * heads * cdiv(seq_len, kMeanChunk) > INT32_MAX || batch * heads * (head_dim / kMeanCols) > INT32_MAX)
    return set_error(SAGE_ERR_UNSUPPORTED, "sage_k_mean: sizes beyond grid limits");
  if (!key || !mean_out || !workspace)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_k_mean: null key/mean_out/workspace");
  if ((rc = check_strides("key", key, stride_b, stride_h, stride_n))) return rc;
  if (!aligned(workspace, 4) || !aligned(mean_out, 2))
    return set_error(SAGE_ERR_ALIGNMENT, "sage_k_mean: misaligned workspace or output");
  MeanParams p;
  p.k = key;
  p.mean = mean_out;
  p.ws = static_cast<float*>(workspace);
  p.sb = stride_b;
  p.sh = stride_h;
  p.sn = stride_n;
  p.h = static_cast<int32_t>(heads);
  p.s = static_cast<int32_t>(seq_len);
  p.nchunks = static_cast<int32_t>(cdiv(seq_len, kMeanChunk));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 g1(static_cast<uint32_t>(batch * heads * p.nchunks));
  const dim3 g2(static_cast<uint32_t>(batch * heads * (head_dim / kMeanCols)));
  if (dtype == SAGE_DTYPE_BF16) {
    if (head_dim == 128) {
      k_mean_partial_kernel<true, 128><<<g1, 256, 0, st>>>(p);
      k_mean_final_kernel<true, 128><<<g2, 256, 0, st>>>(p);
    } else {
      k_mean_partial_kernel<true, 64><<<g1, 256, 0, st>>>(p);
      k_mean_final_kernel<true, 64><<<g2, 256, 0, st>>>(p);
    }
  } else {
    if (head_dim == 128) {
      k_mean_partial_kernel<false, 128><<<g1, 256, 0, st>>>(p);
      k_mean_final_kernel<false, 128><<<g2, 256, 0, st>>>(p);
    } else {
      k_mean_partial_kernel<false, 64><<<g1, 256, 0, st>>>(p);
      k_mean_final_kernel<false, 64><<<g2, 256, 0, st>>>(p);
    }
  }
  return check_launch("sage_k_mean");
}

extern "C" int64_t sage_v_layout_padded_len(int64_t seq_len) {
  if (seq_len <= 0) return 0;
  return cdiv(seq_len, SAGE_VT_ALIGN) * SAGE_VT_ALIGN;
}

extern "C" int sage_v_layout(const void* value, void* value_t, int dtype,
                             int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                             int64_t stride_b, int64_t stride_h, int64_t stride_n, void* stream) {
  clear_error();
  int rc;
  if ((rc = check_dtype(dtype)) || (rc = check_head_dim(head_dim))) return rc;
  if (batch < 0 || heads <= 0 || seq_len < 0)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_v_layout: negative or zero size");
  if (batch == 0 || seq_len == 0) return SAGE_OK;
  if (seq_len > INT32_MAX || heads > INT32_MAX ||
      batch * heads * (sage_v_layout_padded_len(seq_len) / kVTile) > INT32_MAX)
    return set_error(SAGE_ERR_UNSUPPORTED, "sage_v_layout: sizes beyond grid limits");
  if (!value || !value_t) return set_error(SAGE_ERR_INVALID_ARG, "sage_v_layout: null value/value_t");
  if ((rc = check_strides("value", value, stride_b, stride_h, stride_n))) return rc;
  if (!aligned(value_t, 16)) return set_error(SAGE_ERR_ALIGNMENT, "value_t: base pointer must be 16-byte aligned");
  VLayoutParams p;
  p.v = value;
  p.vt = static_cast<uint16_t*>(value_t);
  p.sb = stride_b;
  p.sh = stride_h;
  p.sn = stride_n;
  p.np = sage_v_layout_padded_len(seq_len);
  p.h = static_cast<int32_t>(heads);
  p.s = static_cast<int32_t>(seq_len);
  p.ntiles = static_cast<int32_t>(p.np / kVTile);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(batch * heads * p.ntiles));
  if (dtype == SAGE_DTYPE_BF16) {
    if (head_dim == 128) v_layout_kernel<true, 128><<<grid, 256, 0, st>>>(p);
    else v_layout_kernel<true, 64><<<grid, 256, 0, st>>>(p);
  } else {
    if (head_dim == 128) v_layout_kernel<false, 128><<<grid, 256, 0, st>>>(p);
    else v_layout_kernel<false, 64><<<grid, 256, 0, st>>>(p);
  }
  return check_launch("sage_v_layout");
}

extern "C" int sage_prep_kv_i8(const void* key, const void* value, const void* key_mean, int8_t* k_i8,
                               float* k_scale, void* value_t, int dtype, int64_t batch, int64_t kv_heads,
                               int64_t kv_len, int64_t head_dim, int64_t k_stride_b, int64_t k_stride_h,
                               int64_t k_stride_n, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_n,
                               void* stream) {
  clear_error();
  int rc;
  if ((rc = check_dtype(dtype)) || (rc = check_head_dim(head_dim))) return rc;
  if (batch < 0 || kv_heads <= 0 || kv_len < 0)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_prep_kv_i8: negative or zero size");
  if (batch == 0 || kv_len == 0) return SAGE_OK;
  if (kv_len > INT32_MAX || kv_heads > INT32_MAX ||
      batch * kv_heads * (sage_v_layout_padded_len(kv_len) / kVTile) > INT32_MAX / 2)
    return set_error(SAGE_ERR_UNSUPPORTED, "sage_prep_kv_i8: sizes beyond grid limits");
  if (!key || !value || !k_i8 || !k_scale || !value_t)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_prep_kv_i8: null key/value/k_i8/k_scale/value_t");
  if ((rc = check_strides("key", key, k_stride_b, k_stride_h, k_stride_n))) return rc;
  if ((rc = check_strides("value", value, v_stride_b, v_stride_h, v_stride_n))) return rc;
  if (key_mean && !aligned(key_mean, 16))
    return set_error(SAGE_ERR_ALIGNMENT, "key_mean: base pointer must be 16-byte aligned");
  if (!aligned(k_i8, 8) || !aligned(k_scale, 4) || !aligned(value_t, 16))
    return set_error(SAGE_ERR_ALIGNMENT,
                     "sage_prep_kv_i8: k_i8 needs 8-byte, k_scale 4-byte, value_t 16-byte alignment");
  QuantParams qp = {};
  qp.k = key;
  qp.k_mean = key_mean;
  qp.k8 = k_i8;
  qp.k_scale = k_scale;
  qp.k_sb = k_stride_b;
  qp.k_sh = k_stride_h;
  qp.k_sn = k_stride_n;
  qp.hq = 1;
  qp.hkv = static_cast<int32_t>(kv_heads);
  qp.sk = static_cast<int32_t>(kv_len);
  qp.k_units = static_cast<int32_t>(cdiv(kv_len, 32));
  qp.k_groups = static_cast<int32_t>(cdiv(kv_len, kKGroup));
  qp.n_q_units = 0;
  qp.n_units = batch * kv_heads * qp.k_units;
  qp.s = 1.0f;
  VLayoutParams vp;
  vp.v = value;
  vp.vt = static_cast<uint16_t*>(value_t);
  vp.sb = v_stride_b;
  vp.sh = v_stride_h;
  vp.sn = v_stride_n;
  vp.np = sage_v_layout_padded_len(kv_len);
  vp.h = static_cast<int32_t>(kv_heads);
  vp.s = static_cast<int32_t>(kv_len);
  vp.ntiles = static_cast<int32_t>(vp.np / kVTile);
  const int64_t quant_blocks = cdiv(qp.n_units, 4);
  const int64_t blocks = quant_blocks + batch * kv_heads * vp.ntiles;
  if (blocks > INT32_MAX) return set_error(SAGE_ERR_UNSUPPORTED, "sage_prep_kv_i8: grid too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(blocks)), block(256);
  const int32_t qb = static_cast<int32_t>(quant_blocks);
  if (dtype == SAGE_DTYPE_BF16) {
    if (head_dim == 128) prep_kv_kernel<true, 128><<<grid, block, 0, st>>>(qp, vp, qb);
    else prep_kv_kernel<true, 64><<<grid, block, 0, st>>>(qp, vp, qb);
  } else {
    if (head_dim == 128) prep_kv_kernel<false, 128><<<grid, block, 0, st>>>(qp, vp, qb);
    else prep_kv_kernel<false, 64><<<grid, block, 0, st>>>(qp, vp, qb);
  }
  return check_launch("sage_prep_kv_i8");
}

extern "C" int sage_prep_kv_i8_smooth(const void* key, const void* value, void* key_mean, void* workspace,
                                      int8_t* k_i8, float* k_scale, void* value_t, int dtype, int64_t batch,
                                      int64_t kv_heads, int64_t kv_len, int64_t head_dim, int64_t k_stride_b,
                                      int64_t k_stride_h, int64_t k_stride_n, int64_t v_stride_b,
                                      int64_t v_stride_h, int64_t v_stride_n, void* stream) {
  clear_error();
  int rc;
  if ((rc = check_dtype(dtype)) || (rc = check_head_dim(head_dim))) return rc;
  if (batch < 0 || kv_heads <= 0 || kv_len < 0)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_prep_kv_i8_smooth: negative or zero size");
  if (batch == 0 || kv_len == 0) return SAGE_OK;
  const int64_t nchunks = cdiv(kv_len, kMeanChunk);
  const int64_t units = cdiv(kv_len, 32);
  const int64_t kb_per_head = cdiv(units, 4);
  const int64_t k_blocks = batch * kv_heads * kb_per_head;
  const int64_t ntiles = sage_v_layout_padded_len(kv_len) / kVTile;
  if (kv_len > INT32_MAX || kv_heads > INT32_MAX || batch * kv_heads * nchunks > INT32_MAX ||
      k_blocks + batch * kv_heads * ntiles > INT32_MAX)
    return set_error(SAGE_ERR_UNSUPPORTED, "sage_prep_kv_i8_smooth: sizes beyond grid limits");
  if (!key || !value || !workspace || !k_i8 || !k_scale || !value_t)
    return set_error(SAGE_ERR_INVALID_ARG, "sage_prep_kv_i8_smooth: null key/value/workspace/k_i8/k_scale/value_t");
  if ((rc = check_strides("key", key, k_stride_b, k_stride_h, k_stride_n))) return rc;
  if ((rc = check_strides("value", value, v_stride_b, v_stride_h, v_stride_n))) return rc;
  if (!aligned(workspace, 4) || (key_mean && !aligned(key_mean, 2)))
    return set_error(SAGE_ERR_ALIGNMENT, "sage_prep_kv_i8_smooth: misaligned workspace or key_mean");
  if (!aligned(k_i8, 8) || !aligned(k_scale, 4) || !aligned(value_t, 16))
    return set_error(SAGE_ERR_ALIGNMENT,
                     "sage_prep_kv_i8_smooth: k_i8 needs 8-byte, k_scale 4-byte, value_t 16-byte alignment");
  MeanParams mp;
  mp.k = key;
  mp.mean = key_mean;
  mp.ws = static_cast<float*>(workspace);
  mp.sb = k_stride_b;
  mp.sh = k_stride_h;
  mp.sn = k_stride_n;
  mp.h = static_cast<int32_t>(kv_heads);
  mp.s = static_cast<int32_t>(kv_len);
  mp.nchunks = static_cast<int32_t>(nchunks);
  QuantParams qp = {};
  qp.k = key;
  qp.k8 = k_i8;
  qp.k_scale = k_scale;
  qp.k_sb = k_stride_b;
  qp.k_sh = k_stride_h;
  qp.k_sn = k_stride_n;
  qp.hq = 1;
  qp.hkv = static_cast<int32_t>(kv_heads);
  qp.sk = static_cast<int32_t>(kv_len);
  qp.k_units = static_cast<int32_t>(units);
  qp.k_groups = static_cast<int32_t>(cdiv(kv_len, kKGroup));
  qp.n_q_units = 0;
  qp.n_units = batch * kv_heads * units;
  qp.s = 1.0f;
  VLayoutParams vp;
  vp.v = value;
  vp.vt = static_cast<uint16_t*>(value_t);
  vp.sb = v_stride_b;
  vp.sh = v_stride_h;
  vp.sn = v_stride_n;
  vp.np = sage_v_layout_padded_len(kv_len);
  vp.h = static_cast<int32_t>(kv_heads);
  vp.s = static_cast<int32_t>(kv_len);
  vp.ntiles = static_cast<int32_t>(ntiles);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 g1(static_cast<uint32_t>(batch * kv_heads * nchunks));
  const dim3 g2(static_cast<uint32_t>(k_blocks + batch * kv_heads * ntiles));
  const int32_t kb = static_cast<int32_t>(k_blocks), kbh = static_cast<int32_t>(kb_per_head);
  if (dtype == SAGE_DTYPE_BF16) {
    if (head_dim == 128) {
      k_mean_partial_kernel<true, 128><<<g1, 256, 0, st>>>(mp);
      prep_kv_mean_kernel<true, 128><<<g2, 256, 0, st>>>(qp, mp, vp, kb, kbh);
    } else {
      k_mean_partial_kernel<true, 64><<<g1, 256, 0, st>>>(mp);
      prep_kv_mean_kernel<true, 64><<<g2, 256, 0, st>>>(qp, mp, vp, kb, kbh);
    }
  } else {
    if (head_dim == 128) {
      k_mean_partial_kernel<false, 128><<<g1, 256, 0, st>>>(mp);
      prep_kv_mean_kernel<false, 128><<<g2, 256, 0, st>>>(qp, mp, vp, kb, kbh);
    } else {
      k_mean_partial_kernel<false, 64><<<g1, 256, 0, st>>>(mp);
      prep_kv_mean_kernel<false, 64><<<g2, 256, 0, st>>>(qp, mp, vp, kb, kbh);
    }
  }
  return check_launch("sage_prep_kv_i8_smooth");
}
