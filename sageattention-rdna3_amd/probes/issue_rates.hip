// Issue-rate probe for gfx950: what one SIMD sustains for the instruction mix
// of the attention kernel's key loop, with 1-4 waves per SIMD.
//
// Build and run (no arguments):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       sageattention-rdna3_amd/probes/issue_rates.hip -o issue_rates && ./issue_rates
//
// Every kernel runs one 256*W-thread block per CU (W waves per SIMD) and times
// each wave's loop with s_memtime; a block's time is its span (first wave's
// start to last wave's end), so waves that share a SIMD are charged for each
// other (a per-wave average would not be: waves of one SIMD need not overlap
// in time).  The instruction streams are fixed with inline asm, on independent
// registers (no dependency stalls).  Results are cycles of s_memtime per
// instruction (single kinds) or per unit (mixes), per SIMD.  The first lines
// calibrate s_memtime against the 100 MHz s_memrealtime, once on an idle chip
// and once while every CU runs MFMAs.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <vector>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// kinds: the instructions of one loop iteration ("unit")
enum Kind {
  kMfmaF16 = 0,  // 4 x v_mfma_f32_32x32x16_f16 (the P.V MFMA)
  kMfmaI8,       // 4 x v_mfma_i32_32x32x32_i8 (the QK MFMA)
  kFma,          // 24 x v_fma_f32
  kExp,          // 24 x v_exp_f32
  kMix,          // 4 MFMA f16 + 22 fma + 6 exp: the key loop's ratio (24 MFMA : 135 VALU : 33 exp)
  kLds,          // 4 x ds_read_b128 (16 bytes per lane, consecutive lanes 16 bytes apart), 3 in flight
  kMixLds,       // kMix with each MFMA's A operand read from LDS two MFMAs ahead, as the key loop reads K and V
  kRoles,        // the same work as kMix split by role: waves 0-3 of the block issue only the MFMAs (8 per
                 // iteration), waves 4+ (sharing the SIMDs) only the VALU part (44 fma + 12 exp per iteration)
  kMfmaF16Acc,   // kMfmaF16 with the accumulators in AGPRs
  kMixAcc,       // kMix with the MFMA accumulators in AGPRs
  kMixHalf,      // 4 MFMA f16 + 11 fma + 3 exp: half the VALU of kMix
  kMixFma,       // 4 MFMA f16 + 22 fma: kMix without its exponentials
  kMfma16,       // 4 x v_mfma_f32_16x16x32_f16 (half the work of the 32x32x16 MFMA each)
  kMix16,        // 8 x v_mfma_f32_16x16x32_f16 + 22 fma + 6 exp: kMix's work with the 16x16 MFMA shape
  kExpF16,       // 24 x v_exp_f16
  kMix2,         // 2 MFMA f16 + 22 fma + 6 exp: the D = 64 key loop's ratio (12 MFMA : 135 VALU : 33 exp)
  kMfmaDep,      // 4 x v_mfma_f32_32x32x16_f16 on one accumulator (each reads the previous result)
  kMixSalu,      // kMix + 12 s_add_u32 (the key loop issues ~11 SALU per 4 MFMAs)
  kKinds
};
constexpr int kUnitOps[kKinds] = {4, 4, 24, 24, 4, 4, 4, 4, 4, 4, 4, 4, 4, 8, 24, 2, 4, 4};
const char* kNames[kKinds] = {"v_mfma_f32_32x32x16_f16", "v_mfma_i32_32x32x32_i8", "v_fma_f32", "v_exp_f32",
                              "mix: 4 MFMA f16 + 22 fma + 6 exp", "ds_read_b128", "mix + 4 ds_read_b128 operands",
                              "mix work split: MFMA waves + VALU waves",
                              "v_mfma_f32_32x32x16_f16, AGPR acc", "mix, MFMA accumulators in AGPRs",
                              "4 MFMA f16 + 11 fma + 3 exp", "4 MFMA f16 + 22 fma", "v_mfma_f32_16x16x32_f16",
                              "8 MFMA 16x16x32 + 22 fma + 6 exp", "v_exp_f16",
                              "2 MFMA f16 + 22 fma + 6 exp", "v_mfma_f32_32x32x16_f16, one chain", "mix + 12 SALU"};

#define FMA4 "v_fma_f32 %4, %4, %12, %13\n v_fma_f32 %5, %5, %12, %13\n v_fma_f32 %6, %6, %12, %13\n v_fma_f32 %7, %7, %12, %13\n"
#define FMA2 "v_fma_f32 %8, %8, %12, %13\n v_fma_f32 %9, %9, %12, %13\n"
#define EXP2 "v_exp_f32 %10, %10\n v_exp_f32 %11, %11\n"
#define OPERANDS                                                                                                 \
  : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3), "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5), "+v"(x6), \
    "+v"(x7)                                                                                                     \
  : "v"(m), "v"(k), "v"(a), "v"(b)

template <int KIND>
__global__ __launch_bounds__(1024) void unit_loop(int iters, unsigned long long* t, float* sink) {
  __shared__ __align__(16) char lds[64 << 10];
  if constexpr (KIND == kLds || KIND == kMixLds) {
    for (int i = threadIdx.x; i < (64 << 10) / 4; i += blockDim.x) reinterpret_cast<float*>(lds)[i] = 0.001f * i;
  }
  // wave w reads its own 1 KB rows: lane l at byte 16 l (64 lanes x 16 bytes, no bank conflicts); `lds` is
  // the kernel's only LDS variable, at LDS address 0
  const unsigned addr = (threadIdx.x & 63) * 16 + ((threadIdx.x >> 6) & 7) * 1024;
  f16x8 a, b, a1, a2;
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<_Float16>(threadIdx.x * 0.001f + i);
    b[i] = static_cast<_Float16>(i * 0.5f);
  }
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  i32x16 d0 = {}, d1 = {}, d2 = {}, d3 = {};
  f32x4 e0 = {}, e1 = {}, e2 = {}, e3 = {};
  _Float16 h0 = static_cast<_Float16>(threadIdx.x & 7), h1 = h0 + static_cast<_Float16>(1), h2 = -h0, h3 = -h1,
           h4 = h0 * static_cast<_Float16>(0.5f), h5 = h1 * static_cast<_Float16>(0.25f);
  const i32x4 ia = {static_cast<int>(threadIdx.x), 1, 2, 3}, ib = {5, 6, 7, 8};
  float x0 = threadIdx.x, x1 = x0 + 1, x2 = x0 + 2, x3 = x0 + 3, x4 = x0 + 4, x5 = x0 + 5, x6 = -1.0f, x7 = -2.0f;
  const float m = 0.999f, k = 0.001f;
  a1 = a;
  a2 = b;
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
    if constexpr (KIND == kMfmaF16) {
      asm volatile(
          "v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n v_mfma_f32_32x32x16_f16 %1, %4, %5, %1\n"
          "v_mfma_f32_32x32x16_f16 %2, %4, %5, %2\n v_mfma_f32_32x32x16_f16 %3, %4, %5, %3\n"
          : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3)
          : "v"(a), "v"(b));
    } else if constexpr (KIND == kMfmaF16Acc) {
      asm volatile(
          "v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n v_mfma_f32_32x32x16_f16 %1, %4, %5, %1\n"
          "v_mfma_f32_32x32x16_f16 %2, %4, %5, %2\n v_mfma_f32_32x32x16_f16 %3, %4, %5, %3\n"
          : "+a"(c0), "+a"(c1), "+a"(c2), "+a"(c3)
          : "v"(a), "v"(b));
    } else if constexpr (KIND == kMixAcc) {
      asm volatile(
          "v_mfma_f32_32x32x16_f16 %0, %14, %15, %0\n" FMA4 "v_fma_f32 %8, %8, %12, %13\n" EXP2
          "v_mfma_f32_32x32x16_f16 %1, %14, %15, %1\n" FMA4 FMA2 "v_exp_f32 %10, %10\n"
          "v_mfma_f32_32x32x16_f16 %2, %14, %15, %2\n" FMA4 "v_fma_f32 %9, %9, %12, %13\n" EXP2
          "v_mfma_f32_32x32x16_f16 %3, %14, %15, %3\n" FMA4 FMA2 "v_exp_f32 %11, %11\n"
          : "+a"(c0), "+a"(c1), "+a"(c2), "+a"(c3), "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5),
            "+v"(x6), "+v"(x7)
          : "v"(m), "v"(k), "v"(a), "v"(b));
    } else if constexpr (KIND == kMixHalf) {
      asm volatile(
          "v_mfma_f32_32x32x16_f16 %0, %14, %15, %0\n" FMA2 "v_exp_f32 %10, %10\n"
          "v_mfma_f32_32x32x16_f16 %1, %14, %15, %1\n" FMA4 "v_fma_f32 %8, %8, %12, %13\n"
          "v_mfma_f32_32x32x16_f16 %2, %14, %15, %2\n" FMA2 "v_exp_f32 %11, %11\n"
          "v_mfma_f32_32x32x16_f16 %3, %14, %15, %3\n" "v_fma_f32 %9, %9, %12, %13\n v_fma_f32 %4, %4, %12, %13\n"
          "v_exp_f32 %10, %10\n" OPERANDS);
    } else if constexpr (KIND == kMixFma) {
      asm volatile(
          "v_mfma_f32_32x32x16_f16 %0, %14, %15, %0\n" FMA4 "v_fma_f32 %8, %8, %12, %13\n"
          "v_mfma_f32_32x32x16_f16 %1, %14, %15, %1\n" FMA4 FMA2
          "v_mfma_f32_32x32x16_f16 %2, %14, %15, %2\n" FMA4 "v_fma_f32 %9, %9, %12, %13\n"
          "v_mfma_f32_32x32x16_f16 %3, %14, %15, %3\n" FMA4 FMA2 OPERANDS);
    } else if constexpr (KIND == kMfma16) {
      asm volatile(
          "v_mfma_f32_16x16x32_f16 %0, %4, %5, %0\n v_mfma_f32_16x16x32_f16 %1, %4, %5, %1\n"
          "v_mfma_f32_16x16x32_f16 %2, %4, %5, %2\n v_mfma_f32_16x16x32_f16 %3, %4, %5, %3\n"
          : "+v"(e0), "+v"(e1), "+v"(e2), "+v"(e3)
          : "v"(a), "v"(b));
    } else if constexpr (KIND == kMix16) {
      asm volatile(
          "v_mfma_f32_16x16x32_f16 %0, %14, %15, %0\n" FMA4 "v_mfma_f32_16x16x32_f16 %1, %14, %15, %1\n"
          "v_fma_f32 %8, %8, %12, %13\n" EXP2
          "v_mfma_f32_16x16x32_f16 %2, %14, %15, %2\n" FMA4 "v_mfma_f32_16x16x32_f16 %3, %14, %15, %3\n"
          FMA2 "v_exp_f32 %10, %10\n"
          "v_mfma_f32_16x16x32_f16 %0, %14, %15, %0\n" FMA4 "v_mfma_f32_16x16x32_f16 %1, %14, %15, %1\n"
          "v_fma_f32 %9, %9, %12, %13\n" EXP2
          "v_mfma_f32_16x16x32_f16 %2, %14, %15, %2\n" FMA4 "v_mfma_f32_16x16x32_f16 %3, %14, %15, %3\n"
          FMA2 "v_exp_f32 %11, %11\n"
          : "+v"(e0), "+v"(e1), "+v"(e2), "+v"(e3), "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5),
            "+v"(x6), "+v"(x7)
          : "v"(m), "v"(k), "v"(a), "v"(b));
    } else if constexpr (KIND == kExpF16) {
      asm volatile(
          "v_exp_f16 %0, %0\n v_exp_f16 %1, %1\n v_exp_f16 %2, %2\n v_exp_f16 %3, %3\n v_exp_f16 %4, %4\n"
          "v_exp_f16 %5, %5\n v_exp_f16 %0, %0\n v_exp_f16 %1, %1\n v_exp_f16 %2, %2\n v_exp_f16 %3, %3\n"
          "v_exp_f16 %4, %4\n v_exp_f16 %5, %5\n v_exp_f16 %0, %0\n v_exp_f16 %1, %1\n v_exp_f16 %2, %2\n"
          "v_exp_f16 %3, %3\n v_exp_f16 %4, %4\n v_exp_f16 %5, %5\n v_exp_f16 %0, %0\n v_exp_f16 %1, %1\n"
          "v_exp_f16 %2, %2\n v_exp_f16 %3, %3\n v_exp_f16 %4, %4\n v_exp_f16 %5, %5\n"
          : "+v"(h0), "+v"(h1), "+v"(h2), "+v"(h3), "+v"(h4), "+v"(h5));
    } else if constexpr (KIND == kMix2) {
      asm volatile(
          "v_mfma_f32_32x32x16_f16 %0, %14, %15, %0\n" FMA4 "v_fma_f32 %8, %8, %12, %13\n" EXP2
          FMA4 FMA2 "v_exp_f32 %10, %10\n"
          "v_mfma_f32_32x32x16_f16 %1, %14, %15, %1\n" FMA4 "v_fma_f32 %9, %9, %12, %13\n" EXP2
          FMA4 FMA2 "v_exp_f32 %11, %11\n" OPERANDS);
    } else if constexpr (KIND == kMfmaDep) {
      asm volatile(
          "v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n"
          "v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n"
          : "+v"(c0)
          : "v"(a), "v"(b));
    } else if constexpr (KIND == kMixSalu) {
      asm volatile(
          "v_mfma_f32_32x32x16_f16 %0, %14, %15, %0\n" FMA4 "s_add_u32 s90, s90, 1\n s_add_u32 s91, s91, 3\n"
          "v_fma_f32 %8, %8, %12, %13\n s_add_u32 s90, s90, 5\n" EXP2
          "v_mfma_f32_32x32x16_f16 %1, %14, %15, %1\n" FMA4 "s_add_u32 s91, s91, 1\n s_add_u32 s90, s90, 3\n"
          FMA2 "s_add_u32 s91, s91, 5\n v_exp_f32 %10, %10\n"
          "v_mfma_f32_32x32x16_f16 %2, %14, %15, %2\n" FMA4 "s_add_u32 s90, s90, 1\n s_add_u32 s91, s91, 3\n"
          "v_fma_f32 %9, %9, %12, %13\n s_add_u32 s90, s90, 5\n" EXP2
          "v_mfma_f32_32x32x16_f16 %3, %14, %15, %3\n" FMA4 "s_add_u32 s91, s91, 1\n s_add_u32 s90, s90, 3\n"
          FMA2 "s_add_u32 s91, s91, 5\n v_exp_f32 %11, %11\n"
          : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3), "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5),
            "+v"(x6), "+v"(x7)
          : "v"(m), "v"(k), "v"(a), "v"(b)
          : "s90", "s91", "scc");
    } else if constexpr (KIND == kMfmaI8) {
      asm volatile(
          "v_mfma_i32_32x32x32_i8 %0, %4, %5, %0\n v_mfma_i32_32x32x32_i8 %1, %4, %5, %1\n"
          "v_mfma_i32_32x32x32_i8 %2, %4, %5, %2\n v_mfma_i32_32x32x32_i8 %3, %4, %5, %3\n"
          : "+v"(d0), "+v"(d1), "+v"(d2), "+v"(d3)
          : "v"(ia), "v"(ib));
    } else if constexpr (KIND == kFma) {
      asm volatile(FMA4 FMA4 FMA4 FMA4 FMA4 FMA2 FMA2 OPERANDS);
    } else if constexpr (KIND == kExp) {
      asm volatile(EXP2 "v_exp_f32 %4, %4\n v_exp_f32 %5, %5\n v_exp_f32 %6, %6\n v_exp_f32 %7, %7\n"
                   "v_exp_f32 %8, %8\n v_exp_f32 %9, %9\n" EXP2
                   "v_exp_f32 %4, %4\n v_exp_f32 %5, %5\n v_exp_f32 %6, %6\n v_exp_f32 %7, %7\n"
                   "v_exp_f32 %8, %8\n v_exp_f32 %9, %9\n" EXP2 EXP2
                   "v_exp_f32 %4, %4\n v_exp_f32 %5, %5\n v_exp_f32 %6, %6\n v_exp_f32 %7, %7\n" OPERANDS);
    } else if constexpr (KIND == kRoles) {
      if (threadIdx.x < 256) {
        asm volatile(
            "v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n v_mfma_f32_32x32x16_f16 %1, %4, %5, %1\n"
            "v_mfma_f32_32x32x16_f16 %2, %4, %5, %2\n v_mfma_f32_32x32x16_f16 %3, %4, %5, %3\n"
            "v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n v_mfma_f32_32x32x16_f16 %1, %4, %5, %1\n"
            "v_mfma_f32_32x32x16_f16 %2, %4, %5, %2\n v_mfma_f32_32x32x16_f16 %3, %4, %5, %3\n"
            : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3)
            : "v"(a), "v"(b));
      } else {
        asm volatile(FMA4 "v_fma_f32 %8, %8, %12, %13\n" EXP2 FMA4 FMA2 "v_exp_f32 %10, %10\n"
                     FMA4 "v_fma_f32 %9, %9, %12, %13\n" EXP2 FMA4 FMA2 "v_exp_f32 %11, %11\n"
                     FMA4 "v_fma_f32 %8, %8, %12, %13\n" EXP2 FMA4 FMA2 "v_exp_f32 %10, %10\n"
                     FMA4 "v_fma_f32 %9, %9, %12, %13\n" EXP2 FMA4 FMA2 "v_exp_f32 %11, %11\n" OPERANDS);
      }
    } else if constexpr (KIND == kLds) {
      asm volatile(
          "ds_read_b128 %0, %3 offset:0\n ds_read_b128 %1, %3 offset:8192\n ds_read_b128 %2, %3 offset:16384\n"
          "s_waitcnt lgkmcnt(2)\n ds_read_b128 %0, %3 offset:24576\n s_waitcnt lgkmcnt(2)\n"
          "s_waitcnt lgkmcnt(0)\n"
          : "+v"(a), "+v"(a1), "+v"(a2)
          : "v"(addr));
    } else if constexpr (KIND == kMixLds) {
#define LFMA4 "v_fma_f32 %4, %4, %15, %16\n v_fma_f32 %5, %5, %15, %16\n v_fma_f32 %6, %6, %15, %16\n v_fma_f32 %7, %7, %15, %16\n"
#define LFMA2 "v_fma_f32 %8, %8, %15, %16\n v_fma_f32 %9, %9, %15, %16\n"
#define LEXP2 "v_exp_f32 %10, %10\n v_exp_f32 %11, %11\n"
      // ring of 3 operand registers (%12 %13 %14): the read for MFMA i+2 is issued before MFMA i
      asm volatile(
          "ds_read_b128 %14, %17 offset:0\n s_waitcnt lgkmcnt(2)\n"
          "v_mfma_f32_32x32x16_f16 %0, %12, %18, %0\n" LFMA4 "v_fma_f32 %8, %8, %15, %16\n" LEXP2
          "ds_read_b128 %12, %17 offset:16384\n s_waitcnt lgkmcnt(2)\n"
          "v_mfma_f32_32x32x16_f16 %1, %13, %18, %1\n" LFMA4 LFMA2 "v_exp_f32 %10, %10\n"
          "ds_read_b128 %13, %17 offset:32768\n s_waitcnt lgkmcnt(2)\n"
          "v_mfma_f32_32x32x16_f16 %2, %14, %18, %2\n" LFMA4 "v_fma_f32 %9, %9, %15, %16\n" LEXP2
          "ds_read_b128 %14, %17 offset:49152\n s_waitcnt lgkmcnt(2)\n"
          "v_mfma_f32_32x32x16_f16 %3, %12, %18, %3\n" LFMA4 LFMA2 "v_exp_f32 %11, %11\n"
          : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3), "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5),
            "+v"(x6), "+v"(x7), "+v"(a), "+v"(a1), "+v"(a2)
          : "v"(m), "v"(k), "v"(addr), "v"(b));
    } else {
      asm volatile(
          "v_mfma_f32_32x32x16_f16 %0, %14, %15, %0\n" FMA4 "v_fma_f32 %8, %8, %12, %13\n" EXP2
          "v_mfma_f32_32x32x16_f16 %1, %14, %15, %1\n" FMA4 FMA2 "v_exp_f32 %10, %10\n"
          "v_mfma_f32_32x32x16_f16 %2, %14, %15, %2\n" FMA4 "v_fma_f32 %9, %9, %12, %13\n" EXP2
          "v_mfma_f32_32x32x16_f16 %3, %14, %15, %3\n" FMA4 FMA2 "v_exp_f32 %11, %11\n" OPERANDS);
    }
  }
  if constexpr (KIND == kMixLds) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float s = x0 + x1 + x2 + x3 + x4 + x5 + x6 + x7 + static_cast<float>(a[0] + a1[1] + a2[2]);
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i] + static_cast<float>(d0[i] + d1[i] + d2[i] + d3[i]);
  for (int i = 0; i < 4; ++i) s += e0[i] + e1[i] + e2[i] + e3[i];
  s += static_cast<float>(h0 + h1 + h2 + h3 + h4 + h5);
  sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
  if ((threadIdx.x & 63) == 0) {
    const int w = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    t[2 * w] = t0;
    t[2 * w + 1] = t1;
  }
}

// s_memtime and s_memrealtime (100 MHz) deltas of wave 0 of every block around
// `iters` units of f16 MFMAs
__global__ __launch_bounds__(256) void clock_pair(int iters, unsigned long long* out, float* sink) {
  f16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<_Float16>(threadIdx.x * 0.001f + i);
    b[i] = static_cast<_Float16>(i * 0.5f);
  }
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  const unsigned long long m0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
    asm volatile(
        "v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n v_mfma_f32_32x32x16_f16 %1, %4, %5, %1\n"
        "v_mfma_f32_32x32x16_f16 %2, %4, %5, %2\n v_mfma_f32_32x32x16_f16 %3, %4, %5, %3\n"
        : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3)
        : "v"(a), "v"(b));
  }
  const unsigned long long m1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0;
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
  sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (threadIdx.x == 0) {
    out[2 * blockIdx.x] = m1 - m0;
    out[2 * blockIdx.x + 1] = r1 - r0;
  }
}

static bool per_unit_kind(int kind) {
  return kind == kMix || kind == kMixLds || kind == kMixAcc || kind == kMixHalf || kind == kMixFma || kind == kMix16 ||
         kind == kMix2 || kind == kMixSalu;
}

#define CHECK(x)                                                      \
  do {                                                                \
    if ((x) != hipSuccess) {                                          \
      fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(x)); \
      return 1;                                                       \
    }                                                                 \
  } while (0)

int main() {
  int dev = 0, cus = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int iters = 400;
  unsigned long long* t = nullptr;
  float* sink = nullptr;
  CHECK(hipMalloc(&t, static_cast<size_t>(cus) * 16 * 2 * sizeof(unsigned long long)));
  CHECK(hipMalloc(&sink, static_cast<size_t>(cus) * 1024 * sizeof(float)));

  // s_memtime rate: a lone wave on an idle chip, then every CU's wave 0 under MFMA load
  for (int load = 0; load < 2; ++load) {
    const int blocks = load ? cus : 1, n = load ? 200000 : 20000;
    clock_pair<<<blocks, 256>>>(n, t, sink);
    CHECK(hipDeviceSynchronize());
    std::vector<unsigned long long> h(2 * blocks);
    CHECK(hipMemcpy(h.data(), t, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost));
    double mt = 0, rt = 0;
    for (int i = 0; i < blocks; ++i) {
      mt += h[2 * i];
      rt += h[2 * i + 1];
    }
    printf("s_memtime rate %s: %.1f MHz (%.0f ticks per 100 MHz s_memrealtime tick x 100)\n",
           load ? "with every CU running MFMAs" : "one wave, idle chip", 100.0 * mt / rt, mt / rt);
  }

  printf("\n%-36s %s\n", "kind (per SIMD, s_memtime cycles)", "W=1      W=2      W=3      W=4 waves per SIMD");
  double unit[kKinds][5] = {};
  for (int kind = 0; kind < kKinds; ++kind) {
    printf("%-36s", kNames[kind]);
    for (int W = 1; W <= 4; ++W) {
      const int nw = 4 * W;
      auto launch = [&]() {
        switch (kind) {
          case kMfmaF16: unit_loop<kMfmaF16><<<cus, 256 * W>>>(iters, t, sink); break;
          case kMfmaI8: unit_loop<kMfmaI8><<<cus, 256 * W>>>(iters, t, sink); break;
          case kFma: unit_loop<kFma><<<cus, 256 * W>>>(iters, t, sink); break;
          case kExp: unit_loop<kExp><<<cus, 256 * W>>>(iters, t, sink); break;
          case kLds: unit_loop<kLds><<<cus, 256 * W>>>(iters, t, sink); break;
          case kMixLds: unit_loop<kMixLds><<<cus, 256 * W>>>(iters, t, sink); break;
          case kRoles: unit_loop<kRoles><<<cus, 256 * W>>>(iters, t, sink); break;
          case kMfmaF16Acc: unit_loop<kMfmaF16Acc><<<cus, 256 * W>>>(iters, t, sink); break;
          case kMixAcc: unit_loop<kMixAcc><<<cus, 256 * W>>>(iters, t, sink); break;
          case kMixHalf: unit_loop<kMixHalf><<<cus, 256 * W>>>(iters, t, sink); break;
          case kMixFma: unit_loop<kMixFma><<<cus, 256 * W>>>(iters, t, sink); break;
          case kMfma16: unit_loop<kMfma16><<<cus, 256 * W>>>(iters, t, sink); break;
          case kMix16: unit_loop<kMix16><<<cus, 256 * W>>>(iters, t, sink); break;
          case kExpF16: unit_loop<kExpF16><<<cus, 256 * W>>>(iters, t, sink); break;
          case kMix2: unit_loop<kMix2><<<cus, 256 * W>>>(iters, t, sink); break;
          case kMfmaDep: unit_loop<kMfmaDep><<<cus, 256 * W>>>(iters, t, sink); break;
          case kMixSalu: unit_loop<kMixSalu><<<cus, 256 * W>>>(iters, t, sink); break;
          default: unit_loop<kMix><<<cus, 256 * W>>>(iters, t, sink); break;
        }
      };
      launch();  // warm
      launch();
      CHECK(hipDeviceSynchronize());
      std::vector<unsigned long long> h(static_cast<size_t>(cus) * nw * 2);
      CHECK(hipMemcpy(h.data(), t, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost));
      double span = 0;
      for (int bl = 0; bl < cus; ++bl) {
        unsigned long long lo = ~0ull, hi = 0;
        for (int w = 0; w < nw; ++w) {
          lo = h[2 * (bl * nw + w)] < lo ? h[2 * (bl * nw + w)] : lo;
          hi = h[2 * (bl * nw + w) + 1] > hi ? h[2 * (bl * nw + w) + 1] : hi;
        }
        span += static_cast<double>(hi - lo);
      }
      span /= cus;
      // per SIMD: W waves x iters units in `span`
      // kRoles: per iteration a SIMD runs 2 units of MFMA work (its MFMA wave) and 2(W-1) units of VALU work;
      // charged per unit of mix work, i.e. per 2 units at W=2 (the balanced case)
      const double per_unit = kind == kRoles ? span / (static_cast<double>(iters) * 2)
                                             : span / (static_cast<double>(iters) * W);
      unit[kind][W] = per_unit;
      const bool per_u = kind == kRoles || per_unit_kind(kind);
      printf(" %7.2f", per_u ? per_unit : per_unit / kUnitOps[kind]);
    }
    printf("   %s\n", kind == kRoles ? "(per unit of MFMA work; W=2 is the balanced 1:1 split)"
                     : per_unit_kind(kind) ? "(per unit)" : "(per instruction)");
    if (kind == kLds) {
      // per SIMD, one wave's unit (4 KB) per per_unit cycles; 4 SIMDs per CU
      printf("%-36s", "  = LDS bytes read per clock per CU");
      for (int W = 1; W <= 4; ++W) printf(" %7.1f", 4.0 * 4096.0 / unit[kLds][W]);
      printf("\n");
    }
  }
  printf("\nmix unit against its parts (4 MFMA f16 + 22 fma + 6 exp, each part timed alone at the same W):\n");
  for (int W = 1; W <= 4; ++W) {
    const double mf = unit[kMfmaF16][W];
    const double va = unit[kFma][W] / kUnitOps[kFma] * 22 + unit[kExp][W] / kUnitOps[kExp] * 6;
    const double mix = unit[kMix][W];
    const double hidden = (mf + va - mix) / (mf < va ? mf : va);
    printf("  W=%d: MFMA %.1f + VALU %.1f = %.1f serial, %.1f ideal overlap; measured %.1f (%.0f%% of the smaller part "
           "hidden)\n", W, mf, va, mf + va, mf > va ? mf : va, mix, 100.0 * hidden);
  }
  CHECK(hipFree(t));
  CHECK(hipFree(sink));
  return 0;
}
