// Shared device/host helpers for the gfx950 (CDNA4) kernels of the quantized-GEMM path.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <atomic>
#include <stdint.h>

#include "../../include/ferret_hip.h"

namespace ferret {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// Compile-time integer as a value (for generic lambdas over tile shapes).
template <int V>
struct IntC {
  static constexpr int value = V;
};

// f(IntC<0>{}), ..., f(IntC<N-1>{}) in order.
template <int I, int N, typename Fn>
__device__ __forceinline__ void static_for(Fn&& f) {
  if constexpr (I < N) {
    f(IntC<I>{});
    static_for<I + 1, N>(f);
  }
}

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float -> bf16 (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 h = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v;
  v[0] = static_cast<__bf16>(lo);
  v[1] = static_cast<__bf16>(hi);
  return __builtin_bit_cast(uint32_t, v);
}

// ---------------------------------------------------------------- MFMA wrappers

// D(16x16 f32) += A(16x32 bf16) * B(32x16 bf16). Lane l: A row / B col = l%16,
// K elements 8*(l/16)..+8 of the instruction's 32; D rows 4*(l/16)+i, col l%16.
__device__ __forceinline__ f32x4 mfma_bf16_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// D(16x16 f32) = A(16x128 e4m3) * B(128x16 e4m3) (+ C). Operand formats 0 = OCP
// e4m3 for both; scale operands 0 select the unscaled instruction.
__device__ __forceinline__ f32x4 mfma_fp8_16x16x128(i32x8 a, i32x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// 8 OCP e4m3 bytes (two dwords, byte i = element i) -> 8 bf16, exact
// (v_cvt_scalef32_pk_bf16_fp8 with scale 1.0; every e4m3 value is a bf16 value).
// Built with vector shuffles so the four results land in the MFMA operand
// registers directly.
__device__ __forceinline__ bf16x8 e4m3x8_to_bf16x8(uint32_t w0, uint32_t w1) {
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
  const bf16x4 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3);
  const bf16x4 cd = __builtin_shufflevector(c, d, 0, 1, 2, 3);
  return __builtin_shufflevector(ab, cd, 0, 1, 2, 3, 4, 5, 6, 7);
}

// The same, each value multiplied by 2^(e - 127) for the biased exponent e of
// `scale` (the instruction reads only the exponent): exact for e4m3 inputs
// while the result stays in the bf16 normal range.
__device__ __forceinline__ bf16x8 e4m3x8_to_bf16x8_scaled(uint32_t w0, uint32_t w1, float scale) {
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, true);
  const bf16x4 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3);
  const bf16x4 cd = __builtin_shufflevector(c, d, 0, 1, 2, 3);
  return __builtin_shufflevector(ab, cd, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Block-scaled FP8 partial product of one 128-wide K block on a 16x16 tile.
// a / b hold the lane's 32 bytes (K = 32*(lane/16) .. +32 of the block) as two
// u32x4.  The e4m3 operands are widened to bf16 in registers (exact) and fed to
// four bf16 MFMAs, whose fp32 accumulation is exact to fp32 rounding.  The fp8
// MFMA datapath (16x16x128 and 32x32x64 forms alike) aligns each group of 8
// consecutive K products to the group's largest and drops products more than
// about 2^14 below it, which at K = 7168 costs ~1e-5 of max|C| -- above the
// 1e-2 / 1e-3*max|C| tolerance of the reference check.
__device__ __forceinline__ f32x4 fp8_block_16x16x128(u32x4 a0, u32x4 a1, u32x4 b0, u32x4 b1) {
  f32x4 c = {0.f, 0.f, 0.f, 0.f};
  c = mfma_bf16(e4m3x8_to_bf16x8(a0[0], a0[1]), e4m3x8_to_bf16x8(b0[0], b0[1]), c);
  c = mfma_bf16(e4m3x8_to_bf16x8(a0[2], a0[3]), e4m3x8_to_bf16x8(b0[2], b0[3]), c);
  c = mfma_bf16(e4m3x8_to_bf16x8(a1[0], a1[1]), e4m3x8_to_bf16x8(b1[0], b1[1]), c);
  c = mfma_bf16(e4m3x8_to_bf16x8(a1[2], a1[3]), e4m3x8_to_bf16x8(b1[2], b1[3]), c);
  return c;
}

__device__ __forceinline__ i32x8 cat_i32x8(u32x4 lo, u32x4 hi) {
  i32x8 r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

// ---------------------------------------------------------------- loads

__device__ __forceinline__ u32x4 ld_u32x4(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Streamed-once data (weights): non-temporal hint keeps it from displacing
// reused data in L2 / MALL.
__device__ __forceinline__ u32x4 ld_u32x4_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Global -> LDS copies (global_load_lds): lane l fills lds + size * l; the LDS
// base is taken from the wave's first lane.  Kept in plain device functions:
// the host pass of hipcc drops a kernel template whose lambdas call the
// 16-byte form directly.
__device__ __forceinline__ void g2l_16(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
}
__device__ __forceinline__ void g2l_16_nt(const void* g, void* l) {  // cache policy 2 = nt
  __builtin_amdgcn_global_load_lds(g, l, 16, 0, 2);
}
__device__ __forceinline__ void g2l_4(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds(g, l, 4, 0, 0);
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Sum, in split order, of the split-K partials of f32x4 element i (splits n4
// elements apart): S > 0 splits known at compile time, all loads issued before
// the first add; S == 0 takes the runtime count `splits` one load at a time.
template <int S>
__device__ __forceinline__ f32x4 sum_splits(const f32x4* __restrict__ part, int splits, size_t n4, size_t i) {
  if constexpr (S > 0) {
    f32x4 v[S];
#pragma unroll
    for (int s = 0; s < S; ++s) v[s] = part[(size_t)s * n4 + i];
    f32x4 acc = v[0];
#pragma unroll
    for (int s = 1; s < S; ++s) acc += v[s];
    return acc;
  } else {
    f32x4 acc = part[i];
    for (int s = 1; s < splits; ++s) acc += part[(size_t)s * n4 + i];
    return acc;
  }
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + __expf(-g)) * u;
}

}  // namespace ferret

// ---------------------------------------------------------------- host helpers

#define FERRET_HIP_CHECK(expr)                 \
  do {                                         \
    hipError_t _e = (expr);                    \
    if (_e != hipSuccess) return (int)_e;      \
  } while (0)

// Raise a kernel's dynamic-LDS limit to `bytes` once per device (the call is a
// host-side cost on every launch otherwise); devices past 64 set it each time.
template <auto Kernel>
inline hipError_t set_lds_limit_once(int bytes) {
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 64;
  const uint64_t bit = dev < 64 ? (1ull << dev) : 0;
  if (bit && (done.load(std::memory_order_relaxed) & bit)) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute((const void*)Kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_relaxed);
  return e;
}

#define FERRET_REQUIRE(cond, code) \
  do {                             \
    if (!(cond)) return (code);    \
  } while (0)
