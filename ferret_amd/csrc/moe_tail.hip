// The MoE layer around the grouped GEMMs: the 1x128 activation quantizer
// (bf16 -> OCP e4m3 + fp32 scales, the input format of every FP8 GEMM here)
// and the top-k weighted combine of the w2 (down) outputs.
//
// Quantizer (the library's absmax/448 rule; the reference calls DeepGEMM's
// per_token_cast_to_fp8 at baselines/fp8-gemm/baseline_prefill.py:41, whose
// epsilon clamp is not vendored):
//   amax = max(max_{k in block} |x[m,k]|, 1e-4)
//   q[m,k] = e4m3_RNE(x[m,k] * (448 / amax)),   scale[m, block] = amax / 448
// all in fp32 with correctly rounded division, so the result is bit for bit
// the oracle's.  HBM-bound: 2 bytes read + 1 written per element.
//
// Combine: y[t, n] = bf16_RNE(sum_j w[t, j] * o[t*topk + j, n]) with the fp32
// sum taken in j order (deterministic).  HBM-bound: topk*2 + 2 bytes per output.
#include "common.hpp"

namespace ferret {

// 16 lanes per 128-element block, 8 elements (16 bytes) per lane; each
// 16-lane group quantizes QB consecutive blocks, issuing all their loads
// first (QB = 2: 37.3 -> 35.1 us on [32768, 2048], 5.8 TB/s); a 256-thread
// work-group covers 16 * QB blocks.
template <int QB>
__global__ __launch_bounds__(256) void quant_act_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
                                                        float* __restrict__ scale, long long nblocks) {
  const long long blk0 = ((long long)blockIdx.x * 16 + (threadIdx.x >> 4)) * QB;
  const int sub = threadIdx.x & 15;
  u32x4 v[QB];
#pragma unroll
  for (int b = 0; b < QB; ++b) {
    const long long blk = blk0 + b;
    v[b] = blk < nblocks ? ld_u32x4_stream(x + blk * 128 + sub * 8) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int b = 0; b < QB; ++b) {
    const long long blk = blk0 + b;
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(v[b][i] << 16);
      f[2 * i + 1] = __uint_as_float(v[b][i] & 0xffff0000u);
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
    // max over the 16 lanes of the block (aligned groups of 16 lanes)
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 16));
    amax = fmaxf(amax, 1e-4f);
    const float mult = 448.0f / amax;
    uint32_t lo = 0, hi = 0;
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[0] * mult, f[1] * mult, lo, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[2] * mult, f[3] * mult, lo, true);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[4] * mult, f[5] * mult, hi, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[6] * mult, f[7] * mult, hi, true);
    if (blk < nblocks) {
      *reinterpret_cast<u32x2*>(q + blk * 128 + sub * 8) = u32x2{lo, hi};
      if (sub == 0) scale[blk] = amax / 448.0f;
    }
  }
}

// One thread per 8 outputs (16 bytes of each of the topk rows).
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ o, const float* __restrict__ w,
                                                      uint16_t* __restrict__ y, int T, int topk, int N) {
  const int chunks = N / 8;
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long long)T * chunks) return;
  const int t = (int)(idx / chunks);
  const int c = (int)(idx % chunks);
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  if (topk == 8) {
    // The DeepSeek-V3 top-8: all eight row loads go out before the first use
    // (88.4 -> 84.6 us at T = 4096, N = 7168); the sum keeps j order.
    u32x4 v[8];
    float wj[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = ld_u32x4_stream(o + ((size_t)t * 8 + j) * N + (size_t)c * 8);
#pragma unroll
    for (int j = 0; j < 8; ++j) wj[j] = w[(size_t)t * 8 + j];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = fmaf(wj[j], __uint_as_float(v[j][i] << 16), acc[2 * i]);
        acc[2 * i + 1] = fmaf(wj[j], __uint_as_float(v[j][i] & 0xffff0000u), acc[2 * i + 1]);
      }
  } else {
    for (int j = 0; j < topk; ++j) {
      const float wj = w[(size_t)t * topk + j];
      const u32x4 v = ld_u32x4_stream(o + ((size_t)t * topk + j) * N + (size_t)c * 8);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = fmaf(wj, __uint_as_float(v[i] << 16), acc[2 * i]);
        acc[2 * i + 1] = fmaf(wj, __uint_as_float(v[i] & 0xffff0000u), acc[2 * i + 1]);
      }
    }
  }
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(acc[2 * i], acc[2 * i + 1]);
  *reinterpret_cast<u32x4*>(y + (size_t)t * N + (size_t)c * 8) = r;
}

}  // namespace ferret

using namespace ferret;

extern "C" int ferret_quant_act_e4m3(const void* x, void* q, float* scale, int M, int K, void* stream) {
  FERRET_REQUIRE(x != nullptr && q != nullptr && scale != nullptr, FERRET_ERR_NULL);
  FERRET_REQUIRE(M >= 1 && K >= 128 && K % 128 == 0, FERRET_ERR_SHAPE);
  const long long nblocks = (long long)M * (K / 128);
  FERRET_REQUIRE(nblocks / 32 < (1LL << 31), FERRET_ERR_SHAPE);
  constexpr int QB = 2;
  const unsigned grid = (unsigned)((nblocks + 16 * QB - 1) / (16 * QB));
  hipLaunchKernelGGL(quant_act_kernel<QB>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint16_t*>(x), static_cast<uint8_t*>(q), scale, nblocks);
  return (int)hipGetLastError();
}

extern "C" int ferret_moe_combine(const void* o, const float* w, int T, int topk, int N, void* y, void* stream) {
  FERRET_REQUIRE(o != nullptr && w != nullptr && y != nullptr, FERRET_ERR_NULL);
  FERRET_REQUIRE(T >= 1 && topk >= 1 && topk <= 64 && N >= 8 && N % 8 == 0, FERRET_ERR_SHAPE);
  const long long work = (long long)T * (N / 8);
  FERRET_REQUIRE(work / 256 < (1LL << 31), FERRET_ERR_SHAPE);
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint16_t*>(o), w, static_cast<uint16_t*>(y), T, topk, N);
  return (int)hipGetLastError();
}
