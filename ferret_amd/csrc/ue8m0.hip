// Dense FP8 GEMM with UE8M0 (power-of-two) block scales, in the packed scale
// layout of examples/fp8-gemm/v009_large_m_block_scale_mma_080.cu (prepare_sf
// :386-403 over expand_sb :405-412; decoding as ue8m0_to_float :478-484).
//
// A UE8M0 byte e stands for 2^(e - 127); e = 0 stands for a zero scale.  The
// product of two such scales is exact in fp32, so decoding the bytes to fp32
// block scales and running the fp32-scale GEMM (dispatch.hip) computes
//   c[m,n] = sum_kb P_kb[m,n] * 2^(ea - 127) * 2^(eb - 127)
// with the same per-block products P_kb as the reference's oracle ref_bs
// (v009:486-505).  The decode is one small HBM-bound pass over the scales into
// the caller's workspace (M x nk + ceil(N/128) x nk floats), ahead of the GEMM
// on the same stream.  Shapes of the 256 x 256 kernel skip it: that kernel
// reads the packed bytes and scales each operand exactly while widening it.
#include "common.hpp"

namespace ferret {

__device__ __forceinline__ float ue8m0_value(uint32_t word, int byte) {
  const uint32_t e = (word >> (8 * byte)) & 0xFFu;
  return e == 0 ? 0.0f : __uint_as_float(e << 23);
}

// sfa: uint32 [ceil(nk/4), M] column-major (byte j of word [sk, m]: token m,
// K-block 4 sk + j); sfb: uint32 [ceil(nk/4), N] per weight row, of which row
// 128 nb stands for weight block nb.  Writes sa f32 [M, nk], sb f32 [nbk, nk].
__global__ __launch_bounds__(256) void ue8m0_decode_kernel(const uint32_t* __restrict__ sfa,
                                                          const uint32_t* __restrict__ sfb, long long M, int N,
                                                          int nk, int nbk, float* __restrict__ sa,
                                                          float* __restrict__ sb) {
  const long long na = M * nk;
  const long long total = na + (long long)nbk * nk;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    if (i < na) {
      // token-fastest order: consecutive threads read consecutive words of one sk row
      const long long kb = i / M, m = i - kb * M;
      sa[m * nk + kb] = ue8m0_value(sfa[(kb >> 2) * M + m], (int)(kb & 3));
    } else {
      const long long j = i - na;
      const long long kb = j / nbk, nb = j - kb * nbk;
      sb[nb * nk + kb] = ue8m0_value(sfb[(kb >> 2) * (long long)N + nb * 128], (int)(kb & 3));
    }
  }
}

constexpr size_t kUe8m0Align = 256;
inline size_t align_up(size_t v) { return (v + kUe8m0Align - 1) / kUe8m0Align * kUe8m0Align; }

}  // namespace ferret

using namespace ferret;

size_t ferret_fp8_gemm_workspace(int M, int N, int K);

// Workspace of ferret_fp8_gemm_ue8m0: the decoded scales, then the GEMM's own.
size_t ferret_fp8_gemm_ue8m0_workspace(int M, int N, int K) {
  const size_t nk = (size_t)K / 128, nbk = ((size_t)N + 127) / 128;
  const size_t gemm = M > 16 ? ferret_fp8_gemm_workspace(M, N, K) : 0;
  return align_up((size_t)M * nk * 4) + align_up(nbk * nk * 4) + gemm;
}

extern "C" int ferret_fp8_gemm_blockscale(const void* a, const float* sa, const void* b, const float* sb, void* c,
                                          int M, int N, int K, void* ws, size_t ws_bytes, void* stream);
bool ferret_fp8_square_takes(int M, int N, int K);
int ferret_fp8_gemm_square_ue8m0(const void* a, const uint32_t* sfa, const void* b, const uint32_t* sfb, void* c,
                                 int M, int N, int K, hipStream_t st);

extern "C" int ferret_fp8_gemm_ue8m0(const void* a, const uint32_t* sfa, const void* b, const uint32_t* sfb,
                                     void* c, int M, int N, int K, void* ws, size_t ws_bytes, void* stream) {
  FERRET_REQUIRE(a && sfa && b && sfb && c, FERRET_ERR_NULL);
  FERRET_REQUIRE(M >= 1 && N >= 16 && K >= 128 && N % 16 == 0 && K % 128 == 0 && K / 128 <= 128,
                 FERRET_ERR_SHAPE);
  FERRET_REQUIRE(M <= 16 || N % 128 == 0, FERRET_ERR_SHAPE);
  const size_t need = ferret_fp8_gemm_ue8m0_workspace(M, N, K);
  FERRET_REQUIRE(ws != nullptr && ws_bytes >= need, FERRET_ERR_WORKSPACE);
  // Shapes of the 256 x 256 kernel take the packed bytes directly: each
  // power-of-two scale is applied while its operand is widened to bf16 (no
  // decode pass, no running rescale).
  if (M > 16 && ferret_fp8_square_takes(M, N, K))
    return ferret_fp8_gemm_square_ue8m0(a, sfa, b, sfb, c, M, N, K, (hipStream_t)stream);
  const int nk = K / 128, nbk = (N + 127) / 128;
  uint8_t* base = static_cast<uint8_t*>(ws);
  float* sa = reinterpret_cast<float*>(base);
  float* sb = reinterpret_cast<float*>(base + align_up((size_t)M * nk * 4));
  uint8_t* gemm_ws = base + align_up((size_t)M * nk * 4) + align_up((size_t)nbk * nk * 4);
  const size_t gemm_bytes = need - (size_t)(gemm_ws - base);
  const hipStream_t st = (hipStream_t)stream;
  const long long total = (long long)M * nk + (long long)nbk * nk;
  const int grid = (int)((total + 255) / 256 < 1024 ? (total + 255) / 256 : 1024);
  hipLaunchKernelGGL(ue8m0_decode_kernel, dim3(grid), dim3(256), 0, st, sfa, sfb, (long long)M, N, nk, nbk, sa,
                     sb);
  const int rc = (int)hipGetLastError();
  if (rc != 0) return rc;
  return ferret_fp8_gemm_blockscale(a, sa, b, sb, c, M, N, K, gemm_bytes ? gemm_ws : nullptr, gemm_bytes, stream);
}
