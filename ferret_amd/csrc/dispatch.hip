// Library-level entry points: version / error text, workspace sizing, and the
// shape dispatch between the skinny (<= 16 token) streaming kernels and the
// tiled MFMA kernels.
#include "common.hpp"

int ferret_fp8_gemm_skinny(const void* a, const float* sa, const void* b, const float* sb, void* c, int M,
                           int N, int K, hipStream_t st);
int ferret_fp8_gemm_tiled(const void* a, const float* sa, const void* b, const float* sb, void* c, int M,
                          int N, int K, void* ws, size_t ws_bytes, bool f8, hipStream_t st);
size_t ferret_fp8_gemm_workspace(int M, int N, int K);
bool ferret_fp8_square_takes(int M, int N, int K);
int ferret_fp8_gemm_square(const void* a, const float* sa, const void* b, const float* sb, void* c, int M, int N,
                           int K, hipStream_t st);
size_t ferret_linear_bf16_workspace(int M, int N, int K);
size_t ferret_moe_permute_workspace(long long num_pairs, int E);
size_t ferret_fp8_gemm_ue8m0_workspace(int M, int N, int K);
int ferret_moe_w13_fp8_skinny(const void* x, const float* sx, const void* w, const float* sw,
                              const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                              int max_tiles, int topk, int N, int K, void* out, hipStream_t st);
int ferret_moe_w13_fp8_tiled(const void* x, const float* sx, const void* w, const float* sw,
                             const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                             int max_tiles, int topk, int N, int K, void* out, bool f8, hipStream_t st);

int ferret_moe_w2_fp8_skinny(const void* h, const float* sh, const void* w, const float* sw,
                             const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                             int max_tiles, int N, int K, void* out, hipStream_t st);
int ferret_moe_w2_fp8_tiled(const void* h, const float* sh, const void* w, const float* sw,
                            const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                            int max_tiles, int N, int K, void* out, bool f8, hipStream_t st);

extern "C" const char* ferret_version(void) { return "ferret-hip 0.1.0 gfx950"; }

extern "C" const char* ferret_error_string(int code) {
  switch (code) {
    case FERRET_OK: return "ok";
    case FERRET_ERR_NULL: return "a required pointer is NULL";
    case FERRET_ERR_SHAPE: return "sizes out of range or not supported";
    case FERRET_ERR_WORKSPACE: return "workspace missing or too small";
    default: break;
  }
  return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown ferret error";
}

extern "C" size_t ferret_workspace_bytes(int op, int M, int N, int K, int E) {
  (void)E;
  if (op == 0 && M > 0 && N >= 16 && N % 16 == 0 && K >= 128 && K % 128 == 0)
    return ferret_linear_bf16_workspace(M, N, K);
  if (op == 1 && M > 16 && M > 0 && N > 0 && K >= 128) return ferret_fp8_gemm_workspace(M, N, K);
  if (op == 4 && M > 0 && E > 0) return ferret_moe_permute_workspace(M, E);
  if (op == 5 && M > 0 && N >= 16 && N % 16 == 0 && K >= 128 && K % 128 == 0 && K / 128 <= 128)
    return ferret_fp8_gemm_ue8m0_workspace(M, N, K);
  return 0;
}

// Flags of the *_ex entry points that every FP8 entry point accepts.
static constexpr int kFp8KnownFlags = FERRET_FP8_MMA_E4M3;

extern "C" int ferret_fp8_gemm_blockscale_ex(const void* a, const float* sa, const void* b, const float* sb,
                                             void* c, int M, int N, int K, void* ws, size_t ws_bytes, int flags,
                                             void* stream) {
  FERRET_REQUIRE(a && sa && b && sb && c, FERRET_ERR_NULL);
  FERRET_REQUIRE((flags & ~kFp8KnownFlags) == 0, FERRET_ERR_SHAPE);
  FERRET_REQUIRE(M >= 1 && N >= 16 && K >= 128 && N % 16 == 0 && K % 128 == 0 && K / 128 <= 128,
                 FERRET_ERR_SHAPE);
  if (M <= 16) return ferret_fp8_gemm_skinny(a, sa, b, sb, c, M, N, K, (hipStream_t)stream);
  FERRET_REQUIRE(N % 128 == 0, FERRET_ERR_SHAPE);
  if ((flags & FERRET_FP8_MMA_E4M3) == 0 && ferret_fp8_square_takes(M, N, K))
    return ferret_fp8_gemm_square(a, sa, b, sb, c, M, N, K, (hipStream_t)stream);
  return ferret_fp8_gemm_tiled(a, sa, b, sb, c, M, N, K, ws, ws_bytes, (flags & FERRET_FP8_MMA_E4M3) != 0,
                               (hipStream_t)stream);
}

extern "C" int ferret_fp8_gemm_blockscale(const void* a, const float* sa, const void* b, const float* sb,
                                          void* c, int M, int N, int K, void* ws, size_t ws_bytes,
                                          void* stream) {
  return ferret_fp8_gemm_blockscale_ex(a, sa, b, sb, c, M, N, K, ws, ws_bytes, 0, stream);
}

extern "C" int ferret_moe_w13_fp8_ex(const void* x, const float* sx, const void* w, const float* sw,
                                     const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                                     int max_tiles, int tile_m, int T, int topk, int E, int N, int K, void* out,
                                     int flags, void* stream) {
  FERRET_REQUIRE(x && sx && w && sw && sorted_pair && tiles && ntiles && out, FERRET_ERR_NULL);
  FERRET_REQUIRE((flags & ~kFp8KnownFlags) == 0, FERRET_ERR_SHAPE);
  FERRET_REQUIRE(T >= 1 && topk >= 1 && E >= 1 && max_tiles >= 0, FERRET_ERR_SHAPE);
  FERRET_REQUIRE(N % 256 == 0 && K % 128 == 0 && K >= 128 && K / 128 <= 128, FERRET_ERR_SHAPE);
  if (tile_m == 16)
    return ferret_moe_w13_fp8_skinny(x, sx, w, sw, sorted_pair, tiles, ntiles, max_tiles, topk, N, K, out,
                                     (hipStream_t)stream);
  if (tile_m == 128)
    return ferret_moe_w13_fp8_tiled(x, sx, w, sw, sorted_pair, tiles, ntiles, max_tiles, topk, N, K, out,
                                    (flags & FERRET_FP8_MMA_E4M3) != 0, (hipStream_t)stream);
  return FERRET_ERR_SHAPE;
}

extern "C" int ferret_moe_w13_fp8(const void* x, const float* sx, const void* w, const float* sw,
                                  const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                                  int max_tiles, int tile_m, int T, int topk, int E, int N, int K, void* out,
                                  void* stream) {
  return ferret_moe_w13_fp8_ex(x, sx, w, sw, sorted_pair, tiles, ntiles, max_tiles, tile_m, T, topk, E, N, K, out,
                               0, stream);
}

extern "C" int ferret_moe_w2_fp8_ex(const void* h, const float* sh, const void* w, const float* sw,
                                    const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                                    int max_tiles, int tile_m, int P, int E, int N, int K, void* out, int flags,
                                    void* stream) {
  FERRET_REQUIRE(h && sh && w && sw && sorted_pair && tiles && ntiles && out, FERRET_ERR_NULL);
  FERRET_REQUIRE((flags & ~kFp8KnownFlags) == 0, FERRET_ERR_SHAPE);
  FERRET_REQUIRE(P >= 1 && E >= 1 && max_tiles >= 0, FERRET_ERR_SHAPE);
  FERRET_REQUIRE(N % 128 == 0 && N >= 128 && K % 128 == 0 && K >= 128 && K / 128 <= 128, FERRET_ERR_SHAPE);
  if (tile_m == 16)
    return ferret_moe_w2_fp8_skinny(h, sh, w, sw, sorted_pair, tiles, ntiles, max_tiles, N, K, out,
                                    (hipStream_t)stream);
  if (tile_m == 128)
    return ferret_moe_w2_fp8_tiled(h, sh, w, sw, sorted_pair, tiles, ntiles, max_tiles, N, K, out,
                                   (flags & FERRET_FP8_MMA_E4M3) != 0, (hipStream_t)stream);
  return FERRET_ERR_SHAPE;
}

extern "C" int ferret_moe_w2_fp8(const void* h, const float* sh, const void* w, const float* sw,
                                 const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                                 int max_tiles, int tile_m, int P, int E, int N, int K, void* out, void* stream) {
  return ferret_moe_w2_fp8_ex(h, sh, w, sw, sorted_pair, tiles, ntiles, max_tiles, tile_m, P, E, N, K, out, 0,
                              stream);
}
