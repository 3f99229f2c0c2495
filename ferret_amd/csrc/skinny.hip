// Skinny (<= 16 token) weight-streaming GEMMs for gfx950: bf16 decode linear,
// small-M FP8 block-scaled GEMM, and the decode-sized MoE grouped GEMMs (FP8
// w13 and w2, INT4 W4A16 w13) with the fused SiLU(gate)*up epilogue.  Shapes
// whose K-steps split evenly into 2, 4, 7 or 8 per wave run the persistent
// LDS-staged stream kernel of stream_kernel.hpp (bf16 with K split over a
// workspace where the row units alone would leave CUs idle); the per-unit
// kernel below takes the rest.
//
// Design (swap-AB): the weight rows are the MFMA "A" side (16 rows per MFMA)
// and the <= 16 tokens of a unit are the MFMA "B" side, so a 16x16 MFMA tile
// wastes nothing at 16 tokens.  A work-group owns one unit = (token tile,
// RB blocks of 16 weight rows) and splits K across its waves: wave w streams
// K-steps [w*KS, (w+1)*KS) (one K-step = 128 K = one fp32 scale block), with a
// D-deep register prefetch of the weight and activation fragments.  Each lane
// reads 16-byte vectors; per load instruction a wave covers 16 rows x 64
// contiguous bytes.  The per-wave fp32 partials are summed through LDS and the
// epilogue (bf16 store, + residual, or SiLU(gate)*up) runs once per output.
//
// Reference counterparts: swapab_cg1_kernel / swapab_persistent_kernel
// (examples/qwen3-8b-decode-linear-bs16/v006_cg1_swapab_l2hints.cu:138-375,
// v019_swapab_cg2_l2hints.cu:138-391) and the split-K reduce (v019:395-417);
// grouped_fp8_gemm_bs (examples/fp8-group-gemm/v007_dsv3_decode_verified_105.cu:66-335);
// the INT4 w13 contract (tasks/kimi-moe-w13-int4-grouped-gemm.yaml:68-95,150-167).
#include "skinny_kernel.hpp"
#include "stream_kernel.hpp"

namespace ferret {

// Compute units of the current device (the persistent grid size), cached per
// device; concurrent first calls store the same value.
static int cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Stream-kernel launch (persistent grid, one work-group of NW waves per CU):
// returns 1 if the shape is not covered (the caller then uses the per-unit
// kernel), else the launch status.  KS = K-steps per wave = K / 128 / NW.
template <int F, int EPI, int RB, int D, int NW = 8>
static int try_stream(const SkinnyArgs& a_in, int dense_tiles, int max_tiles, hipStream_t st) {
  // The unit count, K-steps per wave and tile-table span come from the
  // host-only plan (stream_plan.hpp), which the CPU tests check over every
  // configuration instantiated here: a unit is RB 16-row blocks (SiLU: one
  // gate and one up block), counted from RB itself, not from the caller
  // (whose units_n sizes the per-unit fallback kernel).
  static_assert(EPI != kSilu || RB == 2, "SiLU units pair one gate and one up block");
  const bool grouped = a_in.tiles != nullptr;
  // bf16 dense split-K: each work item covers K / nsplit (see stream_gemm_kernel)
  const int nsplit = (F == kBF16 && !grouped && a_in.partial != nullptr) ? a_in.ksplit : 1;
  const int grid = cu_count();
  const StreamPlan plan = stream_plan(EPI == kSilu, RB, NW, a_in.N, a_in.K, grouped ? max_tiles : dense_tiles,
                                      grouped, nsplit, grid);
  if (!plan.ok) return 1;
  // INT4 unit scales are copied as 16-byte chunks of the scale rows.
  if (is_int4(F) && ((reinterpret_cast<uintptr_t>(a_in.w_scale) & 15) != 0 || a_in.K % 256 != 0)) return 1;
  SkinnyArgs a = a_in;
  a.units_n = plan.units_n;
  const int slots = grouped ? max_tiles : dense_tiles;
  // INT4 keeps at most one unit of scales ahead: ring depth <= KS.
  constexpr int D2 = (is_int4(F) && D > 2) ? 2 : D;
  constexpr int D4 = (is_int4(F) && D > 4) ? 4 : D;
  switch (plan.ks) {
    case 2: return launch_stream<F, EPI, RB, NW, 2, D2>(a, slots, grid, st);
    case 4: return launch_stream<F, EPI, RB, NW, 4, D4>(a, slots, grid, st);
    // More than 8 waves leave a wave 128 VGPRs (two work-groups' worth of waves
    // on some SIMDs), too few for 7 or 8 K-steps of activations: those shapes
    // take the 8-wave configuration (the caller's fallback).
    case 7: if constexpr (NW <= 8) return launch_stream<F, EPI, RB, NW, 7, D>(a, slots, grid, st); else return 1;
    case 8: if constexpr (NW <= 8) return launch_stream<F, EPI, RB, NW, 8, D>(a, slots, grid, st); else return 1;
  }
  return 1;
}

// K-steps per wave: prefer a split giving 4..16 waves (balanced reduction
// against per-wave stream depth), else any split with <= 16 waves.
static int choose_ks(int nkb, const int* cand, int ncand) {
  for (int i = 0; i < ncand; ++i) {
    const int ks = cand[i];
    if (nkb % ks == 0 && nkb / ks >= 4 && nkb / ks <= 16) return ks;
  }
  for (int i = 0; i < ncand; ++i) {
    const int ks = cand[i];
    if (nkb % ks == 0 && nkb / ks <= 16) return ks;
  }
  return 0;
}

template <int F, int EPI, int RB>
static int launch_skinny(const SkinnyArgs& a, int ntile_slots, hipStream_t st) {
  const int nkb = a.K >> 7;
  static const int cand[] = {4, 7, 8, 2, 1};
  const int ks = choose_ks(nkb, cand, 5);
  const int grid = ntile_slots * a.units_n;
  if (grid <= 0) return FERRET_OK;
  // Prefetch depth kept so a wave stays within 128 VGPRs (16 waves / CU).
  constexpr int DB = (F == kBF16) ? 2 : ((F == kFP8 && RB == 1) ? 4 : (F == kFP8 ? 3 : 2));
  // 7 or 8 K-steps per wave hold more activations: FP8 row pairs (SiLU) keep a
  // 2-deep prefetch and the ragged single-block form a 3-deep one, or they
  // spill past 128 VGPRs.
  constexpr int D78 = (F == kFP8 && RB >= 2) ? 2 : DB;
  constexpr int D78R = (F == kFP8 && RB == 1) ? 3 : D78;
  if (ks == 0) {
    // No K-step count divides K/128 into <= 16 waves (K/128 = 19, 23, 38, ...):
    // the smallest of 2, 4, 7, 8 that fits 16 waves, the last wave ragged.
    for (const int kr : {2, 4, 7, 8}) {
      const int nw = (nkb + kr - 1) / kr;
      if (nw > 16) continue;
      switch (kr) {
        case 2: return launch_one<F, EPI, RB, 2, 1, true>(a, grid, nw, st);
        case 4: return launch_one<F, EPI, RB, 4, (DB < 3 ? DB : 3), true>(a, grid, nw, st);
        case 7: return launch_one<F, EPI, RB, 7, D78R, true>(a, grid, nw, st);
        case 8: return launch_one<F, EPI, RB, 8, D78R, true>(a, grid, nw, st);
      }
    }
    return FERRET_ERR_SHAPE;  // K/128 > 128: rejected by every entry point first
  }
  const int nwaves = nkb / ks;
  switch (ks) {
    case 1: return launch_one<F, EPI, RB, 1, 0>(a, grid, nwaves, st);
    case 2: return launch_one<F, EPI, RB, 2, 1>(a, grid, nwaves, st);
    case 4: return launch_one<F, EPI, RB, 4, (DB < 3 ? DB : 3)>(a, grid, nwaves, st);
    case 7: return launch_one<F, EPI, RB, 7, D78>(a, grid, nwaves, st);
    case 8: return launch_one<F, EPI, RB, 8, D78>(a, grid, nwaves, st);
  }
  return FERRET_ERR_SHAPE;
}

// y[m, n] = bf16(sum_{s < S} partial[s, m, n] (+ residual[m, n])), splits in
// order; SN > 0: S == SN, all split loads issued before the first add.
template <int SN>
__global__ __launch_bounds__(256) void linear_splitk_reduce_kernel(const float* __restrict__ partial, int S,
                                                                   long long mn4, const uint16_t* __restrict__ res,
                                                                   uint16_t* __restrict__ y) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < mn4; i += (long long)gridDim.x * 256) {
    f32x4 v = sum_splits<SN>(reinterpret_cast<const f32x4*>(partial), S, (size_t)mn4, (size_t)i);
    if (res) {
      const u32x2 r = reinterpret_cast<const u32x2*>(res)[i];
      v[0] += __uint_as_float(r[0] << 16);
      v[1] += __uint_as_float(r[0] & 0xffff0000u);
      v[2] += __uint_as_float(r[1] << 16);
      v[3] += __uint_as_float(r[1] & 0xffff0000u);
    }
    reinterpret_cast<u32x2*>(y)[i] = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  }
}

// K splits of the bf16 stream kernel for y = x.W^T: 1 when a work-group per CU
// is already evenly loaded (>= 90 % of the 256 CUs' share), else the split with
// the best balance whose K-steps per wave (of 8) the kernel instantiates.
// Measured reason: 384 row units (QKV) leave half the CUs with one unit and
// half with two; K = 12288 (Down) needs 12 K-steps per wave, more activation
// registers than a wave has.
static int linear_splits(int M, int N, int K) {
  const int nkb = K / 128;
  const long long units = (long long)((M + 15) / 16) * (N / 16);
  const int ncu = cu_count();
  auto ks_ok = [](int ks) { return ks == 2 || ks == 4 || ks == 7 || ks == 8; };
  auto balance = [&](int s) {
    const long long items = units * s;
    const long long per = (items + ncu - 1) / ncu;
    return (double)items / (double)(per * ncu);
  };
  if (nkb % 8 == 0 && ks_ok(nkb / 8) && balance(1) >= 0.9) return 1;
  int best = 1;
  double best_b = -1.0;
  for (int s = 2; s <= 8; ++s) {
    if (nkb % (8 * s) != 0 || !ks_ok(nkb / (8 * s))) continue;
    const double b = balance(s);
    if (b > best_b + 1e-9) { best = s; best_b = b; }
  }
  return best;
}

}  // namespace ferret

using namespace ferret;

size_t ferret_linear_bf16_workspace(int M, int N, int K) {
  const int s = linear_splits(M, N, K);
  return s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
}

extern "C" int ferret_linear_bf16(const void* x, const void* w, const void* residual, void* y, int M,
                                  int N, int K, void* ws, size_t ws_bytes, void* stream) {
  FERRET_REQUIRE(x && w && y, FERRET_ERR_NULL);
  FERRET_REQUIRE(M >= 1 && N >= 16 && K >= 128, FERRET_ERR_SHAPE);
  FERRET_REQUIRE(N % 16 == 0 && K % 128 == 0 && K / 128 <= 128, FERRET_ERR_SHAPE);
  const hipStream_t st = (hipStream_t)stream;
  SkinnyArgs a{};
  a.w = static_cast<const uint8_t*>(w);
  a.x = static_cast<const uint8_t*>(x);
  a.residual = static_cast<const uint16_t*>(residual);
  a.out = static_cast<uint16_t*>(y);
  a.M = M;
  a.N = N;
  a.K = K;
  a.units_n = N / 16;
  const int splits = linear_splits(M, N, K);
  const size_t need = ferret_linear_bf16_workspace(M, N, K);
  if (splits > 1 && ws != nullptr && ws_bytes >= need && (M * (long long)N) % 4 == 0) {
    a.partial = static_cast<float*>(ws);
    a.ksplit = splits;
    const int rc = try_stream<kBF16, kStore, 1, 3, 8>(a, (M + 15) / 16, 0, st);
    if (rc != 1) {
      if (rc != 0) return rc;
      const long long mn4 = (long long)M * N / 4;
      const int grid = (int)std::min<long long>((mn4 + 255) / 256, 4096);
      auto* reduce = splits == 2 ? linear_splitk_reduce_kernel<2> : splits == 3 ? linear_splitk_reduce_kernel<3>
                   : splits == 4 ? linear_splitk_reduce_kernel<4> : linear_splitk_reduce_kernel<0>;
      hipLaunchKernelGGL(reduce, dim3(grid), dim3(256), 0, st, a.partial, splits, mn4, a.residual, a.out);
      return (int)hipGetLastError();
    }
    a.partial = nullptr;
    a.ksplit = 0;
  }
  // Unsplit: with >= 4 row units per CU, 4 waves of 8 K-steps per unit stream
  // faster than 8 waves of 4 (the work-group's units start sooner and reduce
  // over half the waves): GateUp 39.6 -> 36.7 us, LMHead 202 -> 195 us; with one
  // unit per CU (O) 8 waves keep more bytes in flight.
  const long long units = (long long)((M + 15) / 16) * (N / 16);
  int rc = 1;
  if (units >= 4LL * cu_count()) rc = try_stream<kBF16, kStore, 1, 4, 4>(a, (M + 15) / 16, 0, st);
  if (rc == 1) rc = try_stream<kBF16, kStore, 1, 3, 8>(a, (M + 15) / 16, 0, st);
  if (rc != 1) return rc;
  return launch_skinny<kBF16, kStore, 1>(a, (M + 15) / 16, st);
}

// ---- allocation-free decode linear (no counterpart in the reference).
// Callers that cannot allocate (code under HIP graph capture, serving loops)
// get the split-K partials of ferret_linear_bf16 from this file-scope device
// array instead of a workspace argument.  Each GPU holds its own copy until
// the process ends; its address is looked up once per device
// (hipGetSymbolAddress, with that device current) and only that address is
// handed to kernels.  Calls that overlap on one GPU share the array and race;
// every split writes all of its partials before the reduce reads them, so
// nothing needs clearing between calls.
constexpr size_t kNoAllocScratchBytes = 4u << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
static std::atomic<void*> g_scratch_ptr[64];

// Device address of `scratch` on the current device (cached per device), or
// the hipGetSymbolAddress error.
static hipError_t scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return hipSuccess;
}

// Also looks the array's address up on the current device (errors are left
// for the entry point to report), so that a caller can do it before capturing
// ferret_linear_bf16_noalloc into a graph.
extern "C" size_t ferret_linear_bf16_noalloc_max_bytes(void) {
  void* p = nullptr;
  (void)scratch_address(&p);
  return kNoAllocScratchBytes;
}

extern "C" int ferret_linear_bf16_noalloc(const void* x, const void* w, const void* residual, void* y, int M,
                                          int N, int K, void* stream) {
  FERRET_REQUIRE(x && w && y, FERRET_ERR_NULL);
  FERRET_REQUIRE(M >= 1 && N >= 16 && K >= 128, FERRET_ERR_SHAPE);
  FERRET_REQUIRE(N % 16 == 0 && K % 128 == 0 && K / 128 <= 128, FERRET_ERR_SHAPE);
  const size_t need = ferret_linear_bf16_workspace(M, N, K);
  FERRET_REQUIRE(need <= kNoAllocScratchBytes, FERRET_ERR_WORKSPACE);
  void* ws = nullptr;
  if (need > 0) FERRET_HIP_CHECK(scratch_address(&ws));
  return ferret_linear_bf16(x, w, residual, y, M, N, K, ws, need, stream);
}

extern "C" void launch_gemv(void* input, void* weight, void* residual, void* output, int N, int K,
                            void* stream) {
  (void)ferret_linear_bf16(input, weight, residual, output, 1, N, K, nullptr, 0, stream);
}

// Small-M FP8 block-scaled GEMM (M <= 16 per token tile); called by the dense
// FP8 entry point for skinny shapes.
int ferret_fp8_gemm_skinny(const void* a_, const float* sa, const void* b, const float* sb, void* c,
                           int M, int N, int K, hipStream_t st) {
  SkinnyArgs a{};
  a.w = static_cast<const uint8_t*>(b);
  a.w_scale = sb;
  a.x = static_cast<const uint8_t*>(a_);
  a.x_scale = sa;
  a.out = static_cast<uint16_t*>(c);
  a.M = M;
  a.N = N;
  a.K = K;
  a.units_n = N / 16;  // units of the per-unit fallback (RB = 1)
  // Short K (<= 2 K-steps per wave, e.g. K = 2048): two row blocks per unit
  // halve the per-unit reductions (o_proj, K = 2048: 8.2 -> 7.5 us); at K = 7168
  // one block with a deeper ring is faster (12.2 vs 13.5 us).
  // With at most one 16-row unit per CU (M = 16, N = 4096, K = 7168: 256 units)
  // the whole unit is requested up front, so more waves per unit, each with
  // fewer K-steps, shorten the first-byte-to-last-byte time: 14 waves x 4
  // K-steps (ring depth 4) run 9.0 us against 10.0 us for 8 x 7.
  const long long units16 = (long long)((M + 15) / 16) * (N / 16);
  int rc = 1;
  if ((K >> 7) <= 16) {
    rc = try_stream<kFP8, kStore, 2, 3, 8>(a, (M + 15) / 16, 0, st);
  } else {
    if ((K >> 7) % 14 == 0 && units16 <= cu_count()) rc = try_stream<kFP8, kStore, 1, 4, 14>(a, (M + 15) / 16, 0, st);
    if (rc == 1) rc = try_stream<kFP8, kStore, 1, 6, 8>(a, (M + 15) / 16, 0, st);
  }
  if (rc != 1) return rc;
  return launch_skinny<kFP8, kStore, 1>(a, (M + 15) / 16, st);
}

// Decode-sized FP8 MoE w13 (tile_m = 16).
int ferret_moe_w13_fp8_skinny(const void* x, const float* sx, const void* w, const float* sw,
                              const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                              int max_tiles, int topk, int N, int K, void* out, hipStream_t st) {
  SkinnyArgs a{};
  a.w = static_cast<const uint8_t*>(w);
  a.w_scale = sw;
  a.x = static_cast<const uint8_t*>(x);
  a.x_scale = sx;
  a.out = static_cast<uint16_t*>(out);
  a.sorted_pair = sorted_pair;
  a.tiles = tiles;
  a.ntiles = ntiles;
  a.topk = topk;
  a.N = N;
  a.K = K;
  a.units_n = N / 32;
  if (max_tiles <= 0) return FERRET_OK;
  const int rc = try_stream<kFP8, kSilu, 2, 3, 8>(a, 0, max_tiles, st);
  if (rc != 1) return rc;
  return launch_skinny<kFP8, kSilu, 2>(a, max_tiles, st);
}

// Decode-sized FP8 MoE w2 / down projection (tile_m = 16): the A row and the
// output row of a sorted row are both its routed pair (topk = 1 indexing).
int ferret_moe_w2_fp8_skinny(const void* h, const float* sh, const void* w, const float* sw,
                             const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                             int max_tiles, int N, int K, void* out, hipStream_t st) {
  SkinnyArgs a{};
  a.w = static_cast<const uint8_t*>(w);
  a.w_scale = sw;
  a.x = static_cast<const uint8_t*>(h);
  a.x_scale = sh;
  a.out = static_cast<uint16_t*>(out);
  a.sorted_pair = sorted_pair;
  a.tiles = tiles;
  a.ntiles = ntiles;
  a.topk = 1;
  a.N = N;
  a.K = K;
  if (max_tiles <= 0) return FERRET_OK;
// K = 2048 gives 8 waves only 2 K-steps per 16-row unit, so wider units with
// fewer waves pay (fewer cross-wave reductions per weight byte): two blocks
// per unit took 32 experts x 1 row 79 -> 71 us and 256 experts 605 -> 592 us;
// four blocks on 4 waves of 4 K-steps take 256 experts 593 -> 555 us and
// 32 experts x 16 rows 82 -> 79 us.
  a.units_n = N / 16;  // units of the per-unit fallback (RB = 1); try_stream derives its own
  const int rc = try_stream<kFP8, kStore, 4, 3, 4>(a, 0, max_tiles, st);
  if (rc != 1) return rc;
  return launch_skinny<kFP8, kStore, 1>(a, max_tiles, st);
}

namespace ferret {

// The W4A16 w13 decode over either weight layout (F = kINT4: the checkpoint's
// [E, N, K/8] words; kINT4T: the same words in 16-row x 128-K tiles).
template <int F>
static int moe_w13_w4a16(const void* x, const int32_t* wq, const void* ws, const int32_t* sorted_pair,
                         const int32_t* tiles, const int32_t* ntiles, int max_tiles, int tile_m, int T, int topk,
                         int E, int N, int K, void* out, hipStream_t st) {
  FERRET_REQUIRE(x && wq && ws && sorted_pair && tiles && ntiles && out, FERRET_ERR_NULL);
  FERRET_REQUIRE(T >= 1 && topk >= 1 && E >= 1 && max_tiles >= 0, FERRET_ERR_SHAPE);
  FERRET_REQUIRE(tile_m == 16 && N % 32 == 0 && N >= 32 && K % 128 == 0 && K >= 128, FERRET_ERR_SHAPE);
  SkinnyArgs a{};
  a.w = reinterpret_cast<const uint8_t*>(wq);
  a.w_scale = ws;
  a.x = static_cast<const uint8_t*>(x);
  a.out = static_cast<uint16_t*>(out);
  a.sorted_pair = sorted_pair;
  a.tiles = tiles;
  a.ntiles = ntiles;
  a.topk = topk;
  a.N = N;
  a.K = K;
  a.units_n = N / 32;
  if (max_tiles <= 0) return FERRET_OK;
  const int rc = try_stream<F, kSilu, 2, 5, 8>(a, 0, max_tiles, st);
  if (rc != 1) return rc;
  return launch_skinny<F, kSilu, 2>(a, max_tiles, st);
}

// One thread per 16-byte chunk of the tiled output:
// out[e][n/16][k/128][n%16][64 B] = the K-step k/128 slice (64 B) of row n.
__global__ __launch_bounds__(256) void int4_tile_kernel(const uint8_t* __restrict__ w, uint8_t* __restrict__ t,
                                                        long long nchunks, int nkb) {
  const long long row_bytes = (long long)nkb * 64;
  for (long long o = (long long)blockIdx.x * 256 + threadIdx.x; o < nchunks; o += (long long)gridDim.x * 256) {
    const int c = (int)(o & 3);
    const int row = (int)((o >> 2) & 15);
    const long long tile = o >> 6;  // (e * N/16 + block) * nkb + k-step
    const int ks = (int)(tile % nkb);
    const long long eb = tile / nkb;  // e * N/16 + block: rows 16 * eb .. of the [E * N] row list
    const u32x4 v = ld_u32x4_stream(w + (eb * 16 + row) * row_bytes + ks * 64 + c * 16);
    *reinterpret_cast<u32x4*>(t + o * 16) = v;
  }
}

}  // namespace ferret

using namespace ferret;

extern "C" int ferret_moe_w13_w4a16(const void* x, const int32_t* wq, const void* ws,
                                    const int32_t* sorted_pair, const int32_t* tiles,
                                    const int32_t* ntiles, int max_tiles, int tile_m, int T, int topk,
                                    int E, int N, int K, void* out, void* stream) {
  return moe_w13_w4a16<kINT4>(x, wq, ws, sorted_pair, tiles, ntiles, max_tiles, tile_m, T, topk, E, N, K, out,
                              (hipStream_t)stream);
}

extern "C" int ferret_moe_w13_w4a16_tiled(const void* x, const void* wq_tiled, const void* ws,
                                          const int32_t* sorted_pair, const int32_t* tiles,
                                          const int32_t* ntiles, int max_tiles, int tile_m, int T, int topk,
                                          int E, int N, int K, void* out, void* stream) {
  return moe_w13_w4a16<kINT4T>(x, static_cast<const int32_t*>(wq_tiled), ws, sorted_pair, tiles, ntiles,
                               max_tiles, tile_m, T, topk, E, N, K, out, (hipStream_t)stream);
}

extern "C" int ferret_int4_tile_weights(const int32_t* wq, void* wq_tiled, int E, int N, int K, void* stream) {
  FERRET_REQUIRE(wq && wq_tiled, FERRET_ERR_NULL);
  FERRET_REQUIRE(E >= 1 && N >= 16 && N % 16 == 0 && K >= 128 && K % 128 == 0, FERRET_ERR_SHAPE);
  const long long bytes = (long long)E * N * (K / 2);
  const uint8_t* src = reinterpret_cast<const uint8_t*>(wq);
  uint8_t* dst = static_cast<uint8_t*>(wq_tiled);
  FERRET_REQUIRE(dst + bytes <= src || src + bytes <= dst, FERRET_ERR_SHAPE);  // out of place only
  const long long nchunks = bytes / 16;
  const unsigned grid = (unsigned)std::min<long long>((nchunks + 255) / 256, 65536);
  hipLaunchKernelGGL(int4_tile_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, src, dst, nchunks, K / 128);
  return (int)hipGetLastError();
}
