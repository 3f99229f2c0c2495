// Tiled FP8 (OCP e4m3) block-scaled GEMM for gfx950: the MFMA-bound dense case
// (M > 16) and the prefill-sized MoE w13 grouped GEMM with fused SiLU(gate)*up.
//
// Math (examples/fp8-gemm/v002_dense_tp8_validated_065.cu:277-288):
//   C[m, n] = sum_kb (sum_{k in kb} A[m,k] B[n,k]) * sa[m,kb] * sb[n/128,kb]
// One K-step is one 128-wide scale block.  Per 16x16 sub-tile the block's
// partial product is formed from C = 0 (e4m3 operands widened to bf16 in
// registers, four bf16 MFMAs with exact fp32 accumulation) and the VALU folds
// it into the fp32 accumulator with the (sa * sb) scale.
//
// Swap-AB orientation: weight rows are the MFMA A side and tokens the B side,
// so each lane's accumulator column is one token (one activation scale per
// token sub-tile) and the 16 weight rows of a sub-tile share one weight scale.
//
// Work-group: 256 threads = 4 waves (2 along weight rows x 2 along tokens),
// tile 128 weight rows x 128 tokens, wave tile 64 x 64 (4 x 4 MFMA tiles).
// Global -> VGPR -> LDS double buffering, one barrier per K-step; LDS rows of
// 128 B with the 16-byte chunk index XOR-swizzled by (row & 7) so the MFMA
// fragment reads are bank-conflict free.
//
// Reference counterparts: fp8_gemm<BN,NS> (v002:61-249) and
// grouped_fp8_gemm_bs<BN,NS> (examples/fp8-group-gemm/v007_dsv3_decode_verified_105.cu:66-335),
// whose per-K-block epilogue (v002:179-210) this fuses into the main loop.
#include "common.hpp"

namespace ferret {

constexpr int TB_N = 128;     // weight rows per work-group
constexpr int TB_M = 128;     // tokens per work-group
constexpr int TB_K = 128;     // K per step (one scale block)
constexpr int TB_THREADS = 256;
constexpr int TB_STAGE = (TB_N + TB_M) * TB_K;  // bytes per LDS stage

struct TiledArgs {
  const uint8_t* a;        // e4m3 tokens [T, K]
  const float* sa;         // [T, K/128]
  const uint8_t* b;        // e4m3 weights [G, N, K]
  const float* sb;         // [G, N/128, K/128]
  uint16_t* out;           // dense: [M, N]; SiLU: [P, N/2]
  const int32_t* sorted_pair;
  const int32_t* tiles;    // grouped: [max_tiles, 3]
  const int32_t* ntiles;
  int topk;
  int M, N, K;
  int n_blocks;            // work-group tiles along the weight rows (per token tile)
  int m_blocks;            // dense: token tiles
};

__device__ __forceinline__ int swz(int row, int chunk) { return row * TB_K + ((chunk ^ (row & 7)) << 4); }

template <bool SILU>
__global__ __launch_bounds__(TB_THREADS, 1) void fp8_tiled_kernel(TiledArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * TB_STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = wave & 1;   // weight-row half of the tile
  const int wm = wave >> 1;  // token half of the tile
  const int r = lane & 15;
  const int g = lane >> 4;

  // ---- which tile.
  int e = 0, row0, nrows, nb, mb;
  if constexpr (SILU) {
    // Grouped: bid = tile * n_blocks + nb.  Work-groups are dealt to the 8 XCDs
    // round-robin by block id and n_blocks % 8 == 0, so every tile's block nb
    // lands on XCD nb % 8: the row tiles of one expert share its weight block
    // in that XCD's L2.
    nb = blockIdx.x % p.n_blocks;
    const int tile_idx = blockIdx.x / p.n_blocks;
    if (tile_idx >= p.ntiles[0]) return;
    e = p.tiles[3 * tile_idx];
    row0 = p.tiles[3 * tile_idx + 1];
    nrows = p.tiles[3 * tile_idx + 2];
    mb = 0;
  } else {
    // Dense: give each XCD a contiguous range of logical tiles, then raster
    // the logical tiles in groups of 8 token blocks so the work-groups resident
    // on one XCD share 8 token blocks and 8 weight blocks through its L2.
    const int G = gridDim.x;
    int L = blockIdx.x;
    if ((G & 7) == 0) L = (L & 7) * (G >> 3) + (L >> 3);
    constexpr int GM = 8;
    const int per_group = GM * p.n_blocks;
    const int first_mb = (L / per_group) * GM;
    const int gsize = min(p.m_blocks - first_mb, GM);
    const int in_group = L % per_group;
    mb = first_mb + in_group % gsize;
    nb = in_group / gsize;
    row0 = mb * TB_M;
    nrows = min(TB_M, p.M - row0);
  }

  const int K = p.K, N = p.N;
  const int nkb = K / TB_K;

  // ---- per-thread global source rows for the staging loads.
  // Each thread moves 4 chunks of the weight tile and 4 of the token tile per
  // K-step: chunk index idx = tid + 256*i -> row idx/8, 16-byte chunk idx%8.
  const uint8_t* bsrc[4];
  const uint8_t* asrc[4];
  int srow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + TB_THREADS * i;
    const int rr = idx >> 3;
    const int c = idx & 7;
    srow[i] = rr;
    int wrow;
    if constexpr (SILU) {
      // rows 0..63 of the tile are gate rows nb*64.., rows 64..127 the matching up rows
      wrow = (rr < 64) ? nb * 64 + rr : N / 2 + nb * 64 + (rr - 64);
    } else {
      wrow = nb * TB_N + rr;
    }
    bsrc[i] = p.b + ((size_t)e * N + wrow) * K + c * 16;
    const int t = min(rr, nrows - 1);
    const int tok = SILU ? p.sorted_pair[row0 + t] / p.topk : row0 + t;
    asrc[i] = p.a + (size_t)tok * K + c * 16;
  }

  // ---- fragment rows of this lane
  // weight sub-tile ni covers tile rows wn*32 + (ni&1)*16 + (ni>>1)*64 for SiLU
  // (ni 0,1 gate; 2,3 up) and wn*64 + ni*16 for the dense case.
  int wfrag_row[4];
#pragma unroll
  for (int ni = 0; ni < 4; ++ni)
    wfrag_row[ni] = SILU ? (wn * 32 + (ni & 1) * 16 + (ni >> 1) * 64 + r) : (wn * 64 + ni * 16 + r);
  int afrag_row[4];
  int tok_of[4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    afrag_row[mi] = wm * 64 + mi * 16 + r;
    const int t = min(afrag_row[mi], nrows - 1);
    tok_of[mi] = SILU ? p.sorted_pair[row0 + t] / p.topk : row0 + t;
  }
  // weight-scale row block (uniform per wave): dense: (nb*128 + wn*64)/128;
  // SiLU: gate rows and up rows lie in different 128-row scale blocks.
  const int sb_gate = SILU ? (nb * 64 + wn * 32) >> 7 : (nb * TB_N + wn * 64) >> 7;
  const int sb_up = SILU ? (N / 2 + nb * 64 + wn * 32) >> 7 : sb_gate;
  const float* sbp = p.sb + (size_t)e * (N >> 7) * nkb;

  f32x4 acc[4][4];
#pragma unroll
  for (int ni = 0; ni < 4; ++ni)
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) acc[ni][mi] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 stg_b[4], stg_a[4];
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      stg_b[i] = ld_u32x4_stream(bsrc[i] + (size_t)kb * TB_K);
      stg_a[i] = ld_u32x4(asrc[i] + (size_t)kb * TB_K);
    }
  };
  auto lstore = [&](int buf) {
    uint8_t* base = lds + buf * TB_STAGE;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + TB_THREADS * i;
      const int c = idx & 7;
      *reinterpret_cast<u32x4*>(base + swz(srow[i], c)) = stg_b[i];
      *reinterpret_cast<u32x4*>(base + TB_N * TB_K + swz(srow[i], c)) = stg_a[i];
    }
  };

  gload(0);
  lstore(0);
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < nkb) gload(kb + 1);

    // scales for this K-step
    float sa_v[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) sa_v[mi] = p.sa[(size_t)tok_of[mi] * nkb + kb];
    const float sbg = sbp[(size_t)sb_gate * nkb + kb];
    const float sbu = sbp[(size_t)sb_up * nkb + kb];

    const uint8_t* base = lds + buf * TB_STAGE;
    // Token fragments: read once per K-step and widened to bf16 (K = 32g + 8j .. +8 for MFMA j).
    u32x4 abf[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      const int rr = afrag_row[mi];
      const u32x4 lo = *reinterpret_cast<const u32x4*>(base + TB_N * TB_K + swz(rr, 2 * g));
      const u32x4 hi = *reinterpret_cast<const u32x4*>(base + TB_N * TB_K + swz(rr, 2 * g + 1));
      abf[mi][0] = e4m3x8_to_bf16x8(lo[0], lo[1]);
      abf[mi][1] = e4m3x8_to_bf16x8(lo[2], lo[3]);
      abf[mi][2] = e4m3x8_to_bf16x8(hi[0], hi[1]);
      abf[mi][3] = e4m3x8_to_bf16x8(hi[2], hi[3]);
    }
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      const float sbv = (SILU && ni >= 2) ? sbu : sbg;
      const int rr = wfrag_row[ni];
      const u32x4 lo = *reinterpret_cast<const u32x4*>(base + swz(rr, 2 * g));
      const u32x4 hi = *reinterpret_cast<const u32x4*>(base + swz(rr, 2 * g + 1));
      const u32x4 wbf[4] = {e4m3x8_to_bf16x8(lo[0], lo[1]), e4m3x8_to_bf16x8(lo[2], lo[3]),
                            e4m3x8_to_bf16x8(hi[0], hi[1]), e4m3x8_to_bf16x8(hi[2], hi[3])};
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        f32x4 part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) part = mfma_bf16_16x16x32(wbf[j], abf[mi][j], part);
        const float sc = sa_v[mi] * sbv;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[ni][mi][i] = fmaf(part[i], sc, acc[ni][mi][i]);
      }
    }

    if (kb + 1 < nkb) lstore(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue. acc[ni][mi][i]: weight row wfrag_row[ni] - r + 4g + i, token column r.
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    const int tl = wm * 64 + mi * 16 + r;  // token row inside the tile
    if (tl >= nrows) continue;
    if constexpr (SILU) {
      const int pair = p.sorted_pair[row0 + tl];
      uint16_t* o = p.out + (size_t)pair * (N / 2) + nb * 64 + wn * 32;
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        u32x2 v;
        v[0] = pack_bf16x2(silu_mul(acc[ni][mi][0], acc[ni + 2][mi][0]), silu_mul(acc[ni][mi][1], acc[ni + 2][mi][1]));
        v[1] = pack_bf16x2(silu_mul(acc[ni][mi][2], acc[ni + 2][mi][2]), silu_mul(acc[ni][mi][3], acc[ni + 2][mi][3]));
        *reinterpret_cast<u32x2*>(o + ni * 16 + 4 * g) = v;
      }
    } else {
      uint16_t* o = p.out + (size_t)(row0 + tl) * N + nb * TB_N + wn * 64;
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        u32x2 v;
        v[0] = pack_bf16x2(acc[ni][mi][0], acc[ni][mi][1]);
        v[1] = pack_bf16x2(acc[ni][mi][2], acc[ni][mi][3]);
        *reinterpret_cast<u32x2*>(o + ni * 16 + 4 * g) = v;
      }
    }
  }
}

}  // namespace ferret

using namespace ferret;

int ferret_fp8_gemm_tiled(const void* a, const float* sa, const void* b, const float* sb, void* c, int M,
                          int N, int K, hipStream_t st) {
  TiledArgs p{};
  p.a = static_cast<const uint8_t*>(a);
  p.sa = sa;
  p.b = static_cast<const uint8_t*>(b);
  p.sb = sb;
  p.out = static_cast<uint16_t*>(c);
  p.M = M;
  p.N = N;
  p.K = K;
  p.n_blocks = N / TB_N;
  p.m_blocks = (M + TB_M - 1) / TB_M;
  const int grid = p.n_blocks * p.m_blocks;
  hipLaunchKernelGGL((fp8_tiled_kernel<false>), dim3(grid), dim3(TB_THREADS), 0, st, p);
  return (int)hipGetLastError();
}

int ferret_moe_w13_fp8_tiled(const void* x, const float* sx, const void* w, const float* sw,
                             const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                             int max_tiles, int topk, int N, int K, void* out, hipStream_t st) {
  TiledArgs p{};
  p.a = static_cast<const uint8_t*>(x);
  p.sa = sx;
  p.b = static_cast<const uint8_t*>(w);
  p.sb = sw;
  p.out = static_cast<uint16_t*>(out);
  p.sorted_pair = sorted_pair;
  p.tiles = tiles;
  p.ntiles = ntiles;
  p.topk = topk;
  p.N = N;
  p.K = K;
  p.n_blocks = (N / 2) / 64;
  const int grid = max_tiles * p.n_blocks;
  if (grid <= 0) return FERRET_OK;
  hipLaunchKernelGGL((fp8_tiled_kernel<true>), dim3(grid), dim3(TB_THREADS), 0, st, p);
  return (int)hipGetLastError();
}
