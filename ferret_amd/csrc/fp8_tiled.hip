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
// Work-group (large M): 512 threads = 8 waves (4 along weight rows x 2 along
// tokens, two per SIMD so one wave's conversions overlap the other's MFMAs),
// tile 256 weight rows x 128 tokens, wave tile 64 x 64 (4 x 4 MFMA tiles).
// Small M (<= 256) with a workspace: 128 x 128 tiles of 8 waves (64 weight
// rows x 32 tokens each, again two per SIMD) over K ranges (split-K), fp32
// partials summed in split order by a reduce kernel.  Mid M, where 256 x 128
// tiles would occupy at most half of the CUs: the same 128 x 128 tiles over
// all of K, storing bf16.
// Operands go global -> LDS directly (global_load_lds_dwordx4, no VGPR
// staging) through a 3-stage ring; every load instruction reads complete
// 128-byte lines; LDS rows of 128 B have their 16-byte chunk index
// XOR-swizzled so the MFMA fragment reads are bank-conflict free.
// Per K-step a wave widens its fragments (128 v_cvt_scalef32_pk_bf16_fp8:
// phase X) and issues 64 MFMAs and 64 scale folds (phase Y).  The two token
// halves of the tile run X and Y out of phase (one barrier per K-step), so the
// two waves of a SIMD overlap one's MFMAs with the other's widening; the stage
// refills are spread through the Y phases.  A partial tile (grouped GEMM)
// skips the MFMAs and widening of its empty 16-token sub-tiles.
//
// Reference counterparts: fp8_gemm<BN,NS> (v002:61-249) and
// grouped_fp8_gemm_bs<BN,NS> (examples/fp8-group-gemm/v007_dsv3_decode_verified_105.cu:66-335),
// whose per-K-block epilogue (v002:179-210) this fuses into the main loop.
#include "common.hpp"

namespace ferret {

constexpr int TB_K = 128;  // K per step (one scale block)
constexpr int TB_M = 128;  // tokens per work-group (two token waves carry the 128 activation scales)

// Tile geometry: WN waves along the weight rows (64 rows each) x TW waves along
// the 128 tokens (128 / TW each).  WN = 4, TW = 2: 256 x 128 tile, 8 waves (two
// per SIMD) for large M; WN = 2, TW = 4: 128 x 128 tile, 8 waves of 64 x 32,
// used with split-K for small M.
template <int WN, int TW = 2>
struct TileCfg {
  static constexpr int kWN = WN;
  static constexpr int kTW = TW;
  static constexpr int kWaves = WN * TW;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kTokW = TB_M / TW;                  // tokens per wave
  static constexpr int kMI = kTokW / 16;                   // 16-token sub-tiles per wave
  static constexpr int kN = 64 * WN;                       // weight rows per work-group
  static constexpr int kWBytes = kN * TB_K;                // weight rows (e4m3) of a stage
  static constexpr int kABytes = TB_M * TB_K;              // token rows (e4m3) of a stage
  static constexpr int kWInstr = kWBytes / 1024;           // 1-KB load instructions for the weights
  static constexpr int kLdPerWave = (kWBytes + kABytes) / 1024 / kWaves;
  static constexpr int kSaOff = kWBytes + kABytes;         // token scales follow the operand rows
  static constexpr int kStage = kSaOff + TB_M * 4;         // bytes per LDS stage
  static constexpr int kNS = 3;                            // stages in the ring
  static constexpr int kLds = kNS * kStage;                // WN=4: 145.5 KB of the 160 KB LDS
  static_assert((kWBytes + kABytes) % (1024 * kWaves) == 0, "stage loads split evenly over the waves");
  static_assert(kLds <= 160 * 1024, "LDS budget");
  static_assert(TW == 2 || TW == 4, "token halves pair up on the SIMDs");
  static_assert(kThreads == 64 * WN * TW, "fp8_tiled_kernel launch bounds");
};

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
  int k_steps;             // K-steps per split (split-K: gridDim.y splits)
  float* partial;          // split-K: fp32 [splits, M, N] partial sums
};

// Byte offset of 16-byte chunk `chunk` of stage row `row`.  Rows are 128 B;
// the chunk index is XOR-swizzled with (row & 7) ^ ((row >> 3) & 1), which
// keeps the 16 rows of an MFMA fragment read on distinct banks both when the
// LDS serves 8 lanes x 16 B per cycle and when it serves 16.
__device__ __forceinline__ int swz_key(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int swz(int row, int chunk) { return row * TB_K + ((chunk ^ swz_key(row)) << 4); }

// Sum the split-K fp32 partials in split order (deterministic) and round to
// bf16; S > 0: that many splits, all loaded before the first add.
template <int S>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int splits, size_t n4,
                                                           uint16_t* __restrict__ out) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
    const f32x4 acc = sum_splits<S>(reinterpret_cast<const f32x4*>(part), splits, n4, i);
    u32x2 v;
    v[0] = pack_bf16x2(acc[0], acc[1]);
    v[1] = pack_bf16x2(acc[2], acc[3]);
    reinterpret_cast<u32x2*>(out)[i] = v;
  }
}

// F8 = true multiplies the e4m3 bytes on the FP8 MFMA
// (v_mfma_scale_f32_16x16x128_f8f6f4, unit scales) instead of widening them to
// bf16: one MFMA per 16x16x128 block instead of four and no widening, but the
// FP8 datapath aligns the products of a dot-product group to a narrow window,
// which costs about 1e-5 of max|C| at K = 7168 (an opt-in instance, see
// FERRET_FP8_MMA_E4M3).
template <bool SILU, bool GROUPED, int WN, bool SPLIT, bool FULL, bool F8 = false, int TW = 2>
__global__ __launch_bounds__(64 * WN * TW) void fp8_tiled_kernel(TiledArgs p) {
  static_assert(!SILU || GROUPED, "the SiLU epilogue is the grouped w13 GEMM's");
  static_assert(TW == 2 || !SILU, "the SiLU epilogue takes 64-token waves");
  using C = TileCfg<WN, TW>;
  constexpr int MIX = C::kMI, TOKW = C::kTokW;
  constexpr int TB_WN = C::kWN, TB_WAVES = C::kWaves, TB_N = C::kN;
  constexpr int TB_LD_PER_WAVE = C::kLdPerWave, TB_SA_OFF = C::kSaOff, TB_STAGE = C::kStage;
  constexpr int TB_NS = C::kNS;
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps LDS bases in SGPRs
  const int wn = wave % TB_WN;  // weight-row block of the tile
  const int wm = wave / TB_WN;  // token block of the tile (TOKW tokens)
  // Token half: waves w and w + 4 share a SIMD (work-group waves are dealt to
  // the four SIMDs round-robin) and always sit in opposite halves.
  const bool stag = wm >= TW / 2;
  const int r = lane & 15;
  const int g = lane >> 4;

  // ---- which tile.
  int e = 0, row0, nrows, nb;
  if constexpr (GROUPED) {
    // Grouped: bid = tile * n_blocks + nb.  Work-groups are dealt to the 8
    // XCDs round-robin by block id: with n_blocks a multiple of 8, block nb of
    // every tile lands on XCD nb % 8 and the row tiles of one expert share its
    // weight block in that XCD's L2; otherwise the assignment rotates from
    // tile to tile, which keeps the XCDs evenly loaded (padding each tile to a
    // multiple of 8 blocks left the XCDs of the padding a quarter idle at
    // n_blocks = 28).  Tiles past ntiles exit.
    nb = blockIdx.x % p.n_blocks;
    const int tile_idx = blockIdx.x / p.n_blocks;
    if (tile_idx >= p.ntiles[0]) return;
    e = p.tiles[3 * tile_idx];
    row0 = p.tiles[3 * tile_idx + 1];
    nrows = p.tiles[3 * tile_idx + 2];
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
    const int mb = first_mb + in_group % gsize;
    nb = in_group / gsize;
    row0 = mb * TB_M;
    nrows = min(TB_M, p.M - row0);
  }

  const int K = p.K, N = p.N;
  const int nkb = K / TB_K;  // scale-block stride of sa / sb rows
  // This work-group's K-steps: [kb0, kb0 + nsteps) (all of K without split-K).
  const int kb0 = SPLIT ? blockIdx.y * p.k_steps : 0;
  const int nsteps = SPLIT ? min(p.k_steps, nkb - kb0) : nkb;

  // ---- direct-to-LDS loading.  A stage holds the weight rows, then the token
  // rows (128 B of e4m3 each), then the tile's activation scales.  Load
  // instruction j (= w * TB_LD_PER_WAVE + i for wave w) fills stage bytes
  // j KB .. +1 KB: lane l -> row j*8 + l/8 of its part, LDS slot l%8 holding
  // global chunk (l%8) ^ key(row), so every instruction reads eight complete
  // 128-B lines.
  const uint8_t* wbase = p.b + (size_t)e * N * K;
  // 64-bit: row * K reaches 2^32 at e.g. 2^19 rows of K = 8192 (only the
  // pointers below live on into the loop).
  size_t goff[TB_LD_PER_WAVE];
#pragma unroll
  for (int i = 0; i < TB_LD_PER_WAVE; ++i) {
    const int j = wave * TB_LD_PER_WAVE + i;
    if (j < C::kWInstr) {
      const int row = j * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ swz_key(row);
      int wrow;
      if constexpr (SILU)
        wrow = (row < TB_N / 2) ? nb * (TB_N / 2) + row : N / 2 + nb * (TB_N / 2) + (row - TB_N / 2);
      else
        wrow = min(nb * TB_N + row, N - 1);  // rows past N (last block) are loaded but never stored
      goff[i] = (size_t)wrow * K + chunk * 16;
    } else {
      const int row = (j - C::kWInstr) * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ swz_key(row);
      const int t = max(0, min(row, nrows - 1));  // rows past the tile repeat its last row (a zero-row tile: row0)
      const int tok = GROUPED ? p.sorted_pair[row0 + t] / p.topk : row0 + t;
      goff[i] = (size_t)tok * K + chunk * 16;
    }
  }
  // Per-lane source of each load instruction (weights or tokens), so the
  // stage copy is branch-free.  Both operands use the default cache policy:
  // each is re-read by other tiles through L2.
  const uint8_t* src[TB_LD_PER_WAVE];
#pragma unroll
  for (int i = 0; i < TB_LD_PER_WAVE; ++i) {
    const int j = wave * TB_LD_PER_WAVE + i;
    src[i] = (j < C::kWInstr ? wbase : p.a) + goff[i];
  }
  // The last two waves also move the tile's 128 activation scales of the
  // K-step into the stage (4 bytes per lane): the main loop then issues no
  // other vector loads, so the vmcnt bookkeeping below is exact.
  const bool sa_wave = wave >= TB_WAVES - 2;
  const float* sa_src = nullptr;
  if (sa_wave) {
    const int t = max(0, min((wave - (TB_WAVES - 2)) * 64 + lane, nrows - 1));
    const int tok = GROUPED ? p.sorted_pair[row0 + t] / p.topk : row0 + t;
    sa_src = p.sa + (size_t)tok * nkb;
  }
  // Instruction i of this wave's share of stage `step` (i == TB_LD_PER_WAVE:
  // the activation scales, scale waves only).
  auto issue_one = [&](int step, int i) {
    uint8_t* stage = lds + (step % TB_NS) * TB_STAGE;
    const int kb = kb0 + step;
    if (i < TB_LD_PER_WAVE) {
      g2l_16(src[i] + (size_t)kb * TB_K, stage + (wave * TB_LD_PER_WAVE + i) * 1024);
    } else if (sa_wave) {
      __builtin_amdgcn_global_load_lds(sa_src + kb, stage + TB_SA_OFF + (wave - (TB_WAVES - 2)) * 256, 4, 0, 0);
    }
  };
  auto issue_stage = [&](int step) {
#pragma unroll
    for (int i = 0; i <= TB_LD_PER_WAVE; ++i) issue_one(step, i);
  };
  // This thread's copy of stage kb is complete once at most `younger` later
  // stages remain in flight (vector-memory ops per thread and stage:
  // TB_LD_PER_WAVE, plus one for the scale waves).
  auto wait_stage = [&](int younger) {
    constexpr int L = TB_LD_PER_WAVE;
    if (!sa_wave) {
      if (younger >= 1) wait_vmcnt<L>();
      else wait_vmcnt<0>();
    } else {
      if (younger >= 1) wait_vmcnt<L + 1>();
      else wait_vmcnt<0>();
    }
  };
  static_assert(TB_NS == 3, "wait_stage counts one younger stage in flight");

  // ---- fragment rows of this lane
  // weight sub-tile ni covers tile rows wn*32 + (ni&1)*16 + (ni>>1)*(TB_N/2) for
  // SiLU (ni 0,1 gate; 2,3 up) and wn*64 + ni*16 for the dense case.
  int wfrag_row[4];
#pragma unroll
  for (int ni = 0; ni < 4; ++ni)
    wfrag_row[ni] = SILU ? (wn * 32 + (ni & 1) * 16 + (ni >> 1) * (TB_N / 2) + r) : (wn * 64 + ni * 16 + r);
  int afrag_row[MIX];
#pragma unroll
  for (int mi = 0; mi < MIX; ++mi) afrag_row[mi] = wm * TOKW + mi * 16 + r;

  // The wave's weight-scale rows (<= 128 K-steps) are loaded once into lanes
  // (lane l holds K-steps l and 64 + l) before any stage is in flight; each
  // K-step then picks its value with v_readlane, so the main loop issues no
  // vector loads besides the stage copies.
  const int sb_gate = SILU ? (nb * (TB_N / 2) + wn * 32) >> 7 : min(nb * TB_N + wn * 64, N - 1) >> 7;
  const int sb_up = SILU ? (N / 2 + nb * (TB_N / 2) + wn * 32) >> 7 : sb_gate;
  const float* sbp = p.sb + (size_t)e * (N >> 7) * nkb;
  const float sbg_lo = lane < nkb ? sbp[(size_t)sb_gate * nkb + lane] : 0.f;
  const float sbg_hi = 64 + lane < nkb ? sbp[(size_t)sb_gate * nkb + 64 + lane] : 0.f;
  const float sbu_lo = SILU && lane < nkb ? sbp[(size_t)sb_up * nkb + lane] : 0.f;
  const float sbu_hi = SILU && 64 + lane < nkb ? sbp[(size_t)sb_up * nkb + 64 + lane] : 0.f;

  f32x4 acc[4][MIX];
#pragma unroll
  for (int ni = 0; ni < 4; ++ni)
#pragma unroll
    for (int mi = 0; mi < MIX; ++mi) acc[ni][mi] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Prologue: stages 0 .. NS-2 in flight (and stage NS-1 too from the
  // token-half-1 waves of the staggered loop, see below).
#pragma unroll
  for (int s = 0; s < TB_NS - 1; ++s)
    if (s < nsteps) issue_stage(s);
  if (stag && TB_NS - 1 < nsteps) issue_stage(TB_NS - 1);

  // One K-step is two phases: X (LDS fragment reads + e4m3 -> bf16 widening,
  // VALU only) and Y (the MFMAs + the scale folds).  Fragments widened by X
  // live in registers until Y.  Both take the number MI of 16-token sub-tiles
  // of this wave that hold tokens (a partial tile of a grouped GEMM skips the
  // empty ones; MI is uniform per wave).
  bf16x8 abf[MIX][4], wbf[4][4];
  i32x8 araw[MIX], wraw[4];  // F8: the raw e4m3 bytes of each fragment
  float sa_v[MIX], sbg = 0.f, sbu = 0.f;
  auto phase_x = [&](auto mic, int step) {
    constexpr int MI = decltype(mic)::value;
    const int kb = kb0 + step;
    const uint8_t* base = lds + (step % TB_NS) * TB_STAGE;
    const float* sa_lds = reinterpret_cast<const float*>(base + TB_SA_OFF);
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) sa_v[mi] = sa_lds[afrag_row[mi]];
    sbg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
        __builtin_bit_cast(int, kb < 64 ? sbg_lo : sbg_hi), kb & 63));
    sbu = SILU ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(
        __builtin_bit_cast(int, kb < 64 ? sbu_lo : sbu_hi), kb & 63)) : sbg;
    // K = 32g + 8j .. +8 feeds MFMA j of every sub-tile.
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      const int t = afrag_row[mi];
      const uint8_t* arow = base + C::kWBytes + t * TB_K;
      const int key = swz_key(t);
      const u32x4 lo = *reinterpret_cast<const u32x4*>(arow + (((2 * g) ^ key) << 4));
      const u32x4 hi = *reinterpret_cast<const u32x4*>(arow + (((2 * g + 1) ^ key) << 4));
      if constexpr (F8) {
        araw[mi] = cat_i32x8(lo, hi);
        continue;
      }
      abf[mi][0] = e4m3x8_to_bf16x8(lo[0], lo[1]);
      abf[mi][1] = e4m3x8_to_bf16x8(lo[2], lo[3]);
      abf[mi][2] = e4m3x8_to_bf16x8(hi[0], hi[1]);
      abf[mi][3] = e4m3x8_to_bf16x8(hi[2], hi[3]);
    }
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      const int rr = wfrag_row[ni];
      const u32x4 lo = *reinterpret_cast<const u32x4*>(base + swz(rr, 2 * g));
      const u32x4 hi = *reinterpret_cast<const u32x4*>(base + swz(rr, 2 * g + 1));
      if constexpr (F8) {
        wraw[ni] = cat_i32x8(lo, hi);
        continue;
      }
      wbf[ni][0] = e4m3x8_to_bf16x8(lo[0], lo[1]);
      wbf[ni][1] = e4m3x8_to_bf16x8(lo[2], lo[3]);
      wbf[ni][2] = e4m3x8_to_bf16x8(hi[0], hi[1]);
      wbf[ni][3] = e4m3x8_to_bf16x8(hi[2], hi[3]);
    }
    // Keep the widening in X: unpinned, the compiler sinks most of the cvts
    // past the copy branches into Y, where they queue behind the same wave's
    // MFMAs instead of overlapping the partner wave's (8 % of the M = 4096
    // GEMM; the 4-wave tiles are faster unpinned).
    if constexpr (TB_WAVES == 8 && !F8) {
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(abf[mi][j]));
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
#pragma unroll
        for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(wbf[ni][j]));
    }
  };
  // Issue priority of the wave (s_setprio; the arbiter otherwise favours the
  // older waves, token half 0).  Y (MFMA) phases run above X phases, and
  // token half 1 above half 0 in either, so half 0 no longer races ahead and
  // idles at the barrier while half 1 widens its fragments alone.
  auto set_prio = [&](bool y) {
    if constexpr (TB_WAVES == 8) {
      __builtin_amdgcn_sched_barrier(0);
      if (y) {
        if (stag) __builtin_amdgcn_s_setprio(3);
        else __builtin_amdgcn_s_setprio(2);
      } else {
        if (stag) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Phase Y with this wave's share of the copy of stage `istep` (istep < 0:
  // none) spread over its MFMA blocks: instruction i goes after block 2i+1
  // (or the last block; with no blocks all go at once).  Issued in one burst
  // after a barrier, the eight waves' copies queue behind each other and
  // stall the later waves for most of a phase.
  auto phase_y_copy = [&](auto mic, int istep) {
    constexpr int MI = decltype(mic)::value;
    constexpr int NB = 4 * MI;
    set_prio(true);
    if constexpr (NB == 0) {
      if (istep >= 0) {
#pragma unroll
        for (int i = 0; i <= TB_LD_PER_WAVE; ++i) issue_one(istep, i);
      }
    }
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      const float sbv = (SILU && ni >= 2) ? sbu : sbg;
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        f32x4 part = {0.f, 0.f, 0.f, 0.f};
        if constexpr (F8) {
          part = mfma_fp8_16x16x128(wraw[ni], araw[mi], part);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) part = mfma_bf16(wbf[ni][j], abf[mi][j], part);
        }
        const float sc = sa_v[mi] * sbv;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[ni][mi][i] = fmaf(part[i], sc, acc[ni][mi][i]);
        const int b = ni * MI + mi;
#pragma unroll
        for (int i = 0; i <= TB_LD_PER_WAVE; ++i) {
          if (min(2 * i + 1, NB - 1) == b && istep >= 0) {
            __builtin_amdgcn_sched_barrier(0);
            issue_one(istep, i);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
    set_prio(false);
  };
  auto barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };
  {
    // Staggered halves: waves w and w + 4 share a SIMD (work-group waves are
    // dealt to the four SIMDs round-robin) and lie in opposite token halves
    // (stag).  Between the barriers that open
    // K-steps s and s+1 the token-half-0 waves run X(s) Y(s) and the
    // token-half-1 waves Y(s-1) X(s), so one wave's MFMAs overlap its
    // partner's VALU widening; both halves pass the same nsteps + 1 barriers,
    // one per K-step.  Stage refills ride in the Y phases: half 0 refills
    // stage s+2 in Y(s) (the slot of stage s-1, read by every wave before the
    // barrier opening s), half 1 refills stage s+3 in Y(s) (the slot of stage
    // s, read by every wave before the barrier opening s+1, which precedes
    // its Y(s)).  At each barrier a wave thus has at most one younger stage in
    // flight, as wait_stage assumes; half 1 issued stages 0..2 up front and
    // waits for 0 and 1 at the first barrier.  MI, the number of 16-token
    // sub-tiles of the wave that hold tokens (uniform per wave), picks the
    // loop instance: a partial tile of a grouped GEMM skips the empty ones.
    auto open_wait = [&](int step) {
      if (step < nsteps) wait_stage(min(nsteps - 1 - step, TB_NS - 2));
      barrier();
    };
    auto half0 = [&](auto mic) {
      for (int step = 0; step < nsteps; ++step) {
        open_wait(step);
        if constexpr (decltype(mic)::value > 0) phase_x(mic, step);
        phase_y_copy(mic, step + TB_NS - 1 < nsteps ? step + TB_NS - 1 : -1);
      }
      open_wait(nsteps);
    };
    auto half1 = [&](auto mic) {
      open_wait(0);
      for (int step = 0; step < nsteps; ++step) {
        if constexpr (decltype(mic)::value > 0) phase_x(mic, step);
        open_wait(step + 1);
        phase_y_copy(mic, step + TB_NS < nsteps ? step + TB_NS : -1);
      }
    };
    auto run = [&](auto mic) {
      if (!stag) half0(mic);
      else half1(mic);
    };
    switch (FULL ? MIX : max(0, min(MIX, (nrows - wm * TOKW + 15) / 16))) {
      case 4: if constexpr (MIX >= 4) run(IntC<4>{}); break;
      case 3: if constexpr (MIX >= 3) run(IntC<3>{}); break;
      case 2: run(IntC<2>{}); break;
      case 1: run(IntC<1>{}); break;
      default: run(IntC<0>{}); break;
    }
  }

  // ---- epilogue. acc[ni][mi][i]: weight row wfrag_row[ni] - r + 4g + i, token column r.
  if constexpr (!SILU && !SPLIT) {
    // bf16 store.  Every wave has passed the last barrier (all X phases and
    // stage copies are done), so the ring is idle: the wave stages its TOKW x 64
    // sub-tile through its own LDS rows (pitch 144 B: the 16 rows of one
    // write land on distinct banks) and stores whole 128-B row segments, 16 B
    // per lane.  Direct 8-B stores (16 rows x 32 B per instruction) took
    // ~2 us per work-group; staged, the short-K GEMMs run 10-15 % faster.
    if (nb * TB_N + wn * 64 >= N) return;  // wave's rows lie past N (N % 256 == 128)
    constexpr int PITCH = 144;
    static_assert(TB_WAVES * TOKW * PITCH <= C::kLds, "staging fits the ring");
    uint8_t* stg = lds + wave * TOKW * PITCH;
#pragma unroll
    for (int mi = 0; mi < MIX; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        u32x2 v;
        v[0] = pack_bf16x2(acc[ni][mi][0], acc[ni][mi][1]);
        v[1] = pack_bf16x2(acc[ni][mi][2], acc[ni][mi][3]);
        *reinterpret_cast<u32x2*>(stg + (mi * 16 + r) * PITCH + ni * 32 + g * 8) = v;
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's own rows are written
    const int chunk = lane & 7;
#pragma unroll
    for (int it = 0; it < TOKW / 8; ++it) {
      const int rw = it * 8 + (lane >> 3);
      const int tl = wm * TOKW + rw;  // token row inside the tile
      const u32x4 v = *reinterpret_cast<const u32x4*>(stg + rw * PITCH + chunk * 16);
      if (tl < nrows) {
        // dense: token row; grouped: the routed pair of the sorted row
        const size_t orow = GROUPED ? (size_t)p.sorted_pair[row0 + tl] : (size_t)(row0 + tl);
        *reinterpret_cast<u32x4*>(p.out + orow * N + nb * TB_N + wn * 64 + chunk * 8) = v;
      }
    }
  } else if constexpr (SILU) {
    // silu(gate) * up, bf16, to the routed pair's row (staging these 64-B
    // rows through the LDS measured no faster).
#pragma unroll
    for (int mi = 0; mi < MIX; ++mi) {
      const int tl = wm * TOKW + mi * 16 + r;  // token row inside the tile
      if (tl >= nrows) continue;
      const int pair = p.sorted_pair[row0 + tl];
      uint16_t* o = p.out + (size_t)pair * (N / 2) + nb * (TB_N / 2) + wn * 32;
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        u32x2 v;
        v[0] = pack_bf16x2(silu_mul(acc[ni][mi][0], acc[ni + 2][mi][0]), silu_mul(acc[ni][mi][1], acc[ni + 2][mi][1]));
        v[1] = pack_bf16x2(silu_mul(acc[ni][mi][2], acc[ni + 2][mi][2]), silu_mul(acc[ni][mi][3], acc[ni + 2][mi][3]));
        *reinterpret_cast<u32x2*>(o + ni * 16 + 4 * g) = v;
      }
    }
  } else {
    // split-K: fp32 partials.  As for the bf16 store, the idle ring stages the
    // wave's TOKW x 64 sub-tile (pitch 272 B: the 16 rows of one write land on
    // distinct banks), so that each store writes four whole 256-B row segments
    // instead of 64-B quarters of 16 rows.  (Non-temporal partial stores were
    // 3 % faster back to back but 6 % slower after the reference's write
    // flush, which leaves the caches full of dirty lines; they stay cached.)
    if (nb * TB_N + wn * 64 >= N) return;  // wave's rows lie past N
    constexpr int PITCH = 272;
    static_assert(TB_WAVES * TOKW * PITCH <= C::kLds, "staging fits the ring");
    uint8_t* stg = lds + wave * TOKW * PITCH;
#pragma unroll
    for (int mi = 0; mi < MIX; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
        *reinterpret_cast<f32x4*>(stg + (mi * 16 + r) * PITCH + ni * 64 + g * 16) = acc[ni][mi];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's own rows are written
    const int chunk = lane & 15;
#pragma unroll
    for (int it = 0; it < TOKW / 4; ++it) {
      const int rw = it * 4 + (lane >> 4);
      const int tl = wm * TOKW + rw;  // token row inside the tile
      const f32x4 v = *reinterpret_cast<const f32x4*>(stg + rw * PITCH + chunk * 16);
      if (tl < nrows)
        *reinterpret_cast<f32x4*>(p.partial + ((size_t)blockIdx.y * p.M + row0 + tl) * N + nb * TB_N + wn * 64 +
                                  chunk * 4) = v;
    }
  }
}

}  // namespace ferret

using namespace ferret;

template <bool SILU, bool GROUPED, int WN, bool SPLIT, bool FULL, bool F8, int TW>
static int launch_tiled_one(const TiledArgs& p, dim3 grid, hipStream_t st) {
  using C = TileCfg<WN, TW>;
  FERRET_HIP_CHECK((set_lds_limit_once<fp8_tiled_kernel<SILU, GROUPED, WN, SPLIT, FULL, F8, TW>>(C::kLds)));
  hipLaunchKernelGGL((fp8_tiled_kernel<SILU, GROUPED, WN, SPLIT, FULL, F8, TW>), grid, dim3(C::kThreads), C::kLds,
                     st, p);
  return (int)hipGetLastError();
}

// f8: the FP8-MFMA instance (FERRET_FP8_MMA_E4M3), else the exact bf16 one.
template <bool SILU, bool GROUPED, int WN, bool SPLIT, bool FULL, int TW = 2>
static int launch_tiled(const TiledArgs& p, dim3 grid, hipStream_t st, bool f8) {
  return f8 ? launch_tiled_one<SILU, GROUPED, WN, SPLIT, FULL, true, TW>(p, grid, st)
            : launch_tiled_one<SILU, GROUPED, WN, SPLIT, FULL, false, TW>(p, grid, st);
}

// Split-K plan for small M: 128 x 128 tiles (8 waves) over K ranges, the
// number of splits the largest power of two whose grid still fits the 256 CUs
// in one round (one 97.5-KB work-group per CU): a grid of 448 at
// 128 x 7168 x 2048 ran in two rounds, 26.5 us against 15.7 us with 224.
// At 128 x 4096 x 7168 (256 work-groups) this beat 64 x 128 and 256 x 128
// tiles and two work-groups per CU (28 us vs 29-36 us).  Returns the number
// of splits (1 = no split-K).
constexpr int SPLITK_WN = 2;         // 128 x 128 tiles
constexpr int SPLITK_TW = 4;         // of 8 waves (64 x 32 each, two per SIMD)
constexpr int SPLITK_TARGET = 256;   // work-groups the split grid may not exceed (one per CU)
static int splitk_splits(int M, int N, int K) {
  if (M > 256 || N % (64 * SPLITK_WN) != 0) return 1;
  const int tiles = (N / (64 * SPLITK_WN)) * ((M + TB_M - 1) / TB_M);
  const int nkb = K / TB_K;
  int s = 1;
  while (tiles * s * 2 <= SPLITK_TARGET && s * 2 <= nkb / 2) s *= 2;
  return s;
}

size_t ferret_fp8_gemm_workspace(int M, int N, int K) {
  const int s = splitk_splits(M, N, K);
  return s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
}

int ferret_fp8_gemm_tiled(const void* a, const float* sa, const void* b, const float* sb, void* c, int M,
                          int N, int K, void* ws, size_t ws_bytes, bool f8, hipStream_t st) {
  TiledArgs p{};
  p.a = static_cast<const uint8_t*>(a);
  p.sa = sa;
  p.b = static_cast<const uint8_t*>(b);
  p.sb = sb;
  p.out = static_cast<uint16_t*>(c);
  p.M = M;
  p.N = N;
  p.K = K;
  p.m_blocks = (M + TB_M - 1) / TB_M;
  const int splits = splitk_splits(M, N, K);
  const size_t need = ferret_fp8_gemm_workspace(M, N, K);
  if (splits > 1 && ws != nullptr && ws_bytes >= need) {
    const int nkb = K / TB_K;
    p.k_steps = (nkb + splits - 1) / splits;
    const int used = (nkb + p.k_steps - 1) / p.k_steps;  // splits actually holding K-steps
    p.partial = static_cast<float*>(ws);
    p.n_blocks = N / (64 * SPLITK_WN);
    const dim3 grid(p.n_blocks * p.m_blocks, used);
    const int rc = M % TB_M == 0 ? launch_tiled<false, false, SPLITK_WN, true, true, SPLITK_TW>(p, grid, st, f8)
                                 : launch_tiled<false, false, SPLITK_WN, true, false, SPLITK_TW>(p, grid, st, f8);
    if (rc != 0) return rc;
    const size_t n4 = (size_t)M * N / 4;
    auto* reduce = used == 2 ? splitk_reduce_kernel<2> : used == 4 ? splitk_reduce_kernel<4>
                 : used == 8 ? splitk_reduce_kernel<8> : splitk_reduce_kernel<0>;
    hipLaunchKernelGGL(reduce, dim3(512), dim3(256), 0, st, p.partial, used, n4, static_cast<uint16_t*>(c));
    return (int)hipGetLastError();
  }
  // Mid M: where the 256 x 128 grid would fill at most half of the CUs
  // (DSv3 q_b_proj at M = 512: 48 work-groups, each over all of K), the
  // 128 x 128 tiles of the split-K configuration double it while it still
  // fits one round, and store bf16 directly.
  const int t256 = ((N + 255) / 256) * p.m_blocks;
  const int t128 = (N / (64 * SPLITK_WN)) * p.m_blocks;
  if (2 * t256 <= SPLITK_TARGET && t128 <= SPLITK_TARGET) {
    p.n_blocks = N / (64 * SPLITK_WN);
    if (M % TB_M == 0) return launch_tiled<false, false, SPLITK_WN, false, true, SPLITK_TW>(p, dim3(t128), st, f8);
    return launch_tiled<false, false, SPLITK_WN, false, false, SPLITK_TW>(p, dim3(t128), st, f8);
  }
  // Dense tiles: with every token tile full (M % 128 == 0) the kernel skips
  // the per-wave count of occupied 16-token sub-tiles.
  p.n_blocks = (N + 255) / 256;
  if (M % TB_M == 0) return launch_tiled<false, false, 4, false, true>(p, dim3(p.n_blocks * p.m_blocks), st, f8);
  return launch_tiled<false, false, 4, false, false>(p, dim3(p.n_blocks * p.m_blocks), st, f8);
}

int ferret_moe_w13_fp8_tiled(const void* x, const float* sx, const void* w, const float* sw,
                             const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                             int max_tiles, int topk, int N, int K, void* out, bool f8, hipStream_t st) {
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
  p.n_blocks = (N / 2) / 128;
  const long long grid = (long long)max_tiles * p.n_blocks;
  if (grid <= 0) return FERRET_OK;
  if (grid >= (1LL << 31)) return FERRET_ERR_SHAPE;
  return launch_tiled<true, true, 4, false, false>(p, dim3((unsigned)grid), st, f8);
}

// Prefill-sized MoE w2 / down projection: grouped tiles, bf16 store to the
// routed pair's row; the A row of a sorted row is its pair too (topk = 1).
int ferret_moe_w2_fp8_tiled(const void* h, const float* sh, const void* w, const float* sw,
                            const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                            int max_tiles, int N, int K, void* out, bool f8, hipStream_t st) {
  TiledArgs p{};
  p.a = static_cast<const uint8_t*>(h);
  p.sa = sh;
  p.b = static_cast<const uint8_t*>(w);
  p.sb = sw;
  p.out = static_cast<uint16_t*>(out);
  p.sorted_pair = sorted_pair;
  p.tiles = tiles;
  p.ntiles = ntiles;
  p.topk = 1;
  p.N = N;
  p.K = K;
  p.n_blocks = (N + TileCfg<4>::kN - 1) / TileCfg<4>::kN;
  const long long grid = (long long)max_tiles * p.n_blocks;
  if (grid <= 0) return FERRET_OK;
  if (grid >= (1LL << 31)) return FERRET_ERR_SHAPE;
  return launch_tiled<false, true, 4, false, false>(p, dim3((unsigned)grid), st, f8);
}
