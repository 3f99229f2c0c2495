// Persistent weight-streaming GEMM for decode-sized token tiles (<= 16 tokens)
// on gfx950: the HBM-bound bf16 / FP8 / INT4 linear projections and MoE w13
// grouped GEMMs.
//
// Work decomposition.  A unit is (token tile, RB blocks of 16 weight rows); a
// work-group of NW waves owns a contiguous range of units (a persistent grid
// of one work-group per CU), and within a unit wave w takes the K-steps
// [w*KS, (w+1)*KS) (one K-step = 128 K = one fp32 scale block), so the unit's
// partial sums meet once, in LDS, at the end of the unit.
//
// Data movement.  Weights go global -> LDS with global_load_lds_dwordx4
// (no VGPR staging) into a ring of D stages private to each wave; every bf16 /
// FP8 DMA instruction reads complete 128-byte lines (8 lanes per line), a
// tiled-INT4 (kINT4T) one a contiguous KB, and a checkpoint-layout INT4 one
// 16 half lines (64 B of each of 16 rows).  A wave waits
// only for its own copies (vmcnt), so the main loop has no barrier, and the
// ring runs ahead across unit boundaries.  LDS rows keep their 16-byte chunks
// XOR-swizzled so the MFMA fragment reads are free of bank conflicts.  The
// tile's activations (and FP8 activation scales) are loaded once per token
// tile into registers: a wave holds its K-range of x for the whole range of
// units that share the tile.
//
// Math (swap-AB): weight rows are the MFMA A side, tokens the B side; lane
// (r, g) of a 16x16x32 bf16 MFMA j carries K = 32g + 8j .. +8 of the K-step
// for both operands.  FP8 weights are widened to bf16 (exact) and each K-step
// is folded into the fp32 accumulator with sa * sb; INT4 words are dequantized
// to bf16 = RNE((q - 8) * s) (the group-32 scale sits in the stage next to the
// weights).
#pragma once
#include "skinny_kernel.hpp"
#include "stream_plan.hpp"

namespace ferret {

template <int F>
struct StreamFmt;
template <>
struct StreamFmt<kBF16> {
  static constexpr int kRowB = 256;  // bytes of one weight row per K-step
  static constexpr int kInstr = 4;   // 1-KB DMA instructions per 16-row block and K-step
};
template <>
struct StreamFmt<kFP8> {
  static constexpr int kRowB = 128;
  static constexpr int kInstr = 2;
};
template <>
struct StreamFmt<kINT4> {
  static constexpr int kRowB = 64;
  static constexpr int kInstr = 1;
};
template <>
struct StreamFmt<kINT4T> : StreamFmt<kINT4> {};

template <int F, int RB, int NW, int KS, int D>
struct StreamCfg {
  static constexpr int kWBytes = RB * 16 * StreamFmt<F>::kRowB;       // weights of one stage
  // FP8: + 256 B per stage for the 128 x 128 weight-block scale of each row block.
  static constexpr int kStage = kWBytes + (F == kFP8 ? 256 : 0);
  static constexpr int kLoads = RB * StreamFmt<F>::kInstr + (F == kFP8 ? 1 : 0);  // DMA ops per stage
  // Activation loads of one K-step (vector loads: FP8 two 16-B loads and the
  // scale, bf16 / INT4 four 16-B loads).
  static constexpr int kXLoads = F == kFP8 ? 3 : 4;
  static constexpr int kRing = D * kStage;                            // per wave
  // INT4: the group scales of a unit (RB * 16 rows x this wave's KS K-steps,
  // 8 B per row and K-step) are copied once per unit as whole 16-B chunks:
  // kSclCh chunks per row cover the wave's (8-B aligned) span, double-buffered
  // by unit parity; kSclLoads DMA ops (16 B per lane) per unit.  kSclCh is
  // odd (a spare chunk pads an even count): the 16 rows one read touches then
  // sit at 8 distinct 16-B bank groups, two rows each, where an even row
  // stride of 64 B would pile 8 rows onto each of two groups.
  static constexpr int kSclCh = ((KS * 8 + 8 + 15) / 16) | 1;
  static constexpr int kSclBuf = RB * 16 * kSclCh * 16;
  static constexpr int kSclLoads = is_int4(F) ? (RB * 16 * kSclCh + 63) / 64 : 0;
  static constexpr int kScl = is_int4(F) ? 2 * kSclBuf : 0;            // per wave
  static constexpr int kRed = NW * RB * kRedBlock * 4;                // one reduction buffer
  static constexpr int kTiles = kStreamMaxTiles * 3 * 4;              // grouped tile table
  // LDS layout, in this order: each wave's ring and INT4 scale buffers, the
  // two reduction buffers, the tile table (the kernel takes every offset from
  // here).
  static constexpr int kWaveBytes = kRing + kScl;
  static constexpr int kRedOff = NW * kWaveBytes;
  static constexpr int kTileOff = kRedOff + 2 * kRed;
  static constexpr int kLds = kTileOff + kTiles;
  static_assert(kRedOff % 16 == 0 && kTileOff % 16 == 0, "LDS regions 16-byte aligned");
  static_assert(kTileOff + kStreamMaxTiles * 3 * (int)sizeof(int) == kLds, "the tile table ends the LDS");
  static_assert(!is_int4(F) || D <= KS, "INT4 unit scales are double-buffered: at most one unit ahead");
  static_assert(kLds <= 160 * 1024, "LDS budget");
  // Step s reads the fragments of step s + 1 before refilling, so item s + 1
  // must already be in flight: at least two stages per wave.
  static_assert(D >= 2, "ring depth");
  static_assert(D * (kLoads + kXLoads) + kSclLoads < 64, "vmcnt range");
  // First token tile's activations interleaved with its weight items: when the
  // ring prologue and the first unit's refills reach at most one unit ahead.
  static constexpr bool kInterleave = D <= KS;
};

// Chunk slot of global 16-byte chunk c of LDS row `row` (per row width).
// A ds_read_b128 is served 8 lanes at a time over 128 B of banks, so the 8
// rows that lanes r..r+7 read (same chunk c) must land on 8 distinct 16-B
// bank groups; with a 64-B int4 row that takes the key (row >> 1) & 3.
__device__ __forceinline__ int sw_bf16(int row, int c) { return c ^ (((row & 7) << 1) | ((row >> 3) & 1)); }
__device__ __forceinline__ int sw_fp8(int row, int c) { return c ^ ((row & 7) ^ ((row >> 3) & 1)); }
__device__ __forceinline__ int sw_int4(int row, int c) { return c ^ ((row >> 1) & 3); }

// Wait until item S of a unit (K-step S of KS) has landed, while the
// min(n, N) items issued after it may stay in flight: each item is L DMA ops,
// and the first item of a unit also carries SI ops (the unit's INT4 scales),
// so one of those later items adds SI when the next unit starts within them.
template <int L, int SI, int KS, int S, int N>
__device__ __forceinline__ void wait_items(int n) {
  if constexpr (N == 0) {
    wait_vmcnt<0>();
  } else {
    if (n >= N) {
      wait_vmcnt<N * L + ((KS - S) <= N ? SI : 0)>();
      return;
    }
    wait_items<L, SI, KS, S, N - 1>(n);
  }
}

// Items issued after step s+1's item that may stay in flight while step s
// waits for it: D - 2, one fewer at an odd step when refills go in pairs (the
// even step before it refilled nothing).
constexpr int ring_younger(int D, bool PAIR, int s) {
  return (D >= 2 ? D - 2 : 0) - ((PAIR && (s & 1) != 0) ? 1 : 0);
}

// Vector-memory ops issued after item S of the first unit of the first token
// tile, up to item S + N: item i < KS is preceded by the LX activation loads
// of K-step i, and the next unit's first item carries SI.
constexpr int first_unit_ops(int L, int LX, int SI, int KS, int S, int N) {
  int ops = 0;
  for (int i = S + 1; i <= S + N; ++i) ops += L + (i < KS ? LX : 0) + (i % KS == 0 ? SI : 0);
  return ops;
}
template <int L, int LX, int SI, int KS, int S, int N>
constexpr int first_unit_ops() {
  return first_unit_ops(L, LX, SI, KS, S, N);
}

// Replays the first unit's issue order -- the ring prologue, then after each
// K-step its refill (two after every odd step when PAIR), each item of this
// unit preceded by its K-step's LX activation loads and item 0 of each unit
// followed by its SI scale ops -- and checks that every counted wait in it
// (first_unit_ops) leaves no op of the item it waits for, or of its
// activations, among the ops still allowed in flight.
template <int L, int LX, int SI, int KS, int D, bool PAIR>
constexpr bool first_unit_waits_ok() {
  int issued = 0;
  int end_of[2 * 16] = {};  // one past each item's last op; items < KS + D <= 2 KS
  auto item = [&](int i) {
    issued += (i < KS ? LX : 0) + L + (i % KS == 0 ? SI : 0);
    end_of[i] = issued;
  };
  for (int d = 0; d < D; ++d) item(d);
  if (end_of[0] > issued - first_unit_ops(L, LX, SI, KS, 0, D - 1)) return false;
  for (int s = 0; s < KS; ++s) {
    if (s + 1 < KS) {
      const int NY = ring_younger(D, PAIR, s);
      if (end_of[s + 1] > issued - first_unit_ops(L, LX, SI, KS, s + 1, NY)) return false;
    }
    if (PAIR) {
      if ((s & 1) != 0) {
        item(s - 1 + D);
        item(s + D);
      }
    } else {
      item(s + D);
    }
  }
  return true;
}

// s_waitcnt lgkmcnt(0) only (LDS writes done before a barrier).
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// The weight fragments of one K-step held by a lane: 16-byte LDS chunks per
// 16-row block (bf16 4, fp8 2, int4 1) and the block's scale (fp8 weight-block
// scale; int4 group scale).
template <int F, int RB>
struct StepFrag {
  u32x4 w[RB][F == kBF16 ? 4 : (F == kFP8 ? 2 : 1)];
  float sv[RB];
};

// tile_slots: dense, the token tiles of M; grouped, the rows of the tile table
// (max_tiles), which bounds the device-side count a.ntiles[0].
template <int F, int EPI, int RB, int NW, int KS, int D>
__global__ __launch_bounds__(NW * 64) void stream_gemm_kernel(SkinnyArgs a, int tile_slots) {
  using C = StreamCfg<F, RB, NW, KS, D>;
  constexpr int ROWB = StreamFmt<F>::kRowB;
  constexpr int NI = StreamFmt<F>::kInstr;
  constexpr int L = C::kLoads;
  // Paired refills for the 4-wave bf16 configuration (>= 4 row units per CU:
  // GateUp 34.9 -> 34.4 us, LMHead 192.5 -> 189.0 us; the 8-wave split-K
  // products and the FP8 kernels measured no gain).  They need units of an even
  // number of K-steps (step parity = item parity) and >= 3 ring stages.
  constexpr bool PAIR = F == kBF16 && NW == 4 && KS % 2 == 0 && D >= 3;
  static_assert(!C::kInterleave || first_unit_waits_ok<C::kLoads, C::kXLoads, C::kSclLoads, KS, D, PAIR>(),
                "first unit: a counted wait leaves its item in flight");
  static_assert(EPI != kSilu || RB == 2, "SiLU units pair one gate and one up block");
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15;
  const int g = lane >> 4;
  const bool grouped = a.tiles != nullptr;
  const int N = a.N, K = a.K;
  const int nkb = K >> 7;
  const size_t wrow_bytes = (size_t)K * ROWB / 128;

  // ---- this work-group's units
  // The grouped count is clamped to the table's rows: the host's launch plan
  // (units per work-group, the LDS span of the table) assumes ntiles <= max_tiles.
  const int ntiles = grouped ? min(max(__builtin_amdgcn_readfirstlane(a.ntiles[0]), 0), tile_slots) : tile_slots;
  // bf16 dense split-K: work item u = split * (ntiles * units_n) + unit; the
  // item's waves cover K-steps [(split * NW + kw) * KS, ... + KS).
  const int nsplit = (F == kBF16 && !grouped && a.partial != nullptr) ? a.ksplit : 1;
  // K-range kw of this wave.  Split-K work-groups rotate it by their index, so
  // that the first requests of concurrent work-groups fall on different
  // K-ranges of their rows (bf16 QKV: 13.7 -> 13.2 us at M = 16, 12.5 -> 12.1
  // at M = 1; Down, three splits: +0.6 %); the unit's cross-wave sum still runs
  // in K-range order, so results do not change.
  const int krot = nsplit > 1 ? (int)(blockIdx.x % NW) : 0;
  const int kw = __builtin_amdgcn_readfirstlane((wave + krot) % NW);
  const int units_per_split = ntiles * a.units_n;
  const int units = units_per_split * nsplit;
  const int per = (units + gridDim.x - 1) / gridDim.x;
  const int u_begin = min(units, (int)blockIdx.x * per);
  const int u_end = min(units, u_begin + per);
  const int n_items = (u_end - u_begin) * KS;
  if (n_items == 0) return;

  uint8_t* ring = lds + wave * C::kWaveBytes;
  uint8_t* sclbuf = ring + C::kRing;  // INT4 unit scales (two buffers)
  float* red = reinterpret_cast<float*>(lds + C::kRedOff);
  int* tinfo = reinterpret_cast<int*>(lds + C::kTileOff);

  // Grouped: copy this work-group's rows of the tile table to LDS once, so the
  // loop reads them without vector-memory loads (which would drain the ring).
  const int t_first = (u_begin % units_per_split) / a.units_n;  // grouped: nsplit == 1
  if (grouped) {
    const int t_last = (u_end - 1) / a.units_n;
    for (int i = threadIdx.x; i < 3 * (t_last - t_first + 1); i += NW * 64) tinfo[i] = a.tiles[3 * t_first + i];
    __syncthreads();
  }

  // Row block rb of unit-in-tile nu: first weight row.
  auto block_row = [&](int nu, int rb) {
    if constexpr (EPI == kSilu) return rb == 0 ? nu * 16 : N / 2 + nu * 16;
    else return (nu * RB + rb) * 16;
  };
  auto tile_expert = [&](int tile) { return grouped ? tinfo[3 * (tile - t_first)] : 0; };

  // ---- DMA issue cursor (uniform): unit iu, K-step is of this wave.
  // Lane offsets inside a 16-row block are the same for every unit.
  uint32_t lane_off[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    int row, slot;
    if constexpr (F == kBF16) { row = 4 * i + (lane >> 4); slot = lane & 15; }
    else if constexpr (F == kFP8) { row = 8 * i + (lane >> 3); slot = lane & 7; }
    else { row = lane >> 2; slot = lane & 3; }
    int c;
    if constexpr (F == kBF16) c = sw_bf16(row, slot);
    else if constexpr (F == kFP8) c = sw_fp8(row, slot);
    else c = sw_int4(row, slot);
    // kINT4T: the 16 rows x 64 B of a block's K-step are one contiguous KB.
    lane_off[i] = (uint32_t)row * (F == kINT4T ? 64u : (uint32_t)wrow_bytes) + c * 16;
  }
  int iu = u_begin, is = 0;
  const uint8_t* ibase[RB];
  const uint8_t* isc = nullptr;  // FP8: this lane's per-stage scale source for the unit
  // INT4: this wave's span of a scale row is [s_start, s_start + KS*8) bytes;
  // copy op q, lane l covers chunk (q*64 + l) % kSclCh of unit row (q*64 + l) / kSclCh.
  constexpr int SCH = C::kSclCh, SI = C::kSclLoads;
  const int s_start = kw * KS * 8;
  const int s_a0 = s_start & ~15;
  const int s_nch = (s_start + KS * 8 - s_a0 + 15) / 16;
  const uint8_t* sc_src[SI > 0 ? SI : 1];
  bool sc_live[SI > 0 ? SI : 1];
  auto set_issue_unit = [&](int u) {
    const int su = u % units_per_split;
    const int tile = su / a.units_n, nu = su % a.units_n;
    const int kstep0 = ((u / units_per_split) * NW + kw) * KS;  // first K-step of this wave
    const int e = tile_expert(tile);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      ibase[rb] = F == kINT4T
                      ? a.w + (((size_t)e * (N >> 4) + (block_row(nu, rb) >> 4)) * nkb + kstep0) * (size_t)1024
                      : a.w + ((size_t)e * N + block_row(nu, rb)) * wrow_bytes + (size_t)kstep0 * ROWB;
    if constexpr (is_int4(F)) {
#pragma unroll
      for (int q = 0; q < SI; ++q) {
        const int idx = q * 64 + lane, row = idx / SCH, ch = idx % SCH;
        sc_live[q] = row < RB * 16 && ch < s_nch;
        const int rr = min(row, RB * 16 - 1);
        sc_src[q] = static_cast<const uint8_t*>(a.w_scale) +
                    ((size_t)e * N + block_row(nu, rr >> 4) + (rr & 15)) * (size_t)(K >> 4) + s_a0 + ch * 16;
      }
    } else if constexpr (F == kFP8) {
      // lane l < RB: the 128 x 128 weight-scale of block l (other lanes repeat the last)
      const int rb = min(lane, RB - 1);
      isc = static_cast<const uint8_t*>(a.w_scale) +
            (((size_t)e * (N >> 7) + (block_row(nu, rb) >> 7)) * (size_t)nkb + (size_t)kw * KS) * 4;
    }
  };
  auto issue = [&](int slot) {
    uint8_t* st = ring + slot * C::kStage;
    // Weight rows are streamed once: non-temporal, except checkpoint-layout
    // INT4, whose 64-byte row slice per K-step is half a line -- the other half
    // is the wave's next K-step and must still be in L2 when it is read.  A
    // kINT4T op reads one whole KB (its tile: 8 complete lines).
    constexpr size_t kStepB = F == kINT4T ? 1024 : ROWB;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const uint8_t* src = ibase[rb] + (size_t)is * kStepB + lane_off[i];
        if constexpr (F == kINT4) g2l_16(src, st + (rb * NI + i) * 1024);
        else g2l_16_nt(src, st + (rb * NI + i) * 1024);
      }
    if constexpr (F == kFP8) g2l_4(isc + is * 4, st + C::kWBytes);
    if constexpr (is_int4(F)) {
      if (is == 0) {
        uint8_t* sb = sclbuf + (iu & 1) * C::kSclBuf;
#pragma unroll
        for (int q = 0; q < SI; ++q)
          if (sc_live[q]) g2l_16(sc_src[q], sb + q * 1024);
      }
    }
    if (++is == KS) {
      is = 0;
      if (++iu < u_end) set_issue_unit(iu);
    }
  };

  // ---- activations of the current token tile (registers), per K-step of this wave
  constexpr int XV = (F == kFP8) ? 2 : 4;
  u32x4 xv[KS][XV];
  float sx[KS];
  int cur_tile = -1;
  int my_pair = 0;  // grouped: routed pair of token column r (from sorted_pair)
  int nrows = 0, row0 = 0;
  int cur_split = -1;
  int tok = 0;  // activation row of this lane's token column
  auto set_tile = [&](int u) {
    const int split = u / units_per_split;
    const int tile = (u % units_per_split) / a.units_n;
    cur_tile = tile;
    cur_split = split;
    if (grouped) {
      row0 = tinfo[3 * (tile - t_first) + 1];
      nrows = tinfo[3 * (tile - t_first) + 2];
    } else {
      row0 = tile * 16;
      nrows = min(16, a.M - row0);
    }
    // columns >= nrows compute garbage, never stored (a zero-row tile reads row row0)
    const int tcol = max(0, min(r, nrows - 1));
    tok = row0 + tcol;
    if (grouped) {
      my_pair = a.sorted_pair[row0 + tcol];
      tok = my_pair / a.topk;
    }
  };
  // Activations of this wave's K-step k of the current tile and split:
  // C::kXLoads vector loads.
  auto load_x = [&](int k) {
    const int ks = (cur_split * NW + kw) * KS + k;
    if constexpr (F == kFP8) {
      const uint8_t* xp = a.x + (size_t)tok * K + (size_t)ks * 128 + 32 * g;
      xv[k][0] = ld_u32x4(xp);
      xv[k][1] = ld_u32x4(xp + 16);
      sx[k] = a.x_scale[(size_t)tok * nkb + ks];
    } else {
      const uint8_t* xp = a.x + ((size_t)tok * K + (size_t)ks * 128 + 32 * g) * 2;
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[k][j] = ld_u32x4(xp + 16 * j);
    }
  };
  f32x4 acc[RB];
  int buf = 0;

  // One unit.  FIRST: the work-group's first unit with more to follow, its
  // activations interleaved with its weight items (below); its refills then
  // always reach the next unit (D <= KS), so every issue and wait in it is
  // unconditional and the compiler counts the vector-memory ops ahead of each
  // activation use exactly instead of waiting for all of them.  Otherwise a
  // unit of another token tile (or split) loads its activations all at once.
  auto run_unit = [&](auto firstc, int u) {
    constexpr bool first = decltype(firstc)::value;
    const int split = u / units_per_split;
    const int tile = (u % units_per_split) / a.units_n;
    const int nu = u % a.units_n;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (!first && (tile != cur_tile || split != cur_split)) {
      set_tile(u);
#pragma unroll
      for (int k = 0; k < KS; ++k) load_x(k);
      wait_vmcnt<0>();  // drains the ring as well
    }

    const uint8_t* sb_unit = sclbuf + (u & 1) * C::kSclBuf;
    // One K-step's weight fragments (and their scales), read from its stage.
    auto load_frag = [&](StepFrag<F, RB>& fr, int slot, int s) {
      const uint8_t* st = ring + slot * C::kStage;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const uint8_t* blk = st + rb * 16 * ROWB + r * ROWB;
        if constexpr (F == kBF16) {
#pragma unroll
          for (int j = 0; j < 4; ++j) fr.w[rb][j] = *reinterpret_cast<const u32x4*>(blk + (sw_bf16(r, 4 * g + j) << 4));
        } else if constexpr (F == kFP8) {
          fr.w[rb][0] = *reinterpret_cast<const u32x4*>(blk + (sw_fp8(r, 2 * g) << 4));
          fr.w[rb][1] = *reinterpret_cast<const u32x4*>(blk + (sw_fp8(r, 2 * g + 1) << 4));
          fr.sv[rb] = *reinterpret_cast<const float*>(st + C::kWBytes + 4 * rb);
        } else {
          fr.w[rb][0] = *reinterpret_cast<const u32x4*>(blk + (sw_int4(r, g) << 4));
          fr.sv[rb] = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(
              sb_unit + (rb * 16 + r) * (SCH * 16) + (s_start - s_a0) + s * 8 + g * 2));
        }
      }
    };
    auto compute = [&](const StepFrag<F, RB>& fr, auto sc) {
      constexpr int s = decltype(sc)::value;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        if constexpr (F == kBF16) {
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[rb] = mfma_bf16_16x16x32(fr.w[rb][j], xv[s][j], acc[rb]);
        } else if constexpr (F == kFP8) {
          const f32x4 part = fp8_block_16x16x128(fr.w[rb][0], fr.w[rb][1], xv[s][0], xv[s][1]);
          const float scl = sx[s] * fr.sv[rb];
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[rb][i] = fmaf(part[i], scl, acc[rb][i]);
        } else {
          const Int4Scale ks4 = int4_scale(fr.sv[rb]);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[rb] = mfma_bf16_16x16x32(dequant_int4x8(fr.w[rb][0][j], ks4), xv[s][j], acc[rb]);
        }
      }
    };

    // Software pipeline over the unit's K-steps: the fragments of step s+1 are
    // read from LDS while step s computes, so the LDS latency hides behind the
    // MFMA/dequant work of the same wave.
    StepFrag<F, RB> cur;
    {
      const int it0 = (u - u_begin) * KS;
      if constexpr (first) {
        wait_vmcnt<first_unit_ops<L, C::kXLoads, SI, KS, 0, D - 1>()>();
      } else {
        wait_items<L, SI, KS, 0, D - 1>(min(D - 1, n_items - 1 - it0));
      }
      __builtin_amdgcn_sched_barrier(0);
      load_frag(cur, it0 % D, 0);
    }
    static_for<0, KS>([&](auto sc) {
      constexpr int s = decltype(sc)::value;
      const int it = (u - u_begin) * KS + s;
      StepFrag<F, RB> nxt;
      if constexpr (s + 1 < KS) {
        // Wait for step s+1's stage (items issued after it may stay in flight:
        // D - 2, one fewer after an even step when refills go out in pairs).
        constexpr int NY = ring_younger(D, PAIR, s);
        if constexpr (first) {
          wait_vmcnt<first_unit_ops<L, C::kXLoads, SI, KS, s + 1, NY>()>();
        } else {
          wait_items<L, SI, KS, s + 1, NY>(min(NY, n_items - 2 - it));
        }
        __builtin_amdgcn_sched_barrier(0);
        load_frag(nxt, (it + 1) % D, s + 1);
      }
      compute(cur, sc);
      __builtin_amdgcn_sched_barrier(0);
      // Refill the slot of step s (its fragments were consumed above).  Paired:
      // after each odd step refill the slots of both steps, so the wave asks for
      // two consecutive K-steps (512 B) of each of its rows at once.
      // In the first unit, the activations of a refilled item's K-step (when it
      // lies in this unit) go right before it.
      if constexpr (PAIR) {
        if constexpr ((s & 1) != 0) {
          if constexpr (first && s - 1 + D < KS) {
            load_x(s - 1 + D);
            __builtin_amdgcn_sched_barrier(0);
            issue((s - 1) % D);
          } else if constexpr (first) {
            issue((s - 1) % D);
          } else if (it - 1 + D < n_items) {
            issue((it - 1) % D);
          }
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (first && s + D < KS) {
            load_x(s + D);
            __builtin_amdgcn_sched_barrier(0);
            issue(s % D);
          } else if constexpr (first) {
            issue(s % D);
          } else if (it + D < n_items) {
            issue(it % D);
          }
        }
      } else {
        if constexpr (first && s + D < KS) {
          load_x(s + D);
          __builtin_amdgcn_sched_barrier(0);
          issue(s % D);
        } else if constexpr (first) {
          issue(s % D);
        } else if (it + D < n_items) {
          issue(it % D);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (s + 1 < KS) cur = nxt;
    });

    // ---- unit end: cross-wave K reduction through LDS, then the epilogue.
    // Each wave's partial goes to the slot of its K-range, so the sums below
    // add the K-ranges in order whatever the rotation.
    float* rb_base = red + buf * (C::kRed / 4);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) rb_base[(kw * RB + rb) * kRedBlock + r * kRedStride + 4 * g + i] = acc[rb][i];
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (EPI == kStore) {
      for (int idx = threadIdx.x; idx < RB * 256; idx += NW * 64) {
        const int part = idx >> 8, t = (idx >> 4) & 15, row = idx & 15;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += rb_base[(w * RB + part) * kRedBlock + t * kRedStride + row];
        // dense: token row; grouped: the routed pair of column t (held by lane t;
        // every wave runs this loop a uniform number of times)
        const int orow = grouped ? __shfl(my_pair, t, 64) : row0 + t;
        const size_t o = (size_t)orow * N + block_row(nu, part) + row;
        if (t < nrows) {
          if (nsplit > 1) {
            a.partial[(size_t)split * a.M * N + o] = v;  // summed (+ residual) by the reduce kernel
          } else {
            if (a.residual) v += bf16_bits_to_f32(a.residual[o]);
            a.out[o] = f32_to_bf16_bits(v);
          }
        }
      }
    } else {
      const int idx = threadIdx.x;
      const int t = (idx >> 4) & 15, row = idx & 15;
      // pair of token column t: held by lane t of every wave
      const int pair = __shfl(my_pair, t, 64);
      if (idx < 256 && t < nrows) {
        float gs = 0.f, us = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          gs += rb_base[(w * RB + 0) * kRedBlock + t * kRedStride + row];
          us += rb_base[(w * RB + 1) * kRedBlock + t * kRedStride + row];
        }
        a.out[(size_t)pair * (N / 2) + nu * 16 + row] = f32_to_bf16_bits(silu_mul(gs, us));
      }
    }
    buf ^= 1;
  };
  // First token tile.  With at least two units, the activations of each K-step
  // go out right before its weight item (the ring prologue and the first
  // unit's refills): vector memory retires in issue order, so activations
  // loaded ahead of the whole ring hold back every weight stage -- the
  // work-group's first MFMA came ~5.7 us after its start at GateUp M = 16.
  // A single unit (FP8 M = 16: interleaving it measured no gain), or a ring
  // deeper than one unit, loads all of the tile's activations first.
  set_tile(u_begin);
  set_issue_unit(iu);
  int u_next = u_begin;
  if constexpr (C::kInterleave) {
    if (u_end - u_begin > 1) {
      static_for<0, D>([&](auto dc) {
        constexpr int d = decltype(dc)::value;
        load_x(d);
        __builtin_amdgcn_sched_barrier(0);
        issue(d);
        __builtin_amdgcn_sched_barrier(0);
      });
      run_unit(IntC<1>{}, u_begin);
      u_next = u_begin + 1;
    }
  }
  if (u_next == u_begin) {
#pragma unroll
    for (int k = 0; k < KS; ++k) load_x(k);
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (d < n_items) issue(d);
  }
  for (int u = u_next; u < u_end; ++u) run_unit(IntC<0>{}, u);
}

template <int F, int EPI, int RB, int NW, int KS, int D>
static int launch_stream(const SkinnyArgs& a, int tile_slots, int grid, hipStream_t st) {
  using C = StreamCfg<F, RB, NW, KS, D>;
  FERRET_HIP_CHECK((set_lds_limit_once<stream_gemm_kernel<F, EPI, RB, NW, KS, D>>(C::kLds)));
  hipLaunchKernelGGL((stream_gemm_kernel<F, EPI, RB, NW, KS, D>), dim3(grid), dim3(NW * 64), C::kLds, st, a,
                     tile_slots);
  return (int)hipGetLastError();
}

}  // namespace ferret
