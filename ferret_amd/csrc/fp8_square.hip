// Large-M FP8 (OCP e4m3) block-scaled GEMM for gfx950: 256 x 256 tiles, for
// dense shapes with enough tiles to cover the 256 CUs (M = N = 4096, K = 7168;
// the DeepSeek-V3 attention projections from M = 2048-4096 up).
//
// Math (examples/fp8-gemm/v002_dense_tp8_validated_065.cu:277-288):
//   C[m, n] = sum_kb (sum_{k in kb} A[m,k] B[n,k]) * sa[m,kb] * sb[n/128,kb]
//
// Work-group: 512 threads = 8 waves (2 along the 256 weight rows x 4 along the
// 256 tokens, two waves per SIMD); wave tile 128 weight rows x 64 tokens, as
// 4 x 2 blocks of v_mfma_f32_32x32x16_bf16 (swap-AB: weight rows are the A
// side, tokens the B side).
//
// Widening once per work-group.  Each K-stage (64 wide, half a scale block)
// of 256 weight rows and 256 token rows is loaded by all 512 lanes (16 e4m3
// bytes per lane and row part, buffer loads two stages ahead in registers),
// widened to bf16 in registers (exact: v_cvt_scalef32_pk_bf16_fp8) and
// written to one of two 64 KB LDS slots.  A value is thus widened once per
// work-group instead of once per wave that reads it: 0.5 widening ops per
// 16x16x32-equivalent MFMA against 2 for per-wave widening of a 64 x 64 wave
// tile (measured: the widening and the MFMAs contend for the same issue port).
// The price is LDS traffic: bf16 fragments are twice the bytes of e4m3 ones,
// and at ~157 B/clk per CU (measured, 8 waves) the LDS is the next limit.
//
// Running-scale accumulation.  The fp32 accumulator of each output is kept in
// units of the current block's scale s = sa[m,kb] * sb[n/128,kb]: entering
// block kb multiplies it by r = s_prev / s_kb, then the MFMAs add the block's
// raw products into it directly; the epilogue multiplies by the last s.  That
// is one VALU multiply per accumulator and block, as a separate fold would
// be, but with no partial-sum registers, which is what lets a wave hold a
// 128 x 64 tile in its 256 VGPRs.  r carries one extra fp32 rounding per
// block (~56 * 2^-24 relative at K = 7168); r comes from the reciprocal of s
// while every s of the wave lies in [2^-125, 2^125], else from an IEEE
// division (subnormal products included).  A block whose scale product is 0
// keeps the unit and has its token fragments cleared in the lanes of those
// columns, so it adds nothing.  Precondition: scales are finite, and the
// block sums in units of each block's s stay inside the fp32 range -- with
// |a b| <= 448^2 per product that holds while the non-zero products sa * sb of
// one output span less than 2^90.
//
// Schedule.  The work of a stage is pinned to its 32 MFMA slots (see the
// stage lambda): fragment reads one substep ahead, the widening and LDS
// writes of the next stage and the loads of the one after spread over the
// first 22 slots, one barrier per stage after the stage's last LDS read, and
// the rescale spread over the 16 slots around each scale-block boundary.
//
// Reference counterpart: fp8_gemm<BN,NS> (v002:61-249), whose per-K-block
// TMEM epilogue (v002:179-210) becomes the running rescale.
#include "common.hpp"

namespace ferret {
namespace sq {

constexpr int kBW = 256;                   // weight rows per work-group
constexpr int kBT = 256;                   // tokens per work-group
constexpr int kKS = 64;                    // K per stage (half a scale block)
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kTW = 128;                   // weight rows per wave
constexpr int kTT = 64;                    // tokens per wave
constexpr int kNI = kTW / 32;              // 4 weight blocks of 32 rows per wave
constexpr int kMI = kTT / 32;              // 2 token blocks of 32 per wave
constexpr int kRowB = kKS * 2;             // a bf16 stage row: 128 B
constexpr int kWBytes = kBW * kRowB;       // 32 KB
constexpr int kSlot = kWBytes + kBT * kRowB;  // 64 KB: weights then tokens
constexpr int kRing = 2 * kSlot;           // 128 KB
constexpr int kPitch = 272;                // epilogue staging: bytes per token row (256 + 16)
constexpr int kStg = kWaves * kTT * kPitch;   // 136 KB
constexpr int kLds = kRing > kStg ? kRing : kStg;
static_assert(kLds <= 160 * 1024, "LDS budget");

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Byte offset of 16-byte chunk c (8 bf16 = 8 K) of a bf16 stage row.  The
// chunk index is XOR-swizzled with key(row) = (row & 7) ^ ((row >> 3) & 1): a
// ds_read_b128 of 16 consecutive rows (same chunk) is served 16 lanes per
// cycle over the 64 banks (256 B, two 128-B rows), so the 8 even and the 8 odd
// rows must each take 8 distinct 16-B bank groups (row & 7 alone repeats every
// 8 rows: 22 M bank-conflict cycles at M = N = 4096, K = 7168).
__device__ __forceinline__ int swz_key(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int swz(int row, int c) { return row * kRowB + ((c ^ swz_key(row)) << 4); }

// D(32 x 32 f32) += A(32 x 16 bf16) B(16 x 32 bf16): lane l holds A row /
// B column l % 32, K 8 (l / 32) .. +8; D column l % 32, rows
// 8 (i / 4) + 4 (l / 32) + i % 4 for element i.
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Slot of half `hf` (0, 1) of tile t's rescale at the scale-block boundary,
// counted from the third-to-last... see the stage comment: 0-5 = slots 26-31
// of the block's second stage, 6-12 = slots 0-6 of the next block's first.
constexpr int kRescaleSlot[8][2] = {{0, 1}, {2, 3}, {3, 4}, {5, 6}, {7, 8}, {8, 9}, {10, 11}, {11, 12}};

struct Args {
  const uint8_t* a;   // e4m3 tokens [M, K]
  const float* sa;    // [M, K/128]
  const uint8_t* b;   // e4m3 weights [N, K]
  const float* sb;    // [N/128, K/128]
  uint16_t* out;      // bf16 [M, N]
  // UE8M0 mode: packed power-of-two scale bytes instead of sa / sb (word
  // [sk, m]: token m, K-blocks 4 sk .. +3; sfb per weight row, row 128 nb
  // standing for weight block nb)
  const uint32_t* sfa;
  const uint32_t* sfb;
  int M, N, K;
  int n_blocks;       // N / 256
  int m_blocks;       // ceil(M / 256)
};

}  // namespace sq

// U8: UE8M0 block scales.  A power-of-two scale widens exactly with the value
// (v_cvt_scalef32_pk_bf16_fp8 multiplies by 2^(e - 127) of its scale
// operand's exponent e, the byte itself), so both operands enter LDS already
// scaled and the MFMAs sum absolute products: no running scale, no rescale.
template <bool U8>
__global__ __launch_bounds__(sq::kThreads) void fp8_square_kernel(sq::Args p) {
  using namespace sq;
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ww = wave & 1;     // weight half of the wave's compute tile
  const int wt = wave >> 1;    // token quarter of the wave's compute tile
  const int c32 = lane & 31;   // MFMA row (weights) / column (tokens) of the lane
  const int h = lane >> 5;     // K half of the lane's MFMA operands

  // ---- tile: each XCD (work-groups are dealt to the 8 XCDs round-robin) takes
  // a contiguous range of logical tiles, rastered in groups of 4 token tiles,
  // so the 32 work-groups resident on one XCD share 4 token and 8 weight
  // panels through its L2.
  int L = blockIdx.x;
  const int G = gridDim.x;
  if ((G & 7) == 0) L = (L & 7) * (G >> 3) + (L >> 3);
  constexpr int GM = 4;
  const int per_group = GM * p.n_blocks;
  const int first_mb = (L / per_group) * GM;
  const int gsize = min(p.m_blocks - first_mb, GM);
  const int in_group = L % per_group;
  const int mb = first_mb + in_group % gsize;
  const int nb = in_group / gsize;
  const int tok0 = mb * kBT;
  const int wrow0 = nb * kBW;
  const int tok_rows = min(kBT, p.M - tok0);  // valid token rows of the tile

  const int K = p.K;
  const int nkb = K >> 7;
  const int wbase = ww * kTW;  // first weight row of the wave's compute tile
  const int tbase = wt * kTT;  // first token of the wave's compute tile

  // ---- loads.  A stage is 256 weight rows and 256 token rows of 64 e4m3
  // bytes.  Waves 0-3 load weight rows, 4-7 token rows: part i (0..3) of a
  // lane is row 64 (wave & 3) + 16 i + lane / 4, bytes 16 (lane & 3) .. +16.
  // The lane widens its 16 bytes to bf16 (exact) and writes them as chunks
  // 2q, 2q + 1 (q = lane & 3) of the row in the stage's LDS slot, so each
  // value is widened once per work-group.  Buffer loads: token rows past M
  // fall outside the buffer and read as zeros.
  const bool loads_tokens = wave >= 4;
  const int lrows = loads_tokens ? tok_rows : kBW;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(loads_tokens ? p.a + (size_t)tok0 * K : p.b + (size_t)wrow0 * K), (short)0, lrows * K, 0x00020000);
  const int lrow = 64 * (wave & 3) + (lane >> 2);  // + 16 i
  const int q = lane & 3;
  const unsigned loff = (unsigned)(lrow * K + q * 16);
  const int lds_row0 = (loads_tokens ? kWBytes : 0) + lrow * kRowB;  // + 16 i rows
  const int wkey = swz_key(lrow);  // the same for rows lrow + 16 i
  const int wch0 = ((2 * q) ^ wkey) << 4, wch1 = ((2 * q + 1) ^ wkey) << 4;

  // UE8M0 mode: the scale word of each loaded row (4 K-blocks per byte word),
  // fetched with the stage bytes: lane q of each lane quad loads the word of
  // part q (row lrow + 16 q; a weight row reads the word of its 128-row block,
  // the same for every part) and write_part(i) takes part i's word from lane
  // i of the quad (DPP), one register per stage in flight instead of four.
  // The whole offset goes in voffset, which the buffer range check covers:
  // words past the array read as 0.
  const int nsk = (nkb + 3) >> 2;
  const __amdgpu_buffer_rsrc_t sf_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(U8 ? (loads_tokens ? p.sfa : p.sfb) : nullptr), (short)0,
      U8 ? nsk * (loads_tokens ? p.M : p.N) * 4 : 0, 0x00020000);
  const int sf_ld = loads_tokens ? p.M : p.N;  // words per sk row
  const int sf_row = loads_tokens ? tok0 + lrow + 16 * q : wrow0 + (lrow & ~127);

  // Two stages in flight in registers (stg[st & 1]): the L2 / MALL latency
  // under load is longer than one stage's compute.
  u32x4 stg[2][4];
  uint32_t sfw[2];
  auto load_part = [&](int st, int i) {
    stg[st & 1][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
        rsrc, (int)(loff + (unsigned)(16 * i * K)), st * kKS, 0));
    if constexpr (U8) {
      // with the last part: load_part(st, i) follows write_part(st - 2, i),
      // so the register is refilled only after all four parts of stage st - 2
      // have taken their word from it
      if (i == 3) sfw[st & 1] = __builtin_amdgcn_raw_buffer_load_b32(sf_rsrc, (sf_row + (st >> 3) * sf_ld) * 4, 0, 0);
    }
  };
  auto write_part = [&](int st, int i) {
    uint8_t* row = lds + (st & 1) * kSlot + lds_row0 + 16 * i * kRowB;
    const u32x4& v = stg[st & 1][i];
    if constexpr (U8) {
      // byte of K-block st / 2; a zero byte is a zero scale (the instruction
      // would take it as 2^-127), so its values are cleared instead
      // quad_perm [i, i, i, i]: the word lane i of the quad loaded
      const int wsrc = (int)sfw[st & 1];
      int word;
      switch (i) {
        case 0: word = __builtin_amdgcn_mov_dpp(wsrc, 0x00, 0xF, 0xF, false); break;
        case 1: word = __builtin_amdgcn_mov_dpp(wsrc, 0x55, 0xF, 0xF, false); break;
        case 2: word = __builtin_amdgcn_mov_dpp(wsrc, 0xAA, 0xF, 0xF, false); break;
        default: word = __builtin_amdgcn_mov_dpp(wsrc, 0xFF, 0xF, 0xF, false); break;
      }
      const uint32_t e = ((uint32_t)word >> (8 * ((st >> 1) & 3))) & 0xFFu;
      const float sc = __uint_as_float(e << 23);
      const uint32_t m = e != 0 ? 0xFFFFFFFFu : 0u;
      *reinterpret_cast<bf16x8*>(row + wch0) = e4m3x8_to_bf16x8_scaled(v[0] & m, v[1] & m, sc);
      *reinterpret_cast<bf16x8*>(row + wch1) = e4m3x8_to_bf16x8_scaled(v[2] & m, v[3] & m, sc);
    } else {
      *reinterpret_cast<bf16x8*>(row + wch0) = e4m3x8_to_bf16x8(v[0], v[1]);
      *reinterpret_cast<bf16x8*>(row + wch1) = e4m3x8_to_bf16x8(v[2], v[3]);
    }
  };

  // ---- scales.  Token scales of the lane's 2 token columns
  // (tbase + 32 mi + c32), one K block ahead, by buffer loads with the whole
  // offset in voffset (the range check covers it: columns past M read as 0
  // and are never stored); weight-block scales of the wave's 128 rows in
  // lanes (lane l: blocks l and 64 + l), picked per block with v_readlane.
  const __amdgpu_buffer_rsrc_t sa_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.sa + (size_t)tok0 * nkb), (short)0, tok_rows * nkb * 4, 0x00020000);
  auto load_sa = [&](int mi, int kb) {
    return __builtin_amdgcn_raw_buffer_load_b32(sa_rsrc, ((tbase + 32 * mi + c32) * nkb + kb) * 4, 0, 0);
  };
  float sb_lo = 0.f, sb_hi = 0.f;
  float sa_nx[kMI] = {};
  if constexpr (!U8) {
    const float* sbc = p.sb + (size_t)((wrow0 + wbase) >> 7) * nkb;
    sb_lo = lane < nkb ? sbc[lane] : 0.f;
    sb_hi = 64 + lane < nkb ? sbc[64 + lane] : 0.f;
#pragma unroll
    for (int mi = 0; mi < kMI; ++mi) sa_nx[mi] = __builtin_bit_cast(float, load_sa(mi, 0));
  }

  // ---- running-scale accumulator: acc is in units of `unit` = sa * sb of the
  // current block (per token column); entering block kb multiplies it by
  // rs = old unit / new unit.  A block with a zero scale keeps the unit and
  // its token fragments are cleared in the lanes of those columns (zmask), so
  // it adds nothing.
  f32x16 acc[kNI][kMI];
#pragma unroll
  for (int ni = 0; ni < kNI; ++ni)
#pragma unroll
    for (int mi = 0; mi < kMI; ++mi) acc[ni][mi] = f32x16{};
  float unit[kMI], rs[kMI];
  unsigned zm_cur = 0, zm_nx = 0;  // zero-scale columns of the current / next block
#pragma unroll
  for (int mi = 0; mi < kMI; ++mi) { unit[mi] = 0.f; rs[mi] = 1.f; }
  auto enter_block = [&](int kb) {  // uses sa_nx = sa of block kb
    const float sbv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
        __builtin_bit_cast(int, kb < 64 ? sb_lo : sb_hi), kb & 63));
    zm_nx = 0;
    float s[kMI];
    bool extreme = false;
#pragma unroll
    for (int mi = 0; mi < kMI; ++mi) {
      s[mi] = sa_nx[mi] * sbv;
      const float a = __builtin_fabsf(s[mi]);
      extreme |= a != 0.f && !(a >= 0x1p-125f && a <= 0x1p125f);  // NaN / inf count too
    }
    // rs = unit / s: by the reciprocal while every s of the wave lies in
    // [2^-125, 2^125] (its reciprocal is then a normal float), else by IEEE
    // division, so subnormal scale products are handled as the fp32 oracle does.
    const bool exact_div = __builtin_amdgcn_ballot_w64(extreme) != 0;  // wave-uniform
#pragma unroll
    for (int mi = 0; mi < kMI; ++mi) {
      const bool live = s[mi] != 0.f;
      const float r = exact_div ? unit[mi] / s[mi] : unit[mi] * __builtin_amdgcn_rcpf(s[mi]);
      rs[mi] = (live && unit[mi] != 0.f) ? r : 1.f;
      unit[mi] = live ? s[mi] : unit[mi];
      zm_nx |= live ? 0u : 1u << mi;
    }
  };
  auto rescale_half = [&](int t, int hf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[t >> 1][t & 1][8 * hf + i] *= rs[t & 1];
  };

  // ---- fragments: wf[ni] (weights, refreshed group by group), tf[2][mi]
  // (tokens, double-buffered by substep parity).  Substep u of a stage covers
  // K 16 u .. +16: lane (c32, h) holds K 8 h .. +8 of it, chunk 2 u + h.
  bf16x8 wf[kNI], tf[2][kMI];
  auto read_w = [&](int st, int u, int ni) {
    wf[ni] = *reinterpret_cast<const bf16x8*>(lds + (st & 1) * kSlot + swz(wbase + 32 * ni + c32, 2 * u + h));
  };
  auto read_t = [&](int st, int u) {
#pragma unroll
    for (int mi = 0; mi < kMI; ++mi)
      tf[u & 1][mi] = *reinterpret_cast<const bf16x8*>(lds + (st & 1) * kSlot + kWBytes +
                                                        swz(tbase + 32 * mi + c32, 2 * u + h));
  };
  auto mask_t = [&](int u) {
    // zero-scale columns of the current block (a uniform branch, rarely taken)
    if (__builtin_amdgcn_ballot_w64(zm_cur != 0) != 0) {
#pragma unroll
      for (int mi = 0; mi < kMI; ++mi)
        if (zm_cur >> mi & 1) tf[u & 1][mi] = bf16x8{};
    }
  };

  // One 64-wide K stage st = 2 kb + O (O = 0: first half of scale block kb):
  // 32 MFMA slots, substep u = slot / 8, tile t = slot % 8 (weight block
  // t / 2, token block t % 2).  Pinned to slots:
  //  - the token fragments of substep u + 1 at slot 8 u; each weight
  //    fragment of substep u + 1 after its last MFMA of substep u;
  //  - widen + write part i of stage st + 1 at slot 3 + 6 i (i = 0..3), then
  //    load that part of stage st + 3 into the registers it came from;
  //  - at slot 24 (every read of stage st has returned, this wave's writes of
  //    st + 1 are done): the barrier that publishes stage st + 1, then its
  //    first fragments;
  //  - the rescale at the scale-block boundary, 8 multiplies per slot from
  //    slot 26 of the second stage to slot 6 of the next block's first (tile
  //    t's two halves after its last MFMA of the old block, two slots for the
  //    MFMA to finish, and before its first MFMA of the new block).
  auto stage = [&](auto oc, auto lastc, int kb) {
    constexpr int O = decltype(oc)::value;
    constexpr bool LAST_BLOCK = decltype(lastc)::value;
    constexpr bool NEXT = !(LAST_BLOCK && O == 1);      // stage st + 1 exists
    constexpr bool LOAD = !LAST_BLOCK;                  // stage st + 3 may exist
    const int st = 2 * kb + O;
    if constexpr (O == 0) zm_cur = zm_nx;
    if constexpr (O == 1 && !LAST_BLOCK && !U8) {
      enter_block(kb + 1);
      if (kb + 2 < nkb) {
#pragma unroll
        for (int mi = 0; mi < kMI; ++mi) sa_nx[mi] = __builtin_bit_cast(float, load_sa(mi, kb + 2));
      }
    }
    static_for<0, 32>([&](auto sc) {
      constexpr int slot = decltype(sc)::value;
      constexpr int u = slot / 8, t = slot % 8, ni = t / 2, mi = t % 2;
      if constexpr (t == 0 && !U8) mask_t(u);
      // rescale halves due in this slot (boundary slots 0-12: O = 1 slots
      // 26-31, then O = 0 slots 0-6)
      static_for<0, 8>([&](auto tc) {
        constexpr int tt = decltype(tc)::value;
        static_for<0, 2>([&](auto hc) {
          constexpr int hf = decltype(hc)::value;
          constexpr int bs = kRescaleSlot[tt][hf];
          constexpr bool here = O == 1 ? (bs < 6 && slot == 26 + bs) : (bs >= 6 && slot == bs - 6);
          if constexpr (here && !(O == 1 && LAST_BLOCK) && !U8) rescale_half(tt, hf);
        });
      });
      acc[ni][mi] = mfma32(wf[ni], tf[u & 1][mi], acc[ni][mi]);
      // widen + write part i of stage st + 1, then load part i of stage st + 3
      constexpr int part = (slot >= 3 && (slot - 3) % 6 == 0 && (slot - 3) / 6 < 4) ? (slot - 3) / 6 : -1;
      if constexpr (NEXT && part >= 0) {
        write_part(st + 1, part);
        if constexpr (LOAD) {
          if (O == 0 || kb + 2 < nkb) load_part(st + 3, part);
        }
      }
      if constexpr (u < 3) {
        if constexpr (t == 0) read_t(st, u + 1);
        if constexpr (mi == 1) read_w(st, u + 1, ni);
      } else if constexpr (NEXT) {
        if constexpr (t == 0) {
          // publish stage st + 1
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          __builtin_amdgcn_s_barrier();
          read_t(st + 1, 0);
        }
        if constexpr (mi == 1) read_w(st + 1, 0, ni);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // ---- prologue: block 0's unit, stage 0 in LDS, stage 1 in flight, the
  // first fragments.
  if constexpr (!U8) {
    enter_block(0);
    zm_cur = zm_nx;
    if (nkb > 1) {
#pragma unroll
      for (int mi = 0; mi < kMI; ++mi) sa_nx[mi] = __builtin_bit_cast(float, load_sa(mi, 1));
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) load_part(0, i);
#pragma unroll
  for (int i = 0; i < 4; ++i) load_part(1, i);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    write_part(0, i);
    if (nkb > 1) load_part(2, i);
  }
  __syncthreads();
  read_t(0, 0);
#pragma unroll
  for (int ni = 0; ni < kNI; ++ni) read_w(0, 0, ni);

  for (int kb = 0; kb + 1 < nkb; ++kb) {
    stage(IntC<0>{}, IntC<false>{}, kb);
    stage(IntC<1>{}, IntC<false>{}, kb);
  }
  stage(IntC<0>{}, IntC<true>{}, nkb - 1);
  stage(IntC<1>{}, IntC<true>{}, nkb - 1);

  // ---- epilogue: C[tok][wrow] = acc * unit, bf16, staged through LDS (after
  // a barrier: other waves may still read the last stage) so each store
  // writes whole 256-byte row segments.  acc[ni][mi][i]: weight row
  // 32 ni + 8 (i / 4) + 4 h + i % 4, token 32 mi + c32.
  __syncthreads();
  uint8_t* stgb = lds + wave * kTT * kPitch;
#pragma unroll
  for (int mi = 0; mi < kMI; ++mi)
#pragma unroll
    for (int ni = 0; ni < kNI; ++ni)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const f32x16& a = acc[ni][mi];
        u32x2 v;
        const float un = U8 ? 1.0f : unit[mi];  // U8: the sums are absolute already
        v[0] = pack_bf16x2(a[4 * g4] * un, a[4 * g4 + 1] * un);
        v[1] = pack_bf16x2(a[4 * g4 + 2] * un, a[4 * g4 + 3] * un);
        *reinterpret_cast<u32x2*>(stgb + (32 * mi + c32) * kPitch + (32 * ni + 8 * g4 + 4 * h) * 2) = v;
      }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's own rows are written
  const int chunk = lane & 15;
#pragma unroll
  for (int it = 0; it < kTT / 4; ++it) {
    const int rw = it * 4 + (lane >> 4);
    const int tok = tok0 + tbase + rw;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stgb + rw * kPitch + chunk * 16);
    if (tok < p.M) *reinterpret_cast<u32x4*>(p.out + (size_t)tok * p.N + wrow0 + wbase + chunk * 8) = v;
  }
}

}  // namespace ferret

using namespace ferret;

// Whether the 256 x 256 kernel takes this dense shape: N a multiple of 256,
// at least 192 tiles, and a last round of work-groups at least 3/4 full (one
// work-group per CU).  Measured against the 256 x 128 kernel on the DeepSeek-V3
// prefill shapes: faster at o_proj M = 2048 / 4096 (54 vs 58 / 107 vs 111 us),
// q_b_proj M = 4096 (40 vs 45) and kv_b_proj M = 8192 (40 vs 42), even at
// M = N = 4096, K = 7168 (188 vs 187), slower where the last round is half
// empty (q_b_proj M = 8192, 384 tiles: 80 vs 69; o_proj M = 8192, 896 tiles).
bool ferret_fp8_square_takes(int M, int N, int K) {
  if (N % sq::kBW != 0 || K % 128 != 0 || K / 128 > 128) return false;
  const long long tiles = (long long)(N / sq::kBW) * ((M + sq::kBT - 1) / sq::kBT);
  return tiles >= 192 && (tiles % 256 == 0 || tiles % 256 >= 192);
}

int ferret_fp8_gemm_square(const void* a, const float* sa, const void* b, const float* sb, void* c, int M, int N,
                           int K, hipStream_t st) {
  sq::Args p{};
  p.a = static_cast<const uint8_t*>(a);
  p.sa = sa;
  p.b = static_cast<const uint8_t*>(b);
  p.sb = sb;
  p.out = static_cast<uint16_t*>(c);
  p.M = M;
  p.N = N;
  p.K = K;
  p.n_blocks = N / sq::kBW;
  p.m_blocks = (M + sq::kBT - 1) / sq::kBT;
  FERRET_HIP_CHECK((set_lds_limit_once<fp8_square_kernel<false>>(sq::kLds)));
  hipLaunchKernelGGL(fp8_square_kernel<false>, dim3(p.n_blocks * p.m_blocks), dim3(sq::kThreads), sq::kLds, st, p);
  return (int)hipGetLastError();
}

// The same with UE8M0 scales in the reference's packed layout (ue8m0.hip),
// folded into the widening; the dispatch rule is ferret_fp8_square_takes.
int ferret_fp8_gemm_square_ue8m0(const void* a, const uint32_t* sfa, const void* b, const uint32_t* sfb, void* c,
                                 int M, int N, int K, hipStream_t st) {
  sq::Args p{};
  p.a = static_cast<const uint8_t*>(a);
  p.sfa = sfa;
  p.b = static_cast<const uint8_t*>(b);
  p.sfb = sfb;
  p.out = static_cast<uint16_t*>(c);
  p.M = M;
  p.N = N;
  p.K = K;
  p.n_blocks = N / sq::kBW;
  p.m_blocks = (M + sq::kBT - 1) / sq::kBT;
  FERRET_HIP_CHECK((set_lds_limit_once<fp8_square_kernel<true>>(sq::kLds)));
  hipLaunchKernelGGL(fp8_square_kernel<true>, dim3(p.n_blocks * p.m_blocks), dim3(sq::kThreads), sq::kLds, st, p);
  return (int)hipGetLastError();
}
