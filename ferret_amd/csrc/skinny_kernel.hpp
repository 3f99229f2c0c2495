// Skinny (<= 16 token) weight-streaming GEMM kernel template for gfx950 (see
// skinny.hip for the design notes and the entry points that instantiate it).
#pragma once
#include "common.hpp"

namespace ferret {

// kINT4T: the INT4 weights of kINT4 regrouped into 16-row x 128-K tiles, each
// one contiguous KB (ferret_int4_tile_weights); only the addressing differs.
enum WFmt : int { kBF16 = 0, kFP8 = 1, kINT4 = 2, kINT4T = 3 };
enum EpiKind : int { kStore = 0, kSilu = 1 };

constexpr bool is_int4(int f) { return f == kINT4 || f == kINT4T; }

struct SkinnyArgs {
  const uint8_t* w;         // bf16 / e4m3 [G, N, K] or int32 [G, N, K/8]; kINT4T: [G, N/16, K/128, 16, 64 B]
  const void* w_scale;      // FP8: f32 [G, N/128, K/128]; INT4: bf16 [G, N, K/32]
  const uint8_t* x;         // bf16 / e4m3 [T, K]
  const float* x_scale;     // FP8: f32 [T, K/128]
  const uint16_t* residual; // bf16 [M, N] or null (dense store only)
  uint16_t* out;            // dense: bf16 [M, N]; grouped store: bf16 [P, N] (pair rows); SiLU: bf16 [P, N/2]
  const int32_t* sorted_pair;
  const int32_t* tiles;     // grouped: int32 [max_tiles, 3]; dense: null
  const int32_t* ntiles;
  int topk;
  int M;                    // dense token count
  int N;                    // weight rows (per expert)
  int K;
  int units_n;              // row units per token tile
  float* partial;           // stream kernel, bf16 dense split-K: fp32 [ksplit, M, N] (null: no split)
  int ksplit;               // number of K splits when partial != null
};

template <int F>
struct FmtTraits;
template <>
struct FmtTraits<kBF16> {
  static constexpr int kWVec = 4;  // u32x4 per lane per row block per K-step
  static constexpr int kXVec = 4;
};
template <>
struct FmtTraits<kFP8> {
  static constexpr int kWVec = 2;
  static constexpr int kXVec = 2;
};
template <>
struct FmtTraits<kINT4> {
  static constexpr int kWVec = 1;
  static constexpr int kXVec = 4;
};
template <>
struct FmtTraits<kINT4T> : FmtTraits<kINT4> {};

constexpr int kRedStride = 17;              // padded token stride in the LDS reduction
constexpr int kRedBlock = 16 * kRedStride;  // floats per (wave, row block)

// x & 0x0F0F0F0F through inline asm: hiding the known-zero bits from the
// compiler keeps it converting bytes with v_cvt_f32_ubyte{0..3} (one op each)
// instead of extracting every nibble with v_bfe_u32 first.
// Per-group constants of the INT4 dequant (group scale s, a bf16 value).
struct Int4Scale {
  float s, s16, c1, c2;
};
__device__ __forceinline__ Int4Scale int4_scale(float s) {
  return Int4Scale{s, s * 0.0625f, -1032.0f * s, -72.0f * s};
}

// INT4 word (8 nibbles q0..q7, low first, offset-8) -> 8 bf16 = RNE(float(q - 8) * s).
// The nibbles are placed in fp16 mantissas under the exponent of 1024 with no
// shift: 0x6400 | q reads 1024 + q, 0x6400 | (q << 4) reads 1024 + 16 q.  One
// mixed fma per weight then forms (1024 + q) s - 1032 s, resp.
// (1024 + 16 q)(s / 16) - 72 s: the fma rounds the exact value (q - 8) s once,
// which needs <= 12 significant bits and so is exact in fp32 (as are 1032 s,
// 72 s and s / 16 for a bf16 s), and the bf16 pack rounds it to nearest even.
__device__ __forceinline__ u32x4 dequant_int4x8(uint32_t w, const Int4Scale& k) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  // The three constants as register values (VOP3 takes no literal here), so
  // each mask-and-merge is one v_and_or_b32; the asm is CSE'd and hoisted.
  uint32_t magic, m_lo, m_hi;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(magic));
  asm("s_mov_b32 %0, 0x000F000F" : "=s"(m_lo));
  asm("s_mov_b32 %0, 0x00F000F0" : "=s"(m_hi));
  const uint32_t w8 = w >> 8;
  const h2 t0 = __builtin_bit_cast(h2, (w & m_lo) | magic);   // q0, q4
  const h2 t1 = __builtin_bit_cast(h2, (w & m_hi) | magic);   // q1, q5 (x16)
  const h2 t2 = __builtin_bit_cast(h2, (w8 & m_lo) | magic);  // q2, q6
  const h2 t3 = __builtin_bit_cast(h2, (w8 & m_hi) | magic);  // q3, q7 (x16)
  u32x4 d;
  d[0] = pack_bf16x2(fmaf((float)t0.x, k.s, k.c1), fmaf((float)t1.x, k.s16, k.c2));
  d[1] = pack_bf16x2(fmaf((float)t2.x, k.s, k.c1), fmaf((float)t3.x, k.s16, k.c2));
  d[2] = pack_bf16x2(fmaf((float)t0.y, k.s, k.c1), fmaf((float)t1.y, k.s16, k.c2));
  d[3] = pack_bf16x2(fmaf((float)t2.y, k.s, k.c1), fmaf((float)t3.y, k.s16, k.c2));
  return d;
}

// RAG: K/128 is not a multiple of KS; the last wave takes the remaining
// nkb - wave * KS (< KS) K-steps, behind wave-uniform guards.
template <int F, int EPI, int RB, int KS, int D, bool RAG = false>
__global__ __launch_bounds__(1024) void skinny_gemm_kernel(SkinnyArgs a) {
  constexpr int WV = FmtTraits<F>::kWVec;
  constexpr int XV = FmtTraits<F>::kXVec;
  constexpr int HALF = (EPI == kSilu) ? RB / 2 : RB;
  static_assert(EPI != kSilu || RB % 2 == 0, "SiLU pairs gate and up row blocks");

  extern __shared__ float red[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int r = lane & 15;  // weight row inside a 16-row block (A side) / token column (B side)
  const int g = lane >> 4;  // K group of the lane

  const int nu = blockIdx.x % a.units_n;
  const int tile_idx = blockIdx.x / a.units_n;
  const bool grouped = a.tiles != nullptr;

  int e = 0, row0, nrows;
  if (grouped) {
    if (tile_idx >= __builtin_nontemporal_load(a.ntiles)) return;  // whole work-group exits
    e = a.tiles[3 * tile_idx];
    row0 = a.tiles[3 * tile_idx + 1];
    nrows = a.tiles[3 * tile_idx + 2];
  } else {
    row0 = tile_idx * 16;
    nrows = min(16, a.M - row0);
  }
  // clamp: columns >= nrows compute garbage, never stored (a zero-row tile reads row row0)
  const int tcol = max(0, min(r, nrows - 1));
  const int tok = grouped ? a.sorted_pair[row0 + tcol] / a.topk : row0 + tcol;

  const int N = a.N, K = a.K;
  const int nkb = K >> 7;
  const size_t row_bytes = (F == kBF16) ? (size_t)K * 2 : (F == kFP8 ? (size_t)K : (size_t)K / 2);

  int rowb[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    if (EPI == kSilu)
      rowb[rb] = (rb < HALF) ? (nu * HALF + rb) * 16 : N / 2 + (nu * HALF + rb - HALF) * 16;
    else
      rowb[rb] = (nu * RB + rb) * 16;
  }
  // This lane's weight row at K-step 0; a K-step advances it by ks_bytes.
  // kINT4T: row r of the block's first 1-KB tile.
  const uint8_t* wrow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
    wrow[rb] = F == kINT4T ? a.w + ((size_t)e * (N >> 4) + (rowb[rb] >> 4)) * (size_t)nkb * 1024 + r * 64
                           : a.w + ((size_t)e * N + rowb[rb] + r) * row_bytes;
  const size_t ks_bytes = F == kINT4T ? 1024 : 64;  // INT4 forms only
  const uint8_t* xrow = a.x + (size_t)tok * (F == kFP8 ? (size_t)K : (size_t)K * 2);

  const int ks0 = wave * KS;
  const int kcnt = RAG ? min(KS, nkb - ks0) : KS;  // K-steps of this wave (>= 1)

  u32x4 wbuf[D + 1][RB][WV];
  u32x4 xbuf[D + 1][XV];
  float sx[D + 1];
  float sw[D + 1][RB];
  uint16_t s4[D + 1][RB];

  auto load = [&](int slot, int s) {
    const int ks = ks0 + s;
    if constexpr (F == kBF16) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          wbuf[slot][rb][j] = ld_u32x4_stream(wrow[rb] + (size_t)(ks * 128 + 32 * j + 8 * g) * 2);
#pragma unroll
      for (int j = 0; j < 4; ++j) xbuf[slot][j] = ld_u32x4(xrow + (size_t)(ks * 128 + 32 * j + 8 * g) * 2);
    } else if constexpr (F == kFP8) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        wbuf[slot][rb][0] = ld_u32x4_stream(wrow[rb] + (size_t)ks * 128 + 32 * g);
        wbuf[slot][rb][1] = ld_u32x4_stream(wrow[rb] + (size_t)ks * 128 + 32 * g + 16);
        const float* swp = static_cast<const float*>(a.w_scale);
        sw[slot][rb] = swp[((size_t)e * (N >> 7) + (rowb[rb] >> 7)) * nkb + ks];
      }
      xbuf[slot][0] = ld_u32x4(xrow + (size_t)ks * 128 + 32 * g);
      xbuf[slot][1] = ld_u32x4(xrow + (size_t)ks * 128 + 32 * g + 16);
      sx[slot] = a.x_scale[(size_t)tok * nkb + ks];
    } else {
      const uint16_t* sp = static_cast<const uint16_t*>(a.w_scale);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        wbuf[slot][rb][0] = ld_u32x4_stream(wrow[rb] + (size_t)ks * ks_bytes + 16 * g);
        s4[slot][rb] = sp[((size_t)e * N + rowb[rb] + r) * (size_t)(K >> 5) + ks * 4 + g];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) xbuf[slot][j] = ld_u32x4(xrow + (size_t)(ks * 128 + 32 * g + 8 * j) * 2);
    }
  };

  f32x4 acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < D; ++s)
    if (!RAG || s < kcnt) load(s, s);
  // Keep the prefetches where they are written: without these barriers the
  // scheduler sinks loads next to their first use and leaves only a few in flight.
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if (s + D < KS && (!RAG || s + D < kcnt)) load((s + D) % (D + 1), s + D);
    __builtin_amdgcn_sched_barrier(0);
    if (RAG && s >= kcnt) continue;
    const int slot = s % (D + 1);
    if constexpr (F == kBF16) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[rb] = mfma_bf16_16x16x32(wbuf[slot][rb][j], xbuf[slot][j], acc[rb]);
    } else if constexpr (F == kFP8) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const f32x4 part = fp8_block_16x16x128(wbuf[slot][rb][0], wbuf[slot][rb][1], xbuf[slot][0], xbuf[slot][1]);
        const float sc = sx[slot] * sw[slot][rb];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[rb][i] = fmaf(part[i], sc, acc[rb][i]);
      }
    } else {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const float sc = bf16_bits_to_f32(s4[slot][rb]);
        const Int4Scale ks4 = int4_scale(sc);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[rb] = mfma_bf16_16x16x32(dequant_int4x8(wbuf[slot][rb][0][j], ks4), xbuf[slot][j], acc[rb]);
      }
    }
  }

  // Cross-wave split-K reduction through LDS: red[wave][rb][token*17 + row].
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * RB + rb) * kRedBlock + r * kRedStride + 4 * g + i] = acc[rb][i];
  __syncthreads();

  for (int idx = threadIdx.x; idx < 256 * HALF; idx += blockDim.x) {
    const int part = idx >> 8;
    const int t = (idx >> 4) & 15;
    const int row = idx & 15;
    if (t >= nrows) continue;
    if constexpr (EPI == kStore) {
      float v = 0.f;
      for (int w = 0; w < nwaves; ++w) v += red[(w * RB + part) * kRedBlock + t * kRedStride + row];
      // dense: token row; grouped: the routed pair of the sorted row
      const size_t orow = grouped ? (size_t)a.sorted_pair[row0 + t] : (size_t)(row0 + t);
      const size_t o = orow * N + rowb[0] + part * 16 + row;
      if (a.residual) v += bf16_bits_to_f32(a.residual[o]);
      a.out[o] = f32_to_bf16_bits(v);
    } else {
      float gs = 0.f, us = 0.f;
      for (int w = 0; w < nwaves; ++w) {
        gs += red[(w * RB + part) * kRedBlock + t * kRedStride + row];
        us += red[(w * RB + part + HALF) * kRedBlock + t * kRedStride + row];
      }
      const int pair = a.sorted_pair[row0 + t];
      const size_t o = (size_t)pair * (N / 2) + (nu * HALF + part) * 16 + row;
      a.out[o] = f32_to_bf16_bits(silu_mul(gs, us));
    }
  }
}

// ------------------------------------------------------------------ dispatch

template <int F, int EPI, int RB, int KS, int D, bool RAG = false>
static int launch_one(const SkinnyArgs& a, int grid, int nwaves, hipStream_t st) {
  const size_t lds = (size_t)nwaves * RB * kRedBlock * sizeof(float);
  hipLaunchKernelGGL((skinny_gemm_kernel<F, EPI, RB, KS, D, RAG>), dim3(grid), dim3(nwaves * 64), lds, st, a);
  return (int)hipGetLastError();
}

}  // namespace ferret
