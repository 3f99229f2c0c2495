// On-GPU MoE routing for gfx950: top-k on logits, expert histogram, stable
// expert-major permutation of the routed pairs and the row-tile table the
// grouped GEMMs consume.
//
// The reference has no routing kernel (synthetic m_indices in
// baselines/fp8-group-gemm/baseline_dsv3_decode.py:50 and baseline_dsv3_prefill.py:53;
// randperm routing + vLLM moe_align_block_size in
// baselines/kimi-moe-w13-int4/baseline_marlin.py:92-104,123-126).  The contract
// here is bit-exact and order-deterministic:
//   * top-k by (logit desc, expert asc), NaN ranked as -inf;
//   * pair p = t*topk + j; pairs of one expert keep ascending pair order
//     (computed with wave ballots, never from atomic arrival order);
//   * tiles (expert, first sorted row, rows <= tile_m), expert-major; the
//     entries past the last tile up to max_tiles are (0, 0, 0).
#include "common.hpp"

namespace ferret {

constexpr int kMaxE = 1024;
constexpr int kMaxTopk = 16;
constexpr int kPermThreads = 1024;
constexpr int kPermWaves = kPermThreads / 64;

__device__ __forceinline__ bool better(float v1, int i1, float v2, int i2) {
  return v1 > v2 || (v1 == v2 && i1 < i2);
}

// Order key of a (logit, expert) pair as two words compared lexicographically:
// hi = the logit's bits mapped to unsigned order (NaN taken as -inf, -0 as +0,
// which ties +0), lo = ~expert; a larger key is a larger logit, then a smaller
// expert -- the (logit desc, expert asc) order.  Slots past E get (0, 0), below
// every real pair (the smallest real hi, that of -inf, is 0x007FFFFF).
__device__ __forceinline__ uint32_t order_bits(float x) {
  if (x != x) x = -INFINITY;
  if (x == 0.f) x = 0.f;
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_order_bits(uint32_t h) {
  return __uint_as_float((h & 0x80000000u) ? (h & 0x7FFFFFFFu) : ~h);
}
__device__ __forceinline__ bool key_gt(uint32_t h1, uint32_t l1, uint32_t h2, uint32_t l2) {
  return h1 > h2 || (h1 == h2 && l1 > l2);
}
// Wave maximum of an unsigned word by DPP: quad xor 1 and 2, half-row and row
// mirror (each 16-lane row's maximum in all its lanes), then row broadcasts 15
// (into rows 1 and 3) and 31 (into rows 2 and 3); lane 63 ends with the
// maximum.  Lanes of rows a broadcast does not write keep their value (the
// `old` operand).
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint32_t dpp_max_step(uint32_t x) {
  const uint32_t y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, CTRL, ROWS, 0xF, false);
  return x > y ? x : y;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = dpp_max_step<0xB1>(x);        // quad_perm [1, 0, 3, 2]
  x = dpp_max_step<0x4E>(x);        // quad_perm [2, 3, 0, 1]
  x = dpp_max_step<0x141>(x);       // row_half_mirror
  x = dpp_max_step<0x140>(x);       // row_mirror
  x = dpp_max_step<0x142, 0xA>(x);  // row_bcast:15
  x = dpp_max_step<0x143, 0xC>(x);  // row_bcast:31
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}

// One wave per token; lane l owns experts l, l + 64, ... (PER slots, E <= 64 PER).
// Each of the topk rounds takes the wave's largest untaken key: every lane
// offers its best untaken slot, a DPP wave maximum of the first words names
// the largest logit, the lane offering it gives the expert (a second DPP
// maximum, over the second words of the lanes that tie, when the logit occurs
// in several lanes), and the owning lane marks the slot taken.  Weights: the full softmax over E at the
// chosen experts (not renormalised).
template <int PER>
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ logits, int T, int E,
                                                          int topk, int32_t* __restrict__ ids,
                                                          float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // wave-uniform: the rest of the wave runs with all 64 lanes
  const float* row = logits + (size_t)t * E;
  float v[PER];
  uint32_t kh[PER], kl[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int ex = lane + 64 * i;
    float x = -INFINITY;
    if (ex < E) {
      x = row[ex];
      if (x != x) x = -INFINITY;
    }
    v[i] = x;
    kh[i] = ex < E ? order_bits(x) : 0u;
    kl[i] = ex < E ? ~(uint32_t)ex : 0u;
  }
  uint32_t taken = 0;  // bit i: slot i already selected
  int my_id = 0;       // lane k < topk: the k-th expert
  float my_v = 0.f;
  uint32_t top_h = 0;  // key of the first pick (the row maximum)
  for (int k = 0; k < topk; ++k) {
    uint32_t bh = 0, bl = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (!((taken >> i) & 1u) && key_gt(kh[i], kl[i], bh, bl)) {
        bh = kh[i];
        bl = kl[i];
      }
    // The largest first word; the lanes offering it; if several do (equal
    // logits in different lanes), the largest second word among them.
    const uint32_t wh = wave_max_u32(bh);
    const uint64_t tie = __ballot(bh == wh);
    uint32_t wl;
    if (__popcll(tie) == 1)
      wl = (uint32_t)__builtin_amdgcn_readlane((int)bl, __ffsll((unsigned long long)tie) - 1);
    else
      wl = wave_max_u32(bh == wh ? bl : 0u);
    const int sel = (int)~wl;
    if ((sel & 63) == lane) taken |= 1u << (sel >> 6);
    if (k == lane) {
      my_id = sel;
      my_v = from_order_bits(wh);
    }
    if (k == 0) top_h = wh;
  }
  if (lane < topk) ids[(size_t)t * topk + lane] = my_id;
  if (weights) {
    const float mx = from_order_bits(top_h);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (lane + 64 * i < E) s += expf(v[i] - mx);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    if (lane < topk) weights[(size_t)t * topk + lane] = expf(my_v - mx) / s;
  }
}

// Inclusive scans of a[0..n) and b[0..n) in LDS (n <= 1024) by the 1024-thread
// group: each wave scans its 64 values by shuffles, wave 0 scans the 16 wave
// totals, and every value takes the totals of the waves before it (integer
// sums: the same results as any other order).  Two barriers, where a
// Hillis-Steele scan of each array takes two per doubling.
__device__ void block_scan2_incl(int* a, int* b, int n) {
  __shared__ int wa[kPermWaves], wb[kPermWaves];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int x = tid < n ? a[tid] : 0, y = tid < n ? b[tid] : 0;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int xo = __shfl_up(x, off), yo = __shfl_up(y, off);
    if (lane >= off) {
      x += xo;
      y += yo;
    }
  }
  if (lane == 63) {
    wa[w] = x;
    wb[w] = y;
  }
  __syncthreads();
  if (w == 0) {
    int sx = lane < kPermWaves ? wa[lane] : 0, sy = lane < kPermWaves ? wb[lane] : 0;
#pragma unroll
    for (int off = 1; off < kPermWaves; off <<= 1) {
      const int xo = __shfl_up(sx, off), yo = __shfl_up(sy, off);
      if (lane >= off) {
        sx += xo;
        sy += yo;
      }
    }
    if (lane < kPermWaves) {
      wa[lane] = sx;
      wb[lane] = sy;
    }
  }
  __syncthreads();
  if (tid < n) {
    a[tid] = x + (w > 0 ? wa[w - 1] : 0);
    b[tid] = y + (w > 0 ? wb[w - 1] : 0);
  }
  __syncthreads();
}

// Single work-group: histogram, offsets, tile table, stable placement.
// counts / offsets / tile table from the per-expert counts cnt[0..E) (LDS);
// cursor (LDS, may be null) receives the exclusive offsets.  scan / tscan are
// LDS scratch of kMaxE ints.  Called by every thread of the group.
__device__ void permute_tables(const int* cnt, int* scan, int* tscan, int* cursor, int E, int tile_m,
                               int32_t* counts, int32_t* offsets, int32_t* tiles, int max_tiles,
                               int32_t* ntiles) {
  const int tid = threadIdx.x;
  if (tid < E) {
    scan[tid] = cnt[tid];
    tscan[tid] = (cnt[tid] + tile_m - 1) / tile_m;
  }
  __syncthreads();
  block_scan2_incl(scan, tscan, E);
  if (tid < E) {
    const int c = cnt[tid];
    const int off = scan[tid] - c;
    counts[tid] = c;
    offsets[tid] = off;
    if (cursor) cursor[tid] = off;
    if (tid == E - 1) {
      offsets[E] = scan[tid];
      ntiles[0] = min(tscan[tid], max_tiles);
    }
    int tt = tscan[tid] - (c + tile_m - 1) / tile_m;
    for (int j = 0; j < c; j += tile_m, ++tt) {
      if (tt < max_tiles) {
        tiles[3 * tt] = tid;
        tiles[3 * tt + 1] = off + j;
        tiles[3 * tt + 2] = min(tile_m, c - j);
      }
    }
  }
  // Entries past the last tile up to max_tiles are zero (expert 0, row 0, no
  // rows), so the whole table is a function of the ids.
  for (int t = tscan[E - 1] + tid; t < max_tiles; t += blockDim.x) {
    tiles[3 * t] = 0;
    tiles[3 * t + 1] = 0;
    tiles[3 * t + 2] = 0;
  }
  __syncthreads();
}

// Stable rank of this thread's pair among the earlier pairs (lower thread
// index) of the 1024-thread group with the same expert: within the wave, the
// lanes holding the same expert are found by one ballot per bit of the expert
// id (ebits of them, a fixed count instead of one round per distinct expert);
// across waves from the per-wave counts wcnt[w][e], which must be zero on
// entry and hold this chunk's counts on return.  e = -1 marks an invalid pair
// (rank 0, not counted).
__device__ int chunk_rank(int e, int ebits, uint16_t (*wcnt)[kMaxE]) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const bool valid = e >= 0;
  uint64_t same = __ballot(valid);
  for (int b = 0; b < ebits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t ones = __ballot(bit);
    same &= bit ? ones : ~ones;
  }
  int rank = 0;
  if (valid) {
    const uint64_t before = same & ((lane == 0) ? 0ull : (~0ull >> (64 - lane)));
    rank = __popcll(before);
    if (before == 0) wcnt[wave][e] = (uint16_t)__popcll(same);  // the expert's first lane in the wave
  }
  __syncthreads();
  if (valid)
    for (int w = 0; w < wave; ++w) rank += wcnt[w][e];
  return rank;
}

// Bits of an expert id below E (at least one).
__device__ __forceinline__ int expert_bits(int E) { return 32 - __builtin_clz((unsigned)max(E - 1, 1)); }

// Single work-group: histogram, tables, then stable placement chunk by chunk
// in pair order (the next chunk's ids are loaded while one is placed).
__global__ __launch_bounds__(kPermThreads) void permute_kernel(const int32_t* __restrict__ ids, int P, int E,
                                                               int tile_m, int32_t* __restrict__ counts,
                                                               int32_t* __restrict__ offsets,
                                                               int32_t* __restrict__ sorted_pair,
                                                               int32_t* __restrict__ tiles, int max_tiles,
                                                               int32_t* __restrict__ ntiles) {
  __shared__ int cnt[kMaxE];
  __shared__ int scan[kMaxE];
  __shared__ int tscan[kMaxE];
  __shared__ int cursor[kMaxE];
  __shared__ uint16_t wcnt[kPermWaves][kMaxE];

  const int tid = threadIdx.x;
  // The first chunk's ids are loaded once, before the tables, and kept for its
  // placement.
  const int e_first = tid < P ? ids[tid] : -1;
  for (int i = tid; i < E; i += kPermThreads) {
    cnt[i] = 0;
#pragma unroll
    for (int w = 0; w < kPermWaves; ++w) wcnt[w][i] = 0;
  }
  __syncthreads();
  if (e_first >= 0 && e_first < E) atomicAdd(&cnt[e_first], 1);
  for (int p = tid + kPermThreads; p < P; p += kPermThreads) {
    const int e = ids[p];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  permute_tables(cnt, scan, tscan, cursor, E, tile_m, counts, offsets, tiles, max_tiles, ntiles);

  int e_next = e_first;
  for (int base = 0; base < P; base += kPermThreads) {
    const int p = base + tid;
    int e = e_next;
    e_next = (p + kPermThreads < P) ? ids[p + kPermThreads] : -1;
    if (!(e >= 0 && e < E)) e = -1;
    const int rank = chunk_rank(e, expert_bits(E), wcnt);
    if (e >= 0) sorted_pair[cursor[e] + rank] = p;
    __syncthreads();
    if (tid < E) {
      int add = 0;
      for (int w = 0; w < kPermWaves; ++w) {
        add += wcnt[w][tid];
        wcnt[w][tid] = 0;
      }
      cursor[tid] += add;
    }
    __syncthreads();
  }
}

// ---- multi-work-group path (P > 2 chunks and a workspace of
// ceil(P / 1024) * E ints): per-chunk histograms, one scan group that turns
// them into per-(chunk, expert) output bases and builds the tables, and one
// placement group per chunk.  Same output as permute_kernel.

__global__ __launch_bounds__(256) void perm_hist_kernel(const int32_t* __restrict__ ids, int P, int E,
                                                        int32_t* __restrict__ hist) {
  __shared__ int h[kMaxE];
  for (int i = threadIdx.x; i < E; i += 256) h[i] = 0;
  __syncthreads();
  const int base = blockIdx.x * kPermThreads;
  for (int i = threadIdx.x; i < kPermThreads; i += 256) {
    const int p = base + i;
    const int e = p < P ? ids[p] : -1;
    if (e >= 0 && e < E) atomicAdd(&h[e], 1);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < E; i += 256) hist[(size_t)blockIdx.x * E + i] = h[i];
}

// The per-chunk histograms become per-(chunk, expert) output bases.  G =
// 1024 / E threads share an expert, each over a contiguous run of chunks: its
// counts are loaded eight at a time (independent loads, one latency per batch
// rather than one per chunk), summed, and, once the expert offsets are known,
// loaded again (L2 hits) and overwritten with the running bases.
__global__ __launch_bounds__(kPermThreads) void perm_scan_kernel(int32_t* __restrict__ hist, int nchunks, int E,
                                                                 int tile_m, int32_t* __restrict__ counts,
                                                                 int32_t* __restrict__ offsets,
                                                                 int32_t* __restrict__ tiles, int max_tiles,
                                                                 int32_t* __restrict__ ntiles) {
  __shared__ int cnt[kMaxE];
  __shared__ int scan[kMaxE];
  __shared__ int tscan[kMaxE];
  __shared__ int part[kPermThreads];  // part[g * E + e]: chunk run g's count of expert e
  constexpr int B = 8;
  const int tid = threadIdx.x;
  const int G = kPermThreads / E;  // >= 1 (E <= 1024)
  const int e = tid % E, g = tid / E;
  const bool mine = g < G;
  const int per = (nchunks + G - 1) / G;
  const int c0 = min(nchunks, g * per), c1 = min(nchunks, c0 + per);
  int local = 0;
  if (mine) {
    for (int c = c0; c < c1; c += B) {
      int v[B];
#pragma unroll
      for (int j = 0; j < B; ++j) v[j] = c + j < c1 ? hist[(size_t)(c + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < B; ++j) local += v[j];
    }
    part[tid] = local;
  }
  __syncthreads();
  if (tid < E) {
    int run = 0;
    for (int gg = 0; gg < G; ++gg) run += part[gg * E + tid];
    cnt[tid] = run;
  }
  __syncthreads();
  permute_tables(cnt, scan, tscan, nullptr, E, tile_m, counts, offsets, tiles, max_tiles, ntiles);
  if (mine) {
    int base = scan[e] - cnt[e];
    for (int gg = 0; gg < g; ++gg) base += part[gg * E + e];
    for (int c = c0; c < c1; c += B) {
      int v[B];
#pragma unroll
      for (int j = 0; j < B; ++j) v[j] = c + j < c1 ? hist[(size_t)(c + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < B; ++j)
        if (c + j < c1) {
          hist[(size_t)(c + j) * E + e] = base;
          base += v[j];
        }
    }
  }
}

__global__ __launch_bounds__(kPermThreads) void perm_place_kernel(const int32_t* __restrict__ ids, int P, int E,
                                                                  const int32_t* __restrict__ base,
                                                                  int32_t* __restrict__ sorted_pair) {
  __shared__ uint16_t wcnt[kPermWaves][kMaxE];
  for (int i = threadIdx.x; i < kPermWaves * E; i += kPermThreads) wcnt[i / E][i % E] = 0;
  const int p = blockIdx.x * kPermThreads + threadIdx.x;
  int e = p < P ? ids[p] : -1;
  if (!(e >= 0 && e < E)) e = -1;
  // the chunk's output base of this expert, requested before the ranking
  const int b = e >= 0 ? base[(size_t)blockIdx.x * E + e] : 0;
  __syncthreads();
  const int rank = chunk_rank(e, expert_bits(E), wcnt);
  if (e >= 0) sorted_pair[b + rank] = p;
}

}  // namespace ferret

using namespace ferret;

extern "C" int ferret_moe_route_topk(const float* logits, int T, int E, int topk, int32_t* ids,
                                     float* weights, void* stream) {
  FERRET_REQUIRE(logits && ids, FERRET_ERR_NULL);
  FERRET_REQUIRE(T >= 0 && E >= 1 && E <= kMaxE && topk >= 1 && topk <= kMaxTopk && topk <= E,
                 FERRET_ERR_SHAPE);
  if (T == 0) return FERRET_OK;
  auto* kern = E <= 64 ? route_topk_kernel<1> : E <= 128 ? route_topk_kernel<2> : E <= 256 ? route_topk_kernel<4>
             : E <= 512 ? route_topk_kernel<8> : route_topk_kernel<16>;
  hipLaunchKernelGGL(kern, dim3((T + 3) / 4), dim3(256), 0, (hipStream_t)stream, logits, T, E, topk, ids, weights);
  return (int)hipGetLastError();
}

extern "C" int ferret_moe_max_tiles(int num_pairs, int E, int tile_m) {
  if (num_pairs <= 0 || tile_m <= 0) return 0;
  const long long bound = (long long)(num_pairs + tile_m - 1) / tile_m + E;
  return (int)(bound < num_pairs ? bound : num_pairs);
}

extern "C" int ferret_moe_tile_m(int num_pairs, int E) {
  // decode-sized segments (<= ~16 rows per expert) stream weights with the
  // 16-token skinny kernel; larger segments use 128-row MFMA tiles.
  return (E > 0 && num_pairs / E >= 32) ? 128 : 16;
}

// Workspace of the multi-work-group permutation (0: single work-group).
size_t ferret_moe_permute_workspace(long long num_pairs, int E) {
  const long long nchunks = (num_pairs + kPermThreads - 1) / kPermThreads;
  return nchunks > 2 ? (size_t)nchunks * E * sizeof(int32_t) : 0;
}

extern "C" int ferret_moe_permute(const int32_t* ids, int T, int topk, int E, int tile_m, int32_t* counts,
                                  int32_t* offsets, int32_t* sorted_pair, int32_t* tiles, int max_tiles,
                                  int32_t* ntiles, void* ws, size_t ws_bytes, void* stream) {
  FERRET_REQUIRE(ids && counts && offsets && sorted_pair && tiles && ntiles, FERRET_ERR_NULL);
  FERRET_REQUIRE(T >= 0 && topk >= 1 && E >= 1 && E <= kMaxE && tile_m >= 1, FERRET_ERR_SHAPE);
  const long long P = (long long)T * topk;
  FERRET_REQUIRE(P <= (1ll << 22), FERRET_ERR_SHAPE);
  FERRET_REQUIRE(max_tiles >= ferret_moe_max_tiles((int)P, E, tile_m), FERRET_ERR_SHAPE);
  const hipStream_t st = (hipStream_t)stream;
  const size_t need = ferret_moe_permute_workspace(P, E);
  if (need > 0 && ws != nullptr && ws_bytes >= need) {
    const int nchunks = (int)((P + kPermThreads - 1) / kPermThreads);
    int32_t* hist = static_cast<int32_t*>(ws);
    hipLaunchKernelGGL(perm_hist_kernel, dim3(nchunks), dim3(256), 0, st, ids, (int)P, E, hist);
    hipLaunchKernelGGL(perm_scan_kernel, dim3(1), dim3(kPermThreads), 0, st, hist, nchunks, E, tile_m, counts,
                       offsets, tiles, max_tiles, ntiles);
    hipLaunchKernelGGL(perm_place_kernel, dim3(nchunks), dim3(kPermThreads), 0, st, ids, (int)P, E,
                       (const int32_t*)hist, sorted_pair);
    return (int)hipGetLastError();
  }
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(kPermThreads), 0, st, ids, (int)P, E, tile_m, counts, offsets,
                     sorted_pair, tiles, max_tiles, ntiles);
  return (int)hipGetLastError();
}
