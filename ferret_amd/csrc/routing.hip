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

// One wave per token; each lane owns experts lane, lane+64, ...
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ logits, int T, int E,
                                                          int topk, int32_t* __restrict__ ids,
                                                          float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* row = logits + (size_t)t * E;
  constexpr int PER = kMaxE / 64;
  float v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int ex = lane + 64 * i;
    float x = -INFINITY;
    if (ex < E) {
      x = row[ex];
      if (x != x) x = -INFINITY;
    }
    v[i] = x;
  }
  uint32_t taken = 0;  // bit i: v[i] already selected
  float sel_v[kMaxTopk] = {};
  int sel_i[kMaxTopk] = {};
#pragma unroll
  for (int k = 0; k < kMaxTopk; ++k) {
    if (k >= topk) break;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int ex = lane + 64 * i;
      if (ex < E && !((taken >> i) & 1u) && better(v[i], ex, bv, bi)) {
        bv = v[i];
        bi = ex;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oi = __shfl_xor(bi, off);
      if (better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    sel_v[k] = bv;
    sel_i[k] = bi;
  }
  if (lane < topk) {
    int myi = 0;
#pragma unroll
    for (int k = 0; k < kMaxTopk; ++k)
      if (k < topk && k == lane) myi = sel_i[k];
    ids[(size_t)t * topk + lane] = myi;
  }
  if (weights) {
    const float mx = sel_v[0];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (lane + 64 * i < E) s += expf(v[i] - mx);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    if (lane < topk) {
      float mv = 0.f;
#pragma unroll
      for (int k = 0; k < kMaxTopk; ++k)
        if (k < topk && k == lane) mv = sel_v[k];
      weights[(size_t)t * topk + lane] = expf(mv - mx) / s;
    }
  }
}

// Inclusive Hillis-Steele scan of n <= 1024 ints in LDS by 1024 threads.
__device__ void block_scan_incl(int* buf, int n) {
  for (int off = 1; off < n; off <<= 1) {
    int v = 0;
    if (threadIdx.x < n && threadIdx.x >= off) v = buf[threadIdx.x - off];
    __syncthreads();
    if (threadIdx.x < n && threadIdx.x >= off) buf[threadIdx.x] += v;
    __syncthreads();
  }
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
  block_scan_incl(scan, E);
  block_scan_incl(tscan, E);
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
// index) of the 1024-thread group with the same expert: within the wave from
// ballots (one round per distinct expert), across waves from the per-wave
// counts wcnt[w][e], which must be zero on entry and hold this chunk's counts
// on return.  e = -1 marks an invalid pair (rank 0, not counted).
__device__ int chunk_rank(int e, uint16_t (*wcnt)[kMaxE]) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const bool valid = e >= 0;
  int rank = 0;
  uint64_t remaining = __ballot(valid);
  while (remaining) {
    const int leader = __ffsll((unsigned long long)remaining) - 1;  // wave-uniform
    const int le = __builtin_amdgcn_readlane(e, leader);
    const uint64_t m = __ballot(valid && e == le);
    if (valid && e == le) {
      const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
      rank = __popcll(m & lt);
      if (lane == leader) wcnt[wave][e] = (uint16_t)__popcll(m);
    }
    remaining &= ~m;
  }
  __syncthreads();
  if (valid)
    for (int w = 0; w < wave; ++w) rank += wcnt[w][e];
  return rank;
}

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
  for (int i = tid; i < kMaxE; i += kPermThreads) cnt[i] = 0;
  for (int i = tid; i < kPermWaves * kMaxE; i += kPermThreads) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  for (int p = tid; p < P; p += kPermThreads) {
    const int e = ids[p];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  permute_tables(cnt, scan, tscan, cursor, E, tile_m, counts, offsets, tiles, max_tiles, ntiles);

  int e_next = (tid < P) ? ids[tid] : -1;
  for (int base = 0; base < P; base += kPermThreads) {
    const int p = base + tid;
    int e = e_next;
    e_next = (p + kPermThreads < P) ? ids[p + kPermThreads] : -1;
    if (!(e >= 0 && e < E)) e = -1;
    const int rank = chunk_rank(e, wcnt);
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

__global__ __launch_bounds__(kPermThreads) void perm_scan_kernel(int32_t* __restrict__ hist, int nchunks, int E,
                                                                 int tile_m, int32_t* __restrict__ counts,
                                                                 int32_t* __restrict__ offsets,
                                                                 int32_t* __restrict__ tiles, int max_tiles,
                                                                 int32_t* __restrict__ ntiles) {
  __shared__ int cnt[kMaxE];
  __shared__ int scan[kMaxE];
  __shared__ int tscan[kMaxE];
  const int e = threadIdx.x;
  if (e < E) {
    int run = 0;  // exclusive prefix over the chunks, per expert
    for (int c = 0; c < nchunks; ++c) {
      const int v = hist[(size_t)c * E + e];
      hist[(size_t)c * E + e] = run;
      run += v;
    }
    cnt[e] = run;
  }
  __syncthreads();
  permute_tables(cnt, scan, tscan, nullptr, E, tile_m, counts, offsets, tiles, max_tiles, ntiles);
  if (e < E) {
    const int off = scan[e] - cnt[e];
    for (int c = 0; c < nchunks; ++c) hist[(size_t)c * E + e] += off;
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
  __syncthreads();
  const int rank = chunk_rank(e, wcnt);
  if (e >= 0) sorted_pair[base[(size_t)blockIdx.x * E + e] + rank] = p;
}

}  // namespace ferret

using namespace ferret;

extern "C" int ferret_moe_route_topk(const float* logits, int T, int E, int topk, int32_t* ids,
                                     float* weights, void* stream) {
  FERRET_REQUIRE(logits && ids, FERRET_ERR_NULL);
  FERRET_REQUIRE(T >= 0 && E >= 1 && E <= kMaxE && topk >= 1 && topk <= kMaxTopk && topk <= E,
                 FERRET_ERR_SHAPE);
  if (T == 0) return FERRET_OK;
  hipLaunchKernelGGL(route_topk_kernel, dim3((T + 3) / 4), dim3(256), 0, (hipStream_t)stream, logits, T, E,
                     topk, ids, weights);
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
