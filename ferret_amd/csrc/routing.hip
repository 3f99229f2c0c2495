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
//   * tiles (expert, first sorted row, rows <= tile_m), expert-major.
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
  const int lane = tid & 63;
  const int wave = tid >> 6;

  for (int i = tid; i < kMaxE; i += kPermThreads) cnt[i] = 0;
  for (int i = tid; i < kPermWaves * kMaxE; i += kPermThreads) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  for (int p = tid; p < P; p += kPermThreads) {
    const int e = ids[p];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
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
    cursor[tid] = off;
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
  __syncthreads();

  // Stable placement, chunk by chunk in pair order (the next chunk's ids are
  // loaded while this one is placed).
  int e_next = (tid < P) ? ids[tid] : -1;
  for (int base = 0; base < P; base += kPermThreads) {
    const int p = base + tid;
    int e = e_next;
    e_next = (p + kPermThreads < P) ? ids[p + kPermThreads] : -1;
    const bool valid = e >= 0 && e < E;
    if (!valid) e = -1;
    // rank among earlier lanes of this wave with the same expert
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
    if (valid) {
      int before = 0;
      for (int w = 0; w < wave; ++w) before += wcnt[w][e];
      sorted_pair[cursor[e] + before + rank] = p;
    }
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

extern "C" int ferret_moe_permute(const int32_t* ids, int T, int topk, int E, int tile_m, int32_t* counts,
                                  int32_t* offsets, int32_t* sorted_pair, int32_t* tiles, int max_tiles,
                                  int32_t* ntiles, void* stream) {
  FERRET_REQUIRE(ids && counts && offsets && sorted_pair && tiles && ntiles, FERRET_ERR_NULL);
  FERRET_REQUIRE(T >= 0 && topk >= 1 && E >= 1 && E <= kMaxE && tile_m >= 1, FERRET_ERR_SHAPE);
  const long long P = (long long)T * topk;
  FERRET_REQUIRE(P <= (1ll << 22), FERRET_ERR_SHAPE);
  FERRET_REQUIRE(max_tiles >= ferret_moe_max_tiles((int)P, E, tile_m), FERRET_ERR_SHAPE);
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(kPermThreads), 0, (hipStream_t)stream, ids, (int)P, E,
                     tile_m, counts, offsets, sorted_pair, tiles, max_tiles, ntiles);
  return (int)hipGetLastError();
}
