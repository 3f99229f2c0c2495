/*
 * ferret_hip.h — C ABI of the MI355X (gfx950) quantized-GEMM library
 * (libferret_hip.so).
 *
 * Conventions shared by every entry point:
 *   - All tensor arguments are caller-owned DEVICE pointers; outputs are written
 *     in place.  Nothing is allocated, nothing is freed, the host is never
 *     synchronised: work is enqueued on `stream` (a hipStream_t; NULL = the
 *     default stream) and returns immediately.
 *   - Return value: 0 on success; a negative FERRET_ERR_* code for a rejected
 *     argument (nothing was enqueued); a positive hipError_t if the launch
 *     itself failed.  No entry point ever calls exit() or prints.
 *   - Layouts are row-major.  bf16 tensors are passed as raw 16-bit patterns,
 *     e4m3 tensors as bytes (OCP FP8 E4M3FN), scales as float32.
 *   - Reentrant; thread-safe when different threads use different streams.
 *
 * Paths in the citations are relative to the reference repository root.
 */
#ifndef FERRET_HIP_H_
#define FERRET_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FERRET_OK 0
#define FERRET_ERR_NULL (-1)      /* a required pointer is NULL */
#define FERRET_ERR_SHAPE (-2)     /* sizes out of range / not supported */
#define FERRET_ERR_WORKSPACE (-3) /* workspace missing or too small */

/* Library version string, e.g. "ferret-hip 0.1.0 gfx950". */
const char* ferret_version(void);

/* Human-readable text for a return code. */
const char* ferret_error_string(int code);

/*
 * Reference ctypes ABI for the decode GEMV, kept unchanged:
 * tests/compare_decode_linear.py:110-118 binds
 *   launch_gemv(void* input, void* weight, void* residual, void* output,
 *               int N, int K, void* stream)
 * with input bf16 [1,K], weight bf16 [N,K], residual bf16 [1,N] or NULL,
 * output bf16 [1,N].  No error return (as in the reference): on a rejected
 * argument nothing is enqueued; ferret_linear_bf16 reports the code.
 */
void launch_gemv(void* input, void* weight, void* residual, void* output, int N, int K,
                 void* stream);

/*
 * bf16 decode linear projection, y[M,N] = x[M,K] . w[N,K]^T (+ residual[M,N]),
 * fp32 accumulation, RNE to bf16.  Replaces the host dispatch `launch_kernel`
 * of examples/qwen3-8b-decode-linear-bs16/v019_swapab_cg2_l2hints.cu:422-482
 * (kernel :138-391, split-K reduce :395-417).
 * Requirements: 1 <= M, N % 16 == 0, K % 128 == 0, K/128 <= 128.
 * `ws` (optional): with at least ferret_workspace_bytes(0, M, N, K, 0) bytes
 * (non-zero when splitting K evens out the work over the CUs, e.g. N = 6144 or
 * K = 12288 at M <= 16) the product runs split-K: fp32 partials in the
 * workspace, summed in split order (+ residual) by a second kernel
 * (deterministic); with NULL the same result comes unsplit.
 */
int ferret_linear_bf16(const void* x, const void* w, const void* residual, void* y, int M, int N,
                       int K, void* ws, size_t ws_bytes, void* stream);

/*
 * ferret_linear_bf16 without a workspace argument and without any allocation:
 * no counterpart in the reference.  For callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Shapes that run split-K take their fp32 partials from a
 * library-owned device array of ferret_linear_bf16_noalloc_max_bytes()
 * (4 MiB) per GPU; a shape needing more (ferret_workspace_bytes(0, M, N, K, 0)
 * larger than that) is rejected with FERRET_ERR_WORKSPACE.  The result is
 * bit-identical to ferret_linear_bf16 with a workspace.  Calls that overlap on
 * one GPU (different streams or threads) share the array and race: serialise
 * them.  The array's address is looked up once per device, by the first call
 * of ferret_linear_bf16_noalloc_max_bytes or of this entry point on it: make
 * one of them on each device before capturing this entry point into a graph.
 */
int ferret_linear_bf16_noalloc(const void* x, const void* w, const void* residual, void* y, int M,
                               int N, int K, void* stream);

/* Bytes of the device array ferret_linear_bf16_noalloc uses (its limit); also
 * looks the array's address up on the current device. */
size_t ferret_linear_bf16_noalloc_max_bytes(void);

/*
 * Dense FP8 GEMM with DeepSeek-style fp32 block scales:
 *   c[m,n] = sum_kb (sum_{k in kb} a[m,k] b[n,k]) * sa[m,kb] * sb[n/128,kb]
 * a e4m3 [M,K], sa f32 [M,K/128], b e4m3 [N,K], sb f32 [ceil(N/128),K/128],
 * c bf16 [M,N].  Replaces `run<BN,NS>` / `fp8_gemm` of
 * examples/fp8-gemm/v002_dense_tp8_validated_065.cu:61-275 (oracle `ref` :277-288).
 * Requirements: M >= 1, N % 16 == 0, K % 128 == 0 (N % 128 == 0 when M > 16).
 * For 16 < M <= 256 the product runs split-K when `ws` holds at least
 * ferret_workspace_bytes(1, M, N, K, 0) bytes (fp32 partials, summed in a fixed
 * order: deterministic); with ws == NULL the same result comes from the
 * non-split kernel (slower at these shapes).
 */
int ferret_fp8_gemm_blockscale(const void* a, const float* sa, const void* b, const float* sb,
                               void* c, int M, int N, int K, void* ws, size_t ws_bytes,
                               void* stream);

/*
 * Dense FP8 GEMM with UE8M0 (power-of-two) block scales in the packed layout
 * of examples/fp8-gemm/v009_large_m_block_scale_mma_080.cu (prepare_sf
 * :386-403, expand_sb :405-412); replaces its run_bs / dispatch_run
 * (:414-476, :507-515):
 *   sfa uint32 [ceil(nk/4), M] column-major, byte j of word sfa[sk*M + m] the
 *       scale of token m for K-block 4*sk + j (nk = K/128);
 *   sfb uint32 [ceil(nk/4), N], per weight row (expand_sb's layout: the rows of
 *       a 128-row block carry the same bytes; row 128*(n/128) is read).
 * A byte e stands for 2^(e-127) and e = 0 for a zero scale (ue8m0_to_float,
 * :478-484), so c[m,n] = sum_kb (sum_{k in kb} a[m,k] b[n,k]) * 2^(ea-127) *
 * 2^(eb-127), the reference's oracle ref_bs (:486-505).  a e4m3 [M,K],
 * b e4m3 [N,K], c bf16 [M,N]; requirements as ferret_fp8_gemm_blockscale.
 * `ws` is required: at least ferret_workspace_bytes(5, M, N, K, 0) bytes (the
 * scales decoded to fp32, then the GEMM's split-K partials); a smaller one
 * returns FERRET_ERR_WORKSPACE.
 */
int ferret_fp8_gemm_ue8m0(const void* a, const uint32_t* sfa, const void* b, const uint32_t* sfb, void* c,
                          int M, int N, int K, void* ws, size_t ws_bytes, void* stream);

/*
 * Top-k routing on fp32 logits [T,E]: ids[T,topk] (int32) ordered by
 * (logit desc, expert asc), NaN ranks as -inf; weights[T,topk] (optional,
 * may be NULL) = softmax over all E at the chosen experts.  The reference has
 * no routing kernel (its stand-ins: baselines/kimi-moe-w13-int4/baseline_marlin.py:92-104,
 * baselines/fp8-group-gemm/baseline_dsv3_decode.py:50); this is the library's own
 * contract.  Requirements: 1 <= topk <= min(E, 16), E <= 1024.
 */
int ferret_moe_route_topk(const float* logits, int T, int E, int topk, int32_t* ids,
                          float* weights, void* stream);

/*
 * Expert histogram + stable permutation + tile table of routed pairs
 * (pair p = t*topk + j).  Replaces vLLM's moe_align_block_size as called at
 * baselines/kimi-moe-w13-int4/baseline_marlin.py:123-126 and the m_indices
 * construction of baselines/fp8-group-gemm/baseline_dsv3_prefill.py:53.
 * Outputs: counts[E], offsets[E+1] (exclusive cumsum), sorted_pair[P] (pairs
 * of expert 0 in ascending order, then expert 1, ...; ids outside [0,E) are
 * dropped), tiles[max_tiles*3] rows (expert, first sorted row, rows <= tile_m)
 * in expert order (rows past the last tile are (0, 0, 0)), ntiles[1].
 * max_tiles must be >= ferret_moe_max_tiles().
 * `ws` (optional): with at least ferret_workspace_bytes(4, P, 0, 0, E) bytes
 * the work is spread over one work-group per 1024 pairs (same output); with
 * NULL one work-group does it all (fine for decode-sized P).
 * Requirements: P = T*topk <= 1<<22, E <= 1024.
 */
int ferret_moe_permute(const int32_t* ids, int T, int topk, int E, int tile_m, int32_t* counts,
                       int32_t* offsets, int32_t* sorted_pair, int32_t* tiles, int max_tiles,
                       int32_t* ntiles, void* ws, size_t ws_bytes, void* stream);

/* Upper bound on the tile count of ferret_moe_permute for P pairs. */
int ferret_moe_max_tiles(int num_pairs, int E, int tile_m);

/* Row-tile height the w13 kernels expect for a routing of P pairs over E experts
 * (16 for decode-sized segments, 128 for prefill-sized ones). */
int ferret_moe_tile_m(int num_pairs, int E);

/*
 * FP8 block-scaled MoE gate-up (w13) grouped GEMM with fused SiLU(gate)*up:
 *   out[p, n] = silu(g) * u,  g = x_t . W[e][n], u = x_t . W[e][N/2 + n]
 * for every routed pair p (token t = p / topk, expert e) using the block-scaled
 * product of ferret_fp8_gemm_blockscale.  x e4m3 [T,K], sx f32 [T,K/128],
 * w e4m3 [E,N,K], sw f32 [E,N/128,K/128], out bf16 [T*topk, N/2] in pair order.
 * The tile inputs come from ferret_moe_permute with tile_m =
 * ferret_moe_tile_m(T*topk, E).  Replaces launch_grouped_gemm_bs /
 * grouped_fp8_gemm_bs of examples/fp8-group-gemm/v007_dsv3_decode_verified_105.cu:66-439
 * with the expert taken per row (not per 128-row tile, :162,286).
 * Requirements: N % 256 == 0, K % 128 == 0.
 */
int ferret_moe_w13_fp8(const void* x, const float* sx, const void* w, const float* sw,
                       const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                       int max_tiles, int tile_m, int T, int topk, int E, int N, int K, void* out,
                       void* stream);

/*
 * INT4 W4A16 MoE gate-up (w13) grouped GEMM with fused SiLU(gate)*up.
 * x bf16 [T,K]; wq int32 [E,N,K/8] (8 nibbles per word along K, low nibble
 * first, value = nibble - 8); ws bf16 [E,N,K/32]; out bf16 [T*topk, N/2].
 * Weights are dequantized in registers to bf16 = RNE(float(q) * scale) and fed
 * to bf16 MFMA with fp32 accumulation.  Replaces ops.moe_wna16_marlin_gemm +
 * apply_moe_activation(SILU) of baselines/kimi-moe-w13-int4/baseline_marlin.py:139-168;
 * numerics of correctness/compare_marlin_vs_ref.py:44-100; layout of
 * tasks/kimi-moe-w13-int4-grouped-gemm.yaml:68-83.
 * Requirements: N % 32 == 0, K % 128 == 0, tile_m == 16.  Group scales must be
 * finite with |s| < 2^128 / 1032 (about 3.3e35): the in-register dequant forms
 * -1032 * s in fp32.  Within that range every weight equals the reference's
 * bf16_RNE(float(q) * s) bit for bit (tests/test_gpu_int4_scales.py checks all
 * 65,536 bf16 scale patterns against all 16 nibbles).
 */
int ferret_moe_w13_w4a16(const void* x, const int32_t* wq, const void* ws,
                         const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                         int max_tiles, int tile_m, int T, int topk, int E, int N, int K,
                         void* out, void* stream);

/*
 * One-time load-time regrouping of the INT4 w13 words for
 * ferret_moe_w13_w4a16_tiled: wq int32 [E,N,K/8] -> wq_tiled [E][N/16][K/128]
 * tiles of 16 rows x 64 bytes (the rows' K-step slices, bytes unchanged),
 * each tile one contiguous KB.  Out of place (overlapping buffers are
 * rejected).  Replaces the load-time weight permutation the reference runs
 * before its GEMM, ops.gptq_marlin_moe_repack
 * (baselines/kimi-moe-w13-int4/baseline_marlin.py:62-89), which the task
 * contract allows (tasks/kimi-moe-w13-int4-grouped-gemm.yaml:68-71).
 * Requirements: N % 16 == 0, K % 128 == 0.
 */
int ferret_int4_tile_weights(const int32_t* wq, void* wq_tiled, int E, int N, int K, void* stream);

/*
 * ferret_moe_w13_w4a16 on weights regrouped by ferret_int4_tile_weights: the
 * same arguments and the same result bit for bit; each weight DMA reads one
 * contiguous KB instead of 64 bytes of each of 16 rows.  ws stays [E,N,K/32].
 * Replaces ops.moe_wna16_marlin_gemm on Marlin's permuted weights
 * (baselines/kimi-moe-w13-int4/baseline_marlin.py:139-168).
 * Requirements: as ferret_moe_w13_w4a16.
 */
int ferret_moe_w13_w4a16_tiled(const void* x, const void* wq_tiled, const void* ws,
                               const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                               int max_tiles, int tile_m, int T, int topk, int E, int N, int K,
                               void* out, void* stream);

/*
 * 1x128 activation quantizer: bf16 x [M,K] -> OCP e4m3 q [M,K] and fp32
 * scale [M,K/128] with, per 128-element block of a row (fp32, correctly rounded
 * division):  amax = max(|x| over the block, 1e-4);  q = e4m3_RNE(x * (448/amax));
 * scale = amax / 448.  The input format of every FP8 entry point above.
 * Replaces deep_gemm.per_token_cast_to_fp8 at its call site
 * baselines/fp8-gemm/baseline_prefill.py:41 (layout of A / A_scale:
 * tasks/fp8-group-gemm-dsv3-decode.yaml:19-20); DeepGEMM's own epsilon clamp is
 * not vendored, the floor 1e-4 is this library's.  Requirements: M >= 1,
 * K % 128 == 0.
 */
int ferret_quant_act_e4m3(const void* x, void* q, float* scale, int M, int K, void* stream);

/*
 * FP8 block-scaled MoE down projection (w2) grouped GEMM:
 *   out[p, n] = sum_kb (sum_{k in kb} h[p,k] W[e][n,k]) * sh[p,kb] * sw[e][n/128,kb]
 * for every routed pair p (expert e), h e4m3 [P,K] and sh f32 [P,K/128] in pair
 * order (the w13 output quantized by ferret_quant_act_e4m3), w e4m3 [E,N,K],
 * sw f32 [E,N/128,K/128], out bf16 [P,N] in pair order.  Tile inputs from
 * ferret_moe_permute as for ferret_moe_w13_fp8.  Replaces the down GEMM
 * (K = 2048 -> N = 7168) of tasks/fp8-group-gemm-dsv3-decode.yaml:11-13,67-86 and
 * tasks/fp8-group-gemm-dsv3-prefill.yaml:15,76-95, run by grouped_fp8_gemm_bs
 * (examples/fp8-group-gemm/v007_dsv3_decode_verified_105.cu:66-335).
 * Requirements: N % 128 == 0, K % 128 == 0, K / 128 <= 128, tile_m 16 or 128.
 */
int ferret_moe_w2_fp8(const void* h, const float* sh, const void* w, const float* sw,
                      const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                      int max_tiles, int tile_m, int P, int E, int N, int K, void* out, void* stream);

/*
 * Top-k weighted combine of the down-projection rows:
 *   y[t, n] = bf16_RNE( sum_{j < topk} w[t, j] * o[t*topk + j, n] )
 * o bf16 [T*topk, N] in pair order, w f32 [T, topk] (ferret_moe_route_topk's
 * weights), y bf16 [T, N]; the fp32 sum runs in j order (deterministic).
 * The reference has no combine kernel (its routing weights are computed and
 * left unused by w13: baselines/kimi-moe-w13-int4/baseline_marlin.py:92-104,158);
 * this is the library's own contract.  Requirements: N % 8 == 0, 1 <= topk <= 64.
 */
int ferret_moe_combine(const void* o, const float* w, int T, int topk, int N, void* y, void* stream);

/*
 * Flags of the FP8 *_ex entry points below.  FERRET_FP8_MMA_E4M3 multiplies
 * the e4m3 operands of the tiled (M > 16 / prefill) kernels on the FP8 MFMA
 * (v_mfma_scale_f32_16x16x128_f8f6f4) instead of widening them exactly to
 * bf16: one MFMA per 16x16x128 block instead of four, but the FP8 datapath
 * aligns the products of each dot-product group to a narrow window, so the
 * result can miss the reference's gate |g - r| / max(|r|, 1e-3 max|r|) < 1e-2
 * (examples/fp8-gemm/v002_dense_tp8_validated_065.cu:345-360) that the default
 * path meets.  Opt-in only; decode-sized (<= 16 token) shapes ignore it.
 */
#define FERRET_FP8_MMA_E4M3 1

/* ferret_fp8_gemm_blockscale with flags (0 = the same as the plain call). */
int ferret_fp8_gemm_blockscale_ex(const void* a, const float* sa, const void* b, const float* sb,
                                  void* c, int M, int N, int K, void* ws, size_t ws_bytes, int flags,
                                  void* stream);

/* ferret_moe_w13_fp8 with flags (0 = the same as the plain call). */
int ferret_moe_w13_fp8_ex(const void* x, const float* sx, const void* w, const float* sw,
                          const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                          int max_tiles, int tile_m, int T, int topk, int E, int N, int K, void* out,
                          int flags, void* stream);

/* ferret_moe_w2_fp8 with flags (0 = the same as the plain call). */
int ferret_moe_w2_fp8_ex(const void* h, const float* sh, const void* w, const float* sw,
                         const int32_t* sorted_pair, const int32_t* tiles, const int32_t* ntiles,
                         int max_tiles, int tile_m, int P, int E, int N, int K, void* out, int flags,
                         void* stream);

/* Workspace bytes an op can use (0 = none). op: 0 linear_bf16 (split-K partials),
 * 1 fp8_gemm_blockscale (split-K partials for 16 < M <= 256), 2 moe_w13_fp8,
 * 3 moe_w13_w4a16, 4 moe_permute (M = number of routed pairs P, E experts),
 * 5 fp8_gemm_ue8m0 (decoded scales + split-K partials; required). */
size_t ferret_workspace_bytes(int op, int M, int N, int K, int E);

#ifdef __cplusplus
}
#endif

#endif /* FERRET_HIP_H_ */
