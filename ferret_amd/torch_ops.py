"""torch.library operators over the C ABI (namespace ``ferret``).

The reference binds its GEMM to PyTorch as ``TORCH_LIBRARY(my_matmul)`` ops
``matmul_vX(Tensor A, Tensor B) -> Tensor`` that allocate the output with
``at::empty`` and call the raw kernel on the current stream
(``examples/tcgen05-gemm/matmul.cpp:5,21-33,73-95``).  This module registers
the same kind of functional operators for every entry point of the hot path,
with ``torch.library.custom_op``: the real kernel runs through
``ferret_amd.ops`` (output and workspace from torch's caching allocator, the
current HIP stream), and each op carries a fake (meta) implementation that
states its output shapes, so the ops trace under ``torch.compile`` and
``torch.export`` and run inside captured HIP graphs.

    import ferret_amd.torch_ops  # registers torch.ops.ferret.*
    c = torch.ops.ferret.fp8_gemm_blockscale(a, sa, b, sb)

Importing this module needs no GPU; calling an op on CPU tensors raises (there
is no CPU path).
"""
from __future__ import annotations

import torch

from . import lib as _lib
from . import ops as _ops

FP8 = torch.float8_e4m3fn
_NS = "ferret"


def _routing(sorted_pair, tiles, ntiles, tile_m: int, topk: int, num_experts: int, num_tokens: int):
    return _ops.Routing(counts=None, offsets=None, sorted_pair=sorted_pair, tiles=tiles, ntiles=ntiles,
                        tile_m=tile_m, max_tiles=tiles.shape[0], num_experts=num_experts, topk=topk,
                        num_tokens=num_tokens)


# ---- dense -------------------------------------------------------------------------------------

@torch.library.custom_op(f"{_NS}::linear_bf16", mutates_args=())
def linear_bf16(x: torch.Tensor, w: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
    """y[M,N] = x[M,K] @ w[N,K]^T (+ residual), bf16 (ferret_linear_bf16)."""
    return _ops.linear_bf16(x, w, residual=residual)


@linear_bf16.register_fake
def _(x, w, residual=None):
    return x.new_empty((x.shape[0], w.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::fp8_gemm_blockscale", mutates_args=())
def fp8_gemm_blockscale(a: torch.Tensor, sa: torch.Tensor, b: torch.Tensor, sb: torch.Tensor) -> torch.Tensor:
    """c[M,N] bf16 of e4m3 a[M,K], b[N,K] with fp32 1x128 / 128x128 block scales."""
    return _ops.fp8_gemm_blockscale(a, sa, b, sb)


@fp8_gemm_blockscale.register_fake
def _(a, sa, b, sb):
    return a.new_empty((a.shape[0], b.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::fp8_gemm_ue8m0", mutates_args=())
def fp8_gemm_ue8m0(a: torch.Tensor, sfa: torch.Tensor, b: torch.Tensor, sfb: torch.Tensor) -> torch.Tensor:
    """c[M,N] bf16 of e4m3 a, b with packed UE8M0 block scales (ferret_fp8_gemm_ue8m0)."""
    return _ops.fp8_gemm_ue8m0(a, sfa, b, sfb)


@fp8_gemm_ue8m0.register_fake
def _(a, sfa, b, sfb):
    return a.new_empty((a.shape[0], b.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::quant_act_e4m3", mutates_args=())
def quant_act_e4m3(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 x[M,K] -> (e4m3 q[M,K], fp32 scale[M,K/128]), 1x128 absmax/448."""
    return _ops.quant_act_e4m3(x)


@quant_act_e4m3.register_fake
def _(x):
    M, K = x.shape
    return x.new_empty((M, K), dtype=FP8), x.new_empty((M, K // 128), dtype=torch.float32)


# ---- MoE routing ---------------------------------------------------------------------------------

@torch.library.custom_op(f"{_NS}::moe_route_topk", mutates_args=())
def moe_route_topk(logits: torch.Tensor, topk: int) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 logits[T,E] -> (int32 ids[T,topk], fp32 softmax weights[T,topk])."""
    return _ops.moe_route_topk(logits, topk, with_weights=True)


@moe_route_topk.register_fake
def _(logits, topk):
    T = logits.shape[0]
    return logits.new_empty((T, topk), dtype=torch.int32), logits.new_empty((T, topk), dtype=torch.float32)


def moe_tile_m(num_pairs, num_experts: int):
    """ferret_moe_tile_m (routing.hip) in Python, so that fake tensors and
    symbolic pair counts need no library call: 128-row tiles from an average
    of 32 rows per expert, else 16."""
    return 128 if num_experts > 0 and num_pairs // num_experts >= 32 else 16


def moe_max_tiles(num_pairs, num_experts: int, tile_m: int):
    """ferret_moe_max_tiles (routing.hip) in Python: min(ceil(P / tile_m) + E, P),
    0 without pairs; works on SymInts (torch.sym_min)."""
    if num_pairs <= 0 or tile_m <= 0:
        return 0
    return torch.sym_min((num_pairs + tile_m - 1) // tile_m + num_experts, num_pairs)


def _tile_m(num_pairs, num_experts: int, tile_m: int):
    return tile_m if tile_m > 0 else moe_tile_m(num_pairs, num_experts)


@torch.library.custom_op(f"{_NS}::moe_permute", mutates_args=())
def moe_permute(ids: torch.Tensor, num_experts: int, tile_m: int = 0) -> tuple[torch.Tensor, torch.Tensor,
                                                                                torch.Tensor, torch.Tensor,
                                                                                torch.Tensor]:
    """ids[T,topk] -> (counts[E], offsets[E+1], sorted_pair[P], tiles[max_tiles,3], ntiles[1]);
    tile_m 0 picks the library's choice (ferret_moe_tile_m)."""
    P = ids.shape[0] * ids.shape[1]
    r = _ops.moe_permute(ids, num_experts, tile_m=_tile_m(P, num_experts, tile_m))
    return r.counts, r.offsets, r.sorted_pair, r.tiles, r.ntiles


@moe_permute.register_fake
def _(ids, num_experts, tile_m=0):
    P = ids.shape[0] * ids.shape[1]
    tm = _tile_m(P, num_experts, tile_m)
    max_tiles = torch.sym_max(1, moe_max_tiles(P, num_experts, tm))
    i32 = dict(dtype=torch.int32)
    return (ids.new_empty((num_experts,), **i32), ids.new_empty((num_experts + 1,), **i32),
            ids.new_empty((torch.sym_max(P, 1),), **i32), ids.new_empty((max_tiles, 3), **i32),
            ids.new_empty((1,), **i32))


# ---- MoE GEMMs and tail ----------------------------------------------------------------------------

@torch.library.custom_op(f"{_NS}::moe_w13_fp8", mutates_args=())
def moe_w13_fp8(x: torch.Tensor, sx: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, sorted_pair: torch.Tensor,
                tiles: torch.Tensor, ntiles: torch.Tensor, tile_m: int, topk: int) -> torch.Tensor:
    """silu(gate) * up [T*topk, N/2] bf16 of the FP8 w13 grouped GEMM over moe_permute's tables."""
    r = _routing(sorted_pair, tiles, ntiles, tile_m, topk, w.shape[0], x.shape[0])
    return _ops.moe_w13_fp8(x, sx, w, sw, r)


@moe_w13_fp8.register_fake
def _(x, sx, w, sw, sorted_pair, tiles, ntiles, tile_m, topk):
    return x.new_empty((x.shape[0] * topk, w.shape[1] // 2), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::moe_w13_w4a16", mutates_args=())
def moe_w13_w4a16(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, sorted_pair: torch.Tensor,
                  tiles: torch.Tensor, ntiles: torch.Tensor, tile_m: int, topk: int) -> torch.Tensor:
    """silu(gate) * up [T*topk, N/2] bf16 of the INT4 W4A16 w13 grouped GEMM."""
    r = _routing(sorted_pair, tiles, ntiles, tile_m, topk, wq.shape[0], x.shape[0])
    return _ops.moe_w13_w4a16(x, wq, ws, r)


@moe_w13_w4a16.register_fake
def _(x, wq, ws, sorted_pair, tiles, ntiles, tile_m, topk):
    n = wq.shape[1] * 16 if wq.dim() == 5 else wq.shape[1]  # tiled [E, N/16, K/128, 16, 16] or [E, N, K/8]
    return x.new_empty((x.shape[0] * topk, n // 2), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::int4_tile_weights", mutates_args=())
def int4_tile_weights(wq: torch.Tensor) -> torch.Tensor:
    """INT4 w13 words [E, N, K/8] int32 -> 16-row x 128-K tiles [E, N/16, K/128, 16, 16] int32."""
    return _ops.int4_tile_weights(wq)


@int4_tile_weights.register_fake
def _(wq):
    E, N, K8 = wq.shape
    return wq.new_empty((E, N // 16, K8 // 16, 16, 16), dtype=torch.int32)


@torch.library.custom_op(f"{_NS}::moe_w2_fp8", mutates_args=())
def moe_w2_fp8(h: torch.Tensor, sh: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, sorted_pair: torch.Tensor,
               tiles: torch.Tensor, ntiles: torch.Tensor, tile_m: int, topk: int) -> torch.Tensor:
    """[T*topk, N] bf16 (pair order) of the FP8 w2 (down) grouped GEMM of h [T*topk, K]."""
    r = _routing(sorted_pair, tiles, ntiles, tile_m, topk, w.shape[0], h.shape[0] // topk)
    return _ops.moe_w2_fp8(h, sh, w, sw, r)


@moe_w2_fp8.register_fake
def _(h, sh, w, sw, sorted_pair, tiles, ntiles, tile_m, topk):
    return h.new_empty((h.shape[0], w.shape[1]), dtype=torch.bfloat16)


@torch.library.custom_op(f"{_NS}::moe_combine", mutates_args=())
def moe_combine(o: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """y[T,N] bf16 = sum_j weights[t,j] * o[t*topk + j]."""
    return _ops.moe_combine(o, weights)


@moe_combine.register_fake
def _(o, weights):
    return o.new_empty((weights.shape[0], o.shape[1]), dtype=torch.bfloat16)


OPS = ("linear_bf16", "fp8_gemm_blockscale", "fp8_gemm_ue8m0", "quant_act_e4m3", "moe_route_topk", "moe_permute",
       "moe_w13_fp8", "moe_w13_w4a16", "int4_tile_weights", "moe_w2_fp8", "moe_combine")
