"""PyTorch-facing wrappers over the C ABI (device tensors in, device tensors out).

Every wrapper validates dtype / device / contiguity / shape on the host, passes
raw device pointers plus the current HIP stream, and raises FerretError on a
non-zero return code.  There is no CPU path.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import lib as _lib

FP8 = torch.float8_e4m3fn


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dev(t: torch.Tensor, name: str, dtype=None, ndim=None) -> int:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got {t.device}); ferret_amd has no CPU path")
    if dtype is not None and t.dtype not in (dtype if isinstance(dtype, tuple) else (dtype,)):
        raise TypeError(f"{name} must have dtype {dtype}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


def _out(t: torch.Tensor, name: str, shape: tuple, dtype, device) -> int:
    """Validate a caller-supplied output (or secondary input) tensor: exact shape,
    dtype, contiguity and the same device as the inputs; a smaller buffer would
    let the kernel write past its allocation."""
    ptr = _dev(t, name, dtype)
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, the inputs on {device}")
    return ptr


def _same_device(*ts) -> None:
    devs = {t.device for t in ts if t is not None}
    if len(devs) > 1:
        raise ValueError(f"all tensors must be on one device, got {sorted(str(d) for d in devs)}")


def linear_workspace_bytes(M: int, N: int, K: int) -> int:
    """Split-K workspace ferret_linear_bf16 can use for this shape (0: none)."""
    return int(_lib.load().ferret_workspace_bytes(0, M, N, K, 0))


def linear_bf16(x: torch.Tensor, w: torch.Tensor, residual: torch.Tensor | None = None,
                out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """y[M,N] = x[M,K] @ w[N,K]^T (+ residual), bf16 in/out, fp32 accumulate.

    Shapes that split K (see ferret_hip.h) take their fp32 partials from
    `workspace`, or from torch's caching allocator when none (or a too small
    one) is passed.
    """
    _dev(x, "x", torch.bfloat16, 2)
    _dev(w, "w", torch.bfloat16, 2)
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"w must be [N, {K}], got {tuple(w.shape)}")
    _same_device(x, w, residual, out, workspace)
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    _out(out, "out", (M, N), torch.bfloat16, x.device)
    rp = 0
    if residual is not None:
        rp = _out(residual, "residual", (M, N), torch.bfloat16, x.device)
    need = linear_workspace_bytes(M, N, K) if K % 128 == 0 and N % 16 == 0 else 0
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    rc = _lib.load().ferret_linear_bf16(_dev(x, "x", torch.bfloat16, 2), _dev(w, "w", torch.bfloat16, 2), rp,
                                        _dev(out, "out", torch.bfloat16, 2), M, N, K,
                                        _dev(workspace, "workspace") if need else None, need, _stream())
    _lib.check("ferret_linear_bf16", rc)
    return out


def fp8_workspace_bytes(M: int, N: int, K: int) -> int:
    """Bytes of split-K workspace ferret_fp8_gemm_blockscale uses for this shape (0 if none)."""
    return int(_lib.load().ferret_workspace_bytes(1, M, N, K, 0))


def _mma_flags(mma: str) -> int:
    if mma == "bf16":
        return 0
    if mma == "e4m3":
        return _lib.FP8_MMA_E4M3
    raise ValueError(f"mma must be 'bf16' (exact widening, the default) or 'e4m3' (FP8 MFMA), got {mma!r}")


def fp8_gemm_blockscale(a: torch.Tensor, sa: torch.Tensor, b: torch.Tensor, sb: torch.Tensor,
                        out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                        mma: str = "bf16") -> torch.Tensor:
    """c[M,N] (bf16) = block-scaled a[M,K] (e4m3) . b[N,K]^T (e4m3).

    Shapes with M <= 256 run split-K over a workspace; pass one of at least
    fp8_workspace_bytes(M, N, K) bytes to reuse it across calls (else one is
    taken from torch's caching allocator).  mma="e4m3" opts the tiled (M > 16)
    kernels into the FP8 MFMA (FERRET_FP8_MMA_E4M3: faster, less precise).
    """
    _dev(a, "a", (FP8, torch.uint8), 2)
    _dev(b, "b", (FP8, torch.uint8), 2)
    M, K = a.shape
    N = b.shape[0]
    if b.shape[1] != K:
        raise ValueError("b must be [N, K]")
    if tuple(sa.shape) != (M, K // 128) or tuple(sb.shape) != ((N + 127) // 128, K // 128):
        raise ValueError(f"scale shapes must be sa [M, K/128], sb [ceil(N/128), K/128]; got {tuple(sa.shape)}, {tuple(sb.shape)}")
    _same_device(a, sa, b, sb, out, workspace)
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    _out(out, "out", (M, N), torch.bfloat16, a.device)
    need = fp8_workspace_bytes(M, N, K)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=a.device)
    ws_ptr = _dev(workspace, "workspace") if need else None
    rc = _lib.load().ferret_fp8_gemm_blockscale_ex(
        _dev(a, "a", (FP8, torch.uint8), 2), _dev(sa, "sa", torch.float32, 2), _dev(b, "b", (FP8, torch.uint8), 2),
        _dev(sb, "sb", torch.float32, 2), _dev(out, "out", torch.bfloat16, 2), M, N, K, ws_ptr, need,
        _mma_flags(mma), _stream())
    _lib.check("ferret_fp8_gemm_blockscale", rc)
    return out


_SQRT_HALF = 2.0 ** -0.5


def ue8m0_from_float(scales: torch.Tensor) -> torch.Tensor:
    """UE8M0 bytes (uint8) of fp32 scales: the exponent byte of the power of
    two nearest in log2 (float_to_ue8m0,
    examples/fp8-gemm/v009_large_m_block_scale_mma_080.cu:375-384), taken from
    the mantissa (nearer the upper power when it is >= 2^-0.5) rather than
    from a rounded logarithm.  s <= 0 gives 0; +inf and NaN give 255; the
    exponent is clamped to the byte (subnormal powers 0, 2^128 and up 255).
    Host-side preparation of inputs, any device."""
    x = scales.to(torch.float32)
    m, e = torch.frexp(torch.where(torch.isfinite(x) & (x > 0), x, torch.ones_like(x)))
    k = e.to(torch.int64) - 1 + (m.to(torch.float64) >= _SQRT_HALF).to(torch.int64)  # exact: no float is 2^-0.5
    byte = torch.where(x > 0, (k + 127).clamp(0, 255), torch.zeros_like(k))
    byte = torch.where(torch.isnan(x) | (x == float("inf")), torch.full_like(k, 255), byte)
    return byte.to(torch.uint8)


def pack_ue8m0(ue: torch.Tensor) -> torch.Tensor:
    """UE8M0 bytes [dim, nk] -> int32 words [ceil(nk/4), dim] (prepare_sf,
    v009:386-403): byte j of word [sk, d] is ue[d, 4 sk + j], missing K-blocks 0."""
    if ue.dtype != torch.uint8 or ue.dim() != 2:
        raise ValueError("ue must be uint8 [dim, nk]")
    dim, nk = ue.shape
    nsk = (nk + 3) // 4
    padded = torch.zeros((dim, nsk * 4), dtype=torch.uint8, device=ue.device)
    padded[:, :nk] = ue
    return padded.view(dim, nsk, 4).permute(1, 0, 2).contiguous().view(torch.int32).view(nsk, dim)


def expand_block_scales(sb: torch.Tensor, N: int) -> torch.Tensor:
    """Weight block scales [ceil(N/128), nk] -> one row per weight row [N, nk]
    (expand_sb, v009:405-412)."""
    if sb.dim() != 2 or sb.shape[0] != (N + 127) // 128:
        raise ValueError("sb must be [ceil(N/128), nk]")
    return sb.repeat_interleave(128, dim=0)[:N].contiguous()


def fp8_ue8m0_workspace_bytes(M: int, N: int, K: int) -> int:
    """Workspace bytes ferret_fp8_gemm_ue8m0 needs (decoded scales + split-K partials)."""
    return int(_lib.load().ferret_workspace_bytes(5, M, N, K, 0))


def fp8_gemm_ue8m0(a: torch.Tensor, sfa: torch.Tensor, b: torch.Tensor, sfb: torch.Tensor,
                   out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """c[M,N] (bf16) = a[M,K] (e4m3) . b[N,K]^T (e4m3) with UE8M0 block scales.

    sfa: int32 words [ceil(nk/4), M] and sfb: int32 words [ceil(nk/4), N] in
    the reference's packed layout (pack_ue8m0 of ue8m0_from_float, sfb over
    expand_block_scales); nk = K/128.  A workspace of fp8_ue8m0_workspace_bytes
    is taken from torch's caching allocator unless one is passed.
    """
    _dev(a, "a", (FP8, torch.uint8), 2)
    _dev(b, "b", (FP8, torch.uint8), 2)
    M, K = a.shape
    N = b.shape[0]
    if b.shape[1] != K:
        raise ValueError("b must be [N, K]")
    nsk = (K // 128 + 3) // 4
    if tuple(sfa.shape) != (nsk, M) or tuple(sfb.shape) != (nsk, N):
        raise ValueError(f"packed scales must be sfa [{nsk}, M], sfb [{nsk}, N]; got {tuple(sfa.shape)}, "
                         f"{tuple(sfb.shape)}")
    _same_device(a, sfa, b, sfb, out, workspace)
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    _out(out, "out", (M, N), torch.bfloat16, a.device)
    need = fp8_ue8m0_workspace_bytes(M, N, K)
    if need == 0:
        raise ValueError(f"unsupported shape M={M} N={N} K={K}")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=a.device)
    rc = _lib.load().ferret_fp8_gemm_ue8m0(
        _dev(a, "a", (FP8, torch.uint8), 2), _dev(sfa, "sfa", torch.int32, 2), _dev(b, "b", (FP8, torch.uint8), 2),
        _dev(sfb, "sfb", torch.int32, 2), _dev(out, "out", torch.bfloat16, 2), M, N, K,
        _dev(workspace, "workspace"), workspace.numel() * workspace.element_size(), _stream())
    _lib.check("ferret_fp8_gemm_ue8m0", rc)
    return out


def moe_route_topk(logits: torch.Tensor, topk: int, with_weights: bool = True):
    """ids int32 [T, topk] (logit desc, expert asc) and softmax weights [T, topk]."""
    T, E = logits.shape
    ids = torch.empty((T, topk), dtype=torch.int32, device=logits.device)
    w = torch.empty((T, topk), dtype=torch.float32, device=logits.device) if with_weights else None
    rc = _lib.load().ferret_moe_route_topk(_dev(logits, "logits", torch.float32, 2), T, E, topk,
                                           _dev(ids, "ids"), w.data_ptr() if w is not None else 0, _stream())
    _lib.check("ferret_moe_route_topk", rc)
    return ids, w


@dataclass
class Routing:
    """Device tensors describing how routed pairs are grouped by expert."""
    counts: torch.Tensor        # int32 [E]
    offsets: torch.Tensor       # int32 [E+1]
    sorted_pair: torch.Tensor   # int32 [P]
    tiles: torch.Tensor         # int32 [max_tiles, 3]
    ntiles: torch.Tensor        # int32 [1]
    tile_m: int
    max_tiles: int
    num_experts: int
    topk: int
    num_tokens: int


def tile_m_for(num_pairs: int, num_experts: int) -> int:
    return int(_lib.load().ferret_moe_tile_m(num_pairs, num_experts))


def moe_permute(ids: torch.Tensor, num_experts: int, tile_m: int | None = None,
                workspace: torch.Tensor | None = None) -> Routing:
    """Stable expert-major permutation + tile table of the routed pairs.

    Large P runs over several work-groups through a workspace of
    ferret_workspace_bytes(4, P, 0, 0, E) bytes (taken from torch's caching
    allocator unless one at least that large is passed).
    """
    T, topk = ids.shape
    P = T * topk
    if tile_m is None:
        tile_m = tile_m_for(P, num_experts)
    L = _lib.load()
    need = int(L.ferret_workspace_bytes(4, P, 0, 0, num_experts))
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=ids.device)
    max_tiles = max(1, int(L.ferret_moe_max_tiles(P, num_experts, tile_m)))
    dev = ids.device
    r = Routing(
        counts=torch.empty(num_experts, dtype=torch.int32, device=dev),
        offsets=torch.empty(num_experts + 1, dtype=torch.int32, device=dev),
        sorted_pair=torch.empty(max(P, 1), dtype=torch.int32, device=dev),
        tiles=torch.empty((max_tiles, 3), dtype=torch.int32, device=dev),
        ntiles=torch.empty(1, dtype=torch.int32, device=dev),
        tile_m=tile_m, max_tiles=max_tiles, num_experts=num_experts, topk=topk, num_tokens=T)
    rc = L.ferret_moe_permute(_dev(ids, "ids", torch.int32, 2), T, topk, num_experts, tile_m,
                              r.counts.data_ptr(), r.offsets.data_ptr(), r.sorted_pair.data_ptr(),
                              r.tiles.data_ptr(), max_tiles, r.ntiles.data_ptr(),
                              _dev(workspace, "workspace") if need else None, need, _stream())
    _lib.check("ferret_moe_permute", rc)
    return r


def moe_w13_fp8(x: torch.Tensor, sx: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, routing: Routing,
                out: torch.Tensor | None = None, mma: str = "bf16") -> torch.Tensor:
    """out[P, N/2] bf16 = silu(gate) * up of the FP8 block-scaled w13 projection."""
    T, K = x.shape
    E, N, K2 = w.shape
    if K2 != K or E != routing.num_experts or T != routing.num_tokens:
        raise ValueError("shape mismatch between x, w and routing")
    if tuple(sx.shape) != (T, K // 128) or tuple(sw.shape) != (E, N // 128, K // 128):
        raise ValueError("scale shapes must be sx [T, K/128], sw [E, N/128, K/128]")
    _same_device(x, sx, w, sw, routing.sorted_pair, routing.tiles, out)
    P = T * routing.topk
    if out is None:
        out = torch.empty((P, N // 2), dtype=torch.bfloat16, device=x.device)
    _out(out, "out", (P, N // 2), torch.bfloat16, x.device)
    rc = _lib.load().ferret_moe_w13_fp8_ex(
        _dev(x, "x", (FP8, torch.uint8), 2), _dev(sx, "sx", torch.float32, 2), _dev(w, "w", (FP8, torch.uint8), 3),
        _dev(sw, "sw", torch.float32, 3), routing.sorted_pair.data_ptr(), routing.tiles.data_ptr(),
        routing.ntiles.data_ptr(), routing.max_tiles, routing.tile_m, T, routing.topk, E, N, K,
        _dev(out, "out", torch.bfloat16, 2), _mma_flags(mma), _stream())
    _lib.check("ferret_moe_w13_fp8", rc)
    return out


def int4_tile_weights(wq: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """The INT4 w13 weights wq [E, N, K/8] int32 regrouped into 16-row x 128-K
    tiles: int32 [E, N/16, K/128, 16, 16], tile (e, b, k) = the 64 bytes of
    K-step k of rows 16b .. 16b+15 of expert e.  A one-time load-time
    permutation of the checkpoint words (no value changes); moe_w13_w4a16 on
    the result streams each tile as one contiguous KB."""
    _dev(wq, "wq", torch.int32, 3)
    E, N, K8 = wq.shape
    K = K8 * 8
    if N % 16 != 0 or K % 128 != 0:
        raise ValueError("int4_tile_weights needs N % 16 == 0 and K % 128 == 0")
    _same_device(wq, out)
    shape = (E, N // 16, K // 128, 16, 16)
    if out is None:
        out = torch.empty(shape, dtype=torch.int32, device=wq.device)
    rc = _lib.load().ferret_int4_tile_weights(wq.data_ptr(), _out(out, "out", shape, torch.int32, wq.device),
                                              E, N, K, _stream())
    _lib.check("ferret_int4_tile_weights", rc)
    return out


def moe_w13_w4a16(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, routing: Routing,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """out[P, N/2] bf16 = silu(gate) * up of the INT4 W4A16 w13 projection.
    wq: the checkpoint words int32 [E, N, K/8], or their tiles from
    int4_tile_weights (int32 [E, N/16, K/128, 16, 16]); the result is the same
    bit for bit."""
    T, K = x.shape
    tiled = wq.dim() == 5
    if tiled:
        E, NB, KB, R, C = wq.shape
        if (R, C) != (16, 16) or KB * 128 != K:
            raise ValueError("tiled wq must be [E, N/16, K/128, 16, 16] int32")
        N = NB * 16
    else:
        E, N, K8 = wq.shape
        if K8 * 8 != K:
            raise ValueError("shape mismatch between x and wq")
    if E != routing.num_experts or T != routing.num_tokens:
        raise ValueError("shape mismatch between x, wq and routing")
    if tuple(ws.shape) != (E, N, K // 32):
        raise ValueError("ws must be [E, N, K/32] bf16")
    _same_device(x, wq, ws, routing.sorted_pair, routing.tiles, out)
    P = T * routing.topk
    if out is None:
        out = torch.empty((P, N // 2), dtype=torch.bfloat16, device=x.device)
    _out(out, "out", (P, N // 2), torch.bfloat16, x.device)
    lib = _lib.load()
    fn, name = ((lib.ferret_moe_w13_w4a16_tiled, "ferret_moe_w13_w4a16_tiled") if tiled
                else (lib.ferret_moe_w13_w4a16, "ferret_moe_w13_w4a16"))
    rc = fn(_dev(x, "x", torch.bfloat16, 2), _dev(wq, "wq", torch.int32, wq.dim()), _dev(ws, "ws", torch.bfloat16, 3),
            routing.sorted_pair.data_ptr(), routing.tiles.data_ptr(), routing.ntiles.data_ptr(), routing.max_tiles,
            routing.tile_m, T, routing.topk, E, N, K, _dev(out, "out", torch.bfloat16, 2), _stream())
    _lib.check(name, rc)
    return out


def quant_act_e4m3(x: torch.Tensor, q: torch.Tensor | None = None, scale: torch.Tensor | None = None):
    """bf16 x [M, K] -> (e4m3 q [M, K], fp32 scale [M, K/128]) by the 1x128 absmax/448 rule."""
    _dev(x, "x", torch.bfloat16, 2)
    M, K = x.shape
    _same_device(x, q, scale)
    if q is None:
        q = torch.empty((M, K), dtype=FP8, device=x.device)
    if scale is None:
        scale = torch.empty((M, K // 128), dtype=torch.float32, device=x.device)
    rc = _lib.load().ferret_quant_act_e4m3(_dev(x, "x", torch.bfloat16, 2),
                                           _out(q, "q", (M, K), (FP8, torch.uint8), x.device),
                                           _out(scale, "scale", (M, K // 128), torch.float32, x.device), M, K,
                                           _stream())
    _lib.check("ferret_quant_act_e4m3", rc)
    return q, scale


def moe_w2_fp8(h: torch.Tensor, sh: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, routing: Routing,
               out: torch.Tensor | None = None, mma: str = "bf16") -> torch.Tensor:
    """out[P, N] bf16 (pair order) = the FP8 block-scaled down projection of h [P, K] (pair order)."""
    P, K = h.shape
    E, N, K2 = w.shape
    if K2 != K or E != routing.num_experts or P != routing.num_tokens * routing.topk:
        raise ValueError("shape mismatch between h, w and routing")
    if tuple(sh.shape) != (P, K // 128) or tuple(sw.shape) != (E, N // 128, K // 128):
        raise ValueError("scale shapes must be sh [P, K/128], sw [E, N/128, K/128]")
    _same_device(h, sh, w, sw, routing.sorted_pair, routing.tiles, out)
    if out is None:
        out = torch.empty((P, N), dtype=torch.bfloat16, device=h.device)
    _out(out, "out", (P, N), torch.bfloat16, h.device)
    rc = _lib.load().ferret_moe_w2_fp8_ex(
        _dev(h, "h", (FP8, torch.uint8), 2), _dev(sh, "sh", torch.float32, 2), _dev(w, "w", (FP8, torch.uint8), 3),
        _dev(sw, "sw", torch.float32, 3), routing.sorted_pair.data_ptr(), routing.tiles.data_ptr(),
        routing.ntiles.data_ptr(), routing.max_tiles, routing.tile_m, P, E, N, K,
        _dev(out, "out", torch.bfloat16, 2), _mma_flags(mma), _stream())
    _lib.check("ferret_moe_w2_fp8", rc)
    return out


def moe_combine(o: torch.Tensor, weights: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """y[T, N] bf16 = sum_j weights[t, j] * o[t*topk + j] (fp32, j order)."""
    T, topk = weights.shape
    P, N = o.shape
    if P != T * topk:
        raise ValueError("o must hold T*topk rows in pair order")
    _same_device(o, weights, out)
    if out is None:
        out = torch.empty((T, N), dtype=torch.bfloat16, device=o.device)
    _out(out, "out", (T, N), torch.bfloat16, o.device)
    rc = _lib.load().ferret_moe_combine(_dev(o, "o", torch.bfloat16, 2), _dev(weights, "weights", torch.float32, 2),
                                        T, topk, N, _dev(out, "out", torch.bfloat16, 2), _stream())
    _lib.check("ferret_moe_combine", rc)
    return out
