"""ferret_linear_bf16_noalloc (the allocation-free decode linear) against
ferret_linear_bf16 with a caller workspace, through the C ABI.

Two split-K calls in a row share the library's device array (the second with a
smaller input, so stale partials of the first remain beyond it); each must be
bit-identical to the workspace entry point and within the oracle's tolerance.
A shape that needs no split runs without the array; one whose partials exceed
the array is rejected before any launch (also checked on the CPU in
test_abi.py).
"""
import numpy as np
import pytest
import torch

from oracle import gemm as G
from tests.gpu_helpers import assert_gemm_close, bf16_out, bits16

pytestmark = pytest.mark.gpu


def _run(L, M, N, K, res, seed):
    from ferret_amd import workloads as W
    x = W.randn((M, K), seed, "cuda").to(torch.bfloat16)
    w = W.randn((N, K), seed + 1, "cuda", std=0.02).to(torch.bfloat16)
    r = W.randn((M, N), seed + 2, "cuda").to(torch.bfloat16) if res else None
    stream = torch.cuda.current_stream().cuda_stream
    need = int(L.ferret_workspace_bytes(0, M, N, K, 0))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    y_ws = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    y_na = torch.full((M, N), -1.0, dtype=torch.bfloat16, device="cuda")
    rp = r.data_ptr() if r is not None else None
    assert L.ferret_linear_bf16(x.data_ptr(), w.data_ptr(), rp, y_ws.data_ptr(), M, N, K,
                                ws.data_ptr() if need else None, need, stream) == 0
    assert L.ferret_linear_bf16_noalloc(x.data_ptr(), w.data_ptr(), rp, y_na.data_ptr(), M, N, K, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(y_na.view(torch.int16), y_ws.view(torch.int16)), f"M={M} N={N} K={K}: differs"
    ref = G.linear_bf16(bits16(x), bits16(w), bits16(r) if r is not None else None)
    assert_gemm_close(bf16_out(y_na), ref, f"noalloc M={M} N={N} K={K}")
    return need


def test_noalloc_matches_workspace_entry_point(hip):
    L = hip
    limit = int(L.ferret_linear_bf16_noalloc_max_bytes())
    assert limit == 4 << 20
    # QKV-shaped, then a smaller Down-shaped call with a residual: both split K
    assert 0 < _run(L, 16, 6144, 4096, False, 11) <= limit
    assert 0 < _run(L, 5, 4096, 12288, True, 21) <= limit
    # one unit per CU: no split, no array
    assert _run(L, 16, 4096, 4096, True, 31) == 0


def test_noalloc_rejects_partials_beyond_the_array(hip):
    L = hip
    M, N, K = 100, 4096, 12288
    need = int(L.ferret_workspace_bytes(0, M, N, K, 0))
    assert need > int(L.ferret_linear_bf16_noalloc_max_bytes())
    x = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((N, K), dtype=torch.bfloat16, device="cuda")
    y = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
    rc = L.ferret_linear_bf16_noalloc(x.data_ptr(), w.data_ptr(), None, y.data_ptr(), M, N, K,
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == -3
    assert L.ferret_error_string(rc).decode().startswith("workspace")


def test_noalloc_under_graph_capture(hip):
    """Captured into a HIP graph (after the address lookup that
    ferret_linear_bf16_noalloc_max_bytes does), every replay with new inputs is
    bit-identical to the workspace entry point run eagerly on the same inputs."""
    from ferret_amd import workloads as W
    L = hip
    M, N, K = 16, 6144, 4096                      # splits K: partials in the library's array
    assert int(L.ferret_workspace_bytes(0, M, N, K, 0)) > 0
    assert int(L.ferret_linear_bf16_noalloc_max_bytes()) == 4 << 20
    x = torch.empty((M, K), dtype=torch.bfloat16, device="cuda")
    w = W.randn((N, K), 41, "cuda", std=0.02).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    x.copy_(W.randn((M, K), 40, "cuda").to(torch.bfloat16))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                 # warm-up off the default stream, as capture requires
        assert L.ferret_linear_bf16_noalloc(x.data_ptr(), w.data_ptr(), None, y.data_ptr(), M, N, K,
                                            side.cuda_stream) == 0
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = L.ferret_linear_bf16_noalloc(x.data_ptr(), w.data_ptr(), None, y.data_ptr(), M, N, K,
                                          torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    need = int(L.ferret_workspace_bytes(0, M, N, K, 0))
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    ref = torch.empty_like(y)
    stream = torch.cuda.current_stream().cuda_stream
    for rep in range(3):
        x.copy_(W.randn((M, K), 50 + rep, "cuda").to(torch.bfloat16))
        y.fill_(-1.0)
        g.replay()
        torch.cuda.synchronize()
        assert L.ferret_linear_bf16(x.data_ptr(), w.data_ptr(), None, ref.data_ptr(), M, N, K, ws.data_ptr(),
                                    need, stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"replay {rep} differs"
