"""CPU checks of the C-ABI boundary: the library loads and exports every declared symbol."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ferret_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(\w+)\s*\(", text, flags=re.M)) - {"defined"})


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for must in ("launch_gemv", "ferret_linear_bf16", "ferret_fp8_gemm_blockscale", "ferret_moe_route_topk",
                 "ferret_moe_permute", "ferret_moe_w13_fp8", "ferret_moe_w13_w4a16", "ferret_workspace_bytes",
                 "ferret_quant_act_e4m3", "ferret_moe_w2_fp8", "ferret_moe_combine"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from ferret_amd import lib
    if not os.path.exists(lib.LIB_PATH):
        pytest.skip("libferret_hip.so not built (run python -m ferret_amd.build)")
    L = lib.load()
    for name in declared_functions():
        assert hasattr(L, name), f"{name} declared in ferret_hip.h but not exported"
    assert set(declared_functions()) == set(lib.SIGNATURES), "ctypes signature table out of sync with the header"


def test_version_and_error_strings_without_gpu():
    from ferret_amd import lib
    if not os.path.exists(lib.LIB_PATH):
        pytest.skip("libferret_hip.so not built")
    assert lib.version().startswith("ferret-hip")
    L = lib.load()
    assert L.ferret_error_string(-2).decode().startswith("sizes")
    assert L.ferret_moe_max_tiles(1024, 256, 16) == 320
    assert L.ferret_moe_tile_m(1024, 256) == 16 and L.ferret_moe_tile_m(32768, 256) == 128


def test_argument_errors_are_returned_not_raised_without_gpu():
    """Rejected arguments return a code before any HIP call (safe on a GPU-less host)."""
    from ferret_amd import lib
    if not os.path.exists(lib.LIB_PATH):
        pytest.skip("libferret_hip.so not built")
    L = lib.load()
    assert L.ferret_linear_bf16(None, None, None, None, 1, 16, 128, None, 0, None) == -1
    assert L.ferret_linear_bf16(1, 1, None, 1, 1, 17, 128, None, 0, None) == -2
    assert L.ferret_fp8_gemm_blockscale(1, 1, 1, 1, 1, 4, 64, 100, None, 0, None) == -2
    assert L.ferret_moe_route_topk(1, 4, 2000, 8, 1, None, None) == -2
    assert L.ferret_moe_permute(1, 4, 8, 16, 16, 1, 1, 1, 1, 0, 1, None, 0, None) == -2
    assert L.ferret_workspace_bytes(4, 1024, 0, 0, 256) == 0          # one work-group
    assert L.ferret_workspace_bytes(4, 32768, 0, 0, 256) == 32 * 256 * 4
    assert L.ferret_moe_w13_w4a16(1, 1, 1, 1, 1, 1, 10, 128, 4, 8, 16, 64, 256, 1, None) == -2
    assert L.ferret_workspace_bytes(0, 16, 6144, 4096, 0) == 2 * 16 * 6144 * 4    # QKV: 2 K splits
    assert L.ferret_workspace_bytes(0, 16, 4096, 12288, 0) == 3 * 16 * 4096 * 4   # Down: 3 K splits
    assert L.ferret_workspace_bytes(0, 16, 4096, 4096, 0) == 0                    # one unit per CU
    assert L.ferret_quant_act_e4m3(None, 1, 1, 4, 256, None) == -1
    assert L.ferret_quant_act_e4m3(1, 1, 1, 4, 200, None) == -2
    assert L.ferret_quant_act_e4m3(1, 1, 1, 0, 256, None) == -2
    assert L.ferret_moe_w2_fp8(1, 1, 1, 1, 1, 1, 1, 10, 16, 64, 8, 7168, 2048, None, None) == -1
    assert L.ferret_moe_w2_fp8(1, 1, 1, 1, 1, 1, 1, 10, 16, 64, 8, 7100, 2048, 1, None) == -2
    assert L.ferret_moe_w2_fp8(1, 1, 1, 1, 1, 1, 1, 10, 32, 64, 8, 7168, 2048, 1, None) == -2   # tile_m
    assert L.ferret_moe_combine(1, 1, 4, 8, 100, 1, None) == -2
    assert L.ferret_moe_combine(1, None, 4, 8, 128, 1, None) == -1
    assert L.ferret_moe_combine(1, 1, 4, 0, 128, 1, None) == -2


def test_fp8_entries_reject_before_launch_without_gpu():
    """The dense and grouped FP8 entry points (and their flag variants) return
    their codes before any HIP call; the pointers are never dereferenced."""
    from ferret_amd import lib
    if not os.path.exists(lib.LIB_PATH):
        pytest.skip("libferret_hip.so not built")
    L = lib.load()
    # dense: a NULL operand, N not a multiple of 128 above 16 rows, K/128 > 128, unknown flag bits
    assert L.ferret_fp8_gemm_blockscale(1, None, 1, 1, 1, 64, 4096, 7168, None, 0, None) == -1
    assert L.ferret_fp8_gemm_blockscale(1, 1, 1, 1, 1, 64, 144, 7168, None, 0, None) == -2
    assert L.ferret_fp8_gemm_blockscale(1, 1, 1, 1, 1, 64, 4096, 128 * 129, None, 0, None) == -2
    assert L.ferret_fp8_gemm_blockscale_ex(1, 1, 1, 1, 1, 64, 4096, 7168, None, 0, 2, None) == -2
    # grouped w13: NULL tile table, N % 256, tile_m other than 16 / 128, unknown flag bits
    args = [1, 1, 1, 1, 1, 1, 1, 320, 16, 128, 8, 256, 4096, 7168, 1]
    bad = list(args); bad[5] = None
    assert L.ferret_moe_w13_fp8(*bad, None) == -1
    bad = list(args); bad[12] = 4096 + 128
    assert L.ferret_moe_w13_fp8(*bad, None) == -2
    bad = list(args); bad[8] = 32
    assert L.ferret_moe_w13_fp8(*bad, None) == -2
    assert L.ferret_moe_w13_fp8_ex(*args, 4, None) == -2
    # grouped w2: unknown flag bits
    assert L.ferret_moe_w2_fp8_ex(1, 1, 1, 1, 1, 1, 1, 10, 16, 64, 8, 7168, 2048, 1, 8, None) == -2


def test_noalloc_linear_rejects_oversized_partials_without_gpu():
    """ferret_linear_bf16_noalloc checks its array limit before any HIP call."""
    from ferret_amd import lib
    if not os.path.exists(lib.LIB_PATH):
        pytest.skip("libferret_hip.so not built")
    L = lib.load()
    assert L.ferret_linear_bf16_noalloc_max_bytes() == 4 << 20
    assert L.ferret_linear_bf16_noalloc(None, 1, None, 1, 16, 4096, 4096, None) == -1
    assert L.ferret_linear_bf16_noalloc(1, 1, None, 1, 16, 100, 4096, None) == -2
    # M = 100, N = 4096, K = 12288 splits K three ways: 4.9 MB of partials
    assert L.ferret_workspace_bytes(0, 100, 4096, 12288, 0) > 4 << 20
    assert L.ferret_linear_bf16_noalloc(1, 1, None, 1, 100, 4096, 12288, None) == -3


def test_python_ops_refuse_cpu_tensors():
    import torch
    from ferret_amd import ops
    x = torch.zeros((1, 128), dtype=torch.bfloat16)
    w = torch.zeros((16, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.linear_bf16(x, w, out=torch.zeros((1, 16), dtype=torch.bfloat16))


def test_ue8m0_gemm_rejects_before_launch():
    """ferret_fp8_gemm_ue8m0 validates pointers, shapes and its (required)
    workspace on the host and returns before any HIP call (pointers here are
    never dereferenced)."""
    from ferret_amd import lib
    if not os.path.exists(lib.LIB_PATH):
        pytest.skip("libferret_hip.so not built")
    L = lib.load()
    need = L.ferret_workspace_bytes(5, 256, 4096, 7168, 0)
    assert need >= 256 * 56 * 4 + 32 * 56 * 4
    assert L.ferret_fp8_gemm_ue8m0(None, 1, 1, 1, 1, 256, 4096, 7168, 1, need, None) == -1
    assert L.ferret_fp8_gemm_ue8m0(1, 1, 1, 1, 1, 256, 4096, 7100, 1, need, None) == -2
    assert L.ferret_fp8_gemm_ue8m0(1, 1, 1, 1, 1, 256, 4000, 7168, 1, need, None) == -2
    assert L.ferret_fp8_gemm_ue8m0(1, 1, 1, 1, 1, 256, 4096, 7168, None, 0, None) == -3
    assert L.ferret_fp8_gemm_ue8m0(1, 1, 1, 1, 1, 256, 4096, 7168, 1, need - 1, None) == -3
    assert L.ferret_workspace_bytes(5, 256, 4096, 7100, 0) == 0


def test_int4_tiled_entries_reject_before_launch():
    """ferret_int4_tile_weights and ferret_moe_w13_w4a16_tiled check pointers,
    shapes and (tiling) buffer overlap on the host and return before any HIP
    call (the pointers here are never dereferenced)."""
    from ferret_amd import lib
    if not os.path.exists(lib.LIB_PATH):
        pytest.skip("libferret_hip.so not built")
    L = lib.load()
    assert L.ferret_int4_tile_weights(None, 1, 1, 16, 128, None) == -1
    assert L.ferret_int4_tile_weights(1, None, 1, 16, 128, None) == -1
    assert L.ferret_int4_tile_weights(1 << 20, 1 << 24, 1, 24, 128, None) == -2     # N % 16
    assert L.ferret_int4_tile_weights(1 << 20, 1 << 24, 1, 16, 200, None) == -2     # K % 128
    assert L.ferret_int4_tile_weights(1 << 20, 1 << 24, 0, 16, 128, None) == -2     # E
    # [1, 16, 128] is 1 KB: destinations inside it (or covering it) are rejected
    assert L.ferret_int4_tile_weights(1 << 20, (1 << 20) + 16, 1, 16, 128, None) == -2
    assert L.ferret_int4_tile_weights((1 << 20) + 16, 1 << 20, 1, 16, 128, None) == -2
    assert L.ferret_int4_tile_weights(1 << 20, 1 << 20, 1, 16, 128, None) == -2
    assert L.ferret_moe_w13_w4a16_tiled(1, None, 1, 1, 1, 1, 10, 16, 4, 8, 16, 64, 256, 1, None) == -1
    assert L.ferret_moe_w13_w4a16_tiled(1, 1, 1, 1, 1, 1, 10, 128, 4, 8, 16, 64, 256, 1, None) == -2  # tile_m
    assert L.ferret_moe_w13_w4a16_tiled(1, 1, 1, 1, 1, 1, 10, 16, 4, 8, 16, 48, 256, 1, None) == -2   # N % 32
    assert L.ferret_moe_w13_w4a16_tiled(1, 1, 1, 1, 1, 1, 10, 16, 4, 8, 16, 64, 200, 1, None) == -2   # K % 128


def test_int4_tiled_python_wrappers_check_before_launch():
    import torch
    from ferret_amd import ops
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.int4_tile_weights(torch.zeros((2, 32, 32), dtype=torch.int32))
    x = torch.zeros((4, 256), dtype=torch.bfloat16)
    r = ops.Routing(counts=None, offsets=None, sorted_pair=torch.zeros(8, dtype=torch.int32),
                    tiles=torch.zeros((4, 3), dtype=torch.int32), ntiles=torch.zeros(1, dtype=torch.int32),
                    tile_m=16, max_tiles=4, num_experts=2, topk=2, num_tokens=4)
    ws = torch.zeros((2, 64, 8), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="tiled wq"):
        ops.moe_w13_w4a16(x, torch.zeros((2, 4, 2, 16, 8), dtype=torch.int32), ws, r)
    with pytest.raises(ValueError, match="tiled wq"):
        ops.moe_w13_w4a16(x, torch.zeros((2, 4, 3, 16, 16), dtype=torch.int32), ws, r)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.moe_w13_w4a16(x, torch.zeros((2, 4, 2, 16, 16), dtype=torch.int32), ws, r)


def test_integration_stubs_match_the_library_signatures():
    """The ctypes stubs the integration guide at the repository root shows a
    maintainer agree with lib.SIGNATURES."""
    import ctypes
    import re
    from ferret_amd import lib
    text = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "INTEGRATION.md")).read()
    env = {"vp": ctypes.c_void_p, "i32": ctypes.c_int, "sz": ctypes.c_size_t}
    found = {}
    for name, expr in re.findall(r"L\.(ferret_\w+)\.argtypes(?:, L\.\w+\.restype)? = (\[[^\n`]*?\](?: \* \d+)?"
                                 r"(?: \+ \[[^\n`]*?\](?: \* \d+)?)*)", text):
        found[name] = eval(expr, {}, env)  # noqa: S307 -- the doc's own list expressions
    assert len(found) == 19  # 15 entry points, 3 sizing helpers, the allocation-free linear
    for name, argtypes in found.items():
        assert name in lib.SIGNATURES, name
        assert argtypes == list(lib.SIGNATURES[name][1]), name
