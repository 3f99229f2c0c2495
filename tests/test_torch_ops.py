"""The torch.library layer (ferret_amd.torch_ops) without a GPU: every op is
registered under torch.ops.ferret, its fake implementation gives the output
shapes and dtypes the kernels write (meta tensors), and a CPU tensor is refused
(no CPU path)."""
import os

import pytest
import torch

from ferret_amd import lib


def _ops():
    if not os.path.exists(lib.LIB_PATH):
        pytest.skip("libferret_hip.so not built")
    import ferret_amd.torch_ops as T
    return T


def test_every_op_is_registered():
    T = _ops()
    for name in T.OPS:
        assert hasattr(torch.ops.ferret, name), name


def m(*shape, dtype=torch.float32):
    return torch.empty(shape, dtype=dtype, device="meta")


def test_fake_shapes_dense():
    _ops()
    F = torch.ops.ferret
    bf, f8, i32 = torch.bfloat16, torch.float8_e4m3fn, torch.int32
    y = F.linear_bf16(m(16, 4096, dtype=bf), m(6144, 4096, dtype=bf), None)
    assert y.shape == (16, 6144) and y.dtype == bf
    c = F.fp8_gemm_blockscale(m(300, 7168, dtype=f8), m(300, 56), m(4096, 7168, dtype=f8), m(32, 56))
    assert c.shape == (300, 4096) and c.dtype == bf
    c = F.fp8_gemm_ue8m0(m(64, 2048, dtype=f8), m(4, 64, dtype=i32), m(7168, 2048, dtype=f8), m(4, 7168, dtype=i32))
    assert c.shape == (64, 7168)
    q, s = F.quant_act_e4m3(m(32768, 2048, dtype=bf))
    assert q.shape == (32768, 2048) and q.dtype == f8 and s.shape == (32768, 16) and s.dtype == torch.float32


def test_fake_shapes_moe():
    _ops()
    F = torch.ops.ferret
    bf, f8, i32 = torch.bfloat16, torch.float8_e4m3fn, torch.int32
    ids, w = F.moe_route_topk(m(4096, 256), 8)
    assert ids.shape == (4096, 8) and ids.dtype == i32 and w.shape == (4096, 8)
    counts, offsets, sp, tiles, nt = F.moe_permute(m(4096, 8, dtype=i32), 256, 0)
    assert counts.shape == (256,) and offsets.shape == (257,) and sp.shape == (32768,)
    assert tiles.shape == (lib.load().ferret_moe_max_tiles(32768, 256, 128), 3) and nt.shape == (1,)
    o = F.moe_w13_fp8(m(4096, 7168, dtype=f8), m(4096, 56), m(256, 4096, 7168, dtype=f8), m(256, 32, 56),
                      sp, tiles, nt, 128, 8)
    assert o.shape == (32768, 2048) and o.dtype == bf
    o = F.moe_w13_w4a16(m(64, 7168, dtype=bf), m(384, 4096, 896, dtype=i32), m(384, 4096, 224, dtype=bf),
                        m(512, dtype=i32), m(896, 3, dtype=i32), m(1, dtype=i32), 16, 8)
    assert o.shape == (512, 2048)
    t4 = F.int4_tile_weights(m(384, 4096, 896, dtype=i32))
    assert t4.shape == (384, 256, 56, 16, 16) and t4.dtype == i32
    o = F.moe_w13_w4a16(m(64, 7168, dtype=bf), t4, m(384, 4096, 224, dtype=bf),
                        m(512, dtype=i32), m(896, 3, dtype=i32), m(1, dtype=i32), 16, 8)
    assert o.shape == (512, 2048)
    o2 = F.moe_w2_fp8(m(32768, 2048, dtype=f8), m(32768, 16), m(256, 7168, 2048, dtype=f8), m(256, 56, 16),
                      sp, tiles, nt, 128, 8)
    assert o2.shape == (32768, 7168)
    y = F.moe_combine(m(32768, 7168, dtype=bf), m(4096, 8))
    assert y.shape == (4096, 7168) and y.dtype == bf


def test_cpu_tensors_are_refused():
    _ops()
    with pytest.raises(ValueError, match="GPU tensor"):
        torch.ops.ferret.linear_bf16(torch.zeros(1, 128, dtype=torch.bfloat16),
                                     torch.zeros(16, 128, dtype=torch.bfloat16), None)


def test_tile_formulas_match_the_library():
    """The fake implementations size moe_permute's outputs with Python copies of
    ferret_moe_tile_m / ferret_moe_max_tiles (no library call, SymInt-safe);
    they must equal the C functions."""
    T = _ops()
    L = lib.load()
    for P in (0, 1, 7, 8, 15, 16, 17, 127, 128, 129, 1000, 1024, 8191, 8192, 32768, 1 << 20):
        for E in (1, 8, 32, 256, 384, 1024):
            tm = T.moe_tile_m(P, E)
            assert tm == L.ferret_moe_tile_m(P, E), (P, E)
            for tile_m in (1, 16, 128, tm):
                assert T.moe_max_tiles(P, E, tile_m) == L.ferret_moe_max_tiles(P, E, tile_m), (P, E, tile_m)


def test_moe_permute_fake_calls_no_library(monkeypatch):
    T = _ops()

    def refuse():
        raise AssertionError("the fake implementation called into libferret_hip.so")
    monkeypatch.setattr(T._lib, "load", refuse)
    counts, offsets, sp, tiles, nt = torch.ops.ferret.moe_permute(m(100, 8, dtype=torch.int32), 32, 0)
    # 800 pairs over 32 experts: 25 rows per expert, 16-row tiles, ceil(800 / 16) + 32 table rows
    assert sp.shape == (800,) and tiles.shape == (82, 3) and counts.shape == (32,)


def test_moe_permute_exports_with_a_dynamic_token_count():
    """torch.export traces moe_permute with the token count symbolic: the table
    size comes out as a symbolic expression, not a specialised constant."""
    _ops()

    class Route(torch.nn.Module):
        def forward(self, ids):
            return torch.ops.ferret.moe_permute(ids, 256, 128)

    ids = torch.zeros((4096, 8), dtype=torch.int32)
    ep = torch.export.export(Route(), (ids,), dynamic_shapes=({0: torch.export.Dim("T", min=2, max=1 << 18)},))
    outs = [n for n in ep.graph.nodes if n.op == "output"][0].args[0]
    shapes = [tuple(o.meta["val"].shape) for o in outs]
    assert shapes[0] == (256,) and shapes[1] == (257,)
    assert not isinstance(shapes[2][0], int) and not isinstance(shapes[3][0], int), shapes
