"""GPU checks of the torch.library layer (torch.ops.ferret.*): opcheck of the
schemas and fake implementations against the real kernels, a whole MoE layer
traced by torch.compile (fullgraph) equal to eager, and the same layer captured
in a HIP graph, replayed several times with eager work in between, every replay
equal to the eager result."""
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def T(hip):
    import ferret_amd.torch_ops as _T
    return _T


def _fp8_inputs(M, N, K, seed):
    from ferret_amd import workloads as W
    a, sa = W.quant_act_1x128(W.randn((M, K), seed, "cuda"))
    b, sb = W.quant_weight_128x128(W.randn((N, K), seed + 1, "cuda"))
    return a, sa, b, sb


def test_opcheck_dense(T):
    _say("opcheck dense ops")
    F = torch.ops.ferret
    x = torch.randn(16, 1024, device="cuda").to(torch.bfloat16)
    w = (0.02 * torch.randn(512, 1024, device="cuda")).to(torch.bfloat16)
    torch.library.opcheck(F.linear_bf16.default, (x, w, None))
    # e4m3 operands as uint8 views (the ops take both): opcheck's schema check
    # compares inputs with arithmetic torch does not implement for float8
    a, sa, b, sb = _fp8_inputs(200, 512, 1024, 3)
    torch.library.opcheck(F.fp8_gemm_blockscale.default, (a.view(torch.uint8), sa, b.view(torch.uint8), sb))
    torch.library.opcheck(F.quant_act_e4m3.default, (torch.randn(64, 512, device="cuda").to(torch.bfloat16),),
                          test_utils=("test_autograd_registration", "test_faketensor", "test_aot_dispatch_dynamic"))
    o = torch.randn(32 * 4, 256, device="cuda").to(torch.bfloat16)
    torch.library.opcheck(F.moe_combine.default, (o, torch.rand(32, 4, device="cuda")))


def test_opcheck_routing(T):
    _say("opcheck routing ops")
    F = torch.ops.ferret
    logits = torch.randn(64, 32, device="cuda")
    torch.library.opcheck(F.moe_route_topk.default, (logits, 4))
    ids, _ = F.moe_route_topk(logits, 4)
    torch.library.opcheck(F.moe_permute.default, (ids, 32, 16))


def test_opcheck_int4(T):
    """int4_tile_weights and moe_w13_w4a16 on both weight layouts: schemas and
    fake shapes against the kernels; the two layouts give the same bits."""
    _say("opcheck int4 ops")
    F = torch.ops.ferret
    g = torch.Generator(device="cuda").manual_seed(31)
    Tn, E, N, K, topk = 8, 6, 128, 1024, 2
    x = torch.randn((Tn, K), generator=g, device="cuda").to(torch.bfloat16)
    wq = torch.randint(-2 ** 31, 2 ** 31, (E, N, K // 8), generator=g, device="cuda", dtype=torch.int32)
    ws = (torch.randn((E, N, K // 32), generator=g, device="cuda") * 0.01).to(torch.bfloat16)
    ids, _ = F.moe_route_topk(torch.randn((Tn, E), generator=g, device="cuda"), topk)
    counts, offsets, sp, tiles, nt = F.moe_permute(ids, E, 16)
    torch.library.opcheck(F.int4_tile_weights.default, (wq,))
    wt = F.int4_tile_weights(wq)
    for w in (wq, wt):
        torch.library.opcheck(F.moe_w13_w4a16.default, (x, w, ws, sp, tiles, nt, 16, topk))
    a = F.moe_w13_w4a16(x, wq, ws, sp, tiles, nt, 16, topk)
    b = F.moe_w13_w4a16(x, wt, ws, sp, tiles, nt, 16, topk)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def _moe_inputs(Tn=48, E=8, N=512, K=1024, topk=2, seed=7):
    from ferret_amd import workloads as W
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    logits = torch.randn((Tn, E), generator=g, device="cuda")
    x, sx = W.quant_act_1x128(torch.randn((Tn, K), generator=g, device="cuda"))
    w13 = torch.empty((E, N, K), dtype=torch.float8_e4m3fn, device="cuda")
    s13 = torch.empty((E, N // 128, K // 128), device="cuda")
    w2 = torch.empty((E, K, N // 2), dtype=torch.float8_e4m3fn, device="cuda")
    s2 = torch.empty((E, K // 128, N // 2 // 128), device="cuda")
    for e in range(E):
        w13[e], s13[e] = W.quant_weight_128x128(torch.randn((N, K), generator=g, device="cuda"))
        w2[e], s2[e] = W.quant_weight_128x128(torch.randn((K, N // 2), generator=g, device="cuda"))
    return logits, x, sx, w13, s13, w2, s2, topk, E


def _moe_layer(logits, x, sx, w13, s13, w2, s2, topk: int, E: int):
    F = torch.ops.ferret
    ids, wts = F.moe_route_topk(logits, topk)
    counts, offsets, sp, tiles, nt = F.moe_permute(ids, E, 16)
    h = F.moe_w13_fp8(x, sx, w13, s13, sp, tiles, nt, 16, topk)
    hq, hs = F.quant_act_e4m3(h)
    o = F.moe_w2_fp8(hq, hs, w2, s2, sp, tiles, nt, 16, topk)
    return F.moe_combine(o, wts)


def test_compile_fullgraph_matches_eager(T):
    _say("torch.compile fullgraph MoE layer")
    args = _moe_inputs()
    ref = _moe_layer(*args)
    compiled = torch.compile(_moe_layer, fullgraph=True, backend="aot_eager")
    got = compiled(*args)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_hip_graph_replays_match_eager(T):
    _say("HIP graph capture of the MoE layer")
    args = _moe_inputs(seed=11)
    ref = _moe_layer(*args).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):                 # warm the caching allocator outside the capture
        _moe_layer(*args)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = _moe_layer(*args)
    for i in range(4):
        noise = torch.randn(1024, 1024, device="cuda") @ torch.randn(1024, 1024, device="cuda")  # eager work
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        del noise
