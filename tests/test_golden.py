"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_fixtures.py).

CPU: the oracle still reproduces every fixture: integer, code and index arrays
bit for bit, floating-point outputs to 1e-6 relative (numpy's BLAS may order
the sums differently on another machine), plus the INT4 known answers.
GPU: the HIP path run on the fixture inputs matches the stored outputs:
routing, permutation, tile tables and the quantizer bit for bit, the GEMMs
within the 1e-2 error gate.
"""
import importlib.util
import os

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _maker():
    spec = importlib.util.spec_from_file_location("make_fixtures", os.path.join(HERE, "make_fixtures.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _load(name):
    with np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


CASES = ["routing", "quant_act", "int4", "fp8_gemm", "linear_bf16", "moe_fp8", "moe_w4a16"]


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_fixture(name):
    fresh = _maker().CASES[name]()
    stored = _load(name)
    assert set(fresh) == set(stored)
    for k, v in stored.items():
        got = np.asarray(fresh[k])
        assert got.shape == v.shape and got.dtype == v.dtype, (name, k)
        if np.issubdtype(v.dtype, np.floating):
            assert np.allclose(got, v, rtol=1e-6, atol=1e-6 * float(np.abs(v).max(initial=0.0))), (name, k)
        else:
            assert np.array_equal(got, v), (name, k)


def test_int4_fixture_known_answers():
    z = _load("int4")
    assert z["nibbles"][0, 0:8].tolist() == [-8, -7, -6, -5, -4, -3, -2, -1]      # 0x76543210
    assert z["nibbles"][0, 8:16].tolist() == [0, 1, 2, 3, 4, 5, 6, 7]            # 0xFEDCBA98


# ---------------------------------------------------------------------- GPU

@pytest.fixture(scope="module")
def ops():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from ferret_amd import ops as O
    return O


def _dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.view(dtype) if dtype is not None else t


@pytest.mark.gpu
def test_gpu_routing_and_permutation_match_fixture(ops):
    print("[case] golden routing", flush=True)
    z = _load("routing")
    E = z["logits"].shape[1]
    ids, w = ops.moe_route_topk(_dev(z["logits"]), int(z["topk"]))
    assert np.array_equal(ids.cpu().numpy(), z["ids"])
    assert np.allclose(w.cpu().numpy(), z["weights"], rtol=1e-5, atol=1e-7)
    for tm, key in ((16, "tiles16"), (128, "tiles128")):
        rt = ops.moe_permute(ids, E, tm)
        assert np.array_equal(rt.counts.cpu().numpy(), z["counts"])
        assert np.array_equal(rt.offsets.cpu().numpy(), z["offsets"])
        assert np.array_equal(rt.sorted_pair.cpu().numpy(), z["sorted_pair"])
        assert np.array_equal(rt.tiles.cpu().numpy()[: int(rt.ntiles.item())], z[key])


@pytest.mark.gpu
def test_gpu_quantizer_matches_fixture(ops):
    import torch
    print("[case] golden quant_act", flush=True)
    z = _load("quant_act")
    q, s = ops.quant_act_e4m3(_dev(z["x_bits"].view(np.int16), torch.bfloat16))
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), z["q"])
    assert np.array_equal(s.cpu().numpy().view(np.uint32), z["scale"].view(np.uint32))


@pytest.mark.gpu
def test_gpu_gemms_match_fixtures(ops):
    import torch
    from tests.gpu_helpers import assert_gemm_close, bf16_out
    print("[case] golden dense GEMMs", flush=True)
    fp8 = torch.float8_e4m3fn
    z = _load("fp8_gemm")
    c = ops.fp8_gemm_blockscale(_dev(z["a"], fp8), _dev(z["sa"]), _dev(z["b"], fp8), _dev(z["sb"]))
    assert_gemm_close(bf16_out(c), z["c"], "golden fp8_gemm")
    z = _load("linear_bf16")
    bf = lambda a: _dev(a.view(np.int16), torch.bfloat16)  # noqa: E731
    y = ops.linear_bf16(bf(z["x_bits"]), bf(z["w_bits"]), bf(z["r_bits"]))
    assert_gemm_close(bf16_out(y), z["y"], "golden linear_bf16")


@pytest.mark.gpu
@pytest.mark.parametrize("tile_m", [16, 128])
def test_gpu_moe_fp8_layer_matches_fixture(ops, tile_m):
    import torch
    from tests.gpu_helpers import assert_gemm_close, bf16_out
    print(f"[case] golden moe fp8 tile_m={tile_m}", flush=True)
    fp8 = torch.float8_e4m3fn
    z = _load("moe_fp8")
    E = z["w"].shape[0]
    rt = ops.moe_permute(_dev(z["ids"]), E, tile_m)
    out = ops.moe_w13_fp8(_dev(z["x"], fp8), _dev(z["sx"]), _dev(z["w"], fp8), _dev(z["sw"]), rt)
    assert_gemm_close(bf16_out(out), z["w13"], "golden moe_w13_fp8")
    o = ops.moe_w2_fp8(_dev(z["h"], fp8), _dev(z["sh"]), _dev(z["w2"], fp8), _dev(z["sw2"]), rt)
    assert_gemm_close(bf16_out(o), z["w2_out"], "golden moe_w2_fp8")
    y = ops.moe_combine(_dev(z["o_bits"].view(np.int16), torch.bfloat16), _dev(z["combine_w"]))
    assert np.allclose(bf16_out(y), z["combine"], rtol=2.0 ** -8, atol=1e-6)


@pytest.mark.gpu
def test_gpu_w4a16_matches_fixture(ops):
    import torch
    from tests.gpu_helpers import assert_gemm_close, bf16_out
    print("[case] golden moe w4a16", flush=True)
    z = _load("moe_w4a16")
    E = z["wq"].shape[0]
    rt = ops.moe_permute(_dev(z["ids"]), E, 16)
    out = ops.moe_w13_w4a16(_dev(z["x_bits"].view(np.int16), torch.bfloat16), _dev(z["wq"]),
                            _dev(z["ws_bits"].view(np.int16), torch.bfloat16), rt)
    assert_gemm_close(bf16_out(out), z["out"], "golden moe_w13_w4a16")
