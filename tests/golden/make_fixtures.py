"""Write the golden fixtures of the quantized-GEMM path: small seeded inputs and
the CPU oracle's outputs, one .npz per function (numpy arrays only, loadable
with allow_pickle=False).

    python tests/golden/make_fixtures.py

The reference stores no golden vectors for this path (its in-binary checks
regenerate inputs from rand() seeds and compare against a host loop), so these
come from the oracle, which its own tests pin against closed forms, special
cases and brute force.  tests/test_golden.py checks that the oracle still
reproduces every fixture (CPU) and that the HIP path matches them (GPU).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import formats as F  # noqa: E402
from oracle import gemm as G  # noqa: E402
from oracle import quant as Q  # noqa: E402
from oracle import routing as R  # noqa: E402


def _bf16_bits(x):
    return F.f32_to_bf16_bits(np.asarray(x, np.float32))


def routing_case():
    rng = np.random.default_rng(11)
    T, E, k = 37, 64, 8
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[0, :] = 0.0                       # all tied: the 8 lowest expert ids
    logits[1, 10:20] = 2.5                   # a 10-way tie at the top
    logits[2, ::3] = -1.0                    # repeated values below the top
    ids, w = R.route_topk(logits, k)
    counts, offsets, sp = R.permute(ids, E)
    return dict(logits=logits, topk=np.int32(k), ids=ids.astype(np.int32), weights=w.astype(np.float32),
                counts=counts.astype(np.int32), offsets=offsets.astype(np.int32), sorted_pair=sp.astype(np.int32),
                tiles16=R.tile_table(counts, offsets, 16).astype(np.int32),
                tiles128=R.tile_table(counts, offsets, 128).astype(np.int32))


def quant_case():
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((6, 384)) * 3.0).astype(np.float32)
    x[0, :128] = 0.0                         # all-zero block: the amax floor
    x[1, 128:256] *= 1e-6                    # tiny block: e4m3 subnormals after scaling
    x[2, 0] = 448.0                          # block max exactly 448: scale 1
    x = F.bf16_round(x)
    q, s = Q.quant_act_1x128(x)
    return dict(x_bits=_bf16_bits(x), q=q, scale=s)


def int4_case():
    rng = np.random.default_rng(13)
    words = rng.integers(-2 ** 31, 2 ** 31, size=(4, 16), dtype=np.int64).astype(np.int32)
    words[0, 0] = np.int32(0x76543210)       # nibbles 0..7 -> -8..-1
    words[0, 1] = np.int32(np.uint32(0xFEDCBA98).view(np.int32))  # nibbles 8..15 -> 0..7
    scales = _bf16_bits(rng.standard_normal((4, 4)) * 0.01)
    return dict(words=words, scale_bits=scales, nibbles=F.int4_unpack(words).astype(np.int8),
                w_bits=_bf16_bits(F.int4_dequant(words, scales)))


def fp8_gemm_case():
    rng = np.random.default_rng(14)
    a, sa = Q.quant_act_1x128(rng.standard_normal((5, 384)).astype(np.float32))
    b, sb = Q.quant_weight_128x128(rng.standard_normal((256, 384)).astype(np.float32))
    return dict(a=a, sa=sa, b=b, sb=sb, c=G.fp8_blockscale_gemm(a, sa, b, sb))


def linear_case():
    rng = np.random.default_rng(15)
    x = _bf16_bits(rng.standard_normal((3, 256)))
    w = _bf16_bits(rng.standard_normal((64, 256)) * 0.05)
    r = _bf16_bits(rng.standard_normal((3, 64)))
    return dict(x_bits=x, w_bits=w, r_bits=r, y=G.linear_bf16(x, w, r))


def moe_fp8_case():
    rng = np.random.default_rng(16)
    T, E, k, N, K = 6, 4, 2, 256, 256
    x, sx = Q.quant_act_1x128(rng.standard_normal((T, K)).astype(np.float32))
    w = np.empty((E, N, K), np.uint8)
    sw = np.empty((E, N // 128, K // 128), np.float32)
    for e in range(E):
        w[e], sw[e] = Q.quant_weight_128x128(rng.standard_normal((N, K)).astype(np.float32))
    ids, _ = R.route_topk(rng.standard_normal((T, E)).astype(np.float32), k)
    w13 = G.moe_w13_fp8(x, sx, w, sw, ids)
    # the down projection of the same routing: h [T*k, 128] -> [T*k, 256]
    h, sh = Q.quant_act_1x128(rng.standard_normal((T * k, 128)).astype(np.float32))
    w2 = np.empty((E, 256, 128), np.uint8)
    sw2 = np.empty((E, 2, 1), np.float32)
    for e in range(E):
        w2[e], sw2[e] = Q.quant_weight_128x128(rng.standard_normal((256, 128)).astype(np.float32))
    o = G.moe_w2_fp8(h, sh, w2, sw2, ids)
    wts = rng.random((T, k)).astype(np.float32)
    o_bits = _bf16_bits(o)
    return dict(x=x, sx=sx, w=w, sw=sw, ids=ids.astype(np.int32), w13=w13, h=h, sh=sh, w2=w2, sw2=sw2, w2_out=o,
                o_bits=o_bits, combine_w=wts, combine=G.moe_combine(o_bits, wts))


def w4a16_case():
    rng = np.random.default_rng(17)
    T, E, k, N, K = 5, 3, 2, 64, 256
    x = _bf16_bits(rng.standard_normal((T, K)))
    wq = rng.integers(-2 ** 31, 2 ** 31, size=(E, N, K // 8), dtype=np.int64).astype(np.int32)
    ws = _bf16_bits(rng.standard_normal((E, N, K // 32)) * 0.01)
    ids, _ = R.route_topk(rng.standard_normal((T, E)).astype(np.float32), k)
    return dict(x_bits=x, wq=wq, ws_bits=ws, ids=ids.astype(np.int32), out=G.moe_w13_w4a16(x, wq, ws, ids))


CASES = {"routing": routing_case, "quant_act": quant_case, "int4": int4_case, "fp8_gemm": fp8_gemm_case,
         "linear_bf16": linear_case, "moe_fp8": moe_fp8_case, "moe_w4a16": w4a16_case}


def main():
    for name, fn in CASES.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
