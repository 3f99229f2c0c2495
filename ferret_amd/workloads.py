"""The benchmark configurations of the quantized-GEMM path and their seeded inputs.

The four math cases at their DeepSeek-V3 / Qwen3-8B / Kimi-K2 shapes (the
Qwen3-8B decode projections at M = 1 and 16, the DeepSeek-V3 TP8 attention
projections from M = 1 to 8192), plus the rest of the FP8 MoE layer: the w2
down projection (K = 2048 -> N = 7168, tasks/fp8-group-gemm-dsv3-decode.yaml:11-13),
the 1x128 activation quantizer in front of it and the top-k combine after it.
Inputs are generated with torch on any device from per-tensor seeds;
the quantizer below is the library's absmax/448 rule (1x128 activation blocks,
128x128 weight blocks, fp32 scales), the same rule DeepGEMM's
per_token_cast_to_fp8 / per_block_cast_to_fp8 implement at the reference's call
sites (baselines/fp8-gemm/baseline_prefill.py:41-42,
baselines/fp8-group-gemm/baseline_dsv3_decode.py:45-53).

Algorithmic bytes count every operand byte once and every output byte once;
for the MoE workloads only the experts that received at least one pair count.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

FP8 = torch.float8_e4m3fn


@dataclass(frozen=True)
class Workload:
    key: str
    kind: str            # "linear_bf16" | "fp8_gemm" | "fp8_gemm_ue8m0" | "moe_fp8" | "moe_w4a16" | "moe_fp8_w2"
                         # | "quant_act" | "moe_combine"
    M: int = 0           # dense tokens
    N: int = 0           # output rows (per expert: gate + up)
    K: int = 0
    T: int = 0           # MoE tokens
    E: int = 0
    topk: int = 0
    routing: str = ""    # "softmax" (N(0,1) logits) | "zipf" | "uniform" (T/E rows per expert)
    zipf_s: float = 0.0
    bound: str = "hbm"   # roofline that limits it on MI355X
    residual: bool = False  # linear_bf16: y = x.W^T + residual
    description: str = ""
    seeds: dict = field(default_factory=dict)


WORKLOADS: dict[str, Workload] = {w.key: w for w in [
    Workload("qwen3_gateup_M16", "linear_bf16", M=16, N=24576, K=4096,
             description="Qwen3-8B decode GateUp: X bf16 [16,4096], W bf16 [24576,4096]",
             seeds={"x": 1, "w": 2}),
    *[Workload(f"qwen3_{name.lower()}_M{m}", "linear_bf16", M=m, N=n, K=k, residual=res,
               description=f"Qwen3-8B decode {name}: X bf16 [{m},{k}], W bf16 [{n},{k}]"
                           + (" + residual" if res else ""),
               seeds={"x": 1, "w": 20 + i, "r": 40 + i})
      # tasks/qwen3-8b-decode-linear-bs16-b200.yaml:72-95 (M = 16) and
      # tasks/qwen3-8b-decode-linear-b200.yaml:53-76 (M = 1)
      for m in (16, 1)
      for i, (name, n, k, res) in enumerate([("QKV", 6144, 4096, False), ("O", 4096, 4096, True),
                                             ("GateUp", 24576, 4096, False), ("Down", 4096, 12288, True),
                                             ("LMHead", 153600, 4096, False)])
      if not (m == 16 and name == "GateUp")],
    Workload("dsv3_fp8_M16", "fp8_gemm", M=16, N=4096, K=7168,
             description="DeepSeek-V3 dense FP8 GEMM M=16", seeds={"a": 3, "b": 4}),
    Workload("dsv3_fp8_M128", "fp8_gemm", M=128, N=4096, K=7168,
             description="DeepSeek-V3 dense FP8 GEMM M=128", seeds={"a": 3, "b": 4}),
    Workload("dsv3_fp8_M4096", "fp8_gemm", M=4096, N=4096, K=7168, bound="mfma",
             description="DeepSeek-V3 dense FP8 GEMM M=4096", seeds={"a": 3, "b": 4}),
    # UE8M0 block-scale mode on the reference's block-scale configs
    # (examples/fp8-gemm/v009_large_m_block_scale_mma_080.cu:526-532): random
    # e4m3 codes and scales drawn as 0.5 + (rand() % 100) / 200 (:549-552),
    # rounded to powers of two and packed the reference's way.
    *[Workload(f"dsv3_{proj}_M{m}_ue8m0", "fp8_gemm_ue8m0", M=m, N=n, K=k, bound="mfma",
               description=f"DeepSeek-V3 {proj} FP8 GEMM with UE8M0 block scales: A e4m3 [{m},{k}], B e4m3 [{n},{k}]",
               seeds={"a": 50 + i, "b": 54 + i})
      for i, (proj, m, k, n) in enumerate([("o_proj", 2048, 2048, 7168), ("q_b_proj", 8192, 1536, 3072),
                                           ("kv_b_proj", 8192, 512, 4096), ("o_proj", 4096, 2048, 7168),
                                           ("o_proj", 8192, 2048, 7168)])],
    # DeepSeek-V3 attention projections at TP = 8 (per-rank shapes): decode and
    # a 512-token chunk (tasks/fp8-gemm-dense-tp8.yaml:36-74) and prefill with
    # M up to the 8K kv_len of kv_b_proj (tasks/fp8-gemm-prefill-tp8.yaml:44-117).
    *[Workload(f"dsv3_{proj}_M{m}", "fp8_gemm", M=m, N=n, K=k, bound="mfma" if m >= 512 else "hbm",
               description=f"DeepSeek-V3 TP8 {proj} FP8 GEMM: A e4m3 [{m},{k}], B e4m3 [{n},{k}]",
               seeds={"a": 30 + i, "b": 34 + i})
      for m in (1, 16, 512, 1024, 2048, 4096, 8192)
      for i, (proj, k, n) in enumerate([("q_b_proj", 1536, 3072), ("kv_b_proj", 512, 4096),
                                        ("o_proj", 2048, 7168)])],
    # The reference's own per-rank MoE tasks (EP 8: 32 local experts, uniform
    # segments of M rows per expert, its m_indices = arange(M_total) // M
    # stand-in): tasks/fp8-group-gemm-dsv3-decode.yaml:31-86 and
    # tasks/fp8-group-gemm-dsv3-prefill.yaml:40-95.
    *[Workload(f"dsv3_ep8_{proj}_M{m}", kind, N=n, K=k, T=32 * m, E=32, topk=1, routing="uniform",
               bound="mfma" if m >= 64 else "hbm",
               description=f"DSv3 FP8 grouped GEMM, EP8 rank: 32 experts x {m} rows, {proj} K={k} -> N={n}",
               seeds={"logits": 0, "x": 60 + i, "w": 700 + 100 * i})
      for m in (1, 4, 8, 16, 64, 128, 256, 512)
      for i, (proj, kind, k, n) in enumerate([("gate_up", "moe_fp8", 7168, 4096),
                                             ("down", "moe_fp8_w2", 2048, 7168)])],
    # tasks/kimi-moe-w13-int4-grouped-gemm.yaml:35-40 (TP 8 rank: N_r = 2 I_r = 512); the reference
    # measures T = 1 and T = 8 (correctness/kimi-moe-w13-precision-fix.md:13-14)
    Workload("kimi_w4a16_w13_T8_tp8", "moe_w4a16", N=512, K=7168, T=8, E=384, topk=8, routing="softmax",
             description="Kimi-K2 INT4 W4A16 MoE w13, TP8 rank: 8 tokens, top-8 of 384, N_r=512",
             seeds={"logits": 18, "x": 19, "w": 900}),
    Workload("kimi_w4a16_w13_T1_tp8", "moe_w4a16", N=512, K=7168, T=1, E=384, topk=8, routing="softmax",
             description="Kimi-K2 INT4 W4A16 MoE w13, TP8 rank: 1 token, top-8 of 384, N_r=512",
             seeds={"logits": 16, "x": 17, "w": 901}),
    Workload("dsv3_moe_w13_decode", "moe_fp8", N=4096, K=7168, T=128, E=256, topk=8, routing="softmax",
             description="DSv3 FP8 MoE w13 decode: 128 tokens, top-8 of 256", seeds={"logits": 5, "x": 6, "w": 100}),
    Workload("kimi_w4a16_w13_decode", "moe_w4a16", N=4096, K=7168, T=64, E=384, topk=8, routing="softmax",
             description="Kimi-K2 INT4 W4A16 MoE w13 decode: 64 tokens, top-8 of 384",
             seeds={"logits": 7, "x": 8, "w": 200}),
    Workload("dsv3_moe_w13_prefill", "moe_fp8", N=4096, K=7168, T=4096, E=256, topk=8, routing="zipf",
             zipf_s=1.1, bound="mfma", description="DSv3 FP8 MoE w13 prefill: 4096 tokens, Zipf(1.1) top-8 of 256",
             seeds={"logits": 9, "x": 10, "w": 100}),
    Workload("dsv3_moe_w2_decode", "moe_fp8_w2", N=7168, K=2048, T=128, E=256, topk=8, routing="softmax",
             description="DSv3 FP8 MoE w2 (down) decode: 1024 routed rows [P,2048] -> [P,7168], 256 experts",
             seeds={"logits": 5, "x": 13, "w": 400}),
    Workload("dsv3_moe_w2_prefill", "moe_fp8_w2", N=7168, K=2048, T=4096, E=256, topk=8, routing="zipf",
             zipf_s=1.1, bound="mfma", description="DSv3 FP8 MoE w2 (down) prefill: 32768 routed rows, Zipf(1.1)",
             seeds={"logits": 9, "x": 14, "w": 400}),
    Workload("moe_quant_act_prefill", "quant_act", M=32768, K=2048,
             description="1x128 e4m3 quantization of the w2 input at prefill: bf16 [32768,2048]",
             seeds={"x": 15}),
    Workload("moe_combine_prefill", "moe_combine", N=7168, T=4096, topk=8,
             description="top-8 weighted combine at prefill: bf16 [32768,7168] -> [4096,7168]",
             seeds={"x": 16, "logits": 17}),
]}


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def randn(shape, seed: int, device, std: float = 1.0) -> torch.Tensor:
    x = torch.randn(shape, generator=_gen(seed, device), device=device, dtype=torch.float32)
    return x * std if std != 1.0 else x


def quant_act_1x128(x: torch.Tensor):
    """x fp32 [M, K] -> (e4m3 [M, K], fp32 scales [M, K/128])."""
    M, K = x.shape
    xv = x.view(M, K // 128, 128)
    amax = xv.abs().amax(dim=2).clamp_min(1e-4)
    q = (xv * (448.0 / amax).unsqueeze(2)).to(FP8).view(M, K)
    return q, amax / 448.0


def quant_weight_128x128(w: torch.Tensor):
    """w fp32 [N, K] -> (e4m3 [N, K], fp32 scales [N/128, K/128])."""
    N, K = w.shape
    wv = w.view(N // 128, 128, K // 128, 128)
    amax = wv.abs().amax(dim=(1, 3)).clamp_min(1e-4)
    q = (wv * (448.0 / amax)[:, None, :, None]).to(FP8).view(N, K)
    return q, amax / 448.0


def zipf_logits(T: int, E: int, s: float, seed: int, device) -> torch.Tensor:
    """Gumbel-top-k logits for Zipf(s) expert popularity: -s*ln(rank) + Gumbel noise.

    Top-k of these logits samples k distinct experts without replacement with
    probability proportional to rank^-s (rank = expert id + 1).
    """
    u = torch.rand((T, E), generator=_gen(seed, device), device=device, dtype=torch.float32)
    u = u.clamp(1e-12, 1.0 - 1e-7)
    gumbel = -torch.log(-torch.log(u))
    rank = torch.arange(1, E + 1, device=device, dtype=torch.float32)
    return gumbel - s * torch.log(rank)[None, :]


def make_inputs(w: Workload, device="cuda", experts: list[int] | None = None) -> dict:
    """Generate the workload's inputs on `device`.

    For MoE workloads `experts` limits which expert weights are generated (the
    others stay zero-filled); None generates all of them.
    """
    s = w.seeds
    if w.kind == "quant_act":
        return {"x": randn((w.M, w.K), s["x"], device).to(torch.bfloat16)}
    if w.kind == "moe_combine":
        o = randn((w.T * w.topk, w.N), s["x"], device).to(torch.bfloat16)
        wts = torch.softmax(randn((w.T, w.topk), s["logits"], device), dim=1)
        return {"o": o, "w": wts}
    if w.kind == "linear_bf16":
        x = randn((w.M, w.K), s["x"], device).to(torch.bfloat16)
        wt = randn((w.N, w.K), s["w"], device, std=0.02).to(torch.bfloat16)
        if w.residual:
            return {"x": x, "w": wt, "r": randn((w.M, w.N), s["r"], device).to(torch.bfloat16)}
        return {"x": x, "w": wt}
    if w.kind == "fp8_gemm":
        a, sa = quant_act_1x128(randn((w.M, w.K), s["a"], device))
        b, sb = quant_weight_128x128(randn((w.N, w.K), s["b"], device))
        return {"a": a, "sa": sa, "b": b, "sb": sb}
    if w.kind == "fp8_gemm_ue8m0":
        from . import ops
        nk, nbk = w.K // 128, (w.N + 127) // 128

        def codes(shape, seed):
            c = torch.randint(0, 254, shape, generator=_gen(seed, device), device=device, dtype=torch.int32)
            return torch.where(c >= 0x7F, c + 1, c).to(torch.uint8).view(FP8)   # no NaN codes

        def scales(shape, seed):
            r = torch.randint(0, 100, shape, generator=_gen(seed, device), device=device, dtype=torch.int32)
            return 0.5 + r.to(torch.float32) / 200.0
        sa, sb = scales((w.M, nk), s["a"] + 1000), scales((nbk, nk), s["b"] + 1000)
        sfa = ops.pack_ue8m0(ops.ue8m0_from_float(sa))
        sfb = ops.pack_ue8m0(ops.ue8m0_from_float(ops.expand_block_scales(sb, w.N)))
        return {"a": codes((w.M, w.K), s["a"]), "b": codes((w.N, w.K), s["b"]), "sfa": sfa, "sfb": sfb,
                "sa": sa, "sb": sb}
    if w.routing == "zipf":
        logits = zipf_logits(w.T, w.E, w.zipf_s, s["logits"], device)
    elif w.routing == "uniform":
        # top-1 of a one-hot row: token t goes to expert t // (T / E)
        logits = torch.zeros((w.T, w.E), dtype=torch.float32, device=device)
        logits[torch.arange(w.T, device=device), torch.arange(w.T, device=device) // (w.T // w.E)] = 1.0
    else:
        logits = randn((w.T, w.E), s["logits"], device)
    ex = range(w.E) if experts is None else experts
    if w.kind == "moe_fp8":
        x, sx = quant_act_1x128(randn((w.T, w.K), s["x"], device))
        wq = torch.zeros((w.E, w.N, w.K), dtype=FP8, device=device)
        sw = torch.ones((w.E, w.N // 128, w.K // 128), dtype=torch.float32, device=device)
        for e in ex:
            wq[e], sw[e] = quant_weight_128x128(randn((w.N, w.K), s["w"] + e, device))
        return {"logits": logits, "x": x, "sx": sx, "w": wq, "sw": sw}
    if w.kind == "moe_fp8_w2":
        h, sh = quant_act_1x128(randn((w.T * w.topk, w.K), s["x"], device))
        wq = torch.zeros((w.E, w.N, w.K), dtype=FP8, device=device)
        sw = torch.ones((w.E, w.N // 128, w.K // 128), dtype=torch.float32, device=device)
        for e in ex:
            wq[e], sw[e] = quant_weight_128x128(randn((w.N, w.K), s["w"] + e, device))
        return {"logits": logits, "h": h, "sh": sh, "w": wq, "sw": sw}
    if w.kind == "moe_w4a16":
        x = randn((w.T, w.K), s["x"], device).to(torch.bfloat16)
        wq = torch.zeros((w.E, w.N, w.K // 8), dtype=torch.int32, device=device)
        ws = torch.zeros((w.E, w.N, w.K // 32), dtype=torch.bfloat16, device=device)
        for e in ex:
            g = _gen(s["w"] + e, device)
            wq[e] = torch.randint(-2 ** 31, 2 ** 31, (w.N, w.K // 8), generator=g, device=device, dtype=torch.int32)
            ws[e] = (torch.randn((w.N, w.K // 32), generator=g, device=device) * 0.01).to(torch.bfloat16)
        return {"logits": logits, "x": x, "w": wq, "ws": ws}
    raise ValueError(w.kind)


def experts_hit(ids: torch.Tensor, E: int) -> int:
    return int(torch.unique(ids[(ids >= 0) & (ids < E)]).numel())


def algorithmic_bytes(w: Workload, n_experts_hit: int = 0) -> int:
    """Every operand byte read once + every output byte written once."""
    if w.kind == "linear_bf16":
        return 2 * (w.N * w.K + w.M * w.K + w.M * w.N * (2 if w.residual else 1))
    if w.kind == "fp8_gemm":
        return (w.M * w.K + w.M * (w.K // 128) * 4 + w.N * w.K + ((w.N + 127) // 128) * (w.K // 128) * 4
                + w.M * w.N * 2)
    if w.kind == "fp8_gemm_ue8m0":   # packed scale words: 4 bytes per 4 K-blocks, per token / weight row
        nsk = (w.K // 128 + 3) // 4
        return w.M * w.K + w.N * w.K + (w.M + w.N) * nsk * 4 + w.M * w.N * 2
    P = w.T * w.topk
    if w.kind == "moe_fp8":
        per_e = w.N * w.K + (w.N // 128) * (w.K // 128) * 4
        return (n_experts_hit * per_e + w.T * w.K + w.T * (w.K // 128) * 4 + P * (w.N // 2) * 2
                + P * 4 * 2)  # + the pair index read twice (gather and scatter)
    if w.kind == "moe_w4a16":
        per_e = w.N * w.K // 2 + w.N * (w.K // 32) * 2
        return n_experts_hit * per_e + w.T * w.K * 2 + P * (w.N // 2) * 2 + P * 4 * 2
    if w.kind == "moe_fp8_w2":
        per_e = w.N * w.K + (w.N // 128) * (w.K // 128) * 4
        return n_experts_hit * per_e + P * w.K + P * (w.K // 128) * 4 + P * w.N * 2 + P * 4 * 2
    if w.kind == "quant_act":
        return w.M * w.K * 2 + w.M * w.K + w.M * (w.K // 128) * 4
    if w.kind == "moe_combine":
        return P * w.N * 2 + P * 4 + w.T * w.N * 2
    raise ValueError(w.kind)


def flops(w: Workload) -> int:
    if w.kind in ("linear_bf16", "fp8_gemm", "fp8_gemm_ue8m0"):
        return 2 * w.M * w.N * w.K
    if w.kind == "quant_act":
        return 2 * w.M * w.K               # one scale multiply + one |x| max per element
    if w.kind == "moe_combine":
        return 2 * w.T * w.topk * w.N
    return 2 * w.T * w.topk * w.N * w.K
