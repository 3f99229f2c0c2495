#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-GEMM path.

Default mode prints ONE JSON line for the driver:

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload KEY]

A step is one pass of the hot path over one batch of synthetic input that is
already resident in HBM: the GEMM launch for the dense workloads; route +
permute + grouped GEMM (w13 or w2) for the MoE workloads; one quantizer or
combine launch for those two workloads.  Weights of the dense workloads are
rotated over enough copies (>= 512 MB) that no step finds its operands in the
256 MB MALL.  `roofline` is measured live with HIP events on the launch stream
around the dominant kernel (a pair around each launch and, for the single-launch
workloads, also one pair around a burst of back-to-back launches; the smaller
per-launch time is used and both are reported).  `cpu_baseline` checks the GPU
result against the numpy oracle on a bounded sample of the workload and times
the PyTorch-CPU fp32 dequantize-then-matmul path on that sample with the host's
physical cores; every `also` workload carries the same oracle check.
`roofline.traffic` (HBM bytes per launch of the dominant kernel) is measured
in the run: rocprofv3 FETCH_SIZE / WRITE_SIZE counters over four short child
runs, calibrated on a device copy of known size (`--traffic committed` reports
the figure in profiles/traffic.json instead, as do the `also` workloads).

Ferret scoring mode (the reference's KERNEL_RESULT protocol, task_spec.py:277-356):

    python bench.py --kernel-result {decode_linear,fp8_dense,moe,all}

prints `KERNEL_RESULT {...}` (GPU TFLOPS per config, 0.0 when the result fails
the oracle check), `KERNEL_RESULT_REFERENCE {...}` (CPU fp32 oracle TFLOPS,
same run) and `ROOFLINE {...}` (GB/s, TFLOPS, roofline fraction), timed the
reference's way: a >= 512 MB write flush before every timed iteration (the
reference's 128 MB zero_() flush enlarged past the 256 MB MALL), >= 2 s of
warmup, median of `--iters` event-timed iterations.  --flush-read 1 adds a read
of a second 512 MB buffer after the write (the zeroed lines' write-back then
ends before the timed launch): a different protocol, labelled as such.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "achieved HBM GB/s (decode) / FP8 TFLOPS (prefill) + % roofline, 1×MI355X"
PEAK_HBM_GBPS = 8000.0
PEAK_FP8_TFLOPS = 5000.0
PEAK_BF16_TFLOPS = 2500.0
DEFAULT_WORKLOAD = "dsv3_fp8_M4096"
FAMILIES = {
    "decode_linear": ["qwen3_qkv_M16", "qwen3_o_M16", "qwen3_gateup_M16", "qwen3_down_M16", "qwen3_lmhead_M16"],
    "decode_linear_m1": ["qwen3_qkv_M1", "qwen3_o_M1", "qwen3_gateup_M1", "qwen3_down_M1", "qwen3_lmhead_M1"],
    "fp8_dense": ["dsv3_fp8_M16", "dsv3_fp8_M128", "dsv3_fp8_M4096"],
    "moe": ["dsv3_moe_w13_decode", "kimi_w4a16_w13_decode", "dsv3_moe_w13_prefill"],
    "moe_down": ["dsv3_moe_w2_decode", "dsv3_moe_w2_prefill"],
    "fp8_attn_tp8": [f"dsv3_{p}_M{m}" for m in (1, 16) for p in ("q_b_proj", "kv_b_proj", "o_proj")]
                    + ["dsv3_q_b_proj_M512", "dsv3_o_proj_M512"],
    "fp8_attn_prefill_tp8": [f"dsv3_{p}_M{m}" for m in (512, 1024, 2048, 4096, 8192)
                             for p in ("q_b_proj", "kv_b_proj", "o_proj")],
    "fp8_attn_prefill_large_m": ["dsv3_o_proj_M2048", "dsv3_q_b_proj_M8192", "dsv3_kv_b_proj_M8192",
                                 "dsv3_o_proj_M4096", "dsv3_o_proj_M8192"],
    "moe_ep8_decode": [f"dsv3_ep8_{p}_M{m}" for m in (1, 4, 8, 16) for p in ("gate_up", "down")],
    "moe_ep8_prefill": [f"dsv3_ep8_{p}_M{m}" for m in (64, 128, 256, 512) for p in ("gate_up", "down")],
    "kimi_tp8": ["kimi_w4a16_w13_T1_tp8", "kimi_w4a16_w13_T8_tp8"],
}
DENSE_KINDS = ("linear_bf16", "fp8_gemm", "fp8_gemm_ue8m0", "quant_act", "moe_combine")
# `also` workloads measured like the default one (in-run traffic, own CPU
# baseline): the largest BASELINE configuration, the DSv3 MoE w13 prefill.
MEASURED_ALSO = ("dsv3_moe_w13_prefill",)
INT4_LAYOUT = "tiled"  # --int4-layout
# The reference's own published figure for a workload of exactly this shape.
# It comes from other hardware and in another unit than the workload's metric,
# so it is reported next to the entry as context, never as vs_baseline.
PUBLISHED = {
    "qwen3_gateup_M16": {"value": 62.91, "unit": "TFLOP/s", "hardware": "B200",
                         "what": "the reference's decode kernel (cuBLAS on the same B200: 64.90)",
                         "source": "tasks/qwen3-8b-decode-linear-bs16-b200.yaml:65"},
    "kimi_w4a16_w13_T8_tp8": {"value": 13.19, "unit": "TFLOP/s", "hardware": "B200",
                              "what": "the reference's best INT4 w13 kernel, 128 MB flush before each launch "
                                      "(vLLM Marlin on the same B200: 9.36)",
                              "source": "correctness/kimi-moe-w13-precision-fix.md:14, "
                                        "tasks/kimi-moe-w13-int4-grouped-gemm.yaml:102"},
    "kimi_w4a16_w13_T1_tp8": {"value": 2.96, "unit": "TFLOP/s", "hardware": "B200",
                              "what": "the reference's best INT4 w13 kernel, 128 MB flush before each launch "
                                      "(vLLM Marlin on the same B200: 2.29)",
                              "source": "correctness/kimi-moe-w13-precision-fix.md:13, "
                                        "tasks/kimi-moe-w13-int4-grouped-gemm.yaml:101"},
}
MOE_KINDS = ("moe_fp8", "moe_w4a16", "moe_fp8_w2")
FAMILIES["all"] = list(dict.fromkeys(
    FAMILIES["decode_linear"] + FAMILIES["decode_linear_m1"] + FAMILIES["fp8_dense"] + FAMILIES["moe"]
    + FAMILIES["moe_down"] + FAMILIES["fp8_attn_tp8"] + FAMILIES["fp8_attn_prefill_tp8"]
    + FAMILIES["moe_ep8_decode"] + FAMILIES["moe_ep8_prefill"] + FAMILIES["kimi_tp8"]))


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------- GPU side

class Runner:
    """Inputs resident on the GPU plus a launch function for one step."""

    def __init__(self, wl, rotate_bytes: int = 512 << 20):
        import torch
        from ferret_amd import ops, workloads as W

        self.wl, self.torch, self.ops, self.W = wl, torch, ops, W
        t0 = time.perf_counter()
        self.inp = W.make_inputs(wl, "cuda")
        if wl.kind == "moe_w4a16" and INT4_LAYOUT == "tiled":
            # One-time load-time regrouping into 16-row x 128-K tiles (untimed,
            # as the reference repacks into Marlin's layout before timing).
            self.inp["wt"] = ops.int4_tile_weights(self.inp["w"])
        self.copies = [self.inp]
        if wl.kind in DENSE_KINDS:
            wbytes = sum(t.numel() * t.element_size() for t in self.inp.values())
            ncopy = max(1, math.ceil(rotate_bytes / max(wbytes, 1)))
            self.copies += [{k: v.clone() for k, v in self.inp.items()} for _ in range(ncopy - 1)]
        self.ws = None
        self.n_hit = 0
        if wl.kind in ("linear_bf16", "fp8_gemm", "fp8_gemm_ue8m0"):
            shape = (wl.M, wl.N)
            self.outs = [torch.empty(shape, dtype=torch.bfloat16, device="cuda") for _ in self.copies]
            if wl.kind == "fp8_gemm" and ops.fp8_workspace_bytes(wl.M, wl.N, wl.K):
                self.ws = torch.empty(ops.fp8_workspace_bytes(wl.M, wl.N, wl.K), dtype=torch.uint8, device="cuda")
            if wl.kind == "fp8_gemm_ue8m0":
                self.ws = torch.empty(ops.fp8_ue8m0_workspace_bytes(wl.M, wl.N, wl.K), dtype=torch.uint8,
                                      device="cuda")
        elif wl.kind == "quant_act":
            self.outs = [(torch.empty((wl.M, wl.K), dtype=torch.float8_e4m3fn, device="cuda"),
                          torch.empty((wl.M, wl.K // 128), dtype=torch.float32, device="cuda")) for _ in self.copies]
        elif wl.kind == "moe_combine":
            self.outs = [torch.empty((wl.T, wl.N), dtype=torch.bfloat16, device="cuda") for _ in self.copies]
        else:
            self.ids, _ = ops.moe_route_topk(self.inp["logits"], wl.topk)
            self.rt = ops.moe_permute(self.ids, wl.E)
            self.n_hit = W.experts_hit(self.ids, wl.E)
            cols = wl.N if wl.kind == "moe_fp8_w2" else wl.N // 2
            self.outs = [torch.empty((wl.T * wl.topk, cols), dtype=torch.bfloat16, device="cuda")]
        torch.cuda.synchronize()
        self.bytes = W.algorithmic_bytes(wl, self.n_hit)
        self.flops = W.flops(wl)
        log(f"[bench] {wl.key}: inputs ready in {time.perf_counter() - t0:.1f} s "
            f"({len(self.copies)} resident copies, experts hit {self.n_hit})")

    def gemm(self, i: int = 0):
        """Launch the dominant kernel (the GEMM) for step i."""
        wl, ops = self.wl, self.ops
        c = self.copies[i % len(self.copies)]
        o = self.outs[i % len(self.outs)]
        if wl.kind == "linear_bf16":
            ops.linear_bf16(c["x"], c["w"], residual=c.get("r"), out=o)
        elif wl.kind == "fp8_gemm":
            ops.fp8_gemm_blockscale(c["a"], c["sa"], c["b"], c["sb"], out=o, workspace=self.ws)
        elif wl.kind == "fp8_gemm_ue8m0":
            ops.fp8_gemm_ue8m0(c["a"], c["sfa"], c["b"], c["sfb"], out=o, workspace=self.ws)
        elif wl.kind == "moe_fp8":
            ops.moe_w13_fp8(c["x"], c["sx"], c["w"], c["sw"], self.rt, out=o)
        elif wl.kind == "moe_fp8_w2":
            ops.moe_w2_fp8(c["h"], c["sh"], c["w"], c["sw"], self.rt, out=o)
        elif wl.kind == "quant_act":
            ops.quant_act_e4m3(c["x"], q=o[0], scale=o[1])
        elif wl.kind == "moe_combine":
            ops.moe_combine(c["o"], c["w"], out=o)
        else:
            ops.moe_w13_w4a16(c["x"], c.get("wt", c["w"]), c["ws"], self.rt, out=o)

    def step(self, i: int, ev=None):
        """One pass of the hot path; `ev` = (start, end) events bracket the GEMM."""
        wl, ops = self.wl, self.ops
        if wl.kind in MOE_KINDS:
            self.ids, _ = ops.moe_route_topk(self.inp["logits"], wl.topk, with_weights=False)
            self.rt = ops.moe_permute(self.ids, wl.E, self.rt.tile_m)
        if ev is not None:
            ev[0].record()
        self.gemm(i)
        if ev is not None:
            ev[1].record()

    def output(self):
        return self.outs[0]


def published_of(wl, runner, kernel_us: float) -> dict | None:
    """PUBLISHED's entry for the workload with this run's figure in its unit."""
    p = PUBLISHED.get(wl.key)
    if p is None or not kernel_us:
        return None
    tflops = runner.flops / (kernel_us * 1e-6) / 1e12
    return {**p, "this_run": round(tflops, 2), "ratio": round(tflops / p["value"], 3)}


def unit_of(wl):
    return ("TFLOP/s", "mfma") if wl.bound == "mfma" else ("GB/s", "hbm")


def roofline_of(wl, runner, kernel_ms: float) -> dict:
    """Achieved rate of the dominant kernel against its roofline.

    `frac` is against the peak of the bound named (8 TB/s, or the FP8 / bf16
    MFMA peak); `frac_attainable` against min(peak, AI x 8 TB/s) in the line's
    unit (AI = algorithmic FLOP per algorithmic byte), which is what an
    HBM-limited prefill shape can reach at best; `frac_bf16_peak` (FP8 kinds)
    against the 2.5 PFLOP/s bf16 MFMA peak the exact-widening kernels run on.
    """
    unit, bound = unit_of(wl)
    ai = runner.flops / max(runner.bytes, 1)
    fp8 = wl.kind in ("fp8_gemm", "fp8_gemm_ue8m0", "moe_fp8", "moe_fp8_w2")
    mfma_peak = PEAK_FP8_TFLOPS if fp8 else PEAK_BF16_TFLOPS
    tflops = runner.flops / (kernel_ms * 1e-3) / 1e12
    gbps = runner.bytes / (kernel_ms * 1e-3) / 1e9
    if bound == "mfma":
        achieved, peak = tflops, mfma_peak
        attainable = min(mfma_peak, ai * PEAK_HBM_GBPS / 1e3)
    else:
        achieved, peak = gbps, PEAK_HBM_GBPS
        attainable = min(PEAK_HBM_GBPS, mfma_peak * 1e3 / max(ai, 1e-30))
    out = {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
           "frac": round(achieved / peak, 4), "attainable": round(attainable, 3),
           "frac_attainable": round(achieved / attainable, 4), "ai_flop_per_byte": round(ai, 3),
           "traffic": traffic_of(wl.key), "traffic_source": TRAFFIC_SOURCE,
           "kernel_us": round(kernel_ms * 1e3, 3), "algorithmic_bytes": runner.bytes, "flops": runner.flops}
    if fp8 and wl.kind != "quant_act":
        out["frac_bf16_peak"] = round(tflops / PEAK_BF16_TFLOPS, 4)
    return out


TRAFFIC_SOURCE = ("profiles/traffic.json: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of `bench.py --workload "
                  "KEY --launch-only 3`, scaled by a copy kernel of known size (not measured in this run)")


def _traffic_record(key: str):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as fh:
            return json.load(fh).get(key)
    except (OSError, ValueError):
        return None


def traffic_of(key: str):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary, if any."""
    rec = _traffic_record(key)
    return rec.get("bytes_per_launch") if rec else None


_COPY_FACTORS = None  # (fetch, write) bytes per counted KiB, from the first measurement of a run


def measure_traffic(key: str, timeout_s: float = 90.0):
    """HBM bytes per launch of the workload's dominant kernel (its name as in
    profiles/traffic.json), measured now: child runs under rocprofv3, one
    counter each -- FETCH_SIZE and WRITE_SIZE of `bench.py --workload KEY
    --launch-only 3`, then (once per bench run) of a 256 MiB device copy, whose
    known size turns the KiB counts into bytes.  Each run starts in /tmp
    (TMPDIR=/tmp) in its own process group, which is killed if the run outlives
    timeout_s.  Returns None when rocprofv3 is missing or a pass yields no
    dispatch of the kernel."""
    import shutil
    import signal
    import subprocess
    import tempfile
    from ferret_amd import profiling as P

    rec = _traffic_record(key)
    if not rec or not rec.get("kernel") or shutil.which("rocprofv3") is None:
        return None
    if "rocprof" in os.environ.get("LD_PRELOAD", "") or any(k.startswith("ROCPROF") for k in os.environ):
        log("[bench] already under rocprofv3: reporting the committed traffic figure")
        return None
    copy_bytes = 256 << 20
    tmp = tempfile.mkdtemp(prefix="ferret_pmc_", dir="/tmp")
    env = dict(os.environ, TMPDIR="/tmp")
    dirs = {}
    global _COPY_FACTORS
    passes = [("w", ["--workload", key, "--launch-only", "3"])]
    if _COPY_FACTORS is None:
        passes.append(("copy", ["--copy-bytes", str(copy_bytes)]))
    try:
        for tag, extra in passes:
            for counter in ("FETCH_SIZE", "WRITE_SIZE"):
                out = os.path.join(tmp, f"{tag}_{counter}")
                cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", out, "-o", "p", "--",
                       sys.executable, os.path.join(ROOT, "bench.py"), *extra]
                log(f"[bench] traffic pass: rocprofv3 --pmc {counter} -- bench.py {' '.join(extra)}")
                proc = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL,
                                        stderr=subprocess.DEVNULL, start_new_session=True)
                try:
                    proc.wait(timeout=timeout_s)
                except subprocess.TimeoutExpired:
                    os.killpg(proc.pid, signal.SIGKILL)
                    proc.wait()
                    log(f"[bench] traffic pass {counter} timed out; reporting the committed figure")
                    return None
                # rocprofv3 may exit non-zero after the program finished with its CSV written;
                # the parse below decides.
                dirs[(tag, counter)] = out
        if _COPY_FACTORS is None:
            _COPY_FACTORS = P.copy_factors(dirs[("copy", "FETCH_SIZE")], dirs[("copy", "WRITE_SIZE")], copy_bytes)
        t = P.traffic(rec["kernel"], dirs[("w", "FETCH_SIZE")], dirs[("w", "WRITE_SIZE")], "", "", copy_bytes,
                      factors=_COPY_FACTORS)
    except (OSError, ValueError, IndexError, KeyError) as e:
        log(f"[bench] traffic measurement failed ({e}); reporting the committed figure")
        return None
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    t["kernel"] = rec["kernel"]
    return t


# ---------------------------------------------------------------------------- CPU oracle leg

def cpu_threads() -> dict:
    """Threads for the PyTorch-CPU baseline: the host's physical cores, capped by
    OMP_NUM_THREADS when the environment sets it (the CPU share of one GPU)."""
    logical = os.cpu_count() or 1
    try:
        import psutil
        physical = psutil.cpu_count(logical=False) or logical
    except Exception:
        physical = logical
    n = physical
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return {"threads": n, "physical_cores": physical, "os_cpu_count": logical}


def _sample(wl, runner):
    """A bounded sample of the workload for the CPU legs.

    Returns (oracle_fn, torch_fn, got, s_flops, s_bytes, description, exact):
    oracle_fn runs the pinned numpy oracle (the correctness check), torch_fn the
    PyTorch-CPU fp32 dequantize-then-matmul path (the timed baseline) on the same
    sample, `got` the GPU result on it.
    """
    import numpy as np
    import torch
    from oracle import formats as F, gemm as G, quant as Q, routing as R, torch_cpu as TC

    def bits16(t):
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    def codes(t):
        return t.contiguous().view(torch.uint8).cpu().numpy()

    inp, out = runner.inp, runner.output()
    rng = np.random.default_rng(0)
    if wl.kind == "quant_act":
        nrows = min(wl.M, 2048)
        rows = np.sort(rng.choice(wl.M, size=nrows, replace=False))
        xs = F.bf16_bits_to_f32(bits16(inp["x"])[rows])
        got = (codes(out[0])[rows], out[1].cpu().numpy()[rows])
        return (lambda: Q.quant_act_1x128(xs), lambda: TC.quant_act_1x128(xs), got, 2 * nrows * wl.K,
                nrows * wl.K * 3 + nrows * (wl.K // 128) * 4, f"{nrows} of {wl.M} rows", True)
    got_all = F.bf16_bits_to_f32(bits16(out))
    if wl.kind == "moe_combine":
        ntok = min(wl.T, 1024)
        toks = np.sort(rng.choice(wl.T, size=ntok, replace=False))
        prow = (toks[:, None] * wl.topk + np.arange(wl.topk)[None, :]).reshape(-1)
        ob, wts = bits16(inp["o"])[prow], inp["w"].cpu().numpy()[toks]
        return (lambda: G.moe_combine(ob, wts), lambda: TC.moe_combine(ob, wts), got_all[toks],
                2 * ntok * wl.topk * wl.N, ntok * wl.topk * (wl.N * 2 + 4) + ntok * wl.N * 2,
                f"{ntok} of {wl.T} tokens x all {wl.N} columns", False)
    if wl.kind == "linear_bf16":
        xb, wb = bits16(inp["x"]), bits16(inp["w"])
        rb = bits16(inp["r"]) if "r" in inp else None
        return (lambda: G.linear_bf16(xb, wb, rb), lambda: TC.linear_bf16(xb, wb, rb), got_all,
                2 * wl.M * wl.N * wl.K, runner.bytes, f"all {wl.M} rows x {wl.N} outputs", False)
    if wl.kind == "fp8_gemm_ue8m0":
        from oracle import ue8m0 as U
        nrows = min(wl.M, 512)
        rows = np.sort(rng.choice(wl.M, size=nrows, replace=False)) if nrows < wl.M else np.arange(wl.M)
        a, b = codes(inp["a"])[rows], codes(inp["b"])
        # the scales as the kernel sees them: the packed bytes, decoded
        nk = wl.K // 128
        sa = U.ue8m0_to_float(U.unpack_sf(inp["sfa"].cpu().numpy().view(np.uint32), nk))[rows]
        sb = U.ue8m0_to_float(U.unpack_sf(inp["sfb"].cpu().numpy().view(np.uint32), nk))[::128]
        assert np.array_equal(sa, U.ue8m0_to_float(U.float_to_ue8m0(inp["sa"].cpu().numpy()[rows])))
        return (lambda: G.fp8_blockscale_gemm(a, sa, b, sb), lambda: TC.fp8_blockscale_gemm(a, sa, b, sb),
                got_all[rows], 2 * nrows * wl.N * wl.K, nrows * wl.K * 1 + wl.N * wl.K + nrows * wl.N * 2,
                f"{nrows} of {wl.M} rows x all {wl.N} outputs", False)
    if wl.kind == "fp8_gemm":
        nrows = min(wl.M, 1024)
        rows = np.sort(rng.choice(wl.M, size=nrows, replace=False)) if nrows < wl.M else np.arange(wl.M)
        a, sa, b, sb = codes(inp["a"])[rows], inp["sa"].cpu().numpy()[rows], codes(inp["b"]), inp["sb"].cpu().numpy()
        return (lambda: G.fp8_blockscale_gemm(a, sa, b, sb), lambda: TC.fp8_blockscale_gemm(a, sa, b, sb),
                got_all[rows], 2 * nrows * wl.N * wl.K, nrows * wl.K * 1 + wl.N * wl.K + nrows * wl.N * 2,
                f"{nrows} of {wl.M} rows x all {wl.N} outputs", False)
    ids = runner.ids.cpu().numpy()
    counts, offsets, sp = R.permute(ids, wl.E)
    hit = np.nonzero(counts)[0]
    order = hit[np.argsort(counts[hit], kind="stable")]
    nexp = 4
    experts = sorted({int(order[0]), int(order[-1])} | {int(e) for e in rng.permutation(hit)[: nexp - 2]})
    pairs = []
    for e in experts:
        seg = sp[offsets[e]:offsets[e + 1]]
        pairs.extend(int(p) for p in (seg if len(seg) <= 256 else np.r_[seg[:128], seg[-128:]]))
    pairs = np.array(pairs)
    emap = {e: i for i, e in enumerate(experts)}
    sub = np.vectorize(lambda v: emap.get(int(v), -1))(ids).astype(np.int32)
    ex_t = torch.tensor(experts, device="cuda")
    if wl.kind == "moe_fp8":
        x, sx = codes(inp["x"]), inp["sx"].cpu().numpy()
        w, sw = codes(inp["w"][ex_t]), inp["sw"][ex_t].cpu().numpy()
        fo = lambda: G.moe_w13_fp8(x, sx, w, sw, sub, pairs=pairs)  # noqa: E731
        ft = lambda: TC.moe_w13_fp8(x, sx, w, sw, sub, pairs)  # noqa: E731
        per_e = wl.N * wl.K
    elif wl.kind == "moe_fp8_w2":
        h, sh = codes(inp["h"]), inp["sh"].cpu().numpy()
        w, sw = codes(inp["w"][ex_t]), inp["sw"][ex_t].cpu().numpy()
        fo = lambda: G.moe_w2_fp8(h, sh, w, sw, sub, pairs=pairs)  # noqa: E731
        ft = lambda: TC.moe_w2_fp8(h, sh, w, sw, sub, pairs)  # noqa: E731
        per_e = wl.N * wl.K
    else:
        x = bits16(inp["x"])
        w, ws = inp["w"][ex_t].cpu().numpy(), bits16(inp["ws"][ex_t])
        fo = lambda: G.moe_w13_w4a16(x, w, ws, sub, pairs=pairs)  # noqa: E731
        ft = lambda: TC.moe_w13_w4a16(x, w, ws, sub, pairs)  # noqa: E731
        per_e = wl.N * wl.K // 2
    return (fo, ft, got_all[pairs], 2 * len(pairs) * wl.N * wl.K, len(experts) * per_e + len(pairs) * (wl.K + wl.N),
            f"{len(pairs)} routed rows of {len(experts)} experts (largest + smallest segment + random)", False)


def passes_gate(max_rel_err: float, non_finite: int) -> bool:
    """The reference's correctness gate: max relative error < 1e-2 and no
    NaN/Inf anywhere.  The error alone is not enough: it skips non-finite
    elements, so an all-NaN output would score 0 (the validator failure the
    reference records at tasks/kimi-moe-w13-int4-grouped-gemm.yaml:171-184)."""
    return bool(non_finite == 0 and max_rel_err < 1e-2)


def oracle_check(wl, runner) -> dict:
    """The GPU result on the bounded sample against the numpy oracle (one run)."""
    import numpy as np
    from oracle import metrics as MT
    fo, _, got, _, _, desc, exact = _sample(wl, runner)
    ref = fo()
    if exact:
        ok = bool(np.array_equal(got[0], ref[0]) and np.array_equal(got[1], ref[1]))
        return {"sample": desc, "max_rel_err": 0.0 if ok else float("inf"), "non_finite": 0, "correct": ok,
                "bit_exact": ok}
    err, nbad = MT.fp8_rel_err(got, ref)
    return {"sample": desc, "max_rel_err": err, "non_finite": nbad, "correct": passes_gate(err, nbad)}


def cpu_baseline(wl, runner, budget_s: float = 12.0) -> dict:
    """Check the GPU output against the numpy oracle on a bounded sample, then
    time the PyTorch-CPU fp32 dequantize-then-matmul path (oracle.torch_cpu) on
    the same sample with torch.set_num_threads(physical cores, capped by
    OMP_NUM_THREADS): one warmup, then the median of at least 3 runs, repeated
    up to ~budget_s seconds.  Throughput = the sample's FLOPs (or algorithmic
    bytes) over the median run time.
    """
    import torch
    check = oracle_check(wl, runner)
    _, ft, _, s_flops, s_bytes, desc, _ = _sample(wl, runner)
    thr = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(thr["threads"])
    try:
        ft()
        times = []
        t_start = time.perf_counter()
        while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 100):
            t0 = time.perf_counter()
            ft()
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev)
    med = statistics.median(times)
    unit, bound = unit_of(wl)
    value = s_flops / med / 1e12 if bound == "mfma" else s_bytes / med / 1e9
    log(f"[bench] cpu baseline {wl.key}: {thr['threads']} torch threads (physical cores "
        f"{thr['physical_cores']}, os.cpu_count() {thr['os_cpu_count']}), median {med:.3f} s of {len(times)} runs")
    return {"value": round(value, 6), "unit": unit, "cores": thr["threads"], "kind": "port",
            "sample": f"{desc}; PyTorch-CPU fp32 dequantize-then-matmul (oracle/torch_cpu.py), "
                      f"median of {len(times)} runs ({med:.3f} s each)",
            "physical_cores": thr["physical_cores"], "os_cpu_count": thr["os_cpu_count"],
            "tflops": round(s_flops / med / 1e12, 6), "max_rel_err": check["max_rel_err"],
            "non_finite": check["non_finite"], "correct": check["correct"], "oracle_check": check["sample"]}


# ---------------------------------------------------------------------------- modes

def settle_clocks(runner, seconds: float = 0.5) -> None:
    """Run the step untimed for `seconds` so the GPU leaves its idle clocks
    before the warmup steps (a few ms of warmup alone measures the ramp)."""
    import torch
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end:
        runner.step(i)
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_steps(runner, steps: int, warmup: int):
    """Returns (wall ms per step, kernel ms per launch, detail).

    Pass 1: one event pair per step around the GEMM (a MoE step routes first,
    so the pair brackets the GEMM alone).  For the single-launch workloads
    three more passes each time the same number of back-to-back launches (each
    on its own weight copy) under one event pair; a pass counts only if its
    spin kernel held the GPU until the host had enqueued it, and the fastest
    counted one is the burst figure.  Both over-state the kernel's own
    duration -- the pairs by the event records' few microseconds per launch
    (large for a ~10 us kernel), the burst by the gaps between launches --
    so the kernel time is the smaller of the two; both are reported.  The
    burst is enqueued behind a spin kernel, so the host's issue rate does not
    enter it.  `board_power_w` is the board's mean power (amdgpu hwmon) over
    the untimed settle run, which repeats the step back to back for 0.8 s; the
    first 40 % of its samples (the ramp) are left out.
    """
    import torch
    from ferret_amd.power import PowerSampler
    with PowerSampler(_power_file()) as ps:
        settle_clocks(runner, 0.8)
    pw = ps.summary(skip=0.4)
    power = {"board_power_w": pw["mean_w"] if pw else None}
    for i in range(warmup):
        runner.step(i)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        runner.step(warmup + i, evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    pairs_ms = statistics.mean(s.elapsed_time(e) for s, e in evs)
    if runner.wl.kind in MOE_KINDS:
        return wall * 1e3 / steps, pairs_ms, {"kernel_us_event_pairs": round(pairs_ms * 1e3, 3), **power}
    # The burst is enqueued while a spin kernel holds the GPU, so the launches
    # run back to back however slowly the host issues them (a ~10 us kernel
    # launches faster than Python can enqueue it).  A burst counts only if the
    # spin held the GPU longer than the host took to enqueue it; of three, the
    # fastest counted one is kept.
    enq_est_ms = wall * 1e3
    bursts, enq_ms, held_ms = [], 0.0, []
    for rep in range(3):
        evs, ev0, ev1 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        evs.record()
        _gpu_busy(2.0 * enq_est_ms + 1.0)
        ev0.record()
        t1 = time.perf_counter()
        for i in range(steps):
            runner.step(warmup + (1 + rep) * steps + i)
        ev1.record()
        enq = (time.perf_counter() - t1) * 1e3
        torch.cuda.synchronize()
        enq_ms = max(enq_ms, enq)
        held_ms.append(evs.elapsed_time(ev0))
        if held_ms[-1] > enq:
            bursts.append(ev0.elapsed_time(ev1) / steps)
    burst_ms = min(bursts) if bursts else None
    kernel_ms = pairs_ms if burst_ms is None else min(pairs_ms, burst_ms)
    return wall * 1e3 / steps, kernel_ms, {
        "kernel_us_event_pairs": round(pairs_ms * 1e3, 3),
        "kernel_us_burst": None if burst_ms is None else round(burst_ms * 1e3, 3),
        "bursts_counted": len(bursts), "burst_host_enqueue_ms": round(enq_ms, 3),
        "burst_gpu_held_ms": round(min(held_ms), 3), **power}


_POWER_FILE = []


def _power_file():
    """The device's hwmon board-power file (None where there is none), found once."""
    if not _POWER_FILE:
        from ferret_amd.power import pick_power_file, device_pci_bus
        pick = pick_power_file(device_pci_bus(0))
        _POWER_FILE.append(pick[1] if pick else None)
    return _POWER_FILE[0]


def _gpu_busy(ms: float) -> None:
    """Keep the GPU busy for about `ms` (capped at 50) with torch's bounded spin
    kernel, whose rate (clock cycles) is measured right before: the clock moves
    between workloads."""
    import torch
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    torch.cuda._sleep(200_000)
    b.record()
    b.synchronize()
    per_ms = 200_000 / max(a.elapsed_time(b), 1e-3)
    torch.cuda._sleep(int(per_ms * min(ms, 50.0)))


def driver_mode(args) -> int:
    from ferret_amd import workloads as W, lib

    log(f"[bench] {lib.version()}")
    wl = W.WORKLOADS[args.workload]
    runner = Runner(wl)
    ms_per_step, kernel_ms, timing = time_steps(runner, args.steps, args.warmup)
    unit, bound = unit_of(wl)
    per_step = runner.flops / 1e12 if bound == "mfma" else runner.bytes / 1e9
    value = per_step / (ms_per_step * 1e-3)
    roof = roofline_of(wl, runner, kernel_ms)
    roof.update(timing)
    if args.traffic == "measure":
        t = measure_traffic(wl.key)
        if t is not None:
            roof["traffic"] = t["bytes_per_launch"]
            roof["traffic_source"] = (f"measured in this run: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of "
                                      f"{t['kernel']} (bench.py --workload {wl.key} --launch-only 3), KiB scaled "
                                      f"by a 256 MiB device copy (factors {t['fetch_factor']} / {t['write_factor']})")
            roof["traffic_fetch_bytes"], roof["traffic_write_bytes"] = t["fetch_bytes"], t["write_bytes"]
    if roof.get("traffic"):
        roof["traffic_ratio"] = round(roof["traffic"] / runner.bytes, 3)
    cpu = None if args.no_cpu_baseline else cpu_baseline(wl, runner, args.cpu_budget)
    also = []
    correct_all = True
    for key in args.also:
        w2 = W.WORKLOADS[key]
        r2 = Runner(w2)
        m2, k2, t2 = time_steps(r2, max(10, args.steps), 3)
        u2, _ = unit_of(w2)
        rf = roofline_of(w2, r2, k2)
        entry = {"workload": key, "ms_per_step": round(m2, 5), "kernel_us": rf["kernel_us"],
                 "achieved": rf["achieved"], "unit": u2, "frac": rf["frac"],
                 "frac_attainable": rf["frac_attainable"], "bound": rf["bound"],
                 **({"frac_bf16_peak": rf["frac_bf16_peak"]} if "frac_bf16_peak" in rf else {}),
                 **({"int4_layout": INT4_LAYOUT} if w2.kind == "moe_w4a16" else {}),
                 "traffic": rf["traffic"], "traffic_source": "profiles/traffic.json (committed)"}
        if key in MEASURED_ALSO:
            # The largest configuration gets the default workload's treatment:
            # HBM traffic measured in this run and its own CPU baseline.
            if args.traffic == "measure":
                t = measure_traffic(key)
                if t is not None:
                    entry["traffic"] = t["bytes_per_launch"]
                    entry["traffic_fetch_bytes"], entry["traffic_write_bytes"] = t["fetch_bytes"], t["write_bytes"]
                    entry["traffic_source"] = (f"measured in this run: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of "
                                               f"{t['kernel']} (bench.py --workload {key} --launch-only 3)")
            if not args.no_cpu_baseline:
                entry["cpu_baseline"] = cpu_baseline(w2, r2, min(args.cpu_budget, 8.0))
        if entry["traffic"]:
            entry["traffic_ratio"] = round(entry["traffic"] / r2.bytes, 3)
        pub = published_of(w2, r2, rf["kernel_us"])
        if pub:
            entry["reference_published"] = pub
        chk = oracle_check(w2, r2)
        entry.update({"oracle_check": chk, **t2})
        also.append(entry)
        correct_all = correct_all and chk["correct"]
        del r2
    correct = True if cpu is None else cpu["correct"]
    if not correct_all:
        log("[bench] an `also` workload failed its oracle check (see its oracle_check)")
    line = {
        "metric": METRIC, "value": round(value, 3) if correct else 0.0, "unit": unit, "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype_of(wl),
        "data": "synthetic (seeded torch generators, absmax/448 e4m3 quantization; weights rotated over >=512 MB "
                "of resident copies for dense workloads)",
        "config": config_of(wl, runner), "roofline": roof, "cpu_baseline": cpu, "also": also,
    }
    pub = published_of(wl, runner, roof.get("kernel_us"))
    if pub:
        line["reference_published"] = pub
    print(json.dumps(line), flush=True)
    return 0 if correct else 1


def dtype_of(wl) -> str:
    return {"linear_bf16": "bf16", "fp8_gemm": "e4m3 (fp32 accumulate)",
            "fp8_gemm_ue8m0": "e4m3, UE8M0 block scales (fp32 accumulate)", "moe_fp8": "e4m3 (fp32 accumulate)",
            "moe_w4a16": "int4 weights x bf16 (fp32 accumulate)", "moe_fp8_w2": "e4m3 (fp32 accumulate)",
            "quant_act": "bf16 -> e4m3 (fp32 scale)", "moe_combine": "bf16 (fp32 accumulate)"}[wl.kind]


def config_of(wl, runner) -> dict:
    c = {"workload": wl.key, "description": wl.description, "parallelism": "single GPU"}
    for k in ("M", "N", "K", "T", "E", "topk"):
        v = getattr(wl, k)
        if v:
            c[k] = v
    if runner.n_hit:
        c["experts_hit"] = runner.n_hit
    if wl.kind == "moe_w4a16":
        c["int4_layout"] = INT4_LAYOUT
    return c


def kernel_result_mode(args) -> int:
    import torch
    from ferret_amd import workloads as W

    keys = FAMILIES[args.kernel_result]
    flush = torch.empty(args.flush_mb << 20, dtype=torch.uint8, device="cuda")
    # Read after the write: the zeroed lines sit dirty in L2 / MALL, and without
    # this pass their write-back would run inside the next timed GEMM.
    flush_rd = torch.ones(args.flush_mb << 18, dtype=torch.int32, device="cuda") if args.flush_read else None
    res, ref, roof = {}, {}, {}
    for key in keys:
        wl = W.WORKLOADS[key]
        runner = Runner(wl, rotate_bytes=0)
        runner.gemm(0)
        torch.cuda.synchronize()
        cpu = cpu_baseline(wl, runner, min(args.cpu_budget, 2.0))
        t_end = time.perf_counter() + args.warmup_s
        while time.perf_counter() < t_end:
            for _ in range(10):
                runner.gemm(0)
            torch.cuda.synchronize()
        times = []
        for _ in range(args.iters):
            flush.zero_()
            if flush_rd is not None:
                flush_rd.max()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            runner.gemm(0)
            e.record()
            e.synchronize()
            times.append(s.elapsed_time(e))
        med = statistics.median(times)
        tflops = runner.flops / (med * 1e-3) / 1e12
        res[key] = round(tflops, 4) if cpu["correct"] else 0.0
        ref[key] = round(cpu["tflops"], 6)
        rf = roofline_of(wl, runner, med)
        roof[key] = {"us": round(med * 1e3, 2), "gbps": round(runner.bytes / (med * 1e-3) / 1e9, 1),
                     "flush": "write+read (not the reference protocol)" if args.flush_read else "write (reference)",
                     "tflops": round(tflops, 2), "bound": rf["bound"], "frac": rf["frac"],
                     "valid": cpu["correct"], "max_rel_err": cpu["max_rel_err"], "cpu_cores": cpu["cores"]}
        log(f"[kernel-result] {key}: {med * 1e3:.1f} us, {tflops:.2f} TFLOPS, "
            f"{roof[key]['gbps']:.0f} GB/s, frac {rf['frac']:.3f}, valid {cpu['correct']}")
        del runner
        torch.cuda.empty_cache()
    print("KERNEL_RESULT " + json.dumps(res), flush=True)
    print("KERNEL_RESULT_REFERENCE " + json.dumps(ref), flush=True)
    print("ROOFLINE " + json.dumps(roof), flush=True)
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD)
    ap.add_argument("--also", nargs="*", default=None,
                    help="extra workloads measured in the same run (default with the default workload: all others)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of CPU oracle work for cpu_baseline (KERNEL_RESULT mode: at most 2 per config)")
    ap.add_argument("--kernel-result", choices=sorted(FAMILIES), default=None)
    ap.add_argument("--iters", type=int, default=300)
    ap.add_argument("--warmup-s", type=float, default=2.0)
    ap.add_argument("--flush-mb", type=int, default=512)
    ap.add_argument("--flush-read", type=int, default=0,
                    help="0 (default): the reference's write-only flush; 1: also read a second buffer of the same "
                         "size after it, so the write-back of the zeroed lines ends before the timed launch "
                         "(not the reference's protocol: those numbers are not comparable with its own)")
    ap.add_argument("--launch-only", type=int, default=0, metavar="N",
                    help="only launch the workload's GEMM N times (for hardware-counter runs)")
    ap.add_argument("--copy-bytes", type=int, default=0, metavar="B",
                    help="only run 3 device copies of B bytes (calibrates FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--traffic", choices=("measure", "committed"), default="measure",
                    help="roofline.traffic of the default workload: measured in this run with rocprofv3 "
                         "(four short child runs, about a minute) or the committed profiles/traffic.json figure")
    ap.add_argument("--int4-layout", choices=("tiled", "checkpoint"), default="tiled",
                    help="INT4 w13 weights: regrouped once into 16-row x 128-K tiles (default) or the "
                         "checkpoint's [E, N, K/8] words")
    args = ap.parse_args(argv)
    global INT4_LAYOUT
    INT4_LAYOUT = args.int4_layout
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this benchmark measures the quantized-GEMM path on "
              "one GPU only (no collective or sharded step exists). Run with --gpus 1.", file=sys.stderr)
        return 2
    if args.also is None:
        args.also = [k for k in ("dsv3_fp8_M16", "dsv3_fp8_M128", "qwen3_gateup_M16", "dsv3_moe_w13_decode",
                                 "kimi_w4a16_w13_decode", "dsv3_moe_w13_prefill", "dsv3_moe_w2_decode",
                                 "dsv3_moe_w2_prefill", "moe_quant_act_prefill", "moe_combine_prefill",
                                 "dsv3_o_proj_M4096_ue8m0")
                     ] if args.workload == DEFAULT_WORKLOAD else []
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    if args.copy_bytes:
        src = torch.empty(args.copy_bytes, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copied {args.copy_bytes} bytes x 3")
        return 0
    if args.launch_only:
        from ferret_amd import workloads as W
        r = Runner(W.WORKLOADS[args.workload], rotate_bytes=0)
        for i in range(args.launch_only):
            r.gemm(i)
        torch.cuda.synchronize()
        log(f"[bench] {args.workload}: {args.launch_only} launches")
        return 0
    if args.kernel_result:
        return kernel_result_mode(args)
    return driver_mode(args)


if __name__ == "__main__":
    raise SystemExit(main())
