"""Board power while a workload runs back to back (amdgpu hwmon, read-only).

    python -m ferret_amd.power [--seconds S] SPEC [SPEC ...]

SPEC is a workload key (ferret_amd.workloads.WORKLOADS), optionally followed by
`:full` or `:partial` for a grouped MoE GEMM (only the tiles of the routing's
tile table with tile_m rows, or only those with fewer), or by `:full|partial`
(both subsets launched together on two streams of default priority, each
step waiting for both), or `torch.matmul:MxNxK` for the vendor bf16 GEMM of
that shape.  Each SPEC runs
back to back for S seconds; the table gives the time per launch, the board's
average power over the run (the first fifth, the ramp, left out), the idle
power just before, and the energy per launch.

The reading is the hwmon `power1_average` (else `power1_input`) of the DRM
card whose PCI address is the device's, else of the only card that has one.
"""
from __future__ import annotations

import argparse
import glob
import os
import threading
import time

HWMON_GLOB = "/sys/class/drm/card*/device/hwmon/hwmon*"


def power_files(root_glob: str = HWMON_GLOB) -> dict[str, str]:
    """{card: path} of each card's board-power reading (micro-watts)."""
    out = {}
    for hw in sorted(glob.glob(root_glob)):
        card = hw.split(os.sep)[-4]
        for name in ("power1_average", "power1_input"):
            p = os.path.join(hw, name)
            if os.path.exists(p) and card not in out:
                out[card] = p
    return out


def card_pci(card_path: str) -> str:
    """PCI address (domain:bus:device.function) a DRM card's device links to."""
    return os.path.basename(os.path.realpath(card_path)).lower()


def pick_power_file(pci_bus: str | None = None, root_glob: str = HWMON_GLOB) -> tuple[str, str] | None:
    """(card, path) of the board-power reading of the device at PCI address
    `pci_bus` (any suffix of domain:bus:device.function), else of the only card
    that has one; None when neither identifies one card."""
    files = power_files(root_glob)
    if pci_bus:
        want = pci_bus.lower()
        for card, path in files.items():
            dev = os.path.dirname(os.path.dirname(os.path.dirname(path)))  # .../cardN/device
            if card_pci(dev).endswith(want):
                return card, path
    if len(files) == 1:
        return next(iter(files.items()))
    return None


def device_pci_bus(index: int = 0) -> str | None:
    """PCI address of torch device `index` as "bus:device.function" (hex), or None."""
    try:
        import torch
        p = torch.cuda.get_device_properties(index)
        bus, dev = int(getattr(p, "pci_bus_id")), int(getattr(p, "pci_device_id"))
        return f"{bus:02x}:{dev:02x}.0"
    except Exception:
        return None


class PowerSampler:
    """Samples one hwmon power file every `interval` seconds on a thread.

    `summary()` gives the mean and max in watts over the samples after the
    first `skip` fraction (the ramp), or None when there is no reading."""

    def __init__(self, path: str | None, interval: float = 0.02):
        self.path, self.interval = path, interval
        self.samples: list[float] = []
        self._stop = threading.Event()
        self._t = None

    def _read(self) -> float | None:
        try:
            with open(self.path) as fh:
                return int(fh.read().strip()) / 1e6
        except (OSError, ValueError):
            return None

    def _run(self):
        while not self._stop.is_set():
            v = self._read()
            if v is not None:
                self.samples.append(v)
            self._stop.wait(self.interval)

    def __enter__(self):
        if self.path:
            self._t = threading.Thread(target=self._run, daemon=True)
            self._t.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        if self._t is not None:
            self._t.join()
        return False

    def summary(self, skip: float = 0.2) -> dict | None:
        s = self.samples[int(len(self.samples) * skip):]
        if not s:
            return None
        return {"mean_w": round(sum(s) / len(s), 1), "max_w": round(max(s), 1), "samples": len(s)}


# ---------------------------------------------------------------------------- CLI (needs a GPU)

def tile_subset(tiles_host, ntiles: int, tile_m: int, which: str):
    """Rows of a [max_tiles, 3] (expert, row0, nrows) tile table of one class:
    "full" = nrows == tile_m, "partial" = nrows < tile_m, "all" = every row."""
    t = tiles_host[:ntiles]
    if which == "full":
        return t[t[:, 2] == tile_m]
    if which == "partial":
        return t[t[:, 2] < tile_m]
    if which == "all":
        return t
    raise ValueError(f"tile class {which!r}: expected all, full or partial")


def _launcher(spec: str):
    import dataclasses
    import torch
    from ferret_amd import ops, workloads as W

    key, _, arg = spec.partition(":")
    if key == "torch.matmul":
        M, N, K = (int(v) for v in arg.split("x"))
        xa = torch.randn((M, K), device="cuda").to(torch.bfloat16)
        xb = torch.randn((K, N), device="cuda").to(torch.bfloat16)
        return lambda: torch.matmul(xa, xb)
    wl = W.WORKLOADS[key]
    inp = W.make_inputs(wl, "cuda")
    if wl.kind in ("moe_fp8", "moe_fp8_w2", "moe_w4a16"):
        ids, _ = ops.moe_route_topk(inp["logits"], wl.topk)
        rt_all = ops.moe_permute(ids, wl.E)
        cols = wl.N if wl.kind == "moe_fp8_w2" else wl.N // 2
        wt = ops.int4_tile_weights(inp["w"]) if wl.kind == "moe_w4a16" else None

        def one(which):
            rt = rt_all
            if which:
                nt = int(rt.ntiles.item())
                sel = tile_subset(rt.tiles.cpu(), nt, rt.tile_m, which)
                tiles = torch.zeros_like(rt.tiles)
                tiles[: sel.shape[0]] = sel.to(tiles.device)
                rt = dataclasses.replace(rt, tiles=tiles,
                                         ntiles=torch.tensor([sel.shape[0]], dtype=torch.int32, device="cuda"))
            out = torch.empty((wl.T * wl.topk, cols), dtype=torch.bfloat16, device="cuda")
            if wl.kind == "moe_fp8":
                return lambda: ops.moe_w13_fp8(inp["x"], inp["sx"], inp["w"], inp["sw"], rt, out=out)
            if wl.kind == "moe_fp8_w2":
                return lambda: ops.moe_w2_fp8(inp["h"], inp["sh"], inp["w"], inp["sw"], rt, out=out)
            return lambda: ops.moe_w13_w4a16(inp["x"], wt, inp["ws"], rt, out=out)

        if "|" not in arg:
            return one(arg)
        # Both tile classes at once: each on its own stream (default priority),
        # the caller's stream waiting for both.
        fa, fb = (one(w) for w in arg.split("|"))
        sa, sb = torch.cuda.Stream(), torch.cuda.Stream()

        def both():
            cur = torch.cuda.current_stream()
            sa.wait_stream(cur)
            sb.wait_stream(cur)
            with torch.cuda.stream(sa):
                fa()
            with torch.cuda.stream(sb):
                fb()
            cur.wait_stream(sa)
            cur.wait_stream(sb)
        return both
    if arg:
        raise ValueError(f"{spec}: a tile class applies to grouped MoE workloads only")
    out = torch.empty((wl.M, wl.N), dtype=torch.bfloat16, device="cuda")
    if wl.kind == "fp8_gemm":
        ws = None
        if ops.fp8_workspace_bytes(wl.M, wl.N, wl.K):
            ws = torch.empty(ops.fp8_workspace_bytes(wl.M, wl.N, wl.K), dtype=torch.uint8, device="cuda")
        return lambda: ops.fp8_gemm_blockscale(inp["a"], inp["sa"], inp["b"], inp["sb"], out=out, workspace=ws)
    if wl.kind == "linear_bf16":
        return lambda: ops.linear_bf16(inp["x"], inp["w"], residual=inp.get("r"), out=out)
    raise ValueError(f"{spec}: workload kind {wl.kind} is not covered")


def measure(spec: str, seconds: float, path: str | None) -> dict:
    import torch
    f = _launcher(spec)
    for _ in range(3):
        f()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(); f(); b.record(); b.synchronize()
    batch = max(1, int(20e3 / max(a.elapsed_time(b) * 1e3, 1.0)))  # ~20 ms between host syncs
    with PowerSampler(path) as idle:
        time.sleep(0.5)
    n = 0
    with PowerSampler(path) as busy:
        t_end = time.perf_counter() + seconds
        a.record()
        while time.perf_counter() < t_end:
            for _ in range(batch):
                f()
            n += batch
            torch.cuda.synchronize()
        b.record(); b.synchronize()
    us = a.elapsed_time(b) * 1e3 / n
    p, q = busy.summary(), idle.summary(skip=0.0)
    r = {"spec": spec, "us_per_launch": round(us, 1), "launches": n,
         "power_w": p["mean_w"] if p else None, "power_max_w": p["max_w"] if p else None,
         "idle_w": q["mean_w"] if q else None}
    r["mj_per_launch"] = round(r["power_w"] * us * 1e-3, 1) if p else None
    return r


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--seconds", type=float, default=3.0)
    ap.add_argument("specs", nargs="+")
    args = ap.parse_args(argv)
    pick = pick_power_file(device_pci_bus(0))
    print(f"power reading: {pick[1] if pick else 'none found'}", flush=True)
    print("| run | us per launch | board W (mean / max) | idle W before | mJ per launch |\n|---|---|---|---|---|",
          flush=True)
    for spec in args.specs:
        r = measure(spec, args.seconds, pick[1] if pick else None)
        print(f"| {r['spec']} | {r['us_per_launch']} | {r['power_w']} / {r['power_max_w']} | {r['idle_w']} | "
              f"{r['mj_per_launch']} |", flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
