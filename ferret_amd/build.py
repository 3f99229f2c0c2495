"""Build libferret_hip.so (gfx950) in-tree with hipcc.

    python -m ferret_amd.build            # compile every source, link the library
    python -m ferret_amd.build --verbose  # also print kernel register/LDS usage

Objects go to ferret_amd/_build/, the library to ferret_amd/libferret_hip.so.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libferret_hip.so")
SOURCES = ["skinny.hip", "fp8_tiled.hip", "fp8_square.hip", "routing.hip", "moe_tail.hip", "ue8m0.hip",
           "dispatch.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    # Packed FP32 (v_pk_*_f32) stays off: plain scalar FP32 VALU only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ArchVGPRs: the epilogues read them with VALU ops, and the
    # AGPR form would add a v_accvgpr_read per accumulator element.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    f"-I{os.path.join(ROOT, 'include')}",
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libferret_hip.so)")


def _compile(src: str, verbose: bool) -> tuple[str, str]:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        cmd += ["-Rpass-analysis=kernel-resource-usage"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = res.stdout + res.stderr
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{out}")
    return obj, out


def resource_usage(sources=None, jobs: int | None = None) -> dict[str, dict[str, int]]:
    """Per-kernel register, scratch and LDS use of the device code, from hipcc's
    kernel-resource-usage remarks (a device-only compile into a scratch
    directory; the library is not touched).  Returns {mangled name: {"vgpr",
    "agpr", "sgpr", "scratch" (bytes per lane), "vgpr_spill", "sgpr_spill",
    "occupancy" (waves per SIMD), "lds" (static bytes)}}."""
    import re
    import tempfile

    fields = {"VGPRs": "vgpr", "AGPRs": "agpr", "TotalSGPRs": "sgpr", "ScratchSize [bytes/lane]": "scratch",
              "VGPRs Spill": "vgpr_spill", "SGPRs Spill": "sgpr_spill", "Occupancy [waves/SIMD]": "occupancy",
              "LDS Size [bytes/block]": "lds"}
    keys = sorted(fields, key=len, reverse=True)  # "VGPRs Spill" before "VGPRs"
    pat = re.compile(r"remark:\s+(Function Name|" + "|".join(re.escape(k) for k in keys) + r"): (\S+)")

    def one(src: str, tmp: str) -> str:
        cmd = [hipcc(), *HIPCC_FLAGS, "--offload-device-only", "-c", os.path.join(CSRC, src), "-o",
               os.path.join(tmp, src + ".o"), "-Rpass-analysis=kernel-resource-usage"]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}{res.stderr}")
        return res.stderr

    out: dict[str, dict[str, int]] = {}
    srcs = list(sources or SOURCES)
    with tempfile.TemporaryDirectory() as tmp, \
            cf.ThreadPoolExecutor(max_workers=jobs or min(len(srcs), os.cpu_count() or 1)) as ex:
        for text in ex.map(lambda s: one(s, tmp), srcs):
            cur = None
            for m in pat.finditer(text):
                key, val = m.group(1), m.group(2)
                if key == "Function Name":
                    cur = out.setdefault(val, {})
                elif cur is not None:
                    cur[fields[key]] = int(val)
    return out


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        results = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    objs = []
    for (obj, out), src in zip(results, SOURCES):
        objs.append(obj)
        if verbose and out.strip():
            print(f"== {src}\n{out}", file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    path = build(verbose=args.verbose)
    print(path)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
