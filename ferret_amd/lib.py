"""ctypes binding of libferret_hip.so (the C ABI declared in include/ferret_hip.h).

There is no fallback: if the library is missing or fails to load, every op
raises.  torch is imported before the library so that the HIP runtime torch
bundles (soname libamdhip64.so.7) is the one our library binds to: one runtime,
one set of streams.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libferret_hip.so")

_c_int, _c_void_p, _c_size_t, _c_char_p = ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_char_p
_vp = _c_void_p

# name -> (restype, argtypes); must list every function of include/ferret_hip.h
SIGNATURES = {
    "ferret_version": (_c_char_p, []),
    "ferret_error_string": (_c_char_p, [_c_int]),
    "launch_gemv": (None, [_vp, _vp, _vp, _vp, _c_int, _c_int, _vp]),
    "ferret_linear_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _c_size_t, _vp]),
    "ferret_fp8_gemm_blockscale": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _c_size_t, _vp]),
    "ferret_fp8_gemm_ue8m0": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _c_size_t, _vp]),
    "ferret_moe_route_topk": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "ferret_moe_permute": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _c_int, _vp, _vp,
                                    _c_size_t, _vp]),
    "ferret_moe_max_tiles": (_c_int, [_c_int, _c_int, _c_int]),
    "ferret_moe_tile_m": (_c_int, [_c_int, _c_int]),
    "ferret_moe_w13_fp8": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                    _c_int, _c_int, _vp, _vp]),
    "ferret_moe_w13_w4a16": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                      _c_int, _c_int, _vp, _vp]),
    "ferret_moe_w13_w4a16_tiled": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int,
                                            _c_int, _c_int, _c_int, _vp, _vp]),
    "ferret_int4_tile_weights": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "ferret_quant_act_e4m3": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _vp]),
    "ferret_moe_w2_fp8": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                   _c_int, _vp, _vp]),
    "ferret_moe_combine": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "ferret_linear_bf16_noalloc": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "ferret_linear_bf16_noalloc_max_bytes": (_c_size_t, []),
    "ferret_fp8_gemm_blockscale_ex": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _c_size_t,
                                               _c_int, _vp]),
    "ferret_moe_w13_fp8_ex": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                       _c_int, _c_int, _vp, _c_int, _vp]),
    "ferret_moe_w2_fp8_ex": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                      _c_int, _vp, _c_int, _vp]),
    "ferret_workspace_bytes": (_c_size_t, [_c_int, _c_int, _c_int, _c_int, _c_int]),
}


# Flag bits of the FP8 *_ex entry points (include/ferret_hip.h).
FP8_MMA_E4M3 = 1


class FerretError(RuntimeError):
    """A C-ABI entry point returned a non-zero code."""

    def __init__(self, fn: str, code: int, text: str):
        super().__init__(f"{fn} failed with code {code}: {text}")
        self.code = code


_LIB = None


def load():
    """Load (once) and return the ctypes library; raise if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    import torch  # noqa: F401  (binds the HIP runtime torch ships before ours)

    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m ferret_amd.build`")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def check(fn: str, code: int) -> None:
    if code != 0:
        text = load().ferret_error_string(code).decode()
        raise FerretError(fn, code, text)


def version() -> str:
    return load().ferret_version().decode()
