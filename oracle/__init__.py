"""CPU oracle for the quantized-GEMM path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy on the CPU, the algorithm of every function on
the hot path so that the HIP kernels can be checked against it.  It is what
the tests compare with, never the product: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The ``ferret_amd`` package
never imports it and has no CPU fallback.

Modules (each function cites the reference file:line it follows; paths are
relative to the reference repository root):

* ``formats``  — OCP e4m3fn decode/encode, bf16 round-to-nearest-even, INT4
  nibble unpack + group-32 dequant.
* ``gemm``     — bf16 decode linear, FP8 1x128/128x128 block-scaled GEMM,
  FP8 MoE w13 + SiLU, INT4 W4A16 MoE w13 + SiLU.
* ``routing``  — top-k routing on logits, expert histogram, stable
  permutation, tile table.
* ``quant``    — absmax/448 1x128 (activation) and 128x128 (weight)
  quantizers used to build synthetic inputs.
* ``metrics``  — the reference's error metrics and NaN-aware gates.

Pinning (what fixes each function independently of its own formula) is listed
in each module header and exercised by ``tests/test_oracle_*.py``.
"""
