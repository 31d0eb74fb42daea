"""CPU oracle for the W4A8/W4A4 quantized-linear hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (`kitchen_amd`, `libmq.so`) imports, links
or executes anything under `oracle/`. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` use it, and only as the checker or the timed CPU baseline.

The oracle restates, in numpy float32/integer arithmetic, the arithmetic the reference
(JoaoZaokk/comfy-quant-bench) performs on this path. Every function cites the reference
file:line it follows. The modules are:

    hadamard   closed-form H_b and the pinned-order radix-4 FWHT
    quant      per-token activation quantizers, weight quantizers, int4 packing
    swiglu     the SwiGLU prologue (silu correctly rounded to fp32, product rounded to bf16)
    gemm       exact integer per-group partials and the fp64 epilogue
    torch_path the reference's CPU torch path (rotate, quantize, dequantize, fp32 matmul),
               timed as the CPU baseline

Pinning status of each function (what independent check fixes it) is listed in each module's
docstring; `tests/test_oracle_*.py` hold those checks.
"""

SPEC_VERSION = "mq-oracle-1"
