"""Build libmq.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python comfy-quant-bench_amd/build.py            # -> comfy-quant-bench_amd/kitchen_amd/libmq.so

The library is written for gfx950 only. Every HIP source is compiled with packed fp32
instructions disabled (target feature -packed-fp32-ops) and with floating-point contraction off:
the rotate+quantize kernel must reproduce the reference's rounding order, and every fused
multiply-add the kernels want is written explicitly.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "kitchen_amd", "libmq.so")
SOURCES = ["mq_abi.hip", "mq_rotquant.hip", "mq_rotquant_f16.hip", "mq_rotquant_f32.hip", "mq_swiglu.hip",
           "mq_swiglu_f16.hip", "mq_swiglu_eager.hip", "mq_swiglu_eager_f16.hip",
           "mq_codebook.hip", "mq_wquant.hip", "mq_gemv.hip", "mq_gemm.hip", "mq_gemm_wide.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    if os.path.exists(path):
        return path
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-function",
    ]


def _compile(src: str, build_dir: str, verbose: bool) -> str:
    obj = os.path.join(build_dir, src.replace(".hip", ".o"))
    cmd = [hipcc(), *flags(), "-I", os.path.join(build_dir, "gen"), "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
    noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if noise and verbose:
        print("\n".join(noise), file=sys.stderr)
    return obj


def build(verbose: bool = False) -> str:
    """Compile every source (in parallel) and link libmq.so; returns its path. Always recompiles."""
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(os.path.join(build_dir, "gen"), exist_ok=True)
    # generated constant tables: correctly rounded fp32 silu of the bf16 and fp16 gates (SwiGLU prologue)
    subprocess.run([sys.executable, os.path.join(CSRC, "gen_silu_table.py"),
                    os.path.join(build_dir, "gen", "mq_silu_table.h"),
                    os.path.join(build_dir, "gen", "mq_silu_f16_table.h")], check=True)
    workers = max(1, min(len(SOURCES), os.cpu_count() or 1))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(lambda src: _compile(src, build_dir, verbose), SOURCES))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    # a kernel whose host-side stub was dropped leaves an undefined mq:: symbol behind
    undef = subprocess.run(["nm", "-D", "--undefined-only", tmp], capture_output=True, text=True).stdout
    missing = [ln.split()[-1] for ln in undef.splitlines() if "_ZN2mq" in ln]
    if missing:
        raise RuntimeError("libmq.so has undefined library symbols: " + ", ".join(missing[:4]))
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
