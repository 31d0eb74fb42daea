"""The per-row scale arithmetic of the rotate+quantize kernel, checked on the CPU.

The kernel (comfy-quant-bench_amd/csrc/mq_rotquant_kernel.h) forms s = max(absmax / L, 1e-10)
without a division (div_limit: q0 = RN(am c), c = RN(1/L), one fma for the exact residual, one fma
for the correction) and 1/s from an approximate reciprocal refined by one Newton step
(recip_row). The quantizer this follows (tools/activation_balance.py:65-71) divides; these tests
pin the division-free forms to it:

* div_limit equals the IEEE quotient am / L, after the max with 1e-10, for EVERY non-negative
  float am (2^31 bit patterns, +inf included), for L = 127 (int8 codes) and L = 7 (int4 codes);
* recip_row, started from any reciprocal within 8 ulps, ends within 2^-23 relative of 1/s over a
  sweep of s in [1e-10, 2^127], the bound the kernel's near-tie window assumes.

Both run as a small C program (gcc, OpenMP over the host's cores) with the same fp32 operations
the kernel issues (fmaf is the fused multiply-add, contraction is off).
"""
import os
import shutil
import subprocess

import pytest

C_SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t b) { float x; memcpy(&x, &b, 4); return x; }
static uint32_t u_of(float x) { uint32_t b; memcpy(&b, &x, 4); return b; }

/* device: div_limit<L> */
static float div_limit(float am, float L) {
    const float c = 1.0f / L;
    const float q0 = am * c;
    const float e = fmaf(-q0, L, am);
    const float q1 = fmaf(e, c, q0);
    return isinf(am) ? am : q1;
}

/* device: recip_row, with the first approximation r0 given */
static float recip_refine(float s, float r0) {
    const float e = fmaf(-s, r0, 1.0f);
    return fmaf(e, r0, r0);
}

int main(void) {
    const float Ls[2] = {127.0f, 7.0f};
    unsigned long long bad_div = 0, bad_rcp = 0;
    for (int li = 0; li < 2; ++li) {
        const float L = Ls[li];
        unsigned long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static, 1 << 20)
        for (long long b = 0; b <= 0x7f800000LL; ++b) {
            const float am = f_of((uint32_t)b);
            const float want = fmaxf(am / L, 1e-10f);
            const float got = fmaxf(div_limit(am, L), 1e-10f);
            if (u_of(want) != u_of(got)) ++bad;
        }
        printf("div_limit L=%g mismatches %llu\n", L, bad);
        bad_div += bad;
    }
    /* every 64th float from 1e-10 to 2^127, starting points up to 8 ulps away from RN(1/s) */
    const uint32_t lo = u_of(1e-10f), hi = u_of(0x1p127f);
    unsigned long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static, 1 << 16)
    for (long long b = lo; b <= hi; b += 64) {
        const float s = f_of((uint32_t)b);
        const uint32_t rn = u_of(1.0f / s);
        for (int k = -8; k <= 8; ++k) {
            const float r = recip_refine(s, f_of(rn + k));
            const double exact = 1.0 / (double)s;
            const double rel = fabs((double)r - exact) / exact;
            if (!(rel <= 0x1p-23)) ++bad;
        }
    }
    printf("recip_row bound violations %llu\n", bad);
    bad_rcp += bad;
    return bad_div == 0 && bad_rcp == 0 ? 0 : 1;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_scale_arithmetic_exhaustive(tmp_path):
    src = tmp_path / "scale_check.c"
    exe = tmp_path / "scale_check"
    src.write_text(C_SRC)
    subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", "-fopenmp", str(src), "-o", str(exe), "-lm"],
                   check=True)
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", str(os.cpu_count() or 1))
    res = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=900)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "div_limit L=127 mismatches 0" in res.stdout
    assert "div_limit L=7 mismatches 0" in res.stdout
    assert "recip_row bound violations 0" in res.stdout
