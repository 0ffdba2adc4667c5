"""The device code's three-instruction roundf: truncf(v + copysignf(pred(1/2), v))
equals roundf(v) (half away from zero) bit for bit for every one of the 2^32
float bit patterns (NaN in, NaN out).  The exact-mode kernels round every Q16
quantization (norm statistics, residual sums, activation grids) this way, so
their results are the oracle's roundf/llround results.  Checked exhaustively by
a small C program built here: IEEE single-precision addition with
round-to-nearest-even on the CPU, as on the GPU's VALU."""
import os
import shutil
import subprocess

import pytest

SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
int main(void) {
    uint64_t bad = 0;
    for (uint64_t u = 0; u <= 0xFFFFFFFFull; u++) {
        uint32_t b = (uint32_t)u, fb, rb;
        float v;
        memcpy(&v, &b, 4);
        volatile float c = copysignf(0x1.fffffep-2f, v);
        volatile float s = v + c;
        const float f = truncf(s), r = roundf(v);
        if (isnan(v)) { bad += !isnan(f); continue; }
        memcpy(&fb, &f, 4); memcpy(&rb, &r, 4);
        if (fb != rb && bad++ < 5) printf("v=%a fast=%a roundf=%a\n", v, f, r);
    }
    printf("%llu\n", (unsigned long long)bad);
    return bad != 0;
}
"""


def test_round_away_equals_roundf_for_every_float(tmp_path):
    if not shutil.which("gcc"):
        pytest.skip("gcc is not installed")
    c, exe = tmp_path / "r.c", tmp_path / "r"
    c.write_text(SRC)
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", str(c), "-o", str(exe), "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip().splitlines()[-1] == "0", r.stdout
