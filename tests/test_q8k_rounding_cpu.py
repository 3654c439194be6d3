"""The device Q8K code's rounding (fuel_amd/csrc/q8.hpp, q8k_code) against
f32::round of BlockQ8K::from_float (fuel-quantized/src/k_quants.rs:2253),
over every float the code can see.

The kernel rounds half away from zero as trunc(v + copysign(0.49999997, v))
(0.49999997 is the float below 0.5; the conversion after the clamps
truncates).  The argument v = iscale * x is within 128 (1 + 2^-23) in
magnitude unless it is infinite or NaN, which pass through the sum unchanged,
so checking all 2.25e9 floats with |v| <= 129 against C's roundf (half away
from zero, like Rust's f32::round) covers every finite case.  Plain 0.5 would
fail it: 0.49999997 + 0.5 rounds up to 1.0 in the addition.
"""
import subprocess

import pytest

SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
int main(int argc, char** argv) {
    const float c = argc > 1 ? 0.5f : 0.49999997f;
    unsigned long long bad = 0, n = 0;
    for (uint64_t u = 0; u <= 0xFFFFFFFFull; u++) {
        uint32_t b = (uint32_t)u;
        float v;
        memcpy(&v, &b, 4);
        if (!(fabsf(v) <= 129.0f)) continue;
        n++;
        volatile float s = v + copysignf(c, v);
        if (truncf(s) != roundf(v)) {
            bad++;
            if (argc > 1) break;  /* (the 0.5 check stops at its first miss) */
        }
    }
    printf("%llu %llu\n", n, bad);
    return 0;
}
"""


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    d = tmp_path_factory.mktemp("q8k_round")
    (d / "r.c").write_text(SRC)
    exe = d / "r"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(d / "r.c"), "-lm"], check=True)
    return exe


def test_q8k_rounding_exhaustive(checker):
    n, bad = map(int, subprocess.run([str(checker)], capture_output=True, text=True, check=True).stdout.split())
    assert n == 2248278018
    assert bad == 0


def test_q8k_rounding_half_would_fail(checker):
    # the same check with 0.5 itself finds the values it rounds up wrongly
    n, bad = map(int, subprocess.run([str(checker), "half"], capture_output=True, text=True, check=True).stdout.split())
    assert bad > 0
