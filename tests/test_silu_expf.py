"""The fused SiLU's exponential against the reference's own: siluf
(kernel/qwen35_decoder.cpp:128) calls the host C library's expf, which is not
correctly rounded, so the kernels carry a restatement of its method
(ref_expf in csrc/qmm_common.h).  Here that very function, compiled for the
host, is compared with the C library's expf on all 2^32 float inputs, and
the oracle's silu * u with the expression the reference forms.  CPU only."""
import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest

from conftest import PKG_DIR

HARNESS = r"""
#include "qmm_common.h"
#include <cmath>
#include <cstdio>
#include <cstring>
int main() {
    long long bad = 0, finite = 0;
#pragma omp parallel for reduction(+ : bad, finite) schedule(dynamic, 1 << 16)
    for (long long i = 0; i < (1LL << 32); ++i) {
        const uint32_t u = (uint32_t)i;
        float x;
        std::memcpy(&x, &u, 4);
        const float a = bq::ref_expf(x), b = expf(x);
        uint32_t ua, ub;
        std::memcpy(&ua, &a, 4);
        std::memcpy(&ub, &b, 4);
        if (ua != ub && !(std::isnan(a) && std::isnan(b))) ++bad;
        if (std::isfinite(b) && b != 0.0f) ++finite;
    }
    std::printf("%lld %lld\n", bad, finite);
    return 0;
}
"""


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not present")
    d = tmp_path_factory.mktemp("expf")
    src, exe = d / "harness.hip", d / "harness"
    src.write_text(HARNESS)
    subprocess.run([hipcc, "-x", "hip", "--offload-host-only", "-O2", "-std=c++17", "-fopenmp",
                    "-ffp-contract=off", "-I", os.path.join(PKG_DIR, "csrc"), str(src), "-o", str(exe)],
                   check=True, capture_output=True)
    return str(exe)


def test_ref_expf_equals_the_c_library_expf_on_every_float(harness):
    r = subprocess.run([harness], check=True, capture_output=True, text=True, timeout=600)
    bad, finite = map(int, r.stdout.split())
    assert bad == 0
    # Every float whose exponential is a finite nonzero float went through
    # the table path (about 2.24e9 of them).
    assert finite > 2_200_000_000


def test_oracle_silu_mul_is_the_reference_expression(orc):
    """The oracle forms g / (1 + expf(-g)) * u with the C library's expf,
    in float, each operation rounded once."""
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    rng = np.random.default_rng(3)
    g = np.concatenate([rng.normal(0, 4, 2000), [0.0, -0.0, 88.7, -88.7, 104.0, -104.0, np.inf, -np.inf,
                                                 3e38, -3e38, 1e-40, -1e-40]]).astype(np.float32)
    u = rng.normal(0, 1, g.size).astype(np.float32)
    got = orc.silu_mul(g, u)
    want = np.array([np.float32(x) / (np.float32(1) + np.float32(libm.expf(-float(x)))) * np.float32(y)
                     for x, y in zip(g, u)], np.float32)
    both_nan = np.isnan(got) & np.isnan(want)
    assert np.array_equal(got.view(np.uint32)[~both_nan], want.view(np.uint32)[~both_nan])
