"""CPU check of the erf GELU epilogue's arithmetic (csrc/common.h gelu_erf): the polynomial coefficients are read from
the source and checked against math.erfc, and the fp32 evaluation of the whole formula is checked against the same
formula with a correctly rounded erf on every bf16 input in [-12, 12] (the epilogue's inputs are bf16 values: the
GEMM output is rounded before the activation). A mistyped coefficient or a changed operation order fails here
without a GPU; the kernel itself is compared with torch on the GPU (test_gpu_kernels)."""
import math
import os
import re

import numpy as np
import torch

SRC = os.path.join(os.path.dirname(__file__), "..", "strix-halo-maxx_amd", "csrc", "common.h")


def _coefficients():
    body = open(SRC).read()
    body = body[body.index("float gelu_erf(float x)"):]
    body = body[:body.index("\n}")]
    first = float(re.search(r"float p = ([-0-9.]+)f;", body).group(1))
    rest = [float(v) for v in re.findall(r"p = __builtin_fmaf\(p, t, ([-0-9.]+)f\);", body)]
    return [first] + rest  # Horner order, highest degree first


def test_erfc_fit_fractional_error():
    """erfc(a) = t exp(-a^2 + P(t)), t = 1 / (1 + a / 2): fractional error below 1.2e-7 for a in [0, 9] (exact
    arithmetic), as the fit promises; a wrong or missing coefficient moves it by orders of magnitude."""
    c = _coefficients()
    assert len(c) == 10
    worst = 0.0
    for a in np.linspace(0.0, 9.0, 20001):
        t = 1.0 / (1.0 + 0.5 * a)
        p = 0.0
        for ci in c:
            p = p * t + ci
        approx = t * math.exp(-a * a + p)
        worst = max(worst, abs(approx - math.erfc(a)) / math.erfc(a))
    assert worst < 1.3e-7, worst


def test_gelu_erf_fp32_formula_every_bf16_input():
    """The fp32 evaluation (fused multiply-adds in Horner order, rcp and exp2 exact here) gives, after the bf16
    rounding, the same value as 0.5 x (1 + erf(x / sqrt 2)) with erf correctly rounded to fp32, for every bf16 x in
    [-12, 12]."""
    f = np.float32
    c = [f(v) for v in _coefficients()]

    def fma(a, b, d):
        return f(float(a) * float(b) + float(d))

    def kernel(x):
        z = f(x * f(0.7071067811865476))
        a = f(abs(z))
        t = f(1.0 / float(fma(f(0.5), a, f(1))))
        p = c[0]
        for ci in c[1:]:
            p = fma(p, t, ci)
        e = f(f(1) - f(t * f(2.0 ** float(f(f(p - f(a * a)) * f(1.4426950408889634))))))
        return f(f(f(0.5) * x) * f(f(1) + (-e if z < 0 else e)))

    def exact(x):
        z = f(x * f(0.7071067811865476))
        return f(f(f(0.5) * x) * f(f(1) + f(math.erf(float(z)))))

    allv = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    xs = allv[torch.isfinite(allv) & (allv.abs() <= 12)].unique().numpy()
    got = torch.tensor([float(kernel(f(x))) for x in xs]).to(torch.bfloat16)
    want = torch.tensor([float(exact(f(x))) for x in xs]).to(torch.bfloat16)
    assert len(xs) == 33409
    assert torch.equal(got, want)
