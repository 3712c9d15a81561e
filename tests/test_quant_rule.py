"""The per-token int8 quantisation of the one-launch W8A8 decode step (decode_mk.hip quant_wave_i8) takes the quotient
as x * (1 / s) and falls back to the IEEE quotient x / s only where |t| + 0.5 lies within 1e-4 of an integer. This
pins the claim that the result always equals the reference's rule (tgemm.py:81-91: q = trunc(x / s + 0.5 sign) with
the correctly rounded fp32 quotient), in fp32 numpy arithmetic (IEEE, round to nearest): every bf16 value x against
scales s = amax / 127 drawn over the whole range the decoder meets, with |x| <= amax. (Without the fallback the
multiply form agreed too on 4,000 random scales: bf16 quotients rarely fall within an ulp of a half-integer; the
fallback makes the equality hold by construction rather than by that observation.)"""
import numpy as np


def _bf16_values():
    u = np.arange(1 << 16, dtype=np.uint32) << 16
    v = u.view(np.float32)
    return v[np.isfinite(v)]


def _q_exact(x, s):
    t = (x / s).astype(np.float32)
    return np.trunc(t + np.where(t >= 0, np.float32(0.5), np.float32(-0.5))).astype(np.int32)


def _q_fast(x, s):
    rs = np.float32(1.0) / s
    t = (x * rs).astype(np.float32)
    u = (np.abs(t) + np.float32(0.5)).astype(np.float32)
    fr = (u - np.trunc(u)).astype(np.float32)
    near = (fr < np.float32(1e-4)) | (fr > np.float32(1.0) - np.float32(1e-4))
    t = np.where(near, (x / s).astype(np.float32), t)
    return np.trunc(t + np.where(t >= 0, np.float32(0.5), np.float32(-0.5))).astype(np.int32)


def test_fast_quotient_quantisation_equals_ieee_rule():
    xs = _bf16_values()
    rng = np.random.default_rng(0)
    amaxes = np.concatenate([np.float32(10.0) ** rng.uniform(-5, 3, 300).astype(np.float32),
                             np.array([1e-5, 1.0, 127.0, 0.5, 3.0], dtype=np.float32)]).astype(np.float32)
    checked = 0
    for amax in amaxes:
        s = np.float32(max(amax, np.float32(1e-5)) / np.float32(127.0))
        x = xs[np.abs(xs) <= amax]
        x = np.concatenate([x, np.float32([amax, -amax])]).astype(np.float32)
        assert np.array_equal(_q_fast(x, s), _q_exact(x, s)), amax
        checked += x.size
    assert checked > 1_000_000
