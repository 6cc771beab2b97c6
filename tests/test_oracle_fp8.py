"""Pins the oracle's FP8 E4M3 restatement (OCP E4M3FN, per-head f32 scales).

No reference kernel implements FP8 KV storage (the reference has the format
only in its design notes, openspec/archive/2026-08-28-fp8-kv-cache-quantization/
design.md:3-6), so the oracle is pinned against what fixes the format:
  * decode: all 256 codes against torch.float8_e4m3fn, an independent
    implementation of the same OCP format;
  * quantisation: a brute-force nearest-code search over the 253 finite
    non-negative codes with ties to the even mantissa, and torch's own
    round-to-nearest-even conversion for in-range values;
  * saturation (|x| >= 448 and +-inf -> +-448), NaN -> S.1111.111, signed zero;
  * scaling: code(x, s) == code(x / s in f32, 1).
"""
import numpy as np
import pytest
import torch

from oracle import orc


def table():
    return orc.e4m3_to_f32(np.arange(256, dtype=np.uint8))


def test_decode_matches_torch_all_codes():
    got = table()
    want = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.sum(nan) == 2                      # 0x7F and 0xFF
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))  # incl. -0
    assert np.nanmax(got) == 448.0 and np.nanmin(np.abs(got[got != 0])) == 2.0 ** -9


def brute(x):
    """Nearest finite non-negative code to |x| (ties: even code), with sign."""
    t = table()[:0x7F]                            # codes 0..0x7E, ascending values
    a = np.abs(np.float64(x))
    if a >= 448.0:
        c = 0x7E
    else:
        d = np.abs(t.astype(np.float64) - a)
        best = np.flatnonzero(d == d.min())
        c = int(best[0]) if len(best) == 1 else int(best[best % 2 == 0][0])
    return c | (0x80 if np.signbit(np.float32(x)) else 0)


def test_quantize_brute_force_and_ties():
    rng = np.random.default_rng(5)
    xs = np.concatenate([
        rng.standard_normal(3000) * 10.0 ** rng.uniform(-4, 2.8, 3000),
        rng.uniform(-2 ** -6, 2 ** -6, 500),            # subnormal range
        rng.uniform(440, 470, 100) * rng.choice([-1, 1], 100),
    ]).astype(np.float32)
    t = table()[:0x7F].astype(np.float64)
    mids = ((t[1:] + t[:-1]) / 2).astype(np.float32)   # exact midpoints: every tie
    xs = np.concatenate([xs, mids, -mids, t.astype(np.float32), [0.0, -0.0]]).astype(np.float32)
    got = orc.f32_to_e4m3(xs)
    want = np.array([brute(x) for x in xs], dtype=np.uint8)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (xs[bad[:5]], got[bad[:5]], want[bad[:5]])


def test_quantize_matches_torch_in_range():
    rng = np.random.default_rng(6)
    xs = (rng.standard_normal(20000) * 10.0 ** rng.uniform(-3.5, 2.6, 20000)).astype(np.float32)
    xs = xs[np.abs(xs) <= 448.0]
    want = torch.from_numpy(xs).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(orc.f32_to_e4m3(xs), want)


def test_saturation_nan_and_sign():
    x = np.array([448.0, 449.0, 464.0, 1e30, np.inf, -np.inf, -500.0, np.nan, -np.nan, -0.0,
                  2.0 ** -10, 2.0 ** -10 * 1.0001, -(2.0 ** -11)], dtype=np.float32)
    got = orc.f32_to_e4m3(x)
    assert list(got[:7]) == [0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE]
    assert got[7] & 0x7F == 0x7F and got[8] & 0x7F == 0x7F
    assert got[9] == 0x80
    assert got[10] == 0x00           # tie between 0 and 2^-9: even (zero)
    assert got[11] == 0x01
    assert got[12] == 0x80           # rounds to -0


@pytest.mark.parametrize("scale", [0.5, 0.0123, 3.7, 100.0])
def test_scale_is_a_division(scale):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(4000) * 50).astype(np.float32)
    y = (x / np.float32(scale)).astype(np.float32)
    assert np.array_equal(orc.f32_to_e4m3(x, scale), orc.f32_to_e4m3(y, 1.0))
    deq = orc.e4m3_to_f32(orc.f32_to_e4m3(x, scale), scale)
    assert np.array_equal(deq, (table()[orc.f32_to_e4m3(x, scale)] * np.float32(scale)).astype(np.float32))
    # relative error of the round trip is within half an E4M3 ulp where not saturated
    ok = np.abs(y) < 448.0
    big = ok & (np.abs(y) >= 2.0 ** -6)
    assert np.all(np.abs(deq[big] - x[big]) <= np.abs(x[big]) * 2.0 ** -4 + 1e-30)
