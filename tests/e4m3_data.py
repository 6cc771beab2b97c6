"""E4M3 pool contents for the GPU tests (test infrastructure)."""
import numpy as np

from oracle import orc


def gauss_codes(rng, nb, bt, n_kv, hd, k_spread=1.0):
    """The contract's data, stored as E4M3 the way a quantiser stores it:
    K, V ~ N(0,1) (K times k_spread), one scale per (K or V, kv head) =
    max|x| / 448, codes = quantize(x / scale)."""
    x = rng.standard_normal((nb * bt, 2, n_kv, hd)).astype(np.float32)
    x[:, 0] *= k_spread
    ks = (np.abs(x[:, 0]).max(axis=(0, 2)) / 448.0).astype(np.float32)
    vs = (np.abs(x[:, 1]).max(axis=(0, 2)) / 448.0).astype(np.float32)
    codes = np.empty(x.shape, np.uint8)
    for h in range(n_kv):
        codes[:, 0, h] = orc.f32_to_e4m3(x[:, 0, h], ks[h])
        codes[:, 1, h] = orc.f32_to_e4m3(x[:, 1, h], vs[h])
    return codes.reshape(-1), ks, vs


def all_codes(rng, nb, bt, n_kv, hd):
    """Stress data: every code except NaN, uniform, with random scales, so
    the dequantised K/V span the whole E4M3 range (|x| up to ~22)."""
    codes = rng.integers(0, 256, nb * bt * 2 * n_kv * hd).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x3C             # no NaN codes in the pool
    ks = rng.uniform(0.002, 0.05, n_kv).astype(np.float32)
    vs = rng.uniform(0.002, 0.05, n_kv).astype(np.float32)
    return codes, ks, vs
