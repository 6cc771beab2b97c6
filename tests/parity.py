"""Tolerance checks of the GPU parity tests, and a record of the errors
they reach.

The bar (the benchmark contract): f32 KV max-abs <= 1e-5; f16 / bf16 / E4M3
KV with f32 accumulation max-abs <= 2e-3, and every element also within
2e-3 + 1e-3 * |ref| (implied by the first; kept so a relaxed first bound could
never pass silently).  Each call records (test id, label, max-abs, max-rel,
elements); conftest prints the table at the end of the session and writes
it as JSON lines to $TITAN_PARITY_LOG when that is set.
"""
import os

import numpy as np

RECORDS = []

ABS_16 = 2e-3
REL_16 = 1e-3
ABS_F32 = 1e-5


def _record(what, gpu, ref):
    d = np.abs(gpu - ref)
    max_abs = float(d.max()) if d.size else 0.0
    nz = np.abs(ref) > 1e-6
    max_rel = float((d[nz] / np.abs(ref[nz])).max()) if nz.any() else 0.0
    test = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" (")[0]
    RECORDS.append({"test": test, "what": what, "max_abs": max_abs, "max_rel": max_rel,
                    "n": int(d.size)})
    return d, max_abs


def check_close(gpu, ref, f32=False, what="", stress=False):
    """`stress`: inputs deliberately far outside the contract's N(0,1) data
    (every E4M3 code, |V| up to ~20): only the per-element bound
    2e-3 + 1e-3 * |ref| applies there, since a 2e-3 absolute bar on outputs
    of magnitude ~20 would demand more than the 11-bit precision of the f16
    softmax weights."""
    gpu, ref = np.asarray(gpu, np.float64), np.asarray(ref, np.float64)
    assert gpu.shape == ref.shape, f"{what}: shape {gpu.shape} vs {ref.shape}"
    assert np.all(np.isfinite(gpu)), f"{what}: non-finite output"
    d, max_abs = _record(what + (" [stress]" if stress else ""), gpu, ref)
    if f32:
        assert max_abs <= ABS_F32, f"{what}: max abs err {max_abs}"
        return
    if not stress:
        assert max_abs <= ABS_16, f"{what}: max abs err {max_abs} at {np.argwhere(d > ABS_16)[:4]}"
    bad = d > ABS_16 + REL_16 * np.abs(ref)
    assert not bad.any(), f"{what}: max abs err {max_abs} at {np.argwhere(bad)[:4]}"
