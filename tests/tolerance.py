"""Parity metrics.  Features: max_i |a_i - b_i| / max(|b_i|, rms(b)); the
bars are 1e-4 (f32) and 1e-2 (bf16 operands, f32 accumulate)."""
import numpy as np

TOL_F32 = 1e-4
TOL_BF16 = 1e-2


def rel_err(actual, expected) -> float:
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    if b.size == 0:
        return 0.0
    rms = float(np.sqrt(np.mean(b * b)))
    denom = np.maximum(np.abs(b), rms if rms > 0 else 1.0)
    return float(np.max(np.abs(a - b) / denom))


def assert_close(actual, expected, tol, what=""):
    e = rel_err(actual, expected)
    assert e <= tol, f"{what}: rel err {e:.3e} > {tol:.1e}"
    return e
