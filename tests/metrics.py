"""Parity metrics used by the tests and the benchmark.

snr_db follows the reference's parity harness (tools/stems-parity.cpp:36):
SNR = 10 log10(sum ref^2 / sum (out - ref)^2). rel_err is the elementwise bound of the fp32 ops:
max |a - b| / max(|b|, tau) with tau = 1e-6 * rms(b), so values near zero are judged against
the tensor's scale instead of their own.
"""
import numpy as np


def snr_db(out, ref):
    out = np.asarray(out, dtype=np.complex128 if np.iscomplexobj(out) or np.iscomplexobj(ref) else np.float64)
    ref = np.asarray(ref, dtype=out.dtype)
    num = float(np.sum(np.abs(ref) ** 2))
    den = float(np.sum(np.abs(out - ref) ** 2))
    if den == 0.0:
        return float("inf")
    return 10.0 * np.log10(num / den)


def rel_err(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    tau = 1e-6 * float(np.sqrt(np.mean(b * b))) if b.size else 0.0
    den = np.maximum(np.abs(b), max(tau, 1e-300))
    return float(np.max(np.abs(a - b) / den)) if a.size else 0.0
