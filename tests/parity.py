"""The parity bar for the floating-point products, fixed before the first GPU run.

  NRMSE    = ||y - ref||_2 / ||ref||_2                         <= 1e-5
  max rel  = max_i |y_i - ref_i| / max(|ref_i|, FLOOR * RMS(ref))   <= 1e-4

The floor keeps the relative error defined where an output is near zero: the reference's own
product against its F64 reference shows a max relative error of 5.3e-2 on a real matrix while its
largest absolute error is 4.8e-6 (logs/gates/2026-11-01/174236-check.txt:72-73), and its comparator
falls back on an absolute floor for that reason (tests/host/numcmp.c:64-69). FLOOR = 1/16 of the
output's RMS; ref is the F64 closed form unless a test says otherwise.
"""
import numpy as np

NRMSE_TOL = 1e-5
REL_TOL = 1e-4
FLOOR = 1.0 / 16.0


def metrics(y, ref):
    y = np.asarray(y, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    diff = np.abs(y - ref)
    rms = float(np.sqrt(np.mean(ref * ref)))
    nrmse = float(np.sqrt(np.sum(diff * diff)) / max(np.sqrt(np.sum(ref * ref)), 1e-300))
    den = np.maximum(np.abs(ref), FLOOR * rms)
    max_rel = float(np.max(diff / np.maximum(den, 1e-300))) if diff.size else 0.0
    naive = diff / np.maximum(np.abs(ref), 1e-300)
    return {
        "nrmse": nrmse,
        "max_rel": max_rel,
        "max_abs": float(diff.max()) if diff.size else 0.0,
        "naive_over": int(np.sum(naive > REL_TOL)),
        "n": int(diff.size),
    }


def assert_parity(y, ref, what=""):
    m = metrics(y, ref)
    assert np.all(np.isfinite(np.asarray(y))), f"{what}: non-finite output"
    assert m["nrmse"] <= NRMSE_TOL and m["max_rel"] <= REL_TOL, f"{what}: {m}"
    return m
