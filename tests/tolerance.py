"""Parity bar for floating-point GEMV results against the CPU oracle.

cosine(y, y_ref) >= 0.999999 over the whole output, and per row
|y_r - y_ref_r| <= 1e-4 * ||w_r||_2 * ||x||_2  (the Cauchy-Schwarz scale of
y_r; "max |err| <= 1e-4 x ||row||" of the path's target).
"""
import numpy as np

COS_MIN = 0.999999
ROW_REL = 1e-4


def cosine(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0.0 and nb == 0.0:
        return 1.0
    if na == 0.0 or nb == 0.0:
        return 0.0
    return float(np.dot(a, b) / (na * nb))


def check_gemv(y, y_ref, row_norms, x, what="") -> dict:
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    assert y.shape == y_ref.shape, what
    assert np.all(np.isfinite(y)), f"{what}: non-finite output"
    bound = ROW_REL * np.asarray(row_norms, dtype=np.float64) * float(np.linalg.norm(np.asarray(x, np.float64)))
    err = np.abs(y - y_ref)
    worst = int(np.argmax(err - bound)) if y.size else 0
    c = cosine(y, y_ref)
    stats = {"cosine": c, "max_abs_err": float(err.max()) if y.size else 0.0,
             "worst_row": worst}
    assert c >= COS_MIN, f"{what}: cosine {c:.9f} < {COS_MIN} ({stats})"
    assert np.all(err <= bound), (f"{what}: row {worst} err {err[worst]:.3e} > bound {bound[worst]:.3e}")
    return stats
