"""Shared helpers for the parity tests: tolerances from the benchmark definition."""
import numpy as np

RENDER_ATOL = 1e-4          # RGB / alpha / depth, absolute per channel
GRAD_RTOL = 1e-3            # gradients, relative ...
GRAD_ATOL = 1e-5            # ... with an absolute floor


def np_(t):
    if t is None:
        return None
    if hasattr(t, "detach"):
        return t.detach().cpu().numpy()
    return np.asarray(t)


def frac_close(a, b, atol, rtol=0.0):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    ok = np.abs(a - b) <= atol + rtol * np.abs(b)
    return float(ok.mean()) if ok.size else 1.0


def report(name, a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if a.size == 0:
        return f"{name}: empty"
    d = np.abs(a - b)
    return f"{name}: max|d|={d.max():.3e} mean|d|={d.mean():.3e} max|ref|={np.abs(b).max():.3e}"
