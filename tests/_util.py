"""Shared helpers for the parity tests (not collected)."""

import numpy as np

# Tolerances of the north star: per-feature-column relative error
# max|gpu - oracle| / RMS(oracle column); fp32 results are compared with the
# fp64 oracle evaluated on the same fp32-rounded inputs.
TOL = {"f64": 1e-12, "f32": 2e-5}


def column_rel_error(got, ref):
    got = np.asarray(got, dtype=np.float64).reshape(ref.shape[0], -1)
    ref = np.asarray(ref, dtype=np.float64).reshape(ref.shape[0], -1)
    rms = np.sqrt(np.mean(ref * ref, axis=0))
    scale = np.where(rms > 0, rms, 1.0)
    err = np.max(np.abs(got - ref), axis=0) / scale
    return float(err.max()) if err.size else 0.0


def rounded_inputs(inp, dtype):
    """Inputs as the device sees them: float arrays rounded to the compute dtype."""
    if dtype == "f64":
        return inp
    out = dict(inp)
    for k in ("edge_vectors", "node_features", "radial_mix"):
        if inp.get(k) is not None:
            out[k] = np.asarray(inp[k], dtype=np.float32).astype(np.float64)
    return out


def flush(msg):
    print(msg, flush=True)
