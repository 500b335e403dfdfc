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


def fp32_rounding_ratio(got, ref):
    """Largest elementwise ``|got - ref| / (2^-24 |ref| + 1e-13 RMS(column))``
    of fp32 values ``got`` against fp64 ``ref``: at most 1 when each value of
    ``got`` is ``ref`` rounded once to fp32 (half an ulp, 2^-24 relative) after
    fp64 arithmetic (the second term covers fp64 rounding where a value cancels
    far below its column's scale)."""
    got = np.asarray(got, dtype=np.float64).reshape(ref.shape[0], -1)
    ref = np.asarray(ref, dtype=np.float64).reshape(ref.shape[0], -1)
    rms = np.sqrt(np.mean(ref * ref, axis=0))
    bound = 2.0 ** -24 * np.abs(ref) + 1e-13 * np.where(rms > 0, rms, 1.0)
    return float(np.max(np.abs(got - ref) / bound)) if ref.size else 0.0


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


def rotation(seed):
    """A random proper rotation (unit quaternion)."""
    q = np.random.default_rng(seed).normal(size=4)
    q /= np.linalg.norm(q)
    a, b, c, d = q
    return np.array([[a * a + b * b - c * c - d * d, 2 * (b * c - a * d), 2 * (b * d + a * c)],
                     [2 * (b * c + a * d), a * a - b * b + c * c - d * d, 2 * (c * d - a * b)],
                     [2 * (b * d - a * c), 2 * (c * d + a * b), a * a - b * b - c * c + d * d]])


def wigner_real(R, L):
    """Real-basis D^L(R) with Y_L(R u) = D^L Y_L(u), least squares over random directions."""
    u = np.random.default_rng(3).normal(size=(400, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    import oracle

    y0 = oracle.real_sph_table(u, L)[0][:, L * L:(L + 1) ** 2]
    y1 = oracle.real_sph_table(u @ R.T, L)[0][:, L * L:(L + 1) ** 2]
    D, *_ = np.linalg.lstsq(y0, y1, rcond=None)
    return D.T
