"""Time the oracle's restatements against the reference's own CPU code.

Test infrastructure, run in the development container where ``make -C oracle
ref`` has compiled the reference's CPU core (``_ref/libye3t_ref.so``) and its
schedule runtime (``_ref/ye3t_factorized_ref.so``) from their sources.  Both
sides run on identical inputs, on one thread, best of ``repeats`` runs; the
ratio restatement/reference says how far the ``cpu_baseline`` figure (which
times the restatement on the GPU box's host cores)
sits from the reference's own CPU speed.

    python -m oracle.calibrate [output.md]

writes ``calibration: op=NAME ratio=R restatement_s=T reference_s=T`` lines
that ``bench.py`` copies into its ``cpu_baseline`` record.
"""

import os
import platform
import sys
import time

import numpy as np

import oracle


def _best(fn, repeats=5):
    best = float("inf")
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
    return best


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _factorized_ref():
    import importlib.util

    import torch  # noqa: F401  (the module links against libtorch)

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_ref", "ye3t_factorized_ref.so")
    if not os.path.exists(path):
        return None
    spec = importlib.util.spec_from_file_location("ye3t_factorized_ref", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def measure():
    if oracle.ref_lib() is None:
        raise SystemExit("oracle/_ref/libye3t_ref.so is not built (make -C oracle ref)")
    oracle.set_threads(1)
    rng = np.random.default_rng(0)
    rows = []

    # ChebExpCos radial table, n_max 12 (config-5 width), 200 000 edges
    E = 200_000
    r = rng.uniform(0.8, 5.5, E)
    rc = np.full(E, 5.5)
    lam = np.full(E, 5.0)
    rows.append(("cheb_exp_cos_radial_table_with_derivative", f"E={E} n_max=12",
                 _best(lambda: oracle.radial_table(r, rc, lam, 12)),
                 _best(lambda: oracle.radial_table(r, rc, lam, 12, use_reference=True))))

    # real SH table with Cartesian gradients, l_max 6, 100 000 edges
    vec = rng.normal(size=(100_000, 3))
    rows.append(("real_spherical_harmonics_table_with_derivative", "E=100000 l_max=6",
                 _best(lambda: oracle.real_sph_table(vec, 6)),
                 _best(lambda: oracle.real_sph_table(vec, 6, use_reference=True))))

    # density scatter, config-4 width (256 channels), 1.2 M edges onto 50 000 atoms
    E, C, N = 1_200_000, 256, 50_000
    ev = rng.normal(size=(E, C))
    centers = np.repeat(np.arange(N), E // N)
    rows.append(("density_accumulate", f"E={E} C={C} N={N}",
                 _best(lambda: oracle.density_accumulate(ev, centers, N), 3),
                 _best(lambda: oracle.density_accumulate(ev, centers, N, use_reference=True), 3)))
    del ev

    # Sym^4(V_3) -> Lambda=4 monomials over 20 000 rows
    from ye3t_amd.core.symmetric_power import real_monomial_entries

    entries = real_monomial_entries(4, 3, 4, 0)
    outs = np.array([e[0] for e in entries])
    order = np.argsort(outs, kind="stable")
    counts = np.array([entries[i][1] for i in order], dtype=np.int64)
    vals = np.array([entries[i][2] for i in order])
    offs = np.searchsorted(outs[order], np.arange(2 * 4 + 2))
    x = rng.normal(size=(20_000, 7))
    rows.append(("symmetric_power_monomial", f"Sym^4(V_3)->4 B=20000 terms={len(vals)}",
                 _best(lambda: oracle.symmetric_power_monomial(x, counts, offs, vals)),
                 _best(lambda: oracle.symmetric_power_monomial(x, counts, offs, vals, use_reference=True))))

    # factorized schedule evaluation (factorized_runtime.cpp), a rank-3 L=2 schedule
    ref = _factorized_ref()
    if ref is not None:
        import torch

        from ye3t_amd.core.couplings import generate_factorized_coefficient_schedules_by_L

        torch.set_num_threads(1)
        s = generate_factorized_coefficient_schedules_by_L((1, 2, 3), (2, 3, 3))[2]
        flat = s.flat_arrays()
        bv = rng.normal(size=(20_000, s.basis_count, s.block_count, flat["max_block_m_dim"]))
        args = [torch.from_numpy(a) for a in (bv, flat["component_offsets"], flat["component_label_index"],
                                              flat["block_m_indices"], flat["coeffs"])]
        rows.append(("evaluate_factorized_schedule_cpu", f"(1,2,3),(2,3,3) L=2 B=20000 terms={s.term_count}",
                     _best(lambda: oracle.evaluate_componentwise(bv, flat)),
                     _best(lambda: ref.evaluate_factorized_schedule_cpu(*args, s.component_count, False))))
    oracle.set_threads(oracle.max_threads())
    return rows


def write(rows, path):
    lines = ["# CPU baseline calibration: oracle restatement vs the reference's own CPU code", "",
             "Command: `make -C oracle ref && python -m oracle.calibrate profiles/cpu_baseline_calibration.md`",
             "(development container; the reference's sources compiled with g++ -O2, the oracle with gcc -O3).", "",
             f"Host: {_cpu_model()}, {os.cpu_count()} logical CPUs; both sides on 1 thread "
             "(oracle OpenMP and torch intra-op threads set to 1), best of 3-5 runs.", "",
             "| operation | inputs | restatement s | reference s | ratio |", "|---|---|---|---|---|"]
    for op, what, t_o, t_r in rows:
        lines.append(f"| {op} | {what} | {t_o:.4f} | {t_r:.4f} | {t_o / t_r:.2f} |")
    lines += ["", "A ratio below 1 means the restatement is faster than the reference on the same "
              "work; the cpu_baseline line reports the restatement's rate.", ""]
    for op, what, t_o, t_r in rows:
        lines.append(f"calibration: op={op} ratio={t_o / t_r:.3f} restatement_s={t_o:.4f} "
                     f"reference_s={t_r:.4f} cores=1")
    with open(path, "w") as fh:
        fh.write("\n".join(lines) + "\n")


if __name__ == "__main__":
    out = sys.argv[1] if len(sys.argv) > 1 else os.path.join(os.path.dirname(__file__), "..", "profiles",
                                                             "cpu_baseline_calibration.md")
    write(measure(), out)
    print(open(out).read())
