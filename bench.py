"""Benchmark of the ACE hot path on one MI355X.

A step = stage 1 (fused density) + stage 2 (B-feature product) over the whole
synthetic workload, inputs resident in HBM.  Default workload: configuration 4
(50 000 nodes x 16 channels, 24 neighbours, l<=3, nu=3, L in {0,1,2}, fp32),
the configuration BASELINE.json's HBM target is stated on.

Prints ONE JSON line (rank 0).  Per-kernel durations come from HIP events
recorded on the stream the kernels run on (torch's current stream).
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def algorithmic_bytes(cfg, plan, s):
    """Compulsory traffic per launch as the survey's measurement contract defines
    it: every input read once, every output written once, at the
    configuration's storage element size ``s`` (4 for fp32 configurations,
    also for the density), with 4-byte CSR offsets and neighbour indices:

      stage 1: E (3 s + 4) + (N + 1) 4 + [E 4 species | N C_in s node features] + N a_row s
      stage 2: samples a_width s + samples F s
    """
    d = cfg.density
    N, K = d.atom_count, d.neighbors_per_atom
    E = N * K
    a_row = d.channel_count * d.radial_rows * (d.l_max + 1) ** 2
    stage1 = E * (3 * s + 4) + (N + 1) * 4 + N * a_row * s
    if d.node_channels:
        stage1 += N * d.node_channels * s
    if d.species_count:
        stage1 += E * 4
    samples = cfg.samples()
    stage2 = samples * plan.a_width * s + samples * plan.feature_count * s
    return stage1, stage2


def as_built_bytes(cfg, plan, elem, a_elem):
    """The same compulsory traffic for the buffers as this build lays them out:
    int64 CSR offsets and neighbour indices (the reference's index type), the
    radial-mix table, and the density at its stored element size ``a_elem``."""
    d = cfg.density
    N, K = d.atom_count, d.neighbors_per_atom
    E = N * K
    a_row = d.channel_count * d.radial_rows * (d.l_max + 1) ** 2
    stage1 = E * (3 * elem + 8) + (N + 1) * 8 + N * a_row * a_elem
    if d.node_channels:
        stage1 += N * d.node_channels * elem + d.node_channels * (d.n_max + 1) * elem
    if d.species_count:
        stage1 += N * 4
    samples = cfg.samples()
    stage2 = samples * plan.a_width * a_elem + samples * plan.feature_count * elem
    return stage1, stage2


def counter_traffic(kernel, workload, dtype):
    """HBM bytes per launch from the committed rocprofv3 PMC summaries.

    Each ``profiles/*.md`` summary carries ``traffic:`` lines with the mean
    FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of one kernel on one workload,
    and the factors that map each counter onto the bytes of a plain copy kernel
    of known size.  Returns ``(bytes, source)`` or ``(None, None)``.
    """
    import glob

    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        with open(path) as fh:
            for line in fh:
                if not line.startswith("traffic:"):
                    continue
                kv = dict(item.split("=", 1) for item in line[len("traffic:"):].split())
                if kv.get("kernel") == kernel and kv.get("workload") == workload and kv.get("dtype") == dtype:
                    kib = float(kv["fetch_kib"]) * float(kv["fetch_scale"]) + \
                        float(kv["write_kib"]) * float(kv["write_scale"])
                    return kib * 1024.0, os.path.relpath(path, ROOT)
    return None, None


def host_facts():
    """CPU model, logical CPUs, the CPUs this process may run on and OMP_NUM_THREADS."""
    model = None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity_cpus": affinity,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cpu_calibration():
    """Restatement-over-reference time ratios measured in the development
    container (the reference's own CPU core compiled from its sources, which
    only that container can build), from the committed summary's
    ``calibration:`` lines."""
    path = os.path.join(ROOT, "profiles", "cpu_baseline_calibration.md")
    out = {}
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        for line in fh:
            if line.startswith("calibration:"):
                kv = dict(item.split("=", 1) for item in line[len("calibration:"):].split())
                out[kv.pop("op")] = {k: (float(v) if k.endswith(("ratio", "_s")) else v) for k, v in kv.items()}
    return {"source": os.path.relpath(path, ROOT), "ops": out} if out else None


def cpu_baseline(cfg, pipe, target_seconds=10.0):
    """The C oracle (restatement of the reference CPU path) on a bounded sample."""
    import oracle

    threads = oracle.max_threads()

    def run(atoms):
        sub = type(cfg.density)(**{**cfg.density.__dict__, "atom_count": atoms})
        inp = sub.generate()
        t0 = time.perf_counter()
        A = oracle.ace_density(inp)
        t1 = time.perf_counter()
        oracle.ace_product_flat(A.reshape(-1, pipe.plan.a_width), pipe.plan.flat_arrays())
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1

    pipe.plan.flat_arrays()  # table build is host compile work, not timed
    probe = 200
    s1, s2 = run(probe)
    atoms = int(min(cfg.density.atom_count, max(probe, probe * target_seconds / max(s1 + s2, 1e-6))))
    s1, s2 = run(atoms)
    per_atom_features = cfg.samples() // cfg.density.atom_count * pipe.plan.feature_count
    total = s1 + s2
    out = {"value": atoms * per_atom_features / total, "unit": "B-features/s", "cores": threads,
           "kind": "port", "atoms_per_s": atoms / total,
           "sample": f"{atoms} atoms of the same workload; stage1 {s1:.2f}s (serial edge loop, as the reference), "
                     f"stage2 {s2:.2f}s (OpenMP over samples, {threads} threads)"}
    out.update(host_facts())
    out["calibration"] = cpu_calibration()
    return out


def warm_up(fn, warmup, min_seconds):
    """Run ``fn`` at least ``warmup`` times and for at least ``min_seconds``
    (the GPU reaches its steady clocks only after ~0.1 s of work); returns
    ``(calls, seconds)`` actually spent."""
    import torch

    t0 = time.perf_counter()
    done = 0
    while done < warmup or time.perf_counter() - t0 < min_seconds:
        fn()
        done += 1
        if done % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return done, time.perf_counter() - t0


MIN_WARMUP_S = 0.5


def _time_kernel(fn, steps, warmup, min_warmup_s=MIN_WARMUP_S):
    """Mean wall time per call of ``fn`` (device-resident inputs, K back-to-back
    calls), after ``warmup`` calls and at least ``min_warmup_s`` of them (the
    GPU's clocks ramp up over the first ~0.1 s of work)."""
    import torch

    warm_up(fn, warmup, min_warmup_s)
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


class _NoPlan:
    """Stand-in plan for the stage-1 byte count (stage 2's share is unused)."""
    a_width = 0
    feature_count = 0


def bench_op(args, cfg):
    """One widened op on the configuration's shapes (see ``--op``)."""
    import numpy as np
    import torch

    from ye3t_amd.ace.pipeline import ACEPipeline, to_device_inputs
    from ye3t_amd.ace.program import program_stats
    from ye3t_amd.runtime import density_accumulate_adjoint, native

    d = cfg.density
    dtype = args.dtype or cfg.dtypes[0]
    accumulate = args.accumulate or (cfg.accumulate if dtype == "f32" else None) or dtype
    density = args.density or (cfg.density_dtype if dtype == "f32" and accumulate == cfg.accumulate else None) or accumulate
    workload = f"config{cfg.config_id}-{cfg.name}"
    line = {"op": args.op, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "data": "synthetic",
            "config": {"workload": workload}}
    if args.op == "linear_readout":
        pipe = ACEPipeline(cfg.feature_spec, dtype, args.max_slots, kernel=args.kernel, accumulate=accumulate,
                           density=density)
        A = pipe.density(to_device_inputs(cfg.density.generate(), dtype, "cuda"))
        rows = A.reshape(-1, pipe.plan.a_width)
        S = int(rows.shape[0])
        w = torch.as_tensor(np.random.default_rng(3).normal(size=pipe.feature_count), device="cuda")
        out = torch.empty((S,), dtype=torch.float64 if dtype == "f64" else torch.float32, device="cuda")
        pipe.linear(rows, w, 0.5, out=out)  # compiles and attaches the fused kernel; validates the arguments
        if pipe.last_linear_backend == "fused_generated":
            wk = w.to(torch.float64 if accumulate == "f64" else torch.float32).contiguous()
            t = _time_kernel(lambda: pipe.handle.linear(rows, wk, 0.5, out=out), args.steps, args.warmup)
        else:
            t = _time_kernel(lambda: pipe.linear(rows, w, 0.5, out=out), args.steps, args.warmup)
        nbytes = S * pipe.plan.a_width * rows.element_size() + S * out.element_size() + \
            pipe.feature_count * (8 if accumulate == "f64" else 4)
        st = program_stats(pipe.program)
        flops = S * (st["factor_reads"] + st["terms"] + 2 * pipe.feature_count)
        line.update({
            "metric": "readout samples/s", "value": S / t, "unit": "samples/s", "higher_is_better": True,
            "us_per_call": t * 1e6, "dtype": accumulate, "storage_dtype": dtype, "backend": pipe.last_linear_backend,
            "roofline": {"bound": "hbm", "achieved": nbytes / t / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": nbytes},
            "fp64_arithmetic": {"algorithmic_flops": flops, "achieved_tflops": flops / t / 1e12,
                                "peak_tflops": 78.6, "frac": flops / t / 1e12 / 78.6},
            "samples": S, "features_per_sample": pipe.feature_count})
        line["config"].update({"samples": S, "features": pipe.feature_count})
    elif args.op == "product_adjoint":
        pipe = ACEPipeline(cfg.feature_spec, dtype, args.max_slots, kernel=args.kernel, accumulate=accumulate,
                           density=density)
        A = pipe.density(to_device_inputs(cfg.density.generate(), dtype, "cuda"))
        rows = A.reshape(-1, pipe.plan.a_width)
        S = int(rows.shape[0])
        g_t = torch.float64 if dtype == "f64" else torch.float32
        gB = torch.as_tensor(np.random.default_rng(6).normal(size=(S, pipe.feature_count)), dtype=g_t,
                             device="cuda")
        gA = torch.empty_like(rows)
        pipe.product_adjoint(rows, gB, out=gA)  # compiles and attaches the adjoint kernel
        if pipe.last_adjoint_backend == "generated":
            t = _time_kernel(lambda: pipe.handle.adjoint(rows, gB, out=gA), args.steps, args.warmup)
        elif pipe.last_adjoint_backend == "parts":
            # the column-major copy, the parts on the plan's streams and the fixed-order reduction
            t = _time_kernel(lambda: pipe.product_adjoint(rows, gB, out=gA), args.steps, args.warmup)
        else:
            # the term stream's reverse mode on the column-major density (the copy is
            # the forward's; timed here: clearing the partial sums, the kernel, the sum)
            At = native.transpose(rows)
            t = _time_kernel(lambda: pipe._adjoint_handle.adjoint_stream(At, gB, samples=S, columns=True, out=gA),
                             args.steps, args.warmup)
        line["backend"] = pipe.last_adjoint_backend
        nbytes = S * pipe.plan.a_width * rows.element_size() * 2 + S * pipe.feature_count * gB.element_size()
        line.update({
            "metric": "adjoint samples/s", "value": S / t, "unit": "samples/s", "higher_is_better": True,
            "us_per_call": t * 1e6, "dtype": accumulate, "storage_dtype": dtype,
            "roofline": {"bound": "hbm", "achieved": nbytes / t / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": nbytes},
            "samples": S, "features_per_sample": pipe.feature_count})
        line["config"].update({"samples": S, "features": pipe.feature_count})
    elif args.op == "neighbor_list":
        import ctypes

        # uniform random positions at the config's atom count and cutoff; box
        # edge chosen for a number density of 0.05 per unit volume (26 neighbours
        # inside the box at cutoff 5, about 24 with the open faces)
        N = d.atom_count
        box = (N / 0.05) ** (1.0 / 3.0)
        cutoff = float(d.radius)
        npdt, tdt = (np.float64, torch.float64) if dtype == "f64" else (np.float32, torch.float32)
        pos_np = np.random.default_rng(5).uniform(0.0, box, size=(N, 3)).astype(npdt)
        pos = torch.as_tensor(pos_np, device="cuda")
        nl = native.neighbor_list(pos, cutoff)  # validates the arguments; sizes the outputs
        E = int(nl["edge_sources"].shape[0])
        grid = native.cell_grid(pos_np.min(0), pos_np.max(0), cutoff, N)
        L = native.lib()
        ws_bytes = int(L.ye3t_hip_neighbor_workspace_bytes(N, ctypes.byref(grid)))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        offs = torch.empty(N + 1, dtype=torch.int64, device="cuda")
        cen, nbr, vec = (torch.empty_like(nl[k]) for k in ("edge_targets", "edge_sources", "edge_vectors"))
        code = native.F64 if dtype == "f64" else native.F32
        stream = native._stream()

        def count():
            native._check(L.ye3t_hip_neighbor_count(code, pos.data_ptr(), N, ctypes.byref(grid), cutoff,
                                                    ws.data_ptr(), ws_bytes, offs.data_ptr(), stream), "count")

        def fill():
            native._check(L.ye3t_hip_neighbor_fill(code, N, ctypes.byref(grid), cutoff,
                                                   ws.data_ptr(), ws_bytes, offs.data_ptr(), E, cen.data_ptr(),
                                                   nbr.data_ptr(), vec.data_ptr(), stream), "fill")

        count()
        fill()
        torch.cuda.synchronize()
        assert torch.equal(offs, nl["target_offsets"]) and torch.equal(nbr, nl["edge_sources"])
        t_count = _time_kernel(count, args.steps, args.warmup)
        t_fill = _time_kernel(fill, args.steps, args.warmup)
        t_build = _time_kernel(lambda: native.neighbor_list(pos, cutoff, grid=grid), args.steps, args.warmup)
        elem = pos.element_size()
        nbytes = N * 3 * elem + (N + 1) * 8 + E * (8 + 8 + 3 * elem)
        t = t_count + t_fill
        line.update({
            "metric": "neighbour-list atoms/s", "value": N / t_build, "unit": "atoms/s", "higher_is_better": True,
            "us_per_call": t_build * 1e6, "us_count_pass": t_count * 1e6, "us_fill_pass": t_fill * 1e6,
            "dtype": dtype,
            "roofline": {"bound": "hbm", "achieved": nbytes / t / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": nbytes,
                         "time": "count + fill passes, back to back"},
            "note": "us_per_call: the whole build through the Python binding, including its host "
                    "synchronisation on the edge count and the output allocations"})
        line["config"].update({"atoms": N, "edges": E, "cutoff": cutoff, "box_edge": box})
    elif args.op == "density":
        # stage 1 alone: the fused density of the whole configuration
        inp = cfg.density.generate()
        dev = to_device_inputs(inp, dtype, "cuda")
        N = d.atom_count
        adt = torch.float64 if density == "f64" else torch.float32
        A = torch.empty((N, d.channel_count, d.radial_rows, (d.l_max + 1) ** 2), dtype=adt, device="cuda")
        acc_t = torch.float64 if accumulate == "f64" else torch.float32

        def call(validate):  # the pipeline's stage 1 (ACEPipeline.density) without building a product plan
            return native.ace_density_forward(
                dev["edge_vectors"], dev["row_offsets"], dev["neighbors"], atom_count=N,
                channel_count=d.channel_count, n_max=d.n_max, l_max=d.l_max, cutoff=inp["cutoff"],
                lam=inp["lambda"], epsilon=inp["epsilon"], species=dev.get("species"),
                node_features=dev.get("node_features"), radial_mix=dev.get("radial_mix"), out=A, out_dtype=adt,
                accumulate_dtype=acc_t, validate=validate)

        call(True)  # validates the CSR and neighbour indices once
        kernel = native.last_density_kernel()
        t = _time_kernel(lambda: call(False), args.steps, args.warmup)
        if args.copy_probe:  # a plain elementwise copy of A's size, for the FETCH_SIZE / WRITE_SIZE scales
            probe = torch.empty_like(A)
            torch.neg(A, out=probe)
            torch.cuda.synchronize()
            line["copy_probe_bytes"] = {"read": A.numel() * A.element_size(), "write": probe.numel() * probe.element_size()}
            del probe
        elem = 8 if dtype == "f64" else 4
        b1, _ = algorithmic_bytes(cfg, _NoPlan(), elem)
        a_elem = A.element_size()
        a_bytes = A.numel() * a_elem
        line.update({
            "metric": "density GB/s", "value": b1 / t / 1e9, "unit": "GB/s", "higher_is_better": True,
            "us_per_call": t * 1e6, "atoms_per_s": N / t, "dtype": "f64", "storage_dtype": dtype,
            "density_dtype": density, "kernel": kernel,
            "roofline": {"bound": "hbm", "achieved": b1 / t / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": b1 / t / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": b1,
                         "density_bytes": a_bytes, "density_write_frac": a_bytes / t / 1e9 / HBM_PEAK_GBS},
            "note": "algorithmic bytes per the survey's stage-1 formula at the storage element size; "
                    "timed through the Python binding without its CSR validation (validated once)"})
        line["config"].update({"atoms": N, "edges": int(inp["edge_count"])})
    elif args.op == "density_edge_gradient":
        inp = cfg.density.generate()
        dev = to_device_inputs(inp, dtype, "cuda")
        N, E = d.atom_count, int(inp["edge_count"])
        rows = d.radial_rows
        shape = (N, d.channel_count, rows, (d.l_max + 1) ** 2)
        gdt = torch.float64 if density == "f64" else torch.float32
        gA = torch.as_tensor(np.random.default_rng(4).normal(size=shape), dtype=gdt, device="cuda")
        kw = dict(atom_count=N, channel_count=d.channel_count, n_max=d.n_max, l_max=d.l_max, cutoff=inp["cutoff"],
                  lam=inp["lambda"], epsilon=inp["epsilon"], species=dev.get("species"),
                  node_features=dev.get("node_features"), radial_mix=dev.get("radial_mix"))
        call = lambda v: native.ace_density_edge_gradient(gA, dev["edge_vectors"], dev["row_offsets"],  # noqa: E731
                                                          dev["neighbors"], validate=v, **kw)
        call(True)  # validates the CSR once
        t = _time_kernel(lambda: call(False), args.steps, args.warmup)
        elem = dev["edge_vectors"].element_size()
        # per edge: its vector, neighbour index and gradient; per atom: its CSR offset, the
        # adjoint row and (features) its feature row, each read once
        feat = d.channel_count * elem if inp.get("node_features") is not None else 0
        nbytes = E * (3 * elem + 8 + 3 * elem) + (N + 1) * 8 + gA.numel() * gA.element_size() + N * feat
        line.update({
            "metric": "force edges/s", "value": E / t, "unit": "edges/s", "higher_is_better": True,
            "us_per_call": t * 1e6, "dtype": "f64", "storage_dtype": dtype, "adjoint_dtype": str(gdt)[6:],
            "roofline": {"bound": "hbm", "achieved": nbytes / t / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": nbytes},
            "note": "timed through the Python binding without its CSR validation (validated once)"})
        line["config"].update({"edges": E, "atoms": N})
    else:
        inp = cfg.density.generate()
        N = d.atom_count
        C = d.channel_count * d.radial_rows * (d.l_max + 1) ** 2
        tdt = torch.float64 if accumulate == "f64" else torch.float32
        adj = torch.as_tensor(np.random.default_rng(4).normal(size=(N, C)), dtype=tdt, device="cuda")
        centers = torch.as_tensor(inp["centers"], device="cuda")
        E = int(centers.shape[0])
        density_accumulate_adjoint(adj, centers)  # validates the centres once (a host-side range check)
        t = _time_kernel(lambda: native.density_accumulate_adjoint(adj, centers), args.steps, args.warmup)
        elem = adj.element_size()
        nbytes = E * C * elem + E * 8 + N * C * elem
        line.update({
            "metric": "edge-adjoint GB/s", "value": nbytes / t / 1e9, "unit": "GB/s", "higher_is_better": True,
            "us_per_call": t * 1e6, "dtype": accumulate,
            "roofline": {"bound": "hbm", "achieved": nbytes / t / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": nbytes},
            "note": "timed through the C-ABI binding; the Python wrapper's centre range check ran once"})
        line["config"].update({"edges": E, "atoms": N, "channels": C})
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # the warmup also lasts at least MIN_WARMUP_S seconds whatever --warmup says
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=1000)
    ap.add_argument("--min-warmup-s", type=float, default=MIN_WARMUP_S,
                    help="least warmup time in seconds (counter-collection runs, whose dispatches are "
                         "serialised, pass 0)")
    ap.add_argument("--config", type=int, default=4)
    ap.add_argument("--dtype", default=None, help="storage type of inputs and B-features (f32 / f64)")
    ap.add_argument("--accumulate", default=None, help="type of the arithmetic (default per config)")
    ap.add_argument("--density", default=None, help="storage type of A (default per config)")
    ap.add_argument("--max-slots", type=int, default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--kernel", default="auto", choices=["auto", "generated", "parts", "interpreter"])
    ap.add_argument("--op", default="pipeline",
                    choices=["pipeline", "density", "linear_readout", "density_accumulate_adjoint",
                             "product_adjoint", "neighbor_list", "density_edge_gradient"],
                    help="pipeline: the headline step (stage 1 + stage 2); the others time one widened op "
                         "on the config's shapes and print its own JSON line")
    ap.add_argument("--copy-probe", action="store_true",
                    help="after the timed region, negate B into a new tensor once (a plain elementwise copy "
                         "kernel of known size, for calibrating FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "the ACE product is per-sample independent and shards by atoms, see DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from ye3t_amd.ace import workloads as W
    from ye3t_amd.ace.pipeline import ACEPipeline, to_device_inputs
    from ye3t_amd.ace.program import program_stats
    from ye3t_amd.runtime import native

    cfg = W.config(args.config)
    if args.op != "pipeline":
        print(json.dumps(bench_op(args, cfg)))
        return
    dtype = args.dtype or cfg.dtypes[0]
    accumulate = args.accumulate or (cfg.accumulate if dtype == "f32" else None) or dtype
    density = args.density or (cfg.density_dtype if dtype == "f32" and accumulate == cfg.accumulate else None) or accumulate
    elem = 8 if dtype == "f64" else 4
    a_elem = 8 if density == "f64" else 4
    t_build = time.perf_counter()
    pipe = ACEPipeline(cfg.feature_spec, dtype, args.max_slots, kernel=args.kernel, accumulate=accumulate,
                       density=density)
    t_build = time.perf_counter() - t_build
    inp = cfg.density.generate()
    dev = to_device_inputs(inp, dtype, "cuda")
    d = cfg.density
    A = torch.empty((d.atom_count, d.channel_count, d.radial_rows, (d.l_max + 1) ** 2),
                    dtype=torch.float64 if density == "f64" else torch.float32, device="cuda")
    rows = A.reshape(-1, pipe.plan.a_width)
    B = torch.empty((rows.shape[0], pipe.feature_count),
                    dtype=torch.float64 if dtype == "f64" else torch.float32, device="cuda")

    pipe.density(dev, out=A)  # validates the CSR and neighbour indices once

    def step():
        pipe.density(dev, out=A, validate=False)
        pipe.product(rows, out=B)

    # at least --warmup steps and at least MIN_WARMUP_S seconds of them: the
    # GPU reaches its steady clocks only after ~0.1 s of work (config 4 with 5
    # warmup steps: 0.207 ms per step; after 1 000: 0.157 ms)
    warm_steps, warm_s = warm_up(step, args.warmup, args.min_warmup_s)
    # Per-kernel durations come from HIP events on one timed step in ten: an
    # event record drains the queue between the two kernels (config 4: 0.167 ms
    # per step with events on every step, 0.156 ms without), so the other
    # steps run as a caller would run them.
    every = 10 if args.steps >= 20 else 1
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(0, args.steps, every)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        if i % every:
            pipe.density(dev, out=A, validate=False)
            pipe.product(rows, out=B)
            continue
        e0, e1, e2 = ev[i // every]
        e0.record()
        pipe.density(dev, out=A, validate=False)
        e1.record()
        pipe.product(rows, out=B)
        e2.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    copy_bytes = None
    if args.copy_probe:
        # an elementwise kernel that reads B once and writes a same-size tensor once
        probe = torch.empty_like(B)
        torch.neg(B, out=probe)
        torch.cuda.synchronize()
        copy_bytes = {"read": B.numel() * B.element_size(), "write": probe.numel() * probe.element_size()}
    s1 = float(np.mean([a.elapsed_time(b) for a, b, _ in ev])) * 1e-3
    s2 = float(np.mean([b.elapsed_time(c) for _, b, c in ev])) * 1e-3
    ms_per_step = wall / args.steps * 1e3
    b1, b2 = algorithmic_bytes(cfg, pipe.plan, elem)
    c1, c2 = as_built_bytes(cfg, pipe.plan, elem, a_elem)
    if pipe.kernel == "generated":
        k2 = "ye3t_product_generated"
    elif pipe.kernel == "parts":
        # the stage-2 time includes the column-major copy of the density the parts read
        k2 = "transpose_kernel+ye3t_product_part" if pipe._columns else "ye3t_product_part"
    elif pipe.handle.uses_stream:
        # the stage-2 time includes the column-major copy of the density it reads
        k2 = "transpose_kernel+product_stream_kernel" if pipe._columns else "product_stream_kernel"
    else:
        k2 = "product_kernel"
    features = rows.shape[0] * pipe.feature_count
    value = features / (wall / args.steps)
    stats = program_stats(pipe.program)
    workload = f"config{cfg.config_id}-{cfg.name}"
    prec = f"{accumulate}-{density}A"  # arithmetic and density storage of the counter summaries
    traffic, traffic_src = counter_traffic(k2, workload, prec)
    k1 = native.last_density_kernel()
    traffic1, traffic1_src = counter_traffic(k1, workload, prec)
    line = {
        "metric": "B-features/sec (atoms/s) on 1 MI355X; achieved HBM GB/s vs peak",
        "value": value,
        "unit": "B-features/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm_steps,
        "warmup_s": warm_s,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": accumulate,
        "storage_dtype": dtype,
        "density_dtype": density,
        "data": "synthetic (seeded counter RNG, BASELINE.json configuration shapes)",
        "config": {"workload": workload, "atoms": d.atom_count,
                   "neighbors_per_atom": d.neighbors_per_atom, "channels": d.channel_count,
                   "samples": int(rows.shape[0]), "features_per_sample": pipe.feature_count,
                   "n_max": d.n_max, "l_max": d.l_max, "nu_max": cfg.feature_spec.nu_max,
                   "targets": list(cfg.feature_spec.targets), "parallelism": "single GPU"},
        "atoms_per_s": d.atom_count / (wall / args.steps),
        "roofline": {"bound": "hbm", "achieved": b2 / s2 / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": b2 / s2 / 1e9 / HBM_PEAK_GBS, "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": k2, "algorithmic_bytes": b2, "algorithmic_bytes_as_built": c2,
                     "frac_as_built": c2 / s2 / 1e9 / HBM_PEAK_GBS,
                     "avg_kernel_us": s2 * 1e6, "event_steps": len(ev)},
        "stage1": {"kernel": k1, "avg_kernel_us": s1 * 1e6, "algorithmic_bytes": b1,
                   "achieved_gbs": b1 / s1 / 1e9, "frac": b1 / s1 / 1e9 / HBM_PEAK_GBS,
                   "algorithmic_bytes_as_built": c1, "frac_as_built": c1 / s1 / 1e9 / HBM_PEAK_GBS,
                   "traffic": traffic1, "traffic_source": traffic1_src},
        "stage2": {"kernel": k2, "avg_kernel_us": s2 * 1e6, "algorithmic_bytes": b2,
                   "achieved_gbs": b2 / s2 / 1e9, "frac": b2 / s2 / 1e9 / HBM_PEAK_GBS,
                   "algorithmic_bytes_as_built": c2, "frac_as_built": c2 / s2 / 1e9 / HBM_PEAK_GBS,
                   "program": stats, "plan_compile_s": t_build, "product_kernel": pipe.kernel},
        "bytes_note": "algorithmic_bytes: the survey's compulsory-traffic formula at the configuration's "
                      "storage element size with 4-byte indices; _as_built: int64 indices and the density at "
                      "its stored size",
    }
    if copy_bytes is not None:
        line["copy_probe_bytes"] = copy_bytes
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, pipe, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
