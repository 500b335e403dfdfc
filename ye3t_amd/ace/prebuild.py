"""Compile the generated product kernels of benchmark configurations ahead of use.

Plans between ``GENERATED_MAX_TERMS`` and ``PARTS_MAX_TERMS`` terms run on a
generated kernel in parts (``codegen.generate_parts``, with the reverse sweep
``generate_adjoint_parts`` and the fused readout ``generate_readout_parts``),
one hipRTC module per 9 chunks (64 for plans above 100 000 terms).  hipRTC
compiles one module at a time per process (one to five minutes for a 64-chunk
config-3 part), so the parts are spread over worker processes.  hipRTC needs
no GPU, so this runs on a build host; the code objects land in the JIT cache
(``ye3t_amd/jit_cache`` unless ``YE3T_AMD_JIT_CACHE`` says otherwise), keyed by
architecture, compiler fingerprint (hipRTC version, options, ABI) and source
(``native.rtc_cache_key``), and travel with the tree.

    python -m ye3t_amd.ace.prebuild            # configs 2, 3 and 5, every dtype they are benchmarked in
    python -m ye3t_amd.ace.prebuild 2 --dtype f64
"""

import argparse
import multiprocessing
import os
import sys
import time
from concurrent.futures import ProcessPoolExecutor


def precisions(cfg, dtype):
    """(accumulate, density) of ``dtype`` storage, as ``bench.py`` and the tests choose them."""
    accumulate = (cfg.accumulate if dtype == "f32" else None) or dtype
    density = (cfg.density_dtype if dtype == "f32" and accumulate == cfg.accumulate else None) or accumulate
    return accumulate, density


def _compile(source):
    from ye3t_amd.runtime import native

    return native.rtc_compile(source)


def prebuild(config_ids=(2, 3, 5), dtypes=None, workers=None, log=print):
    from ye3t_amd.ace import workloads as W
    from ye3t_amd.ace.codegen import (generate_adjoint_parts, generate_parts, generate_readout_parts, part_chunks,
                                      part_max_live)
    from ye3t_amd.ace.pipeline import (ADJOINT_PART_CHUNKS, ADJOINT_PART_MAX_LIVE, ADJOINT_PARTS_MAX_TERMS,
                                       GENERATED_MAX_TERMS, PARTS_MAX_TERMS, fit_parts_to_scratch)
    from ye3t_amd.ace.plan import ProductPlan
    from ye3t_amd.runtime import native

    workers = workers or min(16, os.cpu_count() or 1)
    for cid in config_ids:
        cfg = W.config(cid)
        plan = ProductPlan(cfg.feature_spec)
        terms = sum(len(nd.get("terms", ())) for nd in plan.nodes)
        if not GENERATED_MAX_TERMS < terms <= PARTS_MAX_TERMS:
            log(f"config {cid}: {terms} terms, not a parts plan; skipped")
            continue
        for dtype in dtypes or cfg.dtypes:
            accumulate, density = precisions(cfg, dtype)
            live, per = part_max_live(plan, accumulate), part_chunks(plan)
            adjoint = []
            if terms <= ADJOINT_PARTS_MAX_TERMS:
                adjoint, _ = generate_adjoint_parts(plan, accumulate, max_live=ADJOINT_PART_MAX_LIVE,
                                                    chunks_per_part=ADJOINT_PART_CHUNKS, grad_dtype=dtype,
                                                    in_dtype=density)
            t0 = time.time()
            # worker processes (spawned: nothing of this process is inherited) compile in parallel;
            # parts above the library's scratch bound are regenerated in smaller chunks, as the
            # pipeline does (fit_parts_to_scratch)
            with ProcessPoolExecutor(workers, mp_context=multiprocessing.get_context("spawn")) as pool:
                compile_all = lambda sources: list(pool.map(_compile, sources))  # noqa: E731
                parts = fit_parts_to_scratch(
                    lambda n: generate_parts(plan, accumulate, max_live=n, chunks_per_part=per, out_dtype=dtype,
                                             in_dtype=density), live, "ye3t_product_part", compile_all)
                readout = fit_parts_to_scratch(
                    lambda n: generate_readout_parts(plan, accumulate, max_live=n, chunks_per_part=per,
                                                     in_dtype=density)[0], live, "ye3t_product_readout_part",
                    compile_all)
                compile_all([part[0] for part in adjoint])
            log(f"config {cid} {dtype} (arithmetic {accumulate}, density {density}): {len(parts)} forward, "
                f"{len(adjoint)} adjoint and {len(readout)} readout parts in {time.time() - t0:.1f} s "
                f"-> {native._jit_cache_dir()}")


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("configs", nargs="*", type=int, default=[2, 3, 5])
    ap.add_argument("--dtype", action="append", help="storage dtype (default: every dtype of the config)")
    ap.add_argument("--workers", type=int, default=None)
    args = ap.parse_args(argv)
    prebuild(args.configs, args.dtype, args.workers)


if __name__ == "__main__":
    sys.exit(main())
