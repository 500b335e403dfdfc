"""End-to-end ACE hot path on one GPU: density (stage 1) then B-features (stage 2).

``ACEPipeline`` owns a compiled :class:`~ye3t_amd.ace.plan.ProductPlan`, its
device program, and the stage-1 parameters.  Inputs stay resident in HBM;
``forward`` launches exactly two kernels on the current stream.
"""

import os

import numpy as np

from ye3t_amd.ace.plan import ProductPlan
from ye3t_amd.ace.program import compile_program
from ye3t_amd.runtime import native


def to_device_inputs(inp, dtype, device="cuda"):
    """Move a workload dict (``workloads.DensityWorkload.generate``) to the GPU."""
    import torch

    real = torch.float64 if dtype == "f64" else torch.float32
    out = {k: v for k, v in inp.items() if not isinstance(v, np.ndarray)}
    out["row_offsets"] = torch.as_tensor(inp["row_offsets"], dtype=torch.int64, device=device)
    out["neighbors"] = torch.as_tensor(inp["neighbors"], dtype=torch.int64, device=device)
    out["edge_vectors"] = torch.as_tensor(inp["edge_vectors"], dtype=real, device=device).contiguous()
    for key in ("species",):
        if inp.get(key) is not None:
            out[key] = torch.as_tensor(inp[key], dtype=torch.int32, device=device)
    for key in ("node_features", "radial_mix"):
        if inp.get(key) is not None:
            out[key] = torch.as_tensor(inp[key], dtype=real, device=device).contiguous()
    return out


# plans up to this many DAG terms get a plan-specialised (generated) kernel;
# larger plans run the generic interpreter (hipRTC time grows with code size)
GENERATED_MAX_TERMS = 5000
# plans up to this size run on a generated kernel in parts (one hipRTC module per
# 9 chunks, compiled once and cached: config 5's 1.32 M terms are 143 parts);
# larger ones on the interpreter
PARTS_MAX_TERMS = 2000000
# the reverse mode runs in parts up to this plan size (config 3: 196 parts), above
# it on the term stream's reverse mode
ADJOINT_PARTS_MAX_TERMS = 200000
# the reverse mode's parts: chunks of fewer node values (values and gradients are
# live together; 128 compiles without spills at config 2) and chunks per part:
# a part's chunks run back to back on a tile, so fewer parts re-read less of the
# density and gB (config 3 fp64 21.8 / 16.7 / 16.0 ms at 8 / 32 / 64 chunks per
# part; config 2 658 / 633 / 634 us)
ADJOINT_PART_MAX_LIVE = 128
ADJOINT_PART_CHUNKS = 64
# node values taken off a chunk when a compiled part needs more scratch than the
# library runs (config 5's fused readout at 300 values: one part at 1 060 bytes)
PART_LIVE_STEP = 50


def fit_parts_to_scratch(make, live, kernel, compile_all=None):
    """``make(n)`` for the largest node-value budget ``n`` from ``live`` down,
    in steps of ``PART_LIVE_STEP``, whose every compiled part (``kernel`` in
    each code object) needs at most ``native.part_private_limit()`` bytes of
    scratch per lane; the attach entry points refuse any part above it.
    ``make(n)`` returns ``[(source, meta), ...]``; ``compile_all(sources)``
    returns their code objects (default: hipRTC through the JIT cache, one at
    a time)."""
    limit = native.part_private_limit()
    if compile_all is None:
        compile_all = lambda sources: [native.rtc_compile(src) for src in sources]  # noqa: E731
    while True:
        parts = make(live)
        codes = compile_all([src for src, _meta in parts])
        worst = max(native.code_object_kernel_info(code, kernel)["private_segment_bytes"] for code in codes)
        if worst <= limit or live <= PART_LIVE_STEP:
            return parts
        live -= PART_LIVE_STEP


class ACEPipeline:
    """``dtype``: storage type of the inputs and of the B-features.

    ``accumulate``: type of all arithmetic, and of the density ``A`` unless
    ``density`` says otherwise (default: ``dtype``).  "f64" with
    ``dtype="f32"`` keeps fp32 inputs and outputs but carries the density and
    the CG products in fp64, for plans whose features cancel too strongly for
    fp32 intermediates.

    ``density``: storage type of ``A`` (default: ``accumulate``).  "f32" with
    ``accumulate="f64"`` accumulates the density in fp64, rounds each value
    once to fp32 for storage (half the density bytes) and converts it back to
    fp64 for the product; this needs a plan with a generated product kernel.

    ``kernel``: "auto" (a generated kernel when the plan has at most
    ``GENERATED_MAX_TERMS`` terms, a generated kernel in parts up to
    ``PARTS_MAX_TERMS``, else the interpreter), "generated", "parts" or
    "interpreter" (the generic table-driven product kernel)."""

    def __init__(self, feature_spec, dtype="f32", max_slots=None, plan=None, kernel="auto", max_live=None,
                 accumulate=None, density=None):
        self.spec = feature_spec
        self.dtype = dtype
        self.accumulate = accumulate or dtype
        self.density_dtype = density or self.accumulate
        if dtype not in ("f32", "f64") or self.accumulate not in ("f32", "f64") or (
                dtype == "f64" and self.accumulate == "f32"):
            raise ValueError(f"unsupported precision: dtype {dtype!r}, accumulate {accumulate!r}")
        if self.density_dtype not in ("f32", "f64") or (self.accumulate == "f32" and self.density_dtype == "f64"):
            raise ValueError(f"unsupported density dtype {density!r} for {self.accumulate} arithmetic")
        if kernel not in {"auto", "generated", "parts", "interpreter"}:
            raise ValueError(f"unknown product kernel {kernel!r}")
        self.plan = plan if plan is not None else ProductPlan(feature_spec)
        terms = sum(len(nd.get("terms", ())) for nd in self.plan.nodes)
        self._terms = terms
        use_gen = kernel == "generated" or (kernel == "auto" and terms <= GENERATED_MAX_TERMS)
        use_parts = kernel == "parts" or (kernel == "auto" and not use_gen and terms <= PARTS_MAX_TERMS)
        if self.density_dtype != self.accumulate and not (use_gen or use_parts):
            raise ValueError(f"a {self.density_dtype} density with {self.accumulate} arithmetic needs a generated "
                             f"product kernel (plans of at most {PARTS_MAX_TERMS} terms)")
        self.program = compile_program(self.plan, self.accumulate, max_slots)
        self.handle = native.ProductPlanHandle(self.program, out_dtype=dtype, in_dtype=self.density_dtype)
        self._columns = os.environ.get("YE3T_PRODUCT_COLUMNS", "1") != "0"
        self._At = None  # (key, column-major density buffer) of the interpreter path
        self._adjoint_handle = None  # program of the interpreter plans' reverse mode
        self.kernel = "interpreter"
        if use_gen:
            from ye3t_amd.ace.codegen import generate

            from ye3t_amd.ace.codegen import generate_persistent

            rows = os.environ.get("YE3T_PRODUCT_ROWS")  # samples per workgroup (tuning; default by LDS fit)
            persistent = os.environ.get("YE3T_PRODUCT_PERSISTENT", "1") != "0"
            waves = os.environ.get("YE3T_PRODUCT_WAVES")  # waves sharing a tile (tuning)
            if persistent and max_live is None and self.plan.feature_count % 2 and rows is None:
                # two waves share each tile: each computes half the outputs, with
                # half the live values (fp64 config 4: 170 -> 144 us)
                # B is written once and not re-read by this pipeline: non-temporal
                # stores (policy 2) keep it from evicting the next step's inputs and
                # the density from the last-level cache (config 4: ~7 us per step)
                policy = os.environ.get("YE3T_PRODUCT_STORE_POLICY")  # cache-policy bits (tuning)
                source, meta = generate_persistent(self.plan, self.accumulate, out_dtype=dtype,
                                                   waves=int(waves) if waves else 2,
                                                   store_policy=int(policy) if policy else 2,
                                                   in_dtype=self.density_dtype)
            else:
                source, meta = generate(self.plan, self.accumulate, max_live, out_dtype=dtype,
                                        rows=int(rows) if rows else None, in_dtype=self.density_dtype)
            self.handle.attach_generated(source, meta)
            self.kernel = "generated"
        elif use_parts:
            from ye3t_amd.ace.codegen import generate_parts, part_chunks

            # node values per chunk and chunks per part (tuning)
            live = self._parts_max_live()
            per = int(os.environ.get("YE3T_PARTS_CHUNKS", 0)) or part_chunks(self.plan)
            group = int(os.environ.get("YE3T_PARTS_GROUP", 32))  # output columns per staged store
            parts = fit_parts_to_scratch(
                lambda n: generate_parts(self.plan, self.accumulate, max_live=n, chunks_per_part=per,
                                         out_dtype=dtype, in_dtype=self.density_dtype, group=group),
                live, "ye3t_product_part")
            self.handle.attach_generated_parts(parts)
            self.kernel = "parts"

    def _parts_max_live(self):
        """Node values per chunk of the generated parts: ``YE3T_PARTS_MAX_LIVE``
        or ``codegen.part_max_live``.  Chunks above ``PART_MAX_LIVE`` (400) are
        refused: config 5 in 550-value chunks (kernels with 1 260 and 2 052
        bytes of scratch per lane) ended in a memory aperture violation on the
        GPU, while 400-value chunks (772 bytes) ran clean.  The library's attach
        entry points also refuse any part above 1 024 bytes of scratch per lane
        (``native.part_private_limit``), whatever its chunk size."""
        from ye3t_amd.ace.codegen import PART_MAX_LIVE, part_max_live

        env = os.environ.get("YE3T_PARTS_MAX_LIVE")
        live = part_max_live(self.plan, self.accumulate) if env is None else int(env)
        if not 1 <= live <= PART_MAX_LIVE:
            raise ValueError(f"YE3T_PARTS_MAX_LIVE must be in [1, {PART_MAX_LIVE}], got {live}")
        return live

    @staticmethod
    def _adjoint_parts_max_live():
        """Node values per chunk of the reverse-mode parts:
        ``YE3T_ADJOINT_PARTS_MAX_LIVE`` or 128, within the forward's bound."""
        from ye3t_amd.ace.codegen import PART_MAX_LIVE

        live = int(os.environ.get("YE3T_ADJOINT_PARTS_MAX_LIVE", ADJOINT_PART_MAX_LIVE))
        if not 1 <= live <= PART_MAX_LIVE:
            raise ValueError(f"YE3T_ADJOINT_PARTS_MAX_LIVE must be in [1, {PART_MAX_LIVE}], got {live}")
        return live

    @property
    def feature_count(self):
        return self.plan.feature_count

    def density(self, dev_inp, out=None, validate=True):
        """Stage 1.  ``validate`` range-checks the CSR offsets and the neighbour
        and species indices before the launch (a caller that reuses validated
        inputs, such as a timing loop, may skip it)."""
        import torch

        return native.ace_density_forward(
            dev_inp["edge_vectors"], dev_inp["row_offsets"], dev_inp["neighbors"],
            atom_count=int(dev_inp["atom_count"]), channel_count=int(dev_inp["channel_count"]),
            n_max=int(dev_inp["n_max"]), l_max=int(dev_inp["l_max"]), cutoff=float(dev_inp["cutoff"]),
            lam=float(dev_inp["lambda"]), epsilon=float(dev_inp.get("epsilon", 1e-12)),
            species=dev_inp.get("species"), node_features=dev_inp.get("node_features"),
            radial_mix=dev_inp.get("radial_mix"), out=out,
            out_dtype=torch.float64 if self.density_dtype == "f64" else torch.float32,
            accumulate_dtype=torch.float64 if self.accumulate == "f64" else torch.float32, validate=validate)

    def product(self, A_rows, out=None):
        """B-features of the density rows.  Interpreter plans and generated
        parts read a column-major copy of the density (each density column of
        64 samples is one contiguous block for their loads);
        ``YE3T_PRODUCT_COLUMNS=0`` reads the rows directly."""
        columns = self.kernel == "parts" or (self.kernel == "interpreter" and self.handle.uses_stream)
        if columns and self._columns:
            S = int(A_rows.shape[0])
            ld = (S + 63) // 64 * 64
            key = (int(A_rows.shape[1]), ld, A_rows.dtype, A_rows.device)
            if self._At is None or self._At[0] != key:
                import torch

                self._At = (key, torch.empty((key[0], ld), dtype=A_rows.dtype, device=A_rows.device))
            At = native.transpose(A_rows.contiguous(), out=self._At[1], ld=ld)
            return self.handle.forward_columns(At, S, out=out)
        return self.handle.forward(A_rows, out=out)

    def product_adjoint(self, A_rows, gB, out=None):
        """Density gradient ``gA[s] = J(A[s])^T gB[s]`` of a feature gradient
        (reference ``factorized_angular_adjoint``).  Generated plans use a
        plan-specialised kernel compiled on first use; interpreter plans use the
        term stream's reverse mode on the column-major density.  Plans whose
        workspace is too wide for the term stream raise ``NotImplementedError``."""
        self.last_adjoint_backend = None
        if self.kernel == "parts" and self._terms <= ADJOINT_PARTS_MAX_TERMS:
            return self._adjoint_parts(A_rows, gB, out)
        if self.kernel != "generated":
            if self._adjoint_handle is None:
                # the forward's program; YE3T_ADJOINT_SLOTS compiles one with a narrower
                # workspace (the reverse mode keeps values and gradients in LDS; tuning)
                slots = os.environ.get("YE3T_ADJOINT_SLOTS")
                if slots is None:
                    self._adjoint_handle = self.handle
                else:
                    program = compile_program(self.plan, self.accumulate, int(slots))
                    self._adjoint_handle = native.ProductPlanHandle(program, out_dtype=self.dtype)
            if not self._adjoint_handle.uses_stream:
                raise NotImplementedError("no device adjoint for a plan without a term stream "
                                          f"(workspace of {self.program['workspace_slots']} slots)")
            S = int(A_rows.shape[0])
            ld = (S + 63) // 64 * 64
            key = (int(A_rows.shape[1]), ld, A_rows.dtype, A_rows.device)
            if self._At is None or self._At[0] != key:
                import torch

                self._At = (key, torch.empty((key[0], ld), dtype=A_rows.dtype, device=A_rows.device))
            At = native.transpose(A_rows.contiguous(), out=self._At[1], ld=ld)
            self.last_adjoint_backend = "stream"
            return self._adjoint_handle.adjoint_stream(At, gB, samples=S, columns=True, out=out)
        self.last_adjoint_backend = "generated"
        if getattr(self.handle, "adjoint_kernel", None) is None:
            from ye3t_amd.ace.codegen import generate_adjoint

            waves = os.environ.get("YE3T_ADJOINT_WAVES")  # waves sharing a tile (tuning)
            source, meta = generate_adjoint(self.plan, self.accumulate, grad_dtype=self.dtype,
                                            waves=int(waves) if waves else 2, in_dtype=self.density_dtype)
            self.handle.attach_adjoint(source, meta)
        return self.handle.adjoint(A_rows, gB, out=out)

    def _adjoint_parts(self, A_rows, gB, out, block_bytes=2 << 30):
        """Reverse mode of a parts plan: the plan-specialised adjoint in parts
        (compiled on first use) on the column-major density, in sample blocks
        whose partial buffer stays within ``block_bytes``."""
        import torch

        from ye3t_amd.ace.codegen import generate_adjoint_parts

        if getattr(self.handle, "adjoint_part_meta", None) is None:
            # smaller chunks than the forward's: values and gradients are live together (tuning)
            live = self._adjoint_parts_max_live()
            per = int(os.environ.get("YE3T_ADJOINT_PARTS_CHUNKS", ADJOINT_PART_CHUNKS))
            parts, reduction = generate_adjoint_parts(self.plan, self.accumulate, max_live=live, chunks_per_part=per,
                                                      grad_dtype=self.dtype, in_dtype=self.density_dtype)
            self.handle.attach_adjoint_parts(parts, reduction)
            self._adjoint_rows = int(reduction["partial_rows"])
        S = int(A_rows.shape[0])
        W = self.plan.a_width
        a_t = torch.float64 if self.density_dtype == "f64" else torch.float32
        if out is None:
            out = torch.empty((S, W), dtype=a_t, device=A_rows.device)
        if S == 0:
            return out
        ld = (S + 63) // 64 * 64
        key = (W, ld, A_rows.dtype, A_rows.device)
        if self._At is None or self._At[0] != key:
            self._At = (key, torch.empty((W, ld), dtype=A_rows.dtype, device=A_rows.device))
        At = native.transpose(A_rows.contiguous(), out=self._At[1], ld=ld)
        elem = 8 if self.accumulate == "f64" else 4
        blk = max(64, block_bytes // max(1, self._adjoint_rows * elem) // 64 * 64)
        gB = gB.contiguous()
        for s0 in range(0, S, blk):
            s1 = min(S, s0 + blk)
            self.handle.adjoint_parts(At[:, s0:], gB[s0:s1], samples=s1 - s0, columns=True, out=out[s0:s1])
        self.last_adjoint_backend = "parts"
        return out

    def linear(self, A_rows, weight, bias=0.0, out=None, block_bytes=1 << 30):
        """Linear readout ``out[s] = bias + sum_k B[s, k] weight[k]`` (reference
        ``factorized_angular_linear``, ``execution_plan.py:13793-13850``).

        Plans with a generated product kernel, whole or in parts, use a fused,
        plan-specialised readout that never stores B (compiled on first use).
        Interpreter plans materialise B in sample blocks of at most
        ``block_bytes`` and reduce each row with ``rows_dot`` (the reference's
        materialised path).
        ``last_linear_backend`` records which ran.
        """
        import torch

        F = self.plan.feature_count
        weight = torch.as_tensor(weight, device=A_rows.device)
        if weight.ndim != 1 or int(weight.shape[0]) != F:
            raise ValueError(f"weight must be a vector of the {F} features")
        S = int(A_rows.shape[0])
        out_t = torch.float64 if self.dtype == "f64" else torch.float32
        if out is None:
            out = torch.empty((S,), dtype=out_t, device=A_rows.device)
        if self.kernel == "parts":
            from ye3t_amd.ace.codegen import generate_readout_parts, part_chunks

            if getattr(self.handle, "readout_part_meta", None) is None:
                live = self._parts_max_live()
                per = int(os.environ.get("YE3T_PARTS_CHUNKS", 0)) or part_chunks(self.plan)
                parts = fit_parts_to_scratch(
                    lambda n: generate_readout_parts(self.plan, self.accumulate, max_live=n, chunks_per_part=per,
                                                     in_dtype=self.density_dtype)[0],
                    live, "ye3t_product_readout_part")
                self.handle.attach_readout_parts(parts)
            w = weight.to(torch.float64 if self.accumulate == "f64" else torch.float32).contiguous()
            if S == 0:
                return out
            ld = (S + 63) // 64 * 64
            key = (int(A_rows.shape[1]), ld, A_rows.dtype, A_rows.device)
            if self._At is None or self._At[0] != key:
                self._At = (key, torch.empty((key[0], ld), dtype=A_rows.dtype, device=A_rows.device))
            At = native.transpose(A_rows.contiguous(), out=self._At[1], ld=ld)
            self.last_linear_backend = "fused_parts"
            return self.handle.linear_parts(At, w, float(bias), samples=S, columns=True, out=out)
        if self.kernel == "generated":
            if getattr(self.handle, "readout", None) is None:
                from ye3t_amd.ace.codegen import generate_readout

                source, meta = generate_readout(self.plan, self.accumulate, out_dtype=self.dtype,
                                                in_dtype=self.density_dtype)
                self.handle.attach_readout(source, meta)
            w = weight.to(torch.float64 if self.accumulate == "f64" else torch.float32).contiguous()
            self.last_linear_backend = "fused_generated"
            return self.handle.linear(A_rows, w, float(bias), out=out)
        w = weight.to(out_t).contiguous()
        elem = 8 if self.dtype == "f64" else 4
        blk = max(1, min(S, int(block_bytes) // (F * elem)))
        B = torch.empty((min(blk, S), F), dtype=out_t, device=A_rows.device)
        for s0 in range(0, S, blk):
            s1 = min(S, s0 + blk)
            Bb = B[: s1 - s0]
            self.handle.forward(A_rows[s0:s1], out=Bb)
            native.rows_dot(Bb, w, float(bias), out=out[s0:s1])
        self.last_linear_backend = "materialized_blocks"
        return out

    def forward(self, dev_inp, channelwise=False, A_out=None, B_out=None, validate=True):
        A = self.density(dev_inp, out=A_out, validate=validate)
        rows = A.reshape(-1, self.plan.a_width) if channelwise else A.reshape(A.shape[0], -1)
        if rows.shape[1] != self.plan.a_width:
            raise ValueError(f"density row width {rows.shape[1]} != plan width {self.plan.a_width}")
        return A, self.product(rows, out=B_out)
