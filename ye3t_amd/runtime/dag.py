"""The reference's general factorized-angular DAG op on the HIP library.

``factorized_angular`` and ``factorized_angular_linear`` take the reference
op's arguments (schema ``execution_plan_torch.cpp:7586-7594`` and the linear
readout's) and differentiate through the library's adjoint kernels
(``ye3t_hip_factorized_angular_adjoint`` / ``_linear_adjoint``), which follow
the reference's conjugate-transpose convention: the gradient Torch autograd
returns for the reference's own Torch restatement.

``YE3TFactorizedAngularModule`` mirrors the reference module
(``ye3t/runtime/execution_plan.py:13550-13903``): it owns the DAG tables as
buffers, packs per-slot inputs the same way and offers ``forward``,
``linear_readout`` and ``runtime_report``.  It is built from explicit DAG
tables (``from_tables``) or, as the reference's constructor takes it, from an
execution-plan document (``ye3t_amd.runtime.execution_plan.ExecutionPlan``).
"""

import hashlib

import numpy as np
import torch

from ye3t_amd.runtime import native

_PLANS = {}


def _table_arrays(tables, names=native.FA_TABLE_NAMES):
    out = {}
    for name in names:
        v = tables[name]
        out[name] = v.detach().cpu().numpy() if hasattr(v, "detach") else np.asarray(v)
    return out


def _cached_plan(names, tables, dims, dtype, device, make):
    arrays = _table_arrays(tables, names)
    h = hashlib.sha256()
    for name in names:
        a = np.ascontiguousarray(arrays[name])
        h.update(name.encode())
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    key = (names, h.hexdigest(), tuple(int(d) for d in dims), str(dtype), str(device))
    plan = _PLANS.get(key)
    if plan is None:
        import torch

        with torch.cuda.device(device):
            plan = make(arrays)
        if len(_PLANS) > 64:
            _PLANS.clear()
        _PLANS[key] = plan
    return plan


def plan_for(tables, source_dimension, input_dimension, workspace_dimension, output_dimension, dtype, device):
    """The device plan of these tables (validated and uploaded once, cached by
    content, dimensions, dtype and device)."""
    dims = (source_dimension, input_dimension, workspace_dimension, output_dimension)
    return _cached_plan(native.FA_TABLE_NAMES, tables, dims, dtype, device,
                        lambda a: native.FactorizedAngularPlanHandle(a, *dims, dtype))


def segmented_plan_for(tables, packed_input_dimension, total_source_count, workspace_dimension, output_dimension,
                       dtype, device):
    """The device plan of segmented tables (``native.SEGMENT_TABLE_NAMES``),
    cached like :func:`plan_for`."""
    dims = (packed_input_dimension, total_source_count, workspace_dimension, output_dimension)
    return _cached_plan(native.SEGMENT_TABLE_NAMES, tables, dims, dtype, device,
                        lambda a: native.FactorizedAngularSegmentedPlanHandle(a, *dims, dtype))


def _autograd():
    import torch

    class _FactorizedAngular(torch.autograd.Function):
        @staticmethod
        def forward(ctx, packed, plan):
            ctx.plan = plan
            ctx.save_for_backward(packed)
            return plan.forward(packed)

        @staticmethod
        def backward(ctx, grad):
            (packed,) = ctx.saved_tensors
            return ctx.plan.adjoint(grad.contiguous(), packed), None

    class _FactorizedAngularLinear(torch.autograd.Function):
        @staticmethod
        def forward(ctx, packed, weight, bias, plan):
            ctx.plan = plan
            ctx.save_for_backward(packed, weight)
            ctx.bias_shape = bias.shape
            return plan.linear(packed, weight, bias.item())

        @staticmethod
        def backward(ctx, grad):
            packed, weight = ctx.saved_tensors
            gx, gw, gb = ctx.plan.linear_adjoint(grad.contiguous(), packed, weight)
            return gx, gw.to(weight.dtype), gb.reshape(ctx.bias_shape), None

    return _FactorizedAngular, _FactorizedAngularLinear


_FN = None


def _fns():
    global _FN
    if _FN is None:
        _FN = _autograd()
    return _FN


def _check_device(packed):
    if not packed.is_cuda:
        raise NotImplementedError("factorized_angular: ye3t_amd implements the HIP device branch; CPU tensors are "
                                  "served by the reference CPU runtime")


def factorized_angular(packed_slots, node_offsets, node_dimensions, node_leaf_offsets, node_left, node_right,
                       node_coefficient_offsets, coefficient_rows, coefficient_columns, coefficient_values,
                       root_nodes, projection_values, source_dimension, workspace_dimension, output_dimension):
    """``ye3t_runtime::factorized_angular`` (schema ``execution_plan_torch.cpp:7586-7594``):
    ``[batch, output_dimension]`` features of ``packed_slots [batch,
    source_dimension * input_dimension]``; differentiable (conjugate-transpose
    adjoint)."""
    _check_device(packed_slots)
    S = int(source_dimension)
    if S <= 0:
        raise RuntimeError("source_dimension must be positive")
    if packed_slots.ndim != 2 or int(packed_slots.shape[1]) % S:
        raise RuntimeError("packed_slots width must be divisible by source_dimension")
    tables = dict(zip(native.FA_TABLE_NAMES, (node_offsets, node_dimensions, node_leaf_offsets, node_left,
                                              node_right, node_coefficient_offsets, coefficient_rows,
                                              coefficient_columns, coefficient_values, root_nodes,
                                              projection_values)))
    plan = plan_for(tables, S, int(packed_slots.shape[1]) // S, workspace_dimension, output_dimension,
                    packed_slots.dtype, packed_slots.device)
    return _fns()[0].apply(packed_slots.contiguous(), plan)


def factorized_angular_linear(packed_slots, node_offsets, node_dimensions, node_leaf_offsets, node_left, node_right,
                              node_coefficient_offsets, coefficient_rows, coefficient_columns, coefficient_values,
                              root_nodes, projection_values, source_dimension, workspace_dimension, weight, bias):
    """``ye3t_runtime::factorized_angular_linear``: ``bias + features @ weight``
    per sample without materialising the features; differentiable in the slots,
    the weight and the bias."""
    import torch

    _check_device(packed_slots)
    S = int(source_dimension)
    if packed_slots.ndim != 2 or int(packed_slots.shape[1]) % S:
        raise RuntimeError("packed_slots width must be divisible by source_dimension")
    tables = dict(zip(native.FA_TABLE_NAMES, (node_offsets, node_dimensions, node_leaf_offsets, node_left,
                                              node_right, node_coefficient_offsets, coefficient_rows,
                                              coefficient_columns, coefficient_values, root_nodes,
                                              projection_values)))
    weight = torch.as_tensor(weight, device=packed_slots.device).to(packed_slots.dtype)
    bias = torch.as_tensor(bias, device=packed_slots.device).to(packed_slots.dtype).reshape(())
    plan = plan_for(tables, S, int(packed_slots.shape[1]) // S, workspace_dimension, int(weight.numel()),
                    packed_slots.dtype, packed_slots.device)
    return _fns()[1].apply(packed_slots.contiguous(), weight, bias, plan)


def factorized_angular_segmented(packed_slots, segment_source_offsets, segment_input_offsets,
                                 segment_input_dimensions, segment_workspace_offsets, segment_workspace_dimensions,
                                 segment_node_offsets, segment_root_offsets, segment_projection_offsets,
                                 segment_projection_dimensions, segment_output_offsets, node_offsets, node_dimensions,
                                 node_leaf_offsets, node_left, node_right, node_coefficient_offsets,
                                 coefficient_rows, coefficient_columns, coefficient_values, root_nodes,
                                 root_projection_starts, root_projection_dimensions, root_output_offsets,
                                 projection_values, total_source_count, workspace_dimension, output_dimension):
    """``ye3t_runtime::factorized_angular_segmented`` (schema
    ``execution_plan_torch.cpp:7666-7679``): several factorized-angular DAGs
    over disjoint column ranges of ``packed_slots`` in one launch;
    ``[batch, output_dimension]``, differentiable (the segmented adjoint,
    ``:7681-7695``)."""
    _check_device(packed_slots)
    if packed_slots.ndim != 2:
        raise RuntimeError("packed_slots must be [batch, packed width]")
    values = (segment_source_offsets, segment_input_offsets, segment_input_dimensions, segment_workspace_offsets,
              segment_workspace_dimensions, segment_node_offsets, segment_root_offsets, segment_projection_offsets,
              segment_projection_dimensions, segment_output_offsets, node_offsets, node_dimensions,
              node_leaf_offsets, node_left, node_right, node_coefficient_offsets, coefficient_rows,
              coefficient_columns, coefficient_values, root_nodes, root_projection_starts,
              root_projection_dimensions, root_output_offsets, projection_values)
    tables = dict(zip(native.SEGMENT_TABLE_NAMES, values))
    plan = segmented_plan_for(tables, int(packed_slots.shape[1]), total_source_count, workspace_dimension,
                              output_dimension, packed_slots.dtype, packed_slots.device)
    return _fns()[0].apply(packed_slots.contiguous(), plan)


def segmented_tables(members):
    """Concatenated segmented tables of several DAGs, as the reference's
    segmented group builds them (``execution_plan.py:16672-16884``): each
    member (a :class:`YE3TFactorizedAngularModule`, or any object with its
    table attributes and dimensions) becomes one segment with
    the uniform root metadata (every root onto all of its P projection columns,
    root ``r``'s block at ``r * P * (2 L + 1)``).  Returns ``(tables, dims)``,
    ``dims`` = (packed_input_dimension, total_source_count,
    workspace_dimension, output_dimension)."""
    cols = {name: [] for name in native.SEGMENT_TABLE_NAMES}
    src, node_base, root_base, coef_base, in_base, ws_base, proj_base, out_base = 0, 0, 0, 0, 0, 0, 0, 0
    cols["segment_source_offsets"].append(0)
    cols["segment_node_offsets"].append(0)
    cols["segment_root_offsets"].append(0)
    cols["segment_output_offsets"].append(0)
    for k, m in enumerate(members):
        arr = {}
        for n in native.FA_TABLE_NAMES:
            v = getattr(m, n)
            arr[n] = v.detach().cpu().numpy() if hasattr(v, "detach") else np.asarray(v)
        S, D, W = int(m.source_dimension), int(m.input_dimension), int(m.workspace_dimension)
        if int(arr["projection_values"].size) % S:
            raise ValueError("factorized projection table does not match source dimension")
        P = int(arr["projection_values"].size) // S
        R = int(arr["root_nodes"].size)
        if R * P * int(m.magnetic_dimension) != int(m.output_dimension):
            raise ValueError("segmented factorized output does not match roots")
        src += S
        cols["segment_source_offsets"].append(src)
        cols["segment_input_offsets"].append(in_base)
        cols["segment_input_dimensions"].append(D)
        cols["segment_workspace_offsets"].append(ws_base)
        cols["segment_workspace_dimensions"].append(W)
        cols["segment_projection_offsets"].append(proj_base)
        cols["segment_projection_dimensions"].append(P)
        for n in ("node_offsets", "node_dimensions", "node_leaf_offsets", "node_left", "node_right"):
            cols[n].append(arr[n])
        offs = arr["node_coefficient_offsets"] + coef_base
        cols["node_coefficient_offsets"].append(offs if k == 0 else offs[1:])
        for n in ("coefficient_rows", "coefficient_columns", "coefficient_values", "root_nodes",
                  "projection_values"):
            cols[n].append(arr[n])
        cols["root_projection_starts"].append(np.zeros(R, dtype=np.int64))
        cols["root_projection_dimensions"].append(np.full(R, P, dtype=np.int64))
        cols["root_output_offsets"].append(np.arange(R, dtype=np.int64) * P * int(m.magnetic_dimension))
        node_base += int(arr["node_offsets"].size)
        root_base += R
        coef_base += int(arr["coefficient_values"].size)
        proj_base += int(arr["projection_values"].size)
        in_base += S * D
        ws_base += S * W
        out_base += int(m.output_dimension)
        cols["segment_node_offsets"].append(node_base)
        cols["segment_root_offsets"].append(root_base)
        cols["segment_output_offsets"].append(out_base)
    tables = {}
    for n, parts in cols.items():
        if n in ("coefficient_values", "projection_values"):
            tables[n] = np.concatenate(parts)
        elif parts and isinstance(parts[0], np.ndarray):
            tables[n] = np.concatenate(parts).astype(np.int64)
        else:
            tables[n] = np.asarray(parts, dtype=np.int64)
    return tables, (in_base, src, ws_base, out_base)


def _torch():
    return torch


class YE3TFactorizedAngularModule(torch.nn.Module):
    """Prepared factorized-angular DAG runtime (reference
    ``execution_plan.py:13550-13903``).

    ``YE3TFactorizedAngularModule(execution_plan, factorized_angular_plan_id=None,
    backend="auto", dtype=None, device=None)`` takes the reference constructor's
    arguments: an execution-plan document (an :class:`ExecutionPlan` or its
    ``to_dict()`` payload) and the id of one of its factorized-angular plans
    (optional when the document holds exactly one).  ``dtype`` defaults to
    complex128 when any synthesis coefficient has an imaginary part, else
    float64, as in the reference.  :meth:`from_tables` builds one from explicit
    DAG tables.  ``forward(slot_values)`` returns
    ``[..., roots * P, 2 L + 1]``; ``linear_readout(slot_values, weight, bias)``
    the fused readout ``features @ weight + bias``.  The module runs the HIP
    branch only: ``device`` defaults to the current CUDA device and a CPU device
    is refused.
    """

    def __init__(self, execution_plan=None, factorized_angular_plan_id=None, backend="auto", dtype=None,
                 device=None, *, tables=None, input_Ls=None, source_dimension=None, output_L=None, plan_hash=None,
                 plan_id=None):
        torch = _torch()
        super().__init__()
        backend = str(backend)
        if backend == "reference":
            raise NotImplementedError("backend='reference' selects the reference's Torch implementation "
                                      "(ye3t.runtime); ye3t_amd runs the native HIP branch only")
        if backend not in {"auto", "native"}:
            raise ValueError("backend must be 'auto', 'native', or 'reference'")
        dense_elements = None
        identity = {}
        if execution_plan is not None:
            if tables is not None:
                raise ValueError("give an execution plan or explicit tables, not both")
            from ye3t_amd.runtime import execution_plan as ep

            plan = execution_plan if isinstance(execution_plan, ep.ExecutionPlan) else \
                ep.ExecutionPlan.from_dict(execution_plan)
            _, meta = plan.factorized_angular_buffers(factorized_angular_plan_id)
            if dtype is None:
                dtype = torch.complex128 if meta["coefficient_complex"] else torch.float64
            tables, meta = plan.factorized_angular_buffers(factorized_angular_plan_id,
                                                           complex_values=dtype.is_complex)
            input_Ls, source_dimension, output_L = meta["input_Ls"], meta["source_dimension"], meta["output_L"]
            plan_hash, plan_id = plan.plan_hash, meta["plan_id"]
            dense_elements = meta["reference_dense_synthesis_element_count"]
            identity = {k: meta[k] for k in ("node_operator_hashes", "node_subtree_hashes")}
        elif tables is None:
            raise ValueError("YE3TFactorizedAngularModule needs an execution plan or explicit tables")
        values = np.asarray(tables["coefficient_values"])
        proj = np.asarray(tables["projection_values"])
        if dtype is None:
            dtype = torch.complex128 if (np.iscomplexobj(values) and np.any(values.imag != 0)) or \
                (np.iscomplexobj(proj) and np.any(proj.imag != 0)) else torch.float64
        device = torch.device("cuda" if device is None else device)
        if device.type != "cuda":
            raise NotImplementedError("YE3TFactorizedAngularModule: ye3t_amd implements the HIP device branch")
        if not dtype.is_complex:  # a real dtype keeps the real parts (reference execution_plan.py:11392-11397)
            tables = {k: (np.asarray(v).real if k in ("coefficient_values", "projection_values") else v)
                      for k, v in tables.items()}
        for name in native.FA_TABLE_NAMES:
            v = np.asarray(tables[name])
            t = torch.as_tensor(v, dtype=dtype if name in ("coefficient_values", "projection_values") else torch.int64,
                                device=device)
            self.register_buffer(name, t, persistent=False)
        self.input_Ls = tuple(int(x) for x in input_Ls)
        self.input_dimension = sum(2 * L + 1 for L in self.input_Ls)
        self.source_dimension = int(source_dimension)
        offs = np.asarray(tables["node_offsets"])
        dims = np.asarray(tables["node_dimensions"])
        self.workspace_dimension = int(offs[-1] + dims[-1])
        self.magnetic_dimension = 2 * int(output_L) + 1
        P = int(proj.size) // self.source_dimension
        self.logical_channel_tableau_dimension = int(np.asarray(tables["root_nodes"]).size) * P
        self.output_dimension = self.logical_channel_tableau_dimension * self.magnetic_dimension
        self.reference_dense_synthesis_element_count = None if dense_elements is None else int(dense_elements)
        self.node_operator_hashes = tuple(identity.get("node_operator_hashes", ()))
        self.node_subtree_hashes = tuple(identity.get("node_subtree_hashes", ()))
        self.plan_hash = None if plan_hash is None else str(plan_hash)
        self.factorized_angular_plan_id = None if plan_id is None else str(plan_id)
        self.requested_backend = backend
        self.resolved_backend = "native_hip"
        self.last_linear_readout_backend = None
        self.analysis_orientation = "conjugate_transpose"
        self._plan = plan_for(tables, self.source_dimension, self.input_dimension, self.workspace_dimension,
                              self.output_dimension, dtype, device)

    @classmethod
    def from_tables(cls, tables, *, input_Ls, source_dimension, output_L, **kw):
        return cls(tables=tables, input_Ls=input_Ls, source_dimension=source_dimension, output_L=output_L, **kw)

    @classmethod
    def from_execution_plan(cls, execution_plan, factorized_angular_plan_id=None, backend="auto", dtype=None,
                            device=None):
        """Same as the constructor's reference form."""
        return cls(execution_plan, factorized_angular_plan_id, backend=backend, dtype=dtype, device=device)

    def _packed_slots(self, slot_values):
        """Reference ``_packed_slots`` (``execution_plan.py:13688-13734``)."""
        torch = _torch()
        slots = tuple(slot_values)
        if len(slots) != len(self.input_Ls):
            raise ValueError("slot tensor count does not match input_Ls")
        if self.source_dimension == 1:
            leading = tuple(slots[0].shape[:-1])
        else:
            if slots[0].ndim < 2:
                raise ValueError("role-resolved slots require a source-coordinate axis")
            leading = tuple(slots[0].shape[:-2])
        work = []
        for slot, L in zip(slots, self.input_Ls):
            if int(slot.shape[-1]) != 2 * L + 1:
                raise ValueError("slot magnetic dimension does not match input_Ls")
            if self.source_dimension == 1:
                if tuple(slot.shape[:-1]) != leading:
                    raise ValueError("slot tensors must share leading dimensions")
                slot = slot.unsqueeze(-2)
            else:
                if tuple(slot.shape[:-2]) != leading:
                    raise ValueError("slot tensors must share leading dimensions")
                if int(slot.shape[-2]) != self.source_dimension:
                    raise ValueError("slot source axis does not match source assembly")
            work.append(slot.to(dtype=self.coefficient_values.dtype, device=self.coefficient_values.device))
        packed = torch.cat(tuple(work), dim=-1).reshape(-1, self.source_dimension * self.input_dimension)
        return packed.contiguous(), leading

    def forward(self, slot_values):
        packed, leading = self._packed_slots(slot_values)
        if int(packed.shape[0]) == 0:
            out = packed[:, :1].expand(-1, self.output_dimension)
        else:
            out = _fns()[0].apply(packed, self._plan)
        return out.reshape(leading + (self.logical_channel_tableau_dimension, self.magnetic_dimension))

    def linear_readout(self, slot_values, weight, bias):
        torch = _torch()
        packed, leading = self._packed_slots(slot_values)
        dt, dev = self.coefficient_values.dtype, self.coefficient_values.device
        weight = torch.as_tensor(weight, dtype=dt, device=dev)
        bias = torch.as_tensor(bias, dtype=dt, device=dev).reshape(())
        if weight.ndim != 1 or int(weight.numel()) != self.output_dimension:
            raise ValueError("weight must be a vector matching factorized output dimension")
        if int(packed.shape[0]) == 0:
            self.last_linear_readout_backend = "empty_batch"
            return packed[:, 0].reshape(leading)
        out = _fns()[1].apply(packed, weight, bias, self._plan)
        self.last_linear_readout_backend = "native_fused_factorized_linear"
        return out.reshape(leading)

    def runtime_report(self):
        return {
            "backend": self.resolved_backend, "native": True, "operation": "factorized_angular_source_analysis",
            "factorized_angular_plan_id": self.factorized_angular_plan_id, "plan_hash": self.plan_hash,
            "input_Ls": tuple(self.input_Ls), "source_dimension": int(self.source_dimension),
            "workspace_dimension": int(self.workspace_dimension), "runtime_device_scalar_metadata_reads": 0,
            "root_path_count": int(self.root_nodes.numel()), "unique_node_count": int(self.node_offsets.numel()),
            "reference_dense_synthesis_materialized": False,
            "reference_dense_synthesis_element_count": self.reference_dense_synthesis_element_count,
            "reference_dense_synthesis_bytes": 0,
            "per_forward_synthesis_table_reconstruction": False,
            "last_linear_readout_backend": self.last_linear_readout_backend,
            "linear_readout_auto_policy": "fuse",
            "analysis_orientation": self.analysis_orientation,
        }


class YE3TSegmentedFactorizedAngularModuleGroup(torch.nn.Module):
    """Several prepared factorized-angular plans evaluated by one segmented
    launch (reference ``_YE3TSegmentedFactorizedAngularModuleGroup``,
    ``execution_plan.py:16632-17100``).

    ``forward(slot_values_by_plan)`` takes one slot tuple per member module
    (shared leading shape) and returns one ``[..., roots * P, 2 L + 1]``
    tensor per member; ``forward_packed`` returns the concatenated
    ``[batch, output_dimension]`` rows."""

    def __init__(self, modules, plan_indices=None, enable_native=True):
        super().__init__()
        modules = tuple(modules)
        if not modules:
            raise ValueError("segmented factorized group requires at least one plan")
        plan_indices = tuple(range(len(modules))) if plan_indices is None else tuple(int(v) for v in plan_indices)
        if len(plan_indices) != len(modules):
            raise ValueError("segmented factorized plan indices must match modules")
        first = modules[0]
        if any(m.coefficient_values.dtype != first.coefficient_values.dtype or
               m.coefficient_values.device != first.coefficient_values.device for m in modules[1:]):
            raise ValueError("segmented factorized plans must share backend, dtype, and device")
        if not enable_native:
            raise NotImplementedError("ye3t_amd runs the native segmented launch only")
        object.__setattr__(self, "_source_modules", modules)
        self.plan_indices = plan_indices
        tables, dims = segmented_tables(modules)
        self.input_dimension, self.total_source_count, self.workspace_dimension, self.output_dimension = dims
        self._tables = tables
        dt, dev = first.coefficient_values.dtype, first.coefficient_values.device
        self._plan = segmented_plan_for(tables, *dims, dt, dev)
        starts = tables["segment_output_offsets"]
        self.output_slices = tuple({"plan_index": int(i), "start": int(starts[k]), "stop": int(starts[k + 1]),
                                    "logical_channel_tableau_dimension": int(m.logical_channel_tableau_dimension),
                                    "magnetic_dimension": int(m.magnetic_dimension), "plan_hash": str(m.plan_hash)}
                                   for k, (m, i) in enumerate(zip(modules, plan_indices)))
        self.last_backend = None

    def native_tables(self):
        """The op's table arguments (numpy), in the reference schema's order."""
        return tuple(self._tables[n] for n in native.SEGMENT_TABLE_NAMES)

    def forward_packed(self, slot_values_by_plan):
        slot_values_by_plan = tuple(tuple(v) for v in slot_values_by_plan)
        if len(slot_values_by_plan) != len(self._source_modules):
            raise ValueError("segmented factorized input count does not match plans")
        packed, leading = [], []
        for m, values in zip(self._source_modules, slot_values_by_plan):
            p, lead = m._packed_slots(values)
            packed.append(p)
            leading.append(tuple(lead))
        if any(s != leading[0] for s in leading[1:]):
            raise ValueError("segmented factorized plans require matching leading shapes")
        packed = _torch().cat(tuple(packed), dim=1).contiguous()
        self.last_backend = "native_destination_segmented_factorized_angular"
        if int(packed.shape[0]) == 0:
            return packed.new_zeros((0, self.output_dimension))
        return _fns()[0].apply(packed, self._plan)

    def forward(self, slot_values_by_plan):
        slot_values_by_plan = tuple(tuple(v) for v in slot_values_by_plan)
        out = self.forward_packed(slot_values_by_plan)
        first = slot_values_by_plan[0][0]
        lead = tuple(first.shape[:-1] if int(self._source_modules[0].source_dimension) == 1 else first.shape[:-2])
        return tuple(out[:, r["start"]:r["stop"]].reshape(lead + (r["logical_channel_tableau_dimension"],
                                                                  r["magnetic_dimension"]))
                     for r in self.output_slices)

    def runtime_report(self):
        return {
            "runtime": "YE3TSegmentedFactorizedAngularModuleGroup",
            "member_plan_count": len(self._source_modules), "member_plan_indices": tuple(self.plan_indices),
            "member_plan_hashes": tuple(str(m.plan_hash) for m in self._source_modules),
            "source_dimensions": tuple(int(m.source_dimension) for m in self._source_modules),
            "total_source_count": int(self.total_source_count), "input_dimension": int(self.input_dimension),
            "workspace_dimension": int(self.workspace_dimension), "output_dimension": int(self.output_dimension),
            "native_enabled": True, "native_call_count": 1, "last_backend": self.last_backend,
        }
