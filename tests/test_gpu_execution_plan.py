"""The factorized-angular module built from reference-written execution plans, on the GPU.

Each case of ``tests/golden/execution_plan_factorized_v1.json`` is a plan
document the reference serialized and the reference Torch branch's results on
seeded slots.  The module is constructed as the reference's is
(``YE3TFactorizedAngularModule(execution_plan, backend="native", dtype=...)``)
and runs the HIP ``factorized_angular`` kernels: forward, the autograd slot
gradient and the fused linear readout must match the reference branch to
1e-12 absolute (the reference's own native-vs-reference bar,
``tests/test_execution_plan_native.py:6410-6420``).
"""

import json

import numpy as np
import pytest

from tests._util import flush
from tests.test_execution_plan_loader import DATA, _arr

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", DATA["cases"], ids=lambda c: f"{c['plan']}-{c['dtype']}")
def test_module_from_reference_plan_matches_reference_branch(gpu, case):
    flush(f"module from reference plan {case['plan']} {case['dtype']}")
    import torch

    from ye3t_amd.runtime import YE3TFactorizedAngularModule

    rec = DATA["plans"][case["plan"]]
    dt = {"float64": torch.float64, "complex128": torch.complex128}[case["dtype"]]
    mod = YE3TFactorizedAngularModule(json.loads(rec["plan_json"]), backend="native", dtype=dt, device=gpu)
    report = mod.runtime_report()
    assert report["plan_hash"] == rec["plan_hash"]
    assert report["factorized_angular_plan_id"] == rec["factorized_angular_plan_id"]
    assert report["reference_dense_synthesis_element_count"] == rec["buffers"]["reference_dense_synthesis_element_count"]
    assert list(mod.node_subtree_hashes) == rec["buffers"]["node_subtree_hashes"]
    slots = tuple(torch.as_tensor(_arr(s, case["dtype"]), dtype=dt, device=gpu).requires_grad_(True)
                  for s in case["slots"])
    out = mod(slots)
    expected = torch.as_tensor(_arr(case["output"], case["dtype"]), dtype=dt)
    assert tuple(out.shape) == tuple(expected.shape)
    torch.testing.assert_close(out.detach().cpu(), expected, rtol=0.0, atol=1e-12)
    cot = torch.as_tensor(_arr(case["output_cotangent"], case["dtype"]), dtype=dt, device=gpu)
    grads = torch.autograd.grad(out, slots, cot)
    for g, e in zip(grads, case["slot_adjoints"]):
        torch.testing.assert_close(g.cpu(), torch.as_tensor(_arr(e, case["dtype"]), dtype=dt), rtol=0.0, atol=1e-12)
    w = _arr(case["readout_weight"], case["dtype"])
    b = _arr(case["readout_bias"], case["dtype"])
    lin = mod.linear_readout(tuple(s.detach() for s in slots), w, b)
    assert mod.last_linear_readout_backend == "native_fused_factorized_linear"
    torch.testing.assert_close(lin.cpu(), torch.as_tensor(_arr(case["readout"], case["dtype"]), dtype=dt),
                               rtol=0.0, atol=1e-12)
    assert np.isfinite(lin.abs().sum().item())
