"""Scheduled radial-angular edge channels on the GPU, through the C ABI.

fp64: bit for bit the oracle (itself the reference core bit for bit,
``tests/test_scheduled_channels.py``).  fp32: bit for bit the same products
rounded in fp32 one at a time (the reference core's ``float`` instantiation
computes in ``float`` with no fused multiply-adds).  Also the Torch operator,
empty shapes and out-of-range indices refused before any launch.
"""

import numpy as np
import pytest

import oracle
from tests._util import flush
from tests.test_scheduled_channels import _case

pytestmark = pytest.mark.gpu


def _device_case(case, dtype, dev):
    import torch

    out = {}
    for k, v in case.items():
        if v.dtype.kind == "f":
            out[k] = torch.as_tensor(v, dtype=dtype, device=dev)
        else:
            out[k] = torch.as_tensor(v, dtype=torch.int64, device=dev)
    return out


def _f32_restatement(c):
    f = {k: (v.astype(np.float32) if v.dtype.kind == "f" else v) for k, v in c.items()}
    E, K = f["radial_values"].shape[0], f["channel_scales"].shape[0]
    v = np.zeros((E, K), np.float32)
    d = np.zeros((E, K, 3), np.float32)
    for e in range(E):
        for k in range(K):
            t = f["channel_types"][k]
            if t >= 0 and f["edge_types"][e] != t:
                continue
            r = f["radial_values"][e, f["channel_radial_indices"][k]]
            dr = f["radial_derivatives"][e, f["channel_radial_indices"][k]]
            a = f["angular_values"][e, f["channel_angular_indices"][k]]
            da = f["angular_derivatives"][e, f["channel_angular_indices"][k]]
            sc = f["channel_scales"][k]
            v[e, k] = np.float32(np.float32(sc * r) * a)
            for x in range(3):
                d[e, k, x] = np.float32(sc * np.float32(np.float32(np.float32(dr * f["radial_directions"][e, x]) * a)
                                                        + np.float32(r * da[x])))
    return v, d


@pytest.mark.parametrize("seed", [0, 1])
def test_scheduled_channels_match_the_oracle_bit_for_bit(gpu, seed):
    flush(f"scheduled channels seed {seed}")
    import torch

    from ye3t_amd import runtime
    from ye3t_amd.runtime import torch_ops

    case = _case(seed, E=300, K=23)
    dev = _device_case(case, torch.float64, gpu)
    v, d = runtime.scheduled_radial_angular_channels_with_derivative(*dev.values())
    rv, rd = oracle.scheduled_channels(**case)
    assert np.array_equal(v.cpu().numpy(), rv) and np.array_equal(d.cpu().numpy(), rd)
    torch_ops.register()
    v2, d2 = torch.ops.ye3t_runtime.scheduled_radial_angular_channels_with_derivative(*dev.values())
    assert torch.equal(v, v2) and torch.equal(d, d2)

    dev32 = _device_case(case, torch.float32, gpu)
    v32, d32 = runtime.scheduled_radial_angular_channels_with_derivative(*dev32.values())
    fv, fd = _f32_restatement(case)
    assert np.array_equal(v32.cpu().numpy(), fv) and np.array_equal(d32.cpu().numpy(), fd)


def test_scheduled_channels_empty_and_refused(gpu):
    flush("scheduled channels: empty shapes, refused indices")
    import torch

    from ye3t_amd import runtime

    case = _device_case(_case(4, E=0), torch.float64, gpu)
    v, d = runtime.scheduled_radial_angular_channels_with_derivative(*case.values())
    assert v.shape == (0, 11) and d.shape == (0, 11, 3)
    case = _device_case(_case(4, K=0), torch.float64, gpu)
    v, d = runtime.scheduled_radial_angular_channels_with_derivative(*case.values())
    assert v.shape == (40, 0) and d.shape == (40, 0, 3)
    case = _device_case(_case(4), torch.float64, gpu)
    case["channel_angular_indices"] = case["channel_angular_indices"] + 100
    with pytest.raises(ValueError, match="channel angular indices must lie in the angular table"):
        runtime.scheduled_radial_angular_channels_with_derivative(*case.values())


def test_scheduled_channels_autograd(gpu):
    """The Torch operator's backward: gradients in the radial table, the
    angular table and the channel scales equal autograd through the
    reference's value formula (``execution_plan.py:7007-7033``) in fp64, the
    derivative output is not differentiable, and ``opcheck`` passes."""
    flush("scheduled channels: autograd and opcheck")
    import torch

    from ye3t_amd.runtime import torch_ops

    torch_ops.register()
    op = torch.ops.ye3t_runtime.scheduled_radial_angular_channels_with_derivative
    case = _device_case(_case(6, E=64, K=17), torch.float64, gpu)
    leaves = {k: case[k].clone().requires_grad_(True) for k in ("radial_values", "angular_values", "channel_scales")}
    args = dict(case, **leaves)
    values, derivs = op(*args.values())
    assert not derivs.requires_grad
    w = torch.randn_like(values)
    got = torch.autograd.grad((values * w).sum(), tuple(leaves.values()))
    ref_leaves = {k: case[k].clone().requires_grad_(True) for k in leaves}
    act = ((case["channel_types"] < 0).unsqueeze(0)
           | (case["edge_types"].unsqueeze(1) == case["channel_types"].unsqueeze(0))).to(torch.float64)
    ref_values = (ref_leaves["radial_values"].index_select(1, case["channel_radial_indices"])
                  * ref_leaves["angular_values"].index_select(1, case["channel_angular_indices"])
                  * act * ref_leaves["channel_scales"].unsqueeze(0))
    torch.testing.assert_close(values, ref_values.detach(), rtol=1e-14, atol=1e-14)
    want = torch.autograd.grad((ref_values * w).sum(), tuple(ref_leaves.values()))
    for g, r in zip(got, want):
        torch.testing.assert_close(g, r, rtol=1e-13, atol=1e-13)
    result = torch.library.opcheck(op.default, tuple(args.values()), raise_exception=False)
    assert all(v == "SUCCESS" for v in result.values()), result
