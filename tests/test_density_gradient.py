"""Oracle of the stage-1 edge-vector gradient (forces), pinned on the CPU.

``oracle.ace_density_edge_gradient`` restates the reference's force chain
(radial and harmonic derivative tables, the scheduled channel derivative of
``ye3t_runtime_core.cpp:1550-1604``, the density adjoint gathered to edges).
It is pinned by the derivative of the pinned density oracle itself: a
five-point directional derivative of ``<gA, A(v + t dv)>`` (smooth away from
the cutoff, where the constant radial function R_0 switches off), for the
three channel modes (one-hot species, node features with a radial mix, one
channel).  A planted mistake (the adjoint's channels permuted) fails the same
check.
"""

import numpy as np
import pytest

import oracle
from ye3t_amd.ace.workloads import DensityWorkload


def _workload(mode, n_max=6, l_max=4):
    kw = {"species": dict(species_count=4), "features": dict(node_channels=5), "single": {}}[mode]
    return DensityWorkload(30, 7, 5.0, 0.8, n_max, l_max, config_id=1, **kw).generate()


def _directional(inp, gA, dv, h=1e-4):
    def f(t):
        d = dict(inp)
        d["edge_vectors"] = inp["edge_vectors"] + t * dv
        return float(np.sum(gA * oracle.ace_density(d)))

    return (f(-2 * h) - 8 * f(-h) + 8 * f(h) - f(2 * h)) / (12 * h)


@pytest.mark.parametrize("mode", ["species", "features", "single"])
@pytest.mark.parametrize("l_max", [0, 2, 4])
def test_edge_gradient_is_the_directional_derivative(mode, l_max):
    inp = _workload(mode, l_max=l_max)
    rng = np.random.default_rng(7 + l_max)
    gA = rng.normal(size=oracle.ace_density(inp).shape)
    dv = rng.normal(size=inp["edge_vectors"].shape)
    r = np.linalg.norm(inp["edge_vectors"], axis=1)
    dv[r > 0.97 * inp["cutoff"]] = 0.0
    g = oracle.ace_density_edge_gradient(inp, gA)
    assert g.shape == (inp["edge_count"], 3)
    fd = _directional(inp, gA, dv)
    an = float(np.sum(g * dv))
    assert abs(fd - an) <= 1e-9 * max(1.0, abs(an))
    if mode != "single":
        planted = oracle.ace_density_edge_gradient(inp, np.roll(gA, 1, axis=1))
        assert abs(fd - float(np.sum(planted * dv))) > 1e-6 * max(1.0, abs(an))


def test_edges_beyond_the_cutoff_have_no_gradient():
    inp = _workload("species")
    v = inp["edge_vectors"].copy()
    v[:5] *= 1.5 * inp["cutoff"] / np.linalg.norm(v[:5], axis=1, keepdims=True)
    inp["edge_vectors"] = v
    gA = np.random.default_rng(0).normal(size=oracle.ace_density(inp).shape)
    g = oracle.ace_density_edge_gradient(inp, gA)
    assert np.all(g[:5] == 0.0) and np.any(g[5:] != 0.0)
