"""MACEField response on the GPU against the oracle
(_compute_prepared_factorized_field_response, pybind mace_kokkos.cpp:
1865-1879, 2160-2167, 2226-2349; mace_kokkos_response.tpp; the calculator's
becs and polarizability, calculator.py:3783-3817): the field Hessian, the
per-edge force derivative and the Born charge bins in the three model kinds
(L_max 1, density-scaled with ZBL, L_max 2 with a residual), the host-graph
and "current" forms, the evaluation's results left as they were, and the
refusals.

Tolerances: the response is a second derivative accumulated in FP32 (the
reference's Precision) with FP64 readouts and sums; the FP32 oracle lands
within 2e-4 of the FP64 one, and the device within 2e-4 of each quantity's
largest magnitude (measured: 1e-7 to 1.2e-5).
"""

import numpy as np
import pytest

from test_gpu_parity import _system

pytestmark = pytest.mark.gpu

FIELD = np.array([0.12, -0.21, 0.27])
TOL = 2e-4


def _prepare(ev, s, types, skin=0.5):
    cell = np.asarray(s["cell"], float)
    return ev._prepare_periodic_factorized_graph(types, s["positions"], cell, np.linalg.inv(cell), ev.r_cut + skin)


def _close(name, got, want):
    scale = max(float(np.max(np.abs(want))), 1e-30)
    err = float(np.max(np.abs(np.asarray(got) - want))) / scale
    print("%s relative max err %.3e (scale %.3e)" % (name, err, scale))
    assert err < TOL, (name, err)


@pytest.mark.parametrize("model", ["tiny_field", "tiny_field_scaled", "field_l2"])
def test_response_matches_oracle(request, model):
    from oracle import oracle
    from symmetrix.mace_kokkos import MACEKokkosFloat
    path = request.getfixturevalue(model + "_model_path")
    s = _system("tiny")
    n = len(s["numbers"])
    om = oracle.OracleModel(path, fp64=True)
    ref = oracle.field_response_system(om, s, FIELD)
    ev = MACEKokkosFloat(path)
    types = om.types_of(s["numbers"])
    g = _prepare(ev, s, types)
    gen = g["generation"]
    ev._compute_prepared_factorized_positions_field(gen, s["positions"], FIELD)
    e0 = np.array(ev.node_energies)
    f0 = ev._reduce_atom_forces(n, None, None, gen)
    adj0 = ev.electric_field_adj
    # the Hessian alone
    ev._compute_prepared_factorized_field_response(gen, FIELD, False)
    hess = np.asarray(ev.electric_field_hessian).reshape(3, 3)
    _close("hessian", hess, ref["hessian"])
    assert len(ev.electric_field_force_derivative) == 0 and ev.electric_field_bec_bins.shape == (0, 3, 3)
    # with the per-edge force derivative (the graph is the oracle's, edge for edge)
    ev._compute_prepared_factorized_field_response(gen, FIELD, True)
    np.testing.assert_array_equal(np.asarray(ev.electric_field_hessian).reshape(3, 3), hess)
    fd = np.asarray(ev.electric_field_force_derivative).reshape(3, -1, 3)
    assert fd.shape == ref["force_derivative"].shape
    _close("force_derivative", fd, ref["force_derivative"])
    # the device bins: the Born charges, equal to the host reduction of the per-edge values
    ev._compute_prepared_factorized_field_response(gen, FIELD, True, scatter_bec_bins=True)
    bins = ev.electric_field_bec_bins
    assert bins.shape == (n, 3, 3) and len(ev.electric_field_force_derivative) == 0
    _close("bec", bins, ref["bec"])
    gr = ref["graph"]
    host = np.stack([oracle.reduce_forces(n, gr["receivers"], gr["sources"], fd[c]) for c in range(3)], axis=1)
    np.testing.assert_allclose(bins, host, rtol=0, atol=1e-9 * max(1.0, np.max(np.abs(host))))
    # the evaluation's results are as they were
    np.testing.assert_array_equal(ev.node_energies, e0)
    np.testing.assert_array_equal(ev._reduce_atom_forces(n, None, None, gen), f0)
    np.testing.assert_array_equal(ev.electric_field_adj, adj0)
    # the "current" forms read the same prepared evaluation
    ev._compute_current_electric_field_bec_bins(n, types, None, None, None, None, None, FIELD, gen)
    np.testing.assert_array_equal(ev.electric_field_bec_bins, bins)


def _bench_system():
    from symmetrix import systems
    return systems.srtio3_supercell(10, sigma=0.05, seed=0)


def _device_response(ev, s, field):
    lut = {int(z): i for i, z in enumerate(ev.atomic_numbers)}
    types = np.array([lut[int(z)] for z in s["numbers"]], np.int32)
    g = _prepare(ev, s, types)
    ev._compute_prepared_factorized_positions_field(g["generation"], s["positions"], field)
    ev._compute_prepared_factorized_field_response(g["generation"], field, True, scatter_bec_bins=True)
    return np.asarray(ev.electric_field_hessian).reshape(3, 3), ev.electric_field_bec_bins


def test_response_at_the_benchmark_size(field_l2_model_path, tmp_path):
    """The 5,000-atom SrTiO3 system of the benchmark (272,436 edges):
    against the oracle on a 4x4x4 cell of the same crystal, and at full size
    the properties the mathematics fixes: a symmetric Hessian, Born charges
    summing to zero, and rotating atoms and field together rotating both
    (the model's residual kept to its scalar block, as a trained one is)."""
    import json
    from oracle import oracle
    from symmetrix import systems
    from symmetrix.mace_kokkos import MACEKokkosFloat
    with open(field_l2_model_path) as f:
        doc = json.load(f)
    LM, C = (doc["L_max"] + 1) ** 2, doc["num_channels"]
    b = np.asarray(doc["H1_first_residual_weights"], float).reshape(-1, LM, C)
    b[:, 1:, :] = 0.0
    doc["H1_first_residual_weights"] = b.ravel().tolist()
    path = str(tmp_path / "scalar_residual.json")
    with open(path, "w") as f:
        json.dump(doc, f)
    ev = MACEKokkosFloat(path)
    mid = systems.srtio3_supercell(4, sigma=0.05, seed=0)
    ref = oracle.field_response_system(oracle.OracleModel(path, fp64=True), mid, FIELD)
    hess, bins = _device_response(ev, mid, FIELD)
    _close("hessian 320 atoms", hess, ref["hessian"])
    _close("bec 320 atoms", bins, ref["bec"])
    s = _bench_system()
    hess, bins = _device_response(ev, s, FIELD)
    hs, zs = np.max(np.abs(hess)), np.max(np.abs(bins))
    print("5000 atoms: hessian scale %.3e, asymmetry %.3e; bec scale %.3e, sum %.3e" % (
        hs, np.max(np.abs(hess - hess.T)), zs, np.max(np.abs(bins.sum(axis=0)))))
    assert np.max(np.abs(hess - hess.T)) < TOL * hs
    assert np.max(np.abs(bins.sum(axis=0))) < 1e-9 * len(bins) * zs
    R = e3_rotation()
    rot = dict(s, positions=s["positions"] @ R.T, cell=s["cell"] @ R.T)
    hess_r, bins_r = _device_response(ev, rot, R @ FIELD)
    _close("rotated hessian", hess_r, R @ hess @ R.T)
    _close("rotated bec", bins_r, np.einsum("ab,ibc,dc->iad", R, bins, R))


def e3_rotation():
    from symmetrix import e3
    return e3.random_rotation(np.random.default_rng(21))


def test_host_graph_response(tiny_field_scaled_model_path):
    """compute_electric_field_hessian / _force_derivative: the host graph
    evaluated in the field, then its response."""
    from oracle import oracle
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    om = oracle.OracleModel(tiny_field_scaled_model_path, fp64=True)
    ref = oracle.field_response_system(om, s, FIELD)
    types = om.types_of(s["numbers"])
    gr = ref["graph"]
    n = len(types)
    ev = MACEKokkosFloat(tiny_field_scaled_model_path)
    args = (n, types, gr["num_neigh"], gr["sources"], types[gr["sources"]], ref["xyz"], ref["r"], FIELD)
    ev.compute_electric_field_hessian(*args)
    _close("hessian", np.asarray(ev.electric_field_hessian).reshape(3, 3), ref["hessian"])
    ev.compute_electric_field_force_derivative(*args)
    _close("force_derivative", np.asarray(ev.electric_field_force_derivative).reshape(3, -1, 3),
           ref["force_derivative"])


def test_response_refusals(tiny_field_model_path, tiny_model_path):
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    ev = MACEKokkosFloat(tiny_field_model_path)
    lut = {int(z): i for i, z in enumerate(ev.atomic_numbers)}
    types = np.array([lut[int(z)] for z in s["numbers"]], np.int32)
    n = len(types)
    g = _prepare(ev, s, types)
    gen = g["generation"]
    with pytest.raises(RuntimeError, match="completed field evaluation"):
        ev._compute_prepared_factorized_field_response(gen, FIELD, True)
    with pytest.raises(RuntimeError, match="no MACEField response"):
        ev.electric_field_hessian
    ev._compute_prepared_factorized_positions_field(gen, s["positions"], FIELD)
    with pytest.raises(ValueError, match="differs"):
        ev._compute_prepared_factorized_field_response(gen, FIELD + 0.01, True)
    with pytest.raises(ValueError, match="graph-level"):
        ev._compute_prepared_factorized_field_response(gen, np.tile(FIELD, (n, 1)), True)
    with pytest.raises(ValueError, match="stale"):
        ev._compute_prepared_factorized_field_response(gen + 7, FIELD, True)
    with pytest.raises(RuntimeError, match="completed prepared"):
        ev._compute_current_electric_field_hessian(n, types, None, None, None, None, None, FIELD, 0)
    # an evaluation in a per-node field has no graph-level response
    ev._compute_prepared_factorized_positions_field(gen, s["positions"], np.tile(FIELD, (n, 1)))
    with pytest.raises(ValueError, match="graph-level field"):
        ev._compute_prepared_factorized_field_response(gen, FIELD, False)
    plain = MACEKokkosFloat(tiny_model_path)
    gp = _prepare(plain, s, types)
    plain._compute_prepared_factorized_positions(gp["generation"], s["positions"])
    with pytest.raises(ValueError, match="field coupling"):
        plain._compute_prepared_factorized_field_response(gp["generation"], FIELD, False)


def test_calculator_becs_and_polarizability(tiny_field_scaled_model_path):
    from oracle import oracle
    from symmetrix.calculator import Symmetrix
    s = _system("tiny")
    n = len(s["numbers"])
    om = oracle.OracleModel(tiny_field_scaled_model_path, fp64=True)
    ref = oracle.field_response_system(om, s, FIELD)
    V = abs(np.linalg.det(np.asarray(s["cell"], float)))
    calc = Symmetrix(tiny_field_scaled_model_path, electric_field=FIELD)
    assert {"becs", "polarizability"} <= set(calc.implemented_properties)
    res = calc.calculate(dict(s), ["energy", "forces", "becs", "polarizability"])
    eps0 = 8.8541878128e-12 / 1.602176634e-19 / 1e10
    _close("polarizability", res["polarizability"], (-ref["hessian"] / V / eps0).reshape(9))
    _close("becs", res["becs"], ref["bec"].reshape(n, 9))
    # the default calculation leaves the response out
    plain = calc.calculate(dict(s))
    assert "becs" not in plain and "polarizability" not in plain
