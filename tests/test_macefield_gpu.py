"""MACEField models on the GPU against the oracle (field_coupling.hpp;
mace.cpp:322-395, 1147-1240; pybind mace_kokkos.cpp:1837-1864, 2156):
energies, forces, stress and dE/dE in a graph field and in a per-node field,
the positions and xyz forms, the field kept for later calls, and the
refusals (no field, a field for a plain model, the tiled plans)."""

import numpy as np
import pytest

from test_gpu_parity import _assert_efs, _stage_err, _system

pytestmark = pytest.mark.gpu

FIELD = np.array([0.12, -0.21, 0.27])


def _prepare(ev, s, types, skin=0.5):
    cell = np.asarray(s["cell"], float)
    return ev._prepare_periodic_factorized_graph(types, s["positions"], cell, np.linalg.inv(cell), ev.r_cut + skin)


def _results(ev, s, gen, n):
    e = ev.node_energies
    f = ev._reduce_atom_forces(n, None, None, gen)
    st = ev._reduce_stress(abs(np.linalg.det(np.asarray(s["cell"], float))), None, gen)
    return e, f, st


@pytest.mark.parametrize("model", ["tiny_field", "field_l2"])
def test_field_model_matches_oracle(request, model):
    from oracle import oracle
    from symmetrix.mace_kokkos import MACEKokkosFloat
    path = request.getfixturevalue(model + "_model_path")
    s = _system("tiny")
    n = len(s["numbers"])
    om = oracle.OracleModel(path)
    ev = MACEKokkosFloat(path)
    assert ev.has_field_coupling
    types = om.types_of(s["numbers"])
    g = _prepare(ev, s, types)
    per = np.tile(FIELD, (n, 1)) + 0.05 * np.random.default_rng(4).normal(size=(n, 3))
    for field in (FIELD, per):
        ref = oracle.evaluate_system(om, s, skin=0.5, field=field)
        ev._compute_prepared_factorized_positions_field(g["generation"], s["positions"], field)
        e, f, st = _results(ev, s, g["generation"], n)
        _assert_efs(ref, e, f, st, n)
        np.testing.assert_allclose(e, ref["energies"], rtol=0, atol=1e-4)
        err = _stage_err(ev._stage("H1").astype(np.float64), om.stage("H1"))
        print("H1 relative max err %.3e" % err)
        assert err < 1e-4
        adj = ev.electric_field_adj
        assert adj.shape == (np.asarray(field).size,)
        scale = max(np.max(np.abs(ref["field_adj"])), 1e-30)
        print("field_adj relative max err %.3e" % (np.max(np.abs(adj - ref["field_adj"])) / scale))
        np.testing.assert_allclose(adj, ref["field_adj"], rtol=0, atol=2e-5 * scale)
    # the field stays set: a plain positions call repeats the last result
    ev._compute_prepared_factorized_positions(g["generation"], s["positions"])
    e2, f2, s2 = _results(ev, s, g["generation"], n)
    np.testing.assert_array_equal(e2, e)
    np.testing.assert_array_equal(f2, f)
    # the xyz form of the same evaluation
    ref = oracle.evaluate_system(om, s, skin=0.5, field=FIELD)
    ev._compute_prepared_factorized_field(g["generation"], ref["xyz"], ref["r"], FIELD)
    e3, f3, s3 = _results(ev, s, g["generation"], n)
    _assert_efs(ref, e3, f3, s3, n)


def test_field_refusals(tiny_field_model_path, tiny_model_path):
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    ev = MACEKokkosFloat(tiny_field_model_path)
    lut = {int(z): i for i, z in enumerate(ev.atomic_numbers)}
    types = np.array([lut[int(z)] for z in s["numbers"]], np.int32)
    g = _prepare(ev, s, types)
    with pytest.raises(ValueError, match="electric field"):
        ev._compute_prepared_factorized_positions(g["generation"], s["positions"])
    with pytest.raises(ValueError, match="shape"):
        ev._compute_prepared_factorized_positions_field(g["generation"], s["positions"], np.zeros(6))
    plain = MACEKokkosFloat(tiny_model_path)
    assert not plain.has_field_coupling
    gp = _prepare(plain, s, types)
    with pytest.raises(ValueError, match="no field coupling"):
        plain._compute_prepared_factorized_positions_field(gp["generation"], s["positions"], FIELD)
    tiled = MACEKokkosFloat(tiny_field_model_path)
    tiled.set_execution_plan_request("capacity", 64)
    with pytest.raises(ValueError, match="field coupling"):
        _prepare(tiled, s, types)


def test_calculator_polarization_in_a_field(tiny_field_model_path):
    """The calculator on a MACEField model (calculator.py:2774-2805,
    3672-3678): the field from the keyword or the atoms' info, the
    polarization -dE/dE / V, energies and forces against the oracle."""
    from oracle import oracle
    from symmetrix.calculator import Symmetrix
    s = _system("tiny")
    om = oracle.OracleModel(tiny_field_model_path)
    ref = oracle.evaluate_system(om, s, skin=0.5, field=FIELD)
    V = abs(np.linalg.det(np.asarray(s["cell"], float)))
    n = len(s["numbers"])
    calc = Symmetrix(tiny_field_model_path, electric_field=FIELD)
    assert "polarization" in calc.implemented_properties
    res = calc.calculate(dict(s))
    assert abs(res["energy"] - ref["energy"]) / n < 1e-5
    assert np.max(np.abs(res["forces"] - ref["forces"])) < 1e-4
    scale = np.max(np.abs(ref["field_adj"]))
    np.testing.assert_allclose(res["polarization"], -ref["field_adj"] / V, rtol=0, atol=2e-5 * scale / V)
    # the field from the atoms' info; none means zero
    info = Symmetrix(tiny_field_model_path).calculate(dict(s, info={"electric_field": FIELD.reshape(1, 3)}))
    np.testing.assert_allclose(info["forces"], res["forces"], rtol=0, atol=1e-9)
    zero = Symmetrix(tiny_field_model_path).calculate(dict(s))
    z_ref = oracle.evaluate_system(om, s, skin=0.5, field=np.zeros(3))
    assert abs(zero["energy"] - z_ref["energy"]) / n < 1e-5
    with pytest.raises(ValueError, match="per-atom"):
        Symmetrix(tiny_field_model_path, electric_field=np.zeros((n, 3))).calculate(dict(s))


def test_unprepared_call_in_a_field(tiny_field_model_path, tiny_model_path):
    """compute_node_energies_forces_field (pybind mace_kokkos.cpp:2205-2225):
    the host-graph call of a MACEField model, against the oracle."""
    from oracle import oracle
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    om = oracle.OracleModel(tiny_field_model_path)
    ref = oracle.evaluate_system(om, s, skin=0.5, field=FIELD)
    types = om.types_of(s["numbers"])
    g = ref["graph"]
    n = len(types)
    ev = MACEKokkosFloat(tiny_field_model_path)
    ev.compute_node_energies_forces_field(n, types, g["num_neigh"], g["sources"], types[g["sources"]], ref["xyz"],
                                          ref["r"], FIELD)
    np.testing.assert_allclose(ev.node_energies, ref["energies"], rtol=0, atol=1e-4)
    scale = np.max(np.abs(ref["field_adj"]))
    np.testing.assert_allclose(ev.electric_field_adj, ref["field_adj"], rtol=0, atol=2e-5 * scale)
    plain = MACEKokkosFloat(tiny_model_path)
    with pytest.raises(ValueError, match="no field coupling"):
        plain.compute_node_energies_forces_field(n, types, g["num_neigh"], g["sources"], types[g["sources"]],
                                                 ref["xyz"], ref["r"], FIELD)


def test_field_adjoint_keeps_the_evaluated_shape(tiny_field_model_path):
    """dE/dE is that of the last evaluation: a field of another shape set
    afterwards applies to the next evaluation only."""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    ev = MACEKokkosFloat(tiny_field_model_path)
    lut = {int(z): i for i, z in enumerate(ev.atomic_numbers)}
    types = np.array([lut[int(z)] for z in s["numbers"]], np.int32)
    g = _prepare(ev, s, types)
    ev._compute_prepared_factorized_positions_field(g["generation"], s["positions"], FIELD)
    adj = ev.electric_field_adj
    assert adj.shape == (3,)
    n = len(types)
    ev._set_electric_field(np.tile(FIELD, (n, 1)))
    np.testing.assert_array_equal(ev.electric_field_adj, adj)
    ev._compute_prepared_factorized_positions(g["generation"], s["positions"])
    per = ev.electric_field_adj.reshape(n, 3)
    np.testing.assert_allclose(per.sum(axis=0), adj, rtol=0, atol=1e-6 * np.max(np.abs(adj)))
