"""One-interaction models (single_layer_readout; mace.cpp:255-281,
2461-2514) on the GPU against the oracle: the H1 and H1-adjoint stages,
directed forces and E/F/S in the direct plan; the one-sweep tiled plan
(mh0-single-layer-tiled-v1, mace_kokkos_evaluate.cpp:614-752) equals the
direct one; each tiled plan admits only its own model kind
(mace_kokkos_runtime.cpp:2996-3030).  The LAMMPS entry runs a
one-interaction model in tests/test_lammps_entry.py."""

import numpy as np
import pytest

from test_gpu_parity import _assert_efs, _evaluate_both, _run, _stage_err, _system

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("model", ["tiny_single", "tiny_single_residual"])
def test_single_layer_model_matches_oracle(request, model):
    from symmetrix.mace_kokkos import MACEKokkosFloat
    path = request.getfixturevalue(model + "_model_path")
    s = _system("tiny")
    om, ref, ev, g, e, f, st = _evaluate_both(path, s)
    for name in ("H1", "H1_adj", "A0_adj"):
        err = _stage_err(ev._stage(name).astype(np.float64), om.stage(name))
        print(name, "relative max err %.3e" % err)
        assert err < 1e-4, name
    with pytest.raises(ValueError, match="not held"):
        ev._stage("A1")
    np.testing.assert_allclose(e, ref["energies"], rtol=0, atol=1e-4)
    nf = ev.node_forces.reshape(-1, 3)
    assert np.max(np.abs(nf - ref["node_forces"])) < 1e-5
    _assert_efs(ref, e, f, st, len(e))
    assert ev.execution_plan_report["selected_id"] != "mh0-single-layer-tiled-v1"
    for tile in (37, 64):
        b = MACEKokkosFloat(path)
        b.set_execution_plan_request("capacity", tile)
        e1, f1, s1 = _run(b, s, om.types_of(s["numbers"]))
        assert b.execution_plan.startswith("direct-tiled")
        assert b.execution_plan_report["selected_id"] == "mh0-single-layer-tiled-v1"
        np.testing.assert_array_equal(e1, e)
        np.testing.assert_allclose(f1, f, rtol=0, atol=1e-7)
        np.testing.assert_allclose(s1, st, rtol=0, atol=1e-9)


def test_trained_one_interaction_shape(medium_single_model_path):
    """128x0e+128x1o, l_max 3, correlation 3, readout correlation 2, A0
    density scaling (the extracted single-layer checkpoint's shape,
    test_single_layer_mace.py:71-81) on SrTiO3, both plans."""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    om, ref, ev, g, e, f, st = _evaluate_both(medium_single_model_path, s)
    _assert_efs(ref, e, f, st, len(e))
    np.testing.assert_allclose(e, ref["energies"], rtol=0, atol=1e-4)
    b = MACEKokkosFloat(medium_single_model_path)
    b.set_execution_plan_request("capacity", 50)
    e1, f1, s1 = _run(b, s, om.types_of(s["numbers"]))
    assert b.execution_plan_report["selected_id"] == "mh0-single-layer-tiled-v1"
    np.testing.assert_array_equal(e1, e)
    np.testing.assert_allclose(f1, f, rtol=0, atol=1e-6)
    np.testing.assert_allclose(s1, st, rtol=0, atol=1e-9)


def test_tiled_plans_admit_only_their_model_kind(tiny_single_model_path, tiny_model_path):
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    for path, wrong in ((tiny_single_model_path, "mh0-dual-layer-tiled-v1"),
                        (tiny_model_path, "mh0-single-layer-tiled-v1")):
        ev = MACEKokkosFloat(path)
        ev._set_execution_plan_request("direct", "capacity", wrong)
        lut = {int(z): i for i, z in enumerate(ev.atomic_numbers)}
        types = np.array([lut[int(z)] for z in s["numbers"]], np.int32)
        with pytest.raises(ValueError, match="requires"):
            _run(ev, s, types)


def _cluster(count):
    """count atoms on a 1.8 A grid in an 8 A periodic cell, O and Ti
    alternating (the reference's tile-boundary fixture,
    test_single_layer_mace.py:262-267, with this model's elements)."""
    grid = np.indices((3, 3, 3)).reshape(3, -1).T[:count]
    pos = 1.1 + 1.8 * grid.astype(float)
    pos[-1] = [3.0, 3.0, 3.0]
    numbers = np.array([8 if k % 3 == 0 else 22 for k in range(count)])
    return {"numbers": numbers, "positions": pos, "cell": np.diag([8.0, 8.0, 8.0]), "pbc": [True] * 3}


@pytest.mark.parametrize("count", [3, 4, 5, 8, 9])
def test_one_sweep_tiled_plan_at_tile_boundaries(tiny_single_residual_model_path, count):
    """The calculator with the single-layer tiled plan pinned and 4 receivers
    per tile (test_single_layer_mace.py:270-300) against the direct plan and
    the oracle."""
    from oracle import oracle
    from symmetrix.calculator import Symmetrix, full_3x3_to_voigt_6_stress
    path = tiny_single_residual_model_path
    s = _cluster(count)
    direct = Symmetrix(path).calculate(s)
    calc = Symmetrix(path, _debug_execution_plan="mh0-single-layer-tiled-v1")
    calc.evaluator.set_execution_plan_request("capacity", 4)
    tiled = calc.calculate(s)
    assert calc.execution_plan["selected_id"] == "mh0-single-layer-tiled-v1"
    assert calc.evaluator.execution_plan_report["max_tile_receivers"] == min(count, 4)
    for key in ("energy", "energies", "forces", "stress"):
        np.testing.assert_allclose(tiled[key], direct[key], rtol=0, atol=1e-6)
    ref = oracle.evaluate_system(oracle.OracleModel(path), s, skin=0.5)
    assert abs(tiled["energy"] - ref["energy"]) / count < 1e-5
    np.testing.assert_allclose(tiled["forces"], ref["forces"], rtol=0, atol=1e-4)
    np.testing.assert_allclose(tiled["stress"], full_3x3_to_voigt_6_stress(ref["stress"]), rtol=0, atol=1e-6)
