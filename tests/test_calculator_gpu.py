"""The Symmetrix calculator end to end on the GPU.

* A short trajectory within half the neighbour skin reuses one prepared graph
  (calculator.py's neighbour-cache rule, test_symmetrix_calc.py:280-586 in the
  reference); every step's energy, forces and stress equal the oracle's on a
  graph rebuilt at that step's positions.
* Finite differences of the calculator's own energy give its forces and its
  stress (the reference's test_symmetrix_calc_finite_diff,
  test_symmetrix_calc.py:1201). The evaluator computes in FP32, so the energy
  carries ~1e-5 eV of rounding: the steps are sized so that this noise stays
  well below the tolerances written here.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5      # eV/atom, against the oracle
F_TOL = 1e-4      # eV/A, against the oracle
S_TOL = 1e-6      # eV/A^3, against the oracle
FD_F_TOL = 5e-3   # eV/A, central difference with h = 5e-3 A
FD_S_TOL = 5e-5   # eV/A^3, central difference with strain 1e-3


def _system():
    from symmetrix import systems
    return systems.srtio3_supercell(3, sigma=0.05, seed=0)


def _atoms(s, positions=None, cell=None):
    return {"numbers": s["numbers"], "positions": s["positions"] if positions is None else positions,
            "cell": s["cell"] if cell is None else cell, "pbc": [True, True, True]}


def test_calculator_trajectory_reuses_graph_and_matches_oracle(tiny_model_path):
    from oracle import oracle
    from symmetrix.calculator import Symmetrix, full_3x3_to_voigt_6_stress
    s = _system()
    om = oracle.OracleModel(tiny_model_path)
    calc = Symmetrix(tiny_model_path, neighbor_skin=0.5)
    n = len(s["numbers"])
    rng = np.random.default_rng(3)
    pos = np.array(s["positions"], float)
    for step in range(4):
        if step:
            pos = pos + rng.uniform(-0.04, 0.04, size=pos.shape)   # max drift stays < skin/2
        res = calc.calculate(_atoms(s, pos))
        ref = oracle.evaluate_system(om, dict(s, positions=pos), skin=0.5)   # its own fresh graph
        assert abs(res["energy"] - ref["energy"]) / n < E_TOL
        assert abs(np.sum(res["energies"]) - res["energy"]) < 1e-9
        assert np.max(np.abs(res["forces"] - ref["forces"])) < F_TOL
        np.testing.assert_allclose(res["stress"], full_3x3_to_voigt_6_stress(ref["stress"]), rtol=0, atol=S_TOL)
    assert calc.neighbor_graph_rebuilds == 1
    # a displacement beyond half the skin rebuilds the graph
    pos = pos.copy()
    pos[0] += [0.4, 0.0, 0.0]
    calc.calculate(_atoms(s, pos))
    assert calc.neighbor_graph_rebuilds == 2


def test_calculator_finite_differences(tiny_model_path):
    from symmetrix.calculator import Symmetrix, full_3x3_to_voigt_6_stress
    s = _system()
    calc = Symmetrix(tiny_model_path, neighbor_skin=0.5)
    pos0 = np.array(s["positions"], float)
    cell0 = np.array(s["cell"], float)
    res = calc.calculate(_atoms(s, pos0))
    forces = np.array(res["forces"])
    stress = np.array(res["stress"])

    def energy(pos=pos0, cell=cell0):
        return calc.calculate(_atoms(s, pos, cell), ["energy"])["energy"]

    h = 5e-3
    for atom, comp in [(0, 0), (1, 1), (7, 2), (40, 0), (134, 1)]:
        dp = np.zeros_like(pos0)
        dp[atom, comp] = h
        fd = -(energy(pos0 + dp) - energy(pos0 - dp)) / (2 * h)
        assert abs(fd - forces[atom, comp]) < FD_F_TOL, (atom, comp, fd, forces[atom, comp])
    # stress = (1/V) dE/d(strain), atoms moved with the cell
    eps = 1e-3
    V = abs(np.linalg.det(cell0))
    fd = np.zeros((3, 3))
    for a in range(3):
        for b in range(a, 3):
            d = np.zeros((3, 3))
            d[a, b] = d[b, a] = eps if a == b else 0.5 * eps
            up, dn = np.eye(3) + d, np.eye(3) - d
            e_up = energy(pos0 @ up, cell0 @ up)
            e_dn = energy(pos0 @ dn, cell0 @ dn)
            fd[a, b] = fd[b, a] = (e_up - e_dn) / (2 * eps * V)
    np.testing.assert_allclose(stress, full_3x3_to_voigt_6_stress(fd), rtol=0, atol=FD_S_TOL)
    # the checks bite: a sign or index slip would exceed the tolerances
    assert np.max(np.abs(stress)) > 10 * FD_S_TOL
    assert np.max(np.abs(forces[[0, 1, 7, 40, 134], [0, 1, 2, 0, 1]])) > 10 * FD_F_TOL


# ---------------------------------------------------------------------------
# Host-graph routes: open and mixed boundaries, small cells, strained cells
# (calculator.py:83-84, 165-173, 2838-3093, 3224-3300)
# ---------------------------------------------------------------------------
def _oracle_host_graph(om, numbers, positions, cell, pbc, skin=0.5):
    """The oracle on the caller's host "ijS" graph (the list the reference
    calculator takes from matscipy/ASE), with the Cartesian prepared geometry."""
    from oracle import oracle
    from symmetrix.neighbors import neighbor_list_ijS
    i, j, S = neighbor_list_ijS(positions, cell, pbc, om.r_cut + skin)
    ref_xyz = positions[j] - positions[i] + S @ cell
    xyz, r = oracle.prepared_geometry_kind("cartesian", i, j, positions, ref_xyz, cell, positions, om.r_cut,
                                           pbc=np.asarray(pbc, np.int32))
    types = om.types_of(numbers)
    num_neigh = np.bincount(i, minlength=len(types)).astype(np.int32)
    e, f = om.evaluate(types, num_neigh, j, types[j], xyz, r)
    forces = oracle.reduce_forces(len(types), i, j, f)
    vol = abs(np.linalg.det(cell))
    stress = oracle.reduce_stress(f, xyz, vol) if vol > 0 else None
    return {"energy": float(np.sum(e)), "forces": forces, "stress": stress, "edges": len(j)}


def _cluster(radius=7.0):
    """A SrTiO3 cluster in vacuum: atoms within radius of the supercell centre."""
    from symmetrix import systems
    s = systems.srtio3_supercell(4, sigma=0.05, seed=2)
    c = np.mean(s["positions"], axis=0)
    keep = np.linalg.norm(s["positions"] - c, axis=1) < radius
    return s["numbers"][keep], s["positions"][keep] - c


def test_calculator_open_molecule_and_slab_against_oracle(tiny_model_path, monkeypatch):
    from oracle import oracle
    from symmetrix import systems
    from symmetrix.calculator import Symmetrix, full_3x3_to_voigt_6_stress
    monkeypatch.delenv("SYMMETRIX_NEIGHBOR_BACKEND", raising=False)
    om = oracle.OracleModel(tiny_model_path)
    numbers, pos = _cluster()
    print("cluster of %d atoms" % len(numbers), flush=True)
    calc = Symmetrix(tiny_model_path, neighbor_skin=0.5)
    res = calc.calculate({"numbers": numbers, "positions": pos, "cell": np.zeros((3, 3)),
                          "pbc": [False, False, False]}, ["energy", "forces"])
    ref = _oracle_host_graph(om, numbers, pos, np.zeros((3, 3)), [False, False, False])
    assert calc.neighbor_graph_backend == "host"
    assert abs(res["energy"] - ref["energy"]) / len(numbers) < E_TOL
    assert np.max(np.abs(res["forces"] - ref["forces"])) < F_TOL
    assert abs(np.sum(res["forces"], axis=0)).max() < 1e-6 * len(numbers)   # no external field
    # a slab: periodic in x and y, 12 A of vacuum along z
    s = systems.srtio3_supercell(3, sigma=0.05, seed=4)
    cell = np.array(s["cell"], float)
    cell[2, 2] += 12.0
    pbc = [True, True, False]
    res = calc.calculate({"numbers": s["numbers"], "positions": s["positions"], "cell": cell, "pbc": pbc})
    ref = _oracle_host_graph(om, s["numbers"], s["positions"], cell, pbc)
    n = len(s["numbers"])
    assert abs(res["energy"] - ref["energy"]) / n < E_TOL
    assert np.max(np.abs(res["forces"] - ref["forces"])) < F_TOL
    np.testing.assert_allclose(res["stress"], full_3x3_to_voigt_6_stress(ref["stress"]), rtol=0, atol=S_TOL)
    # moved within half the skin: same graph
    res2 = calc.calculate({"numbers": s["numbers"], "positions": s["positions"] + 0.1, "cell": cell, "pbc": pbc})
    assert calc.neighbor_graph_rebuilds == 2
    ref2 = _oracle_host_graph(om, s["numbers"], s["positions"] + 0.1, cell, pbc)
    assert np.max(np.abs(res2["forces"] - ref2["forces"])) < F_TOL


@pytest.mark.parametrize("cells,backend", [(2, "automatic"), (3, "automatic"), (5, "automatic"), (3, "kokkos")])
def test_calculator_strained_cell_reuses_graph(tiny_model_path, monkeypatch, cells, backend):
    """40 and 135 atoms take the host graph (fractional geometry), 625 atoms
    and a forced device backend the device builder; a 0.4% strain with the
    atoms carried along (plus thermal noise) keeps the topology and only
    updates the evaluator's cell, and matches the oracle on a fresh graph of
    the strained system."""
    from oracle import oracle
    from symmetrix import systems
    from symmetrix.calculator import Symmetrix, full_3x3_to_voigt_6_stress
    monkeypatch.setenv("SYMMETRIX_NEIGHBOR_BACKEND", backend)
    s = systems.srtio3_supercell(cells, sigma=0.05, seed=1)
    n = len(s["numbers"])
    print("cells %d (%d atoms), backend %s" % (cells, n, backend), flush=True)
    om = oracle.OracleModel(tiny_model_path)
    calc = Symmetrix(tiny_model_path, neighbor_skin=0.5)
    calc.calculate(_atoms(s))
    expect = "device" if (n >= 512 or backend == "kokkos") else "host"
    assert calc.neighbor_graph_backend == expect
    strain = np.array([[1.004, 0.001, 0.0], [0.001, 0.997, 0.0], [0.0, 0.0, 1.002]])
    rng = np.random.default_rng(9)
    pos = s["positions"] @ strain + rng.uniform(-0.02, 0.02, size=s["positions"].shape)
    cell = s["cell"] @ strain
    res = calc.calculate(_atoms(s, pos, cell))
    assert calc.neighbor_graph_rebuilds == 1 and calc.neighbor_cache_cell_update_count == 1
    ref = oracle.evaluate_system(om, dict(s, positions=pos, cell=cell), skin=0.5)
    assert abs(res["energy"] - ref["energy"]) / n < E_TOL
    assert np.max(np.abs(res["forces"] - ref["forces"])) < F_TOL
    np.testing.assert_allclose(res["stress"], full_3x3_to_voigt_6_stress(ref["stress"]), rtol=0, atol=S_TOL)


def test_shift_geometry_under_the_tiled_plan(tiny_model_path):
    """prepare_factorized_shift_geometry (lifecycle.cpp:2570-2697): refused
    outside the tiled plan; under it the integer-shift geometry gives the
    oracle's results; the cell then updates like the fractional form."""
    from oracle import oracle
    from symmetrix import systems
    from symmetrix.mace_kokkos import MACEKokkosFloat
    from symmetrix.neighbors import neighbor_list_ijS
    s = systems.srtio3_supercell(3, sigma=0.05, seed=0)
    om = oracle.OracleModel(tiny_model_path)
    types = om.types_of(s["numbers"])
    cell = np.array(s["cell"], float)
    inv = np.linalg.inv(cell)
    pos = np.array(s["positions"], float)
    i, j, S = neighbor_list_ijS(pos, cell, [True] * 3, om.r_cut + 0.5)
    num_neigh = np.bincount(i, minlength=len(types)).astype(np.int32)
    ev = MACEKokkosFloat(tiny_model_path)
    gen = ev._prepare_factorized_graph(len(types), types, num_neigh, j, types[j])
    with pytest.raises(ValueError, match="tiled"):
        ev._prepare_factorized_shift_geometry(gen, pos, S, cell, inv, [1, 1, 1])
    ev.set_execution_plan_request("capacity", 50)
    gen = ev._prepare_factorized_graph(len(types), types, num_neigh, j, types[j])
    assert ev.execution_plan_report["selected_id"] == "mh0-dual-layer-tiled-v1"
    ev._prepare_factorized_shift_geometry(gen, pos, S, cell, inv, [1, 1, 1])
    for strain in (np.eye(3), np.diag([1.003, 0.998, 1.001])):
        c = cell @ strain
        p = pos @ strain
        if not np.array_equal(c, cell):
            ev._update_factorized_cell(gen, c, np.linalg.inv(c))
        ev._compute_prepared_factorized_positions(gen, p)
        e = ev.node_energies
        f = ev._reduce_atom_forces(len(types), None, None, gen)
        xyz, r = oracle.prepared_geometry_kind("shifts", i, j, pos, S, c, p, om.r_cut)
        ee, ff = om.evaluate(types, num_neigh, j, types[j], xyz, r)
        fr = oracle.reduce_forces(len(types), i, j, ff)
        assert abs(np.sum(e) - np.sum(ee)) / len(types) < E_TOL
        assert np.max(np.abs(f - fr)) < F_TOL


def test_geometry_errors_and_counters(tiny_model_path):
    """Geometry validation (lifecycle.cpp:2463-2490, 2702-2716) and the
    plan report and timing counters."""
    from symmetrix import systems
    from symmetrix.mace_kokkos import MACEKokkosFloat
    from symmetrix.neighbors import neighbor_list_ijS
    s = systems.srtio3_supercell(2, sigma=0.05, seed=0)
    ev = MACEKokkosFloat(tiny_model_path)
    types = np.array([{8: 0, 22: 1, 38: 2}[int(z)] for z in s["numbers"]], np.int32)
    cell = np.array(s["cell"], float)
    pos = np.array(s["positions"], float)
    i, j, S = neighbor_list_ijS(pos, cell, [True] * 3, ev.r_cut + 0.5)
    nn = np.bincount(i, minlength=len(types)).astype(np.int32)
    gen = ev._prepare_factorized_graph(len(types), types, nn, j, types[j])
    with pytest.raises(ValueError):   # positions call without a geometry
        ev._compute_prepared_factorized_positions(gen, pos)
    frac = pos @ np.linalg.inv(cell)
    fxyz = frac[j] - frac[i] + S
    with pytest.raises(ValueError, match="periodic"):
        ev._prepare_factorized_fractional_geometry(gen, frac, fxyz, cell, np.linalg.inv(cell), [1, 1, 0])
    bad = fxyz.copy()
    bad[3, 1] = np.nan
    with pytest.raises(ValueError, match="non-finite"):
        ev._prepare_factorized_fractional_geometry(gen, frac, bad, cell, np.linalg.inv(cell), [1, 1, 1])
    with pytest.raises(ValueError, match="extents"):
        ev._prepare_factorized_fractional_geometry(gen, frac, fxyz[:-1], cell, np.linalg.inv(cell), [1, 1, 1])
    ev._prepare_factorized_fractional_geometry(gen, frac, fxyz, cell, np.linalg.inv(cell), [1, 1, 1])
    with pytest.raises(ValueError, match="invertible"):
        ev._update_factorized_cell(gen, np.zeros(9), np.zeros(9))
    ev._compute_prepared_factorized_positions(gen, pos)
    assert ev.factorized_last_evaluation_ms > 0.0 and ev.factorized_last_graph_prepare_ms > 0.0
    rep = ev.execution_plan_report
    assert rep["state"] == "resolved" and rep["selected_id"] == "mh0-direct-capacity-retained"
    assert rep["requested_profile"] == "capacity" and not rep["allow_fixed_workspace"]
    ev._set_execution_plan_request("direct", "speed", "")
    ev._prepare_factorized_graph(len(types), types, nn, j, types[j])
    assert ev.execution_plan_report["selected_id"] == "mh0-direct-speed"
    with pytest.raises(ValueError):
        ev._set_execution_plan_request("materialized", "speed", "")
    ev.prepare_active_types([0, 1, 2])


@pytest.mark.parametrize("plan", ["direct", "tiled"])
def test_results_call_equals_the_calls_in_turn(tiny_model_path, plan):
    """smx_compute_prepared_factorized_positions_results, the calculator's
    one-call path: bit-identical to the positions call followed by
    node_energies, _reduce_atom_forces and _reduce_stress, under the direct
    and the tiled plan; without a volume no stress; non-finite positions and
    a non-positive volume raise."""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system()
    ev = MACEKokkosFloat(tiny_model_path)
    if plan == "tiled":
        ev.set_execution_plan_request("capacity", 16)
    lut = {int(z): i for i, z in enumerate(ev.atomic_numbers)}
    types = np.array([lut[int(z)] for z in s["numbers"]], np.int32)
    cell = np.asarray(s["cell"], float)
    g = ev._prepare_periodic_factorized_graph(types, s["positions"], cell, np.linalg.inv(cell), ev.r_cut + 0.5)
    gen = g["generation"]
    V = abs(np.linalg.det(cell))
    pos = s["positions"] + 0.01 * np.random.default_rng(5).normal(size=s["positions"].shape)
    ev._compute_prepared_factorized_positions(gen, pos)
    e_ref = np.array(ev.node_energies)
    f_ref = ev._reduce_atom_forces(len(types), None, None, gen)
    s_ref = ev._reduce_stress(V, None, gen)
    e, f, st = ev._compute_prepared_factorized_positions_results(gen, pos, V)
    np.testing.assert_array_equal(e, e_ref)
    np.testing.assert_array_equal(f, f_ref)
    np.testing.assert_array_equal(st, s_ref)
    e2, f2, st2 = ev._compute_prepared_factorized_positions_results(gen, pos)
    assert st2 is None
    np.testing.assert_array_equal(e2, e_ref)
    np.testing.assert_array_equal(f2, f_ref)
    bad = pos.copy()
    bad[1, 0] = np.nan
    with pytest.raises(ValueError, match="finite"):
        ev._compute_prepared_factorized_positions_results(gen, bad, V)
    with pytest.raises(ValueError, match="volume"):
        ev._compute_prepared_factorized_positions_results(gen, pos, -1.0)
    # the evaluator still evaluates afterwards
    e3, f3, _ = ev._compute_prepared_factorized_positions_results(gen, pos, V)
    np.testing.assert_array_equal(f3, f_ref)
