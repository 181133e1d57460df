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
