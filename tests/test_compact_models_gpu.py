"""HIP path against the oracle on models written by the reference's own
writer (symmetrix/test/compact_r1_model.py, fixtures tests/golden/compact_*),
whose layouts tests/test_model_layout.py pins stage by stage: the medium
shape and the shapes of the MACE-OMAT-0 small (L_max 0) and MP-0b2 large
(L_max 2) checkpoints at 128 channels, and of the MACE-OFF23 small (96
channels, L_max 0) and large (224 channels, L_max 2) checkpoints, which run
on 128 and 256 lanes with zero extra channels.

Bars: FP32 energy within 1e-5 eV/atom, forces 1e-4 eV/Angstrom, stress
1e-6 eV/Angstrom^3; stages within 1e-4 of their largest magnitude.
"""

import numpy as np
import pytest

from _compact import compact_model, fixture_system

pytestmark = pytest.mark.gpu

E_TOL, F_TOL, S_TOL = 1e-5, 1e-4, 1e-6


def _run(name, cells, skin=0.5, model_file=None):
    from oracle import oracle
    from symmetrix.mace_kokkos import MACEKokkosFloat
    path, _ = compact_model(name)
    system = fixture_system(name, cells=cells)
    om = oracle.OracleModel(path)
    ref = oracle.evaluate_system(om, system, skin=skin)
    ev = MACEKokkosFloat(model_file or path)
    types = om.types_of(system["numbers"])
    cell = np.asarray(system["cell"], float)
    g = ev._prepare_periodic_factorized_graph(types, system["positions"], cell, np.linalg.inv(cell),
                                              ev.r_cut + skin)
    assert g["num_edges"] == len(ref["graph"]["sources"])
    ev._compute_prepared_factorized_positions(g["generation"], system["positions"])
    e = ev.node_energies
    f = ev._reduce_atom_forces(len(types), None, None, g["generation"])
    s = ev._reduce_stress(abs(np.linalg.det(cell)), None, g["generation"])
    return om, ref, ev, e, f, s


@pytest.mark.parametrize("name,cells", [("compact_medium_m0", 3), ("compact_medium_linear", 3),
                                        ("compact_medium_linear", 10), ("compact_omat0_small", 3),
                                        ("compact_mp0b2_large", 3), ("compact_off23_small", 3),
                                        ("compact_off23_large", 3)])
def test_reference_written_model_efs(name, cells):
    print("case", name, cells, flush=True)
    om, ref, ev, e, f, s = _run(name, cells)
    n = len(e)
    de = abs(np.sum(e) - ref["energy"]) / n
    df = np.max(np.abs(f - ref["forces"]))
    ds = np.max(np.abs(s - ref["stress"]))
    print("energy/atom err %.3e  force err %.3e  stress err %.3e" % (de, df, ds))
    assert de < E_TOL and df < F_TOL and ds < S_TOL
    np.testing.assert_allclose(e, ref["energies"], rtol=0, atol=1e-5 * max(1.0, np.max(np.abs(ref["energies"]))))


@pytest.mark.parametrize("name", ["compact_medium_m0", "compact_medium_linear", "compact_omat0_small",
                                  "compact_mp0b2_large"])
def test_reference_written_model_stages(name):
    print("case", name, flush=True)
    om, ref, ev, e, f, s = _run(name, 3)
    for stage in ("A0", "M0", "H1", "Phi1", "A1", "A1_adj", "dPhi1", "H1_adj", "A0_adj"):
        mine = ev._stage(stage).astype(np.float64)
        theirs = om.stage(stage)
        err = float(np.max(np.abs(mine - theirs)) / max(np.max(np.abs(theirs)), 1e-30))
        print(stage, "relative max err %.3e" % err)
        assert err < 1e-4, stage
    nf = ev.node_forces.reshape(-1, 3)
    assert np.max(np.abs(nf - ref["node_forces"])) < 1e-5


def test_binary_model_file_evaluates_like_its_json(tmp_path):
    # the SMXB form of a model loads to the same arrays: identical results
    from symmetrix import model_format
    print("case compact_medium_linear binary", flush=True)
    path, _ = compact_model("compact_medium_linear")
    binary = tmp_path / "model.smxb"
    model_format.convert(path, binary)
    _, ref, _, e0, f0, s0 = _run("compact_medium_linear", 3)
    _, _, _, e1, f1, s1 = _run("compact_medium_linear", 3, model_file=binary)
    assert np.array_equal(e0, e1) and np.array_equal(f0, f1) and np.array_equal(s0, s1)
    assert np.max(np.abs(f1 - ref["forces"])) < F_TOL
