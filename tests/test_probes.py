"""The probe-subgraph evaluation (tests/_probes.py) that checks the tiled
plan at millions of atoms, pinned on the CPU: on a system the oracle can
evaluate whole (SrTiO3 14^3, 13,720 atoms, the medium model), each probe's
energy and force from its subgraph equal the whole-system oracle's to FP32
summation-order noise (1e-7).  A subgraph whose receivers lie within one
edge of the probe still gives its energy but not its force: the sources' H1
adjoints then miss the receivers two edges away, which move this model's
forces by about 2e-5 eV/A, far above that noise.  (Between two and three
edges only the curvature of the readout and product basis differs, which the
random-init medium model makes too small to show.)"""

import numpy as np

from _probes import oracle_probe


def test_probe_subgraph_equals_whole_system(medium_model_path):
    from oracle import oracle
    from symmetrix import systems
    s = systems.srtio3_supercell(14, sigma=0.05, seed=4)
    om = oracle.OracleModel(medium_model_path)
    ref = oracle.evaluate_system(om, s, skin=0.5)
    types = om.types_of(s["numbers"])
    pos = np.asarray(s["positions"], np.float64)
    L = float(s["cell"][0, 0])
    cutoff = om.r_cut + 0.5
    for probe in (0, 4321, 13719):
        e, F, nrec = oracle_probe(om, pos, types, L, probe, cutoff)
        print("probe", probe, nrec, e - ref["energies"][probe], F - ref["forces"][probe])
        assert abs(e - ref["energies"][probe]) < 2e-7
        assert np.max(np.abs(F - ref["forces"][probe])) < 1e-7
    # too shallow for the force: receivers within one edge only
    e1, F1, _ = oracle_probe(om, pos, types, L, 4321, cutoff, hops=1)
    print("one edge deep:", e1 - ref["energies"][4321], F1 - ref["forces"][4321])
    assert abs(e1 - ref["energies"][4321]) < 2e-7
    assert np.max(np.abs(F1 - ref["forces"][4321])) > 5e-6
