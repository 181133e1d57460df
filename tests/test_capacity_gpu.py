"""The tiled capacity plan at the sizes of the capacity config (perturbed
cubic SrTiO3 n^3 supercells from about 1M to over 11M atoms, the medium
model, r_cut 6.0 A + 0.5 A skin; the reference's dual-layer tiled plan,
mace_kokkos_evaluate.cpp:755-1148) against the CPU oracle.

The oracle cannot evaluate 11.5M atoms in a test, but MACE is local: with two
interactions, the energy of atom k depends only on atoms within two edges of
k, and the force on k only on the energies within two edges of k, hence on
atoms within four edges.  So for a probe atom k the oracle evaluates the
subgraph made of the atoms within three edges of k, each with its full
neighbour list (all its neighbours within cutoff + skin in the periodic
system), plus the atoms at four edges as nodes without edges.  Every state
that k's energy and force read is then the whole system's, and the oracle's
energy and force of k are the whole system's (tolerance-level agreement only
from the FP32 summation order of the edges).  Probes sit on both sides of
tile boundaries (multiples of the tile size in receiver order), where a
receiver's sources lie in other tiles and the source adjoint crosses tiles,
at the last atoms (the highest edge offsets), and at random.

Full-system properties at the same size: the atom forces sum to zero
(every directed edge force enters once with each sign), and on the
unperturbed crystal, where every site is an inversion centre, every atom's
energy equals its site's energy in the oracle's 3x3x3 cell, every force
vanishes and the stress equals the oracle's.  The unperturbed check also
runs at n = 164 (22M atoms, 2.18B edges), past the 2^31 - 4096 edges that
32-bit edge ids hold: the tiled plan's 64-bit source transpose and
tile-relative offsets carry every edge beyond that index.

Bars: energy 1e-5 eV/atom, forces 1e-4 eV/A, stress 1e-6 eV/A^3.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL, F_TOL, S_TOL = 1e-5, 1e-4, 1e-6
TILE = 32768
SKIN = 0.5


def _say(*a):
    print(*a, flush=True)


from _probes import oracle_probe as _oracle_probe  # noqa: E402


def _tiled_call(model_path, system):
    from symmetrix.mace_kokkos import MACEKokkosFloat
    ev = MACEKokkosFloat(model_path)
    ev.set_execution_plan_request("capacity", TILE)
    lut = {int(z): i for i, z in enumerate(ev.atomic_numbers)}
    types = np.array([lut[int(z)] for z in system["numbers"]], np.int32)
    pos = np.ascontiguousarray(system["positions"], np.float64)
    cell = np.asarray(system["cell"], np.float64)
    g = ev._prepare_periodic_factorized_graph(types, pos.reshape(-1), cell.reshape(-1),
                                              np.linalg.inv(cell).reshape(-1), ev.r_cut + SKIN)
    plan = ev.execution_plan
    _say("graph: %d edges, plan %s" % (g["num_edges"], plan))
    assert "tiled" in plan
    ev._compute_prepared_factorized_positions(g["generation"], pos.reshape(-1))
    n = len(types)
    e = np.array(ev.node_energies, dtype=np.float64)
    f = ev._reduce_atom_forces(n, None, None, g["generation"])
    s = ev._reduce_stress(abs(np.linalg.det(cell)), None, g["generation"])
    total = ev._total_energy()
    ev.close()
    return types, e, f, s, total, g["num_edges"]


def _probes(n, count, seed):
    rng = np.random.default_rng(seed)
    k = np.arange(1, n // TILE + 1)
    k = k[np.linspace(0, len(k) - 1, min(len(k), 6)).astype(int)]
    boundary = np.concatenate([k * TILE - 1, k * TILE])
    ends = np.array([0, n - 2, n - 1])
    rand = rng.choice(n, size=count, replace=False)
    return np.unique(np.concatenate([boundary[boundary < n], ends, rand]))


@pytest.mark.parametrize("cells,random_probes", [(59, 10), (132, 6)])
def test_tiled_plan_against_oracle_probes_at_size(medium_model_path, cells, random_probes):
    """n = 59 (1,026,895 atoms, 32 tiles) and n = 132 (11,499,840 atoms,
    351 tiles, 1.14B edges): energies and forces of probe atoms against the
    oracle's subgraph evaluation; the forces sum to zero."""
    from oracle import oracle
    from symmetrix import systems
    system = systems.srtio3_supercell(cells, sigma=0.05, seed=0)
    n = len(system["numbers"])
    _say("capacity case: SrTiO3 n=%d, %d atoms, tiles of %d receivers" % (cells, n, TILE))
    types, e, f, s, total, E = _tiled_call(medium_model_path, system)
    _say("tiled call done: energy %.6f eV" % total)
    assert abs(total - np.sum(e)) < 1e-9 * n
    # every directed force enters two atoms with opposite signs (one missing
    # edge force would leave a net force of order 0.1 eV/A)
    net = np.abs(np.sum(f, axis=0))
    _say("net force", net)
    assert np.all(net < 1e-10 * n)
    om = oracle.OracleModel(medium_model_path)
    L = float(system["cell"][0, 0])
    pos = np.asarray(system["positions"], np.float64)
    cutoff = om.r_cut + SKIN
    worst_e = worst_f = 0.0
    for probe in _probes(n, random_probes, seed=cells):
        ep, Fp, nrec = _oracle_probe(om, pos, types, L, int(probe), cutoff)
        de, dF = abs(e[probe] - ep), float(np.max(np.abs(f[probe] - Fp)))
        _say("probe %9d (tile %3d, subgraph %d receivers): dE %.2e eV, max|dF| %.2e eV/A, |F| %.3f"
             % (probe, probe // TILE, nrec, de, dF, np.linalg.norm(Fp)))
        worst_e, worst_f = max(worst_e, de), max(worst_f, dF)
    assert worst_e < E_TOL and worst_f < F_TOL
    # and well below what the layer-2 source adjoint adds to the forces of
    # this model (about 2e-5 eV/A): a source row lost or doubled across tiles
    # would show
    assert worst_e < 1e-6 and worst_f < 1e-6


@pytest.mark.parametrize("cells", [132, 164])
def test_unperturbed_crystal_at_size(medium_model_path, cells):
    """n = 132 (11.5M atoms) and n = 164 (22M atoms, beyond 2^31 edges)
    unperturbed (every site an inversion centre): each atom's energy equals
    its species' site energy in the oracle's 3x3x3 cell, every force
    vanishes, and the stress equals the oracle's."""
    from oracle import oracle
    from symmetrix import systems
    om = oracle.OracleModel(medium_model_path)
    small = systems.srtio3_supercell(3, sigma=0.0)
    ref = oracle.evaluate_system(om, small, skin=SKIN)
    site = {}
    for z, ez in zip(small["numbers"], ref["energies"]):
        site.setdefault(int(z), []).append(ez)
    for z, v in site.items():
        assert np.ptp(v) < 5e-6, (z, np.ptp(v))    # equivalent sites in the oracle too
    site = {z: float(np.mean(v)) for z, v in site.items()}
    system = systems.srtio3_supercell(cells, sigma=0.0)
    n = len(system["numbers"])
    _say("capacity case: unperturbed SrTiO3 n=%d, %d atoms" % (cells, n))
    types, e, f, s, total, E = _tiled_call(medium_model_path, system)
    if cells == 164:
        assert E > 2**31, E   # edge ids beyond 32 bits
    expect = np.array([site[int(z)] for z in system["numbers"][:5]])
    de = np.max(np.abs(e.reshape(-1, 5) - expect[None, :]))
    df = float(np.max(np.abs(f)))
    ds = float(np.max(np.abs(s - ref["stress"])))
    _say("max |E_i - site energy| %.2e eV, max |F| %.2e eV/A, max |dS| %.2e eV/A^3" % (de, df, ds))
    assert de < E_TOL and df < F_TOL and ds < S_TOL
    assert abs(total / n - ref["energy"] / len(small["numbers"])) < E_TOL


def test_graphs_beyond_32_bit_edge_ids_are_planned_tiled(medium_model_path):
    """n = 164 unperturbed (2.27B edges): the speed profile, which keeps the
    direct plan for a graph of 32-bit edge ids, gets the tiled plan with the
    reason stated; a request pinning a direct plan is refused with the
    reference's edge limit named."""
    from symmetrix import systems
    from symmetrix.mace_kokkos import MACEKokkosFloat
    system = systems.srtio3_supercell(164, sigma=0.0)
    pos = np.ascontiguousarray(system["positions"], np.float64).reshape(-1)
    cell = np.asarray(system["cell"], np.float64)
    args = (cell.reshape(-1), np.linalg.inv(cell).reshape(-1))

    def prepare(ev):
        lut = {int(z): i for i, z in enumerate(ev.atomic_numbers)}
        types = np.array([lut[int(z)] for z in system["numbers"]], np.int32)
        return ev._prepare_periodic_factorized_graph(types, pos, *args, ev.r_cut + SKIN)

    ev = MACEKokkosFloat(medium_model_path)
    ev.set_execution_plan_request("speed")
    g = prepare(ev)
    report = ev.execution_plan_report
    _say("speed profile at %d edges: %s (%s)" % (g["num_edges"], report["selected_id"], report["selection_reason"]))
    assert g["num_edges"] > 2**31
    assert report["selected_id"] == "mh0-dual-layer-tiled-v1"
    assert "32-bit edge ids" in report["selection_reason"]
    ev.close()
    ev = MACEKokkosFloat(medium_model_path)
    ev._set_execution_plan_request("direct", "speed", "mh0-direct-speed")
    with pytest.raises(ValueError, match="2\\^31 - 4096"):
        prepare(ev)
    ev.close()

