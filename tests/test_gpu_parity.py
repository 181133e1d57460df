"""Parity of the HIP path (through the C ABI) with the CPU oracle.

Bars (north star): neighbour lists bit-exact; FP32 energy within 1e-5
eV/atom, forces within 1e-4 eV/Angstrom, stress within 1e-6 eV/Angstrom^3 of
the oracle's FP32 restatement of the reference CPU path on the same inputs.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5   # eV/atom
F_TOL = 1e-4   # eV/A
S_TOL = 1e-6   # eV/A^3


def _oracle():
    from oracle import oracle
    return oracle


def _system(name):
    from symmetrix import systems
    if name == "tiny":
        return systems.srtio3_supercell(3, sigma=0.05, seed=0)
    if name == "medium":
        return systems.srtio3_supercell(10, sigma=0.05, seed=0)
    raise KeyError(name)


def _check_graph(pos, cell, cutoff):
    from symmetrix.mace_kokkos import neighbor_list
    ora = _oracle().neighbor_graph(pos, cell, cutoff)
    dev = neighbor_list(pos, cell, cutoff)
    for key in ("num_neigh", "offsets", "sources", "shifts"):
        np.testing.assert_array_equal(dev[key], ora[key], err_msg=key)
    # fractional edge vectors bit for bit
    assert dev["fractional_xyz"].tobytes() == ora["fractional_xyz"].tobytes()
    return dev


@pytest.mark.parametrize("name,cutoff", [("tiny", 5.5), ("tiny", 5.0), ("medium", 6.5)])
def test_neighbor_list_bit_exact(name, cutoff):
    s = _system(name)
    g = _check_graph(s["positions"], s["cell"], cutoff)
    assert len(g["sources"]) > 0


def test_neighbor_list_triclinic_and_wrapped():
    rng = np.random.default_rng(3)
    cell = np.array([[9.0, 0.0, 0.0], [2.5, 8.0, 0.0], [-1.5, 1.0, 10.0]])
    frac = rng.uniform(-0.5, 1.5, size=(60, 3))  # outside the cell on purpose
    pos = frac @ cell
    _check_graph(pos, cell, 4.0)


def test_neighbor_list_small_cell_many_images():
    cell = np.eye(3) * 3.0
    pos = np.array([[0.1, 0.2, 0.3], [1.6, 1.4, 1.5]])
    g = _check_graph(pos, cell, 5.0)
    # ~39 neighbours per atom within 5 A at 2 atoms per 27 A^3, images up to 3 cells away
    assert 60 < len(g["sources"]) < 100


def _evaluate_both(model_path, system, skin=0.5):
    from symmetrix.mace_kokkos import MACEKokkosFloat
    ora = _oracle()
    om = ora.OracleModel(model_path)
    ref = ora.evaluate_system(om, system, skin=skin)
    ev = MACEKokkosFloat(model_path)
    types = om.types_of(system["numbers"])
    cell = np.asarray(system["cell"], float)
    g = ev._prepare_periodic_factorized_graph(types, system["positions"], cell, np.linalg.inv(cell),
                                              ev.r_cut + skin)
    assert g["num_edges"] == len(ref["graph"]["sources"])
    ev._compute_prepared_factorized_positions(g["generation"], system["positions"])
    e = ev.node_energies
    f = ev._reduce_atom_forces(len(types), None, None, g["generation"])
    s = ev._reduce_stress(abs(np.linalg.det(cell)), None, g["generation"])
    return om, ref, ev, g, e, f, s


def _assert_efs(ref, e, f, s, n):
    de = abs(np.sum(e) - ref["energy"]) / n
    df = np.max(np.abs(f - ref["forces"]))
    ds = np.max(np.abs(s - ref["stress"]))
    print("energy/atom err %.3e  force err %.3e  stress err %.3e" % (de, df, ds))
    assert de < E_TOL
    assert df < F_TOL
    assert ds < S_TOL


def test_energy_forces_stress_tiny(tiny_model_path):
    s = _system("tiny")
    om, ref, ev, g, e, f, st = _evaluate_both(tiny_model_path, s)
    np.testing.assert_allclose(e, ref["energies"], rtol=0, atol=1e-4)
    _assert_efs(ref, e, f, st, len(e))


def _stage_err(a, b):
    scale = max(np.max(np.abs(b)), 1e-30)
    return float(np.max(np.abs(a - b)) / scale)


def test_stages_tiny(tiny_model_path):
    s = _system("tiny")
    om, ref, ev, g, e, f, st = _evaluate_both(tiny_model_path, s)
    for name in ("A0", "M0", "H1", "Phi1", "A1", "A1_adj", "dPhi1", "H1_adj", "A0_adj"):
        mine = ev._stage(name).astype(np.float64)
        theirs = om.stage(name)
        err = _stage_err(mine, theirs)
        print(name, "relative max err %.3e" % err)
        assert err < 1e-4, name
    m0adj = ev._stage("M0_adj").astype(np.float64).reshape(len(e), -1, om.num_channels)
    m0adj[:, 0, :] += ev._stage("direct").reshape(len(e), om.num_channels)
    assert _stage_err(m0adj.ravel(), om.stage("M0_adj")) < 1e-4
    # directed forces per edge
    nf = ev.node_forces.reshape(-1, 3)
    assert np.max(np.abs(nf - ref["node_forces"])) < 1e-5



def test_density_scaled_stages_and_efs(tiny_scaled_model_path):
    """A0/A1 density scaling (mace_kokkos_first_interaction.cpp:1335-1531,
    mace_kokkos_second_interaction.cpp:1310-1720) against the oracle: the
    scaled A0 and A1, the scaled adjoints, directed forces and E/F/S."""
    s = _system("tiny")
    om, ref, ev, g, e, f, st = _evaluate_both(tiny_scaled_model_path, s)
    for name in ("A0", "A1", "A1_adj", "dPhi1", "A0_adj"):
        err = _stage_err(ev._stage(name).astype(np.float64), om.stage(name))
        print(name, "relative max err %.3e" % err)
        assert err < 1e-4, name
    nf = ev.node_forces.reshape(-1, 3)
    assert np.max(np.abs(nf - ref["node_forces"])) < 1e-5
    _assert_efs(ref, e, f, st, len(e))


@pytest.mark.parametrize("tile", [37, 64])
def test_density_scaled_tiled_plan_matches_untiled(tiny_scaled_model_path, tile):
    """The three-sweep tiled plan with density scaling: the factors are
    per receiver, so tiles recompute them (A0 in sweeps 1 and 3, A1 in
    sweep 2) and add their edge-force terms to each tile's forces."""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    a = MACEKokkosFloat(tiny_scaled_model_path)
    types = np.array([{8: 0, 22: 1, 38: 2}[int(z)] for z in s["numbers"]], np.int32)
    e0, f0, s0 = _run(a, s, types)
    b = MACEKokkosFloat(tiny_scaled_model_path)
    b.set_execution_plan_request("capacity", tile)
    e1, f1, s1 = _run(b, s, types)
    assert b.execution_plan.startswith("direct-tiled")
    np.testing.assert_array_equal(e1, e0)
    np.testing.assert_allclose(f1, f0, rtol=0, atol=1e-7)
    np.testing.assert_allclose(s1, s0, rtol=0, atol=1e-9)


def test_zbl_efs_and_tiled_plan(tiny_zbl_model_path):
    """ZBL pair repulsion (zbl_kokkos.cpp:92-199) against the oracle: node
    energies, directed forces and E/F/S; the tiled plan equals the direct one."""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    om, ref, ev, g, e, f, st = _evaluate_both(tiny_zbl_model_path, s)
    assert np.max(np.abs(om.stage("zbl_forces"))) > 1e-3
    np.testing.assert_allclose(e, ref["energies"], rtol=0, atol=1e-4)
    nf = ev.node_forces.reshape(-1, 3)
    assert np.max(np.abs(nf - ref["node_forces"])) < 1e-5
    _assert_efs(ref, e, f, st, len(e))
    b = MACEKokkosFloat(tiny_zbl_model_path)
    b.set_execution_plan_request("capacity", 64)
    e1, f1, s1 = _run(b, s, om.types_of(s["numbers"]))
    assert b.execution_plan.startswith("direct-tiled")
    np.testing.assert_array_equal(e1, e)
    np.testing.assert_allclose(f1, f, rtol=0, atol=1e-7)
    np.testing.assert_allclose(s1, st, rtol=0, atol=1e-9)


@pytest.mark.parametrize("model", ["tiny_plu", "tiny_residual"])
def test_pre_linear_up_basis_and_residual(request, model):
    """The pre_linear_up H1 basis (x = M0[:,0,:] P0 for readout_1 and the H2
    skip, its adjoint entering M0 as P0 d) and the first-interaction residual
    (H1 += residual U, x += residual[lm 0]; mace.cpp:1759-1875) against the
    oracle: H1, the adjoints, directed forces and E/F/S; the tiled plan
    equals the direct one."""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    path = request.getfixturevalue(model + "_model_path")
    s = _system("tiny")
    om, ref, ev, g, e, f, st = _evaluate_both(path, s)
    for name in ("H1", "A1", "dPhi1", "H1_adj", "A0_adj"):
        err = _stage_err(ev._stage(name).astype(np.float64), om.stage(name))
        print(name, "relative max err %.3e" % err)
        assert err < 1e-4, name
    np.testing.assert_allclose(e, ref["energies"], rtol=0, atol=1e-4)
    nf = ev.node_forces.reshape(-1, 3)
    assert np.max(np.abs(nf - ref["node_forces"])) < 1e-5
    _assert_efs(ref, e, f, st, len(e))
    b = MACEKokkosFloat(path)
    b.set_execution_plan_request("capacity", 64)
    e1, f1, s1 = _run(b, s, om.types_of(s["numbers"]))
    assert b.execution_plan.startswith("direct-tiled")
    np.testing.assert_array_equal(e1, e)
    np.testing.assert_allclose(f1, f, rtol=0, atol=1e-7)
    np.testing.assert_allclose(s1, st, rtol=0, atol=1e-9)


def test_prediction_heads(tiny_heads_model_path, tiny_model_path, tmp_path):
    """MACEKokkos(filename, head) (mace_kokkos.hpp:91; prediction_heads.hpp):
    the head's energies and readouts are used, selected_head and
    available_heads are reported, unknown heads and malformed sections are
    refused; a file without a section names no head."""
    import json
    from symmetrix.mace_kokkos import MACEKokkosFloat
    ora = _oracle()
    s = _system("tiny")
    ev = MACEKokkosFloat(tiny_heads_model_path, "finetune")
    assert ev.selected_head == "finetune" and ev.available_heads == ["default", "finetune"]
    assert MACEKokkosFloat(tiny_heads_model_path).selected_head == "default"
    plain = MACEKokkosFloat(tiny_model_path)
    assert plain.selected_head == "" and plain.available_heads == []
    om = ora.OracleModel(tiny_heads_model_path, head="finetune")
    ref = ora.evaluate_system(om, s, skin=0.5)
    e, f, st = _run(ev, s, om.types_of(s["numbers"]))
    _assert_efs(ref, e, f, st, len(e))
    with pytest.raises(ValueError, match="not in the model"):
        MACEKokkosFloat(tiny_heads_model_path, "absent")
    with pytest.raises(ValueError, match="names no prediction head"):
        MACEKokkosFloat(tiny_model_path, "finetune")
    with open(tiny_heads_model_path) as fh:
        j = json.load(fh)
    j["prediction_heads"]["parameters"]["finetune"]["zbl_c"] = [0.1, 0.2, 0.3, 0.4]
    bad = tmp_path / "bad_heads.json"
    bad.write_text(json.dumps(j))
    with pytest.raises(ValueError, match="per-head fields"):
        MACEKokkosFloat(str(bad))


@pytest.mark.parametrize("tile", [0, 64])
def test_agnesi_per_pair_tables(tiny_agnesi_model_path, tile):
    """Agnesi distance transform (compact_radial.cpp:144-163): every pair of
    active types has its own R0/R1 and density tables, selected per edge;
    direct and tiled plans against the oracle."""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    ora = _oracle()
    s = _system("tiny")
    om = ora.OracleModel(tiny_agnesi_model_path)
    ref = ora.evaluate_system(om, s, skin=0.5)
    ev = MACEKokkosFloat(tiny_agnesi_model_path)
    if tile:
        ev.set_execution_plan_request("capacity", tile)
    e, f, st = _run(ev, s, om.types_of(s["numbers"]))
    if not tile:
        nf = ev.node_forces.reshape(-1, 3)
        assert np.max(np.abs(nf - ref["node_forces"])) < 1e-5
    _assert_efs(ref, e, f, st, len(e))

def test_energy_forces_stress_medium(medium_model_path):
    s = _system("medium")
    om, ref, ev, g, e, f, st = _evaluate_both(medium_model_path, s)
    _assert_efs(ref, e, f, st, len(e))


def test_energy_forces_stress_irregular(medium_model_path):
    """20,000 atoms uniform at 0.08 /A^3 with a 1.8 A
    minimum separation, 10 species (55 pair types) -- a wide spread of
    neighbour counts per receiver."""
    from symmetrix import systems
    s = systems.irregular_box(20000, density=0.08, min_distance=1.8, seed=0)
    om, ref, ev, g, e, f, st = _evaluate_both(medium_model_path, s)
    counts = np.diff(ref["graph"]["offsets"])
    print("neighbours per receiver: min %d max %d mean %.1f" % (counts.min(), counts.max(), counts.mean()))
    assert counts.max() - counts.min() > 20
    _assert_efs(ref, e, f, st, len(e))


def test_energy_forces_stress_wide(wide_model_path):
    """BASELINE configs[4] shape: 256 channels, 0e+1o+2e hidden (L_max 2, 243
    coupling rows run as two source-component passes), l_max 3,
    correlation 3, r_cut 5 A, on a rigid-water box (1,000 molecules, 3,000
    atoms; the config's 30,000-atom box has the same per-atom work)."""
    from symmetrix import systems
    s = systems.water_box(1000, seed=0)
    om, ref, ev, g, e, f, st = _evaluate_both(wide_model_path, s)
    assert "polynomials=unrolled" in ev.execution_plan
    for name in ("Phi1", "A1", "dPhi1", "H1_adj"):
        err = _stage_err(ev._stage(name).astype(np.float64), om.stage(name))
        print(name, "relative max err %.3e" % err)
        assert err < 1e-4, name
    _assert_efs(ref, e, f, st, len(e))


@pytest.mark.timeout(900)
def test_energy_forces_stress_wide_full_size(wide_model_path):
    """BASELINE configs[4] at its stated size: 10,000 rigid waters (30,000
    atoms, L = 66.9 A) with the wide model, against the oracle."""
    from symmetrix import systems
    s = systems.water_box(10000, seed=0)
    print("wide 30,000-atom box: oracle and HIP path", flush=True)
    om, ref, ev, g, e, f, st = _evaluate_both(wide_model_path, s)
    assert len(e) == 30000
    print("edges %d, plan %s" % (g["num_edges"], ev.execution_plan), flush=True)
    _assert_efs(ref, e, f, st, len(e))


def test_repeat_calls_bitwise_deterministic(tiny_model_path):
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    ev = MACEKokkosFloat(tiny_model_path)
    types = np.array([{8: 0, 22: 1, 38: 2}[int(z)] for z in s["numbers"]], np.int32)
    cell = s["cell"]
    g = ev._prepare_periodic_factorized_graph(types, s["positions"], cell, np.linalg.inv(cell), ev.r_cut + 0.5)
    outs = []
    for _ in range(3):
        ev._compute_prepared_factorized_positions(g["generation"], s["positions"])
        outs.append((ev.node_energies.tobytes(), ev.node_forces.tobytes()))
    assert outs[0] == outs[1] == outs[2]


def _run(ev, s, types, skin=0.5):
    cell = np.asarray(s["cell"], float)
    g = ev._prepare_periodic_factorized_graph(types, s["positions"], cell, np.linalg.inv(cell), ev.r_cut + skin)
    ev._compute_prepared_factorized_positions(g["generation"], s["positions"])
    e = ev.node_energies
    f = ev._reduce_atom_forces(len(types), None, None, g["generation"])
    st = ev._reduce_stress(abs(np.linalg.det(cell)), None, g["generation"])
    return e, f, st


@pytest.mark.parametrize("tile", [37, 64, 135])
def test_tiled_plan_matches_untiled_tiny(tiny_model_path, tile):
    """Three-sweep tiled plan (mace_kokkos_evaluate.cpp:755-1148) against the
    untiled direct plan on the same graph (test_dual_layer_fixed_workspace.py:
    106-128 compares the two at rtol 2e-4 / atol 2e-5 in FP32)."""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    a = MACEKokkosFloat(tiny_model_path)
    a.set_execution_plan_request("speed")
    types = np.array([{8: 0, 22: 1, 38: 2}[int(z)] for z in s["numbers"]], np.int32)
    e0, f0, s0 = _run(a, s, types)
    assert a.execution_plan.startswith("direct ")
    b = MACEKokkosFloat(tiny_model_path)
    b.set_execution_plan_request("capacity", tile)
    e1, f1, s1 = _run(b, s, types)
    assert b.execution_plan.startswith("direct-tiled")
    np.testing.assert_array_equal(e1, e0)
    np.testing.assert_allclose(f1, f0, rtol=0, atol=1e-7)
    np.testing.assert_allclose(s1, s0, rtol=0, atol=1e-9)
    with pytest.raises(RuntimeError):
        b.node_forces  # directed forces are not retained by the tiled plan


def test_tiled_plan_medium_against_oracle(medium_model_path):
    from symmetrix.mace_kokkos import MACEKokkosFloat
    ora = _oracle()
    s = _system("medium")
    om = ora.OracleModel(medium_model_path)
    ref = ora.evaluate_system(om, s, skin=0.5)
    ev = MACEKokkosFloat(medium_model_path)
    ev.set_execution_plan_request("capacity", 1024)
    e, f, st = _run(ev, s, om.types_of(s["numbers"]))
    assert "tiles=5" in ev.execution_plan
    _assert_efs(ref, e, f, st, len(e))


def test_host_edge_vectors_path(tiny_model_path):
    """compute_node_energies_forces with host xyz/r (token 0) equals the
    prepared-positions path on the same graph."""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    ora = _oracle()
    s = _system("tiny")
    om = ora.OracleModel(tiny_model_path)
    ref = ora.evaluate_system(om, s, skin=0.5)
    g = ref["graph"]
    types = om.types_of(s["numbers"])
    ev = MACEKokkosFloat(tiny_model_path)
    ev.compute_node_energies_forces(len(types), types, g["num_neigh"], g["sources"], types[g["sources"]],
                                    ref["xyz"], ref["r"])
    e = ev.node_energies
    nf = ev.node_forces.reshape(-1, 3)
    f = ev._reduce_atom_forces(len(types), g["receivers"], g["sources"], 0)
    assert abs(e.sum() - ref["energy"]) / len(e) < E_TOL
    assert np.max(np.abs(f - ref["forces"])) < F_TOL
    assert np.max(np.abs(nf - ref["node_forces"])) < 1e-5


def _run_tiny(model_path, system):
    from symmetrix.mace_kokkos import MACEKokkosFloat
    ev = MACEKokkosFloat(model_path)
    lut = {z: i for i, z in enumerate(ev.atomic_numbers)}
    types = np.array([lut[int(z)] for z in system["numbers"]], np.int32)
    cell = np.asarray(system["cell"], float)
    g = ev._prepare_periodic_factorized_graph(types, system["positions"], cell, np.linalg.inv(cell),
                                              ev.r_cut + 0.5)
    ev._compute_prepared_factorized_positions(g["generation"], system["positions"])
    f = ev._reduce_atom_forces(len(types), None, None, g["generation"])
    return ev, ev.node_energies, f


def test_table_driven_polynomials_match_unrolled(tiny_model_path, tmp_path):
    """A model whose M0 list carries one extra zero-coefficient monomial is
    the same function, but its canonical list no longer equals the compiled
    table, so it runs through the table-driven polynomial kernels."""
    import json
    s = _system("tiny")
    ev_a, e_a, f_a = _run_tiny(tiny_model_path, s)
    assert "polynomials=unrolled" in ev_a.execution_plan
    with open(tiny_model_path) as fh:
        j = json.load(fh)
    monos = j["M0_monomials"]["1"]
    extra = [5]
    assert extra not in monos
    monos.append(extra)
    for t in j["M0_weights"]:
        for k in j["M0_weights"][t]["1"]:
            j["M0_weights"][t]["1"][k].append(0.0)
    path = str(tmp_path / "tiny_extra_monomial.json")
    with open(path, "w") as fh:
        json.dump(j, fh)
    ev_b, e_b, f_b = _run_tiny(path, s)
    assert "polynomials=table" in ev_b.execution_plan
    np.testing.assert_allclose(e_b, e_a, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(f_b, f_a, rtol=1e-5, atol=1e-7)


def _device_copy(a):
    """Device copy of a numpy array through the HIP runtime the library
    uses (hipMalloc + hipMemcpy); returns (pointer, free)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipFree.argtypes = [ctypes.c_void_p]
    a = np.ascontiguousarray(a, dtype=np.float64)
    p = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(a.nbytes)) == 0
    assert hip.hipMemcpy(p, a.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(a.nbytes), 1) == 0
    return p.value, lambda: hip.hipFree(p)


def test_device_positions_call_matches_host_positions(tiny_model_path):
    """The device-positions call returns once the geometry is checked and
    leaves the model kernels queued on the evaluator stream; outputs read
    through the stream-ordered reductions equal the host-positions call's."""
    from symmetrix._native import check, lib
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    ev = MACEKokkosFloat(tiny_model_path)
    types = np.array([{8: 0, 22: 1, 38: 2}[int(z)] for z in s["numbers"]], np.int32)
    cell = np.asarray(s["cell"], float)
    vol = abs(np.linalg.det(cell))
    e0, f0, s0 = _run(ev, s, types)
    gen = ev._prepare_periodic_factorized_graph(types, s["positions"], cell, np.linalg.inv(cell),
                                                ev.r_cut + 0.5)["generation"]
    d_pos, free = _device_copy(s["positions"])
    try:
        for _ in range(2):
            ev._compute_prepared_factorized_positions_device(gen, d_pos)
            check(lib.smx_reduce_prepared_node_forces(ev._h, gen, None))
            check(lib.smx_reduce_prepared_stress(ev._h, gen, vol, None))
        ev.synchronize()
    finally:
        free()
    f1 = ev._reduce_atom_forces(len(types), None, None, gen)
    s1 = ev._reduce_stress(vol, None, gen)
    assert ev.node_energies.tobytes() == e0.tobytes()
    assert f1.tobytes() == f0.tobytes()
    assert s1.tobytes() == s0.tobytes()


def test_invalid_positions_raise_and_next_call_recovers(tiny_model_path):
    """A non-finite position is refused on the host for host positions
    (mace_kokkos_factorized_lifecycle.cpp:686-690); on the device it makes
    every edge of that atom invalid and the call raises after the geometry
    (mace_kokkos_factorized_lifecycle.cpp:766-794).  A following valid call
    gives the same results as before."""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    ev = MACEKokkosFloat(tiny_model_path)
    types = np.array([{8: 0, 22: 1, 38: 2}[int(z)] for z in s["numbers"]], np.int32)
    cell = np.asarray(s["cell"], float)
    g = ev._prepare_periodic_factorized_graph(types, s["positions"], cell, np.linalg.inv(cell), ev.r_cut + 0.5)
    gen = g["generation"]
    ev._compute_prepared_factorized_positions(gen, s["positions"])
    e0 = ev.node_energies.copy()
    bad = np.array(s["positions"], dtype=np.float64)
    bad[1, 0] = np.nan
    with pytest.raises(ValueError, match="finite"):
        ev._compute_prepared_factorized_positions(gen, bad)
    d_bad, free = _device_copy(bad)
    try:
        with pytest.raises(ValueError, match="invalid edge geometry"):
            ev._compute_prepared_factorized_positions_device(gen, d_bad)
        ev.synchronize()
    finally:
        free()
    ev._compute_prepared_factorized_positions(gen, s["positions"])
    assert ev.node_energies.tobytes() == e0.tobytes()


def test_atomic_energies_and_active_elements(tiny_model_path, tiny_agnesi_model_path):
    """atomic_energies and active_atomic_numbers (pybind mace_kokkos.cpp:
    1900-1909): E0 as the file holds it; every element for a model without
    per-pair tables, the tabulated ones for a model with them."""
    import json
    from symmetrix.mace_kokkos import MACEKokkosFloat
    with open(tiny_model_path) as f:
        e0 = np.asarray(json.load(f)["atomic_energies"], float).ravel()
    ev = MACEKokkosFloat(tiny_model_path)
    np.testing.assert_array_equal(ev.atomic_energies, e0[: ev.num_elements])
    assert ev.active_atomic_numbers == ev.atomic_numbers
    ag = MACEKokkosFloat(tiny_agnesi_model_path)
    ag.prepare_active_types([1])
    assert ag.active_atomic_numbers == [ag.atomic_numbers[1]]


def test_a_failed_prepare_voids_the_previous_token(tiny_field_model_path):
    """A prepare that fails after it has started to replace the graph (here
    the plan step: a MACEField model with the tiled plan pinned) leaves no
    token that runs on the half-replaced graph: the previous token is stale,
    and a new prepare works."""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    ev = MACEKokkosFloat(tiny_field_model_path)
    lut = {int(z): i for i, z in enumerate(ev.atomic_numbers)}
    types = np.array([lut[int(z)] for z in s["numbers"]], np.int32)
    pos = np.ascontiguousarray(s["positions"], np.float64).reshape(-1)
    cell = np.asarray(s["cell"], np.float64)

    def prepare():
        return ev._prepare_periodic_factorized_graph(types, pos, cell.reshape(-1), np.linalg.inv(cell).reshape(-1),
                                                     ev.r_cut + 0.5)["generation"]

    field = np.array([0.1, 0.0, -0.05])
    g1 = prepare()
    ev._compute_prepared_factorized_positions_field(g1, pos, field)
    e1 = np.array(ev.node_energies)
    ev._set_execution_plan_request("direct", "capacity", "mh0-dual-layer-tiled-v1")
    with pytest.raises(ValueError, match="field coupling"):
        prepare()
    with pytest.raises(ValueError, match="stale"):
        ev._compute_prepared_factorized_positions_field(g1, pos, field)
    ev._set_execution_plan_request("direct", "capacity", "")
    g2 = prepare()
    ev._compute_prepared_factorized_positions_field(g2, pos, field)
    np.testing.assert_array_equal(np.array(ev.node_energies), e1)
    ev.close()
