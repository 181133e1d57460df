"""One GPU's share of a domain-decomposed evaluation (the LAMMPS multi-rank
path, pair_symmetrix_mace_kokkos.cpp:1285-1704; the evaluator's split phases,
mace_kokkos_evaluate.cpp:1495-1990; feature graphs, mace_kokkos_factorized_
lifecycle.cpp:949-1104).

A periodic system is cut into slabs.  Each slab gets its own evaluator over a
graph of its receivers and the ghost atoms their edges leave, with the
feature nodes in a shuffled order (receivers among them).  Between the phases
the H1 rows and their adjoints are exchanged on the host, as LAMMPS's forward
and reverse communication would move them between ranks.  The sums over the
slabs must give the whole system's energies, forces and stress: the oracle's,
and this library's own whole-system evaluation to FP32 summation order.
"""

import numpy as np
import pytest

from test_gpu_parity import _assert_efs, _system

pytestmark = pytest.mark.gpu


def _slabs(s, ref, parts, seed):
    """per slab: receivers (global ids, shuffled), feature nodes (global ids,
    shuffled), the receivers' feature indices and the slab's CSR"""
    g = ref["graph"]
    cell = np.asarray(s["cell"], float)
    frac = (np.asarray(s["positions"], float) @ np.linalg.inv(cell))[:, 0] % 1.0
    owner = np.minimum((frac * parts).astype(int), parts - 1)
    rng = np.random.default_rng(seed)
    off, src = g["offsets"], g["sources"]
    out = []
    for d in range(parts):
        recv = rng.permutation(np.flatnonzero(owner == d))
        edges = np.concatenate([np.arange(off[i], off[i + 1]) for i in recv]) if recv.size else np.zeros(0, int)
        ghosts = np.setdiff1d(np.unique(src[edges]), recv)
        feats = rng.permutation(np.concatenate([recv, ghosts]))
        index = {int(a): k for k, a in enumerate(feats)}
        out.append(dict(recv=recv, feats=feats, edges=edges,
                        rfi=np.array([index[int(a)] for a in recv], np.int32),
                        neigh=np.array([index[int(a)] for a in src[edges]], np.int32),
                        num_neigh=(off[recv + 1] - off[recv]).astype(np.int32)))
    return out


def _run(path, s, ref, types, parts, seed=0, field=None, tile=0):
    """the slabs' split-phase evaluations with the host exchange; energies,
    forces and stress summed over the slabs (and dE/dE in a field: one field,
    or one per atom given to each slab for its feature nodes)"""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    n = len(types)
    slabs = _slabs(s, ref, parts, seed)
    evs = []
    for sl in slabs:
        ev = MACEKokkosFloat(path)
        if tile:
            ev.set_execution_plan_request("capacity", tile)
        if field is not None:
            ev._set_electric_field(field if np.size(field) == 3 else np.asarray(field)[sl["feats"]])
        sl["gen"] = ev._prepare_factorized_feature_graph(
            len(sl["recv"]), len(sl["feats"]), sl["rfi"], types[sl["recv"]], types[sl["feats"]], sl["num_neigh"],
            sl["neigh"], types[ref["graph"]["sources"][sl["edges"]]])
        if tile:
            assert ev.execution_plan_report["selected_id"].endswith("tiled-v1")
        sl["xyz"] = ref["xyz"].reshape(-1, 3)[sl["edges"]]
        sl["r"] = ref["r"][sl["edges"]]
        evs.append(ev)
    if evs[0].num_interactions == 1:
        for ev, sl in zip(evs, slabs):
            ev._compute_factorized_single_layer_distributed_evaluation(sl["gen"], sl["xyz"], sl["r"])
    else:
        for ev, sl in zip(evs, slabs):
            ev._begin_factorized_distributed_evaluation(sl["gen"], sl["xyz"], sl["r"])
        # forward communication: each atom's H1 row from its owner
        rows = [ev._distributed_h1() for ev in evs]
        H1 = np.zeros((n, rows[0].shape[1]), np.float32)
        for sl, h in zip(slabs, rows):
            H1[sl["recv"]] = h
        for ev, sl in zip(evs, slabs):
            ev._continue_factorized_distributed_evaluation(H1[sl["feats"]])
        # reverse communication: every image's adjoint summed onto the owner
        adj = np.zeros_like(H1, dtype=np.float64)
        for ev, sl in zip(evs, slabs):
            np.add.at(adj, sl["feats"], ev._distributed_h1_adjoint().astype(np.float64))
        for ev, sl in zip(evs, slabs):
            ev._finish_factorized_distributed_evaluation(adj[sl["feats"]].astype(np.float32))
    e = np.zeros(n)
    f = np.zeros((n, 3))
    st = np.zeros((3, 3))
    adj = None if field is None else np.zeros(np.shape(field))
    V = abs(np.linalg.det(np.asarray(s["cell"], float)))
    for ev, sl in zip(evs, slabs):
        e[sl["recv"]] = ev.node_energies
        np.add.at(f, sl["feats"], ev._reduce_atom_forces(len(sl["feats"]), None, None, sl["gen"]))
        st += ev._reduce_stress(V, None, sl["gen"])
        if field is not None and np.size(field) == 3:
            adj += ev.electric_field_adj
        elif field is not None:
            np.add.at(adj, sl["feats"], ev.electric_field_adj.reshape(-1, 3))
    if field is not None:
        return e, f, st, adj
    return e, f, st


@pytest.mark.parametrize("model", ["tiny", "tiny_residual", "tiny_agnesi", "tiny_scaled", "tiny_zbl",
                                   "tiny_single"])
@pytest.mark.parametrize("parts,tile", [(2, 0), (3, 0), (2, 16)])
def test_slabs_sum_to_the_whole_system(request, model, parts, tile):
    """tile > 0: each slab under its tiled plan, tiles of at most that many
    receivers (the sweeps split at the same exchanges)"""
    from oracle import oracle
    from symmetrix.mace_kokkos import MACEKokkosFloat
    path = request.getfixturevalue(model + "_model_path")
    s = _system("tiny")
    om = oracle.OracleModel(path)
    ref = oracle.evaluate_system(om, s, skin=0.5)
    types = om.types_of(s["numbers"])
    n = len(types)
    e, f, st = _run(path, s, ref, types, parts, tile=tile)
    _assert_efs(ref, e, f, st, n)
    np.testing.assert_allclose(e, ref["energies"], rtol=0, atol=1e-4)
    # the whole system on one evaluator, same graph and edge vectors
    whole = MACEKokkosFloat(path)
    g = ref["graph"]
    gen = whole._prepare_factorized_graph(n, types, g["num_neigh"], g["sources"], types[g["sources"]])
    whole._compute_prepared_factorized(gen, ref["xyz"], ref["r"])
    fw = whole._reduce_atom_forces(n, None, None, gen)
    print("slabs vs whole: energy %.3e force %.3e" % (np.max(np.abs(e - whole.node_energies)),
                                                     np.max(np.abs(f - fw))))
    np.testing.assert_allclose(e, whole.node_energies, rtol=0, atol=2e-5)
    np.testing.assert_allclose(f, fw, rtol=0, atol=2e-5)


@pytest.mark.parametrize("model", ["tiny_field", "field_l2"])
def test_slabs_in_an_electric_field(request, model):
    """MACEField: H1 is exchanged before the field (H1p) and the field paths
    run over every feature node; each slab's dE/dE is its part of the whole
    (one field), or its feature nodes' parts (one field per atom)"""
    from oracle import oracle
    path = request.getfixturevalue(model + "_model_path")
    s = _system("tiny")
    om = oracle.OracleModel(path)
    types = om.types_of(s["numbers"])
    n = len(types)
    field = np.array([0.12, -0.21, 0.27])
    per = np.tile(field, (n, 1)) + 0.05 * np.random.default_rng(4).normal(size=(n, 3))
    for fld in (field, per):
        ref = oracle.evaluate_system(om, s, skin=0.5, field=fld)
        e, f, st, adj = _run(path, s, ref, types, 3, seed=2, field=fld)
        _assert_efs(ref, e, f, st, n)
        np.testing.assert_allclose(e, ref["energies"], rtol=0, atol=1e-4)
        scale = max(np.max(np.abs(ref["field_adj"])), 1e-30)
        err = np.max(np.abs(adj.ravel() - ref["field_adj"])) / scale
        print("dE/dE relative max err %.3e" % err)
        assert err < 2e-5


def test_a_slab_without_receivers(tiny_model_path):
    """a rank whose domain holds no atoms still passes through the phases
    (its H1 adjoint rows are zero)"""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    ev = MACEKokkosFloat(tiny_model_path)
    gen = ev._prepare_factorized_feature_graph(0, 4, [], [], [0, 1, 2, 0], [], [], [])
    ev._begin_factorized_distributed_evaluation(gen, np.zeros((0, 3)), np.zeros(0))
    assert ev._distributed_h1().shape[0] == 0
    w = ev._distributed_rows(0).shape[1]
    ev._continue_factorized_distributed_evaluation(np.ones((4, w), np.float32))
    adj = ev._distributed_h1_adjoint()
    assert adj.shape == (4, w) and not adj.any()
    ev._finish_factorized_distributed_evaluation()
    assert ev.node_energies.size == 0
    assert not ev._reduce_atom_forces(4, None, None, gen).any()


def test_phase_order_and_refusals(tiny_model_path, tiny_single_model_path, tiny_field_model_path):
    from oracle import oracle
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = _system("tiny")
    om = oracle.OracleModel(tiny_model_path)
    ref = oracle.evaluate_system(om, s, skin=0.5)
    types = om.types_of(s["numbers"])
    sl = _slabs(s, ref, 2, 1)[0]
    args = (len(sl["recv"]), len(sl["feats"]), sl["rfi"], types[sl["recv"]], types[sl["feats"]], sl["num_neigh"],
            sl["neigh"], types[ref["graph"]["sources"][sl["edges"]]])
    xyz, r = ref["xyz"].reshape(-1, 3)[sl["edges"]], ref["r"][sl["edges"]]
    ev = MACEKokkosFloat(tiny_model_path)
    assert ev.low_memory
    ev._set_low_memory(False)
    assert not ev.low_memory
    gen = ev._prepare_factorized_feature_graph(*args)
    assert ev.factorized_graph_generation == gen and ev.factorized_prepared_graph_count == 1
    assert (ev.execution_active_receiver_count, ev.execution_active_feature_node_count,
            ev.execution_active_edge_count) == (len(sl["recv"]), len(sl["feats"]), len(sl["edges"]))
    # a two-interaction model needs the exchange: no plain call over ghosts
    with pytest.raises(ValueError, match="split phases"):
        ev._compute_prepared_factorized(gen, xyz, r)
    from symmetrix._native import check, lib
    with pytest.raises(RuntimeError, match="prefix"):
        check(lib.smx_continue_factorized_distributed_evaluation(ev._h, None, 0, 0))
    ev._begin_factorized_distributed_evaluation(gen, xyz, r)
    with pytest.raises(RuntimeError, match="already active"):
        ev._begin_factorized_distributed_evaluation(gen, xyz, r)
    with pytest.raises(RuntimeError, match="distributed evaluation"):
        ev._prepare_factorized_feature_graph(*args)
    w = ev._distributed_h1().shape[1]
    with pytest.raises(ValueError, match="shape"):
        ev._continue_factorized_distributed_evaluation(np.zeros((len(sl["feats"]) - 1, w), np.float32))
    with pytest.raises(RuntimeError, match="middle phase"):
        ev._finish_factorized_distributed_evaluation()
    # a refused phase leaves the evaluator idle: the one-call form still runs
    ev2 = MACEKokkosFloat(tiny_single_model_path)
    gen2 = ev2._prepare_factorized_feature_graph(*args)
    with pytest.raises(ValueError, match="one call"):
        ev2._begin_factorized_distributed_evaluation(gen2, xyz, r)
    ev2._compute_factorized_single_layer_distributed_evaluation(gen2, xyz, r)
    assert np.all(np.isfinite(ev2.node_energies))
    # graph checks
    bad = list(args)
    bad[2] = np.zeros_like(sl["rfi"])
    with pytest.raises(ValueError, match="unique|disagree"):
        MACEKokkosFloat(tiny_model_path)._prepare_factorized_feature_graph(*bad)
    bad = list(args)
    bad[6] = np.where(np.arange(len(sl["neigh"])) == 0, len(sl["feats"]), sl["neigh"]).astype(np.int32)
    with pytest.raises(ValueError, match="out of range"):
        MACEKokkosFloat(tiny_model_path)._prepare_factorized_feature_graph(*bad)
    # the positions form needs explicit feature nodes
    pl = MACEKokkosFloat(tiny_model_path)
    g = ref["graph"]
    pg = pl._prepare_factorized_graph(len(types), types, g["num_neigh"], g["sources"], types[g["sources"]])
    with pytest.raises(ValueError, match="feature nodes"):
        pl._begin_factorized_distributed_positions_evaluation(pg, s["positions"])
    # a field-coupled model needs its field before the phases
    fev = MACEKokkosFloat(tiny_field_model_path)
    fgen = fev._prepare_factorized_feature_graph(*args)
    with pytest.raises(ValueError, match="electric field"):
        fev._begin_factorized_distributed_evaluation(fgen, xyz, r)


def test_device_forms_as_the_pair_style_calls_them(tiny_model_path):
    """The C entry points with device arrays, in the order the pair style's
    mpi_message_passing compute makes them: the feature graph from device
    arrays, device edge vectors, the exchange rows read and (reverse
    communication) written in place in device memory, finish without rows."""
    import ctypes
    from oracle import oracle
    from symmetrix._native import check, lib
    from symmetrix.mace_kokkos import MACEKokkosFloat
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipFree.argtypes = [ctypes.c_void_p]
    held = []

    def dev(a):
        a = np.ascontiguousarray(a)
        p = ctypes.c_void_p()
        assert hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(max(a.nbytes, 8))) == 0
        assert hip.hipMemcpy(p, a.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(a.nbytes), 1) == 0
        held.append(p)
        return p

    def to_host(p, shape):
        out = np.zeros(shape, np.float32)
        assert hip.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), p, ctypes.c_size_t(out.nbytes), 2) == 0
        return out

    s = _system("tiny")
    om = oracle.OracleModel(tiny_model_path)
    ref = oracle.evaluate_system(om, s, skin=0.5)
    types = om.types_of(s["numbers"]).astype(np.int32)
    n = len(types)
    slabs = _slabs(s, ref, 2, 3)
    evs = []
    try:
        for sl in slabs:
            ev = MACEKokkosFloat(tiny_model_path)
            gen = ctypes.c_uint64()
            src = ref["graph"]["sources"][sl["edges"]]
            check(lib.smx_prepare_factorized_feature_graph_device(
                ev._h, len(sl["recv"]), len(sl["feats"]), dev(sl["rfi"]), dev(types[sl["recv"]]),
                dev(types[sl["feats"]]), dev(sl["num_neigh"]), len(sl["edges"]), dev(sl["neigh"]),
                dev(types[src]), ctypes.byref(gen)))
            sl["gen"] = gen.value
            check(lib.smx_begin_factorized_distributed_evaluation(
                ev._h, gen.value, len(sl["recv"]), len(sl["feats"]), dev(ref["xyz"].reshape(-1, 3)[sl["edges"]]),
                dev(ref["r"][sl["edges"]]), 1))
            ev._num_nodes, ev._num_feature_nodes, ev._num_edges = len(sl["recv"]), len(sl["feats"]), len(sl["edges"])
            evs.append(ev)

        def rows(ev, which):
            p, cnt, w = ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_int64()
            check(lib.smx_distributed_exchange(ev._h, which, ctypes.byref(p), ctypes.byref(cnt), ctypes.byref(w)))
            return p, cnt.value, w.value

        H1 = None
        for ev, sl in zip(evs, slabs):
            p, cnt, w = rows(ev, 0)
            H1 = np.zeros((n, w), np.float32) if H1 is None else H1
            H1[sl["recv"]] = to_host(p, (cnt, w))
        for ev, sl in zip(evs, slabs):
            check(lib.smx_continue_factorized_distributed_evaluation(ev._h, dev(H1[sl["feats"]]), len(sl["feats"]),
                                                                     1))
        adj = np.zeros(H1.shape)
        ptrs = []
        for ev, sl in zip(evs, slabs):
            p, cnt, w = rows(ev, 1)
            np.add.at(adj, sl["feats"], to_host(p, (cnt, w)).astype(np.float64))
            ptrs.append(p)
        for ev, sl, p in zip(evs, slabs, ptrs):
            mine = np.ascontiguousarray(adj[sl["feats"]], dtype=np.float32)
            assert hip.hipMemcpy(p, mine.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(mine.nbytes), 1) == 0
            check(lib.smx_finish_factorized_distributed_evaluation(ev._h, None, 0, 1))
        e = np.zeros(n)
        f = np.zeros((n, 3))
        for ev, sl in zip(evs, slabs):
            e[sl["recv"]] = ev.node_energies
            np.add.at(f, sl["feats"], ev._reduce_atom_forces(len(sl["feats"]), None, None, sl["gen"]))
        np.testing.assert_allclose(e, ref["energies"], rtol=0, atol=1e-4)
        assert np.max(np.abs(f - ref["forces"])) < 1e-4
    finally:
        for p in held:
            hip.hipFree(p)


@pytest.mark.parametrize("model,form,tile", [("tiny", "xyz", 0), ("tiny_field", "xyz", 0),
                                             ("tiny", "positions", 0), ("tiny", "positions", 16),
                                             ("tiny_single", "positions", 16)])
def test_one_rank_with_ghost_images_as_the_pair_style_runs_it(request, model, form, tile):
    """The pair style's mpi_message_passing compute on one rank: local atoms
    (in a shuffled ilist order) are the receivers, the local atoms and their
    26 ghost images are the feature nodes by LAMMPS index, the forward
    communication copies each ghost's H1 row from its owner, the reverse
    communication adds each ghost's adjoint row onto its owner, and the ghost
    rows of the forces are folded onto their owners (LAMMPS's reverse
    communication of f)."""
    from oracle import oracle
    from symmetrix.mace_kokkos import MACEKokkosFloat
    from test_lammps_entry import _lammps_arrays
    path = request.getfixturevalue(model + "_model_path")
    s = _system("tiny")
    om = oracle.OracleModel(path)
    field = np.array([0.12, -0.21, 0.27]) if model == "tiny_field" else None
    ref = oracle.evaluate_system(om, s, skin=0.5, field=field)
    ev = MACEKokkosFloat(path)
    lut = {int(z): i for i, z in enumerate(ev.atomic_numbers)}
    species = sorted(set(int(z) for z in s["numbers"]))
    allpos, owner, alltypes, rows = _lammps_arrays(np.asarray(s["positions"], float), np.asarray(s["cell"], float),
                                                   s["numbers"], ev.r_cut + 0.5,
                                                   {z: t + 1 for t, z in enumerate(species)})
    n, nall = len(rows), len(allpos)
    model_type = np.array([lut[species[t - 1]] for t in alltypes], np.int32)
    ilist = np.random.default_rng(5).permutation(n).astype(np.int32)
    neigh = np.concatenate([rows[i] for i in ilist]).astype(np.int32)
    recv = np.repeat(ilist, [len(rows[i]) for i in ilist])
    xyz = allpos[neigh] - allpos[recv]
    d = np.linalg.norm(xyz, axis=1)
    sc = np.where(d >= ev.r_cut, ev.r_cut / d, 1.0)
    xyz, r = xyz * sc[:, None], d * sc
    if field is not None:
        ev._set_electric_field(field)
    if tile:
        ev.set_execution_plan_request("capacity", tile)
    gen = ev._prepare_factorized_feature_graph(n, nall, ilist, model_type[ilist], model_type,
                                               np.array([len(rows[i]) for i in ilist], np.int32), neigh,
                                               model_type[neigh])
    if ev.num_interactions == 1:
        ev._compute_factorized_single_layer_distributed_positions_evaluation(gen, allpos)
    else:
        if form == "positions":
            ev._begin_factorized_distributed_positions_evaluation(gen, allpos)
        else:
            ev._begin_factorized_distributed_evaluation(gen, xyz, r)
        h = ev._distributed_h1()
        H1 = np.zeros((nall, h.shape[1]), np.float32)
        H1[ilist] = h
        H1[n:] = H1[owner[n:]]                      # forward communication
        ev._continue_factorized_distributed_evaluation(H1)
        adj = ev._distributed_h1_adjoint().astype(np.float64)
        np.add.at(adj, owner[n:], adj[n:])          # reverse communication
        ev._finish_factorized_distributed_evaluation(adj.astype(np.float32))
    e = np.zeros(n)
    e[ilist] = ev.node_energies
    f_all = ev._reduce_atom_forces(nall, None, None, gen)
    f = np.zeros((n, 3))
    np.add.at(f, owner, f_all)                  # ghost forces onto owners
    st = ev._reduce_stress(abs(np.linalg.det(np.asarray(s["cell"], float))), None, gen)
    _assert_efs(ref, e, f, st, n)
    np.testing.assert_allclose(e, ref["energies"], rtol=0, atol=1e-4)
    if field is not None:
        scale = np.max(np.abs(ref["field_adj"]))
        np.testing.assert_allclose(ev.electric_field_adj, ref["field_adj"], rtol=0, atol=2e-5 * scale)


def test_medium_slabs_sum_to_the_whole_system(medium_model_path):
    """The benchmark workload (5,000 atoms, 496k edges) cut into two slabs:
    the slabs' energies, forces and stress equal the one-evaluator call on
    the same graph and edge vectors (size-independent check of the split
    phases at full size)."""
    from symmetrix.mace_kokkos import MACEKokkosFloat, neighbor_list
    s = _system("medium")
    whole = MACEKokkosFloat(medium_model_path)
    lut = {int(z): i for i, z in enumerate(whole.atomic_numbers)}
    types = np.array([lut[int(z)] for z in s["numbers"]], np.int32)
    cell = np.asarray(s["cell"], float)
    g = neighbor_list(np.asarray(s["positions"], float), cell, whole.r_cut + 0.5)
    xyz = g["fractional_xyz"] @ cell
    d = np.linalg.norm(xyz, axis=1)
    sc = np.where(d >= whole.r_cut, whole.r_cut / d, 1.0)
    ref = {"graph": g, "xyz": (xyz * sc[:, None]).ravel(), "r": d * sc}
    n = len(types)
    gen = whole._prepare_factorized_graph(n, types, g["num_neigh"], g["sources"], types[g["sources"]])
    whole._compute_prepared_factorized(gen, ref["xyz"], ref["r"])
    V = abs(np.linalg.det(cell))
    ew, fw, sw = whole.node_energies, whole._reduce_atom_forces(n, None, None, gen), whole._reduce_stress(V, None, gen)
    whole.close()
    e, f, st = _run(medium_model_path, s, ref, types, 2)
    print("medium slabs vs whole: energy %.3e force %.3e stress %.3e" % (
        np.max(np.abs(e - ew)), np.max(np.abs(f - fw)), np.max(np.abs(st - sw))))
    np.testing.assert_allclose(e, ew, rtol=0, atol=2e-5)
    np.testing.assert_allclose(f, fw, rtol=0, atol=2e-5)
    np.testing.assert_allclose(st, sw, rtol=0, atol=1e-8)


@pytest.mark.parametrize("model", ["tiny", "tiny_residual"])
def test_pair_style_modes_give_the_same_virial(request, model):
    """One rank, the same LAMMPS arrays: the virial the pair style's
    mpi_message_passing compute forms from the split phases (unit-volume
    stress, each off-diagonal pair averaged) equals the one
    no_domain_decomposition takes from smx_lammps_compute, and both match
    -V times the oracle's stress."""
    from oracle import oracle
    from symmetrix.mace_kokkos import MACEKokkosFloat
    from test_lammps_entry import _Hip, _lammps_arrays, _run as lammps_run
    path = request.getfixturevalue(model + "_model_path")
    s = _system("tiny")
    ref = oracle.evaluate_system(oracle.OracleModel(path), s, skin=0.5)
    ev = MACEKokkosFloat(path)
    lut = {int(z): i for i, z in enumerate(ev.atomic_numbers)}
    species = sorted(set(int(z) for z in s["numbers"]))
    lmp_type = {z: t + 1 for t, z in enumerate(species)}
    allpos, owner, alltypes, rows = _lammps_arrays(np.asarray(s["positions"], float), np.asarray(s["cell"], float),
                                                   s["numbers"], ev.r_cut + 0.5, lmp_type)
    n, nall = len(rows), len(allpos)
    model_type = np.array([lut[species[t - 1]] for t in alltypes], np.int32)
    ilist = np.random.default_rng(7).permutation(n).astype(np.int32)
    neigh = np.concatenate([rows[i] for i in ilist]).astype(np.int32)
    gen = ev._prepare_factorized_feature_graph(n, nall, ilist, model_type[ilist], model_type,
                                               np.array([len(rows[i]) for i in ilist], np.int32), neigh,
                                               model_type[neigh])
    ev._begin_factorized_distributed_positions_evaluation(gen, allpos)
    h = ev._distributed_h1()
    H1 = np.zeros((nall, h.shape[1]), np.float32)
    H1[ilist] = h
    H1[n:] = H1[owner[n:]]
    ev._continue_factorized_distributed_evaluation(H1)
    adj = ev._distributed_h1_adjoint().astype(np.float64)
    np.add.at(adj, owner[n:], adj[n:])
    ev._finish_factorized_distributed_evaluation(adj.astype(np.float32))
    w = ev._reduce_stress(1.0, None, gen).ravel()
    mpi_virial = -np.array([w[0], w[4], w[8], 0.5 * (w[1] + w[3]), 0.5 * (w[2] + w[6]), 0.5 * (w[5] + w[7])])
    hip = _Hip()
    try:
        ev2 = MACEKokkosFloat(path)
        type_to_model = [lut[z] for z in species]
        _, ndd_virial, _, _ = lammps_run(ev2, hip, allpos, owner, alltypes, rows, ilist, type_to_model, True)
    finally:
        hip.free()
    ndd_virial = np.asarray(ndd_virial, float)
    V = abs(np.linalg.det(np.asarray(s["cell"], float)))
    st = ref["stress"]
    oracle_virial = -V * np.array([st[0, 0], st[1, 1], st[2, 2], 0.5 * (st[0, 1] + st[1, 0]),
                                   0.5 * (st[0, 2] + st[2, 0]), 0.5 * (st[1, 2] + st[2, 1])])
    print("virial mpi", mpi_virial, "ndd", ndd_virial)
    scale = max(1.0, np.max(np.abs(oracle_virial)))
    np.testing.assert_allclose(mpi_virial, ndd_virial, rtol=0, atol=1e-6 * scale)
    np.testing.assert_allclose(mpi_virial, oracle_virial, rtol=0, atol=1e-6 * V)
