"""The LAMMPS pair-style entry (smx_lammps_compute) against the oracle.

The inputs are built the way LAMMPS holds them for pair_style
symmetrix/mace/kk without domain decomposition
(pair_symmetrix_mace_kokkos.cpp:1010-1282): local atoms plus ghost images
of the periodic cell, 1-based atom types with a type map, a full neighbour
list in a column-major (Kokkos LayoutLeft) array with special-bond bits set
on some entries, an ilist that is not the identity, and atom->map(tag) as
`owner`.  Forces land on local and ghost rows; folded onto their owners they
must equal the oracle's periodic forces, the energy and per-atom energies
the oracle's, and -virial/V the oracle's stress.  A second call without a
neighbour-list rebuild uses moved positions on the same list.  The same
calls run under the direct plan and the tiled (capacity) plan, whose forces
reach the LAMMPS rows tile by tile; both must give the same rows.
"""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5   # eV/atom
F_TOL = 1e-4   # eV/A
S_TOL = 1e-6   # eV/A^3


class _Hip:
    def __init__(self):
        h = ctypes.CDLL("libamdhip64.so")
        h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        h.hipFree.argtypes = [ctypes.c_void_p]
        self.h = h
        self.held = []

    def put(self, a):
        a = np.ascontiguousarray(a)
        p = ctypes.c_void_p()
        assert self.h.hipMalloc(ctypes.byref(p), max(a.nbytes, 8)) == 0
        if a.nbytes:
            assert self.h.hipMemcpy(p, a.ctypes.data_as(ctypes.c_void_p), a.nbytes, 1) == 0
        self.held.append(p)
        return p.value

    def get(self, ptr, like):
        out = np.empty_like(like)
        assert self.h.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(ptr), out.nbytes, 2) == 0
        return out

    def free(self):
        for p in self.held:
            self.h.hipFree(p)
        self.held = []


def _lammps_arrays(positions, cell, numbers, cutoff, lmp_type_of_z):
    """Local atoms, 26 ghost images, full neighbour list within cutoff."""
    n = len(positions)
    shifts = [np.array([a, b, c]) for a in (-1, 0, 1) for b in (-1, 0, 1) for c in (-1, 0, 1)
              if (a, b, c) != (0, 0, 0)]
    allpos = np.concatenate([positions] + [positions + s @ cell for s in shifts])
    owner = np.tile(np.arange(n, dtype=np.int32), 1 + len(shifts))
    types = np.array([lmp_type_of_z[int(z)] for z in numbers], np.int32)
    alltypes = np.tile(types, 1 + len(shifts))
    rows = []
    for i in range(n):
        d = np.linalg.norm(allpos - positions[i], axis=1)
        js = np.nonzero(d < cutoff)[0]
        rows.append(js[js != i].astype(np.int32))
    return allpos, owner, alltypes, rows


def _args(hip, allpos, owner, alltypes, rows, ilist, type_to_model, rebuild, f0=None, eatom0=None, stream=None):
    """LAMMPS-shaped arguments on the device (SmxLammpsArgsV2 when a stream
    is given), with f and eatom starting from f0 / eatom0 (zero)."""
    from symmetrix._native import SmxLammpsArgsV1, SmxLammpsArgsV2
    n, nall = len(rows), len(allpos)
    maxn = max(len(r) for r in rows)
    # column-major [maxn][n] with special-bond bits on every 7th entry
    nb = np.zeros((maxn, n), np.int32)
    for i, r in enumerate(rows):
        marked = r.copy()
        marked[::7] |= (1 << 30)
        nb[:len(r), i] = marked
    numneigh = np.array([len(r) for r in rows], np.int32)
    f = np.zeros((nall, 3)) if f0 is None else np.array(f0, dtype=np.float64)
    eatom = np.zeros(nall) if eatom0 is None else np.array(eatom0, dtype=np.float64)
    a = SmxLammpsArgsV1() if stream is None else SmxLammpsArgsV2()
    a.inum, a.nall, a.ntypes = n, nall, len(type_to_model)
    a.ilist = hip.put(ilist)
    a.numneigh = hip.put(numneigh)
    a.neighbors = hip.put(nb)
    a.stride_atom, a.stride_neighbor = 1, n
    a.x = hip.put(allpos)
    a.type = hip.put(alltypes)
    a.type_to_model = hip.put(np.asarray(type_to_model, np.int32))
    a.owner = hip.put(owner)
    a.rebuild = 1 if rebuild else 0
    a.f = hip.put(f)
    a.eatom = hip.put(eatom)
    if stream is not None:
        a.stream = stream
    return a, f, eatom


def _run(ev, hip, allpos, owner, alltypes, rows, ilist, type_to_model, rebuild):
    a, f, eatom = _args(hip, allpos, owner, alltypes, rows, ilist, type_to_model, rebuild)
    energy, virial = ev._lammps_compute(a)
    return energy, virial, hip.get(a.f, f), hip.get(a.eatom, eatom)


_ROWS = {}  # (model, plan, step) -> LAMMPS force rows, for the cross-plan check


@pytest.mark.parametrize("model", ["tiny", "tiny_scaled", "tiny_zbl", "tiny_agnesi", "tiny_residual",
                                   "tiny_single_residual"])
@pytest.mark.parametrize("tile", [None, 32], ids=["direct", "tiled32"])
def test_lammps_entry_matches_oracle(request, model, tile):
    # plain, density-scaled, ZBL, Agnesi (per-pair tables), residual-first and
    # one-interaction models
    tiny_model_path = request.getfixturevalue(model + "_model_path")
    from oracle import oracle
    from symmetrix import systems
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = systems.srtio3_supercell(3, sigma=0.05, seed=0)
    om = oracle.OracleModel(tiny_model_path)
    ref = oracle.evaluate_system(om, s, skin=0.5)
    ev = MACEKokkosFloat(tiny_model_path)
    if tile is not None:
        ev.set_execution_plan_request("capacity", tile)
    # LAMMPS types: O=1, Ti=2, Sr=3 ; model types follow the model's atomic numbers
    lmp_type_of_z = {8: 1, 22: 2, 38: 3}
    model_of_z = {int(z): k for k, z in enumerate(ev.atomic_numbers)}
    type_to_model = [model_of_z[8], model_of_z[22], model_of_z[38]]
    cell = np.asarray(s["cell"], float)
    V = abs(np.linalg.det(cell))
    n = len(s["numbers"])
    allpos, owner, alltypes, rows = _lammps_arrays(s["positions"], cell, s["numbers"], ev.r_cut + 0.5,
                                                   lmp_type_of_z)
    assert sum(len(r) for r in rows) == len(ref["graph"]["sources"])
    ilist = np.arange(n, dtype=np.int32)[::-1].copy()
    hip = _Hip()
    try:
        for step, pos in enumerate([s["positions"],
                                    s["positions"] + 0.03 * np.random.default_rng(1).normal(size=(n, 3))]):
            if step:
                ref = oracle.evaluate_system(om, s, skin=0.5, positions=pos, graph=ref["graph"])
                shifts = allpos - s["positions"][owner]
                allpos_step = pos[owner] + shifts
            else:
                allpos_step = allpos
            energy, virial, f, eatom = _run(ev, hip, allpos_step, owner, alltypes, rows, ilist, type_to_model,
                                            rebuild=(step == 0))
            folded = np.zeros((n, 3))
            np.add.at(folded, owner, f)
            print("step %d energy/atom err %.3e force err %.3e" % (
                step, abs(energy - ref["energy"]) / n, np.max(np.abs(folded - ref["forces"]))))
            assert abs(energy - ref["energy"]) / n < E_TOL
            np.testing.assert_allclose(eatom[:n], ref["energies"], rtol=0, atol=1e-4)
            assert np.all(eatom[n:] == 0.0)
            assert np.max(np.abs(folded - ref["forces"])) < F_TOL
            st = ref["stress"]
            mine = -np.array(virial) / V
            expect = [st[0, 0], st[1, 1], st[2, 2], 0.5 * (st[0, 1] + st[1, 0]), 0.5 * (st[0, 2] + st[2, 0]),
                      0.5 * (st[1, 2] + st[2, 1])]
            np.testing.assert_allclose(mine, expect, rtol=0, atol=S_TOL)
            _ROWS[(model, tile, step)] = f
            if tile is not None:
                assert ev.execution_plan.startswith("direct-tiled")
                if (model, None, step) in _ROWS:
                    # ghost rows included; the plans differ only in FP32
                    # summation order (3e-8 measured), a misplaced row by ~0.1
                    np.testing.assert_allclose(f, _ROWS[(model, None, step)], rtol=0, atol=1e-6)
    finally:
        hip.free()


def test_lammps_entry_in_an_electric_field(tiny_field_model_path):
    # pair_style symmetrix/mace/kk electric_field Ex Ey Ez
    # (pair_symmetrix_mace_kokkos.cpp:207-224, 598-599): the field set once
    # applies to every compute; without it a MACEField model is refused
    from oracle import oracle
    from symmetrix import systems
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = systems.srtio3_supercell(3, sigma=0.05, seed=0)
    field = np.array([0.1, -0.05, 0.2])
    om = oracle.OracleModel(tiny_field_model_path)
    ref = oracle.evaluate_system(om, s, skin=0.5, field=field)
    ev = MACEKokkosFloat(tiny_field_model_path)
    model_of_z = {int(z): k for k, z in enumerate(ev.atomic_numbers)}
    type_to_model = [model_of_z[8], model_of_z[22], model_of_z[38]]
    cell = np.asarray(s["cell"], float)
    n = len(s["numbers"])
    allpos, owner, alltypes, rows = _lammps_arrays(s["positions"], cell, s["numbers"], ev.r_cut + 0.5,
                                                   {8: 1, 22: 2, 38: 3})
    ilist = np.arange(n, dtype=np.int32)
    hip = _Hip()
    try:
        with pytest.raises(ValueError, match="electric field"):
            _run(ev, hip, allpos, owner, alltypes, rows, ilist, type_to_model, True)
        ev._set_electric_field(field)
        energy, virial, f, eatom = _run(ev, hip, allpos, owner, alltypes, rows, ilist, type_to_model, True)
        folded = np.zeros((n, 3))
        np.add.at(folded, owner, f)
        assert abs(energy - ref["energy"]) / n < E_TOL
        assert np.max(np.abs(folded - ref["forces"])) < F_TOL
        np.testing.assert_allclose(eatom[:n], ref["energies"], rtol=0, atol=1e-4)
    finally:
        hip.free()


def test_lammps_entry_rejects_unmapped_types(tiny_model_path):
    from symmetrix import systems
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = systems.srtio3_supercell(3, sigma=0.05, seed=0)
    ev = MACEKokkosFloat(tiny_model_path)
    cell = np.asarray(s["cell"], float)
    allpos, owner, alltypes, rows = _lammps_arrays(s["positions"], cell, s["numbers"], ev.r_cut + 0.5,
                                                   {8: 1, 22: 2, 38: 3})
    hip = _Hip()
    try:
        with pytest.raises(ValueError, match="type"):
            _run(ev, hip, allpos, owner, alltypes, rows, np.arange(len(rows), dtype=np.int32), [0, -1, 2], True)
    finally:
        hip.free()


@pytest.mark.parametrize("model", ["tiny", "tiny_single"])
@pytest.mark.parametrize("tile", [None, 32], ids=["direct", "tiled32"])
def test_lammps_entry_zero_length_edge_raises_and_next_call_recovers(request, model, tile):
    # a ghost placed on the local atom that lists it (the last receiver, in
    # the last tile): exactly one zero-length edge, counted once in either
    # plan; the next call on good positions (same list, no rebuild) gives
    # the first call's results again
    from symmetrix import systems
    from symmetrix.mace_kokkos import MACEKokkosFloat
    s = systems.srtio3_supercell(3, sigma=0.05, seed=0)
    ev = MACEKokkosFloat(request.getfixturevalue(model + "_model_path"))
    if tile is not None:
        ev.set_execution_plan_request("capacity", tile)
    model_of_z = {int(z): k for k, z in enumerate(ev.atomic_numbers)}
    type_to_model = [model_of_z[8], model_of_z[22], model_of_z[38]]
    cell = np.asarray(s["cell"], float)
    allpos, owner, alltypes, rows = _lammps_arrays(s["positions"], cell, s["numbers"], ev.r_cut + 0.5,
                                                   {8: 1, 22: 2, 38: 3})
    n = len(rows)
    ghost = int(next(j for j in rows[n - 1] if j >= n))
    bad = allpos.copy()
    bad[ghost] = allpos[n - 1]
    ilist = np.arange(n, dtype=np.int32)
    hip = _Hip()
    try:
        e0, v0, f0, _ = _run(ev, hip, allpos, owner, alltypes, rows, ilist, type_to_model, True)
        # the failed call leaves the caller's force and energy rows as they were
        rng = np.random.default_rng(1)
        fill_f, fill_e = rng.normal(size=(len(bad), 3)), rng.normal(size=len(bad))
        a, _, _ = _args(hip, bad, owner, alltypes, rows, ilist, type_to_model, False, fill_f, fill_e)
        with pytest.raises(ValueError, match=r"invalid edge geometry \(1 zero-length"):
            ev._lammps_compute(a)
        np.testing.assert_array_equal(hip.get(a.f, fill_f), fill_f)
        np.testing.assert_array_equal(hip.get(a.eatom, fill_e), fill_e)
        e1, v1, f1, _ = _run(ev, hip, allpos, owner, alltypes, rows, ilist, type_to_model, False)
        assert e1 == e0
        np.testing.assert_array_equal(f1, f0)
        np.testing.assert_array_equal(v1, v0)
    finally:
        hip.free()


@pytest.mark.parametrize("version", ["v1", "v2"])
def test_lammps_entry_orders_after_caller_stream(tiny_model_path, version):
    """The caller updates x and clears f with asynchronous copies on its own
    stream (behind a long fill, as Kokkos queues fix nve and force_clear)
    right before the call; V2 passes that stream, V1 relies on the device
    synchronisation on entry.  The results are those of the new positions
    (the oracle's) with f cleared first."""
    from oracle import oracle
    from symmetrix import systems
    from symmetrix.mace_kokkos import MACEKokkosFloat
    h = ctypes.CDLL("libamdhip64.so")
    h.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    h.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    h.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
    h.hipMemsetAsync.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p]
    h.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    s = systems.srtio3_supercell(3, sigma=0.05, seed=0)
    ev = MACEKokkosFloat(tiny_model_path)
    om = oracle.OracleModel(tiny_model_path)
    model_of_z = {int(z): k for k, z in enumerate(ev.atomic_numbers)}
    type_to_model = [model_of_z[8], model_of_z[22], model_of_z[38]]
    cell = np.asarray(s["cell"], float)
    allpos, owner, alltypes, rows = _lammps_arrays(s["positions"], cell, s["numbers"], ev.r_cut + 0.5,
                                                   {8: 1, 22: 2, 38: 3})
    n = len(rows)
    moved = s["positions"] + np.random.default_rng(7).normal(scale=0.02, size=s["positions"].shape)
    shifts = allpos[n:] - np.tile(s["positions"], (26, 1))
    moved_all = np.concatenate([moved, np.tile(moved, (26, 1)) + shifts])
    ref = oracle.evaluate_system(om, s, positions=moved)
    ilist = np.arange(n, dtype=np.int32)
    hip = _Hip()
    stream = ctypes.c_void_p()
    assert h.hipStreamCreate(ctypes.byref(stream)) == 0
    try:
        # first call builds the list on the old positions
        _run(ev, hip, allpos, owner, alltypes, rows, ilist, type_to_model, True)
        a, _, _ = _args(hip, allpos, owner, alltypes, rows, ilist, type_to_model, False,
                        f0=np.full((len(allpos), 3), 1e3), stream=stream.value if version == "v2" else None)
        staged = hip.put(moved_all)
        big = hip.put(np.zeros(1 << 27, np.uint8))   # 128 MiB fill ahead of the updates
        assert h.hipMemsetAsync(big, 0, 1 << 27, stream) == 0
        assert h.hipMemcpyAsync(a.x, staged, moved_all.nbytes, 3, stream) == 0
        assert h.hipMemsetAsync(a.f, 0, len(allpos) * 24, stream) == 0
        energy, virial = ev._lammps_compute(a)
        assert h.hipStreamSynchronize(stream) == 0
        f = hip.get(a.f, np.zeros((len(allpos), 3)))
        folded = np.zeros((n, 3))
        np.add.at(folded, owner, f)
        assert abs(energy - ref["energy"]) / n < E_TOL
        assert np.max(np.abs(folded - ref["forces"])) < F_TOL
    finally:
        h.hipStreamDestroy(stream)
        hip.free()


def test_lammps_entry_rejects_bad_arguments(tiny_model_path):
    # host-side checks, before any device work: struct size, counts, arrays
    import ctypes
    from symmetrix import _native
    from symmetrix._native import SmxLammpsArgsV1
    from symmetrix.mace_kokkos import MACEKokkosFloat
    ev = MACEKokkosFloat(tiny_model_path)
    energy, virial = ctypes.c_double(), (ctypes.c_double * 6)()

    def call(**fields):
        a = SmxLammpsArgsV1()
        a.struct_size = ctypes.sizeof(SmxLammpsArgsV1)
        a.inum, a.nall, a.ntypes = 0, 0, 1
        a.type_to_model = 8          # any non-null: never read for these cases
        for k, v in fields.items():
            setattr(a, k, v)
        rc = _native.lib.smx_lammps_compute(ev._h, ctypes.byref(a), ctypes.byref(energy), virial)
        return rc, _native.lib.smx_last_error()

    for fields, text in [({"struct_size": 8}, b"struct_size"),
                         ({"inum": 2, "nall": 1}, b"counts"),
                         ({"ntypes": 0}, b"counts"),
                         ({"inum": 1, "nall": 1}, b"neighbour list arrays"),
                         ({"nall": 3}, b"per-atom arrays"),
                         ({"type_to_model": None}, b"type map")]:
        rc, msg = call(**fields)
        assert rc == _native.SMX_ERR_INVALID_ARGUMENT, (fields, msg)
        assert text in msg, (fields, msg)
