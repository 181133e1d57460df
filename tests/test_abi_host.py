"""CPU tests of the C ABI library and the host-side logic (no GPU needed):
every declared entry point is exported, model validation raises the
reference's error kinds before any device work, and the calculator's
neighbour-cache policy (calculator.py:2838-3093) with a fake evaluator, in the
style of the reference's test_symmetrix_calc.py:280-586.
"""

import ctypes
import json
import os
import re

import numpy as np
import pytest

from symmetrix import _native, random_model, systems
from symmetrix.calculator import Symmetrix, full_3x3_to_voigt_6_stress

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    names = []
    inc = os.path.join(ROOT, "include")
    for fn in sorted(os.listdir(inc)):
        if fn.endswith(".h"):
            with open(os.path.join(inc, fn)) as f:
                text = f.read()
            names += re.findall(r"SMX_API\s+[^;(]*?\b(smx_\w+)\s*\(", text)
    return names


def test_library_exports_every_declared_entry_point():
    names = _declared_symbols()
    assert len(names) >= 25
    lib = ctypes.CDLL(_native.LIB_PATH)
    for n in names:
        assert hasattr(lib, n), n
    # and the Python binding covers them all
    bound = {s[0] for s in _native.SIGNATURES}
    assert set(names) <= bound


def test_lammps_pair_style_uses_only_declared_entry_points():
    # the pair-style class (built inside LAMMPS, not here) calls only what the
    # header declares and fills only fields SmxLammpsArgsV2 has
    src = os.path.join(ROOT, "symmetrix-xl_amd", "lammps", "pair_symmetrix_mace_mi355x.cpp")
    with open(src) as f:
        text = f.read()
    declared = set(_declared_symbols())
    used = set(re.findall(r"\b(smx_\w+)\s*\(", text))
    assert used and used <= declared, used - declared
    fields = {name for name, _ in _native.SmxLammpsArgsV2._fields_}
    assigned = set(re.findall(r"\ba\.(\w+)\s*=", text))
    assert assigned <= fields, assigned - fields
    # every input field is set (reserved stays zero from the initialiser)
    assert fields - {"reserved"} <= assigned, fields - {"reserved"} - assigned


def test_lammps_pair_style_type_checks():
    """The pair-style class (its settings, coeff, both compute modes and the
    eight forward/reverse communication callbacks, with their Kokkos lambdas
    and views) compiles with -fsyntax-only against stand-ins of the LAMMPS
    and Kokkos declarations it uses (tests/lammps_stub) and the library's
    real header; the explicit instantiation for the device type makes every
    member and lambda body checked."""
    import shutil
    import subprocess
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not available")
    src = os.path.join(ROOT, "symmetrix-xl_amd", "lammps", "pair_symmetrix_mace_mi355x.cpp")
    cmd = [gxx, "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-Werror",
           "-I", os.path.join(ROOT, "tests", "lammps_stub"), "-I", os.path.join(ROOT, "include"), src]
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-4000:]


def test_abi_version_and_error_string():
    assert _native.lib.smx_abi_version() == 1
    assert isinstance(_native.lib.smx_last_error(), bytes)


def _create(path):
    h = ctypes.c_void_p()
    rc = _native.lib.smx_evaluator_create(path.encode(), b"", ctypes.byref(h))
    return rc, h


def test_missing_model_file_is_invalid_argument(tmp_path):
    rc, _ = _create(str(tmp_path / "nope.json"))
    assert rc == _native.SMX_ERR_INVALID_ARGUMENT
    assert b"cannot open model file" in _native.lib.smx_last_error()


def _edited_tiny(tmp_path, **changes):
    src = random_model.cached_model("tiny")
    with open(src) as f:
        j = json.load(f)
    j.update(changes)
    p = tmp_path / "edited.json"
    p.write_text(json.dumps(j))
    return str(p)


def test_unsupported_features_are_rejected(tmp_path):
    # ZBL without its parameters, other formats and bases, other model families
    for change in ({"has_zbl": True}, {"symmetrix_format_version": 3}, {"h1_affine_mode": "legacy"},
                   {"has_field_coupling": True}, {"first_interaction_residual": True},
                   {"single_layer_readout": True}, {"A0_scaled": True}):
        rc, _ = _create(_edited_tiny(tmp_path, **change))
        assert rc == _native.SMX_ERR_INVALID_ARGUMENT, change


def test_malformed_numbers_are_rejected(tmp_path):
    # strict JSON numbers: no non-finite spellings, no leading '+', no overflow
    text = open(random_model.cached_model("tiny")).read()
    key = '"r_max": '
    at = text.index(key) + len(key)
    end = at
    while text[end] not in ",}":
        end += 1
    for bad in ("NaN", "-Infinity", "+6.0", "1e999", "6.0.0"):
        p = tmp_path / "bad_number.json"
        p.write_text(text[:at] + bad + text[end:])
        rc, _ = _create(str(p))
        assert rc == _native.SMX_ERR_INVALID_ARGUMENT, bad
        assert b"model" in _native.lib.smx_last_error().lower() or b"number" in _native.lib.smx_last_error(), bad


def test_shape_without_kernel_set_is_unsupported(tmp_path):
    cfg = random_model.ModelConfig("small", 16, 1, 0, 2, [1, 8], radial_mlp=[8], r_cut=4.0,
                                   num_spline_points=32)
    p = random_model.write_model(cfg, str(tmp_path / "small.json"))
    rc, _ = _create(p)
    assert rc == _native.SMX_ERR_UNSUPPORTED


def test_reference_written_fixture_loads_or_is_unsupported():
    """The product's loader reads the models the reference's own writer makes
    (symmetrix/test/compact_r1_model.py): the medium-shape ones load their
    radial tables; the four-channel l_max 0 fixture has no kernel set."""
    from _compact import compact_model
    for name in ("compact_medium_m0", "compact_medium_linear"):
        path, _ = compact_model(name)
        cnt = ctypes.c_int64()
        dims = (ctypes.c_int32 * 4)()
        rc = _native.lib.smx_model_array_f32(path.encode(), b"R0_spline", None, 0, ctypes.byref(cnt), dims,
                                             None, None)
        assert rc == 0, _native.lib.smx_last_error()
        assert list(dims)[:3] == [15, 4, 4 * 128]
    path, _ = compact_model("compact_c4")
    rc, _ = _create(path)
    assert rc == _native.SMX_ERR_UNSUPPORTED


def test_inconsistent_model_arrays_are_invalid(tmp_path):
    src = random_model.cached_model("tiny")
    with open(src) as f:
        j = json.load(f)
    j["H0_weights"] = j["H0_weights"][:-1]
    p = tmp_path / "bad.json"
    p.write_text(json.dumps(j))
    rc, _ = _create(str(p))
    assert rc == _native.SMX_ERR_INVALID_ARGUMENT


def test_voigt_order():
    s = np.arange(9.0).reshape(3, 3)
    np.testing.assert_allclose(full_3x3_to_voigt_6_stress(s), [0, 4, 8, 6, 4, 2])


# ---------------------------------------------------------------------------
# Calculator logic with a fake evaluator
# ---------------------------------------------------------------------------
class FakeEvaluator:
    r_cut = 5.0
    atomic_numbers = [8, 22, 38]

    def __init__(self, tiled=False):
        self.prepared = 0
        self.device_prepared = 0
        self.geometry = []
        self.cell_updates = 0
        self.computed = []
        self._gen = 0
        self.tiled = tiled

    def _prepare_periodic_factorized_graph(self, types, positions, cell, inv, cutoff):
        self.prepared += 1
        self.device_prepared += 1
        self._gen += 1
        self.n = len(types)
        self.cutoff = cutoff
        return {"generation": self._gen, "num_edges": 10}

    def _prepare_factorized_graph(self, n, types, num_neigh, sources, neigh_types):
        assert int(np.sum(num_neigh)) == len(sources) and len(types) == n
        self.prepared += 1
        self._gen += 1
        self.n = n
        self.edges = len(sources)
        return self._gen

    def _prepare_factorized_geometry(self, gen, ref_positions, ref_xyz, cell, inv, pbc):
        assert gen == self._gen and np.asarray(ref_xyz).size == 3 * self.edges
        self.geometry.append("cartesian")

    def _prepare_factorized_fractional_geometry(self, gen, frac, frac_xyz, cell, inv, pbc):
        assert gen == self._gen and np.asarray(frac_xyz).size == 3 * self.edges
        self.geometry.append("fractional")

    def _prepare_factorized_shift_geometry(self, gen, ref_positions, shifts, cell, inv, pbc):
        assert gen == self._gen and np.asarray(shifts).size == 3 * self.edges
        self.geometry.append("shifts")

    def _update_factorized_cell(self, gen, cell, inv):
        assert gen == self._gen
        self.cell_updates += 1

    @property
    def execution_plan_report(self):
        return {"selected_id": "mh0-dual-layer-tiled-v1" if self.tiled else "mh0-direct-capacity-retained"}

    def _compute_prepared_factorized_positions(self, gen, positions):
        assert gen == self._gen
        self.computed.append(positions.copy())

    def _compute_prepared_factorized_positions_results(self, gen, positions, volume=None):
        self._compute_prepared_factorized_positions(gen, positions)
        return self.node_energies, self._reduce_atom_forces(self.n, None, None, gen), (
            None if volume is None else self._reduce_stress(volume, None, gen))

    @property
    def node_energies(self):
        return np.full(self.n, -1.5)

    def _reduce_atom_forces(self, n, rcv, src, gen):
        return np.zeros((n, 3))

    def _reduce_stress(self, volume, xyz, gen):
        return np.eye(3) * 0.01


def _calc(skin=0.5, tiled=False):
    c = Symmetrix.__new__(Symmetrix)
    Symmetrix.__bases__[0].__init__(c)
    c.evaluator = FakeEvaluator(tiled)
    c.cutoff = 5.0
    c.neighbor_skin = skin
    c._types = {8: 0, 22: 1, 38: 2}
    c._neighbor_cache = None
    c.neighbor_cache_build_count = 0
    c.neighbor_cache_reuse_count = 0
    c.neighbor_cache_cell_update_count = 0
    c.neighbor_graph_backend = None
    c.results = {}
    return c


def test_calculator_reuses_graph_within_half_skin():
    c = _calc(skin=0.5)
    s = systems.srtio3_supercell(2, sigma=0.0)
    r = c.calculate(s, ["energy", "forces", "stress"])
    assert c.evaluator.prepared == 1 and c.neighbor_graph_backend == "host"   # 40 atoms < 512
    assert c.evaluator.geometry == ["fractional"]
    assert r["energy"] == pytest.approx(-1.5 * len(s["numbers"]))
    np.testing.assert_allclose(r["stress"], [0.01, 0.01, 0.01, 0, 0, 0])
    moved = dict(s)
    moved["positions"] = s["positions"] + 0.24 * np.array([1.0, 0.0, 0.0])
    c.calculate(moved)
    assert c.evaluator.prepared == 1  # 0.24 <= skin/2
    moved["positions"] = s["positions"] + np.array([[0.26, 0.0, 0.0]] + [[0.0, 0.0, 0.0]] * (len(s["numbers"]) - 1))
    c.calculate(moved)
    assert c.evaluator.prepared == 2  # one atom moved more than skin/2


def test_calculator_keeps_topology_under_affine_strain(monkeypatch):
    """calculator.py:2858-2887: a strained cell with the atoms carried along
    updates the evaluator's cell; a large strain or new numbers rebuild."""
    for backend, device in (("host", 0), ("kokkos", 1)):
        monkeypatch.setenv("SYMMETRIX_NEIGHBOR_BACKEND", backend)
        c = _calc()
        s = systems.srtio3_supercell(2, sigma=0.0)
        c.calculate(s)
        assert c.evaluator.device_prepared == device
        strained = dict(s)
        strained["cell"] = s["cell"] * 1.001
        strained["positions"] = s["positions"] * 1.001
        c.calculate(strained)
        assert c.evaluator.prepared == 1 and c.evaluator.cell_updates == 1
        far = dict(s)
        far["cell"] = s["cell"] * 0.85
        far["positions"] = s["positions"] * 0.85
        c.calculate(far)
        assert c.evaluator.prepared == 2   # compression: cutoff / 0.85 exceeds cutoff + skin
        swapped = dict(far)
        swapped["numbers"] = s["numbers"][::-1].copy()
        c.calculate(swapped)
        assert c.evaluator.prepared == 3


def test_calculator_wrapped_positions_do_not_force_rebuild():
    c = _calc()
    s = systems.srtio3_supercell(2, sigma=0.0)
    c.calculate(s)
    wrapped = dict(s)
    wrapped["positions"] = s["positions"] + s["cell"][0]  # one full lattice vector
    c.calculate(wrapped)
    assert c.evaluator.prepared == 1


def test_calculator_geometry_forms_by_boundary_and_plan(monkeypatch):
    """Host graphs take the Cartesian form for open or mixed boundaries, the
    fractional form for periodic cells and the shift form under the tiled
    plan (calculator.py:3224-3300); large periodic systems use the device
    builder (calculator.py:83-84, 165-173)."""
    monkeypatch.delenv("SYMMETRIX_NEIGHBOR_BACKEND", raising=False)
    s = systems.srtio3_supercell(2, sigma=0.0)
    slab = dict(s, pbc=np.array([True, True, False]))
    c = _calc()
    c.calculate(slab, ["energy", "forces"])
    assert c.evaluator.geometry == ["cartesian"]
    molecule = dict(s, pbc=np.array([False, False, False]))
    c = _calc()
    c.calculate(molecule, ["energy", "forces"])
    assert c.evaluator.geometry == ["cartesian"]
    with pytest.raises(ValueError, match="volume"):
        c.calculate(dict(molecule, cell=np.zeros((3, 3))), ["stress"])
    c = _calc(tiled=True)
    c.calculate(s)
    assert c.evaluator.geometry == ["shifts"]
    big = systems.srtio3_supercell(5, sigma=0.0)   # 625 atoms
    c = _calc()
    c.calculate(big)
    assert c.evaluator.device_prepared == 1 and c.neighbor_graph_backend == "device"
    monkeypatch.setenv("SYMMETRIX_NEIGHBOR_BACKEND", "host")
    c = _calc()
    c.calculate(big)
    assert c.evaluator.device_prepared == 0 and c.evaluator.geometry == ["fractional"]


def test_calculator_rejects_unknown_species():
    c = _calc()
    s = systems.srtio3_supercell(2, sigma=0.0)
    bad = dict(s)
    bad["numbers"] = s["numbers"].copy()
    bad["numbers"][0] = 1
    with pytest.raises(ValueError):
        c.calculate(bad)


def _brute_force_ijS(positions, cell, pbc, cutoff, reach=3):
    out = set()
    rng = [range(-reach, reach + 1) if p else range(0, 1) for p in pbc]
    for i in range(len(positions)):
        for j in range(len(positions)):
            for a in rng[0]:
                for b in rng[1]:
                    for c in rng[2]:
                        if i == j and a == b == c == 0:
                            continue
                        d = positions[j] - positions[i] + np.array([a, b, c]) @ cell
                        if np.linalg.norm(d) < cutoff:
                            out.add((i, j, a, b, c))
    return out


@pytest.mark.parametrize("pbc", [(True, True, True), (True, False, True), (False, False, False)])
def test_host_neighbor_list_matches_brute_force(pbc):
    """The host "ijS" list (the reference's matscipy/ASE list) on a
    triclinic cell with atoms outside it: every pair closer than the cutoff,
    receiver-major."""
    from symmetrix.neighbors import neighbor_list_ijS
    rng = np.random.default_rng(5)
    cell = np.array([[6.0, 0.0, 0.0], [1.5, 5.5, 0.0], [-1.0, 0.5, 6.5]])
    pos = rng.uniform(-0.3, 1.3, size=(30, 3)) @ cell
    i, j, S = neighbor_list_ijS(pos, cell, pbc, 4.2)
    assert np.all(np.diff(i) >= 0)
    got = {(int(a), int(b), *map(int, s)) for a, b, s in zip(i, j, S)}
    assert len(got) == len(i)
    assert got == _brute_force_ijS(pos, cell, pbc, 4.2)


def test_reference_caller_members_resolve():
    """Every evaluator member the reference calculator reaches by getattr on
    its prepared-execution route (calculator.py:1165-1190, 2838-3093,
    3224-3300, 3418-3440) exists on MACEKokkosFloat."""
    from symmetrix.mace_kokkos import MACEKokkosFloat
    names = ["_set_allow_fixed_workspace", "_set_execution_plan_request", "_resolve_execution_plan",
             "execution_plan_report", "streamed_edges_mode", "atomic_numbers",
             "_prepare_periodic_factorized_graph", "_prepare_factorized_graph", "_compute_prepared_factorized",
             "_prepare_factorized_geometry", "_prepare_factorized_fractional_geometry",
             "_prepare_factorized_shift_geometry", "_update_factorized_cell",
             "_compute_prepared_factorized_positions", "_reduce_atom_forces", "_reduce_stress", "node_energies",
             "node_forces", "compute_node_energies_forces", "prepare_active_types",
             "factorized_last_evaluation_ms", "factorized_last_graph_prepare_ms", "allow_fixed_workspace"]
    missing = [n for n in names if not hasattr(MACEKokkosFloat, n)]
    assert not missing, missing


class FakeMH1:
    """Stands in for MACENonlinearKokkosFloat: records the graph it gets and
    returns node energy 1 per node and node_forces[e] = xyz[e] * r[e]."""

    has_field_coupling = False

    def __init__(self):
        self.calls = []

    def compute_node_energies_forces(self, n, types, num_neigh, src, neigh_types, xyz, r):
        self.calls.append((n, np.array(num_neigh), np.array(src), np.array(xyz).reshape(-1, 3), np.array(r)))
        self._n = n
        self._nf = (np.array(xyz).reshape(-1, 3) * np.array(r)[:, None]).reshape(-1)

    @property
    def node_energies(self):
        return np.ones(self._n)

    @property
    def node_forces(self):
        return self._nf


def test_calculator_mh1_passes_edges_inside_cutoff_and_reduces():
    """The MH-1 route (calculator.py:3087-3093): the skin graph's edges with
    r < r_cut, in receiver order; F_i = sum over edges with source i of f_e
    minus those with receiver i; sigma = -sum f_e xyz_e^T / V."""
    c = _calc(skin=0.5)
    c._nonlinear = True
    c.evaluator = FakeMH1()
    s = systems.srtio3_supercell(2, sigma=0.1, seed=4)
    res = c.calculate(s, ["energy", "forces", "stress"])
    n, num_neigh, src, xyz, r = c.evaluator.calls[-1]
    pos, cell = np.asarray(s["positions"]), np.asarray(s["cell"])
    # brute force over images
    want = []
    for i in range(n):
        for j in range(n):
            for S in np.ndindex(5, 5, 5):
                d = pos[j] - pos[i] + (np.array(S) - 2) @ cell
                rr = np.linalg.norm(d)
                if 0 < rr < c.cutoff:
                    want.append((i, j, rr))
    assert len(r) == len(want) and num_neigh.sum() == len(r)
    assert np.all(r < c.cutoff)
    recv = np.repeat(np.arange(n), num_neigh)
    np.testing.assert_allclose(np.linalg.norm(xyz, axis=1), r)
    np.testing.assert_allclose(sorted(r), sorted(w[2] for w in want), rtol=1e-12)
    f = xyz * r[:, None]
    F = np.zeros((n, 3))
    np.add.at(F, src, f)
    np.add.at(F, recv, -f)
    np.testing.assert_allclose(res["forces"], F, atol=1e-12)
    sig = -np.einsum("ea,eb->ab", f, xyz) / abs(np.linalg.det(cell))
    np.testing.assert_allclose(res["stress"], [sig[0, 0], sig[1, 1], sig[2, 2], sig[1, 2], sig[0, 2], sig[0, 1]],
                               atol=1e-12)
    assert res["energy"] == n
    # a second call inside half the skin reuses the graph
    moved = dict(s)
    moved["positions"] = pos + 0.1
    c.calculate(moved)
    assert c.neighbor_cache_build_count == 1 and c.neighbor_cache_reuse_count == 1
