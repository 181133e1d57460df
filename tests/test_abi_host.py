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

    def __init__(self):
        self.prepared = 0
        self.computed = []
        self._gen = 0

    def _prepare_periodic_factorized_graph(self, types, positions, cell, inv, cutoff):
        self.prepared += 1
        self._gen += 1
        self.n = len(types)
        self.cutoff = cutoff
        return {"generation": self._gen, "num_edges": 10}

    def _compute_prepared_factorized_positions(self, gen, positions):
        assert gen == self._gen
        self.computed.append(positions.copy())

    @property
    def node_energies(self):
        return np.full(self.n, -1.5)

    def _reduce_atom_forces(self, n, rcv, src, gen):
        return np.zeros((n, 3))

    def _reduce_stress(self, volume, xyz, gen):
        return np.eye(3) * 0.01


def _calc(skin=0.5):
    c = Symmetrix.__new__(Symmetrix)
    Symmetrix.__bases__[0].__init__(c)
    c.evaluator = FakeEvaluator()
    c.cutoff = 5.0
    c.neighbor_skin = skin
    c._types = {8: 0, 22: 1, 38: 2}
    c._neighbor_cache = None
    c.neighbor_graph_rebuilds = 0
    c.results = {}
    return c


def test_calculator_reuses_graph_within_half_skin():
    c = _calc(skin=0.5)
    s = systems.srtio3_supercell(2, sigma=0.0)
    r = c.calculate(s, ["energy", "forces", "stress"])
    assert c.evaluator.prepared == 1
    assert c.evaluator.cutoff == pytest.approx(5.5)
    assert r["energy"] == pytest.approx(-1.5 * len(s["numbers"]))
    np.testing.assert_allclose(r["stress"], [0.01, 0.01, 0.01, 0, 0, 0])
    moved = dict(s)
    moved["positions"] = s["positions"] + 0.24 * np.array([1.0, 0.0, 0.0])
    c.calculate(moved)
    assert c.evaluator.prepared == 1  # 0.24 <= skin/2
    moved["positions"] = s["positions"] + np.array([[0.26, 0.0, 0.0]] + [[0.0, 0.0, 0.0]] * (len(s["numbers"]) - 1))
    c.calculate(moved)
    assert c.evaluator.prepared == 2  # one atom moved more than skin/2


def test_calculator_rebuilds_on_cell_or_numbers_change():
    c = _calc()
    s = systems.srtio3_supercell(2, sigma=0.0)
    c.calculate(s)
    strained = dict(s)
    strained["cell"] = s["cell"] * 1.001
    c.calculate(strained)
    assert c.evaluator.prepared == 2
    swapped = dict(strained)
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


def test_calculator_rejects_unknown_species_and_open_cells():
    c = _calc()
    s = systems.srtio3_supercell(2, sigma=0.0)
    bad = dict(s)
    bad["numbers"] = s["numbers"].copy()
    bad["numbers"][0] = 1
    with pytest.raises(ValueError):
        c.calculate(bad)
    open_ = dict(s)
    open_["pbc"] = np.array([True, True, False])
    with pytest.raises(NotImplementedError):
        c.calculate(open_)
