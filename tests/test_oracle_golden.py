"""Pins the CPU oracle (and the model generator it reads) against the
reference's own fixtures and against what the mathematics fixes.

Each test names the reference file:line or the closed form it checks.  The
oracle is the checker of the HIP path; nothing here needs a GPU.
"""

import json
import math
import os

import numpy as np
import pytest
from scipy.interpolate import CubicSpline
from scipy.special import sph_harm_y

from oracle import oracle
from symmetrix import e3, random_model, systems

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---------------------------------------------------------------------------
# R1 coupling and product-basis structure (reference fixtures)
# ---------------------------------------------------------------------------
def _r1_fixtures():
    with open(os.path.join(GOLDEN, "r1_coupling.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("name", sorted(_r1_fixtures()))
def test_r1_coupling_matches_reference_contract(name):
    """symmetrix/test/data/execution_contracts/jit_r1_*_contract.json:
    paths and every sparse term (lm1, lm2, lme, row, coefficient)."""
    fx = _r1_fixtures()[name]
    lmax, Lmax = fx["edge_l_max"], fx["source_l_max"]
    paths = e3.r1_paths(lmax, Lmax)
    assert [list(p) for p in paths] == fx["paths"]
    cpl = e3.r1_coupling(lmax, Lmax)
    mine = sorted(zip(cpl["_lm1"], cpl["_lm2"], cpl["Phi1_lme"], cpl["Phi1_lelm1lm2"], cpl["Phi1_clebsch_gordan"]))
    ref = sorted(tuple(t) for t in fx["terms"])
    assert len(mine) == len(ref)
    for a, b in zip(mine, ref):
        assert a[:4] == tuple(b[:4])
        # the fixture holds FP32-rounded coefficients (e3nn float32 export)
        assert a[4] == pytest.approx(b[4], abs=2e-7)


def test_m0_monomials_match_reference_contract():
    """standard_m0_contract.json monomial groups (94/118/92/118 terms, in the
    reference's (degree, lex) order) equal the generator's monomial lists."""
    with open(os.path.join(GOLDEN, "m0_monomials.json")) as f:
        fx = json.load(f)
    lin, lout, corr = fx["input_l_max"], fx["output_l_max"], fx["correlation"]
    keys = []
    for L in range(lout + 1):
        keys += e3.structural_support(lin, L, corr)
    assert len(keys) == len(fx["groups"])
    for g, mine in zip(fx["groups"], keys):
        assert [list(m) for m in mine] == g["terms"], g["output_component"]
        degs = [sum(1 for t in mine if len(t) == d) for d in (1, 2, 3)]
        assert degs == g["degree_counts"]


def test_m0_equivariant_support_within_reference_terms():
    """The equivariant polynomials (null space of the rotation constraint)
    live on the reference's terms; the terms outside them have an exactly
    vanishing symmetrised coefficient in every coupling path."""
    import itertools
    for L in (0, 1):
        keys = e3.structural_support(3, L, 3)
        eq = e3.product_basis_support(3, L, 3)
        tensors = e3.coupling_chain_tensors(3, L, 3)
        for M in range(2 * L + 1):
            k, s = set(map(tuple, keys[M])), set(map(tuple, eq[M]))
            assert s <= k
            for extra in k - s:
                if len(extra) != 3:
                    continue
                for T in tensors:
                    sym = sum(T[M][p] for p in set(itertools.permutations(extra)))
                    assert abs(sym) < 1e-12


# ---------------------------------------------------------------------------
# Polynomial semantics (multivariate_polynomial.cpp:11-131)
# ---------------------------------------------------------------------------
def _poly(nvar, coef, monos, x):
    lib = oracle.lib()
    offs = np.zeros(len(monos) + 1, np.int32)
    for i, m in enumerate(monos):
        offs[i + 1] = offs[i] + len(m)
    vars_ = np.array([v for m in monos for v in m] or [0], np.int32)
    g = np.zeros(nvar)
    f = lib.oracle_polynomial(nvar, len(monos), np.asarray(coef, float), offs, vars_, np.asarray(x, float), g)
    return f, g


def test_polynomial_repeated_monomial_keeps_first_coefficient():
    """Known answer of test_multivariate_polynomial.py:65-68."""
    f, _ = _poly(2, [2.0, 9.0, 3.0], [[0], [0], [0, 1]], [4.0, 5.0])
    assert f == pytest.approx(68.0)


def test_polynomial_gradient_matches_finite_differences():
    """test_multivariate_polynomial.py:18-28 (gradient vs simple evaluation),
    here against central differences."""
    rng = np.random.default_rng(0)
    monos = [[7], [0, 1], [1, 3], [1, 1, 2], [0, 2, 4], [4, 5, 6]]
    coef = rng.random(len(monos))
    x = rng.random(8)
    f0, g = _poly(8, coef, monos, x)
    simple = sum(c * np.prod([x[v] for v in m]) for c, m in zip(coef, monos))
    assert f0 == pytest.approx(simple, rel=1e-14)
    for v in range(8):
        dx = np.zeros(8)
        dx[v] = 1e-6
        fd = (_poly(8, coef, monos, x + dx)[0] - _poly(8, coef, monos, x - dx)[0]) / 2e-6
        assert g[v] == pytest.approx(fd, rel=1e-6, abs=1e-9)


# ---------------------------------------------------------------------------
# Splines (compact_radial.cpp:326-366; cubic_spline_set.cpp:8-46)
# ---------------------------------------------------------------------------
def test_spline_node_derivatives_are_not_a_knot_left_clamped_right():
    """The node-derivative solve equals scipy's CubicSpline with
    bc_type=("not-a-knot", "clamped") -- the restatement in
    test_mace_streamed_edges.py:217-326."""
    r, h = np.linspace(1e-12, 5.0, 64, retstep=True)
    v = np.sin(3 * r) * np.exp(-r) * (5.0 - r) ** 2
    d = np.zeros_like(v)
    assert oracle.lib().oracle_spline_derivatives(v, len(v), h, d) == 0
    ref = CubicSpline(r, v, bc_type=("not-a-knot", "clamped")).derivative()(r)
    np.testing.assert_allclose(d, ref, rtol=1e-9, atol=1e-10)


def test_hermite_spline_fp32_matches_scipy():
    """FP32 Hermite evaluation (test_cubic_spline_set.py:8-80 in FP32),
    including the clamped ends outside the grid."""
    r_cut = 5.0
    grid, h = np.linspace(0.0, r_cut, 20, retstep=True)
    fs = [np.sin(grid) * grid**2 * (r_cut - grid) ** 2, np.cos(grid) * grid**2 * (r_cut - grid) ** 2]
    spl = [CubicSpline(grid, f) for f in fs]
    vals = np.array([f for f in fs], np.float32)
    ders = np.array([s.derivative()(grid) for s in spl], np.float32)
    rr = np.concatenate([np.linspace(0, r_cut, 1000, endpoint=False), [r_cut, r_cut + 1.0, -0.5]])
    ov = np.zeros((len(rr), 2), np.float32)
    od = np.zeros((len(rr), 2), np.float32)
    oracle.lib().oracle_spline_eval_f32(np.float32(h), np.float32(0.0), 2, len(grid), vals.ravel(), ders.ravel(),
                                        rr, len(rr), ov.ravel(), od.ravel())
    inside = rr[:1000]
    for k in range(2):
        scale = np.max(np.abs(fs[k]))
        np.testing.assert_allclose(ov[:1000, k], spl[k](inside), rtol=0, atol=2e-6 * scale)
        np.testing.assert_allclose(od[:1000, k], spl[k].derivative()(inside), rtol=0, atol=2e-5 * scale)
        # clamping: beyond the last node the value is the end value; before the first, the first
        assert ov[1001, k] == pytest.approx(float(vals[k, -1]), abs=1e-4 * scale)
        assert ov[1002, k] == pytest.approx(float(vals[k, 0]), abs=1e-6)


def test_radial_features_closed_form(tiny_model_path):
    """Bessel x polynomial cutoff features (compact_radial.cpp:227-267)."""
    m = oracle.OracleModel(tiny_model_path)
    feats = m.radial_features()
    with open(tiny_model_path) as f:
        j = json.load(f)
    cr = j["compact_radial"]
    S = cr["num_spline_points"]
    r = cr["spline_grid_min"] + np.arange(S) * (j["r_cut"] - cr["spline_grid_min"]) / (S - 1)
    p = cr["cutoff"]["p"]
    s = r / j["r_cut"]
    u = 1 - (p + 1) * (p + 2) / 2 * s**p + p * (p + 2) * s ** (p + 1) - p * (p + 1) / 2 * s ** (p + 2)
    u[r >= j["r_cut"]] = 0.0
    w = np.array(cr["basis"]["weights"])
    ref = cr["basis"]["prefactor"] * np.sin(np.outer(r, w)) / r[:, None] * u[:, None]
    np.testing.assert_allclose(feats, ref, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# Spherical harmonics (spherical_harmonic_device.hpp:15-199)
# ---------------------------------------------------------------------------
def _real_sh_scipy(l, u):
    """Orthonormal real harmonics from scipy's complex ones (Condon-Shortley
    phase removed), columns m = -l..l."""
    x, y, z = u[:, 0], u[:, 1], u[:, 2]
    theta = np.arccos(np.clip(z, -1, 1))
    phi = np.arctan2(y, x)
    out = []
    for m in range(-l, l + 1):
        Y = sph_harm_y(l, abs(m), theta, phi)
        if m < 0:
            out.append(np.sqrt(2) * (-1) ** m * Y.imag)
        elif m == 0:
            out.append(Y.real)
        else:
            out.append(np.sqrt(2) * (-1) ** m * Y.real)
    return np.stack(out, axis=1)


def test_harmonics_match_scipy_in_the_shuffled_frame():
    """Y_lm(r) = sqrt(4 pi) * real SH at (z, x, y) (spherical_harmonic_device.hpp:160-176)."""
    rng = np.random.default_rng(1)
    v = rng.normal(size=(500, 3)) * 3.0
    Y = np.zeros((500, 16), np.float32)
    oracle.lib().oracle_harmonics(np.ascontiguousarray(v), 500, 3, Y.ravel(), None)
    u = v / np.linalg.norm(v, axis=1, keepdims=True)
    shuffled = u[:, [2, 0, 1]]
    for l in range(4):
        ref = math.sqrt(4 * math.pi) * _real_sh_scipy(l, shuffled)
        np.testing.assert_allclose(Y[:, l * l:(l + 1) ** 2], ref, rtol=0, atol=5e-6)


def test_harmonics_normalisation_and_y00():
    """Y00 == 1.0f exactly (test_spherical_harmonic_normalization.py:258) and
    the addition theorem sum_m Y_lm^2 = 2l+1."""
    rng = np.random.default_rng(2)
    v = rng.normal(size=(300, 3))
    Y = np.zeros((300, 16), np.float32)
    oracle.lib().oracle_harmonics(np.ascontiguousarray(v), 300, 3, Y.ravel(), None)
    assert np.all(Y[:, 0] == np.float32(1.0))
    for l in range(4):
        s = np.sum(Y[:, l * l:(l + 1) ** 2].astype(np.float64) ** 2, axis=1)
        np.testing.assert_allclose(s, 2 * l + 1, rtol=2e-6)


def test_harmonics_gradient_matches_finite_differences():
    """dY/dxyz (mace.cpp:1290-1298) against central differences of Y(xyz)."""
    rng = np.random.default_rng(4)
    v = rng.normal(size=(50, 3)) * 2.0
    G = np.zeros((50, 3, 16), np.float32)
    Y = np.zeros((50, 16), np.float32)
    oracle.lib().oracle_harmonics(np.ascontiguousarray(v), 50, 3, Y.ravel(), G.ctypes.data)
    h = 1e-5
    for c in range(3):
        dv = np.zeros(3)
        dv[c] = h
        fd = (e3.spherical_harmonics(v + dv, 3) - e3.spherical_harmonics(v - dv, 3)) / (2 * h)
        np.testing.assert_allclose(G[:, c, :], fd, rtol=0, atol=2e-4)


def test_generator_harmonics_equal_the_oracle():
    """The generator's float64 harmonics (used for equivariance tables) are
    the oracle's (same frame and normalisation)."""
    rng = np.random.default_rng(5)
    v = rng.normal(size=(100, 3))
    Y = np.zeros((100, 16), np.float32)
    oracle.lib().oracle_harmonics(np.ascontiguousarray(v), 100, 3, Y.ravel(), None)
    np.testing.assert_allclose(Y, e3.spherical_harmonics(v, 3), rtol=0, atol=5e-6)


# ---------------------------------------------------------------------------
# Neighbour list (neighbor_graph_kokkos.cpp:38-405) against brute force
# ---------------------------------------------------------------------------
def _brute_force_edges(pos, cell, cutoff):
    inv = np.linalg.inv(cell)
    frac = pos @ inv
    reach = [int(math.ceil(cutoff * np.linalg.norm(inv[:, a]))) + 1 for a in range(3)]
    out = set()
    n = len(pos)
    for i in range(n):
        for j in range(n):
            for a in range(-reach[0] - 1, reach[0] + 2):
                for b in range(-reach[1] - 1, reach[1] + 2):
                    for c in range(-reach[2] - 1, reach[2] + 2):
                        if i == j and a == b == c == 0:
                            continue
                        img = np.array([a, b, c]) - np.floor(frac[j]).astype(int) + np.floor(frac[i]).astype(int)
                        d = pos[j] - pos[i] + img @ cell
                        if d @ d <= cutoff * cutoff:
                            out.add((i, j, tuple(img)))
    return out


@pytest.mark.parametrize("seed,cutoff", [(0, 3.0), (1, 4.5), (2, 6.0)])
def test_neighbor_list_equals_brute_force(seed, cutoff):
    rng = np.random.default_rng(seed)
    cell = np.array([[7.0, 0.0, 0.0], [1.5, 6.5, 0.0], [-1.0, 0.8, 8.0]])
    pos = rng.uniform(-0.3, 1.3, size=(12, 3)) @ cell
    g = oracle.neighbor_graph(pos, cell, cutoff)
    got = set()
    for e, (i, j) in enumerate(zip(g["receivers"], g["sources"])):
        got.add((int(i), int(j), tuple(int(s) for s in g["shifts"][e])))
    assert len(got) == len(g["sources"])  # no duplicates
    assert got == _brute_force_edges(pos, cell, cutoff)
    # receiver-major order; fractional edge vectors reproduce the geometry
    assert np.all(np.diff(g["receivers"]) >= 0)
    d = g["fractional_xyz"] @ cell
    ref = pos[g["sources"]] - pos[g["receivers"]] + g["shifts"] @ cell
    np.testing.assert_allclose(d, ref, atol=1e-10)


# ---------------------------------------------------------------------------
# Whole model: forces/stress are derivatives of the energy; invariances
# ---------------------------------------------------------------------------
def _small_system():
    s = systems.srtio3_supercell(2, sigma=0.08, seed=3)
    return s


def test_oracle_forces_and_stress_are_energy_derivatives(tiny_model_path):
    """Central differences of the FP64 oracle energy (test_mace.py:713-750,
    test_symmetrix_calc.py:1201)."""
    m = oracle.OracleModel(tiny_model_path, fp64=True)
    s = _small_system()
    base = oracle.evaluate_system(m, s, skin=0.5)
    h = 1e-4
    rng = np.random.default_rng(7)
    for a in rng.choice(len(s["numbers"]), 4, replace=False):
        for c in range(3):
            plus = dict(s)
            minus = dict(s)
            pp = s["positions"].copy()
            pm = s["positions"].copy()
            pp[a, c] += h
            pm[a, c] -= h
            plus["positions"], minus["positions"] = pp, pm
            ep = oracle.evaluate_system(m, plus, skin=0.5)["energy"]
            em = oracle.evaluate_system(m, minus, skin=0.5)["energy"]
            assert base["forces"][a, c] == pytest.approx(-(ep - em) / (2 * h), abs=2e-6)
    # stress: sigma = (1/V) dE/d(strain)
    V = abs(np.linalg.det(s["cell"]))
    for (i, j) in [(0, 0), (1, 2), (2, 1)]:
        eps = np.zeros((3, 3))
        eps[i, j] = h
        def strained(sign):
            t = dict(s)
            F = np.eye(3) + sign * eps
            t["positions"] = s["positions"] @ F.T
            t["cell"] = s["cell"] @ F.T
            return oracle.evaluate_system(m, t, skin=0.5)["energy"]
        fd = (strained(+1) - strained(-1)) / (2 * h) / V
        assert base["stress"][i, j] == pytest.approx(fd, abs=1e-7)


def test_oracle_energy_invariances(tiny_model_path):
    """Rotation, translation and permutation invariance of the energy; forces
    rotate with the system."""
    m = oracle.OracleModel(tiny_model_path, fp64=True)
    s = _small_system()
    base = oracle.evaluate_system(m, s, skin=0.5)
    R = e3.random_rotation(np.random.default_rng(11))
    rot = dict(s)
    rot["positions"] = s["positions"] @ R.T
    rot["cell"] = s["cell"] @ R.T
    r = oracle.evaluate_system(m, rot, skin=0.5)
    assert r["energy"] == pytest.approx(base["energy"], abs=1e-9)
    np.testing.assert_allclose(r["forces"], base["forces"] @ R.T, atol=1e-9)
    tr = dict(s)
    tr["positions"] = s["positions"] + np.array([0.37, -1.2, 2.5])
    assert oracle.evaluate_system(m, tr, skin=0.5)["energy"] == pytest.approx(base["energy"], abs=1e-9)
    perm = np.random.default_rng(12).permutation(len(s["numbers"]))
    pm = dict(s)
    pm["positions"] = s["positions"][perm]
    pm["numbers"] = s["numbers"][perm]
    p = oracle.evaluate_system(m, pm, skin=0.5)
    assert p["energy"] == pytest.approx(base["energy"], abs=1e-9)
    np.testing.assert_allclose(p["forces"], base["forces"][perm], atol=1e-9)


def test_oracle_fp32_tracks_fp64(tiny_model_path):
    """FP32 vs FP64 of the same path (test_mace_streamed_edges.py:556)."""
    s = _small_system()
    r32 = oracle.evaluate_system(oracle.OracleModel(tiny_model_path), s, skin=0.5)
    r64 = oracle.evaluate_system(oracle.OracleModel(tiny_model_path, fp64=True), s, skin=0.5)
    n = len(s["numbers"])
    assert abs(r32["energy"] - r64["energy"]) / n < 1e-5
    assert np.max(np.abs(r32["forces"] - r64["forces"])) < 1e-4
    assert np.max(np.abs(r32["stress"] - r64["stress"])) < 1e-6


# ---------------------------------------------------------------------------
# Density scaling (A0_scaled / A1_scaled)
# ---------------------------------------------------------------------------
def _silu_mlp(net, x):
    """multilayer_perceptron.cpp:30-80 in numpy: [out][in] weights, scaled
    SiLU on hidden layers, linear output."""
    h = np.asarray(x, dtype=np.float64)
    layers = [np.asarray(w, dtype=np.float64).reshape(b, a)
              for w, a, b in zip(net["weights"], net["shape"][:-1], net["shape"][1:])]
    for k, W in enumerate(layers):
        h = h @ W.T
        if k + 1 < len(layers):
            h = net["activation_scale"] * h / (1.0 + np.exp(-h))
    return h


def _density_splines(path, model):
    with open(path) as f:
        j = json.load(f)
    cr = j["compact_radial"]
    S = cr["num_spline_points"]
    grid = cr["spline_grid_min"] + np.arange(S) * (j["r_cut"] - cr["spline_grid_min"]) / (S - 1)
    feats = model.radial_features()
    out = {}
    for which, name in ((2, "A0"), (3, "A1")):
        net = cr["networks"][name]
        assert net["postprocess"] == "tanh-square" and net["shape"][-1] == 1
        v = np.tanh(_silu_mlp(net, feats)[:, 0] ** 2)
        ov, od = model.radial_tables(which)
        np.testing.assert_allclose(ov[0], v, rtol=1e-12, atol=1e-14)
        spl = CubicSpline(grid, v, bc_type=("not-a-knot", "clamped"))
        np.testing.assert_allclose(od[0], spl.derivative()(grid), rtol=1e-8, atol=1e-9)
        out[name] = spl
    return out, j


def test_density_networks_and_scale_factors(tiny_scaled_model_path, tiny_model_path):
    """A0/A1 density networks: tanh(MLP(features)^2) on the grid (compact_radial.cpp:
    295-303), spline node derivatives not-a-knot/clamped; per-receiver factor
    s = 1 + sum over every CSR edge (skin edges at r clamped to the cutoff)
    of f(r) (mace_kokkos_first_interaction.cpp:1389-1406); A0 /= s in FP64
    after the A0 linear (:1409-1415), checked bit for bit against the
    unscaled model (identical weights otherwise)."""
    m = oracle.OracleModel(tiny_scaled_model_path)
    spl, _ = _density_splines(tiny_scaled_model_path, m)
    s = systems.srtio3_supercell(3, sigma=0.05, seed=0)
    ref = oracle.evaluate_system(m, s, skin=0.5)
    g, r = ref["graph"], ref["r"]
    assert np.any(r >= m.r_cut)  # the graph holds skin edges
    for name in ("A0", "A1"):
        fr = spl[name](np.clip(r, 1e-12, m.r_cut))
        expect = 1.0 + np.bincount(g["receivers"], weights=fr, minlength=len(s["numbers"]))
        np.testing.assert_allclose(m.stage(name + "_scale"), expect, rtol=1e-11)
    m0 = oracle.OracleModel(tiny_model_path)
    oracle.evaluate_system(m0, s, skin=0.5)
    n, C, nY = len(s["numbers"]), m.num_channels, m.num_lm
    a0_plain = m0.stage("A0").reshape(n, nY * C).astype(np.float32)
    a0_scaled = m.stage("A0").reshape(n, nY * C).astype(np.float32)
    expect = (a0_plain.astype(np.float64) / m.stage("A0_scale")[:, None]).astype(np.float32)
    assert a0_scaled.tobytes() == expect.tobytes()


def test_density_scaled_A1_is_linear_times_inverse_factor(tiny_scaled_model_path):
    """A1 = (A1 linear of Phi1) * float(1/s1) (mace_kokkos_second_interaction.cpp:
    1474-1487), the linear restated here in FP64 numpy."""
    m = oracle.OracleModel(tiny_scaled_model_path)
    with open(tiny_scaled_model_path) as f:
        j = json.load(f)
    s = systems.srtio3_supercell(3, sigma=0.05, seed=0)
    oracle.evaluate_system(m, s, skin=0.5)
    n, C, nY = len(s["numbers"]), m.num_channels, m.num_lm
    phi1 = m.stage("Phi1").reshape(n, m.num_lme, C)
    paths_l = j["Phi1_l"]
    lin = np.zeros((n, nY, C))
    base = 0
    for l in range(m.l_max + 1):
        ne = sum(1 for x in paths_l if x == l)
        if ne == 0:
            continue
        W = np.asarray(j["A1_weights"][l]).reshape(ne, C, C)
        for mm in range(2 * l + 1):
            for e in range(ne):
                lin[:, l * l + mm, :] += phi1[:, base + mm * ne + e, :] @ W[e]
        base += (2 * l + 1) * ne
    inv = (1.0 / m.stage("A1_scale")).astype(np.float32).astype(np.float64)
    a1 = m.stage("A1").reshape(n, nY, C)
    np.testing.assert_allclose(a1, lin * inv[:, None, None], rtol=0, atol=2e-6 * np.abs(lin).max())


def test_density_scaled_forces_and_stress_are_energy_derivatives(tiny_scaled_model_path):
    """Central differences of the FP64 oracle energy with both density scales:
    pins the reverse (edge-force terms (dot/s) f'(r) r^ and the scaled
    adjoints)."""
    m = oracle.OracleModel(tiny_scaled_model_path, fp64=True)
    s = _small_system()
    base = oracle.evaluate_system(m, s, skin=0.5)
    assert np.max(np.abs(m.stage("density_forces"))) > 1e-3
    h = 1e-4
    rng = np.random.default_rng(8)
    for a in rng.choice(len(s["numbers"]), 4, replace=False):
        for c in range(3):
            plus, minus = dict(s), dict(s)
            pp, pm = s["positions"].copy(), s["positions"].copy()
            pp[a, c] += h
            pm[a, c] -= h
            plus["positions"], minus["positions"] = pp, pm
            ep = oracle.evaluate_system(m, plus, skin=0.5)["energy"]
            em = oracle.evaluate_system(m, minus, skin=0.5)["energy"]
            assert base["forces"][a, c] == pytest.approx(-(ep - em) / (2 * h), abs=2e-6)
    V = abs(np.linalg.det(s["cell"]))
    for (i, k) in [(0, 0), (2, 1)]:
        eps = np.zeros((3, 3))
        eps[i, k] = h

        def strained(sign):
            t = dict(s)
            F = np.eye(3) + sign * eps
            t["positions"] = s["positions"] @ F.T
            t["cell"] = s["cell"] @ F.T
            return oracle.evaluate_system(m, t, skin=0.5)["energy"]
        assert base["stress"][i, k] == pytest.approx((strained(+1) - strained(-1)) / (2 * h) / V, abs=1e-7)


# ---------------------------------------------------------------------------
# ZBL pair repulsion (zbl_kokkos.cpp)
# ---------------------------------------------------------------------------
_ZBL_RADII = [0.2, 0.31, 0.28, 1.28, 0.96, 0.84, 0.76, 0.71, 0.66, 0.57, 0.58]
_ZBL_C = [0.1818, 0.5099, 0.2802, 0.02817]


def test_zbl_known_answers():
    """The reference's test_zbl.py:1-44 values: envelope 0.4374788794430078
    and V 0.3166652764835175 for Z 5-10 at 1 A; zero at r_max; gradients
    against central differences."""
    r_max = _ZBL_RADII[5] + _ZBL_RADII[10]
    v, g, env, env_g = oracle.zbl_pair(0.3, 0.4543, _ZBL_C, _ZBL_RADII, 6, 5, 10, 1.0)
    assert env == pytest.approx(0.4374788794430078)
    assert v == pytest.approx(0.3166652764835175)
    assert oracle.zbl_pair(0.3, 0.4543, _ZBL_C, _ZBL_RADII, 6, 5, 10, r_max)[:4] == (0.0, 0.0, 0.0, 0.0)
    dx = 1e-4
    vp, _, ep, _ = oracle.zbl_pair(0.3, 0.4543, _ZBL_C, _ZBL_RADII, 6, 5, 10, 1.0 + dx)
    vm, _, em, _ = oracle.zbl_pair(0.3, 0.4543, _ZBL_C, _ZBL_RADII, 6, 5, 10, 1.0 - dx)
    assert g == pytest.approx((vp - vm) / (2 * dx))
    assert env_g == pytest.approx((ep - em) / (2 * dx))


def test_zbl_model_energy_is_the_pair_sum(tiny_zbl_model_path, tiny_model_path):
    """A ZBL model's energy is the plain model's plus sum over directed edges
    of V(Z_i, Z_j, r) (test_mace.py:753-790; mace_kokkos_evaluate.cpp:418-434),
    skin edges included (they lie beyond r_max)."""
    with open(tiny_zbl_model_path) as f:
        j = json.load(f)
    s = systems.srtio3_supercell(3, sigma=0.05, seed=0)
    mz = oracle.OracleModel(tiny_zbl_model_path, fp64=True)
    m0 = oracle.OracleModel(tiny_model_path, fp64=True)
    rz = oracle.evaluate_system(mz, s, skin=0.5)
    r0 = oracle.evaluate_system(m0, s, skin=0.5)
    g = rz["graph"]
    Z = np.asarray(s["numbers"])
    pairs = [oracle.zbl_pair(j["zbl_a_exp"], j["zbl_a_prefactor"], j["zbl_c"], j["zbl_covalent_radii"], j["zbl_p"],
                             int(Z[i]), int(Z[k]), float(r))[0]
             for i, k, r in zip(g["receivers"], g["sources"], rz["r"])]
    assert sum(v != 0.0 for v in pairs) > 10
    per_node = np.bincount(g["receivers"], weights=pairs, minlength=len(Z))
    np.testing.assert_allclose(rz["energies"] - r0["energies"], per_node, rtol=0, atol=1e-12)


def test_zbl_forces_and_stress_are_energy_derivatives(tiny_zbl_model_path):
    m = oracle.OracleModel(tiny_zbl_model_path, fp64=True)
    s = systems.srtio3_supercell(2, sigma=0.15, seed=5)
    base = oracle.evaluate_system(m, s, skin=0.5)
    assert np.max(np.abs(m.stage("zbl_forces"))) > 1e-3
    h = 1e-5
    rng = np.random.default_rng(9)
    for a in rng.choice(len(s["numbers"]), 5, replace=False):
        for c in range(3):
            plus, minus = dict(s), dict(s)
            pp, pm = s["positions"].copy(), s["positions"].copy()
            pp[a, c] += h
            pm[a, c] -= h
            plus["positions"], minus["positions"] = pp, pm
            ep = oracle.evaluate_system(m, plus, skin=0.5)["energy"]
            em = oracle.evaluate_system(m, minus, skin=0.5)["energy"]
            assert base["forces"][a, c] == pytest.approx(-(ep - em) / (2 * h), abs=2e-6)
    V = abs(np.linalg.det(s["cell"]))
    eps = np.zeros((3, 3))
    eps[0, 1] = h

    def strained(sign):
        t = dict(s)
        F = np.eye(3) + sign * eps
        t["positions"] = s["positions"] @ F.T
        t["cell"] = s["cell"] @ F.T
        return oracle.evaluate_system(m, t, skin=0.5)["energy"]
    assert base["stress"][0, 1] == pytest.approx((strained(+1) - strained(-1)) / (2 * h) / V, abs=1e-7)


# ---------------------------------------------------------------------------
# Prediction heads (prediction_heads.hpp)
# ---------------------------------------------------------------------------
def test_prediction_head_payload_replaces_the_top_level_fields(tiny_heads_model_path, tiny_model_path, tmp_path):
    """Selecting a head equals a single-head file whose top-level fields are
    that head's payload (prediction_heads.hpp:83-88); the default head is the
    section's default; an unknown head is refused."""
    with open(tiny_heads_model_path) as f:
        j = json.load(f)
    section = j.pop("prediction_heads")
    flat = dict(j)
    flat.update(section["parameters"]["finetune"])
    flat_path = tmp_path / "finetune_flat.json"
    flat_path.write_text(json.dumps(flat))
    s = systems.srtio3_supercell(3, sigma=0.05, seed=0)
    a = oracle.evaluate_system(oracle.OracleModel(tiny_heads_model_path, head="finetune"), s, skin=0.5)
    b = oracle.evaluate_system(oracle.OracleModel(str(flat_path)), s, skin=0.5)
    assert a["energies"].tobytes() == b["energies"].tobytes()
    assert a["forces"].tobytes() == b["forces"].tobytes()
    d = oracle.evaluate_system(oracle.OracleModel(tiny_heads_model_path), s, skin=0.5)
    t = oracle.evaluate_system(oracle.OracleModel(tiny_model_path), s, skin=0.5)
    assert d["energies"].tobytes() == t["energies"].tobytes()
    assert abs(a["energy"] - d["energy"]) > 1.0
    with pytest.raises(ValueError, match="not in the model"):
        oracle.OracleModel(tiny_heads_model_path, head="absent")


# ---------------------------------------------------------------------------
# Agnesi distance transform (compact_radial.cpp:144-163, 227-267)
# ---------------------------------------------------------------------------
def test_agnesi_features_closed_form(tiny_agnesi_model_path):
    """Per-pair features: the Bessel basis at x = 1/(1 + a s^q/(1 + s^(q-p))),
    s = r/r0, r0 the mean covalent radius of the pair, times the polynomial
    cutoff of r itself."""
    m = oracle.OracleModel(tiny_agnesi_model_path)
    with open(tiny_agnesi_model_path) as f:
        j = json.load(f)
    cr = j["compact_radial"]
    tr = cr["distance_transform"]
    S = cr["num_spline_points"]
    r = cr["spline_grid_min"] + np.arange(S) * (j["r_cut"] - cr["spline_grid_min"]) / (S - 1)
    p = cr["cutoff"]["p"]
    s = r / j["r_cut"]
    u = 1 - (p + 1) * (p + 2) / 2 * s**p + p * (p + 2) * s ** (p + 1) - p * (p + 1) / 2 * s ** (p + 2)
    u[r >= j["r_cut"]] = 0.0
    w = np.array(cr["basis"]["weights"])
    for ti, tj in [(0, 0), (0, 1), (1, 2), (2, 0)]:
        r0 = 0.5 * (tr["covalent_radii"][ti] + tr["covalent_radii"][tj])
        sr = r / r0
        x = 1.0 / (1.0 + tr["a"] * sr ** tr["q"] / (1.0 + sr ** (tr["q"] - tr["p"])))
        ref = cr["basis"]["prefactor"] * np.sin(np.outer(x, w)) / x[:, None] * u[:, None]
        np.testing.assert_allclose(m.radial_features(ti, tj), ref, rtol=1e-12, atol=1e-12)


def test_agnesi_edges_use_their_pair_tables(tiny_agnesi_model_path, tmp_path):
    """An O-Ti dimer: with every covalent radius set to the O-Ti mean the
    model's tables are all the O-Ti pair's, so the dimer's energy and forces
    are unchanged only if its edges use the O-Ti pair's tables."""
    with open(tiny_agnesi_model_path) as f:
        j = json.load(f)
    z = j["atomic_numbers"]
    radii = j["compact_radial"]["distance_transform"]["covalent_radii"]
    mean = 0.5 * (radii[z.index(8)] + radii[z.index(22)])
    j["compact_radial"]["distance_transform"]["covalent_radii"] = [mean] * len(radii)
    flat = tmp_path / "agnesi_flat.json"
    flat.write_text(json.dumps(j))
    dimer = {"positions": np.array([[1.0, 1.0, 1.0], [2.9, 1.3, 1.2]]), "cell": np.eye(3) * 12.0,
             "numbers": np.array([8, 22])}
    a = oracle.evaluate_system(oracle.OracleModel(tiny_agnesi_model_path, fp64=True), dimer, skin=0.5)
    b = oracle.evaluate_system(oracle.OracleModel(str(flat), fp64=True), dimer, skin=0.5)
    assert len(a["graph"]["sources"]) == 2
    np.testing.assert_allclose(a["energies"], b["energies"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(a["forces"], b["forces"], rtol=1e-10, atol=1e-12)
    # and the O-O table differs: the same dimer with all radii at the O radius
    j["compact_radial"]["distance_transform"]["covalent_radii"] = [radii[z.index(8)]] * len(radii)
    oo = tmp_path / "agnesi_oo.json"
    oo.write_text(json.dumps(j))
    c = oracle.evaluate_system(oracle.OracleModel(str(oo), fp64=True), dimer, skin=0.5)
    assert abs(c["energy"] - a["energy"]) > 1e-6


def test_agnesi_forces_are_energy_derivatives(tiny_agnesi_model_path):
    m = oracle.OracleModel(tiny_agnesi_model_path, fp64=True)
    s = _small_system()
    base = oracle.evaluate_system(m, s, skin=0.5)
    h = 1e-4
    for a in (0, 5, 17):
        for c in range(3):
            plus, minus = dict(s), dict(s)
            pp, pm = s["positions"].copy(), s["positions"].copy()
            pp[a, c] += h
            pm[a, c] -= h
            plus["positions"], minus["positions"] = pp, pm
            fd = -(oracle.evaluate_system(m, plus, skin=0.5)["energy"]
                   - oracle.evaluate_system(m, minus, skin=0.5)["energy"]) / (2 * h)
            assert base["forces"][a, c] == pytest.approx(fd, abs=2e-6)
