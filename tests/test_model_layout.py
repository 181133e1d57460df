"""Pins the oracle's reading of the format-4 model file against the
reference's own writer and exporter (no GPU).

The fixtures tests/golden/compact_*.json.gz were written by the reference's
`foundation_r1_test_model` (symmetrix/test/compact_r1_model.py:8-189; script
tests/golden/make_compact_models.py).  Its construction fixes what each JSON
index means, so each stage of the oracle is checked against a closed form in
the writer's own terms, taken from the oracle's previous stage:

* radial networks: `weights[output * embedding + feature]`, one linear layer
  (compact_r1_model.py:30-41; MultilayerPerceptron::evaluate, row-major
  weights, no activation on the last layer, multilayer_perceptron.cpp:34-79);
  R0 output l*C+k, R1 output p*C+k (the contract's "path_channel" message
  layout);
* H0_weights [element][channel] (compact_r1_model.py:117-121);
* A0_weights[element][l], diagonal 0.4+0.02 l (:122-128);
* M0_monomials {LM: [[vars]]}, M0_weights {element}{LM}{channel}[term]
  (:49-82);
* H1_weights blocks per l, diagonal 0.5/(l+1) (:150, repeated_diagonal);
* Phi1 rows as the contract's terms number them (per output l: m-major,
  path-minor);
* A1_weights[l] blocks per path e, diagonal 0.3/(e+1) (:157-159);
* M1 linear monomials, M1_weights {element}{channel}[component] (:83-90);
* H2 = 0.5 M1 (H2_weights_for_M0 zero), node energy
  sum_h 0.4 silu(sum_c W1[h][c] H2[c]) with readout_2_weights_1[h*C + c]
  (:91-93, 161-167; extract_mace_data.py:1669-1674 writes the same
  [hidden][channel] order).

The writer's square blocks are diagonal, so their orientation is pinned
separately, on a model with non-symmetric weights, by the exporter's
conventions: e3nn linears act as x @ W with W [in][out]
(extract_mace_data.py:985-1001 for A0, 1170-1184 for H1, 1432-1446 for A1,
1600-1611 for H2; symmetrix/source/symmetrix/h1_affine.py:184-186 "row = M0
channel, col = H1 channel", and its identity h2 = m @ T_z, :402-404).
"""

import json

import numpy as np
import pytest
from scipy.interpolate import CubicSpline

from _compact import compact_model, fixture_system
from oracle import oracle
from symmetrix import systems


def _l_of(lm):
    return int(np.floor(np.sqrt(lm)))


class Run:
    """One FP64 oracle evaluation of a fixture with its stages."""

    def __init__(self, name, fp64=True):
        self.path, self.j = compact_model(name)
        self.m = oracle.OracleModel(self.path, fp64=fp64)
        self.sys = fixture_system(name)
        self.out = oracle.evaluate_system(self.m, self.sys)
        g = self.out["graph"]
        self.types = self.m.types_of(self.sys["numbers"])
        self.recv = g["receivers"]
        self.src = g["sources"]
        self.r = self.out["r"]
        self.N = len(self.types)
        self.C = self.m.num_channels
        self.nY = (self.m.l_max + 1) ** 2
        self.nH = (self.m.L_max + 1) ** 2

    def stage(self, name, *shape):
        return self.m.stage(name).reshape(*shape)

    def radial(self, which):
        """Closed-form nodal values of network which (R0, R1) on the spline
        grid: W[out][feature] @ features (one linear layer)."""
        cr = self.j["compact_radial"]
        net = cr["networks"][which]
        emb, width = net["shape"]
        assert len(net["weights"]) == 1
        W = np.array(net["weights"][0]).reshape(width, emb)
        S = cr["num_spline_points"]
        x0 = cr["spline_grid_min"]
        grid = x0 + np.arange(S) * (self.j["r_cut"] - x0) / (S - 1)
        p = cr["cutoff"]["p"]
        s = grid / cr["cutoff"]["r_max"]
        u = 1 - (p + 1) * (p + 2) / 2 * s**p + p * (p + 2) * s ** (p + 1) - p * (p + 1) / 2 * s ** (p + 2)
        u[grid >= cr["cutoff"]["r_max"]] = 0.0
        w = np.array(cr["basis"]["weights"])
        feats = cr["basis"]["prefactor"] * np.sin(np.outer(grid, w)) / grid[:, None] * u[:, None]
        return grid, W @ feats.T  # [function][point]

    def radial_at_edges(self, which):
        """The network's spline (not-a-knot left, clamped right) at each
        edge length, r clamped to the cutoff: [edge][function]."""
        grid, values = self.radial(which)
        spl = CubicSpline(grid, values.T, bc_type=("not-a-knot", "clamped"), axis=0)
        return spl(np.minimum(self.r, self.j["r_cut"]))

    def lme_layout(self):
        """(l, e, m) -> Phi1 row, read from the contract's terms: a term's
        path is the one with its (l(lm1), l(lm2), l(lme)), e is that path's
        place among the paths of its output l.  The terms put the rows of an
        output l as m-major, path-minor: row = base(l) + m*n_e(l) + e."""
        paths = self.j["execution_contracts"]["R1"]["paths"]
        ne = [sum(1 for p in paths if p["output_l"] == l) for l in range(self.m.l_max + 1)]
        base = np.concatenate([[0], np.cumsum([ne[l] * (2 * l + 1) for l in range(self.m.l_max + 1)])])
        assert base[-1] == self.m.num_lme
        layout = {}
        for t in self.j["execution_contracts"]["R1"]["sparse_coupling"]["terms"]:
            l = int(np.searchsorted(base, t["lme"], side="right")) - 1
            key = (_l_of(t["lm1"]), _l_of(t["lm2"]), l)
            p = [i for i, q in enumerate(paths) if (q["edge_l"], q["source_l"], q["output_l"]) == key]
            assert len(p) == 1
            e = [i for i, q in enumerate(paths) if q["output_l"] == l].index(p[0])
            m, rem = divmod(int(t["lme"] - base[l]), ne[l])
            assert rem == e and 0 <= m < 2 * l + 1
            assert layout.setdefault((l, e, m), (int(t["lme"]), p[0])) == (int(t["lme"]), p[0])
        assert len(layout) == self.m.num_lme
        return layout


@pytest.fixture(scope="module", params=["compact_medium_m0", "compact_medium_linear", "compact_c4",
                                        "compact_omat0_small", "compact_mp0b2_large", "compact_off23_small",
                                        "compact_off23_large"])
def run(request):
    return Run(request.param)


def test_fixture_shapes_match_the_contracts(run):
    """The written files carry the contracts' shapes (channels, l_max,
    L_max, paths) and load in the oracle."""
    j = run.j
    contract = j["execution_contracts"]["R1"]
    assert run.m.num_channels == contract["channels"]
    assert run.m.l_max == contract["edge_harmonics"]["l_max"]
    assert run.m.L_max == contract["source_harmonics"]["l_max"]
    assert run.m.num_paths == len(contract["paths"])
    assert list(run.m.atomic_numbers) == j["atomic_numbers"]


def test_radial_tables_are_the_writers_linear_network(run):
    """Nodal R0 and R1 tables equal W[out][feature] @ features."""
    for which, idx in (("R0", 0), ("R1", 1)):
        _, ref = run.radial(which)
        got, _ = run.m.radial_tables(idx)
        np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-14)


def test_phi0_uses_l_major_r0_functions_and_h0_rows(run):
    """Phi0[i,lm,k] = sum_j R0_{l*C+k}(r) Y_lm H0[type_j][k]."""
    C, nY = run.C, run.nY
    R0 = run.radial_at_edges("R0")  # [E][(l_max+1) C]
    Y = run.stage("Y", -1, nY)
    H0 = np.array(run.j["H0_weights"]).reshape(run.m.num_elements, C)
    ref = np.zeros((run.N, nY, C))
    for lm in range(nY):
        l = _l_of(lm)
        msg = R0[:, l * C:(l + 1) * C] * Y[:, lm:lm + 1] * H0[run.types[run.src]]
        np.add.at(ref[:, lm, :], run.recv, msg)
    got = run.stage("Phi0", run.N, nY, C)
    np.testing.assert_allclose(got, ref, rtol=1e-9, atol=1e-12 * np.max(np.abs(ref)))


def test_a0_blocks_per_element_and_l(run):
    """A0 = Phi0 x A0_weights[type][l] (diagonal 0.4 + 0.02 l)."""
    C, nY = run.C, run.nY
    Phi0 = run.stage("Phi0", run.N, nY, C)
    A0 = run.stage("A0", run.N, nY, C)
    W = run.j["A0_weights"]
    for i in range(run.N):
        for lm in range(nY):
            l = _l_of(lm)
            d = np.array(W[run.types[i]][l]).reshape(C, C).diagonal()
            np.testing.assert_allclose(A0[i, lm], Phi0[i, lm] * d, rtol=1e-13, atol=1e-15)
    # the diagonal the writer puts there
    for l in range(run.m.l_max + 1):
        assert W[0][l][0] == pytest.approx(0.4 + 0.02 * l)


def test_m0_monomials_and_weight_nesting(run):
    """M0[i,LM,k] = sum_t c[type][LM][k][t] prod_{v in mono_t} A0[i,v,k]."""
    C, nY, nH = run.C, run.nY, run.nH
    A0 = run.stage("A0", run.N, nY, C)
    monos = run.j["M0_monomials"]
    coef = run.j["M0_weights"]
    ref = np.zeros((run.N, nH, C))
    for LM in range(nH):
        terms = monos[str(LM)]
        for i in range(run.N):
            c = np.array([coef[str(run.types[i])][str(LM)][str(k)] for k in range(C)])  # [C][term]
            for t, vars_ in enumerate(terms):
                prod = np.ones(C)
                for v in vars_:
                    prod = prod * A0[i, v]
                ref[i, LM] += c[:, t] * prod
    got = run.stage("M0", run.N, nH, C)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-13 * np.max(np.abs(ref)))


def test_h1_blocks_per_l(run):
    """H1[i,LM,k] = M0[i,LM,k] * 0.5/(l+1) (H1_weights blocks by l)."""
    C, nH = run.C, run.nH
    M0 = run.stage("M0", run.N, nH, C)
    H1 = run.stage("H1", run.N, nH, C)
    W = np.array(run.j["H1_weights"]).reshape(run.m.L_max + 1, C, C)
    for LM in range(nH):
        np.testing.assert_allclose(H1[:, LM], M0[:, LM] * W[_l_of(LM)].diagonal(), rtol=1e-13, atol=1e-16)


def test_phi1_rows_paths_and_r1_functions(run):
    """Phi1[i, lme, k] = sum_j sum_terms c R1_{p*C+k}(r) Y[lm1] H1[j,lm2,k]
    with the contract's terms, p the term's path."""
    C, nY, nH = run.C, run.nY, run.nH
    R1 = run.radial_at_edges("R1")
    Y = run.stage("Y", -1, nY)
    H1 = run.stage("H1", run.N, nH, C)
    layout = run.lme_layout()
    row_path = {row: p for (row, p) in layout.values()}
    contract = run.j["execution_contracts"]["R1"]
    ref = np.zeros((run.N, run.m.num_lme, C))
    Hs = H1[run.src]
    for t in contract["sparse_coupling"]["terms"]:
        lme, lm1, lm2, c = t["lme"], t["lm1"], t["lm2"], t["coefficient"]
        p = row_path[lme]
        msg = c * R1[:, p * C:(p + 1) * C] * Y[:, lm1:lm1 + 1] * Hs[:, lm2]
        np.add.at(ref[:, lme, :], run.recv, msg)
    got = run.stage("Phi1", run.N, run.m.num_lme, C)
    # the JSON restates the contract's terms
    assert run.j["Phi1_lme"] == [t["lme"] for t in contract["sparse_coupling"]["terms"]]
    np.testing.assert_allclose(got, ref, rtol=1e-9, atol=1e-11 * np.max(np.abs(ref)))


def test_a1_block_order_over_paths(run):
    """A1[i,lm,k] = sum_e 0.3/(e+1) Phi1[i, row(l,e,m), k]: the e-blocks of
    A1_weights[l] follow the paths of the Phi1 rows."""
    C, nY = run.C, run.nY
    Phi1 = run.stage("Phi1", run.N, run.m.num_lme, C)
    A1 = run.stage("A1", run.N, nY, C)
    layout = run.lme_layout()
    ref = np.zeros_like(A1)
    for (l, e, m), (row, _) in layout.items():
        W = np.array(run.j["A1_weights"][l]).reshape(-1, C, C)
        d = W[e].diagonal()
        assert d[0] == pytest.approx(0.3 / (e + 1))
        ref[:, l * l + m] += Phi1[:, row] * d
    np.testing.assert_allclose(A1, ref, rtol=1e-12, atol=1e-14 * max(1.0, np.max(np.abs(ref))))


def test_m1_h2_and_readout_layout(run):
    """M1 = sum_c 0.2/(1+c%4) A1[c] (linear monomials), H2 = 0.5 M1, and
    node energy sum_h W2[h] silu(sum_c W1[h][c] H2[c]) with W1 [hidden][C]."""
    C, nY = run.C, run.nY
    A1 = run.stage("A1", run.N, nY, C)
    M1 = run.stage("M1", run.N, C)
    monos = run.j["M1_monomials"]
    coef = run.j["M1_weights"]
    ref = np.zeros((run.N, C))
    for i in range(run.N):
        c = np.array([coef[str(run.types[i])][str(k)] for k in range(C)])  # [C][term]
        for t, vars_ in enumerate(monos):
            prod = np.ones(C)
            for v in vars_:
                prod = prod * A1[i, v]
            ref[i] += c[:, t] * prod
    np.testing.assert_allclose(M1, ref, rtol=1e-12, atol=1e-14 * max(1.0, np.max(np.abs(ref))))
    H2 = run.stage("H2", run.N, C)
    np.testing.assert_allclose(H2, 0.5 * M1, rtol=1e-12, atol=1e-16)
    hidden = run.j.get("readout_2_hidden_size", 16)
    W1 = np.array(run.j["readout_2_weights_1"]).reshape(hidden, C)
    W2 = np.array(run.j["readout_2_weights_2"])
    pre = H2 @ W1.T
    act = run.j["readout_2_scale_factor"] * pre / (1 + np.exp(-pre))
    E0 = np.array(run.j["atomic_energies"])[run.types]
    energies = E0 + act @ W2
    np.testing.assert_allclose(run.out["energies"], energies, rtol=1e-11, atol=1e-14)
    # a [C][hidden] misreading gives another energy
    W1_wrong = np.array(run.j["readout_2_weights_1"]).reshape(C, hidden).T if C >= hidden else W1
    pre_w = H2 @ W1_wrong.T
    wrong = E0 + (pre_w / (1 + np.exp(-pre_w))) @ W2
    if C > hidden:
        assert np.max(np.abs(wrong - energies)) > 1e-3 * np.max(np.abs(energies))


def test_forces_of_the_reference_written_model_match_finite_differences():
    """The reverse of the fixture model: central differences of the FP64
    oracle energy for a few atoms' forces."""
    r = Run("compact_medium_linear")
    pos0 = np.asarray(r.sys["positions"], dtype=np.float64)
    h = 1e-5
    for atom in (0, 7, 21):
        for c in range(3):
            e = []
            for sgn in (1, -1):
                p = pos0.copy()
                p[atom, c] += sgn * h
                e.append(oracle.evaluate_system(r.m, r.sys, positions=p, graph=r.out["graph"])["energy"])
            fd = -(e[0] - e[1]) / (2 * h)
            assert r.out["forces"][atom, c] == pytest.approx(fd, rel=1e-6, abs=1e-9)


# ---------------------------------------------------------------------------
# Orientation of the square blocks (exporter conventions), random weights
# ---------------------------------------------------------------------------
def test_square_blocks_are_in_by_out(tiny_model_path):
    """With non-symmetric random weights: A0 = Phi0 @ A0_weights[type][l],
    H1 = M0 @ H1_weights[l], A1 = Phi1_block(l) @ A1_weights[l] over rows
    (e, k_in), H2 = x @ T_type + M1 @ W_M1 (all [in][out])."""
    m = oracle.OracleModel(tiny_model_path, fp64=True)
    with open(tiny_model_path) as f:
        j = json.load(f)
    s = systems.srtio3_supercell(2, sigma=0.08, seed=5)
    out = oracle.evaluate_system(m, s)
    types = m.types_of(s["numbers"])
    N, C = len(types), m.num_channels
    nY, nH, nL = (m.l_max + 1) ** 2, (m.L_max + 1) ** 2, m.num_lme
    Phi0 = m.stage("Phi0").reshape(N, nY, C)
    A0 = m.stage("A0").reshape(N, nY, C)
    for i in range(N):
        for lm in range(nY):
            W = np.array(j["A0_weights"][types[i]][_l_of(lm)]).reshape(C, C)
            assert np.max(np.abs(W - W.T)) > 1e-3
            np.testing.assert_allclose(A0[i, lm], Phi0[i, lm] @ W, rtol=1e-10, atol=1e-12)
    M0 = m.stage("M0").reshape(N, nH, C)
    H1 = m.stage("H1").reshape(N, nH, C)
    W = np.array(j["H1_weights"]).reshape(m.L_max + 1, C, C)
    for LM in range(nH):
        np.testing.assert_allclose(H1[:, LM], M0[:, LM] @ W[_l_of(LM)], rtol=1e-10, atol=1e-12)
    Phi1 = m.stage("Phi1").reshape(N, nL, C)
    A1 = m.stage("A1").reshape(N, nY, C)
    row = 0
    for l in range(m.l_max + 1):
        ne = sum(1 for lo in j["Phi1_l"] if lo == l)
        W = np.array(j["A1_weights"][l]).reshape(ne * C, C)
        for mm in range(2 * l + 1):
            x = np.concatenate([Phi1[:, row + mm * ne + e] for e in range(ne)], axis=1)
            np.testing.assert_allclose(A1[:, l * l + mm], x @ W, rtol=1e-9, atol=1e-11)
        row += ne * (2 * l + 1)
    M1 = m.stage("M1").reshape(N, C)
    H2 = m.stage("H2").reshape(N, C)
    T = np.array(j["H2_weights_for_M0"]).reshape(m.num_elements, C, C)
    WM1 = np.array(j["H2_weights_for_M1"]).reshape(C, C)
    x = M0[:, 0]
    ref = np.stack([x[i] @ T[types[i]] for i in range(N)]) + M1 @ WM1
    np.testing.assert_allclose(H2, ref, rtol=1e-9, atol=1e-11)
