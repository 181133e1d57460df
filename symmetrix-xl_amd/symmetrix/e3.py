"""Equivariance tables for MACE models: real spherical harmonics, Wigner 3j
couplings and symmetric-contraction (product basis) supports.

Everything here is float64 numpy, used only to *build* a model file (the random
model generator) and by tests.  Nothing here runs on the evaluation path.

Conventions (they fix which model files are equivariant with which kernels):

* Real spherical harmonics follow the sphericart/Wikipedia real form evaluated
  at the shuffled direction (x', y', z') = (z, x, y) and scaled by sqrt(4 pi)
  ("component" normalisation, sum_m Y_lm^2 = 2l+1 on the unit sphere).  This is
  the reference's Y (libsymmetrix/source/mace.cpp:1269-1300,
  spherical_harmonic_device.hpp:160-176), and it equals e3nn's
  spherical_harmonics(normalize=True, normalization="component").
* Wigner 3j symbols are e3nn's real ones: complex Condon-Shortley
  Clebsch-Gordan coefficients (Racah formula) moved to the real basis with the
  (-i)^l-phased change of basis, then scaled to unit Frobenius norm.  The R1
  coupling coefficient of a "uvu" path is sqrt(2 l_out + 1) * w3j(l_source,
  l_edge, l_out)[m_source, m_edge, m_out]; this reproduces the reference's
  extracted coefficients (symmetrix/source/symmetrix/extract_mace_data.py:
  1326-1400) and its fixture
  symmetrix/test/data/execution_contracts/jit_r1_mace_mpa0_medium_contract.json.
* Product-basis (symmetric contraction) tensors are a basis of the space of
  degree-nu polynomials in the (l_max+1)^2 harmonic components that transform
  as the output irrep (with O(3) parity), computed as the null space of the
  equivariance constraint.  Their monomial support is basis independent and
  matches the reference's fixture
  symmetrix/test/data/execution_contracts/standard_m0_contract.json.
"""

from __future__ import annotations

import itertools
import math
from functools import lru_cache

import numpy as np

SQRT_4PI = math.sqrt(4.0 * math.pi)


# --------------------------------------------------------------------------
# Real spherical harmonics, l <= 3
# --------------------------------------------------------------------------

def _sph_unit_standard(x, y, z, l_max):
    """Standard real SH (orthonormal, no Condon-Shortley phase) of a unit
    vector, index lm = l*l + l + m."""
    pi = math.pi
    out = []
    out.append(np.full_like(x, 0.5 / math.sqrt(pi)))
    if l_max >= 1:
        c1 = math.sqrt(3.0 / (4.0 * pi))
        out += [c1 * y, c1 * z, c1 * x]
    if l_max >= 2:
        c2 = 0.5 * math.sqrt(15.0 / pi)
        c20 = 0.25 * math.sqrt(5.0 / pi)
        c22 = 0.25 * math.sqrt(15.0 / pi)
        out += [c2 * x * y, c2 * y * z, c20 * (2 * z * z - x * x - y * y),
                c2 * x * z, c22 * (x * x - y * y)]
    if l_max >= 3:
        c33 = 0.25 * math.sqrt(35.0 / (2.0 * pi))
        c32 = 0.5 * math.sqrt(105.0 / pi)
        c31 = 0.25 * math.sqrt(21.0 / (2.0 * pi))
        c30 = 0.25 * math.sqrt(7.0 / pi)
        c32b = 0.25 * math.sqrt(105.0 / pi)
        r2 = x * x + y * y
        out += [c33 * y * (3 * x * x - y * y), c32 * x * y * z,
                c31 * y * (4 * z * z - r2), c30 * z * (2 * z * z - 3 * r2),
                c31 * x * (4 * z * z - r2), c32b * z * (x * x - y * y),
                c33 * x * (x * x - 3 * y * y)]
    if l_max > 3:
        raise ValueError("real spherical harmonics are tabulated for l <= 3")
    return np.stack(out, axis=-1)


def spherical_harmonics(vectors, l_max):
    """MACE-normalised real SH of (N,3) vectors (normalised first), float64.
    Column lm = l*l + l + m."""
    v = np.asarray(vectors, dtype=np.float64)
    n = np.linalg.norm(v, axis=-1, keepdims=True)
    u = v / n
    # shuffle (x, y, z) -> (z, x, y) before the standard real form
    xs, ys, zs = u[..., 2], u[..., 0], u[..., 1]
    return SQRT_4PI * _sph_unit_standard(xs, ys, zs, l_max)


# --------------------------------------------------------------------------
# Rotations and Wigner D matrices in the real SH basis
# --------------------------------------------------------------------------

def random_rotation(rng):
    q = rng.normal(size=4)
    q /= np.linalg.norm(q)
    a, b, c, d = q
    return np.array([
        [a * a + b * b - c * c - d * d, 2 * (b * c - a * d), 2 * (b * d + a * c)],
        [2 * (b * c + a * d), a * a - b * b + c * c - d * d, 2 * (c * d - a * b)],
        [2 * (b * d - a * c), 2 * (c * d + a * b), a * a - b * b - c * c + d * d],
    ])


def wigner_D(l, R, samples=64, seed=12345):
    """D^l(R) with Y_l(R u) = D^l(R) Y_l(u) in the MACE real SH basis."""
    rng = np.random.default_rng(seed)
    u = rng.normal(size=(samples, 3))
    sl = slice(l * l, (l + 1) * (l + 1))
    Y = spherical_harmonics(u, l)[:, sl]
    YR = spherical_harmonics(u @ R.T, l)[:, sl]
    D, *_ = np.linalg.lstsq(Y, YR, rcond=None)
    return D.T


# --------------------------------------------------------------------------
# Wigner 3j (e3nn real convention)
# --------------------------------------------------------------------------

def _su2_cg(j1, m1, j2, m2, j3, m3):
    """Condon-Shortley Clebsch-Gordan <j1 m1 j2 m2 | j3 m3> (Racah formula)."""
    if m3 != m1 + m2 or abs(m1) > j1 or abs(m2) > j2 or abs(m3) > j3:
        return 0.0
    if j3 < abs(j1 - j2) or j3 > j1 + j2:
        return 0.0
    f = math.factorial
    pref = math.sqrt(
        (2 * j3 + 1) * f(j3 + j1 - j2) * f(j3 - j1 + j2) * f(j1 + j2 - j3)
        / f(j1 + j2 + j3 + 1))
    pref *= math.sqrt(f(j3 + m3) * f(j3 - m3) * f(j1 - m1) * f(j1 + m1)
                      * f(j2 - m2) * f(j2 + m2))
    s = 0.0
    for k in range(0, j1 + j2 - j3 + 1):
        a = [k, j1 + j2 - j3 - k, j1 - m1 - k, j2 + m2 - k,
             j3 - j2 + m1 + k, j3 - j1 - m2 + k]
        if min(a) < 0:
            continue
        den = 1
        for v in a:
            den *= f(v)
        s += (-1) ** k / den
    return pref * s


def _real_to_complex(l):
    """Unitary change of basis q[complex m, real m] with the (-i)^l phase that
    makes the coupling tensors real."""
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=np.complex128)
    s2 = 1.0 / math.sqrt(2.0)
    for m in range(-l, 0):
        q[l + m, l + abs(m)] = s2
        q[l + m, l - abs(m)] = -1j * s2
    q[l, l] = 1.0
    for m in range(1, l + 1):
        q[l + m, l + abs(m)] = (-1) ** m * s2
        q[l + m, l - abs(m)] = 1j * (-1) ** m * s2
    return (-1j) ** l * q


@lru_cache(maxsize=None)
def wigner_3j(l1, l2, l3):
    """Real Wigner 3j tensor [2l1+1, 2l2+1, 2l3+1], unit Frobenius norm."""
    C = np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1), dtype=np.complex128)
    for m1 in range(-l1, l1 + 1):
        for m2 in range(-l2, l2 + 1):
            m3 = m1 + m2
            if abs(m3) <= l3:
                C[l1 + m1, l2 + m2, l3 + m3] = _su2_cg(l1, m1, l2, m2, l3, m3)
    Q1, Q2, Q3 = _real_to_complex(l1), _real_to_complex(l2), _real_to_complex(l3)
    # q is indexed [complex m, real m]:
    # C_real[a, b, c] = sum_{ikn} q1[i,a] q2[k,b] conj(q3[n,c]) C[i,k,n]
    R = np.einsum("ia,kb,nc,ikn->abc", Q1, Q2, np.conj(Q3), C)
    if np.abs(R.imag).max() > 1e-10:
        raise RuntimeError("Wigner 3j change of basis is not real")
    R = R.real
    nrm = np.linalg.norm(R)
    return R / nrm if nrm > 0 else R


# --------------------------------------------------------------------------
# R1 (second interaction) tensor-product structure
# --------------------------------------------------------------------------

def r1_paths(l_max, L_max):
    """uvu paths of the second interaction, in e3nn's sorted order.

    Returns a list of (edge_l, source_l, output_l), built as MACE's
    tp_out_irreps_with_instructions: loop source irreps, then edge irreps, then
    the output irreps of their product that the target 0e+1o+...+l_max holds,
    then a stable sort by output irrep (l, parity)."""
    paths = []
    for ls in range(L_max + 1):
        ps = (-1) ** ls
        for le in range(l_max + 1):
            pe = (-1) ** le
            for lo in range(abs(ls - le), ls + le + 1):
                if lo <= l_max and ps * pe == (-1) ** lo:
                    paths.append((le, ls, lo))
    return sorted(paths, key=lambda p: p[2])


def r1_coupling(l_max, L_max):
    """Sparse R1 coupling in the reference's JSON form.

    Returns dict with Phi1_l, Phi1_l1, Phi1_l2, Phi1_lme, Phi1_clebsch_gordan,
    Phi1_lelm1lm2 (extract_mace_data.py:1326-1400 semantics: lm1 edge harmonic,
    lm2 source feature, rows enumerate (path, m1, m2), lme = [l][m][path-in-l])."""
    paths = r1_paths(l_max, L_max)
    Phi1_l = [p[2] for p in paths]
    Phi1_l1 = [p[0] for p in paths]
    Phi1_l2 = [p[1] for p in paths]
    num_e = [sum(1 for l in Phi1_l if l == ll) for ll in range(l_max + 1)]
    row_base = []
    acc = 0
    for (le, ls, lo) in paths:
        row_base.append(acc)
        acc += (2 * le + 1) * (2 * ls + 1)

    def lme_of(p, m):
        lo = Phi1_l[p]
        e = p - sum(1 for l in Phi1_l if l < lo)
        base = sum((2 * ll + 1) * num_e[ll] for ll in range(lo))
        return base + (lo + m) * num_e[lo] + e

    terms = []
    for p, (le, ls, lo) in enumerate(paths):
        W = wigner_3j(ls, le, lo) * math.sqrt(2 * lo + 1)
        for m1 in range(-le, le + 1):
            for m2 in range(-ls, ls + 1):
                row = row_base[p] + (le + m1) * (2 * ls + 1) + (ls + m2)
                for m in range(-lo, lo + 1):
                    c = W[ls + m2, le + m1, lo + m]
                    if abs(c) > 1e-12:
                        terms.append((le * le + le + m1, ls * ls + ls + m2,
                                      p, lme_of(p, m), row, float(c)))
    # reference ordering: edge_lm, source_lm, path, output_m
    terms.sort(key=lambda t: (t[0], t[1], t[2], t[3]))
    return {
        "Phi1_l": Phi1_l,
        "Phi1_l1": Phi1_l1,
        "Phi1_l2": Phi1_l2,
        "Phi1_lme": [t[3] for t in terms],
        "Phi1_clebsch_gordan": [t[5] for t in terms],
        "Phi1_lelm1lm2": [t[4] for t in terms],
        "_lm1": [t[0] for t in terms],
        "_lm2": [t[1] for t in terms],
    }


# --------------------------------------------------------------------------
# Symmetric contraction (product basis) tensors
# --------------------------------------------------------------------------

def _component_l(n_in):
    lmax = int(round(math.sqrt(n_in))) - 1
    return np.array([l for l in range(lmax + 1) for _ in range(2 * l + 1)])


@lru_cache(maxsize=None)
def symmetric_basis(l_in_max, L_out, nu, samples_factor=3, seed=7):
    """Basis of degree-nu O(3)-equivariant polynomials R^{(l_in_max+1)^2} ->
    irrep L_out (parity (-1)^L_out).

    Returns (monomials, U) with monomials a list of sorted index tuples and U
    an array [n_basis, 2L_out+1, n_monomials] (orthonormal rows)."""
    n_in = (l_in_max + 1) ** 2
    comp_l = _component_l(n_in)
    monos = [m for m in itertools.combinations_with_replacement(range(n_in), nu)
             if (sum(int(comp_l[i]) for i in m) - L_out) % 2 == 0]
    n_m = len(monos)
    d_out = 2 * L_out + 1
    rng = np.random.default_rng(seed)
    rots = [random_rotation(rng) for _ in range(2)]
    D_in = []
    D_out = []
    for R in rots:
        blocks = np.zeros((n_in, n_in))
        for l in range(l_in_max + 1):
            sl = slice(l * l, (l + 1) * (l + 1))
            blocks[sl, sl] = wigner_D(l, R)
        D_in.append(blocks)
        D_out.append(wigner_D(L_out, R))
    idx = np.array(monos, dtype=np.int64)  # [n_m, nu]
    n_samples = max(32, (samples_factor * n_m * d_out) // (2 * d_out) + 8)
    rows = []
    for D, Do in zip(D_in, D_out):
        x = rng.normal(size=(n_samples, n_in))
        xr = x @ D.T
        mx = np.prod(x[:, idx], axis=2)    # [S, n_m]
        mxr = np.prod(xr[:, idx], axis=2)  # [S, n_m]
        # T(Dx)_M - sum_M' Do[M,M'] T(x)_M' = 0 ; unknowns c[M', mono]
        for M in range(d_out):
            A = np.zeros((n_samples, d_out, n_m))
            A[:, M, :] += mxr
            for Mp in range(d_out):
                A[:, Mp, :] -= Do[M, Mp] * mx
            rows.append(A.reshape(n_samples, d_out * n_m))
    A = np.concatenate(rows, axis=0)
    # scale columns to unit norm for conditioning
    _, s, vt = np.linalg.svd(A, full_matrices=False)
    tol = s.max() * 1e-9
    null = vt[s < tol] if np.any(s < tol) else np.zeros((0, vt.shape[1]))
    # the SVD returns at most min(rows, cols) vectors; rows > cols here
    if null.shape[0] == 0:
        return monos, np.zeros((0, d_out, n_m))
    # clean tiny entries and re-orthonormalise
    null[np.abs(null) < 1e-10] = 0.0
    q, _ = np.linalg.qr(null.T)
    U = q.T.reshape(-1, d_out, n_m)
    U[np.abs(U) < 1e-11] = 0.0
    return monos, U


def product_basis_support(l_in_max, L_out, correlation):
    """For each output m, the sorted list of monomials (tuples) that carry a
    nonzero coefficient in some equivariant polynomial of degree <= correlation,
    ordered by (degree, lexicographic) as the reference's polynomial sorts them
    (libsymmetrix/source/multivariate_polynomial.cpp:22-40)."""
    d_out = 2 * L_out + 1
    support = [[] for _ in range(d_out)]
    for nu in range(1, correlation + 1):
        monos, U = symmetric_basis(l_in_max, L_out, nu)
        if U.shape[0] == 0:
            continue
        nz = np.abs(U).max(axis=0) > 1e-9  # [d_out, n_m]
        for M in range(d_out):
            support[M].extend(monos[j] for j in np.nonzero(nz[M])[0])
    return support


def coupling_chain_tensors(l_in_max, L_out, nu):
    """The unsymmetrised coupling-path tensors of MACE's symmetric contraction
    (e3nn's iterated Wigner 3j products over (l_1..l_nu) and every
    intermediate irrep, keeping the chains that end in L_out with parity
    (-1)^L_out), each embedded as [2L_out+1, n_in, ..., n_in]."""
    n_in = (l_in_max + 1) ** 2
    out = []
    for ls in itertools.product(range(l_in_max + 1), repeat=nu):
        states = [(ls[0], (-1) ** ls[0], np.eye(2 * ls[0] + 1))]
        for l in ls[1:]:
            nxt = []
            for (L, p, T) in states:
                for L2 in range(abs(L - l), L + l + 1):
                    W = wigner_3j(L, l, L2)
                    nxt.append((L2, p * (-1) ** l, np.einsum("M...,MmN->N...m", T, W)))
            states = nxt
        for (L, p, T) in states:
            if L == L_out and p == (-1) ** L_out:
                full = np.zeros((2 * L_out + 1,) + (n_in,) * nu)
                idx = tuple(slice(l * l, (l + 1) ** 2) for l in ls)
                full[(slice(None),) + idx] = T
                out.append(full)
    return out


@lru_cache(maxsize=None)
def structural_support(l_in_max, L_out, correlation):
    """Monomials per output m as the reference's extractor keys them
    (extract_mace_data.py:1013-1060): a sorted index tuple is a term when
    any *ordered* entry of any coupling-path tensor exceeds 1e-12, even if
    the symmetrised coefficient vanishes.  Ordered by (degree, lex) like
    multivariate_polynomial.cpp:22-40."""
    d_out = 2 * L_out + 1
    keys = [set() for _ in range(d_out)]
    for nu in range(1, correlation + 1):
        for T in coupling_chain_tensors(l_in_max, L_out, nu):
            for M in range(d_out):
                for t in np.argwhere(np.abs(T[M]) > 1e-12):
                    keys[M].add(tuple(sorted(int(v) for v in t)))
    return [sorted(k, key=lambda m: (len(m), m)) for k in keys]

