"""CPU restatement (numpy, float64) of the reference's MH-1 (``MACE_Nonlinear``)
evaluator.

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's cpu_baseline leg
as the checker of the HIP path.  The product (symmetrix-xl_amd/) never
imports this module.

It follows libsymmetrix/source/mace_nonlinear.cpp (the serial evaluator):

* irreps strings, e3nn ``Linear`` and the "uvu"/"uuu" tensor product:
  e3nn.cpp:83-407 (weights ``[mul_in, mul_out]`` row-major, path weight,
  optional bias per output element, output mask);
* the affine MLP (Linear / LayerNorm / SiLU): affine_mlp.cpp:38-330;
* the symmetric-contraction product basis with U tensors and element
  weights (degree nu uses ``weights_max`` at nu == correlation, else
  ``weights[correlation-nu-1]``), then the product linear plus the skip
  connection: e3nn_product.cpp:58-120, 296-470;
* the gate (SiLU scalars, sigmoid gates): mace_nonlinear.cpp:56-142;
* readouts (linear; linear-SiLU-linear): mace_nonlinear.cpp:216-258;
* radial features (Bessel of the optionally Agnesi-transformed distance,
  polynomial cutoff applied to the features or to the edge weights):
  mace_nonlinear.cpp:383-449;
* spherical harmonics: sphericart's real SH of (z, x, y) scaled by
  2 sqrt(pi): mace_nonlinear.cpp:451-469;
* the layer loop and energies: mace_nonlinear.cpp:523-781; ZBL:
  zbl.cpp:103-136, energies and forces scaled by the model scale.

Forces come from a reverse pass of this module's own (the adjoint order of
mace_nonlinear.cpp:782-1010), ending in dE/d(edge vector) per edge; the
per-edge derivatives of the radial features, the cutoff and the harmonics
are taken by complex-step differentiation of the same functions (exact to
rounding).  ``node_forces[e] = -dE/dxyz[e]``, the reference's per-edge
output; atom forces and stress follow from the standard reductions.

What pins it: central finite differences of the energy (forces and
stress), rotation/translation/permutation invariance (which fixes the
Wigner 3j, harmonics and U tensors to one basis), a hand-computed known
answer for each block's layout convention, and planted mistakes that those
checks must catch (tests/test_mh1_oracle.py).
"""

from __future__ import annotations

import json
import math
import re

import numpy as np

SQRT_4PI = math.sqrt(4.0 * math.pi)


def _vals(t):
    return np.asarray(t["values"], dtype=np.float64)


class Irreps:
    """'16x0e+16x1o' -> blocks (mul, l, parity, offset) (e3nn.cpp:83-112)."""

    def __init__(self, spec):
        self.blocks = []
        off = 0
        for token in spec.replace(" ", "").split("+"):
            m = re.fullmatch(r"(\d+)x(\d+)([eo])", token)
            if not m:
                raise ValueError("unsupported irreps %r" % spec)
            mul, l = int(m.group(1)), int(m.group(2))
            self.blocks.append((mul, l, 1 if m.group(3) == "e" else -1, off))
            off += mul * (2 * l + 1)
        self.dim = off


class Linear:
    """e3nn Linear (e3nn.cpp:114-245)."""

    def __init__(self, d):
        self.inp = Irreps(d["irreps_in"])
        self.out = Irreps(d["irreps_out"])
        w = _vals(d["weight"])
        self.instr = []
        off = 0
        for ins in d["instructions"]:
            mi, li, _, oi = self.inp.blocks[ins["i_in"]]
            mo, lo, _, oo = self.out.blocks[ins["i_out"]]
            if list(ins["path_shape"]) != [mi, mo] or li != lo:
                raise ValueError("unsupported linear path")
            self.instr.append((oi, mi, oo, mo, 2 * li + 1, float(ins.get("path_weight", 1.0)),
                               w[off:off + mi * mo].reshape(mi, mo)))
            off += mi * mo
        if off != len(w):
            raise ValueError("linear weight size")
        b = _vals(d["bias"])
        self.bias = b if len(b) else np.zeros(self.out.dim)
        self.mask = _vals(d["output_mask"])

    def forward(self, X):
        N = X.shape[0]
        Y = np.zeros((N, self.out.dim))
        for oi, mi, oo, mo, dd, pw, W in self.instr:
            xb = X[:, oi:oi + mi * dd].reshape(N, mi, dd)
            Y[:, oo:oo + mo * dd] += pw * np.einsum("nud,uw->nwd", xb, W).reshape(N, mo * dd)
        return (Y + self.bias) * self.mask

    def reverse(self, G):
        N = G.shape[0]
        Gm = G * self.mask
        X = np.zeros((N, self.inp.dim))
        for oi, mi, oo, mo, dd, pw, W in self.instr:
            gb = Gm[:, oo:oo + mo * dd].reshape(N, mo, dd)
            X[:, oi:oi + mi * dd] += pw * np.einsum("nwd,uw->nud", gb, W).reshape(N, mi * dd)
        return X


class TensorProduct:
    """e3nn TensorProduct with "uvu" and "uuu" paths (e3nn.cpp:247-407)."""

    def __init__(self, d):
        self.in1 = Irreps(d["irreps_in1"])
        self.in2 = Irreps(d["irreps_in2"])
        self.out = Irreps(d["irreps_out"])
        self.instr = []
        off = 0
        for ins in d["instructions"]:
            m1, l1, _, o1 = self.in1.blocks[ins["i_in1"]]
            m2, l2, _, o2 = self.in2.blocks[ins["i_in2"]]
            m3, l3, _, o3 = self.out.blocks[ins["i_out"]]
            w3j = _vals(ins["wigner_3j"]).reshape(2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1)
            mode = ins["connection_mode"]
            if mode == "uvu":
                if m3 != m1 or list(ins["path_shape"]) != [m1, m2]:
                    raise ValueError("uvu shape")
                n = m1 * m2
            elif mode == "uuu":
                if m3 != m1 or m2 != m1 or list(ins["path_shape"]) != [m1]:
                    raise ValueError("uuu shape")
                n = m1
            else:
                raise ValueError("mode %s" % mode)
            has_w = bool(ins["has_weight"])
            self.instr.append((mode, o1, m1, 2 * l1 + 1, o2, m2, 2 * l2 + 1, o3, 2 * l3 + 1,
                               float(ins.get("path_weight", 1.0)), w3j, has_w, off))
            if has_w:
                off += n
        self.numel = off
        self.internal = _vals(d["weight"])
        self.mask = _vals(d["output_mask"])

    def _w(self, Wt, B, mode, m1, m2, has_w, off):
        if not has_w:
            return np.ones((B, m1, m2)) if mode == "uvu" else np.ones((B, m1))
        if Wt is None:
            Wt = np.broadcast_to(self.internal, (B, self.numel))
        if mode == "uvu":
            return Wt[:, off:off + m1 * m2].reshape(B, m1, m2)
        return Wt[:, off:off + m1]

    def forward(self, X1, X2, Wt):
        B = X1.shape[0]
        Y = np.zeros((B, self.out.dim))
        for mode, o1, m1, d1, o2, m2, d2, o3, d3, pw, w3j, has_w, off in self.instr:
            x1 = X1[:, o1:o1 + m1 * d1].reshape(B, m1, d1)
            x2 = X2[:, o2:o2 + m2 * d2].reshape(B, m2, d2)
            w = self._w(Wt, B, mode, m1, m2, has_w, off)
            if mode == "uvu":
                y = np.einsum("buv,ijk,bui,bvj->buk", w, w3j, x1, x2, optimize=True)
            else:
                y = np.einsum("bu,ijk,bui,buj->buk", w, w3j, x1, x2)
            Y[:, o3:o3 + m1 * d3] += pw * y.reshape(B, m1 * d3)
        return Y * self.mask

    def reverse(self, X1, X2, Wt, G):
        B = X1.shape[0]
        Gm = G * self.mask
        A1 = np.zeros_like(X1)
        A2 = np.zeros_like(X2)
        AW = np.zeros((B, self.numel))
        for mode, o1, m1, d1, o2, m2, d2, o3, d3, pw, w3j, has_w, off in self.instr:
            x1 = X1[:, o1:o1 + m1 * d1].reshape(B, m1, d1)
            x2 = X2[:, o2:o2 + m2 * d2].reshape(B, m2, d2)
            g = pw * Gm[:, o3:o3 + m1 * d3].reshape(B, m1, d3)
            w = self._w(Wt, B, mode, m1, m2, has_w, off)
            if mode == "uvu":
                A1[:, o1:o1 + m1 * d1] += np.einsum("buv,ijk,bvj,buk->bui", w, w3j, x2, g, optimize=True).reshape(B, m1 * d1)
                A2[:, o2:o2 + m2 * d2] += np.einsum("buv,ijk,bui,buk->bvj", w, w3j, x1, g, optimize=True).reshape(B, m2 * d2)
                if has_w:
                    AW[:, off:off + m1 * m2] += np.einsum("ijk,bui,bvj,buk->buv", w3j, x1, x2, g, optimize=True).reshape(B, m1 * m2)
            else:
                A1[:, o1:o1 + m1 * d1] += np.einsum("bu,ijk,buj,buk->bui", w, w3j, x2, g).reshape(B, m1 * d1)
                A2[:, o2:o2 + m2 * d2] += np.einsum("bu,ijk,bui,buk->buj", w, w3j, x1, g).reshape(B, m2 * d2)
                if has_w:
                    AW[:, off:off + m1] += np.einsum("ijk,bui,buj,buk->bu", w3j, x1, x2, g)
        return A1, A2, AW


def _sigmoid(x):
    return 0.5 * (1.0 + np.tanh(0.5 * x))


class AffineMLP:
    """Linear / LayerNorm / SiLU stack (affine_mlp.cpp:38-330); LayerNorm with
    the biased variance."""

    def __init__(self, d):
        self.layers = []
        for L in d["layers"]:
            t = L["type"]
            if t == "linear":
                shape = L["weight"]["shape"]
                self.layers.append(("linear", _vals(L["weight"]).reshape(shape), _vals(L["bias"])))
            elif t == "layer_norm":
                self.layers.append(("ln", _vals(L["weight"]), _vals(L["bias"]), float(L["eps"])))
            elif t == "silu":
                self.layers.append(("silu",))
            else:
                raise ValueError("layer %s" % t)

    def forward(self, X):
        tape = [X]
        for L in self.layers:
            if L[0] == "linear":
                X = X @ L[1].T + L[2]
            elif L[0] == "ln":
                mu = X.mean(axis=1, keepdims=True)
                var = ((X - mu) ** 2).mean(axis=1, keepdims=True)
                X = (X - mu) / np.sqrt(var + L[3]) * L[1] + L[2]
            else:
                X = X * _sigmoid(X)
            tape.append(X)
        return X, tape

    def reverse(self, tape, G):
        for k in range(len(self.layers) - 1, -1, -1):
            L = self.layers[k]
            X = tape[k]
            if L[0] == "linear":
                G = G @ L[1]
            elif L[0] == "ln":
                mu = X.mean(axis=1, keepdims=True)
                var = ((X - mu) ** 2).mean(axis=1, keepdims=True)
                s = np.sqrt(var + L[3])
                xh = (X - mu) / s
                gh = G * L[1]
                G = (gh - gh.mean(axis=1, keepdims=True) - xh * (gh * xh).mean(axis=1, keepdims=True)) / s
            else:
                p = _sigmoid(X)
                G = G * (p + X * p * (1.0 - p))
        return G


class Gate:
    """SiLU on the scalars, sigmoid gates on the gated blocks
    (mace_nonlinear.cpp:56-142)."""

    def __init__(self, d):
        if d["scalar_activation"] != "silu" or d["gate_activation"] != "sigmoid":
            raise ValueError("gate activations")
        self.inp = Irreps(d["irreps_in"])
        self.scalars = Irreps(d["irreps_scalars"])
        self.gates = Irreps(d["irreps_gates"])
        self.gated = Irreps(d["irreps_gated"])
        self.sc = list(d["scalar_activation_constants"])
        self.gc = list(d["gate_activation_constants"])
        self.out_dim = self.scalars.dim + self.gated.dim

    def _segments(self):
        gate_off = self.scalars.dim
        gated_off = self.scalars.dim + self.gates.dim
        out_off = self.scalars.dim
        for k, (mul, l, _, _) in enumerate(self.gated.blocks):
            d = 2 * l + 1
            yield k, mul, d, gate_off, gated_off, out_off
            gate_off += mul
            gated_off += mul * d
            out_off += mul * d

    def forward(self, X):
        N = X.shape[0]
        Y = np.zeros((N, self.out_dim))
        for k, (mul, l, _, off) in enumerate(self.scalars.blocks):
            x = X[:, off:off + mul * (2 * l + 1)]
            Y[:, off:off + x.shape[1]] = self.sc[k] * x * _sigmoid(x)
        for k, mul, d, go, vo, oo in self._segments():
            g = self.gc[k] * _sigmoid(X[:, go:go + mul])
            Y[:, oo:oo + mul * d] = (g[:, :, None] * X[:, vo:vo + mul * d].reshape(N, mul, d)).reshape(N, mul * d)
        return Y

    def reverse(self, X, G):
        N = X.shape[0]
        A = np.zeros_like(X)
        for k, (mul, l, _, off) in enumerate(self.scalars.blocks):
            n = mul * (2 * l + 1)
            x = X[:, off:off + n]
            p = _sigmoid(x)
            A[:, off:off + n] = G[:, off:off + n] * self.sc[k] * (p + x * p * (1.0 - p))
        for k, mul, d, go, vo, oo in self._segments():
            p = _sigmoid(X[:, go:go + mul])
            v = X[:, vo:vo + mul * d].reshape(N, mul, d)
            g = G[:, oo:oo + mul * d].reshape(N, mul, d)
            A[:, vo:vo + mul * d] = (self.gc[k] * p[:, :, None] * g).reshape(N, mul * d)
            A[:, go:go + mul] = self.gc[k] * p * (1.0 - p) * np.sum(v * g, axis=2)
        return A


class Product:
    """Symmetric contraction + linear + skip (e3nn_product.cpp)."""

    def __init__(self, d):
        sc = d["symmetric_contractions"]
        self.inp = Irreps(sc["irreps_in"])
        self.out = Irreps(sc["irreps_out"])
        self.linear = Linear(d["linear"])
        self.use_sc = bool(d["use_sc"])
        self.agnostic = bool(d.get("use_agnostic_product", False))
        self.C = self.inp.blocks[0][0]
        self.ang = sum(2 * l + 1 for _, l, _, _ in self.inp.blocks)
        self.contractions = []
        for k, c in enumerate(sc["contractions"]):
            corr = int(c["correlation"])
            L = self.out.blocks[k][1]
            terms = []
            for nu in range(1, corr + 1):
                U = _vals(c["u_tensors"][nu - 1]).reshape(c["u_tensors"][nu - 1]["shape"])
                Wd = c["weights_max"] if nu == corr else c["weights"][corr - nu - 1]
                W = _vals(Wd).reshape(Wd["shape"])  # [elements, K, C]
                if L == 0:
                    U = U[None]
                # coefficients per element: [el, M, i1..inu, C]
                terms.append(np.einsum("...k,ekc->e...c", U, W))
            self.contractions.append((L, terms))

    def feature_major(self, X):
        N = X.shape[0]
        F = np.zeros((N, self.C, self.ang))
        a = 0
        for mul, l, _, off in self.inp.blocks:
            d = 2 * l + 1
            F[:, :, a:a + d] = X[:, off:off + mul * d].reshape(N, mul, d)
            a += d
        return F

    _FWD = {1: "mic,nci->ncm", 2: "mijc,nci,ncj->ncm", 3: "mijkc,nci,ncj,nck->ncm"}

    def _contract(self, F, elems):
        N = F.shape[0]
        out = np.zeros((N, self.out.dim))
        for (mul, l, _, off), (L, terms) in zip(self.out.blocks, self.contractions):
            acc = np.zeros((N, self.C, 2 * L + 1))
            for nu, coef in enumerate(terms, start=1):
                if nu > 3:
                    raise ValueError("correlation above 3")
                for e in np.unique(elems):
                    sel = elems == e
                    f = F[sel]
                    acc[sel] += np.einsum(self._FWD[nu], coef[e], *([f] * nu), optimize=True)
            out[:, off:off + mul * (2 * L + 1)] = acc.reshape(N, mul * (2 * L + 1))
        return out

    def forward(self, X, skip, elems):
        contracted = self._contract(self.feature_major(X), elems)
        y = self.linear.forward(contracted)
        return y + skip if self.use_sc else y

    def reverse(self, X, elems, G):
        F = self.feature_major(X)
        N = F.shape[0]
        gc = self.linear.reverse(G)
        AF = np.zeros_like(F)
        for (mul, l, _, off), (L, terms) in zip(self.out.blocks, self.contractions):
            g = gc[:, off:off + mul * (2 * L + 1)].reshape(N, self.C, 2 * L + 1)
            for nu, coef in enumerate(terms, start=1):
                for e in np.unique(elems):
                    sel = elems == e
                    c, f, gs = coef[e], F[sel], g[sel]
                    if nu == 1:
                        a = np.einsum("mic,ncm->nci", c, gs, optimize=True)
                    elif nu == 2:
                        a = (np.einsum("mijc,ncj,ncm->nci", c, f, gs, optimize=True)
                             + np.einsum("mjic,ncj,ncm->nci", c, f, gs, optimize=True))
                    else:
                        a = (np.einsum("mijkc,ncj,nck,ncm->nci", c, f, f, gs, optimize=True)
                             + np.einsum("mjikc,ncj,nck,ncm->nci", c, f, f, gs, optimize=True)
                             + np.einsum("mjkic,ncj,nck,ncm->nci", c, f, f, gs, optimize=True))
                    AF[sel] += a
        AX = np.zeros((N, self.inp.dim))
        a = 0
        for mul, l, _, off in self.inp.blocks:
            d = 2 * l + 1
            AX[:, off:off + mul * d] = AF[:, :, a:a + d].reshape(N, mul * d)
            a += d
        return AX, (G if self.use_sc else np.zeros_like(G))


class Readout:
    def __init__(self, d):
        self.nonlinear = d["class"] == "NonLinearReadoutBlock"
        if self.nonlinear:
            if d["activation"] != "silu":
                raise ValueError("readout activation")
            self.l1 = Linear(d["linear_1"])
            self.l2 = Linear(d["linear_2"])
            self.c = float(d["activation_constants"][0])
        elif d["class"] == "LinearReadoutBlock":
            self.l1 = Linear(d["linear"])
        else:
            raise ValueError("readout class %s" % d["class"])

    def forward(self, X):
        if not self.nonlinear:
            return self.l1.forward(X)[:, 0]
        h = self.l1.forward(X)
        return self.l2.forward(self.c * h * _sigmoid(h))[:, 0]

    def reverse(self, X, g):
        G = np.asarray(g, dtype=np.float64).reshape(-1, 1) * np.ones((X.shape[0], 1))
        if not self.nonlinear:
            return self.l1.reverse(G)
        h = self.l1.forward(X)
        p = _sigmoid(h)
        ah = self.l2.reverse(G) * self.c * (p + h * p * (1.0 - p))
        return self.l1.reverse(ah)


class Interaction:
    def __init__(self, d):
        if d["class"] != "RealAgnosticResidualNonLinearInteractionBlock":
            raise ValueError("interaction class")
        self.src = Linear(d["source_embedding"])
        self.tgt = Linear(d["target_embedding"])
        self.up = Linear(d["linear_up"])
        self.skip = Linear(d["skip_tp"])
        self.res = Linear(d["linear_res"])
        self.l1 = Linear(d["linear_1"])
        self.l2 = Linear(d["linear_2"])
        self.tp = TensorProduct(d["conv_tp"])
        self.wmlp = AffineMLP(d["conv_tp_weights"])
        self.dmlp = AffineMLP(d["density_fn"])
        self.gate = Gate(d["gate"])
        self.alpha = float(d["alpha"])
        self.beta = float(d["beta"])


def _sh(v, l_max):
    """Real SH of edge vectors (any dtype, complex-step safe), column
    l*l+l+m: sphericart's orthonormal form at (z, x, y)/r, times 2 sqrt(pi)."""
    r = np.sqrt(v[:, 0] * v[:, 0] + v[:, 1] * v[:, 1] + v[:, 2] * v[:, 2])
    x, y, z = v[:, 2] / r, v[:, 0] / r, v[:, 1] / r
    pi = math.pi
    out = [np.ones_like(x) * (0.5 / math.sqrt(pi))]
    if l_max >= 1:
        c1 = math.sqrt(3.0 / (4.0 * pi))
        out += [c1 * y, c1 * z, c1 * x]
    if l_max >= 2:
        c2, c20, c22 = 0.5 * math.sqrt(15.0 / pi), 0.25 * math.sqrt(5.0 / pi), 0.25 * math.sqrt(15.0 / pi)
        out += [c2 * x * y, c2 * y * z, c20 * (2 * z * z - x * x - y * y), c2 * x * z, c22 * (x * x - y * y)]
    if l_max >= 3:
        c33, c32 = 0.25 * math.sqrt(35.0 / (2.0 * pi)), 0.5 * math.sqrt(105.0 / pi)
        c31, c30, c32b = 0.25 * math.sqrt(21.0 / (2.0 * pi)), 0.25 * math.sqrt(7.0 / pi), 0.25 * math.sqrt(105.0 / pi)
        q = x * x + y * y
        out += [c33 * y * (3 * x * x - y * y), c32 * x * y * z, c31 * y * (4 * z * z - q), c30 * z * (2 * z * z - 3 * q),
                c31 * x * (4 * z * z - q), c32b * z * (x * x - y * y), c33 * x * (x * x - 3 * y * y)]
    if l_max > 3:
        raise ValueError("harmonics tabulated for l <= 3")
    return SQRT_4PI * np.stack(out, axis=1)


def _complex_step(fn, v, h=1e-30):
    """[E, 3, ...] derivatives of fn(v) (rows of v) by complex steps."""
    outs = []
    for c in range(3):
        vc = v.astype(np.complex128)
        vc[:, c] += 1j * h
        outs.append(np.imag(fn(vc)) / h)
    return np.stack(outs, axis=1)


class MH1Oracle:
    """The serial MH-1 evaluator in float64 (mace_nonlinear.cpp)."""

    def __init__(self, path):
        with open(path) as f:
            d = json.load(f)
        if d.get("model_type") != "MACE_Nonlinear" or d["symmetrix_format_version"] not in (3, 4):
            raise ValueError("not a MACE_Nonlinear file")
        self.atomic_numbers = list(d["atomic_numbers"])
        self.model_atomic_numbers = list(d["model_atomic_numbers"])
        self.model_indices = list(d["model_indices"])
        self.n_model = len(self.model_atomic_numbers)
        self.r_cut = float(d["r_cut"])
        self.l_max = int(d["l_max"])
        rad = d["radial_embedding"]
        self.apply_cutoff = bool(rad["apply_cutoff"])
        self.bessel = _vals(rad["basis"]["weights"])
        self.prefactor = float(rad["basis"]["prefactor"])
        self.p = int(rad["cutoff"]["p"])
        tr = rad["distance_transform"]
        self.agnesi = tr["type"] == "agnesi"
        if self.agnesi:
            self.ag = (float(tr["a"]), float(tr["q"]), float(tr["p"]))
            self.cov = np.asarray(tr["covalent_radii"], dtype=np.float64)
        self.scale = float(_vals(d["scale_shift"]["scale"])[0])
        self.shift = float(_vals(d["scale_shift"]["shift"])[0])
        ae = _vals(d["atomic_energies"])
        self.atomic_energies = np.array([ae[i] for i in self.model_indices])
        self.embedding = Linear(d["node_embedding"])
        self.interactions = [Interaction(x) for x in d["interactions"]]
        self.products = [Product(x) for x in d["products"]]
        self.readouts = [Readout(x) for x in d["readouts"]]
        self.has_zbl = bool(d["has_zbl"])
        if self.has_zbl:
            z = d["zbl"]
            self.zbl = (float(z["a_exp"]), float(z["a_prefactor"]), _vals(z["c"]), _vals(z["covalent_radii"]),
                        int(_vals(z["p"])[0]))

    def types_of(self, numbers):
        lut = {z: i for i, z in enumerate(self.atomic_numbers)}
        return np.array([lut[int(z)] for z in numbers], dtype=np.int32)

    # ---- per-edge scalar functions (complex-step safe) -------------------
    def _cutoff(self, r):
        x = r / self.r_cut
        p = float(self.p)
        v = (1.0 - 0.5 * (p + 1.0) * (p + 2.0) * x ** self.p + p * (p + 2.0) * x ** (self.p + 1)
             - 0.5 * p * (p + 1.0) * x ** (self.p + 2))
        return np.where(np.real(r) < self.r_cut, v, 0.0)

    def _radial(self, r, zs, zt):
        t = r
        if self.agnesi:
            a, q, p = self.ag
            r0 = 0.5 * (self.cov[zs] + self.cov[zt])
            x = r / r0
            t = 1.0 / (1.0 + a * x ** q / (1.0 + x ** (q - p)))
        f = self.prefactor * np.sin(self.bessel[None, :] * t[:, None]) / t[:, None]
        if self.apply_cutoff:
            f = f * self._cutoff(r)[:, None]
        return f

    def _zbl_edges(self, r, zi, zj):
        a_exp, a_pref, c, radii, p = self.zbl
        inv_a = (zi.astype(float) ** a_exp + zj.astype(float) ** a_exp) / (a_pref * 0.529)
        ra = r * inv_a
        k = (-3.2, -0.9423, -0.4028, -0.2016)
        phi = sum(c[i] * np.exp(k[i] * ra) for i in range(4))
        bare = 14.3996 * (zi * zj) / r * phi
        rmax = radii[zi] + radii[zj]
        x = r / rmax
        env = 1.0 - (p + 1.0) * (p + 2.0) / 2.0 * x ** p + p * (p + 2.0) * x ** (p + 1) \
            - p * (p + 1.0) / 2.0 * x ** (p + 2)
        return np.where(np.real(r) < rmax, 0.5 * bare * env, 0.0)

    @staticmethod
    def _density_adjoint(it, a_pre, s):
        """d/d(density) of pre_gate = lin1 / (alpha + beta density) + res."""
        return -np.sum(a_pre * s["lin1"], axis=1) * it.beta / s["norm"] ** 2

    # ---- evaluation -------------------------------------------------------
    def evaluate(self, types, receivers, sources, xyz, forces=True):
        """Node energies [N] and per-edge node_forces [E, 3] (= -dE/dxyz) of
        one graph: edge e points from receiver to source (xyz = r_source -
        r_receiver + shift), receivers sorted."""
        types = np.asarray(types)
        recv = np.asarray(receivers, dtype=np.int64)
        src = np.asarray(sources, dtype=np.int64)
        xyz = np.asarray(xyz, dtype=np.float64).reshape(-1, 3)
        N, E = len(types), len(src)
        midx = np.array(self.model_indices)[types]
        Z = np.array(self.atomic_numbers)[types]
        zs, zt = Z[src], Z[recv]
        r = np.sqrt(np.sum(xyz * xyz, axis=1))
        Y = _sh(xyz, self.l_max)
        cut = self._cutoff(r)
        rad = self._radial(r, zs, zt)
        onehot = np.zeros((N, self.n_model))
        onehot[np.arange(N), midx] = 1.0
        feats = self.embedding.forward(onehot)
        states = []
        layer_feats = []
        for it, prod in zip(self.interactions, self.products):
            s = {"input": feats}
            s["up"] = it.up.forward(feats)
            s["res"] = it.res.forward(s["up"])
            s["skip"] = it.skip.forward(feats)
            se, te = it.src.forward(onehot), it.tgt.forward(onehot)
            s["edge_in"] = np.concatenate([rad, se[src], te[recv]], axis=1)
            w, s["wtape"] = it.wmlp.forward(s["edge_in"])
            s["wraw"] = w
            if not self.apply_cutoff:
                w = w * cut[:, None]
            s["w"] = w
            m = it.tp.forward(s["up"][src], Y, w)
            s["msg"] = np.zeros((N, it.tp.out.dim))
            np.add.at(s["msg"], recv, m)
            draw, s["dtape"] = it.dmlp.forward(s["edge_in"])
            s["draw"] = draw[:, 0]
            s["dbase"] = np.tanh(s["draw"] ** 2)
            dv = s["dbase"] * cut if not self.apply_cutoff else s["dbase"]
            s["density"] = np.bincount(recv, weights=dv, minlength=N)
            s["lin1"] = it.l1.forward(s["msg"])
            s["norm"] = it.alpha + it.beta * s["density"]
            s["pre_gate"] = s["lin1"] / s["norm"][:, None] + s["res"]
            s["gated"] = it.gate.forward(s["pre_gate"])
            s["int_out"] = it.l2.forward(s["gated"])
            s["elems"] = np.zeros(N, dtype=np.int64) if prod.agnostic else midx
            feats = prod.forward(s["int_out"], s["skip"], s["elems"])
            layer_feats.append(feats)
            states.append(s)
        inter = sum(ro.forward(f) for ro, f in zip(self.readouts, layer_feats))
        energies = self.atomic_energies[types] + self.scale * inter + self.shift
        if self.has_zbl:
            ez = self._zbl_edges(r, zt, zs)
            energies = energies + self.scale * np.bincount(recv, weights=ez, minlength=N)
        self.stages = {"Y": Y, "radial": rad, "layer_features": layer_feats, "states": states}
        if not forces:
            return energies, None

        # ---- reverse (mace_nonlinear.cpp:782-1010) -------------------------
        adj = [ro.reverse(f, self.scale) for ro, f in zip(self.readouts, layer_feats)]
        rad_adj = np.zeros_like(rad)
        Y_adj = np.zeros_like(Y)
        cut_adj = np.zeros(E)
        for k in range(len(self.interactions) - 1, -1, -1):
            it, prod, s = self.interactions[k], self.products[k], states[k]
            a_out, a_skip = prod.reverse(s["int_out"], s["elems"], adj[k])
            a_gated = it.l2.reverse(a_out)
            a_pre = it.gate.reverse(s["pre_gate"], a_gated)
            a_lin = a_pre / s["norm"][:, None]
            a_res = a_pre
            a_dens = self._density_adjoint(it, a_pre, s)
            a_msg = it.l1.reverse(a_lin)
            a_up = it.res.reverse(a_res)
            a1, a2, aw = it.tp.reverse(s["up"][src], Y, s["w"], a_msg[recv])
            np.add.at(a_up, src, a1)
            Y_adj += a2
            if not self.apply_cutoff:
                cut_adj += np.sum(aw * s["wraw"], axis=1)
                aw = aw * cut[:, None]
            a_draw = a_dens[recv] * (1.0 - s["dbase"] ** 2) * 2.0 * s["draw"]
            if not self.apply_cutoff:
                cut_adj += a_dens[recv] * s["dbase"]
                a_draw = a_draw * cut
            a_in = it.wmlp.reverse(s["wtape"], aw) + it.dmlp.reverse(s["dtape"], a_draw[:, None])
            nb = rad.shape[1]
            rad_adj += a_in[:, :nb]
            a_feat = it.up.reverse(a_up) + it.skip.reverse(a_skip)
            if k > 0:
                adj[k - 1] = adj[k - 1] + a_feat
        # dE/dxyz through the radial features, the cutoff and the harmonics
        d_rad = _complex_step(lambda v: self._radial(np.sqrt(np.sum(v * v, axis=1)), zs, zt), xyz)
        d_cut = _complex_step(lambda v: self._cutoff(np.sqrt(np.sum(v * v, axis=1))), xyz)
        d_Y = _complex_step(lambda v: _sh(v, self.l_max), xyz)
        g = (np.einsum("eck,ek->ec", d_rad, rad_adj) + d_cut * cut_adj[:, None]
             + np.einsum("eck,ek->ec", d_Y, Y_adj))
        node_forces = -g
        if self.has_zbl:
            d_z = _complex_step(lambda v: self._zbl_edges(np.sqrt(np.sum(v * v, axis=1)), zt, zs), xyz)
            node_forces = node_forces - self.scale * d_z
        return energies, node_forces


def reduce_forces(n, receivers, sources, node_forces):
    """Atom forces of per-edge forces (xyz = r_source - r_receiver): the
    source gains node_forces[e], the receiver loses it."""
    F = np.zeros((n, 3))
    np.add.at(F, np.asarray(sources), node_forces)
    np.add.at(F, np.asarray(receivers), -node_forces)
    return F


def reduce_stress(node_forces, xyz, volume):
    """sigma = -(1/V) sum_e f_e xyz_e^T."""
    return -np.einsum("ea,eb->ab", node_forces, xyz) / volume


def evaluate_graph(model, types, receivers, sources, xyz, volume=None):
    e, f = model.evaluate(types, receivers, sources, xyz)
    out = {"energy": float(np.sum(e)), "energies": e, "node_forces": f,
           "forces": reduce_forces(len(types), receivers, sources, f)}
    if volume:
        out["stress"] = reduce_stress(f, np.asarray(xyz).reshape(-1, 3), volume)
    return out
