"""The table of harmonic-gradient coefficients the R0 reverse is compiled
against (csrc/harmonic_gradients.hpp).

The kernel forms the edge records' gradient terms through
    dY^c_q = (sum_q' G[q][c][q'] Y_q' - l u_c Y_q) / r     (q' of degree l - 1)
and reads 1/r as the trace of the l = 1 gradient block over 2 sqrt(3).  Both
are checked here against central differences of the package's real
spherical harmonics (symmetrix.e3, the edge convention: shuffled frame,
sqrt(4 pi) scale), which other tests pin against scipy; a wrong coefficient,
sign or axis fails.  The header is also what its generator writes.
"""

import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
HEADER = os.path.join(HERE, "..", "symmetrix-xl_amd", "csrc", "harmonic_gradients.hpp")


def _table():
    with open(HEADER) as f:
        text = f.read()
    body = text[text.index("kHarmonicGrad"):]
    body = body[body.index("= {"):body.index("};")]
    vals = [float(v) for v in re.findall(r"-?\d+\.\d+(?:e[-+]?\d+)?", body)]
    assert len(vals) == 16 * 3 * 9
    return np.array(vals).reshape(16, 3, 9)


def _gradients(vectors, h=1e-6):
    """d Y_q / d x_c of the edge vector x (central differences, FP64)."""
    from symmetrix import e3
    out = np.zeros((len(vectors), 3, 16))
    for c in range(3):
        d = np.zeros(3)
        d[c] = h
        out[:, c] = (e3.spherical_harmonics(vectors + d, 3) - e3.spherical_harmonics(vectors - d, 3)) / (2 * h)
    return out


def test_gradient_identity_against_the_harmonics():
    from symmetrix import e3
    G = _table()
    rng = np.random.default_rng(3)
    u = rng.normal(size=(200, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    r = rng.uniform(0.8, 6.5, size=(200, 1))
    x = u * r
    Y = e3.spherical_harmonics(x, 3)
    dY = _gradients(x)
    for q in range(16):
        l = int(np.floor(np.sqrt(q)))
        for c in range(3):
            lower = Y[:, (l - 1) ** 2:l * l] @ G[q, c, :2 * l - 1] if l > 0 else 0.0
            want = (lower - l * u[:, c] * Y[:, q]) / r[:, 0]
            np.testing.assert_allclose(dY[:, c, q], want, rtol=0, atol=2e-8, err_msg="q=%d c=%d" % (q, c))
    # 1/r from the trace of the l = 1 block
    trace = dY[:, 0, 1] + dY[:, 1, 2] + dY[:, 2, 3]
    np.testing.assert_allclose(trace / (2 * np.sqrt(3.0)), 1.0 / r[:, 0], rtol=1e-7)
    # a plausible slip: the l = 1 rows with their X and Z axes swapped
    bad = G.copy()
    bad[1:4, [0, 2]] = bad[1:4, [2, 0]]
    lower = Y[:, 0:1] @ bad[3, 0, :1]
    assert np.max(np.abs(dY[:, 0, 3] - (lower - u[:, 0] * Y[:, 3]) / r[:, 0])) > 1e-2


def test_header_is_what_its_generator_writes(tmp_path):
    import importlib.util
    gen = os.path.join(os.path.dirname(HEADER), "gen_harmonic_gradients.py")
    spec = importlib.util.spec_from_file_location("gen_harmonic_gradients", gen)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    mod.HERE = str(tmp_path)
    mod.main()
    with open(HEADER) as f, open(tmp_path / "harmonic_gradients.hpp") as g:
        assert f.read() == g.read()
