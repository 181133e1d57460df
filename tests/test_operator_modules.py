"""The reference's M0 / R0 operator-module container (code objects with the
``symmetrix_operator_*_v1`` identity symbols and ``symmetrix_{m0,r0}_*_v1``
kernels that OperatorModule::load reads, jit_operator_module.cpp:236-637)
built from this project's kernels.

CPU: the argument packets are the reference's byte layouts
(jit_operator_module_abi.h:23-79; the reference asserts 80 / 40 / 256 B,
jit_operator_module.cpp:18-20); a module rendered from reference-style
operator metadata compiles to a raw ELF64 code object carrying every
identity symbol and kernel; the model arrays a caller passes are exported in
the module layouts.

GPU: modules loaded and launched the way the reference's loader does
(identity read from the code object, min(ceil(work/threads), persistent)
blocks of the module's thread count, the packet by value), against the CPU
oracle's layer-1 stages of the same inputs:
  * M0 forward = the oracle's M0 from its A0; M0 reverse = its A0 adjoint
    from its M0 adjoint (which includes the readout's direct adjoint);
  * R0 forward with the ordered-pair table (R0 spline times the neighbour's
    H0 embedding) = the oracle's Phi0 (mace.cpp:1356-1403 before the A0
    linear); R0 coordinate reverse from the oracle's Phi0 adjoint = the
    oracle's R0 directed forces, with stored harmonic gradients and with
    gradients formed from FP32 unit coordinates, whole and in two receiver
    batches;
  * the density-scale chain (density prepare, scaled forward, reverse
    prepare, density term of the coordinate reverse) against central
    differences of the scaled forward along each edge's direction.
Tolerances: FP32 stages relative to their largest magnitude 1e-5 (forward)
and 2e-5 (adjoints); directed forces 1e-5 eV/A absolute.
"""

import ctypes
import os

import numpy as np
import pytest

from symmetrix import _native
from symmetrix import operator_modules as opm


def test_packet_layouts_match_the_reference_header():
    assert ctypes.sizeof(opm.M0Args) == 80
    assert opm.M0Args.input_scale_adjoint.offset == 72 and opm.M0Args.node_types.offset == 24
    assert ctypes.sizeof(opm.R0Spline) == 40
    assert ctypes.sizeof(opm.R0Args) == 256
    assert opm.R0Args.radial.offset == 112 and opm.R0Args.density.offset == 152
    assert opm.R0Args.harmonics.offset == 192 and opm.R0Args.cutoff.offset == 248


def _small_m0_metadata(artifact="jit-m0-test-artifact", structure="sha256:0123456789abcdef"):
    # reference-style metadata (jit_operator_codegen.py:40-84): 4 harmonics in,
    # 2 outputs, terms listed per output as component tuples
    return {
        "artifact_id": artifact, "structure_fingerprint": structure, "target": "gfx950", "precision": "float32",
        "input_components": 4, "output_components": 2, "correlation": 3,
        "contract": {"channels": 64, "monomial_groups": [
            {"output_component": 0, "terms": [[0], [0, 0], [1, 1], [2, 2], [3, 3], [0, 1, 1]]},
            {"output_component": 1, "terms": [[1], [0, 1], [1, 2, 3]]}]},
    }


def test_rendered_module_is_an_elf_code_object_with_the_identity(tmp_path):
    out = str(tmp_path / "m0.co")
    opm.build_m0_module(_small_m0_metadata(), out)
    data = opm.read_code_object(out)
    for name in ("symmetrix_m0_forward_v1", "symmetrix_m0_reverse_v1", "symmetrix_operator_artifact_id_v1",
                 "symmetrix_operator_structure_fingerprint_v1", "symmetrix_operator_target_v1",
                 "symmetrix_operator_term_count_v1", "symmetrix_operator_threads_v1"):
        assert name.encode() in data, name
    assert b"jit-m0-test-artifact\0" in data and b"sha256:0123456789abcdef\0" in data
    r0 = str(tmp_path / "r0.co")
    opm.build_r0_module({"artifact_id": "jit-r0-test", "structure_fingerprint": "sha256:r0", "target": "gfx950",
                         "input_components": 9, "contract": {"channels": 32}}, r0)
    data = opm.read_code_object(r0)
    for name in opm.R0_KERNELS:
        assert name.encode() in data, name


def test_builder_rejects_what_the_kernels_cannot_run(tmp_path):
    bad = _small_m0_metadata()
    bad["contract"]["monomial_groups"][0]["terms"].append([0, 1, 2, 3])   # degree 4
    with pytest.raises(ValueError):
        opm.build_m0_module(bad, str(tmp_path / "x.co"))
    with pytest.raises(ValueError):
        opm.render_r0_source(96, 2, "a", "b")                             # 96 does not divide 256
    with pytest.raises(ValueError):
        opm.render_r0_source(32, 2, 'quote"d', "b")
    with pytest.raises(ValueError):
        opm.read_code_object(__file__)


def test_compiled_shape_modules_are_built():
    for args in ((opm.KIND_M0, 32, 2, 1, 2), (opm.KIND_M0, 128, 3, 1, 3), (opm.KIND_M0, 256, 3, 2, 3),
                 (opm.KIND_R0, 32, 2), (opm.KIND_R0, 128, 3), (opm.KIND_R0, 256, 3)):
        path, _ = opm.compiled_module_path(*args)
        assert os.path.exists(path), path
        opm.read_code_object(path)


def test_model_arrays_in_module_layouts(tiny_model_path):
    w = _native.model_array(tiny_model_path, "M0_weights")
    terms = _native.model_array(tiny_model_path, "M0_terms")
    offsets = _native.model_array(tiny_model_path, "M0_offsets")
    spline, h, x0 = _native.model_array(tiny_model_path, "R0_spline")
    H0 = _native.model_array(tiny_model_path, "H0")
    assert w.shape == (3, 27, 32) and terms.shape == (27,)
    np.testing.assert_array_equal(offsets, [0, 10, 16, 21, 27])      # the tiny shape's compiled table
    assert spline.shape == (255, 4, 3 * 32) and H0.shape == (3, 32)
    assert h > 0 and x0 >= 0
    with pytest.raises(ValueError):
        _native.model_array(tiny_model_path, "no_such_array")


# --------------------------------------------------------------------- GPU
def _oracle_run(model_path, cells):
    from oracle import oracle
    from symmetrix import systems
    s = systems.srtio3_supercell(cells, sigma=0.05, seed=0)
    om = oracle.OracleModel(model_path)
    ref = oracle.evaluate_system(om, s, skin=0.5)
    return s, om, ref


def _relerr(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.mark.gpu
@pytest.mark.parametrize("name,cells,shape", [("tiny", 3, (32, 2, 1, 2)), ("medium", 10, (128, 3, 1, 3))])
def test_m0_module_matches_oracle(name, cells, shape, request):
    from _hip import DeviceArray, hip
    model_path = request.getfixturevalue("%s_model_path" % name)
    s, om, ref = _oracle_run(model_path, cells)
    C, l_max, L_max, corr = shape
    path, mod_name = opm.compiled_module_path(opm.KIND_M0, C, l_max, L_max, corr)
    mod = opm.CodeObject(path)
    terms = _native.model_array(model_path, "M0_terms")
    ident = mod.identity
    assert ident["abi_version"] == 1 and ident["kind"] == opm.KIND_M0 and ident["scalar_kind"] == 1
    assert ident["capabilities"] == opm.M0_CAPABILITIES and ident["threads"] == opm.THREADS
    assert ident["input_components"] == (l_max + 1) ** 2 and ident["output_components"] == (L_max + 1) ** 2
    assert ident["term_count"] == len(terms) and ident["correlation"] == corr
    assert ident["artifact_id"] == "symmetrix-mi355x-" + mod_name and ident["target"] == "gfx950"

    N = len(s["numbers"])
    NY, NH = (l_max + 1) ** 2, (L_max + 1) ** 2
    types = om.types_of(s["numbers"]).astype(np.int32)
    d_types = DeviceArray(types)
    d_w = DeviceArray(_native.model_array(model_path, "M0_weights"))
    d_in = DeviceArray(om.stage("A0").astype(np.float32))
    m0_ref = om.stage("M0").reshape(N, NH, C)
    for blocks in (3, 100000):
        d_out = DeviceArray(np.full((N, NH, C), np.nan, np.float32))
        a = opm.M0Args(ctypes.sizeof(opm.M0Args), 0, N, C, 0, d_types.value, d_in.value, d_w.value, None,
                       d_out.value, None, None)
        assert mod.launch("symmetrix_m0_forward_v1", a, N * C, blocks) == 0
        assert hip().hipDeviceSynchronize() == 0
        err = _relerr(d_out.get().astype(np.float64), m0_ref)
        print("%s M0 forward (%d blocks) relative max err %.3e" % (name, blocks, err))
        assert err < 1e-5

    adj_ref = om.stage("A0_adj").reshape(N, NY, C)
    d_adj = DeviceArray(om.stage("M0_adj").astype(np.float32))
    d_grad = DeviceArray(np.full((N, NY, C), np.nan, np.float32))
    d_scale = DeviceArray(np.zeros(N))
    a = opm.M0Args(ctypes.sizeof(opm.M0Args), 0, N, C, 1, d_types.value, d_in.value, d_w.value, d_adj.value,
                   None, d_grad.value, d_scale.value)
    assert mod.launch("symmetrix_m0_reverse_v1", a, N * C, 7) == 0
    assert hip().hipDeviceSynchronize() == 0
    grad = d_grad.get()
    err = _relerr(grad.astype(np.float64), adj_ref)
    print("%s M0 reverse relative max err %.3e" % (name, err))
    assert err < 2e-5
    # scale adjoint: sum over components and channels of input * input_adjoint
    x = d_in.get().reshape(N, NY, C).astype(np.float64)
    want = np.sum(x * grad.astype(np.float64), axis=(1, 2))
    np.testing.assert_allclose(d_scale.get(), want, rtol=1e-9, atol=1e-9 * np.max(np.abs(want)))
    # alias safety: the adjoint written over the input buffer
    d_alias = DeviceArray(om.stage("A0").astype(np.float32))
    a = opm.M0Args(ctypes.sizeof(opm.M0Args), 0, N, C, 0, d_types.value, d_alias.value, d_w.value, d_adj.value,
                   None, d_alias.value, None)
    assert mod.launch("symmetrix_m0_reverse_v1", a, N * C, 64) == 0
    assert hip().hipDeviceSynchronize() == 0
    assert d_alias.get().tobytes() == grad.tobytes()


def _r0_setup(model_path, s, om, ref, C, l_max):
    """Device inputs of the R0 module for the oracle's graph: the ordered-pair
    table [receiver*n + neighbour][interval][4][l*C + k] = R0 spline times
    H0[neighbour type][k]."""
    from _hip import DeviceArray
    g = ref["graph"]
    N, E = len(s["numbers"]), len(g["sources"])
    types = om.types_of(s["numbers"]).astype(np.int32)
    active = np.unique(types)
    n = len(active)
    to_active = np.full(int(types.max()) + 1, -1, np.int32)
    to_active[active] = np.arange(n, dtype=np.int32)
    spline, h, x0 = _native.model_array(model_path, "R0_spline")
    H0 = _native.model_array(model_path, "H0")
    table = np.empty((n * n,) + spline.shape, np.float32)
    for rt in range(n):
        for nt in range(n):
            emb = np.tile(H0[active[nt]], l_max + 1)                     # function l*C + k -> H0[k]
            table[rt * n + nt] = spline * emb[None, None, :]
    offsets = g["offsets"].astype(np.int32)
    sources = g["sources"].astype(np.int32)
    unit = (ref["xyz"] / ref["r"][:, None]).astype(np.float32)
    d = {
        "N": N, "E": E, "n": n, "types": types, "offsets": offsets,
        "table": DeviceArray(table), "h": h, "x0": x0, "intervals": spline.shape[0], "functions": spline.shape[2],
        "types_d": DeviceArray(types), "num": DeviceArray(np.diff(offsets).astype(np.int32)),
        "first": DeviceArray(offsets[:-1].copy()), "ntypes": DeviceArray(types[sources]),
        "recv": DeviceArray(np.repeat(np.arange(N, dtype=np.int32), np.diff(offsets))),
        "map": DeviceArray(to_active), "xyz": DeviceArray(ref["xyz"].astype(np.float64)),
        "unit": DeviceArray(unit), "r": DeviceArray(ref["r"].astype(np.float64)),
        "Y": DeviceArray(om.stage("Y").astype(np.float32)), "G": DeviceArray(om.stage("Ygrad").astype(np.float32)),
    }
    return d


def _r0_args(d, C, l_max, cutoff, **kw):
    radial = opm.spline(d["table"].value, d["n"] ** 2, d["intervals"], d["functions"], d["h"], d["x0"])
    a = opm.R0Args(ctypes.sizeof(opm.R0Args), 0, d["N"], d["E"], d["n"], C, l_max, 0, 0, 0, d["types_d"].value,
                   d["num"].value, d["first"].value, d["ntypes"].value, d["recv"].value, d["map"].value,
                   d["xyz"].value, d["r"].value, radial, opm.spline(), d["Y"].value, d["G"].value, None, None,
                   None, None, None, cutoff)
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.gpu
def test_r0_module_matches_oracle(tiny_model_path):
    from _hip import DeviceArray, hip
    s, om, ref = _oracle_run(tiny_model_path, 3)
    C, l_max = 32, 2
    NY = (l_max + 1) ** 2
    mod = opm.CodeObject(opm.compiled_module_path(opm.KIND_R0, C, l_max)[0])
    ident = mod.identity
    assert ident["kind"] == opm.KIND_R0 and ident["capabilities"] == opm.R0_CAPABILITIES
    assert ident["input_components"] == NY and ident["term_count"] == NY and ident["correlation"] == 1
    d = _r0_setup(tiny_model_path, s, om, ref, C, l_max)
    N, E = d["N"], d["E"]

    phi_ref = om.stage("Phi0").reshape(N, NY, C)
    d_out = DeviceArray(np.full((N, NY, C), np.nan, np.float32))
    a = _r0_args(d, C, l_max, om.r_cut, output=d_out.value)
    assert mod.launch("symmetrix_r0_forward_v1", a, N * NY * C, 5) == 0
    assert hip().hipDeviceSynchronize() == 0
    err = _relerr(d_out.get().astype(np.float64), phi_ref)
    print("R0 module forward relative max err %.3e" % err)
    assert err < 1e-5

    f_ref = om.stage("node_forces_r0").reshape(E, 3)
    d_adj = DeviceArray(om.stage("Phi0_adj").astype(np.float32))
    base = np.full((E, 3), 0.75)
    for label, kw in (("stored gradients", {}),
                      ("unit coordinates, gradients formed", {"coordinates_are_unit": 1,
                                                              "coordinates": d["unit"].value,
                                                              "harmonic_gradients": None})):
        d_f = DeviceArray(base)
        a = _r0_args(d, C, l_max, om.r_cut, output_adjoint=d_adj.value, directed_forces=d_f.value, **kw)
        assert mod.launch("symmetrix_r0_coordinate_reverse_v1", a, E, 11) == 0
        assert hip().hipDeviceSynchronize() == 0
        ferr = float(np.max(np.abs((d_f.get() - base) - f_ref)))
        print("R0 module coordinate reverse (%s) max abs err %.3e (scale %.3e)" % (label, ferr,
                                                                                   np.max(np.abs(f_ref))))
        assert ferr < 1e-5

    # two receiver batches: edge arrays offset to the batch, receivers
    # relative to receiver_base, node arrays of the batch
    split = N // 2
    e_split = int(d["offsets"][split])
    d_f = DeviceArray(base)
    keep = []
    for r0, r1 in ((0, split), (split, N)):
        e0, e1 = int(d["offsets"][r0]), int(d["offsets"][r1])
        adj = om.stage("Phi0_adj").reshape(N, NY, C)[r0:r1].astype(np.float32)
        bt = DeviceArray(d["types"][r0:r1].copy())
        badj = DeviceArray(adj)
        keep += [bt, badj]
        a = _r0_args(d, C, l_max, om.r_cut, receiver_base=r0, num_nodes=r1 - r0, num_edges=e1 - e0,
                     node_types=bt.value, output_adjoint=badj.value,
                     neigh_types=d["ntypes"].value + 4 * e0, edge_receivers=d["recv"].value + 4 * e0,
                     coordinates=d["xyz"].value + 24 * e0, radius=d["r"].value + 8 * e0,
                     harmonics=d["Y"].value + 4 * NY * e0, harmonic_gradients=d["G"].value + 12 * NY * e0,
                     directed_forces=d_f.value + 24 * e0)
        assert mod.launch("symmetrix_r0_coordinate_reverse_v1", a, e1 - e0, 9) == 0
    assert hip().hipDeviceSynchronize() == 0
    assert e_split > 0
    ferr = float(np.max(np.abs((d_f.get() - base) - f_ref)))
    print("R0 module coordinate reverse in receiver batches max abs err %.3e" % ferr)
    assert ferr < 1e-5


def _density_table(n, intervals, h, x0):
    """FP64 Hermite table [symmetric pair][interval][4][1] of a smooth
    per-pair density rho_t(r) = a_t exp(-r / 2)."""
    pairs = n * (n + 1) // 2
    knots = x0 + h * np.arange(intervals + 1)
    tab = np.zeros((pairs, intervals, 4, 1))
    for t in range(pairs):
        a = 0.02 * (t + 1)
        v, dv = a * np.exp(-knots / 2), -0.5 * a * np.exp(-knots / 2)
        y0, y1, d0, d1 = v[:-1], v[1:], dv[:-1], dv[1:]
        tab[t, :, 0, 0] = y0
        tab[t, :, 1, 0] = d0
        tab[t, :, 2, 0] = (-3 * y0 - 2 * h * d0 + 3 * y1 - h * d1) / h ** 2
        tab[t, :, 3, 0] = (2 * y0 + h * d0 - 2 * y1 + h * d1) / h ** 3
    return tab


@pytest.mark.gpu
def test_r0_module_density_chain_matches_finite_differences(tiny_model_path):
    """E = sum_i adj_i . s_i Phi0_i with s_i = 1 / (1 + rho_i): the module's
    directed force of an edge, projected on its direction, equals -dE/dr_e
    (moving an edge along its direction keeps Y and dY fixed)."""
    from _hip import DeviceArray, hip
    s, om, ref = _oracle_run(tiny_model_path, 3)
    C, l_max = 32, 2
    NY = (l_max + 1) ** 2
    mod = opm.CodeObject(opm.compiled_module_path(opm.KIND_R0, C, l_max)[0])
    d = _r0_setup(tiny_model_path, s, om, ref, C, l_max)
    N, E = d["N"], d["E"]
    dens = DeviceArray(_density_table(d["n"], d["intervals"], d["h"], d["x0"]))
    density = opm.spline(dens.value, d["n"] * (d["n"] + 1) // 2, d["intervals"], 1, d["h"], d["x0"])
    rng = np.random.default_rng(5)
    adj = rng.normal(size=(N, NY, C)).astype(np.float32)
    r0 = ref["r"].astype(np.float64)

    def energy_terms(r):
        """per-receiver E_i of the scaled forward at edge lengths r (FP64 sums)"""
        d_r = DeviceArray(r)
        d_state = DeviceArray(np.zeros(N))
        d_out = DeviceArray(np.zeros((N, NY, C), np.float32))
        a = _r0_args(d, C, l_max, om.r_cut, radius=d_r.value, density=density, apply_density_scale=1,
                     density_state=d_state.value, output=d_out.value)
        assert mod.launch("symmetrix_r0_density_prepare_v1", a, N, 4) == 0
        assert mod.launch("symmetrix_r0_forward_v1", a, N * NY * C, 4) == 0
        assert hip().hipDeviceSynchronize() == 0
        return np.sum(adj.astype(np.float64) * d_out.get(), axis=(1, 2)), d_out.get(), d_state.get()

    _, out0, state0 = energy_terms(r0)
    # reverse: prepare (dot, adjoint scaling) then the coordinate reverse
    d_out = DeviceArray(out0)
    d_adj = DeviceArray(adj.copy())
    d_state = DeviceArray(state0)
    d_f = DeviceArray(np.zeros((E, 3)))
    a = _r0_args(d, C, l_max, om.r_cut, density=density, apply_density_scale=1, density_state=d_state.value,
                 output=d_out.value, output_adjoint=d_adj.value, directed_forces=d_f.value)
    assert mod.launch("symmetrix_r0_reverse_prepare_v1", a, N, 2) == 0
    assert mod.launch("symmetrix_r0_coordinate_reverse_v1", a, E, 6) == 0
    assert hip().hipDeviceSynchronize() == 0
    # prepare: adjoint scaled by s_i, state = s_i * sum(out * adj)
    np.testing.assert_allclose(d_adj.get(), adj * state0[:, None, None].astype(np.float32), rtol=1e-6)
    dot = np.sum(out0.astype(np.float64) * adj, axis=(1, 2))
    np.testing.assert_allclose(d_state.get(), dot * state0, rtol=1e-9, atol=1e-12)
    f = d_f.get()
    unit = ref["xyz"] / r0[:, None]
    recv = np.repeat(np.arange(N), np.diff(d["offsets"]))
    active = np.nonzero(r0 < om.r_cut - 0.01)[0]   # stays active under the perturbation
    picks = rng.choice(active, size=12, replace=False)
    delta = 2e-3
    for e in picks:
        i = recv[e]
        rp, rm = r0.copy(), r0.copy()
        rp[e] += delta
        rm[e] -= delta
        dE = (energy_terms(rp)[0][i] - energy_terms(rm)[0][i]) / (2 * delta)
        fd = -dE
        got = float(np.dot(f[e], unit[e]))
        print("edge %d: module %.6e, central difference %.6e" % (e, got, fd))
        assert abs(got - fd) <= 2e-2 * abs(fd) + 2e-3

    # precomputed scale adjoint: dot taken from the caller
    pre = DeviceArray(np.full(N, 0.5))
    d_state = DeviceArray(state0)
    d_adj = DeviceArray(adj.copy())
    a = _r0_args(d, C, l_max, om.r_cut, use_precomputed_scale_adjoint=1, precomputed_scale_adjoint=pre.value,
                 density_state=d_state.value, output=d_out.value, output_adjoint=d_adj.value)
    assert mod.launch("symmetrix_r0_reverse_prepare_v1", a, N, 3) == 0
    assert hip().hipDeviceSynchronize() == 0
    np.testing.assert_allclose(d_state.get(), 0.5 * state0, rtol=1e-12)
