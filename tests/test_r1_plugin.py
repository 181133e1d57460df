"""The reference's R1 HIP plugin ABI exported by libsymmetrix_mi355x.so
(symmetrix_jit_hip_plugin_query_v1, jit_hip_plugin_abi.h:28-269).

CPU: the descriptor and argument-packet layouts are pinned byte for byte
(sizes and offsets compiled from the reference's header in the build
container: plugin 144 B with r1_forward_launch at 128, forward and source
packets 152 B, edge packet 176 B with directed_forces at 160, radial spline
40 B), and the query returns NULL until a model is configured.

GPU: the launchers driven exactly as the reference evaluator drives them --
its separate per-edge arrays, spline table [edge type][interval][4][function],
type maps and receiver/source schedules -- against the CPU oracle's R1 stages
on the tiny system: Phi1 (forward), the source adjoint (H1 adjoint) and the
R1 part of the directed forces (coordinate reverse).
"""

import ctypes

import numpy as np
import pytest

from symmetrix import _native, r1_plugin


def test_abi_layouts_match_the_reference_header():
    P = r1_plugin
    assert ctypes.sizeof(P.RadialSpline) == 40
    assert ctypes.sizeof(P.ForwardArgs) == 152 and P.ForwardArgs.cutoff.offset == 144
    assert ctypes.sizeof(P.SourceArgs) == 152
    assert ctypes.sizeof(P.EdgeArgs) == 176 and P.EdgeArgs.directed_forces.offset == 160
    assert ctypes.sizeof(P.PluginV1) == 144 and P.PluginV1.r1_forward_launch.offset == 128


def test_query_is_null_until_configured_and_bad_model_is_rejected(tmp_path):
    lib = ctypes.CDLL(_native.LIB_PATH)
    assert hasattr(lib, "symmetrix_jit_hip_plugin_query_v1")
    assert r1_plugin.descriptor() is None
    ident = _native.SmxR1PluginIdentity(ctypes.sizeof(_native.SmxR1PluginIdentity), b"a", b"c", b"", b"", b"",
                                        8, 0, 4)
    rc = _native.lib.smx_r1_plugin_configure(str(tmp_path / "missing.json").encode(), ctypes.byref(ident))
    assert rc == _native.SMX_ERR_INVALID_ARGUMENT
    ident.embedding = 0
    rc = _native.lib.smx_r1_plugin_configure(b"whatever.json", ctypes.byref(ident))
    assert rc == _native.SMX_ERR_INVALID_ARGUMENT
    assert r1_plugin.descriptor() is None


class _PluginCase:
    """Device arrays of the tiny system in the reference's per-edge layout,
    with the oracle's R1 stages as inputs and references."""

    def __init__(self, model_path, cells=3, system=None):
        from _hip import DeviceArray
        from oracle import oracle
        from symmetrix import systems

        s = system if system is not None else systems.srtio3_supercell(cells, sigma=0.05, seed=0)
        om = oracle.OracleModel(model_path)
        ref = oracle.evaluate_system(om, s, skin=0.5)
        self.om, self.ref = om, ref
        g = ref["graph"]
        self.N = N = len(s["numbers"])
        self.E = E = len(g["sources"])
        self.C = om.num_channels
        types = om.types_of(s["numbers"]).astype(np.int32)
        # active types: the types present, numbered in order (type_to_active)
        active = np.unique(types)
        self.ntypes = len(active)
        tmap = np.full(int(types.max()) + 1, 0, np.int32)
        tmap[active] = np.arange(len(active), dtype=np.int32)
        self.offsets = offsets = g["offsets"].astype(np.int32)
        self.sources = sources = g["sources"].astype(np.int32)
        self.receivers = receivers = np.repeat(np.arange(N, dtype=np.int32), np.diff(offsets))
        self.d_types = DeviceArray(types)
        self.d_num = DeviceArray(np.diff(offsets).astype(np.int32))
        self.d_first = DeviceArray(offsets[:-1].copy())
        self.d_src = DeviceArray(sources)
        self.d_ntypes = DeviceArray(types[sources])
        self.d_map = DeviceArray(tmap)
        self.d_r = DeviceArray(ref["r"].astype(np.float64))
        self.d_xyz = DeviceArray(ref["xyz"].astype(np.float64))
        self.d_Y = DeviceArray(om.stage("Y").astype(np.float32))
        self.d_G = DeviceArray(om.stage("Ygrad").astype(np.float32))
        self.d_H1 = DeviceArray(om.stage("H1").astype(np.float32))
        self.d_dphi = DeviceArray(om.stage("dPhi1").astype(np.float32))
        order = np.argsort(sources, kind="stable")
        soff = np.zeros(N + 1, np.int32)
        np.cumsum(np.bincount(sources, minlength=N), out=soff[1:])
        self.d_soff = DeviceArray(soff)
        self.d_sedges = DeviceArray(order.astype(np.int32))
        self.d_recv = DeviceArray(receivers)
        self.cutoff = om.r_cut

    def radial(self):
        from _hip import DeviceArray
        table, h, x0 = r1_plugin.spline_table()
        pairs = self.ntypes * (self.ntypes + 1) // 2
        self._coef = DeviceArray(np.repeat(table, pairs, axis=0))   # same tabulation for every pair type
        return r1_plugin.RadialSpline(ctypes.sizeof(r1_plugin.RadialSpline), pairs, table.shape[1],
                                      table.shape[3], h, x0, self._coef.value)

    def forward(self, d, radial):
        from _hip import DeviceArray, hip
        out = DeviceArray(np.full(self.om.stage("Phi1").shape, np.nan, np.float32))
        fa = r1_plugin.ForwardArgs(ctypes.sizeof(r1_plugin.ForwardArgs), self.ntypes, self.N, self.E,
                                   self.d_types.value, self.d_num.value, self.d_first.value, self.d_src.value,
                                   self.d_ntypes.value, self.d_map.value, self.d_r.value, radial, self.d_Y.value,
                                   self.d_H1.value, out.value, self.cutoff)
        assert d.r1_forward_launch(ctypes.byref(fa), None, 1) == 0
        assert hip().hipDeviceSynchronize() == 0
        return out.get(), fa

    def reverse(self, d, radial, launch=None):
        """(source adjoint added to a quarter of its scale, forces subtracted
        from -0.5) of one reverse launch through d (or through `launch`, same
        arguments).  The base is scaled like the adjoint so that its FP32
        rounding stays below the comparison's bar."""
        from _hip import DeviceArray, hip
        ref = self.om.stage("H1_adj")
        base = np.float32(0.25 * max(np.max(np.abs(ref)), 1e-30))
        base_adj = np.full(ref.shape, base, np.float32)
        d_adj = DeviceArray(base_adj)
        base_f = np.full((self.E, 3), -0.5, np.float64)
        d_f = DeviceArray(base_f)
        sa = r1_plugin.SourceArgs(ctypes.sizeof(r1_plugin.SourceArgs), self.ntypes, self.N, self.E,
                                  self.d_types.value, self.d_ntypes.value, self.d_soff.value, self.d_sedges.value,
                                  self.d_recv.value, self.d_map.value, self.d_r.value, radial, self.d_Y.value,
                                  self.d_dphi.value, d_adj.value, self.cutoff)
        ea = r1_plugin.EdgeArgs(ctypes.sizeof(r1_plugin.EdgeArgs), self.ntypes, 8, 0, self.N, self.E,
                                self.d_types.value, self.d_src.value, self.d_ntypes.value, self.d_recv.value,
                                self.d_map.value, self.d_xyz.value, self.d_r.value, radial, self.d_Y.value,
                                self.d_G.value, self.d_H1.value, self.d_dphi.value, d_f.value, self.cutoff)
        rc = (launch or d.r1_coordinate_reverse_launch)(ctypes.byref(sa), ctypes.byref(ea), None, 1)
        assert rc == 0, rc
        assert hip().hipDeviceSynchronize() == 0
        return d_adj.get().astype(np.float64) - np.float64(base), d_f.get() - base_f


@pytest.mark.gpu
def test_plugin_launchers_match_oracle_r1_stages(tiny_model_path):
    case = _PluginCase(tiny_model_path)
    om = case.om
    d = r1_plugin.configure(tiny_model_path, artifact_id="tiny-test", contract_fingerprint="fp-tiny",
                            embedding=8)
    assert d.capabilities & (r1_plugin.FORWARD | r1_plugin.COORDINATE_REVERSE) == 3
    assert d.abi_tag == r1_plugin.ABI_TAG and d.channels == om.num_channels
    assert d.contract_fingerprint == b"fp-tiny" and d.target_architecture == b"gfx950"
    radial = case.radial()

    phi_ref = om.stage("Phi1")
    phi, fa = case.forward(d, radial)
    err = np.max(np.abs(phi.astype(np.float64) - phi_ref)) / np.max(np.abs(phi_ref))
    print("plugin forward Phi1 relative max err %.3e" % err)
    assert err < 1e-5

    # coordinate reverse with the oracle's dPhi1 as the output adjoint
    adj, f = case.reverse(d, radial)
    h1adj_ref = om.stage("H1_adj")
    err = np.max(np.abs(adj - h1adj_ref)) / np.max(np.abs(h1adj_ref))
    print("plugin source adjoint relative max err %.3e" % err)
    assert err < 1e-5
    f_ref = om.stage("node_forces_r1").reshape(case.E, 3)
    ferr = np.max(np.abs(f - f_ref))
    print("plugin R1 directed forces max abs err %.3e (scale %.3e)" % (ferr, np.max(np.abs(f_ref))))
    assert ferr < 1e-5

    # malformed packets are rejected without launching
    bad = r1_plugin.ForwardArgs.from_buffer_copy(fa)
    bad.struct_size = 8
    assert d.r1_forward_launch(ctypes.byref(bad), None, 1) != 0
    assert d.r1_forward_launch(ctypes.byref(fa), None, 0) != 0


@pytest.mark.gpu
def test_descriptor_keeps_its_model_after_another_configure(tiny_model_path, tmp_path):
    """A loader that holds the descriptor of model A keeps launching A after
    model B (same shape, coupling coefficients doubled) is configured; B's
    descriptor launches B.  The reverse workspace sized by
    smx_r1_plugin_reserve gives the same results as one grown by a launch."""
    import json
    case = _PluginCase(tiny_model_path)
    dA = r1_plugin.configure(tiny_model_path, artifact_id="model-a", contract_fingerprint="fp-a", embedding=8)
    pA = r1_plugin._query()
    radial = case.radial()
    phiA, _ = case.forward(dA, radial)
    adjA, fA = case.reverse(dA, radial)
    with open(tiny_model_path) as fh:
        j = json.load(fh)
    j["Phi1_clebsch_gordan"] = [2.0 * c for c in j["Phi1_clebsch_gordan"]]
    path_b = tmp_path / "tiny_double_cg.json"
    path_b.write_text(json.dumps(j))
    dB = r1_plugin.configure(str(path_b), artifact_id="model-b", contract_fingerprint="fp-b", embedding=8)
    assert r1_plugin.descriptor().artifact_id == b"model-b"
    phiA2, _ = case.forward(dA, radial)
    np.testing.assert_array_equal(phiA2, phiA)
    phiB, _ = case.forward(dB, radial)
    np.testing.assert_allclose(phiB, 2.0 * phiA, rtol=1e-6, atol=1e-7 * np.max(np.abs(phiA)))
    assert _native.lib.smx_r1_plugin_reserve(pA, case.N, case.E) == 0
    adjA2, fA2 = case.reverse(dA, radial)
    np.testing.assert_array_equal(adjA2, adjA)
    np.testing.assert_array_equal(fA2, fA)
    assert _native.lib.smx_r1_plugin_reserve(None, case.N, case.E) == _native.SMX_ERR_INVALID_ARGUMENT


def test_configure_reuses_a_slot_for_the_same_model_and_identity(tmp_path):
    """Configure is host work: the same model bytes and identity give back
    the same descriptor however often they are configured; distinct models
    take launcher slots up to the library's limit, after which configure is
    refused (run in a child process, whose slots are its own)."""
    import subprocess
    import sys
    import textwrap
    from symmetrix import random_model
    tiny = random_model.cached_model("tiny")
    script = textwrap.dedent("""
        import ctypes, json, shutil, sys
        sys.path[:0] = %r
        from symmetrix import _native, r1_plugin
        tiny, tmp = %r, %r
        first = r1_plugin._query
        d1 = r1_plugin.configure(tiny, artifact_id="same", contract_fingerprint="fp")
        p1 = ctypes.addressof(r1_plugin._query().contents)
        for _ in range(40):
            r1_plugin.configure(tiny, artifact_id="same", contract_fingerprint="fp")
            assert ctypes.addressof(r1_plugin._query().contents) == p1
        # a different identity of the same file takes a new slot
        r1_plugin.configure(tiny, artifact_id="other", contract_fingerprint="fp")
        assert ctypes.addressof(r1_plugin._query().contents) != p1
        # the same path with other bytes is another model
        j = json.load(open(tiny))
        j["Phi1_clebsch_gordan"] = [2.0 * c for c in j["Phi1_clebsch_gordan"]]
        path = tmp + "/changed.json"
        json.dump(j, open(path, "w"))
        r1_plugin.configure(path, artifact_id="same", contract_fingerprint="fp")
        json.dump(dict(j, Phi1_clebsch_gordan=[3.0 * c for c in j["Phi1_clebsch_gordan"]]), open(path, "w"))
        r1_plugin.configure(path, artifact_id="same", contract_fingerprint="fp")
        n = 4
        while True:
            ident = _native.SmxR1PluginIdentity(ctypes.sizeof(_native.SmxR1PluginIdentity),
                                                b"id-%%d" %% n, b"fp", b"", b"", b"", 8, 0, 4)
            rc = _native.lib.smx_r1_plugin_configure(tiny.encode(), ctypes.byref(ident))
            if rc != 0:
                break
            n += 1
        assert rc == _native.SMX_ERR_LOGIC and b"distinct R1 plugin models" in _native.lib.smx_last_error()
        # a configured identity still configures once the slots are full
        r1_plugin.configure(tiny, artifact_id="same", contract_fingerprint="fp")
        assert ctypes.addressof(r1_plugin._query().contents) == p1
        print("slots", n)
    """) % (sys.path, tiny, str(tmp_path))
    out = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "slots 16" in out.stdout, out.stdout


def _shape_case(name):
    """(model path, system) of each evaluator shape beyond the tiny one."""
    from _compact import compact_model, fixture_system
    from symmetrix import random_model, systems
    if name == "wide":
        return random_model.cached_model("wide"), systems.water_box(num_molecules=120, seed=2)
    path, _ = compact_model(name)
    return path, fixture_system(name, cells=2)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["wide", "compact_mp0b2_large", "compact_omat0_small", "compact_off23_small",
                                  "compact_off23_large"])
def test_plugin_serves_every_evaluator_shape(name):
    """The launchers of the (256,3,2) wide, (128,3,2) MP-0b2 large and
    (128,3,0) OMAT-0 small shapes, and of the OFF23 shapes whose 96 and 224
    channels run on 128 and 256 lanes over the caller's unpadded arrays,
    against the oracle's R1 stages (L_max 2: one pass per source-component
    group, as the evaluator runs them)."""
    path, system = _shape_case(name)
    print("plugin shape case", name, flush=True)
    case = _PluginCase(path, system=system)
    om = case.om
    d = r1_plugin.configure(path, artifact_id="shape-" + name, contract_fingerprint="fp-" + name, embedding=8)
    assert d.channels == om.num_channels
    radial = case.radial()
    phi_ref = om.stage("Phi1")
    phi, _ = case.forward(d, radial)
    err = np.max(np.abs(phi.astype(np.float64) - phi_ref)) / np.max(np.abs(phi_ref))
    print("%s: Phi1 relative max err %.3e" % (name, err))
    assert err < 1e-5
    adj, f = case.reverse(d, radial)
    h1adj_ref = om.stage("H1_adj")
    err = np.max(np.abs(adj - h1adj_ref)) / np.max(np.abs(h1adj_ref))
    print("%s: source adjoint relative max err %.3e" % (name, err))
    assert err < 1e-5
    f_ref = om.stage("node_forces_r1").reshape(case.E, 3)
    ferr = np.max(np.abs(f - f_ref)) / max(1.0, np.max(np.abs(f_ref)))
    print("%s: R1 directed forces max err %.3e (scale %.3e)" % (name, ferr, np.max(np.abs(f_ref))))
    assert ferr < 1e-5
