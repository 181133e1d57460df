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


@pytest.mark.gpu
def test_plugin_launchers_match_oracle_r1_stages(tiny_model_path):
    from _hip import DeviceArray, hip
    from oracle import oracle
    from symmetrix import systems

    s = systems.srtio3_supercell(3, sigma=0.05, seed=0)
    om = oracle.OracleModel(tiny_model_path)
    ref = oracle.evaluate_system(om, s, skin=0.5)
    g = ref["graph"]
    d = r1_plugin.configure(tiny_model_path, artifact_id="tiny-test", contract_fingerprint="fp-tiny",
                            embedding=8)
    assert d.capabilities & (r1_plugin.FORWARD | r1_plugin.COORDINATE_REVERSE) == 3
    assert d.abi_tag == r1_plugin.ABI_TAG and d.channels == om.num_channels
    assert d.contract_fingerprint == b"fp-tiny" and d.target_architecture == b"gfx950"

    N = len(s["numbers"])
    E = len(g["sources"])
    C = om.num_channels
    types = om.types_of(s["numbers"]).astype(np.int32)
    ntypes = int(types.max()) + 1
    table, h, x0 = r1_plugin.spline_table()
    pairs = ntypes * (ntypes + 1) // 2
    coef = DeviceArray(np.repeat(table, pairs, axis=0))   # same tabulation for every pair type
    radial = r1_plugin.RadialSpline(ctypes.sizeof(r1_plugin.RadialSpline), pairs, table.shape[1], table.shape[3],
                                    h, x0, coef.value)
    offsets = g["offsets"].astype(np.int32)
    sources = g["sources"].astype(np.int32)
    receivers = np.repeat(np.arange(N, dtype=np.int32), np.diff(offsets))
    d_types = DeviceArray(types)
    d_num = DeviceArray(np.diff(offsets).astype(np.int32))
    d_first = DeviceArray(offsets[:-1].copy())
    d_src = DeviceArray(sources)
    d_ntypes = DeviceArray(types[sources])
    d_map = DeviceArray(np.arange(ntypes, dtype=np.int32))
    d_r = DeviceArray(ref["r"].astype(np.float64))
    d_xyz = DeviceArray(ref["xyz"].astype(np.float64))
    d_Y = DeviceArray(om.stage("Y").astype(np.float32))
    d_G = DeviceArray(om.stage("Ygrad").astype(np.float32))
    d_H1 = DeviceArray(om.stage("H1").astype(np.float32))
    phi_ref = om.stage("Phi1")
    d_out = DeviceArray(np.full(phi_ref.shape, np.nan, np.float32))
    cutoff = om.r_cut

    fa = r1_plugin.ForwardArgs(ctypes.sizeof(r1_plugin.ForwardArgs), ntypes, N, E, d_types.value, d_num.value,
                               d_first.value, d_src.value, d_ntypes.value, d_map.value, d_r.value, radial,
                               d_Y.value, d_H1.value, d_out.value, cutoff)
    assert d.r1_forward_launch(ctypes.byref(fa), None, 1) == 0
    assert hip().hipDeviceSynchronize() == 0
    phi = d_out.get().astype(np.float64)
    err = np.max(np.abs(phi - phi_ref)) / np.max(np.abs(phi_ref))
    print("plugin forward Phi1 relative max err %.3e" % err)
    assert err < 1e-5

    # coordinate reverse with the oracle's dPhi1 as the output adjoint
    order = np.argsort(sources, kind="stable")
    soff = np.zeros(N + 1, np.int32)
    np.cumsum(np.bincount(sources, minlength=N), out=soff[1:])
    d_soff = DeviceArray(soff)
    d_sedges = DeviceArray(order.astype(np.int32))
    d_recv = DeviceArray(receivers)
    d_dphi = DeviceArray(om.stage("dPhi1").astype(np.float32))
    h1adj_ref = om.stage("H1_adj")
    base_adj = np.full(h1adj_ref.shape, 0.25, np.float32)   # the launcher adds to what is there
    d_adj = DeviceArray(base_adj)
    base_f = np.full((E, 3), -0.5, np.float64)                # and subtracts its forces
    d_f = DeviceArray(base_f)
    sa = r1_plugin.SourceArgs(ctypes.sizeof(r1_plugin.SourceArgs), ntypes, N, E, d_types.value, d_ntypes.value,
                              d_soff.value, d_sedges.value, d_recv.value, d_map.value, d_r.value, radial,
                              d_Y.value, d_dphi.value, d_adj.value, cutoff)
    ea = r1_plugin.EdgeArgs(ctypes.sizeof(r1_plugin.EdgeArgs), ntypes, 8, 0, N, E, d_types.value, d_src.value,
                            d_ntypes.value, d_recv.value, d_map.value, d_xyz.value, d_r.value, radial, d_Y.value,
                            d_G.value, d_H1.value, d_dphi.value, d_f.value, cutoff)
    assert d.r1_coordinate_reverse_launch(ctypes.byref(sa), ctypes.byref(ea), None, 1) == 0
    assert hip().hipDeviceSynchronize() == 0
    adj = d_adj.get().astype(np.float64) - 0.25
    err = np.max(np.abs(adj - h1adj_ref)) / np.max(np.abs(h1adj_ref))
    print("plugin source adjoint relative max err %.3e" % err)
    assert err < 1e-5
    f = d_f.get() - base_f
    f_ref = om.stage("node_forces_r1").reshape(E, 3)
    ferr = np.max(np.abs(f - f_ref))
    print("plugin R1 directed forces max abs err %.3e (scale %.3e)" % (ferr, np.max(np.abs(f_ref))))
    assert ferr < 1e-5

    # malformed packets are rejected without launching
    bad = r1_plugin.ForwardArgs.from_buffer_copy(fa)
    bad.struct_size = 8
    assert d.r1_forward_launch(ctypes.byref(bad), None, 1) != 0
    assert d.r1_forward_launch(ctypes.byref(fa), None, 0) != 0
