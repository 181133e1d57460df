"""The allocation-free R1 reverse launch (smx_r1_plugin_reverse_launch_noalloc,
workspace in the library's fixed device scratch) against the plugin's own
coordinate reverse launcher on the same arguments: two calls in a row, the
second on a smaller graph, then a graph beyond the scratch, which is refused
before anything is launched."""

import ctypes

import numpy as np
import pytest

from symmetrix import _native, r1_plugin
from test_r1_plugin import _PluginCase

pytestmark = pytest.mark.gpu


def _noalloc(plugin_ptr):
    def launch(sa, ea, stream, blocks):
        return _native.lib.smx_r1_plugin_reverse_launch_noalloc(plugin_ptr, sa, ea, stream, blocks)
    return launch


def test_noalloc_reverse_matches_the_plugin_launcher(tiny_model_path):
    d = r1_plugin.configure(tiny_model_path, artifact_id="noalloc", contract_fingerprint="fp-noalloc", embedding=8)
    ptr = r1_plugin._query()
    for cells in (3, 2):   # the second call on a smaller graph reuses the scratch
        case = _PluginCase(tiny_model_path, cells=cells)
        print("noalloc reverse: %d nodes, %d edges" % (case.N, case.E), flush=True)
        radial = case.radial()
        adj_ref, f_ref = case.reverse(d, radial)
        adj, f = case.reverse(d, radial, launch=_noalloc(ptr))
        np.testing.assert_array_equal(adj, adj_ref)
        np.testing.assert_array_equal(f, f_ref)
        # and within the bar of the oracle's R1 stages
        h1 = case.om.stage("H1_adj")
        assert np.max(np.abs(adj - h1)) / np.max(np.abs(h1)) < 1e-5
        assert np.max(np.abs(f - case.om.stage("node_forces_r1").reshape(case.E, 3))) < 1e-5


def test_noalloc_reverse_refuses_graphs_beyond_the_scratch(tiny_model_path):
    r1_plugin.configure(tiny_model_path, artifact_id="noalloc-big", contract_fingerprint="fp", embedding=8)
    ptr = r1_plugin._query()
    case = _PluginCase(tiny_model_path, cells=2)
    radial = case.radial()
    sa = r1_plugin.SourceArgs(ctypes.sizeof(r1_plugin.SourceArgs), case.ntypes, case.N, 1 << 28,
                              case.d_types.value, case.d_ntypes.value, case.d_soff.value, case.d_sedges.value,
                              case.d_recv.value, case.d_map.value, case.d_r.value, radial, case.d_Y.value,
                              case.d_dphi.value, case.d_H1.value, case.cutoff)
    ea = r1_plugin.EdgeArgs(ctypes.sizeof(r1_plugin.EdgeArgs), case.ntypes, 8, 0, case.N, 1 << 28,
                            case.d_types.value, case.d_src.value, case.d_ntypes.value, case.d_recv.value,
                            case.d_map.value, case.d_xyz.value, case.d_r.value, radial, case.d_Y.value,
                            case.d_G.value, case.d_H1.value, case.d_dphi.value, case.d_xyz.value, case.cutoff)
    rc = _native.lib.smx_r1_plugin_reverse_launch_noalloc(ptr, ctypes.byref(sa), ctypes.byref(ea), None, 1)
    assert rc != 0
    assert b"fixed scratch" in _native.lib.smx_last_error()
    assert _native.lib.smx_r1_plugin_reverse_launch_noalloc(None, ctypes.byref(sa), ctypes.byref(ea), None, 1) != 0
