"""MH-1 loader and C-ABI host logic on the CPU (the evaluator parses and
checks a file, and checks a call's graph, before any device work).

Reference behaviour mirrored: the family facts and rejection reasons of
analyze_mh1_family_architecture (mace_nonlinear_schema.cpp:108-207; pybind
mace_nonlinear_kokkos.cpp:26-45), refusal of malformed nonlinear JSON and of
inconsistent species mappings before evaluation (test_mh1.py:1324-1383), and
the graph checks of compute_node_energies_forces (mace_nonlinear.cpp:475-521).
"""

import copy
import json

import numpy as np
import pytest

from symmetrix import random_mh1
from symmetrix._native import SymmetrixUnsupportedError
from symmetrix.mace_nonlinear import MACENonlinearKokkosFloat, is_nonlinear_model


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("mh1load"))
    return {n: random_mh1.cached_mh1(n, directory=d) for n in ("mh1_tiny", "mh1_tiny_l2e", "mh1_medium")}


@pytest.fixture(scope="module")
def tiny_doc(models):
    with open(models["mh1_tiny"]) as f:
        return json.load(f)


def _write(tmp_path, doc, name="m.json"):
    p = tmp_path / name
    p.write_text(json.dumps(doc))
    return str(p)


def test_family_facts_and_rejection(models):
    ev = MACENonlinearKokkosFloat(models["mh1_medium"])
    assert ev.is_mh1_family and ev.mh1_family_rejection_reason == ""
    assert (ev.mh1_node_channels, ev.mh1_edge_channels, ev.mh1_radial_size, ev.mh1_l_max) == (64, 32, 8, 3)
    assert ev.r_cut == 6.0 and ev.num_interactions == 2 and not ev.has_zbl
    tiny = MACENonlinearKokkosFloat(models["mh1_tiny"])
    assert tiny.is_mh1_family and (tiny.mh1_node_channels, tiny.mh1_edge_channels, tiny.mh1_l_max) == (16, 8, 2)
    other = MACENonlinearKokkosFloat(models["mh1_tiny_l2e"])
    assert not other.is_mh1_family
    assert other.mh1_family_rejection_reason == "MH-1 node, edge and hidden irreps do not chain"
    assert (other.mh1_node_channels, other.mh1_l_max) == (0, 0)


def test_model_type_dispatch(models, tmp_path):
    assert is_nonlinear_model(models["mh1_tiny"])
    p = tmp_path / "plain.json"
    p.write_text(json.dumps({"model_type": "MACE", "symmetrix_format_version": 4}))
    assert not is_nonlinear_model(str(p))


def _mutate(doc, path, value):
    d = copy.deepcopy(doc)
    node = d
    for k in path[:-1]:
        node = node[k]
    node[path[-1]] = value
    return d


BAD = [
    (("symmetrix_format_version",), 2, "format version"),
    (("model_indices",), [0, 1, 3, 2], "model_indices"),
    (("atomic_numbers",), [1, 6, 8, 8], "element lists"),
    (("node_embedding", "irreps_out"), "16y0e", "irreps"),
    (("interactions", 0, "linear_up", "weight", "values"), [0.0, 1.0], "linear weight"),
    (("interactions", 0, "gate", "scalar_activation"), "tanh", "gate activations"),
    (("interactions", 0, "class"), "RealAgnosticInteractionBlock", "interaction class"),
    (("interactions", 1, "conv_tp", "instructions", 1, "wigner_3j", "shape"), [1, 1, 1], "Wigner 3j"),
    (("interactions", 1, "conv_tp", "instructions", 0, "connection_mode"), "uvw", "uvu"),
    (("interactions", 0, "conv_tp_weights", "layers", 3, "weight", "shape"), [16, 17], "MLP"),
    (("products", 0, "symmetric_contractions", "contractions", 0, "correlation"), 4, "correlation"),
    (("readouts", 1, "activation"), "tanh", "SiLU"),
    (("radial_embedding", "basis", "type"), "chebyshev", "Bessel"),
    (("radial_embedding", "distance_transform", "type"), "soft", "distance transform"),
    (("scale_shift", "scale"), {"shape": [2], "values": [1.0, 2.0]}, "single numbers"),
]


@pytest.mark.parametrize("path,value,message", BAD, ids=[m for _, _, m in BAD])
def test_malformed_files_are_refused(tiny_doc, tmp_path, path, value, message):
    with pytest.raises(ValueError, match=message):
        MACENonlinearKokkosFloat(_write(tmp_path, _mutate(tiny_doc, path, value)))


def test_shapes_without_a_kernel_are_unsupported(tmp_path):
    cfg = random_mh1.MH1Config("mh1_e12", node_channels=8, edge_channels=12)
    path = random_mh1.write_mh1(cfg, str(tmp_path / "e12.json"))
    with pytest.raises(SymmetrixUnsupportedError, match="power of two"):
        MACENonlinearKokkosFloat(path)


def test_head_selection(models, tiny_doc, tmp_path):
    ev = MACENonlinearKokkosFloat(models["mh1_tiny"])
    assert ev.selected_head == "" and ev.available_heads == []
    named = _write(tmp_path, _mutate(tiny_doc, ("head",), "omat_pbe"))
    ev = MACENonlinearKokkosFloat(named, "omat_pbe")
    assert ev.selected_head == "omat_pbe" and ev.available_heads == ["omat_pbe"]
    with pytest.raises(ValueError, match="holds head 'omat_pbe'"):
        MACENonlinearKokkosFloat(named, "spice")


def test_atomic_facts_follow_the_species_mapping(tiny_doc, tmp_path):
    d = copy.deepcopy(tiny_doc)
    # local types reorder the model's elements: energies follow model_indices
    d["atomic_numbers"] = [14, 1, 8, 6]
    d["model_indices"] = [3, 0, 2, 1]
    ev = MACENonlinearKokkosFloat(_write(tmp_path, d))
    ae = tiny_doc["atomic_energies"]["values"]
    assert ev.atomic_numbers == [14, 1, 8, 6]
    assert np.allclose(ev.atomic_energies, [ae[3], ae[0], ae[2], ae[1]])


def test_graph_checks_precede_device_work(models):
    ev = MACENonlinearKokkosFloat(models["mh1_tiny"])
    t = np.array([0, 1], dtype=np.int32)
    xyz = np.array([[1.0, 0.0, 0.0], [-1.0, 0.0, 0.0]])
    ok = dict(num_nodes=2, node_types=t, num_neigh=[1, 1], neigh_indices=[1, 0], neigh_types=[1, 0], xyz=xyz,
              r=np.ones(2))
    for bad, msg in ((dict(neigh_types=[0, 0]), "wrong type"), (dict(neigh_indices=[2, 0]), "out of range"),
                     (dict(num_neigh=[2, 1]), "do not sum"), (dict(r=np.array([1.0, np.inf])), "finite"),
                     (dict(node_types=np.array([0, 9], np.int32)), "node type"),
                     (dict(num_neigh=[1, -1]), "negative")):
        args = dict(ok)
        args.update(bad)
        with pytest.raises(ValueError, match=msg):
            ev.compute_node_energies_forces(**args)
