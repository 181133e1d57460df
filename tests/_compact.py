"""Shared helpers of the tests that run the reference-written model fixtures
(tests/golden/compact_*.json.gz, written by the reference's
symmetrix/test/compact_r1_model.py through tests/golden/make_compact_models.py)."""

import gzip
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODEL_DIR = os.environ.get("SYMMETRIX_MODEL_CACHE", "/tmp/symmetrix_models")

# atomic numbers of each fixture, by the SrTiO3 site (Sr, Ti, O) they stand on
SPECIES = {
    "compact_medium_m0": {38: 22, 22: 22, 8: 8},
    "compact_medium_linear": {38: 38, 22: 22, 8: 8},
    "compact_c4": {38: 1, 22: 8, 8: 8},
    "compact_omat0_small": {38: 38, 22: 22, 8: 8},
    "compact_mp0b2_large": {38: 38, 22: 22, 8: 8},
    "compact_off23_small": {38: 38, 22: 22, 8: 8},
    "compact_off23_large": {38: 38, 22: 22, 8: 8},
}


def compact_model(name):
    """Path of the decompressed fixture (written once per content), and its JSON."""
    os.makedirs(MODEL_DIR, exist_ok=True)
    path = os.path.join(MODEL_DIR, name + ".json")
    with gzip.open(os.path.join(GOLDEN, name + ".json.gz")) as f:
        data = f.read()
    if not os.path.exists(path) or open(path, "rb").read() != data:
        tmp = "%s.%d.tmp" % (path, os.getpid())
        with open(tmp, "wb") as f:
            f.write(data)
        os.replace(tmp, path)
    return path, json.loads(data)


def fixture_system(name, cells=2, seed=3, sigma=0.08):
    """A perturbed SrTiO3 supercell with the fixture's species on its sites."""
    from symmetrix import systems
    s = systems.srtio3_supercell(cells, sigma=sigma, seed=seed)
    s["numbers"] = np.array([SPECIES[name][int(z)] for z in s["numbers"]])
    return s
