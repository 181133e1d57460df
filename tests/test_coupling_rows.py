"""The table of live R1 coupling rows the kernels are compiled against
(csrc/coupling_rows.hpp) checked against the reference's own files.

A row (m1, m2) of a path (l_e, l_s, l_o) is live when some output m has a
nonzero coefficient.  The kernels hold only live rows, so the table must
contain every row that carries a term in the reference's R1 execution
contracts (symmetrix/test/data/execution_contracts/jit_r1_*_contract.json)
and in the models its writer produced; it is checked to be exactly the set
of rows those terms occupy, path by path, so a bit flipped either way fails.
"""

import gzip
import json
import os
import re

import pytest

from _compact import GOLDEN

HEADER = os.path.join(os.path.dirname(GOLDEN), "..", "symmetrix-xl_amd", "csrc", "coupling_rows.hpp")


def _table():
    with open(HEADER) as f:
        text = f.read()
    lmax = int(re.search(r"kCouplingLMax = (\d+);", text).group(1))
    body = text[text.index("kCouplingLive"):]
    body = body[body.index("= {"):body.index("};")]
    vals = [int(v, 16) for v in re.findall(r"0x([0-9a-f]+)ull", body)]
    n = lmax + 1
    assert len(vals) == n ** 3
    return lmax, {(le, ls, lo): vals[(le * n + ls) * n + lo]
                  for le in range(n) for ls in range(n) for lo in range(n)}


def _occupied(paths, terms):
    """rows with a nonzero term, per path: {(le, ls, lo): set of bits}"""
    base = [0]
    for le, ls, lo in paths:
        base.append(base[-1] + (2 * le + 1) * (2 * ls + 1))
    out = {tuple(p): 0 for p in paths}
    for lm1, lm2, _lme, row, coef in terms:
        q = max(i for i in range(len(paths)) if base[i] <= row)
        le, ls, lo = paths[q]
        m1, m2 = lm1 - le * le, lm2 - ls * ls
        assert row - base[q] == m1 * (2 * ls + 1) + m2
        if coef != 0.0:
            out[(le, ls, lo)] |= 1 << (m1 * (2 * ls + 1) + m2)
    return out


def _contracts():
    with open(os.path.join(GOLDEN, "r1_coupling.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("name", sorted(_contracts()))
def test_live_rows_are_the_rows_of_the_reference_contract_terms(name):
    lmax, table = _table()
    fx = _contracts()[name]
    for path, bits in _occupied([tuple(p) for p in fx["paths"]], fx["terms"]).items():
        assert max(path) <= lmax
        assert bits == table[path], (name, path)


@pytest.mark.parametrize("name", ["compact_medium_m0", "compact_mp0b2_large", "compact_off23_small"])
def test_reference_written_models_have_terms_only_in_live_rows(name):
    lmax, table = _table()
    with gzip.open(os.path.join(GOLDEN, name + ".json.gz"), "rt") as f:
        doc = json.load(f)
    paths = list(zip(doc["Phi1_l1"], doc["Phi1_l2"], doc["Phi1_l"]))
    # (lm1, lm2) from the row and its path; the lme index is not needed here
    base = [0]
    for le, ls, lo in paths:
        base.append(base[-1] + (2 * le + 1) * (2 * ls + 1))
    terms = []
    for row, coef in zip(doc["Phi1_lelm1lm2"], doc["Phi1_clebsch_gordan"]):
        q = max(i for i in range(len(paths)) if base[i] <= row)
        le, ls, _ = paths[q]
        local = row - base[q]
        terms.append((le * le + local // (2 * ls + 1), ls * ls + local % (2 * ls + 1), 0, row, coef))
    for path, bits in _occupied(paths, terms).items():
        assert bits == table[path], (name, path)


def test_header_is_what_its_generator_writes(tmp_path):
    import importlib.util
    gen = os.path.join(os.path.dirname(HEADER), "gen_coupling_rows.py")
    spec = importlib.util.spec_from_file_location("gen_coupling_rows", gen)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    # write into a scratch copy of the directory, then compare
    mod.HERE = str(tmp_path)
    mod.main()
    with open(HEADER) as f, open(tmp_path / "coupling_rows.hpp") as g:
        assert f.read() == g.read()
