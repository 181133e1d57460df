"""Writes model-file fixtures with the reference's own JSON writer,
symmetrix/test/compact_r1_model.py:8-189 (`foundation_r1_test_model`), which
the reference's tests use to build compact format-4 models without a
checkpoint (symmetrix/test/conftest.py:7, test_dual_layer_fixed_workspace.py:8,
pair_symmetrix/test/test_pair_symmetrix_kokkos_compact.py:122-125).

Run in the build container, where /root/reference exists; the reference file
is imported from there and never copied.  Only the models it writes are
committed (gzip-compressed JSON data), so the GPU box needs no reference.

Fixtures (tests/golden/compact_*.json.gz):
* compact_medium_m0: the MPA-0 medium R1 contract
  (jit_r1_mace_mpa0_medium_contract.json: 128 channels, l_max 3, L_max 1,
  10 paths, 86 terms) with the standard M0 contract (standard_m0_contract.json:
  422 monomials, two types), atomic numbers O and Ti;
* compact_medium_linear: the same R1 contract without an M0 contract (the
  writer then gives each M0 output one linear monomial), atomic numbers O, Ti
  and Sr, so the SrTiO3 systems run on it;
* compact_c4: the reference's four-channel fixture contract
  (jit_r1_fixture_c4_e3_l0_contract.json: l_max 0, L_max 0);
* compact_omat0_small, compact_mp0b2_large, compact_off23_small,
  compact_off23_large: the R1 contracts of the MACE-OMAT-0 small (128x0e
  hidden, 4 paths), MP-0b2 large (128x0e+128x1o+128x2e, 17 paths),
  MACE-OFF23 small (96x0e) and large (224x0e+224x1o+224x2e) checkpoints,
  atomic numbers O, Ti and Sr.
"""

import gzip
import importlib.util
import json
import os
import sys

REF = "/root/reference/symmetrix/test"
CONTRACTS = os.path.join(REF, "data", "execution_contracts")
HERE = os.path.dirname(os.path.abspath(__file__))

FIXTURES = {
    "compact_medium_m0": ("jit_r1_mace_mpa0_medium_contract.json", "standard_m0_contract.json", (8, 22)),
    "compact_medium_linear": ("jit_r1_mace_mpa0_medium_contract.json", None, (8, 22, 38)),
    "compact_c4": ("jit_r1_fixture_c4_e3_l0_contract.json", None, (1, 8)),
    "compact_omat0_small": ("jit_r1_mace_omat0_small_contract.json", None, (8, 22, 38)),
    "compact_mp0b2_large": ("jit_r1_mace_mp0b2_large_contract.json", None, (8, 22, 38)),
    "compact_off23_small": ("jit_r1_mace_off23_small_contract.json", None, (8, 22, 38)),
    "compact_off23_large": ("jit_r1_mace_off23_large_contract.json", None, (8, 22, 38)),
}


def _writer():
    spec = importlib.util.spec_from_file_location("compact_r1_model", os.path.join(REF, "compact_r1_model.py"))
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module.foundation_r1_test_model


def main():
    if not os.path.isdir(REF):
        sys.exit("the reference is not available at %s" % REF)
    write = _writer()
    for name, (r1, m0, numbers) in FIXTURES.items():
        with open(os.path.join(CONTRACTS, r1)) as f:
            contract = json.load(f)
        m0_contract = None
        if m0 is not None:
            with open(os.path.join(CONTRACTS, m0)) as f:
                m0_contract = json.load(f)
        model = write(contract, atomic_numbers=numbers, m0_contract=m0_contract)
        text = json.dumps(model, separators=(",", ":"))
        path = os.path.join(HERE, name + ".json.gz")
        # mtime 0 keeps the compressed bytes reproducible
        with open(path, "wb") as raw, gzip.GzipFile(fileobj=raw, mode="wb", mtime=0) as f:
            f.write(text.encode())
        print("wrote %s (%d bytes of JSON, %d compressed)" % (path, len(text), os.path.getsize(path)))


if __name__ == "__main__":
    main()
