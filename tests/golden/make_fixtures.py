"""Writes the golden fixtures of the reference's own test data that pin the
model structure (run in the build container, where /root/reference exists):

* r1_coupling.json: the R1 sparse coupling (paths; terms with coefficient,
  lm1, lm2, lme, row) of the reference's execution-contract fixtures
  symmetrix/test/data/execution_contracts/jit_r1_*_contract.json;
* m0_monomials.json: the product-basis monomial groups of
  symmetrix/test/data/execution_contracts/standard_m0_contract.json.

Only data is copied (the JSON fields the tests compare), not source.
"""

import json
import os
import sys

REF = "/root/reference/symmetrix/test/data/execution_contracts"
HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    if not os.path.isdir(REF):
        sys.exit("reference fixtures are not available at %s" % REF)
    r1 = {}
    for name in sorted(os.listdir(REF)):
        if not (name.startswith("jit_r1_") and name.endswith("_contract.json")):
            continue
        with open(os.path.join(REF, name)) as f:
            j = json.load(f)
        if "sparse_coupling" not in j or "paths" not in j:
            continue
        r1[name] = {
            "source": "symmetrix/test/data/execution_contracts/" + name,
            "edge_l_max": j["edge_harmonics"]["l_max"],
            "source_l_max": j["source_harmonics"]["l_max"],
            "channels": j["channels"],
            "paths": [[p["edge_l"], p["source_l"], p["output_l"]] for p in j["paths"]],
            "terms": [[t["lm1"], t["lm2"], t["lme"], t["row"], t["coefficient"]]
                      for t in j["sparse_coupling"]["terms"]],
        }
    with open(os.path.join(HERE, "r1_coupling.json"), "w") as f:
        json.dump(r1, f, indent=0, sort_keys=True)
    with open(os.path.join(REF, "standard_m0_contract.json")) as f:
        m0 = json.load(f)
    out = {"source": "symmetrix/test/data/execution_contracts/standard_m0_contract.json",
           "input_l_max": m0["input_l_max"], "output_l_max": m0["output_l_max"],
           "correlation": m0["correlation"],
           "groups": [{"output_component": g["output_component"], "term_count": g["term_count"],
                       "degree_counts": g["degree_counts"], "terms": g["terms"]}
                      for g in m0["monomial_groups"]]}
    with open(os.path.join(HERE, "m0_monomials.json"), "w") as f:
        json.dump(out, f, indent=0)
    print("wrote", len(r1), "R1 contracts and", len(out["groups"]), "M0 groups")


if __name__ == "__main__":
    main()
