"""Writes tests/golden/planner_traces.json from the reference slot planner.

Run in the build container after `make -C oracle ref`, which compiles the
reference's native/locali_core.c unchanged into oracle/_ref/. Every workload in
planner_traces.all_cases() is replayed through that library; small cases keep
their full per-operation records, the two bounded-arena-shaped cases keep a
sha256 digest of them.
"""

import ctypes
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import planner_traces as pt  # noqa: E402

LIB = HERE.parents[1] / "oracle" / "_ref" / "liblocali_core_ref.so"


def main():
    lib = pt.bind(ctypes.CDLL(str(LIB)))
    out = {"source": "reference native/locali_core.c compiled by oracle/Makefile",
           "probe": pt.PROBE, "cases": []}
    for name, cap, slots, prot, pol, ops, keep in pt.all_cases():
        planner = pt.CPlanner(lib, cap, slots, prot, pol)
        records = pt.resolve_and_run(planner, ops, pt.PROBE, cap)
        planner.close()
        case = {"name": name, "key_capacity": cap, "slots": slots,
                "protected": prot, "policy": pol, "n_ops": len(ops),
                "digest": pt.digest(records)}
        if keep:
            case["records"] = records
        out["cases"].append(case)
        print(name, len(ops), case["digest"][:12])
    (HERE / "planner_traces.json").write_text(json.dumps(out, separators=(",", ":")))


if __name__ == "__main__":
    main()
