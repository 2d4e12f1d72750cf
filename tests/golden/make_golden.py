"""Write tests/golden/golden.json from the compiled reference CPU core.

Run in a container that has the reference checkout (oracle/_ref is built by
`make -C oracle ref`).  Every entry records the pair count, the canonical
SHA-256 of the sorted (i, j, Sx, Sy, Sz) rows and the order-independent
multiset checksum, produced by the reference's own `neighbor_list_cpu`.
Inputs are regenerated from the seeded generators named in each entry, so
the fixture holds only data.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from tests.golden.cases import CASES  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.json")


def main() -> None:
    if not oracle.available("reference"):
        oracle.build(reference=True)
    results = {}
    for name, (make, options) in CASES.items():
        cfg = make()
        pairs, shifts = oracle.neighbor_pairs(
            cfg["positions"], cfg["cell"], cfg["pbc"], cfg["cutoff"], cfg["batch_ptr"],
            half_list=options.get("half_list", False),
            include_self=options.get("include_self", False),
            algorithm=options.get("algorithm", "auto"), threads=8, kind="reference",
        )
        entry = {
            "pairs": int(len(pairs)),
            "multiset": f"{oracle.multiset_hash(pairs, shifts):016x}",
        }
        if len(pairs) <= 20_000_000:
            entry["sha256"] = oracle.key_hash(pairs, shifts)
        if len(pairs) <= 64:
            entry["keys"] = oracle.canonical_keys(pairs, shifts).tolist()
        results[name] = entry
        print(name, entry["pairs"], flush=True)
    with open(OUT, "w") as fh:
        json.dump(results, fh, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
