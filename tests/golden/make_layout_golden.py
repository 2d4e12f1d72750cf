"""Write tests/golden/layout_limit.json from the compiled reference CPU core.

The reference's CPU path refuses an explicit cell_list when its dense bin
layout would hold more than 64 bins per atom image (or more than 2^26 bins)
(``csrc/core/neighbors_cpu.cpp:380-430``), with a search cutoff padded in
long double and rounded up to the input type (``neighbors_cpu.cpp:157-218``).
This script finds, for a few shapes whose layout grows with one length L
(non-periodic lines, a slab periodic in x and y whose padding comes from
wrapped atoms and images, and a sparse fully periodic box), the last L (to the ulp of the input type) that
the reference accepts, and records that L and its neighbours a few ulps either side with
the reference's outcome: the pair count, or "refused".  Inputs are written
as exact hexadecimal floats, so the fixture holds only data.

Run in a container that has the reference checkout (oracle/_ref is built by
``make -C oracle ref``):

    python tests/golden/make_layout_golden.py
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "layout_limit.json")


def shape(kind: str, L: float, dtype) -> dict:
    """Non-periodic structures whose bin layout grows with L."""
    if kind == "line2":
        # two atoms L apart on x: 4 * ceil(L / s + 2) bins, refused past 128
        pos = [[0.0, 0.0, 0.0], [L, 0.0, 0.0]]
        rc = 1.0
    elif kind == "line3":
        # three atoms up to L apart on x, one off-axis at 0.75 (a pair)
        pos = [[0.0, 0.0, 0.0], [L, 0.0, 0.0], [0.0, 0.75, 0.0]]
        rc = 1.0
    elif kind == "slab":
        # a skewed slab periodic in x and y (9 images) whose layout grows
        # with the z extent L; one atom far along x, wrapped by hundreds
        # (float32) or tens of thousands (float64) of cells, makes the x
        # component of the operation scale, with its image and wrap terms,
        # set the padding
        far = 1000.37 if np.dtype(dtype) == np.float32 else 123456.789
        pos = [[far, 0.5, 0.0], [0.25, 0.61, L], [-77.3, 2.9, 0.4]]
        cell = np.array([[[4.1, 0.3, 0.0], [0.2, 3.9, 0.0], [0.0, 0.0, 0.0]]], dtype=dtype)
        return {
            "positions": np.asarray(pos, dtype=dtype),
            "cell": cell,
            "pbc": np.array([[True, True, False]]),
            "batch_ptr": np.array([0, len(pos)], dtype=np.int64),
            "cutoff": 1.0,
        }
    elif kind == "box":
        # a fully periodic cubic cell of edge L (27 images) holding three
        # atoms, one of them wrapped by (1, -1, 2) cells, spread over the cell
        pos = [[0.1, 0.2, 0.3], [0.93 * L, 0.91 * L, 0.95 * L], [L + 0.3, -0.2, 2 * L + 0.5]]
        return {
            "positions": np.asarray(pos, dtype=dtype),
            "cell": (np.eye(3)[None] * L).astype(dtype),
            "pbc": np.ones((1, 3), dtype=bool),
            "batch_ptr": np.array([0, len(pos)], dtype=np.int64),
            "cutoff": 1.0,
        }
    else:  # "offset": the line of two atoms 1000 A from the origin
        pos = [[1000.0, -3.0, 2.0], [1000.0 + L, -3.0, 2.0]]
        rc = 1.5
    return {
        "positions": np.asarray(pos, dtype=dtype),
        "cell": np.zeros((1, 3, 3), dtype=dtype),
        "pbc": np.zeros((1, 3), dtype=bool),
        "batch_ptr": np.array([0, len(pos)], dtype=np.int64),
        "cutoff": rc,
    }


def outcome(cfg) -> int | None:
    """Pair count of the reference's explicit cell_list, None when refused."""
    try:
        pairs, _ = oracle.neighbor_pairs(cfg["positions"], cfg["cell"], cfg["pbc"], cfg["cutoff"],
                                         cfg["batch_ptr"], algorithm="cell_list", threads=1,
                                         kind="reference")
    except RuntimeError as error:
        assert "cannot safely process" in str(error), error
        return None
    return int(len(pairs))


def boundary(kind: str, dtype, lo: float, hi: float) -> float:
    """The last L in [lo, hi] (values of dtype) the reference accepts."""
    t = np.dtype(dtype).type
    lo, hi = t(lo), t(hi)
    assert outcome(shape(kind, float(lo), dtype)) is not None
    assert outcome(shape(kind, float(hi), dtype)) is None
    while np.nextafter(lo, hi) != hi:
        mid = t((float(lo) + float(hi)) / 2)
        if mid in (lo, hi):
            mid = np.nextafter(lo, hi)
        if outcome(shape(kind, float(mid), dtype)) is not None:
            lo = mid
        else:
            hi = mid
    return float(lo)


def main() -> None:
    if not oracle.available("reference"):
        oracle.build(reference=True)
    cases = []
    for kind, lo, hi in (("line2", 29.0, 31.0), ("line3", 28.0, 33.0), ("offset", 43.0, 47.0),
                         ("slab", 80.0, 120.0), ("box", 15.0, 16.0)):
        for dtype in (np.float32, np.float64):
            t = np.dtype(dtype).type
            last = t(boundary(kind, dtype, lo, hi))
            values = [last]
            up = down = last
            for _ in range(3):
                up = np.nextafter(up, t(np.inf))
                down = np.nextafter(down, t(-np.inf))
                values += [up, down]
            for L in sorted(values):
                cfg = shape(kind, float(L), dtype)
                result = outcome(cfg)
                cases.append({
                    "kind": kind,
                    "dtype": np.dtype(dtype).name,
                    "L": float(L).hex(),
                    "pairs": result,
                })
                print(kind, np.dtype(dtype).name, float(L), result, flush=True)
    with open(OUT, "w") as fh:
        json.dump(cases, fh, indent=1)


if __name__ == "__main__":
    main()
