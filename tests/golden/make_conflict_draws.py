"""Writes tests/golden/conflict_draws.json from oracle/_ref, the reference's own
RNG header (src/nanorts/core/cuda/conflict_draw.cuh) compiled by oracle/Makefile.

Run from the repository root in a checkout where oracle/_ref builds:
    python3 tests/golden/make_conflict_draws.py
The vectors pin the oracle's threefry / fold_in / randint01 / CANCEL_RANDOM
draws where oracle/_ref is not available (the GPU box, a fresh clone).
"""
from __future__ import annotations

import ctypes
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as orc  # noqa: E402


def main() -> None:
    ref = orc.load_reference_draws()
    if ref is None:
        raise SystemExit("oracle/_ref is not built (needs the reference checkout)")
    ref.ref_conflict_draw.restype = ctypes.c_int32
    ref.ref_randint01.restype = ctypes.c_int32
    rng = np.random.default_rng(20260101)
    U2 = ctypes.c_uint32 * 2

    def key():
        return [int(v) for v in rng.integers(0, 2**32, 2, dtype=np.uint64)]

    out = {"source": "src/nanorts/core/cuda/conflict_draw.cuh via oracle/_ref", "fold_in": [], "randint01": [],
           "conflict_draw": [], "race": []}
    for _ in range(48):
        k, d = key(), int(rng.integers(-(2**31), 2**31))
        o = U2()
        ref.ref_fold_in(U2(*k), ctypes.c_int32(d), o)
        out["fold_in"].append({"key": k, "data": d, "out": [int(o[0]), int(o[1])]})
    for _ in range(48):
        k = key()
        out["randint01"].append({"key": k, "out": int(ref.ref_randint01(U2(*k)))})
    for _ in range(96):
        k = key()
        t, b, n = (int(v) for v in rng.integers(0, 6000, 3))
        n %= 8
        out["conflict_draw"].append({"root": k, "time": t, "birth": b, "ordinal": n,
                                     "out": int(ref.ref_conflict_draw(U2(*k), t, b, n))})
    # the two-worker race of the oracle tests: time 0, player 1's worker (birth 5), ordinal 0
    for _ in range(12):
        k = key()
        out["race"].append({"root": k, "out": int(ref.ref_conflict_draw(U2(*k), 0, 5, 0))})
    # Hand-traced rule tests (tests/test_oracle_rules.py), drawn from a
    # stream of their own so the vectors above stay as they were:
    #   "settle": one request with two same-cycle conflicts, the request's
    #     slot born 3, ordinals 0 and 1 at time 0;
    #   "race3": a three-unit race into one cell, the second and third
    #     requests born 6 and 7, ordinal 0 each at time 0.
    extra = np.random.default_rng(20261202)

    def extra_key():
        return [int(v) for v in extra.integers(0, 2**32, 2, dtype=np.uint64)]

    out["settle"] = []
    for _ in range(24):
        k = extra_key()
        out["settle"].append({"root": k, "time": 0, "birth": 3,
                              "out": [int(ref.ref_conflict_draw(U2(*k), 0, 3, n)) for n in (0, 1)]})
    out["race3"] = []
    for _ in range(24):
        k = extra_key()
        out["race3"].append({"root": k, "time": 0, "births": [6, 7],
                             "out": [int(ref.ref_conflict_draw(U2(*k), 0, b, 0)) for b in (6, 7)]})
    path = Path(__file__).with_name("conflict_draws.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
