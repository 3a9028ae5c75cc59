#!/usr/bin/env python3
"""Copy the exact mask scalars the reference's result files record into a fixture.

Sources (data, not code):
    results/results_bf16_512k_h200.csv, results/results_bf16_512k_a100pcie.csv
        one row per (T, d) of the published prefill sweep (chunk 128):
        q, B, N0, n, T_R, I_prof, I_tok, deg, plus the published prefill_ms
    results/theory_counting.csv    (T, d) at chunk 128: q, N0, B, deg, I_prof, I_tok
    results/theory_structure.csv   (T, d) at chunk 64: n, T_R, q, B, N0 and
                                   nnz / density of the materialised T x T mask

Run from the repository root:  python tests/golden/extract_reference_tables.py
"""
from __future__ import annotations

import csv
import json
import os

REF = "/root/reference/results"
HERE = os.path.dirname(os.path.abspath(__file__))


def _rows(name, keep, chunk):
    out = []
    with open(os.path.join(REF, name)) as f:
        for i, r in enumerate(csv.DictReader(f), start=2):
            row = {k: (int(float(r[k])) if k not in ("density", "prefill_ms")
                       else float(r[k])) for k in keep if r.get(k, "") != ""}
            row.update(source=f"results/{name}:{i}", chunk=chunk)
            out.append(row)
    return out


def main():
    prefill_keys = ["T", "d", "nb", "r", "q", "B", "N0", "n", "T_R", "I_prof",
                    "I_tok", "deg", "prefill_ms"]
    tables = {
        "prefill_h200": _rows("results_bf16_512k_h200.csv", prefill_keys, 128),
        "prefill_a100": _rows("results_bf16_512k_a100pcie.csv", prefill_keys, 128),
        "theory_counting": _rows("theory_counting.csv",
                                 ["T", "d", "q", "N0", "B", "deg", "I_prof",
                                  "I_tok"], 128),
        "theory_structure": _rows("theory_structure.csv",
                                  ["T", "d", "n", "T_R", "q", "B", "N0", "nnz",
                                   "density"], 64),
    }
    with open(os.path.join(HERE, "reference_tables.json"), "w") as f:
        json.dump(tables, f, indent=1)
    for k, v in tables.items():
        print(f"{k}: {len(v)} rows")


if __name__ == "__main__":
    main()
