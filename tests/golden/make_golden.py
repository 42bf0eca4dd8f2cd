#!/usr/bin/env python3
"""Copies the reference's committed numerics outputs (data, not code) into fixtures under tests/golden/.

Sources (relative to the reference checkout):
  docs/research/qmv-numerics-2026-10-10.txt      -> qmv_numerics.txt   (tests/qmv_numerics.cpp output)
  docs/research/error-budget-sm60-2026-10-10.txt -> error_budget_sm60.txt (tests/error_budget_sm60.cpp --long)
  docs/research/error-budget-split-2026-10-10.txt -> error_budget_split.txt (tests/error_budget_split.cpp --long)
Only the data rows are kept. Run here, where the reference checkout exists:
  python tests/golden/make_golden.py [/root/reference]
"""
import pathlib
import sys

REF = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = pathlib.Path(__file__).resolve().parent


def rows(src, keep):
    lines = (REF / src).read_text().splitlines()
    return [ln for ln in lines if keep(ln)]


def main():
    qmv = rows("docs/research/qmv-numerics-2026-10-10.txt",
               lambda ln: ln.split(" ")[0] in ("q4_0", "q8_0", "q4_K"))
    (OUT / "qmv_numerics.txt").write_text("\n".join(qmv) + "\n")
    eb = rows("docs/research/error-budget-sm60-2026-10-10.txt",
              lambda ln: ln.split(" ")[0] in ("PO", "L60", "L60o32", "C2", "C4", "C8") and len(ln.split()) == 10)
    (OUT / "error_budget_sm60.txt").write_text("\n".join(eb) + "\n")
    split = rows("docs/research/error-budget-split-2026-10-10.txt",
                 lambda ln: ln[:3] in ("600", "700") or ln.startswith("consistency"))
    (OUT / "error_budget_split.txt").write_text("\n".join(split) + "\n")
    print(f"qmv_numerics {len(qmv)} rows, error_budget_sm60 {len(eb)} rows, error_budget_split {len(split)} rows")


if __name__ == "__main__":
    main()
