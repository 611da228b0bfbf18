"""Regenerates k_sweep_analytic.csv: the analytic IOCost columns of the
reference's experiments/results/k_sweep.csv (hpcyhr/CATFuse), the only
committed numeric fixture of this path in the reference.  Data only; run in
a checkout that has the reference at REF_ROOT."""
import csv
import os
import sys

REF_ROOT = os.environ.get("REF_ROOT", "/root/reference")
SRC = os.path.join(REF_ROOT, "experiments", "results", "k_sweep.csv")
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "k_sweep_analytic.csv")
COLS = ["config", "impl", "T", "B", "Cin", "Cout", "H", "W", "K", "num_blocks",
        "analytic_x_load", "analytic_w_load", "analytic_z_io", "analytic_v_io",
        "analytic_spike_write", "analytic_intermediate_io", "analytic_total"]

if __name__ == "__main__":
    rows = list(csv.DictReader(open(SRC)))
    with open(OUT, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=COLS)
        w.writeheader()
        for r in rows:
            w.writerow({k: r[k].strip() for k in COLS})
    print(f"{len(rows)} rows -> {OUT}", file=sys.stderr)
