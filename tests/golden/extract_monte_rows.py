"""Writes monte_rows.json from the reference's committed Monte rows
(experiments/dot-product-scaling/results/monte.jsonl): per distribution and
K, the 'acc' statistics of rep 0 and the per-rep-count averages, as printed.
Run in a tree that has /root/reference; the tests read only the JSON."""
import json
import os
import sys

SRC = "/root/reference/experiments/dot-product-scaling/results/monte.jsonl"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "monte_rows.json")

if __name__ == "__main__":
    src = sys.argv[1] if len(sys.argv) > 1 else SRC
    rows = []
    for line in open(src):
        d = json.loads(line)
        rows.append({"dist": d["dist"], "K": d["K"], "outputs": d["outputs"], "acc": d["acc"], "avg": d["avg"]})
    json.dump({"_source": "experiments/dot-product-scaling/results/monte.jsonl (the reference's committed rows: "
                          "dot-bench.cpp synth --reps 32 --outputs 2048 on LNSCUDA16 monte, run.py:98-105, with "
                          "the post-merge libraries of experiments/README.md:28-37); 'acc' of rep 0 and the "
                          "averages over the first 1, 2, 4, ... 32 reps, as printed",
               "rows": rows}, open(OUT, "w"), indent=0)
    print("wrote %d rows to %s" % (len(rows), OUT))
