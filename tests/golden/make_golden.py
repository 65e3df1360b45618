"""Write the golden fixtures of this directory from the reference's result files.

    python tests/golden/make_golden.py [/root/reference]

Reads data only (JSON results the reference committed); imports and runs
nothing from the reference.

  plan_balanced.json             results/plan_balanced.json (owners per layer/expert):
                                 the reference's plan_balanced() output for the
                                 counts below, world 4, 2 slots (scripts/make_plan.py:24-29)
  route_counts_bench_naive.json  per-(layer, expert) routing counts of
                                 results/bench_naive.json summed over the 4 ranks
                                 (the input of scripts/make_plan.py:26)
"""
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent


def main(ref_root: str = "/root/reference") -> None:
    res = Path(ref_root) / "results"
    plan = json.loads((res / "plan_balanced.json").read_text())
    (HERE / "plan_balanced.json").write_text(json.dumps(plan, sort_keys=True) + "\n")
    bench = json.loads((res / "bench_naive.json").read_text())
    ranks = bench["ranks"]
    n_l = len(ranks[0]["stats"]["route_counts"])
    n_e = len(ranks[0]["stats"]["route_counts"][0])
    counts = [[sum(r["stats"]["route_counts"][l][e] for r in ranks) for e in range(n_e)]
              for l in range(n_l)]
    out = {"world": bench["world"], "slots_per_rank": 2, "target_ratio": 1.05,
           "source": "results/bench_naive.json ranks[*].stats.route_counts, summed", "counts": counts}
    (HERE / "route_counts_bench_naive.json").write_text(json.dumps(out) + "\n")
    print("wrote", HERE / "plan_balanced.json", HERE / "route_counts_bench_naive.json")


if __name__ == "__main__":
    main(*sys.argv[1:])
