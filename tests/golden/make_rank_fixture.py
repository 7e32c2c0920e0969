"""Generate the head-wise K rank lists of the synthetic workloads (seed 0).

cfg2 (Llama-2-7B shape, 32 KV heads): ranks drawn uniformly from
{16, 32, 48, 64, 96}, rescaled so that the total is 40% of 4096 and rounded
to multiples of 8 (total 1640).
cfg4 (Llama-3.1-8B shape, 8 KV heads): ranks drawn uniformly from the
multiples of 16 in [32, 128].
Run: python tests/golden/make_rank_fixture.py
"""
import json
import os

import numpy as np


def cfg2(rng):
    r = rng.choice([16, 32, 48, 64, 96], size=32).astype(np.float64)
    r = np.clip(np.rint(r * (0.4 * 4096 / r.sum()) / 8) * 8, 8, 128).astype(int)
    target = 1640
    i = 0
    while r.sum() != target:
        h = i % 32
        if r.sum() < target and r[h] < 128:
            r[h] += 8
        elif r.sum() > target and r[h] > 8:
            r[h] -= 8
        i += 7
    return [int(v) for v in r]


def cfg4(rng):
    return [int(v) for v in rng.choice(np.arange(32, 129, 16), size=8)]


def main():
    rng = np.random.default_rng(0)
    out = {"cfg2_k_ranks": cfg2(rng), "cfg4_k_ranks": cfg4(rng)}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cfg_ranks.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(out, sum(out["cfg2_k_ranks"]))


if __name__ == "__main__":
    main()
