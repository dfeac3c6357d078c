"""Writes the committed golden fixtures of tests/golden/ from the CPU oracle.

c1_readme.json — BASELINE config 1 (the README-scale CPU case), in full:
  f32 logits [S=4, B=2, T=8, V=16] = 2 * N(0,1) from rng::derive(2024, "c1/logits") (Box-Muller,
  src/nn/init.rs:28-37), rounded to f32; u8 keep-mask, each token kept when a
  rng::derive(2024, "c1/mask") u32 word < 0.75 * 2^32, and token 0 kept where a row would have none;
  temperature 1.0; one uniform per row from rng::derive(2024, "c1/uniforms") (rl.rs:493-494).
  Expected: the inverse-CDF token, its log-probability and the entropy of each row (f64 oracle),
  and each draw's distance to the nearest CDF edge.

tiny_invcdf.json — the sampler on tiny rows (V <= 8) for every u on a 1e-3 grid.

Run: python tests/golden/make_golden.py  (rewrites the files; the tests check that the oracle
still reproduces them).
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", ".."))
from oracle import oracle as O  # noqa: E402

SEED = 2024


def c1_inputs():
    S, B, T, V = 4, 2, 8, 16
    rows = S * B * T
    r = O.Rng(SEED, "c1/logits")
    logits = (2.0 * r.normals(rows * V)).astype(np.float32).reshape(rows, V)
    rm = O.Rng(SEED, "c1/mask")
    words = np.array([rm.next_u32() for _ in range(rows * V)], dtype=np.uint64)
    keep = (words < int(0.75 * 2 ** 32)).astype(np.uint8).reshape(rows, V)
    for i in range(rows):
        if keep[i].sum() == 0:
            keep[i, 0] = 1
    u = O.Rng(SEED, "c1/uniforms").uniforms(rows)
    return (S, B, T, V), logits, keep, u


def c1_fixture():
    shape, logits, keep, u = c1_inputs()
    z = O.tempered(logits, 1.0, keep=keep)
    ids, edges = O.sample_invcdf(z, u)
    logp = O.token_logp(z, ids)
    ent = O.entropy(z)
    return {
        "what": "BASELINE config 1: f32 [4,2,8,16] ~ 2*N(0,1), u8 mask Bernoulli(0.75), T=1, one uniform per row",
        "shape": list(shape),
        "temperature": 1.0,
        "logits_f32_hex": [x.tobytes().hex() for x in logits],
        "keep_u8": keep.tolist(),
        "uniforms": [float(x) for x in u],
        "ids": ids.tolist(),
        "logp": [float(x) for x in logp],
        "entropy": [float(x) for x in ent],
        "edge_distance": [float(x) for x in edges],
    }


def tiny_fixture():
    cases = []
    rng = np.random.default_rng(7)
    for V in (1, 2, 3, 5, 8):
        for tau in (1.0, 0.7):
            x = rng.normal(0.0, 2.0, V).astype(np.float32)
            keep = np.ones(V, dtype=np.uint8)
            if V > 2:
                keep[rng.integers(0, V)] = 0
            z = O.tempered(x[None, :], tau, keep=keep[None, :])
            grid = (np.arange(1, 1000) / 1000.0).astype(np.float64)
            ids, _ = O.sample_invcdf(np.repeat(z, grid.size, axis=0), grid)
            cases.append({"V": V, "temperature": tau, "logits_f32_hex": x.tobytes().hex(),
                          "keep_u8": keep.tolist(), "ids_on_grid": ids.tolist()})
    return {"what": "inverse-CDF sampler on tiny rows for u = k/1000, k = 1..999", "cases": cases}


def main():
    with open(os.path.join(HERE, "c1_readme.json"), "w") as f:
        json.dump(c1_fixture(), f, indent=1)
    with open(os.path.join(HERE, "tiny_invcdf.json"), "w") as f:
        json.dump(tiny_fixture(), f)
    print("wrote", os.path.join(HERE, "c1_readme.json"), os.path.join(HERE, "tiny_invcdf.json"))


if __name__ == "__main__":
    main()
