"""Writes tests/golden/transform_ref.npz from the REFERENCE Sampler: sequences of
draws (core/sampler.cpp:7-105; each draw recorded into the history, as
Sampler::sample does) over one logits row, for parameter sets with top_p < 1
and top_k in {0, 40}, with and without a repeat penalty.

tests/test_oracle.py checks each drawn id against the interval of the
oracle's orco_transform_probs (the p / q of the min(1, p/q) loop) that the
draw's uniform falls in, which pins the transform's kept set and its
probabilities to the reference's sampler.

Run: python tests/golden/make_golden_transform.py   (needs /root/reference, in this container)
"""
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(HERE))
from make_golden import run  # noqa: E402

CASES = [  # T, top_p, top_k, penalty, repeat_last, seed
    (0.8, 0.9, 40, 1.1, 64, 11),
    (0.8, 0.5, 0, 1.1, 64, 12),
    (1.2, 0.95, 0, 1.0, 64, 13),
    (0.7, 0.7, 40, 1.3, 16, 14),
    (1.0, 0.8, 0, 1.15, 32, 15),
]
N_DRAWS = 400


def main():
    tmp = tempfile.mkdtemp(prefix="orc_golden_tr_")
    w = lambda name: os.path.join(tmp, name)  # noqa: E731
    V = 3000
    # flat enough that the cut keeps dozens to hundreds of ids, so the draws
    # resolve the kept probabilities finely; the history's ids get a head start
    lg = np.random.default_rng(31).normal(0, 0.7, V).astype(np.float32)
    lg[:60] += 1.5
    hist = np.random.default_rng(32).integers(0, 60, 40).astype(np.int32)
    lg.tofile(w("lg.bin"))
    hist.tofile(w("h.bin"))
    out = {"logits": lg, "history": hist}
    for i, (T, P, K, pen, last, seed) in enumerate(CASES):
        run("sample", w("lg.bin"), T, P, K, pen, last, seed, w("h.bin"), N_DRAWS, w("d.bin"))
        out[f"case/{i}/params"] = np.array([T, P, K, pen, last], np.float64)
        out[f"case/{i}/seed"] = np.array([seed], np.uint64)
        out[f"case/{i}/draws"] = np.fromfile(w("d.bin"), np.int32)
    dst = os.path.join(HERE, "transform_ref.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst}: {len(out)} arrays, {os.path.getsize(dst) / 1e6:.3f} MB")


if __name__ == "__main__":
    main()
