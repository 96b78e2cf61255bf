"""Writes tests/golden/c1_ref.npz: the REFERENCE's greedy decode on the
full-size C1 workload.

  * model = synthetic Llama-3.2-1B-shape model, every linear weight Q8_0
    (bin/synth_gguf c1: 16 layers, d_model 2048, 32 q / 8 kv heads, head_dim
    64, FFN 8192, vocab 128256, rope_theta 500000, tied head); its SHA-256 is
    stored so a test can prove it regenerated the same file;
  * prompt = 32 uniform-random ids, numpy default_rng(1234) (bench.py's);
  * greedy: Model::forward decode of 128 tokens after prefilling 31, context
    512 (benchmark/bench_engine.cpp:226-243 protocol, via oracle/_ref/ref_driver);
  * logits of the first 4 decode steps, stored as every 8th entry plus the 64
    largest (index, value) pairs of each step (the whole rows are 2 MB).

The reference is compiled from its own sources by oracle/Makefile (make ref).
Run: python tests/golden/make_golden_c1.py   (in the container that holds
/root/reference; about a minute on 8 cores)
"""
import hashlib
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
SYNTH = os.path.join(ROOT, "oracle-engine_amd", "bin", "synth_gguf")
DRV = os.path.join(ROOT, "oracle", "_ref", "ref_driver")
N_PROMPT, N_GEN, N_LOGIT_STEPS, V, STRIDE, TOP = 32, 128, 4, 128256, 8, 64


def sha(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def main():
    tmp = tempfile.mkdtemp(prefix="orc_c1_")
    path = os.path.join(tmp, "c1.gguf")
    subprocess.run([SYNTH, "c1", path], check=True)
    prompt = np.random.default_rng(1234).integers(0, V, N_PROMPT).astype(np.int32)
    pf, tf, lf = (os.path.join(tmp, n) for n in ("prompt.bin", "tokens.bin", "logits.bin"))
    prompt.tofile(pf)
    subprocess.run([DRV, "greedy", path, pf, str(N_GEN), tf, lf, str(N_LOGIT_STEPS)], check=True)
    lg = np.fromfile(lf, np.float32).reshape(N_LOGIT_STEPS, V)
    top = np.argsort(-lg, axis=1, kind="stable")[:, :TOP].astype(np.int32)
    out = {
        "prompt": prompt,
        "greedy_tokens": np.fromfile(tf, np.int32),
        "logits_strided": np.ascontiguousarray(lg[:, ::STRIDE]),
        "logits_stride": np.array([STRIDE], np.int32),
        "logits_top_idx": top,
        "logits_top_val": np.take_along_axis(lg, top, axis=1),
        "logits_absmax": np.abs(lg).max(axis=1),
        "sha/c1": np.frombuffer(sha(path).encode(), np.uint8),
    }
    dst = os.path.join(HERE, "c1_ref.npz")
    np.savez_compressed(dst, **out)
    os.remove(path)
    print(f"wrote {dst}: {out['greedy_tokens'][:8]} ...")


if __name__ == "__main__":
    sys.exit(main())
