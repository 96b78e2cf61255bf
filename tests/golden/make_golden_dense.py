"""Writes tests/golden/dense_ref.npz from the REFERENCE implementation on the
t-dense model (bin/synth_gguf t-dense): an F16 token embedding, a BF16 LM
head, an all-F32 layer 0 and a Q8_0 layer 1 whose attn_norm is declared F16
while its bytes are F32 norm weights.

The reference runs dense matrices through its dequantize + ops::matmul
fallback (core/model.cpp:370-381, gemv_q returning false) and reads norm
weights as raw F32 bytes whatever their declared type (core/model.cpp:317-320).
Stored: the model's SHA-256, greedy decode (40 tokens, the first 4 steps'
logits), 5-token verify logits (Model::forward_batch) and dequantize_row of
the F16, BF16 and F32 tensors.

Run: python tests/golden/make_golden_dense.py   (needs /root/reference, in this container)
"""
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)
import oracle_lib as ol  # noqa: E402
from make_golden import run, sha  # noqa: E402

SYNTH = os.path.join(ROOT, "oracle-engine_amd", "bin", "synth_gguf")


def main():
    tmp = tempfile.mkdtemp(prefix="orc_golden_dense_")
    w = lambda name: os.path.join(tmp, name)  # noqa: E731
    path = w("t-dense.gguf")
    subprocess.run([SYNTH, "t-dense", path], check=True, capture_output=True)
    out = {"sha/t-dense": np.frombuffer(sha(path).encode(), np.uint8)}
    prompt = np.random.default_rng(2026).integers(0, 2048, 16).astype(np.int32)
    prompt.tofile(w("p.bin"))
    run("greedy", path, w("p.bin"), 40, w("tok.bin"), w("lg.bin"), 4)
    out["greedy/prompt"] = prompt
    out["greedy/tokens"] = np.fromfile(w("tok.bin"), np.int32)
    out["greedy/logits"] = np.fromfile(w("lg.bin"), np.float32).reshape(4, -1)
    seq = np.concatenate([prompt, np.random.default_rng(5).integers(0, 2048, 5).astype(np.int32)])
    seq.tofile(w("s.bin"))
    run("batch", path, w("s.bin"), 16, 5, w("blg.bin"))
    out["batch/tokens"] = seq
    out["batch/logits"] = np.fromfile(w("blg.bin"), np.float32).reshape(5, -1)
    for t in ("token_embd.weight", "output.weight", "blk.0.ffn_down.weight"):
        run("dqrow", path, t, 3, 4, w("row.bin"))
        out[f"dqrow/{t}"] = np.fromfile(w("row.bin"), np.float32)
    dst = os.path.join(HERE, "dense_ref.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst}: {len(out)} arrays, {os.path.getsize(dst) / 1e6:.2f} MB")


if __name__ == "__main__":
    main()
