"""Writes tests/golden/surface_ref.npz: the REFERENCE's Model::embed_tokens and
.orkv state files on the small synthetic models (bin/synth_gguf t-q8, t-q4k),
via oracle/_ref/ref_driver (compiled from the reference's own sources by
oracle/Makefile).

  * embed/<m>: Model::embed_tokens (core/model.cpp:248-270) of 20 ids drawn by
    numpy default_rng(77) below the vocabulary, and those ids;
  * orkv/<m>/file: the bytes of the .orkv file save_state (core/model.cpp:
    156-181) writes after forward_prefill of the first 11 of 12 prompt ids
    (default_rng(78)), stored compressed (the 512-position cache is mostly
    zeros); orkv/<m>/logits: the logits a second Model returns for the 12th
    id after load_state of that file (core/model.cpp:184-236); orkv/<m>/prompt.

Run: python tests/golden/make_golden_surface.py   (in the container that holds
/root/reference; seconds)
"""
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
SYNTH = os.path.join(ROOT, "oracle-engine_amd", "bin", "synth_gguf")
DRV = os.path.join(ROOT, "oracle", "_ref", "ref_driver")
MODELS = ["t-q8", "t-q4k"]
VOCAB = 2048


def main():
    tmp = tempfile.mkdtemp(prefix="orc_surface_")
    out = {}
    for m in MODELS:
        path = os.path.join(tmp, m + ".gguf")
        subprocess.run([SYNTH, m, path], check=True, stdout=subprocess.DEVNULL)
        ids = np.random.default_rng(77).integers(0, VOCAB, 20).astype(np.int32)
        tf, ef = os.path.join(tmp, "ids.bin"), os.path.join(tmp, "emb.bin")
        ids.tofile(tf)
        subprocess.run([DRV, "embed", path, tf, ef], check=True)
        out[f"embed/{m}/ids"], out[f"embed/{m}"] = ids, np.fromfile(ef, np.float32)
        prompt = np.random.default_rng(78).integers(0, VOCAB, 12).astype(np.int32)
        pf, sf, lf = (os.path.join(tmp, n) for n in ("prompt.bin", "state.orkv", "logits.bin"))
        prompt.tofile(pf)
        subprocess.run([DRV, "orkv", path, pf, sf, lf], check=True)
        out[f"orkv/{m}/prompt"] = prompt
        out[f"orkv/{m}/file"] = np.fromfile(sf, np.uint8)
        out[f"orkv/{m}/logits"] = np.fromfile(lf, np.float32)
    dst = os.path.join(HERE, "surface_ref.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({os.path.getsize(dst)} bytes)", file=sys.stderr)


if __name__ == "__main__":
    main()
