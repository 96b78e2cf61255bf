"""Writes tests/golden/c4_ref.npz: the REFERENCE's token stream and
acceptance counts on the full-size C4 workload.

  * target = synthetic Qwen2.5-7B-shape Q4_K_M model with QKV bias
    (bin/synth_gguf c4), draft = Qwen2.5-0.5B-shape Q8_0 model
    (bin/synth_gguf c4d); their SHA-256 is stored so a test can prove it
    regenerated the same files;
  * prompt = 256 uniform-random ids, numpy default_rng(4321);
  * the Engine's stochastic speculative loop (core/engine.cpp, via
    oracle/_ref/ref_driver espec) with k = 6, temperature 0.8, top-p 0.95,
    top-k 40, repeat penalty 1.1 over the last 64 tokens, seed 4242, and its
    accepted / proposed / passes; 240 tokens: the reference's Model fixes its
    context at 512 positions (core/model.cpp:64), so the run stays below that
    bound (BASELINE's 512 tokens at ctx 4096 would end at position 511 there).

The reference is compiled from its own sources by oracle/Makefile (make ref).
Run: python tests/golden/make_golden_c4.py   (in the container that holds
/root/reference; about 15 minutes on 8 cores)
"""
import hashlib
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
SYNTH = os.path.join(ROOT, "oracle-engine_amd", "bin", "synth_gguf")
DRV = os.path.join(ROOT, "oracle", "_ref", "ref_driver")
N_PROMPT, N_GEN, K, VOCAB = 256, 240, 6, 152064
SAMPLER = {"temp": 0.8, "top_p": 0.95, "top_k": 40, "pen": 1.1, "last": 64, "seed": 4242}


def sha(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def main():
    tmp = tempfile.mkdtemp(prefix="orc_c4_")
    paths = {}
    for m in ("c4", "c4d"):
        paths[m] = os.path.join(tmp, m + ".gguf")
        subprocess.run([SYNTH, m, paths[m]], check=True)
    prompt = np.random.default_rng(4321).integers(0, VOCAB, N_PROMPT).astype(np.int32)
    pf = os.path.join(tmp, "prompt.bin")
    prompt.tofile(pf)
    sf = os.path.join(tmp, "espec.bin")
    s = SAMPLER
    r = subprocess.run([DRV, "espec", paths["c4"], paths["c4d"], pf, str(N_GEN), str(K), str(s["temp"]),
                        str(s["top_p"]), str(s["top_k"]), str(s["pen"]), str(s["last"]), str(s["seed"]), sf],
                       check=True, capture_output=True, text=True)
    st = json.loads(r.stderr.strip().splitlines()[-1])
    out = {
        "prompt": prompt,
        "espec_tokens": np.fromfile(sf, np.int32),
        "espec_stats": np.array([st["accepted"], st["proposed"], st["passes"]], np.int64),
        "k": np.array([K], np.int32),
        "sampler": np.array([s["temp"], s["top_p"], s["top_k"], s["pen"], s["last"], s["seed"]], np.float64),
        "sha/c4": np.frombuffer(sha(paths["c4"]).encode(), np.uint8),
        "sha/c4d": np.frombuffer(sha(paths["c4d"]).encode(), np.uint8),
    }
    dst = os.path.join(HERE, "c4_ref.npz")
    np.savez_compressed(dst, **out)
    for p in paths.values():
        os.remove(p)
    print(f"wrote {dst}: {out['espec_tokens'].size} tokens, stats {st}")


if __name__ == "__main__":
    sys.exit(main())
