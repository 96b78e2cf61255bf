"""Writes tests/golden/c3_ref.npz: the REFERENCE's token streams on the
full-size C2 / C3 workload.

  * target = synthetic Llama-3.2-3B-shape Q4_K_M model (bin/synth_gguf c2),
    draft = its 8-layer Q8_0 draft (bin/synth_gguf c3d); their SHA-256 is
    stored so a test can prove it regenerated the same files;
  * prompt = 128 uniform-random ids, numpy default_rng(1234) (bench.py's);
  * greedy: Model::forward decode of 256 tokens after prefilling 127
    (benchmark/bench_engine.cpp:226-243 protocol, via oracle/_ref/ref_driver);
  * spec: the batched speculative-greedy loop with k = 4 for 256 tokens
    (benchmark/bench_engine.cpp:300-363) and its accepted / proposed / passes.

The reference is compiled from its own sources by oracle/Makefile (make ref).
Run: python tests/golden/make_golden_c3.py   (in the container that holds
/root/reference; about 6 minutes on 8 cores)
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
N_PROMPT, N_GEN, K = 128, 256, 4


def sha(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def main():
    tmp = tempfile.mkdtemp(prefix="orc_c3_")
    paths = {}
    for m in ("c2", "c3d"):
        paths[m] = os.path.join(tmp, m + ".gguf")
        subprocess.run([SYNTH, m, paths[m]], check=True)
    prompt = np.random.default_rng(1234).integers(0, 128256, N_PROMPT).astype(np.int32)
    pf = os.path.join(tmp, "prompt.bin")
    prompt.tofile(pf)
    gf, sf = os.path.join(tmp, "greedy.bin"), os.path.join(tmp, "spec.bin")
    subprocess.run([DRV, "greedy", paths["c2"], pf, str(N_GEN), gf], check=True)
    r = subprocess.run([DRV, "spec", paths["c2"], paths["c3d"], pf, str(N_GEN), str(K), sf], check=True,
                       capture_output=True, text=True)
    st = json.loads(r.stderr.strip().splitlines()[-1])
    out = {
        "prompt": prompt,
        "greedy_tokens": np.fromfile(gf, np.int32),
        "spec_tokens": np.fromfile(sf, np.int32),
        "spec_stats": np.array([st["accepted"], st["proposed"], st["passes"]], np.int64),
        "k": np.array([K], np.int32),
        "sha/c2": np.frombuffer(sha(paths["c2"]).encode(), np.uint8),
        "sha/c3d": np.frombuffer(sha(paths["c3d"]).encode(), np.uint8),
    }
    dst = os.path.join(HERE, "c3_ref.npz")
    np.savez_compressed(dst, **out)
    for p in paths.values():
        os.remove(p)
    print(f"wrote {dst}: stats {st}, greedy == spec: {np.array_equal(out['greedy_tokens'], out['spec_tokens'])}")


if __name__ == "__main__":
    sys.exit(main())
