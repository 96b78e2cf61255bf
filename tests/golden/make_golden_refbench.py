"""Writes tests/golden/refbench_ref.json: what the REFERENCE's own benchmark
harness (benchmark/bench_engine.cpp, compiled from its sources into
oracle/_ref/oracle_bench by oracle/Makefile) prints for the greedy and the
batched speculative-greedy loops on this build's synthetic models.

The harness builds its prompt itself: it tokenizes its fixed benchmark text
with the model's tokenizer, BOS first, and tiles the ids to -p tokens
(bench_engine.cpp:193-200). The models are therefore written with the
tokenizer-vocab stub (bin/synth_gguf --vocab), and this script takes the
same ids from the reference's Tokenizer (oracle/_ref/ref_driver tokenize),
reading the text out of the harness source at generation time; the fixture
holds only the resulting ids. Per case it records:
  * the prompt ids, the models' SHA-256;
  * the greedy checksum (FNV-1a of the generated ids, bench_engine.cpp:233-241),
  * the speculative loop's checksum, accepted / proposed drafts and the
    printed main passes per token (bench_engine.cpp:300-376).

Cases: the tiny Q4_K_M pair (t-q4k + t-q4k-d), the tiny Qwen2 pair with QKV
bias (t-qwen + t-qwen-d) at k = 3, and the full-size C3 pair (c2 + c3d,
prompt 128, 256 tokens, k = 4).

Run: python tests/golden/make_golden_refbench.py   (in the container that
holds /root/reference; about 4 minutes on 8 cores, almost all of it C3)
"""
import hashlib
import json
import os
import re
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
SYNTH = os.path.join(ROOT, "oracle-engine_amd", "bin", "synth_gguf")
DRV = os.path.join(ROOT, "oracle", "_ref", "ref_driver")
BENCH = os.path.join(ROOT, "oracle", "_ref", "oracle_bench")
SRC = "/root/reference/benchmark/bench_engine.cpp"
CASES = [("t-q4k", "t-q4k-d", 32, 48, 4), ("t-qwen", "t-qwen-d", 40, 64, 3), ("c2", "c3d", 128, 256, 4)]


def sha(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def harness_text():
    """The harness's benchmark text: the concatenated C string literals of
    its prompt constant, unescaped."""
    src = open(SRC, encoding="utf-8").read()
    m = re.search(r"static const char\*\s+REF_PROMPT\s*=\s*(.*?);", src, re.S)
    parts = re.findall(r'"((?:[^"\\]|\\.)*)"', m.group(1))
    return "".join(parts).encode("utf-8").decode("unicode_escape").encode("latin-1")


def main():
    text = harness_text()
    out = {"cases": []}
    with tempfile.TemporaryDirectory() as d:
        tf = os.path.join(d, "text.bin")
        with open(tf, "wb") as f:
            f.write(text)
        for tgt, dft, p, g, k in CASES:
            paths = []
            for name in (tgt, dft):
                path = os.path.join(d, name + ".gguf")
                if not os.path.exists(path):
                    subprocess.run([SYNTH, name, path, "--vocab"], check=True, capture_output=True)
                paths.append(path)
            ids_f = os.path.join(d, "ids.bin")
            subprocess.run([DRV, "tokenize", paths[0], tf, "1", ids_f], check=True, capture_output=True)
            base = np.fromfile(ids_f, np.int32)
            prompt = np.resize(base, p)  # tiled to p ids, as bench_engine.cpp:197-200
            print(f"[refbench] {tgt} + {dft}: p={p} g={g} k={k} (base text {len(base)} ids)", flush=True)
            r = subprocess.run([BENCH, "-m", paths[0], "--draft", paths[1], "-p", str(p), "-g", str(g), "-r", "2",
                                "-t", str(min(16, os.cpu_count() or 1)), "--spec-n", str(k)],
                               check=True, capture_output=True, text=True)
            so = r.stdout
            greedy = re.search(r"Checksum\s*:\s*([0-9a-f]{16})", so).group(1)
            acc = re.search(r"\((\d+)/(\d+) tokens draft", so)
            passes = re.search(r"Passes main/tok\s*:\s*([0-9.]+)", so).group(1)
            spec = re.search(r"checksum spec ([0-9a-f]{16}) vs greedy ([0-9a-f]{16})", so)
            case = {"target": tgt, "draft": dft, "n_prompt": p, "n_gen": g, "k": k,
                    "target_sha256": sha(paths[0]), "draft_sha256": sha(paths[1]),
                    "prompt": prompt.tolist(), "greedy_checksum": greedy, "spec_checksum": spec.group(1),
                    "accepted": int(acc.group(1)), "proposed": int(acc.group(2)), "passes_per_token": passes}
            assert spec.group(2) == greedy
            print(f"[refbench]   greedy {greedy} spec {spec.group(1)} accepted {acc.group(1)}/{acc.group(2)} "
                  f"passes/tok {passes}", flush=True)
            out["cases"].append(case)
            for path in paths:
                if os.path.getsize(path) > 100 << 20:
                    os.remove(path)
    with open(os.path.join(HERE, "refbench_ref.json"), "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", os.path.join(HERE, "refbench_ref.json"))


if __name__ == "__main__":
    sys.exit(main())
