"""The drop-in benchmark CLI (bin/oracle_bench) keeps the reference harness's
protocol (benchmark/bench_engine.cpp:221-263, 300-376): R runs with the first
discarded, medians, the FNV-1a checksum of the generated ids, and the
speculative run's "exact" check (its checksum equals greedy's). The checksum
is compared with the FNV-1a of the reference's own greedy stream on the same
model and prompt (ref_fixtures.npz greedy/t-q4k), and bench.py's fnv1a is
checked against a value computed by hand. The speculative loop's checksum,
accepted / proposed drafts and main passes per token are compared with what
the reference's own harness (benchmark/bench_engine.cpp compiled from its
sources, tests/golden/make_golden_refbench.py) printed on the same files and
prompt ids, up to the full-size C3 pair.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import GOLDEN, PKG, ROOT

FIX = np.load(os.path.join(GOLDEN, "ref_fixtures.npz"))
BENCH = os.path.join(PKG, "bin", "oracle_bench")


def _fnv(ids):
    sys.path.insert(0, ROOT)
    from bench import fnv1a

    return fnv1a(ids)


def test_fnv1a_known_values():
    # the reference harness's basis 1469598103934665603 (benchmark/bench_engine.cpp:233; one digit short
    # of the standard FNV-1a 64 basis) and the FNV prime; one id folds in as one uint32
    assert _fnv([]) == f"{1469598103934665603:016x}"
    h = (1469598103934665603 ^ 7) * 0x100000001b3 % (1 << 64)
    assert _fnv([7]) == f"{h:016x}"
    h2 = (h ^ 0xFFFFFFFF) * 0x100000001b3 % (1 << 64)  # -1 as uint32
    assert _fnv([7, -1]) == f"{h2:016x}"
    # the checksum the reference build printed (REF_BENCH, oracle/_ref/ref_driver bench) for the first 32
    # ids of its C3 speculative stream (c3_ref.npz)
    c3 = np.load(os.path.join(GOLDEN, "c3_ref.npz"))
    assert _fnv(c3["spec_tokens"][:32]) == "d4aef56b75e7b077"


@pytest.mark.gpu
def test_oracle_bench_protocol_and_checksum(models_dir, tmp_path):
    print("[gpu] oracle_bench t-q4k --draft t-q4k-d", flush=True)
    prompt = FIX["greedy/t-q4k/prompt"].astype(np.int32)
    want = FIX["greedy/t-q4k/tokens"]
    pf, js = tmp_path / "prompt.bin", tmp_path / "out.json"
    prompt.tofile(pf)
    r = subprocess.run([BENCH, "-m", str(models_dir / "t-q4k.gguf"), "--draft", str(models_dir / "t-q4k-d.gguf"),
                        "--prompt-file", str(pf), "-g", str(len(want)), "-r", "3", "--spec-n", "4", "--json", str(js)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "run 1/3 [warmup]" in r.stdout and "RESULTS (median of 2 runs)" in r.stdout, r.stdout
    d = json.loads(js.read_text())
    assert d["gen_checksum"] == _fnv(want)
    assert d["spec_exact"] is True
    assert d["generation_tok_s"] > 0 and d["prefill_tok_s"] > 0 and d["spec_tok_s"] > 0
    assert d["prompt_tokens"] == len(prompt) - 1 and d["gen_tokens"] == len(want)


REFBENCH = os.path.join(GOLDEN, "refbench_ref.json")


def _sha(path):
    import hashlib

    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(3))
def test_spec_loop_matches_reference_harness(case, tmp_path):
    """The reference's OWN benchmark harness (benchmark/bench_engine.cpp,
    compiled from its sources; tests/golden/make_golden_refbench.py) on the
    same files and the same prompt ids: our bin/oracle_bench's greedy
    checksum, speculative checksum, accepted / proposed drafts and main
    passes per token equal what the harness printed (bench_engine.cpp:233-241,
    300-376). Cases: the tiny Q4_K_M pair, the tiny Qwen2 pair at k = 3, and
    the full-size C3 pair (prompt 128, 256 tokens, k = 4). The models are
    regenerated here with the tokenizer-vocab stub and checked by SHA-256."""
    from conftest import SYNTH

    c = json.load(open(REFBENCH))["cases"][case]
    print(f"[gpu] oracle_bench vs reference harness: {c['target']} + {c['draft']} p={c['n_prompt']} "
          f"g={c['n_gen']} k={c['k']}", flush=True)
    paths = []
    for name, key in ((c["target"], "target_sha256"), (c["draft"], "draft_sha256")):
        path = tmp_path / f"{name}.gguf"
        subprocess.run([SYNTH, name, str(path), "--vocab"], check=True, capture_output=True)
        assert _sha(path) == c[key], name
        paths.append(path)
    pf, js = tmp_path / "prompt.bin", tmp_path / "out.json"
    np.asarray(c["prompt"], np.int32).tofile(pf)
    r = subprocess.run([BENCH, "-m", str(paths[0]), "--draft", str(paths[1]), "--prompt-file", str(pf),
                        "-g", str(c["n_gen"]), "-r", "2", "--spec-n", str(c["k"]), "--json", str(js)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    d = json.loads(js.read_text())
    assert d["gen_checksum"] == c["greedy_checksum"]
    assert d["spec_checksum"] == c["spec_checksum"] and d["spec_exact"] is True
    assert (d["accepted"], d["proposed"]) == (c["accepted"], c["proposed"])
    assert d["spec_tokens"] == c["n_gen"]
    assert f"{d['passes'] / d['spec_tokens']:.2f}" == c["passes_per_token"]
