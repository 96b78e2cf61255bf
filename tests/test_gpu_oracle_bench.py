"""The drop-in benchmark CLI (bin/oracle_bench) keeps the reference harness's
protocol (benchmark/bench_engine.cpp:221-263, 300-376): R runs with the first
discarded, medians, the FNV-1a checksum of the generated ids, and the
speculative run's "exact" check (its checksum equals greedy's). The checksum
is compared with the FNV-1a of the reference's own greedy stream on the same
model and prompt (ref_fixtures.npz greedy/t-q4k), and bench.py's fnv1a is
checked against a value computed by hand.
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
