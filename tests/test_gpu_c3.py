"""The north-star check at full size: on the C2 / C3 workload (3B-shape Q4_K_M
target, 8-layer Q8_0 draft, k = 4, prompt 128, 256 tokens) the device's greedy
and speculative-greedy token streams equal the REFERENCE's, and so do the
speculative loop's accepted / proposed / target-pass counts
(benchmark/bench_engine.cpp:300-376).

The expected streams are tests/golden/c3_ref.npz, written by
tests/golden/make_golden_c3.py from the reference build; the models are
regenerated here by bin/synth_gguf and checked against the stored SHA-256.
"""
import hashlib
import os
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, SYNTH

pytestmark = pytest.mark.gpu
FIX = np.load(os.path.join(GOLDEN, "c3_ref.npz"))


def _sha(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 22), b""):
            h.update(chunk)
    return h.hexdigest()


@pytest.fixture(scope="module")
def c3_models(tmp_path_factory):
    import orc

    d = os.environ.get("ORC_MODEL_DIR") or str(tmp_path_factory.mktemp("c3"))
    os.makedirs(d, exist_ok=True)
    paths = {}
    for m in ("c2", "c3d"):
        p = os.path.join(d, f"{m}.gguf")
        if not os.path.exists(p):
            print(f"[gpu] writing {m}", flush=True)
            subprocess.run([SYNTH, m, p + ".tmp"], check=True, capture_output=True)
            os.replace(p + ".tmp", p)
        assert _sha(p) == bytes(FIX[f"sha/{m}"]).decode(), f"{p} differs from the model the reference ran"
        paths[m] = p
    print("[gpu] loading c2 + c3d", flush=True)
    tgt, dft = orc.Model(paths["c2"], 2048), orc.Model(paths["c3d"], 2048)
    yield tgt, dft
    tgt.close()
    dft.close()


def test_c2_greedy_stream_matches_reference(c3_models):
    tgt, _ = c3_models
    print("[gpu] c2 greedy 256 tokens", flush=True)
    toks = tgt.greedy(FIX["prompt"], len(FIX["greedy_tokens"]), prefill=True)
    assert np.array_equal(toks, FIX["greedy_tokens"])


def test_c3_spec_stream_and_stats_match_reference(c3_models):
    tgt, dft = c3_models
    k = int(FIX["k"][0])
    print(f"[gpu] c3 speculative greedy k={k}, 256 tokens", flush=True)
    toks, st = tgt.spec_greedy(dft, FIX["prompt"], len(FIX["spec_tokens"]), k, prefill=True)
    assert np.array_equal(toks, FIX["spec_tokens"])
    acc, prop, passes = (int(v) for v in FIX["spec_stats"])
    assert (st["accepted"], st["proposed"], st["passes"]) == (acc, prop, passes)
