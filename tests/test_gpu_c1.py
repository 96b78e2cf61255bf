"""C1 at full size: the Llama-3.2-1B-shape model
with every linear weight Q8_0 (regrouped at load into the aligned Q8_0_X8
layout), prompt of 32 random ids, greedy decode of 128 tokens, context 512.

The device's token stream equals the REFERENCE's, and so do the first four
decode steps' logits (within 1e-2 relative; asserted at
1e-4 of the largest logit), from tests/golden/c1_ref.npz, written by
tests/golden/make_golden_c1.py from the reference build. The model is
regenerated here by bin/synth_gguf and checked against the stored SHA-256.
"""
import hashlib
import os
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, SYNTH

pytestmark = pytest.mark.gpu
FIX = np.load(os.path.join(GOLDEN, "c1_ref.npz"))


def _sha(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 22), b""):
            h.update(chunk)
    return h.hexdigest()


def fnv1a(tokens):
    """benchmark/bench_engine.cpp:233-241: FNV-1a over the generated ids."""
    h = 1469598103934665603
    for t in tokens:
        h = ((h ^ (int(t) & 0xFFFFFFFF)) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


@pytest.fixture(scope="module")
def c1_model(tmp_path_factory):
    import orc

    d = os.environ.get("ORC_MODEL_DIR") or str(tmp_path_factory.mktemp("c1"))
    os.makedirs(d, exist_ok=True)
    p = os.path.join(d, "c1.gguf")
    if not os.path.exists(p):
        print("[gpu] writing c1", flush=True)
        subprocess.run([SYNTH, "c1", p + ".tmp"], check=True, capture_output=True)
        os.replace(p + ".tmp", p)
    assert _sha(p) == bytes(FIX["sha/c1"]).decode(), f"{p} differs from the model the reference ran"
    print("[gpu] loading c1 ctx=512", flush=True)
    m = orc.Model(p, 512)
    yield m
    m.close()


def test_c1_layers_run_regrouped(c1_model):
    assert c1_model.gguf_device_type("blk.0.ffn_down.weight") == 258
    assert c1_model.gguf_device_type("token_embd.weight") == 8  # gathered rows keep the GGUF layout


@pytest.mark.parametrize("graphs", [True, False])
def test_c1_greedy_stream_matches_reference(c1_model, graphs):
    import orc

    print(f"[gpu] c1 greedy 128 tokens, graphs={graphs}", flush=True)
    H = orc.load_host_lib()
    prev = H.orch_set_graphs(int(graphs))
    try:
        toks = c1_model.greedy(FIX["prompt"], len(FIX["greedy_tokens"]), prefill=True)
    finally:
        H.orch_set_graphs(prev)
    assert np.array_equal(toks, FIX["greedy_tokens"])
    assert fnv1a(toks) == fnv1a(FIX["greedy_tokens"])


def test_c1_first_logits_match_reference(c1_model):
    prompt = FIX["prompt"]
    stride = int(FIX["logits_stride"][0])
    c1_model.reset()
    c1_model.forward_batch(prompt[:-1], 0, logits=False)
    cur, pos = int(prompt[-1]), len(prompt) - 1
    for s in range(FIX["logits_strided"].shape[0]):
        lg = c1_model.forward(cur, pos)
        amax = float(FIX["logits_absmax"][s])
        sub, ref = lg[::stride], FIX["logits_strided"][s]
        assert np.abs(sub - ref).max() <= 1e-4 * amax, (s, np.abs(sub - ref).max() / amax)
        assert np.linalg.norm(sub - ref) <= 1e-2 * np.linalg.norm(ref)
        idx, val = FIX["logits_top_idx"][s], FIX["logits_top_val"][s]
        assert np.abs(lg[idx] - val).max() <= 1e-4 * amax, s
        assert int(np.argmax(lg)) == int(FIX["greedy_tokens"][s])
        cur, pos = int(np.argmax(lg)), pos + 1
