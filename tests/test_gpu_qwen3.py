"""Per-head QK-norm (Qwen3) on the device path, against the reference's own
outputs on the t-qwen3 model (tests/golden/qwen3_ref.npz, written by
make_golden_qwen3.py from the reference build).

The reference normalises every q and k head over head_dim with the layer's
attn_q_norm / attn_k_norm weights after the QKV bias and before RoPE, with the
model's rms epsilon (core/model.cpp:390-399 in forward, 584-593 in
forward_prefill). The build runs that as one `orc_qk_norm` launch between the
Q|K|V GEMM and the attention launch of every layer. t-qwen3 also has a q width
(1024) above d_model (512), as Qwen3's smaller models do.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu
FIX = np.load(os.path.join(GOLDEN, "qwen3_ref.npz"))


@pytest.fixture(scope="module")
def q3(models_dir):
    import orc

    print("[gpu] loading t-qwen3", flush=True)
    m = orc.Model(models_dir / "t-qwen3.gguf")
    yield m
    m.close()


def test_qwen3_config_and_norm_cache(q3):
    import json

    ref = json.loads(bytes(FIX["cfg"]).decode())
    assert (q3.n_vocab, ref["qk_norm"], ref["head_dim"]) == (ref["n_vocab"], 1, 128)
    assert q3.norm_cache_matches()  # every norm, the QK-norm weights included, equals the file's bytes


def test_qwen3_greedy_stream_matches_reference(q3):
    print("[gpu] t-qwen3 greedy", flush=True)
    assert np.array_equal(q3.greedy(FIX["greedy/prompt"], 40), FIX["greedy/tokens"])


def test_qwen3_decode_and_verify_logits_match_reference(q3):
    print("[gpu] t-qwen3 logits", flush=True)
    prompt = FIX["greedy/prompt"]
    q3.reset()
    q3.forward_batch(prompt[:-1], 0, logits=False)
    cur, pos = int(prompt[-1]), len(prompt) - 1
    for s in range(4):
        lg = q3.forward(cur, pos)
        ref = FIX["greedy/logits"][s]
        assert np.abs(lg - ref).max() <= 1e-4 * np.abs(ref).max(), s
        cur, pos = int(np.argmax(lg)), pos + 1
    # verify logits after a 16-id prefill (verify kernels) and a 300-id
    # prefill (the prefill GEMM and prefill attention)
    for npf in (16, 300):
        print(f"[gpu] t-qwen3 verify after {npf} ids", flush=True)
        seq = FIX[f"batch{npf}/tokens"]
        q3.reset()
        q3.forward_batch(seq[:npf], 0, logits=False)
        lg = q3.forward_batch(seq[npf:], npf)
        ref = FIX[f"batch{npf}/logits"]
        assert np.abs(lg - ref).max() <= 1e-4 * np.abs(ref).max(), npf


@pytest.mark.parametrize("graphs", [True, False])
def test_qwen3_spec_greedy_matches_reference(q3, models_dir, graphs):
    import orc

    print(f"[gpu] t-qwen3 spec greedy graphs={graphs}", flush=True)
    H = orc.load_host_lib()
    dft = orc.Model(models_dir / "t-qwen-d.gguf")
    prev = H.orch_set_graphs(int(graphs))
    try:
        q3.reset()
        toks, st = q3.spec_greedy(dft, FIX["greedy/prompt"], 40, 3)
    finally:
        H.orch_set_graphs(prev)
        dft.close()
    assert np.array_equal(toks, FIX["spec/tokens"])
    assert np.array_equal(toks, FIX["greedy/tokens"])  # speculation keeps the greedy stream
    assert [st["accepted"], st["proposed"], st["passes"]] == list(FIX["spec/stats"])
