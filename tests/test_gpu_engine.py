"""Engine::generate on the device path against the reference's Engine
(engine_ref.npz, written by the reference build on the same stub-vocabulary
models): the chat template, the tokenized prompt, the batched prefill with the
prompt recorded in the sampler history, the per-token sampler (temperature 0:
repeat penalty, then argmax), the speculative path (greedy draft, target
samples at every verify position), the EOS stop and the on_token stream must
give the reference's pieces exactly. Also: the 128256-token stub layout's
tokenization, Engine::embed, and the prompt-too-long refusal.
"""
import os
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, SYNTH

pytestmark = pytest.mark.gpu
ENG = np.load(os.path.join(GOLDEN, "engine_ref.npz"))
MESSAGES = {
    "plain": [("user", "Say hello to the fox.")],
    "sys": [("system", "You are terse."), ("user", "hi"), ("assistant", "hello"), ("user", "again\nplease")],
}
CASES = {  # case: (target, draft, messages)
    "plain": ("t-q8", None, "plain"), "sys": ("t-q8", None, "sys"), "draft": ("t-q4k", "t-q4k-d", "plain"),
    "qwen": ("t-qwen", "t-qwen-d", "plain"), "eos": ("t-q8", None, "plain"),
    "eosdraft": ("t-q4k", "t-q4k-d", "plain"),
}


@pytest.fixture(scope="module")
def vmodels(tmp_path_factory):
    d = tmp_path_factory.mktemp("vmodels")

    def get(name, eot=-1):
        p = d / f"{name}{'' if eot < 0 else '_e' + str(eot)}.gguf"
        if not p.exists():
            cmd = [SYNTH, name, str(p), "--vocab"] + ([] if eot < 0 else ["--eot-id", str(eot)])
            subprocess.run(cmd, check=True, capture_output=True)
        return p

    return get


@pytest.mark.parametrize("case", list(CASES))
def test_generate_matches_reference_engine(vmodels, case):
    import orc

    tgt, dft, msgs = CASES[case]
    eot = int(ENG[f"eng/{case}/eot"][0])
    print(f"[gpu] engine {case} target={tgt} draft={dft} eot={eot}", flush=True)
    e = orc.Engine(vmodels(tgt, eot), vmodels(dft, eot) if dft else None, seed=7)
    try:
        got = e.generate(MESSAGES[msgs], n_predict=24, temperature=0.0)
    finally:
        e.close()
    want = orc.split_pieces(bytes(ENG[f"eng/{case}"]))
    assert got == want, (case, got[:8], want[:8])


def test_c2_layout_tokenizes_like_reference(vmodels):
    import orc

    print("[gpu] c2 tokenizer", flush=True)
    tok = orc.Tokenizer(vmodels("c2"))
    n = len([k for k in ENG.files if k.startswith("tok/c2/") and k.endswith("/text")])
    for i in range(n):
        text = bytes(ENG[f"tok/c2/{i}/text"])
        assert np.array_equal(tok.encode(text, True), ENG[f"tok/c2/{i}/bos"]), i
        assert np.array_equal(tok.encode(text, False), ENG[f"tok/c2/{i}/nobos"]), i
    assert tok.bos_eos() == (128000, 128009)


def test_embed_and_long_prompt(vmodels):
    import orc

    print("[gpu] engine embed / long prompt", flush=True)
    path = vmodels("t-q8")
    e = orc.Engine(path, seed=1)
    m = orc.Model(path)
    try:
        text = "the fox and the dog"
        got = e.embed(text, m.embed_dim)
        want = m.embed_tokens(orc.Tokenizer(path).encode(text, True))
        assert np.array_equal(got, want)
        # a prompt of more than ctx - 4 ids: empty reply, no pieces (core/engine.cpp:93-98)
        assert e.generate([("user", "x " * 600)], n_predict=4, temperature=0.0) == []
    finally:
        e.close()
        m.close()
