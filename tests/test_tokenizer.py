"""The host Tokenizer and the GGUF tokenizer stub, on the CPU.

The synthetic models written with --vocab carry a byte-level BPE vocabulary
(tokenizer.ggml.*) that the reference's Tokenizer loads; the host Tokenizer
must give the reference's ids for every text and the reference's piece for
every id (engine_ref.npz, written by the reference build). The tokenizer reads
only the GGUF metadata (GGUFParser::load_meta), so no GPU is involved.
"""
import os
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, SYNTH

ENG = np.load(os.path.join(GOLDEN, "engine_ref.npz"))
N_TEXTS = len([k for k in ENG.files if k.startswith("tok/t-q8/") and k.endswith("/text")])


@pytest.fixture(scope="module")
def vocab_models(tmp_path_factory):
    d = tmp_path_factory.mktemp("vocab")
    for name in ("t-q8", "t-qwen"):
        subprocess.run([SYNTH, name, str(d / f"{name}.gguf"), "--vocab"], check=True, capture_output=True)
    subprocess.run([SYNTH, "t-q8", str(d / "t-q8-e.gguf"), "--vocab", "--eot-id", "413"], check=True,
                   capture_output=True)
    return d


@pytest.mark.parametrize("m", ["t-q8", "t-qwen"])
def test_encode_matches_reference(vocab_models, m):
    import orc

    tok = orc.Tokenizer(vocab_models / f"{m}.gguf")
    for i in range(N_TEXTS):
        text = bytes(ENG[f"tok/{m}/{i}/text"])
        assert np.array_equal(tok.encode(text, True), ENG[f"tok/{m}/{i}/bos"]), (m, i)
        assert np.array_equal(tok.encode(text, False), ENG[f"tok/{m}/{i}/nobos"]), (m, i)


@pytest.mark.parametrize("m", ["t-q8", "t-qwen"])
def test_decode_one_matches_reference(vocab_models, m):
    import orc

    tok = orc.Tokenizer(vocab_models / f"{m}.gguf")
    want = orc.split_pieces(bytes(ENG[f"detok/{m}"]))
    assert len(want) == 2048
    got = [tok.decode_one(i) for i in range(2048)]
    assert got == want
    assert tok.decode_one(-1) == b"" and tok.decode_one(2048) == b""


def test_stub_layout(vocab_models):
    """Specials are control tokens at the architecture's places; --eot-id moves
    the end-of-turn token and the eos id with it; decoding every byte symbol
    gives the byte back (GPT-2 byte map round trip)."""
    import orc

    llama, qwen = orc.Tokenizer(vocab_models / "t-q8.gguf"), orc.Tokenizer(vocab_models / "t-qwen.gguf")
    assert llama.bos_eos() == (2048 - 16, 2048 - 16 + 9)
    assert llama.special_id("<|eot_id|>") == 2048 - 7 and llama.special_id("<|start_header_id|>") == 2048 - 10
    assert qwen.bos_eos() == (2048 - 16, 2048 - 14) and qwen.special_id("<|im_start|>") == 2048 - 15
    assert llama.special_id("<|im_end|>") == -1
    assert llama.decode_one(2048 - 7) == b""  # control tokens print nothing
    moved = orc.Tokenizer(vocab_models / "t-q8-e.gguf")
    assert moved.special_id("<|eot_id|>") == 413 and moved.bos_eos()[1] == 413
    assert [llama.decode_one(b) for b in range(256)] == [bytes([b]) for b in range(256)]
    # a whole-word control token encodes to its id; glued to text it does not
    assert list(llama.encode("\n<|eot_id|>", False)) == [10, 2048 - 7]
    assert 2048 - 7 not in list(llama.encode("x<|eot_id|>", False))
