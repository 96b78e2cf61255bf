"""Writes tests/golden/engine_ref.npz: the REFERENCE's Tokenizer and
Engine::generate on small synthetic models written with the tokenizer stub
(bin/synth_gguf <preset> --vocab), via oracle/_ref/ref_driver (compiled from
the reference's own sources by oracle/Makefile).

  * tok/<m>/<i>/{text,bos,nobos}: Tokenizer::encode (core/tokenizer.cpp:
    252-273) of TEXTS[i] with and without BOS, for m in t-q8 (Llama-3 style
    specials), t-qwen (ChatML specials) and c2 (the 128256-token layout);
  * detok/<m>: Tokenizer::decode_one of every id of the tiny vocabularies
    (records: uint32 byte length, bytes);
  * eng/<case>: the on_token pieces of Engine::generate (core/engine.cpp:
    83-243) at temperature 0 (the reference seeds its sampler from the clock,
    so only T = 0 is reproducible; its repeat penalty still applies), for:
      plain    - t-q8, one user message, 24 tokens;
      sys      - t-q8, system + user + assistant + user messages, 24 tokens;
      draft    - t-q4k with the t-q4k-d draft (speculative path), 24 tokens;
      qwen     - t-qwen with the t-qwen-d draft (ChatML template), 24 tokens;
      eos      - t-q8 rewritten with <|eot_id|> at the id of the 5th token the
                 plain case generates (--eot-id): the reply stops before it;
      eosdraft - the same EOS id on the speculative path (t-q4k / t-q4k-d).
    eng/<case>/eot: the --eot-id used (-1: none).

Run: python tests/golden/make_golden_engine.py   (in the container that holds
/root/reference; seconds)
"""
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

TEXTS = [
    "Hello world, the fox!",
    "  two  spaces\tand\ttabs\n\nnew lines\r\nand the end ",
    "café € 100 \U0001F600 naïve",
    "<|eot_id|>\n<|im_end|>\n<|start_header_id|>user",
    "<|begin_of_text|><|start_header_id|>system<|end_header_id|>\n\nTu es un assistant utile.<|eot_id|>",
    "the quick brown fox jumps over the lazy dog and the assistant gives an answer",
    "",
]
MESSAGES = {
    "plain": [("user", "Say hello to the fox.")],
    "sys": [("system", "You are terse."), ("user", "hi"), ("assistant", "hello"), ("user", "again\nplease")],
}


def pieces(path):
    b = open(path, "rb").read()
    out, i = [], 0
    while i < len(b):
        n = int.from_bytes(b[i:i + 4], "little")
        out.append(b[i + 4:i + 4 + n])
        i += 4 + n
    return out


def pack(ps):
    return np.frombuffer(b"".join(len(p).to_bytes(4, "little") + p for p in ps), np.uint8)


def main():
    tmp = tempfile.mkdtemp(prefix="orc_engine_")
    out = {}

    def model(preset, eot=-1):
        path = os.path.join(tmp, f"{preset}{'' if eot < 0 else '_e' + str(eot)}.gguf")
        if not os.path.exists(path):
            cmd = [SYNTH, preset, path, "--vocab"] + ([] if eot < 0 else ["--eot-id", str(eot)])
            subprocess.run(cmd, check=True, stderr=subprocess.DEVNULL)
        return path

    f = os.path.join(tmp, "f.bin")
    for m in ("t-q8", "t-qwen", "c2"):
        p = model(m)
        for i, t in enumerate(TEXTS):
            open(os.path.join(tmp, "t.txt"), "wb").write(t.encode())
            for bos in (1, 0):
                subprocess.run([DRV, "tokenize", p, os.path.join(tmp, "t.txt"), str(bos), f], check=True,
                               stderr=subprocess.DEVNULL)
                out[f"tok/{m}/{i}/{'bos' if bos else 'nobos'}"] = np.fromfile(f, np.int32)
            out[f"tok/{m}/{i}/text"] = np.frombuffer(t.encode(), np.uint8)
        if m != "c2":
            np.arange(2048, dtype=np.int32).tofile(os.path.join(tmp, "ids.bin"))
            subprocess.run([DRV, "detok", p, os.path.join(tmp, "ids.bin"), f], check=True, stderr=subprocess.DEVNULL)
            out[f"detok/{m}"] = np.fromfile(f, np.uint8)

    def engine(case, tgt, dft, msgs, n=24, eot=-1):
        mf = os.path.join(tmp, "msgs.bin")
        open(mf, "wb").write(b"".join(r.encode() + b"\0" + c.encode() + b"\0" for r, c in msgs))
        r = subprocess.run([DRV, "engine", model(tgt, eot), model(dft, eot) if dft else "-", str(n), "0", mf, f],
                           capture_output=True, text=True)
        if r.returncode:
            sys.exit(f"engine {case} failed: {r.stderr[-500:]}")
        ps = pieces(f)
        out[f"eng/{case}"] = pack(ps)
        out[f"eng/{case}/eot"] = np.array([eot], np.int32)
        return ps

    plain = engine("plain", "t-q8", None, MESSAGES["plain"])
    engine("sys", "t-q8", None, MESSAGES["sys"])
    draft = engine("draft", "t-q4k", "t-q4k-d", MESSAGES["plain"])
    engine("qwen", "t-qwen", "t-qwen-d", MESSAGES["plain"])
    # EOS: the id of the 5th generated piece (a filler token "<unusedN>")
    for case, ps, tgt, dft in (("eos", plain, "t-q8", None), ("eosdraft", draft, "t-q4k", "t-q4k-d")):
        ids = [int(m.group(1)) for p in ps for m in [re.fullmatch(rb"<unused(\d+)>", p)] if m]
        eot = ids[4]
        got = engine(case, tgt, dft, MESSAGES["plain"], eot=eot)
        assert 0 < len(got) < len(ps), (case, len(got))
    dst = os.path.join(HERE, "engine_ref.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({os.path.getsize(dst)} bytes)", file=sys.stderr)


if __name__ == "__main__":
    main()
