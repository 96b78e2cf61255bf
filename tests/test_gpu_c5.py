"""The C5 long-context workload at full size: the
Qwen2.5-7B-shape target requantized to Q6_K throughout with the
Qwen2.5-0.5B-shape Q8_0 draft, an 8192-id prompt in a 16384-position KV
cache and k = 8. The reference's Model fixes its context at 512 positions
(core/model.cpp:64), so it cannot run this case; the check is the property
the speculative-greedy loop guarantees at any size: its token stream equals
the target's own greedy stream (every verify pass here reads ~8.2-8.5 K
cached positions, so the long-context attention and the 9-token verify
GEMMs must agree with the one-token decode path: to fp32 rounding, which
changes no argmax unless two logits tie within it).
"""
import os
import subprocess
import time

import numpy as np
import pytest

from conftest import SYNTH

pytestmark = pytest.mark.gpu
N_PROMPT, N_GEN, K, CTX, VOCAB = 8192, 512, 8, 16384, 152064  # the config's 512 generated tokens


@pytest.fixture(scope="module")
def c5(tmp_path_factory):
    import orc

    d = os.environ.get("ORC_MODEL_DIR") or str(tmp_path_factory.mktemp("c5"))
    os.makedirs(d, exist_ok=True)
    paths = {}
    for m in ("c5", "c4d"):
        p = os.path.join(d, f"{m}.gguf")
        if not os.path.exists(p):
            with open(p + ".log", "wb") as log:
                proc = subprocess.Popen([SYNTH, m, p + ".tmp"], stdout=log, stderr=log)
                t0 = time.time()
                while True:
                    try:
                        proc.wait(timeout=15)
                        break
                    except subprocess.TimeoutExpired:
                        print(f"[gpu] writing {m}: {time.time() - t0:.0f} s", flush=True)
            assert proc.returncode == 0, open(p + ".log").read()
            os.replace(p + ".tmp", p)
        paths[m] = p
    print("[gpu] loading c5 + c4d", flush=True)
    tgt, dft = orc.Model(paths["c5"], CTX), orc.Model(paths["c4d"], CTX)
    yield tgt, dft
    tgt.close()
    dft.close()


def test_c5_long_context_spec_equals_greedy(c5):
    tgt, dft = c5
    prompt = np.random.default_rng(8192).integers(0, VOCAB, N_PROMPT).astype(np.int32)
    print(f"[gpu] c5 greedy {N_GEN} tokens after {N_PROMPT - 1} prefilled", flush=True)
    greedy = tgt.greedy(prompt, N_GEN, prefill=True)
    print(f"[gpu] c5 speculative greedy k={K}", flush=True)
    toks, st = tgt.spec_greedy(dft, prompt, N_GEN, K, prefill=True)
    assert len(greedy) == N_GEN and np.all((greedy >= 0) & (greedy < VOCAB))
    assert np.array_equal(toks, greedy)
    assert st["proposed"] > 0 and st["passes"] > 0
