"""Writes tests/golden/qwen3_ref.npz from the REFERENCE implementation on the
t-qwen3 model (bin/synth_gguf t-qwen3): qwen3 architecture with per-head
QK-norm (attn_q_norm / attn_k_norm weights 1 + N(0, 0.1^2)), head_dim 128 with
a q width (1024) above d_model (512), rms epsilon 1e-6, Q4_K_M-style types.

The reference applies ops::rmsnorm to every q and k head after the bias and
before RoPE, with cfg.rms_eps (core/model.cpp:390-399 in forward,
584-593 in forward_prefill). Stored: the model's SHA-256 and config, greedy
decode (40 tokens, the first 4 steps' logits), 5-token verify logits after a
16-id prefill and after a 300-id prefill (the long one takes the prefill
kernels on the GPU), and the batched speculative loop with the t-qwen-d draft
(k = 3: tokens and accepted / proposed / passes).

Run: python tests/golden/make_golden_qwen3.py   (needs /root/reference, in this container)
"""
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)
from make_golden import _stats, run, sha  # noqa: E402

SYNTH = os.path.join(ROOT, "oracle-engine_amd", "bin", "synth_gguf")


def main():
    tmp = tempfile.mkdtemp(prefix="orc_golden_qwen3_")
    w = lambda name: os.path.join(tmp, name)  # noqa: E731
    path, dpath = w("t-qwen3.gguf"), w("t-qwen-d.gguf")
    subprocess.run([SYNTH, "t-qwen3", path], check=True, capture_output=True)
    subprocess.run([SYNTH, "t-qwen-d", dpath], check=True, capture_output=True)
    out = {"sha/t-qwen3": np.frombuffer(sha(path).encode(), np.uint8)}
    cfg = json.loads(run("cfg", path).stdout.strip().splitlines()[-1])  # the last line (the log goes first)
    assert cfg["qk_norm"] == 1 and cfg["head_dim"] == 128, cfg
    out["cfg"] = np.frombuffer(json.dumps(cfg, sort_keys=True).encode(), np.uint8)
    prompt = np.random.default_rng(3003).integers(0, 2048, 16).astype(np.int32)
    prompt.tofile(w("p.bin"))
    run("greedy", path, w("p.bin"), 40, w("tok.bin"), w("lg.bin"), 4)
    out["greedy/prompt"] = prompt
    out["greedy/tokens"] = np.fromfile(w("tok.bin"), np.int32)
    out["greedy/logits"] = np.fromfile(w("lg.bin"), np.float32).reshape(4, -1)
    for npf in (16, 300):
        seq = np.random.default_rng(npf).integers(0, 2048, npf + 5).astype(np.int32)
        seq.tofile(w("s.bin"))
        run("batch", path, w("s.bin"), npf, 5, w("blg.bin"))
        out[f"batch{npf}/tokens"] = seq
        out[f"batch{npf}/logits"] = np.fromfile(w("blg.bin"), np.float32).reshape(5, -1)
    r = run("spec", path, dpath, w("p.bin"), 40, 3, w("st.bin"))
    out["spec/tokens"] = np.fromfile(w("st.bin"), np.int32)
    out["spec/stats"] = _stats(r)
    dst = os.path.join(HERE, "qwen3_ref.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst}: {len(out)} arrays, {os.path.getsize(dst) / 1e6:.2f} MB")


if __name__ == "__main__":
    main()
