"""Writes tests/golden/ref_fixtures.npz from the REFERENCE implementation.

The reference (compiled from its own sources by oracle/Makefile into
oracle/_ref/ref_driver) is run on:
  * random GGML blocks through its public codec hooks (test_dq_q4_0/q4_k/q6_k,
    core/gguf_parser.hpp:127-132) and dequantize_row;
  * gemv_q / gemm_q on every weight of small synthetic models;
  * Model::forward greedy decode (logits of the first steps + token stream),
    forward_batch verify logits, the batched speculative loop
    (benchmark/bench_engine.cpp:300-356) and the Engine's stochastic
    speculative loop with a fixed seed (core/engine.cpp:150-240);
  * Sampler draws and the ops:: primitives.
The models are written by the build's own generator (bin/synth_gguf); their
SHA-256 is stored so the tests can prove they regenerated the same files.

Run: python tests/golden/make_golden.py   (needs /root/reference, in this container)
"""
import hashlib
import json
import os
import subprocess
import sys
import tempfile
import zlib

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(HERE))
from conftest import rand_blocks  # noqa: E402
import oracle_lib as ol  # noqa: E402
import gguf_read  # noqa: E402

SYNTH = os.path.join(ROOT, "oracle-engine_amd", "bin", "synth_gguf")
DRV = ol.REF_DRIVER
MODELS = ["t-q8", "t-q40", "t-q4k", "t-q4k-d", "t-q6k", "t-qwen", "t-qwen-d"]


def run(*args):
    r = subprocess.run([DRV, *map(str, args)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"ref_driver {args} failed: {r.stderr[-2000:]}")
    return r


def sha(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def main():
    out = {}
    tmp = tempfile.mkdtemp(prefix="orc_golden_")
    paths = {}
    for m in MODELS:
        p = os.path.join(tmp, m + ".gguf")
        subprocess.run([SYNTH, m, p], check=True, capture_output=True)
        paths[m] = p
        out[f"sha/{m}"] = np.frombuffer(sha(p).encode(), np.uint8)

    def f32(path):
        return np.fromfile(path, np.float32)

    def i32(path):
        return np.fromfile(path, np.int32)

    w = lambda name: os.path.join(tmp, name)  # noqa: E731

    # 1. codec hooks on random blocks
    rng = np.random.default_rng(2024)
    for name, qt in (("q4_0", ol.Q4_0), ("q4_k", ol.Q4_K), ("q6_k", ol.Q6_K)):
        n = 256 * 24
        raw = rand_blocks(qt, n, rng)
        raw.tofile(w("blk.bin"))
        run("dqhook", name, w("blk.bin"), n, w("dq.bin"))
        out[f"dq/{name}/raw"] = raw
        out[f"dq/{name}/out"] = f32(w("dq.bin"))
    # dequantize_row for Q8_0 (no hook) and the other types through real tensors
    for m, t in (("t-q8", "blk.0.attn_q.weight"), ("t-q4k", "blk.1.ffn_up.weight"), ("t-q4k", "token_embd.weight"),
                 ("t-q40", "blk.0.ffn_down.weight"), ("t-q6k", "output.weight")):
        run("dqrow", paths[m], t, 3, 4, w("row.bin"))
        out[f"dqrow/{m}/{t}"] = f32(w("row.bin"))

    # 2. gemv_q / gemm_q on every 2-D weight of four models (x ~ U(-1,1), seed 1234 as micro_gemm.cpp:88-91)
    for m in ("t-q4k", "t-qwen", "t-q8", "t-q40"):
        names = [f"{n} {sh[0]} {sh[1]}" for n, (_, sh, _) in sorted(gguf_read.tensors(paths[m]).items())
                 if len(sh) == 2]
        for line in names:
            t, n_in, n_out = line.split()
            xr = np.random.default_rng(1234).uniform(-1, 1, int(n_in)).astype(np.float32)
            xr.tofile(w("x.bin"))
            run("gemv", paths[m], t, w("x.bin"), w("y.bin"))
            out[f"gemv/{m}/{t}"] = f32(w("y.bin"))
        for t in ("blk.0.attn_q.weight", "blk.1.ffn_down.weight"):
            line = [ln for ln in names if ln.startswith(t + " ")][0]
            n_in = int(line.split()[1])
            X = np.random.default_rng(99).uniform(-1, 1, (5, n_in)).astype(np.float32)
            X.tofile(w("X.bin"))
            run("gemm", paths[m], t, w("X.bin"), 5, w("Y.bin"))
            out[f"gemm/{m}/{t}"] = f32(w("Y.bin"))

    # 3. decode / verify / spec loops
    for m in ("t-q8", "t-q40", "t-q4k", "t-q6k", "t-qwen"):
        prompt = np.random.default_rng(zlib.crc32(m.encode())).integers(0, 2048, 16).astype(np.int32)
        prompt.tofile(w("p.bin"))
        run("greedy", paths[m], w("p.bin"), 40, w("tok.bin"), w("lg.bin"), 4)
        out[f"greedy/{m}/prompt"] = prompt
        out[f"greedy/{m}/tokens"] = i32(w("tok.bin"))
        out[f"greedy/{m}/logits"] = f32(w("lg.bin")).reshape(4, -1)
        seq = np.concatenate([prompt, np.random.default_rng(5).integers(0, 2048, 5).astype(np.int32)])
        seq.tofile(w("s.bin"))
        run("batch", paths[m], w("s.bin"), 16, 5, w("blg.bin"))
        out[f"batch/{m}/tokens"] = seq
        out[f"batch/{m}/logits"] = f32(w("blg.bin")).reshape(5, -1)
    prompt = out["greedy/t-q4k/prompt"]
    for k in (2, 4):
        r = run("spec", paths["t-q4k"], paths["t-q4k-d"], _save(w("sp.bin"), prompt), 40, k, w("st.bin"))
        out[f"spec/k{k}/tokens"] = i32(w("st.bin"))
        out[f"spec/k{k}/stats"] = _stats(r)
    # stochastic engine loop, fixed seed
    qprompt = out["greedy/t-qwen/prompt"]
    r = run("espec", paths["t-qwen"], paths["t-qwen-d"], _save(w("qp.bin"), qprompt), 40, 3, 0.8, 0.95, 40, 1.1, 64,
            4242, w("es.bin"))
    out["espec/tokens"] = i32(w("es.bin"))
    out["espec/stats"] = _stats(r)

    # 4. sampler draws
    lg = np.random.default_rng(77).normal(0, 2, 3000).astype(np.float32)
    lg.tofile(w("lg.bin"))
    hist = np.random.default_rng(78).integers(0, 3000, 90).astype(np.int32)
    hist.tofile(w("h.bin"))
    out["sample/logits"] = lg
    out["sample/history"] = hist
    for i, (T, P, K, pen, last, seed) in enumerate([(0.8, 0.95, 40, 1.1, 64, 4242), (0.7, 0.9, 40, 1.15, 64, 1),
                                                    (1.0, 1.0, 0, 1.0, 64, 7), (0.0, 0.9, 40, 1.3, 16, 3),
                                                    (1.5, 0.5, 10, 1.1, 32, 2**40 + 5)]):
        run("sample", w("lg.bin"), T, P, K, pen, last, seed, w("h.bin"), 64, w("draw.bin"))
        out[f"sample/{i}/params"] = np.array([T, P, K, pen, last], np.float64)
        out[f"sample/{i}/seed"] = np.array([seed], np.uint64)
        out[f"sample/{i}/draws"] = i32(w("draw.bin"))

    # 5. ops
    x = np.random.default_rng(3).normal(0, 1.5, 3072).astype(np.float32)
    g = np.random.default_rng(4).uniform(0.5, 1.5, 3072).astype(np.float32)
    x.tofile(w("x.bin"))
    g.tofile(w("g.bin"))
    run("op", "rmsnorm", w("x.bin"), w("g.bin"), 1e-5, w("o.bin"))
    out["op/x"], out["op/g"], out["op/rmsnorm"] = x, g, f32(w("o.bin"))
    run("op", "softmax", w("x.bin"), w("o.bin"))
    out["op/softmax"] = f32(w("o.bin"))
    run("op", "silu", w("x.bin"), w("o.bin"))
    out["op/silu"] = f32(w("o.bin"))
    q = np.random.default_rng(8).normal(0, 1, 24 * 128).astype(np.float32)
    k = np.random.default_rng(9).normal(0, 1, 8 * 128).astype(np.float32)
    q.tofile(w("q.bin"))
    k.tofile(w("k.bin"))
    run("op", "rope", w("q.bin"), w("k.bin"), 24, 8, 128, 301, 500000, w("oq.bin"), w("ok.bin"))
    out["op/rope_q_in"], out["op/rope_k_in"] = q, k
    out["op/rope_q"], out["op/rope_k"] = f32(w("oq.bin")), f32(w("ok.bin"))

    dst = os.path.join(HERE, "ref_fixtures.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst}: {len(out)} arrays, {os.path.getsize(dst) / 1e6:.2f} MB")


def _stats(r):
    d = json.loads(r.stderr.strip().splitlines()[-1])
    return np.array([d["accepted"], d["proposed"], d["passes"]], np.int64)


def _save(path, arr):
    np.ascontiguousarray(arr, np.int32).tofile(path)
    return path


if __name__ == "__main__":
    main()
