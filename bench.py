#!/usr/bin/env python3
"""bench.py — speculative-decoding throughput of the ORACLE hot path on one MI355X.

Workload (the metric's config): target = Llama-3.2-3B
shape, Q4_K_M mix (Q6_K attn_v / ffn_down / tied head), random-init N(0, 0.02);
draft = Q8_0 model built from the target's float layers 0-7 with a Q8_0 copy of
its embedding / head; greedy speculative decoding with k = 4; prompt of 128
uniform-random ids; 256 generated tokens; ctx 2048. Both models are generated
by the build's own writer (bin/synth_gguf) and uploaded as raw GGUF blocks.

A step is one full generation of 256 tokens from the prefilled prompt (the
prefill of both models is done once, untimed, as the reference harness does:
benchmark/bench_engine.cpp:300-310). `value` is generated tokens per second
over the K timed steps; every step's token stream is checked against the
target's plain greedy stream (spec decode must be exact).

roofline: the dominant kernel family (most GPU time in the timed region) is
timed live with HIP events around each of its launches on its stream;
achieved = algorithmic bytes (weight blocks + activations) / kernel time.
cpu_baseline: the reference implementation (oracle/_ref, built from the
reference's sources) on the same two models, bounded sample: prompt 8 ids,
16 generated tokens, k = 4.
"""
import argparse
import json
import os
import re
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "oracle-engine_amd")
sys.path.insert(0, os.path.join(PKG, "python"))

SYNTH = os.path.join(PKG, "bin", "synth_gguf")
REF_DRIVER = os.path.join(ROOT, "oracle", "_ref", "ref_driver")
HBM_PEAK_GBS = 8000.0
TYPE_NAMES = {2: "Q4_0", 8: "Q8_0", 12: "Q4_K", 14: "Q6_K"}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def ensure_model(name, models_dir):
    path = os.path.join(models_dir, f"{name}.gguf")
    if not os.path.exists(path):
        os.makedirs(models_dir, exist_ok=True)
        t0 = time.time()
        subprocess.run([SYNTH, name, path], check=True)
        log(f"generated {name} in {time.time() - t0:.1f}s")
    return path


def cpu_baseline(tgt_path, dft_path, prompt, k):
    if not os.path.exists(REF_DRIVER):
        return None
    threads = min(16, os.cpu_count() or 1)
    p = os.path.join(os.path.dirname(tgt_path), "cpu_prompt.bin")
    np.ascontiguousarray(prompt[:8], np.int32).tofile(p)
    log(f"cpu baseline: reference build, {threads} threads, prompt 8, 16 tokens, k={k}")
    r = subprocess.run([REF_DRIVER, "bench", tgt_path, dft_path, p, "16", str(k), str(threads)],
                       capture_output=True, text=True, timeout=900)
    m = re.search(r"REF_BENCH (\{.*\})", r.stderr)
    if r.returncode != 0 or not m:
        log(f"cpu baseline failed: {r.stderr[-500:]}")
        return None
    d = json.loads(m.group(1))
    return {"value": round(d["tok_s"], 4), "unit": "tok/s", "cores": d["threads"], "kind": "reference",
            "sample": f"reference build (oracle/_ref), same C3 target+draft, prompt 8 ids, {d['tokens']} generated "
                      f"tokens, k={k}, accepted {d['accepted']}/{d['proposed']}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--n-gen", type=int, default=256)
    ap.add_argument("--n-prompt", type=int, default=128)
    ap.add_argument("--k", type=int, default=4)
    ap.add_argument("--ctx", type=int, default=2048)
    ap.add_argument("--models-dir", default=os.environ.get("ORC_MODEL_DIR", "/tmp/orc_models"))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prof", action="store_true", help="skip the live per-kernel event timing")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {a.gpus}); this build has no multi-GPU path.",
              file=sys.stderr)
        sys.exit(2)

    import orc

    tgt_path = ensure_model("c2", a.models_dir)
    dft_path = ensure_model("c3d", a.models_dir)
    dev = orc.Device(0)
    name, n_cu, hbm = dev.info()
    log(f"device {name}, {n_cu} CUs, {hbm / 1e9:.0f} GB")
    t0 = time.time()
    tgt = orc.Model(tgt_path, a.ctx)
    dft = orc.Model(dft_path, a.ctx)
    log(f"loaded target ({tgt.weight_bytes() / 1e9:.3f} GB/token) and draft ({dft.weight_bytes() / 1e9:.3f} "
        f"GB/token) in {time.time() - t0:.1f}s")
    prompt = np.random.default_rng(1234).integers(0, tgt.n_vocab, a.n_prompt).astype(np.int32)

    greedy = tgt.greedy(prompt, a.n_gen, prefill=True)  # reference stream for the exactness check
    toks, st = tgt.spec_greedy(dft, prompt, a.n_gen, a.k, prefill=True)  # prefills both models
    exact = bool(np.array_equal(toks, greedy))
    for _ in range(a.warmup):
        toks, st = tgt.spec_greedy(dft, prompt, a.n_gen, a.k, prefill=False)
        exact &= bool(np.array_equal(toks, greedy))

    L = orc.load_hip_lib()
    if not a.no_prof:
        L.orc_prof_enable(1)
    tot = {"accepted": 0, "proposed": 0, "passes": 0, "rounds": 0}
    orc.load_host_lib().orch_sync()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        toks, st = tgt.spec_greedy(dft, prompt, a.n_gen, a.k, prefill=False)
        exact &= bool(np.array_equal(toks, greedy))
        for key in tot:
            tot[key] += st[key]
    orc.load_host_lib().orch_sync()
    dt = time.perf_counter() - t0
    L.orc_prof_enable(0)
    value = a.steps * a.n_gen / dt

    roofline, fams = None, []
    if not a.no_prof:
        import ctypes as C

        for ty in (2, 8, 12, 14):
            for nt in range(1, 6):
                n, ms, by = C.c_int64(), C.c_double(), C.c_double()
                L.orc_prof_read(ty, nt, C.byref(n), C.byref(ms), C.byref(by))
                if n.value:
                    fams.append({"kernel": f"k_gemm {TYPE_NAMES[ty]} n_tok={nt}", "launches": n.value,
                                 "ms": ms.value, "bytes": by.value, "gbs": by.value / (ms.value * 1e-3) / 1e9})
        fams.sort(key=lambda f: -f["ms"])
        if fams:
            f = fams[0]
            roofline = {"bound": "hbm", "achieved": round(f["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(f["gbs"] / HBM_PEAK_GBS, 4), "traffic": None, "kernel": f["kernel"],
                        "avg_launch_us": round(1e3 * f["ms"] / f["launches"], 3),
                        "bytes_per_launch": round(f["bytes"] / f["launches"]), "gemm_share_of_step":
                            round(sum(x["ms"] for x in fams) / (dt * 1e3), 4)}

    cpu = None if a.no_cpu_baseline else cpu_baseline(tgt_path, dft_path, prompt, a.k)
    out = {
        "metric": "spec-decode tok/s (3B Q4_K, k=4); quant-GEMV HBM GB/s vs peak",
        "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(1e3 * dt / a.steps, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (random-init N(0,0.02) GGUF, uniform random prompt ids)",
        "config": {"workload": "C3 spec greedy: 3B-shape Q4_K_M target + 8-layer Q8_0 draft",
                   "k": a.k, "prompt": a.n_prompt, "gen_tokens": a.n_gen, "ctx": a.ctx},
        "acceptance": round(tot["accepted"] / max(1, tot["proposed"]), 4),
        "target_passes_per_token": round(tot["passes"] / max(1, a.steps * a.n_gen), 4),
        "exact_vs_greedy": exact,
        "roofline": roofline, "cpu_baseline": cpu,
        "kernel_families": [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in f.items()} for f in fams],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
