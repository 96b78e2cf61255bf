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

The timed region replays captured HIP graphs (one per spec round; positions
live on the device; --no-graphs launches every kernel from the host).
roofline: right after it, a kernel timing pass runs the same spec rounds
launched from the host for --prof-tokens tokens, every GEMM launch carrying
start / stop HIP events that take the timestamps of its own dispatch on its
stream (hipExtLaunchKernelGGL). The dominant kernel family is the one with
the most GEMM time there; achieved = algorithmic bytes (weight blocks +
activations + outputs) / its average launch duration. traffic: that kernel
family's HBM bytes per launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE
runs (scaled by a copy kernel of known size), read from the committed
summary in profiles/.
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
TYPE_NAMES = {2: "Q4_0", 8: "Q8_0", 12: "Q4_K", 14: "Q6_K", 256: "Q4_K|Q6_K"}


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


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (profiles/*.md, a 'TRAFFIC <kernel> bytes_per_launch=N' line), scaled there by a copy kernel."""
    pdir = os.path.join(ROOT, "profiles")
    for name in sorted(os.listdir(pdir)) if os.path.isdir(pdir) else []:
        if name.endswith(".md"):
            for line in open(os.path.join(pdir, name)):
                m = re.match(r"TRAFFIC (.+) bytes_per_launch=(\d+)\s*$", line)
                if m and m.group(1) == kernel:
                    return int(m.group(2)), f"profiles/{name}"
    return None, None


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
    ap.add_argument("--prof-tokens", type=int, default=64, help="tokens generated by the kernel timing pass")
    ap.add_argument("--no-graphs", action="store_true",
                    help="launch every kernel from the host instead of replaying captured graphs")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB (a kernel of known HBM traffic that "
                         "calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
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
    if a.calib_copy_mb > 0:
        nb = a.calib_copy_mb << 20
        src, dst = dev.alloc(nb), dev.alloc(nb)
        dev.check(dev.L.orc_fill(src.ptr, 1, nb, None))
        dev.sync()
        dev.check(dev.L.orc_memcpy_d2d(dst.ptr, src.ptr, nb, None))
        dev.sync()
        log(f"calibration copy: {nb} bytes device to device")
        src.free()
        dst.free()
    t0 = time.time()
    tgt = orc.Model(tgt_path, a.ctx)
    dft = orc.Model(dft_path, a.ctx)
    log(f"loaded target ({tgt.weight_bytes() / 1e9:.3f} GB/token) and draft ({dft.weight_bytes() / 1e9:.3f} "
        f"GB/token) in {time.time() - t0:.1f}s")
    prompt = np.random.default_rng(1234).integers(0, tgt.n_vocab, a.n_prompt).astype(np.int32)
    if a.no_graphs:
        orc.load_host_lib().orch_set_graphs(0)

    greedy = tgt.greedy(prompt, a.n_gen, prefill=True)  # reference stream for the exactness check
    toks, st = tgt.spec_greedy(dft, prompt, a.n_gen, a.k, prefill=True)  # prefills both models
    exact = bool(np.array_equal(toks, greedy))
    # the reference implementation's own streams on these models (tests/golden/c3_ref.npz)
    ref_identical = None
    fix_path = os.path.join(ROOT, "tests", "golden", "c3_ref.npz")
    if os.path.exists(fix_path):
        fix = np.load(fix_path)
        if (a.n_prompt, a.n_gen, a.k) == (len(fix["prompt"]), len(fix["spec_tokens"]), int(fix["k"][0])) and \
                np.array_equal(prompt, fix["prompt"]):
            ref_identical = bool(np.array_equal(greedy, fix["greedy_tokens"]) and
                                 np.array_equal(toks, fix["spec_tokens"]) and
                                 (st["accepted"], st["proposed"], st["passes"]) == tuple(int(v) for v in fix["spec_stats"]))
    for _ in range(a.warmup):
        toks, st = tgt.spec_greedy(dft, prompt, a.n_gen, a.k, prefill=False)
        exact &= bool(np.array_equal(toks, greedy))

    L, H = orc.load_hip_lib(), orc.load_host_lib()
    tot = {"accepted": 0, "proposed": 0, "passes": 0, "rounds": 0}
    H.orch_sync()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        toks, st = tgt.spec_greedy(dft, prompt, a.n_gen, a.k, prefill=False)
        exact &= bool(np.array_equal(toks, greedy))
        for key in tot:
            tot[key] += st[key]
    H.orch_sync()
    dt = time.perf_counter() - t0
    value = a.steps * a.n_gen / dt

    roofline, fams = None, []
    if not a.no_prof:
        import ctypes as C

        # Kernel timing pass right after the timed region: the same spec
        # rounds launched from the host, every GEMM launch carrying start /
        # stop HIP events taken from its own dispatch on its stream.
        L.orc_prof_enable(1)
        H.orch_set_graphs(0)
        tp = time.perf_counter()
        try:
            ptoks, pst = tgt.spec_greedy(dft, prompt, a.prof_tokens, a.k, prefill=False)
            exact &= bool(np.array_equal(ptoks, greedy[:len(ptoks)]))
            H.orch_sync()
            if L.orc_prof_accumulate():
                raise orc.OrcError(L.orc_last_error().decode())
        except orc.OrcError as e:
            log(f"kernel timing pass failed: {e}")
            pst = None
        prof_dt = time.perf_counter() - tp
        L.orc_prof_enable(0)
        H.orch_set_graphs(0 if a.no_graphs else 1)
        for ty in ((2, 8, 12, 14, 256) if pst else ()):
            for nt in range(1, 6):
                n, ms, by = C.c_int64(), C.c_double(), C.c_double()
                L.orc_prof_read(ty, nt, C.byref(n), C.byref(ms), C.byref(by))
                if n.value:
                    fams.append({"kernel": f"k_gemm {TYPE_NAMES[ty]} n_tok={nt}", "launches": n.value,
                                 "ms": ms.value, "bytes": by.value, "gbs": by.value / (ms.value * 1e-3) / 1e9})
        fams.sort(key=lambda f: -f["ms"])
        if fams:
            f = fams[0]
            traffic, traffic_src = measured_traffic(f["kernel"])
            roofline = {"bound": "hbm", "achieved": round(f["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(f["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                        "traffic_source": traffic_src, "kernel": f["kernel"],
                        "avg_launch_us": round(1e3 * f["ms"] / f["launches"], 3),
                        "bytes_per_launch": round(f["bytes"] / f["launches"]),
                        "timing": f"start/stop HIP events of each launch's dispatch over {pst['rounds']} "
                                  f"host-launched spec rounds"}

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
        "exact_vs_greedy": exact, "reference_stream_identical": ref_identical,
        "roofline": roofline, "cpu_baseline": cpu,
        "kernel_families": [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in f.items()} for f in fams],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
