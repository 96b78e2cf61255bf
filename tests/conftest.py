import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "oracle-engine_amd")
sys.path.insert(0, os.path.join(PKG, "python"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import oracle_lib  # noqa: E402

SYNTH = os.path.join(PKG, "bin", "synth_gguf")
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")


def _ensure_oracle():
    if not os.path.exists(oracle_lib.ORACLE_SO):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "oracle"], check=True)


@pytest.fixture(scope="session")
def oracle():
    _ensure_oracle()
    return oracle_lib.Oracle()


@pytest.fixture(scope="session")
def models_dir(tmp_path_factory):
    """Small synthetic GGUF models written by the product's own generator."""
    if not os.path.exists(SYNTH):
        pytest.fail(f"{SYNTH} missing: run __graft_entry__.build()")
    d = tmp_path_factory.mktemp("models")
    for name in ("t-q8", "t-q40", "t-q4k", "t-q4k-d", "t-q6k", "t-qwen", "t-qwen-d", "t-dense", "t-q8-a64",
                 "t-qwen3"):
        subprocess.run([SYNTH, name, str(d / f"{name}.gguf")], check=True, capture_output=True)
    return d


@pytest.fixture(scope="session")
def dev():
    import orc

    print(f"[gpu] opening device 0", flush=True)
    return orc.Device(0)


def rand_blocks(qtype, n_el, rng):
    """Random but valid GGML blocks: every code pattern, finite fp16 scales."""
    be, bb = oracle_lib.BLOCK[qtype]
    nb = n_el // be
    raw = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)

    def f16(lo, hi, size):
        return rng.uniform(lo, hi, size=size).astype(np.float16).view(np.uint8).reshape(-1, 2)

    if qtype in (oracle_lib.Q8_0, oracle_lib.Q4_0):
        raw[:, 0:2] = f16(-0.004, 0.004, nb)
    elif qtype == oracle_lib.Q4_K:
        raw[:, 0:2] = f16(0.0, 0.002, nb)
        raw[:, 2:4] = f16(0.0, 0.004, nb)
    elif qtype == oracle_lib.Q6_K:
        raw[:, 208:210] = f16(0.0, 0.0005, nb)
    elif qtype == oracle_lib.F16:
        raw = f16(-1, 1, n_el).reshape(nb, bb)
    return raw.reshape(-1)
