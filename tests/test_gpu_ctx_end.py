"""Speculative loops run into the end of the 512-position context on the
device: the draft proposes fewer than k tokens once pos + k reaches the last
position, and the bonus token (with the Engine's extra target pass) is
withheld at the end (benchmark/bench_engine.cpp:310-356, core/engine.cpp:
140-240). Token streams and accepted / proposed / pass counts equal the
REFERENCE's (tests/golden/ctx_end_ref.npz, written by
tests/golden/make_golden_ctx_end.py), with captured graphs and with
host-launched rounds."""
import os

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu
FIX = np.load(os.path.join(GOLDEN, "ctx_end_ref.npz"))


@pytest.fixture(scope="module")
def cmodels(models_dir):
    import orc

    cache = {}

    def get(name):
        if name not in cache:
            print(f"[gpu] loading {name} ctx=512", flush=True)
            cache[name] = orc.Model(models_dir / f"{name}.gguf", 512)
        return cache[name]

    yield get
    for m in cache.values():
        m.close()


def _graphs(on):
    import orc

    return orc.load_host_lib().orch_set_graphs(int(on))


@pytest.mark.parametrize("graphs", [True, False])
@pytest.mark.parametrize("k", [2, 3, 4])
def test_spec_greedy_context_end(cmodels, k, graphs):
    print(f"[gpu] ctx-end spec greedy k={k} graphs={graphs}", flush=True)
    tgt, dft = cmodels("t-q4k"), cmodels("t-q4k-d")
    prev = _graphs(graphs)
    try:
        toks, st = tgt.spec_greedy(dft, FIX[f"spec/k{k}/prompt"], 64, k)
    finally:
        _graphs(prev)
    assert np.array_equal(toks, FIX[f"spec/k{k}/tokens"])
    assert [st["accepted"], st["proposed"], st["passes"]] == list(FIX[f"spec/k{k}/stats"])


@pytest.mark.parametrize("graphs", [True, False])
def test_engine_spec_context_end(cmodels, graphs):
    print(f"[gpu] ctx-end Engine spec graphs={graphs}", flush=True)
    tgt, dft = cmodels("t-qwen"), cmodels("t-qwen-d")
    prev = _graphs(graphs)
    try:
        toks, st = tgt.spec_engine(dft, FIX["espec/prompt"], 40, 3, 0.8, 0.95, 40, 1.1, 64, 4242)
    finally:
        _graphs(prev)
    assert np.array_equal(toks, FIX["espec/tokens"])
    assert [st["accepted"], st["proposed"], st["passes"]] == list(FIX["espec/stats"])


@pytest.mark.parametrize("graphs", [True, False])
@pytest.mark.parametrize("name", ["draft_longer", "draft_shorter"])
def test_spec_greedy_unequal_contexts(models_dir, name, graphs):
    """Target and draft of different context lengths: the draft's bounds the
    proposals, the target's the verify width (bench_engine.cpp:313-323); when
    the target's context cuts the verify pass short, the last round compares
    fewer drafts than it proposed and emits no bonus."""
    import orc

    tc, dc, k = (int(v) for v in FIX[f"uneq/{name}/cfg"])
    print(f"[gpu] unequal contexts {name}: target {tc}, draft {dc}, k={k}, graphs={graphs}", flush=True)
    tgt, dft = orc.Model(models_dir / "t-q4k.gguf", tc), orc.Model(models_dir / "t-q4k-d.gguf", dc)
    prev = _graphs(graphs)
    try:
        toks, st = tgt.spec_greedy(dft, FIX[f"uneq/{name}/prompt"], 64, k)
    finally:
        _graphs(prev)
        tgt.close()
        dft.close()
    assert np.array_equal(toks, FIX[f"uneq/{name}/tokens"])
    assert [st["accepted"], st["proposed"], st["passes"]] == list(FIX[f"uneq/{name}/stats"])
