"""The reference API on a loaded model, beyond the decode loops:

* model.gguf().gemv_q / gemv_q_range / gemm_q / dequantize_row read every
  tensor in the layout its HBM bytes hold after Model::load — including the
  Q8_0 matrices the load regroups into the aligned ORC_Q8_0_X8 layout — and
  match the reference's outputs (tests/golden/ref_fixtures.npz: gemv_q of
  every weight within 1e-3, gemm_q of 5 tokens, dequantize_row bit-exact);
* token ids outside [0, n_vocab) are read as id 0 (core/model.cpp:352-356,
  552-556), through Model::forward, forward_batch and the embedding gather;
* argument errors come back as errors: a prompt longer than the context, a
  draft context longer than the target's in the Engine loop, top_k = 0 (all
  tokens) on a vocabulary larger than the device sampler's candidate sort.
"""
import os

import numpy as np
import pytest

import oracle_lib as ol
from conftest import GOLDEN

pytestmark = pytest.mark.gpu
FIX = np.load(os.path.join(GOLDEN, "ref_fixtures.npz"))


@pytest.fixture(scope="module")
def q8(models_dir):
    import orc

    print("[gpu] loading t-q8 (regrouped Q8_0 layers)", flush=True)
    m = orc.Model(models_dir / "t-q8.gguf")
    yield m
    m.close()


def _shape(models_dir, m, t):
    import gguf_read

    return gguf_read.tensors(str(models_dir / f"{m}.gguf"))[t][1]


def test_regrouped_tensors_report_their_layout(q8):
    assert q8.gguf_device_type("blk.0.attn_q.weight") == 258  # ORC_Q8_0_X8
    assert q8.gguf_device_type("blk.1.ffn_down.weight") == 258
    assert q8.gguf_device_type("token_embd.weight") == ol.Q8_0  # the row gather keeps the file layout
    assert q8.gguf_device_type("blk.0.attn_norm.weight") == ol.F32
    assert q8.gguf_device_type("no.such.tensor") == -1


@pytest.mark.parametrize("m", ["t-q8", "t-q4k"])
def test_parser_gemv_matches_reference_after_load(models_dir, m):
    """gemv_q through the model's own parser on every fixture tensor."""
    import orc

    print(f"[gpu] parser gemv_q on {m}", flush=True)
    mod = orc.Model(models_dir / f"{m}.gguf")
    try:
        worst = 0.0
        keys = [k for k in FIX.files if k.startswith(f"gemv/{m}/")]
        assert keys
        for key in keys:
            t = key.split("/", 2)[2]
            n_in, n_out = _shape(models_dir, m, t)
            x = np.random.default_rng(1234).uniform(-1, 1, n_in).astype(np.float32)
            got = mod.gguf_gemv(t, x, n_out=n_out)
            ref = FIX[key]
            err = np.abs(got - ref).max() / np.abs(ref).max()
            worst = max(worst, err)
            assert err <= 1e-3, (key, err)
            # a row range [j0, j1) is the same rows of the full result
            j0, j1 = 3, min(n_out, 3 + 37)
            sub = mod.gguf_gemv(t, x, j0=j0, j1=j1)
            assert np.array_equal(sub.view(np.uint32), got[j0:j1].view(np.uint32)), key
        print(f"[gpu] {m}: worst parser gemv_q error vs reference {worst:.2e}", flush=True)
    finally:
        mod.close()


@pytest.mark.parametrize("m", ["t-q8", "t-q4k"])
def test_parser_gemm_matches_reference_after_load(models_dir, m):
    import orc

    print(f"[gpu] parser gemm_q on {m}", flush=True)
    mod = orc.Model(models_dir / f"{m}.gguf")
    try:
        for t in ("blk.0.attn_q.weight", "blk.1.ffn_down.weight"):
            n_in, n_out = _shape(models_dir, m, t)
            X = np.random.default_rng(99).uniform(-1, 1, (5, n_in)).astype(np.float32)
            got = mod.gguf_gemm(t, X, n_out)
            ref = FIX[f"gemm/{m}/{t}"].reshape(5, n_out)
            err = np.abs(got - ref).max() / np.abs(ref).max()
            assert err <= 1e-3, (m, t, err)
    finally:
        mod.close()


def test_parser_dequantize_row_bit_exact_after_load(q8, models_dir):
    t = "blk.0.attn_q.weight"
    n_in, _ = _shape(models_dir, "t-q8", t)
    rows = np.concatenate([q8.gguf_dequant_row(t, r, n_in) for r in range(3, 7)])
    assert np.array_equal(rows.view(np.uint32), FIX[f"dqrow/t-q8/{t}"].view(np.uint32))


def test_out_of_range_ids_read_token_zero(q8):
    """core/model.cpp:352-356 (forward) and 552-556 (forward_prefill)."""
    V = q8.n_vocab
    prompt = np.array([5, 17, 99, 3], np.int32)
    ref = []
    for bad in (0, V, V + 7, -1, -100000):
        q8.reset()
        q8.forward_batch(prompt, 0, logits=False)
        ref.append(q8.forward(bad, len(prompt)))
    for lg in ref[1:]:
        assert np.array_equal(lg.view(np.uint32), ref[0].view(np.uint32))
    q8.reset()
    batch = q8.forward_batch(np.array([5, V + 3, 17, -2], np.int32), 0)
    q8.reset()
    want = q8.forward_batch(np.array([5, 0, 17, 0], np.int32), 0)
    assert np.array_equal(batch.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("m", ["t-q8", "t-q4k", "t-q6k"])
def test_embed_gather_clamps_ids(dev, oracle, models_dir, m):
    """orc_embed: row ids[t] of the table, bit-exact with the oracle's codec;
    ids outside [0, n_rows) read row 0."""
    import gguf_read

    tt, (n_in, n_rows), off = gguf_read.tensors(str(models_dir / f"{m}.gguf"))["token_embd.weight"]
    rb = ol.row_bytes(tt, n_in)
    raw = np.fromfile(models_dir / f"{m}.gguf", np.uint8, count=rb * n_rows, offset=off)
    ids = np.array([0, n_rows - 1, n_rows, -1, 2**31 - 1, 7], np.int32)
    dt, di, dy = dev.upload(raw), dev.upload(ids), dev.alloc(len(ids) * n_in * 4)
    dev.check(dev.L.orc_embed(tt, dt.ptr, n_in, n_rows, di.ptr, len(ids), dy.ptr, n_in, None))
    got = dy.read(np.float32).reshape(len(ids), n_in)
    for r, w in enumerate([0, n_rows - 1, 0, 0, 0, 7]):
        ref = oracle.dequant(tt, raw[w * rb:(w + 1) * rb], n_in)
        assert np.array_equal(got[r].view(np.uint32), ref.view(np.uint32)), (m, r)


def test_prompt_longer_than_context_is_an_error(models_dir):
    import orc

    m = orc.Model(models_dir / "t-q4k.gguf", 64)
    try:
        with pytest.raises(orc.OrcError, match="context"):
            m.greedy(np.arange(65, dtype=np.int32), 4)
        # a prompt that fits still decodes afterwards
        assert len(m.greedy(np.arange(40, dtype=np.int32), 4)) == 4
    finally:
        m.close()


def test_engine_loop_rejects_a_longer_draft_context(models_dir):
    import orc

    tgt, dft = orc.Model(models_dir / "t-qwen.gguf", 256), orc.Model(models_dir / "t-qwen-d.gguf", 300)
    try:
        with pytest.raises(orc.OrcError, match="draft context"):
            tgt.spec_engine(dft, np.arange(16, dtype=np.int32), 8, 3)
    finally:
        tgt.close()
        dft.close()


def test_all_tokens_top_k_refuses_large_vocabulary(dev):
    import ctypes as C

    V = 20000
    st = dev.alloc(dev.L.orc_sampler_state_bytes())
    x = np.random.default_rng(5).normal(size=V).astype(np.float32)
    lg = dev.upload(x)
    out = dev.alloc(16)
    dev.check(dev.L.orc_sampler_init(st.ptr, C.c_float(0.8), C.c_float(0.95), 0, C.c_float(1.1), 64, 42, None, 0,
                                     None))
    rc = dev.L.orc_sample(st.ptr, lg.ptr, V, out.ptr, None)
    assert rc == -2, rc  # ORC_E_UNSUPPORTED
    assert b"top_k = 0" in dev.L.orc_last_error()
    # a vocabulary within the candidate sort is sampled
    dev.check(dev.L.orc_sample(st.ptr, lg.ptr, 16384, out.ptr, None))
    # and the same state re-initialised with top_k = 40 samples the large one
    dev.check(dev.L.orc_sampler_init(st.ptr, C.c_float(0.8), C.c_float(0.95), 40, C.c_float(1.1), 64, 42, None, 0,
                                     None))
    dev.check(dev.L.orc_sample(st.ptr, lg.ptr, V, out.ptr, None))
    # T = 0 is the argmax (sampler.cpp:50): top_k = 0 sorts nothing then, so any vocabulary works
    dev.check(dev.L.orc_sampler_init(st.ptr, C.c_float(0.0), C.c_float(0.95), 0, C.c_float(1.0), 64, 42, None, 0,
                                     None))
    lg = dev.upload(x)  # orc_sample leaves probabilities in the row it sampled
    dev.check(dev.L.orc_sample(st.ptr, lg.ptr, V, out.ptr, None))
    assert int(out.read(np.int32, 1)[0]) == int(np.argmax(x))
    assert 0 <= int(out.read(np.int32, 1)[0]) < V


def test_alignment_64_file_decodes_as_its_32_byte_twin(models_dir):
    """t-q8-a64 declares general.alignment = 64 (the t-q8 tensors): the
    device path reads it at the declared alignment, so greedy tokens and the
    decode logits equal t-q8's bit for bit."""
    import orc

    print("[gpu] general.alignment = 64", flush=True)
    prompt = np.array([5, 17, 99, 3, 1000, 42], np.int32)
    outs = []
    for name in ("t-q8", "t-q8-a64"):
        m = orc.Model(models_dir / f"{name}.gguf")
        toks = m.greedy(prompt, 12)
        m.reset()
        m.forward_batch(prompt[:-1], 0, logits=False)
        outs.append((toks, m.forward(int(prompt[-1]), len(prompt) - 1)))
        m.close()
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32))
