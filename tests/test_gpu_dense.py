"""Dense weight matrices (F32, F16, BF16) on the device path, against the
reference's own outputs on the t-dense model (tests/golden/dense_ref.npz,
written by make_golden_dense.py from the reference build).

The reference accepts these types at load (core/gguf_parser.cpp:96-110) and
runs them through its fallback, dequantize + ops::matmul (core/model.cpp:
370-381, and the same for o / gate / up / down / head); the build runs them
on the vector GEMV with the values widened exactly to fp32. t-dense has an
F16 token embedding, a BF16 LM head, an all-F32 layer 0 and a Q8_0 layer 1
whose attn_norm is declared F16 while its bytes are F32 norm weights: like
the reference (core/model.cpp:317-320) the build reads a norm's bytes as F32
whatever the declared type.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu
FIX = np.load(os.path.join(GOLDEN, "dense_ref.npz"))


@pytest.fixture(scope="module")
def dense(models_dir):
    import orc

    print("[gpu] loading t-dense", flush=True)
    m = orc.Model(models_dir / "t-dense.gguf")
    yield m
    m.close()


def test_dense_greedy_stream_matches_reference(dense):
    print("[gpu] t-dense greedy", flush=True)
    toks = dense.greedy(FIX["greedy/prompt"], 40)
    assert np.array_equal(toks, FIX["greedy/tokens"])


def test_dense_decode_and_verify_logits_match_reference(dense):
    print("[gpu] t-dense logits", flush=True)
    prompt = FIX["greedy/prompt"]
    dense.reset()
    dense.forward_batch(prompt[:-1], 0, logits=False)
    cur, pos = int(prompt[-1]), len(prompt) - 1
    for s in range(4):
        lg = dense.forward(cur, pos)
        ref = FIX["greedy/logits"][s]
        assert np.abs(lg - ref).max() <= 1e-4 * np.abs(ref).max(), s
        cur, pos = int(np.argmax(lg)), pos + 1
    seq = FIX["batch/tokens"]
    dense.reset()
    dense.forward_batch(seq[:16], 0, logits=False)
    lg = dense.forward_batch(seq[16:], 16)
    ref = FIX["batch/logits"]
    assert np.abs(lg - ref).max() <= 1e-4 * np.abs(ref).max()
    # dense and Q8_0 matrices run one kernel family at every token count:
    # the 5-token verify equals five decodes bit for bit
    dense.reset()
    dense.forward_batch(seq[:16], 0, logits=False)
    one = np.stack([dense.forward(int(t), 16 + i) for i, t in enumerate(seq[16:])])
    assert np.array_equal(one.view(np.uint32), lg.view(np.uint32))


@pytest.mark.parametrize("t", ["token_embd.weight", "output.weight", "blk.0.ffn_down.weight"])
def test_dense_dequantize_row_bit_exact(dense, t):
    n_in = FIX[f"dqrow/{t}"].size // 4
    rows = np.concatenate([dense.gguf_dequant_row(t, r, n_in) for r in range(3, 7)])
    assert np.array_equal(rows.view(np.uint32), FIX[f"dqrow/{t}"].view(np.uint32))


def test_dense_gemm_matches_float64(dev):
    """orc_gemm on F32 / F16 / BF16 rows: every (token, row) within 2e-6 of
    sum |w x| of the float64 product of the exactly widened values, the
    same at 1 and at 5 tokens bit for bit."""
    import ctypes as C

    rng = np.random.default_rng(41)
    n_out, n_in = 77, 3072
    W = rng.normal(0, 0.02, (n_out, n_in)).astype(np.float32)
    X = rng.normal(0, 1, (5, n_in)).astype(np.float32)
    for ty, raw, wide in ((0, W, W),
                          (1, W.astype(np.float16), W.astype(np.float16).astype(np.float32)),
                          (30, (W.view(np.uint32) >> 16).astype(np.uint16),
                           ((W.view(np.uint32) >> 16) << 16).view(np.float32))):
        print(f"[gpu] dense gemm type={ty}", flush=True)
        wd, xd, yd = dev.upload(np.ascontiguousarray(raw)), dev.upload(X), dev.alloc(4 * 5 * n_out)
        dev.check(dev.L.orc_gemm(ty, wd.ptr, 5, n_out, n_in, xd.ptr, n_in, yd.ptr, n_out, None))
        got = yd.read(np.float32).reshape(5, n_out)
        exact = X.astype(np.float64) @ wide.astype(np.float64).T
        scale = np.abs(X.astype(np.float64)) @ np.abs(wide.astype(np.float64)).T
        assert np.all(np.abs(got - exact) <= 2e-6 * scale), ty
        for t in range(5):
            dev.check(dev.L.orc_gemm(ty, wd.ptr, 1, n_out, n_in, C.c_void_p(xd.ptr + 4 * t * n_in), n_in, yd.ptr,
                                     n_out, None))
            assert np.array_equal(yd.read(np.float32, n_out).view(np.uint32), got[t].view(np.uint32)), (ty, t)
