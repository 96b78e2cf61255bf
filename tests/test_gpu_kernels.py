"""Parity of the HIP kernels (through the C ABI) against the CPU oracle.

Bars: dequant bit-exact; GEMV within 2e-6 of sum|w*x| of the float64 result
and 1e-3 relative (norm-wise) of the oracle's fp32 gemv; the tokens of an
n-token GEMM independent bit for bit (and, for Q8_0 / Q4_0, bit-identical to n
separate GEMVs); elementwise ops within 1e-6 relative.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as ol
from conftest import rand_blocks

pytestmark = pytest.mark.gpu

TYPES = [ol.Q4_K, ol.Q6_K, ol.Q8_0, ol.Q4_0]
_libm = C.CDLL("libm.so.6")
_libm.powf.restype = C.c_float
_libm.powf.argtypes = [C.c_float, C.c_float]
_libm.cosf.restype = C.c_float
_libm.cosf.argtypes = [C.c_float]
_libm.sinf.restype = C.c_float
_libm.sinf.argtypes = [C.c_float]


def rope_table(max_pos, hd, base):
    """cos/sin pairs with the reference's float powf/cosf/sinf (ops.cpp:461-466)."""
    half = hd // 2
    t = np.zeros((max_pos, half, 2), np.float32)
    inv = [np.float32(_libm.powf(C.c_float(base), C.c_float(np.float32(2 * i) / np.float32(hd)))) for i in range(half)]
    for p in range(max_pos):
        for i in range(half):
            th = np.float32(np.float32(p) / inv[i])
            t[p, i, 0] = _libm.cosf(C.c_float(th))
            t[p, i, 1] = _libm.sinf(C.c_float(th))
    return t


@pytest.mark.parametrize("qt", TYPES + [ol.F16])
def test_dequant_bitexact(dev, oracle, qt):
    print(f"[gpu] dequant type={qt}", flush=True)
    rng = np.random.default_rng(qt)
    n = 256 * 40
    raw = rand_blocks(qt, n, rng)
    want = oracle.dequant(qt, raw, n)
    dw, dy = dev.upload(raw), dev.alloc(n * 4)
    dev.check(dev.L.orc_dequant(qt, dw.ptr, n, dy.ptr, None))
    got = dy.read(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_fp16_exhaustive(dev, oracle):
    print("[gpu] fp16 sweep", flush=True)
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.uint8)
    want = oracle.dequant(ol.F16, raw, 65536)
    dw, dy = dev.upload(raw), dev.alloc(65536 * 4)
    dev.check(dev.L.orc_dequant(ol.F16, dw.ptr, 65536, dy.ptr, None))
    got = dy.read(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _gemm(dev, qt, w_dev, n_tok, n_out, n_in, X):
    dx = dev.upload(np.ascontiguousarray(X, np.float32))
    dy = dev.alloc(n_tok * n_out * 4)
    dev.check(dev.L.orc_gemm(qt, w_dev.ptr, n_tok, n_out, n_in, dx.ptr, n_in, dy.ptr, n_out, None))
    return dy.read(np.float32).reshape(n_tok, n_out)


SHAPES = [(ol.Q4_K, 515, 3072), (ol.Q4_K, 64, 3584), (ol.Q6_K, 301, 3072), (ol.Q6_K, 130, 8192),
          (ol.Q8_0, 700, 896), (ol.Q8_0, 129, 2048), (ol.Q4_0, 257, 2048), (ol.Q6_K, 40, 18944),
          (ol.Q8_0, 40000, 896)]  # the last: an LM-head-tall matrix (double-buffered row groups)


@pytest.mark.parametrize("qt,n_out,n_in", SHAPES)
def test_gemv_vs_exact(dev, oracle, qt, n_out, n_in):
    print(f"[gpu] gemv type={qt} {n_out}x{n_in}", flush=True)
    rng = np.random.default_rng(n_out * 7 + n_in)
    raw = rand_blocks(qt, n_out * n_in, rng)
    x = rng.uniform(-1, 1, n_in).astype(np.float32)
    got = _gemm(dev, qt, dev.upload(raw), 1, n_out, n_in, x[None])[0]
    W = oracle.dequant(qt, raw, n_out * n_in).reshape(n_out, n_in).astype(np.float64)
    exact = W @ x.astype(np.float64)
    scale = np.abs(W) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(got - exact) <= 2e-6 * scale + 1e-30), np.max(np.abs(got - exact) / scale)
    ref = oracle.gemv(qt, raw, n_out, n_in, x)  # fp32 restatement of gemv_q
    assert np.linalg.norm(got - ref) <= 1e-3 * np.linalg.norm(ref)


@pytest.mark.parametrize("qt,n_out,n_in", [(ol.Q4_K, 200, 3072), (ol.Q6_K, 77, 8192), (ol.Q8_0, 90, 896),
                                           (ol.Q4_0, 33, 2048), (ol.Q6_K, 24, 18944), (ol.Q8_0, 40000, 896),
                                           (ol.Q4_K, 8192, 3072), (ol.Q6_K, 70000, 1024),
                                           (ol.Q4_K, 140000, 512)])
def test_gemm_batch_invariant(dev, oracle, qt, n_out, n_in):
    """Tokens of a launch are independent: verify(n)[t] is bit-identical for
    every n. Q8_0 / Q4_0 run one kernel family for all n, so verify(n)[t] also
    equals the decode GEMV of token t bit for bit. The K-quants decode one
    token on the vector ALUs and verify 2..16 on the matrix cores (up to 8
    tokens as stacked hi / lo rows, 9-16 as two tiles), like the reference,
    whose gemv_q and gemm_q round differently: decode and verify then agree
    within 4e-6 of sum |w x|. The 70000- and 140000-row matrices take the
    whole-tile kernels (LM-head shapes; the Q4_K one with two tiles per
    wave), whose launches hold up to 16 tokens when the staged row fits."""
    print(f"[gpu] gemm invariance type={qt} {n_out}x{n_in}", flush=True)
    rng = np.random.default_rng(3)
    raw = rand_blocks(qt, n_out * n_in, rng)
    wd = dev.upload(raw)
    X = rng.normal(0, 1, (16, n_in)).astype(np.float32)
    single = np.stack([_gemm(dev, qt, wd, 1, n_out, n_in, X[t:t + 1])[0] for t in range(16)])
    kq = qt in (ol.Q4_K, ol.Q6_K)
    full = _gemm(dev, qt, wd, 16, n_out, n_in, X)
    for nt in (2, 5, 7, 9, 12, 16):
        got = _gemm(dev, qt, wd, nt, n_out, n_in, X[:nt])
        assert np.array_equal(got.view(np.uint32), full[:nt].view(np.uint32)), nt
        if not kq:
            assert np.array_equal(got.view(np.uint32), single[:nt].view(np.uint32)), nt
    if kq:
        W = oracle.dequant(qt, raw, n_out * n_in).reshape(n_out, n_in).astype(np.float64)
        scale = np.abs(X.astype(np.float64)) @ np.abs(W).T
        assert np.all(np.abs(full - single) <= 4e-6 * scale + 1e-30), np.max(np.abs(full - single) / scale)


@pytest.mark.parametrize("qt,n_out,n_in,nt", [(ol.Q4_K, 300, 3072, 300), (ol.Q6_K, 130, 2048, 256),
                                              (ol.Q6_K, 200, 18944, 263), (ol.Q4_K, 64, 512, 640),
                                              (ol.Q4_K, 8192, 3072, 256), (ol.Q8_0, 300, 3072, 300),
                                              (ol.Q8_0, 200, 896, 263), (ol.Q8_0, 70, 4864, 256),
                                              (ol.Q8_0_X8, 257, 3072, 256)])
def test_gemm_prefill_vs_exact_and_blocks(dev, oracle, qt, n_out, n_in, nt):
    """Calls of 256 tokens or more on a K-quant or Q8_0 matrix run the
    prefill kernel (64 tokens per workgroup, each weight slice decoded once
    for all of them; Q8_0 from the GGUF blocks or the regrouped Q8_0_X8
    layout, each block's scale applied to its own products): every (token,
    row) within 2e-6 of sum |w x| of the float64 product and within 4e-6 of
    the same tokens in 16-token calls (the verify path), with partial token
    and row blocks; a token's row does not depend on the call's other tokens
    (bit for bit)."""
    print(f"[gpu] prefill gemm type={qt} {n_out}x{n_in} nt={nt}", flush=True)
    rng = np.random.default_rng(n_out + nt)
    x8 = qt == ol.Q8_0_X8
    raw = rand_blocks(ol.Q8_0 if x8 else qt, n_out * n_in, rng)
    wd = dev.upload(raw)
    if x8:  # the Q8_0 blocks regrouped in place; the oracle reads the GGUF blocks
        dev.check(dev.L.orc_q8_0_regroup(wd.ptr, n_out * n_in // 256, None))
    X = rng.normal(0, 1, (nt, n_in)).astype(np.float32)
    full = _gemm(dev, qt, wd, nt, n_out, n_in, X)
    blocks = np.concatenate([_gemm(dev, qt, wd, min(16, nt - t), n_out, n_in, X[t:t + 16]) for t in range(0, nt, 16)])
    W = oracle.dequant(ol.Q8_0 if x8 else qt, raw, n_out * n_in).reshape(n_out, n_in).astype(np.float64)
    exact = X.astype(np.float64) @ W.T
    scale = np.abs(X.astype(np.float64)) @ np.abs(W).T
    assert np.all(np.abs(full - exact) <= 2e-6 * scale + 1e-30), np.max(np.abs(full - exact) / scale)
    assert np.all(np.abs(full - blocks) <= 4e-6 * scale + 1e-30), np.max(np.abs(full - blocks) / scale)
    tail = _gemm(dev, qt, wd, 256, n_out, n_in, X[nt - 256:])
    assert np.array_equal(tail.view(np.uint32), full[nt - 256:].view(np.uint32))


def test_gemm_prefill_epilogues(dev):
    """The prefill kernel's RMSNorm prologue, bias, three output segments,
    SwiGLU pairs and residual accumulation agree with the verify kernel's
    (16-token calls of the same fused entry point)."""
    print("[gpu] prefill gemm epilogues", flush=True)
    import orc

    rng = np.random.default_rng(17)
    n_in, nq, nk, ff, nt = 1024, 256, 128, 320, 300
    X = rng.normal(0, 1, (nt, n_in)).astype(np.float32)
    dx = dev.upload(X)
    dnorm = dev.upload(rng.uniform(0.5, 1.5, n_in).astype(np.float32))
    wq, wk, wv = (dev.upload(rand_blocks(ol.Q4_K, n * n_in, rng)) for n in (nq, nk, nk))
    bq = dev.upload(rng.normal(0, 0.1, nq).astype(np.float32))

    def both(run, ld, init=None):
        """run(t0, n, dy) for the whole call and for 16-token calls; returns both outputs"""
        outs = []
        for chunk in (nt, 16):
            dy = dev.upload(init) if init is not None else dev.alloc(nt * ld * 4)
            for t0 in range(0, nt, chunk):
                run(t0, min(chunk, nt - t0), dy)
            outs.append(dy.read(np.float32).reshape(nt, ld))
        return outs

    ld = nq + 2 * nk

    def qkv(t0, n, dy):
        yo = dy.ptr + t0 * ld * 4
        segs = (orc.Seg * 3)(orc.Seg(wq.ptr, nq, yo, bq.ptr), orc.Seg(wk.ptr, nk, yo + nq * 4, None),
                             orc.Seg(wv.ptr, nk, yo + (nq + nk) * 4, None))
        dev.check(dev.L.orc_gemm_fused(ol.Q4_K, segs, 3, n, n_in, dx.ptr + t0 * n_in * 4, n_in, ld, dnorm.ptr,
                                       C.c_float(1e-5), orc.EPI_STORE, None))

    a, b = both(qkv, ld)
    assert np.allclose(a, b, rtol=0, atol=2e-5 * np.abs(b).max())
    for st in (ol.Q6_K, ol.Q4_K, ol.Q8_0):  # Q8_0: SwiGLU in two passes (gate rows, then up)
        wg, wu = (dev.upload(rand_blocks(st, ff * n_in, rng)) for _ in range(2))

        def swiglu(t0, n, dy):
            yo = dy.ptr + t0 * ff * 4
            segs = (orc.Seg * 2)(orc.Seg(wg.ptr, ff, yo, None), orc.Seg(wu.ptr, ff, yo, None))
            dev.check(dev.L.orc_gemm_fused(st, segs, 2, n, n_in, dx.ptr + t0 * n_in * 4, n_in, ff, dnorm.ptr,
                                           C.c_float(1e-5), orc.EPI_SWIGLU, None))

        a, b = both(swiglu, ff)
        assert np.allclose(a, b, rtol=1e-5, atol=1e-5 * np.abs(b).max()), st
    res = rng.normal(0, 1, (nt, nk)).astype(np.float32)

    def accum(t0, n, dy):
        segs = (orc.Seg * 1)(orc.Seg(wk.ptr, nk, dy.ptr + t0 * nk * 4, None))
        dev.check(dev.L.orc_gemm_fused(ol.Q4_K, segs, 1, n, n_in, dx.ptr + t0 * n_in * 4, n_in, nk, None,
                                       C.c_float(0), orc.EPI_ACCUM, None))

    a, b = both(accum, nk, res)
    assert np.allclose(a, b, rtol=0, atol=2e-5 * np.abs(b).max())


@pytest.mark.parametrize("n_in", [512, 3072])  # 3072: the streamed-weight kernel
def test_gemm_fused_epilogues(dev, n_in):
    print(f"[gpu] fused epilogues n_in={n_in}", flush=True)
    import orc

    rng = np.random.default_rng(11)
    nq, nk, ff = 256, 128, 384
    wq, wk, wv = (dev.upload(rand_blocks(ol.Q4_K, n * n_in, rng)) for n in (nq, nk, nk))
    bq = dev.upload(rng.normal(0, 0.1, nq).astype(np.float32))
    normw = rng.uniform(0.5, 1.5, n_in).astype(np.float32)
    dnorm = dev.upload(normw)
    for nt in (1, 4, 11):
        X = rng.normal(0, 1, (nt, n_in)).astype(np.float32)
        dx = dev.upload(X)
        # reference composition: rmsnorm kernel, then plain GEMMs, bias on the host
        dxn = dev.alloc(X.nbytes)
        dev.check(dev.L.orc_rmsnorm(dxn.ptr, dx.ptr, dnorm.ptr, n_in, nt, C.c_float(1e-5), None))
        Xn = dxn.read(np.float32).reshape(nt, n_in)
        ref = [_gemm(dev, ol.Q4_K, w, nt, n, n_in, Xn) for w, n in ((wq, nq), (wk, nk), (wv, nk))]
        ref[0] = ref[0] + bq.read(np.float32)[None]
        ld = nq + 2 * nk
        dy = dev.alloc(nt * ld * 4)
        segs = (orc.Seg * 3)(orc.Seg(wq.ptr, nq, dy.ptr, bq.ptr), orc.Seg(wk.ptr, nk, dy.ptr + nq * 4, None),
                             orc.Seg(wv.ptr, nk, dy.ptr + (nq + nk) * 4, None))
        dev.check(dev.L.orc_gemm_fused(ol.Q4_K, segs, 3, nt, n_in, dx.ptr, n_in, ld, dnorm.ptr, C.c_float(1e-5),
                                       orc.EPI_STORE, None))
        Y = dy.read(np.float32).reshape(nt, ld)
        # fused: s * dot(w, x*g); unfused: dot(w, (x*s)*g) -- equal up to rounding
        for got, want in ((Y[:, :nq], ref[0]), (Y[:, nq:nq + nk], ref[1]), (Y[:, nq + nk:], ref[2])):
            assert np.allclose(got, want, rtol=0, atol=2e-5 * np.abs(want).max())
        # SwiGLU: silu(gate) * up
        for st in (ol.Q6_K, ol.Q4_K):
            wg, wu = (dev.upload(rand_blocks(st, ff * n_in, rng)) for _ in range(2))
            g = _gemm(dev, st, wg, nt, ff, n_in, X)
            u = _gemm(dev, st, wu, nt, ff, n_in, X)
            dh = dev.alloc(nt * ff * 4)
            segs2 = (orc.Seg * 2)(orc.Seg(wg.ptr, ff, dh.ptr, None), orc.Seg(wu.ptr, ff, None, None))
            segs2[1].d_y = dh.ptr
            dev.check(dev.L.orc_gemm_fused(st, segs2, 2, nt, n_in, dx.ptr, n_in, ff, None, C.c_float(0),
                                           orc.EPI_SWIGLU, None))
            h = dh.read(np.float32).reshape(nt, ff)
            want = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
            assert np.allclose(h, want, rtol=1e-5, atol=1e-6), st
        # residual accumulate
        res = rng.normal(0, 1, (nt, nk)).astype(np.float32)
        dr = dev.upload(res)
        segs3 = (orc.Seg * 1)(orc.Seg(wk.ptr, nk, dr.ptr, None))
        dev.check(dev.L.orc_gemm_fused(ol.Q4_K, segs3, 1, nt, n_in, dx.ptr, n_in, nk, None, C.c_float(0),
                                       orc.EPI_ACCUM, None))
        plain = _gemm(dev, ol.Q4_K, wk, nt, nk, n_in, X)
        assert np.array_equal(dr.read(np.float32).reshape(nt, nk), res + plain)


@pytest.mark.parametrize("n_in,rows,types,bias", [(3072, (3072, 1024, 1024), (ol.Q4_K, ol.Q4_K, ol.Q6_K), False),
                                                  (512, (448, 64, 64), (ol.Q4_K, ol.Q4_K, ol.Q6_K), True),
                                                  (3584, (3584, 512, 512), (ol.Q4_K, ol.Q4_K, ol.Q6_K), True),
                                                  (8192, (160, 96), (ol.Q6_K, ol.Q4_K), False)])
def test_gemm_mixed_equals_per_type(dev, n_in, rows, types, bias):
    """One launch over Q4_K and Q6_K segments (a Q4_K_M layer's Q|K|V) gives
    every segment's rows as the per-type launches do, for 1..16 tokens, with
    the RMSNorm prologue and QKV bias. The launches may split K differently
    (the split follows each launch's row count), so the match is to fp32
    summation order: 1e-5 of the largest output of the token. Within the
    multi-token mixed launch the tokens are independent: token t of an
    n-token launch is bit for bit token t of a two-token launch. One token
    over Q4_K segments then Q6_K segments is one vector launch whose row
    groups each keep their type's unit, lane split and reduction: equal to
    the per-type launches bit for bit."""
    import orc

    print(f"[gpu] gemm mixed n_in={n_in} rows={rows} types={types}", flush=True)
    rng = np.random.default_rng(n_in + len(rows))
    ws = [dev.upload(rand_blocks(t, r * n_in, rng)) for t, r in zip(types, rows)]
    bs = [dev.upload(rng.normal(0, 0.1, r).astype(np.float32)) if bias else None for r in rows]
    g = dev.upload(rng.uniform(0.5, 1.5, n_in).astype(np.float32))
    ld = sum(rows)
    offs = np.cumsum((0,) + rows)[:-1]
    for nt in (1, 5, 8, 9, 16):
        dx = dev.upload(rng.normal(0, 1, (nt, n_in)).astype(np.float32))
        dy, dz = dev.alloc(nt * ld * 4), dev.alloc(nt * ld * 4)
        segs = (orc.Seg * len(rows))(*[orc.Seg(w.ptr, r, dy.ptr + int(o) * 4, b.ptr if b else None)
                                       for w, r, o, b in zip(ws, rows, offs, bs)])
        ty = np.array(types, np.int32)
        dev.check(dev.L.orc_gemm_fused_mixed(ty.ctypes.data_as(C.POINTER(C.c_int32)), segs, len(rows), nt, n_in,
                                             dx.ptr, n_in, ld, g.ptr, C.c_float(1e-5), orc.EPI_STORE, None))
        for i, (t, w, r, o, b) in enumerate(zip(types, ws, rows, offs, bs)):
            one = (orc.Seg * 1)(orc.Seg(w.ptr, r, dz.ptr + int(o) * 4, b.ptr if b else None))
            dev.check(dev.L.orc_gemm_fused(t, one, 1, nt, n_in, dx.ptr, n_in, ld, g.ptr, C.c_float(1e-5),
                                           orc.EPI_STORE, None))
        got, want = dy.read(np.float32).reshape(nt, ld), dz.read(np.float32).reshape(nt, ld)
        scale = np.abs(want).max(axis=1, keepdims=True)
        assert np.all(np.abs(got - want) <= 1e-5 * scale), (nt, float(np.abs(got - want).max()))
        if nt == 1 and types[0] == ol.Q4_K:
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        if nt in (5, 16):
            t = nt - 2
            d2 = dev.alloc(2 * ld * 4)
            segs2 = (orc.Seg * len(rows))(*[orc.Seg(w.ptr, r, d2.ptr + int(o) * 4, b.ptr if b else None)
                                            for w, r, o, b in zip(ws, rows, offs, bs)])
            dev.check(dev.L.orc_gemm_fused_mixed(ty.ctypes.data_as(C.POINTER(C.c_int32)), segs2, len(rows), 2,
                                                 n_in, dx.ptr + t * n_in * 4, n_in, ld, g.ptr, C.c_float(1e-5),
                                                 orc.EPI_STORE, None))
            two = d2.read(np.float32).reshape(2, ld)
            assert np.array_equal(two.view(np.uint32), got[t:t + 2].view(np.uint32)), nt
    # error path: a segment that is not a whole number of 16-row tiles
    bad = (orc.Seg * 2)(orc.Seg(ws[0].ptr, 40, dy.ptr, None), orc.Seg(ws[1].ptr, 16, dy.ptr, None))
    ty = np.array(types[:2], np.int32)
    assert dev.L.orc_gemm_fused_mixed(ty.ctypes.data_as(C.POINTER(C.c_int32)), bad, 2, 1, n_in, dx.ptr, n_in, ld,
                                      None, C.c_float(0), orc.EPI_STORE, None) != 0


@pytest.mark.parametrize("qt,epi,nt", [(ol.Q4_K, "norm", 8), (ol.Q6_K, "swiglu", 8), (ol.Q4_K, "accum", 8),
                                       (ol.Q6_K, "swiglu", 9), (ol.Q4_K, "norm", 16), (ol.Q6_K, "accum", 12)])
def test_gemm_staging_windows(dev, oracle, qt, epi, nt):
    """Rows too long for every token's activations to fit the LDS at once
    (n_in = 18944) are staged in windows: with the RMSNorm prologue, the
    SwiGLU pair and the residual epilogue, over more tiles than workgroups (so
    windows are restaged for later tiles), the tokens of an nt-token call
    equal those of two-token calls bit for bit, and they and the one-token
    (vector) call match float64 within 2e-6 of sum |w x|."""
    import orc

    print(f"[gpu] gemm staging windows type={qt} epi={epi} nt={nt}", flush=True)
    rng = np.random.default_rng(19)
    n_in, n_out = 18944, 16 * 300
    raw = rand_blocks(qt, (2 if epi == "swiglu" else 1) * n_out * n_in, rng)
    wd = dev.upload(raw)
    X = rng.normal(0, 1, (nt, n_in)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, n_in).astype(np.float32)
    dg = dev.upload(g)
    res = rng.normal(0, 1, (nt, n_out)).astype(np.float32)

    def run(lo, n):
        dx = dev.upload(X[lo:lo + n])
        dy = dev.upload(res[lo:lo + n]) if epi == "accum" else dev.alloc(n * n_out * 4)
        rb = ol.row_bytes(qt, n_in)
        if epi == "swiglu":
            segs = (orc.Seg * 2)(orc.Seg(wd.ptr, n_out, dy.ptr, None), orc.Seg(wd.ptr + n_out * rb, n_out, dy.ptr, None))
            dev.check(dev.L.orc_gemm_fused(qt, segs, 2, n, n_in, dx.ptr, n_in, n_out, None, C.c_float(0),
                                           orc.EPI_SWIGLU, None))
        else:
            segs = (orc.Seg * 1)(orc.Seg(wd.ptr, n_out, dy.ptr, None))
            dev.check(dev.L.orc_gemm_fused(qt, segs, 1, n, n_in, dx.ptr, n_in, n_out,
                                           dg.ptr if epi == "norm" else None, C.c_float(1e-5),
                                           orc.EPI_ACCUM if epi == "accum" else orc.EPI_STORE, None))
        return dy.read(np.float32).reshape(n, n_out)

    got = run(0, nt)
    pairs = np.concatenate([run(t, 2)[:1] for t in range(nt - 1)] + [run(nt - 2, 2)[1:]])
    assert np.array_equal(got.view(np.uint32), pairs.view(np.uint32))
    one = run(0, 1)
    W = oracle.dequant(qt, raw, raw.size // ol.row_bytes(qt, n_in) * n_in).reshape(-1, n_in).astype(np.float64)
    Xd = X.astype(np.float64)
    if epi == "norm":
        Xd = Xd / np.sqrt((Xd ** 2).mean(axis=1, keepdims=True) + 1e-5) * g
    dot = Xd @ W.T
    scale = np.abs(Xd) @ np.abs(W).T
    if epi == "swiglu":
        gt, up = dot[:, :n_out], dot[:, n_out:]
        want = gt / (1 + np.exp(-gt)) * up
        tol = 3e-6 * (scale[:, :n_out] * np.abs(up) + scale[:, n_out:] * np.abs(gt)) + 1e-30  # |silu'| <= 1.1
        assert np.all(np.abs(got - want) <= tol + 1e-6 * np.abs(want))
        assert np.all(np.abs(one - want[:1]) <= tol[:1] + 1e-6 * np.abs(want[:1]))
    else:
        want = dot + (res if epi == "accum" else 0)
        assert np.all(np.abs(got - want) <= 2e-6 * scale + 1e-6 * np.abs(want) + 1e-30)
        assert np.all(np.abs(one - want[:1]) <= 2e-6 * scale[:1] + 1e-6 * np.abs(want[:1]) + 1e-30)


def test_rmsnorm(dev, oracle):
    rng = np.random.default_rng(5)
    for n in (896, 2048, 3072, 3584):
        x = rng.normal(0, 2, (3, n)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        dx, dw, dy = dev.upload(x), dev.upload(w), dev.alloc(x.nbytes)
        dev.check(dev.L.orc_rmsnorm(dy.ptr, dx.ptr, dw.ptr, n, 3, C.c_float(1e-5), None))
        got = dy.read(np.float32).reshape(3, n)
        for r in range(3):
            assert np.allclose(got[r], oracle.rmsnorm(x[r], w), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("H,KVH,hd,nt", [(8, 2, 128, 3), (32, 8, 128, 5), (14, 2, 64, 2), (5, 1, 96, 1)])
def test_qk_norm(dev, H, KVH, hd, nt):
    """orc_qk_norm (Qwen3, core/model.cpp:390-399): every q head and every k
    head of each token's QKV row is RMS-normalised over head_dim with its own
    weight vector (q heads qw, k heads kw), in place; v and the row padding
    stay untouched. Checked against the float64 closed form; half the heads
    are tiny (mean square ~1e-6), so an epsilon of 1e-5 instead of the 1e-6
    passed would move them by ~2x."""
    print(f"[gpu] qk_norm H={H} KVH={KVH} hd={hd} nt={nt}", flush=True)
    rng = np.random.default_rng(H * 100 + hd)
    ld = (H + 2 * KVH) * hd + 7  # row stride past the q | k | v columns
    qkv = rng.normal(0, 1, (nt, ld)).astype(np.float32)
    for h in range(0, H + KVH, 2):  # tiny heads: the epsilon matters
        qkv[:, h * hd:(h + 1) * hd] *= 1e-3
    qw = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    d, dq, dk = dev.upload(qkv), dev.upload(qw), dev.upload(kw)
    eps = 1e-6
    dev.check(dev.L.orc_qk_norm(d.ptr, ld, nt, H, KVH, hd, dq.ptr, dk.ptr, C.c_float(eps), None))
    got = d.read(np.float32).reshape(nt, ld)
    x = qkv.astype(np.float64)
    for t in range(nt):
        for h in range(H + KVH):
            v = x[t, h * hd:(h + 1) * hd]
            want = v / np.sqrt((v * v).mean() + eps) * (qw if h < H else kw)
            assert np.allclose(got[t, h * hd:(h + 1) * hd], want, rtol=2e-6, atol=1e-30), (t, h)
        assert np.array_equal(got[t, (H + KVH) * hd:], qkv[t, (H + KVH) * hd:])  # v and padding untouched
    # argument checks
    assert dev.L.orc_qk_norm(d.ptr, (H + 2 * KVH) * hd - 1, nt, H, KVH, hd, dq.ptr, dk.ptr, C.c_float(eps), None) != 0
    assert dev.L.orc_qk_norm(d.ptr, ld, nt, H, KVH, 256, dq.ptr, dk.ptr, C.c_float(eps), None) != 0


@pytest.mark.parametrize("H,KVH,hd,base", [(24, 8, 128, 500000.0), (28, 4, 128, 1e6), (14, 2, 64, 1e6)])
def test_rope_kv_store(dev, oracle, H, KVH, hd, base):
    print(f"[gpu] rope H={H} KVH={KVH} hd={hd}", flush=True)
    rng = np.random.default_rng(H)
    ctx, nt, sp = 64, 5, 37
    ld = (H + 2 * KVH) * hd
    qkv = rng.normal(0, 1, (nt, ld)).astype(np.float32)
    tab = rope_table(ctx, hd, base)
    dq, dt = dev.upload(qkv), dev.upload(tab)
    kc, vc = dev.alloc(KVH * ctx * hd * 4), dev.alloc(KVH * ctx * hd * 4)
    dev.check(dev.L.orc_rope_kv_store(dq.ptr, ld, nt, H, KVH, hd, sp, dt.ptr, kc.ptr, vc.ptr, ctx, None))
    got = dq.read(np.float32).reshape(nt, ld)
    K = kc.read(np.float32).reshape(KVH, ctx, hd)
    V = vc.read(np.float32).reshape(KVH, ctx, hd)
    for t in range(nt):
        q, k = oracle.rope(qkv[t, :H * hd], qkv[t, H * hd:(H + KVH) * hd], H, KVH, hd, sp + t, base)
        assert np.allclose(got[t, :H * hd], q, rtol=1e-5, atol=2e-6)
        assert np.allclose(got[t, H * hd:(H + KVH) * hd], k, rtol=1e-5, atol=2e-6)
        assert np.array_equal(K[:, sp + t, :].reshape(-1), got[t, H * hd:(H + KVH) * hd])
        assert np.array_equal(V[:, sp + t, :].reshape(-1), qkv[t, (H + KVH) * hd:])


@pytest.mark.parametrize("H,KVH,hd,sp,nt", [(24, 8, 128, 0, 1), (24, 8, 128, 200, 1), (24, 8, 128, 127, 5),
                                            (28, 4, 128, 700, 7), (14, 2, 64, 31, 9), (32, 8, 64, 1000, 1)])
def test_attention(dev, oracle, H, KVH, hd, sp, nt):
    print(f"[gpu] attention H={H} KVH={KVH} hd={hd} sp={sp} nt={nt}", flush=True)
    rng = np.random.default_rng(sp + nt)
    ctx = sp + nt + 3
    K = rng.normal(0, 1, (KVH, ctx, hd)).astype(np.float32)
    V = rng.normal(0, 1, (KVH, ctx, hd)).astype(np.float32)
    Q = rng.normal(0, 1, (nt, H * hd)).astype(np.float32)
    dK, dV, dQ = dev.upload(K), dev.upload(V), dev.upload(Q)
    dO = dev.alloc(nt * H * hd * 4)
    ws = dev.alloc(dev.L.orc_attn_workspace(nt, H, hd, ctx))
    dev.check(dev.L.orc_attn_gqa(dQ.ptr, H * hd, nt, H, KVH, hd, sp, dK.ptr, dV.ptr, ctx, dO.ptr, H * hd, ws.ptr,
                                 None))
    got = dO.read(np.float32).reshape(nt, H * hd)
    kc = K.transpose(1, 0, 2).reshape(ctx, KVH * hd)  # oracle layout [pos][kv*hd]
    vc = V.transpose(1, 0, 2).reshape(ctx, KVH * hd)
    for t in range(nt):
        want = oracle.attention(Q[t], kc, vc, H, KVH, hd, sp + t)
        assert np.allclose(got[t], want, rtol=1e-5, atol=2e-6), np.abs(got[t] - want).max()


def _attn_ws(dev, H, KVH, hd):
    return dev.alloc(dev.L.orc_attn_fused_workspace(H, KVH, hd))


@pytest.mark.parametrize("H,KVH,hd,sp,nt,devpos,lim,flo",
                         [(24, 8, 128, 0, 1, False, 0, 0), (24, 8, 128, 200, 1, True, 0, 0),
                          (24, 8, 128, 127, 5, True, 140, 0), (28, 4, 128, 700, 7, False, 0, 0),
                          (14, 2, 64, 31, 9, True, 512, 0), (32, 8, 64, 1000, 1, False, 0, 0),
                          (24, 8, 128, 1300, 5, True, 1400, 0), (24, 8, 128, 62, 5, False, 0, 0),
                          (28, 4, 128, 2045, 9, True, 0, 0), (14, 2, 64, 4100, 16, False, 0, 0),
                          (24, 8, 128, 505, 9, True, 520, 0), (24, 8, 128, 380, 5, True, 512, 0),
                          (24, 8, 128, 1020, 9, True, 1100, 0), (14, 2, 64, 1019, 9, False, 0, 0),
                          (24, 8, 128, 100, 5, True, 256, 0), (24, 8, 128, 251, 5, True, 256, 0),
                          (24, 8, 128, 250, 9, True, 512, 0), (24, 8, 128, 256, 5, True, 512, 256),
                          (24, 8, 128, 300, 9, True, 512, 256), (14, 2, 64, 253, 9, False, 0, 0),
                          (28, 4, 128, 1500, 5, True, 2048, 256), (28, 4, 128, 8400, 9, False, 0, 0),
                          (14, 2, 64, 16370, 9, True, 16384, 8192), (14, 2, 64, 16380, 9, True, 16400, 16000),
                          (14, 2, 64, 20000, 3, False, 0, 0), (24, 8, 128, 508, 9, True, 1024, 0),
                          (24, 8, 128, 512, 5, True, 1024, 512), (28, 4, 128, 400, 9, True, 1024, 300),
                          (14, 2, 64, 509, 9, False, 0, 0)])
def test_attn_fused(dev, oracle, H, KVH, hd, sp, nt, devpos, lim, flo):
    """Fused RoPE + KV store + attention equals the oracle's rope then
    attention over the prefilled cache plus the new rows; the new K/V rows
    land in the cache; the QKV rows are left as they were. Cases cross chunk
    boundaries (64 positions per chunk up to 16384, then wider chunks; merges
    of more than 32 chunks split over lane groups) and the
    switch between the one-workgroup path and the split (512 positions), and
    a second call on the same workspace repeats the first's outputs. lim, flo:
    the bounds flo <= position < lim declared by a device-position call (lim
    0: the context), which select its kernels and size their grids."""
    print(f"[gpu] attn_fused H={H} KVH={KVH} hd={hd} sp={sp} nt={nt} devpos={devpos} lim={lim} flo={flo}", flush=True)
    assert dev.L.orc_attn_wg_limit() == 512
    rng = np.random.default_rng(sp * 7 + nt)
    base = 500000.0
    ctx = max(sp + nt + 5, lim)
    lim = lim or ctx
    ld = (H + 2 * KVH) * hd
    qkv = rng.normal(0, 1, (nt, ld)).astype(np.float32)
    K = rng.normal(0, 1, (KVH, ctx, hd)).astype(np.float32)
    V = rng.normal(0, 1, (KVH, ctx, hd)).astype(np.float32)
    tab = rope_table(ctx, hd, base)
    dq, dt, dK, dV = dev.upload(qkv), dev.upload(tab), dev.upload(K), dev.upload(V)
    dO = dev.alloc(nt * H * hd * 4)
    ws = _attn_ws(dev, H, KVH, hd)
    dp = dev.upload(np.array([sp - 3], np.int32))

    def run():
        if devpos:
            dev.check(dev.L.orc_attn_fused_at(dq.ptr, ld, nt, H, KVH, hd, dp.ptr, 3, dt.ptr, dK.ptr, dV.ptr, ctx, flo,
                                              lim, dO.ptr, H * hd, ws.ptr, None))
        else:
            dev.check(dev.L.orc_attn_fused_at(dq.ptr, ld, nt, H, KVH, hd, None, sp, dt.ptr, dK.ptr, dV.ptr, ctx, 0,
                                              ctx, dO.ptr, H * hd, ws.ptr, None))
        return dO.read(np.float32).reshape(nt, H * hd)

    got = run()
    assert np.array_equal(run(), got)
    Kc = dK.read(np.float32).reshape(KVH, ctx, hd)
    Vc = dV.read(np.float32).reshape(KVH, ctx, hd)
    assert np.array_equal(dq.read(np.float32).reshape(nt, ld), qkv)
    kref, vref = K.copy(), V.copy()
    qs = []
    for t in range(nt):
        q, k = oracle.rope(qkv[t, :H * hd], qkv[t, H * hd:(H + KVH) * hd], H, KVH, hd, sp + t, base)
        qs.append(q)
        kref[:, sp + t, :] = k.reshape(KVH, hd)
        vref[:, sp + t, :] = qkv[t, (H + KVH) * hd:].reshape(KVH, hd)
    assert np.allclose(Kc[:, :sp + nt], kref[:, :sp + nt], rtol=1e-5, atol=2e-6)
    assert np.array_equal(Vc[:, :sp + nt], vref[:, :sp + nt])
    assert np.array_equal(Kc[:, sp + nt:], K[:, sp + nt:]) and np.array_equal(Vc[:, sp + nt:], V[:, sp + nt:])
    kc = kref.transpose(1, 0, 2).reshape(ctx, KVH * hd)
    vc = vref.transpose(1, 0, 2).reshape(ctx, KVH * hd)
    for t in range(nt):
        want = oracle.attention(qs[t], kc, vc, H, KVH, hd, sp + t)
        assert np.allclose(got[t], want, rtol=2e-5, atol=4e-6), (t, np.abs(got[t] - want).max())


@pytest.mark.parametrize("H,KVH,hd,sp,nt", [(24, 8, 128, 0, 256), (14, 2, 64, 100, 300), (28, 4, 128, 700, 260),
                                            (24, 8, 128, 3, 40), (32, 4, 64, 1000, 17)])
def test_attn_prefill(dev, oracle, H, KVH, hd, sp, nt):
    """The prefill attention (one workgroup per 16-token block and kv head,
    online softmax over every key chunk, no partials) equals the oracle's
    rope then causal attention over the prefilled cache plus the new rows
    (2e-5), agrees with 16-token calls of the decode / verify path (4e-6 of
    the largest output), stores the same K / V rows, and leaves the QKV rows
    as they were; partial last blocks, a cache prefix and chunk boundaries
    included."""
    print(f"[gpu] attn_prefill H={H} KVH={KVH} hd={hd} sp={sp} nt={nt}", flush=True)
    rng = np.random.default_rng(sp + nt)
    base = 500000.0
    ctx = sp + nt + 3
    ld = (H + 2 * KVH) * hd
    qkv = rng.normal(0, 1, (nt, ld)).astype(np.float32)
    K = rng.normal(0, 1, (KVH, ctx, hd)).astype(np.float32)
    V = rng.normal(0, 1, (KVH, ctx, hd)).astype(np.float32)
    dq, dt = dev.upload(qkv), dev.upload(rope_table(ctx, hd, base))
    outs = []
    for mode in ("prefill", "blocks"):
        dK, dV = dev.upload(K), dev.upload(V)
        dO = dev.alloc(nt * H * hd * 4)
        if mode == "prefill":
            dev.check(dev.L.orc_attn_prefill(dq.ptr, ld, nt, H, KVH, hd, sp, dt.ptr, dK.ptr, dV.ptr, ctx, dO.ptr,
                                             H * hd, None))
        else:
            ws = _attn_ws(dev, H, KVH, hd)
            for t0 in range(0, nt, 16):
                n = min(16, nt - t0)
                dev.check(dev.L.orc_attn_fused_at(dq.at(t0 * ld * 4), ld, n, H, KVH, hd, None, sp + t0, dt.ptr,
                                                  dK.ptr, dV.ptr, ctx, 0, ctx, dO.at(t0 * H * hd * 4), H * hd, ws.ptr,
                                                  None))
        outs.append((dO.read(np.float32).reshape(nt, H * hd), dK.read(np.float32).reshape(KVH, ctx, hd),
                     dV.read(np.float32).reshape(KVH, ctx, hd)))
    (got, Kc, Vc), (blk, Kb, Vb) = outs
    assert np.array_equal(dq.read(np.float32).reshape(nt, ld), qkv)
    assert np.array_equal(Kc, Kb) and np.array_equal(Vc, Vb)
    assert np.allclose(got, blk, rtol=0, atol=4e-6 * np.abs(blk).max()), np.abs(got - blk).max()
    kref, vref = K.copy(), V.copy()
    qs = []
    for t in range(nt):
        q, k = oracle.rope(qkv[t, :H * hd], qkv[t, H * hd:(H + KVH) * hd], H, KVH, hd, sp + t, base)
        qs.append(q)
        kref[:, sp + t, :] = k.reshape(KVH, hd)
        vref[:, sp + t, :] = qkv[t, (H + KVH) * hd:].reshape(KVH, hd)
    assert np.allclose(Kc, kref, rtol=1e-5, atol=2e-6) and np.array_equal(Vc, vref)
    kc = kref.transpose(1, 0, 2).reshape(ctx, KVH * hd)
    vc = vref.transpose(1, 0, 2).reshape(ctx, KVH * hd)
    for t in range(0, nt, max(1, nt // 24)):
        want = oracle.attention(qs[t], kc, vc, H, KVH, hd, sp + t)
        assert np.allclose(got[t], want, rtol=2e-5, atol=4e-6), (t, np.abs(got[t] - want).max())


@pytest.mark.parametrize("H,KVH,hd,sp,nt", [(24, 8, 128, 250, 5), (14, 2, 64, 2040, 9), (28, 4, 128, 60, 7),
                                            (24, 8, 128, 508, 9), (28, 4, 128, 1019, 9), (14, 2, 64, 3, 16),
                                            (24, 8, 128, 252, 9), (14, 2, 64, 250, 9), (28, 4, 128, 8400, 9),
                                            (14, 2, 64, 16380, 9), (28, 4, 128, 505, 9), (24, 8, 128, 380, 9)])
def test_attn_fused_batch_invariant(dev, H, KVH, hd, sp, nt):
    """One n-token call equals n one-token calls at the following positions
    bit for bit (the verify pass of a speculative round equals decode)."""
    print(f"[gpu] attn_fused batch invariance H={H} KVH={KVH} hd={hd} sp={sp} nt={nt}", flush=True)
    rng = np.random.default_rng(sp + 11 * nt)
    ctx = sp + nt + 2
    ld = (H + 2 * KVH) * hd
    qkv = rng.normal(0, 1, (nt, ld)).astype(np.float32)
    K = rng.normal(0, 1, (KVH, ctx, hd)).astype(np.float32)
    V = rng.normal(0, 1, (KVH, ctx, hd)).astype(np.float32)
    dq, dt = dev.upload(qkv), dev.upload(rope_table(ctx, hd, 1e6))
    ws = _attn_ws(dev, H, KVH, hd)
    outs = []
    for n in (nt, 1):
        dK, dV = dev.upload(K), dev.upload(V)
        dO = dev.alloc(nt * H * hd * 4)
        if n == nt:
            dev.check(dev.L.orc_attn_fused_at(dq.ptr, ld, nt, H, KVH, hd, None, sp, dt.ptr, dK.ptr, dV.ptr, ctx, 0,
                                              ctx, dO.ptr, H * hd, ws.ptr, None))
        else:
            for t in range(nt):
                dev.check(dev.L.orc_attn_fused_at(dq.at(t * ld * 4), ld, 1, H, KVH, hd, None, sp + t, dt.ptr, dK.ptr,
                                                  dV.ptr, ctx, 0, ctx, dO.at(t * H * hd * 4), H * hd, ws.ptr, None))
        outs.append((dO.read(np.float32), dK.read(np.float32), dV.read(np.float32)))
    for a, b in zip(*outs):
        assert np.array_equal(a, b)


def test_argmax_first_index(dev, oracle):
    rng = np.random.default_rng(9)
    rows, n = 6, 128256
    x = rng.normal(0, 1, (rows, n)).astype(np.float32)
    x[1, 5] = x[1, 99999] = 50.0          # tie: first index wins
    x[2, :] = 1.0                          # all equal -> 0
    x[3, n - 1] = 77.0                     # maximum at the end
    x[4, 0] = 77.0                         # maximum at the start
    dx, do = dev.upload(x), dev.alloc(rows * 4)
    ws = dev.alloc(dev.L.orc_argmax_workspace(rows, n))
    dev.check(dev.L.orc_argmax(dx.ptr, rows, n, n, do.ptr, ws.ptr, None))
    got = do.read(np.int32)
    assert list(got) == [oracle.argmax(x[r]) for r in range(rows)]
    assert got[1] == 5 and got[2] == 0 and got[3] == n - 1 and got[4] == 0


def test_accept_greedy(dev):
    cases = [([5, 6, 7, 8, 9], [5, 6, 7, 8], 4, 9), ([5, 6, 7, 8, 9], [5, 1, 7, 8], 1, 6),
             ([3, 6, 7, 8, 9], [5, 6, 7, 8], 0, 3), ([1, 2], [1], 1, 2)]
    for tgt, dft, a, nxt in cases:
        dt, dd, do = dev.upload(np.array(tgt, np.int32)), dev.upload(np.array(dft, np.int32)), dev.alloc(8)
        dev.check(dev.L.orc_spec_accept_greedy(dt.ptr, dd.ptr, len(dft), do.ptr, None))
        assert list(do.read(np.int32)) == [a, nxt]


def test_error_paths(dev):
    """Bad shapes and unsupported types are rejected before any launch."""
    import orc

    d = dev.alloc(4096)
    assert dev.L.orc_gemm(13, d.ptr, 1, 4, 256, d.ptr, 256, d.ptr, 4, None) == -2  # Q5_K unsupported
    assert dev.L.orc_gemm(ol.Q4_K, d.ptr, 1, 4, 100, d.ptr, 100, d.ptr, 4, None) == -1  # n_in not a block multiple
    assert dev.L.orc_rope_kv_store(d.ptr, 1024, 2, 4, 2, 64, 63, d.ptr, d.ptr, d.ptr, 64, None) == -1  # past ctx
    assert b"ctx" in dev.L.orc_last_error() or b"context" in dev.L.orc_last_error()
    with pytest.raises(orc.OrcError):
        dev.check(dev.L.orc_dequant(13, d.ptr, 256, d.ptr, None))


def _x8_layout(raw, n_out, n_in):
    """The ORC_Q8_0_X8 bytes of a Q8_0 matrix: per 8 blocks, their fp16 scales,
    then their 32-byte code runs."""
    b = raw.reshape(n_out * n_in // 256, 8, 34)
    return np.concatenate([b[:, :, :2].reshape(-1, 16), b[:, :, 2:].reshape(-1, 256)], axis=1).reshape(-1)


@pytest.mark.parametrize("n_out,n_in", [(90, 3072), (1024, 8192), (40000, 3072), (8192, 256)])
def test_q8_0_regroup_gemm_bit_identical(dev, n_out, n_in):
    """orc_q8_0_regroup writes the 8-block grouped layout in place, and a GEMM
    over it (1..5 tokens; plain, the LM-head-tall shape, and fused norm /
    SwiGLU / residual / bias epilogues) equals the same GEMM over the Q8_0
    blocks bit for bit."""
    import orc

    print(f"[gpu] q8_0 regroup {n_out}x{n_in}", flush=True)
    rng = np.random.default_rng(n_out + n_in)
    raw = rand_blocks(ol.Q8_0, n_out * n_in, rng)
    wq, wx = dev.upload(raw), dev.upload(raw)
    dev.check(dev.L.orc_q8_0_regroup(wx.ptr, n_out * n_in // 256, None))
    dev.sync()
    assert np.array_equal(wx.read(np.uint8), _x8_layout(raw, n_out, n_in))
    assert dev.L.orc_row_bytes(orc.Q8_0_X8, n_in) == n_in // 32 * 34
    X = rng.normal(0, 1, (5, n_in)).astype(np.float32)
    for nt in (1, 2, 5):
        a = _gemm(dev, ol.Q8_0, wq, nt, n_out, n_in, X[:nt])
        b = _gemm(dev, orc.Q8_0_X8, wx, nt, n_out, n_in, X[:nt])
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), nt
    if n_out % 2 or n_out > 20000:
        return
    half = n_out // 2
    rb = n_in // 32 * 34
    g = dev.upload(rng.uniform(0.5, 1.5, n_in).astype(np.float32))
    bias = dev.upload(rng.normal(0, 0.1, n_out).astype(np.float32))
    for nt in (1, 4):
        dx = dev.upload(X[:nt])
        res = rng.normal(0, 1, (nt, n_out)).astype(np.float32)
        outs = []
        for ty, w in ((ol.Q8_0, wq), (orc.Q8_0_X8, wx)):
            got = []
            dy = dev.upload(res)  # residual epilogue with norm and bias
            segs = (orc.Seg * 1)(orc.Seg(w.ptr, n_out, dy.ptr, bias.ptr))
            dev.check(dev.L.orc_gemm_fused(ty, segs, 1, nt, n_in, dx.ptr, n_in, n_out, g.ptr, C.c_float(1e-5),
                                           orc.EPI_ACCUM, None))
            got.append(dy.read(np.float32))
            dz = dev.alloc(nt * half * 4)  # SwiGLU pair with norm
            segs = (orc.Seg * 2)(orc.Seg(w.ptr, half, dz.ptr, None), orc.Seg(w.ptr + half * rb, half, dz.ptr, None))
            dev.check(dev.L.orc_gemm_fused(ty, segs, 2, nt, n_in, dx.ptr, n_in, half, g.ptr, C.c_float(1e-5),
                                           orc.EPI_SWIGLU, None))
            got.append(dz.read(np.float32))
            outs.append(got)
        for a, b in zip(*outs):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), nt
