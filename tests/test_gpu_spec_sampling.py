"""Speculative sampling on the device (min(1, p/q) acceptance with residual
resampling) against the CPU oracle.

Bars: the transform's kept set identical to the oracle's and probabilities
within 2e-6 absolute (the device's softmax sums in another order); draws,
acceptance decisions and emitted ids identical (index work); the sampler
history identical after a chain; the full loop's stream and stats equal to
the oracle's loop on the synthetic models, and at T = 0 to the reference's
speculative greedy stream.
"""
import ctypes as C
import os

import numpy as np
import pytest

import oracle_lib as ol
from conftest import GOLDEN

pytestmark = pytest.mark.gpu
FIX = np.load(os.path.join(GOLDEN, "ref_fixtures.npz"))


def _uniform(oracle, s):
    """generate_canonical<float, 24>(mt19937) from the oracle's engine."""
    r = np.float32(np.float32(oracle.L.orco_mt_next(s)) / np.float32(4294967296.0))
    return float(min(r, np.nextafter(np.float32(1), np.float32(0))))


def _window(oracle, s, extra, last):
    h = np.zeros(8192, np.int32)
    n = oracle.L.orco_sampler_history(s, ol.iptr(h), h.size)
    w = np.concatenate([h[:n], np.asarray(extra, np.int32)])
    return w[max(0, w.size - last):] if last > 0 else w[:0]


def _oracle_probs(oracle, lg, T, P, K, pen, win):
    p = np.zeros(lg.size, np.float32)
    win = np.ascontiguousarray(win, np.int32)
    oracle.L.orco_transform_probs(ol.fptr(np.ascontiguousarray(lg, np.float32)), lg.size, ol.iptr(win), win.size,
                                  T, P, K, pen, ol.fptr(p))
    return p


# top_p = 1.0 is left out: the float running sum of the sorted probabilities
# reaches 1.0 (or not) at an index set by rounding, so two correct
# implementations whose softmax sums in different orders cut the tail at
# different places.
CASES = [  # (V, T, top_p, top_k, penalty, repeat_last)
    (2048, 0.8, 0.95, 40, 1.1, 64),
    (2048, 1.0, 0.999, 0, 1.0, 64),
    (5000, 1.3, 0.9, 0, 1.2, 16),
    (4096, 0.0, 0.9, 40, 1.3, 8),
    (32000, 0.7, 0.5, 200, 1.05, 32),
    (151936, 0.8, 0.95, 40, 1.1, 64),
]


def _check_transform(dev, oracle, lg, T, P, K, pen, last, hist, extra, base):
    """orc_transform_probs over the rows of lg against the oracle's transform
    of each row (row r's window: hist + extra[:base + r])."""
    L = dev.L
    rows, V = lg.shape
    state = dev.alloc(L.orc_sampler_state_bytes())
    dh, dx = dev.upload(hist), dev.upload(extra)
    dl, dp = dev.upload(lg), dev.alloc(lg.nbytes)
    dev.check(L.orc_sampler_init(state.ptr, T, P, K, pen, last, 7, dh.ptr, hist.size, None))
    dev.check(L.orc_transform_probs(state.ptr, dl.ptr, V, V, rows, dx.ptr, base, dp.ptr, V, None))
    got = dp.read(np.float32).reshape(rows, V)
    s = oracle.L.orco_sampler_new(T, P, K, pen, last, 7)
    for h in hist:
        oracle.L.orco_sampler_record(s, int(h))
    for r in range(rows):
        ref = _oracle_probs(oracle, lg[r], T, P, K, pen, _window(oracle, s, extra[:base + r], last))
        assert np.array_equal(got[r] > 0, ref > 0), r
        assert np.abs(got[r] - ref).max() <= 2e-6, (r, np.abs(got[r] - ref).max())
    oracle.L.orco_sampler_free(s)


def _penalty_rows(V, rows, n_hist, seed):
    rng = np.random.default_rng(seed)
    lg = rng.normal(0, 3, (rows, V)).astype(np.float32)
    hist = rng.integers(0, V, n_hist).astype(np.int32)
    hist[:40] = rng.integers(0, 50, 40)  # repeats compound
    extra = rng.integers(0, 60, rows + 2).astype(np.int32)
    lg[:, :60] += 4.0  # the penalised ids matter to the kept set
    return lg, hist, extra


@pytest.mark.parametrize("case", CASES)
def test_transform_probs_matches_oracle(dev, oracle, case):
    """orc_transform_probs over several rows, each with its own pending
    proposals in the penalty window, equals the oracle's transform."""
    V, T, P, K, pen, last = case
    print(f"[gpu] transform V={V} T={T} top_p={P} top_k={K}", flush=True)
    lg, hist, extra = _penalty_rows(V, 4, 150, V + K)
    _check_transform(dev, oracle, lg, T, P, K, pen, last, hist, extra, 2)


# The split transform (T > 0, 1 <= top_k <= 128, up to 17 rows of up to
# 196608 logits in slices of 4096): a partial last slice, the largest
# vocabulary, top_k 1 and 128, a peaked distribution whose tail underflows
# to zero, a penalty window longer than 256 entries.
SPLIT_CASES = [  # (V, T, top_p, top_k, penalty, repeat_last, history)
    (16385, 0.8, 0.95, 40, 1.1, 64, 150),
    (151936, 0.3, 0.5, 1, 1.3, 256, 150),
    (151936, 1.0, 0.99, 128, 1.0, 64, 150),
    (196608, 1.7, 0.9, 100, 1.2, 16, 150),
    (128256, 0.05, 0.95, 40, 1.1, 64, 150),
    (151936, 0.8, 0.95, 40, 1.1, 3000, 2900),
]


@pytest.mark.parametrize("case", SPLIT_CASES)
def test_transform_split_matches_oracle(dev, oracle, case):
    V, T, P, K, pen, last, n_hist = case
    print(f"[gpu] split transform V={V} T={T} top_p={P} top_k={K} window={last}", flush=True)
    lg, hist, extra = _penalty_rows(V, 3, n_hist, V + K + n_hist)
    _check_transform(dev, oracle, lg, T, P, K, pen, last, hist, extra, 2)


@pytest.mark.parametrize("rows", [1, 17, 18])
def test_transform_ties_and_row_counts(dev, oracle, rows):
    """Rows of tied logits: 9000 equal maxima (slices with thousands of tied
    candidates: the row is redone by the one-workgroup transform), logits on
    a 0.5 grid (~1900 ties at the top value spread over every slice), and a
    plain row; 17 rows (the most the split path takes) and 18 (the
    one-workgroup kernel)."""
    print(f"[gpu] transform ties rows={rows}", flush=True)
    V = 151936
    rng = np.random.default_rng(rows)
    lg = rng.normal(0, 2, (rows, V)).astype(np.float32)
    for r in range(rows):
        if r % 3 == 0:
            lg[r, 5000:14000] = lg[r].max() + 1.0
        elif r % 3 == 1:
            lg[r] = rng.integers(-20, 20, V) * 0.5
    hist = rng.integers(0, V, 100).astype(np.int32)
    extra = rng.integers(0, V, rows + 1).astype(np.int32)
    _check_transform(dev, oracle, lg, 0.9, 0.95, 40, 1.1, 64, hist, extra, 1)


@pytest.mark.parametrize("V,K", [(2048, 40), (2048, 0), (151936, 40), (151936, 0)])
def test_transform_draw_matches_oracle(dev, oracle, V, K):
    """orc_transform_draw: the distribution as orc_transform_probs writes it
    and, call after call, the oracle's draw (orco_pick with the oracle's
    mt19937 uniform) from that distribution; top_k 0 takes the
    one-workgroup transform and draw. top_k 0 at V > 16384 is refused as
    orc_transform_probs refuses it."""
    print(f"[gpu] transform_draw V={V} top_k={K}", flush=True)
    L = dev.L
    rng = np.random.default_rng(V + 11)
    T, P, pen, last = 0.8, 0.95, 1.1, 64
    state = dev.alloc(L.orc_sampler_state_bytes())
    hist = rng.integers(0, V, 80).astype(np.int32)
    dh = dev.upload(hist)
    dev.check(L.orc_sampler_init(state.ptr, T, P, K, pen, last, 31, dh.ptr, hist.size, None))
    dp, do = dev.alloc(V * 4), dev.alloc(8)
    if K == 0 and V > 16384:
        dl = dev.upload(rng.normal(0, 2, V).astype(np.float32))
        assert L.orc_transform_draw(state.ptr, dl.ptr, V, None, 0, dp.ptr, do.ptr, None, None) != 0
        return
    s = oracle.L.orco_sampler_new(T, P, K, pen, last, 31)
    for h in hist:
        oracle.L.orco_sampler_record(s, int(h))
    extra = rng.integers(0, 100, 8).astype(np.int32)
    dx = dev.upload(extra)
    for call in range(8):
        lg = rng.normal(0, 2, V).astype(np.float32)
        lg[:100] += 2.0
        dl = dev.upload(lg)
        dev.check(L.orc_transform_draw(state.ptr, dl.ptr, V, dx.ptr, call, dp.ptr, do.ptr, do.ptr + 4, None))
        got = dp.read(np.float32)
        ref = _oracle_probs(oracle, lg, T, P, K, pen, _window(oracle, s, extra[:call], last))
        assert np.array_equal(got > 0, ref > 0), call
        assert np.abs(got - ref).max() <= 2e-6, call
        tok = oracle.L.orco_pick(ol.fptr(got), V, _uniform(oracle, s))
        assert list(do.read(np.int32, 2)) == [tok, tok], call
    oracle.L.orco_sampler_free(s)


def test_draw_and_accept_resample_match_oracle(dev, oracle):
    """orc_draw (mt19937 uniform) and orc_accept_resample (explicit uniforms)
    pick the oracle's ids on the same distributions."""
    L = dev.L
    rng = np.random.default_rng(5)
    V = 3000
    state = dev.alloc(L.orc_sampler_state_bytes())
    dev.check(L.orc_sampler_init(state.ptr, 0.8, 0.95, 40, 1.0, 64, 99, None, 0, None))
    s = oracle.L.orco_sampler_new(0.8, 0.95, 40, 1.0, 64, 99)
    do = dev.alloc(8)
    for trial in range(6):
        p = _oracle_probs(oracle, rng.normal(0, 2, V), 1.0, 0.97, [0, 50, 400][trial % 3], 1.0, [])
        q = _oracle_probs(oracle, rng.normal(0, 2, V), 0.9, 0.99, 0, 1.0, [])
        dp, dq = dev.upload(p), dev.upload(q)
        for _ in range(8):
            dev.check(L.orc_draw(state.ptr, dp.ptr, V, do.ptr, None, None))
            assert int(do.read(np.int32, 1)[0]) == oracle.L.orco_pick(ol.fptr(p), V, _uniform(oracle, s))
        acc = C.c_int()
        xs = list(np.nonzero(q)[0][:6]) + list(np.nonzero(p)[0][:6])
        for x in xs:
            for ua, ur in ((0.05, 0.3), (0.5, 0.77), (0.97, 0.001), (0.999, 0.9999)):
                dev.check(L.orc_accept_resample(dp.ptr, dq.ptr, V, int(x), ua, ur, do.ptr, None))
                got = do.read(np.int32, 2)
                tok = oracle.L.orco_accept_resample(ol.fptr(p), ol.fptr(q), V, int(x), ua, ur, C.byref(acc))
                assert (int(got[0]), int(got[1])) == (tok, acc.value), (trial, x, ua, ur)
    oracle.L.orco_sampler_free(s)


@pytest.mark.parametrize("k,V", [(1, 1024), (3, 1024), (6, 1024), (3, 151936), (6, 196608)])
def test_accept_chain_matches_oracle(dev, oracle, k, V):
    """orc_spec_accept_stochastic over many rounds (accepts, rejections,
    bonus draws, budget cuts) equals the oracle's chain: emitted ids,
    counts, the round state and the sampler history. The draw's weights are
    summed per slice of 4096 entries; the large vocabularies put the kept
    sets in many slices."""
    L = dev.L
    rng = np.random.default_rng(k + V)
    print(f"[gpu] accept chain k={k} V={V}", flush=True)
    state = dev.alloc(L.orc_sampler_state_bytes())
    dev.check(L.orc_sampler_init(state.ptr, 0.8, 0.95, 40, 1.1, 64, 1234, None, 0, None))
    s = oracle.L.orco_sampler_new(0.8, 0.95, 40, 1.1, 64, 1234)
    dout, dpos = dev.alloc((k + 8) * 4), dev.alloc(8)
    budget = dev.alloc(4)
    paths = {"accept": 0, "reject": 0, "bonus": 0}
    for rnd in range(40 if V <= 4096 else 12):
        base = rng.normal(0, 2, V)
        # target and draft close enough that every path occurs
        p = np.stack([_oracle_probs(oracle, base + rng.normal(0, 0.3 + 0.1 * (rnd % 5), V), 1.0, 0.99, 30, 1.0, [])
                      for _ in range(k + 1)])
        q = np.stack([_oracle_probs(oracle, base + rng.normal(0, 0.3, V), 1.0, 0.99, 30, 1.0, [])
                      for _ in range(k)])
        x = np.array([oracle.L.orco_pick(ol.fptr(q[i]), V, float(rng.random())) for i in range(k)], np.int32)
        max_emit = k + 1 if rnd % 7 else 1 + rnd % (k + 1)
        use_budget = rnd % 2 == 0
        dp, dq, dx = dev.upload(p), dev.upload(q), dev.upload(x)
        dpos.write(np.array([100, 0], np.int32))
        if use_budget:
            budget.write(np.array([max_emit], np.int32))
        dev.check(L.orc_spec_accept_stochastic(state.ptr, dp.ptr, V, dq.ptr, V, V, dx.ptr, k,
                                               0 if use_budget else max_emit, budget.ptr if use_budget else None,
                                               dout.ptr, dpos.ptr, dpos.ptr + 4, None))
        got = dout.read(np.int32, k + 5)
        out = np.zeros(k + 1, np.int32)
        acc, al = C.c_int(), C.c_int()
        n = oracle.L.orco_accept_chain(s, ol.fptr(p), ol.fptr(q), V, ol.iptr(x), k, max_emit, ol.iptr(out),
                                       C.byref(acc), C.byref(al))
        assert (got[0], got[1], got[3]) == (n, acc.value, al.value), rnd
        assert np.array_equal(got[4:4 + n], out[:n]), rnd
        assert list(dpos.read(np.int32, 2)) == [100 + n, out[n - 1]], rnd
        if use_budget:
            assert int(budget.read(np.int32, 1)[0]) == max_emit - n
        paths["accept"] += acc.value
        paths["bonus"] += al.value
        paths["reject"] += n - acc.value - al.value
    assert min(paths.values()) > 0 if V <= 4096 else paths["reject"] > 0, paths
    hn, hd = dev.alloc(4), dev.alloc(4 * 512)
    dev.check(L.orc_sampler_history(state.ptr, hd.ptr, 512, hn.ptr, None))
    nh = int(hn.read(np.int32, 1)[0])
    h = np.zeros(512, np.int32)
    nref = oracle.L.orco_sampler_history(s, ol.iptr(h), 512)
    assert nh == nref and np.array_equal(hd.read(np.int32, nh), h[:nref])
    oracle.L.orco_sampler_free(s)


@pytest.fixture(scope="module")
def pair(models_dir, oracle):
    import orc

    out = {}
    for name in ("t-qwen", "t-qwen-d", "t-q4k", "t-q4k-d"):
        print(f"[gpu] loading {name}", flush=True)
        out[name] = (orc.Model(models_dir / f"{name}.gguf", 0), ol.OracleModel(oracle, str(models_dir / f"{name}.gguf")))
    yield out
    for m, _ in out.values():
        m.close()


def _set_graphs(on):
    import orc

    return orc.load_host_lib().orch_set_graphs(int(on))


@pytest.mark.parametrize("k", [2, 4])
def test_spec_sampled_greedy_limit_matches_reference(pair, k):
    """At T = 0 without penalty the loop is the reference's speculative
    greedy decode: same stream and stats."""
    tgt, dft = pair["t-q4k"][0], pair["t-q4k-d"][0]
    toks, st = tgt.spec_sampled(dft, FIX["greedy/t-q4k/prompt"], 40, k, 0.0, 1.0, 0, 1.0, 64, 3)
    assert np.array_equal(toks, FIX[f"spec/k{k}/tokens"])
    assert [st["accepted"], st["proposed"], st["passes"]] == list(FIX[f"spec/k{k}/stats"])


@pytest.mark.parametrize("k,T,seed", [(3, 0.8, 4242), (2, 1.2, 7), (5, 0.6, 99)])
def test_spec_sampled_matches_oracle(pair, k, T, seed):
    """The device loop (graphs and host launches) gives the oracle loop's
    stream and stats on the qwen2 pair (independent draft) and on the Q4_K
    pair (draft close to the target, so long accepted runs occur)."""
    for tn, dn in (("t-qwen", "t-qwen-d"), ("t-q4k", "t-q4k-d")):
        (tgt, otgt), (dft, odft) = pair[tn], pair[dn]
        prompt = FIX[f"greedy/{tn}/prompt"]
        ref, rst = otgt.spec_sampled(odft, prompt, 40, k, T, 0.95, 40, 1.1, 64, seed)
        for graphs in (True, False):
            print(f"[gpu] spec_sampled {tn} k={k} T={T} graphs={graphs}", flush=True)
            prev = _set_graphs(graphs)
            try:
                toks, st = tgt.spec_sampled(dft, prompt, 40, k, T, 0.95, 40, 1.1, 64, seed)
            finally:
                _set_graphs(prev)
            assert np.array_equal(toks, ref), (tn, graphs, toks, ref)
            assert st == rst, (tn, graphs)
