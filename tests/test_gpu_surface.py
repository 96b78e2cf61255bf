"""The rest of the reference's C++ surface on the device path, against the
reference's own outputs:

  * namespace ops on host arrays (core/ops.hpp:42-92): rmsnorm, softmax, silu
    and rope against the reference's outputs (ref_fixtures.npz op/*), the rest
    against float64 closed forms; argmax exact, first index on ties;
  * the Sampler class (core/sampler.hpp:24-48): the reference's draws
    (sample/* fixtures), plus reset / set_params semantics;
  * Model::embed_tokens (core/model.cpp:248-270) against the reference's
    vector (surface_ref.npz embed/*);
  * .orkv files (core/model.cpp:156-236): a file the reference wrote loads
    and decodes to the reference's logits; our file has the reference's
    header and KV values; a save / reset / load round trip leaves the next
    logits bit for bit; load rejects a foreign configuration;
  * snapshot_kv / restore_kv (core/model.hpp:103-105) and
    test_norm_cache_matches (core/model.hpp:119-121).
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu
FIX = np.load(os.path.join(GOLDEN, "ref_fixtures.npz"))
SURF = np.load(os.path.join(GOLDEN, "surface_ref.npz"))


@pytest.fixture(scope="module")
def hops():
    import orc

    return orc.HostOps()


@pytest.fixture(scope="module")
def smodels(models_dir):
    import orc

    cache = {}

    def get(name):
        if name not in cache:
            print(f"[gpu] loading {name}", flush=True)
            cache[name] = orc.Model(models_dir / f"{name}.gguf")
        return cache[name]

    yield get
    for m in cache.values():
        m.close()


def test_ops_match_reference(hops):
    print("[gpu] ops vs reference", flush=True)
    x, g = FIX["op/x"], FIX["op/g"]
    for name, got in (("rmsnorm", hops.rmsnorm(x, g, 1e-5)), ("softmax", hops.softmax(x)), ("silu", hops.silu(x))):
        want = FIX[f"op/{name}"]
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7 * np.abs(want).max()), (name, np.abs(got - want).max())
    q, k = hops.rope(FIX["op/rope_q_in"], FIX["op/rope_k_in"], 24, 8, 128, 301, 500000.0)
    assert np.allclose(q, FIX["op/rope_q"], rtol=1e-6, atol=1e-6)
    assert np.allclose(k, FIX["op/rope_k"], rtol=1e-6, atol=1e-6)


def test_ops_any_size(hops):
    # rmsnorm of a length that is not a multiple of 4 (the reference's scalar
    # tail, core/ops.cpp:149-195) and rope with an odd head_dim (pairs
    # (i, i + hd/2), the last value untouched, core/ops.cpp:440-485),
    # against float64 closed forms
    print("[gpu] ops at odd sizes", flush=True)
    rng = np.random.default_rng(12)
    for n in (1, 3, 5, 3071):
        x = rng.normal(0, 1, n).astype(np.float32)
        g = rng.normal(1, 0.1, n).astype(np.float32)
        xd = x.astype(np.float64)
        want = xd / np.sqrt((xd * xd).mean() + 1e-5) * g
        got = hops.rmsnorm(x, g, 1e-5)
        assert np.allclose(got, want, rtol=1e-5, atol=1e-6 * np.abs(want).max()), (n, np.abs(got - want).max())
    hd, nh, nk, pos, base = 7, 3, 2, 5, 10000.0
    q = rng.normal(0, 1, nh * hd).astype(np.float32)
    k = rng.normal(0, 1, nk * hd).astype(np.float32)
    gq, gk = hops.rope(q, k, nh, nk, hd, pos, base)
    half = hd // 2
    i = np.arange(half)
    th = pos / np.power(base, 2.0 * i / hd)
    for got, src, nheads in ((gq, q, nh), (gk, k, nk)):
        want = src.astype(np.float64).reshape(nheads, hd).copy()
        a, b = want[:, :half].copy(), want[:, half:2 * half].copy()
        want[:, :half] = a * np.cos(th) - b * np.sin(th)
        want[:, half:2 * half] = a * np.sin(th) + b * np.cos(th)
        assert np.allclose(got.reshape(nheads, hd), want, rtol=1e-5, atol=1e-5)
        assert np.array_equal(got.reshape(nheads, hd)[:, -1], src.reshape(nheads, hd)[:, -1])


def test_ops_closed_forms(hops):
    print("[gpu] ops closed forms", flush=True)
    rng = np.random.default_rng(11)
    a = rng.normal(0, 1, (7, 300)).astype(np.float32)
    b = rng.normal(0, 1, (13, 300)).astype(np.float32)
    c = rng.normal(0, 1, (300, 13)).astype(np.float32)
    ad = a.astype(np.float64)
    for got, want, scale in ((hops.matmul(a, b), ad @ b.astype(np.float64).T, np.abs(ad) @ np.abs(b).T),
                             (hops.matmul(a, c, nn=True), ad @ c.astype(np.float64), np.abs(ad) @ np.abs(c))):
        assert np.all(np.abs(got - want) <= 1e-6 * scale + 1e-30)
    u, v = a[0], a[1]
    assert np.array_equal(hops.mul(u, v), u * v)
    assert np.array_equal(hops.add(u, v), u + v)
    assert np.array_equal(hops.copy(u), u)
    d = hops.dot(u, v)
    assert abs(d - float(u.astype(np.float64) @ v)) <= 1e-6 * float(np.abs(u) @ np.abs(v))
    t = np.zeros(1000, np.float32)
    t[[17, 400, 999]] = 3.0  # ties: the first index wins
    assert hops.argmax(t) == 17
    t[5] = np.float32(-1e30)
    assert hops.argmax(t) == 17
    assert hops.argmax(-np.abs(a[2])) == int(np.argmax(-np.abs(a[2])))


def test_sampler_class_matches_reference():
    """Sampler(params, seed) with the history recorded through record() draws
    the reference's ids; the row is rewritten in place (probabilities when
    T > 0); reset() clears the history but keeps the generator; set_params()
    keeps both."""
    import orc

    lg, hist = FIX["sample/logits"], FIX["sample/history"].astype(np.int32)
    for i in range(5):
        T, P, K, pen, last = FIX[f"sample/{i}/params"]
        seed = int(FIX[f"sample/{i}/seed"][0])
        print(f"[gpu] Sampler case {i}", flush=True)
        s = orc.Sampler(float(T), float(P), int(K), float(pen), int(last), seed)
        for h in hist:
            s.record(int(h))
        draws = []
        for _ in range(64):
            row = lg.copy()
            draws.append(s.sample(row))
        assert draws == list(FIX[f"sample/{i}/draws"]), i
        if T > 0:
            assert abs(float(row.astype(np.float64).sum()) - 1.0) < 1e-4  # softmaxed in place
    # reset: history gone, generator continues. Compare with a fresh sampler
    # that drew the same number of times without history.
    T, P, K, pen, last = FIX["sample/1/params"]
    seed = int(FIX["sample/1/seed"][0])
    a = orc.Sampler(float(T), float(P), int(K), float(pen), int(last), seed)
    b = orc.Sampler(float(T), float(P), int(K), float(pen), int(last), seed)
    for h in hist:
        a.record(int(h))
    for _ in range(3):
        a.sample(lg.copy())
        b.sample(lg.copy())
    a.reset()
    b.reset()
    assert [a.sample(lg.copy()) for _ in range(8)] == [b.sample(lg.copy()) for _ in range(8)]
    # set_params: T = 0 makes the next draw the argmax
    a.set_params(0.0, float(P), int(K), 1.0, int(last))
    assert a.sample(lg.copy()) == int(np.argmax(lg))


def test_sampler_repeat_window_limits(oracle):
    """A repeat window of up to 4095 ids penalises exactly as the reference's
    Sampler (core/sampler.cpp:15-27, 99-105; the CPU oracle restates it) over a
    history longer than the device buffer; a larger window is refused when the
    Sampler is built (the C API returns no handle), not later as -1 ids."""
    import orc

    with pytest.raises(orc.OrcError):
        orc.Sampler(0.8, 0.95, 40, 1.1, 4096, 3)
    rng = np.random.default_rng(21)
    V = 512
    for last in (3000, 4095):
        print(f"[gpu] Sampler repeat_last={last}", flush=True)
        s = orc.Sampler(0.0, 1.0, 40, 1.5, last, 3)  # T = 0: argmax after the penalty
        o = oracle.L.orco_sampler_new(0.0, 1.0, 40, 1.5, last, 3)
        hist = rng.integers(0, 40, 9000).astype(np.int32)  # more than the 4096 the device holds
        for h in hist:
            s.record(int(h))
            oracle.L.orco_sampler_record(o, int(h))
        for trial in range(6):
            lg = rng.normal(0, 1, V).astype(np.float32)
            lg[:40] += 3.0  # penalised ids compete for the argmax
            lo = lg.copy()
            want = oracle.L.orco_sampler_sample(o, lo.ctypes.data_as(orc._fp), V)
            assert s.sample(lg.copy()) == want, (last, trial)
        oracle.L.orco_sampler_free(o)


@pytest.mark.parametrize("m", ["t-q8", "t-q4k"])
def test_embed_tokens_matches_reference(smodels, m):
    print(f"[gpu] embed_tokens {m}", flush=True)
    mod = smodels(m)
    got = mod.embed_tokens(SURF[f"embed/{m}/ids"])
    want = SURF[f"embed/{m}"]
    assert abs(float(np.linalg.norm(got)) - 1.0) < 1e-5
    assert np.abs(got - want).max() <= 1e-4, np.abs(got - want).max()
    # the KV cache is cleared afterwards: a decode from position 0 equals a fresh one
    mod.reset()
    fresh = mod.forward(5, 0)
    mod.embed_tokens(SURF[f"embed/{m}/ids"])
    assert np.array_equal(mod.forward(5, 0), fresh)


@pytest.mark.parametrize("m", ["t-q8", "t-q4k"])
def test_orkv_reference_file_loads_and_decodes(smodels, m, tmp_path):
    print(f"[gpu] orkv reference file {m}", flush=True)
    mod = smodels(m)
    ref_file = tmp_path / "ref.orkv"
    SURF[f"orkv/{m}/file"].tofile(ref_file)
    prompt = SURF[f"orkv/{m}/prompt"]
    mod.reset()
    assert mod.load_state(ref_file) == len(prompt) - 1
    lg = mod.forward(int(prompt[-1]), len(prompt) - 1)
    want = SURF[f"orkv/{m}/logits"]
    assert np.abs(lg - want).max() <= 1e-4 * np.abs(want).max()


@pytest.mark.parametrize("m", ["t-q8", "t-q4k"])
def test_orkv_save_matches_reference_format_and_round_trips(smodels, m, tmp_path):
    print(f"[gpu] orkv save {m}", flush=True)
    mod = smodels(m)
    prompt = SURF[f"orkv/{m}/prompt"]
    n = len(prompt) - 1
    mod.reset()
    mod.forward_batch(prompt[:n], 0, logits=False)
    path = tmp_path / "ours.orkv"
    mod.save_state(path, n)
    ours, ref = np.fromfile(path, np.uint8), SURF[f"orkv/{m}/file"]
    assert ours.size == ref.size
    # magic, version, the ModelConfig fields (44 bytes, the last 3 padding), pos, n
    assert np.array_equal(ours[:49], ref[:49]) and np.array_equal(ours[52:64], ref[52:64])
    kv_o, kv_r = ours[64:].view(np.float32), ref[64:].view(np.float32)
    assert np.abs(kv_o - kv_r).max() <= 1e-4 * max(1.0, float(np.abs(kv_r).max()))
    # round trip: decode after save / reset / load equals decode without it
    want = mod.forward(int(prompt[-1]), n)
    mod.reset()
    assert mod.load_state(path) == n
    assert np.array_equal(mod.forward(int(prompt[-1]), n), want)
    # a file of another configuration is rejected, and a missing one too
    other = smodels("t-q8" if m != "t-q8" else "t-qwen-d")
    if other.embed_dim != mod.embed_dim or other.n_kv_heads != mod.n_kv_heads or other.n_layers != mod.n_layers:
        assert other.load_state(path) is None
    assert mod.load_state(tmp_path / "missing.orkv") is None


def test_snapshot_restore_and_norm_cache(smodels):
    print("[gpu] snapshot / restore", flush=True)
    mod = smodels("t-q4k")
    prompt = SURF["orkv/t-q4k/prompt"]
    mod.reset()
    mod.forward_batch(prompt[:8], 0, logits=False)
    snap = mod.snapshot_kv(8)
    assert snap.pos == 8
    a = [mod.forward(int(t), 8 + i) for i, t in enumerate(prompt[8:11])]
    mod.forward_batch(prompt[:3], 8, logits=False)  # overwrite positions 8..10
    mod.restore_kv(snap)
    b = [mod.forward(int(t), 8 + i) for i, t in enumerate(prompt[8:11])]
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    assert mod.norm_cache_matches()
