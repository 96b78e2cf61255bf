"""orc_argmax_noalloc, the allocation-free variant of orc_argmax (its partial
maxima live in a library-owned device array instead of a caller workspace),
called through the C ABI: on two calls in a row, the second with a smaller
input, it returns exactly what orc_argmax returns on the same rows (first
index of the maximum, ties to the lowest index as ops::argmax,
core/ops.cpp:490-497), and it refuses more rows than its array holds."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _rows(rng, n_rows, n, ld):
    x = rng.standard_normal((n_rows, ld)).astype(np.float32)
    x[:, n:] = 1e30  # padding past n must never be chosen
    for r in range(n_rows):
        top = float(x[r, :n].max()) + 1.0
        a, b = sorted(rng.choice(n, 2, replace=False))
        x[r, a] = x[r, b] = top  # a tie: the lower index wins
    x[0, :n] = -3.5  # an all-equal row: index 0
    return x


def _argmax_ws(dev, dx, n_rows, n, ld):
    ws = dev.alloc(dev.L.orc_argmax_workspace(n_rows, n))
    out = dev.alloc(4 * n_rows)
    dev.check(dev.L.orc_argmax(dx.ptr, n_rows, n, ld, out.ptr, ws.ptr, None))
    return out.read(np.int32)


def test_argmax_noalloc_matches_argmax(dev):
    rng = np.random.default_rng(31)
    for n_rows, n in ((16, 152064), (3, 5000)):  # the second call is smaller
        ld = n + 12
        print(f"[gpu] argmax_noalloc rows={n_rows} n={n}", flush=True)
        x = _rows(rng, n_rows, n, ld)
        dx, out = dev.upload(x), dev.alloc(4 * n_rows)
        dev.check(dev.L.orc_argmax_noalloc(dx.ptr, n_rows, n, ld, out.ptr, None))
        got = out.read(np.int32)
        want = _argmax_ws(dev, dx, n_rows, n, ld)
        assert np.array_equal(got, want), (n_rows, n)
        assert np.array_equal(got, np.argmax(x[:, :n], axis=1).astype(np.int32)), (n_rows, n)
        assert got[0] == 0


def test_argmax_noalloc_refuses_more_rows_than_its_scratch(dev):
    x = dev.upload(np.zeros((17, 64), np.float32))
    out = dev.alloc(4 * 17)
    assert dev.L.orc_argmax_noalloc(x.ptr, 17, 64, 64, out.ptr, None) == -1  # ORC_E_INVALID
    assert b"at most 16 rows" in dev.L.orc_last_error()
