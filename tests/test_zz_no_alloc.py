"""rsv_sample_noalloc (the allocation-free sampler entry point) against
rsv_sample, through the C-ABI: the same token on the same inputs, on two
calls in a row (the second with a smaller vocabulary, so the static work
area holds the first call's larger contents), with and without a
penalty history; sizes past the work area's limit are rejected."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NONE = 0xFFFFFFFF


@pytest.fixture(scope="module")
def be():
    import rsv
    b = rsv.Backend(0)
    yield b
    b.close()


def _pair(be, logits, temperature, top_k, top_p, seed, rep=1.0, freq=0.0, pres=0.0, hist=()):
    import rsv
    lt = be.tensor(logits)
    t_alloc, t_free = be.tensor(n=1, dtype=rsv.U32), be.tensor(n=1, dtype=rsv.U32)
    h = np.ascontiguousarray(np.asarray(hist, np.uint32)) if len(hist) else np.zeros(1, np.uint32)
    be.call("rsv_sample", lt, t_alloc, logits.size, temperature, top_k, top_p, seed, rep, freq, pres,
            h.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(hist))
    ht = be.tensor(h.astype(np.uint32), dtype=rsv.U32) if len(hist) else NONE
    be.call("rsv_sample_noalloc", lt, t_free, logits.size, temperature, top_k, top_p, seed, rep, freq, pres,
            ht, len(hist))
    return int(be.get(t_alloc, 1, rsv.U32)[0]), int(be.get(t_free, 1, rsv.U32)[0])


@pytest.mark.parametrize("top_k,top_p", [(0, 0.9), (40, 0.8), (0, 1.0), (300, 0.95)])
def test_sample_noalloc_matches_sample(be, top_k, top_p):
    rng = np.random.default_rng(7 + top_k)
    # second call smaller than the first; 65529 and 3000 are not multiples
    # of 1024 (the general kernels), 65536 and 4096 the register-resident ones
    for n, seed in ((65536, 11), (4096, 12), (65529, 13), (3000, 14)):
        lg = rng.standard_normal(n).astype(np.float32) * 2.0
        a, b = _pair(be, lg, 1.0, top_k, top_p, seed)
        assert a == b, (n, a, b)
        hist = rng.integers(0, n, size=37).tolist()
        a, b = _pair(be, lg, 0.7, top_k, top_p, seed + 1, rep=1.3, freq=0.2, pres=0.1, hist=hist)
        assert a == b, (n, a, b)


def test_sample_noalloc_limits(be):
    import rsv
    lt = be.tensor(n=262145)
    tok = be.tensor(n=1, dtype=rsv.U32)
    with pytest.raises(rsv.RsvError, match="work area"):
        be.call("rsv_sample_noalloc", lt, tok, 262145, 1.0, 0, 0.9, 1, 1.0, 0.0, 0.0, NONE, 0)
    short = be.tensor(np.zeros(3, np.uint32), dtype=rsv.U32)
    with pytest.raises(rsv.RsvError):
        be.call("rsv_sample_noalloc", lt, tok, 1000, 1.0, 0, 0.9, 1, 1.1, 0.0, 0.0, short, 5)


def test_sample_noalloc_one_context_per_device(be):
    """A second context on the device is refused while the owner lives (the
    work area is per device); it may use it once the owner is destroyed."""
    import rsv
    lg = np.random.default_rng(3).standard_normal(4096).astype(np.float32)
    lt, tok = be.tensor(lg), be.tensor(n=1, dtype=rsv.U32)
    be.call("rsv_sample_noalloc", lt, tok, 4096, 1.0, 0, 0.9, 5, 1.0, 0.0, 0.0, NONE, 0)
    other = rsv.Backend(0)
    try:
        lt2, tok2 = other.tensor(lg), other.tensor(n=1, dtype=rsv.U32)
        with pytest.raises(rsv.RsvError, match="another context"):
            other.call("rsv_sample_noalloc", lt2, tok2, 4096, 1.0, 0, 0.9, 5, 1.0, 0.0, 0.0, NONE, 0)
        first = rsv.Backend(0)
        first.close()  # destroying a non-owner leaves the owner in place
        with pytest.raises(rsv.RsvError, match="another context"):
            other.call("rsv_sample_noalloc", lt2, tok2, 4096, 1.0, 0, 0.9, 5, 1.0, 0.0, 0.0, NONE, 0)
    finally:
        other.close()
