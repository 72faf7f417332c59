"""marian_hip_vocab_argmax_noalloc against marian_hip_vocab_argmax, through the C ABI.

The allocation-free entry point keeps its partial argmax keys in the library's
fixed device array instead of library scratch; tokens and logits must be
identical to the allocating entry point's, bit for bit, on consecutive calls
(the second with fewer rows, so stale keys of the first call stay in the array)
and at the largest input the array holds.
"""

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

V, K = 32000, 512
MAX_ROWS = 131072 // ((V + 127) // 128)  # 524 rows at V = 32000


@pytest.fixture(scope="module")
def dev(pkg):
    from importlib import import_module

    d = import_module(pkg.__name__ + ".device")
    assert d.device_count() >= 1, "no HIP device visible"
    return d


@pytest.fixture(scope="module")
def weights(dev):
    rng = np.random.default_rng(71)
    emb = rng.integers(-127, 128, size=(V, K)).astype(np.int8)
    mult = rng.uniform(50.0, 1000.0, size=V).astype(np.float32)
    bias = (rng.standard_normal(V) * 0.02).astype(np.float32)
    return tuple(dev.DeviceArray.from_host(x) for x in (emb, mult, bias))


def run(pkg, dev, weights, M, seed, entry):
    lib = pkg._lib.load()
    rng = np.random.default_rng(seed)
    xq = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
    xa = rng.uniform(1.0, 50.0, size=M).astype(np.float32)
    dq, da = dev.DeviceArray.from_host(xq), dev.DeviceArray.from_host(xa)
    tok = dev.DeviceArray.zeros(M, np.int32)
    lg = dev.DeviceArray.zeros((M, V), np.float32)
    emb, mult, bias = weights
    fn = getattr(lib, entry)
    rc = fn(dq.ptr, da.ptr, M, K, emb.ptr, mult.ptr, bias.ptr, V, 0, tok.ptr, lg.ptr, None)
    dev.synchronize()
    return rc, tok.host(), lg.host()


def test_noalloc_matches_allocating_entry_point(pkg, dev, weights):
    for M, seed in ((96, 1), (5, 2), (MAX_ROWS, 3)):
        print(f"vocab_argmax_noalloc M={M} V={V}", flush=True)
        rc0, t0, l0 = run(pkg, dev, weights, M, seed, "marian_hip_vocab_argmax")
        rc1, t1, l1 = run(pkg, dev, weights, M, seed, "marian_hip_vocab_argmax_noalloc")
        assert rc0 == 0 and rc1 == 0
        assert np.array_equal(t0, t1), f"tokens differ at M={M}"
        assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32)), f"logits differ at M={M}"
        assert np.array_equal(t1, np.argmax(np.where(np.isfinite(l1), l1, -np.inf), axis=1))


def test_noalloc_rejects_inputs_beyond_its_array(pkg, dev, weights):
    lib = pkg._lib.load()
    M = MAX_ROWS + 1
    xq = dev.DeviceArray.zeros((M, K), np.int8)
    xa = dev.DeviceArray.from_host(np.ones(M, np.float32))
    tok = dev.DeviceArray.zeros(M, np.int32)
    emb, mult, bias = weights
    rc = lib.marian_hip_vocab_argmax_noalloc(xq.ptr, xa.ptr, M, K, emb.ptr, mult.ptr, bias.ptr, V,
                                             0, tok.ptr, None, None)
    assert rc == pkg._lib.ERR_INVALID_INPUT
    assert "exceed" in pkg._lib.op_error()
    # the array is still usable afterwards
    rc1, t1, _ = run(pkg, dev, weights, 3, 9, "marian_hip_vocab_argmax_noalloc")
    rc0, t0, _ = run(pkg, dev, weights, 3, 9, "marian_hip_vocab_argmax")
    assert rc1 == 0 and np.array_equal(t0, t1)
