"""hy_dispatch_pairs_noalloc (the dispatch with its workspace in a fixed device array)
against hy_dispatch_pairs (the entry point that allocates its workspace per call):
bit-exact counts, offsets and positions on two calls in a row, the second smaller,
so the second call runs over the stale contents the first left in the shared
array; both are also held to the brute-force capacity-slot order."""
import numpy as np
import pytest

from test_gpu_parity import _dispatch_expected

pytestmark = pytest.mark.gpu


def _pairs(T, K, E, seed, skew):
    rng = np.random.default_rng(seed)
    p = np.ones(E) if not skew else 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    idx = np.stack([rng.choice(E, size=K, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    return idx, rng.random((T, K)).astype(np.float32)


def _dispatch(gpu, fn, idx, w, E, stream=None):
    T, K = idx.shape
    ib, wb = gpu.Buf.from_array(idx), gpu.Buf.from_array(w)
    cb, ob, pb = gpu.Buf.empty((E,), np.int32), gpu.Buf.empty((E + 1,), np.int32), gpu.Buf.empty((T, K), np.int32)
    gpu.check(fn(ib.ptr, wb.ptr, T, K, E, cb.ptr, ob.ptr, pb.ptr, stream))
    return cb.numpy(), ob.numpy(), pb.numpy()   # numpy() waits for the device


def test_noalloc_dispatch_equals_allocating_entry_point(gpu):
    E, K = 64, 8
    for T, skew in ((5000, True), (300, False)):
        idx, w = _pairs(T, K, E, seed=T, skew=skew)
        ref = _dispatch(gpu, gpu.lib().hy_dispatch_pairs, idx, w, E)
        got = _dispatch(gpu, gpu.lib().hy_dispatch_pairs_noalloc, idx, w, E)
        for name, a, b, c in zip(("counts", "offsets", "pos"), got, ref, _dispatch_expected(idx, E)):
            np.testing.assert_array_equal(a, b, err_msg=f"T={T} {name}")
            np.testing.assert_array_equal(a, c, err_msg=f"T={T} {name} (brute force)")


def test_noalloc_dispatch_largest_shape(gpu):
    """T = 16384, K = 16, E = 64: the largest call the entry point accepts fits its array."""
    T, K, E = 16384, 16, 64
    idx, w = _pairs(T, K, E, seed=1, skew=True)
    ref = _dispatch(gpu, gpu.lib().hy_dispatch_pairs, idx, w, E)
    got = _dispatch(gpu, gpu.lib().hy_dispatch_pairs_noalloc, idx, w, E)
    for a, b in zip(got, ref):
        np.testing.assert_array_equal(a, b)


def test_noalloc_dispatch_back_to_back_on_one_stream(gpu):
    """Two calls queued on one stream with no host wait between them: the stream
    orders them, so the second's use of the shared array follows the first's."""
    E, K = 64, 8
    st = gpu.Stream()
    cases = [_pairs(T, K, E, seed=7 + T, skew=False) for T in (2048, 40)]
    bufs = []
    for idx, w in cases:
        T = idx.shape[0]
        b = dict(i=gpu.Buf.from_array(idx), w=gpu.Buf.from_array(w), c=gpu.Buf.empty((E,), np.int32),
                 o=gpu.Buf.empty((E + 1,), np.int32), p=gpu.Buf.empty((T, K), np.int32))
        gpu.check(gpu.lib().hy_dispatch_pairs_noalloc(b["i"].ptr, b["w"].ptr, T, K, E, b["c"].ptr, b["o"].ptr,
                                                      b["p"].ptr, st.h))
        bufs.append(b)
    st.synchronize()
    for (idx, _), b in zip(cases, bufs):
        for a, c in zip((b["c"].numpy(), b["o"].numpy(), b["p"].numpy()), _dispatch_expected(idx, E)):
            np.testing.assert_array_equal(a, c)
    st.close()


def test_noalloc_dispatch_rejects_bad_shapes(gpu):
    # too many tokens, top-k past its bound, too many experts, no tokens, and a shape
    # whose workspace exceeds the fixed array (T*K = 524,288 pairs)
    for T, K, E in ((16385, 8, 64), (4, 65, 64), (4, 8, 65), (0, 8, 64), (16384, 32, 64)):
        idx = gpu.Buf.empty((max(T, 1), K), np.int32)
        w = gpu.Buf.empty((max(T, 1), K))
        out = gpu.Buf.empty((max(T, 1) * K + E + 1,), np.int32)
        with pytest.raises(gpu.HyError):
            gpu.check(gpu.lib().hy_dispatch_pairs_noalloc(idx.ptr, w.ptr, T, K, E, out.ptr, out.ptr, out.ptr, None))
