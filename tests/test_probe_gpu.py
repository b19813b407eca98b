"""The measurement probes bench.py reports ceilings from (libhy_probe.so, built beside
the product library): they must do the work they claim.  The stream probe's per-lane
checksum equals the bytes it read; the block-mix probe's variants run and give finite
results; bad arguments are rejected."""
import numpy as np
import pytest

import bench

pytestmark = pytest.mark.gpu


def test_stream_probe_reads_every_step(gpu):
    """Each wave's lane l adds word l of every 8 KB step it streamed: with the buffer set
    to bytes of 1, every lane's sum is steps x 0x01010101, so a step read before its copy
    landed (or skipped) would show."""
    P = bench.probe_lib()
    waves, steps = 96, 5
    nbytes = waves * steps * 8192
    buf = gpu.Buf(nbytes, np.uint8)
    gpu.check(gpu.lib().hy_memset(buf.ptr, 1, nbytes))
    out = gpu.Buf.empty((waves * 64,))
    for variant in (0, 2):  # plain and non-temporal copies
        bench.probe_check(P.hyp_stream(variant, buf.ptr, nbytes, waves, out.ptr, None))
        gpu.sync()
        np.testing.assert_array_equal(out.numpy(), np.full(waves * 64, np.float32(steps * 0x01010101)))
    bench.probe_check(P.hyp_stream(1, buf.ptr, nbytes, waves, out.ptr, None))
    gpu.sync()
    assert np.all(np.isfinite(out.numpy()))


def test_stream_probe_rejects_bad_sizes(gpu):
    P = bench.probe_lib()
    buf = gpu.Buf(8192 * 8, np.uint8)
    out = gpu.Buf.empty((8 * 64,))
    for variant, nbytes, waves in ((0, 8192 * 8 - 16, 8), (0, 8192 * 8, 0), (3, 8192 * 8, 8), (1, 8192 * 6, 6)):
        with pytest.raises(RuntimeError, match="bad stream probe arguments"):
            bench.probe_check(P.hyp_stream(variant, buf.ptr, nbytes, waves, out.ptr, None))


def test_block_mix_probe_variants(gpu):
    P = bench.probe_lib()
    wgs = 8
    out = gpu.Buf.empty((wgs * 512,))
    for variant in range(5):
        bench.probe_check(P.hyp_block_mix(variant, wgs, 20, out.ptr, None))
        gpu.sync()
        assert np.all(np.isfinite(out.numpy()))
    for variant in (5, -1):
        with pytest.raises(RuntimeError, match="bad block-mix probe arguments"):
            bench.probe_check(P.hyp_block_mix(variant, wgs, 20, out.ptr, None))


def test_l2_window_probe_copies(gpu):
    """Every wave's lane l reads back word l of the last batch's first copied KB: with the
    window set to bytes of 1 it is 0x01010101, so a batch read before its copies landed
    would show; windows that are not a power-of-two number of KB are rejected."""
    P = bench.probe_lib()
    kb, wgs = 64, 16
    buf = gpu.Buf(kb * 1024, np.uint8)
    gpu.check(gpu.lib().hy_memset(buf.ptr, 1, kb * 1024))
    out = gpu.Buf.empty((wgs * 256,))
    bench.probe_check(P.hyp_l2_window(buf.ptr, kb * 1024, wgs, 7, out.ptr, None))
    gpu.sync()
    np.testing.assert_array_equal(out.numpy(), np.full(wgs * 256, np.float32(0x01010101)))
    for nbytes in (kb * 1024 - 16, 48 * 1024, 0):
        with pytest.raises(RuntimeError, match="bad L2 window probe arguments"):
            bench.probe_check(P.hyp_l2_window(buf.ptr, nbytes, wgs, 7, out.ptr, None))
