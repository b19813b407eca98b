"""Graph capture of the MoE forward (hy_graph_*): a captured hy_moe_forward /
hy_moe_stack_forward, replayed several times with the program's own eager work and
synchronizations between the replays, equals the eager call bit for bit on every
replay, including after the input buffer's contents change (a replay reads the
captured pointers).  Covers the decode GEMV path (T=1, 4) and the MFMA path (T=100),
Q4_0 and Q8_0."""
import numpy as np
import pytest

import hy_oracle as O

pytestmark = pytest.mark.gpu

H, I, E, K = 256, 128, 16, 4


def _x(seed, T):
    return O.synth(seed, 0, O.T_X, 0, (T, H), 1.0)


@pytest.mark.parametrize("wtype,T", [(O.Q4_0, 1), (O.Q8_0, 4), (O.Q8_0, 100), (O.Q4_0, 100)])
def test_forward_replay_equals_eager(gpu, wtype, T):
    m = gpu.Moe(H, I, E, K, wtype, num_layers=2, max_tokens=128)
    m.synth(0, seed=11, std=0.05)
    m.synth(1, seed=12, std=0.05)
    st = gpu.Stream()
    xb, outg = gpu.Buf.from_array(_x(1, T)), gpu.Buf.empty((T, H))
    other_x, other_out = gpu.Buf.from_array(_x(2, 128)), gpu.Buf.empty((128, H))
    g = gpu.Graph(st, lambda: m.forward(0, xb, T, outg, st.h))
    try:
        for rep in range(3):
            # eager work in between: another layer / shape through the same work arena
            m.forward(1, other_x, 128 if rep % 2 == 0 else 3, other_out, st.h)
            st.synchronize()
            g.launch()
            st.synchronize()
            got = outg.numpy()
            ref_out = gpu.Buf.empty((T, H))
            m.forward(0, xb, T, ref_out, st.h)
            st.synchronize()
            np.testing.assert_array_equal(got.view(np.uint32), ref_out.numpy().view(np.uint32),
                                          err_msg=f"replay {rep}")
    finally:
        g.close()
        st.close()
        m.close()


def test_replay_reads_current_input_contents(gpu):
    T = 4
    m = gpu.Moe(H, I, E, K, O.Q4_0, num_layers=1, max_tokens=16)
    m.synth(0, seed=21, std=0.05)
    st = gpu.Stream()
    xb, outg = gpu.Buf.from_array(_x(5, T)), gpu.Buf.empty((T, H))
    g = gpu.Graph(st, lambda: m.forward(0, xb, T, outg, st.h))
    try:
        for seed in (6, 7):
            x = _x(seed, T)
            gpu.lib().hy_memcpy_h2d(xb.ptr, x.ctypes.data, x.nbytes)
            g.launch()
            st.synchronize()
            got = outg.numpy()
            ref = gpu.Buf.empty((T, H))
            m.forward(0, gpu.Buf.from_array(x), T, ref, st.h)
            st.synchronize()
            np.testing.assert_array_equal(got.view(np.uint32), ref.numpy().view(np.uint32), err_msg=f"seed {seed}")
    finally:
        g.close()
        st.close()
        m.close()


def test_stack_forward_replay(gpu):
    T, L = 8, 3
    m = gpu.Moe(H, I, E, K, O.Q8_0, num_layers=L, max_tokens=16)
    for l in range(L):
        m.synth(l, seed=30 + l, std=0.05)
    st = gpu.Stream()
    xb, outg, ref = gpu.Buf.from_array(_x(8, T)), gpu.Buf.empty((T, H)), gpu.Buf.empty((T, H))
    g = gpu.Graph(st, lambda: m.stack_forward(0, L, xb, T, 1e-5, outg, st.h))
    try:
        m.stack_forward(0, L, xb, T, 1e-5, ref, st.h)
        st.synchronize()
        want = ref.numpy().view(np.uint32)
        for rep in range(3):
            m.forward(1, xb, T, ref, st.h)   # eager work between replays
            st.synchronize()
            g.launch()
            st.synchronize()
            np.testing.assert_array_equal(outg.numpy().view(np.uint32), want, err_msg=f"replay {rep}")
    finally:
        g.close()
        st.close()
        m.close()


def test_capture_rejects_null_stream(gpu):
    with pytest.raises(gpu.HyError):
        gpu.check(gpu.lib().hy_graph_begin(None))


@pytest.mark.parametrize("T", [4, 100])
def test_routing_options_replay(gpu, T):
    """Group-limited greedy, dropping and the aux loss under capture: every replay equals
    the eager call, output and gate statistics (aux loss, capacity, capacity rate)."""
    m = gpu.Moe(H, I, E, K, O.Q8_0, num_layers=1, max_tokens=128, group_limited_greedy=1, n_group=4,
                topk_group=2, drop_tokens=1, capacity_factor=0.75, min_capacity=0, compute_aux_loss=1)
    m.synth(0, seed=41, std=0.05)
    st = gpu.Stream()
    xb, outg = gpu.Buf.from_array(_x(9, T)), gpu.Buf.empty((T, H))
    other = gpu.Buf.from_array(_x(10, 128))
    other_out = gpu.Buf.empty((128, H))
    g = gpu.Graph(st, lambda: m.forward(0, xb, T, outg, st.h))
    try:
        for rep in range(3):
            m.forward(0, other, 128 - 60 * rep, other_out, st.h)
            st.synchronize()
            g.launch()
            st.synchronize()
            got, gate_g = outg.numpy(), m.last_gate()  # the replay's own T, not the eager call's
            ref = gpu.Buf.empty((T, H))
            m.forward(0, xb, T, ref, st.h)
            st.synchronize()
            np.testing.assert_array_equal(got.view(np.uint32), ref.numpy().view(np.uint32), err_msg=f"replay {rep}")
            assert gate_g == m.last_gate()
    finally:
        g.close()
        st.close()
        m.close()


def test_lm_head_scratch_shape_refused_under_capture(gpu):
    """hy_lm_head_f32 shapes that take the stream-K split share a per-device scratch
    ordered by an event of the eager calls: under capture they are refused before
    anything is launched, and eager calls before and after agree bit for bit."""
    T, Hd, V = 256, 1024, 4096   # 64 output tiles of 128 x 128: the stream-K range
    rng = np.random.default_rng(5)
    x = rng.standard_normal((T, Hd)).astype(np.float32)
    w = (0.02 * rng.standard_normal((V, Hd))).astype(np.float32)
    before = gpu.lm_head_f32(x, w)
    xb, wb, ob = gpu.Buf.from_array(x), gpu.Buf.from_array(w), gpu.Buf.empty((T, V))
    st = gpu.Stream()
    with pytest.raises(gpu.HyError, match="cannot be captured"):
        gpu.Graph(st, lambda: gpu.check(gpu.lib().hy_lm_head_f32(xb.ptr, wb.ptr, None, T, Hd, V, ob.ptr, st.h)))
    st.close()
    after = gpu.lm_head_f32(x, w)
    np.testing.assert_array_equal(after.view(np.uint32), before.view(np.uint32))
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(after - ref).max() / np.abs(ref).max() < 1e-5
