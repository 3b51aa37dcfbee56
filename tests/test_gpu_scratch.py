"""The context's scratch under HIP graph capture (include/spq4k.h,
spq4k_reserve): a graph captured before the scratch grows keeps working
after it grows, and a call that would have to grow the scratch while its
stream is being captured is refused with -EBUSY instead of allocating.

Outputs are checked against the CPU oracle (close_enough, 1e-4 relative or
1e-5 absolute, tests/desktop/test_sp_kernels.cpp:34-48) on a sample of the
tokens of the large calls (every token of a matmul is independent)."""
import errno

import numpy as np
import pytest

from _oracle import close_enough

pytestmark = pytest.mark.gpu

M, K = 256, 4096
T_SMALL, T_BIG = 64, 4096   # Q8_K planes of 4096 rows of K = 4096: 22 MiB, above the initial 16 MiB


def _setup(oracle, seed):
    import spq4k
    from spq4k.hip import DeviceArray
    c = spq4k.Context(0)
    rng = np.random.default_rng(seed)
    W = oracle.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
    Wd = c.upload(W, M, K)
    Xs = rng.standard_normal((T_SMALL, K)).astype(np.float32)
    Xb = rng.standard_normal((T_BIG, K)).astype(np.float32)
    bufs = {"xs": DeviceArray.from_host(Xs), "ys": DeviceArray((T_SMALL, M)),
            "xb": DeviceArray.from_host(Xb), "yb": DeviceArray((T_BIG, M))}
    return c, W, Wd, Xs, Xb, bufs


def _check_sample(oracle, W, X, Y, what):
    idx = np.r_[0:8, X.shape[0] - 8:X.shape[0]]
    exp = oracle.mul_mat(W, M, K, np.ascontiguousarray(X[idx]))
    ok = close_enough(Y[idx], exp)
    assert ok.all(), f"{what}: {int((~ok).sum())}/{ok.size} outside tolerance"


def test_graph_survives_scratch_growth(oracle):
    from spq4k.hip import DeviceArray, Graph
    c, W, Wd, Xs, Xb, b = _setup(oracle, 11)
    try:
        with Graph.capture(c.stream) as g:
            c.mul_mat_dev(Wd, b["xs"].ptr, b["ys"].ptr, T_SMALL)
        # a larger call grows the scratch; memory taken after it would reuse
        # a scratch buffer that had been freed
        c.mul_mat_dev(Wd, b["xb"].ptr, b["yb"].ptr, T_BIG)
        c.synchronize()
        _check_sample(oracle, W, Xb, b["yb"].to_host(), "call that grew the scratch")
        fill = [DeviceArray(16 << 20, np.uint8) for _ in range(4)]
        for f in fill:
            f.fill_byte(0xA5)
        for _ in range(3):
            g.launch()
            c.synchronize()
            _check_sample(oracle, W, Xs, b["ys"].to_host(), "graph captured before the growth")
        for i, f in enumerate(fill):
            assert (f.to_host() == 0xA5).all(), f"allocation {i} made after the growth was written by the replay"
    finally:
        c.close()


def test_growth_during_capture_is_refused(oracle):
    import spq4k
    from spq4k.hip import Graph
    c, W, Wd, Xs, Xb, b = _setup(oracle, 12)
    try:
        with pytest.raises(spq4k.Spq4kError) as ei:
            with Graph.capture(c.stream):
                c.mul_mat_dev(Wd, b["xb"].ptr, b["yb"].ptr, T_BIG)
        assert ei.value.rc == -errno.EBUSY, str(ei.value)
        # calls that fit still capture and replay
        with Graph.capture(c.stream) as g:
            c.mul_mat_dev(Wd, b["xs"].ptr, b["ys"].ptr, T_SMALL)
        g.launch()
        c.synchronize()
        _check_sample(oracle, W, Xs, b["ys"].to_host(), "small call after the refused capture")
        # reserving ahead of the capture lets the large call in
        c.reserve(64 << 20, 0)
        with Graph.capture(c.stream) as g2:
            c.mul_mat_dev(Wd, b["xb"].ptr, b["yb"].ptr, T_BIG)
        for _ in range(2):
            g2.launch()
            c.synchronize()
            _check_sample(oracle, W, Xb, b["yb"].to_host(), "large call captured after spq4k_reserve")
    finally:
        c.close()
