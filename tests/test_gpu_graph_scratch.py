"""Kernel-level calls captured into a HIP graph and the per-stream scratch.

lh_linear quantizes its input and keeps split-K sums in a scratch buffer of
its stream.  A graph captured with it keeps that buffer's address, so:
* replays equal the eager call bit for bit, with other eager work and
  synchronizations between them;
* a call that would have to grow the scratch while the stream captures is
  refused with LH_ERROR_STATE, the stream leaves capture and still works;
* an eager call that grows the scratch afterwards keeps the old buffer alive,
  and the earlier graph still replays to the same outputs.
"""
from __future__ import annotations

import numpy as np
import pytest

from leaf_amd.artifact import quantize

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from leaf_amd import runtime
    runtime.library()
    return runtime


def test_captured_linear_replays_and_scratch_growth_is_refused_in_capture(rt):
    rng = np.random.default_rng(29)
    K, N, M, M_big = 2048, 2048, 64, 4096
    w = (0.02 * rng.standard_normal((N, K))).astype(np.float32)
    data, scales = quantize(w, 8, K)
    dw = rt.DeviceWeight(data, 8, K, scales, K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    x_big = rng.standard_normal((M_big, K), dtype=np.float32)
    dx, dx_big = rt.DeviceArray.of(x), rt.DeviceArray.of(x_big)
    dy, dy_big = rt.DeviceArray((M, N), np.float32), rt.DeviceArray((M_big, N), np.float32)
    dacc = rt.DeviceArray((M, N, 1), np.int32)

    stream = rt.Stream()
    rt.linear(dw, dx, M, 8, dy, dacc, stream=stream.handle)   # sizes the stream's scratch
    stream.synchronize()
    want_y, want_acc = dy.numpy(), dacc.numpy()

    graph = rt.Graph(stream, lambda: rt.linear(dw, dx, M, 8, dy, dacc, stream=stream.handle))

    def replay_matches():
        dy.zero()
        dacc.zero()
        rt.linear(dw, dx, M, 8, dy_big, stream=None)   # unrelated eager work on the null stream
        rt.synchronize()                                # the stream is non-blocking: order by hand
        graph.launch()
        stream.synchronize()
        return (np.array_equal(dy.numpy().view(np.uint32), want_y.view(np.uint32))
                and np.array_equal(dacc.numpy(), want_acc))

    for replay in range(3):
        assert replay_matches(), f"replay {replay} differs from the eager call"

    with pytest.raises(rt.LeafError, match="grow outside stream capture"):
        rt.Graph(stream, lambda: rt.linear(dw, dx_big, M_big, 8, dy_big, stream=stream.handle))
    assert replay_matches(), "replay after the refused capture differs"

    rt.linear(dw, dx_big, M_big, 8, dy_big, stream=stream.handle)   # grows the scratch eagerly
    stream.synchronize()
    assert replay_matches(), "replay after the scratch grew differs"
    graph.close()
    stream.close()


def test_destroyed_streams_release_their_scratch_and_captured_ones_keep_it(rt):
    """lh_stream_destroy frees the stream's kernel scratch (a caller that makes
    a stream per request does not leak device memory), except for a stream
    that was captured: its graph may still be launched on another stream."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]

    def free_bytes():
        free, total = C.c_size_t(), C.c_size_t()
        assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
        return free.value

    rng = np.random.default_rng(31)
    K, N, M = 2048, 2048, 64
    data, scales = quantize((0.02 * rng.standard_normal((N, K))).astype(np.float32), 8, K)
    dw = rt.DeviceWeight(data, 8, K, scales, K)
    dx = rt.DeviceArray.of(rng.standard_normal((M, K), dtype=np.float32))
    dy = rt.DeviceArray((M, N), np.float32)
    rt.linear(dw, dx, M, 8, dy, stream=None)
    rt.synchronize()
    want = dy.numpy()

    streams = 48
    before = free_bytes()
    for _ in range(streams):
        s = rt.Stream()
        rt.linear(dw, dx, M, 8, dy, stream=s.handle)   # at least 1 MiB of scratch for this stream
        s.close()
    dropped = before - free_bytes()
    print(f"device memory after {streams} streams: {dropped / 2**20:.1f} MiB less free")
    assert dropped < 16 << 20, f"{streams} destroyed streams kept {dropped} bytes"
    assert np.array_equal(dy.numpy().view(np.uint32), want.view(np.uint32))

    captured = rt.Stream()
    rt.linear(dw, dx, M, 8, dy, stream=captured.handle)
    captured.synchronize()
    graph = rt.Graph(captured, lambda: rt.linear(dw, dx, M, 8, dy, stream=captured.handle))
    captured.close()
    other = rt.Stream()
    for replay in range(3):
        dy.zero()
        rt.synchronize()
        rt.check(rt.library().lh_graph_launch(graph.handle, other.handle))
        other.synchronize()
        assert np.array_equal(dy.numpy().view(np.uint32), want.view(np.uint32)), f"replay {replay} differs"
    graph.close()
    other.close()
