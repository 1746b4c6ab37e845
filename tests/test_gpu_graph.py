"""HIP graph capture of the encoder path.

A serving loop captures the encoder once and replays it (hipGraphLaunch),
which removes the per-kernel host launch cost.  That works when a run, once
its runtime's workspaces exist, issues only kernel launches on the runtime's
stream: no allocation, no synchronisation, no memset (the balanced tail's
arrival counters are cleared by the kernels themselves).  The test warms
the runtime with one eager run, captures a block run (and a 3-layer encoder
run) on the runtime's stream through the HIP runtime API, and replays each
graph several times, alternating with the same run issued eagerly on a
second copy of the input and synchronising in between; every replay must
equal the eager result bit for bit.
"""
import ctypes

import numpy as np
import pytest

from conftest import assert_bits_equal
from vestra_hip import da3, seeded

pytestmark = pytest.mark.gpu

_CAPTURE_RELAXED = 2  # hipStreamCaptureModeRelaxed


def _hip():
    h = ctypes.CDLL("libamdhip64.so")
    vp, pvp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
    for name, args in (("hipStreamBeginCapture", [vp, ctypes.c_int]),
                       ("hipStreamEndCapture", [vp, pvp]),
                       ("hipGraphInstantiate", [pvp, vp, pvp, ctypes.c_char_p, ctypes.c_size_t]),
                       ("hipGraphLaunch", [vp, vp]),
                       ("hipStreamSynchronize", [vp]),
                       ("hipGraphExecDestroy", [vp]),
                       ("hipGraphDestroy", [vp])):
        getattr(h, name).argtypes = args
        getattr(h, name).restype = ctypes.c_int
    return h


def _capture(hip, stream, run):
    """The kernels `run` issues on `stream`, as an instantiated graph."""
    assert hip.hipStreamBeginCapture(stream, _CAPTURE_RELAXED) == 0
    try:
        run()
    finally:
        graph = ctypes.c_void_p()
        rc = hip.hipStreamEndCapture(stream, ctypes.byref(graph))
    assert rc == 0 and graph.value
    exe = ctypes.c_void_p()
    assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
    return graph, exe


@pytest.mark.parametrize("layers, q8", [(1, False), (3, False), (2, True)],
                         ids=["block", "encoder3", "q8_encoder2"])
def test_encoder_graph_replays_equal_eager(rt, layers, q8):
    hip = _hip()
    stream = ctypes.c_void_p(rt.stream())
    blocks = [rt.prepare_block(da3.block_weights(seed=90 + i, layerscale="uniform"), q8_0=q8)
              for i in range(layers)]
    pos = da3.positions_yx(24, 36)
    x0 = seeded.normal(9000 + layers, 865 * 768)
    x, y = rt.upload_f32(x0), rt.upload_f32(x0)

    def run(t):
        if layers == 1:
            rt.vit_block_run(blocks[0], t, 1, 865, pos)
        else:
            rt.encoder_run(blocks, t, 1, 865, pos)

    run(y)  # warm-up: workspaces and the RoPE table exist before the capture
    rt.synchronize()
    x_ref = rt.download_f32(y)
    y = rt.upload_f32(x0)
    rt.synchronize()
    graph, exe = _capture(hip, stream, lambda: run(x))
    try:
        # The capture recorded the kernels without running them.
        assert np.array_equal(rt.download_f32(x), x0)
        for replay in range(3):
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            run(y)  # the same run, eagerly, between the replays
            rt.synchronize()
            got, exp = rt.download_f32(x), rt.download_f32(y)
            assert_bits_equal(got, exp, f"replay {replay}")
            if replay == 0:
                assert_bits_equal(got, x_ref, "first replay against the warm-up run")
    finally:
        hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)
