"""The allocation-free decode attention (asmhip_attention_decode_rope_noalloc) against
the entry point it mirrors (asmhip_attention_decode_rope with a caller workspace):
outputs and cache writes equal bit for bit, on two calls in a row (the second smaller,
so stale scratch contents from the first would show), and oversized shapes refused."""

import ctypes

import numpy as np
import pytest

from asmllm_amd import native
from asmllm_amd.device import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu


def _inputs(n_heads, n_kv, hd, pos, max_ctx, seed):
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal((n_heads + 2 * n_kv) * hd).astype(np.float32)
    kc = np.zeros((n_kv, max_ctx, hd), np.float16)
    vc = np.zeros((n_kv, max_ctx, hd), np.float16)
    kc[:, :pos] = rng.standard_normal((n_kv, pos, hd))
    vc[:, :pos] = rng.standard_normal((n_kv, pos, hd))
    return qkv, kc, vc


def _run(hip, noalloc, n_heads, n_kv, hd, pos, max_ctx, seed):
    qkv, kc, vc = _inputs(n_heads, n_kv, hd, pos, max_ctx, seed)
    dqkv, dkc, dvc = DeviceBuffer.from_numpy(qkv), DeviceBuffer.from_numpy(kc), DeviceBuffer.from_numpy(vc)
    dpos = DeviceBuffer.from_numpy(np.array([pos], np.int32))
    dout = DeviceBuffer.from_numpy(np.full(n_heads * hd, np.nan, np.float32))
    if noalloc:
        rc = hip.asmhip_attention_decode_rope_noalloc(dqkv.ptr, dkc.ptr, dvc.ptr, dout.ptr, n_heads, n_kv, hd,
                                                      dpos.ptr, max_ctx, 10000.0, None)
    else:
        dws = DeviceBuffer(hip.asmhip_attention_decode_workspace(n_heads, hd, max_ctx) * 4)
        rc = hip.asmhip_attention_decode_rope(dqkv.ptr, dkc.ptr, dvc.ptr, dws.ptr, dout.ptr, n_heads, n_kv, hd,
                                              dpos.ptr, max_ctx, 10000.0, None)
    assert rc == 0, hip.asmhip_last_error()
    synchronize()
    return (dout.download(np.float32, n_heads * hd), dkc.download(np.float16, kc.shape),
            dvc.download(np.float16, vc.shape))


CASES = [(32, 32, 128, 2048, 2176), (8, 2, 64, 129, 300)]  # the 7B step, then a smaller one


def test_noalloc_matches_workspace_entry_point_twice(hip):
    for i, (n_heads, n_kv, hd, pos, max_ctx) in enumerate(CASES):
        ref = _run(hip, False, n_heads, n_kv, hd, pos, max_ctx, seed=100 + i)
        got = _run(hip, True, n_heads, n_kv, hd, pos, max_ctx, seed=100 + i)
        for a, b in zip(got, ref):
            np.testing.assert_array_equal(a.view(np.uint16 if a.dtype == np.float16 else np.uint32),
                                          b.view(np.uint16 if b.dtype == np.float16 else np.uint32))
        assert np.all(np.isfinite(got[0]))


def test_noalloc_rejects_shapes_beyond_its_scratch(hip):
    cap = hip.asmhip_attention_decode_noalloc_max_floats()
    assert cap == 1 << 20
    # 512 heads x 16 splits x 132 floats > 2^20
    assert hip.asmhip_attention_decode_rope_noalloc(1, 1, 1, 1, 512, 512, 128, 1, 8192, 10000.0, None) == \
        native.ERR_INVALID_ARGUMENT
    assert "scratch" in hip.asmhip_last_error().decode()


def test_noalloc_captured_graph_replays_match_eager(hip):
    """The entry point inside a HIP graph (its advertised use): one eager call first
    (the first call on a device looks up the scratch address), then the same call
    captured and replayed three times with other work on the GPU between replays;
    every replay bit for bit equal to the eager result."""
    n_heads, n_kv, hd, pos, max_ctx = CASES[1]
    want = _run(hip, True, n_heads, n_kv, hd, pos, max_ctx, seed=7)  # eager, also the first call
    qkv, kc, vc = _inputs(n_heads, n_kv, hd, pos, max_ctx, seed=7)
    dqkv, dkc, dvc = DeviceBuffer.from_numpy(qkv), DeviceBuffer.from_numpy(kc), DeviceBuffer.from_numpy(vc)
    dpos = DeviceBuffer.from_numpy(np.array([pos], np.int32))
    dout = DeviceBuffer(n_heads * hd * 4)
    st = hip.asmhip_stream_create()
    assert hip.asmhip_stream_begin_capture(st) == 0, hip.asmhip_last_error()
    rc = hip.asmhip_attention_decode_rope_noalloc(dqkv.ptr, dkc.ptr, dvc.ptr, dout.ptr, n_heads, n_kv, hd,
                                                  dpos.ptr, max_ctx, 10000.0, st)
    graph = ctypes.c_void_p()
    assert hip.asmhip_stream_end_capture(st, ctypes.byref(graph)) == 0, hip.asmhip_last_error()
    assert rc == 0, hip.asmhip_last_error()
    for r in range(3):
        dout.upload(np.full(n_heads * hd, np.nan, np.float32))
        assert hip.asmhip_graph_launch(graph, st) == 0, hip.asmhip_last_error()
        assert hip.asmhip_stream_synchronize(st) == 0
        got = (dout.download(np.float32, n_heads * hd), dkc.download(np.float16, kc.shape),
               dvc.download(np.float16, vc.shape))
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a.view(np.uint16 if a.dtype == np.float16 else np.uint32),
                                          b.view(np.uint16 if b.dtype == np.float16 else np.uint32))
        _run(hip, False, *CASES[0], seed=200 + r)  # other work between the replays
    hip.asmhip_graph_destroy(graph)
    hip.asmhip_stream_destroy(st)


_FIRST_CALL_IN_CAPTURE = """
import ctypes, sys
sys.path.insert(0, {root!r})
from asmllm_amd import native
from asmllm_amd.device import DeviceBuffer
hip = native.lib()
import numpy as np
bufs = [DeviceBuffer.from_numpy(np.zeros(1 << 18, np.float32)) for _ in range(5)]  # position 0, zero data
st = hip.asmhip_stream_create()
assert hip.asmhip_stream_begin_capture(st) == 0
rc = hip.asmhip_attention_decode_rope_noalloc(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, 8, 2, 64,
                                              bufs[4].ptr, 300, 10000.0, st)
g = ctypes.c_void_p()
hip.asmhip_stream_end_capture(st, ctypes.byref(g))
if g.value:
    hip.asmhip_graph_destroy(g)
print(rc, hip.asmhip_last_error().decode())
"""


def test_noalloc_first_call_inside_capture_is_refused():
    """In a fresh process, a first call made inside stream capture returns
    ASMHIP_ERR_INVALID_ARGUMENT with a message instead of looking the scratch
    address up mid-capture."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    out = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE.format(root=root)], capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    rc, msg = out.stdout.strip().split(" ", 1)
    assert int(rc) == native.ERR_INVALID_ARGUMENT
    assert "outside stream capture" in msg
