"""The allocation-free decode attention (asmhip_attention_decode_rope_noalloc) against
the entry point it mirrors (asmhip_attention_decode_rope with a caller workspace):
outputs and cache writes equal bit for bit, on two calls in a row (the second smaller,
so stale scratch contents from the first would show), and oversized shapes refused."""

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
