"""The allocation-free verify attention (nmi_gqa_attention_noalloc) against the workspace form
(nmi_gqa_attention), both through the C ABI: same kernels and plan, so outputs and cache bytes must
be bit-identical, on consecutive calls sharing the device's static scratch (the second call smaller
than the first, then a batch), and within the usual 2e-3 of the FP64 oracle. A plan needing more
than the static scratch is rejected on the host before any launch.
"""
import numpy as np
import pytest

import ninfer_amd as na
from ninfer_amd import ops
from ninfer_amd.device import DeviceArray, DeviceBuffer, synchronize
from ninfer_amd.kv_cache import KVCacheLayer
from helpers import AttnCase, rel_l2
import gpu_runner

pytestmark = pytest.mark.gpu


def _run(case, noalloc):
    D, Hq, Hkv, T, B = case.D, case.Hq, case.Hkv, case.T, case.B
    cache = gpu_runner.upload_cache(case)
    q = DeviceArray.from_numpy(na.BF16, case.q, (D, Hq, T, B))
    k = DeviceArray.from_numpy(na.BF16, case.k_new, (D, Hkv, T, B))
    v = DeviceArray.from_numpy(na.BF16, case.v_new, (D, Hkv, T, B))
    pos = DeviceArray.from_numpy(na.I32, case.positions, (T, B))
    out = DeviceArray(na.BF16, (D, Hq, T, B))
    out.buf.fill(0xFF)
    env = (1, case.max_context)
    if noalloc:
        ops.gqa_attention_noalloc(q.tensor(), k.tensor(), v.tensor(), pos.tensor(), case.scale, cache.view(), env,
                                  out.tensor())
    else:
        ws = DeviceBuffer(ops.gqa_attention_workspace_bytes(Hq, Hkv, D, T, B, env[1]))
        ws.fill(0xFF)
        ops.gqa_attention(q.tensor(), k.tensor(), v.tensor(), pos.tensor(), case.scale, cache.view(), env, ws,
                          out.tensor())
    synchronize()
    return out.numpy(), cache.download()


@pytest.mark.parametrize("calls", [[([7680], 4, 1), ([1000], 3, 2), ([3000, 17, 900, 5000], 4, 3)]])
def test_noalloc_matches_workspace_form(gpu, calls):
    for Ls, T, seed in calls:
        print(f"case noalloc Ls={Ls} T={T}", flush=True)
        case = AttnCase(Ls, T=T, seed=500 + seed)
        want_out, want_cache = _run(case, noalloc=False)
        got_out, got_cache = _run(case, noalloc=True)
        assert np.array_equal(got_out, want_out), "noalloc output differs from the workspace form"
        for g, w in zip(got_cache, want_cache):
            assert np.array_equal(g, w), "noalloc cache bytes differ from the workspace form"
        _, ref = case.oracle_after_append()
        got = (got_out.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        assert rel_l2(got, ref) <= 2e-3


def test_noalloc_rejects_plans_beyond_the_static_scratch(gpu):
    """200 sequences need 200 partial slots per KV head (about 26 MB): more than the 16 MiB scratch."""
    B, T, D, Hq, Hkv = 200, 4, 128, 40, 8
    assert ops.gqa_attention_workspace_bytes(Hq, Hkv, D, T, B, 128) > 16 << 20
    cache = KVCacheLayer(128, Hkv, D, B)
    q = DeviceArray(na.BF16, (D, Hq, T, B))
    k = DeviceArray(na.BF16, (D, Hkv, T, B))
    v = DeviceArray(na.BF16, (D, Hkv, T, B))
    pos = DeviceArray.from_numpy(na.I32, np.tile(np.arange(4, dtype=np.int32), B), (T, B))
    out = DeviceArray(na.BF16, (D, Hq, T, B))
    with pytest.raises(NotImplementedError, match="static scratch"):
        ops.gqa_attention_noalloc(q.tensor(), k.tensor(), v.tensor(), pos.tensor(), float(np.float32(1 / np.sqrt(D))),
                                  cache.view(), (1, 128), out.tensor())
