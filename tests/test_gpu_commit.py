"""GPU parity of the KV commit side: INT8 quantize-and-commit of an accepted prefix (no byte of a
rejected column written), explicit rollback, and tree-path compaction — all byte-exact against the
oracle (reference contract include/ninfer/ops/kv_cache_append_prefix.h:22-32)."""
import numpy as np
import pytest

import ninfer_amd as na
from ninfer_amd import ops
from ninfer_amd import synthetic as syn
from ninfer_amd.device import DeviceArray, synchronize
from ninfer_amd.kv_cache import KVCacheLayer

pytestmark = pytest.mark.gpu

H, D, MAXC = 8, 128, 1000


def _random_cache(seed, B=1):
    cache = KVCacheLayer(MAXC, H, D, B)
    P = cache.padded_context
    rng = np.random.default_rng(seed)
    planes = (rng.integers(-127, 128, (B, H, P, D)).astype(np.int8),
              rng.integers(-127, 128, (B, H, P, D)).astype(np.int8),
              rng.integers(0, 0x7BFF, (B, H, P, 2)).astype(np.uint16),
              rng.integers(0, 0x7BFF, (B, H, P, 2)).astype(np.uint16))
    cache.upload(*planes)
    return cache, [p.copy() for p in planes]


@pytest.mark.parametrize("count", [0, 1, 3, 4])
def test_int8_commit_prefix(gpu, oracle, count):
    cache, planes = _random_cache(1)
    T = 4
    k = syn.normal_bf16(5, D * H * T)
    v = syn.normal_bf16(6, D * H * T)
    pos = np.arange(600, 600 + T, dtype=np.int32)
    dk = DeviceArray.from_numpy(na.BF16, k, (D, H, T))
    dv = DeviceArray.from_numpy(na.BF16, v, (D, H, T))
    dp = DeviceArray.from_numpy(na.I32, pos, (T,))
    dc = DeviceArray.from_numpy(na.I32, np.array([count], np.int32), (1,))
    ops.kv_cache_append_prefix(dk.tensor(), dv.tensor(), dp.tensor(), dc.tensor(), (0, T), cache.view())
    synchronize()
    kc, vc, ks, vs = [p[0] for p in planes]
    oracle.kv_commit_prefix(k, v, pos, T, count, H, D, cache.padded_context, kc, vc, ks, vs)
    got = cache.download()
    for g, e in zip(got, (kc, vc, ks, vs)):
        assert np.array_equal(g[0], e)


def test_rollback_and_compaction_batch(gpu, oracle):
    B, T = 3, 8
    cache, planes = _random_cache(2, B)
    P = cache.padded_context
    pos = np.concatenate([np.arange(L, L + T, dtype=np.int32) for L in (100, 400, 900 - T)])
    keep = np.array([2, 8, 0], np.int32)
    dp = DeviceArray.from_numpy(na.I32, pos, (T, B))
    dk = DeviceArray.from_numpy(na.I32, keep, (B,))
    ops.kv_cache_rollback(dp.tensor(), dk.tensor(), cache.view())
    synchronize()
    exp = [[p[b].copy() for p in planes] for b in range(B)]
    for b in range(B):
        oracle.kv_rollback(pos[b * T:(b + 1) * T], T, int(keep[b]), H, D, P, *exp[b])
    got = cache.download()
    for b in range(B):
        for g, e in zip(got, exp[b]):
            assert np.array_equal(g[b], e), f"rollback b={b}"

    bases = np.array([100, 400, 892], np.int32)
    paths = np.array([[0, 1, 3, 7, 0, 0, 0, 0], [0, 2, 5, 6, 7, 0, 0, 0], [0, 0, 0, 0, 0, 0, 0, 0]], np.int32)
    lens = np.array([4, 5, 1], np.int32)
    db = DeviceArray.from_numpy(na.I32, bases, (B,))
    dpath = DeviceArray.from_numpy(na.I32, paths, (T, B))
    dl = DeviceArray.from_numpy(na.I32, lens, (B,))
    ops.kv_cache_compact_path(db.tensor(), dpath.tensor(), dl.tensor(), cache.view())
    synchronize()
    for b in range(B):
        oracle.kv_compact_path(int(bases[b]), paths[b], int(lens[b]), H, D, P, *exp[b])
    got = cache.download()
    for b in range(B):
        for g, e in zip(got, exp[b]):
            assert np.array_equal(g[b], e), f"compaction b={b}"


def test_bf16_commit_prefix_is_bit_copy(gpu):
    T, P = 4, 1024
    k = syn.normal_bf16(7, D * H * T)
    v = syn.normal_bf16(8, D * H * T)
    ck = DeviceArray.from_numpy(na.BF16, np.full((H, P, D), 0x1234, np.uint16), (D, P, H))
    cv = DeviceArray.from_numpy(na.BF16, np.full((H, P, D), 0x4321, np.uint16), (D, P, H))
    view = na.KVLayerView()
    view.k, view.v = ck.tensor(), cv.tensor()
    view.k_scale = na.Tensor.make(0, na.FP16, (1,))
    view.v_scale = na.Tensor.make(0, na.FP16, (1,))
    view.max_context, view.padded_context, view.num_kv_heads, view.head_dim = 1000, P, H, D
    view.dtype, view.quant_group = na.BF16, 0
    dk = DeviceArray.from_numpy(na.BF16, k, (D, H, T))
    dv = DeviceArray.from_numpy(na.BF16, v, (D, H, T))
    dp = DeviceArray.from_numpy(na.I32, np.arange(10, 14, dtype=np.int32), (T,))
    dc = DeviceArray.from_numpy(na.I32, np.array([2], np.int32), (1,))
    ops.kv_cache_append_prefix(dk.tensor(), dv.tensor(), dp.tensor(), dc.tensor(), (0, T), view)
    synchronize()
    gk = ck.numpy().reshape(H, P, D)
    kk = k.reshape(T, H, D)
    for t in range(T):
        for h in range(H):
            if t < 2:
                assert np.array_equal(gk[h, 10 + t], kk[t, h])
            else:
                assert (gk[h, 10 + t] == 0x1234).all()
    assert (np.delete(gk, [10, 11], axis=1) == 0x1234).all()


def test_codec_tie_fixture_on_gpu(gpu):
    """The generated tie group encodes with the header's reciprocal form on the device too."""
    import json
    from pathlib import Path
    fx = json.loads((Path(__file__).parent / "golden" / "codec_tie.json").read_text())
    grp = np.array(fx["group_bf16"], np.uint16)
    k = np.tile(grp, H * 2)  # [D=128, H, T=1]: both 64-groups of every head
    cache = KVCacheLayer(MAXC, H, D)
    dk = DeviceArray.from_numpy(na.BF16, k, (D, H, 1))
    dp = DeviceArray.from_numpy(na.I32, np.array([5], np.int32), (1,))
    ops.gqa_kv_append(dk.tensor(), dk.tensor(), dp.tensor(), cache.view())
    synchronize()
    kc, _, ks, _ = cache.download()
    assert kc[0, 0, 5, fx["element"]] == fx["code_header_form"]
    assert ks[0, 0, 5, 0] == fx["scale_bits"]
