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


# ---- the reference's kv_cache_append_prefix matrix (tests/ops/test_kv_cache_append_prefix.cpp) ----

RD, RH, LIN_CAP, LIN_PADDED, WINDOW = 128, 8, 64, 72, 4096


def _patterned(count, seed):
    """The reference test's LCG bit pattern (test_kv_cache_append_prefix.cpp:38-46)."""
    out = np.empty(count, np.uint16)
    state = seed & 0xFFFFFFFF
    # vectorized in blocks: state_{n+1} = a * state_n + c (mod 2^32)
    a, c = 1664525, 1013904223
    for i in range(count):
        state = (state * a + c) & 0xFFFFFFFF
        out[i] = state >> 16
    return out


_PATTERN_CACHE = {}


def _pattern(count, seed):
    key = (count, seed)
    if key not in _PATTERN_CACHE:
        _PATTERN_CACHE[key] = _patterned(count, seed)
    return _PATTERN_CACHE[key]


def _bf16_views(padded, cyclic):
    ck = DeviceArray(na.BF16, (RD, padded, RH))
    cv = DeviceArray(na.BF16, (RD, padded, RH))
    view = na.CyclicKVLayerView() if cyclic else na.KVLayerView()
    view.k, view.v = ck.tensor(), cv.tensor()
    view.k_scale = na.Tensor.make(0, na.FP16, (1,))
    view.v_scale = na.Tensor.make(0, na.FP16, (1,))
    if cyclic:
        view.capacity, view.padded_capacity = WINDOW, padded
    else:
        view.max_context, view.padded_context = LIN_CAP, padded
    view.num_kv_heads, view.head_dim, view.dtype, view.quant_group = RH, RD, na.BF16, 0
    return ck, cv, view


def _apply(exp_k, exp_v, k, v, count, position0, padded, cyclic):
    """apply_oracle of the reference test: token i lands in slot (position0 + i) [mod 4096]."""
    ek = exp_k.reshape(RH, padded, RD)
    ev = exp_v.reshape(RH, padded, RD)
    kk = k.reshape(-1, RH, RD)
    vv = v.reshape(-1, RH, RD)
    for t in range(count):
        slot = (position0 + t) & (WINDOW - 1) if cyclic else position0 + t
        ek[:, slot] = kk[t]
        ev[:, slot] = vv[t]


def _append(views, k, v, pos, count, envelope, cyclic, stream=None):
    T = len(pos)
    dk = DeviceArray.from_numpy(na.BF16, k, (RD, RH, T))
    dv = DeviceArray.from_numpy(na.BF16, v, (RD, RH, T))
    dp = DeviceArray.from_numpy(na.I32, np.asarray(pos, np.int32), (T,))
    dc = DeviceArray.from_numpy(na.I32, np.array([count], np.int32), (1,))
    fn = ops.kv_cache_append_prefix_cyclic if cyclic else ops.kv_cache_append_prefix
    fn(dk.tensor(), dv.tensor(), dp.tensor(), dc.tensor(), envelope, views[2], stream)
    synchronize()
    assert np.array_equal(dk.numpy(), k) and np.array_equal(dv.numpy(), v), "inputs changed"
    assert np.array_equal(dp.numpy(), pos) and dc.numpy()[0] == count, "inputs changed"


@pytest.mark.parametrize("cyclic", [False, True], ids=["linear", "cyclic"])
def test_reference_append_prefix_matrix(gpu, cyclic):
    """Every T in 1..16 and count in 0..T at the reference's positions (17 linear; 2*4096-2 cyclic,
    which wraps), cache seeded with patterned bits: exactly the accepted rows change, bit for bit."""
    padded = WINDOW if cyclic else LIN_PADDED
    position = 2 * WINDOW - 2 if cyclic else 17
    n_cache = RD * padded * RH
    seeded_k, seeded_v = _pattern(n_cache, 0x90a0b0c0), _pattern(n_cache, 0xd0e0f001)
    views = _bf16_views(padded, cyclic)
    print(f"case append prefix matrix cyclic={cyclic}", flush=True)
    for T in range(1, 17):
        for count in range(T + 1):
            k = _pattern(RD * RH * T, 0x10203040 + T)
            v = _pattern(RD * RH * T, 0x50607080 + count)
            views[0].upload(seeded_k)
            views[1].upload(seeded_v)
            _append(views, k, v, np.arange(position, position + T, dtype=np.int32), count, (0, T), cyclic)
            ek, ev = seeded_k.copy(), seeded_v.copy()
            _apply(ek, ev, k, v, count, position, padded, cyclic)
            assert np.array_equal(views[0].numpy(), ek), (T, count)
            assert np.array_equal(views[1].numpy(), ev), (T, count)


@pytest.mark.parametrize("cyclic,count,env_min", [(False, 17, 0), (True, 4, 5), (True, 17, 0), (False, -1, 0)])
def test_reference_append_prefix_outside_envelope_writes_nothing(gpu, cyclic, count, env_min):
    """A device count above T (17 > 16) or below the envelope's minimum writes no byte
    (test_kv_cache_append_prefix.cpp:292-294)."""
    T = 16
    padded = WINDOW if cyclic else LIN_PADDED
    position = 2 * WINDOW - 2 if cyclic else 17
    n_cache = RD * padded * RH
    seeded_k, seeded_v = _pattern(n_cache, 0x90a0b0c0), _pattern(n_cache, 0xd0e0f001)
    views = _bf16_views(padded, cyclic)
    views[0].upload(seeded_k)
    views[1].upload(seeded_v)
    k, v = _pattern(RD * RH * T, 0x10203040 + T), _pattern(RD * RH * T, 0x50607080 + 16)
    _append(views, k, v, np.arange(position, position + T, dtype=np.int32), count, (env_min, T), cyclic)
    assert np.array_equal(views[0].numpy(), seeded_k) and np.array_equal(views[1].numpy(), seeded_v)


def test_reference_cyclic_graph_and_resume(gpu):
    """graph_and_resume_case (test_kv_cache_append_prefix.cpp:171-268): one captured cyclic commit at
    position 3*4096-3 replayed for every committed count 0..16 (set on the device), each followed by
    an eager two-token resume at position + committed."""
    from ninfer_amd.device import Graph, Stream
    T, R, position = 16, 2, 3 * WINDOW - 3
    n_cache = RD * WINDOW * RH
    first_k, first_v = _pattern(RD * RH * T, 0x11112222), _pattern(RD * RH * T, 0x33334444)
    next_k, next_v = _pattern(RD * RH * R, 0x55556666), _pattern(RD * RH * R, 0x77778888)
    seeded_k, seeded_v = _pattern(n_cache, 0x9999aaaa), _pattern(n_cache, 0xbbbbcccc)
    views = _bf16_views(WINDOW, True)
    dk = DeviceArray.from_numpy(na.BF16, first_k, (RD, RH, T))
    dv = DeviceArray.from_numpy(na.BF16, first_v, (RD, RH, T))
    dp = DeviceArray.from_numpy(na.I32, np.arange(position, position + T, dtype=np.int32), (T,))
    dc = DeviceArray.from_numpy(na.I32, np.zeros(1, np.int32), (1,))
    stream = Stream()
    graph = Graph(stream)
    with graph:
        ops.kv_cache_append_prefix_cyclic(dk.tensor(), dv.tensor(), dp.tensor(), dc.tensor(), (0, T), views[2],
                                          stream)
    for committed in range(T + 1):
        views[0].upload(seeded_k)
        views[1].upload(seeded_v)
        ops.set_i32_scalar(dc.tensor(), committed, stream)
        graph.launch()
        stream.synchronize()
        ek, ev = seeded_k.copy(), seeded_v.copy()
        _apply(ek, ev, first_k, first_v, committed, position, WINDOW, True)
        assert np.array_equal(views[0].numpy(), ek) and np.array_equal(views[1].numpy(), ev), committed
        _append(views, next_k, next_v, np.arange(position + committed, position + committed + R, dtype=np.int32), R,
                (R, R), True)
        _apply(ek, ev, next_k, next_v, R, position + committed, WINDOW, True)
        assert np.array_equal(views[0].numpy(), ek) and np.array_equal(views[1].numpy(), ev), committed


def test_int8_cyclic_commit_prefix(gpu, oracle):
    """INT8-G64 ring (extension): the accepted columns are quantized into rows position % capacity,
    bytes equal to the oracle's commit at the wrapped rows."""
    cap, T, count, position = 256, 6, 5, 2 * 256 - 3
    cache = KVCacheLayer(cap, H, D)
    P = cache.padded_context
    rng = np.random.default_rng(4)
    planes = (rng.integers(-127, 128, (1, H, P, D)).astype(np.int8),
              rng.integers(-127, 128, (1, H, P, D)).astype(np.int8),
              rng.integers(0, 0x7BFF, (1, H, P, 2)).astype(np.uint16),
              rng.integers(0, 0x7BFF, (1, H, P, 2)).astype(np.uint16))
    cache.upload(*planes)
    view = na.CyclicKVLayerView()
    lin = cache.view()
    view.k, view.v, view.k_scale, view.v_scale = lin.k, lin.v, lin.k_scale, lin.v_scale
    view.capacity, view.padded_capacity = cap, P
    view.num_kv_heads, view.head_dim, view.dtype, view.quant_group = H, D, na.I8, 64
    k = syn.normal_bf16(15, D * H * T)
    v = syn.normal_bf16(16, D * H * T)
    pos = np.arange(position, position + T, dtype=np.int32)
    dk = DeviceArray.from_numpy(na.BF16, k, (D, H, T))
    dv = DeviceArray.from_numpy(na.BF16, v, (D, H, T))
    dp = DeviceArray.from_numpy(na.I32, pos, (T,))
    dc = DeviceArray.from_numpy(na.I32, np.array([count], np.int32), (1,))
    ops.kv_cache_append_prefix_cyclic(dk.tensor(), dv.tensor(), dp.tensor(), dc.tensor(), (0, T), view)
    synchronize()
    kc, vc, ks, vs = [p[0].copy() for p in planes]
    oracle.kv_commit_prefix(k, v, pos % cap, T, count, H, D, P, kc, vc, ks, vs)
    for g, e in zip(cache.download(), (kc, vc, ks, vs)):
        assert np.array_equal(g[0], e)
