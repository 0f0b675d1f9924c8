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


ROUNDS = 4


def _elem(arr, i):
    return DeviceArray(na.I32, (1,), buf=arr.buf, offset=arr.offset + 4 * i)


@pytest.mark.parametrize("Ls,T,Hq,Hkv,D", [([3000], 4, 40, 8, 128), ([2500], 16, 40, 8, 128), ([1800], 4, 24, 4, 256)],
                         ids=["A1-40-8", "80row-T16", "D256-24-4"])
def test_noalloc_under_capture(gpu, oracle, Ls, T, Hq, Hkv, D):
    """The allocation-free entry is for callers under graph capture. The first test of this file, so
    the process's first nmi_gqa_attention_noalloc call (which resolves the device's scratch address)
    runs inside an active capture. The captured round (positions from the device-side length, then
    the attention into the static scratch) is replayed over several rounds with the length advanced
    on the device, against eager workspace-form calls on a twin state (bit-exact) and the oracle."""
    from ninfer_amd import synthetic as syn
    from ninfer_amd.device import Graph, Stream
    print(f"case noalloc capture Ls={Ls} T={T} {Hq}|{Hkv} D={D}", flush=True)
    B, K = len(Ls), T - 1
    base = AttnCase(Ls, T=T, Hq=Hq, Hkv=Hkv, D=D, seed=700 + T + D, max_context=max(Ls) + ROUNDS * T + T)
    P = base.P
    stream = Stream()
    states = []
    for _ in range(2):  # [graph with the no-alloc entry, eager workspace form]
        st = dict(cache=gpu_runner.upload_cache(base),
                  token=DeviceArray.from_numpy(na.I32, np.arange(B, dtype=np.int32) + 7, (B,)),
                  drafts=DeviceArray.from_numpy(na.I32, np.arange(B * K, dtype=np.int32) + 100, (K, B)),
                  length=DeviceArray.from_numpy(na.I32, np.array(Ls, np.int32), (B,)),
                  ids=DeviceArray(na.I32, (T, B)), pos=DeviceArray(na.I32, (T, B)),
                  q=DeviceArray(na.BF16, (D, Hq, T, B)), k=DeviceArray(na.BF16, (D, Hkv, T, B)),
                  v=DeviceArray(na.BF16, (D, Hkv, T, B)), out=DeviceArray(na.BF16, (D, Hq, T, B)),
                  ws=DeviceBuffer(ops.gqa_attention_workspace_bytes(Hq, Hkv, D, T, B, base.max_context)))
        st["ws"].fill(0xFF)
        states.append(st)
    env = (1, base.max_context)

    def round_ops(st, noalloc):
        ops.speculative_prepare_verify_inputs(st["token"].tensor(), st["drafts"].tensor(), st["length"].tensor(),
                                              st["ids"].tensor(), st["pos"].tensor(), stream)
        if noalloc:
            ops.gqa_attention_noalloc(st["q"].tensor(), st["k"].tensor(), st["v"].tensor(), st["pos"].tensor(),
                                      base.scale, st["cache"].view(), env, st["out"].tensor(), stream)
        else:
            ops.gqa_attention(st["q"].tensor(), st["k"].tensor(), st["v"].tensor(), st["pos"].tensor(), base.scale,
                              st["cache"].view(), env, st["ws"], st["out"].tensor(), stream)

    graph = Graph(stream)
    with graph:
        round_ops(states[0], True)
    kc, vc, ks, vs = (a.copy() for a in base.cache_planes())
    lengths = np.array(Ls, np.int64)
    rng = np.random.default_rng(41 + T)
    for r in range(ROUNDS):
        q = syn.normal_bf16(syn.derive_seed(9, r, 1, D), D * Hq * T * B)
        k = syn.normal_bf16(syn.derive_seed(9, r, 2, D), D * Hkv * T * B)
        v = syn.normal_bf16(syn.derive_seed(9, r, 3, D), D * Hkv * T * B)
        for st in states:
            st["q"].upload(q)
            st["k"].upload(k)
            st["v"].upload(v)
        graph.launch()
        round_ops(states[1], False)
        stream.synchronize()
        pos = (lengths[:, None] + np.arange(T)[None, :]).astype(np.int32).reshape(-1)
        oracle.kv_append(k, v, pos, T, B, Hkv, D, P, kc, vc, ks, vs)
        ref = oracle.attention(q, kc, vc, ks, vs, pos, None, T, B, Hq, Hkv, D, P, base.scale)
        g_out, e_out = states[0]["out"].numpy(), states[1]["out"].numpy()
        assert np.array_equal(states[0]["pos"].numpy(), pos), "device positions differ"
        assert np.array_equal(g_out, e_out), "replayed no-alloc round differs from the workspace form"
        for got_g, got_e, want in zip(states[0]["cache"].download(), states[1]["cache"].download(), (kc, vc, ks, vs)):
            assert np.array_equal(got_g, got_e) and np.array_equal(got_g, want), "cache bytes differ"
        got = (g_out.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        assert rel_l2(got, ref) <= 2e-3
        produced = rng.integers(1, T + 1, size=B)
        for st in states:
            for b, a in enumerate(produced):
                for _ in range(int(a)):
                    ops.increment_i32_scalar(_elem(st["length"], b).tensor(), stream)
        lengths += produced


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


@pytest.mark.parametrize("calls", [[([7680], 4, 1), ([1000], 3, 2), ([3000, 17, 900, 5000], 4, 3),
                                    ([1200], 70, 4), ([300], 4, 5)]])
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
    """320 sequences need 320 partial slots per KV head (about 22 MB): more than the 16 MiB scratch."""
    B, T, D, Hq, Hkv = 320, 4, 128, 40, 8
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
