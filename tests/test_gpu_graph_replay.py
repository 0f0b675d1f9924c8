"""Graph replay: each op captured once in a HIP graph and replayed over several rounds, with the
device-resident state (length, positions, token, stats, token counts, commit counts, recurrent-state
slots) advanced on the device between replays, as a serving loop replays a captured round. Every
replay is compared with the same sequence of eager calls on a twin state (bit-exact: same kernels,
same inputs) and with the oracle run round by round.

Mirrors the reference's graph-relaunch case (tests/ops/test_gqa_attention.cpp:1309) and its
replayable-op contract (docs/maintainer/op-development.md:106-123: device scalars, no host reads, a
workspace the op resets itself). No op records a memset: counters are cleared by kernels.
"""
import numpy as np
import pytest

import ninfer_amd as na
from ninfer_amd import ops, synthetic as syn
from ninfer_amd.device import DeviceArray, DeviceBuffer, Graph, Stream, synchronize
from helpers import AttnCase, reference_composite_ok, rel_l2
import gpu_runner

pytestmark = pytest.mark.gpu

ROUNDS = 4


def _capture(stream, fn):
    g = Graph(stream)
    with g:
        fn()
    return g


def _elem(arr, i):
    """Element i of a 1-D I32 device array as a one-element tensor view."""
    return DeviceArray(na.I32, (1,), buf=arr.buf, offset=arr.offset + 4 * i)


def _advance(lengths, amounts, stream):
    """length[b] += amounts[b] on the device (one-thread increments on the stream)."""
    for b, a in enumerate(amounts):
        e = _elem(lengths, b)
        for _ in range(int(a)):
            ops.increment_i32_scalar(e.tensor(), stream)


def _f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


# ---- A1: prepare (positions = length + i on the device) + attention ----------------------------

@pytest.mark.parametrize("Ls", [[3000], [1024 + 397 * b for b in range(16)]], ids=["B1", "B16"])
def test_a1_round_graph_replay(gpu, oracle, Ls):
    B, T, K, Hq, Hkv, D = len(Ls), 4, 3, 40, 8, 128
    base = AttnCase(Ls, T=T, seed=900 + B, max_context=max(Ls) + ROUNDS * T + T)
    P = base.P
    stream = Stream()
    states = []
    for _ in range(2):  # [graph, eager]
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

    def round_ops(st):
        ops.speculative_prepare_verify_inputs(st["token"].tensor(), st["drafts"].tensor(), st["length"].tensor(),
                                              st["ids"].tensor(), st["pos"].tensor(), stream)
        ops.gqa_attention(st["q"].tensor(), st["k"].tensor(), st["v"].tensor(), st["pos"].tensor(), base.scale,
                          st["cache"].view(), env, st["ws"], st["out"].tensor(), stream)

    graph = _capture(stream, lambda: round_ops(states[0]))
    kc, vc, ks, vs = (a.copy() for a in base.cache_planes())
    lengths = np.array(Ls, np.int64)
    rng = np.random.default_rng(31 + B)
    for r in range(ROUNDS):
        print(f"case A1 graph B={B} round {r}", flush=True)
        q = syn.normal_bf16(syn.derive_seed(7, r, 1, B), D * Hq * T * B)
        k = syn.normal_bf16(syn.derive_seed(7, r, 2, B), D * Hkv * T * B)
        v = syn.normal_bf16(syn.derive_seed(7, r, 3, B), D * Hkv * T * B)
        for st in states:
            st["q"].upload(q)
            st["k"].upload(k)
            st["v"].upload(v)
        graph.launch()
        round_ops(states[1])
        stream.synchronize()
        pos = (lengths[:, None] + np.arange(T)[None, :]).astype(np.int32).reshape(-1)
        oracle.kv_append(k, v, pos, T, B, Hkv, D, P, kc, vc, ks, vs)
        ref = oracle.attention(q, kc, vc, ks, vs, pos, None, T, B, Hq, Hkv, D, P, base.scale)
        g_out, e_out = states[0]["out"].numpy(), states[1]["out"].numpy()
        assert np.array_equal(states[0]["pos"].numpy(), pos), "device positions differ"
        assert np.array_equal(g_out, e_out), "graph replay differs from the eager calls"
        for got_g, got_e, want in zip(states[0]["cache"].download(), states[1]["cache"].download(), (kc, vc, ks, vs)):
            assert np.array_equal(got_g, got_e) and np.array_equal(got_g, want), "cache bytes differ"
        assert rel_l2(_f32(g_out), ref) <= 2e-3
        ok, msg = reference_composite_ok(_f32(g_out), ref)
        assert ok, msg
        # the round produced A + 1 tokens per sequence: advance length on the device
        produced = rng.integers(1, T + 1, size=B)
        for st in states:
            _advance(st["length"], produced, stream)
        lengths += produced


# ---- acceptance: argmax + greedy/Mode R (one config per sequence), and Mode F -------------------

def _cfg(temperature=0.0, top_k=0, top_p=1.0, presence=0.0, frequency=0.0, seed=0):
    c = na.SamplingConfig()
    c.temperature, c.top_k, c.top_p = temperature, top_k, top_p
    c.presence_penalty, c.frequency_penalty, c.seed = presence, frequency, seed
    return c


def _ocfg(c):
    from oracle import pyoracle
    o = pyoracle.SamplingConfig()
    o.temperature, o.top_k, o.top_p, o.min_p = c.temperature, c.top_k, c.top_p, c.min_p
    o.presence_penalty, o.frequency_penalty, o.seed = c.presence_penalty, c.frequency_penalty, c.seed
    return o


def test_accept_graph_replay(gpu, oracle):
    """argmax -> accept in one graph over B = 4 sequences (greedy, top-20 stochastic with and without
    penalties): length, token, stats and token counts advance on the device through the op itself."""
    B, K, rows, domain = 4, 3, 32768, 32000
    cfgs = [_cfg(), _cfg(0.7, top_p=0.95, seed=11), _cfg(1.0, top_k=8, presence=0.5, frequency=0.25, seed=12),
            _cfg(0.9, top_p=0.8, seed=13)]
    counts0 = [np.zeros(domain, np.int32) if b == 2 else None for b in range(B)]
    stream = Stream()
    states = []
    for _ in range(2):
        cfg_buf, keep = gpu_runner.upload_configs(cfgs, [None if c is None else c.copy() for c in counts0])
        st = dict(cfg=cfg_buf, keep=keep,
                  logits=DeviceArray(na.BF16, (rows, K + 1, B)), target=DeviceArray(na.I32, (K + 1, B)),
                  drafts=DeviceArray(na.I32, (K, B)),
                  length=DeviceArray.from_numpy(na.I32, np.array([100, 2000, 50, 7], np.int32), (B,)),
                  token=DeviceArray.from_numpy(na.I32, np.full(B, -1, np.int32), (B,)),
                  so=DeviceArray(na.I32, (K + 1, B)), ns=DeviceArray(na.I32, (B,)), acc=DeviceArray(na.I32, (B,)),
                  stats=DeviceArray.from_numpy(na.I64, np.zeros((B, 4 + K), np.int64), (4 + K, B)),
                  ws=DeviceBuffer(max(256, ops.sampling_workspace_bytes(domain, K + 1, B))))
        st["ws"].fill(0xFF)
        states.append(st)

    def accept_ops(st):
        ops.argmax(st["logits"].tensor(), st["target"].tensor(), domain, stream)
        ops.speculative_accept_greedy_drafts(st["target"].tensor(), st["logits"].tensor(), st["drafts"].tensor(),
                                             st["length"].tensor(), st["token"].tensor(), st["so"].tensor(),
                                             st["ns"].tensor(), st["acc"].tensor(), st["stats"].tensor(), domain,
                                             st["cfg"].ptr, st["ws"], stream)

    graph = _capture(stream, lambda: accept_ops(states[0]))
    L = [100, 2000, 50, 7]
    stats = [np.zeros(4 + K, np.int64) for _ in range(B)]
    counts = [None if c is None else c.copy() for c in counts0]
    for r in range(ROUNDS):
        print(f"case accept graph round {r}", flush=True)
        logits = syn.normal_bf16(syn.derive_seed(8, r), B * (K + 1) * rows, 2.0).reshape(B, K + 1, rows)
        drafts = np.zeros((B, K), np.int32)
        for b in range(B):
            f = syn.bf16_bits_to_f32(logits[b])
            top = np.argsort(-f, axis=1)[:, :3]
            drafts[b] = [int(top[i, (r + b + i) % 3]) for i in range(K)]  # mostly likely tokens
        for st in states:
            st["logits"].upload(logits)
            st["drafts"].upload(drafts)
        graph.launch()
        accept_ops(states[1])
        stream.synchronize()
        names = ("so", "ns", "acc", "token", "length", "stats")
        g = {n: states[0][n].numpy() for n in names}
        e = {n: states[1][n].numpy() for n in names}
        for n in names:
            assert np.array_equal(g[n], e[n]), f"graph replay differs from the eager calls in {n}"
        g_counts = [tc.numpy() for tc in states[0]["keep"]]
        e_counts = [tc.numpy() for tc in states[1]["keep"]]
        assert all(np.array_equal(a, b) for a, b in zip(g_counts, e_counts))
        tgt = [oracle.argmax(logits[b].reshape(-1), rows, K + 1, domain) for b in range(B)]
        assert np.array_equal(states[0]["target"].numpy().reshape(B, K + 1), np.array(tgt))
        for b in range(B):
            exp = oracle.speculative_accept(tgt[b], logits[b].reshape(-1), rows, drafts[b], L[b], stats[b], domain,
                                            _ocfg(cfgs[b]), token_counts=counts[b])
            assert list(g["so"].reshape(B, K + 1)[b]) == list(exp["sampled_out"]), (r, b)
            assert g["length"][b] == exp["length"] and g["token"][b] == exp["token"], (r, b)
            assert list(g["stats"].reshape(B, 4 + K)[b]) == list(exp["stats"]), (r, b)
            L[b], stats[b] = exp["length"], exp["stats"]
            if counts[b] is not None:
                counts[b] = exp["token_counts"]
        assert np.array_equal(g_counts[0], counts[2])


def test_general_accept_graph_replay(gpu, oracle):
    """Mode F over B = 2 sequences at configs[3]'s temperature and top-p, replayed with new logits and
    uniforms each round; the op's own counters are cleared by its kernels on every replay."""
    B, K, rows, domain = 2, 3, 32768, 32768
    stream = Stream()
    cfg = na.GeneralConfig()
    cfg.temperature, cfg.top_p = 0.7, 0.95
    states = []
    for _ in range(2):
        cb = DeviceBuffer(8)
        cb.upload(np.frombuffer(bytes(memoryview(cfg)), dtype=np.uint8))
        st = dict(cfg=cb, t=DeviceArray(na.BF16, (rows, K + 1, B)), d=DeviceArray(na.BF16, (rows, K, B)),
                  drafts=DeviceArray(na.I32, (K, B)), ua=DeviceArray(na.FP32, (K + 1, B)),
                  ur=DeviceArray(na.FP32, (1, B)),
                  length=DeviceArray.from_numpy(na.I32, np.array([300, 40], np.int32), (B,)),
                  token=DeviceArray(na.I32, (B,)), so=DeviceArray(na.I32, (K + 1, B)), ns=DeviceArray(na.I32, (B,)),
                  acc=DeviceArray(na.I32, (B,)),
                  stats=DeviceArray.from_numpy(na.I64, np.zeros((B, 4 + K), np.int64), (4 + K, B)),
                  ws=DeviceBuffer(ops.general_accept_workspace_bytes(domain, K, B)))
        st["ws"].fill(0xFF)
        states.append(st)

    def accept_ops(st):
        ops.speculative_accept_general(st["t"].tensor(), st["d"].tensor(), st["drafts"].tensor(), st["ua"].tensor(),
                                       st["ur"].tensor(), st["length"].tensor(), st["token"].tensor(),
                                       st["so"].tensor(), st["ns"].tensor(), st["acc"].tensor(),
                                       st["stats"].tensor(), domain, st["cfg"].ptr, st["ws"], stream)

    graph = _capture(stream, lambda: accept_ops(states[0]))
    from oracle import pyoracle
    ocfg = pyoracle.GeneralConfig()
    ocfg.temperature, ocfg.top_p = 0.7, 0.95
    L = [300, 40]
    stats = [np.zeros(4 + K, np.int64) for _ in range(B)]
    for r in range(ROUNDS):
        print(f"case mode F graph round {r}", flush=True)
        rng = np.random.default_rng(50 + r)
        t = rng.standard_normal((B, K + 1, rows), dtype=np.float32) * np.float32(np.sqrt(3.0))
        d = 0.9 * t[:, :K] + np.float32(np.sqrt(1 - 0.81)) * rng.standard_normal((B, K, rows), dtype=np.float32) \
            * np.float32(np.sqrt(3.0))
        tb, db = syn.f32_to_bf16_bits(t), syn.f32_to_bf16_bits(d.astype(np.float32))
        drafts = np.argmax(syn.bf16_bits_to_f32(db), axis=2).astype(np.int32)
        ua = rng.random((B, K + 1), dtype=np.float32)
        ur = rng.random(B, dtype=np.float32)
        for st in states:
            st["t"].upload(tb)
            st["d"].upload(db)
            st["drafts"].upload(drafts)
            st["ua"].upload(ua)
            st["ur"].upload(ur)
        graph.launch()
        accept_ops(states[1])
        stream.synchronize()
        names = ("so", "ns", "acc", "token", "length", "stats")
        g = {n: states[0][n].numpy() for n in names}
        for n in names:
            assert np.array_equal(g[n], states[1][n].numpy()), f"graph replay differs from the eager calls in {n}"
        for b in range(B):
            exp = oracle.general_accept(tb[b].reshape(-1), db[b].reshape(-1), rows, drafts[b], L[b], stats[b], domain,
                                        ocfg, ua[b], float(ur[b]))
            assert list(g["so"].reshape(B, K + 1)[b]) == list(exp["sampled_out"]), (r, b)
            assert g["length"][b] == exp["length"] and list(g["stats"].reshape(B, 4 + K)[b]) == list(exp["stats"])
            L[b], stats[b] = exp["length"], exp["stats"]


# ---- commit: prepare + INT8 prefix commit, commit count set on the device -----------------------

def test_prefix_commit_graph_replay(gpu, oracle):
    B, T, K, Hkv, D = 2, 4, 3, 8, 128
    base = AttnCase([500, 1300], T=T, seed=77, max_context=1300 + ROUNDS * T + T)
    P = base.P
    stream = Stream()
    states = []
    for _ in range(2):
        st = dict(cache=gpu_runner.upload_cache(base),
                  token=DeviceArray.from_numpy(na.I32, np.array([1, 2], np.int32), (B,)),
                  drafts=DeviceArray.from_numpy(na.I32, np.arange(B * K, dtype=np.int32), (K, B)),
                  length=DeviceArray.from_numpy(na.I32, np.array([500, 1300], np.int32), (B,)),
                  ids=DeviceArray(na.I32, (T, B)), pos=DeviceArray(na.I32, (T, B)),
                  count=DeviceArray.from_numpy(na.I32, np.zeros(B, np.int32), (B,)),
                  k=DeviceArray(na.BF16, (D, Hkv, T, B)), v=DeviceArray(na.BF16, (D, Hkv, T, B)))
        states.append(st)

    def commit_ops(st):
        ops.speculative_prepare_verify_inputs(st["token"].tensor(), st["drafts"].tensor(), st["length"].tensor(),
                                              st["ids"].tensor(), st["pos"].tensor(), stream)
        ops.kv_cache_append_prefix(st["k"].tensor(), st["v"].tensor(), st["pos"].tensor(), st["count"].tensor(),
                                   (0, T), st["cache"].view(), stream)

    graph = _capture(stream, lambda: commit_ops(states[0]))
    kc, vc, ks, vs = (a.copy() for a in base.cache_planes())
    lengths = [500, 1300]
    for r in range(ROUNDS):
        print(f"case prefix commit graph round {r}", flush=True)
        k = syn.normal_bf16(syn.derive_seed(9, r, 1), D * Hkv * T * B)
        v = syn.normal_bf16(syn.derive_seed(9, r, 2), D * Hkv * T * B)
        counts = [(r + b) % (T + 1) for b in range(B)]  # 0..T columns accepted
        for st in states:
            st["k"].upload(k)
            st["v"].upload(v)
            for b, c in enumerate(counts):
                ops.set_i32_scalar(_elem(st["count"], b).tensor(), c, stream)
        graph.launch()
        commit_ops(states[1])
        stream.synchronize()
        per = D * Hkv * T
        for b in range(B):
            pos = np.arange(lengths[b], lengths[b] + T, dtype=np.int32)
            oracle.kv_commit_prefix(k[b * per:(b + 1) * per], v[b * per:(b + 1) * per], pos, T, counts[b], Hkv, D, P,
                                    kc[b], vc[b], ks[b], vs[b])
        for got_g, got_e, want in zip(states[0]["cache"].download(), states[1]["cache"].download(), (kc, vc, ks, vs)):
            assert np.array_equal(got_g, got_e), "graph replay differs from the eager calls"
            assert np.array_equal(got_g, want), "cache bytes differ from the oracle"
        for st in states:
            _advance(st["length"], counts, stream)
        lengths = [lengths[b] + counts[b] for b in range(B)]


# ---- recurrent state: conv + GDN snapshots, then the accepted slot becomes the next initial slot ---

def test_gdn_snapshot_graph_replay(gpu, oracle):
    S, Hqk, Hv, T, C = 128, 4, 8, 4, 1024
    slots = T
    rng = np.random.default_rng(5)
    ssm0 = rng.uniform(-0.1, 0.1, (slots, Hv, S, S)).astype(np.float32)
    conv0 = syn.f32_to_bf16_bits(rng.uniform(-2, 2, (slots, 3, C)).astype(np.float32))
    w = syn.f32_to_bf16_bits(rng.uniform(-1, 1, (4, C)).astype(np.float32))
    stream = Stream()
    states = []
    for _ in range(2):
        st = dict(ssm=DeviceArray.from_numpy(na.FP32, ssm0, (S, S, Hv, slots)),
                  conv=DeviceArray.from_numpy(na.BF16, conv0, (C, 3, slots)),
                  w=DeviceArray.from_numpy(na.BF16, w, (C, 4)),
                  slot=DeviceArray.from_numpy(na.I32, np.array([1], np.int32), (1,)),
                  accepted=DeviceArray.from_numpy(na.I32, np.array([0], np.int32), (1,)),
                  x=DeviceArray(na.BF16, (C, T)), xo=DeviceArray(na.BF16, (C, T)),
                  q=DeviceArray(na.BF16, (S, Hqk, T)), k=DeviceArray(na.BF16, (S, Hqk, T)),
                  v=DeviceArray(na.BF16, (S, Hv, T)), g=DeviceArray(na.FP32, (Hv, T)),
                  beta=DeviceArray(na.FP32, (Hv, T)), out=DeviceArray(na.BF16, (S, Hv, T)))
        states.append(st)
    scale = float(np.float32(1 / np.sqrt(S)))

    def gdn_ops(st):
        ops.causal_conv1d_silu_snapshot(st["x"].tensor(), st["w"].tensor(), st["conv"].tensor(), st["slot"].tensor(),
                                        st["xo"].tensor(), stream)
        ops.gated_delta_rule_snapshot(st["q"].tensor(), st["k"].tensor(), st["v"].tensor(), st["g"].tensor(),
                                      st["beta"].tensor(), scale, True, st["ssm"].tensor(), st["slot"].tensor(),
                                      st["out"].tensor(), stream)
        ops.assign_i32_scalar(st["accepted"].tensor(), st["slot"].tensor(), stream)

    graph = _capture(stream, lambda: gdn_ops(states[0]))
    ssm, conv, slot = ssm0.astype(np.float64), conv0.copy(), 1
    for r in range(ROUNDS):
        print(f"case gdn graph round {r}", flush=True)
        q = syn.f32_to_bf16_bits(rng.uniform(-1, 1, (T, Hqk, S)).astype(np.float32))
        k = syn.f32_to_bf16_bits(rng.uniform(-1, 1, (T, Hqk, S)).astype(np.float32))
        v = syn.f32_to_bf16_bits(rng.uniform(-1, 1, (T, Hv, S)).astype(np.float32))
        g = rng.uniform(-4.0, 0.0, (T, Hv)).astype(np.float32)
        beta = rng.uniform(0.05, 0.95, (T, Hv)).astype(np.float32)
        x = syn.f32_to_bf16_bits(rng.uniform(-2, 2, (T, C)).astype(np.float32))
        accepted = (r * 3 + 1) % T
        for st in states:
            for n, a in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta), ("x", x)):
                st[n].upload(a)
            ops.set_i32_scalar(st["accepted"].tensor(), accepted, stream)
        graph.launch()
        gdn_ops(states[1])
        stream.synchronize()
        for n in ("out", "xo", "ssm", "conv", "slot"):
            assert np.array_equal(states[0][n].numpy(), states[1][n].numpy()), f"graph replay differs in {n}"
        ref, _, snaps = oracle.gdn_recurrent(q, k, v, g, beta, ssm[slot].astype(np.float32), S, Hqk, Hv, T,
                                             normalize_qk=True, snapshots=True)
        ok, msg = reference_composite_ok(_f32(states[0]["out"].numpy()), ref.reshape(-1),
                                         (1e-3, 1.0e-2, 2e-3, 5.0, 8e-3))
        assert ok, msg
        got_ssm = states[0]["ssm"].numpy().reshape(slots, Hv, S, S)
        ok, msg = reference_composite_ok(got_ssm[:T].astype(np.float64), snaps, (5e-4, 5.0e-3, 2e-2, 5.0, 5e-3))
        assert ok, msg
        cref, windows = oracle.causal_conv1d_silu(x, w, conv[slot], C, T)
        ok, msg = reference_composite_ok(_f32(states[0]["xo"].numpy()), cref.reshape(-1),
                                         (2e-3, 1.6e-2, 2e-3, 5.0, 8e-3))
        assert ok, msg
        got_conv = states[0]["conv"].numpy().reshape(slots, 3, C)
        assert np.array_equal(got_conv[:T], windows)
        assert states[0]["slot"].numpy()[0] == accepted
        # the next round starts from the accepted slot of the states the GPU holds now
        ssm, conv, slot = got_ssm.astype(np.float64), got_conv.copy(), accepted
