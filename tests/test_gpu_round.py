"""One whole verify round captured once as a HIP graph and replayed round after round, as a serving
loop runs the MTP decode (reference src/targets/qwen3_6/impl/runtime/speculative_impl.h:35-45 and
program_impl.h:780-870; replay contract docs/maintainer/op-development.md:106-123):

  prepare verify ids / positions (from the device length) -> A1 attention of every full-attention
  layer (INT8-G64 caches, new rows appended at the device positions) -> lm_head (Q6G64 linear) ->
  argmax -> greedy acceptance (advances length, sets token, stats) -> accepted hidden row ->
  MTP alignment ids -> recurrent-state slot = accepted.

The "fused" form runs the lm_head and the acceptance as one call (nmi_speculative_accept_fused_head:
per-workgroup top-20 keys, no logits written); its logits for the oracle check come from an eager
linear on the same input after each replay.

Between replays only the round's inputs change (per-layer q/k/v, the lm_head input rows, the draft
tokens and the hidden rows), uploaded by the host; every piece of state the round carries (length,
token, positions, caches, stats, the state slot) moves on the device. Every replay is checked against
the same calls made eagerly on a twin state (bit-exact) and against the oracle (attention within
2e-3 relative L2, cache bytes, accept decisions and ids exact, targets = the argmax of the logits)."""
import numpy as np
import pytest

import ninfer_amd as na
import q6_pack as qp
from helpers import AttnCase, rel_l2
from ninfer_amd import ops, synthetic as syn
from ninfer_amd.device import DeviceArray, DeviceBuffer, Graph, Stream
from test_gpu_linear import DeviceWeight, oracle_logits
import gpu_runner

pytestmark = pytest.mark.gpu

ROUNDS, LAYERS, T, K = 4, 3, 4, 3
Hq, Hkv, D = 40, 8, 128
V, VALID, HID = 2048, 2000, 512


def _f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("head_form", ["unfused", "fused"])
def test_full_round_graph_replay(gpu, oracle, head_form):
    fused = head_form == "fused"
    L0 = 1500
    max_ctx = L0 + ROUNDS * T + T
    rng = np.random.default_rng(2024)
    codes = rng.integers(-32, 32, (V, HID))
    nib, high = qp.pack_codes(codes)
    sc = np.float16(rng.uniform(0.005, 0.03, (V, HID // 64))).view(np.uint16)
    head = DeviceWeight(nib, high, sc, V, HID)
    cases = [AttnCase([L0], T=T, seed=300 + l, max_context=max_ctx) for l in range(LAYERS)]
    P = cases[0].P
    stream = Stream()

    def make_state():
        st = dict(caches=[gpu_runner.upload_cache(c) for c in cases],
                  q=[DeviceArray(na.BF16, (D, Hq, T)) for _ in range(LAYERS)],
                  k=[DeviceArray(na.BF16, (D, Hkv, T)) for _ in range(LAYERS)],
                  v=[DeviceArray(na.BF16, (D, Hkv, T)) for _ in range(LAYERS)],
                  out=[DeviceArray(na.BF16, (D, Hq, T)) for _ in range(LAYERS)],
                  ws=DeviceBuffer(ops.gqa_attention_workspace_bytes(Hq, Hkv, D, T, 1, max_ctx)),
                  token=DeviceArray.from_numpy(na.I32, np.array([11], np.int32), (1,)),
                  drafts=DeviceArray(na.I32, (K,)),
                  length=DeviceArray.from_numpy(na.I32, np.array([L0], np.int32), (1,)),
                  ids=DeviceArray(na.I32, (T,)), pos=DeviceArray(na.I32, (T,)),
                  x=DeviceArray(na.BF16, (HID, T)), logits=DeviceArray(na.BF16, (V, T)),
                  target=DeviceArray(na.I32, (T,)), so=DeviceArray(na.I32, (T,)), ns=DeviceArray(na.I32, (1,)),
                  acc=DeviceArray(na.I32, (1,)),
                  stats=DeviceArray.from_numpy(na.I64, np.zeros(4 + K, np.int64), (4 + K,)),
                  sws=DeviceBuffer(max(256, ops.sampling_workspace_bytes(VALID, T))),
                  hws=DeviceBuffer(ops.speculative_accept_fused_head_workspace_bytes(K, 1)),
                  hidden=DeviceArray(na.BF16, (HID, T)), sel=DeviceArray(na.BF16, (HID, 1)),
                  align=DeviceArray.from_numpy(na.I32, np.full(T, -1, np.int32), (T,)),
                  slot=DeviceArray.from_numpy(na.I32, np.array([-1], np.int32), (1,)))
        cfg, keep = gpu_runner.upload_configs([na.SamplingConfig()])  # greedy (temperature 0)
        st["cfg"], st["keep"] = cfg, keep
        st["ws"].fill(0xFF)
        st["hws"].fill(0xFF)
        st["x3"] = DeviceArray(na.BF16, (HID, T, 1), buf=st["x"].buf)
        return st

    states = [make_state(), make_state()]  # [graph, eager]

    def round_ops(st):
        ops.speculative_prepare_verify_inputs(st["token"].tensor(), st["drafts"].tensor(), st["length"].tensor(),
                                              st["ids"].tensor(), st["pos"].tensor(), stream)
        for l in range(LAYERS):
            ops.gqa_attention(st["q"][l].tensor(), st["k"][l].tensor(), st["v"][l].tensor(), st["pos"].tensor(),
                              cases[0].scale, st["caches"][l].view(), (1, max_ctx), st["ws"],
                              st["out"][l].tensor(), stream)
        if fused:
            ops.speculative_accept_fused_head(st["x3"].tensor(), head.w, st["drafts"].tensor(), st["length"].tensor(),
                                              st["token"].tensor(), st["so"].tensor(), st["ns"].tensor(),
                                              st["acc"].tensor(), st["stats"].tensor(), VALID, st["cfg"].ptr,
                                              st["hws"], stream)
        else:
            ops.linear(st["x"].tensor(), head.w, st["logits"].tensor(), stream)
            ops.argmax(st["logits"].tensor(), st["target"].tensor(), VALID, stream)
            ops.speculative_accept_greedy_drafts(st["target"].tensor(), st["logits"].tensor(), st["drafts"].tensor(),
                                                 st["length"].tensor(), st["token"].tensor(), st["so"].tensor(),
                                                 st["ns"].tensor(), st["acc"].tensor(), st["stats"].tensor(), VALID,
                                                 st["cfg"].ptr, st["sws"], stream)
        ops.speculative_select_accepted_hidden(st["hidden"].tensor(), st["acc"].tensor(), st["sel"].tensor(), stream)
        ops.mtp_prepare_alignment_ids(st["ids"].tensor(), st["token"].tensor(), st["acc"].tensor(),
                                      st["align"].tensor(), stream)
        ops.assign_i32_scalar(st["acc"].tensor(), st["slot"].tensor(), stream)

    graph = Graph(stream)
    with graph:
        round_ops(states[0])

    planes = [list(c.cache_planes()) for c in cases]
    planes = [[a.copy() for a in p] for p in planes]
    length, token, stats = L0, 11, np.zeros(4 + K, np.int64)
    align = np.full(T, -1, np.int32)
    for r in range(ROUNDS):
        print(f"case whole round graph replay ({head_form}) round {r} length {length}", flush=True)
        q = [syn.normal_bf16(syn.derive_seed(40, r, l, 1), D * Hq * T) for l in range(LAYERS)]
        kk = [syn.normal_bf16(syn.derive_seed(40, r, l, 2), D * Hkv * T) for l in range(LAYERS)]
        vv = [syn.normal_bf16(syn.derive_seed(40, r, l, 3), D * Hkv * T) for l in range(LAYERS)]
        x = syn.f32_to_bf16_bits(rng.uniform(-1, 1, (T, HID)).astype(np.float32))
        hidden = syn.normal_bf16(syn.derive_seed(41, r), HID * T)
        # drafts planted to agree with the first `agree` targets of this round (from the oracle's
        # logits), then one disagreement; the GPU's own logits decide in the end
        ref64 = oracle_logits(head, x)
        want = [qp.argmax_lowest(qp.f64_to_bf16_bits(ref64[t]), VALID) for t in range(T)]
        agree = r % (K + 1)
        drafts = np.array([want[i] if i < agree else (want[i] + 1) % VALID for i in range(K)], np.int32)
        for st in states:
            for l in range(LAYERS):
                st["q"][l].upload(q[l])
                st["k"][l].upload(kk[l])
                st["v"][l].upload(vv[l])
            st["x"].upload(x)
            st["hidden"].upload(hidden)
            st["drafts"].upload(drafts)
        graph.launch()
        round_ops(states[1])
        if fused:  # the logits the fused call never wrote, for the checks below
            ops.linear(states[0]["x"].tensor(), head.w, states[0]["logits"].tensor(), stream)
        stream.synchronize()
        g, e = states
        names = ["ids", "pos", "so", "ns", "acc", "length", "token", "stats", "sel", "align", "slot"]
        if not fused:
            names += ["logits", "target"]
        for name in names:
            assert np.array_equal(g[name].numpy(), e[name].numpy()), f"round {r}: graph != eager in {name}"
        for l in range(LAYERS):
            assert np.array_equal(g["out"][l].numpy(), e["out"][l].numpy()), f"round {r} layer {l}"
        # verify inputs
        pos = np.arange(length, length + T, dtype=np.int32)
        assert list(g["pos"].numpy()) == list(pos)
        assert list(g["ids"].numpy()) == [token] + list(drafts)
        # attention and caches against the oracle
        for l in range(LAYERS):
            kc, vc, ks, vs = planes[l]
            oracle.kv_append(kk[l], vv[l], pos, T, 1, Hkv, D, P, kc, vc, ks, vs)
            ref = oracle.attention(q[l], kc, vc, ks, vs, pos, None, T, 1, Hq, Hkv, D, P, cases[0].scale)
            assert rel_l2(_f32(g["out"][l].numpy()), ref) <= 2e-3, (r, l)
            for got, exp in zip(g["caches"][l].download(), planes[l]):
                assert np.array_equal(got, exp), (r, l)
        # targets are the argmax of the logits the lm_head wrote; acceptance follows the oracle
        logits = g["logits"].numpy().reshape(T, V)
        tgt = np.array([qp.argmax_lowest(logits[t], VALID) for t in range(T)], np.int32)
        if not fused:
            assert list(g["target"].numpy()) == list(tgt)
        exp = oracle.speculative_accept(tgt, logits.reshape(-1), V, drafts, length, stats, VALID,
                                        oracle.SamplingConfig())
        assert list(g["so"].numpy()) == list(exp["sampled_out"]), r
        assert g["length"].numpy()[0] == exp["length"] and g["token"].numpy()[0] == exp["token"]
        assert list(g["stats"].numpy()) == list(exp["stats"])
        a = exp["accepted"]
        assert g["acc"].numpy()[0] == a and g["slot"].numpy()[0] == a
        assert np.array_equal(g["sel"].numpy(), hidden.reshape(T, HID)[a])
        align = oracle.mtp_prepare_alignment_ids(np.array([token] + list(drafts), np.int32), exp["token"], a, align)
        assert list(g["align"].numpy()) == list(align)
        length, token, stats = exp["length"], exp["token"], exp["stats"]
