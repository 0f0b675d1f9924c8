"""GPU parity of the fused lm_head + acceptance (nmi_speculative_accept_fused_head): the Q6G64 lm_head
keeps, per verify column, the 20 largest (penalty-adjusted) logit keys per workgroup instead of writing
the [V, K+1] logits, and the acceptance merges them (the top-cap half of the reference's deferred
FUT-F03 fusion, docs/maintainer/qwen3.6-35b-a3b-dflash-op-checklist.md:985-1001, replacing the
per-tile candidate pass of src/ops/kernel/speculative_round.cuh:169-211).

Two bars, as the route composes an FP32-summed linear with a bit-exact acceptance:
  * composition, bit-exact: the fused call decides exactly what the oracle's acceptance
    (orc_speculative_accept) decides on the BF16 logits the unfused GPU lm_head writes for the same
    input (sampled tokens, counts, length, token, stats and the token_counts side effect);
  * the FP64 oracle end to end: the oracle's Q6 linear (BF16 of the FP64 sums) then the oracle's
    acceptance. The two agree unless a logit that enters the decision (a column's 20 candidates, or
    the argmax of a greedy column) is one BF16 step away from the oracle's, which the linear's bar
    allows; the test checks that this is the only way they differ.
Workloads: the reference's [248320, 5120] output head (patterned, seed 4226) with K = 3 drafts at
B = 1 (greedy and every Mode R option) and B = 16 (mixed configurations), plus small heads that take
several column passes, a token domain below the row count and a domain smaller than the cap."""
import numpy as np
import pytest

import ninfer_amd as na
import q6_pack as qp
from ninfer_amd import ops, synthetic as syn
from ninfer_amd.device import DeviceArray, DeviceBuffer, synchronize
from test_gpu_linear import VOCAB, DeviceWeight, check_logits, oracle_logits, run_linear
import gpu_runner

pytestmark = pytest.mark.gpu

K = 3


def _cfg(temperature=0.0, top_k=0, top_p=1.0, min_p=0.0, presence=0.0, frequency=0.0, seed=0):
    c = na.SamplingConfig()
    c.temperature, c.top_k, c.top_p, c.min_p = temperature, top_k, top_p, min_p
    c.presence_penalty, c.frequency_penalty, c.seed = presence, frequency, seed
    return c


def _ocfg(c):
    from oracle import pyoracle
    o = pyoracle.SamplingConfig()
    for f, _ in pyoracle.SamplingConfig._fields_:
        setattr(o, f, getattr(c, f))
    return o


def run_fused(dw, x, drafts, length, stats, token_domain, cfgs, token_counts=None):
    """x uint16 [B, K+1, hidden]; drafts int32 [B, K]."""
    B = len(cfgs)
    hidden = x.shape[-1]
    d_x = DeviceArray.from_numpy(na.BF16, x, (hidden, K + 1, B))
    d_drafts = DeviceArray.from_numpy(na.I32, np.asarray(drafts, np.int32), (K, B))
    d_len = DeviceArray.from_numpy(na.I32, np.asarray(length, np.int32), (B,))
    d_tok = DeviceArray.from_numpy(na.I32, np.full(B, -1, np.int32), (B,))
    d_so = DeviceArray.from_numpy(na.I32, np.full((B, K + 1), -7, np.int32), (K + 1, B))
    d_ns = DeviceArray.from_numpy(na.I32, np.zeros(B, np.int32), (B,))
    d_acc = DeviceArray.from_numpy(na.I32, np.zeros(B, np.int32), (B,))
    st = np.asarray(stats, np.int64).reshape(B, -1)
    d_stats = DeviceArray.from_numpy(na.I64, st, (st.shape[1], B))
    cfg_buf, keep = gpu_runner.upload_configs(cfgs, token_counts)
    ws = DeviceBuffer(ops.speculative_accept_fused_head_workspace_bytes(K, B))
    ws.fill(0xFF)
    ops.speculative_accept_fused_head(d_x.tensor(), dw.w, d_drafts.tensor(), d_len.tensor(), d_tok.tensor(),
                                      d_so.tensor(), d_ns.tensor(), d_acc.tensor(), d_stats.tensor(), token_domain,
                                      cfg_buf.ptr, ws)
    synchronize()
    out = dict(sampled_out=d_so.numpy().reshape(B, K + 1), num_sampled=d_ns.numpy(), accepted=d_acc.numpy(),
               token=d_tok.numpy(), length=d_len.numpy(), stats=d_stats.numpy().reshape(B, -1))
    if token_counts is None:
        out["token_counts"] = None
    else:  # upload_configs keeps a device array for each sequence that has counts, in order
        it = iter(keep)
        out["token_counts"] = [None if tc is None else next(it).numpy() for tc in token_counts]
    return out


def oracle_accept(logits, drafts, length, stats, token_domain, cfgs, token_counts=None):
    """The oracle's acceptance per sequence over BF16 logits uint16 [B, K+1, N]."""
    from oracle import pyoracle
    B, _, N = logits.shape
    res = []
    for b in range(B):
        tgt = np.array([qp.argmax_lowest(logits[b, c], token_domain) for c in range(K + 1)], np.int32)
        tc = None if token_counts is None or token_counts[b] is None else token_counts[b].copy()
        res.append(pyoracle.speculative_accept(tgt, logits[b].reshape(-1), N, drafts[b], int(length[b]), stats[b],
                                               token_domain, _ocfg(cfgs[b]), tc))
    return res


def _same(got, exp, b):
    return (list(got["sampled_out"][b]) == list(exp["sampled_out"]) and got["num_sampled"][b] == exp["num_sampled"]
            and got["accepted"][b] == exp["accepted"] and got["token"][b] == exp["token"]
            and got["length"][b] == exp["length"] and list(got["stats"][b]) == list(exp["stats"]))


def _decision_rows(logits_b, token_domain, cfg, drafts_b, counts_b):
    """Rows whose logit can enter a sequence's decision: per column the 40 largest raw logits (the
    argmax and the 20 candidates with room to spare) and, with penalties, the 40 largest adjusted."""
    rows = set()
    for c in range(K + 1):
        raw = syn.bf16_bits_to_f32(logits_b[c][:token_domain]).astype(np.float64)
        rows.update(np.argsort(-raw, kind="stable")[:40].tolist())
        if cfg.presence_penalty != 0.0 or cfg.frequency_penalty != 0.0:
            cnt = np.zeros(token_domain, np.int64) if counts_b is None else counts_b[:token_domain].astype(np.int64)
            for d in drafts_b[:c]:
                if d < token_domain:
                    cnt[d] += 1
            adj = raw - cfg.presence_penalty * (cnt > 0) - cfg.frequency_penalty * cnt
            rows.update(np.argsort(-adj, kind="stable")[:40].tolist())
    return sorted(rows)


def check_case(dw, x, drafts, length, token_domain, cfgs, token_counts=None, tag=""):
    B = len(cfgs)
    T = B * (K + 1)
    stats = np.zeros((B, 4 + K), np.int64)
    stats[:, 0] = np.arange(B) * 7  # prior counts carry through
    got = run_fused(dw, x, drafts, length, stats, token_domain, cfgs, token_counts)
    x2 = x.reshape(T, -1)
    gpu_logits = run_linear(dw, x2).reshape(B, K + 1, dw.n)
    ref64 = oracle_logits(dw, x2)
    check_logits(gpu_logits.reshape(T, dw.n), ref64, f"{tag} lm_head")
    orc_logits = qp.f64_to_bf16_bits(ref64).reshape(B, K + 1, dw.n)
    comp = oracle_accept(gpu_logits, drafts, length, stats, token_domain, cfgs, token_counts)
    full = oracle_accept(orc_logits, drafts, length, stats, token_domain, cfgs, token_counts)
    for b in range(B):
        print(f"{tag} seq {b}: T={cfgs[b].temperature} accepted {got['accepted'][b]} sampled "
              f"{list(got['sampled_out'][b])}", flush=True)
        assert _same(got, comp[b], b), (tag, b, got["sampled_out"][b], comp[b]["sampled_out"])
        if token_counts is not None and token_counts[b] is not None:
            assert np.array_equal(got["token_counts"][b], comp[b]["token_counts"]), (tag, b)
        if not _same(got, full[b], b):
            rows = _decision_rows(orc_logits[b], token_domain, cfgs[b], drafts[b],
                                  None if token_counts is None else token_counts[b])
            differ = any(not np.array_equal(gpu_logits[b, :, r], orc_logits[b, :, r]) for r in rows)
            assert differ, f"{tag} seq {b}: differs from the FP64 oracle with equal decision logits"
            print(f"{tag} seq {b}: a decision logit is one BF16 step from the FP64 oracle's", flush=True)


def _x(seed, B, hidden):
    rng = np.random.default_rng(seed)
    return syn.f32_to_bf16_bits(rng.uniform(-1, 1, (B, K + 1, hidden)).astype(np.float32))


def _plant(dw, x, token_domain, mode, seed):
    """Drafts: the oracle's top candidates of the columns (accepted often), a runner-up and a miss."""
    B = x.shape[0]
    ref = qp.f64_to_bf16_bits(oracle_logits(dw, x.reshape(B * (K + 1), -1))).reshape(B, K + 1, dw.n)
    rng = np.random.default_rng(seed)
    drafts = np.zeros((B, K), np.int32)
    for b in range(B):
        for i in range(K):
            key = qp.bf16_order_key(ref[b, i][:token_domain]).astype(np.int64)
            order = np.argsort(-key, kind="stable")
            pick = 0 if mode < 0 else (mode + b + i) % 3
            drafts[b, i] = order[0] if pick == 0 else (order[1] if pick == 1 else rng.integers(0, token_domain))
    return drafts


@pytest.fixture(scope="module")
def big_head():
    print(f"case fused head Q6 [{VOCAB}, 5120] patterned seed 4226", flush=True)
    nib, high, sc = qp.patterned(VOCAB, 5120, 4226)
    return DeviceWeight(nib, high, sc, VOCAB, 5120)


B1_CONFIGS = {
    "greedy": _cfg(),
    "t07_top_p": _cfg(temperature=0.7, top_p=0.95, seed=11),
    "t1_top_k5": _cfg(temperature=1.0, top_k=5, seed=12),
    "t08_min_p": _cfg(temperature=0.8, min_p=0.1, seed=13),
    "t2_flat": _cfg(temperature=2.0, seed=14),
    "penalties": _cfg(temperature=0.7, top_p=0.9, presence=0.5, frequency=0.25, seed=15),
}


@pytest.mark.parametrize("name", list(B1_CONFIGS))
def test_fused_head_b1(gpu, big_head, name):
    print(f"case fused head B=1 {name}", flush=True)
    x = _x(500 + len(name), 1, 5120)
    for L, mode in ((600, 0), (601, 1), (602, 2), (603, -1)):
        # mode -1: every draft is its column's top candidate, so acceptance runs deep
        drafts = _plant(big_head, x, VOCAB, mode, 7)
        counts = None
        if name == "penalties":
            rng = np.random.default_rng(3)
            tc = np.zeros(VOCAB, np.int32)
            tc[rng.integers(0, VOCAB, 4000)] = rng.integers(1, 4, 4000)
            tc[drafts[0]] = 2  # the planted drafts carry history
            counts = [tc]
        check_case(big_head, x, drafts, [L], VOCAB, [B1_CONFIGS[name]], counts, tag=f"B=1 {name} L={L}")


def test_fused_head_b1_token_domain(gpu, big_head):
    """Rows [151936, 248320) are padding: neither a candidate nor the argmax."""
    print("case fused head B=1 token_domain 151936", flush=True)
    x = _x(77, 1, 5120)
    drafts = _plant(big_head, x, 151936, 0, 8)
    for cfg in (_cfg(), _cfg(temperature=0.9, top_p=0.8, seed=5)):
        check_case(big_head, x, drafts, [1000], 151936, [cfg], tag=f"domain T={cfg.temperature}")


def test_fused_head_b16(gpu, big_head):
    print("case fused head B=16 mixed configurations", flush=True)
    B = 16
    x = _x(1616, B, 5120)
    drafts = _plant(big_head, x, VOCAB, 1, 9)
    names = list(B1_CONFIGS)
    cfgs = []
    for b in range(B):
        c = B1_CONFIGS[names[b % len(names)]]
        cfgs.append(_cfg(c.temperature, c.top_k, c.top_p, c.min_p, c.presence_penalty, c.frequency_penalty,
                         seed=100 + b))
    rng = np.random.default_rng(4)
    counts = []
    for b in range(B):
        if cfgs[b].presence_penalty != 0.0:
            tc = np.zeros(VOCAB, np.int32)
            tc[rng.integers(0, VOCAB, 2000)] = 1
            tc[drafts[b]] = 1
            counts.append(tc)
        else:
            counts.append(None)
    length = 400 + 37 * np.arange(B)
    check_case(big_head, x, drafts, length, VOCAB, cfgs, counts, tag="B=16")


@pytest.mark.parametrize("N,hidden,B,domain", [(1000, 512, 1, 1000), (5000, 640, 3, 4321), (3000, 1024, 5, 3000),
                                               (17, 256, 2, 9), (2048, 8192, 2, 2048), (6000, 1024, 9, 5000),
                                               (20000, 2048, 16, 19000)])
def test_fused_head_small_heads(gpu, N, hidden, B, domain):
    """Rows not a multiple of 16, a token domain below the cap (9 < 20 candidates), padded K and the
    largest K; more than 16 columns (B = 5, 9, 16) take the K-outer form, 32 columns per pass. The
    penalty counts hold exactly the token domain."""
    print(f"case fused head N={N} hidden={hidden} B={B} domain={domain}", flush=True)
    rng = np.random.default_rng(N + hidden + B)
    Kp = qp.align_up(hidden, 128)
    nib, high = qp.pack_codes(rng.integers(-32, 32, (N, Kp)))
    sc = np.float16(rng.uniform(0.001, 0.05, (N, Kp // 64))).view(np.uint16)
    dw = DeviceWeight(nib, high, sc, N, hidden)
    x = _x(N * 3 + B, B, hidden)
    drafts = _plant(dw, x, domain, 2, 10)
    names = list(B1_CONFIGS)
    cfgs = [B1_CONFIGS[names[(b + N) % len(names)]] for b in range(B)]
    counts = [np.ones(domain, np.int32) if c.presence_penalty != 0.0 else None for c in cfgs]
    check_case(dw, x, drafts, 50 + np.arange(B), domain, cfgs, counts, tag=f"N={N} hidden={hidden} B={B}")


def test_fused_head_rejects_bad_shapes(gpu, big_head):
    x = DeviceArray(na.BF16, (5120, K + 1, 2))
    drafts = DeviceArray(na.I32, (K, 1))
    scal = [DeviceArray(na.I32, (1,)) for _ in range(4)]
    so = DeviceArray(na.I32, (K + 1, 1))
    stats = DeviceArray(na.I64, (4 + K, 1))
    cfg_buf, _ = gpu_runner.upload_configs([_cfg()])
    ws = DeviceBuffer(ops.speculative_accept_fused_head_workspace_bytes(K, 1))
    with pytest.raises(ValueError):  # x has 2 sequences, drafts 1
        ops.speculative_accept_fused_head(x.tensor(), big_head.w, drafts.tensor(), scal[0].tensor(), scal[1].tensor(),
                                          so.tensor(), scal[2].tensor(), scal[3].tensor(), stats.tensor(), VOCAB,
                                          cfg_buf.ptr, ws)
    x1 = DeviceArray(na.BF16, (5120, K + 1, 1))
    with pytest.raises(ValueError):  # token domain past the rows
        ops.speculative_accept_fused_head(x1.tensor(), big_head.w, drafts.tensor(), scal[0].tensor(), scal[1].tensor(),
                                          so.tensor(), scal[2].tensor(), scal[3].tensor(), stats.tensor(), VOCAB + 1,
                                          cfg_buf.ptr, ws)
    small = DeviceBuffer(ops.speculative_accept_fused_head_workspace_bytes(K, 1) - 256)
    with pytest.raises(ValueError):  # workspace below the query
        ops.speculative_accept_fused_head(x1.tensor(), big_head.w, drafts.tensor(), scal[0].tensor(), scal[1].tensor(),
                                          so.tensor(), scal[2].tensor(), scal[3].tensor(), stats.tensor(), VOCAB,
                                          cfg_buf.ptr, small)
