"""GPU parity of the acceptance half (argmax, greedy and reference-stochastic acceptance, tree
acceptance, accepted-hidden selection) against the reference's known answers and the CPU oracle.
Every comparison here is bit-exact."""
import json
from pathlib import Path

import numpy as np
import pytest

import ninfer_amd as na
from ninfer_amd import ops
from ninfer_amd import synthetic as syn
from ninfer_amd.device import DeviceArray, synchronize
import gpu_runner

pytestmark = pytest.mark.gpu

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
BF = syn.f32_to_bf16_bits


def _cfg(temperature=0.0, top_k=0, top_p=1.0, min_p=0.0, presence=0.0, frequency=0.0, seed=0):
    c = na.SamplingConfig()
    c.temperature, c.top_k, c.top_p, c.min_p = temperature, top_k, top_p, min_p
    c.presence_penalty, c.frequency_penalty, c.seed = presence, frequency, seed
    return c


def _ocfg(c):
    from oracle import pyoracle
    o = pyoracle.SamplingConfig()
    o.temperature, o.top_k, o.top_p, o.min_p = c.temperature, c.top_k, c.top_p, c.min_p
    o.presence_penalty, o.frequency_penalty, o.seed = c.presence_penalty, c.frequency_penalty, c.seed
    return o


def _flat(res, b=0):
    K1 = res["sampled_out"].shape[1]
    return list(res["sampled_out"][b][:K1]) + [int(res["num_sampled"][b]), int(res["accepted"][b])]


# ---- argmax -----------------------------------------------------------------------------------------

def test_argmax_ties_and_domain(gpu, oracle):
    rows, domain, C = 248320, 248077, 4
    x = syn.normal_bf16(7, rows * C, std=2.0).reshape(C, rows)
    peak = BF(np.array([50.0], dtype=np.float32))[0]
    x[0, 1000] = peak
    x[0, 500] = peak          # tie: lowest id (500) wins
    x[1, domain + 5] = BF(np.array([99.0], dtype=np.float32))[0]  # outside the token domain
    x[2, domain - 1] = peak   # last valid row
    x[3, :] = BF(np.array([-0.0], dtype=np.float32))[0]
    x[3, 9] = 0               # +0 ties with -0: lowest id (0) wins
    d = DeviceArray.from_numpy(na.BF16, x, (rows, C))
    out = DeviceArray(na.I32, (C,))
    ops.argmax(d.tensor(), out.tensor(), domain)
    synchronize()
    got = out.numpy()
    exp = oracle.argmax(x.reshape(-1), rows, C, domain)
    brute = [int(np.argmax(syn.bf16_bits_to_f32(x[c, :domain]))) for c in range(C)]
    assert list(got) == list(exp) == brute
    assert got[0] == 500 and got[2] == domain - 1 and got[3] == 0


def test_argmax_packed_key_cases(gpu, oracle):
    """Cases the packed 16-bit pass resolves afterwards: the maximum inside a load, ties inside one
    load and across threads, all-negative columns, zero maxima with -0 after +0, and an odd
    physical stride (scalar path)."""
    C = 8
    rows, domain = 248320, 248320
    x = syn.normal_bf16(11, rows * C, std=2.0).reshape(C, rows)
    big = BF(np.array([40.0], dtype=np.float32))[0]
    x[0, 8 * 777 + 5] = big
    x[1, 8 * 900 + 6] = big
    x[1, 8 * 900 + 3] = big                                   # tie inside one load: id ...3 wins
    x[2, 8 * 5000 + 1] = big
    x[2, 8 * 4000 + 7] = big                                  # tie across threads: lower id wins
    x[3, :] = BF(-np.abs(syn.bf16_bits_to_f32(x[3])) - 1.0)   # all negative
    x[4, :] = BF(np.array([-3.0], dtype=np.float32))[0]
    x[4, 8 * 1200 + 2] = 0                                    # +0 first ...
    x[4, 8 * 3000 + 4] = BF(np.array([-0.0], dtype=np.float32))[0]  # ... then -0: +0 (lower id) wins
    x[5, :] = BF(np.array([-3.0], dtype=np.float32))[0]
    x[5, 8 * 2000 + 1] = BF(np.array([-0.0], dtype=np.float32))[0]  # only -0 at the top
    x[6, 8 * 31000 + 7] = BF(np.array([np.inf], dtype=np.float32))[0]
    x[7, :] = big                                             # everything ties: id 0
    d = DeviceArray.from_numpy(na.BF16, x, (rows, C))
    out = DeviceArray(na.I32, (C,))
    ops.argmax(d.tensor(), out.tensor(), domain)
    synchronize()
    got = out.numpy()
    exp = oracle.argmax(x.reshape(-1), rows, C, domain)
    brute = [int(np.argmax(syn.bf16_bits_to_f32(x[c, :domain]))) for c in range(C)]
    assert list(got) == list(exp) == brute
    # odd physical stride: columns are not 16-byte aligned
    rows2, dom2 = 4099, 4097
    y = syn.normal_bf16(12, rows2 * 3, std=2.0).reshape(3, rows2)
    y[1, 4096] = big
    d2 = DeviceArray.from_numpy(na.BF16, y, (rows2, 3))
    out2 = DeviceArray(na.I32, (3,))
    ops.argmax(d2.tensor(), out2.tensor(), dom2)
    synchronize()
    exp2 = oracle.argmax(y.reshape(-1), rows2, 3, dom2)
    assert list(out2.numpy()) == list(exp2)


@pytest.mark.parametrize("prior", ["low_row", "negative", "huge", "answer", "last_row"])
def test_argmax_whatever_out_held_before(gpu, oracle, prior):
    """The tiled argmax folds its tiles into out[] by compare-and-swap without zeroing it first: an
    in-range prior value is a real candidate the argmax beats or equals, an out-of-range one is
    none, so the result is the argmax whatever out held (here also an odd physical stride, so the
    columns take the unaligned path)."""
    for rows, domain in ((248320, 248077), (100001, 99999)):
        C = 4
        x = syn.normal_bf16(13 + rows % 7, rows * C, std=2.0).reshape(C, rows)
        x[1, 77] = BF(np.array([30.0], dtype=np.float32))[0]
        x[2, domain - 1] = BF(np.array([30.0], dtype=np.float32))[0]
        exp = oracle.argmax(x.reshape(-1), rows, C, domain)
        low = [int(np.argmin(syn.bf16_bits_to_f32(x[c, :domain]))) for c in range(C)]
        init = {"low_row": low, "negative": [-5] * C, "huge": [1 << 30] * C, "answer": list(exp),
                "last_row": [domain - 1] * C}[prior]
        d = DeviceArray.from_numpy(na.BF16, x, (rows, C))
        out = DeviceArray.from_numpy(na.I32, np.array(init, np.int32), (C,))
        ops.argmax(d.tensor(), out.tensor(), domain)
        synchronize()
        assert list(out.numpy()) == list(exp), (rows, prior)


# ---- reference known answers -------------------------------------------------------------------------

def test_prepare_verify_inputs_kat(gpu):
    k = KATS["prepare_verify"]
    K = len(k["drafts"])
    tok = DeviceArray.from_numpy(na.I32, np.array([k["token"]], dtype=np.int32), (1,))
    dr = DeviceArray.from_numpy(na.I32, np.array(k["drafts"], dtype=np.int32), (K,))
    ln = DeviceArray.from_numpy(na.I32, np.array([k["length"]], dtype=np.int32), (1,))
    ids = DeviceArray(na.I32, (K + 1,))
    pos = DeviceArray(na.I32, (K + 1,))
    ops.speculative_prepare_verify_inputs(tok.tensor(), dr.tensor(), ln.tensor(), ids.tensor(), pos.tensor())
    synchronize()
    assert list(ids.numpy()) == k["verify_ids"]
    assert list(pos.numpy()) == k["positions"]
    assert ln.numpy()[0] == k["length"]


@pytest.mark.parametrize("idx", range(4))
def test_greedy_kats(gpu, idx):
    k = KATS["greedy"][idx]
    K = k["K"]
    logits = np.zeros((1, K + 1, k["vocab"]), dtype=np.uint16)
    res = gpu_runner.run_accept(logits, [k["drafts"]], [k["length"]], [k["stats_in"]], k["vocab"], [_cfg()],
                                target_tokens=[k["targets"]])
    assert list(res["sampled_out"][0]) == k["sampled_out"]
    assert res["num_sampled"][0] == k["num_sampled"]
    assert res["accepted"][0] == k["accepted"]
    assert res["length"][0] == k["length_out"]
    assert res["token"][0] == k["token"]
    assert list(res["stats"][0]) == k["stats_out"]


def test_exact_k_matrix(gpu):
    m = KATS["exact_k_matrix"]
    rows, domain = m["physical_rows"], m["token_domain"]
    for K in range(1, 16):
        logits = np.full((K + 1, rows), BF(np.array([-20.0], np.float32))[0], dtype=np.uint16)
        ids = [(17 + col * 7919) % domain for col in range(K + 1)]
        for col in range(K + 1):
            logits[col, ids[col]] = BF(np.array([20.0], np.float32))[0]
            logits[col, domain] = BF(np.array([100.0], np.float32))[0]
        drafts = ids[:K]
        cfg = _cfg(temperature=1.0, top_k=1, seed=20260716 + K)
        res = gpu_runner.run_accept(logits[None], [drafts], [100], [[0] * (4 + K)], domain, [cfg])
        assert _flat(res) == drafts + [ids[K], K + 1, K], f"stochastic K={K}"
        mismatch = K // 2
        gd = list(drafts)
        gd[mismatch] = (gd[mismatch] + 1) % domain
        expected = gd[:mismatch] + [ids[mismatch]] + [0] * (K - mismatch) + [mismatch + 1, mismatch]
        res = gpu_runner.run_accept(logits[None], [gd], [100], [[0] * (4 + K)], domain, [_cfg()],
                                    target_tokens=[ids])
        assert _flat(res) == expected, f"greedy K={K}"


def test_physical_stride_token_domain(gpu):
    m = KATS["physical_stride_token_domain"]
    rows, domain = m["physical_rows"], m["token_domain"]
    logits = np.full((2, rows), BF(np.array([-20.0], np.float32))[0], dtype=np.uint16)
    logits[0, m["first"]] = BF(np.array([20.0], np.float32))[0]
    logits[1, m["bonus"]] = BF(np.array([20.0], np.float32))[0]
    for col in range(2):
        logits[col, domain] = BF(np.array([100.0], np.float32))[0]
        logits[col, rows - 1] = BF(np.array([200.0], np.float32))[0]
    cfg = _cfg(temperature=1.0, top_k=1, seed=m["seed"])
    res = gpu_runner.run_accept(logits[None], [m["accept_drafts"]], [m["length"]], [[0] * 5], domain, [cfg])
    assert _flat(res) == m["accept_expected"]
    res = gpu_runner.run_accept(logits[None], [m["reject_drafts"]], [m["length"]], [[0] * 5], domain, [cfg])
    assert _flat(res) == m["reject_expected"]


@pytest.mark.parametrize("name", ["overlay_frequency", "overlay_presence", "overlay_frequency_real_shape"])
def test_overlay_penalties(gpu, name):
    m = KATS[name]
    vocab = m["vocab"]
    domain = m.get("token_domain", vocab)
    K = m["K"]
    logits = np.full((K + 1, vocab), BF(np.array([m["background"]], np.float32))[0], dtype=np.uint16)
    for col, tok, val in m["set"]:
        logits[col, tok] = BF(np.array([val], np.float32))[0]
    for seed in m["seeds"]:
        for L in m["lengths"]:
            cfg = _cfg(temperature=m["temperature"], top_k=m["top_k"], seed=seed,
                       presence=m.get("presence_penalty", 0.0), frequency=m.get("frequency_penalty", 0.0))
            res = gpu_runner.run_accept(logits[None], [m["drafts"]], [L], [[0] * (4 + K)], domain, [cfg])
            assert _flat(res) == m["expected"], f"seed={seed} L={L}"


# ---- randomized parity with the oracle ----------------------------------------------------------------

def _stochastic_batch(B, K, rows, domain, seed, temperature=0.7, top_p=0.95, top_k=0, min_p=0.0,
                      presence=0.0, frequency=0.0):
    logits = np.stack([syn.normal_bf16(syn.derive_seed(seed, 1, b), (K + 1) * rows, std=np.sqrt(3.0))
                       .reshape(K + 1, rows) for b in range(B)])
    # drafts: the column's argmax with probability ~0.8, else a seeded id
    drafts = np.zeros((B, K), dtype=np.int32)
    u = syn.uniforms(syn.derive_seed(seed, 2), B * K).reshape(B, K)
    alt = syn.int_uniform(syn.derive_seed(seed, 3), B * K, 0, domain).reshape(B, K)
    for b in range(B):
        for i in range(K):
            top = int(np.argmax(syn.bf16_bits_to_f32(logits[b, i, :domain])))
            drafts[b, i] = top if u[b, i] < 0.8 else alt[b, i]
    lengths = syn.int_uniform(syn.derive_seed(seed, 4), B, 1024, 32768).astype(np.int32)
    cfgs = [_cfg(temperature=temperature, top_k=top_k, top_p=top_p, min_p=min_p, presence=presence,
                 frequency=frequency, seed=syn.derive_seed(seed, 5, b) & 0xFFFFFFFFFFFF) for b in range(B)]
    return logits, drafts, lengths, cfgs


@pytest.mark.parametrize("seed,top_k,top_p,min_p", [(1, 0, 0.95, 0.0), (2, 5, 1.0, 0.0), (3, 0, 0.8, 0.05),
                                                    (4, 20, 0.95, 0.0)])
def test_stochastic_batch_matches_oracle(gpu, oracle, seed, top_k, top_p, min_p):
    B, K, rows, domain = 16, 3, 248320, 248320
    logits, drafts, lengths, cfgs = _stochastic_batch(B, K, rows, domain, seed, top_k=top_k, top_p=top_p,
                                                      min_p=min_p)
    stats = np.zeros((B, 4 + K), dtype=np.int64)
    res = gpu_runner.run_accept(logits, drafts, lengths, stats, domain, cfgs)
    for b in range(B):
        exp = oracle.speculative_accept(None, logits[b].reshape(-1), rows, drafts[b], int(lengths[b]), stats[b],
                                        domain, _ocfg(cfgs[b]))
        assert list(res["sampled_out"][b]) == list(exp["sampled_out"]), f"b={b}"
        assert res["num_sampled"][b] == exp["num_sampled"]
        assert res["accepted"][b] == exp["accepted"]
        assert res["token"][b] == exp["token"]
        assert res["length"][b] == exp["length"]
        assert list(res["stats"][b]) == list(exp["stats"])


@pytest.mark.parametrize("pattern", ["all_equal", "tie_at_max", "coarse_levels"])
def test_stochastic_ties_match_oracle(gpu, oracle, pattern):
    """Heavy ties: more than 64 keys share the top high word in a wave or a column, so the exact
    64-bit selection path of the candidate merge runs (ties order by token id)."""
    B, K, rows, domain = 4, 3, 248320, 248320
    rng = np.random.default_rng(77)
    if pattern == "all_equal":
        x = np.full((B, K + 1, rows), 1.5, np.float32)
    elif pattern == "tie_at_max":
        x = rng.standard_normal((B, K + 1, rows), dtype=np.float32) * 3.0
        for b in range(B):
            for c in range(K + 1):
                x[b, c, rng.choice(rows, 300, replace=False)] = 14.0
    else:
        x = np.round(rng.standard_normal((B, K + 1, rows), dtype=np.float32) * 1.5)
    logits = BF(x)
    drafts = np.zeros((B, K), np.int32)
    for b in range(B):
        for i in range(K):
            order = np.lexsort((np.arange(rows), -x[b, i]))
            drafts[b, i] = order[int(rng.integers(0, 30))]
    lengths = np.full(B, 4096, np.int32)
    cfgs = [_cfg(temperature=0.7, top_p=0.95, seed=1000 + b) for b in range(B)]
    stats = np.zeros((B, 4 + K), dtype=np.int64)
    res = gpu_runner.run_accept(logits, drafts, lengths, stats, domain, cfgs)
    for b in range(B):
        exp = oracle.speculative_accept(None, logits[b].reshape(-1), rows, drafts[b], int(lengths[b]), stats[b],
                                        domain, _ocfg(cfgs[b]))
        assert list(res["sampled_out"][b]) == list(exp["sampled_out"]), f"b={b}"
        assert res["accepted"][b] == exp["accepted"]
        assert list(res["stats"][b]) == list(exp["stats"])


def test_penalties_and_token_counts_match_oracle(gpu, oracle):
    B, K, rows, domain = 4, 4, 50000, 49999
    logits, drafts, lengths, cfgs = _stochastic_batch(B, K, rows, domain, 9, temperature=1.0, top_p=0.9,
                                                      presence=0.5, frequency=0.25)
    counts = [syn.int_uniform(syn.derive_seed(9, 7, b), domain, 0, 3).astype(np.int32) for b in range(B)]
    stats = np.zeros((B, 4 + K), dtype=np.int64)
    res = gpu_runner.run_accept(logits, drafts, lengths, stats, domain, cfgs, token_counts=counts)
    for b in range(B):
        exp = oracle.speculative_accept(None, logits[b].reshape(-1), rows, drafts[b], int(lengths[b]), stats[b],
                                        domain, _ocfg(cfgs[b]), token_counts=counts[b])
        assert list(res["sampled_out"][b]) == list(exp["sampled_out"]), f"b={b}"
        assert np.array_equal(res["token_counts"][b], exp["token_counts"])


def test_select_accepted_hidden(gpu):
    rows, cols = 5120, 4
    hidden = syn.normal_bf16(3, rows * cols).reshape(cols, rows)
    h = DeviceArray.from_numpy(na.BF16, hidden, (rows, cols))
    for a in range(cols):
        acc = DeviceArray.from_numpy(na.I32, np.array([a], dtype=np.int32), (1,))
        out = DeviceArray(na.BF16, (rows, 1))
        ops.speculative_select_accepted_hidden(h.tensor(), acc.tensor(), out.tensor())
        synchronize()
        assert np.array_equal(out.numpy(), hidden[a])


def test_mtp_alignment_ids(gpu, oracle):
    k = KATS["mtp_alignment"]
    cases = [(k["verify_ids"], k["token"], c["accepted"], k["initial"]) for c in k["cases"]]
    rng = np.random.default_rng(8)
    for T in range(2, 7):
        for acc in range(T):
            cases.append((rng.integers(0, 248320, T), int(rng.integers(0, 248320)), acc, rng.integers(-5, 0, T)))
    for verify, tok, acc, init in cases:
        T = len(verify)
        v = DeviceArray.from_numpy(na.I32, np.asarray(verify, np.int32), (T,))
        t = DeviceArray.from_numpy(na.I32, np.array([tok], np.int32), (1,))
        a = DeviceArray.from_numpy(na.I32, np.array([acc], np.int32), (1,))
        out = DeviceArray.from_numpy(na.I32, np.asarray(init, np.int32), (T,))
        ops.mtp_prepare_alignment_ids(v.tensor(), t.tensor(), a.tensor(), out.tensor())
        synchronize()
        assert list(out.numpy()) == list(oracle.mtp_prepare_alignment_ids(verify, tok, acc, init)), (T, acc)


def test_tree_accept_matches_oracle(gpu, oracle):
    B, N = 8, 16
    parents = np.array([[-1] + [(u - 1) // 2 for u in range(1, N)]] * B, dtype=np.int32)
    rng = np.random.default_rng(5)
    node_tokens = rng.integers(0, 6, size=(B, N)).astype(np.int32)
    target_tokens = rng.integers(0, 6, size=(B, N)).astype(np.int32)
    dev = {n: DeviceArray.from_numpy(na.I32, a, (N, B)) for n, a in
           [("p", parents), ("nt", node_tokens), ("tt", target_tokens)]}
    path = DeviceArray(na.I32, (N, B))
    plen = DeviceArray(na.I32, (B,))
    length = DeviceArray.from_numpy(na.I32, np.full(B, 1000, np.int32), (B,))
    token = DeviceArray(na.I32, (B,))
    so = DeviceArray(na.I32, (N, B))
    ns = DeviceArray(na.I32, (B,))
    acc = DeviceArray(na.I32, (B,))
    stats = DeviceArray.from_numpy(na.I64, np.zeros((B, 4 + N), np.int64), (4 + N, B))
    ops.tree_accept_greedy(dev["p"].tensor(), dev["nt"].tensor(), dev["tt"].tensor(), path.tensor(), plen.tensor(),
                           length.tensor(), token.tensor(), so.tensor(), ns.tensor(), acc.tensor(), stats.tensor())
    synchronize()
    P = path.numpy().reshape(B, N)
    L = plen.numpy()
    S = so.numpy().reshape(B, N)
    for b in range(B):
        exp = oracle.tree_longest_path(parents[b], node_tokens[b], target_tokens[b])
        assert list(P[b][: L[b]]) == list(exp)
        produced = [int(node_tokens[b][u]) for u in exp[1:]] + [int(target_tokens[b][exp[-1]])]
        assert list(S[b][: len(produced)]) == produced
        assert ns.numpy()[b] == len(exp) and acc.numpy()[b] == len(exp) - 1
        assert length.numpy()[b] == 1000 + len(exp)


@pytest.mark.parametrize("N", [1, 5, 16, 32])
def test_tree_accept_full_outputs(gpu, oracle, N):
    """Every output of the greedy tree acceptance against the oracle's longest accepted path: the
    path and the sampled tokens zero-padded to N, token, counts, length, and the statistics row
    ([0] += N - 1 drafted nodes, [1] += accepted, [2] += 1 round, [4 + j] += 1 for j < accepted,
    other entries unchanged) with a stride wider than 4 + N and nonzero starting values. Random
    parents include malformed ones (negative, or not below the node), which the contract treats as
    rejected."""
    B, stride = 4, 4 + N + 3
    rng = np.random.default_rng(100 + N)
    parents = np.full((B, N), -1, np.int32)
    for b in range(B):
        for u in range(1, N):
            r = rng.random()
            parents[b, u] = rng.integers(0, u) if r < 0.8 else (u + rng.integers(0, 3) if r < 0.9 else -2)
    node_tokens = rng.integers(0, 3, size=(B, N)).astype(np.int32)
    target_tokens = rng.integers(0, 3, size=(B, N)).astype(np.int32)
    stats0 = rng.integers(0, 50, size=(B, stride)).astype(np.int64)
    dev = {n: DeviceArray.from_numpy(na.I32, a, (N, B)) for n, a in
           [("p", parents), ("nt", node_tokens), ("tt", target_tokens)]}
    path = DeviceArray.from_numpy(na.I32, np.full((B, N), 77, np.int32), (N, B))
    so = DeviceArray.from_numpy(na.I32, np.full((B, N), 77, np.int32), (N, B))
    plen, token, ns, acc = (DeviceArray(na.I32, (B,)) for _ in range(4))
    length = DeviceArray.from_numpy(na.I32, np.arange(B, dtype=np.int32) * 10 + 500, (B,))
    stats = DeviceArray.from_numpy(na.I64, stats0, (stride, B))
    ops.tree_accept_greedy(dev["p"].tensor(), dev["nt"].tensor(), dev["tt"].tensor(), path.tensor(), plen.tensor(),
                           length.tensor(), token.tensor(), so.tensor(), ns.tensor(), acc.tensor(), stats.tensor())
    synchronize()
    P, S, ST = path.numpy().reshape(B, N), so.numpy().reshape(B, N), stats.numpy().reshape(B, stride)
    for b in range(B):
        exp = list(oracle.tree_longest_path(parents[b], node_tokens[b], target_tokens[b]))
        a = len(exp) - 1
        assert list(P[b]) == exp + [0] * (N - len(exp)), b
        produced = [int(node_tokens[b][u]) for u in exp[1:]] + [int(target_tokens[b][exp[-1]])]
        assert list(S[b]) == produced + [0] * (N - len(produced)), b
        assert plen.numpy()[b] == len(exp) and ns.numpy()[b] == a + 1 and acc.numpy()[b] == a
        assert token.numpy()[b] == target_tokens[b][exp[-1]]
        assert length.numpy()[b] == 500 + 10 * b + a + 1
        want = stats0[b].copy()
        want[0] += N - 1
        want[1] += a
        want[2] += 1
        want[4:4 + a] += 1
        assert list(ST[b]) == list(want), b
