"""GPU parity of the general speculative acceptance ("Mode F", an extension with no reference
symbol): full-vocabulary temperature + top-p, min(1, p/q) acceptance and normalized max(0, p - q)
resampling with supplied uniforms. Every decision and token must equal the CPU oracle's
(orc_general_accept), whose own correctness is pinned by invariants in test_oracle_golden.py."""
import numpy as np
import pytest

from ninfer_amd import synthetic as syn

import gpu_runner

pytestmark = pytest.mark.gpu


def _cfg(oracle, t, p):
    c = oracle.GeneralConfig()
    c.temperature, c.top_p = t, p
    return c


def _check(oracle, target, draft, drafts, ua, ur, lengths, V, t, p):
    B, Kp1, rows = target.shape
    K = Kp1 - 1
    stats = np.zeros((B, 4 + K), np.int64)
    got = gpu_runner.run_general(target, draft, drafts, ua, ur, lengths, stats, V, t, p)
    for b in range(B):
        exp = oracle.general_accept(target[b].ravel(), draft[b].ravel(), rows, drafts[b], int(lengths[b]),
                                    stats[b], V, _cfg(oracle, t, p), ua[b], float(ur[b]))
        assert list(got["sampled_out"][b]) == list(exp["sampled_out"]), (b, got["sampled_out"][b], exp)
        assert got["num_sampled"][b] == exp["num_sampled"] and got["accepted"][b] == exp["accepted"]
        assert got["token"][b] == exp["token"] and got["length"][b] == exp["length"]
        assert list(got["stats"][b]) == list(exp["stats"])
    return got


def _case(seed, B, K, rows, corr=0.9, std=np.sqrt(3.0)):
    t = syn.normal_bf16(seed, B * (K + 1) * rows, std).reshape(B, K + 1, rows)
    tf = syn.bf16_bits_to_f32(t[:, :K, :])
    z = syn.bf16_bits_to_f32(syn.normal_bf16(seed + 1, B * K * rows, std)).reshape(B, K, rows)
    d = syn.f32_to_bf16_bits((corr * tf + np.sqrt(1 - corr * corr) * z).astype(np.float32))
    u = syn.uniforms(seed + 2, B * (K + 3)).reshape(B, K + 3)
    # drafts: the draft column's argmax or a seeded token, alternately
    dr = np.zeros((B, K), np.int32)
    for b in range(B):
        for i in range(K):
            dr[b, i] = int(np.argmax(syn.bf16_bits_to_f32(d[b, i]))) if (b + i) % 2 == 0 else int(u[b, K + 2] * rows) % rows
    return t, d, dr, u[:, :K + 1].astype(np.float32), u[:, K + 1].astype(np.float32)


@pytest.mark.parametrize("seed,B,K,rows,temp,top_p", [
    (1, 4, 3, 5000, 0.7, 0.95),
    (2, 3, 1, 3001, 1.0, 1.0),
    (3, 2, 4, 8192, 0.5, 0.5),
    (4, 5, 2, 4097, 1.3, 0.99),
    (5, 2, 3, 248320, 0.7, 0.95),
])
def test_general_matches_oracle(gpu, oracle, seed, B, K, rows, temp, top_p):
    t, d, dr, ua, ur = _case(seed, B, K, rows)
    _check(oracle, t, d, dr, ua, ur, np.arange(B, dtype=np.int32) * 100 + 7, rows, temp, top_p)


def test_general_ties_rank_cut(gpu, oracle):
    """Many equal values: the nucleus cut falls inside a run of equal logits (ids ascending)."""
    B, K, rows = 3, 2, 9000
    rng = np.random.default_rng(7)
    vals = np.array([0.0, 0.5, 1.0, -1.0], np.float32)
    t = syn.f32_to_bf16_bits(vals[rng.integers(0, 4, B * (K + 1) * rows)]).reshape(B, K + 1, rows)
    d = syn.f32_to_bf16_bits(vals[rng.integers(0, 4, B * K * rows)]).reshape(B, K, rows)
    dr = rng.integers(0, rows, (B, K)).astype(np.int32)
    u = syn.uniforms(8, B * (K + 2)).reshape(B, K + 2).astype(np.float32)
    for top_p in (0.3, 0.77, 1.0):
        _check(oracle, t, d, dr, u[:, :K + 1], u[:, K + 1], np.full(B, 50, np.int32), rows, 1.0, top_p)


def test_general_q_equals_p_accepts_all(gpu, oracle):
    """q = p accepts every draft q can emit (here: each column's top token, inside the nucleus)."""
    B, K, rows = 4, 3, 6000
    t, _, _, ua, ur = _case(11, B, K, rows)
    dr = np.array([[int(np.argmax(syn.bf16_bits_to_f32(t[b, i]))) for i in range(K)] for b in range(B)], np.int32)
    got = _check(oracle, t, t[:, :K, :].copy(), dr, ua, ur, np.full(B, 9, np.int32), rows, 0.8, 0.9)
    assert (got["accepted"] == K).all()


def test_general_out_of_domain_draft_is_rejected(gpu, oracle):
    B, K, rows = 1, 2, 5000
    t, d, dr, ua, ur = _case(12, B, K, rows)
    dr[0, 0] = rows + 5  # outside the token domain (inside the physical rows below)
    tt = np.concatenate([t, np.zeros((B, K + 1, 16), np.uint16)], axis=2)
    dd = np.concatenate([d, np.zeros((B, K, 16), np.uint16)], axis=2)
    stats = np.zeros((B, 4 + K), np.int64)
    got = gpu_runner.run_general(tt, dd, dr, ua, ur, [3], stats, rows, 0.7, 0.95)
    assert got["accepted"][0] == 0 and got["num_sampled"][0] == 1
    assert 0 <= got["sampled_out"][0][0] < rows


def test_general_c4_shape(gpu, oracle):
    """configs[3] shape: batch 16, vocab 248,320, draft logits correlated 0.9 with the target,
    temperature 0.7, top-p 0.95, seeded uniforms supplied as input."""
    B, K, rows = 16, 3, 248320
    t, d, dr, ua, ur = _case(40, B, K, rows)
    _check(oracle, t, d, dr, ua, ur, np.arange(B, dtype=np.int32) * 1000 + 1024, rows, 0.7, 0.95)


@pytest.mark.parametrize("top_p", [0.95, 1.0])
def test_general_saturated_histogram(gpu, oracle, top_p):
    """Columns whose tokens sit at the column maximum: in every tile, each replica word of the
    coarse histogram then counts 256 tokens of the largest weight (2^40, or slightly more when
    fma(x, 1/T, -x/T) rounds above zero at T = 0.7), the load its packed count and mass fields are
    sized for; with top-p below 1 the nucleus cut falls inside a run of equal values. Sequence 0:
    every token equal; sequence 1: the even ids at the maximum, the odd ids below it."""
    B, K, rows = 2, 3, 248320
    rng = np.random.default_rng(21)
    t = np.empty((B, K + 1, rows), np.uint16)
    d = np.empty((B, K, rows), np.uint16)
    t[0] = syn.f32_to_bf16_bits(np.full(rows, 3.0, np.float32))
    d[0] = syn.f32_to_bf16_bits(np.full(rows, 2.5, np.float32))
    for c in range(K + 1):
        col = np.full(rows, -1.75, np.float32)
        col[1::2] = -1.75 - np.abs(rng.normal(0.0, 3.0, rows // 2)).astype(np.float32) - 0.125
        t[1, c] = syn.f32_to_bf16_bits(col)
    for c in range(K):
        col = np.full(rows, 0.625, np.float32)
        col[1::2] = 0.5 - np.abs(rng.normal(0.0, 2.0, rows // 2)).astype(np.float32)
        d[1, c] = syn.f32_to_bf16_bits(col)
    dr = rng.integers(0, rows, (B, K)).astype(np.int32)
    u = syn.uniforms(22, B * (K + 2)).reshape(B, K + 2).astype(np.float32)
    _check(oracle, t, d, dr, u[:, :K + 1], u[:, K + 1], np.array([5, 6], np.int32), rows, 0.7, top_p)
