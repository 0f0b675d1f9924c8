"""Pin the CPU oracle (test infrastructure) before trusting it as the checker.

Each function of oracle/oracle.cpp is checked against the reference's own known answers
(tests/golden/reference_kats.json), published algorithm vectors, closed forms, or an independent
brute-force restatement chosen so that a plausible mistake (dropped term, wrong sign, transposed
operand, off-by-one position) fails."""
import json
import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from ninfer_amd import synthetic as syn

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
BF = syn.f32_to_bf16_bits


def _cfg(oracle, temperature=0.0, top_k=0, top_p=1.0, min_p=0.0, presence=0.0, frequency=0.0, seed=0):
    c = oracle.SamplingConfig()
    c.temperature, c.top_k, c.top_p, c.min_p = temperature, top_k, top_p, min_p
    c.presence_penalty, c.frequency_penalty, c.seed = presence, frequency, seed
    return c


# ---- scalar numerics -------------------------------------------------------------------------------

def test_splitmix64_published_vectors(oracle):
    m = KATS["splitmix64"]
    assert oracle.splitmix64(0) == int(m["state0_first"], 16)
    G, M = 0x9E3779B97F4A7C15, (1 << 64) - 1
    assert [oracle.splitmix64((1234567 + i * G) & M) for i in range(5)] == [int(x) for x in m["seed1234567"]]


def test_sampling_uniform_closed_form(oracle):
    """u = (k >> 40) * 2^-24 with the two-round key of sampling_device.cuh:62-73, recomputed here."""
    M = (1 << 64) - 1

    def sm(x):
        x = (x + 0x9E3779B97F4A7C15) & M
        x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M
        x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M
        return x ^ (x >> 31)

    for seed, pos, purpose in [(0, 0, 0), (20260716, 101, 2), (1234, 11, 4), (M, 2**31 - 1, 3), (7, -5, 2)]:
        k = sm(seed ^ (((pos & 0xFFFFFFFF) * 0xD1B54A32D192ED03) & M))
        k = sm(k ^ ((purpose & 0xFFFFFFFF) << 21) ^ 0)
        assert oracle.sampling_uniform(seed, pos, purpose) == (k >> 40) / 16777216.0


def test_f16_conversion_matches_ieee(oracle):
    vals = np.concatenate([
        syn.normals(1, 4000) * 10.0,
        syn.normals(2, 2000) * 1e-5,                       # subnormal half range
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, 5.960464477539063e-08, 2.98e-8, 2.99e-8]),
        np.ldexp(1.0 + syn.uniforms(3, 2000), syn.int_uniform(4, 2000, -26, 16)),
    ]).astype(np.float32)
    got = np.array([oracle.f32_to_f16_bits(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, vals.astype(np.float16).view(np.uint16))


def test_det_expf_accuracy(oracle):
    xs = np.concatenate([np.linspace(-103.9, 88.7, 20001), syn.normals(5, 5000) * 4.0]).astype(np.float32)
    worst = 0.0
    for x in xs:
        got = oracle.det_expf(float(x))
        ref = math.exp(float(x))
        if ref < 1.2e-38:
            assert abs(got - ref) <= 2 ** -149 * 2
            continue
        ulp = np.spacing(np.float32(ref))
        worst = max(worst, abs(got - ref) / float(ulp))
    assert worst <= 1.0, worst
    assert oracle.det_expf(0.0) == 1.0
    assert oracle.det_expf(-200.0) == 0.0


# ---- INT8-G64 codec --------------------------------------------------------------------------------

def _codec_brute(x_bf16):
    """gqa_attention.h:25-30 restated with numpy's IEEE conversions."""
    x = syn.bf16_bits_to_f32(x_bf16)
    a = np.float32(np.abs(x).max())
    s16 = np.float16(np.float32(a / np.float32(127.0)) if a > 0 else np.float32(0))
    s = np.float32(s16)
    if s == 0:
        return np.zeros(x.size, np.int8), int(s16.view(np.uint16))
    inv = np.float32(np.float32(1.0) / s)
    prod = (x * inv).astype(np.float32)
    return np.clip(np.rint(prod), -127, 127).astype(np.int8), int(s16.view(np.uint16))


def test_codec_matches_header_contract(oracle):
    for seed in range(200):
        x = syn.normal_bf16_with_outliers(seed, 64) if seed % 3 == 0 else syn.normal_bf16(seed, 64, 0.5 + seed)
        codes, scale = oracle.quantize_group(x)
        bc, bs = _codec_brute(x)
        assert scale == bs
        assert np.array_equal(codes, bc)


def test_codec_special_cases(oracle):
    zeros = np.zeros(64, np.uint16)
    codes, scale = oracle.quantize_group(zeros)
    assert scale == 0 and not codes.any()
    x = syn.normal_bf16(9, 64)
    x[7] = BF(np.array([20.0], np.float32))[0]
    x[9] = BF(np.array([-20.0], np.float32))[0]
    codes, scale = oracle.quantize_group(x)
    assert scale == int(np.float16(np.float32(20.0) / np.float32(127.0)).view(np.uint16))
    assert codes[7] == 127 and codes[9] == -127
    # a group whose absmax/127 underflows FP16 to zero encodes as all zeros
    tiny = BF(np.full(64, 1e-10, np.float32))
    codes, scale = oracle.quantize_group(tiny)
    assert scale == 0 and not codes.any()


def test_codec_tie_follows_header_form(oracle):
    """The header encodes RNE(x * FP32(1/s)) (include/ninfer/ops/gqa_attention.h:28-29) while the
    reference's CPU test and PyTorch restatement divide, RNE(x / s)
    (tests/ops/test_gqa_attention.cpp:350-374, tools/reference/qwen3_6_27b/state.py:43-49). The
    fixture (tests/golden/make_codec_tie.py) is a BF16 group where the two disagree; the oracle
    follows the header."""
    fx = json.loads((Path(__file__).parent / "golden" / "codec_tie.json").read_text())
    codes, scale = oracle.quantize_group(np.array(fx["group_bf16"], np.uint16))
    assert scale == fx["scale_bits"]
    assert codes[fx["element"]] == fx["code_header_form"] != fx["code_division_form"]
    bc, bs = _codec_brute(np.array(fx["group_bf16"], np.uint16))
    assert np.array_equal(codes, bc) and bs == scale


# ---- attention -------------------------------------------------------------------------------------

def _numpy_attention(q, kd, vd, visible, scale):
    """Independent vectorized restatement: softmax(q K^T * scale) V over visible keys."""
    s = (q @ kd.T) * scale
    s = np.where(visible, s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    return (p / p.sum(axis=-1, keepdims=True)) @ vd


def _decode(codes, scales, D):
    c = codes.astype(np.float32).reshape(codes.shape[0], D // 64, 64)
    s = syn.bf16_bits_to_f32(np.zeros(1, np.uint16))  # placeholder for dtype
    sc = np.array(scales, dtype=np.uint16).view(np.float16).astype(np.float32).reshape(codes.shape[0], D // 64, 1)
    return (c * sc).reshape(codes.shape[0], D).astype(np.float64)


@pytest.mark.parametrize("tree", [False, True])
def test_attention_vs_numpy_restatement(oracle, tree):
    from helpers import AttnCase
    T, Hq, Hkv, D = 5, 6, 2, 128
    parents = np.array([-1, 0, 0, 1, 2], dtype=np.int32) if tree else None
    case = AttnCase([37], T=T, Hq=Hq, Hkv=Hkv, D=D, seed=3, parents=parents)
    (kc, vc, ks, vs), out = case.oracle_after_append()
    L = 37
    out = out.reshape(T, Hq, D)
    q = syn.bf16_bits_to_f32(case.q).astype(np.float64).reshape(T, Hq, D)
    G = Hq // Hkv
    for h in range(Hkv):
        kd = _decode(kc[0, h, : L + T], ks[0, h, : L + T], D)
        vd = _decode(vc[0, h, : L + T], vs[0, h, : L + T], D)
        for t in range(T):
            anc = set()
            u = t
            while u >= 0:
                anc.add(u)
                u = (parents[u] if tree else u - 1)
            vis = np.array([j < L or (j - L) in anc for j in range(L + T)])
            for g in range(G):
                ref = _numpy_attention(q[t, h * G + g], kd, vd, vis, case.scale)
                np.testing.assert_allclose(out[t, h * G + g], ref, rtol=1e-9, atol=1e-12)


def test_attention_single_key_returns_value_row(oracle):
    from helpers import AttnCase
    case = AttnCase([0], T=1, Hq=4, Hkv=2, D=128, seed=4)
    (kc, vc, ks, vs), out = case.oracle_after_append()
    for qh in range(4):
        h = qh // 2
        v = _decode(vc[0, h, :1], vs[0, h, :1], 128)[0]
        np.testing.assert_allclose(out[qh * 128:(qh + 1) * 128], v, rtol=0, atol=1e-15)


def test_chain_tree_equals_causal_oracle(oracle):
    from helpers import AttnCase
    par = np.array([-1, 0, 1, 2], dtype=np.int32)
    a = AttnCase([50], T=4, Hq=8, Hkv=2, seed=5, parents=par).oracle_after_append()[1]
    b = AttnCase([50], T=4, Hq=8, Hkv=2, seed=5).oracle_after_append()[1]
    assert np.array_equal(a, b)


@pytest.mark.parametrize("tree", [False, True])
def test_attention_bf16_equals_int8_oracle_on_exact_values(oracle, tree):
    """With power-of-two FP16 scales every decoded INT8 value code * 2^e is exact in BF16, so the
    BF16-cache oracle over those values must return the pinned INT8 oracle's output bit for bit
    (checks its row decode, plane indexing and visibility against the INT8 path)."""
    from helpers import AttnCase
    T, Hq, Hkv, D = 5, 8, 2, 128
    # parents [T, B]: one tree per sequence
    parents = np.array([-1, 0, 0, 1, 2, -1, 0, 1, 1, 3], dtype=np.int32) if tree else None
    case = AttnCase([0, 41], T=T, Hq=Hq, Hkv=Hkv, D=D, seed=8, parents=parents)
    (kc, vc, ks, vs), _ = case.oracle_after_append()
    rng = np.random.default_rng(8)
    exps = rng.integers(-9, -2, size=ks.shape)
    ks2 = ((exps + 15) << 10).astype(np.uint16)
    vs2 = ((rng.integers(-9, -2, size=vs.shape) + 15) << 10).astype(np.uint16)
    out_i8 = oracle.attention(case.q, kc, vc, ks2, vs2, case.positions, parents, T, case.B, Hq, Hkv, D,
                              case.P, case.scale)
    kval = kc.astype(np.float32).reshape(*kc.shape[:3], D // 64, 64) * \
        ks2.view(np.float16).astype(np.float32)[..., None]
    vval = vc.astype(np.float32).reshape(*vc.shape[:3], D // 64, 64) * \
        vs2.view(np.float16).astype(np.float32)[..., None]
    kb = syn.f32_to_bf16_bits(kval.reshape(kc.shape))
    vb = syn.f32_to_bf16_bits(vval.reshape(vc.shape))
    assert np.array_equal(syn.bf16_bits_to_f32(kb), kval.reshape(kc.shape))  # exact in BF16
    out_bf = oracle.attention_bf16(case.q, kb, vb, case.positions, parents, T, case.B, Hq, Hkv, D, case.P,
                                   case.scale)
    assert np.array_equal(out_i8, out_bf)


def test_attention_bf16_case_vs_numpy_restatement(oracle):
    """BF16 case: the new rows land at their positions, rows past them keep the marker, and the
    output equals an independent numpy softmax over the stored values."""
    from helpers import AttnCase
    T, Hq, Hkv, D, L = 4, 6, 2, 256, 29
    case = AttnCase([L], T=T, Hq=Hq, Hkv=Hkv, D=D, seed=9, kv="bf16", dist="uniform")
    (kb, vb), out = case.oracle_after_append()
    kn = case.k_new.reshape(T, Hkv, D)
    assert np.array_equal(kb[0, :, L:L + T], kn.transpose(1, 0, 2))
    assert np.all(kb[0, :, L + T:] == 0x7F80) and np.all(vb[0, :, L + T:] == 0x7F80)
    q = syn.bf16_bits_to_f32(case.q).astype(np.float64).reshape(T, Hq, D)
    out = out.reshape(T, Hq, D)
    G = Hq // Hkv
    for h in range(Hkv):
        kd = syn.bf16_bits_to_f32(kb[0, h, :L + T]).astype(np.float64)
        vd = syn.bf16_bits_to_f32(vb[0, h, :L + T]).astype(np.float64)
        for t in range(T):
            vis = np.arange(L + T) <= L + t
            for g in range(G):
                ref = _numpy_attention(q[t, h * G + g], kd, vd, vis, case.scale)
                np.testing.assert_allclose(out[t, h * G + g], ref, rtol=1e-9, atol=1e-12)


def test_attention_bf16_stress_closed_form(oracle):
    """The reference's stress decode (tests/ops/test_gqa_attention.cpp:772-777): Q = K_new = 8,
    history K = -8. The new row's score exceeds every history score by 128 sqrt(D), so the output
    is the new V row exactly."""
    from helpers import AttnCase
    D, Hq, Hkv, L = 256, 24, 4, 17
    case = AttnCase([L], T=1, Hq=Hq, Hkv=Hkv, D=D, seed=31, kv="bf16")
    eight = syn.f32_to_bf16_bits(np.array([8.0], np.float32))[0]
    case.q[:] = eight
    case.k_new[:] = eight
    case.kb[0, :, :L] = syn.f32_to_bf16_bits(np.array([-8.0], np.float32))[0]
    case.v_new[:] = syn.uniform_bf16(32, case.v_new.size, -8.0, 8.0)
    case.vb[0, :, :L] = syn.uniform_bf16(33, Hkv * L * D, -8.0, 8.0).reshape(Hkv, L, D)
    _, out = case.oracle_after_append()
    vn = syn.bf16_bits_to_f32(case.v_new).astype(np.float64).reshape(Hkv, D)
    expect = np.repeat(vn, Hq // Hkv, axis=0).ravel()
    assert np.array_equal(out, expect)


# ---- lm_head: Q6G64_F16S RowSplit linear ---------------------------------------------------------

def test_q6_packer_known_bytes():
    """One group holding codes -32 .. 31 in order: by the packer's definition
    (tests/ops/row_split_pack.h:143-172) code i = i - 32 has u = i ^ 32, so byte j of the nibble plane
    is (u(2j) & 15) | (u(2j+1) & 15) << 4 and each high byte packs four 2-bit fields: codes -32..-17
    give 0xAA, -16..-1 give 0xFF, 0..15 give 0x00, 16..31 give 0x55."""
    import q6_pack as qp
    codes = np.arange(-32, 32).reshape(1, 64)
    nib, high = qp.pack_codes(codes)
    u = np.arange(64) ^ 32
    assert np.array_equal(nib[0, 0], ((u[0::2] & 15) | ((u[1::2] & 15) << 4)).astype(np.uint8))
    assert np.array_equal(high[0, 0], np.array([0xAA] * 4 + [0xFF] * 4 + [0x00] * 4 + [0x55] * 4, np.uint8))
    assert np.array_equal(qp.unpack_codes(nib, high), codes)


def test_q6_patterned_generator_known_values():
    """make_patterned_weight (tests/ops/row_split_pack.h:228-285) by hand: row 3 (mix 3), group 2,
    seed 4226: nibble byte b = (3*37 + 2*29 + 17b + 4226) & 255 = 43 + 17b, high byte b =
    (3*43 + 2*31 + 13b + 3*4226) & 255; scale index (3 ^ 2 ^ 4226) & 3 = 3 -> 0x3d00."""
    import q6_pack as qp
    nib, high, sc = qp.patterned(8, 300, 4226)
    assert list(nib[3, 2, :3]) == [43, 60, 77]
    assert high[3, 2, 1] == (3 * 43 + 2 * 31 + 13 + 3 * 4226) & 255
    assert sc[3, 2] == 0x3D00
    nib2, _, _ = qp.patterned(301, 64, 7)  # row 300: mix = 300 ^ (300 >> 8) = 301
    assert nib2[300, 0, 0] == ((300 ^ 1) * 37 + 7) & 255


def test_linear_q6_oracle_unit_columns(oracle):
    """x = unit columns e_{k_t}: out[t, n] is exactly code[n, k_t] * scale[n, k_t / 64] (pins the
    oracle's decode of every nibble and high-bit position against the packer)."""
    import q6_pack as qp
    rng = np.random.default_rng(12)
    N, K = 37, 200
    Kp = qp.align_up(K, 128)
    codes = rng.integers(-32, 32, (N, Kp))
    nib, high = qp.pack_codes(codes)
    sc = np.float16(rng.uniform(0.01, 2.0, (N, Kp // 64))).view(np.uint16)
    ks = np.arange(K)
    T = K
    x = np.zeros((T, K), np.uint16)
    x[np.arange(T), ks] = 0x3F80  # BF16 1.0
    out = oracle.linear_q6(nib, high, sc, N, K, x, T)
    expect = codes[:, ks].T * sc.view(np.float16).astype(np.float64)[:, ks // 64].T
    assert np.array_equal(out, expect)


def test_linear_q6_oracle_vs_numpy(oracle):
    import q6_pack as qp
    rng = np.random.default_rng(13)
    N, K, T = 50, 384, 3
    nib, high, sc = qp.patterned(N, K, 99)
    codes = qp.unpack_codes(nib, high)[:, :K].astype(np.float64)
    w = codes * np.repeat(sc.view(np.float16).astype(np.float64), 64, axis=1)[:, :K]
    x = syn.f32_to_bf16_bits(rng.uniform(-1, 1, (T, K)).astype(np.float32))
    out = oracle.linear_q6(nib, high, sc, N, K, x, T)
    np.testing.assert_allclose(out, (w @ syn.bf16_bits_to_f32(x).astype(np.float64).T).T, rtol=1e-12, atol=1e-12)


# ---- recurrent state (Gated DeltaNet, causal conv1d) ----------------------------------------------

def _bf(x):
    return syn.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


def _gdn_numpy(q, k, v, g, beta, state, normalize):
    """Independent vectorized restatement over all heads: q/k [T,Hqk,S], v [T,Hv,S], g/beta [T,Hv],
    state [Hv,S,S] (row = value index)."""
    T, Hv, S = v.shape
    Hqk = q.shape[1]
    if normalize:
        q = (q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6)).astype(np.float32).astype(np.float64)
        k = (k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)).astype(np.float32).astype(np.float64)
    St = state.astype(np.float64).copy()
    rep = Hv // Hqk
    outs, snaps = [], []
    for t in range(T):
        kt = np.repeat(k[t], rep, axis=0)  # [Hv,S]
        qt = np.repeat(q[t], rep, axis=0)
        St = St * np.exp(g[t].astype(np.float64))[:, None, None]
        delta = beta[t][:, None] * (v[t] - np.einsum("hrc,hc->hr", St, kt))
        St = St + delta[:, :, None] * kt[:, None, :]
        outs.append(np.einsum("hrc,hc->hr", St, qt) / np.sqrt(S))
        snaps.append(St.copy())
    return np.stack(outs), St, np.stack(snaps)


def _gdn_inputs(seed, S, Hqk, Hv, T, raw=False):
    rng = np.random.default_rng(seed)
    q = rng.uniform(-1, 1, (T, Hqk, S)).astype(np.float32)
    k = rng.uniform(-1, 1, (T, Hqk, S)).astype(np.float32)
    if not raw:
        q /= np.linalg.norm(q, axis=-1, keepdims=True)
        k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.uniform(-1, 1, (T, Hv, S)).astype(np.float32)
    g = rng.uniform(-4, 0, (T, Hv)).astype(np.float32)
    beta = rng.uniform(0.05, 0.95, (T, Hv)).astype(np.float32)
    state = rng.uniform(-0.1, 0.1, (Hv, S, S)).astype(np.float32)
    return _bf(q), _bf(k), _bf(v), g, beta, state


@pytest.mark.parametrize("normalize", [False, True])
def test_gdn_oracle_vs_numpy_restatement(oracle, normalize):
    S, Hqk, Hv, T = 32, 2, 6, 5
    q, k, v, g, beta, state = _gdn_inputs(21, S, Hqk, Hv, T, raw=normalize)
    out, st, snaps = oracle.gdn_recurrent(q, k, v, g, beta, state, S, Hqk, Hv, T, normalize, snapshots=True)
    f = lambda a: syn.bf16_bits_to_f32(a).astype(np.float64)  # noqa: E731
    ro, rst, rsn = _gdn_numpy(f(q), f(k), f(v), g, beta, state, normalize)
    np.testing.assert_allclose(out, ro, rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(st, rst, rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(snaps, rsn, rtol=1e-10, atol=1e-13)


def test_gdn_unit_key_writes_value_column(oracle):
    """k = e_j, beta = 1: delta = v - alpha S e_j, so the new state's column j is v exactly and the
    other columns are alpha S (a wrong row/column index or a misplaced alpha breaks this)."""
    S, Hqk, Hv, j = 16, 1, 2, 5
    q, _, v, _, _, state = _gdn_inputs(22, S, Hqk, Hv, 1)
    k = np.zeros((1, Hqk, S), np.float32)
    k[0, 0, j] = 1.0
    g = np.full((1, Hv), -0.75, np.float32)
    beta = np.ones((1, Hv), np.float32)
    out, st, _ = oracle.gdn_recurrent(q, _bf(k), v, g, beta, state, S, Hqk, Hv, 1)
    alpha = np.exp(np.float64(-0.75))
    vf = syn.bf16_bits_to_f32(v).astype(np.float64).reshape(Hv, S)
    np.testing.assert_allclose(st[:, :, j], vf, rtol=0, atol=1e-15)
    others = [c for c in range(S) if c != j]
    np.testing.assert_allclose(st[:, :, others], alpha * state[:, :, others].astype(np.float64), rtol=1e-15, atol=0)
    qf = syn.bf16_bits_to_f32(q).astype(np.float64).reshape(S)
    np.testing.assert_allclose(out[0], st @ qf / 4.0, rtol=1e-14, atol=1e-16)


def test_gdn_zero_beta_is_pure_decay(oracle):
    """beta = 0: the state only decays, S_T = exp(sum g) S_0, and out_t = scale S_t q_t."""
    S, Hqk, Hv, T = 16, 2, 4, 3
    q, k, v, g, _, state = _gdn_inputs(23, S, Hqk, Hv, T)
    beta = np.zeros((T, Hv), np.float32)
    out, st, snaps = oracle.gdn_recurrent(q, k, v, g, beta, state, S, Hqk, Hv, T, snapshots=True)
    decay = np.exp(np.cumsum(g.astype(np.float64), axis=0))  # [T,Hv]
    for t in range(T):
        np.testing.assert_allclose(snaps[t], decay[t][:, None, None] * state, rtol=1e-13)


def _conv_numpy(x, w, st):
    """x [T,C], w [4,C], st [3,C] as floats."""
    u = np.concatenate([st, x], axis=0)
    T = x.shape[0]
    acc = sum(w[j][None, :] * u[j:j + T] for j in range(4))
    return acc / (1.0 + np.exp(-acc)), np.stack([u[t + 1:t + 4] for t in range(T)])


def test_conv_oracle_vs_numpy_and_windows(oracle):
    C, T = 37, 6
    rng = np.random.default_rng(5)
    x, w, st = _bf(rng.uniform(-2, 2, (T, C))), _bf(rng.uniform(-1, 1, (4, C))), _bf(rng.uniform(-2, 2, (3, C)))
    out, win = oracle.causal_conv1d_silu(x, w, st, C, T)
    f = lambda a: syn.bf16_bits_to_f32(a).astype(np.float64)  # noqa: E731
    ro, rw = _conv_numpy(f(x), f(w), f(st))
    np.testing.assert_allclose(out, ro, rtol=1e-13, atol=1e-15)
    u = np.concatenate([st, x], axis=0)
    for t in range(T):
        assert np.array_equal(win[t], u[t + 1:t + 4])  # window after token t: u[t-2], u[t-1], u[t]


@pytest.mark.parametrize("tap", [0, 3])
def test_conv_one_hot_tap(oracle, tap):
    """weight = e_tap: out[t] = SiLU(u[t - 3 + tap]) (tap 3 reads x[t], tap 0 reads the state for t < 3)."""
    C, T = 8, 5
    rng = np.random.default_rng(6)
    x, st = _bf(rng.uniform(-3, 3, (T, C))), _bf(rng.uniform(-3, 3, (3, C)))
    w = np.zeros((4, C), np.float32)
    w[tap] = 1.0
    out, _ = oracle.causal_conv1d_silu(x, _bf(w), st, C, T)
    u = syn.bf16_bits_to_f32(np.concatenate([st, x], axis=0)).astype(np.float64)
    a = u[tap:tap + T]
    np.testing.assert_allclose(out, a / (1.0 + np.exp(-a)), rtol=1e-15, atol=0)


# ---- argmax ---------------------------------------------------------------------------------------

def test_argmax_brute_force(oracle):
    rows, C, valid = 1000, 3, 977
    x = syn.normal_bf16(11, rows * C).reshape(C, rows)
    x[0, 5] = x[0, 700] = BF(np.array([9.0], np.float32))[0]
    x[1, 990] = BF(np.array([99.0], np.float32))[0]
    got = oracle.argmax(x.reshape(-1), rows, C, valid)
    for c in range(C):
        f = syn.bf16_bits_to_f32(x[c, :valid])
        assert got[c] == int(np.flatnonzero(f == f.max())[0])
    assert got[0] == 5


# ---- speculative acceptance (Mode R) --------------------------------------------------------------

def test_prepare_verify_kat(oracle):
    k = KATS["prepare_verify"]
    ids, pos = oracle.prepare_verify_inputs(k["token"], k["drafts"], k["length"])
    assert list(ids) == k["verify_ids"] and list(pos) == k["positions"]


def test_mtp_alignment_kat(oracle):
    k = KATS["mtp_alignment"]
    for case in k["cases"]:
        got = oracle.mtp_prepare_alignment_ids(k["verify_ids"], k["token"], case["accepted"], k["initial"])
        assert list(got) == case["alignment_ids"]


@pytest.mark.parametrize("idx", range(4))
def test_greedy_kats(oracle, idx):
    k = KATS["greedy"][idx]
    logits = np.zeros(k["vocab"] * (k["K"] + 1), np.uint16)
    r = oracle.speculative_accept(k["targets"], logits, k["vocab"], k["drafts"], k["length"], k["stats_in"],
                                  k["vocab"], _cfg(oracle))
    assert list(r["sampled_out"]) == k["sampled_out"]
    assert (r["num_sampled"], r["accepted"], r["length"], r["token"]) == (
        k["num_sampled"], k["accepted"], k["length_out"], k["token"])
    assert list(r["stats"]) == k["stats_out"]


def test_one_hot_residual_kats(oracle):
    m = KATS["one_hot_residual"]
    idx = np.array(m["indices"], np.int32)
    prob = np.array(m["probabilities"], np.float32)
    for d, u, accept in m["accept"]:
        pd = float(prob[list(idx).index(d)]) if d in idx else 0.0
        assert (np.float32(u) < np.float32(pd)) == accept
    for excl, u, expected in m["residual"]:
        assert oracle.pick_from_support(idx, prob, excl, u) == expected


def test_exact_k_matrix_oracle(oracle):
    m = KATS["exact_k_matrix"]
    rows, domain = m["physical_rows"], m["token_domain"]
    for K in (1, 3, 7, 15):
        logits = np.full((K + 1, rows), BF(np.array([-20.0], np.float32))[0], dtype=np.uint16)
        ids = [(17 + c * 7919) % domain for c in range(K + 1)]
        for c in range(K + 1):
            logits[c, ids[c]] = BF(np.array([20.0], np.float32))[0]
            logits[c, domain] = BF(np.array([100.0], np.float32))[0]
        r = oracle.speculative_accept(None, logits.reshape(-1), rows, ids[:K], 100, [0] * (4 + K), domain,
                                      _cfg(oracle, 1.0, 1, seed=20260716 + K))
        assert list(r["sampled_out"]) + [r["num_sampled"], r["accepted"]] == ids[:K] + [ids[K], K + 1, K]


@pytest.mark.parametrize("name", ["overlay_frequency", "overlay_presence"])
def test_overlay_kats_oracle(oracle, name):
    m = KATS[name]
    K, vocab = m["K"], m["vocab"]
    logits = np.full((K + 1, vocab), BF(np.array([m["background"]], np.float32))[0], dtype=np.uint16)
    for col, tok, val in m["set"]:
        logits[col, tok] = BF(np.array([val], np.float32))[0]
    for seed in m["seeds"]:
        for L in m["lengths"]:
            cfg = _cfg(oracle, m["temperature"], m["top_k"], seed=seed, presence=m.get("presence_penalty", 0.0),
                       frequency=m.get("frequency_penalty", 0.0))
            r = oracle.speculative_accept(None, logits.reshape(-1), vocab, m["drafts"], L, [0] * (4 + K), vocab, cfg)
            assert list(r["sampled_out"]) + [r["num_sampled"], r["accepted"]] == m["expected"]


def test_truncated_distribution_properties(oracle):
    """Support is a prefix of the sorted candidates, probabilities sum to 1, top-k/top-p/min-p cut."""
    col = syn.normal_bf16(21, 5000, 3.0)
    f = syn.bf16_bits_to_f32(col)
    order = np.lexsort((np.arange(5000), -f))
    for top_k, top_p, min_p in [(0, 1.0, 0.0), (5, 1.0, 0.0), (0, 0.5, 0.0), (0, 1.0, 0.3), (20, 0.9, 0.1)]:
        idx, prob = oracle.truncated_distribution(col, 5000, _cfg(oracle, 0.7, top_k, top_p, min_p, seed=1))
        cap = top_k if 0 < top_k < 20 else 20
        assert len(idx) <= cap and list(idx) == list(order[: len(idx)])
        assert abs(float(prob.sum(dtype=np.float64)) - 1.0) < 1e-5
        if top_p == 1.0 and min_p == 0.0:
            assert len(idx) == cap
        w = np.exp((f[order[:cap]].astype(np.float64) - f[order[0]]) / 0.7)
        keep = cap
        if min_p > 0:
            below = np.flatnonzero(w < min_p * w[0])
            keep = int(below[0]) if below.size else cap
        if top_p < 1.0:
            reach = int(np.searchsorted(np.cumsum(w), top_p * w.sum())) + 1
            keep = min(keep, reach)
        assert abs(len(idx) - max(keep, 1)) <= 1, (top_k, top_p, min_p, len(idx), keep)


def test_stochastic_distribution_matches_target(oracle):
    """Emitted-token distribution of one accept round equals p0 (reference check at
    tests/ops/test_speculative_round.cpp:499-587, gap <= 0.015), over many seeds."""
    vocab, K = 6, 1
    x0 = np.array([2.0, 1.5, 1.0, 0.5, 0.0, -1.0], np.float32)
    x1 = np.array([0.0, 1.0, 0.0, 0.0, 0.0, 0.0], np.float32)
    logits = np.concatenate([BF(x0), BF(x1)])
    idx, prob = oracle.truncated_distribution(BF(x0), vocab, _cfg(oracle, 1.0, 0, 1.0, 0.0, seed=0))
    p0 = np.zeros(vocab)
    p0[idx] = prob
    counts = np.zeros(vocab)
    n = 20000
    for s in range(n):
        r = oracle.speculative_accept(None, logits, vocab, [0], 10, [0] * 5, vocab, _cfg(oracle, 1.0, seed=s))
        counts[r["sampled_out"][0]] += 1
    assert np.abs(counts / n - p0).max() <= 0.015


# ---- general acceptance (Mode F) -------------------------------------------------------------------

def _gcfg(oracle, t=0.7, top_p=0.95):
    c = oracle.GeneralConfig()
    c.temperature, c.top_p = t, top_p
    return c


def test_general_column_nucleus_is_minimal_prefix(oracle):
    col = syn.normal_bf16(31, 3000, np.sqrt(3.0))
    n, w, member, zs, z = oracle.general_column(col, 3000, _gcfg(oracle))
    f = syn.bf16_bits_to_f32(col)
    order = np.lexsort((np.arange(3000), -f))
    assert member[order[:n]].all() and not member[order[n:]].any()
    wf = np.zeros(3000, dtype=object)
    _, wall, _, _, _ = oracle.general_column(col, 3000, _gcfg(oracle, top_p=1.0))
    target = (z * int(round(0.95 * 2 ** 24))) >> 24
    cum = np.cumsum([int(wall[i]) for i in order], dtype=object)
    assert cum[n - 1] >= target and (n == 1 or cum[n - 2] < target)
    assert zs == sum(int(x) for x in w)


def test_general_q_equals_p_always_accepts(oracle):
    rows, K = 4000, 3
    t = syn.normal_bf16(41, rows * (K + 1), np.sqrt(3.0))
    d = t[: rows * K].copy()
    drafts = [int(np.argsort(-syn.bf16_bits_to_f32(t[i * rows:(i + 1) * rows]))[3]) for i in range(K)]
    for s in range(20):
        ua = syn.uniforms(s, K + 1).astype(np.float32)
        r = oracle.general_accept(t, d, rows, drafts, 50, [0] * (4 + K), rows, _gcfg(oracle, 0.7, 1.0), ua, 0.5)
        assert r["accepted"] == K


def test_general_residual_mass_identity(oracle):
    """sum max(0, p - q) == 1 - sum min(p, q) in exact rationals on a tiny vocabulary."""
    rows = 9
    t = BF(np.array([1.0, 0.5, 0.2, -0.3, 2.0, 0.0, 0.7, -1.0, 0.1], np.float32))
    d = BF(np.array([0.2, 1.5, 0.2, 0.3, 1.0, 0.0, -0.7, 0.0, 0.4], np.float32))
    _, wp, _, zp, _ = oracle.general_column(t, rows, _gcfg(oracle, 1.0, 1.0))
    _, wq, _, zq, _ = oracle.general_column(d, rows, _gcfg(oracle, 1.0, 1.0))
    p = [Fraction(int(x), zp) for x in wp]
    q = [Fraction(int(x), zq) for x in wq]
    assert sum(max(Fraction(0), a - b) for a, b in zip(p, q)) == 1 - sum(min(a, b) for a, b in zip(p, q))


def test_general_emitted_distribution_equals_target(oracle):
    """Speculative sampling emits exactly p whatever q is: chi-square over many uniform draws."""
    rows = 5
    t = BF(np.array([1.0, 0.2, -0.5, 0.8, 0.0], np.float32))
    d = BF(np.array([-1.0, 1.2, 0.5, 0.0, 0.3], np.float32))
    _, wp, _, zp, _ = oracle.general_column(t, rows, _gcfg(oracle, 1.0, 1.0))
    _, wq, _, zq, _ = oracle.general_column(d, rows, _gcfg(oracle, 1.0, 1.0))
    p = np.array([int(x) for x in wp], dtype=np.float64) / zp
    q = np.array([int(x) for x in wq], dtype=np.float64) / zq
    logits = np.concatenate([t, t])  # column 1 is the bonus column
    n = 30000
    counts = np.zeros(rows)
    us = syn.uniforms(99, 3 * n)
    for i in range(n):
        dr = int(np.searchsorted(np.cumsum(q), us[3 * i]))  # draft token sampled from q
        dr = min(dr, rows - 1)
        r = oracle.general_accept(logits, d, rows, [dr], 10, [0] * 5, rows, _gcfg(oracle, 1.0, 1.0),
                                  np.array([us[3 * i + 1], 0.5], np.float32), float(us[3 * i + 2]))
        counts[r["sampled_out"][0]] += 1
    expected = p * n
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    assert chi2 < 20.0, (chi2, counts / n, p)


# Mode F against the mathematics (numpy float64, independent of the oracle's fixed-point code):
# weights, the top-p nucleus, the emitted distribution at the C4 temperature and top-p, and the
# reduction to Mode R when the draft distribution is one-hot.

def _np_probs(x, temperature, top_p):
    """float64 restatement: w = exp((x - max) / T); nucleus = shortest prefix in (value desc, id asc)
    order whose mass reaches top_p * sum(w); p = w / mass on the nucleus, else 0."""
    x = np.asarray(x, dtype=np.float64)
    w = np.exp((x - x.max()) / temperature)
    order = np.lexsort((np.arange(x.size), -x))
    cum = np.cumsum(w[order])
    n = x.size if top_p >= 1.0 else int(np.searchsorted(cum, top_p * cum[-1], side="left")) + 1
    p = np.zeros_like(w)
    keep = order[:n]
    p[keep] = w[keep] / w[keep].sum()
    return p, n, cum, order


@pytest.mark.parametrize("temperature", [0.5, 0.7, 1.3])
def test_general_weights_match_exp(oracle, temperature):
    """Weights / 2^40 equal exp((x - max) / T) within the error of the FP32 evaluation: det_expf
    (<= 1 ulp, 2^-23 relative), the FP32 reciprocal of T and the rounded products x / T and max / T
    (each 2^-24 relative to the argument), then the 2^40 fixed-point rounding (2^-41 absolute). A
    temperature applied the wrong way or a wrong maximum shift is off by orders of magnitude."""
    V = 50000
    col = syn.normal_bf16(60 + int(temperature * 10), V, np.sqrt(3.0))
    x = syn.bf16_bits_to_f32(col).astype(np.float64)
    n, w, member, zs, z = oracle.general_column(col, V, _gcfg(oracle, temperature, 1.0))
    assert n == V and member.all() and zs == z == sum(int(v) for v in w)
    exact = np.exp((x - x.max()) / temperature)
    arg = (np.abs(x) + abs(x.max())) / temperature
    bound = exact * (2.0 ** -22 + 4.0 * 2.0 ** -24 * arg) + 2.0 ** -41
    got = w.astype(np.float64) / 2.0 ** 40
    assert np.all(np.abs(got - exact) <= bound), float(np.max(np.abs(got - exact) / bound))
    # the maximum's weight is exp(e) with e the FP32 rounding error of max / T (at most 2^-24 relative)
    assert abs(int(w[int(np.argmax(x))]) / 2.0 ** 40 - 1.0) <= 2.0 ** -22 * (1.0 + abs(x.max()) / temperature)


@pytest.mark.parametrize("temperature,top_p", [(0.7, 0.95), (0.5, 0.9), (1.3, 0.5), (0.7, 0.999)])
def test_general_nucleus_matches_numpy(oracle, temperature, top_p):
    """The nucleus is the float64 nucleus: the same size, except +-1 where the float64 cumulative
    mass lies within 1e-6 of top_p * sum (the fixed-point sums may then round either way)."""
    V = 20000
    for seed in range(3):
        col = syn.normal_bf16(700 + seed, V, np.sqrt(3.0))
        x = syn.bf16_bits_to_f32(col).astype(np.float64)
        n, w, member, zs, z = oracle.general_column(col, V, _gcfg(oracle, temperature, top_p))
        _, n_np, cum, order = _np_probs(x, temperature, top_p)
        if n != n_np:
            edge = cum[min(n, n_np) - 1]
            assert abs(n - n_np) == 1 and abs(edge - top_p * cum[-1]) <= 1e-6 * cum[-1], (n, n_np)
        assert member[order[:n]].all() and member.sum() == n


def test_general_emitted_distribution_t07_top_p(oracle):
    """configs[3]'s temperature 0.7 and top-p 0.95: the first emitted token is distributed as the
    float64 nucleus distribution of the target column (chi-square, 9 degrees of freedom at most),
    with the draft token drawn from the float64 draft distribution."""
    rows = 12
    t = BF(np.array([1.9, 1.4, 1.2, 0.9, 0.7, 0.5, 0.1, -0.2, -0.6, -1.0, -1.5, -2.5], np.float32))
    d = BF(np.array([0.4, 1.8, 0.3, 1.1, -0.5, 0.9, 0.6, -0.1, 0.2, -1.2, -0.4, 0.0], np.float32))
    p, _, _, _ = _np_probs(syn.bf16_bits_to_f32(t), 0.7, 0.95)
    q, _, _, _ = _np_probs(syn.bf16_bits_to_f32(d), 0.7, 0.95)
    assert 0 < (p == 0).sum() and 0 < (q == 0).sum()  # both nuclei cut something off
    logits = np.concatenate([t, t])
    n = 30000
    counts = np.zeros(rows)
    us = syn.uniforms(1234, 3 * n)
    cq = np.cumsum(q)
    for i in range(n):
        dr = min(int(np.searchsorted(cq, us[3 * i] * cq[-1], side="right")), rows - 1)
        r = oracle.general_accept(logits, d, rows, [dr], 10, [0] * 5, rows, _gcfg(oracle, 0.7, 0.95),
                                  np.array([us[3 * i + 1], 0.5], np.float32), float(us[3 * i + 2]))
        counts[r["sampled_out"][0]] += 1
    assert counts[p == 0].sum() == 0, "a token outside the target nucleus was emitted"
    sel = p > 0
    expected = p[sel] * n
    chi2 = float(((counts[sel] - expected) ** 2 / expected).sum())
    assert chi2 < 27.9, (chi2, counts / n, p)  # p = 0.001 quantile of chi2(9)


def test_general_one_hot_q_reproduces_mode_r(oracle):
    """With a one-hot draft distribution q = e_d, min(1, p/q) accepts iff u < p(d), and the residual
    max(0, p - q) is p without d: Mode R's rule. Fed Mode R's own uniforms (accept, correction and
    bonus streams at positions L+i+1 / L+K+1) and target columns whose nucleus is ordered by id
    (logits strictly decreasing in id, so both inverse CDFs walk the same order), Mode F returns
    Mode R's accept count and token. Trials with a uniform within 1e-5 of a float64 decision or CDF
    boundary are skipped (FP32 versus fixed-point rounding may decide those either way)."""
    V, K, L = 64, 3, 100
    rng = np.random.default_rng(77)
    compared = 0
    trials = 300
    for trial in range(trials):
        cols, ps = [], []
        for i in range(K + 1):
            while True:
                head = np.sort(rng.uniform(-1.0, 3.0, 8))[::-1].astype(np.float32)
                x = np.full(V, -30.0, np.float32)
                x[:8] = head
                xb = BF(x)
                xf = syn.bf16_bits_to_f32(xb)
                if np.all(np.diff(xf[:8]) < 0):
                    p, n_np, cum, _ = _np_probs(xf, 0.7, 0.95)
                    if np.min(np.abs(cum[:8] - 0.95 * cum[-1])) > 1e-4 * cum[-1]:
                        break
            cols.append(xb)
            ps.append(p)
        target = np.concatenate(cols)
        drafts = [int(v) for v in rng.integers(0, 8, K)]
        seed = 1000 + trial
        cfg = _cfg(oracle, 0.7, top_p=0.95, seed=seed)
        r_mode = oracle.speculative_accept(None, target, V, drafts, L, [0] * (4 + K), V, cfg)
        a = r_mode["accepted"]
        u_acc = [oracle.sampling_uniform(seed, L + i + 1, 2) for i in range(K)]
        u_bonus = oracle.sampling_uniform(seed, L + K + 1, 4)
        u_corr = oracle.sampling_uniform(seed, L + a + 1, 3) if a < K else 0.5
        # margins of every decision Mode R took
        near = any(abs(u_acc[i] - ps[i][drafts[i]]) < 1e-5 for i in range(min(a + 1, K)))
        if a < K:
            rest = ps[a].copy()
            rest[drafts[a]] = 0.0
            u_pick, edges = u_corr, np.cumsum(rest) / max(rest.sum(), 1e-300)
        else:
            u_pick, edges = u_bonus, np.cumsum(ps[K])
        near = near or np.min(np.abs(edges - u_pick)) < 1e-5
        if near:
            continue
        one_hot = np.full((K, V), BF(np.array([-100.0], np.float32))[0], np.uint16)
        for i, dr in enumerate(drafts):
            one_hot[i, dr] = BF(np.array([0.0], np.float32))[0]
        r_gen = oracle.general_accept(target, one_hot.reshape(-1), V, drafts, L, [0] * (4 + K), V,
                                      _gcfg(oracle, 0.7, 0.95), np.array(u_acc + [u_bonus], np.float32),
                                      float(u_corr))
        assert r_gen["accepted"] == a, (trial, r_gen, r_mode)
        assert r_gen["token"] == r_mode["token"], (trial, r_gen, r_mode)
        assert list(r_gen["sampled_out"]) == list(r_mode["sampled_out"])
        compared += 1
    assert compared >= 0.9 * trials


# ---- commit / rollback / compaction / tree ---------------------------------------------------------

def _planes(P=256, H=2, D=128, seed=0):
    rng = np.random.default_rng(seed)
    return (rng.integers(-127, 128, (H, P, D)).astype(np.int8), rng.integers(-127, 128, (H, P, D)).astype(np.int8),
            rng.integers(0, 0x7BFF, (H, P, 2)).astype(np.uint16), rng.integers(0, 0x7BFF, (H, P, 2)).astype(np.uint16))


def test_commit_prefix_writes_only_accepted(oracle):
    H, D, P, T = 2, 128, 256, 4
    kc, vc, ks, vs = _planes(P, H, D)
    before = [a.copy() for a in (kc, vc, ks, vs)]
    k = syn.normal_bf16(1, D * H * T)
    v = syn.normal_bf16(2, D * H * T)
    pos = np.arange(100, 104, dtype=np.int32)
    oracle.kv_commit_prefix(k, v, pos, T, 2, H, D, P, kc, vc, ks, vs)
    changed = np.zeros(P, bool)
    for a, b in zip((kc, vc, ks, vs), before):
        changed |= (a != b).reshape(H, P, -1).any(axis=(0, 2))
    assert set(np.flatnonzero(changed)) <= {100, 101}
    for t in range(2):
        for h in range(H):
            for g in range(2):
                src = k[D * (h + H * t) + 64 * g: D * (h + H * t) + 64 * g + 64]
                codes, scale = oracle.quantize_group(src)
                assert np.array_equal(kc[h, 100 + t, 64 * g: 64 * g + 64], codes) and ks[h, 100 + t, g] == scale


def test_rollback_zeroes_rejected_rows_only(oracle):
    H, D, P, T = 2, 128, 256, 5
    kc, vc, ks, vs = _planes(P, H, D, 1)
    before = [a.copy() for a in (kc, vc, ks, vs)]
    pos = np.arange(50, 55, dtype=np.int32)
    oracle.kv_rollback(pos, T, 2, H, D, P, kc, vc, ks, vs)
    for a, b in zip((kc, vc, ks, vs), before):
        assert not a[:, 52:55].any()
        keep = np.ones(P, bool)
        keep[52:55] = False
        assert np.array_equal(a[:, keep], b[:, keep])


def test_compact_path_moves_rows(oracle):
    H, D, P = 2, 128, 256
    kc, vc, ks, vs = _planes(P, H, D, 2)
    before = [a.copy() for a in (kc, vc, ks, vs)]
    base, path = 60, np.array([0, 2, 5, 11], np.int32)
    oracle.kv_compact_path(base, path, 4, H, D, P, kc, vc, ks, vs)
    for a, b in zip((kc, vc, ks, vs), before):
        for j, u in enumerate(path):
            assert np.array_equal(a[:, base + j], b[:, base + u])


def test_tree_longest_path_brute_force(oracle):
    rng = np.random.default_rng(0)
    for _ in range(300):
        n = int(rng.integers(1, 17))
        parents = [-1] + [int(rng.integers(0, u)) for u in range(1, n)]
        tok = rng.integers(0, 3, n).astype(np.int32)
        tgt = rng.integers(0, 3, n).astype(np.int32)
        acc = {0}
        for u in range(1, n):
            if parents[u] in acc and tok[u] == tgt[parents[u]]:
                acc.add(u)
        depth = {0: 0}
        for u in sorted(acc)[1:]:
            depth[u] = depth[parents[u]] + 1
        best = min(acc, key=lambda u: (-depth[u], u))
        chain = []
        u = best
        while u >= 0:
            chain.append(u)
            u = parents[u]
        assert list(oracle.tree_longest_path(np.array(parents, np.int32), tok, tgt)) == chain[::-1]
