"""GPU parity of the verify attention over a BF16 KV cache (include/ninfer/ops/gqa_attention.h:
52-66 admits BF16 or INT8-G64 planes). The cases follow the reference's BF16 ones: single-token
decode at several positions and its stress input (tests/ops/test_gqa_attention.cpp:768-844,
1621-1629), T = 1..6 at cache offsets 0, 1, 17, 128 (:1550-1555), and the split-API parity sweep
T = 1..16 for the 16|2 geometry with A1, A2 and A3 (:1572-1601). Inputs are the reference's
ranges (Q, K uniform in [-0.25, 0.25), V in [-1, 1)). Criteria: new rows written bit-exactly and no
other byte changed (rows past each history hold a +inf marker the kernel must never let into the
output), output within 2e-3 relative L2 of the FP64 oracle and the reference's attention_bf16
composite (tests/ops/op_check.h:61)."""
import numpy as np
import pytest

from helpers import AttnCase, reference_composite_ok, rel_l2
from ninfer_amd import synthetic as syn
import gpu_runner

pytestmark = pytest.mark.gpu

GEOMETRIES = [(24, 4), (16, 2)]


def _check_cache(cache, expected):
    k, v = cache.download()
    ek, ev = expected
    assert np.array_equal(k, ek), "K plane differs"
    assert np.array_equal(v, ev), "V plane differs"


def _check(got, ref, bound=2e-3):
    err = rel_l2(got, ref)
    ok, msg = reference_composite_ok(got, ref)
    print(f"rel_l2={err:.3e} composite: {msg}", flush=True)
    assert ok, msg
    assert err <= bound, f"rel_l2 {err:.3e} > {bound:.1e}"


def _run_a1(case, out_f32=False, mode="A1"):
    print(f"case BF16 D={case.D} {case.Hq}|{case.Hkv} L={case.Ls} T={case.T} {mode}", flush=True)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=out_f32, mode=mode)
    _check_cache(cache, expected_cache)
    _check(out, ref)
    return out, ref


@pytest.mark.parametrize("Hq,Hkv", GEOMETRIES)
@pytest.mark.parametrize("pos", [1, 17, 2048, 2882, 8191, 32768])
def test_bf16_decode_positions(gpu, Hq, Hkv, pos):
    case = AttnCase([pos], T=1, Hq=Hq, Hkv=Hkv, D=256, seed=11 + pos, kv="bf16", dist="uniform")
    _run_a1(case)


@pytest.mark.parametrize("Hq,Hkv", GEOMETRIES)
def test_bf16_stress_returns_new_value_row(gpu, Hq, Hkv):
    """Q = K_new = 8 and history K = -8: the new row takes all the weight, so the output is the
    new V row (tests/ops/test_gqa_attention.cpp:772-777)."""
    D, L = 256, 17
    case = AttnCase([L], T=1, Hq=Hq, Hkv=Hkv, D=D, seed=31, kv="bf16")
    eight = syn.f32_to_bf16_bits(np.array([8.0], np.float32))[0]
    case.q[:] = eight
    case.k_new[:] = eight
    case.kb[0, :, :L] = syn.f32_to_bf16_bits(np.array([-8.0], np.float32))[0]
    case.v_new[:] = syn.uniform_bf16(32, case.v_new.size, -8.0, 8.0)
    case.vb[0, :, :L] = syn.uniform_bf16(33, Hkv * L * D, -8.0, 8.0).reshape(Hkv, L, D)
    out, ref = _run_a1(case, out_f32=True)
    assert rel_l2(out, ref) <= 1e-6  # O / l with P of the new row near 1 and the rest 0


@pytest.mark.parametrize("Hq,Hkv", GEOMETRIES)
@pytest.mark.parametrize("offset", [0, 1, 17, 128])
@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 6])
def test_bf16_tokens_at_offsets(gpu, Hq, Hkv, offset, T):
    case = AttnCase([offset], T=T, Hq=Hq, Hkv=Hkv, D=256, seed=100 * T + offset, kv="bf16", dist="uniform")
    _run_a1(case)


def _split_api(case):
    """A1 against the oracle; A2 then A3 on a second cache: same planes, output against the oracle
    and within the reference's A1-versus-A3 criterion of A1 (tests/ops/test_gqa_attention.cpp:
    1077-1078)."""
    out1, _ = _run_a1(case, out_f32=True)
    expected_cache, ref = case.oracle_after_append()
    cache = gpu_runner.upload_cache(case)
    gpu_runner.append(case, cache)
    _check_cache(cache, expected_cache)
    out3, _ = gpu_runner.run_attention(case, out_f32=True, mode="A3", cache=cache)
    _check(out3, ref)
    ok, msg = reference_composite_ok(out3, out1)
    assert ok, msg


@pytest.mark.parametrize("T", list(range(1, 17)))
def test_bf16_group8_split_api(gpu, T):
    _split_api(AttnCase([17], T=T, Hq=16, Hkv=2, D=256, seed=1500 + T, kv="bf16", dist="uniform"))
    if T > 6:
        frontier = 512 if T <= 12 else 1024
        base = frontier - T + 1
        _split_api(AttnCase([base], T=T, Hq=16, Hkv=2, D=256, seed=1700 + T, kv="bf16", dist="uniform"))


@pytest.mark.parametrize("base", [1008, 1009])
def test_bf16_group8_chunk_frontier(gpu, base):
    _split_api(AttnCase([base], T=16, Hq=16, Hkv=2, D=256, seed=1916 + base, kv="bf16", dist="uniform"))


@pytest.mark.parametrize("Hq,Hkv,L,T", [(40, 8, 7680, 4), (40, 8, 0, 4), (32, 8, 4096, 16),
                                        (32, 8, 100, 1), (40, 8, 70001, 6)])
def test_bf16_head_dim_128(gpu, Hq, Hkv, L, T):
    """head_dim 128: the 40|8 geometry of the verify step and the 32|8 BF16 drafter cache."""
    case = AttnCase([L], T=T, Hq=Hq, Hkv=Hkv, D=128, seed=7 + L + T, kv="bf16")
    _run_a1(case, out_f32=True)


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 40, 8), (256, 24, 4)])
def test_bf16_batch_ragged(gpu, D, Hq, Hkv):
    case = AttnCase([0, 300, 4096, 1777], T=4, Hq=Hq, Hkv=Hkv, D=D, seed=5, kv="bf16")
    _run_a1(case, out_f32=True)


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 40, 8), (256, 16, 2)])
def test_bf16_tree(gpu, D, Hq, Hkv):
    T = 16
    parents = np.array([-1] + [(u - 1) // 2 for u in range(1, T)], dtype=np.int32)
    case = AttnCase([3000], T=T, Hq=Hq, Hkv=Hkv, D=D, seed=31, parents=parents, kv="bf16")
    _run_a1(case, out_f32=True, mode="TREE")


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 40, 8), (256, 24, 4)])
def test_bf16_future_token_isolation(gpu, D, Hq, Hkv):
    """Changing token t's new K/V and Q leaves the outputs of tokens < t bit-identical."""
    T = 6
    case = AttnCase([2000], T=T, Hq=Hq, Hkv=Hkv, D=D, seed=12, kv="bf16")
    out_a, _ = gpu_runner.run_attention(case, out_f32=True)
    kn = case.k_new.reshape(T, Hkv, D)
    kn[T - 1] = kn[T - 1][::-1].copy()
    vn = case.v_new.reshape(T, Hkv, D)
    vn[T - 1] = vn[T - 2]
    case.q.reshape(T, Hq, D)[T - 1] = case.q.reshape(T, Hq, D)[T - 2]
    out_b, _ = gpu_runner.run_attention(case, out_f32=True)
    a = out_a.reshape(T, Hq, D)
    b = out_b.reshape(T, Hq, D)
    assert np.array_equal(a[:T - 1], b[:T - 1])
    assert not np.array_equal(a[T - 1], b[T - 1])
