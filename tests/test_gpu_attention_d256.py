"""GPU parity of the verify attention at the reference's registered geometries: head_dim 256 with
24 query / 4 KV heads (group 6) and 16 / 2 (group 8), INT8-G64 cache
(include/ninfer/ops/gqa_attention.h:57-58). The (history, T) cases are the reference's INT8
decode cases (tests/ops/test_gqa_attention.cpp:1541-1558, plus its long decode case :1612); the
criteria are those of the head_dim 128 tests: codes and scale bits bit-exact, output within 2e-3
relative L2 of the FP64 oracle (BF16) and the reference's attention_bf16 composite, 1e-3 for the
FP32-output extension."""
import numpy as np
import pytest

from helpers import AttnCase, reference_composite_ok, rel_l2
import gpu_runner

pytestmark = pytest.mark.gpu

GEOMETRIES = [(24, 4), (16, 2)]
REFERENCE_INT8_DECODE = [(0, 6), (17, 1), (2882, 1), (100, 2), (100, 3), (100, 4), (2048, 4), (100, 5),
                         (256, 5), (128, 6), (8192, 6), (40800, 1)]


def _check_cache(cache, expected):
    kc, vc, ks, vs = cache.download()
    ekc, evc, eks, evs = expected
    assert np.array_equal(kc, ekc), "K codes differ"
    assert np.array_equal(vc, evc), "V codes differ"
    assert np.array_equal(ks, eks), "K scale bits differ"
    assert np.array_equal(vs, evs), "V scale bits differ"


def _check(got, ref, bound):
    err = rel_l2(got, ref)
    ok, msg = reference_composite_ok(got, ref)
    print(f"rel_l2={err:.3e} composite: {msg}", flush=True)
    assert err <= bound, f"rel_l2 {err:.3e} > {bound:.1e}"
    return ok


@pytest.mark.parametrize("Hq,Hkv", GEOMETRIES)
@pytest.mark.parametrize("L,T", REFERENCE_INT8_DECODE)
def test_d256_a1_reference_cases(gpu, Hq, Hkv, L, T):
    print(f"case D=256 {Hq}|{Hkv} L={L} T={T}", flush=True)
    case = AttnCase([L], T=T, Hq=Hq, Hkv=Hkv, D=256, seed=900 + L + T + Hq)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=False)
    _check_cache(cache, expected_cache)
    assert _check(out, ref, 2e-3)
    out32, _ = gpu_runner.run_attention(case, out_f32=True)
    _check(out32, ref, 1e-3)


@pytest.mark.parametrize("T", list(range(1, 17)))
def test_d256_group8_tokens_1_to_16(gpu, T):
    """The 35B (16|2) qualification sweep: every T from 1 to 16 at history 17, A1 and A3 (after
    A2) against the oracle (tests/ops/test_gqa_attention.cpp:1577-1585)."""
    case = AttnCase([17], T=T, Hq=16, Hkv=2, D=256, seed=1600 + T)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True)
    _check_cache(cache, expected_cache)
    _check(out, ref, 1e-3)
    cache3 = gpu_runner.upload_cache(case)
    gpu_runner.append(case, cache3)
    _check_cache(cache3, expected_cache)
    out3, _ = gpu_runner.run_attention(case, out_f32=True, mode="A3", cache=cache3)
    _check(out3, ref, 1e-3)


@pytest.mark.parametrize("Hq,Hkv", GEOMETRIES)
def test_d256_a2_a3_equals_a1(gpu, Hq, Hkv):
    case = AttnCase([5000], T=4, Hq=Hq, Hkv=Hkv, D=256, seed=77 + Hq)
    out1, c1 = gpu_runner.run_attention(case, out_f32=True)
    cache = gpu_runner.upload_cache(case)
    gpu_runner.append(case, cache)
    out3, _ = gpu_runner.run_attention(case, out_f32=True, mode="A3", cache=cache)
    for x, y in zip(c1.download(), cache.download()):
        assert np.array_equal(x, y)
    # reference A1-versus-A3 criterion (tests/ops/test_gqa_attention.cpp:1077-1078)
    ok, msg = reference_composite_ok(out3, out1)
    assert ok, msg
    assert rel_l2(out3, out1) <= 5e-4


def test_d256_batch_ragged(gpu):
    case = AttnCase([0, 300, 4096, 1777], T=4, Hq=24, Hkv=4, D=256, seed=5)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True)
    _check_cache(cache, expected_cache)
    _check(out, ref, 1e-3)


@pytest.mark.parametrize("L", [5000, 60000])
def test_d256_device_split_plan(gpu, L):
    """Batch-1 (16|2, T = 4: 32 rows) under the envelope (1, 65,540): the host plan's 103 splits of
    640 keys divide the window read from the device positions instead (5,004 keys: 20 splits of
    256; 60,004: 94 of 640)."""
    env = 65540
    print(f"case D=256 device plan L={L} envelope=(1, {env})", flush=True)
    case = AttnCase([L], T=4, Hq=16, Hkv=2, D=256, seed=77 + L, max_context=env, gen="pcg")
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True, envelope=(1, env))
    _check_cache(cache, expected_cache)
    _check(out, ref, 1e-3)


def test_d256_tree(gpu):
    T = 16
    parents = np.array([-1] + [(u - 1) // 2 for u in range(1, T)], dtype=np.int32)
    case = AttnCase([3000], T=T, Hq=16, Hkv=2, D=256, seed=31, parents=parents)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True, mode="TREE")
    _check_cache(cache, expected_cache)
    _check(out, ref, 1e-3)


def test_d256_future_token_isolation(gpu):
    """Changing token t's new K/V and Q leaves the outputs of tokens < t bit-identical."""
    case = AttnCase([2000], T=6, Hq=24, Hkv=4, D=256, seed=12)
    out_a, _ = gpu_runner.run_attention(case, out_f32=True)
    D, Hkv, Hq = 256, 4, 24
    kn = case.k_new.reshape(6, Hkv, D)
    kn[5] = kn[5][::-1].copy()
    case.v_new.reshape(6, Hkv, D)[5] += 1
    case.q.reshape(6, Hq, D)[5] = case.q.reshape(6, Hq, D)[4]
    out_b, _ = gpu_runner.run_attention(case, out_f32=True)
    a = out_a.reshape(6, Hq, D)
    b = out_b.reshape(6, Hq, D)
    assert np.array_equal(a[:5], b[:5])
