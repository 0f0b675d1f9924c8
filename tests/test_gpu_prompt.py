"""GPU parity of the prompt route: A1/A3 above 32 query tokens (reference
src/ops/wrapper/gqa_attention.cpp:202-213,262-275, contract include/ninfer/ops/gqa_attention.h:59-73:
"T may be any positive value", one sequence, causal). The rows are appended first and the tokens
attend in launches of 32 through one workspace; every case is compared with the FP64 oracle at the
verify bars (2e-3 BF16 output, 1e-3 FP32 output), with the cache codes and scale bits bit-exact,
and A1 is bit-equal to A2 followed by A3."""
import numpy as np
import pytest

import ninfer_amd as na
from ninfer_amd import ops
from ninfer_amd.device import DeviceArray, DeviceBuffer, synchronize
from helpers import AttnCase, reference_composite_ok, rel_l2
import gpu_runner

pytestmark = pytest.mark.gpu

REL_L2_BF16 = 2e-3
REL_L2_F32 = 1e-3


def _check(case, out, ref, bound):
    err = rel_l2(out, ref)
    print(f"rel_l2={err:.3e}", flush=True)
    assert err <= bound, f"rel_l2 {err:.3e} > {bound:.1e}"


@pytest.mark.parametrize("L,T", [(0, 33), (300, 100), (1000, 64), (2882, 257), (1024, 512)])
def test_prompt_a1_int8(gpu, L, T):
    print(f"case prompt A1 int8 L={L} T={T}", flush=True)
    case = AttnCase([L], T=T, seed=4000 + L + T)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=False)
    kc, vc, ks, vs = cache.download()
    for got, want, name in zip((kc, vc, ks, vs), expected_cache, ("K codes", "V codes", "K scales", "V scales")):
        assert np.array_equal(got, want), f"{name} differ"
    _check(case, out, ref, REL_L2_BF16)
    out32, _ = gpu_runner.run_attention(case, out_f32=True)
    _check(case, out32, ref, REL_L2_F32)


@pytest.mark.parametrize("Hq,Hkv,D,kv,L,T", [(24, 4, 256, "i8", 500, 77), (16, 2, 256, "i8", 129, 40),
                                              (24, 4, 256, "bf16", 700, 50), (40, 8, 128, "bf16", 1500, 96)])
def test_prompt_a1_geometries(gpu, Hq, Hkv, D, kv, L, T):
    print(f"case prompt A1 {Hq}/{Hkv}/{D} {kv} L={L} T={T}", flush=True)
    case = AttnCase([L], T=T, Hq=Hq, Hkv=Hkv, D=D, kv=kv, seed=5000 + L + T)
    _, ref = case.oracle_after_append()
    out32, _ = gpu_runner.run_attention(case, out_f32=True)
    _check(case, out32, ref, REL_L2_F32)


def test_prompt_a2_then_a3_equals_a1(gpu):
    case = AttnCase([640], T=70, seed=71)
    out_a1, _ = gpu_runner.run_attention(case, out_f32=True)
    cache = gpu_runner.upload_cache(case)
    k = DeviceArray.from_numpy(na.BF16, case.k_new, (case.D, case.Hkv, case.T, 1))
    v = DeviceArray.from_numpy(na.BF16, case.v_new, (case.D, case.Hkv, case.T, 1))
    pos = DeviceArray.from_numpy(na.I32, case.positions, (case.T, 1))
    ops.gqa_kv_append(k.tensor(), v.tensor(), pos.tensor(), cache.view())
    synchronize()
    out_a3, _ = gpu_runner.run_attention(case, out_f32=True, mode="A3", cache=cache)
    assert np.array_equal(out_a1, out_a3)


def test_prompt_rows_match_verify_launches(gpu):
    """Tokens 32..63 of a 64-token prompt equal an A3 verify call of 32 tokens at positions L+32..
    over the same cache: the prompt's launches are exactly verify launches."""
    L, T = 400, 64
    case = AttnCase([L], T=T, seed=64)
    out_all, _ = gpu_runner.run_attention(case, out_f32=True)
    tail = AttnCase([L], T=T, seed=64)
    tail.T = 32
    D, Hq, Hkv = case.D, case.Hq, case.Hkv
    tail.q = case.q[32 * Hq * D:]
    tail.k_new = case.k_new[32 * Hkv * D:]
    tail.v_new = case.v_new[32 * Hkv * D:]
    tail.positions = case.positions[32:]
    cache = gpu_runner.upload_cache(case)
    gpu_runner.append(case, cache)
    synchronize()
    out_tail, _ = gpu_runner.run_attention(tail, out_f32=True, mode="A3", cache=cache, envelope=(1, case.max_context))
    assert np.array_equal(out_all.reshape(T, -1)[32:], out_tail.reshape(32, -1))


# The reference's prompt-route matrix at its registered geometries (tests/ops/test_gqa_attention.cpp:
# 1543-1546 INT8 prefill cases, 1564-1569 BF16 prefill cases, 1575-1576 the T = 1024 split-API
# case), with its input distribution: Q and K uniform in [-0.25, 0.25), V in [-1, 1) (:778-782).
GEOMETRIES = [(24, 4), (16, 2)]


@pytest.mark.parametrize("Hq,Hkv", GEOMETRIES)
@pytest.mark.parametrize("T,base", [(65, 0), (192, 0), (65, 384)])
def test_prompt_reference_int8_cases(gpu, Hq, Hkv, T, base):
    print(f"case prompt int8 {Hq}|{Hkv} T={T} base={base}", flush=True)
    case = AttnCase([base], T=T, Hq=Hq, Hkv=Hkv, D=256, dist="uniform", seed=904 + T + base + Hq)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=False)
    kc, vc, ks, vs = cache.download()
    for got, want, name in zip((kc, vc, ks, vs), expected_cache, ("K codes", "V codes", "K scales", "V scales")):
        assert np.array_equal(got, want), f"{name} differ"
    _check(case, out, ref, REL_L2_BF16)
    ok, msg = reference_composite_ok(out, ref)
    assert ok, msg


@pytest.mark.parametrize("Hq,Hkv", GEOMETRIES)
@pytest.mark.parametrize("T,base", [(128, 0), (512, 0), (128, 128), (512, 128), (65, 384)])
def test_prompt_reference_bf16_cases(gpu, Hq, Hkv, T, base):
    print(f"case prompt bf16 {Hq}|{Hkv} T={T} base={base}", flush=True)
    case = AttnCase([base], T=T, Hq=Hq, Hkv=Hkv, D=256, kv="bf16", dist="uniform", seed=113 + T + base + Hq)
    _, ref = case.oracle_after_append()
    out, _ = gpu_runner.run_attention(case, out_f32=False)
    _check(case, out, ref, REL_L2_BF16)
    ok, msg = reference_composite_ok(out, ref)
    assert ok, msg


@pytest.mark.parametrize("kv", ["i8", "bf16"])
def test_prompt_final_row_against_a3(gpu, kv):
    """A1 over a 1,024-token prompt at history 17, then A3 of the final token alone over the cache
    that A2 filled: both equal the oracle's final row (the reference's split-API case with
    final_row_only, :975-1060)."""
    T, base, Hq, Hkv, D = 1024, 17, 24, 4, 256
    case = AttnCase([base], T=T, Hq=Hq, Hkv=Hkv, D=D, kv=kv, dist="uniform", seed=1405)
    _, ref = case.oracle_after_append()
    out, _ = gpu_runner.run_attention(case, out_f32=True)
    _check(case, out, ref, REL_L2_F32)
    cache = gpu_runner.upload_cache(case)
    gpu_runner.append(case, cache)
    synchronize()
    last = AttnCase([base], T=1, Hq=Hq, Hkv=Hkv, D=D, kv=kv, dist="uniform", seed=1405)
    last.q = case.q[(T - 1) * Hq * D:]
    last.positions = case.positions[T - 1:]
    out1, _ = gpu_runner.run_attention(last, out_f32=True, mode="A3", cache=cache, envelope=(1, case.max_context))
    ref_last = ref.reshape(T, -1)[T - 1]
    _check(case, out1.reshape(-1), ref_last, REL_L2_F32)
    _check(case, out.reshape(T, -1)[T - 1], ref_last, REL_L2_F32)
