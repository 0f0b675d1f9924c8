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
from helpers import AttnCase, rel_l2
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
