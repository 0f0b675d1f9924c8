"""GPU parity at the benchmark's own workload sizes (4 and 5) against the FP64
oracle, so the split plans the benchmark times are the ones checked:

- C3: one sequence at context 260,096 with 1% +-20 outliers (the host split plan at its largest);
- C4: 16 sequences with contexts uniform in [1,024, 32,768] (the device batch split plan);
- C5: 8 BFS-16 draft trees over contexts log-uniform in [1,024, 131,072] (the tree mask over three
  row-chunk workgroups per KV head), and a chain tree against the causal mask at a long context.

Criteria as in test_gpu_attention.py: INT8 codes and FP16 scale bits of the whole cache
bit-exact after the append, BF16 output within 2e-3 relative L2 of the FP64 oracle plus the
reference's attention_bf16 composite (tests/ops/op_check.h:61), FP32 output within 1e-3. The
histories come from the oracle library's threaded generator (same distributions as the small
tests, 10^8+ values in seconds).
"""
import numpy as np
import pytest

from helpers import AttnCase, reference_composite_ok, rel_l2
import gpu_runner

pytestmark = pytest.mark.gpu

REL_L2_BF16 = 2e-3
REL_L2_F32 = 1e-3


def _check_cache(cache, expected):
    got = cache.download()
    for name, g, e in zip(("K codes", "V codes", "K scale bits", "V scale bits"), got, expected):
        assert np.array_equal(g, e), f"{name} differ"


def _check(got, ref, bound, composite):
    err = rel_l2(got, ref)
    ok, msg = reference_composite_ok(got, ref)
    print(f"rel_l2={err:.3e} composite: {msg}", flush=True)
    assert err <= bound, f"rel_l2 {err:.3e} > {bound:.1e}"
    if composite:
        assert ok, msg


def _bfs_tree(n):
    return [-1] + [(u - 1) // 2 for u in range(1, n)]


def test_c3_long_context_260k(gpu):
    """batch 1, q_len 4, 40/8/128, context 260,096, K/V N(0,1) with 1% +-20."""
    print("case C3 L=260096 T=4 outliers", flush=True)
    case = AttnCase([260096], T=4, seed=0xC3, outliers=True, gen="pcg")
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=False)
    _check_cache(cache, expected_cache)
    _check(out, ref, REL_L2_BF16, composite=True)
    out32, _ = gpu_runner.run_attention(case, out_f32=True, cache=cache)
    _check(out32, ref, REL_L2_F32, composite=False)


def test_c4_batch16_ragged(gpu):
    """configs[3] attention: B = 16, contexts seeded uniform in [1,024, 32,768], q_len 4."""
    rng = np.random.default_rng(0xC4)
    Ls = [int(x) for x in rng.integers(1024, 32769, size=16)]
    print(f"case C4 B=16 Ls={Ls}", flush=True)
    case = AttnCase(Ls, T=4, seed=0xC4, gen="pcg")
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=False)
    _check_cache(cache, expected_cache)
    _check(out, ref, REL_L2_BF16, composite=True)
    out32, _ = gpu_runner.run_attention(case, out_f32=True, cache=cache)
    _check(out32, ref, REL_L2_F32, composite=False)


def test_c5_tree_batch8(gpu):
    """configs[4] attention: B = 8 trees of 16 nodes (binary, BFS order, depth 4 pruned to 16) under
    the ancestor mask, contexts log-uniform in [1,024, 131,072]."""
    rng = np.random.default_rng(0xC5)
    Ls = [int(x) for x in np.exp(rng.uniform(np.log(1024), np.log(131072), size=8))]
    print(f"case C5 B=8 N=16 Ls={Ls}", flush=True)
    parents = np.array([_bfs_tree(16)] * 8, dtype=np.int32).reshape(-1)
    case = AttnCase(Ls, T=16, seed=0xC5, parents=parents, gen="pcg")
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=False, mode="TREE")
    _check_cache(cache, expected_cache)
    _check(out, ref, REL_L2_BF16, composite=True)
    out32, _ = gpu_runner.run_attention(case, out_f32=True, mode="TREE", cache=cache)
    _check(out32, ref, REL_L2_F32, composite=False)


def test_c5_chain_tree_equals_causal_long(gpu):
    """A chain of 16 nodes under the tree mask equals causal A1 bit for bit at context 131,056."""
    T = 16
    print("case C5 chain T=16 L=131056", flush=True)
    parents = np.array([-1] + list(range(T - 1)), dtype=np.int32)
    case = AttnCase([131072 - T], T=T, seed=0xC55, parents=parents, gen="pcg")
    out_tree, cache = gpu_runner.run_attention(case, out_f32=True, mode="TREE")
    out_causal, _ = gpu_runner.run_attention(case, out_f32=True, mode="A1", cache=cache)
    assert np.array_equal(out_tree, out_causal)
