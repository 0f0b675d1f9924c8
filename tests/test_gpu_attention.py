"""GPU parity of the verify attention (A1/A2/A3, trees, batches) against the CPU oracle.

Criteria (BASELINE): INT8 codes and FP16 scale bits bit-exact; attention output within 2e-3
relative L2 error against the FP64 oracle (BF16 output, the reference's contract) and the
reference's attention_bf16 composite (tests/ops/op_check.h:61); the FP32-output extension is held
to 1e-3, which isolates the kernel's own arithmetic from the final BF16 rounding.
"""
import numpy as np
import pytest

from helpers import AttnCase, reference_composite_ok, rel_l2
import gpu_runner

pytestmark = pytest.mark.gpu

REL_L2_BF16 = 2e-3
REL_L2_F32 = 1e-3


def _check_cache(cache, expected):
    kc, vc, ks, vs = cache.download()
    ekc, evc, eks, evs = expected
    assert np.array_equal(kc, ekc), "K codes differ"
    assert np.array_equal(vc, evc), "V codes differ"
    assert np.array_equal(ks, eks), "K scale bits differ"
    assert np.array_equal(vs, evs), "V scale bits differ"


def _check_out(got, ref, bound):
    err = rel_l2(got, ref)
    ok, msg = reference_composite_ok(got, ref)
    print(f"rel_l2={err:.3e} composite: {msg}", flush=True)
    assert err <= bound, f"rel_l2 {err:.3e} > {bound:.1e}"
    return ok


@pytest.mark.parametrize("L,T", [(4096, 4), (0, 4), (1, 1), (17, 3), (100, 6), (127, 4), (128, 4),
                                 (255, 2), (256, 5), (1000, 4), (2882, 4), (7680, 4)])
def test_a1_parity(gpu, L, T):
    print(f"case A1 L={L} T={T}", flush=True)
    case = AttnCase([L], T=T, seed=1000 + L + T)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=False)
    _check_cache(cache, expected_cache)
    assert _check_out(out, ref, REL_L2_BF16)
    out32, _ = gpu_runner.run_attention(case, out_f32=True)
    _check_out(out32, ref, REL_L2_F32)


def test_c1_config_seed0(gpu):
    """Config 1: batch 1, q_len 4, 40/8/128, context 4096, seed 0."""
    case = AttnCase([4096], T=4, seed=0)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=False)
    _check_cache(cache, expected_cache)
    assert _check_out(out, ref, REL_L2_BF16)


def test_outliers_long(gpu):
    """Config 3 statistics (1% outliers at +-20) at a context the oracle finishes quickly."""
    case = AttnCase([16384], T=4, seed=3, outliers=True)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True)
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


@pytest.mark.parametrize("L", [60000, 130000])
def test_power_of_two_split_lengths_moved(gpu, L):
    """Batch-1 contexts whose split plan rounds to 1,024 and 2,048 keys per split: the plan moves
    such lengths one 128-key step up (fewer splits, cached partials), and every key stays covered."""
    print(f"case pow2 split L={L}", flush=True)
    case = AttnCase([L], T=4, seed=77 + L)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True)
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


def test_a2_then_a3_equals_a1(gpu):
    """A2 then A3 against A1: identical cache bytes, and outputs within the reference's A1/A3 parity
    criterion (attention_bf16 composite, tests/ops/test_gqa_attention.cpp:1077-1078). A1 attends to
    the new rows from registers, A3 reads them back, so the sums are ordered differently."""
    case = AttnCase([3000], T=4, seed=11)
    expected_cache, ref = case.oracle_after_append()
    cache = gpu_runner.upload_cache(case)
    gpu_runner.append(case, cache)
    _check_cache(cache, expected_cache)
    out3, _ = gpu_runner.run_attention(case, out_f32=True, mode="A3", cache=cache)
    out1, cache1 = gpu_runner.run_attention(case, out_f32=True, mode="A1")
    _check_cache(cache1, expected_cache)
    ok, msg = reference_composite_ok(out1, out3)
    assert ok, f"A1/A3 parity: {msg}"
    assert rel_l2(out1, out3) <= 5e-4
    _check_out(out3, ref, REL_L2_F32)
    _check_out(out1, ref, REL_L2_F32)


def test_future_token_isolation(gpu):
    """Changing the last token's K/V must not change earlier tokens' outputs (bit-exact)."""
    case = AttnCase([2500], T=4, seed=12)
    out_a, _ = gpu_runner.run_attention(case, out_f32=True)
    per_tok = case.D * case.Hkv
    case.k_new = case.k_new.copy()
    case.v_new = case.v_new.copy()
    case.k_new[3 * per_tok:] ^= np.uint16(0x0040)
    case.v_new[3 * per_tok:] ^= np.uint16(0x0040)
    out_b, _ = gpu_runner.run_attention(case, out_f32=True)
    per_q = case.D * case.Hq
    assert np.array_equal(out_a[: 3 * per_q], out_b[: 3 * per_q])
    assert not np.array_equal(out_a[3 * per_q:], out_b[3 * per_q:])


@pytest.mark.parametrize("L,env", [(7680, 9732), (8400, 9732), (7000, 12000), (12000, 12004)])
def test_envelope_past_window(gpu, L, env):
    """Batch-1 A1 under an envelope wider than the window, as in a replayed round (from this window
    up): the host plan's last splits hold no keys and return (m, l) = (-inf, 0), and the
    head-fastest dispatch puts them last. 9,732 and 12,000 keys plan one workgroup per CU (26 and
    32 splits of 384 keys; 256-key splits would make 312 and 376 workgroups); 12,004 keys a 384-key
    plan over the whole window."""
    print(f"case A1 L={L} envelope={(L + 4, env)}", flush=True)
    case = AttnCase([L], T=4, seed=2 * L + env, max_context=env)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True, envelope=(L + 4, env))
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


@pytest.mark.parametrize("L,T", [(0, 4), (200, 3), (3000, 1), (7680, 4), (9000, 4), (40000, 3), (131000, 4)])
def test_device_split_plan(gpu, L, T):
    """Batch-1 A1 under an envelope far wider than the window (1 .. 131,076 keys), as in a graph
    replayed from a short context up to a long one: the launched splits (61 of 2,176 keys for the
    envelope's end) divide the window read from the device positions instead, at least 256 keys
    each. Windows shorter than one split, 7,684 keys (31 splits of 256), 9,004 and 40,003 keys (one
    workgroup per CU: 24 splits of 384 rather than 36 of 256, 32 of 1,280 rather than 53 of 768), a
    window at the envelope's end (61 of 2,176), and one and two row tiles (T = 1 and 3: 5 and 15
    rows; T = 4: 20 rows)."""
    env = 131076
    print(f"case A1 device plan L={L} T={T} envelope=(1, {env})", flush=True)
    case = AttnCase([L], T=T, seed=7 * L + T, max_context=env, gen="pcg")
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True, envelope=(1, env))
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


def test_split_count_independence(gpu):
    """The same problem under two envelopes (different split plans) stays within tolerance of the
    oracle both ways; the two differ only by the FP16 rounding of probabilities, which is relative
    to each split's running maximum."""
    case = AttnCase([9000], T=4, seed=13, max_context=200000)
    _, ref = case.oracle_after_append()
    out_small, _ = gpu_runner.run_attention(case, out_f32=True, envelope=(1, 9004))
    out_large, _ = gpu_runner.run_attention(case, out_f32=True, envelope=(1, 200000))
    _check_out(out_small, ref, REL_L2_F32)
    _check_out(out_large, ref, REL_L2_F32)
    assert rel_l2(out_small, out_large) < 1e-3


def test_batch_ragged(gpu):
    case = AttnCase([1024, 5000, 17, 3000], T=4, seed=21)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True)
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


def test_batch_one_long_many_short(gpu):
    """The batch plan gives every workgroup the same number of keys: the long sequence spans most
    of them, and one workgroup's range holds several short (or empty) sequences, each with a
    partial of its own; each sequence's partials merge in order."""
    case = AttnCase([60000, 5, 0, 300, 1, 2000, 17, 128, 0, 9, 4000, 33], T=4, seed=22)
    print("case batch B=12 one long", flush=True)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True)
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


def test_batch_more_sequences_than_split_budget(gpu):
    """72 sequences over 8 KV heads exceed the 64 workgroups per KV head the plan targets: each
    workgroup's range then holds several sequences, and sequences 64-71 take the plan's second
    64-sequence round."""
    rng = np.random.default_rng(23)
    case = AttnCase([int(x) for x in rng.integers(0, 150, size=72)], T=4, seed=23)
    print("case batch B=72", flush=True)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True)
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


def test_batch_ragged_past_64_sequences(gpu):
    """80 ragged contexts, some long: spans that cross the 64-sequence rounds of the batch plan."""
    rng = np.random.default_rng(24)
    Ls = [int(x) for x in rng.integers(0, 3000, size=80)]
    Ls[70] = 20000
    case = AttnCase(Ls, T=4, seed=24)
    print("case batch B=80 ragged", flush=True)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True)
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


@pytest.mark.parametrize("T,Hq,Hkv,Ls", [(16, 40, 8, [3000]), (8, 64, 8, [2500]), (32, 40, 8, [1900]),
                                          (7, 40, 8, [4100]), (12, 16, 2, [2222]), (16, 40, 8, [700, 5000, 0])])
def test_many_query_rows(gpu, T, Hq, Hkv, Ls):
    """More than 32 query rows per KV head: several row-chunk workgroups per (split, KV head), the
    new rows appended by their own launch first."""
    case = AttnCase(Ls, T=T, Hq=Hq, Hkv=Hkv, seed=2000 + T + Hq + len(Ls))
    print(f"case rows T={T} Hq={Hq} Hkv={Hkv} Ls={Ls}", flush=True)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True)
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


def _bfs_tree(n):
    """Binary tree in BFS order pruned to n nodes: parent(u) = (u - 1) // 2."""
    return [-1] + [(u - 1) // 2 for u in range(1, n)]


def test_tree_attention(gpu):
    parents = np.array([_bfs_tree(16), _bfs_tree(16)], dtype=np.int32).reshape(-1)
    case = AttnCase([1500, 4000], T=16, seed=31, parents=parents)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True, mode="TREE")
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


def test_rising_scores_a1(gpu):
    """Boosted key rows late in 512-position windows: splits' running maxima rise past the lazy
    threshold in mid-stream, so the two-tile path rescales non-zero accumulators."""
    case = AttnCase([40000], T=4, seed=34, k_boost=4.0, gen="pcg")
    print("case rising scores A1 40000", flush=True)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True)
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


@pytest.mark.parametrize("Ls", [[40000], [9000, 30000]])
def test_rising_scores_tree(gpu, Ls):
    """The same mid-stream rises through the five-tile (80-row) tree form, whose lazy rescale works
    on the accumulators in place in AGPRs; batch 1 and a batch of two."""
    parents = np.array([_bfs_tree(16)] * len(Ls), dtype=np.int32).reshape(-1)
    case = AttnCase(Ls, T=16, seed=35 + len(Ls), parents=parents, k_boost=4.0, gen="pcg")
    print(f"case rising scores tree {Ls}", flush=True)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True, mode="TREE")
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


def test_tree_attention_outliers(gpu):
    """Five-tile tree form under the long-context statistics (1% of K/V entries at +-20)."""
    parents = np.array([_bfs_tree(16), _bfs_tree(16)], dtype=np.int32).reshape(-1)
    case = AttnCase([3000, 9000], T=16, seed=33, parents=parents, outliers=True)
    print("case tree outliers", flush=True)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True, mode="TREE")
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


def test_chain_tree_equals_causal(gpu):
    T = 6
    parents = np.array([-1] + list(range(T - 1)), dtype=np.int32)
    case = AttnCase([2000], T=T, seed=32, parents=parents)
    out_tree, _ = gpu_runner.run_attention(case, out_f32=True, mode="TREE")
    out_causal, _ = gpu_runner.run_attention(case, out_f32=True, mode="A1")
    assert np.array_equal(out_tree, out_causal)


@pytest.mark.parametrize("Hq,Hkv", [(24, 4), (16, 2), (8, 8)])
def test_other_group_sizes(gpu, Hq, Hkv):
    case = AttnCase([1777], T=4, Hq=Hq, Hkv=Hkv, seed=40 + Hq)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True)
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


def test_large_magnitude_groups_within_fp16_range(gpu):
    """K' and V' enter the MFMA as FP16(code * scale): groups whose absolute maximum stays below
    65,504 (FP16's largest finite value) decode exactly as the reference's FP32 decode does. Here
    1% of the history's entries are +-20 and a few whole groups are scaled to an absolute maximum
    of 6e4 (K and V), with Q small enough to keep the softmax non-degenerate."""
    case = AttnCase([3000], T=4, seed=61, outliers=True, qstd=0.002)
    rng = np.random.default_rng(61)
    # the scales of 20 random (head, row, group) of K and of V become 6e4 / 127
    for s in (case.ks, case.vs):
        for _ in range(20):
            h, r, g = int(rng.integers(0, 8)), int(rng.integers(0, 3000)), int(rng.integers(0, 2))
            s[0, h, r, g] = np.float16(60000.0 / 127.0).view(np.uint16)
    expected_cache, ref = case.oracle_after_append()
    out, cache = gpu_runner.run_attention(case, out_f32=True)
    _check_cache(cache, expected_cache)
    _check_out(out, ref, REL_L2_F32)


@pytest.mark.parametrize("absmax", [1e5, 1e6])
@pytest.mark.parametrize("form", ["a1", "tree", "d256", "long", "wide_envelope"])
def test_fp32_range_groups(gpu, absmax, form):
    """The reference decodes cached K/V as FP32(code) * scale (include/ninfer/ops/gqa_attention.h:30),
    and INT8-G64 scales reach 65,504, so a group's values may exceed FP16's range. Groups with an
    absolute maximum of 1e5 and 1e6 (scale absmax / 127, above 512) in the history of K and of V, and
    a new token whose K/V rows the op itself quantizes at that size, against the FP64 oracle: chunks
    holding such a scale divide their K scales by a power of two (undone on the FP32 scores) and the
    wave's V scales by a running power of two (undone on O). Causal (two-tile), tree (five-tile),
    head_dim 256 (24|4 heads), a long context (splits of 1,024+ keys), and a window of 9,004 keys
    under the envelope (1, 131,076), whose splits the device plans (24 of 384 keys)."""
    T, Hq, Hkv, D, L = 4, 40, 8, 128, 3000
    parents = None
    env = None
    if form == "tree":
        T = 16
        parents = np.array(_bfs_tree(16), dtype=np.int32)
    elif form == "d256":
        Hq, Hkv, D = 24, 4, 256
    elif form == "long":
        L = 60000
    elif form == "wide_envelope":
        L, env = 9000, 131076
    print(f"case fp32 range {form} absmax={absmax:g}", flush=True)
    case = AttnCase([L], T=T, Hq=Hq, Hkv=Hkv, D=D, seed=int(absmax) % 1000 + len(form), parents=parents,
                    qstd=2e-5, gen="pcg" if (env or L) > 10000 else "splitmix", max_context=env)
    rng = np.random.default_rng(int(absmax) + len(form))
    G = D // 64
    big = np.float16(absmax / 127.0).view(np.uint16)
    for sc in (case.ks, case.vs):
        for _ in range(24):
            h, r, g = int(rng.integers(0, Hkv)), int(rng.integers(0, L)), int(rng.integers(0, G))
            sc[0, h, r, g] = big
    # the new rows of token 1 carry absmax-sized values: the in-kernel quantization gives them such scales
    per_tok = D * Hkv
    for arr in (case.k_new, case.v_new):
        x = (arr[per_tok:2 * per_tok].astype(np.uint32) << 16).view(np.float32)
        x = x * np.float32(absmax / max(1e-6, float(np.abs(x).max())))
        arr[per_tok:2 * per_tok] = ((x.view(np.uint32) + 0x7FFF + ((x.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
    expected_cache, ref = case.oracle_after_append()
    mode = "TREE" if parents is not None else "A1"
    envelope = (1, env) if env else None
    out, cache = gpu_runner.run_attention(case, out_f32=True, mode=mode, envelope=envelope)
    _check_cache(cache, expected_cache)
    assert np.all(np.isfinite(out))
    # The rel-L2 bars only: the reference's attention_bf16 composite is an elementwise envelope for
    # its registered activation range, and outputs here cancel next to values of 1e6 (it is printed).
    _check_out(out, ref, REL_L2_F32)
    out16, _ = gpu_runner.run_attention(case, out_f32=False, mode=mode, envelope=envelope)
    _check_out(out16, ref, REL_L2_BF16)


def test_repeated_calls_one_workspace(gpu):
    """Successive calls on one workspace (filled with a non-zero pattern first): no call depends on
    what an earlier one left in the split scratch. Three A3 calls with different queries on one
    cache and workspace, each against the oracle, then the first query again, bit-exact against its
    first result."""
    import ninfer_amd as na
    from ninfer_amd import ops
    from ninfer_amd.device import DeviceArray, DeviceBuffer, synchronize
    case = AttnCase([5000], T=4, seed=4200, max_context=5100)
    _, ref0 = case.oracle_after_append()
    cache = gpu_runner.upload_cache(case)
    gpu_runner.append(case, cache)
    D, Hq, T = case.D, case.Hq, case.T
    env = (1, case.max_context)
    ws = DeviceBuffer(ops.gqa_attention_workspace_bytes(Hq, case.Hkv, D, T, 1, env[1]))
    ws.fill(0xA5)
    pos = DeviceArray.from_numpy(na.I32, case.positions, (T, 1))
    rng = np.random.default_rng(4201)
    queries = [case.q] + [((rng.standard_normal(case.q.size).astype(np.float32)).view(np.uint32) >> 16).astype(np.uint16)
                          for _ in range(2)]
    outs = []
    for qv in queries + [case.q]:
        q = DeviceArray.from_numpy(na.BF16, qv, (D, Hq, T, 1))
        out = DeviceArray(na.FP32, (D, Hq, T, 1))
        ops.gqa_attention_cached(q.tensor(), pos.tensor(), case.scale, cache.view(), env, ws, out.tensor(), None)
        synchronize()
        outs.append(out.numpy().astype(np.float64))
    for qv, got in zip(queries, outs):
        case.q = qv
        _, ref = case.oracle_after_append()
        _check_out(got, ref, REL_L2_F32)
    assert np.array_equal(outs[0], outs[3])
