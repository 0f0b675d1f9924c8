"""GPU parity of the recurrent-state ops of the hybrid layers and their commit after acceptance:
gated_delta_rule (snapshot, distinct-state and in-place forms), causal_conv1d_silu (snapshot and
regular forms) and the device scalar ops.

The cases restate the reference's (tests/ops/test_gated_delta_rule.cpp:863-904,
tests/ops/test_causal_conv1d_silu.cpp, tests/ops/test_speculative_round.cpp:356-497): inputs uniform
q, k, v in [-1, 1] (q/k rows normalized unless the op normalizes them), g in [-4, 0] ([-1, -0.05]
for the stress case), beta in [0.05, 0.95], state in [-0.1, 0.1]; unused snapshot slots hold 17.0
and must keep it. Criteria are the reference's named tolerances (tests/ops/op_check.h:39-42,86-88)
against the FP64 oracle; BF16 windows are bit-exact copies."""
import numpy as np
import pytest

import ninfer_amd as na
from helpers import reference_composite_ok
from ninfer_amd import ops, synthetic as syn
from ninfer_amd.device import DeviceArray, DeviceBuffer, synchronize
import gpu_runner

pytestmark = pytest.mark.gpu

GDN_OUTPUT_BF16 = (1e-3, 1.0e-2, 2e-3, 5.0, 8e-3)
GDN_STATE_FP32 = (5e-4, 5.0e-3, 2e-2, 5.0, 5e-3)
BF16_REDUCTION = (2e-3, 1.6e-2, 2e-3, 5.0, 8e-3)


def _bf(x):
    return syn.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


def _f(bits):
    return syn.bf16_bits_to_f32(bits).astype(np.float64)


def _inputs(seed, S, Hqk, Hv, T, normalized=True, stress_g=False, near_zero=False):
    rng = np.random.default_rng(seed)
    q = rng.uniform(-1, 1, (T, Hqk, S)).astype(np.float32)
    k = rng.uniform(-1, 1, (T, Hqk, S)).astype(np.float32)
    v = rng.uniform(-1, 1, (T, Hv, S)).astype(np.float32)
    g = rng.uniform(-1.0, -0.05, (T, Hv)) if stress_g else rng.uniform(-4.0, 0.0, (T, Hv))
    beta = rng.uniform(0.05, 0.95, (T, Hv)).astype(np.float32)
    state = rng.uniform(-0.1, 0.1, (Hv, S, S)).astype(np.float32)
    if normalized:
        q /= np.linalg.norm(q, axis=-1, keepdims=True)
        k /= np.linalg.norm(k, axis=-1, keepdims=True)
    if near_zero:
        q *= 1e-4
        k *= 1e-4
    return dict(q=_bf(q), k=_bf(k), v=_bf(v), g=g.astype(np.float32), beta=beta, state=state)


def _ok(got, ref, tol, tag):
    ok, msg = reference_composite_ok(got, ref, tol)
    print(f"{tag}: {msg}", flush=True)
    assert ok, f"{tag}: {msg}"


def _dev(inp, S, Hqk, Hv, T):
    return dict(q=DeviceArray.from_numpy(na.BF16, inp["q"], (S, Hqk, T)),
                k=DeviceArray.from_numpy(na.BF16, inp["k"], (S, Hqk, T)),
                v=DeviceArray.from_numpy(na.BF16, inp["v"], (S, Hv, T)),
                g=DeviceArray.from_numpy(na.FP32, inp["g"], (Hv, T)),
                beta=DeviceArray.from_numpy(na.FP32, inp["beta"], (Hv, T)),
                out=DeviceArray(na.BF16, (S, Hv, T)))


def run_snapshot(inp, S, Hqk, Hv, T, slots, initial_slot, normalize):
    d = _dev(inp, S, Hqk, Hv, T)
    d["out"].buf.fill(0xFF)
    states = np.full((slots, Hv, S, S), 17.0, dtype=np.float32)
    states[initial_slot] = inp["state"]
    dst = DeviceArray.from_numpy(na.FP32, states, (S, S, Hv, slots))
    dslot = DeviceArray.from_numpy(na.I32, np.array([initial_slot], np.int32), (1,))
    ops.gated_delta_rule_snapshot(d["q"].tensor(), d["k"].tensor(), d["v"].tensor(), d["g"].tensor(),
                                  d["beta"].tensor(), float(np.float32(1 / np.sqrt(S))), normalize, dst.tensor(),
                                  dslot.tensor(), d["out"].tensor())
    synchronize()
    return _f(d["out"].numpy()).reshape(T, Hv, S), dst.numpy().reshape(slots, Hv, S, S)


def check_snapshot(seed, S, Hqk, Hv, T, slots, initial_slot, normalize, **kw):
    print(f"case gdn snapshot S={S} Hqk={Hqk} Hv={Hv} T={T} slots={slots} slot={initial_slot} norm={normalize} {kw}",
          flush=True)
    from oracle import pyoracle
    inp = _inputs(seed, S, Hqk, Hv, T, normalized=not normalize, **kw)
    ref_out, _, ref_snap = pyoracle.gdn_recurrent(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["state"],
                                                  S, Hqk, Hv, T, normalize, snapshots=True)
    out, states = run_snapshot(inp, S, Hqk, Hv, T, slots, initial_slot, normalize)
    expected = np.full((slots, Hv, S, S), 17.0)
    expected[initial_slot] = inp["state"]
    expected[:T] = ref_snap
    _ok(out, ref_out, GDN_OUTPUT_BF16, "out")
    _ok(states, expected, GDN_STATE_FP32, "slots")
    assert np.array_equal(states[T:], expected[T:].astype(np.float32)), "slots >= T changed"


@pytest.mark.parametrize("seed", [7028, 8128])
@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 6])
def test_gdn_snapshot_reference_cases(gpu, seed, T):
    check_snapshot(seed + T, 128, 16, 48, T, T, 0, False)


def test_gdn_snapshot_stress_g(gpu):
    check_snapshot(9028, 128, 16, 48, 6, 6, 0, False, stress_g=True)


@pytest.mark.parametrize("T", list(range(1, 17)))
def test_gdn_fused_norm_snapshot_t1_to_16(gpu, T):
    check_snapshot(9520 + T, 128, 16, 32, T, 17, 16, True)


@pytest.mark.parametrize("initial_slot", list(range(16)))
def test_gdn_fused_norm_initial_slots(gpu, initial_slot):
    """The initial slot lies among the slots the call overwrites: it is read before any write."""
    check_snapshot(9600 + initial_slot, 128, 16, 32, 16, 17, initial_slot, True)


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 6])
def test_gdn_fused_norm_hv48(gpu, T):
    check_snapshot(9680 + T, 128, 16, 48, T, 7, 6, True)


@pytest.mark.parametrize("Hv,slots,slot", [(32, 17, 16), (48, 7, 6)])
def test_gdn_fused_norm_near_zero(gpu, Hv, slots, slot):
    check_snapshot(9740 + Hv, 128, 16, Hv, 4, slots, slot, True, near_zero=True)


@pytest.mark.parametrize("S,Hqk,Hv,T,slot", [(128, 16, 48, 4, 0), (128, 16, 48, 4, 2), (128, 16, 48, 5, 5),
                                             (128, 16, 32, 6, 6), (16, 4, 4, 3, 5), (32, 4, 8, 6, 1),
                                             (64, 4, 16, 2, 6)])
def test_gdn_selected_slot(gpu, S, Hqk, Hv, T, slot):
    check_snapshot(10028 + 10 * slot + S, S, Hqk, Hv, T, 7, slot, False)


def run_regular(inp, S, Hqk, Hv, T, normalize, in_place):
    d = _dev(inp, S, Hqk, Hv, T)
    s_in = DeviceArray.from_numpy(na.FP32, inp["state"], (S, S, Hv))
    s_out = s_in if in_place else DeviceArray(na.FP32, (S, S, Hv))
    ops.gated_delta_rule(d["q"].tensor(), d["k"].tensor(), d["v"].tensor(), d["g"].tensor(), d["beta"].tensor(),
                         float(np.float32(1 / np.sqrt(S))), normalize, s_in.tensor(), s_out.tensor(), d["out"].tensor())
    synchronize()
    return d["out"].numpy(), s_out.numpy().reshape(Hv, S, S)


@pytest.mark.parametrize("S,Hqk,Hv,T", [(128, 16, 48, 1), (128, 16, 48, 2), (128, 16, 48, 7), (128, 16, 48, 64),
                                        (16, 4, 4, 1), (32, 4, 8, 3), (64, 4, 16, 70), (128, 16, 32, 128)])
def test_gdn_regular_forms(gpu, S, Hqk, Hv, T):
    """Distinct-state form against the oracle (tests/ops/test_gated_delta_rule.cpp:865-871,
    891-894); the in-place form gives the same bits."""
    print(f"case gdn regular S={S} Hqk={Hqk} Hv={Hv} T={T}", flush=True)
    from oracle import pyoracle
    inp = _inputs(2026 + T + S, S, Hqk, Hv, T)
    ref_out, ref_state, _ = pyoracle.gdn_recurrent(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["state"],
                                                   S, Hqk, Hv, T)
    out, state = run_regular(inp, S, Hqk, Hv, T, False, in_place=False)
    _ok(_f(out).reshape(T, Hv, S), ref_out, GDN_OUTPUT_BF16, "out")
    _ok(state, ref_state, GDN_STATE_FP32, "state")
    out2, state2 = run_regular(inp, S, Hqk, Hv, T, False, in_place=True)
    assert np.array_equal(out, out2) and np.array_equal(state, state2)


def test_gdn_snapshot_chain_equals_one_call(gpu):
    """T one-token snapshot calls, each resuming from the slot the previous one wrote, give the
    bits of one T-token call (slot t = state after token t)."""
    S, Hqk, Hv, T = 128, 16, 32, 5
    inp = _inputs(4411, S, Hqk, Hv, T)
    out_all, st_all = run_snapshot(inp, S, Hqk, Hv, T, T, 0, False)
    state = inp["state"]
    for t in range(T):
        one = {key: (val[t:t + 1] if key != "state" else state) for key, val in inp.items()}
        out1, st1 = run_snapshot(one, S, Hqk, Hv, 1, 1, 0, False)
        assert np.array_equal(out1[0], out_all[t])
        assert np.array_equal(st1[0], st_all[t])
        state = st1[0]


# ---- causal conv1d + SiLU ---------------------------------------------------------------------------

def _conv_inputs(seed, C, T, slots):
    rng = np.random.default_rng(seed)
    x = _bf(rng.uniform(-2, 2, (T, C)))
    w = _bf(rng.uniform(-1, 1, (4, C)))
    states = _bf(rng.uniform(-2, 2, (slots, 3, C)))
    return x, w, states


def run_conv_snapshot(x, w, states, slot, C, T):
    slots = states.shape[0]
    dx = DeviceArray.from_numpy(na.BF16, x, (C, T))
    dw = DeviceArray.from_numpy(na.BF16, w, (C, 4))
    ds = DeviceArray.from_numpy(na.BF16, states, (C, 3, slots))
    dslot = DeviceArray.from_numpy(na.I32, np.array([slot], np.int32), (1,))
    dout = DeviceArray(na.BF16, (C, T))
    ops.causal_conv1d_silu_snapshot(dx.tensor(), dw.tensor(), ds.tensor(), dslot.tensor(), dout.tensor())
    synchronize()
    return dout.numpy().reshape(T, C), ds.numpy().reshape(slots, 3, C)


@pytest.mark.parametrize("C,T,slots,slot", [(8192, 1, 17, 16), (8192, 4, 5, 4), (8192, 16, 17, 3),
                                            (6144, 6, 7, 0), (37, 5, 5, 2), (10240, 2, 3, 1)])
def test_conv_snapshot(gpu, C, T, slots, slot):
    print(f"case conv snapshot C={C} T={T} slots={slots} slot={slot}", flush=True)
    from oracle import pyoracle
    x, w, states = _conv_inputs(C + T + slot, C, T, slots)
    ref, windows = pyoracle.causal_conv1d_silu(x, w, states[slot], C, T)
    out, got_states = run_conv_snapshot(x, w, states, slot, C, T)
    _ok(_f(out), ref, BF16_REDUCTION, "out")
    assert np.array_equal(got_states[:T], windows), "snapshot windows differ"
    assert np.array_equal(got_states[T:], states[T:]), "slots >= T changed"


@pytest.mark.parametrize("C,T", [(8192, 1), (8192, 7), (64, 128)])
def test_conv_regular_and_decode_chain(gpu, C, T):
    """Regular form against the oracle; in place equals distinct; T one-token calls chained through
    the in-place state give the bits of one T-token call."""
    from oracle import pyoracle
    x, w, states = _conv_inputs(77 + C + T, C, T, 1)
    ref, windows = pyoracle.causal_conv1d_silu(x, w, states[0], C, T)
    dx = DeviceArray.from_numpy(na.BF16, x, (C, T))
    dw = DeviceArray.from_numpy(na.BF16, w, (C, 4))
    s_in = DeviceArray.from_numpy(na.BF16, states[0], (C, 3))
    s_out = DeviceArray(na.BF16, (C, 3))
    dout = DeviceArray(na.BF16, (C, T))
    ops.causal_conv1d_silu(dx.tensor(), dw.tensor(), s_in.tensor(), s_out.tensor(), dout.tensor())
    synchronize()
    out = dout.numpy().reshape(T, C)
    _ok(_f(out), ref, BF16_REDUCTION, "out")
    assert np.array_equal(s_out.numpy().reshape(3, C), windows[-1])
    s_chain = DeviceArray.from_numpy(na.BF16, states[0], (C, 3))
    for t in range(T):
        dxt = DeviceArray.from_numpy(na.BF16, x[t], (C, 1))
        dot = DeviceArray(na.BF16, (C, 1))
        ops.causal_conv1d_silu(dxt.tensor(), dw.tensor(), s_chain.tensor(), s_chain.tensor(), dot.tensor())
        synchronize()
        assert np.array_equal(dot.numpy(), out[t])
    assert np.array_equal(s_chain.numpy().reshape(3, C), windows[-1])


# ---- device scalars and the commit after acceptance ----------------------------------------------

def test_scalar_ops(gpu):
    a = DeviceArray.from_numpy(na.I32, np.array([5], np.int32), (1,))
    b = DeviceArray.from_numpy(na.I32, np.array([-1], np.int32), (1,))
    c = DeviceArray.from_numpy(na.I64, np.array([2 ** 40], np.int64), (1,))
    for value in range(16):
        ops.set_i32_scalar(a.tensor(), value)
        ops.assign_i32_scalar(a.tensor(), b.tensor())
        synchronize()
        assert b.numpy()[0] == value
    ops.increment_i32_scalar(b.tensor())
    ops.increment_i64_scalar(c.tensor())
    synchronize()
    assert b.numpy()[0] == 16 and c.numpy()[0] == 2 ** 40 + 1


def test_accepted_state_resume(gpu):
    """tests/ops/test_speculative_round.cpp:356-497: after a greedy round with A accepted drafts,
    assign_i32_scalar(accepted -> initial_slot) selects slot A, and one more token from the snapshot
    form equals (bit for bit) the regular form started from a copy of slot A."""
    K, slots, vocab, S = 15, 17, 32, 16
    targets = np.arange(1, K + 2, dtype=np.int32)
    conv_states = _bf(np.array([[0.125 * (s + 1) + 0.03125 * i for i in range(3)] for s in range(slots)]))
    ssm_states = np.array([[0.002 * (s + 1) + 0.00001 * (i % S) for i in range(S * S)] for s in range(slots)],
                          np.float32)
    conv_x, conv_w = _bf([0.375]), _bf([0.5, -0.25, 0.75, 0.125])
    q = _bf(0.02 * np.arange(1, S + 1))
    k = _bf(0.015 * (S - np.arange(S)))
    v = _bf(0.01 * ((np.arange(S) % 5) - 2))
    g, beta = np.zeros(1, np.float32), np.full(1, 0.25, np.float32)
    for A in range(K + 1):
        drafts = np.array([targets[i] if i < A else 0 for i in range(K)], np.int32)
        d_target = DeviceArray.from_numpy(na.I32, targets, (K + 1,))
        d_logits = DeviceArray.from_numpy(na.BF16, np.zeros((K + 1, vocab), np.uint16), (vocab, K + 1))
        d_drafts = DeviceArray.from_numpy(na.I32, drafts, (K,))
        d_len = DeviceArray.from_numpy(na.I32, np.array([100], np.int32), (1,))
        d_tok = DeviceArray.from_numpy(na.I32, np.array([-1], np.int32), (1,))
        d_so = DeviceArray(na.I32, (K + 1,))
        d_ns = DeviceArray(na.I32, (1,))
        d_acc = DeviceArray(na.I32, (1,))
        d_stats = DeviceArray.from_numpy(na.I64, np.zeros(4 + K, np.int64), (4 + K,))
        d_slot = DeviceArray.from_numpy(na.I32, np.array([-1], np.int32), (1,))
        cfg, keep = gpu_runner.upload_configs([na.SamplingConfig()])
        ws = DeviceBuffer(max(256, ops.sampling_workspace_bytes(vocab, K + 1)))
        ops.speculative_accept_greedy_drafts(d_target.tensor(), d_logits.tensor(), d_drafts.tensor(), d_len.tensor(),
                                             d_tok.tensor(), d_so.tensor(), d_ns.tensor(), d_acc.tensor(),
                                             d_stats.tensor(), vocab, cfg.ptr, ws)
        ops.assign_i32_scalar(d_acc.tensor(), d_slot.tensor())
        synchronize()
        assert d_slot.numpy()[0] == A

        # conv: snapshot form from slot A vs regular form from a copy of slot A
        out_s, st_s = run_conv_snapshot(conv_x, conv_w, conv_states.reshape(slots, 3, 1), A, 1, 1)
        ds = DeviceArray.from_numpy(na.BF16, conv_states.reshape(slots, 3, 1), (1, 3, slots))
        dx = DeviceArray.from_numpy(na.BF16, conv_x, (1, 1))
        dw = DeviceArray.from_numpy(na.BF16, conv_w, (1, 4))
        do = DeviceArray(na.BF16, (1, 1))
        ops.causal_conv1d_silu_snapshot(dx.tensor(), dw.tensor(), ds.tensor(), d_slot.tensor(), do.tensor())
        ref_state = DeviceArray.from_numpy(na.BF16, conv_states[A], (1, 3))
        ref_out = DeviceArray(na.BF16, (1, 1))
        ops.causal_conv1d_silu(dx.tensor(), dw.tensor(), ref_state.tensor(), ref_state.tensor(), ref_out.tensor())
        synchronize()
        assert np.array_equal(do.numpy(), ref_out.numpy()) and np.array_equal(do.numpy(), out_s.ravel())
        assert np.array_equal(ds.numpy().reshape(slots, 3)[0], ref_state.numpy())

        # GDN: the same with the device slot written by the acceptance
        dst = DeviceArray.from_numpy(na.FP32, ssm_states, (S, S, 1, slots))
        dq, dk = DeviceArray.from_numpy(na.BF16, q, (S, 1, 1)), DeviceArray.from_numpy(na.BF16, k, (S, 1, 1))
        dv = DeviceArray.from_numpy(na.BF16, v, (S, 1, 1))
        dg, db = DeviceArray.from_numpy(na.FP32, g, (1, 1)), DeviceArray.from_numpy(na.FP32, beta, (1, 1))
        dout = DeviceArray(na.BF16, (S, 1, 1))
        ops.gated_delta_rule_snapshot(dq.tensor(), dk.tensor(), dv.tensor(), dg.tensor(), db.tensor(), 0.25, False,
                                      dst.tensor(), d_slot.tensor(), dout.tensor())
        sref = DeviceArray.from_numpy(na.FP32, ssm_states[A], (S, S, 1))
        oref = DeviceArray(na.BF16, (S, 1, 1))
        ops.gated_delta_rule(dq.tensor(), dk.tensor(), dv.tensor(), dg.tensor(), db.tensor(), 0.25, False,
                             sref.tensor(), sref.tensor(), oref.tensor())
        synchronize()
        assert np.array_equal(dout.numpy(), oref.numpy())
        assert np.array_equal(dst.numpy().reshape(slots, S * S)[0], sref.numpy())
        del keep
