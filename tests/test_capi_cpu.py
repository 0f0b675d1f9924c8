"""CPU-side checks of the drop-in boundary: the library loads, exports every entry point the
public headers declare, and rejects invalid arguments on the host before any launch (the
reference wrappers' validation, e.g. src/ops/wrapper/gqa_attention.cpp:59-136). No call here
reaches a kernel, so no GPU is needed."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import ninfer_amd as na
from ninfer_amd import ops
from ninfer_amd._capi import INVALID_ARGUMENT, Tensor, lib

ROOT = Path(__file__).resolve().parent.parent


def _declared(header):
    text = (ROOT / "include" / header).read_text()
    return sorted(set(re.findall(r"\b(nmi_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = lib()
    names = _declared("ninfer_amd.h") + _declared("ninfer_amd_runtime.h")
    assert len(names) >= 38
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_cpp_header_wraps_every_op():
    hpp = (ROOT / "include" / "ninfer_amd" / "ops.hpp").read_text()
    for name in _declared("ninfer_amd.h"):
        if name in ("nmi_last_error", "nmi_build_info"):
            continue
        assert name in hpp, f"ops.hpp does not wrap {name}"


def test_build_info_names_gfx950():
    assert "gfx950" in na.build_info()


def _t(dtype, shape, ptr=0x10000):
    return Tensor.make(ptr, dtype, shape)


def _cache(Hkv=8, D=128, P=4224, max_ctx=4100, B=1):
    v = na.KVLayerView()
    v.k = _t(na.I8, (D, P, Hkv, B))
    v.v = _t(na.I8, (D, P, Hkv, B))
    v.k_scale = _t(na.FP16, (D // 64, P, Hkv, B))
    v.v_scale = _t(na.FP16, (D // 64, P, Hkv, B))
    v.max_context, v.padded_context = max_ctx, P
    v.num_kv_heads, v.head_dim, v.dtype, v.quant_group = Hkv, D, na.I8, 64
    return v


class _WS:
    def __init__(self, n):
        self._buf = (C.c_uint8 * (n + 512))()
        base = C.addressof(self._buf)
        self.ptr = (base + 255) & ~255
        self.nbytes = n


def _attention_args(**over):
    D, Hq, Hkv, T = 128, 40, 8, 4
    a = dict(q=_t(na.BF16, (D, Hq, T)), k=_t(na.BF16, (D, Hkv, T)), v=_t(na.BF16, (D, Hkv, T)),
             positions=_t(na.I32, (T,)), scale=float(np.float32(1 / np.sqrt(128))), cache=_cache(),
             envelope=(1, 4100), out=_t(na.BF16, (D, Hq, T)))
    a.update(over)
    ws = _WS(ops.gqa_attention_workspace_bytes(Hq, Hkv, D, T, 1, a["envelope"][1]))
    return a, ws


@pytest.mark.parametrize("override,needle", [
    (dict(scale=0.0625), "scale must be 1/sqrt(head_dim)"),
    (dict(q=_t(na.FP32, (128, 40, 4))), "q/out must be BF16"),
    (dict(positions=_t(na.I64, (4,))), "positions must be I32"),
    (dict(positions=_t(na.I32, (5,))), "invalid shape for positions"),
    (dict(envelope=(0, 4100)), "invalid execution envelope"),
    (dict(envelope=(1, 5000)), "invalid execution envelope"),
    (dict(envelope=(1, 3)), "execution envelope is shorter than T"),
    (dict(k=_t(na.BF16, (128, 4, 4))), "invalid shape for k"),
    (dict(q=_t(na.BF16, (128, 36, 4))), "unsupported Q/KV head geometry"),
])
def test_gqa_attention_validation(override, needle):
    a, ws = _attention_args(**override)
    with pytest.raises(ValueError, match=re.escape(needle)):
        ops.gqa_attention(a["q"], a["k"], a["v"], a["positions"], a["scale"], a["cache"], a["envelope"], ws,
                          a["out"])


def test_gqa_attention_prompt_route_limits():
    """T above 32 is the reference's prompt route (gqa_attention.h:59-60, one sequence, causal): a
    batch of several sequences there is NMI_UNSUPPORTED (NotImplementedError), not an invalid
    argument, and so is an ancestor mask above 32 tokens."""
    a, ws = _attention_args(q=_t(na.BF16, (128, 40, 33, 2)), out=_t(na.BF16, (128, 40, 33, 2)),
                            k=_t(na.BF16, (128, 8, 33, 2)), v=_t(na.BF16, (128, 8, 33, 2)),
                            positions=_t(na.I32, (33, 2)))
    with pytest.raises(NotImplementedError, match="prompt route"):
        ops.gqa_attention(a["q"], a["k"], a["v"], a["positions"], a["scale"], a["cache"], a["envelope"], ws,
                          a["out"])
    a, ws = _attention_args(q=_t(na.BF16, (128, 40, 33)), out=_t(na.BF16, (128, 40, 33)),
                            k=_t(na.BF16, (128, 8, 33)), v=_t(na.BF16, (128, 8, 33)), positions=_t(na.I32, (33,)))
    with pytest.raises(NotImplementedError, match="ancestor masks"):
        ops.gqa_attention_tree(a["q"], a["k"], a["v"], a["positions"], _t(na.I32, (33,), 0x40000), a["scale"],
                               a["cache"], a["envelope"], True, ws, a["out"])


def test_prompt_route_workspace_sizes():
    """Above 32 tokens one workspace serves the launches of 32 tokens and the shorter last one."""
    for T, tail in ((33, 1), (64, 0), (100, 4), (4096, 0)):
        want = max(ops.gqa_attention_workspace_bytes(40, 8, 128, 32, 1, 8192),
                   ops.gqa_attention_workspace_bytes(40, 8, 128, tail, 1, 8192) if tail else 0)
        assert ops.gqa_attention_workspace_bytes(40, 8, 128, T, 1, 8192) == want > 0
        bound = max(ops.gqa_attention_workspace_bound(24, 32), ops.gqa_attention_workspace_bound(24, tail) if tail else 0)
        assert ops.gqa_attention_workspace_bound(24, T) == bound > 0
    assert ops.gqa_attention_workspace_bytes(40, 8, 128, 33, 2, 8192) == 0


def _b1_workspace(kv_heads, head_dim, splits):
    """Bytes of a batch-1 plan of one 32-row chunk per KV head: FP16 O [32 x head_dim] and FP32
    (m, l) per row of every (KV head, split) slot, then the 8-byte sequence table, each 256-aligned."""
    up = lambda n: (n + 255) // 256 * 256
    units = kv_heads * splits
    return up(up(up(units * 32 * head_dim * 2) + units * 2 * 32 * 4) + 8)


def test_batch1_plan_avoids_partly_doubled_cus():
    """Batch-1 splits of 256 keys over 40/8 heads: an envelope of 7,684 keys (C2) keeps 31 splits
    (248 workgroups, one per CU); 9,732 keys (C2 plus the round's spare rows) would give 39 splits
    = 312 workgroups, so that 56 CUs hold two, and is planned as 26 splits of 384 keys; 16,384
    keys (64 splits, 512 workgroups, two per CU) and the C3 context (62 splits of 4,224 keys)
    keep their plans."""
    sizes = {env: ops.gqa_attention_workspace_bytes(40, 8, 128, 4, 1, env) for env in (7684, 9732, 16384, 260096)}
    assert sizes[7684] == _b1_workspace(8, 128, 31)
    assert sizes[9732] == _b1_workspace(8, 128, 26)
    assert sizes[16384] == _b1_workspace(8, 128, 64)
    assert sizes[260096] == _b1_workspace(8, 128, 62)


def test_gqa_attention_cache_validation():
    c = _cache()
    c.quant_group = 32
    a, ws = _attention_args(cache=c)
    with pytest.raises(ValueError, match="quant_group 64"):
        ops.gqa_attention(a["q"], a["k"], a["v"], a["positions"], a["scale"], c, a["envelope"], ws, a["out"])
    c = _cache()
    c.padded_context = 4100
    with pytest.raises(ValueError, match="multiple of 128"):
        ops.gqa_attention(a["q"], a["k"], a["v"], a["positions"], a["scale"], c, a["envelope"], ws, a["out"])
    c = _cache()
    c.k_scale = _t(na.BF16, (2, 4224, 8, 1))
    with pytest.raises(ValueError, match="scale dtype"):
        ops.gqa_attention(a["q"], a["k"], a["v"], a["positions"], a["scale"], c, a["envelope"], ws, a["out"])


def test_overflow_error_for_huge_padded_context():
    c = _cache(P=0x80000000, max_ctx=0x7FFFFFFF)
    a, ws = _attention_args(cache=c, envelope=(1, 4100))
    with pytest.raises(OverflowError):
        ops.gqa_attention(a["q"], a["k"], a["v"], a["positions"], a["scale"], c, a["envelope"], ws, a["out"])


def test_workspace_too_small_is_rejected():
    a, _ = _attention_args()
    small = _WS(1024)
    with pytest.raises(ValueError, match="workspace"):
        ops.gqa_attention(a["q"], a["k"], a["v"], a["positions"], a["scale"], a["cache"], a["envelope"], small,
                          a["out"])


def test_workspace_sizing_grows_with_envelope():
    small = ops.gqa_attention_workspace_bytes(40, 8, 128, 4, 1, 8192)
    large = ops.gqa_attention_workspace_bytes(40, 8, 128, 4, 1, 262144)
    assert 0 < small <= large
    assert ops.gqa_attention_workspace_bytes(40, 8, 128, 0, 1, 8192) == 0
    assert ops.sampling_workspace_bytes(248320, 4) > 0


def test_accept_validation():
    K = 3
    args = [_t(na.I32, (K + 1,)), _t(na.BF16, (248320, K + 1)), _t(na.I32, (K,)), _t(na.I32, (1,)),
            _t(na.I32, (1,)), _t(na.I32, (K + 1,)), _t(na.I32, (1,)), _t(na.I32, (1,)), _t(na.I64, (4 + K,))]
    ws = _WS(ops.sampling_workspace_bytes(248320, K + 1))
    with pytest.raises(ValueError, match="token_domain"):
        ops.speculative_accept_greedy_drafts(*args, 248321, 0x1000, ws)
    bad = list(args)
    bad[8] = _t(na.I64, (3 + K,))
    with pytest.raises(ValueError, match="stats"):
        ops.speculative_accept_greedy_drafts(*bad, 248320, 0x1000, ws)
    with pytest.raises(ValueError, match="config must be non-null"):
        ops.speculative_accept_greedy_drafts(*args, 248320, 0, ws)
    bad = list(args)
    bad[2] = _t(na.I32, (0,))
    with pytest.raises(ValueError, match="K must be >=1"):
        ops.speculative_accept_greedy_drafts(*bad, 248320, 0x1000, ws)


def test_mtp_alignment_validation():
    # src/ops/wrapper/mtp_round.cpp:36-48: T in [2,6], I32 contiguous vectors, distinct buffers.
    with pytest.raises(ValueError, match=re.escape("T must be in [2,6]")):
        ops.mtp_prepare_alignment_ids(_t(na.I32, (7,)), _t(na.I32, (1,)), _t(na.I32, (1,)), _t(na.I32, (7,), 0x20000))
    with pytest.raises(ValueError, match=re.escape("T must be in [2,6]")):
        ops.mtp_prepare_alignment_ids(_t(na.I32, (1,)), _t(na.I32, (1,)), _t(na.I32, (1,)), _t(na.I32, (1,), 0x20000))
    with pytest.raises(ValueError, match="alignment_ids"):
        ops.mtp_prepare_alignment_ids(_t(na.I32, (4,)), _t(na.I32, (1,)), _t(na.I32, (1,)), _t(na.I32, (3,), 0x20000))
    with pytest.raises(ValueError, match="token"):
        ops.mtp_prepare_alignment_ids(_t(na.I32, (4,)), _t(na.BF16, (1,)), _t(na.I32, (1,)), _t(na.I32, (4,), 0x20000))
    with pytest.raises(ValueError, match="distinct"):
        ops.mtp_prepare_alignment_ids(_t(na.I32, (4,)), _t(na.I32, (1,)), _t(na.I32, (1,)), _t(na.I32, (4,)))


class _Arena:
    """Distinct fake device addresses, one region per tensor (validation only, nothing launches)."""

    def __init__(self):
        self.at = 0x100000

    def __call__(self, dtype, shape):
        t = _t(dtype, shape, self.at)
        self.at += 0x1000000
        return t


def _gdn_args(arena, S=128, Hqk=16, Hv=48, T=4):
    return dict(q=arena(na.BF16, (S, Hqk, T)), k=arena(na.BF16, (S, Hqk, T)), v=arena(na.BF16, (S, Hv, T)),
                g=arena(na.FP32, (Hv, T)), beta=arena(na.FP32, (Hv, T)), out=arena(na.BF16, (S, Hv, T)))


def test_gdn_validation():
    # src/ops/wrapper/gated_delta_rule.cpp:51-139
    A = _Arena()
    a = _gdn_args(A)
    st = A(na.FP32, (128, 128, 48, 5))
    slot = A(na.I32, (1,))
    sc = 1.0 / np.sqrt(128.0)
    with pytest.raises(ValueError, match="invalid shape for ssm_states snapshot"):
        ops.gated_delta_rule_snapshot(a["q"], a["k"], a["v"], a["g"], a["beta"], sc, True,
                                      A(na.FP32, (128, 128, 48, 3)), slot, a["out"])
    with pytest.raises(ValueError, match="scale must be 1/sqrt"):
        ops.gated_delta_rule_snapshot(a["q"], a["k"], a["v"], a["g"], a["beta"], 0.1, True, st, slot, a["out"])
    with pytest.raises(ValueError, match="head dimension must be 16, 32, 64, or 128"):
        b = _gdn_args(A, S=96)
        ops.gated_delta_rule_snapshot(b["q"], b["k"], b["v"], b["g"], b["beta"], 1 / np.sqrt(96.0), False,
                                      A(na.FP32, (96, 96, 48, 4)), slot, b["out"])
    with pytest.raises(ValueError, match="divisible"):
        b = _gdn_args(A, Hqk=16, Hv=40)
        ops.gated_delta_rule_snapshot(b["q"], b["k"], b["v"], b["g"], b["beta"], sc, False,
                                      A(na.FP32, (128, 128, 40, 4)), slot, b["out"])
    with pytest.raises(ValueError, match="initial_slot"):
        ops.gated_delta_rule_snapshot(a["q"], a["k"], a["v"], a["g"], a["beta"], sc, True, st,
                                      A(na.I64, (1,)), a["out"])
    with pytest.raises(ValueError, match="g"):
        ops.gated_delta_rule_snapshot(a["q"], a["k"], a["v"], A(na.BF16, (48, 4)), a["beta"], sc, True, st, slot,
                                      a["out"])
    with pytest.raises(ValueError, match="ssm_states must not overlap"):
        ops.gated_delta_rule_snapshot(a["q"], a["k"], a["v"], a["g"], a["beta"], sc, True,
                                      _t(na.FP32, (128, 128, 48, 5), a["out"].data), slot, a["out"])
    s0, s1 = A(na.FP32, (128, 128, 48)), A(na.FP32, (128, 128, 48))
    with pytest.raises(ValueError, match="ssm_state_out"):
        ops.gated_delta_rule(a["q"], a["k"], a["v"], a["g"], a["beta"], sc, False, s0, A(na.FP32, (128, 128, 47)),
                             a["out"])
    with pytest.raises(ValueError, match="disjoint or the same storage"):
        ops.gated_delta_rule(a["q"], a["k"], a["v"], a["g"], a["beta"], sc, False, s0,
                             _t(na.FP32, (128, 128, 48), s0.data + 64), a["out"])
    assert ops.gated_delta_rule_workspace_bytes(128, 16, 48, 4096, True) == 0
    with pytest.raises(ValueError, match="invalid geometry"):
        ops.gated_delta_rule_workspace_bytes(128, 16, 40, 4, True)
    del s1


def test_conv_and_scalar_validation():
    # src/ops/wrapper/causal_conv1d_silu.cpp:35-200, src/ops/wrapper/scalar.cpp:11-41
    A = _Arena()
    x, w, out = A(na.BF16, (256, 4)), A(na.BF16, (256, 4)), A(na.BF16, (256, 4))
    slot = A(na.I32, (1,))
    with pytest.raises(ValueError, match=re.escape("conv_states must have shape [C,3,S] with S>=T")):
        ops.causal_conv1d_silu_snapshot(x, w, A(na.BF16, (256, 3, 3)), slot, out)
    with pytest.raises(ValueError, match="weight"):
        ops.causal_conv1d_silu_snapshot(x, A(na.BF16, (256, 3)), A(na.BF16, (256, 3, 4)), slot, out)
    with pytest.raises(ValueError, match="out"):
        ops.causal_conv1d_silu_snapshot(x, w, A(na.BF16, (256, 3, 4)), slot, A(na.BF16, (256, 5)))
    with pytest.raises(ValueError, match="conv_state_out"):
        ops.causal_conv1d_silu(x, w, A(na.BF16, (256, 3)), A(na.BF16, (255, 3)), out)
    with pytest.raises(ValueError, match="x"):
        ops.causal_conv1d_silu(A(na.FP32, (256, 4)), w, A(na.BF16, (256, 3)), A(na.BF16, (256, 3)), out)
    s = A(na.I32, (1,))
    with pytest.raises(ValueError, match="must not alias"):
        ops.assign_i32_scalar(s, s)
    with pytest.raises(ValueError, match="non-null contiguous scalar"):
        ops.set_i32_scalar(A(na.I32, (2,)), 3)
    with pytest.raises(ValueError, match="non-null contiguous scalar"):
        ops.increment_i64_scalar(A(na.I32, (1,)))


def _q6_weight(n=248320, k=5120, base=0x10000000):
    G = (k + 127) // 128 * 2
    nb, hb, sb = n * G * 32, n * G * 16, n * G * 2
    hoff = (nb + 255) // 256 * 256
    soff = hoff + (hb + 255) // 256 * 256
    w = na.Weight()
    w.payload, w.payload_bytes, w.high_plane_bytes = base, soff + sb, hb
    w.qtype, w.group_size, w.ndim = 2, 64, 2
    w.shape[:] = [n, k, 1, 1]
    w.padded_shape[:] = [n, G * 64, 1, 1]
    w.qdata, w.qhigh, w.scales = base, base + hoff, base + soff
    w.n, w.k, w.group, w.layout, w.scale_dtype = n, k, 64, 0, na.FP16
    return w


def test_linear_validation():
    # src/ops/linear/linear.cpp:65-152 and the Q6 alignment rule :200-209
    x, out = _t(na.BF16, (5120, 4), 0x100000), _t(na.BF16, (248320, 4), 0x200000)
    w = _q6_weight()
    w.payload_bytes -= 1
    with pytest.raises(ValueError, match="payload is too small"):
        ops.linear(x, w, out)
    w = _q6_weight()
    w.padded_shape[1] = 5248
    with pytest.raises(ValueError, match="padded shape is invalid"):
        ops.linear(x, w, out)
    w = _q6_weight()
    w.qtype = 0
    with pytest.raises(ValueError, match="only Q6G64_F16S"):
        ops.linear(x, w, out)
    w = _q6_weight()
    w.scales += 2
    with pytest.raises(ValueError, match="alignment"):
        ops.linear(x, w, out)
    with pytest.raises(ValueError, match="x K dimension"):
        ops.linear(_t(na.BF16, (2048, 4), 0x100000), _q6_weight(), out)
    with pytest.raises(ValueError, match="out must have shape"):
        ops.linear(x, _q6_weight(), _t(na.BF16, (248320, 3), 0x200000))
    w = _q6_weight(k=16384)
    with pytest.raises(NotImplementedError, match="padded K <= 8192"):
        ops.linear(_t(na.BF16, (16384, 4), 0x100000), w, out)
    ws = _WS(ops.linear_argmax_workspace_bytes(4))
    with pytest.raises(ValueError, match="valid_rows"):
        ops.linear_argmax(x, _q6_weight(), 248321, ws, _t(na.I32, (4,), 0x300000))
    with pytest.raises(ValueError, match="workspace"):
        ops.linear_argmax(x, _q6_weight(), 248320, _WS(1024), _t(na.I32, (4,), 0x300000))
    with pytest.raises(ValueError, match="I32"):
        ops.linear_argmax(x, _q6_weight(), 248320, ws, _t(na.BF16, (4,), 0x300000))


def test_fused_head_rejects_strided_batch():
    """The fused lm_head + acceptance reads the (K+1) * B hidden columns as one packed operand: an x
    whose batch stride is not the packed one (the first K+1 columns of a wider hidden buffer) is
    rejected before any launch, as is a packed x with a wrong column count."""
    K, B = 3, 2
    state = [_t(na.I32, (K, B)), _t(na.I32, (B,)), _t(na.I32, (B,)), _t(na.I32, (K + 1, B)),
             _t(na.I32, (B,)), _t(na.I32, (B,)), _t(na.I64, (4 + K, B))]
    ws = _WS(ops.speculative_accept_fused_head_workspace_bytes(K, B))
    x = _t(na.BF16, (5120, K + 1, B), 0x100000)
    x.nb[2] = x.nb[1] * 16  # columns 0..K of a [5120, 16, B] buffer
    with pytest.raises(ValueError, match="x must be contiguous"):
        ops.speculative_accept_fused_head(x, _q6_weight(), *state, 248320, 0x1000, ws)
    with pytest.raises(ValueError, match="x must be"):
        ops.speculative_accept_fused_head(_t(na.BF16, (5120, K, B), 0x100000), _q6_weight(), *state, 248320, 0x1000, ws)


def test_argmax_validation():
    with pytest.raises(ValueError, match="valid_rows"):
        ops.argmax(_t(na.BF16, (100, 4)), _t(na.I32, (4,)), 101)
    with pytest.raises(ValueError, match="out shape"):
        ops.argmax(_t(na.BF16, (100, 4)), _t(na.I32, (3,)), 100)
    with pytest.raises(ValueError, match="logits must be BF16"):
        ops.argmax(_t(na.FP32, (100, 4)), _t(na.I32, (4,)), 100)


def test_commit_validation():
    k = _t(na.BF16, (128, 8, 4))
    with pytest.raises(ValueError, match="invalid execution envelope"):
        ops.kv_cache_append_prefix(k, k, _t(na.I32, (4,)), _t(na.I32, (1,)), (0, 5), _cache())
    with pytest.raises(ValueError, match="commit_count"):
        ops.kv_cache_append_prefix(k, k, _t(na.I32, (4,)), _t(na.I32, (2,)), (0, 4), _cache())
    with pytest.raises(ValueError, match="path capacity"):
        ops.kv_cache_compact_path(_t(na.I32, (1,)), _t(na.I32, (40,)), _t(na.I32, (1,)), _cache())


def test_sampling_config_layout_matches_reference():
    """SamplingConfig is device-resident and shared with reference callers: same 40-byte layout
    (include/ninfer/ops/sampling.h:24-33)."""
    assert C.sizeof(na.SamplingConfig) == 40
    assert na.SamplingConfig.seed.offset == 24 and na.SamplingConfig.token_counts.offset == 32


def test_dtype_values_match_reference_enum():
    """nmi_dtype carries ninfer::DType's values (src/core/dtype.h:8-16), so a reference-side
    binding converts a Tensor's dtype with a cast."""
    assert (na.BF16, na.FP32, na.I32, na.U8, na.I64, na.I8, na.FP16) == (0, 1, 2, 3, 4, 5, 6)
    hdr = (ROOT / "include" / "ninfer_amd.h").read_text()
    for name, val in (("NMI_BF16", 0), ("NMI_FP32", 1), ("NMI_I32", 2), ("NMI_U8", 3), ("NMI_I64", 4),
                      ("NMI_I8", 5), ("NMI_FP16", 6)):
        assert re.search(rf"\b{name} = {val}\b", hdr), name


def _general_args(K=3, B=1, V=248320, **over):
    a = dict(logits=_t(na.BF16, (V, K + 1, B)), draft=_t(na.BF16, (V, K, B)), drafts=_t(na.I32, (K, B)),
             ua=_t(na.FP32, (K + 1, B)), ur=_t(na.FP32, (1, B)), length=_t(na.I32, (B,)), token=_t(na.I32, (B,)),
             so=_t(na.I32, (K + 1, B)), ns=_t(na.I32, (B,)), acc=_t(na.I32, (B,)), stats=_t(na.I64, (4 + K, B)))
    a.update(over)
    return a


def _call_general(a, V=248320, ws=None, cfg=0x1000):
    K = a["drafts"].ne[0]
    ws = ws or _WS(ops.general_accept_workspace_bytes(V, max(K, 1), a["drafts"].ne[1]))
    ops.speculative_accept_general(a["logits"], a["draft"], a["drafts"], a["ua"], a["ur"], a["length"], a["token"],
                                   a["so"], a["ns"], a["acc"], a["stats"], V, cfg, ws)


@pytest.mark.parametrize("override,needle", [
    (dict(ua=_t(na.FP32, (3, 1))), "invalid vector shape for u_accept"),
    (dict(ur=_t(na.I32, (1, 1))), "invalid dtype for u_residual"),
    (dict(draft=_t(na.BF16, (248320, 2, 1))), "draft_logits must be"),
    (dict(logits=_t(na.FP32, (248320, 4, 1))), "invalid dtype for logits"),
    (dict(stats=_t(na.I64, (6, 1))), "invalid vector shape for stats"),
])
def test_general_accept_validation(override, needle):
    with pytest.raises(ValueError, match=re.escape(needle)):
        _call_general(_general_args(**override))


def test_general_accept_limits():
    with pytest.raises(ValueError, match="config must be non-null"):
        _call_general(_general_args(), cfg=0)
    with pytest.raises(ValueError, match="workspace"):
        _call_general(_general_args(), ws=_WS(1024))
    big = 1 << 21
    with pytest.raises(ValueError, match="exceeds 1048576"):
        _call_general(_general_args(V=big), V=big, ws=_WS(1 << 20))
    assert ops.general_accept_workspace_bytes(248320, 3, 16) > 0
    assert ops.general_accept_workspace_bytes(big, 3, 1) == 0


# ---- reference-signature workspace query, plane limits, cyclic commit validation -------------------

@pytest.mark.parametrize("q_heads,kv_heads,head_dim", [(40, 8, 128), (24, 4, 256), (16, 2, 256)])
def test_workspace_bound_covers_every_envelope(q_heads, kv_heads, head_dim):
    """gqa_attention_workspace_bytes(q_heads, tokens) (gqa_attention.h:50) is at least the exact size of
    every batch-1 envelope, and equals the largest of them."""
    for T in (1, 2, 4, 6, 7, 16, 32):
        bound = ops.gqa_attention_workspace_bound(q_heads, T)
        sizes = [ops.gqa_attention_workspace_bytes(q_heads, kv_heads, head_dim, T, 1, keys)
                 for keys in list(range(1, 4096, 61)) + [2 ** k + d for k in range(12, 31) for d in (-1, 0, 77)]]
        assert max(sizes) <= bound and bound in sizes, (T, bound, max(sizes))


def test_static_scratch_holds_every_batch1_plan():
    """The allocation-free entry's 16 MiB static scratch holds the largest batch-1 plan of every
    registered geometry and T <= 32 (5.2 MiB: the 80-row form at 40/8 heads, T = 16)."""
    worst = max(ops.gqa_attention_workspace_bound(qh, T) for qh in (40, 24, 16) for T in range(1, 33))
    assert worst == ops.gqa_attention_workspace_bound(40, 16)
    assert 5 << 20 < worst <= 16 << 20


def test_workspace_bound_reference_call_shapes():
    """The reference sizes its arenas with gqa_attention_workspace_bytes(query_heads, tokens)
    (src/targets/qwen3_6/impl/runtime/layouts_impl.h:152,253,286), including prefill token counts."""
    assert ops.gqa_attention_workspace_bound(24, 1) > 0
    assert ops.gqa_attention_workspace_bound(16, 4) > 0
    assert ops.gqa_attention_workspace_bound(40, 0) == 0
    assert ops.gqa_attention_workspace_bound(24, 4096) == ops.gqa_attention_workspace_bound(24, 32)  # prompt route
    with pytest.raises(ValueError, match="unsupported Q/KV head geometry"):
        ops.gqa_attention_workspace_bound(36, 4)


def test_head_plane_of_2_31_bytes_is_unsupported():
    """Kernels address a KV head's plane with 32-bit offsets: P * D * element bytes >= 2^31 is rejected
    before any launch instead of reading wrong rows."""
    P = 1 << 24  # INT8 at head_dim 128: exactly 2^31 bytes per plane
    c = _cache(P=P, max_ctx=P - 8)
    a, ws = _attention_args(cache=c, envelope=(1, 4100))
    with pytest.raises(NotImplementedError, match="2\\^31"):
        ops.gqa_attention(a["q"], a["k"], a["v"], a["positions"], a["scale"], c, a["envelope"], ws, a["out"])
    c = _cache(P=P - 128, max_ctx=P - 200)
    a, ws = _attention_args(cache=c, envelope=(1, 4100))
    with pytest.raises(ValueError, match="workspace"):  # passes the plane check, fails later on the host
        ops.gqa_attention(a["q"], a["k"], a["v"], a["positions"], a["scale"], c, a["envelope"], _WS(16), a["out"])


def _cyclic(cap=4096, padded=4096, dtype=None):
    v = na.CyclicKVLayerView()
    dtype = na.BF16 if dtype is None else dtype
    v.k = _t(dtype, (128, padded, 8))
    v.v = _t(dtype, (128, padded, 8))
    v.k_scale = _t(na.FP16, (1,), ptr=0)
    v.v_scale = _t(na.FP16, (1,), ptr=0)
    v.capacity, v.padded_capacity, v.num_kv_heads, v.head_dim = cap, padded, 8, 128
    v.dtype, v.quant_group = dtype, 0
    return v


def test_cyclic_commit_validation():
    k = _t(na.BF16, (128, 8, 4))
    pos, cnt = _t(na.I32, (4,)), _t(na.I32, (1,))
    with pytest.raises(ValueError, match="invalid cyclic cache"):
        ops.kv_cache_append_prefix_cyclic(k, k, pos, cnt, (0, 4), _cyclic(cap=3000, padded=3072))
    with pytest.raises(ValueError, match="invalid cyclic cache"):
        ops.kv_cache_append_prefix_cyclic(k, k, pos, cnt, (0, 4), _cyclic(padded=2048))
    with pytest.raises(ValueError, match="invalid execution envelope"):
        ops.kv_cache_append_prefix_cyclic(k, k, pos, cnt, (3, 2), _cyclic())
    with pytest.raises(ValueError, match="16-byte aligned"):
        kk = _t(na.BF16, (128, 8, 4), ptr=0x10002)
        ops.kv_cache_append_prefix_cyclic(kk, kk, pos, cnt, (0, 4), _cyclic())
    with pytest.raises(ValueError, match="must not have scales"):
        c = _cyclic()
        c.k_scale = _t(na.FP16, (1,))
        ops.kv_cache_append_prefix_cyclic(k, k, pos, cnt, (0, 4), c)
    # the cache planes too (reference require_vector_aligned(cache.k/v))
    for plane in ("k", "v"):
        c = _cyclic()
        setattr(c, plane, _t(na.BF16, (128, 4096, 8), ptr=0x20008))
        with pytest.raises(ValueError, match=f"cache {plane} must be 16-byte aligned"):
            ops.kv_cache_append_prefix_cyclic(k, k, pos, cnt, (0, 4), c)


def _driver():
    """The compiled ops.hpp driver (tests/cpp), built by __graft_entry__.build(); rebuilt here if absent."""
    import subprocess
    exe = ROOT / "tests" / "cpp" / "ops_hpp_driver"
    if not exe.exists():
        subprocess.run(["make", "-s", "-C", str(exe.parent)], check=True)
    return exe


def test_compiled_cpp_layer_maps_statuses_to_reference_exceptions():
    """include/ninfer_amd/ops.hpp compiled by hipcc as a reference caller would compile it: the
    (q_heads, tokens) workspace query of layouts_impl.h:152, std::invalid_argument /
    std::overflow_error from host validation, and std::runtime_error for a batch on the prompt route."""
    import subprocess
    r = subprocess.run([str(_driver()), "errors"], capture_output=True, text=True, timeout=60)
    print(r.stdout)
    assert r.returncode == 0 and "ERRORS PASS" in r.stdout, r.stdout + r.stderr


def test_runtime_helper_validation():
    L = lib()
    fake = C.c_void_p(1 << 20)
    # host checks reject before any launch
    assert L.nmi_rt_stream_copy(fake, fake, 17, None) == INVALID_ARGUMENT
    assert L.nmi_rt_stream_copy(None, fake, 16, None) == INVALID_ARGUMENT
    assert L.nmi_rt_read_ceiling(fake, 24, 0, fake, None) == INVALID_ARGUMENT
    assert L.nmi_rt_read_ceiling(fake, 32, 7, fake, None) == INVALID_ARGUMENT
    assert L.nmi_rt_next_row_i32(None, 4, 3, fake, fake, None) == INVALID_ARGUMENT
    assert L.nmi_rt_next_row_i32(fake, 0, 3, fake, fake, None) == INVALID_ARGUMENT
    assert L.nmi_rt_next_row_i32(fake, 4, 1025, fake, fake, None) == INVALID_ARGUMENT
