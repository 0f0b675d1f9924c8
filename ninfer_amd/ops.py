"""Python mirror of the reference op surface for the verify step (ninfer::ops).

Same names, argument meaning and error behaviour as include/ninfer/ops/*.h: invalid shapes or
dtypes raise ValueError (std::invalid_argument), int32 overflow raises OverflowError
(std::overflow_error). Tensors are nmi_tensor views (see ninfer_amd.device.DeviceArray.tensor()),
streams are ninfer_amd.device.Stream or None, workspaces are DeviceBuffer regions sized by the
*_workspace_bytes queries. Every call launches hand-written gfx950 kernels through the C ABI.
"""
from __future__ import annotations

import ctypes as C

from . import _capi
from ._capi import CommitEnvelope, GqaEnvelope, Tensor, check, lib


def _s(stream):
    return stream.handle if stream is not None else None


def _ws(workspace):
    if workspace is None:
        return None, 0
    return C.c_void_p(workspace.ptr), workspace.nbytes


def _p(t: Tensor | None):
    return C.byref(t) if t is not None else None


# ---- verify attention (include/ninfer/ops/gqa_attention.h) -------------------------------------

def gqa_attention_workspace_bytes(q_heads: int, kv_heads: int, head_dim: int, tokens: int,
                                  batch: int, max_visible_keys: int) -> int:
    return int(lib().nmi_gqa_attention_workspace_bytes(q_heads, kv_heads, head_dim, tokens, batch, max_visible_keys))


def gqa_attention_workspace_bound(q_heads: int, tokens: int) -> int:
    """gqa_attention_workspace_bytes(q_heads, tokens) with the reference signature
    (gqa_attention.h:50): enough for every envelope of one sequence."""
    n = C.c_size_t(0)
    check(lib().nmi_gqa_attention_workspace_bound(int(q_heads), int(tokens), C.byref(n)))
    return int(n.value)


def gqa_attention(q, k, v, positions, scale, cache, envelope, workspace, out, stream=None) -> None:
    """A1: quantize-append k/v at `positions`, then causal GQA (gqa_attention.h:71-73)."""
    ws, nb = _ws(workspace)
    check(lib().nmi_gqa_attention(_p(q), _p(k), _p(v), _p(positions), float(scale), C.byref(cache),
                                  GqaEnvelope(*envelope), ws, nb, _p(out), _s(stream)))


def gqa_attention_noalloc(q, k, v, positions, scale, cache, envelope, out, stream=None) -> None:
    """A1 with the split partials in the library's static per-device scratch: allocates nothing,
    takes no workspace (no reference counterpart; for callers that cannot allocate)."""
    check(lib().nmi_gqa_attention_noalloc(_p(q), _p(k), _p(v), _p(positions), float(scale), C.byref(cache),
                                          GqaEnvelope(*envelope), _p(out), _s(stream)))


def gqa_kv_append(k, v, positions, cache, stream=None) -> None:
    """A2 (gqa_attention.h:80-81)."""
    check(lib().nmi_gqa_kv_append(_p(k), _p(v), _p(positions), C.byref(cache), _s(stream)))


def gqa_attention_cached(q, positions, scale, cache, envelope, workspace, out, stream=None) -> None:
    """A3 (gqa_attention.h:89-91)."""
    ws, nb = _ws(workspace)
    check(lib().nmi_gqa_attention_cached(_p(q), _p(positions), float(scale), C.byref(cache),
                                         GqaEnvelope(*envelope), ws, nb, _p(out), _s(stream)))


def gqa_attention_tree(q, k, v, positions, parents, scale, cache, envelope, write_cache, workspace,
                       out, stream=None) -> None:
    """Tree verification attention with an ancestor mask (extension)."""
    ws, nb = _ws(workspace)
    check(lib().nmi_gqa_attention_tree(_p(q), _p(k), _p(v), _p(positions), _p(parents), float(scale),
                                       C.byref(cache), GqaEnvelope(*envelope), int(bool(write_cache)),
                                       ws, nb, _p(out), _s(stream)))


# ---- acceptance (argmax.h, sampling.h, speculative_round.h) ------------------------------------

def argmax(logits, out, valid_rows: int, stream=None) -> None:
    check(lib().nmi_argmax(_p(logits), _p(out), int(valid_rows), _s(stream)))


def sampling_workspace_bytes(token_domain: int, columns: int, batch: int = 1) -> int:
    return int(lib().nmi_sampling_workspace_bytes(token_domain, columns, batch))


def speculative_prepare_verify_inputs(token, drafts, length, verify_ids, positions, stream=None) -> None:
    check(lib().nmi_speculative_prepare_verify_inputs(_p(token), _p(drafts), _p(length), _p(verify_ids),
                                                      _p(positions), _s(stream)))


def speculative_accept_greedy_drafts(target_tokens, logits, drafts, length, token, sampled_out,
                                     num_sampled, accepted, stats, token_domain: int, config_ptr: int,
                                     workspace, stream=None) -> None:
    """Greedy or reference-stochastic acceptance; `config_ptr` addresses device SamplingConfig[B]."""
    ws, nb = _ws(workspace)
    check(lib().nmi_speculative_accept_greedy_drafts(
        _p(target_tokens), _p(logits), _p(drafts), _p(length), _p(token), _p(sampled_out),
        _p(num_sampled), _p(accepted), _p(stats), int(token_domain), C.c_void_p(config_ptr), ws, nb,
        _s(stream)))


def general_accept_workspace_bytes(token_domain: int, K: int, batch: int = 1) -> int:
    return int(lib().nmi_general_accept_workspace_bytes(token_domain, K, batch))


def speculative_accept_general(logits, draft_logits, drafts, u_accept, u_residual, length, token,
                               sampled_out, num_sampled, accepted, stats, token_domain: int,
                               config_ptr: int, workspace, stream=None) -> None:
    """min(1, p/q) acceptance with normalized max(0, p - q) resampling (extension)."""
    ws, nb = _ws(workspace)
    check(lib().nmi_speculative_accept_general(
        _p(logits), _p(draft_logits), _p(drafts), _p(u_accept), _p(u_residual), _p(length), _p(token),
        _p(sampled_out), _p(num_sampled), _p(accepted), _p(stats), int(token_domain),
        C.c_void_p(config_ptr), ws, nb, _s(stream)))


def speculative_select_accepted_hidden(hidden, accepted, out, stream=None) -> None:
    check(lib().nmi_speculative_select_accepted_hidden(_p(hidden), _p(accepted), _p(out), _s(stream)))


def mtp_prepare_alignment_ids(verify_ids, token, accepted, alignment_ids, stream=None) -> None:
    """include/ninfer/ops/mtp_round.h:19-20."""
    check(lib().nmi_mtp_prepare_alignment_ids(_p(verify_ids), _p(token), _p(accepted), _p(alignment_ids), _s(stream)))


def tree_accept_greedy(parents, node_tokens, target_tokens, path, path_len, length, token,
                       sampled_out, num_sampled, accepted, stats, stream=None) -> None:
    check(lib().nmi_tree_accept_greedy(_p(parents), _p(node_tokens), _p(target_tokens), _p(path),
                                       _p(path_len), _p(length), _p(token), _p(sampled_out),
                                       _p(num_sampled), _p(accepted), _p(stats), _s(stream)))


# ---- lm_head (linear.h + the fused linear -> argmax) ----------------------------------------------

def linear(x, weight, out, stream=None) -> None:
    """include/ninfer/ops/linear.h:27 (Q6G64_F16S RowSplit weights)."""
    check(lib().nmi_linear(_p(x), C.byref(weight), _p(out), _s(stream)))


def linear_argmax_workspace_bytes(tokens) -> int:
    return lib().nmi_linear_argmax_workspace_bytes(tokens)


def linear_argmax(x, weight, valid_rows, ws, out, stream=None) -> None:
    """Fused linear -> argmax (the reference's deferred FUT-F03 contract)."""
    check(lib().nmi_linear_argmax(_p(x), C.byref(weight), int(valid_rows), C.c_void_p(ws.ptr), ws.nbytes, _p(out),
                                  _s(stream)))


def speculative_accept_fused_head_workspace_bytes(K: int, batch: int = 1) -> int:
    return int(lib().nmi_speculative_accept_fused_head_workspace_bytes(K, batch))


def speculative_accept_fused_head(x, weight, drafts, length, token, sampled_out, num_sampled, accepted, stats,
                                  token_domain: int, config_ptr: int, workspace, stream=None) -> None:
    """lm_head (Q6G64 linear) + speculative_accept_greedy_drafts in one call, the logits never written:
    x BF16 [hidden, K+1, B]; `config_ptr` addresses device SamplingConfig[B]."""
    ws, nb = _ws(workspace)
    check(lib().nmi_speculative_accept_fused_head(
        _p(x), C.byref(weight), _p(drafts), _p(length), _p(token), _p(sampled_out), _p(num_sampled), _p(accepted),
        _p(stats), int(token_domain), C.c_void_p(config_ptr), ws, nb, _s(stream)))


# ---- recurrent state of the hybrid layers (gated_delta_rule.h, causal_conv1d_silu.h, scalar.h) --

def gated_delta_rule_workspace_bytes(head_dim, qk_heads, value_heads, tokens, normalize_qk) -> int:
    """include/ninfer/ops/gated_delta_rule.h:18-21 (raises ValueError on an invalid geometry)."""
    import ctypes as C
    n = C.c_size_t(0)
    check(lib().nmi_gated_delta_rule_workspace_bytes(head_dim, qk_heads, value_heads, tokens,
                                                     1 if normalize_qk else 0, C.byref(n)))
    return n.value


def gated_delta_rule(q, k, v, g, beta, scale, normalize_qk, ssm_state_in, ssm_state_out, out,
                     stream=None) -> None:
    """include/ninfer/ops/gated_delta_rule.h:41-55; pass the same tensor twice for the in-place form."""
    check(lib().nmi_gated_delta_rule(_p(q), _p(k), _p(v), _p(g), _p(beta), scale, 1 if normalize_qk else 0,
                                     _p(ssm_state_in), _p(ssm_state_out), _p(out), _s(stream)))


def gated_delta_rule_snapshot(q, k, v, g, beta, scale, normalize_qk, ssm_states, initial_slot, out,
                              stream=None) -> None:
    """include/ninfer/ops/gated_delta_rule.h:57-68."""
    check(lib().nmi_gated_delta_rule_snapshot(_p(q), _p(k), _p(v), _p(g), _p(beta), scale,
                                              1 if normalize_qk else 0, _p(ssm_states), _p(initial_slot),
                                              _p(out), _s(stream)))


def causal_conv1d_silu(x, weight, conv_state_in, conv_state_out, out, stream=None) -> None:
    """include/ninfer/ops/causal_conv1d_silu.h:23-31; pass the same tensor twice for the in-place form."""
    check(lib().nmi_causal_conv1d_silu(_p(x), _p(weight), _p(conv_state_in), _p(conv_state_out), _p(out),
                                       _s(stream)))


def causal_conv1d_silu_snapshot(x, weight, conv_states, initial_slot, out, stream=None) -> None:
    """include/ninfer/ops/causal_conv1d_silu.h:33-40."""
    check(lib().nmi_causal_conv1d_silu_snapshot(_p(x), _p(weight), _p(conv_states), _p(initial_slot), _p(out),
                                                _s(stream)))


def set_i32_scalar(destination, value, stream=None) -> None:
    check(lib().nmi_set_i32_scalar(_p(destination), value, _s(stream)))


def assign_i32_scalar(source, destination, stream=None) -> None:
    check(lib().nmi_assign_i32_scalar(_p(source), _p(destination), _s(stream)))


def increment_i32_scalar(scalar, stream=None) -> None:
    check(lib().nmi_increment_i32_scalar(_p(scalar), _s(stream)))


def increment_i64_scalar(scalar, stream=None) -> None:
    check(lib().nmi_increment_i64_scalar(_p(scalar), _s(stream)))


# ---- commit / rollback (kv_cache_append_prefix.h + extensions) ----------------------------------

def kv_cache_append_prefix(k, v, positions, commit_count, envelope, cache, stream=None) -> None:
    check(lib().nmi_kv_cache_append_prefix(_p(k), _p(v), _p(positions), _p(commit_count),
                                           CommitEnvelope(*envelope), C.byref(cache), _s(stream)))


def kv_cache_append_prefix_cyclic(k, v, positions, commit_count, envelope, cache, stream=None) -> None:
    """The cyclic overload (kv_cache_append_prefix.h:40-51): row = position % capacity."""
    check(lib().nmi_kv_cache_append_prefix_cyclic(_p(k), _p(v), _p(positions), _p(commit_count),
                                                  CommitEnvelope(*envelope), C.byref(cache), _s(stream)))


def kv_cache_rollback(positions, keep_count, cache, stream=None) -> None:
    check(lib().nmi_kv_cache_rollback(_p(positions), _p(keep_count), C.byref(cache), _s(stream)))


def kv_cache_compact_path(base_position, path, path_len, cache, stream=None) -> None:
    check(lib().nmi_kv_cache_compact_path(_p(base_position), _p(path), _p(path_len), C.byref(cache),
                                          _s(stream)))
