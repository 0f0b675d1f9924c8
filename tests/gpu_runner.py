"""Drive the product library on the GPU for tests (inputs from numpy, results back to numpy)."""
from __future__ import annotations

import numpy as np

import ninfer_amd as na
from ninfer_amd import ops
from ninfer_amd.device import DeviceArray, DeviceBuffer, Stream
from ninfer_amd.kv_cache import KVCacheLayer


def upload_cache(case) -> KVCacheLayer:
    dtype = na.BF16 if getattr(case, "kv", "i8") == "bf16" else na.I8
    cache = KVCacheLayer(case.max_context, case.Hkv, case.D, case.B, dtype=dtype)
    cache.upload(*case.cache_planes())
    return cache


def run_attention(case, out_f32=False, mode="A1", cache=None, stream=None, envelope=None):
    """mode: A1 (append + attend), A3 (attend only; caller appended), TREE (A1 with parents)."""
    D, Hq, Hkv, T, B = case.D, case.Hq, case.Hkv, case.T, case.B
    cache = cache or upload_cache(case)
    q = DeviceArray.from_numpy(na.BF16, case.q, (D, Hq, T, B))
    k = DeviceArray.from_numpy(na.BF16, case.k_new, (D, Hkv, T, B))
    v = DeviceArray.from_numpy(na.BF16, case.v_new, (D, Hkv, T, B))
    pos = DeviceArray.from_numpy(na.I32, case.positions, (T, B))
    out = DeviceArray(na.FP32 if out_f32 else na.BF16, (D, Hq, T, B))
    # default: from the shortest window the case holds up to its capacity (an exact envelope when
    # max_context is the window, as for the reference's eager calls)
    env = envelope or (min(case.Ls) + T, case.max_context)
    ws = DeviceBuffer(ops.gqa_attention_workspace_bytes(Hq, Hkv, D, T, B, env[1]))
    ws.fill(0xFF)  # NaN bit patterns: the op may not depend on what scratch held before
    view = cache.view()
    if mode == "A1":
        ops.gqa_attention(q.tensor(), k.tensor(), v.tensor(), pos.tensor(), case.scale, view, env, ws,
                          out.tensor(), stream)
    elif mode == "A3":
        ops.gqa_attention_cached(q.tensor(), pos.tensor(), case.scale, view, env, ws, out.tensor(), stream)
    elif mode == "TREE":
        par = DeviceArray.from_numpy(na.I32, np.asarray(case.parents, dtype=np.int32), (T, B))
        ops.gqa_attention_tree(q.tensor(), k.tensor(), v.tensor(), pos.tensor(), par.tensor(), case.scale,
                               view, env, True, ws, out.tensor(), stream)
    else:
        raise ValueError(mode)
    if stream is not None:
        stream.synchronize()
    from ninfer_amd.device import synchronize
    synchronize()
    raw = out.numpy()
    if out_f32:
        res = raw.astype(np.float64)
    else:
        res = (raw.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return res, cache


def append(case, cache, stream=None):
    D, Hkv, T, B = case.D, case.Hkv, case.T, case.B
    k = DeviceArray.from_numpy(na.BF16, case.k_new, (D, Hkv, T, B))
    v = DeviceArray.from_numpy(na.BF16, case.v_new, (D, Hkv, T, B))
    pos = DeviceArray.from_numpy(na.I32, case.positions, (T, B))
    ops.gqa_kv_append(k.tensor(), v.tensor(), pos.tensor(), cache.view(), stream)
    from ninfer_amd.device import synchronize
    synchronize()


def upload_configs(cfgs, token_counts=None):
    """Device SamplingConfig[B]; token_counts (numpy int32 [V] per sequence) become device arrays."""
    import ctypes as C
    keep = []
    blob = bytearray()
    for b, cfg in enumerate(cfgs):
        c = na.SamplingConfig()
        C.memmove(C.addressof(c), C.addressof(cfg), C.sizeof(c))
        if token_counts is not None and token_counts[b] is not None:
            tc = DeviceArray.from_numpy(na.I32, np.asarray(token_counts[b], dtype=np.int32))
            keep.append(tc)
            c.token_counts = tc.ptr
        blob += bytes(memoryview(c))
    buf = DeviceBuffer(len(blob))
    buf.upload(np.frombuffer(bytes(blob), dtype=np.uint8))
    return buf, keep


def run_accept(logits, drafts, length, stats, token_domain, cfgs, target_tokens=None, token_counts=None,
               physical_rows=None):
    """Batch acceptance. logits: uint16 [B][C][rows]; drafts int32 [B][K]; length int32 [B]."""
    logits = np.asarray(logits, dtype=np.uint16)
    B, Ccols, rows = logits.shape
    drafts = np.asarray(drafts, dtype=np.int32).reshape(B, -1)
    K = drafts.shape[1]
    stats = np.asarray(stats, dtype=np.int64).reshape(B, -1)
    if target_tokens is None:
        target_tokens = np.zeros((B, K + 1), dtype=np.int32)
    d_logits = DeviceArray.from_numpy(na.BF16, logits, (rows, Ccols, B))
    d_drafts = DeviceArray.from_numpy(na.I32, drafts, (K, B))
    d_target = DeviceArray.from_numpy(na.I32, np.asarray(target_tokens, dtype=np.int32), (K + 1, B))
    d_len = DeviceArray.from_numpy(na.I32, np.asarray(length, dtype=np.int32), (B,))
    d_tok = DeviceArray.from_numpy(na.I32, np.full(B, -1, dtype=np.int32), (B,))
    d_so = DeviceArray.from_numpy(na.I32, np.full((B, K + 1), -7, dtype=np.int32), (K + 1, B))
    d_ns = DeviceArray.from_numpy(na.I32, np.zeros(B, dtype=np.int32), (B,))
    d_acc = DeviceArray.from_numpy(na.I32, np.zeros(B, dtype=np.int32), (B,))
    d_stats = DeviceArray.from_numpy(na.I64, stats, (stats.shape[1], B))
    cfg_buf, keep = upload_configs(cfgs, token_counts)
    ws = DeviceBuffer(max(256, ops.sampling_workspace_bytes(token_domain, K + 1, B)))
    ops.speculative_accept_greedy_drafts(d_target.tensor(), d_logits.tensor(), d_drafts.tensor(), d_len.tensor(),
                                         d_tok.tensor(), d_so.tensor(), d_ns.tensor(), d_acc.tensor(),
                                         d_stats.tensor(), token_domain, cfg_buf.ptr, ws)
    from ninfer_amd.device import synchronize
    synchronize()
    out = dict(sampled_out=d_so.numpy().reshape(B, K + 1), num_sampled=d_ns.numpy(), accepted=d_acc.numpy(),
               token=d_tok.numpy(), length=d_len.numpy(), stats=d_stats.numpy().reshape(B, -1))
    out["token_counts"] = [tc.numpy() for tc in keep] if keep else None
    return out


def run_general(target, draft, drafts, u_accept, u_residual, length, stats, token_domain, temperature, top_p):
    """Mode F batch acceptance. target uint16 [B][K+1][rows]; draft uint16 [B][K][rows]."""
    target = np.asarray(target, dtype=np.uint16)
    draft = np.asarray(draft, dtype=np.uint16)
    B, Kp1, rows = target.shape
    K = Kp1 - 1
    drafts = np.asarray(drafts, dtype=np.int32).reshape(B, K)
    stats = np.asarray(stats, dtype=np.int64).reshape(B, -1)
    d_t = DeviceArray.from_numpy(na.BF16, target, (rows, K + 1, B))
    d_d = DeviceArray.from_numpy(na.BF16, draft, (rows, K, B))
    d_dr = DeviceArray.from_numpy(na.I32, drafts, (K, B))
    d_ua = DeviceArray.from_numpy(na.FP32, np.asarray(u_accept, dtype=np.float32).reshape(B, K + 1), (K + 1, B))
    d_ur = DeviceArray.from_numpy(na.FP32, np.asarray(u_residual, dtype=np.float32).reshape(B), (1, B))
    d_len = DeviceArray.from_numpy(na.I32, np.asarray(length, dtype=np.int32), (B,))
    d_tok = DeviceArray.from_numpy(na.I32, np.full(B, -1, dtype=np.int32), (B,))
    d_so = DeviceArray.from_numpy(na.I32, np.full((B, K + 1), -7, dtype=np.int32), (K + 1, B))
    d_ns = DeviceArray.from_numpy(na.I32, np.zeros(B, dtype=np.int32), (B,))
    d_acc = DeviceArray.from_numpy(na.I32, np.zeros(B, dtype=np.int32), (B,))
    d_stats = DeviceArray.from_numpy(na.I64, stats, (stats.shape[1], B))
    cfg = na.GeneralConfig()
    cfg.temperature, cfg.top_p = temperature, top_p
    cfg_buf = DeviceBuffer(8)
    cfg_buf.upload(np.frombuffer(bytes(memoryview(cfg)), dtype=np.uint8))
    ws = DeviceBuffer(ops.general_accept_workspace_bytes(token_domain, K, B))
    ws.fill(0xFF)  # the op may not depend on what scratch held before
    ops.speculative_accept_general(d_t.tensor(), d_d.tensor(), d_dr.tensor(), d_ua.tensor(), d_ur.tensor(),
                                   d_len.tensor(), d_tok.tensor(), d_so.tensor(), d_ns.tensor(), d_acc.tensor(),
                                   d_stats.tensor(), token_domain, cfg_buf.ptr, ws)
    from ninfer_amd.device import synchronize
    synchronize()
    return dict(sampled_out=d_so.numpy().reshape(B, K + 1), num_sampled=d_ns.numpy(), accepted=d_acc.numpy(),
                token=d_tok.numpy(), length=d_len.numpy(), stats=d_stats.numpy().reshape(B, -1))
