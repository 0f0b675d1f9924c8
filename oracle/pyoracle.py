"""ctypes binding of the CPU oracle (oracle/liboracle.so). TEST INFRASTRUCTURE ONLY.

Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, only as the checker or
the reported CPU baseline. Arrays are numpy, in the layouts documented in oracle/oracle.h.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"


class SamplingConfig(C.Structure):
    _fields_ = [
        ("temperature", C.c_float),
        ("top_k", C.c_int32),
        ("top_p", C.c_float),
        ("min_p", C.c_float),
        ("presence_penalty", C.c_float),
        ("frequency_penalty", C.c_float),
        ("seed", C.c_uint64),
    ]


class GeneralConfig(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float)]


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = C.CDLL(os.fspath(LIB))
        L = _lib
        L.orc_f32_to_f16_bits.restype = C.c_uint16
        L.orc_f32_to_f16_bits.argtypes = [C.c_float]
        L.orc_f16_bits_to_f32.restype = C.c_float
        L.orc_f16_bits_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_bf16_bits.restype = C.c_uint16
        L.orc_f32_to_bf16_bits.argtypes = [C.c_float]
        L.orc_det_expf.restype = C.c_float
        L.orc_det_expf.argtypes = [C.c_float]
        L.orc_splitmix64.restype = C.c_uint64
        L.orc_splitmix64.argtypes = [C.c_uint64]
        L.orc_sampling_uniform.restype = C.c_float
        L.orc_sampling_uniform.argtypes = [C.c_uint64, C.c_int32, C.c_int32, C.c_uint32]
        L.orc_sort_key.restype = C.c_uint64
        L.orc_sort_key.argtypes = [C.c_float, C.c_int32]
        L.orc_truncated_distribution.restype = C.c_int32
        L.orc_pick_from_support.restype = C.c_int32
        L.orc_general_column.restype = C.c_int32
        L.orc_tree_longest_path.restype = C.c_int32
    return _lib


def _threads(threads: int) -> int:
    """Worker threads for the FP64 kernels: the caller's count, else the host's cores capped at 16
    (the CPU share of one GPU box)."""
    return threads if threads > 0 else max(1, min(16, os.cpu_count() or 1))


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def f32_to_f16_bits(x: float) -> int:
    return int(lib().orc_f32_to_f16_bits(x))


def det_expf(x: float) -> float:
    return float(lib().orc_det_expf(x))


def splitmix64(x: int) -> int:
    return int(lib().orc_splitmix64(x))


def sampling_uniform(seed: int, pos: int, purpose: int, sub: int = 0) -> float:
    return float(lib().orc_sampling_uniform(seed, pos, purpose, sub))


def fill_normal_bf16(seed: int, n: int, std: float = 1.0, outlier_frac: float = 0.0,
                     outlier_value: float = 20.0, threads: int = 0) -> np.ndarray:
    """Seeded BF16 normals for workload-sized test inputs (synth.cpp)."""
    out = np.empty(n, dtype=np.uint16)
    lib().orc_fill_normal_bf16(C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF), C.c_size_t(n), C.c_float(std),
                               C.c_float(outlier_frac), C.c_float(outlier_value), _ptr(out),
                               C.c_int32(_threads(threads)))
    return out


def quantize_group(src_bf16: np.ndarray):
    src = np.ascontiguousarray(src_bf16, dtype=np.uint16)
    codes = np.zeros(src.size, dtype=np.int8)
    scale = np.zeros(1, dtype=np.uint16)
    lib().orc_quantize_group(_ptr(src), C.c_int32(src.size), _ptr(codes), _ptr(scale))
    return codes, int(scale[0])


def kv_append(k, v, positions, T, B, Hkv, D, P, kc, vc, ks, vs) -> None:
    """In-place update of (kc, vc, ks, vs) numpy cache planes."""
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    positions = np.ascontiguousarray(positions, dtype=np.int32)
    lib().orc_kv_append(_ptr(k), _ptr(v), _ptr(positions), C.c_int32(T), C.c_int32(B), C.c_int32(Hkv),
                        C.c_int32(D), C.c_int32(P), _ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs))


def attention(q, kc, vc, ks, vs, positions, parents, T, B, Hq, Hkv, D, P, scale, threads=0):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    positions = np.ascontiguousarray(positions, dtype=np.int32)
    par = None if parents is None else np.ascontiguousarray(parents, dtype=np.int32)
    out = np.zeros(D * Hq * T * B, dtype=np.float64)
    lib().orc_attention(_ptr(q), _ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs), _ptr(positions), _ptr(par),
                        C.c_int32(T), C.c_int32(B), C.c_int32(Hq), C.c_int32(Hkv), C.c_int32(D),
                        C.c_int32(P), C.c_double(scale), _ptr(out), C.c_int32(_threads(threads)))
    return out


def attention_bf16(q, kb, vb, positions, parents, T, B, Hq, Hkv, D, P, scale, threads=0):
    """FP64 attention over BF16 cache planes kb/vb [B][Hkv][P][D] (new rows already written)."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    kb = np.ascontiguousarray(kb, dtype=np.uint16)
    vb = np.ascontiguousarray(vb, dtype=np.uint16)
    positions = np.ascontiguousarray(positions, dtype=np.int32)
    par = None if parents is None else np.ascontiguousarray(parents, dtype=np.int32)
    out = np.zeros(D * Hq * T * B, dtype=np.float64)
    lib().orc_attention_bf16(_ptr(q), _ptr(kb), _ptr(vb), _ptr(positions), _ptr(par), C.c_int32(T),
                             C.c_int32(B), C.c_int32(Hq), C.c_int32(Hkv), C.c_int32(D), C.c_int32(P),
                             C.c_double(scale), _ptr(out), C.c_int32(_threads(threads)))
    return out


def linear_q6(qdata, qhigh, scales, N, K, x, T, threads=0):
    """FP64 Q6 linear: [T, N] doubles (before the BF16 boundary). x uint16 BF16 [T, K]."""
    qdata = np.ascontiguousarray(qdata, dtype=np.uint8)
    qhigh = np.ascontiguousarray(qhigh, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out = np.zeros(N * T, dtype=np.float64)
    lib().orc_linear_q6(_ptr(qdata), _ptr(qhigh), _ptr(scales), C.c_int32(N), C.c_int32(K), _ptr(x), C.c_int32(T),
                        _ptr(out), C.c_int32(_threads(threads)))
    return out.reshape(T, N)


def gdn_recurrent(q, k, v, g, beta, state, S, Hqk, Hv, T, normalize_qk=False, snapshots=False):
    """FP64 Gated DeltaNet recurrence: (out [T,Hv,S], state_out [Hv,S,S], snapshots [T,Hv,S,S] or None)."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    g = np.ascontiguousarray(g, dtype=np.float32)
    beta = np.ascontiguousarray(beta, dtype=np.float32)
    state = np.ascontiguousarray(state, dtype=np.float32)
    out = np.zeros(S * Hv * T, dtype=np.float64)
    st = np.zeros(S * S * Hv, dtype=np.float64)
    snap = np.zeros(S * S * Hv * T, dtype=np.float64) if snapshots else None
    lib().orc_gdn_recurrent(_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(state), C.c_int32(S),
                            C.c_int32(Hqk), C.c_int32(Hv), C.c_int32(T), C.c_double(1.0 / np.sqrt(S)),
                            C.c_int32(1 if normalize_qk else 0), _ptr(out), _ptr(st), _ptr(snap))
    return (out.reshape(T, Hv, S), st.reshape(Hv, S, S),
            None if snap is None else snap.reshape(T, Hv, S, S))


def causal_conv1d_silu(x, weight, state, channels, T):
    """FP64 conv + SiLU: (out [T,C] before the BF16 boundary, windows uint16 [T,3,C])."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    weight = np.ascontiguousarray(weight, dtype=np.uint16)
    state = np.ascontiguousarray(state, dtype=np.uint16)
    out = np.zeros(channels * T, dtype=np.float64)
    win = np.zeros(3 * channels * T, dtype=np.uint16)
    lib().orc_causal_conv1d_silu(_ptr(x), _ptr(weight), _ptr(state), C.c_int32(channels), C.c_int32(T), _ptr(out),
                                 _ptr(win))
    return out.reshape(T, channels), win.reshape(T, 3, channels)


def argmax(logits, physical_rows, columns, valid_rows):
    logits = np.ascontiguousarray(logits, dtype=np.uint16)
    out = np.zeros(columns, dtype=np.int32)
    lib().orc_argmax(_ptr(logits), C.c_int32(physical_rows), C.c_int32(columns), C.c_int32(valid_rows), _ptr(out))
    return out


def prepare_verify_inputs(token, drafts, length):
    drafts = np.ascontiguousarray(drafts, dtype=np.int32)
    K = drafts.size
    ids = np.zeros(K + 1, dtype=np.int32)
    pos = np.zeros(K + 1, dtype=np.int32)
    lib().orc_prepare_verify_inputs(C.c_int32(token), _ptr(drafts), C.c_int32(length), C.c_int32(K), _ptr(ids), _ptr(pos))
    return ids, pos


def mtp_prepare_alignment_ids(verify_ids, token, accepted, alignment_ids):
    """Returns the updated alignment ids (a copy of `alignment_ids` with the op applied)."""
    verify_ids = np.ascontiguousarray(verify_ids, dtype=np.int32)
    out = np.array(alignment_ids, dtype=np.int32, copy=True)
    lib().orc_mtp_prepare_alignment_ids(_ptr(verify_ids), C.c_int32(verify_ids.size), C.c_int32(token),
                                        C.c_int32(accepted), _ptr(out))
    return out


def speculative_accept(target_tokens, logits, physical_rows, drafts, length, stats, token_domain, cfg,
                       token_counts=None):
    """Returns dict(sampled_out, num_sampled, accepted, token, length, stats, token_counts)."""
    drafts = np.ascontiguousarray(drafts, dtype=np.int32)
    K = drafts.size
    target = np.ascontiguousarray(target_tokens if target_tokens is not None else np.zeros(K + 1), dtype=np.int32)
    logits = np.ascontiguousarray(logits, dtype=np.uint16)
    L = C.c_int32(length)
    tok = C.c_int32(-1)
    so = np.zeros(K + 1, dtype=np.int32)
    ns = C.c_int32(0)
    acc = C.c_int32(0)
    st = np.ascontiguousarray(np.array(stats, dtype=np.int64))
    tc = None if token_counts is None else np.ascontiguousarray(np.array(token_counts, dtype=np.int32))
    lib().orc_speculative_accept(_ptr(target), _ptr(logits), C.c_int32(physical_rows), _ptr(drafts),
                                 C.c_int32(K), C.byref(L), C.byref(tok), _ptr(so), C.byref(ns),
                                 C.byref(acc), _ptr(st), C.c_int32(token_domain), C.byref(cfg), _ptr(tc))
    return dict(sampled_out=so, num_sampled=ns.value, accepted=acc.value, token=tok.value, length=L.value,
                stats=st, token_counts=tc)


def truncated_distribution(column, token_domain, cfg, token_counts=None, overlay=None):
    column = np.ascontiguousarray(column, dtype=np.uint16)
    idx = np.zeros(20, dtype=np.int32)
    prob = np.zeros(20, dtype=np.float32)
    ov = None if overlay is None else np.ascontiguousarray(overlay, dtype=np.int32)
    tc = None if token_counts is None else np.ascontiguousarray(token_counts, dtype=np.int32)
    n = lib().orc_truncated_distribution(_ptr(column), C.c_int32(token_domain), C.byref(cfg), _ptr(tc), _ptr(ov),
                                         C.c_int32(0 if ov is None else ov.size), _ptr(idx), _ptr(prob))
    return idx[:n].copy(), prob[:n].copy()


def pick_from_support(cand_idx, prob, exclude, u):
    ci = np.ascontiguousarray(cand_idx, dtype=np.int32)
    pr = np.ascontiguousarray(prob, dtype=np.float32)
    return int(lib().orc_pick_from_support(_ptr(ci), _ptr(pr), C.c_int32(ci.size), C.c_int32(exclude), C.c_float(u)))


def general_column(column, token_domain, cfg):
    column = np.ascontiguousarray(column, dtype=np.uint16)
    w = np.zeros(token_domain, dtype=np.uint64)
    member = np.zeros(token_domain, dtype=np.uint8)
    zs = C.c_uint64(0)
    z = C.c_uint64(0)
    n = lib().orc_general_column(_ptr(column), C.c_int32(token_domain), C.byref(cfg), _ptr(w), _ptr(member),
                                 C.byref(zs), C.byref(z))
    return int(n), w, member, int(zs.value), int(z.value)


def general_accept(target_logits, draft_logits, physical_rows, drafts, length, stats, token_domain, cfg,
                   u_accept, u_residual):
    drafts = np.ascontiguousarray(drafts, dtype=np.int32)
    K = drafts.size
    tl = np.ascontiguousarray(target_logits, dtype=np.uint16)
    dl = np.ascontiguousarray(draft_logits, dtype=np.uint16)
    ua = np.ascontiguousarray(u_accept, dtype=np.float32)
    L = C.c_int32(length)
    tok = C.c_int32(-1)
    so = np.zeros(K + 1, dtype=np.int32)
    ns = C.c_int32(0)
    acc = C.c_int32(0)
    st = np.ascontiguousarray(np.array(stats, dtype=np.int64))
    lib().orc_general_accept(_ptr(tl), _ptr(dl), C.c_int32(physical_rows), _ptr(drafts), C.c_int32(K),
                             C.c_int32(token_domain), C.byref(cfg), _ptr(ua), C.c_float(u_residual),
                             C.byref(L), C.byref(tok), _ptr(so), C.byref(ns), C.byref(acc), _ptr(st))
    return dict(sampled_out=so, num_sampled=ns.value, accepted=acc.value, token=tok.value, length=L.value,
                stats=st)


def kv_commit_prefix(k, v, positions, T, commit_count, Hkv, D, P, kc, vc, ks, vs):
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    positions = np.ascontiguousarray(positions, dtype=np.int32)
    lib().orc_kv_commit_prefix(_ptr(k), _ptr(v), _ptr(positions), C.c_int32(T), C.c_int32(commit_count),
                               C.c_int32(Hkv), C.c_int32(D), C.c_int32(P), _ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs))


def kv_rollback(positions, T, keep_count, Hkv, D, P, kc, vc, ks, vs):
    positions = np.ascontiguousarray(positions, dtype=np.int32)
    lib().orc_kv_rollback(_ptr(positions), C.c_int32(T), C.c_int32(keep_count), C.c_int32(Hkv), C.c_int32(D),
                          C.c_int32(P), _ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs))


def kv_compact_path(base, path, count, Hkv, D, P, kc, vc, ks, vs):
    path = np.ascontiguousarray(path, dtype=np.int32)
    lib().orc_kv_compact_path(C.c_int32(base), _ptr(path), C.c_int32(count), C.c_int32(Hkv), C.c_int32(D),
                              C.c_int32(P), _ptr(kc), _ptr(vc), _ptr(ks), _ptr(vs))


def tree_longest_path(parents, node_tokens, target_tokens):
    parents = np.ascontiguousarray(parents, dtype=np.int32)
    nt = np.ascontiguousarray(node_tokens, dtype=np.int32)
    tt = np.ascontiguousarray(target_tokens, dtype=np.int32)
    path = np.zeros(parents.size, dtype=np.int32)
    n = lib().orc_tree_longest_path(_ptr(parents), _ptr(nt), _ptr(tt), C.c_int32(parents.size), _ptr(path))
    return path[:n].copy()
