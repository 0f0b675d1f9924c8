"""Shared builders and checkers for the verify-step tests."""
from __future__ import annotations

import numpy as np

from ninfer_amd import synthetic as syn
from ninfer_amd.kv_cache import align_up

# Named tolerance of the reference (tests/ops/op_check.h:61): atol, rtol, tail_frac,
# worst_ratio_max, rel_l2_tol.
ATTENTION_BF16 = (2e-3, 1.6e-2, 2e-3, 5.0, 8e-3)


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def reference_composite_ok(got: np.ndarray, ref: np.ndarray, tol=ATTENTION_BF16) -> tuple[bool, str]:
    """tests/ops/op_check.h:119-179: strict allclose, or bounded tail + worst ratio + rel-L2."""
    atol, rtol, tail_frac, worst_max, l2_max = tol
    g = np.asarray(got, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    if not np.all(np.isfinite(g)):
        return False, "non-finite output"
    bound = atol + rtol * np.abs(r)
    err = np.abs(g - r)
    viol = err > bound
    l2 = rel_l2(g, r)
    if not viol.any():
        return True, f"strict ok, rel_l2={l2:.3e}"
    frac = viol.mean()
    worst = float((err[viol] / bound[viol]).max())
    ok = frac <= tail_frac and worst <= worst_max and l2 <= l2_max
    return ok, f"viol_frac={frac:.2e} worst={worst:.2f} rel_l2={l2:.3e}"


def fast_normal_bf16(seed: int, n: int, std: float = 1.0, outliers: bool = False) -> np.ndarray:
    """n N(0, std^2) values as BF16 bits from the oracle library's threaded generator; with
    `outliers`, a seeded 1% of entries become +-20 (the long-context configuration's statistics)."""
    from oracle import pyoracle
    return pyoracle.fill_normal_bf16(seed, n, std, 0.01 if outliers else 0.0, 20.0)


class AttnCase:
    """One verify-attention problem: BF16 history K/V quantized into INT8-G64 planes (or stored
    as BF16 when kv="bf16"), T new K/V columns, BF16 Q, positions L..L+T-1 per sequence."""

    def __init__(self, Ls, T=4, Hq=40, Hkv=8, D=128, seed=0, outliers=False, parents=None,
                 max_context=None, qstd=1.0, kv="i8", dist="normal", gen="splitmix", k_boost=0.0):
        """k_boost > 0 multiplies the history key rows in the last quarter of every 512-position
        window by k_boost: a split that starts in the plain rows meets scores several log2 units
        above its running maximum in mid-stream, so its lazy rescale acts on non-zero
        accumulators, with scores of moderate size."""
        self.Ls = list(Ls)
        self.B = len(self.Ls)
        self.T, self.Hq, self.Hkv, self.D = T, Hq, Hkv, D
        self.max_context = max_context or (max(self.Ls) + T)
        self.P = align_up(self.max_context, 128)
        self.parents = parents
        self.kv = kv
        B, P, G = self.B, self.P, D // 64
        if gen == "pcg":
            # workload-sized histories (10^8+ values): the same distributions from a threaded
            # generator, at a fraction of the numpy SplitMix64/Box-Muller generator's cost
            gen = (lambda sd, n: fast_normal_bf16(sd, n, outliers=True)) if outliers else fast_normal_bf16
            gen_q = lambda sd, n: fast_normal_bf16(sd, n, qstd)  # noqa: E731
        else:
            gen = syn.normal_bf16_with_outliers if outliers else syn.normal_bf16
            gen_q = lambda sd, n: syn.normal_bf16(sd, n, qstd)  # noqa: E731
        gen_k = gen_v = gen
        if dist == "uniform":
            # the reference's op-test inputs: Q, K in [-0.25, 0.25), V in [-1, 1)
            # (tests/ops/test_gqa_attention.cpp:778-782)
            gen_k = gen_q = lambda sd, n: syn.uniform_bf16(sd, n, -0.25, 0.25)  # noqa: E731
            gen_v = lambda sd, n: syn.uniform_bf16(sd, n, -1.0, 1.0)  # noqa: E731
        if kv == "bf16":
            # rows past each history hold a marker value the attention must never read
            self.kb = np.full((B, Hkv, P, D), 0x7F80, dtype=np.uint16)
            self.vb = np.full((B, Hkv, P, D), 0x7F80, dtype=np.uint16)
            for b, L in enumerate(self.Ls):
                if L > 0:
                    hk = gen_k(syn.derive_seed(seed, 1, b), D * Hkv * L).reshape(L, Hkv, D)
                    hv = gen_v(syn.derive_seed(seed, 2, b), D * Hkv * L).reshape(L, Hkv, D)
                    self.kb[b, :, :L] = hk.transpose(1, 0, 2)
                    self.vb[b, :, :L] = hv.transpose(1, 0, 2)
        else:
            self.kc = np.zeros((B, Hkv, P, D), dtype=np.int8)
            self.vc = np.zeros((B, Hkv, P, D), dtype=np.int8)
            self.ks = np.zeros((B, Hkv, P, G), dtype=np.uint16)
            self.vs = np.zeros((B, Hkv, P, G), dtype=np.uint16)
            from oracle import pyoracle
            for b, L in enumerate(self.Ls):
                if L > 0:
                    hk = gen_k(syn.derive_seed(seed, 1, b), D * Hkv * L)
                    hv = gen_v(syn.derive_seed(seed, 2, b), D * Hkv * L)
                    if k_boost > 0.0:
                        boost = np.where(np.arange(L) % 512 >= 384, k_boost, 1.0).astype(np.float32)
                        kf = syn.bf16_bits_to_f32(hk).reshape(L, Hkv * D) * boost[:, None]
                        hk = syn.f32_to_bf16_bits(kf.reshape(-1))
                    pos = np.arange(L, dtype=np.int32)
                    kcb, vcb, ksb, vsb = self.kc[b], self.vc[b], self.ks[b], self.vs[b]
                    pyoracle.kv_append(hk, hv, pos, L, 1, Hkv, D, P, kcb, vcb, ksb, vsb)
        self.k_new = np.concatenate([gen_k(syn.derive_seed(seed, 3, b), D * Hkv * T) for b in range(B)])
        self.v_new = np.concatenate([gen_v(syn.derive_seed(seed, 4, b), D * Hkv * T) for b in range(B)])
        self.q = np.concatenate([gen_q(syn.derive_seed(seed, 5, b), D * Hq * T) for b in range(B)])
        self.positions = np.concatenate([np.arange(L, L + T, dtype=np.int32) for L in self.Ls])
        self.scale = float(np.float32(1.0 / np.sqrt(D)))

    def cache_planes(self):
        """Host planes in the order KVCacheLayer.upload/download use."""
        if self.kv == "bf16":
            return self.kb, self.vb
        return self.kc, self.vc, self.ks, self.vs

    def oracle_after_append(self):
        """Cache planes after appending the new columns, and the FP64 attention output."""
        from oracle import pyoracle
        if self.kv == "bf16":
            kb, vb = self.kb.copy(), self.vb.copy()
            T, Hkv, D = self.T, self.Hkv, self.D
            for b in range(self.B):
                rows = self.positions[b * T:(b + 1) * T]
                kn = self.k_new[b * D * Hkv * T:(b + 1) * D * Hkv * T].reshape(T, Hkv, D)
                vn = self.v_new[b * D * Hkv * T:(b + 1) * D * Hkv * T].reshape(T, Hkv, D)
                kb[b][:, rows] = kn.transpose(1, 0, 2)
                vb[b][:, rows] = vn.transpose(1, 0, 2)
            out = pyoracle.attention_bf16(self.q, kb, vb, self.positions, self.parents, self.T, self.B,
                                          self.Hq, self.Hkv, self.D, self.P, float(self.scale))
            return (kb, vb), out
        kc, vc, ks, vs = self.kc.copy(), self.vc.copy(), self.ks.copy(), self.vs.copy()
        pyoracle.kv_append(self.k_new, self.v_new, self.positions, self.T, self.B, self.Hkv, self.D, self.P,
                           kc, vc, ks, vs)
        out = pyoracle.attention(self.q, kc, vc, ks, vs, self.positions, self.parents, self.T, self.B,
                                 self.Hq, self.Hkv, self.D, self.P, float(self.scale))
        return (kc, vc, ks, vs), out
