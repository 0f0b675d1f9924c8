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


class AttnCase:
    """One verify-attention problem: BF16 history K/V quantized into INT8-G64 planes, T new K/V
    columns, BF16 Q, positions L..L+T-1 per sequence."""

    def __init__(self, Ls, T=4, Hq=40, Hkv=8, D=128, seed=0, outliers=False, parents=None,
                 max_context=None, qstd=1.0):
        self.Ls = list(Ls)
        self.B = len(self.Ls)
        self.T, self.Hq, self.Hkv, self.D = T, Hq, Hkv, D
        self.max_context = max_context or (max(self.Ls) + T)
        self.P = align_up(self.max_context, 128)
        self.parents = parents
        B, P, G = self.B, self.P, D // 64
        self.kc = np.zeros((B, Hkv, P, D), dtype=np.int8)
        self.vc = np.zeros((B, Hkv, P, D), dtype=np.int8)
        self.ks = np.zeros((B, Hkv, P, G), dtype=np.uint16)
        self.vs = np.zeros((B, Hkv, P, G), dtype=np.uint16)
        gen = syn.normal_bf16_with_outliers if outliers else syn.normal_bf16
        from oracle import pyoracle
        for b, L in enumerate(self.Ls):
            if L > 0:
                hk = gen(syn.derive_seed(seed, 1, b), D * Hkv * L)
                hv = gen(syn.derive_seed(seed, 2, b), D * Hkv * L)
                pos = np.arange(L, dtype=np.int32)
                kcb, vcb, ksb, vsb = self.kc[b], self.vc[b], self.ks[b], self.vs[b]
                pyoracle.kv_append(hk, hv, pos, L, 1, Hkv, D, P, kcb, vcb, ksb, vsb)
        self.k_new = np.concatenate([gen(syn.derive_seed(seed, 3, b), D * Hkv * T) for b in range(B)])
        self.v_new = np.concatenate([gen(syn.derive_seed(seed, 4, b), D * Hkv * T) for b in range(B)])
        self.q = np.concatenate([syn.normal_bf16(syn.derive_seed(seed, 5, b), D * Hq * T, qstd) for b in range(B)])
        self.positions = np.concatenate([np.arange(L, L + T, dtype=np.int32) for L in self.Ls])
        self.scale = float(np.float32(1.0 / np.sqrt(D)))

    def oracle_after_append(self):
        """Cache planes after appending the new columns, and the FP64 attention output."""
        from oracle import pyoracle
        kc, vc, ks, vs = self.kc.copy(), self.vc.copy(), self.ks.copy(), self.vs.copy()
        pyoracle.kv_append(self.k_new, self.v_new, self.positions, self.T, self.B, self.Hkv, self.D, self.P,
                           kc, vc, ks, vs)
        out = pyoracle.attention(self.q, kc, vc, ks, vs, self.positions, self.parents, self.T, self.B,
                                 self.Hq, self.Hkv, self.D, self.P, float(self.scale))
        return (kc, vc, ks, vs), out
