"""GPU parity of the lm_head: Q6G64_F16S RowSplit linear (include/ninfer/ops/linear.h:10-27) and the
fused linear -> argmax (the reference's deferred FUT-F03 contract,
docs/maintainer/qwen3.6-35b-a3b-dflash-op-checklist.md:985-1001).

Weights: the reference's registered output heads [248320, 5120] and [248320, 2048] filled by its
deterministic test generator (make_patterned_weight, tests/ops/row_split_pack.h:228-285, restated in
tests/q6_pack.py), and random codes for edge shapes. The oracle decodes exactly and sums in FP64; the
observable logit is BF16 of that sum. The kernel sums exact products in FP32, so a logit may land one
BF16 step away where the FP64 sum sits next to a rounding boundary, or a few steps for a logit near
zero (where a step is far below the FP32 summation error): the bar is one step or 2^-16 of the
column's rms magnitude for every logit, at least 99.9% bit-equal, and the reference's bf16_reduction
composite
(tests/ops/op_check.h:39-42). The fused argmax must equal the oracle's lowest-index argmax over the
BF16 logits except at a near tie (the two candidates within one BF16 step), and must always equal
argmax over the logits the unfused kernel writes (the composed route linear -> argmax)."""
import numpy as np
import pytest

import ninfer_amd as na
import q6_pack as qp
from helpers import reference_composite_ok
from ninfer_amd import ops, synthetic as syn
from ninfer_amd._capi import Q6G64_F16S
from ninfer_amd.device import DeviceArray, DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu

BF16_REDUCTION = (2e-3, 1.6e-2, 2e-3, 5.0, 8e-3)
VOCAB = 248320


class DeviceWeight:
    """Reference payload layout (src/artifact/storage_layouts.cpp:129-151): nibble plane, high plane
    at the next 256-byte boundary, scale plane after it."""

    def __init__(self, nib, high, sc, n, k):
        nb, hb, sb = nib.size, high.size, sc.size * 2
        hoff = qp.align_up(nb, 256)
        soff = hoff + qp.align_up(hb, 256)
        payload = np.zeros(soff + sb, np.uint8)
        payload[:nb] = nib.ravel()
        payload[hoff:hoff + hb] = high.ravel()
        payload[soff:] = np.ascontiguousarray(sc).view(np.uint8).ravel()
        self.buf = DeviceBuffer(payload.size)
        self.buf.upload(payload)
        w = na.Weight()
        w.payload, w.payload_bytes, w.high_plane_bytes = self.buf.ptr, payload.size, hb
        w.qtype, w.group_size, w.ndim = Q6G64_F16S, 64, 2
        w.shape[:] = [n, k, 1, 1]
        w.padded_shape[:] = [n, qp.align_up(k, 128), 1, 1]
        w.qdata, w.qhigh, w.scales = self.buf.ptr, self.buf.ptr + hoff, self.buf.ptr + soff
        w.n, w.k, w.group, w.layout, w.scale_dtype = n, k, 64, 0, na.FP16
        self.w = w
        self.nib, self.high, self.sc, self.n, self.k = nib, high, sc, n, k


def _x(seed, T, K):
    rng = np.random.default_rng(seed)
    return syn.f32_to_bf16_bits(rng.uniform(-1, 1, (T, K)).astype(np.float32))


def run_linear(dw, x):
    T, K = x.shape
    dx = DeviceArray.from_numpy(na.BF16, x, (K, T))
    dout = DeviceArray(na.BF16, (dw.n, T))
    dout.buf.fill(0xFF)
    ops.linear(dx.tensor(), dw.w, dout.tensor())
    synchronize()
    return dout.numpy().reshape(T, dw.n)


def run_argmax(dw, x, valid_rows):
    T, K = x.shape
    dx = DeviceArray.from_numpy(na.BF16, x, (K, T))
    dout = DeviceArray.from_numpy(na.I32, np.full(T, -7, np.int32), (T,))
    ws = DeviceBuffer(ops.linear_argmax_workspace_bytes(T))
    ws.fill(0xFF)
    ops.linear_argmax(dx.tensor(), dw.w, valid_rows, ws, dout.tensor())
    synchronize()
    return dout.numpy()


def oracle_logits(dw, x):
    from oracle import pyoracle
    T, K = x.shape
    return pyoracle.linear_q6(dw.nib, dw.high, dw.sc, dw.n, K, x, T)


def check_logits(got, ref64, tag):
    """Every logit within one BF16 step of BF16(FP64 sum), or, near zero where a step is tiny, within
    the FP32 summation error of the column (2^-16 of its rms magnitude); at least 99.9% bit-equal."""
    ref = qp.f64_to_bf16_bits(ref64)
    dist = np.abs(qp.bf16_order_key(got) - qp.bf16_order_key(ref))
    gotf = syn.bf16_bits_to_f32(got).astype(np.float64)
    err = np.abs(gotf - ref64)
    floor = 2.0 ** -16 * np.sqrt(np.mean(ref64 * ref64, axis=1, keepdims=True))
    bad = (dist > 1) & (err > floor)
    exact = float(np.mean(dist == 0))
    ok, msg = reference_composite_ok(gotf, ref64, BF16_REDUCTION)
    worst = np.unravel_index(np.argmax(dist), dist.shape)
    print(f"{tag}: bit-equal {exact:.6f}, max step {dist.max()} (ref {ref64[worst]:.6g}, got {gotf[worst]:.6g}, "
          f"floor {floor[worst[0], 0]:.3g}), composite {msg}", flush=True)
    assert not bad.any(), f"{int(bad.sum())} logits outside one step and the summation floor"
    assert exact >= 0.999
    assert ok, msg


def check_argmax(got, ref64, valid_rows, tag):
    refb = qp.f64_to_bf16_bits(ref64)
    for t in range(ref64.shape[0]):
        want = qp.argmax_lowest(refb[t], valid_rows)
        if got[t] != want:
            key = qp.bf16_order_key(refb[t][:valid_rows])
            print(f"{tag} t={t}: got {got[t]} want {want}, keys {key[got[t]]} vs {key[want]}", flush=True)
            assert 0 <= got[t] < valid_rows and key[want] - key[got[t]] <= 1, "not a near tie"


@pytest.fixture(scope="module", params=[5120, 2048])
def head(request):
    K = request.param
    print(f"case lm_head Q6 [{VOCAB}, {K}] patterned seed 4226", flush=True)
    nib, high, sc = qp.patterned(VOCAB, K, 4226)
    return DeviceWeight(nib, high, sc, VOCAB, K)


@pytest.mark.parametrize("T", [1, 4, 9, 16, 24, 64])
def test_linear_full_head(gpu, head, T):
    x = _x(100 + T, T, head.k)
    got = run_linear(head, x)
    check_logits(got, oracle_logits(head, x), f"linear [{head.n},{head.k}] T={T}")


@pytest.mark.parametrize("T,valid", [(4, VOCAB), (16, VOCAB), (4, 151936), (40, VOCAB)])
def test_linear_argmax_full_head(gpu, head, T, valid):
    x = _x(200 + T, T, head.k)
    got = run_argmax(head, x, valid)
    ref64 = oracle_logits(head, x)
    check_argmax(got, ref64, valid, f"argmax [{head.n},{head.k}] T={T} valid={valid}")
    # composed route: the unfused kernel's BF16 logits, then the same argmax rule
    logits = run_linear(head, x)
    for t in range(T):
        assert got[t] == qp.argmax_lowest(logits[t], valid)


@pytest.mark.parametrize("N,K,T", [(1, 64, 1), (17, 200, 3), (100, 1000, 5), (250, 4096, 9), (33, 640, 17),
                                   (4096, 8192, 4), (64, 128, 16), (100, 1000, 33), (4096, 8192, 40),
                                   (50, 1004, 20), (3000, 320, 64)])
def test_linear_edge_shapes(gpu, N, K, T):
    """Rows not a multiple of 16, padded K (groups past K hold codes that x = 0 cancels), K up to the
    8192 limit, several column passes. T > 16 with K % 8 == 0 takes the K-outer form (32 columns per
    pass: T = 17, 33, 40, 64); K = 1004 keeps the column passes."""
    print(f"case linear edge N={N} K={K} T={T}", flush=True)
    rng = np.random.default_rng(N * 7 + K + T)
    Kp = qp.align_up(K, 128)
    nib, high = qp.pack_codes(rng.integers(-32, 32, (N, Kp)))
    sc = np.float16(rng.uniform(0.001, 0.05, (N, Kp // 64))).view(np.uint16)
    dw = DeviceWeight(nib, high, sc, N, K)
    x = _x(N + T, T, K)
    got = run_linear(dw, x)
    ref = oracle_logits(dw, x)
    check_logits(got, ref, f"edge N={N} K={K} T={T}")
    am = run_argmax(dw, x, N)
    check_argmax(am, ref, N, "edge argmax")
    for t in range(T):
        assert am[t] == qp.argmax_lowest(got[t], N)


def test_linear_argmax_ties_take_lowest_row(gpu):
    """Duplicated rows tie exactly: the lowest index wins; with x = 0 every logit is +0 and row 0 wins."""
    rng = np.random.default_rng(5)
    N, K = 1000, 512
    codes = rng.integers(-32, 32, (N, K))
    codes[717] = codes[391] = codes[950]
    sc = np.float16(rng.uniform(0.01, 0.02, (N, K // 64)))
    sc[717] = sc[391] = sc[950]
    nib, high = qp.pack_codes(codes)
    dw = DeviceWeight(nib, high, sc.view(np.uint16), N, K)
    w = codes.astype(np.float64) * np.repeat(sc.astype(np.float64), 64, axis=1)
    x = np.zeros((2, K), np.uint16)
    # column 0: x along row 391's weights makes that row's logit the largest
    x[0] = syn.f32_to_bf16_bits(np.sign(w[391]).astype(np.float32))
    got = run_argmax(dw, x, N)
    assert got[0] == 391 and got[1] == 0
