"""Q6G64_F16S RowSplit payloads for the lm_head tests (test infrastructure).

Restates, vectorized, the reference test packer: pack_lowbit_group for 6-bit codes
(tests/ops/row_split_pack.h:143-172: code i's low nibble in byte i/2, high half for odd i; its two
high bits at bit 2i of the group's high bytes) and make_patterned_weight (:228-285: deterministic
bytes from (row, group, byte, seed), scales from a 4-entry table), plus exact FP64 -> BF16
rounding for the oracle's logits.
"""
from __future__ import annotations

import numpy as np

SCALE_TABLE = np.array([0x3800, 0x3A00, 0x3C00, 0x3D00], dtype=np.uint16)  # row_split_pack.h:276


def align_up(v, a):
    return (v + a - 1) // a * a


def pack_codes(codes: np.ndarray):
    """codes int [N, Kp] in [-32, 31] -> (nibble [N, G, 32], high [N, G, 16]) uint8."""
    N, Kp = codes.shape
    assert Kp % 64 == 0 and codes.min() >= -32 and codes.max() <= 31
    u = (codes.astype(np.int64) & 63).reshape(N, Kp // 64, 64)
    low, hi = u & 15, u >> 4
    nib = (low[..., 0::2] | (low[..., 1::2] << 4)).astype(np.uint8)
    h = hi.reshape(N, Kp // 64, 16, 4)
    high = (h[..., 0] | (h[..., 1] << 2) | (h[..., 2] << 4) | (h[..., 3] << 6)).astype(np.uint8)
    return nib, high


def unpack_codes(nib: np.ndarray, high: np.ndarray) -> np.ndarray:
    """Inverse of pack_codes: [N, G, 32] + [N, G, 16] -> int [N, G * 64]."""
    N, G, _ = nib.shape
    low = np.empty((N, G, 64), dtype=np.int64)
    low[..., 0::2] = nib & 15
    low[..., 1::2] = nib >> 4
    hb = high.astype(np.int64)
    hi = np.stack([(hb >> (2 * m)) & 3 for m in range(4)], axis=-1).reshape(N, G, 64)
    u = low | (hi << 4)
    return np.where(u & 32, u - 64, u).reshape(N, G * 64)


def patterned(n: int, k: int, seed: int, block: int = 8192):
    """make_patterned_weight for Q6: (nibble [n, G, 32], high [n, G, 16], scales [n, G])."""
    kg = align_up(k, 128) // 64
    nib = np.empty((n, kg, 32), dtype=np.uint8)
    high = np.empty((n, kg, 16), dtype=np.uint8)
    sc = np.empty((n, kg), dtype=np.uint16)
    g = np.arange(kg, dtype=np.uint32)[None, :, None]
    bn = np.arange(32, dtype=np.uint32)[None, None, :]
    bh = np.arange(16, dtype=np.uint32)[None, None, :]
    s = np.uint32(seed)
    with np.errstate(over="ignore"):
        for r0 in range(0, n, block):
            row = np.arange(r0, min(n, r0 + block), dtype=np.uint32)[:, None, None]
            mix = row ^ (row >> np.uint32(8)) ^ (row >> np.uint32(16))
            nib[r0:r0 + row.shape[0]] = ((mix * np.uint32(37) + g * np.uint32(29) + bn * np.uint32(17) + s)
                                          & np.uint32(0xFF)).astype(np.uint8)
            high[r0:r0 + row.shape[0]] = ((mix * np.uint32(43) + g * np.uint32(31) + bh * np.uint32(13) + s * np.uint32(3))
                                           & np.uint32(0xFF)).astype(np.uint8)
            idx = (row[:, :, 0] ^ (row[:, :, 0] >> np.uint32(8)) ^ g[:, :, 0] ^ s) & np.uint32(3)
            sc[r0:r0 + row.shape[0]] = SCALE_TABLE[idx]
    return nib, high, sc


def f64_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even FP64 -> BF16 in one step (no FP32 intermediate), finite normal values
    and zero (the range of the logits here)."""
    v = np.asarray(v, dtype=np.float64)
    b = v.view(np.uint64)
    sign = (b >> np.uint64(63)).astype(np.uint64)
    exp = ((b >> np.uint64(52)) & np.uint64(0x7FF)).astype(np.int64)
    man = (b & np.uint64((1 << 52) - 1)) | np.uint64(1 << 52)  # 53-bit significand
    e32 = exp - 1023 + 127
    ok = (v == 0) | ((e32 >= 1) & (e32 <= 254))
    assert ok.all(), "logit outside the normal BF16 range"
    shift = np.uint64(52 - 7)
    q = man >> shift
    rem = man & np.uint64((1 << 45) - 1)
    half = np.uint64(1 << 44)
    up = (rem > half) | ((rem == half) & ((q & np.uint64(1)) == np.uint64(1)))
    q = q + up.astype(np.uint64)
    carry = q >> np.uint64(8)  # significand overflowed to 2.0
    q = np.where(carry > 0, q >> np.uint64(1), q)
    e32 = e32 + carry.astype(np.int64)
    bits = (sign << np.uint64(15)) | (e32.astype(np.uint64) << np.uint64(7)) | (q & np.uint64(0x7F))
    return np.where(v == 0, sign << np.uint64(15), bits).astype(np.uint16)


def bf16_order_key(bits: np.ndarray) -> np.ndarray:
    """Ordered value of BF16 bits as a float comparison (-0 = +0)."""
    b = np.asarray(bits, dtype=np.uint32)
    b = np.where(b == 0x8000, 0, b)
    return np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000).astype(np.int64)


def argmax_lowest(bits: np.ndarray, valid_rows: int) -> int:
    """Lowest row attaining the largest BF16 value among rows [0, valid_rows)."""
    key = bf16_order_key(bits[:valid_rows])
    return int(np.argmax(key))  # numpy argmax returns the first maximum
