"""Independent numpy restatement of the GGUF block formulas (test helper).

Written from the block layouts, not from the C oracle, so the two can pin each
other: float32 numpy operations round once each, as Java's do.
  Q8_0  y = q * d
  Q4_0  y = (nib - 8) * d + 0.0
  Q4_K  y = (d * sc) * nib - m,  m = 0 if dmin == 0 or the min code is 0,
        else dmin * min_code;  sc / min codes unpacked from the 12-byte field.
  Q5_K  as Q4_K with q = nib + 16 * (bit of qh) (bits 2c / 2c+1 for chunk c).
  Q6_K  y = (d * sc8) * (q6 - 32), q6 = 4 low bits from ql, 2 high from qh.
"""
from __future__ import annotations

import numpy as np


def _f16(lo, hi):
    bits = (lo.astype(np.uint16) | (hi.astype(np.uint16) << 8))
    v = bits.view(np.float16).astype(np.float32)
    # IEEE decode; NaN canonicalised like the reference's lookup table.
    v = np.where(np.isnan(v), np.float32(np.nan), v).astype(np.float32)
    return v


def k4_codes(scales):
    """scales (..., 12) uint8 -> sc, m (..., 8) int."""
    b = scales.astype(np.int32)
    sc = np.empty(b.shape[:-1] + (8,), np.int32)
    m = np.empty_like(sc)
    for j in range(4):
        sc[..., j] = b[..., j] & 63
        m[..., j] = b[..., j + 4] & 63
    for j in range(4, 8):
        sc[..., j] = (b[..., j + 4] & 15) | ((b[..., j - 4] >> 6) << 4)
        m[..., j] = (b[..., j + 4] >> 4) | ((b[..., j] >> 6) << 4)
    return sc, m


def dequant(type_id: int, data: np.ndarray, cols: int) -> np.ndarray:
    d8 = np.asarray(data, np.uint8)
    if type_id == 8:
        blk = d8.reshape(-1, 34)
        d = _f16(blk[:, 0], blk[:, 1])
        q = blk[:, 2:].view(np.int8).astype(np.float32)
        y = q * d[:, None]
    elif type_id == 2:
        blk = d8.reshape(-1, 18)
        d = _f16(blk[:, 0], blk[:, 1])
        qs = blk[:, 2:].astype(np.int32)
        q = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=1).astype(np.float32)
        y = (q * d[:, None]) + np.float32(0.0)
    elif type_id == 12:
        blk = d8.reshape(-1, 144)
        d = _f16(blk[:, 0], blk[:, 1])
        dmin = _f16(blk[:, 2], blk[:, 3])
        sc, mc = k4_codes(blk[:, 4:16])
        qs = blk[:, 16:].reshape(-1, 4, 32).astype(np.int32)
        y = np.empty((blk.shape[0], 256), np.float32)
        for c in range(4):
            for half, nib in ((0, qs[:, c] & 15), (1, qs[:, c] >> 4)):
                j = 2 * c + half
                dj = (d * sc[:, j].astype(np.float32)).astype(np.float32)
                with np.errstate(invalid="ignore"):
                    mj = np.where((dmin == 0) | (mc[:, j] == 0), np.float32(0.0),
                                  dmin * mc[:, j].astype(np.float32)).astype(np.float32)
                    y[:, 64 * c + 32 * half: 64 * c + 32 * half + 32] = (
                        dj[:, None] * nib.astype(np.float32)) - mj[:, None]
    elif type_id == 13:
        blk = d8.reshape(-1, 176)
        d = _f16(blk[:, 0], blk[:, 1])
        dmin = _f16(blk[:, 2], blk[:, 3])
        sc, mc = k4_codes(blk[:, 4:16])
        qh = blk[:, 16:48].astype(np.int32)
        qs = blk[:, 48:].reshape(-1, 4, 32).astype(np.int32)
        y = np.empty((blk.shape[0], 256), np.float32)
        for c in range(4):
            for half, nib in ((0, qs[:, c] & 15), (1, qs[:, c] >> 4)):
                j = 2 * c + half
                q = nib + ((qh >> j) & 1) * 16
                dj = (d * sc[:, j].astype(np.float32)).astype(np.float32)
                with np.errstate(invalid="ignore"):
                    mj = np.where((dmin == 0) | (mc[:, j] == 0), np.float32(0.0),
                                  dmin * mc[:, j].astype(np.float32)).astype(np.float32)
                    y[:, 64 * c + 32 * half: 64 * c + 32 * half + 32] = (
                        dj[:, None] * q.astype(np.float32)) - mj[:, None]
    elif type_id == 14:
        blk = d8.reshape(-1, 210)
        d = _f16(blk[:, 208], blk[:, 209])
        ql = blk[:, :128].astype(np.int32)
        qh = blk[:, 128:192].astype(np.int32)
        sc = blk[:, 192:208].view(np.int8).astype(np.float32)
        y = np.empty((blk.shape[0], 256), np.float32)
        for h in range(2):
            for g in range(4):  # value groups of 32: low/high nibble of ql[64h + 32*(g%2) + l]
                l8 = ql[:, 64 * h + 32 * (g % 2): 64 * h + 32 * (g % 2) + 32]
                nib = (l8 & 15) if g < 2 else (l8 >> 4)
                q6 = nib | (((qh[:, 32 * h: 32 * h + 32] >> (2 * g)) & 3) << 4)
                for part in range(2):
                    s = (d * sc[:, 8 * h + 2 * g + part]).astype(np.float32)
                    cols_ = slice(128 * h + 32 * g + 16 * part, 128 * h + 32 * g + 16 * part + 16)
                    y[:, cols_] = s[:, None] * (q6[:, 16 * part: 16 * part + 16] - 32).astype(np.float32)
    else:
        raise ValueError(type_id)
    return y.reshape(-1, cols).astype(np.float32)
