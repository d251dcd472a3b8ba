"""Seeded synthetic GGUF workloads (weights in packed GGUF bytes, activations).

Distributions of the benchmark workloads:
  Q8_0  int8 quants uniform in [-127, 127]; fp16 scale d = |N(0,1)| * 0.01.
  Q4_0  4-bit quants uniform in [0, 15] (offset -8 at decode); d = |N| * 0.02.
  Q4_K  per 256-element superblock fp16 d and dmin = |N| * 0.01; eight 6-bit
        scales and mins uniform in [0, 63]; 4-bit quants uniform in [0, 15].
  x     fp32 N(0, 1); GEMM activations bf16 = round-to-nearest-even(N(0, 1)).
  MoE   per token 8 distinct expert ids uniform over the experts; router
        weights = softmax of 8 N(0, 1) draws.
Byte layouts follow the GGUF blocks the reference decodes (RT/ =
runner/gguf/gollek-gguf-core/src/main/java/tech/kayys/gollek/gguf/runtime/):
RT/GgufRowDequantizer.java:141-152 (Q8_0), RT/GgufBlockDequantizer.java:32-36
and :402-414 (Q4_0), RT/GgufKBlockDequantizer.java:31-88 with the 6-bit
scale/min packing unpacked by RT/GgufKQuantLayout.java:37-49 (Q4_K).
"""
from __future__ import annotations

import numpy as np

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 8, 12, 13, 14


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def f16_bits(values) -> np.ndarray:
    """Round to IEEE half (RNE) and return the raw uint16 bits."""
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def bf16_bits(values) -> np.ndarray:
    """Round fp32 to bfloat16 (RNE) and return the raw uint16 bits."""
    bits = np.asarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounding = ((bits >> 16) & 1) + 0x7FFF
    return ((bits + rounding) >> 16).astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _put_u16(dst: np.ndarray, offset: int, values: np.ndarray) -> None:
    v = values.astype(np.uint16)
    dst[..., offset] = (v & 0xFF).astype(np.uint8)
    dst[..., offset + 1] = (v >> 8).astype(np.uint8)


def pack_q4k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Inverse of the 6-bit scale/min unpack (RT/GgufKQuantLayout.java:37-49).

    sc, mn: (..., 8) integer codes in [0, 63] -> (..., 12) packed bytes."""
    sc = np.asarray(sc, dtype=np.uint16)
    mn = np.asarray(mn, dtype=np.uint16)
    out = np.zeros(sc.shape[:-1] + (12,), dtype=np.uint16)
    for j in range(4):
        out[..., j] = sc[..., j] | ((sc[..., j + 4] >> 4) << 6)
        out[..., j + 4] = mn[..., j] | ((mn[..., j + 4] >> 4) << 6)
    for j in range(4, 8):
        out[..., j + 4] = (sc[..., j] & 15) | ((mn[..., j] & 15) << 4)
    return out.astype(np.uint8)


def q8_0_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    """(rows, cols/32*34) uint8."""
    g = rng(seed)
    nb = cols // 32
    out = np.empty((rows, nb, 34), dtype=np.uint8)
    _put_u16(out, 0, f16_bits(np.abs(g.standard_normal((rows, nb), dtype=np.float32)) * 0.01))
    out[..., 2:] = g.integers(-127, 128, size=(rows, nb, 32), dtype=np.int8).view(np.uint8)
    return out.reshape(rows, nb * 34)


def q4_0_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    """(rows, cols/32*18) uint8; byte i = element i | element i+16 << 4."""
    g = rng(seed)
    nb = cols // 32
    out = np.empty((rows, nb, 18), dtype=np.uint8)
    _put_u16(out, 0, f16_bits(np.abs(g.standard_normal((rows, nb), dtype=np.float32)) * 0.02))
    lo = g.integers(0, 16, size=(rows, nb, 16), dtype=np.uint8)
    hi = g.integers(0, 16, size=(rows, nb, 16), dtype=np.uint8)
    out[..., 2:] = lo | (hi << 4)
    return out.reshape(rows, nb * 18)


def q4_k_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    """(rows, cols/256*144) uint8."""
    g = rng(seed)
    ns = cols // 256
    out = np.empty((rows, ns, 144), dtype=np.uint8)
    _put_u16(out, 0, f16_bits(np.abs(g.standard_normal((rows, ns), dtype=np.float32)) * 0.01))
    _put_u16(out, 2, f16_bits(np.abs(g.standard_normal((rows, ns), dtype=np.float32)) * 0.01))
    sc = g.integers(0, 64, size=(rows, ns, 8), dtype=np.uint16)
    mn = g.integers(0, 64, size=(rows, ns, 8), dtype=np.uint16)
    out[..., 4:16] = pack_q4k_scales(sc, mn)
    out[..., 16:] = g.integers(0, 256, size=(rows, ns, 128), dtype=np.uint8)
    return out.reshape(rows, ns * 144)


def q5_k_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    """(rows, cols/256*176) uint8: d, dmin = fp16(|N| * 0.01), 6-bit scale and
    min codes ~ U{0..63}, qh and qs bytes ~ U{0..255}."""
    g = rng(seed)
    ns = cols // 256
    out = np.empty((rows, ns, 176), dtype=np.uint8)
    _put_u16(out, 0, f16_bits(np.abs(g.standard_normal((rows, ns), dtype=np.float32)) * 0.01))
    _put_u16(out, 2, f16_bits(np.abs(g.standard_normal((rows, ns), dtype=np.float32)) * 0.01))
    sc = g.integers(0, 64, size=(rows, ns, 8), dtype=np.uint16)
    mn = g.integers(0, 64, size=(rows, ns, 8), dtype=np.uint16)
    out[..., 4:16] = pack_q4k_scales(sc, mn)
    out[..., 16:] = g.integers(0, 256, size=(rows, ns, 160), dtype=np.uint8)
    return out.reshape(rows, ns * 176)


def q6_k_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    """(rows, cols/256*210) uint8: ql, qh bytes ~ U{0..255}, int8 scales
    ~ U{-64..63}, d = fp16(|N| * 0.002)."""
    g = rng(seed)
    ns = cols // 256
    out = np.empty((rows, ns, 210), dtype=np.uint8)
    out[..., :192] = g.integers(0, 256, size=(rows, ns, 192), dtype=np.uint8)
    out[..., 192:208] = g.integers(-64, 64, size=(rows, ns, 16)).astype(np.int8).view(np.uint8)
    _put_u16(out, 208, f16_bits(np.abs(g.standard_normal((rows, ns), dtype=np.float32)) * 0.002))
    return out.reshape(rows, ns * 210)


def matrix(type_id: int, rows: int, cols: int, seed: int) -> np.ndarray:
    if type_id == Q5_K:
        return q5_k_matrix(rows, cols, seed)
    if type_id == Q6_K:
        return q6_k_matrix(rows, cols, seed)
    if type_id == Q8_0:
        return q8_0_matrix(rows, cols, seed)
    if type_id == Q4_0:
        return q4_0_matrix(rows, cols, seed)
    if type_id == Q4_K:
        return q4_k_matrix(rows, cols, seed)
    raise ValueError(f"unsupported type id {type_id}")


def activation(n: int, seed: int) -> np.ndarray:
    return rng(seed).standard_normal(n, dtype=np.float32)


def activation_bf16(m: int, k: int, seed: int) -> np.ndarray:
    """(m, k) uint16 bf16 bits of N(0, 1)."""
    return bf16_bits(rng(seed).standard_normal((m, k), dtype=np.float32))


def moe_routing(tokens: int, experts: int, top_k: int, seed: int):
    """(ids int32 (tokens, top_k), weights float32 (tokens, top_k))."""
    g = rng(seed)
    ids = np.stack([g.choice(experts, size=top_k, replace=False) for _ in range(tokens)])
    logits = g.standard_normal((tokens, top_k))
    w = np.exp(logits - logits.max(axis=1, keepdims=True))
    w /= w.sum(axis=1, keepdims=True)
    return ids.astype(np.int32), w.astype(np.float32)
