"""Python wrapper of the CPU oracle (gguf_oracle.c) plus fp64 references.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the gollek_amd package.  It checks the
HIP library; it is not a fallback for it.

  * dequantize / dot / matvec: the C restatement of gollek's Java raw route
    (RT/ = runner/gguf/gollek-gguf-core/src/main/java/tech/kayys/gollek/gguf/
    runtime/; citations in gguf_oracle.c).
  * gemm_reference: fp64 brute force Y = X W^T over the bit-exact dequantized
    weights (the Linear convention of runner/safetensor/gollek-safetensor-core/
    src/main/java/tech/kayys/gollek/safetensor/core/tensor/AccelOps.java:
    370-376; no GGUF GEMM exists in the reference).
  * moe_reference: fp64 restatement of MoeForwardPass.computeAccel's expert
    loop (runner/safetensor/gollek-safetensor-engine/src/main/java/tech/kayys/
    gollek/safetensor/engine/generation/moe/MoeForwardPass.java:217-240,
    :461-472) with swigluFfn = down(silu(gate x) * up x)
    (.../engine/forward/DirectForwardFfnService.java:40-61).
  * moe_shared_expert_reference: the shared expert added after the routes
    (MoeForwardPass.java:240-247, runSharedExpert :418-426,
    resolveSharedExpertGate :428-442).
  * rel_err: the tolerance metric, max_i |y_i - r_i| / max(|r_i|, 1e-3 ||r||_inf).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "build" / "libgguf_oracle.so"

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 8, 12, 13, 14
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = load(LIB_PATH)
    return _lib


def build_planted(n: int, out_dir) -> Path:
    """Build a copy of the oracle with planted mistake n (gguf_oracle.c's
    GO_PLANT list) into out_dir, for tests that show the checks catch it."""
    out = Path(out_dir) / f"libgguf_oracle_plant{n}.so"
    subprocess.run(["gcc", "-O1", "-ffp-contract=off", "-fno-fast-math", "-std=c11", "-fPIC", "-shared",
                    f"-DGO_PLANT={int(n)}", str(ORACLE_DIR / "gguf_oracle.c"), "-o", str(out),
                    "-lpthread", "-lm"], check=True)
    return out


def load(path) -> ctypes.CDLL:
    """Load an oracle build (the default one, or a planted copy)."""
    L = ctypes.CDLL(str(path))
    P, I, I64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    L.go_f16_to_f32.restype = F
    L.go_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.go_f16_to_f32_n.argtypes = [P, I64, P]
    L.go_k4_scale_min.argtypes = [P, I, P, P]
    L.go_row_bytes.restype = I64
    L.go_row_bytes.argtypes = [I, I64]
    L.go_dequantize_rows.restype = I
    L.go_dequantize_rows.argtypes = [I, P, I64, I64, I64, I64, P]
    L.go_dot_row.restype = I
    L.go_dot_row.argtypes = [I, P, I64, P, P]
    L.go_matvec_rows.restype = I
    L.go_matvec_rows.argtypes = [I, P, I64, I64, I64, P, P, I64, I]
    L.go_default_threads.restype = I
    L.go_group_sums32.argtypes = [P, I64, P]
    L.go_group_sums16.argtypes = [P, I64, P]
    L.go_k_rows_have_mins.restype = I
    L.go_k_rows_have_mins.argtypes = [I, P, I64, I64, I64]
    L.go_moe_select_topk.restype = I
    L.go_moe_select_topk.argtypes = [P, I64, I64, I64, I, P, P]
    L.go_q4k_rows_have_mins.restype = I
    L.go_q4k_rows_have_mins.argtypes = [P, I64, I64, I64]
    return L


def _u8(data) -> np.ndarray:
    return np.ascontiguousarray(data, dtype=np.uint8)


def row_bytes(type_id: int, cols: int) -> int:
    return int(lib().go_row_bytes(type_id, cols))


def f16_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().go_f16_to_f32_n(b.ctypes.data, b.size, out.ctypes.data)
    return out


def k4_scale_min(scales12, j: int) -> tuple[int, int]:
    s = _u8(scales12)
    sc, m = ctypes.c_int(), ctypes.c_int()
    lib().go_k4_scale_min(s.ctypes.data, j, ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def dequantize(type_id: int, data, cols: int, row0: int = 0, nrows: int | None = None) -> np.ndarray:
    d = _u8(data)
    rb = row_bytes(type_id, cols)
    rows = d.size // rb if rb > 0 else 0
    if nrows is None:
        nrows = rows - row0
    out = np.empty((nrows, cols), dtype=np.float32)
    rc = lib().go_dequantize_rows(type_id, d.ctypes.data, rb, cols, row0, nrows, out.ctypes.data)
    if rc != 0:
        raise ValueError(f"oracle dequantize failed: {rc}")
    return out


def dot_row(type_id: int, row_data, cols: int, x, _lib=None) -> float:
    d = _u8(row_data)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    out = ctypes.c_float()
    rc = (_lib or lib()).go_dot_row(type_id, d.ctypes.data, cols, xv.ctypes.data, ctypes.byref(out))
    if rc != 0:
        raise ValueError(f"oracle dot failed: {rc}")
    return out.value


def matvec(type_id: int, data, cols: int, x, row_count: int | None = None,
           threads: int = 0, _lib=None) -> np.ndarray:
    d = _u8(data)
    rb = row_bytes(type_id, cols)
    rows = d.size // rb
    if row_count is None:
        row_count = rows
    xv = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(max(row_count, 1), dtype=np.float32)
    rc = (_lib or lib()).go_matvec_rows(type_id, d.ctypes.data, rows, cols, rb, xv.ctypes.data,
                              y.ctypes.data, row_count, threads)
    if rc != 0:
        raise ValueError(f"oracle matvec failed: {rc}")
    return y[:row_count]


def default_threads() -> int:
    return int(lib().go_default_threads())


def group_sums32(x) -> np.ndarray:
    xv = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(xv.size // 32, dtype=np.float32)
    lib().go_group_sums32(xv.ctypes.data, xv.size, out.ctypes.data)
    return out


def group_sums16(x) -> np.ndarray:
    xv = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(xv.size // 16, dtype=np.float32)
    lib().go_group_sums16(xv.ctypes.data, xv.size, out.ctypes.data)
    return out


def q4k_rows_have_mins(data, cols: int, row_count: int) -> bool:
    d = _u8(data)
    return bool(lib().go_q4k_rows_have_mins(d.ctypes.data, row_bytes(Q4_K, cols), cols, row_count))


def k_rows_have_mins(type_id: int, data, cols: int, row_count: int) -> bool:
    """Q4_K / Q5_K: whether any of the first row_count rows has an active min."""
    d = _u8(data)
    rc = lib().go_k_rows_have_mins(type_id, d.ctypes.data, row_bytes(type_id, cols), cols, row_count)
    if rc < 0:
        raise ValueError(f"oracle min scan failed: {rc}")
    return bool(rc)


# ---- fp64 references -----------------------------------------------------

def matvec_fp64(type_id: int, data, cols: int, x) -> np.ndarray:
    """fp64 dot over the bit-exact dequantized rows (textbook GEMV)."""
    w = dequantize(type_id, data, cols).astype(np.float64)
    return w @ np.asarray(x, dtype=np.float64)


def gemm_reference(type_id: int, data, cols: int, x_bf16_bits) -> np.ndarray:
    """fp64 Y[m, n] = sum_k X[m, k] W[n, k]; X given as bf16 bits (m, k)."""
    w = dequantize(type_id, data, cols).astype(np.float64)
    x = (np.asarray(x_bf16_bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    return x.astype(np.float64) @ w.T


def moe_select_topk(logits, top_k: int, sigmoid: bool):
    """MoE router (go_moe_select_topk): logits (T, E) fp32 -> ids (T, k)
    int32, weights (T, k) fp32, as MoeForwardPass.java:174-203,286-306."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = lg.shape
    ids = np.zeros((T, top_k), np.int32)
    w = np.zeros((T, top_k), np.float32)
    rc = lib().go_moe_select_topk(lg.ctypes.data, T, E, top_k, int(bool(sigmoid)),
                                  ids.ctypes.data, w.ctypes.data)
    if rc != 0:
        raise ValueError(f"go_moe_select_topk: status {rc}")
    return ids, w


def silu(v: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):  # exp(-v) = inf for v << 0 gives the right limit, -0
        return v / (1.0 + np.exp(-v))


def moe_reference(gate_w: np.ndarray, up_w: np.ndarray, down_w: np.ndarray, x: np.ndarray,
                  ids: np.ndarray, weights: np.ndarray) -> np.ndarray:
    """fp64 MoE FFN over dequantized stacked expert weights.

    gate_w, up_w: (E, I, H); down_w: (E, H, I); x: (T, H); ids, weights:
    (T, k).  out[t] = sum_k w[t,k] * down_e(silu(gate_e x_t) * up_e x_t),
    accumulated over k in routing order (MoeForwardPass.java:217-240)."""
    T, k = ids.shape
    out = np.zeros((T, down_w.shape[1]), dtype=np.float64)
    for t in range(T):
        xt = x[t].astype(np.float64)
        for j in range(k):
            e = int(ids[t, j])
            h = silu(gate_w[e] @ xt) * (up_w[e] @ xt)
            out[t] += float(weights[t, j]) * (down_w[e] @ h)
    return out


def moe_reference_q4k(gate: np.ndarray, up: np.ndarray, down: np.ndarray, n_experts: int,
                      x: np.ndarray, ids: np.ndarray, weights: np.ndarray,
                      down_type: int = Q4_K, gate_type: int = Q4_K) -> np.ndarray:
    """moe_reference over packed stacked gate / up experts of gate_type and
    down experts of down_type (Q8_0, Q4_0, Q4_K, Q5_K or Q6_K), dequantizing
    only the experts the routes use (bit-exact dequantization, fp64
    arithmetic).

    gate, up: (E * I, row bytes of H columns); down: (E * H, row bytes of I
    columns); x: (T, H).  Routes with an id outside [0, E) or a zero weight
    are skipped (MoeForwardPass.java:222)."""
    H = np.asarray(x).shape[1]
    I = gate.shape[0] // n_experts
    T, k = ids.shape
    out = np.zeros((T, H), dtype=np.float64)
    cache = {}
    for t in range(T):
        xt = x[t].astype(np.float64)
        for j in range(k):
            e, wj = int(ids[t, j]), float(weights[t, j])
            if e < 0 or e >= n_experts or wj == 0.0:
                continue
            if e not in cache:
                cache[e] = (dequantize(gate_type, gate[e * I:(e + 1) * I], H).astype(np.float64),
                            dequantize(gate_type, up[e * I:(e + 1) * I], H).astype(np.float64),
                            dequantize(down_type, down[e * H:(e + 1) * H], I).astype(np.float64))
            g, u, d = cache[e]
            h = silu(g @ xt) * (u @ xt)
            out[t] += wj * (d @ h)
    return out


def shared_expert_gate(x_t: np.ndarray, gate_inp) -> np.float32:
    """resolveSharedExpertGate (MoeForwardPass.java:428-442): 1 without the
    gate row, else 1.0f / (1.0f + (float)Math.exp(-s)) in float with exp in
    double, s = x_t . gate_inp as a float (here the exact dot rounded once)."""
    if gate_inp is None:
        return np.float32(1.0)
    s = np.float32(np.dot(np.asarray(x_t, np.float64), np.asarray(gate_inp, np.float64)))
    with np.errstate(over="ignore"):
        e = np.float32(np.exp(np.float64(-s)))
    return np.float32(np.float32(1.0) / (np.float32(1.0) + e))


def moe_shared_expert_reference(gate: np.ndarray, up: np.ndarray, down: np.ndarray, x: np.ndarray,
                                out: np.ndarray, gate_inp=None, gate_type: int = Q4_K,
                                down_type: int = Q4_K) -> np.ndarray:
    """out[t] + g_t * y_t for every token (MoeForwardPass.java:240-247): y_t =
    down(silu(gate x_t) * (up x_t)) (runSharedExpert :418-426, one expert of
    the packed gate / up (I, row bytes of H) and down (H, row bytes of I), in
    fp64 over the bit-exact dequantized weights) and g_t from
    shared_expert_gate; the sum in fp64."""
    x = np.asarray(x, dtype=np.float32)
    T = x.shape[0]
    ids = np.zeros((T, 1), np.int32)
    w = np.ones((T, 1), np.float32)
    y = moe_reference_q4k(gate, up, down, 1, x, ids, w, down_type=down_type, gate_type=gate_type)
    g = np.array([shared_expert_gate(x[t], gate_inp) for t in range(T)], np.float64)
    return np.asarray(out, np.float64) + g[:, None] * y


def rel_err(y, ref) -> float:
    """max_i |y_i - r_i| / max(|r_i|, 1e-3 * ||r||_inf)."""
    y = np.asarray(y, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    if r.size == 0:
        return 0.0
    floor = 1e-3 * np.max(np.abs(r))
    denom = np.maximum(np.abs(r), floor)
    denom[denom == 0] = 1.0
    return float(np.max(np.abs(y - r) / denom))


def normwise_err(y, ref) -> float:
    y = np.asarray(y, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    m = np.max(np.abs(r)) if r.size else 0.0
    return float(np.max(np.abs(y - r)) / m) if m > 0 else float(np.max(np.abs(y - r), initial=0.0))
