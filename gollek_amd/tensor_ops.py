"""Host-side mirror of gollek's GgufTensorOps facade over libgollek_hip.so.

The reference facade is RT/GgufTensorOps.java (RT/ = runner/gguf/
gollek-gguf-core/src/main/java/tech/kayys/gollek/gguf/runtime/): static
dequantizeRow / dotRow / matVec / matVecParallel / matVecRows over a
(GGUFModel, GGUFTensorInfo) pair whose bytes live in an mmapped file.  Here a
GgufTensor carries the same (name, shape, type id, bytes) facts and uploads its
bytes once to a device handle, the way the Java drop-in would key a handle by
(model, tensor).  Calls have the reference's names, argument meaning and
exceptions:

    NullPointerError       <- GOLLEK_HIP_ERR_NULL      (Objects.requireNonNull)
    IllegalArgumentError   <- GOLLEK_HIP_ERR_ARG       (IllegalArgumentException)
    UnsupportedOperationError <- GOLLEK_HIP_ERR_UNSUPPORTED
    DeviceError            <- GOLLEK_HIP_ERR_DEVICE / NOMEM

Every call goes through the C ABI; there is no host fallback.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _native

BLOCK = {_native.Q4_0: (32, 18), _native.Q8_0: (32, 34), _native.Q4_K: (256, 144),
         _native.Q5_K: (256, 176), _native.Q6_K: (256, 210)}
TYPE_NAMES = {_native.Q4_0: "Q4_0", _native.Q8_0: "Q8_0", _native.Q4_K: "Q4_K",
              _native.Q5_K: "Q5_K", _native.Q6_K: "Q6_K"}


class GgufHipError(RuntimeError):
    code = 0


class NullPointerError(GgufHipError, TypeError):
    code = _native.ERR_NULL


class IllegalArgumentError(GgufHipError, ValueError):
    code = _native.ERR_ARG


class UnsupportedOperationError(GgufHipError, NotImplementedError):
    code = _native.ERR_UNSUPPORTED


class DeviceError(GgufHipError):
    code = _native.ERR_DEVICE


_BY_CODE = {
    _native.ERR_NULL: NullPointerError,
    _native.ERR_ARG: IllegalArgumentError,
    _native.ERR_UNSUPPORTED: UnsupportedOperationError,
    _native.ERR_DEVICE: DeviceError,
    _native.ERR_NOMEM: DeviceError,
}


def check(rc: int, err: _native.ErrBuf) -> None:
    if rc != _native.OK:
        raise _BY_CODE.get(rc, GgufHipError)(err.text or f"status {rc}")


def row_bytes_for(type_id: int, cols: int) -> int:
    bs, bb = BLOCK[type_id]
    return cols // bs * bb


def init(device: int = 0) -> None:
    lib = _native.load()
    err = _native.ErrBuf()
    check(lib.gollek_hip_init(device, err.buf, err.size), err)


def set_option(key: str, value: int) -> None:
    """Test-only kernel-family switch (gollek_hip_testing_set_option): the
    parity tests force each GEMV / MoE kernel family onto shapes another one
    is picked for.  Not part of the reference's interface."""
    lib = _native.load()
    err = _native.ErrBuf()
    check(lib.gollek_hip_testing_set_option(key.encode(), int(value), err.buf, err.size), err)


@dataclass
class GgufTensor:
    """GGUFTensorInfo(name, shape, typeId, ...) plus its bytes.

    shape[0] is the column count (contiguous); the remaining dimensions form
    the rows (RT/GgufTensorOps.java:621-630)."""

    name: str
    shape: tuple[int, ...]
    type_id: int
    data: np.ndarray  # uint8, rows * row_bytes
    _handle: int | None = field(default=None, repr=False)
    # set for tensors of a GgufFile: the handle comes from the file upload
    _file: "GgufFile | None" = field(default=None, repr=False)
    _index: int = field(default=-1, repr=False)

    @property
    def columns(self) -> int:
        return int(self.shape[0])

    @property
    def rows(self) -> int:
        r = 1
        for d in self.shape[1:]:
            r *= int(d)
        return r

    @property
    def row_bytes(self) -> int:
        bs, bb = BLOCK.get(self.type_id, (1, 1))
        return self.columns // bs * bb

    def handle(self) -> int:
        """Device handle, created on first use (the prepared-cache analogue)."""
        if self._handle is None and self._file is not None:
            self._handle = self._file.upload(self._index)
        if self._handle is None:
            lib = _native.load()
            err = _native.ErrBuf()
            buf = np.ascontiguousarray(self.data, dtype=np.uint8)
            h = lib.gollek_hip_weight_upload(self.type_id, buf.ctypes.data, self.rows,
                                             self.columns, self.row_bytes, err.buf, err.size)
            if not h:
                raise _BY_CODE.get(lib.gollek_hip_last_status(), GgufHipError)(err.text)
            self._handle = h
        return self._handle

    def prepare(self) -> None:
        """Build the handle's prepared mat-vec layout (gollek_hip_weight_prepare;
        the reference builds its prepared matrices at model load)."""
        err = _native.ErrBuf()
        check(_native.load().gollek_hip_weight_prepare(self.handle(), err.buf, err.size), err)

    def unprepare(self) -> None:
        """Free the prepared layout (gollek_hip_weight_unprepare); full
        mat-vecs read the GGUF bytes again (the prepared-cache clear)."""
        if self._handle is not None:
            err = _native.ErrBuf()
            check(_native.load().gollek_hip_weight_unprepare(self._handle, err.buf, err.size), err)

    def compact(self) -> None:
        """Keep only the prepared layout (gollek_hip_weight_compact): the
        packed bytes are held once; GEMM and MoE then raise
        UnsupportedOperationError."""
        err = _native.ErrBuf()
        check(_native.load().gollek_hip_weight_compact(self.handle(), err.buf, err.size), err)

    def close(self) -> None:
        if self._handle is not None:
            _native.load().gollek_hip_weight_free(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _f32_out(arr, name: str) -> np.ndarray:
    if arr is None:
        raise NullPointerError(name)
    if not (isinstance(arr, np.ndarray) and arr.dtype == np.float32 and arr.flags.c_contiguous):
        raise IllegalArgumentError(f"{name} must be a contiguous float32 array")
    return arr


def _f32_in(arr, name: str) -> np.ndarray:
    if arr is None:
        raise NullPointerError(name)
    return np.ascontiguousarray(arr, dtype=np.float32)


def dequantize_row(tensor: GgufTensor, row: int, dst: np.ndarray) -> None:
    """GgufTensorOps.dequantizeRow (RT/GgufTensorOps.java:636-642)."""
    if tensor is None:
        raise NullPointerError("tensor")
    dst = _f32_out(dst, "dst")
    lib = _native.load()
    err = _native.ErrBuf()
    if dst.size < tensor.columns:
        raise IllegalArgumentError(
            f"Vector length {dst.size} is smaller than columns {tensor.columns}")
    check(lib.gollek_hip_dequantize_rows(tensor.handle(), int(row), 1, dst.ctypes.data,
                                         tensor.columns, err.buf, err.size), err)


def dequantize_rows(tensor: GgufTensor, row0: int, nrows: int) -> np.ndarray:
    """Bit-exact dequantization of a row range (for parity checks)."""
    out = np.empty((max(nrows, 0), tensor.columns), dtype=np.float32)
    lib = _native.load()
    err = _native.ErrBuf()
    check(lib.gollek_hip_dequantize_rows(tensor.handle(), int(row0), int(nrows),
                                         out.ctypes.data, out.size, err.buf, err.size), err)
    return out


def dot_row(tensor: GgufTensor, row: int, vector) -> float:
    """GgufTensorOps.dotRow (RT/GgufTensorOps.java:644-650)."""
    if tensor is None:
        raise NullPointerError("tensor")
    x = _f32_in(vector, "vector")
    out = np.zeros(1, dtype=np.float32)
    lib = _native.load()
    err = _native.ErrBuf()
    check(lib.gollek_hip_dot_row(tensor.handle(), int(row), x.ctypes.data, x.size,
                                 out.ctypes.data, err.buf, err.size), err)
    return float(out[0])


def mat_vec_rows(tensor: GgufTensor, vector, output: np.ndarray, row_count: int,
                 parallel: bool = True) -> None:
    """GgufTensorOps.matVecRows (RT/GgufTensorOps.java:666-674).

    `parallel` is accepted for signature parity; the GPU always runs all
    rows concurrently."""
    if tensor is None:
        raise NullPointerError("tensor")
    x = _f32_in(vector, "vector")
    y = _f32_out(output, "output")
    lib = _native.load()
    err = _native.ErrBuf()
    check(lib.gollek_hip_matvec_rows(tensor.handle(), x.ctypes.data, x.size, y.ctypes.data,
                                     y.size, int(row_count), err.buf, err.size), err)


def mat_vec(tensor: GgufTensor, vector, output: np.ndarray) -> None:
    """GgufTensorOps.matVec (RT/GgufTensorOps.java:658-660)."""
    if tensor is None:
        raise NullPointerError("tensor")
    mat_vec_rows(tensor, vector, output, tensor.rows, False)


def mat_vec_parallel(tensor: GgufTensor, vector, output: np.ndarray) -> None:
    """GgufTensorOps.matVecParallel (RT/GgufTensorOps.java:662-664)."""
    if tensor is None:
        raise NullPointerError("tensor")
    mat_vec_rows(tensor, vector, output, tensor.rows, True)


# ---- GGUF files -------------------------------------------------------------

@dataclass(frozen=True)
class GgufTensorInfo:
    """GC/loader/GGUFTensorInfo.java:8-14 (GC/ = runner/gguf/gollek-gguf-core/
    src/main/java/tech/kayys/gollek/gguf/): name, shape (shape[0] contiguous),
    ggml type id, offset from the data start, size in bytes."""

    name: str
    shape: tuple[int, ...]
    type_id: int
    offset: int
    size_in_bytes: int


class GgufFile:
    """A GGUF file opened through the native parser: the facts GGUFModel holds
    (GC/loader/GGUFParser.java:17-62: version, tensor infos, data start) and a
    device upload per tensor (GC/runtime/GgufTensorData.java:97-104's range
    check, then the weight upload).  Metadata values other than
    general.alignment are not kept."""

    def __init__(self, path):
        lib = _native.load()
        err = _native.ErrBuf()
        self.path = str(path)
        h = lib.gollek_hip_gguf_open(self.path.encode(), err.buf, err.size)
        if not h:
            raise _BY_CODE.get(lib.gollek_hip_last_status(), GgufHipError)(err.text)
        self._h = h
        v, nt, nkv, al, ds, fb = (ctypes.c_int32(), ctypes.c_int64(), ctypes.c_int64(),
                                  ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64())
        lib.gollek_hip_gguf_info(h, *(ctypes.byref(o) for o in (v, nt, nkv, al, ds, fb)))
        self.version, self.n_kv, self.alignment = v.value, nkv.value, al.value
        self.data_start, self.file_bytes = ds.value, fb.value
        self.tensors: list[GgufTensorInfo] = [self._info(i) for i in range(nt.value)]
        self._map = None

    def _info(self, index: int) -> GgufTensorInfo:
        lib = _native.load()
        name = ctypes.create_string_buffer(4096)
        tid, nd = ctypes.c_int32(), ctypes.c_int32()
        dims = (ctypes.c_int64 * 8)()
        off, size = ctypes.c_int64(), ctypes.c_int64()
        rc = lib.gollek_hip_gguf_tensor(self._h, index, name, 4096, ctypes.byref(tid),
                                        ctypes.byref(nd), dims, ctypes.byref(off),
                                        ctypes.byref(size))
        if rc != 0:
            raise _BY_CODE.get(rc, GgufHipError)(f"tensor index {index}")
        return GgufTensorInfo(name.value.decode("utf-8", "replace"),
                              tuple(int(dims[d]) for d in range(nd.value)), tid.value,
                              off.value, size.value)

    def find(self, name: str) -> int:
        """Index of the tensor called `name`, or -1."""
        return int(_native.load().gollek_hip_gguf_find(self._h, name.encode()))

    def upload(self, index: int) -> int:
        """A new device weight handle holding tensor `index` (caller frees it)."""
        lib = _native.load()
        err = _native.ErrBuf()
        h = lib.gollek_hip_gguf_upload(self._h, index, err.buf, err.size)
        if not h:
            raise _BY_CODE.get(lib.gollek_hip_last_status(), GgufHipError)(err.text)
        return h

    def tensor(self, name: str) -> GgufTensor:
        """GgufTensor for `name` whose bytes are a read-only view of the file
        (empty where they fall outside it) and whose handle comes from
        upload()."""
        index = self.find(name)
        if index < 0:
            raise IllegalArgumentError(f"Tensor not found: {name}")
        info = self.tensors[index]
        if self._map is None:
            self._map = np.memmap(self.path, dtype=np.uint8, mode="r")
        start = self.data_start + info.offset
        data = self._map[start:start + info.size_in_bytes] if start >= 0 else self._map[:0]
        return GgufTensor(info.name, info.shape, info.type_id, data, _file=self, _index=index)

    def close(self) -> None:
        if self._h:
            _native.load().gollek_hip_gguf_close(self._h)
            self._h = None
        self._map = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- device-pointer entry points (inputs already resident in HBM) ---------

class DeviceWeight:
    """A handle over GGUF bytes already in device memory (borrowed)."""

    def __init__(self, type_id: int, device_ptr: int, rows: int, cols: int):
        lib = _native.load()
        err = _native.ErrBuf()
        self.type_id, self.rows, self.cols = type_id, rows, cols
        self.row_bytes = row_bytes_for(type_id, cols)
        h = lib.gollek_hip_weight_wrap_device(type_id, ctypes.c_void_p(device_ptr), rows, cols,
                                              self.row_bytes, err.buf, err.size)
        if not h:
            raise _BY_CODE.get(lib.gollek_hip_last_status(), GgufHipError)(err.text)
        self.handle = h

    def prepare(self) -> None:
        """Build the handle's prepared mat-vec layout (gollek_hip_weight_prepare)."""
        err = _native.ErrBuf()
        check(_native.load().gollek_hip_weight_prepare(self.handle, err.buf, err.size), err)

    def unprepare(self) -> None:
        """Free the prepared layout (gollek_hip_weight_unprepare)."""
        err = _native.ErrBuf()
        check(_native.load().gollek_hip_weight_unprepare(self.handle, err.buf, err.size), err)

    def compact(self) -> None:
        """Keep only the prepared layout (gollek_hip_weight_compact)."""
        err = _native.ErrBuf()
        check(_native.load().gollek_hip_weight_compact(self.handle, err.buf, err.size), err)

    def close(self) -> None:
        if self.handle:
            _native.load().gollek_hip_weight_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def matvec(self, x_ptr: int, y_ptr: int, row_count: int | None = None,
               stream: int = 0) -> None:
        lib = _native.load()
        err = _native.ErrBuf()
        rc = lib.gollek_hip_matvec_device(self.handle, ctypes.c_void_p(x_ptr),
                                          ctypes.c_void_p(y_ptr),
                                          self.rows if row_count is None else row_count,
                                          ctypes.c_void_p(stream), err.buf, err.size)
        check(rc, err)

    def dequantize(self, row0: int, nrows: int, dst_ptr: int, stream: int = 0) -> None:
        lib = _native.load()
        err = _native.ErrBuf()
        rc = lib.gollek_hip_dequantize_rows_device(self.handle, row0, nrows,
                                                   ctypes.c_void_p(dst_ptr),
                                                   ctypes.c_void_p(stream), err.buf, err.size)
        check(rc, err)

    def gemm_bf16(self, x_ptr: int, m: int, y_ptr: int, stream: int = 0) -> None:
        lib = _native.load()
        err = _native.ErrBuf()
        rc = lib.gollek_hip_gemm_bf16_device(self.handle, ctypes.c_void_p(x_ptr), m,
                                             ctypes.c_void_p(y_ptr), ctypes.c_void_p(stream),
                                             err.buf, err.size)
        check(rc, err)


def gemm_bf16(tensor: GgufTensor, x_bf16: np.ndarray, output: np.ndarray) -> None:
    """Y = X W^T for a Q8_0, Q4_0 or Q4_K tensor: x_bf16 (m, columns) uint16 bf16 bit patterns,
    output (m, rows) float32.  The reference runs m matVecRows calls instead
    (RT/GgufTensorOps.java:666-674)."""
    if tensor is None:
        raise NullPointerError("tensor")
    if x_bf16 is None:
        raise NullPointerError("input")
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    y = _f32_out(output, "output")
    m = x.shape[0] if x.ndim == 2 else x.size // max(tensor.columns, 1)
    lib = _native.load()
    err = _native.ErrBuf()
    check(lib.gollek_hip_gemm_bf16(tensor.handle(), x.ctypes.data, x.size, int(m), y.ctypes.data,
                                   y.size, err.buf, err.size), err)


def moe_grouped(gate: GgufTensor, up: GgufTensor, down: GgufTensor, n_experts: int, x, ids,
                weights) -> np.ndarray:
    """Grouped MoE expert FFN over Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K experts
    (gate, up and down may differ; the expert loop of MoeForwardPass.computeAccel,
    runner/safetensor/gollek-safetensor-engine/src/main/java/tech/kayys/gollek/
    safetensor/engine/generation/moe/MoeForwardPass.java:217-240): x (tokens,
    hidden) float32, ids (tokens, top_k) int32, weights (tokens, top_k) float32
    -> (tokens, hidden) float32."""
    for name, t in (("gate", gate), ("up", up), ("down", down)):
        if t is None:
            raise NullPointerError(name)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    iv = np.ascontiguousarray(ids, dtype=np.int32)
    wv = np.ascontiguousarray(weights, dtype=np.float32)
    tokens, top_k = iv.shape
    out = np.zeros((tokens, gate.columns), dtype=np.float32)
    lib = _native.load()
    err = _native.ErrBuf()
    check(lib.gollek_hip_moe_grouped(gate.handle(), up.handle(), down.handle(), n_experts,
                                     xv.ctypes.data, tokens, iv.ctypes.data, wv.ctypes.data,
                                     top_k, out.ctypes.data, out.size, err.buf, err.size), err)
    return out


def moe_workspace_bytes(tokens: int, top_k: int, hidden: int, inter: int, n_experts: int) -> int:
    return int(_native.load().gollek_hip_moe_workspace_bytes(tokens, top_k, hidden, inter,
                                                             n_experts))


def moe_grouped_device(gate: DeviceWeight, up: DeviceWeight, down: DeviceWeight, n_experts: int,
                       x_ptr: int, ids_ptr: int, w_ptr: int, tokens: int, top_k: int,
                       out_ptr: int, ws_ptr: int, ws_bytes: int, stream: int = 0) -> None:
    lib = _native.load()
    err = _native.ErrBuf()
    V = ctypes.c_void_p
    rc = lib.gollek_hip_moe_grouped_device(gate.handle, up.handle, down.handle, n_experts,
                                           V(x_ptr), V(ids_ptr), V(w_ptr), tokens, top_k,
                                           V(out_ptr), V(ws_ptr), ws_bytes, V(stream), err.buf,
                                           err.size)
    check(rc, err)


# ---- MoE router and routed block ---------------------------------------------

ROUTER_SOFTMAX = 0
ROUTER_SIGMOID = 1


def router_scoring(model_type: str | None) -> int:
    """The reference's choice (MoeForwardPass.java:174-175): sigmoid when the
    model type contains "qwen" or "moe", softmax otherwise."""
    mt = model_type or ""
    return ROUTER_SIGMOID if ("qwen" in mt or "moe" in mt) else ROUTER_SOFTMAX


def moe_select_topk(logits, top_k: int, scoring: int):
    """Router probabilities and renormalised top-k (MoeForwardPass.java:174-203
    with selectTopK :286-306) on the GPU: logits (tokens, n_experts) float32
    -> ids (tokens, top_k) int32, weights (tokens, top_k) float32."""
    lv = np.ascontiguousarray(logits, dtype=np.float32)
    if lv.ndim != 2:
        raise IllegalArgumentError("logits must be (tokens, n_experts)")
    tokens, n_experts = lv.shape
    ids = np.zeros((tokens, top_k), np.int32)
    w = np.zeros((tokens, top_k), np.float32)
    lib = _native.load()
    err = _native.ErrBuf()
    check(lib.gollek_hip_moe_select_topk(lv.ctypes.data, tokens, n_experts, top_k, scoring,
                                         ids.ctypes.data, w.ctypes.data, err.buf, err.size), err)
    return ids, w


def moe_block(gate: GgufTensor, up: GgufTensor, down: GgufTensor, n_experts: int, x, logits,
              top_k: int, scoring: int) -> np.ndarray:
    """The routed MoE block (MoeForwardPass.java:174-240 after the router
    linear): router on `logits`, then the grouped expert FFN (expert types as
    moe_grouped)."""
    for name, t in (("gate", gate), ("up", up), ("down", down)):
        if t is None:
            raise NullPointerError(name)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    lv = np.ascontiguousarray(logits, dtype=np.float32)
    tokens = xv.shape[0]
    out = np.zeros((tokens, gate.columns), dtype=np.float32)
    lib = _native.load()
    err = _native.ErrBuf()
    check(lib.gollek_hip_moe_block(gate.handle(), up.handle(), down.handle(), n_experts,
                                   xv.ctypes.data, tokens, lv.ctypes.data, top_k, scoring,
                                   out.ctypes.data, out.size, err.buf, err.size), err)
    return out


def moe_block_device(gate: DeviceWeight, up: DeviceWeight, down: DeviceWeight, n_experts: int,
                     x_ptr: int, logits_ptr: int, tokens: int, top_k: int, scoring: int,
                     ids_ptr: int, w_ptr: int, out_ptr: int, ws_ptr: int, ws_bytes: int,
                     stream: int = 0) -> None:
    lib = _native.load()
    err = _native.ErrBuf()
    V = ctypes.c_void_p
    rc = lib.gollek_hip_moe_block_device(gate.handle, up.handle, down.handle, n_experts,
                                         V(x_ptr), V(logits_ptr), tokens, top_k, scoring,
                                         V(ids_ptr), V(w_ptr), V(out_ptr), V(ws_ptr), ws_bytes,
                                         V(stream), err.buf, err.size)
    check(rc, err)


def moe_shared_expert(gate: GgufTensor, up: GgufTensor, down: GgufTensor, x, out,
                      gate_inp=None) -> np.ndarray:
    """The shared expert added to the routed output `out` (MoeForwardPass.java:
    240-247, runSharedExpert :418-426, resolveSharedExpertGate :428-442):
    out[t] + g_t * down(silu(gate x_t) * (up x_t)) with g_t = sigmoid(x_t .
    gate_inp) (1 without gate_inp).  Returns the new output; `out` is not
    modified."""
    for name, t in (("gate", gate), ("up", up), ("down", down)):
        if t is None:
            raise NullPointerError(name)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    res = np.array(out, dtype=np.float32, order="C", copy=True)
    gi = None if gate_inp is None else np.ascontiguousarray(gate_inp, dtype=np.float32)
    lib = _native.load()
    err = _native.ErrBuf()
    V = ctypes.c_void_p
    check(lib.gollek_hip_moe_shared_expert(gate.handle(), up.handle(), down.handle(),
                                           V(None) if gi is None else V(gi.ctypes.data),
                                           V(xv.ctypes.data), xv.shape[0], V(res.ctypes.data),
                                           res.size, err.buf, err.size), err)
    return res


def moe_shared_workspace_bytes(tokens: int, hidden: int, inter: int) -> int:
    return int(_native.load().gollek_hip_moe_shared_workspace_bytes(tokens, hidden, inter))


def moe_shared_expert_device(gate: DeviceWeight, up: DeviceWeight, down: DeviceWeight,
                             gate_inp_ptr: int, x_ptr: int, tokens: int, out_ptr: int, ws_ptr: int,
                             ws_bytes: int, stream: int = 0) -> None:
    lib = _native.load()
    err = _native.ErrBuf()
    V = ctypes.c_void_p
    rc = lib.gollek_hip_moe_shared_expert_device(gate.handle, up.handle, down.handle,
                                                 V(gate_inp_ptr or None), V(x_ptr), tokens,
                                                 V(out_ptr), V(ws_ptr), ws_bytes, V(stream),
                                                 err.buf, err.size)
    check(rc, err)
