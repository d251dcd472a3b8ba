"""GPU parity of tensors uploaded from a GGUF file (MI355X).

A file holding Q4_0, Q8_0 and Q4_K matrices (from under one 4 MiB staging
chunk to 17 of them, so that one copy lane reuses its slots) is opened with
the native loader; each tensor is
uploaded from the file and checked against the oracle: dequantized rows at
the start, at every chunk boundary and at the end bit-exact, the full GEMV
within GEMV_TOL, and bit-identical to the same bytes uploaded from host
memory with gollek_hip_weight_upload.
"""
import numpy as np
import pytest

from gollek_amd import synthetic as syn
from gollek_amd import tensor_ops as ops
from oracle import oracle as o
from gollek_amd import gguf_writer as gw
from tests.test_gpu_gemv import GEMV_TOL, assert_same_bits

pytestmark = pytest.mark.gpu

CHUNK = 4 << 20  # staging chunk of the loader (8 copy lanes, 2 slots each)
Q4_0, Q8_0, Q4_K = 2, 8, 12

# (name, type, rows, cols): 1.6 MB, 33 MB (eight full chunks and a part),
# 71 MB (17 chunks: lane 0 takes chunks 0, 8 and 16, reusing its first
# slot), 0.2 MB (one part chunk).
TENSORS = [("blk.0.attn_q.weight", Q4_0, 300, 4096),
           ("blk.0.ffn_up.weight", Q4_K, 14336, 4096),
           ("blk.0.ffn_down.weight", Q8_0, 8192, 8192),
           ("output.weight", Q4_K, 100, 2048)]


@pytest.fixture(scope="module")
def gguf(tmp_path_factory):
    print("[gpu] init device 0; writing the GGUF file", flush=True)
    ops.init(0)
    blobs, mats = [], {}
    for k, (name, tid, rows, cols) in enumerate(TENSORS):
        data = syn.matrix(tid, rows, cols, seed=900 + k)
        mats[name] = data
        blobs.append((name, (cols, rows), tid, data.tobytes()))
    kvs = [("general.architecture", gw.STRING, "llama"), ("general.alignment", gw.U32, 64),
           ("llama.block_count", gw.U32, 1)]
    raw, _, start, offsets = gw.gguf_file(kvs, blobs, alignment=64)
    path = tmp_path_factory.mktemp("gguf") / "model.gguf"
    path.write_bytes(raw)
    f = ops.GgufFile(path)
    assert f.data_start == start and [t.offset for t in f.tensors] == offsets
    yield f, mats
    f.close()


def _check_rows(t, data, rows, cols, tid):
    rb = o.row_bytes(tid, cols)
    picks = {0, rows - 1}
    for b in range(CHUNK, rows * rb, CHUNK):  # rows holding a chunk's first / last byte
        picks |= {b // rb, (b - 1) // rb}
    for r in sorted(picks):
        got = ops.dequantize_rows(t, r, 1)
        exp = o.dequantize(tid, data, cols, r, 1)
        assert_same_bits(got, exp, f"{t.name} row {r}")


@pytest.mark.parametrize("index", range(len(TENSORS)))
def test_uploaded_tensor_matches_oracle(gguf, index):
    f, mats = gguf
    name, tid, rows, cols = TENSORS[index]
    print(f"[gpu] gguf upload {name} type {tid} {rows}x{cols}", flush=True)
    t = f.tensor(name)
    assert (t.rows, t.columns, t.type_id) == (rows, cols, tid)
    assert np.array_equal(np.asarray(t.data), mats[name].reshape(-1))
    _check_rows(t, mats[name], rows, cols, tid)
    x = syn.activation(cols, seed=77 + index)
    y = np.zeros(rows, np.float32)
    ops.mat_vec(t, x, y)
    ref = o.matvec_fp64(tid, mats[name], cols, x)
    assert o.rel_err(y, ref) <= GEMV_TOL, name
    host = ops.GgufTensor(name, (cols, rows), tid, mats[name])
    y2 = np.zeros(rows, np.float32)
    ops.mat_vec(host, x, y2)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32)), name
    host.close()
    t.close()


def test_repeated_uploads_are_independent_handles(gguf):
    f, mats = gguf
    name, tid, rows, cols = TENSORS[3]
    print("[gpu] gguf repeated uploads", flush=True)
    idx = f.find(name)
    handles = [f.upload(idx) for _ in range(3)]
    assert len(set(handles)) == 3
    from gollek_amd import _native
    lib = _native.load()
    lib.gollek_hip_weight_free(handles[0])
    t = f.tensor(name)
    _check_rows(t, mats[name], rows, cols, tid)
    t.close()
    for h in handles[1:]:
        lib.gollek_hip_weight_free(h)
