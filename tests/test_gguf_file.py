"""CPU tests of the GGUF file loader (open / parse / tensor table / range
checks) through the C ABI.  Parsing and the checks ahead of an upload make no
device call.

The reference's own cases (GGUFParserTest, runner/gguf/gollek-gguf-core/src/
test/java/tech/kayys/gollek/gguf/loader/GGUFParserTest.java:15-31) are
reproduced byte for byte; the type table is pinned by the byte sizes of the
published ggml block layouts, written below as sums of their fields."""
import struct

import numpy as np
import pytest

from gollek_amd import tensor_ops as ops
from oracle import oracle as o
from gollek_amd import gguf_writer as gw

F32, F16, Q4_0, Q8_0, Q4_K = 0, 1, 2, 8, 12

# id -> (elements per block, bytes per block) as field sums of each ggml block.
BLOCKS = {
    0: (1, 4), 1: (1, 2), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8), 30: (1, 2),
    2: (32, 2 + 16),                  # Q4_0: d, 32 x 4-bit
    3: (32, 2 + 2 + 16),              # Q4_1: d, m, quants
    6: (32, 2 + 4 + 16),              # Q5_0: d, qh[4], quants
    7: (32, 2 + 2 + 4 + 16),          # Q5_1: d, m, qh[4], quants
    8: (32, 2 + 32),                  # Q8_0: d, 32 x int8
    9: (32, 2 + 2 + 32),              # Q8_1: d, s, 32 x int8
    10: (256, 16 + 64 + 2 + 2),       # Q2_K: scales, qs, d, dmin
    11: (256, 32 + 64 + 12 + 2),      # Q3_K: hmask, qs, scales, d
    12: (256, 2 + 2 + 12 + 128),      # Q4_K: d, dmin, scales, qs
    13: (256, 2 + 2 + 12 + 32 + 128),  # Q5_K: d, dmin, scales, qh, qs
    14: (256, 128 + 64 + 16 + 2),     # Q6_K: ql, qh, scales, d
    15: (256, 4 + 256 + 16 * 2),      # Q8_K: f32 d, qs, bsums
    16: (256, 2 + 32 * 2),            # IQ2_XXS: d, qs u16[32]
    17: (256, 2 + 32 * 2 + 8),        # IQ2_XS: d, qs, scales
    18: (256, 2 + 3 * 256 // 8),      # IQ3_XXS: d, qs
    19: (256, 2 + 32 + 8 * 2),        # IQ1_S: d, qs, qh u16[8]
    20: (32, 2 + 16),                 # IQ4_NL: d, qs
    21: (256, 2 + 64 + 8 + 32 + 4),   # IQ3_S: d, qs, qh, signs, scales
    22: (256, 2 + 64 + 8 + 8),        # IQ2_S: d, qs, qh, scales
    23: (256, 2 + 2 + 4 + 128),       # IQ4_XS: d, scales_h, scales_l, qs
    29: (256, 32 + 16 + 8),           # IQ1_M: qs, qh, scales
    34: (256, (256 - 4 * 256 // 64) // 5 + 256 // 64 + 2),  # TQ1_0: qs, qh, d
    35: (256, 64 + 2),                # TQ2_0: qs, d
    39: (32, 1 + 16),                 # MXFP4: e8m0 scale, qs
    40: (64, 4 + 32),                 # NVFP4: 4 scales, qs
    41: (128, 2 + 16),                # Q1_0: d, 128 sign bits
}
NOT_LOADABLE = [4, 5, 31, 32, 33, 36, 37, 38, 42, 100, -1]


def _write(tmp_path, data: bytes, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return p


def _reference_minimal(type_id: int, elements: int) -> bytes:
    """GGUFParserTest.minimalGgufWithSingleTensor (:33-51): one tensor "w",
    no KV pairs, the file ending at the 32-aligned data start."""
    b = bytearray(b"GGUF")
    b += struct.pack("<iqq", 3, 1, 0)
    b += struct.pack("<q", 1) + b"w"
    b += struct.pack("<iqiq", 1, elements, type_id, 0)
    b += bytes((-len(b)) % 32)
    return bytes(b)


def test_reference_parses_modern_known_quant_tensor_sizes(tmp_path):
    # GGUFParserTest.java:15-26.
    with ops.GgufFile(_write(tmp_path, _reference_minimal(34, 256))) as f:
        assert f.version == 3
        assert len(f.tensors) == 1
        t = f.tensors[0]
        assert (t.name, t.type_id, t.size_in_bytes) == ("w", 34, 54)


def test_reference_rejects_removed_runtime_repacked_layouts(tmp_path):
    # GGUFParserTest.java:28-31.
    with pytest.raises(ops.UnsupportedOperationError,
                       match=r"Unsupported or misaligned GGUF tensor type 31 with 32 element\(s\)"):
        ops.GgufFile(_write(tmp_path, _reference_minimal(31, 32)))


@pytest.mark.parametrize("type_id", sorted(BLOCKS))
def test_tensor_sizes_follow_block_layouts(tmp_path, type_id):
    block, nbytes = BLOCKS[type_id]
    blobs = [(f"t{k}", dims, type_id, b"") for k, dims in
             enumerate([(block,), (block * 3, 5), (block, 2, 3, 4), (0, 7)])]
    data, _, _, _ = gw.gguf_file([], blobs)
    with ops.GgufFile(_write(tmp_path, data)) as f:
        sizes = [t.size_in_bytes for t in f.tensors]
    assert sizes == [nbytes, 15 * nbytes, 24 * nbytes, 0]
    if block > 1:
        with pytest.raises(ops.UnsupportedOperationError, match="misaligned"):
            ops.GgufFile(_write(tmp_path, gw.gguf_file([], [("x", (block + 1,), type_id, b"")])[0],
                                "odd.gguf"))


def test_quant_block_sizes_agree_with_the_oracle():
    for type_id in (Q4_0, Q8_0, Q4_K):
        block, nbytes = BLOCKS[type_id]
        assert o.row_bytes(type_id, block * 4) == 4 * nbytes


@pytest.mark.parametrize("type_id", NOT_LOADABLE)
def test_unknown_and_repacked_types_are_rejected(tmp_path, type_id):
    data = gw.gguf_file([], [("w", (256,), type_id, b"")])[0]
    with pytest.raises(ops.UnsupportedOperationError, match=f"tensor type {type_id} with 256"):
        ops.GgufFile(_write(tmp_path, data))


ALL_KVS = [
    ("general.architecture", gw.STRING, "llama"),
    ("k.u8", gw.U8, 200), ("k.i8", gw.I8, -5), ("k.u16", gw.U16, 60000), ("k.i16", gw.I16, -300),
    ("k.u32", gw.U32, 4_000_000_000), ("k.i32", gw.I32, -7), ("k.f32", gw.F32, 1.5),
    ("k.bool", gw.BOOL, True), ("k.u64", gw.U64, 2 ** 63 + 5), ("k.i64", gw.I64, -(2 ** 40)),
    ("k.f64", gw.F64, -2.25), ("k.utf8 é", gw.STRING, "üß" * 100),
    ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, ["a", "", "中文", "tok" * 50])),
    ("tokenizer.ggml.scores", gw.ARRAY, (gw.F32, [0.5, -1.0, 3.0])),
    ("k.nested", gw.ARRAY, (gw.ARRAY, [(gw.I16, [1, 2, 3]), (gw.STRING, ["x"]), (gw.U8, [])])),
    ("k.empty_unknown", gw.ARRAY, (77, [])),
]


@pytest.mark.parametrize("alignment", [None, 1, 16, 64, 4096])
def test_metadata_is_skipped_and_tensor_table_read(tmp_path, alignment):
    kvs = list(ALL_KVS)
    if alignment is not None:
        kvs.insert(3, ("general.alignment", gw.U32, alignment))
    al = 32 if alignment is None else alignment
    blobs = [("blk.0.ffn_up.weight", (4096, 14336), Q4_K, b""),
             ("blk.0.attn_q.weight", (64, 3), Q8_0, b""),
             ("token_embd.weight", (256, 8), Q4_0, b""),
             ("output_norm.weight", (4096,), F32, b""),
             ("s", (), F32, b"")]
    data, hlen, start, offsets = gw.gguf_file(kvs, blobs, alignment=al, version=2)
    with ops.GgufFile(_write(tmp_path, data)) as f:
        assert (f.version, f.n_kv, f.alignment, f.file_bytes) == (2, len(kvs), al, len(data))
        assert f.data_start % al == 0 and 0 <= f.data_start - hlen < al
        assert f.data_start == start
        assert [t.name for t in f.tensors] == [b[0] for b in blobs]
        assert [t.shape for t in f.tensors] == [b[1] for b in blobs]
        assert [t.type_id for t in f.tensors] == [b[2] for b in blobs]
        assert [t.offset for t in f.tensors] == offsets
        assert [t.size_in_bytes for t in f.tensors] == [4096 // 256 * 144 * 14336, 2 * 34 * 3,
                                                        8 * 8 * 18, 4096 * 4, 4]
        for i, b in enumerate(blobs):
            assert f.find(b[0]) == i
        assert f.find("missing") == -1
        assert f.find("blk.0.ffn_up") == -1


@pytest.mark.parametrize("kv_type,value,expect", [
    (gw.U8, 64, 64), (gw.I16, 128, 128), (gw.I64, 256, 256), (gw.F32, 16.7, 16), (gw.F64, 8.0, 8),
    (gw.U64, 2 ** 32 + 64, 64),  # a 32-bit int is kept: the low 32 bits
])
def test_alignment_value_types(tmp_path, kv_type, value, expect):
    data = gw.header([("general.alignment", kv_type, value)], [("w", (32,), Q8_0, 0)])
    with ops.GgufFile(_write(tmp_path, data)) as f:
        assert f.alignment == expect
        assert f.data_start == gw.padded(len(data), expect)


@pytest.mark.parametrize("kv_type,value", [(gw.BOOL, True), (gw.STRING, "32"), (gw.U32, 0),
                                           (gw.I32, -32), (gw.ARRAY, (gw.U32, [32]))])
def test_alignment_that_is_not_a_positive_number_is_rejected(tmp_path, kv_type, value):
    data = gw.header([("general.alignment", kv_type, value)], [])
    with pytest.raises(ops.IllegalArgumentError, match="alignment"):
        ops.GgufFile(_write(tmp_path, data))


def test_not_a_gguf_file(tmp_path):
    for blob in (b"", b"GGU", b"GGUG" + bytes(40), b"ggUF" + bytes(40)):
        with pytest.raises(ops.IllegalArgumentError, match="Not a valid GGUF file"):
            ops.GgufFile(_write(tmp_path, blob))
    with pytest.raises(ops.IllegalArgumentError, match="Cannot open"):
        ops.GgufFile(tmp_path / "absent.gguf")


def test_unsupported_kv_type_reports_its_position(tmp_path):
    # The position is the cursor after the type field (GGUFParser.java:83-84).
    head = b"GGUF" + struct.pack("<iqq", 3, 0, 2) + gw.string("a") + struct.pack("<iB", gw.U8, 1)
    bad = head + gw.string("b") + struct.pack("<i", 13)
    with pytest.raises(ops.UnsupportedOperationError,
                       match=f"Unsupported GGUF KV type: 13 at pos {len(bad)}$"):
        ops.GgufFile(_write(tmp_path, bad + bytes(16)))
    # Inside an array it is the cursor after the element type and count.
    arr = b"GGUF" + struct.pack("<iqq", 3, 0, 1) + gw.string("c") + struct.pack("<iiq", gw.ARRAY, 13, 2)
    with pytest.raises(ops.UnsupportedOperationError, match=f"KV type: 13 at pos {len(arr)}$"):
        ops.GgufFile(_write(tmp_path, arr + bytes(16)))


def test_every_truncation_of_the_header_is_rejected(tmp_path):
    blobs = [("w", (32, 2), Q8_0, bytes(68)), ("v", (256,), Q4_K, bytes(144))]
    data, hlen, _, _ = gw.gguf_file(ALL_KVS[:8] + ALL_KVS[13:], blobs)
    p = tmp_path / "t.gguf"
    for n in range(hlen):
        p.write_bytes(data[:n])
        with pytest.raises(ops.IllegalArgumentError):
            ops.GgufFile(p)
    p.write_bytes(data[:hlen])
    with ops.GgufFile(p) as f:  # the tensor table is whole; the data is not there
        assert len(f.tensors) == 2


@pytest.mark.parametrize("patch,match", [
    (lambda h: h[:4] + struct.pack("<iqq", 3, 1, 0) + struct.pack("<q", -1), "string length"),
    (lambda h: h[:4] + struct.pack("<iqq", 3, 1, 0) + struct.pack("<q", 2 ** 31), "string length"),
    (lambda h: h[:4] + struct.pack("<iqq", 3, -1, 0), "counts"),
    (lambda h: h[:4] + struct.pack("<iqq", 3, 2 ** 62, 0), "counts"),
    (lambda h: h[:4] + struct.pack("<iqq", 3, 1, 0) + gw.string("w") + struct.pack("<i", 9), "dimensions"),
    (lambda h: h[:4] + struct.pack("<iqq", 3, 1, 0) + gw.string("w") + struct.pack("<iq", 1, -32),
     "shape"),
    (lambda h: h[:4] + struct.pack("<iqq", 3, 1, 0) + gw.string("w") +
     struct.pack("<iqqq", 3, 2 ** 31, 2 ** 31, 2 ** 31), "shape"),
    (lambda h: h[:4] + struct.pack("<iqq", 3, 0, 1) + gw.string("a") +
     struct.pack("<iiq", gw.ARRAY, gw.U8, -1), "array"),
])
def test_malformed_fields_are_rejected(tmp_path, patch, match):
    data = patch(gw.header([], [])) + bytes(64)
    with pytest.raises(ops.IllegalArgumentError, match=match):
        ops.GgufFile(_write(tmp_path, data))


@pytest.mark.parametrize("n_tensors,n_kv", [(2 ** 33, 0), (0, 2 ** 33), (2 ** 31, 2 ** 31)])
def test_counts_beyond_what_the_file_can_hold_are_rejected(tmp_path, n_tensors, n_kv):
    # A 64 GiB sparse file whose header claims more tensor infos (>= 24 bytes
    # each) or metadata entries (>= 12 bytes each) than its bytes can hold is
    # rejected before anything is sized by the counts (this used to reserve
    # a tensor table for 2^33 entries and abort the process).
    p = tmp_path / "sparse.gguf"
    with open(p, "wb") as fh:
        fh.write(b"GGUF" + struct.pack("<iqq", 3, n_tensors, n_kv))
        fh.truncate(64 << 30)
    if p.stat().st_blocks * 512 > (1 << 30):
        pytest.skip("the filesystem does not keep sparse files sparse")
    with pytest.raises(ops.IllegalArgumentError, match="counts"):
        ops.GgufFile(p)


def test_upload_checks_the_tensor_range_before_the_device(tmp_path):
    # GgufTensorData.checkedSlice (RT/GgufTensorData.java:97-104): the bytes
    # must lie inside the file.  Each case fails ahead of any device call.
    blobs = [("in", (32, 2), Q8_0, bytes(68)), ("tail", (32, 1), Q8_0, bytes(34))]
    data, _, start, offsets = gw.gguf_file([], blobs)
    cut = data[:-1]  # "tail" now ends one byte past the end
    hdr = gw.header([], [("neg", (32,), Q8_0, -64), ("far", (32,), Q8_0, 2 ** 62),
                         ("wrap", (32,), Q8_0, 2 ** 63 - 8)])
    with ops.GgufFile(_write(tmp_path, cut)) as f:
        with pytest.raises(ops.IllegalArgumentError,
                           match="Tensor data range is outside model segment: tail"):
            f.upload(f.find("tail"))
        with pytest.raises(ops.IllegalArgumentError, match="outside"):
            f.upload(7)
        with pytest.raises(ops.IllegalArgumentError, match="outside"):
            f.upload(-1)
    with ops.GgufFile(_write(tmp_path, hdr + bytes(4096), "h.gguf")) as f:
        for name in ("neg", "far", "wrap"):
            with pytest.raises(ops.IllegalArgumentError, match=f"outside model segment: {name}$"):
                f.upload(f.find(name))


def test_upload_rejects_types_without_a_kernel_before_the_device(tmp_path):
    blobs = [("norm", (64,), F32, bytes(256)), ("h", (64, 2), F16, bytes(256)),
             ("q2", (256, 2), 10, bytes(168))]
    data = gw.gguf_file([], blobs)[0]
    with ops.GgufFile(_write(tmp_path, data)) as f:
        for name, tid in (("norm", 0), ("h", 1), ("q2", 10)):
            with pytest.raises(ops.UnsupportedOperationError, match=f"type id: {tid}$"):
                f.upload(f.find(name))


def test_tensor_view_reads_the_file_bytes(tmp_path):
    rng = np.random.default_rng(5)
    a = rng.integers(0, 256, 68, dtype=np.uint8).tobytes()
    b = rng.integers(0, 256, 144 * 3, dtype=np.uint8).tobytes()
    data, _, start, offsets = gw.gguf_file([("general.alignment", gw.U32, 128)],
                                           [("a", (32, 2), Q8_0, a), ("b", (256, 3), Q4_K, b)],
                                           alignment=128)
    with ops.GgufFile(_write(tmp_path, data)) as f:
        ta, tb = f.tensor("a"), f.tensor("b")
        assert (ta.rows, ta.columns, tb.rows, tb.columns) == (2, 32, 3, 256)
        assert bytes(ta.data) == a and bytes(tb.data) == b
        assert offsets == [0, 128] and f.data_start == start
        with pytest.raises(ops.IllegalArgumentError, match="not found"):
            f.tensor("c")


def test_close_is_idempotent_and_null_safe(tmp_path):
    f = ops.GgufFile(_write(tmp_path, _reference_minimal(8, 32)))
    f.close()
    f.close()
    from gollek_amd import _native
    _native.load().gollek_hip_gguf_close(None)
    assert _native.load().gollek_hip_gguf_find(None, b"w") == -1
