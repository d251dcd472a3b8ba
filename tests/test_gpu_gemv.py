"""GPU parity of dequantization and GEMV through the C ABI (MI355X).

Bar: dequantized weights bit-exact with the oracle; GEMV outputs within
rel_err <= 1e-3 (max_i |y_i - r_i| / max(|r_i|, 1e-3 ||r||_inf)) of the fp64
dot over the bit-exact dequantized rows, and within the same bound of the
oracle's Java-order fp32 mat-vec.  The golden fixtures from gollek's own tests
are checked at their own tolerances.
"""
import zlib

import numpy as np
import pytest

from gollek_amd import _native
from gollek_amd import synthetic as syn
from gollek_amd import tensor_ops as ops
from oracle import oracle as o

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3


def _tensor(type_id, data, cols, name="w"):
    rows = data.size // o.row_bytes(type_id, cols)
    return ops.GgufTensor(name, (cols, rows), type_id, np.ascontiguousarray(data).reshape(-1))


def _data(fx):
    return np.frombuffer(bytes.fromhex(fx["data_hex"]), dtype=np.uint8)


def assert_same_bits(got, exp, what=""):
    """Bit-exact where the oracle is a number; NaN exactly where it is NaN.

    NaN sign/payload bits are not part of the contract: the reference's own
    are platform-specific (an x86 JVM returns its negative default NaN for
    invalid operations and propagates the lookup table's canonical NaN, other
    hosts differ) and its tests check NaN with isNaN only
    (TST/GgufF16SpecialTest.java:43)."""
    got = np.asarray(got, np.float32)
    exp = np.asarray(exp, np.float32)
    gn, en = np.isnan(got), np.isnan(exp)
    assert np.array_equal(gn, en), (what, "NaN positions differ")
    assert np.array_equal(got[~en].view(np.uint32), exp[~en].view(np.uint32)), what


@pytest.fixture(scope="module", autouse=True)
def _init():
    print("[gpu] init device 0", flush=True)
    ops.init(0)


def test_golden_fixtures_on_gpu(golden):
    for fx in golden:
        print(f"[gpu] golden {fx['name']}", flush=True)
        t = _tensor(fx["type_id"], _data(fx), fx["cols"], fx["name"])
        if fx["expected_dequant_bits"]:
            got = ops.dequantize_rows(t, 0, fx["rows"])
            exp = np.asarray(fx["expected_dequant_bits"], dtype=np.uint32).view(np.float32)
            assert_same_bits(got, exp, fx["name"])
        if fx["expected_matvec"] is not None:
            vec = np.asarray(fx["vector"], dtype=np.float32)[fx["vector_offset"]:]
            y = np.zeros(fx["row_count"], np.float32)
            ops.mat_vec_rows(t, vec, y, fx["row_count"], True)
            exp = np.asarray(fx["expected_matvec"], dtype=np.float64)
            assert np.all(np.abs(y - exp) <= max(fx["tolerance"], 1e-6 * np.abs(exp).max())), \
                (fx["name"], y, exp)
            for r in range(fx["row_count"]):
                assert ops.dot_row(t, r, vec) == pytest.approx(float(y[r]), rel=1e-6, abs=1e-6)
        t.close()


def test_f16_scale_decode_exhaustive():
    # Every fp16 code as a Q8_0 block scale with all quants = 1: the dequantized
    # block equals the decoded scale, so all 65536 codes are checked bitwise.
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    blocks = np.empty((65536, 34), np.uint8)
    blocks[:, 0] = (codes & 0xFF).astype(np.uint8)
    blocks[:, 1] = (codes >> 8).astype(np.uint8)
    blocks[:, 2:] = 1
    t = _tensor(syn.Q8_0, blocks.reshape(-1), 1024)
    got = ops.dequantize_rows(t, 0, t.rows)
    exp = o.dequantize(syn.Q8_0, blocks.reshape(-1), 1024)
    assert_same_bits(got, exp)
    t.close()


@pytest.mark.parametrize("type_id", [syn.Q8_0, syn.Q4_0, syn.Q4_K])
def test_dequant_bit_exact_random(type_id):
    cols, rows = 4096, 257
    data = syn.matrix(type_id, rows, cols, seed=100 + type_id).copy()
    if type_id == syn.Q4_K:
        specials = [0x0000, 0x8000, 0x7E00, 0x7C00, 0xFC00, 0x0001, 0x8001]
        for r, h in enumerate(specials):
            data[r, 2::144] = h & 0xFF
            data[r, 3::144] = h >> 8
        data[10:20, 4::144] = 0  # zero codes in part of the scale field
    t = _tensor(type_id, data, cols)
    got = ops.dequantize_rows(t, 0, rows)
    exp = o.dequantize(type_id, data, cols)
    assert_same_bits(got, exp)
    # a middle range through the row0 offset
    got2 = ops.dequantize_rows(t, 100, 17)
    assert_same_bits(got2, exp[100:117])
    t.close()


CONFIGS = [
    ("c0_q8_0_4096x4096", syn.Q8_0, 4096, 4096),
    ("c1_q4_0_4096x11008", syn.Q4_0, 11008, 4096),
    ("c2a_q4_k_4096x14336", syn.Q4_K, 14336, 4096),
    ("moe_gate_q4_k_2048x768", syn.Q4_K, 768, 2048),
    ("moe_down_q4_k_768x2048", syn.Q4_K, 2048, 768),
    ("q8_0_odd_blocks_160", syn.Q8_0, 7, 160),
    ("q4_0_odd_blocks_160", syn.Q4_0, 7, 160),
    ("q4_k_5_superblocks", syn.Q4_K, 5, 1280),
    ("q4_k_k8192", syn.Q4_K, 333, 8192),
    ("q4_k_k14336", syn.Q4_K, 129, 14336),
    ("q8_0_k14336", syn.Q8_0, 65, 14336),
]


@pytest.mark.parametrize("name,type_id,rows,cols", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_gemv_parity(name, type_id, rows, cols):
    print(f"[gpu] gemv {name}", flush=True)
    data = syn.matrix(type_id, rows, cols, seed=zlib.crc32(name.encode()) & 0xFFFF)
    x = syn.activation(cols, seed=17)
    t = _tensor(type_id, data, cols, name)
    y = np.zeros(rows, np.float32)
    ops.mat_vec(t, x, y)
    ref = o.matvec_fp64(type_id, data, cols, x)
    assert o.rel_err(y, ref) <= GEMV_TOL, (name, o.rel_err(y, ref))
    java_order = o.matvec(type_id, data, cols, x)
    assert o.rel_err(y, java_order) <= GEMV_TOL
    t.close()


ACCURACY_CONFIGS = [("c0_q8_0", syn.Q8_0, 4096, 4096), ("c1_q4_0", syn.Q4_0, 11008, 4096),
                    ("c2a_q4_k", syn.Q4_K, 14336, 4096), ("q4_k_k2048", syn.Q4_K, 4096, 2048),
                    ("q5_k_4096", syn.Q5_K, 4096, 4096), ("q6_k_14336x4096", syn.Q6_K, 14336, 4096),
                    ("q6_k_k14336", syn.Q6_K, 4096, 14336)]


@pytest.mark.parametrize("name,type_id,rows,cols", ACCURACY_CONFIGS, ids=[c[0] for c in ACCURACY_CONFIGS])
@pytest.mark.parametrize("seed", [1, 2])
def test_gemv_error_within_twice_java_order_fp32(name, type_id, rows, cols, seed):
    # The GPU mat-vec is at least as accurate as the reference's own fp32
    # loop, up to a factor 2: both against the fp64 dot over the bit-exact
    # dequantized rows, on the same inputs.
    print(f"[gpu] accuracy {name} seed {seed}", flush=True)
    data = syn.matrix(type_id, rows, cols, seed=seed)
    x = syn.activation(cols, seed=seed + 1)
    t = _tensor(type_id, data, cols, name)
    y = np.zeros(rows, np.float32)
    ops.mat_vec(t, x, y)
    ref = o.matvec_fp64(type_id, data, cols, x)
    e_gpu = o.rel_err(y, ref)
    e_java = o.rel_err(o.matvec(type_id, data, cols, x), ref)
    print(f"[gpu] accuracy {name} seed {seed}: gpu {e_gpu:.3e} java-order fp32 {e_java:.3e}", flush=True)
    assert e_gpu <= 2.0 * e_java, (e_gpu, e_java)
    t.close()


# Q4_K shapes at the edges of the matrix-core kernels' work split: one row,
# rows around a 16-row tile, odd superblock counts (a half-empty last ring
# stage), K-parts summed across waves (few tiles per workgroup), K = 16384
# (the 64-superblock tables) and an uneven share of rows per workgroup.  For
# K <= 4096 and at most 64 rows per CU (one superblock column per wave):
# 1..64 rows per workgroup (a partial last tile, one row in the last tile),
# fewer superblocks than waves, and one row past the limit (shared tiles).
Q4K_SHAPES = [(1, 256), (15, 512), (17, 768), (33, 4096), (100, 1280), (1000, 2304),
              (4103, 4096), (64, 16384), (40, 8448), (3000, 14336), (14336, 4096),
              (16384, 4096), (16385, 4096), (4096, 2048), (9000, 3840), (257, 4096),
              (15000, 4096), (14500, 2048)]


@pytest.mark.parametrize("rows,cols", Q4K_SHAPES, ids=[f"{r}x{c}" for r, c in Q4K_SHAPES])
def test_q4k_gemv_kernels_agree_with_oracle(rows, cols):
    print(f"[gpu] q4k gemv variants {rows}x{cols}", flush=True)
    data = syn.q4_k_matrix(rows, cols, seed=rows * 7 + cols)
    x = syn.activation(cols, seed=rows + 5)
    t = _tensor(syn.Q4_K, data, cols)
    ref = o.matvec_fp64(syn.Q4_K, data, cols, x)
    try:
        for variant in (0, 3, 1):  # matrix cores (CU block or shared tiles), fp32
            ops.set_option("gemv_variant", variant)
            y = np.zeros(rows, np.float32)
            ops.mat_vec(t, x, y)
            assert o.rel_err(y, ref) <= GEMV_TOL, (variant, o.rel_err(y, ref))
    finally:
        ops.set_option("gemv_variant", 0)
    t.close()


def test_q4k_gemv_special_headers_match_java_order():
    # NaN / infinite / zero / subnormal d and dmin: non-finite results appear
    # in the same rows with the same sign as in the oracle's Java-order
    # mat-vec, and zero min codes keep a non-finite dmin out of the sum
    # (minContribution, RT/GgufKQuantLayout.java:67-69).
    rows, cols = 64, 4096
    data = syn.q4_k_matrix(rows, cols, seed=77).copy()
    specials = [0x0000, 0x8000, 0x7E00, 0x7C00, 0xFC00, 0x0001, 0x8001]
    for i, hbits in enumerate(specials):
        data[i, 0::144] = hbits & 0xFF          # d of every superblock
        data[i, 1::144] = hbits >> 8
        data[16 + i, 2::144] = hbits & 0xFF     # dmin of every superblock
        data[16 + i, 3::144] = hbits >> 8
        data[32 + i, 2::144] = hbits & 0xFF     # dmin, with every min code zero
        data[32 + i, 3::144] = hbits >> 8
        for sb in range(cols // 256):
            base = sb * 144 + 4
            sc = data[32 + i, base:base + 12].copy()
            sc[4:8] = 0      # min codes 0-3 and the high bits of min codes 4-7
            sc[8:12] &= 0x0F  # low bits of min codes 4-7
            data[32 + i, base:base + 12] = sc
    x = syn.activation(cols, seed=78)
    t = _tensor(syn.Q4_K, data, cols)
    exp = o.matvec(syn.Q4_K, data, cols, x)
    assert np.all(np.isfinite(exp[32:39])), "zero min codes must hide dmin"
    try:
        for variant in (0, 3):
            ops.set_option("gemv_variant", variant)
            y = np.zeros(rows, np.float32)
            ops.mat_vec(t, x, y)
            assert np.array_equal(np.isnan(y), np.isnan(exp)), (variant, y, exp)
            assert np.array_equal(np.isposinf(y), np.isposinf(exp)), variant
            assert np.array_equal(np.isneginf(y), np.isneginf(exp)), variant
            fin = np.isfinite(exp)
            assert o.rel_err(y[fin], exp[fin]) <= GEMV_TOL, variant
    finally:
        ops.set_option("gemv_variant", 0)
    t.close()


# Q8_0 / Q4_0 shapes at the edges of the ring kernel's split (workgroups of
# 4 to 16 4-row waves, 512-column items): one row, ragged row counts, a
# single item (fewer than the ring's slots), K = 16384 (all of x in LDS) and
# past it (the fp32 kernels take over), 11 and 16 waves per workgroup with a
# partial last workgroup, the two configurations.
Q80_Q40_SHAPES = [(syn.Q8_0, 1, 512), (syn.Q8_0, 15, 512), (syn.Q8_0, 17, 1536), (syn.Q8_0, 4096, 4096),
                  (syn.Q8_0, 33, 16384), (syn.Q8_0, 6, 16896), (syn.Q4_0, 1, 512), (syn.Q4_0, 7, 1024),
                  (syn.Q4_0, 11008, 4096), (syn.Q4_0, 35, 16384), (syn.Q4_0, 11003, 4096),
                  (syn.Q8_0, 6000, 8192), (syn.Q4_0, 40000, 2048),
                  # the matrix-core column kernel's edges: the most rows per CU
                  # (Q8_0 32, Q4_0 64) and one past them, one superblock
                  # column, an odd number of them, a partial last tile
                  (syn.Q8_0, 8192, 4096), (syn.Q8_0, 8193, 4096), (syn.Q4_0, 16384, 4096),
                  (syn.Q4_0, 16385, 4096), (syn.Q8_0, 4000, 256), (syn.Q4_0, 3000, 2304),
                  (syn.Q8_0, 5000, 2304), (syn.Q4_0, 300, 768),
                  # K a multiple of 32 but not of 512 (the ring's last item
                  # holds fewer than 16 blocks): the 7B FFN down projection,
                  # one block past whole items, fewer blocks than one item
                  (syn.Q4_0, 4096, 11008), (syn.Q8_0, 100, 11008), (syn.Q8_0, 33, 4128),
                  (syn.Q4_0, 17, 160), (syn.Q8_0, 9, 1312)]


@pytest.mark.parametrize("type_id,rows,cols", Q80_Q40_SHAPES,
                         ids=[f"{'q8_0' if t == syn.Q8_0 else 'q4_0'}_{r}x{c}" for t, r, c in Q80_Q40_SHAPES])
def test_q8_0_q4_0_gemv_kernels_agree_with_oracle(type_id, rows, cols):
    print(f"[gpu] q8_0/q4_0 gemv variants type={type_id} {rows}x{cols}", flush=True)
    data = syn.matrix(type_id, rows, cols, seed=rows * 5 + cols + type_id)
    x = syn.activation(cols, seed=rows + 6)
    t = _tensor(type_id, data, cols)
    ref = o.matvec_fp64(type_id, data, cols, x)
    try:
        for variant in (0, 4, 1):  # matrix-core column kernel where it applies, buffer->LDS ring, fp32
            ops.set_option("gemv_variant", variant)
            y = np.zeros(rows, np.float32)
            ops.mat_vec(t, x, y)
            assert o.rel_err(y, ref) <= GEMV_TOL, (variant, o.rel_err(y, ref))
            part = np.full(rows, -3.0, np.float32)
            ops.mat_vec_rows(t, x, part, rows // 2, True)  # a row prefix
            assert np.array_equal(part[:rows // 2], y[:rows // 2]), variant
            assert np.all(part[rows // 2:] == -3.0), variant
    finally:
        ops.set_option("gemv_variant", 0)
    t.close()


@pytest.mark.parametrize("type_id", [syn.Q8_0, syn.Q4_0])
def test_q8_0_q4_0_gemv_special_scales_match_java_order(type_id):
    # NaN / infinite / zero / subnormal block scales on every block of a row:
    # the non-finite results land in the same rows with the same sign as the
    # oracle's Java-order mat-vec (one d_b * sum per block, as there).
    rows, cols = 32, 4096
    bb = 34 if type_id == syn.Q8_0 else 18
    data = syn.matrix(type_id, rows, cols, seed=91 + type_id).copy()
    specials = [0x0000, 0x8000, 0x7E00, 0x7C00, 0xFC00, 0x0001, 0x8001]
    for i, hbits in enumerate(specials):
        data[i, 0::bb] = hbits & 0xFF
        data[i, 1::bb] = hbits >> 8
        data[16 + i, 0:16 * bb:bb] = hbits & 0xFF   # the first 16 blocks only
        data[16 + i, 1:16 * bb:bb] = hbits >> 8
    x = syn.activation(cols, seed=92)
    t = _tensor(type_id, data, cols)
    exp = o.matvec(type_id, data, cols, x)
    try:
        for variant in (0, 4, 1):
            ops.set_option("gemv_variant", variant)
            y = np.zeros(rows, np.float32)
            ops.mat_vec(t, x, y)
            assert np.array_equal(np.isnan(y), np.isnan(exp)), (variant, y, exp)
            assert np.array_equal(np.isposinf(y), np.isposinf(exp)), variant
            assert np.array_equal(np.isneginf(y), np.isneginf(exp)), variant
            fin = np.isfinite(exp)
            assert o.rel_err(y[fin], exp[fin]) <= GEMV_TOL, variant
    finally:
        ops.set_option("gemv_variant", 0)
    t.close()


def _fp64_all_rows(type_id, data, cols, x, chunk=8192):
    """fp64 dot of every row over the bit-exact dequantized rows, a chunk of
    rows at a time (the whole fp64 matrix would not fit in memory)."""
    return np.concatenate([o.matvec_fp64(type_id, data[i:i + chunk], cols, x)
                           for i in range(0, data.shape[0], chunk)])


def test_gemv_lm_head_full_size_all_rows():
    # Q4_K K=4096 x N=128256 (lm_head): full-size GPU run against the fp64 dot
    # and the oracle's Java-order mat-vec on every row, plus linearity in x.
    rows, cols = 128256, 4096
    print("[gpu] gemv lm_head 128256x4096", flush=True)
    data = syn.q4_k_matrix(rows, cols, seed=2024)
    t = _tensor(syn.Q4_K, data, cols, "output.weight")
    x1, x2 = syn.activation(cols, 1), syn.activation(cols, 2)
    y1, y2, y12 = (np.zeros(rows, np.float32) for _ in range(3))
    ops.mat_vec(t, x1, y1)
    ops.mat_vec(t, x2, y2)
    ops.mat_vec(t, (x1 + x2).astype(np.float32), y12)
    err64 = o.rel_err(y1, _fp64_all_rows(syn.Q4_K, data, cols, x1))
    errj = o.rel_err(y1, o.matvec(syn.Q4_K, data, cols, x1))
    print(f"[gpu] gemv lm_head all rows rel_err fp64={err64:.3e} java={errj:.3e}", flush=True)
    assert err64 <= GEMV_TOL and errj <= GEMV_TOL
    lin = y1.astype(np.float64) + y2
    assert o.normwise_err(y12, lin) <= 1e-5
    t.close()


def test_row_count_prefix_zero_and_long_vector():
    data = syn.q4_k_matrix(300, 4096, seed=8)
    t = _tensor(syn.Q4_K, data, 4096)
    x = syn.activation(4096 + 37, seed=9)  # extra entries are ignored
    full = np.zeros(300, np.float32)
    ops.mat_vec(t, x, full)
    part = np.full(300, -7.0, np.float32)
    ops.mat_vec_rows(t, x, part, 123, True)
    assert np.array_equal(part[:123], full[:123])
    assert np.all(part[123:] == -7.0)  # rows beyond row_count untouched
    ops.mat_vec_rows(t, x, part, 0, True)  # no-op
    with pytest.raises(ops.IllegalArgumentError):
        ops.mat_vec_rows(t, x, part, 301, True)
    with pytest.raises(ops.IllegalArgumentError):
        ops.mat_vec_rows(t, x[:100], part, 10, True)
    with pytest.raises(ops.IllegalArgumentError):
        ops.mat_vec_rows(t, x, np.zeros(5, np.float32), 10, True)
    with pytest.raises(ops.IllegalArgumentError):
        ops.dot_row(t, 300, x)
    t.close()


@pytest.mark.parametrize("rows,cols,prefix", [(20000, 4096, 9000), (300, 4096, 1), (2000, 8192, 17),
                                             (700, 16384, 64), (8000, 8192, 256), (30000, 8192, 300)])
def test_q4k_row_prefix(rows, cols, prefix):
    # A prefix of the rows runs on a different work split (or kernel) than
    # the full matrix.  K <= 4096: 9000 rows on the column kernel, 20000 on
    # the shared tiles; each row's sum keeps its order, so the bits agree.
    # K > 4096: the number of K-parts follows the tiles per workgroup, and a
    # row's parts are added in order, so a prefix on another split agrees to
    # rounding (within the parity bar) rather than bit for bit.
    print(f"[gpu] q4k prefix {rows}x{cols} prefix {prefix}", flush=True)
    data = syn.q4_k_matrix(rows, cols, seed=rows + prefix)
    t = _tensor(syn.Q4_K, data, cols)
    x = syn.activation(cols, seed=prefix)
    full = np.zeros(rows, np.float32)
    ops.mat_vec(t, x, full)
    part = np.zeros(prefix, np.float32)
    ops.mat_vec_rows(t, x, part, prefix, True)
    if cols <= 4096:
        assert np.array_equal(part, full[:prefix])
    else:
        assert o.rel_err(part, full[:prefix]) <= 1e-4
        assert o.rel_err(part, o.matvec_fp64(syn.Q4_K, data[:prefix], cols, x)) <= GEMV_TOL
    t.close()


def test_repeated_calls_are_deterministic():
    data = syn.q8_0_matrix(1000, 4096, seed=21)
    t = _tensor(syn.Q8_0, data, 4096)
    x = syn.activation(4096, seed=22)
    a, b = np.zeros(1000, np.float32), np.zeros(1000, np.float32)
    ops.mat_vec(t, x, a)
    ops.mat_vec(t, x, b)
    assert np.array_equal(a, b)
    t.close()


def test_device_pointer_entry_points_match_host():
    import torch
    rows, cols = 4096, 4096
    for type_id in (syn.Q8_0, syn.Q4_0, syn.Q4_K):
        data = syn.matrix(type_id, rows, cols, seed=31 + type_id)
        x = syn.activation(cols, seed=32)
        host_t = _tensor(type_id, data, cols)
        yh = np.zeros(rows, np.float32)
        ops.mat_vec(host_t, x, yh)
        w_dev = torch.from_numpy(data.reshape(-1)).cuda()
        x_dev = torch.from_numpy(x).cuda()
        y_dev = torch.zeros(rows, dtype=torch.float32, device="cuda")
        dw = ops.DeviceWeight(type_id, w_dev.data_ptr(), rows, cols)
        stream = torch.cuda.current_stream().cuda_stream
        dw.matvec(x_dev.data_ptr(), y_dev.data_ptr(), rows, stream)
        deq = torch.empty((3, cols), dtype=torch.float32, device="cuda")
        dw.dequantize(5, 3, deq.data_ptr(), stream)
        torch.cuda.synchronize()
        assert np.array_equal(y_dev.cpu().numpy(), yh)
        exp = o.dequantize(type_id, data, cols, 5, 3)
        assert_same_bits(deq.cpu().numpy(), exp)
        dw.close()
        host_t.close()


# Column-kernel shapes (at most 64 / 48 / 32 rows per CU for Q4_K and Q4_0
# / Q5_K / Q8_0, the last two capped by more workgroups; K <= 4096 one
# column per wave, up to 16384 several; Q4_0 with K <= 4096 in whole 16-row
# tiles per workgroup, as 3001 x 2048: 16 rows on 188 workgroups, the last
# one 9), a ragged one, and shapes with no
# prepared layout (too many rows per CU, Q6_K, K > 16384) where prepare() is
# a no-op.
PREP_SHAPES = [(syn.Q4_K, 14336, 4096), (syn.Q4_K, 1001, 2304), (syn.Q4_K, 4000, 256),
               (syn.Q8_0, 4096, 4096), (syn.Q8_0, 9000, 1024), (syn.Q4_0, 11008, 4096),
               (syn.Q5_K, 4096, 4096), (syn.Q5_K, 12289, 4096), (syn.Q4_K, 16385, 4096),
               (syn.Q6_K, 4096, 4096), (syn.Q4_K, 33, 8192), (syn.Q4_K, 4096, 14336),
               (syn.Q8_0, 4096, 11008), (syn.Q4_0, 1001, 16384), (syn.Q5_K, 3000, 14336),
               (syn.Q4_K, 20000, 6144), (syn.Q8_0, 200, 16896), (syn.Q4_0, 3001, 2048)]


@pytest.mark.parametrize("type_id,rows,cols", PREP_SHAPES,
                         ids=[f"type{t}_{r}x{c}" for t, r, c in PREP_SHAPES])
def test_prepared_layout_matches_gguf_bytes(type_id, rows, cols):
    # The prepared copy holds the same pieces in the column kernel's read
    # order, so a full mat-vec reading it is bit-identical to one reading the
    # GGUF bytes; row prefixes keep reading the GGUF bytes.
    import torch
    print(f"[gpu] prepared layout type={type_id} {rows}x{cols}", flush=True)
    data = syn.matrix(type_id, rows, cols, seed=50 + rows + type_id)
    x = syn.activation(cols, seed=51)
    ref = o.matvec_fp64(type_id, data, cols, x)
    t = _tensor(type_id, data, cols)
    y_raw = np.zeros(rows, np.float32)
    ops.mat_vec(t, x, y_raw)
    assert o.rel_err(y_raw, ref) <= GEMV_TOL
    t.prepare()
    t.prepare()  # idempotent
    y_prep = np.zeros(rows, np.float32)
    ops.mat_vec(t, x, y_prep)
    assert np.array_equal(y_prep, y_raw)
    part = np.full(rows, -3.0, np.float32)
    ops.mat_vec_rows(t, x, part, rows - 1, True)
    assert np.array_equal(part[:rows - 1], y_raw[:rows - 1]) and part[-1] == -3.0
    try:
        # Q4_K variant 3 (shared tiles) and the fp32 / ring variants do not
        # read the layout; back at 0 the layout is used again.
        for variant in (3, 4, 0):
            ops.set_option("gemv_variant", variant)
            y = np.zeros(rows, np.float32)
            ops.mat_vec(t, x, y)
            assert o.rel_err(y, ref) <= GEMV_TOL, variant
        assert np.array_equal(y, y_raw)
    finally:
        ops.set_option("gemv_variant", 0)
    t.close()

    w_dev = torch.from_numpy(data.reshape(-1)).cuda()
    x_dev = torch.from_numpy(x).cuda()
    y_dev = torch.full((rows,), -7.0, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    dw = ops.DeviceWeight(type_id, w_dev.data_ptr(), rows, cols)
    dw.prepare()
    dw.matvec(x_dev.data_ptr(), y_dev.data_ptr(), rows, stream)
    torch.cuda.synchronize()
    assert np.array_equal(y_dev.cpu().numpy(), y_raw)
    y_dev.fill_(-7.0)
    dw.matvec(x_dev.data_ptr(), y_dev.data_ptr(), rows // 2, stream)
    torch.cuda.synchronize()
    got = y_dev.cpu().numpy()
    assert np.all(got[rows // 2:] == -7.0)
    if type_id == syn.Q4_K and cols > 4096:
        # a prefix with another rows-per-CU count may take the other K > 4096
        # kernel (x as 22-bit instead of 30-bit integers): both meet the bar
        assert o.rel_err(got[:rows // 2], ref[:rows // 2]) <= GEMV_TOL
    else:
        assert np.array_equal(got[:rows // 2], y_raw[:rows // 2])
    dw.close()


def test_unprepare_returns_to_the_gguf_bytes():
    # prepare() snapshots a borrowed buffer: after the caller rewrites it, a
    # full mat-vec still reads the old copy until unprepare(), and then
    # equals a never-prepared handle on the new bytes.  Repeated unprepare
    # calls and unprepare without a copy are no-ops.
    import torch
    rows, cols = 14336, 4096
    print(f"[gpu] unprepare Q4_K {rows}x{cols}", flush=True)
    old = syn.matrix(syn.Q4_K, rows, cols, seed=61)
    new = syn.matrix(syn.Q4_K, rows, cols, seed=62)
    x_dev = torch.from_numpy(syn.activation(cols, seed=63)).cuda()
    y_dev = torch.zeros(rows, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    w_dev = torch.from_numpy(old.reshape(-1)).cuda()

    def run(dw):
        y_dev.fill_(-7.0)
        dw.matvec(x_dev.data_ptr(), y_dev.data_ptr(), rows, stream)
        torch.cuda.synchronize()
        return y_dev.cpu().numpy().copy()

    dw = ops.DeviceWeight(syn.Q4_K, w_dev.data_ptr(), rows, cols)
    dw.unprepare()  # nothing to free
    y_old = run(dw)
    dw.prepare()
    assert np.array_equal(run(dw), y_old)
    w_dev.copy_(torch.from_numpy(new.reshape(-1)))
    torch.cuda.synchronize()
    assert np.array_equal(run(dw), y_old)  # the snapshot
    dw.unprepare()
    dw.unprepare()
    y_new = run(dw)
    fresh = ops.DeviceWeight(syn.Q4_K, w_dev.data_ptr(), rows, cols)
    assert np.array_equal(y_new, run(fresh))
    assert not np.array_equal(y_new, y_old)
    dw.prepare()  # a new snapshot of the new bytes
    assert np.array_equal(run(dw), y_new)
    fresh.close()
    dw.close()

    t = _tensor(syn.Q4_K, new, cols)
    t.unprepare()  # no handle yet: nothing to do
    x = x_dev.cpu().numpy()
    y0 = np.zeros(rows, np.float32)
    ops.mat_vec(t, x, y0)
    t.prepare()
    t.unprepare()
    y1 = np.zeros(rows, np.float32)
    ops.mat_vec(t, x, y1)
    assert np.array_equal(y0, y1) and np.array_equal(y0, y_new)
    t.close()


COMPACT_SHAPES = [(syn.Q4_K, 14336, 4096), (syn.Q8_0, 4096, 4096), (syn.Q4_0, 11008, 4096),
                  (syn.Q5_K, 4096, 4096), (syn.Q4_K, 4096, 14336), (syn.Q4_K, 1001, 2304)]


@pytest.mark.parametrize("type_id,rows,cols", COMPACT_SHAPES,
                         ids=[f"type{t}_{r}x{c}" for t, r, c in COMPACT_SHAPES])
def test_compact_handle_holds_one_copy(type_id, rows, cols):
    # After compact() only the prepared layout is held.  Full mat-vecs equal
    # the prepared handle's bit for bit; a prefix and dot_row return exactly
    # the full call's rows; dequantization gathers the rows back from the
    # layout and stays bit-exact; GEMM runs up to four rows of X (two past K
    # = 4096) on the layout and raises past that; unprepare() rebuilds the
    # GGUF copy.
    import ctypes

    import torch
    print(f"[gpu] compact type={type_id} {rows}x{cols}", flush=True)
    data = syn.matrix(type_id, rows, cols, seed=70 + rows + type_id)
    x = syn.activation(cols, seed=71)
    ref = o.matvec_fp64(type_id, data, cols, x)
    t = _tensor(type_id, data, cols)
    t.prepare()
    y_full = np.zeros(rows, np.float32)
    ops.mat_vec(t, x, y_full)
    assert o.rel_err(y_full, ref) <= GEMV_TOL
    rows_sel = [0, rows // 3, rows - 1]
    deq = {r: np.zeros(cols, np.float32) for r in rows_sel}
    for r, dst in deq.items():
        ops.dequantize_row(t, r, dst)
    block = ops.dequantize_rows(t, rows // 2, min(5, rows - rows // 2))
    t.close()

    c = _tensor(type_id, data, cols)
    c.prepare()
    c.compact()
    c.compact()  # idempotent
    y = np.zeros(rows, np.float32)
    ops.mat_vec(c, x, y)
    assert np.array_equal(y, y_full)
    part = np.full(rows, -3.0, np.float32)
    ops.mat_vec_rows(c, x, part, rows - 1, True)
    assert np.array_equal(part[:rows - 1], y_full[:rows - 1]) and part[-1] == -3.0
    for r in rows_sel:
        assert ops.dot_row(c, r, x) == y_full[r]
        got = np.zeros(cols, np.float32)
        ops.dequantize_row(c, r, got)
        assert np.array_equal(got.view(np.uint32), deq[r].view(np.uint32))
    got = ops.dequantize_rows(c, rows // 2, min(5, rows - rows // 2))
    assert np.array_equal(got.view(np.uint32), block.view(np.uint32))
    # GEMM: up to four rows of X (two past K = 4096) run the column kernels
    # on the layout (each row of Y the mat-vec's bits on that X row); more
    # rows need the GGUF rows and raise
    xb = syn.activation_bf16(4, cols, seed=1)
    for m in (1, 2, 4):
        yb = np.full((m, rows), np.nan, np.float32)
        if cols > 4096 and m > 2:
            with pytest.raises(ops.UnsupportedOperationError):
                ops.gemm_bf16(c, xb[:m], yb)
            continue
        ops.gemm_bf16(c, xb[:m], yb)
        for r in range(m):
            g = np.zeros(rows, np.float32)
            ops.mat_vec(c, syn.bf16_to_f32(xb[r]), g)
            assert np.array_equal(yb[r].view(np.uint32), g.view(np.uint32)), (m, r)
    with pytest.raises(ops.UnsupportedOperationError):
        ops.gemm_bf16(c, syn.activation_bf16(5, cols, seed=2), np.zeros((5, rows), np.float32))

    # the device entries of the compact handle (through the C ABI)
    lib = _native.load()
    err = _native.ErrBuf()
    stream = torch.cuda.current_stream().cuda_stream
    xs = torch.zeros(cols + 1, dtype=torch.float32, device="cuda")
    xs[1:] = torch.from_numpy(x).cuda()
    for x_dev in (xs[1:].clone(), xs[1:]):  # 16-byte aligned, then 4 bytes off
        y_dev = torch.full((rows,), -7.0, dtype=torch.float32, device="cuda")
        for n in (rows, rows // 2):
            y_dev.fill_(-7.0)
            rc = lib.gollek_hip_matvec_device(c.handle(), ctypes.c_void_p(x_dev.data_ptr()),
                                              ctypes.c_void_p(y_dev.data_ptr()), n,
                                              ctypes.c_void_p(stream), err.buf, err.size)
            torch.cuda.synchronize()
            assert rc == 0, err.text
            got = y_dev.cpu().numpy()
            assert np.array_equal(got[:n], y_full[:n]) and np.all(got[n:] == -7.0), n
    d_dev = torch.zeros((3, cols), dtype=torch.float32, device="cuda")
    rc = lib.gollek_hip_dequantize_rows_device(c.handle(), rows // 2, min(3, rows - rows // 2),
                                               ctypes.c_void_p(d_dev.data_ptr()), ctypes.c_void_p(stream),
                                               err.buf, err.size)
    torch.cuda.synchronize()
    assert rc == 0, err.text
    n3 = min(3, rows - rows // 2)
    assert np.array_equal(d_dev.cpu().numpy()[:n3].view(np.uint32), block[:n3].view(np.uint32))

    c.unprepare()  # the GGUF rows again, from the layout
    y_raw = np.zeros(rows, np.float32)
    ops.mat_vec(c, x, y_raw)
    assert o.rel_err(y_raw, ref) <= GEMV_TOL
    got = ops.dequantize_rows(c, rows // 2, min(5, rows - rows // 2))
    assert np.array_equal(got.view(np.uint32), block.view(np.uint32))
    c.prepare()
    y2 = np.zeros(rows, np.float32)
    ops.mat_vec(c, x, y2)
    assert np.array_equal(y2, y_full)
    c.close()


def test_compact_needs_an_owned_prepared_handle():
    import torch
    rows, cols = 4096, 4096
    data = syn.matrix(syn.Q6_K, rows, cols, seed=3)
    t = _tensor(syn.Q6_K, data, cols)
    t.prepare()  # no prepared layout for Q6_K: a no-op
    with pytest.raises(ops.UnsupportedOperationError):
        t.compact()
    t.close()
    q = syn.matrix(syn.Q4_K, rows, cols, seed=4)
    w_dev = torch.from_numpy(q.reshape(-1)).cuda()
    dw = ops.DeviceWeight(syn.Q4_K, w_dev.data_ptr(), rows, cols)
    dw.prepare()
    with pytest.raises(ops.IllegalArgumentError):
        dw.compact()  # borrowed bytes
    dw.close()


# ---- Q5_K / Q6_K -----------------------------------------------------------

K56_SHAPES = [(syn.Q5_K, 1, 256), (syn.Q5_K, 7, 768), (syn.Q5_K, 4096, 4096), (syn.Q5_K, 33, 16384),
              (syn.Q5_K, 4096, 14336), (syn.Q5_K, 1001, 6144), (syn.Q5_K, 100, 8192), (syn.Q5_K, 17, 4352),
              (syn.Q5_K, 12545, 4352),
              (syn.Q5_K, 1003, 2304), (syn.Q5_K, 12289, 4096), (syn.Q5_K, 20000, 1024), (syn.Q6_K, 1, 256), (syn.Q6_K, 5, 768), (syn.Q6_K, 4096, 4096),
              (syn.Q6_K, 37, 16384), (syn.Q6_K, 1001, 2304), (syn.Q6_K, 14336, 4096), (syn.Q6_K, 17, 4096),
              (syn.Q6_K, 300, 2048), (syn.Q6_K, 4113, 2048), (syn.Q6_K, 4096, 14336), (syn.Q6_K, 100, 6144),
              (syn.Q6_K, 33, 8192)]


@pytest.mark.parametrize("type_id,rows,cols", K56_SHAPES,
                         ids=[f"{'q5_k' if t == syn.Q5_K else 'q6_k'}_{r}x{c}" for t, r, c in K56_SHAPES])
def test_q5_k_q6_k_dequant_and_gemv(type_id, rows, cols):
    # Odd superblock counts (3, 9) put every other Q6_K superblock at a 2-byte
    # aligned offset; the last row exercises the realigned reads at the end.
    print(f"[gpu] k56 type={type_id} {rows}x{cols}", flush=True)
    data = syn.matrix(type_id, rows, cols, seed=rows * 3 + cols + type_id)
    x = syn.activation(cols, seed=rows + 9)
    t = _tensor(type_id, data, cols)
    for r0, n in {(0, min(rows, 64)), (max(0, rows - 3), min(rows, 3))}:
        assert_same_bits(ops.dequantize_rows(t, r0, n), o.dequantize(type_id, data, cols, r0, n),
                         (type_id, r0))
    ref = o.matvec_fp64(type_id, data, cols, x)
    java = o.matvec(type_id, data, cols, x)
    try:
        # Q5_K with K up to 16384 and Q6_K with K a multiple of 2048 up to
        # 14336: the matrix-core kernels (0) and the fp32 kernel (4); the
        # others run the fp32 kernel either way.
        for variant in (0, 4):
            ops.set_option("gemv_variant", variant)
            y = np.zeros(rows, np.float32)
            ops.mat_vec(t, x, y)
            assert o.rel_err(y, ref) <= GEMV_TOL, (variant, o.rel_err(y, ref))
            assert o.rel_err(y, java) <= GEMV_TOL, (variant, o.rel_err(y, java))
            part = np.full(rows, -3.0, np.float32)
            ops.mat_vec_rows(t, x, part, rows // 2, True)
            assert np.array_equal(part[:rows // 2], y[:rows // 2]), variant
            assert np.all(part[rows // 2:] == -3.0)
            r = rows - 1
            assert ops.dot_row(t, r, x) == pytest.approx(float(y[r]), rel=1e-6, abs=1e-6)
    finally:
        ops.set_option("gemv_variant", 0)
    t.close()


def test_q6_k_lm_head_full_size_all_rows():
    # Q6_K K=4096 x N=128256 (the lm_head type of Q4_K_M files): full-size
    # GPU run against the fp64 dot and the oracle's Java-order mat-vec on
    # every row, plus linearity in x.
    rows, cols = 128256, 4096
    print("[gpu] q6_k gemv lm_head 128256x4096", flush=True)
    data = syn.q6_k_matrix(rows, cols, seed=2025)
    t = _tensor(syn.Q6_K, data, cols, "output.weight")
    x1, x2 = syn.activation(cols, 3), syn.activation(cols, 4)
    y1, y2, y12 = (np.zeros(rows, np.float32) for _ in range(3))
    ops.mat_vec(t, x1, y1)
    ops.mat_vec(t, x2, y2)
    ops.mat_vec(t, (x1 + x2).astype(np.float32), y12)
    err64 = o.rel_err(y1, _fp64_all_rows(syn.Q6_K, data, cols, x1))
    errj = o.rel_err(y1, o.matvec(syn.Q6_K, data, cols, x1))
    print(f"[gpu] q6_k lm_head all rows rel_err fp64={err64:.3e} java={errj:.3e}", flush=True)
    assert err64 <= GEMV_TOL and errj <= GEMV_TOL
    assert o.normwise_err(y12, y1.astype(np.float64) + y2) <= 1e-5
    t.close()


# One shape per kernel family: the column kernel (K = 4096), the wide-row
# kernel (K = 14336 / 11008), the shared-tile and ring kernels (many rows per
# CU, K not a multiple of 256), the K > 4096 Q4_K kernel, Q6_K both paths.
NONFINITE_X = [(syn.Q4_K, 4096, 4096), (syn.Q4_K, 4096, 14336), (syn.Q4_K, 20000, 4096),
               (syn.Q4_K, 20000, 6144), (syn.Q8_0, 4096, 4096), (syn.Q8_0, 300, 4128),
               (syn.Q4_0, 4096, 11008), (syn.Q5_K, 4096, 4096), (syn.Q5_K, 1000, 8192),
               (syn.Q6_K, 4096, 4096), (syn.Q6_K, 1000, 14336)]


@pytest.mark.parametrize("type_id,rows,cols", NONFINITE_X, ids=[f"type{t}_{r}x{c}" for t, r, c in NONFINITE_X])
def test_non_finite_x_poisons_every_row(type_id, rows, cols):
    # A NaN in x makes every row NaN, as in the reference's fp32 loop (every
    # row multiplies it, 0 x NaN included).  An infinity makes every row
    # non-finite in both: the loop gives +-inf or NaN per row (0 x inf,
    # +inf - inf), these kernels NaN (x's scale for that superblock is NaN).
    print(f"[gpu] non-finite x type={type_id} {rows}x{cols}", flush=True)
    data = syn.matrix(type_id, rows, cols, seed=rows + cols + type_id)
    t = _tensor(type_id, data, cols)
    try:
        for variant in (0, 4):
            ops.set_option("gemv_variant", variant)
            for bad in (np.nan, np.inf, -np.inf):
                x = syn.activation(cols, seed=7).copy()
                x[(cols * 2) // 3 + 5] = bad
                y = np.zeros(rows, np.float32)
                ops.mat_vec(t, x, y)
                java = o.matvec(type_id, data, cols, x)
                if np.isnan(bad):
                    assert np.all(np.isnan(y)) and np.all(np.isnan(java)), (variant, bad)
                else:
                    assert not np.any(np.isfinite(y)) and not np.any(np.isfinite(java)), (variant, bad)
    finally:
        ops.set_option("gemv_variant", 0)
    t.close()


UNALIGNED = [(t, off) for t in (syn.Q8_0, syn.Q4_0, syn.Q4_K, syn.Q5_K, syn.Q6_K) for off in (1, 2)]


@pytest.mark.parametrize("type_id,w_off", UNALIGNED, ids=[f"type{t}_w+{o_}" for t, o_ in UNALIGNED])
def test_unaligned_device_buffers(type_id, w_off):
    # Borrowed device buffers at any byte offset: weights 1 or 2 bytes past
    # an aligned address and x 4 bytes past a 16-byte boundary go to the
    # generic kernel (byte loads of the weights, scalar loads of x), which
    # meets the same bar as the fast kernels; an aligned x with the same
    # misaligned weights as well.
    import torch
    rows, cols = 300, 2304
    print(f"[gpu] unaligned type={type_id} w+{w_off}", flush=True)
    data = syn.matrix(type_id, rows, cols, seed=40 + type_id + w_off)
    x = syn.activation(cols, seed=41)
    ref = o.matvec_fp64(type_id, data, cols, x)
    java = o.matvec(type_id, data, cols, x)
    flat = torch.from_numpy(np.ascontiguousarray(data).reshape(-1))
    wbuf = torch.zeros(flat.numel() + 64, dtype=torch.uint8, device="cuda")
    wbuf[w_off:w_off + flat.numel()].copy_(flat.cuda())
    xbuf = torch.zeros(cols + 8, dtype=torch.float32, device="cuda")
    y_dev = torch.zeros(rows, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    dw = ops.DeviceWeight(type_id, wbuf.data_ptr() + w_off, rows, cols)
    for x_off in (1, 0):
        xbuf[x_off:x_off + cols].copy_(torch.from_numpy(x).cuda())
        y_dev.fill_(-5.0)
        dw.matvec(xbuf.data_ptr() + 4 * x_off, y_dev.data_ptr(), rows, stream)
        torch.cuda.synchronize()
        y = y_dev.cpu().numpy()
        assert o.rel_err(y, ref) <= GEMV_TOL, (x_off, o.rel_err(y, ref))
        assert o.rel_err(y, java) <= GEMV_TOL, (x_off, o.rel_err(y, java))
    deq = torch.empty((3, cols), dtype=torch.float32, device="cuda")
    dw.dequantize(7, 3, deq.data_ptr(), stream)
    torch.cuda.synchronize()
    assert_same_bits(deq.cpu().numpy(), o.dequantize(type_id, data, cols, 7, 3))
    dw.close()
