"""GPU parity of the Q8_0 / Q4_0 / Q4_K / Q5_K x bf16 MFMA GEMM and the Q6_K
fp32 MFMA GEMM (small-M prefill / batched decode).

Bar: rel_err <= 1e-2 against the fp64 product of the bf16 activations and the
bit-exact dequantized weights (the quants are contracted exactly and each
block's scale is applied in fp32, so the observed error is ~1e-6).
"""
import numpy as np
import pytest

from gollek_amd import synthetic as syn
from gollek_amd import tensor_ops as ops
from oracle import oracle as o

pytestmark = pytest.mark.gpu
GEMM_TOL = 1e-2


@pytest.fixture(scope="module", autouse=True)
def _init():
    ops.init(0)


@pytest.fixture(scope="module")
def q8_4096():
    data = syn.q8_0_matrix(4096, 4096, seed=77)
    t = ops.GgufTensor("blk.0.attn_q.weight", (4096, 4096), syn.Q8_0, data.reshape(-1))
    yield data, t
    t.close()


@pytest.mark.parametrize("m", [1, 5, 16, 17, 100, 128, 129, 256, 512, 1024])
def test_gemm_parity_4096(q8_4096, m):
    data, t = q8_4096
    print(f"[gpu] gemm m={m}", flush=True)
    x = syn.activation_bf16(m, 4096, seed=m)
    y = np.zeros((m, 4096), np.float32)
    ops.gemm_bf16(t, x, y)
    ref = o.gemm_reference(syn.Q8_0, data, 4096, x)
    err = o.rel_err(y, ref)
    print(f"[gpu] gemm m={m} rel_err={err:.3e}", flush=True)
    assert err <= GEMM_TOL


def test_gemm_row_equals_gemv(q8_4096):
    data, t = q8_4096
    x = syn.activation_bf16(3, 4096, seed=9)
    y = np.zeros((3, 4096), np.float32)
    ops.gemm_bf16(t, x, y)
    for r in range(3):
        xf = syn.bf16_to_f32(x[r])
        g = np.zeros(4096, np.float32)
        ops.mat_vec(t, xf, g)
        assert o.rel_err(y[r], g) <= 1e-4


# M = 1 .. 4 run the GEMV's column kernel with two vectors in each MFMA (the
# second of a pair in A rows 8..15; vectors 2 and 3 in a second operand
# set), and M = 1, 2 past K = 4096 its wide kernel: every row of Y equals,
# bit for bit, the
# mat-vec of that row of X widened to fp32 (the same digits, products and
# sums), and sits within the GEMM bar of the fp64 oracle.  Row counts that
# end in a partial 16-row tile (4000) included.
COLUMN_GEMM_CASES = [(t, r, c, m) for t, r, c in [(syn.Q4_K, 14336, 4096), (syn.Q5_K, 4096, 4096),
                                                   (syn.Q4_0, 11008, 4096), (syn.Q8_0, 4096, 4096),
                                                   (syn.Q8_0, 4000, 2048), (syn.Q4_K, 1792, 4096)]
                     for m in (1, 2, 3, 4)] + \
                    [(t, r, c, m) for t, r, c in [(syn.Q4_K, 4096, 14336), (syn.Q5_K, 4096, 14336),
                                                   (syn.Q4_0, 4096, 11008), (syn.Q8_0, 4096, 8192)]
                     for m in (1, 2)]


@pytest.mark.parametrize("type_id,rows,cols,m", COLUMN_GEMM_CASES)
def test_gemm_small_m_on_the_column_kernel_equals_gemv(type_id, rows, cols, m):
    print(f"[gpu] gemm column kernel type={type_id} m={m} n={rows} k={cols}", flush=True)
    data = syn.matrix(type_id, rows, cols, seed=rows + m)
    t = ops.GgufTensor("w", (cols, rows), type_id, data.reshape(-1))
    x = syn.activation_bf16(m, cols, seed=11 + m)
    y = np.full((m, rows), np.nan, np.float32)
    ops.gemm_bf16(t, x, y)
    for r in range(m):
        g = np.zeros(rows, np.float32)
        ops.mat_vec(t, syn.bf16_to_f32(x[r]), g)
        assert np.array_equal(y[r].view(np.uint32), g.view(np.uint32)), r
    t.close()
    assert o.rel_err(y, o.gemm_reference(type_id, data, cols, x)) <= GEMM_TOL


@pytest.mark.parametrize("rows,cols,m", [(48, 96, 3), (16, 64, 20), (80, 4096, 7), (4096, 192, 130)])
def test_gemm_odd_shapes(rows, cols, m):
    data = syn.q8_0_matrix(rows, cols, seed=rows + cols)
    t = ops.GgufTensor("w", (cols, rows), syn.Q8_0, data.reshape(-1))
    x = syn.activation_bf16(m, cols, seed=1)
    y = np.zeros((m, rows), np.float32)
    ops.gemm_bf16(t, x, y)
    assert o.rel_err(y, o.gemm_reference(syn.Q8_0, data, cols, x)) <= GEMM_TOL
    t.close()


MATRIX = {syn.Q8_0: syn.q8_0_matrix, syn.Q4_0: syn.q4_0_matrix, syn.Q4_K: syn.q4_k_matrix,
          syn.Q5_K: syn.q5_k_matrix, syn.Q6_K: syn.q6_k_matrix}
# (Q6_K rows of an odd superblock count, K = 256 here, are not dword
# multiples and take the fp32 Q6_K kernel instead of the tile kernel.)
TYPES = [syn.Q8_0, syn.Q4_0, syn.Q4_K, syn.Q5_K, syn.Q6_K]


def _gemm_case(type_id, rows, cols, m, seed):
    data = MATRIX[type_id](rows, cols, seed=seed)
    t = ops.GgufTensor("w", (cols, rows), type_id, data.reshape(-1))
    x = syn.activation_bf16(m, cols, seed=seed + 1)
    y = np.full((m, rows), np.nan, np.float32)
    try:
        ops.gemm_bf16(t, x, y)
    finally:
        t.close()
    return y, o.gemm_reference(type_id, data, cols, x)


@pytest.mark.parametrize("type_id", TYPES)
@pytest.mark.parametrize("rows,cols,m", [(128, 256, 33), (192, 4096, 300), (80, 512, 129), (4096, 256, 257),
                                          (1000, 1024, 64), (256, 2048, 1024), (64, 4096, 40), (300, 1024, 96)])
def test_gemm_tile_kernel_shapes(type_id, rows, cols, m):
    # The tile kernel (16 MT x 128 tiles: MT = 8 past M = 64, 4 for M = 33
    # .. 64 and for Q8_0 up to 128 when N has at most 32 column tiles, as
    # at M = 96 here): K from one four-stage round (256) up, a
    # partial last M tile (rows past M read zeros) and N tile (rows past N),
    # one to many tiles, grids that are and are not a multiple of 8, and the
    # K splits the CU count allows (none for K = 256, up to 8).
    print(f"[gpu] gemm tile type={type_id} rows={rows} cols={cols} m={m}", flush=True)
    y, ref = _gemm_case(type_id, rows, cols, m, seed=rows + 3 * cols + m + type_id)
    err = o.rel_err(y, ref)
    print(f"[gpu] gemm tile type={type_id} rel_err={err:.3e}", flush=True)
    assert err <= GEMM_TOL


@pytest.mark.parametrize("type_id", TYPES)
@pytest.mark.parametrize("rows,cols,m", [(100, 512, 5), (1000, 1024, 16), (64, 256, 1), (200, 2048, 32),
                                          (520, 4096, 17), (3000, 4096, 48), (14336, 4096, 8)])
def test_gemm_tile_kernel_small_m(type_id, rows, cols, m):
    # Tiles of 16, 32 and 64 rows of X for M up to 16, 32 and 64 (Q8_0 with
    # 16-row multiples of N and M <= 32 takes the skinny kernel instead).
    print(f"[gpu] gemm small-m type={type_id} rows={rows} cols={cols} m={m}", flush=True)
    y, ref = _gemm_case(type_id, rows, cols, m, seed=rows + 5 * cols + m + type_id)
    err = o.rel_err(y, ref)
    print(f"[gpu] gemm small-m type={type_id} rel_err={err:.3e}", flush=True)
    assert err <= GEMM_TOL


@pytest.mark.parametrize("type_id", [syn.Q4_0, syn.Q4_K, syn.Q5_K, syn.Q6_K])
@pytest.mark.parametrize("m", [16, 128, 512])
def test_gemm_q4_parity_14336(type_id, m):
    # Q4_0 / Q4_K / Q5_K / Q6_K weights at the FFN shape K = 4096, N = 14336.
    print(f"[gpu] gemm q4 type={type_id} m={m} 14336x4096", flush=True)
    y, ref = _gemm_case(type_id, 14336, 4096, m, seed=1400 + m)
    err = o.rel_err(y, ref)
    print(f"[gpu] gemm q4 type={type_id} m={m} rel_err={err:.3e}", flush=True)
    assert err <= GEMM_TOL


# Q4_K rows are whole 256-element superblocks, so only Q4_0 takes the
# K = 64 and K = 96 cases.
@pytest.mark.parametrize(
    "type_id,rows,cols,m",
    [(syn.Q4_0, 48, 96, 3), (syn.Q4_0, 16, 64, 20), (syn.Q4_0, 40, 512, 7), (syn.Q4_0, 20, 768, 5),
     (syn.Q4_K, 40, 512, 7), (syn.Q4_K, 20, 768, 5)])
def test_gemm_q4_generic_shapes(type_id, rows, cols, m):
    # K = 64 and 96 are not multiples of 256: the one-thread-per-output
    # kernel.  K = 512 and 768 with fewer than 128 rows and tokens: one
    # partial tile of the tile kernel.
    print(f"[gpu] gemm generic type={type_id} rows={rows} cols={cols} m={m}", flush=True)
    y, ref = _gemm_case(type_id, rows, cols, m, seed=rows + cols + m)
    assert o.rel_err(y, ref) <= GEMM_TOL


def test_gemm_q4k_special_headers():
    # Q4_K superblocks with zero min codes under a NaN dmin (the min term is
    # skipped, as RT/GgufKQuantLayout.java:67-69), zero d, and a subnormal
    # dmin: the tile kernel equals the fp64 product of the bit-exact rows.
    rows, cols, m = 256, 1024, 160
    data = syn.q4_k_matrix(rows, cols, seed=17).copy()
    blocks = data.reshape(rows, cols // 256, 144)
    blocks[0:16, :, 2:4] = np.frombuffer(np.float16(np.nan).tobytes(), np.uint8)
    blocks[0:16, :, 8:12] = 0  # m codes 0..3 (low 6 bits) and the high bits of 4..7
    blocks[0:16, :, 12:16] &= 0x0F  # low 4 bits of m codes 4..7
    blocks[16:32, :, 0:2] = 0
    blocks[32:48, :, 2:4] = np.frombuffer(np.uint16(1).tobytes(), np.uint8)
    t = ops.GgufTensor("w", (cols, rows), syn.Q4_K, data.reshape(-1))
    x = syn.activation_bf16(m, cols, seed=3)
    y = np.full((m, rows), np.nan, np.float32)
    ops.gemm_bf16(t, x, y)
    t.close()
    ref = o.gemm_reference(syn.Q4_K, data, cols, x)
    assert np.isfinite(ref).all()
    assert o.rel_err(y, ref) <= GEMM_TOL


@pytest.mark.parametrize("rows,cols,m", [(16, 256, 1), (16, 256, 16), (48, 512, 17), (32, 1280, 32),
                                          (64, 4096, 9), (4096, 768, 16), (208, 2048, 31)])
def test_gemm_small_m_ring_shapes(rows, cols, m):
    # The small-M ring kernel: one 16-row tile up to many, K from one stage
    # (fewer stages than ring slots) up, one or two token tiles, partial tiles.
    print(f"[gpu] gemm small-m rows={rows} cols={cols} m={m}", flush=True)
    data = syn.q8_0_matrix(rows, cols, seed=rows * 3 + cols + m)
    t = ops.GgufTensor("w", (cols, rows), syn.Q8_0, data.reshape(-1))
    x = syn.activation_bf16(m, cols, seed=m + 11)
    y = np.full((m, rows), np.nan, np.float32)
    ops.gemm_bf16(t, x, y)
    assert o.rel_err(y, o.gemm_reference(syn.Q8_0, data, cols, x)) <= GEMM_TOL
    t.close()


@pytest.mark.parametrize("rows,cols,m", [(256, 256, 40), (512, 1024, 33), (64, 2048, 200), (64, 1024, 384),
                                          (128, 192, 100), (1024, 4096, 256)])
def test_gemm_split_k_shapes(rows, cols, m):
    # The 128 x 64 tiles split over K when they leave CUs idle: one stage a
    # split (256 x 256), eight splits (N = 64, 512), a partial M tile, an odd
    # stage count that cannot split (K = 192), and two M tiles split in two.
    print(f"[gpu] gemm split-k rows={rows} cols={cols} m={m}", flush=True)
    data = syn.q8_0_matrix(rows, cols, seed=rows + 5 * cols + m)
    t = ops.GgufTensor("w", (cols, rows), syn.Q8_0, data.reshape(-1))
    x = syn.activation_bf16(m, cols, seed=m + 21)
    y = np.full((m, rows), np.nan, np.float32)
    ops.gemm_bf16(t, x, y)
    assert o.rel_err(y, o.gemm_reference(syn.Q8_0, data, cols, x)) <= GEMM_TOL
    t.close()


# Q6_K weights (the Q6_K tensors of Q4_K_M files): the tile kernel for rows
# of an even superblock count (superblocks of odd index start 2 bytes past a
# dword; K = 14336 and M = 512 too), the fp32 matrix-core kernel for odd
# counts (K = 768), with partial tiles on both sides.
@pytest.mark.parametrize("tid,rows,cols,m", [(syn.Q6_K, 4096, 4096, 16), (syn.Q6_K, 33, 768, 1),
                                             (syn.Q6_K, 1024, 4096, 128), (syn.Q6_K, 100, 512, 37),
                                             (syn.Q6_K, 4096, 14336, 24), (syn.Q6_K, 14336, 4096, 512)])
def test_gemm_q5_k_q6_k(tid, rows, cols, m):
    print(f"[gpu] gemm type={tid} rows={rows} cols={cols} m={m}", flush=True)
    data = syn.matrix(tid, rows, cols, rows + cols + m)
    t = ops.GgufTensor("w", (cols, rows), tid, data.reshape(-1))
    x = syn.activation_bf16(m, cols, seed=m + 31)
    y = np.full((m, rows), np.nan, np.float32)
    ops.gemm_bf16(t, x, y)
    t.close()
    err = o.rel_err(y, o.gemm_reference(tid, data, cols, x))
    print(f"[gpu] gemm type={tid} rel_err={err:.3e}", flush=True)
    assert err <= GEMM_TOL


@pytest.mark.parametrize("tid", [syn.Q5_K, syn.Q6_K])
def test_gemm_k_quant_unaligned_x_takes_the_generic_kernel(tid):
    # x 2 bytes past a 16-byte boundary: the Q5_K tile kernel's loads need
    # 16 and the Q6_K kernel's 4, so the device entry runs the per-output
    # fp32 kernel (gemm_kquant_generic_kernel), with the same values.
    import torch
    rows, cols, m = 272, 1024, 9
    data = syn.matrix(tid, rows, cols, 77)
    x = syn.activation_bf16(m, cols, seed=78)
    w_dev = torch.from_numpy(data.reshape(-1)).cuda()
    dw = ops.DeviceWeight(tid, w_dev.data_ptr(), rows, cols)
    try:
        buf = torch.zeros(m * cols + 8, dtype=torch.int16, device="cuda")
        buf[1:1 + m * cols] = torch.from_numpy(x.view(np.int16).reshape(-1)).cuda()
        y_dev = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
        dw.gemm_bf16(buf.data_ptr() + 2, m, y_dev.data_ptr(), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert o.rel_err(y_dev.cpu().numpy(), o.gemm_reference(tid, data, cols, x)) <= GEMM_TOL
    finally:
        dw.close()


def test_gemm_rejects_short_buffers():
    data = syn.q8_0_matrix(16, 64, seed=1)
    t = ops.GgufTensor("w", (64, 16), syn.Q8_0, data.reshape(-1))
    with pytest.raises(ops.IllegalArgumentError):
        ops.gemm_bf16(t, np.zeros((2, 64), np.uint16), np.zeros((1, 16), np.float32))
    t.close()


@pytest.mark.parametrize("m", [128, 512])
def test_gemm_device_entry_matches_host(q8_4096, m):
    # m = 128: eight K splits; m = 512: two (the same kernels in both entries).
    import torch
    data, t = q8_4096
    x = syn.activation_bf16(m, 4096, seed=5)
    yh = np.zeros((m, 4096), np.float32)
    ops.gemm_bf16(t, x, yh)
    w_dev = torch.from_numpy(data.reshape(-1)).cuda()
    x_dev = torch.from_numpy(x.view(np.int16)).cuda()
    y_dev = torch.empty((m, 4096), dtype=torch.float32, device="cuda")
    dw = ops.DeviceWeight(syn.Q8_0, w_dev.data_ptr(), 4096, 4096)
    dw.gemm_bf16(x_dev.data_ptr(), m, y_dev.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(y_dev.cpu().numpy(), yh)
    dw.close()


@pytest.mark.parametrize("m", [64, 384, 40])
def test_gemm_device_entry_split_k_workspace(m):
    # The device entry's workspace is sized at the first call that splits for
    # every later m of the handle (m = 384 needs more than m = 64 here); a
    # y that is not 16-byte aligned runs unsplit.
    import torch
    rows, cols = 64, 1024
    data = syn.q8_0_matrix(rows, cols, seed=31)
    w_dev = torch.from_numpy(data.reshape(-1)).cuda()
    dw = ops.DeviceWeight(syn.Q8_0, w_dev.data_ptr(), rows, cols)
    try:
        for mm in (m, 384, 64):
            print(f"[gpu] gemm device split-k m={mm}", flush=True)
            x = syn.activation_bf16(mm, cols, seed=mm)
            ref = o.gemm_reference(syn.Q8_0, data, cols, x)
            x_dev = torch.from_numpy(x.view(np.int16)).cuda()
            y_dev = torch.full((mm * rows + 1,), float("nan"), dtype=torch.float32, device="cuda")
            for off in (0, 1):
                y_view = y_dev[off:off + mm * rows]
                dw.gemm_bf16(x_dev.data_ptr(), mm, y_view.data_ptr(), torch.cuda.current_stream().cuda_stream)
                torch.cuda.synchronize()
                got = y_view.cpu().numpy().reshape(mm, rows)
                assert o.rel_err(got, ref) <= GEMM_TOL
    finally:
        dw.close()


@pytest.mark.parametrize("type_id,rows,m", [(syn.Q8_0, 4096, 512), (syn.Q4_K, 4096, 512), (syn.Q4_0, 2048, 1024),
                                           (syn.Q5_K, 4096, 128), (syn.Q6_K, 4096, 128)])
def test_gemm_two_split_repeatable(type_id, rows, m):
    # Two K splits added in split order by the reduction kernel: the same
    # bits on every call, within the bar of the oracle, on repeated calls
    # with the handle's workspace reused.
    import torch
    cols = 4096
    data = MATRIX[type_id](rows, cols, seed=rows + m)
    w_dev = torch.from_numpy(data.reshape(-1)).cuda()
    dw = ops.DeviceWeight(type_id, w_dev.data_ptr(), rows, cols)
    stream = torch.cuda.current_stream().cuda_stream
    try:
        for seed in (1, 2):
            print(f"[gpu] gemm two-split type={type_id} rows={rows} m={m} seed={seed}", flush=True)
            x = syn.activation_bf16(m, cols, seed=seed)
            x_dev = torch.from_numpy(x.view(np.int16)).cuda()
            outs = []
            for _ in range(3):
                y_dev = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
                dw.gemm_bf16(x_dev.data_ptr(), m, y_dev.data_ptr(), stream)
                torch.cuda.synchronize()
                outs.append(y_dev.cpu().numpy())
            for o_ in outs[1:]:
                assert np.array_equal(o_.view(np.uint32), outs[0].view(np.uint32))
            assert o.rel_err(outs[0], o.gemm_reference(type_id, data, cols, x)) <= GEMM_TOL
    finally:
        dw.close()
