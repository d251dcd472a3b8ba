"""GPU parity of the Q8_0 x bf16 MFMA GEMM (small-M prefill / batched decode).

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


@pytest.mark.parametrize("rows,cols,m", [(48, 96, 3), (16, 64, 20), (80, 4096, 7), (4096, 192, 130)])
def test_gemm_odd_shapes(rows, cols, m):
    data = syn.q8_0_matrix(rows, cols, seed=rows + cols)
    t = ops.GgufTensor("w", (cols, rows), syn.Q8_0, data.reshape(-1))
    x = syn.activation_bf16(m, cols, seed=1)
    y = np.zeros((m, rows), np.float32)
    ops.gemm_bf16(t, x, y)
    assert o.rel_err(y, o.gemm_reference(syn.Q8_0, data, cols, x)) <= GEMM_TOL
    t.close()


@pytest.mark.parametrize("rows,cols,m,variant", [(128, 256, 300, 0), (64, 128, 5, 2), (192, 4096, 257, 0),
                                                  (64, 64, 128, 2), (4096, 192, 384, 0)])
def test_gemm_large_m_kernel_shapes(rows, cols, m, variant):
    # The 128 x 64 tiled kernel: partial last M tile (rows past M read zeros),
    # several N tiles, K down to one block pair; variant 2 forces it below M = 256.
    print(f"[gpu] gemm large-m rows={rows} cols={cols} m={m} variant={variant}", flush=True)
    data = syn.q8_0_matrix(rows, cols, seed=rows * 7 + cols)
    t = ops.GgufTensor("w", (cols, rows), syn.Q8_0, data.reshape(-1))
    x = syn.activation_bf16(m, cols, seed=m + 3)
    y = np.full((m, rows), np.nan, np.float32)
    ops.set_option("gemm_variant", variant)
    try:
        ops.gemm_bf16(t, x, y)
    finally:
        ops.set_option("gemm_variant", 0)
    assert o.rel_err(y, o.gemm_reference(syn.Q8_0, data, cols, x)) <= GEMM_TOL
    t.close()


@pytest.mark.parametrize("cfg", [0, 5, 1, 3])
@pytest.mark.parametrize("rows,cols,m", [(192, 4096, 300), (4096, 192, 257), (64, 64, 130)])
def test_gemm_large_m_configs(rows, cols, m, cfg):
    # The large-M kernels: the buffer->LDS ring fed by loader waves (cfg 0)
    # or by every wave (cfg 5), K from one block pair, fewer stages than ring
    # slots, up to 64 stages; and two register-pipelined configurations.
    print(f"[gpu] gemm large-m cfg={cfg} rows={rows} cols={cols} m={m}", flush=True)
    data = syn.q8_0_matrix(rows, cols, seed=rows + cols + cfg)
    t = ops.GgufTensor("w", (cols, rows), syn.Q8_0, data.reshape(-1))
    x = syn.activation_bf16(m, cols, seed=m + cfg)
    y = np.full((m, rows), np.nan, np.float32)
    ops.set_option("gemm_big_config", cfg)
    try:
        ops.gemm_bf16(t, x, y)
    finally:
        ops.set_option("gemm_big_config", 0)
    assert o.rel_err(y, o.gemm_reference(syn.Q8_0, data, cols, x)) <= GEMM_TOL
    t.close()


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


def test_gemm_rejects_other_types_and_short_buffers():
    data = syn.q4_k_matrix(16, 256, seed=1)
    t = ops.GgufTensor("w", (256, 16), syn.Q4_K, data.reshape(-1))
    with pytest.raises(ops.UnsupportedOperationError):
        ops.gemm_bf16(t, np.zeros((2, 256), np.uint16), np.zeros((2, 16), np.float32))
    t.close()
    data = syn.q8_0_matrix(16, 64, seed=1)
    t = ops.GgufTensor("w", (64, 16), syn.Q8_0, data.reshape(-1))
    with pytest.raises(ops.IllegalArgumentError):
        ops.gemm_bf16(t, np.zeros((2, 64), np.uint16), np.zeros((1, 16), np.float32))
    t.close()


def test_gemm_device_entry_matches_host(q8_4096):
    import torch
    data, t = q8_4096
    m = 128
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
