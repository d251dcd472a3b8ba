"""gollek_hip_gemm_bf16_device_noalloc against gollek_hip_gemm_bf16_device.

The no-allocation entry point runs the same kernels with its split-K
partials in the library's static per-GPU scratch instead of the handle's
workspace, so its output must equal the allocating entry point's bit for
bit, and both must be within the GEMM bar (rel_err <= 1e-2) of the fp64
oracle.  Calls in a row on one handle, each with fewer rows of X than the
one before, all split over K so all use the scratch, and none may read an
earlier call's partials: Q8_0 at 4096 rows (m = 512 with two splits, the
others with more), Q4_K at 14336 rows (m = 128 in 128-row tiles, m = 16 in
16-row tiles), Q4_0 at 4096 rows (m = 300, then 20 in 32-row tiles) and
Q5_K at 4096 rows (m = 64, then 16); Q6_K (the fp32 kernel, no split) too.
"""
import ctypes

import numpy as np
import pytest

from gollek_amd import _native
from gollek_amd import synthetic as syn
from gollek_amd import tensor_ops as ops
from oracle import oracle as o

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-2


@pytest.mark.parametrize("type_id,rows,cols,ms", [(syn.Q8_0, 4096, 4096, (512, 200, 48)),
                                                  (syn.Q4_K, 14336, 4096, (128, 16)),
                                                  (syn.Q4_0, 4096, 4096, (300, 20)),
                                                  (syn.Q5_K, 4096, 4096, (64, 16)),
                                                  (syn.Q6_K, 1024, 2048, (37, 5))])
def test_noalloc_gemm_matches_allocating_entry_point(type_id, rows, cols, ms):
    import torch

    ops.init(0)
    lib = _native.load()
    data = syn.matrix(type_id, rows, cols, seed=404)
    w_dev = torch.from_numpy(data.reshape(-1)).cuda()
    dw = ops.DeviceWeight(type_id, w_dev.data_ptr(), rows, cols)
    stream = torch.cuda.current_stream().cuda_stream
    err = _native.ErrBuf()
    for m in ms:
        print(f"[gpu] noalloc gemm type={type_id} m={m} n={rows} k={cols}", flush=True)
        xb = syn.activation_bf16(m, cols, seed=m)
        x = torch.from_numpy(xb.view("int16")).cuda()
        y_ref = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
        y = torch.full((m, rows), float("nan"), dtype=torch.float32, device="cuda")
        dw.gemm_bf16(x.data_ptr(), m, y_ref.data_ptr(), stream)
        rc = lib.gollek_hip_gemm_bf16_device_noalloc(dw.handle, ctypes.c_void_p(x.data_ptr()), m,
                                                     ctypes.c_void_p(y.data_ptr()),
                                                     ctypes.c_void_p(stream), err.buf, err.size)
        torch.cuda.synchronize()
        assert rc == 0, err.text
        got, ref = y.cpu().numpy(), y_ref.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), m
        exp = o.gemm_reference(type_id, data, cols, xb)
        assert o.rel_err(got.reshape(-1), exp.reshape(-1)) <= GEMM_TOL, m
    dw.close()


def test_noalloc_gemm_checks_arguments():
    import torch

    ops.init(0)
    lib = _native.load()
    data = syn.q8_0_matrix(64, 256, seed=5)
    w_dev = torch.from_numpy(data.reshape(-1)).cuda()
    dw = ops.DeviceWeight(syn.Q8_0, w_dev.data_ptr(), 64, 256)
    err = _native.ErrBuf()
    buf = torch.zeros(64 * 256, dtype=torch.float32, device="cuda")
    # a negative row count of X
    rc = lib.gollek_hip_gemm_bf16_device_noalloc(dw.handle, ctypes.c_void_p(buf.data_ptr()), -1,
                                                 ctypes.c_void_p(buf.data_ptr()), None, err.buf,
                                                 err.size)
    assert rc == _native.ERR_ARG
    rc = lib.gollek_hip_gemm_bf16_device_noalloc(None, ctypes.c_void_p(buf.data_ptr()), 1,
                                                 ctypes.c_void_p(buf.data_ptr()), None, err.buf,
                                                 err.size)
    assert rc == _native.ERR_NULL
    dw.close()
