"""GPU parity of the grouped Q4_K MoE expert FFN.

Bar: rel_err <= 1e-3 against the fp64 restatement of MoeForwardPass's expert
loop over the bit-exact dequantized experts.
"""
import numpy as np
import pytest

from gollek_amd import synthetic as syn
from gollek_amd import tensor_ops as ops
from oracle import oracle as o

pytestmark = pytest.mark.gpu
MOE_TOL = 1e-3


@pytest.fixture(scope="module", autouse=True)
def _init():
    ops.init(0)


def _experts(E, H, I, seed):
    gate = syn.q4_k_matrix(E * I, H, seed)
    up = syn.q4_k_matrix(E * I, H, seed + 1)
    down = syn.q4_k_matrix(E * H, I, seed + 2)
    tg = ops.GgufTensor("blk.0.ffn_gate_exps.weight", (H, I, E), syn.Q4_K, gate.reshape(-1))
    tu = ops.GgufTensor("blk.0.ffn_up_exps.weight", (H, I, E), syn.Q4_K, up.reshape(-1))
    td = ops.GgufTensor("blk.0.ffn_down_exps.weight", (I, H, E), syn.Q4_K, down.reshape(-1))
    return gate, up, down, tg, tu, td


# The expert passes give each (expert, route group) unit its own workgroups
# when the units fit the grid (up to tens per unit here, 3 for the 128-expert
# layer, one at 400 tokens x top-2 over 32 experts: 210 units) and
# split the items evenly past the grid (600 tokens: 314 units).
@pytest.mark.parametrize("E,H,I,T,k", [(8, 512, 256, 4, 2), (16, 1024, 512, 9, 4),
                                       (128, 2048, 768, 16, 8), (32, 512, 256, 400, 2),
                                       (32, 512, 256, 600, 2)])
def test_moe_parity(E, H, I, T, k):
    print(f"[gpu] moe E={E} H={H} I={I} T={T} k={k}", flush=True)
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=E + H)
    ids, w = syn.moe_routing(T, E, k, seed=3)
    x = syn.activation(T * H, seed=4).reshape(T, H)
    out = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    ref = o.moe_reference_q4k(gate, up, down, E, x, ids, w)
    err = o.rel_err(out, ref)
    print(f"[gpu] moe rel_err={err:.3e}", flush=True)
    assert err <= MOE_TOL
    for t in (tg, tu, td):
        t.close()


def test_moe_skips_invalid_routes_and_shares_experts():
    E, H, I, T, k = 8, 512, 256, 6, 3
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=11)
    ids = np.array([[0, 1, 2], [2, 1, 0], [7, -1, 3], [3, 8, 3], [5, 5, 5], [1, 2, 4]], np.int32)
    w = np.array([[0.5, 0.3, 0.2], [0.1, 0.0, 0.9], [0.4, 0.4, 0.2], [0.6, 0.2, 0.2],
                  [0.2, 0.3, 0.5], [1.0, 0.0, 0.0]], np.float32)
    x = syn.activation(T * H, seed=12).reshape(T, H)
    out = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    ref = o.moe_reference_q4k(gate, up, down, E, x, ids, w)
    assert o.rel_err(out, ref) <= MOE_TOL
    assert np.all(np.isfinite(out))
    # tokens = 0 is a no-op
    assert ops.moe_grouped(tg, tu, td, E, np.zeros((0, H), np.float32), np.zeros((0, k), np.int32),
                           np.zeros((0, k), np.float32)).shape == (0, H)
    for t in (tg, tu, td):
        t.close()


def test_moe_rejects_bad_shapes():
    E, H, I = 4, 512, 256  # H != I, so swapped up / down shapes differ
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=21)
    ids, w = syn.moe_routing(2, E, 2, seed=1)
    x = syn.activation(2 * H, seed=2).reshape(2, H)
    with pytest.raises(ops.IllegalArgumentError):
        ops.moe_grouped(tg, tu, td, 3, x, ids, w)  # rows not a multiple of 3 experts
    with pytest.raises(ops.IllegalArgumentError):
        ops.moe_grouped(tg, td, tu, E, x, ids, w)  # up / down swapped
    for t in (tg, tu, td):
        t.close()


def test_moe_device_entry_matches_host():
    import torch
    E, H, I, T, k = 16, 1024, 512, 5, 4
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=31)
    ids, w = syn.moe_routing(T, E, k, seed=5)
    x = syn.activation(T * H, seed=6).reshape(T, H)
    host = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    bufs = [torch.from_numpy(a.reshape(-1)).cuda() for a in (gate, up, down)]
    dg = ops.DeviceWeight(syn.Q4_K, bufs[0].data_ptr(), E * I, H)
    du = ops.DeviceWeight(syn.Q4_K, bufs[1].data_ptr(), E * I, H)
    dd = ops.DeviceWeight(syn.Q4_K, bufs[2].data_ptr(), E * H, I)
    nbytes = ops.moe_workspace_bytes(T, k, H, I, E)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    xd, idd, wd = (torch.from_numpy(a).cuda() for a in (x, ids, w))
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    ops.moe_grouped_device(dg, du, dd, E, xd.data_ptr(), idd.data_ptr(), wd.data_ptr(), T, k,
                           out.data_ptr(), ws.data_ptr(), nbytes,
                           torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), host)
    for d in (dg, du, dd):
        d.close()
    for t in (tg, tu, td):
        t.close()
