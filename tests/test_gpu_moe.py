"""GPU parity of the grouped Q4_K MoE expert FFN.

Bar: rel_err <= 1e-3 against the fp64 restatement of MoeForwardPass's expert
loop over the bit-exact dequantized experts.
"""
import numpy as np
import pytest

from gollek_amd import synthetic as syn
from gollek_amd import tensor_ops as ops
from oracle import oracle as o
from tests.test_oracle import (MOE_CF_E, moe_closed_form_case, moe_closed_form_expected,
                               shared_closed_form_case, shared_closed_form_expected)

pytestmark = pytest.mark.gpu
MOE_TOL = 1e-3


@pytest.fixture(scope="module", autouse=True)
def _init():
    ops.init(0)


def _experts(E, H, I, seed, down_type=syn.Q4_K, gate_type=syn.Q4_K):
    gate = syn.matrix(gate_type, E * I, H, seed)
    up = syn.matrix(gate_type, E * I, H, seed + 1)
    down = syn.matrix(down_type, E * H, I, seed + 2)
    tg = ops.GgufTensor("blk.0.ffn_gate_exps.weight", (H, I, E), gate_type, gate.reshape(-1))
    tu = ops.GgufTensor("blk.0.ffn_up_exps.weight", (H, I, E), gate_type, up.reshape(-1))
    td = ops.GgufTensor("blk.0.ffn_down_exps.weight", (I, H, E), down_type, down.reshape(-1))
    return gate, up, down, tg, tu, td


# The expert passes give each (expert, route group) unit its own workgroups
# when that leaves at most 1/8 of the grid idle (8 and 16 experts: tens of
# workgroups per unit) and split the items evenly otherwise (the 128-expert
# layer's 87 units; 210 and 314 units at 400 / 600 tokens x top-2).
# Hidden sizes past 2048 (an even number of superblocks up to 16) cut each
# gate/up tile into two K-halves: 2560 (halves of 5), 3072 (of 6), 4096 (of
# 8, with inter 1536 on the expert-major down pass).  The few-route cases
# give every route group its own workgroups; 300 and 280 tokens x top-2
# (~150 route groups on 256 workgroups) take the even split, whose slices
# start on whole tiles so a tile's two halves stay in one workgroup (with
# the token-major and the expert-major down pass respectively).
@pytest.mark.parametrize("E,H,I,T,k", [(8, 512, 256, 4, 2), (16, 1024, 512, 9, 4),
                                       (128, 2048, 768, 16, 8), (32, 512, 256, 400, 2),
                                       (32, 512, 256, 600, 2), (8, 4096, 1536, 9, 2),
                                       (8, 3072, 512, 5, 2), (16, 2560, 256, 12, 4),
                                       (32, 4096, 256, 300, 2), (16, 3072, 1280, 280, 2)])
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


# Q4_K_M files store some layers' ffn_down_exps as Q6_K: the token-major
# down pass reads them (inter 256 .. 1024; odd rows start 2 bytes off a
# dword, so every tile takes the realigned reads).
@pytest.mark.parametrize("E,H,I,T,k", [(8, 512, 256, 4, 2), (16, 1024, 512, 9, 4),
                                       (128, 2048, 768, 16, 8), (32, 512, 1024, 40, 2),
                                       (8, 4096, 512, 9, 2)])
def test_moe_q6_k_down_parity(E, H, I, T, k):
    print(f"[gpu] moe q6_k down E={E} H={H} I={I} T={T} k={k}", flush=True)
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=E + H + 1, down_type=syn.Q6_K)
    ids, w = syn.moe_routing(T, E, k, seed=5)
    x = syn.activation(T * H, seed=6).reshape(T, H)
    out = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    ref = o.moe_reference_q4k(gate, up, down, E, x, ids, w, down_type=syn.Q6_K)
    err = o.rel_err(out, ref)
    print(f"[gpu] moe q6_k down rel_err={err:.3e}", flush=True)
    assert err <= MOE_TOL
    for t in (tg, tu, td):
        t.close()


# Q5_K gate / up on the matrix-core passes (Q5_K_M / Q5_K_S layers; their
# ring has two 46 KB slots): hidden 512 .. 2048 in one half, 3072 cut into
# K-halves of 6 superblocks; down rows Q6_K / Q4_K / Q5_K on the token-major
# pass (inter 256 .. 1024), Q5_K on the expert-major pass past that (2 to 8
# row tiles per item); Q4_K gate / up with Q5_K down; the even split at 300
# tokens x top-2.
@pytest.mark.parametrize("gt,dt,E,H,I,T,k", [
    (syn.Q5_K, syn.Q6_K, 128, 2048, 768, 16, 8), (syn.Q5_K, syn.Q5_K, 128, 2048, 768, 16, 8),
    (syn.Q5_K, syn.Q4_K, 16, 1536, 512, 9, 4), (syn.Q5_K, syn.Q5_K, 8, 3072, 1536, 9, 2),
    (syn.Q5_K, syn.Q5_K, 32, 512, 256, 300, 2), (syn.Q4_K, syn.Q5_K, 16, 1024, 1280, 9, 4),
    (syn.Q5_K, syn.Q6_K, 8, 2048, 1024, 40, 2), (syn.Q4_K, syn.Q5_K, 16, 1024, 1024, 40, 2),
    (syn.Q5_K, syn.Q5_K, 8, 1024, 512, 9, 4)])
def test_moe_q5_k_parity(gt, dt, E, H, I, T, k):
    print(f"[gpu] moe q5_k gate={gt} down={dt} E={E} H={H} I={I} T={T} k={k}", flush=True)
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=E + H + I + 2, down_type=dt, gate_type=gt)
    ids, w = syn.moe_routing(T, E, k, seed=7)
    x = syn.activation(T * H, seed=8).reshape(T, H)
    out = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    ref = o.moe_reference_q4k(gate, up, down, E, x, ids, w, down_type=dt, gate_type=gt)
    err = o.rel_err(out, ref)
    print(f"[gpu] moe q5_k rel_err={err:.3e}", flush=True)
    assert err <= MOE_TOL
    for t in (tg, tu, td):
        t.close()


# All-Q4_0 experts up to hidden 2048 take the matrix-core passes with Q4_0
# rows (odd and even superblock counts, inter up to 4096, many routes).
# Expert types and shapes the matrix-core passes do not take: Q8_0 / Q4_0
# gate and up or down on the fp32 row kernels (rows of 3 to 448 blocks, 8 to
# 64 lanes per row, route groups limited by LDS, experts with many routes),
# Q6_K gate and up at hidden 512 (the matrix-core gate/up pass since it takes
# Q6_K rows), mixed gate / up types, and
# Q6_K down beyond the token-major down pass (inter above 1024, hidden past
# 2048 with an odd superblock count); also Q5_K gate / up at hidden 4096
# (K-halves of 8) and 1792 (7 superblocks in one half) on the matrix-core
# passes, and Q4_K gate / up with Q6_K down over 2400 routes (token slices).
@pytest.mark.parametrize("gt,dt,E,H,I,T,k", [
    (syn.Q8_0, syn.Q8_0, 128, 2048, 768, 16, 8), (syn.Q4_0, syn.Q4_0, 128, 2048, 768, 16, 8),
    (syn.Q4_0, syn.Q4_0, 4, 512, 14336, 12, 2), (syn.Q8_0, syn.Q8_0, 2, 4096, 1024, 20, 2),
    (syn.Q4_0, syn.Q8_0, 3, 2048, 2048, 33, 3), (syn.Q4_0, syn.Q4_0, 16, 1280, 512, 9, 4),
    (syn.Q4_0, syn.Q4_0, 8, 256, 4096, 5, 2), (syn.Q4_0, syn.Q4_0, 32, 512, 256, 300, 2),
    (syn.Q8_0, syn.Q6_K, 16, 1024, 512, 9, 4), (syn.Q4_0, syn.Q5_K, 16, 512, 256, 7, 2),
    (syn.Q4_K, syn.Q5_K, 8, 512, 256, 5, 2), (syn.Q5_K, syn.Q4_K, 8, 512, 256, 5, 2),
    (syn.Q6_K, syn.Q6_K, 8, 512, 256, 5, 2), (syn.Q4_K, syn.Q8_0, 8, 512, 256, 5, 2),
    (syn.Q4_K, syn.Q6_K, 4, 512, 1280, 6, 2), (syn.Q4_K, syn.Q6_K, 4, 2304, 256, 6, 2),
    (syn.Q4_K, syn.Q6_K, 16, 512, 256, 300, 8), (syn.Q8_0, syn.Q4_0, 8, 96, 160, 5, 2),
    (syn.Q5_K, syn.Q6_K, 4, 4096, 512, 6, 2), (syn.Q5_K, syn.Q5_K, 4, 1792, 512, 6, 2)])
def test_moe_other_types_parity(gt, dt, E, H, I, T, k):
    print(f"[gpu] moe types gate={gt} down={dt} E={E} H={H} I={I} T={T} k={k}", flush=True)
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=E + H + I, down_type=dt, gate_type=gt)
    ids, w = syn.moe_routing(T, E, k, seed=5)
    x = syn.activation(T * H, seed=6).reshape(T, H)
    out = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    ref = o.moe_reference_q4k(gate, up, down, E, x, ids, w, down_type=dt, gate_type=gt)
    err = o.rel_err(out, ref)
    print(f"[gpu] moe types rel_err={err:.3e}", flush=True)
    assert err <= MOE_TOL
    for t in (tg, tu, td):
        t.close()


# Q6_K gate / up experts on the matrix-core gate/up pass (one route per
# MFMA, route groups of two, 210-byte superblocks realigned in LDS): the
# 128-expert layer with Q6_K down (token-major), Q4_K down, Q5_K down past
# inter 1024 (the expert-major down pass), 300 tokens x top-2 (the even
# split), 600 x top-4 (token slices); odd superblock counts (hidden 768) and
# hidden 4096 stay on the row kernels.
@pytest.mark.parametrize("dt,E,H,I,T,k", [
    (syn.Q6_K, 128, 2048, 768, 16, 8), (syn.Q4_K, 16, 1024, 512, 9, 4), (syn.Q5_K, 8, 1536, 1280, 9, 2),
    (syn.Q6_K, 32, 512, 256, 300, 2), (syn.Q6_K, 8, 2048, 1024, 40, 2), (syn.Q6_K, 16, 1024, 512, 600, 4),
    (syn.Q6_K, 8, 768, 256, 5, 2), (syn.Q6_K, 4, 4096, 512, 6, 2)])
def test_moe_q6_k_gate_up_parity(dt, E, H, I, T, k):
    print(f"[gpu] moe q6_k gate/up down={dt} E={E} H={H} I={I} T={T} k={k}", flush=True)
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=E + H + I + 5, down_type=dt, gate_type=syn.Q6_K)
    ids, w = syn.moe_routing(T, E, k, seed=41)
    x = syn.activation(T * H, seed=42).reshape(T, H)
    out = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    ref = o.moe_reference_q4k(gate, up, down, E, x, ids, w, down_type=dt, gate_type=syn.Q6_K)
    err = o.rel_err(out, ref)
    print(f"[gpu] moe q6_k gate/up rel_err={err:.3e}", flush=True)
    assert err <= MOE_TOL
    for t in (tg, tu, td):
        t.close()


# Prefill: more than 2048 routes (tokens x top_k) run the matrix-core passes
# over token slices of 2048 / top_k tokens (256 + 44 at top-8, 512 + 88 at
# top-4, 1024 + 76 and 1024 + 6 at top-2; expert-major down at inter 1280).
# A token's output depends on its own routes only, so the sliced call equals,
# bit for bit, one call per slice, and both are within the bar of the oracle.
@pytest.mark.parametrize("gt,dt,E,H,I,T,k", [
    (syn.Q4_K, syn.Q4_K, 32, 512, 256, 300, 8), (syn.Q5_K, syn.Q6_K, 16, 1024, 512, 600, 4),
    (syn.Q4_0, syn.Q4_0, 32, 512, 256, 1100, 2), (syn.Q4_K, syn.Q5_K, 8, 512, 1280, 1030, 2)])
def test_moe_prefill_token_slices(gt, dt, E, H, I, T, k):
    print(f"[gpu] moe prefill gate={gt} down={dt} E={E} H={H} I={I} T={T} k={k}", flush=True)
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=E + I, down_type=dt, gate_type=gt)
    ids, w = syn.moe_routing(T, E, k, seed=31)
    x = syn.activation(T * H, seed=32).reshape(T, H)
    out = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    ref = o.moe_reference_q4k(gate, up, down, E, x, ids, w, down_type=dt, gate_type=gt)
    err = o.rel_err(out, ref)
    print(f"[gpu] moe prefill rel_err={err:.3e}", flush=True)
    assert err <= MOE_TOL
    step = 2048 // k
    parts = [ops.moe_grouped(tg, tu, td, E, x[t0:t0 + step], ids[t0:t0 + step], w[t0:t0 + step])
             for t0 in range(0, T, step)]
    assert np.array_equal(out.view(np.uint32), np.concatenate(parts).view(np.uint32))
    for t in (tg, tu, td):
        t.close()


@pytest.fixture
def moe_variant():
    def set_variant(v):
        ops.set_option("moe_variant", v)
    yield set_variant
    ops.set_option("moe_variant", 0)


@pytest.mark.parametrize("gt,dt", [(syn.Q4_0, syn.Q4_0), (syn.Q5_K, syn.Q6_K), (syn.Q5_K, syn.Q5_K),
                                   (syn.Q6_K, syn.Q6_K)])
def test_moe_matrix_core_equals_row_kernels(gt, dt, moe_variant):
    # All-Q4_0, Q5_K and Q6_K experts: the matrix-core passes (22-bit x digits)
    # against the fp32 row kernels (moe_variant 1), both against the oracle.
    E, H, I, T, k = 32, 2048, 768, 16, 8
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=21, down_type=dt, gate_type=gt)
    ids, w = syn.moe_routing(T, E, k, seed=22)
    x = syn.activation(T * H, seed=23).reshape(T, H)
    ref = o.moe_reference_q4k(gate, up, down, E, x, ids, w, down_type=dt, gate_type=gt)
    out_mc = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    moe_variant(1)
    out_rows = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    for out in (out_mc, out_rows):
        assert o.rel_err(out, ref) <= MOE_TOL
    assert o.rel_err(out_mc, out_rows) <= MOE_TOL
    for t in (tg, tu, td):
        t.close()


def test_moe_rejects_compacted_experts():
    # A compacted handle holds only the mat-vec layout; the expert passes
    # read GGUF rows and refuse it.
    E, H, I = 8, 512, 256
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=5)
    tg.prepare()
    tg.compact()
    ids, w = syn.moe_routing(3, E, 2, seed=6)
    x = syn.activation(3 * H, seed=7).reshape(3, H)
    with pytest.raises(ops.UnsupportedOperationError):
        ops.moe_grouped(tg, tu, td, E, x, ids, w)
    tg.unprepare()  # GGUF rows rebuilt: the layer runs again
    out = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    assert o.rel_err(out, o.moe_reference_q4k(gate, up, down, E, x, ids, w)) <= MOE_TOL
    for t in (tg, tu, td):
        t.close()


def test_moe_v_dot4_variant_parity(moe_variant):
    # moe_variant 1: the v_dot4 expert kernels at a shape the matrix-core
    # passes also take.
    E, H, I, T, k = 16, 1024, 512, 9, 4
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=E + H)
    ids, w = syn.moe_routing(T, E, k, seed=3)
    x = syn.activation(T * H, seed=4).reshape(T, H)
    moe_variant(1)
    out = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    assert o.rel_err(out, o.moe_reference_q4k(gate, up, down, E, x, ids, w)) <= MOE_TOL
    for t in (tg, tu, td):
        t.close()


@pytest.mark.parametrize("variant", [0, 1])
def test_moe_closed_form(variant, moe_variant):
    # Constant experts and tokens: every output element is
    # sum_j w_j d_e I silu(g_e S_t) u_e S_t (see tests/test_oracle.py).
    gate, up, down, x, ids, w = moe_closed_form_case()
    E, H, I = MOE_CF_E, x.shape[1], gate.shape[0] // MOE_CF_E
    tg = ops.GgufTensor("g", (H, I, E), syn.Q4_K, gate.reshape(-1))
    tu = ops.GgufTensor("u", (H, I, E), syn.Q4_K, up.reshape(-1))
    td = ops.GgufTensor("d", (I, H, E), syn.Q4_K, down.reshape(-1))
    moe_variant(variant)
    out = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    assert o.rel_err(out, moe_closed_form_expected()) <= MOE_TOL
    for t in (tg, tu, td):
        t.close()


@pytest.mark.parametrize("variant", [0, 1])
def test_moe_nan_activation_poisons_only_its_token(variant, moe_variant):
    # A NaN in x makes every output of that token NaN, as in the reference's
    # loop (gate . x is NaN), and leaves the other tokens untouched.
    E, H, I, T, k = 8, 512, 256, 4, 2
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=31)
    ids, w = syn.moe_routing(T, E, k, seed=32)
    x = syn.activation(T * H, seed=33).reshape(T, H)
    x[1, 300] = np.nan
    moe_variant(variant)
    out = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    assert np.all(np.isnan(out[1]))
    keep = [0, 2, 3]
    ref = o.moe_reference_q4k(gate, up, down, E, x[keep], ids[keep], w[keep])
    assert o.rel_err(out[keep], ref) <= MOE_TOL
    for t in (tg, tu, td):
        t.close()


def _nan_dmin_zero_mins(blocks, pb, rows, every=3):
    """Every `every`-th superblock of the given rows: dmin = NaN and all
    eight min codes 0 (scale codes 5), which the reference's minContribution
    (RT/GgufKQuantLayout.java:67-69) keeps out of the sum."""
    b = blocks.reshape(blocks.shape[0], -1, pb)
    hdr = syn.pack_q4k_scales(np.full(8, 5), np.zeros(8, np.int64))
    for r in rows:
        for j in range(0, b.shape[1], every):
            b[r, j, 2], b[r, j, 3] = 0x00, 0x7E  # fp16 NaN
            b[r, j, 4:16] = hdr
    return b.reshape(blocks.shape)


# K-quant experts whose superblocks carry a NaN dmin with all min codes 0:
# the matrix-core passes' non-finite branch (and the row kernels) give the
# reference's finite values for them, on gate / up and on Q4_K / Q5_K down rows.
@pytest.mark.parametrize("gt,dt", [(syn.Q4_K, syn.Q4_K), (syn.Q5_K, syn.Q6_K), (syn.Q5_K, syn.Q5_K),
                                   (syn.Q4_K, syn.Q5_K)])
def test_moe_nan_dmin_with_zero_min_codes(gt, dt):
    E, H, I, T, k = 8, 512, 256, 5, 2
    pb = {syn.Q4_K: 144, syn.Q5_K: 176}
    gate = syn.matrix(gt, E * I, H, 61)
    up = syn.matrix(gt, E * I, H, 62)
    down = syn.matrix(dt, E * H, I, 63)
    rows = range(0, E * I, 5)
    gate = _nan_dmin_zero_mins(gate, pb[gt], rows)
    up = _nan_dmin_zero_mins(up, pb[gt], rows[1:])
    if dt in pb:
        down = _nan_dmin_zero_mins(down, pb[dt], range(0, E * H, 7), every=1)
    ts = [ops.GgufTensor("blk.0.ffn_gate_exps.weight", (H, I, E), gt, gate.reshape(-1)),
          ops.GgufTensor("blk.0.ffn_up_exps.weight", (H, I, E), gt, up.reshape(-1)),
          ops.GgufTensor("blk.0.ffn_down_exps.weight", (I, H, E), dt, down.reshape(-1))]
    ids, w = syn.moe_routing(T, E, k, seed=64)
    x = syn.activation(T * H, seed=65).reshape(T, H)
    ref = o.moe_reference_q4k(gate, up, down, E, x, ids, w, down_type=dt, gate_type=gt)
    assert np.all(np.isfinite(ref))
    out = ops.moe_grouped(*ts, E, x, ids, w)
    assert np.all(np.isfinite(out))
    assert o.rel_err(out, ref) <= MOE_TOL
    for t in ts:
        t.close()


# Q6_K down rows whose codes are all 63 against h that is the same over each
# 16-element quarter (every gate / up row identical, so h is constant per
# token): the quarter's sum q X reaches 16 * 63 * 2^22 * m (m in [0.5, 1)
# the h mantissa), past int32 for nearly every token, so the token-major
# down pass must combine those planes in fp32.
def test_moe_q6_k_down_sums_past_int32():
    E, H, I, T, k = 2, 512, 256, 6, 2
    gate = np.tile(syn.matrix(syn.Q4_K, 1, H, 71), (E * I, 1))
    up = np.tile(syn.matrix(syn.Q4_K, 1, H, 72), (E * I, 1))
    down = syn.matrix(syn.Q6_K, E * H, I, 73).reshape(E * H, I // 256, 210).copy()
    down[..., :192] = 0xFF  # ql nibbles 15, qh bits 3: q = 63
    down[..., 192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)
    down = down.reshape(E * H, -1)
    ts = [ops.GgufTensor("blk.0.ffn_gate_exps.weight", (H, I, E), syn.Q4_K, gate.reshape(-1)),
          ops.GgufTensor("blk.0.ffn_up_exps.weight", (H, I, E), syn.Q4_K, up.reshape(-1)),
          ops.GgufTensor("blk.0.ffn_down_exps.weight", (I, H, E), syn.Q6_K, down.reshape(-1))]
    ids = np.tile(np.arange(E, dtype=np.int32), (T, 1))
    w = np.full((T, k), 0.5, np.float32)
    x = syn.activation(T * H, seed=74).reshape(T, H)
    ref = o.moe_reference_q4k(gate, up, down, E, x, ids, w, down_type=syn.Q6_K, gate_type=syn.Q4_K)
    out = ops.moe_grouped(*ts, E, x, ids, w)
    assert o.rel_err(out, ref) <= MOE_TOL
    for t in ts:
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


# ---- shared expert --------------------------------------------------------------

# The shared expert (one expert, every token, weight g_t) after a routed
# output: Qwen1.5-MoE's shape (hidden 2048, shared inter 5632: past the
# matrix-core passes, on the row kernels), a DeepSeek-style 2 x 1408 (the
# matrix-core passes with Q6_K down), Q8_0 and Q5_K experts, with and
# without the shared_expert_gate row.
@pytest.mark.parametrize("gt,dt,H,I,T,gated", [
    (syn.Q4_K, syn.Q4_K, 2048, 5632, 16, True), (syn.Q4_K, syn.Q6_K, 2048, 2816, 16, True),
    (syn.Q8_0, syn.Q8_0, 1024, 512, 5, False), (syn.Q5_K, syn.Q5_K, 2048, 768, 9, True),
    (syn.Q4_0, syn.Q4_0, 512, 1024, 1, True)])
def test_moe_shared_expert_parity(gt, dt, H, I, T, gated):
    print(f"[gpu] moe shared gate={gt} down={dt} H={H} I={I} T={T} gated={gated}", flush=True)
    gate, up, down, tg, tu, td = _experts(1, H, I, seed=H + I + T, down_type=dt, gate_type=gt)
    x = syn.activation(T * H, seed=9).reshape(T, H)
    routed = syn.activation(T * H, seed=10).reshape(T, H)
    gi = (np.random.default_rng(11).standard_normal(H) / np.sqrt(H)).astype(np.float32) if gated else None
    got = ops.moe_shared_expert(tg, tu, td, x, routed, gate_inp=gi)
    ref = o.moe_shared_expert_reference(gate, up, down, x, routed, gate_inp=gi, gate_type=gt,
                                        down_type=dt)
    err = o.rel_err(got, ref)
    print(f"[gpu] moe shared rel_err={err:.3e}", flush=True)
    assert err <= MOE_TOL
    for t in (tg, tu, td):
        t.close()


def test_moe_shared_expert_closed_form():
    gate, up, down, x, gi = shared_closed_form_case()
    H, I = x.shape[1], gate.shape[0]
    routed = moe_closed_form_expected().astype(np.float32)
    ts = [ops.GgufTensor("blk.0.ffn_gate_shexp.weight", (H, I), syn.Q4_K, gate.reshape(-1)),
          ops.GgufTensor("blk.0.ffn_up_shexp.weight", (H, I), syn.Q4_K, up.reshape(-1)),
          ops.GgufTensor("blk.0.ffn_down_shexp.weight", (I, H), syn.Q4_K, down.reshape(-1))]
    for gate_inp, gated in ((gi, True), (None, False)):
        got = ops.moe_shared_expert(*ts, x, routed, gate_inp=gate_inp)
        exp = shared_closed_form_expected(routed, gated=gated)
        assert o.rel_err(got, exp) <= MOE_TOL
    # a zero gate row gives g = 1/2 exactly: the shared part is half of the ungated one
    half = ops.moe_shared_expert(*ts, x, np.zeros_like(routed), gate_inp=np.zeros(H, np.float32))
    full = ops.moe_shared_expert(*ts, x, np.zeros_like(routed))
    assert np.array_equal(half, np.float32(0.5) * full)
    for t in ts:
        t.close()


def test_moe_shared_expert_device_entry_matches_host():
    import torch
    H, I, T = 1024, 768, 7
    gate, up, down, tg, tu, td = _experts(1, H, I, seed=41)
    x = syn.activation(T * H, seed=42).reshape(T, H)
    routed = syn.activation(T * H, seed=43).reshape(T, H)
    gi = (np.random.default_rng(44).standard_normal(H) / np.sqrt(H)).astype(np.float32)
    host = ops.moe_shared_expert(tg, tu, td, x, routed, gate_inp=gi)
    bufs = [torch.from_numpy(a.reshape(-1)).cuda() for a in (gate, up, down)]
    dg = ops.DeviceWeight(syn.Q4_K, bufs[0].data_ptr(), I, H)
    du = ops.DeviceWeight(syn.Q4_K, bufs[1].data_ptr(), I, H)
    dd = ops.DeviceWeight(syn.Q4_K, bufs[2].data_ptr(), H, I)
    nbytes = ops.moe_shared_workspace_bytes(T, H, I)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    xd, gd = torch.from_numpy(x).cuda(), torch.from_numpy(gi).cuda()
    out = torch.from_numpy(routed.copy()).cuda()
    ops.moe_shared_expert_device(dg, du, dd, gd.data_ptr(), xd.data_ptr(), T, out.data_ptr(),
                                 ws.data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), host)
    for d in (dg, du, dd):
        d.close()
    for t in (tg, tu, td):
        t.close()


def test_moe_shared_expert_rejects_bad_arguments():
    H, I, T = 512, 256, 2
    gate, up, down, tg, tu, td = _experts(1, H, I, seed=51)
    x = syn.activation(T * H, seed=52).reshape(T, H)
    with pytest.raises(ops.NullPointerError):
        ops.moe_shared_expert(tg, tu, None, x, np.zeros((T, H), np.float32))
    # the output must hold tokens x hidden floats
    lib = ops._native.load()
    err = ops._native.ErrBuf()
    short = np.zeros(T * H - 1, np.float32)
    rc = lib.gollek_hip_moe_shared_expert(tg.handle(), tu.handle(), td.handle(), None,
                                          x.ctypes.data, T, short.ctypes.data, short.size,
                                          err.buf, err.size)
    assert rc == ops._native.ERR_ARG
    # up and gate disagree (gate of 2 experts' rows)
    g2, _, _, tg2, tu2, td2 = _experts(2, H, I, seed=53)
    with pytest.raises(ops.IllegalArgumentError):
        ops.moe_shared_expert(tg2, tu, td, x, np.zeros((T, H), np.float32))
    assert ops.moe_shared_workspace_bytes(-1, H, I) == -1
    for t in (tg, tu, td, tg2, tu2, td2):
        t.close()


# ---- router and routed block -------------------------------------------------

def _same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return np.array_equal(np.isnan(a), np.isnan(b)) and \
        np.array_equal(a[~np.isnan(b)].view(np.uint32), b[~np.isnan(b)].view(np.uint32))


def _router_cases():
    rng = np.random.default_rng(31)
    cases = [("normal", rng.standard_normal((16, 128)).astype(np.float32), 8),
             ("e60", rng.standard_normal((7, 60)).astype(np.float32), 4),
             ("e300", (3 * rng.standard_normal((5, 300))).astype(np.float32), 16),
             ("e4096", rng.standard_normal((2, 4096)).astype(np.float32), 32),
             ("k_past_e", rng.standard_normal((3, 5)).astype(np.float32), 8),
             ("ties", np.round(rng.standard_normal((9, 64)) * 2).astype(np.float32), 8),
             ("wide", (rng.standard_normal((4, 128)) * 40).astype(np.float32), 8),
             ("single", rng.standard_normal((1, 1)).astype(np.float32), 1)]
    sp = rng.standard_normal((6, 32)).astype(np.float32)
    sp[0, 3] = np.nan
    sp[1, 5] = np.inf
    sp[2, :] = -np.inf
    sp[3, 7] = -np.inf
    sp[4, :] = 0.0
    sp[5, ::2] = -0.0
    cases.append(("specials", sp, 4))
    return cases


@pytest.mark.parametrize("scoring", [ops.ROUTER_SOFTMAX, ops.ROUTER_SIGMOID])
def test_router_matches_oracle_bit_for_bit(scoring):
    for name, lg, k in _router_cases():
        print(f"[gpu] router {name} scoring={scoring} shape={lg.shape} k={k}", flush=True)
        ids, w = ops.moe_select_topk(lg, k, scoring)
        rids, rw = o.moe_select_topk(lg, k, scoring == ops.ROUTER_SIGMOID)
        assert np.array_equal(ids, rids), name
        assert _same_bits(w, rw), name
    ids, w = ops.moe_select_topk(np.zeros((0, 8), np.float32), 2, scoring)
    assert ids.shape == (0, 2)


def test_router_rejects_bad_arguments():
    lg = np.zeros((2, 8), np.float32)
    with pytest.raises(ops.IllegalArgumentError):
        ops.moe_select_topk(lg, 2, 7)
    with pytest.raises(ops.IllegalArgumentError):
        ops.moe_select_topk(lg, 0, ops.ROUTER_SOFTMAX)
    with pytest.raises(ops.IllegalArgumentError):
        ops.moe_select_topk(np.zeros((1, 5000), np.float32), 2, ops.ROUTER_SOFTMAX)
    assert ops.router_scoring("qwen3_moe") == ops.ROUTER_SIGMOID
    assert ops.router_scoring("mixtral") == ops.ROUTER_SOFTMAX


@pytest.mark.parametrize("E,H,I,T,k,scoring", [(128, 2048, 768, 16, 8, ops.ROUTER_SIGMOID),
                                               (16, 1024, 512, 9, 4, ops.ROUTER_SOFTMAX)])
def test_moe_block_routes_then_runs_the_grouped_ffn(E, H, I, T, k, scoring):
    print(f"[gpu] moe block E={E} H={H} I={I} T={T} k={k} scoring={scoring}", flush=True)
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=E + 5)
    x = syn.activation(T * H, seed=41).reshape(T, H)
    logits = (2 * np.random.default_rng(42).standard_normal((T, E))).astype(np.float32)
    out = ops.moe_block(tg, tu, td, E, x, logits, k, scoring)
    ids, w = o.moe_select_topk(logits, k, scoring == ops.ROUTER_SIGMOID)
    grouped = ops.moe_grouped(tg, tu, td, E, x, ids, w)
    assert np.array_equal(out.view(np.uint32), grouped.view(np.uint32))
    ref = o.moe_reference_q4k(gate, up, down, E, x, ids, w)
    assert o.rel_err(out, ref) <= MOE_TOL
    for t in (tg, tu, td):
        t.close()


def test_moe_block_device_entry_matches_host():
    import torch
    E, H, I, T, k = 16, 1024, 512, 9, 4
    print("[gpu] moe block device entry", flush=True)
    gate, up, down, tg, tu, td = _experts(E, H, I, seed=77)
    x = syn.activation(T * H, seed=78).reshape(T, H)
    logits = np.random.default_rng(79).standard_normal((T, E)).astype(np.float32)
    host = ops.moe_block(tg, tu, td, E, x, logits, k, ops.ROUTER_SOFTMAX)
    dev = {n: torch.from_numpy(a.reshape(-1)).cuda() for n, a in
           (("g", gate), ("u", up), ("d", down))}
    dw = [ops.DeviceWeight(syn.Q4_K, dev["g"].data_ptr(), E * I, H),
          ops.DeviceWeight(syn.Q4_K, dev["u"].data_ptr(), E * I, H),
          ops.DeviceWeight(syn.Q4_K, dev["d"].data_ptr(), E * H, I)]
    dx = torch.from_numpy(x).cuda()
    dl = torch.from_numpy(logits).cuda()
    ids = torch.zeros((T, k), dtype=torch.int32, device="cuda")
    w = torch.zeros((T, k), dtype=torch.float32, device="cuda")
    out = torch.zeros((T, H), dtype=torch.float32, device="cuda")
    nbytes = ops.moe_workspace_bytes(T, k, H, I, E)
    ws = torch.zeros(nbytes + 256, dtype=torch.uint8, device="cuda")
    base = (ws.data_ptr() + 255) // 256 * 256
    stream = torch.cuda.current_stream().cuda_stream
    ops.moe_block_device(dw[0], dw[1], dw[2], E, dx.data_ptr(), dl.data_ptr(), T, k,
                         ops.ROUTER_SOFTMAX, ids.data_ptr(), w.data_ptr(), out.data_ptr(), base,
                         nbytes, stream)
    torch.cuda.synchronize()
    rids, rw = o.moe_select_topk(logits, k, False)
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert _same_bits(w.cpu().numpy(), rw)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), host.view(np.uint32))
    for d in dw:
        d.close()
    for t in (tg, tu, td):
        t.close()
