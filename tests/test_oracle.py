"""CPU tests that pin the oracle before it is trusted as the GPU checker.

  * every golden fixture from gollek's own tests (closed forms at 0.0, the
    independent-reference cases at their 1e-3);
  * fp16 decode against numpy's IEEE half decoder, all 65536 codes;
  * 6-bit scale/min unpack against the generator's inverse packer;
  * dequantization bit-exact against an independent numpy restatement;
  * mat-vec against an fp64 dot over the dequantized rows;
  * planted mistakes in a copy of the restatement are caught by the fixtures;
  * Q5_K / Q6_K dots: exact-arithmetic cases (every walker must return the
    fp64 dot of the independently dequantized rows bit for bit) and planted
    mistakes built into copies of the C oracle (GO_PLANT) that they catch.
"""
import math

import numpy as np
import pytest

from oracle import oracle as o
from gollek_amd import synthetic as syn
from tests import npref


def _data(fx):
    return np.frombuffer(bytes.fromhex(fx["data_hex"]), dtype=np.uint8)


def _vec(fx):
    return np.asarray(fx["vector"], dtype=np.float32)[fx["vector_offset"]:]


def test_golden_dequant_bit_exact(golden):
    for fx in golden:
        if not fx["expected_dequant_bits"]:
            continue
        got = o.dequantize(fx["type_id"], _data(fx), fx["cols"])
        exp = np.asarray(fx["expected_dequant_bits"], dtype=np.uint32)
        assert np.array_equal(got.view(np.uint32), exp), fx["name"]


def test_golden_matvec(golden):
    for fx in golden:
        if fx["expected_matvec"] is None:
            continue
        y = o.matvec(fx["type_id"], _data(fx), fx["cols"], _vec(fx), fx["row_count"])
        exp = np.asarray(fx["expected_matvec"], dtype=np.float64)
        # JUnit assertEquals(expected, actual, delta): absolute difference.
        assert np.all(np.abs(y - exp) <= fx["tolerance"]), (fx["name"], y, exp)


def test_golden_single_row_dot_matches_matvec(golden):
    # TST/GgufFx.java:26-35: single-row matVecRows equals dotRow exactly.
    for fx in golden:
        if fx["vector"] is None:
            continue
        data, cols = _data(fx), fx["cols"]
        rb = o.row_bytes(fx["type_id"], cols)
        one = o.matvec(fx["type_id"], data[:rb], cols, _vec(fx), 1)[0]
        assert one == o.dot_row(fx["type_id"], data[:rb], cols, _vec(fx)), fx["name"]


def test_f16_decode_exhaustive():
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = o.f16_to_f32(codes)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # The reference maps every NaN to the canonical quiet NaN.
    assert np.all(got[nan].view(np.uint32) == 0x7FC00000)


def test_k4_scale_min_round_trip():
    g = np.random.default_rng(7)
    for _ in range(200):
        sc = g.integers(0, 64, 8)
        mn = g.integers(0, 64, 8)
        packed = syn.pack_q4k_scales(sc, mn)
        for j in range(8):
            assert o.k4_scale_min(packed, j) == (sc[j], mn[j])


@pytest.mark.parametrize("type_id", [syn.Q8_0, syn.Q4_0, syn.Q4_K, syn.Q5_K, syn.Q6_K])
def test_dequant_matches_numpy_restatement(type_id):
    cols = 512
    data = syn.matrix(type_id, 33, cols, seed=11 + type_id)
    a = o.dequantize(type_id, data, cols)
    b = npref.dequant(type_id, data, cols)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q4k_special_scales_match_numpy_restatement():
    # dmin in {+0, -0, NaN, inf} with random codes: both restatements agree bit
    # for bit, including the zero-min-code and dMin == 0 branches.
    data = syn.q4_k_matrix(8, 256, seed=5).copy()
    specials = [0x0000, 0x8000, 0x7E00, 0x7C00, 0xFC00, 0x0001, 0x3C00, 0x8001]
    for r, h in enumerate(specials):
        data[r, 2], data[r, 3] = h & 0xFF, h >> 8
    data[::2, 4:16] &= np.uint8(0x0F)  # half the rows with many zero min codes
    a = o.dequantize(syn.Q4_K, data, 256)
    b = npref.dequant(syn.Q4_K, data, 256)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("type_id,cols", [(syn.Q8_0, 4096), (syn.Q4_0, 4096), (syn.Q4_K, 4096),
                                          (syn.Q4_K, 768), (syn.Q8_0, 160)])
def test_matvec_against_fp64(type_id, cols):
    rows = 37
    data = syn.matrix(type_id, rows, cols, seed=3)
    x = syn.activation(cols, seed=4)
    ref = o.matvec_fp64(type_id, data, cols, x)
    for threads in (1, 4):
        y = o.matvec(type_id, data, cols, x, threads=threads)
        assert o.rel_err(y, ref) <= 1e-3


def test_parallel_equals_serial():
    # TST/GgufParRowsTest.java:14-30: chunked rows equal the serial walk.
    data = syn.q4_k_matrix(301, 2048, seed=9)
    x = syn.activation(2048, seed=10)
    a = o.matvec(syn.Q4_K, data, 2048, x, threads=1)
    b = o.matvec(syn.Q4_K, data, 2048, x, threads=7)
    assert np.array_equal(a, b)


def test_row_count_prefix_and_zero():
    data = syn.q8_0_matrix(10, 64, seed=1)
    x = syn.activation(64, seed=2)
    full = o.matvec(syn.Q8_0, data, 64, x)
    assert np.array_equal(o.matvec(syn.Q8_0, data, 64, x, row_count=4), full[:4])
    assert o.matvec(syn.Q8_0, data, 64, x, row_count=0).size == 0


# ---- planted mistakes: the fixtures must catch each one -------------------

def _mutant_dequant(kind, type_id, data, cols):
    y = npref.dequant(type_id, data, cols).copy()
    if kind == "q4k_swapped_nibbles" and type_id == syn.Q4_K:
        y = y.reshape(-1, 4, 2, 32)[:, :, ::-1, :].reshape(-1, cols)
    elif kind == "q4k_dropped_min" and type_id == syn.Q4_K:
        d8 = np.asarray(data, np.uint8).reshape(-1, 144).copy()
        d8[:, 2:4] = 0
        y = npref.dequant(type_id, d8.reshape(-1), cols)
    elif kind == "q4_0_no_offset" and type_id == syn.Q4_0:
        y = y + np.float32(8.0)
    elif kind == "q8_sign_flip" and type_id == syn.Q8_0:
        y = -y
    return y


@pytest.mark.parametrize("kind", ["q4k_swapped_nibbles", "q4k_dropped_min", "q4_0_no_offset",
                                  "q8_sign_flip"])
def test_planted_mistakes_fail_the_fixtures(golden, kind):
    caught = False
    for fx in golden:
        if not fx["expected_dequant_bits"]:
            continue
        got = _mutant_dequant(kind, fx["type_id"], _data(fx), fx["cols"])
        exp = np.asarray(fx["expected_dequant_bits"], dtype=np.uint32)
        if not np.array_equal(got.view(np.uint32), exp):
            caught = True
    assert caught, kind


def test_moe_reference_q6_k_down_matches_dense():
    # Q6_K down experts: the packed reference dequantizes them as Q6_K (the
    # dequantization is pinned by the reference's Q6_K fixtures) and equals
    # the dense reference on those rows; read as Q4_K bytes they would not.
    E, H, I, T, k = 3, 256, 512, 2, 2
    gate = syn.q4_k_matrix(E * I, H, 11)
    up = syn.q4_k_matrix(E * I, H, 12)
    down = syn.q6_k_matrix(E * H, I, 13)
    ids, w = syn.moe_routing(T, E, k, 14)
    x = syn.activation(T * H, 15).reshape(T, H)
    packed = o.moe_reference_q4k(gate, up, down, E, x, ids, w, down_type=syn.Q6_K)
    dense = o.moe_reference(o.dequantize(12, gate, H).reshape(E, I, H).astype(np.float64),
                            o.dequantize(12, up, H).reshape(E, I, H).astype(np.float64),
                            o.dequantize(syn.Q6_K, down, I).reshape(E, H, I).astype(np.float64),
                            x, ids, w)
    assert np.allclose(packed, dense, rtol=1e-12, atol=1e-12)


def test_moe_reference_paths_agree_and_properties():
    # The packed-expert reference equals the dense one on the same dequantized
    # weights; the output is linear in the route weights; route order within a
    # token does not change the fp64 result; invalid routes contribute zero.
    E, H, I, T, k = 4, 256, 256, 3, 2
    gate = syn.q4_k_matrix(E * I, H, 1)
    up = syn.q4_k_matrix(E * I, H, 2)
    down = syn.q4_k_matrix(E * H, I, 3)
    ids, w = syn.moe_routing(T, E, k, 4)
    x = syn.activation(T * H, 5).reshape(T, H)
    packed = o.moe_reference_q4k(gate, up, down, E, x, ids, w)
    dense = o.moe_reference(o.dequantize(12, gate, H).reshape(E, I, H).astype(np.float64),
                            o.dequantize(12, up, H).reshape(E, I, H).astype(np.float64),
                            o.dequantize(12, down, I).reshape(E, H, I).astype(np.float64),
                            x, ids, w)
    assert np.allclose(packed, dense, rtol=1e-12, atol=1e-12)
    twice = o.moe_reference_q4k(gate, up, down, E, x, ids, 2 * w)
    assert np.allclose(twice, 2 * packed, rtol=1e-12, atol=1e-12)
    flipped = o.moe_reference_q4k(gate, up, down, E, x, ids[:, ::-1], w[:, ::-1])
    assert np.allclose(flipped, packed, rtol=1e-12, atol=1e-12)
    bad = ids.copy()
    bad[0, 0] = E  # out of range: skipped
    wz = w.copy()
    wz[0, 0] = 0.0
    assert np.allclose(o.moe_reference_q4k(gate, up, down, E, x, bad, w),
                       o.moe_reference_q4k(gate, up, down, E, x, ids, wz), rtol=1e-12, atol=1e-12)


# ---- MoE expert FFN in closed form ------------------------------------------
#
# Experts whose every gate / up / down element is one constant (Q4_K blocks
# with equal codes; a negative d gives a negative constant, a nonzero dmin
# with equal min codes shifts it) and tokens whose x is one constant make
# every dot product a closed form: gate_e . x_t = g_e S_t, up_e . x_t = u_e S_t
# (S_t = sum of x_t), every element of h = silu(g_e S_t) u_e S_t, and every
# output element sum_j w_tj d_e I silu(g_e S_t) u_e S_t.  The constants put
# silu in its curved range with a != b, so a gate <-> up swap, a missing
# silu, a sigmoid in its place and a route weight applied twice each change
# the result far beyond rounding (the planted-mistake check below).

MOE_CF_E, MOE_CF_H, MOE_CF_I = 3, 256, 512
# (d, dmin, scale code, min code, nibble): value d * sc * q - dmin * m
MOE_CF_GATE = [(0.5, 0.25, 2, 4, 3), (-0.25, 0.0, 2, 9, 1), (0.125, 0.0, 2, 0, 1)]   # 2.0, -0.5, 0.25
MOE_CF_UP = [(-0.25, 0.0, 1, 0, 3), (0.25, 0.0, 1, 0, 5), (0.5, 0.5, 1, 1, 2)]       # -0.75, 1.25, 0.5
MOE_CF_DOWN = [(0.125, 0.0, 1, 0, 1), (0.0625, 0.0, 1, 3, 1), (-0.25, 0.125, 1, 2, 1)]  # 0.125, 0.0625, -0.5
MOE_CF_IDS = np.array([[0, 1], [2, 0]], np.int32)
MOE_CF_W = np.array([[0.75, 0.25], [0.625, 0.375]], np.float32)
MOE_CF_XV = (1.0 / 256, -1.0 / 512)  # per-token constant x: S_t = 1.0, -0.5


def _const_q4k(rows, cols, d, dmin, sc, m, q):
    nsb = cols // 256
    blk = np.zeros((rows, nsb, 144), np.uint8)
    dd = syn.f16_bits(np.array([d, dmin], np.float32))
    blk[..., 0], blk[..., 1] = dd[0] & 0xFF, dd[0] >> 8
    blk[..., 2], blk[..., 3] = dd[1] & 0xFF, dd[1] >> 8
    blk[..., 4:16] = syn.pack_q4k_scales(np.full(8, sc), np.full(8, m))
    blk[..., 16:] = q | (q << 4)
    return blk.reshape(rows, nsb * 144)


def moe_closed_form_case():
    E, H, I = MOE_CF_E, MOE_CF_H, MOE_CF_I
    gate = np.concatenate([_const_q4k(I, H, *p) for p in MOE_CF_GATE])
    up = np.concatenate([_const_q4k(I, H, *p) for p in MOE_CF_UP])
    down = np.concatenate([_const_q4k(H, I, *p) for p in MOE_CF_DOWN])
    x = np.stack([np.full(H, v, np.float32) for v in MOE_CF_XV])
    return gate, up, down, x, MOE_CF_IDS, MOE_CF_W


def _value(p):
    d, dmin, sc, m, q = p
    return d * sc * q - (dmin * m if m else 0.0)


def moe_closed_form_expected(act=None, swap=False, weight_power=1):
    act = act or (lambda v: v / (1.0 + math.exp(-v)))
    out = np.zeros((len(MOE_CF_XV), MOE_CF_H))
    for t, xv in enumerate(MOE_CF_XV):
        S = xv * MOE_CF_H
        for j in range(MOE_CF_IDS.shape[1]):
            e, wj = int(MOE_CF_IDS[t, j]), float(MOE_CF_W[t, j])
            a, b = _value(MOE_CF_GATE[e]) * S, _value(MOE_CF_UP[e]) * S
            if swap:
                a, b = b, a
            out[t] += wj ** weight_power * _value(MOE_CF_DOWN[e]) * MOE_CF_I * act(a) * b
    return out


def test_moe_reference_closed_form():
    gate, up, down, x, ids, w = moe_closed_form_case()
    # the constructed blocks dequantize to the intended constants
    for blocks, params, cols in ((gate, MOE_CF_GATE, MOE_CF_H), (up, MOE_CF_UP, MOE_CF_H),
                                 (down, MOE_CF_DOWN, MOE_CF_I)):
        rows = blocks.shape[0] // MOE_CF_E
        for e, p in enumerate(params):
            deq = o.dequantize(12, blocks[e * rows:(e + 1) * rows], cols)
            assert np.all(deq == np.float32(_value(p))), (e, p)
    got = o.moe_reference_q4k(gate, up, down, MOE_CF_E, x, ids, w)
    exp = moe_closed_form_expected()
    assert np.allclose(got, exp, rtol=1e-12, atol=1e-12)
    # Each plausible mistake moves the answer by at least 5 %.
    mutants = {
        "gate/up swapped": moe_closed_form_expected(swap=True),
        "no silu": moe_closed_form_expected(act=lambda v: v),
        "sigmoid for silu": moe_closed_form_expected(act=lambda v: 1.0 / (1.0 + math.exp(-v))),
        "relu for silu": moe_closed_form_expected(act=lambda v: max(v, 0.0)),
        "route weight twice": moe_closed_form_expected(weight_power=2),
    }
    for name, mut in mutants.items():
        assert np.max(np.abs(mut - exp)) > 0.05 * np.max(np.abs(exp)), name


# Shared expert: expert 0 of the closed-form experts (gate 2.0, up -0.75,
# down 0.125) and a constant shared_expert_gate row of 2.0, so s_t = 2 S_t.
SHARED_CF_GATE_INP = 2.0


def shared_closed_form_case():
    H, I = MOE_CF_H, MOE_CF_I
    gate = _const_q4k(I, H, *MOE_CF_GATE[0])
    up = _const_q4k(I, H, *MOE_CF_UP[0])
    down = _const_q4k(H, I, *MOE_CF_DOWN[0])
    x = np.stack([np.full(H, v, np.float32) for v in MOE_CF_XV])
    return gate, up, down, x, np.full(H, SHARED_CF_GATE_INP, np.float32)


def shared_closed_form_expected(out, gated=True, gate_sign=1.0, gate_power=1, swap=False):
    res = np.array(out, np.float64, copy=True)
    for t, xv in enumerate(MOE_CF_XV):
        S = xv * MOE_CF_H
        a, b = _value(MOE_CF_GATE[0]) * S, _value(MOE_CF_UP[0]) * S
        if swap:
            a, b = b, a
        y = _value(MOE_CF_DOWN[0]) * MOE_CF_I * (a / (1.0 + math.exp(-a))) * b
        g = 1.0 / (1.0 + math.exp(-gate_sign * SHARED_CF_GATE_INP * S)) if gated else 1.0
        res[t] += g ** gate_power * y
    return res


def test_moe_shared_expert_reference_closed_form():
    gate, up, down, x, gi = shared_closed_form_case()
    out = moe_closed_form_expected().astype(np.float32)  # the routed output
    got = o.moe_shared_expert_reference(gate, up, down, x, out, gate_inp=gi)
    exp = shared_closed_form_expected(out)
    assert np.allclose(got, exp, rtol=1e-6, atol=1e-9)  # g is a float
    assert np.allclose(o.moe_shared_expert_reference(gate, up, down, x, out),
                       shared_closed_form_expected(out, gated=False), rtol=1e-12, atol=1e-12)
    # Each plausible mistake moves the answer by at least 5 % of the shared
    # expert's contribution.
    scale = np.max(np.abs(exp - out))
    mutants = {
        "gate ignored": shared_closed_form_expected(out, gated=False),
        "sigmoid(+s) for sigmoid(-s)": shared_closed_form_expected(out, gate_sign=-1.0),
        "gate applied twice": shared_closed_form_expected(out, gate_power=2),
        "gate/up swapped": shared_closed_form_expected(out, swap=True),
        "routed output dropped": shared_closed_form_expected(np.zeros_like(out)),
    }
    for name, mut in mutants.items():
        assert np.max(np.abs(mut - exp)) > 0.05 * scale, name


def test_shared_expert_gate_special_values():
    x = np.full(8, 0.25, np.float32)
    assert o.shared_expert_gate(x, None) == np.float32(1.0)
    assert o.shared_expert_gate(x, np.zeros(8, np.float32)) == np.float32(0.5)
    # s = 8 * 0.25 * ln 3 / 2 = ln 3: 1 / (1 + 1/3) = 0.75 (to a float ulp)
    g = o.shared_expert_gate(x, np.full(8, math.log(3.0) / 2, np.float32))
    assert abs(float(g) - 0.75) <= 2 ** -23
    # exp(-s) overflows to inf for s far below zero: the gate is exactly 0
    assert o.shared_expert_gate(x, np.full(8, -1e4, np.float32)) == np.float32(0.0)
    assert o.shared_expert_gate(x, np.full(8, 1e4, np.float32)) == np.float32(1.0)


def _moe_reference_mutant(kind, gate, up, down, E, x, ids, w):
    """moe_reference_q4k with one planted mistake (CPU only)."""
    H = gate.shape[1] // 144 * 256
    I = gate.shape[0] // E
    out = np.zeros((ids.shape[0], H))
    for t in range(ids.shape[0]):
        xt = x[t].astype(np.float64)
        for j in range(ids.shape[1]):
            e, wj = int(ids[t, j]), float(w[t, j])
            g = o.dequantize(12, gate[e * I:(e + 1) * I], H).astype(np.float64)
            u = o.dequantize(12, up[e * I:(e + 1) * I], H).astype(np.float64)
            d = o.dequantize(12, down[e * H:(e + 1) * H], I).astype(np.float64)
            if kind == "swap":
                h = o.silu(u @ xt) * (g @ xt)
            elif kind == "nosilu":
                h = (g @ xt) * (u @ xt)
            else:  # weight applied inside the activation
                h = o.silu(wj * (g @ xt)) * (u @ xt)
                wj = 1.0
            out[t] += wj * (d @ h)
    return out


@pytest.mark.parametrize("kind", ["swap", "nosilu", "weight_inside"])
def test_moe_closed_form_catches_planted_mistakes(kind):
    gate, up, down, x, ids, w = moe_closed_form_case()
    mut = _moe_reference_mutant(kind, gate, up, down, MOE_CF_E, x, ids, w)
    assert not np.allclose(mut, moe_closed_form_expected(), rtol=1e-3, atol=1e-6), kind


# ---- MoE router oracle (MoeForwardPass.java:174-203, 286-306) ----------------

def _sig64(v):
    return 1.0 / (1.0 + np.exp(-np.asarray(v, np.float64)))


@pytest.mark.parametrize("sigmoid", [False, True])
def test_router_uniform_logits_take_the_first_k_with_equal_weights(sigmoid):
    # Equal probabilities: a stable sort keeps index order, and k equal
    # weights renormalise to 1/k (exact for k = 8: 16 x 1/16 and 8 x 0.5).
    lg = np.zeros((3, 16), np.float32)
    ids, w = o.moe_select_topk(lg, 8, sigmoid)
    assert np.array_equal(ids, np.tile(np.arange(8, dtype=np.int32), (3, 1)))
    assert np.array_equal(w, np.full((3, 8), 0.125, np.float32))


@pytest.mark.parametrize("sigmoid", [False, True])
def test_router_distinct_logits_follow_a_descending_sort(sigmoid):
    rng = np.random.default_rng(8)
    T, E, k = 5, 64, 6
    lg = np.stack([rng.permutation(np.linspace(-4, 4, E)) for _ in range(T)]).astype(np.float32)
    ids, w = o.moe_select_topk(lg, k, sigmoid)
    for t in range(T):
        exp_ids = np.argsort(-lg[t].astype(np.float64), kind="stable")[:k]
        assert np.array_equal(ids[t], exp_ids)
        s = _sig64(lg[t, exp_ids]) if sigmoid else np.exp(lg[t, exp_ids].astype(np.float64))
        assert np.allclose(w[t], s / s.sum(), rtol=2e-6, atol=0)
        assert abs(float(w[t].astype(np.float64).sum()) - 1.0) < 2e-6


def test_router_ties_keep_index_order():
    lg = np.array([[1, 3, 3, 2, 3]], np.float32)
    for sigmoid in (False, True):
        ids, w = o.moe_select_topk(lg, 2, sigmoid)
        assert ids.tolist() == [[1, 2]]
        assert w.tolist() == [[0.5, 0.5]]


def test_router_nan_ranks_first_and_skips_renormalisation():
    ids, w = o.moe_select_topk(np.array([[0, 1, np.nan, 2]], np.float32), 2, True)
    assert ids.tolist() == [[2, 3]]
    assert np.isnan(w[0, 0])
    assert abs(float(w[0, 1]) - _sig64(2.0)) <= 1e-7  # the raw sigmoid, not renormalised
    # softmax: a NaN max makes every probability NaN; all tie, index order.
    ids, w = o.moe_select_topk(np.array([[0, 1, np.nan, 2]], np.float32), 3, False)
    assert ids.tolist() == [[0, 1, 2]] and np.all(np.isnan(w))
    # +inf logit: inf - inf = NaN at that expert, exp(-inf) = 0 elsewhere, sum NaN.
    ids, w = o.moe_select_topk(np.array([[0, np.inf, 1]], np.float32), 2, False)
    assert ids.tolist() == [[0, 1]] and np.all(np.isnan(w))


def test_router_pads_past_the_expert_count_and_keeps_zero_sums():
    ids, w = o.moe_select_topk(np.array([[0.0, 2.0, 1.0]], np.float32), 5, False)
    assert ids.tolist() == [[1, 2, 0, 0, 0]]
    assert w[0, 3] == 0 and w[0, 4] == 0
    assert abs(float(w[0, :3].astype(np.float64).sum()) - 1.0) < 2e-7
    assert w[0, 0] > w[0, 1] > w[0, 2] > 0
    ids, w = o.moe_select_topk(np.full((1, 4), -np.inf, np.float32), 2, True)
    assert ids.tolist() == [[0, 1]] and w.tolist() == [[0.0, 0.0]]


# ---- Q5_K / Q6_K dots ------------------------------------------------------
#
# Blocks whose scales are powers of two times small integers and x values
# that are multiples of 1/4 in [-1, 1] make every product and every partial
# sum of the Java loops exactly representable in fp32 (below 2^24 units of
# the smallest step), so each walker -- the single-row dot, the no-min
# unrolled dot, the inline-min direct rows (2..4) and the group-sum rows --
# must equal the fp64 dot over tests/npref.py's dequantized rows exactly,
# whatever its summation order.  That pins which code, which high-bit plane,
# which scale, min and x sum each element pairs with.

def _exact_q5_k(rows, cols, seed, mins=True):
    g = np.random.default_rng(seed)
    ns = cols // 256
    out = np.zeros((rows, ns, 176), np.uint8)
    out[..., 0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    out[..., 2:4] = np.frombuffer(np.float16(0.125 if mins else 0.0).tobytes(), np.uint8)
    out[..., 4:16] = syn.pack_q4k_scales(g.integers(0, 8, (rows, ns, 8)), g.integers(0, 8, (rows, ns, 8)))
    out[..., 16:] = g.integers(0, 256, (rows, ns, 160), dtype=np.uint8)
    return out.reshape(rows, ns * 176)


def _exact_q6_k(rows, cols, seed):
    g = np.random.default_rng(seed)
    ns = cols // 256
    out = np.zeros((rows, ns, 210), np.uint8)
    out[..., :192] = g.integers(0, 256, (rows, ns, 192), dtype=np.uint8)
    out[..., 192:208] = g.integers(-8, 8, (rows, ns, 16)).astype(np.int8).view(np.uint8)
    out[..., 208:210] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
    return out.reshape(rows, ns * 210)


def _exact_x(cols, seed):
    return (np.random.default_rng(seed).integers(-4, 5, cols) / 4.0).astype(np.float32)


EXACT_CASES = [("q5_k_mins", syn.Q5_K, True), ("q5_k_nomins", syn.Q5_K, False), ("q6_k", syn.Q6_K, None)]


def _exact_case(type_id, mins, rows, cols, seed):
    data = _exact_q5_k(rows, cols, seed, mins) if type_id == syn.Q5_K else _exact_q6_k(rows, cols, seed)
    return data, _exact_x(cols, seed + 1)


def _exact_mismatches(type_id, data, cols, x, lib=None):
    """Rows (over every walker) where the oracle differs from the exact dot."""
    exact = npref.dequant(type_id, data, cols).astype(np.float64) @ x.astype(np.float64)
    rows = exact.size
    bad = []
    rb = o.row_bytes(type_id, cols)
    flat = np.ascontiguousarray(data).reshape(-1)
    for r in range(rows):  # single-row dots
        if o.dot_row(type_id, flat[r * rb:(r + 1) * rb], cols, x, _lib=lib) != exact[r]:
            bad.append(("dot", r))
    for n in (2, 4, rows):  # direct rows, group-sum / no-min rows
        y = o.matvec(type_id, data, cols, x, row_count=n, threads=1, _lib=lib)
        bad += [("rows%d" % n, r) for r in np.nonzero(y != exact[:n])[0]]
    return bad


@pytest.mark.parametrize("name,type_id,mins", EXACT_CASES, ids=[c[0] for c in EXACT_CASES])
@pytest.mark.parametrize("cols", [256, 1280, 2048])
def test_k56_dots_exact_cases(name, type_id, mins, cols):
    data, x = _exact_case(type_id, mins, 9, cols, cols + type_id)
    if type_id == syn.Q5_K:
        assert o.k_rows_have_mins(type_id, data, cols, 9) == mins
    assert _exact_mismatches(type_id, data, cols, x) == []


@pytest.mark.parametrize("type_id", [syn.Q5_K, syn.Q6_K])
@pytest.mark.parametrize("cols", [256, 768, 4096])
def test_k56_walkers_agree_with_fp64(type_id, cols):
    # Random fp16 scales and Gaussian x: every walker within rounding of the
    # fp64 dot over the bit-exact dequantized rows, and threads do not change
    # the bits.  1e-4: the Q6_K group-sum rows subtract 32 x the x sums from
    # raw-code dots, which cancels about two decimal digits on these rows.
    rows = 23
    data = syn.matrix(type_id, rows, cols, seed=cols + 3 * type_id)
    x = syn.activation(cols, seed=cols + 1)
    ref = o.matvec_fp64(type_id, data, cols, x)
    y = o.matvec(type_id, data, cols, x, threads=1)
    assert o.rel_err(y, ref) <= 1e-4
    assert np.array_equal(y, o.matvec(type_id, data, cols, x, threads=5))
    for n in (1, 2, 4):
        assert o.rel_err(o.matvec(type_id, data, cols, x, row_count=n), ref[:n]) <= 1e-4


def test_group_sums16_exact():
    x = _exact_x(512, 3)
    assert np.array_equal(o.group_sums16(x), x.reshape(-1, 16).astype(np.float64).sum(1))


PLANTS = {1: EXACT_CASES[0], 2: EXACT_CASES[2], 3: EXACT_CASES[2], 4: EXACT_CASES[2], 5: EXACT_CASES[0]}


@pytest.mark.parametrize("plant", sorted(PLANTS))
def test_k56_exact_cases_catch_planted_mistakes(plant, tmp_path):
    # A copy of the oracle with one planted mistake (gguf_oracle.c GO_PLANT)
    # fails the exact-arithmetic check on the walkers the mistake touches.
    lib = o.load(o.build_planted(plant, tmp_path))
    _, type_id, mins = PLANTS[plant]
    data, x = _exact_case(type_id, mins, 9, 1280, 77)
    assert _exact_mismatches(type_id, data, cols=1280, x=x) == []
    bad = _exact_mismatches(type_id, data, 1280, x, lib=lib)
    assert bad, plant
    walkers = {w for w, _ in bad}
    if plant == 4:  # only the group-sum rows subtract the per-16 x sums
        assert walkers == {"rows9"}, walkers
