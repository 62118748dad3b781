"""CPU tests: the oracle pinned against the reference's golden vectors, its
unit-test known answers, its kernel benchmark checksums, closed forms and
brute force; the libm restatement against the host libm; the product
library's exported C ABI. No GPU is touched here."""
import ctypes as C
import json
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from common import (ROOT, bf16_bits, bf16_input, bf16_values, expert_slot, make_layer,
                    max_rel_err, pyoracle, same_bits)

GOLDEN = os.path.join(ROOT, "tests", "golden", "ref_vectors.npz")
BENCH = os.path.join(ROOT, "tests", "golden", "ref_bench.json")


@pytest.fixture(scope="module")
def orc():
    return pyoracle.Oracle()


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN, allow_pickle=False)


def layer_from_golden(g, tag):
    H, I, E, K, stride, srun = (int(v) for v in g[f"{tag}_meta"])
    L = dict(hidden=H, inter=I, n_experts=E, topk=K, route_scale=1.5, swiglu_limit=10.0,
             expert_stride=stride, scale_run=srun, bias=None, tid2eid=None)
    for k in ("gate_w", "experts", "sh1", "sh1_s", "sh3", "sh3_s", "sh2", "sh2_s"):
        L[k] = np.ascontiguousarray(g[f"{tag}_{k}"])
    if g[f"{tag}_bias"].size:
        L["bias"] = np.ascontiguousarray(g[f"{tag}_bias"])
    if g[f"{tag}_t2e"].size:
        L["tid2eid"] = np.ascontiguousarray(g[f"{tag}_t2e"])
    return L


# ------------------------------------------------------------ golden vectors
def test_golden_decode_tables(orc, gold):
    assert np.array_equal(np.isnan(orc.fp8_table()), np.isnan(gold["fp8_table"]))
    fin = ~np.isnan(gold["fp8_table"])
    assert same_bits(orc.fp8_table()[fin], gold["fp8_table"][fin])
    fin = ~np.isnan(gold["e8m0_table"])
    assert same_bits(orc.e8m0_table()[fin], gold["e8m0_table"][fin])
    assert np.isnan(orc.e8m0_table()[255])


def test_golden_rounding(orc, gold):
    assert same_bits(orc.round_e4m3(gold["round_in"]), gold["round_out"])
    assert np.array_equal(orc.f32_to_bf16(gold["round_in"]), gold["bf16_out"])
    qx, qs = orc.quant_fp8_act(gold["quant_in"])
    assert same_bits(qx, gold["quant_qx"]) and same_bits(qs, gold["quant_qs"])


def test_golden_gemvs(orc, gold):
    g = gold
    IN, R = 256, 48
    assert same_bits(orc.gemv_fp4_q(g["g_qx"], g["g_qs"], g["g_W4"], g["g_S4"], IN, R), g["g_fp4"])
    y0, y1 = orc.gemv_fp4_pair_q(g["g_qx"], g["g_qs"], g["g_W4"], g["g_S4"], g["g_W4b"],
                                 g["g_S4b"], IN, R)
    assert same_bits(y0, g["g_fp4_pair0"]) and same_bits(y1, g["g_fp4_pair1"])
    assert same_bits(orc.gemv_fp8_q(g["g_qx"], g["g_qs"], g["g_W8"], g["g_S8"], IN, R, 1), g["g_fp8"])
    assert same_bits(orc.gemv_fp8_q(g["g_qx"], g["g_qs"], g["g_W8"], g["g_S8"], IN, R, 0),
                     g["g_fp8_raw"])
    y0, y1 = orc.gemv_fp8_pair_q(g["g_qx"], g["g_qs"], g["g_W8"], g["g_S8"], g["g_W8b"],
                                 g["g_S8b"], IN, R)
    assert same_bits(y0, g["g_fp8_pair0"]) and same_bits(y1, g["g_fp8_pair1"])
    assert same_bits(orc.gemv_fp4_batch_q(g["g_bqx"], g["g_bqs"], g["g_W4"], g["g_S4"], IN, R),
                     g["g_fp4_batch"])
    assert same_bits(orc.gemv_fp8_batch_q(g["g_bqx"], g["g_bqs"], g["g_W8"], g["g_S8"], IN, R, 1),
                     g["g_fp8_batch"])
    assert same_bits(orc.gemv_bf16(g["g_bf16_x"], g["g_bf16_W"], IN, R, 0), g["g_bf16"])
    assert same_bits(orc.gemv_fp8_legacy(g["g_bf16_x"], g["g_f8_codes"], g["g_f8_scales"], IN, R),
                     g["g_fp8_legacy"])
    assert same_bits(orc.gemv_fp8_tbl(g["g_bf16_x"], g["g_f8_codes"], g["g_f8_scales"], IN, R),
                     g["g_fp8_tbl"])
    assert same_bits(orc.gemv_fp4_legacy(g["g_qx"], g["g_qs"], g["g_W4"], g["g_fp4_wscale"], IN, R),
                     g["g_fp4_legacy"])


def test_golden_swiglu_router(orc, gold):
    g = gold
    y, qy, qs = orc.swiglu_quant(g["sw_gate"], g["sw_up"], 10, 0.3716)
    assert same_bits(y, g["sw_y"]) and same_bits(qy, g["sw_qy"]) and same_bits(qs, g["sw_qs"])
    assert same_bits(orc.sqrt_softplus(g["ssp_in"]), g["ssp_out"])
    idx, wt = orc.router_public(g["rt_x"], g["rt_G"], g["rt_bias"], None, 0, 256, 16, 6, 0, 1.5)
    assert np.array_equal(idx, g["rt_idx"]) and same_bits(wt, g["rt_wt"])
    idx, wt = orc.router_public(g["rt_x"], g["rt_G"], None, g["rt_t2e"], 2, 256, 16, 6, 1, 1.5)
    assert np.array_equal(idx, g["rt_hidx"]) and same_bits(wt, g["rt_hwt"])


@pytest.mark.parametrize("tag", ["moe", "moeh"])
def test_golden_moe(orc, gold, tag):
    L = layer_from_golden(gold, tag)
    X, tok = gold[f"{tag}_x"], gold[f"{tag}_tok"]
    for t in range(X.shape[0]):
        o, i, w = orc.moe_forward(L, X[t], int(tok[t]))
        assert same_bits(o, gold[f"{tag}_out"][t])
        assert np.array_equal(i, gold[f"{tag}_idx"][t]) and same_bits(w, gold[f"{tag}_wt"][t])
    ob, _, _ = orc.moe_forward_batch(L, X, tok)
    assert same_bits(ob, gold[f"{tag}_batch_out"])
    qx, qs = orc.quant_fp8_act(X[0])
    s, w = expert_slot(L, 3)
    assert same_bits(orc.expert_forward(qx, qs, s, w, 256, 128, 10, 0.41), gold[f"{tag}_exp3"])
    assert same_bits(orc.shared_expert_forward(qx, qs, L, 256, 128, 10), gold[f"{tag}_shared"])


@pytest.mark.parametrize("tag", ["moe", "moeh"])
def test_route_tokens_and_route_outputs_pinned(orc, gold, tag):
    """The many-token router and the pre-BF16 per-route outputs (the checks
    the full-size GPU tests use) against the golden moe_forward: same
    routing; each route rounded to BF16 equals the reference's expert output
    (expert_forward / shared_expert_forward) and their ordered sum is the
    golden layer output."""
    L = layer_from_golden(gold, tag)
    X, tok = gold[f"{tag}_x"], gold[f"{tag}_tok"]
    idx, wt = orc.route_tokens(L, X, tok)
    assert np.array_equal(idx, gold[f"{tag}_idx"]) and same_bits(wt, gold[f"{tag}_wt"])
    H, I = L["hidden"], L["inter"]
    for t in range(X.shape[0]):
        routes, i, w = orc.moe_route_outputs(L, X[t], int(tok[t]))
        assert np.array_equal(i, gold[f"{tag}_idx"][t]) and same_bits(w, gold[f"{tag}_wt"][t])
        qx, qs = orc.quant_fp8_act(X[t])
        for k in range(L["topk"]):
            s, wb = expert_slot(L, i[k])
            assert same_bits(bf16_values(routes[k]),
                             orc.expert_forward(qx, qs, s, wb, H, I, 10, w[k])), (t, k)
        assert same_bits(bf16_values(routes[-1]), orc.shared_expert_forward(qx, qs, L, H, I, 10))
        acc = np.zeros(H, np.float32)
        for k in range(L["topk"] + 1):
            acc = (acc + bf16_values(routes[k])).astype(np.float32)
        assert same_bits(bf16_values(acc), gold[f"{tag}_out"][t])


# ------------------------------------------------ reference unit-test KATs
def test_reference_kats(orc):
    """tests/unit/test_dsv4_ops.c:23-79 known answers."""
    assert orc.f32_to_bf16([1.0])[0] == 0x3F80
    assert orc.f32_to_bf16([1.0 + 2 ** -8])[0] == 0x3F80
    assert orc.f32_to_bf16([1.0 + 2 ** -7])[0] == 0x3F81
    t = orc.fp8_table()
    assert t[0x00] == 0 and t[0x7E] == 448 and t[0xFE] == -448
    assert t[0x3F] == 1.875 and t[0x38] == 1.0 and t[0x01] == 2.0 ** -9 and np.isnan(t[0x7F])
    mid = np.float32(15 / 1024)
    below = np.nextafter(mid, np.float32(0))
    above = np.nextafter(mid, np.float32(1))
    r = orc.round_e4m3(np.array([below, mid, above, -mid], np.float32))
    assert list(r) == [7 / 512, 8 / 512, 8 / 512, -8 / 512]
    e = orc.e8m0_table()
    assert e[127] == 1 and e[126] == 0.5 and e[128] == 2 and np.isnan(e[255])
    x = np.where(np.arange(128) % 2 == 1, 1.0, -1.0).astype(np.float32)
    qx, qs = orc.quant_fp8_act(x)
    assert qs[0] == 2.0 ** -8 and qx[0] == -256 and qx[1] == 256
    big = np.zeros(128, np.float32)
    big[0] = 448 * 1024
    qx, qs = orc.quant_fp8_act(big)
    assert qs[0] == 2.0 ** 10 and qx[0] == 448


def test_fp4_nibble_order(orc):
    """Low nibble is the even column (src/dsv4/dsv4_model.c:1063): a row
    [6, -2, 1, 0.5] packs as bytes 0xC7, 0x12 (the reference's own test of
    this is a placeholder, tests/unit/test_dsv4_ops.c:81-91)."""
    W = np.zeros((1, 16), np.uint8)
    W[0, 0], W[0, 1] = 0xC7, 0x12
    S = np.full((1, 1), 127, np.uint8)
    qx = np.zeros(32, np.float32)
    qs = np.ones(1, np.float32)
    want = [6.0, -2.0, 1.0, 0.5]
    for c in range(4):
        qx[:] = 0
        qx[c] = 1.0
        assert orc.gemv_fp4_q(qx, qs, W, S, 32, 1)[0] == want[c]


# ----------------------------------------------- closed forms, brute force
def test_round_e4m3_is_nearest_grid_value(orc):
    """Every output is the nearest value of the E4M3 grid (ties to the even
    code), checked by brute force over the grid, independent of the oracle's
    frexp arithmetic. The reference's grid includes 480 (the magnitude of the
    NaN code 0x7F); only rounded values >= 512 overflow to 448. Inputs above
    448 never reach it in the activation quantiser (they are clamped first)."""
    t = orc.fp8_table().astype(np.float64)
    codes = np.arange(128)
    grid = t[codes].copy()
    grid[0x7F] = 480.0
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.uniform(-470, 470, 20000), rng.uniform(-0.05, 0.05, 20000),
                        (grid[:, None] + np.array([-1e-7, 0, 1e-7])).ravel(),
                        ((grid[1:] + grid[:-1]) / 2)]).astype(np.float32)
    got = orc.round_e4m3(v).astype(np.float64)
    a = np.abs(v.astype(np.float64))
    d = np.abs(a[:, None] - grid[None, :])
    best = d.min(axis=1)
    ties = np.isclose(d, best[:, None], rtol=0, atol=0)
    pick = np.where(ties.sum(1) > 1, [grid[np.flatnonzero(r)[np.argmin(codes[np.flatnonzero(r)] & 1)]]
                                      for r in ties], grid[d.argmin(1)])
    pick = np.where(pick >= 512, 448, pick)
    assert np.array_equal(np.abs(got), pick)
    assert np.all(np.sign(got[got != 0]) == np.sign(v[got != 0]))


def dequant_fp4_np(orc, W, S, cols):
    f = orc.fp4_table().astype(np.float64)
    v = np.empty((W.shape[0], cols))
    v[:, 0::2] = f[W & 15]
    v[:, 1::2] = f[W >> 4]
    sc = np.ldexp(1.0, S.astype(np.int64) - 127)
    return v * np.repeat(sc, 32, axis=1)[:, :cols]


def test_gemv_against_float64_and_invariants(orc):
    """GEMVs against a float64 product of the dequantised operands (catches a
    dropped term, wrong scale index or transposed operand) and the reference's
    own invariants: pair == two singles, batch == repeated singles."""
    rng = np.random.default_rng(9)
    R, IN = 64, 512
    W = rng.integers(0, 256, (R, IN // 2), dtype=np.uint8)
    S = rng.integers(122, 132, (R, IN // 32), dtype=np.uint8)
    x = rng.standard_normal((3, IN), dtype=np.float32)
    qx, qs = orc.quant_fp8_act(x)
    xd = qx.astype(np.float64) * np.repeat(qs, 128, axis=1)
    ref = dequant_fp4_np(orc, W, S, IN) @ xd[0]
    y = orc.gemv_fp4_q(qx[0], qs[0], W, S, IN, R)
    assert np.max(np.abs(y - ref)) <= 2 ** -8 * np.max(np.abs(ref)) + 1e-6
    yb = orc.gemv_fp4_batch_q(qx, qs, W, S, IN, R)
    for t in range(3):
        assert same_bits(yb[t], orc.gemv_fp4_q(qx[t], qs[t], W, S, IN, R))
    W8 = rng.integers(0, 126, (R, IN), dtype=np.uint8)
    S8 = rng.integers(122, 132, (1, IN // 128), dtype=np.uint8)
    t8 = orc.fp8_table().astype(np.float64)
    d8 = t8[W8] * np.repeat(np.ldexp(1.0, S8.astype(np.int64) - 127), 128, axis=1)
    ref8 = d8 @ xd[1]
    y8 = orc.gemv_fp8_q(qx[1], qs[1], W8, S8, IN, R, 0)
    assert np.max(np.abs(y8 - ref8)) <= 1e-5 * np.max(np.abs(ref8))
    a, b = orc.gemv_fp8_pair_q(qx[1], qs[1], W8, S8, W8[::-1].copy(), S8, IN, R)
    assert same_bits(a, orc.gemv_fp8_q(qx[1], qs[1], W8, S8, IN, R, 1))
    assert same_bits(b, orc.gemv_fp8_q(qx[1], qs[1], W8[::-1].copy(), S8, IN, R, 1))


def test_moe_against_float64(orc):
    """The oracle's MoE composition against an independent float64 evaluation
    of the same math (routing recomputed in float64, experts from dequantised
    weights): pins slot offsets, w1/w2/w3 roles, combine and weights."""
    H, I, E, K = 256, 128, 16, 6
    L = make_layer(orc, H, I, E, K, seed=12, bias=True)
    rng = np.random.default_rng(4)
    x = bf16_input(rng, H)
    out, idx, wt = orc.moe_forward(L, x)
    G = bf16_values(np.zeros(1)) if False else (L["gate_w"].astype(np.uint32) << 16).view(np.float32)
    z = G.astype(np.float64) @ x.astype(np.float64)
    score = np.sqrt(np.log1p(np.exp(z)))
    choice = score + L["bias"]
    sel = np.sort(np.argsort(-choice, kind="stable")[:K])
    assert np.array_equal(sel, idx)
    w64 = score[sel] * 1.5 / score[sel].sum()
    assert np.allclose(wt, w64, rtol=1e-5)
    qx, qs = orc.quant_fp8_act(x)
    xd = qx.astype(np.float64) * np.repeat(qs, 128)
    acc = np.zeros(H)
    t8 = orc.fp8_table().astype(np.float64)
    for k, e in enumerate(sel):
        s, w = expert_slot(L, e)
        g1, g2 = I * (H // 32), H * (I // 32)
        n1, n2 = I * H // 2, H * I // 2
        W1 = dequant_fp4_np(orc, w[:n1].reshape(I, H // 2), s[:g1].reshape(I, H // 32), H)
        W2 = dequant_fp4_np(orc, w[n1:n1 + n2].reshape(H, I // 2), s[g1:g1 + g2].reshape(H, I // 32), I)
        W3 = dequant_fp4_np(orc, w[n1 + n2:].reshape(I, H // 2), s[g1 + g2:].reshape(I, H // 32), H)
        gt, up = W1 @ xd, W3 @ xd
        up = np.clip(up, -10, 10)
        gt = np.minimum(gt, 10)
        acc += W2 @ (gt / (1 + np.exp(-gt)) * up * w64[k])
    def fp8deq(c, s, r, cc):
        return t8[c] * np.kron(np.ldexp(1.0, s.astype(np.int64) - 127), np.ones((128, 128)))[:r, :cc]
    gt = fp8deq(L["sh1"], L["sh1_s"], I, H) @ xd
    up = np.clip(fp8deq(L["sh3"], L["sh3_s"], I, H) @ xd, -10, 10)
    gt = np.minimum(gt, 10)
    acc += fp8deq(L["sh2"], L["sh2_s"], H, I) @ (gt / (1 + np.exp(-gt)) * up)
    # FP8 requant of the intermediates bounds the agreement at a few percent
    assert max_rel_err(out, acc) < 0.08


def test_moe_batch_equals_decode(orc):
    """moe_forward_batch is bit-identical to token-by-token moe_forward
    (tests/unit/test_dsv4_model.c:195-215)."""
    L = make_layer(orc, 256, 128, 16, 6, seed=2, hash_vocab=4)
    rng = np.random.default_rng(5)
    X = bf16_input(rng, (11, 256))
    tok = np.arange(11) % 4
    ob, ib, wb = orc.moe_forward_batch(L, X, tok)
    for t in range(11):
        o, i, w = orc.moe_forward(L, X[t], int(tok[t]))
        assert same_bits(o, ob[t]) and np.array_equal(i, ib[t]) and same_bits(w, wb[t])


# ------------------------------------------- reference benchmark checksums
def xorshift_inputs(orc):
    """benchmarks/bench_dsv4_kernels.c:78-111 input protocol."""
    st = C.c_uint64(0x9E3779B97F4A7C15)
    nxt = orc.lib.orc_xorshift_next
    nxt.argtypes = [C.POINTER(C.c_uint64)]
    nxt.restype = C.c_uint64

    def draw(n):
        return np.array([nxt(C.byref(st)) for _ in range(n)], dtype=np.uint64)
    x2048 = ((draw(4096) % 2001).astype(np.int64) - 1000).astype(np.float32) / np.float32(1000)
    x4096 = ((draw(4096) % 2001).astype(np.int64) - 1000).astype(np.float32) / np.float32(1000)
    w2048 = (draw(2048 * 2048) & 0xFF).astype(np.uint8).reshape(2048, 2048)
    w2048p = (draw(2048 * 2048) & 0xFF).astype(np.uint8).reshape(2048, 2048)
    w4096d = (draw(4096 * 1024) & 0xFF).astype(np.uint8).reshape(4096, 1024)
    w4096f = (draw(4096 * 4096) % 127).astype(np.uint8).reshape(4096, 4096)
    return x2048, x4096, w2048, w2048p, w4096d, w4096f


@pytest.mark.slow
def test_bench_checksums_oracle(orc):
    """The oracle reproduces the reference benchmark's printed checksums at
    full shapes (FP4 2048x4096, 4096x2048; FP8 4096x4096, 2048x4096)."""
    want = json.load(open(BENCH))["checksums"]
    x2048, x4096, w2048, w2048p, w4096d, w4096f = xorshift_inputs(orc)
    s4 = np.full((2048, 128), 127, np.uint8)
    s4d = np.full((4096, 64), 127, np.uint8)
    s8 = np.full((32, 32), 127, np.uint8)
    qa, sa = orc.quant_fp8_act(x2048)
    qb, sb = orc.quant_fp8_act(x4096)
    ck = lambda y: "%.6f" % np.float32(np.sqrt(np.sum(y.astype(np.float64) ** 2)))
    assert ck(orc.gemv_fp4_q(qa, sa, w2048, s4, 4096, 2048)) == want["FP4 2048x4096"][0]
    a, b = orc.gemv_fp4_pair_q(qa, sa, w2048, s4, w2048p, s4, 4096, 2048)
    assert [ck(a), ck(b)] == want["paired FP4 2x(2048x4096)"]
    assert ck(orc.gemv_fp4_q(qb, sb, w4096d, s4d, 2048, 4096)) == want["FP4 4096x2048"][0]
    assert ck(orc.gemv_fp8_q(qb, sb, w4096f, s8, 4096, 4096, 1)) == want["FP8 4096x4096"][0]
    flat = w4096f.ravel()
    a, b = orc.gemv_fp8_pair_q(qa, sa, flat[:2048 * 4096], s8.ravel()[:16 * 32],
                               flat[2048 * 4096:], s8.ravel()[16 * 32:], 4096, 2048)
    assert [ck(a), ck(b)] == want["paired FP8 2x(2048x4096)"]


# ----------------------------------------------------------- live reference
@pytest.mark.skipif(not pyoracle.ref_available(), reason="oracle/_ref not built")
def test_oracle_matches_compiled_reference_full_size(orc):
    ref = pyoracle.RefLib()
    rng = np.random.default_rng(17)
    H, I = 4096, 2048
    L = make_layer(orc, H, I, 3, 2, seed=8)
    x = bf16_input(rng, H)
    qx, qs = orc.quant_fp8_act(x)
    qx2, qs2 = ref.quant_fp8_act(x)
    assert same_bits(qx, qx2) and same_bits(qs, qs2)
    s, w = expert_slot(L, 2)
    assert same_bits(orc.expert_forward(qx, qs, s, w, H, I, 10, 0.3),
                     ref.expert_forward(qx, qs, s, w, H, I, 10, 0.3))
    assert same_bits(orc.shared_expert_forward(qx, qs, L, H, I, 10),
                     ref.shared_expert_forward(qx, qs, L, H, I, 10))
    z = rng.standard_normal(4000, dtype=np.float32) * 8
    assert same_bits(orc.sqrt_softplus(z), ref.sqrt_softplus(z))


@pytest.mark.skipif(not pyoracle.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("vocab,n", [(1003, 1), (1003, 7), (517, 40)])
def test_oracle_gemv_bf16_is_the_reference_head(orc, vocab, n):
    """head_logits (AVX2 8-row blocks plus a scalar tail block) and
    head_logits_batch (tokens in runs of DSV4_MAX_TOPK + 1) of the compiled
    reference equal the oracle's per-row BF16 chain, token by token: the GPU
    head is checked against the latter."""
    ref = pyoracle.RefLib()
    rng = np.random.default_rng(vocab + n)
    hid = 768
    W = bf16_bits(rng.standard_normal((vocab, hid), dtype=np.float32) * 0.02)
    h = rng.standard_normal((n, hid)).astype(np.float32)
    y = ref.head_logits(h, W, 4)
    for t in range(n):
        assert same_bits(y[t], orc.gemv_bf16(h[t], W, hid, vocab, 0)), t


# ---------------------------------------------------------- libm restatement
def test_libm_restatement_matches_host_libm(tmp_path):
    """The GPU's expf/log1pf source (dsv4_libm.h) is bit-identical to the host
    glibc on a stride of all inputs (the exhaustive run, stride 1, also passes:
    2,246,049,794 expf inputs with |x| <= 120 and 2,139,095,041 log1pf inputs
    with x >= 0)."""
    exe = tmp_path / "libm_check"
    src = os.path.join(ROOT, "tests", "libm_check.c")
    inc = os.path.join(ROOT, "deepseek-v4-flash-0731-in-c_amd", "csrc")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-I", inc, "-o", str(exe), src, "-lm"],
                   check=True)
    res = subprocess.run([str(exe), "251"], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout
    for line in res.stdout.splitlines():
        name, n, bad = line.split()
        assert int(n) > 1_000_000 and int(bad) == 0


# --------------------------------------------------------- product library
LIB = os.path.join(ROOT, "deepseek-v4-flash-0731-in-c_amd", "lib", "libdsv4_gpu.so")
HDR = os.path.join(ROOT, "include", "dsv4_gpu.h")


def declared_functions():
    txt = open(HDR).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    names = re.findall(r"\b(dsv4g?_[a-z0-9_]+)\s*\(", txt)
    return sorted(set(n for n in names if not n.startswith("dsv4_bf16_to")))


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = C.CDLL(LIB)
    names = declared_functions()
    assert len(names) > 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_probes_live_in_the_test_library_only():
    """The ISA probes the layout tests use are exported by tests/hip's
    library, not by the product library."""
    from common import PROBE_LIB
    assert not hasattr(C.CDLL(LIB), "dsv4g_probe_mfma")
    assert not hasattr(C.CDLL(LIB), "dsv4g_probe_converts")
    if os.path.exists(PROBE_LIB):
        probe = C.CDLL(PROBE_LIB)
        assert hasattr(probe, "dsv4p_probe_mfma") and hasattr(probe, "dsv4p_probe_converts")


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_library_scalar_entry_points(orc):
    """The drop-in scalar helpers (host-side pure functions)."""
    lib = C.CDLL(LIB)
    lib.dsv4_fp8_e4m3.restype = C.c_float
    lib.dsv4_fp8_e4m3.argtypes = [C.c_uint8]
    lib.dsv4_e8m0.restype = C.c_float
    lib.dsv4_e8m0.argtypes = [C.c_uint8]
    lib.dsv4_round_e4m3.restype = C.c_float
    lib.dsv4_round_e4m3.argtypes = [C.c_float]
    lib.dsv4_f32_to_bf16.restype = C.c_uint16
    lib.dsv4_f32_to_bf16.argtypes = [C.c_float]
    t8, e8 = orc.fp8_table(), orc.e8m0_table()
    for c in range(256):
        a, b = lib.dsv4_fp8_e4m3(c), t8[c]
        assert (np.isnan(a) and np.isnan(b)) or np.float32(a).view(np.uint32) == b.view(np.uint32)
        a, b = lib.dsv4_e8m0(c), e8[c]
        assert (np.isnan(a) and np.isnan(b)) or np.float32(a).view(np.uint32) == b.view(np.uint32)
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.standard_normal(3000) * 200, rng.standard_normal(3000) * 0.01,
                        [470.0, 500.0, 520.0, 15 / 1024]]).astype(np.float32)
    got = np.array([lib.dsv4_round_e4m3(float(a)) for a in v], np.float32)
    assert same_bits(got, orc.round_e4m3(v))
    got = np.array([lib.dsv4_f32_to_bf16(float(a)) for a in v], np.uint16)
    assert np.array_equal(got, orc.f32_to_bf16(v))


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
@pytest.mark.parametrize("fn,kind", [("dsv4_gemv_fp4_batch_q", "FP4"),
                                     ("dsv4_gemv_fp8_batch_q", "FP8"),
                                     ("dsv4_gemv_bf16_batch", "BF16")])
def test_dropin_batch_limit_exits_like_the_reference(fn, kind):
    """The batched drop-ins exit(1) with a message above 33 token vectors, as
    the reference does (src/dsv4/dsv4_model.c:689-693, 1094-1098); the check
    comes before any GPU work, so it runs here in a child process."""
    args = {"dsv4_gemv_fp4_batch_q": "None, None, None, 34, None, None, 4096, 2048",
            "dsv4_gemv_fp8_batch_q": "None, None, None, 34, None, None, 4096, 2048, 1",
            "dsv4_gemv_bf16_batch": "None, None, 34, None, 4096, 256, 0"}[fn]
    code = f"import ctypes as C; C.CDLL({LIB!r}).{fn}({args}); print('returned')"
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 1, (r.returncode, r.stdout, r.stderr)
    assert f"dsv4: {kind} batch 34 exceeds 33" in r.stderr
    assert "returned" not in r.stdout
