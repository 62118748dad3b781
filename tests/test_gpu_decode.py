"""GPU parity of the decode path (MI355X): hardware converts, dequant,
activation quant, the exact FP4/FP8 GEMVs, router, SwiGLU requant and the
decode MoE layer, all against the oracle / golden vectors on identical inputs.

Bar: bit-exact (same float32 bits) everywhere, the BF16 GEMV and the public
float-scale GEMVs (one sequential chain per row, as in the reference)
included; the tolerance-mode decode entry is checked against its stated
tolerance."""
import json
import os

import numpy as np
import pytest

from common import (ROOT, bf16_bits, bf16_input, expert_slot, make_layer, probe_lib, pyoracle,
                    same_bits, max_rel_err)

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(ROOT, "tests", "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def env():
    import torch
    import dsv4_gpu
    lib = dsv4_gpu.lib()
    return dict(torch=torch, lib=lib, orc=pyoracle.Oracle(), dev=torch.device("cuda:0"),
                gold=np.load(GOLDEN, allow_pickle=False), dsv4_gpu=dsv4_gpu)


def T(env, a):
    torch = env["torch"]
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a.copy()).to(env["dev"])


def H(t):
    return t.detach().cpu().numpy()


def test_hw_converts_match_reference_decode(env):
    fp4, fp8 = probe_lib().converts(env["dev"])
    fp4, fp8 = H(fp4), H(fp8)
    orc = env["orc"]
    t4 = orc.fp4_table()
    want4 = np.stack([t4[np.arange(256) & 15], t4[np.arange(256) >> 4]], 1).ravel()
    assert same_bits(fp4, want4)
    t8 = orc.fp8_table()
    nan = np.isnan(t8)
    assert np.array_equal(np.isnan(fp8), nan)
    assert same_bits(fp8[~nan], t8[~nan])


def test_dequant_bit_exact(env):
    orc, lib = env["orc"], env["lib"]
    rng = np.random.default_rng(0)
    R, C = 256, 512
    W4 = rng.integers(0, 256, (R, C // 2), dtype=np.uint8)
    S4 = rng.integers(0, 255, (R, C // 32), dtype=np.uint8)
    got = H(lib.dequant_fp4(T(env, W4), T(env, S4), R, C))
    t4 = orc.fp4_table()
    vals = np.empty((R, C), np.float32)
    vals[:, 0::2] = t4[W4 & 15]
    vals[:, 1::2] = t4[W4 >> 4]
    want = vals * np.repeat(orc.e8m0_table()[S4], 32, axis=1)
    assert same_bits(got, want)
    W8 = rng.integers(0, 256, (R, C), dtype=np.uint8)
    S8 = rng.integers(0, 255, (R // 128, C // 128), dtype=np.uint8)
    got = H(lib.dequant_fp8(T(env, W8), T(env, S8), R, C))
    want = orc.fp8_table()[W8] * np.kron(orc.e8m0_table()[S8], np.ones((128, 128), np.float32))
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert same_bits(got[~nan], want[~nan])


def test_quant_fp8_act_golden_and_edges(env):
    orc, lib, g = env["orc"], env["lib"], env["gold"]
    x = g["quant_in"]
    qx, qs = lib.quant_fp8_act(T(env, x))
    assert same_bits(H(qx), g["quant_qx"]) and same_bits(H(qs), g["quant_qs"])
    rng = np.random.default_rng(1)
    X = np.concatenate([rng.standard_normal((7, 4096), dtype=np.float32) * s
                        for s in (1e-6, 1e-3, 1.0, 30.0, 1e4)]).astype(np.float32)
    X[0, :128] = 0.0
    qx, qs = lib.quant_fp8_act(T(env, X))
    wq, ws = orc.quant_fp8_act(X)
    assert same_bits(H(qx), wq) and same_bits(H(qs), ws)


def test_gemvs_golden(env):
    lib, g = env["lib"], env["gold"]
    IN, R = 256, 48
    qx, qs = T(env, g["g_qx"]), T(env, g["g_qs"])
    W4, S4, W4b, S4b = (T(env, g[k]) for k in ("g_W4", "g_S4", "g_W4b", "g_S4b"))
    W8, S8, W8b, S8b = (T(env, g[k]) for k in ("g_W8", "g_S8", "g_W8b", "g_S8b"))
    assert same_bits(H(lib.gemv_fp4_q(qx, qs, W4, S4, IN, R)), g["g_fp4"])
    a, b = lib.gemv_fp4_pair_q(qx, qs, W4, S4, W4b, S4b, IN, R)
    assert same_bits(H(a), g["g_fp4_pair0"]) and same_bits(H(b), g["g_fp4_pair1"])
    assert same_bits(H(lib.gemv_fp8_q(qx, qs, W8, S8, IN, R, 1)), g["g_fp8"])
    assert same_bits(H(lib.gemv_fp8_q(qx, qs, W8, S8, IN, R, 0)), g["g_fp8_raw"])
    a, b = lib.gemv_fp8_pair_q(qx, qs, W8, S8, W8b, S8b, IN, R)
    assert same_bits(H(a), g["g_fp8_pair0"]) and same_bits(H(b), g["g_fp8_pair1"])
    bqx, bqs = T(env, g["g_bqx"]), T(env, g["g_bqs"])
    assert same_bits(H(lib.gemv_fp4_batch_q(bqx, bqs, W4, S4, IN, R)), g["g_fp4_batch"])
    assert same_bits(H(lib.gemv_fp8_batch_q(bqx, bqs, W8, S8, IN, R, 1)), g["g_fp8_batch"])
    # the standalone BF16 and float-scale GEMVs run the reference's sequential
    # column-order chain per row: bit-exact
    y = H(lib.gemv_bf16(T(env, g["g_bf16_x"]), T(env, g["g_bf16_W"]), IN, R, 0))[0]
    assert same_bits(y, g["g_bf16"])
    y = H(lib.gemv_fp8_float(T(env, g["g_bf16_x"]), T(env, g["g_f8_codes"]),
                             T(env, g["g_f8_scales"]), IN, R, 128, 0))
    assert same_bits(y, g["g_fp8_legacy"])
    y = H(lib.gemv_fp8_float(T(env, g["g_bf16_x"]), T(env, g["g_f8_codes"]),
                             T(env, g["g_f8_scales"]), IN, R, 128, 1))
    assert same_bits(y, g["g_fp8_tbl"])
    y = H(lib.gemv_fp4_float(qx, qs, W4, T(env, g["g_fp4_wscale"]), IN, R, 32))
    assert same_bits(y, g["g_fp4_legacy"])


@pytest.mark.parametrize("rows,in_", [(2048, 4096), (4096, 2048), (16, 128), (200, 1024)])
def test_fp4_gemv_full_size_bit_exact(env, rows, in_):
    orc, lib = env["orc"], env["lib"]
    rng = np.random.default_rng(rows + in_)
    W = rng.integers(0, 256, (rows, in_ // 2), dtype=np.uint8)
    S = rng.integers(118, 136, (rows, in_ // 32), dtype=np.uint8)
    S[rows // 2, 1] = 255
    x = bf16_input(rng, (3, in_))
    qx, qs = orc.quant_fp8_act(x)
    gq, gs, gW, gS = T(env, qx), T(env, qs), T(env, W), T(env, S)
    assert same_bits(H(lib.gemv_fp4_q(gq[0], gs[0], gW, gS, in_, rows)),
                     orc.gemv_fp4_q(qx[0], qs[0], W, S, in_, rows))
    assert same_bits(H(lib.gemv_fp4_batch_q(gq, gs, gW, gS, in_, rows)),
                     orc.gemv_fp4_batch_q(qx, qs, W, S, in_, rows))


@pytest.mark.parametrize("rows,in_", [(2048, 4096), (4096, 2048), (4096, 4096), (130, 384)])
def test_fp8_gemv_full_size_bit_exact(env, rows, in_):
    orc, lib = env["orc"], env["lib"]
    rng = np.random.default_rng(rows * 3 + in_)
    W = rng.integers(0, 256, (rows, in_), dtype=np.uint8)
    W[(W & 0x7F) == 0x7F] = 0x33
    S = rng.integers(118, 136, ((rows + 127) // 128, in_ // 128), dtype=np.uint8)
    x = bf16_input(rng, (2, in_))
    qx, qs = orc.quant_fp8_act(x)
    gq, gs, gW, gS = T(env, qx), T(env, qs), T(env, W), T(env, S)
    for ro in (0, 1):
        assert same_bits(H(lib.gemv_fp8_q(gq[0], gs[0], gW, gS, in_, rows, ro)),
                         orc.gemv_fp8_q(qx[0], qs[0], W, S, in_, rows, ro))
    assert same_bits(H(lib.gemv_fp8_batch_q(gq, gs, gW, gS, in_, rows, 1)),
                     orc.gemv_fp8_batch_q(qx, qs, W, S, in_, rows, 1))


@pytest.mark.parametrize("rows,in_", [(256, 4096), (2048, 4096), (37, 200), (37, 4096),
                                     (300, 2048)])
def test_bf16_and_float_gemvs_full_size_bit_exact(env, rows, in_):
    """The standalone BF16 GEMV (batch of 3, with and without BF16 output
    rounding) and the float-scale FP8 / FP4 GEMVs against the oracle's
    sequential chains at the router's and an expert's full shapes."""
    orc, lib = env["orc"], env["lib"]
    rng = np.random.default_rng(rows * 7 + in_)
    Gb = bf16_bits(rng.standard_normal((rows, in_), dtype=np.float32) * 0.02)
    x = bf16_input(rng, (3, in_))
    for ro in (0, 1):
        y = H(lib.gemv_bf16(T(env, x), T(env, Gb), in_, rows, ro))
        for t in range(3):
            assert same_bits(y[t], orc.gemv_bf16(x[t], Gb, in_, rows, ro)), (t, ro)
    codes = rng.integers(0, 256, (rows, in_), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x33
    fsc = (rng.random(((rows + 127) // 128, (in_ + 127) // 128)) * 0.01 + 1e-4).astype(np.float32)
    gx, gc, gs = T(env, x[0]), T(env, codes), T(env, fsc)
    assert same_bits(H(lib.gemv_fp8_float(gx, gc, gs, in_, rows, 128, 0)),
                     orc.gemv_fp8_legacy(x[0], codes, fsc, in_, rows, 128))
    assert same_bits(H(lib.gemv_fp8_float(gx, gc, gs, in_, rows, 128, 1)),
                     orc.gemv_fp8_tbl(x[0], codes, fsc, in_, rows, 128))
    W4 = rng.integers(0, 256, (rows, (in_ + 1) // 2), dtype=np.uint8)
    w4s = (rng.random((rows, (in_ + 31) // 32)) * 0.05 + 1e-3).astype(np.float32)
    qx, qs = orc.quant_fp8_act(x)
    assert same_bits(H(lib.gemv_fp4_float(T(env, qx[0]), T(env, qs[0]), T(env, W4),
                                          T(env, w4s), in_, rows, 32)),
                     orc.gemv_fp4_legacy(qx[0], qs[0], W4, w4s, in_, rows, 32))


def test_reference_bench_checksums_on_gpu(env):
    """The reference benchmark's input protocol at full shapes reproduces its
    printed checksums on the GPU (FP4 2048x4096 / 4096x2048, FP8 4096x4096)."""
    from test_oracle_cpu import xorshift_inputs
    orc, lib = env["orc"], env["lib"]
    want = json.load(open(os.path.join(ROOT, "tests", "golden", "ref_bench.json")))["checksums"]
    x2048, x4096, w2048, w2048p, w4096d, w4096f = xorshift_inputs(orc)
    ck = lambda y: "%.6f" % np.float32(np.sqrt(np.sum(H(y).astype(np.float64) ** 2)))
    qa, sa = lib.quant_fp8_act(T(env, x2048))
    qb, sb = lib.quant_fp8_act(T(env, x4096))
    s4 = T(env, np.full((2048, 128), 127, np.uint8))
    s4d = T(env, np.full((4096, 64), 127, np.uint8))
    s8 = T(env, np.full((32, 32), 127, np.uint8))
    assert ck(lib.gemv_fp4_q(qa, sa, T(env, w2048), s4, 4096, 2048)) == want["FP4 2048x4096"][0]
    a, b = lib.gemv_fp4_pair_q(qa, sa, T(env, w2048), s4, T(env, w2048p), s4, 4096, 2048)
    assert [ck(a), ck(b)] == want["paired FP4 2x(2048x4096)"]
    assert ck(lib.gemv_fp4_q(qb, sb, T(env, w4096d), s4d, 2048, 4096)) == want["FP4 4096x2048"][0]
    assert ck(lib.gemv_fp8_q(qb, sb, T(env, w4096f), s8, 4096, 4096, 1)) == want["FP8 4096x4096"][0]


def test_swiglu_quant_golden(env):
    lib, g = env["lib"], env["gold"]
    gu = T(env, np.concatenate([g["sw_gate"], g["sw_up"]]))
    wt = T(env, np.array([0.3716], np.float32))
    qy, qs = lib.swiglu_quant(gu, 512, 10.0, wt=wt, K=0)
    assert same_bits(H(qy)[0], g["sw_qy"]) and same_bits(H(qs)[0], g["sw_qs"])


def test_router_public_golden(env):
    lib, g = env["lib"], env["gold"]
    idx, wt = lib.router_public(T(env, g["rt_x"]), T(env, g["rt_G"]), T(env, g["rt_bias"]), None,
                                256, 16, 6, 0, 1.5)
    assert np.array_equal(H(idx), g["rt_idx"]) and same_bits(H(wt), g["rt_wt"])
    idx, wt = lib.router_public(T(env, g["rt_x"]), T(env, g["rt_G"]), None,
                                T(env, g["rt_t2e"][2]), 256, 16, 6, 1, 1.5)
    assert np.array_equal(H(idx), g["rt_hidx"]) and same_bits(H(wt), g["rt_hwt"])


@pytest.mark.parametrize("kw", [dict(), dict(bias=True), dict(hash_vocab=9)])
def test_router_exact_many_tokens(env, kw):
    """Top-k indices identical and route weights bit-exact over many tokens at
    the real shape (256 experts x 4096, top-6)."""
    orc, lib, dg = env["orc"], env["lib"], env["dsv4_gpu"]
    L = make_layer(orc, 4096, 128, 256, 6, seed=3, **kw)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    rng = np.random.default_rng(11)
    X = bf16_input(rng, (64, 4096))
    tok = np.arange(64, dtype=np.int32) % 9
    idx, wt = lib.router(DL, T(env, X), T(env, tok))
    idx, wt = H(idx), H(wt)
    for t in range(64):
        z = orc.gemv_bf16(X[t], L["gate_w"], 4096, 256, 0)
        row = L["tid2eid"][tok[t]] if L["tid2eid"] is not None else None
        i, w = orc.route(z, L["bias"], row, 6, 1.5)
        assert np.array_equal(idx[t], i), t
        assert same_bits(wt[t], w), t


@pytest.mark.parametrize("tag", ["moe", "moeh"])
def test_moe_forward_golden(env, tag):
    from test_oracle_cpu import layer_from_golden
    g, lib, dg = env["gold"], env["lib"], env["dsv4_gpu"]
    L = layer_from_golden(g, tag)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    out, idx, wt = lib.moe_forward(DL, T(env, g[f"{tag}_x"]), T(env, g[f"{tag}_tok"]))
    assert np.array_equal(H(idx), g[f"{tag}_idx"])
    assert same_bits(H(wt), g[f"{tag}_wt"])
    assert same_bits(H(out), g[f"{tag}_out"])


def test_moe_forward_full_size_bit_exact(env):
    """One MoE layer at the real shape (hidden 4096, inter 2048, top-6 + shared
    FP8), experts restricted to 16 to keep the oracle quick: outputs, indices
    and weights bit-identical to the oracle for several tokens."""
    orc, lib, dg = env["orc"], env["lib"], env["dsv4_gpu"]
    L = make_layer(orc, 4096, 2048, 16, 6, seed=21, bias=True)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    rng = np.random.default_rng(5)
    X = bf16_input(rng, (3, 4096))
    out, idx, wt = lib.moe_forward(DL, T(env, X))
    out, idx, wt = H(out), H(idx), H(wt)
    for t in range(3):
        o, i, w = orc.moe_forward(L, X[t])
        assert np.array_equal(idx[t], i) and same_bits(wt[t], w)
        assert same_bits(out[t], o), max_rel_err(out[t], o)


@pytest.mark.parametrize("kw", [dict(), dict(bias=True), dict(hash_vocab=11)])
def test_moe_forward_256_experts_bit_exact(env, kw):
    """The decode layer with all 256 experts (hidden 4096, inter 128 to keep
    the oracle quick) for 5 tokens at once: candidates, exact chains, final
    top-k, weights and outputs bit-identical to the oracle."""
    orc, lib, dg = env["orc"], env["lib"], env["dsv4_gpu"]
    L = make_layer(orc, 4096, 128, 256, 6, seed=8, **kw)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    X = bf16_input(np.random.default_rng(13), (5, 4096))
    tok = (np.arange(5, dtype=np.int32) * 3) % 11
    out, idx, wt = lib.moe_forward(DL, T(env, X), T(env, tok))
    out, idx, wt = H(out), H(idx), H(wt)
    for t in range(5):
        o, i, w = orc.moe_forward(L, X[t], int(tok[t]))
        assert np.array_equal(idx[t], i), t
        assert same_bits(wt[t], w), t
        assert same_bits(out[t], o), (t, max_rel_err(out[t], o))


def tie_layer(orc, n_experts, winners, hidden=4096):
    """Identical gate rows except one element, raised by k BF16 ulps (k = 1,
    2, ...) for the experts in `winners`: every expert stays within the
    parallel-sum bound of the k-th best, so all are candidates, and the exact
    logits rank the winners first."""
    L = make_layer(orc, hidden, 128, n_experts, 6, seed=17)
    base = L["gate_w"][0].copy()
    base[7] = 0x3A80  # 2^-10 (BF16 ulp there: 2^-17)
    G = np.tile(base, (n_experts, 1))
    for k, e in enumerate(winners):
        G[e, 7] = base[7] + k + 1
    L["gate_w"] = np.ascontiguousarray(G)
    return L


@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("winners", [[], [26, 27, 28, 29, 30, 31], [2, 20, 5, 30, 17, 9]])
def test_moe_forward_ties_and_overflow_candidates(env, winners, fast):
    """More candidates than gate/up slots (32 experts, 16 slots): with a
    constant gate the lowest ids win; with winners beyond the slots the down
    kernel computes their gate/up itself. Bit-exact either way, in fast mode
    too (more candidates than routes: the exact chains decide)."""
    orc, lib, dg = env["orc"], env["lib"], env["dsv4_gpu"]
    L = tie_layer(orc, 32, winners)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    X = bf16_input(np.random.default_rng(23), (2, 4096))
    X[:, 7] = 1.0
    out, idx, wt = lib.moe_forward(DL, T(env, X), fast=fast)
    out, idx, wt = H(out), H(idx), H(wt)
    for t in range(2):
        o, i, w = orc.moe_forward(L, X[t])
        if winners:
            assert sorted(i) == sorted(winners)  # the construction's premise
        else:
            assert list(i) == [0, 1, 2, 3, 4, 5]
        assert np.array_equal(idx[t], i), t
        assert same_bits(wt[t], w), t
        assert same_bits(out[t], o), (t, max_rel_err(out[t], o))


@pytest.mark.parametrize("winners", [[], [300, 17, 260, 5, 299, 111]])
def test_moe_forward_more_than_256_candidates(env, winners):
    """320 experts all within the bound (constant gate): more than 256
    candidates per token, the long selection path, bit-exact."""
    orc, lib, dg = env["orc"], env["lib"], env["dsv4_gpu"]
    L = tie_layer(orc, 320, winners, hidden=512)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    X = bf16_input(np.random.default_rng(29), (2, 512))
    X[:, 7] = 1.0
    out, idx, wt = lib.moe_forward(DL, T(env, X))
    out, idx, wt = H(out), H(idx), H(wt)
    for t in range(2):
        o, i, w = orc.moe_forward(L, X[t])
        if winners:
            assert sorted(i) == sorted(winners)
        else:
            assert list(i) == [0, 1, 2, 3, 4, 5]
        assert np.array_equal(idx[t], i), t
        assert same_bits(wt[t], w), t
        assert same_bits(out[t], o), (t, max_rel_err(out[t], o))


def test_moe_phases_and_graph_replay_match_fused(env):
    """The three launches in order on one stream, and a captured graph of the
    fused entry replayed several times with eager calls on the same
    workspace between the replays: every result has the fused call's bits,
    which match the oracle."""
    torch, orc, lib, dg = env["torch"], env["orc"], env["lib"], env["dsv4_gpu"]
    L = make_layer(orc, 4096, 128, 64, 6, seed=31, bias=True)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    Xh = bf16_input(np.random.default_rng(37), (3, 4096))
    X = T(env, Xh)
    ref, idx, wt = lib.moe_forward(DL, X)
    torch.cuda.synchronize()
    for t in range(3):
        o, i, w = orc.moe_forward(L, Xh[t])
        assert np.array_equal(H(idx)[t], i) and same_bits(H(wt)[t], w)
        assert same_bits(H(ref)[t], o), t
    ws = lib.new_moe_workspace(DL, 3, env["dev"])
    out = torch.zeros_like(X)
    for ph in range(dg.DECODE_PHASES):
        lib.moe_decode_phase(ph, DL, X, out, ws)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    out2 = torch.zeros_like(X)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lib.moe_forward_into(DL, X, out2, ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lib.moe_forward_into(DL, X, out2, ws)
    for r in range(4):
        out2.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out2, ref), r
        e, _, _ = lib.moe_forward(DL, X, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(e, ref), r
    assert lib.decode_status(ws) == 0


def test_moe_workspace_serves_any_token_count(env):
    """One workspace sized for 4 tokens, used by calls of 4, 1, 3, 2 and 4
    tokens in turn: each token's records and flags sit at the same offsets
    whatever the call's token count, so every call matches the oracle and
    no wait runs out."""
    torch, orc, lib, dg = env["torch"], env["orc"], env["lib"], env["dsv4_gpu"]
    L = make_layer(orc, 4096, 128, 64, 6, seed=41, bias=True)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    Xh = bf16_input(np.random.default_rng(43), (4, 4096))
    refs = [orc.moe_forward(L, Xh[t]) for t in range(4)]
    ws = lib.new_moe_workspace(DL, 4, env["dev"])
    for n in (4, 1, 3, 2, 4):
        out, idx, wt = lib.moe_forward(DL, T(env, Xh[:n]), workspace=ws)
        out, idx, wt = H(out), H(idx), H(wt)
        for t in range(n):
            o, i, w = refs[t]
            assert np.array_equal(idx[t], i) and same_bits(wt[t], w), (n, t)
            assert same_bits(out[t], o), (n, t, max_rel_err(out[t], o))
    assert lib.decode_status(ws) == 0


@pytest.mark.parametrize("hidden,experts", [(384, 24), (1280, 40)])
def test_moe_forward_odd_widths_bit_exact(env, hidden, experts):
    """Hidden sizes whose exact-chain slices are 128 columns (384: three
    slices) or 256 (1280: five), with expert counts that leave a partial
    chain block: outputs, indices and weights bit-identical to the oracle."""
    orc, lib, dg = env["orc"], env["lib"], env["dsv4_gpu"]
    L = make_layer(orc, hidden, 256, experts, 6, seed=41, bias=True)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    X = bf16_input(np.random.default_rng(43), (2, hidden))
    out, idx, wt = lib.moe_forward(DL, T(env, X))
    out, idx, wt = H(out), H(idx), H(wt)
    for t in range(2):
        o, i, w = orc.moe_forward(L, X[t])
        assert np.array_equal(idx[t], i), t
        assert same_bits(wt[t], w), t
        assert same_bits(out[t], o), (t, max_rel_err(out[t], o))


def bf16_ulp(v):
    """Spacing of BF16 values at |v| (normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return np.ldexp(1.0, (e - 7).astype(int))


@pytest.mark.parametrize("shape,kw", [((4096, 128, 256), dict()),
                                      ((4096, 128, 256), dict(bias=True)),
                                      ((4096, 128, 256), dict(hash_vocab=11)),
                                      ((4096, 2048, 16), dict(bias=True))])
def test_moe_forward_fast_tolerance(env, shape, kw):
    """dsv4g_moe_forward_fast: top-k indices identical to the oracle; route
    weights from the parallel logits within 1e-5 relative; outputs within
    1e-3 norm-wise and, elementwise, one BF16 ulp plus 1e-3 of the largest
    element (the rounding of the final BF16 output may flip)."""
    orc, lib, dg = env["orc"], env["lib"], env["dsv4_gpu"]
    hidden, inter, experts = shape
    L = make_layer(orc, hidden, inter, experts, 6, seed=8, **kw)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    X = bf16_input(np.random.default_rng(13), (5, hidden))
    tok = (np.arange(5, dtype=np.int32) * 3) % 11
    out, idx, wt = lib.moe_forward(DL, T(env, X), T(env, tok), fast=True)
    out, idx, wt = H(out), H(idx), H(wt)
    worst = 0.0
    for t in range(5):
        o, i, w = orc.moe_forward(L, X[t], int(tok[t]))
        assert np.array_equal(idx[t], i), t
        assert np.max(np.abs(wt[t] - w) / np.maximum(np.abs(w), 1e-30)) <= 1e-5, t
        d = out[t].astype(np.float64) - o
        r = float(np.linalg.norm(d) / max(np.linalg.norm(o), 1e-30))
        worst = max(worst, r)
        assert r <= 1e-3, (t, r)
        bound = bf16_ulp(o) + 1e-3 * np.max(np.abs(o))
        assert np.all(np.abs(d) <= bound), (t, float(np.max(np.abs(d) / bound)))
    print(f"\n  fast decode: max norm-relative error {worst:.2e}")


@pytest.mark.parametrize("block", [16, 64, 256])
def test_fp8_float_gemv_block_sizes(env, block):
    """dsv4_gemv_fp8 / _tbl with other block sizes than the model's 128: the
    product-chain kernel's rows share one row block for every block size that
    is a multiple of 16; 44 rows leave a partial last workgroup."""
    orc, lib = env["orc"], env["lib"]
    rows, in_ = 44, 1024
    rng = np.random.default_rng(block)
    x = rng.standard_normal(in_).astype(np.float32)
    codes = rng.integers(0, 256, (rows, in_), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x35
    fsc = (rng.random(((rows + block - 1) // block, (in_ + block - 1) // block)) * 0.01
           + 1e-4).astype(np.float32)
    gx, gc, gs = T(env, x), T(env, codes), T(env, fsc)
    assert same_bits(H(lib.gemv_fp8_float(gx, gc, gs, in_, rows, block, 0)),
                     orc.gemv_fp8_legacy(x, codes, fsc, in_, rows, block))
    assert same_bits(H(lib.gemv_fp8_float(gx, gc, gs, in_, rows, block, 1)),
                     orc.gemv_fp8_tbl(x, codes, fsc, in_, rows, block))
