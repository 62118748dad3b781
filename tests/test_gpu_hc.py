"""GPU parity of the caller step around the MoE layer: rmsnorm_bf16,
dsv4_hc_split, hc_pre (+ the fused RMSNorm), hc_post and the whole FFN half
of a decoder layer (dsv4g_ffn_step), all bit-exact against the oracle on the
same inputs, including the sums of squares that land exactly on a float
rounding midpoint (settled by the kernels' sequential fallback)."""
from __future__ import annotations

import os
import time

import numpy as np
import pytest

from common import ROOT, bf16_bits, bf16_input, bf16_values, make_layer, pyoracle, same_bits

pytestmark = pytest.mark.gpu

TINY = os.path.join(ROOT, "tests", "golden", "tiny_dsv4")


@pytest.fixture(scope="module")
def env():
    import torch
    import dsv4_gpu
    return dict(torch=torch, lib=dsv4_gpu.lib(), orc=pyoracle.Oracle(),
                dev=torch.device("cuda:0"), dg=dsv4_gpu)


def T(env, a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return env["torch"].from_numpy(a.copy()).to(env["dev"])


def H(t):
    return t.detach().cpu().numpy()


def hc_inputs(rng, mult, hid, fn_sigma=0.01):
    mix_n = (2 + mult) * mult
    state = bf16_values(rng.standard_normal(mult * hid).astype(np.float32))
    fn = (rng.standard_normal((mix_n, mult * hid)) * fn_sigma).astype(np.float32)
    scale3 = (0.5 + rng.random(3)).astype(np.float32)
    base = (rng.standard_normal(mix_n) * 0.5).astype(np.float32)
    return state, fn, scale3, base


def midpoint_vec(n):
    """n = 2^k (k even) values whose sum of squares divided by n is exactly
    1 + 2^-24, a float midpoint."""
    k = int(np.log2(n))
    assert 2 ** k == n and k % 2 == 0
    s = np.zeros(n, np.float32)
    s[: n // 4] = 2.0
    s[n // 4] = np.float32(2.0 ** ((k - 24) // 2))
    return s


def test_rmsnorm_bit_exact(env):
    orc, lib = env["orc"], env["lib"]
    rng = np.random.default_rng(11)
    for n in (4096, 1024, 7168, 8, 4, 5):
        x = (rng.standard_normal((5, n)) * rng.random((5, 1)) * 3).astype(np.float32)
        x[1] = 0.0
        if n in (4096, 1024):
            x[2] = midpoint_vec(n)
        w = bf16_bits((1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32))
        for gain in (w, None):
            for rnd in (0, 1):
                for eps in (1e-6, 0.0):
                    got = H(lib.rmsnorm_bf16(T(env, x), None if gain is None else T(env, gain),
                                             eps, rnd))
                    assert same_bits(got, orc.rmsnorm_bf16(x, gain, eps, rnd)), (n, rnd, eps)
    # in place
    x = bf16_input(rng, (3, 4096))
    w = bf16_bits((1.0 + 0.1 * rng.standard_normal(4096)).astype(np.float32))
    xt = T(env, x)
    lib.rmsnorm_bf16(xt, T(env, w), 1e-6, 1, out=xt)
    assert same_bits(H(xt), orc.rmsnorm_bf16(x, w, 1e-6, 1))


def test_hc_split_bit_exact(env):
    orc, lib = env["orc"], env["lib"]
    rng = np.random.default_rng(12)
    for mult in (1, 2, 3, 4, 7):
        mix_n = (2 + mult) * mult
        for iters in (1, 20):
            mixes = (rng.standard_normal((64, mix_n)) * 3).astype(np.float32)
            sc = (rng.random(3) * 2).astype(np.float32)
            base = rng.standard_normal(mix_n).astype(np.float32)
            pre, post, comb = (H(v) for v in lib.hc_split(T(env, mixes), T(env, sc),
                                                         T(env, base), mult, iters))
            for r in range(64):
                p, q, c = orc.hc_split(mixes[r], sc, base, mult, iters, 1e-6)
                assert same_bits(pre[r], p) and same_bits(post[r], q) and same_bits(comb[r], c), \
                    (mult, iters, r)


@pytest.mark.parametrize("mult,hid,n", [(4, 4096, 3), (4, 256, 2), (2, 8, 2), (1, 64, 1),
                                        (3, 100, 2), (7, 32, 2), (4, 4100, 1)])
def test_hc_pre_bit_exact(env, mult, hid, n):
    orc, lib = env["orc"], env["lib"]
    rng = np.random.default_rng(mult * 100 + hid)
    states, fn, sc, base = [], None, None, None
    for t in range(n):
        st, fn_t, sc_t, base_t = hc_inputs(rng, mult, hid)
        states.append(st)
        if fn is None:
            fn, sc, base = fn_t, sc_t, base_t
    S = np.stack(states)
    norm = bf16_bits((1.0 + 0.1 * rng.standard_normal(hid)).astype(np.float32))
    for w in (None, norm):
        b, p, c = (H(v) for v in lib.hc_pre(T(env, S), T(env, fn), T(env, sc), T(env, base), mult,
                                            None if w is None else T(env, w)))
        for t in range(n):
            ob, op, oc = orc.hc_pre(S[t], fn, sc, base, mult)
            if w is not None:
                ob = orc.rmsnorm_bf16(ob[None], w, 1e-6, 1)[0]
            assert same_bits(p[t], op) and same_bits(c[t], oc), (t, "post/comb")
            assert same_bits(b[t], ob), (t, "bin")


def test_hc_pre_midpoint_sum(env):
    """The state's sum of squares on a float midpoint (ss/n = 1 + 2^-24): the
    scale comes from the sequential fallback. (The RMSNorm's own midpoint
    case is in test_rmsnorm_bit_exact.)"""
    orc, lib = env["orc"], env["lib"]
    mult, hid = 4, 4096
    rng = np.random.default_rng(13)
    _, fn, sc, base = hc_inputs(rng, mult, hid)
    S = midpoint_vec(mult * hid)[None]
    norm = bf16_bits(np.ones(hid, np.float32))
    b, p, c = (H(v) for v in lib.hc_pre(T(env, S), T(env, fn), T(env, sc), T(env, base), mult,
                                        T(env, norm)))
    ob, op, oc = orc.hc_pre(S[0], fn, sc, base, mult)
    assert same_bits(p[0], op) and same_bits(c[0], oc)
    assert same_bits(b[0], orc.rmsnorm_bf16(ob[None], norm, 1e-6, 1)[0])


def test_hc_post_bit_exact(env):
    orc, lib = env["orc"], env["lib"]
    rng = np.random.default_rng(14)
    for mult, hid, n in ((4, 4096, 3), (2, 8, 1), (7, 300, 2)):
        S = bf16_values(rng.standard_normal((n, mult * hid)).astype(np.float32))
        br = bf16_values(rng.standard_normal((n, hid)).astype(np.float32))
        post = (rng.random((n, mult)) * 2).astype(np.float32)
        comb = rng.random((n, mult * mult)).astype(np.float32)
        st = T(env, S)
        lib.hc_post(st, T(env, br), T(env, post), T(env, comb), mult)
        got = H(st)
        for t in range(n):
            assert same_bits(got[t], orc.hc_post(S[t], br[t], post[t], comb[t], mult))


def test_tiny_checkpoint_hc_weights(env):
    """The reference's tiny checkpoint (hidden 8, hc_mult 2): hc_pre with its
    hc_ffn weights and ffn_norm, read through the checkpoint index."""
    orc, lib, dg = env["orc"], env["lib"], env["dg"]
    ck = dg.Checkpoint(TINY)
    rng = np.random.default_rng(15)
    for layer in range(4):
        pre = f"layers.{layer}."
        fn = ck.read_f32(pre + "hc_ffn_fn").reshape(8, 16)
        sc = ck.read_f32(pre + "hc_ffn_scale")
        base = ck.read_f32(pre + "hc_ffn_base")
        norm = np.frombuffer(ck.read(pre + "ffn_norm.weight"), np.uint16).copy()
        S = bf16_values(rng.standard_normal((2, 16)).astype(np.float32))
        b, p, c = (H(v) for v in lib.hc_pre(T(env, S), T(env, fn), T(env, sc), T(env, base), 2,
                                            T(env, norm)))
        for t in range(2):
            ob, op, oc = orc.hc_pre(S[t], fn, sc, base, 2)
            assert same_bits(p[t], op) and same_bits(c[t], oc)
            assert same_bits(b[t], orc.rmsnorm_bf16(ob[None], norm, 1e-6, 1)[0])


def run_ffn_step(env, L, mult, n, seed, token_ids=None, DL=None, workspace=None):
    orc, lib, dg, torch = env["orc"], env["lib"], env["dg"], env["torch"]
    rng = np.random.default_rng(seed)
    hid = L["hidden"]
    S = bf16_values((rng.standard_normal((n, mult * hid)) * 0.5).astype(np.float32))
    _, fn, sc, base = hc_inputs(rng, mult, hid, fn_sigma=0.005)
    norm = bf16_bits((1.0 + 0.1 * rng.standard_normal(hid)).astype(np.float32))
    DL = dg.DeviceLayer.from_host(L, env["dev"]) if DL is None else DL
    st = T(env, S)
    tok = None if token_ids is None else torch.from_numpy(token_ids).to(env["dev"])
    _, idx, wt = lib.ffn_step(st, T(env, fn), T(env, sc), T(env, base), T(env, norm), DL, mult,
                              token_ids=tok, workspace=workspace)
    got, idx, wt = H(st), H(idx), H(wt)
    for t in range(n):
        x, post, comb = orc.hc_pre(S[t], fn, sc, base, mult)
        x = orc.rmsnorm_bf16(x[None], norm, 1e-6, 1)[0]
        out, i, w = orc.moe_forward(L, x, 0 if token_ids is None else int(token_ids[t]))
        want = orc.hc_post(S[t], out, post, comb, mult)
        assert np.array_equal(idx[t], i) and same_bits(wt[t], w), t
        assert same_bits(got[t], want), t
    return st, (fn, sc, base, norm, DL)


def test_ffn_step_bit_exact(env):
    """hc_pre + RMSNorm -> decode MoE -> hc_post on device for 3 tokens of a
    synthetic layer, against the oracle's composition of the same steps."""
    L = make_layer(env["orc"], 256, 128, 16, 6, seed=31, bias=True)
    run_ffn_step(env, L, 4, 3, seed=32)


def test_ffn_step_workspace_reused_across_token_counts(env):
    """One workspace sized for 4 tokens serves steps of 4, 1, 3 and 4 tokens
    in a row, each bit-exact: a step with fewer tokens must not write its
    own buffers over the decode records and flags of the tokens it does not
    use (a later step with more tokens needs them zero)."""
    torch, lib, dg = env["torch"], env["lib"], env["dg"]
    L = make_layer(env["orc"], 256, 128, 16, 6, seed=37, bias=True)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    ws = torch.zeros(lib.ffn_step_workspace_bytes(DL, 4, 4), dtype=torch.uint8,
                     device=env["dev"])
    for i, n in enumerate((4, 1, 3, 4)):
        print(f"ffn_step on a 4-token workspace: {n} tokens", flush=True)
        run_ffn_step(env, L, 4, n, seed=38 + i, DL=DL, workspace=ws)


def test_ffn_step_hash_layer(env):
    L = make_layer(env["orc"], 256, 128, 16, 6, seed=33, hash_vocab=40)
    run_ffn_step(env, L, 4, 2, seed=34, token_ids=np.array([3, 39], np.int32))


def test_ffn_step_full_size(env):
    """hidden 4096 (state 4 x 4096, hc_fn 24 x 16384), inter 2048, 16
    experts, top-6; prints the hc_pre, hc_post and whole-step times."""
    torch, lib = env["torch"], env["lib"]
    L = make_layer(env["orc"], 4096, 2048, 16, 6, seed=35, bias=True)
    st, (fn, sc, base, norm, DL) = run_ffn_step(env, L, 4, 1, seed=36)
    fn_t, sc_t, base_t, norm_t = T(env, fn), T(env, sc), T(env, base), T(env, norm)
    ws = torch.zeros(lib.ffn_step_workspace_bytes(DL, 4, 1), dtype=torch.uint8,
                     device=env["dev"])

    def timed(fn_call, reps=50):
        fn_call()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn_call()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / reps * 1e6

    t_pre = timed(lambda: lib.hc_pre(st, fn_t, sc_t, base_t, 4, norm_t))
    b, p, c = lib.hc_pre(st, fn_t, sc_t, base_t, 4, norm_t)
    t_post = timed(lambda: lib.hc_post(st, b, p, c, 4))
    t_step = timed(lambda: lib.ffn_step(st, fn_t, sc_t, base_t, norm_t, DL, 4, workspace=ws,
                                        check=False))
    lib.check_decode_status(ws)
    print(f"\nhc_pre+norm {t_pre:.1f} us, hc_post {t_post:.1f} us, ffn_step {t_step:.1f} us "
          f"(1 token, host-timed launches)", flush=True)
