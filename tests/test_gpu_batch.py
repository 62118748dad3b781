"""GPU parity of the batched path (speculative verify / prefill grouped GEMM)
against the oracle's moe_forward_batch (bit-identical to the reference's,
tests/test_oracle_cpu.py), plus the MFMA operand layouts the kernels assume.

Bar: top-k indices identical and route weights bit-exact for every token;
expert outputs are exact products summed by the BF16 MFMA in fp32, in another
order than the reference's sequential chain, and every reference expert
output is rounded to BF16 (one ulp = 2^-8 relative), so an fp32 difference of
one ulp can flip one BF16 output element. Per token: norm-wise relative error
||out - ref|| / ||ref|| <= 1e-3, and every element within one BF16 ulp of the
reference element plus 1e-3 * max|ref|. The fraction of bit-exact tokens is
printed."""
import numpy as np
import pytest

from common import bf16_input, make_layer, max_rel_err, probe_lib, pyoracle, same_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    import dsv4_gpu
    return dict(torch=torch, lib=dsv4_gpu.lib(), orc=pyoracle.Oracle(), dg=dsv4_gpu,
                dev=torch.device("cuda:0"))


def T(env, a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return env["torch"].from_numpy(a.copy()).to(env["dev"])


def test_mfma_layouts(env):
    """The kernels' operand and result layouts for the block-scaled FP4/FP8
    MFMA and the BF16 MFMA, against a float64 matmul."""
    orc, probe = env["orc"], probe_lib()
    rng = np.random.default_rng(0)
    t4, t8 = orc.fp4_table().astype(np.float64), orc.fp8_table().astype(np.float64)
    B8 = rng.integers(0, 126, (16, 128), dtype=np.uint8)
    sa = rng.integers(124, 131, (16, 4), dtype=np.uint8)
    sb = rng.integers(124, 131, (16, 4), dtype=np.uint8)
    Bd = t8[B8] * np.repeat(np.ldexp(1.0, sb.astype(int) - 127), 32, axis=1)
    A4 = rng.integers(0, 256, (16, 64), dtype=np.uint8)
    A4d = np.empty((16, 128))
    A4d[:, 0::2], A4d[:, 1::2] = t4[A4 & 15], t4[A4 >> 4]
    A4d *= np.repeat(np.ldexp(1.0, sa.astype(int) - 127), 32, axis=1)
    # the block-scaled MFMA sums each 128-K window with about 12 bits below its
    # largest product (measured: error <= 2^-11 of the largest |a*b|)
    def mx_ok(D, Ad, Bd):
        big = np.max(np.abs(Ad[:, None, :] * Bd[None, :, :]), axis=2)
        return np.all(np.abs(D - Ad @ Bd.T) <= 2.0 ** -10 * big)
    D = probe.mfma(0, T(env, A4), T(env, B8), T(env, sa), T(env, sb)).cpu().numpy()
    assert mx_ok(D, A4d, Bd)
    A8 = rng.integers(0, 126, (16, 128), dtype=np.uint8)
    A8d = t8[A8] * np.repeat(np.ldexp(1.0, sa.astype(int) - 127), 32, axis=1)
    D = probe.mfma(1, T(env, A8), T(env, B8), T(env, sa), T(env, sb)).cpu().numpy()
    assert mx_ok(D, A8d, Bd)
    from common import bf16_bits
    Ab = bf16_bits(rng.standard_normal((16, 32), dtype=np.float32))
    Bb = bf16_bits(rng.standard_normal((16, 32), dtype=np.float32))
    f = lambda u: (u.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    D = probe.mfma(2, T(env, Ab), T(env, Bb)).cpu().numpy()
    assert np.allclose(D, f(Ab) @ f(Bb).T, rtol=1e-5, atol=1e-5)


def zipf_bias(n_experts, seed, s=1.2):
    """Per-expert bias giving Zipf(s)-skewed routing over a seeded permutation
    (with 32 experts, the busiest gets ~85% of tokens, the median ~10%)."""
    rng = np.random.default_rng(seed)
    p = np.arange(1, n_experts + 1, dtype=np.float64) ** -s
    b = np.empty(n_experts)
    b[rng.permutation(n_experts)] = np.log(p / p.sum())
    return (0.2 * (b - b.mean())).astype(np.float32)


def bf16_ulp(v):
    """Spacing of BF16 values at |v| (normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return np.ldexp(1.0, (e - 7).astype(int))


def check_batch(env, L, X, tok, out, idx, wt, sample):
    orc = env["orc"]
    rel, mre, exact = [], [], 0
    for t in sample:
        o, i, w = orc.moe_forward(L, X[t], int(tok[t]))
        assert np.array_equal(idx[t], i), t
        assert same_bits(wt[t], w), t
        d = out[t].astype(np.float64) - o
        r = float(np.linalg.norm(d) / max(np.linalg.norm(o), 1e-30))
        rel.append(r)
        mre.append(max_rel_err(out[t], o))
        exact += int(np.all(d == 0))
        bound = bf16_ulp(o) + 1e-3 * np.max(np.abs(o))
        assert np.all(np.abs(d) <= bound), (t, float(np.max(np.abs(d) / bound)))
    rel = np.array(rel)
    print(f"\n  tokens checked {len(rel)}: bit-exact {exact / len(rel):.3f}, "
          f"max norm-relative error {rel.max():.2e}, max |d|/max|ref| {max(mre):.2e}")
    assert rel.max() <= 1e-3
    return rel


@pytest.mark.parametrize("hash_vocab", [0, 50])
def test_verify_batch_64_tokens(env, hash_vocab):
    orc, lib, dg = env["orc"], env["lib"], env["dg"]
    L = make_layer(orc, 4096, 2048, 32, 6, seed=31, hash_vocab=hash_vocab)
    L["bias"] = zipf_bias(32, 5)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    rng = np.random.default_rng(9)
    X = bf16_input(rng, (64, 4096))
    tok = (np.arange(64) * 7 % 50).astype(np.int32)
    out, idx, wt = lib.moe_forward_batch(DL, T(env, X), T(env, tok))
    out, idx, wt = out.cpu().numpy(), idx.cpu().numpy(), wt.cpu().numpy()
    assert np.all(np.isfinite(out))
    check_batch(env, L, X, tok, out, idx, wt, range(64))


def test_batch_matches_decode_path_routing(env):
    """Batch and decode entries agree on routing for the same tokens."""
    orc, lib, dg = env["orc"], env["lib"], env["dg"]
    L = make_layer(orc, 4096, 256, 64, 6, seed=4, bias=True)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    X = bf16_input(np.random.default_rng(2), (40, 4096))
    _, i1, w1 = lib.moe_forward_batch(DL, T(env, X))
    _, i2, w2 = lib.moe_forward(DL, T(env, X))
    assert np.array_equal(i1.cpu().numpy(), i2.cpu().numpy())
    assert same_bits(w1.cpu().numpy(), w2.cpu().numpy())


def test_prefill_4096_tokens(env):
    """4096 tokens with Zipf(1.2)-skewed routing over 32 experts at the real
    hidden/inter sizes: every token's routing checked, a token sample's outputs
    against the oracle."""
    orc, lib, dg = env["orc"], env["lib"], env["dg"]
    E = 32
    L = make_layer(orc, 4096, 2048, E, 6, seed=41)
    L["bias"] = zipf_bias(E, 8)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    rng = np.random.default_rng(3)
    X = bf16_input(rng, (4096, 4096))
    out, idx, wt = lib.moe_forward_batch(DL, T(env, X))
    out, idx, wt = out.cpu().numpy(), idx.cpu().numpy(), wt.cpu().numpy()
    assert np.all(np.isfinite(out))
    for t in range(0, 4096, 7):
        z = orc.gemv_bf16(X[t], L["gate_w"], 4096, E, 0)
        i, w = orc.route(z, L["bias"], None, 6, 1.5)
        assert np.array_equal(idx[t], i), t
        assert same_bits(wt[t], w), t
    counts = np.bincount(idx.ravel(), minlength=E)
    print("\n  tokens per expert: max", counts.max(), "median", int(np.median(counts)))
    check_batch(env, L, X, np.zeros(4096, np.int32), out, idx, wt,
                list(rng.choice(4096, 24, replace=False)))


def test_batch_graph_replay_matches_eager(env):
    """The batched entry captured into a HIP graph (the shared expert's fork
    onto the library's second stream and the join become graph edges),
    replayed three times with eager calls between the replays: every replay
    gives the eager result bit for bit."""
    import torch
    orc, lib, dg = env["orc"], env["lib"], env["dg"]
    L = make_layer(orc, 4096, 512, 16, 4, seed=12, bias=True)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    X = T(env, bf16_input(np.random.default_rng(5), (40, 4096)))
    ref, ri, rw = lib.moe_forward_batch(DL, X)  # eager: also creates the second stream
    ref, ri, rw = ref.cpu().numpy(), ri.cpu().numpy(), rw.cpu().numpy()
    ws = torch.empty(lib.moe_batch_workspace_bytes(DL, 40), dtype=torch.uint8, device=X.device)
    out = torch.empty_like(X)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lib.moe_forward_batch(DL, X, workspace=ws, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _, gi, gw = lib.moe_forward_batch(DL, X, workspace=ws, out=out)
    for r in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert same_bits(out.cpu().numpy(), ref), r
        assert np.array_equal(gi.cpu().numpy(), ri) and same_bits(gw.cpu().numpy(), rw), r
        e, _, _ = lib.moe_forward_batch(DL, X)  # eager work between the replays
        torch.cuda.synchronize()
        assert same_bits(e.cpu().numpy(), ref), r


@pytest.mark.parametrize("hidden,inter,experts,n", [(1280, 384, 40, 100), (512, 256, 24, 300),
                                                    (2048, 640, 16, 257)])
def test_batch_generic_widths(env, hidden, inter, experts, n):
    """Widths off the model's (the per-window GEMM loops, the unsplit or
    generic router logits), token counts on both sides of the few-token
    router kernels (256) and not a multiple of the 64-token tile: routing
    bit-exact, outputs within the tolerance, every token checked."""
    orc, lib, dg = env["orc"], env["lib"], env["dg"]
    L = make_layer(orc, hidden, inter, experts, 4, seed=hidden + n, bias=True)
    L["bias"] = zipf_bias(experts, 3)
    DL = dg.DeviceLayer.from_host(L, env["dev"])
    X = bf16_input(np.random.default_rng(n), (n, hidden))
    out, idx, wt = lib.moe_forward_batch(DL, T(env, X))
    out, idx, wt = out.cpu().numpy(), idx.cpu().numpy(), wt.cpu().numpy()
    assert np.all(np.isfinite(out))
    check_batch(env, L, X, np.zeros(n, np.int32), out, idx, wt, range(n))
