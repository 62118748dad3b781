"""GPU parity of the streaming row-chain GEMVs and what uses them, against
the oracle on identical inputs, bit for bit:

* the vocabulary head, the reference's per-row fmaf chain
  (head_logits_block, src/dsv4/dsv4_model.c:7221-7255), at its full shape
  (129280 x 4096 BF16, about 1 GiB) for one token and for 3- and 64-token
  verify batches (head_logits_block_batch, :7257-7308), then the greedy token
  of every row (src/cli/dsv4_run.c:357-359, NaN and tie edges included);
* dsv4_gemv_bf16_batch at the batch sizes of each kernel instance;
* dsv4_gemv_fp8 / _tbl at the FP8 matvec benchmark's shape (2048 x 4096,
  fp32 absmax block scales, fp32 x);
* expert_forward (src/dsv4/dsv4_model.c:6289-6345) at the model's expert
  shape, with and without a route weight."""
import numpy as np
import pytest

from common import bf16_bits, bf16_input, expert_slot, make_layer, pyoracle, same_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    import dsv4_gpu
    return dict(torch=torch, lib=dsv4_gpu.lib(), orc=pyoracle.Oracle(),
                dev=torch.device("cuda:0"))


def T(env, a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return env["torch"].from_numpy(a.copy()).to(env["dev"])


def H(t):
    return t.detach().cpu().numpy()


def cli_greedy(row):
    """src/cli/dsv4_run.c:357-359 restated: best = 0; v wins if strictly
    greater."""
    best = 0
    for v in range(1, row.shape[0]):
        if row[v] > row[best]:
            best = v
    return best


def cli_greedy_fast(row):
    """The same rule vectorised: 0 when row[0] is NaN, else the first index of
    the largest non-NaN value (pinned against cli_greedy below)."""
    if np.isnan(row[0]):
        return 0
    m = np.nanmax(row)
    return int(np.flatnonzero(row == m)[0])


def test_vocab_head_full_size_and_greedy(env):
    orc, lib, torch = env["orc"], env["lib"], env["torch"]
    vocab, hid = 129280, 4096
    rng = np.random.default_rng(2)
    W = bf16_bits(rng.standard_normal((vocab, hid), dtype=np.float32) * 0.02)
    h = bf16_input(rng, (3, hid))
    Wd, hd = T(env, W), T(env, h)
    one = H(lib.gemv_bf16(hd[0:1], Wd, hid, vocab, 0))[0]
    assert same_bits(one, orc.gemv_bf16(h[0], W, hid, vocab, 0))
    three = H(lib.gemv_bf16(hd, Wd, hid, vocab, 0))
    for t in range(3):
        assert same_bits(three[t], orc.gemv_bf16(h[t], W, hid, vocab, 0)), t
    idx = H(lib.argmax(torch.from_numpy(three).to(env["dev"])))
    for t in range(3):
        assert idx[t] == cli_greedy_fast(three[t]), t
    # 64 tokens (a verify batch; the batched row chains): every token equal to
    # its own one-token head, three of them to the oracle
    h64 = bf16_input(rng, (64, hid))
    h64d = T(env, h64)
    b64 = H(lib.gemv_bf16(h64d, Wd, hid, vocab, 0))
    for t in range(64):
        assert same_bits(b64[t], H(lib.gemv_bf16(h64d[t:t + 1], Wd, hid, vocab, 0))[0]), t
    for t in (0, 37, 63):
        assert same_bits(b64[t], orc.gemv_bf16(h64[t], W, hid, vocab, 0)), t
    del Wd


def test_greedy_edges(env):
    lib, torch = env["lib"], env["torch"]
    rng = np.random.default_rng(4)
    rows = [rng.standard_normal(1000).astype(np.float32) for _ in range(6)]
    rows[1][[17, 500, 999]] = 9.0                 # ties: the first wins
    rows[2][0] = np.nan                           # logits[0] NaN: 0
    rows[3][[3, 40]] = np.nan
    rows[3][41] = 50.0                            # NaNs never taken
    rows[4][:] = -np.inf
    rows[4][700] = -1e30                          # all -inf but one
    rows[5][:] = 0.0
    rows[5][::2] = -0.0                           # signed zeros compare equal
    L = np.stack(rows)
    for r in L:
        assert cli_greedy(r) == cli_greedy_fast(r)
    got = H(lib.argmax(torch.from_numpy(L).to(env["dev"])))
    assert [int(g) for g in got] == [cli_greedy(r) for r in L]


@pytest.mark.parametrize("rows,in_,batch", [(300, 1024, 5), (300, 1024, 9), (1000, 256, 33),
                                            (64, 4096, 2), (200, 4096, 5), (130, 4096, 71),
                                            (64, 2048, 40), (100, 1024, 20), (77, 4096, 3),
                                            (300, 1000, 3), (50, 2056, 9)])
def test_bf16_batch_instances(env, rows, in_, batch):
    """Every kernel form: for in a multiple of 64, the register-blocked chains
    in runs of 64/32/16/8/4 tokens and the tiled chains for a remainder of 1
    to 3 (5 = 4 + 1, 71 = 64 + 4 + 3, 40 = 32 + 8, ragged last row tiles);
    for other in, the x-in-LDS row chains (x up to 64 KB) and the
    one-row-per-(row, token) fallback."""
    orc, lib = env["orc"], env["lib"]
    rng = np.random.default_rng(rows + batch)
    W = bf16_bits(rng.standard_normal((rows, in_), dtype=np.float32) * 0.05)
    x = rng.standard_normal((batch, in_)).astype(np.float32)
    for ro in (0, 1):
        y = H(lib.gemv_bf16(T(env, x), T(env, W), in_, rows, ro))
        for t in range(batch):
            assert same_bits(y[t], orc.gemv_bf16(x[t], W, in_, rows, ro)), (t, ro)


def test_fp8_matvec_benchmark_shape(env):
    """W N(0, 0.02) quantised per 128x128 block with fp32 absmax/448 scales,
    x fp32 N(0, 1): both float-scale chains, every row."""
    orc, lib = env["orc"], env["lib"]
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((2048, 4096)) * 0.02).astype(np.float32)
    codes, scales = orc.quant_fp8_blocks_absmax(w)
    x = rng.standard_normal(4096).astype(np.float32)
    gx, gc, gs = T(env, x), T(env, codes), T(env, scales)
    assert same_bits(H(lib.gemv_fp8_float(gx, gc, gs, 4096, 2048, 128, 0)),
                     orc.gemv_fp8_legacy(x, codes, scales, 4096, 2048, 128))
    assert same_bits(H(lib.gemv_fp8_float(gx, gc, gs, 4096, 2048, 128, 1)),
                     orc.gemv_fp8_tbl(x, codes, scales, 4096, 2048, 128))


def test_expert_forward_full_size(env):
    orc, lib, torch = env["orc"], env["lib"], env["torch"]
    L = make_layer(orc, 4096, 2048, 2, 1, seed=12)
    scales, weights = expert_slot(L, 1)
    slot = np.concatenate([scales, weights])
    rng = np.random.default_rng(3)
    x = bf16_input(rng, (1, 4096))
    qx, qs = orc.quant_fp8_act(x)
    gslot = T(env, slot)
    gqx, gqs = T(env, qx[0]), T(env, qs[0])
    for w in (None, 0.3712):
        out = torch.empty(4096, dtype=torch.float32, device=env["dev"])
        gw = None if w is None else torch.tensor([w], dtype=torch.float32, device=env["dev"])
        lib.expert_forward(out, gqx, gqs, gslot, L["scale_run"], 4096, 2048, 10.0, gw)
        ref = orc.expert_forward(qx[0], qs[0], scales, weights, 4096, 2048, 10,
                                 1.0 if w is None else w)
        assert same_bits(H(out), ref), w


@pytest.mark.parametrize("hidden,inter", [(256, 128), (1024, 384), (2048, 4096)])
def test_expert_forward_shapes(env, hidden, inter):
    """The two-launch expert_forward (gate/up with the SwiGLU epilogue, then the
    down rows with the requant folded in) at other shapes: an inter that is not
    a multiple of 512 and the widest inter the fused path takes."""
    orc, lib, torch = env["orc"], env["lib"], env["torch"]
    L = make_layer(orc, hidden, inter, 2, 1, seed=hidden + inter)
    scales, weights = expert_slot(L, 0)
    slot = np.concatenate([scales, weights])
    rng = np.random.default_rng(inter)
    x = bf16_input(rng, (1, hidden))
    qx, qs = orc.quant_fp8_act(x)
    out = torch.empty(hidden, dtype=torch.float32, device=env["dev"])
    gw = torch.tensor([0.618], dtype=torch.float32, device=env["dev"])
    lib.expert_forward(out, T(env, qx[0]), T(env, qs[0]), T(env, slot), L["scale_run"], hidden,
                       inter, 10.0, gw)
    ref = orc.expert_forward(qx[0], qs[0], scales, weights, hidden, inter, 10, 0.618)
    assert same_bits(H(out), ref)
