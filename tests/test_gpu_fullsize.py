"""GPU parity at the configurations the benchmark times: one MoE layer of 256
FP4 experts (hidden 4096, inter 2048, top-6) + the FP8 shared expert, built
on the device by the library's quantisers and copied to the host once for the
oracle.

* Decode (dsv4g_moe_forward, one token per call and several per call):
  outputs, indices and weights bit-identical to the oracle's moe_forward.
  The tolerance mode (dsv4g_moe_forward_fast): indices identical, outputs
  within 1e-3 norm-wise and one BF16 ulp + 1e-3 max|ref| elementwise.
* Speculative verify, 64 tokens, and prefill, 4096 tokens, with the Zipf(1.2)
  router bias of the benchmark (dsv4g_moe_forward_batch): routing
  bit-identical for every token; outputs within the batched tolerance
  (every token at 64, a sample at 4096); and each route's expert output
  before its BF16 rounding (dsv4g_moe_forward_batch_routes) within
  max|d| / max|ref| <= 1e-3 of the oracle's fp32 accumulators (the north
  star's "max relative error 1e-3, fp32 accumulate").
* 512 experts: the wider candidate kernels (8 experts per lane) in decode
  and in the batched router on both sides of 256 tokens."""
import numpy as np
import pytest

from common import bf16_ulp, bf16_values, max_rel_err, pyoracle, same_bits, zipf_bias

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    import dsv4_gpu
    import synth
    return dict(torch=torch, lib=dsv4_gpu.lib(), orc=pyoracle.Oracle(), synth=synth,
                dev=torch.device("cuda:0"))


@pytest.fixture(scope="module")
def full_layer(env):
    """The benchmark's layer 0 (seed 100) on the device and on the host."""
    DL = env["synth"].device_layer(seed=100, device=env["dev"])
    env["torch"].cuda.synchronize()
    return DL, env["synth"].host_copy(DL)


def with_zipf(env, DL, L, n_experts):
    b = zipf_bias(n_experts)
    return DL.with_bias(env["torch"].from_numpy(b).to(env["dev"])), dict(L, bias=b)


def H(t):
    return t.detach().cpu().numpy()


def check_tolerance(orc, L, X, out, sample, tok=None):
    """Batched-path tolerance against the oracle for the tokens in sample.
    The reference rounds every route's expert output to BF16 and sums them in
    fp32 (src/dsv4/dsv4_model.c:6795-6805); an fp32 accumulation difference
    far below a BF16 ulp can flip each route's rounding by one ulp of that
    route, so elementwise |d| <= ulp(out) + sum_k ulp(route_k) (with
    cancellation a route's ulp exceeds the output's); norm-wise <= 1e-3."""
    worst, exact = 0.0, 0
    for t in sample:
        routes, _, _ = orc.moe_route_outputs(L, X[t], 0 if tok is None else int(tok[t]))
        rb = bf16_values(routes)
        acc = np.zeros(rb.shape[1], np.float32)
        for k in range(rb.shape[0]):
            acc = (acc + rb[k]).astype(np.float32)
        o = bf16_values(acc)
        d = out[t].astype(np.float64) - o
        r = float(np.linalg.norm(d) / max(np.linalg.norm(o), 1e-30))
        assert r <= 1e-3, (t, r)
        bound = bf16_ulp(o) + np.sum(bf16_ulp(rb), axis=0)
        assert np.all(np.abs(d) <= bound), (t, float(np.max(np.abs(d) / bound)))
        worst = max(worst, r)
        exact += int(np.all(d == 0))
    return worst, exact


def check_route_outputs(orc, L, X, ro32, idx, sample):
    """Each route's fp32 expert output (before BF16) within 1e-3 of the
    oracle's accumulators, max|d| / max|ref| per route."""
    worst = 0.0
    for t in sample:
        ref, i, _ = orc.moe_route_outputs(L, X[t])
        assert np.array_equal(i, idx[t]), t
        errs = [max_rel_err(ro32[t, k], ref[k]) for k in range(ref.shape[0])]
        if max(errs) > 1e-5:
            print(f"\n  sample {t}: per-route max|d|/max|ref| " +
                  " ".join(f"{e:.1e}" for e in errs))
        assert max(errs) <= 1e-3, (t, errs)
        worst = max(worst, max(errs))
    return worst


def test_decode_full_size_bit_exact(env, full_layer):
    """Config 3 at its real size: one token per call over several tokens, then
    four tokens in one call, with and without the Zipf bias."""
    orc, lib, synth = env["orc"], env["lib"], env["synth"]
    DL, L = full_layer
    X = synth.bf16_tokens(10, 4096, seed=7, device=env["dev"])
    Xh = H(X)
    for DLb, Lb in ((DL, L), with_zipf(env, DL, L, 256)):
        for t in range(6):
            out, idx, wt = lib.moe_forward(DLb, X[t:t + 1])
            o, i, w = orc.moe_forward(Lb, Xh[t])
            assert np.array_equal(H(idx)[0], i), t
            assert same_bits(H(wt)[0], w), t
            assert same_bits(H(out)[0], o), (t, max_rel_err(H(out)[0], o))
        out, idx, wt = lib.moe_forward(DLb, X[6:10])
        out, idx, wt = H(out), H(idx), H(wt)
        for t in range(4):
            o, i, w = orc.moe_forward(Lb, Xh[6 + t])
            assert np.array_equal(idx[t], i) and same_bits(wt[t], w), t
            assert same_bits(out[t], o), t


def test_decode_full_size_fast_tolerance(env, full_layer):
    orc, lib, synth = env["orc"], env["lib"], env["synth"]
    DL, L = full_layer
    X = synth.bf16_tokens(8, 4096, seed=9, device=env["dev"])
    Xh = H(X)
    worst = 0.0
    for t in range(8):
        out, idx, wt = lib.moe_forward(DL, X[t:t + 1], fast=True)
        o, i, w = orc.moe_forward(L, Xh[t])
        assert np.array_equal(H(idx)[0], i), t
        assert np.max(np.abs(H(wt)[0] - w) / np.abs(w)) <= 1e-5, t
        w_, _ = check_tolerance(orc, L, Xh[t:t + 1], H(out), [0])
        worst = max(worst, w_)
    print(f"\n  fast decode, full size: max norm-relative error {worst:.2e}")


def test_verify_64_full_size(env, full_layer):
    """Config 4: 64 tokens, Zipf(1.2) bias, 256 experts x inter 2048."""
    torch, orc, lib, synth = env["torch"], env["orc"], env["lib"], env["synth"]
    DL, L = with_zipf(env, *full_layer, 256)
    X = synth.bf16_tokens(64, 4096, seed=11 + 64, device=env["dev"])
    Xh = H(X)
    ro32 = torch.empty(64, 7, 4096, dtype=torch.float32, device=env["dev"])
    out, idx, wt = lib.moe_forward_batch(DL, X, route_out=ro32)
    out, idx, wt, ro32 = H(out), H(idx), H(wt), H(ro32)
    assert np.all(np.isfinite(out))
    ri, rw = orc.route_tokens(L, Xh)
    assert np.array_equal(idx, ri)
    assert same_bits(wt, rw)
    print("\n  verify 64: experts hit", len(np.unique(idx)))
    worst, exact = check_tolerance(orc, L, Xh, out, range(64))
    wr = check_route_outputs(orc, L, Xh, ro32, idx, range(0, 64, 4))
    print(f"  outputs: bit-exact {exact}/64, max norm-relative {worst:.2e}; "
          f"per-route fp32 max|d|/max|ref| {wr:.2e}")


def test_prefill_4096_full_size(env, full_layer):
    """Config 5: 4096 tokens, Zipf(1.2) bias: routing of every token, outputs
    and pre-rounding route outputs of a sample."""
    torch, orc, lib, synth = env["torch"], env["orc"], env["lib"], env["synth"]
    DL, L = with_zipf(env, *full_layer, 256)
    X = synth.bf16_tokens(4096, 4096, seed=11 + 4096, device=env["dev"])
    Xh = H(X)
    ro32 = torch.empty(4096, 7, 4096, dtype=torch.float32, device=env["dev"])
    out, idx, wt = lib.moe_forward_batch(DL, X, route_out=ro32)
    out, idx, wt = H(out), H(idx), H(wt)
    assert np.all(np.isfinite(out))
    ri, rw = orc.route_tokens(L, Xh)
    bad = np.nonzero(~np.all(idx == ri, axis=1))[0]
    assert bad.size == 0, bad[:10]
    assert same_bits(wt, rw)
    counts = np.bincount(idx.ravel(), minlength=256)
    print(f"\n  prefill 4096: experts hit {(counts > 0).sum()}, max {counts.max()}, "
          f"median {np.median(counts)}")
    sample = list(np.random.default_rng(3).choice(4096, 16, replace=False))
    ro = H(ro32[torch.tensor(sample, device=env["dev"])])
    wr = check_route_outputs(orc, L, Xh[sample], ro, idx[sample], range(len(sample)))
    worst, exact = check_tolerance(orc, L, Xh, out, sample)
    print(f"  sample outputs: bit-exact {exact}/16, max norm-relative {worst:.2e}; "
          f"per-route fp32 max|d|/max|ref| {wr:.2e}")


def test_512_experts_decode_and_batch(env):
    """512 experts (hidden 4096, inter 256): decode bit-exact; the batched
    router at 64 and 300 tokens (both router kernel sets) routes every token
    bit-identically, outputs within the tolerance."""
    orc, lib, synth = env["orc"], env["lib"], env["synth"]
    DL = synth.device_layer(seed=5, hidden=4096, inter=256, n_experts=512, device=env["dev"])
    L = synth.host_copy(DL)
    DL, L = with_zipf(env, DL, L, 512)
    X = synth.bf16_tokens(300, 4096, seed=13, device=env["dev"])
    Xh = H(X)
    out, idx, wt = lib.moe_forward(DL, X[:3])
    for t in range(3):
        o, i, w = orc.moe_forward(L, Xh[t])
        assert np.array_equal(H(idx)[t], i) and same_bits(H(wt)[t], w), t
        assert same_bits(H(out)[t], o), t
    for n in (64, 300):
        out, idx, wt = lib.moe_forward_batch(DL, X[:n])
        out, idx, wt = H(out), H(idx), H(wt)
        ri, rw = orc.route_tokens(L, Xh[:n])
        assert np.array_equal(idx, ri) and same_bits(wt, rw), n
        check_tolerance(orc, L, Xh, out, range(0, n, 3))


@pytest.mark.parametrize("n", [64, 4096])
def test_batch_result_independent_of_workspace_contents(env, full_layer, n):
    """The batched layer reads nothing of its workspace that it has not
    written in the same call: a workspace full of 0xFF bytes (NaN patterns)
    and one full of zeros give the same bits."""
    torch, lib, synth = env["torch"], env["lib"], env["synth"]
    DL, L = with_zipf(env, *full_layer, 256)
    X = synth.bf16_tokens(n, 4096, seed=11 + n, device=env["dev"])
    need = lib.moe_batch_workspace_bytes(DL, n)
    res = []
    for fill in (0x00, 0xFF, 0x00):
        ws = torch.full((need,), fill, dtype=torch.uint8, device=env["dev"])
        out, idx, wt = lib.moe_forward_batch(DL, X, workspace=ws)
        torch.cuda.synchronize()
        res.append((H(out), H(idx), H(wt)))
        del ws
    for r in res[1:]:
        assert np.array_equal(r[1], res[0][1]) and same_bits(r[2], res[0][2])
        diff = np.nonzero(~np.all(r[0].view(np.uint32) == res[0][0].view(np.uint32), axis=1))[0]
        assert diff.size == 0, (diff.size, diff[:10])
