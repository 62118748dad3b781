"""The oracle's caller step around the MoE (rmsnorm_bf16, dsv4_hc_split,
hc_pre, hc_post) pinned on the CPU: against the reference's own functions
compiled in oracle/_ref (rmsnorm_bf16, hc_pre_scratch and hc_post_scratch of
src/dsv4/dsv4_model.c:4934-4951, 7123-7177 through ref_shim.c, and the public
dsv4_hc_split of src/dsv4/dsv4_ops.c:415-466), on the reference's tiny
checkpoint weights, and against closed forms that a dropped term, a wrong
index or a transposed operand would break."""
from __future__ import annotations

import os

import numpy as np
import pytest

from common import ROOT, bf16_bits, bf16_values, same_bits
import pyoracle

TINY = os.path.join(ROOT, "tests", "golden", "tiny_dsv4")


@pytest.fixture(scope="module")
def orc():
    return pyoracle.Oracle()


@pytest.fixture(scope="module")
def ref():
    if not pyoracle.ref_available():
        pytest.skip("oracle/_ref not built")
    return pyoracle.RefLib()


def hc_inputs(rng, mult, hid, fn_sigma=0.01):
    mix_n = (2 + mult) * mult
    state = bf16_values(rng.standard_normal(mult * hid).astype(np.float32))
    fn = (rng.standard_normal((mix_n, mult * hid)) * fn_sigma).astype(np.float32)
    scale3 = (0.5 + rng.random(3)).astype(np.float32)
    base = (rng.standard_normal(mix_n) * 0.5).astype(np.float32)
    return state, fn, scale3, base


def midpoint_state(mult, hid):
    """A state of n = mult*hid = 2^k values (k even) whose sum of squares is
    n + n*2^-24 exactly (n/4 values of 2, one of 2^((k-24)/2), zeros), so
    ss/n = 1 + 2^-24 is the midpoint between two floats and its float
    conversion rounds to even (1.0)."""
    n = mult * hid
    k = int(np.log2(n))
    assert 2 ** k == n and k % 2 == 0
    s = np.zeros(n, np.float32)
    s[: n // 4] = 2.0
    s[n // 4] = np.float32(2.0 ** ((k - 24) // 2))
    return s


def fmaf(a, b, c):
    """The host libm's fmaf (correctly rounded fused multiply-add)."""
    import ctypes
    f = ctypes.CDLL("libm.so.6").fmaf
    f.restype = ctypes.c_float
    f.argtypes = [ctypes.c_float] * 3
    return np.float32(f(float(a), float(b), float(c)))


def test_rmsnorm_matches_reference(orc, ref):
    rng = np.random.default_rng(1)
    for n in (4096, 1024, 512, 64, 8, 7):
        x = rng.standard_normal((3, n)).astype(np.float32) * rng.random((3, 1)).astype(np.float32)
        w = bf16_bits(1.0 + 0.1 * rng.standard_normal(n).astype(np.float32))
        for gain in (w, None):
            for rnd in (0, 1):
                assert same_bits(orc.rmsnorm_bf16(x, gain, 1e-6, rnd),
                                 ref.rmsnorm_bf16(x, gain, 1e-6, rnd))


def test_rmsnorm_closed_forms(orc):
    """x all ones: ss = n exactly, r = 1/sqrtf(1 + eps); x zero: y zero;
    the midpoint sum rounds to even before the reciprocal square root."""
    n = 4096
    w = bf16_bits(np.linspace(0.5, 1.5, n).astype(np.float32))
    y = orc.rmsnorm_bf16(np.ones((1, n), np.float32), w, 1e-6, 0)[0]
    r = np.float32(1) / np.sqrt(np.float32(1) + np.float32(1e-6))
    want = (np.float32(1) * r) * bf16_values(np.linspace(0.5, 1.5, n).astype(np.float32))
    assert same_bits(y, want)
    assert not orc.rmsnorm_bf16(np.zeros((1, n), np.float32), w, 1e-6, 1).any()
    x = midpoint_state(1, n)
    y = orc.rmsnorm_bf16(x[None], None, 0.0, 0)[0]
    assert same_bits(y, x * np.float32(1.0))  # (float)(1 + 2^-24) == 1.0: r == 1


def test_hc_split_matches_reference(orc, ref):
    rng = np.random.default_rng(2)
    for mult in (1, 2, 3, 4, 7):
        mix_n = (2 + mult) * mult
        for it in (1, 2, 20):
            for _ in range(20):
                mixes = (rng.standard_normal(mix_n) * 3).astype(np.float32)
                sc = (rng.random(3) * 2).astype(np.float32)
                base = rng.standard_normal(mix_n).astype(np.float32)
                a = orc.hc_split(mixes, sc, base, mult, it, 1e-6)
                b = ref.hc_split(mixes, sc, base, mult, it, 1e-6)
                assert all(same_bits(u, v) for u, v in zip(a, b)), (mult, it)


def test_hc_split_invariants(orc):
    """pre in (eps, 1 + eps], post in [0, 2], comb column sums 1 after the
    final column pass and row sums near 1 after 20 iterations; scale 0
    gives pre = sigmoid(base) + eps exactly."""
    rng = np.random.default_rng(3)
    mult = 4
    mixes = (rng.standard_normal(24) * 2).astype(np.float32)
    base = rng.standard_normal(24).astype(np.float32)
    pre, post, comb = orc.hc_split(mixes, np.ones(3, np.float32), base, mult, 20, 1e-6)
    c = comb.reshape(4, 4).astype(np.float64)
    assert np.all(pre > 1e-6) and np.all(pre <= 1 + 1e-6)
    assert np.all(post >= 0) and np.all(post <= 2)
    assert np.allclose(c.sum(0), 1, atol=1e-5) and np.allclose(c.sum(1), 1, atol=5e-3)
    pre0, _, _ = orc.hc_split(mixes, np.zeros(3, np.float32), base, mult, 20, 1e-6)
    sig = np.where(base[:4] >= 0, 1 / (1 + np.exp(-base[:4].astype(np.float64))),
                   np.exp(base[:4].astype(np.float64)) / (1 + np.exp(base[:4].astype(np.float64))))
    assert np.allclose(pre0, sig + 1e-6, rtol=1e-6)


@pytest.mark.parametrize("mult,hid", [(4, 4096), (4, 256), (2, 8), (1, 64), (3, 100), (7, 32)])
def test_hc_pre_matches_reference(orc, ref, mult, hid):
    rng = np.random.default_rng(mult * 1000 + hid)
    state, fn, sc, base = hc_inputs(rng, mult, hid)
    a = orc.hc_pre(state, fn, sc, base, mult)
    b = ref.hc_pre(state, fn, sc, base, mult)
    assert all(same_bits(u, v) for u, v in zip(a, b))


def test_hc_pre_closed_form(orc):
    """fn = 0 gives mixes 0, so pre = sigmoid(base) + eps from the split
    alone, and bin[c] = bf16 of the fmaf chain of pre over the mult streams
    (pre from hc_split, each step the host libm's correctly rounded fmaf)."""
    mult, hid = 4, 256
    rng = np.random.default_rng(4)
    state, fn, sc, base = hc_inputs(rng, mult, hid)
    fn[:] = 0
    bin_, post, comb = orc.hc_pre(state, fn, sc, base, mult)
    pre, post2, comb2 = orc.hc_split(np.zeros(24, np.float32), sc, base, mult, 20, 1e-6)
    assert same_bits(post, post2) and same_bits(comb, comb2)
    S = state.reshape(mult, hid)
    acc = np.zeros(hid, np.float32)
    for i in range(mult):
        acc = np.array([fmaf(pre[i], S[i, c], acc[c]) for c in range(hid)], np.float32)
    assert same_bits(bin_, bf16_values(acc))


def test_hc_pre_midpoint_sum(orc, ref):
    """The sum of squares lands exactly on a float midpoint (the case the
    GPU settles with its sequential fallback)."""
    mult, hid = 4, 4096
    rng = np.random.default_rng(5)
    _, fn, sc, base = hc_inputs(rng, mult, hid)
    state = midpoint_state(mult, hid)
    a = orc.hc_pre(state, fn, sc, base, mult)
    b = ref.hc_pre(state, fn, sc, base, mult)
    assert all(same_bits(u, v) for u, v in zip(a, b))


def test_hc_post_matches_reference_and_closed_forms(orc, ref):
    rng = np.random.default_rng(6)
    for mult, hid in ((4, 4096), (2, 8), (7, 33)):
        state = bf16_values(rng.standard_normal(mult * hid).astype(np.float32))
        br = bf16_values(rng.standard_normal(hid).astype(np.float32))
        post = (rng.random(mult) * 2).astype(np.float32)
        comb = rng.random(mult * mult).astype(np.float32)
        assert same_bits(orc.hc_post(state, br, post, comb, mult),
                         ref.hc_post(state, br, post, comb, mult))
        eye = np.eye(mult, dtype=np.float32).ravel()
        assert same_bits(orc.hc_post(state, br, np.zeros(mult, np.float32), eye, mult), state)
        out = orc.hc_post(state, br, np.ones(mult, np.float32), np.zeros(mult * mult, np.float32),
                          mult)
        assert same_bits(out, np.tile(br, mult))


def test_tiny_checkpoint_hc_weights(orc, ref):
    """The reference's tiny checkpoint (hidden 8, hc_mult 2): its layers'
    hc_ffn_fn / scale / base through hc_pre, and ffn_norm through rmsnorm."""
    from dsv4_gpu import Checkpoint
    ck = Checkpoint(TINY)
    rng = np.random.default_rng(7)
    for layer in range(4):
        pre = f"layers.{layer}."
        fn = ck.read_f32(pre + "hc_ffn_fn").reshape(8, 16)
        sc = ck.read_f32(pre + "hc_ffn_scale")
        base = ck.read_f32(pre + "hc_ffn_base")
        norm = np.frombuffer(ck.read(pre + "ffn_norm.weight"), np.uint16)
        state = bf16_values(rng.standard_normal(16).astype(np.float32))
        a = orc.hc_pre(state, fn, sc, base, 2)
        b = ref.hc_pre(state, fn, sc, base, 2)
        assert all(same_bits(u, v) for u, v in zip(a, b))
        assert same_bits(orc.rmsnorm_bf16(a[0][None], norm), ref.rmsnorm_bf16(b[0][None], norm))
