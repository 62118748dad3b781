"""The attention FP8 projections (src/dsv4/dsv4_internal.h:57-62): wq_a
[1024][4096], wq_b [32768][1024], wkv [512][4096] and wo_b [4096][8192], FP8
E4M3 with 128 x 128 E8M0 block scales, through dsv4_gemv_fp8_q (one token,
src/dsv4/dsv4_model.c:5271-5296, 5414) and dsv4_gemv_fp8_batch_q (up to
DSV4_MAX_TOPK + 1 = 33 tokens, :7859-7898, 8024), bit-exact against the
oracle; plus the paired form and odd widths."""
from __future__ import annotations

import numpy as np
import pytest

from common import bf16_values, pyoracle, same_bits

pytestmark = pytest.mark.gpu

SHAPES = {"wq_a": (1024, 4096), "wq_b": (32768, 1024), "wkv": (512, 4096),
          "wo_b": (4096, 8192)}


@pytest.fixture(scope="module")
def env():
    import torch
    import dsv4_gpu
    return dict(torch=torch, lib=dsv4_gpu.lib(), orc=pyoracle.Oracle(),
                dev=torch.device("cuda:0"))


def T(env, a):
    return env["torch"].from_numpy(np.ascontiguousarray(a).copy()).to(env["dev"])


def fp8_weights(orc, rng, rows, cols, nan_block=False):
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    codes, scales = orc.quant_fp8_blocks_e8m0(w)
    if nan_block:
        scales = scales.copy()
        scales[0, min(1, scales.shape[1] - 1)] = 255  # NaN scale: the block is skipped
    return codes, scales


@pytest.mark.parametrize("name", sorted(SHAPES))
def test_projection_shapes_bit_exact(env, name):
    orc, lib = env["orc"], env["lib"]
    rows, cols = SHAPES[name]
    rng = np.random.default_rng(rows + cols)
    W, S = fp8_weights(orc, rng, rows, cols, nan_block=True)
    Wt, St = T(env, W), T(env, S)
    for n in (1, 5, 33):
        x = bf16_values(rng.standard_normal((n, cols)).astype(np.float32))
        qx, qs = orc.quant_fp8_act(x)
        if n == 1:
            y = lib.gemv_fp8_q(T(env, qx[0]), T(env, qs[0]), Wt, St, cols, rows)
            y = y.cpu().numpy()[None]
        else:
            y = lib.gemv_fp8_batch_q(T(env, qx), T(env, qs), Wt, St, cols, rows).cpu().numpy()
        rows_chk = np.unique(np.r_[0, 1, 127, 128, rows - 1,
                                   rng.integers(0, rows, 256 if rows > 4096 else rows)])
        Wc, Sc = W[rows_chk], S[rows_chk // 128]
        for t in range(n) if n <= 5 else (0, 7, 16, 31, 32):
            # oracle on the sampled rows: each row with its own block-scale row
            want = np.array([orc.gemv_fp8_q(qx[t], qs[t], Wc[k:k + 1], Sc[k:k + 1], cols, 1)[0]
                             for k in range(len(rows_chk))], np.float32)
            assert same_bits(y[t][rows_chk], want), (name, n, t)


def test_full_rows_and_unrounded(env):
    """Every row of wkv and of a 300 x 2000 matrix (width not a multiple of
    128), with and without BF16 output rounding, one and 9 tokens."""
    orc, lib = env["orc"], env["lib"]
    rng = np.random.default_rng(3)
    for rows, cols in ((512, 4096), (300, 2000)):
        W, S = fp8_weights(orc, rng, rows, cols)
        x = bf16_values(rng.standard_normal((9, cols)).astype(np.float32))
        qx, qs = orc.quant_fp8_act(x)
        for ro in (1, 0):
            y = lib.gemv_fp8_batch_q(T(env, qx), T(env, qs), T(env, W), T(env, S), cols, rows,
                                     round_out=ro).cpu().numpy()
            want = orc.gemv_fp8_batch_q(qx, qs, W, S, cols, rows, round_out=ro)
            assert same_bits(y, want), (rows, cols, ro)
            y1 = lib.gemv_fp8_q(T(env, qx[4]), T(env, qs[4]), T(env, W), T(env, S), cols, rows,
                                round_out=ro).cpu().numpy()
            assert same_bits(y1, want[4]), (rows, cols, ro)


def test_pair(env):
    orc, lib = env["orc"], env["lib"]
    rng = np.random.default_rng(4)
    rows, cols = 2048, 4096
    W0, S0 = fp8_weights(orc, rng, rows, cols)
    W1, S1 = fp8_weights(orc, rng, rows, cols)
    x = bf16_values(rng.standard_normal(cols).astype(np.float32))
    qx, qs = orc.quant_fp8_act(x)
    y0, y1 = lib.gemv_fp8_pair_q(T(env, qx), T(env, qs), T(env, W0), T(env, S0), T(env, W1),
                                 T(env, S1), cols, rows)
    w0, w1 = orc.gemv_fp8_pair_q(qx, qs, W0, S0, W1, S1, cols, rows)
    assert same_bits(y0.cpu().numpy(), w0) and same_bits(y1.cpu().numpy(), w1)
