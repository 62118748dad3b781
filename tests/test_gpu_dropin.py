"""GPU tests of the drop-in layer: the reference-named entry points with host
buffers (include/dsv4/dsv4.h:185-211, 251-254; src/dsv4/dsv4_internal.h:
256-286, 326-331), called through ctypes exactly as the reference's C callers
would call them, bit for bit against the reference's golden vectors and the
oracle; and the weight residency rules: a registered range stays resident
until re-registered or forgotten, an unregistered buffer refilled with other
weights is never served stale."""
import ctypes as C

import numpy as np
import pytest

from common import bf16_bits, bf16_input, pyoracle, same_bits
from test_gpu_decode import GOLDEN

pytestmark = pytest.mark.gpu

f32p, u8p, u16p = C.POINTER(C.c_float), C.POINTER(C.c_uint8), C.POINTER(C.c_uint16)
i32p, i64p = C.POINTER(C.c_int), C.POINTER(C.c_int64)


def P(a, t):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(t)


def PP(rows):
    """float *const * over the rows of a 2-D float32 array."""
    arr = (f32p * rows.shape[0])(*[r.ctypes.data_as(f32p) for r in rows])
    return arr


@pytest.fixture(scope="module")
def env():
    import torch  # noqa: F401  (initialises the ROCm runtime the library uses)
    import dsv4_gpu
    lib = C.CDLL(dsv4_gpu.LIB_PATH)
    lib.dsv4_gpu_register_weights.restype = C.c_int
    lib.dsv4_gpu_register_weights.argtypes = [C.c_void_p, C.c_size_t]
    lib.dsv4_gpu_forget_weights.argtypes = [C.c_void_p]
    lib.dsv4_gpu_forget_weights_range.argtypes = [C.c_void_p, C.c_size_t]
    lib.dsv4_router.argtypes = [i32p, f32p, f32p, C.c_void_p, f32p, i64p, C.c_int, C.c_int,
                                C.c_int, C.c_int, C.c_int, C.c_float, C.c_float]
    return dict(lib=lib, orc=pyoracle.Oracle(), gold=np.load(GOLDEN, allow_pickle=False))


def test_dropin_gemvs_golden(env):
    """Every GEMV drop-in on the reference's own golden vectors."""
    lib, g = env["lib"], env["gold"]
    IN, R = 256, 48
    qx, qs = np.ascontiguousarray(g["g_qx"]), np.ascontiguousarray(g["g_qs"])
    W4, S4, W4b, S4b = (np.ascontiguousarray(g[k]) for k in ("g_W4", "g_S4", "g_W4b", "g_S4b"))
    W8, S8, W8b, S8b = (np.ascontiguousarray(g[k]) for k in ("g_W8", "g_S8", "g_W8b", "g_S8b"))
    y, y1 = np.empty(R, np.float32), np.empty(R, np.float32)
    lib.dsv4_gemv_fp4_q(P(y, f32p), P(qx, f32p), P(qs, f32p), P(W4, u8p), P(S4, u8p), IN, R)
    assert same_bits(y, g["g_fp4"])
    lib.dsv4_gemv_fp4_pair_q(P(y, f32p), P(y1, f32p), P(qx, f32p), P(qs, f32p), P(W4, u8p),
                             P(S4, u8p), P(W4b, u8p), P(S4b, u8p), IN, R)
    assert same_bits(y, g["g_fp4_pair0"]) and same_bits(y1, g["g_fp4_pair1"])
    for ro, key in ((1, "g_fp8"), (0, "g_fp8_raw")):
        lib.dsv4_gemv_fp8_q(P(y, f32p), P(qx, f32p), P(qs, f32p), P(W8, u8p), P(S8, u8p), IN,
                            R, ro)
        assert same_bits(y, g[key]), key
    lib.dsv4_gemv_fp8_pair_q(P(y, f32p), P(y1, f32p), P(qx, f32p), P(qs, f32p), P(W8, u8p),
                             P(S8, u8p), P(W8b, u8p), P(S8b, u8p), IN, R)
    assert same_bits(y, g["g_fp8_pair0"]) and same_bits(y1, g["g_fp8_pair1"])
    bqx, bqs = np.ascontiguousarray(g["g_bqx"]), np.ascontiguousarray(g["g_bqs"])
    nb = bqx.shape[0]
    Y = np.empty((nb, R), np.float32)
    lib.dsv4_gemv_fp4_batch_q(PP(Y), PP(bqx), PP(bqs), nb, P(W4, u8p), P(S4, u8p), IN, R)
    assert same_bits(Y, g["g_fp4_batch"])
    lib.dsv4_gemv_fp8_batch_q(PP(Y), PP(bqx), PP(bqs), nb, P(W8, u8p), P(S8, u8p), IN, R, 1)
    assert same_bits(Y, g["g_fp8_batch"])
    x = np.ascontiguousarray(g["g_bf16_x"])
    Wb = np.ascontiguousarray(g["g_bf16_W"])
    lib.dsv4_gemv_bf16(P(y, f32p), P(x, f32p), P(Wb, u16p), IN, R, 0)
    assert same_bits(y, g["g_bf16"])
    codes, fsc = np.ascontiguousarray(g["g_f8_codes"]), np.ascontiguousarray(g["g_f8_scales"])
    lib.dsv4_gemv_fp8(P(y, f32p), P(x, f32p), P(codes, u8p), P(fsc, f32p), IN, R, 128)
    assert same_bits(y, g["g_fp8_legacy"])
    lib.dsv4_gemv_fp8_tbl(P(y, f32p), P(x, f32p), P(codes, u8p), P(fsc, f32p), IN, R, 128)
    assert same_bits(y, g["g_fp8_tbl"])
    w4s = np.ascontiguousarray(g["g_fp4_wscale"])
    lib.dsv4_gemv_fp4(P(y, f32p), P(qx, f32p), P(qs, f32p), P(W4, u8p), P(w4s, f32p), IN, R, 32)
    assert same_bits(y, g["g_fp4_legacy"])


def test_dropin_quant_router_bf16_batch(env):
    """dsv4_quant_fp8_act / _codes, dsv4_router (plain and hash) on the golden
    vectors, dsv4_gemv_bf16_batch against the oracle at the router's shape."""
    lib, g, orc = env["lib"], env["gold"], env["orc"]
    x = np.ascontiguousarray(g["quant_in"])
    n = x.shape[-1]
    for name in ("dsv4_quant_fp8_act", "dsv4_quant_fp8_codes"):
        qx, qs = np.empty(n, np.float32), np.empty((n + 127) // 128, np.float32)
        getattr(lib, name)(P(qx, f32p), P(qs, f32p), P(x, f32p), n)
        assert same_bits(qx, g["quant_qx"]) and same_bits(qs, g["quant_qs"]), name
    rx, rG = np.ascontiguousarray(g["rt_x"]), np.ascontiguousarray(g["rt_G"])
    rb, t2e = np.ascontiguousarray(g["rt_bias"]), np.ascontiguousarray(g["rt_t2e"])
    idx, wt = np.empty(6, np.int32), np.empty(6, np.float32)
    lib.dsv4_router(P(idx, i32p), P(wt, f32p), P(rx, f32p), rG.ctypes.data, P(rb, f32p), None,
                    0, 256, 16, 6, 0, C.c_float(1.5), C.c_float(1e-6))
    assert np.array_equal(idx, g["rt_idx"]) and same_bits(wt, g["rt_wt"])
    lib.dsv4_router(P(idx, i32p), P(wt, f32p), P(rx, f32p), rG.ctypes.data, None,
                    P(t2e, i64p), 2, 256, 16, 6, 1, C.c_float(1.5), C.c_float(1e-6))
    assert np.array_equal(idx, g["rt_hidx"]) and same_bits(wt, g["rt_hwt"])
    rng = np.random.default_rng(3)
    Gb = bf16_bits(rng.standard_normal((256, 4096), dtype=np.float32) / 64)
    X = bf16_input(rng, (5, 4096))
    Y = np.empty((5, 256), np.float32)
    lib.dsv4_gemv_bf16_batch(PP(Y), PP(X), 5, P(Gb, u16p), 4096, 256, 0)
    for t in range(5):
        assert same_bits(Y[t], orc.gemv_bf16(X[t], Gb, 4096, 256, 0)), t


def slot_buffer(orc, rng, rows, in_):
    """A reference-style expert slot: [scales | weights] of one FP4 matrix in
    one host buffer (the reference passes pointers into such buffers)."""
    w = rng.standard_normal((rows, in_), dtype=np.float32) * 0.02
    packed, scales = orc.quant_fp4_rows(w)
    buf = np.concatenate([scales.ravel(), packed.ravel()])
    return buf, scales.size


def call_fp4(lib, buf, nsc, qx, qs, rows, in_):
    y = np.empty(rows, np.float32)
    base = buf.ctypes.data
    lib.dsv4_gemv_fp4_q(P(y, f32p), P(qx, f32p), P(qs, f32p), C.cast(base + nsc, u8p),
                        C.cast(base, u8p), in_, rows)
    return y


def test_dropin_weight_residency(env):
    """Unregistered buffers are read afresh every call; a registered slot
    buffer (pointers into its middle included) is served from HBM, refreshed
    by re-registration, and read afresh again once forgotten."""
    lib, orc = env["lib"], env["orc"]
    rng = np.random.default_rng(7)
    rows, in_ = 512, 1024
    x = bf16_input(rng, in_)
    qx, qs = orc.quant_fp8_act(x)
    buf, nsc = slot_buffer(orc, rng, rows, in_)
    other, _ = slot_buffer(orc, rng, rows, in_)
    want = lambda b: orc.gemv_fp4_q(qx, qs, b[nsc:], b[:nsc], in_, rows)
    w_a, w_b = want(buf.copy()), want(other)
    assert not same_bits(w_a, w_b)
    # unregistered: refilling the buffer (as an expert cache does on a miss)
    # changes the next call's result
    assert same_bits(call_fp4(lib, buf, nsc, qx, qs, rows, in_), w_a)
    keep = buf.copy()
    buf[:] = other
    assert same_bits(call_fp4(lib, buf, nsc, qx, qs, rows, in_), w_b)
    buf[:] = keep
    # registered: resident; re-registration after a refill uploads the new
    # contents (the pointers into the buffer's middle resolve inside it)
    assert lib.dsv4_gpu_register_weights(buf.ctypes.data, buf.nbytes) == 0
    assert same_bits(call_fp4(lib, buf, nsc, qx, qs, rows, in_), w_a)
    buf[:] = other
    assert lib.dsv4_gpu_register_weights(buf.ctypes.data, buf.nbytes) == 0
    assert same_bits(call_fp4(lib, buf, nsc, qx, qs, rows, in_), w_b)
    # forgetting by any address inside the range drops it
    lib.dsv4_gpu_forget_weights(C.c_void_p(buf.ctypes.data + nsc + 100))
    buf[:] = keep
    assert same_bits(call_fp4(lib, buf, nsc, qx, qs, rows, in_), w_a)
    # forget_range over part of a registered range drops the whole entry
    assert lib.dsv4_gpu_register_weights(buf.ctypes.data, buf.nbytes) == 0
    lib.dsv4_gpu_forget_weights_range(C.c_void_p(buf.ctypes.data + 10), 20)
    buf[:] = other
    assert same_bits(call_fp4(lib, buf, nsc, qx, qs, rows, in_), w_b)
