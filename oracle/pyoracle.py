"""ctypes bindings for the CPU checker (TEST INFRASTRUCTURE ONLY).

``Oracle`` wraps oracle/liboracle.so (the C restatement). ``RefLib`` wraps
oracle/_ref/libdsv4_ref.so, the reference engine compiled from its own sources
(oracle/Makefile), exposing the same methods with the reference's own
functions behind them. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module.

All arrays are numpy; batched methods take [batch, n] arrays.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libdsv4_ref.so")

_f32p = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_u16p = C.POINTER(C.c_uint16)
_i32p = C.POINTER(C.c_int)
_i64p = C.POINTER(C.c_int64)


def _p(a, t):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return a.ctypes.data_as(t)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class OrcLayer(C.Structure):
    """Mirror of OrcLayer in oracle/dsv4_oracle.h."""

    _fields_ = [
        ("hidden", C.c_int), ("inter", C.c_int), ("n_experts", C.c_int),
        ("topk", C.c_int), ("route_scale", C.c_float),
        ("swiglu_limit", C.c_float), ("gate_w", _u16p), ("bias", _f32p),
        ("tid2eid", _i64p), ("is_hash", C.c_int), ("experts", _u8p),
        ("expert_stride", C.c_size_t), ("scale_run", C.c_size_t),
        ("sh1", _u8p), ("sh1_s", _u8p), ("sh3", _u8p), ("sh3_s", _u8p),
        ("sh2", _u8p), ("sh2_s", _u8p),
    ]


def make_layer_struct(layer) -> OrcLayer:
    """Build an OrcLayer from a host-side layer dict (see tests/common.py)."""
    L = OrcLayer()
    L.hidden, L.inter = layer["hidden"], layer["inter"]
    L.n_experts, L.topk = layer["n_experts"], layer["topk"]
    L.route_scale, L.swiglu_limit = layer["route_scale"], layer["swiglu_limit"]
    L.gate_w = _p(layer["gate_w"], _u16p)
    L.bias = _p(layer.get("bias"), _f32p)
    L.tid2eid = _p(layer.get("tid2eid"), _i64p)
    L.is_hash = 1 if layer.get("tid2eid") is not None else 0
    L.experts = _p(layer["experts"], _u8p)
    L.expert_stride = layer["expert_stride"]
    L.scale_run = layer["scale_run"]
    for k in ("sh1", "sh1_s", "sh3", "sh3_s", "sh2", "sh2_s"):
        setattr(L, k, _p(layer[k], _u8p))
    return L


class _Base:
    """Shared numpy-level API; subclasses bind symbol names."""

    lib: C.CDLL

    # ---- scalar decode ----
    def fp8_table(self):
        return np.array([self._fp8(i) for i in range(256)], dtype=np.float32)

    def e8m0_table(self):
        return np.array([self._e8m0(i) for i in range(256)], dtype=np.float32)

    def f32_to_bf16(self, x):
        x = f32(x).ravel()
        return np.array([self._bf16(float(v)) for v in x], dtype=np.uint16)

    def round_e4m3(self, x):
        x = f32(x).ravel()
        return np.array([self._rnd(float(v)) for v in x], dtype=np.float32)

    def quant_fp8_act(self, x):
        x = f32(x)
        n = x.shape[-1]
        qx = np.empty_like(x)
        qs = np.empty(x.shape[:-1] + ((n + 127) // 128,), np.float32)
        for i in np.ndindex(x.shape[:-1]):
            self._quant(_p(qx[i], _f32p), _p(qs[i], _f32p), _p(x[i], _f32p), n)
        return qx, qs

    # ---- caller step around the MoE (symbol names from _STEP) ----
    _STEP = {}

    def _step(self, key):
        return getattr(self.lib, self._STEP[key])

    def rmsnorm_bf16(self, x, w=None, eps=1e-6, round_out=1):
        """Rows of x [.., n] (w: BF16 gain bits [n] or None)."""
        x = f32(x)
        y = np.empty_like(x)
        n = x.shape[-1]
        wp = None if w is None else _p(np.ascontiguousarray(w, np.uint16), _u16p)
        fn = self._step("rmsnorm")
        for i in np.ndindex(x.shape[:-1]):
            fn(_p(y[i], _f32p), _p(x[i], _f32p), wp, n, C.c_float(eps), round_out)
        return y

    def hc_split(self, mixes, scale3, base, mult, iters=20, eps=1e-6):
        mixes, scale3, base = f32(mixes), f32(scale3), f32(base)
        pre = np.empty(mult, np.float32)
        post = np.empty(mult, np.float32)
        comb = np.empty(mult * mult, np.float32)
        self._step("split")(_p(pre, _f32p), _p(post, _f32p), _p(comb, _f32p),
                            _p(mixes, _f32p), _p(scale3, _f32p), _p(base, _f32p), mult, iters,
                            C.c_float(eps))
        return pre, post, comb

    def hc_pre(self, state, fn, scale3, base, mult, iters=20, rms_eps=1e-6, hc_eps=1e-6):
        """One token: state [mult*hid] -> bin [hid], post [mult], comb [mult*mult]."""
        state, fn, scale3, base = f32(state), f32(fn), f32(scale3), f32(base)
        hid = state.size // mult
        bin_ = np.empty(hid, np.float32)
        post = np.empty(mult, np.float32)
        comb = np.empty(mult * mult, np.float32)
        self._step("pre")(_p(bin_, _f32p), _p(post, _f32p), _p(comb, _f32p),
                          _p(state, _f32p), _p(fn, _f32p), _p(scale3, _f32p), _p(base, _f32p),
                          mult, hid, iters, C.c_float(rms_eps), C.c_float(hc_eps))
        return bin_, post, comb

    def hc_post(self, state, branch, post, comb, mult):
        """One token: the new state [mult*hid] (input not modified)."""
        st = f32(state).copy()
        branch, post, comb = f32(branch), f32(post), f32(comb)
        self._step("post")(_p(st, _f32p), _p(branch, _f32p), _p(post, _f32p), _p(comb, _f32p),
                           mult, st.size // mult)
        return st


class Oracle(_Base):
    """The C restatement (oracle/dsv4_oracle.c)."""

    _STEP = {"rmsnorm": "orc_rmsnorm_bf16", "split": "orc_hc_split", "pre": "orc_hc_pre",
             "post": "orc_hc_post"}

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        lib = self.lib = C.CDLL(path)
        for name, res in [("orc_fp8_e4m3", C.c_float), ("orc_e8m0", C.c_float),
                          ("orc_round_e4m3", C.c_float),
                          ("orc_sqrt_softplus", C.c_float),
                          ("orc_f32_to_bf16", C.c_uint16),
                          ("orc_fp4_e2m1", C.c_float),
                          ("orc_e4m3_code", C.c_uint8),
                          ("orc_checksum", C.c_double),
                          ("orc_xorshift_next", C.c_uint64)]:
            getattr(lib, name).restype = res
        lib.orc_fp8_e4m3.argtypes = [C.c_uint8]
        lib.orc_e8m0.argtypes = [C.c_uint8]
        lib.orc_fp4_e2m1.argtypes = [C.c_uint8]
        lib.orc_round_e4m3.argtypes = [C.c_float]
        lib.orc_sqrt_softplus.argtypes = [C.c_float]
        lib.orc_f32_to_bf16.argtypes = [C.c_float]
        lib.orc_e4m3_code.argtypes = [C.c_float]
        self._fp8, self._e8m0 = lib.orc_fp8_e4m3, lib.orc_e8m0
        self._bf16, self._rnd = lib.orc_f32_to_bf16, lib.orc_round_e4m3
        self._quant = lib.orc_quant_fp8_act

    def sqrt_softplus(self, z):
        return np.array([self.lib.orc_sqrt_softplus(float(v)) for v in f32(z).ravel()],
                        dtype=np.float32)

    def fp4_table(self):
        return np.array([self.lib.orc_fp4_e2m1(i) for i in range(16)], np.float32)

    def route_tokens(self, layer, x, token_ids=None):
        """Router of moe_forward for every row of x: idx, wt [n][topk]."""
        x = f32(x)
        n = x.shape[0]
        tok = np.ascontiguousarray(np.zeros(n) if token_ids is None else token_ids, np.int32)
        L = make_layer_struct(layer)
        idx = np.empty((n, layer["topk"]), np.int32)
        wt = np.empty((n, layer["topk"]), np.float32)
        self.lib.orc_route_tokens(C.byref(L), _p(x, _f32p), _p(tok, _i32p), n, _p(idx, _i32p),
                                  _p(wt, _f32p))
        return idx, wt

    def moe_route_outputs(self, layer, x, token_id=0):
        """Per-route expert outputs of moe_forward before BF16 rounding:
        [topk + 1][hidden] (routes in ascending id, then the shared expert),
        with the routing."""
        L = make_layer_struct(layer)
        K, H = layer["topk"], layer["hidden"]
        routes = np.empty((K + 1, H), np.float32)
        idx = np.empty(K, np.int32)
        wt = np.empty(K, np.float32)
        self.lib.orc_moe_route_outputs(C.byref(L), _p(f32(x), _f32p), int(token_id),
                                       _p(routes, _f32p), _p(idx, _i32p), _p(wt, _f32p))
        return routes, idx, wt

    # ---- GEMVs ----
    def gemv_bf16(self, x, W, in_, out, round_out=0):
        x = f32(x)
        y = np.empty(out, np.float32)
        self.lib.orc_gemv_bf16(_p(y, _f32p), _p(x, _f32p), _p(W, _u16p), in_, out, round_out)
        return y

    def gemv_fp8_q(self, qx, qs, W, S, in_, out, round_out=1):
        y = np.empty(out, np.float32)
        self.lib.orc_gemv_fp8_q(_p(y, _f32p), _p(f32(qx), _f32p), _p(f32(qs), _f32p),
                                _p(W, _u8p), _p(S, _u8p), in_, out, round_out)
        return y

    def gemv_fp8_batch_q(self, qx, qs, W, S, in_, out, round_out=1):
        qx, qs = f32(qx), f32(qs)
        y = np.empty((qx.shape[0], out), np.float32)
        self.lib.orc_gemv_fp8_batch_q(_p(y, _f32p), _p(qx, _f32p), _p(qs, _f32p),
                                      qx.shape[0], _p(W, _u8p), _p(S, _u8p), in_, out,
                                      round_out)
        return y

    def gemv_fp8_pair_q(self, qx, qs, W0, S0, W1, S1, in_, out):
        y0, y1 = np.empty(out, np.float32), np.empty(out, np.float32)
        self.lib.orc_gemv_fp8_pair_q(_p(y0, _f32p), _p(y1, _f32p), _p(f32(qx), _f32p),
                                     _p(f32(qs), _f32p), _p(W0, _u8p), _p(S0, _u8p),
                                     _p(W1, _u8p), _p(S1, _u8p), in_, out)
        return y0, y1

    def gemv_fp4_q(self, qx, qs, W, S, in_, rows):
        y = np.empty(rows, np.float32)
        self.lib.orc_gemv_fp4_q(_p(y, _f32p), _p(f32(qx), _f32p), _p(f32(qs), _f32p),
                                _p(W, _u8p), _p(S, _u8p), in_, rows)
        return y

    def gemv_fp4_batch_q(self, qx, qs, W, S, in_, rows):
        qx, qs = f32(qx), f32(qs)
        y = np.empty((qx.shape[0], rows), np.float32)
        self.lib.orc_gemv_fp4_batch_q(_p(y, _f32p), _p(qx, _f32p), _p(qs, _f32p),
                                      qx.shape[0], _p(W, _u8p), _p(S, _u8p), in_, rows)
        return y

    def gemv_fp4_pair_q(self, qx, qs, W0, S0, W1, S1, in_, rows):
        y0, y1 = np.empty(rows, np.float32), np.empty(rows, np.float32)
        self.lib.orc_gemv_fp4_pair_q(_p(y0, _f32p), _p(y1, _f32p), _p(f32(qx), _f32p),
                                     _p(f32(qs), _f32p), _p(W0, _u8p), _p(S0, _u8p),
                                     _p(W1, _u8p), _p(S1, _u8p), in_, rows)
        return y0, y1

    def gemv_fp8_legacy(self, x, W, wscale, in_, rows, block=128):
        y = np.empty(rows, np.float32)
        self.lib.orc_gemv_fp8_legacy(_p(y, _f32p), _p(f32(x), _f32p), _p(W, _u8p),
                                     _p(f32(wscale), _f32p), in_, rows, block)
        return y

    def gemv_fp8_tbl(self, x, W, wscale, in_, rows, block=128):
        y = np.empty(rows, np.float32)
        self.lib.orc_gemv_fp8_tbl(_p(y, _f32p), _p(f32(x), _f32p), _p(W, _u8p),
                                  _p(f32(wscale), _f32p), in_, rows, block)
        return y

    def gemv_fp4_legacy(self, qx, qs, W, wscale, in_, rows, group=32):
        y = np.empty(rows, np.float32)
        self.lib.orc_gemv_fp4_legacy(_p(y, _f32p), _p(f32(qx), _f32p), _p(f32(qs), _f32p),
                                     _p(W, _u8p), _p(f32(wscale), _f32p), in_, rows, group)
        return y

    # ---- router / expert ----
    def route(self, z, bias, tid2eid_row, topk, route_scale):
        z = f32(z)
        idx = np.empty(topk, np.int32)
        wt = np.empty(topk, np.float32)
        b = None if bias is None else f32(bias)
        t = None if tid2eid_row is None else np.ascontiguousarray(tid2eid_row, np.int64)
        self.lib.orc_route(_p(idx, _i32p), _p(wt, _f32p), _p(z, _f32p), _p(b, _f32p),
                           _p(t, _i64p), z.shape[0], topk, C.c_float(route_scale))
        return idx, wt

    def router_public(self, x, gate, bias, tid2eid, token_id, hidden, n_experts,
                      topk, hash_layer, route_scale):
        idx = np.empty(topk, np.int32)
        wt = np.empty(topk, np.float32)
        b = None if bias is None else f32(bias)
        self.lib.orc_router_public(_p(idx, _i32p), _p(wt, _f32p), _p(f32(x), _f32p),
                                   _p(gate, _u16p), _p(b, _f32p), _p(tid2eid, _i64p),
                                   token_id, hidden, n_experts, topk, hash_layer,
                                   C.c_float(route_scale))
        return idx, wt

    def swiglu_quant(self, gate, up, limit, w):
        gate, up = f32(gate), f32(up)
        n = gate.shape[0]
        y, qy = np.empty(n, np.float32), np.empty(n, np.float32)
        qs = np.empty((n + 127) // 128, np.float32)
        self.lib.orc_swiglu_quant(_p(y, _f32p), _p(qy, _f32p), _p(qs, _f32p),
                                  _p(gate, _f32p), _p(up, _f32p), n, int(limit),
                                  C.c_float(w))
        return y, qy, qs

    def expert_forward(self, qx, qs, scales, weights, hidden, inter, limit, w):
        out = np.empty(hidden, np.float32)
        self.lib.orc_expert_forward(_p(out, _f32p), _p(f32(qx), _f32p), _p(f32(qs), _f32p),
                                    _p(scales, _u8p), _p(weights, _u8p), hidden, inter,
                                    int(limit), C.c_float(w))
        return out

    def shared_expert_forward(self, qx, qs, sh, hidden, inter, limit):
        out = np.empty(hidden, np.float32)
        self.lib.orc_shared_expert_forward(
            _p(out, _f32p), _p(f32(qx), _f32p), _p(f32(qs), _f32p),
            _p(sh["sh1"], _u8p), _p(sh["sh1_s"], _u8p), _p(sh["sh3"], _u8p),
            _p(sh["sh3_s"], _u8p), _p(sh["sh2"], _u8p), _p(sh["sh2_s"], _u8p),
            hidden, inter, int(limit))
        return out

    def moe_forward(self, layer, x, token_id=0):
        L = make_layer_struct(layer)
        out = np.empty(layer["hidden"], np.float32)
        idx = np.empty(layer["topk"], np.int32)
        wt = np.empty(layer["topk"], np.float32)
        self.lib.orc_moe_forward(C.byref(L), _p(f32(x), _f32p), token_id, _p(out, _f32p),
                                 _p(idx, _i32p), _p(wt, _f32p))
        return out, idx, wt

    def moe_forward_batch(self, layer, x, token_ids=None):
        x = f32(x)
        n = x.shape[0]
        tok = np.ascontiguousarray(np.zeros(n) if token_ids is None else token_ids, np.int32)
        L = make_layer_struct(layer)
        out = np.empty_like(x)
        idx = np.empty((n, layer["topk"]), np.int32)
        wt = np.empty((n, layer["topk"]), np.float32)
        self.lib.orc_moe_forward_batch(C.byref(L), _p(x, _f32p), _p(tok, _i32p), n,
                                       _p(out, _f32p), _p(idx, _i32p), _p(wt, _f32p))
        return out, idx, wt

    # ---- synthetic weights ----
    def quant_fp4_rows(self, w):
        w = f32(w)
        rows, cols = w.shape
        packed = np.empty((rows, (cols + 1) // 2), np.uint8)
        scales = np.empty((rows, (cols + 31) // 32), np.uint8)
        self.lib.orc_quant_fp4_rows(_p(packed, _u8p), _p(scales, _u8p), _p(w, _f32p), rows, cols)
        return packed, scales

    def quant_fp8_blocks_e8m0(self, w):
        w = f32(w)
        rows, cols = w.shape
        codes = np.empty((rows, cols), np.uint8)
        scales = np.empty(((rows + 127) // 128, (cols + 127) // 128), np.uint8)
        self.lib.orc_quant_fp8_blocks_e8m0(_p(codes, _u8p), _p(scales, _u8p), _p(w, _f32p),
                                           rows, cols)
        return codes, scales

    def quant_fp8_blocks_absmax(self, w):
        w = f32(w)
        rows, cols = w.shape
        codes = np.empty((rows, cols), np.uint8)
        scales = np.empty(((rows + 127) // 128, (cols + 127) // 128), np.float32)
        self.lib.orc_quant_fp8_blocks_absmax(_p(codes, _u8p), _p(scales, _f32p),
                                             _p(w, _f32p), rows, cols)
        return codes, scales


class RefLib(_Base):
    """The reference engine compiled from its sources (oracle/_ref)."""

    _STEP = {"rmsnorm": "ref_shim_rmsnorm_bf16", "split": "dsv4_hc_split",
             "pre": "ref_shim_hc_pre", "post": "ref_shim_hc_post"}

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle` where the reference is mounted")
        lib = self.lib = C.CDLL(path)
        for name, res in [("dsv4_fp8_e4m3", C.c_float), ("dsv4_e8m0", C.c_float),
                          ("dsv4_round_e4m3", C.c_float), ("dsv4_f32_to_bf16", C.c_uint16),
                          ("ref_shim_sqrt_softplus", C.c_float)]:
            getattr(lib, name).restype = res
        lib.dsv4_fp8_e4m3.argtypes = [C.c_uint8]
        lib.dsv4_e8m0.argtypes = [C.c_uint8]
        lib.dsv4_round_e4m3.argtypes = [C.c_float]
        lib.dsv4_f32_to_bf16.argtypes = [C.c_float]
        lib.ref_shim_sqrt_softplus.argtypes = [C.c_float]
        self._fp8, self._e8m0 = lib.dsv4_fp8_e4m3, lib.dsv4_e8m0
        self._bf16, self._rnd = lib.dsv4_f32_to_bf16, lib.dsv4_round_e4m3
        self._quant = lib.dsv4_quant_fp8_codes

    def quant_fp8_act_public(self, x):
        x = f32(x)
        n = x.shape[0]
        qx = np.empty_like(x)
        qs = np.empty((n + 127) // 128, np.float32)
        self.lib.dsv4_quant_fp8_act(_p(qx, _f32p), _p(qs, _f32p), _p(x, _f32p), n)
        return qx, qs

    def sqrt_softplus(self, z):
        return np.array([self.lib.ref_shim_sqrt_softplus(float(v)) for v in f32(z).ravel()],
                        dtype=np.float32)

    @staticmethod
    def _ptrs(rows):
        arr = (_f32p * len(rows))(*[_p(r, _f32p) for r in rows])
        return arr

    def gemv_bf16(self, x, W, in_, out, round_out=0):
        y = np.empty(out, np.float32)
        self.lib.dsv4_gemv_bf16(_p(y, _f32p), _p(f32(x), _f32p), _p(W, _u16p), in_, out,
                                round_out)
        return y

    def head_logits(self, h, W, threads):
        """head_logits (1 token) / head_logits_batch (more) of the reference
        engine on BF16 head rows W [vocab][hid]: fp32 logits [n][vocab]."""
        h = f32(np.atleast_2d(h))
        n, hid = h.shape
        vocab = W.shape[0]
        y = np.empty((n, vocab), np.float32)
        self.lib.ref_shim_head_logits(_p(y, _f32p), _p(h, _f32p), _p(W, _u16p), hid, vocab, n,
                                      int(threads))
        return y

    def gemv_fp8_q(self, qx, qs, W, S, in_, out, round_out=1):
        y = np.empty(out, np.float32)
        self.lib.dsv4_gemv_fp8_q(_p(y, _f32p), _p(f32(qx), _f32p), _p(f32(qs), _f32p),
                                 _p(W, _u8p), _p(S, _u8p), in_, out, round_out)
        return y

    def gemv_fp8_batch_q(self, qx, qs, W, S, in_, out, round_out=1):
        qx, qs = f32(qx), f32(qs)
        y = np.empty((qx.shape[0], out), np.float32)
        self.lib.dsv4_gemv_fp8_batch_q(self._ptrs(list(y)), self._ptrs(list(qx)),
                                       self._ptrs(list(qs)), qx.shape[0], _p(W, _u8p),
                                       _p(S, _u8p), in_, out, round_out)
        return y

    def gemv_fp8_pair_q(self, qx, qs, W0, S0, W1, S1, in_, out):
        y0, y1 = np.empty(out, np.float32), np.empty(out, np.float32)
        self.lib.dsv4_gemv_fp8_pair_q(_p(y0, _f32p), _p(y1, _f32p), _p(f32(qx), _f32p),
                                      _p(f32(qs), _f32p), _p(W0, _u8p), _p(S0, _u8p),
                                      _p(W1, _u8p), _p(S1, _u8p), in_, out)
        return y0, y1

    def gemv_fp4_q(self, qx, qs, W, S, in_, rows):
        y = np.empty(rows, np.float32)
        self.lib.dsv4_gemv_fp4_q(_p(y, _f32p), _p(f32(qx), _f32p), _p(f32(qs), _f32p),
                                 _p(W, _u8p), _p(S, _u8p), in_, rows)
        return y

    def gemv_fp4_batch_q(self, qx, qs, W, S, in_, rows):
        qx, qs = f32(qx), f32(qs)
        y = np.empty((qx.shape[0], rows), np.float32)
        self.lib.dsv4_gemv_fp4_batch_q(self._ptrs(list(y)), self._ptrs(list(qx)),
                                       self._ptrs(list(qs)), qx.shape[0], _p(W, _u8p),
                                       _p(S, _u8p), in_, rows)
        return y

    def gemv_fp4_pair_q(self, qx, qs, W0, S0, W1, S1, in_, rows):
        y0, y1 = np.empty(rows, np.float32), np.empty(rows, np.float32)
        self.lib.dsv4_gemv_fp4_pair_q(_p(y0, _f32p), _p(y1, _f32p), _p(f32(qx), _f32p),
                                      _p(f32(qs), _f32p), _p(W0, _u8p), _p(S0, _u8p),
                                      _p(W1, _u8p), _p(S1, _u8p), in_, rows)
        return y0, y1

    def gemv_fp8_legacy(self, x, W, wscale, in_, rows, block=128):
        y = np.empty(rows, np.float32)
        self.lib.dsv4_gemv_fp8(_p(y, _f32p), _p(f32(x), _f32p), _p(W, _u8p),
                               _p(f32(wscale), _f32p), in_, rows, block)
        return y

    def gemv_fp8_tbl(self, x, W, wscale, in_, rows, block=128):
        y = np.empty(rows, np.float32)
        self.lib.dsv4_gemv_fp8_tbl(_p(y, _f32p), _p(f32(x), _f32p), _p(W, _u8p),
                                   _p(f32(wscale), _f32p), in_, rows, block)
        return y

    def gemv_fp4_legacy(self, qx, qs, W, wscale, in_, rows, group=32):
        y = np.empty(rows, np.float32)
        self.lib.dsv4_gemv_fp4(_p(y, _f32p), _p(f32(qx), _f32p), _p(f32(qs), _f32p),
                               _p(W, _u8p), _p(f32(wscale), _f32p), in_, rows, group)
        return y

    def router_public(self, x, gate, bias, tid2eid, token_id, hidden, n_experts,
                      topk, hash_layer, route_scale):
        idx = np.empty(topk, np.int32)
        wt = np.empty(topk, np.float32)
        b = None if bias is None else f32(bias)
        self.lib.dsv4_router(_p(idx, _i32p), _p(wt, _f32p), _p(f32(x), _f32p),
                             _p(gate, _u16p), _p(b, _f32p), _p(tid2eid, _i64p),
                             token_id, hidden, n_experts, topk, hash_layer,
                             C.c_float(route_scale), C.c_float(1e-6))
        return idx, wt

    def swiglu_quant(self, gate, up, limit, w):
        gate, up = f32(gate), f32(up)
        n = gate.shape[0]
        y, qy = np.empty(n, np.float32), np.empty(n, np.float32)
        qs = np.empty((n + 127) // 128, np.float32)
        self.lib.ref_shim_routed_swiglu_quant(_p(y, _f32p), _p(qy, _f32p), _p(qs, _f32p),
                                              _p(gate, _f32p), _p(up, _f32p), n, int(limit),
                                              C.c_float(w))
        return y, qy, qs

    def expert_forward(self, qx, qs, scales, weights, hidden, inter, limit, w):
        out = np.empty(hidden, np.float32)
        self.lib.ref_shim_expert_forward(_p(out, _f32p), _p(f32(qx), _f32p),
                                         _p(f32(qs), _f32p), _p(scales, _u8p),
                                         _p(weights, _u8p), hidden, inter, int(limit),
                                         C.c_float(w))
        return out

    def shared_expert_forward(self, qx, qs, sh, hidden, inter, limit):
        out = np.empty(hidden, np.float32)
        self.lib.ref_shim_shared_expert_forward(
            _p(out, _f32p), _p(f32(qx), _f32p), _p(f32(qs), _f32p),
            _p(sh["sh1"], _u8p), _p(sh["sh1_s"], _u8p), _p(sh["sh3"], _u8p),
            _p(sh["sh3_s"], _u8p), _p(sh["sh2"], _u8p), _p(sh["sh2_s"], _u8p),
            hidden, inter, int(limit))
        return out

    def moe_forward(self, layer, x, token_id=0):
        L = make_layer_struct(layer)
        out = np.empty(layer["hidden"], np.float32)
        idx = np.empty(layer["topk"], np.int32)
        wt = np.empty(layer["topk"], np.float32)
        self.lib.ref_shim_moe_forward(C.byref(L), _p(f32(x), _f32p), token_id,
                                      _p(out, _f32p), _p(idx, _i32p), _p(wt, _f32p))
        return out, idx, wt

    def moe_forward_batch(self, layer, x, token_ids=None):
        x = f32(x)
        n = x.shape[0]
        tok = np.ascontiguousarray(np.zeros(n) if token_ids is None else token_ids, np.int32)
        L = make_layer_struct(layer)
        out = np.empty_like(x)
        self.lib.ref_shim_moe_forward_batch(C.byref(L), _p(x, _f32p), _p(tok, _i32p), n,
                                            _p(out, _f32p))
        return out


class StTensor(C.Structure):
    """Tensor record of a safetensors index: the reference's K3Tensor
    (src/io/k3_st.h:37-45) and DSV4GTensor share this layout."""

    _fields_ = [("name", C.c_char_p), ("shard", C.c_int), ("dtype", C.c_int),
                ("ndim", C.c_int), ("shape", C.c_int64 * 4), ("off", C.c_int64),
                ("nbytes", C.c_int64)]

    def as_dict(self):
        return dict(name=self.name.decode("latin-1"), shard=self.shard, dtype=self.dtype,
                    shape=tuple(self.shape[:self.ndim]), off=self.off, nbytes=self.nbytes)


class RefSt:
    """The reference reader k3_st (compiled in oracle/_ref) over one checkpoint
    directory: open, iterate, find, read, read_f32."""

    def __init__(self, ref: "RefLib", directory: str):
        lib = self.lib = ref.lib
        lib.ref_shim_st_open.restype = C.c_void_p
        lib.ref_shim_st_open.argtypes = [C.c_char_p]
        lib.ref_shim_st_close.argtypes = [C.c_void_p]
        lib.ref_shim_st_count.argtypes = [C.c_void_p]
        lib.ref_shim_st_nshard.argtypes = [C.c_void_p]
        lib.ref_shim_st_tensor.restype = C.POINTER(StTensor)
        lib.ref_shim_st_tensor.argtypes = [C.c_void_p, C.c_int]
        lib.k3_st_find.restype = C.POINTER(StTensor)
        lib.k3_st_find.argtypes = [C.c_void_p, C.c_char_p]
        lib.k3_st_read.restype = C.c_int64
        lib.k3_st_read.argtypes = [C.c_void_p, C.POINTER(StTensor), C.c_void_p]
        lib.k3_st_read_f32.restype = C.c_int64
        lib.k3_st_read_f32.argtypes = [C.c_void_p, C.POINTER(StTensor), C.c_void_p]
        self.h = lib.ref_shim_st_open(directory.encode())
        self.ok = bool(self.h)

    def close(self):
        if self.h:
            self.lib.ref_shim_st_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def nshard(self):
        return self.lib.ref_shim_st_nshard(self.h)

    def tensors(self):
        return [self.lib.ref_shim_st_tensor(self.h, i).contents.as_dict()
                for i in range(self.lib.ref_shim_st_count(self.h))]

    def find(self, name: str):
        t = self.lib.k3_st_find(self.h, name.encode("latin-1"))
        return t.contents.as_dict() if t else None

    def read(self, name: str) -> bytes:
        t = self.lib.k3_st_find(self.h, name.encode("latin-1"))
        buf = C.create_string_buffer(max(t.contents.nbytes, 1))
        got = self.lib.k3_st_read(self.h, t, buf)
        return buf.raw[:got]

    def read_f32(self, name: str):
        t = self.lib.k3_st_find(self.h, name.encode("latin-1"))
        n = 1
        for d in t.contents.shape[:t.contents.ndim]:
            n *= d
        out = np.zeros(max(n, 1), np.float32)
        got = self.lib.k3_st_read_f32(self.h, t, out.ctypes.data_as(C.c_void_p))
        return out[:got]


def ref_available() -> bool:
    return os.path.exists(REF_SO)
