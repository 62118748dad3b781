"""ctypes binding of libdsv4_gpu.so (include/dsv4_gpu.h) for Python callers.

Device buffers are torch tensors on a ROCm device (torch only allocates and
orders streams; all compute runs in the library's HIP kernels). Every wrapper
launches on torch's current stream and raises RuntimeError with the
library's message on failure. If the library is missing the import fails
loudly: there is no fallback.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB_PATH = os.path.join(PKG, "lib", "libdsv4_gpu.so")
DECODE_PHASES = 3  # DSV4G_DECODE_PHASES: ordered launches of one decode layer

_vp = C.c_void_p


class DSV4GLayer(C.Structure):
    """Mirror of DSV4GLayer (include/dsv4_gpu.h)."""

    _fields_ = [
        ("hidden", C.c_int), ("inter", C.c_int), ("n_experts", C.c_int), ("topk", C.c_int),
        ("route_scale", C.c_float), ("swiglu_limit", C.c_float),
        ("gate_w", _vp), ("bias", _vp), ("tid2eid", _vp), ("experts", _vp),
        ("expert_stride", C.c_size_t), ("scale_run", C.c_size_t),
        ("sh1", _vp), ("sh1_s", _vp), ("sh3", _vp), ("sh3_s", _vp),
        ("sh2", _vp), ("sh2_s", _vp),
    ]


# (name, argtypes) for the device-pointer ABI; all return int.
_I, _F, _Z = C.c_int, C.c_float, C.c_size_t
_SIGS = {
    "dsv4g_quant_fp8_act": [_vp, _vp, _vp, _I, _I, _vp],
    "dsv4g_dequant_fp4": [_vp, _vp, _vp, _I, _I, _vp],
    "dsv4g_dequant_fp8": [_vp, _vp, _vp, _I, _I, _vp],
    "dsv4g_gemv_fp4_q": [_vp, _vp, _vp, _vp, _vp, _I, _I, _vp],
    "dsv4g_gemv_fp4_pair_q": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _I, _I, _vp],
    "dsv4g_gemv_fp4_batch_q": [_vp, _vp, _vp, _I, _vp, _vp, _I, _I, _vp],
    "dsv4g_gemv_fp8_q": [_vp, _vp, _vp, _vp, _vp, _I, _I, _I, _vp],
    "dsv4g_gemv_fp8_pair_q": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _I, _I, _vp],
    "dsv4g_gemv_fp8_batch_q": [_vp, _vp, _vp, _I, _vp, _vp, _I, _I, _I, _vp],
    "dsv4g_gemv_bf16": [_vp, _vp, _vp, _I, _I, _I, _I, _vp],
    "dsv4g_gemv_fp8_float": [_vp, _vp, _vp, _vp, _I, _I, _I, _I, _vp],
    "dsv4g_gemv_fp4_float": [_vp, _vp, _vp, _vp, _vp, _I, _I, _I, _vp],
    "dsv4g_router": [_vp, _vp, _vp, C.POINTER(DSV4GLayer), _vp, _I, _vp, _vp, _vp],
    "dsv4g_router_public": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _I, _I, _I, _I, _F, _vp, _vp,
                            _vp],
    "dsv4g_swiglu_quant": [_vp, _vp, _vp, _vp, _I, _I, _I, _F, _vp],
    "dsv4g_argmax": [_vp, _vp, _I, _I, C.c_size_t, _vp],
    "dsv4g_expert_forward": [_vp, _vp, _vp, _vp, C.c_size_t, _I, _I, _F, _vp, _vp, C.c_size_t,
                             _vp],
    "dsv4g_moe_forward": [_vp, _vp, C.POINTER(DSV4GLayer), _vp, _I, _vp, _Z, _vp, _vp, _vp],
    "dsv4g_moe_forward_fast": [_vp, _vp, C.POINTER(DSV4GLayer), _vp, _I, _vp, _Z, _vp, _vp, _vp],
    "dsv4g_moe_decode_phase": [_I, _vp, _vp, C.POINTER(DSV4GLayer), _vp, _I, _vp, _Z, _vp],
    "dsv4g_moe_decode_routing": [_vp, _vp, C.POINTER(DSV4GLayer), _I, _vp, _vp],
    "dsv4g_moe_workspace_init": [_vp, _Z, _vp],
    "dsv4g_moe_decode_status": [_vp, _vp, _vp],
    "dsv4g_moe_noalloc_status": [_vp, _vp],
    "dsv4g_moe_forward_routes": [_vp, _vp, C.POINTER(DSV4GLayer), _vp, _I, _vp, _Z, _vp, _vp,
                                 _vp, _I, _vp],
    "dsv4g_moe_forward_batch": [_vp, _vp, C.POINTER(DSV4GLayer), _vp, _I, _vp, _Z, _vp, _vp,
                                _vp],
    "dsv4g_moe_forward_batch_routes": [_vp, _vp, C.POINTER(DSV4GLayer), _vp, _I, _vp, _Z, _vp,
                                       _vp, _vp, _vp],
    "dsv4g_quant_fp4_rows": [_vp, _vp, _vp, _I, _I, _vp],
    "dsv4g_quant_fp8_blocks": [_vp, _vp, _vp, _I, _I, _I, _vp],
    "dsv4g_rmsnorm_bf16": [_vp, _vp, _vp, _I, _F, _I, _I, _vp],
    "dsv4g_hc_split": [_vp, _vp, _vp, _vp, _vp, _vp, _I, _I, _F, _I, _vp],
    "dsv4g_hc_pre": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _I, _I, _I, _F, _F, _I, _vp, _vp],
    "dsv4g_hc_post": [_vp, _vp, _vp, _vp, _I, _I, _I, _vp],
    "dsv4g_ffn_step": [_vp, _vp, _vp, _vp, _vp, C.POINTER(DSV4GLayer), _vp, _I, _I, _I, _F, _F,
                       _vp, _Z, _vp, _vp, _vp],
}


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


class GpuLib:
    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build it with `make -C "
                               f"deepseek-v4-flash-0731-in-c_amd` (or __graft_entry__.build())")
        self.path = path
        lib = self.lib = C.CDLL(path)
        lib.dsv4g_last_error.restype = C.c_char_p
        lib.dsv4g_version.restype = C.c_char_p
        lib.dsv4g_moe_workspace_bytes.restype = C.c_size_t
        lib.dsv4g_moe_workspace_bytes.argtypes = [C.POINTER(DSV4GLayer), _I]
        lib.dsv4g_moe_batch_workspace_bytes.restype = C.c_size_t
        lib.dsv4g_moe_batch_workspace_bytes.argtypes = [C.POINTER(DSV4GLayer), _I]
        lib.dsv4g_ffn_step_workspace_bytes.restype = C.c_size_t
        lib.dsv4g_ffn_step_workspace_bytes.argtypes = [C.POINTER(DSV4GLayer), _I, _I]
        for name, args in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = C.c_int
        _st_sigs(lib)

    # ---- plumbing
    def _call(self, name, *args):
        rc = getattr(self.lib, name)(*args)
        if rc != 0:
            raise RuntimeError(f"{name}: {self.lib.dsv4g_last_error().decode()}")

    @staticmethod
    def _stream():
        import torch
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)

    # ---- kernels (torch tensors in, torch tensors out)
    def quant_fp8_act(self, x):
        import torch
        n = x.shape[-1]
        nvec = x.numel() // n
        qx = torch.empty_like(x)
        qs = torch.empty(x.shape[:-1] + ((n + 127) // 128,), dtype=torch.float32, device=x.device)
        self._call("dsv4g_quant_fp8_act", _ptr(qx), _ptr(qs), _ptr(x), n, nvec, self._stream())
        return qx, qs

    def dequant_fp4(self, W, S, rows, cols):
        import torch
        out = torch.empty(rows, cols, dtype=torch.float32, device=W.device)
        self._call("dsv4g_dequant_fp4", _ptr(out), _ptr(W), _ptr(S), rows, cols, self._stream())
        return out

    def dequant_fp8(self, W, S, rows, cols):
        import torch
        out = torch.empty(rows, cols, dtype=torch.float32, device=W.device)
        self._call("dsv4g_dequant_fp8", _ptr(out), _ptr(W), _ptr(S), rows, cols, self._stream())
        return out

    def gemv_fp4_q(self, qx, qs, W, S, in_, rows, y=None):
        import torch
        y = torch.empty(rows, dtype=torch.float32, device=qx.device) if y is None else y
        self._call("dsv4g_gemv_fp4_q", _ptr(y), _ptr(qx), _ptr(qs), _ptr(W), _ptr(S), in_, rows,
                   self._stream())
        return y

    def gemv_fp4_pair_q(self, qx, qs, W0, S0, W1, S1, in_, rows):
        import torch
        y0 = torch.empty(rows, dtype=torch.float32, device=qx.device)
        y1 = torch.empty_like(y0)
        self._call("dsv4g_gemv_fp4_pair_q", _ptr(y0), _ptr(y1), _ptr(qx), _ptr(qs), _ptr(W0),
                   _ptr(S0), _ptr(W1), _ptr(S1), in_, rows, self._stream())
        return y0, y1

    def gemv_fp4_batch_q(self, qx, qs, W, S, in_, rows):
        import torch
        b = qx.shape[0]
        y = torch.empty(b, rows, dtype=torch.float32, device=qx.device)
        self._call("dsv4g_gemv_fp4_batch_q", _ptr(y), _ptr(qx), _ptr(qs), b, _ptr(W), _ptr(S),
                   in_, rows, self._stream())
        return y

    def gemv_fp8_q(self, qx, qs, W, S, in_, out, round_out=1, y=None):
        import torch
        y = torch.empty(out, dtype=torch.float32, device=qx.device) if y is None else y
        self._call("dsv4g_gemv_fp8_q", _ptr(y), _ptr(qx), _ptr(qs), _ptr(W), _ptr(S), in_, out,
                   round_out, self._stream())
        return y

    def gemv_fp8_pair_q(self, qx, qs, W0, S0, W1, S1, in_, out):
        import torch
        y0 = torch.empty(out, dtype=torch.float32, device=qx.device)
        y1 = torch.empty_like(y0)
        self._call("dsv4g_gemv_fp8_pair_q", _ptr(y0), _ptr(y1), _ptr(qx), _ptr(qs), _ptr(W0),
                   _ptr(S0), _ptr(W1), _ptr(S1), in_, out, self._stream())
        return y0, y1

    def gemv_fp8_batch_q(self, qx, qs, W, S, in_, out, round_out=1):
        import torch
        b = qx.shape[0]
        y = torch.empty(b, out, dtype=torch.float32, device=qx.device)
        self._call("dsv4g_gemv_fp8_batch_q", _ptr(y), _ptr(qx), _ptr(qs), b, _ptr(W), _ptr(S),
                   in_, out, round_out, self._stream())
        return y

    def gemv_bf16(self, x, W, in_, out, round_out=0):
        import torch
        b = x.numel() // in_
        y = torch.empty(b, out, dtype=torch.float32, device=x.device)
        self._call("dsv4g_gemv_bf16", _ptr(y), _ptr(x), _ptr(W), in_, out, round_out, b,
                   self._stream())
        return y

    def gemv_bf16_into(self, y, x, W, in_, out, round_out=0):
        """dsv4g_gemv_bf16 into a caller's y [batch][out] (no allocation)."""
        self._call("dsv4g_gemv_bf16", _ptr(y), _ptr(x), _ptr(W), in_, out, round_out,
                   x.numel() // in_, self._stream())
        return y

    def argmax(self, logits, idx=None):
        """dsv4g_argmax over the rows of logits [n][vocab] (int32 [n])."""
        import torch
        n, vocab = (1, logits.shape[0]) if logits.dim() == 1 else logits.shape
        idx = torch.empty(n, dtype=torch.int32, device=logits.device) if idx is None else idx
        self._call("dsv4g_argmax", _ptr(idx), _ptr(logits), vocab, n, vocab, self._stream())
        return idx

    def expert_workspace_bytes(self, inter):
        self.lib.dsv4g_expert_workspace_bytes.restype = C.c_size_t
        self.lib.dsv4g_expert_workspace_bytes.argtypes = [_I]
        return int(self.lib.dsv4g_expert_workspace_bytes(inter))

    def expert_forward(self, out, qx, qs, slot, scale_run, hidden, inter, limit, weight=None,
                       workspace=None):
        """dsv4g_expert_forward: out [hidden] from one expert slot (uint8, the
        checkpoint layout) at one token."""
        import torch
        need = self.expert_workspace_bytes(inter)
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=qx.device)
        self._call("dsv4g_expert_forward", _ptr(out), _ptr(qx), _ptr(qs), _ptr(slot),
                   int(scale_run), hidden, inter, float(limit), _ptr(weight), _ptr(workspace),
                   workspace.numel(), self._stream())
        return out

    def gemv_fp8_float(self, x, W, wscale, in_, rows, block=128, mode=0, y=None):
        import torch
        y = torch.empty(rows, dtype=torch.float32, device=x.device) if y is None else y
        self._call("dsv4g_gemv_fp8_float", _ptr(y), _ptr(x), _ptr(W), _ptr(wscale), in_, rows,
                   block, mode, self._stream())
        return y

    def gemv_fp4_float(self, qx, qs, W, wscale, in_, rows, group=32):
        import torch
        y = torch.empty(rows, dtype=torch.float32, device=qx.device)
        self._call("dsv4g_gemv_fp4_float", _ptr(y), _ptr(qx), _ptr(qs), _ptr(W), _ptr(wscale),
                   in_, rows, group, self._stream())
        return y

    def router(self, layer, x, token_ids=None):
        import torch
        L = layer.struct
        n = x.shape[0]
        idx = torch.empty(n, L.topk, dtype=torch.int32, device=x.device)
        wt = torch.empty(n, L.topk, dtype=torch.float32, device=x.device)
        ws = torch.empty(2, n, L.n_experts, dtype=torch.float32, device=x.device)
        self._call("dsv4g_router", _ptr(idx), _ptr(wt), _ptr(x), C.byref(L), _ptr(token_ids), n,
                   _ptr(ws[0]), _ptr(ws[1]), self._stream())
        return idx, wt

    def router_public(self, x, gate, bias, t2e_row, hidden, n_experts, topk, hash_layer,
                      route_scale):
        import torch
        idx = torch.empty(topk, dtype=torch.int32, device=x.device)
        wt = torch.empty(topk, dtype=torch.float32, device=x.device)
        ws = torch.empty(2, n_experts, dtype=torch.float32, device=x.device)
        tok = torch.zeros(1, dtype=torch.int32, device=x.device)
        self._call("dsv4g_router_public", _ptr(idx), _ptr(wt), _ptr(x), _ptr(gate), _ptr(bias),
                   _ptr(t2e_row), _ptr(tok), hidden, n_experts, topk, int(hash_layer),
                   C.c_float(route_scale), _ptr(ws[0]), _ptr(ws[1]), self._stream())
        return idx, wt

    def swiglu_quant(self, gate_up, inter, limit, wt=None, K=0):
        import torch
        n_slots = gate_up.numel() // (2 * inter)
        qy = torch.empty(n_slots, inter, dtype=torch.float32, device=gate_up.device)
        qs = torch.empty(n_slots, inter // 128, dtype=torch.float32, device=gate_up.device)
        self._call("dsv4g_swiglu_quant", _ptr(qy), _ptr(qs), _ptr(gate_up), _ptr(wt), K, n_slots,
                   inter, C.c_float(limit), self._stream())
        return qy, qs

    def moe_workspace_bytes(self, layer, n_tokens):
        return int(self.lib.dsv4g_moe_workspace_bytes(C.byref(layer.struct), n_tokens))

    def moe_forward(self, layer, x, token_ids=None, workspace=None, out=None, fast=False,
                    route_out=None, check=True):
        """dsv4g_moe_forward(_fast); with route_out ([n][topk+1][hidden] fp32)
        dsv4g_moe_forward_routes. check: read the workspace status after the
        call (synchronises) and raise if a cross-workgroup wait ran out."""
        import torch
        n = x.shape[0]
        L = layer.struct
        need = self.moe_workspace_bytes(layer, n)
        if workspace is None or workspace.numel() < need:
            workspace = self.new_moe_workspace(layer, n, x.device)
        out = torch.empty_like(x) if out is None else out
        idx = torch.empty(n, L.topk, dtype=torch.int32, device=x.device)
        wt = torch.empty(n, L.topk, dtype=torch.float32, device=x.device)
        if route_out is not None:
            self._call("dsv4g_moe_forward_routes", _ptr(out), _ptr(x), C.byref(L),
                       _ptr(token_ids), n, _ptr(workspace), workspace.numel(), _ptr(idx),
                       _ptr(wt), _ptr(route_out), 1 if fast else 0, self._stream())
        else:
            self._call("dsv4g_moe_forward_fast" if fast else "dsv4g_moe_forward", _ptr(out),
                       _ptr(x), C.byref(L), _ptr(token_ids), n, _ptr(workspace),
                       workspace.numel(), _ptr(idx), _ptr(wt), self._stream())
        if check:
            self.check_decode_status(workspace)
        return out, idx, wt

    def decode_status(self, workspace):
        """The decode workspace's sticky status word (0: fine), cleared."""
        st = C.c_uint(0)
        self._call("dsv4g_moe_decode_status", C.byref(st), _ptr(workspace), self._stream())
        return st.value

    def check_decode_status(self, workspace):
        """Raise if a cross-workgroup wait of the calls on this workspace ran
        out; the workspace is zeroed again first (that call's records and
        flags may be left set), so it serves the next call."""
        s = self.decode_status(workspace)
        if s:
            self.moe_workspace_init(workspace)
            raise RuntimeError(f"decode: a cross-workgroup wait ran out (status {s:#x})")

    def noalloc_status(self):
        """Status word of dsv4g_moe_forward_noalloc's device array (0: fine);
        a nonzero status also clears the array."""
        st = C.c_uint(0)
        self._call("dsv4g_moe_noalloc_status", C.byref(st), self._stream())
        return st.value

    def moe_workspace_init(self, workspace):
        """Zero a decode workspace, once, before its first dsv4g_moe_forward."""
        self._call("dsv4g_moe_workspace_init", _ptr(workspace), workspace.numel(), self._stream())

    def moe_forward_into(self, layer, x, out, workspace, token_ids=None, fast=False):
        """dsv4g_moe_forward(_fast) into out with a prepared workspace, routing
        not copied out: the form a captured decode loop uses."""
        self._call("dsv4g_moe_forward_fast" if fast else "dsv4g_moe_forward", _ptr(out), _ptr(x),
                   C.byref(layer.struct),
                   _ptr(token_ids), x.shape[0], _ptr(workspace), workspace.numel(), None, None,
                   self._stream())

    def new_moe_workspace(self, layer, n_tokens, device):
        """A decode workspace, zeroed as dsv4g_moe_forward requires before its
        first use (every call leaves it reusable)."""
        import torch
        ws = torch.empty(self.moe_workspace_bytes(layer, n_tokens), dtype=torch.uint8,
                         device=device)
        self._call("dsv4g_moe_workspace_init", _ptr(ws), ws.numel(), self._stream())
        return ws

    def moe_batch_workspace_bytes(self, layer, n_tokens):
        return int(self.lib.dsv4g_moe_batch_workspace_bytes(C.byref(layer.struct), n_tokens))

    def moe_forward_batch(self, layer, x, token_ids=None, workspace=None, out=None,
                          route_out=None):
        """dsv4g_moe_forward_batch; with route_out ([n][topk+1][hidden] fp32)
        dsv4g_moe_forward_batch_routes, which also writes the per-route
        outputs before their BF16 rounding."""
        import torch
        n = x.shape[0]
        L = layer.struct
        need = self.moe_batch_workspace_bytes(layer, n)
        if workspace is None or workspace.numel() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
        out = torch.empty_like(x) if out is None else out
        idx = torch.empty(n, L.topk, dtype=torch.int32, device=x.device)
        wt = torch.empty(n, L.topk, dtype=torch.float32, device=x.device)
        if route_out is None:
            self._call("dsv4g_moe_forward_batch", _ptr(out), _ptr(x), C.byref(L),
                       _ptr(token_ids), n, _ptr(workspace), workspace.numel(), _ptr(idx),
                       _ptr(wt), self._stream())
        else:
            self._call("dsv4g_moe_forward_batch_routes", _ptr(out), _ptr(x), C.byref(L),
                       _ptr(token_ids), n, _ptr(workspace), workspace.numel(), _ptr(idx),
                       _ptr(wt), _ptr(route_out), self._stream())
        return out, idx, wt

    def moe_decode_phase(self, phase, layer, x, out, workspace, token_ids=None):
        self._call("dsv4g_moe_decode_phase", phase, _ptr(out), _ptr(x), C.byref(layer.struct),
                   _ptr(token_ids), x.shape[0], _ptr(workspace), workspace.numel(),
                   self._stream())

    def quant_fp4_rows(self, w, packed, scales):
        rows, cols = w.shape
        self._call("dsv4g_quant_fp4_rows", _ptr(packed), _ptr(scales), _ptr(w), rows, cols,
                   self._stream())

    def quant_fp8_blocks(self, w, codes, scales, mode=0):
        rows, cols = w.shape
        self._call("dsv4g_quant_fp8_blocks", _ptr(codes), _ptr(scales), _ptr(w), rows, cols,
                   mode, self._stream())


    # ---- caller step around the MoE (RMSNorm, Hyper-Connections)
    def rmsnorm_bf16(self, x, w=None, eps=1e-6, round_out=1, out=None):
        """Rows of x [rows][n] (w: BF16 gain bits as int16/uint16 tensor)."""
        import torch
        rows, n = x.shape
        out = torch.empty_like(x) if out is None else out
        self._call("dsv4g_rmsnorm_bf16", _ptr(out), _ptr(x), _ptr(w), n, C.c_float(eps),
                   round_out, rows, self._stream())
        return out

    def hc_split(self, mixes, scale3, base, mult, iters=20, eps=1e-6):
        import torch
        n = mixes.shape[0]
        f = dict(dtype=torch.float32, device=mixes.device)
        pre, post = torch.empty(n, mult, **f), torch.empty(n, mult, **f)
        comb = torch.empty(n, mult * mult, **f)
        self._call("dsv4g_hc_split", _ptr(pre), _ptr(post), _ptr(comb), _ptr(mixes),
                   _ptr(scale3), _ptr(base), mult, iters, C.c_float(eps), n, self._stream())
        return pre, post, comb

    def hc_pre(self, state, fn, scale3, base, mult, norm_w=None, iters=20, rms_eps=1e-6,
               hc_eps=1e-6, status=None):
        """state [n][mult*hid] -> bin [n][hid] (RMSNormed with norm_w),
        post [n][mult], comb [n][mult*mult]."""
        import torch
        n, K = state.shape
        hid = K // mult
        f = dict(dtype=torch.float32, device=state.device)
        bin_, post = torch.empty(n, hid, **f), torch.empty(n, mult, **f)
        comb = torch.empty(n, mult * mult, **f)
        self._call("dsv4g_hc_pre", _ptr(bin_), _ptr(post), _ptr(comb), _ptr(state), _ptr(fn),
                   _ptr(scale3), _ptr(base), _ptr(norm_w), mult, hid, iters, C.c_float(rms_eps),
                   C.c_float(hc_eps), n, _ptr(status), self._stream())
        return bin_, post, comb

    def hc_post(self, state, branch, post, comb, mult):
        """In place on state [n][mult*hid]."""
        n, K = state.shape
        self._call("dsv4g_hc_post", _ptr(state), _ptr(branch), _ptr(post), _ptr(comb), mult,
                   K // mult, n, self._stream())
        return state

    def ffn_step_workspace_bytes(self, layer, mult, n_tokens):
        return int(self.lib.dsv4g_ffn_step_workspace_bytes(C.byref(layer.struct), mult,
                                                            n_tokens))

    def ffn_step(self, state, hc_fn, hc_scale, hc_base, ffn_norm, layer, mult, token_ids=None,
                 workspace=None, iters=20, rms_eps=1e-6, hc_eps=1e-6, check=True):
        """The FFN half of a decoder layer on state [n][mult*hid], in place.
        Returns (state, idx, wt)."""
        import torch
        n = state.shape[0]
        L = layer.struct
        need = self.ffn_step_workspace_bytes(layer, mult, n)
        if workspace is None or workspace.numel() < need:
            workspace = torch.zeros(need, dtype=torch.uint8, device=state.device)
        idx = torch.empty(n, L.topk, dtype=torch.int32, device=state.device)
        wt = torch.empty(n, L.topk, dtype=torch.float32, device=state.device)
        self._call("dsv4g_ffn_step", _ptr(state), _ptr(hc_fn), _ptr(hc_scale), _ptr(hc_base),
                   _ptr(ffn_norm), C.byref(L), _ptr(token_ids), n, mult, iters,
                   C.c_float(rms_eps), C.c_float(hc_eps), _ptr(workspace), workspace.numel(),
                   _ptr(idx), _ptr(wt), self._stream())
        if check:
            self.check_decode_status(workspace)
        return state, idx, wt


class DeviceLayer:
    """A DSV4GLayer whose buffers are torch tensors kept alive here."""

    def __init__(self, tensors: dict, meta: dict):
        self.tensors = tensors
        L = DSV4GLayer()
        L.hidden, L.inter = meta["hidden"], meta["inter"]
        L.n_experts, L.topk = meta["n_experts"], meta["topk"]
        L.route_scale, L.swiglu_limit = meta["route_scale"], meta["swiglu_limit"]
        L.expert_stride, L.scale_run = meta["expert_stride"], meta["scale_run"]
        for k in ("gate_w", "bias", "tid2eid", "experts", "sh1", "sh1_s", "sh3", "sh3_s", "sh2",
                  "sh2_s"):
            t = tensors.get(k)
            setattr(L, k, None if t is None else t.data_ptr())
        self.struct = L
        self.meta = meta

    def with_bias(self, bias):
        """The same weights (shared, not copied) with another router bias."""
        return DeviceLayer(dict(self.tensors, bias=bias), self.meta)

    @classmethod
    def from_host(cls, layer: dict, device="cuda"):
        """Upload a host (numpy) layer dict as built by tests/common.make_layer."""
        import torch
        t = {}
        for k in ("gate_w", "bias", "tid2eid", "experts", "sh1", "sh1_s", "sh3", "sh3_s", "sh2",
                  "sh2_s"):
            v = layer.get(k)
            if v is None:
                continue
            if v.dtype.name == "uint16":
                v = v.view("int16")
            t[k] = torch.from_numpy(v.copy()).to(device)
        meta = {k: layer[k] for k in ("hidden", "inter", "n_experts", "topk", "route_scale",
                                      "swiglu_limit", "expert_stride", "scale_run")}
        return cls(t, meta)


class StTensor(C.Structure):
    """Mirror of DSV4GTensor (include/dsv4_gpu.h)."""

    _fields_ = [("name", C.c_char_p), ("shard", C.c_int), ("dtype", C.c_int),
                ("ndim", C.c_int), ("shape", C.c_int64 * 4), ("off", C.c_int64),
                ("nbytes", C.c_int64)]

    def as_dict(self):
        return dict(name=self.name.decode("latin-1"), shard=self.shard, dtype=self.dtype,
                    shape=tuple(self.shape[:self.ndim]), off=self.off, nbytes=self.nbytes)


DTYPE_CODES = {"U8": 1, "BF16": 2, "F16": 3, "F32": 4, "I8": 5, "I64": 6, "F8_E4M3": 7,
               "F8_E8M0": 8}


def _st_sigs(lib):
    sp = C.POINTER(StTensor)
    for name, res, args in [
            ("dsv4g_st_open", C.c_int, [C.POINTER(_vp), C.c_char_p]),
            ("dsv4g_st_close", None, [_vp]),
            ("dsv4g_st_find", sp, [_vp, C.c_char_p]),
            ("dsv4g_st_read", C.c_int64, [_vp, sp, _vp]),
            ("dsv4g_st_read_f32", C.c_int64, [_vp, sp, _vp]),
            ("dsv4g_st_read_range", C.c_int64, [_vp, C.c_int, C.c_int64, C.c_int64, _vp]),
            ("dsv4g_st_numel", C.c_int64, [sp]),
            ("dsv4g_st_elemsize", C.c_int, [C.c_int]),
            ("dsv4g_st_count", C.c_int, [_vp]),
            ("dsv4g_st_tensor", sp, [_vp, C.c_int]),
            ("dsv4g_st_nshard", C.c_int, [_vp]),
            ("dsv4g_st_shard_path", C.c_char_p, [_vp, C.c_int]),
            ("dsv4g_st_dtype_name", C.c_char_p, [C.c_int]),
            ("dsv4g_st_upload", C.c_int, [_vp, sp, _vp, _vp]),
            ("dsv4g_moe_layer_bytes", C.c_size_t, [C.POINTER(DSV4GLayer), C.c_int, C.c_int]),
            ("dsv4g_load_moe_layer", C.c_int, [C.POINTER(DSV4GLayer), _vp, C.c_size_t, _vp,
                                               C.c_char_p, C.c_int, C.c_int, C.c_int, _vp])]:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


class Checkpoint:
    """A safetensors checkpoint directory indexed by dsv4g_st_open (host
    only: opening, finding and reading touch no GPU)."""

    def __init__(self, directory: str, gpu: "GpuLib | None" = None):
        self.gl = gpu or lib()
        self.lib = self.gl.lib
        h = _vp()
        rc = self.lib.dsv4g_st_open(C.byref(h), directory.encode())
        if rc != 0:
            raise RuntimeError(f"dsv4g_st_open: {self.lib.dsv4g_last_error().decode()}")
        self.h = h

    def close(self):
        if self.h:
            self.lib.dsv4g_st_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self):
        return self.lib.dsv4g_st_count(self.h)

    def nshard(self):
        return self.lib.dsv4g_st_nshard(self.h)

    def shard_path(self, i):
        p = self.lib.dsv4g_st_shard_path(self.h, i)
        return None if p is None else p.decode()

    def tensors(self):
        return [self.lib.dsv4g_st_tensor(self.h, i).contents.as_dict() for i in range(len(self))]

    def _find(self, name):
        return self.lib.dsv4g_st_find(self.h, name.encode("latin-1"))

    def find(self, name: str):
        t = self._find(name)
        return t.contents.as_dict() if t else None

    def read(self, name: str) -> bytes:
        t = self._find(name)
        if not t:
            raise KeyError(name)
        buf = C.create_string_buffer(max(t.contents.nbytes, 1))
        got = self.lib.dsv4g_st_read(self.h, t, buf)
        if got != t.contents.nbytes:
            raise RuntimeError(f"dsv4g_st_read: {self.lib.dsv4g_last_error().decode()}")
        return buf.raw[:got]

    def read_f32(self, name: str):
        import numpy as np
        t = self._find(name)
        if not t:
            raise KeyError(name)
        n = int(self.lib.dsv4g_st_numel(t))
        out = np.zeros(max(n, 1), np.float32)
        got = self.lib.dsv4g_st_read_f32(self.h, t, out.ctypes.data_as(_vp))
        return out[:got]

    def upload(self, name: str, dst):
        """One tensor's bytes into the device tensor dst (at least nbytes)."""
        t = self._find(name)
        if not t:
            raise KeyError(name)
        if dst.numel() * dst.element_size() < t.contents.nbytes:
            raise ValueError("destination too small")
        self.gl._call("dsv4g_st_upload", self.h, t, _ptr(dst), self.gl._stream())

    def load_moe_layer(self, meta: dict, scope="layers", layer=0, is_hash=False, vocab=0,
                       device="cuda"):
        """dsv4g_load_moe_layer into a fresh device arena: a layer object
        with .struct, .meta and .arena usable wherever a DeviceLayer is."""
        import torch
        L = DSV4GLayer()
        L.hidden, L.inter = meta["hidden"], meta["inter"]
        L.n_experts, L.topk = meta["n_experts"], meta["topk"]
        L.route_scale, L.swiglu_limit = meta["route_scale"], meta["swiglu_limit"]
        need = int(self.lib.dsv4g_moe_layer_bytes(C.byref(L), int(is_hash), vocab))
        if need == 0:
            raise RuntimeError(f"dsv4g_moe_layer_bytes: {self.lib.dsv4g_last_error().decode()}")
        arena = torch.empty(need, dtype=torch.uint8, device=device)
        self.gl._call("dsv4g_load_moe_layer", C.byref(L), _ptr(arena), need, self.h,
                      scope.encode(), layer, int(is_hash), vocab, self.gl._stream())
        return LoadedLayer(L, arena, dict(meta, expert_stride=L.expert_stride,
                                          scale_run=L.scale_run))


class LoadedLayer:
    """A DSV4GLayer whose pointers point into one loader arena (kept alive)."""

    def __init__(self, struct, arena, meta):
        self.struct, self.arena, self.meta = struct, arena, meta

    def offset(self, field: str) -> int:
        """Byte offset of a DSV4GLayer pointer field inside the arena."""
        p = getattr(self.struct, field)
        return None if p is None else p - self.arena.data_ptr()


_LIB = None


def lib() -> GpuLib:
    global _LIB
    if _LIB is None:
        _LIB = GpuLib()
    return _LIB
