"""Shared helpers for the parity tests: seeded synthetic layers in the
reference's on-disk formats, and the tolerance measures the tests use.

Layout of one routed expert (src/dsv4/dsv4_internal.h:8-17, 33-37 and
src/dsv4/dsv4_model.c:6298-6305): a scale run [s1 | s2 | s3] of E8M0 codes
(per row, per 32 columns) followed by a weight run [w1 | w2 | w3] of packed
E2M1 nibbles (two per byte, low nibble = even column). w1 = gate [I][H],
w2 = down [H][I], w3 = up [I][H].
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "deepseek-v4-flash-0731-in-c_amd", "python"))

import pyoracle  # noqa: E402


def bf16_bits(x):
    """RNE BF16 narrowing of a float32 array (the reference's integer rule)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    return (u >> 16).astype(np.uint16)


def bf16_values(x):
    return (bf16_bits(x).astype(np.uint32) << 16).view(np.float32)


def expert_geometry(hidden, inter):
    w1 = inter * ((hidden + 1) // 2)
    w2 = hidden * ((inter + 1) // 2)
    s1 = inter * ((hidden + 31) // 32)
    s2 = hidden * ((inter + 31) // 32)
    scale_run = 2 * s1 + s2
    weight_run = 2 * w1 + w2
    return dict(w1=w1, w2=w2, s1=s1, s2=s2, scale_run=scale_run,
                weight_run=weight_run, stride=scale_run + weight_run)


def make_expert_bytes(orc, rng, hidden, inter, sigma=0.02):
    """One routed expert slot (scale run + weight run) from N(0, sigma)."""
    g = expert_geometry(hidden, inter)
    w1 = rng.standard_normal((inter, hidden), dtype=np.float32) * sigma
    w2 = rng.standard_normal((hidden, inter), dtype=np.float32) * sigma
    w3 = rng.standard_normal((inter, hidden), dtype=np.float32) * sigma
    p1, s1 = orc.quant_fp4_rows(w1)
    p2, s2 = orc.quant_fp4_rows(w2)
    p3, s3 = orc.quant_fp4_rows(w3)
    slot = np.concatenate([s1.ravel(), s2.ravel(), s3.ravel(),
                           p1.ravel(), p2.ravel(), p3.ravel()])
    assert slot.size == g["stride"]
    return slot


def make_layer(orc, hidden=256, inter=128, n_experts=16, topk=6, seed=0,
               bias=False, hash_vocab=0, sigma=0.02, gate_sigma=None,
               route_scale=1.5, swiglu_limit=10.0):
    """A seeded synthetic MoE layer in the reference formats."""
    rng = np.random.default_rng(seed)
    g = expert_geometry(hidden, inter)
    experts = np.concatenate([make_expert_bytes(orc, rng, hidden, inter, sigma)
                              for _ in range(n_experts)])
    gsig = gate_sigma if gate_sigma is not None else 1.0 / np.sqrt(hidden)
    gate = bf16_bits(rng.standard_normal((n_experts, hidden), dtype=np.float32) * gsig)
    sh = {}
    for name, (r, c) in (("sh1", (inter, hidden)), ("sh3", (inter, hidden)),
                         ("sh2", (hidden, inter))):
        w = rng.standard_normal((r, c), dtype=np.float32) * sigma
        codes, scales = orc.quant_fp8_blocks_e8m0(w)
        sh[name] = codes
        sh[name + "_s"] = scales
    layer = dict(hidden=hidden, inter=inter, n_experts=n_experts, topk=topk,
                 route_scale=route_scale, swiglu_limit=swiglu_limit,
                 gate_w=np.ascontiguousarray(gate), experts=experts,
                 expert_stride=g["stride"], scale_run=g["scale_run"],
                 bias=None, tid2eid=None, **sh)
    if bias:
        layer["bias"] = (rng.standard_normal(n_experts, dtype=np.float32) * 0.1)
    if hash_vocab:
        t = np.stack([rng.permutation(n_experts)[:topk] for _ in range(hash_vocab)])
        layer["tid2eid"] = np.ascontiguousarray(t.astype(np.int64))
    return layer


def expert_slot(layer, e):
    s = layer["expert_stride"]
    slot = layer["experts"][e * s:(e + 1) * s]
    return slot[:layer["scale_run"]], slot[layer["scale_run"]:]


def bf16_input(rng, shape):
    """x ~ N(0,1) rounded to BF16 values, as the MoE input is."""
    return bf16_values(rng.standard_normal(shape, dtype=np.float32))


def max_rel_err(got, ref):
    """max |got - ref| / max |ref| (normwise relative error)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = max(np.max(np.abs(ref)), 1e-30)
    return float(np.max(np.abs(got - ref)) / denom)


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.uint32)
    b = np.ascontiguousarray(b, np.float32).view(np.uint32)
    return a.shape == b.shape and bool(np.array_equal(a, b))


def zipf_bias(n_experts, seed=8, s=1.2, strength=0.15):
    """Router bias giving Zipf(s)-skewed expert popularity over a seeded
    permutation of the experts: strength * (log p_rank - mean), p ~ rank^-s
    (the bias bench.py times the batched path with)."""
    rng = np.random.default_rng(seed)
    p = np.arange(1, n_experts + 1, dtype=np.float64) ** -s
    b = np.empty(n_experts)
    b[rng.permutation(n_experts)] = np.log(p / p.sum())
    return (strength * (b - b.mean())).astype(np.float32)


def bf16_ulp(v):
    """Spacing of BF16 values at |v| (normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return np.ldexp(1.0, (e - 7).astype(int))


# ------------------------------------------------------------ safetensors
from st_writer import ST_ITEMSIZE, moe_layer_tensors, write_checkpoint, write_safetensors  # noqa: E402,F401


PROBE_LIB = os.path.join(ROOT, "tests", "hip", "libdsv4_probe.so")


class ProbeLib:
    """The test-only ISA probes (tests/hip/dsv4_probe.hip): one tile of each
    MFMA form the grouped kernels use, and the hardware FP4/FP8 converts over
    every code. Not part of the product library."""

    def __init__(self, path=PROBE_LIB):
        import ctypes as C
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build it with `make -C tests/hip` "
                               f"(or __graft_entry__.build())")
        self.C, self.lib = C, C.CDLL(path)
        vp = C.c_void_p
        self.lib.dsv4p_probe_converts.argtypes = [vp, vp, vp]
        self.lib.dsv4p_probe_mfma.argtypes = [C.c_int, vp, vp, vp, vp, vp, vp]
        for f in (self.lib.dsv4p_probe_converts, self.lib.dsv4p_probe_mfma):
            f.restype = C.c_int

    def _p(self, t):
        return None if t is None else self.C.c_void_p(t.data_ptr())

    def _stream(self):
        import torch
        return self.C.c_void_p(torch.cuda.current_stream().cuda_stream)

    def converts(self, device):
        """(fp4 [512]: both nibbles of bytes 0..255, fp8 [256]) as fp32."""
        import torch
        a = torch.empty(512, dtype=torch.float32, device=device)
        b = torch.empty(256, dtype=torch.float32, device=device)
        assert self.lib.dsv4p_probe_converts(self._p(a), self._p(b), self._stream()) == 0
        return a, b

    def mfma(self, kind, A, B, sa=None, sb=None):
        """One 16x16 tile, row-major operands (kind 0: FP4 x FP8 block-scaled,
        1: FP8 x FP8 block-scaled, 2: BF16); D [16][16] fp32 row-major."""
        import torch
        D = torch.empty(16, 16, dtype=torch.float32, device=A.device)
        rc = self.lib.dsv4p_probe_mfma(kind, self._p(D), self._p(A), self._p(B), self._p(sa),
                                       self._p(sb), self._stream())
        assert rc == 0, rc
        return D


_PROBE = None


def probe_lib() -> ProbeLib:
    global _PROBE
    if _PROBE is None:
        _PROBE = ProbeLib()
    return _PROBE
