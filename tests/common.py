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
ST_ITEMSIZE = {"U8": 1, "I8": 1, "I64": 8, "BF16": 2, "F16": 2, "F32": 4, "F8_E4M3": 1,
               "F8_E8M0": 1}


def write_safetensors(path, entries, metadata=None, header_pad=8):
    """Write one shard: [u64 LE header length][JSON header][data], tensors
    stored in the order given. entries: (name, dtype, shape, raw bytes).
    The header is space-padded to a multiple of header_pad bytes."""
    import json
    import struct
    header = {}
    if metadata is not None:
        header["__metadata__"] = metadata
    off = 0
    for name, dt, shape, raw in entries:
        n = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
        assert len(raw) == n * ST_ITEMSIZE[dt], (name, len(raw), shape, dt)
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * ((-len(h)) % header_pad)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for _, _, _, raw in entries:
            f.write(raw)


def moe_layer_tensors(layer, scope="layers", index=0, order="reference", seed=0):
    """The named tensors of a make_layer() layer, as the checkpoint stores
    them (src/dsv4/dsv4_model.c:2014-2053, 3063-3136;
    docs/DSV4_ARCHITECTURE.md:58-113): a list of (name, dtype, shape, bytes).
    order "reference": each expert's scale run then weight run, w1 w2 w3;
    "scrambled": each expert's six tensors in a seeded random order and the
    experts themselves shuffled."""
    H, I, E = layer["hidden"], layer["inter"], layer["n_experts"]
    g = expert_geometry(H, I)
    pre = f"{scope}.{index}."
    out = [(pre + "ffn.gate.weight", "BF16", (E, H), layer["gate_w"].tobytes())]
    if layer.get("tid2eid") is not None:
        t = layer["tid2eid"]
        out.append((pre + "ffn.gate.tid2eid", "I64", t.shape, t.tobytes()))
    else:
        b = layer["bias"] if layer.get("bias") is not None else np.zeros(E, np.float32)
        out.append((pre + "ffn.gate.bias", "F32", (E,), np.asarray(b, np.float32).tobytes()))
    bi, bh = (I + 127) // 128, (H + 127) // 128
    for m, (r, c, sr, sc) in (("w1", (I, H, bi, bh)), ("w3", (I, H, bi, bh)),
                              ("w2", (H, I, bh, bi))):
        key = {"w1": "sh1", "w3": "sh3", "w2": "sh2"}[m]
        out.append((pre + f"ffn.shared_experts.{m}.weight", "F8_E4M3", (r, c),
                    np.ascontiguousarray(layer[key]).tobytes()))
        out.append((pre + f"ffn.shared_experts.{m}.scale", "F8_E8M0", (sr, sc),
                    np.ascontiguousarray(layer[key + "_s"]).tobytes()))
    rng = np.random.default_rng(seed)
    experts = list(range(E))
    if order == "scrambled":
        rng.shuffle(experts)
    for e in experts:
        scales, weights = expert_slot(layer, e)
        s_sz = (g["s1"], g["s2"], g["s1"])
        w_sz = (g["w1"], g["w2"], g["w1"])
        shapes = ((I, H), (H, I), (I, H))
        items = []
        so = wo = 0
        for k in range(3):
            r, c = shapes[k]
            items.append((pre + f"ffn.experts.{e}.w{k + 1}.scale", "F8_E8M0", (r, (c + 31) // 32),
                          scales[so:so + s_sz[k]].tobytes()))
            so += s_sz[k]
        for k in range(3):
            r, c = shapes[k]
            items.append((pre + f"ffn.experts.{e}.w{k + 1}.weight", "I8", (r, (c + 1) // 2),
                          weights[wo:wo + w_sz[k]].tobytes()))
            wo += w_sz[k]
        if order == "scrambled":
            items = [items[i] for i in rng.permutation(len(items))]
        out.extend(items)
    return out


def write_checkpoint(directory, tensors, n_shards=1, prefix="model"):
    """Split tensors (in order) over n_shards files named like the
    checkpoint's (model-0000k-of-0000n.safetensors)."""
    os.makedirs(directory, exist_ok=True)
    bounds = np.linspace(0, len(tensors), n_shards + 1).astype(int)
    for k in range(n_shards):
        write_safetensors(os.path.join(directory, f"{prefix}-{k + 1:05d}-of-{n_shards:05d}"
                                       ".safetensors"),
                          tensors[bounds[k]:bounds[k + 1]], metadata={"format": "pt"})
