"""Synthetic safetensors checkpoints in the reference's format and tensor
names, for the loader's tests and benchmark: [u64 LE header length][JSON
header][data], tensors named as the checkpoint names them
(src/dsv4/dsv4_model.c:2014-2053, 3063-3136; docs/DSV4_ARCHITECTURE.md:58-113).
numpy only."""
from __future__ import annotations

import json
import os
import struct

import numpy as np

ST_ITEMSIZE = {"U8": 1, "I8": 1, "I64": 8, "BF16": 2, "F16": 2, "F32": 4, "F8_E4M3": 1,
               "F8_E8M0": 1}


def write_safetensors(path, entries, metadata=None, header_pad=8):
    """Write one shard, tensors stored in the order given. entries:
    (name, dtype, shape, raw bytes). The header is space-padded to a multiple
    of header_pad bytes."""
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
    """The named tensors of one MoE layer given as a dict of host arrays
    (hidden, inter, n_experts, gate_w BF16 bits, bias or tid2eid, experts in
    the [scale run | weight run] slot layout with expert_stride / scale_run,
    sh1/sh3/sh2 FP8 codes and their _s E8M0 scales), as (name, dtype, shape,
    bytes). order "reference": each expert's scale run then weight run, w1 w2
    w3; "scrambled": each expert's six tensors in a seeded random order and
    the experts shuffled."""
    H, I, E = layer["hidden"], layer["inter"], layer["n_experts"]
    s_sz = (I * ((H + 31) // 32), H * ((I + 31) // 32), I * ((H + 31) // 32))
    w_sz = (I * ((H + 1) // 2), H * ((I + 1) // 2), I * ((H + 1) // 2))
    stride, srun = layer["expert_stride"], layer["scale_run"]
    pre = f"{scope}.{index}."
    out = [(pre + "ffn.gate.weight", "BF16", (E, H),
            np.ascontiguousarray(layer["gate_w"]).tobytes())]
    if layer.get("tid2eid") is not None:
        t = np.ascontiguousarray(layer["tid2eid"], np.int64)
        out.append((pre + "ffn.gate.tid2eid", "I64", t.shape, t.tobytes()))
    else:
        b = layer["bias"] if layer.get("bias") is not None else np.zeros(E, np.float32)
        out.append((pre + "ffn.gate.bias", "F32", (E,), np.asarray(b, np.float32).tobytes()))
    bi, bh = (I + 127) // 128, (H + 127) // 128
    for m, key, (r, c, sr, sc) in (("w1", "sh1", (I, H, bi, bh)), ("w3", "sh3", (I, H, bi, bh)),
                                   ("w2", "sh2", (H, I, bh, bi))):
        out.append((pre + f"ffn.shared_experts.{m}.weight", "F8_E4M3", (r, c),
                    np.ascontiguousarray(layer[key]).tobytes()))
        out.append((pre + f"ffn.shared_experts.{m}.scale", "F8_E8M0", (sr, sc),
                    np.ascontiguousarray(layer[key + "_s"]).tobytes()))
    rng = np.random.default_rng(seed)
    experts = list(range(E))
    if order == "scrambled":
        rng.shuffle(experts)
    shapes = ((I, H), (H, I), (I, H))
    for e in experts:
        slot = layer["experts"][e * stride:(e + 1) * stride]
        scales, weights = slot[:srun], slot[srun:]
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
