"""Seeded synthetic MoE layers built directly in HBM, in the reference's
checkpoint formats: routed experts as FP4 E2M1 with per-row per-32 E8M0
scales in the per-expert [scale run | weight run] slot layout, the shared
expert as FP8 E4M3 with per-128x128 E8M0 scales, the router gate as BF16.
Weights are N(0, sigma) from torch's device generator, quantised by the
library's HIP quantisers (dsv4g_quant_fp4_rows / dsv4g_quant_fp8_blocks)."""
from __future__ import annotations

import torch

import dsv4_gpu


def expert_geometry(hidden: int, inter: int) -> dict:
    s1, s2 = inter * (hidden // 32), hidden * (inter // 32)
    w1, w2 = inter * (hidden // 2), hidden * (inter // 2)
    return dict(s1=s1, s2=s2, w1=w1, w2=w2, scale_run=2 * s1 + s2,
                stride=2 * s1 + s2 + 2 * w1 + w2)


def device_layer(seed: int, hidden=4096, inter=2048, n_experts=256, topk=6, sigma=0.02,
                 gate_sigma=None, bias=False, device="cuda") -> dsv4_gpu.DeviceLayer:
    lib = dsv4_gpu.lib()
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    H, I, E = hidden, inter, n_experts
    geo = expert_geometry(H, I)
    stride, srun = geo["stride"], geo["scale_run"]
    experts = torch.empty(E * stride, dtype=torch.uint8, device=device)
    buf = torch.empty(H * I, dtype=torch.float32, device=device)
    mats = [(I, H, 0, 0), (H, I, geo["s1"], geo["w1"]),
            (I, H, geo["s1"] + geo["s2"], geo["w1"] + geo["w2"])]
    for e in range(E):
        base = e * stride
        for rows, cols, soff, woff in mats:
            w = buf[:rows * cols].view(rows, cols)
            torch.randn(rows, cols, generator=g, device=device, out=w)
            w.mul_(sigma)
            lib.quant_fp4_rows(w, experts[base + srun + woff:], experts[base + soff:])
    t = {"experts": experts}
    gs = gate_sigma if gate_sigma is not None else 1.0 / (H ** 0.5)
    gw = torch.randn(E, H, generator=g, device=device) * gs
    t["gate_w"] = gw.to(torch.bfloat16).view(torch.int16).contiguous()
    for name, (rows, cols) in (("sh1", (I, H)), ("sh3", (I, H)), ("sh2", (H, I))):
        w = torch.randn(rows, cols, generator=g, device=device) * sigma
        codes = torch.empty(rows, cols, dtype=torch.uint8, device=device)
        scales = torch.empty((rows + 127) // 128, (cols + 127) // 128, dtype=torch.uint8,
                             device=device)
        lib.quant_fp8_blocks(w, codes, scales, mode=0)
        t[name], t[name + "_s"] = codes, scales
    if bias:
        t["bias"] = torch.randn(E, generator=g, device=device) * 0.1
    meta = dict(hidden=H, inter=I, n_experts=E, topk=topk, route_scale=1.5, swiglu_limit=10.0,
                expert_stride=stride, scale_run=srun)
    return dsv4_gpu.DeviceLayer(t, meta)


def host_copy(layer: dsv4_gpu.DeviceLayer) -> dict:
    """The same layer as host numpy arrays (the oracle / reference inputs)."""
    d = dict(layer.meta)
    for k in ("gate_w", "bias", "tid2eid", "experts", "sh1", "sh1_s", "sh3", "sh3_s", "sh2",
              "sh2_s"):
        v = layer.tensors.get(k)
        if v is None:
            d[k] = None
            continue
        a = v.cpu().numpy()
        d[k] = a.view("uint16") if a.dtype.name == "int16" else a
    return d


def bf16_tokens(n: int, hidden: int, seed: int, device="cuda") -> torch.Tensor:
    """x ~ N(0,1) rounded to BF16 values, stored as fp32 (the MoE input)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    x = torch.randn(n, hidden, generator=g, device=device)
    return x.to(torch.bfloat16).to(torch.float32).contiguous()
