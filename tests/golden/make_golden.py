"""Writes the golden fixtures under tests/golden/ from the reference engine
compiled from its own sources (oracle/_ref, built by oracle/Makefile).

Run in the container that has the reference mounted:
    make -C oracle && python tests/golden/make_golden.py

Outputs (inputs and expected outputs only):
  ref_vectors.npz   small seeded cases of every kernel on the MoE path
  ref_bench.json    checksums printed by the reference's kernel benchmark
                    (benchmarks/bench_dsv4_kernels.c), run here
"""
from __future__ import annotations

import json
import os
import re
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))

from common import bf16_bits, bf16_input, make_layer, expert_slot, pyoracle  # noqa: E402


def main():
    ref = pyoracle.RefLib()
    orc = pyoracle.Oracle()
    rng = np.random.default_rng(20260731)
    out = {}

    # scalar decode tables and rounding
    out["fp8_table"] = ref.fp8_table()
    out["e8m0_table"] = ref.e8m0_table()
    probe = np.concatenate([
        rng.standard_normal(2000, dtype=np.float32) * 100,
        rng.standard_normal(500, dtype=np.float32) * 0.01,
        np.array([0.0, -0.0, 448.0, -448.0, 470.0, 500.0, 1e-9, 15 / 1024, 7 / 512,
                  8 / 512, 0.1, 1 + 2 ** -8, 1 + 2 ** -7, 3e38, -3e38], np.float32),
    ]).astype(np.float32)
    out["round_in"] = probe
    out["round_out"] = ref.round_e4m3(probe)
    out["bf16_out"] = ref.f32_to_bf16(probe)

    # activation quant: random, ramp, tiny, huge, partial last group
    qin = np.concatenate([rng.standard_normal(4096, dtype=np.float32),
                          np.linspace(-3, 3, 256, dtype=np.float32),
                          np.full(128, 1e-7, np.float32),
                          np.full(128, 448.0 * 1024, np.float32),
                          rng.standard_normal(100, dtype=np.float32) * 50]).astype(np.float32)
    out["quant_in"] = qin
    qx, qs = ref.quant_fp8_act(qin)
    out["quant_qx"], out["quant_qs"] = qx, qs

    # GEMVs at small shapes, scale codes include NaN (255) and subnormal (0, 3)
    R, IN = 48, 256
    x = rng.standard_normal(IN, dtype=np.float32)
    qx, qs = ref.quant_fp8_act(x)
    W4 = rng.integers(0, 256, (R, IN // 2), dtype=np.uint8)
    S4 = rng.integers(120, 134, (R, IN // 32), dtype=np.uint8)
    S4[3, 2] = 255
    S4[5, 0] = 0
    S4[6, 1] = 3
    W4b = rng.integers(0, 256, (R, IN // 2), dtype=np.uint8)
    S4b = rng.integers(120, 134, (R, IN // 32), dtype=np.uint8)
    W8 = rng.integers(0, 256, (R, IN), dtype=np.uint8)
    W8[W8 & 0x7F == 0x7F] = 0x11  # keep the weights finite
    S8 = rng.integers(120, 134, ((R + 127) // 128, IN // 128), dtype=np.uint8)
    S8[0, 1] = 255
    W8b = rng.integers(0, 126, (R, IN), dtype=np.uint8)
    S8b = rng.integers(120, 134, ((R + 127) // 128, IN // 128), dtype=np.uint8)
    out.update(g_qx=qx, g_qs=qs, g_W4=W4, g_S4=S4, g_W4b=W4b, g_S4b=S4b, g_W8=W8,
               g_S8=S8, g_W8b=W8b, g_S8b=S8b)
    out["g_fp4"] = ref.gemv_fp4_q(qx, qs, W4, S4, IN, R)
    out["g_fp4_pair0"], out["g_fp4_pair1"] = ref.gemv_fp4_pair_q(qx, qs, W4, S4, W4b, S4b, IN, R)
    out["g_fp8"] = ref.gemv_fp8_q(qx, qs, W8, S8, IN, R, 1)
    out["g_fp8_raw"] = ref.gemv_fp8_q(qx, qs, W8, S8, IN, R, 0)
    out["g_fp8_pair0"], out["g_fp8_pair1"] = ref.gemv_fp8_pair_q(qx, qs, W8, S8, W8b, S8b, IN, R)
    xb = rng.standard_normal((5, IN), dtype=np.float32)
    qxb, qsb = ref.quant_fp8_act(xb)
    out["g_bqx"], out["g_bqs"] = qxb, qsb
    out["g_fp4_batch"] = ref.gemv_fp4_batch_q(qxb, qsb, W4, S4, IN, R)
    out["g_fp8_batch"] = ref.gemv_fp8_batch_q(qxb, qsb, W8, S8, IN, R, 1)
    Gb = bf16_bits(rng.standard_normal((R, IN), dtype=np.float32) * 0.05)
    out["g_bf16_W"] = Gb
    out["g_bf16_x"] = x
    out["g_bf16"] = ref.gemv_bf16(x, Gb, IN, R, 0)
    # public float-scale GEMVs
    wf = rng.standard_normal((R, IN), dtype=np.float32) * 0.02
    codes, fsc = orc.quant_fp8_blocks_absmax(wf)
    out["g_f8_codes"], out["g_f8_scales"] = codes, fsc
    out["g_fp8_legacy"] = ref.gemv_fp8_legacy(x, codes, fsc, IN, R, 128)
    out["g_fp8_tbl"] = ref.gemv_fp8_tbl(x, codes, fsc, IN, R, 128)
    w4s = np.ldexp(1.0, S4.astype(np.int32) - 127).astype(np.float32)
    w4s[3, 2] = 1.0
    out["g_fp4_wscale"] = w4s
    out["g_fp4_legacy"] = ref.gemv_fp4_legacy(qx, qs, W4, w4s, IN, R, 32)

    # SwiGLU + requant, sqrt-softplus
    gate = bf16_bits(rng.standard_normal(512, dtype=np.float32) * 4).astype(np.uint32) << 16
    up = bf16_bits(rng.standard_normal(512, dtype=np.float32) * 4).astype(np.uint32) << 16
    gate, up = gate.view(np.float32), up.view(np.float32)
    gate[:4] = [30.0, -30.0, 10.0, -100.0]
    up[:4] = [-20.0, 15.0, 10.5, 3.0]
    out["sw_gate"], out["sw_up"] = gate, up
    out["sw_y"], out["sw_qy"], out["sw_qs"] = ref.swiglu_quant(gate, up, 10, 0.3716)
    zz = np.concatenate([np.linspace(-30, 30, 601, dtype=np.float32),
                         rng.standard_normal(400, dtype=np.float32) * 3]).astype(np.float32)
    out["ssp_in"], out["ssp_out"] = zz, ref.sqrt_softplus(zz)

    # public router (bias; hash)
    H, E, K = 256, 16, 6
    Gr = bf16_bits(rng.standard_normal((E, H), dtype=np.float32) / 16)
    xr = bf16_input(rng, H)
    bias = rng.standard_normal(E, dtype=np.float32) * 0.1
    t2e = np.stack([rng.permutation(E)[:K] for _ in range(4)]).astype(np.int64)
    out.update(rt_G=Gr, rt_x=xr, rt_bias=bias, rt_t2e=t2e)
    out["rt_idx"], out["rt_wt"] = ref.router_public(xr, Gr, bias, None, 0, H, E, K, 0, 1.5)
    out["rt_hidx"], out["rt_hwt"] = ref.router_public(xr, Gr, None, t2e, 2, H, E, K, 1, 1.5)

    # one small MoE layer: moe_forward (bias and hash) and moe_forward_batch
    for tag, kw in (("moe", dict(bias=True)), ("moeh", dict(hash_vocab=7))):
        L = make_layer(orc, 256, 128, 16, 6, seed=5 if tag == "moe" else 6, **kw)
        X = bf16_input(rng, (9, 256))
        tok = np.arange(9, dtype=np.int32) % 7
        outs, idxs, wts = [], [], []
        for t in range(9):
            o, i, w = ref.moe_forward(L, X[t], int(tok[t]))
            outs.append(o)
            idxs.append(i)
            wts.append(w)
        out[f"{tag}_x"], out[f"{tag}_tok"] = X, tok
        out[f"{tag}_out"] = np.stack(outs)
        out[f"{tag}_idx"], out[f"{tag}_wt"] = np.stack(idxs), np.stack(wts)
        out[f"{tag}_batch_out"] = ref.moe_forward_batch(L, X, tok)
        for k in ("gate_w", "experts", "sh1", "sh1_s", "sh3", "sh3_s", "sh2", "sh2_s"):
            out[f"{tag}_{k}"] = L[k]
        out[f"{tag}_bias"] = L["bias"] if L["bias"] is not None else np.zeros(0, np.float32)
        out[f"{tag}_t2e"] = (L["tid2eid"] if L["tid2eid"] is not None
                             else np.zeros((0, 6), np.int64))
        out[f"{tag}_meta"] = np.array([L["hidden"], L["inter"], L["n_experts"], L["topk"],
                                       L["expert_stride"], L["scale_run"]], np.int64)
        # one expert forward at this size
        s, w = expert_slot(L, 3)
        qx1, qs1 = ref.quant_fp8_act(X[0])
        out[f"{tag}_exp3"] = ref.expert_forward(qx1, qs1, s, w, 256, 128, 10, 0.41)
        out[f"{tag}_shared"] = ref.shared_expert_forward(qx1, qs1, L, 256, 128, 10)

    np.savez_compressed(os.path.join(HERE, "ref_vectors.npz"), **out)

    # the reference kernel benchmark's checksums
    bench = os.path.join(ROOT, "oracle", "_ref", "bench_dsv4_kernels")
    txt = subprocess.run([bench], capture_output=True, text=True, check=True).stdout
    lines = txt.splitlines()
    cks = {}
    for i, ln in enumerate(lines):
        if ln.startswith("bench_dsv4: "):
            name = ln[len("bench_dsv4: "):]
            vals = re.findall(r"checksums? ([-0-9.]+)(?: ([-0-9.]+))?", lines[i + 1])
            if vals:
                cks[name] = [v for v in vals[0] if v]
    with open(os.path.join(HERE, "ref_bench.json"), "w") as f:
        json.dump({"source": "benchmarks/bench_dsv4_kernels.c, compiled from the reference "
                             "sources by oracle/Makefile and run in this container",
                   "checksums": cks}, f, indent=1)
    print("wrote", sorted(out)[:5], "...", len(out), "arrays;", len(cks), "bench checksums")


if __name__ == "__main__":
    main()
