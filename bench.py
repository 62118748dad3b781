#!/usr/bin/env python3
"""Benchmark of the gfx950 quantized MoE expert path (one MI355X).

Default workload: one MoE layer decode at 1 token: hidden 4096, 256 routed
FP4 experts (inter 2048) top-6 by sqrt-softplus router + 1 shared FP8 expert,
all weights resident in HBM. A step is one token through one layer (router,
activation quant, 6 routed + shared experts, combine). Eight seeded layers
(about 27.6 GB) are rotated step by step so the 256 MB Infinity Cache cannot
serve the weights; each step has its own token. The K timed steps are
captured in a HIP graph and replayed, so the time is the GPU's, not Python's.

Prints ONE JSON line. value = algorithmic HBM bytes per step / time per step.
roofline: the dominant kernel (the front launch, the second of three: exact
router chains, the routed gate/up GEMVs and the shared expert's down GEMV),
timed live with HIP events around a graph of its launches on the launch
stream. cpu_baseline: the
reference's own moe_forward (oracle/_ref, compiled from the reference sources)
on the same layer on the host cores.

The kernels entries (config keys fp8_matvec_2048x4096, fp4_expert_1_token,
ffn_step_1_token, attention_projections, checkpoint_load) time the
standalone FP8 matvec, one FP4 expert, the FFN half of a decoder layer on
device (hyper-connection pre-mix, RMSNorm, MoE layer, post-mix), the four
attention FP8 projections and the checkpoint-to-HBM loader.

The same run also measures the batched path on layer 0 with a Zipf(1.2)
router bias (config keys "verify_64" and "prefill_4096"): 64 tokens
(speculative verify) and 4096 tokens (prefill) through the grouped GEMMs,
timed with HIP events on the launch stream, FLOPs = 6 * hidden * inter per
(token, expert) pair including the shared expert. --workload picks one part
alone (for profiling); the JSON line then carries that part's numbers.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "deepseek-v4-flash-0731-in-c_amd", "python"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0   # dense MFMA peaks of one MI355X
FP8_PEAK_TFLOPS = 5000.0
# fp32 vector FMA: 256 CUs x 64 lanes x 2 flops x 2.4 GHz issued one FMA per
# lane per clock; the published 157.3 TFLOP/s is the packed (two-wide) rate,
# which this build does not emit
FP32_FMA_PEAK_TFLOPS = 78.6
VOCAB = 129280
METRIC = "MoE layer decode GB/s (% HBM peak); prefill grouped-GEMM TFLOPS (% MFMA)"

H, I, E, K = 4096, 2048, 256, 6
EXPERT_BYTES = 13_369_344                     # one FP4 expert: weights + E8M0 scales
SHARED_BYTES = 3 * (8_388_608 + 512)          # FP8 shared expert: weights + scales
GATE_BYTES = E * H * 2                        # BF16 router gate
# algorithmic bytes of one decode step: 6 routed experts, the shared expert,
# the router gate, the BF16 input and the BF16 output
DECODE_BYTES = K * EXPERT_BYTES + SHARED_BYTES + GATE_BYTES + H * 2 + H * 2
DECODE_FLOPS = 7 * 2 * 3 * I * H + 2 * E * H
# the front launch (dominant kernel, phase 1 of three): w1 and w3 of the 6
# routed experts with their scales, the shared expert's down matrix w2 with
# its scales, and the BF16 input
FRONT_BYTES = K * 2 * (4_194_304 + 262_144) + (8_388_608 + 512) + H * 2


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=240)
    p.add_argument("--warmup", type=int, default=16)
    p.add_argument("--layers", type=int, default=8)
    p.add_argument("--replays", type=int, default=5)
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--workload", choices=("all", "decode", "verify", "prefill", "kernels",
                                          "head", "dropin"),
                   default="all")
    p.add_argument("--zipf-strength", type=float, default=0.15)
    p.add_argument("--copy-calibration", action="store_true",
                   help="after the decode part, copy 1 GiB device-to-device 3 times: the "
                        "known-size copy that scales rocprofv3 FETCH_SIZE / WRITE_SIZE")
    return p.parse_args()


def zipf_bias(n_experts, seed=8, s=1.2, strength=0.15):
    """Router bias giving Zipf(s)-skewed expert popularity over a seeded
    permutation of the experts: strength * (log p_rank - mean), p ~ rank^-s."""
    import numpy as np
    rng = np.random.default_rng(seed)
    p = np.arange(1, n_experts + 1, dtype=np.float64) ** -s
    b = np.empty(n_experts)
    b[rng.permutation(n_experts)] = np.log(p / p.sum())
    return (strength * (b - b.mean())).astype(np.float32)


def bench_batch(lib, layer, n_tokens, iters):
    """Time moe_forward_batch on n_tokens seeded tokens (warm-up call first)."""
    import numpy as np
    import torch
    import synth
    dev = torch.device("cuda:0")
    X = synth.bf16_tokens(n_tokens, H, seed=11 + n_tokens, device=dev)
    ws = torch.empty(lib.moe_batch_workspace_bytes(layer, n_tokens), dtype=torch.uint8,
                     device=dev)
    out, idx, wt = lib.moe_forward_batch(layer, X, workspace=ws)
    torch.cuda.synchronize()
    counts = torch.bincount(idx.flatten().long(), minlength=E).cpu().numpy()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        lib.moe_forward_batch(layer, X, workspace=ws, out=out)
    e1.record()
    torch.cuda.synchronize()
    ms_eager = e0.elapsed_time(e1) / iters
    # the calls captured in one HIP graph and replayed: the device time without
    # the host's per-launch cost (eager calls of a few-token batch can be
    # host-bound)
    ms = graph_time(lambda i: lib.moe_forward_batch(layer, X, workspace=ws, out=out), iters,
                    replays=3)
    pairs = int(counts.sum()) + n_tokens              # routed + shared (token, expert) pairs
    flops = 6 * H * I * pairs
    hit = int((counts > 0).sum())
    wbytes = hit * EXPERT_BYTES + SHARED_BYTES + GATE_BYTES
    return {
        "tokens": n_tokens, "ms_per_layer": round(ms, 4), "ms_per_layer_eager": round(ms_eager, 4),
        "timing": "HIP graph of the calls, replayed (ms_per_layer_eager: the same calls launched "
                  "one by one)",
        "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
        "frac_bf16_mfma_peak": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
        "frac_fp8_mfma_peak": round(flops / (ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
        "weight_gbs": round(wbytes / (ms * 1e-3) / 1e9, 1),
        "experts_hit": hit, "max_tokens_per_expert": int(counts.max()),
        "median_tokens_per_expert": float(np.median(counts)),
        "expert_flops": flops, "iters": iters,
        "mfma": "v_mfma_f32_16x16x32_bf16 (FP4/FP8 weights converted to BF16 x block scale "
                "in registers; exact products, fp32 accumulate)",
        "roofline": {"bound": "mfma", "achieved": round(flops / (ms * 1e-3) / 1e12, 2),
                     "unit": "TFLOP/s", "peak_bf16_mfma": BF16_PEAK_TFLOPS,
                     "peak_fp8_mfma": FP8_PEAK_TFLOPS,
                     "frac_bf16": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                     "frac_fp8": round(flops / (ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
                     "mfma_busy_fraction_gateup": read_mfma_util(),
                     "mfma_busy_source": "profiles/prefill_4096_grouped_gemm_mfma_counters.md "
                                         "(SQ_VALU_MFMA_BUSY_CYCLES / 4 SQ_BUSY_CU_CYCLES)"},
    }


def graph_time(fn, iters, replays=5):
    """ms per call of fn(i), i < iters, captured in one HIP graph (one eager
    warm-up pass first) and replayed `replays` times."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(iters):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / (replays * iters)


def cpu_loop(fn, seconds, max_calls=100000):
    """Seconds per call of fn() on the host: one warm-up call, then calls until
    `seconds` have elapsed."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= max_calls:
            return el / n, n


def bench_fp8_matvec(lib, cpu_seconds):
    """FP8 E4M3 matvec as the reference's CPU kernel path runs it (dsv4_gemv_fp8,
    src/dsv4/dsv4_ops.c:176-209): W [2048 x 4096] N(0, 0.02) quantised per
    128 x 128 block with fp32 absmax scales, x fp32 N(0, 1), seed 0. 48
    copies of W at distinct addresses rotate so that each call streams its
    matrix from HBM (48 x 8.4 MB exceeds the 256 MB last-level cache)."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    rows, cols, copies = 2048, 4096, 48
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    w = torch.randn(rows, cols, generator=g, device=dev) * 0.02
    x = torch.randn(cols, generator=g, device=dev)
    codes = torch.empty(copies, rows, cols, dtype=torch.uint8, device=dev)
    scales = torch.empty(copies, rows // 128, cols // 128, dtype=torch.float32, device=dev)
    lib.quant_fp8_blocks(w, codes[0], scales[0], mode=1)
    for i in range(1, copies):
        codes[i].copy_(codes[0])
        scales[i].copy_(scales[0])
    Y = torch.empty(copies, rows, dtype=torch.float32, device=dev)
    ms = graph_time(lambda i: lib.gemv_fp8_float(x, codes[i % copies], scales[i % copies], cols,
                                                 rows, 128, 0, y=Y[i % copies]), 4 * copies)
    nbytes = rows * cols + scales[0].numel() * 4 + cols * 4 + rows * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    r = {"workload": "FP8 E4M3 matvec 2048 x 4096, fp32 absmax 128x128 block scales, fp32 x "
                     "(dsv4_gemv_fp8; bit-exact unfused sequential chain per row)",
         "ms_per_call": round(ms, 5), "bytes_per_call": nbytes, "gbs": round(gbs, 1),
         "roofline": {"bound": "chain latency", "achieved": round(gbs, 1),
                      "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(gbs / HBM_PEAK_GBS, 4)},
         "note": "the products w*xs of 8 rows per workgroup are formed into LDS by all "
                 "waves; one lane per row then runs the reference's 4096 dependent adds "
                 "in column order (about 3.7 ns per add when fed from LDS, 2.6 from "
                 "registers), starting once the first half's products are in LDS: the "
                 "chain, not the 8.4 MB, bounds the call"}
    if cpu_seconds and cpu_available():
        ref = cpu_ref()
        xh, ch, sh = x.cpu().numpy(), codes[0].cpu().numpy(), scales[0].cpu().numpy()
        y_ref = ref.gemv_fp8_legacy(xh, ch, sh, cols, rows, 128)
        same = bool(np.array_equal(y_ref.view(np.uint32), Y[0].cpu().numpy().view(np.uint32)))
        sec, n = cpu_loop(lambda: ref.gemv_fp8_legacy(xh, ch, sh, cols, rows, 128), cpu_seconds)
        r["cpu_baseline"] = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": 1,
                             "kind": "reference", "ms_per_call": round(sec * 1e3, 3),
                             "gpu_output_bit_exact_vs_reference": same,
                             "sample": f"{n} calls of the reference dsv4_gemv_fp8 (oracle/_ref, "
                                       f"single-threaded as the reference kernel is) on the "
                                       f"same W and x"}
    return r


def bench_fp4_expert(lib, layer, cpu_seconds):
    """One FP4 expert's SwiGLU at one token (expert_forward,
    src/dsv4/dsv4_model.c:6289-6345): gate/up [2048 x 4096] and down
    [4096 x 2048] E2M1 with per-32 E8M0 scales, weights N(0, 0.02), x BF16
    N(0, 1). Calls rotate over the layer's 256 experts (3.4 GB), so each
    streams its 13.4 MB from HBM."""
    import numpy as np
    import torch
    import synth
    dev = torch.device("cuda:0")
    m = layer.meta
    stride, srun = m["expert_stride"], m["scale_run"]
    experts = layer.tensors["experts"]
    X = synth.bf16_tokens(1, H, seed=5, device=dev)
    qx, qs = lib.quant_fp8_act(X)
    iters = E
    OUT = torch.empty(iters, H, dtype=torch.float32, device=dev)
    ws = torch.empty(lib.expert_workspace_bytes(I), dtype=torch.uint8, device=dev)
    ms = graph_time(lambda i: lib.expert_forward(OUT[i], qx[0], qs[0],
                                                 experts[(i % E) * stride:(i % E + 1) * stride],
                                                 srun, H, I, m["swiglu_limit"], None, ws), iters)
    nbytes = EXPERT_BYTES + H * 4 + (H // 128) * 4 + H * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    r = {"workload": "FP4 E2M1 single-expert SwiGLU at 1 token: gate/up 2048 x 4096, down "
                     "4096 x 2048, per-32 E8M0 scales (expert_forward: paired FP4 GEMV "
                     "with the SwiGLU epilogue, then the FP4 down GEMV with the per-128 "
                     "FP8 requant folded in; two launches)",
         "ms_per_call": round(ms, 5), "bytes_per_call": nbytes, "gbs": round(gbs, 1),
         "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                      "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    if cpu_seconds and cpu_available():
        threads, _ = host_cores()
        set_omp_threads(threads)
        ref = cpu_ref()
        eh = experts[:8 * stride].cpu().numpy()
        qxh, qsh = qx[0].cpu().numpy(), qs[0].cpu().numpy()
        outs = OUT[:8].cpu().numpy()
        same = 0
        for e in range(8):
            sl = eh[e * stride:(e + 1) * stride]
            o = ref.expert_forward(qxh, qsh, sl[:srun], sl[srun:], H, I, m["swiglu_limit"], 1.0)
            same += int(np.array_equal(o.view(np.uint32), outs[e].view(np.uint32)))
        k = [0]

        def one():
            sl = eh[(k[0] % 8) * stride:(k[0] % 8 + 1) * stride]
            k[0] += 1
            ref.expert_forward(qxh, qsh, sl[:srun], sl[srun:], H, I, m["swiglu_limit"], 1.0)
        sec, n = cpu_loop(one, cpu_seconds)
        r["cpu_baseline"] = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s",
                             "cores": threads, "kind": "reference",
                             "ms_per_call": round(sec * 1e3, 3),
                             "gpu_outputs_bit_exact_vs_reference": f"{same}/8",
                             "sample": f"{n} calls of the reference expert_forward "
                                       f"(oracle/_ref, OMP_NUM_THREADS={threads}) over 8 "
                                       f"experts of the same layer and the same token"}
    return r


HC_MULT = 4                                   # hyper-connection streams
HC_MIX = (2 + HC_MULT) * HC_MULT              # 24 mixes per hc_pre
HC_K = HC_MULT * H                            # 16384 products per mix


def bench_ffn_step(lib, layers, cpu_seconds):
    """The FFN half of a decoder layer at one token (forward_loaded_layer,
    src/dsv4/dsv4_model.c:7549-7559) on device: hc_pre with its Sinkhorn split
    and the RMSNorm (24 exact fmaf chains of 16384 steps), the decode MoE
    layer, hc_post. State [4][4096] BF16 values; per layer its own hc_ffn_fn
    [24][16384] N(0, 0.01), scale, base and ffn_norm; the calls rotate over
    the decode layers like the decode benchmark."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    nl = len(layers)
    g = torch.Generator(device=dev)
    g.manual_seed(11)

    def bf16(t):
        return (t.view(torch.int32) & -65536).view(torch.float32)

    fn = [torch.randn(HC_MIX, HC_K, generator=g, device=dev) * 0.01 for _ in range(nl)]
    sc = [torch.rand(3, generator=g, device=dev) + 0.5 for _ in range(nl)]
    base = [torch.randn(HC_MIX, generator=g, device=dev) * 0.5 for _ in range(nl)]
    norm = [(bf16(1 + 0.1 * torch.randn(H, generator=g, device=dev)).view(torch.int32) >> 16)
            .to(torch.int16) for _ in range(nl)]
    state0 = bf16(torch.randn(1, HC_K, generator=g, device=dev) * 0.5)
    state = state0.clone()
    ws = torch.zeros(lib.ffn_step_workspace_bytes(layers[0], HC_MULT, 1), dtype=torch.uint8,
                     device=dev)
    iters = 8 * nl
    ms_step = graph_time(lambda i: lib.ffn_step(state, fn[i % nl], sc[i % nl], base[i % nl],
                                                norm[i % nl], layers[i % nl], HC_MULT,
                                                workspace=ws, check=False), iters)
    lib.check_decode_status(ws)
    b, po, co = lib.hc_pre(state, fn[0], sc[0], base[0], HC_MULT, norm[0])
    ms_pre = graph_time(lambda i: lib.hc_pre(state, fn[i % nl], sc[i % nl], base[i % nl],
                                             HC_MULT, norm[i % nl]), iters)
    st2 = state.clone()
    ms_post = graph_time(lambda i: lib.hc_post(st2, b, po, co, HC_MULT), iters)
    pre_bytes = HC_MIX * HC_K * 4 + HC_K * 4 + H * 2 + H * 4
    r = {"workload": "FFN half of a decoder layer at 1 token: hc_pre (24 mixes, each an exact "
                     "fmaf chain of 16384 steps) + Sinkhorn split + RMSNorm, the decode MoE "
                     "layer, hc_post; dsv4g_ffn_step, bit-exact",
         "ms_per_step": round(ms_step, 5), "ms_hc_pre_rmsnorm": round(ms_pre, 5),
         "ms_hc_post": round(ms_post, 5),
         "hc_pre_ns_per_chain_step": round(ms_pre * 1e6 / HC_K, 3),
         "roofline": {"bound": "fmaf chain latency (hc_pre)",
                      "achieved": round(pre_bytes / (ms_pre * 1e-3) / 1e9, 1),
                      "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(pre_bytes / (ms_pre * 1e-3) / 1e9 / HBM_PEAK_GBS, 5),
                      "note": "hc_pre streams 1.6 MB but its 16384-step dependent chains bound "
                              "it: 2.05-2.4 ns per step for a lone chain from registers on "
                              "gfx950 (a floor of about 34 us)"}}
    if cpu_seconds and cpu_available():
        threads, _ = host_cores()
        set_omp_threads(threads)
        ref = cpu_ref()
        import synth
        L = synth.host_copy(layers[0])
        fh, sch, bh = fn[0].cpu().numpy(), sc[0].cpu().numpy(), base[0].cpu().numpy()
        nh = norm[0].cpu().numpy().view(np.uint16)
        s0 = state0.cpu().numpy()[0]

        def one(st):
            x, post, comb = ref.hc_pre(st, fh, sch, bh, HC_MULT)
            x = ref.rmsnorm_bf16(x[None], nh, 1e-6, 1)[0]
            out, _, _ = ref.moe_forward(L, x)
            return ref.hc_post(st, out, post, comb, HC_MULT)
        want = one(s0)
        st = state0.clone()
        lib.ffn_step(st, fn[0], sc[0], base[0], norm[0], layers[0], HC_MULT, workspace=ws)
        same = bool(np.array_equal(want.view(np.uint32), st.cpu().numpy()[0].view(np.uint32)))
        sec, n = cpu_loop(lambda: one(s0), cpu_seconds)
        r["cpu_baseline"] = {"value": round(sec * 1e3, 3), "unit": "ms per step",
                             "cores": threads, "kind": "reference",
                             "gpu_output_bit_exact_vs_reference": same,
                             "sample": f"{n} steps of the reference hc_pre_scratch, "
                                       f"rmsnorm_bf16, moe_forward and hc_post_scratch "
                                       f"(oracle/_ref, OMP_NUM_THREADS={threads}) on layer 0 "
                                       f"and the same state"}
        del L
    return r


ATTN_PROJ = (("wq_a", 1024, 4096), ("wq_b", 32768, 1024), ("wkv", 512, 4096),
             ("wo_b", 4096, 8192))


def bench_attn_proj(lib, cpu_seconds):
    """The attention FP8 projections of one layer (src/dsv4/dsv4_internal.h:57-62)
    through dsv4_gemv_fp8_q (1 token) and dsv4_gemv_fp8_batch_q (5 tokens, the
    reference bench's dense batch, benchmarks/bench_dsv4_kernels.c:194-215):
    E4M3 weights N(0, 0.02) with 128 x 128 E8M0 scales, x BF16 N(0, 1)
    quantised per 128. Copies of each matrix rotate so that each call streams
    from HBM."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(21)
    out = {}
    total_ms = {1: 0.0, 5: 0.0}
    mats = {}
    for name, rows, cols in ATTN_PROJ:
        copies = max(2, min(24, (512 << 20) // (rows * cols)))
        w = torch.randn(rows, cols, generator=g, device=dev) * 0.02
        codes = torch.empty(copies, rows, cols, dtype=torch.uint8, device=dev)
        scales = torch.empty(copies, (rows + 127) // 128, (cols + 127) // 128,
                             dtype=torch.uint8, device=dev)
        lib.quant_fp8_blocks(w, codes[0], scales[0], mode=0)
        for i in range(1, copies):
            codes[i].copy_(codes[0])
            scales[i].copy_(scales[0])
        del w
        x = (torch.randn(5, cols, generator=g, device=dev).to(torch.bfloat16)
             .to(torch.float32).contiguous())
        qx, qs = lib.quant_fp8_act(x)
        r = {"shape": [rows, cols], "weight_bytes": rows * cols}
        for n in (1, 5):
            def call(i, n=n):
                if n == 1:
                    lib.gemv_fp8_q(qx[0], qs[0], codes[i % copies], scales[i % copies], cols, rows)
                else:
                    lib.gemv_fp8_batch_q(qx[:n], qs[:n], codes[i % copies], scales[i % copies],
                                         cols, rows)
            ms = graph_time(call, 4 * copies)
            total_ms[n] += ms
            r[f"ms_{n}_token" + ("s" if n > 1 else "")] = round(ms, 5)
            r[f"gbs_{n}_token" + ("s" if n > 1 else "")] = round(rows * cols / (ms * 1e-3) / 1e9,
                                                                   1)
        out[name] = r
        mats[name] = (codes[0].cpu().numpy(), scales[0].cpu().numpy(), qx.cpu().numpy(),
                      qs.cpu().numpy(), lib.gemv_fp8_q(qx[0], qs[0], codes[0], scales[0], cols,
                                                       rows).cpu().numpy())
        del codes, scales
    wbytes = sum(r * c for _, r, c in ATTN_PROJ)
    res = {"workload": "attention FP8 projections wq_a 1024x4096, wq_b 32768x1024, wkv "
                       "512x4096, wo_b 4096x8192 (dsv4_gemv_fp8_q / _batch_q, bit-exact)",
           "per_matrix": out, "weight_bytes": wbytes,
           "ms_1_token": round(total_ms[1], 5), "ms_5_tokens": round(total_ms[5], 5),
           "roofline": {"bound": "hbm", "achieved": round(wbytes / (total_ms[1] * 1e-3) / 1e9, 1),
                        "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(wbytes / (total_ms[1] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}}
    if cpu_seconds and cpu_available():
        threads, _ = host_cores()
        set_omp_threads(threads)
        ref = cpu_ref()
        same = 0
        sec = 0.0
        for name, rows, cols in ATTN_PROJ:
            W, S, qx, qs, y = mats[name]
            yr = ref.gemv_fp8_q(qx[0], qs[0], W, S, cols, rows)
            same += int(np.array_equal(yr.view(np.uint32), y.view(np.uint32)))
            s1, _ = cpu_loop(lambda: ref.gemv_fp8_q(qx[0], qs[0], W, S, cols, rows),
                             cpu_seconds / 4)
            sec += s1
        res["cpu_baseline"] = {"value": round(sec * 1e3, 3), "unit": "ms per token (4 matrices)",
                               "cores": threads, "kind": "reference",
                               "gpu_outputs_bit_exact_vs_reference": f"{same}/4",
                               "sample": f"the reference dsv4_gemv_fp8_q (oracle/_ref, "
                                         f"OMP_NUM_THREADS={threads}) on each matrix and the "
                                         f"same token, {cpu_seconds / 4:.1f} s each"}
    return res


def bench_vocab_head(lib, cpu_seconds):
    """The vocabulary head (head_logits / head_logits_batch,
    src/dsv4/dsv4_model.c:7313-7445) through dsv4_gemv_bf16: BF16 rows
    [129280][4096] N(0, 0.02), hidden states N(0, 1) rounded to BF16 values
    and held as fp32, fp32 logits; 1 token (decode) and 64 tokens (a verify
    batch). The 1.06 GB head exceeds every cache, so each call streams it
    from HBM. Bit-exact per-row fmaf chains in column order."""
    import numpy as np
    import torch
    import synth
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(33)
    W = torch.empty(VOCAB, H, dtype=torch.bfloat16, device=dev)
    for r0 in range(0, VOCAB, 16384):
        r1 = min(VOCAB, r0 + 16384)
        W[r0:r1] = (torch.randn(r1 - r0, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    Wu = W.view(torch.int16)
    X = synth.bf16_tokens(64, H, seed=9, device=dev)
    Y = torch.empty(64, VOCAB, dtype=torch.float32, device=dev)
    wbytes = VOCAB * H * 2
    res = {"workload": "vocabulary head 129280 x 4096 BF16, fp32 logits (dsv4_gemv_bf16; "
                       "1 token: coalesced 64 x 64 tiles transposed through LDS, a lane per "
                       "row, HBM-bound; 64 tokens: 4 rows x 16 tokens of chains per lane, x "
                       "from LDS, fp32-FMA-bound)", "weight_bytes": wbytes}
    for n in (1, 64):
        ms = graph_time(lambda i, n=n: lib.gemv_bf16_into(Y[:n], X[:n], Wu, H, VOCAB, 0),
                        8 if n == 1 else 2)
        nbytes = wbytes + n * H * 4 + n * VOCAB * 4
        gbs = nbytes / (ms * 1e-3) / 1e9
        tf = 2.0 * VOCAB * H * n / (ms * 1e-3) / 1e12
        r = {"ms_per_call": round(ms, 5), "bytes_per_call": nbytes, "gbs": round(gbs, 1),
             "tflops": round(tf, 2)}
        if n == 1:
            r["roofline"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                             "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}
        else:
            r["roofline"] = {"bound": "fp32 fma issue (the per-row chains are fmaf in column "
                                      "order, so no matrix-core form is exact)",
                             "achieved": round(tf, 2), "peak": FP32_FMA_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(tf / FP32_FMA_PEAK_TFLOPS, 4),
                             "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        res[f"{n}_token" + ("s" if n > 1 else "")] = r
    if cpu_seconds and cpu_available():
        threads, _ = host_cores()
        set_omp_threads(threads)
        ref = cpu_ref()
        Wh = Wu.cpu().numpy().view(np.uint16)
        Xh = X.cpu().numpy()
        for n in (1, 64):
            lib.gemv_bf16_into(Y[:n], X[:n], Wu, H, VOCAB, 0)
            got = Y[:n].cpu().numpy()
            yr = ref.head_logits(Xh[:n], Wh, threads)
            same = bool(np.array_equal(yr.view(np.uint32), got.view(np.uint32)))
            sec, calls = cpu_loop(lambda n=n: ref.head_logits(Xh[:n], Wh, threads),
                                  cpu_seconds / 2, max_calls=50)
            key = f"{n}_token" + ("s" if n > 1 else "")
            nbytes = res[key]["bytes_per_call"]
            res[key]["cpu_baseline"] = {
                "value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": threads,
                "kind": "reference", "ms_per_call": round(sec * 1e3, 3),
                "gpu_output_bit_exact_vs_reference": same,
                "sample": f"{calls} calls of the reference "
                          f"{'head_logits' if n == 1 else 'head_logits_batch'} (oracle/_ref, "
                          f"AVX2, OMP_NUM_THREADS={threads}) on the same head and tokens"}
        del Wh
    del W, Wu, Y
    return res


def bench_dropin(cpu_seconds):
    """The reference-named entry points on host buffers, called through the C
    ABI as a reference caller would (src/dsv4/dsv4_internal.h:261-272):
    dsv4_gemv_fp8_q at 2048 x 4096 (E4M3, 128 x 128 E8M0 scales) and
    dsv4_gemv_fp4_pair_q at one expert's gate/up shape (two 2048 x 4096 E2M1
    matrices, per-32 E8M0 scales), weights N(0, 0.02), x BF16 N(0, 1)
    quantised per 128. Every call copies its activations in and its outputs
    back and synchronises; unregistered weights are also copied from pageable
    host memory on every call, registered ones (dsv4_gpu_register_weights)
    stay in HBM. Host wall clock per call."""
    import ctypes as C
    import numpy as np
    import torch
    import dsv4_gpu
    dev = torch.device("cuda:0")
    glib = dsv4_gpu.lib()
    lib = C.CDLL(dsv4_gpu.LIB_PATH)
    f32p, u8p = C.POINTER(C.c_float), C.POINTER(C.c_uint8)
    lib.dsv4_gpu_register_weights.restype = C.c_int
    lib.dsv4_gpu_register_weights.argtypes = [C.c_void_p, C.c_size_t]
    lib.dsv4_gpu_forget_weights.argtypes = [C.c_void_p]
    P = lambda a, t: a.ctypes.data_as(t)
    g = torch.Generator(device=dev)
    g.manual_seed(41)
    rows, cols = 2048, 4096
    w = torch.randn(rows, cols, generator=g, device=dev) * 0.02
    c8 = torch.empty(rows, cols, dtype=torch.uint8, device=dev)
    s8 = torch.empty(rows // 128, cols // 128, dtype=torch.uint8, device=dev)
    glib.quant_fp8_blocks(w, c8, s8, mode=0)
    fp4 = []
    for _ in range(2):
        torch.randn(rows, cols, generator=g, device=dev, out=w)
        w.mul_(0.02)
        pk = torch.empty(rows, cols // 2, dtype=torch.uint8, device=dev)
        sc = torch.empty(rows, cols // 32, dtype=torch.uint8, device=dev)
        glib.quant_fp4_rows(w, pk, sc)
        fp4.append((pk.cpu().numpy(), sc.cpu().numpy()))
    W8, S8 = c8.cpu().numpy(), s8.cpu().numpy()
    x = synth_tokens(1, cols, 43)
    qx, qs = glib.quant_fp8_act(x)
    qx, qs = qx[0].cpu().numpy().copy(), qs[0].cpu().numpy().copy()
    del w, c8, s8
    y8 = np.empty(rows, np.float32)
    y0, y1 = np.empty(rows, np.float32), np.empty(rows, np.float32)
    (W0, S0), (W1, S1) = fp4

    def fp8():
        lib.dsv4_gemv_fp8_q(P(y8, f32p), P(qx, f32p), P(qs, f32p), P(W8, u8p), P(S8, u8p),
                            cols, rows, 1)

    def pair():
        lib.dsv4_gemv_fp4_pair_q(P(y0, f32p), P(y1, f32p), P(qx, f32p), P(qs, f32p),
                                 P(W0, u8p), P(S0, u8p), P(W1, u8p), P(S1, u8p), cols, rows)

    res = {"workload": "drop-in entry points on host buffers: dsv4_gemv_fp8_q 2048 x 4096 "
                       "E4M3 (8.4 MB) and dsv4_gemv_fp4_pair_q 2 x 2048 x 4096 E2M1 (8.9 MB), "
                       "activations in and outputs out through pageable host memory, one "
                       "synchronising call at a time"}
    wts = {"fp8_q": [W8, S8], "fp4_pair_q": [W0, S0, W1, S1]}
    fns = {"fp8_q": fp8, "fp4_pair_q": pair}
    outs = {}
    for name in ("fp8_q", "fp4_pair_q"):
        fn = fns[name]
        r = {"weight_bytes": int(sum(a.nbytes for a in wts[name]))}
        sec, n = cpu_loop(fn, 1.0, max_calls=2000)
        r["unregistered_ms"] = round(sec * 1e3, 4)
        for a in wts[name]:
            assert lib.dsv4_gpu_register_weights(a.ctypes.data, a.nbytes) == 0
        sec, n = cpu_loop(fn, 1.0, max_calls=20000)
        r["registered_ms"] = round(sec * 1e3, 4)
        fn()
        outs[name] = (y8.copy(),) if name == "fp8_q" else (y0.copy(), y1.copy())
        for a in wts[name]:
            lib.dsv4_gpu_forget_weights(C.c_void_p(a.ctypes.data))
        res[name] = r
    if cpu_seconds and cpu_available():
        threads, _ = host_cores()
        set_omp_threads(threads)
        ref = cpu_ref()
        yr = ref.gemv_fp8_q(qx, qs, W8, S8, cols, rows)
        res["fp8_q"]["bit_exact_vs_reference"] = bool(
            np.array_equal(yr.view(np.uint32), outs["fp8_q"][0].view(np.uint32)))
        sec, _ = cpu_loop(lambda: ref.gemv_fp8_q(qx, qs, W8, S8, cols, rows), cpu_seconds / 4)
        res["fp8_q"]["reference_cpu_ms"] = round(sec * 1e3, 4)
        r0, r1 = ref.gemv_fp4_pair_q(qx, qs, W0, S0, W1, S1, cols, rows)
        res["fp4_pair_q"]["bit_exact_vs_reference"] = bool(
            np.array_equal(r0.view(np.uint32), outs["fp4_pair_q"][0].view(np.uint32)) and
            np.array_equal(r1.view(np.uint32), outs["fp4_pair_q"][1].view(np.uint32)))
        sec, _ = cpu_loop(lambda: ref.gemv_fp4_pair_q(qx, qs, W0, S0, W1, S1, cols, rows),
                          cpu_seconds / 4)
        res["fp4_pair_q"]["reference_cpu_ms"] = round(sec * 1e3, 4)
        res["reference_cpu"] = (f"the reference kernels (oracle/_ref, OMP_NUM_THREADS={threads}) "
                                f"on the same host buffers")
    return res


def synth_tokens(n, hidden, seed):
    import synth
    return synth.bf16_tokens(n, hidden, seed=seed, device="cuda")


def bench_checkpoint_load(lib, layer):
    """Checkpoint to HBM (dsv4g_load_moe_layer): 16 full-size routed experts of
    one layer, its FP8 shared expert, gate and bias, written as three
    safetensors shards with the checkpoint's tensor names to a temporary
    directory, then loaded twice; the second load is timed (page cache
    warm, so the rate is the loader's, not the disk's)."""
    import shutil
    import tempfile
    import numpy as np
    import torch
    import dsv4_gpu
    from st_writer import moe_layer_tensors, write_checkpoint
    import synth
    n_exp = 16
    L = synth.host_copy(layer)
    stride = L["expert_stride"]
    L = dict(L, n_experts=n_exp, experts=L["experts"][:n_exp * stride],
             gate_w=L["gate_w"][:n_exp], bias=np.zeros(n_exp, np.float32))
    d = tempfile.mkdtemp(prefix="dsv4_ckpt_")
    try:
        write_checkpoint(d, moe_layer_tensors(L, "layers", 3), n_shards=3)
        ck = dsv4_gpu.Checkpoint(d)
        meta = {k: L[k] for k in ("hidden", "inter", "n_experts", "topk", "route_scale",
                                  "swiglu_limit")}
        ck.load_moe_layer(meta, "layers", 3)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        loaded = ck.load_moe_layer(meta, "layers", 3)
        sec = time.perf_counter() - t0
        nbytes = sum(t["nbytes"] for t in ck.tensors())
        same = bool(np.array_equal(loaded.arena[:n_exp * stride].cpu().numpy(), L["experts"]))
        ck.close()
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return {"workload": f"{n_exp} full-size routed experts + FP8 shared expert + gate/bias of "
                        f"one layer, 3 safetensors shards -> one HBM arena "
                        f"(dsv4g_load_moe_layer), page cache warm",
            "bytes": nbytes, "ms": round(sec * 1e3, 3),
            "gbs": round(nbytes / sec / 1e9, 2), "arena_experts_match_source": same,
            "note": "file -> pinned staging -> HBM; a cold load is bound by the disk"}


def cpu_available():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    return pyoracle.ref_available()


def cpu_ref():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    return pyoracle.RefLib()


def cpu_batch_baseline(layer_host, n_tokens, flops_per_token, seconds):
    """The reference moe_forward_batch (oracle/_ref) on the host in chunks of 32
    tokens (its batch limit is 33), on the same Zipf-biased layer: tokens per
    second and the TFLOP/s that rate is worth."""
    import numpy as np
    threads, hw = host_cores()
    set_omp_threads(threads)
    ref = cpu_ref()
    rng = np.random.default_rng(11 + n_tokens)
    x = rng.standard_normal((32, H)).astype(np.float32)
    x = (x.view(np.uint32) + 0x7FFF + ((x.view(np.uint32) >> 16) & 1)) & 0xFFFF0000
    x = x.view(np.float32)
    sec, n = cpu_loop(lambda: ref.moe_forward_batch(layer_host, x), seconds, max_calls=50)
    tps = 32 / sec
    return {"value": round(tps * flops_per_token / 1e12, 5), "unit": "TFLOP/s",
            "cores": threads, "kind": "reference", "tokens_per_s": round(tps, 1),
            "host": hw,
            "sample": f"{n} calls of the reference moe_forward_batch on 32 BF16 tokens "
                      f"(oracle/_ref, OMP_NUM_THREADS={threads}) of the same layer (256 FP4 "
                      f"experts + FP8 shared, the same Zipf router bias), after one warm-up "
                      f"call; the rate stands for the {n_tokens}-token workload"}


def host_cores():
    """Threads for the CPU legs: the box's CPU share (OMP_NUM_THREADS where set,
    else the CPUs this process may run on), with what the host reports."""
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    env = os.environ.get("OMP_NUM_THREADS")
    threads = int(env) if env and env.isdigit() else (avail or 1)
    return threads, {"nproc": os.cpu_count(), "affinity_cpus": avail,
                     "omp_num_threads_env": env}


def set_omp_threads(n):
    """OpenMP team size for the reference's parallel regions started from this
    thread (libgomp read OMP_NUM_THREADS when torch loaded it already)."""
    import ctypes
    try:
        ctypes.CDLL("libgomp.so.1").omp_set_num_threads(int(n))
    except OSError:
        pass


def cpu_baseline(layer_dev, tokens, gpu_out, seconds):
    """Reference moe_forward (compiled from the reference sources) on the host
    on the tokens the GPU decoded through the same layer: each GPU output is
    compared bit for bit with the reference's, then tokens are repeated until
    `seconds` have elapsed (one warm-up token first)."""
    threads, hw = host_cores()
    set_omp_threads(threads)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "deepseek-v4-flash-0731-in-c_amd", "python"))
    import numpy as np
    import pyoracle
    import synth
    if not pyoracle.ref_available():
        return None
    ref = pyoracle.RefLib()
    L = synth.host_copy(layer_dev)
    x = tokens.cpu().numpy()
    go = gpu_out.cpu().numpy()
    o, _, _ = ref.moe_forward(L, x[0])
    same = int(np.array_equal(o.view(np.uint32), go[0].view(np.uint32)))
    checked = 1
    n, t0 = 0, time.perf_counter()
    while True:
        i = (n + 1) % x.shape[0]
        o, _, _ = ref.moe_forward(L, x[i])
        if n + 1 < x.shape[0]:
            same += int(np.array_equal(o.view(np.uint32), go[i].view(np.uint32)))
            checked += 1
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n + 1 >= x.shape[0]) or n >= 2000:
            break
    sec = el / n
    return {"value": round(DECODE_BYTES / sec / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "reference", "ms_per_step": round(sec * 1e3, 3), "host": hw,
            "gpu_outputs_bit_exact_vs_reference": f"{same}/{checked}",
            "sample": f"{n} decode tokens through the reference moe_forward (oracle/_ref, built "
                      f"from src/dsv4/*.c with -O3 -mavx2 -mfma -fopenmp) on one full "
                      f"synthetic layer (256 FP4 experts + FP8 shared), OMP_NUM_THREADS="
                      f"{threads}, after one warm-up token; the tokens are those the GPU "
                      f"decoded through this layer, whose outputs are compared bit for bit"}


def ref_kernel_bench():
    """The reference's kernel microbenchmark binary, built from its sources."""
    exe = os.path.join(ROOT, "oracle", "_ref", "bench_dsv4_kernels")
    if not os.path.exists(exe):
        return None
    import subprocess
    env = dict(os.environ, OMP_NUM_THREADS=str(host_cores()[0]))
    out = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300).stdout
    res, name = {}, None
    for ln in out.splitlines():
        if ln.startswith("bench_dsv4: "):
            name = ln[len("bench_dsv4: "):]
        elif name and "ms" in ln:
            res[name] = float(ln.split()[0])
            name = None
    return res


def read_traffic():
    """HBM bytes per k_dec_front launch from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the reading of a 1 GiB
    device copy); None if that summary is absent."""
    p = os.path.join(ROOT, "profiles", "k_dec_front_hbm_traffic.md")
    if not os.path.exists(p):
        return None
    for ln in open(p):
        if ln.startswith("traffic_bytes_per_launch:"):
            return {"bytes": int(ln.split(":")[1]),
                    "source": "profiles/k_dec_front_hbm_traffic.md (rocprofv3 --pmc "
                              "FETCH_SIZE, WRITE_SIZE; copy-calibrated)"}
    return None


def read_mfma_util():
    """MFMA-busy fraction of the FP4 grouped gate/up GEMM from the committed
    rocprofv3 --pmc summary; None if that summary is absent."""
    p = os.path.join(ROOT, "profiles", "prefill_4096_grouped_gemm_mfma_counters.md")
    if not os.path.exists(p):
        return None
    for ln in open(p):
        if ln.startswith("mfma_utilisation_k_grouped_gateup_fp4:"):
            return float(ln.split(":")[1])
    return None


def bench_decode(args, lib, layers):
    """Graph-replayed decode steps over the rotated layers; returns the
    per-step and gate/up-pass times and the graph/eager agreement."""
    import torch
    import dsv4_gpu
    import synth
    dev = torch.device("cuda:0")
    nl = len(layers)
    nsteps = args.steps
    X = synth.bf16_tokens(nsteps + args.warmup, H, seed=7, device=dev)
    OUT = torch.empty_like(X)
    wsb = lib.moe_workspace_bytes(layers[0], 1)
    wsb = (wsb + 4095) // 4096 * 4096
    WS = torch.empty(nsteps + args.warmup, wsb, dtype=torch.uint8, device=dev)
    for i in range(nsteps + args.warmup):
        lib.moe_workspace_init(WS[i])

    def step(i, phases=None, fast=False):
        L = layers[i % nl]
        if phases is None:  # the fused entry
            lib.moe_forward_into(L, X[i:i + 1], OUT[i:i + 1], WS[i], fast=fast)
        else:
            for ph in phases:
                lib.moe_decode_phase(ph, L, X[i:i + 1], OUT[i:i + 1], WS[i])

    # eager warm-up, then capture the K timed steps in one graph
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(args.warmup):
            step(nsteps + i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(nsteps):
            step(i)
    graph.replay()
    torch.cuda.synchronize()
    ref_out = OUT[:nsteps].clone()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(args.replays):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    ms_step = ev0.elapsed_time(ev1) / (args.replays * nsteps)
    replay_ok = bool(torch.equal(OUT[:nsteps], ref_out))

    # eager re-run of a few steps must match the replayed graph
    chk = torch.empty_like(OUT[:4])
    for i in range(4):
        L = layers[i % nl]
        for ph in range(dsv4_gpu.DECODE_PHASES):  # the launches in order
            lib.moe_decode_phase(ph, L, X[i:i + 1], chk[i:i + 1], WS[i])
    torch.cuda.synchronize()
    eager_ok = bool(torch.equal(chk, ref_out[:4]))

    # the tolerance mode (dsv4g_moe_forward_fast), same steps
    g3 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g3):
        for i in range(nsteps):
            step(i, fast=True)
    g3.replay()
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(args.replays):
        g3.replay()
    ev1.record()
    torch.cuda.synchronize()
    ms_fast = ev0.elapsed_time(ev1) / (args.replays * nsteps)
    del g3
    # rerun the exact steps so the routing held per step is the exact one
    for i in range(nsteps):
        step(i)
    torch.cuda.synchronize()

    # dominant kernel: the front launch (phase 1) of every step, timed in a
    # graph of its own. It reads what the route launch (phase 0) left in each
    # step's workspace, which only the back launch (phase 2) clears, so
    # phase 0 runs once for every step first and the front graph replays
    # on those records; phase 2 then cleans every workspace.
    for i in range(nsteps):
        step(i, phases=(0,))
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        for i in range(nsteps):
            step(i, phases=(1,))
    g2.replay()
    torch.cuda.synchronize()
    ms_front = 0.0
    for _ in range(args.replays):
        ev0.record()
        g2.replay()
        ev1.record()
        torch.cuda.synchronize()
        ms_front += ev0.elapsed_time(ev1)
    ms_front /= args.replays * nsteps
    for i in range(nsteps):
        step(i, phases=tuple(range(2, dsv4_gpu.DECODE_PHASES)))
    torch.cuda.synchronize()
    status = sum(lib.decode_status(WS[i]) for i in range(nsteps))
    del graph, g2
    return ms_step, ms_front, ms_fast, eager_ok and replay_ok and status == 0, X, OUT


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              f"(the multi-GPU expert-parallel design is described, not built)", file=sys.stderr)
        sys.exit(2)
    import torch
    import dsv4_gpu
    import synth

    dev = torch.device("cuda:0")
    lib = dsv4_gpu.lib()
    wl = args.workload
    cpu_s = 0.0 if args.no_cpu else min(args.cpu_seconds, 6.0)
    if wl == "head":
        print(json.dumps({"vocab_head": bench_vocab_head(lib, cpu_s)}))
        return
    if wl == "dropin":
        print(json.dumps({"dropin": bench_dropin(cpu_s)}))
        return
    nl = args.layers if wl in ("all", "decode") else 1
    t0 = time.perf_counter()
    layers = [synth.device_layer(seed=100 + l, device=dev) for l in range(nl)]
    torch.cuda.synchronize()
    gen_s = time.perf_counter() - t0

    kernels = {}
    if wl in ("all", "kernels"):
        kernels["fp8_matvec_2048x4096"] = bench_fp8_matvec(lib, cpu_s)
        kernels["fp4_expert_1_token"] = bench_fp4_expert(lib, layers[0], cpu_s)
        kernels["ffn_step_1_token"] = bench_ffn_step(lib, layers, cpu_s)
        kernels["attention_projections"] = bench_attn_proj(lib, cpu_s)
        kernels["vocab_head"] = bench_vocab_head(lib, cpu_s)
        kernels["dropin_host_buffers"] = bench_dropin(cpu_s)
        kernels["checkpoint_load"] = bench_checkpoint_load(lib, layers[0])
        if wl == "kernels":
            print(json.dumps(kernels))
            return

    batch = {}
    if wl in ("all", "verify", "prefill"):
        zb = zipf_bias(E, strength=args.zipf_strength)
        zl = layers[0].with_bias(torch.from_numpy(zb).to(dev))
        if wl in ("all", "verify"):
            batch["verify_64"] = bench_batch(lib, zl, 64, 50)
        if wl in ("all", "prefill"):
            batch["prefill_4096"] = bench_batch(lib, zl, 4096, 10)
        for v in batch.values():
            v["router"] = (f"Zipf(1.2) expert skew: bias {args.zipf_strength} * centred "
                           f"log rank^-1.2 over a seeded expert permutation")
        if cpu_s and cpu_available():
            Lh = synth.host_copy(layers[0])
            Lh["bias"] = zb
            for v in batch.values():
                fpt = v["expert_flops"] / v["tokens"]
                v["cpu_baseline"] = cpu_batch_baseline(Lh, v["tokens"], fpt, 2 * cpu_s)
                v["speedup_vs_cpu"] = round(v["tflops"] / v["cpu_baseline"]["value"], 1)
            del Lh

    if wl in ("verify", "prefill"):
        key = "verify_64" if wl == "verify" else "prefill_4096"
        r = batch[key]
        result = {
            "metric": METRIC, "value": r["tflops"], "unit": "TFLOP/s", "n_gpus": 1,
            "steps": r["iters"], "warmup": 1, "ms_per_step": r["ms_per_layer"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16 MFMA operands (exact FP4/FP8 x E8M0 values), fp32 accumulate",
            "data": "synthetic",
            "config": dict(workload=f"{key}: {r['tokens']} tokens through one MoE layer (256 "
                                    f"FP4 experts top-6 + FP8 shared), grouped GEMMs", **r),
            "roofline": {"bound": "mfma", "achieved": r["tflops"], "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": r["frac_bf16_mfma_peak"], "traffic": None},
        }
        if "cpu_baseline" in r:
            result["cpu_baseline"] = r["cpu_baseline"]
        print(json.dumps(result))
        return

    ms_step, ms_front, ms_fast, graph_ok, X, OUT = bench_decode(args, lib, layers)
    if args.copy_calibration:
        src = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    traffic = read_traffic()
    value = DECODE_BYTES / (ms_step * 1e-3) / 1e9
    achieved = FRONT_BYTES / (ms_front * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32-accumulate (fp4-e2m1 / fp8-e4m3 weights x fp8-e4m3 activations)",
        "data": "synthetic",
        "config": {
            "workload": "MoE layer decode, 1 token: hidden 4096, 256 routed FP4 experts "
                        "(inter 2048) top-6 sqrt-softplus router + 1 shared FP8 expert, all "
                        "weights in HBM; 8 seeded layers (27.6 GB) rotated per step",
            "hbm_frac": round(value / HBM_PEAK_GBS, 4),
            "mode": "dsv4g_moe_forward: bit-exact (outputs, indices, weights) with the reference",
            "fast_mode": {
                "entry": "dsv4g_moe_forward_fast: indices identical, weights from the parallel "
                         "router logits when the candidates are exactly top-k",
                "ms_per_step": round(ms_fast, 5),
                "value_gbs": round(DECODE_BYTES / (ms_fast * 1e-3) / 1e9, 2),
                "hbm_frac": round(DECODE_BYTES / (ms_fast * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            },
            "algorithmic_bytes_per_step": DECODE_BYTES,
            "algorithmic_flops_per_step": DECODE_FLOPS,
            "layers_rotated": nl,
            "graph_replay_matches_eager": graph_ok,
            "layer_generation_s": round(gen_s, 2),
            **kernels,
            **batch,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "k_dec_front (candidates, exact router chains and top-k, 6 routed FP4 "
                      "gate/up pairs with the SwiGLU epilogue, the shared FP8 expert's down)",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic["bytes"] if traffic else None,
            "traffic_source": traffic["source"] if traffic else None,
            "bytes_per_launch": FRONT_BYTES,
            "ms_per_launch": round(ms_front, 5),
        },
    }
    if not args.no_cpu:
        # the steps the GPU ran through layer 0 (step i uses layer i % nl)
        cb = cpu_baseline(layers[0], X[:args.steps:nl], OUT[:args.steps:nl], args.cpu_seconds)
        if cb:
            result["cpu_baseline"] = cb
            result["config"]["speedup_vs_cpu"] = round(value / cb["value"], 1)
        kb = ref_kernel_bench()
        if kb:
            result["config"]["reference_kernel_bench_ms"] = kb
    print(json.dumps(result))


if __name__ == "__main__":
    main()
