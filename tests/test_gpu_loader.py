"""GPU tests of the checkpoint-to-HBM loader (dsv4g_load_moe_layer).

A layer written as safetensors shards with the reference's tensor names
(src/dsv4/dsv4_model.c:2014-2053, 3063-3136) is loaded into one device arena;
every byte of the arena is checked against the source tensors (read back
through the reference reader k3_st where oracle/_ref is built, else from the
files), and the MoE layer run on the loaded weights is checked bit for bit
against the oracle. The reference's tiny checkpoint (tests/fixtures/tiny_dsv4,
copied as data into tests/golden/) is loaded layer by layer the same way.
"""
from __future__ import annotations

import os
import time

import numpy as np
import pytest

from common import (ROOT, bf16_input, expert_geometry, make_layer, max_rel_err, moe_layer_tensors,
                    pyoracle, same_bits, write_checkpoint)

pytestmark = pytest.mark.gpu

TINY_DIR = os.path.join(ROOT, "tests", "golden", "tiny_dsv4")


@pytest.fixture(scope="module")
def env():
    import torch
    import dsv4_gpu
    return dict(torch=torch, lib=dsv4_gpu.lib(), orc=pyoracle.Oracle(),
                dev=torch.device("cuda:0"), dg=dsv4_gpu)


def meta_of(layer):
    return {k: layer[k] for k in ("hidden", "inter", "n_experts", "topk", "route_scale",
                                  "swiglu_limit")}


def check_arena(loaded, layer):
    """Every piece of the arena equals the layer's bytes; padding is zero."""
    A = loaded.arena.cpu().numpy()
    H, I, E = layer["hidden"], layer["inter"], layer["n_experts"]
    g = expert_geometry(H, I)
    stride = loaded.struct.expert_stride
    assert loaded.struct.scale_run == g["scale_run"]
    assert stride >= g["stride"] and stride % 256 == 0
    assert loaded.offset("experts") == 0
    used = np.zeros(A.size, bool)
    for e in range(E):
        slot = A[e * stride:(e + 1) * stride]
        want = layer["experts"][e * g["stride"]:(e + 1) * g["stride"]]
        assert np.array_equal(slot[:g["stride"]], want), f"expert {e}"
        used[e * stride:e * stride + g["stride"]] = True
    pieces = [("gate_w", layer["gate_w"])]
    if layer.get("tid2eid") is not None:
        pieces.append(("tid2eid", layer["tid2eid"]))
        assert loaded.struct.bias is None
    else:
        pieces.append(("bias", layer["bias"]))
        assert loaded.struct.tid2eid is None
    for k in ("sh1", "sh1_s", "sh3", "sh3_s", "sh2", "sh2_s"):
        pieces.append((k, layer[k]))
    for k, v in pieces:
        raw = np.frombuffer(np.ascontiguousarray(v).tobytes(), np.uint8)
        o = loaded.offset(k)
        assert o % 256 == 0, k
        assert np.array_equal(A[o:o + raw.size], raw), k
        used[o:o + raw.size] = True
    assert not A[~used].any(), "padding not cleared"


def run_both(env, L_host, layer_dev, n_tok=3, seed=5, token_ids=None):
    torch, lib, orc = env["torch"], env["lib"], env["orc"]
    X = bf16_input(np.random.default_rng(seed), (n_tok, L_host["hidden"]))
    tok = None if token_ids is None else torch.from_numpy(token_ids).to(env["dev"])
    out, idx, wt = lib.moe_forward(layer_dev, torch.from_numpy(X).to(env["dev"]), tok)
    out, idx, wt = out.cpu().numpy(), idx.cpu().numpy(), wt.cpu().numpy()
    for t in range(n_tok):
        o, i, w = orc.moe_forward(L_host, X[t], 0 if token_ids is None else int(token_ids[t]))
        assert np.array_equal(idx[t], i), t
        assert same_bits(wt[t], w), t
        assert same_bits(out[t], o), (t, max_rel_err(out[t], o))


@pytest.mark.parametrize("order,shards", [("reference", 1), ("reference", 3), ("scrambled", 4)])
def test_load_layer_bytes_and_forward(env, tmp_path, order, shards):
    """Reference file order (runs contiguous, read as long spans) and a
    scrambled order (tensors assembled by name) give the same arena, and the
    MoE layer on it is bit-identical to the oracle."""
    orc, dg = env["orc"], env["dg"]
    L = make_layer(orc, 256, 128, 16, 6, seed=3, bias=True)
    extra = [("layers.2.attn_norm.weight", "BF16", (256,), bytes(512)),
             ("layers.1.ffn.gate.bias", "F32", (16,), bytes(64))]
    tensors = extra[:1] + moe_layer_tensors(L, "layers", 2, order=order, seed=9) + extra[1:]
    d = str(tmp_path / "ckpt")
    write_checkpoint(d, tensors, n_shards=shards)
    ck = dg.Checkpoint(d)
    loaded = ck.load_moe_layer(meta_of(L), "layers", 2, device=env["dev"])
    check_arena(loaded, L)
    run_both(env, L, loaded)


def test_load_hash_layer_mtp_scope(env, tmp_path):
    """A hash-routed layer (tid2eid [vocab][topk] in place of the bias) under
    the "mtp" scope."""
    orc, dg = env["orc"], env["dg"]
    L = make_layer(orc, 256, 128, 16, 6, seed=4, hash_vocab=50)
    d = str(tmp_path / "hash")
    write_checkpoint(d, moe_layer_tensors(L, "mtp", 1), n_shards=2)
    ck = dg.Checkpoint(d)
    loaded = ck.load_moe_layer(meta_of(L), "mtp", 1, is_hash=True, vocab=50, device=env["dev"])
    check_arena(loaded, L)
    run_both(env, L, loaded, n_tok=4, token_ids=np.array([0, 7, 49, 23], np.int32))


def test_load_full_size_layer(env, tmp_path):
    """hidden 4096, inter 2048 (13,369,344-byte experts, FP8 shared expert
    of 25 MB) with 12 experts over 3 shards: arena exact, decode bit-exact.
    Prints the file-to-HBM rate of the load."""
    orc, dg, torch = env["orc"], env["dg"], env["torch"]
    L = make_layer(orc, 4096, 2048, 12, 6, seed=21, bias=True)
    d = str(tmp_path / "full")
    write_checkpoint(d, moe_layer_tensors(L, "layers", 5), n_shards=3)
    ck = dg.Checkpoint(d)
    meta = meta_of(L)
    loaded = ck.load_moe_layer(meta, "layers", 5, device=env["dev"])  # warm page cache
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    loaded = ck.load_moe_layer(meta, "layers", 5, device=env["dev"])
    dt = time.perf_counter() - t0
    nbytes = sum(t["nbytes"] for t in ck.tensors())
    print(f"\nloader: {nbytes / 1e6:.1f} MB file->HBM in {dt * 1e3:.1f} ms "
          f"({nbytes / dt / 1e9:.2f} GB/s, page cache warm)", flush=True)
    check_arena(loaded, L)
    run_both(env, L, loaded, n_tok=2)


def test_load_reference_tiny_checkpoint(env):
    """The reference's tiny DeepSeek-V4 checkpoint (hidden 8, moe_inter 4,
    4 experts, top-2; I8 / F8_E4M3 / F8_E8M0 / BF16 / F32 tensors): each of its
    four layers loads, and every arena piece equals the tensor bytes the
    reference reader returns."""
    dg = env["dg"]
    ck = dg.Checkpoint(TINY_DIR)
    ref = pyoracle.RefSt(pyoracle.RefLib(), TINY_DIR) if pyoracle.ref_available() else None
    read = ref.read if ref is not None else ck.read
    meta = dict(hidden=8, inter=4, n_experts=4, topk=2, route_scale=1.5, swiglu_limit=10.0)
    for layer in range(4):
        loaded = ck.load_moe_layer(meta, "layers", layer, device=env["dev"])
        A = loaded.arena.cpu().numpy()
        pre = f"layers.{layer}."

        def piece(field, name):
            raw = np.frombuffer(read(pre + name), np.uint8)
            o = loaded.offset(field)
            assert np.array_equal(A[o:o + raw.size], raw), (layer, name)

        piece("gate_w", "ffn.gate.weight")
        piece("bias", "ffn.gate.bias")
        for m, f in (("w1", "sh1"), ("w3", "sh3"), ("w2", "sh2")):
            piece(f, f"ffn.shared_experts.{m}.weight")
            piece(f + "_s", f"ffn.shared_experts.{m}.scale")
        stride, run = loaded.struct.expert_stride, loaded.struct.scale_run
        for e in range(4):
            s = b"".join(read(pre + f"ffn.experts.{e}.w{k}.scale") for k in (1, 2, 3))
            w = b"".join(read(pre + f"ffn.experts.{e}.w{k}.weight") for k in (1, 2, 3))
            assert run == len(s)
            slot = A[e * stride:e * stride + len(s) + len(w)].tobytes()
            assert slot == s + w, (layer, e)


def test_loader_errors(env, tmp_path):
    """Missing tensor, wrong dtype, wrong shape, arena too small: refused
    with the reference's messages, before anything is copied."""
    orc, dg, torch = env["orc"], env["dg"], env["torch"]
    import ctypes as C
    L = make_layer(orc, 256, 128, 4, 2, seed=1, bias=True)
    good = moe_layer_tensors(L, "layers", 0)
    meta = meta_of(L)

    def load(tensors, name):
        d = str(tmp_path / name)
        write_checkpoint(d, tensors)
        return dg.Checkpoint(d).load_moe_layer(meta, "layers", 0, device=env["dev"])

    with pytest.raises(RuntimeError, match="missing tensor layers.0.ffn.experts.3.w2.scale"):
        load([t for t in good if t[0] != "layers.0.ffn.experts.3.w2.scale"], "missing")
    bad = [(n, "F32" if n.endswith("gate.weight") else dt,
            (s[0], s[1] // 2) if n.endswith("gate.weight") else s, r) for n, dt, s, r in good]
    with pytest.raises(RuntimeError, match="ffn.gate.weight has dtype F32, want BF16"):
        load(bad, "dtype")
    bad = [(n, dt, (s[0] * 2, s[1] // 2) if n.endswith("experts.1.w1.weight") else s, r)
           for n, dt, s, r in good]
    with pytest.raises(RuntimeError, match=r"experts.1.w1.weight shape\[0\]=256, want 128"):
        load(bad, "shape")
    with pytest.raises(RuntimeError, match="missing tensor layers.0.ffn.gate.tid2eid"):
        d = str(tmp_path / "nohash")
        write_checkpoint(d, good)
        dg.Checkpoint(d).load_moe_layer(meta, "layers", 0, is_hash=True, vocab=8,
                                        device=env["dev"])
    ck = dg.Checkpoint(str(tmp_path / "missing"))
    S = dg.DSV4GLayer()
    S.hidden, S.inter, S.n_experts, S.topk = 256, 128, 4, 2
    small = torch.empty(1024, dtype=torch.uint8, device=env["dev"])
    rc = ck.lib.dsv4g_load_moe_layer(C.byref(S), C.c_void_p(small.data_ptr()), 1024, ck.h,
                                     b"layers", 0, 0, 0, None)
    assert rc == 1 and "arena holds 1024 bytes" in ck.lib.dsv4g_last_error().decode()


def test_st_upload_one_tensor(env):
    dg, torch = env["dg"], env["torch"]
    ck = dg.Checkpoint(TINY_DIR)
    name = "layers.1.attn.wq_a.weight"
    dst = torch.zeros(64, dtype=torch.uint8, device=env["dev"])
    ck.upload(name, dst)
    raw = ck.read(name)
    assert dst.cpu().numpy()[:len(raw)].tobytes() == raw
    assert not dst.cpu().numpy()[len(raw):].any()
