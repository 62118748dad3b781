"""Decode wait failures reach the caller.

Every cross-workgroup wait of the decode kernels is bounded: one that runs
out (or that sees the sticky status word already set, checked every 64
polls) leaves its workgroup, sets the word, and the kernels end normally.
These tests set that word from the host before a call, so every wait gives
up at its first status check; no kernel is made to fault or hang. Then:

* the caller of INTEGRATION.md section 1 (tests/integration_caller.c, the
  same function compiled as it stands) takes the reference's fatal path:
  a message on stderr and exit(1);
* the Python binding raises, and re-initialises the workspace, after which
  the next call is bit-exact again;
* the no-allocation entry's status query reads 0 after normal calls.

The caller is compiled with gcc here (a host program; the library is the
prebuilt lib/libdsv4_gpu.so).
"""
from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

from common import ROOT, bf16_input, make_layer, pyoracle, same_bits

LIBDIR = os.path.join(ROOT, "deepseek-v4-flash-0731-in-c_amd", "lib")
SRC = os.path.join(ROOT, "tests", "integration_caller.c")


def build_caller(tmp_path):
    exe = str(tmp_path / "integration_caller")
    subprocess.run(["gcc", "-O1", "-std=c99", "-Wall", "-Werror", "-I",
                    os.path.join(ROOT, "include"), SRC, "-o", exe, "-L", LIBDIR,
                    "-ldsv4_gpu", f"-Wl,-rpath,{LIBDIR}"], check=True)
    return exe


def test_integration_caller_compiles(tmp_path):
    """The INTEGRATION.md caller compiles against include/dsv4_gpu.h and
    links against the library (no GPU needed)."""
    assert os.path.exists(os.path.join(LIBDIR, "libdsv4_gpu.so"))
    assert os.path.exists(build_caller(tmp_path))


@pytest.mark.gpu
def test_integration_caller_exits_on_wait_failure(tmp_path):
    exe = build_caller(tmp_path)
    print("integration caller: plain call", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert r.stdout.startswith("ok")
    print("integration caller: status word preset by the host", flush=True)
    r = subprocess.run([exe, "preset"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1, (r.returncode, r.stdout, r.stderr)
    assert "MoE decode failed on the GPU (status 0x1)" in r.stderr
    assert not r.stdout.startswith("ok")


@pytest.mark.gpu
def test_python_caller_raises_then_recovers():
    import torch
    import dsv4_gpu

    dev = torch.device("cuda:0")
    orc = pyoracle.Oracle()
    lib = dsv4_gpu.lib()
    L = make_layer(orc, 256, 128, 16, 6, seed=71, bias=True)
    DL = dsv4_gpu.DeviceLayer.from_host(L, dev)
    x = bf16_input(np.random.default_rng(72), (2, 256))
    X = torch.from_numpy(x).to(dev)
    ws = lib.new_moe_workspace(DL, 2, dev)
    ws[:4].view(torch.int32).fill_(1)  # the sticky status word, set by the host
    torch.cuda.synchronize()
    print("python caller: status word preset", flush=True)
    with pytest.raises(RuntimeError, match="wait ran out"):
        lib.moe_forward(DL, X, workspace=ws)
    # the binding zeroed the workspace again: the next call is exact
    out, idx, wt = lib.moe_forward(DL, X, workspace=ws)
    out, idx, wt = out.cpu().numpy(), idx.cpu().numpy(), wt.cpu().numpy()
    for t in range(2):
        o, i, w = orc.moe_forward(L, x[t])
        assert np.array_equal(i, idx[t]) and same_bits(w, wt[t]) and same_bits(o, out[t]), t


@pytest.mark.gpu
def test_noalloc_status_clean_after_normal_calls():
    import torch
    import dsv4_gpu

    dev = torch.device("cuda:0")
    orc = pyoracle.Oracle()
    lib = dsv4_gpu.lib()
    L = make_layer(orc, 256, 128, 16, 6, seed=73, bias=True)
    DL = dsv4_gpu.DeviceLayer.from_host(L, dev)
    x = bf16_input(np.random.default_rng(74), (1, 256))
    X = torch.from_numpy(x).to(dev)
    out = torch.empty_like(X)
    import ctypes as C
    raw = lib.lib
    raw.dsv4g_moe_forward_noalloc.restype = C.c_int
    raw.dsv4g_moe_forward_noalloc.argtypes = [C.c_void_p, C.c_void_p, C.POINTER(type(DL.struct)),
                                              C.c_void_p, C.c_int, C.c_void_p, C.c_void_p,
                                              C.c_void_p]
    rc = raw.dsv4g_moe_forward_noalloc(C.c_void_p(out.data_ptr()), C.c_void_p(X.data_ptr()),
                                       C.byref(DL.struct), None, 1, None, None, None)
    assert rc == 0, lib.lib.dsv4g_last_error()
    assert lib.noalloc_status() == 0
    o, _, _ = orc.moe_forward(L, x[0])
    assert same_bits(out.cpu().numpy()[0], o)
