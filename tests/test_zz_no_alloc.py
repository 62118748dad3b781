"""The no-allocation decode entry (dsv4g_moe_forward_noalloc) through the C
ABI against the workspace entry (dsv4g_moe_forward), bit for bit, on two
calls in a row (the second with fewer tokens, on the state the first left in
the shared scratch), plus the size limit's error and no change in the
device's free memory across the calls."""
import ctypes as C

import numpy as np
import pytest

from common import pyoracle, same_bits

pytestmark = pytest.mark.gpu


def test_noalloc_matches_workspace_entry():
    import torch
    import dsv4_gpu
    import synth
    dev = torch.device("cuda:0")
    lib = dsv4_gpu.lib()
    raw = lib.lib
    raw.dsv4g_moe_forward_noalloc.restype = C.c_int
    raw.dsv4g_moe_forward_noalloc.argtypes = [C.c_void_p, C.c_void_p,
                                               C.POINTER(dsv4_gpu.DSV4GLayer), C.c_void_p,
                                               C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    hip = C.CDLL("libamdhip64.so")
    free_b, total_b = C.c_size_t(), C.c_size_t()

    def free_mem():
        torch.cuda.synchronize()
        assert hip.hipMemGetInfo(C.byref(free_b), C.byref(total_b)) == 0
        return free_b.value

    DL = synth.device_layer(seed=3, hidden=4096, inter=2048, n_experts=64, device=dev)
    X = synth.bf16_tokens(5, 4096, seed=21, device=dev)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    ptr = lambda t: C.c_void_p(t.data_ptr())
    outs, idxs, wts = [], [], []
    for n in (5, 5, 2):  # warm-up call, then two calls in a row, the second smaller
        outs.append(torch.full((n, 4096), float("nan"), device=dev))
        idxs.append(torch.full((n, 6), -7, dtype=torch.int32, device=dev))
        wts.append(torch.zeros(n, 6, device=dev))
    rc = raw.dsv4g_moe_forward_noalloc(ptr(outs[0]), ptr(X), C.byref(DL.struct), None, 5,
                                       ptr(idxs[0]), ptr(wts[0]), st)
    assert rc == 0, raw.dsv4g_last_error()
    before = free_mem()
    for j, n in ((1, 5), (2, 2)):
        rc = raw.dsv4g_moe_forward_noalloc(ptr(outs[j]), ptr(X[:n]), C.byref(DL.struct), None,
                                           n, ptr(idxs[j]), ptr(wts[j]), st)
        assert rc == 0, raw.dsv4g_last_error()
    assert free_mem() == before
    for j, n in ((1, 5), (2, 2)):
        ref, ri, rw = lib.moe_forward(DL, X[:n])
        torch.cuda.synchronize()
        assert same_bits(outs[j].cpu().numpy(), ref.cpu().numpy()), n
        assert np.array_equal(idxs[j].cpu().numpy(), ri.cpu().numpy()), n
        assert same_bits(wts[j].cpu().numpy(), rw.cpu().numpy()), n
    # the oracle agrees too (the workspace entry is itself bit-exact)
    orc = pyoracle.Oracle()
    L = synth.host_copy(DL)
    o, i, w = orc.moe_forward(L, X[1].cpu().numpy())
    assert same_bits(outs[2][1].cpu().numpy(), o)
    # beyond the scratch: a clear error, nothing launched
    raw.dsv4g_moe_workspace_bytes.restype = C.c_size_t
    raw.dsv4g_moe_workspace_bytes.argtypes = [C.POINTER(dsv4_gpu.DSV4GLayer), C.c_int]
    nbig = 1
    while raw.dsv4g_moe_workspace_bytes(C.byref(DL.struct), nbig) <= 16 << 20:
        nbig += 1
    assert nbig <= 1020  # the decode entry's own token limit is not what fails
    big = torch.zeros(nbig, DL.struct.hidden, device=dev)
    rc = raw.dsv4g_moe_forward_noalloc(ptr(big), ptr(big), C.byref(DL.struct), None, nbig, None,
                                       None, st)
    assert rc != 0
    assert b"scratch" in raw.dsv4g_last_error()


def test_noalloc_layers_of_two_shapes():
    """Calls with layers of two shapes in turn on the one scratch array: a
    change of shape clears it first, so every call matches the workspace
    entry bit for bit."""
    import torch
    import dsv4_gpu
    import synth
    dev = torch.device("cuda:0")
    lib = dsv4_gpu.lib()
    raw = lib.lib
    raw.dsv4g_moe_forward_noalloc.restype = C.c_int
    raw.dsv4g_moe_forward_noalloc.argtypes = [C.c_void_p, C.c_void_p,
                                               C.POINTER(dsv4_gpu.DSV4GLayer), C.c_void_p,
                                               C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    A = synth.device_layer(seed=5, hidden=4096, inter=2048, n_experts=64, device=dev)
    B = synth.device_layer(seed=6, hidden=4096, inter=512, n_experts=32, topk=4, device=dev)
    X = synth.bf16_tokens(3, 4096, seed=23, device=dev)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    ptr = lambda t: C.c_void_p(t.data_ptr())
    for DL, n in ((A, 3), (B, 2), (A, 1), (B, 3)):
        k = DL.struct.topk
        out = torch.full((n, 4096), float("nan"), device=dev)
        idx = torch.full((n, k), -7, dtype=torch.int32, device=dev)
        wt = torch.zeros(n, k, device=dev)
        rc = raw.dsv4g_moe_forward_noalloc(ptr(out), ptr(X[:n]), C.byref(DL.struct), None, n,
                                           ptr(idx), ptr(wt), st)
        assert rc == 0, raw.dsv4g_last_error()
        ref, ri, rw = lib.moe_forward(DL, X[:n])
        torch.cuda.synchronize()
        assert same_bits(out.cpu().numpy(), ref.cpu().numpy()), (k, n)
        assert np.array_equal(idx.cpu().numpy(), ri.cpu().numpy()), (k, n)
        assert same_bits(wt.cpu().numpy(), rw.cpu().numpy()), (k, n)
