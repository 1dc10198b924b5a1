"""tg_block_scaled_matmul_noalloc (include/tg_fp8.h): the forward composite of
fp8.py:50-78 on the library's static scratch instead of a caller workspace.

Checked through the C ABI against tg_block_scaled_matmul with a torch-allocated
workspace (same kernels, so the bar is bit equality), on two calls in a row,
the second with a smaller input (the scratch keeps the first call's bytes), and
the host-side rejection of a shape whose workspace exceeds the scratch.
"""
import ctypes

import numpy as np
import pytest
import torch

import _tglib as L
from helpers import to_dev
from oracle import bf16 as ob

pytestmark = pytest.mark.gpu


def _pair(dev, M, N, K, seed):
    rng = np.random.default_rng(seed)
    a = to_dev(ob.randn_bf16(rng, (M, K)), dev)
    b = to_dev(ob.randn_bf16(rng, (K, N), std=0.02), dev)
    return a, b


def _with_workspace(a, b, M, N, K):
    lib = L.lib()
    ws = torch.empty(lib.tg_block_scaled_matmul_workspace(M, N, K, 128), dtype=torch.uint8,
                     device=a.device)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    L.check(lib.tg_block_scaled_matmul(L.ptr(a), L.ptr(b), L.ptr(out), M, N, K, 128, L.ptr(ws),
                                       ctypes.c_size_t(ws.numel()), L.stream_of(a)))
    return out


def _noalloc(a, b, M, N, K):
    out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    L.check(L.lib().tg_block_scaled_matmul_noalloc(L.ptr(a), L.ptr(b), L.ptr(out), M, N, K, 128,
                                                   L.stream_of(a)))
    return out


def test_noalloc_equals_workspace_entry_point_twice(dev):
    # C1's shape, then a smaller ragged one: the second call must not depend on
    # what the first left in the scratch
    for (M, N, K), seed in (((2048, 3072, 768), 0), ((200, 136, 384), 1)):
        print(f"noalloc case M={M} N={N} K={K}", flush=True)
        a, b = _pair(dev, M, N, K, seed)
        got = _noalloc(a, b, M, N, K)
        want = _with_workspace(a, b, M, N, K)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_rejects_shapes_beyond_the_scratch(dev):
    lib = L.lib()
    M, N, K = 16384, 16384, 2048              # 69 MB of workspace
    assert lib.tg_block_scaled_matmul_workspace(M, N, K, 128) > L.TG_NOALLOC_SCRATCH_BYTES
    one = torch.zeros(16, dtype=torch.uint8, device=dev)     # never read: rejected before launch
    rc = lib.tg_block_scaled_matmul_noalloc(L.ptr(one), L.ptr(one), L.ptr(one), M, N, K, 128,
                                            L.stream_of(one))
    assert rc == L.TG_EINVAL
    assert b"static scratch" in lib.tg_last_error()
