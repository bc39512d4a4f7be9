"""s2x_mul_mat_q8_0_f32_static, the allocation-free drop-in matmul, through
the C-ABI: bit for bit the output of s2x_mul_mat_q8_0_f32 with a caller
workspace, on two calls in a row (the second smaller, so it runs over what
the first left in the static scratch array), and a shape larger than the
array rejected before any launch."""
import ctypes

import numpy as np
import pytest
import torch

import s2x
from s2x import synth
from gpu_util import assert_same, dev, empty, host, ptr, say, stream

pytestmark = pytest.mark.gpu


def _case(seed, M, K, K_pad, N):
    rng = np.random.default_rng(seed)
    raw = synth.quantize_q8_0(rng.normal(0, 0.02, (N, K)).astype(np.float32), K_pad)
    x = rng.standard_normal((M, K)).astype(np.float32)
    return dev(raw), dev(x)


def _with_workspace(wd, K_pad, N, xd, K, M):
    wsb = s2x.lib.s2x_mul_mat_workspace_size(K_pad, N, M)
    ws = empty((wsb,), torch.uint8)
    y = empty((M, N), torch.float32)
    s2x.call("s2x_mul_mat_q8_0_f32", ptr(wd), K_pad, N, ptr(xd), K, K, M, ptr(y), ptr(ws),
             ctypes.c_size_t(wsb), stream())
    return host(y)


def _static(wd, K_pad, N, xd, K, M):
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda:0")
    s2x.call("s2x_mul_mat_q8_0_f32_static", ptr(wd), K_pad, N, ptr(xd), K, K, M, ptr(y), stream())
    return host(y)


def test_static_matches_workspace_entry_point(orc):
    # first the fc2 shape at one image (K 4304 padded to 4320), then a
    # smaller QKV-shaped call over the same scratch array
    for seed, M, K, K_pad, N in [(61, 729, 4304, 4320, 1152), (62, 300, 1152, 1152, 3456)]:
        say(f"static-scratch mul_mat M={M} K={K} N={N}")
        wd, xd = _case(seed, M, K, K_pad, N)
        got = _static(wd, K_pad, N, xd, K, M)
        assert_same(got, _with_workspace(wd, K_pad, N, xd, K, M), f"static M={M} N={N}")
        rows = np.arange(0, M, 37)
        rq, rd = orc.quantize_q8_1(host(xd)[rows], K_pad)
        assert_same(got[rows], orc.mul_mat_q8_0_q8_1(host(wd), K_pad, N, rq, rd), "vs oracle")


def test_static_rejects_shapes_beyond_the_array():
    cap = s2x.lib.s2x_mul_mat_workspace_size(4320, 1152, 12720)
    assert cap <= 64 << 20 < s2x.lib.s2x_mul_mat_workspace_size(4320, 1152, 12721)
    wd, xd = _case(63, 4, 4304, 4320, 1152)
    y = empty((4, 1152), torch.float32)
    st = s2x.lib.s2x_mul_mat_q8_0_f32_static(ptr(wd), 4320, 1152, ptr(xd), 4304, 4304, 12721,
                                              ptr(y), stream())
    assert st == 2 and b"static scratch" in s2x.lib.s2x_last_error()
