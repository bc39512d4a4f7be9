"""Device-memory plumbing for the GPU tests: torch allocates and copies, the
library is always called through its C-ABI (s2x)."""
import ctypes
import sys

import numpy as np
import torch


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a, dtype=None):
    """numpy -> cuda tensor (uint8 view for raw bytes)."""
    a = np.ascontiguousarray(a)
    t = torch.from_numpy(a.view(np.uint8) if dtype == "bytes" else a)
    return t.to("cuda:0")


def empty(shape, dtype):
    return torch.empty(shape, dtype=dtype, device="cuda:0")


def zeros(shape, dtype):
    return torch.zeros(shape, dtype=dtype, device="cuda:0")


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def assert_same(got, ref, what="", show=12):
    """Bitwise equality with a report of the first mismatches."""
    got, ref = np.asarray(got), np.asarray(ref)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    bad = np.argwhere(got != ref)
    if len(bad):
        say(f"{what}: {len(bad)} of {got.size} differ; first:")
        for idx in bad[:show]:
            t = tuple(idx)
            say(f"   {t}: got {got[t]!r} ref {ref[t]!r}")
    assert len(bad) == 0, f"{what}: {len(bad)} mismatches"


def cos(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def h5_rel(y, ref, terms_abs):
    """max |y - ref| / max(|ref|, tau) with tau = 1e-3 * rms of the row of
    sum|terms| (the tolerance metric of the GEMM)."""
    tau = 1e-3 * np.sqrt((terms_abs.astype(np.float64) ** 2).mean(1, keepdims=True))
    den = np.maximum(np.abs(ref), tau)
    return float((np.abs(y.astype(np.float64) - ref) / den).max())
