"""Device-buffer plumbing for the GPU tests (torch holds the memory; the
engine is called through its C ABI with raw pointers)."""
import ctypes

import numpy as np


def D(a):
    """Copy a numpy array's bytes to a new cuda uint8 tensor."""
    import torch
    a = np.ascontiguousarray(a)
    if a.nbytes == 0:
        return torch.zeros(16, dtype=torch.uint8, device="cuda")
    return torch.from_numpy(a.view(np.uint8).reshape(-1).copy()).cuda()


def E(nbytes):
    import torch
    return torch.zeros(max(int(nbytes), 16), dtype=torch.uint8, device="cuda")


def H(t, dtype, count=None):
    import torch
    torch.cuda.synchronize()
    a = t.cpu().numpy().view(dtype)
    return a if count is None else a[:count].copy()


def p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def banner(msg):
    print(f"\n[gpu-test] {msg}", flush=True)
