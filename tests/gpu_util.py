"""Device-memory plumbing for the GPU tests: torch allocates HBM and owns the
stream; every kernel call goes through the C-ABI of libkai_gdn_hip.so."""
from __future__ import annotations

import ctypes

import numpy as np


def torch_mod():
    import torch
    return torch


def dev(a: np.ndarray):
    """Copy a numpy array to a new device tensor (same dtype)."""
    torch = torch_mod()
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to("cuda", non_blocking=False)


def empty(shape, dtype):
    torch = torch_mod()
    return torch.empty(shape, dtype=dtype, device="cuda")


def P(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def stream() -> ctypes.c_void_p:
    torch = torch_mod()
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def host(t) -> np.ndarray:
    torch = torch_mod()
    torch.cuda.synchronize()
    return t.cpu().numpy()


def u16(t_np: np.ndarray):
    """A uint16 numpy array as an int16 device tensor (torch has no uint16
    arithmetic; only the bits matter)."""
    return dev(np.ascontiguousarray(t_np, np.uint16).view(np.int16))


def host_u16(t) -> np.ndarray:
    return host(t).view(np.uint16)


def np_ptr(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)
