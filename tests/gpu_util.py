"""Helpers for the GPU parity tests: host numpy <-> device torch tensors."""
import numpy as np
import torch


def to_dev(a, dev="cuda:0"):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(dev)
    if a.dtype == np.uint8:
        return torch.from_numpy(a).to(dev)
    return torch.from_numpy(a).to(dev)


def from_dev(t, dtype=None):
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def empty_f16(n, dev="cuda:0"):
    return torch.empty(n, dtype=torch.int16, device=dev)


def empty_f32(n, dev="cuda:0"):
    return torch.empty(n, dtype=torch.float32, device=dev)


def f16_to_f64(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


def rel_inf(got, want):
    """max |got - want| / max |want|  (the fp32 parity metric)."""
    want = np.asarray(want, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


def print_case(*a):
    print("CASE", *a, flush=True)
