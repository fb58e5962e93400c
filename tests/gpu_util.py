"""Helpers shared by the GPU parity tests."""
import numpy as np


def torch_mod():
    import torch
    return torch


def dev(a):
    torch = torch_mod()
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
    torch.cuda.synchronize()
    return t


def empty(shape, dtype):
    torch = torch_mod()
    t = torch.empty(shape, dtype=dtype, device="cuda")
    torch.cuda.synchronize()
    return t


def host(ctx, t):
    ctx.sync()
    torch = torch_mod()
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits_equal(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


def cosine(a, b):
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))
