"""Helpers shared by the GPU parity tests (device upload, error metrics)."""
import numpy as np
import torch


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def rel_l2(got, ref):
    got = np.asarray(got, np.float64); ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-300))


def max_rel_mag(got, ref, mag):
    """The reference validator's metric (engine/bench/bench_gemv.cpp:95-104): |ref-got| / sum|w*x|."""
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref) / (mag + 1e-20)))
