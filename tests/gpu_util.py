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


def assert_route_matches(ids, w, ids_ref, w_ref, logits, nexp):
    """ids bit-exact, except where two candidates' probabilities are within 1e-6 of each other: the
    selection runs on the rounded p (as the reference), and the device exp (__expf) and the host libm's
    expf may differ by an ulp, which can swap such a near-tie.  Weights within 1e-5."""
    bad = np.nonzero((ids != ids_ref).any(axis=1))[0]
    for t in bad:
        l = logits[t, :nexp].astype(np.float64)
        p = np.exp(l - l.max()); p /= p.sum()
        for a, b in zip(ids[t], ids_ref[t]):
            if a != b:
                assert a >= 0 and b >= 0 and abs(p[a] - p[b]) <= 1e-6 * max(p[a], p[b]), (t, a, b, p[a], p[b])
    assert len(bad) <= 2, bad
    ok = np.setdiff1d(np.arange(ids.shape[0]), bad)
    np.testing.assert_allclose(w[ok], w_ref[ok], rtol=1e-5, atol=1e-7)
