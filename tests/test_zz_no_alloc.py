"""The workspace-free MoE decode step (qmm_moe_decode_noalloc) against qmm_moe_decode, through the C ABI.

qmm_moe_decode_noalloc keeps its workspace in a static per-GPU device array instead of a caller's
buffer.  Two calls in a row, the second on a smaller input (so stale contents of the shared array from
the first call are present), must each give ids, weights and y bit for bit equal to qmm_moe_decode's on
the same inputs; a shape whose workspace exceeds the array is refused before anything runs.
"""
import ctypes

import numpy as np
import pytest
import torch

from hipster_amd import _lib, qmm, synth
from tests.gpu_util import dev, host

pytestmark = pytest.mark.gpu

H, F, NEXP_TOTAL, TOPK = 2048, 512, 512, 10


def _weights(seed):
    Wg = synth.experts(seed, synth.Q4_K, NEXP_TOTAL, F, H)
    Wu = synth.experts(seed + 1, synth.Q4_K, NEXP_TOTAL, F, H)
    Wd = synth.experts(seed + 2, synth.Q4_K, NEXP_TOTAL, H, F)
    S = [synth.matrix(seed + 3 + i, synth.Q4_K, *s) for i, s in enumerate(((F, H), (F, H), (H, F)))]
    return [Wg, Wu, Wd] + S, Wg[0].nbytes, Wd[0].nbytes


def _inputs(seed, T):
    x = synth.normal_f32(seed, (T, H))
    lg = dev(synth.router_logits(seed + 1, T, NEXP_TOTAL))
    xb = qmm.XQ8Buf(T, H)
    qmm.quantize_x_q8(dev(x), xb, T, H)
    return lg, xb


def _outs(T):
    nexp = TOPK + 1
    return (torch.full((T, nexp), -7, dtype=torch.int32, device="cuda"), torch.full((T, nexp), float("nan"), device="cuda"),
            torch.full((T, H), float("nan"), device="cuda"))


def _noalloc(W, eb_gu, eb_d, lg, xb, T, ids, w, y):
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    return _lib.lib().qmm_moe_decode_noalloc(synth.Q4_K, p(W[0]), p(W[1]), p(W[2]), eb_gu, eb_d, p(W[3]), p(W[4]), p(W[5]), p(lg),
                                             NEXP_TOTAL + 1, NEXP_TOTAL, TOPK, xb.c(), T, H, F, p(ids), p(w), p(y),
                                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_noalloc_matches_workspace_entry(gpu):
    Wh, eb_gu, eb_d = _weights(1400)
    W = [dev(a) for a in Wh]
    for call, T in enumerate((8, 1)):            # the second call on a smaller input
        print(f"moe_decode_noalloc call {call} T={T}", flush=True)
        lg, xb = _inputs(1410 + T, T)
        ids, w, y = _outs(T)
        ws = torch.zeros(qmm.moe_decode_ws_bytes(T, TOPK, F) // 4, device="cuda")
        qmm.moe_decode(synth.Q4_K, W[0], W[1], W[2], eb_gu, eb_d, W[3], W[4], W[5], lg, NEXP_TOTAL + 1, NEXP_TOTAL, TOPK, xb, T, H, F,
                       ids, w, ws, y)
        ids2, w2, y2 = _outs(T)
        assert _noalloc(W, eb_gu, eb_d, lg, xb, T, ids2, w2, y2) == 0
        torch.cuda.synchronize()
        assert np.array_equal(host(ids2), host(ids))
        assert np.array_equal(host(w2).view(np.uint32), host(w).view(np.uint32))
        assert np.array_equal(host(y2).view(np.uint32), host(y).view(np.uint32))
        assert np.isfinite(host(y2)).all()


def test_noalloc_every_legal_shape_fits(gpu):
    # the workspace is the q8 of h, T * (topk + 1) * F * 5/4 bytes, and an accepted shape has
    # (topk + 1) * F * 5/4 <= 64 KiB (the down projection's LDS), so at most 8 * 64 KiB = 0.5 MiB:
    # inside the 2 MiB array, no accepted call is refused for its size
    for topk, FF in ((15, 3072), (10, 4608), (3, 6144)):
        assert (topk + 1) * FF * 5 // 4 <= 64 * 1024
        assert qmm.moe_decode_ws_bytes(8, topk, FF) == 8 * (topk + 1) * FF * 5 // 4 <= qmm.moe_decode_scratch_max() == 2 << 20


def _q4k_device(gen, rows, K):
    """rows x K Q4_K weights drawn on the GPU: random quant and scale bytes, d and dmin small halves."""
    nb = rows * (K // 256)
    raw = torch.randint(0, 256, (nb, 144), dtype=torch.uint8, device="cuda", generator=gen)
    dd = (torch.rand((nb, 2), device="cuda", generator=gen) * 0.01).half()
    raw[:, 0:4] = dd.view(torch.uint8).reshape(nb, 4)
    return raw.reshape(rows, -1)


def test_largest_accepted_and_first_refused_shape(gpu):
    """T = 8, 16 slots, H = 6144 at the largest accepted F (3072) runs through both entry points with the
    same bits; F = 3328 (the down projection's LDS would exceed 64 KiB) is refused by both before any
    output (ids, w, y) or workspace byte is written."""
    T, topk, nexp_total, HH = 8, 15, 16, 6144
    gen = torch.Generator(device="cuda")
    for FF, ok in ((3072, True), (3328, False)):
        print(f"moe_decode largest shape T={T} topk={topk} H={HH} F={FF}", flush=True)
        gen.manual_seed(1500 + FF)
        Wg, Wu = _q4k_device(gen, nexp_total * FF, HH), _q4k_device(gen, nexp_total * FF, HH)
        Wd = _q4k_device(gen, nexp_total * HH, FF)
        Sg, Su, Sd = _q4k_device(gen, FF, HH), _q4k_device(gen, FF, HH), _q4k_device(gen, HH, FF)
        eb_gu, eb_d = FF * (HH // 256) * 144, HH * (FF // 256) * 144
        lg = dev(synth.router_logits(1510, T, nexp_total))
        xb = qmm.XQ8Buf(T, HH)
        qmm.quantize_x_q8(dev(synth.normal_f32(1511, (T, HH))), xb, T, HH)
        outs = []
        for noalloc in (False, True):
            ids = torch.full((T, topk + 1), -7, dtype=torch.int32, device="cuda")
            w = torch.full((T, topk + 1), float("nan"), device="cuda")
            y = torch.full((T, HH), float("nan"), device="cuda")
            ws = torch.full((qmm.moe_decode_ws_bytes(T, topk, FF) // 4,), float("nan"), device="cuda")
            p = lambda t: ctypes.c_void_p(t.data_ptr())
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            L = _lib.lib()
            if noalloc:
                rc = L.qmm_moe_decode_noalloc(synth.Q4_K, p(Wg), p(Wu), p(Wd), eb_gu, eb_d, p(Sg), p(Su), p(Sd), p(lg), nexp_total + 1,
                                              nexp_total, topk, xb.c(), T, HH, FF, p(ids), p(w), p(y), st)
            else:
                rc = L.qmm_moe_decode(synth.Q4_K, p(Wg), p(Wu), p(Wd), eb_gu, eb_d, p(Sg), p(Su), p(Sd), p(lg), nexp_total + 1, nexp_total,
                                      topk, xb.c(), T, HH, FF, p(ids), p(w), p(ws), ws.numel() * 4, p(y), st)
            torch.cuda.synchronize()
            if ok:
                assert rc == 0
                assert np.isfinite(host(y)).all() and (host(ids) >= -1).all()
            else:
                assert rc == -2                                       # QMM_ERR_SHAPE, nothing written
                assert (host(ids) == -7).all() and np.isnan(host(w)).all() and np.isnan(host(y)).all()
                assert np.isnan(host(ws)).all()
            outs.append((host(ids), host(w).view(np.uint32), host(y).view(np.uint32)))
        for a, b in zip(*outs):
            assert np.array_equal(a, b)
