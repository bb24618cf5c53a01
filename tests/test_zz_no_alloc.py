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
    # the workspace is the q8 of h: at the largest shape qmm_moe_decode accepts (T = 8, 16 slots,
    # F = 6144) 0.94 MiB, inside the 2 MiB array, so no legal call is refused for its size
    T, topk, FF = 8, 15, 6144
    assert qmm.moe_decode_ws_bytes(T, topk, FF) == T * (topk + 1) * FF * 5 // 4
    assert qmm.moe_decode_ws_bytes(T, topk, FF) <= qmm.moe_decode_scratch_max() == 2 << 20
