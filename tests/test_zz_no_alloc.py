"""The not-allocating conditioning entry point (oasis_dit_conditioning_noalloc) against
oasis_dit_conditioning through the C ABI: two calls in a row, the second with fewer rows, each
bit-equal to the entry point with a caller-supplied scratch buffer; sizes past the static
scratch are rejected."""
import ctypes

import pytest
import torch

from helpers import cuda, pkg

pytestmark = pytest.mark.gpu

L = pkg._lib


def _conditioning(dit, ws, t, act, noalloc):
    R = t.shape[0]
    ws.t[:R].copy_(t)
    ws.act[:R].zero_()
    ws.act[:R, :dit.ext_dim].copy_(act)
    ws.cond.fill_(float("nan"))
    ws.ada.fill_(float("nan"))
    h = L.stream_handle()
    if noalloc:
        L.call("oasis_dit_conditioning_noalloc", ctypes.byref(dit.struct), L.ptr(ws.t), L.ptr(ws.act), R,
               L.ptr(ws.cond), L.ptr(ws.ada), h)
    else:
        L.call("oasis_dit_conditioning", ctypes.byref(dit.struct), L.ptr(ws.t), L.ptr(ws.act), R, L.ptr(ws.hid),
               L.ptr(ws.cond), L.ptr(ws.ada), h)
    torch.cuda.synchronize()
    return ws.cond[:R].clone(), ws.ada[:R].clone()


def test_noalloc_conditioning_equals_the_scratch_entry_point():
    dr = pkg.synth.Draw(83)
    w = pkg.synth.dit_weights(dr, n_blocks=2, dtype=torch.float32)
    dit = pkg.DiT(w, "cuda")
    ws = dit.workspace(144, max_cond=64)
    for R in (37, 5):   # the second call has fewer rows than the first
        t = torch.rand(R, generator=dr.g) * 999
        act = torch.zeros(R, 25)
        act[torch.arange(R), torch.randint(0, 25, (R,), generator=dr.g)] = 1.0
        c_ref, a_ref = _conditioning(dit, ws, cuda(t), cuda(act), noalloc=False)
        c_got, a_got = _conditioning(dit, ws, cuda(t), cuda(act), noalloc=True)
        assert torch.isfinite(a_got).all() and torch.isfinite(c_got).all()
        assert torch.equal(c_got, c_ref), R
        assert torch.equal(a_got, a_ref), R


def test_noalloc_conditioning_rejects_sizes_past_its_scratch():
    dr = pkg.synth.Draw(84)
    w = pkg.synth.dit_weights(dr, n_blocks=1, d=256, n_heads=4, d_mlp=512)
    dit = pkg.DiT(w, "cuda")
    ws = dit.workspace(144, max_cond=80)
    with pytest.raises(L.OasisError, match="static scratch"):
        L.call("oasis_dit_conditioning_noalloc", ctypes.byref(dit.struct), L.ptr(ws.t), L.ptr(ws.act), 65,
               L.ptr(ws.cond), L.ptr(ws.ada), L.stream_handle())
