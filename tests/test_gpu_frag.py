"""The fragment-order projections (oasis_gemm_bf16_frag and the passes of at most 320 tokens that
run on it) against the row-major kernels: the same products with every epilogue the DiT uses,
and whole sub-blocks and steps with and without the fragment-order weights. The two differ only in
the order K is summed (8 wave slices against 4), so results agree to fp32 rounding before the
bf16 outputs are rounded.

The library's default masks keep O's and FC2's operands in fragment order at one frame (FC2's
written by the row-major FC1) and O's alone at two; the DiT built with every role's weights runs
whichever roles OASIS_FRAG names (run this file once more with OASIS_FRAG=15 for all four)."""
import ctypes

import pytest
import torch

import oracle
from helpers import COS_SUB, REL_SUB, assert_close, cuda, pkg

pytestmark = pytest.mark.gpu

L = pkg._lib
M_ = pkg.model


def _frag(x, rows):
    """Row-major [r, K] -> fragment order with the rows zero-padded to `rows`."""
    r, k = x.shape
    p = torch.zeros(rows, k, dtype=x.dtype, device=x.device)
    p[:r] = x
    return M_.tile_rows16(p)


def _blk(w, i, kind):
    p = "blocks.%d.%s." % (i, kind)
    return {k[len(p):]: v for k, v in w.items() if k.startswith(p)}


def _epi(**kw):
    e = L.Epilogue()
    for k, v in kw.items():
        setattr(e, k, v)
    return e


@pytest.mark.parametrize("M", [144, 288])
@pytest.mark.parametrize("role", ["fc1", "fc1_frag_out", "fc1_row_major_frag_out", "fc2", "o", "qkv"])
def test_frag_gemm_matches_row_major(M, role):
    g = torch.Generator().manual_seed(M + len(role))
    D, Dm = 1024, 4096
    N, K = (D, Dm) if role == "fc2" else (D, D) if role == "o" else (3 * D, D) if role == "qkv" else (Dm, D)
    splits = 4 if role == "fc2" else 1
    A = cuda(torch.randn(M, K, generator=g), torch.bfloat16)
    W = cuda(torch.randn(N, K, generator=g) * 0.03, torch.bfloat16)
    bias = cuda(torch.randn(N, generator=g) * 0.1)
    rows = M_.frag_rows(M)
    Af, Wf = _frag(A, rows), M_.tile_rows16(W)
    h = L.stream_handle()
    if role.startswith("fc1"):
        ref = torch.zeros(M, N, device="cuda", dtype=torch.bfloat16)
        L.call("oasis_gemm_bf16", L.ptr(A), K, L.ptr(W), K, M, N, K,
               ctypes.byref(_epi(kind=L.EPI_GELU_TANH, bias=bias.data_ptr(), out_bf16=ref.data_ptr(), ld_out=N)), h)
        if role == "fc1":
            got = torch.zeros(M, N, device="cuda", dtype=torch.bfloat16)
            e = _epi(kind=L.EPI_GELU_TANH, bias=bias.data_ptr(), out_bf16=got.data_ptr(), ld_out=N)
        else:   # into fragment order, as FC1 writes FC2's operand
            gf = torch.full((rows, N), float("nan"), device="cuda", dtype=torch.bfloat16)
            e = _epi(kind=L.EPI_GELU_TANH_FRAG, bias=bias.data_ptr(), out_bf16=gf.data_ptr(), ld_out=N)
        if role == "fc1_row_major_frag_out":   # row-major operands, fragment-order output
            L.call("oasis_gemm_bf16", L.ptr(A), K, L.ptr(W), K, M, N, K, ctypes.byref(e), h)
        else:
            L.call("oasis_gemm_bf16_frag", L.ptr(Af), rows, L.ptr(Wf), M, N, K, ctypes.byref(e), 1, h)
        torch.cuda.synchronize()
        if role != "fc1":
            got = M_.untile_rows16(gf)[:M]
        diff = (got.float() - ref.float()).abs().max().item()
        # two fp32 sums of the same products rounded to bf16: at most an ulp of the output
        assert diff <= 2 ** -7 * ref.float().abs().max().item(), diff
        assert_close(got, ref, 0.99999, 1e-2, "frag %s M=%d" % (role, M))
    elif role in ("fc2", "o"):
        ref = torch.zeros(splits, M, N, device="cuda")
        got = torch.zeros(splits, M, N, device="cuda")
        for out, fn in ((ref, "ref"), (got, "frag")):
            e = _epi(kind=L.EPI_PARTIAL_F32, out_f32=out.data_ptr(), ld_out=N, split_stride=M * N)
            if fn == "ref":
                L.call("oasis_gemm_bf16_config", L.ptr(A), K, L.ptr(W), K, M, N, K, ctypes.byref(e), -1, splits, h)
            else:
                L.call("oasis_gemm_bf16_frag", L.ptr(Af), rows, L.ptr(Wf), M, N, K, ctypes.byref(e), splits, h)
        torch.cuda.synchronize()
        # the slices cover the same K ranges; summed they are the product
        assert_close(got.sum(0), ref.sum(0), 0.9999999, 1e-5, "frag %s M=%d (sum of %d slices)" % (role, M, splits))
        exact = (A.double() @ W.double().t())
        assert_close(got.sum(0).double(), exact, 0.9999999, 1e-5, "frag %s M=%d vs fp64" % (role, M))
    else:  # QKV + RoPE + head split (heads-first spatial layout, 144-token frames)
        H, P = D // 64, 144
        ang = oracle.spatial_rope_angles(torch.rand(16, generator=g) * 3, 9, 16)
        cs, ss = (cuda(t) for t in oracle.rope_cos_sinperm(ang, 64))
        outs = []
        for fn in ("ref", "frag"):
            q, k, v = (torch.zeros(M, D, device="cuda", dtype=torch.bfloat16) for _ in range(3))
            T = M // P
            e = _epi(kind=L.EPI_QKV_ROPE, n_heads=H, rows_per_frame=P, frames_per_stream=T, q=q.data_ptr(),
                     k=k.data_ptr(), v=v.data_ptr(), rope_cos=cs.data_ptr(), rope_sinp=ss.data_ptr(), rope_by_frame=0,
                     bias=bias.data_ptr(),
                     s_b=T * H * P * 64, s_t=H * P * 64, s_h=P * 64, s_p=64)
            if fn == "ref":
                L.call("oasis_gemm_bf16", L.ptr(A), K, L.ptr(W), K, M, N, K, ctypes.byref(e), h)
            else:
                L.call("oasis_gemm_bf16_frag", L.ptr(Af), rows, L.ptr(Wf), M, N, K, ctypes.byref(e), 1, h)
            outs.append((q, k, v))
        torch.cuda.synchronize()
        for name, r, gt in zip("qkv", outs[0], outs[1]):
            assert_close(gt, r, 0.99999, 1e-2, "frag qkv M=%d %s" % (M, name))


def test_frag_gemm_rejects_what_it_does_not_cover():
    A = torch.zeros(320, 1024, device="cuda", dtype=torch.bfloat16)
    W = torch.zeros(4096, 1024, device="cuda", dtype=torch.bfloat16)
    out = torch.zeros(288, 4096, device="cuda", dtype=torch.bfloat16)
    e = _epi(kind=L.EPI_GELU_TANH, out_bf16=out.data_ptr(), ld_out=4096)
    h = L.stream_handle()
    with pytest.raises(L.OasisError, match="rows"):   # 80-row tiles read 320 rows
        L.call("oasis_gemm_bf16_frag", L.ptr(A), 288, L.ptr(W), 288, 4096, 1024, ctypes.byref(e), 1, h)
    with pytest.raises(L.OasisError, match="320"):
        L.call("oasis_gemm_bf16_frag", L.ptr(A), 320, L.ptr(W), 336, 4096, 1024, ctypes.byref(e), 1, h)
    with pytest.raises(L.OasisError, match="K/splits"):
        L.call("oasis_gemm_bf16_frag", L.ptr(A), 320, L.ptr(W), 288, 4096, 1024, ctypes.byref(e), 8, h)


@pytest.fixture(scope="module")
def dits():
    dr = pkg.synth.Draw(43)
    w = pkg.synth.dit_weights(dr, n_blocks=2)
    return w, {"default": pkg.DiT(w, "cuda", frag=True), "all": pkg.DiT(w, "cuda", frag=M_.FRAG_ROLES_ALL),
               "none": pkg.DiT(w, "cuda", frag=False)}


def test_frag_roles():
    with pytest.raises(ValueError, match="frag roles"):
        pkg.DiT(pkg.synth.dit_weights(pkg.synth.Draw(1), n_blocks=1), "cuda", frag=("o",))


@pytest.mark.parametrize("T", [1, 2])
def test_sub_blocks_frag_against_row_major(dits, T):
    """Four sub-blocks (spatial and temporal) at one and two frames: the fragment-order passes and
    the row-major pass give the same residual stream to bf16 rounding, and all match the oracle."""
    w, ds = dits
    dr = pkg.synth.Draw(44 + T)
    x = dr.normal(T * 144, 1024)
    cond = dr.normal(T, 1024)
    upd = {}
    for name, dit in ds.items():
        ws = dit.workspace(T * 144, max_cond=16)
        assert (ws.struct.frag_rows > 0) == dit.frag
        ada = dit.adaln_from_cond(cuda(cond), ws)
        ws.x[:T * 144].copy_(cuda(x))
        dit.sub_blocks_inplace(ws, 1, T, ada, dit.ada_width, 0, dit.n_sub)
        torch.cuda.synchronize()
        upd[name] = ws.x[:T * 144].cpu() - x
    for name in ("default", "all"):
        assert_close(upd[name], upd["none"], 0.99999, 1e-2, "frag (%s) vs row-major update, T=%d" % (name, T))
    cs, ss = oracle.rope_cos_sinperm(oracle.spatial_rope_angles(w["rope.spatial_freqs"].float()), 64)
    ct, st = oracle.rope_cos_sinperm(oracle.temporal_rope_angles(w["rope.temporal_freqs"].float(), T), 64)
    z, sc = x.reshape(T, 144, 1024).float(), oracle.silu(cond.float())
    for i in range(2):
        z = oracle.sub_block(z, sc, _blk(w, i, "s"), "s", cs, ss)
        z = oracle.sub_block(z, sc, _blk(w, i, "t"), "t", ct, st)
    ref = z.reshape(T * 144, 1024) - x
    for name, u in upd.items():
        assert_close(u, ref, COS_SUB, REL_SUB, "four sub-blocks T=%d (%s) update vs oracle" % (T, name))


def test_step_frag_against_row_major_and_oracle(dits):
    """A two-block DiT step at T=2 (288 tokens, the 80-row tiles) with and without the
    fragment-order weights, each against the fp32 oracle."""
    w, ds = dits
    dr = pkg.synth.Draw(46)
    lat = dr.normal(2, 16, 18, 32)
    t = torch.tensor([14.0, 500.0])
    act = torch.zeros(2, 25)
    act[1, 4] = 1.0
    ref = oracle.dit_forward(oracle.patch_embed(lat, w), oracle.conditioning(t, act, w), w).reshape(-1, 64)
    vs = {}
    for name, dit in ds.items():
        step = pkg.DiTStep(dit, B=1, T=2)
        step.set_inputs(cuda(oracle.patchify_to_output_space(lat).reshape(-1, 64)), cuda(t), cuda(act))
        vs[name] = step.run().clone()
        torch.cuda.synchronize()
    for name, v in vs.items():
        assert_close(v, ref, COS_SUB, REL_SUB, "two-block step (%s) vs oracle" % name)
    for name in ("default", "all"):
        assert_close(vs[name], vs["none"], 0.99999, 1e-2, "two-block step frag (%s) vs row-major" % name)
