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


def _ln_inputs(M, D, T, g):
    """x, the LN-before-QKV row means it is centred by (of a nearby x), and per-frame gate /
    scale / shift rows at a frame stride wider than D (as in the adaLN table)."""
    x = torch.randn(M, D, generator=g) * 2 + torch.randn(M, 1, generator=g)
    center = x.mean(1) + torch.randn(M, generator=g) * 0.05
    fs = 6 * D
    ada = torch.randn(T, fs, generator=g) * 0.5
    ada[:, D:2 * D] += 1.0     # scale + 1
    return x, center, ada, fs


def _stat_cols(M):
    """Columns per statistics group of the carried LayerNorm at D = 1024: O's fragment-order tiles
    are 32 columns wide above 160 rows (then 32-column groups), 16 at one frame."""
    return 32 if M > 160 else 16


def _frame_rows(ada, off, D, P, M):
    """[M, D]: row m takes frame m // P's row of ada at column offset off."""
    return ada[:, off:off + D].repeat_interleave(P, 0)[:M]


@pytest.mark.parametrize("M", [144, 288])
def test_gated_res_ln_epilogue(M):
    """O with GATED_RES_LN: x += gate * (acc + bias); h = bf16((x - centre) * scale) in fragment
    order; per-group (16 or 32 columns) sums of x - centre and its squares; the modulate block."""
    D, P = 1024, 144
    T = (M + P - 1) // P
    g = torch.Generator().manual_seed(M + 7)
    A = torch.randn(M, D, generator=g).to(torch.bfloat16)
    W = (torch.randn(D, D, generator=g) * 0.03).to(torch.bfloat16)
    bias = torch.randn(D, generator=g) * 0.1
    x, center, ada, fs = _ln_inputs(M, D, T, g)
    gate_off, scale_off, shift_off = 2 * D, D, 0
    rows = M_.frag_rows(M)
    xd, cd, adad, bd = cuda(x), cuda(center), cuda(ada), cuda(bias)
    h = torch.full((rows, D), float("nan"), device="cuda", dtype=torch.bfloat16)
    G = _stat_cols(M)
    stats = torch.full((M, D // G, 2), float("nan"), device="cuda")
    mod = torch.full((16, D), float("nan"), device="cuda", dtype=torch.bfloat16)
    Af, Wf = _frag(cuda(A), rows), M_.tile_rows16(cuda(W))
    e = _epi(kind=L.EPI_GATED_RES_LN, bias=bd.data_ptr(), out_f32=xd.data_ptr(), out_bf16=h.data_ptr(), ld_out=D,
             gate=adad.data_ptr() + gate_off * 4, gate_fstride=fs, rows_per_frame=P,
             mod_scale=adad.data_ptr() + scale_off * 4, mod_shift=adad.data_ptr() + shift_off * 4,
             ln_center=cd.data_ptr(), ln_stats=stats.data_ptr(), ln_mod=mod.data_ptr())
    L.call("oasis_gemm_bf16_frag", L.ptr(Af), rows, L.ptr(Wf), M, D, D, ctypes.byref(e), 1, L.stream_handle())
    torch.cuda.synchronize()
    gate, scale = _frame_rows(ada, gate_off, D, P, M), _frame_rows(ada, scale_off, D, P, M)
    x_ref = x.double() + gate.double() * (A.double() @ W.double().t() + bias.double())
    assert_close(xd.cpu(), x_ref, 0.9999999, 1e-5, "GATED_RES_LN x M=%d" % M)
    # h and the statistics from the kernel's own x: the same fp32 operations, so h is the
    # correctly rounded bf16 of (x - centre) * scale
    xg = xd.cpu()
    y = xg - center[:, None]
    h_ref = (y * scale).to(torch.bfloat16)
    hg = M_.untile_rows16(h)[:M].cpu()
    assert torch.equal(hg, h_ref), (hg.float() - h_ref.float()).abs().max().item()
    st_ref = torch.stack([y.double().reshape(M, D // G, G).sum(-1), (y.double() ** 2).reshape(M, D // G, G).sum(-1)], -1)
    assert_close(stats.cpu(), st_ref, 0.9999999, 1e-5, "GATED_RES_LN statistics M=%d" % M)
    # the modulate block: rows 2f, 2f + 1 = bf16 scale, shift of frame f (the rest untouched)
    mb = M_.untile_rows16(mod).cpu()
    for f in range(T):
        assert torch.equal(mb[2 * f], ada[f, scale_off:scale_off + D].to(torch.bfloat16))
        assert torch.equal(mb[2 * f + 1], ada[f, shift_off:shift_off + D].to(torch.bfloat16))
    assert torch.isnan(mb[2 * T:].float()).all()


@pytest.mark.parametrize("M,out_frag", [(144, 1), (288, 0), (288, 1)])
def test_gelu_tanh_ln_epilogue(M, out_frag):
    """FC1 with GELU_TANH_LN on the output of GATED_RES_LN (y * scale, the statistics and the
    modulate block) equals gelu(LN(x) * scale + shift) @ W^T + bias: against that in fp64, and
    against the unfused order (bf16 LN output, then the GEMM)."""
    D, Dm, P = 1024, 4096, 144
    T = (M + P - 1) // P
    g = torch.Generator().manual_seed(M + 11 + out_frag)
    x, center, ada, fs = _ln_inputs(M, D, T, g)
    W = (torch.randn(Dm, D, generator=g) * 0.03).to(torch.bfloat16)
    bias = torch.randn(Dm, generator=g) * 0.1
    scale_off, shift_off = D, 0
    scale, shift = _frame_rows(ada, scale_off, D, P, M), _frame_rows(ada, shift_off, D, P, M)
    y = x - center[:, None]
    ys = (y * scale).to(torch.bfloat16)
    G = _stat_cols(M)
    stats = torch.stack([y.reshape(M, D // G, G).sum(-1), (y * y).reshape(M, D // G, G).sum(-1)], -1)
    rows = M_.frag_rows(M)
    sd, bd = cuda(stats), cuda(bias)
    mod = torch.zeros(16, D)
    for f in range(T):
        mod[2 * f], mod[2 * f + 1] = ada[f, scale_off:scale_off + D], ada[f, shift_off:shift_off + D]
    modd = M_.tile_rows16(cuda(mod, torch.bfloat16))
    out = torch.full((rows if out_frag else M, Dm), float("nan"), device="cuda", dtype=torch.bfloat16)
    e = _epi(kind=L.EPI_GELU_TANH_LN, bias=bd.data_ptr(), out_bf16=out.data_ptr(), ld_out=Dm, rows_per_frame=P,
             ln_stats=sd.data_ptr(), ln_mod=modd.data_ptr(), ln_eps=1e-6, out_frag=out_frag)
    A, Wf = _frag(cuda(ys), rows), M_.tile_rows16(cuda(W))
    L.call("oasis_gemm_bf16_frag", L.ptr(A), rows, L.ptr(Wf), M, Dm, D, ctypes.byref(e), 1, L.stream_handle())
    torch.cuda.synchronize()
    got = (M_.untile_rows16(out)[:M] if out_frag else out).cpu()
    ln = (x.double() - x.double().mean(1, keepdim=True)) / torch.sqrt(x.double().var(1, unbiased=False, keepdim=True) + 1e-6)
    hm = ln * scale.double() + shift.double()
    ref = oracle.gelu_tanh(hm @ W.double().t() + bias.double())
    assert_close(got, ref, 0.99999, 1e-2, "GELU_TANH_LN M=%d vs fp64" % M)
    unfused = oracle.gelu_tanh(hm.to(torch.bfloat16).double() @ W.double().t() + bias.double())
    assert_close(got, unfused, 0.99999, 1e-2, "GELU_TANH_LN M=%d vs the unfused order" % M)


def test_ln_kinds_rejected_where_unsupported():
    M, D = 288, 1024
    A = torch.zeros(320, D, device="cuda", dtype=torch.bfloat16)
    W = torch.zeros(4096, D, device="cuda", dtype=torch.bfloat16)
    buf = torch.zeros(M * 4096 * 2, device="cuda")
    e = _epi(kind=L.EPI_GELU_TANH_LN, out_bf16=buf.data_ptr(), ld_out=4096, ln_mod=buf.data_ptr(),
             ln_stats=buf.data_ptr(), rows_per_frame=16, ln_eps=1e-6)
    h = L.stream_handle()
    with pytest.raises(L.OasisError, match="frag only"):
        L.call("oasis_gemm_bf16", L.ptr(A), D, L.ptr(W), D, M, 4096, D, ctypes.byref(e), h)
    with pytest.raises(L.OasisError, match="8 frames"):        # the modulate block holds 8 frames
        L.call("oasis_gemm_bf16_frag", L.ptr(A), 320, L.ptr(W), M, 4096, D, ctypes.byref(e), 1, h)
    e.rows_per_frame = 144
    with pytest.raises(L.OasisError, match="PARTIAL_F32"):     # one split only
        L.call("oasis_gemm_bf16_frag", L.ptr(A), 320, L.ptr(W), M, 4096, D, ctypes.byref(e), 2, h)


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
