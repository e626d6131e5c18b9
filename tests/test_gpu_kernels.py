"""Per-kernel parity on the GPU through the C ABI against fp32 CPU references.

Inputs are seeded; GEMM-type references use the same bf16-rounded operands the kernel
sees, so the only differences are accumulation order and the bf16 rounding of outputs.
"""
import ctypes
import math

import pytest
import torch

import oracle
from helpers import L, assert_close, bf, cuda, noise_reference, pkg, stream, sync

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


_ALIVE = []  # device tensors whose raw pointers were handed to C (freed at test end)


@pytest.fixture(autouse=True)
def _release_device_temporaries():
    yield
    _ALIVE.clear()


def dev(t):
    """Device copy kept alive until the test ends (a bare temporary could be freed and its
    memory reused before the kernel reading it has run)."""
    d = cuda(t)
    _ALIVE.append(d)
    return d


def _epi(**kw):
    e = L.Epilogue()
    for k, v in kw.items():
        if isinstance(v, torch.Tensor):
            _ALIVE.append(v)
            v = v.data_ptr()
        setattr(e, k, v)
    return e


def _gemm(A, B, M, N, K, epi, lda=None, ldb=None):
    L.call("oasis_gemm_bf16", L.ptr(A), lda or K, L.ptr(B), ldb or K, M, N, K, ctypes.byref(epi), stream())


# ---------------------------------------------------------------- GEMM
@pytest.mark.parametrize("M,N,K", [(288, 3072, 1024), (288, 1024, 4096), (576, 1200, 1024), (13, 64, 64),
                                   (1, 8, 128), (100, 520, 192)])
def test_gemm_store_f32(M, N, K):
    g = _gen(M + N + K)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn(N, generator=g)
    out = torch.zeros(M, N, device="cuda")
    _gemm(dev(A), dev(B), M, N, K, _epi(kind=L.EPI_STORE_F32, bias=dev(bias), out_f32=out, ld_out=N))
    sync()
    ref = A.float() @ B.float().t() + bias
    assert_close(out, ref, 0.999999, 1e-4, "gemm %dx%dx%d" % (M, N, K))


@pytest.mark.parametrize("kind", ["bf16", "gelu_tanh", "gelu_erf"])
def test_gemm_bf16_epilogues(kind):
    M, N, K = 288, 4096, 1024
    g = _gen(3)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = (torch.randn(N, K, generator=g) * 0.03).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    out = torch.zeros(M, N, device="cuda", dtype=torch.bfloat16)
    k = {"bf16": L.EPI_STORE_BF16, "gelu_tanh": L.EPI_GELU_TANH, "gelu_erf": L.EPI_GELU_ERF}[kind]
    _gemm(dev(A), dev(B), M, N, K, _epi(kind=k, bias=dev(bias), out_bf16=out, ld_out=N))
    sync()
    ref = A.float() @ B.float().t() + bias
    ref = {"bf16": ref, "gelu_tanh": oracle.gelu_tanh(ref), "gelu_erf": oracle.gelu_erf(ref)}[kind]
    assert_close(out, ref, 0.99999, 1e-2, "gemm epilogue " + kind)


@pytest.mark.parametrize("tile", [-1, 5])
def test_gelu_erf_epilogue_values(tile):
    """The erf-GELU epilogue on chosen inputs (an identity weight passes A through, K = 256): over
    [-12, 12] every output within one bf16 step of torch's exact GELU in fp32 (the reference's),
    or within 1e-6 where that is below 1e-4 (its negative tail: 0 past x ~ -5.5), and at most 2%
    of the others not torch's value rounded to bf16; on the default tile and the large-token tile (the
    compile-time GELU_ERF epilogue of the VAE's FC1)."""
    M, K = 320, 256
    x = torch.linspace(-12.0, 12.0, M * K).reshape(M, K).to(torch.bfloat16)
    B = torch.eye(K).to(torch.bfloat16)
    out = torch.zeros(M, K, device="cuda", dtype=torch.bfloat16)
    e = _epi(kind=L.EPI_GELU_ERF, out_bf16=out, ld_out=K)
    L.call("oasis_gemm_bf16_config", L.ptr(dev(x)), K, L.ptr(dev(B)), K, M, K, K, ctypes.byref(e), tile, 1, stream())
    sync()
    ref = torch.nn.functional.gelu(x.float()).double()
    got = out.cpu().double()
    tol = torch.where(ref.abs() < 1e-4, torch.full_like(ref, 1e-6), ref.abs() * 2.0 ** -7)
    assert ((got - ref).abs() <= tol).all(), ((got - ref).abs() / tol).max()
    body = ref.abs() >= 1e-4
    off = (got != ref.to(torch.bfloat16).double())[body].double().mean().item()
    print("gelu_erf tile %d: %.5f of outputs (|GELU| >= 1e-4) not torch's GELU rounded to bf16" % (tile, off),
          flush=True)
    assert off <= 0.02, off


def test_gemm_gated_and_plain_residual():
    M, N, K, P = 288, 1024, 4096, 144
    g = _gen(4)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(N, generator=g)
    x0 = torch.randn(M, N, generator=g)
    fstride = 3 * N
    ada = torch.randn(2, fstride, generator=g)
    gate = ada[:, N:2 * N]
    x = dev(x0)
    ada_d = dev(ada)
    _gemm(dev(A), dev(B), M, N, K, _epi(kind=L.EPI_GATED_RES, bias=dev(bias), out_f32=x, ld_out=N,
                                          gate=ada_d[0, N:], gate_fstride=fstride, rows_per_frame=P))
    sync()
    y = A.float() @ B.float().t() + bias
    ref = x0 + torch.cat([gate[0].expand(P, N), gate[1].expand(P, N)]) * y
    assert_close(x, ref, 0.999999, 1e-5, "gated residual")
    _gemm(dev(A), dev(B), M, N, K, _epi(kind=L.EPI_RESIDUAL, bias=dev(bias), out_f32=x, ld_out=N))
    sync()
    assert_close(x, ref + y, 0.999999, 1e-5, "residual")


@pytest.mark.parametrize("layout,tile", [("spatial", -1), ("temporal", -1), ("vae", -1), ("spatial", 11),
                                         ("temporal", 11), ("spatial", 12), ("vae", 11), ("spatial", 5),
                                         ("temporal", 5), ("temporal", 6), ("spatial", 6), ("temporal", 7),
                                         ("vae", 6), ("temporal", 16), ("spatial", 16)])
def test_gemm_qkv_rope(layout, tile):
    """QKV + RoPE + head split into each attention layout: the default tile (K = 256), the
    wave-split tiles 11 / 12 with the kernels specialised for this epilogue (K = 1024), and the
    large-token tiles 5-7 and 16 (288 x 256 / 192 / 128, 144 x 128; their epilogue steps each
    lane's row through positions, frames and streams 16 rows at a time, here over two streams of
    two frames)."""
    H, D = 4, 256
    K = 256 if tile < 0 else 1024
    if layout == "vae":
        B_, T, P = (1, 1, 576) if tile < 5 else (1, 2, 576)
    else:
        B_, T, P = (2, 2, 144) if tile < 0 or tile >= 5 else (1, 2, 144)
    M, N = B_ * T * P, 3 * D
    g = _gen(5)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    if layout == "spatial":
        ang = oracle.spatial_rope_angles(torch.rand(16, generator=g) * 2, 9, 16)
    elif layout == "temporal":
        ang = oracle.temporal_rope_angles(torch.rand(32, generator=g), T)
    else:
        ang = oracle.vae_rope_angles(torch.rand(8, generator=g) * 2, 18, 32)
    cos, sinp = oracle.rope_cos_sinperm(ang, 64)
    q, k, v = (torch.zeros(M * D, device="cuda", dtype=torch.bfloat16) for _ in range(3))
    if layout == "temporal":
        s_b, s_t, s_p, s_h = P * H * T * 64, 64, H * T * 64, T * 64
    else:
        s_b, s_t, s_p, s_h = T * H * P * 64, H * P * 64, 64, P * 64
    e = _epi(kind=L.EPI_QKV_ROPE, n_heads=H, bias=dev(bias), q=q, k=k, v=v, rope_cos=dev(cos),
             rope_sinp=dev(sinp), rope_by_frame=int(layout == "temporal"), rows_per_frame=P,
             frames_per_stream=T, s_b=s_b, s_t=s_t, s_p=s_p, s_h=s_h)
    L.call("oasis_gemm_bf16_config", L.ptr(dev(A)), K, L.ptr(dev(W)), K, M, N, K, ctypes.byref(e), tile, 1, stream())
    sync()
    y = (A.float() @ W.float().t() + bias).reshape(B_, T, P, 3, H, 64)
    pos_c = cos[torch.arange(T)] if layout == "temporal" else cos
    pos_s = sinp[torch.arange(T)] if layout == "temporal" else sinp
    if layout == "temporal":
        c4, s4 = pos_c[None, :, None, None, :], pos_s[None, :, None, None, :]
    else:
        c4, s4 = pos_c[None, None, :, None, :], pos_s[None, None, :, None, :]
    rq = oracle.apply_rope_swap(y[:, :, :, 0], c4, s4)     # [B,T,P,H,64]
    rk = oracle.apply_rope_swap(y[:, :, :, 1], c4, s4)
    rv = y[:, :, :, 2]
    perm = (0, 2, 3, 1, 4) if layout == "temporal" else (0, 1, 3, 2, 4)
    for name, got, ref in (("q", q, rq), ("k", k, rk), ("v", v, rv)):
        assert_close(got, ref.permute(*perm).contiguous(), 0.99999, 1e-2, "qkv_rope %s tile %d %s" % (layout, tile, name))


def test_gemm_unpatchify():
    gh, gw, ps, D = 18, 32, 20, 256
    M, N = gh * gw, 3 * ps * ps
    g = _gen(6)
    A = torch.randn(M, D, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, D, generator=g) * 0.1).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    frame = torch.zeros(3, gh * ps, gw * ps, device="cuda")
    _gemm(dev(A), dev(W), M, N, D, _epi(kind=L.EPI_UNPATCHIFY, bias=dev(bias), out_f32=frame, rows_per_frame=M,
                                          unpatch_grid_w=gw, unpatch_patch=ps, unpatch_channels=3))
    sync()
    ref = oracle.vae_unpatchify(A.float() @ W.float().t() + bias, gh, gw, ps)
    assert_close(frame, ref, 0.999999, 1e-4, "unpatchify epilogue")


def test_gemm_rejects_bad_shapes():
    A = torch.zeros(4, 96, device="cuda", dtype=torch.bfloat16)
    out = torch.zeros(4, 8, device="cuda")
    with pytest.raises(L.OasisError, match="multiple of 64"):
        _gemm(A, A, 4, 8, 96, _epi(kind=L.EPI_STORE_F32, out_f32=out, ld_out=8))
    # rows are addressed by 32-bit byte offsets from a tile's first row: leading dimensions of
    # 2^22 elements or more are refused before any launch (the pointers are never dereferenced)
    with pytest.raises(L.OasisError, match="below 2\\^22"):
        _gemm(A, A, 4, 8, 64, _epi(kind=L.EPI_STORE_F32, out_f32=out, ld_out=8), lda=1 << 22)


@pytest.mark.parametrize("layout", [0, 1])
def test_linear_surface(layout):
    M, K, N = 160, 1024, 320
    g = _gen(7)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(K, N, generator=g) * 0.05).to(torch.bfloat16)
    wd = dev(w) if layout == 0 else dev(w.t().contiguous())
    out = torch.zeros(M, N, device="cuda")
    L.call("oasis_linear", L.ptr(dev(x)), L.ptr(wd), L.ptr(out), M, K, N, layout, L.F32, stream())
    sync()
    assert_close(out, x.float() @ w.float(), 0.999999, 1e-4, "linear layout %d" % layout)


# ---------------------------------------------------------------- norms
def test_ln_modulate():
    M, D, P = 288, 1024, 144
    g = _gen(8)
    x = torch.randn(M, D, generator=g) * 3 + 1
    ada = torch.randn(2, 4 * D, generator=g) * 0.2
    shift, scale_p1 = ada[:, :D], ada[:, D:2 * D] + 1
    ada[:, D:2 * D] += 1
    out = torch.zeros(M, D, device="cuda", dtype=torch.bfloat16)
    ad = dev(ada)
    L.call("oasis_ln_modulate", L.ptr(dev(x)), M, D, L.ptr(ad[0, :]), L.ptr(ad[0, D:]), 4 * D, P, L.ptr(out),
           1e-6, stream())
    sync()
    f = torch.arange(M) // P
    ref = oracle.layer_norm(x) * scale_p1[f] + shift[f]
    assert_close(out, ref, 0.99999, 1e-2, "ln_modulate")


@pytest.mark.parametrize("dtype,cols,expanded", [(torch.float32, 1024, False), (torch.bfloat16, 1024, False),
                                                 (torch.bfloat16, 256, True), (torch.float32, 512, True),
                                                 (torch.bfloat16, 2048, False), (torch.bfloat16, 4096, True)])
def test_layernorm_surface(dtype, cols, expanded):
    """Every column count the kernel takes (256: 4 floats per lane; 512 and up: 16-byte vectors),
    with [cols] affine vectors or the reference's row-expanded [rows, cols] ones."""
    rows = 160
    g = _gen(9)
    x = (torch.randn(rows, cols, generator=g) * 2).to(dtype)
    w = torch.randn(rows if expanded else 1, cols, generator=g)
    b = torch.randn(rows if expanded else 1, cols, generator=g)
    out = torch.zeros(rows, cols, device="cuda", dtype=dtype)
    L.call("oasis_layernorm", L.ptr(dev(x)), L.ptr(dev(w)), L.ptr(dev(b)), cols if expanded else 0, L.ptr(out),
           rows, cols, 1e-6, L.F32 if dtype == torch.float32 else L.BF16, stream())
    sync()
    ref = oracle.layer_norm(x.float(), w, b)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert_close(out, ref, 0.9999, tol, "layernorm %s" % dtype)


def test_ln_affine():
    M, D = 576, 1024
    g = _gen(10)
    x = torch.randn(M, D, generator=g)
    w = torch.randn(D, generator=g)
    b = torch.randn(D, generator=g)
    out = torch.zeros(M, D, device="cuda", dtype=torch.bfloat16)
    L.call("oasis_ln_affine", L.ptr(dev(x)), M, D, L.ptr(dev(w)), L.ptr(dev(b)), L.ptr(out), 1e-6, stream())
    sync()
    assert_close(out, oracle.layer_norm(x, w, b), 0.99999, 1e-2, "ln_affine")


# ---------------------------------------------------------------- attention
@pytest.mark.parametrize("L_,F_", [(144, 2), (144, 5), (576, 2), (37, 2), (144, 64), (160, 2), (192, 2),
                                   (150, 64), (240, 2), (600, 1), (1152, 1)])
def test_attention_heads_first(L_, F_):
    """Frames of L_ tokens: a whole frame staged at once (up to 160 or 192 keys), the VAE's
    576, a ragged 37. At L = 144: up to 16 (frame, head) pairs take one workgroup per 16-query
    block (2 x 4 heads), up to 255 three blocks per workgroup (5 x 4), and 64 frames x 4 heads
    (256 pairs) the 9-wave one-workgroup-per-frame path. From 193 keys two waves share each 16-query block, each taking every other 64-key
    chunk: 240 (48-query workgroups), 600 (a ragged second 576-key stage where only one of the
    two waves has a chunk) and 1152 (two full stages)."""
    H = 4
    g = _gen(11 + L_)
    q, k, v = (torch.randn(F_ * H, L_, 64, generator=g).to(torch.bfloat16) for _ in range(3))
    out = torch.zeros(F_ * L_, H * 64, device="cuda", dtype=torch.bfloat16)
    L.call("oasis_attention", L.ptr(dev(q)), L.ptr(dev(k)), L.ptr(dev(v)), L.ptr(out), F_, L_, H, 0.125, stream())
    sync()
    ref = oracle.attention(q.float(), k.float(), v.float())          # [F*H, L, 64]
    ref = ref.reshape(F_, H, L_, 64).permute(0, 2, 1, 3).reshape(F_ * L_, H * 64)
    assert_close(out, ref, 0.9999, 1e-2, "attention L=%d" % L_)


@pytest.mark.parametrize("dtype,causal,bias,n", [(torch.float32, False, False, 32), (torch.bfloat16, True, False, 32),
                                                 (torch.float32, False, True, 32), (torch.bfloat16, True, False, 320),
                                                 (torch.float32, False, True, 320), (torch.bfloat16, False, True, 320)])
def test_sdpa_surface(dtype, causal, bias, n):
    """n = 320: the key-split kernel with a causal mask (whole chunks masked for one of the two
    waves of the first query blocks) and with the additive bias."""
    nh, sq, skv = 6, n, n
    g = _gen(12)
    Q, K, V = (torch.randn(nh * sq, 64, generator=g).to(dtype) for _ in range(3))
    bmask = None
    if bias:  # the reference's block-diagonal causal bias (oasis_inference.py:843-857), T=2 pairs
        bmask = torch.zeros(sq, skv)
        for i in range(sq):
            for j in range(skv):
                if i // 2 != j // 2 or j % 2 > i % 2:
                    bmask[i, j] = -1e4
    out = torch.zeros(nh * sq, 64, device="cuda", dtype=dtype)
    L.call("oasis_sdpa", L.ptr(dev(Q)), L.ptr(dev(K)), L.ptr(dev(V)), L.ptr(out), nh, sq, skv, 64, 0.125,
           L.ptr(None if bmask is None else dev(bmask)), int(causal), L.F32 if dtype == torch.float32 else L.BF16,
           stream())
    sync()
    q4, k4, v4 = (t.float().reshape(nh, sq, 64) for t in (Q, K, V))
    if bias:
        s = q4 @ k4.transpose(1, 2) * 0.125 + bmask
        ref = torch.softmax(s, -1) @ v4
    else:
        ref = oracle.attention(bf(q4), bf(k4), bf(v4), causal=causal)
    assert_close(out, ref.reshape(nh * sq, 64), 0.9999, 2e-2, "sdpa %s causal=%s bias=%s" % (dtype, causal, bias))


@pytest.mark.parametrize("T", [1, 2, 5, 8, 32, 48])
def test_temporal_attention(T):
    B_, P, H = 2, 144, 4
    g = _gen(13 + T)
    q, k, v = (torch.randn(B_, P, H, T, 64, generator=g).to(torch.bfloat16) for _ in range(3))
    out = torch.zeros(B_ * T * P, H * 64, device="cuda", dtype=torch.bfloat16)
    L.call("oasis_temporal_attention", L.ptr(dev(q)), L.ptr(dev(k)), L.ptr(dev(v)), L.ptr(out), B_, T, P, H,
           0.125, stream())
    sync()
    ref = oracle.attention(q.float(), k.float(), v.float(), causal=True)   # [B,P,H,T,64]
    ref = ref.permute(0, 3, 1, 2, 4).reshape(B_ * T * P, H * 64)
    assert_close(out, ref, 0.9999, 1e-2, "temporal T=%d" % T)
    if T == 1:  # a single causal key: out == v exactly (bf16 round trip)
        assert torch.equal(out.cpu(), v.permute(0, 3, 1, 2, 4).reshape(B_ * T * P, H * 64))


@pytest.mark.parametrize("B_,T_", [(1, 2), (2, 2), (1, 1), (3, 1)])
def test_temporal_qkv_attention(B_, T_):
    """QKV projection + temporal RoPE + causal attention of a two-frame window in one kernel,
    against the oracle's temporal branch. T = 2: both frames, with the K/V cache written
    (slot t = frame t's rotated K and its V). T = 1: the current frame (RoPE position 1) against
    a cache whose slot 0 holds the context frame's rotated K and V; the cache is read only."""
    P, H = 144, 4
    D = 64 * H
    g = _gen(170 + 10 * B_ + T_)
    h = torch.randn(B_ * T_ * P, D, generator=g).to(torch.bfloat16)
    W = (torch.randn(3 * D, D, generator=g) * 0.05).to(torch.bfloat16)
    cos, sp = oracle.rope_cos_sinperm(oracle.temporal_rope_angles(pkg.synth.theta_freqs(32, 64), 2), 64)
    kc0 = (torch.randn(B_, P, H, 2, 64, generator=g) * 2).to(torch.bfloat16)
    vc0 = torch.randn(B_, P, H, 2, 64, generator=g).to(torch.bfloat16)
    kc, vc = dev(kc0), dev(vc0)
    out = torch.zeros(B_ * T_ * P, D, device="cuda", dtype=torch.bfloat16)
    L.call("oasis_temporal_qkv_attention", L.ptr(dev(h)), D, L.ptr(dev(W)), L.ptr(out), B_, T_, P, H,
           L.ptr(dev(cos.contiguous())), L.ptr(dev(sp.contiguous())), L.ptr(kc), L.ptr(vc), 0.125, stream())
    sync()
    qkv = (h.float() @ W.float().t()).reshape(B_, T_, P, 3 * D)
    q, k, v = qkv[..., :D], qkv[..., D:2 * D], qkv[..., 2 * D:]
    got = out.cpu().reshape(B_, T_, P, D)
    if T_ == 2:
        for b in range(B_):
            ref = oracle.temporal_attention(q[b], k[b], v[b], cos, sp, H)          # [T, P, D]
            assert_close(got[b], ref, 0.9999, 1e-2, "temporal qkv T=2 stream %d" % b)
        kr = oracle.apply_rope_swap(k.reshape(B_, 2, P, H, 64), cos[None, :, None, None, :],
                                    sp[None, :, None, None, :])
        assert_close(kc.cpu(), kr.permute(0, 2, 3, 1, 4), 0.99999, 1e-2, "temporal qkv cache K")
        assert_close(vc.cpu(), v.reshape(B_, 2, P, H, 64).permute(0, 2, 3, 1, 4), 0.99999, 1e-2, "cache V")
    else:
        qh = oracle.apply_rope_swap(q.reshape(B_, P, H, 64), cos[1], sp[1])
        k1 = oracle.apply_rope_swap(k.reshape(B_, P, H, 64), cos[1], sp[1])
        keys = torch.stack([kc0[:, :, :, 0].float(), k1], 3)                       # [B, P, H, 2, 64]
        vals = torch.stack([vc0[:, :, :, 0].float(), v.reshape(B_, P, H, 64)], 3)
        p = torch.softmax((qh[:, :, :, None, :] * keys).sum(-1) / 8.0, -1)          # [B, P, H, 2]
        ref = (p[..., None] * vals).sum(3).reshape(B_, P, D)
        assert_close(got[:, 0], ref, 0.9999, 1e-2, "temporal qkv T=1")
        assert torch.equal(kc.cpu(), kc0) and torch.equal(vc.cpu(), vc0), "T=1 must not write the cache"


# ---------------------------------------------------------------- skinny GEMM
@pytest.mark.parametrize("R,K,N,act_in,act_out,acc", [(2, 1024, 6144 * 2 + 2048, 1, 0, 0), (5, 256, 1024, 0, 1, 0),
                                                       (16, 1024, 1024, 0, 0, 1), (1, 64, 1024, 0, 0, 0),
                                                       (32, 1024, 2048, 1, 0, 0), (23, 256, 1024, 0, 1, 1),
                                                       (70, 1024, 512, 0, 0, 1), (40, 2048, 256, 0, 0, 0),
                                                       (3, 128, 1040, 0, 0, 0), (4, 192, 528, 1, 0, 1),
                                                       (17, 512, 1040, 0, 1, 0)])
def test_gemv(R, K, N, act_in, act_out, acc):
    """Large N: one wave per 16-row weight tile. Small N: 4 waves (K = 128: 2; K = 192: 1) share
    each tile over K quarters, with tile counts that leave the last workgroup's second tile
    slot empty (N = 1040 with 2 waves per tile)."""
    g = _gen(14 + R)
    x = torch.randn(R, K, generator=g)
    W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, generator=g)
    out0 = torch.randn(R, N, generator=g)
    out = dev(out0)
    L.call("oasis_gemv_bf16", L.ptr(dev(x)), K, R, L.ptr(dev(W)), N, K, L.ptr(dev(b)), L.ptr(out), N, act_in,
           act_out, acc, stream())
    sync()
    xi = oracle.silu(x) if act_in else x
    ref = xi.double() @ W.double().t() + b.double()
    if act_out:
        ref = oracle.silu(ref)
    if acc:
        ref = ref + out0.double()
    # x is split into bf16 hi+lo, so the result keeps ~fp32 accuracy
    assert_close(out, ref, 0.9999999, 1e-4, "gemv R=%d K=%d N=%d" % (R, K, N))
    # the same weights in 16-row tile order give the same bits
    out_t = dev(out0)
    L.call("oasis_gemv_bf16_tiled", L.ptr(dev(x)), K, R, L.ptr(dev(pkg.model.tile_rows16(W))), N, K, L.ptr(dev(b)),
           L.ptr(out_t), N, act_in, act_out, acc, stream())
    sync()
    assert torch.equal(out_t, out), "tiled gemv R=%d K=%d N=%d" % (R, K, N)


@pytest.mark.parametrize("R,K,N,act_in,act_out,acc", [(2, 1024, 2048, 1, 0, 0), (5, 256, 1024, 2, 1, 0),
                                                       (5, 1024, 1024, 0, 0, 1), (13, 64, 1024, 0, 0, 0),
                                                       (3, 4096, 20, 1, 1, 1), (80, 256, 1024, 2, 1, 0)])
def test_gemv_f32(R, K, N, act_in, act_out, acc):
    """fp32 weights and arithmetic: within 1e-6 of an fp64 product (the bf16 GEMV keeps ~1e-5).
    act_in 2 forms the timestep embedding of x[r, 0] in LDS; 13 and 80 rows take 2 and 10
    passes of 8 rows; N = 20 leaves part of a wave's 4-row group past N."""
    g = _gen(40 + R)
    if act_in == 2:
        x = torch.rand(R, 1, generator=g) * 1000
    else:
        x = torch.randn(R, K, generator=g)
    W = torch.randn(N, K, generator=g) * 0.02
    b = torch.randn(N, generator=g)
    out0 = torch.randn(R, N, generator=g)
    out = dev(out0)
    L.call("oasis_gemv_f32", L.ptr(dev(x)), x.shape[1], R, L.ptr(dev(W)), N, K, L.ptr(dev(b)), L.ptr(out), N,
           act_in, act_out, acc, stream())
    sync()
    if act_in == 2:
        xi = oracle.timestep_embedding(x[:, 0].double(), K).double()
    else:
        xi = oracle.silu(x.double()) if act_in else x.double()
    ref = xi @ W.double().t() + b.double()
    if act_out:
        ref = oracle.silu(ref)
    if acc:
        ref = ref + out0.double()
    err = ((out.double().cpu() - ref).abs().max() / ref.abs().max()).item()
    print("gemv_f32 R=%d K=%d N=%d: max rel %.2e" % (R, K, N, err), flush=True)
    assert err < (2e-5 if act_in == 2 else 1e-6), err


# ---------------------------------------------------------------- small ops
def test_timestep_embedding():
    t = torch.tensor([0.0, 14.0, 249.0, 999.0, 517.0])
    out = torch.zeros(5, 256, device="cuda")
    L.call("oasis_timestep_embedding", L.ptr(dev(t)), 5, 256, L.ptr(out), stream())
    sync()
    assert_close(out, oracle.timestep_embedding(t), 0.9999999, 2e-4, "timestep embedding")


def test_small_linear_and_ddim_and_bridge():
    g = _gen(15)
    x = torch.randn(144, 64, generator=g)
    W = (torch.randn(1024, 64, generator=g) * 0.05).to(torch.bfloat16)
    b = torch.randn(1024, generator=g)
    out = torch.zeros(144, 1024, device="cuda")
    L.call("oasis_small_linear", L.ptr(dev(x)), 64, 144, 64, L.ptr(dev(W)), L.BF16, 0, 1024, L.ptr(dev(b)),
           L.ptr(out), 1024, stream())
    sync()
    assert_close(out, x @ W.float().t() + b, 0.9999999, 1e-5, "small_linear")
    # fp32 weights (the patch embed's W_rt), both layouts: fp32 arithmetic, against an fp64 product
    W32 = torch.randn(1024, 64, generator=g) * 0.05
    ref = x.double() @ W32.double().t() + b.double()
    for layout, wt in ((0, W32), (1, W32.t().contiguous())):
        out.zero_()
        L.call("oasis_small_linear", L.ptr(dev(x)), 64, 144, 64, L.ptr(dev(wt)), L.F32, layout, 1024, L.ptr(dev(b)),
               L.ptr(out), 1024, stream())
        sync()
        assert ((out.double().cpu() - ref).abs().max() / ref.abs().max()).item() < 1e-6, layout
    for M in (147, 2050):  # ragged row blocks of the 4-row and 16-row variants
        xm = torch.randn(M, 40, generator=g)
        Wm = (torch.randn(1000, 32, generator=g) * 0.05).to(torch.bfloat16)
        om = torch.full((M, 1000), 7.0, device="cuda")
        L.call("oasis_small_linear", L.ptr(dev(xm)), 40, M, 32, L.ptr(dev(Wm)), L.BF16, 0, 1000, None, L.ptr(om),
               1000, stream())
        sync()
        assert_close(om, xm[:, :32] @ Wm.float().t(), 0.9999999, 1e-5, "small_linear M=%d" % M)

    ac = oracle.cosine_alphas_cumprod()
    v = torch.randn(144, 64, generator=g)
    chunk = dev(x)
    c = oracle.ddim_coeffs(ac, 749, 499, last=False)
    L.call("oasis_ddim_update", L.ptr(chunk), L.ptr(dev(v)), chunk.numel(), *[ctypes.c_float(z) for z in c],
           stream())
    sync()
    assert_close(chunk, oracle.ddim_update(x, v, c), 0.9999999, 1e-5, "ddim update")

    lat = torch.zeros(576, 32, device="cuda")
    L.call("oasis_bridge", L.ptr(dev(x)), L.ptr(lat), 9, 16, 16, 32, 1.0 / oracle.SCALING_FACTOR, stream())
    sync()
    assert torch.allclose(lat.cpu(), oracle.bridge(x), rtol=1e-6, atol=1e-6)

    patches = torch.randn(576, 1200, generator=g) * 2
    frame = torch.zeros(3, 360, 640, device="cuda")
    L.call("oasis_vae_unpatchify", L.ptr(dev(patches)), L.ptr(frame), 18, 32, 20, stream())
    sync()
    assert torch.equal(frame.cpu(), oracle.vae_unpatchify(patches))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,off", [(160 * 1024 + 3, 0), (5, 0), (160 * 1024 + 3, 1)])
def test_elementwise_surface(dtype, n, off):
    """16-byte vectors with a ragged tail (off 0), fewer elements than one vector, and operands one
    element off 16-byte alignment (off 1: the one-element-per-step kernel)."""
    g = _gen(16)
    a, b, c, d = (torch.randn(n, generator=g).to(dtype) for _ in range(4))
    code = L.F32 if dtype == torch.float32 else L.BF16
    out = torch.zeros(n + off, device="cuda", dtype=dtype)[off:]
    A, Bd, C, Dd = (torch.cat([torch.zeros(off, dtype=dtype), t]).cuda()[off:] for t in (a, b, c, d))
    af, bf_, cf, df = a.float(), b.float(), c.float(), d.float()
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    L.call("oasis_silu", L.ptr(A), L.ptr(out), n, code, stream())
    sync()
    assert_close(out, oracle.silu(af), 0.99999, tol, "silu")
    L.call("oasis_adaln_modulate", L.ptr(A), L.ptr(Bd), L.ptr(C), L.ptr(out), n, code, stream())
    sync()
    assert_close(out, oracle.modulate(af, bf_, cf), 0.99999, tol, "modulate")
    L.call("oasis_gated_residual", L.ptr(A), L.ptr(Bd), L.ptr(C), L.ptr(out), n, code, stream())
    sync()
    assert_close(out, af + bf_ * cf, 0.99999, tol, "gated_residual")
    L.call("oasis_bias_gated_residual", L.ptr(A), L.ptr(Bd), L.ptr(C), L.ptr(Dd), L.ptr(out), n, code, stream())
    sync()
    assert_close(out, af + (bf_ + cf) * df, 0.99999, tol, "bias_gated_residual")


@pytest.mark.parametrize("dt,mode", [(torch.float32, 0), (torch.bfloat16, 0), (torch.bfloat16, 1),
                                     (torch.float32, 1)])
def test_rope_layout_surface(dt, mode):
    """Reference-layout inputs: qkv_full [SEQ, 5D] with swap columns and [SEQ, D] tables; heads-first
    (mode 0) and token-major (mode 1) outputs, fp32 and bf16."""
    T, S, H = 2, 160, 4
    D = H * 64
    g = _gen(17)
    qkv = torch.randn(T * S, 5 * D, generator=g).to(dt).float()
    ang = oracle.spatial_rope_angles(torch.rand(16, generator=g), 9, 16)
    cos, sinp = oracle.rope_cos_sinperm(ang, 64)
    ctab = torch.zeros(T * S, D)
    stab = torch.zeros(T * S, D)
    for t in range(T):
        ctab[t * S:t * S + 144] = cos.repeat(1, H)
        stab[t * S:t * S + 144] = sinp.repeat(1, H)
    qo, ko, vo = (torch.zeros(T * H * S, 64, device="cuda", dtype=dt) for _ in range(3))
    L.call("oasis_rope_layout", L.ptr(dev(qkv.to(dt))), 5 * D, L.ptr(dev(ctab)), L.ptr(dev(stab)), D, 64, 1, T * S,
           L.ptr(qo), L.ptr(ko), L.ptr(vo), T * S, S, H, 64, mode, L.F32 if dt == torch.float32 else L.BF16,
           stream())
    sync()
    x = qkv.reshape(T, S, 5, H, 64)
    c4 = ctab.reshape(T, S, H, 64)
    s4 = stab.reshape(T, S, H, 64)
    tol = 1e-5 if dt == torch.float32 else 8e-3

    def layout(t):   # [T, S, H, 64] -> the output layout of the mode
        return t.permute(0, 2, 1, 3).reshape(-1, 64) if mode == 0 else t.reshape(-1, 64)
    for i, (name, got) in enumerate((("q", qo), ("k", ko))):
        ref = layout(oracle.apply_rope_swap(x[:, :, i], c4, s4))
        assert_close(got.float(), ref, 0.99999, tol, "rope_layout %s %s mode %d" % (name, dt, mode))
    assert torch.equal(vo.float().cpu(), layout(x[:, :, 2]))


@pytest.mark.parametrize("H,T", [(16, 5), (4, 3), (2, 21), (40, 2)])
def test_rope_layout_shared_positions(H, T):
    """T frames of 144 positions over one [144, D] table (pos_mod = 144, the layout the bench
    times): the rows of a position share its table row, one workgroup each; with H = 40 the 320
    column groups of a row stride over 256 threads. bf16, both output layouts."""
    P, D = 144, H * 64
    g = _gen(29 + H)
    qkv = torch.randn(T * P, 3 * D, generator=g).to(torch.bfloat16)
    cs, sn = torch.randn(P, D, generator=g), torch.randn(P, D, generator=g)
    x = qkv.float().reshape(T, P, 3, H, 64)
    c4 = cs.reshape(1, P, H, 64).expand(T, P, H, 64)
    s4 = sn.reshape(1, P, H, 64).expand(T, P, H, 64)
    for mode in (0, 1):
        qo, ko, vo = (torch.zeros(T * P * H, 64, device="cuda", dtype=torch.bfloat16) for _ in range(3))
        L.call("oasis_rope_layout", L.ptr(dev(qkv)), 3 * D, L.ptr(dev(cs)), L.ptr(dev(sn)), D, 64, 1, P,
               L.ptr(qo), L.ptr(ko), L.ptr(vo), T * P, P, H, 64, mode, L.BF16, stream())
        sync()

        def layout(t):   # [T, P, H, 64] -> the output layout of the mode
            return t.permute(0, 2, 1, 3).reshape(-1, 64) if mode == 0 else t.reshape(-1, 64)
        for i, (name, got) in enumerate((("q", qo), ("k", ko))):
            ref = layout(oracle.apply_rope_swap(x[:, :, i], c4, s4))
            assert_close(got.float(), ref, 0.99999, 8e-3, "rope_layout H=%d T=%d %s mode %d" % (H, T, name, mode))
        assert torch.equal(vo.float().cpu(), layout(x[:, :, 2])), (H, T, mode)


# ---------------------------------------------------------------- tile configs, split-K, fused LN
@pytest.mark.parametrize("tile", list(range(18)))
def test_gemm_tile_configs(tile):
    M, N, K = 288, 1024, 1024
    g = _gen(30 + tile)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    out = torch.zeros(M, N, device="cuda")
    e = _epi(kind=L.EPI_STORE_F32, out_f32=out, ld_out=N)
    L.call("oasis_gemm_bf16_config", L.ptr(dev(A)), K, L.ptr(dev(B)), K, M, N, K, ctypes.byref(e), tile, 1, stream())
    sync()
    assert_close(out, A.float() @ B.float().t(), 0.999999, 1e-4, "tile %d" % tile)


@pytest.mark.parametrize("tile", list(range(5)))
def test_gemm_direct_lds_ragged(tile):
    """The direct-to-LDS configurations (0, 1, and 2-4 on the 8-wave kernel's code) on a ragged
    shape: K = 5 tiles (not a multiple of the stage count), M and N not multiples of the tile,
    GELU epilogue and split-K slices."""
    M, N, K = 300, 520, 320
    g = _gen(60 + tile)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    out = torch.zeros(M, N, device="cuda", dtype=torch.bfloat16)
    e = _epi(kind=L.EPI_GELU_TANH, bias=dev(bias), out_bf16=out, ld_out=N)
    L.call("oasis_gemm_bf16_config", L.ptr(dev(A)), K, L.ptr(dev(B)), K, M, N, K, ctypes.byref(e), tile, 1, stream())
    part = torch.zeros(5, M, N, device="cuda")
    ep = _epi(kind=L.EPI_PARTIAL_F32, out_f32=part, ld_out=N, split_stride=M * N)
    L.call("oasis_gemm_bf16_config", L.ptr(dev(A)), K, L.ptr(dev(B)), K, M, N, K, ctypes.byref(ep), tile, 5, stream())
    sync()
    ref = A.float() @ B.float().t()
    assert_close(out, torch.nn.functional.gelu(ref + bias, approximate="tanh"), 0.99999, 1e-2, "tile %d gelu" % tile)
    assert_close(part.sum(0), ref, 0.999999, 1e-4, "tile %d split-K x5" % tile)


@pytest.mark.parametrize("tile", list(range(8, 13)))
def test_gemm_wave_tiles_ragged(tile):
    """The wave-split tiles (8-12: four waves split each K slice, each over its own LDS ring; 8
    computes 80-row tiles every 72 rows) on a ragged shape (M and N not multiples of the tile) with every K-loop length they unroll: GELU
    with K = 1024 (4 K tiles per wave, the GELU kernel), split-K x2 of K = 1024 (2 tiles, the
    split-K kernel), one K = 2048 slice (8 tiles) and K = 256 (1 tile, the generic kernel); K
    slices that are not 256 x a power of two are refused."""
    M, N = 300, 520
    g = _gen(120 + tile)
    # 4096 columns, so the refused shapes below stay in bounds should a check ever let one through
    A = torch.randn(M, 4096, generator=g).to(torch.bfloat16)
    B = (torch.randn(N, 4096, generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    Ad, Bd = dev(A), dev(B)

    def ref(K):
        return A[:, :K].float() @ B[:, :K].float().t()
    out = torch.zeros(M, N, device="cuda", dtype=torch.bfloat16)
    e = _epi(kind=L.EPI_GELU_TANH, bias=dev(bias), out_bf16=out, ld_out=N)
    L.call("oasis_gemm_bf16_config", L.ptr(Ad), 4096, L.ptr(Bd), 4096, M, N, 1024, ctypes.byref(e), tile, 1, stream())
    part = torch.zeros(2, M, N, device="cuda")
    ep = _epi(kind=L.EPI_PARTIAL_F32, out_f32=part, ld_out=N, split_stride=M * N)
    L.call("oasis_gemm_bf16_config", L.ptr(Ad), 4096, L.ptr(Bd), 4096, M, N, 1024, ctypes.byref(ep), tile, 2, stream())
    part8 = torch.zeros(1, M, N, device="cuda")
    ep8 = _epi(kind=L.EPI_PARTIAL_F32, out_f32=part8, ld_out=N, split_stride=M * N)
    L.call("oasis_gemm_bf16_config", L.ptr(Ad), 4096, L.ptr(Bd), 4096, M, N, 2048, ctypes.byref(ep8), tile, 1, stream())
    o32 = torch.zeros(M, N, device="cuda")
    e32 = _epi(kind=L.EPI_STORE_F32, bias=dev(bias), out_f32=o32, ld_out=N)
    L.call("oasis_gemm_bf16_config", L.ptr(Ad), 4096, L.ptr(Bd), 4096, M, N, 256, ctypes.byref(e32), tile, 1, stream())
    sync()
    r1 = ref(1024)
    assert_close(out, torch.nn.functional.gelu(r1 + bias, approximate="tanh"), 0.99999, 1e-2, "tile %d gelu" % tile)
    assert_close(part.sum(0), r1, 0.999999, 1e-4, "tile %d split-K x2" % tile)
    assert_close(part8[0], ref(2048), 0.999999, 1e-4, "tile %d K=2048" % tile)
    assert_close(o32, ref(256) + bias, 0.999999, 1e-4, "tile %d K=256" % tile)
    for K, splits in ((320, 1), (768, 1), (4096, 1)):
        with pytest.raises(L.OasisError):
            L.call("oasis_gemm_bf16_config", L.ptr(Ad), 4096, L.ptr(Bd), 4096, M, N, K, ctypes.byref(e32), tile,
                   splits, stream())


@pytest.mark.parametrize("tile", list(range(5, 8)))
def test_gemm_large_token_tiles_ragged(tile):
    """The 8-wave large-token tiles on a ragged shape: M and N not multiples of the tile (the
    last tile row and column are partial), K = 5 tiles, GELU epilogue with bias, split-K x5,
    and the 4608 x 4096 x 1024 product they are sized for."""
    M, N, K = 600, 520, 320
    g = _gen(90 + tile)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    out = torch.zeros(M, N, device="cuda", dtype=torch.bfloat16)
    e = _epi(kind=L.EPI_GELU_TANH, bias=dev(bias), out_bf16=out, ld_out=N)
    L.call("oasis_gemm_bf16_config", L.ptr(dev(A)), K, L.ptr(dev(B)), K, M, N, K, ctypes.byref(e), tile, 1, stream())
    part = torch.zeros(5, M, N, device="cuda")
    ep = _epi(kind=L.EPI_PARTIAL_F32, out_f32=part, ld_out=N, split_stride=M * N)
    L.call("oasis_gemm_bf16_config", L.ptr(dev(A)), K, L.ptr(dev(B)), K, M, N, K, ctypes.byref(ep), tile, 5, stream())
    sync()
    ref = A.float() @ B.float().t()
    assert_close(out, torch.nn.functional.gelu(ref + bias, approximate="tanh"), 0.99999, 1e-2, "tile %d gelu" % tile)
    assert_close(part.sum(0), ref, 0.999999, 1e-4, "tile %d split-K x5" % tile)
    M, N, K = 4608, 4096, 1024
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    out = torch.zeros(M, N, device="cuda")
    e = _epi(kind=L.EPI_STORE_F32, out_f32=out, ld_out=N)
    Ad, Bd = dev(A), dev(B)
    L.call("oasis_gemm_bf16_config", L.ptr(Ad), K, L.ptr(Bd), K, M, N, K, ctypes.byref(e), tile, 1, stream())
    sync()
    assert_close(out, Ad.float() @ Bd.float().t(), 0.999999, 1e-4, "tile %d 4608x4096x1024" % tile)


@pytest.mark.parametrize("tile", [2, 3, 4, 5, 6, 7, 13, 14, 15, 16, 17])
def test_gemm_staged_epilogue_residuals(tile):
    """The per-wave staged epilogue's residual kinds (x and gate fetched a 16-row group ahead) on
    every tile of that kernel, on a ragged shape (the last tile row and column partial, lanes with
    no unit where a wave's tile is 16 or 48 columns wide) whose 100-row frames change the gate row
    inside tiles and 16-row groups: gated residual, then plain residual, into the same x."""
    M, N, K, P = 600, 520, 320, 100
    g = _gen(150 + tile)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    x0 = torch.randn(M, N, generator=g)
    fstride = 2 * N
    ada = torch.randn(M // P, fstride, generator=g)
    x, ada_d = dev(x0), dev(ada)
    Ad, Bd = dev(A), dev(B)
    e = _epi(kind=L.EPI_GATED_RES, bias=dev(bias), out_f32=x, ld_out=N, gate=ada_d[0, N:], gate_fstride=fstride,
             rows_per_frame=P)
    L.call("oasis_gemm_bf16_config", L.ptr(Ad), K, L.ptr(Bd), K, M, N, K, ctypes.byref(e), tile, 1, stream())
    sync()
    y = A.float() @ B.float().t() + bias
    ref = x0 + ada[:, N:].repeat_interleave(P, 0) * y
    assert_close(x, ref, 0.999999, 1e-5, "tile %d gated residual" % tile)
    e = _epi(kind=L.EPI_RESIDUAL, bias=dev(bias), out_f32=x, ld_out=N)
    L.call("oasis_gemm_bf16_config", L.ptr(Ad), K, L.ptr(Bd), K, M, N, K, ctypes.byref(e), tile, 1, stream())
    sync()
    assert_close(x, ref + y, 0.999999, 1e-5, "tile %d residual" % tile)


def test_gemm_fp8_epilogue_needs_aligned_lanes():
    """A tile whose epilogue lanes do not cover whole 32-column blocks refuses GELU_TANH_FP8."""
    M, N, K = 288, 384, 64
    A = torch.zeros(M, K, device="cuda", dtype=torch.bfloat16)
    B = torch.zeros(N, K, device="cuda", dtype=torch.bfloat16)
    q = torch.zeros(M, N, device="cuda", dtype=torch.uint8)
    sc = torch.zeros(M, N // 32, device="cuda", dtype=torch.uint8)
    e = _epi(kind=L.EPI_GELU_TANH_FP8, out_fp8=q, out_scale=sc, ld_out=N, ld_scale=N // 32)
    with pytest.raises(L.OasisError):
        L.call("oasis_gemm_bf16_config", L.ptr(A), K, L.ptr(B), K, M, N, K, ctypes.byref(e), 47, 1, stream())


@pytest.mark.parametrize("splits", [1, 2, 4, 8])
def test_gemm_split_k_partials(splits):
    M, N, K = 288, 1024, 4096
    g = _gen(40 + splits)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    part = torch.zeros(splits, M, N, device="cuda")
    e = _epi(kind=L.EPI_PARTIAL_F32, out_f32=part, ld_out=N, split_stride=M * N)
    L.call("oasis_gemm_bf16_config", L.ptr(dev(A)), K, L.ptr(dev(B)), K, M, N, K, ctypes.byref(e), 0, splits,
           stream())
    sync()
    ref = A.float() @ B.float().t()
    assert_close(part.sum(0), ref, 0.999999, 1e-4, "split-K %d" % splits)
    kk = K // splits  # each slice is the product over its own K range
    assert_close(part[-1], A[:, -kk:].float() @ B[:, -kk:].float().t(), 0.999999, 1e-4, "last slice")


@pytest.mark.parametrize("np_,mode", [(0, "mod"), (4, "mod"), (2, "affine"), (3, "residual_only")])
def test_residual_ln(np_, mode):
    M, D, P = 288, 1024, 144
    g = _gen(50 + np_)
    x0 = torch.randn(M, D, generator=g) * 2
    part = torch.randn(max(np_, 1), M, D, generator=g)
    bias = torch.randn(D, generator=g)
    fs = 6 * D
    ada = torch.randn(2, fs, generator=g) * 0.3
    x = dev(x0)
    y = torch.zeros(M, D, device="cuda", dtype=torch.bfloat16)
    ada_d = dev(ada)
    f = torch.arange(M) // P
    if mode == "affine":
        w_aff, b_aff = torch.randn(D, generator=g), torch.randn(D, generator=g)
        la, lb, lfs, gate, gfs = dev(w_aff), dev(b_aff), 0, None, 0
    else:
        la, lb, lfs, gate, gfs = ada_d[0, D:], ada_d[0, :], fs, ada_d[0, 2 * D:], fs
    yp = None if mode == "residual_only" else y
    L.call("oasis_residual_ln", L.ptr(x), M, D, L.ptr(dev(part)), np_, M * D, L.ptr(dev(bias)), L.ptr(gate), gfs, P,
           L.ptr(la), L.ptr(lb), lfs, L.ptr(yp), 1e-6, stream())
    sync()
    xr = x0.clone()
    if np_ > 0:
        upd = part[:np_].sum(0) + bias
        xr = xr + (upd if mode == "affine" else ada[f, 2 * D:3 * D] * upd)
    assert_close(x, xr, 0.9999999, 1e-5, "residual (%s, %d partials)" % (mode, np_))
    if mode == "mod":
        assert_close(y, oracle.layer_norm(xr) * ada[f, D:2 * D] + ada[f, :D], 0.99999, 1e-2, "ln modulate")
    elif mode == "affine":
        assert_close(y, oracle.layer_norm(xr, w_aff, b_aff), 0.99999, 1e-2, "ln affine")


# ---------------------------------------------------------------- interactive-loop helpers
def test_noise_normal_and_frame_hwc():
    """oasis_noise_normal against the host Philox + Box-Muller (ragged n, the copy, the clamp, the
    counter bump: every call draws anew), and oasis_frame_hwc against torch."""
    n, seed = 9216 + 3, 0x1234_5678_9ABC
    out = torch.zeros(n, device="cuda")
    cp = torch.zeros(n, device="cuda")
    ctr = torch.zeros(1, dtype=torch.int32, device="cuda")
    draws = []
    for frame in range(3):
        L.call("oasis_noise_normal", L.ptr(out), L.ptr(cp), n, ctypes.c_uint64(seed), L.ptr(ctr), 20.0, stream())
        sync()
        got = out.cpu().double().numpy()
        ref = noise_reference(n, seed, frame, 20.0)
        assert abs(got - ref).max() < 1e-4, (frame, abs(got - ref).max())
        assert torch.equal(out, cp) and int(ctr.item()) == frame + 1
        draws.append(got)
    assert not (draws[0] == draws[1]).all()
    L.call("oasis_noise_normal", L.ptr(out), None, n, ctypes.c_uint64(seed), L.ptr(ctr), 0.5, stream())
    sync()
    assert out.abs().max().item() <= 0.5 and abs(out.cpu().double().numpy() - noise_reference(n, seed, 3, 0.5)).max() < 1e-4
    frame = torch.randn(3, 7, 11, generator=_gen(77)) * 1.3
    hwc = torch.zeros(7, 11, 3, device="cuda")
    L.call("oasis_frame_hwc", L.ptr(dev(frame)), L.ptr(hwc), 3, 7, 11, stream())
    sync()
    assert torch.equal(hwc.cpu(), ((frame + 1.0) * 0.5).clamp(0.0, 1.0).permute(1, 2, 0))
