"""The fp8 weight path on the GPU (config 4): the e4m3 weight quantizer, the block-scaled
fp8 GEMM against the oracle's quantized operands, the fp8 DiT step against the oracle with
dequantized weights, and the full config-4 batch (8 streams x T=4) against the bf16 path."""
import ctypes

import pytest
import torch

import oracle
from helpers import COS_SUB, REL_SUB, L, assert_close, cuda, metrics, pkg, stream, sync

pytestmark = pytest.mark.gpu

_ALIVE = []


def dev(t):
    t = cuda(t)
    _ALIVE.append(t)
    return t


@pytest.fixture(autouse=True)
def _release():
    yield
    torch.cuda.synchronize()
    _ALIVE.clear()


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _quantize(W):
    """Device quantizer on a bf16 [N, K] weight -> (q uint8 [N, K], scale [N]) on the GPU."""
    N, K = W.shape
    q = torch.empty(N, K, dtype=torch.uint8, device="cuda")
    s = torch.empty(N, device="cuda")
    Wd = dev(W)
    L.call("oasis_quantize_fp8_rows", L.ptr(Wd), N, K, L.ptr(q), L.ptr(s), stream())
    sync()
    return q, s


def test_quantize_rows_matches_torch_e4m3():
    W = (torch.randn(384, 1024, generator=_gen(1)) * 0.02).to(torch.bfloat16)
    W[5] = 0
    q, s = _quantize(W)
    ref_q, ref_s = oracle.quantize_e4m3_rows(W)
    assert torch.equal(s.cpu(), ref_s)
    got = q.cpu().view(torch.float8_e4m3fn).float()
    assert torch.equal(got, ref_q), (got - ref_q).abs().max()


def _epi(**kw):
    e = L.Epilogue()
    for k, v in kw.items():
        if isinstance(v, torch.Tensor):
            _ALIVE.append(v)
            v = v.data_ptr()
        setattr(e, k, v)
    return e


def _ref(A, W):
    """fp64 product of the operands exactly as the fp8 GEMM quantizes them."""
    q, s = oracle.quantize_e4m3_rows(W)
    return oracle.quantize_act_blocks(A).double() @ (q.double() * s.double()[:, None]).t()


# every tile on the small shapes; the 4608-row shape on the default and the wide tiles
_FP8_CASES = [(t, 300, 384, 512) for t in (-1, 0, 1, 2, 3, 4)] + [(t, 4608, 1024, 1024) for t in (-1, 0, 1)] + \
    [(t, 33, 64, 256) for t in (-1, 0, 1, 2, 3, 4)]


@pytest.mark.parametrize("tile,M,N,K", _FP8_CASES)
def test_gemm_fp8_store_f32(tile, M, N, K):
    g = _gen(M + N + K)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    A[:, :32] *= 100.0  # blocks of very different magnitude
    W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(N, generator=g)
    q, s = _quantize(W)
    out = torch.zeros(M, N, device="cuda")
    L.call("oasis_gemm_fp8", L.ptr(dev(A)), K, L.ptr(q), K, L.ptr(s), M, N, K,
           ctypes.byref(_epi(kind=L.EPI_STORE_F32, bias=dev(bias), out_f32=out, ld_out=N)), tile, 1, stream())
    sync()
    ref = _ref(A, W) + bias.double()
    cos, rel = metrics(out, ref)
    print("fp8 gemm %dx%dx%d tile %d: cos=%.7f rel=%.2e" % (M, N, K, tile, cos, rel), flush=True)
    assert rel <= 1e-4, rel  # fp32 accumulation against the fp64 reference


def test_gemm_fp8_gelu_and_split_k():
    M, N, K = 288, 512, 1024
    g = _gen(7)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    q, s = _quantize(W)
    out = torch.zeros(M, N, device="cuda", dtype=torch.bfloat16)
    L.call("oasis_gemm_fp8", L.ptr(dev(A)), K, L.ptr(q), K, L.ptr(s), M, N, K,
           ctypes.byref(_epi(kind=L.EPI_GELU_TANH, bias=dev(bias), out_bf16=out, ld_out=N)), -1, 1, stream())
    part = torch.zeros(4, M, N, device="cuda")
    L.call("oasis_gemm_fp8", L.ptr(dev(A)), K, L.ptr(q), K, L.ptr(s), M, N, K,
           ctypes.byref(_epi(kind=L.EPI_PARTIAL_F32, out_f32=part, ld_out=N, split_stride=M * N)), 3, 4, stream())
    sync()
    ref = _ref(A, W)
    assert_close(out, oracle.gelu_tanh((ref + bias.double()).float()), 0.99999, 1e-2, "fp8 gemm gelu")
    assert_close(part.sum(0), ref, 0.9999999, 1e-4, "fp8 gemm split-K x4")


def test_gemm_fp8_rejects_bad_shapes():
    e = _epi(kind=L.EPI_STORE_F32, out_f32=torch.zeros(1, device="cuda"), ld_out=64)
    fake = ctypes.c_void_p(16)
    with pytest.raises(L.OasisError, match="multiple of 128"):
        L.call("oasis_gemm_fp8", fake, 64, fake, 64, fake, 16, 64, 64, ctypes.byref(e), -1, 1, stream())


def _step(dit, c, B, T):
    P = dit.P
    step = pkg.DiTStep(dit, B=B, T=T)
    patches = oracle.patchify_to_output_space(c["latent"].reshape(B * T, 16, 18, 32)).reshape(-1, 64)
    step.set_inputs(cuda(patches), cuda(c["t"].reshape(-1)), cuda(c["actions"].reshape(B * T, -1)))
    v = step.run().clone()
    torch.cuda.synchronize()
    return v.cpu().reshape(B, T * P, 64), step


def test_fp8_dit_step_reduced_vs_oracle():
    """2 blocks at the full width, B=2 streams x T=4: the fp8 path against the fp32 oracle
    run on the dequantized e4m3 weights (the remaining gap is the activation quantization)."""
    c = pkg.synth.config4(seed=41, B=2, T=4, n_blocks=2)
    dit = pkg.DiT(c["w"], "cuda", weights="fp8")
    v, _ = _step(dit, c, 2, 4)
    w8 = oracle.fp8_weights(c["w"])
    for b in range(2):
        z = oracle.patch_embed(c["latent"][b], w8)
        cond = oracle.conditioning(c["t"][b], c["actions"][b], w8)
        ref = oracle.dit_forward(z, cond, w8).reshape(-1, 64)
        cos, rel = metrics(v[b], ref)
        print("fp8 reduced step stream %d vs oracle(e4m3 weights): cos=%.6f rel=%.3e" % (b, cos, rel), flush=True)
        assert cos >= 0.995, cos


def test_config4_fp8_vs_bf16():
    """Config 4 at full size: 8 streams x T=4 (4608 tokens), 16 blocks; the fp8 weight
    path must hold cosine >= 0.99 against the bf16 path on the same inputs."""
    c = pkg.synth.config4()
    v16, s16 = _step(pkg.DiT(c["w"], "cuda"), c, 8, 4)
    del s16
    torch.cuda.empty_cache()
    v8, _ = _step(pkg.DiT(c["w"], "cuda", weights="fp8"), c, 8, 4)
    worst = 1.0
    for b in range(8):
        cos, rel = metrics(v8[b], v16[b])
        worst = min(worst, cos)
    cos, rel = metrics(v8, v16)
    print("config4 fp8 vs bf16: cos=%.6f (worst stream %.6f) rel=%.3e" % (cos, worst, rel), flush=True)
    assert worst >= 0.99, worst


def test_config4_bf16_stream_matches_oracle():
    """One stream of the batched bf16 step equals the single-stream oracle (batch rows
    are independent): 2 blocks, B=8, T=4."""
    c = pkg.synth.config4(seed=42, n_blocks=2)
    v, _ = _step(pkg.DiT(c["w"], "cuda"), c, 8, 4)
    for b in (0, 5):
        z = oracle.patch_embed(c["latent"][b], c["w"])
        cond = oracle.conditioning(c["t"][b], c["actions"][b], c["w"])
        ref = oracle.dit_forward(z, cond, c["w"]).reshape(-1, 64)
        assert_close(v[b], ref, COS_SUB, REL_SUB, "config4 bf16 stream %d (2 blocks)" % b)


def test_quantize_act_fp8_matches_oracle():
    M, K = 300, 1024
    g = _gen(11)
    x = (torch.randn(M, K, generator=g) * torch.logspace(-3, 2, K // 32).repeat_interleave(32)).to(torch.bfloat16)
    x[7] = 0
    q = torch.zeros(M, K, dtype=torch.uint8, device="cuda")
    sc = torch.zeros(M, K // 32, dtype=torch.uint8, device="cuda")
    L.call("oasis_quantize_act_fp8", L.ptr(dev(x)), K, M, K, L.ptr(q), K, L.ptr(sc), K // 32, stream())
    sync()
    deq = q.cpu().view(torch.float8_e4m3fn).float() * torch.pow(2.0, sc.cpu().float() - 127).repeat_interleave(32, 1)
    assert torch.equal(deq, oracle.quantize_act_blocks(x))


@pytest.mark.parametrize("kind,F,T,H", [("spatial", 2, 1, 16), ("spatial", 1, 1, 4), ("temporal", 2, 2, 4),
                                         ("temporal", 2, 4, 4), ("temporal", 1, 13, 4), ("temporal", 1, 32, 2)])
def test_attention_fp8_output_equals_quantized_bf16(kind, F, T, H):
    """The attention kernels' fp8-block output (the fp8 step's O operand, written in the attention
    launch) is bit for bit oasis_quantize_act_fp8 of their bf16 output: the spatial flash kernel,
    the temporal VALU kernel (T = 2 and its general loop) and the causal flash kernel (T >= 8)."""
    P = 144
    rows = F * T * P
    D = H * 64
    g = _gen(300 + F * 7 + T * 13 + H)
    q, k, v = (dev((torch.randn(rows * D, generator=g) * 2).to(torch.bfloat16)) for _ in range(3))
    out = torch.zeros(rows, D, device="cuda", dtype=torch.bfloat16)
    o8 = torch.full((rows, D), 0x7F, dtype=torch.uint8, device="cuda")
    o8s = torch.full((rows, D // 32), 0xEE, dtype=torch.uint8, device="cuda")
    if kind == "spatial":
        print("attention fp8 spatial F=%d H=%d" % (F, H), flush=True)
        L.call("oasis_attention", L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(out), F, P, H, 0.125, stream())
        L.call("oasis_attention_fp8", L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(o8), L.ptr(o8s), F, P, H, 0.125, stream())
    else:
        print("attention fp8 temporal B=%d T=%d H=%d" % (F, T, H), flush=True)
        L.call("oasis_temporal_attention", L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(out), F, T, P, H, 0.125, stream())
        L.call("oasis_temporal_attention_fp8", L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(o8), L.ptr(o8s), F, T, P, H,
               0.125, stream())
    ref8 = torch.zeros(rows, D, dtype=torch.uint8, device="cuda")
    ref8s = torch.zeros(rows, D // 32, dtype=torch.uint8, device="cuda")
    L.call("oasis_quantize_act_fp8", L.ptr(out), D, rows, D, L.ptr(ref8), D, L.ptr(ref8s), D // 32, stream())
    sync()
    assert torch.equal(o8, ref8) and torch.equal(o8s, ref8s), (kind, F, T, H)


def test_gemm_fp8_a8_equals_in_kernel_quantization():
    """Pre-quantized A blocks give bit-identical results to quantizing A inside the GEMM,
    and the fp8 GELU epilogue writes the blocks the next fp8 GEMM reads."""
    M, N, K = 600, 1024, 1024
    g = _gen(12)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    q, s = _quantize(W)
    Ad = dev(A)
    a8 = torch.zeros(M, K, dtype=torch.uint8, device="cuda")
    a8s = torch.zeros(M, K // 32, dtype=torch.uint8, device="cuda")
    L.call("oasis_quantize_act_fp8", L.ptr(Ad), K, M, K, L.ptr(a8), K, L.ptr(a8s), K // 32, stream())
    for tile in (0, 1, 2, 3, 4):
        o1 = torch.zeros(M, N, device="cuda")
        o2 = torch.zeros(M, N, device="cuda")
        L.call("oasis_gemm_fp8", L.ptr(Ad), K, L.ptr(q), K, L.ptr(s), M, N, K,
               ctypes.byref(_epi(kind=L.EPI_STORE_F32, out_f32=o1, ld_out=N)), tile, 1, stream())
        L.call("oasis_gemm_fp8_a8", L.ptr(a8), K, L.ptr(a8s), K // 32, L.ptr(q), K, L.ptr(s), M, N, K,
               ctypes.byref(_epi(kind=L.EPI_STORE_F32, out_f32=o2, ld_out=N)), tile, 1, stream())
        sync()
        assert torch.equal(o1, o2), "tile %d" % tile
    m8 = torch.zeros(M, N, dtype=torch.uint8, device="cuda")
    m8s = torch.zeros(M, N // 32, dtype=torch.uint8, device="cuda")
    L.call("oasis_gemm_fp8_a8", L.ptr(a8), K, L.ptr(a8s), K // 32, L.ptr(q), K, L.ptr(s), M, N, K,
           ctypes.byref(_epi(kind=L.EPI_GELU_TANH_FP8, bias=dev(bias), out_fp8=m8, out_scale=m8s, ld_out=N,
                             ld_scale=N // 32)), -1, 1, stream())
    sync()
    deq = m8.cpu().view(torch.float8_e4m3fn).float() * torch.pow(2.0, m8s.cpu().float() - 127).repeat_interleave(32, 1)
    ref = oracle.quantize_act_blocks(oracle.gelu_tanh((_ref(A, W) + bias.double()).float()))
    cos, rel = metrics(deq, ref)
    print("fp8 GELU epilogue blocks: cos=%.7f rel=%.3e" % (cos, rel), flush=True)
    assert cos >= 0.9999 and rel <= 7e-2, (cos, rel)  # a value near a rounding midpoint may move one e4m3 step


@pytest.mark.parametrize("M,N", [(600, 520), (4608, 1024)])
def test_gemm_fp8_large_token_tiles(M, N):
    """The 6- and 8-wave large-token fp8 tiles (fp8 A only) equal the 4-wave tiles bit for bit (the same
    MFMA sequence per output), on a ragged shape and on the config-4 projection shape, for plain,
    split-K and GELU -> fp8-block epilogues; a tile whose lanes do not cover 32-column blocks
    refuses the fp8 epilogue, and the large tiles refuse bf16 A."""
    K = 1024
    g = _gen(M + N)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    q, s = _quantize(W)
    Ad = dev(A)
    a8 = torch.zeros(M, K, dtype=torch.uint8, device="cuda")
    a8s = torch.zeros(M, K // 32, dtype=torch.uint8, device="cuda")
    L.call("oasis_quantize_act_fp8", L.ptr(Ad), K, M, K, L.ptr(a8), K, L.ptr(a8s), K // 32, stream())

    # residual epilogues into x0, gates of 100-row frames (the gate row changes inside tiles)
    P = 100
    x0 = torch.randn(M, N, generator=g)
    ada = dev(torch.randn((M + P - 1) // P, 2 * N, generator=g))

    def run(tile, splits=1, kind=None):
        if kind in ("gated", "res"):
            o = dev(x0)
            e = _epi(kind=L.EPI_GATED_RES, bias=dev(bias), out_f32=o, ld_out=N, gate=ada[0, N:], gate_fstride=2 * N,
                     rows_per_frame=P) if kind == "gated" else _epi(kind=L.EPI_RESIDUAL, bias=dev(bias), out_f32=o,
                                                                     ld_out=N)
            out = o
        elif kind == "gelu8":
            m8 = torch.zeros(M, N, dtype=torch.uint8, device="cuda")
            m8s = torch.zeros(M, N // 32, dtype=torch.uint8, device="cuda")
            e = _epi(kind=L.EPI_GELU_TANH_FP8, bias=dev(bias), out_fp8=m8, out_scale=m8s, ld_out=N, ld_scale=N // 32)
            out = (m8, m8s)
        elif splits > 1:
            part = torch.zeros(splits, M, N, device="cuda")
            e = _epi(kind=L.EPI_PARTIAL_F32, out_f32=part, ld_out=N, split_stride=M * N)
            out = part
        else:
            o = torch.zeros(M, N, device="cuda")
            e = _epi(kind=L.EPI_STORE_F32, bias=dev(bias), out_f32=o, ld_out=N)
            out = o
        L.call("oasis_gemm_fp8_a8", L.ptr(a8), K, L.ptr(a8s), K // 32, L.ptr(q), K, L.ptr(s), M, N, K,
               ctypes.byref(e), tile, splits, stream())
        sync()
        return out

    ref = run(0)
    ref_part = run(0, 2)
    ref8 = run(0, kind="gelu8") if N % 32 == 0 else None
    ref_gated, ref_res = run(0, kind="gated"), run(0, kind="res")
    for tile in (5, 6, 7, 8, 9, 10, 11):
        assert torch.equal(run(tile), ref), "tile %d" % tile
        assert torch.equal(run(tile, 2), ref_part), "tile %d split-K x2" % tile
        assert torch.equal(run(tile, kind="gated"), ref_gated), "tile %d gated residual" % tile
        assert torch.equal(run(tile, kind="res"), ref_res), "tile %d residual" % tile
        if ref8 is not None and tile not in (6, 9):
            m8, m8s = run(tile, kind="gelu8")
            assert torch.equal(m8, ref8[0]) and torch.equal(m8s, ref8[1]), "tile %d gelu8" % tile
    cos, rel = metrics(ref, _ref(A, W) + bias.double())
    assert rel <= 1e-4, rel
    gates = ada[:, N:].cpu().repeat_interleave(P, 0)[:M]
    assert metrics(ref_gated, x0 + gates * ref.cpu())[1] <= 1e-6
    assert metrics(ref_res, x0 + ref.cpu())[1] <= 1e-6
    if N % 32 == 0:
        with pytest.raises(L.OasisError, match="GELU_TANH_FP8"):
            run(6, kind="gelu8")
    o = torch.zeros(M, N, device="cuda")
    with pytest.raises(L.OasisError, match="fp8 blocks"):
        L.call("oasis_gemm_fp8", L.ptr(Ad), K, L.ptr(q), K, L.ptr(s), M, N, K,
               ctypes.byref(_epi(kind=L.EPI_STORE_F32, out_f32=o, ld_out=N)), 5, 1, stream())


@pytest.mark.parametrize("layout", ["temporal", "spatial", "vae"])
def test_gemm_fp8_large_token_qkv_rope(layout):
    """QKV + RoPE + head split on the 8-wave large-token fp8 tiles (their epilogue steps each
    lane's row through positions, frames and streams 16 rows at a time) equals the 4-wave tile
    bit for bit, over two streams of two frames, and matches the rotated fp64 product."""
    H, D, K = 4, 256, 1024
    B_, T, P = (1, 2, 576) if layout == "vae" else (2, 2, 144)
    M, N = B_ * T * P, 3 * D
    g = _gen(40 + len(layout))
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
    if layout == "temporal":
        s_b, s_t, s_p, s_h = P * H * T * 64, 64, H * T * 64, T * 64
    else:
        s_b, s_t, s_p, s_h = T * H * P * 64, H * P * 64, 64, P * 64
    q8, s8 = _quantize(W)
    a8 = torch.zeros(M, K, dtype=torch.uint8, device="cuda")
    a8s = torch.zeros(M, K // 32, dtype=torch.uint8, device="cuda")
    L.call("oasis_quantize_act_fp8", L.ptr(dev(A)), K, M, K, L.ptr(a8), K, L.ptr(a8s), K // 32, stream())
    cos_d, sinp_d, bias_d = dev(cos), dev(sinp), dev(bias)

    def run(tile):
        q, k, v = (torch.zeros(M * D, device="cuda", dtype=torch.bfloat16) for _ in range(3))
        e = _epi(kind=L.EPI_QKV_ROPE, n_heads=H, bias=bias_d, q=q, k=k, v=v, rope_cos=cos_d, rope_sinp=sinp_d,
                 rope_by_frame=int(layout == "temporal"), rows_per_frame=P, frames_per_stream=T,
                 s_b=s_b, s_t=s_t, s_p=s_p, s_h=s_h)
        print("fp8 qkv_rope %s tile %d M=%d" % (layout, tile, M), flush=True)
        L.call("oasis_gemm_fp8_a8", L.ptr(a8), K, L.ptr(a8s), K // 32, L.ptr(q8), K, L.ptr(s8), M, N, K,
               ctypes.byref(e), tile, 1, stream())
        sync()
        return q, k, v

    ref = run(0)
    for tile in (5, 6, 7, 10, 11):
        got = run(tile)
        for name, a, b in zip("qkv", got, ref):
            assert torch.equal(a, b), "tile %d %s" % (tile, name)
    y = (_ref(A, W) + bias.double()).float().reshape(B_, T, P, 3, H, 64)
    pos_c = cos[torch.arange(T)] if layout == "temporal" else cos
    pos_s = sinp[torch.arange(T)] if layout == "temporal" else sinp
    if layout == "temporal":
        c4, s4 = pos_c[None, :, None, None, :], pos_s[None, :, None, None, :]
    else:
        c4, s4 = pos_c[None, None, :, None, :], pos_s[None, None, :, None, :]
    perm = (0, 2, 3, 1, 4) if layout == "temporal" else (0, 1, 3, 2, 4)
    exp = (oracle.apply_rope_swap(y[:, :, :, 0], c4, s4), oracle.apply_rope_swap(y[:, :, :, 1], c4, s4), y[:, :, :, 2])
    for name, got, r in zip("qkv", ref, exp):
        assert_close(got, r.permute(*perm).contiguous(), 0.99999, 1e-2, "fp8 qkv_rope %s %s" % (layout, name))
