"""Pins the fp32 CPU oracle (CPU only).

The reference ships no golden vectors and its own tests need Tenstorrent hardware, so
each oracle function is checked against something independent of its own formula:
torch.nn.functional, closed forms evaluated in fp64 with ``math``, invariants the
mathematics fixes, or fp64 brute-force loops written from the reference's semantics.
Each check is chosen so that a plausible mistake (dropped term, wrong sign, wrong index,
transposed operand) fails it.
"""
import math

import pytest
import torch
import torch.nn.functional as F

import oracle

torch.set_default_dtype(torch.float32)


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _close(a, b, tol):
    a, b = a.double(), b.double()
    err = (a - b).abs().max().item() / max(b.abs().max().item(), 1e-30)
    assert err <= tol, err


# ----------------------------------------------------------------- elementwise
def test_activations_against_torch_and_scalars():
    x = torch.linspace(-8, 8, 2001)
    _close(oracle.silu(x), F.silu(x), 1e-6)
    _close(oracle.gelu_tanh(x), F.gelu(x, approximate="tanh"), 1e-6)
    _close(oracle.gelu_erf(x), F.gelu(x), 1e-6)
    for v in (-3.7, -0.5, 0.0, 0.25, 2.0, 6.5):  # fp64 closed forms
        t = torch.tensor([v])
        ref = 0.5 * v * (1 + math.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)))
        assert abs(oracle.gelu_tanh(t).item() - ref) < 1e-6
        assert abs(oracle.gelu_erf(t).item() - 0.5 * v * (1 + math.erf(v / math.sqrt(2)))) < 1e-6
        assert abs(oracle.silu(t).item() - v / (1 + math.exp(-v))) < 1e-6


def test_layer_norm_and_modulate():
    g = _g(1)
    x = torch.randn(7, 1024, generator=g) * 3 + 2
    w, b = torch.randn(1024, generator=g), torch.randn(1024, generator=g)
    _close(oracle.layer_norm(x), F.layer_norm(x, (1024,), eps=1e-6), 1e-5)
    _close(oracle.layer_norm(x, w, b), F.layer_norm(x, (1024,), w, b, eps=1e-6), 1e-5)
    # eps matters for a constant row: (x - mean) = 0 -> output == b exactly
    c = torch.full((1, 1024), 5.0)
    assert torch.equal(oracle.layer_norm(c, w, b), b[None])
    sh, sc = torch.randn(1024, generator=g), torch.randn(1024, generator=g)
    _close(oracle.modulate(x, sh, sc), x + x * sc + sh, 1e-6)


# ----------------------------------------------------------------- conditioning, schedules
def test_timestep_embedding_closed_form():
    t = torch.tensor([0.0, 1.0, 14.0, 999.0])
    e = oracle.timestep_embedding(t, 256)
    assert e.shape == (4, 256)
    for r, tv in enumerate(t.tolist()):
        for i in (0, 1, 37, 127):
            f = math.exp(-math.log(10000) * i / 128)
            assert abs(e[r, i].item() - math.cos(tv * f)) < 2e-4
            assert abs(e[r, 128 + i].item() - math.sin(tv * f)) < 2e-4
    assert torch.equal(e[0, :128], torch.ones(128)) and torch.equal(e[0, 128:], torch.zeros(128))


def test_sigmoid_schedule_closed_form():
    ac = oracle.sigmoid_alphas_cumprod(1000)
    assert ac.shape == (1000,) and bool((ac[1:] < ac[:-1]).all())
    sig = lambda z: 1 / (1 + math.exp(-z))  # noqa: E731

    def f(k):  # normalised alpha-bar before clipping, oasis_inference.py:313-321
        u = k / 1000
        return (sig(3) - sig(u * 6 - 3)) / (sig(3) - sig(-3))
    for k in (1, 10, 250, 500, 750, 990):
        # cumprod of (1 - beta_i) telescopes to f(k+1)/f(0) while no beta is clipped
        assert abs(ac[k].item() - f(k + 1) / f(0)) < 1e-5


def test_cosine_schedule_closed_form():
    ac = oracle.cosine_alphas_cumprod(1000)
    f = lambda k: math.cos((k / 1000 + 0.008) / 1.008 * math.pi / 2) ** 2  # noqa: E731
    for k in (0, 249, 499, 749, 900):
        assert abs(ac[k].item() - f(k + 1) / f(0)) < 1e-5


def test_ddim_timesteps_follow_the_reference_linspace():
    assert oracle.ddim_timesteps(4) == [(999, 749), (749, 499), (499, 249), (249, -1)]
    steps = oracle.ddim_timesteps(12)
    assert steps[0][0] == 999 and steps[-1] == (82, -1) and len(steps) == 12


def test_conditioning_brute_force():
    g = _g(2)
    D, Fd = 32, 16
    w = {"t_emb.w0": torch.randn(D, Fd, generator=g), "t_emb.b0": torch.randn(D, generator=g),
         "t_emb.w2": torch.randn(D, D, generator=g), "t_emb.b2": torch.randn(D, generator=g),
         "ext.w": torch.randn(D, 25, generator=g), "ext.b": torch.randn(D, generator=g)}
    t = torch.tensor([3.0, 700.0])
    a = torch.zeros(2, 25)
    a[0, 11] = a[1, 15] = 1.0
    got = oracle.conditioning(t, a, w)
    for r in range(2):
        half = Fd // 2
        tf = [math.cos(t[r].item() * math.exp(-math.log(1e4) * i / half)) for i in range(half)] + \
             [math.sin(t[r].item() * math.exp(-math.log(1e4) * i / half)) for i in range(half)]
        h = [sum(w["t_emb.w0"][o, i].item() * tf[i] for i in range(Fd)) + w["t_emb.b0"][o].item() for o in range(D)]
        h = [v / (1 + math.exp(-v)) for v in h]
        for o in range(D):
            c = sum(w["t_emb.w2"][o, i].item() * h[i] for i in range(D)) + w["t_emb.b2"][o].item()
            c += sum(w["ext.w"][o, i].item() * a[r, i].item() for i in range(25)) + w["ext.b"][o].item()
            assert abs(got[r, o].item() - c) < 1e-3 * max(1.0, abs(c))


# ----------------------------------------------------------------- RoPE
def test_rotate_half_and_swap_trick():
    g = _g(3)
    x = torch.randn(5, 64, generator=g)
    assert torch.equal(oracle.rotate_half(oracle.rotate_half(x)), -x)
    assert torch.equal(oracle.rotate_half(x)[:, 0], -x[:, 1]) and torch.equal(oracle.rotate_half(x)[:, 1], x[:, 0])
    ang = torch.randn(5, 64, generator=g)
    cos, sinp = oracle.rope_cos_sinperm(ang, 64)
    # the reference's device formulation x*cos + swap(x)*sin_perm == apply_rotary_emb
    _close(oracle.apply_rope_swap(x, cos, sinp), oracle.apply_rotary_emb(ang, x), 1e-6)
    # ... which is also what the Q_swap weight columns produce (oasis_inference.py:375-403)
    W = torch.randn(64, 64, generator=g)
    Wswap = W.clone()
    Wswap[:, 0::2], Wswap[:, 1::2] = W[:, 1::2], W[:, 0::2]
    h = torch.randn(5, 64, generator=g)
    _close((h @ W) * cos + (h @ Wswap) * sinp, oracle.apply_rotary_emb(ang, h @ W), 1e-5)


def test_rope_invariants():
    g = _g(4)
    x = torch.randn(3, 64, generator=g)
    ang = torch.randn(3, 64, generator=g).repeat_interleave(1, -1)
    ang = ang[:, ::2].repeat_interleave(2, -1)  # one angle per pair
    y = oracle.apply_rotary_emb(ang, x)
    pn = lambda t: (t.reshape(3, 32, 2) ** 2).sum(-1)  # noqa: E731
    _close(pn(y), pn(x), 1e-5)                          # rotations preserve each pair's norm
    assert torch.equal(oracle.apply_rotary_emb(torch.zeros(3, 64), x), x)  # position 0 is the identity
    # partial rotation (the VAE rotates 32 of 64 dims): the tail passes through unchanged
    y2 = oracle.apply_rotary_emb(ang[:, :32], x)
    assert torch.equal(y2[:, 32:], x[:, 32:])


def test_axial_angles_match_broadcast_construction():
    freqs = torch.rand(16, generator=_g(5))
    a = oracle.spatial_rope_angles(freqs, 9, 16)
    assert a.shape == (144, 64)
    hpos = torch.linspace(-1, 1, 9)
    wpos = torch.linspace(-1, 1, 16)
    for p in (0, 17, 80, 143):
        hh, ww = divmod(p, 16)
        for d in range(64):  # dims 0-31 use the row position, 32-63 the column position
            ref = (hpos[hh] if d < 32 else wpos[ww]).item() * freqs[(d % 32) // 2].item()
            assert abs(a[p, d].item() - ref) < 1e-6
    t = oracle.temporal_rope_angles(torch.rand(32, generator=_g(6)), 5)
    assert torch.equal(t[0], torch.zeros(64)) and t.shape == (5, 64)


# ----------------------------------------------------------------- attention
def _attn_loops(q, k, v, causal):
    Lq, Lk, d = q.shape[0], k.shape[0], q.shape[1]
    out = torch.zeros(Lq, d, dtype=torch.float64)
    for i in range(Lq):
        keys = [j for j in range(Lk) if not causal or j <= i]
        s = [sum(q[i, c].item() * k[j, c].item() for c in range(d)) / math.sqrt(d) for j in keys]
        m = max(s)
        e = [math.exp(x - m) for x in s]
        z = sum(e)
        for j, ej in zip(keys, e):
            out[i] += (ej / z) * v[j].double()
    return out


@pytest.mark.parametrize("causal", [False, True])
def test_attention_brute_force(causal):
    g = _g(7)
    q, k, v = (torch.randn(5, 8, generator=g) for _ in range(3))
    _close(oracle.attention(q, k, v, causal=causal), _attn_loops(q, k, v, causal), 1e-5)


def test_attention_invariants():
    g = _g(8)
    v = torch.randn(6, 16, generator=g)
    k = torch.randn(6, 16, generator=g)
    q = torch.zeros(6, 16)  # constant scores -> the mean of V
    _close(oracle.attention(q, k, v), v.mean(0, keepdim=True).expand(6, 16), 1e-6)
    q = torch.randn(1, 16, generator=g)  # one causal key -> V itself
    _close(oracle.attention(q, k[:1], v[:1], causal=True), v[:1], 1e-6)
    # the reference's additive causal bias (oasis_inference.py:843-857) == the causal flag
    q = torch.randn(6, 16, generator=g)
    bias = torch.zeros(6, 6).masked_fill(torch.ones(6, 6, dtype=torch.bool).triu(1), -1e4)
    s = q @ k.t() / 4.0 + bias
    _close(oracle.attention(q, k, v, causal=True), torch.softmax(s, -1) @ v, 1e-5)
    # zero-padded keys as in tests/test_dit_block.py:548-554
    qp, kp, vp = (F.pad(t, [0, 0, 0, 3]) for t in (q, k, v))
    ref = F.scaled_dot_product_attention(qp[None], kp[None], vp[None])[0][:6]
    _close(oracle.attention(q, k, v, pad_keys_to=9), ref, 1e-5)


# ----------------------------------------------------------------- sub-block and step (fp64 loops)
def _ln64(x):
    m = x.mean(-1, keepdim=True)
    return (x - m) / torch.sqrt(((x - m) ** 2).mean(-1, keepdim=True) + 1e-6)


def _rope64(x, ang):  # x [..., 64], ang [..., 64] one angle per pair; rotates pairs (2k, 2k+1)
    y = x.clone()
    for kk in range(32):
        a = ang[..., 2 * kk]
        c, s = torch.cos(a), torch.sin(a)
        y[..., 2 * kk] = x[..., 2 * kk] * c - x[..., 2 * kk + 1] * s
        y[..., 2 * kk + 1] = x[..., 2 * kk + 1] * c + x[..., 2 * kk] * s
    return y


def _sub_block_loops(x, c, w, kind, ang):
    """fp64 restatement of run_sub_block (oasis_inference.py:995-1215) with explicit loops
    over frames, tokens and heads. x [T, P, D]; c [T, D] (pre-SiLU); ang: spatial [P, 64]
    or temporal [T, 64]."""
    T, P, D = x.shape
    H = D // 64
    W = {k: v.double() for k, v in w.items()}
    x = x.double().clone()
    sc = c.double() * torch.sigmoid(c.double())
    ada = sc @ W["ada_w"].t() + W["ada_b"]
    out = x.clone()
    q = torch.zeros(T, P, D, dtype=torch.float64)
    k = torch.zeros_like(q)
    v = torch.zeros_like(q)
    for t in range(T):
        sh, s1 = ada[t, 0:D], ada[t, D:2 * D]
        hmod = _ln64(x[t]) * (1 + s1) + sh
        qkv = hmod @ W["qkv_w"].t()
        q[t], k[t], v[t] = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
    attn = torch.zeros_like(q)
    for h in range(H):
        sl = slice(64 * h, 64 * h + 64)
        if kind == "s":
            for t in range(T):
                qq = _rope64(q[t, :, sl], ang)
                kk = _rope64(k[t, :, sl], ang)
                attn[t, :, sl] = _attn_loops(qq, kk, v[t, :, sl], False) if P <= 8 else \
                    torch.softmax(qq @ kk.t() / 8.0, -1) @ v[t, :, sl]
        else:
            for p in range(P):
                qq = _rope64(q[:, p, sl], ang[:T])
                kk = _rope64(k[:, p, sl], ang[:T])
                attn[:, p, sl] = _attn_loops(qq, kk, v[:, p, sl], True)
    for t in range(T):
        g_a, sh_m, s_m, g_m = ada[t, 2 * D:3 * D], ada[t, 3 * D:4 * D], ada[t, 4 * D:5 * D], ada[t, 5 * D:]
        y = out[t] + g_a * (attn[t] @ W["out_w"].t() + W["out_b"])
        hh = _ln64(y) * (1 + s_m) + sh_m
        gg = hh @ W["fc1_w"].t() + W["fc1_b"]
        gg = 0.5 * gg * (1 + torch.tanh(math.sqrt(2 / math.pi) * (gg + 0.044715 * gg ** 3)))
        out[t] = y + g_m * (gg @ W["fc2_w"].t() + W["fc2_b"])
    return out


def _tiny_sub_w(g, D=128, Dm=256, bias=True):
    r = lambda *s: torch.randn(*s, generator=g) * 0.1  # noqa: E731
    return {"ada_w": r(6 * D, D), "ada_b": r(6 * D) if bias else torch.zeros(6 * D), "qkv_w": r(3 * D, D),
            "out_w": r(D, D), "out_b": r(D), "fc1_w": r(Dm, D), "fc1_b": r(Dm), "fc2_w": r(D, Dm), "fc2_b": r(D)}


@pytest.mark.parametrize("kind", ["s", "t"])
def test_sub_block_against_loops(kind):
    g = _g(9 if kind == "s" else 10)
    T, P, D = (2, 6, 128) if kind == "s" else (3, 4, 128)
    w = _tiny_sub_w(g, D)
    x = torch.randn(T, P, D, generator=g)
    c = torch.randn(T, D, generator=g)
    if kind == "s":
        ang = oracle.spatial_rope_angles(torch.rand(16, generator=g) * 3, 2, 3)
    else:
        ang = oracle.temporal_rope_angles(torch.rand(32, generator=g), T)
    cs, sp = oracle.rope_cos_sinperm(ang, 64)
    got = oracle.sub_block(x, oracle.silu(c), w, kind, cs, sp)
    _close(got, _sub_block_loops(x, c, w, kind, ang), 1e-4)


def test_dit_forward_context_rows_do_not_see_the_generated_frame():
    """KV-invariance (docs/kv_cache_plan.md:15-39): frame-0 rows depend on frame 0 only."""
    g = _g(11)
    D = 128
    w = {"rope.spatial_freqs": torch.rand(16, generator=g), "rope.temporal_freqs": torch.rand(32, generator=g),
         "final.ada_w": torch.randn(2 * D, D, generator=g) * 0.1, "final.ada_b": torch.randn(2 * D, generator=g),
         "final.w": torch.randn(64, D, generator=g) * 0.1, "final.b": torch.randn(64, generator=g)}
    for i in range(2):
        for kind in "st":
            for k, v in _tiny_sub_w(g, D).items():
                w["blocks.%d.%s.%s" % (i, kind, k)] = v
    z = torch.randn(2, 6, D, generator=g)
    c = torch.randn(2, D, generator=g)
    v1 = oracle.dit_forward(z, c, w, grid=(2, 3))
    z2, c2 = z.clone(), c.clone()
    z2[1] += torch.randn(6, D, generator=g)
    c2[1] += 1.0
    v2 = oracle.dit_forward(z2, c2, w, grid=(2, 3))
    assert torch.equal(v1[0], v2[0]) and not torch.allclose(v1[1], v2[1])


# ----------------------------------------------------------------- DDIM, patches, bridge
def test_ddim_exact_v_recovers_x0_and_eps():
    g = _g(12)
    ac = oracle.cosine_alphas_cumprod()
    x0, eps = torch.randn(144, 64, generator=g).double(), torch.randn(144, 64, generator=g).double()
    for (t, tn), last in ((((749, 499)), False), ((249, -1), True)):
        a = ac[t].double()
        xt = a.sqrt() * x0 + (1 - a).sqrt() * eps
        v = a.sqrt() * eps - (1 - a).sqrt() * x0          # v-parametrisation target
        c = oracle.ddim_coeffs(ac, t, tn, last)
        an = 1.0 if last else ac[tn].item()
        _close(oracle.ddim_update(xt, v, c), an ** 0.5 * x0 + (1 - an) ** 0.5 * eps, 1e-6)
    assert oracle.ddim_coeffs(ac, 249, -1, True)[4:] == (1.0, 0.0)  # last step returns x0


def test_patchify_unpatchify_and_embed():
    g = _g(13)
    img = torch.randn(2, 16, 18, 32, generator=g)
    p = oracle.patchify_to_output_space(img)
    assert p.shape == (2, 144, 64)
    assert torch.equal(oracle.unpatchify(p), img)
    # column (p, q, c) of row (h, w) is pixel (c, 2h+p, 2w+q)
    assert p[1, 5 * 16 + 7, (1 * 2 + 0) * 16 + 3].item() == img[1, 3, 11, 14].item()
    w = {"x_emb.w": torch.randn(64, 16, 2, 2, generator=g), "x_emb.b": torch.randn(64, generator=g)}
    _close(oracle.patch_embed(img, w), p @ oracle.patch_embed_roundtrip_weight(w) + w["x_emb.b"], 1e-5)


def test_bridge_is_the_pixel_grid_of_the_latent():
    g = _g(14)
    img = torch.randn(1, 16, 18, 32, generator=g)
    lat = oracle.bridge(oracle.patchify_to_output_space(img)[0])
    # VAE row r = y*32 + x holds the 16 latent channels of pixel (y, x), scaled
    _close(lat[:, :16], img[0].permute(1, 2, 0).reshape(576, 16) / oracle.SCALING_FACTOR, 1e-6)
    assert torch.equal(lat[:, 16:], torch.zeros(576, 16))


def test_vae_unpatchify_pixels():
    g = _g(15)
    patches = torch.randn(576, 1200, generator=g) * 2
    fr = oracle.vae_unpatchify(patches)
    assert fr.shape == (3, 360, 640) and fr.abs().max().item() <= 1.0
    for c, y, x in ((0, 0, 0), (2, 359, 639), (1, 123, 457)):
        v = patches[(y // 20) * 32 + x // 20, c * 400 + (y % 20) * 20 + x % 20].clamp(-1, 1)
        assert fr[c, y, x].item() == v.item()


def _tiny_vae_w(g, D=128, lat=8, out=12):
    r = lambda *s: torch.randn(*s, generator=g) * 0.1  # noqa: E731
    return {"pq_w": r(D, lat), "pq_b": r(D), "dec.0.n1_w": 1 + r(D), "dec.0.n1_b": r(D), "dec.0.qkv_w": r(3 * D, D),
            "dec.0.qkv_b": r(3 * D), "dec.0.proj_w": r(D, D), "dec.0.proj_b": r(D), "dec.0.n2_w": 1 + r(D),
            "dec.0.n2_b": r(D), "dec.0.fc1_w": r(2 * D, D), "dec.0.fc1_b": r(2 * D), "dec.0.fc2_w": r(D, 2 * D),
            "dec.0.fc2_b": r(D), "norm_w": 1 + r(D), "norm_b": r(D), "pred_w": r(out, D), "pred_b": r(out),
            "rope.vae_freqs": torch.rand(8, generator=g)}


def _vae_loops(lat, w, grid):
    """fp64 restatement of vae_decode_forward (oasis_inference.py:1546-1618) for one block,
    with the attention and RoPE as loops (2 heads of 64, dims >= 32 unrotated)."""
    W = {k: v.double() for k, v in w.items()}
    L_, D = grid[0] * grid[1], W["pq_w"].shape[0]
    x = lat.double() @ W["pq_w"].t() + W["pq_b"]
    ang = oracle.vae_rope_angles(w["rope.vae_freqs"], *grid).double()   # [L, 32]
    h = _ln64(x) * W["dec.0.n1_w"] + W["dec.0.n1_b"]
    qkv = h @ W["dec.0.qkv_w"].t() + W["dec.0.qkv_b"]
    att = torch.zeros(L_, D, dtype=torch.float64)
    for hd in range(D // 64):
        sl = slice(64 * hd, 64 * hd + 64)
        q, k, v = qkv[:, sl], qkv[:, D:][:, sl], qkv[:, 2 * D:][:, sl]
        full = torch.cat([ang, torch.zeros(L_, 32, dtype=torch.float64)], -1)  # dims >= 32 unrotated
        att[:, sl] = _attn_loops(_rope64(q, full), _rope64(k, full), v, False)
    x = x + att @ W["dec.0.proj_w"].t() + W["dec.0.proj_b"]
    hh = _ln64(x) * W["dec.0.n2_w"] + W["dec.0.n2_b"]
    gg = hh @ W["dec.0.fc1_w"].t() + W["dec.0.fc1_b"]
    gg = 0.5 * gg * (1 + torch.erf(gg / math.sqrt(2)))
    x = x + gg @ W["dec.0.fc2_w"].t() + W["dec.0.fc2_b"]
    return (_ln64(x) * W["norm_w"] + W["norm_b"]) @ W["pred_w"].t() + W["pred_b"]


def test_vae_decode_against_loops():
    g = _g(16)
    w = _tiny_vae_w(g)
    lat = torch.randn(16, 8, generator=g)
    _close(oracle.vae_decode(lat, w, grid=(4, 4)), _vae_loops(lat, w, (4, 4)), 1e-4)


# ----------------------------------------------------------------- final layer, DiT forward, DDIM frame
# Loop-level fp64 restatements of the compositions (oasis_inference.py:1438-1526 and
# 1909-1932, 2131-2148), each followed by checks that a planted mistake in the oracle
# (monkeypatched on the CPU) is caught by the same comparison.

def _err(a, b):
    a, b = a.double(), b.double()
    return (a - b).abs().max().item() / max(b.abs().max().item(), 1e-30)


def _final_loops(x, c, w):
    """final layer (oasis_inference.py:1497-1521) per token: adaLN of silu(c) has two
    chunks, shift = cols [0, D) and scale = cols [D, 2D) (the reference folds +1 into the
    scale half, 528-532); LN without affine, eps 1e-6; then Linear(D -> 64) + bias."""
    T, P, D = x.shape
    Wa, ba = w["final.ada_w"].double(), w["final.ada_b"].double()
    Wf, bfin = w["final.w"].double(), w["final.b"].double()
    n_out = Wf.shape[0]
    out = torch.zeros(T, P, n_out, dtype=torch.float64)
    for t in range(T):
        cc = c[t].double()
        s = [v / (1 + math.exp(-v)) for v in cc.tolist()]
        shift = [sum(Wa[o, k].item() * s[k] for k in range(D)) + ba[o].item() for o in range(D)]
        scale_p1 = [1.0 + sum(Wa[D + o, k].item() * s[k] for k in range(D)) + ba[D + o].item() for o in range(D)]
        for p in range(P):
            row = x[t, p].double().tolist()
            mean = sum(row) / D
            var = sum((v - mean) ** 2 for v in row) / D
            h = [(row[k] - mean) / math.sqrt(var + 1e-6) * scale_p1[k] + shift[k] for k in range(D)]
            for n in range(n_out):
                out[t, p, n] = sum(h[k] * Wf[n, k].item() for k in range(D)) + bfin[n].item()
    return out


def _tiny_dit_w(g, D=32, n_blocks=1, n_out=64):
    r = lambda *s: torch.randn(*s, generator=g) * 0.1  # noqa: E731
    w = {"rope.spatial_freqs": torch.rand(16, generator=g) * 3, "rope.temporal_freqs": torch.rand(32, generator=g),
         "final.ada_w": r(2 * D, D), "final.ada_b": r(2 * D), "final.w": r(n_out, D), "final.b": r(n_out),
         "x_emb.w": r(D, 16, 2, 2), "x_emb.b": r(D)}
    for i in range(n_blocks):
        for kind in "st":
            for k, v in _tiny_sub_w(g, D).items():
                w["blocks.%d.%s.%s" % (i, kind, k)] = v
    return w


def test_final_layer_against_loops_and_planted_mistakes(monkeypatch):
    g = _g(20)
    D = 32
    w = _tiny_dit_w(g, D, n_out=8)
    x = torch.randn(2, 3, D, generator=g) * 2 + 0.5
    c = torch.randn(2, D, generator=g)
    ref = _final_loops(x, c, w)
    _close(oracle.final_layer(x, oracle.silu(c), w), ref, 1e-5)
    ref_mod = oracle.oasis_ref.modulate
    planted = {
        "shift and scale swapped": lambda h, shift, scale: h * (1.0 + shift) + scale,
        "+1 of the scale dropped": lambda h, shift, scale: h * scale + shift,
        "shift dropped": lambda h, shift, scale: h * (1.0 + scale),
    }
    for name, bad in planted.items():
        monkeypatch.setattr(oracle.oasis_ref, "modulate", bad)
        assert _err(oracle.final_layer(x, oracle.silu(c), w), ref) > 1e-2, name
    monkeypatch.setattr(oracle.oasis_ref, "modulate", ref_mod)
    # chunks read in the wrong order (scale from cols [0, D))
    w_sw = dict(w)
    w_sw["final.ada_w"] = torch.cat([w["final.ada_w"][D:], w["final.ada_w"][:D]])
    w_sw["final.ada_b"] = torch.cat([w["final.ada_b"][D:], w["final.ada_b"][:D]])
    assert _err(oracle.final_layer(x, oracle.silu(c), w_sw), ref) > 1e-2
    # LN over the wrong axis (tokens instead of features) is caught too
    monkeypatch.setattr(oracle.oasis_ref, "layer_norm",
                        lambda t, *a, **k: (t - t.mean(-2, keepdim=True)) / t.std(-2, keepdim=True))
    assert _err(oracle.final_layer(x, oracle.silu(c), w), ref) > 1e-2


def _dit_loops(z, c, w, grid):
    """dit_forward_device (oasis_inference.py:1438-1526): SiLU of each frame's cond once,
    then per block the spatial sub-block (blocks.i.s) followed by the temporal one
    (blocks.i.t), then the final layer; every piece as the fp64 loops above."""
    T = z.shape[0]
    s_ang = oracle.spatial_rope_angles(w["rope.spatial_freqs"].float(), *grid).double()
    t_ang = oracle.temporal_rope_angles(w["rope.temporal_freqs"].float(), T).double()
    x = z.double()
    i = 0
    while "blocks.%d.s.ada_w" % i in w:
        for kind, ang in (("s", s_ang), ("t", t_ang)):
            p = "blocks.%d.%s." % (i, kind)
            bw = {k[len(p):]: v for k, v in w.items() if k.startswith(p)}
            x = _sub_block_loops(x, c, bw, kind, ang)
        i += 1
    return _final_loops(x, c, w)


def test_dit_forward_against_loops_and_planted_mistakes(monkeypatch):
    g = _g(21)
    D = 128
    w = _tiny_dit_w(g, D, n_out=8)
    z = torch.randn(2, 6, D, generator=g)
    c = torch.randn(2, D, generator=g)
    ref = _dit_loops(z, c, w, (2, 3))
    _close(oracle.dit_forward(z, c, w, grid=(2, 3)), ref, 1e-4)
    # SiLU skipped (raw cond into the adaLN projections)
    monkeypatch.setattr(oracle.oasis_ref, "silu", lambda t: t)
    assert _err(oracle.dit_forward(z, c, w, grid=(2, 3)), ref) > 1e-2
    monkeypatch.undo()
    # temporal sub-block run before the spatial one of each block
    monkeypatch.setattr(oracle.oasis_ref, "_blk",
                        lambda ww, i, kind: {k[len("blocks.%d.%s." % (i, "ts"[kind == "t"])):]: v
                                             for k, v in ww.items()
                                             if k.startswith("blocks.%d.%s." % (i, "ts"[kind == "t"]))})
    assert _err(oracle.dit_forward(z, c, w, grid=(2, 3)), ref) > 1e-2
    monkeypatch.undo()
    # the temporal attention made non-causal (frame 0 sees frame 1)
    orig = oracle.oasis_ref.attention
    monkeypatch.setattr(oracle.oasis_ref, "attention", lambda q, k, v, causal=False, pad_keys_to=None:
                        orig(q, k, v, causal=False, pad_keys_to=pad_keys_to))
    assert _err(oracle.dit_forward(z, c, w, grid=(2, 3)), ref) > 1e-2


def _frame_loops(x_noise, ctx_z, ctx_cond, gen_conds, w, vae_w, ac, steps, grid, vae_grid):
    """One generated frame (oasis_inference.py:1909-1932, traced as 2131-2148), loop form:
      - W_rt[(p*2+q)*C + c, d] = conv_w[d, c, p, q] (1821-1826); gen_z = chunk @ W_rt + b;
      - z = [context frame; generated frame] (1912), cond likewise (cond_traced_per_step);
      - v = the DiT output rows of frame 1 (1915-1916);
      - a = alphas[t], a' = alphas[t_next] or 1 on the last step (1843-1852);
        x0 = sqrt(a) x - sqrt(1-a) v and eps = sqrt(1-a) x + sqrt(a) v (the v-parametrisation
        solved for eps, equal to the reference's (x/sqrt(a) - x0)/sqrt(1/a - 1));
        x <- sqrt(a') x0 + sqrt(1-a') eps;
      - bridge (1651-1709): VAE row (2h+p)*(2gw) + (2w+q), channel c <- chunk[h*gw + w,
        (p*2+q)*C + c] / 0.07843137255;
      - VAE decoder, then unpatchify (c, y, x) <- pred[(y//20)*vgw + x//20, c*400 + (y%20)*20 + x%20],
        clamped to [-1, 1] (1636-1645, 2292)."""
    gh, gw = grid
    C = 16
    cw = w["x_emb.w"].double()
    D = cw.shape[0]
    W_rt = torch.zeros(4 * C, D, dtype=torch.float64)
    for d in range(D):
        for cc in range(C):
            for p in range(2):
                for q in range(2):
                    W_rt[(p * 2 + q) * C + cc, d] = cw[d, cc, p, q]
    chunk = x_noise.double()
    for i, (t, tn) in enumerate(steps):
        gen_z = chunk @ W_rt + w["x_emb.b"].double()
        z = torch.stack([ctx_z.double(), gen_z])
        cond = torch.stack([ctx_cond.double(), gen_conds[i].double()])
        v = _dit_loops(z, cond, w, grid)[1]
        a = ac[t].item()
        an = 1.0 if i == len(steps) - 1 else ac[tn].item()
        x0 = math.sqrt(a) * chunk - math.sqrt(1 - a) * v
        eps = math.sqrt(1 - a) * chunk + math.sqrt(a) * v
        chunk = math.sqrt(an) * x0 + math.sqrt(1 - an) * eps
    vgh, vgw = vae_grid
    lat = torch.zeros(vgh * vgw, 32, dtype=torch.float64)
    for h in range(gh):
        for ww in range(gw):
            for p in range(2):
                for q in range(2):
                    r = (2 * h + p) * vgw + (2 * ww + q)
                    for cc in range(C):
                        lat[r, cc] = chunk[h * gw + ww, (p * 2 + q) * C + cc] / 0.07843137255
    pred = _vae_loops(lat, vae_w, vae_grid)
    frame = torch.zeros(3, vgh * 20, vgw * 20, dtype=torch.float64)
    for cc in range(3):
        for y in range(vgh * 20):
            for xx in range(vgw * 20):
                val = pred[(y // 20) * vgw + xx // 20, cc * 400 + (y % 20) * 20 + xx % 20].item()
                frame[cc, y, xx] = min(1.0, max(-1.0, val))
    return chunk, frame


def test_ddim_frame_against_loops_and_planted_mistakes(monkeypatch):
    g = _g(22)
    D, grid, vae_grid = 128, (2, 3), (4, 6)
    w = _tiny_dit_w(g, D, n_out=64)
    vae_w = _tiny_vae_w(g, D, lat=32, out=1200)
    vae_w["pred_w"] = vae_w["pred_w"] * 5   # frame values reach the clamp at +-1
    ac = oracle.cosine_alphas_cumprod()
    steps = oracle.ddim_timesteps(2)          # [(999, 499), (499, -1)]
    assert steps == [(999, 499), (499, -1)]
    x_noise = torch.randn(6, 64, generator=g)
    ctx_z = torch.randn(6, D, generator=g)
    ctx_cond = torch.randn(D, generator=g)
    gen_conds = [torch.randn(D, generator=g) for _ in steps]
    args = (x_noise, ctx_z, ctx_cond, gen_conds, w, vae_w, ac, steps)
    ref_chunk, ref_frame = _frame_loops(*args, grid, vae_grid)
    assert ref_frame.abs().max().item() == 1.0 and ref_frame.abs().min().item() < 0.9
    chunk, frame = oracle.ddim_frame(*args, grid=grid, vae_grid=vae_grid)
    _close(chunk, ref_chunk, 1e-4)
    _close(frame, ref_frame, 1e-4)

    def planted(name):
        c2, f2 = oracle.ddim_frame(*args, grid=grid, vae_grid=vae_grid)
        monkeypatch.undo()
        assert _err(c2, ref_chunk) > 1e-3, name

    orig_dit = oracle.oasis_ref.dit_forward
    monkeypatch.setattr(oracle.oasis_ref, "dit_forward", lambda *a, **k: orig_dit(*a, **k).flip(0))
    planted("v taken from the context frame (frame 0)")
    monkeypatch.setattr(oracle.oasis_ref, "dit_forward",
                        lambda z, c, *a, **k: orig_dit(z.flip(0), c.flip(0), *a, **k).flip(0))
    planted("generated frame stacked before the context frame")
    orig_c = oracle.oasis_ref.ddim_coeffs
    monkeypatch.setattr(oracle.oasis_ref, "ddim_coeffs", lambda ac_, t, tn, last: orig_c(ac_, t, tn, False))
    planted("a' = 1 not applied on the last step")
    monkeypatch.setattr(oracle.oasis_ref, "ddim_coeffs", lambda ac_, t, tn, last: orig_c(ac_, tn if tn >= 0 else t,
                                                                                          tn, last))
    planted("alphas read at the next timestep")
    orig_pe = oracle.oasis_ref.patch_embed_roundtrip_weight
    monkeypatch.setattr(oracle.oasis_ref, "patch_embed_roundtrip_weight",
                        lambda ww: ww["x_emb.w"].float().permute(0, 1, 2, 3).reshape(ww["x_emb.w"].shape[0], -1)
                        .t().contiguous())
    planted("W_rt columns in (c, p, q) order instead of (p, q, c)")
    del orig_pe
    # the bridge's row order: a transposed pixel grid changes the frame, not the chunk
    orig_b = oracle.oasis_ref.bridge
    monkeypatch.setattr(oracle.oasis_ref, "bridge",
                        lambda ch, gh, gw, *a: orig_b(ch, gh, gw, *a).reshape(2 * gh, 2 * gw, -1)
                        .transpose(0, 1).reshape(4 * gh * gw, -1))
    _, f2 = oracle.ddim_frame(*args, grid=grid, vae_grid=vae_grid)
    monkeypatch.undo()
    assert _err(f2, ref_frame) > 1e-2


# ----------------------------------------------------------------- fp8 (config 4)
def _e4m3_decode(c):
    s, e, m = c >> 7, (c >> 3) & 15, c & 7
    if e == 15 and m == 7:
        return float("nan")
    v = (m / 8) * 2.0 ** -6 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
    return -v if s else v


_GRID = sorted({(_e4m3_decode(c), c) for c in range(128) if _e4m3_decode(c) == _e4m3_decode(c)})


def _nearest_e4m3(x):
    """Round-to-nearest-even onto the e4m3 grid by brute force (|x| <= 448)."""
    a = abs(x)
    best = min(_GRID, key=lambda vc: (abs(vc[0] - a), vc[1] & 1))
    return math.copysign(best[0], x) if best[0] != 0 else 0.0


def test_e4m3_grid():
    assert _GRID[-1][0] == 448.0 and len(_GRID) == 127  # 0 .. 448, NaN excluded
    assert _GRID[1][0] == 2.0 ** -9                      # smallest subnormal


def test_quantize_e4m3_rows_is_nearest_on_the_grid():
    g = _g(17)
    w = torch.randn(8, 96, generator=g) * 0.02
    w[3] = 0.0
    q, s = oracle.quantize_e4m3_rows(w)
    assert s[3].item() == 1.0 and torch.equal(q[3], torch.zeros(96))
    for n in (0, 5, 7):
        assert abs(s[n].item() - w[n].abs().max().item() / 448.0) <= 1e-9
        assert q[n].abs().max().item() == 448.0        # the row maximum lands on the top code
        for k in range(0, 96, 7):
            x = w[n, k].item() / s[n].item()
            assert q[n, k].item() == _nearest_e4m3(x), (n, k)


def test_quantize_act_blocks():
    g = _g(18)
    x = torch.randn(4, 128, generator=g) * torch.tensor([1e-3, 1.0, 30.0, 0.0]).repeat_interleave(32)
    xq = oracle.quantize_act_blocks(x)
    assert torch.equal(xq[:, 96:], torch.zeros(4, 32))
    for r in range(4):
        for b in range(3):
            blk, qb = x[r, 32 * b:32 * b + 32], xq[r, 32 * b:32 * b + 32]
            amax = blk.abs().max().item()
            e = math.floor(math.log2(amax)) - 7          # power-of-two scale of the block
            sc = 2.0 ** e
            assert 128 <= amax / sc < 256
            for k in range(0, 32, 5):
                assert qb[k].item() == _nearest_e4m3(blk[k].item() / sc) * sc


def test_fp8_weights_replace_only_the_projections():
    g = _g(19)
    w = {"blocks.0.s.qkv_w": torch.randn(6, 32, generator=g), "blocks.0.s.ada_w": torch.randn(6, 32, generator=g),
         "final.w": torch.randn(4, 32, generator=g)}
    w8 = oracle.fp8_weights(w)
    assert w8["blocks.0.s.ada_w"] is w["blocks.0.s.ada_w"] and w8["final.w"] is w["final.w"]
    q, s = oracle.quantize_e4m3_rows(w["blocks.0.s.qkv_w"])
    assert torch.equal(w8["blocks.0.s.qkv_w"], q * s[:, None])
