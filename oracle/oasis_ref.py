"""fp32 CPU restatement of the Oasis DiT step, DDIM update, bridge and VAE decoder.

Test infrastructure only (see the package docstring). Weights come in as a dict
of tensors in the model's native ``nn.Linear`` layout ``[out, in]`` (any dtype;
they are upcast to fp32 here). Shapes are read from the weights, so the same
functions run at the Oasis-500M shapes and at tiny shapes in the brute-force
tests.

Layout conventions:
  - DiT activations are ``[T, P, D]``: T frames, P = gh*gw patches per frame.
  - adaLN rows are one per frame: ``[T, 6*D]`` in the chunk order
    ``shift_a, scale_a, gate_a, shift_m, scale_m, gate_m``
    (oasis_inference.py:1054-1055,1160,1169-1170,1200).
"""
import math

import torch
import torch.nn.functional as F

__all__ = [
    "D_MODEL", "N_HEADS", "D_HEAD", "D_MLP", "N_BLOCKS", "PATCH", "IN_CH", "GRID_H", "GRID_W",
    "N_PATCHES", "OUT_DIM", "FREQ_DIM", "EXT_COND_DIM", "SCALING_FACTOR",
    "VAE_GRID_H", "VAE_GRID_W", "VAE_SEQ", "VAE_PATCH", "VAE_PATCH_DIM", "VAE_ROPE_DIM",
    "timestep_embedding", "sigmoid_beta_schedule", "sigmoid_alphas_cumprod",
    "cosine_alphas_cumprod", "ddim_timesteps",
    "rotate_half", "apply_rotary_emb", "spatial_rope_angles", "temporal_rope_angles",
    "vae_rope_angles", "rope_cos_sinperm", "apply_rope_swap",
    "silu", "gelu_tanh", "gelu_erf", "layer_norm", "modulate", "attention",
    "adaln", "spatial_attention", "temporal_attention", "sub_block", "final_layer",
    "conditioning", "dit_forward", "patch_embed", "patchify_to_output_space",
    "unpatchify", "patch_embed_roundtrip_weight", "ddim_coeffs", "ddim_update",
    "bridge", "vae_decode", "vae_unpatchify", "ddim_frame",
    "E4M3_MAX", "quantize_e4m3_rows", "quantize_act_blocks", "fp8_weights",
]

# ---- model constants (oasis_inference.py:90-163) ----
D_MODEL = 1024
N_HEADS = 16
D_HEAD = 64
D_MLP = 4096
N_BLOCKS = 16
PATCH = 2
IN_CH = 16
GRID_H = 9            # 18 / 2
GRID_W = 16           # 32 / 2
N_PATCHES = GRID_H * GRID_W
OUT_DIM = PATCH * PATCH * IN_CH
FREQ_DIM = 256
EXT_COND_DIM = 25
SCALING_FACTOR = 0.07843137255
VAE_GRID_H = 18
VAE_GRID_W = 32
VAE_SEQ = VAE_GRID_H * VAE_GRID_W
VAE_PATCH = 20
VAE_PATCH_DIM = 3 * VAE_PATCH * VAE_PATCH
VAE_ROPE_DIM = 32     # first 32 of the 64 head dims are rotated (oasis_inference.py:154)
LN_EPS = 1e-6


def _f(t):
    return t.float()


# ---------------------------------------------------------------------------
# conditioning and schedules
# ---------------------------------------------------------------------------

def timestep_embedding(t, dim=FREQ_DIM, max_period=10000):
    """Sinusoidal embedding ``[cos(t f), sin(t f)]``, ``f_i = exp(-ln(P) i / (dim/2))``.

    Follows oasis_inference.py:307-311.
    """
    half = dim // 2
    freqs = torch.exp(-math.log(max_period) * torch.arange(0, half, dtype=torch.float32) / half)
    args = t.reshape(-1).float()[:, None] * freqs[None]
    return torch.cat([torch.cos(args), torch.sin(args)], dim=-1)


def sigmoid_beta_schedule(timesteps=1000, start=-3, end=3, tau=1, clamp_min=1e-5):
    """Betas of the sigmoid schedule. Follows oasis_inference.py:313-321."""
    steps = timesteps + 1
    t = torch.linspace(0, timesteps, steps, dtype=torch.float64) / timesteps
    v_start = torch.tensor(start / tau).sigmoid()
    v_end = torch.tensor(end / tau).sigmoid()
    ac = (-((t * (end - start) + start) / tau).sigmoid() + v_end) / (v_end - v_start)
    ac = ac / ac[0]
    betas = 1 - (ac[1:] / ac[:-1])
    return torch.clip(betas, 0, 0.999)


def sigmoid_alphas_cumprod(timesteps=1000):
    """``cumprod(1 - betas)`` in fp32, as oasis_inference.py:1769-1771 builds it."""
    betas = sigmoid_beta_schedule(timesteps).float()
    return torch.cumprod(1.0 - betas, dim=0)


def cosine_alphas_cumprod(timesteps=1000, s=0.008):
    """Cosine schedule (Nichol & Dhariwal 2021, eq. 17) with betas clipped to 0.999.

    The configuration asks for 1000-step cosine alphas; the reference itself uses the
    sigmoid schedule (oasis_inference.py:1769). The DDIM update does not depend on
    which schedule produced the alphas.
    """
    steps = timesteps + 1
    x = torch.linspace(0, timesteps, steps, dtype=torch.float64)
    ac = torch.cos(((x / timesteps) + s) / (1 + s) * math.pi * 0.5) ** 2
    ac = ac / ac[0]
    betas = torch.clip(1 - (ac[1:] / ac[:-1]), 0, 0.999)
    return torch.cumprod(1.0 - betas.float(), dim=0)


def ddim_timesteps(n_steps, max_noise_level=1000):
    """``linspace(-1, 999, n+1)``; step i uses (noise_range[n-i], noise_range[n-i-1]).

    Follows oasis_inference.py:1765 and the reversed loop at 1843-1852. With 4 steps
    this yields [(999, 749), (749, 499), (499, 249), (249, -1)].
    """
    nr = torch.linspace(-1, max_noise_level - 1, n_steps + 1)
    out = []
    for noise_idx in reversed(range(1, n_steps + 1)):
        out.append((int(nr[noise_idx].item()), int(nr[noise_idx - 1].item())))
    return out


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

def rotate_half(x):
    """Pairs (2k, 2k+1) -> (-x[2k+1], x[2k]). Follows oasis_inference.py:327-332."""
    x = x.reshape(*x.shape[:-1], -1, 2)
    x1, x2 = x.unbind(dim=-1)
    return torch.stack((-x2, x1), dim=-1).reshape(*x.shape[:-2], -1)


def apply_rotary_emb(angles, t):
    """Rotate the first ``angles.shape[-1]`` dims of ``t``; the rest pass through.

    Follows oasis_inference.py:334-342.
    """
    rot = angles.shape[-1]
    t_rot, t_pass = t[..., :rot], t[..., rot:]
    t_rot = t_rot * angles.cos() + rotate_half(t_rot) * angles.sin()
    return torch.cat((t_rot, t_pass), dim=-1)


def _pair_repeat(a):
    return a.repeat_interleave(2, dim=-1)


def spatial_rope_angles(freqs, gh=GRID_H, gw=GRID_W):
    """Axial 2D angles ``[gh*gw, 4*len(freqs)]``: dims [0, 2F) use the row position,
    dims [2F, 4F) the column position, positions ``linspace(-1, 1)`` per axis, each
    frequency repeated for its pair. Follows oasis_inference.py:344-362.
    """
    h_pos = torch.linspace(-1, 1, steps=gh)
    w_pos = torch.linspace(-1, 1, steps=gw)
    hf = _pair_repeat(h_pos[:, None] * freqs[None].float())
    wf = _pair_repeat(w_pos[:, None] * freqs[None].float())
    hb = hf[:, None, :].expand(gh, gw, -1)
    wb = wf[None, :, :].expand(gh, gw, -1)
    return torch.cat([hb, wb], dim=-1).reshape(gh * gw, -1)


def temporal_rope_angles(freqs, T):
    """1D angles ``[T, 2*len(freqs)]`` at positions ``arange(T)``.

    Follows oasis_inference.py:364-373.
    """
    pos = torch.arange(T, dtype=torch.float32)
    return _pair_repeat(pos[:, None] * freqs[None].float())


def vae_rope_angles(freqs, gh=VAE_GRID_H, gw=VAE_GRID_W):
    """VAE 2D pixel angles ``[gh*gw, 4*len(freqs)]`` (same axial construction as the
    spatial DiT table; the reference reads them from the upstream VAE module,
    oasis_inference.py:455-479, which is not available)."""
    return spatial_rope_angles(freqs, gh, gw)


def rope_cos_sinperm(angles, head_dim):
    """Device-style tables: cos and ``sin_perm`` (sign -,+ baked in) over a full head,
    identity (cos=1, sin=0) past the rotated dims. Follows oasis_inference.py:390-403,
    464-473."""
    n, rot = angles.shape
    cos = torch.ones(n, head_dim)
    sin = torch.zeros(n, head_dim)
    cos[:, :rot] = angles.cos()
    sin[:, :rot] = angles.sin()
    sign = torch.ones(head_dim)
    sign[0:rot:2] = -1
    return cos, sin * sign


def apply_rope_swap(x, cos, sinperm):
    """``x*cos + swap_pairs(x)*sinperm``: the reference's device formulation
    (src/rope_layout_kernel.py:49-53, src/vae_rope.py:38-42)."""
    xs = x.reshape(*x.shape[:-1], -1, 2).flip(-1).reshape(x.shape)
    return x * cos + xs * sinperm


# ---------------------------------------------------------------------------
# elementwise pieces
# ---------------------------------------------------------------------------

def silu(x):
    """``x * sigmoid(x)``. Follows src/silu.py:25."""
    return x * torch.sigmoid(x)


def gelu_tanh(x):
    """``0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3)))``.

    Follows tests/test_kernels.py:262-281 (ttnn ``activation="gelu"`` in the DiT).
    """
    return 0.5 * x * (1.0 + torch.tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)))


def gelu_erf(x):
    """``0.5 x (1 + erf(x / sqrt 2))``: timm ``Mlp`` default ``nn.GELU`` used by the VAE
    (oasis_inference.py:35-51)."""
    return 0.5 * x * (1.0 + torch.erf(x / math.sqrt(2.0)))


def layer_norm(x, w=None, b=None, eps=LN_EPS):
    """LayerNorm over the last dim, eps 1e-6; affine only when ``w`` is given.

    Follows src/layernorm.py:42-68 and ttnn.layer_norm at oasis_inference.py:1053.
    """
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    y = (x - mu) / torch.sqrt(var + eps)
    if w is not None:
        y = y * _f(w) + _f(b)
    return y


def modulate(x, shift, scale):
    """``x (1 + scale) + shift``. Follows src/adaln_modulate.py:29."""
    return x * (1.0 + scale) + shift


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def attention(q, k, v, causal=False, pad_keys_to=None):
    """softmax(q k^T / sqrt(d)) v over the last two dims.

    Follows src/sdpa.py:69-87 (non-causal) and src/sdpa_causal.py:55-73 (additive
    causal bias, oasis_inference.py:843-857). ``pad_keys_to`` reproduces the
    reference's zero-padded key rows (tests/test_dit_block.py:548-554): extra keys
    with zero q/k/v that add exp(0 - max) to every denominator.
    """
    d = q.shape[-1]
    s = (q @ k.transpose(-1, -2)) / math.sqrt(d)
    if pad_keys_to is not None and pad_keys_to > k.shape[-2]:
        extra = pad_keys_to - k.shape[-2]
        s = torch.cat([s, torch.zeros(*s.shape[:-1], extra)], dim=-1)
        v = torch.cat([v, torch.zeros(*v.shape[:-2], extra, v.shape[-1])], dim=-2)
    if causal:
        lq, lk = s.shape[-2], s.shape[-1]
        mask = torch.ones(lq, lk, dtype=torch.bool).triu(1)
        s = s.masked_fill(mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return p @ v


# ---------------------------------------------------------------------------
# DiT
# ---------------------------------------------------------------------------

def adaln(silu_c, w, b):
    """Per-frame adaLN parameters ``silu(c) @ W^T + b`` -> ``[T, n*D]``.

    Follows build_per_frame_adaln (oasis_inference.py:971-993); the reference folds
    the +1 of ``(1 + scale)`` into the bias at load time (oasis_inference.py:553-554),
    here it stays in ``modulate``.
    """
    return silu_c @ _f(w).t() + _f(b)


def _heads(x, H):
    # [..., N, D] -> [..., H, N, d]
    *lead, n, dm = x.shape
    return x.reshape(*lead, n, H, dm // H).transpose(-2, -3)


def _unheads(x):
    # [..., H, N, d] -> [..., N, H*d]
    x = x.transpose(-2, -3)
    return x.reshape(*x.shape[:-2], -1)


def spatial_attention(q, k, v, cos, sinperm, H, pad_keys_to=None):
    """RoPE2D then full attention within each frame, per head.

    q,k,v: ``[T, P, D]``; cos/sinperm: ``[P, d]``. Follows the spatial branch of
    run_sub_block (oasis_inference.py:1076-1098) with src/rope_layout_kernel.py:16-86
    and src/sdpa.py:27-113.
    """
    qh, kh, vh = _heads(q, H), _heads(k, H), _heads(v, H)        # [T, H, P, d]
    qh = apply_rope_swap(qh, cos, sinperm)
    kh = apply_rope_swap(kh, cos, sinperm)
    o = attention(qh, kh, vh, causal=False, pad_keys_to=pad_keys_to)
    return _unheads(o)                                          # [T, P, D]


def temporal_attention(q, k, v, cos, sinperm, H):
    """RoPE1D over frame index then causal attention over frames, per position and head.

    q,k,v: ``[T, P, D]``; cos/sinperm: ``[T, d]``. Follows the temporal branch of
    run_sub_block (oasis_inference.py:1099-1139) with src/sdpa_causal.py:17-100 and
    the block-diagonal causal bias of oasis_inference.py:843-857.
    """
    qh, kh, vh = _heads(q, H), _heads(k, H), _heads(v, H)        # [T, H, P, d]
    c, s = cos[:, None, None, :], sinperm[:, None, None, :]
    qh = apply_rope_swap(qh, c, s)
    kh = apply_rope_swap(kh, c, s)
    # [T, H, P, d] -> [P, H, T, d]
    qt, kt, vt = (x.permute(2, 1, 0, 3) for x in (qh, kh, vh))
    o = attention(qt, kt, vt, causal=True)
    return _unheads(o.permute(2, 1, 0, 3))                     # [T, P, D]


def sub_block(x, silu_c, w, kind, rope_cos, rope_sinperm, n_heads=None, pad_keys_to=None):
    """One spatial (``kind='s'``) or temporal (``kind='t'``) sub-block.

    x: ``[T, P, D]`` fp32 residual stream; silu_c: ``[T, Dc]``. ``w`` holds
    ``ada_w, ada_b, qkv_w, out_w, out_b, fc1_w, fc1_b, fc2_w, fc2_b``.
    Follows run_sub_block (oasis_inference.py:995-1215):
      adaLN -> LN+modulate -> QKV (no bias) -> RoPE+attention -> O+bias, gated
      residual -> LN+modulate -> FC1+bias, tanh-GELU -> FC2+bias, gated residual.
    """
    D = x.shape[-1]
    n_heads = n_heads or D // D_HEAD
    ada = adaln(silu_c, w["ada_w"], w["ada_b"])[:, None, :]          # [T, 1, 6D]
    sh_a, sc_a, g_a, sh_m, sc_m, g_m = ada.split(D, dim=-1)
    h = modulate(layer_norm(x), sh_a, sc_a)
    qkv = h @ _f(w["qkv_w"]).t()
    q, k, v = qkv.split(D, dim=-1)
    if kind == "s":
        a = spatial_attention(q, k, v, rope_cos, rope_sinperm, n_heads, pad_keys_to)
    else:
        a = temporal_attention(q, k, v, rope_cos, rope_sinperm, n_heads)
    x = x + g_a * (a @ _f(w["out_w"]).t() + _f(w["out_b"]))
    h = modulate(layer_norm(x), sh_m, sc_m)
    g = gelu_tanh(h @ _f(w["fc1_w"]).t() + _f(w["fc1_b"]))
    x = x + g_m * (g @ _f(w["fc2_w"]).t() + _f(w["fc2_b"]))
    return x


def final_layer(x, silu_c, w):
    """adaLN(2 chunks) + LN + modulate + linear. Follows oasis_inference.py:1497-1521."""
    D = x.shape[-1]
    ada = adaln(silu_c, w["final.ada_w"], w["final.ada_b"])[:, None, :]
    shift, scale = ada.split(D, dim=-1)
    h = modulate(layer_norm(x), shift, scale)
    return h @ _f(w["final.w"]).t() + _f(w["final.b"])


def conditioning(t, action, w):
    """cond = MLP(timestep_embedding(t)) + Linear(action). Returns ``[T, D]``.

    Follows compute_cond_for_frame (oasis_inference.py:1406-1427):
    Linear(256->D), SiLU, Linear(D->D), plus external_cond Linear(25->D).
    """
    tf = timestep_embedding(torch.as_tensor(t), w["t_emb.w0"].shape[1])
    h = silu(tf @ _f(w["t_emb.w0"]).t() + _f(w["t_emb.b0"]))
    c = h @ _f(w["t_emb.w2"]).t() + _f(w["t_emb.b2"])
    if action is not None:
        c = c + (_f(action) @ _f(w["ext.w"]).t() + _f(w["ext.b"]))
    return c


def _grid(P):
    if P == N_PATCHES:
        return GRID_H, GRID_W
    raise ValueError("pass (gh, gw) explicitly for P=%d" % P)


def dit_forward(z, cond, w, n_blocks=None, n_heads=None, grid=None, pad_keys_to=None,
                return_hidden=False):
    """Full DiT forward on embedded tokens.

    z: ``[T, P, D]`` fp32 (patch-embedded frames); cond: ``[T, D]`` (pre-SiLU).
    Returns v: ``[T, P, OUT]``. Follows dit_forward_device
    (oasis_inference.py:1438-1526): SiLU once per frame (1459-1463), then
    ``n_blocks`` x (spatial, temporal) sub-blocks (1474-1492), then the final layer.
    """
    T, P, D = z.shape
    gh, gw = grid if grid is not None else _grid(P)
    n_heads = n_heads or D // D_HEAD
    d = D // n_heads
    sa = spatial_rope_angles(_f(w["rope.spatial_freqs"]), gh, gw)
    ta = temporal_rope_angles(_f(w["rope.temporal_freqs"]), T)
    s_cos, s_sin = rope_cos_sinperm(sa, d)
    t_cos, t_sin = rope_cos_sinperm(ta, d)
    sc = silu(_f(cond))
    x = _f(z)
    nb = n_blocks if n_blocks is not None else _count(w, "blocks.%d.s.ada_w")
    for i in range(nb):
        x = sub_block(x, sc, _blk(w, i, "s"), "s", s_cos, s_sin, n_heads, pad_keys_to)
        x = sub_block(x, sc, _blk(w, i, "t"), "t", t_cos, t_sin, n_heads)
    v = final_layer(x, sc, w)
    return (v, x) if return_hidden else v


def _count(w, pattern):
    n = 0
    while (pattern % n) in w:
        n += 1
    return n


def _blk(w, i, kind):
    p = "blocks.%d.%s." % (i, kind)
    return {k[len(p):]: v for k, v in w.items() if k.startswith(p)}


# ---------------------------------------------------------------------------
# patches, DDIM, bridge
# ---------------------------------------------------------------------------

def patch_embed(latent, w):
    """Conv2d(C->D, k=2, s=2) on ``[T, C, H, W]`` -> ``[T, P, D]`` (row-major patches).

    Follows patch_embed_host (oasis_inference.py:950-956).
    """
    y = F.conv2d(_f(latent), _f(w["x_emb.w"]), _f(w["x_emb.b"]), stride=PATCH)
    T, D, h, ww = y.shape
    return y.permute(0, 2, 3, 1).reshape(T, h * ww, D)


def patchify_to_output_space(img):
    """``[T, C, H, W]`` -> ``[T, P, p*q*C]`` with column order (p, q, c).

    Follows oasis_inference.py:958-963.
    """
    T, C, H, W = img.shape
    x = _f(img).reshape(T, C, H // PATCH, PATCH, W // PATCH, PATCH)
    x = torch.einsum("nchpwq->nhwpqc", x)
    return x.reshape(T, (H // PATCH) * (W // PATCH), PATCH * PATCH * C)


def unpatchify(x, gh=GRID_H, gw=GRID_W, C=IN_CH):
    """Inverse of ``patchify_to_output_space``. Follows oasis_inference.py:965-969."""
    T = x.shape[0]
    x = _f(x).reshape(T, gh, gw, PATCH, PATCH, C)
    x = torch.einsum("nhwpqc->nchpwq", x)
    return x.reshape(T, C, gh * PATCH, gw * PATCH)


def patch_embed_roundtrip_weight(w):
    """``W_rt [64, D]``: conv weight reordered to the (p, q, c) patch column order, so
    ``patchify(img) @ W_rt + b == patch_embed(img)``. Follows oasis_inference.py:1821-1826.
    """
    cw = _f(w["x_emb.w"])                       # [D, C, 2, 2]
    D = cw.shape[0]
    return cw.permute(0, 2, 3, 1).reshape(D, -1).t().contiguous()


def ddim_coeffs(alphas_cumprod, t, t_next, last):
    """``(sqrt a, sqrt(1-a), sqrt(1/a), 1/sqrt(1/a-1), sqrt a', sqrt(1-a'))`` with a'=1 on
    the last step. Follows oasis_inference.py:1843-1860."""
    at = float(alphas_cumprod[t].item())
    an = 1.0 if last else float(alphas_cumprod[max(t_next, 0)].item())
    return (at ** 0.5, (1 - at) ** 0.5, (1.0 / at) ** 0.5, 1.0 / ((1.0 / at - 1) ** 0.5),
            an ** 0.5, (1 - an) ** 0.5)


def ddim_update(x, v, c):
    """v-prediction DDIM step. Follows ddim_step_fn (oasis_inference.py:1919-1931):
    ``x0 = sqrt(a) x - sqrt(1-a) v``; ``eps = (sqrt(1/a) x - x0) / sqrt(1/a - 1)``;
    ``x' = sqrt(a') x0 + sqrt(1-a') eps``."""
    at_s, omat_s, inv_at_s, inv_sig, an_s, oman_s = c
    x0 = at_s * x - omat_s * v
    eps = (inv_at_s * x - x0) * inv_sig
    return an_s * x0 + oman_s * eps


def bridge(chunk, gh=GRID_H, gw=GRID_W, C=IN_CH, out_cols=32):
    """DiT patches ``[P, p*q*C]`` -> VAE latent ``[(gh*2)*(gw*2), out_cols]``, scaled by
    1/SCALING_FACTOR, channels in cols [0, C), zeros after.

    VAE row ``r = (h*2+p)*(gw*2) + (w*2+q)`` takes DiT row ``h*gw + w``, cols
    ``(p*2+q)*C + c``. Follows build_bridge_matrices/bridge_unpatchify
    (oasis_inference.py:1651-1709).
    """
    x = _f(chunk).reshape(gh, gw, PATCH, PATCH, C)              # h w p q c
    x = x.permute(0, 2, 1, 3, 4).reshape(gh * PATCH * gw * PATCH, C)
    out = torch.zeros(x.shape[0], out_cols)
    out[:, :C] = x / SCALING_FACTOR
    return out


# ---------------------------------------------------------------------------
# VAE decoder
# ---------------------------------------------------------------------------

def vae_decode(latent, w, n_heads=None, grid=(VAE_GRID_H, VAE_GRID_W)):
    """ViT decoder ``[N, Lc] -> [N, 3*20*20]``.

    Follows vae_decode_forward (oasis_inference.py:1546-1618): post_quant linear;
    ``depth`` x [LN(affine) -> QKV+bias -> RoPE on the first 32 dims of each head
    -> SDPA (non-causal) -> proj+bias -> residual -> LN(affine) -> FC1+bias, GELU
    -> FC2+bias -> residual]; final LN(affine); predictor linear.
    """
    x = _f(latent) @ _f(w["pq_w"]).t() + _f(w["pq_b"])
    D = x.shape[-1]
    n_heads = n_heads or D // D_HEAD
    d = D // n_heads
    if "rope.vae_angles" in w:     # the model's own angle table (oasis_inference.py:455-468)
        ang = _f(w["rope.vae_angles"]).reshape(x.shape[0], -1)
    else:
        ang = vae_rope_angles(_f(w["rope.vae_freqs"]), *grid)
    cos, sinp = rope_cos_sinperm(ang, d)
    for i in range(_count(w, "dec.%d.qkv_w")):
        p = "dec.%d." % i
        h = layer_norm(x, w[p + "n1_w"], w[p + "n1_b"])
        qkv = h @ _f(w[p + "qkv_w"]).t() + _f(w[p + "qkv_b"])
        q, k, v = (_heads(t, n_heads) for t in qkv.split(D, dim=-1))  # [H, N, d]
        q = apply_rope_swap(q, cos, sinp)
        k = apply_rope_swap(k, cos, sinp)
        a = _unheads(attention(q, k, v))
        x = x + (a @ _f(w[p + "proj_w"]).t() + _f(w[p + "proj_b"]))
        h = layer_norm(x, w[p + "n2_w"], w[p + "n2_b"])
        g = gelu_erf(h @ _f(w[p + "fc1_w"]).t() + _f(w[p + "fc1_b"]))
        x = x + (g @ _f(w[p + "fc2_w"]).t() + _f(w[p + "fc2_b"]))
    h = layer_norm(x, w["norm_w"], w["norm_b"])
    return h @ _f(w["pred_w"]).t() + _f(w["pred_b"])


def vae_unpatchify(patches, gh=VAE_GRID_H, gw=VAE_GRID_W, ps=VAE_PATCH):
    """``[gh*gw, 3*ps*ps]`` (cols ordered c, p, q) -> ``[3, gh*ps, gw*ps]`` clamped to [-1, 1].

    Follows vae_unpatchify (oasis_inference.py:1636-1645) and the clamp at 2292.
    """
    x = _f(patches).reshape(gh, gw, 3, ps, ps)                   # h w c p q
    x = x.permute(2, 0, 3, 1, 4).reshape(3, gh * ps, gw * ps)
    return x.clamp(-1.0, 1.0)


def ddim_frame(x_noise, ctx_z, ctx_cond, gen_conds, w, vae_w, alphas_cumprod, steps,
               n_blocks=None, grid=None, vae_grid=(VAE_GRID_H, VAE_GRID_W)):
    """One generated frame: ``len(steps)`` DDIM steps over the T=2 DiT, then the bridge,
    the VAE decoder and unpatchify.

    x_noise: ``[P, 64]`` patchified noise chunk; ctx_z: ``[P, D]`` embedded context
    frame; ctx_cond: ``[D]``; gen_conds: one ``[D]`` cond per step; steps: list of
    ``(t, t_next)``. Follows ddim_step_fn (oasis_inference.py:1909-1932) and the
    traced frame (2131-2148).
    Returns (chunk ``[P, 64]``, frame ``[3, H, W]``).
    """
    W_rt = patch_embed_roundtrip_weight(w)
    b_rt = _f(w["x_emb.b"])
    chunk = _f(x_noise)
    for i, (t, tn) in enumerate(steps):
        gen_z = chunk @ W_rt + b_rt
        z = torch.stack([_f(ctx_z), gen_z], dim=0)
        cond = torch.stack([_f(ctx_cond), _f(gen_conds[i])], dim=0)
        v = dit_forward(z, cond, w, n_blocks=n_blocks, grid=grid)[1]
        c = ddim_coeffs(alphas_cumprod, t, tn, last=(i == len(steps) - 1))
        chunk = ddim_update(chunk, v, c)
    gh, gw = grid if grid is not None else (GRID_H, GRID_W)
    lat = bridge(chunk, gh, gw)
    pred = vae_decode(lat, vae_w, grid=vae_grid)
    return chunk, vae_unpatchify(pred, *vae_grid)


# ---------------------------------------------------------------------------
# fp8 weight path (config 4). The reference has no sub-fp32 path, so these restate the
# build's own scheme: OCP e4m3 (max 448), round to nearest even.
# ---------------------------------------------------------------------------
E4M3_MAX = 448.0


def quantize_e4m3_rows(w):
    """Per-output-channel e4m3 weights: s_n = max_k |W[n, k]| / 448 (1 for a zero row),
    q = round_e4m3(W / s_n). Returns (q as fp32 values on the e4m3 grid, s [N])."""
    w = _f(w)
    amax = w.abs().amax(dim=1)
    s = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    q = (w / s[:, None]).to(torch.float8_e4m3fn).float()
    return q, s


def quantize_act_blocks(x, block=32):
    """Activations as the fp8 GEMM sees them: each `block`-wide run of a row gets a
    power-of-two scale 2^e with max |x| / 2^e in [128, 256) (e >= -127), then
    round_e4m3(x / 2^e) * 2^e."""
    x = _f(x)
    M, K = x.shape
    xb = x.reshape(M, K // block, block)
    amax = xb.abs().amax(dim=-1, keepdim=True)
    _, ex = torch.frexp(amax)               # amax = m * 2^ex, m in [0.5, 1)
    e = torch.clamp(ex - 8, min=-127).float()
    scale = torch.pow(2.0, e)
    q = (xb / scale).to(torch.float8_e4m3fn).float() * scale
    return q.reshape(M, K)


def fp8_weights(w):
    """A copy of a DiT weight dict whose QKV / O / FC1 / FC2 weights are replaced by
    their per-channel e4m3 dequantized values (what the fp8 path multiplies by)."""
    out = dict(w)
    for k, v in w.items():
        if k.startswith("blocks.") and k.rsplit(".", 1)[1] in ("qkv_w", "out_w", "fc1_w", "fc2_w"):
            q, s = quantize_e4m3_rows(v)
            out[k] = q * s[:, None]
    return out
