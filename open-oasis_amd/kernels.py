"""The reference's kernel surface on liboasis_hip.so.

Same names, factory arguments and destination-passing call signatures as the TT-Lang
kernels that oasis_inference.py imports (oasis_inference.py:75-84): inputs first,
preallocated outputs last, written in place, nothing returned. Tensors are torch-ROCm
device tensors; 2-D shapes follow the reference (heads stacked along rows, tables and
biases row-expanded). ``scaler``, ``mean_scale`` and ``attn_scratch`` are Tensix
reduction constants / dtype templates in the reference and are accepted and ignored.

Errors: a shape or dtype the kernels do not support raises ``OasisError`` (the
reference fails at JIT compile or hangs).
"""
import math

import torch

from . import _lib as L
from .model import DiT, VAE, DiTWorkspace, VAEWorkspace

TILE = 32

_DT = {torch.float32: L.F32, torch.bfloat16: L.BF16}


def _dtype(*ts):
    d = ts[0].dtype
    if any(t.dtype != d for t in ts) or d not in _DT:
        raise L.OasisError("dtype", L.OASIS_OK - 3, "tensors must all be fp32 or all bf16, got %s"
                           % [t.dtype for t in ts])
    return _DT[d]


def _chk(*ts):
    for t in ts:
        if not (t.is_cuda and t.is_contiguous()):
            raise L.OasisError("tensor", -2, "expected contiguous device tensors")


def _f32(t):
    return t if t.dtype == torch.float32 else t.float()


def silu_kernel(x, out):
    """out = x * sigmoid(x) (src/silu.py:8-25)."""
    _chk(x, out)
    L.call("oasis_silu", L.ptr(x), L.ptr(out), x.numel(), _dtype(x, out), L.stream_handle())


def gated_residual_kernel(residual, x, gate, out):
    """out = residual + x * gate (src/gated_residual.py:16-38)."""
    _chk(residual, x, gate, out)
    L.call("oasis_gated_residual", L.ptr(residual), L.ptr(x), L.ptr(gate), L.ptr(out),
           out.numel(), _dtype(residual, x, gate, out), L.stream_handle())


def bias_gated_residual_kernel(residual, x, bias, gate, out):
    """out = residual + (x + bias) * gate (src/gated_residual.py:65-89)."""
    _chk(residual, x, bias, gate, out)
    L.call("oasis_bias_gated_residual", L.ptr(residual), L.ptr(x), L.ptr(bias), L.ptr(gate),
           L.ptr(out), out.numel(), _dtype(residual, x, bias, gate, out), L.stream_handle())


def adaln_modulate_kernel(x, shift, scale, out):
    """out = x * (scale + 1) + shift (src/adaln_modulate.py:8-29)."""
    _chk(x, shift, scale, out)
    L.call("oasis_adaln_modulate", L.ptr(x), L.ptr(shift), L.ptr(scale), L.ptr(out), out.numel(),
           _dtype(x, shift, scale, out), L.stream_handle())


def make_layernorm_kernel(dim_tiles, eps=1e-6):
    """LayerNorm with affine over dim_tiles*32 columns (src/layernorm.py:15-96)."""
    cols = dim_tiles * TILE

    def layernorm_kernel(x, weight, ln_bias, scaler, mean_scale, out):
        _chk(x, out)
        if x.shape[-1] != cols:
            raise L.OasisError("layernorm", -2, "expected %d columns, got %d" % (cols, x.shape[-1]))
        w, b = _f32(weight).contiguous(), _f32(ln_bias).contiguous()
        wb_ld = cols if w.dim() == 2 and w.shape[0] > 1 else 0
        L.call("oasis_layernorm", L.ptr(x), L.ptr(w), L.ptr(b), wb_ld, L.ptr(out),
               x.numel() // cols, cols, eps, _dtype(x, out), L.stream_handle())
    return layernorm_kernel


def make_linear_kernel(k_chunk):
    """out = x @ w with w [K, N] (src/linear.py:10-53). x and w bf16; out fp32 or bf16."""
    def linear_kernel(x, w, out):
        _chk(x, w, out)
        M, K = x.shape
        N = w.shape[1]
        if K != k_chunk * TILE:
            raise L.OasisError("linear", -2, "K=%d does not match k_chunk=%d" % (K, k_chunk))
        xb = x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)
        wb = w if w.dtype == torch.bfloat16 else w.to(torch.bfloat16)
        L.call("oasis_linear", L.ptr(xb), L.ptr(wb), L.ptr(out), M, K, N, 0, _DT[out.dtype],
               L.stream_handle())
    return linear_kernel


def _rope_call(qkv_full, cos_tab, sin_tab, q_out, k_out, v_out, n_heads, seq, mode):
    _chk(qkv_full, q_out, k_out, v_out)
    c, s = _f32(cos_tab).contiguous(), _f32(sin_tab).contiguous()
    rows = qkv_full.shape[0]
    L.call("oasis_rope_layout", L.ptr(qkv_full), qkv_full.shape[1], L.ptr(c), L.ptr(s), c.shape[1], 64,
           1, c.shape[0], L.ptr(q_out), L.ptr(k_out), L.ptr(v_out), rows, seq, n_heads, 64, mode,
           _dtype(qkv_full, q_out, k_out, v_out), L.stream_handle())


def make_rope_layout_kernel(seq_tiles, head_tiles, n_heads_val):
    """RoPE on Q/K + heads-first split: out row (frame*H + h)*seq + p
    (src/rope_layout_kernel.py:16-86). Tables are [SEQ, H*64] per row."""
    assert head_tiles * TILE == 64

    def rope_layout(qkv_full, cos_tab, sin_tab, q_out, k_out, v_out):
        _rope_call(qkv_full, cos_tab, sin_tab, q_out, k_out, v_out, n_heads_val, seq_tiles * TILE, 0)
    return rope_layout


def make_rope_temporal_kernel(head_tiles, n_heads_val):
    """RoPE on Q/K, token-major outputs (src/rope_layout_kernel.py:89-161)."""
    assert head_tiles * TILE == 64

    def rope_temporal(qkv_full, cos_tab, sin_tab, q_out, k_out, v_out):
        _rope_call(qkv_full, cos_tab, sin_tab, q_out, k_out, v_out, n_heads_val, qkv_full.shape[0], 1)
    return rope_temporal


def make_vae_rope_kernel(n_heads, head_tiles):
    """VAE RoPE + heads-first split: out row h*seq + row (src/vae_rope.py:8-74)."""
    assert head_tiles * TILE == 64

    def vae_rope_kernel(qkv_full, cos_tab, sin_tab, q_out, k_out, v_out):
        _rope_call(qkv_full, cos_tab, sin_tab, q_out, k_out, v_out, n_heads, qkv_full.shape[0], 0)
    return vae_rope_kernel


def _sdpa_call(Q, K, V, out, sq, skv, scale, bias, causal, total_heads):
    _chk(Q, K, V, out)
    nh = total_heads if total_heads is not None else Q.shape[0] // sq
    b = None if bias is None else _f32(bias).contiguous()
    L.call("oasis_sdpa", L.ptr(Q), L.ptr(K), L.ptr(V), L.ptr(out), nh, sq, skv, Q.shape[1], scale,
           L.ptr(b), int(causal), _dtype(Q, K, V, out), L.stream_handle())


def make_sdpa_kernel(sq_tiles, skv_tiles, head_tiles, scale_val):
    """Non-causal multi-head SDPA, heads stacked along rows (src/sdpa.py:27-113)."""
    def sdpa_kernel(Q_all, K_all, V_all, scaler, attn_scratch, out):
        _sdpa_call(Q_all, K_all, V_all, out, sq_tiles * TILE, skv_tiles * TILE, scale_val, None, False, None)
    return sdpa_kernel


def make_sdpa_causal_kernel(sq_tiles, skv_tiles, head_tiles, scale_val, total_heads=None):
    """SDPA with an additive [sq, skv] bias shared by all heads (src/sdpa_causal.py:17-100)."""
    def sdpa_causal_kernel(Q_all, K_all, V_all, scaler, bias, attn_scratch, out):
        _sdpa_call(Q_all, K_all, V_all, out, sq_tiles * TILE, skv_tiles * TILE, scale_val, bias, False,
                   total_heads)
    return sdpa_causal_kernel


def make_adaln_matmul_expand_kernel(k_tiles, n_repeat):
    """out = expand(silu_cond[0] @ adaln_w + adaln_b) over n_repeat row tiles
    (src/adaln_matmul_expand.py:13-62)."""
    def adaln_matmul_expand(silu_cond, adaln_w, adaln_b, out):
        _chk(silu_cond, adaln_w, out)
        K, N = adaln_w.shape
        c = _f32(silu_cond[0]).contiguous()
        w = adaln_w if adaln_w.dtype == torch.bfloat16 else adaln_w.to(torch.bfloat16)
        b = _f32(adaln_b.reshape(-1, N)[0]).contiguous()
        o = out if out.dtype == torch.float32 else torch.empty(out.shape, device=out.device)
        L.call("oasis_adaln_matmul_expand", L.ptr(c), L.ptr(w), L.ptr(b), L.ptr(o), K, N,
               min(out.shape[0], n_repeat * TILE), L.stream_handle())
        if o is not out:
            out.copy_(o)
    return adaln_matmul_expand


# instances with the reference's names (oasis_inference.py:171-209)
linear_k32 = make_linear_kernel(32)
layernorm_d1024 = make_layernorm_kernel(32)


def padded_rows(rows):
    """Rows per frame in the reference's TILE layout: 144 -> 160 (N_PATCH_PAD,
    oasis_inference.py:103)."""
    return -(-rows // TILE) * TILE


def _surface_workspace(dev, scr, T):
    """The DiTWorkspace a reference-named composite call runs in: scr when it is one (the
    caller's buffers), else one kept on dev and replaced only when T frames do not fit, so calls
    in sequence allocate nothing (the reference's composite calls never allocate,
    oasis_inference.py:1546-1549; a call that grows it must not be inside a graph capture)."""
    M = T * dev.P
    if isinstance(scr, DiTWorkspace):
        if scr.max_rows < M or scr.max_cond < T:
            raise L.OasisError("dit_forward", -2, "workspace holds %d rows / %d cond rows, the call needs %d / %d"
                               % (scr.max_rows, scr.max_cond, M, T))
        return scr
    ws = getattr(dev, "_surface_ws", None)
    if ws is None or ws.max_rows < M or ws.max_cond < T:
        ws = dev._surface_ws = dev.workspace(M, max_cond=max(16, T))
    return ws


def _padded_v(ws, dev, T):
    """ws's v rows in the padded layout [T*160, 64]: frame t's 144 rows at t*160, the 16 pad
    rows after them zero (written once here and never again)."""
    Pp = padded_rows(dev.P)
    vp = getattr(ws, "v_pad", None)
    if vp is None or vp.shape[0] < T * Pp:
        vp = ws.v_pad = torch.zeros(max(ws.max_rows // dev.P, T) * Pp, dev.patch_dim, device=dev.device)
    return vp[:T * Pp]


def dit_forward_device(z_cur, cond_list, dev, scr=None, tt_device=None, scaler=None, mean_scale=None,
                       profile_step=False):
    """DiT forward (oasis_inference.py:1438-1526).

    z_cur: embedded tokens, fp32 (or bf16) device tensor, either the reference's padded
    layout [T*160, D] (SEQ = N_PATCH_PAD*T, oasis_inference.py:1445: frame t's 144 tokens at
    row t*160, the 16 pad rows after them ignored) or packed [T*144, D].
    cond_list: T conditioning vectors (pre-SiLU; [D] or the reference's row-expanded [32, D])
    or a [T, D] tensor. dev: a ``DiT``. scr: a ``DiTWorkspace``, or anything else (the
    reference's scratch dict): then a workspace kept on dev is used.
    Returns v fp32 in the layout z_cur came in: [T*160, 64] with the pad rows zero, so that
    ddim_step_fn's slice at gen_start = (T-1)*160 works unchanged (oasis_inference.py:1915-
    1918), or [T*144, 64]. The result is a view of the workspace, valid until its next call.
    Nothing is allocated once the workspace exists (the inputs are copied into it). Spatial
    attention runs over the 144 tokens of each frame (the reference also lets the 16 pad keys
    into every softmax, with logit 0).
    """
    assert isinstance(dev, DiT)
    D, P = dev.d, dev.P
    T = len(cond_list) if isinstance(cond_list, (list, tuple)) else cond_list.shape[0]
    rows = z_cur.numel() // D
    Pp = padded_rows(P)
    if rows == T * P:
        padded = False
    elif rows == T * Pp:
        padded = True
    else:
        raise L.OasisError("dit_forward", -2, "z_cur has %d rows; expected T*%d (padded) or T*%d for T=%d"
                           % (rows, Pp, P, T))
    ws = _surface_workspace(dev, scr, T)
    for t in range(T):
        c = cond_list[t]
        ws.cond[t].copy_(c.reshape(-1, D)[0])
    ada = dev.adaln_inplace(T, ws)
    z = z_cur.reshape(rows, D)
    if padded:
        ws.x[:T * P].view(T, P, D).copy_(z.view(T, Pp, D)[:, :P])
    else:
        ws.x[:T * P].copy_(z)
    dev.forward_inplace(ws, 1, T, ada, dev.ada_width, ws.v_out)
    if not padded:
        return ws.v_out[:T * P]
    out = _padded_v(ws, dev, T)
    out.view(T, Pp, -1)[:, :P].copy_(ws.v_out[:T * P].view(T, P, -1))
    return out


dit_forward = dit_forward_device


def _vae_workspace(vae_dev, vae_scr):
    if isinstance(vae_scr, VAEWorkspace):
        return vae_scr
    ws = getattr(vae_dev, "_surface_ws", None)
    if ws is None:
        ws = vae_dev._surface_ws = vae_dev.workspace()
    return ws


def vae_decode_forward(vae_dev, vae_scr, scaler=None, mean_scale=None, fused_frame=False):
    """VAE decode of vae_scr.latent[:L] (the reference's vae_input), oasis_inference.py:1546-1618.

    Returns vae_scr.pred_out, fp32 [L, 1216] as the reference returns vae_scr["pred_out"]: the
    predictor's rows, unclamped, columns 1200.. zero (TILE padding). fused_frame=True runs the
    fast path instead: vae_unpatchify and the clamp (oasis_inference.py:1636-1645,2292) fused
    into the predictor, returning vae_scr.frame [3, 360, 640] in [-1, 1].
    """
    assert isinstance(vae_dev, VAE)
    ws = _vae_workspace(vae_dev, vae_scr)
    if fused_frame:
        vae_dev.decode_inplace(ws.latent, ws.frame, ws)
        return ws.frame
    vae_dev.decode_patches(ws.latent[:vae_dev.L], ws.pred_out, ws)
    return ws.pred_out


def vae_decode_device(z_flat, vae_dev, vae_scr=None, tt_device=None, scaler=None, mean_scale=None):
    """z_flat [L, C] (C <= latent_dim; already divided by the scaling factor) -> the predictor's
    rows as a host fp32 tensor [L, 1200] (oasis_inference.py:1620-1634): the latent is
    zero-padded to latent_dim columns in the workspace, decoded, and read back without the
    TILE padding, ready for the reference's host-side vae_unpatchify."""
    assert isinstance(vae_dev, VAE)
    ws = _vae_workspace(vae_dev, vae_scr)
    z = z_flat.reshape(vae_dev.L, -1)
    c = z.shape[1]
    if c > vae_dev.latent_dim:
        raise L.OasisError("vae_decode_device", -2, "z_flat has %d columns, the decoder takes %d"
                           % (c, vae_dev.latent_dim))
    lat = ws.latent[:vae_dev.L]
    lat[:, c:].zero_()
    lat[:, :c].copy_(z)
    pred = vae_decode_forward(vae_dev, ws)
    return pred[:, :vae_dev.patch_dim].cpu()


def vae_decode(latent, vae_dev, vae_scr=None):
    """latent [L, latent_dim] fp32 -> frame [3, H, W] in [-1, 1] (the fused fast path)."""
    ws = _vae_workspace(vae_dev, vae_scr)
    ws.latent[:vae_dev.L].copy_(latent.reshape(vae_dev.L, -1))
    return vae_decode_forward(vae_dev, ws, fused_frame=True)


def attention_scale(head_dim=64):
    return 1.0 / math.sqrt(head_dim)
