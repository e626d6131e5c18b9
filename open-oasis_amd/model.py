"""Device-resident Oasis DiT, ViT VAE decoder and the DDIM frame pipeline.

Host side of the hot path: it lays the weights out in HBM once, owns the activation
workspaces (allocated up front, so nothing allocates inside a step or a captured
graph), fills the C structs of include/oasis_hip.h and calls the composite entry
points of liboasis_hip.so on a torch-ROCm stream.

HBM layout (nn.Linear [out, in] weights, fp32 biases/tables):
  - ``ada_w`` (bf16): every sub-block's adaLN projection stacked, [n_sub*6D, D] (403 MB at
    Oasis-500M), in the 16-row MFMA tile order of ``oasis_gemv_bf16_tiled`` (``tile_rows16``),
    so each wave of the skinny GEMM streams 1 KB contiguous per load. One pass over it produces
    the adaLN rows of all 32 sub-blocks for every conditioning row at once.
  - per sub-block (bf16): qkv_w [3D, D], out_w [D, D], fc1_w [Dm, D], fc2_w [D, Dm], each
    contiguous (37.7 MB of the 1.21 GB weight set per sub-block incl. adaLN).
  - per sub-block (bf16), for the passes of at most 320 tokens: out_w, fc1_w and fc2_w once
    more in the MFMA fragment order of ``tile_rows16`` (``DiT(frag=...)`` picks the roles; 604 MB
    at Oasis-500M for the default three).
  - fp32, as the reference keeps them (oasis_inference.py:512-532,1821-1826): the
    conditioning MLP and action projection (zero-padded to 64 inputs), the patch embed
    [D, 64] in (p, q, c) column order, the final layer's adaLN [2D, D] and linear [64, D].
  - RoPE cos/sin tables (fp32).
"""
import ctypes
import math

import torch

from . import _lib as L

HEAD_DIM = 64


def tile_rows16(W):
    """[N, K] -> the 16-row MFMA tile order of oasis_gemv_bf16_tiled (same shape, [N, K]): for
    tile t and 32-wide K step s, 64 pieces of 8 values, piece l = row 16t + (l % 16), columns
    32s + 8(l // 16) .. +7."""
    N, K = W.shape
    assert N % 16 == 0 and K % 32 == 0
    return W.reshape(N // 16, 16, K // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(N, K).contiguous()


FRAG_ROLES_ALL = ("qkv", "out", "fc1", "fc2")
FRAG_ROLES_DEFAULT = ("out", "fc1", "fc2")


def frag_rows(m):
    """Rows of h, attn and mlp a fragment-order pass of m tokens reads: m rounded up to its row
    tiles (48 rows up to 160 tokens; 48 or 80 above)."""
    r48, r80 = -(-m // 48) * 48, -(-m // 80) * 80
    return r48 if m <= 160 else max(r48, r80)


def untile_rows16(Wt):
    """Inverse of tile_rows16."""
    N, K = Wt.shape
    return Wt.reshape(N // 16, K // 32, 4, 16, 8).permute(0, 3, 1, 2, 4).reshape(N, K).contiguous()


def _count(w, pattern):
    n = 0
    while (pattern % n) in w:
        n += 1
    return n


def _axial_angles(freqs, gh, gw):
    """Axial 2D RoPE angles [gh*gw, 4F]: dims [0,2F) row position, [2F,4F) column
    position, positions linspace(-1, 1), each frequency repeated for its pair
    (precompute_spatial_rope_freqs, oasis_inference.py:344-362)."""
    hp = torch.linspace(-1, 1, gh, dtype=torch.float64)
    wp = torch.linspace(-1, 1, gw, dtype=torch.float64)
    f = freqs.double()
    ha = (hp[:, None] * f[None]).repeat_interleave(2, dim=1)   # [gh, 2F]
    wa = (wp[:, None] * f[None]).repeat_interleave(2, dim=1)   # [gw, 2F]
    a = torch.cat([ha[:, None, :].expand(gh, gw, -1), wa[None, :, :].expand(gh, gw, -1)], dim=-1)
    return a.reshape(gh * gw, -1)


def rope_tables(angles, head_dim=HEAD_DIM):
    """cos and sign-baked sin ([-sin, +sin] per pair) over a full head; identity past
    the rotated dims (build_*_rope_device_tables, oasis_inference.py:390-403,464-473)."""
    n, rot = angles.shape
    cos = torch.ones(n, head_dim, dtype=torch.float64)
    sin = torch.zeros(n, head_dim, dtype=torch.float64)
    cos[:, :rot] = torch.cos(angles)
    sin[:, :rot] = torch.sin(angles)
    sin[:, 0:rot:2] *= -1
    return cos.float(), sin.float()


def temporal_angles(freqs, t_max):
    """1D angles [t_max, 2F] at positions arange (oasis_inference.py:364-373)."""
    pos = torch.arange(t_max, dtype=torch.float64)
    return (pos[:, None] * freqs.double()[None]).repeat_interleave(2, dim=1)


class DiT:
    """Oasis DiT weights resident on one GPU.

    weights="bf16" keeps the projection weights in bf16. weights="fp8" stores the QKV, O,
    FC1 and FC2 weights as OCP e4m3 with one fp32 scale per output channel (quantized on
    the device by oasis_quantize_fp8_rows) and runs those projections on the fp8 GEMM;
    the sub-blocks' adaLN stays bf16, and conditioning, patch embed and the final layer
    fp32, in both modes."""

    def __init__(self, w, device="cuda", grid=(9, 16), t_max=32, weights="bf16", frag=True):
        if weights not in ("bf16", "fp8"):
            raise ValueError("weights must be 'bf16' or 'fp8'")
        self.weights = weights
        # bf16: projection weights also in MFMA fragment order (tile_rows16) for the passes of at
        # most 320 tokens (the step, the K/V-cache passes), for the roles whose operands those passes
        # keep in that order (OASIS_FRAG in the library; by default O, FC1 with the LayerNorm after
        # O carried into it, and FC2 at one frame). frag: True for those three, False for none, or
        # an iterable of "qkv", "out", "fc1", "fc2".
        roles = FRAG_ROLES_DEFAULT if frag is True else (() if not frag else tuple(frag))
        if any(r not in FRAG_ROLES_ALL for r in roles):
            raise ValueError("frag roles must be among %s" % (FRAG_ROLES_ALL,))
        self.frag_roles = roles if weights == "bf16" else ()
        self.frag = bool(self.frag_roles)
        self.device = torch.device(device)
        dev = self.device
        self.d = d = w["t_emb.w2"].shape[0]
        assert d % HEAD_DIM == 0
        self.n_heads = d // HEAD_DIM
        self.n_blocks = _count(w, "blocks.%d.s.ada_w")
        self.n_sub = 2 * self.n_blocks
        assert 0 < self.n_sub <= L.MAX_SUB
        self.d_mlp = w["blocks.0.s.fc1_w"].shape[0]
        self.grid = grid
        self.P = grid[0] * grid[1]
        self.in_ch = w["x_emb.w"].shape[1]
        self.patch_dim = w["final.w"].shape[0]
        self.freq_dim = w["t_emb.w0"].shape[1]
        self.ext_dim = w["ext.w"].shape[1]
        self.ext_pad = 64 * ((self.ext_dim + 63) // 64)
        self.t_max = t_max
        bf = torch.bfloat16
        keep = []
        frag_keep = []

        def put(t, dtype):
            x = t.to(device=dev, dtype=dtype).contiguous()
            keep.append(x)
            return x

        f32 = torch.float32
        # adaLN projections of all sub-blocks (bf16), +1 folded into each scale chunk
        # (oasis_inference.py:549-556); the final layer's in fp32 (527-532)
        ws, bs = [], []
        for i in range(self.n_blocks):
            for kind in "st":
                ws.append(w["blocks.%d.%s.ada_w" % (i, kind)])
                b = w["blocks.%d.%s.ada_b" % (i, kind)].float().clone()
                b[d:2 * d] += 1.0
                b[4 * d:5 * d] += 1.0
                bs.append(b)
        self.ada_width = self.n_sub * 6 * d + 2 * d   # adaLN row width: every sub-block, then the final layer
        self.ada_w = put(tile_rows16(torch.cat([x.to(bf) for x in ws], 0)), bf)
        self.ada_b = put(torch.cat(bs, 0), f32)
        del ws, bs
        fb = w["final.ada_b"].float().clone()
        fb[d:2 * d] += 1.0
        self.final_ada_w = put(w["final.ada_w"], f32)
        self.final_ada_b = put(fb, f32)

        S = L.DiTWeights()
        S.n_sub, S.d_model, S.n_heads, S.d_mlp = self.n_sub, d, self.n_heads, self.d_mlp
        S.grid_h, S.grid_w, S.patch_dim = grid[0], grid[1], self.patch_dim
        S.freq_dim, S.ext_dim_pad = self.freq_dim, self.ext_pad
        S.ada_w, S.ada_b = self.ada_w.data_ptr(), self.ada_b.data_ptr()
        S.final_ada_w, S.final_ada_b = self.final_ada_w.data_ptr(), self.final_ada_b.data_ptr()
        fp8 = weights == "fp8"
        if fp8 and self.device.type != "cuda":
            raise ValueError("fp8 weights are quantized on the GPU")

        def proj(t):
            """(weight pointer, scale pointer or None) of one projection weight."""
            x = put(t, bf)
            if not fp8:
                return x.data_ptr(), None
            n, k = x.shape
            q = torch.empty(n, k, dtype=torch.uint8, device=dev)
            sc = torch.empty(n, dtype=torch.float32, device=dev)
            L.call("oasis_quantize_fp8_rows", L.ptr(x), n, k, L.ptr(q), L.ptr(sc), L.stream_handle())
            keep.pop()            # the bf16 copy is dropped once quantized
            keep.extend([q, sc])
            return q.data_ptr(), sc.data_ptr()

        S.weight_format = L.WEIGHTS_FP8 if fp8 else L.WEIGHTS_BF16
        for j in range(self.n_sub):
            p = "blocks.%d.%s." % (j // 2, "st"[j % 2])
            S.qkv_w[j], S.qkv_s[j] = proj(w[p + "qkv_w"])
            S.out_w[j], S.out_s[j] = proj(w[p + "out_w"])
            S.out_b[j] = put(w[p + "out_b"], torch.float32).data_ptr()
            S.fc1_w[j], S.fc1_s[j] = proj(w[p + "fc1_w"])
            S.fc1_b[j] = put(w[p + "fc1_b"], torch.float32).data_ptr()
            S.fc2_w[j], S.fc2_s[j] = proj(w[p + "fc2_w"])
            S.fc2_b[j] = put(w[p + "fc2_b"], torch.float32).data_ptr()
            for r in self.frag_roles:   # second copies: not in keep, so not in weight_bytes
                wf = tile_rows16(w[p + r + "_w"].to(device=dev, dtype=bf))
                frag_keep.append(wf)
                getattr(S, r + "_wf")[j] = wf.data_ptr()
        if fp8:
            torch.cuda.synchronize(dev)
        S.final_w = put(w["final.w"], f32).data_ptr()
        S.final_b = put(w["final.b"], f32).data_ptr()
        # patch embed: conv [D, C, 2, 2] -> [(p, q, c), D], W_rt (oasis_inference.py:1821-1826), stored
        # K-major so that the lanes computing consecutive outputs read consecutive weights
        cw = w["x_emb.w"]
        S.xemb_w = put(cw.float().permute(0, 2, 3, 1).reshape(d, -1).t().contiguous(), f32).data_ptr()
        S.xemb_b = put(w["x_emb.b"], f32).data_ptr()
        S.temb_w0 = put(w["t_emb.w0"], f32).data_ptr()
        S.temb_b0 = put(w["t_emb.b0"], f32).data_ptr()
        # the MLP's second linear and the action projection side by side: one GEMV multiplies
        # [hid | action] by [W2 | Wext] (action zero-padded to ext_pad inputs)
        cw2 = torch.zeros(d, d + self.ext_pad, dtype=f32)
        cw2[:, :d] = w["t_emb.w2"].float()
        cw2[:, d:d + self.ext_dim] = w["ext.w"].float()
        S.cond_w = put(cw2, f32).data_ptr()
        S.cond_b = put(w["t_emb.b2"].float() + w["ext.b"].float(), f32).data_ptr()
        sc, ss = rope_tables(_axial_angles(w["rope.spatial_freqs"].float(), *grid))
        tc, ts = rope_tables(temporal_angles(w["rope.temporal_freqs"].float(), t_max))
        self.s_cos, self.s_sinp = put(sc, torch.float32), put(ss, torch.float32)
        self.t_cos, self.t_sinp = put(tc, torch.float32), put(ts, torch.float32)
        S.s_cos, S.s_sinp = self.s_cos.data_ptr(), self.s_sinp.data_ptr()
        S.t_cos, S.t_sinp = self.t_cos.data_ptr(), self.t_sinp.data_ptr()
        S.t_max = t_max
        self.struct = S
        self._keep = keep
        self._frag_keep = frag_keep

    @property
    def weight_bytes(self):
        """Bytes of one copy of every weight (what a forward pass reads); the fragment-order
        second copies are frag_weight_bytes."""
        return sum(t.numel() * t.element_size() for t in self._keep)

    def frag_weight_bytes(self):
        return sum(t.numel() * t.element_size() for t in self._frag_keep)

    def ada_w_rows(self):
        """The stacked adaLN weights in row-major [n_sub*6D, D] order (a copy; the device keeps
        them in tile order)."""
        return untile_rows16(self.ada_w)

    def workspace(self, max_rows, max_cond=16, max_splits=None):
        return DiTWorkspace(self, max_rows, max_cond, max_splits)

    # -- building blocks ---------------------------------------------------------------
    def conditioning(self, t, actions, ws, stream=None):
        """ada rows [R, ada_width] for R frames: cond = MLP(temb(t)) + ext(action), then
        silu + every adaLN projection. t: [R] fp32, actions: [R, ext_dim] fp32 (device)."""
        R = t.shape[0]
        assert R <= ws.max_cond
        ws.t[:R].copy_(t.reshape(-1))
        ws.act[:R, :self.ext_dim].copy_(actions.reshape(R, -1))
        ws.act[:R, self.ext_dim:].zero_()
        self.conditioning_inplace(R, ws, stream)
        return ws.ada[:R]

    def conditioning_inplace(self, R, ws, stream=None):
        """Conditioning from ws.t[:R] / ws.act[:R] into ws.cond / ws.ada (no host work)."""
        L.call("oasis_dit_conditioning", ctypes.byref(self.struct), L.ptr(ws.t), L.ptr(ws.act), R,
               L.ptr(ws.hid), L.ptr(ws.cond), L.ptr(ws.ada), L.stream_handle(stream))

    def adaln_from_cond(self, cond, ws, stream=None):
        """ada rows from given (pre-SiLU) cond vectors [R, D] (the reference passes cond
        computed on the host, oasis_inference.py:1406-1427)."""
        R = cond.shape[0]
        ws.cond[:R].copy_(cond)
        return self.adaln_inplace(R, ws, stream)

    def adaln_inplace(self, R, ws, stream=None):
        """ada rows from the pre-SiLU cond rows already in ws.cond[:R] (nothing allocated)."""
        ns = self.n_sub * 6 * self.d
        h = L.stream_handle(stream)
        L.call("oasis_gemv_bf16_tiled", L.ptr(ws.cond), self.d, R, L.ptr(self.ada_w), ns, self.d,
               L.ptr(self.ada_b), L.ptr(ws.ada), self.ada_width, L.ACT_SILU, L.ACT_NONE, 0, h)
        L.call("oasis_gemv_f32", L.ptr(ws.cond), self.d, R, L.ptr(self.final_ada_w), 2 * self.d, self.d,
               L.ptr(self.final_ada_b), ctypes.c_void_p(ws.ada.data_ptr() + 4 * ns), self.ada_width, L.ACT_SILU,
               L.ACT_NONE, 0, h)
        return ws.ada[:R]

    def patch_embed(self, patches, out, stream=None):
        """out[M, D] = patches[M, 64] @ W_rt + b (patches in (p, q, c) column order)."""
        M = patches.shape[0]
        L.call("oasis_small_linear", L.ptr(patches), self.patch_dim, M, self.patch_dim,
               ctypes.c_void_p(self.struct.xemb_w), L.F32, 1, self.d, ctypes.c_void_p(self.struct.xemb_b),
               L.ptr(out), self.d, L.stream_handle(stream))

    def sub_blocks_inplace(self, ws, B, T, ada, ada_fstride, j0, j1, stream=None):
        """Sub-blocks [j0, j1) on ws.x[:B*T*P] in place (run_sub_block, oasis_inference.py:995)."""
        L.call("oasis_dit_sub_blocks", ctypes.byref(self.struct), ctypes.byref(ws.struct), B, T,
               L.ptr(ada), ada_fstride, j0, j1, L.stream_handle(stream))

    def precompute_past(self, ws, kv, B, ada, ada_fstride, stream=None):
        """K/V-cache past pass on ws.x[:B*P] (precompute_past_state, oasis_inference.py:1354)."""
        L.call("oasis_dit_precompute_past", ctypes.byref(self.struct), ctypes.byref(ws.struct),
               ctypes.byref(kv.struct), B, L.ptr(ada), ada_fstride, L.stream_handle(stream))

    def forward_current(self, ws, kv, B, ada, ada_fstride, v_out, stream=None):
        """K/V-cache current-frame pass on ws.x[:B*P] (dit_forward_currentonly,
        oasis_inference.py:1372)."""
        L.call("oasis_dit_forward_current", ctypes.byref(self.struct), ctypes.byref(ws.struct),
               ctypes.byref(kv.struct), B, L.ptr(ada), ada_fstride, L.ptr(v_out), L.stream_handle(stream))

    def forward_inplace(self, ws, B, T, ada, ada_fstride, v_out, stream=None):
        """Blocks + final layer on ws.x[:B*T*P] (in place); v_out [B*T*P, 64] fp32."""
        L.call("oasis_dit_forward", ctypes.byref(self.struct), ctypes.byref(ws.struct), B, T,
               L.ptr(ada), ada_fstride, L.ptr(v_out), L.stream_handle(stream))


class KVCache:
    """The context frame's rotated temporal K/V for every temporal sub-block, for up to
    max_streams streams: k, v bf16 [n_sub/2, max_streams, P, H, 2, 64] (slot 0 context,
    slot 1 current frame; the t1_past_k/v scratches of oasis_inference.py:1218-1352)."""

    def __init__(self, dit, max_streams=1):
        shape = (dit.n_sub // 2, max_streams, dit.P, dit.n_heads, 2, HEAD_DIM)
        self.k = torch.zeros(shape, device=dit.device, dtype=torch.bfloat16)
        self.v = torch.zeros(shape, device=dit.device, dtype=torch.bfloat16)
        self.max_streams = max_streams
        self.struct = L.KVCache(k=self.k.data_ptr(), v=self.v.data_ptr(), max_streams=max_streams)


class DiTWorkspace:
    """Activation buffers for up to max_rows tokens and max_cond conditioning rows."""

    def __init__(self, dit, max_rows, max_cond=16, max_splits=None):
        dev, d, bf = dit.device, dit.d, torch.bfloat16
        # split-K slices for the O / FC2 projections; small token counts need more splits
        if max_splits is None:
            max_splits = 8 if max_rows <= 640 else 2
        self.max_rows, self.max_cond = max_rows, max_cond
        # h, attn and mlp hold the rows a fragment-order pass rounds up to (dit.frag)
        fr = max(max_rows, frag_rows(min(max_rows, 320))) if dit.frag else max_rows
        self.x = torch.zeros(max_rows, d, device=dev)
        self.h = torch.zeros(fr, d, device=dev, dtype=bf)
        self.q = torch.zeros(max_rows, d, device=dev, dtype=bf)
        self.k = torch.zeros(max_rows, d, device=dev, dtype=bf)
        self.v = torch.zeros(max_rows, d, device=dev, dtype=bf)
        self.attn = torch.zeros(fr, d, device=dev, dtype=bf)
        self.mlp = torch.zeros(fr, dit.d_mlp, device=dev, dtype=bf)
        self.max_splits = max_splits
        self.partial = torch.zeros(max_splits, max_rows, d, device=dev)
        self.v_out = torch.zeros(max_rows, dit.patch_dim, device=dev)
        self.t = torch.zeros(max_cond, device=dev)
        self.act = torch.zeros(max_cond, dit.ext_pad, device=dev)
        self.hid = torch.zeros(max_cond, d, device=dev)
        self.cond = torch.zeros(max_cond, d, device=dev)
        self.ada = torch.zeros(max_cond, dit.ada_width, device=dev)
        S = L.DiTBuffers()
        S.max_rows = max_rows
        for name in ("x", "h", "q", "k", "v", "attn", "mlp", "partial"):
            setattr(S, name, getattr(self, name).data_ptr())
        S.max_splits = max_splits
        S.frag_rows = fr if dit.frag else 0
        if "fc1" in dit.frag_roles:   # the LayerNorm after O carried into FC1: row means and statistics
            self.ln_mean = torch.zeros(max_rows, device=dev)
            self.ln_stats = torch.zeros(max_rows, d // 16, 2, device=dev)
            self.ln_mod = torch.zeros(16, d, device=dev, dtype=bf)
            S.ln_mean, S.ln_stats, S.ln_mod = self.ln_mean.data_ptr(), self.ln_stats.data_ptr(), self.ln_mod.data_ptr()
        if dit.weights == "fp8":  # fp8 activation blocks: e4m3 bytes + one e8m0 scale per 32 columns
            u8 = torch.uint8
            self.act8 = torch.zeros(max_rows, d, device=dev, dtype=u8)
            self.act8_scale = torch.zeros(max_rows, d // 32, device=dev, dtype=u8)
            self.mlp8 = torch.zeros(max_rows, dit.d_mlp, device=dev, dtype=u8)
            self.mlp8_scale = torch.zeros(max_rows, dit.d_mlp // 32, device=dev, dtype=u8)
            for name in ("act8", "act8_scale", "mlp8", "mlp8_scale"):
                setattr(S, name, getattr(self, name).data_ptr())
        self.struct = S


class VAE:
    """ViT VAE decoder weights resident on one GPU."""

    def __init__(self, vw, device="cuda", grid=(18, 32), patch=20):
        dev = self.device = torch.device(device)
        self.d = d = vw["pq_w"].shape[0]
        self.n_heads = d // HEAD_DIM
        self.depth = _count(vw, "dec.%d.qkv_w")
        assert 0 < self.depth <= L.MAX_SUB
        self.d_mlp = vw["dec.0.fc1_w"].shape[0]
        self.latent_dim = vw["pq_w"].shape[1]
        self.grid, self.patch = grid, patch
        self.L = grid[0] * grid[1]
        bf, f32 = torch.bfloat16, torch.float32
        keep = []

        def put(t, dtype):
            x = t.to(device=dev, dtype=dtype).contiguous()
            keep.append(x)
            return x.data_ptr()

        S = L.VAEWeights()
        S.depth, S.d_model, S.n_heads, S.d_mlp = self.depth, d, self.n_heads, self.d_mlp
        S.latent_dim, S.grid_h, S.grid_w, S.patch = self.latent_dim, grid[0], grid[1], patch
        S.pq_w, S.pq_b = put(vw["pq_w"], bf), put(vw["pq_b"], f32)
        for i in range(self.depth):
            p = "dec.%d." % i
            S.n1_w[i], S.n1_b[i] = put(vw[p + "n1_w"], f32), put(vw[p + "n1_b"], f32)
            S.qkv_w[i], S.qkv_b[i] = put(vw[p + "qkv_w"], bf), put(vw[p + "qkv_b"], f32)
            S.proj_w[i], S.proj_b[i] = put(vw[p + "proj_w"], bf), put(vw[p + "proj_b"], f32)
            S.n2_w[i], S.n2_b[i] = put(vw[p + "n2_w"], f32), put(vw[p + "n2_b"], f32)
            S.fc1_w[i], S.fc1_b[i] = put(vw[p + "fc1_w"], bf), put(vw[p + "fc1_b"], f32)
            S.fc2_w[i], S.fc2_b[i] = put(vw[p + "fc2_w"], bf), put(vw[p + "fc2_b"], f32)
        S.norm_w, S.norm_b = put(vw["norm_w"], f32), put(vw["norm_b"], f32)
        S.pred_w, S.pred_b = put(vw["pred_w"], bf), put(vw["pred_b"], f32)
        # the angle table as given (the upstream model's rotary_freqs buffer, oasis_inference.py:
        # 455-468), else the axial construction from frequencies (synthetic weights)
        if "rope.vae_angles" in vw:
            ang = vw["rope.vae_angles"].double().reshape(self.L, -1)
        else:
            ang = _axial_angles(vw["rope.vae_freqs"].float(), *grid)
        c, s = rope_tables(ang)
        S.rope_cos, S.rope_sinp = put(c, f32), put(s, f32)
        self.struct = S
        self._keep = keep
        self.frame_shape = (3, grid[0] * patch, grid[1] * patch)
        self.patch_dim = 3 * patch * patch

    @property
    def weight_bytes(self):
        return sum(t.numel() * t.element_size() for t in self._keep)

    def workspace(self, max_frames=1):
        return VAEWorkspace(self, max_frames)

    def decode_inplace(self, latent, frame, ws, stream=None):
        L.call("oasis_vae_decode", ctypes.byref(self.struct), ctypes.byref(ws.struct),
               L.ptr(latent), L.ptr(frame), L.stream_handle(stream))

    def decode_batch(self, latents, frames, ws, stream=None):
        """B latents [B, L, latent_dim] -> frames [B, 3, H, W] in one pass of B*L tokens."""
        B = latents.shape[0]
        L.call("oasis_vae_decode_batch", ctypes.byref(self.struct), ctypes.byref(ws.struct), B,
               L.ptr(latents), L.ptr(frames), L.stream_handle(stream))

    def decode_patches(self, latents, pred_out, ws, stream=None):
        """B latents [B*L, latent_dim] -> the predictor's unclamped rows pred_out [B*L, ld]
        (ld >= patch_dim; vae_decode_forward's pred_out, oasis_inference.py:1546-1618)."""
        rows = latents.numel() // self.latent_dim
        if rows % self.L or pred_out.shape[0] < rows or pred_out.shape[-1] < self.patch_dim:
            raise L.OasisError("vae_decode_patches", -2, "latents of %d rows / pred_out %s do not fit L=%d, "
                               "patch_dim=%d" % (rows, tuple(pred_out.shape), self.L, self.patch_dim))
        L.call("oasis_vae_decode_patches", ctypes.byref(self.struct), ctypes.byref(ws.struct), rows // self.L,
               L.ptr(latents), L.ptr(pred_out), pred_out.stride(0), L.stream_handle(stream))


class VAEWorkspace:
    """Activation buffers for up to max_frames latents decoded together (max_frames * L rows)."""

    def __init__(self, vae, max_frames=1):
        dev, d, bf = vae.device, vae.d, torch.bfloat16
        n = vae.L * max_frames
        self.max_frames = max_frames
        self.x = torch.zeros(n, d, device=dev)
        self.h = torch.zeros(n, d, device=dev, dtype=bf)
        self.q = torch.zeros(n, d, device=dev, dtype=bf)
        self.k = torch.zeros(n, d, device=dev, dtype=bf)
        self.v = torch.zeros(n, d, device=dev, dtype=bf)
        self.attn = torch.zeros(n, d, device=dev, dtype=bf)
        self.mlp = torch.zeros(n, vae.d_mlp, device=dev, dtype=bf)
        self.max_splits = 4
        self.partial = torch.zeros(self.max_splits, n, d, device=dev)
        self.latent = torch.zeros(n, vae.latent_dim, device=dev)
        self.frame = torch.zeros(*vae.frame_shape, device=dev)
        # the predictor's rows as the reference keeps them (pred_out, TILE-padded columns that
        # stay zero: 1200 -> 1216), for the reference-named vae_decode_forward
        self.pred_out = torch.zeros(vae.L, -(-vae.patch_dim // 32) * 32, device=dev)
        S = L.VAEBuffers()
        S.max_rows = n
        for name in ("x", "h", "q", "k", "v", "attn", "mlp", "partial"):
            setattr(S, name, getattr(self, name).data_ptr())
        S.max_splits = self.max_splits
        self.struct = S


class Graph:
    """A hipGraph captured from a sequence of liboasis_hip calls on one stream
    (ttnn begin/end_trace_capture + execute_trace, oasis_inference.py:2133-2146,2224)."""

    def __init__(self, fn, stream):
        self.stream = stream
        self.exec = ctypes.c_void_p()
        torch.cuda.synchronize()
        h = L.stream_handle(stream)
        L.call("oasis_graph_begin", h)
        try:
            fn()
        except BaseException:
            g = ctypes.c_void_p()
            L.lib().oasis_graph_end(h, ctypes.byref(g))
            if g.value:
                L.lib().oasis_graph_destroy(g)
            raise
        L.call("oasis_graph_end", h, ctypes.byref(self.exec))

    def launch(self):
        L.call("oasis_graph_launch", self.exec, L.stream_handle(self.stream))

    def __del__(self):
        # at interpreter exit the module globals may already be gone; the process teardown
        # releases the graph then
        if L is None or getattr(self, "exec", None) is None or not self.exec.value:
            return
        L.lib().oasis_graph_destroy(self.exec)
        self.exec = None


class DiTStep:
    """One full DiT denoising step for B streams of T frames, on fixed device buffers:
    conditioning (timestep MLP + action projection + every adaLN projection), patch embed
    of the patch-space latent, 16 x (spatial, temporal) sub-blocks and the final layer.
    Inputs: self.patches [B*T*P, 64], self.ws.t [B*T], self.ws.act [B*T, :25]."""

    def __init__(self, dit, B=1, T=2, stream=None):
        self.dit, self.B, self.T = dit, B, T
        self.M = B * T * dit.P
        self.ws = dit.workspace(self.M, max_cond=max(16, B * T))
        self.patches = torch.zeros(self.M, dit.patch_dim, device=dit.device)
        self.stream = stream if stream is not None else torch.cuda.Stream(device=dit.device)
        # the buffers were zero-filled on the allocating stream: work on self.stream follows that
        self.stream.wait_stream(torch.cuda.current_stream(dit.device))
        self.graph = None

    def set_inputs(self, patches, t, actions):
        R = self.B * self.T
        self.patches.copy_(patches.reshape(self.M, -1))
        self.ws.t[:R].copy_(t.reshape(-1))
        self.ws.act[:R].zero_()
        self.ws.act[:R, :self.dit.ext_dim].copy_(actions.reshape(R, -1))
        torch.cuda.synchronize(self.dit.device)

    def enqueue(self):
        d, ws = self.dit, self.ws
        L.call("oasis_dit_step", ctypes.byref(d.struct), ctypes.byref(ws.struct), self.B, self.T, L.ptr(ws.t),
               L.ptr(ws.act), L.ptr(self.patches), L.ptr(ws.hid), L.ptr(ws.cond), L.ptr(ws.ada),
               L.ptr(ws.v_out), L.stream_handle(self.stream))

    def capture(self):
        self.graph = Graph(self.enqueue, self.stream)
        return self.graph

    def run(self):
        """Enqueue one step on self.stream; the caller's current stream waits for it."""
        if self.graph is not None:
            self.graph.launch()
        else:
            self.enqueue()
        torch.cuda.current_stream(self.dit.device).wait_stream(self.stream)
        return self.ws.v_out[:self.M]


class FramePipeline:
    """One generated frame (reference traced frame, oasis_inference.py:2131-2148):
    conditioning for the context row and the n_steps generated rows, context patch
    embed, n_steps DDIM v-prediction steps, bridge, VAE decode and unpatchify. With
    kv_cache (the default, as the reference's OASIS_KV=1) the first step runs at T=2 and
    stores the context frame's temporal K/V; the later steps run the generated frame alone
    at T=1 against that cache. kv_cache=False runs every step at T=2.
    Inputs: self.chunk [P, 64] noise (patch space), self.ctx_patches [P, 64],
    self.ws.t / self.ws.act rows [0] context and [1+i] generated frame at step i.
    run() denoises self.chunk in place: the next frame needs new noise in self.chunk and its
    context in self.ctx_patches first (set_inputs, or PlaySession, which does both on the
    device)."""

    def __init__(self, dit, vae, steps, alphas_cumprod, stream=None, kv_cache=True):
        from .schedule import ddim_coefficients
        self.dit, self.vae = dit, vae
        # steps after the first run the generated frame alone against the context's cached K/V
        self.kv = KVCache(dit, 1) if kv_cache else None
        self.steps = list(steps)
        self.n = len(self.steps)
        P, dev = dit.P, dit.device
        self.ws = dit.workspace(2 * P, max_cond=max(16, 1 + self.n))
        self.vws = vae.workspace()
        self.chunk = torch.zeros(P, dit.patch_dim, device=dev)
        self.ctx_patches = torch.zeros(P, dit.patch_dim, device=dev)
        self.ctx_z = torch.zeros(P, dit.d, device=dev)
        self.coeffs = (ctypes.c_float * (6 * self.n))(*ddim_coefficients(alphas_cumprod, self.steps))
        self.stream = stream if stream is not None else torch.cuda.Stream(device=dev)
        # the buffers were zero-filled on the allocating stream: work on self.stream follows that
        self.stream.wait_stream(torch.cuda.current_stream(dev))
        self.graph = None

    def set_inputs(self, noise_patches, ctx_patches, ctx_t, ctx_action, gen_action):
        R = 1 + self.n
        self.chunk.copy_(noise_patches)
        self.ctx_patches.copy_(ctx_patches)
        t = torch.tensor([float(ctx_t)] + [float(t) for t, _ in self.steps])
        self.ws.t[:R].copy_(t)
        self.ws.act[:R].zero_()
        e = self.dit.ext_dim
        self.ws.act[0, :e].copy_(ctx_action)
        self.ws.act[1:R, :e].copy_(gen_action.reshape(1, -1).expand(self.n, -1))
        torch.cuda.synchronize(self.dit.device)

    def enqueue(self):
        d, ws = self.dit, self.ws
        L.call("oasis_ddim_frame", ctypes.byref(d.struct), ctypes.byref(ws.struct),
               ctypes.byref(self.vae.struct), ctypes.byref(self.vws.struct),
               ctypes.byref(self.kv.struct) if self.kv is not None else None, L.ptr(self.chunk),
               L.ptr(self.ctx_patches), L.ptr(ws.t), L.ptr(ws.act), self.n,
               ctypes.cast(self.coeffs, ctypes.c_void_p), L.ptr(ws.hid), L.ptr(ws.cond),
               L.ptr(ws.ada), L.ptr(self.ctx_z), L.ptr(ws.v_out), L.ptr(self.vws.latent), L.ptr(self.vws.frame),
               L.stream_handle(self.stream))

    def capture(self):
        self.graph = Graph(self.enqueue, self.stream)
        return self.graph

    def run(self):
        """Enqueue one frame on self.stream; the caller's current stream waits for it."""
        if self.graph is not None:
            self.graph.launch()
        else:
            self.enqueue()
        torch.cuda.current_stream(self.dit.device).wait_stream(self.stream)
        return self.vws.frame


class VideoPipeline:
    """n_frames consecutive frames of one stream per batch (oasis_video_frames): frame f's
    context is frame f-1's denoised latent, rolled on the device (the interactive loop's
    context window, oasis_inference.py:2296-2306).

    overlap_decode=False: one hipGraph per batch, the frames' DDIM steps, then their VAE decodes
    as one batched decode of the n_frames latents.
    overlap_decode=True: the batch's DDIM steps (oasis_video_frames with frames = NULL) and its
    batched decodes (oasis_video_decode) are two single-stream graphs on two streams, and batch k's
    decodes run while batch k+1 denoises. launch() enqueues batch k, then waits on the host
    for batch k-1's DDIM steps (batch k is already queued behind them) and launches its
    decodes: a device-side wait of one stream on the other's event serialises the two graphs
    on this runtime, a host-side wait does not. drain() launches the last batch's decodes.
    Chunk and frame buffers alternate between two sets, so a batch's frames stay valid until
    two batches later.

    Inputs: self.chunks [n_frames, P, 64] noise, self.ctx_patches [P, 64] the first context,
    conditioning rows built by set_inputs (context t and action, then each step's t with
    the frame's action; the context of frame f > 0 carries frame f-1's action).

    Each launch denoises the chunk buffers in place and starts from self.ctx_patches; it does
    not draw new noise or carry the context over from the previous batch. A continuing video
    calls set_inputs before every batch with fresh noise and, as ctx_patches, the previous
    batch's last latent (self.chunks[-1] once that batch is done). Launches without it re-run
    the same batch on the previous outputs (what a timing loop does)."""

    def __init__(self, dit, vae, steps, alphas_cumprod, n_frames, stream=None, kv_cache=True, overlap_decode=False):
        from .schedule import ddim_coefficients
        self.dit, self.vae, self.n_frames = dit, vae, n_frames
        self.overlap_decode = overlap_decode
        self.steps = list(steps)
        self.n = len(self.steps)
        P, dev = dit.P, dit.device
        R = n_frames * (1 + self.n)
        self.ws = dit.workspace(2 * P, max_cond=max(16, R))
        # the decodes of a batch run batched: the VAE workspace holds all n_frames latents
        self.vws = vae.workspace(max_frames=n_frames)
        # oasis_video_frames / oasis_video_decode write as many latents into the latent scratch as
        # the VAE workspace's rows hold (max_rows / L); the scratch must have that many rows
        assert self.vws.latent.shape[0] >= self.vws.struct.max_rows, "latent scratch below the VAE workspace"
        self.kv = KVCache(dit, 1) if kv_cache else None
        nb = 2 if overlap_decode else 1
        self.chunk_bufs = [torch.zeros(n_frames, P, dit.patch_dim, device=dev) for _ in range(nb)]
        self.frame_bufs = [torch.zeros(n_frames, *vae.frame_shape, device=dev) for _ in range(nb)]
        self.ctx_patches = torch.zeros(P, dit.patch_dim, device=dev)
        self.ctx_z = torch.zeros(P, dit.d, device=dev)
        self.coeffs = (ctypes.c_float * (6 * self.n))(*ddim_coefficients(alphas_cumprod, self.steps))
        self.stream = stream if stream is not None else torch.cuda.Stream(device=dev)
        self.decode_stream = torch.cuda.Stream(device=dev) if overlap_decode else None
        # the buffers were zero-filled on the allocating stream: work on the others follows that
        for st in (self.stream, self.decode_stream):
            if st is not None:
                st.wait_stream(torch.cuda.current_stream(dev))
        self.graph = None
        self.graphs, self.decode_graphs = [], []
        self._ev_dit = [torch.cuda.Event() for _ in range(nb)]
        self._ev_dec = [torch.cuda.Event() for _ in range(nb)]
        self._pending = [False] * nb  # decodes launched that read buffer set b
        self._undecoded = None        # buffer set of the batch whose decodes are still to launch
        self._k = 0
        self._last = 0

    @property
    def chunks(self):
        """Denoised latents of the last batch (noise before the first)."""
        return self.chunk_bufs[self._last]

    @property
    def frames(self):
        return self.frame_bufs[self._last]

    def set_inputs(self, noise_patches, ctx_patches, ctx_t, ctx_action, actions):
        """noise_patches [n_frames, P, 64], ctx_patches [P, 64], actions [n_frames, ext_dim]."""
        F, n, e = self.n_frames, self.n, self.dit.ext_dim
        torch.cuda.synchronize(self.dit.device)  # no batch still reads or writes the buffers
        for c in self.chunk_bufs:
            c.copy_(noise_patches.reshape(c.shape))
        self.ctx_patches.copy_(ctx_patches)
        t = torch.tensor(([float(ctx_t)] + [float(ts) for ts, _ in self.steps]) * F)
        act = torch.zeros(F, 1 + n, self.dit.ext_pad)
        acts = actions.detach().float().cpu().reshape(F, e)
        act[0, 0, :e] = ctx_action.detach().float().cpu()
        act[1:, 0, :e] = acts[:-1]
        act[:, 1:, :e] = acts[:, None, :]
        self.ws.t[:F * (1 + n)].copy_(t)
        self.ws.act[:F * (1 + n)].copy_(act.reshape(F * (1 + n), -1))
        torch.cuda.synchronize(self.dit.device)

    def _enqueue_frames(self, b, decode):
        d, ws = self.dit, self.ws
        L.call("oasis_video_frames", ctypes.byref(d.struct), ctypes.byref(ws.struct), ctypes.byref(self.vae.struct),
               ctypes.byref(self.vws.struct) if decode else None,
               ctypes.byref(self.kv.struct) if self.kv is not None else None,
               self.n_frames, L.ptr(self.chunk_bufs[b]), L.ptr(self.ctx_patches), L.ptr(ws.t), L.ptr(ws.act), self.n,
               ctypes.cast(self.coeffs, ctypes.c_void_p), L.ptr(ws.hid), L.ptr(ws.cond),
               L.ptr(ws.ada), L.ptr(self.ctx_z), L.ptr(ws.v_out), L.ptr(self.vws.latent) if decode else None,
               L.ptr(self.frame_bufs[b]) if decode else None, L.stream_handle(self.stream))

    def _enqueue_decode(self, b):
        L.call("oasis_video_decode", ctypes.byref(self.dit.struct), ctypes.byref(self.vae.struct),
               ctypes.byref(self.vws.struct), self.n_frames, L.ptr(self.chunk_bufs[b]), L.ptr(self.vws.latent),
               L.ptr(self.frame_bufs[b]), L.stream_handle(self.decode_stream))

    def enqueue(self):
        """One batch, uncaptured (overlap_decode=False)."""
        self._enqueue_frames(0, True)

    def capture(self):
        if not self.overlap_decode:
            self.graph = Graph(self.enqueue, self.stream)
            self.graphs = [self.graph]
            return self.graph
        self.graphs = [Graph(lambda b=b: self._enqueue_frames(b, False), self.stream) for b in range(2)]
        self.decode_graphs = [Graph(lambda b=b: self._enqueue_decode(b), self.decode_stream) for b in range(2)]
        return self.graphs

    def launch(self):
        """Enqueue one batch and return its frame buffer. With overlap_decode the frames are
        complete once the next launch() or drain() has launched their decodes and the decode
        stream has run them."""
        if not self.overlap_decode:
            if self.graph is not None:
                self.graph.launch()
            else:
                self.enqueue()
            return self.frame_bufs[0]
        b = self._k % 2
        self._k += 1
        if self._pending[b]:  # the decodes that read chunk set b (two batches ago) are done
            self._ev_dec[b].synchronize()
            self._pending[b] = False
        if self.graphs:
            self.graphs[b].launch()
        else:
            self._enqueue_frames(b, False)
        self._ev_dit[b].record(self.stream)
        self.drain()
        self._undecoded = b
        self._last = b
        return self.frame_bufs[b]

    def drain(self):
        """Launch the decodes still owed (those of the last launched batch), once that batch's
        DDIM steps have finished; the decode stream runs them."""
        pb = self._undecoded
        if pb is None:
            return
        self._ev_dit[pb].synchronize()
        if self.decode_graphs:
            self.decode_graphs[pb].launch()
        else:
            self._enqueue_decode(pb)
        self._ev_dec[pb].record(self.decode_stream)
        self._pending[pb] = True
        self._undecoded = None

    def run(self):
        """Enqueue one batch and its decodes; the caller's current stream waits for its frames."""
        frames = self.launch()
        self.drain()
        cur = torch.cuda.current_stream(self.dit.device)
        cur.wait_stream(self.stream)
        if self.decode_stream is not None:
            cur.wait_stream(self.decode_stream)
        return frames


def attention_scale(head_dim=HEAD_DIM):
    return 1.0 / math.sqrt(head_dim)
