"""Seeded synthetic weights and inputs for the benchmark configurations.

There is no checkpoint offline, so every configuration draws its inputs and then its
weights from one CPU ``torch.Generator`` seeded with the configuration seed, in a
fixed order: inputs first, then the weights layer by layer in forward order. Weights
are N(0, 0.02) rounded to bf16 (the model's storage type), biases are zero, LayerNorm
affines are (1, 0). RoPE frequencies are the theta=10000 ladders (the reference loads
learned ones from the checkpoint, oasis_inference.py:630-631).

Weight dict keys follow the model's nn.Linear layout ``[out, in]``:
  t_emb.w0 [D,256] t_emb.b0  t_emb.w2 [D,D] t_emb.b2  ext.w [D,25] ext.b
  x_emb.w [D,16,2,2] x_emb.b
  blocks.{i}.{s|t}.{ada_w [6D,D], ada_b, qkv_w [3D,D], out_w, out_b, fc1_w [Dm,D], fc1_b,
                    fc2_w [D,Dm], fc2_b}
  final.ada_w [2D,D] final.ada_b final.w [64,D] final.b
  rope.spatial_freqs [d/4] rope.temporal_freqs [d/2]
VAE: pq_w [D,32] pq_b dec.{i}.{n1_w,n1_b,qkv_w,qkv_b,proj_w,proj_b,n2_w,n2_b,fc1_w,fc1_b,
     fc2_w,fc2_b} norm_w norm_b pred_w [1200,D] pred_b rope.vae_freqs [d/8]
"""
import torch

WEIGHT_STD = 0.02


def theta_freqs(n, dim, theta=10000.0):
    """``theta^(-2k/dim)`` for k < n."""
    return theta ** (-2.0 * torch.arange(n, dtype=torch.float64) / dim).float()


class Draw:
    """Seeded draws in a fixed order."""

    def __init__(self, seed):
        self.g = torch.Generator().manual_seed(seed)

    def normal(self, *shape, std=1.0):
        return torch.randn(*shape, generator=self.g) * std

    def weight(self, *shape, dtype=torch.bfloat16):
        return (torch.randn(*shape, generator=self.g) * WEIGHT_STD).to(dtype)

    def randint(self, lo, hi, shape):
        return torch.randint(lo, hi, shape, generator=self.g)


def sub_block_weights(dr, d=1024, d_mlp=4096, dtype=torch.bfloat16):
    z = lambda n: torch.zeros(n, dtype=dtype)  # noqa: E731
    return {
        "ada_w": dr.weight(6 * d, d, dtype=dtype), "ada_b": z(6 * d),
        "qkv_w": dr.weight(3 * d, d, dtype=dtype),
        "out_w": dr.weight(d, d, dtype=dtype), "out_b": z(d),
        "fc1_w": dr.weight(d_mlp, d, dtype=dtype), "fc1_b": z(d_mlp),
        "fc2_w": dr.weight(d, d_mlp, dtype=dtype), "fc2_b": z(d),
    }


def dit_weights(dr, n_blocks=16, d=1024, n_heads=16, d_mlp=4096, in_ch=16, patch=2, freq_dim=256,
                ext_dim=25, dtype=torch.bfloat16):
    """All DiT weights, drawn in forward order."""
    hd = d // n_heads
    z = lambda n: torch.zeros(n, dtype=dtype)  # noqa: E731
    w = {
        "t_emb.w0": dr.weight(d, freq_dim, dtype=dtype), "t_emb.b0": z(d),
        "t_emb.w2": dr.weight(d, d, dtype=dtype), "t_emb.b2": z(d),
        "ext.w": dr.weight(d, ext_dim, dtype=dtype), "ext.b": z(d),
        "x_emb.w": dr.weight(d, in_ch, patch, patch, dtype=dtype), "x_emb.b": z(d),
    }
    for i in range(n_blocks):
        for kind in ("s", "t"):
            for k, v in sub_block_weights(dr, d, d_mlp, dtype).items():
                w["blocks.%d.%s.%s" % (i, kind, k)] = v
    w["final.ada_w"] = dr.weight(2 * d, d, dtype=dtype)
    w["final.ada_b"] = z(2 * d)
    w["final.w"] = dr.weight(patch * patch * in_ch, d, dtype=dtype)
    w["final.b"] = z(patch * patch * in_ch)
    w["rope.spatial_freqs"] = theta_freqs(hd // 4, hd // 2)
    w["rope.temporal_freqs"] = theta_freqs(hd // 2, hd)
    return w


def vae_weights(dr, depth=12, d=1024, n_heads=16, d_mlp=4096, latent_dim=32, patch=20,
                dtype=torch.bfloat16):
    """ViT VAE decoder weights, drawn in forward order."""
    hd = d // n_heads
    z = lambda n: torch.zeros(n, dtype=dtype)  # noqa: E731
    o = lambda n: torch.ones(n, dtype=dtype)  # noqa: E731
    w = {"pq_w": dr.weight(d, latent_dim, dtype=dtype), "pq_b": z(d)}
    for i in range(depth):
        p = "dec.%d." % i
        w[p + "n1_w"], w[p + "n1_b"] = o(d), z(d)
        w[p + "qkv_w"], w[p + "qkv_b"] = dr.weight(3 * d, d, dtype=dtype), z(3 * d)
        w[p + "proj_w"], w[p + "proj_b"] = dr.weight(d, d, dtype=dtype), z(d)
        w[p + "n2_w"], w[p + "n2_b"] = o(d), z(d)
        w[p + "fc1_w"], w[p + "fc1_b"] = dr.weight(d_mlp, d, dtype=dtype), z(d_mlp)
        w[p + "fc2_w"], w[p + "fc2_b"] = dr.weight(d, d_mlp, dtype=dtype), z(d)
    w["norm_w"], w["norm_b"] = o(d), z(d)
    w["pred_w"] = dr.weight(3 * patch * patch, d, dtype=dtype)
    w["pred_b"] = z(3 * patch * patch)
    w["rope.vae_freqs"] = theta_freqs(hd // 8, hd // 4)
    return w


def one_hot_actions(dr, n, dim=25):
    idx = dr.randint(0, dim, (n,))
    a = torch.zeros(n, dim)
    a[torch.arange(n), idx] = 1.0
    return a


# ---------------------------------------------------------------------------
# configurations (the benchmark plan's configs 0..4)
# ---------------------------------------------------------------------------

def config0(seed=0, dtype=torch.float32):
    """One spatial sub-block, x [1,2,144,1024], cond [1,2,1024], fp32 weights."""
    dr = Draw(seed)
    x = dr.normal(1, 2, 144, 1024)
    cond = dr.normal(1, 2, 1024)
    w = sub_block_weights(dr, dtype=dtype)
    return {"x": x, "cond": cond, "w": w,
            "spatial_freqs": theta_freqs(16, 32), "temporal_freqs": theta_freqs(32, 64)}


def config1(seed=1, T=2, n_blocks=16, d=1024, n_heads=16, d_mlp=4096):
    """Full DiT step: latent [1,T,16,18,32], t ~ U[0,1000) per frame, one-hot actions."""
    dr = Draw(seed)
    latent = dr.normal(1, T, 16, 18, 32)
    t = dr.randint(0, 1000, (T,)).float()
    actions = one_hot_actions(dr, T)
    w = dit_weights(dr, n_blocks=n_blocks, d=d, n_heads=n_heads, d_mlp=d_mlp)
    return {"latent": latent, "t": t, "actions": actions, "w": w}


def config2(seed=2, T=32, d=1024, n_heads=16, d_mlp=4096):
    """Temporal stress: x [1,T,144,1024], cond [1,T,1024], one temporal sub-block."""
    dr = Draw(seed)
    x = dr.normal(1, T, 144, d)
    cond = dr.normal(1, T, d)
    w = sub_block_weights(dr, d, d_mlp)
    return {"x": x, "cond": cond, "w": w, "temporal_freqs": theta_freqs(d // n_heads // 2, d // n_heads)}


def config3(seed=3, n_blocks=16, vae_depth=12):
    """DDIM frame: x_T, context latent, actions, VAE latent, DiT + VAE weights."""
    dr = Draw(seed)
    x_T = dr.normal(1, 16, 18, 32).clamp(-20, 20)
    ctx_latent = dr.normal(1, 16, 18, 32)
    gen_action = one_hot_actions(dr, 1)[0]
    vae_latent = dr.normal(576, 32)
    w = dit_weights(dr, n_blocks=n_blocks)
    vw = vae_weights(dr, depth=vae_depth)
    return {"x_T": x_T, "ctx_latent": ctx_latent, "ctx_t": 14.0, "ctx_action": torch.zeros(25),
            "gen_action": gen_action, "vae_latent": vae_latent, "w": w, "vw": vw,
            "steps": [(999, 749), (749, 499), (499, 249), (249, -1)]}


def config4(seed=4, B=8, T=4, n_blocks=16, d=1024, n_heads=16, d_mlp=4096):
    """Batched serving: B independent streams of T frames, latent [B,T,16,18,32], t per
    frame ~ U[0,1000), one-hot actions; the weights are quantized to e4m3 by the model."""
    dr = Draw(seed)
    latent = dr.normal(B, T, 16, 18, 32)
    t = dr.randint(0, 1000, (B, T)).float()
    actions = one_hot_actions(dr, B * T).reshape(B, T, -1)
    w = dit_weights(dr, n_blocks=n_blocks, d=d, n_heads=n_heads, d_mlp=d_mlp)
    return {"latent": latent, "t": t, "actions": actions, "w": w}
