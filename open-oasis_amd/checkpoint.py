"""Weights from the upstream Oasis checkpoints: the DiT (keys blocks.*, t_embedder.*, ...) and
the ViT VAE (keys encoder.*, decoder.*, ...), read from safetensors files (nothing in the file is
executed) and renamed into this package's weight dicts. This follows the reference's
preload_dit_weights and preload_vae_decoder_weights (oasis_inference.py:505-677,679-760), and
its file discovery by key prefix (_find_weights_by_prefix, oasis_inference.py:485-503).

Tensors keep their checkpoint layout: linear weights [out, in], the patch-embed conv
[D, C, 2, 2]. DiT / VAE fold the adaLN +1 and convert dtypes when they place them on the device.
The VAE decoder's RoPE angles are not in its checkpoint: the reference reads them from the
upstream model's non-persistent ``rotary_freqs`` buffer, an (18, 32, 32) table of per-pixel angles
for the first 32 dims of each head (precompute_vae_rope, oasis_inference.py:455-468), which the
upstream vae.py computes and which is not available here. load_vae_decoder therefore takes that
table as a required input (``rope_angles``); nothing fills in a guess. Its values are parity
unpinned: no fixture of the reference holds them.
"""
import os

from safetensors import safe_open

import torch

DIT_PREFIX = "blocks."       # find_dit_weights (oasis_inference.py:499-500)
VAE_PREFIX = "encoder."      # find_vae_weights (oasis_inference.py:502-503)


def dit_names(n_blocks):
    """(checkpoint name, weight-dict key) pairs of a DiT with n_blocks blocks
    (oasis_inference.py:513-539,549-599,630-631)."""
    pairs = [("t_embedder.mlp.0.weight", "t_emb.w0"), ("t_embedder.mlp.0.bias", "t_emb.b0"),
             ("t_embedder.mlp.2.weight", "t_emb.w2"), ("t_embedder.mlp.2.bias", "t_emb.b2"),
             ("external_cond.weight", "ext.w"), ("external_cond.bias", "ext.b"),
             ("x_embedder.proj.weight", "x_emb.w"), ("x_embedder.proj.bias", "x_emb.b"),
             ("final_layer.adaLN_modulation.1.weight", "final.ada_w"),
             ("final_layer.adaLN_modulation.1.bias", "final.ada_b"),
             ("final_layer.linear.weight", "final.w"), ("final_layer.linear.bias", "final.b"),
             ("blocks.0.s_attn.rotary_emb.freqs", "rope.spatial_freqs"),
             ("blocks.0.t_attn.rotary_emb.freqs", "rope.temporal_freqs")]
    for i in range(n_blocks):
        for kind in ("s", "t"):
            up, me = "blocks.%d.%s_" % (i, kind), "blocks.%d.%s." % (i, kind)
            pairs += [(up + "adaLN_modulation.1.weight", me + "ada_w"),
                      (up + "adaLN_modulation.1.bias", me + "ada_b"),
                      (up + "attn.to_qkv.weight", me + "qkv_w"),
                      (up + "attn.to_out.weight", me + "out_w"), (up + "attn.to_out.bias", me + "out_b"),
                      (up + "mlp.fc1.weight", me + "fc1_w"), (up + "mlp.fc1.bias", me + "fc1_b"),
                      (up + "mlp.fc2.weight", me + "fc2_w"), (up + "mlp.fc2.bias", me + "fc2_b")]
    return pairs


def vae_decoder_names(depth):
    """(checkpoint name, weight-dict key) pairs of a ViT VAE decoder with depth blocks
    (oasis_inference.py:686-751)."""
    pairs = [("post_quant_conv.weight", "pq_w"), ("post_quant_conv.bias", "pq_b")]
    for i in range(depth):
        up, me = "decoder.%d." % i, "dec.%d." % i
        pairs += [(up + "norm1.weight", me + "n1_w"), (up + "norm1.bias", me + "n1_b"),
                  (up + "attn.qkv.weight", me + "qkv_w"), (up + "attn.qkv.bias", me + "qkv_b"),
                  (up + "attn.proj.weight", me + "proj_w"), (up + "attn.proj.bias", me + "proj_b"),
                  (up + "norm2.weight", me + "n2_w"), (up + "norm2.bias", me + "n2_b"),
                  (up + "mlp.fc1.weight", me + "fc1_w"), (up + "mlp.fc1.bias", me + "fc1_b"),
                  (up + "mlp.fc2.weight", me + "fc2_w"), (up + "mlp.fc2.bias", me + "fc2_b")]
    pairs += [("dec_norm.weight", "norm_w"), ("dec_norm.bias", "norm_b"),
              ("predictor.weight", "pred_w"), ("predictor.bias", "pred_b")]
    return pairs


def _count(keys, fmt):
    n = 0
    while fmt % n in keys:
        n += 1
    return n


def _read(path, pairs_for, count_fmt, what):
    with safe_open(path, framework="pt") as st:
        keys = set(st.keys())
        n = _count(keys, count_fmt)
        if n == 0:
            raise ValueError("%s: no %s blocks (no key %r)" % (path, what, count_fmt % 0))
        missing = [up for up, _ in pairs_for(n) if up not in keys]
        if missing:
            raise KeyError("%s: %s checkpoint lacks %s" % (path, what, ", ".join(missing[:5])))
        return {me: st.get_tensor(up) for up, me in pairs_for(n)}


def load_dit(path):
    """DiT weight dict (for model.DiT) from an upstream DiT checkpoint."""
    return _read(path, dit_names, "blocks.%d.s_adaLN_modulation.1.weight", "DiT")


def load_vae_decoder(path, rope_angles):
    """ViT VAE decoder weight dict (for model.VAE) from an upstream VAE checkpoint (the encoder's
    tensors are not read).

    rope_angles: the decoder attention's RoPE angle table, the upstream model's
    ``decoder[0].attn.rotary_freqs`` buffer: [grid_h, grid_w, rot] or [grid_h*grid_w, rot] with
    rot <= head_dim (18 x 32 x 32 at Oasis-500M, oasis_inference.py:460-462). It is stored as
    ``rope.vae_angles`` and used as given. Required: the checkpoint does not hold it."""
    if rope_angles is None:
        raise ValueError("load_vae_decoder needs rope_angles: the decoder's RoPE angle table "
                         "(the upstream model's rotary_freqs buffer) is not in the checkpoint")
    a = torch.as_tensor(rope_angles).float()
    if a.dim() == 3:
        a = a.reshape(-1, a.shape[-1])
    if a.dim() != 2 or a.shape[1] % 2:
        raise ValueError("rope_angles must be [grid_h, grid_w, rot] or [grid_h*grid_w, rot] with rot even")
    w = _read(path, vae_decoder_names, "decoder.%d.attn.qkv.weight", "VAE decoder")
    w["rope.vae_angles"] = a.contiguous()
    return w


def find_checkpoint(directory, prefix):
    """The first safetensors file in directory (sorted by name) with a key starting with
    prefix; other files are skipped (oasis_inference.py:485-497)."""
    for f in sorted(os.listdir(directory)):
        path = os.path.join(directory, f)
        try:
            with safe_open(path, framework="pt") as st:
                if any(k.startswith(prefix) for k in st.keys()):
                    return path
        except Exception:
            continue
    raise FileNotFoundError("no safetensors file with keys %r... in %s" % (prefix, directory))
