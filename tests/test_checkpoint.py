"""Loading the upstream checkpoints (open-oasis_amd/checkpoint.py) on the CPU: safetensors files
written with the upstream tensor names (oasis_inference.py:505-760) from seeded weights load back
into the weight dicts model.DiT / model.VAE take, bit for bit; discovery by key prefix skips
files that are not safetensors; missing tensors raise."""
import os

import pytest
import torch
from safetensors.torch import save_file

from helpers import pkg

ck = pkg.checkpoint
synth = pkg.synth
M = pkg.model


def _small():
    dr = synth.Draw(71)
    w = synth.dit_weights(dr, n_blocks=2, d=128, n_heads=2, d_mlp=256)
    vw = synth.vae_weights(dr, depth=2, d=128, n_heads=2, d_mlp=256)
    return w, vw


def _write(path, pairs, w, extra=None):
    t = {up: w[me].contiguous() for up, me in pairs}
    t.update(extra or {})
    save_file(t, path)


def test_dit_checkpoint_round_trip(tmp_path):
    w, _ = _small()
    path = str(tmp_path / "dit.safetensors")
    _write(path, ck.dit_names(2), w)
    got = ck.load_dit(path)
    assert set(got) == set(w)
    for k in w:
        assert got[k].dtype == w[k].dtype and torch.equal(got[k], w[k]), k


def test_vae_decoder_checkpoint_round_trip_ignores_the_encoder(tmp_path):
    _, vw = _small()
    path = str(tmp_path / "vae.safetensors")
    enc = {"encoder.0.attn.qkv.weight": torch.zeros(3, 3), "quant_conv.weight": torch.zeros(2, 2)}
    _write(path, ck.vae_decoder_names(2), vw, enc)
    with pytest.raises(ValueError, match="rope_angles"):
        ck.load_vae_decoder(path, None)
    angles = torch.rand(18, 32, 32, generator=torch.Generator().manual_seed(5))
    got = ck.load_vae_decoder(path, angles)
    assert set(got) == (set(vw) - {"rope.vae_freqs"}) | {"rope.vae_angles"}
    for k in vw:
        if k != "rope.vae_freqs":
            assert torch.equal(got[k], vw[k]), k
    # the angle table is used as given: the model's RoPE tables are its cos / signed sin
    assert torch.equal(got["rope.vae_angles"], angles.reshape(576, 32))
    vae = M.VAE(got, "cpu")
    cos = vae._keep[[t.data_ptr() for t in vae._keep].index(vae.struct.rope_cos)]
    assert torch.allclose(cos[:, :32], angles.reshape(576, 32).double().cos().float(), atol=1e-6)
    assert torch.equal(cos[:, 32:], torch.ones(576, 32))


def test_find_checkpoint_by_prefix_skips_other_files(tmp_path):
    w, vw = _small()
    (tmp_path / "README").write_text("not a checkpoint")
    _write(str(tmp_path / "b_dit"), ck.dit_names(2), w)
    _write(str(tmp_path / "c_vae"), ck.vae_decoder_names(2), vw, {"encoder.0.norm1.weight": torch.ones(4)})
    assert os.path.basename(ck.find_checkpoint(str(tmp_path), ck.DIT_PREFIX)) == "b_dit"
    assert os.path.basename(ck.find_checkpoint(str(tmp_path), ck.VAE_PREFIX)) == "c_vae"
    with pytest.raises(FileNotFoundError):
        ck.find_checkpoint(str(tmp_path), "nothing.")


def test_missing_tensor_raises(tmp_path):
    w, _ = _small()
    pairs = [p for p in ck.dit_names(2) if p[0] != "blocks.1.t_mlp.fc2.bias"]
    path = str(tmp_path / "dit.safetensors")
    _write(path, pairs, w)
    with pytest.raises(KeyError, match="blocks.1.t_mlp.fc2.bias"):
        ck.load_dit(path)
    empty = str(tmp_path / "empty.safetensors")
    save_file({"x": torch.zeros(1)}, empty)
    with pytest.raises(ValueError):
        ck.load_dit(empty)
