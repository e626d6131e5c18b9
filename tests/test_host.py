"""Host-side logic on the CPU: schedules and DDIM coefficients, the RoPE tables and the
weight packing the device kernels consume (laid out on device='cpu' here), and the
determinism of the synthetic inputs."""
import numpy as np
import torch

import oracle
from helpers import noise_reference, philox4x32_10, pkg

M = pkg.model
S = pkg.schedule
synth = pkg.synth


def test_schedules_match_the_oracle():
    assert torch.equal(S.sigmoid_alphas_cumprod(), oracle.sigmoid_alphas_cumprod())
    assert torch.equal(S.cosine_alphas_cumprod(), oracle.cosine_alphas_cumprod())
    for n in (1, 4, 10, 50):
        assert S.ddim_steps(n) == oracle.ddim_timesteps(n)


def test_ddim_coefficients_match_the_oracle():
    ac = S.cosine_alphas_cumprod()
    steps = S.ddim_steps(4)
    flat = S.ddim_coefficients(ac, steps)
    assert len(flat) == 24
    for i, (t, tn) in enumerate(steps):
        ref = oracle.ddim_coeffs(ac, t, tn, i == len(steps) - 1)
        for a, b in zip(flat[6 * i:6 * i + 6], ref):
            assert abs(a - b) <= 1e-6 * max(1.0, abs(b))


def test_rope_tables_match_the_oracle():
    f = synth.theta_freqs(16, 32)
    cos, sinp = M.rope_tables(M._axial_angles(f, 9, 16))
    rc, rs = oracle.rope_cos_sinperm(oracle.spatial_rope_angles(f, 9, 16), 64)
    assert torch.allclose(cos, rc, atol=1e-6) and torch.allclose(sinp, rs, atol=1e-6)
    ft = synth.theta_freqs(32, 64)
    cos, sinp = M.rope_tables(M.temporal_angles(ft, 32))
    rc, rs = oracle.rope_cos_sinperm(oracle.temporal_rope_angles(ft, 32), 64)
    assert torch.allclose(cos, rc, atol=1e-6) and torch.allclose(sinp, rs, atol=1e-6)
    # VAE: 32 of the 64 head dims rotate; the rest is the identity
    fv = synth.theta_freqs(8, 16)
    cos, sinp = M.rope_tables(M._axial_angles(fv, 18, 32))
    assert cos.shape == (576, 64)
    assert torch.equal(cos[:, 32:], torch.ones(576, 32)) and torch.equal(sinp[:, 32:], torch.zeros(576, 32))
    x = torch.randn(576, 64, generator=torch.Generator().manual_seed(0))
    ref = oracle.apply_rotary_emb(oracle.vae_rope_angles(fv, 18, 32), x)
    assert torch.allclose(oracle.apply_rope_swap(x, cos, sinp), ref, atol=1e-5)


def _small_dit(seed=3):
    dr = synth.Draw(seed)
    return synth.dit_weights(dr, n_blocks=2, d=128, n_heads=2, d_mlp=256)


def test_dit_packing_adaln_rows():
    w = _small_dit()
    dit = M.DiT(w, "cpu")
    assert dit.ada_width == 4 * 6 * 128 + 2 * 128 and dit.ada_w.shape == (4 * 6 * 128, 128)
    assert dit.ada_w.dtype == torch.bfloat16 and dit.final_ada_w.dtype == torch.float32
    cond = torch.randn(3, 128, generator=torch.Generator().manual_seed(1))
    rows = oracle.silu(cond) @ dit.ada_w_rows().float().t() + dit.ada_b
    for j in range(4):  # sub-block j: blocks.(j//2).(s|t), chunks shift, scale+1, gate, shift, scale+1, gate
        p = "blocks.%d.%s." % (j // 2, "st"[j % 2])
        ref = oracle.silu(cond) @ w[p + "ada_w"].float().t() + w[p + "ada_b"]
        got = rows[:, j * 768:(j + 1) * 768]
        for c in range(6):
            add = 1.0 if c in (1, 4) else 0.0
            assert torch.allclose(got[:, c * 128:(c + 1) * 128], ref[:, c * 128:(c + 1) * 128] + add, atol=1e-4)
    # the final layer's adaLN stays fp32 and unrounded (oasis_inference.py:527-532)
    assert torch.equal(dit.final_ada_w, w["final.ada_w"].float())
    ref = oracle.silu(cond) @ w["final.ada_w"].float().t() + w["final.ada_b"]
    fin = oracle.silu(cond) @ dit.final_ada_w.t() + dit.final_ada_b
    assert torch.allclose(fin[:, :128], ref[:, :128], atol=1e-4)
    assert torch.allclose(fin[:, 128:], ref[:, 128:] + 1.0, atol=1e-4)


def test_philox_known_answers_and_noise_reference():
    """The host Philox4x32-10 the device noise is checked against reproduces the published
    known-answer vectors of the Random123 distribution (counter, key -> output), and its
    Box-Muller draws have the moments of N(0, 1)."""
    kat = [((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
           ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
           ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
            (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1))]
    for ctr, key, want in kat:
        got = philox4x32_10(np.array([ctr], dtype=np.uint32), key)[0]
        assert tuple(int(v) for v in got) == want
    z = noise_reference(200000, 5, 0, 20.0)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    assert not np.array_equal(noise_reference(64, 5, 0, 20.0), noise_reference(64, 5, 1, 20.0))
    assert np.abs(noise_reference(4096, 5, 2, 0.5)).max() <= 0.5


def test_tile_rows16_layout():
    """The 16-row MFMA tile order of the adaLN stack (oasis_gemv_bf16_tiled): piece l of tile t,
    K step s is row 16t + (l % 16), columns 32s + 8(l // 16) .. +7, at element (t*K/32 + s)*512 +
    8l; untile_rows16 inverts it."""
    N, K = 48, 96
    W = torch.arange(N * K, dtype=torch.float32).reshape(N, K)
    T = M.tile_rows16(W)
    assert T.shape == (N, K) and torch.equal(M.untile_rows16(T), W)
    flat = T.reshape(-1)
    for t in range(N // 16):
        for s_ in range(K // 32):
            for l in (0, 5, 16, 37, 63):
                off = (t * (K // 32) + s_) * 512 + 8 * l
                r, c = 16 * t + l % 16, 32 * s_ + 8 * (l // 16)
                assert torch.equal(flat[off:off + 8], W[r, c:c + 8]), (t, s_, l)


def test_dit_packing_patch_embed_and_action_pad():
    w = _small_dit()
    dit = M.DiT(w, "cpu")
    lat = torch.randn(2, 16, 18, 32, generator=torch.Generator().manual_seed(2))
    patches = oracle.patchify_to_output_space(lat)                  # [2, 144, 64], (p, q, c) columns
    xw = dit._keep[[t.data_ptr() for t in dit._keep].index(dit.struct.xemb_w)]
    assert xw.dtype == torch.float32 and xw.shape == (64, 128)  # the reference's fp32 W_rt, K-major (1821-1826)
    got = patches @ xw + w["x_emb.b"]
    ref = oracle.patch_embed(lat, {k: v.float() for k, v in w.items()})
    assert torch.allclose(got, ref, atol=1e-5 * ref.abs().max().item())
    cw = dit._keep[[t.data_ptr() for t in dit._keep].index(dit.struct.cond_w)]
    assert cw.shape == (128, 128 + 64)       # [W2 | Wext], the action zero-padded to 64 inputs
    assert torch.equal(cw[:, :128], w["t_emb.w2"].float()) and torch.equal(cw[:, 128:153], w["ext.w"].float())
    assert torch.equal(cw[:, 153:], torch.zeros(128, 39))
    cb = dit._keep[[t.data_ptr() for t in dit._keep].index(dit.struct.cond_b)]
    assert torch.equal(cb, w["t_emb.b2"].float() + w["ext.b"].float())
    for name in ("temb_w0", "cond_w", "final_w"):   # conditioning and final layer: fp32
        t = dit._keep[[t.data_ptr() for t in dit._keep].index(getattr(dit.struct, name))]
        assert t.dtype == torch.float32, name
    assert dit.struct.n_sub == 4 and dit.struct.d_model == 128 and dit.struct.t_max == 32


def test_vae_packing():
    dr = synth.Draw(4)
    vw = synth.vae_weights(dr, depth=2, d=128, n_heads=2, d_mlp=256)
    vae = M.VAE(vw, "cpu")
    assert vae.depth == 2 and vae.frame_shape == (3, 360, 640)
    assert vae.struct.depth == 2 and vae.struct.latent_dim == 32 and vae.struct.patch == 20
    ws = vae.workspace()
    assert ws.struct.max_splits == ws.partial.shape[0]


def test_synthetic_inputs_are_deterministic():
    a, b = synth.config0(), synth.config0()
    for k in ("x", "cond"):
        assert torch.equal(a[k], b[k])
    for k in a["w"]:
        assert torch.equal(a["w"][k], b["w"][k])
    acts = synth.one_hot_actions(synth.Draw(5), 7)
    assert acts.shape == (7, 25) and torch.equal(acts.sum(-1), torch.ones(7))


def test_workspace_split_sizing():
    dit = M.DiT(_small_dit(), "cpu")
    assert dit.workspace(288).max_splits == 8
    assert dit.workspace(2048).max_splits == 2
    ws = dit.workspace(4608)  # the large-token O / FC2 tiles use 2 K slices at N = 1024
    assert ws.max_splits == 2 and ws.struct.max_rows == 4608
    assert ws.partial.shape == (2, 4608, dit.d)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU's share; --gpus N > 1 (or a multi-rank launch) exits with a
    message before touching a device."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for extra_env, argv in (({}, ["--gpus", "2"]), ({"WORLD_SIZE": "8"}, [])):
        env = dict(os.environ, **extra_env)
        r = subprocess.run([sys.executable, os.path.join(root, "bench.py")] + argv, capture_output=True,
                           text=True, timeout=120, env=env)
        assert r.returncode != 0 and "one MI355X" in (r.stdout + r.stderr), (argv, r.returncode, r.stderr[-300:])
