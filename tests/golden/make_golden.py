"""Writes tests/golden/oasis_golden.safetensors: known-answer vectors of the fp32 CPU
oracle for small, seeded cases of the hot path.

The reference holds no golden vectors or fixture files (its tests draw random inputs
and need Tenstorrent hardware), so these vectors come from the oracle, after the oracle
itself is pinned by tests/test_oracle.py. They serve two checks:
  - tests/test_golden.py (CPU): the oracle still reproduces them (catches drift of the
    oracle or of the seeded synthetic inputs);
  - tests/test_gpu_golden.py (GPU): the HIP path matches them without running the oracle.

Weights are not stored (they would be megabytes); each case redraws them from its seed
with the package's seeded generator and the file keeps a checksum of every weight set,
which both tests verify before comparing.

    python tests/golden/make_golden.py
"""
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
PATH = os.path.join(HERE, "oasis_golden.safetensors")

if REPO not in sys.path:
    sys.path.insert(0, REPO)


def _pkg():
    import __graft_entry__
    return __graft_entry__.load_package()


def checksum(tensors):
    """[sum, sum of |x|, sum of x*i mod 9973 weights] in fp64 over a dict or list of tensors."""
    items = [tensors[k] for k in sorted(tensors)] if isinstance(tensors, dict) else list(tensors)
    s = torch.zeros(3, dtype=torch.float64)
    for t in items:
        x = t.detach().double().flatten()
        idx = (torch.arange(x.numel(), dtype=torch.float64) % 9973) + 1
        s += torch.stack([x.sum(), x.abs().sum(), (x * idx).sum()])
    return s


# ----------------------------------------------------------------- the cases
def case_dit2():
    """A reduced DiT step: 2 blocks, D=256, 4 heads, T=2 frames at the full 9x16 grid."""
    synth = _pkg().synth
    dr = synth.Draw(31)
    latent = dr.normal(2, 16, 18, 32)
    t = torch.tensor([14.0, 640.0])
    act = synth.one_hot_actions(dr, 2)
    w = synth.dit_weights(dr, n_blocks=2, d=256, n_heads=4, d_mlp=1024)
    return {"latent": latent, "t": t, "actions": act, "w": w}


def case_c0():
    """Config 0: one spatial sub-block at D=1024 (fp32 weights)."""
    return _pkg().synth.config0()


def case_vae2():
    """A reduced ViT decoder: 2 blocks, D=256, 4 heads, full 18x32 grid."""
    synth = _pkg().synth
    dr = synth.Draw(32)
    latent = dr.normal(576, 32)
    vw = synth.vae_weights(dr, depth=2, d=256, n_heads=4, d_mlp=1024)
    return {"latent": latent, "vw": vw}


def case_frame2():
    """The 4-step DDIM frame over the reduced DiT and decoder."""
    synth = _pkg().synth
    dr = synth.Draw(33)
    x_T = dr.normal(1, 16, 18, 32)
    ctx_latent = dr.normal(1, 16, 18, 32)
    gen_action = synth.one_hot_actions(dr, 1)[0]
    w = synth.dit_weights(dr, n_blocks=2, d=256, n_heads=4, d_mlp=1024)
    vw = synth.vae_weights(dr, depth=2, d=256, n_heads=4, d_mlp=1024)
    return {"x_T": x_T, "ctx_latent": ctx_latent, "ctx_t": 14.0, "ctx_action": torch.zeros(25),
            "gen_action": gen_action, "w": w, "vw": vw,
            "steps": [(999, 749), (749, 499), (499, 249), (249, -1)]}


C0_ROWS = list(range(0, 16)) + list(range(280, 288))
FRAME_STRIDE = 8


def frame_sample(frame):
    """Every 8th pixel of a [3, 360, 640] frame, plus per-channel sums."""
    return frame[:, ::FRAME_STRIDE, ::FRAME_STRIDE].contiguous(), frame.double().sum((1, 2))


# ----------------------------------------------------------------- expected outputs (oracle)
def expected():
    import oracle
    out = {}
    # scalars and tables
    ac = oracle.cosine_alphas_cumprod()
    sc = oracle.sigmoid_alphas_cumprod()
    idx = torch.tensor([0, 249, 499, 749, 999])
    out["sched.cosine"] = ac[idx]
    out["sched.sigmoid"] = sc[idx]
    steps = oracle.ddim_timesteps(4)
    out["sched.ddim_coeffs"] = torch.tensor(
        [c for i, (t, tn) in enumerate(steps) for c in oracle.ddim_coeffs(ac, t, tn, i == 3)], dtype=torch.float64)
    out["temb"] = oracle.timestep_embedding(torch.tensor([0.0, 14.0, 999.0]), 256)

    c = case_dit2()
    z = oracle.patch_embed(c["latent"], c["w"])
    cond = oracle.conditioning(c["t"], c["actions"], c["w"])
    out["dit2.weights"] = checksum(c["w"])
    out["dit2.v"] = oracle.dit_forward(z, cond, c["w"]).reshape(-1, 64)

    c = case_c0()
    cs, ss = oracle.rope_cos_sinperm(oracle.spatial_rope_angles(c["spatial_freqs"]), 64)
    x = c["x"][0]
    y = oracle.sub_block(x, oracle.silu(c["cond"][0]), c["w"], "s", cs, ss)
    upd = (y - x).reshape(288, -1)
    out["c0.weights"] = checksum(c["w"])
    out["c0.update_rows"] = upd[C0_ROWS].contiguous()
    out["c0.update_row_sums"] = upd.double().sum(-1)

    c = case_vae2()
    fr = oracle.vae_unpatchify(oracle.vae_decode(c["latent"], c["vw"]))
    out["vae2.weights"] = checksum(c["vw"])
    out["vae2.frame_sample"], out["vae2.frame_channel_sums"] = frame_sample(fr)

    c = case_frame2()
    w = c["w"]
    noise = oracle.patchify_to_output_space(c["x_T"])[0]
    ctx_z = oracle.patch_embed(c["ctx_latent"], w)[0]
    ctx_cond = oracle.conditioning(torch.tensor([c["ctx_t"]]), c["ctx_action"][None], w)[0]
    gen = [oracle.conditioning(torch.tensor([float(t)]), c["gen_action"][None], w)[0] for t, _ in c["steps"]]
    chunk, fr = oracle.ddim_frame(noise, ctx_z, ctx_cond, gen, w, c["vw"], ac, c["steps"])
    out["frame2.weights"] = checksum(list(w.values()) + list(c["vw"].values()))
    out["frame2.chunk"] = chunk
    out["frame2.frame_sample"], out["frame2.frame_channel_sums"] = frame_sample(fr)
    return {k: v.contiguous() for k, v in out.items()}


def load():
    from safetensors.torch import load_file
    return load_file(PATH)


def main():
    from safetensors.torch import save_file
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    out = expected()
    save_file(out, PATH, metadata={"generator": "tests/golden/make_golden.py", "source": "fp32 CPU oracle"})
    print("wrote %s (%d tensors, %d bytes)" % (PATH, len(out), os.path.getsize(PATH)))


if __name__ == "__main__":
    main()
