"""The interactive frame loop (PlaySession, the reference's play loop play.py:241-531) on the
GPU: frames against the oracle run as the same chain (noise drawn by the session, actions
through the hold, context rolled and reset to the prompt), and DDIM step-count switches."""
import pytest
import torch

import oracle
from helpers import COS_STEP, metrics, pkg

pytestmark = pytest.mark.gpu


def _models(seed):
    synth = pkg.synth
    dr = synth.Draw(seed)
    prompt = dr.normal(1, 16, 18, 32)
    w = synth.dit_weights(dr, n_blocks=2)
    vw = synth.vae_weights(dr, depth=2)
    return prompt, w, vw


def _session_chain(noises, prompt, prompt_action, actions, w, vw, ac, steps, reset_every, ctx_t=14.0):
    W_rt, b = oracle.patch_embed_roundtrip_weight(w), w["x_emb.b"].float()
    prompt_z = oracle.patch_embed(prompt, w)[0]
    ctx_z, prev = prompt_z, prompt_action
    out = []
    for f, x in enumerate(noises):
        ctx_cond = oracle.conditioning(torch.tensor([ctx_t]), prev[None], w)[0]
        gen = [oracle.conditioning(torch.tensor([float(t)]), actions[f][None], w)[0] for t, _ in steps]
        chunk, frame = oracle.ddim_frame(x, ctx_z, ctx_cond, gen, w, vw, ac, steps)
        out.append((chunk, frame))
        ctx_z, prev = chunk @ W_rt + b, actions[f]
        if f > 0 and f % reset_every == 0:  # play.py:497-500
            ctx_z, prev = prompt_z, prompt_action
    return out


@pytest.mark.parametrize("kv", [True, False])
def test_session_frames_match_the_oracle_chain(kv):
    prompt, w, vw = _models(61)
    dit, vae = pkg.DiT(w, "cuda"), pkg.VAE(vw, "cuda")
    ac = pkg.schedule.sigmoid_alphas_cumprod()
    s = pkg.PlaySession(dit, vae, prompt, ddim_steps=2, reset_every=2, seed=5, keep_noise=True, kv_cache=kv)
    a0, a3 = torch.zeros(25), torch.zeros(25)
    a0[4], a3[9] = 1.0, 1.0
    z = torch.zeros(25)
    sent = [a0, z, z, a3]
    held = [a0, a0, z, a3]  # one frame of hold after the release
    frames, noises = [], []
    for a in sent:
        frames.append(s.frame(a).clone())
        noises.append(s.last_noise.cpu())
    torch.cuda.synchronize()
    # the reference's numbering: the 4th frame is frame 3 (play.py:517-525)
    assert s.frame_index == 4 and s.status()["frame_index"] == 3 and s.status()["ddim_steps"] == 2 and s.fps > 0
    for x in noises:
        assert x.abs().max() <= 20.0
    steps = pkg.schedule.ddim_steps(2)
    ref = _session_chain(noises, prompt, torch.zeros(25), held, w, vw, ac, steps, reset_every=2)
    for f, (chunk, frame) in enumerate(ref):
        want = ((frame + 1) * 0.5).clamp(0, 1).permute(1, 2, 0)
        got = frames[f]
        assert got.shape == want.shape and got.min() >= 0 and got.max() <= 1
        cf, rf = metrics(got, want)
        print("session (kv=%s) frame %d: cos=%.6f rel=%.2e" % (kv, f, cf, rf), flush=True)
        assert cf >= COS_STEP, (f, cf)


def test_session_ddim_switch_resets_and_reuses_graphs():
    prompt, w, vw = _models(62)
    dit, vae = pkg.DiT(w, "cuda"), pkg.VAE(vw, "cuda")
    s = pkg.PlaySession(dit, vae, prompt, ddim_steps=2, seed=1)
    a = torch.zeros(25)
    a[2] = 1.0
    first = s.frame(a).clone()
    s.frame(a)
    fp2 = s.fp
    assert not torch.equal(fp2.ctx_patches, s.prompt)  # context rolled
    s.set_ddim_steps(3)
    s.stream.synchronize()  # the reset copies run on the session's stream
    assert s.ddim_steps == 3 and s.frame_index == 0 and s.fp is not fp2
    assert torch.equal(s.fp.ctx_patches, s.prompt)
    s.frame(a)
    s.set_ddim_steps(2)
    s.stream.synchronize()
    assert s.fp is fp2 and torch.equal(fp2.ctx_patches, s.prompt)
    s.set_ddim_steps(0)
    assert s.ddim_steps == 1
    # same seed, same prompt and action: the first frame of a fresh session repeats
    s2 = pkg.PlaySession(dit, vae, prompt, ddim_steps=2, seed=1)
    again = s2.frame(a)
    torch.cuda.synchronize()
    assert torch.equal(again, first)
