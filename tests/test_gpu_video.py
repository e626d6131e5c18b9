"""Multi-frame generation on the GPU (oasis_video_frames): frame f's context is frame f-1's
denoised latent rolled on the device. With overlap_decode the batch's DDIM steps
(oasis_video_frames without frames) and its decodes (oasis_video_decode) are two graphs on two
streams, alternating between two buffer sets. Checked against the oracle run as the same
chain of frames (reduced depth, full width)."""
import pytest
import torch

import oracle
from helpers import COS_STEP, cuda, metrics, pkg

pytestmark = pytest.mark.gpu


def _case(n_frames=3, seed=51):
    synth = pkg.synth
    dr = synth.Draw(seed)
    noise = dr.normal(n_frames, 16, 18, 32)
    ctx_latent = dr.normal(1, 16, 18, 32)
    actions = synth.one_hot_actions(dr, n_frames)
    w = synth.dit_weights(dr, n_blocks=2)
    vw = synth.vae_weights(dr, depth=2)
    return noise, ctx_latent, actions, w, vw


def _oracle_chain(noise, ctx_latent, actions, w, vw, ac, steps, ctx_t=14.0):
    W_rt, b = oracle.patch_embed_roundtrip_weight(w), w["x_emb.b"].float()
    ctx_z = oracle.patch_embed(ctx_latent, w)[0]
    prev_action = torch.zeros(25)
    out = []
    for f in range(noise.shape[0]):
        x = oracle.patchify_to_output_space(noise[f:f + 1])[0]
        ctx_cond = oracle.conditioning(torch.tensor([ctx_t]), prev_action[None], w)[0]
        gen = [oracle.conditioning(torch.tensor([float(t)]), actions[f][None], w)[0] for t, _ in steps]
        chunk, frame = oracle.ddim_frame(x, ctx_z, ctx_cond, gen, w, vw, ac, steps)
        out.append((chunk, frame))
        ctx_z = chunk @ W_rt + b          # the generated frame becomes the next context
        prev_action = actions[f]
    return out


@pytest.mark.parametrize("kv,overlap", [(True, False), (False, False), (True, True)])
def test_video_frames_match_the_oracle_chain(kv, overlap):
    noise, ctx_latent, actions, w, vw = _case()
    F = noise.shape[0]
    ac = pkg.schedule.cosine_alphas_cumprod()
    steps = [(999, 749), (749, 499), (499, 249), (249, -1)]
    dit, vae = pkg.DiT(w, "cuda"), pkg.VAE(vw, "cuda")
    vp = pkg.VideoPipeline(dit, vae, steps, ac, F, kv_cache=kv, overlap_decode=overlap)
    noise_p = oracle.patchify_to_output_space(noise)
    ctx_p = oracle.patchify_to_output_space(ctx_latent)[0]
    vp.set_inputs(cuda(noise_p), cuda(ctx_p), 14.0, torch.zeros(25), actions)
    vp.capture()
    frames = vp.run().clone()
    chunks = vp.chunks.clone()
    vp.set_inputs(cuda(noise_p), cuda(ctx_p), 14.0, torch.zeros(25), actions)
    frames2 = vp.run().clone()
    torch.cuda.synchronize()
    assert torch.equal(frames, frames2), "graph replay differs"
    ref = _oracle_chain(noise, ctx_latent, actions, w, vw, ac, steps)
    for f in range(F):
        cc, rc = metrics(chunks[f], ref[f][0])
        cf, rf = metrics(frames[f], ref[f][1])
        print("video (kv=%s) frame %d: chunk cos=%.6f rel=%.2e | frame cos=%.6f rel=%.2e" % (kv, f, cc, rc, cf, rf),
              flush=True)
        assert cc >= COS_STEP and cf >= COS_STEP, (f, cc, cf)


def test_pipelined_batches_equal_in_order_batches():
    """Three pipelined batches in a row (buffer sets 0, 1, 0: the third waits for the first's
    decodes) give the frames of the in-order pipeline, bit for bit. The chunks are denoised in
    place, so a buffer set's second batch starts from its first batch's latents: pipelined
    batch k matches in-order batch k // 2."""
    noise, ctx_latent, actions, w, vw = _case(n_frames=2, seed=52)
    F = noise.shape[0]
    ac = pkg.schedule.cosine_alphas_cumprod()
    steps = [(999, 499), (499, -1)]
    dit, vae = pkg.DiT(w, "cuda"), pkg.VAE(vw, "cuda")
    noise_p = cuda(oracle.patchify_to_output_space(noise))
    ctx_p = cuda(oracle.patchify_to_output_space(ctx_latent)[0])
    outs = {}
    for overlap in (False, True):
        vp = pkg.VideoPipeline(dit, vae, steps, ac, F, overlap_decode=overlap)
        vp.set_inputs(noise_p, ctx_p, 14.0, torch.zeros(25), actions)
        vp.capture()
        got = []
        for _ in range(3):
            got.append(vp.run().clone())
        torch.cuda.synchronize()
        outs[overlap] = got
    for k in range(3):
        assert torch.equal(outs[True][k], outs[False][k // 2]), "pipelined batch %d differs" % k


def test_pipelined_launches_overlap_correctly():
    """Three launch() calls and a drain(), the throughput loop: each batch's decodes are launched
    by the next launch. The two buffer sets then hold batches 1 and 2, equal to in-order
    batches 0 and 1 (chunks denoised in place, as above)."""
    noise, ctx_latent, actions, w, vw = _case(n_frames=2, seed=53)
    F = noise.shape[0]
    ac = pkg.schedule.cosine_alphas_cumprod()
    steps = [(999, 499), (499, -1)]
    dit, vae = pkg.DiT(w, "cuda"), pkg.VAE(vw, "cuda")
    noise_p = cuda(oracle.patchify_to_output_space(noise))
    ctx_p = cuda(oracle.patchify_to_output_space(ctx_latent)[0])
    ref = pkg.VideoPipeline(dit, vae, steps, ac, F)
    ref.set_inputs(noise_p, ctx_p, 14.0, torch.zeros(25), actions)
    ref.capture()
    want = [ref.run().clone() for _ in range(2)]
    vp = pkg.VideoPipeline(dit, vae, steps, ac, F, overlap_decode=True)
    vp.set_inputs(noise_p, ctx_p, 14.0, torch.zeros(25), actions)
    vp.capture()
    for _ in range(3):
        vp.launch()
    vp.drain()
    torch.cuda.synchronize()
    assert torch.equal(vp.frame_bufs[1], want[0]), "batch 1 differs"
    assert torch.equal(vp.frame_bufs[0], want[1]), "batch 2 differs"

