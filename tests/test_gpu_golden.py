"""The HIP path against the committed known-answer vectors (no oracle run on the box):
the reduced DiT step, the config-0 spatial sub-block update, the reduced ViT decoder and
the reduced 4-step DDIM frame."""
import os
import sys

import pytest
import torch

from helpers import COS_STEP, COS_SUB, REL_SUB, assert_close, cuda, pkg

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def golden():
    return make_golden.load()


def _patchify(lat):
    """[B, C, 2*gh, 2*gw] -> [B, gh*gw, 64], columns (p, q, c) (oasis_inference.py:958-969)."""
    B, C, H, W = lat.shape
    x = lat.reshape(B, C, H // 2, 2, W // 2, 2).permute(0, 2, 4, 3, 5, 1)
    return x.reshape(B, (H // 2) * (W // 2), 4 * C)


def test_golden_dit2_step(golden):
    c = make_golden.case_dit2()
    assert torch.allclose(make_golden.checksum(c["w"]), golden["dit2.weights"], rtol=1e-12, atol=0)
    dit = pkg.DiT(c["w"], "cuda")
    step = pkg.DiTStep(dit, B=1, T=2)
    step.set_inputs(cuda(_patchify(c["latent"]).reshape(-1, 64)), cuda(c["t"]), cuda(c["actions"]))
    v = step.run()
    torch.cuda.synchronize()
    assert_close(v, golden["dit2.v"], COS_SUB, REL_SUB, "golden dit2 step")


def test_golden_config0_update(golden):
    c = make_golden.case_c0()
    assert torch.allclose(make_golden.checksum(c["w"]), golden["c0.weights"], rtol=1e-12, atol=0)
    dr = pkg.synth.Draw(99)
    w = pkg.synth.dit_weights(dr, n_blocks=1)
    for k, v in c["w"].items():
        w["blocks.0.s." + k] = v.to(torch.bfloat16)
    w["rope.spatial_freqs"] = c["spatial_freqs"]
    dit = pkg.DiT(w, "cuda")
    ws = dit.workspace(288)
    ada = dit.adaln_from_cond(cuda(c["cond"][0]), ws)
    x = c["x"][0].reshape(288, -1)
    ws.x[:288].copy_(cuda(x))
    dit.sub_blocks_inplace(ws, 1, 2, ada, dit.ada_width, 0, 1)
    torch.cuda.synchronize()
    upd = ws.x[:288].cpu() - x
    assert_close(upd[make_golden.C0_ROWS], golden["c0.update_rows"], COS_SUB, REL_SUB, "golden c0 update rows")
    assert_close(upd.double().sum(-1), golden["c0.update_row_sums"], COS_SUB, 5e-2, "golden c0 row sums")


def _check_frame(frame, golden, prefix):
    sample = frame[:, ::make_golden.FRAME_STRIDE, ::make_golden.FRAME_STRIDE]
    assert_close(sample, golden[prefix + ".frame_sample"], COS_STEP, 5e-2, prefix + " frame sample")
    sums = frame.double().sum((1, 2)).cpu()
    ref = golden[prefix + ".frame_channel_sums"]
    assert torch.allclose(sums, ref, rtol=2e-2, atol=2e-3 * frame[0].numel()), (sums, ref)


def test_golden_vae2(golden):
    c = make_golden.case_vae2()
    assert torch.allclose(make_golden.checksum(c["vw"]), golden["vae2.weights"], rtol=1e-12, atol=0)
    vae = pkg.VAE(c["vw"], "cuda")
    frame = pkg.kernels.vae_decode(cuda(c["latent"]), vae)
    torch.cuda.synchronize()
    _check_frame(frame.cpu(), golden, "vae2")


def test_golden_frame2(golden):
    c = make_golden.case_frame2()
    ref_w = make_golden.checksum(list(c["w"].values()) + list(c["vw"].values()))
    assert torch.allclose(ref_w, golden["frame2.weights"], rtol=1e-12, atol=0)
    dit = pkg.DiT(c["w"], "cuda")
    vae = pkg.VAE(c["vw"], "cuda")
    fp = pkg.FramePipeline(dit, vae, c["steps"], pkg.schedule.cosine_alphas_cumprod())
    fp.set_inputs(cuda(_patchify(c["x_T"])[0]), cuda(_patchify(c["ctx_latent"])[0]), c["ctx_t"],
                  cuda(c["ctx_action"]), cuda(c["gen_action"]))
    frame = fp.run()
    torch.cuda.synchronize()
    assert_close(fp.chunk.cpu(), golden["frame2.chunk"], COS_STEP, 5e-2, "golden frame2 chunk")
    _check_frame(frame.cpu(), golden, "frame2")
