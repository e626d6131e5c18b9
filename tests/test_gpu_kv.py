"""The temporal K/V-cache path on the GPU: the past-frame pass + current-frame pass equal
the current rows of the T=2 forward (the reference's gate: PCC >= 0.999,
oasis_inference.py:2076-2123), for one and for several streams, and the K/V-cache frame
pipeline equals the all-T=2 one."""
import pytest
import torch

import oracle
from helpers import COS_STEP, cuda, metrics, pkg

pytestmark = pytest.mark.gpu


def _pcc(a, b):
    a = a.double().flatten().cpu()
    b = b.double().flatten().cpu()
    a, b = a - a.mean(), b - b.mean()
    return ((a * b).sum() / ((a * a).sum() * (b * b).sum()).sqrt()).item()


def _kv_vs_t2(c, B, weights="bf16"):
    """v of the current frames by the T=2 forward and by past pass + current pass."""
    dit = pkg.DiT(c["w"], "cuda", weights=weights)
    P = dit.P
    lat = c["latent"].reshape(B, 2, 16, 18, 32)
    patches = oracle.patchify_to_output_space(lat.reshape(B * 2, 16, 18, 32)).reshape(-1, 64)
    step = pkg.DiTStep(dit, B=B, T=2)
    step.set_inputs(cuda(patches), cuda(c["t"].reshape(-1)), cuda(c["actions"].reshape(B * 2, -1)))
    v_t2 = step.run().clone().reshape(B, 2, P, 64)
    torch.cuda.synchronize()
    ada = step.ws.ada[:2 * B].clone()                   # rows b*2 + t
    ws = dit.workspace(2 * B * P, max_cond=max(16, 2 * B))
    kv = pkg.model.KVCache(dit, B)
    ptc = cuda(patches).reshape(B, 2, P, 64)
    dit.patch_embed(ptc[:, 0].reshape(-1, 64).contiguous(), ws.x)      # past frames
    dit.precompute_past(ws, kv, B, ada[0::2].contiguous(), dit.ada_width)
    ada_cur = ada[1::2].contiguous()
    dit.patch_embed(ptc[:, 1].reshape(-1, 64).contiguous(), ws.x)      # current frames
    v_cur = torch.zeros(B * P, 64, device="cuda")
    dit.forward_current(ws, kv, B, ada_cur, dit.ada_width, v_cur)
    torch.cuda.synchronize()
    return v_t2[:, 1].cpu(), v_cur.reshape(B, P, 64).cpu()


def test_kv_cache_equals_t2_config1():
    c = pkg.synth.config1()
    ref, got = _kv_vs_t2(c, 1)
    pcc = _pcc(got, ref)
    cos, rel = metrics(got, ref)
    print("KV cache vs T=2 (config1): pcc=%.7f cos=%.7f max_rel=%.2e" % (pcc, cos, rel), flush=True)
    assert pcc >= 0.999 and rel <= 2e-2


def test_kv_cache_equals_t2_four_streams():
    c = pkg.synth.config4(seed=43, B=4, T=2, n_blocks=4)
    ref, got = _kv_vs_t2(c, 4)
    for b in range(4):
        pcc = _pcc(got[b], ref[b])
        print("KV cache vs T=2, stream %d: pcc=%.7f" % (b, pcc), flush=True)
        assert pcc >= 0.999


def test_kv_cache_fp8_weights():
    c = pkg.synth.config4(seed=44, B=2, T=2, n_blocks=2)
    ref, got = _kv_vs_t2(c, 2, weights="fp8")
    pcc = _pcc(got, ref)
    print("KV cache vs T=2 (fp8 weights): pcc=%.7f" % pcc, flush=True)
    assert pcc >= 0.999


def test_frame_pipeline_kv_equals_t2():
    c = pkg.synth.config3()
    dit = pkg.DiT(c["w"], "cuda")
    vae = pkg.VAE(c["vw"], "cuda")
    ac = pkg.schedule.cosine_alphas_cumprod()
    noise = oracle.patchify_to_output_space(c["x_T"])[0]
    ctx = oracle.patchify_to_output_space(c["ctx_latent"])[0]
    out = {}
    for kv in (False, True):
        fp = pkg.FramePipeline(dit, vae, c["steps"], ac, kv_cache=kv)
        fp.set_inputs(cuda(noise), cuda(ctx), c["ctx_t"], cuda(c["ctx_action"]), cuda(c["gen_action"]))
        fp.capture()
        for _ in range(2):  # replays are stateless: the context K/V are rebuilt every frame
            fp.set_inputs(cuda(noise), cuda(ctx), c["ctx_t"], cuda(c["ctx_action"]), cuda(c["gen_action"]))
            frame = fp.run().clone()
        torch.cuda.synchronize()
        out[kv] = (fp.chunk.cpu(), frame.cpu())
    pc = _pcc(out[True][0], out[False][0])
    cf, rf = metrics(out[True][1], out[False][1])
    print("frame with KV cache vs all-T=2: chunk pcc=%.7f | frame cos=%.7f rel=%.2e" % (pc, cf, rf), flush=True)
    assert pc >= 0.999 and cf >= COS_STEP
