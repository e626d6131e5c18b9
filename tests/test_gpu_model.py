"""Model-level parity on the GPU: sub-blocks (configs 0 and 2), the full DiT step
(config 1), the VAE decoder and the 4-step DDIM frame (config 3), graph replay and the
context-frame invariance property. References are the fp32 CPU oracle run on the same
bf16-valued weights the GPU holds.
"""
import ctypes

import pytest
import torch

import oracle
from helpers import COS_STEP, COS_SUB, REL_SUB, assert_close, cuda, metrics, pkg

pytestmark = pytest.mark.gpu

synth = pkg.synth


def _bf16_weights(w):
    return {k: (v.to(torch.bfloat16) if v.dtype == torch.float32 and k != "rope.spatial_freqs"
                and k != "rope.temporal_freqs" else v) for k, v in w.items()}


def _single_block_dit(sub_w, kind, d=1024, d_mlp=4096, spatial_freqs=None, temporal_freqs=None):
    """A one-block DiT whose `kind` sub-block carries `sub_w` (the other one is zeros)."""
    dr = synth.Draw(99)
    w = synth.dit_weights(dr, n_blocks=1, d=d, n_heads=d // 64, d_mlp=d_mlp)
    for k, v in sub_w.items():
        w["blocks.0.%s.%s" % (kind, k)] = v.to(torch.bfloat16)
    if spatial_freqs is not None:
        w["rope.spatial_freqs"] = spatial_freqs
    if temporal_freqs is not None:
        w["rope.temporal_freqs"] = temporal_freqs
    return w


def _check_sub_block(x, cond, w, kind, T, what):
    dit = pkg.DiT(w, "cuda", t_max=max(T, 2))
    ws = dit.workspace(T * dit.P, max_cond=max(16, T))
    ada = dit.adaln_from_cond(cuda(cond), ws)
    ws.x[:T * dit.P].copy_(cuda(x.reshape(T * dit.P, -1)))
    j = 0 if kind == "s" else 1
    dit.sub_blocks_inplace(ws, 1, T, ada, dit.ada_width, j, j + 1)
    torch.cuda.synchronize()
    got = ws.x[:T * dit.P].cpu().reshape(T, dit.P, -1)
    blk = {k[len("blocks.0.%s." % kind):]: v for k, v in w.items() if k.startswith("blocks.0.%s." % kind)}
    if kind == "s":
        cs, ss = oracle.rope_cos_sinperm(oracle.spatial_rope_angles(w["rope.spatial_freqs"].float()), 64)
    else:
        cs, ss = oracle.rope_cos_sinperm(oracle.temporal_rope_angles(w["rope.temporal_freqs"].float(), T), 64)
    ref = oracle.sub_block(x.reshape(T, dit.P, -1).float(), oracle.silu(cond.float()), blk, kind, cs, ss)
    assert_close(got, ref, COS_SUB, REL_SUB, what + " output")
    # the residual update alone is the stricter check (the output is dominated by x)
    assert_close(got - x.reshape(T, dit.P, -1), ref - x.reshape(T, dit.P, -1), COS_SUB, REL_SUB, what + " update")


def test_spatial_sub_block_config0():
    c = synth.config0()
    w = _single_block_dit(c["w"], "s", spatial_freqs=c["spatial_freqs"], temporal_freqs=c["temporal_freqs"])
    _check_sub_block(c["x"][0], c["cond"][0], w, "s", 2, "config0 spatial sub-block")


def test_temporal_sub_block_config2():
    c = synth.config2()
    w = _single_block_dit(c["w"], "t", temporal_freqs=c["temporal_freqs"])
    _check_sub_block(c["x"][0], c["cond"][0], w, "t", 32, "config2 temporal sub-block T=32")


@pytest.mark.parametrize("kind,T", [("s", 1), ("t", 1), ("s", 4), ("t", 4), ("t", 13), ("t", 16), ("s", 33)])
def test_sub_blocks_between_sizes(kind, T):
    """Sub-blocks at the token counts between configs: one 144-token frame (the K/V-cache
    steps' tile and split choices), 576 tokens (tile 2 with the QKV + RoPE epilogue in both
    layouts), 1872 tokens (the largest count below the 8-wave tall tiles), 2304 tokens (the tall
    tiles with O and FC2 as split-K partials, below where unsplit 144 x 128 tiles fill the CUs) and
    4752 tokens (O and FC2 unsplit, 264 tiles: a second partial round)."""
    c0, c2 = synth.config0(), synth.config2()
    dr = synth.Draw(70 + T)
    x, cond = dr.normal(T, 144, 1024), dr.normal(T, 1024)
    src = c0["w"] if kind == "s" else c2["w"]
    w = _single_block_dit(src, kind, spatial_freqs=c0["spatial_freqs"], temporal_freqs=c2["temporal_freqs"])
    _check_sub_block(x, cond, w, kind, T, "%s sub-block T=%d" % (kind, T))


@pytest.fixture(scope="module")
def c1():
    c = synth.config1()
    dit = pkg.DiT(c["w"], "cuda")
    return c, dit


def _c1_reference(c, latent=None):
    lat = c["latent"][0] if latent is None else latent
    z = oracle.patch_embed(lat, c["w"])
    cond = oracle.conditioning(c["t"], c["actions"], c["w"])
    return oracle.dit_forward(z, cond, c["w"]).reshape(-1, 64)


def test_dit_step_config1(c1):
    c, dit = c1
    step = pkg.DiTStep(dit, B=1, T=2)
    patches = oracle.patchify_to_output_space(c["latent"][0]).reshape(-1, 64)
    step.set_inputs(cuda(patches), cuda(c["t"]), cuda(c["actions"]))
    v = step.run()
    torch.cuda.synchronize()
    ref = _c1_reference(c)
    cos, rel = metrics(v, ref)
    print("config1 DiT step: cos=%.6f max_rel=%.3e" % (cos, rel), flush=True)
    assert cos >= COS_STEP, cos


def _rel(got, ref):
    got, ref = got.double().cpu(), ref.double().cpu()
    return ((got - ref).abs().max() / ref.abs().max()).item()


def test_fp32_islands_match_the_fp32_oracle_on_unrounded_weights():
    """The pieces the reference keeps in fp32 (oasis_inference.py:512-532,1406-1427,1497-1521,
    1821-1826) run in fp32 here: a DiT built from fp32 weights that were never rounded to bf16
    gives the conditioning rows, the final layer's adaLN rows, the final layer and the patch
    embed within rel 1e-4 of the fp32 oracle on those same weights (bf16 storage of any of
    them would leave ~4e-3)."""
    dr = synth.Draw(31)
    w = synth.dit_weights(dr, n_blocks=1, dtype=torch.float32)
    for k in ("t_emb.b0", "t_emb.b2", "ext.b", "final.ada_b", "final.b", "x_emb.b"):
        w[k] = dr.normal(*w[k].shape, std=0.1)
    for k in ("t_emb.w0", "t_emb.w2", "ext.w", "final.ada_w", "final.w"):
        w[k] = w[k] * 3   # larger projections: any bf16 rounding shows clearly above 1e-4
    dit = pkg.DiT(w, "cuda")
    R, D, P = 3, dit.d, dit.P
    ws = dit.workspace(R * P, max_cond=16)
    t = torch.tensor([14.0, 749.0, 249.0])
    act = torch.zeros(R, 25)
    act[0, 3] = act[1, 11] = act[2, 24] = 1.0
    ada = dit.conditioning(cuda(t), cuda(act), ws)
    torch.cuda.synchronize()
    cond_ref = oracle.conditioning(t, act, w)
    assert _rel(ws.cond[:R], cond_ref) < 1e-4, _rel(ws.cond[:R], cond_ref)
    ns = dit.n_sub * 6 * D
    fin_ref = oracle.silu(cond_ref) @ w["final.ada_w"].t() + w["final.ada_b"]
    fin_ref[:, D:] += 1.0   # scale_p1
    e = _rel(ada[:, ns:], fin_ref)
    print("fp32 islands: cond %.2e, final adaLN %.2e" % (_rel(ws.cond[:R], cond_ref), e), flush=True)
    assert e < 1e-4, e
    # final layer on a given hidden state (3 frames of 144 tokens), against the oracle
    x = dr.normal(R, P, D) * 2 + 0.3
    ws.x[:R * P].copy_(cuda(x.reshape(R * P, D)))
    v = torch.zeros(R * P, 64, device="cuda")
    L = pkg._lib
    L.call("oasis_dit_final", ctypes.byref(dit.struct), ctypes.byref(ws.struct), R * P, L.ptr(ada), dit.ada_width,
           L.ptr(v), L.stream_handle())
    torch.cuda.synchronize()
    v_ref = oracle.final_layer(x, oracle.silu(cond_ref), w).reshape(R * P, 64)
    e = _rel(v, v_ref)
    print("fp32 islands: final layer %.2e" % e, flush=True)
    assert e < 1e-4, e
    # patch embed with the fp32 W_rt
    lat = dr.normal(2, 16, 18, 32)
    patches = oracle.patchify_to_output_space(lat).reshape(2 * P, 64)
    z = torch.zeros(2 * P, D, device="cuda")
    dit.patch_embed(cuda(patches), z)
    torch.cuda.synchronize()
    e = _rel(z, oracle.patch_embed(lat, w).reshape(2 * P, D))
    assert e < 1e-5, e


def test_dit_step_adaln_rows_of_every_consumer(c1):
    """The adaLN rows a step computes for every consumer, the final layer's included, equal
    silu(cond) @ W^T + b of the packed weights (fp64 on the CPU): the sub-blocks' bf16 stack
    and the final layer's fp32 projection."""
    c, dit = c1
    step = pkg.DiTStep(dit, B=1, T=2)
    step.ws.ada.fill_(float("nan"))  # a slice that is never written stays NaN
    patches = oracle.patchify_to_output_space(c["latent"][0]).reshape(-1, 64)
    step.set_inputs(cuda(patches), cuda(c["t"]), cuda(c["actions"]))
    step.run()
    torch.cuda.synchronize()
    cond = step.ws.cond[:2].double().cpu()
    W = torch.cat([dit.ada_w_rows().double().cpu(), dit.final_ada_w.double().cpu()])
    B_ = torch.cat([dit.ada_b.double().cpu(), dit.final_ada_b.double().cpu()])
    ref = torch.nn.functional.silu(cond) @ W.t() + B_
    got = step.ws.ada[:2].double().cpu()
    assert torch.isfinite(got).all(), "adaLN rows left unwritten"
    D = dit.d
    for j in range(dit.n_sub + 1):
        a, b = j * 6 * D, min((j + 1) * 6 * D, dit.ada_width)
        err = ((got[:, a:b] - ref[:, a:b]).abs().max() / ref[:, a:b].abs().max()).item()
        assert err < 1e-4, (j, err)


def test_dit_step_graph_replay_and_context_invariance(c1):
    c, dit = c1
    step = pkg.DiTStep(dit, B=1, T=2)
    patches = oracle.patchify_to_output_space(c["latent"][0]).reshape(-1, 64)
    step.set_inputs(cuda(patches), cuda(c["t"]), cuda(c["actions"]))
    eager = step.run().clone()
    torch.cuda.synchronize()
    step.capture()
    for i in range(3):
        v = step.run()
        torch.cuda.synchronize()
        assert torch.equal(v, eager), "graph replay %d differs from eager" % i
        torch.randn(1000, device="cuda").sum().item()  # unrelated eager work between replays
    # causal temporal attention + per-frame ops: frame-0 rows never see frame 1
    P = dit.P
    patches2 = patches.clone()
    patches2[P:] = torch.randn(P, 64, generator=torch.Generator().manual_seed(5))
    step.set_inputs(cuda(patches2), cuda(c["t"]), cuda(c["actions"]))
    v2 = step.run()
    torch.cuda.synchronize()
    assert torch.equal(v2[:P], eager[:P]), "context rows changed with the generated frame"
    assert not torch.equal(v2[P:], eager[P:])


def test_dit_forward_surface_reduced():
    dr = synth.Draw(21)
    w = synth.dit_weights(dr, n_blocks=2, d=256, n_heads=4, d_mlp=1024)
    z = dr.normal(2, 144, 256)
    cond = dr.normal(2, 256)
    dit = pkg.DiT(w, "cuda")
    v = pkg.kernels.dit_forward_device(cuda(z.reshape(-1, 256)), [cuda(cond[0]), cuda(cond[1])], dit)
    torch.cuda.synchronize()
    ref = oracle.dit_forward(z, cond, w).reshape(-1, 64)
    assert_close(v, ref, COS_SUB, REL_SUB, "dit_forward surface (2 blocks, D=256)")


def test_dit_forward_device_takes_the_reference_padded_layout(c1):
    """dit_forward_device on the reference's SEQ = 160*T rows (oasis_inference.py:1445): z_cur
    [320, D] holds each frame's 144 tokens at row 160*t and junk in the 16 pad rows; cond_list
    holds the reference's row-expanded [32, D] vectors; scr is the reference's scratch dict. The
    result [320, 64], sliced at gen_start = 160 as ddim_step_fn slices it (oasis_inference.py:
    1915-1918), gives the generated frame's v (config 1, against the oracle) with its pad rows
    zero. The packed [288, D] layout gives the same rows bit for bit, and the calls share one
    workspace."""
    c, dit = c1
    K = pkg.kernels
    D, P = dit.d, dit.P
    z = oracle.patch_embed(c["latent"][0], c["w"])                     # [2, 144, D]
    cond = oracle.conditioning(c["t"], c["actions"], c["w"])           # [2, D]
    ref = oracle.dit_forward(z, cond, c["w"])                          # [2, 144, 64]
    zp = synth.Draw(33).normal(2, 160, D) * 1e3
    zp[:, :P] = z
    conds = [cuda(cond[t].expand(32, D).contiguous()) for t in range(2)]
    scr = {}
    out = K.dit_forward_device(cuda(zp.reshape(320, D)), conds, dit, scr, None, None, None)
    torch.cuda.synchronize()
    ws = dit._surface_ws
    assert out.shape == (320, 64)
    v_dev = out[160:320]                                               # ddim_step_fn's slice
    assert torch.count_nonzero(v_dev[P:]) == 0 and torch.count_nonzero(out[P:160]) == 0
    for t, rows in ((0, out[:P]), (1, v_dev[:P])):
        cos, rel = metrics(rows, ref[t])
        print("padded dit_forward_device frame %d: cos=%.6f rel=%.3e" % (t, cos, rel), flush=True)
        assert cos >= COS_STEP, (t, cos)
    padded = out.clone()
    packed = K.dit_forward_device(cuda(z.reshape(2 * P, D)), conds, dit, scr)
    torch.cuda.synchronize()
    assert torch.equal(packed[:P], padded[:P]) and torch.equal(packed[P:], padded[160:160 + P])
    assert dit._surface_ws is ws
    with pytest.raises(pkg._lib.OasisError, match="rows"):
        K.dit_forward_device(cuda(zp.reshape(320, D)[:300]), conds, dit, scr)


@pytest.fixture(scope="module")
def c3():
    c = synth.config3()
    dit = pkg.DiT(c["w"], "cuda")
    vae = pkg.VAE(c["vw"], "cuda")
    return c, dit, vae


def test_vae_decode_config3(c3):
    c, _, vae = c3
    frame = pkg.kernels.vae_decode(cuda(c["vae_latent"]), vae)
    torch.cuda.synchronize()
    ref = oracle.vae_unpatchify(oracle.vae_decode(c["vae_latent"], c["vw"]))
    cos, rel = metrics(frame, ref)
    print("config3 VAE decode: cos=%.6f max_rel=%.3e" % (cos, rel), flush=True)
    assert cos >= COS_STEP and rel <= 5e-2, (cos, rel)


def test_vae_decode_forward_returns_pred_out(c3):
    """vae_decode_forward returns the reference's pred_out (oasis_inference.py:1546-1618): the
    predictor's rows, unclamped, [576, 1216] with zero TILE-padding columns; vae_decode_device
    (oasis_inference.py:1620-1634) pads a [576, 16] latent to the decoder's width and reads
    back [576, 1200] on the host. Both match the oracle's predictor rows, and unpatchified and
    clamped they give the fused fast path's frame."""
    c, _, vae = c3
    K = pkg.kernels
    ws = vae.workspace()
    ws.latent.copy_(cuda(c["vae_latent"]))
    pred = K.vae_decode_forward(vae, ws, None, None)
    torch.cuda.synchronize()
    ref = oracle.vae_decode(c["vae_latent"], c["vw"])                  # [576, 1200]
    assert pred.shape == (576, 1216) and torch.count_nonzero(pred[:, 1200:]) == 0
    assert_close(pred[:, :1200], ref, COS_STEP, 5e-2, "vae_decode_forward pred_out vs oracle")
    frame = K.vae_decode_forward(vae, ws, fused_frame=True).clone()
    torch.cuda.synchronize()
    assert_close(oracle.vae_unpatchify(pred[:, :1200].cpu()), frame, 0.99999, 1e-3,
                 "unpatchified pred_out vs the fused frame")
    # the reference's 16-channel latent, zero-padded on the device
    z16 = c["vae_latent"][:, :16].contiguous()
    lat32 = torch.zeros(576, 32)
    lat32[:, :16] = z16
    host = K.vae_decode_device(cuda(z16), vae, ws, None, None, None)
    assert host.device.type == "cpu" and host.shape == (576, 1200)
    assert_close(host, oracle.vae_decode(lat32, c["vw"]), COS_STEP, 5e-2, "vae_decode_device vs oracle")


@pytest.mark.parametrize("B", [3, 8])
def test_vae_decode_batch_matches_single_decodes(c3, B):
    """B latents decoded as one pass of B*576 tokens (B = 3: the small-token tiles; B = 8: 4608
    tokens on the large-token tiles, config 4's 8 streams) give each latent's frame as its own
    decode does, and the first one matches the oracle."""
    c, _, vae = c3
    dr = synth.Draw(90 + B)
    lats = dr.normal(B, 576, 32)
    ws = vae.workspace(max_frames=B)
    frames = torch.zeros(B, *vae.frame_shape, device="cuda")
    vae.decode_batch(cuda(lats), frames, ws)
    one = vae.workspace()
    single = torch.zeros(B, *vae.frame_shape, device="cuda")
    for b in range(B):
        vae.decode_inplace(cuda(lats[b]), single[b], one)
    torch.cuda.synchronize()
    for b in range(B):
        # two bf16 paths (4608 tokens run the large-token tiles, another summation order)
        assert_close(frames[b], single[b], 0.9999, 5e-2, "batched VAE decode B=%d, latent %d vs alone" % (B, b))
    ref = oracle.vae_unpatchify(oracle.vae_decode(lats[0], c["vw"]))
    assert_close(frames[0], ref, COS_STEP, 5e-2, "batched VAE decode B=%d, latent 0 vs oracle" % B)
    with pytest.raises(pkg._lib.OasisError, match="exceed the workspace"):
        vae.decode_batch(cuda(lats), frames, one)


def test_ddim_frame_config3(c3):
    c, dit, vae = c3
    ac = pkg.schedule.cosine_alphas_cumprod()
    fp = pkg.FramePipeline(dit, vae, c["steps"], ac)
    noise = oracle.patchify_to_output_space(c["x_T"])[0]
    ctx = oracle.patchify_to_output_space(c["ctx_latent"])[0]
    fp.set_inputs(cuda(noise), cuda(ctx), c["ctx_t"], cuda(c["ctx_action"]), cuda(c["gen_action"]))
    fp.capture()
    frame = fp.run()
    torch.cuda.synchronize()
    chunk = fp.chunk.cpu()
    w = c["w"]
    ctx_z = oracle.patch_embed(c["ctx_latent"], w)[0]
    ctx_cond = oracle.conditioning(torch.tensor([c["ctx_t"]]), c["ctx_action"][None], w)[0]
    gen_conds = [oracle.conditioning(torch.tensor([float(t)]), c["gen_action"][None], w)[0] for t, _ in c["steps"]]
    ref_chunk, ref_frame = oracle.ddim_frame(noise, ctx_z, ctx_cond, gen_conds, w, c["vw"], ac, c["steps"])
    cc, rc = metrics(chunk, ref_chunk)
    cf, rf = metrics(frame, ref_frame)
    print("config3 frame: chunk cos=%.6f rel=%.3e | frame cos=%.6f rel=%.3e" % (cc, rc, cf, rf), flush=True)
    assert cc >= COS_STEP and cf >= COS_STEP, (cc, cf)


def test_frame_ddim_update_fused_into_the_final_layer(c3):
    """The frame's DDIM update runs inside the final layer's launch; on a one-step frame it gives
    the chunk the stand-alone oasis_ddim_update gives from the same noise and v rows, bit for bit
    (with and without the K/V cache)."""
    c, dit, vae = c3
    ac = pkg.schedule.cosine_alphas_cumprod()
    steps = c["steps"][:1]
    noise = cuda(oracle.patchify_to_output_space(c["x_T"])[0])
    ctx = cuda(oracle.patchify_to_output_space(c["ctx_latent"])[0])
    coeffs = pkg.schedule.ddim_coefficients(ac, steps)
    P = dit.P
    for kv in (False, True):
        fp = pkg.FramePipeline(dit, vae, steps, ac, kv_cache=kv)
        fp.set_inputs(noise, ctx, c["ctx_t"], cuda(c["ctx_action"]), cuda(c["gen_action"]))
        fp.run()
        torch.cuda.synchronize()
        v = fp.ws.v_out[P:2 * P].clone()   # the generated frame's v rows of the T=2 step
        want = noise.clone()
        pkg._lib.call("oasis_ddim_update", pkg._lib.ptr(want), pkg._lib.ptr(v), want.numel(),
                      *[ctypes.c_float(z) for z in coeffs], pkg._lib.stream_handle())
        torch.cuda.synchronize()
        assert torch.equal(fp.chunk, want), "fused DDIM update differs (kv_cache=%s)" % kv
        assert not torch.equal(fp.chunk, noise)


@pytest.mark.parametrize("B,T", [(8, 4), (1, 2)])
def test_final_layer_with_pending_residual_matches_residual_ln_then_final(B, T):
    """oasis_dit_forward folds the last FC2's split-K partials (bias + gated residual) into the
    final layer's launch. At 4608 rows (config 4's batch, more workgroups than run at once) and at
    288 rows it leaves x bit-equal to oasis_dit_sub_blocks (which applies that residual with
    oasis_residual_ln), and its v rows equal oasis_dit_final's on that x: every row's residual is
    added once, whatever order the workgroups run in."""
    dr = synth.Draw(57)
    w = synth.dit_weights(dr, n_blocks=1)
    dit = pkg.DiT(w, "cuda", t_max=max(T, 2))
    M, D = B * T * dit.P, dit.d
    ws = dit.workspace(M, max_cond=B * T)
    ada = dit.adaln_from_cond(cuda(dr.normal(B * T, D)), ws)
    x0 = cuda(dr.normal(M, D))
    ws.x[:M].copy_(x0)
    v_fused = torch.zeros(M, 64, device="cuda")
    dit.forward_inplace(ws, B, T, ada, dit.ada_width, v_fused)
    torch.cuda.synchronize()
    x_fused = ws.x[:M].clone()
    ws.x[:M].copy_(x0)
    dit.sub_blocks_inplace(ws, B, T, ada, dit.ada_width, 0, dit.n_sub)
    v_sep = torch.zeros(M, 64, device="cuda")
    L = pkg._lib
    L.call("oasis_dit_final", ctypes.byref(dit.struct), ctypes.byref(ws.struct), M, L.ptr(ada), dit.ada_width,
           L.ptr(v_sep), L.stream_handle())
    torch.cuda.synchronize()
    assert torch.equal(x_fused, ws.x[:M]), "residual applied differently (B=%d, T=%d)" % (B, T)
    e = _rel(v_fused, v_sep)
    print("final layer with pending residual, M=%d: v rel %.2e, bit-equal %s"
          % (M, e, torch.equal(v_fused, v_sep)), flush=True)
    assert e < 1e-6, e


def test_dit_from_an_upstream_checkpoint_steps_identically(tmp_path):
    """A DiT built from an upstream-named safetensors checkpoint (checkpoint.load_dit) runs the
    same step, bit for bit, as one built from the weight dict it was written from."""
    from safetensors.torch import save_file
    ck = pkg.checkpoint
    dr = pkg.synth.Draw(81)
    w = pkg.synth.dit_weights(dr, n_blocks=2)
    path = str(tmp_path / "dit.safetensors")
    save_file({up: w[me].contiguous() for up, me in ck.dit_names(2)}, path)
    outs = []
    for weights in (w, ck.load_dit(path)):
        dit = pkg.DiT(weights, "cuda")
        step = pkg.DiTStep(dit, B=1, T=2)
        lat = pkg.synth.Draw(82).normal(2, 16, 18, 32)
        step.set_inputs(cuda(oracle.patchify_to_output_space(lat).reshape(-1, 64)), cuda(torch.tensor([10.0, 500.0])),
                        cuda(torch.zeros(2, 25)))
        outs.append(step.run().clone())
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
