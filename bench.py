"""Benchmark: ms per Oasis-500M DiT denoising step (config 1: T=2, bf16, 16 blocks) and FPS of
the 4-step DDIM + VAE frame (config 3) on one MI355X, with synthetic seeded inputs and
random-init weights.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--frames F] [--no-cpu-baseline]

A step is one replay of the captured hipGraph of the full DiT step: on-device
conditioning (timestep MLP, action projection and all 33 adaLN projections), patch
embed of the two frames, 16 x (spatial, temporal) sub-blocks and the final layer.
Inputs are resident in HBM before the timed region. Prints one JSON line.
"""
import argparse
import ctypes
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0


def _event_ms(fn, stream, n, graph=None):
    """Average duration of fn() over n launches, HIP events on `stream`. With `graph` (the
    package's Graph class) the n launches are captured in one hipGraph and the timed region is
    one replay, so host-side launch cost cannot stretch kernels of a few microseconds."""
    import torch
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if graph is not None:
        def many():
            for _ in range(n):
                fn()
        g = graph(many, stream)
        g.launch()
        s.record(stream)
        g.launch()
        e.record(stream)
        e.synchronize()
        return s.elapsed_time(e) / n
    with torch.cuda.stream(stream):
        fn()
        s.record(stream)
        for _ in range(n):
            fn()
        e.record(stream)
    e.synchronize()
    return s.elapsed_time(e) / n


# HBM-side bytes per launch (L2-miss fetch + write) of the roofline kernels, from
# `rocprofv3 --pmc FETCH_SIZE` and `--pmc WRITE_SIZE` runs of `bench.py --probe`, each
# scaled by what the same counter reads for a plain device copy of known size.
TRAFFIC = {"fc1_ln": 16877545, "fc1_row": 15622976, "gemv": 405109565, "fc1_4608_bf16": 90367489,
           "fc1_4608_fp8": 46325337}


def _fc1_timing(pkg, dit, ws, stream, n=100, graph=True):
    """The FC1 projection alone, as the step runs it at 288 tokens (the same kernel, buffers and
    tile: with the library's default plan FC1 with the carried LayerNorm on the fragment-order
    weights), timed with HIP events on the step stream. Launch i uses the weights of sub-block
    i % 32: as in the step, each launch reads weights that 31 launches (268 MB of other weights,
    more than the 256 MB memory-side cache) have passed over since their last use, so they come
    from HBM. Returns (ms, flop, algorithmic bytes, kind)."""
    L = pkg._lib
    M, D, Dm, P = 288, dit.d, dit.d_mlp, dit.P
    S, n_sub = dit.struct, dit.n_sub
    plan = L.frag_plan(M)
    ln = bool(plan & L.FRAG_LN and plan & L.FRAG_O) and "fc1" in dit.frag_roles and hasattr(ws, "ln_mod")
    frag = ln or (bool(plan & L.FRAG_FC1) and "fc1" in dit.frag_roles)
    out_frag = 1 if plan & L.FRAG_FC2 and "fc2" in dit.frag_roles else 0
    F = (M + P - 1) // P
    rows = ws.struct.frag_rows
    eps = []
    for j in range(n_sub):
        e = L.Epilogue()
        e.bias, e.out_bf16, e.ld_out = S.fc1_b[j], ws.mlp.data_ptr(), Dm
        if ln:
            e.kind, e.rows_per_frame, e.ln_eps, e.out_frag = L.EPI_GELU_TANH_LN, P, 1e-6, out_frag
            e.ln_stats, e.ln_mod = ws.ln_stats.data_ptr(), ws.ln_mod.data_ptr()
        else:
            e.kind = L.EPI_GELU_TANH_FRAG if out_frag and frag else L.EPI_GELU_TANH
        eps.append((ctypes.c_void_p(S.fc1_wf[j] if frag else S.fc1_w[j]), e))
    A, it = L.ptr(ws.h), [0]

    def fc1():
        B, e = eps[it[0] % n_sub]
        it[0] += 1
        if frag:
            L.call("oasis_gemm_bf16_frag", A, rows, B, M, Dm, D, ctypes.byref(e), 1, L.stream_handle(stream))
        else:
            L.call("oasis_gemm_bf16", A, D, B, D, M, Dm, D, ctypes.byref(e), L.stream_handle(stream))
    ms = _event_ms(fc1, stream, n, pkg.Graph if graph else None)
    flop = 2 * M * D * Dm
    nbytes = M * D * 2 + Dm * D * 2 + Dm * 4 + M * Dm * 2   # A, W, bias, out (bf16)
    if ln:   # the row statistics (sums over 32-column groups at 288 tokens) and the frames' modulate rows
        G = 32 if M > 160 else 16
        nbytes += M * (D // G) * 8 + 2 * F * D * 2
    kind = "ln" if ln else ("frag" if frag else "row")
    return ms, flop, nbytes, kind


def _gemv_timing(pkg, dit, ws, stream, R=2, n=50, graph=True):
    """The adaLN skinny GEMM over every sub-block's adaLN weights (403 MB bf16). Launch i reads
    copy i % 2 of the weights, so 806 MB pass between two reads of the same bytes (more than the
    256 MB memory-side cache): every launch streams its weights from HBM."""
    import torch
    L = pkg._lib
    ns = dit.n_sub * 6 * dit.d   # the sub-blocks' rows (the final layer's 2D fp32 rows run apart)
    copies = [dit.ada_w, dit.ada_w.clone()]
    it = [0]

    def gemv():
        W = copies[it[0] % 2]
        it[0] += 1
        L.call("oasis_gemv_bf16_tiled", L.ptr(ws.cond), dit.d, R, L.ptr(W), ns, dit.d,
               L.ptr(dit.ada_b), L.ptr(ws.ada), dit.ada_width, L.ACT_SILU, L.ACT_NONE, 0,
               L.stream_handle(stream))
    ms = _event_ms(gemv, stream, n, pkg.Graph if graph else None)
    del copies
    torch.cuda.empty_cache()
    nbytes = ns * dit.d * 2 + R * dit.d * 4 + R * ns * 4 + ns * 4
    return ms, nbytes


def probe(pkg, n=10):
    """Short run for hardware-counter passes: n launches each of the FC1 GEMM and the
    adaLN GEMV on config-1 buffers, n each of the 4608-token FC1 GEMM in bf16 and in fp8
    (config-4 shape, random operands), and n plain 256 MiB device copies (the calibration
    kernel, 268435456 bytes read and written per launch)."""
    import torch
    c1 = pkg.synth.config1()
    dit = pkg.DiT(c1["w"], "cuda")
    step = pkg.DiTStep(dit, B=1, T=2)
    patches = pkg.patchify_latent(c1["latent"][0]).reshape(-1, 64)
    step.set_inputs(patches.cuda(), c1["t"].cuda(), c1["actions"].cuda())
    step.run()
    torch.cuda.synchronize()
    _fc1_timing(pkg, dit, step.ws, step.stream, n, graph=False)
    _gemv_timing(pkg, dit, step.ws, step.stream, n=n, graph=False)
    del step, dit
    L = pkg._lib
    M, D, Dm = 4608, 1024, 4096
    g = torch.Generator(device="cuda").manual_seed(0)
    A = torch.randn(M, D, device="cuda", generator=g).to(torch.bfloat16)
    W = (torch.randn(Dm, D, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    out = torch.empty(M, Dm, device="cuda", dtype=torch.bfloat16)
    h = L.stream_handle(torch.cuda.current_stream())
    e = L.Epilogue()
    e.kind, e.out_bf16, e.ld_out = L.EPI_GELU_TANH, out.data_ptr(), Dm
    for _ in range(n + 1):
        L.call("oasis_gemm_bf16", L.ptr(A), D, L.ptr(W), D, M, Dm, D, ctypes.byref(e), h)
    q = torch.empty(Dm, D, device="cuda", dtype=torch.uint8)
    sc = torch.empty(Dm, device="cuda")
    a8 = torch.empty(M, D, device="cuda", dtype=torch.uint8)
    a8s = torch.empty(M, D // 32, device="cuda", dtype=torch.uint8)
    m8 = torch.empty(M, Dm, device="cuda", dtype=torch.uint8)
    m8s = torch.empty(M, Dm // 32, device="cuda", dtype=torch.uint8)
    L.call("oasis_quantize_fp8_rows", L.ptr(W), Dm, D, L.ptr(q), L.ptr(sc), h)
    L.call("oasis_quantize_act_fp8", L.ptr(A), D, M, D, L.ptr(a8), D, L.ptr(a8s), D // 32, h)
    e8 = L.Epilogue()
    e8.kind, e8.out_fp8, e8.out_scale, e8.ld_out, e8.ld_scale = (L.EPI_GELU_TANH_FP8, m8.data_ptr(), m8s.data_ptr(),
                                                                 Dm, Dm // 32)
    for _ in range(n + 1):
        L.call("oasis_gemm_fp8_a8", L.ptr(a8), D, L.ptr(a8s), D // 32, L.ptr(q), D, L.ptr(sc), M, Dm, D,
               ctypes.byref(e8), -1, 1, h)
    torch.cuda.synchronize()
    src = torch.ones(64 << 20, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(n):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "fc1 gemm x%d, adaLN gemv x%d, 4608-token fc1 gemm bf16 and fp8 x%d each, "
                               "256 MiB copy x%d" % (n + 1, n + 1, n + 1, n)}), flush=True)


def kernel_probe(pkg, n=10):
    """Short run for hardware-counter passes over the other kernels, in order: two eager config-1
    DiT steps (every step kernel, 32 sub-blocks each), two eager config-3 VAE decodes (12 blocks
    each), the bandwidth kernels of `bandwidth_kernels` (n + 1 launches each), and n plain 256 MiB
    device copies (the calibration kernel)."""
    import torch
    c1 = pkg.synth.config1()
    dit = pkg.DiT(c1["w"], "cuda")
    step = pkg.DiTStep(dit, B=1, T=2)
    patches = pkg.patchify_latent(c1["latent"][0]).reshape(-1, 64)
    step.set_inputs(patches.cuda(), c1["t"].cuda(), c1["actions"].cuda())
    for _ in range(2):
        step.run()
    torch.cuda.synchronize()
    del step, dit
    c3 = pkg.synth.config3()
    vae = pkg.VAE(c3["vw"], "cuda")
    vws = vae.workspace()
    latent = c3["vae_latent"].cuda()
    frame = torch.empty(vae.frame_shape, device="cuda")
    for _ in range(2):
        vae.decode_inplace(latent, frame, vws, torch.cuda.current_stream())
    torch.cuda.synchronize()
    bandwidth_kernels(pkg, n, graph=False)
    src = torch.ones(64 << 20, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(n):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "2 config-1 steps, 2 config-3 VAE decodes, bandwidth kernels x%d, 256 MiB copy x%d"
                      % (n + 1, n)}), flush=True)


def _graph_step_ms(step, steps, warmup):
    import torch
    step.capture()
    for _ in range(warmup):
        step.graph.launch()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step.graph.launch()
    torch.cuda.synchronize()
    return 1e3 * (time.perf_counter() - t0) / steps


def config4(pkg, steps, warmup):
    """Config 4: 8 independent streams x T=4 frames (4608 tokens) per DiT step, QKV/O/FC1/FC2
    on e4m3 weights, against the same batch on bf16 weights. A generated frame needs 4 DDIM
    steps, so DiT frames/s = 8 streams / (4 x step time); with the decodes, frames/s =
    8 / (4 x step time + the 8 streams' bridges and VAE decodes, batched as one 4608-token pass)."""
    import torch
    c = pkg.synth.config4()
    B, T = 8, 4
    patches = pkg.patchify_latent(c["latent"].reshape(B * T, 16, 18, 32)).reshape(-1, 64).cuda()
    res = {"workload": "config4: 8 streams x T=4 (4608 tokens), 16 blocks, D=1024; QKV/O/FC1/FC2 weights "
                       "e4m3 with per-channel fp32 scales, activations in e4m3 blocks of 32 with power-of-two "
                       "scales (written by the LN / GELU producers) on the block-scaled fp8 MFMA; "
                       "adaLN/conditioning/final layer bf16"}
    for fmt in ("bf16", "fp8"):
        dit = pkg.DiT(c["w"], "cuda", weights=fmt)
        step = pkg.DiTStep(dit, B=B, T=T)
        step.set_inputs(patches, c["t"].reshape(-1).cuda(), c["actions"].reshape(B * T, -1).cuda())
        ms = _graph_step_ms(step, steps, warmup)
        res["ms_per_step_" + fmt] = round(ms, 4)
        res["dit_frames_per_s_" + fmt] = round(B * 1e3 / (4 * ms), 1)
        # the FC1 projection of sub-block 0 alone (same buffers, same kernel choice)
        M, D, Dm = B * T * dit.P, dit.d, dit.d_mlp
        L = pkg._lib
        e = L.Epilogue()
        e.kind, e.bias, e.out_bf16, e.ld_out = L.EPI_GELU_TANH, dit.struct.fc1_b[0], step.ws.mlp.data_ptr(), Dm
        A, W = L.ptr(step.ws.h), ctypes.c_void_p(dit.struct.fc1_w[0])
        if fmt == "fp8":  # as in the step: A in fp8 blocks (LN output), GELU output in fp8 blocks
            S = ctypes.c_void_p(dit.struct.fc1_s[0])
            A8, A8s = L.ptr(step.ws.act8), L.ptr(step.ws.act8_scale)
            e.kind, e.out_fp8, e.out_scale, e.ld_scale = (L.EPI_GELU_TANH_FP8, step.ws.mlp8.data_ptr(),
                                                          step.ws.mlp8_scale.data_ptr(), Dm // 32)
            fn = lambda: L.call("oasis_gemm_fp8_a8", A8, D, A8s, D // 32, W, D, S, M, Dm, D,  # noqa: E731
                                ctypes.byref(e), -1, 1, L.stream_handle(step.stream))
            peak = FP8_PEAK_TFLOPS
        else:
            fn = lambda: L.call("oasis_gemm_bf16", A, D, W, D, M, Dm, D, ctypes.byref(e),  # noqa: E731
                                L.stream_handle(step.stream))
            peak = BF16_PEAK_TFLOPS
        gms = _event_ms(fn, step.stream, 50)
        tf = 2 * M * D * Dm / (gms * 1e-3) / 1e12
        res["fc1_gemm_" + fmt] = {"avg_launch_ms": round(gms, 5), "achieved": round(tf, 1), "peak": peak,
                                  "unit": "TFLOP/s", "frac": round(tf / peak, 4),
                                  "traffic": TRAFFIC.get("fc1_4608_" + fmt)}
        del step, dit
        torch.cuda.empty_cache()
    res["speedup_fp8_vs_bf16"] = round(res["ms_per_step_bf16"] / res["ms_per_step_fp8"], 3)
    # the 8 streams' decodes: bridge of each denoised latent, then one VAE decode of the 8 latents
    # (4608 tokens) as a captured graph; beside it the same 8 decodes one after another
    dr = pkg.synth.Draw(4)
    vae = pkg.VAE(pkg.synth.vae_weights(dr), "cuda")
    dit = pkg.DiT(pkg.synth.dit_weights(dr, n_blocks=1), "cuda")   # only its grid is read
    chunks = dr.normal(B, dit.P, 64).cuda()
    L = pkg._lib
    stream = torch.cuda.Stream()
    for nb in (B, 1):
        vws = vae.workspace(max_frames=nb)
        lat = torch.zeros(nb * vae.L, vae.latent_dim, device="cuda")
        frames = torch.zeros(B, *vae.frame_shape, device="cuda")
        fn = lambda: L.call("oasis_video_decode", ctypes.byref(dit.struct), ctypes.byref(vae.struct),  # noqa: E731
                            ctypes.byref(vws.struct), B, L.ptr(chunks), L.ptr(lat), L.ptr(frames),
                            L.stream_handle(stream))
        dms = _event_ms(fn, stream, 10, pkg.Graph)
        res["decode_%d_streams_ms_%s" % (B, "batched" if nb == B else "one_by_one")] = round(dms, 4)
        del vws, lat, frames
    dms = res["decode_%d_streams_ms_batched" % B]
    for fmt in ("bf16", "fp8"):
        res["frames_per_s_with_decode_" + fmt] = round(B * 1e3 / (4 * res["ms_per_step_" + fmt] + dms), 1)
    res["decode_workload"] = ("8 bridges + one VAE decode of the 8 latents (12 ViT blocks over 8 x 576 = 4608 "
                              "tokens, attention per latent) + unpatchify, one hipGraph; frames_per_s_with_decode = "
                              "8 / (4 DDIM steps + that decode)")
    del vae, dit
    torch.cuda.empty_cache()
    return res


def config2(pkg, n=20):
    """Config 2: one temporal sub-block over T=32 frames x 144 positions (4608 tokens), causal
    attention over the 32 frames of each position; adaLN rows from the config's cond vectors.
    Algorithmic work: the projections, 2 x 4608 x 1024 x (3072 + 1024 + 4096 + 4096) = 115.96 GFLOP,
    and the causal attention, 4 x 64 x (1 + 2 + ... + 32) per (position, head) = 0.31 GFLOP."""
    import torch
    c = pkg.synth.config2()
    dr = pkg.synth.Draw(99)
    w = pkg.synth.dit_weights(dr, n_blocks=1)
    for k, v in c["w"].items():
        w["blocks.0.t.%s" % k] = v.to(torch.bfloat16)
    w["rope.temporal_freqs"] = c["temporal_freqs"]
    T = 32
    dit = pkg.DiT(w, "cuda", t_max=T)
    ws = dit.workspace(T * dit.P, max_cond=T)
    stream = torch.cuda.Stream()
    ada = dit.adaln_from_cond(c["cond"][0].cuda(), ws)
    x0 = c["x"][0].reshape(T * dit.P, -1).cuda()
    ws.x[:T * dit.P].copy_(x0)
    torch.cuda.synchronize()
    ms = _event_ms(lambda: dit.sub_blocks_inplace(ws, 1, T, ada, dit.ada_width, 1, 2, stream), stream, n, pkg.Graph)
    M, D, Dm = T * dit.P, dit.d, dit.d_mlp
    proj = 2 * M * D * (3 * D + D + 2 * Dm)
    attn = 4 * dit.P * (dit.d // 64) * (T * (T + 1) // 2) * 64   # causal QK^T and PV over 32 frames
    flop = proj + attn
    tf = flop / (ms * 1e-3) / 1e12
    return {"workload": "config2: one temporal sub-block, T=32 x 144 positions (4608 tokens), D=1024, causal "
                        "attention over frames, bf16 weights, fp32 residual",
            "ms_per_sub_block": round(ms, 4), "algorithmic_gflop": round(flop / 1e9, 2),
            "achieved_tflops": round(tf, 1), "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4),
            "floor_ms": round(flop / (BF16_PEAK_TFLOPS * 1e12) * 1e3, 4)}


def bandwidth_kernels(pkg, n=200, graph=True):
    """The memory-bound kernels on their own, D=1024, at the config-1 step's 288 rows and at
    4608 rows (configs 2 and 4), each timed with HIP events over n launches on one stream. Launch i
    works on operand set i % S, with S sets spanning at least 640 MB, so that every launch reads
    operands the 256 MB memory-side cache no longer holds (`achieved`). `cache_warm` repeats one
    operand set, which then stays in that cache, as in the step, where each of these kernels reads
    what the kernel before it has just written.
    Algorithmic bytes are every input and output read or written once:
      residual_ln  (the step's fused split-K sum + bias + gated residual + LN + adaLN modulate,
                   4 fp32 partials): x read and written (fp32), 4 partials, bias, one gate,
                   shift and scale row per frame, the bf16 LN output;
      adaln_modulate (bf16): x, shift, scale in, out;
      layernorm (bf16, [D] fp32 weight and bias): x in, out;
      rope_layout (bf16, heads-first): the [rows, 3D] QKV in, Q/K/V out, fp32 cos and sin
                   tables of 144 positions x D."""
    import torch
    L = pkg._lib
    D, P = 1024, 144
    stream = torch.cuda.Stream()
    g = torch.Generator(device="cuda").manual_seed(7)
    out = []

    def n_sets(set_bytes):
        return max(2, -(-(640 << 20) // set_bytes))

    def rnd(*shape, dtype=torch.float32):
        return torch.randn(*shape, device="cuda", generator=g).to(dtype)

    def timed(name, rows, nbytes, launch):
        """launch(i) enqueues the launch on operand set i; nbytes is the algorithmic bytes."""
        sets, it = n_sets(nbytes), [0]

        def fn():
            launch(it[0] % sets)
            it[0] += 1
        gcls = pkg.Graph if graph else None
        ms = _event_ms(fn, stream, n, gcls)
        ms_warm = _event_ms(lambda: launch(0), stream, n, gcls)
        gbs, gbs_warm = nbytes / (ms * 1e-3) / 1e9, nbytes / (ms_warm * 1e-3) / 1e9
        out.append({"kernel": name, "rows": rows, "bound": "hbm", "achieved": round(gbs, 1),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                    "avg_launch_ms": round(ms, 5), "algorithmic_bytes": nbytes, "operand_sets": sets,
                    "cache_warm": {"achieved": round(gbs_warm, 1), "avg_launch_ms": round(ms_warm, 5)}})
        return sets

    h = L.stream_handle(stream)
    bf = torch.bfloat16
    for M in (288, 4608):
        F = M // P
        E = M * D
        # residual_ln: x (per set), partials (per set), per-frame rows (shared, small)
        nb = E * (4 + 4 * 4 + 4 + 2) + D * 4 + 3 * F * D * 4
        S_ = n_sets(nb)
        x, part = rnd(S_, E), rnd(S_, 4, E)
        y = torch.empty(S_, E, device="cuda", dtype=bf)
        bias, gate, sh, sc = rnd(D), rnd(F, D), rnd(F, D), rnd(F, D)
        timed("residual_ln (4 split-K partials + bias + gated residual + LN + modulate)", M, nb,
              lambda i: L.call("oasis_residual_ln", L.ptr(x[i]), M, D, L.ptr(part[i]), 4, E, L.ptr(bias),
                               L.ptr(gate), D, P, L.ptr(sc), L.ptr(sh), D, L.ptr(y[i]), 1e-6, h))
        del x, part, y
        nb = 4 * E * 2
        S_ = n_sets(nb)
        xb, shb, scb, ob = (rnd(S_, E, dtype=bf) for _ in range(4))
        timed("adaln_modulate (bf16)", M, nb,
              lambda i: L.call("oasis_adaln_modulate", L.ptr(xb[i]), L.ptr(shb[i]), L.ptr(scb[i]), L.ptr(ob[i]), E,
                               L.BF16, h))
        del xb, shb, scb, ob
        nb = 2 * E * 2 + 2 * D * 4
        S_ = n_sets(nb)
        xl, ol = rnd(S_, E, dtype=bf), torch.empty(S_, E, device="cuda", dtype=bf)
        lw, lb = rnd(D), rnd(D)
        timed("layernorm (bf16, affine)", M, nb,
              lambda i: L.call("oasis_layernorm", L.ptr(xl[i]), L.ptr(lw), L.ptr(lb), 0, L.ptr(ol[i]), M, D, 1e-6,
                               L.BF16, h))
        del xl, ol
        nb = 6 * E * 2 + 2 * P * D * 4
        S_ = n_sets(nb)
        qkv = rnd(S_, 3 * E, dtype=bf)
        q, k, v = (torch.empty(S_, E, device="cuda", dtype=bf) for _ in range(3))
        cs, sn = rnd(P, D), rnd(P, D)
        timed("rope_layout (bf16, heads-first)", M, nb,
              lambda i: L.call("oasis_rope_layout", L.ptr(qkv[i]), 3 * D, L.ptr(cs), L.ptr(sn), D, 64, 1, P,
                               L.ptr(q[i]), L.ptr(k[i]), L.ptr(v[i]), M, P, D // 64, 64, 0, L.BF16, h))
        del qkv, q, k, v
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def _median_ms(fn, runs=5, seconds=6.0):
    """2 warm-ups, then the median of at least `runs` timed calls (more while `seconds` last, at most 20)."""
    for _ in range(2):
        fn()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < runs or (time.perf_counter() < t_end and len(times) < 20):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return 1e3 * times[len(times) // 2], len(times)


def cpu_baseline(cfg, oracle, pkg):
    """The fp32 oracle (same weights and inputs) on this host's cores: the config-1 DiT step (the
    headline figure), one config-0 spatial sub-block, and one config-3 frame (4 DDIM steps + VAE)."""
    import torch
    # the host cores this job may use (the GPU box exports its CPU share as OMP_NUM_THREADS)
    torch.set_num_threads(int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count() or 1)
    with torch.inference_mode():
        w = cfg["w"]

        def step():
            z = oracle.patch_embed(cfg["latent"][0], w)
            oracle.dit_forward(z, oracle.conditioning(cfg["t"], cfg["actions"], w), w)
        step_ms, n_step = _median_ms(step, seconds=5.0)

        c0 = pkg.synth.config0()
        blk = {k: v.float() for k, v in c0["w"].items()}
        cs, ss = oracle.rope_cos_sinperm(oracle.spatial_rope_angles(c0["spatial_freqs"].float()), 64)
        x0, sc0 = c0["x"][0].float(), oracle.silu(c0["cond"][0].float())
        sub_ms, n_sub = _median_ms(lambda: oracle.sub_block(x0, sc0, blk, "s", cs, ss), seconds=2.0)

        c3 = pkg.synth.config3()
        w3, ac = c3["w"], pkg.schedule.cosine_alphas_cumprod()
        noise = oracle.patchify_to_output_space(c3["x_T"])[0]

        def frame():
            ctx_z = oracle.patch_embed(c3["ctx_latent"], w3)[0]
            ctx_cond = oracle.conditioning(torch.tensor([c3["ctx_t"]]), c3["ctx_action"][None], w3)[0]
            gen = [oracle.conditioning(torch.tensor([float(t)]), c3["gen_action"][None], w3)[0] for t, _ in c3["steps"]]
            oracle.ddim_frame(noise, ctx_z, ctx_cond, gen, w3, c3["vw"], ac, c3["steps"])
        frame_ms, n_frame = _median_ms(frame, seconds=0.0)
    return {"value": round(step_ms, 2), "unit": "ms/DiT step",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": "median of %d full config-1 DiT steps (T=2, 16 blocks) of the fp32 CPU oracle "
                      "after 2 warm-ups" % n_step,
            "config0_sub_block_ms": round(sub_ms, 2),
            "config0_sample": "median of %d config-0 spatial sub-blocks (x [2,144,1024]) after 2 warm-ups" % n_sub,
            "config3_frame_ms": round(frame_ms, 1),
            "config3_fps": round(1e3 / frame_ms, 3),
            "config3_sample": "median of %d config-3 frames (4 DDIM steps at T=2 + bridge + 12-block VAE decode) "
                              "after 2 warm-ups" % n_frame}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--frames", type=int, default=100)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-frame", action="store_true")
    ap.add_argument("--no-c4", action="store_true", help="skip the config-4 (fp8, 8 streams x T=4) lines")
    ap.add_argument("--probe", action="store_true", help="short run of the roofline kernels for counter passes")
    ap.add_argument("--probe-kernels", action="store_true",
                    help="short run of the step, VAE and bandwidth kernels for counter passes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build targets one MI355X; multi-GPU runs are not part of it "
              "(the path would shard by independent streams, one per GPU)", file=sys.stderr)
        sys.exit(2)

    import torch
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    if args.probe:
        probe(pkg)
        return
    if args.probe_kernels:
        kernel_probe(pkg)
        return
    synth = pkg.synth

    # ---------------- config 1: the DiT step ----------------
    c1 = synth.config1()
    dit = pkg.DiT(c1["w"], "cuda")
    step = pkg.DiTStep(dit, B=1, T=2)
    patches = pkg.patchify_latent(c1["latent"][0]).reshape(-1, 64)
    step.set_inputs(patches.cuda(), c1["t"].cuda(), c1["actions"].cuda())
    step.capture()
    for _ in range(args.warmup):
        step.graph.launch()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(step.stream)
    for _ in range(args.steps):
        step.graph.launch()
    ev1.record(step.stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = 1e3 * (t1 - t0) / args.steps
    ms_step_gpu = ev0.elapsed_time(ev1) / args.steps

    ws = step.ws
    fc1_ms, fc1_flop, fc1_bytes, fc1_kind = _fc1_timing(pkg, dit, ws, step.stream)
    ada_ms, ada_bytes = _gemv_timing(pkg, dit, ws, step.stream)
    fc1_tflops = fc1_flop / (fc1_ms * 1e-3) / 1e12
    ada_gbs = ada_bytes / (ada_ms * 1e-3) / 1e9

    # The FC1 GEMM's bound on the roofline: its arithmetic intensity (213 flop per algorithmic
    # byte at M=288) is below the ridge point (2.5 PFLOP/s / 8 TB/s = 312.5), so HBM bounds it;
    # the MFMA utilisation is reported beside it.
    fc1_ai = fc1_flop / fc1_bytes
    ridge = BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
    fc1_gbs = fc1_bytes / (fc1_ms * 1e-3) / 1e9
    fc1_desc = {
        "ln": "gemm_frag_kernel<5,4,4,GELU_TANH_LN> (bf16 MFMA GEMM on fragment-order operands, 1 KB per wave load "
              "straight into registers, 8 waves splitting K; 80 x 64 tiles, 256 workgroups), FC1 projection + the "
              "LayerNorm + modulate carried from O (row statistics, modulate rows as one more MFMA block) + bias + "
              "tanh-GELU (M=288, N=4096, K=1024)",
        "frag": "gemm_frag_kernel<5,4,4,GELU_TANH> (bf16 MFMA GEMM on fragment-order operands, 8 waves splitting K; "
                "80 x 64 tiles, 256 workgroups), FC1 projection + bias + tanh-GELU (M=288, N=4096, K=1024)",
        "row": "gemm_wave_kernel<80,64,2,4,GELU_TANH,72> (bf16 MFMA GEMM, 4 waves splitting K, each over its own "
               "direct-to-LDS ring; 80-row tiles every 72 rows, 256 workgroups), FC1 projection + bias + tanh-GELU "
               "(M=288, N=4096, K=1024)"}[fc1_kind]
    fc1_roofline = {"kernel": fc1_desc + ", the step's longest kernel (32 launches per step); launch i uses sub-block "
                              "i % 32's weights (cold, as in the step); 100 launches in one hipGraph"}
    if fc1_ai < ridge:
        fc1_roofline.update({"bound": "hbm", "achieved": round(fc1_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(fc1_gbs / HBM_PEAK_GBS, 4)})
    else:
        fc1_roofline.update({"bound": "mfma", "achieved": round(fc1_tflops, 1), "peak": BF16_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(fc1_tflops / BF16_PEAK_TFLOPS, 4)})
    fc1_roofline.update({"traffic": TRAFFIC.get("fc1_" + fc1_kind), "avg_launch_ms": round(fc1_ms, 5),
                         "algorithmic_flop": fc1_flop, "algorithmic_bytes": fc1_bytes,
                         "arithmetic_intensity": round(fc1_ai, 1), "ridge_flop_per_byte": round(ridge, 1),
                         "mfma_tflops": round(fc1_tflops, 1), "mfma_frac": round(fc1_tflops / BF16_PEAK_TFLOPS, 4)})

    # whole-step floor: every weight (1.21 GB) must stream from HBM once per step
    step_bytes = dit.weight_bytes
    step_floor_ms = step_bytes / (HBM_PEAK_GBS * 1e9) * 1e3

    out = {
        "metric": "ms/DiT step (T=2 bf16) + FPS for 4-step DDIM+VAE frame on 1 MI355X",
        "value": round(ms_step, 4), "unit": "ms/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "config1: Oasis-500M DiT denoising step, latent [1,2,16,18,32], "
                               "16 blocks, D=1024, 16 heads, T=2 (288 tokens), bf16 weights, fp32 residual",
                   "global_batch": 1, "seq_len": 288, "parallelism": "none (1 GPU)"},
        "ms_per_step_gpu_events": round(ms_step_gpu, 4),
        "step_weight_bytes": step_bytes,
        "step_hbm_floor_ms": round(step_floor_ms, 4),
        "step_roofline_frac": round(step_floor_ms / ms_step, 4),
        "roofline": fc1_roofline,
        "roofline_hbm": {"kernel": "gemv_kernel<1,1,tiled> (weights in 16-row MFMA tile order, 1 KB contiguous per "
                                   "wave load, streaming loads), adaLN projections of the 32 sub-blocks (R=2 rows; the "
                                   "final layer's runs apart in fp32), 50 launches in one hipGraph alternating between "
                                   "two copies of the 403 MB weights (cold)",
                         "bound": "hbm", "achieved": round(ada_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ada_gbs / HBM_PEAK_GBS, 4), "traffic": TRAFFIC.get("gemv"),
                         "avg_launch_ms": round(ada_ms, 5), "algorithmic_bytes": ada_bytes},
        "roofline_bandwidth_kernels": bandwidth_kernels(pkg),
    }

    # ---------------- config 3: the DDIM + VAE frame ----------------
    if not args.no_frame:
        del step
        c3 = synth.config3()
        dit3 = pkg.DiT(c3["w"], "cuda")
        vae3 = pkg.VAE(c3["vw"], "cuda")
        fp = pkg.FramePipeline(dit3, vae3, c3["steps"], pkg.schedule.cosine_alphas_cumprod())
        noise = pkg.patchify_latent(c3["x_T"])[0]
        ctx = pkg.patchify_latent(c3["ctx_latent"])[0]
        fp.set_inputs(noise.cuda(), ctx.cuda(), c3["ctx_t"], c3["ctx_action"].cuda(), c3["gen_action"].cuda())
        fp.capture()
        for _ in range(max(3, args.warmup // 4)):
            fp.graph.launch()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.frames):
            fp.graph.launch()
        torch.cuda.synchronize()
        ms_frame = 1e3 * (time.perf_counter() - t0) / args.frames
        # per-frame host inputs (noise chunk, context patches, conditioning rows) over PCIe
        noise_h = noise.pin_memory()
        ctx_h = ctx.pin_memory()
        t0 = time.perf_counter()
        for _ in range(args.frames):
            # the copies go on the frame's own stream: a per-frame device-side wait between it
            # and torch's default stream costs ~0.5 ms here
            with torch.cuda.stream(fp.stream):
                fp.chunk.copy_(noise_h, non_blocking=True)
                fp.ctx_patches.copy_(ctx_h, non_blocking=True)
            fp.graph.launch()
        torch.cuda.synchronize()
        ms_frame_h2d = 1e3 * (time.perf_counter() - t0) / args.frames
        frame_floor_ms = (len(c3["steps"]) * dit3.weight_bytes + vae3.weight_bytes) / (HBM_PEAK_GBS * 1e9) * 1e3
        # the same frame with every DDIM step at T=2 (no temporal K/V cache)
        fp2 = pkg.FramePipeline(dit3, vae3, c3["steps"], pkg.schedule.cosine_alphas_cumprod(), kv_cache=False)
        fp2.set_inputs(noise.cuda(), ctx.cuda(), c3["ctx_t"], c3["ctx_action"].cuda(), c3["gen_action"].cuda())
        fp2.capture()
        for _ in range(3):
            fp2.graph.launch()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.frames):
            fp2.graph.launch()
        torch.cuda.synchronize()
        ms_frame_t2 = 1e3 * (time.perf_counter() - t0) / args.frames
        del fp2
        # steady state of a video: batches of 16 frames, each frame's context the previous
        # frame's latent (rolled on the device); with overlap_decode, batch k's VAE decodes run
        # on a second stream while batch k+1 denoises
        nv = 16
        ms_video = {}
        for overlap in (False, True):
            vp = pkg.VideoPipeline(dit3, vae3, c3["steps"], pkg.schedule.cosine_alphas_cumprod(), nv,
                                   overlap_decode=overlap)
            vp.set_inputs(noise.reshape(1, -1, 64).expand(nv, -1, -1).cuda(), ctx.cuda(), c3["ctx_t"],
                          c3["ctx_action"].cuda(), c3["gen_action"].reshape(1, -1).expand(nv, -1).cuda())
            vp.capture()
            vp.run()
            torch.cuda.synchronize()
            reps = max(4, args.frames // 8)
            t0 = time.perf_counter()
            for _ in range(reps):
                vp.launch()
            vp.drain()
            torch.cuda.synchronize()
            ms_video[overlap] = 1e3 * (time.perf_counter() - t0) / (reps * nv)
            del vp
        ms_video_frame = ms_video[False]
        # the interactive loop (PlaySession, play.py:241-531): one frame per action, each frame
        # drawing its noise, writing its conditioning rows, replaying the frame graph, rolling
        # the context and waiting for the frame on the host
        sess = pkg.PlaySession(dit3, vae3, c3["ctx_latent"], ddim_steps=len(c3["steps"]),
                               alphas_cumprod=pkg.schedule.cosine_alphas_cumprod(), seed=1)
        for _ in range(3):
            sess.frame(c3["gen_action"])
        t0 = time.perf_counter()
        for _ in range(args.frames):
            sess.frame(c3["gen_action"])
        ms_play = 1e3 * (time.perf_counter() - t0) / args.frames
        del sess
        out["frame_ms"] = round(ms_frame, 4)
        out["frame_fps"] = round(1e3 / ms_frame, 1)
        out["frame_hbm_floor_ms"] = round(frame_floor_ms, 4)
        out["frame_roofline_frac"] = round(frame_floor_ms / ms_frame, 4)
        out["frame_fps_with_h2d"] = round(1e3 / ms_frame_h2d, 1)
        out["frame_fps_all_t2"] = round(1e3 / ms_frame_t2, 1)
        out["video_fps"] = round(1e3 / ms_video_frame, 1)
        out["video_fps_overlap_decode"] = round(1e3 / ms_video[True], 1)
        out["play_fps"] = round(1e3 / ms_play, 1)
        out["video_workload"] = ("batches of 16 consecutive frames, within a batch each frame's context = the "
                                 "previous frame's denoised latent rolled on the device; the timed batches are "
                                 "repeated replays of one batch's graph (each replay starts from the same first "
                                 "context and denoises the chunk buffers in place; the work is data-independent); "
                                 "video_fps: one hipGraph per batch (the 16 frames' DDIM "
                                 "steps, then their 16 decodes as one batched VAE pass of 16 x 576 tokens); "
                                 "video_fps_overlap_decode: the batch's DDIM steps and its batched decodes as two "
                                 "single-stream hipGraphs on two streams, batch k's decodes (launched once its DDIM "
                                 "steps are done) overlapping batch k+1's DDIM steps")
        out["play_workload"] = ("interactive loop (PlaySession): one config-3 frame per action, host-synchronised "
                                "per frame; one hipGraph per frame holding the noise draw (Philox on the device), "
                                "the DDIM steps and decode, the [360,640,3] conversion to [0,1] and the context "
                                "roll; action rows uploaded when they change, the frame copied out")
        out["frame_workload"] = ("config3: 4 DDIM v-prediction steps (t=999,749,499,249, cosine alphas) "
                                 "over the DiT (step 1 at T=2 storing the context frame's temporal K/V, steps "
                                 "2-4 on the generated frame at T=1 against that cache; frame_fps_all_t2: every "
                                 "step at T=2) + bridge + 12-block ViT VAE decode + unpatchify to [3,360,640], "
                                 "one hipGraph")

    if not args.no_c4:
        fp = dit3 = vae3 = None  # release the config-3 model before loading configs 2 and 4
        torch.cuda.empty_cache()
        out["config2"] = config2(pkg)
        out["config4"] = config4(pkg, max(10, args.steps // 4), max(3, args.warmup // 4))

    if not args.no_cpu_baseline:
        import oracle  # the CPU baseline's leg only: the GPU path above never touches it
        out["cpu_baseline"] = cpu_baseline(c1, oracle, pkg)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
