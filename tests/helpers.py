"""Shared test helpers: the parity metrics, device shortcuts, and a host Philox4x32-10 (the
generator behind oasis_noise_normal) to check the device draws against."""
import sys

import numpy as np
import torch

pkg = sys.modules["open_oasis_amd"]
L = pkg._lib

# Tolerances of the north star: bf16 sub-blocks cos >= 0.999 and max relative error
# <= 2e-2; a full DDIM step cos >= 0.995. "Max relative error" is the largest absolute
# deviation divided by the largest reference magnitude.
COS_SUB = 0.999
REL_SUB = 2e-2
COS_STEP = 0.995


def metrics(got, ref):
    g = got.detach().float().cpu().flatten()
    r = ref.detach().float().cpu().flatten()
    cos = torch.nn.functional.cosine_similarity(g.double(), r.double(), dim=0).item()
    rel = ((g - r).abs().max() / r.abs().max().clamp_min(1e-30)).item()
    return cos, rel


def assert_close(got, ref, cos_min=COS_SUB, rel_max=REL_SUB, what=""):
    cos, rel = metrics(got, ref)
    print("%s: cos=%.7f max_rel=%.3e" % (what, cos, rel), flush=True)
    assert cos >= cos_min and rel <= rel_max, "%s: cos=%.7f rel=%.3e" % (what, cos, rel)
    return cos, rel


def bf(t):
    """Round to bf16 and back (what the kernels see of a bf16 operand)."""
    return t.to(torch.bfloat16).float()


def cuda(t, dtype=None):
    return t.to(device="cuda", dtype=dtype or t.dtype).contiguous()


def stream():
    return L.stream_handle()


def sync():
    torch.cuda.synchronize()


def philox4x32_10(ctr, key):
    """Philox4x32-10 (Salmon, Moraes, Dror and Shaw, SC 2011) on uint32 arrays: ctr [..., 4], key
    (k0, k1). Returns the [..., 4] output words."""
    m0, m1, w0, w1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57), 0x9E3779B9, 0xBB67AE85
    c = [np.asarray(ctr[..., i], dtype=np.uint64) for i in range(4)]
    k0, k1 = int(key[0]), int(key[1])
    mask = np.uint64(0xFFFFFFFF)
    for _ in range(10):
        p0, p1 = m0 * c[0], m1 * c[2]
        hi0, lo0, hi1, lo1 = p0 >> np.uint64(32), p0 & mask, p1 >> np.uint64(32), p1 & mask
        c = [hi1 ^ c[1] ^ np.uint64(k0), lo1, hi0 ^ c[3] ^ np.uint64(k1), lo0]
        k0, k1 = (k0 + w0) & 0xFFFFFFFF, (k1 + w1) & 0xFFFFFFFF
    return np.stack([x.astype(np.uint32) for x in c], -1)


def noise_reference(n, seed, frame, lim):
    """What oasis_noise_normal draws for frame counter `frame`: Box-Muller of Philox block
    (i // 4, frame) under key seed, clamped to +-lim (float64 on the host)."""
    q = np.arange((n + 3) // 4, dtype=np.uint64)
    ctr = np.stack([q & np.uint64(0xFFFFFFFF), q >> np.uint64(32), np.full_like(q, frame), np.zeros_like(q)], -1)
    x = philox4x32_10(ctr, (seed & 0xFFFFFFFF, seed >> 32))
    # the uniforms exactly as the device forms them in float32: ((float)x + 0.5f) * 2^-32
    u = ((x.astype(np.float32) + np.float32(0.5)) * np.float32(2.0 ** -32)).astype(np.float64)
    r0, r1 = np.sqrt(-2 * np.log(u[:, 0])), np.sqrt(-2 * np.log(u[:, 2]))
    t0, t1 = 2 * np.pi * u[:, 1], 2 * np.pi * u[:, 3]
    z = np.stack([r0 * np.cos(t0), r0 * np.sin(t0), r1 * np.cos(t1), r1 * np.sin(t1)], -1).reshape(-1)[:n]
    return np.clip(z, -lim, lim)
