"""Writes tests/golden/rope_reference.safetensors: rotary-embedding vectors computed by the
reference's own restatement of rotary_embedding_torch, the functions ref_rotate_queries_or_keys,
ref_get_axial_freqs and ref_apply_rotary_emb of /root/reference/tests/test_rope.py:12-53.

Those functions fix what the oracle's closed-form checks leave open: the temporal positions past
frame 0 (arange(T), not a normalised position), the axial split of the spatial angles, and the
pair layout of the rotation. The reference module imports only torch, einops and safetensors at
its top and keeps its checkpoint scan under ``if __name__ == "__main__"``, so loading it defines
the functions and runs nothing else.

Run in the build container only (the reference is not on the GPU box); the fixture holds the
seeded inputs and the reference's outputs, nothing of the reference's code:

    python tests/golden/make_rope_golden.py
"""
import importlib.util
import os

import torch
from safetensors.torch import load_file, save_file

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "rope_reference.safetensors")
REFERENCE = "/root/reference/tests/test_rope.py"

TEMPORAL_T = (5, 32)
SPATIAL_GRID = (9, 16)
VAE_GRID = (18, 32)


def theta_freqs(n, dim):
    """1 / 10000^(2k / dim), k < n (the synthetic frequencies the build's weights use)."""
    return 1.0 / 10000.0 ** (torch.arange(0, 2 * n, 2, dtype=torch.float64) / dim)


def cases(seed=2024):
    """Seeded inputs: frequency sets (theta-10000 and learned-like random ones) and rows to rotate."""
    g = torch.Generator().manual_seed(seed)
    c = {}
    c["temporal.theta.freqs"] = theta_freqs(32, 64).float()
    c["temporal.rand.freqs"] = torch.rand(32, generator=g) * 2
    for name in ("theta", "rand"):
        for T in TEMPORAL_T:
            c["temporal.%s.T%d.x" % (name, T)] = torch.randn(2, T, 64, generator=g)   # [heads, T, d]
    c["spatial.freqs"] = torch.rand(16, generator=g) * 3
    c["spatial.x"] = torch.randn(1, *SPATIAL_GRID, 64, generator=g)
    c["vae.freqs"] = torch.rand(8, generator=g) * 3          # the first 32 dims rotate
    c["vae.x"] = torch.randn(1, *VAE_GRID, 40, generator=g)  # 8 dims past them pass through
    return c


def _reference():
    spec = importlib.util.spec_from_file_location("_reference_tests_test_rope", REFERENCE)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def generate():
    ref = _reference()
    out = cases()
    for name in ("theta", "rand"):
        f = out["temporal.%s.freqs" % name]
        for T in TEMPORAL_T:
            x = out["temporal.%s.T%d.x" % (name, T)]
            out["temporal.%s.T%d.y" % (name, T)] = ref.ref_rotate_queries_or_keys(x, f)
    for key, grid in (("spatial", SPATIAL_GRID), ("vae", VAE_GRID)):
        ang = ref.ref_get_axial_freqs(out[key + ".freqs"], *grid)      # [gh, gw, 4F]
        if key == "spatial":
            out[key + ".angles"] = ang.contiguous()
        out[key + ".y"] = ref.ref_apply_rotary_emb(ang, out[key + ".x"]).contiguous()
    return {k: v.contiguous() for k, v in out.items()}


def load():
    return load_file(PATH)


if __name__ == "__main__":
    vec = generate()
    save_file(vec, PATH)
    print("wrote %s: %d tensors, %d bytes" % (PATH, len(vec), os.path.getsize(PATH)))
