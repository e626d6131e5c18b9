"""RoPE against the reference's own restatement of rotary_embedding_torch (CPU only).

tests/golden/rope_reference.safetensors holds vectors that ref_rotate_queries_or_keys,
ref_get_axial_freqs and ref_apply_rotary_emb (/root/reference/tests/test_rope.py:12-53) computed
from seeded inputs (tests/golden/make_rope_golden.py wrote them in the build container). The
oracle's angle builders and rotation, and the model's device tables that the GPU kernels read,
must reproduce them: the temporal positions past frame 0, the axial split of the spatial and VAE
angles, the pair layout and the sign of the rotation. Planted mistakes in those places fail.
"""
import os
import sys

import pytest
import torch

import oracle
from helpers import pkg

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_rope_golden  # noqa: E402

M = pkg.model
TOL = 1e-5


@pytest.fixture(scope="module")
def vec():
    return make_rope_golden.load()


def _err(a, b):
    a, b = a.double(), b.double()
    return (a - b).abs().max().item() / max(b.abs().max().item(), 1e-30)


def _pairs(a):
    return a.repeat_interleave(2, dim=-1)


def test_fixture_inputs_are_the_seeded_cases(vec):
    for k, t in make_rope_golden.cases().items():
        assert torch.equal(vec[k], t), k


def _temporal_err(vec, name, T, angles_fn):
    f, x, y = (vec["temporal.%s.%s" % (name, s)] for s in ("freqs", "T%d.x" % T, "T%d.y" % T))
    return _err(oracle.apply_rotary_emb(angles_fn(f, T), x), y)


@pytest.mark.parametrize("name", ["theta", "rand"])
@pytest.mark.parametrize("T", make_rope_golden.TEMPORAL_T)
def test_temporal_rope_matches_the_reference(vec, name, T):
    assert _temporal_err(vec, name, T, oracle.temporal_rope_angles) <= TOL
    f, x, y = (vec["temporal.%s.%s" % (name, s)] for s in ("freqs", "T%d.x" % T, "T%d.y" % T))
    # the device formulation (x*cos + swap(x)*sin_perm) on the oracle's and on the model's tables
    cos, sp = oracle.rope_cos_sinperm(oracle.temporal_rope_angles(f, T), 64)
    assert _err(oracle.apply_rope_swap(x, cos, sp), y) <= TOL
    mc, ms = M.rope_tables(M.temporal_angles(f, T))
    assert _err(oracle.apply_rope_swap(x, mc, ms), y) <= TOL


@pytest.mark.parametrize("T", make_rope_golden.TEMPORAL_T)
def test_temporal_rope_planted_mistakes_fail(vec, T):
    planted = {
        "normalised positions arange(T)/(T-1)":
            lambda f, T: _pairs((torch.arange(T) / (T - 1))[:, None] * f[None]),
        "positions from 1": lambda f, T: _pairs(torch.arange(1, T + 1.0)[:, None] * f[None]),
        "frequencies tiled instead of paired": lambda f, T: (torch.arange(T * 1.0)[:, None] * f[None]).repeat(1, 2),
        "rotation sign": lambda f, T: -oracle.temporal_rope_angles(f, T),
    }
    for name, fn in planted.items():
        assert _temporal_err(vec, "rand", T, fn) > 1e-2, name


def test_spatial_rope_matches_the_reference(vec):
    f, x, y = vec["spatial.freqs"], vec["spatial.x"].reshape(144, 64), vec["spatial.y"].reshape(144, 64)
    ang = oracle.spatial_rope_angles(f, 9, 16)
    assert _err(ang, vec["spatial.angles"].reshape(144, 64)) <= 1e-6
    assert _err(oracle.apply_rotary_emb(ang, x), y) <= TOL
    mc, ms = M.rope_tables(M._axial_angles(f, 9, 16))
    assert _err(oracle.apply_rope_swap(x, mc, ms), y) <= TOL
    # planted: the axes swapped (columns on dims 0-31), positions arange instead of linspace(-1, 1)
    swapped = ang.reshape(9, 16, 64).roll(32, dims=-1).reshape(144, 64)
    assert _err(oracle.apply_rotary_emb(swapped, x), y) > 1e-2
    hp, wp = torch.arange(9.0), torch.arange(16.0)
    ar = torch.cat([_pairs(hp[:, None] * f[None])[:, None].expand(9, 16, 32),
                    _pairs(wp[:, None] * f[None])[None].expand(9, 16, 32)], -1).reshape(144, 64)
    assert _err(oracle.apply_rotary_emb(ar, x), y) > 1e-2


def test_vae_rope_matches_the_reference(vec):
    """The VAE rotates the first 32 of each head's 64 dims over the 18 x 32 latent grid; the
    dims past them pass through (the fixture keeps 8 of them)."""
    f, x, y = vec["vae.freqs"], vec["vae.x"].reshape(576, 40), vec["vae.y"].reshape(576, 40)
    ang = oracle.vae_rope_angles(f, 18, 32)
    assert ang.shape == (576, 32)
    assert _err(oracle.apply_rotary_emb(ang, x), y) <= TOL
    mc, ms = M.rope_tables(M._axial_angles(f, 18, 32))
    x64 = torch.cat([x, torch.zeros(576, 24)], -1)
    assert _err(oracle.apply_rope_swap(x64, mc, ms)[:, :40], y) <= TOL
    assert torch.equal(y[:, 32:], x[:, 32:])
