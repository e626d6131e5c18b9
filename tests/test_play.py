"""Host logic of the interactive frame loop (open-oasis_amd/play.py) on the CPU: the action
hold of the reference's read_action (play.py:80-100) and the patch layout of the prompt."""
import pytest
import torch

import oracle
from helpers import pkg

play = pkg.play


def test_action_hold_keeps_the_last_action_one_frame_after_a_release():
    hold = play.ActionHold(25, hold=1)
    a, b, z = torch.zeros(25), torch.zeros(25), torch.zeros(25)
    a[3], b[7] = 1.0, 1.0
    seq = [hold(x) for x in (a, z, z, b, b, z, z)]
    expect = [a, a, z, b, b, b, z]
    for i, (got, want) in enumerate(zip(seq, expect)):
        assert torch.equal(got, want), i


def test_action_hold_zero_frames_passes_actions_through():
    hold = play.ActionHold(25, hold=0)
    a, z = torch.zeros(25), torch.zeros(25)
    a[1] = 1.0
    assert torch.equal(hold(a), a) and torch.equal(hold(z), z)


def test_patchify_latent_matches_the_oracle_layout():
    g = torch.Generator().manual_seed(3)
    lat = torch.randn(16, 18, 32, generator=g)
    got = play.patchify_latent(lat)
    assert got.shape == (144, 64)
    assert torch.equal(got, oracle.patchify_to_output_space(lat[None])[0])
    # leading dims (streams, frames) are kept
    lat4 = torch.randn(2, 3, 16, 18, 32, generator=g)
    got4 = play.patchify_latent(lat4)
    assert got4.shape == (2, 3, 144, 64)
    assert torch.equal(got4, oracle.patchify_to_output_space(lat4.reshape(6, 16, 18, 32)).reshape(2, 3, 144, 64))


def test_session_rejects_a_batch_of_prompts():
    """Only one prompt frame: leading dims of size 1 are dropped, anything else is an error
    (raised before any device work)."""

    class Fake:
        device = torch.device("cpu")
        ext_dim = 25

    with pytest.raises(ValueError, match="one frame"):
        play.PlaySession(Fake(), None, torch.zeros(2, 16, 18, 32))
