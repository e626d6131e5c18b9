"""The committed known-answer vectors (tests/golden/oasis_golden.safetensors) are still
what the oracle computes from the seeded cases (CPU only)."""
import os
import sys

import pytest
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden  # noqa: E402


@pytest.fixture(scope="module")
def golden():
    return make_golden.load()


@pytest.fixture(scope="module")
def fresh():
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    return make_golden.expected()


def test_fixture_holds_every_vector(golden, fresh):
    assert set(golden) == set(fresh)


@pytest.mark.parametrize("key", ["dit2.weights", "c0.weights", "vae2.weights", "frame2.weights"])
def test_seeded_weights_unchanged(golden, fresh, key):
    assert torch.allclose(fresh[key], golden[key], rtol=1e-12, atol=0), key


def test_oracle_reproduces_the_vectors(golden, fresh):
    for k, ref in golden.items():
        got = fresh[k]
        assert got.shape == ref.shape, k
        tol = 1e-5 * max(ref.double().abs().max().item(), 1e-30)
        err = (got.double() - ref.double()).abs().max().item()
        assert err <= tol, (k, err, tol)


def test_schedule_vectors_are_the_closed_forms(golden):
    import math
    f = lambda k: math.cos((k / 1000 + 0.008) / 1.008 * math.pi / 2) ** 2  # noqa: E731
    for i, k in enumerate((0, 249, 499, 749, 999)):
        assert abs(golden["sched.cosine"][i].item() - max(f(k + 1) / f(0), 0)) < 1e-5
