"""CPU fp32 oracle for the Oasis-500M DiT step, DDIM loop, bridge and ViT VAE decoder.

TEST INFRASTRUCTURE ONLY. This package is the checker, never the thing measured
or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it. The product path (``open-oasis_amd``) runs
hand-written HIP kernels and raises if its shared library is missing; it never
falls back to anything in here.

Every function restates the reference algorithm in plain PyTorch fp32 on the CPU
and cites the reference file:line it follows (paths relative to the
zoecarver/open-oasis root).

Pinning (what each function is checked against, in ``tests/test_oracle.py``):
  - layer_norm, gelu_tanh, gelu_erf, silu: torch.nn.functional and fp64 closed
    forms on scalars.
  - rope tables / apply_rope: rotate_half identity, pair-norm preservation,
    position-0 identity, the swap-column/sign trick of the reference tables,
    and the axial broadcast construction of tests/test_rope.py:32-45.
  - attention: fp64 brute-force softmax loops on tiny inputs, T=1 causal == V,
    constant-score == mean(V), causal bias mask == is_causal.
  - conditioning: fp64 scalar loops over the timestep MLP and action projection.
  - schedules: the telescoped closed forms of the sigmoid and cosine alpha-bar.
  - sub-blocks and the DiT step: fp64 loop-level restatement over frames, tokens
    and heads at small dims (D=128, 2 heads, 2x3 grid / T=3), and the
    KV-invariance property (context-frame rows do not depend on the generated
    frame).
  - DDIM: exact v-target recovers x0 and eps; last step returns x0.
  - bridge / patchify / unpatchify: permutation round trips.
  - VAE decoder: fp64 restatement of one block at D=128 on a 4x4 grid.
  - tests/golden/ holds known-answer vectors generated from this oracle (the
    reference ships none); tests/test_golden.py checks the oracle still
    reproduces them.
    Parity unpinned for what only the absent upstream vae.py fixes (its RoPE
    frequencies and GELU flavour): those are synthesised from the build's
    stated configuration, not from the real model.
"""
from .oasis_ref import *  # noqa: F401,F403
