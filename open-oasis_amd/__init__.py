"""open-oasis_amd: MI355X-native (gfx950) Oasis-500M DiT denoising step and ViT VAE decoder.

Python host code over hand-written HIP kernels in liboasis_hip.so (C ABI in
include/oasis_hip.h). The directory name is not an identifier, so it is imported as
``open_oasis_amd`` through ``__graft_entry__.load_package()`` or ``tests/conftest.py``.
"""
from . import _lib  # noqa: F401
from ._lib import OasisError  # noqa: F401
from .model import DiT, VAE, DiTStep, FramePipeline, VideoPipeline, Graph  # noqa: F401
from .play import PlaySession, ActionHold, patchify_latent  # noqa: F401
from . import checkpoint, kernels, schedule, synth  # noqa: F401
