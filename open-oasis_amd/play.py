"""Interactive frame loop: one generated frame per action, as the reference's play loop runs it
(play.py:241-531), without its file / HTTP interface to the browser UI (play_server.py).

- One captured frame graph per DDIM step count, kept once built. The reference releases its
  trace and re-traces when the slider changes ddim_steps (play.py:446-462). A change clamps
  the count to [1, 12] (play.py:55-56,103-108) and resets the context to the prompt and the
  frame index to 0, as the reference does.
- Each frame draws fresh noise, N(0, 1) clamped to +-noise_abs_max (play.py:466-472). Patchify
  is a permutation of iid noise, so it is drawn directly in patch space, on the device, by a
  counter-based generator (`oasis_noise_normal`: Philox4x32-10 keyed by the session's seed, its
  frame counter in device memory) inside the frame's graph.
- The context is the previous frame's denoised latent. Its conditioning is at
  stabilization_level - 1 with the previous frame's action (play.py:486-496); the first context
  is the prompt with the prompt action. After frame index k (k > 0, k % reset_every == 0) the
  context returns to the prompt (play.py:497-500).
- The action passes through the reference's hold: the last non-zero action is kept for
  `hold` frames after a release (read_action, play.py:80-100).
- Everything stays on the device. The context moves device-to-device. The frame comes back as
  [H, W, 3] in [0, 1], that is (x + 1) / 2 of the decoder's clamped output (play.py:476-480).
- One hipGraph per step count holds the whole frame: the noise draw, the DDIM steps and the
  decode, the [H, W, 3] conversion (`oasis_frame_hwc`) and the context roll. Per frame the host
  launches it, uploads the action rows when they change, and copies the frame out.
"""
import ctypes
import time

import torch

from . import _lib as L
from .model import FramePipeline, Graph
from .schedule import ddim_steps as ddim_schedule
from .schedule import sigmoid_alphas_cumprod

MIN_DDIM_STEPS, MAX_DDIM_STEPS = 1, 12   # play.py:55-56
NOISE_ABS_MAX = 20.0                     # play.py:58
STABILIZATION_LEVEL = 15                 # play.py:59
RESET_EVERY = 80                         # play.py:497
ACTION_HOLD = 1                          # play.py:83
FPS_WINDOW = 10                          # frames in the rolling FPS figure (play.py:519-522)


def patchify_latent(latent, patch=2):
    """[..., C, H, W] latent -> [..., (H/p)(W/p), p*p*C] patch rows with columns ordered
    (p, q, c), the reference's patchify_to_output_space (oasis_inference.py:958-963); leading
    dims (frames, streams) are kept."""
    *lead, C, H, W = latent.shape
    n = len(lead)
    x = latent.reshape(*lead, C, H // patch, patch, W // patch, patch)
    x = x.permute(*range(n), n + 1, n + 3, n + 2, n + 4, n)
    return x.reshape(*lead, (H // patch) * (W // patch), patch * patch * C)


class ActionHold:
    """The reference's read_action hold (play.py:80-100): a non-zero action is returned and
    remembered; after a release (all-zero action) the last non-zero one is returned for
    `hold` more frames."""

    def __init__(self, dim, hold=ACTION_HOLD):
        self.last = torch.zeros(dim)
        self.left = 0
        self.hold = hold

    def __call__(self, action):
        cur = torch.as_tensor(action, dtype=torch.float32).reshape(-1).cpu()
        if cur.abs().sum() > 0:
            self.last = cur.clone()
            self.left = self.hold
            return cur
        if self.left > 0:
            self.left -= 1
            return self.last
        return cur


class PlaySession:
    """Frame-by-frame generation driven by one action per frame.

    dit, vae: device-resident models. prompt_latent: [C, H, W] (or [1, C, H, W]) latent of the
    prompt frame; prompt_action: [ext_dim] (zeros by default, as play.py:193).
    alphas_cumprod defaults to the sigmoid schedule the play loop uses (play.py:188-191).
    frame(action) returns the decoded frame; status() gives frame_index / fps / ddim_steps as
    the reference's write_status does (play.py:121-126)."""

    def __init__(self, dit, vae, prompt_latent, prompt_action=None, ddim_steps=4, alphas_cumprod=None,
                 noise_abs_max=NOISE_ABS_MAX, stabilization_level=STABILIZATION_LEVEL,
                 reset_every=RESET_EVERY, hold=ACTION_HOLD, seed=0, kv_cache=True, stream=None,
                 keep_noise=False):
        lat = torch.as_tensor(prompt_latent, dtype=torch.float32)
        while lat.dim() > 3:
            if lat.shape[0] != 1:
                raise ValueError("prompt_latent: one frame [C, H, W] (leading dims of size 1 allowed), got %s"
                                 % (tuple(prompt_latent.shape),))
            lat = lat[0]
        dev = dit.device
        self.dit, self.vae, self.device = dit, vae, dev
        self.alphas = alphas_cumprod if alphas_cumprod is not None else sigmoid_alphas_cumprod()
        self.noise_abs_max = float(noise_abs_max)
        self.ctx_t = float(stabilization_level - 1)
        self.reset_every = int(reset_every)
        self.kv_cache = kv_cache
        self.keep_noise = keep_noise
        self.last_noise = None
        self.stream = stream if stream is not None else torch.cuda.Stream(device=dev)
        self.prompt = patchify_latent(lat).to(dev).contiguous()
        e = dit.ext_dim
        self.prompt_action = (torch.zeros(e) if prompt_action is None else
                              torch.as_tensor(prompt_action, dtype=torch.float32).reshape(e).clone())
        self.hold = ActionHold(e, hold)
        # the noise generator's key and its frame counter (bumped on the device by every draw)
        self.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        self.counter = torch.zeros(1, dtype=torch.int32, device=dev)
        P = dit.P
        self.noise_buf = torch.zeros(P, dit.patch_dim, device=dev) if keep_noise else None
        self.img_buf = torch.zeros(vae.frame_shape[1], vae.frame_shape[2], vae.frame_shape[0], device=dev)
        self.pipelines = {}
        self.graphs = {}
        # action rows go up through a pinned buffer; the event guards its reuse
        self.act_host = torch.zeros(1 + MAX_DDIM_STEPS, dit.ext_pad, pin_memory=True)
        self.act_copied = torch.cuda.Event()
        self.rows_key = None  # (pipeline, context action, action) of the rows on the device
        self.stream.wait_stream(torch.cuda.current_stream(dev))  # the prompt rows are ready
        self.set_ddim_steps(ddim_steps)

    def _pipeline(self, n):
        fp = self.pipelines.get(n)
        if fp is None:
            fp = FramePipeline(self.dit, self.vae, ddim_schedule(n), self.alphas, stream=self.stream,
                               kv_cache=self.kv_cache)
            # the timestep rows (context, then each DDIM step) are fixed for a step count
            t_rows = torch.tensor([self.ctx_t] + [float(t) for t, _ in fp.steps], dtype=torch.float32)
            with torch.cuda.stream(self.stream):
                fp.ws.t[:1 + n].copy_(t_rows)
            self.pipelines[n] = fp
            self.graphs[n] = Graph(lambda: self._enqueue(fp), self.stream)
        return fp

    def _enqueue(self, fp):
        """One frame on self.stream: noise into fp.chunk, the frame, its [H, W, 3] copy, and the
        context roll (this frame's denoised latent is the next context)."""
        h = L.stream_handle(self.stream)
        L.call("oasis_noise_normal", L.ptr(fp.chunk), L.ptr(self.noise_buf) if self.noise_buf is not None else None,
               fp.chunk.numel(), ctypes.c_uint64(self.seed), L.ptr(self.counter), self.noise_abs_max, h)
        fp.enqueue()
        C, H, W = self.vae.frame_shape
        L.call("oasis_frame_hwc", L.ptr(fp.vws.frame), L.ptr(self.img_buf), C, H, W, h)
        with torch.cuda.stream(self.stream):
            fp.ctx_patches.copy_(fp.chunk)

    def set_ddim_steps(self, n):
        """Switch to n DDIM steps per frame (clamped to [1, 12]); resets the context to the
        prompt and the frame index to 0."""
        n = max(MIN_DDIM_STEPS, min(MAX_DDIM_STEPS, int(n)))
        self.ddim_steps = n
        self.fp = self._pipeline(n)
        self.reset_context()
        self.frame_index = 0
        self.frame_times = []

    def reset_context(self):
        """The context window back to the prompt frame and the prompt action."""
        with torch.cuda.stream(self.stream):
            self.fp.ctx_patches.copy_(self.prompt)
        self.ctx_action = self.prompt_action.clone()

    def frame(self, action, sync=True):
        """Generate the next frame for `action` ([ext_dim]). Returns [H, W, 3] in [0, 1] on the
        device. sync=True waits for it on the host and counts the frame in the FPS figure;
        sync=False makes the caller's current stream wait for it instead."""
        t0 = time.perf_counter()
        a = self.hold(action)
        fp, n, e = self.fp, self.ddim_steps, self.dit.ext_dim
        R = 1 + n
        # the action rows go up only when they change: a host-to-device copy ahead of the
        # frame graph costs far more than the few hundred bytes it moves
        key = (id(fp), self.ctx_action.tolist(), a.tolist())
        upload = key != self.rows_key
        if upload:
            self.act_copied.synchronize()  # the previous copy out of act_host is done
            rows = self.act_host[:R]
            rows.zero_()
            rows[0, :e] = self.ctx_action
            rows[1:, :e] = a
            self.rows_key = key
        if upload:
            with torch.cuda.stream(self.stream):
                fp.ws.act[:R].copy_(rows, non_blocking=True)
                self.act_copied.record(self.stream)
        self.graphs[n].launch()
        with torch.cuda.stream(self.stream):
            img = self.img_buf.clone()
            if self.keep_noise:
                self.last_noise = self.noise_buf.clone()
        self.ctx_action = a.clone()
        cur = torch.cuda.current_stream(self.device)
        img.record_stream(cur)
        if self.frame_index > 0 and self.frame_index % self.reset_every == 0:
            self.reset_context()
        self.frame_index += 1
        if sync:
            self.stream.synchronize()
            self.frame_times = (self.frame_times + [time.perf_counter() - t0])[-FPS_WINDOW:]
        else:
            # a device-side wait of the caller's stream; with sync the host has already waited
            # (and a wait of the default stream per frame holds back the next frame's launches)
            cur.wait_stream(self.stream)
        return img

    @property
    def fps(self):
        return len(self.frame_times) / sum(self.frame_times) if self.frame_times else 0.0

    def status(self):
        """frame_index is the index of the last generated frame, numbered from 0 as the reference's
        write_status(frame_idx, ...) reports it before its frame_idx += 1 (play.py:517-525); -1
        before the first frame. self.frame_index counts the frames generated so far."""
        return {"frame_index": self.frame_index - 1, "fps": round(self.fps, 1), "ddim_steps": self.ddim_steps}
