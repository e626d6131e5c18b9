"""Noise schedules, DDIM timesteps and DDIM coefficients (host-side scalars).

The coefficients are baked into the captured frame graph as kernel arguments, as the
reference uploads them once per frame into fixed device tensors
(oasis_inference.py:1843-1860,2194-2201).
"""
import math

import torch


def sigmoid_alphas_cumprod(timesteps=1000, start=-3.0, end=3.0, tau=1.0):
    """Sigmoid schedule of oasis_inference.py:313-321, cumprod at 1769-1771."""
    t = torch.linspace(0, timesteps, timesteps + 1, dtype=torch.float64) / timesteps
    v_start = torch.tensor(start / tau).sigmoid()
    v_end = torch.tensor(end / tau).sigmoid()
    ac = (-((t * (end - start) + start) / tau).sigmoid() + v_end) / (v_end - v_start)
    ac = ac / ac[0]
    betas = torch.clip(1 - ac[1:] / ac[:-1], 0, 0.999).float()
    return torch.cumprod(1.0 - betas, dim=0)


def cosine_alphas_cumprod(timesteps=1000, s=0.008):
    """Cosine schedule (Nichol & Dhariwal 2021) with betas clipped to 0.999."""
    x = torch.linspace(0, timesteps, timesteps + 1, dtype=torch.float64)
    ac = torch.cos(((x / timesteps) + s) / (1 + s) * math.pi * 0.5) ** 2
    ac = ac / ac[0]
    betas = torch.clip(1 - ac[1:] / ac[:-1], 0, 0.999).float()
    return torch.cumprod(1.0 - betas, dim=0)


def ddim_steps(n_steps, max_noise_level=1000):
    """[(t, t_next)] from ``linspace(-1, max-1, n+1)`` walked backwards (oasis_inference.py:1765)."""
    nr = torch.linspace(-1, max_noise_level - 1, n_steps + 1)
    return [(int(nr[i].item()), int(nr[i - 1].item())) for i in range(n_steps, 0, -1)]


def ddim_coefficients(alphas_cumprod, steps):
    """Flat list of 6 floats per step in the order the device update expects:
    sqrt(a), sqrt(1-a), sqrt(1/a), 1/sqrt(1/a - 1), sqrt(a'), sqrt(1-a'); a' = 1 on the last
    step (oasis_inference.py:1843-1860)."""
    out = []
    for i, (t, tn) in enumerate(steps):
        at = float(alphas_cumprod[t].item())
        an = 1.0 if i == len(steps) - 1 else float(alphas_cumprod[max(tn, 0)].item())
        out += [at ** 0.5, (1 - at) ** 0.5, (1.0 / at) ** 0.5, 1.0 / ((1.0 / at - 1) ** 0.5),
                an ** 0.5, (1 - an) ** 0.5]
    return out
