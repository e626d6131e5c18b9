"""Shared test helpers: the parity metrics and device shortcuts."""
import sys

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
