"""ctypes binding of liboasis_hip.so (the C ABI declared in include/oasis_hip.h).

The library is loaded from ``lib/liboasis_hip.so`` next to this file. There is no
fallback: if it is missing, or no GPU is visible when a kernel is called, the call
raises. Build it with ``python open-oasis_amd/build.py`` (or ``__graft_entry__.build()``).
"""
import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "liboasis_hip.so")

OASIS_OK = 0
F32, BF16 = 0, 1
MAX_SUB = 64

EPI_STORE_F32, EPI_STORE_BF16, EPI_GELU_TANH, EPI_GELU_ERF = 0, 1, 2, 3
EPI_GATED_RES, EPI_RESIDUAL, EPI_QKV_ROPE, EPI_UNPATCHIFY = 4, 5, 6, 7
EPI_PARTIAL_F32, EPI_GELU_TANH_FP8, EPI_GELU_TANH_FRAG = 8, 9, 10
EPI_GATED_RES_LN, EPI_GELU_TANH_LN = 11, 12
FRAG_QKV, FRAG_O, FRAG_FC1, FRAG_FC2, FRAG_LN = 1, 2, 4, 8, 16
ACT_NONE, ACT_SILU, ACT_TEMB = 0, 1, 2
ABI_VERSION = 6
WEIGHTS_BF16, WEIGHTS_FP8 = 0, 1


class OasisError(RuntimeError):
    """A liboasis_hip call returned an error code."""

    def __init__(self, fn, code, msg):
        super().__init__("%s failed (code %d): %s" % (fn, code, msg))
        self.code = code


c_p = ctypes.c_void_p
c_i64 = ctypes.c_int64
c_i = ctypes.c_int
c_f = ctypes.c_float


class Epilogue(ctypes.Structure):
    _fields_ = [
        ("kind", c_i), ("n_heads", c_i), ("bias", c_p), ("out_f32", c_p), ("out_bf16", c_p),
        ("ld_out", c_i64), ("gate", c_p), ("gate_fstride", c_i64), ("rows_per_frame", c_i64),
        ("frames_per_stream", c_i64), ("q", c_p), ("k", c_p), ("v", c_p), ("rope_cos", c_p),
        ("rope_sinp", c_p), ("rope_by_frame", c_i), ("unpatch_grid_w", c_i),
        ("s_b", c_i64), ("s_t", c_i64), ("s_p", c_i64), ("s_h", c_i64),
        ("unpatch_patch", c_i), ("unpatch_channels", c_i), ("split_stride", c_i64),
        ("out_fp8", c_p), ("out_scale", c_p), ("ld_scale", c_i64),
        ("mod_scale", c_p), ("mod_shift", c_p), ("ln_center", c_p), ("ln_stats", c_p), ("ln_mod", c_p),
        ("ln_eps", c_f),
        ("out_frag", c_i),
    ]


class DiTWeights(ctypes.Structure):
    _fields_ = [
        ("n_sub", c_i), ("d_model", c_i), ("n_heads", c_i), ("d_mlp", c_i), ("grid_h", c_i),
        ("grid_w", c_i), ("patch_dim", c_i), ("freq_dim", c_i), ("ext_dim_pad", c_i),
        ("ada_w", c_p), ("ada_b", c_p), ("final_ada_w", c_p), ("final_ada_b", c_p),
        ("qkv_w", c_p * MAX_SUB), ("out_w", c_p * MAX_SUB), ("out_b", c_p * MAX_SUB),
        ("fc1_w", c_p * MAX_SUB), ("fc1_b", c_p * MAX_SUB), ("fc2_w", c_p * MAX_SUB),
        ("fc2_b", c_p * MAX_SUB),
        ("final_w", c_p), ("final_b", c_p), ("xemb_w", c_p), ("xemb_b", c_p),
        ("temb_w0", c_p), ("temb_b0", c_p), ("cond_w", c_p), ("cond_b", c_p),
        ("s_cos", c_p), ("s_sinp", c_p), ("t_cos", c_p), ("t_sinp", c_p), ("t_max", c_i),
        ("weight_format", c_i), ("qkv_s", c_p * MAX_SUB), ("out_s", c_p * MAX_SUB), ("fc1_s", c_p * MAX_SUB),
        ("fc2_s", c_p * MAX_SUB),
        ("qkv_wf", c_p * MAX_SUB), ("out_wf", c_p * MAX_SUB), ("fc1_wf", c_p * MAX_SUB), ("fc2_wf", c_p * MAX_SUB),
    ]


class DiTBuffers(ctypes.Structure):
    _fields_ = [("max_rows", c_i64), ("x", c_p), ("h", c_p), ("q", c_p), ("k", c_p), ("v", c_p),
                ("attn", c_p), ("mlp", c_p), ("partial", c_p), ("max_splits", c_i64),
                ("act8", c_p), ("act8_scale", c_p), ("mlp8", c_p), ("mlp8_scale", c_p), ("frag_rows", c_i64),
                ("ln_mean", c_p), ("ln_stats", c_p), ("ln_mod", c_p)]


class KVCache(ctypes.Structure):
    _fields_ = [("k", c_p), ("v", c_p), ("max_streams", c_i64)]


class VAEWeights(ctypes.Structure):
    _fields_ = [
        ("depth", c_i), ("d_model", c_i), ("n_heads", c_i), ("d_mlp", c_i), ("latent_dim", c_i),
        ("grid_h", c_i), ("grid_w", c_i), ("patch", c_i),
        ("pq_w", c_p), ("pq_b", c_p),
        ("n1_w", c_p * MAX_SUB), ("n1_b", c_p * MAX_SUB), ("qkv_w", c_p * MAX_SUB),
        ("qkv_b", c_p * MAX_SUB), ("proj_w", c_p * MAX_SUB), ("proj_b", c_p * MAX_SUB),
        ("n2_w", c_p * MAX_SUB), ("n2_b", c_p * MAX_SUB), ("fc1_w", c_p * MAX_SUB),
        ("fc1_b", c_p * MAX_SUB), ("fc2_w", c_p * MAX_SUB), ("fc2_b", c_p * MAX_SUB),
        ("norm_w", c_p), ("norm_b", c_p), ("pred_w", c_p), ("pred_b", c_p),
        ("rope_cos", c_p), ("rope_sinp", c_p),
    ]


class VAEBuffers(ctypes.Structure):
    _fields_ = [("max_rows", c_i64), ("x", c_p), ("h", c_p), ("q", c_p), ("k", c_p), ("v", c_p), ("attn", c_p),
                ("mlp", c_p), ("partial", c_p), ("max_splits", c_i64)]


P = ctypes.POINTER
# name -> argtypes (every function returns int except oasis_last_error)
SIGNATURES = {
    "oasis_abi_version": [],
    "oasis_silu": [c_p, c_p, c_i64, c_i, c_p],
    "oasis_adaln_modulate": [c_p, c_p, c_p, c_p, c_i64, c_i, c_p],
    "oasis_gated_residual": [c_p, c_p, c_p, c_p, c_i64, c_i, c_p],
    "oasis_bias_gated_residual": [c_p, c_p, c_p, c_p, c_p, c_i64, c_i, c_p],
    "oasis_layernorm": [c_p, c_p, c_p, c_i64, c_p, c_i64, c_i64, c_f, c_i, c_p],
    "oasis_linear": [c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i, c_i, c_p],
    "oasis_adaln_matmul_expand": [c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_p],
    "oasis_rope_layout": [c_p, c_i64, c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_p, c_p, c_p,
                          c_i64, c_i64, c_i64, c_i64, c_i, c_i, c_p],
    "oasis_sdpa": [c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_f, c_p, c_i, c_i, c_p],
    "oasis_gemm_bf16": [c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_i64, P(Epilogue), c_p],
    "oasis_gemm_bf16_config": [c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_i64, P(Epilogue), c_i, c_i, c_p],
    "oasis_gemm_bf16_frag": [c_p, c_i64, c_p, c_i64, c_i64, c_i64, P(Epilogue), c_i, c_p],
    "oasis_dit_frag_plan": [c_i64],
    "oasis_gemm_fp8": [c_p, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_i64, P(Epilogue), c_i, c_i, c_p],
    "oasis_quantize_fp8_rows": [c_p, c_i64, c_i64, c_p, c_p, c_p],
    "oasis_gemm_fp8_a8": [c_p, c_i64, c_p, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_i64, P(Epilogue), c_i, c_i,
                          c_p],
    "oasis_quantize_act_fp8": [c_p, c_i64, c_i64, c_i64, c_p, c_i64, c_p, c_i64, c_p],
    "oasis_ln_modulate": [c_p, c_i64, c_i64, c_p, c_p, c_i64, c_i64, c_p, c_f, c_p],
    "oasis_ln_affine": [c_p, c_i64, c_i64, c_p, c_p, c_p, c_f, c_p],
    "oasis_residual_ln": [c_p, c_i64, c_i64, c_p, c_i, c_i64, c_p, c_p, c_i64, c_i64, c_p, c_p, c_i64, c_p,
                          c_f, c_p],
    "oasis_attention": [c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_f, c_p],
    "oasis_temporal_attention": [c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_f, c_p],
    "oasis_attention_fp8": [c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_f, c_p],
    "oasis_temporal_attention_fp8": [c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_f, c_p],
    "oasis_temporal_qkv_attention": [c_p, c_i64, c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_p, c_p, c_p, c_p, c_f,
                                     c_p],
    "oasis_gemv_bf16": [c_p, c_i64, c_i64, c_p, c_i64, c_i64, c_p, c_p, c_i64, c_i, c_i, c_i, c_p],
    "oasis_gemv_bf16_tiled": [c_p, c_i64, c_i64, c_p, c_i64, c_i64, c_p, c_p, c_i64, c_i, c_i, c_i, c_p],
    "oasis_gemv_f32": [c_p, c_i64, c_i64, c_p, c_i64, c_i64, c_p, c_p, c_i64, c_i, c_i, c_i, c_p],
    "oasis_timestep_embedding": [c_p, c_i64, c_i64, c_p, c_p],
    "oasis_noise_normal": [c_p, c_p, c_i64, ctypes.c_uint64, c_p, c_f, c_p],
    "oasis_frame_hwc": [c_p, c_p, c_i64, c_i64, c_i64, c_p],
    "oasis_small_linear": [c_p, c_i64, c_i64, c_i64, c_p, c_i, c_i, c_i64, c_p, c_p, c_i64, c_p],
    "oasis_ddim_update": [c_p, c_p, c_i64, c_f, c_f, c_f, c_f, c_f, c_f, c_p],
    "oasis_bridge": [c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_f, c_p],
    "oasis_vae_unpatchify": [c_p, c_p, c_i64, c_i64, c_i64, c_p],
    "oasis_dit_conditioning": [P(DiTWeights), c_p, c_p, c_i64, c_p, c_p, c_p, c_p],
    "oasis_dit_conditioning_noalloc": [P(DiTWeights), c_p, c_p, c_i64, c_p, c_p, c_p],
    "oasis_dit_forward": [P(DiTWeights), P(DiTBuffers), c_i64, c_i64, c_p, c_i64, c_p, c_p],
    "oasis_dit_sub_blocks": [P(DiTWeights), P(DiTBuffers), c_i64, c_i64, c_p, c_i64, c_i64, c_i64, c_p],
    "oasis_dit_final": [P(DiTWeights), P(DiTBuffers), c_i64, c_p, c_i64, c_p, c_p],
    "oasis_vae_decode": [P(VAEWeights), P(VAEBuffers), c_p, c_p, c_p],
    "oasis_vae_decode_batch": [P(VAEWeights), P(VAEBuffers), c_i64, c_p, c_p, c_p],
    "oasis_vae_decode_patches": [P(VAEWeights), P(VAEBuffers), c_i64, c_p, c_p, c_i64, c_p],
    "oasis_video_decode": [P(DiTWeights), P(VAEWeights), P(VAEBuffers), c_i64, c_p, c_p, c_p, c_p],
    "oasis_dit_step": [P(DiTWeights), P(DiTBuffers), c_i64, c_i64, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p],
    "oasis_ddim_frame": [P(DiTWeights), P(DiTBuffers), P(VAEWeights), P(VAEBuffers), P(KVCache), c_p, c_p, c_p,
                         c_p, c_i64, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p],
    "oasis_video_frames": [P(DiTWeights), P(DiTBuffers), P(VAEWeights), P(VAEBuffers), P(KVCache), c_i64, c_p, c_p,
                           c_p, c_p, c_i64, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p],
    "oasis_dit_precompute_past": [P(DiTWeights), P(DiTBuffers), P(KVCache), c_i64, c_p, c_i64, c_p],
    "oasis_dit_forward_current": [P(DiTWeights), P(DiTBuffers), P(KVCache), c_i64, c_p, c_i64, c_p, c_p],
    "oasis_graph_begin": [c_p],
    "oasis_graph_end": [c_p, P(c_p)],
    "oasis_graph_launch": [c_p, c_p],
    "oasis_graph_destroy": [c_p],
    "oasis_stream_sync": [c_p],
}

_LIB = None


def lib():
    """Load (once) and return the ctypes handle. Raises if the library is not built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError("liboasis_hip.so is not built (%s); run open-oasis_amd/build.py" % LIB_PATH)
        h = ctypes.CDLL(LIB_PATH)
        h.oasis_last_error.restype = ctypes.c_char_p
        h.oasis_last_error.argtypes = []
        h.oasis_abi_struct_size.restype = c_i64
        h.oasis_abi_struct_size.argtypes = [c_i]
        for name, argt in SIGNATURES.items():
            f = getattr(h, name)
            f.argtypes = argt
            f.restype = c_i
        _LIB = h
        if h.oasis_abi_version() != ABI_VERSION:
            _LIB = None
            raise ImportError("liboasis_hip.so has ABI version %d, this binding expects %d; rebuild it"
                              % (h.oasis_abi_version(), ABI_VERSION))
        check_struct_layouts()
    return _LIB


def exported_names():
    """Names of the C entry points this binding knows (all declared in oasis_hip.h)."""
    return ["oasis_last_error", "oasis_abi_struct_size"] + list(SIGNATURES)


STRUCTS = (Epilogue, DiTWeights, DiTBuffers, VAEWeights, VAEBuffers)


def check_struct_layouts():
    """Raise if a ctypes mirror's size differs from the C struct's."""
    h = lib()
    for i, st in enumerate(STRUCTS):
        c = h.oasis_abi_struct_size(i)
        if c != ctypes.sizeof(st):
            raise ImportError("ABI mismatch: %s is %d bytes in C, %d in ctypes" % (st.__name__, c, ctypes.sizeof(st)))


def call(name, *args):
    """Call an int-returning entry point and raise OasisError on a non-zero code."""
    h = lib()
    rc = getattr(h, name)(*args)
    if rc != OASIS_OK:
        raise OasisError(name, rc, h.oasis_last_error().decode(errors="replace"))
    return rc


def frag_plan(rows):
    """The library's fragment-order mask (FRAG_* bits) for DiT passes of `rows` tokens."""
    return lib().oasis_dit_frag_plan(rows)


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(stream=None):
    """hipStream_t of a torch stream (default: the current stream)."""
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)
