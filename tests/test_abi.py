"""The C ABI library on the CPU: it loads, exports every entry point the header declares,
the ctypes mirrors match the C structs and argument lists, and argument validation
returns error codes with messages before any device work (no kernel runs here)."""
import ctypes
import os
import re

import pytest

from helpers import L

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "oasis_hip.h")

ERR_NULL, ERR_SHAPE, ERR_DTYPE, ERR_ARG = -1, -2, -3, -5


def _declarations():
    """name -> number of parameters, for every function declared in oasis_hip.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^(?:const char\*|int64_t|int|void)\s+(oasis_\w+)\s*\(([^)]*)\)\s*;", text, re.M):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


@pytest.fixture(scope="module")
def h():
    return L.lib()


def test_header_parses():
    decl = _declarations()
    assert len(decl) >= 35
    assert {"oasis_dit_step", "oasis_ddim_frame", "oasis_vae_decode", "oasis_sdpa", "oasis_linear"} <= set(decl)


def test_every_declared_symbol_is_exported(h):
    for name in _declarations():
        assert hasattr(h, name), "liboasis_hip.so does not export %s" % name


def test_binding_covers_the_header_with_matching_arity():
    decl = _declarations()
    assert set(L.exported_names()) == set(decl)
    for name, argt in L.SIGNATURES.items():
        assert len(argt) == decl[name], "%s: ctypes has %d args, header %d" % (name, len(argt), decl[name])


def test_abi_version_and_struct_sizes(h):
    assert h.oasis_abi_version() == L.ABI_VERSION == int(
        re.search(r"#define OASIS_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    for i, st in enumerate(L.STRUCTS):
        assert h.oasis_abi_struct_size(i) == ctypes.sizeof(st)
    assert h.oasis_abi_struct_size(99) == -1
    # the per-sub-block pointer arrays hold OASIS_MAX_SUB entries
    assert L.MAX_SUB == int(re.search(r"#define OASIS_MAX_SUB (\d+)", open(HEADER).read()).group(1))


def _rc(name, *args):
    h = L.lib()
    rc = getattr(h, name)(*args)
    return rc, h.oasis_last_error().decode()


FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails validation first


@pytest.mark.parametrize("name,args,code,needle", [
    ("oasis_silu", (None, FAKE, 16, 0, None), ERR_NULL, "null"),
    ("oasis_silu", (FAKE, FAKE, -1, 0, None), ERR_SHAPE, "negative"),
    ("oasis_silu", (FAKE, FAKE, 16, 7, None), ERR_DTYPE, "dtype"),
    ("oasis_gated_residual", (FAKE, FAKE, None, FAKE, 8, 0, None), ERR_NULL, "null"),
    ("oasis_timestep_embedding", (FAKE, 1, 255, FAKE, None), ERR_SHAPE, "shape"),
    ("oasis_small_linear", (FAKE, 512, 1, 512, FAKE, 0, 0, 64, None, FAKE, 64, None), ERR_SHAPE, ""),
    ("oasis_small_linear", (FAKE, 64, 1, 64, FAKE, 5, 0, 64, None, FAKE, 64, None), ERR_DTYPE, "w_dtype"),
    ("oasis_small_linear", (FAKE, 64, 1, 64, FAKE, 0, 2, 64, None, FAKE, 64, None), ERR_ARG, "w_layout"),
    ("oasis_gemv_f32", (FAKE, 64, 2, FAKE, 64, 62, None, FAKE, 64, 0, 0, 0, None), ERR_SHAPE, "multiple of 4"),
    ("oasis_gemv_f32", (FAKE, 64, 2, FAKE, 64, 64, None, FAKE, 64, 7, 0, 0, None), ERR_ARG, "activation"),
    ("oasis_rope_layout", (FAKE, 3 * 1024, FAKE, FAKE, 288, 144, 16, 32, FAKE, FAKE, FAKE, 1, 1, 1, 1, 0, 1, None),
     ERR_SHAPE, "head_dim"),
    ("oasis_bridge", (FAKE, FAKE, 0, 32, 16, 16, 1.0, None), ERR_SHAPE, "shape"),
    ("oasis_vae_unpatchify", (None, FAKE, 18, 32, 20, None), ERR_NULL, "null"),
    ("oasis_graph_launch", (None, None), ERR_NULL, ""),
])
def test_validation_errors(name, args, code, needle):
    rc, msg = _rc(name, *args)
    assert rc == code, (rc, msg)
    assert needle in msg.lower()


def test_empty_input_is_a_no_op():
    rc, _ = _rc("oasis_silu", FAKE, FAKE, 0, 0, None)
    assert rc == 0
    assert _rc("oasis_graph_destroy", None)[0] == 0  # destroying NULL is allowed


def test_gemm_validation():
    e = L.Epilogue(kind=L.EPI_STORE_F32, out_f32=FAKE, ld_out=64)
    rc, msg = _rc("oasis_gemm_bf16", FAKE, 96, FAKE, 96, 16, 64, 96, ctypes.byref(e), None)
    assert rc == ERR_SHAPE and "multiple of 64" in msg
    rc, msg = _rc("oasis_gemm_bf16", FAKE, 64, FAKE, 64, 16, 60, 64, ctypes.byref(e), None)
    assert rc == ERR_SHAPE and "multiple of 8" in msg
    rc, msg = _rc("oasis_gemm_bf16_config", FAKE, 256, FAKE, 256, 16, 64, 256, ctypes.byref(e), 0, 2, None)
    assert rc == ERR_ARG and "split" in msg.lower()
    rc, _ = _rc("oasis_gemm_bf16", None, 64, FAKE, 64, 16, 64, 64, ctypes.byref(e), None)
    assert rc == ERR_NULL


ODD = ctypes.c_void_p(0x1004)  # 4-byte but not 16-byte aligned


def test_misaligned_pointers_are_rejected():
    """Kernels move 16-byte vectors from their base pointers: a misaligned pointer is an
    argument error, never a launch."""
    e = L.Epilogue(kind=L.EPI_STORE_F32, out_f32=FAKE, ld_out=64)
    rc, msg = _rc("oasis_gemm_bf16", ODD, 64, FAKE, 64, 16, 64, 64, ctypes.byref(e), None)
    assert rc == ERR_ARG and "aligned" in msg, msg
    e = L.Epilogue(kind=L.EPI_STORE_F32, out_f32=ODD, ld_out=64)
    rc, msg = _rc("oasis_gemm_bf16", FAKE, 64, FAKE, 64, 16, 64, 64, ctypes.byref(e), None)
    assert rc == ERR_ARG and "aligned" in msg, msg
    rc, msg = _rc("oasis_attention", FAKE, ODD, FAKE, FAKE, 2, 144, 16, ctypes.c_float(0.125), None)
    assert rc == ERR_ARG and "aligned" in msg, msg
    rc, msg = _rc("oasis_residual_ln", ODD, 288, 1024, FAKE, 1, 288 * 1024, None, None, 0, 144, FAKE, FAKE, 0, FAKE,
                  ctypes.c_float(1e-6), None)
    assert rc == ERR_ARG and "aligned" in msg, msg
    rc, msg = _rc("oasis_gemv_bf16", FAKE, 64, 2, ODD, 64, 64, None, FAKE, 64, 0, 0, 0, None)
    assert rc == ERR_ARG and "aligned" in msg, msg


def test_model_entry_points_validate_structs():
    w = L.DiTWeights(n_sub=3, d_model=1024, n_heads=16)
    b = L.DiTBuffers()
    rc, msg = _rc("oasis_dit_sub_blocks", ctypes.byref(w), ctypes.byref(b), 1, 2, FAKE, 0, 0, 2, None)
    assert rc == ERR_SHAPE and "sub" in msg, msg
    vw = L.VAEWeights()
    rc, _ = _rc("oasis_vae_decode", ctypes.byref(vw), None, FAKE, FAKE, None)
    assert rc == ERR_NULL


def test_python_call_raises_with_the_message():
    with pytest.raises(L.OasisError) as ei:
        L.call("oasis_silu", None, FAKE, 16, 0, None)
    assert ei.value.code == ERR_NULL and "silu" in str(ei.value)
