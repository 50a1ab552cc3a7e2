"""ctypes binding of ``librwkv7_hip.so`` (declared in ``include/rwkv7_hip.h``).

The library is loaded after ``torch`` so that its ``libamdhip64.so.7``
dependency binds to the HIP runtime torch already loaded: device pointers and
stream handles from torch are then valid inside the library. There is no
fallback: if the library is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must be imported before the HIP library)

LIB_NAME = "librwkv7_hip.so"
ABI_VERSION = 11

# rwkv7_model.flags
MODEL_MULTI_LAUNCH_DECODE = 1
MODEL_INT8_DECODE = 2
MODEL_BF16 = 4

# enum indices of the per-layer fp32 vector block (RWKV7_V_*)
VEC_NAMES = (
    "ln1_w", "ln1_b", "x_r", "x_w", "x_k", "x_v", "x_a", "x_g", "w0", "a0", "v0",
    "k_k", "k_a", "r_k", "lnx_w", "lnx_b", "ln2_w", "ln2_b", "ffn_x_k",
)
NVEC = len(VEC_NAMES)

ERRORS = {1: "EINVAL", 2: "ESHAPE", 3: "EWORKSPACE", 4: "ELAUNCH"}

# exported symbols, in header order
SYMBOLS = (
    "rwkv7_abi_version",
    "rwkv7_strerror",
    "rwkv7_layer_layout_get",
    "rwkv7_head_q_scale_offset",
    "rwkv7_workspace_bytes",
    "rwkv7_workspace_errors",
    "rwkv7_decode_launches",
    "rwkv7_step_f32_activations",
    "rwkv7_decode",
    "rwkv7_decode_noalloc",
    "rwkv7_prefill",
    "rwkv7_wkv7",
    "rwkv7_wkv7_chunked_workspace_bytes",
    "rwkv7_wkv7_chunked",
    "rwkv7_wkv7_f32",
    "rwkv7_wkv7_backward",
    "rwkv7_layernorm",
    "rwkv7_lerp",
    "rwkv7_gemv_f16",
    "rwkv7_gemv_i8",
    "rwkv7_gemv_any4",
    "rwkv7_gemm_f16",
    "rwkv7_w_gate",
    "rwkv7_v_gate",
    "rwkv7_a_kk_k",
    "rwkv7_gates",
    "rwkv7_rank_gemv",
    "rwkv7_l2norm_neg_kk_a",
    "rwkv7_gn_rkrk",
    "rwkv7_sample_workspace_bytes",
    "rwkv7_sample",
)


class Dims(ctypes.Structure):
    _fields_ = [
        ("n_layer", ctypes.c_int32),
        ("n_embd", ctypes.c_int32),
        ("n_head", ctypes.c_int32),
        ("n_ffn", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("rank_w", ctypes.c_int32),
        ("rank_a", ctypes.c_int32),
        ("rank_v", ctypes.c_int32),
        ("rank_g", ctypes.c_int32),
    ]


class LayerLayout(ctypes.Structure):
    _fields_ = [
        (n, ctypes.c_int64)
        for n in ("w_rkv", "w_lora1", "w_lora2", "w_o", "w_fk", "w_fv", "vec", "bytes", "f_rkv")
    ] + [("f_l1", ctypes.c_int64 * 4), ("f_l2", ctypes.c_int64 * 4)] + [
        (n, ctypes.c_int64) for n in ("f_o", "f_fk", "f_fv", "frag_bytes", "q_rkv", "q_o", "q_fk", "q_fv",
                                      "q_scale", "q_bytes")
    ]


class Model(ctypes.Structure):
    _fields_ = [
        ("dims", Dims),
        ("layers", ctypes.c_void_p),
        ("emb", ctypes.c_void_p),
        ("head", ctypes.c_void_p),
        ("ln_out", ctypes.c_void_p),
        ("layers_frag", ctypes.c_void_p),
        ("head_frag", ctypes.c_void_p),
        ("flags", ctypes.c_uint32),
        ("layers_q", ctypes.c_void_p),
        ("head_q", ctypes.c_void_p),
    ]


class StateDesc(ctypes.Structure):
    _fields_ = [
        ("tmix_x", ctypes.c_void_p),
        ("rnn", ctypes.c_void_p),
        ("cmix_x", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
    ]


class GatesIO(ctypes.Structure):
    """``rwkv7_gates_io``: operands of ``rwkv7_gates`` (all f16 device pointers)."""

    _fields_ = [
        (n, ctypes.c_void_p)
        for n in (
            "vr", "wr", "ar", "gr", "v2t", "w2t", "a2t", "g2t",
            "v", "v_first", "k", "v0", "w0", "a0", "k_k", "k_a",
            "v_out", "w_out", "a_out", "kk_out", "k_out", "g_out",
        )
    ]


class Sampling(ctypes.Structure):
    """``rwkv7_sampling``: parameters of one ``rwkv7_sample`` call."""

    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_int32),
        ("top_p", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
        ("seed", ctypes.c_uint64),
        ("offset", ctypes.c_uint64),
    ]


class HipError(RuntimeError):
    """A nonzero return code from the HIP library."""


def lib_path() -> Path:
    env = os.environ.get("RWKV7_HIP_LIB")
    if env:
        return Path(env)
    return Path(__file__).resolve().parent / LIB_NAME


_LIB: ctypes.CDLL | None = None


def _declare(lib: ctypes.CDLL) -> None:
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    sig = {
        "rwkv7_abi_version": (ctypes.c_int, []),
        "rwkv7_strerror": (ctypes.c_char_p, [ctypes.c_int]),
        "rwkv7_layer_layout_get": (ctypes.c_int, [ctypes.POINTER(Dims), ctypes.POINTER(LayerLayout)]),
        "rwkv7_head_q_scale_offset": (i64, [ctypes.POINTER(Dims)]),
        "rwkv7_workspace_bytes": (i64, [ctypes.POINTER(Dims), i32, i32]),
        "rwkv7_workspace_errors": (ctypes.c_int, [vp, i64, ctypes.POINTER(ctypes.c_uint32), vp]),
        "rwkv7_decode_launches": (ctypes.c_int, [ctypes.POINTER(Model), i32, i32]),
        "rwkv7_step_f32_activations": (ctypes.c_int, [ctypes.POINTER(Model), i32, i32]),
        "rwkv7_decode": (ctypes.c_int, [ctypes.POINTER(Model), ctypes.POINTER(StateDesc), vp, vp, vp, i64, vp]),
        "rwkv7_decode_noalloc": (ctypes.c_int, [ctypes.POINTER(Model), ctypes.POINTER(StateDesc), vp, vp, vp]),
        "rwkv7_prefill": (ctypes.c_int, [ctypes.POINTER(Model), ctypes.POINTER(StateDesc), vp, i32, vp, i64, vp]),
        "rwkv7_wkv7": (ctypes.c_int, [vp, vp, vp, i32, vp, vp, vp, vp, vp, i32, i32, i32, i32, vp]),
        "rwkv7_wkv7_chunked_workspace_bytes": (ctypes.c_int64, [i32, i32, i32]),
        "rwkv7_wkv7_chunked": (ctypes.c_int, [vp, vp, vp, i32, vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, i64, vp]),
        "rwkv7_wkv7_f32": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, vp]),
        "rwkv7_wkv7_backward": (ctypes.c_int, [vp] * 17 + [i32, i32, i32, vp]),
        "rwkv7_layernorm": (ctypes.c_int, [vp, i32, vp, vp, vp, i32, i32, i32, vp]),
        "rwkv7_lerp": (ctypes.c_int, [vp, vp, vp, i32, vp, vp, i32, i32, vp]),
        "rwkv7_gemv_f16": (ctypes.c_int, [vp, vp, i64, vp, i32, i32, i32, vp]),
        "rwkv7_gemv_i8": (ctypes.c_int, [vp, vp, i64, vp, vp, i32, i32, vp]),
        "rwkv7_gemv_any4": (ctypes.c_int, [vp, vp, i64, vp, vp, i32, i32, vp]),
        "rwkv7_gemm_f16": (ctypes.c_int, [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, i32, vp]),
        "rwkv7_w_gate": (ctypes.c_int, [vp, vp, vp, i32, i32, vp]),
        "rwkv7_v_gate": (ctypes.c_int, [vp, vp, vp, vp, vp, i32, i32, vp]),
        "rwkv7_a_kk_k": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, vp]),
        "rwkv7_gates": (ctypes.c_int, [ctypes.POINTER(GatesIO), i32, i32, i32, i32, i32, i32, vp]),
        "rwkv7_rank_gemv": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp]),
        "rwkv7_l2norm_neg_kk_a": (ctypes.c_int, [vp, vp, vp, vp, i32, i32, vp]),
        "rwkv7_gn_rkrk": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, vp]),
        "rwkv7_sample_workspace_bytes": (i64, [i32, i32]),
        "rwkv7_sample": (ctypes.c_int, [vp, i32, i64, i32, i32, ctypes.POINTER(Sampling), vp, i64, i32, vp, vp, i64,
                                        vp, i64, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    p = Path(path) if path else lib_path()
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is not built; run `python rwkv-tl_amd/build_hip.py` "
            "(or __graft_entry__.build()) first"
        )
    lib = ctypes.CDLL(str(p), mode=ctypes.RTLD_GLOBAL)
    _declare(lib)
    ver = lib.rwkv7_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"{p}: ABI version {ver}, expected {ABI_VERSION}")
    _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    """Raise ``HipError`` for a nonzero return code."""
    if rc != 0:
        msg = _LIB.rwkv7_strerror(rc).decode() if _LIB is not None else ERRORS.get(rc, "?")
        raise HipError(f"{what} failed: {msg} (code {rc})")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle() -> int:
    """The current torch stream as a hipStream_t (captured by HIP graphs)."""
    return torch.cuda.current_stream().cuda_stream
