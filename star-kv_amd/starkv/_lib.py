"""ctypes binding of libstarkv.so (the C ABI declared in include/starkv.h).

The library is the product: there is no Python or CPU fallback.  Loading
fails loudly when the shared object is missing.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libstarkv.so")

F16, BF16, F32, I8, U8 = 1, 2, 3, 4, 5
FMT_DENSE, FMT_INT4_REF, FMT_INT8_SYM, FMT_INT4_G64 = 0, 1, 2, 3

c_i64p = ctypes.POINTER(ctypes.c_int64)
c_intp = ctypes.POINTER(ctypes.c_int)


class StarKVError(RuntimeError):
    """Raised for a non-zero status from libstarkv or a missing library."""


class KLatent(ctypes.Structure):
    _fields_ = [
        ("n_kv_heads", ctypes.c_int),
        ("rank", c_intp),
        ("head_offset", c_i64p),
        ("pos_stride", c_i64p),
        ("stride_b", ctypes.c_int64),
        ("format", ctypes.c_int),
        ("data", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
        ("scale_stride_b", ctypes.c_int64),
        ("scale_stride_h", ctypes.c_int64),
        ("bk", ctypes.c_void_p),
        ("bk_head_offset", c_i64p),
        ("bk_row_stride", ctypes.c_int64),
        ("split", ctypes.c_int), ("split_format", ctypes.c_int),
        ("data2", ctypes.c_void_p),
        ("head_offset2", c_i64p),
        ("pos_stride2", c_i64p),
        ("stride2_b", ctypes.c_int64),
        ("scale2", ctypes.c_void_p),
        ("scale2_stride_b", ctypes.c_int64),
        ("scale2_stride_h", ctypes.c_int64),
    ]


class KLogitsDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int), ("n_q_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("seq_len", ctypes.c_int),
        ("dtype", ctypes.c_int),
        ("q", ctypes.c_void_p), ("q_stride_b", ctypes.c_int64), ("q_stride_h", ctypes.c_int64),
        ("k", KLatent),
        ("rope_table", ctypes.c_void_p), ("rope_max_positions", ctypes.c_int),
        ("scale", ctypes.c_float),
        ("mask", ctypes.c_void_p), ("mask_dtype", ctypes.c_int), ("mask_stride_b", ctypes.c_int64), ("mask_stride_h", ctypes.c_int64),
        ("out", ctypes.c_void_p), ("out_dtype", ctypes.c_int), ("out_stride_b", ctypes.c_int64), ("out_stride_h", ctypes.c_int64),
    ]


class VLatent(ctypes.Structure):
    _fields_ = [
        ("rank", ctypes.c_int),
        ("format", ctypes.c_int),
        ("data", ctypes.c_void_p), ("stride_b", ctypes.c_int64), ("stride_s", ctypes.c_int64),
        ("scale", ctypes.c_void_p), ("scale_stride_b", ctypes.c_int64), ("scale_stride_s", ctypes.c_int64),
        ("split", ctypes.c_int), ("split_format", ctypes.c_int),
        ("data2", ctypes.c_void_p), ("stride2_b", ctypes.c_int64), ("stride2_s", ctypes.c_int64),
        ("scale2", ctypes.c_void_p), ("scale2_stride_b", ctypes.c_int64), ("scale2_stride_s", ctypes.c_int64),
        ("zero", ctypes.c_void_p),
        ("capacity", ctypes.c_int),
    ]


class PVDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int), ("n_heads", ctypes.c_int), ("seq_len", ctypes.c_int),
        ("dtype", ctypes.c_int),
        ("p", ctypes.c_void_p), ("p_stride_b", ctypes.c_int64), ("p_stride_h", ctypes.c_int64),
        ("v", VLatent),
        ("out", ctypes.c_void_p), ("out_stride_b", ctypes.c_int64), ("out_stride_h", ctypes.c_int64),
    ]


class DecodeDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int), ("n_q_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("seq_len", ctypes.c_int),
        ("dtype", ctypes.c_int),
        ("q", ctypes.c_void_p), ("q_stride_b", ctypes.c_int64), ("q_stride_h", ctypes.c_int64),
        ("k", KLatent),
        ("v", VLatent),
        ("uv", ctypes.c_void_p), ("uv_row_stride", ctypes.c_int64),
        ("rope_table", ctypes.c_void_p), ("rope_max_positions", ctypes.c_int),
        ("scale", ctypes.c_float),
        ("mask", ctypes.c_void_p), ("mask_dtype", ctypes.c_int), ("mask_stride_b", ctypes.c_int64), ("mask_stride_h", ctypes.c_int64),
        ("out", ctypes.c_void_p), ("out_dtype", ctypes.c_int), ("out_stride_b", ctypes.c_int64), ("out_stride_h", ctypes.c_int64),
        ("last_pos_device", ctypes.c_void_p),
    ]


class KAppendDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int), ("n_tokens", ctypes.c_int), ("pos0", ctypes.c_int), ("capacity", ctypes.c_int),
        ("dtype", ctypes.c_int),
        ("src", ctypes.c_void_p), ("src_stride_b", ctypes.c_int64), ("src_stride_h", ctypes.c_int64),
        ("src_stride_t", ctypes.c_int64),
        ("k", KLatent),
        ("src_head_offset", ctypes.POINTER(ctypes.c_int64)),
        ("pos0_device", ctypes.c_void_p),
        ("error_flag", ctypes.c_void_p),
    ]


class VAppendDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int), ("n_tokens", ctypes.c_int), ("pos0", ctypes.c_int), ("capacity", ctypes.c_int),
        ("dtype", ctypes.c_int),
        ("src", ctypes.c_void_p), ("src_stride_b", ctypes.c_int64), ("src_stride_t", ctypes.c_int64),
        ("v", VLatent),
        ("pos0_device", ctypes.c_void_p),
        ("error_flag", ctypes.c_void_p),
    ]


class PrefillDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int), ("n_q_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("n_tokens", ctypes.c_int),
        ("pos0", ctypes.c_int), ("dtype", ctypes.c_int),
        ("q", ctypes.c_void_p), ("q_stride_b", ctypes.c_int64), ("q_stride_h", ctypes.c_int64),
        ("q_stride_t", ctypes.c_int64),
        ("k", KLatent),
        ("v", VLatent),
        ("uv", ctypes.c_void_p), ("uv_row_stride", ctypes.c_int64),
        ("rope_table", ctypes.c_void_p), ("rope_max_positions", ctypes.c_int),
        ("scale", ctypes.c_float),
        ("out", ctypes.c_void_p), ("out_stride_b", ctypes.c_int64), ("out_stride_h", ctypes.c_int64),
        ("out_stride_t", ctypes.c_int64),
    ]


class RopeApplyDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int), ("n_heads", ctypes.c_int), ("n_tokens", ctypes.c_int), ("dtype", ctypes.c_int),
        ("x", ctypes.c_void_p), ("stride_b", ctypes.c_int64), ("stride_h", ctypes.c_int64),
        ("stride_t", ctypes.c_int64),
        ("rope_table", ctypes.c_void_p), ("rope_max_positions", ctypes.c_int),
        ("pos0", ctypes.c_int),
        ("pos0_device", ctypes.c_void_p),
        ("error_flag", ctypes.c_void_p),
    ]


class RmsNormDesc(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int), ("hidden", ctypes.c_int), ("dtype", ctypes.c_int),
        ("x", ctypes.c_void_p), ("x_stride", ctypes.c_int64),
        ("residual", ctypes.c_void_p), ("residual_stride", ctypes.c_int64),
        ("residual_out", ctypes.c_void_p), ("residual_out_stride", ctypes.c_int64),
        ("weight", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("out", ctypes.c_void_p), ("out_stride", ctypes.c_int64),
    ]


class SiluMulDesc(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int), ("width", ctypes.c_int), ("dtype", ctypes.c_int),
        ("gate", ctypes.c_void_p), ("gate_stride", ctypes.c_int64),
        ("up", ctypes.c_void_p), ("up_stride", ctypes.c_int64),
        ("out", ctypes.c_void_p), ("out_stride", ctypes.c_int64),
    ]


class SkinnyGemmDesc(ctypes.Structure):
    _fields_ = [
        ("m", ctypes.c_int), ("n", ctypes.c_int), ("k", ctypes.c_int), ("dtype", ctypes.c_int),
        ("epilogue", ctypes.c_int),
        ("x", ctypes.c_void_p), ("x_stride", ctypes.c_int64),
        ("w", ctypes.c_void_p), ("w_stride", ctypes.c_int64),
        ("out", ctypes.c_void_p), ("out_stride", ctypes.c_int64),
        ("w_packed", ctypes.c_int),
        ("rms", ctypes.c_int), ("rms_eps", ctypes.c_float),
    ]


EXPORTS = (
    "starkv_abi_version", "starkv_status_string",
    "starkv_rope_table_bytes", "starkv_rope_build", "starkv_rope_apply",
    "starkv_k_logits_workspace_bytes", "starkv_k_logits",
    "starkv_pv_latent_workspace_bytes", "starkv_pv_latent",
    "starkv_decode_workspace_bytes", "starkv_decode_attention", "starkv_decode_attention_timed",
    "starkv_decode_attention_noalloc",
    "starkv_k_append", "starkv_v_append", "starkv_decode_append",
    "starkv_prefill_workspace_bytes", "starkv_prefill_attention", "starkv_prefill_attention_timed",
    "starkv_rms_norm", "starkv_silu_mul", "starkv_skinny_gemm",
)

ABI_VERSION = 5          # STARKV_ABI_VERSION of include/starkv.h that these structs mirror
NOALLOC_SCRATCH_BYTES = 128 << 20   # STARKV_NOALLOC_SCRATCH_BYTES

_lib = None


def lib() -> ctypes.CDLL:
    """Load libstarkv.so once; raise StarKVError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise StarKVError(f"{LIB_PATH} is missing: build it with `make -C star-kv_amd` "
                          "(or __graft_entry__.build()); there is no fallback path")
    L = ctypes.CDLL(LIB_PATH)
    L.starkv_abi_version.restype = ctypes.c_int
    L.starkv_status_string.restype = ctypes.c_char_p
    L.starkv_status_string.argtypes = [ctypes.c_int]
    L.starkv_rope_table_bytes.restype = ctypes.c_size_t
    L.starkv_rope_table_bytes.argtypes = [ctypes.c_int]
    L.starkv_rope_build.restype = ctypes.c_int
    L.starkv_rope_build.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_float, ctypes.c_int,
                                    ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    for name, desc in (("k_logits", KLogitsDesc), ("pv_latent", PVDesc), ("decode", DecodeDesc),
                       ("prefill", PrefillDesc)):
        wsf = getattr(L, f"starkv_{name}_workspace_bytes")
        wsf.restype = ctypes.c_size_t
        wsf.argtypes = [ctypes.POINTER(desc)]
    for name, desc in (("k_logits", KLogitsDesc), ("pv_latent", PVDesc), ("decode_attention", DecodeDesc),
                       ("prefill_attention", PrefillDesc)):
        f = getattr(L, f"starkv_{name}")
        f.restype = ctypes.c_int
        f.argtypes = [ctypes.POINTER(desc), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    L.starkv_decode_attention_timed.restype = ctypes.c_int
    L.starkv_decode_attention_timed.argtypes = [ctypes.POINTER(DecodeDesc), ctypes.c_void_p, ctypes.c_size_t,
                                                ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    L.starkv_prefill_attention_timed.restype = ctypes.c_int
    L.starkv_prefill_attention_timed.argtypes = [ctypes.POINTER(PrefillDesc), ctypes.c_void_p, ctypes.c_size_t,
                                                 ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    L.starkv_decode_attention_noalloc.restype = ctypes.c_int
    L.starkv_decode_attention_noalloc.argtypes = [ctypes.POINTER(DecodeDesc), ctypes.c_void_p]
    L.starkv_rope_apply.restype = ctypes.c_int
    L.starkv_rope_apply.argtypes = [ctypes.POINTER(RopeApplyDesc), ctypes.c_void_p]
    L.starkv_k_append.restype = ctypes.c_int
    L.starkv_k_append.argtypes = [ctypes.POINTER(KAppendDesc), ctypes.c_void_p]
    L.starkv_v_append.restype = ctypes.c_int
    L.starkv_v_append.argtypes = [ctypes.POINTER(VAppendDesc), ctypes.c_void_p]
    L.starkv_decode_append.restype = ctypes.c_int
    L.starkv_decode_append.argtypes = [ctypes.POINTER(KAppendDesc), ctypes.POINTER(VAppendDesc),
                                       ctypes.POINTER(RopeApplyDesc), ctypes.c_void_p]
    if L.starkv_abi_version() != ABI_VERSION:
        raise StarKVError(f"{LIB_PATH} has ABI version {L.starkv_abi_version()}, this binding needs "
                          f"{ABI_VERSION}: rebuild it with `make -C star-kv_amd`")
    L.starkv_rms_norm.restype = ctypes.c_int
    L.starkv_rms_norm.argtypes = [ctypes.POINTER(RmsNormDesc), ctypes.c_void_p]
    L.starkv_silu_mul.restype = ctypes.c_int
    L.starkv_silu_mul.argtypes = [ctypes.POINTER(SiluMulDesc), ctypes.c_void_p]
    L.starkv_skinny_gemm.restype = ctypes.c_int
    L.starkv_skinny_gemm.argtypes = [ctypes.POINTER(SkinnyGemmDesc), ctypes.c_void_p]
    _lib = L
    return L


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().starkv_status_string(status).decode()
        raise StarKVError(f"{what} failed with status {status}: {msg}")


def i64_array(vals):
    return (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])


def int_array(vals):
    return (ctypes.c_int * len(vals))(*[int(v) for v in vals])
