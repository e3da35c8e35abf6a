"""Loader for libaero_hip.so and the ctypes prototypes of every symbol in
include/aero_hip.h.

There is no CPU fallback anywhere in this package: if the library is missing,
or no GPU is visible, every op raises (AeroHipUnavailable or the reference's
*Unavailable classes, which derive from it).
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_uint8, c_uint32, c_void_p

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("AERO_HIP_LIB", os.path.join(HERE, "libaero_hip.so"))


class AeroHipUnavailable(RuntimeError):
    """libaero_hip.so is not built or no MI355X is visible."""


class AeroHipError(RuntimeError):
    """A libaero_hip entry point refused its arguments or hit a HIP error."""


fp = POINTER(c_float)
ip = POINTER(c_int32)
u8p = POINTER(c_uint8)
vp = c_void_p



class AttnInput(ctypes.Structure):
    """aero_attn_input_t of include/aero_hip.h, field for field."""
    _fields_ = [("dtype", c_int), ("n_mat", c_int), ("w", POINTER(vp)),
                ("w_bytes", POINTER(c_int64)), ("n_rows", POINTER(c_int64)), ("y", POINTER(vp)),
                ("n_cols", c_int64), ("n_tok", c_int64), ("x", vp), ("d", vp), ("x_out", vp),
                ("emb_type", c_int), ("emb", vp), ("emb_bytes", c_int64), ("vocab", c_int64),
                ("ids", vp), ("emb_scale", c_float), ("norm_w", vp), ("eps", c_float),
                ("norm", c_int), ("n_rope", c_int), ("head_dim", c_int64), ("n_rot", c_int64),
                ("rope_mode", c_int), ("pos", vp), ("inv_freq", vp), ("q_norm_w", vp),
                ("k_norm_w", vp), ("qk_eps", c_float), ("qk_flags", c_int)]


# name -> (restype, argtypes), exactly the prototypes of include/aero_hip.h
PROTOTYPES = {
    # reference-compatible host ABI
    "aero_tensor_threads": (c_int, []),
    "aero_tensor_matvec": (c_int, [fp, fp, fp, c_int64, c_int64, c_int]),
    "aero_tensor_matmul": (c_int, [fp, fp, fp, c_int64, c_int64, c_int64, c_int]),
    "aero_tensor_argmax": (c_int, [fp, c_int64]),
    "aero_tensor_silu": (c_int, [fp, c_int64]),
    "aero_tensor_gelu": (c_int, [fp, c_int64]),
    "aero_tensor_mul": (c_int, [fp, fp, c_int64]),
    "aero_tensor_swiglu": (c_int, [fp, fp, c_int64]),
    "aero_tensor_rmsnorm": (c_int, [fp, fp, fp, c_int64, c_float]),
    "aero_tensor_l2norm": (c_int, [fp, fp, fp, c_int64, c_float, c_int]),
    "aero_tensor_rmsnorm_rows": (c_int, [fp, c_int64, c_int64, c_float]),
    "aero_rope_tables": (c_int64, [c_int64, ip, c_int64, c_float, c_int64, fp, c_int64,
                                   fp, fp]),
    "aero_apply_rope": (None, [fp, c_int64, c_int64, c_int64, fp, fp, ip, c_int]),
    "aero_rmsnorm_rows": (None, [fp, fp, fp, c_int64, c_int64, c_float]),
    "aero_l2norm_rows": (None, [fp, fp, fp, c_int64, c_int64, c_float]),
    "aero_gelu": (None, [fp, c_int64]),
    "aero_silu": (None, [fp, c_int64]),
    "aero_swiglu": (None, [fp, fp, c_int64]),
    "aero_dtype_block_bytes": (c_int64, [c_int]),
    "aero_dtype_block_values": (c_int64, [c_int]),
    "aero_hardware_threads": (c_int, []),
    "aero_dequant_ref": (c_int, [c_int, u8p, c_int64, fp, c_int64]),
    "aero_dequant_threaded": (c_int, [c_int, u8p, c_int64, fp, c_int64, c_int]),
    "aero_matvec": (c_int, [c_int, u8p, fp, fp, c_int64, c_int64, c_int]),
    "aero_matmul": (c_int, [c_int, u8p, fp, fp, c_int64, c_int64, c_int64, c_int]),
    "aero_tensor_softmax": (c_int, [fp, c_int64]),
    "aero_softmax": (None, [fp, c_int64]),
    "aero_softmax_rows": (None, [fp, c_int64, c_int64]),
    "aero_attention_tiled": (c_int, [fp, fp, fp, fp, c_int64, c_int64, c_int64, c_int64,
                                     c_int64, c_float, ip, ip, c_int64, c_int, c_int64]),
    "aero_attention": (c_int, [fp, fp, fp, fp, c_int64, c_int64, c_int64, c_int64, c_float,
                               c_int64, c_int]),
    "aero_kv_write_vec": (c_int, [c_int, fp, c_int64, vp, fp]),
    "aero_kv_read_vec": (c_int, [c_int, vp, fp, c_int64, fp]),
    "aero_kv_ring_indices": (c_int, [c_int64, c_int64, POINTER(c_int64)]),
    "aero_kv_ring_rotate": (c_int, [c_int64, c_int64, c_int64, POINTER(c_int64)]),
    "aero_kv_span_error": (c_int, [c_int, vp, fp, c_int64, fp, fp]),
    "aero_kv_slot_new": (vp, [c_int64, c_int64, c_int64, c_int, c_int]),
    "aero_kv_slot_free": (None, [vp]),
    "aero_kv_slot_bytes": (c_int64, [vp]),
    "aero_kv_slot_write": (c_int, [vp, c_int64, c_int64, fp]),
    "aero_kv_slot_read": (c_int, [vp, c_int64, c_int64, fp]),
    "aero_hip_kv_slot_view": (c_int, [vp, POINTER(vp), POINTER(fp), POINTER(c_int64),
                                      POINTER(c_int64), POINTER(c_int64), POINTER(c_int),
                                      POINTER(c_int)]),
    # device-pointer fused ops
    "aero_hip_rmsnorm": (c_int, [vp, vp, vp, c_int64, c_int64, c_float, c_int, vp]),
    "aero_hip_gated_rmsnorm_silu": (c_int, [vp, vp, vp, c_int64, vp, c_int64, c_int64,
                                            c_int64, c_float, vp]),
    "aero_hip_act_mul": (c_int, [c_int, vp, vp, vp, c_int64, vp]),
    "aero_hip_add_rmsnorm": (c_int, [vp, vp, vp, vp, vp, c_int64, c_int64, c_float, c_int,
                                     vp]),
    "aero_hip_post_norm_add": (c_int, [vp, vp, vp, vp, c_float, c_float, vp, vp, c_int64,
                                       c_int64, c_float, c_int, vp]),
    "aero_hip_rope_inv_freq": (c_int64, [c_int64, c_int64, c_float, fp, c_int64, fp]),
    "aero_hip_rope_tables": (c_int, [vp, c_int64, vp, c_int64, vp, vp, vp]),
    "aero_hip_qk_norm_rope": (c_int, [vp, vp, c_int64, vp, vp, c_int64, vp, vp, c_float,
                                      c_int, c_int64, c_int64, c_int64, c_int, vp, vp, vp,
                                      vp, c_int64, vp]),
    "aero_hip_embed_gather": (c_int, [c_int, vp, c_int64, c_int64, c_int64, vp, c_int64,
                                      c_float, vp, vp, vp]),
    "aero_hip_dequant": (c_int, [c_int, vp, c_int64, vp, c_int64, vp]),
    "aero_hip_embed_rmsnorm": (c_int, [c_int, vp, c_int64, c_int64, c_int64, vp, c_int64,
                                       c_float, vp, vp, c_float, c_int, vp, vp, vp]),
    "aero_hip_tensor_rows": (c_int, [c_int, vp, c_int64, c_int64, c_int64, c_int64, c_int64,
                                     vp, vp]),
    # gated DeltaNet
    "aero_ssm_softplus": (c_float, [c_float]),
    "aero_ssm_delta_step": (None, [fp] * 8 + [c_int, c_int, c_float, c_float, fp]),
    "aero_ssm_scan": (None, [fp] * 8 + [c_int] * 4 + [c_float, c_float, fp]),
    "aero_ssm_conv": (None, [fp, fp, fp, POINTER(c_int), fp, c_int, c_int, c_int]),
    "aero_hip_ssm_workspace": (c_int64, [c_int64] * 4),
    "aero_hip_ssm_scan": (c_int, [vp] * 8 + [c_int64] * 4 + [c_float, c_float, vp, vp, c_int64,
                                                              vp]),
    "aero_hip_ssm_conv": (c_int, [vp, vp, vp, c_int64, vp, vp, c_int64, c_int64, c_int64,
                                  POINTER(c_int64), vp]),
    "aero_hip_ssm_scan_strided": (c_int, [vp, c_int64, vp, c_int64, vp, c_int64] + [vp] * 5
                                  + [c_int64] * 4 + [c_float, c_float, vp, vp, c_int64, vp]),
    "aero_hip_ssm_conv_silu": (c_int, [vp, vp, vp, c_int64, vp, vp, c_int64, c_int64, c_int64,
                                       POINTER(c_int64), vp]),
    # GGUF reader
    "aero_gguf_open": (vp, [ctypes.c_char_p]),
    "aero_gguf_close": (None, [vp]),
    "aero_gguf_file_size": (c_int64, [vp]),
    "aero_gguf_version": (c_int, [vp]),
    "aero_gguf_alignment": (c_int64, [vp]),
    "aero_gguf_data_offset": (c_int64, [vp]),
    "aero_gguf_arch": (ctypes.c_char_p, [vp]),
    "aero_gguf_n_kv": (c_int64, [vp]),
    "aero_gguf_kv_key": (ctypes.c_char_p, [vp, c_int64]),
    "aero_gguf_kv_type": (c_int, [vp, ctypes.c_char_p]),
    "aero_gguf_get_int": (c_int, [vp, ctypes.c_char_p, POINTER(c_int64)]),
    "aero_gguf_get_float": (c_int, [vp, ctypes.c_char_p, POINTER(ctypes.c_double)]),
    "aero_gguf_get_str": (vp, [vp, ctypes.c_char_p, POINTER(c_int64)]),
    "aero_gguf_array_len": (c_int64, [vp, ctypes.c_char_p]),
    "aero_gguf_array_ints": (c_int64, [vp, ctypes.c_char_p, POINTER(c_int64), c_int64]),
    "aero_gguf_array_floats": (c_int64, [vp, ctypes.c_char_p, POINTER(ctypes.c_double),
                                         c_int64]),
    "aero_gguf_array_str": (vp, [vp, ctypes.c_char_p, c_int64, POINTER(c_int64)]),
    "aero_gguf_kv_json": (vp, [vp, POINTER(c_int64)]),
    "aero_gguf_n_tensors": (c_int64, [vp]),
    "aero_gguf_tensor_name": (vp, [vp, c_int64]),
    "aero_gguf_tensor_info": (c_int64, [vp, ctypes.c_char_p, POINTER(c_int), POINTER(c_int),
                                        POINTER(c_int64), POINTER(c_int64), POINTER(c_int64)]),
    "aero_gguf_tensor_data": (vp, [vp, ctypes.c_char_p]),
    "aero_gguf_read": (c_int, [vp, ctypes.c_char_p, c_int64, c_int64, vp]),
    "aero_gguf_upload": (c_int, [vp, ctypes.c_char_p, c_int64, c_int64, vp, vp]),
    "aero_hip_matvec": (c_int, [c_int, vp, c_int64, vp, vp, c_int64, c_int64, c_int64, vp]),
    "aero_hip_norm_matvec": (c_int, [c_int, c_int, POINTER(vp), POINTER(c_int64), POINTER(c_int64),
                                     POINTER(vp), vp, vp, c_float, c_int, c_int64, c_int64, vp]),
    "aero_hip_norm_gate_up": (c_int, [c_int, vp, vp, c_int64, vp, vp, c_float, c_int, c_int, vp,
                                      c_int64, c_int64, c_int64, vp]),
    "aero_hip_ssm_proj_conv": (c_int, [c_int, c_int, POINTER(vp), POINTER(c_int64), POINTER(c_int64),
                                       POINTER(vp), vp, c_int64, vp, vp, c_int64, vp, vp]),
    "aero_hip_gated_norm_matvec": (c_int, [c_int, vp, c_int64, c_int64, vp, vp, vp, vp, c_int64,
                                           c_float, c_int64, c_int64, vp]),
    "aero_hip_gated_norm_matmul": (c_int, [c_int, vp, c_int64, c_int64, vp, vp, vp, vp, c_int64,
                                           c_float, c_int64, c_int64, vp, c_int64, vp]),
    "aero_hip_matmul_workspace": (c_int64, [c_int, c_int64, c_int64]),
    "aero_hip_norm_matmul_workspace": (c_int64, [c_int, c_int64, c_int64, c_int64]),
    "aero_hip_split_partials_bytes": (c_int64, [c_int64, c_int64, c_int64]),
    "aero_hip_split_ok": (c_int, [c_int, c_int64, c_int64, c_int64]),
    "aero_hip_norm_matmul": (c_int, [c_int, c_int, POINTER(vp), POINTER(c_int64), POINTER(c_int64),
                                     POINTER(vp), vp, vp, vp, vp, c_float, c_int, c_int64,
                                     c_int64, vp, c_int64, vp]),
    "aero_hip_norm_matmul_rope": (c_int, [c_int, c_int, POINTER(vp), POINTER(c_int64),
                                          POINTER(c_int64), POINTER(vp), vp, vp, vp, vp, c_float,
                                          c_int, c_int64, c_int64, c_int, c_int64, c_int, vp, vp,
                                          vp, c_int64, vp]),
    "aero_hip_attn_input": (c_int, [POINTER(AttnInput), vp, c_int64, vp]),
    "aero_hip_norm_matmul_gate_up": (c_int, [c_int, vp, vp, c_int64, vp, vp, vp, vp, c_float,
                                             c_int, c_int, vp, c_int64, c_int64, c_int64, vp,
                                             c_int64, vp]),
    "aero_hip_matmul_noalloc": (c_int, [c_int, vp, c_int64, vp, vp, c_int64, c_int64, c_int64,
                                        vp]),
    "aero_hip_matmul_noalloc_max_bytes": (c_int64, []),
    "aero_hip_matmul": (c_int, [c_int, vp, c_int64, vp, vp, c_int64, c_int64, c_int64, vp,
                                c_int64, vp]),
    "aero_hip_attention_workspace": (c_int64, [c_int64, c_int64, c_int64, c_int64, c_int64,
                                               c_int64]),
    "aero_hip_attention": (c_int, [vp, c_int, vp, vp, vp, vp, vp, c_int64, c_int64, c_int64,
                                   c_int64, c_int64, c_float, vp, vp, c_int64, c_int, vp,
                                   c_int64, vp]),
    "aero_hip_kv_write": (c_int, [c_int, vp, c_int64, c_int64, c_int64, c_int64, c_int64, vp,
                                  vp, vp]),
    "aero_hip_softmax_rows": (c_int, [vp, vp, c_int64, c_int64, vp]),
    "aero_hip_copy_f32": (c_int, [vp, vp, c_int64, vp]),
    "aero_hip_fill_f32": (c_int, [vp, c_float, c_int64, vp]),
    # runtime
    "aero_hip_last_error": (c_char_p, []),
    "aero_hip_version": (c_char_p, []),
    "aero_hip_device_count": (c_int, []),
    "aero_hip_set_device": (c_int, [c_int]),
    "aero_hip_malloc": (vp, [c_int64]),
    "aero_hip_free": (c_int, [vp]),
    "aero_hip_memcpy_htod": (c_int, [vp, vp, c_int64]),
    "aero_hip_memcpy_dtoh": (c_int, [vp, vp, c_int64]),
    "aero_hip_memcpy_dtod": (c_int, [vp, vp, c_int64, vp]),
    "aero_hip_memset": (c_int, [vp, c_int, c_int64]),
    "aero_hip_tune_set": (c_int, [c_char_p, c_int, c_int]),
    "aero_hip_stream_create": (vp, []),
    "aero_hip_stream_destroy": (c_int, [vp]),
    "aero_hip_stream_synchronize": (c_int, [vp]),
    "aero_hip_device_synchronize": (c_int, []),
    "aero_hip_event_create": (vp, []),
    "aero_hip_event_destroy": (c_int, [vp]),
    "aero_hip_event_record": (c_int, [vp, vp]),
    "aero_hip_event_synchronize": (c_int, [vp]),
    "aero_hip_event_elapsed_ms": (c_float, [vp, vp]),
    "aero_hip_time_next_kernel": (c_int, [vp, vp]),
    "aero_hip_plan_create": (vp, []),
    "aero_hip_plan_begin": (c_int, [vp]),
    "aero_hip_plan_end": (c_int, [vp]),
    "aero_hip_plan_size": (c_int64, [vp]),
    "aero_hip_plan_launch": (c_int, [vp, vp, POINTER(vp), POINTER(vp)]),
    "aero_hip_plan_destroy": (c_int, [vp]),
}

_lib = None
_load_error: str | None = None


def load(path: str | None = None):
    """Load libaero_hip.so once and declare every prototype. Returns None and
    records the reason when the file is missing or lacks a symbol."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if _load_error is not None and path is None:
        return None
    p = path or LIB_PATH
    if not os.path.exists(p):
        _load_error = f"{p} not found; build it with `python -m aero_amd.build`"
        return None
    try:
        L = ctypes.CDLL(p)
        for name, (res, args) in PROTOTYPES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
    except (OSError, AttributeError) as e:
        _load_error = f"{p}: {e}"
        return None
    _lib = L
    return _lib


def unavailable_reason() -> str:
    load()
    if _lib is None:
        return _load_error or "libaero_hip not loaded"
    if _lib.aero_hip_device_count() <= 0:
        return "no HIP device visible"
    return ""


def available() -> bool:
    """Library loaded and at least one GPU visible."""
    return unavailable_reason() == ""


_ready = None


def lib(exc: type = AeroHipUnavailable):
    """The loaded library with a usable GPU, or raise `exc`."""
    global _ready
    if _ready is not None:
        return _ready
    L = load()
    if L is None or L.aero_hip_device_count() <= 0:
        raise exc(unavailable_reason())
    _ready = L
    return L


def last_error() -> str:
    L = load()
    if L is None:
        return ""
    return (L.aero_hip_last_error() or b"").decode(errors="replace")


def check(ok, what: str):
    """Raise AeroHipError with the library's reason when an entry point refused."""
    if not ok:
        raise AeroHipError(f"{what}: {last_error()}")
