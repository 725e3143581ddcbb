"""ctypes binding of libndx.so (include/ndx.h).

The library must be built (``python -m naivediffusion_amd.build``); there is
no fallback: every operator runs in the HIP library or not at all.
Statuses become the exceptions the reference throws (Dml/DeviceExceptions.cs,
ArgumentException, InvalidOperationException).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libndx.so"


class NdxError(RuntimeError):
    """Base of the library's failures."""


class ArgumentError(NdxError, ValueError):
    """ArgumentException: a shape, type or argument the operator refuses."""


class InvalidOperationError(NdxError):
    """InvalidOperationException: a call out of order."""


class OutOfVideoMemoryError(NdxError, MemoryError):
    """OutOfVideoMemoryException (Dml/DeviceExceptions.cs:5-12): the device stays usable."""


class DeviceRemovedError(NdxError):
    """DeviceRemovedException (Dml/DmlDevice.cs:948-953): the device is gone."""


class UnsupportedError(NdxError, NotImplementedError):
    """A combination this backend does not implement."""


_STATUS = {
    1: ArgumentError,
    2: InvalidOperationError,
    3: OutOfVideoMemoryError,
    4: DeviceRemovedError,
    5: UnsupportedError,
}

# Every exported entry point: (name, restype, argtypes). Also the list the
# symbol-export test checks against include/ndx.h.
vp = ctypes.c_void_p
i32 = ctypes.c_int32
i64 = ctypes.c_int64
u64 = ctypes.c_uint64
f32 = ctypes.c_float
f64 = ctypes.c_double
P = ctypes.POINTER
cstr = ctypes.c_char_p

SIGNATURES = [
    ("ndx_last_error", cstr, []),
    ("ndx_version", cstr, []),
    ("ndx_device_count", i32, [P(i32)]),
    ("ndx_device_create", i32, [i32, P(vp)]),
    ("ndx_device_destroy", i32, [vp]),
    ("ndx_device_name", i32, [vp, ctypes.c_char_p, i32]),
    ("ndx_device_memory", i32, [vp, P(u64), P(u64)]),
    ("ndx_device_release_pooled", i32, [vp]),
    ("ndx_device_synchronize", i32, [vp]),
    ("ndx_device_set_fault_injection", i32, [vp, i32]),
    ("ndx_tensor_upload", i32, [vp, i32, P(i64), i32, vp, u64, P(vp)]),
    ("ndx_tensor_empty", i32, [vp, i32, P(i64), i32, P(vp)]),
    ("ndx_tensor_download", i32, [vp, vp, u64]),
    ("ndx_tensor_release", i32, [vp]),
    ("ndx_tensor_info", i32, [vp, P(i32), P(i64), P(i32)]),
    ("ndx_tensor_fill_normal", i32, [vp, u64, f32, f32]),
    ("ndx_quantize_fits", i32, [i64, i32, i32]),
    ("ndx_quantize_block_int8", i32, [vp, i32, i64, i64, i32, i32, vp, vp]),
    ("ndx_quantize_block_int8_device", i32, [vp, i32, i32, vp, vp]),
    ("ndx_graph_create", i32, [vp, i32, i32, P(vp)]),
    ("ndx_graph_destroy", i32, [vp]),
    ("ndx_graph_set_stream", i32, [vp, i32]),
    ("ndx_graph_input", i32, [vp, i32, P(i64), i32, P(i32)]),
    ("ndx_graph_constant", i32, [vp, i32, P(i64), i32, vp, i32, P(i32)]),
    ("ndx_graph_constant_device", i32, [vp, vp, P(i32)]),
    ("ndx_graph_weight", i32, [vp, P(i64), i32, vp, i32, i32, P(i32)]),
    ("ndx_graph_weight_device", i32, [vp, vp, i32, P(i32)]),
    ("ndx_graph_weight_int8", i32, [vp, vp, vp, i32, P(i32)]),
    ("ndx_value_info", i32, [vp, i32, P(i32), P(i64), P(i32)]),
    ("ndx_op_reinterpret", i32, [vp, i32, P(i64), i32, P(i64), P(i32)]),
    ("ndx_op_slice", i32, [vp, i32, P(i64), P(i64), P(i64), P(i32)]),
    ("ndx_op_join", i32, [vp, P(i32), i32, i32, P(i32)]),
    ("ndx_op_cast", i32, [vp, i32, i32, P(i32)]),
    ("ndx_op_unary", i32, [vp, i32, i32, P(i32)]),
    ("ndx_op_scale_bias", i32, [vp, i32, f32, f32, P(i32)]),
    ("ndx_op_binary", i32, [vp, i32, i32, i32, P(i32)]),
    ("ndx_op_linear", i32, [vp, i32, i32, i32, i32, i32, i32, P(i32)]),
    ("ndx_op_gemm", i32, [vp, i32, i32, i32, i32, i32, f32, f32, P(i32)]),
    ("ndx_op_attention", i32, [vp, i32, i32, i32, i32, f32, i32, i32, P(i32)]),
    ("ndx_op_head_norm_rotate", i32, [vp, i32, i32, f32, i32, i32, i32, i32, P(i32)]),
    ("ndx_op_layer_norm", i32, [vp, i32, i32, i32, f32, P(i32)]),
    ("ndx_op_modulate", i32, [vp, i32, i32, i32, f32, i32, P(i32)]),
    ("ndx_op_rms_norm", i32, [vp, i32, i32, f32, P(i32)]),
    ("ndx_op_group_norm", i32, [vp, i32, i32, i32, i32, f32, i32, P(i32)]),
    ("ndx_op_conv2d", i32, [vp, i32, i32, i32, i32, i32, i32, i32, P(i32)]),
    ("ndx_op_upsample_nearest", i32, [vp, i32, i32, P(i32)]),
    ("ndx_op_patchify", i32, [vp, i32, i32, i32, P(i32)]),
    ("ndx_op_unpatchify", i32, [vp, i32, i32, i32, i32, i32, i32, P(i32)]),
    ("ndx_op_guided_euler_step", i32, [vp, i32, i32, i32, i32, P(i32)]),
    ("ndx_op_softmax", i32, [vp, i32, f32, P(i32)]),
    ("ndx_graph_compile", i32, [vp, P(i32), i32, P(vp)]),
    ("ndx_model_sizes", i32, [vp, P(u64), P(u64)]),
    ("ndx_model_counts", i32, [vp, P(i32), P(i32), P(i32)]),
    ("ndx_model_run", i32, [vp, P(vp), i32, P(vp), i32]),
    ("ndx_model_run_into_async", i32, [vp, P(vp), i32, P(vp), i32]),
    ("ndx_model_run_into_static_async", i32, [vp, P(vp), i32, P(vp), i32]),
    ("ndx_model_set_graph_replay", i32, [vp, i32]),
    ("ndx_model_set_profiling", i32, [vp, i32]),
    ("ndx_model_set_profile_filter", i32, [vp, ctypes.c_char_p]),
    ("ndx_model_profile_entry", i32, [vp, i32, ctypes.c_char_p, i32, P(i64), P(f64), P(f64), P(f64)]),
    ("ndx_model_release", i32, [vp]),
    ("ndx_safetensors_open", i32, [cstr, P(vp)]),
    ("ndx_safetensors_close", i32, [vp]),
    ("ndx_safetensors_count", i32, [vp, P(i32), P(i32)]),
    ("ndx_safetensors_entry", i32, [vp, i32, P(cstr), P(cstr), P(i64), P(i32), P(u64)]),
    ("ndx_safetensors_metadata", i32, [vp, i32, P(cstr), P(cstr)]),
    ("ndx_safetensors_data", i32, [vp, cstr, P(vp), P(u64)]),
    ("ndx_safetensors_read", i32, [vp, cstr, vp, i32, P(vp)]),
    ("ndx_lora_fold", i32, [vp, vp, i32, i32, P(vp)]),
]


class LoraPatch(ctypes.Structure):
    """ndx_lora_patch."""
    _fields_ = [("down", vp), ("up", vp), ("scale", f32), ("first_row", i32)]


MAX_LORA_PATCHES = 16  # NDX_MAX_LORA_PATCHES

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded libndx.so; raises if it was never built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build the HIP library first "
                "(python -m naivediffusion_amd.build). There is no CPU fallback.")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _check_fresh(L)
        _lib = L
    return _lib


def _check_fresh(L) -> None:
    """Refuses a library built from sources other than the ones beside it:
    ndx_version() ends with the hash build.py embeds."""
    from .build import CSRC, source_hash
    if not CSRC.is_dir():
        return  # an installed library without its sources: nothing to compare
    built = L.ndx_version().decode().rsplit(" ", 1)[-1]
    want = source_hash()
    if built != want:
        raise ImportError(
            f"{LIB_PATH} is stale: built from sources with hash {built}, the sources here hash to {want}. "
            "Rebuild it (python -m naivediffusion_amd.build).")


def check(status: int) -> None:
    if status != 0:
        msg = lib().ndx_last_error().decode("utf-8", "replace")
        raise _STATUS.get(status, NdxError)(msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


def shape_array(shape):
    arr = (i64 * max(len(shape), 1))(*[int(s) for s in shape])
    return arr
