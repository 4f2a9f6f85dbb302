"""ctypes binding of ``libminispeed_boundary.so`` (include/minispeed_boundary.h).

The boundary step of this package runs only as the HIP kernels of that
library.  Loading fails loudly (``NativeLibraryError``) when the library has
not been built; nothing in the package falls back to another implementation.

torch is imported first so that the library's ``libamdhip64.so.7`` dependency
binds to the HIP runtime torch already loaded: the stream handles and device
pointers handed across the ABI then belong to one runtime.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch  # noqa: F401  (must precede the dlopen below, see module doc)

LIB_NAME = "libminispeed_boundary.so"
ABI_VERSION = 8

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

SCALE_NONE = 0
SCALE_DIVIDE = 1
SCALE_MULTIPLY = 2

_TORCH_TO_MS = {
    torch.float32: DTYPE_F32,
    torch.float16: DTYPE_F16,
    torch.bfloat16: DTYPE_BF16,
}


class NativeLibraryError(RuntimeError):
    """The HIP library is missing, stale, or cannot be loaded."""


class Segment(ctypes.Structure):
    """``ms_segment_t``: one contiguous piece of a flat group."""

    _fields_ = [
        ("begin", ctypes.c_int64),
        ("numel", ctypes.c_int64),
        ("grad", ctypes.c_void_p),
        ("model", ctypes.c_void_p),
    ]


class StepScalars(ctypes.Structure):
    """``ms_step_scalars_t``: K2's result, read back once per boundary."""

    _fields_ = [
        ("overflow", ctypes.c_uint32),
        ("clip_applied", ctypes.c_uint32),
        ("sumsq", ctypes.c_float),
        ("norm", ctypes.c_float),
        ("coef", ctypes.c_float),
        ("ready", ctypes.c_uint32),
        ("coef64", ctypes.c_double),
        ("next_scale", ctypes.c_double),
        ("next_good_steps", ctypes.c_int64),
        ("next_skipped_steps", ctypes.c_int64),
    ]


class AdamWParams(ctypes.Structure):
    """``ms_adamw_params_t``: one group's rounded AdamW scalars."""

    _fields_ = [
        ("neg_lr", ctypes.c_float),
        ("decay_alpha", ctypes.c_float),
        ("beta1", ctypes.c_float),
        ("one_minus_beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("one_minus_beta2", ctypes.c_float),
        ("bias_c1", ctypes.c_float),
        ("bias_c2", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("grad_scale", ctypes.c_float),
        ("decay", ctypes.c_int32),
        ("unscale", ctypes.c_int32),
    ]


class GroupScan(ctypes.Structure):
    """``ms_group_scan_t``: one group of ms_boundary_scalars_noalloc."""

    _fields_ = [
        ("segs", ctypes.c_void_p),
        ("nseg", ctypes.c_int32),
        ("grad_dtype", ctypes.c_int32),
        ("begin", ctypes.c_int64),
        ("end", ctypes.c_int64),
        ("own_begin", ctypes.c_int64),
        ("own_end", ctypes.c_int64),
    ]


class AccumRow(ctypes.Structure):
    """``ms_accum_row_t``: one gradient of ms_accumulate_grads."""

    _fields_ = [
        ("dst", ctypes.c_void_p),
        ("src", ctypes.c_void_p),
        ("numel", ctypes.c_int64),
        ("first", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("tile_sumsq", ctypes.c_void_p),
        ("tile_flag", ctypes.c_void_p),
    ]


ACCUM_ROWS_PER_LAUNCH = 64
ACCUM_TILE = 2048
# flat indices per K1 tile (MS_SCAN_TILE)
SCAN_TILE = 2048

SEGMENT_BYTES = ctypes.sizeof(Segment)
SCALARS_BYTES = ctypes.sizeof(StepScalars)

# exported symbol -> (restype, argtypes)
_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F = ctypes.c_float
_D = ctypes.c_double
SIGNATURES = {
    "ms_abi_version": (ctypes.c_int, []),
    "ms_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "ms_stats_blocks": (ctypes.c_int, []),
    "ms_grad_stats": (
        ctypes.c_int,
        [_P, _I32, _I32, _I64, _I64, _I64, _I64, _I32, _F, _P, _P, _P, _I64, _P, _P, _I32, _P],
    ),
    "ms_norm_clip": (
        ctypes.c_int,
        [_P, _P, _I32, _I32, _I32, _D, _I32, _D, _I64, _I64, _I64, _D, _D, _P, _P, _P],
    ),
    "ms_fused_adamw": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I64, _I64,
         ctypes.POINTER(AdamWParams), _P, _P],
    ),
    "ms_cast_to_model": (ctypes.c_int, [_P, _I64, _I64, _P, _I32, _I32, _P]),
    "ms_accumulate_grad": (ctypes.c_int, [_P, _P, _I32, _I64, _I32, _P]),
    "ms_accumulate_grads": (ctypes.c_int, [_P, _I32, _I32, _I32, _F, _P]),
    "ms_reduce_tile_stats": (ctypes.c_int, [_P, _P, _I64, _P, _P, _I32, _P]),
    "ms_boundary_scalars_noalloc": (
        ctypes.c_int,
        [ctypes.POINTER(GroupScan), _I32, _I32, _F, _I32, _D, _I32, _D, _I64, _I64, _I64, _D, _D,
         _P, _P, _P],
    ),
}

SCRATCH_MAX_GROUPS = 8
SCRATCH_MAX_TILES = 1 << 21
ESCRATCH = -4

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def library_path() -> str:
    """Where the in-tree build puts the library (next to this file)."""
    override = os.environ.get("MINISPEED_AMD_LIB")
    if override:
        return override
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)


def load() -> ctypes.CDLL:
    """Load (once) and type the library; raise NativeLibraryError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise NativeLibraryError(
                f"{LIB_NAME} not found at {path}; build it with "
                "`python -m minispeed_amd.build` (hipcc --offload-arch=gfx950)"
            )
        try:
            lib = ctypes.CDLL(path)
        except OSError as exc:  # pragma: no cover - loader failure text
            raise NativeLibraryError(f"cannot load {path}: {exc}") from exc
        for name, (restype, argtypes) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as exc:
                raise NativeLibraryError(f"{path} does not export {name}") from exc
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.ms_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryError(
                f"{path} has ABI version {version}, expected {ABI_VERSION}; rebuild it"
            )
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    """Turn a non-zero return code into RuntimeError (engine error convention)."""
    if rc != 0:
        msg = load().ms_error_string(rc)
        text = msg.decode() if msg else "unknown error"
        raise RuntimeError(f"{what} failed with code {rc}: {text}")


def ms_dtype(dtype: torch.dtype) -> int:
    try:
        return _TORCH_TO_MS[dtype]
    except KeyError:
        raise TypeError(
            f"unsupported parameter dtype {dtype}; expected float32, float16 or bfloat16"
        ) from None


def stats_blocks() -> int:
    return int(load().ms_stats_blocks())


def scan_tiles(n: int) -> int:
    """K1's tile slots for a scan of n flat indices."""
    return (int(n) + SCAN_TILE - 1) // SCAN_TILE


def require_hip_tensor(t: torch.Tensor, what: str) -> None:
    """The package computes on HIP devices only; anything else is an error."""
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{what} is on {t.device}; minispeed_amd runs the boundary step as "
            "HIP kernels and needs tensors on a ROCm GPU (device 'cuda')"
        )


def stream_handle(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


# Timing-only HIP events.  hipEventDisableSystemFence (hip_runtime_api.h)
# records an event without the system-scope release that a default event
# performs, i.e. without writing back and invalidating the caches between
# the kernels it brackets; the elapsed time between two such events is valid
# once the stream has been synchronised.
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000
_hip: Optional[ctypes.CDLL] = None


def hip_runtime() -> ctypes.CDLL:
    """The HIP runtime torch has already loaded (RTLD_NOLOAD: never a second
    copy), typed for the event calls."""
    global _hip
    if _hip is not None:
        return _hip
    with _lock:
        if _hip is None:
            try:
                hip = ctypes.CDLL("libamdhip64.so.7", mode=os.RTLD_NOLOAD)
            except OSError as exc:
                raise NativeLibraryError(f"the HIP runtime is not loaded: {exc}") from exc
            hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(_P), ctypes.c_uint]
            hip.hipEventRecord.argtypes = [_P, _P]
            hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(_F), _P, _P]
            hip.hipEventDestroy.argtypes = [_P]
            hip.hipStreamSynchronize.argtypes = [_P]
            for fn in (hip.hipEventCreateWithFlags, hip.hipEventRecord, hip.hipEventElapsedTime,
                       hip.hipEventDestroy, hip.hipStreamSynchronize):
                fn.restype = ctypes.c_int
            _hip = hip
    return _hip


def hip_check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed with hipError_t {rc}")
