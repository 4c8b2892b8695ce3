"""ctypes binding of libse12_gfx950.so (C ABI: include/se12_gfx950.h).

The library is loaded after torch so that both use the one HIP runtime torch
ships (same soname, libamdhip64.so.7), which keeps device pointers and stream
handles valid across the boundary. There is no fallback: if the library is
missing the import fails with instructions to build it.
"""

from __future__ import annotations

import ctypes
import pathlib

import torch  # noqa: F401  (loads the HIP runtime this library binds to)

LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libse12_gfx950.so"

SE12_OK = 0
SE12_E_INVALID = -1
SE12_E_HIP = -2
SE12_E_CAPACITY = -3
SE12_E_DEVICE = -4

X_BF16 = 0
X_F32 = 1
FORMAT_SE12 = 0
FORMAT_RAW_BF16 = 1
MAX_BATCH = 32
MAX_GROUP = 4

c_void_p = ctypes.c_void_p
c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_u8p = ctypes.POINTER(ctypes.c_uint8)


class Se12Error(RuntimeError):
    """A failed call into the SE12 library (status code and message)."""

    def __init__(self, code: int, message: str) -> None:
        super().__init__(f"[{code}] {message}")
        self.code = code


class Se12CapacityError(Se12Error):
    pass


class Streams(ctypes.Structure):
    _fields_ = [
        ("sm_dev", c_void_p),
        ("ec_dev", c_void_p),
        ("esc_dev", c_void_p),
        ("codebook_dev", c_void_p),
        ("fallback_bitmap_dev", c_void_p),
        ("fallback_raw_dev", c_void_p),
        ("fallback_raw_elems", c_i64),
    ]


class StreamsOut(ctypes.Structure):
    _fields_ = [
        ("sm_dev", c_void_p),
        ("ec_dev", c_void_p),
        ("esc_dev", c_void_p),
        ("fallback_bitmap_dev", c_void_p),
        ("fallback_raw_dev", c_void_p),
        ("fallback_raw_tiles", c_i64),
    ]


class Launch(ctypes.Structure):
    _fields_ = [("threads_per_block", c_i32), ("blocks", c_i32)]


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("compute_units", c_i32),
        ("wavefront_size", c_i32),
        ("l2_bytes", c_i64),
        ("lds_bytes_per_cu", c_i64),
        ("lds_bytes_per_block", c_i64),
        ("total_memory_bytes", c_i64),
        ("clock_khz", c_i32),
        ("memory_clock_khz", c_i32),
        ("memory_bus_width_bits", c_i32),
        ("max_threads_per_block", c_i32),
        ("pci_domain_id", c_i32),
        ("pci_bus_id", c_i32),
        ("pci_device_id", c_i32),
        ("ecc_enabled", c_i32),
        ("kernel_timeout", c_i32),
        ("runtime_version", c_i32),
        ("driver_version", c_i32),
    ]


# name -> (restype, argtypes): every symbol include/se12_gfx950.h and
# include/se12_step.h declare
SIGNATURES = {
    "se12_last_error": (ctypes.c_char_p, []),
    "se12_version": (ctypes.c_char_p, []),
    "se12_device_info_get": (c_i32, [c_i32, ctypes.POINTER(DeviceInfo)]),
    "se12_bind": (c_i32, [ctypes.POINTER(Streams), c_i64, c_i64, c_i32, c_void_p, ctypes.POINTER(c_void_p)]),
    "se12_bind_raw_bf16": (c_i32, [c_void_p, c_i64, c_i64, c_i32, c_void_p, ctypes.POINTER(c_void_p)]),
    "se12_release": (c_i32, [c_void_p]),
    "se12_handle_shape": (
        c_i32,
        [c_void_p, ctypes.POINTER(c_i64), ctypes.POINTER(c_i64), ctypes.POINTER(c_i64), ctypes.POINTER(c_i64), ctypes.POINTER(c_i32)],
    ),
    "se12_handle_bind_stats": (c_i32, [c_void_p, ctypes.POINTER(c_i64), ctypes.POINTER(c_i64)]),
    "se12_default_launch": (c_i32, [c_void_p, c_i32, ctypes.POINTER(Launch)]),
    "se12_set_compute_units": (c_i32, [c_void_p, c_i32]),
    "se12_read_probe": (c_i32, [c_void_p, c_i64, c_void_p, c_i64, c_void_p]),
    "se12_gemv": (c_i32, [c_void_p, c_void_p, c_i32, c_i32, c_void_p, ctypes.POINTER(Launch), c_void_p]),
    "se12_gemv_noalloc": (c_i32, [c_void_p, c_void_p, c_i32, c_i32, c_void_p, ctypes.POINTER(Launch), c_void_p]),
    "se12_gemv_grouped": (
        c_i32,
        [ctypes.POINTER(c_void_p), c_i32, c_void_p, c_i32, c_i32, ctypes.POINTER(c_void_p), ctypes.POINTER(Launch), c_void_p],
    ),
    "se12_gemv_gelu_mul": (
        c_i32,
        [ctypes.POINTER(c_void_p), c_void_p, c_i32, c_i32, ctypes.POINTER(c_void_p), c_void_p, ctypes.POINTER(Launch),
         c_void_p],
    ),
    "se12_gemv_rmsnorm": (
        c_i32,
        [c_void_p, c_void_p, c_i32, c_i32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_float,
         ctypes.POINTER(Launch), c_void_p],
    ),
    "se12_gemv_prenorm": (
        c_i32,
        [ctypes.POINTER(c_void_p), c_i32, c_void_p, c_void_p, c_i32, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, ctypes.c_float, ctypes.POINTER(c_void_p), c_void_p, ctypes.POINTER(Launch), c_void_p],
    ),
    "se12_gemv_rowss": (
        c_i32, [c_void_p, c_void_p, c_i32, c_i32, c_void_p, c_void_p, ctypes.POINTER(Launch), c_void_p],
    ),
    "se12_decode": (c_i32, [c_void_p, c_void_p, c_void_p]),
    "se12_decode_rows": (c_i32, [c_void_p, c_void_p, c_i64, c_void_p, c_void_p]),
    "se12_codebook_from_histogram": (c_i32, [ctypes.POINTER(ctypes.c_uint64), c_u8p]),
    "se12_encode_prepare": (c_i32, [c_void_p, c_i64, c_i64, c_i64, c_u8p, ctypes.POINTER(c_i64), c_void_p]),
    "se12_encode": (
        c_i32,
        [c_void_p, c_i64, c_i64, c_i64, c_u8p, ctypes.POINTER(StreamsOut), ctypes.POINTER(c_i64), c_void_p],
    ),
    # decode-step kernels (include/se12_step.h)
    "se12_step_last_error": (ctypes.c_char_p, []),
    "se12_step_rmsnorm": (
        c_i32,
        [c_void_p, c_i32, c_i64, c_void_p, c_void_p, c_void_p, c_void_p, c_i32, c_i32, ctypes.c_float, ctypes.c_float,
         c_i32, c_void_p],
    ),
    "se12_step_attention_workspace": (c_i64, [c_i32, c_i32, c_i32, c_i32, c_i32]),
    "se12_step_attention": (
        c_i32,
        [c_void_p, c_void_p, c_void_p, c_i32, c_i64, c_i64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_i32, c_i32,
         c_i32, c_i32, c_i32, ctypes.c_float, ctypes.c_float, c_i32, c_void_p, c_i64, c_void_p],
    ),
    "se12_step_gelu_mul": (c_i32, [c_void_p, c_void_p, c_i32, c_i64, c_void_p, c_i32, c_i32, c_void_p]),
    "se12_step_logits_workspace": (c_i64, [c_i32, c_i32]),
    "se12_step_logits_argmax": (
        c_i32,
        [c_void_p, c_i32, c_i64, c_i32, c_i32, ctypes.c_float, c_void_p, c_void_p, c_void_p, c_i64, c_void_p, c_void_p,
         c_i64, c_void_p],
    ),
    "se12_step_advance": (c_i32, [c_void_p, c_void_p, c_void_p]),
    "se12_step_logits_argmax_advance": (
        c_i32,
        [c_void_p, c_i32, c_i64, c_i32, c_i32, ctypes.c_float, c_void_p, c_void_p, c_void_p, c_i64, c_void_p, c_void_p,
         c_void_p, c_i64, c_void_p],
    ),
}

STEP_BF16 = 0
STEP_F32 = 1

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library (loaded on first use)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"SE12 HIP library not found at {LIB_PATH}; build it with "
                "`python -m se12_amd.csrc.build` (hipcc, gfx950) before using the GPU path"
            )
        handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().se12_last_error()
    return msg.decode() if msg else ""


def step_check(rc: int) -> None:
    """Raises the step kernels' last error for a non-zero status."""
    if rc != 0:
        raise Se12Error(rc, (lib().se12_step_last_error() or b"").decode())


def check(rc: int) -> None:
    """Raises the library's last error for a non-zero status."""
    if rc == SE12_OK:
        return
    if rc == SE12_E_CAPACITY:
        raise Se12CapacityError(rc, last_error())
    raise Se12Error(rc, last_error())


def ptr(t) -> c_void_p:
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return c_void_p(None)
    return c_void_p(t.data_ptr())


def stream_ptr(stream=None) -> c_void_p:
    """hipStream_t of a torch stream (default: the current stream)."""
    s = stream if stream is not None else torch.cuda.current_stream()
    return c_void_p(s.cuda_stream)


def version() -> str:
    return lib().se12_version().decode()
