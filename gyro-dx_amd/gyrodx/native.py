"""ctypes binding of the gyro_native C ABI (include/gyro_native.h), the drop-in replacement of
the reference's native/include/gyro_native.h. Struct layouts match src/native_abi.zig:87-95."""
from __future__ import annotations

import ctypes as C

from . import BUILD_DIR

LIB_PATH = BUILD_DIR / "libgyro_native.so"

E_INVALIDARG = -2147024809  # 0x80070057
ERROR_INVALID_DATA = -2147024883  # 0x8007000D
E_ILLEGAL_METHOD_CALL = -2147483634  # 0x8000000E
E_FAIL = -2147467259  # 0x80004005

# Every symbol the header declares (native/include/gyro_native.h:71-137 of the reference).
SYMBOLS = [
    "gd_create", "gd_get_caps", "gd_open_file", "gd_file_size", "gd_create_buffer", "gd_read_ranges",
    "gd_poll", "gd_wait_storage", "gd_readback", "gd_validate_linalg", "gd_validate_gyro",
    "gd_create_resource", "gd_create_pipeline", "gd_release_pipeline", "gd_begin", "gd_dispatch",
    "gd_barrier", "gd_timestamp", "gd_submit", "gd_wait_compute", "gd_read_timestamps",
    "gd_queue_wait_storage", "gd_read_ranges_after", "gd_release_buffer", "gd_release_file", "gd_destroy",
    # Extensions without a counterpart in the reference ABI: timed dispatch for profiling, and the
    # stream launch and caller-memory table entries of the MoE engine's no-allocation entry point.
    "gd_dispatch_timed", "gd_dispatch_on", "gd_wrap_memory",
]


class Options(C.Structure):
    _fields_ = [("adapter_index", C.c_uint32), ("enable_debug", C.c_uint32), ("require_linalg", C.c_uint32),
                ("staging_bytes", C.c_uint32), ("queue_capacity", C.c_uint32)]


class Caps(C.Structure):
    _fields_ = [("abi_version", C.c_uint32), ("vendor_id", C.c_uint32), ("device_id", C.c_uint32),
                ("shader_model", C.c_uint32), ("linalg_tier", C.c_uint32),
                ("wave16_fp16_fp32_flags", C.c_uint32), ("vector_fp16_fp32_flags", C.c_uint32),
                ("experimental_features_enabled", C.c_uint32), ("dedicated_video_bytes", C.c_uint64),
                ("local_budget_bytes", C.c_uint64), ("local_usage_bytes", C.c_uint64),
                ("adapter_name", C.c_char * 128)]


class Range(C.Structure):
    _fields_ = [("file_offset", C.c_uint64), ("buffer_offset", C.c_uint64), ("bytes", C.c_uint32),
                ("reserved", C.c_uint32)]


class BufferInfo(C.Structure):
    _fields_ = [("srv_index", C.c_uint32), ("uav_index", C.c_uint32), ("mapped", C.c_void_p),
                ("gpu_address", C.c_uint64), ("allocated_bytes", C.c_uint64)]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run gyro-dx_amd/build.py")
        L = C.CDLL(str(LIB_PATH))
        vp, u32, u64, i32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32
        sig = {
            "gd_create": [C.POINTER(Options), C.POINTER(vp)],
            "gd_get_caps": [vp, C.POINTER(Caps)],
            "gd_open_file": [vp, C.c_char_p, C.POINTER(vp)],
            "gd_file_size": [vp, C.POINTER(u64)],
            "gd_create_buffer": [vp, u64, C.POINTER(vp)],
            "gd_read_ranges": [vp, vp, vp, C.POINTER(Range), u32, C.POINTER(u64)],
            "gd_poll": [vp, C.POINTER(u64), C.POINTER(u64)],
            "gd_wait_storage": [vp, u64, u32],
            "gd_readback": [vp, vp, u64, u32, vp, u32],
            "gd_validate_linalg": [vp, vp, C.c_size_t, C.POINTER(C.c_float), u32],
            "gd_validate_gyro": [vp, vp, C.c_size_t, vp, C.c_size_t, vp, C.c_size_t, u32, vp, u32,
                                 C.POINTER(C.c_float), u32],
            "gd_create_resource": [vp, u64, u32, C.POINTER(vp), C.POINTER(BufferInfo)],
            "gd_create_pipeline": [vp, vp, C.c_size_t, C.POINTER(vp)],
            "gd_release_pipeline": [vp, vp, u32],
            "gd_begin": [vp, u32],
            "gd_dispatch": [vp, vp, C.POINTER(u32), u32, u32, u32, u32],
            "gd_barrier": [vp],
            "gd_timestamp": [vp, C.POINTER(u32)],
            "gd_submit": [vp, C.POINTER(u64)],
            "gd_wait_compute": [vp, u64, u32],
            "gd_read_timestamps": [vp, u32, C.POINTER(u64), C.POINTER(u64)],
            "gd_queue_wait_storage": [vp, u64],
            "gd_read_ranges_after": [vp, vp, vp, C.POINTER(Range), u32, u64, C.POINTER(u64)],
            "gd_release_buffer": [vp, vp, u32],
            "gd_release_file": [vp, vp, u32],
            "gd_destroy": [vp, u32],
            "gd_dispatch_timed": [vp, vp, C.POINTER(u32), u32, u32, u32, u32, C.POINTER(u32)],
            "gd_dispatch_on": [vp, vp, C.POINTER(u32), u32, u32, u32, u32, vp],
            "gd_wrap_memory": [vp, vp, u64, C.POINTER(vp), C.POINTER(BufferInfo)],
        }
        for name, args in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = i32
        _lib = L
    return _lib


def hresult(code: int) -> str:
    return f"0x{code & 0xFFFFFFFF:08x}"


def check(code: int, what: str = "native call") -> None:
    """src/gpu.zig:7-13: a negative result is a failure."""
    if code < 0:
        raise RuntimeError(f"{what} failed: native HRESULT {hresult(code)}")
