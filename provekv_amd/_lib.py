"""ctypes binding of libpkv_hip.so (include/pkv_codec.h).

Loading is strict: a missing library raises ``ImportError`` naming the build
command, so no caller can silently fall back to a CPU path.  When the process
uses torch, import torch first: the library then binds to torch's HIP runtime
(same soname), so device pointers and streams are shared.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpkv_hip.so")

OK = 0
ERR_INVALID_ARG = 1
ERR_DIM_MISMATCH = 2
ERR_OOM = 3
ERR_DEVICE = 4
ERR_CORRUPT_PAYLOAD = 5
ERR_UNSUPPORTED = 6
ERR_NONFINITE_INPUT = 7
ERR_ZERO_NORM = 8
ERR_NORM_UNREPRESENTABLE = 9
ERR_EMPTY_BATCH = 10
ERR_CAPACITY = 11
ERR_NONFINITE_CODE = 12
ERR_SCRATCH_LIMIT = 13
NOALLOC_MAX_SEGMENTS = 4096

CODEC_TURBO = 1
CODEC_FIB = 2
TURBO_POLAR_ONLY = 0
TURBO_POLAR_WITH_QJL = 1
RADII_F32 = 0
RADII_LOG_U8 = 1
DT_F32 = 0
DT_BF16 = 1
DT_F16 = 2

# every symbol include/pkv_codec.h declares
EXPORTS = (
    "pkv_status_string", "pkv_ctx_create", "pkv_ctx_destroy", "pkv_device_available",
    "pkv_turbo_profile_create", "pkv_turbo_profile_create_with_constants", "pkv_fib_profile_create",
    "pkv_fib_profile_create_with_constants", "pkv_profile_destroy", "pkv_fib_decode_path", "pkv_turbo_constants",
    "pkv_fib_constants", "pkv_profile_constants", "pkv_payload_len", "pkv_header_len", "pkv_blob_len",
    "pkv_write_header",
    "pkv_segments_status", "pkv_encode_segments", "pkv_encode_segments_bounded", "pkv_decode_segments", "pkv_decode_segments_ex",
    "pkv_decode_segments_bounded", "pkv_decode_segments_noalloc",
    "pkv_encode_batch_compact",
    "pkv_decode_batch_compact", "pkv_parse_header", "pkv_record_len", "pkv_encode_vectors", "pkv_decode_vectors",
    "pkv_constants_cache_stats", "pkv_constants_cache_clear", "pkv_prepared_len", "pkv_turbo_prepare_queries",
    "pkv_turbo_score_segments", "pkv_score_status", "pkv_turbo_score_batch", "pkv_encode_diagnostics",
    "pkv_radii_log_bound", "pkv_fb2_n_blocks", "pkv_lloyd_refine", "pkv_blake3_ranges", "pkv_blake3_layer_digests",
    "pkv_blake3_tier_digests", "pkv_blake3",
    "pkv_host_angle_bins", "pkv_host_octant_bins", "pkv_host_logf",
    "pkv_host_expf", "pkv_host_f32_stable_rel50", "pkv_code_from_json", "pkv_fib_digests", "pkv_host_blake3",
)


class Seg(C.Structure):
    _fields_ = [
        ("elem_offset", C.c_uint64),
        ("stride_outer", C.c_uint64),
        ("stride_inner", C.c_uint64),
        ("wire_offset", C.c_uint64),
        ("n_vectors", C.c_uint32),
        ("group", C.c_uint32),
    ]


class CodecParams(C.Structure):
    """pkv_codec_params: a codec profile by its adapter parameters."""
    _fields_ = [
        ("kind", C.c_int32),
        ("dim", C.c_uint32),
        ("bits", C.c_uint32),
        ("projections", C.c_uint32),
        ("k", C.c_uint32),
        ("n", C.c_uint32),
        ("training_samples", C.c_uint32),
        ("lloyd_restarts", C.c_uint32),
        ("lloyd_iterations", C.c_uint32),
        ("seed", C.c_uint64),
    ]


def turbo_params(dim: int, bits: int, projections: int, seed: int) -> CodecParams:
    return CodecParams(CODEC_TURBO, dim, bits, projections, 0, 0, 0, 0, 0, seed)


def fib_params(dim: int, k: int, n: int, seed: int, training: int = 2048, restarts: int = 4,
               iterations: int = 8) -> CodecParams:
    return CodecParams(CODEC_FIB, dim, 0, 0, k, n, training, restarts, iterations, seed)


class Error(C.Structure):
    _fields_ = [("status", C.c_int32), ("segment", C.c_int32), ("index", C.c_uint64)]


class PkvError(RuntimeError):
    """A non-OK status from the library."""

    def __init__(self, status: int, where: str = "", segment: int = -1, index: int = 0):
        self.status = status
        self.segment = segment
        self.index = index
        msg = f"{where}: {status_string(status)} (status {status}"
        if segment >= 0:
            msg += f", segment {segment}, vector {index}"
        super().__init__(msg + ")")


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python provekv_amd/build.py` "
                              "(or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH, mode=C.RTLD_GLOBAL)
        _declare(L)
        _lib = L
    return _lib


def _declare(L):
    P = C.c_void_p
    U32, U64, I32 = C.c_uint32, C.c_uint64, C.c_int
    sig = {
        "pkv_status_string": ([I32], C.c_char_p),
        "pkv_ctx_create": ([I32, P], I32),
        "pkv_ctx_destroy": ([P], None),
        "pkv_device_available": ([], I32),
        "pkv_turbo_profile_create": ([P, U32, U32, U32, U64, I32, P], I32),
        "pkv_turbo_profile_create_with_constants": ([P, U32, U32, U32, U64, I32, P, P, P], I32),
        "pkv_fib_profile_create": ([P, U32, U32, U32, U64, U32, U32, U32, P], I32),
        "pkv_fib_profile_create_with_constants": ([P, U32, U32, U32, P, P, P], I32),
        "pkv_profile_destroy": ([P], None),
        "pkv_fib_decode_path": ([P], I32),
        "pkv_turbo_constants": ([U32, U32, U64, P, P], I32),
        "pkv_fib_constants": ([U32, U32, U32, U64, U32, U32, U32, P, P, P, P], I32),
        "pkv_profile_constants": ([P, P, C.c_size_t, P, C.c_size_t], I32),
        "pkv_payload_len": ([P, I32], U32),
        "pkv_header_len": ([P], U32),
        "pkv_blob_len": ([P, I32, U64], U64),
        "pkv_write_header": ([P, I32, U64, P, U64], I32),
        "pkv_segments_status": ([P, P, U32, P], I32),
        "pkv_encode_segments": ([P, P, I32, I32, P, U64, P, U32, P, U64, P, P], I32),
        "pkv_encode_segments_bounded": ([P, P, I32, I32, P, U64, P, U32, P, U64, U32, P, P], I32),
        "pkv_decode_segments": ([P, P, I32, P, U64, P, U32, P, U64, P, P], I32),
        "pkv_decode_segments_ex": ([P, P, I32, P, U64, P, U32, P, I32, U64, U32, U64, P, P], I32),
        "pkv_decode_segments_bounded": ([P, P, I32, P, U64, P, U32, P, I32, U64, U32, U64, U32, P, P], I32),
        "pkv_decode_segments_noalloc": ([P, P, I32, P, U64, P, U32, P, I32, U64, U32, U64, P, P], I32),
        "pkv_encode_batch_compact": ([P, P, I32, P, U64, P, U64, P, P], I32),
        "pkv_decode_batch_compact": ([P, P, P, U64, P, U64, P, P], I32),
        "pkv_parse_header": ([P, P, U64, P, P], I32),
        "pkv_record_len": ([P], U32),
        "pkv_encode_vectors": ([P, P, I32, P, U64, P, U64, P, P], I32),
        "pkv_decode_vectors": ([P, P, I32, P, P, U64, P, U64, P], I32),
        "pkv_constants_cache_stats": ([P, P, P], None),
        "pkv_constants_cache_clear": ([], None),
        "pkv_prepared_len": ([P], U32),
        "pkv_turbo_prepare_queries": ([P, P, P, U32, P, P, P], I32),
        "pkv_turbo_score_segments": ([P, P, I32, P, U64, P, U32, P, U64, U32, U64, C.c_float, P, U64, U64, P, P],
                                     I32),
        "pkv_score_status": ([P, U32, P], I32),
        "pkv_turbo_score_batch": ([P, P, P, U64, P, U32, C.c_float, P, U64, P, P], I32),
        "pkv_encode_diagnostics": ([P, P, I32, P, U64, P, U64, P, U64, P, P, P], I32),
        "pkv_radii_log_bound": ([P, P], I32),
        "pkv_fb2_n_blocks": ([P, U64, P], I32),
        "pkv_lloyd_refine": ([P, P, U32, U32, U32, P, U32, U32, P, P, P], I32),
        "pkv_blake3_ranges": ([P, P, U64, P, U32, P, P], I32),
        "pkv_blake3_layer_digests": ([P, P, U32, U32, P, P], I32),
        "pkv_blake3_tier_digests": ([P, P, U64, P, U32, U32, P, P, P], I32),
        "pkv_blake3": ([P, P, U64, P], I32),
        "pkv_host_angle_bins": ([P, P, U64, U32, P], None),
        "pkv_host_octant_bins": ([P, P, U64, P, P], None),
        "pkv_host_logf": ([P, U64, P], None),
        "pkv_host_f32_stable_rel50": ([P, U64, P], None),
        "pkv_host_expf": ([P, U64, P], None),
        "pkv_code_from_json": ([P, P, U64, P, U64, P, P], I32),
        "pkv_fib_digests": ([P, P, P, P], I32),
        "pkv_host_blake3": ([P, U64, P], None),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res


def status_string(status: int) -> str:
    try:
        return lib().pkv_status_string(status).decode()
    except ImportError:
        return f"status {status}"


def check(rc: int, where: str):
    if rc != OK:
        raise PkvError(rc, where)


def code_from_json(params: CodecParams, text: bytes):
    """pkv_code_from_json: (status, stage, payload bytes) of a JSON code."""
    buf = C.create_string_buffer(bytes(text), max(len(text), 1))
    out = C.create_string_buffer(4096)
    n = C.c_uint64()
    stage = C.c_int()
    rc = lib().pkv_code_from_json(C.byref(params), buf, len(text), out, 4096, C.byref(n), C.byref(stage))
    return rc, stage.value, out.raw[:n.value] if rc == OK else b""


def fib_digests(params: CodecParams):
    """pkv_fib_digests: (profile, codebook, rotation) digest strings."""
    bufs = [C.create_string_buffer(72) for _ in range(3)]
    check(lib().pkv_fib_digests(C.byref(params), bufs[0], bufs[1], bufs[2]), "pkv_fib_digests")
    return tuple(b.value.decode() for b in bufs)


def host_blake3(data: bytes) -> bytes:
    out = C.create_string_buffer(32)
    buf = C.create_string_buffer(bytes(data), max(len(data), 1))
    lib().pkv_host_blake3(buf, len(data), out)
    return out.raw
