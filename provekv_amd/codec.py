"""proveKV's codec plugin surface over the MI355X library.

Mirrors proveKV/src/codec.rs: the ``KVecCodec`` trait (8-66), the
``TurboQuantAdapter`` (172-422) and ``FibQuantAdapter`` (429-693) with their
inherent batch methods ``encode_batch_compact`` / ``decode_batch_compact``
(TQB1 248-326, FB2 513-569), and ``create_codec`` (700-758).  Same names,
argument meaning and error classes; the work runs in libpkv_hip.so through
``pkv_encode_batch_compact`` / ``pkv_decode_batch_compact`` (batched TQB1 /
FB2 blobs) and ``pkv_encode_vectors`` / ``pkv_decode_vectors`` (the trait's
per-vector TQW1 / FB1 records, and the serde_json codes older proveKV
versions stored, which the adapters still decode).
"""
from __future__ import annotations

from enum import Enum

import numpy as np

from . import _lib as L
from .device import default_context

CODEC_FIB_K4_N32 = "fib_k4_n32"
CODEC_FIB_K4_N32_BATCHED = "fib_k4_n32_batched"
CODEC_TURBO_8BIT = "turbo_8bit"
CODEC_TURBO_8BIT_BATCHED = "turbo_8bit_batched"
CODEC_TURBO_8BIT_BATCHED_LOSSY = "turbo_8bit_batched_lossy"


def turbo_batched_codec_id(bits: int, lossy_radii: bool) -> str:
    """proveKV/src/policy.rs:78-82."""
    return f"turbo_{bits}bit_batched" + ("_lossy" if lossy_radii else "")


class RadiiCompression(Enum):
    """proveKV/src/policy.rs RadiiCompression."""
    Lossless = 0
    Lossy = 1


# ---------------------------------------------------------------- errors
class ProveKvError(RuntimeError):
    """proveKV/src/error.rs ProveKvError (string-carrying variants)."""


class CompressionFailed(ProveKvError):
    pass


class DecompressionFailed(ProveKvError):
    pass


class InvalidPolicy(ProveKvError):
    pass


class DimensionMismatch(ProveKvError):
    def __init__(self, expected: int, got: int):
        super().__init__(f"dimension mismatch: expected {expected}, got {got}")
        self.expected = expected
        self.got = got


class CorruptPayload(ProveKvError):
    pass


def _wrap(exc: L.PkvError, cls, what: str):
    return cls(f"{what}: {exc}")


# ---------------------------------------------------------------- trait
class KVecCodec:
    """proveKV/src/codec.rs:8-66."""

    def codec_id(self) -> str:
        raise NotImplementedError

    def encode_batch(self, vectors, seed: int):
        return [self.encode(v, seed) for v in vectors]

    def decode_batch(self, payloads, seed: int):
        return [self.decode(p, seed) for p in payloads]

    def dim(self) -> int:
        raise NotImplementedError

    def compression_ratio(self) -> float:
        raise NotImplementedError

    def is_gpu_accelerated(self) -> bool:
        return L.lib().pkv_device_available() == 1

    def is_gpu_accelerated_for(self, n: int, d: int) -> bool:
        return self.is_gpu_accelerated()


def _as_batch(vectors, dim: int) -> np.ndarray:
    if isinstance(vectors, np.ndarray) and vectors.ndim == 2:
        x = vectors
    else:
        rows = list(vectors)
        for r in rows:
            if len(r) != dim:
                raise DimensionMismatch(dim, len(r))
        x = np.array(rows, dtype=np.float32).reshape(len(rows), dim)
    if x.shape[1] != dim:
        raise DimensionMismatch(dim, x.shape[1])
    return np.ascontiguousarray(x, dtype=np.float32)


class TurboQuantAdapter(KVecCodec):
    """proveKV/src/codec.rs:172-422 (TQB1 batch path)."""

    def __init__(self, dim: int, bits: int, projections: int,
                 radii_compression: RadiiCompression = RadiiCompression.Lossless):
        if dim == 0:
            raise InvalidPolicy("turbo dim must be > 0")
        if dim % 2 != 0:
            raise InvalidPolicy(f"turbo requires even dimension, got {dim}")
        self._dim = dim
        self.bits = bits
        self.projections = projections
        self.radii_compression = radii_compression

    @classmethod
    def with_radii_compression(cls, dim, bits, projections, radii_compression):
        return cls(dim, bits, projections, radii_compression)

    def _profile(self, seed: int, what: str):
        try:
            return default_context().turbo_profile(self._dim, self.bits, self.projections, seed)
        except L.PkvError as e:
            raise _wrap(e, CompressionFailed if what == "encode" else DecompressionFailed,
                        "turbo quantizer init failed")

    def codec_id(self) -> str:
        return CODEC_TURBO_8BIT

    def dim(self) -> int:
        return self._dim

    def compression_ratio(self) -> float:
        return 8.0

    def encode_batch_compact(self, vectors, seed: int) -> bytes:
        x = _as_batch(vectors, self._dim)
        prof = self._profile(seed, "encode")
        radii = L.RADII_LOG_U8 if self.radii_compression == RadiiCompression.Lossy else L.RADII_F32
        try:
            return prof.encode_batch_compact(x, radii)
        except L.PkvError as e:
            raise _wrap(e, CompressionFailed, "turbo batched wire encode failed")

    def decode_batch_compact(self, payload: bytes, seed: int) -> np.ndarray:
        prof = self._profile(seed, "decode")
        try:
            return prof.decode_batch_compact(payload)
        except L.PkvError as e:
            raise _wrap(e, DecompressionFailed, "turbo batched wire decode failed")

    # ---- KVecCodec per-vector methods: one TQW1 record per vector
    # (codec.rs:339-405; encode_batch / decode_batch are the trait's loops)
    def encode(self, vector, seed: int) -> bytes:
        return self.encode_batch([vector], seed)[0]

    def encode_batch(self, vectors, seed: int) -> list:
        x = _as_batch(vectors, self._dim)
        prof = self._profile(seed, "encode")
        try:
            return prof.encode_vectors(x, each=True)
        except L.PkvError as e:
            raise _wrap(e, CompressionFailed, "turbo encode failed")

    def decode(self, payload: bytes, seed: int) -> np.ndarray:
        return self.decode_batch([payload], seed)[0]

    def decode_batch(self, payloads, seed: int) -> np.ndarray:
        """A TQW1 record, or else the serde_json TurboCode an older proveKV
        stored (codec.rs:367-405), per payload; the first failing payload
        raises."""
        payloads = [bytes(p) for p in payloads]
        prof = self._profile(seed, "decode")
        try:
            return prof.decode_vectors(payloads, each=True)
        except L.PkvError as e:
            raise _wrap(e, DecompressionFailed, "turbo decode failed")


class FibQuantAdapter(KVecCodec):
    """proveKV/src/codec.rs:429-693 (FB2 batch path)."""

    def __init__(self, dim: int, k: int, n: int, training_samples: int = 2048, lloyd_restarts: int = 4,
                 lloyd_iterations: int = 8):
        if dim == 0:
            raise InvalidPolicy("fib dim must be > 0")
        if dim % k != 0:
            raise InvalidPolicy(f"fib ambient dim ({dim}) must be divisible by k ({k})")
        self._dim = dim
        self.k = k
        self.n = n
        self.training_samples = training_samples
        self.lloyd_restarts = lloyd_restarts
        self.lloyd_iterations = lloyd_iterations

    def build_quantizer(self, seed: int):
        try:
            return default_context().fib_profile(self._dim, self.k, self.n, seed, self.training_samples,
                                                 self.lloyd_restarts, self.lloyd_iterations)
        except L.PkvError as e:
            raise _wrap(e, CompressionFailed, "fib quantizer build failed")

    def codec_id(self) -> str:
        return CODEC_FIB_K4_N32

    def dim(self) -> int:
        return self._dim

    def compression_ratio(self) -> float:
        return 50.0

    def encode_batch_compact(self, vectors, seed: int) -> bytes:
        x = _as_batch(vectors, self._dim)
        prof = self.build_quantizer(seed)
        try:
            return prof.encode_batch_compact(x)
        except L.PkvError as e:
            raise _wrap(e, CompressionFailed, "fib encode_batch failed")

    def decode_batch_compact(self, payload: bytes, seed: int) -> np.ndarray:
        """An FB2 blob; else one FB1 record; else one serde_json FibCodeV1
        (codec.rs:530-569), each through decode_batch_fast."""
        prof = self.build_quantizer(seed)
        try:
            return prof.decode_batch_compact(payload)
        except L.PkvError as e:
            raise _wrap(e, DecompressionFailed, "fib batched wire decode failed")

    # ---- KVecCodec per-vector methods: one compact FB1 record per vector
    # (codec.rs:582-665)
    def encode(self, vector, seed: int) -> bytes:
        x = _as_batch([vector], self._dim)
        prof = self.build_quantizer(seed)
        try:
            return prof.encode_vectors(x, each=True)[0]
        except L.PkvError as e:
            raise _wrap(e, CompressionFailed, "fib encode failed")

    def encode_batch(self, vectors, seed: int) -> list:
        x = _as_batch(vectors, self._dim)
        prof = self.build_quantizer(seed)
        try:
            return prof.encode_vectors(x, each=False)
        except L.PkvError as e:
            raise _wrap(e, CompressionFailed, "fib encode_batch failed")

    def decode(self, payload: bytes, seed: int) -> np.ndarray:
        """An FB1 record, or else the serde_json FibCodeV1 an older proveKV
        stored (codec.rs:612-637), through FibQuantizer::decode."""
        prof = self.build_quantizer(seed)
        try:
            return prof.decode_vectors([bytes(payload)], each=True)[0]
        except L.PkvError as e:
            raise _wrap(e, DecompressionFailed, "fib decode failed")

    def decode_batch(self, payloads, seed: int) -> np.ndarray:
        """Every payload parsed first (FB1 or JSON), then decode_batch_fast
        (codec.rs:639-665)."""
        payloads = [bytes(p) for p in payloads]
        prof = self.build_quantizer(seed)
        try:
            return prof.decode_vectors(payloads, each=False)
        except L.PkvError as e:
            raise _wrap(e, DecompressionFailed, "fib decode_batch_fast failed")


def create_codec(codec_id: str, dim: int, fib_config=None, turbo_config=None) -> KVecCodec:
    """proveKV/src/codec.rs:700-758."""
    if codec_id in (CODEC_FIB_K4_N32, CODEC_FIB_K4_N32_BATCHED):
        if fib_config is None:
            raise InvalidPolicy("fib codec requires fib_config")
        return FibQuantAdapter(dim, fib_config["k"], fib_config["n"], fib_config["training_samples"],
                               fib_config["lloyd_restarts"], fib_config["lloyd_iterations"])
    if codec_id in (CODEC_TURBO_8BIT, CODEC_TURBO_8BIT_BATCHED) or codec_id.startswith("turbo_"):
        if turbo_config is None:
            raise InvalidPolicy("turbo codec requires turbo_config")
        rc = turbo_config.get("radii_compression", RadiiCompression.Lossless)
        return TurboQuantAdapter(dim, turbo_config["bits"], turbo_config["projections"], rc)
    raise InvalidPolicy(f"unknown codec id: {codec_id}")


def fib_config_default_k4_n32() -> dict:
    """proveKV/src/policy.rs:137-145."""
    return {"k": 4, "n": 32, "training_samples": 2048, "lloyd_restarts": 4, "lloyd_iterations": 8}


def turbo_config_default_4bit(lossy: bool = False) -> dict:
    """proveKV/src/policy.rs:238-255."""
    return {"bits": 4, "projections": 32,
            "radii_compression": RadiiCompression.Lossy if lossy else RadiiCompression.Lossless}
