"""Device-level API: contexts, profiles and segment tables over torch tensors.

Thin Python view of the C ABI in include/pkv_codec.h.  torch supplies device
memory and streams only; every byte of codec work runs in libpkv_hip.so.
"""
from __future__ import annotations

import ctypes as C
import threading

import numpy as np

from . import _lib as L

SEG_DTYPE = np.dtype([
    ("elem_offset", "<u8"),
    ("stride_outer", "<u8"),
    ("stride_inner", "<u8"),
    ("wire_offset", "<u8"),
    ("n_vectors", "<u4"),
    ("group", "<u4"),
])
assert SEG_DTYPE.itemsize == C.sizeof(L.Seg)


def segments(rows) -> np.ndarray:
    """Build a segment table from (elem_offset, stride_outer, stride_inner,
    wire_offset, n_vectors, group) tuples."""
    return np.array([tuple(int(v) for v in r) for r in rows], dtype=SEG_DTYPE)


def contiguous_segment(elem_offset: int, n: int, dim: int, wire_offset: int) -> tuple:
    """n row-major dim-vectors starting at elem_offset, one blob at wire_offset."""
    return (elem_offset, 0, dim, wire_offset, n, max(n, 1))


def _torch():
    import torch  # noqa: F401  (binds the library to torch's HIP runtime)
    return torch


def _stream_ptr(stream):
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream)


class Context:
    """pkv_ctx bound to one HIP device."""

    def __init__(self, device: int = 0):
        _torch()
        self._ptr = C.c_void_p()
        L.check(L.lib().pkv_ctx_create(device, C.byref(self._ptr)), "pkv_ctx_create")
        self.device = device
        self._profiles: dict = {}
        self._lock = threading.Lock()

    @property
    def ptr(self):
        return self._ptr

    def close(self):
        for p in list(self._profiles.values()):
            p.close()
        self._profiles.clear()
        if self._ptr:
            L.lib().pkv_ctx_destroy(self._ptr)
            self._ptr = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def radii_log_bound(self) -> np.ndarray:
        """The BlockLogU8 encode's cheap-log error bounds measured on this
        device: 256 floats, entry e covering every radius whose logf has a
        biased f32 exponent <= e (pkv_radii_log_bound)."""
        out = np.zeros(256, np.float32)
        L.check(L.lib().pkv_radii_log_bound(self.ptr, out.ctypes.data), "pkv_radii_log_bound")
        return out

    # ------------------------------------------------------------ digests
    def blake3_ranges(self, buf, ranges, out=None, stream=None):
        """BLAKE3 of byte ranges of device uint8 tensor `buf` (rows of
        (offset, len)), hashed where they lie: a [n, 32] uint8 device tensor
        (CompressedBlock::new's payload digest of each range,
        proveKV/src/codec.rs:85-95)."""
        torch = _torch()
        rg = np.ascontiguousarray(np.asarray(ranges, dtype=np.uint64).reshape(-1, 2))
        if buf.dtype != torch.uint8 or not buf.is_contiguous():
            raise TypeError("buf must be a contiguous uint8 tensor")
        if out is None:
            out = torch.empty((len(rg), 32), dtype=torch.uint8, device=buf.device)
        if out.dtype != torch.uint8 or not out.is_contiguous() or out.numel() < 32 * len(rg):
            raise ValueError(f"out must be a contiguous uint8 tensor of >= {32 * len(rg)} bytes")
        rc = L.lib().pkv_blake3_ranges(self.ptr, buf.data_ptr(), buf.numel(), rg.ctypes.data, len(rg),
                                       out.data_ptr(), _stream_ptr(stream))
        L.check(rc, "pkv_blake3_ranges")
        return out

    def layer_digests(self, kv_digests, layers: int, out=None, stream=None):
        """Layer digests (PoolLayer / ShellLayer::compute_digest,
        proveKV/src/pool.rs:83-103, shell.rs:48-66) from [n, 2, 32] key/value
        payload digests on the device, entry i being layer i % layers: a
        [n, 32] uint8 device tensor."""
        torch = _torch()
        if kv_digests.dtype != torch.uint8 or not kv_digests.is_contiguous() or kv_digests.numel() % 64:
            raise TypeError("kv_digests must be a contiguous uint8 tensor of 64-byte entries")
        n = kv_digests.numel() // 64
        if out is None:
            out = torch.empty((n, 32), dtype=torch.uint8, device=kv_digests.device)
        if out.dtype != torch.uint8 or not out.is_contiguous() or out.numel() < 32 * n:
            raise ValueError(f"out must be a contiguous uint8 tensor of >= {32 * n} bytes")
        rc = L.lib().pkv_blake3_layer_digests(self.ptr, kv_digests.data_ptr(), n, layers, out.data_ptr(),
                                              _stream_ptr(stream))
        L.check(rc, "pkv_blake3_layer_digests")
        return out

    def tier_digests(self, buf, ranges, layers: int, blob_out, layer_out, stream=None) -> None:
        """One tier of a build (pkv_blake3_tier_digests): the payload digests
        of its 2 n blobs (rows of `ranges`, key then value per entry) into
        `blob_out` [n, 2, 32] and the layer digests into `layer_out` [n, 32],
        one call for what blake3_ranges and layer_digests do in two."""
        torch = _torch()
        rg = np.ascontiguousarray(np.asarray(ranges, dtype=np.uint64).reshape(-1, 2))
        if len(rg) % 2:
            raise ValueError("ranges come in key / value pairs")
        n = len(rg) // 2
        for t, need in ((buf, 0), (blob_out, 64 * n), (layer_out, 32 * n)):
            if t.dtype != torch.uint8 or not t.is_contiguous() or t.numel() < need:
                raise ValueError("buf, blob_out and layer_out must be contiguous uint8 tensors of the needed size")
        rc = L.lib().pkv_blake3_tier_digests(self.ptr, buf.data_ptr(), buf.numel(), rg.ctypes.data, n, layers,
                                             blob_out.data_ptr(), layer_out.data_ptr(), _stream_ptr(stream))
        L.check(rc, "pkv_blake3_tier_digests")

    def blake3(self, data: bytes) -> bytes:
        """blake3::hash of host bytes, computed on this device."""
        data = bytes(data)
        out = C.create_string_buffer(32)
        L.check(L.lib().pkv_blake3(self.ptr, data, len(data), out), "pkv_blake3")
        return out.raw

    # profiles are cached per parameters: the reference rebuilds its codebook,
    # rotation and QJL matrix on every adapter call (proveKV/src/codec.rs:249,
    # 296, 471-499); here they are built once and stay resident.
    def turbo_profile(self, dim: int, bits: int, projections: int, seed: int,
                      mode: int = L.TURBO_POLAR_WITH_QJL) -> "Profile":
        key = ("turbo", dim, bits, projections, seed, mode)
        with self._lock:
            if key not in self._profiles:
                self._profiles[key] = Profile._turbo(self, dim, bits, projections, seed, mode)
            return self._profiles[key]

    def fib_profile(self, dim: int, k: int, n: int, seed: int, training_samples: int = 2048,
                    lloyd_restarts: int = 4, lloyd_iterations: int = 8) -> "Profile":
        key = ("fib", dim, k, n, seed, training_samples, lloyd_restarts, lloyd_iterations)
        with self._lock:
            if key not in self._profiles:
                self._profiles[key] = Profile._fib(self, dim, k, n, seed, training_samples, lloyd_restarts,
                                                   lloyd_iterations)
            return self._profiles[key]

    def fib_profile_with_constants(self, codebook: np.ndarray, rotation: np.ndarray) -> "Profile":
        """fib_k4_n32 profile from a caller's FibCodebookV1::codewords [32, 4]
        f32 and StoredRotation::matrix [64, 64] f64 (not cached: the caller
        owns the profile)."""
        cb = np.ascontiguousarray(codebook, dtype=np.float32).reshape(-1)
        rot = np.ascontiguousarray(rotation, dtype=np.float64).reshape(-1)
        n, k = 32, 4
        dim = int(round(np.sqrt(rot.size)))
        if cb.size != n * k or dim * dim != rot.size:
            raise ValueError("codebook must be [32, 4] and rotation [dim, dim]")
        ptr = C.c_void_p()
        L.check(L.lib().pkv_fib_profile_create_with_constants(self.ptr, dim, k, n, cb.ctypes.data, rot.ctypes.data,
                                                              C.byref(ptr)), "pkv_fib_profile_create_with_constants")
        return Profile(self, ptr, L.CODEC_FIB, dim, k=k, n=n, seed=None)


_default_ctx = None
_default_lock = threading.Lock()


def default_context() -> Context:
    global _default_ctx
    with _default_lock:
        if _default_ctx is None:
            _default_ctx = Context(0)
        return _default_ctx


class Profile:
    """pkv_profile: constants resident on the device."""

    def __init__(self, ctx: Context, ptr: C.c_void_p, kind: int, dim: int, **params):
        self.ctx = ctx
        self._ptr = ptr
        self.kind = kind
        self.dim = dim
        self.params = params

    @classmethod
    def _turbo(cls, ctx, dim, bits, projections, seed, mode):
        ptr = C.c_void_p()
        L.check(L.lib().pkv_turbo_profile_create(ctx.ptr, dim, bits, projections, seed, mode, C.byref(ptr)),
                "pkv_turbo_profile_create")
        return cls(ctx, ptr, L.CODEC_TURBO, dim, bits=bits, projections=projections, seed=seed, mode=mode)

    @classmethod
    def _fib(cls, ctx, dim, k, n, seed, training, restarts, iterations):
        ptr = C.c_void_p()
        L.check(L.lib().pkv_fib_profile_create(ctx.ptr, dim, k, n, seed, training, restarts, iterations,
                                               C.byref(ptr)), "pkv_fib_profile_create")
        return cls(ctx, ptr, L.CODEC_FIB, dim, k=k, n=n, seed=seed)

    @property
    def ptr(self):
        return self._ptr

    def close(self):
        if self._ptr:
            L.lib().pkv_profile_destroy(self._ptr)
            self._ptr = C.c_void_p()

    def fib_decode_path(self) -> str:
        """'matrix' (products verified bit-exact at creation) or 'valu'."""
        p = int(L.lib().pkv_fib_decode_path(self._ptr))
        return {1: "matrix", 0: "valu"}.get(p, "none")

    def payload_len(self, radii: int = L.RADII_F32) -> int:
        return int(L.lib().pkv_payload_len(self._ptr, radii))

    def header_len(self) -> int:
        return int(L.lib().pkv_header_len(self._ptr))

    def blob_len(self, n: int, radii: int = L.RADII_F32) -> int:
        return int(L.lib().pkv_blob_len(self._ptr, radii, n))

    def constants(self):
        if self.kind == L.CODEC_TURBO:
            a = np.zeros(self.dim, np.float32)
            rows = self.params["projections"] if self.params["mode"] == L.TURBO_POLAR_WITH_QJL else 0
            b = np.zeros(max(1, rows) * self.dim, np.float32)
        else:
            a = np.zeros(self.params["n"] * self.params["k"], np.float32)
            b = np.zeros(self.dim * self.dim, np.float64)
        L.check(L.lib().pkv_profile_constants(self._ptr, a.ctypes.data, a.nbytes, b.ctypes.data, b.nbytes),
                "pkv_profile_constants")
        return a, b

    # ------------------------------------------------------------ segments
    @staticmethod
    def _status_ptr(status, nseg: int):
        """The kernels write 2 uint32 words per segment into `status`."""
        if status is None:
            return None
        if status.element_size() != 4 or status.numel() < 2 * nseg or not status.is_contiguous():
            raise ValueError(f"status must be a contiguous 32-bit tensor of >= {2 * nseg} elements")
        return status.data_ptr()

    def encode_segments(self, inp, segs: np.ndarray, wire, radii: int = L.RADII_F32, status=None,
                        stream=None, max_workgroups: int = 0) -> None:
        """Encode every segment of `segs` from device tensor `inp` (f32 or
        bf16) into device uint8 tensor `wire` in one launch.  max_workgroups
        > 0 bounds the fib encode's persistent grid (pkv_encode_segments_bounded)."""
        torch = _torch()
        segs = np.ascontiguousarray(segs, dtype=SEG_DTYPE)
        dtype = L.DT_BF16 if inp.dtype == torch.bfloat16 else L.DT_F32
        if inp.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError("encode input must be float32 or bfloat16")
        if wire.dtype != torch.uint8:
            raise TypeError("wire must be uint8")
        if not (inp.is_contiguous() and wire.is_contiguous()):
            raise ValueError("tensors must be contiguous")
        st = self._status_ptr(status, len(segs))
        if max_workgroups:
            rc = L.lib().pkv_encode_segments_bounded(self.ctx.ptr, self._ptr, radii, dtype, inp.data_ptr(),
                                                     inp.numel(), segs.ctypes.data, len(segs), wire.data_ptr(),
                                                     wire.numel(), max_workgroups, st, _stream_ptr(stream))
            L.check(rc, "pkv_encode_segments_bounded")
            return
        rc = L.lib().pkv_encode_segments(self.ctx.ptr, self._ptr, radii, dtype, inp.data_ptr(), inp.numel(),
                                         segs.ctypes.data, len(segs), wire.data_ptr(), wire.numel(), st,
                                         _stream_ptr(stream))
        L.check(rc, "pkv_encode_segments")

    def decode_segments(self, wire, segs: np.ndarray, out, radii: int = L.RADII_F32, status=None,
                        stream=None, fanout: int = 1, fanout_stride: int = 0, max_workgroups: int = 0) -> None:
        """Decode into `out` (float32, bfloat16 or float16; the latter two are
        the f32 decode rounded to nearest even), each vector written `fanout`
        times `fanout_stride` elements apart.  max_workgroups > 0 bounds the
        head_dim-64 turbo decode's grid (it then loops over the tiles)."""
        torch = _torch()
        segs = np.ascontiguousarray(segs, dtype=SEG_DTYPE)
        dts = {torch.float32: L.DT_F32, torch.bfloat16: L.DT_BF16, torch.float16: L.DT_F16}
        if out.dtype not in dts or wire.dtype != torch.uint8:
            raise TypeError("decode writes float32 / bfloat16 / float16 from a uint8 wire")
        if not (out.is_contiguous() and wire.is_contiguous()):
            raise ValueError("tensors must be contiguous")
        st = self._status_ptr(status, len(segs))
        if max_workgroups:
            rc = L.lib().pkv_decode_segments_bounded(self.ctx.ptr, self._ptr, radii, wire.data_ptr(), wire.numel(),
                                                     segs.ctypes.data, len(segs), out.data_ptr(), dts[out.dtype],
                                                     out.numel(), fanout, fanout_stride, max_workgroups, st,
                                                     _stream_ptr(stream))
            L.check(rc, "pkv_decode_segments_bounded")
            return
        if out.dtype == torch.float32 and fanout == 1:
            rc = L.lib().pkv_decode_segments(self.ctx.ptr, self._ptr, radii, wire.data_ptr(), wire.numel(),
                                             segs.ctypes.data, len(segs), out.data_ptr(), out.numel(), st,
                                             _stream_ptr(stream))
            L.check(rc, "pkv_decode_segments")
            return
        rc = L.lib().pkv_decode_segments_ex(self.ctx.ptr, self._ptr, radii, wire.data_ptr(), wire.numel(),
                                            segs.ctypes.data, len(segs), out.data_ptr(), dts[out.dtype], out.numel(),
                                            fanout, fanout_stride, st, _stream_ptr(stream))
        L.check(rc, "pkv_decode_segments_ex")

    def encode_diagnostics(self, inp, wire, diag, radii: int = L.RADII_F32, status=None, stream=None) -> float:
        """pkv_encode_diagnostics: encode the contiguous float32 device vectors
        `inp` [n, dim] into one blob in `wire` and write the matrix-core values
        the kernel decided from into float32 `diag` (fib: n x 16 x 32 keys;
        turbo: n x proj x (dot, bound)).  Returns the fib key threshold (0 for
        turbo)."""
        torch = _torch()
        if inp.dtype != torch.float32 or diag.dtype != torch.float32 or wire.dtype != torch.uint8:
            raise TypeError("float32 input and diag, uint8 wire")
        n = inp.numel() // self.dim
        thr = C.c_float()
        st = self._status_ptr(status, 1)
        rc = L.lib().pkv_encode_diagnostics(self.ctx.ptr, self._ptr, radii, inp.data_ptr(), n, wire.data_ptr(),
                                            wire.numel(), diag.data_ptr(), diag.numel(), C.byref(thr), st,
                                            _stream_ptr(stream))
        L.check(rc, "pkv_encode_diagnostics")
        return float(thr.value)

    def status_error(self, status_host: np.ndarray, segs: np.ndarray | None = None):
        """Turn per-segment status words (2 per segment, host copy) into a
        PkvError (or None).  The fib batch path reports input-validation
        failures before norm-encoding failures (fib-quant/src/codec.rs:592-610
        precede 694-704); everything else reports the first failing vector."""
        st = np.ascontiguousarray(status_host, dtype=np.uint32).reshape(-1, 2)
        for s, (w0, w1) in enumerate(st):
            if w0 == 0xFFFFFFFF and w1 == 0xFFFFFFFF:
                continue
            if self.kind == L.CODEC_FIB and (segs is None or int(segs[s]["n_vectors"]) >= 4):
                pick = int(w0) if w0 != 0xFFFFFFFF else int(w1)
            else:
                pick = min(int(w0), int(w1))
            kind = pick & 15
            code = {0: L.ERR_NONFINITE_INPUT, 1: L.ERR_ZERO_NORM, 2: L.ERR_NORM_UNREPRESENTABLE,
                    3: L.ERR_NONFINITE_CODE, 4: L.ERR_NONFINITE_CODE}.get(kind, L.ERR_CORRUPT_PAYLOAD)
            return L.PkvError(code, "segment status", s, pick >> 4)
        return None

    # ------------------------------------------------------------ scoring
    def prepared_len(self) -> int:
        return int(L.lib().pkv_prepared_len(self._ptr))

    def prepare_queries(self, queries, prepared=None, status=None, stream=None):
        """TurboQuantizer::prepare_query (turbo-quant/src/turbo.rs:322-338) for
        every row of a float32 device tensor [nq, dim]: [nq, prepared_len]."""
        torch = _torch()
        if queries.dtype != torch.float32 or not queries.is_contiguous():
            raise TypeError("queries must be a contiguous float32 tensor")
        nq = queries.numel() // self.dim
        if queries.numel() != nq * self.dim:
            raise ValueError("queries must hold whole dim-sized rows")
        if prepared is None:
            prepared = torch.empty((nq, self.prepared_len()), dtype=torch.float32, device=queries.device)
        elif prepared.dtype != torch.float32 or prepared.numel() < nq * self.prepared_len():
            raise ValueError("prepared buffer too small")
        st = None if status is None else status.data_ptr()
        rc = L.lib().pkv_turbo_prepare_queries(self.ctx.ptr, self._ptr, queries.data_ptr(), nq, prepared.data_ptr(),
                                               st, _stream_ptr(stream))
        L.check(rc, "pkv_turbo_prepare_queries")
        return prepared

    def score_segments(self, wire, segs: np.ndarray, prepared, scores, ld: int, radii: int = L.RADII_F32,
                       post_scale: float = 1.0, status=None, stream=None, nq: int | None = None,
                       query_stride: int = 0) -> None:
        """inner_product_estimate_prepared (turbo.rs:341-369) of every code of
        every segment against nq prepared queries (segment s: rows
        s * query_stride + q; nq defaults to every row), times post_scale,
        into scores[q * ld + col(i)] (col: the segment addressing in score
        units)."""
        torch = _torch()
        segs = np.ascontiguousarray(segs, dtype=SEG_DTYPE)
        if wire.dtype != torch.uint8 or scores.dtype != torch.float32 or prepared.dtype != torch.float32:
            raise TypeError("score reads a uint8 wire and float32 prepared queries, writes float32")
        if not (wire.is_contiguous() and scores.is_contiguous() and prepared.is_contiguous()):
            raise ValueError("tensors must be contiguous")
        rows = prepared.numel() // self.prepared_len()
        nq = rows if nq is None else nq
        st = self._status_ptr(status, len(segs))
        rc = L.lib().pkv_turbo_score_segments(self.ctx.ptr, self._ptr, radii, wire.data_ptr(), wire.numel(),
                                              segs.ctypes.data, len(segs), prepared.data_ptr(), rows, nq,
                                              query_stride, float(post_scale), scores.data_ptr(), scores.numel(),
                                              ld, st, _stream_ptr(stream))
        L.check(rc, "pkv_turbo_score_segments")

    @staticmethod
    def score_status_error(status_host: np.ndarray):
        """Scoring status words -> PkvError (or None): a rejected code precedes
        a non-finite score within a segment; segments in order."""
        st = np.ascontiguousarray(status_host, dtype=np.uint32)
        err = L.Error()
        rc = L.lib().pkv_score_status(st.ctypes.data, len(st) // 2, C.byref(err))
        return None if rc == 0 else L.PkvError(rc, "score status", err.segment, err.index)

    def score_batch(self, payload: bytes, queries: np.ndarray, post_scale: float = 1.0) -> np.ndarray:
        """Host buffers: scores[nq, n] of one TQB1 blob against host queries
        (prepare_query + score_batch_prepared per query row)."""
        q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, self.dim)
        buf = np.frombuffer(payload, dtype=np.uint8)
        n = C.c_uint64(0)
        err = L.Error()
        rc = L.lib().pkv_parse_header(self._ptr, buf.ctypes.data, len(buf), C.byref(n), None)
        if rc:
            raise L.PkvError(rc, "pkv_parse_header")
        out = np.zeros((len(q), max(int(n.value), 1)), dtype=np.float32)
        rc = L.lib().pkv_turbo_score_batch(self.ctx.ptr, self._ptr, buf.ctypes.data, len(buf), q.ctypes.data, len(q),
                                           float(post_scale), out.ctypes.data, out.size, C.byref(n), C.byref(err))
        if rc:
            raise L.PkvError(rc, "pkv_turbo_score_batch", err.segment, err.index)
        return out[:, :int(n.value)]

    # ------------------------------------------------------------ host buffers
    def encode_batch_compact(self, vectors: np.ndarray, radii: int = L.RADII_F32) -> bytes:
        x = np.ascontiguousarray(vectors, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != self.dim:
            raise L.PkvError(L.ERR_DIM_MISMATCH, "encode_batch_compact")
        n = x.shape[0]
        cap = self.blob_len(n, radii)
        out = np.zeros(max(cap, 1), np.uint8)
        out_len = C.c_uint64()
        err = L.Error()
        rc = L.lib().pkv_encode_batch_compact(self.ctx.ptr, self._ptr, radii, x.ctypes.data if n else None, n,
                                              out.ctypes.data, cap, C.byref(out_len), C.byref(err))
        if rc:
            raise L.PkvError(rc, "encode_batch_compact", err.segment, err.index)
        return out[: out_len.value].tobytes()

    def decode_batch_compact(self, payload: bytes) -> np.ndarray:
        buf = np.frombuffer(bytes(payload) or b"\0", dtype=np.uint8)
        n = C.c_uint64(1)
        radii = C.c_int()
        # a fib payload without the FB2 magic is one FB1 record or one JSON code
        if self.kind != L.CODEC_FIB or payload[:3] == b"FB2":
            rc = L.lib().pkv_parse_header(self._ptr, buf.ctypes.data, len(payload), C.byref(n), C.byref(radii))
            if rc:
                raise L.PkvError(rc, "decode_batch_compact")
        out = np.zeros((max(n.value, 1), self.dim), np.float32)
        n_out = C.c_uint64()
        err = L.Error()
        rc = L.lib().pkv_decode_batch_compact(self.ctx.ptr, self._ptr, buf.ctypes.data, len(payload),
                                              out.ctypes.data, n.value, C.byref(n_out), C.byref(err))
        if rc:
            raise L.PkvError(rc, "decode_batch_compact", err.segment, err.index)
        return out[: n_out.value]


    # ---- per-vector records (TQW1 / FB1): the KVecCodec trait's own methods
    def record_len(self) -> int:
        return int(L.lib().pkv_record_len(self._ptr))

    def encode_vectors(self, vectors: np.ndarray, each: bool) -> list:
        """n vectors -> n TQW1 / FB1 records (``each``: FibQuantizer::encode per
        vector; otherwise encode_batch semantics)."""
        x = np.ascontiguousarray(vectors, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != self.dim:
            raise L.PkvError(L.ERR_DIM_MISMATCH, "encode_vectors")
        n = x.shape[0]
        rec = self.record_len()
        out = np.zeros(max(n * rec, 1), np.uint8)
        out_len = C.c_uint64()
        err = L.Error()
        rc = L.lib().pkv_encode_vectors(self.ctx.ptr, self._ptr, int(each), x.ctypes.data if n else None, n,
                                        out.ctypes.data, n * rec, C.byref(out_len), C.byref(err))
        if rc:
            raise L.PkvError(rc, "encode_vectors", err.segment, err.index)
        b = out.tobytes()
        return [b[i * rec:(i + 1) * rec] for i in range(n)]

    def decode_vectors(self, records, each: bool) -> np.ndarray:
        """TQW1 / FB1 records -> [n, dim] f32 (``each``: FibQuantizer::decode,
        f64 rotation; otherwise decode_batch semantics)."""
        records = [bytes(r) for r in records]
        n = len(records)
        off = np.zeros(n + 1, np.uint64)
        if n:
            off[1:] = np.cumsum([len(r) for r in records], dtype=np.uint64)
        buf = np.frombuffer(b"".join(records) or b"\0", dtype=np.uint8)
        out = np.zeros((max(n, 1), self.dim), np.float32)
        err = L.Error()
        rc = L.lib().pkv_decode_vectors(self.ctx.ptr, self._ptr, int(each), buf.ctypes.data, off.ctypes.data, n,
                                        out.ctypes.data, n, C.byref(err))
        if rc:
            raise L.PkvError(rc, "decode_vectors", err.segment, err.index)
        return out[:n]


# ---------------------------------------------------------------- host only
def turbo_constants(dim: int, projections: int, seed: int):
    signs = np.zeros(dim, np.float32)
    G = np.zeros(max(projections, 1) * dim, np.float32)
    L.check(L.lib().pkv_turbo_constants(dim, projections, seed, signs.ctypes.data,
                                        G.ctypes.data if projections else None), "pkv_turbo_constants")
    return signs, G[: projections * dim].reshape(projections, dim)


def fib_constants(dim: int = 64, k: int = 4, n: int = 32, seed: int = 42, training: int = 2048,
                  restarts: int = 4, iterations: int = 8):
    cb = np.zeros(n * k, np.float32)
    rot = np.zeros(dim * dim, np.float64)
    im, tm = C.c_double(), C.c_double()
    L.check(L.lib().pkv_fib_constants(dim, k, n, seed, training, restarts, iterations, cb.ctypes.data,
                                      rot.ctypes.data, C.byref(im), C.byref(tm)), "pkv_fib_constants")
    return cb.reshape(n, k), rot.reshape(dim, dim), im.value, tm.value
