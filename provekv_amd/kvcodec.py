"""quant-codec-core's codec traits over the device codecs.

The shape and request types restate `quant-codec-core/src/shape.rs`
(KvRole, KvLayout, TokenSpan, KvTensorShape, KvCacheShapeV2, KvSliceRequest)
with the same validation and error kinds (`error.rs`: QuantCodecError), and
`DeviceKvCodec` implements the three traits of `quant-codec-core/src/codec.rs`
(CodecProfile, VectorCodec, KvCacheCodec) over a turbo or fib profile:

* VectorCodec: one self-describing record per vector (TQW1 / FB1, the
  KVecCodec::encode / decode wire form, `proveKV/src/codec.rs:339-413,
  582-637`);
* KvCacheCodec: `encode_kv_cache` turns a whole K|V tensor pair into one
  TQB1 / FB2 blob per (layer, role) in a single launch; `decode_slice` decodes
  one (layer, role) blob on the device and returns the requested token span
  (all heads, or one) in the tensor's own layout.

The reference defines these traits but no codec of the hot path implements
them; the layout conventions below (K then V in one flat array, heads x tokens
or tokens x heads per layer, as `KvLayout` names them) are this module's.
"""
from __future__ import annotations

import enum
from dataclasses import dataclass

import numpy as np

from . import _lib as L
from .device import SEG_DTYPE, Profile


# ---------------------------------------------------------------- errors
class QuantCodecError(ValueError):
    """quant-codec-core/src/error.rs: kind is one of EmptyIdentifier,
    IdentifierWhitespace, InvalidShape, InvalidTokenSpan, ShapeMismatch,
    IntegerOverflow."""

    def __init__(self, kind: str, detail: str = ""):
        self.kind = kind
        super().__init__(f"{kind}: {detail}" if detail else kind)


def _invalid_shape(reason: str) -> QuantCodecError:
    return QuantCodecError("InvalidShape", reason)


# ---------------------------------------------------------------- digests (digest.rs)
class _Digest32:
    """A 32-byte BLAKE3 digest (quant-codec-core/src/digest.rs:6-12): equality,
    ordering and hashing by bytes; str() and to_hex() give lower-case hex.
    The hash runs on a device context (the default one unless given)."""

    __slots__ = ("_b",)

    def __init__(self, digest: bytes):
        digest = bytes(digest)
        if len(digest) != 32:
            raise ValueError("a digest is 32 bytes")
        self._b = digest

    @classmethod
    def from_canonical_bytes(cls, data: bytes, ctx=None):
        """blake3::hash(bytes) (digest.rs:15-17, 34-36)."""
        from .device import default_context
        return cls((ctx or default_context()).blake3(bytes(data)))

    @classmethod
    def from_parts(cls, parts, ctx=None):
        """One hasher fed, per part, its length as a little-endian u64 and then
        its bytes (digest.rs:19-26, 38-45): the hash of that concatenation."""
        buf = bytearray()
        for part in parts:
            part = bytes(part)
            buf += len(part).to_bytes(8, "little") + part
        return cls.from_canonical_bytes(bytes(buf), ctx)

    def as_bytes(self) -> bytes:
        return self._b

    def to_hex(self) -> str:
        return self._b.hex()

    def __str__(self) -> str:
        return self.to_hex()

    def __repr__(self) -> str:
        return f"{type(self).__name__}({self.to_hex()!r})"

    def __eq__(self, other) -> bool:
        return type(other) is type(self) and other._b == self._b

    def __lt__(self, other) -> bool:
        if type(other) is not type(self):
            return NotImplemented
        return self._b < other._b

    def __hash__(self) -> int:
        return hash((type(self).__name__, self._b))


class CodecProfileDigest(_Digest32):
    """quant-codec-core CodecProfileDigest."""


class ArtifactDigest(_Digest32):
    """quant-codec-core ArtifactDigest."""


# ---------------------------------------------------------------- shapes (shape.rs)
class KvRole(enum.Enum):
    KEY = "Key"
    VALUE = "Value"


class DType(enum.Enum):
    F32 = "F32"
    F16 = "F16"
    BF16 = "BF16"
    I8 = "I8"
    U8 = "U8"
    PACKED_BITS = "PackedBits"

    def exact_byte_width(self):
        return {"F32": 4, "F16": 2, "BF16": 2, "I8": 1, "U8": 1}.get(self.value)


@dataclass(frozen=True)
class KvLayout:
    """LayersHeadsTokensDim, LayersTokensHeadsDim or RuntimeSpecific(label)."""
    kind: str
    label: str = ""

    @staticmethod
    def layers_heads_tokens_dim() -> "KvLayout":
        return KvLayout("LayersHeadsTokensDim")

    @staticmethod
    def layers_tokens_heads_dim() -> "KvLayout":
        return KvLayout("LayersTokensHeadsDim")

    @staticmethod
    def runtime_specific(label: str) -> "KvLayout":
        return KvLayout("RuntimeSpecific", label)


@dataclass(frozen=True)
class TokenSpan:
    start: int
    end: int

    @staticmethod
    def new(start: int, end: int) -> "TokenSpan":
        if start >= end:   # shape.rs TokenSpan::new
            raise QuantCodecError("InvalidTokenSpan", f"start={start}, end={end}")
        return TokenSpan(start, end)

    def __len__(self) -> int:
        return self.end - self.start

    def is_empty(self) -> bool:
        return self.start >= self.end


def _checked_product(values, context: str) -> int:
    p = 1
    for v in values:
        p *= int(v)
        if p >= 1 << 64:
            raise QuantCodecError("IntegerOverflow", context)
    return p


def _check_layout(layout: KvLayout) -> None:
    if layout.kind == "RuntimeSpecific" and not layout.label:
        raise _invalid_shape("runtime-specific layout label cannot be empty")


@dataclass(frozen=True)
class KvTensorShape:
    layers: int
    key_heads: int
    value_heads: int
    seq_len: int
    head_dim: int
    layout: KvLayout
    dtype: DType

    @staticmethod
    def gqa(layers, key_heads, value_heads, seq_len, head_dim, layout, dtype) -> "KvTensorShape":
        s = KvTensorShape(layers, key_heads, value_heads, seq_len, head_dim, layout, dtype)
        s.validate()
        return s

    def validate(self) -> None:
        for name in ("layers", "key_heads", "value_heads", "seq_len", "head_dim"):
            if getattr(self, name) == 0:
                raise _invalid_shape(f"{name} must be greater than zero")
        _check_layout(self.layout)

    def heads_for(self, role: KvRole) -> int:
        return self.key_heads if role == KvRole.KEY else self.value_heads

    def layer_element_count(self, role: KvRole) -> int:
        return _checked_product((self.heads_for(role), self.seq_len, self.head_dim), "layer element count")

    def total_element_count(self, role: KvRole) -> int:
        return _checked_product((self.layers, self.heads_for(role), self.seq_len, self.head_dim),
                                "total element count")

    def validate_span(self, span: TokenSpan) -> None:
        if span.is_empty() or span.end > self.seq_len:
            raise QuantCodecError("InvalidTokenSpan", f"start={span.start}, end={span.end}")


@dataclass(frozen=True)
class KvCacheShapeV2:
    batch: int
    layers: int
    num_q_heads: int
    num_kv_heads: int
    seq_len: int
    head_dim: int
    layout: KvLayout
    dtype: DType
    attention_kind: str   # "Mha", "Mqa", "Gqa" or "Unsupported:<label>"

    @staticmethod
    def new(batch, layers, num_q_heads, num_kv_heads, seq_len, head_dim, layout, dtype, attention_kind):
        s = KvCacheShapeV2(batch, layers, num_q_heads, num_kv_heads, seq_len, head_dim, layout, dtype,
                           attention_kind)
        s.validate()
        return s

    @staticmethod
    def mha(batch, layers, heads, seq_len, head_dim, layout, dtype):
        return KvCacheShapeV2.new(batch, layers, heads, heads, seq_len, head_dim, layout, dtype, "Mha")

    @staticmethod
    def mqa(batch, layers, num_q_heads, seq_len, head_dim, layout, dtype):
        return KvCacheShapeV2.new(batch, layers, num_q_heads, 1, seq_len, head_dim, layout, dtype, "Mqa")

    @staticmethod
    def gqa(batch, layers, num_q_heads, num_kv_heads, seq_len, head_dim, layout, dtype):
        return KvCacheShapeV2.new(batch, layers, num_q_heads, num_kv_heads, seq_len, head_dim, layout, dtype, "Gqa")

    def validate(self) -> None:   # shape.rs KvCacheShapeV2::validate
        for name in ("batch", "layers", "num_q_heads", "num_kv_heads", "seq_len", "head_dim"):
            if getattr(self, name) == 0:
                raise _invalid_shape(f"{name} must be greater than zero")
        _check_layout(self.layout)
        q, kv, kind = self.num_q_heads, self.num_kv_heads, self.attention_kind
        if kind == "Mha":
            if q != kv:
                raise _invalid_shape("MHA requires num_q_heads equal to num_kv_heads")
        elif kind == "Mqa":
            if kv != 1 or q <= 1:
                raise _invalid_shape("MQA requires num_kv_heads == 1 and num_q_heads > 1")
        elif kind == "Gqa":
            if q <= kv or kv <= 1:
                raise _invalid_shape("GQA requires num_q_heads > num_kv_heads and num_kv_heads > 1")
            if q % kv:
                raise _invalid_shape("GQA requires num_q_heads divisible by num_kv_heads")
        else:
            label = kind.split(":", 1)[1] if ":" in kind else ""
            if not label.strip():
                raise _invalid_shape("unsupported attention label cannot be empty")
            raise _invalid_shape(f"unsupported attention kind {label} is not adapter-owned")


@dataclass(frozen=True)
class KvSliceRequest:
    layer: int
    role: KvRole
    token_span: TokenSpan
    head: int | None = None

    @staticmethod
    def layer_span(layer: int, token_span: TokenSpan) -> "KvSliceRequest":
        return KvSliceRequest(layer, KvRole.KEY, token_span, None)

    def for_role(self, role: KvRole) -> "KvSliceRequest":
        return KvSliceRequest(self.layer, role, self.token_span, self.head)

    def for_head(self, head: int) -> "KvSliceRequest":
        return KvSliceRequest(self.layer, self.role, self.token_span, head)

    def validate_for_shape(self, shape: KvTensorShape) -> None:
        shape.validate()
        if self.layer >= shape.layers:
            raise QuantCodecError("ShapeMismatch",
                                  f"requested layer {self.layer} but shape has {shape.layers} layers")
        shape.validate_span(self.token_span)
        if self.head is not None and self.head >= shape.heads_for(self.role):
            raise QuantCodecError("ShapeMismatch", f"requested head {self.head} but role has "
                                                   f"{shape.heads_for(self.role)} heads")


# ---------------------------------------------------------------- the codec
@dataclass
class EncodedKvCache:
    """One blob per (layer, role), back to back in `wire` (a device uint8
    tensor): blobs[(layer, role)] = (wire offset, bytes, vectors)."""
    shape: KvTensorShape
    radii: int
    wire: object
    blobs: dict

    @property
    def nbytes(self) -> int:
        return int(self.wire.numel())


class DeviceKvCodec:
    """CodecProfile + VectorCodec + KvCacheCodec (quant-codec-core/src/codec.rs:3-35)
    over one device profile (turbo: pass the radii codec; fib ignores it)."""

    def __init__(self, profile: Profile, codec_id: str, radii: int = L.RADII_F32):
        self.profile = profile
        self._codec_id = codec_id
        self.radii = radii if profile.kind == L.CODEC_TURBO else L.RADII_F32

    # CodecProfile
    def codec_id(self) -> str:
        return self._codec_id

    def codec_version(self) -> str:
        return "TQB1/TQW1 v1" if self.profile.kind == L.CODEC_TURBO else "FB2/FB1 v1"

    def canonical_profile_parts(self) -> list:
        """The profile's canonical parts: codec id, codec version, compact
        sorted-key JSON of the profile kind, head_dim, radii codec and
        constructor parameters, then the resident constants themselves as
        little-endian bytes (turbo: Hadamard signs, QJL matrix; fib: codebook
        f32, rotation f64), so profiles built from caller constants are covered
        too.  No codec of the reference implements CodecProfile; these parts
        are this module's choice."""
        import json
        p = {k: (int(v) if isinstance(v, (int, np.integer)) else v) for k, v in self.profile.params.items()}
        doc = {"kind": "turbo" if self.profile.kind == L.CODEC_TURBO else "fib", "dim": int(self.profile.dim),
               "params": p}
        if self.profile.kind == L.CODEC_TURBO:
            doc["radii"] = "log_u8" if self.radii == L.RADII_LOG_U8 else "f32"
        a, b = self.profile.constants()
        return [self.codec_id().encode(), self.codec_version().encode(),
                json.dumps(doc, sort_keys=True, separators=(",", ":")).encode(),
                np.ascontiguousarray(a).astype(a.dtype.newbyteorder("<")).tobytes(),
                np.ascontiguousarray(b).astype(b.dtype.newbyteorder("<")).tobytes()]

    def profile_digest(self) -> CodecProfileDigest:
        """CodecProfileDigest::from_parts over canonical_profile_parts()
        (quant-codec-core/src/digest.rs:19-26), hashed on the profile's
        device."""
        return CodecProfileDigest.from_parts(self.canonical_profile_parts(), ctx=self.profile.ctx)

    def fixed_rate_bits(self):
        """Bits of one quantized index: the turbo profile's bits, or the fib
        codeword index width (log2 of the codebook size)."""
        p = self.profile.params
        if self.profile.kind == L.CODEC_TURBO:
            return int(p["bits"])
        return int(p["n"]).bit_length() - 1

    def block_dim(self):
        """Values one index covers: the Hadamard block (head_dim) for turbo,
        the sub-vector length k for fib."""
        return self.profile.dim if self.profile.kind == L.CODEC_TURBO else int(self.profile.params["k"])

    def is_lossy(self) -> bool:
        return True

    # VectorCodec: one record per vector
    def encode_block(self, input) -> bytes:
        x = np.ascontiguousarray(input, dtype=np.float32).reshape(1, -1)
        if x.shape[1] != self.profile.dim:
            raise QuantCodecError("ShapeMismatch", f"block of {x.shape[1]} values, codec dim {self.profile.dim}")
        return self.profile.encode_vectors(x, each=True)[0]

    def decode_block(self, block: bytes, out) -> None:
        v = self.profile.decode_vectors([block], each=True)[0]
        if len(out) != v.shape[0]:
            raise QuantCodecError("ShapeMismatch", f"output of {len(out)} values, codec dim {v.shape[0]}")
        out[:] = v

    # KvCacheCodec
    def _check_shape(self, shape: KvTensorShape) -> None:
        shape.validate()
        if shape.head_dim != self.profile.dim:
            raise QuantCodecError("ShapeMismatch", f"head_dim {shape.head_dim}, codec dim {self.profile.dim}")
        if shape.layout.kind not in ("LayersHeadsTokensDim", "LayersTokensHeadsDim"):
            raise QuantCodecError("ShapeMismatch", f"layout {shape.layout.kind}({shape.layout.label}) is not "
                                                   "handled by this codec")

    def encode_kv_cache(self, tensors, shape: KvTensorShape) -> EncodedKvCache:
        """tensors: K ([layers][key_heads x seq_len, in `shape.layout` order][head_dim])
        followed by V (value_heads), one flat f32 array (host or device) or a
        bf16 device tensor.  Vector order inside each (layer, role) blob is the
        tensor's own order (head-major or token-major)."""
        import torch
        self._check_shape(shape)
        want = {DType.F32: torch.float32, DType.BF16: torch.bfloat16}.get(shape.dtype)
        if want is None:
            raise QuantCodecError("ShapeMismatch", f"dtype {shape.dtype.value} is not an encoder input")
        t = tensors if isinstance(tensors, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(tensors))
        t = t.reshape(-1)
        if t.dtype != want:
            raise QuantCodecError("ShapeMismatch", f"tensor dtype {t.dtype}, shape dtype {shape.dtype.value}")
        nk, nv = shape.total_element_count(KvRole.KEY), shape.total_element_count(KvRole.VALUE)
        if t.numel() != nk + nv:
            raise QuantCodecError("ShapeMismatch", f"{t.numel()} values, shape holds {nk + nv}")
        t = t.cuda() if not t.is_cuda else t
        D = shape.head_dim
        rows, blobs, off = [], {}, 0
        for role, base0 in ((KvRole.KEY, 0), (KvRole.VALUE, nk)):
            per_layer = shape.layer_element_count(role)
            n = shape.heads_for(role) * shape.seq_len
            ln = self.profile.blob_len(n, self.radii)
            for layer in range(shape.layers):
                rows.append((base0 + layer * per_layer, 0, D, off, n, n))
                blobs[(layer, role)] = (off, ln, n)
                off += ln
        segs = np.array(rows, dtype=SEG_DTYPE)
        wire = torch.empty(off, dtype=torch.uint8, device=t.device)
        status = torch.empty(2 * len(rows), dtype=torch.int32, device=t.device)
        self.profile.encode_segments(t, segs, wire, radii=self.radii, status=status)
        err = self.profile.status_error(status.cpu().numpy().view(np.uint32), segs)
        if err is not None:
            raise err
        return EncodedKvCache(shape, self.radii, wire, blobs)

    def decode_slice(self, cache: EncodedKvCache, request: KvSliceRequest, out) -> None:
        """Decode request.layer's request.role blob and write the token span
        (one head, or every head) into `out` in the cache's layout:
        [heads][span][head_dim] (LayersHeadsTokensDim) or
        [span][heads][head_dim] (LayersTokensHeadsDim); `out` is a float32
        numpy array or torch tensor with exactly that many values."""
        import torch
        shape = cache.shape
        request.validate_for_shape(shape)
        self._check_shape(shape)
        off, ln, n = cache.blobs[(request.layer, request.role)]
        H, T, D = shape.heads_for(request.role), shape.seq_len, shape.head_dim
        heads = [request.head] if request.head is not None else list(range(H))
        span = request.token_span
        want = len(heads) * len(span) * D
        have = out.size if isinstance(out, np.ndarray) else out.numel()
        if have != want:
            raise QuantCodecError("ShapeMismatch", f"output holds {have} values, the slice {want}")
        scratch = torch.empty(n * D, dtype=torch.float32, device=cache.wire.device)
        seg = np.array([(0, 0, D, off, n, n)], dtype=SEG_DTYPE)
        status = torch.empty(2, dtype=torch.int32, device=cache.wire.device)
        self.profile.decode_segments(cache.wire, seg, scratch, radii=cache.radii, status=status)
        err = self.profile.status_error(status.cpu().numpy().view(np.uint32), seg)
        if err is not None:
            raise err
        idx = torch.tensor(heads, device=scratch.device)
        if shape.layout.kind == "LayersHeadsTokensDim":
            sl = scratch.view(H, T, D).index_select(0, idx)[:, span.start:span.end]
        else:
            sl = scratch.view(T, H, D)[span.start:span.end].index_select(1, idx)
        sl = sl.contiguous().reshape(-1)
        if isinstance(out, np.ndarray):
            out.reshape(-1)[:] = sl.cpu().numpy()
        else:
            out.view(-1).copy_(sl)
