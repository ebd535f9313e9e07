"""quant-codec-core traits over the device codecs (provekv_amd.kvcodec):
encode_kv_cache writes one blob per (layer, role) whose bytes equal the
oracle's batch encode of that role's vectors in the tensor's own order;
decode_slice returns the oracle decode of the requested rows bit for bit;
encode_block / decode_block are the per-vector records (TQW1 / FB1)."""
import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L
from provekv_amd import synth
from provekv_amd.kvcodec import (DeviceKvCodec, DType, KvLayout, KvRole, KvSliceRequest, KvTensorShape,
                                 QuantCodecError, TokenSpan)

pytestmark = pytest.mark.gpu
SEED = 42


def _tensors(seed, shape):
    """K then V, each in `shape.layout` order, float32."""
    parts = []
    for role in (KvRole.KEY, KvRole.VALUE):
        H = shape.heads_for(role)
        x = synth.kv_cache(seed + (role == KvRole.VALUE), shape.layers, H, shape.seq_len, shape.head_dim)[0]
        x = x.astype(np.float32)   # [L][H][T][D]
        if shape.layout.kind == "LayersTokensHeadsDim":
            x = np.ascontiguousarray(x.transpose(0, 2, 1, 3))
        parts.append(x.reshape(-1))
    return np.concatenate(parts)


def _role_rows(flat, shape, layer, role):
    nk = shape.total_element_count(KvRole.KEY)
    base = 0 if role == KvRole.KEY else nk
    per = shape.layer_element_count(role)
    return flat[base + layer * per: base + (layer + 1) * per].reshape(-1, shape.head_dim)


def _codecs(ctx):
    tur = ctx.turbo_profile(64, 4, 32, SEED)
    fib = ctx.fib_profile(64, 4, 32, SEED)
    cb, rot = O.fib_constants(SEED)
    return [
        (DeviceKvCodec(tur, "turbo_8bit_batched"), lambda x: O.turbo_encode_batch(x, SEED),
         lambda b: O.turbo_decode_batch(b, 64, SEED)),
        (DeviceKvCodec(tur, "turbo_8bit_batched_lossy", radii=L.RADII_LOG_U8),
         lambda x: O.turbo_encode_batch(x, SEED, radii_codec=1), lambda b: O.turbo_decode_batch(b, 64, SEED)),
        (DeviceKvCodec(fib, "fib_k4_n32_batched"), lambda x: O.fib_encode_batch(x, cb.reshape(32, 4), rot.reshape(64, 64)),
         lambda b: O.fib_decode_batch(b, cb.reshape(32, 4), rot.reshape(64, 64))),
    ]


@pytest.mark.parametrize("layout", ["LayersHeadsTokensDim", "LayersTokensHeadsDim"])
def test_encode_kv_cache_and_decode_slice_bit_exact(ctx, layout):
    shape = KvTensorShape.gqa(2, 2, 3, 37, 64, KvLayout(layout), DType.F32)
    flat = _tensors(7, shape)
    for codec, enc, dec in _codecs(ctx):
        cache = codec.encode_kv_cache(flat, shape)
        wire = cache.wire.cpu().numpy()
        for (layer, role), (off, ln, n) in cache.blobs.items():
            rows = _role_rows(flat, shape, layer, role)
            assert n == rows.shape[0]
            ref_blob = enc(rows)
            assert wire[off:off + ln].tobytes() == ref_blob, (codec.codec_id(), layer, role)
            ref = dec(ref_blob).reshape(-1, 64)
            H, T = shape.heads_for(role), shape.seq_len
            for head in (None, H - 1):
                req = KvSliceRequest.layer_span(layer, TokenSpan.new(5, 29)).for_role(role)
                if head is not None:
                    req = req.for_head(head)
                heads = [head] if head is not None else list(range(H))
                out = np.zeros(len(heads) * 24 * 64, np.float32)
                codec.decode_slice(cache, req, out)
                if layout == "LayersHeadsTokensDim":
                    want = ref.reshape(H, T, 64)[heads][:, 5:29]
                else:
                    want = ref.reshape(T, H, 64)[5:29][:, heads]
                assert np.array_equal(out.view(np.uint32), np.ascontiguousarray(want).reshape(-1).view(np.uint32))


def test_encode_kv_cache_bf16_device_input(ctx):
    import torch
    shape = KvTensorShape.gqa(1, 4, 2, 50, 64, KvLayout.layers_tokens_heads_dim(), DType.BF16)
    flat = torch.from_numpy(_tensors(3, shape)).to(torch.bfloat16)
    codec, enc, dec = _codecs(ctx)[0]
    cache = codec.encode_kv_cache(flat.cuda(), shape)
    up = flat.to(torch.float32).numpy()
    off, ln, n = cache.blobs[(0, KvRole.VALUE)]
    assert cache.wire[off:off + ln].cpu().numpy().tobytes() == enc(_role_rows(up, shape, 0, KvRole.VALUE))
    out = torch.zeros(50 * 2 * 64, dtype=torch.float32, device="cuda")
    codec.decode_slice(cache, KvSliceRequest.layer_span(0, TokenSpan.new(0, 50)).for_role(KvRole.VALUE), out)
    ref = dec(enc(_role_rows(up, shape, 0, KvRole.VALUE))).reshape(-1)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_vector_codec_blocks_are_records(ctx):
    x = _tensors(9, KvTensorShape.gqa(1, 1, 1, 5, 64, KvLayout.layers_heads_tokens_dim(), DType.F32))[:64]
    tur = ctx.turbo_profile(64, 4, 32, SEED)
    fib = ctx.fib_profile(64, 4, 32, SEED)
    cb, rot = O.fib_constants(SEED)
    tc, fc = DeviceKvCodec(tur, "turbo_8bit"), DeviceKvCodec(fib, "fib_k4_n32")
    tb, fb = tc.encode_block(x), fc.encode_block(x)
    assert tb == O.turbo_encode_tqw1(x[None], SEED)[0]
    assert fb == O.fib_encode_fb1(x[None], cb.reshape(32, 4), rot.reshape(64, 64), each=True)[0]
    out = np.zeros(64, np.float32)
    tc.decode_block(tb, out)
    assert np.array_equal(out.view(np.uint32), O.turbo_decode_tqw1([tb], 64, SEED)[0].view(np.uint32))
    fc.decode_block(fb, out)
    assert np.array_equal(out.view(np.uint32),
                          O.fib_decode_fb1([fb], cb.reshape(32, 4), rot.reshape(64, 64), each=True)[0].view(np.uint32))
    assert (tc.fixed_rate_bits(), tc.block_dim(), fc.fixed_rate_bits(), fc.block_dim()) == (4, 64, 5, 4)
    with pytest.raises(QuantCodecError):
        tc.encode_block(x[:32])


def test_kv_codec_rejects_bad_requests(ctx):
    shape = KvTensorShape.gqa(2, 2, 2, 16, 64, KvLayout.layers_heads_tokens_dim(), DType.F32)
    codec = _codecs(ctx)[0][0]
    cache = codec.encode_kv_cache(_tensors(1, shape), shape)
    out = np.zeros(2 * 4 * 64, np.float32)
    with pytest.raises(QuantCodecError) as e:
        codec.decode_slice(cache, KvSliceRequest.layer_span(2, TokenSpan.new(0, 4)), out)
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(QuantCodecError) as e:
        codec.decode_slice(cache, KvSliceRequest.layer_span(0, TokenSpan.new(14, 18)), out)
    assert e.value.kind == "InvalidTokenSpan"
    with pytest.raises(QuantCodecError) as e:   # output sized for one head, request asks for two
        codec.decode_slice(cache, KvSliceRequest.layer_span(0, TokenSpan.new(0, 8)), out[:8 * 64])
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(QuantCodecError):
        codec.encode_kv_cache(_tensors(1, shape)[:-1], shape)
    bad = KvTensorShape.gqa(1, 1, 1, 4, 128, KvLayout.layers_heads_tokens_dim(), DType.F32)
    with pytest.raises(QuantCodecError):
        codec.encode_kv_cache(np.zeros(2 * 4 * 128, np.float32), bad)
