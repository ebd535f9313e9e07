"""quant-codec-core shape / request validation (quant-codec-core/src/shape.rs),
restated in provekv_amd.kvcodec: the reference's own cases
(quant-codec-core/tests/shape_validation.rs) and the remaining branches."""
import pytest

from provekv_amd.kvcodec import (DType, KvCacheShapeV2, KvLayout, KvRole, KvSliceRequest, KvTensorShape,
                                 QuantCodecError, TokenSpan)

LHTD = KvLayout.layers_heads_tokens_dim()


def test_validates_shape_and_spans():
    assert KvTensorShape.gqa(2, 2, 4, 8, 16, LHTD, DType.F32)
    with pytest.raises(QuantCodecError):
        KvTensorShape.gqa(0, 2, 4, 8, 16, LHTD, DType.F32)
    for a, b in ((4, 4), (5, 4)):
        with pytest.raises(QuantCodecError) as e:
            TokenSpan.new(a, b)
        assert e.value.kind == "InvalidTokenSpan"


def test_rejects_out_of_bounds_slice_request():
    shape = KvTensorShape.gqa(2, 2, 4, 8, 16, LHTD, DType.F32)
    req = KvSliceRequest.layer_span(2, TokenSpan.new(0, 1))
    with pytest.raises(QuantCodecError) as e:
        req.validate_for_shape(shape)
    assert e.value.kind == "ShapeMismatch"


def test_slice_request_head_span_and_role():
    shape = KvTensorShape.gqa(2, 2, 4, 8, 16, LHTD, DType.F32)
    ok = KvSliceRequest.layer_span(1, TokenSpan.new(3, 8)).for_role(KvRole.VALUE).for_head(3)
    ok.validate_for_shape(shape)                      # value role has 4 heads
    with pytest.raises(QuantCodecError) as e:
        KvSliceRequest.layer_span(1, TokenSpan.new(3, 8)).for_head(3).validate_for_shape(shape)   # keys: 2 heads
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(QuantCodecError) as e:
        KvSliceRequest.layer_span(0, TokenSpan.new(3, 9)).validate_for_shape(shape)   # past seq_len
    assert e.value.kind == "InvalidTokenSpan"


def test_shape_counts_and_overflow():
    shape = KvTensorShape.gqa(3, 2, 4, 10, 16, LHTD, DType.BF16)
    assert shape.layer_element_count(KvRole.KEY) == 2 * 10 * 16
    assert shape.total_element_count(KvRole.VALUE) == 3 * 4 * 10 * 16
    huge = KvTensorShape.gqa(1 << 20, 1 << 20, 1, 1 << 20, 1 << 20, LHTD, DType.F32)
    with pytest.raises(QuantCodecError) as e:
        huge.total_element_count(KvRole.KEY)
    assert e.value.kind == "IntegerOverflow"
    with pytest.raises(QuantCodecError) as e:
        KvTensorShape.gqa(1, 1, 1, 1, 64, KvLayout.runtime_specific(""), DType.F32)
    assert e.value.kind == "InvalidShape"
    assert DType.BF16.exact_byte_width() == 2 and DType.PACKED_BITS.exact_byte_width() is None


def test_shape_v2_accepts_mha_mqa_and_gqa_contracts():
    assert KvCacheShapeV2.mha(1, 2, 8, 16, 64, LHTD, DType.F32)
    assert KvCacheShapeV2.mqa(1, 2, 8, 16, 64, LHTD, DType.F32)
    assert KvCacheShapeV2.gqa(1, 2, 8, 2, 16, 64, LHTD, DType.F32)


@pytest.mark.parametrize("args", [
    (0, 2, 8, 8, 16, 64, "Mha"),
    (1, 2, 8, 4, 16, 64, "Mha"),
    (1, 2, 1, 1, 16, 64, "Mqa"),
    (1, 2, 10, 4, 16, 64, "Gqa"),
    (1, 2, 8, 8, 16, 64, "Gqa"),
])
def test_shape_v2_rejects_invalid_attention_contracts(args):
    b, l, q, kv, t, d, kind = args
    with pytest.raises(QuantCodecError) as e:
        KvCacheShapeV2.new(b, l, q, kv, t, d, LHTD, DType.F32, kind)
    assert e.value.kind == "InvalidShape"


def test_shape_v2_unsupported_attention_fails_closed():
    with pytest.raises(QuantCodecError) as e:
        KvCacheShapeV2.new(1, 2, 8, 8, 16, 64, LHTD, DType.F32, "Unsupported:mla")
    assert e.value.kind == "InvalidShape" and "mla" in str(e.value)
