"""Oracle pins for scoring on compressed codes (TurboQuantizer::prepare_query /
inner_product_estimate_prepared, turbo-quant/src/turbo.rs:316-381): each part
of the estimator is checked against an independent float64 computation from
quantities pinned elsewhere (the TQB1 decode, the QJL matrix, the wire's sign
bits), so a transposed rotation, a wrong angle convention, a wrong pair
order, a wrong QJL scale or sign convention fails."""
import math

import numpy as np
import pytest

from oracle import oracle as O

SEED = 42


def _data(seed, n=64, nq=5, dim=64):
    rng = np.random.RandomState(seed)
    return rng.randn(n, dim).astype(np.float32), rng.randn(nq, dim).astype(np.float32)


def test_polar_score_is_inner_product_with_decoded_code():
    """PolarOnly: score = <q, decode(code)> (R orthogonal: the rotated query
    against the rotated reconstruction), up to f32 rounding."""
    x, q = _data(1)
    for bits in (3, 4):
        blob = O.turbo_encode_batch(x, SEED, bits=bits, mode=0)
        s = O.turbo_score(blob, O.turbo_prepare_queries(q, SEED, mode=0), 64, SEED, bits=bits, mode=0)
        dec = O.turbo_decode_batch(blob, 64, SEED, bits=bits, mode=0).astype(np.float64)
        ref = q.astype(np.float64) @ dec.T
        mag = np.abs(q).astype(np.float64) @ np.abs(dec).T
        assert np.all(np.abs(s - ref) <= 1e-5 * mag + 1e-6)


def test_qjl_term_scale_and_sign_convention():
    """With QJL the score adds sqrt(pi/2)/m * sum_j s_j (G q)_j, s_j = +1 for a
    set wire bit, G applied to the raw (unrotated) query, unit source norm."""
    x, q = _data(2)
    blob = O.turbo_encode_batch(x, SEED)                              # bits 4: polar 3 + QJL
    s = O.turbo_score(blob, O.turbo_prepare_queries(q, SEED), 64, SEED)
    polar = O.turbo_score(O.turbo_encode_batch(x, SEED, bits=3, mode=0),
                          O.turbo_prepare_queries(q, SEED, mode=0), 64, SEED, bits=3, mode=0)
    _, G = O.turbo_constants(64, 32, SEED)
    gq = q.astype(np.float64) @ G.astype(np.float64).T                # [nq, 32]
    raw = np.frombuffer(blob, np.uint8)[38:].reshape(len(x), 144)
    bits = np.unpackbits(raw[:, 140:144], axis=1, bitorder="little").astype(np.float64)
    qjl = math.sqrt(math.pi / 2) / 32 * (gq @ (2 * bits - 1).T)       # [nq, n]
    mag = np.abs(gq).sum(axis=1, keepdims=True) * math.sqrt(math.pi / 2) / 32
    assert np.all(np.abs((s - polar) - qjl) <= 1e-5 * (mag + np.abs(polar)) + 1e-5)


def test_zero_vector_closed_form():
    """x = 0: radii 0 (polar term 0) and residual 0, whose sketch signs are all
    +1 (dot >= 0, qjl.rs:215-218): score = sqrt(pi/2)/32 * sum_j (G q)_j."""
    x = np.zeros((3, 64), np.float32)
    q = np.random.RandomState(4).randn(4, 64).astype(np.float32)
    s = O.turbo_score(O.turbo_encode_batch(x, SEED), O.turbo_prepare_queries(q, SEED), 64, SEED)
    _, G = O.turbo_constants(64, 32, SEED)
    ref = math.sqrt(math.pi / 2) / 32 * (q.astype(np.float64) @ G.astype(np.float64).T).sum(axis=1)
    assert np.allclose(s, ref[:, None], rtol=1e-5, atol=1e-5)


def test_score_tracks_the_inner_product_dim128_lossy():
    x, q = _data(5, n=300, nq=4, dim=128)
    blob = O.turbo_encode_batch(x, SEED, radii_codec=1)
    s = O.turbo_score(blob, O.turbo_prepare_queries(q, SEED), 128, SEED)
    ip = q.astype(np.float64) @ x.astype(np.float64).T
    assert np.corrcoef(s.ravel(), ip.ravel())[0, 1] > 0.9


def test_score_errors():
    x, q = _data(6)
    bad_q = q.copy()
    bad_q[2, 7] = np.inf
    with pytest.raises(O.OracleError) as e:
        O.turbo_prepare_queries(bad_q, SEED)
    assert e.value.kind == "nonfinite_input" and e.value.index == 2
    x[9] *= np.float32(1e18)           # radii ~1e18 (finite); with queries ~1e21 only code 9 overflows
    blob = O.turbo_encode_batch(x, SEED)
    with pytest.raises(O.OracleError) as e:
        O.turbo_score(blob, O.turbo_prepare_queries(q * np.float32(1e21), SEED), 64, SEED)
    assert e.value.index == 9
