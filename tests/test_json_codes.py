"""The host half of the adapters' JSON fallback, without a GPU.

Before the compact records, proveKV stored a vector's code as the serde_json
text of TurboCode / FibCodeV1, and the adapters still decode such payloads
(proveKV/src/codec.rs:386-393, 552-561, 622-630, 650-658).  The library
parses and checks them on the host (pkv_code_from_json) and decodes the
equivalent record on the device.  Checked here:
  * the payload pkv_code_from_json returns for the JSON the oracle-side
    writer (oracle/json_codes.py, serde's field order) makes of a code equals
    the payload of the oracle's record for that code, byte for byte;
  * fib digests (profile, rotation, codebook with its Lloyd report) equal the
    oracle's, for the paper profile, other seeds and a starved profile whose
    report holds repair events; BLAKE3 on the host against the published
    vectors;
  * serde_json's reading rules, each case with the outcome serde_json 1.0's
    documented behaviour gives (stage 1: does not deserialize; stage 2: the
    code does not fit the profile -- both the adapters' DecompressionFailed);
  * the float layout of the oracle-side writer against serde_json's and
    ryu's own known outputs.
"""
import json
import math

import numpy as np
import pytest

from oracle import json_codes as J
from oracle import oracle as O
from provekv_amd import _lib as L

SEED = 42
TP = L.turbo_params(64, 4, 32, SEED)
FP = L.fib_params(64, 4, 32, SEED)


@pytest.fixture(scope="module")
def turbo_records():
    x = np.random.RandomState(3).randn(24, 64).astype(np.float32)
    x[3] = 0.0                                   # all-zero vector: radii 0, bins 4
    x[4, :2] = [1e-30, -1e-30]
    return O.turbo_encode_tqw1(x, SEED)


@pytest.fixture(scope="module")
def fib_records():
    cb, rot = O.fib_constants(SEED)
    x = np.random.RandomState(4).randn(16, 64).astype(np.float32)
    return O.fib_encode_fb1(x, cb, rot, each=True)


@pytest.fixture(scope="module")
def digests():
    return J.fib_digests(SEED)


def _turbo_obj(rec):
    return json.loads(J.turbo_json_from_record(rec))


def _fib_obj(rec, digests):
    return json.loads(J.fib_json_from_record(rec, digests))


def _dump(obj) -> bytes:
    return json.dumps(obj, separators=(",", ":")).encode()


def _conv(params, text):
    return L.code_from_json(params, text if isinstance(text, bytes) else text.encode())


# ---------------------------------------------------------------- BLAKE3 and digests
def test_host_blake3_published_vectors():
    v = json.load(open(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                                  "blake3_vectors.json")))
    for e in v["vectors"]:
        data = bytes(i % 251 for i in range(e["input_len"]))
        assert L.host_blake3(data).hex() == e["hash"][:64], e["input_len"]
    for e in v["ascii"]:
        assert L.host_blake3(e["input"].encode()).hex() == e["hash"][:64]


@pytest.mark.parametrize("params", [(42, 2048, 4, 8), (0, 2048, 4, 8), (12345, 2048, 4, 8), (42, 64, 2, 3),
                                    (42, 40, 3, 5)])
def test_fib_digests_equal_the_oracle(params):
    seed, training, restarts, iterations = params
    got = L.fib_digests(L.fib_params(64, 4, 32, seed, training, restarts, iterations))
    want = J.fib_digests(seed, training=training, restarts=restarts, iterations=iterations)
    assert got == want
    assert all(g.startswith("blake3:") and len(g) == 71 for g in got)


def test_starved_profile_report_has_repair_events():
    """The (42, 40 samples, 3 restarts, 5 iterations) profile above repairs
    empty cells, so its codebook digest covers LloydRepairEventV1 entries
    (with split_epsilon printed as 1e-6)."""
    _, _, _, _, events, _ = J.codebook_report(training=40, restarts=3, iterations=5)
    assert len(events) > 0
    assert J.json_float(1e-6) == "1e-6"


def test_profile_digest_text():
    # FibQuantProfileV1 field order (profile.rs:95-130) with the adapter overrides
    t = J.fib_profile_json()
    assert t.startswith('{"schema_version":"fib_quant_profile_v1","ambient_dim":64,"block_dim":4,'
                        '"codebook_size":32,"paper_rate_bits_per_coord":1.25,"wire_index_bits":5,'
                        '"wire_bits_per_coord":1.25,"norm_format":"fp16_paper","rotation_seed":42,')
    assert t.endswith('"lloyd_restarts":4,"lloyd_iterations":8,"training_samples":2048,'
                      '"empty_cell_policy":"split_highest_distortion"}')
    assert '"codebook_seed":11400714819323198527,' in t   # 42 + 0x9e3779b97f4a7c15


def test_initial_quantiles_correctly_rounded():
    """The initial codebook's Normal / Beta quantiles (whose last bits reach
    the codebook digest through the Lloyd report's initial MSE) are the
    correctly rounded values for the fib_k4_n32 d64 profile -- save one Beta
    quantile whose exact value lies 0.012 ulp from a rounding midpoint, which
    the long double evaluation (oracle and library alike) rounds up."""
    mp = pytest.importorskip("mpmath")
    mp.mp.prec = 160
    phi = O.lib().ora_roberts_kronecker
    dirs = np.zeros(32 * 4)
    assert phi(4, 32, O._p(dirs)) == 0
    alpha, beta = 2.0, (4 / 6) * ((64 - 4 - 2) / 2) + 1.0
    off = []
    for i in range(32):
        q = (i + 1 - 0.5) / 32
        got = O.lib().ora_beta_inv(q, alpha, beta)
        exact = mp.findroot(lambda x: mp.betainc(alpha, beta, 0, x, regularized=True) - q, got)
        if got != float(exact):
            lo = float(exact)
            frac = float((exact - lo) / (np.nextafter(lo, 2.0) - lo)) if exact > lo else float(
                (lo - exact) / (lo - np.nextafter(lo, -2.0)))
            off.append((q, frac))
    assert len(off) <= 1 and all(q == 0.515625 and abs(f - 0.5) < 0.02 for q, f in off), off


# ---------------------------------------------------------------- payload equality
def test_turbo_json_payload_equals_record_payload(turbo_records):
    for rec in turbo_records:
        rc, stage, pay = _conv(TP, J.turbo_json_from_record(rec))
        assert (rc, stage) == (L.OK, 0)
        assert pay == rec[46:]


def test_fib_json_payload_equals_record_payload(fib_records, digests):
    for rec in fib_records:
        for dg in (digests, (digests[0], "", ""), (digests[0], digests[1], ""), (digests[0], "", digests[2])):
            rc, stage, pay = _conv(FP, J.fib_json_from_record(rec, dg))
            assert (rc, stage) == (L.OK, 0), dg
            assert pay == rec[11:]


# ---------------------------------------------------------------- serde_json reading rules
def test_serde_struct_forms_are_accepted(turbo_records):
    rec = turbo_records[0]
    want = rec[46:]
    o = _turbo_obj(rec)
    pc, qs = o["polar_code"], o["residual_sketch"]
    variants = [
        # fields in another order, and whitespace between tokens
        _dump({"residual_sketch": qs, "polar_code": dict(reversed(list(pc.items())))}),
        json.dumps(o, indent=2).encode() + b" \n\t\r",
        # unknown fields are skipped, whatever they hold (numbers out of f64
        # range, nested arrays deeper than serde_json's recursion limit)
        _dump(o)[:-1] + b',"extra":{"x":[1e999,"\\ud800",null,true,-0]},"deep":' + b"[" * 3000 +
        b"]" * 3000 + b"}",
        # a struct as the array of its fields in declaration order
        _dump([[pc["dim"], pc["bits"], pc["radii"], pc["angle_indices"]], [qs["dim"], qs["projections"],
                                                                           qs["signs"]]]),
        # escaped key names match their fields
        _dump(o).replace(b'"angle_indices"', b'"angle\\u005findices"'),
    ]
    for v in variants:
        rc, stage, pay = _conv(TP, v)
        assert (rc, stage) == (L.OK, 0), v[:80]
        assert pay == want


def _turbo_case(o, path, value):
    o = json.loads(json.dumps(o))
    node = o
    for k in path[:-1]:
        node = node[k]
    if value is _DEL:
        del node[path[-1]]
    else:
        node[path[-1]] = value
    return _dump(o)


_DEL = object()


def test_serde_rejections_turbo(turbo_records):
    o = _turbo_obj(turbo_records[0])
    base = _dump(o)
    raw = [  # (text, stage)
        (base[:-1], 1),                                  # truncated
        (base + b"x", 1),                                # trailing characters
        (base + b"{}", 1),
        (base[:-1] + b",}", 1),                          # trailing comma
        (b"", 1), (b"null", 1), (b"[]", 1), (b"{}", 1),
        (base.replace(b'"polar_code":{', b'"polar_code":{"dim":64,', 1), 1),   # duplicate field
        (base.replace(b'"bits":3', b'"bits":03'), 1),    # leading zero
        (base.replace(b'"bits":3', b'"bits":+3'), 1),
        (base.replace(b'"bits":3', b'"bits":3.0'), 1),   # a float for an integer field
        (base.replace(b'"bits":3', b'"bits":3e0'), 1),
        (base.replace(b'"bits":3', b'"bits":-0'), 1),    # -0 reads as a float
        (base.replace(b'"bits":3', b'"bits":300'), 1),   # out of u8
        (base.replace(b'"bits":3', b'"bits":"3"'), 1),
        (base.replace(b'"dim":64', b'"dim":-64', 1), 1),
        (base.replace(b'"dim":64', b'"dim":18446744073709551616', 1), 1),   # beyond u64: a float
    ]
    pc = o["polar_code"]
    cases = [
        (["polar_code", "radii"], pc["radii"][:-1], 2),                # radius count
        (["polar_code", "radii"], [-1.0] + pc["radii"][1:], 2),        # negative radius
        (["polar_code", "radii"], [1e39] + pc["radii"][1:], 2),        # f32 overflow: not finite
        (["polar_code", "angle_indices"], [8] + pc["angle_indices"][1:], 2),       # >= 2^bits
        (["polar_code", "angle_indices"], [65536] + pc["angle_indices"][1:], 1),   # out of u16
        (["polar_code", "angle_indices"], pc["angle_indices"] + [0], 2),
        (["polar_code", "bits"], 4, 2),                                # the adapter's bits - 1 is 3
        (["polar_code", "dim"], 128, 2),
        (["polar_code", "radii"], _DEL, 1),                            # missing field
        (["residual_sketch"], _DEL, 1),
        (["residual_sketch", "signs"], [128], 1),                      # out of i8
        (["residual_sketch", "signs"], [1.0], 1),
        (["residual_sketch", "projections"], -1, 1),
    ]
    for path, value, stage in cases:
        raw.append((_turbo_case(o, path, value), stage))
    raw.append((base.replace(b'"radii":[', b'"radii":[1e400,', 1), 1))   # f64 out of range: an error
    for text, stage in raw:
        rc, st, _ = _conv(TP, text)
        assert (rc, st) == (L.ERR_CORRUPT_PAYLOAD, stage), text[:120]


def test_serde_values_accepted_turbo(turbo_records):
    o = _turbo_obj(turbo_records[0])
    pc = o["polar_code"]
    ok = [
        (["polar_code", "radii"], [0] + pc["radii"][1:]),                # an integer for an f32
        (["polar_code", "radii"], [-0.0] + pc["radii"][1:]),             # -0.0 >= 0
        (["polar_code", "radii"], [1e-400] + pc["radii"][1:]),           # underflows to 0
        (["residual_sketch", "signs"], [7, -128, 127]),                  # the sketch is not validated
        (["residual_sketch", "dim"], 12345),
    ]
    for path, value in ok:
        rc, st, pay = _conv(TP, _turbo_case(o, path, value))
        assert (rc, st) == (L.OK, 0), (path, value)
        if path[1] == "radii":
            r0 = np.frombuffer(pay[:4], "<f4")[0]
            assert r0 == 0.0 and (math.copysign(1.0, float(r0)) < 0) == (value[0] == -0.0 and
                                                                          str(value[0]) == "-0.0")


def test_number_conversion_like_serde_json(turbo_records):
    """f32 fields take serde_json's f64 (significand and a power of ten, one
    multiply or divide) cast to f32, or an integer cast directly."""
    o = _turbo_obj(turbo_records[0])
    pc = o["polar_code"]
    for text, want in [("0.5", 0.5), ("1", 1.0), ("16777217", 16777216.0), ("2.5e-3", np.float32(0.0025)),
                       ("123456789012345678901234567890", np.float32(1.2345679e29)),
                       ("0.1000000000000000055511151231257827", np.float32(0.1))]:
        t = _dump(o).replace(b'"radii":[' + json.dumps(pc["radii"][0]).encode(), b'"radii":[' + text.encode(), 1)
        rc, st, pay = _conv(TP, t)
        assert (rc, st) == (L.OK, 0), text
        assert np.frombuffer(pay[:4], "<f4")[0] == np.float32(want), text


def test_serde_rejections_fib(fib_records, digests):
    rec = fib_records[0]
    o = _fib_obj(rec, digests)
    base = _dump(o)

    def case(key, value):
        p = dict(o)
        if value is _DEL:
            del p[key]
        else:
            p[key] = value
        return _dump(p)

    cases = [
        (case("schema_version", "fib_code_v2"), 2),
        (case("profile_digest", "blake3:bad"), 2),                     # ProfileDigestMismatch
        (case("profile_digest", ""), 2),                               # compared always
        (case("codebook_digest", "blake3:bad"), 2),                    # CodebookDigestMismatch
        (case("rotation_digest", "blake3:bad"), 2),                    # RotationDigestMismatch
        (case("codebook_digest", digests[2]), 2),                      # the rotation's digest in its place
        (case("ambient_dim", 128), 2),
        (case("block_dim", 8), 2),
        (case("block_count", 15), 2),
        (case("wire_index_bits", 6), 2),
        (case("norm_format", "f32_reference"), 2),                     # a valid variant, not the profile's
        (case("norm_format", "fp32"), 1),                              # no such variant
        (case("norm_format", {"fp16_paper": 0}), 1),
        (case("norm_payload", [0, 60, 0]), 2),                         # fp16 norm length
        (case("norm_payload", [0, 256]), 1),                           # out of u8
        (case("indices", o["indices"] + [0]), 2),                      # packed index length
        (case("indices", _DEL), 1),
        (case("ambient_dim", 2 ** 32), 1),                             # out of u32
        (base.replace(b'"schema_version"', b'"schema_version":"x","schema_version"', 1), 1),
        (base.replace(b'"fib_code_v1"', b'"fib_code_v1\\ud800"', 1), 1),   # lone surrogate in a read string
        (base.replace(b'"fib_code_v1"', b'"fib_code_v1\x01"', 1), 1),     # control character
        (base.replace(b'"fib_code_v1"', b'"fib_code_v1\xff"', 1), 1),     # not UTF-8
    ]
    for text, stage in cases:
        rc, st, _ = _conv(FP, text)
        assert (rc, st) == (L.ERR_CORRUPT_PAYLOAD, stage), text[:160]


def test_serde_values_accepted_fib(fib_records, digests):
    rec = fib_records[1]
    o = _fib_obj(rec, digests)
    ok = [
        {**o, "norm_format": {"fp16_paper": None}},                    # an enum as {variant: null}
        {**o, "schema_version": "fib\\u005fcode_v1"},                 # escapes are decoded
        {**o, "codebook_digest": "", "rotation_digest": ""},           # empty digests are not compared
        {**o, "zzz": "\udcff".encode("utf-8", "surrogatepass").decode("latin-1")},   # skipped strings unchecked
    ]
    for v in ok:
        text = _dump(v).replace(b"\\\\u005f", b"\\u005f")
        rc, st, pay = _conv(FP, text)
        assert (rc, st) == (L.OK, 0), text[:160]
        assert pay == rec[11:]
    # a skipped string may hold bytes that are not UTF-8, and a lone surrogate escape
    t = _dump(o)[:-1] + b',"zzz":"\xff\xfe","yyy":"\\udc00"}'
    assert _conv(FP, t)[:2] == (L.OK, 0)


def test_invalid_parameters():
    bad = L.fib_params(64, 4, 32, SEED, training=16)    # fewer samples than codewords
    rc, st, _ = _conv(bad, b"{}")
    assert rc == L.ERR_INVALID_ARG and st == 0
    rc, st, _ = _conv(L.turbo_params(63, 4, 32, SEED), b"{}")
    assert rc == L.ERR_INVALID_ARG


# ---------------------------------------------------------------- float layout
@pytest.mark.parametrize("value,text", [
    # serde_json tests/test.rs test_write_f64
    (3.0, "3.0"), (3.1, "3.1"), (-1.5, "-1.5"), (0.5, "0.5"),
    (-1.7976931348623157e308, "-1.7976931348623157e308"), (1.7976931348623157e308, "1.7976931348623157e308"),
    (2.220446049250313e-16, "2.220446049250313e-16"),
    # ryu tests/d2s_test.rs (check! prints the value as written)
    (5e-324, "5e-324"), (-2.109808898695963e16, "-2.109808898695963e16"), (4.940656e-318, "4.940656e-318"),
    (1.2345678, "1.2345678"), (1.0, "1.0"), (-0.0, "-0.0"), (0.0, "0.0"),
    # the layout boundaries of ryu's pretty printer
    (1e15, "1000000000000000.0"), (1e16, "1e16"), (123456789.0, "123456789.0"), (0.0001, "0.0001"),
    (1e-5, "0.00001"), (1.5e-6, "1.5e-6"), (float("nan"), "null"), (float("inf"), "null"),
])
def test_json_float_layout_f64(value, text):
    assert J.json_float(value) == text


@pytest.mark.parametrize("value,text", [
    # ryu tests/f2s_test.rs and serde_json's f32 output
    (1.1754944e-38, "1.1754944e-38"), (3.4028235e38, "3.4028235e38"), (0.3, "0.3"), (1.0, "1.0"),
    (-1.5, "-1.5"), (1234567.0, "1234567.0"),
])
def test_json_float_layout_f32(value, text):
    assert J.json_float(np.float32(value), f32=True) == text
