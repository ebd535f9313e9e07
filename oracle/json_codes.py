"""Writer side of proveKV's legacy JSON code envelope and of fib-quant's
digests, restated in Python over the oracle.

TEST INFRASTRUCTURE ONLY: tests/ use it to write the JSON payloads the
reference stored before its compact records, and the digest strings those
payloads carry, and check the library's reader against them.  Nothing in the
provekv_amd product imports it.

What it restates:
  * serde_json 1.0.150's compact writer (`serde_json::to_vec`) over
    #[derive(Serialize)] structs: fields in declaration order, `"key":value`
    pairs joined by ',' with no whitespace, integers in decimal, Vec<u8> /
    Vec<i8> / Vec<u16> as arrays of integers, snake_case unit variants as
    strings, and floats as the shortest digits that read back to the same
    value, laid out the ryu way (see json_float);
  * TurboCode {polar_code: PolarCode {dim, bits, radii, angle_indices},
    residual_sketch: QjlSketch {dim, projections, signs}}
    (turbo-quant/src/turbo.rs:50-56, polar.rs:35-46, qjl.rs:41-50);
  * FibCodeV1 (fib-quant/src/codec.rs:31-54);
  * json_digest (fib-quant/src/digest.rs:5-13) of FibQuantProfileV1
    (profile.rs:95-130, 256-262), of StoredRotation's digest view
    (rotation.rs:80-100) and of FibCodebookV1's (codebook.rs:133-157, with
    LloydReportV1 / LloydRepairEventV1, lloyd.rs:17-59).
The shortest digits come from Python's float repr (f64) and numpy's float32
str (f32), both independent of the library's std::to_chars.
"""
from __future__ import annotations

import math
from decimal import Decimal

import numpy as np

from oracle import oracle as O


# ---------------------------------------------------------------- serde_json floats
def _digits(text: str):
    """(digit string, kk) with value = 0.digits * 10^kk, trailing zeros removed."""
    t = Decimal(text).normalize().as_tuple()
    digits = "".join(str(d) for d in t.digits)
    return digits, t.exponent + len(digits)


def json_float(x, f32: bool = False) -> str:
    """serde_json's text of an f64 (or f32) field: 'null' if not finite,
    '0.0' / '-0.0' for zeros; else the shortest round-trip digits d with
    10^(kk-1) <= |x| < 10^kk laid out as the ryu crate prints them: digits
    then zeros then '.0' when the value is an integer of at most 16 (f64) /
    13 (f32) digits, a decimal point inside the digits up to that many
    integer digits, '0.' and -kk zeros for kk in (-5, 0], otherwise
    d.ddd 'e' (kk - 1) with no '+' and no zero padding."""
    x = float(x)
    if not math.isfinite(x):
        return "null"
    if x == 0.0:
        return "-0.0" if math.copysign(1.0, x) < 0 else "0.0"
    neg = x < 0
    text = str(np.float32(abs(x))) if f32 else repr(abs(x))
    d, kk = _digits(text)
    k = kk - len(d)
    lim = 13 if f32 else 16
    if k >= 0 and kk <= lim:
        s = d + "0" * k + ".0"
    elif 0 < kk <= lim:
        s = d[:kk] + "." + d[kk:]
    elif -5 < kk <= 0:
        s = "0." + "0" * (-kk) + d
    else:
        s = d[0] + ("." + d[1:] if len(d) > 1 else "") + "e" + str(kk - 1)
    return ("-" if neg else "") + s


def _obj(pairs) -> str:
    return "{" + ",".join('"%s":%s' % (k, v) for k, v in pairs) + "}"


def _arr(items) -> str:
    return "[" + ",".join(items) + "]"


def _s(text: str) -> str:   # the ASCII identifiers and digests written here need no escapes
    return '"%s"' % text


# ---------------------------------------------------------------- turbo
def turbo_code_json(radii, angles, signs, dim: int, polar_bits: int, projections: int) -> bytes:
    """serde_json::to_vec(&TurboCode)."""
    pc = _obj([("dim", str(dim)), ("bits", str(polar_bits)),
               ("radii", _arr(json_float(r, f32=True) for r in np.asarray(radii, np.float32))),
               ("angle_indices", _arr(str(int(a)) for a in angles))])
    qs = _obj([("dim", str(dim)), ("projections", str(projections)), ("signs", _arr(str(int(s)) for s in signs))])
    return _obj([("polar_code", pc), ("residual_sketch", qs)]).encode()


def turbo_code_from_payload(payload: bytes, dim: int, polar_bits: int, projections: int):
    """(radii, angle indices, signs) of one TQW1 / TQB1 f32-radii payload
    (wire.rs:347-398: radii LE f32, LSB-first packed angles, sign bit 1 = +1)."""
    pairs = dim // 2
    radii = np.frombuffer(payload[:4 * pairs], "<f4").copy()
    ab = (pairs * polar_bits + 7) // 8
    angles = O.unpack_bits(payload[4 * pairs:4 * pairs + ab], pairs, polar_bits)
    sb = payload[4 * pairs + ab:4 * pairs + ab + (projections + 7) // 8]
    signs = [1 if (sb[j // 8] >> (j % 8)) & 1 else -1 for j in range(projections)]
    return radii, [int(a) for a in angles], signs


def turbo_json_from_record(record: bytes, dim: int = 64, bits: int = 4, projections: int = 32) -> bytes:
    """The JSON the reference wrote for the code a TQW1 record holds."""
    return turbo_code_json(*turbo_code_from_payload(record[46:], dim, bits - 1, projections), dim, bits - 1,
                           projections)


# ---------------------------------------------------------------- fib
def fib_code_json(norm: bytes, indices: bytes, profile_digest: str, codebook_digest: str, rotation_digest: str,
                  dim: int = 64, k: int = 4, wire_bits: int = 5, norm_format: str = "fp16_paper",
                  schema: str = "fib_code_v1") -> bytes:
    """serde_json::to_vec(&FibCodeV1)."""
    return _obj([("schema_version", _s(schema)), ("profile_digest", _s(profile_digest)),
                 ("codebook_digest", _s(codebook_digest)), ("rotation_digest", _s(rotation_digest)),
                 ("ambient_dim", str(dim)), ("block_dim", str(k)), ("norm_format", _s(norm_format)),
                 ("norm_payload", _arr(str(b) for b in norm)), ("wire_index_bits", str(wire_bits)),
                 ("block_count", str(dim // k)), ("indices", _arr(str(b) for b in indices))]).encode()


def fib_json_from_record(record: bytes, digests, dim: int = 64, k: int = 4) -> bytes:
    """The JSON FibQuantizer::encode's code serialises to, for the code an FB1
    record holds (record = 11-byte header, 2 norm bytes, packed indices);
    digests = (profile, codebook, rotation) as FibQuantizer::encode fills them."""
    return fib_code_json(record[11:13], record[13:], digests[0], digests[1], digests[2], dim, k, record[4])


def fib_profile_json(dim=64, k=4, n=32, seed=42, training=2048, restarts=4, iterations=8) -> str:
    """FibQuantProfileV1 of FibQuantAdapter::build_quantizer (paper_default,
    profile.rs:132-173, with the adapter's training overrides)."""
    wbits = (n - 1).bit_length()
    return _obj([
        ("schema_version", _s("fib_quant_profile_v1")), ("ambient_dim", str(dim)), ("block_dim", str(k)),
        ("codebook_size", str(n)), ("paper_rate_bits_per_coord", json_float(math.log2(n) / k)),
        ("wire_index_bits", str(wbits)), ("wire_bits_per_coord", json_float(wbits / k)),
        ("norm_format", _s("fp16_paper")), ("rotation_seed", str(seed)),
        ("rotation_algorithm_version", _s("qr-gaussian-chacha8-sign-corrected-v1")),
        ("codebook_seed", str((seed + 0x9e3779b97f4a7c15) % 2 ** 64)),
        ("codebook_version", _s("fib-quant:paper-core-v1")), ("source_mode", _s("canonical_spherical_beta")),
        ("radius_method", _s("k2_closed_form" if k == 2 else "beta_quantile")),
        ("direction_method", _s({2: "fibonacci_spiral", 3: "fibonacci_sphere"}.get(k, "roberts_kronecker"))),
        ("lloyd_restarts", str(restarts)), ("lloyd_iterations", str(iterations)),
        ("training_samples", str(training)), ("empty_cell_policy", _s("split_highest_distortion"))])


def json_digest(domain: str, text: str) -> str:
    """fib-quant/src/digest.rs:5-13."""
    return "blake3:" + O.blake3(domain.encode() + b"\0" + text.encode()).hex()


def codebook_report(dim=64, k=4, n=32, seed=42, training=2048, restarts=4, iterations=8):
    """The oracle's codebook build with its LloydReportV1 fields."""
    cb = np.zeros(n * k, np.float32)
    im, tm = np.zeros(1), np.zeros(1)
    best = np.zeros(1, np.uint32)
    cap = 4096
    ev = np.zeros(7 * cap)
    ne = np.zeros(1, np.uint32)
    rc = O.lib().ora_fib_codebook_report(dim, k, n, seed, training, restarts, iterations, O._p(cb), O._p(im),
                                         O._p(tm), O._p(best), O._p(ev), cap, O._p(ne))
    if rc:
        raise O.OracleError(rc)
    events = [tuple(ev[7 * i:7 * i + 7]) for i in range(min(int(ne[0]), cap))]
    return cb, float(im[0]), float(tm[0]), int(best[0]), events, max(training, n)


_DIGESTS = {}


def fib_digests(seed=42, dim=64, k=4, n=32, training=2048, restarts=4, iterations=8):
    """(profile, codebook, rotation) digests of the adapter's fib profile,
    from the oracle's own constants."""
    key = (seed, dim, k, n, training, restarts, iterations)
    if key in _DIGESTS:
        return _DIGESTS[key]
    profile = json_digest("fib_quant_profile_v1", fib_profile_json(dim, k, n, seed, training, restarts, iterations))
    rot, _ = O.stored_rotation(dim, seed)
    rotation = json_digest("fib_rotation_v1", _obj([
        ("rotation_schema", _s("fib_rotation_v1")),
        ("algorithm_version", _s("qr-gaussian-chacha8-sign-corrected-v1")), ("dim", str(dim)), ("seed", str(seed)),
        ("matrix", _arr(json_float(v) for v in rot.reshape(-1)))]))
    cb, init_mse, best_mse, best_restart, events, ns = codebook_report(dim, k, n, seed, training, restarts,
                                                                       iterations)
    report = _obj([
        ("schema_version", _s("lloyd_report_v1")), ("restarts", str(max(restarts, 1))),
        ("iterations", str(iterations)), ("training_samples", str(ns)), ("init_mse", json_float(init_mse)),
        ("best_mse", json_float(best_mse)), ("best_restart", str(best_restart)),
        ("empty_cells_repaired", str(len(events))),
        ("repair_events", _arr(_obj([
            ("restart", str(int(e[0]))), ("iteration", str(int(e[1]))), ("empty_cell", str(int(e[2]))),
            ("donor_cell", str(int(e[3]))), ("donor_count_before", str(int(e[4]))),
            ("donor_distortion", json_float(e[5])), ("residual_norm", json_float(e[6])),
            ("split_epsilon", json_float(1e-6))]) for e in events)),
        ("seed", str((seed + 0x9e3779b97f4a7c15) % 2 ** 64))])
    codebook = json_digest("fib_codebook_v1", _obj([
        ("schema_version", _s("fib_codebook_v1")), ("profile_digest", _s(profile)),
        ("rotation_digest", _s(rotation)), ("codewords", _arr(json_float(v, f32=True) for v in cb)),
        ("init_mse", json_float(init_mse)), ("training_mse", json_float(best_mse)), ("refinement_report", report)]))
    _DIGESTS[key] = (profile, codebook, rotation)
    return _DIGESTS[key]
