"""ctypes wrapper around the CPU oracle (oracle/pkv_oracle.c, oracle/blake3_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
and by the ``cpu_baseline`` leg of ``bench.py`` -- never by the
``provekv_amd`` product.  Builds the shared library on first use when it is
missing (``make -C oracle``); on the GPU box the prebuilt
``oracle/_build/libpkv_oracle.so`` travels with the tree.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libpkv_oracle.so")

ERRORS = {
    0: "ok",
    -1: "invalid_arg",
    -2: "nonfinite_input",
    -3: "zero_norm",
    -4: "norm_unrepresentable",
    -5: "malformed",
    -6: "radius",
    -7: "residual",
    -8: "capacity",
    -9: "empty",
    -10: "numerical",
}


class OracleError(RuntimeError):
    def __init__(self, code: int, index: int | None = None):
        self.code = code
        self.kind = ERRORS.get(code, str(code))
        self.index = index
        super().__init__(f"oracle error {self.kind} (index={index})")


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p
U32 = C.c_uint32
U64 = C.c_uint64
I32 = C.c_int


def _declare(L):
    L.ora_logf_bits.argtypes = [U32, U64, P]
    L.ora_logf_bits.restype = None
    L.ora_track_reset.argtypes = [I32]
    L.ora_track_reset.restype = None
    L.ora_track_counts.argtypes = [P]
    L.ora_track_counts.restype = None
    L.ora_track_margin.argtypes = []
    L.ora_track_margin.restype = C.c_double
    L.ora_track_tail_logs.argtypes = [P, P, U64]
    L.ora_track_tail_logs.restype = U64
    L.ora_set_codebook_perturbation.argtypes = [C.c_double]
    L.ora_set_codebook_perturbation.restype = None
    L.ora_set_zig_glibc.argtypes = [I32]
    L.ora_set_zig_glibc.restype = None
    L.ora_chacha_words.argtypes = [P, I32, U64, P, U64]
    L.ora_seed_key.argtypes = [U64, P]
    L.ora_rng_u64.argtypes = [U64, P, U64]
    L.ora_normal_f64.argtypes = [U64, P, U64]
    L.ora_gamma_f64.argtypes = [U64, C.c_double, P, U64]
    L.ora_zig_tables.argtypes = [P, P, P]
    L.ora_pcg_draws.argtypes = [U64, U64, I32, C.c_double, C.c_double, P, U64]
    L.ora_pcg_draws.restype = I32
    L.ora_stored_rotation.argtypes = [U32, U64, P, P]
    L.ora_stored_rotation.restype = I32
    L.ora_fib_codebook.argtypes = [U32, U32, U32, U64, U32, U32, U32, P, P, P]
    L.ora_fib_codebook.restype = I32
    L.ora_fib_codebook_report.argtypes = [U32, U32, U32, U64, U32, U32, U32, P, P, P, P, P, U32, P]
    L.ora_fib_codebook_report.restype = I32
    L.ora_inv_norm_cdf.argtypes = [C.c_double]
    L.ora_inv_norm_cdf.restype = C.c_double
    L.ora_beta_inv.argtypes = [C.c_double, C.c_double, C.c_double]
    L.ora_beta_inv.restype = C.c_double
    L.ora_radius_quantile.argtypes = [U32, U32, U32, U32]
    L.ora_radius_quantile.restype = C.c_double
    L.ora_roberts_kronecker.argtypes = [U32, U32, P]
    L.ora_roberts_kronecker.restype = I32
    L.ora_turbo_constants.argtypes = [U32, U32, U64, P, P]
    L.ora_turbo_constants.restype = I32
    L.ora_turbo_rotate.argtypes = [U32, P, P, P]
    L.ora_turbo_rotate_inverse.argtypes = [U32, P, P, P]
    L.ora_turbo_encode_vector.argtypes = [U32, U32, U32, I32, P, P, P, P, P, P]
    L.ora_turbo_encode_vector.restype = I32
    L.ora_turbo_payload_len.argtypes = [U32, U32, U32, I32, I32]
    L.ora_turbo_payload_len.restype = U32
    L.ora_turbo_encode_batch.argtypes = [U32, U32, U32, U64, I32, I32, P, P, P, U64, P, U64, P, P]
    L.ora_turbo_encode_batch.restype = I32
    L.ora_turbo_decode_batch.argtypes = [U32, U32, U32, U64, I32, P, P, U64, P, U64, P, P]
    L.ora_turbo_decode_batch.restype = I32
    L.ora_f32_to_f16.argtypes = [C.c_float]
    L.ora_f32_to_f16.restype = C.c_uint16
    L.ora_f16_to_f32.argtypes = [C.c_uint16]
    L.ora_f16_to_f32.restype = C.c_float
    L.ora_nearest_codeword_k4.argtypes = [P, P, I32]
    L.ora_nearest_codeword_k4.restype = I32
    L.ora_nearest_codeword_k4_avx2.argtypes = [P, P, I32]
    L.ora_nearest_codeword_k4_avx2.restype = I32
    L.ora_nearest_codeword_scalar.argtypes = [P, P, I32, I32]
    L.ora_nearest_codeword_scalar.restype = I32
    L.ora_fib_encode_batch.argtypes = [U32, U32, U32, P, P, P, U64, P, U64, P, P]
    L.ora_fib_encode_batch.restype = I32
    L.ora_fib_decode_batch.argtypes = [U32, U32, U32, P, P, P, U64, P, U64, P, P]
    L.ora_fib_decode_batch.restype = I32
    L.ora_tqw1_record_len.argtypes = [U32, U32, U32, I32]
    L.ora_tqw1_record_len.restype = U32
    L.ora_turbo_encode_tqw1.argtypes = [U32, U32, U32, U64, I32, P, P, P, U64, P, U64, P, P]
    L.ora_turbo_encode_tqw1.restype = I32
    L.ora_turbo_decode_tqw1.argtypes = [U32, U32, U32, U64, I32, P, P, P, U64, P, P]
    L.ora_turbo_decode_tqw1.restype = I32
    L.ora_fb1_record_len.argtypes = [U32, U32, U32]
    L.ora_fb1_record_len.restype = U32
    L.ora_fib_encode_fb1.argtypes = [U32, U32, U32, P, P, P, U64, I32, P, U64, P, P]
    L.ora_fib_encode_fb1.restype = I32
    L.ora_fib_decode_fb1.argtypes = [U32, U32, U32, P, P, P, P, U64, I32, P, P]
    L.ora_fib_decode_fb1.restype = I32
    L.ora_turbo_prepare_query.argtypes = [U32, U32, I32, P, P, P, P]
    L.ora_turbo_prepare_query.restype = I32
    L.ora_turbo_score.argtypes = [U32, U32, U32, U64, I32, P, P, U64, P, U32, P, P, P]
    L.ora_turbo_score.restype = I32
    L.ora_pack_bits.argtypes = [P, U64, I32, P]
    L.ora_unpack_bits.argtypes = [P, U64, I32, P]
    L.ora_unpack_bits.restype = I32
    L.ora_lloyd_refine.argtypes = [P, I32, I32, I32, P, I32, I32, P, P, P]
    L.ora_lloyd_refine.restype = I32
    L.ora_blake3.argtypes = [P, U64, P]
    L.ora_blake3.restype = None
    L.ora_layer_digest.argtypes = [U32, P, P, P]
    L.ora_layer_digest.restype = None
    L.ora_blake3_ranges.argtypes = [P, P, P, U32, P]
    L.ora_blake3_ranges.restype = None


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- RNG pins
def chacha_words(key8, rounds: int, n: int, skip: int = 0) -> np.ndarray:
    key = np.ascontiguousarray(key8, dtype=np.uint32)
    out = np.zeros(n, dtype=np.uint32)
    lib().ora_chacha_words(_p(key), rounds, skip, _p(out), n)
    return out


def seed_key(seed: int) -> np.ndarray:
    out = np.zeros(8, dtype=np.uint32)
    lib().ora_seed_key(seed, _p(out))
    return out


def rng_u64(seed: int, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.uint64)
    lib().ora_rng_u64(seed, _p(out), n)
    return out


def normal_f64(seed: int, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float64)
    lib().ora_normal_f64(seed, _p(out), n)
    return out


def gamma_f64(seed: int, shape: float, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float64)
    lib().ora_gamma_f64(seed, shape, _p(out), n)
    return out


PCG_DRAW = {"u32": 0, "u64": 1, "bool": 2, "f64": 3, "open01": 4, "normal": 5, "gamma": 6}


def pcg_draws(state: int, stream: int, what: str, n: int, p0: float = 0.0, p1: float = 0.0) -> np.ndarray:
    """n draws of a conversion of the oracle's RNG chain fed by rand_pcg's
    Pcg32::new(state, stream) (test hook: the generator of rand 0.8's and
    rand_distr 0.4's value-stability tests).  uint64 for u32 / u64 / bool,
    float64 otherwise."""
    out = np.zeros(n, dtype=np.uint64)
    rc = lib().ora_pcg_draws(state, stream, PCG_DRAW[what], p0, p1, _p(out), n)
    if rc != 0:
        raise OracleError(rc)
    return out if what in ("u32", "u64", "bool") else out.view(np.float64)


def zig_tables():
    x = np.zeros(257)
    f = np.zeros(257)
    r = np.zeros(1)
    lib().ora_zig_tables(_p(x), _p(f), _p(r))
    return x, f, float(r[0])


def stored_rotation(d: int, seed: int):
    m = np.zeros((d, d))
    g = np.zeros(d * d)
    rc = lib().ora_stored_rotation(d, seed, _p(m), _p(g))
    if rc:
        raise OracleError(rc)
    return m, g.reshape(d, d).T.copy()   # gaussian as a row-major [row, col] matrix


def fib_codebook(d=64, k=4, n=32, seed=42, training=2048, restarts=4, iterations=8):
    out = np.zeros(n * k, dtype=np.float32)
    i_mse = np.zeros(1)
    t_mse = np.zeros(1)
    rc = lib().ora_fib_codebook(d, k, n, seed, training, restarts, iterations, _p(out), _p(i_mse), _p(t_mse))
    if rc:
        raise OracleError(rc)
    return out.reshape(n, k), float(i_mse[0]), float(t_mse[0])


_FIB_CONSTANTS = {}


def fib_constants(seed: int = 42, d: int = 64, k: int = 4, n: int = 32, training: int = 2048, restarts: int = 4,
                  iterations: int = 8):
    """The oracle's own fib profile constants (FibQuantAdapter::build_quantizer,
    proveKV/src/codec.rs:471-499): codebook [n, k] f32 (codebook.rs:40-60) and
    rotation [d, d] f64 row-major (rotation.rs:24-58), built once per process
    and per parameters.  Parity tests feed THESE to the oracle, never the
    product's constants."""
    key = (seed, d, k, n, training, restarts, iterations)
    if key not in _FIB_CONSTANTS:
        cb, _, _ = fib_codebook(d, k, n, seed, training, restarts, iterations)
        rot, _ = stored_rotation(d, seed)
        cb.setflags(write=False)
        rot.setflags(write=False)
        _FIB_CONSTANTS[key] = (cb, rot)
    return _FIB_CONSTANTS[key]


def inv_norm_cdf(p: float) -> float:
    return lib().ora_inv_norm_cdf(p)


def beta_inv(q: float, a: float, b: float) -> float:
    return lib().ora_beta_inv(q, a, b)


def radius_quantile(d, k, idx, n) -> float:
    return lib().ora_radius_quantile(d, k, idx, n)


def roberts_kronecker(k, n) -> np.ndarray:
    out = np.zeros(k * n)
    rc = lib().ora_roberts_kronecker(k, n, _p(out))
    if rc:
        raise OracleError(rc)
    return out.reshape(n, k)


# ---------------------------------------------------------------- turbo
def turbo_constants(dim: int, proj: int, seed: int):
    signs = np.zeros(dim, dtype=np.float32)
    G = np.zeros(max(proj, 1) * dim, dtype=np.float32)
    rc = lib().ora_turbo_constants(dim, proj, seed, _p(signs), _p(G))
    if rc:
        raise OracleError(rc)
    return signs, G[: proj * dim].reshape(proj, dim)


def turbo_rotate(signs: np.ndarray, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros_like(x)
    lib().ora_turbo_rotate(len(signs), _p(np.ascontiguousarray(signs, np.float32)), _p(x), _p(y))
    return y


def turbo_rotate_inverse(signs: np.ndarray, y: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(y, dtype=np.float32)
    x = np.zeros_like(y)
    lib().ora_turbo_rotate_inverse(len(signs), _p(np.ascontiguousarray(signs, np.float32)), _p(y), _p(x))
    return x


def turbo_payload_len(dim, bits=4, proj=32, mode=1, radii_codec=0) -> int:
    return int(lib().ora_turbo_payload_len(dim, bits, proj, mode, radii_codec))


def turbo_encode_vector(x, signs, G, bits=4, proj=32, mode=1):
    dim = len(signs)
    x = np.ascontiguousarray(x, dtype=np.float32)
    radii = np.zeros(dim // 2, dtype=np.float32)
    idx = np.zeros(dim // 2, dtype=np.uint16)
    sb = np.zeros(max(1, (proj + 7) // 8), dtype=np.uint8)
    Gc = np.ascontiguousarray(G, dtype=np.float32)
    rc = lib().ora_turbo_encode_vector(dim, bits, proj, mode, _p(np.ascontiguousarray(signs, np.float32)),
                                       _p(Gc), _p(x), _p(radii), _p(idx), _p(sb))
    if rc:
        raise OracleError(rc)
    return radii, idx, sb


def turbo_encode_batch(x: np.ndarray, seed: int, bits=4, proj=32, mode=1, radii_codec=0,
                       signs=None, G=None) -> bytes:
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, dim = x.shape
    if signs is None:
        signs, G = turbo_constants(dim, proj if mode else 0, seed)
    if G is None or G.size == 0:
        G = np.zeros((1, dim), dtype=np.float32)
    plen = turbo_payload_len(dim, bits, proj, mode, radii_codec)
    cap = 38 + n * plen
    out = np.zeros(max(cap, 1), dtype=np.uint8)
    out_len = np.zeros(1, dtype=np.uint64)
    fail = np.zeros(1, dtype=np.uint64)
    rc = lib().ora_turbo_encode_batch(dim, bits, proj, seed, mode, radii_codec, _p(signs),
                                      _p(np.ascontiguousarray(G, np.float32)), _p(x), n, _p(out), cap,
                                      _p(out_len), _p(fail))
    if rc:
        raise OracleError(rc, int(fail[0]))
    return out[: int(out_len[0])].tobytes()


def turbo_decode_batch(blob: bytes, dim: int, seed: int, bits=4, proj=32, mode=1, signs=None) -> np.ndarray:
    if signs is None:
        signs, _ = turbo_constants(dim, 0, seed)
    buf = np.frombuffer(blob, dtype=np.uint8).copy()
    if buf.size == 0:
        buf = np.zeros(1, dtype=np.uint8)
    n_out = np.zeros(1, dtype=np.uint64)
    fail = np.zeros(1, dtype=np.uint64)
    n_guess = max(1, len(blob))
    # first call sizes the output
    rc = lib().ora_turbo_decode_batch(dim, bits, proj, seed, mode, _p(signs), _p(buf), len(blob), None, 0,
                                      _p(n_out), _p(fail))
    if rc not in (0, -8):
        raise OracleError(rc, int(fail[0]))
    n = int(n_out[0])
    out = np.zeros((max(n, 1), dim), dtype=np.float32)
    rc = lib().ora_turbo_decode_batch(dim, bits, proj, seed, mode, _p(signs), _p(buf), len(blob), _p(out), n,
                                      _p(n_out), _p(fail))
    if rc:
        raise OracleError(rc, int(fail[0]))
    del n_guess
    return out[:n]


# ---------------------------------------------------------------- fib
def f32_to_f16(v: float) -> int:
    return int(lib().ora_f32_to_f16(v))


def f16_to_f32(h: int) -> float:
    return float(lib().ora_f16_to_f32(h))


def nearest_codeword_k4(s, cb) -> int:
    s = np.ascontiguousarray(s, dtype=np.float32)
    cb = np.ascontiguousarray(cb, dtype=np.float32)
    return int(lib().ora_nearest_codeword_k4(_p(s), _p(cb), cb.size // 4))


def nearest_codeword_k4_avx2(s, cb) -> int:
    s = np.ascontiguousarray(s, dtype=np.float32)
    cb = np.ascontiguousarray(cb, dtype=np.float32)
    return int(lib().ora_nearest_codeword_k4_avx2(_p(s), _p(cb), cb.size // 4))


def nearest_codeword_scalar(s, cb, k) -> int:
    s = np.ascontiguousarray(s, dtype=np.float32)
    cb = np.ascontiguousarray(cb, dtype=np.float32)
    return int(lib().ora_nearest_codeword_scalar(_p(s), _p(cb), k, cb.size // k))


def fib_encode_batch(x: np.ndarray, codebook: np.ndarray, rotation: np.ndarray) -> bytes:
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, d = x.shape
    N, k = codebook.shape
    cb = np.ascontiguousarray(codebook, dtype=np.float32)
    rot = np.ascontiguousarray(rotation, dtype=np.float64)
    bits = int(N - 1).bit_length()
    plen = 2 + (d // k * bits + 7) // 8
    cap = 19 + n * plen
    out = np.zeros(max(cap, 1), dtype=np.uint8)
    out_len = np.zeros(1, dtype=np.uint64)
    fail = np.zeros(1, dtype=np.uint64)
    rc = lib().ora_fib_encode_batch(d, k, N, _p(cb), _p(rot), _p(x), n, _p(out), cap, _p(out_len), _p(fail))
    if rc:
        raise OracleError(rc, int(fail[0]))
    return out[: int(out_len[0])].tobytes()


def fib_decode_batch(blob: bytes, codebook: np.ndarray, rotation: np.ndarray, d: int = 64) -> np.ndarray:
    N, k = codebook.shape
    cb = np.ascontiguousarray(codebook, dtype=np.float32)
    rot = np.ascontiguousarray(rotation, dtype=np.float64)
    buf = np.frombuffer(blob, dtype=np.uint8).copy()
    if buf.size == 0:
        buf = np.zeros(1, dtype=np.uint8)
    n_out = np.zeros(1, dtype=np.uint64)
    fail = np.zeros(1, dtype=np.uint64)
    rc = lib().ora_fib_decode_batch(d, k, N, _p(cb), _p(rot), _p(buf), len(blob), None, 0, _p(n_out), _p(fail))
    if rc not in (0, -8):
        raise OracleError(rc, int(fail[0]))
    n = int(n_out[0])
    out = np.zeros((max(n, 1), d), dtype=np.float32)
    rc = lib().ora_fib_decode_batch(d, k, N, _p(cb), _p(rot), _p(buf), len(blob), _p(out), n, _p(n_out), _p(fail))
    if rc:
        raise OracleError(rc, int(fail[0]))
    return out[:n]


# ---------------------------------------------------------------- legacy per-vector records
def _records(records):
    """list of bytes -> (concatenated buffer, n + 1 offsets)."""
    off = np.zeros(len(records) + 1, dtype=np.uint64)
    off[1:] = np.cumsum([len(r) for r in records], dtype=np.uint64) if records else []
    buf = np.frombuffer(b"".join(records), dtype=np.uint8).copy()
    if buf.size == 0:
        buf = np.zeros(1, dtype=np.uint8)
    return buf, off


def turbo_encode_tqw1(x: np.ndarray, seed: int, bits=4, proj=32, mode=1) -> list:
    """TurboQuantAdapter::encode on each row -> list of TQW1 records."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, dim = x.shape
    signs, G = turbo_constants(dim, proj if mode else 0, seed)
    if G.size == 0:
        G = np.zeros((1, dim), dtype=np.float32)
    rec = int(lib().ora_tqw1_record_len(dim, bits, proj, mode))
    out = np.zeros(max(n * rec, 1), dtype=np.uint8)
    out_len = np.zeros(1, dtype=np.uint64)
    fail = np.zeros(1, dtype=np.uint64)
    rc = lib().ora_turbo_encode_tqw1(dim, bits, proj, seed, mode, _p(signs), _p(np.ascontiguousarray(G, np.float32)),
                                     _p(x), n, _p(out), n * rec, _p(out_len), _p(fail))
    if rc:
        raise OracleError(rc, int(fail[0]))
    b = out.tobytes()
    return [b[i * rec:(i + 1) * rec] for i in range(n)]


def turbo_decode_tqw1(records: list, dim: int, seed: int, bits=4, proj=32, mode=1) -> np.ndarray:
    """TurboQuantAdapter::decode on each TQW1 record (first failure raises)."""
    signs, _ = turbo_constants(dim, 0, seed)
    buf, off = _records(records)
    out = np.zeros((max(len(records), 1), dim), dtype=np.float32)
    fail = np.zeros(1, dtype=np.uint64)
    rc = lib().ora_turbo_decode_tqw1(dim, bits, proj, seed, mode, _p(signs), _p(buf), _p(off), len(records),
                                     _p(out), _p(fail))
    if rc:
        raise OracleError(rc, int(fail[0]))
    return out[:len(records)]


def fib_encode_fb1(x: np.ndarray, codebook: np.ndarray, rotation: np.ndarray, each: bool) -> list:
    """FibQuantAdapter::encode per row (each) or encode_batch -> FB1 records."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, d = x.shape
    N, k = codebook.shape
    cb = np.ascontiguousarray(codebook, dtype=np.float32)
    rot = np.ascontiguousarray(rotation, dtype=np.float64)
    rec = int(lib().ora_fb1_record_len(d, k, N))
    out = np.zeros(max(n * rec, 1), dtype=np.uint8)
    out_len = np.zeros(1, dtype=np.uint64)
    fail = np.zeros(1, dtype=np.uint64)
    rc = lib().ora_fib_encode_fb1(d, k, N, _p(cb), _p(rot), _p(x), n, int(each), _p(out), n * rec, _p(out_len),
                                  _p(fail))
    if rc:
        raise OracleError(rc, int(fail[0]))
    b = out.tobytes()
    return [b[i * rec:(i + 1) * rec] for i in range(n)]


def fib_decode_fb1(records: list, codebook: np.ndarray, rotation: np.ndarray, each: bool, d: int = 64) -> np.ndarray:
    """FibQuantAdapter::decode per record (each: f64 rotation) or decode_batch
    (parse every record first, then the f32 decode_batch_fast)."""
    N, k = codebook.shape
    cb = np.ascontiguousarray(codebook, dtype=np.float32)
    rot = np.ascontiguousarray(rotation, dtype=np.float64)
    buf, off = _records(records)
    out = np.zeros((max(len(records), 1), d), dtype=np.float32)
    fail = np.zeros(1, dtype=np.uint64)
    rc = lib().ora_fib_decode_fb1(d, k, N, _p(cb), _p(rot), _p(buf), _p(off), len(records), int(each), _p(out),
                                  _p(fail))
    if rc:
        raise OracleError(rc, int(fail[0]))
    return out[:len(records)]


# ---------------------------------------------------------------- scoring on codes
def turbo_prepare_queries(q: np.ndarray, seed: int, proj=32, mode=1) -> np.ndarray:
    """TurboQuantizer::prepare_query per row: [nq, dim + proj] (rotated, projected)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    nq, dim = q.shape
    signs, G = turbo_constants(dim, proj if mode else 0, seed)
    if G.size == 0:
        G = np.zeros((1, dim), dtype=np.float32)
    w = dim + (proj if mode else 0)
    out = np.zeros((nq, w), dtype=np.float32)
    for i in range(nq):
        rc = lib().ora_turbo_prepare_query(dim, proj, mode, _p(signs), _p(np.ascontiguousarray(G, np.float32)),
                                           _p(q[i]), out[i].ctypes.data_as(C.c_void_p))
        if rc:
            raise OracleError(rc, i)
    return out


def turbo_score(blob: bytes, prepared: np.ndarray, dim: int, seed: int, bits=4, proj=32, mode=1) -> np.ndarray:
    """inner_product_estimate_prepared of every code of a TQB1 blob against
    every prepared query: [nq, n]."""
    signs, _ = turbo_constants(dim, 0, seed)
    prepared = np.ascontiguousarray(prepared, dtype=np.float32)
    nq = prepared.shape[0]
    buf = np.frombuffer(blob, dtype=np.uint8).copy()
    n_out = np.zeros(1, dtype=np.uint64)
    fail = np.zeros(1, dtype=np.uint64)
    n = (len(blob) - 38) // max(1, turbo_payload_len(dim, bits, proj, mode, blob[15] if len(blob) > 15 else 0))
    scores = np.zeros((max(nq, 1), max(n, 1)), dtype=np.float32)
    rc = lib().ora_turbo_score(dim, bits, proj, seed, mode, _p(signs), _p(buf), len(blob), _p(prepared), nq,
                               _p(scores), _p(n_out), _p(fail))
    if rc:
        raise OracleError(rc, int(fail[0]))
    return scores[:nq, :int(n_out[0])]


def pack_bits(values, bits: int) -> bytes:
    v = np.ascontiguousarray(values, dtype=np.uint32)
    out = np.zeros(max(1, (len(v) * bits + 7) // 8), dtype=np.uint8)
    lib().ora_pack_bits(_p(v), len(v), bits, _p(out))
    return out[: (len(v) * bits + 7) // 8].tobytes()


def unpack_bits(data: bytes, n: int, bits: int) -> np.ndarray:
    buf = np.frombuffer(data, dtype=np.uint8).copy()
    out = np.zeros(max(n, 1), dtype=np.uint32)
    rc = lib().ora_unpack_bits(_p(buf), n, bits, _p(out))
    if rc:
        raise OracleError(rc)
    return out[:n]


def blake3(data) -> bytes:
    """blake3::hash (the blake3 crate's unkeyed 32-byte hash)."""
    buf = np.frombuffer(bytes(data), dtype=np.uint8).copy() if len(data) else np.zeros(1, np.uint8)
    out = np.zeros(32, np.uint8)
    lib().ora_blake3(_p(buf), len(data), _p(out))
    return out.tobytes()


def blake3_ranges(buf: np.ndarray, ranges) -> np.ndarray:
    """blake3 of each (offset, len) range of a uint8 array: [n, 32]."""
    buf = np.ascontiguousarray(buf, dtype=np.uint8)
    rg = np.ascontiguousarray(np.asarray(ranges, dtype=np.uint64).reshape(-1, 2))
    offs, lens = np.ascontiguousarray(rg[:, 0]), np.ascontiguousarray(rg[:, 1])
    out = np.zeros((len(rg), 32), np.uint8)
    lib().ora_blake3_ranges(_p(buf if buf.size else np.zeros(1, np.uint8)), _p(offs), _p(lens), len(rg), _p(out))
    return out


def layer_digest(layer_index: int, key_digest: bytes, value_digest: bytes) -> bytes:
    """PoolLayer / ShellLayer::compute_digest of a batched layer."""
    k = np.frombuffer(bytes(key_digest), np.uint8).copy()
    v = np.frombuffer(bytes(value_digest), np.uint8).copy()
    out = np.zeros(32, np.uint8)
    lib().ora_layer_digest(layer_index, _p(k), _p(v), _p(out))
    return out.tobytes()


def lloyd_refine(samples: np.ndarray, starts: np.ndarray, iterations: int):
    """refine_codebook's restart loop over given samples [ns, k] and starts
    [restarts, n, k]: (codebooks [restarts, n, k], mse [restarts], init_mse)."""
    s = np.ascontiguousarray(samples, dtype=np.float64)
    st = np.ascontiguousarray(starts, dtype=np.float64)
    ns, k = s.shape
    r, n, _ = st.shape
    out = np.zeros_like(st)
    mse = np.zeros(r)
    init = np.zeros(1)
    rc = lib().ora_lloyd_refine(_p(s), ns, k, n, _p(st), r, iterations, _p(out), _p(mse), _p(init))
    if rc:
        raise OracleError(rc)
    return out, mse, float(init[0])
