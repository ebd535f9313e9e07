"""The acceptance bounds of the encode kernels' matrix-core shortcuts, measured
on real data at full size (pkv_encode_diagnostics).

Both encodes take their fast decisions from matrix-core approximations and
keep one only when a proven error bound says it cannot differ from the
reference's exact f32 arithmetic; everything else is redone exactly:

  fib argmin  key'_w = f32(|c_w|^2 + 1.25 - 2 c_w . rho') must lie within E of
              D_w + 1.25 - |rho_b|^2, D_w the reference's f32 distance
              ((d0^2 + d1^2) + (d2^2 + d3^2), simd_nearest.rs:44-104) at the
              reference's rho = f32(Pi f64(x_hat)) (rotation.rs:107-113); a
              block is decided when its two smallest keys differ by more than
              thr = 2E (1 + 2^-10), otherwise redone exactly
  QJL sign    the matrix-core dot must lie within `bound` of the reference's
              sequential f32 dot (qjl.rs:203-220) whenever |dot'| > bound

The proofs give err <= E and err <= bound.  These tests measure the largest
error the hardware actually produced, relative to the bound, on config-1
(fib), config-2 (QJL d64) and config-4-shaped (QJL d128) data, and require a
margin of at least 2x (ratio <= 0.5); they print the ratios and the redo /
undecided rates.  The reference side is computed on the host from the
oracle's own constants and residuals.
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L
from provekv_amd import synth

pytestmark = pytest.mark.gpu
SEED = 42


def _diag_encode(prof, x, radii):
    import torch
    n, dim = x.shape
    dev = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    wire = torch.empty(prof.blob_len(n, radii), dtype=torch.uint8, device="cuda")
    per = 512 if prof.kind == L.CODEC_FIB else 2 * prof.params["projections"]
    diag = torch.empty(n * per, dtype=torch.float32, device="cuda")
    st = torch.empty(2, dtype=torch.int32, device="cuda")
    thr = prof.encode_diagnostics(dev, wire, diag, radii=radii, status=st)
    torch.cuda.synchronize()
    assert prof.status_error(st.cpu().numpy().view(np.uint32)) is None
    return wire.cpu().numpy().tobytes(), diag.cpu().numpy(), thr


def test_fib_argmin_key_margin(ctx):
    K, V = synth.kv_cache(1, 1, 32, 1024, 64)                 # config-1 distribution (seed 1)
    x = np.ascontiguousarray(np.concatenate([K.reshape(-1, 64), V.reshape(-1, 64)]))   # 65,536 vectors
    n = x.shape[0]
    prof = ctx.fib_profile(64, 4, 32, SEED)
    cb, rot = O.fib_constants(SEED)
    blob, diag, thr = _diag_encode(prof, x, L.RADII_F32)
    assert blob == O.fib_encode_batch(x, cb, rot)
    keys = diag.reshape(n, 16, 32).astype(np.float64)
    # the reference's rho and f32 distances (batch path: x_hat = f32(x / |x|), codec.rs:608)
    x64 = x.astype(np.float64)
    nrm = np.sqrt(np.sum(x64 * x64, axis=1, keepdims=True))
    xh = (x64 / nrm).astype(np.float32).astype(np.float64)
    rho = (xh @ rot.T).astype(np.float32).reshape(n, 16, 1, 4)
    d = cb.reshape(1, 1, 32, 4) - rho                          # f32 subtraction
    sq = d * d
    D = (sq[..., 0] + sq[..., 1]) + (sq[..., 2] + sq[..., 3])  # f32, AVX2 order
    rho64 = rho.astype(np.float64)
    target = D.astype(np.float64) + 1.25 - np.sum(rho64 * rho64, axis=-1)
    E = thr / (2.0 * (1.0 + 2.0 ** -10))   # thr = 2E (1 + 2^-10)
    ratio = float(np.max(np.abs(keys - target)) / E)
    # the kernel's decision: keys with the codeword index in the low 5 bits
    kb = (diag.reshape(n, 16, 32).view(np.uint32) & ~np.uint32(31)) | np.arange(32, dtype=np.uint32)
    kb = np.sort(kb, axis=-1)
    gap = (kb[..., 1] & ~np.uint32(31)).view(np.float32).astype(np.float64) - \
        (kb[..., 0] & ~np.uint32(31)).view(np.float32).astype(np.float64)
    redo_blocks = float(np.mean(~(gap > thr)))
    redo_vectors = float(np.mean(np.any(~(gap > thr), axis=1)))
    print(f"\nMARGIN fib argmin: {n} vectors, E = {E:.3e}, max |key' - exact| / E = {ratio:.4f}, "
          f"blocks redone {redo_blocks:.5f}, vectors with a redo {redo_vectors:.5f}", flush=True)
    assert ratio <= 0.5


def _qjl_margin(prof, x, dim, radii, label):
    n = x.shape[0]
    proj = prof.params["projections"]
    signs, G = O.turbo_constants(dim, proj, SEED)
    blob, diag, _ = _diag_encode(prof, x, radii)
    assert blob == O.turbo_encode_batch(x, SEED, proj=proj, radii_codec=radii, signs=signs, G=G)
    dots = diag.reshape(n, proj, 2)[..., 0].astype(np.float64)
    bnd = diag.reshape(n, proj, 2)[..., 1].astype(np.float64)
    # the encoder's residual: x - decode(code with its exact f32 radii)
    chunks = [x[i:i + 16384] for i in range(0, n, 16384)]

    def rec(c):
        b = O.turbo_encode_batch(c, SEED, proj=proj, radii_codec=0, signs=signs, G=G)
        return O.turbo_decode_batch(b, dim, SEED, proj=proj, signs=signs)
    with ThreadPoolExecutor(8) as ex:
        r = np.concatenate(list(ex.map(rec, chunks)))
    res = (x - r).astype(np.float32)
    ref = np.zeros((n, proj), np.float32)
    for c in range(dim):   # the reference's sequential f32 dot, every projection at once
        ref = (ref + (res[:, c:c + 1] * G[:, c][None, :]).astype(np.float32)).astype(np.float32)
    err = np.abs(dots - ref.astype(np.float64))
    ratio = float(np.max(err / bnd))
    undecided = float(np.mean(~(np.abs(dots) > bnd)))
    accepted = np.abs(dots) > bnd
    assert np.all((dots[accepted] >= 0) == (ref[accepted] >= 0))
    print(f"\nMARGIN QJL {label}: {n} vectors x {proj} projections, max |dot' - dot| / bound = {ratio:.4f}, "
          f"signs recomputed {undecided:.6f}", flush=True)
    assert ratio <= 0.5


def test_qjl_dot_margin_d64(ctx):
    corpus = synth.corpus_tokens(2, 24, 32, 224, 64)          # config 2 (seed 2): 344,064 vectors
    x = np.ascontiguousarray(corpus.reshape(-1, 64))
    _qjl_margin(ctx.turbo_profile(64, 4, 32, SEED, 1), x, 64, L.RADII_F32, "d64 (config 2)")


def test_qjl_dot_margin_d128(ctx):
    xb = synth.device_kv_bf16(4, 2, 8, 8192, 128)            # config-4 distribution, 2 layers
    x = np.ascontiguousarray(xb.float().cpu().numpy().reshape(-1, 128))   # exact bf16 upcast: 262,144 vectors
    _qjl_margin(ctx.turbo_profile(128, 4, 32, SEED, 1), x, 128, L.RADII_LOG_U8, "d128 (config-4 shape)")
