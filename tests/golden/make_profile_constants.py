"""Regenerates tests/golden/profile_constants_seed42.npz from the library's
host constant generators (pkv_turbo_constants / pkv_fib_constants, no GPU).
The file lets anyone holding the Rust reference diff the seed-42 profile
constants once (FastHadamardRotation signs, QJL matrix, StoredRotation,
FibCodebookV1 codewords).

The file is the library's own output, so it is a regression pin (it catches
a change in the generators), not a parity pin against the reference."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from provekv_amd import device as D  # noqa: E402

cb, rot, _, _ = D.fib_constants(seed=42)
signs, G = D.turbo_constants(64, 32, 42)
np.savez(os.path.join(ROOT, "tests", "golden", "profile_constants_seed42.npz"), fib_codebook=cb,
         fib_rotation=rot, turbo_signs_d64=signs, turbo_qjl_32x64=G)
