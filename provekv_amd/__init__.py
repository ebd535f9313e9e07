"""provekv_amd -- MI355X (gfx950) implementation of proveKV's codec hot path.

Layers (bottom up):
  * ``libpkv_hip.so`` (csrc/): gfx950 kernels and the C ABI of
    include/pkv_codec.h -- the drop-in for the reference's gpu-backend crate;
  * ``_lib``: ctypes binding of that ABI;
  * ``device``: context / profiles / segment tables over torch device tensors;
  * ``codec``: the proveKV plugin surface (KVecCodec, TurboQuantAdapter,
    FibQuantAdapter with encode_batch_compact / decode_batch_compact);
  * ``pool``: the batched two-tier pool + shell build and rehydrate.
"""
from ._lib import PkvError  # noqa: F401

__all__ = ["PkvError"]
