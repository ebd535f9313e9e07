"""Batched two-tier pool + shell build and rehydrate on one GPU.

The reference builds the cold tier (SharedKVPool::build_with_policy,
proveKV/src/pool.rs:157-392: one FB2 blob per (layer, K|V) over the shared
prefix, vectors gathered token-major / head-minor at pool.rs:246-257) and one
hot-tier shell per agent (shell::materialize_shell, shell.rs:148-376: one
TQB1 blob per (layer, K|V)), each (layer, K|V) through its own adapter call on
a rayon worker.  Decode goes back through decompress_layer (pool.rs:471-614)
and AgentShell::decompress_all_layers_with_seed (shell.rs:92-141), which
re-lay every layer as [tokens][heads][head_dim] f32.

Here every blob of a tier is one segment of ONE launch: the segment strides
read the corpus layout [tokens][layers][heads][K|V][head_dim] in place (no
gather copy), and decode writes each layer's [tokens][heads][head_dim] block
directly.  Blob bytes are identical to the reference's.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _lib as L
from .device import SEG_DTYPE


def read_fb2_n_blocks(payload: bytes):
    """read_fb2_n_blocks (proveKV/src/pool.rs:108-116): the FB2 n_blocks field
    of a batched pool payload, or None for a payload shorter than 14 bytes or
    without the "FB2" magic (no profile check)."""
    import ctypes as C
    buf = bytes(payload)
    n = C.c_uint64()
    rc = L.lib().pkv_fb2_n_blocks(buf, len(buf), C.byref(n))
    if rc == L.ERR_CORRUPT_PAYLOAD:
        return None
    L.check(rc, "pkv_fb2_n_blocks")
    return int(n.value)


@dataclass
class TierLayout:
    """Segment tables of one tier (pool or all shells)."""
    enc: np.ndarray          # segments over the corpus tensor
    dec: np.ndarray          # segments over the rehydrated output tensor
    wire_bytes: int
    out_elems: int
    blob_offsets: list       # (owner, layer, side, wire_offset, blob_len)


def _tier(owners, layers: int, heads: int, dim: int, corpus_tokens: int, hdr: int, plen: int) -> TierLayout:
    """owners: list of (name, first_token, n_tokens) ranges of the corpus."""
    tok_stride = layers * heads * 2 * dim           # elements per corpus token
    enc, dec, blobs = [], [], []
    wire = 0
    out = 0
    for name, t0, nt in owners:
        n = nt * heads
        for layer in range(layers):
            for side in (0, 1):
                blob = hdr + n * plen
                enc.append((t0 * tok_stride + layer * heads * 2 * dim + side * dim,
                            tok_stride, 2 * dim, wire, n, heads))
                dec.append((out, 0, dim, wire, n, max(n, 1)))
                blobs.append((name, layer, side, wire, blob))
                wire += blob
                out += n * dim
    del corpus_tokens
    return TierLayout(np.array(enc, dtype=SEG_DTYPE), np.array(dec, dtype=SEG_DTYPE), wire, out, blobs)


class DeviceKVCache:
    """A KV cache in HuggingFace ``DynamicCache`` layout on the GPU: per layer
    one K and one V tensor [1, H, T, D] (float32, bfloat16 or float16), all in
    one allocation [copies][layers][K|V][H][T][D].  ``copies`` independent
    caches (one per agent served on this GPU) share the allocation so that one
    decode can fan out to all of them.

    Implements proveKV's ``CacheTarget`` (proveKV/src/pool.rs:646-658):
    ``num_layers``, ``append_key``, ``append_value``, ``seq_len``; a key or
    value is one token's [H * D] vector, the [tokens][heads][head_dim] rows of
    ``decompress_all_layers_with_seed`` (pool.rs:447-469).
    """

    def __init__(self, layers: int, heads: int, tokens: int, dim: int, dtype=None, copies: int = 1,
                 device="cuda"):
        import torch
        self.layers, self.heads, self.tokens, self.dim, self.copies = layers, heads, tokens, dim, copies
        self.buf = torch.zeros((copies, layers, 2, heads, tokens, dim), dtype=dtype or torch.float32, device=device)
        self._seq_len = 0

    # ---- layout
    @property
    def copy_stride(self) -> int:
        return self.layers * 2 * self.heads * self.tokens * self.dim

    def elem_offset(self, layer: int, side: int, token: int) -> int:
        """Element offset of (layer, K|V, head 0, token) in copy 0."""
        return ((layer * 2 + side) * self.heads * self.tokens + token) * self.dim

    def keys(self, layer: int, copy: int = 0):
        return self.buf[copy, layer, 0].unsqueeze(0)

    def values(self, layer: int, copy: int = 0):
        return self.buf[copy, layer, 1].unsqueeze(0)

    def segments_for(self, tier: "TierLayout", first_tokens: list) -> np.ndarray:
        """Decode segments writing the blobs of `tier` at the given first token
        of each owner: vector i = t * H + h goes to [h][t0 + t] of its layer."""
        rows = []
        k = 0
        for t0 in first_tokens:
            for layer in range(self.layers):
                for side in (0, 1):
                    _, _, _, wire_off, _ = tier.blob_offsets[k]
                    n = int(tier.enc[k]["n_vectors"])
                    rows.append((self.elem_offset(layer, side, t0), self.dim, self.tokens * self.dim, wire_off, n,
                                 self.heads))
                    k += 1
        assert k == len(tier.blob_offsets)
        return np.array(rows, dtype=SEG_DTYPE)

    # ---- CacheTarget (proveKV/src/pool.rs:646-658)
    def num_layers(self) -> int:
        return self.layers

    def _append(self, side: int, layer: int, position: int, vec) -> None:
        import torch
        if not (0 <= layer < self.layers and 0 <= position < self.tokens):
            raise IndexError(f"layer {layer} / position {position} outside the cache")
        v = torch.as_tensor(np.asarray(vec, dtype=np.float32)).reshape(self.heads, self.dim)
        self.buf[:, layer, side, :, position, :] = v.to(self.buf.device, self.buf.dtype)
        self._seq_len = max(self._seq_len, position + 1)

    def append_key(self, layer: int, position: int, key) -> None:
        self._append(0, layer, position, key)

    def append_value(self, layer: int, position: int, value) -> None:
        self._append(1, layer, position, value)

    def seq_len(self) -> int:
        return self._seq_len

    def mark_filled(self, tokens: int) -> None:
        self._seq_len = max(self._seq_len, tokens)


class TwoTierPlan:
    """Pool over tokens [0, prefix) with fib_k4_n32 (FB2); one turbo (TQB1)
    shell per agent over its own token range.  Decode output per tier is
    [owner][layer][K|V][tokens][heads][head_dim] f32."""

    def __init__(self, ctx, layers: int, heads: int, dim: int, prefix: int, agent_tokens: list,
                 seed: int = 42, turbo_bits: int = 4, projections: int = 32, lossy: bool = False,
                 fib_training: int = 2048, fib_restarts: int = 4, fib_iterations: int = 8):
        self.ctx = ctx
        self.layers, self.heads, self.dim = layers, heads, dim
        self.prefix = prefix
        self.agent_tokens = list(agent_tokens)
        self.tokens = prefix + sum(self.agent_tokens)
        self.radii = L.RADII_LOG_U8 if lossy else L.RADII_F32
        self.fib = ctx.fib_profile(dim, 4, 32, seed, fib_training, fib_restarts, fib_iterations)
        self.turbo = ctx.turbo_profile(dim, turbo_bits, projections, seed)
        self.pool = _tier([("pool", 0, prefix)], layers, heads, dim, self.tokens, 19, self.fib.payload_len())
        owners, t = [], prefix
        for a, nt in enumerate(self.agent_tokens):
            owners.append((f"agent{a}", t, nt))
            t += nt
        self.shells = _tier(owners, layers, heads, dim, self.tokens, 38, self.turbo.payload_len(self.radii))

    @property
    def corpus_elems(self) -> int:
        return self.tokens * self.layers * self.heads * 2 * self.dim

    def alloc(self, device="cuda"):
        import torch
        return {
            "pool_wire": torch.empty(self.pool.wire_bytes, dtype=torch.uint8, device=device),
            "shell_wire": torch.empty(self.shells.wire_bytes, dtype=torch.uint8, device=device),
            "pool_out": torch.empty(self.pool.out_elems, dtype=torch.float32, device=device),
            "shell_out": torch.empty(self.shells.out_elems, dtype=torch.float32, device=device),
            "pool_status": torch.empty(2 * len(self.pool.enc), dtype=torch.int32, device=device),
            "shell_status": torch.empty(2 * len(self.shells.enc), dtype=torch.int32, device=device),
            "pool_dstatus": torch.empty(2 * len(self.pool.dec), dtype=torch.int32, device=device),
            "shell_dstatus": torch.empty(2 * len(self.shells.dec), dtype=torch.int32, device=device),
        }

    def encode(self, corpus, bufs, stream=None):
        """Pool build + all shells: two launches (fib, turbo)."""
        self.fib.encode_segments(corpus, self.pool.enc, bufs["pool_wire"], status=bufs["pool_status"],
                                 stream=stream)
        self.turbo.encode_segments(corpus, self.shells.enc, bufs["shell_wire"], radii=self.radii,
                                   status=bufs["shell_status"], stream=stream)

    def decode(self, bufs, stream=None):
        """Rehydrate the pool once and every shell: two launches."""
        self.fib.decode_segments(bufs["pool_wire"], self.pool.dec, bufs["pool_out"],
                                 status=bufs["pool_dstatus"], stream=stream)
        self.turbo.decode_segments(bufs["shell_wire"], self.shells.dec, bufs["shell_out"], radii=self.radii,
                                   status=bufs["shell_dstatus"], stream=stream)

    def rehydrate(self, bufs, cache: DeviceKVCache, stream=None):
        """Decode the pool and every shell straight into `cache` -- prefix at
        tokens [0, prefix), agent a's tokens after the prefix and the agents
        before it (the cache patch of the reference harness,
        proveKV/scripts/ppl_validate_multi_agent.py:226-272) -- in the cache's
        dtype, once per cache copy: two launches.  Status words land in
        bufs["pool_cstatus"] / bufs["shell_cstatus"]."""
        self._rehydrate_tier("pool", bufs, cache, stream)
        self._rehydrate_tier("shells", bufs, cache, stream)

    def build_and_rehydrate(self, corpus, bufs, cache: DeviceKVCache, stream=None, side=None,
                            side_workgroups: int = 512, pool_workgroups: int = 640):
        """One whole step: each tier's encode followed by its rehydrate into
        `cache`.  The tiers share nothing but the read-only corpus (disjoint
        wires, status words and cache token ranges), so with a `side` stream
        they overlap: the shell encode runs first on `stream`; then the shell
        rehydrate (HBM writes) runs on `side` on at most `side_workgroups`
        workgroups while the pool encode (VALU and matrix cores), on at most
        `pool_workgroups` (0: every slot), takes the rest of the GPU on
        `stream`; then the pool rehydrate.  `stream` waits for
        `side` at the end, so work queued after this call sees both tiers
        done.  Without `side` the four launches run in order on `stream`."""
        import torch
        main = stream if stream is not None else torch.cuda.current_stream()
        if side is None:
            self.encode(corpus, bufs, stream=main)
            self.rehydrate(bufs, cache, stream=main)
            return
        shells_encoded, join = torch.cuda.Event(), torch.cuda.Event()
        self.turbo.encode_segments(corpus, self.shells.enc, bufs["shell_wire"], radii=self.radii,
                                   status=bufs["shell_status"], stream=main)
        shells_encoded.record(main)
        side.wait_event(shells_encoded)
        self._rehydrate_tier("shells", bufs, cache, side, max_workgroups=side_workgroups)
        self.fib.encode_segments(corpus, self.pool.enc, bufs["pool_wire"], status=bufs["pool_status"], stream=main,
                                 max_workgroups=pool_workgroups)
        self._rehydrate_tier("pool", bufs, cache, main)
        join.record(side)
        main.wait_event(join)

    def _cache_tables(self, bufs, cache: DeviceKVCache):
        """Decode segment tables for `cache` (built once per cache shape: the
        table depends on nothing else) and the rehydrate status buffers."""
        import torch
        if cache.dim != self.dim:
            raise ValueError(f"cache head_dim {cache.dim} != plan head_dim {self.dim}")
        if cache.tokens < self.tokens or cache.layers != self.layers or cache.heads != self.heads:
            raise ValueError("cache too small for this plan")
        key = (cache.layers, cache.heads, cache.tokens, cache.dim)
        if getattr(self, "_cache_key", None) != key:
            firsts, t = [], self.prefix
            for nt in self.agent_tokens:
                firsts.append(t)
                t += nt
            self._cache_segs = (cache.segments_for(self.pool, [0]), cache.segments_for(self.shells, firsts))
            self._cache_key = key
        pseg, sseg = self._cache_segs
        for name, n in (("pool_cstatus", len(pseg)), ("shell_cstatus", len(sseg))):
            if name not in bufs:
                bufs[name] = torch.empty(2 * n, dtype=torch.int32, device=cache.buf.device)

    def _rehydrate_tier(self, tier: str, bufs, cache: DeviceKVCache, stream, max_workgroups: int = 0):
        self._cache_tables(bufs, cache)
        pseg, sseg = self._cache_segs
        out = cache.buf.view(-1)
        if tier == "pool":
            self.fib.decode_segments(bufs["pool_wire"], pseg, out, status=bufs["pool_cstatus"], stream=stream,
                                     fanout=cache.copies, fanout_stride=cache.copy_stride)
        else:
            self.turbo.decode_segments(bufs["shell_wire"], sseg, out, radii=self.radii,
                                       status=bufs["shell_cstatus"], stream=stream, fanout=cache.copies,
                                       fanout_stride=cache.copy_stride, max_workgroups=max_workgroups)
            cache.mark_filled(self.tokens)

    def check_rehydrate(self, bufs):
        """Raise the first failure recorded by the last rehydrate."""
        pseg, sseg = self._cache_segs
        for prof, key, segs in ((self.fib, "pool_cstatus", pseg), (self.turbo, "shell_cstatus", sseg)):
            err = prof.status_error(bufs[key].cpu().numpy().view(np.uint32), segs)
            if err is not None:
                raise err

    def check(self, bufs, decode: bool = True):
        """Raise the first failure recorded by the last encode (and decode)."""
        checks = [(self.fib, "pool_status", self.pool.enc), (self.turbo, "shell_status", self.shells.enc)]
        if decode:
            checks += [(self.fib, "pool_dstatus", self.pool.dec), (self.turbo, "shell_dstatus", self.shells.dec)]
        for prof, key, segs in checks:
            st = bufs[key].cpu().numpy().view(np.uint32)
            err = prof.status_error(st, segs)
            if err is not None:
                raise err

    # ------------------------------------------------------------ digests
    def digests(self, bufs, stream=None, side=None) -> None:
        """The build's digests, hashed in HBM where the encode left the blobs:
        bufs["pool_digests"] / bufs["shell_digests"] [owners * layers, 2, 32]
        hold every blob's payload digest (CompressedBlock::new,
        proveKV/src/codec.rs:85-95; key then value), and
        bufs["pool_layer_digests"] / bufs["shell_layer_digests"]
        [owners * layers, 32] every layer's block_digest (PoolLayer /
        ShellLayer::compute_digest, pool.rs:83-103, shell.rs:48-66).  Four
        launches per tier at most (payload passes, then the layer digests), one
        library call per tier.
        With a `side` stream the shell tier runs there, concurrently with the
        pool tier (each tier alone leaves most of the GPU idle); the calling
        stream waits for both."""
        import torch
        main = stream if stream is not None else torch.cuda.current_stream()
        if side is not None:   # two events kept for every call (creating them is most of a wait's cost)
            evs = getattr(self, "_digest_events", None)
            if evs is None:
                evs = self._digest_events = (torch.cuda.Event(), torch.cuda.Event())
            evs[0].record(main)
            side.wait_event(evs[0])
        for tier, name, st in ((self.pool, "pool", main), (self.shells, "shell", side or main)):
            n = len(tier.blob_offsets) // 2
            if f"{name}_digests" not in bufs:
                dev = bufs[f"{name}_wire"].device
                bufs[f"{name}_digests"] = torch.empty((n, 2, 32), dtype=torch.uint8, device=dev)
                bufs[f"{name}_layer_digests"] = torch.empty((n, 32), dtype=torch.uint8, device=dev)
            ranges = getattr(tier, "ranges", None)
            if ranges is None:
                ranges = tier.ranges = np.array([(off, ln) for _, _, _, off, ln in tier.blob_offsets], np.uint64)
            self.ctx.tier_digests(bufs[f"{name}_wire"], ranges, self.layers, bufs[f"{name}_digests"],
                                  bufs[f"{name}_layer_digests"], stream=st)
        if side is not None:
            evs[1].record(side)
            main.wait_event(evs[1])

    def digest_report(self, bufs) -> dict:
        """The digests of the last digests() call as the reference prints them
        (lower-case hex): per owner ("pool", "agent0", ...) a list over layers
        of {"key_payload_digest", "value_payload_digest", "block_digest"};
        pool layers also carry "num_blocks", PoolLayer::num_blocks of a
        batched layer (the key blob's FB2 n_blocks, pool.rs:60-80)."""
        rep = {}
        for tier, name in ((self.pool, "pool"), (self.shells, "shell")):
            pay = bufs[f"{name}_digests"].cpu().numpy()
            lay = bufs[f"{name}_layer_digests"].cpu().numpy()
            for i in range(len(tier.blob_offsets) // 2):
                owner, layer, _, ko, _ = tier.blob_offsets[2 * i]
                entry = {
                    "layer_index": layer,
                    "key_payload_digest": pay[i, 0].tobytes().hex(),
                    "value_payload_digest": pay[i, 1].tobytes().hex(),
                    "block_digest": lay[i].tobytes().hex(),
                }
                if name == "pool":
                    entry["num_blocks"] = read_fb2_n_blocks(bufs["pool_wire"][ko:ko + 14].cpu().numpy().tobytes())
                rep.setdefault(owner, []).append(entry)
        return rep

    # ------------------------------------------------------------ receipts
    def compressed_bytes(self) -> dict:
        """CLAIMS.json-style byte math: pool FB2 + shells TQB1(-L)."""
        return {"pool": self.pool.wire_bytes, "shells": self.shells.wire_bytes,
                "total": self.pool.wire_bytes + self.shells.wire_bytes,
                "per_agent_shell": self.shells.wire_bytes // max(1, len(self.agent_tokens))}

    def blob(self, bufs, tier: str, index: int) -> bytes:
        t = self.pool if tier == "pool" else self.shells
        _, _, _, off, ln = t.blob_offsets[index]
        w = bufs["pool_wire" if tier == "pool" else "shell_wire"]
        return w[off:off + ln].cpu().numpy().tobytes()
