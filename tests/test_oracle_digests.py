"""What pins the oracle's BLAKE3 and the proveKV digests built on it.

* The compression function, the chunk chaining, the flags and the tree: the
  BLAKE3 project's published test vectors (tests/golden/blake3_vectors.json:
  inputs of 0 to 102,400 bytes, i.e. one block, one chunk, and trees of 2 to
  100 chunks, balanced and not), plus the known answer for "abc".
* The tree form the device kernels use (pairwise merging level by level,
  an unpaired last element carried up) against the specification's
  recursive form (left subtree = the largest power-of-two number of chunks
  that leaves at least one for the right), both here in Python, and the
  oracle's own stack-merging form, over every chunk count from 1 to 70.
* The layer digest text: the oracle's JSON against Python's own serializer
  with sorted keys and compact separators -- serde_json's output for its
  default BTreeMap object (the reference's serde_json 1.0.150 is built
  without preserve_order).
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
VECTORS = json.load(open(os.path.join(HERE, "golden", "blake3_vectors.json")))


def pattern(n: int) -> bytes:
    return bytes(i % 251 for i in range(n))


@pytest.mark.parametrize("v", VECTORS["vectors"], ids=lambda v: str(v["input_len"]))
def test_oracle_blake3_known_answers(v):
    assert O.blake3(pattern(v["input_len"])).hex() == v["hash"]


def test_oracle_blake3_ascii_known_answer():
    for v in VECTORS["ascii"]:
        assert O.blake3(v["input"].encode()).hex() == v["hash"]


# ---- an independent Python statement of the tree (chunks chained here too)
IV = (0x6A09E667, 0xBB67AE85, 0x3C6EF372, 0xA54FF53A, 0x510E527F, 0x9B05688C, 0x1F83D9AB, 0x5BE0CD19)
PERM = (2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8)
M32 = 0xFFFFFFFF


def _compress(cv, block: bytes, counter: int, blen: int, flags: int):
    m = list(int.from_bytes(block[4 * i:4 * i + 4], "little") for i in range(16))
    v = list(cv) + list(IV[:4]) + [counter & M32, counter >> 32, blen, flags]

    def g(a, b, c, d, x, y):
        v[a] = (v[a] + v[b] + x) & M32
        v[d] = ((v[d] ^ v[a]) >> 16 | (v[d] ^ v[a]) << 16) & M32
        v[c] = (v[c] + v[d]) & M32
        v[b] = ((v[b] ^ v[c]) >> 12 | (v[b] ^ v[c]) << 20) & M32
        v[a] = (v[a] + v[b] + y) & M32
        v[d] = ((v[d] ^ v[a]) >> 8 | (v[d] ^ v[a]) << 24) & M32
        v[c] = (v[c] + v[d]) & M32
        v[b] = ((v[b] ^ v[c]) >> 7 | (v[b] ^ v[c]) << 25) & M32

    for _ in range(7):
        for i, (a, b, c, d) in enumerate(((0, 4, 8, 12), (1, 5, 9, 13), (2, 6, 10, 14), (3, 7, 11, 15),
                                          (0, 5, 10, 15), (1, 6, 11, 12), (2, 7, 8, 13), (3, 4, 9, 14))):
            g(a, b, c, d, m[2 * i], m[2 * i + 1])
        m = [m[p] for p in PERM]
    return [v[i] ^ v[i + 8] for i in range(8)]


def _chunk(data: bytes, counter: int, root: bool):
    cv = list(IV)
    blocks = [data[i:i + 64] for i in range(0, len(data), 64)] or [b""]
    for j, blk in enumerate(blocks):
        flags = (1 if j == 0 else 0) | (2 | (8 if root else 0) if j == len(blocks) - 1 else 0)
        cv = _compress(cv, blk.ljust(64, b"\0"), counter, len(blk), flags)
    return cv


def _parent(l, r, root: bool):
    block = b"".join(w.to_bytes(4, "little") for w in list(l) + list(r))
    return _compress(IV, block, 0, 64, 4 | (8 if root else 0))


def _words(cv) -> bytes:
    return b"".join(w.to_bytes(4, "little") for w in cv)


def _chunks(data: bytes):
    return [data[i:i + 1024] for i in range(0, len(data), 1024)] or [b""]


def blake3_recursive(data: bytes) -> bytes:
    ch = _chunks(data)
    if len(ch) == 1:
        return _words(_chunk(ch[0], 0, True))

    def subtree(first: int, n: int, root: bool):
        if n == 1:
            return _chunk(ch[first], first, False)
        left = 1 << ((n - 1).bit_length() - 1)   # largest power of two < n
        return _parent(subtree(first, left, False), subtree(first + left, n - left, False), root)

    return _words(subtree(0, len(ch), True))


def blake3_levels(data: bytes) -> bytes:
    ch = _chunks(data)
    if len(ch) == 1:
        return _words(_chunk(ch[0], 0, True))
    cvs = [_chunk(c, i, False) for i, c in enumerate(ch)]
    while len(cvs) > 1:
        nxt = [_parent(cvs[i], cvs[i + 1], len(cvs) == 2) for i in range(0, len(cvs) - 1, 2)]
        if len(cvs) % 2:
            nxt.append(cvs[-1])
        cvs = nxt
    return _words(cvs[0])


def test_python_forms_on_known_answers():
    for v in VECTORS["vectors"]:
        if v["input_len"] <= 8192:
            data = pattern(v["input_len"])
            assert blake3_recursive(data).hex() == v["hash"]
            assert blake3_levels(data).hex() == v["hash"]


def test_tree_forms_agree_for_every_chunk_count():
    rng = np.random.default_rng(7)
    for chunks in range(1, 71):
        n = (chunks - 1) * 1024 + int(rng.integers(1, 1025))
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        want = O.blake3(data)
        assert blake3_levels(data) == want, chunks
        assert blake3_recursive(data) == want, chunks


def test_oracle_ranges_match_single_hashes():
    rng = np.random.default_rng(1)
    buf = rng.integers(0, 256, 70_001, dtype=np.uint8)
    ranges = [(0, 0), (70_001, 0), (3, 1), (5, 64), (7, 1025), (1, 70_000), (0, 70_001)]
    got = O.blake3_ranges(buf, ranges)
    for (off, ln), d in zip(ranges, got):
        assert d.tobytes() == O.blake3(buf[off:off + ln].tobytes())


def test_layer_digest_text_is_serde_json_btreemap():
    rng = np.random.default_rng(3)
    for layer in (0, 7, 23, 4_294_967_295):
        k, v = rng.integers(0, 256, 32, dtype=np.uint8).tobytes(), rng.integers(0, 256, 32, dtype=np.uint8).tobytes()
        text = json.dumps({"layer_index": layer, "key_digests": [k.hex()], "value_digests": [v.hex()]},
                          sort_keys=True, separators=(",", ":"))
        assert O.layer_digest(layer, k, v) == O.blake3(text.encode())
