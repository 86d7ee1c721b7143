"""MARISA trie files (the reference's trie.bin,
lib/marisa/grimoire/trie/louds-trie.cc:696-762) to and from trie images.

No trie.bin ships with the reference and it cannot be built here, so:
* the writer is pinned byte for byte against a KA-1 file assembled below by
  hand from the reference's build rules (louds-trie.cc:477-588, tail.cc:
  185-228, bit-vector.cc:733-836, flat-vector.h:95-131, cache fill at
  louds-trie.cc:645-693);
* the rank / select samples it writes are checked against their definition
  by brute force on tries whose LOUDS spans many 512-bit blocks;
* the reader is checked against the writer on random tries, against a
  hand-made binary-tail file, and on malformed files.
That the bytes equal what the compiled reference writes for the same keys
is parity unpinned (the reference cannot be compiled here)."""

import struct

import numpy as np
import pytest

from helpers import decode_image, image_logical

HDR = b"We love Marisa.\0"
TERM = 0xFFFFFFFF
FLT_MIN_BITS = struct.unpack("<I", struct.pack("<f", np.finfo(np.float32).tiny))[0]


def u32(x):
    return struct.pack("<I", x)


def vec(b):
    return struct.pack("<Q", len(b)) + b + b"\0" * ((8 - len(b) % 8) % 8)


def words(bits):
    out = [0] * ((len(bits) + 63) // 64)
    for i, b in enumerate(bits):
        if b:
            out[i // 64] |= 1 << (i % 64)
    return b"".join(struct.pack("<Q", w) for w in out)


def bitvec(bits, ranks=b"", sel0=(), sel1=()):
    return (vec(words(bits)) + u32(len(bits)) + u32(sum(bits)) + vec(ranks) +
            vec(b"".join(u32(x) for x in sel0)) + vec(b"".join(u32(x) for x in sel1)))


def rank_entry(abs_, rels):
    r = list(rels)
    lo = r[0] | (r[1] << 7) | (r[2] << 15) | (r[3] << 23)
    hi = r[4] | (r[5] << 9) | (r[6] << 18)
    return u32(abs_) + u32(lo) + u32(hi)


def ka1_file(binary_tail=False, config=None, extras_units=b"\0" * 8, extras_vs=0):
    """KA-1 keys {[1,2,3,4], [1,2,3,5], [7]} written out by hand.

    BFS: root 0 -> link node 1 (edge [1,2,3], two keys) and label node 2
    (token 7); node 1 -> label nodes 3 (4) and 4 (5).  LOUDS "10" + "110" +
    "110" + "0" + "0" + "0" + final "0"."""
    louds = [1, 0, 1, 1, 0, 1, 1, 0, 0, 0, 0, 0]
    term = [0, 0, 1, 1, 1, 0]
    link = [0, 1, 0, 0, 0]
    f = HDR
    # one 512-bit block: abs 0 and every relative count = all ones; then the
    # closing entry with the total
    f += bitvec(louds, rank_entry(0, [5] * 7) + rank_entry(5, [0] * 7), (1, 12), (0, 12))
    f += bitvec(term, rank_entry(0, [3] * 7) + rank_entry(3, [0] * 7), (), (2, 6))
    f += bitvec(link, rank_entry(0, [1] * 7) + rank_entry(1, [0] * 7))
    f += vec(struct.pack("<5H", 0, 0, 7, 4, 5))          # bases
    f += vec(extras_units) + u32(extras_vs)              # extras: all zero
    f += u32((0xFFFFFFFF >> (32 - extras_vs)) if extras_vs else 0) + struct.pack("<Q", 5)
    f += vec(b"\0" * 8) + u32(0) + u32(0) + struct.pack("<Q", 1)  # link extras [0]
    if binary_tail:
        f += vec(struct.pack("<3I", 1, 2, 3)) + bitvec([0, 0, 1])
    else:
        f += vec(struct.pack("<4I", 1, 2, 3, TERM)) + bitvec([])
    cache = [(0xFFFFFFFF, 0xFFFFFFFF, FLT_MIN_BITS)] * 256
    # slot (parent ^ parent << 5 ^ first token) & 255 keeps the child of most
    # keys; then its base | extra << 16, bit 31 for a link
    cache[1] = (0, 1, 0x80000000)
    cache[7] = (0, 2, 7)
    cache[(1 ^ 32 ^ 4) & 255] = (1, 3, 4)
    cache[(1 ^ 32 ^ 5) & 255] = (1, 4, 5)
    f += vec(b"".join(struct.pack("<3I", *e) for e in cache))
    f += u32(2)  # level-1 nodes
    f += u32(config if config is not None else (0x12001 if binary_tail else 0x11001))
    return f


KA1_KEYS = [[1, 2, 3, 4], [1, 2, 3, 5], [7]]


def test_writer_matches_hand_built_ka1(ft):
    t = ft.Trie()
    t.build(KA1_KEYS)
    assert t.marisa_bytes().tobytes() == ka1_file()


@pytest.mark.parametrize("binary_tail", [False, True])
def test_reader_decodes_hand_built_ka1(ft, binary_tail):
    t = ft.Trie()
    t.build(KA1_KEYS)
    u = ft.Trie()
    u.load_marisa_bytes(np.frombuffer(ka1_file(binary_tail), dtype=np.uint8))
    cb, edges, term = image_logical(u.image())
    assert cb.tolist() == [1, 3, 5, 5, 5, 5]
    assert edges == [[], [1, 2, 3], [7], [4], [5]]
    assert term.tolist() == [0, 0, 1, 1, 1]
    n, recs, parent, _ = decode_image(u.image())
    assert parent.tolist() == [0, 0, 0, 1, 1]
    assert (recs["meta"][:n] & 0xFFFF).tolist() == [0, 3, 1, 4, 4]   # string depths
    a = image_logical(t.image())
    assert a[0].tolist() == cb.tolist() and a[1] == edges


# ---- an independent decoder of the written file, for the index checks ----

class _Rd:
    def __init__(self, b):
        self.b, self.o = b, 16

    def u32(self):
        v = struct.unpack_from("<I", self.b, self.o)[0]
        self.o += 4
        return v

    def u64(self):
        v = struct.unpack_from("<Q", self.b, self.o)[0]
        self.o += 8
        return v

    def vec(self):
        n = self.u64()
        d = self.b[self.o:self.o + n]
        self.o += n + (8 - n % 8) % 8
        return d

    def bits(self):
        units = np.frombuffer(self.vec(), dtype="<u8")
        size, ones = self.u32(), self.u32()
        ranks = np.frombuffer(self.vec(), dtype="<u4").reshape(-1, 3)
        sel0 = np.frombuffer(self.vec(), dtype="<u4")
        sel1 = np.frombuffer(self.vec(), dtype="<u4")
        b = np.unpackbits(units.view(np.uint8), bitorder="little")[:size].astype(np.int64)
        return b, ones, ranks, sel0, sel1


def _check_index(b, ones, ranks, sel0, sel1, want0, want1):
    """Rank / select samples against their definition."""
    n = len(b)
    assert ones == int(b.sum())
    cum = np.concatenate([[0], np.cumsum(b)])
    nblk = (n + 511) // 512
    assert len(ranks) == nblk + 1
    for k in range(nblk):
        abs_, lo, hi = (int(x) for x in ranks[k])
        base = 512 * k
        assert abs_ == cum[base]
        rel = [lo & 0x7F, (lo >> 7) & 0xFF, (lo >> 15) & 0xFF, (lo >> 23) & 0x1FF,
               hi & 0x1FF, (hi >> 9) & 0x1FF, (hi >> 18) & 0x1FF]
        for j in range(1, 8):
            assert rel[j - 1] == cum[min(base + 64 * j, n)] - cum[base], (k, j)
    assert int(ranks[-1][0]) == ones
    zeros = np.flatnonzero(b == 0)
    onesp = np.flatnonzero(b == 1)
    if want0:
        assert sel0.tolist() == zeros[::512].tolist() + [n]
    else:
        assert len(sel0) == 0
    if want1:
        assert sel1.tolist() == onesp[::512].tolist() + [n]
    else:
        assert len(sel1) == 0


@pytest.mark.parametrize("n,vocab,lmin,lmax,seed", [(20000, 300, 1, 9, 1),
                                                     (3000, 70000, 2, 6, 2),
                                                     (60000, 300000, 3, 12, 4)])
def test_written_index_and_round_trip(ft, n, vocab, lmin, lmax, seed):
    toks, offs = ft.synth_keys(n, vocab, lmin, lmax, 1.1, seed)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    raw = t.marisa_bytes()
    rd = _Rd(raw.tobytes())
    louds = rd.bits()
    term = rd.bits()
    link = rd.bits()
    N = t.num_nodes()
    assert len(louds[0]) == 2 * N + 2 and len(louds[0]) > 4096
    _check_index(*louds, True, True)
    _check_index(*term, False, True)
    _check_index(*link, False, False)
    # labels >= 2^16 go through the packed extras, tail offsets >= 2^16
    # through the packed link extras (3-bit values straddle 64-bit words)
    rd.vec()
    vs = []
    for _ in range(2):
        rd.vec()
        vs.append(rd.u32())
        rd.u32(), rd.u64()
    if vocab == 300000:
        assert vs == [3, 3]
    u = ft.Trie()
    u.load_marisa_bytes(raw)
    a, b = image_logical(t.image()), image_logical(u.image())
    assert a[0].tolist() == b[0].tolist() and a[1] == b[1] and a[2].tolist() == b[2].tolist()
    assert np.array_equal(decode_image(t.image())[2], decode_image(u.image())[2])
    assert u.num_keys() == t.num_keys() and u.num_nodes() == N
    # writing the decoded trie gives the same file
    assert np.array_equal(u.marisa_bytes(), raw)


def test_random_tiny_round_trips(ft):
    rng = np.random.default_rng(11)
    for case in range(200):
        vocab = int(rng.integers(1, 6))
        keys = {tuple(rng.integers(0, vocab, int(rng.integers(0, 8))))
                for _ in range(int(rng.integers(1, 30)))}
        keys = [list(map(int, k)) for k in sorted(keys)]
        t = ft.Trie()
        t.build(keys)
        raw = t.marisa_bytes()
        u = ft.Trie()
        u.load_marisa_bytes(raw)
        a, b = image_logical(t.image()), image_logical(u.image())
        assert a[0].tolist() == b[0].tolist() and a[1] == b[1], case
        assert a[2].tolist() == b[2].tolist(), case
        assert np.array_equal(u.marisa_bytes(), raw), case


def test_shared_tail_suffixes(ft):
    # link edges [5,6,7], [6,7] and [9,6,7] share one tail string
    t = ft.Trie()
    t.build([[1, 5, 6, 7], [2, 6, 7], [3, 9, 6, 7], [1, 8], [2, 1], [3, 2]])
    rd = _Rd(t.marisa_bytes().tobytes())
    for _ in range(3):
        rd.bits()
    rd.vec()                                   # bases
    for _ in range(2):                         # extras, link extras
        rd.vec(), rd.u32(), rd.u32(), rd.u64()
    tail = np.frombuffer(rd.vec(), dtype="<u4").tolist()
    assert tail == [9, 6, 7, TERM, 5, 6, 7, TERM]
    u = ft.Trie()
    u.load_marisa_bytes(t.marisa_bytes())
    assert image_logical(u.image())[1] == image_logical(t.image())[1]


def test_empty_key_and_root_only(ft):
    for keys in ([[]], [[], [4]], [[4]]):
        t = ft.Trie()
        t.build(keys)
        u = ft.Trie()
        u.load_marisa_bytes(t.marisa_bytes())
        assert image_logical(u.image())[1] == image_logical(t.image())[1]
        assert u.num_keys() == len(keys)


@pytest.mark.parametrize("config,match", [(0x11002, "num_tries"),
                                          (0x21001, "LABEL_ORDER"),
                                          (0x11001 | 0x3000, "tail mode")])
def test_rejects_configs(ft, config, match):
    with pytest.raises(RuntimeError, match=match):
        ft.Trie().load_marisa_bytes(np.frombuffer(ka1_file(config=config), dtype=np.uint8))


def test_rejects_malformed(ft):
    good = ka1_file()
    for cut in (16, 20, 40, 100, len(good) // 2, len(good) - 4):
        with pytest.raises(RuntimeError):
            ft.Trie().load_marisa_bytes(np.frombuffer(good[:cut], dtype=np.uint8))
    bad = bytearray(good)
    bad[0] = ord("w")
    with pytest.raises(RuntimeError, match="header"):
        ft.Trie().load_marisa_bytes(np.frombuffer(bytes(bad), dtype=np.uint8))
    bad = bytearray(good)
    bad[16 + 8] ^= 2                           # a second 1 in the super root
    with pytest.raises(RuntimeError):
        ft.Trie().load_marisa_bytes(np.frombuffer(bytes(bad), dtype=np.uint8))
    # label extras of 16 bits: node 2's label becomes 7 | 0x8000 << 16
    units = struct.pack("<Q", 0x8000 << 32)
    with pytest.raises(RuntimeError, match="2\\^31"):
        ft.Trie().load_marisa_bytes(np.frombuffer(
            ka1_file(extras_units=units + b"\0" * 8, extras_vs=16), dtype=np.uint8))


def test_file_paths_and_host_search(ft, tmp_path):
    toks, offs = ft.synth_keys(20000, 4096, 2, 7, 1.1, 3)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    p = str(tmp_path / "trie.bin")
    t.save_marisa(p)
    with open(p, "rb") as f:
        assert f.read(16) == HDR
    u, m = ft.Trie(), ft.Trie()
    u.load(p)
    m.mmap(p)
    for x in (u, m):
        assert image_logical(x.image())[1] == image_logical(t.image())[1]
    # the host search gives the same results on the converted trie
    ids, lp = ft.synth_requests(t, 0, 12, 4096, 7, 32, 8, 0.3, 2.0, True, 5, model=1)
    for r in range(12):
        for early in (False, True):
            a = ft.tbs(t, [8] * 7, ids[r].tolist(), lp[r].tolist(), -10.0, -40.0, 5.0, early)
            b = ft.tbs(u, [8] * 7, ids[r].tolist(), lp[r].tolist(), -10.0, -40.0, 5.0, early)
            assert a[0] == b[0] and list(a[1]) == list(b[1])
