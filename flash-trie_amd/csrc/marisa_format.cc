// marisa_format.cc -- MARISA trie files (trie.bin) to and from the device
// trie image.
//
// Layout of a file (num_tries = 1), every field little-endian:
//   header        16 bytes "We love Marisa." (trie/header.h:13-39)
//   LOUDS bits    BitVector   (louds-trie.cc:746-762 write order)
//   terminal      BitVector
//   link flags    BitVector
//   bases         Vector<u16>  low 16 bits of a label or tail offset
//   extras        FlatVector   label >> 16, per node
//   link extras   FlatVector   tail offset >> 16, per link node
//   tail          Vector<u32> + BitVector end flags (tail.cc:230-243)
//   cache         Vector<Cache> (12 bytes each)
//   u32 number of level-1 nodes, u32 config flags
// Vector<T> = u64 byte count, elements, zero padding to 8 bytes
// (vector/vector.h:228-253); BitVector = units (Vector<u64>), u32 bits,
// u32 ones, rank samples (Vector of 12-byte RankIndex), select-0 and
// select-1 samples (Vector<u32>) (vector/bit-vector.h:183-226); FlatVector
// = units (Vector<u64>), u32 value bits, u32 mask, u64 count
// (vector/flat-vector.h:133-180).
//
// LOUDS: "10" for a super root, then per node in BFS order one 1 per child
// and a 0, then a final 0 (louds-trie.cc:485-574): node n's children are ids
// [z_n - n, z_{n+1} - n - 1) with z_n the position of the n-th 0.
#include "marisa_format.h"

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <cstring>
#include <mutex>
#include <thread>

#if defined(_OPENMP)
#include <parallel/algorithm>
#endif

namespace ftamd {

namespace {

const char kHeader[16] = "We love Marisa.";  // 15 characters and a NUL
constexpr uint32_t kTerminal = 0xFFFFFFFFu;  // ends a text-tail string
constexpr uint32_t kNumTriesMask = 0x0007F;
constexpr uint32_t kTailMask = 0x0F000;
constexpr uint32_t kOrderMask = 0xF0000;
constexpr uint32_t kTextTail = 0x01000;
constexpr uint32_t kBinaryTail = 0x02000;
constexpr uint32_t kLabelOrder = 0x10000;
constexpr uint32_t kNormalCache = 0x00200;  // its value is also the divisor
constexpr uint32_t kMaxEdge = FT_META_ELEN_MASK;
constexpr uint32_t kMaxDepth = FT_META_DEPTH_MASK;

// ---------------------------------------------------------------------------
// Reading
// ---------------------------------------------------------------------------

struct Reader {
  const uint8_t* p;
  size_t n;
  size_t off;
  std::string* err;
  bool ok = true;

  bool fail(const std::string& m) {
    if (ok) *err = m;
    ok = false;
    return false;
  }
  bool u32(uint32_t* v, const char* what) {
    if (!ok) return false;
    if (n - off < 4) return fail(std::string("truncated in ") + what);
    std::memcpy(v, p + off, 4);
    off += 4;
    return true;
  }
  bool u64(uint64_t* v, const char* what) {
    if (!ok) return false;
    if (n - off < 8) return fail(std::string("truncated in ") + what);
    std::memcpy(v, p + off, 8);
    off += 8;
    return true;
  }
  // a serialised Vector of `elem`-byte elements
  bool vec(size_t elem, const uint8_t** data, uint64_t* count, const char* what) {
    uint64_t total = 0;
    if (!u64(&total, what)) return false;
    if (total % elem)
      return fail(std::string(what) + ": byte count is not a multiple of the element size");
    if (total > n - off) return fail(std::string("truncated in ") + what);
    *data = p + off;
    *count = total / elem;
    off += (size_t)total;
    const size_t pad = (size_t)((8 - total % 8) % 8);
    if (pad > n - off) return fail(std::string("truncated in ") + what);
    off += pad;
    return true;
  }
};

struct Bits {
  const uint64_t* units = nullptr;
  uint64_t nunits = 0;
  uint32_t size = 0, num_1s = 0;
  bool get(uint64_t i) const { return (units[i >> 6] >> (i & 63)) & 1u; }
  // ones in [0, i)
  uint64_t ones_before(uint64_t i) const {
    uint64_t c = 0;
    for (uint64_t u = 0; u < (i >> 6); ++u) c += (uint64_t)__builtin_popcountll(units[u]);
    if (i & 63) c += (uint64_t)__builtin_popcountll(units[i >> 6] & ((1ull << (i & 63)) - 1));
    return c;
  }
};

bool read_bits(Reader& r, Bits* b, const char* what) {
  const uint8_t* d = nullptr;
  uint64_t cnt = 0;
  if (!r.vec(8, &d, &cnt, what)) return false;
  b->units = (const uint64_t*)d;
  b->nunits = cnt;
  if (!r.u32(&b->size, what) || !r.u32(&b->num_1s, what)) return false;
  if ((uint64_t)b->size > 64 * cnt)
    return r.fail(std::string(what) + ": fewer units than bits");
  if (b->num_1s > b->size) return r.fail(std::string(what) + ": more ones than bits");
  // rank and select samples: the decoder walks the bits itself
  const uint8_t* x = nullptr;
  uint64_t c2 = 0;
  if (!r.vec(12, &x, &c2, what) || !r.vec(4, &x, &c2, what) || !r.vec(4, &x, &c2, what))
    return false;
  if (b->ones_before(b->size) != b->num_1s)
    return r.fail(std::string(what) + ": stored count of ones does not match the bits");
  return true;
}

struct Packed {
  const uint64_t* units = nullptr;
  uint64_t nunits = 0;
  uint32_t value_size = 0, mask = 0;
  uint64_t size = 0;
  uint32_t get(uint64_t i) const {
    if (value_size == 0) return 0;
    const uint64_t pos = i * value_size;
    const uint64_t u = pos >> 6;
    const uint32_t o = (uint32_t)(pos & 63);
    if (o + value_size <= 64) return (uint32_t)(units[u] >> o) & mask;
    return (uint32_t)((units[u] >> o) | (units[u + 1] << (64 - o))) & mask;
  }
};

bool read_packed(Reader& r, Packed* f, const char* what) {
  const uint8_t* d = nullptr;
  uint64_t cnt = 0;
  if (!r.vec(8, &d, &cnt, what)) return false;
  f->units = (const uint64_t*)d;
  f->nunits = cnt;
  if (!r.u32(&f->value_size, what) || !r.u32(&f->mask, what) || !r.u64(&f->size, what))
    return false;
  if (f->value_size > 32) return r.fail(std::string(what) + ": value size above 32 bits");
  const uint32_t m = f->value_size ? (0xFFFFFFFFu >> (32 - f->value_size)) : 0u;
  if (f->mask != m) return r.fail(std::string(what) + ": mask does not match the value size");
  if (f->size > (1ull << 40) || f->value_size * f->size > 64 * cnt)
    return r.fail(std::string(what) + ": fewer units than values");
  return true;
}

}  // namespace

bool read_marisa_stream(int fd, const uint8_t head[16], std::vector<uint8_t>* out,
                        std::string* err) {
  out->assign(head, head + 16);
  auto need = [&](uint64_t n, const char* what) {
    const size_t o = out->size();
    out->resize(o + (size_t)n);
    if (!read_exact(fd, out->data() + o, (size_t)n)) {
      *err = std::string("read: the stream ends in ") + what;
      return false;
    }
    return true;
  };
  // a Vector: its byte count, then the bytes padded to 8
  auto vec = [&](const char* what) {
    if (!need(8, what)) return false;
    uint64_t total;
    std::memcpy(&total, out->data() + out->size() - 8, 8);
    if (total > (1ull << 44)) {
      *err = std::string("read: implausible size of ") + what;
      return false;
    }
    return need(total + (8 - total % 8) % 8, what);
  };
  // a BitVector: units, size and count of ones, rank and select samples
  auto bits = [&](const char* what) {
    return vec(what) && need(8, what) && vec(what) && vec(what) && vec(what);
  };
  // a FlatVector: units, value size and mask, value count
  auto packed = [&](const char* what) { return vec(what) && need(16, what); };
  // the order LoudsTrie writes them in (louds-trie.cc:747-762)
  return bits("LOUDS bits") && bits("terminal flags") && bits("link flags") &&
         vec("label bases") && packed("label extras") && packed("link extras") &&
         vec("tail") && bits("tail end flags") && vec("cache") &&
         need(8, "level-1 node count and config flags");
}

bool is_marisa_file(const void* data, size_t size) {
  return data && size >= 16 && std::memcmp(data, kHeader, 16) == 0;
}

bool image_from_marisa(const uint8_t* data, size_t size, ImageBlob* out,
                       std::string* err, int threads) {
  if (!is_marisa_file(data, size)) {
    *err = "not a MARISA trie file (header mismatch)";
    return false;
  }
  // every section starts 8-byte aligned relative to the file
  std::vector<uint64_t> aligned;
  if ((uintptr_t)data % 8) {
    aligned.resize((size + 7) / 8);
    std::memcpy(aligned.data(), data, size);
    data = (const uint8_t*)aligned.data();
  }
  Reader r{data, size, 16, err};
  Bits louds, term, link, ends;
  Packed extras, lextras;
  const uint8_t *bp = nullptr, *tp = nullptr, *cp = nullptr;
  uint64_t nbases = 0, tlen = 0, ncache = 0;
  read_bits(r, &louds, "LOUDS bits");
  read_bits(r, &term, "terminal flags");
  read_bits(r, &link, "link flags");
  r.vec(2, &bp, &nbases, "label bases");
  read_packed(r, &extras, "label extras");
  read_packed(r, &lextras, "link extras");
  r.vec(4, &tp, &tlen, "tail");
  read_bits(r, &ends, "tail end flags");
  if (!r.ok) return false;
  if (link.num_1s != 0 && tlen == 0) {
    *err = "the file holds more than one trie (num_tries > 1); the GPU search "
           "needs num_tries = 1 (marisa-build -n 1)";
    return false;
  }
  r.vec(12, &cp, &ncache, "cache");
  uint32_t num_l1 = 0, config = 0;
  r.u32(&num_l1, "level-1 node count");
  r.u32(&config, "config flags");
  if (!r.ok) return false;
  (void)ncache;
  // what the GPU search needs (lib/marisa/trie.cc:122-123)
  if ((config & kNumTriesMask) != 1) {
    *err = "num_tries = " + std::to_string(config & kNumTriesMask) +
           "; the GPU search needs num_tries = 1 (marisa-build -n 1)";
    return false;
  }
  if ((config & kOrderMask) != kLabelOrder) {
    *err = "node order is not MARISA_LABEL_ORDER (siblings must be in token "
           "order; marisa-build -l)";
    return false;
  }
  const uint32_t tmode = config & kTailMask;
  if (tmode != kTextTail && tmode != kBinaryTail) {
    *err = "unknown tail mode in the config flags";
    return false;
  }
  const bool text = tmode == kTextTail;
  if (text ? ends.size != 0 : (uint64_t)ends.size != tlen) {
    *err = "tail end flags do not match the tail mode";
    return false;
  }
  if (louds.size < 4 || (louds.size & 1u)) {
    *err = "LOUDS bits: bad length";
    return false;
  }
  const uint64_t N = louds.size / 2 - 1;
  if (N >= 0xFFFFFFFFull) {
    *err = "more than 2^32 - 2 nodes";
    return false;
  }
  if (louds.num_1s != N || term.size != N + 1 || link.size != N || nbases != N ||
      extras.size != N || lextras.size != link.num_1s) {
    *err = "section sizes disagree with the node count " + std::to_string(N);
    return false;
  }
  if (!louds.get(0) || louds.get(1) || link.get(0)) {
    *err = "LOUDS bits: bad super-root or root";
    return false;
  }
  if (tlen >= 0xFFFFFFFFull) {
    *err = "tail longer than 2^32 - 1 tokens";
    return false;
  }
  if (!out->allocate(N, tlen)) {
    *err = "out of host memory for the trie image";
    return false;
  }
  ft_node_rec* R = out->recs();
  uint32_t* P = out->parent();
  // child ranges from the positions of the 0 bits
  {
    uint64_t z = 0;
    bool bad = false;
    for (uint64_t u = 0; u < louds.nunits && !bad; ++u) {
      const uint64_t base = u * 64;
      if (base >= louds.size) break;
      uint64_t zeros = ~louds.units[u];
      if (louds.size - base < 64) zeros &= (1ull << (louds.size - base)) - 1;
      while (zeros) {
        const uint64_t pos = base + (uint64_t)__builtin_ctzll(zeros);
        zeros &= zeros - 1;
        if (z <= N) {
          const uint64_t cb = pos - z;
          if (z > 0 && cb < R[z - 1].child_begin) bad = true;
          R[z].child_begin = (uint32_t)cb;
        } else if (z == N + 1 && pos != 2 * N + 1) {
          bad = true;
        }
        ++z;
      }
    }
    if (bad || z != N + 2 || R[0].child_begin != 1 || R[N].child_begin != N) {
      *err = "LOUDS bits: inconsistent child ranges";
      return false;
    }
  }
  // labels, link edges and terminal flags, in parallel over node ranges
  const uint32_t* tail = (const uint32_t*)tp;
  const uint16_t* bases = (const uint16_t*)bp;
  int nt = threads > 0 ? threads : (int)std::max(1u, std::thread::hardware_concurrency());
  nt = (int)std::min<uint64_t>((uint64_t)std::min(nt, 64), std::max<uint64_t>(1, N / 65536));
  std::atomic<bool> failed{false};
  std::mutex emu;
  std::string first_err;
  auto worker = [&](uint64_t a, uint64_t b) {
    uint64_t lr = link.ones_before(a);  // link rank of node a
    auto bad = [&](const std::string& m) {
      std::lock_guard<std::mutex> g(emu);
      if (!failed.exchange(true)) first_err = m;
    };
    for (uint64_t v = a; v < b && !failed.load(std::memory_order_relaxed); ++v) {
      uint32_t meta = term.get(v) ? FT_META_TERMINAL : 0u;
      if (v == 0) {
        R[0].first_tok = 0;
        R[0].tail_off = 0;
        R[0].meta = meta;
        continue;
      }
      uint64_t first = 0, elen = 1;
      R[v].tail_off = 0;
      if (link.get(v)) {
        const uint64_t off = (uint64_t)bases[v] | ((uint64_t)lextras.get(lr) << 16);
        ++lr;
        if (off >= tlen) return bad("node " + std::to_string(v) + ": tail offset out of range");
        uint64_t e = off;
        if (text) {
          while (e < tlen && tail[e] != kTerminal && e - off <= kMaxEdge) ++e;
          if (e == tlen) return bad("node " + std::to_string(v) + ": unterminated tail string");
          elen = e - off;
        } else {
          while (e < tlen && !ends.get(e) && e - off <= kMaxEdge) ++e;
          if (e == tlen) return bad("node " + std::to_string(v) + ": unterminated tail string");
          elen = e - off + 1;
        }
        if (elen < 2) return bad("node " + std::to_string(v) + ": link edge shorter than 2");
        if (elen > kMaxEdge)
          return bad("node " + std::to_string(v) + ": edge longer than 16383 tokens");
        for (uint64_t i = off; i < off + elen; ++i)
          if (tail[i] >= 0x80000000u)
            return bad("node " + std::to_string(v) + ": token id >= 2^31 in its edge");
        first = tail[off];
        R[v].tail_off = (uint32_t)off;
        meta |= FT_META_LINK;
      } else {
        first = (uint64_t)bases[v] | ((uint64_t)extras.get(v) << 16);
        if (first >= 0x80000000ull)
          return bad("node " + std::to_string(v) + ": token id >= 2^31");
      }
      R[v].first_tok = (uint32_t)first;
      R[v].meta = meta | ((uint32_t)elen << FT_META_ELEN_SHIFT);
    }
  };
  {
    std::vector<std::thread> pool;
    const uint64_t step = (N + nt - 1) / nt;
    for (int i = 0; i < nt; ++i) {
      const uint64_t a = (uint64_t)i * step, b = std::min<uint64_t>(N, a + step);
      if (a < b) pool.emplace_back(worker, a, b);
    }
    for (auto& t : pool) t.join();
  }
  if (failed) {
    *err = first_err;
    return false;
  }
  // parents and string depths (a parent's id is below its children's)
  P[0] = 0;
  uint32_t max_depth = 0;
  for (uint64_t v = 0; v < N; ++v) {
    const uint32_t c0 = R[v].child_begin, c1 = R[v + 1].child_begin;
    if (c1 > c0 && c0 <= v) {
      *err = "LOUDS bits: node " + std::to_string(v) + " is not in BFS order";
      return false;
    }
    const uint32_t sd = R[v].meta & FT_META_DEPTH_MASK;
    for (uint32_t c = c0; c < c1; ++c) {
      if (c > c0 && R[c].first_tok <= R[c - 1].first_tok) {
        *err = "children of node " + std::to_string(v) +
               " are not in ascending token order (not a label-order trie)";
        return false;
      }
      P[c] = (uint32_t)v;
      const uint32_t el = (R[c].meta >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
      const uint32_t d = sd + el;
      if (d > kMaxDepth) {
        *err = "a key is longer than 65535 tokens";
        return false;
      }
      R[c].meta |= d;
      max_depth = std::max(max_depth, d);
    }
  }
  R[N] = ft_node_rec{(uint32_t)N, 0, 0, 0};
  if (num_l1 != R[1].child_begin - R[0].child_begin) {
    *err = "level-1 node count does not match the root's children";
    return false;
  }
  if (tlen) std::memcpy(out->tail(), tail, tlen * 4);
  ft_image_header& h = out->header();
  h.num_keys = term.ones_before(N);
  h.max_depth = max_depth;
  // (the decode has checked what validate_image checks: BFS child ranges,
  // token order, edge lengths and depths, tail bounds, key count)
  return true;
}

// ---------------------------------------------------------------------------
// Writing
// ---------------------------------------------------------------------------

namespace {

struct BitsOut {
  std::vector<uint64_t> units;
  uint64_t size = 0, ones = 0;
  void push(bool b) {
    if (size == 64 * units.size()) units.push_back(0);
    if (b) {
      units[size >> 6] |= 1ull << (size & 63);
      ++ones;
    }
    ++size;
  }
};

struct RankEntry {  // RankIndex (vector/rank-index.h:10-76)
  uint32_t abs = 0, lo = 0, hi = 0;
  void rel(int k, uint64_t v) {
    switch (k) {
      case 1: lo = (lo & ~0x7Fu) | ((uint32_t)v & 0x7Fu); break;
      case 2: lo = (lo & ~(0xFFu << 7)) | (((uint32_t)v & 0xFFu) << 7); break;
      case 3: lo = (lo & ~(0xFFu << 15)) | (((uint32_t)v & 0xFFu) << 15); break;
      case 4: lo = (lo & ~(0x1FFu << 23)) | (((uint32_t)v & 0x1FFu) << 23); break;
      case 5: hi = (hi & ~0x1FFu) | ((uint32_t)v & 0x1FFu); break;
      case 6: hi = (hi & ~(0x1FFu << 9)) | (((uint32_t)v & 0x1FFu) << 9); break;
      case 7: hi = (hi & ~(0x1FFu << 18)) | (((uint32_t)v & 0x1FFu) << 18); break;
      default: break;
    }
  }
};

struct BitsIndex {
  std::vector<RankEntry> ranks;
  std::vector<uint32_t> sel0, sel1;
};

// position of the i-th (from 0) set bit of `unit`, plus `base`
uint64_t select_in(uint64_t i, uint64_t base, uint64_t unit) {
  for (uint64_t k = 0; k < i; ++k) unit &= unit - 1;
  return base + (uint64_t)__builtin_ctzll(unit);
}

// The rank samples (absolute count per 512 bits, counts at each 64-bit word
// of the block) and select samples (position of every 512th 0 / 1, then the
// bit count), as BitVector::build_index makes them (bit-vector.cc:733-836).
BitsIndex make_index(const BitsOut& bv, bool sel0, bool sel1) {
  BitsIndex ix;
  const uint64_t nbits = bv.size;
  ix.ranks.resize(nbits / 512 + ((nbits % 512) ? 1 : 0) + 1);
  uint64_t n0 = 0, n1 = 0;
  for (uint64_t u = 0; u < bv.units.size(); ++u) {
    const uint64_t bit = u * 64;
    const uint64_t rid = bit / 512;
    const int sub = (int)((bit / 64) % 8);
    if (sub == 0) ix.ranks[rid].abs = (uint32_t)n1;
    else ix.ranks[rid].rel(sub, n1 - ix.ranks[rid].abs);
    const uint64_t unit = bv.units[u];
    const uint64_t u1 = (uint64_t)__builtin_popcountll(unit);
    if (sel0) {
      const uint64_t u0 = std::min<uint64_t>(nbits - bit, 64) - u1;
      const uint64_t zid = (512 - n0 % 512) % 512;
      if (u0 > zid) ix.sel0.push_back((uint32_t)select_in(zid, bit, ~unit));
      n0 += u0;
    }
    if (sel1) {
      const uint64_t oid = (512 - n1 % 512) % 512;
      if (u1 > oid) ix.sel1.push_back((uint32_t)select_in(oid, bit, unit));
    }
    n1 += u1;
  }
  if (nbits % 512) {
    const uint64_t rid = (nbits - 1) / 512;
    const int last = (int)(((nbits - 1) / 64) % 8);
    for (int k = last + 1; k <= 7; ++k) ix.ranks[rid].rel(k, n1 - ix.ranks[rid].abs);
  }
  ix.ranks.back().abs = (uint32_t)n1;
  if (sel0) ix.sel0.push_back((uint32_t)nbits);
  if (sel1) ix.sel1.push_back((uint32_t)nbits);
  return ix;
}

struct Writer {
  std::vector<uint8_t>& b;
  void raw(const void* p, size_t n) {
    const uint8_t* q = (const uint8_t*)p;
    b.insert(b.end(), q, q + n);
  }
  void u32(uint32_t v) { raw(&v, 4); }
  void u64(uint64_t v) { raw(&v, 8); }
  void vec(const void* p, uint64_t bytes) {
    u64(bytes);
    if (bytes) raw(p, (size_t)bytes);
    b.insert(b.end(), (size_t)((8 - bytes % 8) % 8), (uint8_t)0);
  }
  void bits(const BitsOut& bv, const BitsIndex* ix) {
    vec(bv.units.data(), 8 * bv.units.size());
    u32((uint32_t)bv.size);
    u32((uint32_t)bv.ones);
    if (ix) {
      std::vector<uint32_t> rk;
      rk.reserve(ix->ranks.size() * 3);
      for (const RankEntry& e : ix->ranks) {
        rk.push_back(e.abs);
        rk.push_back(e.lo);
        rk.push_back(e.hi);
      }
      vec(rk.data(), 4 * rk.size());
      vec(ix->sel0.data(), 4 * ix->sel0.size());
      vec(ix->sel1.data(), 4 * ix->sel1.size());
    } else {  // never indexed
      vec(nullptr, 0);
      vec(nullptr, 0);
      vec(nullptr, 0);
    }
  }
  // FlatVector::build_ (flat-vector.h:95-131) then its serialisation
  void packed(const std::vector<uint32_t>& values) {
    uint32_t mx = 0;
    for (uint32_t v : values) mx = std::max(mx, v);
    uint32_t vs = 0;
    while (mx) {
      ++vs;
      mx >>= 1;
    }
    uint64_t nunits = values.empty() ? 0 : 1;
    if (vs) nunits = ((uint64_t)vs * values.size() + 63) / 64;
    std::vector<uint64_t> units(nunits, 0);
    const uint32_t mask = vs ? (0xFFFFFFFFu >> (32 - vs)) : 0u;
    if (vs) {
      for (size_t i = 0; i < values.size(); ++i) {
        const uint64_t pos = (uint64_t)i * vs;
        const uint64_t u = pos >> 6;
        const uint32_t o = (uint32_t)(pos & 63);
        units[u] |= (uint64_t)values[i] << o;
        if (o + vs > 64) units[u + 1] |= (uint64_t)values[i] >> (64 - o);
      }
    }
    vec(units.data(), 8 * nunits);
    u32(vs);
    u32(mask);
    u64(values.size());
  }
};

}  // namespace

bool marisa_from_image(const ImageBlob& img, std::vector<uint8_t>* out,
                       std::string* err) {
  std::string verr;
  if (!validate_image(img, &verr)) {
    *err = "image: " + verr;
    return false;
  }
  const ft_image_header& h = img.header();
  const uint64_t N = h.num_nodes;
  const ft_node_rec* R = img.recs();
  const uint32_t* P = img.parent();
  const uint32_t* TL = img.tail();
  auto elen = [&](uint64_t v) { return (R[v].meta >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK; };
  auto is_link = [&](uint64_t v) { return (R[v].meta & FT_META_LINK) != 0; };

  BitsOut louds, term, link;
  louds.push(true);
  louds.push(false);
  for (uint64_t v = 0; v < N; ++v) {
    for (uint32_t c = R[v].child_begin; c < R[v + 1].child_begin; ++c) louds.push(true);
    louds.push(false);
  }
  louds.push(false);
  for (uint64_t v = 0; v < N; ++v) term.push((R[v].meta & FT_META_TERMINAL) != 0);
  term.push(false);
  std::vector<uint64_t> links;
  for (uint64_t v = 0; v < N; ++v) {
    link.push(is_link(v));
    if (is_link(v)) links.push_back(v);
  }

  // tail: link edges sorted by their reversed strings (shorter first on a
  // common suffix), laid out from the last, each string a suffix of the one
  // laid out before it sharing its bytes (tail.cc:185-228)
  const size_t m = links.size();
  struct Edge {
    uint64_t key;  // last token << 32 | the one before (every edge has >= 2)
    uint32_t idx, off, len;
  };
  std::vector<Edge> edges(m);
  for (size_t i = 0; i < m; ++i) {
    const uint64_t v = links[i];
    const uint32_t o = R[v].tail_off, l = elen(v);
    edges[i] = Edge{((uint64_t)TL[o + l - 1] << 32) | TL[o + l - 2], (uint32_t)i, o, l};
  }
  auto edge_less = [&](const Edge& a, const Edge& b) {
    if (a.key != b.key) return a.key < b.key;
    for (uint32_t j = 2;; ++j) {
      if (j == a.len) return j != b.len;
      if (j == b.len) return false;
      const uint32_t x = TL[a.off + a.len - 1 - j], y = TL[b.off + b.len - 1 - j];
      if (x != y) return x < y;
    }
  };
#if defined(_OPENMP)
  __gnu_parallel::sort(edges.begin(), edges.end(), edge_less);
#else
  std::sort(edges.begin(), edges.end(), edge_less);
#endif
  auto tok = [&](const Edge& e, uint32_t j) {  // j-th token from the end
    return TL[e.off + e.len - 1 - j];
  };
  std::vector<uint32_t> buf;
  {
    uint64_t total = 0;
    for (const Edge& e : edges) total += e.len + 1;
    buf.reserve(total);
  }
  std::vector<uint64_t> toff(m, 0);
  {
    const Edge* last = nullptr;
    for (size_t k = m; k > 0; --k) {
      const Edge& cur = edges[k - 1];
      const uint32_t lc = cur.len;
      uint32_t match = 0;
      if (last)
        while (match < lc && match < last->len && tok(*last, match) == tok(cur, match)) ++match;
      if (last && match == lc) {
        toff[cur.idx] = toff[last->idx] + (last->len - match);
      } else {
        toff[cur.idx] = buf.size();
        buf.insert(buf.end(), TL + cur.off, TL + cur.off + lc);
        buf.push_back(kTerminal);
        if (buf.size() > 0xFFFFFFFFull) {
          *err = "tail longer than 2^32 - 1 tokens";
          return false;
        }
      }
      last = &cur;
    }
  }
  std::vector<Edge>().swap(edges);

  std::vector<uint16_t> bases(N, 0);
  std::vector<uint32_t> extras(N, 0), lextras(m, 0);
  {
    size_t li = 0;
    for (uint64_t v = 1; v < N; ++v) {
      if (is_link(v)) {
        bases[v] = (uint16_t)(toff[li] & 0xFFFF);
        lextras[li] = (uint32_t)(toff[li] >> 16);
        ++li;
      } else {
        bases[v] = (uint16_t)(R[v].first_tok & 0xFFFF);
        extras[v] = R[v].first_tok >> 16;
      }
    }
  }

  // the lookup cache (louds-trie.cc:645-693): per (parent, first token) slot
  // the child of largest key count, then its label / link fields
  const uint64_t num_keys = h.num_keys;
  uint64_t csize = 256;
  while (csize < num_keys / kNormalCache) csize *= 2;
  const uint64_t cmask = csize - 1;
  struct CacheEnt {
    uint32_t parent, child, u;
  };
  uint32_t flt_min_bits;
  {
    const float f = FLT_MIN;
    std::memcpy(&flt_min_bits, &f, 4);
  }
  std::vector<CacheEnt> cache(csize, CacheEnt{0, 0, flt_min_bits});
  std::vector<uint64_t> cnt(N, 0);
  for (uint64_t v = 0; v < N; ++v) cnt[v] = (R[v].meta & FT_META_TERMINAL) ? 1 : 0;
  for (uint64_t v = N; v-- > 1;) cnt[P[v]] += cnt[v];
  for (uint64_t v = 0; v < N; ++v) {
    for (uint32_t c = R[v].child_begin; c < R[v + 1].child_begin; ++c) {
      const float w = (float)(double)cnt[c];
      const uint64_t id = (v ^ (v << 5) ^ (uint64_t)R[c].first_tok) & cmask;
      float cur;
      std::memcpy(&cur, &cache[id].u, 4);
      if (w > cur) {
        cache[id].parent = (uint32_t)v;
        cache[id].child = c;
        std::memcpy(&cache[id].u, &w, 4);
      }
    }
  }
  {
    // link rank of each node, for the link extras of cached link children
    std::vector<uint32_t> lrank(N, 0);
    uint32_t k = 0;
    for (uint64_t v = 0; v < N; ++v) {
      lrank[v] = k;
      if (is_link(v)) ++k;
    }
    for (CacheEnt& e : cache) {
      if (e.child != 0) {
        const uint32_t c = e.child;
        const bool lk = is_link(c);
        uint32_t u = (e.u & ~0xFFFFu) | bases[c];
        const uint32_t extra = lk ? lextras[lrank[c]] : extras[c];
        u = (u & 0xFFFFu) | (extra << 16);
        if (lk) u |= 0x80000000u;
        e.u = u;
      } else {
        e.parent = 0xFFFFFFFFu;
        e.child = 0xFFFFFFFFu;
      }
    }
  }

  out->clear();
  // one allocation for the file (an upper bound on its size)
  out->reserve(4096 + (2 * N + 2) / 8 * 2 + 3 * (N / 8 + 64) + 2 * N + 8 * N +
               4 * buf.size() + 12 * cache.size());
  Writer w{*out};
  w.raw(kHeader, 16);
  const BitsIndex lix = make_index(louds, true, true);
  const BitsIndex tix = make_index(term, false, true);
  const BitsIndex kix = make_index(link, false, false);
  w.bits(louds, &lix);
  w.bits(term, &tix);
  w.bits(link, &kix);
  w.vec(bases.data(), 2 * bases.size());
  w.packed(extras);
  w.packed(lextras);
  w.vec(buf.data(), 4 * buf.size());
  w.bits(BitsOut{}, nullptr);  // text tail: no end flags
  std::vector<uint32_t> cwords;
  cwords.reserve(3 * cache.size());
  for (const CacheEnt& e : cache) {
    cwords.push_back(e.parent);
    cwords.push_back(e.child);
    cwords.push_back(e.u);
  }
  w.vec(cwords.data(), 4 * cwords.size());
  w.u32(R[1].child_begin - R[0].child_begin);  // level-1 nodes
  w.u32(1u | kTextTail | kLabelOrder);
  return true;
}

}  // namespace ftamd
