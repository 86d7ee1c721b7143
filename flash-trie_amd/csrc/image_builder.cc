// image_builder.cc -- keys -> device trie image.
//
// The node numbering and edge strings follow the reference's trie build for
// num_tries == 1, TEXT_TAIL, LABEL_ORDER (LoudsTrie::build_current_trie,
// lib/marisa/grimoire/trie/louds-trie.cc:477-588): keys sorted
// lexicographically (labels as int, a prefix first: algorithm/sort.h:15-190),
// nodes numbered breadth first with the root 0, siblings in ascending
// first-token order, and an edge extended while every key below it agrees
// and the shortest key is longer (louds-trie.cc:536-550).  The build itself
// is level by level over the sorted keys (a group's edge only needs its
// first and last key, and group boundaries are found by galloping search),
// not the reference's queue-of-ranges walk.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "image_builder.h"

#include <algorithm>
#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <thread>

#if defined(_OPENMP)
#include <parallel/algorithm>
#include <chrono>
#include <cstdio>
#endif

namespace ftamd {

static inline uint64_t align_up(uint64_t v, uint64_t a) {
  return (v + a - 1) / a * a;
}

ImageBlob::~ImageBlob() { clear(); }

void ImageBlob::clear() {
  if (borrowed_) {
    // the caller's memory
  } else if (mapped_) {
    if (data_) ::munmap(data_, size_);
  } else {
    std::free(data_);
  }
  data_ = nullptr;
  size_ = 0;
  mapped_ = false;
  borrowed_ = false;
}

void ImageBlob::borrow(const void* p, size_t n) {
  clear();
  data_ = (uint8_t*)p;
  size_ = n;
  borrowed_ = true;
}

bool ImageBlob::allocate_bytes(size_t n) {
  clear();
  data_ = (uint8_t*)std::aligned_alloc(256, ((n ? n : 1) + 255) / 256 * 256);
  if (!data_) return false;
  size_ = n;
  return true;
}

bool read_exact(int fd, void* p, size_t n) {
  uint8_t* d = (uint8_t*)p;
  while (n) {
    const ssize_t r = ::read(fd, d, std::min<size_t>(n, 1u << 30));
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return false;
    d += r;
    n -= (size_t)r;
  }
  return true;
}

bool write_all(int fd, const void* p, size_t n) {
  const uint8_t* d = (const uint8_t*)p;
  while (n) {
    const ssize_t r = ::write(fd, d, std::min<size_t>(n, 1u << 30));
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return false;
    d += r;
    n -= (size_t)r;
  }
  return true;
}

bool ImageBlob::read_file(const char* path, std::string* err) {
  clear();
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return *err = std::string("cannot open ") + path, false;
  struct stat st;
  if (::fstat(fd, &st) != 0) {
    ::close(fd);
    return *err = std::string("cannot stat ") + path, false;
  }
  const size_t n = (size_t)st.st_size;
  data_ = (uint8_t*)std::aligned_alloc(256, ((n ? n : 1) + 255) / 256 * 256);
  if (!data_) {
    ::close(fd);
    return *err = "out of host memory", false;
  }
  size_t got = 0;
  while (got < n) {
    const ssize_t r = ::read(fd, data_ + got, std::min<size_t>(n - got, 1u << 30));
    if (r <= 0) {
      ::close(fd);
      clear();
      return *err = std::string("read failed on ") + path, false;
    }
    got += (size_t)r;
  }
  ::close(fd);
  size_ = n;
  return true;
}

bool ImageBlob::map_file(const char* path, std::string* err) {
  clear();
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return *err = std::string("cannot open ") + path, false;
  struct stat st;
  if (::fstat(fd, &st) != 0 || st.st_size == 0) {
    ::close(fd);
    return *err = std::string("cannot map ") + path + " (empty or unreadable)", false;
  }
  void* p = ::mmap(nullptr, (size_t)st.st_size, PROT_READ | PROT_WRITE, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (p == MAP_FAILED) return *err = std::string("mmap failed on ") + path, false;
  data_ = (uint8_t*)p;
  size_ = (size_t)st.st_size;
  mapped_ = true;
  return true;
}

bool ImageBlob::allocate(uint64_t num_nodes, uint64_t tail_len) {
  clear();
  ft_image_header h{};
  std::memcpy(h.magic, FT_IMAGE_MAGIC, 8);
  h.num_nodes = num_nodes;
  h.tail_len = tail_len;
  uint64_t off = 256;
  h.recs_offset = off;
  off = align_up(off + (num_nodes + 1) * sizeof(ft_node_rec), 256);
  h.parent_offset = off;
  off = align_up(off + num_nodes * 4, 256);
  h.tail_offset = off;
  off = align_up(off + tail_len * 4, 256);
  h.total_bytes = off;
  data_ = (uint8_t*)std::calloc(1, off);
  if (!data_) return false;
  size_ = off;
  std::memcpy(data_, &h, sizeof(h));
  return true;
}

bool ImageBlob::assign(const void* p, size_t n) {
  clear();
  data_ = (uint8_t*)std::malloc(n ? n : 1);
  if (!data_) return false;
  std::memcpy(data_, p, n);
  size_ = n;
  return true;
}

namespace {

struct KeySet {
  const uint32_t* toks;
  const uint64_t* offs;
  uint32_t len(uint64_t i) const { return (uint32_t)(offs[i + 1] - offs[i]); }
  const uint32_t* ptr(uint64_t i) const { return toks + offs[i]; }
};

struct Range {
  uint64_t begin, end;  // into the sorted key index
  uint32_t key_pos;
};

}  // namespace

bool build_image_from_keys(const uint32_t* toks, const uint64_t* offs,
                           uint64_t nkeys, ImageBlob* out, std::string* err,
                           int threads, bool progress) {
  (void)threads;
  const auto t_start = std::chrono::steady_clock::now();
  auto report = [&](const std::string& what) {
    if (!progress) return;
    const double s =
        std::chrono::duration<double>(std::chrono::steady_clock::now() - t_start).count();
    std::fprintf(stderr, "[build] %s at %.1f s\n", what.c_str(), s);
    std::fflush(stderr);
  };
  KeySet ks{toks, offs};
  for (uint64_t i = 0; i < nkeys; ++i) {
    const uint32_t L = ks.len(i);
    if (offs[i + 1] < offs[i] || L > 16383) {
      *err = "key " + std::to_string(i) + " is longer than 16383 tokens";
      return false;
    }
    const uint32_t* p = ks.ptr(i);
    for (uint32_t j = 0; j < L; ++j) {
      if (p[j] >= 0x80000000u) {
        *err = "key " + std::to_string(i) + " holds token id >= 2^31";
        return false;
      }
    }
  }
  report("keys validated");
  std::vector<uint64_t> idx(nkeys);
  std::iota(idx.begin(), idx.end(), 0ull);
  auto less = [&](uint64_t a, uint64_t b) {
    const uint32_t la = ks.len(a), lb = ks.len(b);
    const uint32_t* pa = ks.ptr(a);
    const uint32_t* pb = ks.ptr(b);
    const uint32_t m = std::min(la, lb);
    for (uint32_t i = 0; i < m; ++i)
      if (pa[i] != pb[i]) return pa[i] < pb[i];
    return la < lb;
  };
#if defined(_OPENMP)
  __gnu_parallel::sort(idx.begin(), idx.end(), less);
#else
  std::sort(idx.begin(), idx.end(), less);
#endif
  report("keys sorted");
  // merge duplicates
  auto same = [&](uint64_t a, uint64_t b) {
    const uint32_t la = ks.len(a);
    return la == ks.len(b) &&
           std::equal(ks.ptr(a), ks.ptr(a) + la, ks.ptr(b));
  };
  idx.erase(std::unique(idx.begin(), idx.end(), same), idx.end());
  const uint64_t n = idx.size();
  report("duplicates merged (" + std::to_string(n) + " keys)");
  auto key_len = [&](uint64_t i) { return ks.len(idx[i]); };
  auto key_at = [&](uint64_t i, uint32_t p) { return ks.ptr(idx[i])[p]; };

  std::vector<ft_node_rec> recs;
  std::vector<uint32_t> parent;
  std::vector<uint32_t> tail;
  recs.reserve(n * 2 + 2);
  parent.reserve(n * 2 + 2);
  recs.push_back(ft_node_rec{0, 0, 0, 0});
  parent.push_back(0);
  std::vector<Range> level{Range{0, n, 0}}, next_level;
  uint64_t level_base = 0;
  uint64_t num_keys = 0;
  uint32_t max_depth = 0;
  while (!level.empty()) {
    next_level.clear();
    for (size_t li = 0; li < level.size(); ++li) {
      const uint64_t id = level_base + li;
      Range r = level[li];
      if (r.begin < r.end && key_len(r.begin) == r.key_pos) {
        recs[id].meta |= FT_META_TERMINAL;  // louds-trie.cc:503-507
        ++num_keys;
        ++r.begin;
      }
      recs[id].child_begin = (uint32_t)recs.size();
      uint64_t b = r.begin;
      while (b < r.end) {
        const uint32_t tok = key_at(b, r.key_pos);
        // group end: tokens at key_pos are non-decreasing in [b, end)
        uint64_t lo = b, step = 1, hi = b + 1;
        while (hi < r.end && key_at(hi, r.key_pos) == tok) {
          lo = hi;
          step <<= 1;
          hi = std::min(r.end, lo + step);
        }
        // key_at(lo) == tok; the end lies in (lo, hi]
        uint64_t a = lo + 1, z = hi;
        while (a < z) {
          const uint64_t mid = a + (z - a) / 2;
          if (key_at(mid, r.key_pos) == tok) a = mid + 1; else z = mid;
        }
        const uint64_t g_end = a;
        // edge extension: the shortest key (first) must still be longer
        uint32_t p = r.key_pos + 1;
        const uint32_t flen = key_len(b);
        while (p < flen && key_at(b, p) == key_at(g_end - 1, p)) ++p;
        if (recs.size() >= 0xFFFFFFFEull) {
          *err = "more than 2^32 - 2 trie nodes";
          return false;
        }
        const uint32_t elen = p - r.key_pos;
        ft_node_rec c{0, tok, 0, 0};
        c.meta = (p & FT_META_DEPTH_MASK) |
                 ((elen & FT_META_ELEN_MASK) << FT_META_ELEN_SHIFT);
        if (elen >= 2) {
          c.meta |= FT_META_LINK;
          c.tail_off = (uint32_t)tail.size();
          if (tail.size() + elen >= 0xFFFFFFF0ull) {
            *err = "tail longer than 2^32 tokens";
            return false;
          }
          const uint32_t* fp = ks.ptr(idx[b]);
          tail.insert(tail.end(), fp + r.key_pos, fp + p);
        }
        max_depth = std::max(max_depth, p);
        recs.push_back(c);
        parent.push_back((uint32_t)id);
        next_level.push_back(Range{b, g_end, p});
        b = g_end;
      }
    }
    level_base += level.size();
    level.swap(next_level);
    report("level done, " + std::to_string(recs.size()) + " nodes");
  }
  const uint64_t N = recs.size();
  if (!out->allocate(N, tail.size())) {
    *err = "out of host memory for the trie image";
    return false;
  }
  ft_image_header& h = out->header();
  h.num_keys = num_keys;
  h.max_depth = max_depth;
  ft_node_rec* R = out->recs();
  std::memcpy(R, recs.data(), N * sizeof(ft_node_rec));
  R[N] = ft_node_rec{(uint32_t)N, 0, 0, 0};
  std::memcpy(out->parent(), parent.data(), N * 4);
  if (!tail.empty()) std::memcpy(out->tail(), tail.data(), tail.size() * 4);
  return true;
}

bool validate_image(const ImageBlob& img, std::string* err) {
  if (img.size() < sizeof(ft_image_header)) {
    *err = "image too small";
    return false;
  }
  const ft_image_header& h = img.header();
  if (std::memcmp(h.magic, FT_IMAGE_MAGIC, 7) != 0) {
    *err = "bad image magic";
    return false;
  }
  const uint64_t N = h.num_nodes;
  if (N == 0 || N >= 0xFFFFFFFFull || h.total_bytes != img.size() ||
      h.recs_offset % 16 ||
      h.recs_offset + (N + 1) * sizeof(ft_node_rec) > img.size() ||
      h.parent_offset + N * 4 > img.size() ||
      h.tail_offset + h.tail_len * 4 > img.size()) {
    *err = "inconsistent image header";
    return false;
  }
  const ft_node_rec* R = img.recs();
  const uint32_t* P = img.parent();
  const uint32_t* Tl = img.tail();
  if (R[0].child_begin != 1 && !(N == 1 && R[0].child_begin == 1)) {
    *err = "root children must start at id 1";
    return false;
  }
  if (R[N].child_begin != N) {
    *err = "sentinel child_begin must equal num_nodes";
    return false;
  }
  if ((R[0].meta & (FT_META_DEPTH_MASK | FT_META_LINK)) != 0) {
    *err = "root must have depth 0";
    return false;
  }
  uint64_t keys = 0;
  for (uint64_t v = 0; v < N; ++v) {
    const uint32_t c0 = R[v].child_begin, c1 = R[v + 1].child_begin;
    if (c1 < c0 || c1 > N || (c0 <= v && c1 > c0)) {
      *err = "child range of node " + std::to_string(v) + " is not BFS";
      return false;
    }
    if (R[v].meta & FT_META_TERMINAL) ++keys;
    const uint32_t sd = R[v].meta & FT_META_DEPTH_MASK;
    for (uint32_t c = c0; c < c1; ++c) {
      const uint32_t m = R[c].meta;
      const uint32_t el = (m >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
      if (P[c] != v || el == 0 || (m & FT_META_DEPTH_MASK) != sd + el ||
          ((m & FT_META_LINK) != 0) != (el >= 2) ||
          (c > c0 && R[c].first_tok <= R[c - 1].first_tok) ||
          R[c].first_tok >= 0x80000000u) {
        *err = "node " + std::to_string(c) + " is inconsistent with its parent";
        return false;
      }
      if (m & FT_META_LINK) {
        if ((uint64_t)R[c].tail_off + el > h.tail_len ||
            Tl[R[c].tail_off] != R[c].first_tok) {
          *err = "link node " + std::to_string(c) + " has a bad tail";
          return false;
        }
      }
    }
  }
  if (keys != h.num_keys) {
    *err = "num_keys does not match the terminal flags";
    return false;
  }
  return true;
}

}  // namespace ftamd
