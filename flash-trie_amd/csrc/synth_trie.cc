// synth_trie.cc -- paper-scale synthetic trie, generated level by level.
//
// Models `n_keys` keys drawn independently (duplicates dropped): a key's
// length is 3 + Geometric(p) truncated at 16 (mean ~6 for p = 0.25), and
// the token at each position is Zipf(s) over a permutation of the
// vocabulary keyed by the prefix so far.  Instead of materialising the keys
// the generator carries, per trie node, the number of keys below it and
// splits that count position by position:
//   * keys ending at the position: Binomial(n, hazard(pos)); >= 1 makes the
//     node terminal (the copies are the dropped duplicates);
//   * the rest are split over tokens: a multinomial over Zipf ranks, drawn
//     by recursive binomial splitting of the rank range for large groups
//     and by direct draws for small ones.
// A group that neither ends nor branches extends its edge, which is the
// reference's path compression (louds-trie.cc:536-550); nodes are numbered
// breadth first with children in ascending token order
// (louds-trie.cc:477-588), so the image has the reference's node ids for
// the modelled key set.  Every random draw is keyed by the prefix hash, so
// the result does not depend on the thread count.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "synth.h"

namespace ftamd {
namespace synth {

namespace {

// Zipf(s) over ranks [a, b] by rejection-inversion (Hormann & Derflinger);
// also the midpoint-rule mass of a rank range for the binomial splits.
class ZipfRange {
 public:
  explicit ZipfRange(double s) : s_(s) {
    // squeeze: for k >= 2 every x >= k - c_ lies in k's acceptance region
    c_ = 2.0 - Hinv(H(2.5) - h(2.0));
  }
  double H(double x) const {
    const double lx = std::log(x);
    const double y = (1.0 - s_) * lx;
    return (std::fabs(y) > 1e-8 ? std::expm1(y) / y : 1.0 + 0.5 * y) * lx;
  }
  double Hinv(double u) const {
    const double y = (1.0 - s_) * u;
    return std::exp((std::fabs(y) > 1e-8 ? std::log1p(y) / y : 1.0 - 0.5 * y) * u);
  }
  double h(double x) const { return std::exp(-s_ * std::log(x)); }
  double mass(uint64_t a, uint64_t b) const {  // ~ sum_{k=a}^{b} k^-s
    if (!Hk_.empty()) return Hk_[b] - Hk_[a - 1];
    return H((double)b + 0.5) - H((double)a - 0.5);
  }
  // tables H(k + 0.5) for k in [0, n] and k^-s for k in [1, n]
  void tabulate(uint64_t n) {
    Hk_.resize(n + 1);
    hk_.resize(n + 1);
    for (uint64_t k = 0; k <= n; ++k) {
      Hk_[k] = H((double)k + 0.5);
      hk_[k] = k ? h((double)k) : 0.0;
    }
  }
  // u-range of ranks [a, b]
  double lo(uint64_t a) const {
    if (!Hk_.empty()) return Hk_[a] - hk_[a];
    return H((double)a + 0.5) - h((double)a);
  }
  double hi(uint64_t b) const {
    if (!Hk_.empty()) return Hk_[b];
    return H((double)b + 0.5);
  }
  uint64_t sample(Rng& r, uint64_t a, uint64_t b) const {
    return sample(r, a, b, lo(a), hi(b));
  }
  uint64_t sample(Rng& r, uint64_t a, uint64_t b, double ulo, double uhi) const {
    for (int it = 0; it < 1000; ++it) {
      const double u = ulo + r.uniform() * (uhi - ulo);
      const double x = Hinv(u);
      double kd = std::floor(x + 0.5);
      if (kd < (double)a) kd = (double)a;
      if (kd > (double)b) kd = (double)b;
      if (kd - x <= c_) return (uint64_t)kd;
      const uint64_t k = (uint64_t)kd;
      if (u >= (Hk_.empty() ? H(kd + 0.5) - h(kd) : Hk_[k] - hk_[k])) return k;
    }
    return a;
  }

 private:
  double s_, c_;
  std::vector<double> Hk_, hk_;
};

uint64_t binomial(Rng& r, uint64_t n, double p) {
  if (n == 0 || p <= 0.0) return 0;
  if (p >= 1.0) return n;
  if (n <= 32) {
    uint64_t k = 0;
    for (uint64_t i = 0; i < n; ++i) k += r.uniform() < p;
    return k;
  }
  const bool flip = p > 0.5;
  const double q = flip ? 1.0 - p : p;
  const double mean = (double)n * q;
  uint64_t k;
  if (mean < 24.0) {  // inversion over the pmf
    double f = std::exp((double)n * std::log1p(-q));
    double cdf = f;
    const double u = r.uniform();
    k = 0;
    while (u > cdf && k < n && f > 0.0) {
      f *= (double)(n - k) / (double)(k + 1) * q / (1.0 - q);
      ++k;
      cdf += f;
    }
  } else {  // normal approximation
    const double sd = std::sqrt(mean * (1.0 - q));
    double v = std::floor(mean + sd * r.normal() + 0.5);
    if (v < 0) v = 0;
    if (v > (double)n) v = (double)n;
    k = (uint64_t)v;
  }
  return flip ? n - k : k;
}

struct Task {
  uint64_t n;       // keys below this node (with duplicates)
  uint64_t key;     // prefix hash up to and including first_tok
  uint32_t pos;     // string depth of first_tok
  uint32_t tok;     // first token of the edge
  uint32_t parent;  // parent node id
  uint32_t pad;
};

struct Split {
  uint32_t tok;
  uint64_t cnt;
};

// Affine bijections of [0, v): multipliers coprime to v, precomputed once.
struct UnitTable {
  std::vector<uint64_t> units;
  uint64_t v;
  explicit UnitTable(uint64_t vocab) : v(vocab) {
    Rng r(0x9E37ull, vocab);
    while (units.size() < 4096) {
      const uint64_t a = 1 + r.below(v - 1);
      uint64_t x = a, y = v;
      while (y) {
        const uint64_t t = x % y;
        x = y;
        y = t;
      }
      if (x == 1) units.push_back(a);
    }
  }
  uint32_t map(uint64_t key, uint64_t rank) const {
    const uint64_t h = mix64(key ^ 0xA5A5A5A5ull);
    const uint64_t a = units[h & 4095], b = (h >> 12) % v;
    return (uint32_t)((a * rank + b) % v);
  }
};

struct Gen {
  uint64_t vocab;
  ZipfRange zipf;
  double p_end;
  uint32_t lmin, lmax;
  uint64_t seed;
  UnitTable perm;
  double full_lo, full_hi;  // u-range of ranks [1, vocab]

  double hazard(uint32_t pos) const {
    if (pos < lmin) return 0.0;
    if (pos >= lmax) return 1.0;
    return p_end;
  }

  void split_ranks(Rng& r, uint64_t a, uint64_t b, uint64_t cnt,
                   std::vector<std::pair<uint64_t, uint64_t>>* out) const {
    if (cnt == 0) return;
    if (a == b) {
      out->push_back({a, cnt});
      return;
    }
    if (cnt <= 48) {
      const size_t base = out->size();
      for (uint64_t i = 0; i < cnt; ++i) out->push_back({zipf.sample(r, a, b), 1});
      std::sort(out->begin() + base, out->end());
      size_t w = base;
      for (size_t i = base; i < out->size(); ++i) {
        if (w > base && (*out)[w - 1].first == (*out)[i].first) {
          (*out)[w - 1].second += 1;
        } else {
          (*out)[w++] = (*out)[i];
        }
      }
      out->resize(w);
      return;
    }
    const uint64_t mid = a + (b - a) / 2;
    const double pl = zipf.mass(a, mid) / zipf.mass(a, b);
    const uint64_t cl = binomial(r, cnt, pl);
    split_ranks(r, a, mid, cl, out);
    split_ranks(r, mid + 1, b, cnt - cl, out);
  }

  // token groups of n keys at the position after prefix hash `key`
  void split(uint64_t key, uint64_t n, std::vector<Split>* out,
             std::vector<std::pair<uint64_t, uint64_t>>* tmp) const {
    out->clear();
    tmp->clear();
    Rng r(seed, key ^ 0x5B11ull);
    if (n == 1) {
      out->push_back({perm.map(key, zipf.sample(r, 1, vocab, full_lo, full_hi) - 1), 1});
      return;
    }
    split_ranks(r, 1, vocab, n, tmp);
    for (auto& rc : *tmp) out->push_back({perm.map(key, rc.first - 1), rc.second});
    std::sort(out->begin(), out->end(),
              [](const Split& x, const Split& y) { return x.tok < y.tok; });
  }

  static uint64_t child_key(uint64_t key, uint32_t tok, uint32_t pos) {
    return mix64(key ^ ((uint64_t)tok * 0x100000001B3ull + pos));
  }
};

// Growable array of trivially copyable T whose new elements are left
// uninitialised, so the threads that fill a slice also fault its pages in.
template <typename T>
class PodBuf {
 public:
  PodBuf() = default;
  ~PodBuf() { std::free(p_); }
  PodBuf(const PodBuf&) = delete;
  PodBuf& operator=(const PodBuf&) = delete;
  void swap(PodBuf& o) {
    std::swap(p_, o.p_);
    std::swap(n_, o.n_);
    std::swap(cap_, o.cap_);
  }
  bool grow_to(size_t n) {  // size becomes n; new elements uninitialised
    if (n > cap_) {
      size_t c = cap_ ? cap_ : 1024;
      while (c < n) c += c / 2 + 1024;
      T* q = (T*)std::realloc(p_, c * sizeof(T));
      if (!q) return false;
      p_ = q;
      cap_ = c;
    }
    n_ = n;
    return true;
  }
  bool push_back(const T& v) {
    if (!grow_to(n_ + 1)) return false;
    p_[n_ - 1] = v;
    return true;
  }
  void release() {
    std::free(p_);
    p_ = nullptr;
    n_ = cap_ = 0;
  }
  T* data() { return p_; }
  T& operator[](size_t i) { return p_[i]; }
  size_t size() const { return n_; }
  bool empty() const { return n_ == 0; }

 private:
  T* p_ = nullptr;
  size_t n_ = 0, cap_ = 0;
};

struct ChunkOut {
  std::vector<ft_node_rec> recs;
  std::vector<uint32_t> nchild;
  std::vector<uint32_t> tail;
  std::vector<Task> next;
  uint64_t terminals = 0;
  uint32_t max_depth = 0;
};

// Resolves one node: walks its edge until keys end or branch.
void process(const Gen& g, const Task& t, ChunkOut* co,
             std::vector<Split>* sp,
             std::vector<std::pair<uint64_t, uint64_t>>* tmp,
             std::vector<uint32_t>* edge, uint32_t self_id) {
  edge->clear();
  edge->push_back(t.tok);
  uint64_t n = t.n, key = t.key;
  uint32_t pos = t.pos + 1;
  bool terminal = false;
  bool have_split = false;
  if (n == 1) {
    // a single key: the rest of it is one edge (a unique suffix)
    Rng r(g.seed, key ^ 0x51C1ull);
    for (;;) {
      if (r.uniform() < g.hazard(pos)) break;
      const uint64_t rank = g.zipf.sample(r, 1, g.vocab, g.full_lo, g.full_hi);
      const uint32_t tok = g.perm.map(key, rank - 1);
      edge->push_back(tok);
      key = Gen::child_key(key, tok, pos);
      ++pos;
    }
    terminal = true;
    n = 0;
  }
  for (; n > 0;) {
    Rng r(g.seed, key ^ 0xE17Dull);
    const uint64_t e = binomial(r, n, g.hazard(pos));
    if (e) {
      terminal = true;
      n -= e;
    }
    if (terminal || n == 0) break;
    g.split(key, n, sp, tmp);
    have_split = true;
    if (sp->size() == 1) {  // one continuation: extend the edge
      const uint32_t tok = (*sp)[0].tok;
      edge->push_back(tok);
      key = Gen::child_key(key, tok, pos);
      ++pos;
      have_split = false;
      continue;
    }
    break;
  }
  if (n > 0 && !have_split) g.split(key, n, sp, tmp);
  if (n == 0) sp->clear();
  ft_node_rec rec{0, t.tok, 0, 0};
  const uint32_t elen = (uint32_t)edge->size();
  rec.meta = (pos & FT_META_DEPTH_MASK) |
             ((elen & FT_META_ELEN_MASK) << FT_META_ELEN_SHIFT);
  if (terminal) {
    rec.meta |= FT_META_TERMINAL;
    co->terminals++;
  }
  if (elen >= 2) {
    rec.meta |= FT_META_LINK;
    rec.tail_off = (uint32_t)co->tail.size();  // chunk-local, fixed later
    co->tail.insert(co->tail.end(), edge->begin(), edge->end());
  }
  co->max_depth = std::max(co->max_depth, pos);
  co->recs.push_back(rec);
  co->nchild.push_back((uint32_t)sp->size());
  for (const Split& s : *sp)
    co->next.push_back(Task{s.cnt, Gen::child_key(key, s.tok, pos), pos, s.tok,
                            self_id, 0});
}

}  // namespace

bool make_paper_trie(uint64_t n_keys, uint32_t vocab, double zipf_s,
                     uint32_t lmin, uint32_t lmax, double p_end,
                     uint64_t seed, int threads, ImageBlob* out,
                     std::string* err) {
  if (vocab < 2 || lmin < 1 || lmax < lmin || lmax > 16383) {
    *err = "bad generator parameters";
    return false;
  }
  Gen g{vocab, ZipfRange(zipf_s), p_end, lmin, lmax, seed, UnitTable(vocab), 0, 0};
  g.zipf.tabulate(vocab);
  g.full_lo = g.zipf.lo(1);
  g.full_hi = g.zipf.hi(vocab);
  if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
  PodBuf<ft_node_rec> recs;
  PodBuf<uint32_t> parent, tail;
  uint64_t terminals = 0;
  uint32_t max_depth = 0;
  // root: keys are split at position 0
  PodBuf<Task> level;
  const auto t_root = std::chrono::steady_clock::now();
  {
    std::vector<Split> sp;
    std::vector<std::pair<uint64_t, uint64_t>> tmp;
    const uint64_t root_key = mix64(seed ^ 0xC0FFEEull);
    ft_node_rec root{1, 0, 0, 0};
    Rng r(seed, root_key ^ 0xE17Dull);
    uint64_t n = n_keys;
    const uint64_t e = binomial(r, n, g.hazard(0));
    if (e) {
      root.meta |= FT_META_TERMINAL;
      ++terminals;
      n -= e;
    }
    g.split(root_key, n, &sp, &tmp);
    if (!recs.push_back(root) || !parent.push_back(0)) {
      *err = "out of host memory";
      return false;
    }
    for (const Split& s : sp)
      if (!level.push_back(Task{s.cnt, Gen::child_key(root_key, s.tok, 0), 0, s.tok, 0, 0})) {
        *err = "out of host memory";
        return false;
      }
  }
  uint64_t level_base = 1;
  std::vector<ChunkOut> outs;
  const bool verbose = std::getenv("FT_SYNTH_VERBOSE") != nullptr;
  auto clock0 = std::chrono::steady_clock::now();
  auto secs = [&]() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - clock0).count();
  };
  if (verbose)
    std::fprintf(stderr, "[synth] root split: %zu children, %.1fs\n", level.size(), secs());
  int depth = 1;
  while (!level.empty()) {
    const size_t L = level.size();
    const size_t nchunk = std::min<size_t>(L, (size_t)threads * 16);
    outs.assign(nchunk, ChunkOut());
    std::atomic<size_t> next_chunk{0};
    auto worker = [&]() {
      std::vector<Split> sp;
      std::vector<std::pair<uint64_t, uint64_t>> tmp;
      std::vector<uint32_t> edge;
      for (;;) {
        const size_t c = next_chunk.fetch_add(1);
        if (c >= nchunk) break;
        const size_t b = L * c / nchunk, e = L * (c + 1) / nchunk;
        ChunkOut& co = outs[c];
        co.recs.reserve(e - b);
        co.nchild.reserve(e - b);
        for (size_t i = b; i < e; ++i)
          process(g, level[i], &co, &sp, &tmp, &edge, (uint32_t)(level_base + i));
      }
    };
    std::vector<std::thread> pool;
    for (int w = 0; w < threads; ++w) pool.emplace_back(worker);
    for (auto& th : pool) th.join();
    // stitch: child ranges, tail offsets, parents of the next level
    const uint64_t next_base = level_base + L;
    uint64_t child_cursor = next_base;
    size_t next_total = 0;
    for (auto& co : outs) next_total += co.next.size();
    if (next_base + next_total >= 0xFFFFFFFEull) {
      *err = "more than 2^32 - 2 trie nodes";
      return false;
    }
    // per-chunk offsets, then a parallel copy into the global arrays
    std::vector<uint64_t> rec_off(nchunk + 1, 0), tail_off(nchunk + 1, 0),
        next_off(nchunk + 1, 0), child_off(nchunk + 1, 0);
    for (size_t c = 0; c < nchunk; ++c) {
      uint64_t kids = 0;
      for (uint32_t k : outs[c].nchild) kids += k;
      rec_off[c + 1] = rec_off[c] + outs[c].recs.size();
      tail_off[c + 1] = tail_off[c] + outs[c].tail.size();
      next_off[c + 1] = next_off[c] + outs[c].next.size();
      child_off[c + 1] = child_off[c] + kids;
      terminals += outs[c].terminals;
      max_depth = std::max(max_depth, outs[c].max_depth);
    }
    const uint64_t rbase = recs.size(), tbase = tail.size();
    if (tbase + tail_off[nchunk] >= 0xFFFFFFF0ull) {
      *err = "tail longer than 2^32 tokens";
      return false;
    }
    PodBuf<Task> next_level;
    if (!recs.grow_to(rbase + rec_off[nchunk]) || !tail.grow_to(tbase + tail_off[nchunk]) ||
        !next_level.grow_to(next_total) || !parent.grow_to(rbase + rec_off[nchunk])) {
      *err = "out of host memory";
      return false;
    }
    std::atomic<size_t> cc{0};
    auto stitch = [&]() {
      for (;;) {
        const size_t c = cc.fetch_add(1);
        if (c >= nchunk) break;
        ChunkOut& co = outs[c];
        uint64_t cursor = child_cursor + child_off[c];
        const uint32_t toff = (uint32_t)(tbase + tail_off[c]);
        for (size_t i = 0; i < co.recs.size(); ++i) {
          ft_node_rec rc = co.recs[i];
          rc.child_begin = (uint32_t)cursor;
          cursor += co.nchild[i];
          if (rc.meta & FT_META_LINK) rc.tail_off += toff;
          recs[rbase + rec_off[c] + i] = rc;
        }
        if (!co.tail.empty())
          std::memcpy(&tail[tbase + tail_off[c]], co.tail.data(), co.tail.size() * 4);
        if (!co.next.empty())
          std::memcpy(&next_level[next_off[c]], co.next.data(), co.next.size() * sizeof(Task));
        const size_t lb = L * c / nchunk;
        for (size_t i = 0; i < co.recs.size(); ++i) parent[rbase + rec_off[c] + i] = level[lb + i].parent;
        std::vector<ft_node_rec>().swap(co.recs);
        std::vector<uint32_t>().swap(co.tail);
        std::vector<Task>().swap(co.next);
      }
    };
    pool.clear();
    for (int w = 0; w < threads; ++w) pool.emplace_back(stitch);
    for (auto& th : pool) th.join();
    if (verbose)
      std::fprintf(stderr, "[synth] level %d: %zu nodes, %zu tail tokens total, %.1fs\n",
                   depth, level.size(), tail.size(), secs());
    ++depth;
    level.swap(next_level);
    level_base = next_base;
  }
  const uint64_t N = recs.size();
  // root's first child id
  recs[0].child_begin = 1;
  if (!out->allocate(N, tail.size())) {
    *err = "out of host memory for the trie image";
    return false;
  }
  ft_image_header& h = out->header();
  h.num_keys = terminals;
  h.max_depth = max_depth;
  auto pcopy = [&](void* dst, const void* src, size_t bytes) {
    const size_t parts = (size_t)threads;
    std::vector<std::thread> cp;
    for (size_t i = 0; i < parts; ++i) {
      const size_t b = bytes * i / parts, e = bytes * (i + 1) / parts;
      cp.emplace_back([=]() { std::memcpy((char*)dst + b, (const char*)src + b, e - b); });
    }
    for (auto& th : cp) th.join();
  };
  pcopy(out->recs(), recs.data(), N * sizeof(ft_node_rec));
  out->recs()[N] = ft_node_rec{(uint32_t)N, 0, 0, 0};
  recs.release();
  pcopy(out->parent(), parent.data(), N * 4);
  parent.release();
  if (!tail.empty()) pcopy(out->tail(), tail.data(), tail.size() * 4);
  return true;
}

bool add_prefix_keys(ImageBlob* img, uint64_t target_keys, uint32_t min_depth,
                     uint64_t seed, int threads, std::string* err) {
  ft_image_header& h = img->header();
  if (h.num_keys > target_keys) {
    *err = "the trie already holds more than the target number of keys";
    return false;
  }
  const uint64_t need = target_keys - h.num_keys;
  if (need == 0) return true;
  if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
  const uint64_t N = h.num_nodes;
  ft_node_rec* R = img->recs();
  // a candidate is a node that no key ends at but keys continue below (>= 2
  // children), whose string is at least min_depth tokens long; its rank is a
  // seeded hash of its id, and the `need` lowest ranks become keys
  auto cand = [&](uint64_t v) {
    const uint32_t m = R[v].meta;
    return v > 0 && !(m & FT_META_TERMINAL) && R[v + 1].child_begin > R[v].child_begin &&
           (m & FT_META_DEPTH_MASK) >= min_depth;
  };
  auto rank = [&](uint64_t v) { return mix64(seed ^ mix64(v + 0x70F0ull)); };
  auto parallel = [&](auto&& body) {
    std::vector<std::thread> pool;
    for (int w = 0; w < threads; ++w)
      pool.emplace_back([&, w]() { body(N * w / threads, N * (w + 1) / threads, w); });
    for (auto& th : pool) th.join();
  };
  // histogram of the top 16 bits of the ranks
  constexpr int kBins = 1 << 16;
  std::vector<std::vector<uint64_t>> hist(threads, std::vector<uint64_t>(kBins, 0));
  parallel([&](uint64_t b, uint64_t e, int w) {
    for (uint64_t v = b; v < e; ++v)
      if (cand(v)) ++hist[w][rank(v) >> 48];
  });
  uint64_t cum = 0, rem = 0;
  int cut = -1;
  for (int k = 0; k < kBins && cut < 0; ++k) {
    uint64_t c = 0;
    for (int w = 0; w < threads; ++w) c += hist[w][k];
    if (cum + c >= need) {
      cut = k;
      rem = need - cum;
    } else {
      cum += c;
    }
  }
  if (cut < 0) {
    *err = "not enough internal nodes to add the requested keys";
    return false;
  }
  // in the cut bin, the `rem` lowest ranks (ties broken by node id)
  std::vector<std::vector<std::pair<uint64_t, uint32_t>>> inbin(threads);
  parallel([&](uint64_t b, uint64_t e, int w) {
    for (uint64_t v = b; v < e; ++v)
      if (cand(v) && (int)(rank(v) >> 48) == cut) inbin[w].push_back({rank(v), (uint32_t)v});
  });
  std::vector<std::pair<uint64_t, uint32_t>> bin;
  for (auto& x : inbin) bin.insert(bin.end(), x.begin(), x.end());
  std::sort(bin.begin(), bin.end());
  for (uint64_t i = 0; i < rem; ++i) R[bin[i].second].meta |= FT_META_TERMINAL;
  parallel([&](uint64_t b, uint64_t e, int) {
    for (uint64_t v = b; v < e; ++v)
      if (cand(v) && (int)(rank(v) >> 48) < cut) R[v].meta |= FT_META_TERMINAL;
  });
  h.num_keys = target_keys;
  return true;
}

}  // namespace synth
}  // namespace ftamd
