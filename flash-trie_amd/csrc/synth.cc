// synth.cc -- seeded synthetic tries and proposal rows.
#include "synth.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>

namespace ftamd {
namespace synth {

double Rng::normal() {
  double u1 = uniform();
  if (u1 < 1e-300) u1 = 1e-300;
  const double u2 = uniform();
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

// (exp(y) - 1) / y and log(1 + y) / y, stable near 0
static double expm1_over(double y) {
  return std::fabs(y) > 1e-8 ? std::expm1(y) / y : 1.0 + y * 0.5;
}
static double log1p_over(double y) {
  return std::fabs(y) > 1e-8 ? std::log1p(y) / y : 1.0 - y * 0.5;
}

Zipf::Zipf(uint64_t n, double s) : n_(n), s_(s) {
  hx1_ = H(1.5) - 1.0;
  hn_ = H((double)n + 0.5);
  c_ = 2.0 - Hinv(H(2.5) - h(2.0));
}

// H(x) = integral of x^-s = (x^(1-s) - 1) / (1 - s)
double Zipf::H(double x) const {
  const double lx = std::log(x);
  return expm1_over((1.0 - s_) * lx) * lx;
}
double Zipf::Hinv(double u) const {
  return std::exp(log1p_over((1.0 - s_) * u) * u);
}
double Zipf::h(double x) const { return std::exp(-s_ * std::log(x)); }

uint64_t Zipf::sample(Rng& r) const {
  for (;;) {
    const double u = hn_ + r.uniform() * (hx1_ - hn_);
    const double x = Hinv(u);
    double kd = std::floor(x + 0.5);
    if (kd < 1.0) kd = 1.0;
    if (kd > (double)n_) kd = (double)n_;
    if (kd - x <= c_ || u >= H(kd + 0.5) - h(kd)) return (uint64_t)kd;
  }
}

static uint64_t gcd64(uint64_t a, uint64_t b) {
  while (b) {
    const uint64_t t = a % b;
    a = b;
    b = t;
  }
  return a;
}

KeyedPerm::KeyedPerm(uint64_t vocab, uint64_t key) : v(vocab) {
  const uint64_t x = mix64(key ^ 0xA5A5A5A5ull), y = mix64(key + 17);
  b = y % v;
  a = (x % v) | 1ull;
  if (v & (v - 1)) {  // not a power of two
    while (a == 0 || gcd64(a, v) != 1) a = (a + 1) % v;
  } else if (a >= v) {
    a = 1;
  }
}

namespace {

// open-addressing set of 64-bit hashes (0 marks an empty slot)
struct HashSet {
  std::vector<uint64_t> slots;
  uint64_t mask;
  explicit HashSet(uint64_t n) {
    uint64_t cap = 16;
    while (cap < n * 2) cap <<= 1;
    slots.assign(cap, 0);
    mask = cap - 1;
  }
  bool insert(uint64_t h) {
    if (h == 0) h = 1;
    for (uint64_t i = h & mask;; i = (i + 1) & mask) {
      if (slots[i] == h) return false;
      if (slots[i] == 0) {
        slots[i] = h;
        return true;
      }
    }
  }
};

}  // namespace

void make_keys(uint64_t n, uint32_t vocab, uint32_t lmin, uint32_t lmax,
               double s, uint64_t seed, std::vector<uint32_t>* toks,
               std::vector<uint64_t>* offs) {
  toks->clear();
  offs->assign(1, 0);
  if (lmax < lmin) std::swap(lmin, lmax);
  Zipf zipf(vocab, s);
  HashSet seen(n + 16);
  std::vector<uint32_t> key;
  const uint64_t root_key = mix64(seed ^ 0xC0FFEEull);
  for (uint64_t i = 0; offs->size() - 1 < n && i < 64 * n + 1024; ++i) {
    Rng r(seed, i);
    const uint32_t L = lmin + (uint32_t)r.below((uint64_t)(lmax - lmin) + 1);
    key.clear();
    uint64_t h = root_key;
    for (uint32_t p = 0; p < L; ++p) {
      const uint64_t rank = zipf.sample(r) - 1;
      const uint32_t tok = KeyedPerm(vocab, h)(rank);
      key.push_back(tok);
      h = mix64(h ^ ((uint64_t)tok * 0x100000001B3ull + p));
    }
    if (!seen.insert(h ^ L)) continue;
    toks->insert(toks->end(), key.begin(), key.end());
    offs->push_back(toks->size());
  }
}

// Upper-tail normal quantile: x with P(Z > x) = q, 0 < q <= 0.5
// (Abramowitz & Stegun 26.2.23, |error| < 4.5e-4).
static double normal_upper_quantile(double q) {
  if (q > 0.5) q = 0.5;
  if (q < 1e-300) q = 1e-300;
  const double t = std::sqrt(-2.0 * std::log(q));
  return t - (2.515517 + 0.802853 * t + 0.010328 * t * t) /
                 (1.0 + 1.432788 * t + 0.189269 * t * t + 0.001308 * t * t * t);
}

static double logsumexp(const std::vector<double>& v) {
  if (v.empty()) return -INFINITY;
  const double m = *std::max_element(v.begin(), v.end());
  double s = 0.0;
  for (double x : v) s += std::exp(x - m);
  return m + std::log(s);
}

// KB(n)[j] for a terminal link node (same walk as the search kernel)
static uint32_t kb_token(const ImageBlob& img, uint32_t n, uint32_t j) {
  const ft_node_rec* R = img.recs();
  for (;;) {
    const uint32_t m = R[n].meta;
    const uint32_t sd = m & FT_META_DEPTH_MASK;
    const uint32_t el = (m >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
    if (j >= sd - el) {
      if (m & FT_META_LINK) return img.tail()[R[n].tail_off + (j - (sd - el))];
      return R[n].first_tok;
    }
    n = img.parent()[n];
  }
}

void make_request(const ImageBlob& img, const ProposalSpec& sp,
                  uint64_t seed, uint64_t request, uint32_t* ids,
                  float* logp) {
  const uint32_t T = sp.steps, K = sp.topk;
  const ft_node_rec* R = img.recs();
  // Seed paths: uniformly random keys (like the reference's example
  // generator, examples/make_example_data.py:153-154), each replayed through
  // the search state machine along its node path -- the pending key token
  // at a terminal link node, else the next node of the path -- so every
  // forced token is a valid continuation at its step.
  const uint64_t N = img.header().num_nodes;
  std::vector<std::vector<uint32_t>> paths(sp.seed_paths);
  std::vector<uint32_t> chain;
  for (uint32_t sidx = 0; sidx < sp.seed_paths; ++sidx) {
    Rng r(seed ^ 0x5EEDull, request * 1000003ull + sidx);
    if (img.header().num_keys == 0 || N < 2) break;
    uint32_t target = 0;
    for (int tries = 0; tries < 4096; ++tries) {
      const uint32_t v = 1 + (uint32_t)r.below(N - 1);
      if (R[v].meta & FT_META_TERMINAL) {
        target = v;
        break;
      }
    }
    if (!target) continue;
    chain.clear();
    for (uint32_t v = target; v != 0; v = img.parent()[v]) chain.push_back(v);
    uint32_t node = 0;
    size_t next = chain.size();  // chain is target..first; walk backwards
    for (uint32_t t = 0; t < T; ++t) {
      const uint32_t m = R[node].meta;
      uint32_t tok;
      if ((m & FT_META_TERMINAL) && (m & FT_META_DEPTH_MASK) > t) {
        tok = kb_token(img, node, t);
      } else {
        if (next == 0) break;
        node = chain[--next];
        tok = R[node].first_tok;
      }
      paths[sidx].push_back(tok);
      if (node == target && (m & FT_META_DEPTH_MASK) == t + 1) break;
    }
  }
  std::vector<uint32_t> row;
  std::vector<double> zseed, zother;
  std::vector<std::pair<uint32_t, float>> cell;
  for (uint32_t t = 0; t < T; ++t) {
    Rng r(seed ^ 0x70CCull, request * 1000003ull + t);
    row.clear();
    for (auto& p : paths)
      if (t < p.size()) row.push_back(p[t]);
    std::sort(row.begin(), row.end());
    row.erase(std::unique(row.begin(), row.end()), row.end());
    if (row.size() > K) {  // keep a seeded subset
      for (size_t i = 0; i < K; ++i) std::swap(row[i], row[i + r.below(row.size() - i)]);
      row.resize(K);
      std::sort(row.begin(), row.end());
    }
    const size_t m = row.size();
    // distractors: uniformly random tokens carrying the top-tail logits of
    // `vocab` draws of N(0, sigma^2)
    std::vector<uint32_t> dis;
    while (row.size() + dis.size() < K && row.size() + dis.size() < sp.vocab) {
      const uint32_t tok = (uint32_t)r.below(sp.vocab);
      if (std::binary_search(row.begin(), row.begin() + m, tok)) continue;
      if (std::find(dis.begin(), dis.end(), tok) != dis.end()) continue;
      dis.push_back(tok);
    }
    if (sp.model == ProposalSpec::kExample) {
      cell.clear();
      for (size_t i = 0; i < m; ++i)
        cell.push_back({row[i], (float)(-0.2 - 2.0 * r.uniform())});
      for (size_t i = 0; i < dis.size(); ++i)
        cell.push_back({dis[i], (float)(-4.0 - 8.0 * r.uniform())});
      std::sort(cell.begin(), cell.end());
      for (uint32_t k = 0; k < K; ++k) {
        if (k < cell.size()) {
          ids[(uint64_t)t * K + k] = cell[k].first;
          logp[(uint64_t)t * K + k] = cell[k].second;
        } else {
          ids[(uint64_t)t * K + k] = sp.vocab + k;
          logp[(uint64_t)t * K + k] = -INFINITY;
        }
      }
      continue;
    }
    zseed.assign(m, 0.0);
    for (size_t i = 0; i < m; ++i) zseed[i] = sp.sigma * r.normal();
    zother.assign(dis.size(), 0.0);
    const double tail = (double)std::max<size_t>(dis.size(), 1) / sp.vocab;
    for (size_t i = 0; i < dis.size(); ++i)
      zother[i] = sp.sigma * normal_upper_quantile(std::max(1e-12, r.uniform() * tail));
    const double lse_seed = logsumexp(zseed);
    double lz_other;
    if (sp.analytic_rest) {
      lz_other = std::log((double)sp.vocab) + 0.5 * sp.sigma * sp.sigma;
    } else {
      lz_other = logsumexp(zother);
    }
    const double lm_seed = m ? std::log(sp.seed_mass) : 0.0;
    const double lm_other = std::log(m ? 1.0 - sp.seed_mass : 1.0);
    cell.clear();
    for (size_t i = 0; i < m; ++i)
      cell.push_back({row[i], (float)(lm_seed + zseed[i] - lse_seed)});
    for (size_t i = 0; i < dis.size(); ++i)
      cell.push_back({dis[i], (float)(lm_other + zother[i] - lz_other)});
    std::sort(cell.begin(), cell.end());
    for (uint32_t k = 0; k < K; ++k) {
      // rows shorter than K (tiny vocabularies) repeat nothing: pad with
      // ids above the vocabulary and a -inf logp, which never match
      if (k < cell.size()) {
        ids[(uint64_t)t * K + k] = cell[k].first;
        logp[(uint64_t)t * K + k] = cell[k].second;
      } else {
        ids[(uint64_t)t * K + k] = sp.vocab + k;
        logp[(uint64_t)t * K + k] = -INFINITY;
      }
    }
  }
}

}  // namespace synth
}  // namespace ftamd
