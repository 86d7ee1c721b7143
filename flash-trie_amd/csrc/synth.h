// synth.h -- seeded synthetic workloads (tries and proposal rows).
//
// Every random draw comes from a counter-based generator keyed by
// (seed, stream, counter), so any request can be regenerated on its own and
// CPU and GPU paths see identical arrays.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "image_builder.h"

namespace ftamd {
namespace synth {

// SplitMix64 finaliser.
inline uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Counter-based stream: value i of stream (seed, key).
struct Rng {
  uint64_t state;
  explicit Rng(uint64_t seed, uint64_t key = 0)
      : state(mix64(seed ^ mix64(key + 0x51ED27ull))) {}
  uint64_t next() { return mix64(state += 0x9E3779B97F4A7C15ull); }
  double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
  uint64_t below(uint64_t n) { return n ? next() % n : 0; }
  double normal();  // Box-Muller
};

// Zipf(s) over ranks 1..n by rejection-inversion (W. Hormann and
// G. Derflinger, "Rejection-inversion to generate variates from monotone
// discrete distributions", ACM TOMACS 6(3), 1996).
class Zipf {
 public:
  Zipf(uint64_t n, double s);
  uint64_t sample(Rng& r) const;

 private:
  double H(double x) const;
  double Hinv(double x) const;
  double h(double x) const;
  uint64_t n_;
  double s_, hx1_, hn_, c_;
};

// A bijection of [0, v) keyed by `key` (affine map with a multiplier
// coprime to v).
struct KeyedPerm {
  uint64_t v, a, b;
  KeyedPerm(uint64_t vocab, uint64_t key);
  uint32_t operator()(uint64_t r) const { return (uint32_t)((a * r + b) % v); }
};

// `n` unique keys; length uniform in [lmin, lmax]; the token at each
// position is Zipf(s) over a permutation of the vocabulary keyed by the
// prefix so far, so popular prefixes are shared.  Keys are returned as a
// flat token array + offsets, in generation order.
void make_keys(uint64_t n, uint32_t vocab, uint32_t lmin, uint32_t lmax,
               double s, uint64_t seed, std::vector<uint32_t>* toks,
               std::vector<uint64_t>* offs);

struct ProposalSpec {
  uint32_t vocab = 32768;
  uint32_t steps = 8;       // T
  uint32_t topk = 32;       // K
  uint32_t seed_paths = 8;  // random search paths whose tokens are forced in
  double seed_mass = 0.3;   // softmax mass carried by the forced tokens
  double sigma = 2.0;       // logits ~ N(0, sigma^2)
  bool analytic_rest = false;  // include the unproposed vocabulary in logZ
  // Row model.  kSoftmax: log-softmax of N(0, sigma^2) logits with
  // seed_mass of the mass on the forced tokens.  kExample: the shape of the
  // reference's example generator (examples/make_example_data.py:119-145):
  // forced tokens uniform in [-2.2, -0.2], distractors uniform in [-12, -4].
  enum Model { kSoftmax = 0, kExample = 1 } model = kSoftmax;
};

// Proposal rows of one request, sorted by token id: ids[T*K], logp[T*K].
// Seed paths walk the search's own state machine over the image (taking the
// pending key token at a terminal link node, else a uniformly chosen child),
// so a forced token is a valid continuation of its path at that step.
void make_request(const ImageBlob& img, const ProposalSpec& spec,
                  uint64_t seed, uint64_t request, uint32_t* ids,
                  float* logp);

// Paper-scale trie generated level by level without materialising keys:
// n_keys independent keys (duplicates dropped), length lmin + Geometric(p_end)
// truncated at lmax, Zipf(zipf_s) tokens over a prefix-keyed permutation of
// the vocabulary.  Writes the image directly (reference node numbering).
bool make_paper_trie(uint64_t n_keys, uint32_t vocab, double zipf_s,
                     uint32_t lmin, uint32_t lmax, double p_end, uint64_t seed,
                     int threads, ImageBlob* out, std::string* err);

// Makes the trie hold exactly `target_keys` keys by adding keys that are
// prefixes of existing ones: the internal nodes (>= 2 children, no key
// ending there, string depth >= min_depth) with the lowest seeded hash of
// their node id become terminal.  The structure and node ids do not change.
// For topping up a generated trie to an exact unique-key count.
bool add_prefix_keys(ImageBlob* img, uint64_t target_keys, uint32_t min_depth,
                     uint64_t seed, int threads, std::string* err);

}  // namespace synth
}  // namespace ftamd
