// topk_io.cc -- load_topk_keys_and_scores (see marisa/topk_io.h).
#include "marisa/topk_io.h"

#include <algorithm>
#include <fstream>
#include <numeric>
#include <sstream>

#include "marisa/base.h"

namespace marisa {

// The reference's load_topk_keys_and_scores (tools/beam-search-helper.h:26-120):
// first line of each file "num_requests max_output_len topk", then one line
// per (request, depth); rows after depth 0 are re-sorted by token id.
std::tuple<std::vector<std::vector<std::vector<Label>>>,
           std::vector<std::vector<std::vector<float>>>>
load_topk_keys_and_scores(const std::string& dir) {
  const std::string kp = dir + "/topk_keys.txt", sp = dir + "/topk_scores.txt";
  std::ifstream kf(kp), sf(sp);
  if (!kf.is_open()) throw Exception(MARISA_IO_ERROR, "cannot open " + kp);
  if (!sf.is_open()) throw Exception(MARISA_IO_ERROR, "cannot open " + sp);
  std::string kl, sl, buf;
  std::getline(kf, kl);
  std::getline(sf, sl);
  std::stringstream kss(kl), sss(sl);
  uint32_t meta[3];
  for (int i = 0; i < 3; ++i) {
    if (!(kss >> buf)) throw Exception(MARISA_FORMAT_ERROR, "bad header in " + kp);
    meta[i] = (uint32_t)std::stoi(buf);
    if (!(sss >> buf) || (uint32_t)std::stoi(buf) != meta[i])
      throw Exception(MARISA_FORMAT_ERROR, "headers of the two files differ");
  }
  const uint32_t nreq = meta[0], depth = meta[1], topk = meta[2];
  std::vector<std::vector<std::vector<Label>>> keys(nreq);
  std::vector<std::vector<std::vector<float>>> scores(nreq);
  for (uint32_t r = 0; r < nreq; ++r) {
    keys[r].resize(depth);
    scores[r].resize(depth);
    for (uint32_t d = 0; d < depth; ++d) {
      auto& lk = keys[r][d];
      auto& ls = scores[r][d];
      std::getline(kf, kl);
      std::stringstream ks(kl);
      while (ks >> buf) lk.push_back(static_cast<Label>(std::stof(buf)));
      std::getline(sf, sl);
      std::stringstream ss(sl);
      while (ss >> buf) ls.push_back(std::stof(buf));
      if (lk.size() != topk || ls.size() != topk)
        throw Exception(MARISA_FORMAT_ERROR, "row length differs from topk");
      if (d > 0) {
        std::vector<size_t> p(lk.size());
        std::iota(p.begin(), p.end(), 0);
        std::sort(p.begin(), p.end(), [&](size_t a, size_t b) { return lk[a] < lk[b]; });
        std::vector<Label> k2(lk.size());
        std::vector<float> s2(ls.size());
        for (size_t i = 0; i < p.size(); ++i) {
          k2[i] = lk[p[i]];
          s2[i] = ls[p[i]];
        }
        lk.swap(k2);
        ls.swap(s2);
      }
    }
  }
  return std::make_tuple(keys, scores);
}

}  // namespace marisa
