// marisa/tbs_input.h -- one trie beam search request / response.
// Field-for-field the reference's include/marisa/tbs_input.h:7-26, so
// callers construct it the same way; get_msec keeps the reference's
// truncation to 0.01 ms (:28-34).
#ifndef MARISA_TBS_INPUT_H_
#define MARISA_TBS_INPUT_H_

#include <chrono>
#include <vector>

#include "marisa/base.h"

namespace marisa {

struct TbsInput {
  const std::vector<UInt32>& beams;                 // beam width per step
  const std::vector<std::vector<Label>>& topk_id;   // [T][K] proposals
  const std::vector<std::vector<float>>& topk_logp; // [T][K] log-probs
  std::vector<std::vector<Label>>& out_sent;        // results, ascending score
  std::vector<double>& out_logp_norm;
  float token_logp_threshold;
  double sent_logp_threshold;
  double length_norm;
  bool early_exit;

  // Per-request device time split (ms), filled by tbs_gpu*: expansion
  // (child lookup + validation), validation (0: fused into expansion),
  // selection (bounded top-k), overhead (init + output), kernel total.
  double t_expansion_ms = 0.0;
  double t_validation_ms = 0.0;
  double t_selection_ms = 0.0;
  double t_grid_overhead_ms = 0.0;
  double kernel_ms = 0.0;
};

inline double get_msec(
    std::chrono::time_point<std::chrono::high_resolution_clock> start,
    std::chrono::time_point<std::chrono::high_resolution_clock> end) {
  const std::chrono::duration<double> elapsed = end - start;
  const double msec = 1000.0 * elapsed.count();
  return int(100 * msec) / 100.;
}

}  // namespace marisa

#endif  // MARISA_TBS_INPUT_H_
