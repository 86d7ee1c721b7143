// marisa/topk_io.h -- the reference's proposal-file loader.
//
// load_topk_keys_and_scores reads DATASET_DIR/topk_keys.txt and
// DATASET_DIR/topk_scores.txt (tools/beam-search-helper.h:26-120): a first
// line "num_requests max_output_len topk" in both files, then one line of
// `topk` numbers per (request, depth).  Token ids are parsed as floats and
// converted, like the reference.  Rows after depth 0 are re-sorted by token
// id.  Returns (topk_ids[request][depth][k], topk_logps[request][depth][k]).
// Missing files, differing headers and short rows throw marisa::Exception
// (the reference asserts or exits).
#ifndef MARISA_TOPK_IO_H_
#define MARISA_TOPK_IO_H_

#include <string>
#include <tuple>
#include <vector>

#include "marisa/base.h"

namespace marisa {

std::tuple<std::vector<std::vector<std::vector<Label>>>,
           std::vector<std::vector<std::vector<float>>>>
load_topk_keys_and_scores(const std::string& dataset_dir);

}  // namespace marisa

#endif  // MARISA_TOPK_IO_H_
