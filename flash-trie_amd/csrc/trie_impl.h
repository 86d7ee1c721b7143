// trie_impl.h -- state behind marisa::Trie (host image + device context).
#pragma once

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <vector>

#include "../../include/flashtrie_amd.h"
#include "image_builder.h"

namespace marisa {

// Shape of one search request: steps (topk_logp rows), proposals per row
// and the final beam width.
struct TbsShape {
  size_t T = 0, K = 0;
  uint32_t F = 0;
};

class TrieImpl {
 public:
  ftamd::ImageBlob img;
  ft_ctx* ctx = nullptr;  // created by init_tbs_gpu
  size_t max_batch = 0;
  size_t max_topk = 0, max_outpos = 0, max_out_beams = 0;
  // One context has one workspace and one stream: searches on one trie run
  // one at a time (the Python module releases the GIL around them).
  std::mutex search_mu;
  // Trie::tbs_gpu_batched's request and result buffers, kept from call to
  // call (under search_mu)
  struct SearchBuffers {
    struct Rows {
      std::vector<const uint32_t*> id;
      std::vector<const float*> lp;
      std::vector<double> norms;
      std::vector<uint32_t> lens, toks;
    };
    std::vector<ft_request> reqs;
    std::vector<ft_result> res;
    std::vector<TbsShape> shapes;
    std::vector<Rows> rows;
  } sb;
  ~TrieImpl() { drop_gpu(); }
  void drop_gpu() {
    if (ctx) ft_destroy(ctx);
    ctx = nullptr;
    max_batch = 0;
  }
};

}  // namespace marisa
