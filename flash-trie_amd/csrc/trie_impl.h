// trie_impl.h -- state behind marisa::Trie (host image + device context).
#pragma once

#include <cstddef>
#include <mutex>

#include "../../include/flashtrie_amd.h"
#include "image_builder.h"

namespace marisa {

class TrieImpl {
 public:
  ftamd::ImageBlob img;
  ft_ctx* ctx = nullptr;  // created by init_tbs_gpu
  size_t max_batch = 0;
  size_t max_topk = 0, max_outpos = 0, max_out_beams = 0;
  // One context has one workspace and one stream: searches on one trie run
  // one at a time (the Python module releases the GIL around them).
  std::mutex search_mu;
  ~TrieImpl() { drop_gpu(); }
  void drop_gpu() {
    if (ctx) ft_destroy(ctx);
    ctx = nullptr;
    max_batch = 0;
  }
};

}  // namespace marisa
