// marisa/trie.h -- the drop-in trie with trie beam search.
//
// Mirrors the TBS part of the reference's marisa::Trie
// (include/marisa/trie.h:17-71, lib/marisa/trie.cc): build, load/save,
// sizes, and the beam search entry points init_tbs_gpu, get_max_batch_size,
// tbs, tbs_gpu and tbs_gpu_batched with the same signatures and defaults.
// The search runs on the MI355X through the C ABI in flashtrie_amd.h;
// tbs() is the host implementation of the same search.  The classic MARISA
// queries (lookup, predictive search, ...) are not part of this library.
#ifndef MARISA_TRIE_H_
#define MARISA_TRIE_H_

#include <memory>
#include <vector>

#include "marisa/base.h"
#include "marisa/keyset.h"
#include "marisa/tbs_input.h"

namespace marisa {

class TrieImpl;

class Trie {
 public:
  Trie();
  ~Trie();
  Trie(const Trie&) = delete;
  Trie& operator=(const Trie&) = delete;

  // Builds the trie.  Only the layout the reference's GPU path accepts is
  // built: one trie, text tails, label order (num_tries == 1 and
  // MARISA_LABEL_ORDER, lib/marisa/trie.cc:244-245); flags asking for
  // anything else throw MARISA_CODE_ERROR.  0 means that layout.
  void build(Keyset& keyset, int config_flags = 0);
  void build(const std::vector<std::vector<Label>>& keys);

  // load / mmap read either a MARISA trie file written by the reference
  // (trie.bin: num_tries = 1, label order; lib/marisa/trie.cc:21-76) or a
  // trie image in this library's format (flashtrie_amd.h), which save
  // writes.  save_marisa writes the MARISA trie file the reference builds
  // for the same keys.
  void load(const char* filename);
  void mmap(const char* filename);
  void save(const char* filename) const;
  void save_marisa(const char* filename) const;
  // The same from memory and descriptors (lib/marisa/trie.cc:33-43,
  // 57-67, 78-86): map uses a trie image at ptr in place (the caller keeps
  // it alive; a MARISA file there is converted); read takes one trie from
  // the descriptor's current position, reading exactly its bytes; write
  // writes what save does.  A null ptr with size > 0 throws
  // MARISA_NULL_ERROR, fd == -1 MARISA_CODE_ERROR.
  void map(const void* ptr, std::size_t size);
  void read(int fd);
  void write(int fd) const;

  void init_tbs_gpu(size_t max_batch_size, size_t max_num_topk = 1024,
                    size_t max_num_outpos = 64, size_t max_num_out_beams = 8192,
                    size_t max_num_out_tokens = 8192 * 64,
                    size_t max_num_inter_beams = 1024 * 1024,
                    size_t radix_topk_threshold = 1024);
  size_t get_max_batch_size() const;
  void tbs(TbsInput& input) const;
  void tbs_gpu(TbsInput& input, size_t batch_id = 0) const;
  void tbs_gpu_batched(std::vector<TbsInput>& inputs) const;

  std::size_t num_tries() const;
  std::size_t num_keys() const;
  std::size_t num_nodes() const;
  TailMode tail_mode() const;
  NodeOrder node_order() const;
  bool empty() const;
  std::size_t size() const;
  std::size_t total_size() const;
  std::size_t io_size() const;
  void clear();
  void swap(Trie& rhs);

  // Access for tooling: the host image blob (flashtrie_amd.h layout).
  const void* image_data() const;
  std::size_t image_size() const;
  // Adopts an image blob built elsewhere (e.g. a synthetic generator).
  void assign_image(const void* data, std::size_t size);
  TrieImpl* impl() const { return impl_.get(); }

 private:
  std::unique_ptr<TrieImpl> impl_;
};

}  // namespace marisa

#endif  // MARISA_TRIE_H_
