// marisa/keyset.h -- the keys a trie is built from (token sequences).
// Covers the reference Keyset's building interface
// (include/marisa/keyset.h:20-45); keys are stored flat.
#ifndef MARISA_KEYSET_H_
#define MARISA_KEYSET_H_

#include <vector>

#include "marisa/base.h"

namespace marisa {

class Keyset {
 public:
  void push_back(const std::vector<Label>& str, float weight = 1.0) {
    push_back(str.data(), str.size(), weight);
  }
  void push_back(const Label* ptr, std::size_t length, float weight = 1.0) {
    (void)weight;  // node order is label order; weights do not matter
    if (ptr == nullptr && length != 0)
      throw Exception(MARISA_NULL_ERROR, "Keyset::push_back: null key");
    toks_.insert(toks_.end(), ptr, ptr + length);
    offs_.push_back(toks_.size());
  }
  std::size_t size() const { return offs_.size() - 1; }
  std::size_t num_keys() const { return size(); }
  bool empty() const { return size() == 0; }
  std::size_t total_length() const { return toks_.size(); }
  const Label* key_ptr(std::size_t i) const { return toks_.data() + offs_[i]; }
  std::size_t key_length(std::size_t i) const { return offs_[i + 1] - offs_[i]; }
  const std::vector<Label>& tokens() const { return toks_; }
  const std::vector<UInt64>& offsets() const { return offs_; }
  void clear() {
    toks_.clear();
    offs_.assign(1, 0);
  }
  void reset() { clear(); }

 private:
  std::vector<Label> toks_;
  std::vector<UInt64> offs_ = std::vector<UInt64>(1, 0);
};

}  // namespace marisa

#endif  // MARISA_KEYSET_H_
