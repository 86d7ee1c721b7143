// image_builder.h -- builds the device trie image (flashtrie_amd.h layout).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/flashtrie_amd.h"

namespace ftamd {

// An image blob: owned (256-byte aligned heap memory), a private
// read-write mapping of an image file (page aligned; writes stay private),
// or memory the caller owns and keeps alive (borrowed; never freed here).
class ImageBlob {
 public:
  ImageBlob() = default;
  ~ImageBlob();
  ImageBlob(const ImageBlob&) = delete;
  ImageBlob& operator=(const ImageBlob&) = delete;
  ImageBlob(ImageBlob&& o) noexcept { swap(o); }
  ImageBlob& operator=(ImageBlob&& o) noexcept {
    swap(o);
    return *this;
  }
  void swap(ImageBlob& o) noexcept {
    std::swap(data_, o.data_);
    std::swap(size_, o.size_);
    std::swap(mapped_, o.mapped_);
    std::swap(borrowed_, o.borrowed_);
  }
  // Allocates a zeroed blob laid out for the given sizes and fills the header.
  bool allocate(uint64_t num_nodes, uint64_t tail_len);
  // Adopts a copy of an existing blob.
  bool assign(const void* p, size_t n);
  // Reads a whole file into a new blob (one read, no intermediate copy).
  bool read_file(const char* path, std::string* err);
  // Maps a whole file (private, copy-on-write): the pages are read on first
  // use and shared with the page cache.
  bool map_file(const char* path, std::string* err);
  // Uses n bytes at p in place (the caller keeps them alive and unchanged).
  void borrow(const void* p, size_t n);
  // An owned, uninitialised blob of n bytes (256-byte aligned).
  bool allocate_bytes(size_t n);
  bool mapped() const { return mapped_; }
  void clear();

  bool empty() const { return data_ == nullptr; }
  const uint8_t* data() const { return data_; }
  uint8_t* data() { return data_; }
  size_t size() const { return size_; }
  ft_image_header& header() { return *(ft_image_header*)data_; }
  const ft_image_header& header() const { return *(const ft_image_header*)data_; }
  ft_node_rec* recs() { return (ft_node_rec*)(data_ + header().recs_offset); }
  const ft_node_rec* recs() const {
    return (const ft_node_rec*)(data_ + header().recs_offset);
  }
  uint32_t* parent() { return (uint32_t*)(data_ + header().parent_offset); }
  const uint32_t* parent() const {
    return (const uint32_t*)(data_ + header().parent_offset);
  }
  uint32_t* tail() { return (uint32_t*)(data_ + header().tail_offset); }
  const uint32_t* tail() const {
    return (const uint32_t*)(data_ + header().tail_offset);
  }

 private:
  uint8_t* data_ = nullptr;
  size_t size_ = 0;
  bool mapped_ = false;
  bool borrowed_ = false;
};

// Reads exactly n bytes from a descriptor (retrying short reads and EINTR);
// false at end of file or on an error.
bool read_exact(int fd, void* p, size_t n);
// Writes n bytes to a descriptor (retrying short writes and EINTR).
bool write_all(int fd, const void* p, size_t n);

// Builds the trie of `nkeys` keys (key i = toks[offs[i] .. offs[i+1])) with
// the reference's node numbering (MARISA BFS, label order, path compression:
// lib/marisa/grimoire/trie/louds-trie.cc:477-588).  Duplicate keys are
// merged.  Returns false and sets *err on invalid keys (a token >= 2^31, a
// key longer than 16383 tokens, or more than 2^32 - 2 nodes).  With
// `progress`, each phase's end is reported on stderr with its elapsed
// time (validation, sort, duplicate merge, every level of the walk).
bool build_image_from_keys(const uint32_t* toks, const uint64_t* offs,
                           uint64_t nkeys, ImageBlob* out, std::string* err,
                           int threads = 0, bool progress = false);

// Checks the structural invariants of an image (child ranges, depths,
// parents, tail bounds).  Used on images read from disk.
bool validate_image(const ImageBlob& img, std::string* err);

}  // namespace ftamd
