// marisa_format.h -- MARISA trie files (trie.bin) to and from the device
// trie image.
//
// The file is the reference's LoudsTrie serialisation
// (lib/marisa/grimoire/trie/louds-trie.cc:696-762: header, LOUDS bits,
// terminal and link flags, label bases, packed label / link extras, tail,
// cache, level-1 node count, config flags).  Node ids in the file are the
// BFS ids the image uses, so a converted trie searches exactly like the
// reference's.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "image_builder.h"

namespace ftamd {

// True if the bytes begin with the MARISA file header
// (lib/marisa/grimoire/trie/header.h:13-39).
bool is_marisa_file(const void* data, size_t size);

// Decodes a MARISA trie file into an image with the same node ids.  Accepts
// what the GPU search requires (num_tries == 1 and MARISA_LABEL_ORDER,
// lib/marisa/trie.cc:122-123) with a text or binary tail; anything else, a
// truncated or inconsistent file, a token id >= 2^31, an edge longer than
// 16383 tokens or a key deeper than 65535 tokens returns false with *err set.
bool image_from_marisa(const uint8_t* data, size_t size, ImageBlob* out,
                       std::string* err, int threads = 0);

// Reads one MARISA trie file from a descriptor whose first 16 bytes (the
// header, already read) are `head`: exactly the file's bytes, section by
// section (every Vector carries its byte count), so a stream can hold more
// after it -- as the reference's Reader reads one trie (trie.cc:57-67).
// The bytes go to *out for image_from_marisa.  False with *err set on a
// short read or an implausible section size.
bool read_marisa_stream(int fd, const uint8_t head[16], std::vector<uint8_t>* out,
                        std::string* err);

// Encodes an image as the MARISA trie file the reference writes for its keys
// when every key has weight 1 (the Python build's keyset) and the config is
// num_tries = 1 | MARISA_TEXT_TAIL | MARISA_LABEL_ORDER | MARISA_NORMAL_CACHE
// (tools/bindings.cpp:18-20): same LOUDS bits, flags, labels, suffix-shared
// tail, rank/select samples and lookup cache.
bool marisa_from_image(const ImageBlob& img, std::vector<uint8_t>* out,
                       std::string* err);

}  // namespace ftamd
