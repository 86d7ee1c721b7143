// The facade's memory and descriptor I/O as reference code calls it
// (include/marisa/trie.h: map(const void*, size_t), read(int),
// write(int) const; lib/marisa/trie.cc:33-43, 57-67, 78-86), compiled
// against this library's headers and linked with libmarisa_amd.so.  Two
// tries are written back to back into one pipe and read back one after the
// other; a MARISA file is read from a descriptor and mapped from memory; a
// host search on each equals the built trie's.  No GPU.
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <thread>
#include <vector>

#include "marisa.h"

static int fails = 0;
#define CHECK(c)                                           \
  do {                                                     \
    if (!(c)) {                                            \
      std::printf("FAIL line %d: %s\n", __LINE__, #c);     \
      ++fails;                                             \
    }                                                      \
  } while (0)

using marisa::Label;

static std::vector<std::vector<Label>> search(const marisa::Trie& t) {
  const std::vector<marisa::UInt32> beams = {4, 4, 4, 4};
  std::vector<std::vector<Label>> ids(4, std::vector<Label>{1, 2, 3, 4, 5, 7, 9});
  std::vector<std::vector<float>> lps(4, std::vector<float>{-0.5f, -1.0f, -0.7f, -0.9f,
                                                            -0.4f, -0.2f, -1.5f});
  std::vector<std::vector<Label>> out;
  std::vector<double> norms;
  marisa::TbsInput in{beams, ids, lps, out, norms, -10.0f, -40.0, 5.0, false};
  t.tbs(in);
  for (size_t i = 0; i < out.size(); ++i) {
    unsigned long long bits;
    std::memcpy(&bits, &norms[i], 8);
    out[i].push_back((Label)(bits >> 32));
    out[i].push_back((Label)bits);
  }
  return out;
}

int main(int argc, char** argv) {
  const char* tmp = argc > 1 ? argv[1] : "/tmp";
  marisa::Keyset ks1, ks2;
  const std::vector<std::vector<Label>> k1 = {{1, 2, 3}, {1, 2, 4, 5}, {7}, {7, 9, 9, 9, 1}, {3}};
  const std::vector<std::vector<Label>> k2 = {{5, 4}, {5, 3, 2}, {1}};
  for (const auto& k : k1) ks1.push_back(k.data(), k.size());
  for (const auto& k : k2) ks2.push_back(k.data(), k.size());
  marisa::Trie a, b;
  a.build(ks1);
  b.build(ks2);
  const auto want_a = search(a), want_b = search(b);
  CHECK(!want_a.empty());

  // two images back to back through a pipe: each read takes exactly its own
  int p[2];
  CHECK(::pipe(p) == 0);
  std::thread w([&]() {
    a.write(p[1]);
    b.write(p[1]);
    ::close(p[1]);
  });
  marisa::Trie ra, rb;
  ra.read(p[0]);
  rb.read(p[0]);
  w.join();
  char extra;
  CHECK(::read(p[0], &extra, 1) == 0);  // nothing left
  ::close(p[0]);
  CHECK(ra.num_keys() == k1.size() && rb.num_keys() == k2.size());
  CHECK(search(ra) == want_a && search(rb) == want_b);
  CHECK(ra.total_size() == a.total_size() &&
        std::memcmp(ra.image_data(), a.image_data(), a.total_size()) == 0);

  // map: the image in place, and a MARISA file
  std::vector<unsigned char> img((const unsigned char*)a.image_data(),
                                 (const unsigned char*)a.image_data() + a.total_size());
  marisa::Trie ma;
  ma.map(img.data(), img.size());
  CHECK(ma.image_data() == (const void*)img.data());  // no copy
  CHECK(search(ma) == want_a);
  const std::string mf = std::string(tmp) + "/facade_io_marisa.bin";
  a.save_marisa(mf.c_str());
  std::ifstream f(mf, std::ios::binary);
  std::vector<char> mbytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  marisa::Trie mm;
  mm.map(mbytes.data(), mbytes.size());
  CHECK(search(mm) == want_a);

  // a MARISA file then an image in one pipe
  CHECK(::pipe(p) == 0);
  std::thread w2([&]() {
    CHECK(::write(p[1], mbytes.data(), mbytes.size()) == (ssize_t)mbytes.size());
    b.write(p[1]);
    ::close(p[1]);
  });
  marisa::Trie rm, rb2;
  rm.read(p[0]);
  rb2.read(p[0]);
  w2.join();
  ::close(p[0]);
  CHECK(search(rm) == want_a && search(rb2) == want_b);

  // errors: the reference's codes
  int code = 0;
  try { marisa::Trie t; t.read(-1); } catch (const marisa::Exception& e) { code = e.error_code(); }
  CHECK(code == MARISA_CODE_ERROR);
  code = 0;
  try { a.write(-1); } catch (const marisa::Exception& e) { code = e.error_code(); }
  CHECK(code == MARISA_CODE_ERROR);
  code = 0;
  try { marisa::Trie t; t.map(nullptr, 10); } catch (const marisa::Exception& e) { code = e.error_code(); }
  CHECK(code == MARISA_NULL_ERROR);
  code = 0;
  try { marisa::Trie t; t.write(1); } catch (const marisa::Exception& e) { code = e.error_code(); }
  CHECK(code == MARISA_STATE_ERROR);
  // a stream that ends inside a trie
  CHECK(::pipe(p) == 0);
  CHECK(::write(p[1], img.data(), 100) == 100);
  ::close(p[1]);
  code = 0;
  try { marisa::Trie t; t.read(p[0]); } catch (const marisa::Exception& e) { code = e.error_code(); }
  CHECK(code == MARISA_IO_ERROR);
  ::close(p[0]);
  ::unlink(mf.c_str());
  std::printf("%d failures\n", fails);
  return fails ? 1 : 0;
}
