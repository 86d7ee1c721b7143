// marisa_trie.cc -- the drop-in marisa::Trie (TBS surface) over the C ABI.
//
// Mirrors lib/marisa/trie.cc:119-149 (init_tbs_gpu, get_max_batch_size, tbs,
// tbs_gpu, tbs_gpu_batched) and the sizes/build/IO entry points the Python
// module exposes (tools/bindings.cpp:27-43).  tbs_gpu* go through
// flashtrie_amd.h; tbs() is the host implementation of the same search.
#include "marisa/trie.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <exception>
#include <fstream>
#include <memory>
#include <queue>
#include <string>
#include <vector>

#include "../../include/flashtrie_amd.h"
#include "image_builder.h"
#include "marisa_format.h"
#include "trie_impl.h"

#ifndef FT_BUILD_ID
#define FT_BUILD_ID "unknown"
#endif
// the build id tag (see ft_build_id), kept in the binary
extern "C" __attribute__((used)) const char ft_marisa_build_id[] = "FT_BUILD_ID=" FT_BUILD_ID;

namespace marisa {

namespace {

[[noreturn]] void throw_ft(int rc, const char* where) {
  std::string msg = std::string(where) + ": " + ft_strerror(rc);
  const char* detail = ft_last_error();
  if (detail && *detail) msg += std::string(" (") + detail + ")";
  ErrorCode code = MARISA_STATE_ERROR;
  if (rc == FT_E_ARG || rc == FT_E_INPUT) code = MARISA_CODE_ERROR;
  if (rc == FT_E_LIMIT) code = MARISA_SIZE_ERROR;
  if (rc == FT_E_NOMEM) code = MARISA_MEMORY_ERROR;
  if (rc == FT_E_IMAGE) code = MARISA_FORMAT_ERROR;
  throw Exception(code, msg);
}

void require_trie(const TrieImpl* t) {
  if (!t || t->img.empty())
    throw Exception(MARISA_STATE_ERROR, "trie is not built or loaded");
}

// Shape checks shared by the host and device paths.  The step count is the
// number of topk_logp rows (louds-trie.cc:143) and K the length of row 0
// (louds-trie.cc:120-123).
using Shape = TbsShape;

Shape check_shape(const TbsInput& in) {
  Shape s;
  if (in.beams.empty())
    throw Exception(MARISA_CODE_ERROR, "tbs: beams is empty");
  s.F = in.beams.back();
  if (s.F == 0) return s;
  s.T = in.topk_logp.size();
  if (s.T == 0 || in.topk_id.empty())
    throw Exception(MARISA_CODE_ERROR, "tbs: topk rows are empty");
  s.K = in.topk_id[0].size();
  if (s.K == 0) throw Exception(MARISA_CODE_ERROR, "tbs: topk row 0 is empty");
  if (in.topk_id.size() < s.T)
    throw Exception(MARISA_CODE_ERROR, "tbs: fewer topk_id rows than topk_logp rows");
  if (in.beams.size() < s.T)
    throw Exception(MARISA_CODE_ERROR, "tbs: fewer beam widths than steps");
  for (size_t t = 0; t < s.T; ++t) {
    if (in.topk_id[t].size() != s.K || in.topk_logp[t].size() != s.K)
      throw Exception(MARISA_CODE_ERROR,
                      "tbs: ragged topk rows (row " + std::to_string(t) + ")");
    if (in.beams[t] == 0)
      throw Exception(MARISA_CODE_ERROR,
                      "tbs: beam width 0 at step " + std::to_string(t));
  }
  return s;
}

// ---------------------------------------------------------------------------
// Host search: the reference CPU state machine (louds-trie.cc:75-177) over
// the image, with bounded heaps of hypothesis indices.
// ---------------------------------------------------------------------------
struct Hyp {
  double s, norm;
  UInt32 node, depth, hist;
};

struct Worse {  // heap order: top() is the worst (AgentComparer)
  const std::vector<Hyp>* pool;
  bool operator()(UInt32 a, UInt32 b) const {
    const Hyp& x = (*pool)[a];
    const Hyp& y = (*pool)[b];
    if (x.norm == y.norm) return x.node > y.node;
    return x.norm > y.norm;
  }
};

class Bounded {
 public:
  Bounded(size_t cap, const std::vector<Hyp>* pool)
      : cap_(cap), pool_(pool), q_(Worse{pool}) {}
  void push(UInt32 h) {
    if (q_.size() < cap_ || (*pool_)[h].norm > (*pool_)[q_.top()].norm) q_.push(h);
    if (q_.size() > cap_) q_.pop();
  }
  UInt32 pop() {
    const UInt32 h = q_.top();
    q_.pop();
    return h;
  }
  bool empty() const { return q_.empty(); }
  size_t size() const { return q_.size(); }

 private:
  size_t cap_;
  const std::vector<Hyp>* pool_;
  std::priority_queue<UInt32, std::vector<UInt32>, Worse> q_;
};

void host_tbs(const ftamd::ImageBlob& img, TbsInput& in) {
  const Shape sh = check_shape(in);
  if (sh.F == 0) return;  // outputs untouched (louds-trie.cc:114-117)
  const ft_node_rec* R = img.recs();
  const UInt32* P = img.parent();
  const UInt32* TL = img.tail();
  std::vector<double> lnf(sh.T + 1);
  for (size_t d = 0; d <= sh.T; ++d)
    lnf[d] = std::pow(6.0 / (5.0 + (double)d), in.length_norm);
  std::vector<Hyp> pool;
  std::vector<std::pair<UInt32, Label>> hist;  // (parent hist, token)
  pool.push_back(Hyp{0.0, 0.0 * lnf[0], 0, 0, 0xFFFFFFFFu});
  Bounded selected(sh.F, &pool);
  Bounded cur(1, &pool);
  cur.push(0);
  auto kb = [&](UInt32 n, UInt32 j) -> Label {
    for (;;) {
      const UInt32 m = R[n].meta, sd = m & FT_META_DEPTH_MASK;
      const UInt32 el = (m >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
      if (j >= sd - el)
        return (m & FT_META_LINK) ? TL[R[n].tail_off + (j - (sd - el))] : R[n].first_tok;
      n = P[n];
    }
  };
  for (size_t t = 0; t < sh.T; ++t) {
    if (cur.empty() || (in.early_exit && selected.size() >= sh.F)) break;
    Bounded next(in.beams[t], &pool);
    const std::vector<Label>& ids = in.topk_id[t];
    const std::vector<float>& lps = in.topk_logp[t];
    while (!cur.empty()) {
      const UInt32 pi = cur.pop();
      const Hyp p = pool[pi];
      const UInt32 m = R[p.node].meta;
      const bool lp = (m & FT_META_TERMINAL) && (m & FT_META_DEPTH_MASK) > t;
      const Label need = lp ? kb(p.node, (UInt32)t) : 0;
      const UInt32 c0 = R[p.node].child_begin, c1 = R[p.node + 1].child_begin;
      for (size_t k = 0; k < sh.K; ++k) {
        if (in.early_exit && selected.size() >= sh.F) break;
        const Label tok = ids[k];
        const float x = lps[k];
        if ((double)x <= (double)in.token_logp_threshold ||
            p.s + x <= in.sent_logp_threshold)
          continue;
        if (lp && tok != need) continue;
        UInt32 child = p.node;
        if (!lp) {
          UInt32 lo = c0, hi = c1;
          while (lo < hi) {
            const UInt32 mid = lo + (hi - lo) / 2;
            if (R[mid].first_tok < tok) lo = mid + 1; else hi = mid;
          }
          if (lo == c1 || R[lo].first_tok != tok) continue;
          child = lo;
        }
        const UInt32 depth = (UInt32)t + 1;
        const double s = p.s + x;
        hist.push_back({p.hist, tok});
        pool.push_back(Hyp{s, s * lnf[depth], child, depth, (UInt32)hist.size() - 1});
        const UInt32 h = (UInt32)pool.size() - 1;
        const UInt32 cm = R[child].meta;
        if (lp) {
          if ((cm & FT_META_DEPTH_MASK) == depth) selected.push(h); else next.push(h);
        } else {
          if ((cm & FT_META_TERMINAL) && (cm & FT_META_DEPTH_MASK) == depth)
            selected.push(h);
          next.push(h);
        }
      }
    }
    cur = next;
  }
  in.out_sent.assign(selected.size(), {});
  in.out_logp_norm.assign(selected.size(), 0.0);
  size_t i = 0;
  while (!selected.empty()) {
    const Hyp& h = pool[selected.pop()];
    std::vector<Label>& q = in.out_sent[i];
    q.resize(h.depth);
    UInt32 hi = h.hist;
    for (size_t pos = h.depth; pos-- > 0;) {
      q[pos] = hist[hi].second;
      hi = hist[hi].first;
    }
    in.out_logp_norm[i] = h.norm;
    ++i;
  }
}

}  // namespace

Trie::Trie() : impl_(new TrieImpl()) {}
Trie::~Trie() = default;

void Trie::build(Keyset& keyset, int config_flags) {
  const int num_tries = config_flags & MARISA_NUM_TRIES_MASK;
  const int order = config_flags & MARISA_NODE_ORDER_MASK;
  const int tail = config_flags & MARISA_TAIL_MODE_MASK;
  if ((num_tries != 0 && num_tries != 1) ||
      (order != 0 && order != MARISA_LABEL_ORDER) ||
      (tail != 0 && tail != MARISA_TEXT_TAIL))
    throw Exception(MARISA_CODE_ERROR,
                    "build: only num_tries=1, MARISA_TEXT_TAIL and "
                    "MARISA_LABEL_ORDER tries are supported");
  auto fresh = std::unique_ptr<TrieImpl>(new TrieImpl());
  std::string err;
  const auto& offs = keyset.offsets();
  if (!ftamd::build_image_from_keys(keyset.tokens().data(), offs.data(),
                                    keyset.size(), &fresh->img, &err))
    throw Exception(MARISA_SIZE_ERROR, "build: " + err);
  impl_.swap(fresh);
}

void Trie::build(const std::vector<std::vector<Label>>& keys) {
  Keyset ks;
  for (const auto& k : keys) ks.push_back(k.data(), k.size());
  build(ks, 0);
}

namespace {

// load (read the file) and mmap (map it): this library's image is used as
// it is -- in place for a mapping -- and validated; a MARISA trie file
// written by the reference (lib/marisa/trie.cc:21-53) is converted.
void open_trie(const char* filename, bool map, std::unique_ptr<TrieImpl>* out) {
  const char* who = map ? "mmap: " : "load: ";
  if (!filename) throw Exception(MARISA_NULL_ERROR, std::string(who) + "null filename");
  ftamd::ImageBlob file;
  std::string err;
  if (!(map ? file.map_file(filename, &err) : file.read_file(filename, &err)))
    throw Exception(MARISA_IO_ERROR, who + err);
  auto fresh = std::unique_ptr<TrieImpl>(new TrieImpl());
  if (ftamd::is_marisa_file(file.data(), file.size())) {
    if (!ftamd::image_from_marisa(file.data(), file.size(), &fresh->img, &err))
      throw Exception(MARISA_FORMAT_ERROR, std::string(who) + filename + ": " + err);
  } else {
    fresh->img.swap(file);
    if (!ftamd::validate_image(fresh->img, &err))
      throw Exception(MARISA_FORMAT_ERROR, std::string(who) + err);
  }
  out->swap(fresh);
}

}  // namespace

void Trie::load(const char* filename) { open_trie(filename, false, &impl_); }

void Trie::mmap(const char* filename) { open_trie(filename, true, &impl_); }

void Trie::map(const void* ptr, std::size_t size) {
  if (!ptr && size) throw Exception(MARISA_NULL_ERROR, "map: null pointer");
  auto fresh = std::unique_ptr<TrieImpl>(new TrieImpl());
  std::string err;
  if (ftamd::is_marisa_file(ptr, size)) {
    if (!ftamd::image_from_marisa((const uint8_t*)ptr, size, &fresh->img, &err))
      throw Exception(MARISA_FORMAT_ERROR, "map: " + err);
  } else {
    // an image is used in place when its arrays are aligned, else copied
    if ((uintptr_t)ptr % 16 == 0) {
      fresh->img.borrow(ptr, size);
    } else if (!fresh->img.assign(ptr, size)) {
      throw Exception(MARISA_MEMORY_ERROR, "map: out of memory");
    }
    if (!ftamd::validate_image(fresh->img, &err))
      throw Exception(MARISA_FORMAT_ERROR, "map: " + err);
  }
  impl_.swap(fresh);
}

void Trie::read(int fd) {
  if (fd == -1) throw Exception(MARISA_CODE_ERROR, "read: fd == -1");
  auto fresh = std::unique_ptr<TrieImpl>(new TrieImpl());
  std::string err;
  uint8_t head[sizeof(ft_image_header)];
  if (!ftamd::read_exact(fd, head, 16))
    throw Exception(MARISA_IO_ERROR, "read: the stream ends before a trie header");
  if (ftamd::is_marisa_file(head, 16)) {
    std::vector<uint8_t> bytes;
    if (!ftamd::read_marisa_stream(fd, head, &bytes, &err))
      throw Exception(MARISA_IO_ERROR, err);
    if (!ftamd::image_from_marisa(bytes.data(), bytes.size(), &fresh->img, &err))
      throw Exception(MARISA_FORMAT_ERROR, "read: " + err);
  } else {
    if (std::memcmp(head, FT_IMAGE_MAGIC, 8) != 0)
      throw Exception(MARISA_FORMAT_ERROR, "read: neither a MARISA trie file nor a trie image");
    if (!ftamd::read_exact(fd, head + 16, sizeof(head) - 16))
      throw Exception(MARISA_IO_ERROR, "read: the stream ends in the image header");
    ft_image_header h;
    std::memcpy(&h, head, sizeof(h));
    if (h.total_bytes < sizeof(h) || h.total_bytes > (1ull << 44))
      throw Exception(MARISA_FORMAT_ERROR, "read: implausible image size");
    if (!fresh->img.allocate_bytes((size_t)h.total_bytes))
      throw Exception(MARISA_MEMORY_ERROR, "read: out of memory");
    std::memcpy(fresh->img.data(), head, sizeof(h));
    if (!ftamd::read_exact(fd, fresh->img.data() + sizeof(h), (size_t)h.total_bytes - sizeof(h)))
      throw Exception(MARISA_IO_ERROR, "read: the stream ends inside the image");
    if (!ftamd::validate_image(fresh->img, &err))
      throw Exception(MARISA_FORMAT_ERROR, "read: " + err);
  }
  impl_.swap(fresh);
}

void Trie::write(int fd) const {
  require_trie(impl_.get());
  if (fd == -1) throw Exception(MARISA_CODE_ERROR, "write: fd == -1");
  if (!ftamd::write_all(fd, impl_->img.data(), impl_->img.size()))
    throw Exception(MARISA_IO_ERROR, "write: failed on the descriptor");
}

void Trie::save(const char* filename) const {
  require_trie(impl_.get());
  if (!filename) throw Exception(MARISA_NULL_ERROR, "save: null filename");
  std::ofstream f(filename, std::ios::binary);
  if (!f) throw Exception(MARISA_IO_ERROR, std::string("save: cannot open ") + filename);
  f.write((const char*)impl_->img.data(), (std::streamsize)impl_->img.size());
  if (!f) throw Exception(MARISA_IO_ERROR, std::string("save: write failed on ") + filename);
}

void Trie::save_marisa(const char* filename) const {
  require_trie(impl_.get());
  if (!filename) throw Exception(MARISA_NULL_ERROR, "save_marisa: null filename");
  std::vector<uint8_t> bytes;
  std::string err;
  if (!ftamd::marisa_from_image(impl_->img, &bytes, &err))
    throw Exception(MARISA_FORMAT_ERROR, "save_marisa: " + err);
  std::ofstream f(filename, std::ios::binary);
  if (!f) throw Exception(MARISA_IO_ERROR, std::string("save_marisa: cannot open ") + filename);
  f.write((const char*)bytes.data(), (std::streamsize)bytes.size());
  if (!f) throw Exception(MARISA_IO_ERROR, std::string("save_marisa: write failed on ") + filename);
}

void Trie::init_tbs_gpu(size_t max_batch_size, size_t max_num_topk,
                        size_t max_num_outpos, size_t max_num_out_beams,
                        size_t max_num_out_tokens, size_t max_num_inter_beams,
                        size_t radix_topk_threshold) {
  (void)radix_topk_threshold;  // selection is exact at every size here
  require_trie(impl_.get());
  TrieImpl& t = *impl_;
  t.drop_gpu();
  int rc = ft_create(t.img.data(), t.img.size(), 0, &t.ctx);
  if (rc) throw_ft(rc, "init_tbs_gpu");
  rc = ft_reserve(t.ctx, max_batch_size, max_num_topk, max_num_outpos,
                  max_num_out_beams, max_num_out_tokens, max_num_inter_beams);
  if (rc) {
    t.drop_gpu();
    throw_ft(rc, "init_tbs_gpu");
  }
  t.max_batch = max_batch_size;
  t.max_topk = max_num_topk;
  t.max_outpos = max_num_outpos;
  t.max_out_beams = max_num_out_beams;
}

size_t Trie::get_max_batch_size() const {
  require_trie(impl_.get());
  return impl_->max_batch;
}

void Trie::tbs(TbsInput& input) const {
  require_trie(impl_.get());
  host_tbs(impl_->img, input);
}

void Trie::tbs_gpu(TbsInput& input, size_t batch_id) const {
  require_trie(impl_.get());
  if (!impl_->ctx)
    throw Exception(MARISA_STATE_ERROR, "tbs_gpu: init_tbs_gpu was not called");
  if (batch_id >= impl_->max_batch)
    throw Exception(MARISA_BOUND_ERROR, "tbs_gpu: batch_id >= max_batch_size");
  std::vector<TbsInput> one;
  one.push_back(input);
  tbs_gpu_batched(one);
  input.t_expansion_ms = one[0].t_expansion_ms;
  input.t_validation_ms = one[0].t_validation_ms;
  input.t_selection_ms = one[0].t_selection_ms;
  input.t_grid_overhead_ms = one[0].t_grid_overhead_ms;
  input.kernel_ms = one[0].kernel_ms;
}

void Trie::tbs_gpu_batched(std::vector<TbsInput>& inputs) const {
  require_trie(impl_.get());
  TrieImpl& t = *impl_;
  if (!t.ctx) throw Exception(MARISA_STATE_ERROR, "tbs_gpu_batched: init_tbs_gpu was not called");
  if (inputs.empty()) return;
  if (inputs.size() > t.max_batch)
    throw Exception(MARISA_BOUND_ERROR, "tbs_gpu_batched: batch larger than max_batch_size");
  const size_t B = inputs.size();
  // one search at a time per trie; its request and result buffers are kept
  // from call to call
  std::lock_guard<std::mutex> lock(t.search_mu);
  TrieImpl::SearchBuffers& sb = t.sb;
  sb.reqs.resize(B);
  sb.res.resize(B);
  sb.shapes.resize(B);
  if (sb.rows.size() < B) sb.rows.resize(B);
  for (size_t b = 0; b < B; ++b) {
    const TbsInput& in = inputs[b];
    sb.shapes[b] = check_shape(in);
    ft_request& q = sb.reqs[b];
    std::memset(&q, 0, sizeof(q));
    q.beams = in.beams.data();
    q.num_beams = (uint32_t)in.beams.size();
    q.token_logp_threshold = in.token_logp_threshold;
    q.sent_logp_threshold = in.sent_logp_threshold;
    q.length_norm = in.length_norm;
    q.early_exit = in.early_exit ? 1 : 0;
    std::memset(&sb.res[b], 0, sizeof(ft_result));
    if (sb.shapes[b].F == 0) continue;
    const size_t T = sb.shapes[b].T, K = sb.shapes[b].K;
    q.num_steps = (uint32_t)T;
    q.topk = (uint32_t)K;
    TrieImpl::SearchBuffers::Rows& rw = sb.rows[b];
    rw.id.resize(T);
    rw.lp.resize(T);
    for (size_t r = 0; r < T; ++r) {
      rw.id[r] = in.topk_id[r].data();
      rw.lp[r] = in.topk_logp[r].data();
    }
    q.topk_id_rows = rw.id.data();
    q.topk_logp_rows = rw.lp.data();
    // result arrays, grown as needed and never shrunk: the search writes the
    // first count entries of each, and only those are read
    const size_t F = sb.shapes[b].F;
    if (rw.norms.size() < F) rw.norms.resize(F);
    if (rw.lens.size() < F) rw.lens.resize(F);
    if (rw.toks.size() < F * T) rw.toks.resize(F * T);
    ft_result& o = sb.res[b];
    o.capacity = (uint32_t)F;
    o.token_stride = (uint32_t)T;
    o.logp_norm = rw.norms.data();
    o.length = rw.lens.data();
    o.tokens = rw.toks.data();
  }
  // Each request's output vectors are filled as soon as its results are
  // in, while the rest of the batch still searches.  The callback runs
  // inside ft_search_each with the kernel still running, so nothing may
  // unwind through it: an exception (bad_alloc from the vectors) is kept,
  // the search runs to its end, and it is rethrown afterwards.  On any
  // error the outputs filled so far are emptied again: a failed call
  // leaves no partial results.
  struct Fill {
    std::vector<TbsInput>* inputs;
    TrieImpl::SearchBuffers* sb;
    std::exception_ptr err;
    std::vector<size_t> filled;
  } fill{&inputs, &sb, nullptr, {}};
  fill.filled.reserve(B);
  auto on_result = [](void* user, size_t b) {
    Fill& f = *(Fill*)user;
    if (f.err) return;
    TbsInput& in = (*f.inputs)[b];
    if (f.sb->shapes[b].F == 0) return;  // outputs untouched
    try {
      f.filled.push_back(b);
      const ft_result& o = f.sb->res[b];
      const size_t T = f.sb->shapes[b].T;
      const TrieImpl::SearchBuffers::Rows& rw = f.sb->rows[b];
      in.out_sent.resize(o.count);
      in.out_logp_norm.assign(rw.norms.data(), rw.norms.data() + o.count);
      for (uint32_t i = 0; i < o.count; ++i)
        in.out_sent[i].assign(rw.toks.data() + i * T, rw.toks.data() + i * T + rw.lens[i]);
      in.t_expansion_ms = o.device_ms[0];
      in.t_validation_ms = 0.0;
      in.t_selection_ms = o.device_ms[1];
      in.t_grid_overhead_ms = o.device_ms[2];
      in.kernel_ms = o.device_ms[3];
    } catch (...) {
      f.err = std::current_exception();
    }
  };
  const int rc = ft_search_each(t.ctx, sb.reqs.data(), B, sb.res.data(), nullptr, on_result, &fill);
  if (rc || fill.err) {
    for (size_t b : fill.filled) {
      inputs[b].out_sent.clear();
      inputs[b].out_logp_norm.clear();
    }
    if (fill.err) std::rethrow_exception(fill.err);
    throw_ft(rc, "tbs_gpu_batched");
  }
}

std::size_t Trie::num_tries() const {
  require_trie(impl_.get());
  return 1;
}
std::size_t Trie::num_keys() const {
  require_trie(impl_.get());
  return impl_->img.header().num_keys;
}
std::size_t Trie::num_nodes() const {
  require_trie(impl_.get());
  return impl_->img.header().num_nodes;
}
TailMode Trie::tail_mode() const { return MARISA_TEXT_TAIL; }
NodeOrder Trie::node_order() const { return MARISA_LABEL_ORDER; }
bool Trie::empty() const { return num_keys() == 0; }
std::size_t Trie::size() const { return num_keys(); }
std::size_t Trie::total_size() const {
  require_trie(impl_.get());
  return impl_->img.size();
}
std::size_t Trie::io_size() const { return total_size(); }
void Trie::clear() { impl_.reset(new TrieImpl()); }
void Trie::swap(Trie& rhs) { impl_.swap(rhs.impl_); }

const void* Trie::image_data() const {
  require_trie(impl_.get());
  return impl_->img.data();
}
std::size_t Trie::image_size() const {
  require_trie(impl_.get());
  return impl_->img.size();
}
void Trie::assign_image(const void* data, std::size_t size) {
  auto fresh = std::unique_ptr<TrieImpl>(new TrieImpl());
  if (!fresh->img.assign(data, size))
    throw Exception(MARISA_MEMORY_ERROR, "assign_image: out of memory");
  std::string err;
  if (!ftamd::validate_image(fresh->img, &err))
    throw Exception(MARISA_FORMAT_ERROR, "assign_image: " + err);
  impl_.swap(fresh);
}

}  // namespace marisa
