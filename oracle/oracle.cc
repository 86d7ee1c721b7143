// oracle.cc -- TEST INFRASTRUCTURE ONLY (the parity oracle).
//
// A CPU restatement of the reference's trie beam search path, used by
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
// checker and the timed CPU baseline.  No product code links or calls this.
//
// What it restates (paths relative to the reference repository):
//   * trie build, num_tries == 1, TEXT_TAIL, LABEL_ORDER
//       LoudsTrie::build_current_trie  lib/marisa/grimoire/trie/louds-trie.cc:477-588
//       key order of Algorithm().sort  lib/marisa/grimoire/algorithm/sort.h:15-190
//   * the CPU search
//       LoudsTrie::tbs                 louds-trie.cc:113-177
//       tbs_lookup_                    louds-trie.cc:75-111
//       LoudsTrie::predictive_find_child louds-trie.cc:810-856
//       Tail::prefix_match (text tail) lib/marisa/grimoire/trie/tail.cc:132-169
//       Agent(parent, token, score)    lib/marisa/agent.cc:12-37
//       Agent::logp_norm               include/marisa/agent.h:69-72
//       Candidates / AgentComparer     lib/marisa/grimoire/trie/candidates.h:16-80
//
// The reference cannot be compiled here (every translation unit needs the CUDA
// runtime, CUB and NVTX), so there is no oracle/_ref build; the restatement is
// pinned instead by the known-answer cases, brute-force enumeration and
// invariants in tests/test_oracle.py.
//
// Two search variants produce identical outputs:
//   variant 0 "as-written": one std::thread spawned and joined per parent and a
//             linear sibling scan, i.e. the reference's cost model;
//   variant 1 "fast": the same state machine with binary sibling search, no
//             thread spawn and cached norms.  It also fills the work counters
//             used for the algorithmic-bytes figure.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <mutex>
#include <queue>
#include <thread>
#include <vector>

#include "../include/flashtrie_amd.h"

namespace oracle {

typedef uint32_t Label;

// ---------------------------------------------------------------------------
// Trie access.  Node ids are BFS ids with root 0 (louds-trie.cc:496-501); the
// children of node n are the contiguous ids [child_begin(n), child_begin(n+1))
// in ascending first-token order (louds-trie.cc:483, 527-530).  edge(n) is the
// token string on the edge into n: one token for a label node, the whole tail
// (>= 2 tokens) for a link node (louds-trie.cc:554-571).
// ---------------------------------------------------------------------------
struct TrieView {
  virtual ~TrieView() {}
  virtual uint64_t num_nodes() const = 0;
  virtual uint32_t child_begin(uint64_t n) const = 0;
  virtual uint32_t edge_len(uint64_t n) const = 0;
  virtual Label edge_at(uint64_t n, uint32_t i) const = 0;
  virtual bool terminal(uint64_t n) const = 0;
};

// Plain arrays, as produced by the restated builder below.
struct LogicalTrie : TrieView {
  std::vector<uint32_t> cb;   // N + 1
  std::vector<uint64_t> eb;   // N + 1
  std::vector<Label> et;
  std::vector<uint8_t> term;  // N
  uint64_t nkeys = 0;
  uint64_t num_nodes() const override { return term.size(); }
  uint32_t child_begin(uint64_t n) const override { return cb[n]; }
  uint32_t edge_len(uint64_t n) const override {
    return (uint32_t)(eb[n + 1] - eb[n]);
  }
  Label edge_at(uint64_t n, uint32_t i) const override { return et[eb[n] + i]; }
  bool terminal(uint64_t n) const override { return term[n] != 0; }
};

// A read-only view over the device image layout declared in flashtrie_amd.h
// (16-byte node records + tail array).  Used to run the CPU baseline on tries
// that are generated directly in that layout and are too large to rebuild
// from keys.
struct ImageTrie : TrieView {
  const ft_node_rec* rec = nullptr;
  const uint32_t* tail = nullptr;
  uint64_t n = 0;
  uint64_t num_nodes() const override { return n; }
  uint32_t child_begin(uint64_t i) const override { return rec[i].child_begin; }
  uint32_t edge_len(uint64_t i) const override {
    return (rec[i].meta >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
  }
  Label edge_at(uint64_t i, uint32_t k) const override {
    if (rec[i].meta & FT_META_LINK) return tail[rec[i].tail_off + k];
    return rec[i].first_tok;
  }
  bool terminal(uint64_t i) const override {
    return (rec[i].meta & FT_META_TERMINAL) != 0;
  }
};

// ---------------------------------------------------------------------------
// Build (louds-trie.cc:477-588, num_tries == 1).
// ---------------------------------------------------------------------------
struct KeyRef {
  const Label* p;
  uint32_t len;
  Label operator[](size_t i) const { return p[i]; }
};

// Order of Algorithm().sort: labels compared as int, a shorter key that is a
// prefix sorts first (sort.h:16-20 returns -1 past the end).
static bool key_less(const KeyRef& a, const KeyRef& b) {
  const size_t m = std::min(a.len, b.len);
  for (size_t i = 0; i < m; ++i) {
    const int x = (int)a.p[i], y = (int)b.p[i];
    if (x != y) return x < y;
  }
  return a.len < b.len;
}

struct Range {
  size_t begin, end, key_pos;
};

static LogicalTrie* build(const Label* toks, const uint64_t* offs,
                          uint64_t nkeys) {
  std::vector<KeyRef> keys(nkeys);
  for (uint64_t i = 0; i < nkeys; ++i)
    keys[i] = KeyRef{toks + offs[i], (uint32_t)(offs[i + 1] - offs[i])};
  std::sort(keys.begin(), keys.end(), key_less);

  auto* t = new LogicalTrie();
  // Node 0 is the root with an empty edge (louds-trie.cc:486-490).
  t->eb.push_back(0);
  t->eb.push_back(0);
  t->term.push_back(0);
  size_t created = 1;
  std::queue<Range> queue;
  queue.push(Range{0, keys.size(), 0});
  while (!queue.empty()) {
    const size_t node_id = created - queue.size();  // louds-trie.cc:498
    Range range = queue.front();
    queue.pop();
    if (t->cb.size() != node_id) { delete t; return nullptr; }
    t->cb.push_back((uint32_t)created);
    // Keys that end here make the node terminal (louds-trie.cc:503-507).
    while (range.begin < range.end &&
           keys[range.begin].len == range.key_pos) {
      t->term[node_id] = 1;
      ++range.begin;
    }
    if (range.begin == range.end) continue;
    // Split into groups sharing the token at key_pos (louds-trie.cc:514-526).
    std::vector<Range> groups;
    for (size_t i = range.begin + 1; i < range.end; ++i) {
      if (keys[i - 1][range.key_pos] != keys[i][range.key_pos]) {
        groups.push_back(Range{range.begin, i, range.key_pos});
        range.begin = i;
      }
    }
    groups.push_back(Range{range.begin, range.end, range.key_pos});
    // Path compression (louds-trie.cc:536-575).
    for (Range& g : groups) {
      size_t key_pos = g.key_pos + 1;
      while (key_pos < keys[g.begin].len) {
        size_t j;
        for (j = g.begin + 1; j < g.end; ++j)
          if (keys[j - 1][key_pos] != keys[j][key_pos]) break;
        if (j < g.end) break;
        ++key_pos;
      }
      for (size_t p = g.key_pos; p < key_pos; ++p)
        t->et.push_back(keys[g.begin][p]);
      t->eb.push_back(t->et.size());
      t->term.push_back(0);
      ++created;
      queue.push(Range{g.begin, g.end, key_pos});
    }
  }
  t->cb.push_back((uint32_t)created);
  uint64_t nk = 0;
  for (uint8_t b : t->term) nk += b;
  t->nkeys = nk;
  return t;
}

// ---------------------------------------------------------------------------
// Search state (agent.cc:12-37, agent.h:66-72, state.h:101-111).
// ---------------------------------------------------------------------------
struct Agent {
  std::vector<Label> query;    // Q: consumed tokens
  std::vector<Label> key_buf;  // KB: restored key buffer
  uint64_t node = 0;
  size_t query_pos = 0;
  double score = 0.0;          // sum of f32 logps in f64 (agent.cc:36)
  double length_norm = 0.0;
  double norm_cache = 0.0;
  bool cached = false;
  double logp_norm() const {   // agent.h:69-72
    return score * std::pow(6.0 / (5.0 + (double)query.size()), length_norm);
  }
};
typedef std::shared_ptr<Agent> AgentPtr;

// AgentComparer (candidates.h:16-30): the heap top is the minimum norm, ties
// broken towards the smaller node id.
struct AgentComparer {
  bool fast = false;
  double norm(const Agent* a) const {
    return fast ? a->norm_cache : a->logp_norm();
  }
  bool operator()(const AgentPtr& l, const AgentPtr& r) const {
    const double a = norm(l.get()), b = norm(r.get());
    if (a == b) return l->node > r->node;
    return a > b;
  }
};

// Candidates (candidates.h:32-80): bounded heap of the best `max` agents.
struct Candidates {
  std::priority_queue<AgentPtr, std::vector<AgentPtr>, AgentComparer> cand;
  unsigned int max_;
  std::shared_ptr<std::mutex> mtx;
  bool fast;
  Candidates(unsigned int m, bool f)
      : cand(AgentComparer{f}), max_(m), mtx(std::make_shared<std::mutex>()),
        fast(f) {}
  double norm(const AgentPtr& a) const {
    return fast ? a->norm_cache : a->logp_norm();
  }
  // Returns false where the reference would read top() of an empty heap
  // (capacity 0), which is undefined behaviour there.
  bool push(const AgentPtr& a) {
    std::lock_guard<std::mutex> g(*mtx);
    if (cand.size() < max_) {
      cand.push(a);
    } else {
      if (cand.empty()) return false;
      if (norm(a) > norm(cand.top())) cand.push(a);
    }
    if (cand.size() > max_) cand.pop();
    return true;
  }
  AgentPtr pop() {
    AgentPtr r = cand.top();
    cand.pop();
    return r;
  }
  bool empty() const { return cand.empty(); }
  size_t size() const { return cand.size(); }
};

struct Work {
  // Work counters for the algorithmic-bytes model (fast variant only).
  uint64_t steps = 0, parents = 0, lp_parents = 0, child_units = 0,
           pushes = 0, survivors = 0, row_bytes = 0;
};

// predictive_find_child (louds-trie.cc:810-856) with the text-tail
// prefix_match (tail.cc:132-169): the first sibling whose first edge token
// equals the query token wins; the whole edge is appended to key_buf.
static bool find_child(const TrieView& t, Agent& a, bool binary,
                       uint64_t* probes) {
  const uint64_t n = a.node;
  const uint32_t c0 = t.child_begin(n), c1 = t.child_begin(n + 1);
  if (c0 == c1) return false;
  const Label tok = a.query[a.query_pos];
  uint64_t found = UINT64_MAX;
  if (!binary) {
    for (uint32_t c = c0; c < c1; ++c) {
      if (t.edge_at(c, 0) == tok) { found = c; break; }
    }
  } else {
    uint32_t lo = c0, hi = c1;
    while (lo < hi) {
      const uint32_t mid = lo + (hi - lo) / 2;
      if (probes) ++*probes;
      if (t.edge_at(mid, 0) < tok) lo = mid + 1; else hi = mid;
    }
    if (lo < c1 && t.edge_at(lo, 0) == tok) found = lo;
  }
  if (found == UINT64_MAX) return false;
  const uint32_t el = t.edge_len(found);
  for (uint32_t i = 0; i < el; ++i) a.key_buf.push_back(t.edge_at(found, i));
  a.query_pos += 1;
  a.node = found;
  return true;
}

struct Input {
  const uint32_t* beams;
  uint64_t nbeams;
  const uint32_t* ids;
  const float* logp;
  uint64_t T, K;
  float tok_thr;
  double sent_thr, alpha;
  bool early_exit;
};

// tbs_lookup_ (louds-trie.cc:75-111).
static void lookup(const TrieView* t, AgentPtr parent, bool link_parent,
                   const Input* in, uint32_t final_beam, uint64_t row,
                   Candidates* selected, Candidates* next, bool fast,
                   Work* w, bool* bad) {
  const uint32_t* ids = in->ids + row * in->K;
  const float* lp = in->logp + row * in->K;
  uint64_t passing = 0, probes = 0;
  for (uint64_t index = 0; index < in->K; ++index) {
    if (in->early_exit && selected->size() >= final_beam) break;
    const Label token = ids[index];
    const float score = lp[index];
    // thresholds are compared in double (louds-trie.cc:76-78, 87-90)
    if ((double)score <= (double)in->tok_thr ||
        parent->score + score <= in->sent_thr)
      continue;
    ++passing;
    if (link_parent && token != parent->key_buf[parent->query.size()])
      continue;
    auto child = std::make_shared<Agent>();
    child->query = parent->query;
    child->query.push_back(token);
    child->key_buf = parent->key_buf;
    child->node = parent->node;
    child->query_pos = parent->query_pos;
    child->score = parent->score + score;
    child->length_norm = parent->length_norm;
    if (link_parent) {
      if (fast) child->norm_cache = child->logp_norm();
      ++w->pushes;
      if (child->query.size() == child->key_buf.size()) {
        if (!selected->push(child)) *bad = true;
      } else {
        if (!next->push(child)) *bad = true;
      }
    } else if (find_child(*t, *child, fast, &probes)) {
      if (fast) child->norm_cache = child->logp_norm();
      if (t->terminal(child->node) &&
          child->key_buf.size() == child->query.size()) {
        ++w->pushes;
        if (!selected->push(child)) *bad = true;
      }
      ++w->pushes;
      if (!next->push(child)) *bad = true;
    }
  }
  if (fast && !link_parent) {
    const uint64_t d = t->child_begin(parent->node + 1) -
                       t->child_begin(parent->node);
    uint64_t lg = 0;
    while ((1ull << lg) < d + 1) ++lg;
    w->child_units += std::min<uint64_t>(d, passing * lg);
  } else if (fast) {
    w->child_units += 1;
  }
}

// LoudsTrie::tbs (louds-trie.cc:113-177).  Returns 0 on success, negative
// where the reference has undefined behaviour.
static int tbs(const TrieView& t, const Input& in, int variant,
               std::vector<AgentPtr>* out, Work* w) {
  if (in.nbeams == 0) return -1;
  const uint32_t final_beam = in.beams[in.nbeams - 1];
  if (final_beam == 0) return 1;  // outputs untouched (louds-trie.cc:114-117)
  if (in.T == 0 || in.K == 0) return -2;  // topk_id[0] / division by zero
  if (in.nbeams < in.T) return -3;        // beams[outpos] out of range
  const bool fast = variant != 0;
  Candidates selected(final_beam, fast);
  auto root = std::make_shared<Agent>();
  root->length_norm = in.alpha;
  if (fast) root->norm_cache = root->logp_norm();
  Candidates cur(1, fast);
  cur.push(root);
  bool bad = false;
  for (uint64_t outpos = 0; outpos < in.T; ++outpos) {
    if (cur.empty() || (in.early_exit && selected.size() >= final_beam))
      break;
    ++w->steps;
    w->row_bytes += 8 * in.K;
    Candidates next(in.beams[outpos], fast);
    while (!cur.empty()) {
      AgentPtr parent = cur.pop();
      const bool link_parent = t.terminal(parent->node) &&
                               parent->key_buf.size() > parent->query.size();
      ++w->parents;
      if (link_parent) ++w->lp_parents;
      if (variant == 0) {
        // one worker thread per parent (louds-trie.cc:120, 155-163)
        std::thread th(lookup, &t, parent, link_parent, &in, final_beam,
                       outpos, &selected, &next, fast, w, &bad);
        th.join();
      } else {
        lookup(&t, parent, link_parent, &in, final_beam, outpos, &selected,
               &next, fast, w, &bad);
      }
    }
    if (bad) return -4;  // push into a zero-capacity heap
    w->survivors += next.size();
    cur = next;
  }
  out->clear();
  while (!selected.empty()) out->push_back(selected.pop());
  return 0;
}

}  // namespace oracle

using namespace oracle;

extern "C" {

void* ot_build(const uint32_t* toks, const uint64_t* offs, uint64_t nkeys) {
  return build(toks, offs, nkeys);
}

// Wraps an image in the device layout; the arrays are borrowed, not copied.
void* ot_wrap_image(const void* recs, const uint32_t* tail, uint64_t n) {
  auto* v = new ImageTrie();
  v->rec = (const ft_node_rec*)recs;
  v->tail = tail;
  v->n = n;
  return v;
}

void ot_free(void* h) { delete (TrieView*)h; }

uint64_t ot_num_nodes(void* h) { return ((TrieView*)h)->num_nodes(); }

uint64_t ot_num_keys(void* h) {
  auto* lt = dynamic_cast<LogicalTrie*>((TrieView*)h);
  return lt ? lt->nkeys : 0;
}

uint64_t ot_num_edge_tokens(void* h) {
  auto* lt = dynamic_cast<LogicalTrie*>((TrieView*)h);
  return lt ? lt->et.size() : 0;
}

// Copies the logical arrays out (LogicalTrie only).
int ot_export(void* h, uint32_t* cb, uint64_t* eb, uint32_t* et,
              uint8_t* term) {
  auto* lt = dynamic_cast<LogicalTrie*>((TrieView*)h);
  if (!lt) return -1;
  std::memcpy(cb, lt->cb.data(), lt->cb.size() * 4);
  std::memcpy(eb, lt->eb.data(), lt->eb.size() * 8);
  std::memcpy(et, lt->et.data(), lt->et.size() * 4);
  std::memcpy(term, lt->term.data(), lt->term.size());
  return 0;
}

// One request.  Outputs in the reference's order (ascending norm, ties by
// ascending node id): out_norm[i], out_len[i], tokens at out_tok[i*T ...].
// work[7] (nullable): steps, parents, link parents, child units, pushes,
// survivors, row bytes.
int ot_tbs(void* h, const uint32_t* beams, uint64_t nbeams,
           const uint32_t* ids, const float* logp, uint64_t T, uint64_t K,
           float tok_thr, double sent_thr, double alpha, int early_exit,
           int variant, uint64_t out_cap, uint64_t* out_count,
           double* out_norm, uint32_t* out_len, uint32_t* out_tok,
           uint64_t* out_node, uint64_t* work) {
  Input in{beams, nbeams, ids, logp, T, K, tok_thr, sent_thr, alpha,
           early_exit != 0};
  std::vector<AgentPtr> out;
  Work w;
  const int rc = tbs(*(TrieView*)h, in, variant, &out, &w);
  *out_count = 0;
  if (work) {
    work[0] = w.steps; work[1] = w.parents; work[2] = w.lp_parents;
    work[3] = w.child_units; work[4] = w.pushes; work[5] = w.survivors;
    work[6] = w.row_bytes;
  }
  if (rc != 0) return rc;
  if (out.size() > out_cap) return -5;
  for (size_t i = 0; i < out.size(); ++i) {
    out_norm[i] = out[i]->logp_norm();
    out_len[i] = (uint32_t)out[i]->query.size();
    if (out_node) out_node[i] = out[i]->node;
    for (size_t j = 0; j < out[i]->query.size() && j < T; ++j)
      out_tok[i * T + j] = out[i]->query[j];
  }
  *out_count = out.size();
  return 0;
}

}  // extern "C"
