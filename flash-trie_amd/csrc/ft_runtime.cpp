// ft_runtime.cpp -- host side of the C ABI (include/flashtrie_amd.h).
//
// Owns the trie image in HBM, the per-request workspace (allocated once by
// ft_reserve, like LoudsTrie::init_tbs_gpu, tbs-kernels.cu:599-648), the
// pinned staging buffers and the stream.  A batch is packed into one pinned
// buffer, copied with one H2D, searched by one kernel launch and copied
// back with one D2H (compare the per-request launches of tbs_gpu_batched,
// tbs-kernels.cu:686-700).
#include <hip/hip_runtime.h>

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "../../include/flashtrie_amd.h"
#include "tbs_kernel.h"

using namespace ftk;

static_assert(kScratchBytes == FT_NOALLOC_SCRATCH_BYTES, "the header states the scratch size");
static_assert(kStepStats == FT_STEP_STATS, "the header states the per-step profile");

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  g_err = std::string(what) + ": " + hipGetErrorString(e);
  return e == hipErrorOutOfMemory ? FT_E_NOMEM : FT_E_HIP;
}

inline uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

struct StagedReq {
  uint32_t T = 0, K = 0, F = 0;
  bool skip = false;
  uint64_t out_bytes = 0;
  uint64_t bmax = 0;  // widest beam of any step (and the final beam)
  uint64_t hsum = 0;  // sum of the beam widths: bounds the history records
};

}  // namespace

struct ft_ctx {
  int device = 0;
  uint8_t* d_image = nullptr;
  ft_image_header hdr{};
  hipStream_t stream = nullptr;
  int num_cus = 0, lds_per_block = 0, wall_khz = 0;
  char name[64] = {0};

  bool reserved = false;
  size_t max_batch = 0, max_topk = 0, max_steps = 0, max_out_beams = 0,
         max_out_tokens = 0, max_inter = 0;
  WsLayout lay{};
  uint64_t ws_stride = 0;
  uint8_t* d_ws = nullptr;
  uint64_t out_slot_max = 0;
  uint8_t* d_out = nullptr;
  uint8_t* h_out = nullptr;
  uint64_t stage_cap = 0;
  uint8_t* d_stage = nullptr;
  uint8_t* h_stage = nullptr;
  // the device's addresses of h_stage, h_out and h_ready (pinned, coherent
  // host memory mapped for the device), read and written by the kernel in a
  // streamed search
  uint8_t* m_stage = nullptr;
  uint8_t* m_out = nullptr;
  unsigned long long* h_ready = nullptr;  // per staged request: ready word
  unsigned long long* m_ready = nullptr;

  size_t max_staged = 0;  // staging / output capacity in requests
  uint64_t per_req = 0;   // staging bytes bound of one request

  // wide-node index (device)
  WideDirGroup* d_wdir = nullptr;
  WideBucket* d_wtab = nullptr;
  uint64_t* d_wfp = nullptr;     // per bucket: slot fingerprints
  uint32_t* d_labels = nullptr;  // per node: first token | kSlotSel
  // LOUDS child-range directory (FT_CHILD_INDEX=louds), else null
  uint64_t* d_louds_words = nullptr;
  uint32_t* d_louds_z = nullptr;
  uint32_t* d_louds_s = nullptr;
  uint64_t louds_bytes = 0;
  uint32_t wdir_log2 = 0, wide_min = 0;
  uint64_t wide_nodes = 0, wide_buckets = 0, wide_failed = 0;
  // root directory (null: none; FT_ROOT_DIR=0 turns it off, =force makes
  // step 0 use it for a scanned root too)
  RootEnt* d_root_dir = nullptr;
  uint32_t root_n = 0, root_force = 0;

  std::vector<StagedReq> staged;
  // per request of a streamed search: taken, its error and error text
  std::vector<uint8_t> req_got;
  std::vector<int> req_rc;
  std::vector<std::string> req_msg;
  std::vector<std::pair<uint32_t, uint32_t>> sort_tmp;  // max_topk pairs
  // staged requests launched since the last ft_stage (ft_fetch reports the
  // others as FT_E_STATE instead of returning whatever d_out holds)
  std::vector<uint8_t> launched_slot;
  uint64_t out_stride = 0;
  bool launched = false;
  // recorded after each staging copy: the next ft_stage waits for it before
  // it rewrites the pinned buffer that copy reads
  hipEvent_t stage_ev = nullptr;
  bool stage_pending = false;
  // parents with at most scan_mult * K children are scanned (one work item
  // per child), wider ones use their hash table (K items): scanning a child
  // is a coalesced 4-B read, a hashed proposal a random 64-B bucket
  uint32_t scan_mult = 2;
  uint32_t wgs_req = 4096;    // workgroups per request (clamped to residency:
                              // a lone request gets every CU)
  uint32_t share_min = 4096;  // work items from which a step is shared
  // a streamed search publishes each request's first head_rows rows before
  // it packs the rest of any (0: whole requests); helper 1 of the request
  // copies the rest to the device while the leader searches
  uint32_t head_rows = 3;
  // test knob: helpers never claim their slices, so the leader takes every
  // one over after its grace period
  uint32_t no_claims = 0;
  // a streamed search's bounded wait for a request's ready word (ticks),
  // and a delay before the host packs (microseconds): test knobs that
  // make requests come back not ready, to be searched again staged
  uint64_t ready_ticks = kReadyTicks;
  uint32_t pack_delay_us = 0;
  int max_resident = 0;
  // this device's no-allocation scratch (looked up at ft_create), or null
  // with the reason in scratch_err
  uint8_t* d_scratch = nullptr;
  std::string scratch_err;
  // ring of (start, end) event pairs, one pair per launch
  static constexpr size_t kRing = 1024;
  std::vector<hipEvent_t> ring;
  uint64_t launches = 0;
};

static void free_staging(ft_ctx* c) {
  if (c->d_out) (void)hipFree(c->d_out);
  if (c->d_stage) (void)hipFree(c->d_stage);
  if (c->h_out) (void)hipHostFree(c->h_out);
  if (c->h_stage) (void)hipHostFree(c->h_stage);
  if (c->h_ready) (void)hipHostFree(c->h_ready);
  c->d_out = c->d_stage = c->h_out = c->h_stage = c->m_stage = c->m_out = nullptr;
  c->h_ready = c->m_ready = nullptr;
  c->max_staged = 0;
}

static void release_workspace(ft_ctx* c) {
  if (c->d_ws) (void)hipFree(c->d_ws);
  c->d_ws = nullptr;
  free_staging(c);
  c->reserved = false;
}

// Pinned, coherent host memory mapped for the device: *host for the host,
// *dev for kernels.
static int alloc_mapped(void** host, void** dev, size_t bytes, const char* what) {
  hipError_t e = hipHostMalloc(host, bytes, hipHostMallocMapped | hipHostMallocCoherent);
  if (e != hipSuccess) return *host = nullptr, hip_fail(e, what);
  if ((e = hipHostGetDevicePointer(dev, *host, 0)) != hipSuccess) return hip_fail(e, what);
  return FT_OK;
}

// (Re)allocates the staging and output buffers for n requests.
static int alloc_staging(ft_ctx* c, size_t n) {
  free_staging(c);
  c->stage_cap = align_up(n * sizeof(DevReq), 256) + n * c->per_req;
  hipError_t e;
  if ((e = hipMalloc(&c->d_out, c->out_slot_max * n)) != hipSuccess)
    return hip_fail(e, "hipMalloc(output)");
  if ((e = hipMalloc(&c->d_stage, c->stage_cap)) != hipSuccess)
    return hip_fail(e, "hipMalloc(stage)");
  void *h = nullptr, *m = nullptr;
  if (int rc = alloc_mapped(&h, &m, c->out_slot_max * n, "hipHostMalloc(output)")) return rc;
  c->h_out = (uint8_t*)h;
  c->m_out = (uint8_t*)m;
  if (int rc = alloc_mapped(&h, &m, c->stage_cap, "hipHostMalloc(stage)")) return rc;
  c->h_stage = (uint8_t*)h;
  c->m_stage = (uint8_t*)m;
  if (int rc = alloc_mapped(&h, &m, 8 * n, "hipHostMalloc(ready words)")) return rc;
  c->h_ready = (unsigned long long*)h;
  c->m_ready = (unsigned long long*)m;
  std::memset(c->h_ready, 0, 8 * n);
  c->max_staged = n;
  return FT_OK;
}

// Cuckoo insertion of (token word, child) into a node's table: place it in
// a free slot of one of its two buckets, else displace a random occupant of
// one of them and re-insert that one.  False after `max_kicks` displacements
// (the table is then unusable and the node falls back to binary search).
static bool cuckoo_insert(WideBucket* tb, uint32_t lg, uint32_t tokw,
                          uint32_t child, uint64_t* rng) {
  constexpr int max_kicks = 4096;
  for (int kick = 0; kick < max_kicks; ++kick) {
    const uint32_t tok = tokw & kTokMask;
    const uint32_t b1 = cuckoo_h1(tok, lg), b2 = cuckoo_h2(tok, lg);
    for (const uint32_t b : {b1, b2})
      for (uint32_t sl = 0; sl < kBucketSlots; ++sl)
        if (tb[b].child[sl] == 0) {
          tb[b].tok[sl] = tokw;
          tb[b].child[sl] = child;
          return true;
        }
    uint64_t x = *rng;  // xorshift64
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *rng = x;
    const uint32_t b = (x & 1) ? b1 : b2;
    const uint32_t sl = (uint32_t)((x >> 1) % kBucketSlots);
    std::swap(tokw, tb[b].tok[sl]);
    std::swap(child, tb[b].child[sl]);
  }
  return false;
}

// Moves every entry that sits in its second bucket while its first bucket
// has a free slot into that slot, so that a lookup may stop at a first
// bucket with a free slot.  Moves only fill first buckets, so it ends.
static void cuckoo_settle(WideBucket* tb, uint32_t lg) {
  const uint64_t nb = 1ull << lg;
  bool moved = true;
  while (moved) {
    moved = false;
    for (uint64_t b = 0; b < nb; ++b)
      for (uint32_t sl = 0; sl < kBucketSlots; ++sl) {
        if (tb[b].child[sl] == 0) continue;
        const uint32_t tok = tb[b].tok[sl] & kTokMask;
        const uint32_t b1 = cuckoo_h1(tok, lg);
        if (b1 == b) continue;
        for (uint32_t s2 = 0; s2 < kBucketSlots; ++s2)
          if (tb[b1].child[s2] == 0) {
            tb[b1].tok[s2] = tb[b].tok[sl];
            tb[b1].child[s2] = tb[b].child[sl];
            tb[b].tok[sl] = kSlotEmptyTok;
            tb[b].child[sl] = 0;
            moved = true;
            break;
          }
      }
  }
}

// Checks every structural fact the kernel relies on before any of the image
// reaches the device, so that a corrupt or hand-made blob is an FT_E_IMAGE
// and never an out-of-bounds read on the GPU:
//  * BFS child ranges: rec[0] starts the root's children at id 1, ranges are
//    non-decreasing and end at the sentinel rec[N].child_begin == N, and a
//    node's children have larger ids than the node (so parent walks end);
//  * every child c of v has parent[c] == v, an edge of >= 1 token with
//    string depth depth(v) + edge length (a link node exactly when the edge
//    has >= 2 tokens), siblings in strictly ascending first-token order and
//    tokens below 2^31 - 1;
//  * a link node's edge lies inside tail[] and starts with its first token;
//  * the terminal flags count num_keys.
// Parent ranges are split over host threads (each child is checked by the
// thread that owns its parent).
static int validate_image_host(const uint8_t* image, const ft_image_header& h) {
  const uint64_t N = h.num_nodes;
  const ft_node_rec* R = (const ft_node_rec*)(image + h.recs_offset);
  const uint32_t* P = (const uint32_t*)(image + h.parent_offset);
  const uint32_t* Tl = (const uint32_t*)(image + h.tail_offset);
  if (h.parent_offset % 4 || h.tail_offset % 4)
    return fail(FT_E_IMAGE, "ft_create: misaligned parent or tail array");
  if (R[0].child_begin != 1)
    return fail(FT_E_IMAGE, "ft_create: the root's children must start at id 1");
  if (R[N].child_begin != N)
    return fail(FT_E_IMAGE, "ft_create: sentinel child_begin must equal num_nodes");
  if ((R[0].meta & (FT_META_DEPTH_MASK | FT_META_LINK)) != 0)
    return fail(FT_E_IMAGE, "ft_create: the root must have depth 0 and no edge");
  const int T = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::vector<uint64_t> keys(T, 0);
  // first bad node per thread (N: none) and what was wrong with it
  std::vector<uint64_t> bad(T, N);
  std::vector<int> why(T, 0);
  {
    std::vector<std::thread> th;
    for (int w = 0; w < T; ++w)
      th.emplace_back([&, w]() {
        const uint64_t b = N * w / T, e = N * (w + 1) / T;
        uint64_t k = 0;
        for (uint64_t v = b; v < e; ++v) {
          const uint32_t c0 = R[v].child_begin, c1 = R[v + 1].child_begin;
          if (c1 < c0 || c1 > N || (c1 > c0 && c0 <= v)) {
            bad[w] = v, why[w] = 1;
            return;
          }
          if (R[v].meta & FT_META_TERMINAL) ++k;
          const uint32_t sd = R[v].meta & FT_META_DEPTH_MASK;
          for (uint32_t c = c0; c < c1; ++c) {
            const uint32_t m = R[c].meta;
            const uint32_t el = (m >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
            if (P[c] != v || el == 0 || (m & FT_META_DEPTH_MASK) != sd + el ||
                ((m & FT_META_LINK) != 0) != (el >= 2) ||
                (c > c0 && R[c].first_tok <= R[c - 1].first_tok) ||
                R[c].first_tok >= kSlotEmptyTok) {
              bad[w] = c, why[w] = 2;
              return;
            }
            if ((m & FT_META_LINK) &&
                ((uint64_t)R[c].tail_off + el > h.tail_len ||
                 Tl[R[c].tail_off] != R[c].first_tok)) {
              bad[w] = c, why[w] = 3;
              return;
            }
          }
        }
        keys[w] = k;
      });
    for (auto& x : th) x.join();
  }
  static const char* const kWhy[] = {"", "child range is not breadth first",
                                     "is inconsistent with its parent (parent, edge, "
                                     "depth, sibling order or token id >= 2^31 - 1)",
                                     "has an edge outside tail[]"};
  uint64_t nkeys = 0;
  for (int w = 0; w < T; ++w) {
    if (bad[w] != N)
      return fail(FT_E_IMAGE, "ft_create: node " + std::to_string(bad[w]) + " " +
                                  kWhy[why[w]]);
    nkeys += keys[w];
  }
  if (nkeys != h.num_keys)
    return fail(FT_E_IMAGE, "ft_create: num_keys does not match the terminal flags");
  return FT_OK;
}

// Per node, its first edge token with kSlotSel when the node can close a
// key one token below its parent (terminal, one-token edge): what a scan
// of a parent's children needs, 4 bytes a child.  Uploaded to the device.
static int build_labels(ft_ctx* c, const uint8_t* image) {
  const uint64_t N = c->hdr.num_nodes;
  const ft_node_rec* R = (const ft_node_rec*)(image + c->hdr.recs_offset);
  std::unique_ptr<uint32_t[]> lab(new (std::nothrow) uint32_t[N]);
  if (!lab) return fail(FT_E_NOMEM, "labels: host memory");
  const int T = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::atomic<uint64_t> bad{0};
  {
    std::vector<std::thread> th;
    for (int w = 0; w < T; ++w)
      th.emplace_back([&, w]() {
        const uint64_t b = N * w / T, e = N * (w + 1) / T;
        uint64_t nbad = 0;
        for (uint64_t n = b; n < e; ++n) {
          const uint32_t meta = R[n].meta;
          const uint32_t elen = (meta >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
          const bool sel = (meta & FT_META_TERMINAL) && elen == 1;
          if (n > 0 && R[n].first_tok >= kSlotEmptyTok) ++nbad;
          lab[n] = n == 0 ? kSlotEmptyTok : (R[n].first_tok | (sel ? kSlotSel : 0u));
        }
        bad += nbad;
      });
    for (auto& x : th) x.join();
  }
  if (bad) return fail(FT_E_IMAGE, "ft_create: token ids must be below 2^31 - 1");
  hipError_t e;
  if ((e = hipMalloc(&c->d_labels, N * sizeof(uint32_t))) != hipSuccess)
    return hip_fail(e, "hipMalloc(labels)");
  if ((e = hipMemcpy(c->d_labels, lab.get(), N * sizeof(uint32_t),
                     hipMemcpyHostToDevice)) != hipSuccess)
    return hip_fail(e, "hipMemcpy(labels)");
  return FT_OK;
}

// Builds the LOUDS directory of the trie's shape (tbs_kernel.h LoudsDir)
// from the records' child ranges and uploads it: zero v at bit
// child_begin(v + 1) + v - 1, every other bit of the 2N - 1 a one; zeros
// before every 512-bit block; the block of every kLoudsSel-th zero.
static int build_louds(ft_ctx* c, const uint8_t* image) {
  const uint64_t N = c->hdr.num_nodes;
  const ft_node_rec* R = (const ft_node_rec*)(image + c->hdr.recs_offset);
  const uint64_t nbits = 2 * N - 1;
  const uint64_t wpb = kLoudsBlockBits / 64;
  const uint64_t nblocks = (nbits + kLoudsBlockBits - 1) / kLoudsBlockBits;
  const uint64_t nwords = nblocks * wpb;
  const uint64_t nsamp = (N - 1) / kLoudsSel + 2;
  std::unique_ptr<uint64_t[]> W(new (std::nothrow) uint64_t[nwords]);
  std::unique_ptr<uint32_t[]> Z(new (std::nothrow) uint32_t[nblocks + 1]);
  std::unique_ptr<uint32_t[]> S(new (std::nothrow) uint32_t[nsamp]);
  if (!W || !Z || !S) return fail(FT_E_NOMEM, "louds directory: host memory");
  const int T = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  auto zpos = [&](uint64_t v) { return (uint64_t)R[v + 1].child_begin + v - 1; };
  auto par = [&](uint64_t n, auto&& body) {
    std::vector<std::thread> th;
    for (int w = 0; w < T; ++w)
      th.emplace_back([&, w]() { body(n * w / T, n * (w + 1) / T); });
    for (auto& x : th) x.join();
  };
  // words: each thread owns a range of words and clears the zeros of the
  // nodes whose zero falls in it (zpos is increasing in v: binary search)
  par(nwords, [&](uint64_t w0, uint64_t w1) {
    for (uint64_t w = w0; w < w1; ++w) W[w] = ~0ull;
    uint64_t lo = 0, hi = N;  // first v with zpos(v) >= 64 * w0
    while (lo < hi) {
      const uint64_t mid = (lo + hi) / 2;
      if (zpos(mid) < 64 * w0) lo = mid + 1; else hi = mid;
    }
    for (uint64_t v = lo; v < N; ++v) {
      const uint64_t p = zpos(v);
      if (p >= 64 * w1) break;
      W[p >> 6] &= ~(1ull << (p & 63));
    }
  });
  // zeros per block, then the exclusive prefix
  par(nblocks, [&](uint64_t b0, uint64_t b1) {
    for (uint64_t b = b0; b < b1; ++b) {
      uint32_t z = 0;
      for (uint64_t j = 0; j < wpb; ++j) {
        const uint64_t base = (b * wpb + j) * 64;
        uint64_t x = ~W[b * wpb + j];
        if (base + 64 > nbits) x &= base >= nbits ? 0ull : ((1ull << (nbits - base)) - 1ull);
        z += (uint32_t)__builtin_popcountll(x);
      }
      Z[b + 1] = z;
    }
  });
  Z[0] = 0;
  for (uint64_t b = 1; b <= nblocks; ++b) Z[b] += Z[b - 1];
  if (Z[nblocks] != N) return fail(FT_E_IMAGE, "louds directory: zero count mismatch");
  for (uint64_t k = 0; k < nsamp; ++k)
    S[k] = (uint32_t)(zpos(std::min<uint64_t>(k * kLoudsSel, N - 1)) / kLoudsBlockBits);
  hipError_t e;
  if ((e = hipMalloc(&c->d_louds_words, nwords * 8)) != hipSuccess)
    return hip_fail(e, "hipMalloc(louds words)");
  if ((e = hipMalloc(&c->d_louds_z, (nblocks + 1) * 4)) != hipSuccess)
    return hip_fail(e, "hipMalloc(louds z)");
  if ((e = hipMalloc(&c->d_louds_s, nsamp * 4)) != hipSuccess)
    return hip_fail(e, "hipMalloc(louds samples)");
  if ((e = hipMemcpy(c->d_louds_words, W.get(), nwords * 8, hipMemcpyHostToDevice)) != hipSuccess ||
      (e = hipMemcpy(c->d_louds_z, Z.get(), (nblocks + 1) * 4, hipMemcpyHostToDevice)) != hipSuccess ||
      (e = hipMemcpy(c->d_louds_s, S.get(), nsamp * 4, hipMemcpyHostToDevice)) != hipSuccess)
    return hip_fail(e, "hipMemcpy(louds)");
  c->louds_bytes = nwords * 8 + (nblocks + 1) * 4 + nsamp * 4;
  return FT_OK;
}

// Builds the wide-node index on the host (parallel) and uploads it.
static int build_wide_index(ft_ctx* c, const uint8_t* image) {
  const char* env = std::getenv("FT_WIDE_MIN");
  long wmin = env ? std::strtol(env, nullptr, 10) : 512;
  if (wmin <= 0) return FT_OK;  // disabled
  const uint64_t N = c->hdr.num_nodes;
  const ft_node_rec* R = (const ft_node_rec*)(image + c->hdr.recs_offset);
  const int T = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::vector<std::vector<uint32_t>> found(T);
  {
    std::vector<std::thread> th;
    for (int w = 0; w < T; ++w)
      th.emplace_back([&, w]() {
        const uint64_t b = N * w / T, e = N * (w + 1) / T;
        for (uint64_t n = b; n < e; ++n)
          if (R[n + 1].child_begin - R[n].child_begin >= (uint32_t)wmin)
            found[w].push_back((uint32_t)n);
      });
    for (auto& x : th) x.join();
  }
  std::vector<uint32_t> nodes;
  for (auto& f : found) nodes.insert(nodes.end(), f.begin(), f.end());
  if (nodes.empty()) return FT_OK;
  std::vector<WideDir> ent(nodes.size());
  uint64_t buckets = 0;
  for (size_t i = 0; i < nodes.size(); ++i) {
    const uint32_t n = nodes[i];
    const uint64_t deg = R[n + 1].child_begin - R[n].child_begin;
    uint32_t lg = 1;
    while (((uint64_t)kBucketSlots << lg) < 2 * deg) ++lg;  // load <= 1/2
    ent[i] = WideDir{n, lg, (uint32_t)buckets, 0};
    buckets += 1ull << lg;
    if (buckets >= 0xFFFFFFF0ull) return fail(FT_E_IMAGE, "wide-node index too large");
  }
  // uninitialised: every table is cleared by the thread that fills it
  std::unique_ptr<WideBucket[]> tab(new (std::nothrow) WideBucket[buckets]);
  if (!tab) return fail(FT_E_NOMEM, "wide-node index: host memory");
  std::vector<uint8_t> failed(ent.size(), 0);
  {
    std::atomic<size_t> next{0};
    std::vector<std::thread> th;
    for (int w = 0; w < T; ++w)
      th.emplace_back([&]() {
        for (;;) {
          const size_t i = next.fetch_add(1);
          if (i >= ent.size()) break;
          const WideDir& e = ent[i];
          WideBucket* tb = tab.get() + e.bucket_off;
          for (uint64_t b = 0; b < (1ull << e.log2nb); ++b)
            for (uint32_t sl = 0; sl < kBucketSlots; ++sl) {
              tb[b].tok[sl] = kSlotEmptyTok;
              tb[b].child[sl] = 0;
            }
          uint64_t rng = 0x9E3779B97F4A7C15ull ^ ((uint64_t)e.node << 1);
          for (uint32_t ch = R[e.node].child_begin; ch < R[e.node + 1].child_begin; ++ch) {
            const uint32_t meta = R[ch].meta;
            const uint32_t elen = (meta >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
            const bool sel = (meta & FT_META_TERMINAL) && elen == 1;
            const uint32_t tokw = (R[ch].first_tok & kTokMask) | (sel ? kSlotSel : 0u);
            // tokens that do not fit the slot word: no table for this node
            if (R[ch].first_tok >= kSlotEmptyTok ||
                !cuckoo_insert(tb, e.log2nb, tokw, ch, &rng)) {
              failed[i] = 1;
              break;
            }
          }
          if (!failed[i]) cuckoo_settle(tb, e.log2nb);
        }
      });
    for (auto& x : th) x.join();
  }
  // fingerprint words (every bucket, tables that failed included: they are
  // cleared and never read), and the filter flag of small tables
  std::unique_ptr<uint64_t[]> fpw(new (std::nothrow) uint64_t[buckets]);
  if (!fpw) return fail(FT_E_NOMEM, "wide-node index: host memory");
  {
    std::vector<std::thread> th;
    for (int w = 0; w < T; ++w)
      th.emplace_back([&, w]() {
        const uint64_t b0 = buckets * w / T, b1 = buckets * (w + 1) / T;
        for (uint64_t b = b0; b < b1; ++b) {
          uint64_t f = 0;
          for (uint32_t sl = 0; sl < kBucketSlots; ++sl) {
            const uint32_t tw = tab[b].tok[sl];
            if (tw != kSlotEmptyTok) f |= (uint64_t)wide_fp(tw & kTokMask) << (8 * sl);
          }
          fpw[b] = f;
        }
      });
    for (auto& x : th) x.join();
  }
  uint32_t fp_max = kFpMaxLog2;
  if (const char* fe = std::getenv("FT_FP_MAX_LOG2")) {
    const long v = std::strtol(fe, nullptr, 10);
    if (v >= 0 && v <= 32) fp_max = (uint32_t)v;
  }
  for (auto& e : ent) e.flags = e.log2nb <= fp_max ? kWideFiltered : 0u;
  uint64_t n_ok = 0;
  for (size_t i = 0; i < ent.size(); ++i) n_ok += failed[i] ? 0 : 1;
  // directory groups, load <= 1/2
  uint32_t dlg = 0;
  while (((uint64_t)kDirSlots << dlg) < 2 * std::max<uint64_t>(n_ok, 1)) ++dlg;
  WideDirGroup empty_group;
  for (uint32_t k = 0; k < kDirSlots; ++k) {
    empty_group.node[k] = kEmpty;
    empty_group.bucket_off[k] = empty_group.lgf[k] = empty_group.pad[k] = 0;
  }
  std::vector<WideDirGroup> dir(1ull << dlg, empty_group);
  for (size_t i = 0; i < ent.size(); ++i) {
    if (failed[i]) continue;  // searched by binary search instead
    uint32_t g = fib_slot(ent[i].node, dlg);
    for (;;) {
      uint32_t k = 0;
      while (k < kDirSlots && dir[g].node[k] != kEmpty) ++k;
      if (k < kDirSlots) {
        dir[g].node[k] = ent[i].node;
        dir[g].bucket_off[k] = ent[i].bucket_off;
        dir[g].lgf[k] = ent[i].log2nb | (ent[i].flags << 8);
        break;
      }
      g = (g + 1) & ((1u << dlg) - 1);
    }
  }
  hipError_t e;
  if ((e = hipMalloc(&c->d_wdir, dir.size() * sizeof(WideDirGroup))) != hipSuccess)
    return hip_fail(e, "hipMalloc(wide dir)");
  if ((e = hipMalloc(&c->d_wtab, buckets * sizeof(WideBucket))) != hipSuccess)
    return hip_fail(e, "hipMalloc(wide tables)");
  if ((e = hipMalloc(&c->d_wfp, buckets * sizeof(uint64_t))) != hipSuccess)
    return hip_fail(e, "hipMalloc(wide fingerprints)");
  if ((e = hipMemcpy(c->d_wdir, dir.data(), dir.size() * sizeof(WideDirGroup),
                     hipMemcpyHostToDevice)) != hipSuccess)
    return hip_fail(e, "hipMemcpy(wide dir)");
  if ((e = hipMemcpy(c->d_wtab, tab.get(), buckets * sizeof(WideBucket),
                     hipMemcpyHostToDevice)) != hipSuccess)
    return hip_fail(e, "hipMemcpy(wide tables)");
  if ((e = hipMemcpy(c->d_wfp, fpw.get(), buckets * sizeof(uint64_t),
                     hipMemcpyHostToDevice)) != hipSuccess)
    return hip_fail(e, "hipMemcpy(wide fingerprints)");
  c->wdir_log2 = dlg;
  c->wide_min = (uint32_t)wmin;
  c->wide_nodes = n_ok;
  c->wide_buckets = buckets;
  c->wide_failed = ent.size() - n_ok;
  return FT_OK;
}

// The root directory (RootEnt): one entry per token below the root's
// largest child token + 1, filled on the device by parent_entry of each
// child at step 1.  None when the root has no child, a child token is
// kRootDirMax or more, or FT_ROOT_DIR=0.
static int build_root_dir(ft_ctx* c, const uint8_t* image) {
  if (c->d_louds_words) return FT_OK;  // (the records' child ranges only)
  if (const char* s = std::getenv("FT_ROOT_DIR")) {
    if (std::strcmp(s, "0") == 0) return FT_OK;
    if (std::strcmp(s, "force") == 0) c->root_force = 1;
  }
  const ft_node_rec* R = (const ft_node_rec*)(image + c->hdr.recs_offset);
  const uint32_t c0 = R[0].child_begin, deg = R[1].child_begin - c0;
  if (deg == 0) return FT_OK;
  uint32_t top = 0;
  for (uint32_t i = 0; i < deg; ++i) top = std::max(top, R[c0 + i].first_tok);
  if (top >= kRootDirMax) return FT_OK;
  const uint32_t n = top + 1;
  hipError_t e;
  if ((e = hipMalloc(&c->d_root_dir, (size_t)n * sizeof(RootEnt))) != hipSuccess)
    return hip_fail(e, "hipMalloc(root directory)");
  if ((e = hipMemsetAsync(c->d_root_dir, 0, (size_t)n * sizeof(RootEnt), c->stream)) !=
      hipSuccess)
    return hip_fail(e, "hipMemsetAsync(root directory)");
  KArgs a{};
  a.recs = (const ft_node_rec*)(c->d_image + c->hdr.recs_offset);
  a.parent = (const uint32_t*)(c->d_image + c->hdr.parent_offset);
  a.tail = (const uint32_t*)(c->d_image + c->hdr.tail_offset);
  a.wdir = c->d_wdir;
  a.wtab = c->d_wtab;
  a.wfp = c->d_wfp;
  a.labels = c->d_labels;
  a.wdir_log2 = c->wdir_log2;
  a.wide_min = c->wide_min;
  if ((e = launch_root_dir(a, c->d_root_dir, n, c0, deg, c->stream)) != hipSuccess)
    return hip_fail(e, "launch(root directory)");
  if ((e = hipStreamSynchronize(c->stream)) != hipSuccess)
    return hip_fail(e, "hipStreamSynchronize(root directory)");
  c->root_n = n;
  return FT_OK;
}

#ifndef FT_BUILD_ID
#define FT_BUILD_ID "unknown"
#endif
// The build id (a hash of the sources the library was built from), behind
// a tag the build recipe finds in the binary.
static const char g_build_id[] = "FT_BUILD_ID=" FT_BUILD_ID;

extern "C" {

const char* ft_build_id(void) { return g_build_id + 12; }

const char* ft_last_error(void) { return g_err.c_str(); }

const char* ft_strerror(int code) {
  switch (code) {
    case FT_OK: return "ok";
    case FT_E_ARG: return "invalid argument";
    case FT_E_NOMEM: return "out of memory";
    case FT_E_HIP: return "HIP runtime error";
    case FT_E_LIMIT: return "request exceeds the reserved workspace";
    case FT_E_STATE: return "call sequence error (init_tbs_gpu / stage missing)";
    case FT_E_INPUT: return "malformed request";
    case FT_E_IMAGE: return "malformed trie image";
    case FT_E_DEVICE: return "no usable gfx950 device";
    case FT_E_KERNEL: return "search kernel reported an internal error";
    default: return "unknown error";
  }
}

int ft_create(const void* image, size_t image_bytes, int device,
              ft_ctx** out) {
  if (!image || !out || image_bytes < sizeof(ft_image_header))
    return fail(FT_E_ARG, "ft_create: null image or too small");
  *out = nullptr;
  ft_image_header h;
  std::memcpy(&h, image, sizeof(h));
  if (std::memcmp(h.magic, FT_IMAGE_MAGIC, 7) != 0)
    return fail(FT_E_IMAGE, "ft_create: bad image magic");
  if (h.total_bytes != image_bytes || h.num_nodes == 0 ||
      h.num_nodes >= 0xFFFFFFFFull ||
      h.recs_offset + (h.num_nodes + 1) * sizeof(ft_node_rec) > image_bytes ||
      h.parent_offset + h.num_nodes * 4 > image_bytes ||
      h.tail_offset + h.tail_len * 4 > image_bytes || h.recs_offset % 16)
    return fail(FT_E_IMAGE, "ft_create: inconsistent image header");
  // the whole image is checked before any device call
  if (int rc = validate_image_host((const uint8_t*)image, h)) return rc;

  int ndev = 0;
  hipError_t e = hipGetDeviceCount(&ndev);
  if (e != hipSuccess || ndev <= device || device < 0)
    return fail(FT_E_DEVICE, "ft_create: no HIP device " + std::to_string(device));
  if ((e = hipSetDevice(device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
  hipDeviceProp_t prop;
  if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess)
    return hip_fail(e, "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(FT_E_DEVICE, std::string("ft_create: device is ") +
                                 prop.gcnArchName + ", this build targets gfx950");

  auto* c = new ft_ctx();
  c->device = device;
  c->hdr = h;
  c->num_cus = prop.multiProcessorCount;
  c->lds_per_block = (int)prop.sharedMemPerBlock;
  int wc = 0;
  (void)hipDeviceGetAttribute(&wc, hipDeviceAttributeWallClockRate, device);
  c->wall_khz = wc;
  std::snprintf(c->name, sizeof(c->name), "%s", prop.gcnArchName);
  {
    // the no-allocation scratch of this device (the device is current)
    void* sp = nullptr;
    const hipError_t se = scratch_address(device, &sp);
    if (se == hipSuccess) c->d_scratch = (uint8_t*)sp;
    else c->scratch_err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(se);
  }
  if ((e = hipMalloc(&c->d_image, image_bytes)) != hipSuccess) {
    delete c;
    return hip_fail(e, "hipMalloc(image)");
  }
  if ((e = hipMemcpy(c->d_image, image, image_bytes, hipMemcpyHostToDevice)) !=
      hipSuccess) {
    (void)hipFree(c->d_image);
    delete c;
    return hip_fail(e, "hipMemcpy(image)");
  }
  if ((e = hipStreamCreate(&c->stream)) != hipSuccess) {
    (void)hipFree(c->d_image);
    delete c;
    return hip_fail(e, "hipStreamCreate");
  }
  c->ring.assign(2 * ft_ctx::kRing, nullptr);
  for (auto& ev : c->ring) (void)hipEventCreate(&ev);
  (void)hipEventCreateWithFlags(&c->stage_ev, hipEventDisableTiming);
  if (int rc = build_labels(c, (const uint8_t*)image)) {
    ft_destroy(c);
    return rc;
  }
  if (int rc = build_wide_index(c, (const uint8_t*)image)) {
    ft_destroy(c);
    return rc;
  }
  if (const char* ci = std::getenv("FT_CHILD_INDEX")) {
    if (std::strcmp(ci, "louds") == 0) {
      // The LOUDS child-index kernel faulted the GPU once (an out-of-range
      // access on tiny tries) and the cause is not found: the path is off
      // until it is.  build_louds and the kernel instantiation stay.
      ft_destroy(c);
      return fail(FT_E_ARG, "ft_create: FT_CHILD_INDEX=louds is switched off (its kernel "
                            "faulted once and the cause is not found); use the node records");
    }
  }
  if (int rc = build_root_dir(c, (const uint8_t*)image)) {
    ft_destroy(c);
    return rc;
  }
  c->max_resident = tbs_max_resident_blocks(c->num_cus);
  if (c->max_resident <= 0) {
    ft_destroy(c);
    return fail(FT_E_DEVICE, "ft_create: the search kernel cannot be resident");
  }
  if (const char* s = std::getenv("FT_WGS")) {
    const long v = std::strtol(s, nullptr, 10);
    if (v >= 1 && v <= 4096) c->wgs_req = (uint32_t)v;
  }
  if (const char* s = std::getenv("FT_SHARE_MIN")) {
    const long v = std::strtol(s, nullptr, 10);
    if (v >= 0) c->share_min = (uint32_t)v;
  }
  if (const char* s = std::getenv("FT_TEST_NO_CLAIMS")) c->no_claims = std::atoi(s) ? 1u : 0u;
  if (const char* s = std::getenv("FT_SCAN_MULT")) {
    const long v = std::strtol(s, nullptr, 10);
    if (v >= 0 && v < 1000000) c->scan_mult = (uint32_t)v;
  }
  if (const char* s = std::getenv("FT_HEAD_ROWS")) {
    const long v = std::strtol(s, nullptr, 10);
    if (v >= 0 && v < 1000000) c->head_rows = (uint32_t)v;
  }
  if (const char* s = std::getenv("FT_READY_TICKS")) {
    const long long v = std::strtoll(s, nullptr, 10);
    if (v >= 0 && (unsigned long long)v <= kReadyTicks) c->ready_ticks = (uint64_t)v;
  }
  if (const char* s = std::getenv("FT_PACK_DELAY_US")) {
    const long v = std::strtol(s, nullptr, 10);
    if (v >= 0 && v <= 1000000) c->pack_delay_us = (uint32_t)v;
  }
  *out = c;
  return FT_OK;
}

// Launch epochs tag the control words a request's workgroups sync through.
// They come from one process-wide counter, so no launch of any context ever
// reuses one: a workspace may sit on memory another context freed, and a
// stale control word must never look like a step posted by this launch.
static std::atomic<uint32_t> g_launch_epoch{0};

// Byte layout of one request's workspace slot for beams of at most B
// hypotheses, rows of at most K proposals and `hist` history records; the
// candidate lists are sized so that no push can overflow (B * K pushes into
// `next`, B * K + B into `selected`).  Returns the slot stride.
static uint64_t ws_layout(uint64_t B, uint64_t K, uint64_t hist, uint32_t slots,
                          WsLayout* out) {
  const uint64_t BK = B * K;
  WsLayout L{};
  uint64_t off = 0;
  L.cur0 = off; off = align_up(off + B * sizeof(CurRec), 256);
  L.cur1 = off; off = align_up(off + B * sizeof(CurRec), 256);
  L.nextc = off; off = align_up(off + BK * sizeof(NextRec), 256);
  L.selA = off; off = align_up(off + (BK + B) * sizeof(SelRec), 256);
  L.selB = off; off = align_up(off + (BK + B) * sizeof(SelRec), 256);
  L.rank = off; off = align_up(off + B * 4, 256);
  L.hist = off; off = align_up(off + hist * sizeof(HistRec), 256);
  L.ctl = off; off = align_up(off + sizeof(Ctl), 256);
  L.par_c0 = off; off = align_up(off + B * 4, 256);
  L.par_aux = off; off = align_up(off + B * 4, 256);
  L.par_node = off; off = align_up(off + B * 4, 256);
  L.par_mode = off; off = align_up(off + B * 4, 256);
  L.par_woff = off; off = align_up(off + (B + 1) * 4, 256);
  L.claims = off; off = align_up(off + (uint64_t)slots * 8, 256);
  L.dones = off; off = align_up(off + (uint64_t)slots * 16, 256);
  L.claim_slots = slots;
  L.next_cap = (uint32_t)BK;
  L.sel_cap = (uint32_t)(BK + B);
  L.hist_cap = (uint32_t)hist;
  L.cur_cap = (uint32_t)B;
  *out = L;
  return off;
}

int ft_reserve(ft_ctx* c, size_t max_batch, size_t max_topk, size_t max_steps,
               size_t max_out_beams, size_t max_out_tokens,
               size_t max_inter_beams) {
  if (!c) return fail(FT_E_ARG, "ft_reserve: null context");
  if (max_batch == 0 || max_topk == 0 || max_steps == 0 ||
      max_out_beams == 0 || max_out_tokens == 0 || max_inter_beams == 0)
    return fail(FT_E_ARG, "ft_reserve: every limit must be positive");
  if (max_topk > kMaxTopk)
    return fail(FT_E_LIMIT, "ft_reserve: max_num_topk " +
                                std::to_string(max_topk) + " > " +
                                std::to_string(kMaxTopk));
  if (max_out_beams > kMaxBeams)
    return fail(FT_E_LIMIT, "ft_reserve: max_num_out_beams > 65535");
  if (max_steps > 16383)
    return fail(FT_E_LIMIT, "ft_reserve: max_num_outpos > 16383");
  if (max_inter_beams >= 0xFFFFFFF0ull)
    return fail(FT_E_LIMIT, "ft_reserve: max_num_inter_beams too large");
  (void)hipSetDevice(c->device);
  // nothing queued may still read or write the buffers freed here
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  c->stage_pending = false;
  release_workspace(c);
  const uint64_t B = max_out_beams, K = max_topk;
  if (B * K + B >= 0xFFFFFFF0ull) return fail(FT_E_LIMIT, "ft_reserve: beams * topk too large");
  c->ws_stride = ws_layout(B, K, max_inter_beams, (uint32_t)c->max_resident, &c->lay);
  c->out_slot_max = align_up(step_stats_offset((uint32_t)B, 0) + 4 * (uint64_t)max_out_tokens +
                                 8ull * kStepStats * max_steps + 8, 256);
  // per request: lnf + beams + sorted rows (token, logp, index) + key bounds
  c->per_req = align_up(8 * (max_steps + 1), 16) + align_up(4 * max_steps, 16) +
               2 * align_up(4 * max_steps * K, 16) + align_up(2 * max_steps * K, 16) +
               align_up(16 * max_steps, 16) + 256;
  hipError_t e;
  if ((e = hipMalloc(&c->d_ws, c->ws_stride * max_batch)) != hipSuccess)
    return release_workspace(c), hip_fail(e, "hipMalloc(workspace)");
  // control blocks start at "nothing posted" (epoch 0 is never used)
  if ((e = hipMemset(c->d_ws, 0, c->ws_stride * max_batch)) != hipSuccess)
    return release_workspace(c), hip_fail(e, "hipMemset(workspace)");
  int rc = alloc_staging(c, max_batch);
  if (rc) return release_workspace(c), rc;
  c->max_batch = max_batch;
  c->max_topk = max_topk;
  c->sort_tmp.assign(max_topk, {0u, 0u});
  c->max_steps = max_steps;
  c->max_out_beams = max_out_beams;
  c->max_out_tokens = max_out_tokens;
  c->max_inter = max_inter_beams;
  c->reserved = true;
  c->staged.clear();
  c->launched_slot.clear();
  c->launched = false;
  return FT_OK;
}

// The order-preserving 64-bit key of a double that the device computes for
// every norm (-0.0 and +0.0 map alike).
static uint64_t host_norm_key(double v) {
  if (v == 0.0) v = 0.0;
  uint64_t b;
  std::memcpy(&b, &v, 8);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

// Limits a staged request must respect (the reserved workspace, or the
// no-allocation scratch).
struct StageLimits {
  uint64_t max_steps, max_topk, max_out_beams, max_out_tokens;
};

// One proposal row: whether it holds NaN or +inf, whether its token ids are
// strictly ascending, and the least and greatest logp above the token
// threshold (+inf / -inf when none is); the row is copied to oid / olp on
// the way.  One branch-free SSE2 pass, four proposals at a time.
struct RowScan {
  bool bad, sorted;
  float lo, hi;
};
static RowScan scan_row_sse2(const uint32_t* rid, const float* rlp, uint32_t K, float thr,
                             uint32_t* oid, float* olp) {
  const __m128 vinf = _mm_set1_ps(INFINITY), vninf = _mm_set1_ps(-INFINITY);
  const __m128 vthr = _mm_set1_ps(thr);
  const __m128i flip = _mm_set1_epi32((int)0x80000000u), ones = _mm_set1_epi32(-1);
  bool bad = false, sorted = true;
  float lo = INFINITY, hi = -INFINITY;
  uint32_t k = 1;
  if (K >= 5) {
    __m128 vlo = vinf, vhi = vninf, vbad = _mm_setzero_ps();
    __m128i vuns = _mm_setzero_si128();
    for (; k + 4 <= K; k += 4) {
      const __m128 x = _mm_loadu_ps(rlp + k);
      _mm_storeu_ps(olp + k, x);
      vbad = _mm_or_ps(vbad, _mm_or_ps(_mm_cmpunord_ps(x, x), _mm_cmpeq_ps(x, vinf)));
      const __m128 keep = _mm_cmpgt_ps(x, vthr);
      vlo = _mm_min_ps(vlo, _mm_or_ps(_mm_and_ps(keep, x), _mm_andnot_ps(keep, vinf)));
      vhi = _mm_max_ps(vhi, _mm_or_ps(_mm_and_ps(keep, x), _mm_andnot_ps(keep, vninf)));
      // unsigned rid[i] > rid[i - 1] as a signed compare of flipped words
      const __m128i ra = _mm_loadu_si128((const __m128i*)(rid + k));
      _mm_storeu_si128((__m128i*)(oid + k), ra);
      const __m128i a = _mm_xor_si128(ra, flip);
      const __m128i b = _mm_xor_si128(_mm_loadu_si128((const __m128i*)(rid + k - 1)), flip);
      vuns = _mm_or_si128(vuns, _mm_xor_si128(_mm_cmpgt_epi32(a, b), ones));
    }
    alignas(16) float l4[4], h4[4];
    alignas(16) uint32_t b4[4], u4[4];
    _mm_store_ps(l4, vlo);
    _mm_store_ps(h4, vhi);
    _mm_store_si128((__m128i*)b4, _mm_castps_si128(vbad));
    _mm_store_si128((__m128i*)u4, vuns);
    for (int j = 0; j < 4; ++j) {
      lo = std::min(lo, l4[j]);
      hi = std::max(hi, h4[j]);
      bad = bad || b4[j] != 0;
      sorted = sorted && u4[j] == 0;
    }
  }
  auto one = [&](uint32_t i) {
    const float x = rlp[i];
    olp[i] = x;
    oid[i] = rid[i];
    bad = bad || std::isnan(x) || x == INFINITY;
    if (x > thr) {
      lo = std::min(lo, x);
      hi = std::max(hi, x);
    }
    if (i > 0 && rid[i] <= rid[i - 1]) sorted = false;
  };
  if (K) one(0);
  for (; k < K; ++k) one(k);
  return RowScan{bad, sorted, lo, hi};
}

// The same scan, eight proposals at a time (AVX2 hosts).
__attribute__((target("avx2"))) static RowScan scan_row_avx2(const uint32_t* rid,
                                                             const float* rlp, uint32_t K,
                                                             float thr, uint32_t* oid,
                                                             float* olp) {
  const __m256 vinf = _mm256_set1_ps(INFINITY), vninf = _mm256_set1_ps(-INFINITY);
  const __m256 vthr = _mm256_set1_ps(thr);
  const __m256i flip = _mm256_set1_epi32((int)0x80000000u), ones = _mm256_set1_epi32(-1);
  bool bad = false, sorted = true;
  float lo = INFINITY, hi = -INFINITY;
  uint32_t k = 1;
  if (K >= 9) {
    __m256 vlo = vinf, vhi = vninf, vbad = _mm256_setzero_ps();
    __m256i vuns = _mm256_setzero_si256();
    for (; k + 8 <= K; k += 8) {
      const __m256 x = _mm256_loadu_ps(rlp + k);
      _mm256_storeu_ps(olp + k, x);
      vbad = _mm256_or_ps(vbad, _mm256_or_ps(_mm256_cmp_ps(x, x, _CMP_UNORD_Q),
                                             _mm256_cmp_ps(x, vinf, _CMP_EQ_OQ)));
      const __m256 keep = _mm256_cmp_ps(x, vthr, _CMP_GT_OQ);
      vlo = _mm256_min_ps(vlo, _mm256_blendv_ps(vinf, x, keep));
      vhi = _mm256_max_ps(vhi, _mm256_blendv_ps(vninf, x, keep));
      // unsigned rid[i] > rid[i - 1] as a signed compare of flipped words
      const __m256i ra = _mm256_loadu_si256((const __m256i*)(rid + k));
      _mm256_storeu_si256((__m256i*)(oid + k), ra);
      const __m256i a = _mm256_xor_si256(ra, flip);
      const __m256i b = _mm256_xor_si256(_mm256_loadu_si256((const __m256i*)(rid + k - 1)), flip);
      vuns = _mm256_or_si256(vuns, _mm256_xor_si256(_mm256_cmpgt_epi32(a, b), ones));
    }
    alignas(32) float l8[8], h8[8];
    alignas(32) uint32_t b8[8], u8[8];
    _mm256_store_ps(l8, vlo);
    _mm256_store_ps(h8, vhi);
    _mm256_store_si256((__m256i*)b8, _mm256_castps_si256(vbad));
    _mm256_store_si256((__m256i*)u8, vuns);
    for (int j = 0; j < 8; ++j) {
      lo = std::min(lo, l8[j]);
      hi = std::max(hi, h8[j]);
      bad = bad || b8[j] != 0;
      sorted = sorted && u8[j] == 0;
    }
  }
  auto one = [&](uint32_t i) {
    const float x = rlp[i];
    olp[i] = x;
    oid[i] = rid[i];
    bad = bad || std::isnan(x) || x == INFINITY;
    if (x > thr) {
      lo = std::min(lo, x);
      hi = std::max(hi, x);
    }
    if (i > 0 && rid[i] <= rid[i - 1]) sorted = false;
  };
  if (K) one(0);
  for (; k < K; ++k) one(k);
  return RowScan{bad, sorted, lo, hi};
}

using ScanRowFn = RowScan (*)(const uint32_t*, const float*, uint32_t, float, uint32_t*, float*);
static const ScanRowFn g_scan_row =
    __builtin_cpu_supports("avx2") ? scan_row_avx2 : scan_row_sse2;

// Packs one validated request into its block at `base` (see plan_batch):
// the length-norm table, beam widths, per-step key bounds and token-sorted
// rows, and sets d.rk_off / d.in_bytes: the proposals' indices in the
// caller's rows are staged only when some row is out of order (else rk_off
// is 0 and the index is the position), and in_bytes ends the block there.
// Fails on NaN / +inf logps, duplicate token ids in a row and non-finite
// length-norm factors.  `tmp` holds K pairs.  In three parts, so that a
// streamed search can publish a request's first rows before the rest:
// pack_head (length-norm table, beam widths), pack_rows (rows t0 .. t1 - 1
// and their key bounds, in order), pack_end (rk_off, in_bytes).
struct PackState {
  double s_lo = 0.0, s_hi = 0.0;  // bounds of the parent scores at the next row
  uint32_t rk_planned = 0;        // where the row indices go when a row needs them
  bool rk_used = false;
};

static int pack_head(const ft_request& q, size_t r, DevReq& d, uint8_t* base, PackState& ps,
                     std::string* err) {
  const uint32_t T = d.T;
  // length-norm table, exactly Agent::logp_norm's factor (agent.h:69-72)
  double* lnf = (double*)base;
  // (depth 0 is the root alone, whose norm is never compared)
  for (uint32_t dd = 0; dd <= T; ++dd) {
    lnf[dd] = std::pow(6.0 / (5.0 + (double)dd), q.length_norm);
    if (dd > 0 && !std::isfinite(lnf[dd]))
      return *err = "request " + std::to_string(r) + ": length_norm gives a non-finite factor",
             FT_E_INPUT;
  }
  std::memcpy(base + d.beams_off, q.beams, 4ull * T);
  ps = PackState();
  // d.rk_off holds the planned offset of the indices until a row needs them
  ps.rk_planned = d.rk_off;
  return FT_OK;
}

static int pack_rows(const ft_request& q, size_t r, const DevReq& d, uint8_t* base, uint32_t t0,
                     uint32_t t1, std::pair<uint32_t, uint32_t>* tmp, PackState& ps,
                     std::string* err) {
  auto who = [r]() { return "request " + std::to_string(r) + ": "; };
  const uint32_t K = d.K;
  const double* lnf = (const double*)base;
  uint32_t* rid_s = (uint32_t*)(base + d.rid_off);
  float* rlp_s = (float*)(base + d.rlp_off);
  uint16_t* rk_s = (uint16_t*)(base + ps.rk_planned);
  uint64_t* kb = (uint64_t*)(base + d.kb_off);
  // Per step, bounds of the keys pushed into `next`: a push's score is a
  // parent score plus a logp that passes the token threshold, and itself
  // passes the sentence threshold; parent scores are bounded by the same
  // recursion one step earlier.  Double additions and the multiplication
  // by the length factor are monotone, so the bounds hold exactly for the
  // device's arithmetic (which this repeats).  A row with no logp above
  // the threshold contributes 0 to both bounds (it pushes nothing).
  for (uint32_t t = t0; t < t1; ++t) {
    const uint32_t* rid = q.topk_id_rows ? q.topk_id_rows[t] : q.topk_id + (uint64_t)t * K;
    const float* rlp = q.topk_logp_rows ? q.topk_logp_rows[t] : q.topk_logp + (uint64_t)t * K;
    if (!rid || !rlp) return *err = who() + "null topk row", FT_E_ARG;
    // rows in ascending token order, with each proposal's index in the
    // caller's row (the order the reference visits proposals in)
    uint32_t* oid = rid_s + (uint64_t)t * K;
    float* olp = rlp_s + (uint64_t)t * K;
    uint16_t* ok = rk_s + (uint64_t)t * K;
    const RowScan sc = g_scan_row(rid, rlp, K, q.token_logp_threshold, oid, olp);
    if (sc.bad) return *err = who() + "topk_logp holds NaN or +inf", FT_E_INPUT;
    if (sc.sorted) {
      if (ps.rk_used)
        for (uint32_t k = 0; k < K; ++k) ok[k] = (uint16_t)k;
    } else {
      if (!ps.rk_used) {  // the rows before this one, in order: index = position
        for (uint64_t i = 0; i < (uint64_t)t * K; ++i) rk_s[i] = (uint16_t)(i % K);
        ps.rk_used = true;
      }
      for (uint32_t k = 0; k < K; ++k) tmp[k] = {rid[k], k};
      std::sort(tmp, tmp + K);
      for (uint32_t p = 0; p < K; ++p) {
        if (p && tmp[p].first == tmp[p - 1].first)
          return *err = who() + "duplicate token id " + std::to_string(tmp[p].first) +
                        " in topk row " + std::to_string(t),
                 FT_E_INPUT;
        oid[p] = tmp[p].first;
        olp[p] = rlp[tmp[p].second];
        ok[p] = (uint16_t)tmp[p].second;
      }
    }
    const bool any = sc.hi >= sc.lo;
    const double x_lo = any ? (double)sc.lo : 0.0, x_hi = any ? (double)sc.hi : 0.0;
    const double lo = std::max(q.sent_logp_threshold, ps.s_lo + x_lo);
    const double hi = ps.s_hi + x_hi;
    kb[2 * t] = host_norm_key(lo * lnf[t + 1]);
    kb[2 * t + 1] = host_norm_key(hi * lnf[t + 1]);
    ps.s_lo = lo;
    ps.s_hi = hi;
  }
  return FT_OK;
}

static void pack_end(DevReq& d, const PackState& ps) {
  d.rk_off = ps.rk_used ? ps.rk_planned : 0u;
  d.in_bytes = ps.rk_used ? (uint32_t)align_up(ps.rk_planned + 2ull * d.T * d.K, 16)
                          : ps.rk_planned;
}

static int pack_request(const ft_request& q, size_t r, DevReq& d, uint8_t* base,
                        std::pair<uint32_t, uint32_t>* tmp, std::string* err) {
  PackState ps;
  if (int rc = pack_head(q, r, d, base, ps, err)) return rc;
  if (int rc = pack_rows(q, r, d, base, 0, d.T, tmp, ps, err)) return rc;
  pack_end(d, ps);
  return FT_OK;
}

// Checks the shapes of `batch` requests against the limits and lays them
// out in H (cap bytes): DevReq[batch], then each request's block
// (length-norm table, beam widths, key bounds, token-sorted rows, row
// indices), without reading the rows.  Fills staged[0, batch) and the
// DevReqs; *bytes = bytes used, *out_stride = output bytes per request.
// On an error, *first_bad is the first request (in batch order) with a
// shape error, and the requests before it are laid out.
static int plan_batch(const ft_request* reqs, size_t batch, const StageLimits& lim,
                      uint8_t* H, uint64_t cap, StagedReq* staged, uint64_t* bytes,
                      uint64_t* out_stride, size_t* first_bad_out, std::string* msg) {
  DevReq* D = (DevReq*)H;
  uint64_t off = align_up(batch * sizeof(DevReq), 256);
  uint64_t max_out = sizeof(OutHeader);
  size_t first_bad = batch;
  int first_rc = FT_OK;
  std::string first_msg;
  for (size_t r = 0; r < batch && first_bad == batch; ++r) {
    const ft_request& q = reqs[r];
    auto who = [r]() { return "request " + std::to_string(r) + ": "; };
    auto bad = [&](int rc, const std::string& m) {
      first_bad = r;
      first_rc = rc;
      first_msg = m;
    };
    DevReq d{};
    StagedReq& st = staged[r];
    if (q.num_beams == 0 || !q.beams) {
      bad(FT_E_INPUT, who() + "beams is empty");
      break;
    }
    const uint32_t F = q.beams[q.num_beams - 1];
    if (F == 0) {  // outputs untouched (louds-trie.cc:114-117)
      st.skip = true;
      d.flags = kReqSkip;
      d.in_off = off;
      D[r] = d;
      continue;
    }
    const uint32_t T = q.num_steps, K = q.topk;
    if (T == 0 || K == 0) {
      bad(FT_E_INPUT, who() + "topk rows are empty");
      break;
    }
    if (q.num_beams < T) {
      bad(FT_E_INPUT, who() + "fewer beam widths than topk rows");
      break;
    }
    if (T > lim.max_steps) {
      bad(FT_E_LIMIT, who() + "steps " + std::to_string(T) + " > max_num_outpos " +
                          std::to_string(lim.max_steps));
      break;
    }
    if (K > lim.max_topk) {
      bad(FT_E_LIMIT, who() + "topk " + std::to_string(K) + " > max_num_topk " +
                          std::to_string(lim.max_topk));
      break;
    }
    if (F > lim.max_out_beams) {
      bad(FT_E_LIMIT, who() + "final beam > max_num_out_beams");
      break;
    }
    if ((uint64_t)F * T > lim.max_out_tokens) {
      bad(FT_E_LIMIT, who() + "final beam * steps > max_num_out_tokens");
      break;
    }
    uint64_t bmax = F, hsum = 0;
    for (uint32_t t = 0; t < T && first_bad == batch; ++t) {
      if (q.beams[t] == 0)
        bad(FT_E_INPUT, who() + "beam width 0 at step " + std::to_string(t));
      else if (q.beams[t] > lim.max_out_beams)
        bad(FT_E_LIMIT, who() + "beam width > max_num_out_beams");
      bmax = std::max<uint64_t>(bmax, q.beams[t]);
      hsum += q.beams[t];
    }
    if (first_bad != batch) break;
    if (!q.topk_id_rows && (!q.topk_id || !q.topk_logp)) {
      bad(FT_E_ARG, who() + "null topk arrays");
      break;
    }
    if (q.topk_id_rows && !q.topk_logp_rows) {
      bad(FT_E_ARG, who() + "null topk_logp rows");
      break;
    }
    // the block: lnf[T + 1] f64, beams[T], key bounds, rows (token, logp),
    // then the row indices, which the kernel reads only when some row came
    // out of order; it must fit before anything is written
    uint64_t o = align_up(8ull * (T + 1), 16);
    d.beams_off = (uint32_t)o;
    o = align_up(o + 4ull * T, 16);
    d.kb_off = (uint32_t)o;
    o = align_up(o + 16ull * T, 16);
    d.rid_off = (uint32_t)o;
    o = align_up(o + 4ull * T * K, 16);
    d.rlp_off = (uint32_t)o;
    o = align_up(o + 4ull * T * K, 16);
    d.rk_off = (uint32_t)o;
    d.in_bytes = (uint32_t)align_up(o + 2ull * T * K, 16);
    o = d.in_bytes;
    if (off + o > cap) {
      bad(FT_E_LIMIT, who() + "the staged batch exceeds the staging buffer (" +
                          std::to_string(cap) + " bytes)");
      break;
    }
    d.T = T;
    d.K = K;
    d.F = F;
    d.flags = q.early_exit ? kReqEarlyExit : 0u;
    d.tok_thr = q.token_logp_threshold;
    d.sent_thr = q.sent_logp_threshold;
    d.in_off = off;
    d.out_T = T;
    D[r] = d;
    off = align_up(off + o, 256);
    st.T = T;
    st.K = K;
    st.F = F;
    st.bmax = bmax;
    st.hsum = hsum;
    st.out_bytes = step_stats_offset(F, T) + 8ull * kStepStats * T;
    max_out = std::max(max_out, st.out_bytes);
  }
  *first_bad_out = first_bad;
  *out_stride = align_up(max_out, 256);
  *bytes = off;
  if (first_bad != batch) return *msg = first_msg, first_rc;
  return FT_OK;
}

// Validates `batch` requests and packs them into H (cap bytes), laid out by
// plan_batch.  `tmp` holds max_topk pairs (the buffer an unsorted row is
// sorted in).  An error names the first request (in batch order) that has
// one.  Allocates nothing on success.
static int pack_batch(const ft_request* reqs, size_t batch, const StageLimits& lim,
                      uint8_t* H, uint64_t cap, StagedReq* staged,
                      std::pair<uint32_t, uint32_t>* tmp, uint64_t* bytes,
                      uint64_t* out_stride) {
  size_t first_bad = batch;
  std::string plan_msg;
  const int plan_rc = plan_batch(reqs, batch, lim, H, cap, staged, bytes, out_stride,
                                 &first_bad, &plan_msg);
  // the blocks of the requests before the first shape error
  DevReq* D = (DevReq*)H;
  for (size_t r = 0; r < first_bad; ++r) {
    if (staged[r].skip) continue;
    std::string msg;
    if (int rc = pack_request(reqs[r], r, D[r], H + D[r].in_off, tmp, &msg)) return fail(rc, msg);
  }
  if (plan_rc) return fail(plan_rc, plan_msg);
  return FT_OK;
}

int ft_stage(ft_ctx* c, const ft_request* reqs, size_t batch) {
  if (!c || (!reqs && batch)) return fail(FT_E_ARG, "ft_stage: null argument");
  if (!c->reserved) return fail(FT_E_STATE, "ft_stage: init_tbs_gpu (ft_reserve) was not called");
  if (batch == 0 || batch > c->max_staged)
    return fail(FT_E_LIMIT, "ft_stage: batch size " + std::to_string(batch) +
                                " not in [1, " + std::to_string(c->max_staged) + "]");
  (void)hipSetDevice(c->device);
  // the previous staging copy may still be queued behind a running launch:
  // it reads h_stage, which is rewritten below
  if (c->stage_pending) {
    const hipError_t we = hipEventSynchronize(c->stage_ev);
    if (we != hipSuccess) return hip_fail(we, "hipEventSynchronize(stage)");
    c->stage_pending = false;
  }
  c->staged.assign(batch, StagedReq());
  c->launched_slot.assign(batch, 0);
  c->launched = false;
  StageLimits lim{c->max_steps, c->max_topk, c->max_out_beams, c->max_out_tokens};
  uint64_t used = 0;
  if (int rc = pack_batch(reqs, batch, lim, c->h_stage, c->stage_cap, c->staged.data(),
                          c->sort_tmp.data(), &used, &c->out_stride)) {
    c->staged.clear();
    c->launched_slot.clear();
    return rc;
  }
  const uint64_t off = used;
  hipError_t e = hipMemcpyAsync(c->d_stage, c->h_stage, off, hipMemcpyHostToDevice, c->stream);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(stage)");
  if ((e = hipEventRecord(c->stage_ev, c->stream)) != hipSuccess)
    return hip_fail(e, "hipEventRecord(stage)");
  c->stage_pending = true;
  return FT_OK;
}

// Kernel arguments for requests [first, first + count) of a batch staged
// at `stage` (DevReq array first), with workspace slots of `ws_stride`
// bytes from `ws` and output blocks of `out_stride` bytes from `out`.
static KArgs kernel_args(const ft_ctx* c, const uint8_t* stage, size_t first, size_t count,
                         uint32_t kmax, uint8_t* ws, uint64_t ws_stride, const WsLayout& lay,
                         uint8_t* out, uint64_t out_stride) {
  KArgs a{};
  a.recs = (const ft_node_rec*)(c->d_image + c->hdr.recs_offset);
  a.parent = (const uint32_t*)(c->d_image + c->hdr.parent_offset);
  a.tail = (const uint32_t*)(c->d_image + c->hdr.tail_offset);
  a.reqs = (const DevReq*)stage + first;
  a.stage = stage;
  a.ws = ws;
  a.ws_stride = ws_stride;
  a.out = out + first * out_stride;
  a.out_stride = out_stride;
  a.lay = lay;
  a.batch = (uint32_t)count;
  const uint64_t sl = (uint64_t)c->scan_mult * kmax;
  a.scan_limit = (uint32_t)std::min<uint64_t>(sl, 0xFFFFFFFFull);
  // helpers per request: as many as stay co-resident with the batch
  const uint32_t fit = (uint32_t)std::max<int>(1, c->max_resident / (int)count);
  a.wgs = std::max(1u, std::min(std::min(c->wgs_req, fit), lay.claim_slots));
  a.share_min = c->share_min;
  uint32_t ep = ++g_launch_epoch;
  if (ep == 0) ep = ++g_launch_epoch;
  a.epoch = ep;
  a.wdir = c->d_wdir;
  a.wtab = c->d_wtab;
  a.wfp = c->d_wfp;
  a.labels = c->d_labels;
  a.wdir_log2 = c->wdir_log2;
  a.wide_min = c->wide_min;
  a.no_claims = c->no_claims;
  a.head_rows = 0;
  a.louds_words = c->d_louds_words;
  a.louds_z = c->d_louds_z;
  a.louds_s = c->d_louds_s;
  a.stage_src = nullptr;
  a.ready = nullptr;
  a.out_host = nullptr;
  a.stage_bytes = 0;
  a.ready_ticks = c->ready_ticks;
  a.root_dir = c->d_root_dir;
  a.root_n = c->d_root_dir ? c->root_n : 0u;
  a.root_force = c->root_force;
  return a;
}

// One launch of the search kernel on the context stream, timed by a pair of
// the ring's events.  `attached`: events attached to the dispatch, the
// kernel's own run as a kernel trace reports it (the device-resident
// launches, whose durations ft_launch_times reports).  Otherwise markers
// recorded around the launch, which also span the ~5 us the queue spends
// between them and the kernel: the streamed search keeps these, because an
// attached pair made its calls ~16 us slower at the C++ boundary.
static int launch_timed(ft_ctx* c, const KArgs& a, bool attached) {
  (void)hipSetDevice(c->device);
  const size_t slot = (c->launches % ft_ctx::kRing) * 2;
  hipError_t e;
  if (attached) {
    e = launch_tbs(a, c->stream, c->ring[slot], c->ring[slot + 1]);
    if (e != hipSuccess) return hip_fail(e, "launch of the search kernel");
  } else {
    (void)hipEventRecord(c->ring[slot], c->stream);
    e = launch_tbs(a, c->stream);
    if (e != hipSuccess) return hip_fail(e, "launch of the search kernel");
    (void)hipEventRecord(c->ring[slot + 1], c->stream);
  }
  ++c->launches;
  return FT_OK;
}

int ft_launch(ft_ctx* c) {
  if (!c) return fail(FT_E_ARG, "ft_launch: null context");
  return ft_launch_range(c, 0, c->staged.size());
}

int ft_launch_range(ft_ctx* c, size_t first, size_t count) {
  if (!c) return fail(FT_E_ARG, "ft_launch_range: null context");
  if (c->staged.empty()) return fail(FT_E_STATE, "ft_launch: nothing staged");
  if (count == 0 || count > c->max_batch || first + count > c->staged.size())
    return fail(FT_E_LIMIT, "ft_launch_range: [" + std::to_string(first) + ", +" +
                                std::to_string(count) + ") exceeds the staged requests or max_batch_size " +
                                std::to_string(c->max_batch));
  uint32_t kmax = 1;
  for (size_t i = first; i < first + count; ++i) kmax = std::max(kmax, c->staged[i].K);
  const KArgs a = kernel_args(c, c->d_stage, first, count, kmax, c->d_ws, c->ws_stride,
                              c->lay, c->d_out, c->out_stride);
  if (int rc = launch_timed(c, a, true)) return rc;
  c->launched = true;
  for (size_t i = first; i < first + count; ++i) c->launched_slot[i] = 1;
  return FT_OK;
}

int ft_launch_times(ft_ctx* c, double* ms, size_t n) {
  if (!c || (!ms && n)) return fail(FT_E_ARG, "ft_launch_times: null argument");
  if (n > c->launches || n > ft_ctx::kRing)
    return fail(FT_E_ARG, "ft_launch_times: fewer launches recorded");
  (void)hipSetDevice(c->device);
  hipError_t e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  for (size_t i = 0; i < n; ++i) {
    const uint64_t L = c->launches - n + i;
    const size_t slot = (L % ft_ctx::kRing) * 2;
    float f = 0.f;
    e = hipEventElapsedTime(&f, c->ring[slot], c->ring[slot + 1]);
    if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
    ms[i] = f;
  }
  return FT_OK;
}

int ft_reserve_staging(ft_ctx* c, size_t max_staged) {
  if (!c) return fail(FT_E_ARG, "ft_reserve_staging: null context");
  if (!c->reserved) return fail(FT_E_STATE, "ft_reserve_staging: ft_reserve was not called");
  if (max_staged < c->max_batch) max_staged = c->max_batch;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  c->staged.clear();
  c->launched_slot.clear();
  c->launched = false;
  c->stage_pending = false;
  return alloc_staging(c, max_staged);
}

int ft_sync(ft_ctx* c, double* ms) {
  if (!c) return fail(FT_E_ARG, "ft_sync: null context");
  (void)hipSetDevice(c->device);
  hipError_t e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  if (ms) {
    float f = 0.f;
    if (c->launches) {
      const size_t slot = ((c->launches - 1) % ft_ctx::kRing) * 2;
      (void)hipEventElapsedTime(&f, c->ring[slot], c->ring[slot + 1]);
    }
    *ms = f;
  }
  return FT_OK;
}

// Fills `o` from request r's output block `ob` (in h_out, or in host
// memory the kernel wrote directly) and adds its device counters to `tm`.
// Returns the request's error (FT_OK when its results are in `o`), with
// its text in *msg.
static int unpack_one(const uint8_t* ob, const StagedReq& st, bool launched, size_t r,
                      ft_result& o, double tick_ms, ft_timing& tm, std::string* msg) {
  auto err = [&](int rc, const std::string& m) {
    o.count = 0;
    o.status = rc;
    *msg = "request " + std::to_string(r) + m;
    return rc;
  };
  if (!launched)  // staged but not launched since: no result of this request
    return err(FT_E_STATE, ": staged but not launched");
  if (st.skip) {
    o.count = 0;
    o.status = FT_OK;
    return FT_OK;
  }
  const OutHeader* oh = (const OutHeader*)ob;
  const uint32_t status = oh->status & ~kStatusDone;
  tm.expand_ms += oh->ticks_expand * tick_ms;
  tm.select_ms += oh->ticks_select * tick_ms;
  tm.other_ms += (double)(oh->ticks_total - oh->ticks_expand - oh->ticks_select) * tick_ms;
  tm.candidates += oh->candidates;
  tm.parents += oh->parents;
  tm.children += oh->children;
  tm.probes += oh->probes;
  if (status)
    return err((status & kStatusHistory) ? FT_E_LIMIT : FT_E_KERNEL,
               (status & kStatusHistory)    ? ": hypotheses exceed max_num_inter_beams"
               : (status & kStatusNotReady) ? ": its staged data was not ready in time"
                                            : ": kernel status " + std::to_string(status));
  const uint32_t n = oh->count;
  if (n > o.capacity || (n && (!o.logp_norm || !o.length || !o.tokens)) ||
      o.token_stride < st.T)
    return err(FT_E_ARG, ": result arrays too small");
  o.device_ms[0] = oh->ticks_expand * tick_ms;
  o.device_ms[1] = oh->ticks_select * tick_ms;
  o.device_ms[2] = (double)(oh->ticks_total - oh->ticks_expand - oh->ticks_select) * tick_ms;
  o.device_ms[3] = oh->ticks_total * tick_ms;
  const double* norms = (const double*)(ob + sizeof(OutHeader));
  const uint32_t* lens = (const uint32_t*)(norms + st.F);
  const uint32_t* toks = lens + st.F;
  std::memcpy(o.logp_norm, norms, 8ull * n);
  std::memcpy(o.length, lens, 4ull * n);
  for (uint32_t i = 0; i < n; ++i) {
    const uint32_t L = std::min(lens[i], st.T);
    std::memcpy(o.tokens + (uint64_t)i * o.token_stride, toks + (uint64_t)i * st.T, 4ull * L);
  }
  o.count = n;
  o.status = FT_OK;
  if (o.step_stats) {
    const uint64_t* ss = (const uint64_t*)(ob + step_stats_offset(st.F, st.T));
    std::memcpy(o.step_stats, ss, 8ull * kStepStats * st.T);
  }
  return FT_OK;
}

// Fills `res` from the output blocks of a batch copied back to h_out
// (out_stride bytes per request).  Returns the first request error.
static int unpack_results(const uint8_t* h_out, uint64_t out_stride, const StagedReq* staged,
                          const uint8_t* launched, size_t batch, ft_result* res,
                          int wall_khz, double kernel_ms, ft_timing* timing) {
  int first_err = FT_OK;
  ft_timing tm{};
  tm.kernel_ms = kernel_ms;
  const double tick_ms = wall_khz > 0 ? 1.0 / wall_khz : 0.0;
  std::string msg;
  for (size_t r = 0; r < batch; ++r) {
    const int rc = unpack_one(h_out + out_stride * r, staged[r], launched[r] != 0, r, res[r],
                              tick_ms, tm, &msg);
    if (rc && !first_err) {
      first_err = rc;
      g_err = msg;
    }
  }
  if (timing) *timing = tm;
  return first_err;
}

int ft_fetch(ft_ctx* c, ft_result* res, size_t batch, ft_timing* timing) {
  if (!c) return fail(FT_E_ARG, "ft_fetch: null context");
  if (!c->launched) return fail(FT_E_STATE, "ft_fetch: no launch to fetch");
  if (batch != c->staged.size()) return fail(FT_E_ARG, "ft_fetch: batch mismatch");
  (void)hipSetDevice(c->device);
  hipError_t e = hipMemcpyAsync(c->h_out, c->d_out, c->out_stride * batch,
                                hipMemcpyDeviceToHost, c->stream);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(output)");
  double ms = 0.0;
  int rc = ft_sync(c, &ms);
  if (rc) return rc;
  return unpack_results(c->h_out, c->out_stride, c->staged.data(), c->launched_slot.data(),
                        batch, res, c->wall_khz, ms, timing);
}

namespace {
struct PackJob {
  const ft_request* reqs;
  DevReq* D;
  uint8_t* H;
  const StagedReq* staged;
  unsigned long long* ready;
  unsigned long long tag;
  size_t batch;
  // rows a request's first ready word carries (0: all of them)
  uint32_t head_rows = 0;
  std::vector<int> rc;
  std::vector<std::string> msg;
};

// Packs the requests of `j` and writes their ready words (a skipped
// request's workgroups return at once and need none); `tmp` holds max_topk
// pairs.  First, request by request, the length-norm table, beam widths and
// the rows before its split (stream_split), then a kReadyPart word; then, again request by
// request, the other rows, with a kReadyPart word after each, and the
// kReadyOk word.  So every request of a batch can start after a short
// first pass, and its leader finds the other rows when it needs them.  A
// request that fails to pack is withdrawn at once.
void pack_stream(PackJob& j, std::pair<uint32_t, uint32_t>* tmp) {
  std::vector<PackState> ps(j.batch);
  auto publish = [&](size_t r, unsigned long long state) {
    // the block's stores (non-temporal ones included) before the word
    _mm_sfence();
    __atomic_store_n(&j.ready[r], j.tag | state, __ATOMIC_RELEASE);
  };
  auto rows_word = [&](size_t r, uint32_t rows) {
    return ((unsigned long long)rows << kReadyRowsShift) | kReadyPart |
           (ps[r].rk_used ? kReadyRk : 0u);
  };
  auto withdraw = [&](size_t r, int rc) {
    j.rc[r] = rc;
    publish(r, kReadyWithdrawn);
  };
  // The launched header (D[r], in mapped memory) keeps its planned rk_off and
  // in_bytes: the kernel copies it at its start while this thread packs, so
  // a rewrite here could be read half old and half new.  The planned values
  // hold every array; whether the row indices were staged travels in the
  // ready word (kReadyRk) instead of rk_off.
  auto finish = [&](size_t r) {
    publish(r, ((unsigned long long)j.D[r].T << kReadyRowsShift) | kReadyOk |
                   (ps[r].rk_used ? kReadyRk : 0u));
  };
  for (size_t r = 0; r < j.batch; ++r) {
    if (j.staged[r].skip) continue;
    DevReq& d = j.D[r];
    uint8_t* base = j.H + d.in_off;
    const uint32_t h = stream_split(j.head_rows, d.T, d.K);
    int rc = pack_head(j.reqs[r], r, d, base, ps[r], &j.msg[r]);
    if (!rc) rc = pack_rows(j.reqs[r], r, d, base, 0, h, tmp, ps[r], &j.msg[r]);
    if (rc) withdraw(r, rc);
    else if (h == d.T) finish(r);
    else publish(r, rows_word(r, h));
  }
  for (size_t r = 0; r < j.batch; ++r) {
    DevReq& d = j.D[r];
    const uint32_t h = stream_split(j.head_rows, d.T, d.K);
    if (j.staged[r].skip || j.rc[r] || h >= d.T) continue;
    uint8_t* base = j.H + d.in_off;
    int rc = FT_OK;
    for (uint32_t t = h; t < d.T && !rc; ++t) {
      rc = pack_rows(j.reqs[r], r, d, base, t, t + 1, tmp, ps[r], &j.msg[r]);
      if (!rc && t + 1 < d.T) publish(r, rows_word(r, t + 1));
    }
    if (rc) withdraw(r, rc);
    else finish(r);
  }
}
}  // namespace

// A streamed search: the kernel is launched as soon as the batch's shapes
// are checked and laid out, and the requests are packed into mapped host
// memory while it runs.  A request's leader starts once the request's
// ready word is written, copies the packed block to the device itself and
// writes the results back to mapped host memory, so packing overlaps the
// launch and the search of the requests before it, and no copy engine sits
// on the path.  Each request's results are taken (and handed to `fn`) as
// soon as its leader publishes them, while the others still search.
// Errors are those of ft_stage + ft_launch + ft_fetch: a request that fails
// to pack is withdrawn, the kernel is waited for, and the first error in
// request order is returned.
int ft_search(ft_ctx* c, const ft_request* reqs, size_t batch,
              ft_result* results, ft_timing* timing) {
  return ft_search_each(c, reqs, batch, results, timing, nullptr, nullptr);
}

int ft_search_each(ft_ctx* c, const ft_request* reqs, size_t batch, ft_result* results,
                   ft_timing* timing, ft_result_fn fn, void* user) {
  if (!c || (!reqs && batch) || (!results && batch))
    return fail(FT_E_ARG, "ft_search: null argument");
  if (!c->reserved) return fail(FT_E_STATE, "ft_search: init_tbs_gpu (ft_reserve) was not called");
  if (batch == 0 || batch > c->max_batch || batch > c->max_staged)
    return fail(FT_E_LIMIT, "ft_search: batch size " + std::to_string(batch) + " not in [1, " +
                                std::to_string(std::min(c->max_batch, c->max_staged)) + "]");
  if (c->d_louds_words) {
    // the LOUDS directory's kernel has no streamed form
    int rc = ft_stage(c, reqs, batch);
    if (!rc) rc = ft_launch(c);
    if (!rc) rc = ft_fetch(c, results, batch, timing);
    if (fn && rc != FT_E_ARG)
      for (size_t r = 0; r < batch; ++r)
        if (results[r].status == FT_OK) fn(user, r);
    return rc;
  }
  (void)hipSetDevice(c->device);
  // a staging copy of ft_stage may still be queued: it reads h_stage
  if (c->stage_pending) {
    const hipError_t we = hipEventSynchronize(c->stage_ev);
    if (we != hipSuccess) return hip_fail(we, "hipEventSynchronize(stage)");
    c->stage_pending = false;
  }
  c->staged.assign(batch, StagedReq());
  c->launched_slot.assign(batch, 0);
  c->launched = false;
  const StageLimits lim{c->max_steps, c->max_topk, c->max_out_beams, c->max_out_tokens};
  DevReq* D = (DevReq*)c->h_stage;
  auto drop = [c](int rc) {
    c->staged.clear();
    c->launched_slot.clear();
    return rc;
  };
  uint64_t used = 0;
  size_t first_bad = batch;
  std::string msg;
  if (int rc = plan_batch(reqs, batch, lim, c->h_stage, c->stage_cap, c->staged.data(), &used,
                          &c->out_stride, &first_bad, &msg)) {
    // a packing error of a request before the first shape error comes first
    for (size_t r = 0; r < first_bad; ++r) {
      if (c->staged[r].skip) continue;
      std::string m;
      if (int prc = pack_request(reqs[r], r, D[r], c->h_stage + D[r].in_off, c->sort_tmp.data(), &m))
        return drop(fail(prc, m));
    }
    return drop(fail(rc, msg));
  }
  uint32_t kmax = 1;
  for (size_t i = 0; i < batch; ++i) kmax = std::max(kmax, c->staged[i].K);
  KArgs a = kernel_args(c, c->d_stage, 0, batch, kmax, c->d_ws, c->ws_stride, c->lay, c->d_out,
                        c->out_stride);
  a.reqs = (const DevReq*)c->m_stage;
  a.stage_src = c->m_stage;
  a.ready = c->m_ready;
  a.out_host = c->m_out;
  a.stage_bytes = used;
  a.head_rows = c->head_rows;
  // the result headers start unpublished
  for (size_t r = 0; r < batch; ++r)
    __atomic_store_n(&((OutHeader*)(c->h_out + c->out_stride * r))->status, 0u, __ATOMIC_RELAXED);
  if (int rc = launch_timed(c, a, false)) return drop(rc);
  PackJob job;
  job.reqs = reqs;
  job.D = D;
  job.H = c->h_stage;
  job.staged = c->staged.data();
  job.ready = c->h_ready;
  job.tag = (unsigned long long)a.epoch << 32;
  job.batch = batch;
  job.head_rows = a.head_rows;
  job.rc.assign(batch, FT_OK);
  job.msg.resize(batch);
  if (c->pack_delay_us) std::this_thread::sleep_for(std::chrono::microseconds(c->pack_delay_us));
  pack_stream(job, c->sort_tmp.data());
  // Each request's results once its leader has published them (kStatusDone
  // in its header, written last with a system-scope release), in the order
  // the requests finish; the stream is looked at now and then, so that a
  // kernel that ends without publishing one is noticed.
  ft_timing tm{};
  const double tick_ms = c->wall_khz > 0 ? 1.0 / c->wall_khz : 0.0;
  std::vector<int>& rcs = c->req_rc;
  std::vector<std::string>& msgs = c->req_msg;
  rcs.assign(batch, FT_OK);
  if (msgs.size() < batch) msgs.resize(batch);
  std::vector<uint8_t>& got = c->req_got;
  got.assign(batch, 0);
  size_t left = batch;
  // requests whose leader gave up waiting for their rows (the host thread
  // was descheduled, the input pages were faulted in, ...): searched again
  // from the staged path once this launch is over
  std::vector<size_t> retry;
  auto take = [&](size_t r) {
    got[r] = 1;
    --left;
    if (job.rc[r]) return;  // withdrawn: its packing error is reported
    const OutHeader* oh = (const OutHeader*)(c->h_out + c->out_stride * r);
    if (!c->staged[r].skip && (oh->status & kStatusNotReady)) {
      retry.push_back(r);
      return;
    }
    rcs[r] = unpack_one(c->h_out + c->out_stride * r, c->staged[r], true, r, results[r], tick_ms,
                        tm, &msgs[r]);
    if (rcs[r] == FT_OK && fn) fn(user, r);
  };
  for (size_t r = 0; r < batch; ++r)
    if (c->staged[r].skip) take(r);
  bool over = false;
  for (uint32_t it = 1; left; ++it) {
    for (size_t r = 0; r < batch; ++r) {
      if (got[r]) continue;
      const uint32_t* sw = &((const OutHeader*)(c->h_out + c->out_stride * r))->status;
      if (__atomic_load_n(sw, __ATOMIC_ACQUIRE) & kStatusDone) take(r);
    }
    if (!left) break;
    if (over) {  // the kernel ended and these were never published
      for (size_t r = 0; r < batch; ++r)
        if (!got[r]) {
          got[r] = 1;
          rcs[r] = FT_E_KERNEL;
          msgs[r] = "request " + std::to_string(r) + ": the search ended without its results";
          results[r].count = 0;
          results[r].status = FT_E_KERNEL;
        }
      break;
    }
    if ((it & 63u) == 0) {
      const hipError_t q = hipStreamQuery(c->stream);
      if (q == hipSuccess) {
        over = true;  // one more look at the headers, then give up
      } else if (q != hipErrorNotReady) {
        (void)hipStreamSynchronize(c->stream);
        return drop(hip_fail(q, "search kernel"));
      }
    }
    _mm_pause();
  }
  double ms = 0.0;
  if (int rc = ft_sync(c, &ms)) return drop(rc);
  tm.kernel_ms = ms;
  // the results were taken here: d_out holds no batch for ft_fetch
  c->staged.clear();
  c->launched_slot.clear();
  if (!retry.empty()) {
    // (the streamed kernel is over: h_stage is free for ft_stage)
    std::vector<ft_request> sub;
    std::vector<ft_result> sres;
    for (size_t r : retry) {
      sub.push_back(reqs[r]);
      sres.push_back(results[r]);
    }
    ft_timing st{};
    int rc = ft_stage(c, sub.data(), sub.size());
    if (!rc) rc = ft_launch(c);
    if (!rc) rc = ft_fetch(c, sres.data(), sub.size(), &st);
    const std::string why = rc ? ft_last_error() : "";
    for (size_t i = 0; i < retry.size(); ++i) {
      const size_t r = retry[i];
      results[r] = sres[i];
      if (rc && results[r].status == FT_OK) results[r].status = rc;
      rcs[r] = results[r].status;
      if (rcs[r]) {
        results[r].count = 0;
        msgs[r] = "request " + std::to_string(r) + ": not ready in the streamed search, then " +
                  (why.empty() ? std::string(ft_strerror(rcs[r])) : why);
      } else if (fn) {
        fn(user, r);
      }
    }
    tm.expand_ms += st.expand_ms;
    tm.select_ms += st.select_ms;
    tm.other_ms += st.other_ms;
    tm.candidates += st.candidates;
    tm.parents += st.parents;
    tm.children += st.children;
    tm.probes += st.probes;
    tm.kernel_ms += st.kernel_ms;
    c->staged.clear();
    c->launched_slot.clear();
    c->launched = false;
  }
  if (timing) *timing = tm;
  for (size_t r = 0; r < batch; ++r)  // the first packing error in request order
    if (job.rc[r]) return fail(job.rc[r], job.msg[r]);
  for (size_t r = 0; r < batch; ++r)
    if (rcs[r]) return fail(rcs[r], msgs[r]);
  return FT_OK;
}

// Host side of the no-allocation path: pageable buffers in the library's
// own static storage (no allocation), used under g_noalloc_mu.
namespace {
constexpr size_t kNoAllocMaxBatch = 64;
constexpr uint64_t kNoAllocHostBytes = 16ull << 20;
std::mutex g_noalloc_mu;
alignas(256) uint8_t g_na_stage[kNoAllocHostBytes];
alignas(256) uint8_t g_na_out[kNoAllocHostBytes];
StagedReq g_na_staged[kNoAllocMaxBatch];
uint8_t g_na_launched[kNoAllocMaxBatch];
std::pair<uint32_t, uint32_t> g_na_sort[kMaxLdsTopk];
}  // namespace

int ft_search_noalloc(ft_ctx* c, const ft_request* reqs, size_t batch,
                      ft_result* results, ft_timing* timing) {
  if (!c || !reqs || !results) return fail(FT_E_ARG, "ft_search_noalloc: null argument");
  if (batch == 0 || batch > kNoAllocMaxBatch)
    return fail(FT_E_LIMIT, "ft_search_noalloc: batch size " + std::to_string(batch) +
                                " not in [1, " + std::to_string(kNoAllocMaxBatch) + "]");
  if (!c->d_scratch)
    return fail(FT_E_STATE, "ft_search_noalloc: no scratch on this device (" +
                                c->scratch_err + ")");
  // one call at a time in this process: the scratch and the host buffers
  // are shared by every call
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  (void)hipSetDevice(c->device);
  for (size_t r = 0; r < batch; ++r) {
    g_na_staged[r] = StagedReq();
    g_na_launched[r] = 1;
  }
  const StageLimits lim{16383, kMaxLdsTopk, kMaxBeams, ~0ull};
  uint64_t used = 0, out_stride = 0;
  if (int rc = pack_batch(reqs, batch, lim, g_na_stage, kNoAllocHostBytes, g_na_staged,
                          g_na_sort, &used, &out_stride))
    return rc;
  // the workspace this batch needs: its widest beam, longest row and
  // largest history (the sum of a request's beam widths bounds its records)
  uint64_t B = 1, K = 1, H = 1;
  for (size_t r = 0; r < batch; ++r) {
    const StagedReq& st = g_na_staged[r];
    if (st.skip) continue;
    B = std::max(B, st.bmax);
    K = std::max<uint64_t>(K, st.K);
    H = std::max(H, st.hsum);
  }
  if (B * K + B >= 0xFFFFFFF0ull || H >= 0xFFFFFFF0ull)
    return fail(FT_E_LIMIT, "ft_search_noalloc: beams * topk too large");
  WsLayout L{};
  const uint64_t ws_stride = ws_layout(B, K, H, (uint32_t)c->max_resident, &L);
  const uint64_t out_off = align_up(used, 256);
  const uint64_t ws_off = align_up(out_off + out_stride * batch, 256);
  const uint64_t total = ws_off + ws_stride * batch;
  if (total > kScratchBytes || out_stride * batch > kNoAllocHostBytes)
    return fail(FT_E_LIMIT, "ft_search_noalloc: the batch needs " + std::to_string(total) +
                                " bytes of device scratch (limit " +
                                std::to_string(kScratchBytes) + ")");
  uint8_t* base = c->d_scratch;
  hipError_t e = hipMemcpyAsync(base, g_na_stage, used, hipMemcpyHostToDevice, c->stream);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(scratch stage)");
  // the control blocks, claim words and done words start at "nothing
  // posted" (a fill kernel, no memset)
  if ((e = clear_controls(base + ws_off, ws_stride, L.ctl, L.claims, L.dones, L.claim_slots,
                          (uint32_t)batch, c->stream)) != hipSuccess)
    return hip_fail(e, "clear_controls");
  const KArgs a = kernel_args(c, base, 0, batch, (uint32_t)K, base + ws_off, ws_stride, L,
                              base + out_off, out_stride);
  if (int rc = launch_timed(c, a, false)) return rc;
  if ((e = hipMemcpyAsync(g_na_out, base + out_off, out_stride * batch, hipMemcpyDeviceToHost,
                          c->stream)) != hipSuccess)
    return hip_fail(e, "hipMemcpyAsync(scratch output)");
  double ms = 0.0;
  if (int rc = ft_sync(c, &ms)) return rc;
  return unpack_results(g_na_out, out_stride, g_na_staged, g_na_launched, batch, results,
                        c->wall_khz, ms, timing);
}

void ft_destroy(ft_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  release_workspace(c);
  if (c->d_image) (void)hipFree(c->d_image);
  if (c->d_wdir) (void)hipFree(c->d_wdir);
  if (c->d_wtab) (void)hipFree(c->d_wtab);
  if (c->d_wfp) (void)hipFree(c->d_wfp);
  if (c->d_labels) (void)hipFree(c->d_labels);
  if (c->d_root_dir) (void)hipFree(c->d_root_dir);
  if (c->d_louds_words) (void)hipFree(c->d_louds_words);
  if (c->d_louds_z) (void)hipFree(c->d_louds_z);
  if (c->d_louds_s) (void)hipFree(c->d_louds_s);
  for (auto& ev : c->ring)
    if (ev) (void)hipEventDestroy(ev);
  if (c->stage_ev) (void)hipEventDestroy(c->stage_ev);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}

int ft_device_info(ft_ctx* c, int* num_cus, int* lds_per_block,
                   int* wall_clock_khz, char* name, size_t name_len) {
  if (!c) return fail(FT_E_ARG, "ft_device_info: null context");
  if (num_cus) *num_cus = c->num_cus;
  if (lds_per_block) *lds_per_block = c->lds_per_block;
  if (wall_clock_khz) *wall_clock_khz = c->wall_khz;
  if (name && name_len) std::snprintf(name, name_len, "%s", c->name);
  return FT_OK;
}

}  // extern "C"
