// tbs_kernel.hip -- trie beam search (TBS) kernel for gfx950 (MI355X).
//
// The whole batch is one kernel launch with no host round trip between
// decoding steps.  Each request has a leader workgroup of 1024 threads (16
// wave64) that runs every step -- parent table, expansion, validation,
// pruning -- and helper workgroups that join the expansion of the steps
// with many work items: each claims its slice of such a step, and the
// leader takes over slices no helper has claimed, so the launch needs no
// co-residency guarantee.  Semantics are those of the reference CPU path
// LoudsTrie::tbs (lib/marisa/grimoire/trie/louds-trie.cc:75-177):
//
//  * cur is processed parent by parent in ascending (norm, node id) order and
//    each parent's proposals in index order; a parent is a "link parent" when
//    terminal(n) and |KB| > |Q| (louds-trie.cc:151-153), and then only the
//    token KB(n)[|Q|] can extend it (louds-trie.cc:91-102);
//  * otherwise the child whose first edge token equals the proposal is
//    taken (predictive_find_child, louds-trie.cc:810-856); it goes to
//    `selected` if terminal with |KB| == |Q| and always to `next`
//    (louds-trie.cc:103-108);
//  * `next` and `selected` are bounded heaps (candidates.h:32-80).
//
// The bounded heaps are reproduced exactly without a sequential heap.  For
// pushes e_1..e_n (arrival order) into a heap of capacity M with keys
// (norm, node id) -- node ids are distinct inside every heap -- the final
// content is:
//    n <= M: everything;
//    else with v* = the M-th largest norm, G = #{norm > v*}, r = M - G:
//      all items with norm > v*, plus, among A = the norm == v* items that
//      are among the first M items (in arrival order) of {norm >= v*}, the r
//      with the largest node ids.
// Arrival order is (parent rank in ascending (norm, node), proposal index);
// it is only computed when the boundary norm v* is tied (E > r) or when
// early exit truncates `selected` to the first F pushes.
//
// Scores: s is the f64 sum of f32 logps (agent.cc:36); norm = s * lnf[|Q|]
// with lnf[d] = pow(6 / (5 + d), alpha) computed on the host with the same
// libm call as the reference (agent.h:69-72), so norms are bit-identical.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <mutex>

#include "coherent.h"
#include "tbs_kernel.h"

namespace ftk {

constexpr int kBlock = 1024;
constexpr int kWaves = kBlock / 64;
// selection: bins of the first histogram and the keys one bin may hold in LDS
constexpr int kWideBits = 11;
constexpr int kWideBins = 1 << kWideBits;
constexpr int kBinCap = 2048;
constexpr int kKeepCap = 4096;
// expansion: pushes a workgroup buffers in LDS before one global append
constexpr int kPushCap = 1024;
constexpr int kPushSelCap = 256;
// expansion: an LDS hash of the row, token -> sorted position (linear
// probing, load <= 1/2), built for rows of up to kRowHashMaxK proposals
constexpr int kRowHashLog2 = 12;
constexpr int kRowHash = 1 << kRowHashLog2;
constexpr uint32_t kRowHashMaxK = kRowHash / 2;
constexpr uint32_t kRowHashEmpty = 0xFFFFFFFFu;
// the leader hashes the row for steps of at least this many work items (a
// smaller step does too few lookups to repay the build)
constexpr uint32_t kRowHashMinWork = 2048;
// the single-wave tail: at most this many steps' rows in LDS per round,
// and the bits that mark a token its row does not hold (a NaN, which no
// staged logp is)
constexpr uint32_t kTailMaxRows = 32;
constexpr uint32_t kAbsent = 0xFFFFFFFFu;

struct alignas(16) Smem {
  // counters, flags and small arrays first: their LDS addresses fit the
  // immediate offset of one base register
  // expansion: this workgroup's push counts and list bases
  uint32_t lq_next, lq_sel, gb_next, gb_sel;
  // selection
  uint32_t hist[256];
  uint64_t red64[2 * kWaves];
  uint32_t wsum[kWaves];
  uint32_t sel_digit, sel_cum, sel_cnt;
  uint32_t n_keep, collected;
  uint32_t n_next, n_sel, n_out, overflow;
  uint32_t status;
  unsigned long long cnt_parents, cnt_children, cnt_probes;
  unsigned long long bcast;
  uint32_t hstep[7];  // a helper's view of the posted step (+ whether it
                      // took its slice)
  uint32_t lead_flag;   // the leader's broadcast of a decision of thread 0
  uint32_t n_stolen;    // helper slices the leader took over this step
  uint16_t stolen[256];
  uint32_t multi_item;  // some parent of the step has other than one item
  // the single-wave tail (tiny steps): where it stopped, for every thread
  uint32_t tiny_t, tiny_ncur, tiny_nS, tiny_hist, tiny_done, tiny_handback;
  unsigned long long tiny_cands, tiny_ticks;
  uint32_t par_w;       // work items of a step with at most 64 parents
  uint32_t w_children, w_probes;
  // where the leader writes its results: out_host's block of the request,
  // or null for `out` (kept here rather than in registers through the steps)
  unsigned long long res_host;
  // a row longer than the LDS row arrays (K > kMaxLdsTopk) stays in the
  // device stage: the step's row there (tokens, logps), read only by the
  // lookups of such a row
  unsigned long long grow_id, grow_lp;
  // expansion: the current proposal row in ascending token order
  alignas(16) uint32_t row_id[kMaxLdsTopk];
  float row_lp[kMaxLdsTopk];
  // expansion: the parent table of up to kBlock parents (LDS copy): the
  // work-item prefix, first child / table, degree / token / table size,
  // node, lookup mode, score and history record.  Not aliased: the emit of
  // a step writes the next step's table while the selection's arrays are
  // still read.
  uint32_t woff[kBlock + 1];
  uint32_t p_c0[kBlock];
  uint32_t p_aux[kBlock];
  uint32_t p_node[kBlock];
  uint32_t p_hist[kBlock];
  double p_s[kBlock];
  uint8_t p_mode[kBlock];
  // link parents (kNoCursor otherwise): index in tail[] of the pending token
  uint32_t p_lp[kBlock];
  // the leader's own per-parent data for its emit, which overwrites the
  // table above with the next step's, copied by the parent phase: score,
  // history record and, for a link parent that stays one on its own edge,
  // its string depth (else 0) and the tail index of its pending token; the
  // expansion of that parent adds its next pending token (else kNoToken)
  double x_s[kBlock];
  uint32_t x_hist[kBlock];
  uint32_t x_tok[kBlock];
  uint32_t x_tc[kBlock];
  uint16_t x_sd[kBlock];
  union {
    // expansion: the row hash (see kRowHash)
    struct {
      uint32_t rh_tok[kRowHash];
      uint16_t rh_pos[kRowHash];
    };
    // selection: positions of the kept candidates, and the keys and
    // positions of one histogram bin
    struct {
      uint32_t keep_idx[kKeepCap];
      uint64_t bin_key[kBinCap];
      uint32_t bin_idx[kBinCap];
    };
    // selection: wide histogram (done before keep_idx is filled)
    uint32_t whist[kWideBins];
    // the single-wave tail, per round of steps whose rows are in LDS: the
    // pending token of hypothesis (lane) j at the round's step r in
    // tl_tok[r * 64 + j] (kNoToken where it is not read ahead), the bits of
    // its logp in that step's row in tl_x[r * 64 + j] (kAbsent when the
    // row does not hold it), the steps' beam widths, and each hypothesis's
    // last token and parent record between rounds
    struct {
      uint32_t tl_tok[(kTailMaxRows + 1) * 64];
      uint32_t tl_x[kTailMaxRows * 64];
      uint32_t tl_beams[kTailMaxRows];
      uint32_t tl_rtok[64];
      uint32_t tl_rphist[64];
    };
  };
  // expansion: this workgroup's pushes, appended to the request's lists at
  // the end of its share of the step
  NextRec push_next[kPushCap];
  SelRec push_sel[kPushSelCap];
};
// rank scratch aliases the row arrays (used after expansion only)
constexpr int kRankChunk = 1024;
static_assert(offsetof(Smem, row_id) % 16 == 0 && offsetof(Smem, row_lp) % 16 == 0,
              "rank scratch is read 16 bytes at a time");
static_assert(kRankChunk == kBlock, "a thread's own rank entry sits in its own chunk");
static_assert(kRankChunk % 16 == 0, "rank chunks hold whole count_before rounds");

// How many of the m LDS entries (rk_key[q], rk_node[q]) order before (k, n)
// by (key, node).  Every thread reads the same entries (broadcast reads),
// 2 * P keys and their nodes per iteration through 3 * P / 2 16-byte loads
// issued together, compared without branches (a branch per equal key made
// every wave wait for all its outstanding reads).
template <int P>
__device__ __forceinline__ uint32_t count_before(const uint64_t* rk_key,
                                                 const uint32_t* rk_node, uint32_t m,
                                                 uint64_t k, uint32_t n) {
  // m is a multiple of 2 * P; entries past the real ones are kRankPad keys
  uint32_t c = 0;
  for (uint32_t q = 0; q < m; q += 2 * P) {
    asm volatile("" : "+v"(k), "+v"(n));
    ulonglong2 v[P];
    uint4 nd[P / 2];
#pragma unroll
    for (int u = 0; u < P; ++u) v[u] = *(const ulonglong2*)&rk_key[q + 2 * u];
#pragma unroll
    for (int u = 0; u < P / 2; ++u) nd[u] = *(const uint4*)&rk_node[q + 4 * u];
#pragma unroll
    for (int u = 0; u < P / 2; ++u) {
      const ulonglong2 a = v[2 * u], b = v[2 * u + 1];
      c += (a.x < k) | ((a.x == k) & (nd[u].x < n));
      c += (a.y < k) | ((a.y == k) & (nd[u].y < n));
      c += (b.x < k) | ((b.x == k) & (nd[u].z < n));
      c += (b.y < k) | ((b.y == k) & (nd[u].w < n));
    }
  }
  return c;
}
// rank-scratch filler past the real entries: orders after every real key
// (norm_key of a finite score is below it) and never counts
constexpr uint64_t kRankPad = ~0ull;

// lookup mode word of a parent: the mode, and whether the parent sits at
// string depth t (only then can a child -- one token long, terminal --
// close a key of length t + 1)
constexpr uint32_t kModeMask = 0x0Fu;
constexpr uint32_t kModeDepthOk = 0x80u;
// a hashed parent whose table has fingerprint filtering (kWideFiltered)
constexpr uint32_t kModeFiltered = 0x40u;

enum : uint8_t {
  M_NONE = 0,
  M_LP_NEXT = 1,
  M_LP_SEL = 2,
  M_SCAN = 3,
  M_SEARCH = 4,
  M_HASH = 5,
  M_DENSE = 6  // the root at step 0: its children from the root directory
};

__device__ __forceinline__ uint64_t norm_key(double v) {
  // order-preserving map of a double to uint64; -0.0 and +0.0 are equal
  if (v == 0.0) v = 0.0;
  uint64_t b = (uint64_t)__double_as_longlong(v);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63; }

// whether some byte of v is zero
__device__ __forceinline__ bool has_zero_byte(uint64_t v) {
  return ((v - 0x0101010101010101ull) & ~v & 0x8080808080808080ull) != 0;
}

__device__ __forceinline__ uint32_t lanemask_lt_count(uint64_t m) {
  const uint32_t lane = lane_id();
  return (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
}

// Wave-aggregated append: returns this lane's slot (valid if `want`).
__device__ __forceinline__ uint32_t wave_append(bool want, uint32_t* ctr) {
  const uint64_t m = __ballot(want);
  if (m == 0) return 0;
  const int leader = __ffsll((unsigned long long)m) - 1;
  uint32_t base = 0;
  if ((int)lane_id() == leader) base = atomicAdd(ctr, (uint32_t)__popcll(m));
  base = (uint32_t)__builtin_amdgcn_readlane((int)base, leader);
  return base + lanemask_lt_count(m);
}

// wave_append on one half of a 64-bit counter pair (high: the upper 32
// bits), one 64-bit add for the wave; the halves never carry into each
// other (each stays below 2^32).
__device__ __forceinline__ uint32_t wave_append_half(bool want, unsigned long long* ctr,
                                                     bool high) {
  const uint64_t m = __ballot(want);
  if (m == 0) return 0;
  const int leader = __ffsll((unsigned long long)m) - 1;
  uint32_t base = 0;
  if ((int)lane_id() == leader) {
    const unsigned long long old =
        atomicAdd(ctr, (unsigned long long)__popcll(m) << (high ? 32 : 0));
    base = high ? (uint32_t)(old >> 32) : (uint32_t)old;
  }
  base = (uint32_t)__builtin_amdgcn_readlane((int)base, leader);
  return base + lanemask_lt_count(m);
}

// Inclusive scan of x over the 64 lanes of a wave; every lane must be
// active.  Lane moves are DPP operands of the adds (no LDS round trip):
// shifts by 1, 2, 4, 8 within each row of 16 lanes, then lane 15 of each
// row into the next row and lane 31 into the upper half.
template <int Ctrl>
__device__ __forceinline__ uint32_t dpp_move(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, Ctrl, 0xf, 0xf, false);
}
template <int Ctrl>
__device__ __forceinline__ uint64_t dpp_move64(uint64_t x) {
  return ((uint64_t)dpp_move<Ctrl>((uint32_t)(x >> 32)) << 32) | dpp_move<Ctrl>((uint32_t)x);
}
__device__ __forceinline__ uint64_t readlane64(uint64_t x, int lane) {
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), lane) << 32) |
         (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, lane);
}
// min (or max) of v over each 16-lane row, in every lane of the row:
// rotations by 8, 4, 2, 1
__device__ __forceinline__ uint64_t row_reduce64(uint64_t v, bool take_min) {
  uint64_t y = dpp_move64<0x128>(v);  // row_ror:8
  v = take_min ? min(v, y) : max(v, y);
  y = dpp_move64<0x124>(v);           // row_ror:4
  v = take_min ? min(v, y) : max(v, y);
  y = dpp_move64<0x122>(v);           // row_ror:2
  v = take_min ? min(v, y) : max(v, y);
  y = dpp_move64<0x121>(v);           // row_ror:1
  return take_min ? min(v, y) : max(v, y);
}
// Sum of x over the 64 lanes of a wave, in every lane; every lane must be
// active.  Rotations by 8, 4, 2, 1 within each row of 16 lanes, then the
// four row sums.
__device__ __forceinline__ uint32_t wave_sum(uint32_t x) {
  x += dpp_move<0x128>(x);  // row_ror:8
  x += dpp_move<0x124>(x);  // row_ror:4
  x += dpp_move<0x122>(x);  // row_ror:2
  x += dpp_move<0x121>(x);  // row_ror:1
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 0) +
         (uint32_t)__builtin_amdgcn_readlane((int)x, 16) +
         (uint32_t)__builtin_amdgcn_readlane((int)x, 32) +
         (uint32_t)__builtin_amdgcn_readlane((int)x, 48);
}
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  const uint32_t lane = lane_id(), rl = lane & 15u;
  uint32_t y = dpp_move<0x111>(x);  // row_shr:1
  if (rl >= 1u) x += y;
  y = dpp_move<0x112>(x);           // row_shr:2
  if (rl >= 2u) x += y;
  y = dpp_move<0x114>(x);           // row_shr:4
  if (rl >= 4u) x += y;
  y = dpp_move<0x118>(x);           // row_shr:8
  if (rl >= 8u) x += y;
  y = dpp_move<0x142>(x);           // row_bcast:15
  if ((lane & 31u) >= 16u) x += y;
  y = dpp_move<0x143>(x);           // row_bcast:31
  if (lane >= 32u) x += y;
  return x;
}

// Exclusive block scan of v over all kBlock threads.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* total, Smem& sm) {
  const uint32_t lane = lane_id(), wave = threadIdx.x >> 6;
  const uint32_t x = wave_incl_scan(v);
  if (lane == 63) sm.wsum[wave] = x;
  __syncthreads();
  if (wave == 0) {
    const uint32_t w = lane < (uint32_t)kWaves ? sm.wsum[lane] : 0;
    const uint32_t z = wave_incl_scan(w);
    if (lane < (uint32_t)kWaves) sm.wsum[lane] = z - w;  // exclusive
    if (lane == (uint32_t)kWaves - 1) sm.sel_cum = z;      // grand total
  }
  __syncthreads();
  const uint32_t r = x - v + sm.wsum[wave];
  *total = sm.sel_cum;
  __syncthreads();
  return r;
}

// Adds 1 to hist[digit] for every active lane; lanes of a wave that agree on
// the digit are merged into one LDS atomic.
__device__ __forceinline__ void hist_add(bool act, uint32_t digit,
                                         uint32_t* hist) {
  const uint64_t am = __ballot(act);
  if (am == 0) return;
  const int leader = __ffsll((unsigned long long)am) - 1;
  const uint32_t d0 = (uint32_t)__builtin_amdgcn_readlane((int)digit, leader);
  const uint64_t same = __ballot(act && digit == d0);
  if (same == am) {
    if ((int)lane_id() == leader) atomicAdd(&hist[d0], (uint32_t)__popcll(am));
  } else if (act) {
    atomicAdd(&hist[digit], 1u);
  }
}

// Picks the bin holding the `rem`-th smallest item (1-based) from
// sm.hist[256]; writes sel_digit / sel_cum (items in lower bins) / sel_cnt.
__device__ __forceinline__ void hist_pick(uint32_t rem, Smem& sm) {
  if (threadIdx.x < 64) {
    const uint32_t lane = threadIdx.x;
    const uint32_t h0 = sm.hist[4 * lane], h1 = sm.hist[4 * lane + 1],
                   h2 = sm.hist[4 * lane + 2], h3 = sm.hist[4 * lane + 3];
    const uint32_t own = h0 + h1 + h2 + h3;
    const uint32_t x = wave_incl_scan(own);
    const uint64_t hit = __ballot(x >= rem);
    const int first = hit ? __ffsll((unsigned long long)hit) - 1 : 63;
    if ((int)lane == first) {
      uint32_t cum = x - own;
      uint32_t b = 4 * lane;
      const uint32_t hs[4] = {h0, h1, h2, h3};
      int i = 0;
      for (; i < 3; ++i) {
        if (cum + hs[i] >= rem) break;
        cum += hs[i];
      }
      sm.sel_digit = b + i;
      sm.sel_cum = cum;
      sm.sel_cnt = hs[i];
    }
  }
  __syncthreads();
}

// Radix selection of the `need`-th smallest key (1-based) among items
// i < n with filt(i).  Returns it; *eq = items equal to it, *rem = how many
// of those are needed to reach `need`.
template <typename KeyT, typename GetKey, typename Filt>
__device__ __forceinline__ KeyT radix_kth(uint32_t n, uint32_t need, GetKey gk, Filt filt,
                          Smem& sm, uint32_t* eq, uint32_t* rem_out) {
  constexpr int kBits = (int)sizeof(KeyT) * 8;
  KeyT prefix = 0, mask = 0;
  uint32_t rem = need, cnt = 0;
  for (int shift = kBits - 8; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += kBlock) sm.hist[i] = 0;
    __syncthreads();
    for (uint32_t base = 0; base < n; base += kBlock) {
      const uint32_t i = base + threadIdx.x;
      bool act = false;
      uint32_t dg = 0;
      if (i < n && filt(i)) {
        const KeyT k = gk(i);
        if ((k & mask) == prefix) {
          act = true;
          dg = (uint32_t)((k >> shift) & 0xFF);
        }
      }
      hist_add(act, dg, sm.hist);
    }
    __syncthreads();
    hist_pick(rem, sm);
    prefix |= (KeyT)sm.sel_digit << shift;
    mask |= (KeyT)0xFF << shift;
    rem -= sm.sel_cum;
    cnt = sm.sel_cnt;
    __syncthreads();
  }
  *eq = cnt;
  *rem_out = rem;
  return prefix;
}

// Calls f(i, valid, gk(i)) for every item slot i = base + tid of this
// thread (n >= 1 when the loop runs), with U items per thread in flight:
// the reads are unconditional (a slot past the end re-reads item n - 1) so
// that all of them are issued before the first is waited for.
template <uint32_t U = 4, typename GetKey, typename F>
__device__ __forceinline__ void visit_keys(uint32_t n, GetKey gk, F f) {
  for (uint32_t base = 0; base < n; base += U * kBlock) {
    uint64_t k[U];
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t i = base + u * kBlock + threadIdx.x;
      k[u] = gk(min(i, n - 1u));
    }
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t i = base + u * kBlock + threadIdx.x;
      f(i, i < n, k[u]);
    }
  }
}

// The `need`-th smallest (1-based) of n 64-bit keys gk(i): one pass for the
// key range, one histogram pass of
// kWideBits-bit digits starting at the highest bit in which keys differ,
// then the keys of the chosen bin are gathered into LDS (if they fit; else
// another histogram pass narrows the prefix) and the remaining bits are
// resolved there.  *eq = keys equal to the result, *rem = how many of those
// are needed to reach `need`.
//
// With `collect`, the gather pass also lists, in sm.keep_idx, the items in
// bins below the chosen one (sm.n_keep of them) and keeps the chosen bin's
// positions in sm.bin_idx, and sm.collected says that it ran: then a bounded
// selection needs no further pass over the list.
template <typename GetKey>
__device__ __forceinline__ uint64_t kth_u64(uint32_t n, uint32_t need, GetKey gk, Smem& sm,
                            uint32_t* eq, uint32_t* rem_out, bool have_range,
                            uint64_t rmin, uint64_t rmax, bool collect = false) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  if (tid == 0) sm.collected = 0;
  // key range: given (bounds of every key), or one pass
  uint64_t mn = rmin, mx = rmax;
  if (!have_range) {
    mn = ~0ull;
    mx = 0;
    visit_keys(n, gk, [&](uint32_t, bool ok, uint64_t k) {
      if (ok) {
        mn = min(mn, k);
        mx = max(mx, k);
      }
    });
    mn = row_reduce64(mn, true);
    mx = row_reduce64(mx, false);
    mn = min(min(readlane64(mn, 0), readlane64(mn, 16)),
             min(readlane64(mn, 32), readlane64(mn, 48)));
    mx = max(max(readlane64(mx, 0), readlane64(mx, 16)),
             max(readlane64(mx, 32), readlane64(mx, 48)));
    if (lane == 0) {
      sm.red64[wave] = mn;
      sm.red64[kWaves + wave] = mx;
    }
    __syncthreads();
    // every wave combines the partials in one read: lanes 0..15 hold the
    // waves' minima, lanes 16..31 their maxima
    static_assert(kWaves == 16, "one DPP row per partial set");
    const uint64_t v = row_reduce64(sm.red64[lane & 31u], lane < 16u);
    mn = readlane64(v, 0);
    mx = readlane64(v, 16);
    __syncthreads();
  }
  if (mn == mx) {
    *eq = n;
    *rem_out = need;
    return mn;
  }
  // Digits are taken from the offset k - mn (order-preserving for k >= mn):
  // a range that straddles a power of two in the raw key (an exponent
  // boundary of the doubles behind the keys) would otherwise put most keys
  // in a few bins of the first window.  Offsets above bit `top` are zero.
  const uint64_t base = mn;
  int top = 63 - __clzll((long long)(mx - mn));
  uint64_t prefix = 0;
  uint32_t rem = need;
  uint32_t cnt = n;
  for (;;) {
    // histogram of the kWideBits bits at and below `top`
    const int sh = top >= kWideBits - 1 ? top - (kWideBits - 1) : 0;
    const uint32_t nb = 1u << (top - sh + 1);
    const uint64_t hi_mask = (top >= 63) ? 0ull : ~((2ull << top) - 1ull);
    for (uint32_t i = tid; i < nb; i += kBlock) sm.whist[i] = 0;
    __syncthreads();
    visit_keys<6>(n, gk, [&](uint32_t, bool ok, uint64_t k) {
      const uint64_t o = k - base;
      const bool act = ok && (o & hi_mask) == prefix;
      // (the wide bins spread a wave's keys: one LDS add a key, without
      // hist_add's check for a wave-uniform digit)
      if (act) atomicAdd(&sm.whist[(uint32_t)((o >> sh) & (nb - 1))], 1u);
    });
    __syncthreads();
    // the bin holding the rem-th key: each thread owns nb / kBlock bins
    {
      const uint32_t per = (nb + kBlock - 1) / kBlock;
      uint32_t own = 0;
      for (uint32_t q = 0; q < per; ++q) {
        const uint32_t b = tid * per + q;
        if (b < nb) own += sm.whist[b];
      }
      uint32_t tot;
      const uint32_t before = block_excl_scan(own, &tot, sm);
      if (before < rem && rem <= before + own) {
        uint32_t c = before;
        for (uint32_t q = 0; q < per; ++q) {
          const uint32_t b = tid * per + q;
          const uint32_t h = sm.whist[b];
          if (c + h >= rem) {
            sm.sel_digit = b;
            sm.sel_cum = c;
            sm.sel_cnt = h;
            break;
          }
          c += h;
        }
      }
      __syncthreads();
    }
    prefix |= (uint64_t)sm.sel_digit << sh;
    rem -= sm.sel_cum;
    cnt = sm.sel_cnt;
    __syncthreads();
    if (sh == 0) {
      *eq = cnt;
      *rem_out = rem;
      return prefix + base;
    }
    top = sh - 1;
    if (cnt <= (uint32_t)kBinCap) break;
  }
  // gather the keys of the chosen bin, then finish in LDS
  {
    const uint64_t hi_mask = ~((2ull << top) - 1ull);
    if (tid == 0) {
      sm.n_out = 0;
      sm.n_keep = 0;
      sm.collected = collect ? 1u : 0u;
    }
    __syncthreads();
    // U keys per thread per round, all read before the first wait; each
    // list gets one LDS append per wave per round (slots in the order
    // (key slot u, lane))
    constexpr uint32_t U = 6;
    const uint64_t lt = (1ull << lane) - 1ull;
    for (uint32_t b0 = 0; b0 < n; b0 += U * kBlock) {
      uint64_t k[U];
#pragma unroll
      for (uint32_t u = 0; u < U; ++u) k[u] = gk(min(b0 + u * kBlock + tid, n - 1u));
      uint32_t fa = 0, fb = 0, ca = 0, cb = 0;
#pragma unroll
      for (uint32_t u = 0; u < U; ++u) {
        const bool ok = b0 + u * kBlock + tid < n;
        const uint64_t hk = (k[u] - base) & hi_mask;
        const bool act = ok && hk == prefix;
        const bool below = collect && ok && hk < prefix;
        fa |= (uint32_t)act << u;
        fb |= (uint32_t)below << u;
        ca += (uint32_t)__popcll(__ballot(act));
        cb += (uint32_t)__popcll(__ballot(below));
      }
      uint32_t ba = 0, bb = 0;
      if (lane == 0) {
        if (ca) ba = atomicAdd(&sm.n_out, ca);
        if (cb) bb = atomicAdd(&sm.n_keep, cb);
      }
      ba = (uint32_t)__builtin_amdgcn_readfirstlane((int)ba);
      bb = (uint32_t)__builtin_amdgcn_readfirstlane((int)bb);
#pragma unroll
      for (uint32_t u = 0; u < U; ++u) {
        const uint32_t i = b0 + u * kBlock + tid;
        const uint64_t ma = __ballot((fa >> u) & 1u), mb = __ballot((fb >> u) & 1u);
        if ((fa >> u) & 1u) {
          const uint32_t o = ba + (uint32_t)__popcll(ma & lt);
          if (o < (uint32_t)kBinCap) {
            sm.bin_key[o] = k[u];
            sm.bin_idx[o] = i;
          }
        }
        if ((fb >> u) & 1u) {
          const uint32_t q = bb + (uint32_t)__popcll(mb & lt);
          if (q < (uint32_t)kKeepCap) sm.keep_idx[q] = i;
        }
        ba += (uint32_t)__popcll(ma);
        bb += (uint32_t)__popcll(mb);
      }
    }
    __syncthreads();
  }
  // cnt keys in LDS share the prefix above `top`: 8-bit digits downwards,
  // until the boundary bin holds one key
  for (;;) {
    const int s0 = top >= 7 ? top - 7 : 0;
    const uint32_t nb = 1u << (top - s0 + 1);
    const uint64_t msk = ~((2ull << top) - 1ull);
    for (uint32_t i = tid; i < 256; i += kBlock) sm.hist[i] = 0;
    __syncthreads();
    for (uint32_t i = tid; i < cnt; i += kBlock) {
      const uint64_t o = sm.bin_key[i] - base;
      const bool act = (o & msk) == prefix;
      hist_add(act, (uint32_t)((o >> s0) & (nb - 1)), sm.hist);
    }
    __syncthreads();
    hist_pick(rem, sm);
    prefix |= (uint64_t)sm.sel_digit << s0;
    rem -= sm.sel_cum;
    const uint32_t c2 = sm.sel_cnt;
    __syncthreads();
    if (s0 == 0) {
      *eq = c2;
      *rem_out = rem;
      return prefix + base;
    }
    top = s0 - 1;
    if (c2 == 1) {
      // one key left in the bin: it is the answer
      const uint64_t m2 = ~((2ull << top) - 1ull);
      for (uint32_t i = tid; i < cnt; i += kBlock) {
        const uint64_t k = sm.bin_key[i];
        if (((k - base) & m2) == prefix) sm.red64[0] = k;
      }
      __syncthreads();
      const uint64_t r = sm.red64[0];
      __syncthreads();
      *eq = 1;
      *rem_out = 1;
      return r;
    }
  }
}

// Thresholds of the bounded-heap emulation (see the file comment).
struct Bound {
  uint64_t vkey;   // boundary key
  uint32_t tie;    // 1 if the boundary class is cut
  uint32_t astar;  // arrival cutoff (tie only)
  uint32_t nustar; // node-id cutoff (tie only)
  uint32_t all;    // 1 if everything survives
};

__device__ __forceinline__ bool bound_keep(const Bound& b, uint64_t key,
                                           uint32_t arr, uint32_t node) {
  if (b.all) return true;
  if (key > b.vkey) return true;
  if (key != b.vkey) return false;
  if (!b.tie) return true;
  return arr <= b.astar && node >= b.nustar;
}

// Bounded heap of capacity M over n items (see the file comment).  key(i),
// arr(i) and node(i) read the items; arr() is only called on the tie path,
// after `need_ranks()` has made parent ranks available.
// With `have_range`, every key(i) lies in [kmin, kmax].  With `collect`,
// see kth_u64 (the items with a key above the boundary bin are listed).
template <typename GetKey, typename GetArr, typename GetNode, typename Ranks>
__device__ __forceinline__ Bound bounded_select(uint32_t n, uint32_t M, GetKey key,
                                GetArr arr, GetNode node, Ranks need_ranks,
                                Smem& sm, bool have_range = false,
                                uint64_t kmin = 0, uint64_t kmax = ~0ull,
                                bool collect = false) {
  Bound b{0, 0, 0, 0, 0};
  if (n <= M) {
    b.all = 1;
    return b;
  }
  uint32_t eq, rem;
  // M-th largest key == M-th smallest of ~key
  const uint64_t nk = kth_u64(n, M, [&](uint32_t i) { return ~key(i); }, sm, &eq,
                              &rem, have_range, ~kmax, ~kmin, collect);
  b.vkey = ~nk;
  if (eq == rem) return b;  // the whole boundary class fits
  b.tie = 1;
  need_ranks();
  const uint64_t vk = b.vkey;
  // first M of {key >= v*} in arrival order
  uint32_t eq2, rem2;
  b.astar = radix_kth<uint32_t>(
      n, M, [&](uint32_t i) { return arr(i); },
      [&](uint32_t i) { return key(i) >= vk; }, sm, &eq2, &rem2);
  const uint32_t as = b.astar;
  // the `rem` largest node ids of A
  uint32_t eq3, rem3;
  const uint32_t nn = radix_kth<uint32_t>(
      n, rem, [&](uint32_t i) { return ~node(i); },
      [&](uint32_t i) { return key(i) == vk && arr(i) <= as; }, sm, &eq3,
      &rem3);
  b.nustar = ~nn;
  return b;
}

// Position of the i-th zero bit (0-based) of the LOUDS bits (see LoudsDir).
__device__ __forceinline__ uint64_t louds_select0(const KArgs& a, uint32_t i) {
  const uint32_t k = i / kLoudsSel;
  uint32_t lo = a.louds_s[k], hi = a.louds_s[k + 1];
  // the last block b in [lo, hi] with louds_z[b] <= i
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) >> 1;
    if (a.louds_z[mid] <= i) lo = mid; else hi = mid - 1;
  }
  uint32_t r = i - a.louds_z[lo];
  // the word holding it: walk the block's words, two per 16-byte read,
  // while r is past their zeros (the block holds zero i, so the walk stops
  // inside it); one read at a time keeps few registers live
  const uint4* line = (const uint4*)(a.louds_words + (uint64_t)lo * (kLoudsBlockBits / 64));
  uint32_t wi = 0;
  uint64_t z = 0;
  for (uint32_t h = 0; h < kLoudsBlockBits / 128; ++h) {
    const uint4 q = line[h];
    const uint64_t z0 = ~((uint64_t)q.x | ((uint64_t)q.y << 32));
    const uint64_t z1 = ~((uint64_t)q.z | ((uint64_t)q.w << 32));
    const uint32_t c0 = (uint32_t)__popcll(z0);
    if (r < c0) {
      z = z0;
      wi = 2 * h;
      break;
    }
    r -= c0;
    const uint32_t c1 = (uint32_t)__popcll(z1);
    if (r < c1 || h + 1 == kLoudsBlockBits / 128) {
      z = z1;
      wi = 2 * h + 1;
      break;
    }
    r -= c1;
  }
  // the r-th set bit of z, by halving
  uint32_t pos = 0;
#pragma unroll
  for (int width = 32; width >= 1; width >>= 1) {
    const uint64_t low = width == 64 ? ~0ull : ((1ull << width) - 1ull);
    const uint32_t c = (uint32_t)__popcll(z & low);
    if (r >= c) {
      r -= c;
      z >>= width;
      pos += (uint32_t)width;
    }
  }
  return (uint64_t)lo * kLoudsBlockBits + (uint64_t)wi * 64u + pos;
}

// First child id and degree of `node` from the LOUDS directory.
__device__ __forceinline__ void louds_children(const KArgs& a, uint32_t node, uint32_t* c0,
                                               uint32_t* deg) {
  const uint64_t z1 = louds_select0(a, node);
  const uint64_t z0 = node ? louds_select0(a, node - 1) : ~0ull;  // select0(-1) = -1
  *c0 = (uint32_t)(z0 + 2u - node);
  *deg = (uint32_t)(z1 - z0 - 1u);
}

// KB(n)[j] for a link parent: walk up until the edge that covers position j.
__device__ __forceinline__ uint32_t kb_token(const KArgs& a, uint32_t n, ft_node_rec r,
                             uint32_t j, uint32_t* err) {
  for (int guard = 0; guard < 65536; ++guard) {
    const uint32_t sd = r.meta & FT_META_DEPTH_MASK;
    const uint32_t el = (r.meta >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
    const uint32_t start = sd - el;
    if (j >= start) {
      if (r.meta & FT_META_LINK) return a.tail[(uint64_t)r.tail_off + (j - start)];
      return r.first_tok;
    }
    if (n == 0) break;
    n = a.parent[n];
    r = a.recs[n];
  }
  *err = 1;
  return 0xFFFFFFFFu;
}

// A parent's entry in the parent table of step t: lookup mode (with
// kModeDepthOk), first child or hash-table offset (a link parent: its string
// depth), degree / pending token / log2 table size, its number of work
// items, and for a link parent whose pending token lies on its own edge the
// index of that token in tail[] (else kNoCursor).
constexpr uint32_t kNoCursor = 0xFFFFFFFFu;
constexpr uint32_t kNoToken = 0xFFFFFFFFu;
struct ParEntry {
  uint32_t c0, aux, mode, work, lp;
};
template <bool kLouds>
__device__ __forceinline__ ParEntry parent_entry(const KArgs& a, uint32_t node, uint32_t t,
                                                 uint32_t K, uint32_t* err) {
  // the node's home group in the table directory is read with its record
  // (in bounds for any node), not after it: a node with a table then costs
  // one dependent read, not two.  Buffer loads, so that no branch on
  // a.wdir sits between the two reads (a directory of 0 bytes when there is
  // none: its reads return 0 and touch no memory).
  const uint32_t dmask = a.wdir ? (1u << a.wdir_log2) - 1u : 0u;
  uint32_t g = a.wdir ? fib_slot(node, a.wdir_log2) : 0u;
  const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<WideDirGroup*>(a.wdir), 0,
      a.wdir ? (int)((dmask + 1u) * sizeof(WideDirGroup)) : 0, 0x00020000);
  const int dof = (int)(g * sizeof(WideDirGroup));
  uint4 nd, off, lgf;
  {
    const auto v0 = __builtin_amdgcn_raw_buffer_load_b128(drs, dof, 0, 0);
    const auto v1 = __builtin_amdgcn_raw_buffer_load_b128(drs, dof + 16, 0, 0);
    const auto v2 = __builtin_amdgcn_raw_buffer_load_b128(drs, dof + 32, 0, 0);
    nd = make_uint4(v0[0], v0[1], v0[2], v0[3]);
    off = make_uint4(v1[0], v1[1], v1[2], v1[3]);
    lgf = make_uint4(v2[0], v2[1], v2[2], v2[3]);
  }
  const ft_node_rec r = a.recs[node];
  uint32_t c0, deg;
  if constexpr (kLouds) {
    louds_children(a, node, &c0, &deg);
  } else {
    c0 = r.child_begin;
    deg = a.recs[node + 1].child_begin - c0;
  }
  const uint32_t sd = r.meta & FT_META_DEPTH_MASK;
  ParEntry e{c0, deg, (uint32_t)M_NONE, 0u, kNoCursor};
  if ((r.meta & FT_META_TERMINAL) && sd > t) {
    // link parent: only KB(n)[|Q|] extends it (louds-trie.cc:91-102)
    e.aux = kb_token(a, node, r, t, err);
    e.mode = (t + 1 == sd) ? M_LP_SEL : M_LP_NEXT;
    e.work = 1;
    e.c0 = sd;
    const uint32_t el = (r.meta >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
    if ((r.meta & FT_META_LINK) && t + el >= sd) e.lp = r.tail_off + (t + el - sd);
  } else if (deg == 0) {
    e.mode = M_NONE;
  } else if (deg <= a.scan_limit) {
    e.mode = M_SCAN;
    e.work = deg;
  } else {
    e.mode = M_SEARCH;
    e.work = K;
    if (a.wdir && deg >= a.wide_min) {
      // this node has a table: find it in the directory, a 64-B group of
      // entries per read from the home group on (read above)
      for (uint32_t it = 0; it <= dmask; ++it) {
        if (it) {
          const uint4* gp = (const uint4*)&a.wdir[g];
          nd = gp[0];
          off = gp[1];
          lgf = gp[2];
        }
        const uint32_t nds[4] = {nd.x, nd.y, nd.z, nd.w};
        const uint32_t offs[4] = {off.x, off.y, off.z, off.w};
        const uint32_t lgfs[4] = {lgf.x, lgf.y, lgf.z, lgf.w};
        bool found = false, has_free = false;
#pragma unroll
        for (int k = 0; k < (int)kDirSlots; ++k) {
          if (nds[k] == node) {
            found = true;
            e.mode = M_HASH | (((lgfs[k] >> 8) & kWideFiltered) ? kModeFiltered : 0u);
            e.aux = lgfs[k] & 0xFFu;
            e.c0 = offs[k];
          }
          has_free = has_free || nds[k] == kEmpty;
        }
        if (found || has_free) break;
        g = (g + 1) & dmask;
      }
    }
  }
  if ((e.mode & kModeMask) == M_SCAN || (e.mode & kModeMask) == M_HASH) {
    if (sd == t) e.mode |= kModeDepthOk;
  }
  return e;
}

// parent_entry(node, 1, K) of a root child from its root-directory entry
// (x: node, flags, c0, deg; y: tab, link_tok, link_lp, sd): the same
// branches, with the scan limit of this launch.
__device__ __forceinline__ ParEntry root_child_entry(const KArgs& a, const uint4 x,
                                                     const uint4 y, uint32_t K) {
  const uint32_t f = x.y, deg = x.w, sd = y.w;
  ParEntry e{x.z, deg, (uint32_t)M_NONE, 0u, kNoCursor};
  if (f & kRdLink) {
    e.c0 = sd;
    e.aux = y.y;
    e.mode = (sd == 2u) ? M_LP_SEL : M_LP_NEXT;
    e.work = 1;
    e.lp = y.z;
  } else if (deg == 0) {
    e.mode = M_NONE;
  } else if (deg <= a.scan_limit) {
    e.mode = M_SCAN;
    e.work = deg;
  } else {
    e.mode = M_SEARCH;
    e.work = K;
    if (f & kRdTable) {
      e.mode = M_HASH | ((f & kRdFiltered) ? kModeFiltered : 0u);
      e.aux = (f >> 8) & 0xFFu;
      e.c0 = y.x;
    }
  }
  if ((e.mode & kModeMask) == M_SCAN || (e.mode & kModeMask) == M_HASH) {
    if (sd == 1u) e.mode |= kModeDepthOk;
  }
  return e;
}

// Work items of a parent-table entry.
__device__ __forceinline__ uint32_t entry_work(uint32_t mode, uint32_t aux, uint32_t K) {
  switch (mode & kModeMask) {
    case M_LP_NEXT:
    case M_LP_SEL: return 1u;
    case M_SCAN: return aux;
    case M_SEARCH:
    case M_HASH:
    case M_DENSE: return K;
    default: return 0u;
  }
}

__device__ __forceinline__ uint32_t row_hash(uint32_t tok) {
  return (tok * 0x9E3779B1u) >> (32 - kRowHashLog2);
}

// position of tok in the sorted LDS row, or -1: a probe or two when the row
// is hashed, else a binary search
__device__ __forceinline__ int row_find(const Smem& sm, uint32_t K,
                                        uint32_t tok, bool hashed) {
  if (hashed) {
    uint32_t h = row_hash(tok);
    for (int it = 0; it < kRowHash; ++it) {
      const uint32_t e = sm.rh_tok[h];
      const uint32_t p = sm.rh_pos[h];
      if (e == kRowHashEmpty) return -1;
      if (e == tok) return (int)p;
      h = (h + 1) & (kRowHash - 1);
    }
    return -1;
  }
  uint32_t lo = 0, hi = K;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (sm.row_id[mid] < tok) lo = mid + 1; else hi = mid;
  }
  return (lo < K && sm.row_id[lo] == tok) ? (int)lo : -1;
}

// Data shared between a request's workgroups.  They may sit on different
// XCDs, whose L2 caches are not coherent with each other, and an agent-scope
// fence writes back and invalidates the whole L2 of the XCD -- under every
// other workgroup running there.  So shared data never goes through a fence:
// it is written with device-coherent stores (write-through, `sc1`) and read
// by helpers with device-coherent loads; a writer waits for its stores to
// complete (`vmcnt(0)`: acknowledged at device scope) before it signals, and
// a reader issues its loads only after it has seen the signal.  The leader,
// which re-reads the pushes many times during selection, instead invalidates
// its caches once per step (an acquire fence) and then reads normally.
//
// The loads, stores and store wait this goes through are coherent.h's
// (ld_relaxed, st_dev, wait_stores), with what they rest on.
__device__ __forceinline__ unsigned long long pack2(uint32_t lo, uint32_t hi) {
  return (unsigned long long)lo | ((unsigned long long)hi << 32);
}
// Records written with device-coherent stores (8 bytes at a time).
__device__ __forceinline__ void st_next(NextRec* p, uint64_t key, uint32_t node,
                                        uint32_t jk) {
  unsigned long long* q = (unsigned long long*)p;
  st_dev(q, key);
  st_dev(q + 1, pack2(node, jk));
}
__device__ __forceinline__ void st_sel(SelRec* p, const SelRec& r) {
  unsigned long long* q = (unsigned long long*)p;
  st_dev(q, (unsigned long long)__double_as_longlong(r.s));
  st_dev(q + 1, pack2(r.node, r.depth));
  st_dev(q + 2, pack2(r.phist, r.tok));
  st_dev(q + 3, pack2(r.jk, r.isnew));
}
__device__ __forceinline__ void st_cur(CurRec* p, double s, uint32_t node,
                                       uint32_t hist) {
  unsigned long long* q = (unsigned long long*)p;
  st_dev(q, (unsigned long long)__double_as_longlong(s));
  st_dev(q + 1, pack2(node, hist));
}
__device__ __forceinline__ CurRec ld_cur(const CurRec* p) {
  const unsigned long long* q = (const unsigned long long*)p;
  const unsigned long long a = ld_relaxed(q), b = ld_relaxed(q + 1);
  CurRec r;
  r.s = __longlong_as_double((long long)a);
  r.node = (uint32_t)b;
  r.hist = (uint32_t)(b >> 32);
  return r;
}

// Upper bound on spin iterations of a wait (each sleeps ~64 cycles): far
// beyond any step, so a wait only ends this way if the peer is gone.
constexpr uint32_t kSpinLimit = 1u << 28;
// How long the leader waits for helpers to claim their slices of a shared
// step before it takes the unclaimed ones over (wall-clock ticks of
// 10 ns): running helpers claim within a few microseconds of the post.
constexpr unsigned long long kGraceTicks = 5000;

// Everything a workgroup needs to expand a range of work items of one step.
struct StepView {
  const CurRec* cur;
  SelRec* sel;
  NextRec* nextc;
  const uint32_t* pc0;   // first child id, or the hash-table offset
  const uint32_t* paux;  // degree, the link-parent token, or log2 table size
  const uint32_t* pnode;
  const uint32_t* pmode;
  const uint32_t* woff;  // exclusive prefix of work items, n_par + 1 entries
  Ctl* ctl;
  uint32_t n_par, K, t, nS;
  uint32_t next_cap, sel_cap;
  double lnf_next;
  float tok_thr;
  double sent_thr;
  // a solo step whose `next` pushes (at most this many) all survive keeps
  // them in LDS: no flush, the leader emits from the push buffer
  uint32_t keep_lds_max;
  // every parent has exactly one work item (item w belongs to parent w)
  bool one_each;
};

// Position of tok in a sorted row held in the device stage (a row longer
// than the LDS row arrays), or -1.  Device-coherent loads: a streamed
// search's leader copied the row to the stage during this launch.
__device__ __forceinline__ int grow_find(const uint32_t* rid, uint32_t K, uint32_t tok) {
  uint32_t lo = 0, hi = K;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (ld_relaxed(rid + mid) < tok) lo = mid + 1; else hi = mid;
  }
  return (lo < K && ld_relaxed(rid + lo) == tok) ? (int)lo : -1;
}

// Expands the step's work items: each is (parent, child) for a scanned
// parent, (parent, proposal) for a searched or hashed parent, or the single
// pending token of a link parent.  Items go out in chunks of 64 (one per
// lane of a wave), dealt to the step's workgroups first: chunk c goes to
// workgroup slice c mod nwg (nwg = nwaves / kWaves) and to its wave
// (c / nwg) mod kWaves.  So a step of few chunks is spread over as many
// CUs as it has chunks -- a CU issues the scattered reads of its items at a
// bounded rate, which sets the time of a step far more than the latency
// of one read does -- and every wave still gets an even share of every
// region of the item space (hashed parents cost a random read per item,
// scanned ones a coalesced one).  This workgroup is slice gwave0 / kWaves.
// With at most kBlock parents the parent table is read from LDS, where the
// caller has put it (the leader in its parent phase, a helper with the row);
// the caller has also zeroed this workgroup's push counters and
// synchronised.  The `leader` also reads, for its own emit, the next pending
// token of each link parent that stays one.  Pushes go to the request's
// global buffers.  A `solo` workgroup expands the whole
// step alone: its LDS counters are the list lengths and the control block is
// not used (the counts stay in sm.lq_next, sm.lq_sel, sm.w_children and
// sm.w_probes).
__device__ __forceinline__ void expand_range(const KArgs& a, const StepView& v, uint32_t W,
                             uint32_t gwave0, uint32_t nwaves, bool leader, bool solo,
                             bool hashed, Smem& sm) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const bool lds_par = v.n_par <= (uint32_t)kBlock;
  uint32_t my_children = 0, my_probes = 0;
  const uint32_t K = v.K, t = v.t;
  const uint32_t nchunks = (W + 63u) >> 6;
  const uint32_t nwg = nwaves / (uint32_t)kWaves, slice = gwave0 / (uint32_t)kWaves;
  for (uint32_t c = slice + nwg * (tid >> 6); c < nchunks; c += nwaves) {
    const uint32_t w = (c << 6) + lane;
    bool do_next = false, do_sel = false;
    uint32_t cnode = 0, pj = 0, k = 0, tok = 0;
    double s2 = 0.0;
    // The chunk's parents, when the table is in LDS: those of its first and
    // last items (pa, pb) by a 64-ary search of the prefix, two rounds of one
    // LDS read a lane and a ballot (the prefix is non-decreasing, woff[0] is
    // 0 and woff[n_par] is W, so each ballot is a run of low lanes); each
    // lane then searches [pa, pb] alone -- nothing when one parent holds the
    // whole chunk, as a hashed parent's K items mostly do.
    uint32_t pa = 0, pb = v.n_par;
    if (lds_par && !v.one_each) {
      const uint32_t w0 = c << 6, wl = min(w0 + 63u, W - 1u);
      const uint32_t st = (v.n_par + 64u) >> 6;  // 64 st > n_par
      const uint32_t o1 = sm.woff[min(lane * st, v.n_par)];
      const uint64_t m0 = __ballot(o1 <= w0), m1 = __ballot(o1 <= wl);
      const uint32_t b0 = (63u - (uint32_t)__clzll((long long)m0)) * st;
      const uint32_t b1 = (63u - (uint32_t)__clzll((long long)m1)) * st;
      const uint64_t n0 = __ballot(lane < st && sm.woff[min(b0 + lane, v.n_par)] <= w0);
      const uint64_t n1 = __ballot(lane < st && sm.woff[min(b1 + lane, v.n_par)] <= wl);
      pa = b0 + (63u - (uint32_t)__clzll((long long)n0));
      pb = b1 + (63u - (uint32_t)__clzll((long long)n1)) + 1u;
    }
    if (w < W) {
      // parent of work item w: the last j with woff[j] <= w
      uint32_t lo = pa, hi = pb;
      if (v.one_each) {
        lo = w;
      } else {
        while (hi - lo > 1) {
          const uint32_t mid = (lo + hi) >> 1;
          const uint32_t o = lds_par ? sm.woff[mid] : ld_relaxed(&v.woff[mid]);
          if (o <= w) lo = mid; else hi = mid;
        }
      }
      pj = lo;
      uint32_t md, c0, aux, q;
      if (lds_par) {
        q = w - sm.woff[pj];
        md = sm.p_mode[pj];
        c0 = sm.p_c0[pj];
        aux = sm.p_aux[pj];
      } else {
        q = w - ld_relaxed(&v.woff[pj]);
        md = ld_relaxed(&v.pmode[pj]);
        c0 = ld_relaxed(&v.pc0[pj]);
        aux = ld_relaxed(&v.paux[pj]);
      }
      const bool depth_ok = (md & kModeDepthOk) != 0;
      const bool filtered = (md & kModeFiltered) != 0;
      md &= kModeMask;
      int pos = -1;
      bool have_child = false, label_sel = false;
      // the token a link parent or a scanned child looks up in the row
      uint32_t ftok = kNoToken;
      if (md == M_LP_NEXT || md == M_LP_SEL) {
        // the leader reads the next pending token of a link parent that
        // stays one (for its emit) while the row is searched
        uint32_t xtok = kNoToken;
        if (leader && lds_par && md == M_LP_NEXT) {
          const uint32_t tc = sm.p_lp[pj];
          if (tc != kNoCursor) xtok = a.tail[tc + 1u];
        }
        ftok = aux;
        cnode = lds_par ? sm.p_node[pj] : ld_relaxed(&v.pnode[pj]);
        if (xtok != kNoToken) sm.x_tok[pj] = xtok;
      } else if (md == M_SCAN) {
        // the child's label: its first token, and whether it closes a key
        cnode = c0 + q;
        const uint32_t lw = a.labels[cnode];
        ++my_children;
        ftok = lw & kTokMask;
        have_child = true;
        label_sel = (lw & kSlotSel) && depth_ok;
      } else if (md == M_SEARCH || md == M_HASH || md == M_DENSE) {
        pos = (int)q;
      }
      if (ftok != kNoToken)
        pos = K > kMaxLdsTopk ? grow_find((const uint32_t*)sm.grow_id, K, ftok)
                              : row_find(sm, K, ftok, hashed);
      if (pos >= 0) {
        float x;
        if (K > kMaxLdsTopk) {
          x = __uint_as_float(ld_relaxed((const uint32_t*)sm.grow_lp + pos));
          tok = ld_relaxed((const uint32_t*)sm.grow_id + pos);
        } else {
          x = sm.row_lp[pos];
          tok = sm.row_id[pos];
        }
        k = (uint32_t)pos;
        const double ps = lds_par ? sm.p_s[pj] : ld_cur(&v.cur[pj]).s;
        // thresholds in double, `<=` drops (louds-trie.cc:87-90)
        const bool low = ((double)x <= (double)v.tok_thr) ||
                         (ps + (double)x <= v.sent_thr);
        if (!low) {
          s2 = ps + (double)x;
          if (md == M_SEARCH) {
            // lower_bound of tok among the parent's children
            uint32_t lo2 = c0, hi2 = c0 + aux;
            const uint32_t end2 = hi2;
            while (lo2 < hi2) {
              const uint32_t mid = lo2 + ((hi2 - lo2) >> 1);
              ++my_probes;
              if (a.recs[mid].first_tok < tok) lo2 = mid + 1; else hi2 = mid;
            }
            if (lo2 < end2) {
              const ft_node_rec cr = a.recs[lo2];
              if (cr.first_tok == tok) {
                cnode = lo2;
                have_child = true;
                // terminal with |KB| == |Q| -> selected (louds-trie.cc:103-108)
                label_sel = (cr.meta & FT_META_TERMINAL) &&
                            (cr.meta & FT_META_DEPTH_MASK) == t + 1;
              }
            }
          } else if (md == M_HASH) {
            // the token's first cuckoo bucket, and its second only when the
            // first is full without a match
            const uint32_t lg = aux;
            uint32_t b = c0 + cuckoo_h1(tok, lg);
            // a filtered table: no fingerprint match in the first bucket
            // (nor in the second, when the first is full) means no child
            bool maybe = true;
            if (filtered) {
              const uint64_t f8 = (uint64_t)wide_fp(tok) * 0x0101010101010101ull;
              const uint64_t w1 = a.wfp[b];
              maybe = has_zero_byte(w1 ^ f8);
              if (!maybe && !has_zero_byte(w1))
                maybe = has_zero_byte(a.wfp[c0 + cuckoo_h2(tok, lg)] ^ f8);
            }
            uint32_t hw = 0, hc = 0;
            for (int round = 0; round < (maybe ? 2 : 0); ++round) {
              // the whole bucket (tokens and children) in one read
              const uint4* bw = (const uint4*)&a.wtab[b];
              const uint4 ta = bw[0], tb = bw[1], ca = bw[2], cb = bw[3];
              ++my_probes;
              const uint32_t tw[8] = {ta.x, ta.y, ta.z, ta.w, tb.x, tb.y, tb.z, tb.w};
              const uint32_t cw[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
              bool full = true;
#pragma unroll
              for (int sl = 0; sl < 8; ++sl) {
                if ((tw[sl] & kTokMask) == tok) {
                  hw = tw[sl];
                  hc = cw[sl];
                }
                full = full && tw[sl] != kSlotEmptyTok;
              }
              if (hc != 0u || !full) break;
              b = c0 + cuckoo_h2(tok, lg);
            }
            if (hc != 0u) {
              cnode = hc;
              have_child = true;
              label_sel = (hw & kSlotSel) && depth_ok;
            }
          } else if (md == M_DENSE) {
            // the root's child of this token: one read of (node, flags)
            if (tok < a.root_n) {
              const uint2 rd = *(const uint2*)&a.root_dir[tok];
              ++my_probes;
              if (rd.x != 0u) {
                cnode = rd.x;
                have_child = true;
                label_sel = (rd.y & kRdSel) && depth_ok;
              }
            }
          }
          if (md == M_LP_NEXT) {
            do_next = true;
          } else if (md == M_LP_SEL) {
            do_sel = true;
          } else if (have_child) {
            // a child is always next; selected when it closes a key of
            // length t + 1 (louds-trie.cc:103-108)
            do_next = true;
            do_sel = label_sel;
          }
        }
      }
    }
    // appends (every lane of the wave reaches these): into the LDS
    // buffers while they have room, the rest straight to the global lists
    const uint32_t jk = (pj << 16) | k;
    if (__ballot(do_next)) {
      const uint32_t li = wave_append(do_next, &sm.lq_next);
      const bool spill = do_next && li >= (uint32_t)kPushCap;
      const uint32_t gi = solo ? li : wave_append_half(spill, &v.ctl->pushes, false);
      if (do_next) {
        const uint64_t key = norm_key(s2 * v.lnf_next);
        if (!spill) {
          sm.push_next[li].key = key;
          sm.push_next[li].node = cnode;
          sm.push_next[li].jk = jk;
        } else if (gi < v.next_cap) {
          st_next(&v.nextc[gi], key, cnode, jk);
        }
      }
    }
    if (__ballot(do_sel)) {
      const uint32_t li = wave_append(do_sel, &sm.lq_sel);
      const bool spill = do_sel && li >= (uint32_t)kPushSelCap;
      const uint32_t gi = solo ? li : wave_append_half(spill, &v.ctl->pushes, true);
      if (do_sel) {
        SelRec sr;
        sr.s = s2;
        sr.node = cnode;
        sr.depth = t + 1;
        sr.phist = lds_par ? sm.p_hist[pj] : ld_cur(&v.cur[pj]).hist;
        sr.tok = tok;
        sr.jk = jk;
        sr.isnew = 1;
        if (!spill) sm.push_sel[li] = sr;
        else if (v.nS + gi < v.sel_cap) st_sel(&v.sel[v.nS + gi], sr);
      }
    }
  }
  // the workgroup's counters: one LDS add a wave (lane by lane, the adds to
  // one word would run one after another, 1024 of them)
  {
    const uint32_t wc = wave_sum(my_children), wp = wave_sum(my_probes);
    if ((tid & 63u) == 0u) {
      if (wc) atomicAdd(&sm.w_children, wc);
      if (wp) atomicAdd(&sm.w_probes, wp);
    }
  }
  __syncthreads();
  // the buffered pushes: one global append per list (a solo workgroup's
  // lists start at 0)
  const uint32_t nl = min(sm.lq_next, (uint32_t)kPushCap);
  const uint32_t sl = min(sm.lq_sel, (uint32_t)kPushSelCap);
  uint32_t gb_next = 0, gb_sel = 0;
  if (!solo) {
    // both lists' places in one 64-bit add (every workgroup of the step
    // adds to this word: one add each, not one per list and counter)
    if (tid == 0) {
      unsigned long long old = 0;
      if (nl || sl)
        old = atomicAdd(&v.ctl->pushes, (unsigned long long)nl | ((unsigned long long)sl << 32));
      sm.gb_next = (uint32_t)old;
      sm.gb_sel = (uint32_t)(old >> 32);
    }
    __syncthreads();
    gb_next = sm.gb_next;
    gb_sel = sm.gb_sel;
  }
  const bool next_in_lds = solo && sm.lq_next <= v.keep_lds_max;
  for (uint32_t i = tid; i < (next_in_lds ? 0u : nl); i += kBlock) {
    const uint32_t o = gb_next + i;
    const NextRec& r = sm.push_next[i];
    if (o < v.next_cap) st_next(&v.nextc[o], r.key, r.node, r.jk);
  }
  for (uint32_t i = tid; i < sl; i += kBlock) {
    const uint32_t o = gb_sel + i;
    if (v.nS + o < v.sel_cap) st_sel(&v.sel[v.nS + o], sm.push_sel[i]);
  }
}

// Loads the proposal row of step t (staged in ascending token order) into
// LDS.
__device__ __forceinline__ void load_row(const uint32_t* rid, const float* rlp, uint32_t t,
                                         uint32_t K, Smem& sm) {
  const uint64_t o = (uint64_t)t * K;
  for (uint32_t p = threadIdx.x; p < K; p += kBlock) {
    sm.row_id[p] = rid[o + p];
    sm.row_lp[p] = rlp[o + p];
  }
}

// The row hash: emptied by every thread's share of the slots, then filled
// with (token, sorted position) pairs.  Tokens >= 2^31 - 1 never match a trie
// token and are left out.  Row tokens are distinct (staging rejects
// duplicates) and fill at most half the table (K <= kRowHashMaxK), so every
// insert ends in a free slot.
__device__ __forceinline__ void row_hash_clear(Smem& sm) {
  for (uint32_t i = threadIdx.x; i < (uint32_t)kRowHash; i += kBlock)
    sm.rh_tok[i] = kRowHashEmpty;
}
__device__ __forceinline__ void row_hash_insert(uint32_t tok, uint32_t p, Smem& sm) {
  if (tok >= kTokMask) return;
  uint32_t h = row_hash(tok);
  for (int it = 0; it < kRowHash; ++it) {
    if (atomicCAS(&sm.rh_tok[h], kRowHashEmpty, tok) == kRowHashEmpty) {
      sm.rh_pos[h] = (uint16_t)p;
      return;
    }
    h = (h + 1) & (kRowHash - 1);
  }
}

// Hashes the LDS row (the workgroup has synchronised since the row was
// written).  Ends synchronised.
__device__ __forceinline__ void hash_row(uint32_t K, Smem& sm) {
  row_hash_clear(sm);
  __syncthreads();
  for (uint32_t p = threadIdx.x; p < K; p += kBlock) row_hash_insert(sm.row_id[p], p, sm);
  __syncthreads();
}

// The proposal's index in the caller's row at position p (jk's low 16 bits)
// of the token-sorted row t: from the staged indices, or p itself when every
// row came in ascending token order (none staged).
__device__ __forceinline__ uint32_t caller_index(const uint16_t* rk, uint32_t t, uint32_t K,
                                                 uint32_t jk) {
  const uint32_t p = jk & 0xFFFFu;
  return rk ? (uint32_t)rk[(uint64_t)t * K + p] : p;
}

// Streamed search: how much of its block the leader has copied from mapped
// host memory into the device stage (values every thread holds alike).
struct StageState {
  uint32_t rows;     // rows, with their key bounds, in the stage
  uint32_t rk_rows;  // rows whose proposal indices are in the stage
  uint32_t split;    // rows of the first ready word (stream_split)
  bool rk;           // some row came out of order: its indices are read
  bool done;         // the whole block is in
  bool own;          // the leader claimed the copy of the rows after `split`
};

// Thread 0 waits (bounded) for request req's ready word to carry this
// launch's epoch and a final state or at least `need` rows -- a system-scope
// acquire, so that what the host packed before the word is what the reads
// after it see.  Returns the word to every thread, or 0 when it never came.
__device__ __forceinline__ unsigned long long wait_ready(const KArgs& a, uint32_t req,
                                                         uint32_t need, Smem& sm) {
  if (threadIdx.x == 0) {
    const unsigned long long t0 = wall_clock64();
    unsigned long long v = 0;
    for (;;) {
      v = __hip_atomic_load(a.ready + req, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
      if ((v >> 32) == a.epoch &&
          (((uint32_t)v & (kReadyOk | kReadyWithdrawn)) ||
           ((uint32_t)v >> kReadyRowsShift) >= need))
        break;
      if (wall_clock64() - t0 > a.ready_ticks) {
        v = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    sm.bcast = v;
  }
  __syncthreads();
  return sm.bcast;
}

// Copies the byte ranges [b[i], e[i]) of the request's block (each rounded
// out to 16 bytes; none when e[i] <= b[i]) from mapped host memory to the
// device stage, with device-coherent stores: helpers read its rows there.
// Every thread; the loads of a round are all in flight together.  Ends
// synchronised, with the stores complete.  Callers give ranges whose
// rounding takes in only bytes the host has packed for good.
constexpr uint32_t kNoWord = 0xFFFFFFFFu;
template <uint32_t kU>
__device__ __forceinline__ void stage_copy(const KArgs& a, uint64_t in_off, const uint32_t (&b)[4],
                                           const uint32_t (&e)[4]) {
  const uint32_t tid = threadIdx.x;
  uint32_t s16[4], n16[4], total = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t lo = b[r] & ~15u, hi = (e[r] + 15u) & ~15u;
    s16[r] = lo / 16u;
    n16[r] = e[r] > b[r] ? (hi - lo) / 16u : 0u;
    total += n16[r];
  }
  const uint4* src = (const uint4*)(a.stage_src + in_off);
  unsigned long long* dst = (unsigned long long*)(const_cast<uint8_t*>(a.stage) + in_off);
  for (uint32_t i0 = 0; i0 < total; i0 += kBlock * kU) {
    uint4 w[kU];
    uint32_t at[kU];
#pragma unroll
    for (uint32_t u = 0; u < kU; ++u) {
      uint32_t i = i0 + u * kBlock + tid;
      at[u] = kNoWord;
      if (i < total) {
        uint32_t x;
        if (i < n16[0]) {
          x = s16[0] + i;
        } else if ((i -= n16[0]) < n16[1]) {
          x = s16[1] + i;
        } else if ((i -= n16[1]) < n16[2]) {
          x = s16[2] + i;
        } else {
          x = s16[3] + (i - n16[2]);
        }
        at[u] = x;
        w[u] = src[x];
      }
    }
#pragma unroll
    for (uint32_t u = 0; u < kU; ++u) {
      if (at[u] != kNoWord) {
        st_dev(dst + 2ull * at[u], pack2(w[u].x, w[u].y));
        st_dev(dst + 2ull * at[u] + 1, pack2(w[u].z, w[u].w));
      }
    }
  }
  wait_stores();
  __syncthreads();
}

// Rows [h0, h1) of the request's block with their key bounds (with `head`,
// everything before the bounds too: the length-norm table and beam widths)
// and, when the ready word `v` carries kReadyRk, the proposal indices of
// rows [ss.rk_rows, h1); then records them in ss.  Every thread; ends
// synchronised.
template <uint32_t kU>
__device__ __forceinline__ void stage_rows(const KArgs& a, const DevReq& d, bool head,
                                           uint32_t h0, uint32_t h1, unsigned long long v,
                                           StageState& ss) {
  const uint32_t rb = 4u * d.K;  // bytes of a row of tokens (and of logps)
  const bool rk = ((uint32_t)v & kReadyRk) != 0;
  const uint32_t b[4] = {head ? 0u : d.kb_off + 16u * h0, d.rid_off + h0 * rb,
                         d.rlp_off + h0 * rb, d.rk_off + ss.rk_rows * 2u * d.K};
  const uint32_t e[4] = {d.kb_off + 16u * h1, d.rid_off + h1 * rb, d.rlp_off + h1 * rb,
                         rk ? d.rk_off + h1 * 2u * d.K : 0u};
  stage_copy<kU>(a, d.in_off, b, e);
  ss.rows = h1;
  if (rk) {
    ss.rk = true;
    ss.rk_rows = h1;
  }
  ss.done = h1 >= d.T;
}

// Streamed search, the leader's start: waits for the request's first ready
// word and copies its length-norm table, beam widths and first rows (all of
// them when the word is final, else those before its split) to the device
// stage; helpers read rows there in shared steps, after the leader's first
// post (which follows the wait for these stores).  `d` is the request's
// header as planned at the launch: its offsets are final then (rk_off is
// where the indices go when some row needs them).  False when the host
// withdrew the request, the word never came or the planned block does not
// fit the stage -- after releasing the helpers and reporting the status in
// out_host.
__device__ __forceinline__ bool stage_in(const KArgs& a, uint32_t req, const DevReq& d,
                                         uint8_t* ws, StageState& ss, Smem& sm) {
  const unsigned long long tag = (unsigned long long)a.epoch << 32;
  const uint32_t split = stream_split(a.head_rows, d.T, d.K);
  const unsigned long long v = wait_ready(a, req, split, sm);
  const uint32_t rows = (uint32_t)v >> kReadyRowsShift;
  const bool final = ((uint32_t)v & kReadyOk) != 0;
  const bool ok = (v >> 32) == a.epoch && !((uint32_t)v & kReadyWithdrawn) &&
                  (final ? rows == d.T : ((uint32_t)v & kReadyPart) && rows >= split &&
                                             rows < d.T);
  if (!ok || !block_fits(a.stage_bytes, d)) {
    if (threadIdx.x == 0) {
      st_dev(&((Ctl*)(ws + a.lay.ctl))->go, tag | kGoExit);
      OutHeader* oh = (OutHeader*)(a.out_host + (uint64_t)req * a.out_stride);
      oh->count = 0;
      const uint32_t st = ((v >> 32) == a.epoch && ((uint32_t)v & kReadyWithdrawn))
                              ? kStatusWithdrawn
                          : ok ? kStatusStage
                               : kStatusNotReady;
      __hip_atomic_store(&oh->status, st | kStatusDone, __ATOMIC_RELEASE,
                         __HIP_MEMORY_SCOPE_SYSTEM);
    }
    return false;
  }
  ss = StageState{0u, 0u, split, false, false, false};
  stage_rows<8>(a, d, true, 0u, final ? d.T : split, v, ss);
  return true;
}

// Streamed search, helper 1 at its start: the copy of the request's rows
// after the split (with their bounds, and all of its proposal indices when
// some row came out of order) -- claimed here unless the leader claimed it
// first -- once the host has packed the whole request, while the leader
// searches the first rows.  The copy word then says done or failed.
__device__ __forceinline__ void helper_copy(const KArgs& a, uint32_t req, const DevReq& d,
                                            uint8_t* ws, Smem& sm) {
  const uint32_t split = stream_split(a.head_rows, d.T, d.K);
  if (split >= d.T) return;
  Ctl* ctl = (Ctl*)(ws + a.lay.ctl);
  const unsigned long long tag = (unsigned long long)a.epoch << 32;
  if (threadIdx.x == 0)
    sm.lead_flag = atomicMax(&ctl->copy, tag | kCopyClaimed) < (tag | kCopyClaimed) ? 1u : 0u;
  __syncthreads();
  const bool mine = sm.lead_flag != 0;
  __syncthreads();
  if (!mine) return;
  const unsigned long long v = wait_ready(a, req, d.T, sm);
  const bool ok = (v >> 32) == a.epoch && ((uint32_t)v & kReadyOk) &&
                  ((uint32_t)v >> kReadyRowsShift) == d.T && block_fits(a.stage_bytes, d);
  const bool rk = ((uint32_t)v & kReadyRk) != 0;
  if (ok) {
    const uint32_t rb = 4u * d.K;
    const uint32_t b[4] = {d.kb_off + 16u * split, d.rid_off + split * rb, d.rlp_off + split * rb,
                           d.rk_off};
    const uint32_t e[4] = {d.kb_off + 16u * d.T, d.rid_off + d.T * rb, d.rlp_off + d.T * rb,
                           rk ? d.rk_off + 2u * d.T * d.K : 0u};
    stage_copy<8>(a, d.in_off, b, e);
  }
  if (threadIdx.x == 0)
    st_dev(&ctl->copy, tag | (ok ? (kCopyDone | (rk ? kCopyRk : 0u)) : kCopyFailed));
  __syncthreads();
}

// Streamed search: makes rows up to u (< T) of the request available in the
// device stage, a no-op once they are.  The rows after the split come from
// helper 1's copy, waited for when it has claimed it (it is running then),
// else from the leader, which claims the copy and takes the rows as the host
// packs them.  False when the request was withdrawn or the rows never came
// (the status is in sm.status then).  Every thread; ends synchronised.
__device__ __forceinline__ bool ensure_rows(const KArgs& a, uint32_t req, const DevReq& d,
                                            uint8_t* ws, uint32_t u, StageState& ss, Smem& sm) {
  if (ss.done || u < ss.rows) return true;
  uint32_t fail = 0;
  if (!ss.own) {
    Ctl* ctl = (Ctl*)(ws + a.lay.ctl);
    const unsigned long long tag = (unsigned long long)a.epoch << 32;
    if (threadIdx.x == 0) {
      unsigned long long c = atomicMax(&ctl->copy, tag | kCopyClaimed);
      uint32_t st = kCopyClaimed;  // claimed now by the leader
      if (c >= (tag | kCopyClaimed)) {
        // helper 1 has it: wait (bounded) for its end
        const unsigned long long t0 = wall_clock64();
        while ((uint32_t)c == kCopyClaimed && wall_clock64() - t0 <= a.ready_ticks) {
          __builtin_amdgcn_s_sleep(2);
          c = ld_relaxed(&ctl->copy);
        }
        st = (uint32_t)c == kCopyClaimed ? kCopyFailed : (uint32_t)c;
      } else {
        st = 0u;  // the leader's own
      }
      sm.lead_flag = st;
    }
    __syncthreads();
    const uint32_t st = sm.lead_flag;
    __syncthreads();
    if (st & kCopyDone) {
      // helper 1's stores were complete before its word: drop stale lines
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      ss.rows = d.T;
      ss.done = true;
      if (st & kCopyRk) {
        ss.rk = true;
        ss.rk_rows = d.T;
      }
      return true;
    }
    if (st & kCopyFailed) fail = kStatusNotReady;
    ss.own = true;
  }
  unsigned long long v = 0;
  if (!fail) {
    v = wait_ready(a, req, u + 1u, sm);
    const uint32_t rows = (uint32_t)v >> kReadyRowsShift;
    if ((v >> 32) != a.epoch || ((uint32_t)v & kReadyWithdrawn) || rows <= u || rows > d.T)
      fail = ((v >> 32) == a.epoch && ((uint32_t)v & kReadyWithdrawn)) ? kStatusWithdrawn
                                                                       : kStatusNotReady;
  }
  if (fail) {
    if (threadIdx.x == 0) sm.status |= fail;
    __syncthreads();
    return false;
  }
  stage_rows<4>(a, d, false, ss.rows, (uint32_t)v >> kReadyRowsShift, v, ss);
  // The leader reads rows and bounds with ordinary loads, and a row ends
  // inside a cache line: its L1 may hold the start of a row this copy just
  // wrote, read before with the end of the row in front.  Drop such lines.
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return true;
}

// A helper workgroup: waits for shared steps of its request and expands its
// slice of the work items, until the leader posts the exit generation.
template <bool kStreamed>
__device__ __forceinline__ void helper_loop(const KArgs& a, const DevReq& d, uint8_t* ws,
                            uint32_t g, Smem& sm) {
  const uint32_t tid = threadIdx.x;
  Ctl* ctl = (Ctl*)(ws + a.lay.ctl);
  const unsigned long long tag = (unsigned long long)a.epoch << 32;
  unsigned long long seen = tag;  // generation 0: nothing posted yet
  const uint8_t* in = a.stage + d.in_off;
  const double* lnf = (const double*)in;
  const uint32_t* rid = (const uint32_t*)(in + d.rid_off);
  const float* rlp = (const float*)(in + d.rlp_off);
  if constexpr (kStreamed) {
    if (g == 1) helper_copy(a, blockIdx.x % a.batch, d, ws, sm);
  }
  // The helpers that share the leader's XCD (blocks are dealt to the 8 XCDs
  // in turn: block req + g * batch sits with the leader's when g * batch is
  // a multiple of 8) each read a share of the first row's tokens and touch
  // their root-directory entries, while the leader reads its request's
  // set-up (and the row itself): its step-0 reads then find them in their
  // L2.
  const uint32_t pfg = (a.batch & 7u) == 0 ? 1u
                       : (a.batch & 3u) == 0 ? 2u
                       : (a.batch & 1u) == 0 ? 4u : 8u;
  // A streamed request's first rows are read once the leader has copied
  // them to the device stage (helper 1, busy with the copy of the rest,
  // takes no share; a wait ends too once the leader has posted or quit).
  const uint32_t nq = (a.wgs - 1u) / pfg;
  if (a.root_n != 0u && d.T != 0u && g % pfg == 0u && nq != 0u && !(kStreamed && g == 1u)) {
    bool ok = true;
    if constexpr (kStreamed) {
      if (tid == 0) {
        unsigned long long h = 0;
        for (uint32_t it = 0; it < kSpinLimit; ++it) {
          h = ld_relaxed(&ctl->head);
          if ((h >> 32) == a.epoch || (ld_relaxed(&ctl->go) >> 32) == a.epoch) break;
          __builtin_amdgcn_s_sleep(1);
        }
        sm.bcast = h;
      }
      __syncthreads();
      ok = (sm.bcast >> 32) == a.epoch;
      __syncthreads();
    }
    if (ok) {
      const uint32_t per = (d.K + nq - 1u) / nq, lo = (g / pfg - 1u) * per;
      const uint32_t hi = min(d.K, lo + per);
      uint32_t acc = 0;
      for (uint32_t i = lo + tid; i < hi; i += kBlock) {
        uint32_t tok;
        if constexpr (kStreamed) {
          tok = ld_relaxed(rid + i);
          acc ^= ld_relaxed((const uint32_t*)rlp + i);
        } else {
          tok = rid[i];
          acc ^= __float_as_uint(rlp[i]);
        }
        if (tok < a.root_n) acc ^= a.root_dir[tok].node;
      }
      // (a use of the loads, so that they stay; the counter is cleared
      // before the first slice)
      if (acc == 0x9E3779B9u) sm.w_probes = acc;
    }
  }
  row_hash_clear(sm);  // (visible after the first barrier below)
  for (;;) {
    if (tid == 0) {
      unsigned long long v = 0;
      for (uint32_t it = 0; it < kSpinLimit; ++it) {
        v = ld_relaxed(&ctl->go);
        if ((v >> 32) == a.epoch && v != seen) break;
        __builtin_amdgcn_s_sleep(1);
      }
      sm.bcast = v;
      sm.hstep[6] = 0;
      if ((v >> 32) == a.epoch && (uint32_t)v != kGoExit && v != seen) {
        // the step's parameters, read once after `go` and shared through LDS
        // so that every thread takes the same branches below
        // Take this workgroup's slice of the step: its claim word is raised
        // to this step's (epoch, generation) unless it already holds it or
        // a later one -- the leader took the slice over first.  The claim
        // goes out with the reads of the step's parameters; a successful
        // one also proves they are this step's: the leader writes the next
        // step's only after every claimed slice is done.
        unsigned long long* cl = (unsigned long long*)(ws + a.lay.claims) + g;
        const bool claimed = !a.no_claims && atomicMax(cl, v) < v;
        const uint32_t pt = ld_relaxed(&ctl->t), pW = ld_relaxed(&ctl->W),
                       pn = ld_relaxed(&ctl->n_par), pS = ld_relaxed(&ctl->nS);
        sm.hstep[0] = pt;
        sm.hstep[1] = pW;
        sm.hstep[2] = pn;
        sm.hstep[3] = pS;
        sm.hstep[4] = ld_relaxed(&ctl->cur_which);
        sm.hstep[5] = ld_relaxed(&ctl->sel_which);
        // A posted step always satisfies the bounds below; a claimed slice
        // of anything else is counted done without being expanded.
        const uint64_t max_w = (uint64_t)pn * max(a.scan_limit, d.K);
        const bool sane = pt < d.T && pn != 0 && pn <= a.lay.cur_cap &&
                          pS <= a.lay.sel_cap && (uint64_t)pW <= max_w;
        sm.hstep[6] = claimed ? (sane ? 1u : 2u) : 0u;
      }
    }
    __syncthreads();
    const unsigned long long v = sm.bcast;
    const uint32_t t = sm.hstep[0], W = sm.hstep[1], n_par = sm.hstep[2],
                   nS = sm.hstep[3], cur_which = sm.hstep[4], sel_which = sm.hstep[5];
    const uint32_t mine = sm.hstep[6];
    __syncthreads();
    if ((v >> 32) != a.epoch || (uint32_t)v == kGoExit || v == seen) return;
    seen = v;
    if (mine == 0) continue;  // the leader took this slice over
    // this workgroup's done word (its counters, then the step's tag)
    unsigned long long* dw = (unsigned long long*)(ws + a.lay.dones) + 2ull * g;
    if (mine == 2) {          // (never for a posted step)
      if (tid == 0) {
        st_dev(dw + 1, 0ull);
        wait_stores();
        st_dev(dw, v);
      }
      continue;
    }
    StepView sv;
    sv.cur = (const CurRec*)(ws + (cur_which ? a.lay.cur1 : a.lay.cur0));
    sv.sel = (SelRec*)(ws + (sel_which ? a.lay.selB : a.lay.selA));
    sv.nextc = (NextRec*)(ws + a.lay.nextc);
    sv.pc0 = (const uint32_t*)(ws + a.lay.par_c0);
    sv.paux = (const uint32_t*)(ws + a.lay.par_aux);
    sv.pnode = (const uint32_t*)(ws + a.lay.par_node);
    sv.pmode = (const uint32_t*)(ws + a.lay.par_mode);
    sv.woff = (const uint32_t*)(ws + a.lay.par_woff);
    sv.ctl = ctl;
    sv.n_par = n_par;
    sv.K = d.K;
    sv.t = t;
    sv.nS = nS;
    sv.next_cap = a.lay.next_cap;
    sv.sel_cap = a.lay.sel_cap;
    // (a streamed search's leader wrote the stage during this launch: read
    // it device-coherently; a staged one's was copied before the launch)
    if constexpr (kStreamed)
      sv.lnf_next = __longlong_as_double(
          (long long)ld_relaxed((const unsigned long long*)lnf + t + 1));
    else
      sv.lnf_next = lnf[t + 1];
    sv.tok_thr = d.tok_thr;
    sv.sent_thr = d.sent_thr;
    sv.keep_lds_max = 0;
    sv.one_each = false;
    // the step's row (into the row hash too: emptied after the previous
    // step) and parent table in one round of reads; a row longer than the
    // LDS row arrays is searched where it is staged
    const bool hashed = d.K <= kRowHashMaxK;
    const bool lds_par = n_par <= (uint32_t)kBlock;
    const uint64_t ro = (uint64_t)t * d.K;
    const bool big = d.K > kMaxLdsTopk;
    if (big && tid == 0) {
      sm.grow_id = (unsigned long long)(rid + ro);
      sm.grow_lp = (unsigned long long)(rlp + ro);
    }
    const uint32_t Kl = big ? 0u : d.K;  // row entries loaded into LDS
    const uint32_t nload = max(Kl, lds_par ? n_par + 1u : 0u);
    for (uint32_t i = tid; i < nload; i += kBlock) {
      uint32_t tok = 0;
      float lp = 0.0f;
      if (i < Kl) {
        if constexpr (kStreamed) {
          tok = ld_relaxed(rid + ro + i);
          lp = __uint_as_float(ld_relaxed((const uint32_t*)rlp + ro + i));
        } else {
          tok = rid[ro + i];
          lp = rlp[ro + i];
        }
      }
      if (lds_par && i <= n_par) {
        sm.woff[i] = ld_relaxed(&sv.woff[i]);
        if (i < n_par) {
          sm.p_c0[i] = ld_relaxed(&sv.pc0[i]);
          sm.p_aux[i] = ld_relaxed(&sv.paux[i]);
          sm.p_node[i] = ld_relaxed(&sv.pnode[i]);
          sm.p_mode[i] = (uint8_t)ld_relaxed(&sv.pmode[i]);
          const CurRec p = ld_cur(&sv.cur[i]);
          sm.p_s[i] = p.s;
          sm.p_hist[i] = p.hist;
        }
      }
      if (i < Kl) {
        sm.row_id[i] = tok;
        sm.row_lp[i] = lp;
        if (hashed) row_hash_insert(tok, i, sm);
      }
    }
    if (tid == 0) {
      sm.w_children = 0;
      sm.w_probes = 0;
      sm.lq_next = 0;
      sm.lq_sel = 0;
    }
    __syncthreads();
    expand_range(a, sv, W, g * (uint32_t)kWaves, a.wgs * (uint32_t)kWaves, false, false,
                 hashed, sm);
    // the row lookups are done: empty the hash for the next step
    if (hashed) row_hash_clear(sm);
    if (tid == 0) st_dev(dw + 1, pack2(sm.w_children, sm.w_probes));
    wait_stores();  // this slice's pushes and counters are complete
    __syncthreads();
    if (tid == 0) st_dev(dw, v);  // then its done word: no shared counter
    // The first helper that shares the leader's XCD reads a word of every
    // 64 bytes of the request's rows after the next one and of the history
    // records written so far, so that the leader's later reads of them (the
    // single-wave tail's row fills, the output's history walks) find them
    // in their L2.  A streamed request's later rows only once their copy to
    // the device stage is done (before, the lines could be stale); the
    // history is the leader's, written through the same L2.
    if (g == pfg && t + 2u < d.T && !big) {
      bool ready = true;
      if constexpr (kStreamed) {
        if (stream_split(a.head_rows, d.T, d.K) < d.T) {
          const unsigned long long c = ld_relaxed(&ctl->copy);
          ready = (c >> 32) == a.epoch && ((uint32_t)c & kCopyDone);
        }
      }
      if (ready) {
        const uint64_t r0 = (uint64_t)(t + 2u) * d.K;
        const uint32_t n = (d.T - t - 2u) * d.K;  // words of each array
        const HistRec* hist = (const HistRec*)(ws + a.lay.hist);
        const uint32_t nh = min(ld_relaxed(&ctl->hist_n), a.lay.hist_cap);
        uint32_t acc = 0;
        for (uint32_t i = tid * 16u; i < n; i += kBlock * 16u)
          acc ^= rid[r0 + i] ^ __float_as_uint(rlp[r0 + i]);
        for (uint32_t i = tid * 4u; i < nh; i += kBlock * 4u) acc ^= hist[i].tok;
        // (a use of the loads, so that they stay: the slice's counter, already
        // reported in the done word and cleared before the next slice)
        if (acc == 0x9E3779B9u) sm.w_probes = acc;
      }
    }
  }
}

// The single-wave tail of a request's search (see the leader's step loop)
// runs in rounds of up to kTailMaxRows steps.  Each round the whole leader
// workgroup reads the rows of the round's steps into LDS (tail_fill),
// with the steps' beam widths and each hypothesis's pending tokens of those
// steps; then wave 0 runs the steps (tiny_steps) with no global read on its
// path, so that a step costs its LDS searches and stores rather than a
// memory round trip.
//
// tail_fill: rows t .. t + nr - 1 into the LDS row arrays (row r at
// r * Kp), their beam widths into tl_beams, and, for each hypothesis j <
// n_cur of the LDS parent table whose pending token of step t is on its
// node's own edge (tail index tc), the tokens of steps t + r, r = 1 .. nr,
// that come before its key ends (string depth sd: steps < sd), tail[tc + r]
// -- the entries the hypothesis reads if it survives; then every token so
// known is searched in its row (tl_x).  Every thread; the caller
// synchronises afterwards.
__device__ __forceinline__ void tail_fill(const KArgs& a, const uint32_t* rid, const float* rlp,
                                          const uint32_t* beams, uint32_t t, uint32_t nr,
                                          uint32_t K, uint32_t Kp, uint32_t n_cur, Smem& sm) {
  const uint32_t tid = threadIdx.x;
  for (uint32_t r0 = 0; r0 < nr; r0 += 4u) {
    uint32_t id[4];
    float lp[4];
#pragma unroll
    for (uint32_t u = 0; u < 4u; ++u) {
      const uint32_t r = r0 + u;
      if (r < nr && tid < K) {
        const uint64_t o = (uint64_t)(t + r) * K + tid;
        id[u] = rid[o];
        lp[u] = rlp[o];
      }
    }
#pragma unroll
    for (uint32_t u = 0; u < 4u; ++u) {
      const uint32_t r = r0 + u;
      if (r < nr && tid < K) {
        sm.row_id[r * Kp + tid] = id[u];
        sm.row_lp[r * Kp + tid] = lp[u];
      }
    }
  }
  if (tid < nr) sm.tl_beams[tid] = beams[t + tid];
  for (uint32_t i = tid; i < (nr + 1u) * 64u; i += kBlock) {
    const uint32_t r = i >> 6, j = i & 63u;
    uint32_t tok = kNoToken;
    if (r > 0 && j < n_cur) {
      const uint32_t tc = sm.p_lp[j];
      if (tc != kNoCursor && t + r < sm.p_c0[j]) tok = a.tail[tc + r];
    }
    sm.tl_tok[i] = tok;
  }
  __syncthreads();
  // each known pending token in its step's row (binary search): its logp's
  // bits, or kAbsent -- the searches of the whole round at once, one per
  // thread, instead of one after another on wave 0
  for (uint32_t i = tid; i < nr * 64u; i += kBlock) {
    const uint32_t r = i >> 6, j = i & 63u;
    uint32_t xb = kAbsent;
    const uint32_t tok = j >= n_cur ? kNoToken : r == 0 ? sm.p_aux[j] : sm.tl_tok[i];
    if (tok != kNoToken) {
      const uint32_t rb = r * Kp;
      uint32_t lo = 0, hi = K;
      while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (sm.row_id[rb + mid] < tok) lo = mid + 1; else hi = mid;
      }
      if (lo < K && sm.row_id[rb + lo] == tok) xb = __float_as_uint(sm.row_lp[rb + lo]);
    }
    sm.tl_x[i] = xb;
  }
}

// tiny_steps: wave 0 of the leader, lane j holding hypothesis j (j < n_cur)
// of a beam of link parents whose parent table for step t is in LDS, runs
// steps t .. t + nr - 1 on the rows tail_fill put there while every push
// survives: the hypothesis's pending key token is looked up in the row,
// thresholds applied (louds-trie.cc:87-90), and the extension goes to
// `selected` when it completes the key (louds-trie.cc:97-102), else stays a
// link parent in `next`.  Survivors keep their lanes (ranks among the live
// lanes give their beam and history positions).  Stops (sm.tiny_done) when
// the beam empties, the steps run out, or early exit fills `selected`;
// hands back (sm.tiny_handback) at the first step whose pushes overflow a
// heap (bounded selection), would cut `selected` under early exit, or hit
// a capacity limit -- then the beam is written to cur and the LDS / global
// parent table of that step, which the general step reruns from scratch;
// else, after nr steps, leaves the beam in the LDS parent table (and each
// hypothesis's history links in tl_rtok / tl_rphist) for the next round
// (`first` is false there).
// A value every lane of the wave holds alike, marked so: what is derived
// from it can live in scalar registers rather than vector ones.
__device__ __forceinline__ uint32_t uni(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)x);
}
__device__ __forceinline__ uint64_t uni(uint64_t x) {
  return (uint64_t)uni((uint32_t)x) | ((uint64_t)uni((uint32_t)(x >> 32)) << 32);
}
__device__ __forceinline__ float uni(float x) { return __uint_as_float(uni(__float_as_uint(x))); }
__device__ __forceinline__ double uni(double x) {
  return __longlong_as_double((long long)uni((uint64_t)__double_as_longlong(x)));
}

__device__ __forceinline__ void tiny_steps(
    const KArgs& a, const DevReq& d, uint32_t t, uint32_t nr, uint32_t Kp, bool first,
    uint32_t n_cur, uint32_t nS, uint32_t hist_used, uint32_t lane, const double* lnf,
    CurRec* cur, SelRec* selA, HistRec* hist, uint32_t* par_c0, uint32_t* par_aux,
    uint32_t* par_node, uint32_t* par_mode, uint64_t* step_stats, Smem& sm) {
  const uint32_t T = d.T, K = d.K, F = d.F;
  const bool early = (d.flags & kReqEarlyExit) != 0;
  const uint64_t lt = (1ull << lane) - 1ull;
  // this lane's hypothesis
  bool alive = lane < n_cur;
  uint32_t node = 0, hst = kNoHist, mode = M_LP_NEXT, sd = 0, ptok = 0, tc = kNoCursor;
  // the hypothesis's own history record: its last token and its parent's
  // record, the links of the record a step below adds
  uint32_t rtok = 0, rphist = kNoHist;
  double s = 0.0;
  // its pending tokens of this round are in tl_tok (it is on its own edge)
  bool ahead = false;
  if (alive) {
    node = sm.p_node[lane];
    s = sm.p_s[lane];
    hst = sm.p_hist[lane];
    mode = sm.p_mode[lane] & kModeMask;
    sd = sm.p_c0[lane];
    ptok = sm.p_aux[lane];
    tc = sm.p_lp[lane];
    ahead = tc != kNoCursor;
    if (!first) {
      rtok = sm.tl_rtok[lane];
      rphist = sm.tl_rphist[lane];
    } else if (hst < a.lay.hist_cap) {
      const HistRec r = hist[hst];
      rtok = r.tok;
      rphist = r.phist;
    }
  }
  uint32_t status = 0;
  bool done = false, handback = false;
  unsigned long long cands = 0, ticks = 0;
  // one clock read per step: the end of a step is the start of the next
  unsigned long long c0 = wall_clock64();
  for (uint32_t r = 0; r < nr; ++r, ++t) {
    if (n_cur == 0 || (early && nS >= F)) {
      done = true;
      break;
    }
    // the pending token in the row (searched by tail_fill when the token
    // was known there), thresholds in double (`<=` drops)
    bool pass = false;
    double s2 = 0.0;
    if (alive) {
      uint32_t xb = kAbsent;
      if (r == 0 || ahead) {
        xb = sm.tl_x[r * 64u + lane];
      } else {
        const uint32_t rb = r * Kp;
        uint32_t lo = 0, hi = K;
        while (lo < hi) {
          const uint32_t mid = (lo + hi) >> 1;
          if (sm.row_id[rb + mid] < ptok) lo = mid + 1; else hi = mid;
        }
        if (lo < K && sm.row_id[rb + lo] == ptok) xb = __float_as_uint(sm.row_lp[rb + lo]);
      }
      if (xb != kAbsent) {
        const float x = __uint_as_float(xb);
        pass = !(((double)x <= (double)d.tok_thr) || (s + (double)x <= d.sent_thr));
        s2 = s + (double)x;
      }
    }
    const bool to_sel = pass && mode == M_LP_SEL;
    const bool to_next = pass && mode == M_LP_NEXT;
    const uint64_t mS = __ballot(to_sel), mN = __ballot(to_next);
    const uint32_t n_new = (uint32_t)__popcll(mS), n_next = (uint32_t)__popcll(mN);
    const uint32_t Mnext = sm.tl_beams[r];
    // every push survives and no limit is reached, or hand back
    if (n_next > Mnext || nS + n_new > F || nS + n_new > a.lay.sel_cap ||
        hist_used + n_next > a.lay.hist_cap) {
      handback = true;
      break;
    }
    // early exit with `selected` exactly full: every new push is among the
    // first F (louds-trie.cc:81-83), and the search ends after this step
    const bool stop_early = early && nS + n_new >= F;
    if (to_sel) {
      SelRec sr;
      sr.s = s2;
      sr.node = node;
      sr.depth = t + 1;
      sr.phist = hst;
      sr.tok = ptok;
      sr.jk = 0;
      sr.isnew = 0;  // kept: `selected` has room for every push
      st_sel(&selA[nS + (uint32_t)__popcll(mS & lt)], sr);
    }
    if (stop_early) {  // selected is full: the search ends here
      nS += n_new;
      cands += n_new;
      const unsigned long long c1 = wall_clock64();
      if (lane == 0 && t < d.out_T) {
        uint64_t* row = step_stats + (uint64_t)t * kStepStats;
        row[0] = n_cur;
        row[1] = n_cur;
        row[2] = n_next;
        row[3] = n_new;
        row[4] = c1 - c0;
      }
      ticks += c1 - c0;
      done = true;
      break;
    }
    if (to_next) {
      const uint32_t o = hist_used + (uint32_t)__popcll(mN & lt);
      HistRec h;
      h.phist = hst;
      h.tok = ptok;
      h.ptok = rtok;
      h.phist2 = rphist;
      hist[o] = h;
      rtok = ptok;
      rphist = hst;
      hst = o;
      s = s2;
      // the pending token of step t + 1: on the node's own edge the next
      // tail token (read ahead by tail_fill when the round began there),
      // else the walk parent_entry makes
      if (tc != kNoCursor) {
        ++tc;
        // Global reads happen on the rare paths only, and each is waited
        // for inside its own branch (the empty asm statements use the
        // values there): a wait where the paths join would also wait for
        // this step's stores, which count in the same counter.  The LDS
        // read is taken unconditionally and made opaque for the same
        // reason: as one arm of a select it became a flat load.
        uint32_t la = sm.tl_tok[(r + 1u) * 64u + lane];
        asm volatile("" : "+v"(la));
        if (!ahead) {
          la = a.tail[tc];
          asm volatile("" : "+v"(la));
        }
        ptok = la;
        mode = (t + 2 == sd) ? M_LP_SEL : M_LP_NEXT;
      } else {
        // (what parent_entry builds for a link parent at step t + 1)
        uint32_t err = 0;
        const ft_node_rec rec = a.recs[node];
        ptok = kb_token(a, node, rec, t + 1, &err);
        if (err) status |= kStatusCorrupt;
        mode = (t + 2 == sd) ? M_LP_SEL : M_LP_NEXT;
        const uint32_t el = (rec.meta >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
        tc = ((rec.meta & FT_META_LINK) && t + 1 + el >= sd) ? rec.tail_off + (t + 1 + el - sd)
                                                             : kNoCursor;
        asm volatile("" : "+v"(ptok), "+v"(tc), "+v"(status));
      }
    }
    alive = to_next;
    const unsigned long long c1 = wall_clock64();
    if (lane == 0 && t < d.out_T) {
      uint64_t* row = step_stats + (uint64_t)t * kStepStats;
      row[0] = n_cur;
      row[1] = n_cur;
      row[2] = n_next;
      row[3] = n_new;
      row[4] = c1 - c0;
    }
    hist_used += n_next;
    nS += n_new;
    cands += (uint64_t)n_next + n_new;
    if (lane == 0) sm.cnt_parents += n_cur;
    n_cur = n_next;
    ticks += c1 - c0;
    c0 = c1;
    if (status) break;
  }
  // this wave's stores (history, selected, the step profile) are complete
  // before the block barrier that follows
  wait_stores();
  if (!handback && (t >= T || n_cur == 0 || (early && nS >= F))) done = true;
  const uint64_t am = __ballot(alive);
  if (!done && !status) {
    // the beam for the next round, or handed back to the general step:
    // hypothesis of lane j at position rank(j)
    if (alive) {
      const uint32_t o = (uint32_t)__popcll(am & lt);
      sm.p_node[o] = node;
      sm.p_s[o] = s;
      sm.p_hist[o] = hst;
      sm.p_mode[o] = (uint8_t)mode;
      sm.p_c0[o] = sd;
      sm.p_aux[o] = ptok;
      sm.p_lp[o] = tc;
      sm.tl_rtok[o] = rtok;
      sm.tl_rphist[o] = rphist;
      if (handback) {
        st_cur(&cur[o], s, node, hst);
        st_dev(&par_c0[o], sd);
        st_dev(&par_aux[o], ptok);
        st_dev(&par_node[o], node);
        st_dev(&par_mode[o], mode);
      }
    }
  }
  if (lane == 0) {
    sm.tiny_t = t;
    sm.tiny_ncur = n_cur;
    sm.tiny_nS = nS;
    sm.tiny_hist = hist_used;
    sm.tiny_done = done ? 1u : 0u;
    sm.tiny_handback = handback ? 1u : 0u;
    sm.tiny_cands = cands;
    sm.tiny_ticks = ticks;
    if (status) sm.status |= status;
  }
}

// kLouds: child ranges from the LOUDS directory (KArgs::louds_*) instead
// of the node records; kStreamed: the streamed search (KArgs::ready and
// friends).  Separate instantiations, so that each keeps its own register
// allocation and code: the staged search carries none of the streamed
// one's start and output.
template <bool kLouds, bool kStreamed>
__global__ void __launch_bounds__(kBlock) tbs_kernel(KArgs a) {
  __shared__ Smem sm;
  // request-major interleave: request r owns blocks r, r + batch, ...  The
  // dispatcher deals blocks to the 8 XCDs round-robin, so at batch 8 each
  // request's workgroups share one XCD and its L2.
  const uint32_t req = blockIdx.x % a.batch;
  const uint32_t g = blockIdx.x / a.batch;
  const uint32_t tid = threadIdx.x;
  if (g >= a.wgs) return;

  // (a streamed request's header is final at the launch: the host never
  // rewrites it, and whether its row indices are staged comes with the
  // ready words)
  const DevReq d = a.reqs[req];
  uint8_t* ws = a.ws + (uint64_t)req * a.ws_stride;
  if (d.flags & kReqSkip) {
    if (g == 0 && tid == 0) {
      OutHeader* oh = (OutHeader*)(a.out + (uint64_t)req * a.out_stride);
      oh->count = 0;
      oh->status = 0;
    }
    return;
  }
  if (g != 0) {
    helper_loop<kStreamed>(a, d, ws, g, sm);
    return;
  }

  // ---- the leader ----------------------------------------------------------
  // the per-step profile goes to `out` during the search; the results (and
  // a copy of the profile) to out_host in a streamed search, else to `out`
  uint8_t* ob = a.out + (uint64_t)req * a.out_stride;
  // a streamed request's rows come to the device stage as the host packs
  // them (stage_in, ensure_rows); the staged search has them all
  StageState ss{d.T, d.T, d.T, d.rk_off != 0u, true, false};
  if constexpr (kStreamed) {
    if (!stage_in(a, req, d, ws, ss, sm)) return;
    // (stage_in's stores are complete: the helpers may read the first rows)
    if (tid == 0)
      st_dev(&((Ctl*)(ws + a.lay.ctl))->head, ((unsigned long long)a.epoch << 32) | 1ull);
    if (tid == 0) sm.res_host = (unsigned long long)(a.out_host + (uint64_t)req * a.out_stride);
  }
  const uint8_t* in = a.stage + uni(d.in_off);
  const double* lnf = (const double*)in;
  const uint32_t* beams = (const uint32_t*)(in + d.beams_off);
  const uint32_t* rid = (const uint32_t*)(in + d.rid_off);
  const float* rlp = (const float*)(in + d.rlp_off);
  // the proposals' indices in the caller's rows, when some row came out of
  // order (else index = position)
  const uint16_t* rk = ss.rk ? (const uint16_t*)(in + d.rk_off) : nullptr;
  // (streamed) rows up to u in the device stage, or false with sm.status set
  auto rows_upto = [&](uint32_t u) {
    if constexpr (kStreamed) {
      if (!ensure_rows(a, req, d, ws, u, ss, sm)) return false;
      rk = ss.rk ? (const uint16_t*)(in + d.rk_off) : nullptr;
    }
    return true;
  };
  const uint32_t T = d.T, K = d.K, F = d.F;
  const bool early = (d.flags & kReqEarlyExit) != 0;

  CurRec* cur = (CurRec*)(ws + a.lay.cur0);
  CurRec* cur2 = (CurRec*)(ws + a.lay.cur1);
  uint32_t cur_which = 0, sel_which = 0;
  NextRec* nextc = (NextRec*)(ws + a.lay.nextc);
  SelRec* selA = (SelRec*)(ws + a.lay.selA);
  SelRec* selB = (SelRec*)(ws + a.lay.selB);
  uint32_t* rank = (uint32_t*)(ws + a.lay.rank);
  HistRec* hist = (HistRec*)(ws + a.lay.hist);
  Ctl* ctl = (Ctl*)(ws + a.lay.ctl);
  uint32_t* par_c0 = (uint32_t*)(ws + a.lay.par_c0);
  uint32_t* par_aux = (uint32_t*)(ws + a.lay.par_aux);
  uint32_t* par_node = (uint32_t*)(ws + a.lay.par_node);
  uint32_t* par_mode = (uint32_t*)(ws + a.lay.par_mode);
  uint32_t* par_woff = (uint32_t*)(ws + a.lay.par_woff);
  const uint32_t next_cap = a.lay.next_cap, sel_cap = a.lay.sel_cap,
                 hist_cap = a.lay.hist_cap;
  const unsigned long long tag = (unsigned long long)a.epoch << 32;
  uint32_t gen = 0;
  unsigned long long t_post = 0;  // (thread 0) wall clock of the last post

  unsigned long long t_exp = 0, t_sel = 0, t_all0 = wall_clock64();
  // per-step profile rows after the output tokens: kStepStats u64 per step
  uint64_t* step_stats = (uint64_t*)(ob + step_stats_offset(d.F, d.out_T));
  for (uint32_t i = tid; i < d.out_T * kStepStats; i += kBlock) step_stats[i] = 0;
  if (tid == 0) {
    st_cur(&cur[0], 0.0, 0, kNoHist);
    sm.status = 0;
    sm.multi_item = 0;
    sm.cnt_parents = sm.cnt_children = sm.cnt_probes = 0;
  }
  uint32_t n_cur = 1, nS = 0, hist_used = 0;
  uint64_t n_cands = 0;
  // the parent table of the step was written by the previous step's emit,
  // and its row loaded into registers there (pf_*); for step 0 both are
  // read here, the root's entry by one thread of wave 1 while every thread
  // reads its share of row 0
  bool par_ready = true, row_pf = K <= (uint32_t)kBlock;
  uint32_t pf_id = 0;
  float pf_lp = 0.0f;
  if (row_pf && tid < K) {
    pf_id = rid[tid];
    pf_lp = rlp[tid];
  }
  uint32_t root_err = 0;
  if (tid == 64u) {
    ParEntry e = parent_entry<kLouds>(a, 0u, 0u, K, &root_err);
    if (a.root_dir) {
      // a root searched or hashed (or scanned, when forced) looks its
      // children up in the root directory instead; a one-token child
      // closes a key of length 1 when the root's string depth is 0
      const uint32_t m = e.mode & kModeMask;
      if (m == M_SEARCH || m == M_HASH || (m == M_SCAN && a.root_force)) {
        const bool dok = (a.recs[0].meta & FT_META_DEPTH_MASK) == 0u;
        e.mode = M_DENSE | (dok ? kModeDepthOk : 0u);
        e.work = K;
      }
    }
    st_dev(&par_c0[0], e.c0);
    st_dev(&par_aux[0], e.aux);
    st_dev(&par_node[0], 0u);
    st_dev(&par_mode[0], e.mode);
    sm.p_c0[0] = e.c0;
    sm.p_aux[0] = e.aux;
    sm.p_node[0] = 0u;
    sm.p_mode[0] = (uint8_t)e.mode;
    sm.p_lp[0] = e.lp;
    sm.p_s[0] = 0.0;
    sm.p_hist[0] = kNoHist;
  }
  __syncthreads();
  if (root_err) atomicOr(&sm.status, (uint32_t)kStatusCorrupt);

  for (uint32_t t = 0; t < T; ++t) {
    if (n_cur == 0 || (early && nS >= F)) break;
    // ---- the tail of small link-parent steps, on one wave ---------------
    // When the beam holds at most 64 hypotheses and every one is a link
    // parent (it can only continue with its own next key token,
    // louds-trie.cc:91-102), each step is one row lookup per hypothesis.
    // A link parent either stays one (next) or closes its key (selected),
    // so the beam stays in this form until it empties.  Wave 0 runs these
    // steps alone, the hypotheses in its lanes' registers, in rounds of as
    // many steps as the LDS row arrays hold rows (4 at K = 1000; the
    // workgroup reads them, with the tokens the hypotheses will look up,
    // before each round), for as long as every push survives both heaps
    // (no bounded selection cuts and early exit does not fire mid-step); at
    // the first step that needs a cut it hands the beam back to the general
    // step.
    if (par_ready && n_cur <= 64u && K <= (uint32_t)kBlock) {
      const uint32_t lane = tid & 63u;
      const uint32_t md0 = lane < n_cur ? (uint32_t)(sm.p_mode[lane] & kModeMask) : (uint32_t)M_LP_NEXT;
      if (__ballot(md0 != M_LP_NEXT && md0 != M_LP_SEL) == 0) {
        // rows K rounded up to whole waves apart
        const uint32_t Kp = (K + 63u) & ~63u;
        const uint32_t R = min((uint32_t)kMaxLdsTopk / Kp, kTailMaxRows);
        bool first = true, finished = false;
        for (;;) {
          const uint32_t nr = min(R, T - t);
          if (!rows_upto(t + nr - 1u)) {
            finished = true;
            break;
          }
          tail_fill(a, rid, rlp, beams, t, nr, K, Kp, n_cur, sm);
          __syncthreads();
          if (tid < 64u) tiny_steps(a, d, t, nr, Kp, first, n_cur, nS, hist_used, lane, lnf,
                                    cur, selA, hist, par_c0, par_aux, par_node, par_mode,
                                    step_stats, sm);
          __syncthreads();
          t = sm.tiny_t;
          n_cur = sm.tiny_ncur;
          nS = sm.tiny_nS;
          hist_used = sm.tiny_hist;
          n_cands += sm.tiny_cands;
          t_exp += sm.tiny_ticks;
          if (sm.tiny_done || sm.status) {
            finished = true;
            break;
          }
          if (sm.tiny_handback) break;
          first = false;
        }
        if (finished) break;
        // a cut is due at step t: the general step below runs it, with the
        // beam handed back in the parent table and row t reloaded
        row_pf = false;
        if (n_cur == 0 || (early && nS >= F)) break;
      }
    }
    // this step's row, and the next one, which the step reads ahead
    if (!rows_upto(min(t + 1u, T - 1u))) break;
    const unsigned long long t0 = wall_clock64();
    const uint32_t ncur0 = n_cur;
    if (row_pf) {
      if (tid < K) {
        sm.row_id[tid] = pf_id;
        sm.row_lp[tid] = pf_lp;
      }
    } else {
      if (K <= kMaxLdsTopk) {
        load_row(rid, rlp, t, K, sm);
      } else if (tid == 0) {
        // a row longer than the LDS row arrays is searched in the stage
        // (the parent phase ends synchronised: every thread sees these)
        sm.grow_id = (unsigned long long)(rid + (uint64_t)t * K);
        sm.grow_lp = (unsigned long long)(rlp + (uint64_t)t * K);
      }
    }
    const double lnf_next = lnf[t + 1];

    // ---- parents: lookup mode, work items, exclusive prefix ---------------
    // work items of parent j (j < n_cur), writing its table entry unless the
    // previous step's emit did
    auto parent_work = [&](uint32_t j) -> uint32_t {
      // (an opaque index: the per-thread addresses below are formed here,
      // not hoisted out of the step loop into registers held all along)
      asm volatile("" : "+v"(j));
      const bool lp = n_cur <= (uint32_t)kBlock;
      if (par_ready) {
        if (lp) {
          const uint32_t md = sm.p_mode[j], c0 = sm.p_c0[j], cur_lp = sm.p_lp[j];
          sm.x_s[j] = sm.p_s[j];
          sm.x_hist[j] = sm.p_hist[j];
          sm.x_sd[j] = (md == M_LP_NEXT && cur_lp != kNoCursor) ? (uint16_t)c0 : (uint16_t)0;
          sm.x_tc[j] = cur_lp;
          sm.x_tok[j] = kNoToken;
          return entry_work(md, sm.p_aux[j], K);
        }
        return entry_work(ld_relaxed(&par_mode[j]), ld_relaxed(&par_aux[j]), K);
      }
      const CurRec p = cur[j];
      uint32_t err = 0;
      const ParEntry e = parent_entry<kLouds>(a, p.node, t, K, &err);
      if (err) atomicOr(&sm.status, (uint32_t)kStatusCorrupt);
      st_dev(&par_c0[j], e.c0);
      st_dev(&par_aux[j], e.aux);
      st_dev(&par_node[j], p.node);
      st_dev(&par_mode[j], e.mode);
      if (lp) {
        sm.p_c0[j] = e.c0;
        sm.p_aux[j] = e.aux;
        sm.p_node[j] = p.node;
        sm.p_mode[j] = (uint8_t)e.mode;
        sm.p_lp[j] = e.lp;
        sm.p_s[j] = p.s;
        sm.p_hist[j] = p.hist;
        sm.x_s[j] = p.s;
        sm.x_hist[j] = p.hist;
        sm.x_sd[j] = (e.mode == M_LP_NEXT && e.lp != kNoCursor) ? (uint16_t)e.c0 : (uint16_t)0;
        sm.x_tc[j] = e.lp;
        sm.x_tok[j] = kNoToken;
      }
      return e.work;
    };
    uint32_t W = 0;
    const bool one_wave = n_cur <= 64u;
    if (one_wave) {
      // one wave holds every parent: its scan needs no barrier
      if (tid < 64u) {
        const uint32_t work = tid < n_cur ? parent_work(tid) : 0u;
        const uint32_t incl = wave_incl_scan(work);
        const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
        if (tid < n_cur) {
          uint32_t j = tid;
          asm volatile("" : "+v"(j));  // (address formed here, not held)
          st_dev(&par_woff[j], incl - work);
          sm.woff[tid] = incl - work;
          if (work != 1) sm.multi_item = 1;  // cleared before the step began
        }
        if (tid == 0) {
          st_dev(&par_woff[n_cur], tot);
          sm.woff[n_cur] = tot;
          sm.par_w = tot;
        }
      }
    } else {
      for (uint32_t cbase = 0; cbase < n_cur; cbase += kBlock) {
        const uint32_t j = cbase + tid;
        const uint32_t work = j < n_cur ? parent_work(j) : 0u;
        uint32_t Wc;
        const uint32_t off = block_excl_scan(work, &Wc, sm);
        if (j < n_cur) {
          st_dev(&par_woff[j], W + off);
          if (n_cur <= (uint32_t)kBlock) sm.woff[j] = W + off;
          if (work != 1) sm.multi_item = 1;
        }
        W += Wc;
      }
      if (tid == 0) {
        st_dev(&par_woff[n_cur], W);
        if (n_cur <= (uint32_t)kBlock) sm.woff[n_cur] = W;
      }
    }
    if (tid == 0) {
      sm.cnt_parents += n_cur;
      // this workgroup's expansion counters (expand_range of the leader
      // relies on them being zero)
      sm.w_children = 0;
      sm.w_probes = 0;
      sm.lq_next = 0;
      sm.lq_sel = 0;
    }
    __syncthreads();
    if (one_wave) W = sm.par_w;

    StepView sv;
    sv.cur = cur;
    sv.sel = selA;
    sv.nextc = nextc;
    sv.pc0 = par_c0;
    sv.paux = par_aux;
    sv.pnode = par_node;
    sv.pmode = par_mode;
    sv.woff = par_woff;
    sv.ctl = ctl;
    sv.n_par = n_cur;
    sv.K = K;
    sv.t = t;
    sv.nS = nS;
    sv.next_cap = next_cap;
    sv.sel_cap = sel_cap;
    sv.lnf_next = lnf_next;
    sv.tok_thr = d.tok_thr;
    sv.sent_thr = d.sent_thr;
    sv.keep_lds_max = min((uint32_t)kPushCap, beams[t]);
    sv.one_each = n_cur <= (uint32_t)kBlock && sm.multi_item == 0;


    const bool shared = a.wgs > 1 && W >= a.share_min;
    if (shared) {
      // publish the step (the helpers read the row from the staged request),
      // then wake the helpers
      if (tid == 0) {
        st_dev(&ctl->pushes, 0ull);
        st_dev(&ctl->t, t);
        st_dev(&ctl->W, W);
        st_dev(&ctl->n_par, n_cur);
        st_dev(&ctl->nS, nS);
        st_dev(&ctl->sel_which, sel_which);
        st_dev(&ctl->cur_which, cur_which);
        st_dev(&ctl->hist_n, hist_used);
      }
      wait_stores();  // the step's data is complete before `go` moves
      __syncthreads();
      ++gen;
      if (tid == 0) {
        st_dev(&ctl->go, tag | gen);
        t_post = wall_clock64();
      }
    }
    // (the parent table ended synchronised: the row and the emptied hash are
    // visible)
    const bool hashed = K <= kRowHashMaxK && W >= kRowHashMinWork;
    if (hashed) hash_row(K, sm);
    // (streamed) helper 1 copying the request's later rows claims no slice
    // meanwhile: its slice is taken over at once rather than after the
    // grace period (thread 0 stands for slot 1 below)
    bool copying1 = false;
    if constexpr (kStreamed) {
      if (shared && tid == 0 && !ss.done && !ss.own && ss.split < T)
        copying1 = ld_relaxed(&ctl->copy) == (tag | kCopyClaimed);
    }
    expand_range(a, sv, W, 0, (shared ? a.wgs : 1u) * (uint32_t)kWaves, true, !shared,
                 hashed, sm);
    // (shared) the pushes of the step; the counters of the leader's slices
    uint32_t sh_next = 0, sh_sel = 0, lead_ch = sm.w_children, lead_pr = sm.w_probes;
    if (shared) {
      // The helpers' slices: each is claimed by its helper (its claim word
      // set to this step) or, once kGraceTicks have passed since the post,
      // taken over here -- so the step never waits for a workgroup that is
      // not running.  Then every claimed slice is waited for: a helper that
      // claimed one is running and finishes it.
      const unsigned long long tw0 = wall_clock64();
      const unsigned long long mygo = tag | gen;
      unsigned long long* claims = (unsigned long long*)(ws + a.lay.claims);
      const uint32_t nh = a.wgs - 1;  // helper slots 1 .. nh (nh < kBlock)
      bool pending_any = true;
      for (;;) {
        const int pending = __syncthreads_count(tid < nh && !copying1 &&
                                                ld_relaxed(&claims[tid + 1]) != mygo);
        if (pending == 0) {
          pending_any = false;
          break;
        }
        if (tid == 0) sm.lead_flag = (wall_clock64() - t_post > kGraceTicks) ? 1u : 0u;
        __syncthreads();
        const bool expired = sm.lead_flag != 0;
        __syncthreads();
        if (expired) break;
        __builtin_amdgcn_s_sleep(2);
      }
      uint32_t n_stolen = 0;
      bool stole = false;  // (thread i) slice i + 1 was taken over here
      // (thread 0 alone knows whether helper 1 is copying: the takeover
      // runs when any slot is still pending or helper 1 copies)
      if (__syncthreads_or(pending_any || copying1)) {
        if (tid == 0) sm.n_stolen = 0;
        __syncthreads();
        // raise every unclaimed word (helper 1's alone when only it is
        // copying): a slice whose word this raises is taken over here; one
        // a helper raised first stays the helper's
        if (tid < nh && (pending_any || tid == 0) &&
            atomicMax(&claims[tid + 1], mygo) < mygo) {
          stole = true;
          const uint32_t k = atomicAdd(&sm.n_stolen, 1u);
          sm.stolen[k] = (uint16_t)(tid + 1);
        }
        __syncthreads();
        n_stolen = sm.n_stolen;
      }
      for (uint32_t i = 0; i < n_stolen; ++i) {
        const uint32_t slice = sm.stolen[i];
        __syncthreads();
        if (tid == 0) {
          sm.w_children = 0;
          sm.w_probes = 0;
          sm.lq_next = 0;
          sm.lq_sel = 0;
        }
        __syncthreads();
        expand_range(a, sv, W, slice * (uint32_t)kWaves, a.wgs * (uint32_t)kWaves, true, false,
                     hashed, sm);
        lead_ch += sm.w_children;
        lead_pr += sm.w_probes;
      }
      // Every slice a helper claimed: thread i waits for helper i + 1's done
      // word to carry this step's tag (written after its pushes and its
      // counters are complete), unless thread i took that slice over.
      const unsigned long long tw1 = wall_clock64();
      unsigned long long* dones = (unsigned long long*)(ws + a.lay.dones);
      const bool waits = tid < nh && !stole;
      bool all_done = false;
      for (uint32_t it = 0; it < kSpinLimit; ++it) {
        if (__syncthreads_count(waits && ld_relaxed(&dones[2 * (tid + 1)]) != mygo) == 0) {
          all_done = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (tid == 0) {
        if (!all_done) sm.status |= kStatusCorrupt;
        if (t < d.out_T) {
          uint64_t* row = step_stats + (uint64_t)t * kStepStats;
          row[8] = tw1 - tw0;
          row[9] = wall_clock64() - tw1;
        }
      }
      // the helpers' counters and the step's push counts, read together
      const unsigned long long cw = waits ? ld_relaxed(&dones[2 * (tid + 1) + 1]) : 0ull;
      const unsigned long long pw = ld_relaxed(&ctl->pushes);
      sh_next = (uint32_t)pw;
      sh_sel = (uint32_t)(pw >> 32);
      const uint32_t wc = wave_sum((uint32_t)cw), wp = wave_sum((uint32_t)(cw >> 32));
      if (tid == 0) {
        sm.w_children = lead_ch;
        sm.w_probes = lead_pr;
      }
      __syncthreads();
      if ((tid & 63u) == 0u) {
        if (wc) atomicAdd(&sm.w_children, wc);
        if (wp) atomicAdd(&sm.w_probes, wp);
      }
    }
    __syncthreads();
    // the helpers' pushes are complete (they waited for their stores before
    // writing their done words): drop stale cached copies before reading
    if (shared) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const uint32_t n_next = shared ? sh_next : sm.lq_next;
    const uint32_t n_new = shared ? sh_sel : sm.lq_sel;
    const unsigned long long w_ch = sm.w_children;
    const unsigned long long w_pr = sm.w_probes;
    // every writer of the status has passed the barrier above; only thread
    // 0 adds the overflow bit below, which every thread derives itself
    const bool overflow = n_next > next_cap || nS + n_new > sel_cap;
    const bool stop = overflow || sm.status != 0;
    n_cands += (uint64_t)n_next + n_new;
    if (tid == 0) {
      sm.cnt_children += w_ch;
      sm.cnt_probes += w_pr;
      if (overflow) sm.status |= kStatusOverflow;
    }
    if (stop) {
      __syncthreads();
      break;
    }
    const unsigned long long t1 = wall_clock64();
    t_exp += t1 - t0;
    if (tid == 0 && t < d.out_T) {
      uint64_t* row = step_stats + (uint64_t)t * kStepStats;
      row[0] = ncur0;
      row[1] = W;
      row[2] = n_next;
      row[3] = n_new;
      row[4] = t1 - t0;
      row[5] = 0;
      row[6] = w_ch;
      row[7] = w_pr;
    }

    // bounds of every key pushed into `next` at this step, from the staged
    // request (the selection then needs no pass over the list for its range)
    const uint32_t Mnext = beams[t];
    const uint64_t* kbound = (const uint64_t*)(in + d.kb_off) + 2ull * t;

    // ---- parent ranks (only when arrival order is needed) ---------------
    bool ranks_done = false;
    const double lnf_cur = lnf[t];
    const uint32_t ncur_now = n_cur;
    auto compute_ranks = [&]() {
      if (ranks_done) return;
      ranks_done = true;
      uint64_t* rk_key = (uint64_t*)sm.row_id;  // aliases the row (done)
      uint32_t* rk_node = (uint32_t*)sm.row_lp;
      __syncthreads();
      for (uint32_t jb = 0; jb < ncur_now; jb += kBlock) {
        const uint32_t j = jb + tid;
        uint64_t myk = 0;
        uint32_t myn = 0, cntless = 0;
        if (j < ncur_now) {
          myk = norm_key(cur[j].s * lnf_cur);
          myn = cur[j].node;
        }
        for (uint32_t ib = 0; ib < ncur_now; ib += kRankChunk) {
          const uint32_t i = ib + tid;
          if (tid < (uint32_t)kRankChunk && i < ncur_now) {
            // in the thread's own chunk, entry i is its own
            rk_key[tid] = ib == jb ? myk : norm_key(cur[i].s * lnf_cur);
            rk_node[tid] = ib == jb ? myn : cur[i].node;
          } else if (tid < (uint32_t)kRankChunk) {
            rk_key[tid] = kRankPad;
            rk_node[tid] = 0;
          }
          __syncthreads();
          const uint32_t m = (min((uint32_t)kRankChunk, ncur_now - ib) + 3u) & ~3u;
          if (j < ncur_now) cntless += count_before<2>(rk_key, rk_node, m, myk, myn);
          __syncthreads();
        }
        if (j < ncur_now) rank[j] = cntless;
      }
      __syncthreads();
    };

    // ---- selected ----------------------------------------------------------
    bool stop_after = false;
    if (n_new > 0) {
      const uint32_t nU = nS + n_new;
      auto sel_key = [&](uint32_t i) {
        const SelRec& r = selA[i];
        return norm_key(r.s * lnf[r.depth]);
      };
      auto sel_arr = [&](uint32_t i) {
        const SelRec& r = selA[i];
        if (!r.isnew) return 0u;
        return 1u + rank[r.jk >> 16] * K + caller_index(rk, t, K, r.jk);
      };
      auto sel_node = [&](uint32_t i) { return selA[i].node; };
      Bound b{0, 0, 0, 0, 1};
      bool early_cut = false;
      uint32_t acut = 0;
      if (early) {
        if (nU >= F) {
          // the first F - nS new pushes in arrival order, then stop
          compute_ranks();
          const uint32_t want = F - nS;
          uint32_t e1, r1;
          acut = radix_kth<uint32_t>(
              nU, want, [&](uint32_t i) { return sel_arr(i); },
              [&](uint32_t i) { return i >= nS; }, sm, &e1, &r1);
          early_cut = true;
          stop_after = true;
        }
      } else {
        b = bounded_select(nU, F, sel_key, sel_arr, sel_node, compute_ranks, sm);
      }
      if (b.all && !early_cut) {
        // every push fits: the new items simply become old ones (no LDS
        // state changed: no barrier)
        for (uint32_t i = nS + tid; i < nU; i += kBlock) st_dev(&selA[i].isnew, 0u);
        nS = nU;
      } else {
        if (tid == 0) sm.n_out = 0;
        __syncthreads();
        for (uint32_t base = 0; base < nU; base += kBlock) {
          const uint32_t i = base + tid;
          bool keep = false;
          if (i < nU) {
            if (early_cut) keep = (i < nS) || sel_arr(i) <= acut;
            else keep = bound_keep(b, sel_key(i), b.tie ? sel_arr(i) : 0u, sel_node(i));
          }
          const uint32_t o = wave_append(keep, &sm.n_out);
          if (keep && o < sel_cap) {
            SelRec r = selA[i];
            r.isnew = 0;
            st_sel(&selB[o], r);
          }
        }
        __syncthreads();
        nS = sm.n_out;
        SelRec* tmp = selA; selA = selB; selB = tmp;
        sel_which ^= 1u;
        if (nS > F) {  // the bound keeps at most F
          if (tid == 0) sm.status |= kStatusCorrupt;
          __syncthreads();
          break;
        }
        __syncthreads();
      }
    }
    if (stop_after) {
      t_sel += wall_clock64() - t1;
      break;
    }

    // ---- next --------------------------------------------------------------
    const uint32_t M = Mnext;
    auto nk = [&](uint32_t i) { return nextc[i].key; };
    auto na = [&](uint32_t i) {
      const uint32_t jk = nextc[i].jk;
      return rank[jk >> 16] * K + caller_index(rk, t, K, jk);
    };
    auto nn = [&](uint32_t i) { return nextc[i].node; };
    const bool collect = M <= (uint32_t)kKeepCap;
    const uint64_t nk_lo = kbound[0], nk_hi = kbound[1];
    const Bound bn = bounded_select(n_next, M, nk, na, nn, compute_ranks, sm,
                                    nk_lo <= nk_hi, nk_lo, nk_hi, collect);
    // survivors already listed by the selection (keys above its boundary
    // bin), and the boundary bin's size
    bool listed = false;
    uint32_t n_listed = 0, n_bin = 0;
    if (!bn.all) {
      listed = sm.collected != 0;
      n_listed = min(sm.n_keep, (uint32_t)kKeepCap);
      n_bin = min(sm.n_out, (uint32_t)kBinCap);
      __syncthreads();
      if (tid == 0) sm.n_out = 0;
      __syncthreads();
    }
    const uint32_t keep_cnt = bn.all ? n_next : M;
    if (hist_used + keep_cnt > hist_cap) {
      if (tid == 0) sm.status |= kStatusHistory;
      __syncthreads();
      break;
    }
    // a solo step whose pushes all survive left them in LDS (expand_range
    // skipped their flush under the same condition)
    const bool next_in_lds = !shared && n_next <= min((uint32_t)kPushCap, Mnext);
    // survivor i becomes hypothesis o of the next beam
    // the next step's proposal row, into registers while the survivors are
    // emitted (the LDS row is still read until the emit ends)
    row_pf = t + 1 < T && K <= (uint32_t)kBlock;
    if (row_pf && tid < K) {
      const uint64_t o = (uint64_t)(t + 1) * K + tid;
      pf_id = rid[o];
      pf_lp = rlp[o];
    }
    // The next step's parent table is filled here too: the node lookups of a
    // survivor overlap the reads of its parent, and the next step starts
    // with its table in place (in LDS as well when it has at most kBlock
    // parents).
    const bool next_table = t + 1 < T;
    const bool next_lds = keep_cnt <= (uint32_t)kBlock;
    // the parents' scores and history records, and their link tokens, are
    // in LDS when the step had at most kBlock parents; the row is, unless
    // the rank scratch took it
    const bool x_ok = ncur_now <= (uint32_t)kBlock;
    const bool row_ok = !ranks_done && K <= kMaxLdsTopk;
    auto emit = [&](uint32_t i, uint32_t o) {
      const NextRec c = next_in_lds ? sm.push_next[i] : nextc[i];
      const uint32_t j = c.jk >> 16, q = c.jk & 0xFFFFu;
      double ps;
      uint32_t phist;
      if (x_ok) {
        ps = sm.x_s[j];
        phist = sm.x_hist[j];
      } else {
        const CurRec p = cur[j];
        ps = p.s;
        phist = p.hist;
      }
      const float x = row_ok ? sm.row_lp[q] : rlp[(uint64_t)t * K + q];
      const uint32_t tk = row_ok ? sm.row_id[q] : rid[(uint64_t)t * K + q];
      // the parent's record gives the two links of the new one
      HistRec h;
      h.phist = phist;
      h.tok = tk;
      h.ptok = 0u;
      h.phist2 = kNoHist;
      if (phist < hist_cap) {
        const HistRec pr = hist[phist];
        h.ptok = pr.tok;
        h.phist2 = pr.phist;
      }
      ParEntry e{0u, 0u, (uint32_t)M_NONE, 0u, kNoCursor};
      uint32_t err = 0;
      if (next_table) {
        const uint32_t xtok = x_ok ? sm.x_tok[j] : kNoToken;
        if (xtok != kNoToken) {
          // a link parent that stays one, on its own edge: the entry
          // parent_entry() would build, from what its expansion read
          const uint32_t xsd = sm.x_sd[j];
          e.c0 = xsd;
          e.aux = xtok;
          e.mode = (t + 2 == xsd) ? M_LP_SEL : M_LP_NEXT;
          e.work = 1;
          e.lp = sm.x_tc[j] + 1u;
        } else if (t == 0u && tk < a.root_n) {
          // a child of the root: its entry from the root directory
          const uint4* rp = (const uint4*)&a.root_dir[tk];
          const uint4 rx = rp[0], ry = rp[1];
          if (rx.x == c.node && !(rx.y & kRdErr)) e = root_child_entry(a, rx, ry, K);
          else e = parent_entry<kLouds>(a, c.node, t + 1, K, &err);
        } else {
          e = parent_entry<kLouds>(a, c.node, t + 1, K, &err);
        }
      }
      const double s2 = ps + (double)x;
      st_cur(&cur2[o], s2, c.node, hist_used + o);
      hist[hist_used + o] = h;
      if (next_table) {
        if (err) atomicOr(&sm.status, (uint32_t)kStatusCorrupt);
        st_dev(&par_c0[o], e.c0);
        st_dev(&par_aux[o], e.aux);
        st_dev(&par_node[o], c.node);
        st_dev(&par_mode[o], e.mode);
        if (next_lds) {
          sm.p_c0[o] = e.c0;
          sm.p_aux[o] = e.aux;
          sm.p_node[o] = c.node;
          sm.p_mode[o] = (uint8_t)e.mode;
          sm.p_lp[o] = e.lp;
          sm.p_s[o] = s2;
          sm.p_hist[o] = hist_used + o;
        }
      }
    };
    // the survivors: all pushes in push order, or a list of positions in
    // sm.keep_idx; then one emit loop (a list longer than kKeepCap is
    // emitted as it is found)
    uint32_t n_emit = 0;
    bool from_list = false, list_done = true;
    if (bn.all) {
      n_emit = n_next;
      if (tid == 0) sm.n_out = n_next;
    } else if (listed) {
      // the boundary bin's survivors join the listed ones (a record is read
      // only for a key on the boundary of a cut tie)
      if (tid == 0) sm.n_keep = n_listed;
      __syncthreads();
      for (uint32_t b = tid; b < n_bin + ((kBlock - n_bin % kBlock) % kBlock); b += kBlock) {
        bool keep = false;
        uint32_t i = 0;
        if (b < n_bin) {
          const uint64_t key = ~sm.bin_key[b];
          i = sm.bin_idx[b];
          keep = key > bn.vkey ||
                 (key == bn.vkey && (!bn.tie || bound_keep(bn, key, na(i), nn(i))));
        }
        const uint32_t q = wave_append(keep, &sm.n_keep);
        if (keep && q < (uint32_t)kKeepCap) sm.keep_idx[q] = i;
      }
      __syncthreads();
      n_emit = min(sm.n_keep, (uint32_t)kKeepCap);
      from_list = true;
      if (tid == 0) sm.n_out = sm.n_keep;
    } else if (keep_cnt <= (uint32_t)kKeepCap) {
      // positions of the survivors first (from the keys alone; the rest of
      // a record is read only for a key on the boundary of a cut tie)
      visit_keys(n_next, nk, [&](uint32_t i, bool ok, uint64_t key) {
        bool keep = false;
        if (ok) {
          if (bn.all || key > bn.vkey) keep = true;
          else if (key == bn.vkey) keep = bound_keep(bn, key, bn.tie ? na(i) : 0u, nn(i));
        }
        const uint32_t o = wave_append(keep, &sm.n_out);
        if (keep && o < (uint32_t)kKeepCap) sm.keep_idx[o] = i;
      });
      __syncthreads();
      n_emit = min(sm.n_out, (uint32_t)kKeepCap);
      from_list = true;
    } else {
      list_done = false;
    }
    if (list_done) {
      // one dependent chain per survivor
      for (uint32_t o = tid; o < n_emit; o += kBlock)
        if (o < a.lay.cur_cap && hist_used + o < hist_cap)
          emit(from_list ? sm.keep_idx[o] : o, o);
    } else {
      for (uint32_t base = 0; base < n_next; base += kBlock) {
        const uint32_t i = base + tid;
        bool keep = false;
        if (i < n_next) {
          const NextRec c = nextc[i];
          keep = bound_keep(bn, c.key, bn.tie ? na(i) : 0u, c.node);
        }
        const uint32_t o = wave_append(keep, &sm.n_out);
        if (keep && o < a.lay.cur_cap && hist_used + o < hist_cap) emit(i, o);
      }
    }
    if (tid == 0) sm.multi_item = 0;  // for the next step's parent table
    // (also orders this step's LDS reads before the next step's writes)
    __syncthreads();
    n_cur = sm.n_out;
    if (tid == 0 && t < d.out_T) step_stats[(uint64_t)t * kStepStats + 5] = wall_clock64() - t1;
    if (n_cur != keep_cnt) {  // the bound must keep exactly keep_cnt
      if (tid == 0) sm.status |= kStatusCorrupt;
      __syncthreads();
      break;
    }
    hist_used += n_cur;
    {
      CurRec* tmp = cur; cur = cur2; cur2 = tmp;
      cur_which ^= 1u;
    }
    par_ready = next_table;
    t_sel += wall_clock64() - t1;
  }
  // release the helpers
  if (tid == 0) st_dev(&ctl->go, tag | kGoExit);

  // ---- output: selected in ascending (norm, node id) -----------------------
  // (out_host's block is formed as an offset from `ob`, so that the
  // compiler keeps global -- not flat -- stores for it: a mapped host
  // address is a global one too)
  uint8_t* rb = ob;
  if constexpr (kStreamed) rb = ob + (int64_t)(uni((uint64_t)sm.res_host) - (uint64_t)ob);
  OutHeader* oh = (OutHeader*)rb;
  double* onorm = (double*)(rb + sizeof(OutHeader));
  uint32_t* olen = (uint32_t*)(onorm + F);
  uint32_t* otok = olen + F;
  const uint32_t status = sm.status;
  if (status == 0) {
    uint64_t* rk_key = (uint64_t*)sm.row_id;
    uint32_t* rk_node = (uint32_t*)sm.row_lp;
    // result j, of rank cntless among the selected, into output row cntless
    auto put = [&](const SelRec& me, uint32_t cntless) {
      if (cntless >= F) return;
      onorm[cntless] = me.s * lnf[me.depth];
      olen[cntless] = me.depth;
      uint32_t* row = otok + (uint64_t)cntless * d.out_T;
      if (me.depth >= 1 && me.depth <= d.out_T) {
        row[me.depth - 1] = me.tok;
        // each record holds its token and its parent's: two per load
        uint32_t h = me.phist;
        for (int pos = (int)me.depth - 2; pos >= 0; pos -= 2) {
          if (h >= hist_cap) break;
          const HistRec hr = hist[h];
          row[pos] = hr.tok;
          if (pos >= 1) row[pos - 1] = hr.ptok;
          h = hr.phist2;
        }
      }
    };
    if (nS > 0 && nS <= (uint32_t)kBlock / 2) {
      // few results: 2^ls (2..16) neighbouring lanes rank each one, each
      // over its own slice of `per` entries, and add their counts up
      uint32_t ls = 1;
      while (ls < 4 && (nS << (ls + 1)) <= (uint32_t)kBlock) ++ls;
      const uint32_t j = tid >> ls, sub = tid & ((1u << ls) - 1u);
      const uint32_t per = (((nS + (1u << ls) - 1u) >> ls) + 15u) & ~15u;
      // (per << ls) <= nS + (16 << ls) <= kRankChunk: the slices fit
      uint64_t myk = 0;
      uint32_t myn = 0, cntless = 0;
      SelRec me;
      if (j < nS) {
        me = selA[j];
        myk = norm_key(me.s * lnf[me.depth]);
        myn = me.node;
      }
      __syncthreads();
      if (tid < (per << ls)) {
        if (tid < nS) {
          const SelRec o = selA[tid];
          rk_key[tid] = norm_key(o.s * lnf[o.depth]);
          rk_node[tid] = o.node;
        } else {
          rk_key[tid] = kRankPad;
          rk_node[tid] = 0;
        }
      }
      __syncthreads();
      if (j < nS) cntless = count_before<8>(rk_key + sub * per, rk_node + sub * per, per, myk, myn);
      for (uint32_t o = 1; o < (1u << ls); o <<= 1) cntless += __shfl_xor(cntless, o, 64);
      if (j < nS && sub == 0) put(me, cntless);
    }
    for (uint32_t jb = 0; nS > (uint32_t)kBlock / 2 && jb < nS; jb += kBlock) {
      const uint32_t j = jb + tid;
      uint64_t myk = 0;
      uint32_t myn = 0, cntless = 0;
      SelRec me;
      if (j < nS) {
        me = selA[j];
        myk = norm_key(me.s * lnf[me.depth]);
        myn = me.node;
      }
      for (uint32_t ib = 0; ib < nS; ib += kRankChunk) {
        const uint32_t i = ib + tid;
        __syncthreads();
        if (tid < (uint32_t)kRankChunk && i < nS) {
          if (ib == jb) {  // entry i is the thread's own
            rk_key[tid] = myk;
            rk_node[tid] = myn;
          } else {
            const SelRec o = selA[i];
            rk_key[tid] = norm_key(o.s * lnf[o.depth]);
            rk_node[tid] = o.node;
          }
        } else if (tid < (uint32_t)kRankChunk) {
          rk_key[tid] = kRankPad;
          rk_node[tid] = 0;
        }
        __syncthreads();
        const uint32_t m = (min((uint32_t)kRankChunk, nS - ib) + 15u) & ~15u;
        if (j < nS) cntless += count_before<8>(rk_key, rk_node, m, myk, myn);
      }
      if (j < nS) put(me, cntless);
    }
  }
  __syncthreads();
  if constexpr (kStreamed) {
    const uint64_t so = step_stats_offset(d.F, d.out_T);
    const uint64_t* ss = (const uint64_t*)(ob + so);
    uint64_t* hs = (uint64_t*)(rb + so);
    for (uint32_t i = tid; i < d.out_T * kStepStats; i += kBlock) hs[i] = ss[i];
    // every thread's results have reached host memory before the header
    // says so (below)
    wait_stores();
    __syncthreads();
  }
  if (tid == 0) {
    oh->count = status ? 0 : nS;
    const unsigned long long tend = wall_clock64();
    oh->ticks_expand = t_exp;
    oh->ticks_select = t_sel;
    oh->ticks_total = tend - t_all0;
    oh->candidates = n_cands;
    oh->parents = sm.cnt_parents;
    oh->children = sm.cnt_children;
    oh->probes = sm.cnt_probes;
    if constexpr (kStreamed) {
      // published last: the host takes the request's results as soon as it
      // sees kStatusDone, while other requests may still be searching
      __hip_atomic_store(&oh->status, status | kStatusDone, __ATOMIC_RELEASE,
                         __HIP_MEMORY_SCOPE_SYSTEM);
    } else {
      oh->status = status;
    }
  }
}

// The no-allocation scratch (kScratchBytes per device, held from the first
// use of the library on a device until the process ends).  Host code never
// passes `scratch` itself to a kernel or a copy -- on the host the name is
// a stand-in, not a device address -- only the address scratch_address()
// looked up for the device.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

hipError_t scratch_address(int device, void** ptr) {
  if (device < 0 || device >= kMaxDevices || !ptr) return hipErrorInvalidValue;
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  if (cur != device) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[device] = p;
  }
  *ptr = g_scratch_ptr[device];
  return hipSuccess;
}

// One workgroup per slot: the slot's control block, claim words and done
// words, word by word.
__global__ void __launch_bounds__(128) clear_ctl_kernel(uint8_t* ws, uint64_t stride,
                                                        uint64_t ctl_off, uint64_t claims_off,
                                                        uint64_t dones_off, uint32_t claim_slots) {
  uint8_t* slot = ws + (uint64_t)blockIdx.x * stride;
  uint32_t* p = (uint32_t*)(slot + ctl_off);
  for (uint32_t i = threadIdx.x; i < (uint32_t)(sizeof(Ctl) / 4); i += blockDim.x) p[i] = 0u;
  unsigned long long* c = (unsigned long long*)(slot + claims_off);
  for (uint32_t i = threadIdx.x; i < claim_slots; i += blockDim.x) c[i] = 0ull;
  unsigned long long* dn = (unsigned long long*)(slot + dones_off);
  for (uint32_t i = threadIdx.x; i < 2u * claim_slots; i += blockDim.x) dn[i] = 0ull;
}

hipError_t clear_controls(uint8_t* ws, uint64_t stride, uint64_t ctl_off, uint64_t claims_off,
                          uint64_t dones_off, uint32_t claim_slots, uint32_t count,
                          hipStream_t stream) {
  if (count == 0) return hipSuccess;
  hipLaunchKernelGGL(clear_ctl_kernel, dim3(count), dim3(128), 0, stream, ws, stride, ctl_off,
                     claims_off, dones_off, claim_slots);
  return hipGetLastError();
}

// An ordinary launch: the protocol of the shared steps never makes a
// workgroup wait for one that is not running (helpers' slices are claimed,
// and the leader takes over the slices no helper has claimed), so the grid
// needs no co-residency guarantee.
hipError_t launch_tbs(const KArgs& args, hipStream_t stream, hipEvent_t start,
                      hipEvent_t stop) {
  const dim3 grid(args.batch * args.wgs), block(kBlock);
  if (args.louds_words) {
    if (args.ready) return hipErrorInvalidValue;  // (no streamed LOUDS search)
    hipExtLaunchKernelGGL((tbs_kernel<true, false>), grid, block, 0, stream, start, stop, 0,
                          args);
  } else if (args.ready) {
    hipExtLaunchKernelGGL((tbs_kernel<false, true>), grid, block, 0, stream, start, stop, 0,
                          args);
  } else {
    hipExtLaunchKernelGGL((tbs_kernel<false, false>), grid, block, 0, stream, start, stop, 0,
                          args);
  }
  return hipGetLastError();
}

// One thread per root child: its root-directory entry, from parent_entry at
// step 1 with scan limit 0 (so that a child with a hash table reports it;
// the search picks scan or lookup with its own limit, root_child_entry).
__global__ void __launch_bounds__(256) root_dir_kernel(KArgs a, RootEnt* dir, uint32_t root_n,
                                                       uint32_t c0, uint32_t deg) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= deg) return;
  const uint32_t ch = c0 + i;
  const ft_node_rec r = a.recs[ch];
  if (r.first_tok >= root_n) return;  // (the host sized the directory on these tokens)
  uint32_t err = 0;
  const ParEntry e = parent_entry<false>(a, ch, 1u, 1u, &err);
  const uint32_t sd = r.meta & FT_META_DEPTH_MASK;
  const uint32_t el = (r.meta >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
  const bool link = (r.meta & FT_META_TERMINAL) && sd > 1u;
  uint32_t f = 0;
  if ((r.meta & FT_META_TERMINAL) && el == 1u) f |= kRdSel;
  if (link) f |= kRdLink;
  if ((e.mode & kModeMask) == M_HASH)
    f |= kRdTable | ((e.mode & kModeFiltered) ? kRdFiltered : 0u) | ((e.aux & 0xFFu) << 8);
  if (err) f |= kRdErr;
  RootEnt o;
  o.node = ch;
  o.flags = f;
  o.c0 = r.child_begin;
  o.deg = a.recs[ch + 1].child_begin - r.child_begin;
  o.tab = (f & kRdTable) ? e.c0 : 0u;
  o.link_tok = link ? e.aux : 0u;
  o.link_lp = link ? e.lp : kNoCursor;
  o.sd = sd;
  dir[r.first_tok] = o;
}

hipError_t launch_root_dir(const KArgs& args, RootEnt* dir, uint32_t root_n, uint32_t c0,
                           uint32_t deg, hipStream_t stream) {
  if (deg == 0) return hipSuccess;
  KArgs a = args;
  a.scan_limit = 0;
  hipLaunchKernelGGL(root_dir_kernel, dim3((deg + 255u) / 256u), dim3(256), 0, stream, a, dir,
                     root_n, c0, deg);
  return hipGetLastError();
}

int tbs_block_threads() { return kBlock; }

int tbs_max_resident_blocks(int num_cus) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)tbs_kernel<false, false>,
                                                   kBlock, 0) != hipSuccess)
    return 0;
  return per_cu * num_cus;
}

}  // namespace ftk
