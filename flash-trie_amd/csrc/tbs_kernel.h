// tbs_kernel.h -- structures shared by the TBS kernel and its host runtime.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/flashtrie_amd.h"

namespace ftk {

// Largest K whose proposal row is staged in LDS (8 bytes per proposal);
// a longer row is searched where it is staged, in device memory.
constexpr uint32_t kMaxLdsTopk = 4096;
// Largest K: a candidate's position in its row is packed into 16 bits.
constexpr uint32_t kMaxTopk = 65535;
// Parent index and proposal index are packed into 16 bits each.
constexpr uint32_t kMaxBeams = 65535;
constexpr uint32_t kNoHist = 0xFFFFFFFFu;

enum : uint32_t { kReqEarlyExit = 1u, kReqSkip = 2u };

enum : uint32_t {
  kStatusOverflow = 1u,  // candidate buffer too small (never expected)
  kStatusHistory = 2u,   // history capacity (max_num_inter_beams) exceeded
  kStatusCorrupt = 4u,   // a link-parent walk did not terminate
  kStatusWithdrawn = 8u, // streamed search: the host withdrew the request
  kStatusNotReady = 16u, // streamed search: its ready word never came
  kStatusStage = 32u,    // streamed search: the packed block is out of bounds
  // streamed search: set in the status word of a request's header in host
  // memory, written last (a system-scope release): its results are there
  kStatusDone = 0x80000000u,
};

// Streamed search: the ready word of a request, (launch epoch << 32) |
// (rows << kReadyRowsShift) | state, written by the host as the request's
// block is packed: kReadyPart once its length-norm table, beam widths and
// first `rows` rows (with their key bounds) are, kReadyOk once all of it
// is (rows = T), or kReadyWithdrawn when it failed to pack.  kReadyRk is
// added once a row has come out of order: from then on the proposal indices
// of every packed row are in the block, at the DevReq's planned rk_off.
enum : uint32_t { kReadyOk = 1u, kReadyWithdrawn = 2u, kReadyPart = 4u, kReadyRk = 8u };
// The split of a streamed request between its first ready word and the
// rest: the first row h >= head_rows (head_rows > 0) with h * K a multiple of
// 8, so that every row array (u32 tokens, f32 logps, u16 indices) splits on
// a 16-byte boundary; T (no split) when there is none before T.  The host
// and the kernel compute it alike.
__host__ __device__ inline uint32_t stream_split(uint32_t head_rows, uint32_t T, uint32_t K) {
  if (head_rows == 0 || head_rows >= T) return T;
  uint32_t h = head_rows;
  while (h < T && ((uint64_t)h * K) % 8u != 0u) ++h;
  return h;
}
// States of the copy word of a streamed search (Ctl::copy): claimed, done
// (with the row indices when kCopyRk is added too), or failed (the request
// was withdrawn or its rows never came).
enum : uint32_t { kCopyClaimed = 1u, kCopyDone = 2u, kCopyRk = 4u, kCopyFailed = 8u };
constexpr uint32_t kReadyRowsShift = 8;
constexpr uint32_t kReadyStateMask = 0xFFu;
// How long a leader waits for its ready word (wall-clock ticks of 10 ns):
// 1 s.  A request whose word does not come in time reports
// kStatusNotReady, and the host searches it again from the staged path.
constexpr unsigned long long kReadyTicks = 100000000ull;

// Per-request descriptor, packed by the host at the start of the staging
// buffer.  Offsets are relative to in_off; the block holds lnf[T + 1] (f64,
// at offset 0), beams, key bounds, then the rows.
struct DevReq {
  uint32_t T, K, F, flags;
  float tok_thr;
  uint32_t kb_off;     // u64[2T]: per step, bounds of its next-list keys
  double sent_thr;
  uint64_t in_off;     // byte offset of this request's block in the stage
  uint32_t beams_off;
  // proposal rows in ascending token order: token (u32[T * K]), logp
  // (f32[T * K]) and the proposal's index in the caller's row (u16[T * K]);
  // rk_off is 0 when every row came in ascending order (index = position)
  uint32_t rid_off;
  uint32_t rlp_off;
  uint32_t rk_off;
  uint32_t in_bytes;   // bytes of the block the kernel reads (16-aligned)
  uint32_t out_T;      // token stride of the output rows
};
static_assert(sizeof(DevReq) == 64, "DevReq layout");

// A request's block, as planned, fits the stage (stage_bytes) and its
// arrays fit the block.  The host and the kernel evaluate it alike.
__host__ __device__ inline bool block_fits(uint64_t stage_bytes, const DevReq& d) {
  const uint64_t T = d.T, K = d.K;
  return d.in_off + d.in_bytes <= stage_bytes && (d.in_bytes & 15u) == 0 &&
         d.beams_off + 4 * T <= d.in_bytes && d.kb_off + 16 * T <= d.in_bytes &&
         d.rid_off + 4 * T * K <= d.in_bytes && d.rlp_off + 4 * T * K <= d.in_bytes &&
         d.rk_off + 2 * T * K <= d.in_bytes;
}

struct CurRec {     // a hypothesis kept in the beam
  double s;         // f64 sum of logps
  uint32_t node;
  uint32_t hist;    // its history record (kNoHist for the root)
};

struct NextRec {    // a push into `next`
  uint64_t key;     // order-preserving norm
  uint32_t node;
  uint32_t jk;      // parent slot << 16 | position in the token-sorted row
};

struct SelRec {     // a push into `selected`
  double s;
  uint32_t node;
  uint32_t depth;   // |Q|
  uint32_t phist;   // history record of the parent
  uint32_t tok;     // last token
  uint32_t jk;
  uint32_t isnew;   // pushed during the current step
};

// History record of a hypothesis kept in a beam: its last token and its
// parent's, the parent's record and the grandparent's, so that a result's
// tokens are read back two per dependent load.
struct HistRec {
  uint32_t phist;   // the parent's record (kNoHist: the parent is the root)
  uint32_t tok;     // the hypothesis's last token
  uint32_t ptok;    // the parent's last token (when phist != kNoHist)
  uint32_t phist2;  // the grandparent's record (when phist != kNoHist)
};
static_assert(sizeof(HistRec) == 16, "HistRec layout");

struct OutHeader {  // 64 bytes, then norms[F] f64, lengths[F], tokens[F*T]
  uint32_t count;
  uint32_t status;
  uint64_t ticks_expand, ticks_select, ticks_total;
  uint64_t candidates, parents, children, probes;
};
static_assert(sizeof(OutHeader) == 64, "OutHeader layout");

// Per-step profile written after the output tokens of each request:
// parents, work items, next pushes, selected pushes, expansion ticks,
// selection ticks, child records scanned, binary-search probes, and for a
// shared step the leader's waits after its own slice: for the helpers'
// claims (and its take-over of unclaimed slices) and for the claimed
// slices to be done (wall-clock ticks).
constexpr uint32_t kStepStats = 10;
__host__ __device__ inline uint64_t step_stats_offset(uint32_t F, uint32_t T) {
  return (sizeof(OutHeader) + 12ull * F + 4ull * F * T + 7) & ~7ull;
}

// Wide-node index, built by ft_create from the image: every node with at
// least `wide_min` children gets a two-choice bucketed cuckoo table
// token -> child id: 2^log2nb buckets of kBucketSlots slots (64 bytes,
// average load <= 1/2).  A token sits in bucket h1(tok) or h2(tok), and in
// h2(tok) only if h1(tok) is full (the build settles entries into their
// first bucket), so a lookup reads one bucket and reads the second only
// when the first is full and has no match.  A slot's token word carries kSlotSel when the
// child can close a key one token below its parent (terminal, one-token
// edge); an empty slot has child 0 (the root is nobody's child) and token
// word kSlotEmptyTok, which no stored token equals (a node with a child
// token >= kSlotEmptyTok gets no table), so a lookup can match token words
// alone and read the child word of the matching slot only.  Tables are
// found through a directory keyed by node id: 2^wdir_log2 groups of
// kDirSlots entries, one 64-byte line each; an entry sits in the first free
// slot of its home group fib_slot(node) or, when that is full, of the next
// groups in turn (load <= 1/2), so a lookup reads whole groups and stops at
// the first group with a free slot -- almost always after one read.
//
// Every bucket also has an 8-byte fingerprint word: byte s is
// wide_fp(token) of slot s, 0 for an empty slot.  For a table of at most
// 2^kFpMaxLog2 buckets (flag kWideFiltered), a lookup reads the fingerprint
// word of h1(tok) first -- and of h2(tok) when that word is full -- and
// reads no bucket when no byte matches: the token is not a child.  The
// fingerprints are 1/8 of a table's bytes (those of a small table stay
// cached across the K lookups of a step), and most lookups are misses that
// then read 8 bytes instead of a 64-byte bucket.
struct WideDir {        // one node's table (host side)
  uint32_t node;
  uint32_t log2nb;      // log2 of the bucket count (>= 1)
  uint32_t bucket_off;  // first bucket of the node's table
  uint32_t flags;       // kWideFiltered
};
constexpr uint32_t kDirSlots = 4;
struct WideDirGroup {   // kDirSlots directory entries (device side)
  uint32_t node[kDirSlots];        // kEmpty: a free slot
  uint32_t bucket_off[kDirSlots];
  uint32_t lgf[kDirSlots];         // log2nb | flags << 8
  uint32_t pad[kDirSlots];
};
static_assert(sizeof(WideDirGroup) == 64, "WideDirGroup layout");
constexpr uint32_t kWideFiltered = 1u;
constexpr uint32_t kFpMaxLog2 = 16;

// Root directory: the root's children indexed by their first token, one
// 32-byte entry per token below the largest child token + 1.  Step 0 looks
// a proposal up with one read of 8 bytes (node, flags) instead of a
// fingerprint word and a 64-byte bucket, and its emit builds a survivor's
// parent-table entry for step 1 from the same entry (one 32-byte read)
// instead of the node's record, its table-directory group and, for a link
// parent, its pending token.  Built on the device from parent_entry itself
// at context creation; node 0 (the root, never a child) marks a token with
// no child.
struct RootEnt {
  uint32_t node;      // the child, 0: none
  uint32_t flags;     // kRd* | log2 table size << 8
  uint32_t c0, deg;   // first child and degree of the child
  uint32_t tab;       // its hash table's first bucket (kRdTable)
  uint32_t link_tok;  // a link parent (kRdLink): its token of step 1
  uint32_t link_lp;   // ... and that token's index in tail[] (or none)
  uint32_t sd;        // its string depth
};
static_assert(sizeof(RootEnt) == 32, "RootEnt layout");
constexpr uint32_t kRdSel = 1u;       // closes a key of length 1
constexpr uint32_t kRdLink = 2u;      // a link parent at step 1
constexpr uint32_t kRdTable = 4u;     // has a hash table
constexpr uint32_t kRdFiltered = 8u;  // ... with fingerprint filtering
constexpr uint32_t kRdErr = 16u;      // its entry could not be built
// Largest directory built (entries); a root with larger child tokens keeps
// its hash table or binary search.
constexpr uint32_t kRootDirMax = 1u << 25;
constexpr uint32_t kBucketSlots = 8;
struct WideBucket {
  uint32_t tok[kBucketSlots];
  uint32_t child[kBucketSlots];
};
static_assert(sizeof(WideBucket) == 64, "WideBucket layout");
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
constexpr uint32_t kSlotSel = 0x80000000u;
constexpr uint32_t kTokMask = 0x7FFFFFFFu;
constexpr uint32_t kSlotEmptyTok = 0x7FFFFFFFu;
__host__ __device__ inline uint32_t fib_slot(uint32_t x, uint32_t log2n) {
  return log2n ? (uint32_t)((x * 0x9E3779B1u) >> (32 - log2n)) : 0u;
}
__host__ __device__ inline uint32_t cuckoo_h1(uint32_t tok, uint32_t lg) {
  return (tok * 0x9E3779B1u) >> (32 - lg);
}
// 8-bit token fingerprint in [1, 255] (0 marks an empty slot)
__host__ __device__ inline uint32_t wide_fp(uint32_t tok) {
  const uint32_t f = ((tok & 0x7FFFFFFFu) * 0x2545F491u) >> 24;
  return f ? f : 1u;
}
__host__ __device__ inline uint32_t cuckoo_h2(uint32_t tok, uint32_t lg) {
  uint32_t h = (tok ^ 0x2545F491u) * 0x85EBCA6Bu;
  h ^= h >> 13;
  h *= 0xC2B2AE35u;
  const uint32_t b = h >> (32 - lg);
  return b == cuckoo_h1(tok, lg) ? b ^ 1u : b;
}

// Per-request control block shared by the request's leader and helper
// workgroups.  `go` sits on its own 128-byte line.
constexpr uint32_t kGoExit = 0xFFFFFFFFu;
struct Ctl {
  unsigned long long go;  // (launch epoch << 32) | generation of the shared step
  uint32_t pad0[30];
  uint32_t pad1[32];
  // the shared step, written by the leader before `go`
  uint32_t t, W, n_par, nS;
  uint32_t sel_which, cur_which, status;
  uint32_t hist_n;  // history records written before the step
  // pushes of the step into `next` (low 32 bits) and `selected` (high 32
  // bits): one 64-bit atomic add a workgroup
  unsigned long long pushes;
  // streamed search: (launch epoch << 32) | 1 once the leader has copied
  // the request's first rows to the device stage
  unsigned long long head;
  unsigned long long pad4;
  // streamed search: the copy of the rows after the first ready word's
  // (launch epoch << 32) | kCopy* state, claimed by helper 1 or the leader
  unsigned long long copy;
  uint32_t pad3[16];
};
static_assert(sizeof(Ctl) == 384, "Ctl layout");

struct WsLayout {   // byte offsets inside one request's workspace slot
  uint64_t cur0, cur1, nextc, selA, selB, rank, hist;
  uint64_t ctl, par_c0, par_aux, par_node, par_mode, par_woff;
  // claim words of a shared step's slices, one per workgroup of the
  // request: (launch epoch << 32) | generation of the step it was taken for
  uint64_t claims;
  // done words, 16 bytes per workgroup: the (epoch, generation) of the last
  // shared step whose slice it finished, then its children scanned (low
  // 32 bits) and buckets read (high) in that slice, written before it
  uint64_t dones;
  uint32_t next_cap, sel_cap, hist_cap, cur_cap;
  uint32_t claim_slots, pad;
};

struct KArgs {
  const ft_node_rec* recs;
  const uint32_t* parent;
  const uint32_t* tail;
  const DevReq* reqs;
  const uint8_t* stage;
  uint8_t* ws;
  uint64_t ws_stride;
  uint8_t* out;
  uint64_t out_stride;
  WsLayout lay;
  uint32_t batch;
  uint32_t scan_limit;
  const WideDirGroup* wdir;  // null: no wide-node index
  const WideBucket* wtab;
  const uint64_t* wfp;   // fingerprint word per bucket
  const uint32_t* labels;  // per node: first token | kSlotSel
  uint32_t wdir_log2;
  uint32_t wide_min;
  uint32_t wgs;        // workgroups per request (1 leader + wgs-1 helpers)
  uint32_t share_min;  // work items from which a step is shared
  uint32_t epoch;      // launch counter (tags the control words)
  // helpers never claim their slices (a test of the leader's take-over of
  // unclaimed slices; never set otherwise)
  uint32_t no_claims;
  // streamed search: rows of a request its first ready word carries (0:
  // all of them); helper 1 copies the rest once the host has packed them
  uint32_t head_rows;
  // Child ranges from the LOUDS rank/select directory instead of the node
  // records' child_begin (null: records), see LoudsDir.
  const uint64_t* louds_words;  // the LOUDS bits, 64 a word
  const uint32_t* louds_z;      // zeros before each 512-bit block
  const uint32_t* louds_s;      // block of every kLoudsSel-th zero
  // Streamed search (null otherwise): `reqs` and the staged blocks sit in
  // host memory mapped for the device (stage_src), where the host packs
  // each request after the launch.  A request's leader waits for its ready
  // word, copies its block to `stage` (stage_bytes long), and writes its
  // results (header, norms, lengths, tokens) to out_host instead of `out`,
  // where the per-step profile is kept during the search and copied to
  // out_host at the end.
  const uint8_t* stage_src;
  const unsigned long long* ready;
  uint8_t* out_host;
  uint64_t stage_bytes;
  // how long a leader (or helper 1) waits for a ready word, in wall-clock
  // ticks: kReadyTicks, or less when a test asks for it
  uint64_t ready_ticks;
  // the root directory (null: none) and its entries; root_force: step 0
  // uses it even where the root's children would be scanned (tests)
  const RootEnt* root_dir;
  uint32_t root_n;
  uint32_t root_force;
};

// LOUDS directory of the trie's shape: for every node v in breadth-first
// order, deg(v) one bits then one zero bit, so zero v sits at bit
// child_begin(v + 1) + v - 1 and node v's children are the ids
// [select0(v - 1) - v + 2, select0(v) - v + 1) (select0(-1) = -1).
// select0(i): the sample louds_s[i / kLoudsSel] and the next one bound the
// 512-bit block holding zero i; the block is found among them by binary
// search of louds_z (zeros before each block), and the zero within the
// block's 8 words by popcounts.  2 bits per node plus 1/64 of that for
// louds_z and ~1/128 for louds_s.
constexpr uint32_t kLoudsSel = 256;
constexpr uint32_t kLoudsBlockBits = 512;

// Launches the search over `batch` requests (wgs workgroups each) on
// `stream` (an ordinary launch: no workgroup waits for one that may not be
// resident, see tbs_kernel.hip).
// (start / stop, when given, are updated with the kernel's own start and
// stop times: events attached to its dispatch, not markers around it)
hipError_t launch_tbs(const KArgs& args, hipStream_t stream, hipEvent_t start = nullptr,
                      hipEvent_t stop = nullptr);

// Fills the root directory `dir` (root_n entries, zeroed by the caller)
// from the root's `deg` children starting at node c0, on `stream`.  `args`
// needs the image and wide-index fields only.
hipError_t launch_root_dir(const KArgs& args, RootEnt* dir, uint32_t root_n, uint32_t c0,
                           uint32_t deg, hipStream_t stream);

// The no-allocation scratch: one file-scope device array of this many
// bytes per device, holding a search's staged requests, outputs and
// workspace slots when the caller cannot allocate.
constexpr uint64_t kScratchBytes = 128ull << 20;

// Device address of the scratch array on `device`, which must be the
// current device.  Looked up once per device (hipGetSymbolAddress) and
// kept; later calls return the kept address.
hipError_t scratch_address(int device, void** ptr);

// Zeroes the control block (Ctl, at byte ctl_off), the claim words
// (claim_slots of them at claims_off) and the done words (2 * claim_slots
// at dones_off) of `count` workspace slots of `stride` bytes from `ws`,
// with a fill kernel on `stream`.
hipError_t clear_controls(uint8_t* ws, uint64_t stride, uint64_t ctl_off, uint64_t claims_off,
                          uint64_t dones_off,
                          uint32_t claim_slots, uint32_t count, hipStream_t stream);

// Workgroups of the search kernel that fit on the device at once.
int tbs_max_resident_blocks(int num_cus);

// Threads per workgroup of the search kernel.
int tbs_block_threads();

}  // namespace ftk
