/*
 * flashtrie_amd.h -- C ABI of the MI355X (gfx950) trie beam search library.
 *
 * The library holds one trie image in HBM plus a per-request workspace and
 * runs the reference's constrained trie beam search (TBS) for a whole batch
 * in one persistent HIP kernel launch.  Plain pointers and sizes only; every
 * entry point returns 0 on success or a negative FT_E_* code and never
 * aborts or throws.
 *
 * Reference interfaces each entry point replaces (paths relative to the
 * reference repository):
 *   ft_create   -- the managed-memory trie + LoudsTrie::prefetch
 *                  (lib/marisa/grimoire/trie/louds-trie.cc:378-395) and the
 *                  device copy of the LoudsTrie object
 *                  (lib/marisa/grimoire/trie/tbs-kernels.cu:178-184)
 *   ft_reserve  -- LoudsTrie::init_tbs_gpu (tbs-kernels.cu:599-648) and
 *                  BeamSearchState (tbs-kernels.cu:57-90), reached from
 *                  Trie::init_tbs_gpu (lib/marisa/trie.cc:241-251)
 *   ft_stage    -- copy_input_to_gpu (tbs-kernels.cu:702-740)
 *   ft_launch   -- tbs_gpu_launch_async (tbs-kernels.cu:650-671), one
 *                  launch for the whole batch instead of one per request
 *   ft_fetch    -- copy_output_to_cpu (tbs-kernels.cu:742-835)
 *   ft_search   -- LoudsTrie::tbs_gpu / tbs_gpu_batched
 *                  (tbs-kernels.cu:673-700): stage + launch + fetch,
 *                  with the packing overlapping the search
 *   ft_destroy  -- ~BeamSearchState (tbs-kernels.cu:148-166)
 *
 * Search semantics are those of the reference CPU path LoudsTrie::tbs
 * (lib/marisa/grimoire/trie/louds-trie.cc:75-177), not of its CUDA kernel.
 */
#ifndef FLASHTRIE_AMD_H_
#define FLASHTRIE_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------
 * Trie image (host blob, uploaded verbatim to HBM by ft_create).
 *
 * Node ids are the reference's BFS ids (root 0, siblings in ascending
 * first-token order, lib/marisa/grimoire/trie/louds-trie.cc:477-588).  The
 * children of node n are the ids [rec[n].child_begin, rec[n+1].child_begin);
 * rec has num_nodes + 1 entries, the last one a sentinel.
 * ------------------------------------------------------------------------- */
typedef struct ft_node_rec {
  uint32_t child_begin; /* id of the first child */
  uint32_t first_tok;   /* first token of the edge into this node */
  uint32_t tail_off;    /* link nodes: offset of the edge string in tail[] */
  uint32_t meta;        /* FT_META_* bit fields below */
} ft_node_rec;

#define FT_META_TERMINAL 0x80000000u /* a key ends at this node */
#define FT_META_LINK 0x40000000u     /* edge has >= 2 tokens (in tail[]) */
#define FT_META_ELEN_SHIFT 16        /* edge length, 14 bits */
#define FT_META_ELEN_MASK 0x3FFFu
#define FT_META_DEPTH_MASK 0xFFFFu   /* string depth |KB(n)|, 16 bits */

#define FT_IMAGE_MAGIC "FTIMG01"

typedef struct ft_image_header {
  char magic[8];          /* FT_IMAGE_MAGIC */
  uint64_t num_nodes;     /* N (root included) */
  uint64_t num_keys;      /* terminal nodes */
  uint64_t tail_len;      /* tokens in tail[] */
  uint64_t recs_offset;   /* byte offset of rec[N + 1] (16-byte aligned) */
  uint64_t parent_offset; /* byte offset of parent[N] (uint32) */
  uint64_t tail_offset;   /* byte offset of tail[tail_len] (uint32) */
  uint64_t total_bytes;   /* size of the whole blob */
  uint32_t max_depth;     /* largest string depth */
  uint32_t reserved[7];
} ft_image_header;

/* ---------------------------------------------------------------------------
 * Error codes.
 * ------------------------------------------------------------------------- */
#define FT_OK 0
#define FT_E_ARG (-1)      /* invalid argument or null pointer */
#define FT_E_NOMEM (-2)    /* device or pinned host allocation failed */
#define FT_E_HIP (-3)      /* HIP runtime error */
#define FT_E_LIMIT (-4)    /* request exceeds the reserved workspace */
#define FT_E_STATE (-5)    /* ft_reserve / ft_stage not called */
#define FT_E_INPUT (-6)    /* malformed request (see ft_last_error) */
#define FT_E_IMAGE (-7)    /* malformed trie image */
#define FT_E_DEVICE (-8)   /* no usable gfx950 device */
#define FT_E_KERNEL (-9)   /* the kernel reported an internal error */

/* ---------------------------------------------------------------------------
 * One request = one TbsInput (include/marisa/tbs_input.h:7-26).
 * ------------------------------------------------------------------------- */
typedef struct ft_request {
  const uint32_t* beams;    /* [num_beams] beam width per step; the final
                               beam F is beams[num_beams - 1] */
  uint32_t num_beams;
  uint32_t num_steps;       /* T = rows of topk_id / topk_logp */
  uint32_t topk;            /* K = proposals per row */
  const uint32_t* topk_id;  /* [num_steps * topk], row-major */
  const float* topk_logp;   /* [num_steps * topk], row-major */
  /* Optional alternative to topk_id / topk_logp: num_steps row pointers of
   * topk entries each (used when non-null, e.g. for nested vectors). */
  const uint32_t* const* topk_id_rows;
  const float* const* topk_logp_rows;
  float token_logp_threshold;
  double sent_logp_threshold;
  double length_norm;       /* alpha of (6 / (5 + |Q|))^alpha */
  int early_exit;
} ft_request;

/* Caller-owned result arrays for one request.  Results are in the
 * reference's output order: ascending normalised score, ties by ascending
 * node id (louds-trie.cc:168-176). */
typedef struct ft_result {
  uint32_t capacity;     /* beams that fit in the arrays below */
  uint32_t token_stride; /* uint32 slots per beam row of tokens */
  uint32_t count;        /* out: beams returned */
  int32_t status;        /* out: FT_OK, or the request's error code */
  double* logp_norm;     /* [capacity] */
  uint32_t* length;      /* [capacity] */
  uint32_t* tokens;      /* [capacity * token_stride] */
  double device_ms[4];   /* out: expansion, selection, other, total (device
                            wall clock of this request's workgroup) */
  uint64_t* step_stats;  /* optional [num_steps * FT_STEP_STATS]: per step
                            parents, work items, next pushes, selected
                            pushes, expansion and selection ticks (wall
                            clock), child records scanned, binary-search
                            probes, and for a step shared between
                            workgroups the leader's wait for the helpers'
                            claims and for their slices (ticks) */
} ft_result;

#define FT_STEP_STATS 10

/* Per-launch timing and work counters (filled by ft_fetch when non-null). */
typedef struct ft_timing {
  double kernel_ms;       /* HIP-event time of the last launch */
  double expand_ms;       /* summed per-request device phase time */
  double select_ms;
  double other_ms;
  uint64_t candidates;    /* next + selected pushes, summed over requests */
  uint64_t parents;       /* parents expanded */
  uint64_t children;      /* child records read by the scan path */
  uint64_t probes;        /* binary-search probes of the search path */
} ft_timing;

typedef struct ft_ctx ft_ctx;

/* Uploads a trie image (ft_image_header + arrays) to device `device`.
 * The whole image is validated on the host first (BFS child ranges, parent
 * links, edge lengths and depths, sibling order, token ids < 2^31 - 1, tail
 * bounds, key count); a malformed image returns FT_E_IMAGE before any
 * device call. */
int ft_create(const void* image, size_t image_bytes, int device,
              ft_ctx** out);

/* Allocates the per-request workspace once (device + pinned host), sized
 * for max_batch requests (init_tbs_gpu, tbs-kernels.cu:599-648).
 *   max_topk        bounds K, the proposals per row (at most 65535)
 *   max_steps       bounds T, the rows per request (at most 16383)
 *   max_out_beams   bounds every beam width and the final beam F
 *   max_out_tokens  bounds F * T per request
 *   max_inter_beams bounds the hypotheses kept in history per request */
int ft_reserve(ft_ctx* ctx, size_t max_batch, size_t max_topk,
               size_t max_steps, size_t max_out_beams,
               size_t max_out_tokens, size_t max_inter_beams);

/* Validates and packs `batch` requests into pinned memory and copies them to
 * the device workspace (async on the context stream).  It first waits for
 * the previous staging copy, which may still be queued behind a running
 * launch, so the pinned buffer is never rewritten under it.  Staging starts
 * a new batch: results of earlier launches can no longer be fetched. */
int ft_stage(ft_ctx* ctx, const ft_request* reqs, size_t batch);

/* Launches the search kernel over the staged batch (async); at most
 * max_batch requests. */
int ft_launch(ft_ctx* ctx);

/* Grows the staging and result buffers to hold `max_staged` requests, so a
 * larger set can be staged once and searched in ranges (device-resident
 * inputs).  Workspace slots stay at max_batch. */
int ft_reserve_staging(ft_ctx* ctx, size_t max_staged);

/* Launches the staged requests [first, first + count), count <= max_batch
 * (async). */
int ft_launch_range(ft_ctx* ctx, size_t first, size_t count);

/* Kernel durations of the last n launches, oldest first; waits for the
 * stream.  At most 1024 are kept.  A launch of staged requests
 * (ft_launch, ft_launch_range) is timed by HIP events attached to its
 * dispatch (its start to its end); a streamed search (ft_search) by events
 * recorded around it, which also span the queue's time between them. */
int ft_launch_times(ft_ctx* ctx, double* ms, size_t n);

/* Waits for the last launch, copies results back, fills `results`.  A
 * staged request that no ft_launch / ft_launch_range has covered since the
 * last ft_stage gets status FT_E_STATE and count 0 (the call then returns
 * FT_E_STATE); it never returns another launch's output. */
int ft_fetch(ft_ctx* ctx, ft_result* results, size_t batch,
             ft_timing* timing);

/* The results of stage + launch + fetch, streamed: the kernel is launched
 * once the batch's shapes are checked (errors of ft_stage's shape checks
 * come before any launch), then each request is packed into pinned host
 * memory mapped for the device while the kernel runs; a request's leader
 * starts when its request is packed, copies it to the device and writes its
 * results back to mapped host memory (no copy-engine transfers).  A request
 * that fails to pack is withdrawn with every later one, the kernel is
 * waited for, and the first error in request order is returned.  Afterwards
 * ft_fetch has nothing to fetch (FT_E_STATE).  timing->kernel_ms spans the
 * launch, which overlaps the packing. */
int ft_search(ft_ctx* ctx, const ft_request* reqs, size_t batch,
              ft_result* results, ft_timing* timing);

/* ft_search that hands each request's results over as soon as they are
 * there: fn(user, r) is called (on the calling thread) once results[r] is
 * filled and its status is FT_OK -- for a streamed search as each
 * request's leader finishes, while other requests of the batch may still
 * be searching -- so a caller can convert results while the rest run.  No
 * counterpart in the reference; it is what Trie::tbs_gpu_batched calls.
 * Return value, errors and results are those of ft_search (fn is not
 * called for a request with an error). */
typedef void (*ft_result_fn)(void* user, size_t r);
int ft_search_each(ft_ctx* ctx, const ft_request* reqs, size_t batch,
                   ft_result* results, ft_timing* timing, ft_result_fn fn,
                   void* user);

/* ft_search without allocating: no hipMalloc, hipHostMalloc or hipFree,
 * and no ft_reserve needed.  It has no counterpart in the reference; it is
 * for callers that must not allocate (tight serving loops, harnesses that
 * forbid hipMalloc).  The staged requests, outputs and workspace slots of
 * the batch live in one device array of FT_NOALLOC_SCRATCH_BYTES per
 * device, which the library holds from ft_create until the process ends;
 * host packing uses static buffers.  A batch that needs more (the
 * workspace of a request grows with beam x topk: batch 1 at beam = topk =
 * 1000 fits, batch 8 does at beam = topk = 350) returns FT_E_LIMIT; at
 * most 64 requests per call.  Results are identical to ft_search's.  It
 * is a synchronous call: it copies the packed batch from pageable host
 * memory, launches, copies the results back and waits for the context's
 * stream, so it cannot be recorded into a HIP graph (stream capture).
 * Calls in one process are serialised (they share the array, which keeps
 * the last call's contents; the control blocks are cleared on every
 * call); calls from different processes get their own copies. */
#define FT_NOALLOC_SCRATCH_BYTES (128u << 20)
int ft_search_noalloc(ft_ctx* ctx, const ft_request* reqs, size_t batch,
                      ft_result* results, ft_timing* timing);

/* Waits for the context stream; returns the HIP-event time of the last
 * launch in *ms. */
int ft_sync(ft_ctx* ctx, double* ms);

void ft_destroy(ft_ctx* ctx);

const char* ft_strerror(int code);

/* The id of the sources this library was built from (16 hex digits of a
 * sha256 over them); no counterpart in the reference.  Benchmarks and
 * profiles record it, so a figure names the exact build it measured. */
const char* ft_build_id(void);

/* Thread-local text of the most recent error raised on this thread. */
const char* ft_last_error(void);

/* Device properties the launch is sized from (for reports). */
int ft_device_info(ft_ctx* ctx, int* num_cus, int* lds_per_block,
                   int* wall_clock_khz, char* name, size_t name_len);

#ifdef __cplusplus
}
#endif

#endif /* FLASHTRIE_AMD_H_ */
