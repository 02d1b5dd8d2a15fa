/*
 * paged_decode.h -- C ABI of the MI355X (gfx950) split-K paged GQA decode operator.
 *
 * One-token attention decode over a paged KV cache:
 *   q      [batch, query_heads, head_dim]                     float32, float16 or bfloat16
 *   k, v   [physical_pages, page_size, kv_heads, head_dim]      same dtype as q (FP8 too: pd_decode_ex)
 *   table  [batch, table_width]  int32 physical page of each logical page
 *   lengths[batch]               int32 live tokens per sequence
 *   out    [batch, query_heads, head_dim]                     float32
 * out[b,h] = softmax(K q / sqrt(head_dim)) V over the live tokens of sequence b
 * through KV head h / (query_heads / kv_heads); an empty sequence gives zeros.
 * Token t of sequence b is at page table[b, t / page_size], offset
 * t % page_size. Tokens whose page id is outside [0, physical_pages) are
 * skipped, never dereferenced.
 *
 * Work is cut into `splits` partitions of `split_tokens` tokens, each cut into
 * four contiguous quarters; every quarter leaves one max-corrected softmax
 * state per query head in the caller's workspace, and a merge combines them:
 *   numerator [batch, query_heads, 4 * splits, head_dim]  float32
 *   stats     [batch, query_heads, 4 * splits, 2]         float32 (max, denominator)
 * (state 4 * split + quarter; the reference's workspace shape, decode.cu:223-231;
 * a full call with length bounds may lay it out for a coarser split, see pd_decode).
 * Where one workgroup of the partition stage holds several quarters of a
 * partition (few KV heads: 16-head GQA tiles with four quarters per
 * workgroup, or two quarters per workgroup), those quarters are stored
 * combined in the first one's state and the others hold the empty state
 * (max -FLT_MAX, denominator 0), which every merge reads as an identity;
 * pd_decode / pd_decode_ex then merge the combined states only.
 * Only partitions that hold at least one token of their sequence are written
 * (partitions 0 .. ceil(len_b / split_tokens) - 1 of row b, len_b clamped to
 * table_width * page_size) and only those are read by the merge, so the
 * workspace needs no initialisation and a batch with ragged lengths neither
 * writes nor reads states past each sequence's end.
 *
 * All pointers are device pointers. `stream` is a hipStream_t (passed as
 * void* so FFI layers need no HIP headers); calls are asynchronous on it, never
 * allocate, never synchronise, and may be captured into a hipGraph. A call is
 * not reentrant for one workspace: use separate workspaces on concurrent
 * streams.
 *
 * Every function returns PD_OK or a PD_ERR_* code; on error nothing is
 * launched (except PD_ERR_LAUNCH, reported by the runtime after submission).
 */
#ifndef PAGED_DECODE_H
#define PAGED_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum pd_status {
    PD_OK = 0,
    PD_ERR_NULL_POINTER = 1,  /* a required pointer is NULL */
    PD_ERR_SHAPE = 2,         /* a dimension is outside the supported range */
    PD_ERR_DTYPE = 3,         /* unsupported dtype combination, or a scale not finite and > 0 */
    PD_ERR_SPLIT = 4,         /* splits / split_tokens outside their range */
    PD_ERR_MERGE = 5,         /* unknown merge mode or shared-merge bound exceeded */
    PD_ERR_LAUNCH = 6,        /* the HIP runtime rejected a kernel launch */
    PD_ERR_HINT = 7,          /* unknown bits in the hints argument */
    PD_ERR_SCRATCH = 8,       /* pd_decode_scratch: the workspace does not fit PD_SCRATCH_BYTES */
    PD_ERR_PREFIX = 9         /* malformed shared-prefix runs (pd_decode_prefix) */
};

/* Storage formats. q, k and v share F32, F16 or BF16 in pd_decode; the _ex
 * entries also take K/V in FP8 (OCP e4m3 / e5m2, one byte per element) with
 * an F16 or BF16 q. */
enum pd_dtype {
    PD_DTYPE_F32 = 0,
    PD_DTYPE_F16 = 1,
    PD_DTYPE_BF16 = 2,
    PD_DTYPE_FP8_E4M3 = 3,
    PD_DTYPE_FP8_E5M2 = 4
};

/* Merge strategies, numbered as the reference's merge_mode argument. */
enum pd_merge { PD_MERGE_SERIAL = 0, PD_MERGE_SHARED = 1 };

/* Largest state count (4 * splits) the LDS-bounded (shared) merge accepts. */
#define PD_SHARED_MERGE_MAX_PARTS 4096

/*
 * Hints of the _ex entries (a bit set; 0 = none). They only choose how the
 * partition kernel runs, never what it computes:
 *   PD_HINT_UNSHARED_PAGES: no physical page holds live tokens of more than
 *   one sequence (no shared prefix pages). The partition kernel may then
 *   stream K/V past the caches, which is faster when nothing is read twice;
 *   without it, pages that several sequences share stay cacheable. Passing it
 *   for a batch that does share pages is still correct, only slower. Results
 *   are bit-identical with or without it.
 *   PD_HINT_RAGGED_LENGTHS: the sequence lengths differ widely (live tokens
 *   under about 80% of batch x longest). Grids of up to eight 8-wave
 *   workgroups per CU then run in smaller workgroups, which balance ragged
 *   batches better. Results agree to FP32 rounding (the quarters of a
 *   partition are folded in another grouping); a wrong hint is only slower.
 */
enum pd_hint { PD_HINT_NONE = 0, PD_HINT_UNSHARED_PAGES = 1, PD_HINT_RAGGED_LENGTHS = 2 };

/*
 * Full decode on `stream`: a partition launch that writes 4 * splits states
 * per (sequence, query head) row into numerator/stats, then a merge launch
 * that combines them into out. A call whose rows hold at most 128 KB of K and
 * V per (sequence, KV head) -- min(splits * split_tokens, table_width *
 * page_size) tokens -- is instead one whole-row launch: each workgroup
 * folds a row's states in LDS and writes out itself, and numerator/stats
 * are left unwritten (they remain required arguments, the workspace of the
 * reference's plan). Results agree with the two-launch path to FP32
 * rounding; pd_decode_launch_count says which a call takes. With length
 * bounds (pd_decode_ex, pd_decode_scratch) on grids with many waves per CU
 * the two launches run over coarser partitions, a power of two times
 * split_tokens, whose fewer states the workspace holds
 * (pd_decode_kernel_split says which); the workspace's contents are
 * internal to the call.
 * Replaces the native entry `decode(q, k, v, table, lengths, numerator, stats,
 * out, split_tokens, merge_mode)` of reference
 * src/paged_decode/csrc/bindings.cpp:3-9 / decode.cu:197-246, with the tensor
 * shapes passed explicitly. Limits (decode.cu:209-235): 1 <= batch,
 * query_heads <= 65535; head_dim in {64, 128}; page_size in {16, 32};
 * query_heads % kv_heads == 0; 1 <= table_width <= 65536; 1 <= splits <= 65535;
 * 1 <= split_tokens <= 1048576; merge_mode PD_MERGE_SHARED needs
 * 4 * splits <= PD_SHARED_MERGE_MAX_PARTS.
 */
int pd_decode(const void* q, const void* k, const void* v, int dtype,
              const int32_t* table, const int32_t* lengths,
              float* numerator, float* stats, float* out,
              int batch, int query_heads, int kv_heads, int head_dim, int page_size,
              int table_width, int physical_pages, int splits, int split_tokens,
              int merge_mode, void* stream);

/*
 * pd_decode with separate q and K/V formats and per-tensor K/V scales: the
 * attention runs over K' = k_scale * k and V' = v_scale * v. Supported pairs
 * (q_dtype, kv_dtype): (F32, F32), (F16, F16), (BF16, BF16), and F16 or BF16
 * q with FP8_E4M3 or FP8_E5M2 K/V (dequantized exactly in the gather; the
 * scales are applied to the scores and to the output, not per element).
 * Scales must be finite and > 0 (PD_ERR_DTYPE otherwise). Extends the
 * reference's dtype set (decode.cu:215-218: float16, float32); BF16 and FP8
 * KV are listed as future work there (docs/DESIGN.md:97-99).
 *
 * length_bounds: NULL, or a HOST array [batch] of upper bounds on the device
 * lengths the call will find, read during the call (so a captured launch
 * keeps the values of its capture). With bounds, batches of up to 64
 * sequences launch only the partitions the bounds reach, plus one workgroup
 * per 8 partitions past them for lengths that grew on the device since
 * (ragged-batch work-list compaction, reference docs/DESIGN.md:80-82). A
 * bound below the device length is still correct, only slower: the
 * partitions past it run on those fewer workgroups. Results are the same
 * with or without bounds up to the last bits (other launch shapes fold the
 * quarters in another grouping).
 */
int pd_decode_ex(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype,
                 float k_scale, float v_scale,
                 const int32_t* table, const int32_t* lengths,
                 float* numerator, float* stats, float* out,
                 int batch, int query_heads, int kv_heads, int head_dim, int page_size,
                 int table_width, int physical_pages, int splits, int split_tokens,
                 int merge_mode, int hints, const int32_t* length_bounds, void* stream);

/* Partition stage of pd_decode_ex (same hints and length bounds). */
int pd_decode_partial_ex(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype,
                         float k_scale, float v_scale,
                         const int32_t* table, const int32_t* lengths,
                         float* numerator, float* stats,
                         int batch, int query_heads, int kv_heads, int head_dim, int page_size,
                         int table_width, int physical_pages, int splits, int split_tokens,
                         int hints, const int32_t* length_bounds, void* stream);

/*
 * Shared prefixes. pd_prefix_runs describes which sequences of a HOST page
 * table [batch, table_width] share leading pages: runs[2 b] is sequence b's
 * leader -- the first sequence whose row starts with the same page id (b
 * itself if none before it does), or -1 if b's first entry is negative -- and
 * runs[2 b + 1] is the number of leading entries b's row has in common with
 * its leader's (up to the first difference or negative entry). runs is a
 * HOST array [2 * batch]. Returns a status.
 *
 * pd_decode_prefix and pd_decode_partial_prefix are pd_decode_ex and
 * pd_decode_partial_ex with such runs (a HOST array read during the call, or
 * NULL). With runs and length bounds, a work-list launch (batches of up to 64
 * sequences, F16 or BF16 q, GQA groups of up to 8) scores each partition
 * that lies inside the common prefix of several sequences once for up to
 * 16 / GT of them (GT: the GQA group padded to a power of two), reading its
 * K and V once instead of once per sequence. A rectangular grid (lengths
 * close to equal) becomes such a work list where the items remove enough of
 * it and the rest still fill the device; a full call may then run over half
 * the partition span it takes without runs (pd_decode_kernel_split), where
 * only the finer span lets the items pay. The runs are a promise about the
 * device table: on the leading entries they cover, the rows of one leader's
 * sequences must hold the same page ids, or those sequences get wrong
 * results (runs computed from the table uploaded to the device keep it).
 * Runs with a leader outside [-1, batch) or a count outside [0, table_width]
 * return PD_ERR_PREFIX. Results equal those without runs up to the last
 * bits. No counterpart in the reference, whose kernel reads a shared page
 * once per sequence that maps it (its workload has no sharing,
 * src/paged_decode/workload.py:12-13; reuse across readers is left open,
 * docs/DESIGN.md:24-26).
 */
int pd_prefix_runs(const int32_t* table, int batch, int table_width, int32_t* runs);
int pd_decode_prefix(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype,
                     float k_scale, float v_scale,
                     const int32_t* table, const int32_t* lengths,
                     float* numerator, float* stats, float* out,
                     int batch, int query_heads, int kv_heads, int head_dim, int page_size,
                     int table_width, int physical_pages, int splits, int split_tokens,
                     int merge_mode, int hints, const int32_t* length_bounds, const int32_t* prefix_runs,
                     void* stream);
int pd_decode_partial_prefix(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype,
                             float k_scale, float v_scale,
                             const int32_t* table, const int32_t* lengths,
                             float* numerator, float* stats,
                             int batch, int query_heads, int kv_heads, int head_dim, int page_size,
                             int table_width, int physical_pages, int splits, int split_tokens,
                             int hints, const int32_t* length_bounds, const int32_t* prefix_runs, void* stream);

/*
 * Partition stage only (the first launch of pd_decode): fills numerator and
 * stats. Replaces the partial_decode launch of reference decode.cu:176-182.
 */
int pd_decode_partial(const void* q, const void* k, const void* v, int dtype,
                      const int32_t* table, const int32_t* lengths,
                      float* numerator, float* stats,
                      int batch, int query_heads, int kv_heads, int head_dim, int page_size,
                      int table_width, int physical_pages, int splits, int split_tokens,
                      void* stream);

/*
 * Merge stage only (the second launch of pd_decode): combines the live states
 * of each (sequence, query head) row -- 4 * ceil(len_b / split_tokens) of the
 * 4 * splits allocated, empty states included -- into out. Replaces the
 * merge_decode / merge_shared launches of reference decode.cu:183-193. Where
 * the partition stage combined quarters, pd_decode itself merges only the
 * combined states, so the two can differ in the last bits (sums in another
 * order). lengths, page_size, table_width and
 * split_tokens are the values the partition stage was called with.
 */
int pd_decode_merge(const float* numerator, const float* stats, float* out,
                    const int32_t* lengths, int batch, int query_heads, int head_dim,
                    int page_size, int table_width, int splits, int split_tokens,
                    int merge_mode, void* stream);

/*
 * pd_decode_ex without a caller workspace: the partition states live in a
 * static device array of the library, PD_SCRATCH_BYTES per device, held
 * from the library's load on a device until the process exits. No
 * counterpart in the reference (whose workspace the plan allocates,
 * src/paged_decode/runtime.py:64-68); it is for callers that cannot
 * allocate: code under hipGraph capture, tight serving loops, harnesses
 * that forbid hipMalloc. The call allocates and frees nothing.
 *
 * Limit: the states must fit, numerator bytes rounded up to 256 plus stats
 * bytes <= PD_SCRATCH_BYTES, i.e.
 *   ceil(batch * query_heads * 4 * splits * head_dim * 4 / 256) * 256
 *     + batch * query_heads * 4 * splits * 2 * 4 <= PD_SCRATCH_BYTES
 * (Llama-3-8B B4 L4096 at split 256: 4.3 MB; 32 heads x 32K context at
 * split 128: 17 MB); larger requests return PD_ERR_SCRATCH before anything
 * is launched. The states need no initialisation (each call writes every
 * state it reads), so nothing is cleared between calls. Every call on one
 * device shares that device's array: calls that overlap on one device (on
 * different streams, or from several threads) race and must be serialised
 * by the caller. The first call on each device looks up the array's device
 * address (hipGetSymbolAddress); make that first call outside graph capture.
 * Otherwise as pd_decode_ex: same arguments minus numerator and stats, same
 * results bit for bit.
 */
#define PD_SCRATCH_BYTES (32u << 20)
int pd_decode_scratch(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype,
                      float k_scale, float v_scale,
                      const int32_t* table, const int32_t* lengths, float* out,
                      int batch, int query_heads, int kv_heads, int head_dim, int page_size,
                      int table_width, int physical_pages, int splits, int split_tokens,
                      int merge_mode, int hints, const int32_t* length_bounds, void* stream);

/*
 * Paged KV-cache append, the write step before decode. Writes `tokens` new
 * tokens per sequence: k_new, v_new are [batch, tokens, kv_heads, head_dim]
 * (same dtype as the cache), and token j of sequence b goes to logical
 * position positions[b] + j, i.e. page table[b, pos / page_size], slot
 * pos % page_size of k_cache / v_cache [physical_pages, page_size, kv_heads,
 * head_dim] -- the decode's own addressing (reference docs/DESIGN.md:10-13).
 * Tokens whose position is negative or at/after table_width * page_size, or
 * whose page id is outside [0, physical_pages), are skipped. Pages shared by
 * several sequences are written as mapped: copy-on-write is the caller's.
 * No counterpart in the reference, which leaves cache writes to its caller
 * (docs/DESIGN.md:11-13).
 */
int pd_append_kv(const void* k_new, const void* v_new, int dtype,
                 const int32_t* table, const int32_t* positions,
                 void* k_cache, void* v_cache,
                 int batch, int tokens, int kv_heads, int head_dim, int page_size,
                 int table_width, int physical_pages, void* stream);

/*
 * As pd_append_kv with positions[b] = lengths[b], all or nothing per
 * sequence, and lengths advanced on the device: sequence b is written only if
 * all of its `tokens` positions map to valid cache rows below max_context,
 * and then lengths[b] grows by `tokens`; otherwise its cache rows and length
 * are left unchanged. max_context (0 .. 1048576) is the context the caller's
 * decode partitions cover (splits * split_tokens or less), so appended
 * lengths never outgrow what pd_decode reads. An append followed by pd_decode
 * on the same lengths needs no host round trip, so a decode step can be
 * captured in a hipGraph and replayed.
 */
int pd_append_kv_advance(const void* k_new, const void* v_new, int dtype,
                         const int32_t* table, int32_t* lengths,
                         void* k_cache, void* v_cache,
                         int batch, int tokens, int kv_heads, int head_dim, int page_size,
                         int table_width, int physical_pages, int max_context, void* stream);

/*
 * Page table and lengths from CSR page-list metadata held on the device, the
 * inverse of the CSR form reference src/paged_decode/competitors.py:8-18
 * builds: for sequence b, n_b = indptr[b + 1] - indptr[b] page ids are taken
 * from indices[indptr[b]] on, table[b, n_b .. table_width) = -1, and
 * lengths[b] = (n_b - 1) * page_size + last_page_len[b], or 0 for an empty
 * list. indices holds indices_count entries. table is [batch, table_width],
 * lengths [batch], as pd_decode reads them. A sequence that does not fit
 * (n_b < 0, n_b > table_width, a page list reaching outside
 * [0, indices_count), last_page_len outside [1, page_size], or a length
 * above max_context -- the context the caller's splits cover) is
 * written as empty and sets *overflow to 1 if overflow is not NULL (it is
 * never cleared: zero it before the call with a kernel, not a memset, if the
 * call is captured). Page ids are not checked; the decode skips ids outside
 * [0, physical_pages). Lets a caller keeping CSR metadata on the device
 * refresh a plan without a host round trip, inside a captured graph.
 */
int pd_table_from_csr(const int32_t* indptr, const int32_t* indices, int64_t indices_count,
                      const int32_t* last_page_len, int32_t* table, int32_t* lengths, int32_t* overflow,
                      int batch, int table_width, int page_size, int max_context, void* stream);

/*
 * Bytes of numerator + stats for a plan: batch * query_heads * 4 * splits *
 * (head_dim + 2) * 4, the reference's DecodePlan.workspace_bytes
 * (src/paged_decode/runtime.py:71-73, docs/DESIGN.md:69-76). Returns 0 for
 * non-positive arguments.
 */
size_t pd_workspace_bytes(int batch, int query_heads, int head_dim, int splits);

/*
 * Kernel launches pd_decode / pd_decode_ex / pd_decode_scratch make for a call
 * of these formats and shapes (any lengths, bounds and stream): 1 for a
 * whole-row launch, 2 for the partition and merge launches. Returns a status
 * (the shape and format checks of pd_decode_ex) and writes *launches on
 * success. No counterpart in the reference, whose decode always launches
 * twice (decode.cu:170-194); for callers that profile or account per kernel.
 */
int pd_decode_launch_count(int q_dtype, int kv_dtype, int batch, int query_heads, int kv_heads, int head_dim,
                           int page_size, int table_width, int physical_pages, int splits, int split_tokens,
                           int hints, int* launches);

/*
 * Partitions the two launches of pd_decode / pd_decode_ex / pd_decode_scratch
 * run over for a call of these formats, shapes and host length bounds on a
 * device of compute_units CUs (<= 0: the current device's):
 * *kernel_splits partitions of *kernel_split_tokens tokens per row, with
 * kernel_split_tokens = c * split_tokens for a power of two c and
 * kernel_splits = ceil(splits / c). c > 1 only with length bounds (the live
 * partitions they reach set the waves per CU), never for whole-row calls or
 * FP32 inputs. A caller that runs the stages itself (pd_decode_partial_ex, then
 * pd_decode_merge) passes these two values to both to match the full call's
 * partitioning. These are the partitions of a call without prefix runs: with
 * runs, pd_decode_prefix may run over c / 2 where its shared-prefix items pay
 * only there (pd_decode_launch_plan reports the split it takes). Returns a
 * status (the checks of pd_decode_ex). No
 * counterpart in the reference, whose partition count is the caller's
 * (decode.cu:170-194).
 */
int pd_decode_kernel_split(int q_dtype, int kv_dtype, int batch, int query_heads, int kv_heads, int head_dim,
                           int page_size, int table_width, int physical_pages, int splits, int split_tokens,
                           const int32_t* length_bounds, int compute_units, int* kernel_splits,
                           int* kernel_split_tokens);

/*
 * The launches a full decode call (pd_decode_ex / pd_decode_scratch) of these
 * formats, shapes, merge mode, hints and host length bounds makes on a device
 * of compute_units CUs (<= 0: the current device's). No counterpart in the
 * reference, whose launch shape is fixed (decode.cu:170-194); for callers and
 * benchmarks that record which plan a measurement ran.
 */
typedef struct pd_launch_plan {
    int launches;                 /* 1: one whole-row launch, 2: partition + merge */
    int kernel_splits;            /* partitions per row the launches run over ... */
    int kernel_split_tokens;      /* ... of this many tokens (pd_decode_kernel_split) */
    unsigned grid_x, grid_y, grid_z;  /* partition launch grid */
    int waves_per_workgroup;
    int kv_heads_per_workgroup;
    int quarters_per_workgroup;
    int head_tile;                /* query heads per wave's tile */
    int grid_kind;                /* 0 rectangular, 1 rectangular + tail items, 2 work list, 3 whole rows */
    int xcd_grouped;              /* 1: each row group's partition workgroups on one XCD */
    int combined;                 /* 1: a workgroup's quarters stored as one state */
    int stream_mode;              /* non-temporal K/V loads: 0 none, 1 V (FP8: K), 2 K and V */
    int merge_kernel;             /* -1 none (whole rows), 0 one wave per row, 1 column chunks */
    int merge_loads;              /* numerator loads per lane per round */
    int merge_chunk_floats;       /* column chunk width (head_dim for one wave per row) */
    int merge_xcd_grouped;        /* 1: each row merged on the XCD that wrote its states */
    int merge_state_stride;       /* states per read state (combined quarters) */
    int shared_prefix_items;      /* work-list items that score one partition for several sequences */
} pd_launch_plan;

/* prefix_runs: as pd_decode_prefix (NULL: the plan of pd_decode_ex). */
int pd_decode_launch_plan(int q_dtype, int kv_dtype, int batch, int query_heads, int kv_heads, int head_dim,
                          int page_size, int table_width, int physical_pages, int splits, int split_tokens,
                          int merge_mode, int hints, const int32_t* length_bounds, const int32_t* prefix_runs,
                          int compute_units, pd_launch_plan* plan);

/*
 * Streaming read: reads a_bytes of a and b_bytes of b once each (16-byte
 * non-temporal loads, the fastest read form measured here) in one launch and writes at most
 * 8 bytes to sink, a device buffer of at least 2 uint32. Both sizes and
 * pointers must be multiples of 16 (else PD_ERR_SHAPE). No counterpart in
 * the reference: the bandwidth ceiling a decode launch over the same number
 * of K/V bytes is measured against (the reference profiled its partial
 * stage's DRAM throughput, results/2026-10-31-final-t4/profiling/ncu-details.csv:6,22).
 */
int pd_stream_read(const void* a, size_t a_bytes, const void* b, size_t b_bytes, uint32_t* sink, void* stream);

/* Static description of a status code (never NULL). */
const char* pd_status_string(int status);

/* ABI version of this header: bumped on any signature or layout change
 * (3: four states per partition; 4: single-launch entry withdrawn;
 * 5: states past a sequence's end are neither written nor read, so
 * pd_decode_merge takes the lengths; 6: KV-cache append; 7: BF16 and FP8 K/V,
 * pd_decode_ex; 8: pd_table_from_csr; 9: quarters of one workgroup stored
 * combined, the others as empty states; 10: hints argument of the _ex
 * entries; 11: PD_HINT_RAGGED_LENGTHS; 12: max_context argument of
 * pd_append_kv_advance, length_bounds argument of the _ex entries; 13: whole-row launches of small rows,
 * pd_decode_launch_count; 14: coarser partitions for full calls on large
 * grids, pd_decode_kernel_split; 15: pd_stream_read, indices_count argument
 * of pd_table_from_csr, pd_decode_launch_plan; 16: shared-prefix items,
 * pd_prefix_runs, pd_decode_prefix, pd_decode_partial_prefix, the
 * prefix_runs argument of pd_decode_launch_plan). PD_ABI_VERSION is the
 * value this header describes; a binding compares it with what the loaded
 * library returns. */
#define PD_ABI_VERSION 16
int pd_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PAGED_DECODE_H */
