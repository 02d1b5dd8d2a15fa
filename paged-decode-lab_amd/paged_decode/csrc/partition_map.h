// Work and address map of the partition kernels, shared by the device code in
// decode.hip and the host: which (sequence, partition, quarter, KV head, head
// tile) a wave owns, which page-id window and token rows it reads, at which
// byte offsets, and how a launch is shaped. Everything here is plain integer
// arithmetic, so the same functions compile for gfx950 (hipcc) and for the
// host C++ compiler; tests/address_audit.cpp enumerates every workgroup, wave,
// lane and tile of a launch through them and checks each access against the
// buffers the caller passes.
//
// Partitioning follows reference src/paged_decode/csrc/decode.cu:26-83 (split
// of each sequence into split_tokens partitions of four states each, end clamp
// min(len, W * T) at :42-44, page-id guard at :56-58); the decomposition into
// quarters, tiles, workgroups and the compacted work list are this build's.
#ifndef PAGED_DECODE_PARTITION_MAP_H
#define PAGED_DECODE_PARTITION_MAP_H

#include <stdint.h>

#if defined(__HIPCC__)
#define PD_HD __host__ __device__ __forceinline__
#else
#define PD_HD inline
#endif

namespace pd {

constexpr int kWave = 64;
constexpr int kQuarters = 4;     // states per partition (quarters of the partition)
constexpr int kTileTokens = 16;  // tokens per matrix-core tile

// Compacted work lists are passed in the kernel arguments for batches of up
// to kCompactMaxBatch sequences. A tail item covers tail_span (at least
// kTailSpan) of the partitions a sequence may reach only after device-side
// appends, as one partition of tail_span times the tokens.
constexpr int kCompactMaxBatch = 64;
constexpr int kTailSpan = 8;      // partitions per tail item, at least
constexpr int kMaxTailItems = 4;  // tail items per sequence, at most (wider spans above that)
constexpr int kMaxGroupItems = 128;  // shared-prefix items of a work list, at most (plan_prefix_items)

PD_HD int imin(int a, int b) { return a < b ? a : b; }
PD_HD int imax(int a, int b) { return a > b ? a : b; }
PD_HD int64_t lmin(int64_t a, int64_t b) { return a < b ? a : b; }

struct PartialParams {
    const void* q;
    const void* k;
    const void* v;
    const int32_t* table;
    const int32_t* lengths;
    float* numerator;   // [B, Hq, 4 * splits, D]
    float* stats;       // [B, Hq, 4 * splits, 2]
    float* out;         // [B, Hq, D]: written by a whole-row launch (row_mode), which stores no states
    uint32_t grid_x, grid_y;  // the launch's grid (kernel arguments: no dependent load of the dispatch packet)
    int batch;
    int query_heads;
    int group;          // query heads per KV head
    int head_tiles;     // ceil(group / GT)
    int heads_per_wg;   // KV heads per workgroup (hw)
    int tiles_per_wg;   // head tiles per workgroup (tw)
    int quarters_per_wg;  // partition quarters per workgroup (qw)
    int row_waves;        // waves of a whole-row workgroup (row_mode)
    int page_shift;     // log2(page_size)
    int table_width;
    int physical_pages;
    int splits;
    int split_tokens;
    // Tokens of a sequence the call may read: min(caller's splits *
    // split_tokens, table capacity). Lengths are clamped to it, so a full call
    // over coarser partitions (full_call_split) reads exactly the tokens the
    // caller's partitions cover, as the reference's grid of `splits`
    // partitions does (decode.cu:42-44, grid z = splits at :176).
    int reach;
    uint32_t token_bytes;  // bytes between consecutive tokens of a page (kv_heads * D * elem)
    uint64_t page_bytes;   // page_size * token_bytes
    float scale_log2;      // log2(e) * k_scale / sqrt(D)
    float v_scale;         // multiplies every stored numerator
    // XCD-grouped rectangular grid (xcd_shift >= 0, see block_coords): all
    // workgroups of a row group (one sequence's head group, every partition)
    // run on one XCD, so the merge can read those states from that XCD's L2.
    // xcd_shift is log2 of the head groups per sequence; -1: the plain grid.
    // The first xcd_main_rows grid rows hold the main items; tail items (a
    // grid with tails) follow in rows of their own, 2^xcd_tail_shift token
    // groups per row group.
    int xcd_shift;
    uint32_t xcd_main_rows;
    int xcd_tail_shift;
    // Rectangular grid (compact == 0): sequence b's partitions 0 ..
    // main_splits - 1 are items of z-slice b; when main_splits < splits (host
    // bounds reach fewer partitions than reserved), z-slices batch, batch + 1,
    // ... hold the tail items, (1 << tail_shift) per sequence in sequence
    // order, tail item j covering tail_span partitions from main_splits + j *
    // tail_span -- no lookup, so the main items' prologue is that of a plain
    // rectangular grid. Items past the last tail are empty.
    int main_splits;
    int tail_shift;
    int tail_span;
    // Compacted work list (compact != 0): the grid's items are first the
    // shared-prefix items (below), then the main items of every sequence, in
    // sequence order -- sequence b has main_first[b + 1] - main_first[b] of
    // them, partitions main_skip[b], main_skip[b] + 1, ... one each -- and
    // then the tail items, again in sequence order: sequence b's
    // tail_first[b + 1] - tail_first[b] tail items, tail item j covering the
    // tail_span partitions after its main ones from j * tail_span on (fewer
    // at the end), which a sequence reaches only if it grew on the device
    // past the host's bound. Main items come first so that the live
    // workgroups are dispatched, and placed on the CUs, as they would be
    // with no tail at all. Otherwise the grid is rectangular: every partition
    // of every sequence is one item.
    int compact;
    int items;             // grid items (compact), else batch * splits
    int32_t main_first[kCompactMaxBatch + 1];
    int32_t tail_first[kCompactMaxBatch + 1];
    // Shared-prefix items (plan_prefix_items; work lists of the matrix-core
    // kernel): the list's first group_items items each cover one partition of
    // several sequences whose page-table rows name the same pages there, so
    // the partition's K and V are read once for all of them. Item i covers
    // partition group_item[i] >> 16 of the sequences prefix_order[s], ...,
    // prefix_order[s + n - 1], with s = (group_item[i] >> 8) & 0xFF and n =
    // group_item[i] & 0xFF (2 <= n <= 16 / GT): member m takes the tile's
    // columns [m GT, (m + 1) GT). It reads the page ids of row group_row[i],
    // the members' leader, whose row each member's run is measured against.
    // Sequence b's main items then start at partition main_skip[b], not 0.
    int group_items;
    uint32_t group_item[kMaxGroupItems];
    int8_t group_row[kMaxGroupItems];
    int8_t prefix_order[kCompactMaxBatch];
    int16_t main_skip[kCompactMaxBatch];
    // Host only (launch choices, not read by the kernels).
    const int32_t* host_bounds;       // the caller's host length bounds, or null
    const int32_t* host_prefix_runs;  // the caller's shared-prefix runs [2 * batch] (pd_prefix_runs), or null
    int combine;           // the launch stores a workgroup's qw quarters as one state (kFold 1)
    int row_allowed;       // the caller takes the output from the partition launch when row_mode is chosen
    int row_mode;          // whole-row workgroups fold every state of a row into out (kFold 2): no merge launch
    int unshared_pages;    // PD_HINT_UNSHARED_PAGES
    int mid_grid;          // 2-head x 2-quarter workgroups of a mid-size grid
    int ragged_lengths;    // PD_HINT_RAGGED_LENGTHS
    int stream_mode;       // non-temporal loads: 0 none, 1 V (FP8: K), 2 K and V
    int shape_splits;      // partitions per sequence the bounds reach: the workgroup shape's grid (plan_items)
    int live_items;        // items holding tokens as far as the bounds tell (plan_items)
    int head_tile;         // GT: query heads per wave's tile (the GQA group padded to 1/2/4/8/16)
    int uniform_live;      // host bounds given, and every sequence reaches the same partitions (plan_items)
    int merge_xcd_rows;    // rows per row group for an XCD-grouped merge (merge_xcd_row), 0: plain (plan_xcd)
    int merge_xcd_shift;   // log2 of the head groups per sequence, for that merge
};

// ---------------------------------------------------------------------------
// Device-side map (also evaluated on the host by the address audit).

// Kinds of grid, fixed at compile time per kernel (kList): a kernel built for
// plain rectangular grids carries neither the tail arithmetic nor the
// work-list lookup. The lookup's control flow kept the compiler from loading
// the kernel arguments in one batch before the first page-id load (measured
// on MI355X: 0.5 us per launch), and the tail arithmetic took the 8-wave
// kernel from 128 to 131 VGPRs, one wave per SIMD fewer (ragged + shared B16
// partition kernel 36 -> 48 us).
enum GridKind { kGridRect = 0, kGridRectTails = 1, kGridList = 2 };

// Workgroup coordinates (token group, head group) in dispatch order.
//
// Plain grid (xcd_shift < 0): the linear dispatch index x + gx * y is read
// with the head group varying fastest, so consecutively dispatched (and
// co-resident) workgroups cover all KV-head groups of the same tokens -- whole
// token rows -- rather than one head group's slice of many rows.
//
// XCD-grouped grid (xcd_shift >= 0; grid 8 * main token groups x row groups
// / 8, z = 1, plus rows for the tail items of a grid with tails): the
// dispatcher deals workgroups to the eight XCDs round robin by linear index,
// so x % 8 is the workgroup's XCD. In the first xcd_main_rows rows, row group
// r = 8 * y + x % 8 (sequence r >> xcd_shift, head group r % 2^xcd_shift)
// takes main token group x / 8 on XCD r % 8. The tail rows after them hold,
// per XCD, the row groups' tail token groups in row-group order (2^
// xcd_tail_shift per row group; slots past the last row group are empty
// items), so tail items are dispatched after every main item, as on the plain
// grid, and on their row group's XCD. Each XCD holds its own L2, which keeps
// the states the row group's workgroups stored after the launch ends; the
// merge reads a row's states on that same XCD (merge_cols_kernel,
// merge_rows_kernel). Measured on MI355X: a kernel reading 2-17 MB that the
// previous kernel wrote takes 6.1-6.4 us when each workgroup reads its own
// XCD's writes and 7.5-8.2 us when it reads another XCD's.
struct BlockCoords {
    int tokens;  // item * (4 / qw) + quarter group
    int heads;   // KV heads [hg * hw, hg * hw + hw), head tiles [tg * tw, tg * tw + tw)
    int z;       // sequence of a rectangular grid
};

template <int kList>
PD_HD BlockCoords block_coords(uint32_t bx, uint32_t by, uint32_t bz, uint32_t gx, uint32_t gy, int xcd_shift,
                               uint32_t xcd_main_rows, int xcd_tail_shift) {
    if (xcd_shift >= 0) {
        const uint32_t x = bx & 7u;
        uint32_t r = by * 8u + x, tokens = bx >> 3;
        if (kList == kGridRectTails && by >= xcd_main_rows) {
            const uint32_t main_tokens = gx >> 3;
            const uint32_t slot = (by - xcd_main_rows) * main_tokens + tokens;
            r = (slot >> xcd_tail_shift) * 8u + x;
            tokens = main_tokens + (slot & ((1u << xcd_tail_shift) - 1u));
        }
        return BlockCoords{static_cast<int>(tokens), static_cast<int>(r & ((1u << xcd_shift) - 1u)),
                           static_cast<int>(r >> xcd_shift)};
    }
    // Every path reads gx and gy, so the kernel loads them with its other
    // arguments instead of after a branch.
    const uint64_t lin = bx + static_cast<uint64_t>(gx) * by;
    if (lin <= 0xFFFFFFFFull) {
        const uint32_t l32 = static_cast<uint32_t>(lin);
        return BlockCoords{static_cast<int>(l32 / gy), static_cast<int>(l32 % gy), static_cast<int>(bz)};
    }
    return BlockCoords{static_cast<int>(lin / gy), static_cast<int>(lin % gy), static_cast<int>(bz)};
}

// The partitions one workgroup handles: count consecutive partitions from
// first, of sequence b, quarter group qgroup. A main item (or a rectangular
// grid's) is one partition; a tail item is the span of partitions past the
// host's bound, streamed as one partition whose states go to the first
// partition's slots (the span's other live partitions get the empty state).
struct PartitionRange {
    int b, first, count, qgroup;
    // A shared-prefix item's sequences: prefix_order[member0 .. member0 +
    // members), b the first of them, row the leader whose page ids it reads.
    // For every other item members = 1 and row = b.
    int member0, members, row;
};

inline int grid_kind(const PartialParams& prm) {
    return prm.compact ? kGridList : prm.main_splits < prm.splits ? kGridRectTails : kGridRect;
}

template <int kList>
PD_HD PartitionRange partition_range(const PartialParams& p, const BlockCoords& bc) {
    const int groups = kQuarters / p.quarters_per_wg;
    const int item = bc.tokens / groups;
    PartitionRange r;
    r.qgroup = bc.tokens - item * groups;
    r.member0 = 0;
    r.members = 1;
    if (kList == kGridRect) {
        r.b = bc.z;
        r.row = r.b;
        r.first = item;
        r.count = 1;
        return r;
    }
    if (kList == kGridRectTails && p.xcd_shift >= 0) {
        // XCD-grouped grid: tail item j of a row group covers tail_span
        // partitions from main_splits + j * tail_span (none past the last
        // partition, nor in the slots past the last row group).
        const int j = item - p.main_splits;  // negative for main items
        const int tfirst = p.main_splits + j * p.tail_span;
        const bool tail = j >= 0;
        const bool none = (tail && tfirst >= p.splits) || bc.z >= p.batch;
        r.b = imin(bc.z, p.batch - 1);
        r.row = r.b;
        r.first = tail ? imin(tfirst, p.splits - 1) : item;
        r.count = none ? 0 : tail ? imin(p.tail_span, p.splits - tfirst) : 1;
        return r;
    }
    if (kList == kGridRectTails) {
        // Branch-free: a main item's values come out of the same arithmetic.
        const int zt = bc.z - p.batch;  // tail slice, negative for main items
        const int lin = zt * p.main_splits + item;
        const int tb = lin >> p.tail_shift;
        const int tfirst = p.main_splits + (lin & ((1 << p.tail_shift) - 1)) * p.tail_span;
        const bool tail = zt >= 0;
        const bool none = tail && (tb >= p.batch || tfirst >= p.splits);
        r.b = tail ? imin(tb, p.batch - 1) : bc.z;
        r.row = r.b;
        r.first = tail ? imin(tfirst, p.splits - 1) : item;
        r.count = none ? 0 : tail ? imin(p.tail_span, p.splits - tfirst) : 1;
        return r;
    }
    if (item < p.group_items) {
        const uint32_t word = p.group_item[item];
        r.first = static_cast<int>(word >> 16);
        r.member0 = static_cast<int>((word >> 8) & 0xFFu);
        r.members = static_cast<int>(word & 0xFFu);
        r.b = p.prefix_order[r.member0];
        r.row = p.group_row[item];
        r.count = 1;
        return r;
    }
    const int listed = item - p.group_items;
    const int mains = p.main_first[p.batch];
    const bool tail = listed >= mains;
    const int index = tail ? listed - mains : listed;
    // Sequence of the item: the last b with first[b] <= index (a sequence
    // without items of this kind repeats its predecessor's entry), i.e. the
    // number of sequences b < batch with first[b] <= index, minus one (first
    // is non-decreasing and first[0] = 0). On the device lane l loads both
    // arrays' entry l at once (batch <= kCompactMaxBatch = one wave) and a
    // ballot counts: one round of loads, where a search would chain several.
    int b, first_b, next_main, main_b, skip_b;
#if defined(__HIP_DEVICE_COMPILE__)
    static_assert(kCompactMaxBatch <= kWave, "one lane per sequence");
    const int lane = __lane_id();
    const bool in_batch = lane < p.batch;
    const int mf = in_batch ? p.main_first[lane] : 0x7FFFFFFF;
    const int tf = in_batch ? p.tail_first[lane] : 0x7FFFFFFF;
    const int sk = in_batch ? p.main_skip[lane] : 0;
    const int f = tail ? tf : mf;
    b = static_cast<int>(__popcll(__ballot(f <= index))) - 1;
    first_b = __builtin_amdgcn_readlane(f, b);
    main_b = __builtin_amdgcn_readlane(mf, b);
    skip_b = __builtin_amdgcn_readlane(sk, b);
    next_main = b + 1 < p.batch ? __builtin_amdgcn_readlane(mf, b + 1) : mains;
#else
    const int32_t* first = tail ? p.tail_first : p.main_first;
    int count = 0;
    for (int s = 0; s < p.batch; ++s) count += first[s] <= index;
    b = count - 1;
    first_b = first[b];
    main_b = p.main_first[b];
    skip_b = p.main_skip[b];
    next_main = p.main_first[b + 1];
#endif
    r.b = b;
    r.row = b;
    // Sequence b's main items are its partitions skip_b, skip_b + 1, ...
    // (those before skip_b are in shared-prefix items), then its tail items.
    if (!tail) {
        r.first = skip_b + index - first_b;
        r.count = 1;
    } else {
        r.first = skip_b + next_main - main_b + (index - first_b) * p.tail_span;
        r.count = imin(p.tail_span, p.splits - r.first);
    }
    return r;
}

// The page check of a shared-prefix item's wave. The runs that formed the
// item are the caller's description of the table; the kernel does not rely
// on them. Before its loop, a wave compares each member's table entries with
// the leader row's over the pages its tokens [wb, we) touch: pair i of the
// check is member prefix_pair_member(i) on logical page prefix_pair_page(i),
// checked when the member has tokens there (page * page_size < the member's
// end). Members with a differing entry are left out of the shared pass and
// read their own rows in a pass of their own, so results do not depend on
// the runs being right (a plan refreshed after a graph was captured, or runs
// that claim too much, only cost passes).
PD_HD int prefix_span_pages(const PartialParams& p, int wb, int we) {
    return wb < we ? ((we - 1) >> p.page_shift) - (wb >> p.page_shift) + 1 : 0;
}
PD_HD int prefix_pair_member(int pair, int span_pages) { return pair / span_pages; }
PD_HD int prefix_pair_page(const PartialParams& p, int wb, int pair, int span_pages) {
    return (wb >> p.page_shift) + pair % span_pages;
}

// Which KV head, head tile and token range a wave owns in the `count`
// partitions from `split` of sequence b (raw device length len_raw), from its
// workgroup's coordinates; the wave index splits into (head, tile, quarter).
// The range's tokens are cut into four quarters of whole load groups.
struct WaveWork {
    int split, quarter, kv_head, tile, wb, we;
    int64_t q_row;   // first query-head row of the tile
    int heads_here;  // live query heads in the tile
    bool dead;       // the partition starts at or past the sequence end: no state is written
};

template <int GT, int ALIGN>
PD_HD WaveWork wave_work(const PartialParams& p, int b, int split, int count, int qgroup, int heads, int wave,
                         int len_raw) {
    WaveWork w;
    const int qw = p.quarters_per_wg;
    const int qq = wave % qw;
    const int tt = (wave / qw) % p.tiles_per_wg;
    const int hh = wave / (qw * p.tiles_per_wg);
    const int tile_groups = p.head_tiles / p.tiles_per_wg;
    w.split = split;
    w.quarter = qgroup * qw + qq;
    w.kv_head = (heads / tile_groups) * p.heads_per_wg + hh;
    w.tile = (heads % tile_groups) * p.tiles_per_wg + tt;
    const int len = imax(0, imin(len_raw, p.reach));  // decode.cu:42-44
    const int64_t first = static_cast<int64_t>(split) * p.split_tokens;
    w.dead = first >= len || count <= 0;  // count 0: an empty item of the grid
    const int tb = static_cast<int>(lmin(first, len));
    const int te = static_cast<int>(lmin(first + static_cast<int64_t>(count) * p.split_tokens, len));
    int per = (te - tb + kQuarters - 1) / kQuarters;
    per = (per + ALIGN - 1) / ALIGN * ALIGN;
    w.wb = imin(tb + w.quarter * per, te);
    w.we = imin(w.wb + per, te);
    const int member0 = w.tile * GT;
    w.heads_here = imax(0, imin(GT, p.group - member0));
    w.q_row = static_cast<int64_t>(b) * p.query_heads + static_cast<int64_t>(w.kv_head) * p.group + member0;
    return w;
}

// The first logical page a wave reads if its partitions are full length: lets
// the page-id window be requested before the sequence length arrives.
template <int ALIGN>
PD_HD int speculative_page(const PartialParams& p, int split, int count, int qgroup, int wave) {
    const int qw = p.quarters_per_wg;
    const int quarter = qgroup * qw + wave % qw;
    const int per_full = ((count * p.split_tokens + kQuarters - 1) / kQuarters + ALIGN - 1) / ALIGN * ALIGN;
    const int capacity = p.table_width << p.page_shift;
    const int64_t start = static_cast<int64_t>(split) * p.split_tokens + static_cast<int64_t>(quarter) * per_full;
    return static_cast<int>(lmin(start, capacity - 1)) >> p.page_shift;
}

// Whole-row launch (row_mode): one workgroup per (sequence, KV head, head
// tile) -- heads = kv_head * head_tiles + tile -- whose `waves` waves cut the
// row's tokens [0, min(len, splits * split_tokens)) into slices of whole load
// groups, wave w taking slice w. Its states stay in LDS, so the slices need
// not follow the partitions. A wave with an empty slice (dead) still joins
// the workgroup's fold, with the empty state.
template <int GT, int ALIGN>
PD_HD WaveWork row_wave_work(const PartialParams& p, int b, int heads, int wave, int waves, int len_raw) {
    WaveWork w;
    w.split = 0;
    w.quarter = wave;
    w.kv_head = heads / p.head_tiles;
    w.tile = heads % p.head_tiles;
    const int te = imax(0, imin(len_raw, p.reach));  // decode.cu:42-44
    int per = (te + waves - 1) / waves;
    per = (per + ALIGN - 1) / ALIGN * ALIGN;
    w.wb = imin(wave * per, te);
    w.we = imin(w.wb + per, te);
    w.dead = w.wb >= w.we;
    const int member0 = w.tile * GT;
    w.heads_here = imax(0, imin(GT, p.group - member0));
    w.q_row = static_cast<int64_t>(b) * p.query_heads + static_cast<int64_t>(w.kv_head) * p.group + member0;
    return w;
}

// First logical page of a whole-row wave's slice if the row is full length.
template <int ALIGN>
PD_HD int row_speculative_page(const PartialParams& p, int wave, int waves) {
    const int capacity = p.table_width << p.page_shift;
    const int span = static_cast<int>(lmin(static_cast<int64_t>(p.splits) * p.split_tokens, capacity));
    const int per_full = ((span + waves - 1) / waves + ALIGN - 1) / ALIGN * ALIGN;
    return imin(wave * per_full, capacity - 1) >> p.page_shift;
}

// Table entry lane `lane` of a wave loads for the page-id window at `window`
// (clamped into the row, so every lane's load is in bounds).
PD_HD int window_entry(const PartialParams& p, int window, int lane) {
    return imin(window + lane, p.table_width - 1);
}

// One load group of `tokens` tokens starting at t0 (a 16-token matrix-core
// tile, or one token row group of the FP32 kernel) within the wave's current
// range [rb, re): the live token span [lo, hi] (or the last live token when
// the group lies past re) and the page-id window slot of its first token.
struct TileSpan {
    int lo, hi, slot;
};

PD_HD TileSpan tile_span(const PartialParams& p, int t0, int tokens, int rb, int re, int window) {
    TileSpan s;
    s.lo = imax(t0, rb);
    s.hi = imin(t0 + tokens, re) - 1;
    if (s.lo > s.hi) s.lo = s.hi = re - 1;
    s.slot = imin(imax((s.lo >> p.page_shift) - window, 0), kWave - 1);
    return s;
}

// Whether the group's loads go to its page (else to the park row: a group
// past re, or a page id outside [0, physical_pages), decode.cu:56-58).
PD_HD bool tile_live(const PartialParams& p, int t0, int re, int page) {
    return t0 < re && static_cast<uint32_t>(page) < static_cast<uint32_t>(p.physical_pages);
}

// Byte offset of a live group's page from the head's base: page * page_bytes.
PD_HD uint64_t tile_page_offset(const PartialParams& p, bool ok, int page) {
    return static_cast<uint64_t>(ok ? page : 0) * p.page_bytes;
}

// Byte offset within the page (or the park row) of token t, clamped into
// [lo, hi], at lane byte offset lane_bytes of the token's head slice.
PD_HD uint32_t token_offset(const PartialParams& p, bool ok, int t, const TileSpan& s, uint32_t lane_bytes) {
    const int tk = imin(imax(t, s.lo), s.hi);
    return ok ? static_cast<uint32_t>(tk & ((1 << p.page_shift) - 1)) * p.token_bytes + lane_bytes : lane_bytes;
}

// Tile token whose K the q.K^T A operand of matrix-core lane row r (r = lane
// % 16) holds: sigma(r) = r / 4 + 4 (r % 4), which leaves the scores of
// tokens g, g + 4, g + 8, g + 12 in lane group g, the P.V A layout.
PD_HD int k_token_of_row(int r) { return (r >> 2) + 4 * (r & 3); }

// Partitions after the first of a workgroup's span that hold tokens of the
// sequence: their state slots take the empty state (the span's tokens are all
// in the first partition's states). Zero for a single-partition item.
PD_HD int extra_live_partitions(const PartialParams& p, int split, int count, int len_raw) {
    const int64_t len = imax(0, imin(len_raw, p.reach));
    const int64_t live = (len + p.split_tokens - 1) / p.split_tokens;  // partitions holding tokens
    return static_cast<int>(lmin(split + count, live) - lmin(split + 1, live));
}

// Numerator and stats element offsets of state `part` of query-head row `row`.
PD_HD int64_t numerator_offset(const PartialParams& p, int64_t row, int part, int head_dim) {
    return (row * (kQuarters * static_cast<int64_t>(p.splits)) + part) * head_dim;
}
PD_HD int64_t stats_offset(const PartialParams& p, int64_t row, int part) {
    return (row * (kQuarters * static_cast<int64_t>(p.splits)) + part) * 2;
}

// ---------------------------------------------------------------------------
// Launch shape (host).

// Largest divisor of n not above cap.
inline int largest_divisor(int n, int cap) {
    for (int d = imin(n, cap); d > 1; --d)
        if (n % d == 0) return d;
    return 1;
}

// Workgroup shape: up to max_heads KV heads of the same tokens per workgroup
// (their slices of a token row are then read together), all head tiles of
// those heads, and as many partition quarters as fill `waves` waves (8, or
// fewer for small grids: see plan_mfma). A KV head count with no divisor in
// 2..max_heads keeps its whole token row in one workgroup when it fits (5 or
// 7 heads in 8 waves).
//
// The matrix-core kernel takes 4 KV heads: at 8 KV heads, two workgroups of 4
// heads x 2 quarters (quarters combined, V loads streamed when no page is
// shared) measured faster per call than one of 8 heads x 1 quarter on every
// shape tried on MI355X: Llama-3-8B B4 L4096 18.86 -> 17.31 us, the B16 L4096
// batch of the reference's benchmark 50.7 -> 40.2 us, B64 L2048 122.3 ->
// 103.8 us; with 32 KV heads, 32K-context MHA 97.2 -> 89.8 us at split 256.
// Grids that would leave most CUs idle take smaller workgroups instead, and
// grids smaller than the device skip the combine, as do mid-size grids whose
// merge is XCD-grouped (see plan_mfma).
inline void choose_workgroup(PartialParams& prm, int kv_heads, int max_heads, int waves = 8) {
    prm.heads_per_wg = largest_divisor(kv_heads, imin(max_heads, waves));
    if (prm.heads_per_wg == 1 && kv_heads <= waves) prm.heads_per_wg = kv_heads;
    prm.tiles_per_wg = largest_divisor(prm.head_tiles, waves / prm.heads_per_wg);
    const int hw_tw = prm.heads_per_wg * prm.tiles_per_wg;
    prm.quarters_per_wg = hw_tw * 4 <= waves ? 4 : hw_tw * 2 <= waves ? 2 : 1;
}

// Head tile: the GQA group padded to a power of two up to max_tile query
// heads (16 for the matrix-core kernel, whose MFMA column block holds 16
// heads; 8 for the FP32 kernel, whose accumulators grow with the tile);
// larger groups are cut into tiles of max_tile.
inline int head_tile(int group, int max_tile) {
    int gt = 1;
    while (gt < group && gt < max_tile) gt *= 2;
    return gt;
}

// Grids under host bounds. With per-sequence upper bounds on the lengths
// known to the caller at launch (length_bounds, host memory; null if
// unknown), the partitions past sequence b's bound, splits -
// ceil(bound_b / split_tokens) of them, become at most kMaxTailItems tail
// items; the partitions before it are the main items, of a rectangular grid
// or (very ragged batches of at most kCompactMaxBatch) a work list. A bound below the length
// the kernel finds on the device only moves that sequence's later partitions
// onto its tail items: results are the same to rounding, the launch slower.
//
// Why the tail items go last: a launch whose workgroups all fit on the device
// at once is placed round-robin over the XCDs and CUs in dispatch order, and
// it lasts as long as its most loaded CU. Measured on MI355X (Llama-3-8B B4
// L4096, split 256, partition kernel, cold K/V), a rectangular grid reserving
// 17 splits instead of 16 -- eight dead workgroups after each sequence's 128
// live ones -- took 17.5 us instead of 14.6: the dead workgroups shift the
// next sequence's placement so that some CUs hold three live workgroups and
// others one. (24 splits happened to land evenly again: 15.0 us.)
//
// The workgroup shape (plan_mfma) does not follow the launched grid, whose
// size depends on the reserve (tail items) and on the dead partitions a work
// list drops: shape_splits is the partitions per sequence the bounds reach
// (the rectangular grid the shape rules were measured on), live_items the
// main items. Before this, reserving twice the context of the ragged +
// shared B16 batch crossed the mid-size-grid limit and took the partition
// kernel from 33.4 to 44.7 us, and the work list of the reference's ragged
// B4 L4096 batch lost the mid-size shape (14.7 -> 16.0 us per call).
// Partitions per tail item for a sequence with `reserved` partitions past
// its bound: kTailSpan, or wider so that it has at most kMaxTailItems. Each
// dead tail workgroup costs about 1 ns of the launch; a live one (lengths
// grown past the captured bounds) streams its span in four waves.
inline int tail_span_for(int reserved) {
    return imax(kTailSpan, (reserved + kMaxTailItems - 1) / kMaxTailItems);
}

// Partitions of sequence b the host bound reaches (at most splits).
inline int bounded_partitions(const PartialParams& prm, const int32_t* length_bounds, int b) {
    const int64_t bound = lmin(prm.reach, length_bounds[b] < 0 ? 0 : length_bounds[b]);
    return static_cast<int>(lmin((bound + prm.split_tokens - 1) / prm.split_tokens, prm.splits));
}

// The work list (compact) under host bounds: sequence b's main items are the
// partitions its bound reaches, its tail items span the rest (plan_items).
inline void make_work_list(PartialParams& prm, const int32_t* length_bounds) {
    int shortest = prm.splits;
    for (int b = 0; b < prm.batch; ++b) shortest = imin(shortest, bounded_partitions(prm, length_bounds, b));
    prm.tail_span = tail_span_for(prm.splits - shortest);
    int mains = 0, tails = 0;
    for (int b = 0; b < prm.batch; ++b) {
        const int live = bounded_partitions(prm, length_bounds, b);
        prm.main_first[b] = mains;
        prm.tail_first[b] = tails;
        mains += live;
        tails += (prm.splits - live + prm.tail_span - 1) / prm.tail_span;
    }
    prm.main_first[prm.batch] = mains;
    prm.tail_first[prm.batch] = tails;
    prm.compact = 1;
    prm.items = mains + tails;
    prm.main_splits = prm.splits;
    prm.tail_shift = 0;
}

inline void plan_items(PartialParams& prm, const int32_t* length_bounds) {
    prm.xcd_shift = -1;  // plain grid until plan_xcd, once the workgroup shape is known
    prm.compact = 0;
    prm.group_items = 0;
    for (int b = 0; b < kCompactMaxBatch; ++b) {
        prm.main_skip[b] = 0;
        prm.prefix_order[b] = 0;
    }
    prm.items = prm.batch * prm.splits;
    prm.main_splits = prm.splits;
    prm.tail_shift = 0;
    prm.tail_span = kTailSpan;
    prm.shape_splits = prm.splits;
    prm.live_items = prm.items;
    prm.uniform_live = 0;
    if (length_bounds == nullptr) return;
    auto live_of = [&](int b) { return bounded_partitions(prm, length_bounds, b); };
    int64_t live_total = 0;
    int longest = 1;
    int fewest = prm.splits;
    for (int b = 0; b < prm.batch; ++b) {
        const int live = live_of(b);
        live_total += live;
        longest = imax(longest, live);
        fewest = imin(fewest, live);
    }
    prm.uniform_live = fewest == longest;
    prm.shape_splits = longest;
    prm.live_items = static_cast<int>(lmin(live_total > 0 ? live_total : 1, prm.items));
    if (prm.batch <= kCompactMaxBatch && live_total * 2 <= static_cast<int64_t>(prm.batch) * longest) {
        make_work_list(prm, length_bounds);  // very ragged
        return;
    }
    if (longest >= prm.splits) return;
    // Otherwise the rectangular grid of the partitions the bounds reach, then
    // the tail items in z-slices of their own (at most 65535 slices in all).
    const int span = tail_span_for(prm.splits - longest);
    const int tails = (prm.splits - longest + span - 1) / span;
    int shift = 0;
    while ((1 << shift) < tails) ++shift;
    const int64_t tail_items = static_cast<int64_t>(prm.batch) << shift;
    const int64_t slices = (tail_items + longest - 1) / longest;
    if (tail_items > (int64_t{1} << 30) || prm.batch + slices > 65535) return;
    prm.main_splits = longest;
    prm.tail_shift = shift;
    prm.tail_span = span;
    prm.items = static_cast<int>(static_cast<int64_t>(prm.batch) * longest + tail_items);
}

struct Grid {
    uint32_t x, y, z;
};

// Grid rows of the XCD-grouped grid: xcd_main_rows, then the tail rows.
inline uint32_t xcd_rows(const PartialParams& prm) {
    if (prm.main_splits >= prm.splits) return prm.xcd_main_rows;
    const int64_t main_tokens = static_cast<int64_t>(prm.main_splits) * (kQuarters / prm.quarters_per_wg);
    const int64_t tail_slots = static_cast<int64_t>(prm.xcd_main_rows) << prm.xcd_tail_shift;
    return prm.xcd_main_rows + static_cast<uint32_t>((tail_slots + main_tokens - 1) / main_tokens);
}

inline Grid partial_grid(const PartialParams& prm, int kv_heads) {
    const uint32_t groups = static_cast<uint32_t>(kQuarters / prm.quarters_per_wg);
    const uint32_t heads = static_cast<uint32_t>((kv_heads / prm.heads_per_wg) * (prm.head_tiles / prm.tiles_per_wg));
    if (prm.compact) return Grid{static_cast<uint32_t>(prm.items) * groups, heads, 1};
    if (prm.row_mode) return Grid{1, heads, static_cast<uint32_t>(prm.batch)};
    if (prm.xcd_shift >= 0) return Grid{8u * static_cast<uint32_t>(prm.main_splits) * groups, xcd_rows(prm), 1};
    const uint32_t tail_slices = prm.main_splits < prm.splits
        ? static_cast<uint32_t>(((static_cast<int64_t>(prm.batch) << prm.tail_shift) + prm.main_splits - 1) /
                                prm.main_splits)
        : 0u;
    return Grid{static_cast<uint32_t>(prm.main_splits) * groups, heads, static_cast<uint32_t>(prm.batch) + tail_slices};
}

inline int64_t workgroups(const Grid& g) { return static_cast<int64_t>(g.x) * g.y * g.z; }

// Workgroups of `items` partitions in the current workgroup shape.
inline int64_t item_workgroups(const PartialParams& prm, int kv_heads, int64_t items) {
    const int64_t groups = kQuarters / prm.quarters_per_wg;
    const int64_t heads = static_cast<int64_t>(kv_heads / prm.heads_per_wg) * (prm.head_tiles / prm.tiles_per_wg);
    return items * groups * heads;
}

// The rectangular grid of shape_splits partitions per sequence, the one the
// workgroup-shape rules were measured on (see plan_items).
inline int64_t shape_workgroups(const PartialParams& prm, int kv_heads) {
    return item_workgroups(prm, kv_heads, static_cast<int64_t>(prm.shape_splits) * prm.batch);
}

inline int partial_threads(const PartialParams& prm) {
    if (prm.row_mode) return kWave * prm.row_waves;
    return kWave * prm.heads_per_wg * prm.tiles_per_wg * prm.quarters_per_wg;
}

// KV heads per workgroup of the matrix-core kernel, at most (FP32 kernel: 8).
constexpr int kMfmaWorkgroupHeads = 4;

// LDS bytes of one wave's K tile in the matrix-core kernel: 16 token rows of
// head_dim elements of elem bytes, each padded by one operand read (16 bytes
// for 16-bit K, 8 for FP8).
constexpr int mfma_stage_bytes(int head_dim, int elem) { return kTileTokens * (head_dim * elem + 8 * elem); }

// LDS bytes of one quarter-combine slot: per-head max and denominator, and
// head_dim / 16 float4 accumulators per lane. A whole-row launch gives every
// wave one such slot.
constexpr int combine_slot_bytes(int head_dim) { return 2 * 16 * 4 + (head_dim / 16) * kWave * 16; }

// Waves of a whole-row workgroup, at most: the kernel is built for 1024-lane
// workgroups in that mode.
constexpr int kRowMaxWaves = 16;

// Dynamic LDS of a matrix-core launch: every wave's K tile, then the combine
// slots ([waves / qw][qw - 1]) when the launch combines quarters, or one slot
// per wave for a whole-row launch.
inline int mfma_lds_bytes(const PartialParams& prm, int head_dim, int elem) {
    const int waves = partial_threads(prm) / kWave;
    const int slots = prm.row_mode ? waves : prm.combine ? waves / prm.quarters_per_wg * (prm.quarters_per_wg - 1) : 0;
    return waves * mfma_stage_bytes(head_dim, elem) + slots * combine_slot_bytes(head_dim);
}

// Whole-row launch: a full decode call whose rows are small enough to be
// latency-bound -- at most kRowMaxBytes of K and V per (sequence, KV head) --
// runs one workgroup per (sequence, KV head, head tile), its waves on
// consecutive slices of the row, folds their states in LDS with the merge's
// max-corrected sum and writes the output rows: one launch instead of two,
// and as many waves per row as fit (up to one 16-token group each), however
// few partitions the row has. Larger rows keep the partition launch spread
// over all CUs: measured on MI355X, MQA B128 L1024 (256 KB per row) as 128
// workgroups of 16 waves took 14.5 us per call, against 13.9 us for the
// partition launch and the merge.
constexpr int64_t kRowMaxBytes = 128 * 1024;
constexpr int kRowWaveTokens = 16;

// Whether a call's rows -- min(splits * split_tokens, table capacity) tokens
// of K and V per (sequence, KV head), elem bytes per element -- are small
// enough for a whole-row launch.
inline bool rows_fit_one_launch(int64_t splits, int64_t split_tokens, int64_t capacity, int head_dim, int elem) {
    const int64_t span = lmin(splits * split_tokens, capacity);
    return span * head_dim * elem * 2 <= kRowMaxBytes;
}

// The grouping itself, as plain host arithmetic on the runs and bounds (so
// that coarse_split can count the waves it leaves): the items (partition <<
// 16 | first slot << 8 | members), their leader rows, the member order, each
// sequence's shared leading partitions (skip), and the member-partitions the
// items score (covered).
struct PrefixGrouping {
    int items;
    int64_t covered;
    uint32_t item[kMaxGroupItems];
    int8_t row[kMaxGroupItems];
    int8_t order[kCompactMaxBatch];
    int skip[kCompactMaxBatch];
};

inline void group_prefixes(PrefixGrouping& g, const int32_t* runs, const int32_t* bounds, int batch, int64_t reach,
                           int split_tokens, int splits, int page_shift, int slots) {
    g.items = 0;
    g.covered = 0;
    for (int b = 0; b < kCompactMaxBatch; ++b) {
        g.skip[b] = 0;
        g.order[b] = 0;
    }
    if (runs == nullptr || bounds == nullptr || batch > kCompactMaxBatch || slots < 2) return;
    int lead[kCompactMaxBatch];
    for (int b = 0; b < batch; ++b) {
        const int leader = runs[2 * b];
        const int64_t shared = static_cast<int64_t>(runs[2 * b + 1]) << page_shift;
        const int64_t bound = lmin(reach, bounds[b] < 0 ? 0 : bounds[b]);
        const int64_t live = lmin((bound + split_tokens - 1) / split_tokens, splits);
        const int64_t parts = bound <= shared ? live : shared / split_tokens;
        lead[b] = leader < 0 || leader >= batch ? 0 : static_cast<int>(lmin(parts, live));
    }
    bool placed[kCompactMaxBatch] = {};
    int order = 0;
    bool capped = false;
    for (int b0 = 0; b0 < batch && !capped; ++b0) {
        if (placed[b0] || lead[b0] < 1) continue;
        // The class of b0's leader, sorted by lead (descending), then sequence.
        int members[kCompactMaxBatch];
        int n = 0;
        for (int b = b0; b < batch; ++b) {
            if (placed[b] || lead[b] < 1 || runs[2 * b] != runs[2 * b0]) continue;
            placed[b] = true;
            int k = n++;
            while (k > 0 && lead[members[k - 1]] < lead[b]) {
                members[k] = members[k - 1];
                --k;
            }
            members[k] = b;
        }
        if (n < 2) continue;
        const int start = order;
        for (int k = 0; k < n; ++k) g.order[order++] = static_cast<int8_t>(members[k]);
        for (int j = 0; j < lead[members[0]] && !capped; ++j) {
            int covering = 0;
            while (covering < n && lead[members[covering]] > j) ++covering;
            for (int c = 0; c + 1 < covering && !capped; c += slots) {  // chunks of two or more
                const int size = imin(slots, covering - c);
                if (g.items == kMaxGroupItems) {
                    capped = true;
                    break;
                }
                g.row[g.items] = static_cast<int8_t>(runs[2 * b0]);
                g.item[g.items++] = (static_cast<uint32_t>(j) << 16) | (static_cast<uint32_t>(start + c) << 8) |
                                    static_cast<uint32_t>(size);
                g.covered += size;
                for (int k = c; k < c + size; ++k) g.skip[members[k]] = j + 1;
            }
        }
    }
}

// Tile slots for shared-prefix members of a matrix-core launch: 16 / GT
// when a KV head's query heads fit one tile, else 1 (no grouping).
inline int prefix_slots(int group) {
    const int gt = head_tile(group, 16);
    return gt >= group ? 16 / gt : 1;
}

// Whether a rectangular grid (lengths not ragged enough for a work list) of
// `live` items should run shared-prefix items: when grouping removes at least
// 1 / kPrefixListShare of the items and the remaining ones still give
// kCoarseWavesPerCu waves per CU (the grid then becomes a work list). Work
// lists always form the items. Measured on MI355X (decode call, us, graph of
// 200 calls; with runs / without, equal lengths and a shared prompt): B16
// L4096 50% shared over 512-token partitions 35.7 / 38.9, but over the 1024
// tokens the coarse split picks for it (5 waves per CU once grouped) 41.9,
// and B4 L4096 50% (5 waves per CU) 19.2-19.6 / 16.3. coarse_split does not
// count the items; it halves its span instead where they pay only at the
// finer one (prefix_finer_split).
constexpr int kPrefixListShare = 8;
constexpr int kCoarseWavesPerCu = 8;  // waves per CU a grid keeps (coarse_split)

inline bool rect_prefix_items_pay(int64_t live, int64_t saved, int64_t waves_per_item, int cus) {
    return saved > 0 && saved * kPrefixListShare >= live &&
           (live - saved) * waves_per_item >= static_cast<int64_t>(kCoarseWavesPerCu) * cus;
}

// The partitions of a grid over partitions of `span` tokens: the live ones
// the bounds reach, those its shared-prefix items save (members scored by
// an item, less the items), and whether the lengths are ragged enough for a
// work list (plan_items), which forms the items whether or not they pay.
struct PrefixSaving {
    int64_t live, saved;
    bool work_list;
};

inline PrefixSaving prefix_saving(const int32_t* runs, const int32_t* bounds, int batch, int64_t reach,
                                  int64_t span, int splits, int page_shift, int slots) {
    PrefixSaving s{0, 0, false};
    int64_t longest = 1;
    for (int b = 0; b < batch; ++b) {
        const int64_t bound = lmin(reach, bounds[b] < 0 ? 0 : bounds[b]);
        const int64_t live = lmin((bound + span - 1) / span, splits);
        s.live += live;
        longest = live > longest ? live : longest;
    }
    s.work_list = batch <= kCompactMaxBatch && s.live * 2 <= static_cast<int64_t>(batch) * longest;
    PrefixGrouping g;
    group_prefixes(g, runs, bounds, batch, reach, static_cast<int>(span), splits, page_shift, slots);
    s.saved = g.covered - g.items;
    return s;
}

// A rectangular grid at coarse_split's factor c whose shared-prefix items do
// not pay (rect_prefix_items_pay), while at c / 2 they save at least
// 1 / kPrefixFinerShare of the partitions and pay, runs at c / 2 with them.
// Measured on MI355X (graph of 200 calls, K/V rotated over 2 GiB, equal
// lengths, 8 KV heads, GQA 4, page 16, split 256, us; staged call over 512-
// and 1024-token partitions with runs, and the full call at 1024 before this
// rule): B16 L4096 50% shared 35.4 / 39.2, 37.7; B8 L8192 50% 36.6 / 38.8,
// 40.6; B32 L2048 50% 36.0 / 38.0, 38.1; but B16 L4096 25% shared, whose
// items save 3 / 16 of the 512-token partitions, 46.6 / 45.0, 44.7.
constexpr int kPrefixFinerShare = 4;

inline int prefix_finer_split(int c, const int32_t* runs, const int32_t* bounds, int batch, int64_t reach,
                              int splits, int split_tokens, int page_shift, int slots, int64_t waves_per_item,
                              int cus) {
    if (c < 2 || runs == nullptr || bounds == nullptr || batch > kCompactMaxBatch || slots < 2) return c;
    const int64_t span = static_cast<int64_t>(split_tokens) * c;
    const PrefixSaving at = prefix_saving(runs, bounds, batch, reach, span, (splits + c - 1) / c, page_shift, slots);
    if (at.work_list || rect_prefix_items_pay(at.live, at.saved, waves_per_item, cus)) return c;
    const int h = c / 2;
    const PrefixSaving finer =
        prefix_saving(runs, bounds, batch, reach, span / 2, (splits + h - 1) / h, page_shift, slots);
    if (finer.saved * kPrefixFinerShare >= finer.live &&
        rect_prefix_items_pay(finer.live, finer.saved, waves_per_item, cus))
        return h;
    return c;
}

// Coarser partitions for a whole decode call on a large grid. The caller's
// split_tokens sizes the workspace (four states per partition) and is what
// the separate partition and merge entries use; a whole call (partition
// launch, then merge launch, both internal) may instead run over partitions
// of c x split_tokens tokens, c a power of two, which need ceil(splits / c)
// partitions per row: fewer states, so the caller's workspace holds them.
// The attention does not depend on the partitioning; results agree to FP32
// rounding. Longer partitions mean longer waves, so the per-wave latencies
// (page ids and first K/V loads, the last tile, the state stores) and the
// merge's states weigh less per byte -- while the grid keeps enough waves to
// cover the device. c doubles while a wave would read at most
// kCoarseWaveBytes of K and V and the live partitions, as far as the host
// bounds tell, still give kCoarseWavesPerCu waves per CU. A call without
// bounds keeps its split: counting every allocated partition as live
// over-coarsens plans that reserve context (Llama-3-8B B4 L4096 with 4x
// reserved: 21.7 -> 28.4 us). Measured on MI355X (decode call, us, graph of 200 calls, K/V
// rotated over 2 GiB; the split the rule picks in brackets):
//   ragged + shared-prefix B16, page 32, split 128: 40.8 -> 31.9 [512]
//     (1024: 32.5, 2048: 37.7);
//   uniform B16 / B32 L4096, 8 KV heads, split 256: 53.6 -> 48.0 [1024] /
//     102.6 -> 90.6 [1024]; B64 L2048: 101.6 -> 91.3 [1024];
//   FP8 K/V B16 L4096: 36.6 -> 32.4 [1024]; MQA B512 L1024 D64: 36.8 ->
//     32.7 [1024];
//   the reference's B16 L4096 batch: 44.3 -> 41.1 [512] (1024: 39.3);
//   32K-context MHA at split 128: 93.3 -> 85.7 [1024];
//   grids of at most eight waves per CU keep their split: doubling it made
//     the Llama-3-8B B4 L4096 FP8 call 14.8 -> 17.9, MQA B128 L1024 14.1 ->
//     16.3, the reference's B4 batch 14.7 -> 16.2 (FP16 Llama-3-8B: 17.4 ->
//     17.3).
// Going on to four waves per CU helped some shapes and hurt others badly
// (FP16 B2 L8192 17.6 -> 17.2; FP8 K/V B16 L4096 32.5 -> 47.2, MQA B256
// L1024 20.2 -> 25.0, FP16 B6 L4096 22.6 -> 23.0), so the rule stops at eight.
// Whole-row calls and FP32 inputs keep the caller's split. With prefix runs
// (`slots` members per shared-prefix item, pages of 1 << page_shift tokens)
// prefix_finer_split may halve c.
constexpr int64_t kCoarseWaveBytes = 128 * 1024;

struct KernelSplit {
    int splits, split_tokens;
};

inline KernelSplit coarse_split(int batch, int kv_heads, int head_tiles, int head_dim, int elem, int page_size,
                                int table_width, int splits, int split_tokens, const int32_t* length_bounds,
                                int cus, const int32_t* prefix_runs = nullptr, int page_shift = 0, int slots = 1) {
    if (length_bounds == nullptr) return KernelSplit{splits, split_tokens};
    const int64_t capacity = static_cast<int64_t>(table_width) * page_size;
    // Tokens the caller's partitions reach; no partition of a coarser split goes past them.
    const int64_t reach = lmin(static_cast<int64_t>(splits) * split_tokens, capacity);
    // Whether partitions of `span` tokens leave enough waves per CU. Shared-
    // prefix items are not counted: measured with them, the ragged + shared
    // B16 workload ran 27.2 us per staged call at the 512-token partitions
    // this count picks and 32.5 us at 256 tokens, where counting the items'
    // waves against 8 per CU would have stopped.
    auto enough = [&](int64_t span) {
        int64_t parts = 0;
        for (int b = 0; b < batch; ++b) {
            const int64_t bound = lmin(reach, length_bounds[b] < 0 ? 0 : length_bounds[b]);
            parts += (bound + span - 1) / span;
        }
        return parts * kQuarters * kv_heads * head_tiles >= static_cast<int64_t>(kCoarseWavesPerCu) * cus;
    };
    int c = 1;
    while (2 * c <= splits) {
        const int64_t span = static_cast<int64_t>(split_tokens) * 2 * c;
        if (span > (int64_t{1} << 20)) break;
        if ((span + kQuarters - 1) / kQuarters * head_dim * elem * 2 > kCoarseWaveBytes) break;
        if (!enough(span)) break;
        c *= 2;
    }
    c = prefix_finer_split(c, prefix_runs, length_bounds, batch, reach, splits, split_tokens, page_shift, slots,
                           static_cast<int64_t>(kQuarters) * kv_heads * head_tiles, cus);
    return KernelSplit{(splits + c - 1) / c, split_tokens * c};
}

// The partitions of a full decode call's two launches: coarse_split's for a
// matrix-core call (16-bit q) that is not a whole-row launch, else the
// caller's. kv_elem: bytes per stored K/V element; prefix_runs: the call's
// shared-prefix runs, or nullptr.
inline KernelSplit full_call_split(bool fp32, int kv_elem, int batch, int query_heads, int kv_heads, int head_dim,
                                   int page_size, int table_width, int splits, int split_tokens,
                                   const int32_t* length_bounds, int cus, const int32_t* prefix_runs = nullptr) {
    const KernelSplit same{splits, split_tokens};
    if (fp32 || rows_fit_one_launch(splits, split_tokens, static_cast<int64_t>(table_width) * page_size, head_dim,
                                    kv_elem))
        return same;
    const int group = query_heads / kv_heads;
    const int gt = head_tile(group, 16);
    return coarse_split(batch, kv_heads, (group + gt - 1) / gt, head_dim, kv_elem, page_size, table_width, splits,
                        split_tokens, length_bounds, cus, prefix_runs, page_size == 16 ? 4 : 5, prefix_slots(group));
}

// Bytes of one whole-row LDS slot of the FP32 kernel (per-head max and
// denominator, and the head tile's accumulators, GT <= 8).
constexpr int row_slot_bytes_fp32(int head_dim) { return (2 * 8 + 8 * head_dim) * 4; }

// Waves of an FP32 whole-row workgroup, at most: 16, except for head tiles of
// 8, whose q, accumulators and load pipeline (about 160 VGPRs) would not fit
// the 128 VGPRs of a 1024-lane workgroup without spilling: 8.
constexpr int fp32_row_max_waves(int gt) { return gt >= 8 ? 8 : kRowMaxWaves; }

// Sets up a whole-row launch if the call allows it and its rows qualify;
// slot_bytes and stage_bytes are the kernel's LDS per wave.
inline void plan_rows(PartialParams& prm, int head_dim, int elem, int slot_bytes, int stage_bytes,
                      int max_waves = kRowMaxWaves) {
    prm.row_mode = 0;
    if (!prm.row_allowed) return;
    const int64_t capacity = static_cast<int64_t>(prm.table_width) << prm.page_shift;
    if (!rows_fit_one_launch(prm.splits, prm.split_tokens, capacity, head_dim, elem)) return;
    const int64_t span = lmin(static_cast<int64_t>(prm.splits) * prm.split_tokens, capacity);
    int waves = static_cast<int>(lmin(max_waves, (span + kRowWaveTokens - 1) / kRowWaveTokens));
    while (waves > 1 && waves * (slot_bytes + stage_bytes) > 160 * 1024) --waves;
    prm.row_mode = 1;
    prm.row_waves = imax(1, waves);
    prm.heads_per_wg = 1;
    prm.tiles_per_wg = 1;
    prm.quarters_per_wg = kQuarters;
    prm.combine = 0;
    prm.mid_grid = 0;
    prm.compact = 0;
    prm.items = prm.batch * prm.splits;
    prm.main_splits = prm.splits;
    prm.tail_shift = 0;
}

// ---------------------------------------------------------------------------
// Shared prefixes.
//
// Sequences that share a prefix of physical pages (one prompt, several
// continuations) would each read that prefix's K and V. The matrix-core
// tile scores 16 query-head columns per MFMA, and a GQA group fills only GT
// of them, so one wave can score a K/V tile for 16 / GT sequences at the cost
// of one: a shared-prefix item gives each member sequence GT columns (its own
// q rows, its own length mask, its own states) and reads the tile once.
//
// The caller describes the sharing with prefix runs (pd_prefix_runs): for
// each sequence b, runs[2 b] is its leader (the first sequence whose row
// starts with the same page, or -1 when its first entry is not a page) and
// runs[2 b + 1] the number of leading table entries b has in common with the
// leader's row. Two sequences of one leader then share their first
// min(run, run') entries. The device table must hold the rows the runs were
// taken from; DecodePlan keeps the two in step (its table is the host copy it
// uploads, and it drops the runs when the device rewrites the table).

// Prefix runs of a host page table [batch, width] (pd_prefix_runs). A
// sequence's leader is the first sequence whose row starts with the same page
// (found among the leaders so far: the batch is small next to the table).
inline void prefix_runs_of_table(const int32_t* table, int batch, int width, int32_t* runs) {
    for (int b = 0; b < batch; ++b) {
        const int32_t* row = table + static_cast<int64_t>(b) * width;
        int leader = -1;
        if (row[0] >= 0) {
            for (int c = 0; c < b && leader < 0; ++c)
                if (runs[2 * c] == c && table[static_cast<int64_t>(c) * width] == row[0]) leader = c;
            if (leader < 0) leader = b;
        }
        int run = 0;
        if (leader >= 0) {
            const int32_t* lrow = table + static_cast<int64_t>(leader) * width;
            while (run < width && row[run] >= 0 && row[run] == lrow[run]) ++run;
        }
        runs[2 * b] = leader;
        runs[2 * b + 1] = run;
    }
}

// Whether a runs array is well formed for the batch and table width.
inline bool prefix_runs_valid(const int32_t* runs, int batch, int width) {
    for (int b = 0; b < batch; ++b) {
        const int leader = runs[2 * b], run = runs[2 * b + 1];
        if (leader < -1 || leader >= batch || run < 0 || run > width) return false;
    }
    return true;
}

// Shared-prefix items of a work list (compact), for a matrix-core launch
// whose tile holds `slots` = 16 / GT member sequences. Sequence b's leading
// kernel partitions whose tokens below its host bound all lie inside its run
// may be shared, lead_b of them: every partition that holds tokens when the
// bound ends inside the run (a short sequence whose whole context is the
// prefix), else the partitions that end inside it. A length that grows past
// the bound onto pages of its own is caught by the kernel's page check.
// Per leader, the members with lead >= 1 are sorted
// by lead (longest first, then by sequence) into prefix_order; partition j's
// members -- those with lead_b > j, a prefix of that order -- are cut into
// chunks of `slots` in that order, and each chunk of at least two is one
// item. A sequence's shared partitions are then a prefix [0, main_skip[b]):
// its chunk only shrinks as j grows. Items past kMaxGroupItems are not
// formed; the partitions from the first one left out are main items again.
// Batches above kCompactMaxBatch, rectangular grids, whole-row launches and
// calls without host bounds or runs keep one sequence per item.
inline void plan_prefix_items(PartialParams& prm, int slots) {
    prm.group_items = 0;
    for (int b = 0; b < kCompactMaxBatch; ++b) prm.main_skip[b] = 0;
    if (!prm.compact || prm.row_mode) return;
    PrefixGrouping g;
    group_prefixes(g, prm.host_prefix_runs, prm.host_bounds, prm.batch, prm.reach, prm.split_tokens, prm.splits,
                   prm.page_shift, slots);
    if (g.items == 0) return;
    prm.group_items = g.items;
    for (int i = 0; i < g.items; ++i) {
        prm.group_item[i] = g.item[i];
        prm.group_row[i] = g.row[i];
    }
    int mains = 0;
    for (int b = 0; b < prm.batch; ++b) {
        const int live = prm.main_first[b + 1] - prm.main_first[b];
        prm.prefix_order[b] = g.order[b];
        prm.main_first[b] = mains;
        prm.main_skip[b] = static_cast<int16_t>(g.skip[b]);
        mains += live - g.skip[b];
    }
    prm.main_first[prm.batch] = mains;
    prm.items = prm.group_items + mains + prm.tail_first[prm.batch];
}

// A rectangular grid whose shared-prefix items pay (rect_prefix_items_pay)
// becomes a work list; plan_prefix_items then forms them.
inline void prefer_work_list_for_prefixes(PartialParams& prm, int kv_heads, int slots, int cus) {
    if (prm.compact || prm.host_prefix_runs == nullptr || prm.host_bounds == nullptr ||
        prm.batch > kCompactMaxBatch || slots < 2)
        return;
    PrefixGrouping g;
    group_prefixes(g, prm.host_prefix_runs, prm.host_bounds, prm.batch, prm.reach, prm.split_tokens, prm.splits,
                   prm.page_shift, slots);
    int64_t live = 0;
    for (int b = 0; b < prm.batch; ++b) live += bounded_partitions(prm, prm.host_bounds, b);
    if (rect_prefix_items_pay(live, g.covered - g.items, static_cast<int64_t>(kQuarters) * kv_heads * prm.head_tiles,
                              cus))
        make_work_list(prm, prm.host_bounds);
}

// The XCD-grouped grid (block_coords) for a rectangular launch whose row
// groups all carry the same work: host bounds that give every sequence the
// same partitions (and so the same tail items), no work list, no whole-row
// launch. With the dispatcher dealing workgroups round robin, each XCD then
// gets the same number of row groups; ragged batches keep the plain grid,
// which spreads every sequence over all XCDs. A row group must cover whole
// query heads [hg * hw * group, (hg + 1) * hw * group), so the merge can find
// it from a row index: one head-tile group per KV head. Head groups per
// sequence must be a power of two (shifts in the kernels) and sequences x
// head groups a multiple of 8.
//
// With a multiple of 8 head groups per sequence the plain grids (rectangular,
// with tail slices, or a work list) already keep each row group on one XCD:
// their linear dispatch index is (token group) * head groups + head group (+
// a multiple of 8 for later z-slices), so head group hg runs on XCD hg % 8,
// whatever the lengths. Such launches keep their grid and only the merge is
// XCD-grouped.
inline void plan_xcd(PartialParams& prm, int kv_heads) {
    prm.xcd_shift = -1;
    prm.merge_xcd_rows = 0;
    prm.merge_xcd_shift = 0;
    if (prm.row_mode || prm.head_tiles != prm.tiles_per_wg) return;
    const int groups = kv_heads / prm.heads_per_wg;
    if ((groups & (groups - 1)) != 0) return;
    const int64_t row_groups = static_cast<int64_t>(prm.batch) * groups;
    if (row_groups % 8 != 0 || row_groups / 8 > 65535) return;
    int shift = 0;
    while ((1 << shift) < groups) ++shift;
    if (groups % 8 == 0) {
        prm.merge_xcd_rows = prm.heads_per_wg * prm.group;
        prm.merge_xcd_shift = shift;
        return;
    }
    if (!prm.uniform_live || prm.compact) return;
    const int quarter_groups = kQuarters / prm.quarters_per_wg;
    if (8ll * prm.main_splits * quarter_groups > 0x7FFFFFFFll) return;
    int tail_shift = prm.tail_shift;  // tail token groups per row group: 2^tail_shift items x quarter groups
    while ((1 << (tail_shift - prm.tail_shift)) < quarter_groups) ++tail_shift;
    prm.xcd_main_rows = static_cast<uint32_t>(row_groups / 8);
    prm.xcd_tail_shift = tail_shift;
    prm.xcd_shift = shift;
    if (xcd_rows(prm) > 65535u) {
        prm.xcd_shift = -1;
        return;
    }
    prm.merge_xcd_rows = prm.heads_per_wg * prm.group;
    prm.merge_xcd_shift = shift;
}

// Query-head rows of one XCD row group for the merge (plan_xcd), or 0 for
// the plain merge grid.
inline int xcd_row_group_rows(const PartialParams& prm) { return prm.merge_xcd_rows; }

// The merge's side of the XCD-grouped grid: merge workgroup (bx, by) of a
// grid 8 * (group_rows / unit) x row groups / 8 takes `unit` consecutive rows
// of row group r = 8 * by + bx % 8, on XCD r % 8 like the partition
// workgroups that stored them; lane group `sub` of the workgroup takes row
// r * group_rows + (bx / 8) * unit + sub, of sequence r >> xcd_shift.
struct MergeRow {
    int b;
    int64_t row;  // b * query_heads + query head
};

PD_HD MergeRow merge_xcd_row(uint32_t bx, uint32_t by, int group_rows, int xcd_shift, int unit, int sub) {
    const uint32_t r = by * 8u + (bx & 7u);
    return MergeRow{static_cast<int>(r >> xcd_shift),
                    static_cast<int64_t>(r) * group_rows + static_cast<int64_t>(bx >> 3) * unit + sub};
}

// Launch shape of the matrix-core kernel on a device of `cus` compute units,
// for head_dim and K/V elements of elem bytes: head tile, workgroup shape,
// quarter combine or whole rows, and streaming mode.
inline void plan_mfma(PartialParams& prm, int kv_heads, int cus, int head_dim, int elem) {
    const int gt = head_tile(prm.group, 16);
    prm.head_tile = gt;
    prm.head_tiles = (prm.group + gt - 1) / gt;
    prefer_work_list_for_prefixes(prm, kv_heads, prefix_slots(prm.group), cus);
    choose_workgroup(prm, kv_heads, kMfmaWorkgroupHeads);
    // A grid of at most half as many 8-wave workgroups as CUs leaves most CUs
    // idle, and each busy CU can keep only so many loads in flight. The same
    // waves then go in smaller workgroups, the largest of 4, 2 or 1 waves
    // that still gives two workgroups per CU (else 1 wave). Measured on
    // MI355X, Llama-3-8B geometry (decode call, us):
    //   B1 L4096 (64 workgroups of 8 waves): 12.4 -> 10.2 with 1 wave;
    //   B1 L2048: 11.7 -> 9.9; FP8 B1 L4096: 12.6 -> 10.6-11.1;
    //   B2 L4096 and B1 L8192 (128 workgroups): 13.2 -> 12.9 and
    //   13.65 -> 13.1 with 2 waves.
    // At 192 workgroups (B3 L4096) every smaller shape was slower (14.95 ->
    // 15.3-19.0), so larger grids keep 8 waves.
    //
    // Grids of one to two 8-wave workgroups per CU with 2, 4 or 8 KV heads and
    // GQA groups of up to 8 take workgroups of 2 KV heads x 2 quarters instead
    // (4 waves; quarters combined where the merge is not XCD-grouped, see the
    // end of this function). Measured on MI355X by graph replay of 200
    // calls, N(0,1) data, K/V sets rotated past the Infinity Cache (decode
    // call, us): Llama-3-8B B4 L4096 18.0-18.4 -> 17.4-17.6, B8 L4096 29.45
    // -> 28.54, B16 L4096 with 2 KV heads (GQA 8) 20.2-20.9 -> 18.5-18.8, B8
    // L4096 with 4 KV heads 20.05 -> 19.1-19.2; ragged B4 batches within
    // 0.1-0.25. B3 L4096 (192 workgroups) was slower with smaller workgroups
    // of any kind (14.74 -> 15.05). Larger grids keep 8 waves when lengths
    // are uniform (B16 L4096 55.1 -> 56.9, B32 L4096 105.7 -> 109.1) but
    // not when they are ragged (PD_HINT_RAGGED_LENGTHS): then up to eight
    // 8-wave workgroups per CU take the smaller ones (B16 with lengths
    // uniform in [0, 4096] 37.8 -> 33.3, B32 65.1 -> 59.7; the reference's
    // B16 L4096 batch 47.6 -> 44.0 in the benchmark). At sixteen per CU (a
    // B16 page-32 L8192 batch at split 128) it was flat, so those keep 8.
    const int64_t wg8 = shape_workgroups(prm, kv_heads);
    if (wg8 * 2 <= cus) {  // small grid
        const int64_t waves_total = wg8 * (partial_threads(prm) / kWave);
        int waves = 4;
        while (waves > 1 && waves_total / waves < 2 * cus) waves /= 2;
        choose_workgroup(prm, kv_heads, kMfmaWorkgroupHeads, waves);
    } else if (wg8 >= cus &&
               item_workgroups(prm, kv_heads, prm.live_items) <= (prm.ragged_lengths ? 8 : 2) * static_cast<int64_t>(cus) &&
               (kv_heads == 2 || kv_heads == 4 || kv_heads == 8) && gt <= 8) {
        choose_workgroup(prm, kv_heads, 2, 4);
        prm.mid_grid = 1;
    }
    // The kernels for grids with tail items or a work list need 129-136 VGPRs
    // (three waves per SIMD; the plain rectangular one fits 128, four): an
    // 8-wave workgroup of theirs would hold a CU alone, so they take 4-wave
    // workgroups. Measured on MI355X, uniform B32 L4096 with twice the
    // context reserved and host bounds: 120.2 us per call in 8-wave
    // workgroups; 113.2 us as a plain rectangular grid, dead partitions
    // included. Forcing those kernels to 128 VGPRs spilled and cost more
    // elsewhere (ragged + shared B16 40.7 -> 44.9 us).
    if (grid_kind(prm) != kGridRect && partial_threads(prm) / kWave > 4) {
        if ((kv_heads == 2 || kv_heads == 4 || kv_heads == 8) && gt <= 8) {
            choose_workgroup(prm, kv_heads, 2, 4);
            prm.mid_grid = 1;
        } else {
            choose_workgroup(prm, kv_heads, kMfmaWorkgroupHeads, 4);
        }
    }
    // Combining a workgroup's quarters into one state cuts the state stores
    // (written back at the kernel's end) and the merge's reads by qw; its
    // fold runs after the slowest quarter. Measured on MI355X it pays for two
    // quarters, and for four when the head tile is full (16 query heads:
    // MQA-like groups, the largest states per KV byte); four quarters of
    // smaller tiles were 0.3-0.7 us slower per call. A grid smaller than the
    // CUs leaves the fold's tail exposed (B1 L4096: 12.05 us without, 12.43
    // with), so such launches keep four states per partition.
    //
    // Smaller tiles do fold four quarters where the quarters are long: grids
    // of more than two 8-wave workgroups per CU over partitions of at least
    // 1024 tokens (the coarser partitions of a large grid), with at most 8 KV
    // heads, 16-bit K/V and lengths not flagged ragged, run one KV head x four quarters per
    // 4-wave workgroup (`long_quarters`; the streaming mode stays that of
    // the default shape). The fold's tail is then short against a 256-token
    // quarter, and the merge reads a quarter of the states. Measured on
    // MI355X (decode call, us, two quarters -> four): uniform B16 / B32
    // L4096 48.3 -> 47.5 / 90.8 -> 88.4, B64 L2048 91.4 -> 88.4, B16 L8192
    // with 64 / 8 heads 94.7 -> 92.6; FP8 K/V B16 L4096 32.1 -> 34.0, a
    // ragged B32 L8192 batch 100.1 -> 103.0 and 32K-context MHA (32 KV heads,
    // whose default workgroups read four heads of each token row) 86.7 ->
    // 87.1, hence the conditions.
    const bool fills_device = shape_workgroups(prm, kv_heads) >= cus;
    prm.combine = fills_device && (prm.quarters_per_wg == 2 || (prm.quarters_per_wg == 4 && gt == 16));
    const bool long_quarters = fills_device && wg8 * 2 > cus && gt <= 8 && kv_heads <= 8 && elem == 2 &&
                               !prm.ragged_lengths && prm.split_tokens >= 1024;
    const int default_groups = kv_heads / prm.heads_per_wg;
    // When the KV heads need several workgroups (kv_heads > heads_per_wg),
    // each workgroup reads one head group's slice of every token row, and
    // some 16-byte loads may be issued non-temporal. That is faster when
    // nothing is read twice and slower when sequences share prefix pages,
    // which streamed loads do not leave in the caches. Measured on MI355X
    // (decode call, us):
    //   - 4 or more head groups per row (16, 32 KV heads), no shared pages: K
    //     and V streaming is fastest (32K-context MHA at split 256: 92.2; V
    //     only 95.3; neither 98.6). With 25% shared prefix pages (B8 L4096, 32
    //     KV heads): K and V 48.4, V only 43.0.
    //   - 2 head groups (8 KV heads), no shared pages: V only (B64 L2048
    //     103.8, K and V 104.7, neither 112.3; a ragged B16 page-32 batch 57.0
    //     / 62.1 / 64.1). With 25% shared prefix pages (B16 page 32): neither
    //     50.3, V only 52.0, K and V 59.3.
    //   - The 2-head x 2-quarter workgroups of mid-size grids: with 2 KV
    //     heads, one head group, streaming V anyway took B16 L4096 (GQA 8)
    //     from 19.75 to 18.81 us per call. Streaming K as well, on every
    //     mid-size grid with unshared pages, took it to 17.78, and (us per
    //     call, V only -> K and V, graph of 200 calls, best of two) B8 L4096
    //     with 4 KV heads 19.64 -> 17.98, B6 L4096 22.82 -> 22.11, B2 L4096
    //     11.99 -> 11.65, a ragged B8 L4096 batch 23.36 -> 22.36, B4 L4096
    //     with 4 KV heads / 64 query heads 13.92 -> 13.61 (Llama-3-8B B4
    //     L4096, whose 8 KV heads already count 4 head groups there, was
    //     unchanged). No shape of the coarse, small, mid or XCD sweeps got
    //     slower beyond noise.
    //   - One head group (a single KV head, or all KV heads in one
    //     workgroup) on a grid that fills the device, no shared pages:
    //     streaming K and V took (us per call) MQA B512 L1024 D64 from 32.65
    //     to 31.13, B8 L4096 with 2 KV heads (GQA 16) 14.54 -> 12.99, B16
    //     L2048 with 1 KV head 11.10 -> 10.40, MQA B128 L1024 13.84 -> 13.46;
    //     on the small MQA B4 grid it cost 8.29 -> 8.94, so small grids keep
    //     their loads cached.
    // So the mode follows the page-sharing hint: unshared pages stream K and
    // V (4+ groups, any mid-size grid, or one head group on a grid that fills
    // the device) or V (2 groups); pages that may be shared stream V (4+
    // groups) or nothing. FP8 V loads are 8-byte, so FP8 streams its 16-byte
    // K row loads wherever 16-bit K/V would stream V.
    const int groups = default_groups;
    if (prm.mid_grid && prm.unshared_pages) {
        prm.stream_mode = 2;
    } else if (groups == 1) {
        prm.stream_mode = prm.unshared_pages && fills_device ? 2 : 0;
    } else {
        prm.stream_mode = prm.unshared_pages ? (groups >= 4 ? 2 : 1) : (groups >= 4 ? 1 : 0);
    }
    if (long_quarters) {
        choose_workgroup(prm, kv_heads, 1, 4);
        prm.mid_grid = 0;
        prm.combine = prm.quarters_per_wg == 4;
    }
    plan_rows(prm, head_dim, elem, combine_slot_bytes(head_dim), mfma_stage_bytes(head_dim, elem));
    plan_prefix_items(prm, prefix_slots(prm.group));
    plan_xcd(prm, kv_heads);
    // Where the merge reads its states from the XCD's L2 (plan_xcd), the fold
    // of the mid-size grids' two quarters no longer pays for its tail: their
    // states are few per KV byte (GQA groups of up to 8). Measured on MI355X
    // (decode call, us, combined -> not): Llama-3-8B B4 L4096 16.85-16.87 ->
    // 16.64-16.66, its FP8 form 14.31-14.38 -> 13.94-13.96, FP8 B8 L2048
    // 15.28-15.30 -> 14.27-14.30, B8 L4096 27.61 -> 27.43, Llama-3-8B with
    // twice the context reserved 17.39-17.47 -> 17.26-17.32. The same for
    // every XCD-merged launch was slower where states are many per KV byte or
    // the quarters long: MQA B128 13.8 -> 15.15, uniform B32 L4096 (four
    // quarters) 88.5 -> 92.2.
    if (prm.mid_grid && prm.merge_xcd_rows > 0) prm.combine = 0;
    const Grid grid = partial_grid(prm, kv_heads);
    prm.grid_x = grid.x;
    prm.grid_y = grid.y;
}

// Launch shape of the FP32 kernel (and whole rows, as for the matrix-core
// kernel).
inline void plan_fp32(PartialParams& prm, int kv_heads, int head_dim) {
    const int gt = head_tile(prm.group, 8);
    prm.head_tile = gt;
    prm.head_tiles = (prm.group + gt - 1) / gt;
    choose_workgroup(prm, kv_heads, 8);
    plan_rows(prm, head_dim, 4, row_slot_bytes_fp32(head_dim), 0, fp32_row_max_waves(gt));
    plan_xcd(prm, kv_heads);
    const Grid grid = partial_grid(prm, kv_heads);
    prm.grid_x = grid.x;
    prm.grid_y = grid.y;
}

}  // namespace pd

#endif  // PAGED_DECODE_PARTITION_MAP_H
