// Host audit of every memory access the partition kernels form -- TEST
// INFRASTRUCTURE, the CPU stand-in for a GPU memory checker.
//
// For each problem below, the launch is planned with the library's own host
// code (partition_map.h: plan_items, plan_mfma / plan_fp32, partial_grid) and
// then every workgroup, wave, lane and load group of the grid is walked with
// the same device-side functions the kernels call (block_coords,
// partition_range, wave_work, speculative_page, window_entry, tile_span,
// tile_live, tile_page_offset, token_offset, numerator_offset, stats_offset),
// following the kernels' loop structure (page-id windows of 64 entries, load
// groups issued two ahead in blocks of two for the matrix-core kernel -- four
// and four with FP8 K/V outside whole rows -- and four ahead in blocks of sixteen for the FP32
// kernel). Every global load is
// checked to lie inside q, k, v, table or lengths (parked loads of dead
// groups inside q), every store inside numerator or stats, every LDS access
// inside the launch's dynamic LDS; every live token is read from the page its
// table entry names; and every live state slot is written exactly once, none
// past a sequence's end. Built with -fsanitize=address,undefined by
// tests/test_address_audit.py; prints one line per problem and exits nonzero
// on the first problem with a failure.
#include <cinttypes>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "cache_map.h"
#include "merge_map.h"
#include "partition_map.h"

using namespace pd;

namespace {

struct Problem {
    std::string name;
    int batch, q_heads, kv_heads, head_dim, page_size, width, pages;
    int q_elem, kv_elem;  // bytes: 4 (FP32), 2 (FP16/BF16), 1 (FP8 K/V)
    int split_tokens, splits;
    // The caller's partitions: a full call over coarser partitions keeps them
    // here (split_tokens and splits are then the coarser ones), and no token
    // at or past caller_splits * caller_split_tokens may be read.
    int caller_split_tokens, caller_splits;
    std::vector<int32_t> table, lengths, bounds;  // bounds empty: none
    std::vector<int32_t> runs;                    // shared-prefix runs [2 * batch] (pd_prefix_runs); empty: none
    bool unshared = true, ragged = false;
};

uint64_t g_checks = 0;
int g_failures = 0;
bool g_plant_reach = false;  // --plant-reach: launch params that ignore the caller's partitions (negative control)
bool g_plant_no_check = false;  // --plant-prefix: shared-prefix items that trust the runs (negative control)
uint64_t g_own_passes = 0;      // shared-prefix members that read their own rows after the page check

// Tokens of a row the caller's partitions cover, clamped to the table.
int reach_of(const Problem& pr) {
    return static_cast<int>(lmin(static_cast<int64_t>(pr.caller_splits) * pr.caller_split_tokens,
                                 static_cast<int64_t>(pr.width) * pr.page_size));
}

#define AUDIT(cond, ...)                                                    \
    do {                                                                    \
        ++g_checks;                                                         \
        if (!(cond)) {                                                      \
            if (g_failures++ < 20) {                                        \
                std::fprintf(stderr, "  FAIL %s:%d: ", __FILE__, __LINE__); \
                std::fprintf(stderr, __VA_ARGS__);                          \
                std::fprintf(stderr, "\n");                                 \
            }                                                               \
        }                                                                   \
    } while (0)

// Sizes of the buffers a caller passes for a problem.
struct Buffers {
    uint64_t q_bytes, kv_bytes, numerator_elems, stats_elems;
    int64_t table_elems;
};

Buffers buffers(const Problem& pr) {
    Buffers b;
    b.q_bytes = static_cast<uint64_t>(pr.batch) * pr.q_heads * pr.head_dim * pr.q_elem;
    b.kv_bytes = static_cast<uint64_t>(pr.pages) * pr.page_size * pr.kv_heads * pr.head_dim * pr.kv_elem;
    const uint64_t states = static_cast<uint64_t>(pr.batch) * pr.q_heads * kQuarters * pr.splits;
    b.numerator_elems = states * pr.head_dim;
    b.stats_elems = states * 2;
    b.table_elems = static_cast<int64_t>(pr.batch) * pr.width;
    return b;
}

PartialParams params(const Problem& pr, int cus, bool mfma, bool rows) {
    PartialParams p{};
    p.row_allowed = rows;
    p.batch = pr.batch;
    p.query_heads = pr.q_heads;
    p.group = pr.q_heads / pr.kv_heads;
    p.page_shift = pr.page_size == 16 ? 4 : 5;
    p.table_width = pr.width;
    p.physical_pages = pr.pages;
    p.splits = pr.splits;
    p.split_tokens = pr.split_tokens;
    p.reach = g_plant_reach ? pr.width * pr.page_size : reach_of(pr);
    p.token_bytes = static_cast<uint32_t>(pr.kv_heads * pr.head_dim * pr.kv_elem);
    p.page_bytes = static_cast<uint64_t>(pr.page_size) * p.token_bytes;
    p.unshared_pages = pr.unshared;
    p.ragged_lengths = pr.ragged;
    p.host_bounds = pr.bounds.empty() ? nullptr : pr.bounds.data();
    p.host_prefix_runs = pr.runs.empty() ? nullptr : pr.runs.data();
    plan_items(p, p.host_bounds);
    if (mfma) plan_mfma(p, pr.kv_heads, cus, pr.head_dim, pr.kv_elem);
    else plan_fp32(p, pr.kv_heads, pr.head_dim);
    return p;
}

// Writers of each state slot, to check that every live slot is written once.
// Also the XCD (linear dispatch index % 8) of the workgroups storing each
// row's states: -1 none yet, -2 more than one.
struct Coverage {
    std::vector<uint8_t> writes;
    std::vector<int8_t> row_xcd;
    Coverage() = default;
    Coverage(uint64_t states, uint64_t rows) : writes(states, 0), row_xcd(rows, -1) {}
    void store(uint64_t slot, int64_t row, int xcd) {
        AUDIT(slot < writes.size(), "state slot %" PRIu64 " past the workspace", slot);
        if (slot < writes.size() && writes[slot] < 255) ++writes[slot];
        if (row >= 0 && static_cast<uint64_t>(row) < row_xcd.size()) {
            int8_t& x = row_xcd[row];
            x = x == -1 ? static_cast<int8_t>(xcd) : x == xcd ? x : -2;
        }
    }
};

// Writers of each output element of a whole-row launch.
struct OutCoverage {
    std::vector<uint8_t> writes;
    explicit OutCoverage(uint64_t elems) : writes(elems, 0) {}
    void store(int64_t e) {
        AUDIT(e >= 0 && static_cast<uint64_t>(e) < writes.size(), "output element %" PRId64 " past out", e);
        if (e >= 0 && static_cast<uint64_t>(e) < writes.size() && writes[e] < 255) ++writes[e];
    }
};

void check_coverage(const Problem& pr, const Coverage& cov) {
    for (int b = 0; b < pr.batch; ++b) {
        const int len = imax(0, imin(pr.lengths[b], reach_of(pr)));
        const int live_parts = (len + pr.split_tokens - 1) / pr.split_tokens;
        for (int h = 0; h < pr.q_heads; ++h) {
            for (int part = 0; part < kQuarters * pr.splits; ++part) {
                const uint64_t slot = (static_cast<uint64_t>(b) * pr.q_heads + h) * kQuarters * pr.splits + part;
                const int expected = part < kQuarters * live_parts ? 1 : 0;
                AUDIT(cov.writes[slot] == expected, "seq %d head %d state %d written %d times, expected %d", b, h,
                      part, cov.writes[slot], expected);
            }
        }
    }
}

// The merge's side of an XCD-grouped grid (merge_xcd_row), for both merge
// kernels (one row per workgroup, and kMergeRowsPerGroup = 4 rows of one wave
// each): every row is taken exactly once, by a workgroup of its own sequence
// on the XCD whose workgroups stored all of the row's states.
void check_merge_xcd(const Problem& pr, const PartialParams& p, const Coverage& cov) {
    const int group_rows = xcd_row_group_rows(p);
    const int64_t rows = static_cast<int64_t>(pr.batch) * pr.q_heads;
    AUDIT(group_rows > 0 && rows % (8 * group_rows) == 0, "row groups of %d rows over %" PRId64 " rows", group_rows,
          rows);
    if (group_rows <= 0 || rows % (8 * group_rows) != 0) return;
    for (int64_t r = 0; r < rows; ++r) {
        const int len = imax(0, imin(pr.lengths[r / pr.q_heads], pr.width * pr.page_size));
        if (len > 0) AUDIT(cov.row_xcd[r] >= 0, "row %" PRId64 " states stored from XCDs %d", r, cov.row_xcd[r]);
    }
    for (int unit : {1, 4}) {
        if (group_rows % unit != 0) continue;
        const uint32_t gx = static_cast<uint32_t>(8 * group_rows / unit);
        const uint32_t gy = static_cast<uint32_t>(rows / group_rows / 8);
        std::vector<uint8_t> taken(rows, 0);
        for (uint32_t by = 0; by < gy; ++by) {
            for (uint32_t bx = 0; bx < gx; ++bx) {
                const int xcd = static_cast<int>((bx + static_cast<uint64_t>(gx) * by) % 8);
                for (int sub = 0; sub < unit; ++sub) {
                    const MergeRow m = merge_xcd_row(bx, by, group_rows, p.merge_xcd_shift, unit, sub);
                    AUDIT(m.row >= 0 && m.row < rows, "merge row %" PRId64, m.row);
                    if (m.row < 0 || m.row >= rows) continue;
                    AUDIT(m.b == m.row / pr.q_heads, "merge row %" PRId64 " given sequence %d", m.row, m.b);
                    ++taken[m.row];
                    const int stored = cov.row_xcd[m.row];
                    if (stored >= 0)
                        AUDIT(stored == xcd, "merge row %" PRId64 " on XCD %d, states on XCD %d", m.row, xcd, stored);
                }
            }
        }
        for (int64_t r = 0; r < rows; ++r) AUDIT(taken[r] == 1, "merge row %" PRId64 " taken %d times", r, taken[r]);
    }
}

int page_of(const Problem& pr, int b, int window, int slot, const PartialParams& p) {
    const int entry = window_entry(p, window + slot, 0);  // the lane holding slot reads entry window + slot
    return pr.table[static_cast<size_t>(b) * pr.width + entry];
}

// One load group of the matrix-core kernel (a 16-token tile), all 64 lanes.
template <int D>
void mfma_tile(const Problem& pr, const PartialParams& p, const Buffers& buf, const WaveWork& w, int b, int t0,
               int rb, int re, int window, int wave, int waves, int len, const std::vector<int>& members) {
    const int ES = pr.kv_elem;
    const int VH = D / 16, VW = VH * ES / 4, KR = D * ES / 16, TK = kWave / KR, KL = kTileTokens / TK;
    const int stage_row = mfma_stage_bytes(D, ES) / kTileTokens;
    const TileSpan span = tile_span(p, t0, kTileTokens, rb, re, window);
    AUDIT(span.slot >= 0 && span.slot < kWave, "window slot %d", span.slot);
    const int page = page_of(pr, b, window, span.slot, p);
    const bool ok = tile_live(p, t0, re, page);
    if (ok) {
        // The page id read is the table entry of the tile's logical page, and
        // the tile's live tokens lie on that one page, inside the sequence.
        AUDIT((span.lo >> p.page_shift) == window + span.slot, "tile %d reads window slot %d of window %d", t0,
              span.slot, window);
        AUDIT((span.hi >> p.page_shift) == (span.lo >> p.page_shift), "tile %d straddles a page", t0);
        AUDIT(span.lo >= rb && span.hi < re && span.hi < len, "tile %d span [%d, %d] outside [%d, %d)", t0, span.lo,
              span.hi, rb, re);
        // A shared-prefix item reads its leader's page for its members: every
        // reader with live tokens in the tile must name that page.
        {
            const int logical = span.lo >> p.page_shift;
            for (int s : members) {
                const int member_len = imax(0, imin(pr.lengths[s], reach_of(pr)));
                if (span.lo < member_len)
                    AUDIT(pr.table[static_cast<size_t>(s) * pr.width + logical] == page,
                          "tile %d: member %d maps page %d, the item reads page %d", t0, s,
                          pr.table[static_cast<size_t>(s) * pr.width + logical], page);
            }
        }
    }
    const uint64_t page_off = tile_page_offset(p, ok, page);
    const uint64_t head_off = static_cast<uint64_t>(w.kv_head) * D * ES;
    const uint64_t park = static_cast<uint64_t>(w.q_row) * D * 2;
    for (int lane = 0; lane < kWave; ++lane) {
        const int n = lane % 16, g = lane / 16;
        for (int s = 0; s < KL; ++s) {
            const uint32_t off = token_offset(p, ok, t0 + TK * s + lane / KR, span, static_cast<uint32_t>(lane % KR) * 16u);
            if (ok) AUDIT(head_off + page_off + off + 16 <= buf.kv_bytes, "K load past the cache");
            else AUDIT(park + off + 16 <= buf.q_bytes, "parked K load past q");
            const int lds = wave * kTileTokens * stage_row + (TK * s + lane / KR) * stage_row + (lane % KR) * 16;
            AUDIT(lds >= 0 && lds + (ES == 2 ? 16 : 8) <= waves * mfma_stage_bytes(D, ES), "K stage write");
        }
        for (int s = 0; s < D / 32; ++s) {
            const int lds = wave * kTileTokens * stage_row + k_token_of_row(n) * stage_row + (32 * s + 8 * g) * ES;
            AUDIT(lds + (ES == 2 ? 16 : 8) <= (wave + 1) * mfma_stage_bytes(D, ES), "K stage read outside the wave's tile");
        }
        for (int e = 0; e < 4; ++e) {
            const uint32_t off = token_offset(p, ok, t0 + 4 * e + g, span, static_cast<uint32_t>(n) * VH * ES);
            if (ok) AUDIT(head_off + page_off + off + 4u * VW <= buf.kv_bytes, "V load past the cache");
            else AUDIT(park + off + 4u * VW <= buf.q_bytes, "parked V load past q");
        }
    }
}

// One load group of the FP32 kernel (TPL tokens, NL = 1 load per chunk).
template <int D>
void fp32_group(const Problem& pr, const PartialParams& p, const Buffers& buf, const WaveWork& w, int b, int g0,
                int rb, int re, int window, int len) {
    const int LPT = D / 4, TPL = kWave / LPT;
    const TileSpan span = tile_span(p, g0, TPL, rb, re, window);
    const int page = page_of(pr, b, window, span.slot, p);
    const bool ok = tile_live(p, g0, re, page);
    if (ok) {
        AUDIT((span.lo >> p.page_shift) == window + span.slot, "group %d reads the wrong window slot", g0);
        AUDIT((span.hi >> p.page_shift) == (span.lo >> p.page_shift), "group %d straddles a page", g0);
        AUDIT(span.lo >= rb && span.hi < re && span.hi < len, "group %d span outside the range", g0);
    }
    const uint64_t page_off = tile_page_offset(p, ok, page);
    const uint64_t head_off = static_cast<uint64_t>(w.kv_head) * D * 4;
    const uint64_t park = static_cast<uint64_t>(w.q_row) * D * 4;
    for (int lane = 0; lane < kWave; ++lane) {
        const uint32_t off = token_offset(p, ok, g0 + lane / LPT, span, static_cast<uint32_t>(lane % LPT) * 16u);
        if (ok) AUDIT(head_off + page_off + off + 16 <= buf.kv_bytes, "K/V load past the cache");
        else AUDIT(park + off + 16 <= buf.q_bytes, "parked load past q");
    }
}

// Page-id window loads of all lanes at `window`.
void window_loads(const Problem& pr, const PartialParams& p, const Buffers& buf, int b, int window) {
    for (int lane = 0; lane < kWave; ++lane) {
        const int entry = window_entry(p, window, lane);
        AUDIT(entry >= 0 && entry < pr.width, "window entry %d", entry);
        AUDIT(static_cast<int64_t>(b) * pr.width + entry < buf.table_elems, "table load past the table");
    }
}

template <int D, int GT>
void audit_launch(const Problem& pr, const PartialParams& p, bool mfma, Coverage& cov, OutCoverage& out) {
    constexpr int TPLV = kWave / (D / 4);  // FP32 kernel: token rows per 16-byte load group
    const Buffers buf = buffers(pr);
    const Grid grid = partial_grid(p, pr.kv_heads);
    AUDIT(p.grid_x == grid.x && p.grid_y == grid.y, "kernel-argument grid %ux%u, launch %ux%u", p.grid_x, p.grid_y,
          grid.x, grid.y);
    const int waves = partial_threads(p) / kWave;
    AUDIT(waves >= 1 && waves <= (p.row_mode ? kRowMaxWaves : 8), "workgroup of %d waves", waves);
    if (mfma) AUDIT(mfma_lds_bytes(p, D, pr.kv_elem) <= 160 * 1024, "LDS %d bytes", mfma_lds_bytes(p, D, pr.kv_elem));
    const int align = mfma ? kTileTokens : kWave / (D / 4);
    // Load groups per straight-line block and issued ahead, as the kernels'
    // constants: matrix-core 2 and 2 (FP8 K/V outside whole rows: 4 and 4);
    // FP32 16 and 4, whole-row FP32 launches 4 and 4.
    const bool fp8_deep = mfma && pr.kv_elem == 1 && !p.row_mode;
    const int block = mfma ? (fp8_deep ? 4 : 2) : p.row_mode ? 4 : 16;
    const int ahead = mfma ? (fp8_deep ? 4 : 2) : 4, group_tokens = align;
    const int qw = p.quarters_per_wg;
    for (uint32_t bz = 0; bz < grid.z; ++bz) {
        for (uint32_t by = 0; by < grid.y; ++by) {
            for (uint32_t bx = 0; bx < grid.x; ++bx) {
                const int kind = grid_kind(p);
                const BlockCoords bc =
                    kind == kGridRectTails
                        ? block_coords<kGridRectTails>(bx, by, bz, p.grid_x, p.grid_y, p.xcd_shift, p.xcd_main_rows,
                                                       p.xcd_tail_shift)
                        : block_coords<kGridRect>(bx, by, bz, p.grid_x, p.grid_y, p.xcd_shift, p.xcd_main_rows,
                                                  p.xcd_tail_shift);
                const int xcd = static_cast<int>((bx + static_cast<uint64_t>(grid.x) * (by + static_cast<uint64_t>(grid.y) * bz)) % 8);
                const PartitionRange r = kind == kGridList        ? partition_range<kGridList>(p, bc)
                                         : kind == kGridRectTails ? partition_range<kGridRectTails>(p, bc)
                                                                  : partition_range<kGridRect>(p, bc);
                AUDIT(r.b >= 0 && r.b < pr.batch, "sequence %d", r.b);
                AUDIT(r.first >= 0 && r.count >= 0 && r.first + r.count <= pr.splits && r.count <= p.tail_span &&
                          r.first < pr.splits,
                      "partition range %d + %d", r.first, r.count);
                if (r.b < 0 || r.b >= pr.batch) continue;
                const int b = r.b;
                // A shared-prefix item's member sequences (else the item's
                // own); the wave covers the longest member's tokens.
                std::vector<int> members{b};
                if (r.members == 1) AUDIT(r.row == b, "item of sequence %d reads row %d", b, r.row);
                if (r.members != 1) {
                    AUDIT(kind == kGridList && mfma && !p.row_mode, "shared-prefix item outside a matrix-core work list");
                    AUDIT(r.members >= 2 && r.members <= 16 / GT && r.member0 >= 0 &&
                              r.member0 + r.members <= kCompactMaxBatch && r.count == 1,
                          "shared-prefix item of %d members from slot %d, count %d", r.members, r.member0, r.count);
                    members.clear();
                    for (int m = 0; m < r.members && r.member0 + m < kCompactMaxBatch; ++m) {
                        const int s = p.prefix_order[r.member0 + m];
                        AUDIT(s >= 0 && s < pr.batch, "member sequence %d", s);
                        for (int other : members) AUDIT(other != s, "sequence %d twice in one item", s);
                        if (s >= 0 && s < pr.batch) members.push_back(s);
                    }
                    AUDIT(!members.empty() && members[0] == b, "item sequence %d is not its first member", b);
                    AUDIT(r.row >= 0 && r.row < pr.batch && !pr.runs.empty() && pr.runs[2 * members[0]] == r.row,
                          "item reads row %d, not its members' leader", r.row);
                    if (members.empty() || r.row < 0 || r.row >= pr.batch) continue;
                }
                int len_raw = 0;
                for (int s : members) len_raw = imax(len_raw, pr.lengths[s]);
                // Live tokens: the length clamped to the table and to the
                // caller's partitions; every read below is checked against it.
                const int len = imax(0, imin(len_raw, reach_of(pr)));
                const bool rows = p.row_mode != 0;
                const int row_limit = mfma ? kRowMaxWaves : fp32_row_max_waves(GT);
                if (rows) {
                    AUDIT(!p.compact && waves == p.row_waves && waves <= row_limit, "whole-row launch of %d waves",
                          waves);
                    AUDIT(grid.x == 1 && r.first == 0 && r.count == 1 && r.qgroup == 0, "whole-row workgroup item");
                }
                int64_t row_q = -1;
                int row_heads = -1, row_next = 0;
                const int row_end = static_cast<int>(lmin(static_cast<int64_t>(pr.splits) * pr.split_tokens, len));
                for (int wave = 0; wave < waves; ++wave) {
                    const int split = r.first;
                    int window = rows ? (mfma ? row_speculative_page<kTileTokens>(p, wave, waves)
                                              : row_speculative_page<TPLV>(p, wave, waves))
                                      : mfma ? speculative_page<kTileTokens>(p, split, r.count, r.qgroup, wave)
                                             : speculative_page<TPLV>(p, split, r.count, r.qgroup, wave);
                    window_loads(pr, p, buf, r.row, window);
                    {
                        const WaveWork w =
                            rows ? (mfma ? row_wave_work<GT, kTileTokens>(p, b, bc.heads, wave, waves, len_raw)
                                         : row_wave_work<GT, TPLV>(p, b, bc.heads, wave, waves, len_raw))
                            : mfma ? wave_work<GT, kTileTokens>(p, b, split, r.count, r.qgroup, bc.heads, wave,
                                                                len_raw)
                                   : wave_work<GT, TPLV>(p, b, split, r.count, r.qgroup, bc.heads, wave, len_raw);
                        if (rows) {
                            // Every wave writes its LDS slot (an empty slice
                            // the empty state); the slices tile the row's
                            // tokens [0, min(len, splits * split_tokens)) in
                            // wave order; all waves share the row.
                            if (mfma) {
                                const int lds = mfma_lds_bytes(p, D, pr.kv_elem);
                                const int base = waves * mfma_stage_bytes(D, pr.kv_elem);
                                AUDIT(base + (wave + 1) * combine_slot_bytes(D) <= lds && lds <= 160 * 1024,
                                      "row slot write");
                            } else {
                                AUDIT(waves * row_slot_bytes_fp32(D) <= 160 * 1024, "row slots");
                            }
                            if (row_q < 0) {
                                row_q = w.q_row;
                                row_heads = w.heads_here;
                            }
                            AUDIT(w.q_row == row_q && w.heads_here == row_heads, "waves of one row disagree");
                            if (!w.dead) {
                                AUDIT(w.wb == row_next, "slice %d starts at %d, expected %d", wave, w.wb, row_next);
                                row_next = w.we;
                            }
                            if (wave == waves - 1) AUDIT(row_next == row_end, "slices end at %d of %d", row_next, row_end);
                        }
                        AUDIT(r.count > 0 || w.dead, "an empty grid item is not dead");
                        if (w.dead) {
                            AUDIT(!rows || w.wb == w.we, "dead row wave with tokens");
                            continue;
                        }
                        AUDIT(w.kv_head >= 0 && w.kv_head < pr.kv_heads, "KV head %d", w.kv_head);
                        AUDIT(w.tile >= 0 && w.tile < p.head_tiles, "head tile %d", w.tile);
                        AUDIT(w.q_row >= 0 && w.q_row + w.heads_here <= static_cast<int64_t>(pr.batch) * pr.q_heads,
                              "q row %" PRId64, w.q_row);
                        // A wave's tokens lie in its partitions (a whole-row
                        // wave's: in the row's, [0, splits * split_tokens)).
                        const int64_t first = rows ? 0 : static_cast<int64_t>(split) * pr.split_tokens;
                        const int64_t parts = rows ? pr.splits : r.count;
                        AUDIT(w.wb >= first && w.we <= first + parts * pr.split_tokens && w.wb <= w.we && w.we <= len,
                              "wave range [%d, %d) of partitions %d + %" PRId64, w.wb, w.we, split, parts);
                        // q loads of the tile's live heads (a shared-prefix
                        // item: column n is member n / GT's head n % GT).
                        const int64_t row_base = static_cast<int64_t>(w.kv_head) * p.group +
                                                 static_cast<int64_t>(w.tile) * GT;
                        for (int lane = 0; lane < kWave; ++lane) {
                            if (mfma && members.size() > 1) {
                                const int n = lane % 16, g = lane / 16, m = n / GT, h = n % GT;
                                if (m < static_cast<int>(members.size()) && h < w.heads_here)
                                    for (int s = 0; s < D / 32; ++s)
                                        AUDIT(static_cast<uint64_t>((members[m] * static_cast<int64_t>(pr.q_heads) +
                                                                     row_base + h) * D + 32 * s + 8 * g) * 2 + 16 <=
                                                  buf.q_bytes, "member q load");
                            } else if (mfma) {
                                const int n = lane % 16, g = lane / 16;
                                if (n < w.heads_here)
                                    for (int s = 0; s < D / 32; ++s)
                                        AUDIT(static_cast<uint64_t>((w.q_row + n) * D + 32 * s + 8 * g) * 2 + 16 <=
                                                  buf.q_bytes, "q load");
                            } else {
                                for (int h = 0; h < w.heads_here; ++h)
                                    AUDIT(static_cast<uint64_t>((w.q_row + h) * D + (lane % (D / 4)) * 4) * 4 + 16 <=
                                              buf.q_bytes, "q load");
                            }
                        }
                        // A shared-prefix item's page check (prefix_span_pages):
                        // the table loads of every pair, and the members whose
                        // rows differ from the first member's where they have
                        // tokens, which then read their own rows.
                        std::vector<int> shared_members = members, own;
                        if (members.size() > 1) {
                            const int span = prefix_span_pages(p, w.wb, w.we);
                            const int pairs = span * static_cast<int>(members.size());
                            std::vector<bool> differs(members.size(), false);
                            for (int pair = 0; pair < pairs; ++pair) {
                                const int m = prefix_pair_member(pair, span);
                                const int page = prefix_pair_page(p, w.wb, pair, span);
                                const int m_end = imin(imax(0, imin(pr.lengths[members[m]], reach_of(pr))), w.we);
                                if ((page << p.page_shift) >= m_end) continue;
                                AUDIT(page >= 0 && page < pr.width, "page check entry %d", page);
                                if (page < 0 || page >= pr.width) continue;
                                if (pr.table[static_cast<size_t>(members[m]) * pr.width + page] !=
                                    pr.table[static_cast<size_t>(r.row) * pr.width + page])
                                    differs[m] = true;
                            }
                            shared_members.clear();
                            for (size_t m = 0; m < members.size(); ++m) {
                                if (differs[m] && !g_plant_no_check) own.push_back(members[m]);
                                else shared_members.push_back(members[m]);
                            }
                            g_own_passes += own.size();
                        }
                        // The kernels' token loop: page-id windows of 64 pages,
                        // load groups issued `ahead` in blocks of `block`; a
                        // shared-prefix item runs it once over the first
                        // member's row for the members that share it, then
                        // once per member with a row of its own.
                        auto walk = [&](int row_b, int end, const std::vector<int>& readers) {
                            int rb = w.wb, re = w.wb;
                            int win = row_b == r.row ? window : -1;
                            for (rb = w.wb; rb < end; rb = re) {
                                if ((rb >> p.page_shift) != win) {
                                    win = rb >> p.page_shift;
                                    window_loads(pr, p, buf, row_b, win);
                                }
                                re = imin(end, (win + kWave) << p.page_shift);
                                for (int s0 = rb & ~(group_tokens - 1); s0 < re; s0 += block * group_tokens) {
                                    auto issue = [&](int t0) {
                                        if (mfma)
                                            mfma_tile<D>(pr, p, buf, w, row_b, t0, rb, re, win, wave, waves, len,
                                                         readers);
                                        else fp32_group<D>(pr, p, buf, w, row_b, t0, rb, re, win, len);
                                    };
                                    for (int n0 = 0; n0 < ahead; ++n0) issue(s0 + n0 * group_tokens);
                                    for (int c = 0; c < block; ++c) {
                                        if (s0 + c * group_tokens >= re) break;
                                        if (c + ahead < block) issue(s0 + (c + ahead) * group_tokens);
                                    }
                                }
                            }
                        };
                        walk(r.row, w.we, members.size() > 1 ? shared_members : members);
                        for (int s : own)
                            walk(s, imin(w.we, imax(0, imin(pr.lengths[s], reach_of(pr)))), std::vector<int>{s});
                        if (rows) continue;  // no state stores: the fold below writes out
                        // State stores: one state per live head of the tile;
                        // a combining workgroup's later quarters store the empty
                        // state in their own slots.
                        const int part = split * kQuarters + w.quarter;
                        AUDIT(part >= 0 && part < kQuarters * pr.splits, "state %d", part);
                        // A shared-prefix item stores each member's states,
                        // for members whose own length reaches the partition.
                        for (size_t m = 1; m < members.size(); ++m) {
                            const int member_len = imax(0, imin(pr.lengths[members[m]], reach_of(pr)));
                            if (static_cast<int64_t>(split) * pr.split_tokens >= member_len) continue;
                            for (int h = 0; h < w.heads_here; ++h) {
                                const int64_t row = members[m] * static_cast<int64_t>(pr.q_heads) + row_base + h;
                                AUDIT(numerator_offset(p, row, part, D) + D <= static_cast<int64_t>(buf.numerator_elems),
                                      "member numerator store");
                                AUDIT(stats_offset(p, row, part) + 2 <= static_cast<int64_t>(buf.stats_elems),
                                      "member stats store");
                                cov.store(static_cast<uint64_t>(row) * kQuarters * pr.splits + part, row, xcd);
                            }
                        }
                        const int lead_len = imax(0, imin(pr.lengths[b], reach_of(pr)));
                        const bool lead_stores = members.size() == 1 ||
                                                 static_cast<int64_t>(split) * pr.split_tokens < lead_len;
                        for (int h = 0; h < (lead_stores ? w.heads_here : 0); ++h) {
                            const int64_t row = w.q_row + h;
                            AUDIT(numerator_offset(p, row, part, D) + D <= static_cast<int64_t>(buf.numerator_elems),
                                  "numerator store");
                            AUDIT(stats_offset(p, row, part) + 2 <= static_cast<int64_t>(buf.stats_elems), "stats store");
                            cov.store(static_cast<uint64_t>(row) * kQuarters * pr.splits + part, row, xcd);
                            // Empty states of the span's other live partitions.
                            const int extra = extra_live_partitions(p, split, r.count, len_raw);
                            for (int e = 1; e <= extra; ++e) {
                                const int ep = (split + e) * kQuarters + w.quarter;
                                AUDIT(stats_offset(p, row, ep) + 2 <= static_cast<int64_t>(buf.stats_elems),
                                      "empty-state store");
                                cov.store(static_cast<uint64_t>(row) * kQuarters * pr.splits + ep, row, xcd);
                            }
                        }
                        if (mfma && p.combine) {
                            const int qq = wave % qw;
                            const int slot_bytes = combine_slot_bytes(D);
                            const int base = waves * mfma_stage_bytes(D, pr.kv_elem);
                            const int lds = mfma_lds_bytes(p, D, pr.kv_elem);
                            if (qq != 0)
                                AUDIT(base + (wave / qw * (qw - 1) + qq) * slot_bytes <= lds, "combine slot write");
                            else
                                AUDIT(base + (wave / qw * (qw - 1) + qw - 1) * slot_bytes <= lds, "combine slot read");
                        }
                    }
                }
                if (rows) {
                    // The fold. Matrix-core kernel: output element o of the
                    // row's live heads, o < heads_here * D, is column o % 16,
                    // dims (o / 16) % (D / 16) of head o / D, read from lane
                    // 16 (h / 4) + col of each slot. FP32 kernel: element o is
                    // slot word 16 + o.
                    const int vh = D / 16;
                    for (int o = 0; o < row_heads * D; ++o) {
                        if (mfma) {
                            const int col = o % 16, j = (o / 16) % vh, h = o / D;
                            AUDIT(h < GT && 16 * (h / 4) + col < kWave && j < vh, "fold element %d", o);
                            out.store((row_q + h) * D + col * vh + j);
                        } else {
                            AUDIT(16 + o < row_slot_bytes_fp32(D) / 4 && o / D < GT, "fold element %d", o);
                            out.store(row_q * D + o);
                        }
                    }
                }
            }
        }
    }
}

template <int D>
void audit_gt(const Problem& pr, const PartialParams& p, bool mfma, Coverage& cov, OutCoverage& out) {
    switch (p.head_tile) {
        case 1: return audit_launch<D, 1>(pr, p, mfma, cov, out);
        case 2: return audit_launch<D, 2>(pr, p, mfma, cov, out);
        case 4: return audit_launch<D, 4>(pr, p, mfma, cov, out);
        case 8: return audit_launch<D, 8>(pr, p, mfma, cov, out);
        default: return audit_launch<D, 16>(pr, p, mfma, cov, out);
    }
}

// Audits the launch planned for a partition-only call (states), and for a
// full decode call (rows: the planner may choose a whole-row launch); leaves
// the launch's params and which state slots it wrote in p and cov.
bool audit(const Problem& pr, bool rows, PartialParams& p, Coverage& cov) {
    const int before = g_failures;
    const uint64_t checks_before = g_checks;
    const uint64_t own_before = g_own_passes;
    const bool mfma = pr.q_elem == 2;
    p = params(pr, 256, mfma, rows);
    cov = Coverage(static_cast<uint64_t>(pr.batch) * pr.q_heads * kQuarters * pr.splits,
                   static_cast<uint64_t>(pr.batch) * pr.q_heads);
    OutCoverage out(static_cast<uint64_t>(pr.batch) * pr.q_heads * pr.head_dim);
    if (pr.head_dim == 64) audit_gt<64>(pr, p, mfma, cov, out);
    else audit_gt<128>(pr, p, mfma, cov, out);
    if (!mfma || p.row_mode) AUDIT(p.group_items == 0, "shared-prefix items in a %s launch", mfma ? "whole-row" : "fp32");
    if (p.row_mode) {
        AUDIT(mfma_lds_bytes(p, pr.head_dim, pr.kv_elem) <= 160 * 1024, "whole-row LDS");
        for (size_t e = 0; e < out.writes.size(); ++e)
            AUDIT(out.writes[e] == 1, "output element %zu written %d times", e, out.writes[e]);
    } else {
        check_coverage(pr, cov);
        if (p.merge_xcd_rows > 0) check_merge_xcd(pr, p, cov);
    }
    const Grid grid = partial_grid(p, pr.kv_heads);
    std::string shared = p.group_items > 0 ? ", " + std::to_string(p.group_items) + " shared-prefix items" : "";
    if (g_own_passes > own_before) shared += " (" + std::to_string(g_own_passes - own_before) + " own passes)";
    std::printf("%-44s %s grid %ux%ux%u x %d waves, GT %d, qw %d, %s%s%s%s, %" PRIu64 " checks: %s\n",
                (pr.name + (rows ? " [call]" : "")).c_str(), mfma ? "mfma" : "fp32", grid.x, grid.y, grid.z,
                partial_threads(p) / kWave, p.head_tile, p.quarters_per_wg,
                p.row_mode ? "whole rows" : p.compact ? "compact" : p.main_splits < p.splits ? "rectangular+tails"
                                                                                              : "rectangular",
                p.combine ? ", combined" : "",
                p.xcd_shift >= 0 ? ", xcd-grouped" : p.merge_xcd_rows > 0 ? ", xcd merge" : "", shared.c_str(),
                g_checks - checks_before, g_failures == before ? "ok" : "FAILED");
    std::fflush(stdout);
    return g_failures == before;
}


// ---------------------------------------------------------------------------
// Merge launches (merge_map.h): every workgroup, wave and lane of the merge a
// call runs after its partition launch, following the kernels' loop
// structure (decode.hip: merge_cols_kernel's optimistic first round, its two
// statistics scans and its accumulation rounds; merge_rows_kernel's single
// round). Every numerator and statistics load is checked against the
// workspace, every LDS weight against the launch's dynamic LDS, every output
// store against out (each element written exactly once), and every state the
// merge counts as live must have been written by the partition launch.

uint64_t g_merge_launches = 0;
bool g_plant_merge_live = false;  // --plant-merge-live: merge params that count one partition too many

struct MergeWalk {
    const Problem& pr;
    const MergeParams& mp;
    const MergeLaunch& ml;
    const Coverage& written;  // state slots the partition launch wrote
    uint64_t numerator_elems, stats_elems;
    OutCoverage out;

    MergeWalk(const Problem& p, const MergeParams& m, const MergeLaunch& l, const Coverage& w)
        : pr(p), mp(m), ml(l), written(w), out(static_cast<uint64_t>(p.batch) * p.q_heads * p.head_dim) {
        const Buffers buf = buffers(p);
        numerator_elems = buf.numerator_elems;
        stats_elems = buf.stats_elems;
    }
    int parts() const { return mp.parts >> mp.stride_shift; }
    int live(int b) const {
        const int per_part = (kQuarters >> mp.stride_shift) + (g_plant_merge_live ? kQuarters : 0);
        return live_states(pr.lengths[b], mp.split_tokens, mp.reach, per_part, parts());
    }
    void numerator_load(int64_t base, int j) {
        AUDIT(j >= 0 && j < parts(), "merge read unit %d of %d", j, parts());
        const int64_t idx = base + merge_numerator_offset(mp, pr.head_dim, j);
        AUDIT(idx >= 0 && static_cast<uint64_t>(idx + 1) * 4 <= numerator_elems, "numerator load %" PRId64, idx);
    }
    void stats_load(int64_t base, int j) {
        AUDIT(j >= 0 && j < parts(), "merge stats unit %d of %d", j, parts());
        const int64_t idx = base + merge_stats_offset(mp, j);
        AUDIT(idx >= 0 && static_cast<uint64_t>(idx + 1) * 2 <= stats_elems, "stats load %" PRId64, idx);
    }
    // A state the merge weighs in (j < live) holds what the partition launch wrote.
    void used(int64_t row, int j) {
        const uint64_t slot = static_cast<uint64_t>(row) * kQuarters * pr.splits + merge_stats_offset(mp, j);
        AUDIT(slot < written.writes.size() && written.writes[slot] == 1, "merge uses state %d of row %" PRId64
              " that the partition launch did not write", j, row);
    }
    void check_row(const MergeRow& mr) {
        AUDIT(mr.row >= 0 && mr.row < static_cast<int64_t>(pr.batch) * pr.q_heads && mr.b == mr.row / pr.q_heads,
              "merge row %" PRId64 " of sequence %d", mr.row, mr.b);
    }
};

void walk_merge_cols(MergeWalk& mw) {
    const MergeParams& mp = mw.mp;
    const MergeLaunch& ml = mw.ml;
    const int D = mw.pr.head_dim, CH = ml.ch, TPR = CH / 4, PG = kMergeThreads / TPR, NB = ml.nb, SU = NB / 2;
    const int scan = ml.shared ? kMergeThreads : kWave, scan_round = SU * scan;
    const int parts = mw.parts(), last = parts - 1;
    AUDIT(D % CH == 0 && ml.grid_z == static_cast<uint32_t>(D / CH) && ml.threads == kMergeThreads, "merge_cols launch");
    if (ml.shared) AUDIT(ml.lds_bytes == parts * 4 && ml.lds_bytes <= 160 * 1024, "shared merge LDS %d", ml.lds_bytes);
    for (uint32_t bz = 0; bz < ml.grid_z; ++bz)
        for (uint32_t by = 0; by < ml.grid_y; ++by)
            for (uint32_t bx = 0; bx < ml.grid_x; ++bx) {
                const MergeRow mr = merge_cols_row(mp, bx, by);
                mw.check_row(mr);
                if (mr.row < 0 || mr.b < 0 || mr.b >= mw.pr.batch) continue;
                const int chunk = static_cast<int>(bz);
                const int live = mw.live(mr.b);
                const int first_n = imax(1, imin(parts, mp.first_states));
                const int64_t sbase = merge_stats_base(mp, mr.row);
                for (int t = 0; t < kMergeThreads; ++t) {
                    const int lane = t % kWave, col = t % TPR, pg = t / TPR, scan0 = ml.shared ? t : lane;
                    const int64_t nbase = merge_numerator_base(mp, mr.row, D, chunk, CH, col);
                    auto load_round = [&](int base, int k0, int k1) {
                        for (int k = k0; k < k1 && k < NB; ++k) {
                            const int j = merge_load_unit(base, pg, k, PG, last);
                            mw.numerator_load(nbase, j);
                            if (!ml.shared) mw.stats_load(sbase, j);
                        }
                    };
                    const int optimistic = imin(kOptimisticRounds, merge_cols_rounds(0, first_n, NB, PG));
                    load_round(0, 0, optimistic);
                    load_round(0, optimistic, merge_cols_rounds(0, live, NB, PG));
                    const int scan_end = imin(scan_round, (first_n + scan - 1) / scan * scan);
                    for (int pass = 0; pass < 2; ++pass) {  // maximum, then denominator (and weights)
                        auto scan_at = [&](int base, int limit, bool load) {
                            for (int i = 0; i < SU; ++i) {
                                if (base + i * scan >= limit) continue;
                                if (load) mw.stats_load(sbase, imin(base + scan0 + i * scan, last));
                                const int j = base + scan0 + i * scan;
                                if (pass == 1 && ml.shared && j < live)
                                    AUDIT((j + 1) * 4 <= ml.lds_bytes, "weight[%d] write past %d B", j, ml.lds_bytes);
                            }
                        };
                        scan_at(0, first_n, pass == 0);  // the first round stays in registers for pass 1
                        for (int base = scan_end; base < live; base += scan_round) scan_at(base, live, true);
                    }
                    for (int base = 0;;) {
                        const int rounds = merge_cols_rounds(base, live, NB, PG);
                        for (int k = 0; k < rounds && k < NB; ++k) {
                            const int j = base + pg + k * PG;
                            if (j < live) {
                                mw.used(mr.row, j);
                                if (ml.shared) AUDIT((j + 1) * 4 <= ml.lds_bytes, "weight[%d] read", j);
                            }
                        }
                        base += NB * PG;
                        if (base >= live) break;
                        load_round(base, 0, merge_cols_rounds(base, live, NB, PG));
                    }
                    AUDIT(pg < PG && col < TPR, "column_sum[%d][%d]", pg, col);
                    if (t < CH) mw.out.store(mr.row * D + chunk * CH + t);
                }
            }
}

void walk_merge_rows(MergeWalk& mw) {
    const MergeParams& mp = mw.mp;
    const MergeLaunch& ml = mw.ml;
    const int D = mw.pr.head_dim, TPR = D / 4, PGW = kWave / TPR, NB = ml.nb, RPG = kMergeRowsPerGroup;
    const int parts = mw.parts(), last = parts - 1, rounds = (parts + PGW - 1) / PGW;
    AUDIT(rounds <= NB && parts <= kWave && ml.threads == kWave * RPG, "merge_rows launch of %d states", parts);
    for (uint32_t by = 0; by < ml.grid_y; ++by)
        for (uint32_t bx = 0; bx < ml.grid_x; ++bx)
            for (int wave = 0; wave < RPG; ++wave) {
                const MergeRow mr = merge_rows_row(mp, bx, by, wave, RPG);
                if (mr.row < 0) {
                    AUDIT(mp.xcd_rows == 0 && static_cast<int>(bx) * RPG + wave >= mp.query_heads, "wave skipped");
                    continue;
                }
                mw.check_row(mr);
                if (mr.b < 0 || mr.b >= mw.pr.batch) continue;
                const int live = mw.live(mr.b);
                const int64_t sbase = merge_stats_base(mp, mr.row);
                for (int lane = 0; lane < kWave; ++lane) {
                    const int col = lane % TPR, pg = lane / TPR;
                    const int64_t nbase = merge_numerator_base(mp, mr.row, D, 0, D, col);
                    for (int k = 0; k < NB && k < rounds; ++k) {
                        const int j = merge_load_unit(0, pg, k, PGW, last);
                        mw.numerator_load(nbase, j);
                        if (!ml.shared) mw.stats_load(sbase, j);
                        const int jj = pg + k * PGW;
                        if (jj < live) {
                            mw.used(mr.row, jj);
                            AUDIT(jj < kWave, "state %d's weight is outside the wave", jj);
                        }
                    }
                    mw.stats_load(sbase, imin(lane, last));  // lane j holds state j's (m, l)
                    if (pg == 0)
                        for (int e = 0; e < 4; ++e) mw.out.store(mr.row * D + col * 4 + e);
                }
            }
}

// The merge a call runs over the states of partition launch p: the staged
// entry's (pd_decode_merge: every state, plain rows, no bounds) or the full
// call's (combined quarters, XCD-grouped rows, bounds), for both merge modes.
bool audit_merges(const Problem& pr, const PartialParams& p, const Coverage& cov, bool full_call) {
    const int before = g_failures;
    const uint64_t checks_before = g_checks;
    std::string kinds;
    for (int shared = 0; shared < 2; ++shared) {
        if (shared && kQuarters * pr.splits > 4096) continue;  // PD_SHARED_MERGE_MAX_PARTS
        MergeParams mp{};
        mp.parts = kQuarters * pr.splits;
        const int stride = full_call && p.combine ? p.quarters_per_wg : 1;
        mp.stride_shift = stride == 4 ? 2 : stride == 2 ? 1 : 0;
        mp.query_heads = pr.q_heads;
        mp.split_tokens = pr.split_tokens;
        mp.reach = reach_of(pr);
        mp.first_states = merge_first_states(mp.parts, mp.stride_shift, mp.split_tokens, mp.reach,
                                             full_call && !pr.bounds.empty() ? pr.bounds.data() : nullptr, pr.batch);
        mp.xcd_rows = full_call ? p.merge_xcd_rows : 0;
        mp.xcd_shift = full_call ? p.merge_xcd_shift : 0;
        const MergeLaunch ml = plan_merge(mp, pr.batch, pr.head_dim, shared != 0, 256);
        mp.xcd_rows = ml.xcd_rows;
        MergeWalk mw(pr, mp, ml, cov);
        if (ml.kind == kMergeRows) walk_merge_rows(mw);
        else walk_merge_cols(mw);
        for (size_t e = 0; e < mw.out.writes.size(); ++e)
            AUDIT(mw.out.writes[e] == 1, "merge output element %zu written %d times", e, mw.out.writes[e]);
        ++g_merge_launches;
        kinds += std::string(shared ? " shared:" : " serial:") + (ml.kind == kMergeRows ? "rows" : "cols") +
                 (ml.kind == kMergeCols ? "/NB" + std::to_string(ml.nb) + "/CH" + std::to_string(ml.ch) : "") +
                 (ml.xcd_rows > 0 ? "/xcd" : "") + (mp.stride_shift ? "/stride" + std::to_string(stride) : "");
    }
    std::printf("%-44s merge%s%s, %" PRIu64 " checks: %s\n", (pr.name + (full_call ? " [call]" : " [stage]")).c_str(),
                kinds.c_str(), "", g_checks - checks_before, g_failures == before ? "ok" : "FAILED");
    std::fflush(stdout);
    return g_failures == before;
}


// ---------------------------------------------------------------------------
// KV-cache append (cache_map.h; decode.hip: append_kv_kernel with explicit
// positions, grid tokens x batch, and append_kv_advance_kernel, grid batch,
// all or nothing per sequence), 256 threads each copying 16-byte chunks of
// a token's K and V rows. Every table read, new-token read and cache write is
// checked against its buffer, and every written row is the one the decode
// reads the token from (page table[b, pos / T], slot pos % T).

bool g_plant_append_capacity = false;  // --plant-append: capacity one page past the table (negative control)
bool g_plant_csr_count = false;        // --plant-csr: no bound on the indices read (negative control)

struct AppendProblem {
    std::string name;
    int batch, tokens, kv_heads, head_dim, elem, page_size, width, pages, max_context;
    std::vector<int32_t> table, starts;  // starts: positions (explicit) or lengths (advance)
    bool advance;
};

bool audit_append(const AppendProblem& ap) {
    const int before = g_failures;
    const uint64_t checks_before = g_checks;
    AppendParams a{};
    a.tokens = ap.tokens;
    a.table_width = ap.width;
    a.page_shift = ap.page_size == 16 ? 4 : 5;
    a.physical_pages = ap.pages;
    a.capacity = static_cast<int64_t>(ap.width) << a.page_shift;
    if (ap.advance) a.capacity = lmin(a.capacity, ap.max_context);
    if (g_plant_append_capacity) a.capacity = static_cast<int64_t>(ap.width + 1) << a.page_shift;
    a.row_bytes = static_cast<uint32_t>(ap.kv_heads * ap.head_dim * ap.elem);
    const int64_t new_bytes = static_cast<int64_t>(ap.batch) * ap.tokens * a.row_bytes;
    const int64_t cache_bytes = static_cast<int64_t>(ap.pages) * ap.page_size * a.row_bytes;
    const uint32_t chunks = a.row_bytes / 16u;
    AUDIT(a.row_bytes % 16 == 0, "row of %u bytes", a.row_bytes);
    std::vector<uint8_t> row_writes(static_cast<size_t>(ap.pages) * ap.page_size, 0);
    int written = 0;
    // Cache row of (b, pos) through the kernel's map, its table read checked.
    auto row_of = [&](int b, int64_t pos) -> int64_t {
        const int64_t entry = append_table_entry(a, pos);
        if (entry < 0) return -1;
        AUDIT(entry < ap.width, "append reads table entry %" PRId64 " of a %d-wide row", entry, ap.width);
        if (entry >= ap.width) return -1;
        const int page = ap.table[static_cast<size_t>(b) * ap.width + entry];
        const int64_t row = append_cache_row(a, page, pos);
        if (row >= 0) {
            AUDIT(pos < static_cast<int64_t>(ap.width) * ap.page_size && page >= 0 && page < ap.pages &&
                      row == static_cast<int64_t>(page) * ap.page_size + pos % ap.page_size,
                  "append row %" PRId64 " for position %" PRId64, row, pos);
            if (ap.advance) AUDIT(pos < ap.max_context, "append past max_context at %" PRId64, pos);
        }
        return row;
    };
    auto copy = [&](int b, int j, int64_t dst) {
        const int64_t src = append_source_row(a, b, j);
        AUDIT(src >= 0 && src < static_cast<int64_t>(ap.batch) * ap.tokens, "source row %" PRId64, src);
        for (int t = 0; t < 256; ++t)
            for (uint32_t c = static_cast<uint32_t>(t); c < chunks; c += 256) {
                const int64_t so = append_chunk_offset(a, src, c), d = append_chunk_offset(a, dst, c);
                AUDIT(so >= 0 && so + 16 <= new_bytes, "new-token read at %" PRId64, so);
                AUDIT(d >= 0 && d + 16 <= cache_bytes, "cache write at %" PRId64, d);
            }
        if (dst >= 0 && static_cast<size_t>(dst) < row_writes.size()) ++row_writes[dst];
        ++written;
    };
    for (int b = 0; b < ap.batch; ++b) {
        if (ap.advance) {  // workgroup b
            const int64_t base = ap.starts[b];
            bool fits = true;
            for (int j = 0; j < ap.tokens; ++j) fits &= row_of(b, base + j) >= 0;
            if (fits)
                for (int j = 0; j < ap.tokens; ++j) copy(b, j, row_of(b, base + j));
        } else {  // workgroups (j, b)
            for (int j = 0; j < ap.tokens; ++j) {
                const int64_t dst = row_of(b, static_cast<int64_t>(ap.starts[b]) + j);
                if (dst >= 0) copy(b, j, dst);
            }
        }
    }
    std::printf("%-44s %s %d tokens x %d sequences, %d rows written, %" PRIu64 " checks: %s\n", ap.name.c_str(),
                ap.advance ? "append+advance" : "append", ap.tokens, ap.batch, written, g_checks - checks_before,
                g_failures == before ? "ok" : "FAILED");
    std::fflush(stdout);
    return g_failures == before;
}

// CSR page lists -> page table (cache_map.h; decode.hip: table_from_csr_kernel,
// grid batch x 256 threads). Every indptr, last-page-length and indices read
// and every table and lengths write is checked against its buffer.
struct CsrProblem {
    std::string name;
    int batch, width, page_size, max_context;
    std::vector<int32_t> indptr, indices, last;
};

bool audit_csr(const CsrProblem& cp) {
    const int before = g_failures;
    const uint64_t checks_before = g_checks;
    CsrParams c{};
    c.indices_count = g_plant_csr_count ? (int64_t{1} << 40) : static_cast<int64_t>(cp.indices.size());
    c.table_width = cp.width;
    c.page_size = cp.page_size;
    c.max_context = cp.max_context;
    std::vector<uint8_t> table_writes(static_cast<size_t>(cp.batch) * cp.width, 0);
    int rejected = 0;
    for (int b = 0; b < cp.batch; ++b) {
        AUDIT(b + 1 < static_cast<int>(cp.indptr.size()), "indptr read %d", b + 1);
        const int64_t begin = cp.indptr[b], end = cp.indptr[b + 1];
        int last = 0;
        if (end > begin) {
            AUDIT(b < static_cast<int>(cp.last.size()), "last_page_len read %d", b);
            last = cp.last[b];
        }
        const CsrRow r = csr_row(c, begin, end, last);
        rejected += r.fits ? 0 : 1;
        for (int t = 0; t < 256; ++t)
            for (int i = t; i < cp.width; i += 256) {
                const int64_t e = static_cast<int64_t>(b) * cp.width + i;
                AUDIT(e < static_cast<int64_t>(table_writes.size()), "table write %" PRId64, e);
                if (e < static_cast<int64_t>(table_writes.size())) ++table_writes[e];
                if (i < r.live)
                    AUDIT(r.begin + i >= 0 && r.begin + i < static_cast<int64_t>(cp.indices.size()),
                          "indices read %" PRId64 " of %zu", r.begin + i, cp.indices.size());
            }
        if (r.fits) AUDIT(r.length <= cp.max_context && r.live <= cp.width, "row %d length %" PRId64, b, r.length);
    }
    for (size_t e = 0; e < table_writes.size(); ++e)
        AUDIT(table_writes[e] == 1, "table entry %zu written %d times", e, table_writes[e]);
    std::printf("%-44s csr -> table, %d of %d rows rejected, %" PRIu64 " checks: %s\n", cp.name.c_str(), rejected,
                cp.batch, g_checks - checks_before, g_failures == before ? "ok" : "FAILED");
    std::fflush(stdout);
    return g_failures == before;
}

// Deterministic generator for tables and lengths.
struct Lcg {
    uint64_t s;
    uint32_t next() {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        return static_cast<uint32_t>(s >> 33);
    }
    int below(int n) { return static_cast<int>(next() % static_cast<uint32_t>(n)); }
};

// Problem with shuffled pages, `width` logical pages per sequence and the
// given lengths; splits cover `reserve` times the longest sequence.
Problem make(const std::string& name, int batch, int q_heads, int kv_heads, int head_dim, int page_size, int width,
             std::vector<int32_t> lengths, int split_tokens, int q_elem, int kv_elem, uint64_t seed,
             int reserve = 1) {
    Problem pr;
    pr.name = name;
    pr.batch = batch;
    pr.q_heads = q_heads;
    pr.kv_heads = kv_heads;
    pr.head_dim = head_dim;
    pr.page_size = page_size;
    pr.width = width;
    pr.pages = batch * width;
    pr.q_elem = q_elem;
    pr.kv_elem = kv_elem;
    pr.split_tokens = split_tokens;
    pr.caller_split_tokens = split_tokens;
    pr.lengths = lengths;
    int longest = 0;
    for (int v : lengths) longest = imax(longest, v);
    const int capacity = width * page_size;
    const int reserved = imin(capacity, imax(1, longest) * reserve);
    pr.splits = imax(1, (reserved + split_tokens - 1) / split_tokens);
    pr.caller_splits = pr.splits;
    std::vector<int32_t> perm(pr.pages);
    for (int i = 0; i < pr.pages; ++i) perm[i] = i;
    Lcg rng{seed};
    for (int i = pr.pages - 1; i > 0; --i) std::swap(perm[i], perm[rng.below(i + 1)]);
    pr.table.assign(static_cast<size_t>(batch) * width, -1);
    for (int b = 0; b < batch; ++b)
        for (int i = 0; i < width; ++i) pr.table[static_cast<size_t>(b) * width + i] = perm[b * width + i];
    return pr;
}

std::vector<int32_t> uniform(int batch, int len) { return std::vector<int32_t>(batch, len); }

std::vector<int32_t> ragged(int batch, int hi, uint64_t seed) {
    Lcg rng{seed};
    std::vector<int32_t> v(batch);
    for (auto& x : v) x = rng.below(hi + 1);
    v[0] = hi;
    if (batch > 2) v[1] = 0;
    return v;
}

// Sequences [first, last) of pr map the first `pages` logical pages of
// sequence `from` (a shared prefix).
void share_prefix(Problem& pr, int from, int first, int last, int pages) {
    for (int b = first; b < last; ++b)
        for (int i = 0; i < pages; ++i)
            pr.table[static_cast<size_t>(b) * pr.width + i] = pr.table[static_cast<size_t>(from) * pr.width + i];
    pr.unshared = false;
}

// The problem with shared-prefix runs taken from its own table (pd_prefix_runs).
Problem with_runs(Problem pr) {
    pr.name += " prefix runs";
    pr.runs.assign(2 * static_cast<size_t>(pr.batch), 0);
    prefix_runs_of_table(pr.table.data(), pr.batch, pr.width, pr.runs.data());
    return pr;
}

// Runs that claim each sequence's whole row in common with its leader: the
// description of a table the device no longer holds (a plan refreshed after
// a graph captured it). Items then reach past the shared pages.
Problem with_stale_runs(Problem pr) {
    pr = with_runs(pr);
    pr.name += " stale";
    for (int b = 0; b < pr.batch; ++b)
        if (pr.runs[2 * b] >= 0) pr.runs[2 * b + 1] = pr.width;
    return pr;
}

// The same problem with host bounds: exact lengths, half, zero, or none.
std::vector<Problem> with_bounds(const Problem& base) {
    std::vector<Problem> out{base};
    const char* kinds[] = {"exact", "half", "zero"};
    for (int k = 0; k < 3; ++k) {
        Problem pr = base;
        pr.name += std::string(" bounds=") + kinds[k];
        pr.bounds = base.lengths;
        for (auto& x : pr.bounds) x = k == 0 ? x : k == 1 ? x / 2 : 0;
        out.push_back(pr);
    }
    return out;
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "";
    const bool quick = mode == "--quick";
    std::vector<Problem> problems;
    auto add = [&](const Problem& pr, bool bounds = true) {
        if (bounds) for (const auto& x : with_bounds(pr)) problems.push_back(x);
        else problems.push_back(pr);
    };
    // The five measured workloads (FP32 oracle case; Llama-3-8B FP16 and FP8;
    // ragged + shared pages; MQA; long-context MHA over its split sweep).
    add(make("fp32 B2 Hq8/2 D64 L[100,256] split 256", 2, 8, 2, 64, 16, 16, {100, 256}, 256, 4, 4, 1));
    add(make("fp32 B2 Hq8/2 D64 L[100,256] split 32", 2, 8, 2, 64, 16, 16, {100, 256}, 32, 4, 4, 1));
    add(make("llama3-8b B4 L4096 fp16", 4, 32, 8, 128, 16, 256, uniform(4, 4096), 256, 2, 2, 2));
    add(make("llama3-8b B4 L4096 fp8", 4, 32, 8, 128, 16, 256, uniform(4, 4096), 256, 2, 1, 2));
    {
        Problem pr = make("ragged shared B16 T32 split 128", 16, 32, 8, 128, 32, 256, ragged(16, 8192, 3), 128, 2, 2, 3);
        for (int b = 1; b < 16; ++b)  // a 25% shared prefix: the first 64 pages of sequence 0
            for (int i = 0; i < 64; ++i) pr.table[static_cast<size_t>(b) * 256 + i] = pr.table[i];
        pr.unshared = false;
        pr.ragged = true;
        add(pr);
        add(with_runs(pr));
        Problem fp8 = pr;
        fp8.name = "ragged shared B16 T32 split 128 fp8";
        fp8.kv_elem = 1;
        add(with_runs(fp8));
        Problem reserved = make("ragged B16 T32 split 128 reserve x4", 16, 32, 8, 128, 32, 1024, ragged(16, 8192, 3),
                                128, 2, 2, 3, 4);
        add(reserved);
    }
    // Shared prefixes of other tile widths, several sharing classes, and more
    // items than kMaxGroupItems (each with runs from its table).
    {
        // MHA: 16 members per item. 24 sequences share 32 pages of sequence 0.
        std::vector<int32_t> lens(24);
        Lcg rng{601};
        for (auto& x : lens) x = 520 + rng.below(1000);
        lens[0] = 4096;
        Problem mha = make("prefix mha B24 Hq8/8 D64 T16 split 64", 24, 8, 8, 64, 16, 256, lens, 64, 2, 2, 601);
        share_prefix(mha, 0, 1, 24, 32);
        add(with_runs(mha));
        add(with_stale_runs(mha));
        // Rows padded with -1 past each length, as plans and workloads hold
        // them: a short member's run ends at its last page, and items still
        // read every member's pages from the leader's row (no own passes).
        Problem padded = mha;
        padded.name = "prefix padded rows B24 Hq8/8 D64 T16 split 64";
        for (int b = 0; b < padded.batch; ++b)
            for (int i = (padded.lengths[b] + 15) / 16; i < padded.width; ++i)
                padded.table[static_cast<size_t>(b) * padded.width + i] = -1;
        add(with_runs(padded));
        Problem padded4 = make("prefix padded rows B32 Hq32/8 D128 T16 split 256", 32, 32, 8, 128, 16, 256, [] {
            std::vector<int32_t> v(32);
            Lcg r{611};
            for (auto& x : v) x = r.below(2049);
            v[0] = 4096;
            return v;
        }(), 256, 2, 2, 611);
        share_prefix(padded4, 0, 1, 32, 64);
        for (int b = 0; b < padded4.batch; ++b)
            for (int i = (padded4.lengths[b] + 15) / 16; i < padded4.width; ++i)
                padded4.table[static_cast<size_t>(b) * padded4.width + i] = -1;
        add(with_runs(padded4));
        // GQA 8 (Hq16/Hkv2): 2 members per item.
        Problem gqa8 = make("prefix gqa8 B6 Hq16/2 D128 T16 split 64", 6, 16, 2, 128, 16, 128,
                            {2048, 400, 700, 300, 650, 520}, 64, 2, 2, 603);
        share_prefix(gqa8, 0, 1, 6, 16);
        add(with_runs(gqa8));
        // Two classes; one member diverges early, one shares more than the rest.
        std::vector<int32_t> two(16);
        for (int b = 0; b < 16; ++b) two[b] = 600 + 97 * b;
        two[0] = 8192;
        Problem classes = make("prefix two classes B16 Hq32/8 D128 T32 split 128", 16, 32, 8, 128, 32, 256, two, 128,
                               2, 2, 605);
        share_prefix(classes, 0, 1, 8, 48);
        share_prefix(classes, 8, 9, 16, 24);
        share_prefix(classes, 8, 12, 13, 40);
        for (int i = 10; i < 48; ++i) classes.table[3 * 256 + i] = classes.table[15 * 256 + 200 + i];
        add(with_runs(classes));
        add(with_stale_runs(classes));
        // Members shorter on the device than their host bounds: a length of
        // 0, one inside a shared partition, one at a partition boundary, and
        // a shorter first member (whose row the items read).
        Problem shrunk = with_runs(classes);
        shrunk.name += " lengths below bounds";
        shrunk.bounds = classes.lengths;
        shrunk.lengths[1] = 0;
        shrunk.lengths[2] = 300;
        shrunk.lengths[4] = 512;
        shrunk.lengths[9] = 1000;
        shrunk.lengths[0] = 700;
        add(shrunk, false);
        // 64 sequences sharing 40 partitions of 16 tokens: 160 items before the cap.
        std::vector<int32_t> many(64);
        Lcg rng2{607};
        for (auto& x : many) x = 700 + rng2.below(700);
        many[0] = 4096;
        Problem cap = make("prefix cap B64 Hq8/8 D64 T16 split 16", 64, 8, 8, 64, 16, 256, many, 16, 2, 2, 607);
        share_prefix(cap, 0, 1, 64, 40);
        add(with_runs(cap));
        // Equal lengths (a rectangular grid) with a shared prompt: several
        // samples of one prompt. The grid becomes a work list when the items
        // remove enough of it (prefer_work_list_for_prefixes).
        Problem samples = make("prefix samples B16 Hq32/8 D128 T16 L4096 split 256", 16, 32, 8, 128, 16, 256,
                               uniform(16, 4096), 256, 2, 2, 613);
        share_prefix(samples, 0, 1, 16, 128);
        add(with_runs(samples));
        Problem few = make("prefix samples B8 Hq32/8 D128 T16 L4096 split 256 6% shared", 8, 32, 8, 128, 16, 256,
                           uniform(8, 4096), 256, 2, 2, 617);
        share_prefix(few, 0, 1, 8, 16);
        add(with_runs(few));
        // FP32 inputs take no shared-prefix items.
        Problem f32 = make("prefix fp32 B24 Hq8/8 D64 T16 split 64", 24, 8, 8, 64, 16, 256, lens, 64, 4, 4, 601);
        share_prefix(f32, 0, 1, 24, 32);
        add(with_runs(f32));
    }
    add(make("mqa B128 Hq16/1 D64 L1024", 128, 16, 1, 64, 16, 64, uniform(128, 1024), 256, 2, 2, 4), false);
    add(make("mqa B64 Hq16/1 D64 ragged split 64", 64, 16, 1, 64, 16, 64, ragged(64, 1024, 41), 64, 2, 2, 41));
    for (int split : {128, 256, 512, 1024})
        add(make("long mha B1 Hq32/32 L32768 split " + std::to_string(split), 1, 32, 32, 128, 16, 2048,
                 uniform(1, 32768), split, 2, 2, 5),
            !quick && split == 128);
    // XCD-grouped grids (plan_xcd) under exact bounds, the shapes of
    // tests/test_gpu_xcd_grid.py: both merge kernels' row maps are walked too.
    add(make("xcd gqa4 B8 Hq32/8 D128 L1024 split 128 fp16", 8, 32, 8, 128, 16, 64, uniform(8, 1024), 128, 2, 2, 71));
    add(make("xcd gqa4 B8 Hq32/8 D128 L1024 split 128 fp8", 8, 32, 8, 128, 16, 64, uniform(8, 1024), 128, 2, 1, 71));
    add(make("xcd mqa B64 Hq16/1 D64 L1024 split 256 fp16", 64, 16, 1, 64, 16, 64, uniform(64, 1024), 256, 2, 2, 73));
    add(make("xcd mha B2 Hq16/16 D128 L2048 split 256 fp16", 2, 16, 16, 128, 16, 128, uniform(2, 2048), 256, 2, 2, 75));
    add(make("xcd fp32 B8 Hq16/8 D64 L1024 split 128", 8, 16, 8, 64, 16, 64, uniform(8, 1024), 128, 4, 4, 77));
    // Eight head groups per sequence: the plain grids (rectangular, with
    // tails, or a work list) already keep a row group on one XCD, and only
    // the merge is XCD-grouped, whatever the lengths.
    add(make("xcd merge ragged mha B16 Hq32/32 D128 split 128", 16, 32, 32, 128, 16, 64, ragged(16, 1024, 83), 128, 2,
             2, 83));
    // Seeded random problems (small sizes), each with every kind of bounds:
    // batch sizes and head layouts that do and do not make the XCD-grouped
    // grids, uniform and ragged lengths, reserved context, both page sizes,
    // head dimensions and element sizes.
    {
        Lcg rng{2026};
        const int kv_choices[] = {1, 2, 4, 8, 16, 32};
        const int group_choices[] = {1, 2, 3, 4, 8, 16};
        const int batch_choices[] = {1, 2, 3, 4, 6, 8, 12, 16};
        const int split_choices[] = {16, 32, 64, 128, 256};
        for (int i = 0; i < (quick ? 8 : 40); ++i) {
            const int kv = kv_choices[rng.below(6)];
            const int group = group_choices[rng.below(6)];
            const int batch = batch_choices[rng.below(8)];
            const int dim = rng.below(2) ? 128 : 64;
            const int page = rng.below(2) ? 32 : 16;
            const int split = split_choices[rng.below(5)];
            const int len = 1 + rng.below(1024);
            const bool uni = rng.below(2) != 0;
            const int reserve = 1 + rng.below(2);
            const int elems = rng.below(3);  // 0: FP16, 1: FP8 K/V, 2: FP32
            const int q_elem = elems == 2 ? 4 : 2, kv_elem = elems == 0 ? 2 : elems == 1 ? 1 : 4;
            const int width = (len * reserve + page - 1) / page;
            const std::string name = "random " + std::to_string(i) + " B" + std::to_string(batch) + " Hq" +
                                     std::to_string(kv * group) + "/" + std::to_string(kv) + " D" +
                                     std::to_string(dim) + " T" + std::to_string(page) + (uni ? " L" : " ragged L") +
                                     std::to_string(len) + " x" + std::to_string(reserve) + " split " +
                                     std::to_string(split) + (elems == 2 ? " fp32" : elems == 1 ? " fp8" : " fp16");
            add(make(name, batch, kv * group, kv, dim, page, width,
                     uni ? uniform(batch, len) : ragged(batch, len, 100 + i), split, q_elem, kv_elem, 100 + i,
                     reserve));
        }
    }
    // Seeded random shared-prefix problems: head layouts that form items
    // (GQA groups up to 8, MHA) and one that does not (GQA 3 pads to 4),
    // one to three sharing classes with random leaders, members and shared
    // page counts, some members diverging earlier, rows padded past their
    // lengths or not, uniform, ragged or skewed lengths, FP16 or FP8 K/V;
    // runs taken from the table (every kind of bounds), and for every fourth
    // problem stale runs as well.
    {
        Lcg rng{3031};
        const int kv_choices[] = {1, 2, 4, 8};
        const int group_choices[] = {1, 2, 3, 4, 8};
        const int batch_choices[] = {2, 3, 5, 8, 12, 16, 24, 33};
        const int split_choices[] = {16, 32, 64, 128, 256};
        for (int i = 0; i < (quick ? 4 : 24); ++i) {
            const int kv = kv_choices[rng.below(4)];
            const int group = group_choices[rng.below(5)];
            const int batch = batch_choices[rng.below(8)];
            const int dim = rng.below(2) ? 128 : 64;
            const int page = rng.below(2) ? 32 : 16;
            const int split = split_choices[rng.below(5)];
            const int len = 64 + rng.below(2048);
            const int kind = rng.below(3);  // 0: uniform, 1: ragged, 2: skewed (one at len, the rest up to len / 2)
            const bool fp8 = rng.below(3) == 0;
            const bool pad = rng.below(2) != 0;
            const int width = (len + page - 1) / page;
            std::vector<int32_t> lens = kind == 0 ? uniform(batch, len) : ragged(batch, len, 300 + i);
            if (kind == 2)
                for (int b = 1; b < batch; ++b) lens[b] = rng.below(len / 2 + 1);
            const std::string name = "prefix random " + std::to_string(i) + " B" + std::to_string(batch) + " Hq" +
                                     std::to_string(kv * group) + "/" + std::to_string(kv) + " D" +
                                     std::to_string(dim) + " T" + std::to_string(page) +
                                     (kind == 0 ? " L" : kind == 1 ? " ragged L" : " skewed L") +
                                     std::to_string(len) + " split " + std::to_string(split) +
                                     (fp8 ? " fp8" : " fp16") + (pad ? " padded" : "");
            Problem pr = make(name, batch, kv * group, kv, dim, page, width, lens, split, 2, fp8 ? 1 : 2, 300 + i);
            const int classes = 1 + rng.below(3);
            for (int c = 0; c < classes; ++c) {
                const int leader = rng.below(batch);
                const int pages = 1 + rng.below(width);
                for (int b = 0; b < batch; ++b) {
                    if (b == leader || rng.below(3) == 0) continue;  // about two rows in three join
                    const int mine = rng.below(4) == 0 ? rng.below(pages + 1) : pages;
                    for (int e = 0; e < mine; ++e)
                        pr.table[static_cast<size_t>(b) * width + e] = pr.table[static_cast<size_t>(leader) * width + e];
                }
            }
            if (pad)
                for (int b = 0; b < batch; ++b)
                    for (int e = (lens[b] + page - 1) / page; e < width; ++e)
                        pr.table[static_cast<size_t>(b) * width + e] = -1;
            pr.unshared = false;
            pr.ragged = kind != 0;
            add(with_runs(pr));
            if (i % 4 == 0) add(with_stale_runs(pr));
        }
    }
    // Reserved context over uniform lengths: tail rows, partly empty slots.
    add(make("xcd llama3-8b B4 L4096 reserve x4", 4, 32, 8, 128, 16, 1024, uniform(4, 4096), 256, 2, 2, 79, 4));
    add(make("xcd mqa B128 Hq16/1 D64 L1024 reserve x2", 128, 16, 1, 64, 16, 128, uniform(128, 1024), 256, 2, 2, 81,
             2));
    // Device lengths past the caller's partitions (splits * split_tokens <
    // length <= table capacity): a full call over coarser partitions must
    // still read only the first splits * split_tokens tokens. B64, 3
    // partitions of 256 tokens, lengths 1000 in a 1024-token table: the
    // coarse split is 2 x 512, whose second partition would reach token 999.
    {
        Problem pr = make("past reach B64 Hq32/8 D128 splits 3x256 L1000", 64, 32, 8, 128, 16, 64, uniform(64, 1000),
                          256, 2, 2, 19);
        pr.splits = pr.caller_splits = 3;
        add(pr);
        Problem ragged_past = make("past reach B16 Hq8/2 D64 splits 5x64 ragged", 16, 8, 2, 64, 16, 32,
                                   ragged(16, 512, 23), 64, 2, 2, 23);
        ragged_past.splits = ragged_past.caller_splits = 5;
        add(ragged_past);
        Problem fp8_past = make("past reach B32 Hq16/4 D128 fp8 splits 6x128 L900", 32, 16, 4, 128, 32, 32,
                                uniform(32, 900), 128, 2, 1, 29);
        fp8_past.splits = fp8_past.caller_splits = 6;
        add(fp8_past);
    }
    // Edge lengths around page and partition boundaries, both page sizes.
    for (int page : {16, 32}) {
        add(make("edges fp16 page " + std::to_string(page), 8, 8, 2, 128, page, 8,
                 {0, 1, page - 1, page, page + 1, 2 * page - 1, 2 * page + 1, 8 * page}, 33, 2, 2, 7));
        add(make("edges fp32 page " + std::to_string(page), 8, 8, 2, 64, page, 8,
                 {0, 1, page - 1, page, page + 1, 2 * page - 1, 2 * page + 1, 8 * page}, 1, 4, 4, 7));
    }
    // Invalid page ids inside live ranges (parked loads) and lengths beyond
    // the table (clamped).
    {
        Problem pr = make("invalid page ids fp16", 4, 16, 4, 128, 16, 16, {256, 200, 300, 17}, 64, 2, 2, 9);
        pr.table[3] = -1;
        pr.table[16 + 5] = pr.pages;
        pr.table[32 + 0] = 2147483647;
        pr.table[48 + 1] = -2147483647 - 1;
        add(pr);
        Problem f = make("invalid page ids fp32", 4, 16, 4, 64, 16, 16, {256, 200, 300, 17}, 64, 4, 4, 9);
        f.table = pr.table;
        add(f);
        Problem e8 = make("invalid page ids fp8", 4, 16, 4, 64, 16, 16, {256, 200, 300, 17}, 64, 2, 1, 9);
        e8.table = pr.table;
        add(e8);
    }
    // Uncommon head layouts (partial and multiple head tiles, odd workgroups).
    for (auto hk : std::vector<std::pair<int, int>>{{12, 4}, {20, 4}, {48, 2}, {96, 4}, {21, 3}, {35, 5}, {42, 7},
                                                    {66, 11}, {80, 20}, {72, 12}, {24, 1}}) {
        add(make("heads " + std::to_string(hk.first) + "/" + std::to_string(hk.second) + " fp16", 3, hk.first,
                 hk.second, 128, 16, 12, {192, 77, 150}, 64, 2, 2, 11),
            false);
        add(make("heads " + std::to_string(hk.first) + "/" + std::to_string(hk.second) + " fp32", 3, hk.first,
                 hk.second, 64, 16, 12, {192, 77, 150}, 64, 4, 4, 11),
            false);
    }
    // Whole-row launches (a full decode call of at most four partitions per
    // row): ragged lengths with empty rows and partial partitions, GQA and
    // MQA tiles, both head dimensions, FP8 K/V, page 32, a single partition
    // per row, invalid page ids.
    add(make("rows mqa B128 D64 ragged split 256", 128, 16, 1, 64, 16, 64, ragged(128, 1024, 51), 256, 2, 2, 51),
        false);
    add(make("rows B64 Hq32/8 D128 ragged split 192", 64, 32, 8, 128, 16, 32, ragged(64, 512, 53), 192, 2, 2, 53),
        false);
    add(make("rows B64 Hq32/8 D128 fp8 split 192", 64, 32, 8, 128, 32, 16, ragged(64, 512, 55), 192, 2, 1, 55),
        false);
    add(make("rows B2 Hq8/2 D64 L[100,256] split 256", 2, 8, 2, 64, 16, 16, {100, 256}, 256, 2, 2, 57), false);
    add(make("rows B3 Hq20/4 D128 split 512 page 32", 3, 20, 4, 128, 32, 16, {512, 1, 0}, 512, 2, 2, 59), false);
    {
        Problem pr = make("rows invalid page ids B32 Hq16/4 split 64", 32, 16, 4, 64, 16, 16, ragged(32, 256, 61), 64,
                          2, 2, 61);
        pr.table[3] = -1;
        pr.table[16 + 5] = pr.pages;
        pr.table[32 + 0] = 2147483647;
        add(pr, false);
    }
    if (!quick) {
        // A 1M-token context in a 65536-wide table (16384 states per row).
        add(make("1M context W65536 fp16", 1, 8, 2, 128, 16, 65536, uniform(1, 1 << 20), 256, 2, 2, 13), false);
        // Live pages above 4 GiB of cache (64-bit page offsets).
        Problem big = make("pages above 4 GiB", 2, 32, 8, 128, 16, 64, {1024, 700}, 128, 2, 2, 17);
        big.pages = 163840;  // 5 GiB per K/V tensor at 32 KB per page
        for (int i = 0; i < 128; ++i) big.table[i] = 163840 - 1 - i;
        add(big);
    }
    // KV-cache appends: explicit positions inside, at and past the table's end
    // and negative; invalid page ids (-1, physical_pages, INT_MAX); several
    // tokens per sequence; both page sizes; FP8, 16-bit and FP32 rows of D 64
    // and 128; the advance variant below, at and past max_context.
    std::vector<AppendProblem> appends;
    {
        Lcg rng{909};
        for (int i = 0; i < (quick ? 6 : 32); ++i) {
            AppendProblem ap;
            ap.batch = 1 + rng.below(8);
            ap.tokens = 1 + rng.below(40);
            ap.kv_heads = 1 << rng.below(4);
            ap.head_dim = rng.below(2) ? 128 : 64;
            ap.elem = 1 << rng.below(3);
            ap.page_size = rng.below(2) ? 32 : 16;
            ap.width = 1 + rng.below(12);
            ap.pages = ap.batch * ap.width + rng.below(3);
            ap.advance = rng.below(2) != 0;
            const int cap = ap.width * ap.page_size;
            ap.max_context = rng.below(cap + 1);
            ap.table.resize(static_cast<size_t>(ap.batch) * ap.width);
            for (auto& id : ap.table) id = rng.below(ap.pages);
            const int32_t invalid[] = {-1, ap.pages, 2147483647};
            for (int k = 0; k < 3; ++k) ap.table[rng.below(static_cast<int>(ap.table.size()))] = invalid[k];
            ap.starts.resize(ap.batch);
            for (auto& st : ap.starts) st = rng.below(cap + 12) - 6;
            ap.starts[0] = cap - ap.tokens;  // exactly up to the table's end
            ap.name = "append " + std::to_string(i) + (ap.advance ? " advance" : " positions") + " B" +
                      std::to_string(ap.batch) + " n" + std::to_string(ap.tokens) + " T" + std::to_string(ap.page_size) +
                      " W" + std::to_string(ap.width) + " row " + std::to_string(ap.kv_heads * ap.head_dim * ap.elem);
            appends.push_back(ap);
        }
        AppendProblem end{"append at the table's end", 2, 4, 8, 128, 2, 16, 4, 8, 64, {}, {60, 61}, false};
        end.table = {0, 1, 2, 3, 4, 5, 6, 7};
        appends.push_back(end);
    }
    // CSR page lists: valid lists (empty rows included), lists longer than
    // the table, last-page lengths outside [1, T], lengths past max_context,
    // negative counts, and lists reaching before or past the indices tensor.
    std::vector<CsrProblem> csrs;
    {
        Lcg rng{4242};
        for (int i = 0; i < (quick ? 6 : 32); ++i) {
            CsrProblem cp;
            cp.batch = 1 + rng.below(10);
            cp.width = 1 + rng.below(300);
            cp.page_size = rng.below(2) ? 32 : 16;
            cp.max_context = rng.below(cp.width * cp.page_size + 1);
            cp.indptr.assign(1, 0);
            for (int b = 0; b < cp.batch; ++b) cp.indptr.push_back(cp.indptr.back() + rng.below(cp.width + 3));
            cp.indices.resize(cp.indptr.back());
            for (auto& x : cp.indices) x = rng.below(1000);
            cp.last.resize(cp.batch);
            for (auto& l : cp.last) l = rng.below(cp.page_size + 2);  // 0 and T + 1 are invalid
            const int kind = rng.below(4);  // 0: as drawn; 1: a negative count; 2: past the end; 3: before the start
            const int b = rng.below(cp.batch);
            if (kind == 1) cp.indptr[b + 1] = cp.indptr[b] - 1;
            if (kind == 2) cp.indptr[b + 1] = static_cast<int32_t>(cp.indices.size()) + 1 + rng.below(5);
            if (kind == 3) cp.indptr[b] = -1 - rng.below(5);
            cp.name = "csr " + std::to_string(i) + " B" + std::to_string(cp.batch) + " W" + std::to_string(cp.width) +
                      " T" + std::to_string(cp.page_size) + (kind == 1 ? " negative count" : kind == 2 ? " past end"
                                                             : kind == 3 ? " before start" : "");
            csrs.push_back(cp);
        }
        // A list that meets every other rule but reaches past the indices
        // tensor (5 pages from entry 4 of 6): only the indices bound rejects it.
        csrs.push_back(CsrProblem{"csr list past the indices end", 2, 8, 16, 128, {0, 4, 9}, {0, 1, 2, 3, 4, 5}, {16, 16}});
    }
    if (mode == "--plant-merge-live" || mode == "--plant-append" || mode == "--plant-csr") {
        // Negative controls: merge params that count one partition too many
        // as live, an append capacity one page past the table, a CSR
        // conversion without its indices bound. Each walk must report it.
        g_plant_merge_live = mode == "--plant-merge-live";
        g_plant_append_capacity = mode == "--plant-append";
        g_plant_csr_count = mode == "--plant-csr";
        std::vector<Problem> kept;
        if (g_plant_merge_live)
            for (const auto& pr : problems)
                if (pr.name.rfind("llama3-8b B4 L4096 fp16", 0) == 0 || pr.name.rfind("edges fp16", 0) == 0)
                    kept.push_back(pr);
        problems = kept;
        if (!g_plant_append_capacity) appends.clear();
        if (!g_plant_csr_count) csrs.clear();
    }
    if (mode == "--plant-prefix") {
        // Negative control: the stale-runs problems walked as a kernel
        // without the page check would run them (every member in the shared
        // pass). The walk must report members reading pages they do not map.
        g_plant_no_check = true;
        std::vector<Problem> planted;
        for (const auto& pr : problems)
            if (pr.name.find(" prefix runs stale") != std::string::npos) planted.push_back(pr);
        problems = planted;
        appends.clear();
        csrs.clear();
    }
    if (mode == "--plant-reach") {
        // Negative control: the same problems with launch params that clamp
        // lengths to the table only. The walk must report reads past the
        // caller's partitions.
        g_plant_reach = true;
        std::vector<Problem> planted;
        for (const auto& pr : problems)
            if (pr.name.rfind("past reach", 0) == 0) planted.push_back(pr);
        problems = planted;
    }
    int failed = 0;
    for (const auto& pr : problems) {
        // The staged entries: the partition launch, then pd_decode_merge over
        // every state slot it left.
        PartialParams stage;
        Coverage stage_cov;
        failed += audit(pr, false, stage, stage_cov) ? 0 : 1;
        failed += audit_merges(pr, stage, stage_cov, false) ? 0 : 1;
        // The full decode call: over coarser partitions (fewer of them,
        // covering at least the caller's, their states inside the caller's
        // workspace: the audited buffers are those of the coarser split, a
        // prefix), or one whole-row launch, or the staged partition launch
        // with the full call's merge.
        const KernelSplit ks = full_call_split(pr.q_elem == 4, pr.kv_elem, pr.batch, pr.q_heads, pr.kv_heads,
                                               pr.head_dim, pr.page_size, pr.width, pr.splits, pr.split_tokens,
                                               pr.bounds.empty() ? nullptr : pr.bounds.data(), 256,
                                               pr.runs.empty() ? nullptr : pr.runs.data());
        Problem call = pr;
        const bool coarse = ks.splits != pr.splits || ks.split_tokens != pr.split_tokens;
        if (coarse) {
            AUDIT(ks.splits < pr.splits && ks.split_tokens % pr.split_tokens == 0 &&
                      static_cast<int64_t>(ks.splits) * ks.split_tokens >=
                          static_cast<int64_t>(pr.splits) * pr.split_tokens,
                  "coarse split %d x %d for %d x %d", ks.splits, ks.split_tokens, pr.splits, pr.split_tokens);
            call.name += " coarse x" + std::to_string(ks.split_tokens / pr.split_tokens);
            call.splits = ks.splits;
            call.split_tokens = ks.split_tokens;
        }
        const PartialParams planned = params(call, 256, call.q_elem == 2, true);
        const bool same_launch = !coarse && !planned.row_mode && planned.grid_x == stage.grid_x &&
                                 planned.grid_y == stage.grid_y && planned.combine == stage.combine &&
                                 planned.quarters_per_wg == stage.quarters_per_wg &&
                                 planned.heads_per_wg == stage.heads_per_wg && planned.xcd_shift == stage.xcd_shift;
        if (same_launch) {
            failed += audit_merges(call, planned, stage_cov, true) ? 0 : 1;
        } else {
            PartialParams p;
            Coverage cov;
            failed += audit(call, true, p, cov) ? 0 : 1;
            if (!p.row_mode) failed += audit_merges(call, p, cov, true) ? 0 : 1;
        }
    }
    for (const auto& ap : appends) failed += audit_append(ap) ? 0 : 1;
    for (const auto& cp : csrs) failed += audit_csr(cp) ? 0 : 1;
    std::printf("%zu problems, %" PRIu64 " merge launches, %zu appends, %zu csr conversions, %" PRIu64
                " shared-prefix own passes, %" PRIu64 " checks, %d failures\n", problems.size(), g_merge_launches,
                appends.size(), csrs.size(), g_own_passes, g_checks, g_failures);
    return failed == 0 ? 0 : 1;
}
