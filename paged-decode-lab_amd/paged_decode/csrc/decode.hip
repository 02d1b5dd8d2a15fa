// Split-K paged GQA decode attention for gfx950 (AMD Instinct MI355X), and the
// paged KV-cache append that feeds it.
//
// Implements the C ABI declared in include/paged_decode.h. pd_decode makes two
// launches per call, both on the caller's stream. This unit holds the entry
// points, the merge, append and CSR kernels; the partition kernels are
// templates in partition_kernels.h, instantiated per q format and head
// dimension in the partial_*.hip units, with their work and address map in
// partition_map.h (shared with a host audit of every access).
//
//  1. Partition kernel. Each partition of split_tokens tokens is cut into four
//     quarters, and each (quarter, KV head, head tile) is one wave's work: it
//     reads that KV head's K and V rows of the quarter from HBM exactly once,
//     uses them for every query head of the tile (the GQA group, padded to
//     GT = 1/2/4/8/16 heads), and stores one (m, l, n[D]) state per query head
//     in slot 4 * partition + quarter of the workspace. A workgroup gathers up
//     to four KV heads (eight in the FP32 kernel) of the same tokens (their
//     head slices of a token row are then read together) plus enough quarters
//     to make eight waves, or fewer waves when eight-wave workgroups would
//     leave most CUs idle. Waves
//     do not synchronise while they stream; where a workgroup holds several
//     quarters of one partition (few KV heads), one barrier at the end lets
//     the first quarter fold the others into a single state. Partitions that
//     start at or past their sequence's end exit before any load and write
//     nothing. With host length bounds the grid holds only the partitions the
//     bounds reach, then a few tail workgroups for lengths that grew past
//     them on the device.
//       partial_mfma_kernel (q in FP16 or BF16; K/V in the same type or in
//       OCP FP8): 16-token tiles; q.K^T and P.V on the matrix cores, online
//       softmax with one running max per head and lazy rescaling (the
//       accumulators are rescaled only when a tile's max exceeds the running
//       max by 2^8); each lane ends with its own slice of the state and
//       stores it directly.
//       partial_kernel (FP32): the same decomposition on the vector ALU;
//       q.k is reduced over each token row's lanes with DPP, every token row
//       keeps its own online-softmax stream, and the rows' streams are
//       combined with lane shuffles before the store.
//     Page ids come from a 64-entry, lane-indexed window read once per wave
//     and indexed with v_readlane; loads stream through a short register
//     pipeline in fully unrolled blocks, K and V alike as whole token rows
//     (K reaches the MFMA operand layout through LDS). Scores are kept in log2 units
//     (scale * log2 e) and exponentiated with v_exp_f32.
//  2. Merge: max-corrected combination of the live states of each (sequence,
//     query head) row (every stride-th one after a quarter combine).
//     merge_rows_kernel gives a row one wave when it has few states and there
//     are many rows; merge_cols_kernel cuts a row's columns into 128-byte chunks, one
//     256-lane workgroup each, so long rows are read by several workgroups at
//     once. The serial variants have every wave recompute the maximum and the
//     denominator; the shared variants form each state's weight once in LDS
//     and are bounded to PD_SHARED_MERGE_MAX_PARTS states.
//
// append_kv_kernel / append_kv_advance_kernel copy new token rows into their
// cache slots through the same page table.
//
// Semantics follow reference src/paged_decode/csrc/decode.cu:26-168 (online
// softmax and merge algebra, empty rows -> 0, l > 0 merge guard, page-id guard)
// and docs/DESIGN.md:5-76 (workspace of 4 * S states); the decomposition and
// data paths are this file's own.

#include "device_common.h"  // first: the HIP runtime header the maps' __host__ __device__ need
#include "cache_map.h"
#include "merge_map.h"
#include "partition_kernels.h"

namespace {

using namespace pd;

// ---------------------------------------------------------------------------
// Merge kernels: the max-corrected combination of a (sequence, query head)
// row's live states. A state with l == 0 is the identity (decode.cu:94-107).
// Two ways to form the weights, as the reference's two merges:
//   serial: every wave scans all states itself for the max and the denominator
//           (lanes share the scan, reduced with DPP), and each lane recomputes
//           the weight of the states it accumulates; no weight storage.
//   shared: the workgroup forms each state's weight once, into LDS
//           (4 bytes per state, hence the PD_SHARED_MERGE_MAX_PARTS bound).

// States of row b to merge (merge_map.h: live_states), from its device length.
__device__ __forceinline__ int live_parts(const MergeParams& mp, int b, int per_part, int states) {
    return live_states(mp.lengths[b], mp.split_tokens, mp.reach, per_part, states);
}

// merge_cols_kernel: a row's D columns are cut into chunks of CH floats and
// each (row, chunk) is one 256-lane workgroup, so D / CH workgroups read a
// row's states together. Lane t owns the 16-byte column t % (CH / 4) of the
// chunk for the states j == t / (CH / 4) (mod 1024 / CH) and issues up to NB
// of those loads in one round (NB = 8 or 32), together with the first round
// of the statistics scan, which is kept in registers for the denominator.
// Longer rows repeat both rounds. All loads use clamped indexes and are masked
// afterwards, so they issue back to back.
//
// Every workgroup of a row scans the row's statistics, so wider chunks scan
// them fewer times per row. That pays where the states come from other XCDs'
// writes; an XCD-grouped merge (states in its own L2) keeps the narrower
// chunk and twice the workgroups. Measured on MI355X (decode call, us, 32 ->
// 64 floats): ragged + shared B16 (plain grids, 512 rows of 28 states) 32.24-
// 32.28 -> 30.48-30.73, the reference's B4 / B16 batches 14.60 -> 14.51 /
// 41.11 -> 41.07; XCD-grouped 32K-context MHA 86.05 -> 86.17 and B1 L4096
// 9.60 -> 9.68, Llama-3-8B B4 L4096 unchanged.

template <int D, bool kSharedWeights, int NB, int CH>
__global__ void __launch_bounds__(kMergeThreads) merge_cols_kernel(const MergeParams mp) {
    constexpr int TPR = CH / 4;              // lanes per state slice
    constexpr int PG = kMergeThreads / TPR;  // state groups per workgroup
    constexpr int SU = NB / 2;  // (m, l) loads per scanning lane per round: a serial wave scans NB * PG states
    constexpr int kWaves = kMergeThreads / kWave;
    constexpr int kScan = kSharedWeights ? kMergeThreads : kWave;  // lanes sharing the state scan
    constexpr int kScanRound = SU * kScan;
    static_assert(D % CH == 0, "whole chunks");
    extern __shared__ float weight[];  // [parts], shared variant only
    __shared__ f32x4 column_sum[PG][TPR];
    __shared__ float wave_partial[2][kWaves];
    const MergeRow mr = merge_cols_row(mp, blockIdx.x, blockIdx.y);
    const int b = mr.b;
    const int64_t row = mr.row;
    const int chunk = blockIdx.z;
    const int shift = mp.stride_shift;
    const int parts = mp.parts >> shift;  // states read: j <-> allocated state j << shift
    const int t = threadIdx.x;
    const int lane = t % kWave;
    const int wave = t / kWave;
    const int col = t % TPR;
    const int pg = t / TPR;
    const int scan0 = kSharedWeights ? t : lane;
    const int last = parts - 1;
    const float2* st = reinterpret_cast<const float2*>(mp.stats) + merge_stats_base(mp, row);
    const f32x4* num = reinterpret_cast<const f32x4*>(mp.numerator) + merge_numerator_base(mp, row, D, chunk, CH, col);

    auto rounds_from = [&](int base, int limit) { return merge_cols_rounds(base, limit, NB, PG); };
    f32x4 buf[NB];
    float2 own[NB];
    // Loads k0 <= k < k1 (uniform bounds) of the round starting at state base.
    auto load_rounds = [&](int base, int k0, int k1) {
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            if (k >= k0 && k < k1) {
                const int j = merge_load_unit(base, pg, k, PG, last);
                buf[k] = num[merge_numerator_offset(mp, D, j)];
                if constexpr (!kSharedWeights) own[k] = read_state(st, merge_stats_offset(mp, j));
            }
        }
    };
    // The first kOptimisticRounds loads are issued before the live count
    // arrives (it comes with them) and masked afterwards: for the row's first
    // first_n states, the host's bound on live states where it has one (a plan
    // reserving context does not read its unwritten reserve), else the whole
    // row. The rest of the round covers live states only, so a ragged batch
    // does not read the states past its sequences' ends, and states past the
    // bound (lengths grown on the device) are still read.
    const int first_n = max(1, min(parts, mp.first_states));
    const int optimistic = min(kOptimisticRounds, rounds_from(0, first_n));
    load_rounds(0, 0, optimistic);
    const int live = live_parts(mp, b, kQuarters >> shift, parts);
    load_rounds(0, optimistic, rounds_from(0, live));

    auto scan_round = [&](int base, int limit, float2 (&sv)[SU]) {
#pragma unroll
        for (int i = 0; i < SU; ++i) {
            if (base + i * kScan < limit) sv[i] = read_state(st, merge_stats_offset(mp, min(base + scan0 + i * kScan, last)));
        }
    };
    auto round_max = [&](const float2 (&sv)[SU], int base, int limit, float m) {
#pragma unroll
        for (int i = 0; i < SU; ++i) {
            if (base + i * kScan < limit) {
                const bool ok = (base + scan0 + i * kScan < live) & (sv[i].y > 0.0f);
                m = ok ? fmaxf(m, sv[i].x) : m;
            }
        }
        return m;
    };
    // The statistics scan's first round covers the same first_n states (whole
    // kScan blocks of them); later rounds start where it ended.
    const int scan_end = min(kScanRound, (first_n + kScan - 1) / kScan * kScan);
    float2 first[SU];
    scan_round(0, first_n, first);
    float mx = round_max(first, 0, first_n, kNoToken);
    for (int base = scan_end; base < live; base += kScanRound) {
        float2 sv[SU];
        scan_round(base, live, sv);
        mx = round_max(sv, base, live, mx);
    }
    mx = wave_max(mx);
    if constexpr (kSharedWeights) {
        if (lane == 0) wave_partial[0][wave] = mx;
        __syncthreads();
        mx = wave_partial[0][0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, wave_partial[0][w]);
    }

    float den = 0.0f;
    auto accumulate_den = [&](const float2 (&sv)[SU], int base, int limit) {
#pragma unroll
        for (int i = 0; i < SU; ++i) {
            if (base + i * kScan < limit) {
                const int j = base + scan0 + i * kScan;
                const bool ok = (j < live) & (sv[i].y > 0.0f);
                const float f = ok ? fast_exp2(sv[i].x - mx) : 0.0f;
                if constexpr (kSharedWeights) {
                    if (j < live) weight[j] = f;
                }
                den = fmaf(f, ok ? sv[i].y : 0.0f, den);
            }
        }
    };
    accumulate_den(first, 0, first_n);
    for (int base = scan_end; base < live; base += kScanRound) {
        float2 sv[SU];
        scan_round(base, live, sv);
        accumulate_den(sv, base, live);
    }
    den = wave_sum(den);
    if constexpr (kSharedWeights) {
        if (lane == 0) wave_partial[1][wave] = den;
        __syncthreads();  // also publishes weight[]
        den = wave_partial[1][0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) den += wave_partial[1][w];
    }

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int base = 0;;) {
        const int rounds = rounds_from(base, live);
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            if (k < rounds) {
                const int j = base + pg + k * PG;
                float f;
                if constexpr (kSharedWeights) {
                    f = j < live ? weight[j] : 0.0f;
                } else {
                    f = ((j < live) & (own[k].y > 0.0f)) ? fast_exp2(own[k].x - mx) : 0.0f;
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] = f > 0.0f ? fmaf(f, buf[k][e], acc[e]) : acc[e];
            }
        }
        base += NB * PG;
        if (base >= live) break;
        load_rounds(base, 0, rounds_from(base, live));
    }
    column_sum[pg][col] = acc;
    __syncthreads();
    if (t < CH) {
        float sum = 0.0f;
#pragma unroll
        for (int g = 0; g < PG; ++g) sum += reinterpret_cast<const float*>(column_sum[g])[t];
        mp.out[row * D + chunk * CH + t] = den > 0.0f ? sum / den : 0.0f;
    }
}

// Small rows: one wave per (sequence, query head) row, four rows per
// workgroup, no barriers. Lane l owns column l % TPR of the states
// j == l / TPR (mod PGW) and lane j reads state j's (m, l) for the row
// maximum and denominator, reduced with DPP. The shared variant forms each
// state's weight once, in lane j, and broadcasts it with a cross-lane read;
// the serial variant has every lane recompute the weights it uses. The PGW
// column sums meet through permlane swaps. Used when a row's allocated states
// fit in NB loads per lane (NB = kMergeWaveBatch = 8: 16 states at D = 128, 32
// at D = 64); all loads are issued at once and masked with the live count.
// RPG rows (waves) per workgroup.
template <int D, bool kSharedWeights, int NB, int RPG>
__global__ void __launch_bounds__(kWave * RPG) merge_rows_kernel(const MergeParams mp) {
    constexpr int TPR = D / 4;        // lanes per state row
    constexpr int PGW = kWave / TPR;  // state groups per wave (2 or 4)
    static_assert(merge_wave_max_parts(D, NB) <= kWave, "one state per lane for the statistics");
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const MergeRow mr = merge_rows_row(mp, blockIdx.x, blockIdx.y, wave, RPG);
    if (mr.row < 0) return;  // whole wave past the last head; nothing below synchronises across waves
    const int b = mr.b;
    const int64_t row = mr.row;
    const int shift = mp.stride_shift;
    const int parts = mp.parts >> shift;  // states read: j <-> allocated state j << shift
    const int col = lane % TPR;
    const int pg = lane / TPR;
    const int last = parts - 1;
    const float2* st = reinterpret_cast<const float2*>(mp.stats) + merge_stats_base(mp, row);
    const f32x4* num = reinterpret_cast<const f32x4*>(mp.numerator) + merge_numerator_base(mp, row, D, 0, D, col);
    const int rounds = (parts + PGW - 1) / PGW;  // uniform, <= NB
    const int live = live_parts(mp, b, kQuarters >> shift, parts);

    f32x4 buf[NB];
    float2 own[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        if (k < rounds) {
            const int j = merge_load_unit(0, pg, k, PGW, last);
            buf[k] = num[merge_numerator_offset(mp, D, j)];
            if constexpr (!kSharedWeights) own[k] = read_state(st, merge_stats_offset(mp, j));
        }
    }
    const float2 mine = read_state(st, merge_stats_offset(mp, min(lane, last)));
    const bool ok = (lane < live) & (mine.y > 0.0f);
    const float mx = wave_max(ok ? mine.x : kNoToken);
    const float f = ok ? fast_exp2(mine.x - mx) : 0.0f;  // weight of state `lane`
    const float den = wave_sum(f * (ok ? mine.y : 0.0f));

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        if (k < rounds) {
            const int j = pg + k * PGW;
            float wj;
            if constexpr (kSharedWeights) {
                wj = __shfl(f, min(j, kWave - 1));
            } else {
                wj = own[k].y > 0.0f ? fast_exp2(own[k].x - mx) : 0.0f;
            }
            wj = j < live ? wj : 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = wj > 0.0f ? fmaf(wj, buf[k][e], acc[e]) : acc[e];
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if constexpr (PGW == 4) acc[e] = sum_over_lane_groups(acc[e]);
        else acc[e] = swap32_sum(acc[e], acc[e]);
    }
    if (pg == 0) {
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = den > 0.0f ? acc[e] / den : 0.0f;
        *reinterpret_cast<f32x4*>(mp.out + row * D + col * 4) = o;
    }
}

// ---------------------------------------------------------------------------
// Paged KV-cache append: the write step before decode. Token j of sequence b
// goes to logical position pos_b + j: page table[b, (pos_b + j) / T], slot
// (pos_b + j) % T, where one token row (all KV heads) is row_bytes contiguous
// bytes in both the new-token tensors [B, tokens, Hkv, D] and the cache
// [P, T, Hkv, D], so a token is a straight 16-byte-per-lane copy of its K row
// and its V row. Same addressing as the gather (reference docs/DESIGN.md:10-13).

// Physical row of logical position pos of the sequence whose page-table row
// is `pages`, or -1 if pos is outside [0, capacity) or its page id is outside
// [0, physical_pages) (cache_map.h).
__device__ __forceinline__ int64_t cache_row(const AppendParams& a, const int32_t* pages, int64_t pos) {
    const int64_t entry = append_table_entry(a, pos);
    if (entry < 0) return -1;
    return append_cache_row(a, pages[entry], pos);
}

__device__ __forceinline__ void copy_token_row(const AppendParams& a, int64_t src_row, int64_t dst_row) {
    const uint32_t chunks = a.row_bytes / 16u;
    for (uint32_t c = threadIdx.x; c < chunks; c += blockDim.x) {
        const int64_t src = append_chunk_offset(a, src_row, c);
        const int64_t dst = append_chunk_offset(a, dst_row, c);
        *reinterpret_cast<u32x4*>(a.k_cache + dst) = *reinterpret_cast<const u32x4*>(a.k_new + src);
        *reinterpret_cast<u32x4*>(a.v_cache + dst) = *reinterpret_cast<const u32x4*>(a.v_new + src);
    }
}

// Explicit positions: workgroup (j, b) writes token j of sequence b; tokens
// that do not map to a valid cache row are skipped.
__global__ void __launch_bounds__(256) append_kv_kernel(const AppendParams a) {
    const int j = blockIdx.x;
    const int b = blockIdx.y;
    const int32_t* pages = a.table + static_cast<int64_t>(b) * a.table_width;
    const int64_t dst = cache_row(a, pages, static_cast<int64_t>(a.positions[b]) + j);
    if (dst < 0) return;
    copy_token_row(a, append_source_row(a, b, j), dst);
}

// Positions from lengths, all or nothing per sequence: workgroup b writes its
// `tokens` tokens at lengths[b] .. lengths[b] + tokens - 1 only if every one of
// them maps to a valid cache row below the caller's context capacity (the
// context its partitions cover), then advances lengths[b]; otherwise the
// sequence and its length are left unchanged, so lengths never outgrow the
// partitions that decode them.
__global__ void __launch_bounds__(256) append_kv_advance_kernel(const AppendParams a) {
    const int b = blockIdx.x;
    const int32_t* pages = a.table + static_cast<int64_t>(b) * a.table_width;
    const int64_t base = a.lengths[b];
    bool fits = true;
    for (int j = 0; j < a.tokens; ++j) fits &= cache_row(a, pages, base + j) >= 0;  // uniform
    if (!fits) return;
    for (int j = 0; j < a.tokens; ++j) copy_token_row(a, append_source_row(a, b, j), cache_row(a, pages, base + j));
    __syncthreads();  // every thread has read lengths[b] before it changes
    if (threadIdx.x == 0) a.lengths[b] = static_cast<int32_t>(base + a.tokens);
}

// ---------------------------------------------------------------------------
// CSR page lists -> page table and lengths on the device: the inverse of the
// CSR form reference src/paged_decode/competitors.py:8-18 builds from a table.
// Row b takes the n_b = indptr[b + 1] - indptr[b] page ids from
// indices[indptr[b]] on and -1 past them; lengths[b] = (n_b - 1) * page_size +
// last_page_len[b], or 0 for an empty list. A row that does not fit (n_b < 0,
// n_b > table_width, last_page_len outside [1, page_size], or a length above
// max_context, or a page list reaching outside [0, indices_count)) is written
// empty and raises *overflow, so a malformed indptr never reads past indices.
// Page ids are not checked here: the partition kernel skips ids outside
// [0, physical_pages).
__global__ void __launch_bounds__(256) table_from_csr_kernel(const CsrParams c) {
    const int b = blockIdx.x;
    const int64_t begin = c.indptr[b];
    const int64_t end = c.indptr[b + 1];
    const CsrRow r = csr_row(c, begin, end, end > begin ? c.last_page_len[b] : 0);
    int32_t* row = c.table + static_cast<int64_t>(b) * c.table_width;
    for (int i = threadIdx.x; i < c.table_width; i += blockDim.x) row[i] = i < r.live ? c.indices[r.begin + i] : -1;
    if (threadIdx.x == 0) {
        c.lengths[b] = r.fits ? static_cast<int32_t>(r.length) : 0;
        if (!r.fits && c.overflow != nullptr) *c.overflow = 1;
    }
}

// ---------------------------------------------------------------------------
// Host side.

size_t element_size(int dtype) {
    switch (dtype) {
        case PD_DTYPE_F32: return 4;
        case PD_DTYPE_F16:
        case PD_DTYPE_BF16: return 2;
        default: return 1;  // FP8 formats
    }
}

// (q dtype, K/V dtype) pairs the partition kernels implement.
bool supported_formats(int q_dtype, int kv_dtype) {
    if (q_dtype == PD_DTYPE_F32) return kv_dtype == PD_DTYPE_F32;
    if (q_dtype == PD_DTYPE_F16 || q_dtype == PD_DTYPE_BF16)
        return kv_dtype == q_dtype || kv_dtype == PD_DTYPE_FP8_E4M3 || kv_dtype == PD_DTYPE_FP8_E5M2;
    return false;
}

int check_common(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype, float k_scale, float v_scale,
                 const int32_t* table, const int32_t* lengths, const float* numerator, const float* stats, int batch,
                 int query_heads, int kv_heads, int head_dim, int page_size, int table_width, int physical_pages,
                 int splits, int split_tokens) {
    if (!q || !k || !v || !table || !lengths || !numerator || !stats) return PD_ERR_NULL_POINTER;
    if (!supported_formats(q_dtype, kv_dtype)) return PD_ERR_DTYPE;
    if (!(k_scale > 0.0f && k_scale < INFINITY) || !(v_scale > 0.0f && v_scale < INFINITY)) return PD_ERR_DTYPE;
    if (batch < 1 || batch > 65535 || query_heads < 1 || query_heads > 65535) return PD_ERR_SHAPE;
    if (kv_heads < 1 || query_heads % kv_heads != 0) return PD_ERR_SHAPE;
    if (head_dim != 64 && head_dim != 128) return PD_ERR_SHAPE;
    if (page_size != 16 && page_size != 32) return PD_ERR_SHAPE;
    if (table_width < 1 || table_width > 65536 || physical_pages < 1) return PD_ERR_SHAPE;
    if (splits < 1 || splits > 65535 || split_tokens < 1 || split_tokens > (1 << 20)) return PD_ERR_SPLIT;
    return PD_OK;
}

int dispatch_partial(PartialParams& prm, int q_dtype, int kv_dtype, int kv_heads, int head_dim,
                     hipStream_t stream) {
    if (q_dtype == PD_DTYPE_F32)
        return head_dim == 64 ? dispatch_partial_f32_d64(prm, kv_dtype, kv_heads, stream)
                              : dispatch_partial_f32_d128(prm, kv_dtype, kv_heads, stream);
    if (q_dtype == PD_DTYPE_BF16)
        return head_dim == 64 ? dispatch_partial_bf16_d64(prm, kv_dtype, kv_heads, stream)
                              : dispatch_partial_bf16_d128(prm, kv_dtype, kv_heads, stream);
    return head_dim == 64 ? dispatch_partial_f16_d64(prm, kv_dtype, kv_heads, stream)
                          : dispatch_partial_f16_d128(prm, kv_dtype, kv_heads, stream);
}

// Partition-launch parameters of a call (pointers may be null for a plan
// query). With out given, the planner may choose a whole-row launch, which
// writes out itself.
PartialParams partial_params(const void* q, const void* k, const void* v, int kv_dtype, float k_scale,
                             float v_scale, const int32_t* table, const int32_t* lengths, float* numerator,
                             float* stats, float* out, int batch, int query_heads, int kv_heads, int head_dim,
                             int page_size, int table_width, int physical_pages, int splits, int split_tokens,
                             int hints, const int32_t* length_bounds, int reach,
                             const int32_t* prefix_runs = nullptr) {
    PartialParams prm{};
    prm.batch = batch;
    prm.host_bounds = length_bounds;
    prm.host_prefix_runs = prefix_runs;
    prm.unshared_pages = (hints & PD_HINT_UNSHARED_PAGES) != 0;
    prm.ragged_lengths = (hints & PD_HINT_RAGGED_LENGTHS) != 0;
    prm.q = q;
    prm.k = k;
    prm.v = v;
    prm.table = table;
    prm.lengths = lengths;
    prm.numerator = numerator;
    prm.stats = stats;
    prm.out = out;
    prm.row_allowed = out != nullptr;
    prm.query_heads = query_heads;
    prm.group = query_heads / kv_heads;
    prm.page_shift = page_size == 16 ? 4 : 5;
    prm.table_width = table_width;
    prm.physical_pages = physical_pages;
    prm.splits = splits;
    prm.split_tokens = split_tokens;
    prm.reach = reach;
    prm.token_bytes = static_cast<uint32_t>(static_cast<size_t>(kv_heads) * head_dim * element_size(kv_dtype));
    prm.page_bytes = static_cast<uint64_t>(page_size) * prm.token_bytes;
    prm.scale_log2 = kLog2e * k_scale / sqrtf(static_cast<float>(head_dim));
    prm.v_scale = v_scale;
    plan_items(prm, length_bounds);
    return prm;
}

// Tokens of a row that `splits` partitions of `split_tokens` reach in a table
// of `table_width` pages: the reference's grid of splits partitions reads no
// further (decode.cu:42-44, :176).
int call_reach(int splits, int split_tokens, int table_width, int page_size) {
    return static_cast<int>(lmin(static_cast<int64_t>(splits) * split_tokens,
                                 static_cast<int64_t>(table_width) * page_size));
}

// state_stride (if given) receives the merge's stride over the states: 1,
// the quarters combined per state, or 0 after a whole-row launch (no merge).
// reach: the caller's call_reach, when the launch runs over a coarser split
// than the caller's (else taken from splits and split_tokens).
int run_partial(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype, float k_scale, float v_scale,
                const int32_t* table, const int32_t* lengths, float* numerator, float* stats, int batch,
                int query_heads, int kv_heads, int head_dim, int page_size, int table_width, int physical_pages,
                int splits, int split_tokens, int hints, const int32_t* length_bounds, hipStream_t stream,
                float* out = nullptr, int* state_stride = nullptr, int* xcd_rows = nullptr,
                int* xcd_shift = nullptr, int reach = -1, const int32_t* prefix_runs = nullptr) {
    if (reach < 0) reach = call_reach(splits, split_tokens, table_width, page_size);
    PartialParams prm = partial_params(q, k, v, kv_dtype, k_scale, v_scale, table, lengths, numerator, stats, out,
                                       batch, query_heads, kv_heads, head_dim, page_size, table_width, physical_pages,
                                       splits, split_tokens, hints, length_bounds, reach, prefix_runs);
    const int status = dispatch_partial(prm, q_dtype, kv_dtype, kv_heads, head_dim, stream);
    if (state_stride) *state_stride = prm.row_mode ? 0 : prm.combine ? prm.quarters_per_wg : 1;
    if (xcd_rows) *xcd_rows = xcd_row_group_rows(prm);
    if (xcd_shift) *xcd_shift = prm.merge_xcd_shift;
    return status;
}


template <int D, int CH>
void launch_merge_cols(const MergeLaunch& ml, dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                       const MergeParams& mp) {
    if (ml.shared && ml.nb == kMergeColBatchLong) {
        hipLaunchKernelGGL((merge_cols_kernel<D, true, kMergeColBatchLong, CH>), grid, block, lds, stream, mp);
    } else if (ml.shared) {
        hipLaunchKernelGGL((merge_cols_kernel<D, true, kMergeColBatchShort, CH>), grid, block, lds, stream, mp);
    } else if (ml.nb == kMergeColBatchLong) {
        hipLaunchKernelGGL((merge_cols_kernel<D, false, kMergeColBatchLong, CH>), grid, block, lds, stream, mp);
    } else {
        hipLaunchKernelGGL((merge_cols_kernel<D, false, kMergeColBatchShort, CH>), grid, block, lds, stream, mp);
    }
}

// Launches the merge plan_merge chooses (kernel, variant, grid).
template <int D>
int launch_merge(MergeParams mp, int batch, int merge_mode, hipStream_t stream) {
    const MergeLaunch ml = plan_merge(mp, batch, D, merge_mode == PD_MERGE_SHARED, device_compute_units());
    mp.xcd_rows = ml.xcd_rows;
    const dim3 grid(ml.grid_x, ml.grid_y, ml.grid_z);
    const dim3 block(ml.threads);
    const size_t lds = static_cast<size_t>(ml.lds_bytes);
    if (ml.kind == kMergeRows) {
        if (ml.shared) {
            hipLaunchKernelGGL((merge_rows_kernel<D, true, kMergeWaveBatch, kMergeRowsPerGroup>), grid, block, 0,
                               stream, mp);
        } else {
            hipLaunchKernelGGL((merge_rows_kernel<D, false, kMergeWaveBatch, kMergeRowsPerGroup>), grid, block, 0,
                               stream, mp);
        }
    } else if (ml.ch == kMergeChunkLocal) {
        launch_merge_cols<D, kMergeChunkLocal>(ml, grid, block, lds, stream, mp);
    } else {
        launch_merge_cols<D, kMergeChunkWide>(ml, grid, block, lds, stream, mp);
    }
    return launch_status();
}

int check_hints(int hints) {
    return (hints & ~(PD_HINT_UNSHARED_PAGES | PD_HINT_RAGGED_LENGTHS)) == 0 ? PD_OK : PD_ERR_HINT;
}

int check_prefix_runs(const int32_t* prefix_runs, int batch, int table_width) {
    return prefix_runs == nullptr || prefix_runs_valid(prefix_runs, batch, table_width) ? PD_OK : PD_ERR_PREFIX;
}

int check_merge(const float* numerator, const float* stats, const float* out, const int32_t* lengths, int batch,
                int query_heads, int head_dim, int page_size, int table_width, int splits, int split_tokens,
                int merge_mode) {
    if (!numerator || !stats || !out || !lengths) return PD_ERR_NULL_POINTER;
    if (batch < 1 || batch > 65535 || query_heads < 1 || query_heads > 65535) return PD_ERR_SHAPE;
    if (head_dim != 64 && head_dim != 128) return PD_ERR_SHAPE;
    if (page_size != 16 && page_size != 32) return PD_ERR_SHAPE;
    if (table_width < 1 || table_width > 65536) return PD_ERR_SHAPE;
    if (splits < 1 || splits > 65535 || split_tokens < 1 || split_tokens > (1 << 20)) return PD_ERR_SPLIT;
    if (merge_mode != PD_MERGE_SERIAL && merge_mode != PD_MERGE_SHARED) return PD_ERR_MERGE;
    if (merge_mode == PD_MERGE_SHARED && kQuarters * splits > PD_SHARED_MERGE_MAX_PARTS) return PD_ERR_MERGE;
    return PD_OK;
}

// length_bounds (host, or null): upper bounds on the device lengths, which
// bound the states the merge loads before it knows a row's live count.
// reach: as run_partial's.
int run_merge(const float* numerator, const float* stats, float* out, const int32_t* lengths, int batch,
              int query_heads, int head_dim, int page_size, int table_width, int splits, int split_tokens,
              int merge_mode, int stride, hipStream_t stream, const int32_t* length_bounds = nullptr,
              int xcd_rows = 0, int xcd_shift = 0, int reach = -1) {
    MergeParams mp{};
    mp.numerator = numerator;
    mp.stats = stats;
    mp.out = out;
    mp.lengths = lengths;
    mp.parts = kQuarters * splits;
    mp.stride_shift = stride == 4 ? 2 : stride == 2 ? 1 : 0;
    mp.query_heads = query_heads;
    mp.split_tokens = split_tokens;
    mp.reach = reach < 0 ? call_reach(splits, split_tokens, table_width, page_size) : reach;
    mp.first_states = merge_first_states(mp.parts, mp.stride_shift, split_tokens, mp.reach, length_bounds, batch);
    mp.xcd_rows = xcd_rows;
    mp.xcd_shift = xcd_shift;
    return head_dim == 64 ? launch_merge<64>(mp, batch, merge_mode, stream)
                          : launch_merge<128>(mp, batch, merge_mode, stream);
}

int check_append(const void* k_new, const void* v_new, int dtype, const int32_t* table, const int32_t* positions,
                 const void* k_cache, const void* v_cache, int batch, int tokens, int kv_heads, int head_dim,
                 int page_size, int table_width, int physical_pages) {
    if (!k_new || !v_new || !table || !positions || !k_cache || !v_cache) return PD_ERR_NULL_POINTER;
    if (dtype < PD_DTYPE_F32 || dtype > PD_DTYPE_FP8_E5M2) return PD_ERR_DTYPE;
    if (batch < 1 || batch > 65535 || tokens < 1 || tokens > 65535 || kv_heads < 1 || kv_heads > 65535)
        return PD_ERR_SHAPE;
    if (head_dim != 64 && head_dim != 128) return PD_ERR_SHAPE;
    if (page_size != 16 && page_size != 32) return PD_ERR_SHAPE;
    if (table_width < 1 || table_width > 65536 || physical_pages < 1) return PD_ERR_SHAPE;
    return PD_OK;
}

AppendParams append_params(const void* k_new, const void* v_new, int dtype, const int32_t* table, void* k_cache,
                           void* v_cache, int tokens, int kv_heads, int head_dim, int page_size, int table_width,
                           int physical_pages) {
    AppendParams a{};
    a.k_new = static_cast<const char*>(k_new);
    a.v_new = static_cast<const char*>(v_new);
    a.table = table;
    a.k_cache = static_cast<char*>(k_cache);
    a.v_cache = static_cast<char*>(v_cache);
    a.tokens = tokens;
    a.table_width = table_width;
    a.page_shift = page_size == 16 ? 4 : 5;
    a.physical_pages = physical_pages;
    a.capacity = static_cast<int64_t>(table_width) << a.page_shift;
    a.row_bytes = static_cast<uint32_t>(static_cast<size_t>(kv_heads) * head_dim * element_size(dtype));
    return a;
}

// ---------------------------------------------------------------------------
// Streaming read (pd_stream_read): the bandwidth ceiling a decode launch is
// measured against. Reads a_bytes of a, then b_bytes of b, once each, in
// 16-byte non-temporal loads, each lane keeping kStreamLoads loads in flight.
// The workgroups of the first ceil(a / block) grid slots read a, the rest b.
// The loaded words are folded with XOR into a value that is stored only if it
// equals `magic`, so no load is dead code and the kernel writes (almost
// always) nothing. The shape is the fastest of those measured on MI355X
// (graph of 200 launches over a 2.3 GB rotation; 2, 4, 8 or 16 loads per lane,
// 256, 512 or 1024 threads, plain or non-temporal loads): 8 non-temporal loads
// per lane in 256-thread workgroups read 33.5 / 67 / 201 / 537 MB in 6.13 /
// 10.69 / 29.8 / 77.9 us, against 6.41 / 11.33 / 32.0 / 83.5 us for the best
// plain-load shape.
constexpr int kStreamThreads = 256;
constexpr int kStreamLoads = 8;
constexpr uint64_t kStreamBlockVectors = static_cast<uint64_t>(kStreamThreads) * kStreamLoads;

struct StreamParams {
    const u32x4* a;
    const u32x4* b;
    uint64_t a_vectors, b_vectors;  // 16-byte vectors of each buffer to read
    uint64_t a_blocks;              // workgroups reading a
    uint32_t magic;
    uint32_t* sink;
};

__global__ void __launch_bounds__(kStreamThreads) stream_read_kernel(const StreamParams sp) {
    const bool in_a = blockIdx.x < sp.a_blocks;
    const u32x4* base = in_a ? sp.a : sp.b;
    const uint64_t vectors = in_a ? sp.a_vectors : sp.b_vectors;
    const uint64_t block = in_a ? blockIdx.x : blockIdx.x - sp.a_blocks;
    const uint64_t first = block * kStreamBlockVectors + threadIdx.x;
    u32x4 v[kStreamLoads];
#pragma unroll
    for (int i = 0; i < kStreamLoads; ++i) {
        const uint64_t idx = first + static_cast<uint64_t>(i) * kStreamThreads;
        v[i] = idx < vectors ? __builtin_nontemporal_load(base + idx) : u32x4{0u, 0u, 0u, 0u};
    }
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < kStreamLoads; ++i) acc ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
    if (acc == sp.magic) sp.sink[threadIdx.x & 1] = acc;
}

// ---------------------------------------------------------------------------
// Static scratch for pd_decode_scratch: the partition states of callers that
// cannot allocate (graph capture, serving loops, harnesses that forbid
// hipMalloc). One array per device, PD_SCRATCH_BYTES long, held by the
// process until it exits; every pd_decode_scratch call on a device uses the
// same array, so calls that overlap on one device race. Host code never
// passes `scratch` itself to a kernel (in host code the name is a stand-in,
// not a device address): the device address comes from hipGetSymbolAddress,
// looked up once per device with that device current, and only that pointer
// is used.
static __device__ __align__(256) float scratch[PD_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxDevices = 64;

// Device address of `scratch` on the current device, or nullptr if the
// runtime cannot give it.
float* scratch_address() {
    static std::atomic<float*> cached[kMaxDevices];
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return nullptr;
    float* ptr = cached[device].load(std::memory_order_acquire);
    if (ptr == nullptr) {
        void* address = nullptr;
        if (hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)) != hipSuccess || address == nullptr) return nullptr;
        ptr = static_cast<float*>(address);
        cached[device].store(ptr, std::memory_order_release);
    }
    return ptr;
}

// Partitions the two launches of a full decode call run over: the caller's
// split for FP32 inputs and whole-row calls, else coarse_split's.
KernelSplit call_split(int q_dtype, int kv_dtype, int batch, int query_heads, int kv_heads, int head_dim,
                       int page_size, int table_width, int splits, int split_tokens, const int32_t* length_bounds,
                       int cus, const int32_t* prefix_runs = nullptr) {
    return full_call_split(q_dtype == PD_DTYPE_F32, element_size(kv_dtype), batch, query_heads, kv_heads, head_dim,
                           page_size, table_width, splits, split_tokens, length_bounds, cus, prefix_runs);
}

// The scratch holds numerator [B, Hq, 4 * splits, D] at offset 0 and stats
// [B, Hq, 4 * splits, 2] after it, at the next 256-byte boundary.
size_t scratch_stats_offset(int batch, int query_heads, int head_dim, int splits) {
    const size_t numerator = static_cast<size_t>(batch) * query_heads * kQuarters * splits * head_dim * sizeof(float);
    return (numerator + 255) / 256 * 256;
}

}  // namespace

extern "C" {

int pd_decode_partial_prefix(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype, float k_scale,
                             float v_scale, const int32_t* table, const int32_t* lengths, float* numerator,
                             float* stats, int batch, int query_heads, int kv_heads, int head_dim, int page_size,
                             int table_width, int physical_pages, int splits, int split_tokens, int hints,
                             const int32_t* length_bounds, const int32_t* prefix_runs, void* stream) {
    int status = check_common(q, q_dtype, k, v, kv_dtype, k_scale, v_scale, table, lengths, numerator, stats, batch,
                              query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                              split_tokens);
    if (status == PD_OK) status = check_hints(hints);
    if (status == PD_OK) status = check_prefix_runs(prefix_runs, batch, table_width);
    if (status != PD_OK) return status;
    return run_partial(q, q_dtype, k, v, kv_dtype, k_scale, v_scale, table, lengths, numerator, stats, batch,
                       query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits, split_tokens,
                       hints, length_bounds, static_cast<hipStream_t>(stream), nullptr, nullptr, nullptr, nullptr, -1,
                       prefix_runs);
}

int pd_decode_partial_ex(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype, float k_scale,
                         float v_scale, const int32_t* table, const int32_t* lengths, float* numerator, float* stats,
                         int batch, int query_heads, int kv_heads, int head_dim, int page_size, int table_width,
                         int physical_pages, int splits, int split_tokens, int hints, const int32_t* length_bounds,
                         void* stream) {
    return pd_decode_partial_prefix(q, q_dtype, k, v, kv_dtype, k_scale, v_scale, table, lengths, numerator, stats,
                                    batch, query_heads, kv_heads, head_dim, page_size, table_width, physical_pages,
                                    splits, split_tokens, hints, length_bounds, nullptr, stream);
}

int pd_decode_partial(const void* q, const void* k, const void* v, int dtype, const int32_t* table,
                      const int32_t* lengths, float* numerator, float* stats, int batch, int query_heads,
                      int kv_heads, int head_dim, int page_size, int table_width, int physical_pages, int splits,
                      int split_tokens, void* stream) {
    return pd_decode_partial_ex(q, dtype, k, v, dtype, 1.0f, 1.0f, table, lengths, numerator, stats, batch,
                                query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                                split_tokens, PD_HINT_NONE, nullptr, stream);
}

int pd_decode_merge(const float* numerator, const float* stats, float* out, const int32_t* lengths, int batch,
                    int query_heads, int head_dim, int page_size, int table_width, int splits, int split_tokens,
                    int merge_mode, void* stream) {
    const int status = check_merge(numerator, stats, out, lengths, batch, query_heads, head_dim, page_size,
                                   table_width, splits, split_tokens, merge_mode);
    if (status != PD_OK) return status;
    return run_merge(numerator, stats, out, lengths, batch, query_heads, head_dim, page_size, table_width, splits,
                     split_tokens, merge_mode, 1, static_cast<hipStream_t>(stream));
}

int pd_decode_prefix(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype, float k_scale,
                     float v_scale, const int32_t* table, const int32_t* lengths, float* numerator, float* stats,
                     float* out, int batch, int query_heads, int kv_heads, int head_dim, int page_size,
                     int table_width, int physical_pages, int splits, int split_tokens, int merge_mode, int hints,
                     const int32_t* length_bounds, const int32_t* prefix_runs, void* stream) {
    int status = check_common(q, q_dtype, k, v, kv_dtype, k_scale, v_scale, table, lengths, numerator, stats, batch,
                              query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                              split_tokens);
    if (status == PD_OK)
        status = check_merge(numerator, stats, out, lengths, batch, query_heads, head_dim, page_size, table_width,
                             splits, split_tokens, merge_mode);
    if (status == PD_OK) status = check_hints(hints);
    if (status == PD_OK) status = check_prefix_runs(prefix_runs, batch, table_width);
    if (status != PD_OK) return status;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // Both launches run over the same partitions, at most `splits` of them
    // per row, so the states fit the caller's workspace, and read no token
    // past the caller's partitions (reach).
    const KernelSplit ks = call_split(q_dtype, kv_dtype, batch, query_heads, kv_heads, head_dim, page_size,
                                      table_width, splits, split_tokens, length_bounds, device_compute_units(),
                                      prefix_runs);
    const int reach = call_reach(splits, split_tokens, table_width, page_size);
    int stride = 1, xcd_rows = 0, xcd_shift = 0;
    status = run_partial(q, q_dtype, k, v, kv_dtype, k_scale, v_scale, table, lengths, numerator, stats, batch,
                         query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, ks.splits,
                         ks.split_tokens, hints, length_bounds, s, out, &stride, &xcd_rows, &xcd_shift, reach,
                         prefix_runs);
    if (status != PD_OK || stride == 0) return status;
    return run_merge(numerator, stats, out, lengths, batch, query_heads, head_dim, page_size, table_width, ks.splits,
                     ks.split_tokens, merge_mode, stride, s, length_bounds, xcd_rows, xcd_shift, reach);
}

int pd_decode_ex(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype, float k_scale,
                 float v_scale, const int32_t* table, const int32_t* lengths, float* numerator, float* stats,
                 float* out, int batch, int query_heads, int kv_heads, int head_dim, int page_size, int table_width,
                 int physical_pages, int splits, int split_tokens, int merge_mode, int hints,
                 const int32_t* length_bounds, void* stream) {
    return pd_decode_prefix(q, q_dtype, k, v, kv_dtype, k_scale, v_scale, table, lengths, numerator, stats, out,
                            batch, query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                            split_tokens, merge_mode, hints, length_bounds, nullptr, stream);
}

int pd_prefix_runs(const int32_t* table, int batch, int table_width, int32_t* runs) {
    if (!table || !runs) return PD_ERR_NULL_POINTER;
    if (batch < 1 || batch > 65535 || table_width < 1 || table_width > 65536) return PD_ERR_SHAPE;
    prefix_runs_of_table(table, batch, table_width, runs);
    return PD_OK;
}

int pd_decode(const void* q, const void* k, const void* v, int dtype, const int32_t* table,
              const int32_t* lengths, float* numerator, float* stats, float* out, int batch, int query_heads,
              int kv_heads, int head_dim, int page_size, int table_width, int physical_pages, int splits,
              int split_tokens, int merge_mode, void* stream) {
    return pd_decode_ex(q, dtype, k, v, dtype, 1.0f, 1.0f, table, lengths, numerator, stats, out, batch,
                        query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits, split_tokens,
                        merge_mode, PD_HINT_NONE, nullptr, stream);
}

int pd_decode_scratch(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype, float k_scale,
                      float v_scale, const int32_t* table, const int32_t* lengths, float* out, int batch,
                      int query_heads, int kv_heads, int head_dim, int page_size, int table_width,
                      int physical_pages, int splits, int split_tokens, int merge_mode, int hints,
                      const int32_t* length_bounds, void* stream) {
    // Shapes are checked before any runtime call, so a rejected request
    // touches no device; the stand-in pointers only pass the null checks.
    float* const stand_in = reinterpret_cast<float*>(alignof(float));
    int status = check_common(q, q_dtype, k, v, kv_dtype, k_scale, v_scale, table, lengths, stand_in, stand_in,
                              batch, query_heads, kv_heads, head_dim, page_size, table_width, physical_pages,
                              splits, split_tokens);
    if (status == PD_OK)
        status = check_merge(stand_in, stand_in, out, lengths, batch, query_heads, head_dim, page_size, table_width,
                             splits, split_tokens, merge_mode);
    if (status == PD_OK) status = check_hints(hints);
    if (status != PD_OK) return status;
    const size_t stats_offset = scratch_stats_offset(batch, query_heads, head_dim, splits);
    const size_t stats_bytes = static_cast<size_t>(batch) * query_heads * kQuarters * splits * 2 * sizeof(float);
    if (stats_offset + stats_bytes > PD_SCRATCH_BYTES) return PD_ERR_SCRATCH;
    float* const base = scratch_address();
    if (base == nullptr) return PD_ERR_SCRATCH;
    float* const numerator = base;
    float* const stats = base + stats_offset / sizeof(float);
    return pd_decode_ex(q, q_dtype, k, v, kv_dtype, k_scale, v_scale, table, lengths, numerator, stats, out, batch,
                        query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits, split_tokens,
                        merge_mode, hints, length_bounds, stream);
}

int pd_append_kv(const void* k_new, const void* v_new, int dtype, const int32_t* table, const int32_t* positions,
                 void* k_cache, void* v_cache, int batch, int tokens, int kv_heads, int head_dim, int page_size,
                 int table_width, int physical_pages, void* stream) {
    const int status = check_append(k_new, v_new, dtype, table, positions, k_cache, v_cache, batch, tokens, kv_heads,
                                     head_dim, page_size, table_width, physical_pages);
    if (status != PD_OK) return status;
    AppendParams a = append_params(k_new, v_new, dtype, table, k_cache, v_cache, tokens, kv_heads, head_dim,
                                   page_size, table_width, physical_pages);
    a.positions = positions;
    hipLaunchKernelGGL(append_kv_kernel, dim3(tokens, batch), dim3(256), 0, static_cast<hipStream_t>(stream), a);
    return launch_status();
}

int pd_append_kv_advance(const void* k_new, const void* v_new, int dtype, const int32_t* table, int32_t* lengths,
                         void* k_cache, void* v_cache, int batch, int tokens, int kv_heads, int head_dim,
                         int page_size, int table_width, int physical_pages, int max_context, void* stream) {
    int status = check_append(k_new, v_new, dtype, table, lengths, k_cache, v_cache, batch, tokens, kv_heads,
                              head_dim, page_size, table_width, physical_pages);
    if (status == PD_OK && (max_context < 0 || max_context > (1 << 20))) status = PD_ERR_SHAPE;
    if (status != PD_OK) return status;
    AppendParams a = append_params(k_new, v_new, dtype, table, k_cache, v_cache, tokens, kv_heads, head_dim,
                                   page_size, table_width, physical_pages);
    a.capacity = std::min<int64_t>(a.capacity, max_context);
    a.lengths = lengths;
    hipLaunchKernelGGL(append_kv_advance_kernel, dim3(batch), dim3(256), 0, static_cast<hipStream_t>(stream), a);
    return launch_status();
}

int pd_stream_read(const void* a, size_t a_bytes, const void* b, size_t b_bytes, uint32_t* sink, void* stream) {
    if (!sink || (a_bytes && !a) || (b_bytes && !b)) return PD_ERR_NULL_POINTER;
    if (a_bytes % 16 != 0 || b_bytes % 16 != 0 || reinterpret_cast<uintptr_t>(a) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(b) % 16 != 0)
        return PD_ERR_SHAPE;
    StreamParams sp{};
    sp.a = static_cast<const u32x4*>(a);
    sp.b = static_cast<const u32x4*>(b);
    sp.a_vectors = a_bytes / 16;
    sp.b_vectors = b_bytes / 16;
    sp.a_blocks = (sp.a_vectors + kStreamBlockVectors - 1) / kStreamBlockVectors;
    const uint64_t blocks = sp.a_blocks + (sp.b_vectors + kStreamBlockVectors - 1) / kStreamBlockVectors;
    if (blocks == 0) return PD_OK;
    if (blocks > 0x7FFFFFFFull) return PD_ERR_SHAPE;
    sp.magic = 0x9E3779B9u;
    sp.sink = sink;
    hipLaunchKernelGGL(stream_read_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kStreamThreads), 0,
                       static_cast<hipStream_t>(stream), sp);
    return launch_status();
}

int pd_table_from_csr(const int32_t* indptr, const int32_t* indices, int64_t indices_count,
                      const int32_t* last_page_len, int32_t* table, int32_t* lengths, int32_t* overflow, int batch,
                      int table_width, int page_size, int max_context, void* stream) {
    if (!indptr || !last_page_len || !table || !lengths || (!indices && indices_count > 0)) return PD_ERR_NULL_POINTER;
    if (batch < 1 || batch > 65535 || table_width < 1 || table_width > 65536 || indices_count < 0)
        return PD_ERR_SHAPE;
    if (page_size != 16 && page_size != 32) return PD_ERR_SHAPE;
    if (max_context < 0 || max_context > (1 << 20)) return PD_ERR_SHAPE;
    CsrParams c{indptr, indices, last_page_len, table, lengths, overflow, indices_count, table_width, page_size,
                max_context};
    hipLaunchKernelGGL(table_from_csr_kernel, dim3(batch), dim3(256), 0, static_cast<hipStream_t>(stream), c);
    return launch_status();
}

int pd_decode_launch_count(int q_dtype, int kv_dtype, int batch, int query_heads, int kv_heads, int head_dim,
                           int page_size, int table_width, int physical_pages, int splits, int split_tokens,
                           int hints, int* launches) {
    if (!launches) return PD_ERR_NULL_POINTER;
    // The shape checks of pd_decode_ex, with stand-ins for the buffers.
    const char* const stand_in = reinterpret_cast<const char*>(alignof(float));
    float* const f_stand_in = reinterpret_cast<float*>(alignof(float));
    int status = check_common(stand_in, q_dtype, stand_in, stand_in, kv_dtype, 1.0f, 1.0f,
                              reinterpret_cast<const int32_t*>(stand_in), reinterpret_cast<const int32_t*>(stand_in),
                              f_stand_in, f_stand_in, batch, query_heads, kv_heads, head_dim, page_size, table_width,
                              physical_pages, splits, split_tokens);
    if (status == PD_OK) status = check_hints(hints);
    if (status != PD_OK) return status;
    PartialParams prm = partial_params(nullptr, nullptr, nullptr, kv_dtype, 1.0f, 1.0f, nullptr, nullptr, nullptr,
                                       nullptr, f_stand_in, batch, query_heads, kv_heads, head_dim, page_size,
                                       table_width, physical_pages, splits, split_tokens, hints, nullptr,
                                       call_reach(splits, split_tokens, table_width, page_size));
    if (q_dtype == PD_DTYPE_F32) plan_fp32(prm, kv_heads, head_dim);
    else plan_mfma(prm, kv_heads, device_compute_units(), head_dim, element_size(kv_dtype));
    *launches = prm.row_mode ? 1 : 2;
    return PD_OK;
}

int pd_decode_kernel_split(int q_dtype, int kv_dtype, int batch, int query_heads, int kv_heads, int head_dim,
                           int page_size, int table_width, int physical_pages, int splits, int split_tokens,
                           const int32_t* length_bounds, int compute_units, int* kernel_splits,
                           int* kernel_split_tokens) {
    if (!kernel_splits || !kernel_split_tokens) return PD_ERR_NULL_POINTER;
    const char* const stand_in = reinterpret_cast<const char*>(alignof(float));
    float* const f_stand_in = reinterpret_cast<float*>(alignof(float));
    const int status = check_common(stand_in, q_dtype, stand_in, stand_in, kv_dtype, 1.0f, 1.0f,
                                    reinterpret_cast<const int32_t*>(stand_in),
                                    reinterpret_cast<const int32_t*>(stand_in), f_stand_in, f_stand_in, batch,
                                    query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                                    split_tokens);
    if (status != PD_OK) return status;
    const KernelSplit ks = call_split(q_dtype, kv_dtype, batch, query_heads, kv_heads, head_dim, page_size,
                                      table_width, splits, split_tokens, length_bounds,
                                      compute_units > 0 ? compute_units : device_compute_units());
    *kernel_splits = ks.splits;
    *kernel_split_tokens = ks.split_tokens;
    return PD_OK;
}

int pd_decode_launch_plan(int q_dtype, int kv_dtype, int batch, int query_heads, int kv_heads, int head_dim,
                          int page_size, int table_width, int physical_pages, int splits, int split_tokens,
                          int merge_mode, int hints, const int32_t* length_bounds, const int32_t* prefix_runs,
                          int compute_units, pd_launch_plan* plan) {
    if (!plan) return PD_ERR_NULL_POINTER;
    const char* const stand_in = reinterpret_cast<const char*>(alignof(float));
    float* const f_stand_in = reinterpret_cast<float*>(alignof(float));
    int status = check_common(stand_in, q_dtype, stand_in, stand_in, kv_dtype, 1.0f, 1.0f,
                              reinterpret_cast<const int32_t*>(stand_in), reinterpret_cast<const int32_t*>(stand_in),
                              f_stand_in, f_stand_in, batch, query_heads, kv_heads, head_dim, page_size, table_width,
                              physical_pages, splits, split_tokens);
    if (status == PD_OK)
        status = check_merge(f_stand_in, f_stand_in, f_stand_in, reinterpret_cast<const int32_t*>(stand_in), batch,
                             query_heads, head_dim, page_size, table_width, splits, split_tokens, merge_mode);
    if (status == PD_OK) status = check_hints(hints);
    if (status == PD_OK) status = check_prefix_runs(prefix_runs, batch, table_width);
    if (status != PD_OK) return status;
    const int cus = compute_units > 0 ? compute_units : device_compute_units();
    // The planning of pd_decode_ex, without its launches.
    const KernelSplit ks = call_split(q_dtype, kv_dtype, batch, query_heads, kv_heads, head_dim, page_size,
                                      table_width, splits, split_tokens, length_bounds, cus, prefix_runs);
    const int reach = call_reach(splits, split_tokens, table_width, page_size);
    PartialParams prm = partial_params(nullptr, nullptr, nullptr, kv_dtype, 1.0f, 1.0f, nullptr, nullptr, nullptr,
                                       nullptr, f_stand_in, batch, query_heads, kv_heads, head_dim, page_size,
                                       table_width, physical_pages, ks.splits, ks.split_tokens, hints, length_bounds,
                                       reach, prefix_runs);
    if (q_dtype == PD_DTYPE_F32) plan_fp32(prm, kv_heads, head_dim);
    else plan_mfma(prm, kv_heads, cus, head_dim, static_cast<int>(element_size(kv_dtype)));
    const Grid grid = partial_grid(prm, kv_heads);
    pd_launch_plan p{};
    p.launches = prm.row_mode ? 1 : 2;
    p.kernel_splits = ks.splits;
    p.kernel_split_tokens = ks.split_tokens;
    p.grid_x = grid.x;
    p.grid_y = grid.y;
    p.grid_z = grid.z;
    p.waves_per_workgroup = partial_threads(prm) / kWave;
    p.kv_heads_per_workgroup = prm.heads_per_wg;
    p.quarters_per_workgroup = prm.quarters_per_wg;
    p.head_tile = prm.head_tile;
    p.grid_kind = prm.row_mode ? 3 : grid_kind(prm);
    p.xcd_grouped = prm.xcd_shift >= 0;
    p.combined = prm.combine;
    p.stream_mode = prm.stream_mode;
    p.shared_prefix_items = prm.group_items;
    p.merge_kernel = -1;
    if (!prm.row_mode) {
        const int stride = prm.combine ? prm.quarters_per_wg : 1;
        MergeParams mp{};
        mp.parts = kQuarters * ks.splits;
        mp.stride_shift = stride == 4 ? 2 : stride == 2 ? 1 : 0;
        mp.query_heads = query_heads;
        mp.split_tokens = ks.split_tokens;
        mp.reach = reach;
        mp.first_states = merge_first_states(mp.parts, mp.stride_shift, ks.split_tokens, reach, length_bounds, batch);
        mp.xcd_rows = xcd_row_group_rows(prm);
        mp.xcd_shift = prm.merge_xcd_shift;
        const MergeLaunch ml = plan_merge(mp, batch, head_dim, merge_mode == PD_MERGE_SHARED, cus);
        p.merge_kernel = ml.kind == kMergeRows ? 0 : 1;
        p.merge_loads = ml.nb;
        p.merge_chunk_floats = ml.ch;
        p.merge_xcd_grouped = ml.xcd_rows > 0;
        p.merge_state_stride = stride;
    }
    *plan = p;
    return PD_OK;
}

size_t pd_workspace_bytes(int batch, int query_heads, int head_dim, int splits) {
    if (batch <= 0 || query_heads <= 0 || head_dim <= 0 || splits <= 0) return 0;
    return static_cast<size_t>(batch) * query_heads * kQuarters * splits * (head_dim + 2) * sizeof(float);
}

const char* pd_status_string(int status) {
    switch (status) {
        case PD_OK: return "success";
        case PD_ERR_NULL_POINTER: return "a required pointer is null";
        case PD_ERR_SHAPE: return "a dimension is outside the supported range";
        case PD_ERR_DTYPE: return "unsupported dtype combination or non-positive/non-finite scale";
        case PD_ERR_SPLIT: return "invalid split configuration";
        case PD_ERR_MERGE: return "unknown merge mode or shared merge requires at most 4096 partial states (4 per split)";
        case PD_ERR_LAUNCH: return "kernel launch failed";
        case PD_ERR_HINT: return "unknown hint bits";
        case PD_ERR_SCRATCH:
            return "the workspace does not fit the library's static scratch (PD_SCRATCH_BYTES), or its device "
                   "address could not be obtained";
        case PD_ERR_PREFIX: return "malformed shared-prefix runs (a leader outside [-1, batch) or a count outside [0, table_width])";
        default: return "unknown status";
    }
}

int pd_abi_version(void) { return PD_ABI_VERSION; }

}  // extern "C"
