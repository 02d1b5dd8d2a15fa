// Split-K paged GQA decode attention for gfx950 (AMD Instinct MI355X), and the
// paged KV-cache append that feeds it.
//
// Implements the C ABI declared in include/paged_decode.h. pd_decode makes two
// launches per call, both on the caller's stream:
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
//     nothing.
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

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <cstdint>
#include <type_traits>

#include "paged_decode.h"
#include "partition_map.h"

namespace {

using namespace pd;

constexpr float kNoToken = -FLT_MAX;  // running max before any live token
constexpr float kLog2e = 1.4426950408889634f;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// Note: reinterpret whole vectors (bit_cast of a u32x4 to f16x8 / f32x4), never
// a single element: clang 22 lowers __builtin_bit_cast of a vector-element
// lvalue to a read of element 0.

// ---------------------------------------------------------------------------
// Wave64 lane primitives.
// DPP controls: quad_perm [1,0,3,2] and [2,3,0,1] swap neighbours at distance
// 1 and 2; row_half_mirror reverses each 8-lane half-row; row_mirror reverses
// each 16-lane row. Applied in that order, a sum/max reaches every lane of an
// aligned 8- or 16-lane group. ds_swizzle in bit mode with xor 0x10 exchanges
// lanes 16 apart within each 32-lane half.
constexpr int kDppQuadSwap1 = 0xB1;
constexpr int kDppQuadSwap2 = 0x4E;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kSwizzleSwap16 = 0x401F;

template <int kCtrl>
__device__ __forceinline__ float dpp_move(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float swizzle_swap16(float x) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), kSwizzleSwap16));
}

// Sum over each aligned group of kLanes (8, 16 or 32) lanes, result in every lane.
template <int kLanes>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(kLanes == 8 || kLanes == 16 || kLanes == 32, "unsupported group");
    x += dpp_move<kDppQuadSwap1>(x);
    x += dpp_move<kDppQuadSwap2>(x);
    x += dpp_move<kDppRowHalfMirror>(x);
    if constexpr (kLanes >= 16) x += dpp_move<kDppRowMirror>(x);
    if constexpr (kLanes >= 32) x += swizzle_swap16(x);
    return x;
}

__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp_move<kDppQuadSwap1>(x));
    x = fmaxf(x, dpp_move<kDppQuadSwap2>(x));
    x = fmaxf(x, dpp_move<kDppRowHalfMirror>(x));
    x = fmaxf(x, dpp_move<kDppRowMirror>(x));
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

__device__ __forceinline__ float wave_sum(float x) {
    x = group_sum<16>(x);
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// gfx950 v_permlane32_swap / v_permlane16_swap on float pairs. For (a, b):
//   swap32: lanes 0-31 get (a[l], a[l+32]), lanes 32-63 get (b[l-32], b[l]);
//   swap16: even 16-lane rows get (a[l], a[l+16]), odd rows (b[l-16], b[l]).
// The pair's sum is a + partner's a in the lower half (even rows) and
// b + partner's b in the upper half (odd rows): one reduce-scatter step.
// The builtins return a two-element vector; its elements are copied into
// scalars before the bit cast (a bit cast of a vector-element lvalue reads
// element 0 with this compiler).
struct FloatPair {
    float first, second;
};

__device__ __forceinline__ FloatPair permlane32_swap(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, a), __builtin_bit_cast(unsigned, b),
                                                    false, false);
    const unsigned first = r[0], second = r[1];
    return {__builtin_bit_cast(float, first), __builtin_bit_cast(float, second)};
}

__device__ __forceinline__ FloatPair permlane16_swap(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, a), __builtin_bit_cast(unsigned, b),
                                                    false, false);
    const unsigned first = r[0], second = r[1];
    return {__builtin_bit_cast(float, first), __builtin_bit_cast(float, second)};
}

__device__ __forceinline__ float swap32_sum(float a, float b) {
    const FloatPair r = permlane32_swap(a, b);
    return r.first + r.second;
}

__device__ __forceinline__ float swap16_sum(float a, float b) {
    const FloatPair r = permlane16_swap(a, b);
    return r.first + r.second;
}

// Max / sum over lanes l, l ^ 16, l ^ 32, l ^ 48, result in every lane.
__device__ __forceinline__ float max_over_lane_groups(float x) {
    const FloatPair r = permlane32_swap(x, x);
    x = fmaxf(r.first, r.second);
    const FloatPair s = permlane16_swap(x, x);
    return fmaxf(s.first, s.second);
}

__device__ __forceinline__ float sum_over_lane_groups(float x) {
    x = swap32_sum(x, x);
    return swap16_sum(x, x);
}

// State j of a row, read as one 8-byte load. Callers clamp j into the row and
// mask the result, so loads are unconditional and issue back to back.
__device__ __forceinline__ float2 read_state(const float2* st, int j) {
    return __builtin_bit_cast(float2, reinterpret_cast<const uint64_t*>(st)[j]);
}

// ---------------------------------------------------------------------------
// Element types of the vector-ALU kernel. A lane moves 16 bytes per load: 4 floats.
template <typename T>
struct Elem;

template <>
struct Elem<float> {
    static constexpr int kPerLoad = 4;
    static __device__ __forceinline__ float dot(const u32x4& a, const u32x4& b) {
        const f32x4 af = __builtin_bit_cast(f32x4, a);
        const f32x4 bf = __builtin_bit_cast(f32x4, b);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = fmaf(af[i], bf[i], acc);
        return acc;
    }
    static __device__ __forceinline__ void widen(const u32x4& x, float (&f)[4]) {
        const f32x4 v = __builtin_bit_cast(f32x4, x);
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = v[i];
    }
};

// ---------------------------------------------------------------------------
// Partition kernels.
//
// Both kernels cut every partition of split_tokens tokens into kQuarters
// contiguous quarters and give each quarter of each KV head (and head tile) to
// one wave, which leaves its own max-corrected state per query head in the
// workspace: numerator [B, Hq, 4 * splits, D] and stats [B, Hq, 4 * splits, 2],
// state index 4 * split + quarter. Waves never combine with each other, so the
// kernels have no workgroup barrier on the hot path.


// A chunk's scores may exceed the running max by up to 2^kRescaleSlack before
// the accumulators are rescaled; weights then stay <= 2^8, far from overflow.
constexpr float kRescaleSlack = 8.0f;

// Stores one wave's state for its GT heads. acc[g][e] lives in the row layout
// (lanes [r*LPT, (r+1)*LPT) = token row r, dims col*EPL .. col*EPL+EPL-1) and
// has already been summed over rows into the lanes of row 0; m and l for head g
// are in lane g.
template <int D, int GT, int EPL, int LPT>
__device__ __forceinline__ void store_wave_state(const PartialParams& p, const WaveWork& w, int lane,
                                                 const float (&acc)[GT][EPL], float m, float l) {
    const int part = w.split * kQuarters + w.quarter;
    if (lane < LPT) {
        const int col = lane;
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            if (g < w.heads_here) {
                f32x4* dst = reinterpret_cast<f32x4*>(p.numerator + numerator_offset(p, w.q_row + g, part, D) + col * EPL);
#pragma unroll
                for (int e = 0; e < EPL; e += 4)
                    dst[e / 4] = f32x4{acc[g][e], acc[g][e + 1], acc[g][e + 2], acc[g][e + 3]} * p.v_scale;
            }
        }
    }
    if (lane < w.heads_here) {
        float2* st = reinterpret_cast<float2*>(p.stats + stats_offset(p, w.q_row + lane, part));
        *st = make_float2(l > 0.0f ? m : kNoToken, l);
    }
}

// Empty states (m = -FLT_MAX, l = 0: an identity of every merge) for the
// wave's quarter of the `extra` live partitions after its first one, when a
// tail item streamed several partitions as one.
__device__ __forceinline__ void store_empty_states(const PartialParams& p, const WaveWork& w, int lane, int extra) {
    if (lane >= w.heads_here) return;
    for (int e = 1; e <= extra; ++e)
        *reinterpret_cast<float2*>(p.stats + stats_offset(p, w.q_row + lane, (w.split + e) * kQuarters + w.quarter)) =
            make_float2(kNoToken, 0.0f);
}

// ---------------------------------------------------------------------------
// FP32 (and generic) partition kernel, VALU only.
//
// Lanes [r*LPT, (r+1)*LPT) hold token r of a TPL-token load (16 bytes each);
// q.k is a per-lane partial dot reduced over the LPT lanes of the row with DPP;
// every token row keeps its own online-softmax stream, combined across rows at
// the end of the wave. Chunks of NL loads stream through PD + 1 register
// buffers in fully unrolled blocks of NC chunks.
template <typename T, int D, int GT, int NL, int PD, int NC>
__global__ void __launch_bounds__(kWave * 8) partial_kernel(const PartialParams p) {
    using E = Elem<T>;
    constexpr int EPL = E::kPerLoad;
    constexpr int LPT = D / EPL;
    constexpr int TPL = kWave / LPT;
    constexpr int CT = NL * TPL;
    static_assert(TPL >= 2 && TPL <= 8 && (TPL & (TPL - 1)) == 0, "unsupported row split");

    struct Chunk {
        u32x4 k[NL];
        u32x4 v[NL];
        uint32_t live;
    };

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int row = lane / LPT;
    const int col = lane % LPT;
    const BlockCoords bc = block_coords(blockIdx.x, blockIdx.y, blockIdx.z, gridDim.x, gridDim.y);
    const PartitionRange pr = partition_range(p, bc);
    const int32_t* pages = p.table + static_cast<int64_t>(pr.b) * p.table_width;
    int window = speculative_page<TPL>(p, pr.first, pr.count, pr.qgroup, wave);
    int window_ids = pages[window_entry(p, window, lane)];
    const int len_raw = p.lengths[pr.b];
    const WaveWork w = wave_work<GT, TPL>(p, pr.b, pr.first, pr.count, pr.qgroup, bc.heads, wave, len_raw);
    if (w.dead) return;  // never read: the merge stops at the sequence's last live partition
    const T* q_base = static_cast<const T*>(p.q) + w.q_row * D;

    u32x4 qv[GT];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        qv[g] = u32x4{0u, 0u, 0u, 0u};
        if (g < w.heads_here) qv[g] = *reinterpret_cast<const u32x4*>(q_base + g * D + col * EPL);
    }
    float m[GT], l[GT], acc[GT][EPL];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        m[g] = kNoToken;
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = 0.0f;
    }
    const char* k_head = static_cast<const char*>(p.k) + static_cast<size_t>(w.kv_head) * D * sizeof(T);
    const char* v_head = static_cast<const char*>(p.v) + static_cast<size_t>(w.kv_head) * D * sizeof(T);
    // Groups with no live token are redirected to this tile's q row: always
    // mapped, finite, and the same line for every lane.
    const char* park = reinterpret_cast<const char*>(q_base);
    const uint32_t lane_bytes = static_cast<uint32_t>(col) * 16u;
    int rb = w.wb, re = w.wb;

    auto issue = [&](Chunk& ch, int c0, int ids, int win) {
        const char* kp[NL];
        const char* vp[NL];
        uint32_t off[NL];
        uint32_t live = 0;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int g = c0 + i * TPL;
            const TileSpan span = tile_span(p, g, TPL, rb, re, win);
            const int page = __builtin_amdgcn_readlane(ids, span.slot);
            const bool ok = tile_live(p, g, re, page);
            live |= static_cast<uint32_t>(ok) << i;
            const uint64_t page_off = tile_page_offset(p, ok, page);
            kp[i] = ok ? k_head + page_off : park;
            vp[i] = ok ? v_head + page_off : park;
            off[i] = token_offset(p, ok, g + row, span, lane_bytes);
        }
        ch.live = live;
#pragma unroll
        for (int i = 0; i < NL; ++i) ch.k[i] = *reinterpret_cast<const u32x4*>(kp[i] + off[i]);
#pragma unroll
        for (int i = 0; i < NL; ++i) ch.v[i] = *reinterpret_cast<const u32x4*>(vp[i] + off[i]);
        __builtin_amdgcn_sched_barrier(0);
    };

    auto consume = [&](const Chunk& ch, int c0) {
        float s[NL][GT];
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int t = c0 + i * TPL + row;
            const bool valid = (((ch.live >> i) & 1u) != 0u) & (t >= rb) & (t < re);
#pragma unroll
            for (int g = 0; g < GT; ++g) {
                const float d = group_sum<LPT>(E::dot(qv[g], ch.k[i]));
                s[i][g] = valid ? d : -INFINITY;
            }
        }
        float chunk_max[GT];
        bool grow = false;
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            float cm = s[0][g];
#pragma unroll
            for (int i = 1; i < NL; ++i) cm = fmaxf(cm, s[i][g]);
            chunk_max[g] = cm * p.scale_log2;
            grow |= chunk_max[g] > m[g] + kRescaleSlack;
        }
        if (__any(grow)) {
#pragma unroll
            for (int g = 0; g < GT; ++g) {
                const float m_new = fmaxf(m[g], chunk_max[g]);
                const float alpha = fast_exp2(m[g] - m_new);
                m[g] = m_new;
                l[g] *= alpha;
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
            }
        }
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            float sum = l[g];
#pragma unroll
            for (int i = 0; i < NL; ++i) {
                s[i][g] = fast_exp2(fmaf(s[i][g], p.scale_log2, -m[g]));
                sum += s[i][g];
            }
            l[g] = sum;
        }
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            float vf[EPL];
            E::widen(ch.v[i], vf);
#pragma unroll
            for (int g = 0; g < GT; ++g)
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(s[i][g], vf[e], acc[g][e]);
        }
    };

    for (rb = w.wb; rb < w.we; rb = re) {
        if ((rb >> p.page_shift) != window) {
            window = rb >> p.page_shift;
            window_ids = pages[window_entry(p, window, lane)];
        }
        re = min(w.we, (window + kWave) << p.page_shift);
        for (int s0 = rb & ~(TPL - 1); s0 < re; s0 += NC * CT) {
            Chunk buf[PD + 1];
#pragma unroll
            for (int n = 0; n < PD; ++n) issue(buf[n], s0 + n * CT, window_ids, window);
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                if (s0 + n * CT >= re) break;
                if (n + PD < NC) issue(buf[(n + PD) % (PD + 1)], s0 + (n + PD) * CT, window_ids, window);
                consume(buf[n % (PD + 1)], s0 + n * CT);
            }
        }
    }

    // Combine the TPL token-row streams (lanes LPT, 2*LPT, ... apart).
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        float mw = m[g];
#pragma unroll
        for (int x = LPT; x < kWave; x <<= 1) mw = fmaxf(mw, __shfl_xor(mw, x));
        const float f = l[g] > 0.0f ? fast_exp2(m[g] - mw) : 0.0f;
        float lw = l[g] * f;
#pragma unroll
        for (int x = LPT; x < kWave; x <<= 1) lw += __shfl_xor(lw, x);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float a = acc[g][e] * f;
#pragma unroll
            for (int x = LPT; x < kWave; x <<= 1) a += __shfl_xor(a, x);
            acc[g][e] = a;
        }
        m[g] = mw;
        l[g] = lw;
    }
    // Lane g needs head g's (m, l): every lane holds every head's values.
    float m_lane = m[0], l_lane = l[0];
#pragma unroll
    for (int g = 1; g < GT; ++g) {
        m_lane = lane == g ? m[g] : m_lane;
        l_lane = lane == g ? l[g] : l_lane;
    }
    store_wave_state<D, GT, EPL, LPT>(p, w, lane, acc, m_lane, l_lane);
    store_empty_states(p, w, lane, extra_live_partitions(p, pr.first, pr.count, len_raw));
}

// ---------------------------------------------------------------------------
// 16-bit partition kernel (q in FP16 or BF16; K/V in the same type or in FP8):
// q.K^T and P.V both on the matrix cores.
//
// A 16-token tile is scored with D/32 v_mfma_f32_16x16x32_{f16,bf16}: K in the
// A layout (lane l holds 8 consecutive dims, [32 s + 8 (l / 16), +8) of k-step
// s, of tile token sigma(l % 16)), q in the B layout (lane l: query head
// l % 16, zero past the group). K is loaded as whole token rows (16 bytes per
// lane, full cache lines, like V) and reaches the A layout through a per-wave
// LDS tile. With sigma(r) = r / 4 + 4 (r % 4) the result
// leaves lane l with head n = l % 16 and tokens g, g + 4, g + 8, g + 12 of the
// tile (g = l / 16): exactly the A operand of v_mfma_f32_16x16x16_{f16,bf16}
// for P (row = head, k = 4 g + e <-> token g + 4 e), so the weights never
// leave their lanes. V is loaded in the row layout -- load e covers tokens
// 4 e .. 4 e + 3, lanes [16 r, 16 r + 16) token 4 e + r, VH consecutive dims
// per lane -- so lane (g, n) holds tokens g + 4 e of dims n VH .. n VH + VH - 1,
// and element j of its four V loads is the B operand of MFMA block j (column
// n <-> dim n VH + j). P is split into high and low parts of the compute type
// (two MFMAs per block), which keeps the weights exact to about 2^-22 (FP16)
// or 2^-17 (BF16) relative. Each (head, dim) sum lives in exactly one lane:
// lane (g, n) ends with heads 4 g .. 4 g + 3 of dims n VH .. n VH + VH - 1,
// stored directly. One running max per head is shared by the wave, with lazy
// rescaling as in the FP32 kernel.
//
// FP8 K/V (OCP e4m3 or e5m2) are loaded as bytes and converted to the compute
// type after they arrive; both formats convert exactly. The per-tensor scales
// cost nothing per element: k_scale is folded into the softmax scale and
// v_scale into the stored numerator.

enum KvFormat { kKvNative = 0, kKvE4M3 = 1, kKvE5M2 = 2 };


// N stored words from src. kStream marks 16-byte loads non-temporal (see
// plan_mfma for when that is used).
template <int N, bool kStream>
__device__ __forceinline__ void load_words(const char* src, uint32_t (&w)[N]) {
    if constexpr (N == 4) {
        const u32x4 x = kStream ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src))
                                : *reinterpret_cast<const u32x4*>(src);
        w[0] = x[0];
        w[1] = x[1];
        w[2] = x[2];
        w[3] = x[3];
    } else if constexpr (N == 2) {
        const u32x2 x = *reinterpret_cast<const u32x2*>(src);
        w[0] = x[0];
        w[1] = x[1];
    } else {
        w[0] = *reinterpret_cast<const uint32_t*>(src);
    }
}

// Matrix-core operations and conversions of one 16-bit compute type.
template <typename QT>
struct Compute;

template <>
struct Compute<_Float16> {
    static __device__ __forceinline__ f32x4 qk(const u32x4& a, const u32x4& b, const f32x4& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
    }
    static __device__ __forceinline__ f32x4 pv(const u32x2& a, const u32x2& b, const f32x4& c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0,
                                                     0, 0);
    }
    // Nearest 16-bit value of x, and that value back as FP32.
    static __device__ __forceinline__ uint16_t round(float x, float& back) {
        const _Float16 h = static_cast<_Float16>(x);
        back = static_cast<float>(h);
        return __builtin_bit_cast(uint16_t, h);
    }
    // Bytes 2 HIGH, 2 HIGH + 1 of an FP8 word as a packed pair (exact).
    template <int KVF, bool HIGH>
    static __device__ __forceinline__ uint32_t from_fp8(uint32_t word) {
        f16x2 h;
        if constexpr (KVF == kKvE4M3) h = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(word, 1.0f, HIGH);
        else h = __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(word, 1.0f, HIGH);
        return __builtin_bit_cast(uint32_t, h);
    }
};

template <>
struct Compute<__bf16> {
    static __device__ __forceinline__ f32x4 qk(const u32x4& a, const u32x4& b, const f32x4& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 pv(const u32x2& a, const u32x2& b, const f32x4& c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                         0, 0, 0);
    }
    static __device__ __forceinline__ uint16_t round(float x, float& back) {
        const __bf16 h = static_cast<__bf16>(x);
        back = static_cast<float>(h);
        return __builtin_bit_cast(uint16_t, h);
    }
    template <int KVF, bool HIGH>
    static __device__ __forceinline__ uint32_t from_fp8(uint32_t word) {
        f32x2 f;
        if constexpr (KVF == kKvE4M3) f = __builtin_amdgcn_cvt_pk_f32_fp8(word, HIGH);
        else f = __builtin_amdgcn_cvt_pk_f32_bf8(word, HIGH);
        const float f0 = f[0], f1 = f[1];  // FP8 values are exact in BF16: keep the top halves
        return (__builtin_bit_cast(uint32_t, f0) >> 16) | (__builtin_bit_cast(uint32_t, f1) & 0xFFFF0000u);
    }
};

// N stored words of K or V as compute-type pairs (2 N words for FP8).
template <typename QT, int KVF, int N>
__device__ __forceinline__ void to_compute(const uint32_t (&raw)[N], uint32_t (&out)[KVF == kKvNative ? N : 2 * N]) {
    if constexpr (KVF == kKvNative) {
#pragma unroll
        for (int i = 0; i < N; ++i) out[i] = raw[i];
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            out[2 * i] = Compute<QT>::template from_fp8<KVF, false>(raw[i]);
            out[2 * i + 1] = Compute<QT>::template from_fp8<KVF, true>(raw[i]);
        }
    }
}

// Element j of each of the four V loads (VH elements per load, as VH / 2
// packed words), packed as an MFMA operand (k = load index).
template <int VH>
__device__ __forceinline__ u32x2 v_operand(const uint32_t (&v)[4][VH / 2], int j) {
    const uint32_t d0 = v[0][j / 2], d1 = v[1][j / 2], d2 = v[2][j / 2], d3 = v[3][j / 2];
    if (j % 2 == 0) return u32x2{(d0 & 0xFFFFu) | (d1 << 16), (d2 & 0xFFFFu) | (d3 << 16)};
    return u32x2{(d0 >> 16) | (d1 & 0xFFFF0000u), (d2 >> 16) | (d3 & 0xFFFF0000u)};
}

// LDS slot of the quarter combine: one quarter's state of one (KV head,
// head tile) -- per-head max and denominator, and the accumulator in the
// lanes' own layout (acc[j] of lane l at acc[j][l]).
template <int VH>
struct CombineSlot {
    float m[16];
    float l[16];
    f32x4 acc[VH][kWave];
};

// kStream: which 16-byte loads are non-temporal (see plan_mfma):
// 0 none, 1 V (and FP8 K, whose V loads are 8-byte), 2 K and V.
template <typename QT, int KVF, int D, int GT, int PD, int NC, int kStream, bool kCombine>
__global__ void __launch_bounds__(kWave * 8) partial_mfma_kernel(const PartialParams p) {
    using C = Compute<QT>;
    constexpr int ES = KVF == kKvNative ? 2 : 1;  // stored bytes per K/V element
    constexpr int KS = D / 32;                    // q.K^T k-steps (K loads) per tile
    constexpr int VH = D / 16;                    // V elements per lane per load = P.V MFMA blocks
    constexpr int VI = 4;                         // V loads per tile
    constexpr int VW = VH * ES / 4;               // stored words per V load
    static_assert(GT <= 16, "one MFMA column block holds at most 16 query heads");

    // K is loaded whole rows at a time (KR lanes x 16 bytes per token, TK
    // tokens per load, KL loads per tile) and turned into the q.K^T operand
    // layout through a per-wave LDS tile. Its rows are padded by the size of
    // one operand read (16 bytes for 16-bit K, 8 for FP8), so the transposed
    // reads of 16 different rows fall in distinct banks.
    constexpr bool kStreamK = kStream == 2 || (kStream == 1 && KVF != kKvNative);
    constexpr int KR = D * ES / 16;
    constexpr int TK = kWave / KR;
    constexpr int KL = kTileTokens / TK;
    constexpr int kStageRow = mfma_stage_bytes(D, ES) / kTileTokens;
    static_assert(TK <= kTileTokens && kTileTokens % TK == 0, "whole row loads per tile");
    // Dynamic LDS: the waves' K tiles, then (kCombine) the quarter-combine
    // slots, [waves / qw][qw - 1] CombineSlot<VH>; sized by the launch.
    extern __shared__ __attribute__((aligned(16))) char lds[];
    char* const k_stage = lds;
    char* const combine_lds = lds + mfma_stage_bytes(D, ES) * (blockDim.x / kWave);

    struct Tile {
        uint32_t k[KL][4];
        uint32_t v[VI][VW];
        uint32_t live;
    };

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int n = lane % 16;  // head (q.K^T, P) / column (P.V)
    const int g = lane / 16;  // lane group: tokens g + 4 e
    const BlockCoords bc = block_coords(blockIdx.x, blockIdx.y, blockIdx.z, gridDim.x, gridDim.y);
    const PartitionRange pr = partition_range(p, bc);
    const int32_t* pages = p.table + static_cast<int64_t>(pr.b) * p.table_width;
    int window = speculative_page<kTileTokens>(p, pr.first, pr.count, pr.qgroup, wave);
    int window_ids = pages[window_entry(p, window, lane)];
    const int len_raw = p.lengths[pr.b];
    const WaveWork w = wave_work<GT, kTileTokens>(p, pr.b, pr.first, pr.count, pr.qgroup, bc.heads, wave, len_raw);
    if (w.dead) return;  // never read: the merge stops at the sequence's last live partition
    const char* q_row = static_cast<const char*>(p.q) + w.q_row * D * 2;

    u32x4 qb[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        qb[s] = u32x4{0u, 0u, 0u, 0u};
        if (n < w.heads_here) qb[s] = *reinterpret_cast<const u32x4*>(q_row + (n * D + 32 * s + 8 * g) * 2);
    }

    float m_head = kNoToken;  // running max (log2 units) of head n, equal in all lane groups
    float l_part = 0.0f;      // this lane's share of head n's denominator
    f32x4 acc[VH];            // acc[j][i]: head 4 g + i, dim n VH + j
#pragma unroll
    for (int j = 0; j < VH; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const char* k_head = static_cast<const char*>(p.k) + static_cast<size_t>(w.kv_head) * D * ES;
    const char* v_head = static_cast<const char*>(p.v) + static_cast<size_t>(w.kv_head) * D * ES;
    const char* park = q_row;  // dead tiles read the wave's own q row: mapped, D * 2 bytes
    const uint32_t v_lane_bytes = static_cast<uint32_t>(n) * VH * ES;
    const int k_row_token = k_token_of_row(n);
    int rb = w.wb, re = w.wb;

    auto issue = [&](Tile& tl, int t0, int ids, int win) {
        const TileSpan span = tile_span(p, t0, kTileTokens, rb, re, win);
        const int page = __builtin_amdgcn_readlane(ids, span.slot);
        const bool ok = tile_live(p, t0, re, page);
        tl.live = ok;
        const uint64_t page_off = tile_page_offset(p, ok, page);
        const char* kp = ok ? k_head + page_off : park;
        const char* vp = ok ? v_head + page_off : park;
        const uint32_t k_lane_bytes = static_cast<uint32_t>(lane % KR) * 16u;
#pragma unroll
        for (int s = 0; s < KL; ++s)
            load_words<4, kStreamK>(kp + token_offset(p, ok, t0 + TK * s + lane / KR, span, k_lane_bytes), tl.k[s]);
#pragma unroll
        for (int e = 0; e < VI; ++e)
            load_words<VW, (kStream >= 1)>(vp + token_offset(p, ok, t0 + 4 * e + g, span, v_lane_bytes), tl.v[e]);
        __builtin_amdgcn_sched_barrier(0);
    };

    auto consume = [&](const Tile& tl, int t0) {
        f32x4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
        char* stage = k_stage + wave * (kTileTokens * kStageRow);
        __builtin_amdgcn_wave_barrier();  // the previous tile's reads are issued before these writes
#pragma unroll
        for (int s = 0; s < KL; ++s) {
            char* dst = stage + (TK * s + lane / KR) * kStageRow + (lane % KR) * 16;
            if constexpr (kStageRow % 16 == 0) {
                *reinterpret_cast<u32x4*>(dst) = u32x4{tl.k[s][0], tl.k[s][1], tl.k[s][2], tl.k[s][3]};
            } else {  // FP8 rows are 8-byte aligned
                reinterpret_cast<u32x2*>(dst)[0] = u32x2{tl.k[s][0], tl.k[s][1]};
                reinterpret_cast<u32x2*>(dst)[1] = u32x2{tl.k[s][2], tl.k[s][3]};
            }
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const char* src = stage + k_row_token * kStageRow + (32 * s + 8 * g) * ES;
            if constexpr (KVF == kKvNative) {
                sc = C::qk(*reinterpret_cast<const u32x4*>(src), qb[s], sc);
            } else {
                const u32x2 raw2 = *reinterpret_cast<const u32x2*>(src);
                const uint32_t raw[2] = {raw2[0], raw2[1]};
                uint32_t kq[4];
                to_compute<QT, KVF, 2>(raw, kq);
                sc = C::qk(u32x4{kq[0], kq[1], kq[2], kq[3]}, qb[s], sc);
            }
        }
        float x[4];
        float mx = -INFINITY;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = t0 + g + 4 * e;
            const bool valid = (tl.live != 0u) & (t >= rb) & (t < re);
            x[e] = valid ? sc[e] : -INFINITY;
            mx = fmaxf(mx, x[e]);
        }
        const float tile_max = max_over_lane_groups(mx) * p.scale_log2;
        if (__any((n < GT) & (tile_max > m_head + kRescaleSlack))) {
            const float m_new = fmaxf(m_head, tile_max);
            const float alpha = fast_exp2(m_head - m_new);
            m_head = m_new;
            l_part *= alpha;
            // acc[.][i] belongs to head 4 g + i, whose factor lives in lane 4 g + i.
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float a = __shfl(alpha, 4 * g + i);
#pragma unroll
                for (int j = 0; j < VH; ++j) acc[j][i] *= a;
            }
        }
        uint16_t hi_bits[4], lo_bits[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float wt = fast_exp2(fmaf(x[e], p.scale_log2, -m_head));
            l_part += wt;
            float back, unused;
            hi_bits[e] = C::round(wt, back);
            lo_bits[e] = C::round(wt - back, unused);
        }
        const u32x2 p_hi = {hi_bits[0] | (static_cast<uint32_t>(hi_bits[1]) << 16),
                            hi_bits[2] | (static_cast<uint32_t>(hi_bits[3]) << 16)};
        const u32x2 p_lo = {lo_bits[0] | (static_cast<uint32_t>(lo_bits[1]) << 16),
                            lo_bits[2] | (static_cast<uint32_t>(lo_bits[3]) << 16)};
        uint32_t vq[VI][VH / 2];
#pragma unroll
        for (int e = 0; e < VI; ++e) {
            uint32_t raw[VW];
#pragma unroll
            for (int i = 0; i < VW; ++i) raw[i] = (KVF == kKvNative || tl.live) ? tl.v[e][i] : 0u;  // FP8 park bytes may decode to NaN
            to_compute<QT, KVF, VW>(raw, vq[e]);
        }
#pragma unroll
        for (int j = 0; j < VH; ++j) acc[j] = C::pv(p_hi, v_operand<VH>(vq, j), acc[j]);
#pragma unroll
        for (int j = 0; j < VH; ++j) acc[j] = C::pv(p_lo, v_operand<VH>(vq, j), acc[j]);
    };

    for (rb = w.wb; rb < w.we; rb = re) {
        if ((rb >> p.page_shift) != window) {
            window = rb >> p.page_shift;
            window_ids = pages[window_entry(p, window, lane)];
        }
        re = min(w.we, (window + kWave) << p.page_shift);
        for (int s0 = rb & ~(kTileTokens - 1); s0 < re; s0 += NC * kTileTokens) {
            Tile buf[PD + 1];
#pragma unroll
            for (int n0 = 0; n0 < PD; ++n0) issue(buf[n0], s0 + n0 * kTileTokens, window_ids, window);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                if (s0 + c * kTileTokens >= re) break;
                if (c + PD < NC) issue(buf[(c + PD) % (PD + 1)], s0 + (c + PD) * kTileTokens, window_ids, window);
                consume(buf[c % (PD + 1)], s0 + c * kTileTokens);
            }
        }
    }

    // Lane (g, n) holds heads 4 g + i of dims n VH .. n VH + VH - 1; the
    // denominator of head n is summed over the four lane groups.
    float l_head = sum_over_lane_groups(l_part);
    const int part = w.split * kQuarters + w.quarter;
    store_empty_states(p, w, lane, extra_live_partitions(p, pr.first, pr.count, len_raw));
    if constexpr (kCombine) {
        // The workgroup's qw quarters of one (KV head, head tile) -- waves
        // wave - wave % qw onwards, all of one partition, so all live or all
        // gone above -- become one state: quarters 1 .. qw - 1 leave theirs in
        // LDS, and after one barrier the first quarter folds them into its own
        // in quarter order (the merge's max-corrected sum) and stores the
        // result. The other quarters' slots get the empty state (l = 0), which
        // every merge of the four-states-per-partition layout reads as an
        // identity.
        const int qw = p.quarters_per_wg;
        const int qq = wave % qw;
        CombineSlot<VH>* slots = reinterpret_cast<CombineSlot<VH>*>(combine_lds) + wave / qw * (qw - 1);
        if (qq != 0) {
            CombineSlot<VH>* slot = slots + (qq - 1);
            if (lane < 16) {
                slot->m[n] = m_head;
                slot->l[n] = l_head;
            }
#pragma unroll
            for (int j = 0; j < VH; ++j) slot->acc[j][lane] = acc[j];
            if (lane < w.heads_here)
                *reinterpret_cast<float2*>(p.stats + stats_offset(p, w.q_row + lane, part)) =
                    make_float2(kNoToken, 0.0f);
        }
        __syncthreads();
        if (qq != 0) return;
        for (int s = 0; s < qw - 1; ++s) {
            const CombineSlot<VH>* slot = slots + s;
            f32x4 in[VH];
#pragma unroll
            for (int j = 0; j < VH; ++j) in[j] = slot->acc[j][lane];
            const float m_in = slot->m[n];
            const float m_new = fmaxf(m_head, m_in);
            const float f_in = fast_exp2(m_in - m_new);  // 0 for an empty state, 1 if both are empty
            const float f_own = fast_exp2(m_head - m_new);
            l_head = fmaf(f_in, slot->l[n], f_own * l_head);
            m_head = m_new;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float a_in = __shfl(f_in, 4 * g + i);  // factors of head 4 g + i
                const float a_own = __shfl(f_own, 4 * g + i);
#pragma unroll
                for (int j = 0; j < VH; ++j) acc[j][i] = fmaf(a_in, in[j][i], a_own * acc[j][i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int h = 4 * g + i;
        if (h < w.heads_here) {
            f32x4* dst = reinterpret_cast<f32x4*>(p.numerator + numerator_offset(p, w.q_row + h, part, D) + n * VH);
#pragma unroll
            for (int j = 0; j < VH; j += 4)
                dst[j / 4] = f32x4{acc[j][i], acc[j + 1][i], acc[j + 2][i], acc[j + 3][i]} * p.v_scale;
        }
    }
    if (lane < w.heads_here) {
        float2* st = reinterpret_cast<float2*>(p.stats + stats_offset(p, w.q_row + lane, part));
        *st = make_float2(l_head > 0.0f ? m_head : kNoToken, l_head);
    }
}

// ---------------------------------------------------------------------------
// Merge kernels: the max-corrected combination of a (sequence, query head)
// row's live states. A state with l == 0 is the identity (decode.cu:94-107).
// Two ways to form the weights, as the reference's two merges:
//   serial: every wave scans all states itself for the max and the denominator
//           (lanes share the scan, reduced with DPP), and each lane recomputes
//           the weight of the states it accumulates; no weight storage.
//   shared: the workgroup forms each state's weight once, into LDS
//           (4 bytes per state, hence the PD_SHARED_MERGE_MAX_PARTS bound).

constexpr int kMergeThreads = 256;

// States of row b to merge: per_part per partition up to the last one
// holding a token of the sequence (none for an empty sequence), capped at the
// row's states. Partitions past the end are never written and never read.
__device__ __forceinline__ int live_parts(const int32_t* lengths, int b, int split_tokens, int capacity,
                                          int per_part, int states) {
    const int len = max(0, min(lengths[b], capacity));  // decode.cu:42-44
    const int64_t live = (static_cast<int64_t>(len) + split_tokens - 1) / split_tokens;
    return static_cast<int>(min<int64_t>(per_part * live, states));
}

struct MergeParams {
    const float* numerator;  // [B, Hq, parts, D]
    const float* stats;      // [B, Hq, parts, 2]
    float* out;              // [B, Hq, D]
    const int32_t* lengths;  // [B]
    int parts;               // allocated states per row (4 * splits)
    int stride_shift;        // read every (1 << stride_shift)-th state: 0, or log2 of the combined quarters
    int query_heads;
    int split_tokens;
    int capacity;            // table_width * page_size
};

// merge_cols_kernel: a row's D columns are cut into 128-byte chunks and each
// (row, chunk) is one 256-lane workgroup, so D / 32 workgroups read a row's
// states together. Lane t owns the 16-byte column t % 8 of the chunk for the
// states j == t / 8 (mod 32) and issues up to NB of those loads in one round
// (NB = 8 or 32: 256 or 1024 states), together with the first round of the
// statistics scan, which is kept in registers for the denominator. Longer rows
// repeat both rounds. All loads use clamped indexes and are masked afterwards,
// so they issue back to back.
constexpr int kMergeChunk = 32;                                   // floats per column chunk
constexpr int kMergeColLanes = kMergeChunk / 4;                   // lanes per state slice
constexpr int kMergeColGroups = kMergeThreads / kMergeColLanes;  // state groups per workgroup
constexpr int kMergeColBatchShort = 8;                            // numerator loads per lane per round
constexpr int kMergeColBatchLong = 32;
constexpr int kOptimisticRounds = 2;  // first-round loads issued before the live count (64 states)

template <int D, bool kSharedWeights, int NB>
__global__ void __launch_bounds__(kMergeThreads) merge_cols_kernel(const MergeParams mp) {
    constexpr int TPR = kMergeColLanes;
    constexpr int PG = kMergeColGroups;
    constexpr int SU = NB / 2;  // (m, l) loads per scanning lane per round: a serial wave scans NB * PG states
    constexpr int kWaves = kMergeThreads / kWave;
    constexpr int kScan = kSharedWeights ? kMergeThreads : kWave;  // lanes sharing the state scan
    constexpr int kScanRound = SU * kScan;
    static_assert(D % kMergeChunk == 0, "whole chunks");
    extern __shared__ float weight[];  // [parts], shared variant only
    __shared__ f32x4 column_sum[PG][TPR];
    __shared__ float wave_partial[2][kWaves];
    const int b = blockIdx.y;
    const int64_t row = static_cast<int64_t>(b) * mp.query_heads + blockIdx.x;
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
    const float2* st = reinterpret_cast<const float2*>(mp.stats) + row * mp.parts;
    const f32x4* num = reinterpret_cast<const f32x4*>(mp.numerator + row * mp.parts * D + chunk * kMergeChunk) + col;
    const int64_t num_step = static_cast<int64_t>(D / 4) << shift;

    auto rounds_from = [&](int base, int limit) { return min(NB, (limit - base + PG - 1) / PG); };
    f32x4 buf[NB];
    float2 own[NB];
    // Loads k0 <= k < k1 (uniform bounds) of the round starting at state base.
    auto load_rounds = [&](int base, int k0, int k1) {
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            if (k >= k0 && k < k1) {
                const int j = min(base + pg + k * PG, last);
                buf[k] = num[j * num_step];
                if constexpr (!kSharedWeights) own[k] = read_state(st, j << shift);
            }
        }
    };
    // The first kOptimisticRounds loads are issued for the allocated row
    // before the live count arrives (it comes with them) and masked
    // afterwards; the rest of the round covers live states only, so a ragged
    // batch does not read the states past its sequences' ends.
    const int optimistic = min(kOptimisticRounds, rounds_from(0, parts));
    load_rounds(0, 0, optimistic);
    const int live = live_parts(mp.lengths, b, mp.split_tokens, mp.capacity, kQuarters >> shift, parts);
    load_rounds(0, optimistic, rounds_from(0, live));

    auto scan_round = [&](int base, int limit, float2 (&sv)[SU]) {
#pragma unroll
        for (int i = 0; i < SU; ++i) {
            if (base + i * kScan < limit) sv[i] = read_state(st, min(base + scan0 + i * kScan, last) << shift);
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
    float2 first[SU];
    scan_round(0, parts, first);
    float mx = round_max(first, 0, parts, kNoToken);
    for (int base = kScanRound; base < live; base += kScanRound) {
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
    accumulate_den(first, 0, parts);
    for (int base = kScanRound; base < live; base += kScanRound) {
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
    if (t < kMergeChunk) {
        float sum = 0.0f;
#pragma unroll
        for (int g = 0; g < PG; ++g) sum += reinterpret_cast<const float*>(column_sum[g])[t];
        mp.out[row * D + chunk * kMergeChunk + t] = den > 0.0f ? sum / den : 0.0f;
    }
}

// Small rows: one wave per (sequence, query head) row, four rows per
// workgroup, no barriers. Lane l owns column l % TPR of the states
// j == l / TPR (mod PGW) and lane j reads state j's (m, l) for the row
// maximum and denominator, reduced with DPP. The shared variant forms each
// state's weight once, in lane j, and broadcasts it with a cross-lane read;
// the serial variant has every lane recompute the weights it uses. The PGW
// column sums meet through permlane swaps. Used when a row's allocated states
// fit in kMergeWaveBatch loads per lane (at most 64 states); all loads are
// issued at once and masked with the live count.
constexpr int kMergeWaveBatch = 8;
constexpr int kMergeRowsMin = 256;  // rows (sequences x query heads) from which merge_rows takes rows of > 2 rounds
constexpr int kMergeRowsPerGroup = 4;

template <int D>
constexpr int merge_wave_max_parts() { return kMergeWaveBatch * (kWave / (D / 4)); }

template <int D, bool kSharedWeights>
__global__ void __launch_bounds__(kWave * kMergeRowsPerGroup) merge_rows_kernel(const MergeParams mp) {
    constexpr int TPR = D / 4;        // lanes per state row
    constexpr int PGW = kWave / TPR;  // state groups per wave (2 or 4)
    constexpr int NB = kMergeWaveBatch;
    static_assert(merge_wave_max_parts<D>() <= kWave, "one state per lane for the statistics");
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const int h = blockIdx.x * kMergeRowsPerGroup + wave;
    if (h >= mp.query_heads) return;  // whole wave; nothing below synchronises across waves
    const int b = blockIdx.y;
    const int64_t row = static_cast<int64_t>(b) * mp.query_heads + h;
    const int shift = mp.stride_shift;
    const int parts = mp.parts >> shift;  // states read: j <-> allocated state j << shift
    const int col = lane % TPR;
    const int pg = lane / TPR;
    const int last = parts - 1;
    const float2* st = reinterpret_cast<const float2*>(mp.stats) + row * mp.parts;
    const f32x4* num = reinterpret_cast<const f32x4*>(mp.numerator + row * mp.parts * D) + col;
    const int rounds = (parts + PGW - 1) / PGW;  // uniform, <= NB
    const int live = live_parts(mp.lengths, b, mp.split_tokens, mp.capacity, kQuarters >> shift, parts);

    f32x4 buf[NB];
    float2 own[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        if (k < rounds) {
            const int j = min(pg + k * PGW, last);
            buf[k] = num[(static_cast<int64_t>(j) << shift) * TPR];
            if constexpr (!kSharedWeights) own[k] = read_state(st, j << shift);
        }
    }
    const float2 mine = read_state(st, min(lane, last) << shift);
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

struct AppendParams {
    const char* k_new;
    const char* v_new;
    const int32_t* table;
    const int32_t* positions;  // explicit variant: first position per sequence
    int32_t* lengths;          // advance variant: positions in, advanced lengths out
    char* k_cache;
    char* v_cache;
    int tokens;
    int table_width;
    int page_shift;
    int physical_pages;
    int64_t capacity;          // positions [0, capacity) may be written: the table's, or less (advance variant)
    uint32_t row_bytes;        // kv_heads * head_dim * element size
};

// Physical row of logical position pos, or -1 if pos is outside
// [0, capacity) or its page id is outside [0, physical_pages).
__device__ __forceinline__ int64_t cache_row(const AppendParams& a, const int32_t* pages, int64_t pos) {
    if (pos < 0 || pos >= a.capacity) return -1;
    const int page = pages[pos >> a.page_shift];
    if (static_cast<uint32_t>(page) >= static_cast<uint32_t>(a.physical_pages)) return -1;
    return (static_cast<int64_t>(page) << a.page_shift) + (pos & ((1 << a.page_shift) - 1));
}

__device__ __forceinline__ void copy_token_row(const AppendParams& a, int64_t src_row, int64_t dst_row) {
    const u32x4* ks = reinterpret_cast<const u32x4*>(a.k_new + src_row * a.row_bytes);
    const u32x4* vs = reinterpret_cast<const u32x4*>(a.v_new + src_row * a.row_bytes);
    u32x4* kd = reinterpret_cast<u32x4*>(a.k_cache + dst_row * a.row_bytes);
    u32x4* vd = reinterpret_cast<u32x4*>(a.v_cache + dst_row * a.row_bytes);
    const uint32_t chunks = a.row_bytes / 16u;
    for (uint32_t c = threadIdx.x; c < chunks; c += blockDim.x) {
        kd[c] = ks[c];
        vd[c] = vs[c];
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
    copy_token_row(a, static_cast<int64_t>(b) * a.tokens + j, dst);
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
    for (int j = 0; j < a.tokens; ++j) copy_token_row(a, static_cast<int64_t>(b) * a.tokens + j, cache_row(a, pages, base + j));
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
// max_context) is written empty and raises *overflow. Page ids are not
// checked here: the partition kernel skips ids outside [0, physical_pages).
struct CsrParams {
    const int32_t* indptr;
    const int32_t* indices;
    const int32_t* last_page_len;
    int32_t* table;
    int32_t* lengths;
    int32_t* overflow;  // may be null
    int table_width;
    int page_size;
    int max_context;
};

__global__ void __launch_bounds__(256) table_from_csr_kernel(const CsrParams c) {
    const int b = blockIdx.x;
    const int64_t begin = c.indptr[b];
    const int64_t n = static_cast<int64_t>(c.indptr[b + 1]) - begin;
    const int last = n > 0 ? c.last_page_len[b] : 0;
    const int64_t length = n > 0 ? (n - 1) * c.page_size + last : 0;
    const bool fits = n >= 0 && n <= c.table_width && (n == 0 || (last >= 1 && last <= c.page_size)) &&
                      length <= c.max_context;
    const int64_t live = fits ? n : 0;
    int32_t* row = c.table + static_cast<int64_t>(b) * c.table_width;
    for (int i = threadIdx.x; i < c.table_width; i += blockDim.x) row[i] = i < live ? c.indices[begin + i] : -1;
    if (threadIdx.x == 0) {
        c.lengths[b] = fits ? static_cast<int32_t>(length) : 0;
        if (!fits && c.overflow != nullptr) *c.overflow = 1;
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

int launch_status() { return hipGetLastError() == hipSuccess ? PD_OK : PD_ERR_LAUNCH; }

// FP32 kernel: 16-byte loads of K (and of V) per lane per chunk, chunks in
// flight ahead of the one being consumed, chunks per straight-line block.
constexpr int kFp32ChunkLoads = 1;
constexpr int kFp32Prefetch = 4;
constexpr int kFp32BlockChunks = 16;
// Matrix-core kernel: 16-token tiles issued ahead of the one being consumed,
// and tiles per straight-line block (with 2 and 2, each block's two tiles are
// requested together and consumed in order). Short blocks keep the kernel's
// code small: with 8 waves per CU running through cold straight-line code,
// instruction fetch is on the critical path (two-tile blocks measured 1 us
// faster per Llama-3-8B-shape call than eight-tile blocks, same loads).
constexpr int kMfmaPrefetch = 2;
constexpr int kMfmaBlock = 2;

// Compute units of the current device, read once per device.
int device_compute_units() {
    static std::atomic<int> cached[64];
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 256;
    int cus = cached[device].load(std::memory_order_relaxed);
    if (cus == 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0)
            cus = 256;  // MI355X
        cached[device].store(cus, std::memory_order_relaxed);
    }
    return cus;
}

dim3 to_dim3(const Grid& g) { return dim3(g.x, g.y, g.z); }

// Launches the matrix-core kernel planned by plan_mfma (head tile GT, stream
// mode and quarter combine chosen there).
template <typename QT, int KVF, int D, int GT>
int launch_mfma(const PartialParams& prm, int kv_heads, hipStream_t stream) {
    static_assert(sizeof(CombineSlot<D / 16>) == 2 * 16 * 4 + (D / 16) * kWave * 16, "combine_slot_bytes");
    const dim3 grid = to_dim3(partial_grid(prm, kv_heads));
    const dim3 block(partial_threads(prm));
    const size_t lds = static_cast<size_t>(mfma_lds_bytes(prm, D, KVF == kKvNative ? 2 : 1));
    constexpr int kPD = kMfmaPrefetch, kNC = kMfmaBlock;
#define PD_LAUNCH_MFMA(MODE, COMBINE)                                                                             \
    hipLaunchKernelGGL((partial_mfma_kernel<QT, KVF, D, GT, kPD, kNC, MODE, COMBINE>), grid, block, lds, stream, prm)
    if constexpr (KVF == kKvNative) {
        if (prm.stream_mode == 2) {
            if (prm.combine) PD_LAUNCH_MFMA(2, true);
            else PD_LAUNCH_MFMA(2, false);
            return launch_status();
        }
    }
    if (prm.stream_mode >= 1) {
        if (prm.combine) PD_LAUNCH_MFMA(1, true);
        else PD_LAUNCH_MFMA(1, false);
    } else {
        if (prm.combine) PD_LAUNCH_MFMA(0, true);
        else PD_LAUNCH_MFMA(0, false);
    }
#undef PD_LAUNCH_MFMA
    return launch_status();
}

template <int D, int GT>
int launch_fp32(const PartialParams& prm, int kv_heads, hipStream_t stream) {
    hipLaunchKernelGGL((partial_kernel<float, D, GT, kFp32ChunkLoads, kFp32Prefetch, kFp32BlockChunks>),
                       to_dim3(partial_grid(prm, kv_heads)), dim3(partial_threads(prm)), 0, stream, prm);
    return launch_status();
}

template <typename QT, int KVF, int D>
int dispatch_mfma(PartialParams& prm, int kv_heads, hipStream_t stream) {
    plan_mfma(prm, kv_heads, device_compute_units());
    switch (prm.head_tile) {
        case 1: return launch_mfma<QT, KVF, D, 1>(prm, kv_heads, stream);
        case 2: return launch_mfma<QT, KVF, D, 2>(prm, kv_heads, stream);
        case 4: return launch_mfma<QT, KVF, D, 4>(prm, kv_heads, stream);
        case 8: return launch_mfma<QT, KVF, D, 8>(prm, kv_heads, stream);
        default: return launch_mfma<QT, KVF, D, 16>(prm, kv_heads, stream);
    }
}

template <int D>
int dispatch_fp32(PartialParams& prm, int kv_heads, hipStream_t stream) {
    plan_fp32(prm, kv_heads);
    switch (prm.head_tile) {
        case 1: return launch_fp32<D, 1>(prm, kv_heads, stream);
        case 2: return launch_fp32<D, 2>(prm, kv_heads, stream);
        case 4: return launch_fp32<D, 4>(prm, kv_heads, stream);
        default: return launch_fp32<D, 8>(prm, kv_heads, stream);
    }
}

template <typename QT, int D>
int dispatch_kv(PartialParams& prm, int kv_dtype, int kv_heads, hipStream_t stream) {
    switch (kv_dtype) {
        case PD_DTYPE_FP8_E4M3: return dispatch_mfma<QT, kKvE4M3, D>(prm, kv_heads, stream);
        case PD_DTYPE_FP8_E5M2: return dispatch_mfma<QT, kKvE5M2, D>(prm, kv_heads, stream);
        default: return dispatch_mfma<QT, kKvNative, D>(prm, kv_heads, stream);
    }
}

template <int D>
int dispatch_formats(PartialParams& prm, int q_dtype, int kv_dtype, int kv_heads, hipStream_t stream) {
    if (q_dtype == PD_DTYPE_F32) return dispatch_fp32<D>(prm, kv_heads, stream);
    if (q_dtype == PD_DTYPE_BF16) return dispatch_kv<__bf16, D>(prm, kv_dtype, kv_heads, stream);
    return dispatch_kv<_Float16, D>(prm, kv_dtype, kv_heads, stream);
}

int run_partial(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype, float k_scale, float v_scale,
                const int32_t* table, const int32_t* lengths, float* numerator, float* stats, int batch,
                int query_heads, int kv_heads, int head_dim, int page_size, int table_width, int physical_pages,
                int splits, int split_tokens, int hints, const int32_t* length_bounds, hipStream_t stream,
                int* state_stride = nullptr) {
    PartialParams prm{};
    prm.batch = batch;
    prm.unshared_pages = (hints & PD_HINT_UNSHARED_PAGES) != 0;
    prm.ragged_lengths = (hints & PD_HINT_RAGGED_LENGTHS) != 0;
    prm.q = q;
    prm.k = k;
    prm.v = v;
    prm.table = table;
    prm.lengths = lengths;
    prm.numerator = numerator;
    prm.stats = stats;
    prm.query_heads = query_heads;
    prm.group = query_heads / kv_heads;
    prm.page_shift = page_size == 16 ? 4 : 5;
    prm.table_width = table_width;
    prm.physical_pages = physical_pages;
    prm.splits = splits;
    prm.split_tokens = split_tokens;
    prm.token_bytes = static_cast<uint32_t>(static_cast<size_t>(kv_heads) * head_dim * element_size(kv_dtype));
    prm.page_bytes = static_cast<uint64_t>(page_size) * prm.token_bytes;
    prm.scale_log2 = kLog2e * k_scale / sqrtf(static_cast<float>(head_dim));
    prm.v_scale = v_scale;
    plan_items(prm, length_bounds);
    const int status = head_dim == 64 ? dispatch_formats<64>(prm, q_dtype, kv_dtype, kv_heads, stream)
                                      : dispatch_formats<128>(prm, q_dtype, kv_dtype, kv_heads, stream);
    if (state_stride) *state_stride = prm.combine ? prm.quarters_per_wg : 1;
    return status;
}


template <int D>
int launch_merge(const MergeParams& mp, int batch, int merge_mode, hipStream_t stream) {
    const bool shared = merge_mode == PD_MERGE_SHARED;
    const int states = mp.parts >> mp.stride_shift;
    // merge_rows keeps a row in one wave, loading (states / PGW) 16-byte
    // columns per lane; with few rows of many states, merge_cols (D / 32
    // workgroups per row) finishes sooner.
    const int rounds = (states + kWave / (D / 4) - 1) / (kWave / (D / 4));
    const bool many_rows = static_cast<int64_t>(batch) * mp.query_heads >= kMergeRowsMin;
    if (states <= merge_wave_max_parts<D>() && (many_rows || rounds <= 2)) {
        const dim3 grid((mp.query_heads + kMergeRowsPerGroup - 1) / kMergeRowsPerGroup, batch);
        if (shared) {
            hipLaunchKernelGGL((merge_rows_kernel<D, true>), grid, dim3(kWave * kMergeRowsPerGroup), 0, stream, mp);
        } else {
            hipLaunchKernelGGL((merge_rows_kernel<D, false>), grid, dim3(kWave * kMergeRowsPerGroup), 0, stream, mp);
        }
        return launch_status();
    }
    const dim3 grid(mp.query_heads, batch, D / kMergeChunk);
    const dim3 block(kMergeThreads);
    const size_t lds = shared ? states * sizeof(float) : 0;
    // The long-row variant issues 1024 states' loads per round but holds one
    // (serial) or two (shared) workgroups per CU: it pays only while the grid
    // fits the device in one round. Larger grids take 256-state rounds at full
    // occupancy (rows of a plan whose reserved context exceeds the live one
    // among them: the variant follows the allocated states).
    const int64_t workgroups = static_cast<int64_t>(grid.x) * grid.y * grid.z;
    const bool long_rows = states > kMergeColBatchShort * kMergeColGroups && workgroups <= device_compute_units();
    if (shared && long_rows) {
        hipLaunchKernelGGL((merge_cols_kernel<D, true, kMergeColBatchLong>), grid, block, lds, stream, mp);
    } else if (shared) {
        hipLaunchKernelGGL((merge_cols_kernel<D, true, kMergeColBatchShort>), grid, block, lds, stream, mp);
    } else if (long_rows) {
        hipLaunchKernelGGL((merge_cols_kernel<D, false, kMergeColBatchLong>), grid, block, lds, stream, mp);
    } else {
        hipLaunchKernelGGL((merge_cols_kernel<D, false, kMergeColBatchShort>), grid, block, lds, stream, mp);
    }
    return launch_status();
}

int check_hints(int hints) {
    return (hints & ~(PD_HINT_UNSHARED_PAGES | PD_HINT_RAGGED_LENGTHS)) == 0 ? PD_OK : PD_ERR_HINT;
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

int run_merge(const float* numerator, const float* stats, float* out, const int32_t* lengths, int batch,
              int query_heads, int head_dim, int page_size, int table_width, int splits, int split_tokens,
              int merge_mode, int stride, hipStream_t stream) {
    MergeParams mp{};
    mp.numerator = numerator;
    mp.stats = stats;
    mp.out = out;
    mp.lengths = lengths;
    mp.parts = kQuarters * splits;
    mp.stride_shift = stride == 4 ? 2 : stride == 2 ? 1 : 0;
    mp.query_heads = query_heads;
    mp.split_tokens = split_tokens;
    mp.capacity = table_width * page_size;
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

// The scratch holds numerator [B, Hq, 4 * splits, D] at offset 0 and stats
// [B, Hq, 4 * splits, 2] after it, at the next 256-byte boundary.
size_t scratch_stats_offset(int batch, int query_heads, int head_dim, int splits) {
    const size_t numerator = static_cast<size_t>(batch) * query_heads * kQuarters * splits * head_dim * sizeof(float);
    return (numerator + 255) / 256 * 256;
}

}  // namespace

extern "C" {

int pd_decode_partial_ex(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype, float k_scale,
                         float v_scale, const int32_t* table, const int32_t* lengths, float* numerator, float* stats,
                         int batch, int query_heads, int kv_heads, int head_dim, int page_size, int table_width,
                         int physical_pages, int splits, int split_tokens, int hints, const int32_t* length_bounds,
                         void* stream) {
    int status = check_common(q, q_dtype, k, v, kv_dtype, k_scale, v_scale, table, lengths, numerator, stats, batch,
                              query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                              split_tokens);
    if (status == PD_OK) status = check_hints(hints);
    if (status != PD_OK) return status;
    return run_partial(q, q_dtype, k, v, kv_dtype, k_scale, v_scale, table, lengths, numerator, stats, batch,
                       query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits, split_tokens,
                       hints, length_bounds, static_cast<hipStream_t>(stream));
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

int pd_decode_ex(const void* q, int q_dtype, const void* k, const void* v, int kv_dtype, float k_scale,
                 float v_scale, const int32_t* table, const int32_t* lengths, float* numerator, float* stats,
                 float* out, int batch, int query_heads, int kv_heads, int head_dim, int page_size, int table_width,
                 int physical_pages, int splits, int split_tokens, int merge_mode, int hints,
                 const int32_t* length_bounds, void* stream) {
    int status = check_common(q, q_dtype, k, v, kv_dtype, k_scale, v_scale, table, lengths, numerator, stats, batch,
                              query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                              split_tokens);
    if (status == PD_OK)
        status = check_merge(numerator, stats, out, lengths, batch, query_heads, head_dim, page_size, table_width,
                             splits, split_tokens, merge_mode);
    if (status == PD_OK) status = check_hints(hints);
    if (status != PD_OK) return status;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int stride = 1;
    status = run_partial(q, q_dtype, k, v, kv_dtype, k_scale, v_scale, table, lengths, numerator, stats, batch,
                         query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                         split_tokens, hints, length_bounds, s, &stride);
    if (status != PD_OK) return status;
    return run_merge(numerator, stats, out, lengths, batch, query_heads, head_dim, page_size, table_width, splits,
                     split_tokens, merge_mode, stride, s);
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

int pd_table_from_csr(const int32_t* indptr, const int32_t* indices, const int32_t* last_page_len, int32_t* table,
                      int32_t* lengths, int32_t* overflow, int batch, int table_width, int page_size,
                      int max_context, void* stream) {
    if (!indptr || !indices || !last_page_len || !table || !lengths) return PD_ERR_NULL_POINTER;
    if (batch < 1 || batch > 65535 || table_width < 1 || table_width > 65536) return PD_ERR_SHAPE;
    if (page_size != 16 && page_size != 32) return PD_ERR_SHAPE;
    if (max_context < 0 || max_context > (1 << 20)) return PD_ERR_SHAPE;
    CsrParams c{indptr, indices, last_page_len, table, lengths, overflow, table_width, page_size, max_context};
    hipLaunchKernelGGL(table_from_csr_kernel, dim3(batch), dim3(256), 0, static_cast<hipStream_t>(stream), c);
    return launch_status();
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
        default: return "unknown status";
    }
}

int pd_abi_version(void) { return PD_ABI_VERSION; }

}  // extern "C"
