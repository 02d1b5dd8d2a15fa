// Split-K paged GQA decode attention for gfx950 (AMD Instinct MI355X).
//
// Implements the C ABI declared in include/paged_decode.h. pd_decode makes two
// launches per call, both on the caller's stream:
//
//  1. partial_kernel: one workgroup of NW waves per (partition, KV head [,
//     head tile], sequence). Each K/V row is loaded from HBM exactly once and
//     used by every query head of the GQA group, held in registers. The waves
//     take contiguous shares of the partition; inside a wave, a 16-byte load
//     covers TPL consecutive tokens (lanes [r*LPT, (r+1)*LPT) hold token r's
//     row), chunks of NL loads stream through PD + 1 register buffers in fully
//     unrolled blocks (PD chunks in flight), q.k is reduced with DPP row
//     operations, page ids come from a lane-indexed window via v_readlane
//     (requested at kernel start, in parallel with the length), and each token row r
//     keeps its own online-softmax stream. Streams are combined within the
//     wave by lane shuffles and across waves through LDS, leaving one
//     (m, l, n[D]) state per query head and partition. Scores are kept in log2
//     units (scale * log2 e) and exponentiated with v_exp_f32.
//  2. merge_serial_kernel or merge_shared_kernel: max-corrected combination of
//     the partition states of one (sequence, query head) row, one lane per
//     output dimension; the shared variant computes each partition's weight
//     once into LDS and is bounded to PD_SHARED_MERGE_MAX_PARTS partitions.
//
// pd_decode_fused runs the same merge algebra (serial or LDS-weighted) inside
// the partition kernel: the last workgroup to finish a row, detected with a
// device-scope arrival counter, combines that row's states. One launch per call.
//
// Semantics follow reference src/paged_decode/csrc/decode.cu:26-168 (online
// softmax and merge algebra, empty rows -> 0, l > 0 merge guard, page-id guard)
// and docs/DESIGN.md:5-65; the decomposition and data paths are this file's own.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <cstdint>

#include "paged_decode.h"

namespace {

constexpr int kWave = 64;
constexpr float kNoToken = -FLT_MAX;  // running max before any live token
constexpr float kLog2e = 1.4426950408889634f;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
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

// Partition states (max, denominator) are float pairs. Merge loops are
// branch-free and unrolled so the loads of kMergeUnroll states are in flight
// together; a data-dependent branch per state would chain their latencies.
constexpr int kMergeUnroll = 8;

__device__ __forceinline__ float2 load_state(const float2* st, int j) { return st[j]; }

// ---------------------------------------------------------------------------
// Element types. A lane moves 16 bytes per load: 8 halves or 4 floats.
template <typename T>
struct Elem;

template <>
struct Elem<_Float16> {
    static constexpr int kPerLoad = 8;
    // q.k over one 16-byte chunk with FP32 accumulation (v_dot2c_f32_f16).
    static __device__ __forceinline__ float dot(const u32x4& a, const u32x4& b) {
        const f16x8 ah = __builtin_bit_cast(f16x8, a);
        const f16x8 bh = __builtin_bit_cast(f16x8, b);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f16x2 x = {ah[2 * i], ah[2 * i + 1]};
            const f16x2 y = {bh[2 * i], bh[2 * i + 1]};
            acc = __builtin_amdgcn_fdot2(x, y, acc, false);
        }
        return acc;
    }
    static __device__ __forceinline__ void widen(const u32x4& x, float (&f)[8]) {
        const f16x8 h = __builtin_bit_cast(f16x8, x);
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] = static_cast<float>(h[i]);
    }
};

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
// Partition kernel.

// Fused-merge modes of the partition kernel (PartialParams::fuse).
enum FuseMode { kFuseNone = 0, kFuseSerial = 1, kFuseShared = 2 };

// A chunk's scores may exceed the running max by up to 2^kRescaleSlack before
// the accumulators are rescaled; weights then stay <= 2^8, far from overflow.
constexpr float kRescaleSlack = 8.0f;

struct PartialParams {
    const void* q;
    const void* k;
    const void* v;
    const int32_t* table;
    const int32_t* lengths;
    float* numerator;  // [B, Hq, splits, D]
    float* stats;      // [B, Hq, splits, 2]
    float* out;        // [B, Hq, D], written by the fused merge
    int32_t* counters; // [B * Hkv * head_tiles] arrival counters, zero between calls
    int query_heads;
    int group;       // query heads per KV head
    int head_tiles;  // ceil(group / GT)
    int page_shift;  // log2(page_size)
    int table_width;
    int physical_pages;
    int splits;
    int split_tokens;
    int fuse;              // FuseMode
    uint32_t token_bytes;  // bytes between consecutive tokens of a page (kv_heads * D * elem)
    uint64_t page_bytes;   // page_size * token_bytes
    float scale_log2;      // log2(e) / sqrt(D)
};

template <int NL>
struct Chunk {
    u32x4 k[NL];
    u32x4 v[NL];
    uint32_t live;  // bit i: group i addresses a live page inside the wave's range
};

// Floats of dynamic LDS the partition kernel needs: the per-wave states of the
// workgroup combine, or (fused LDS-bounded merge) one weight per head tile and
// partition, whichever is larger; the two uses never overlap in time.
template <int D, int GT, int NW>
constexpr int wave_state_floats() { return NW * GT * (D + 2); }

// T: element type; D: head dim; GT: query heads per tile (the GQA group, padded
// to a power of two, or a slice of it); NL: 16-byte loads of K (and of V) per
// lane per chunk; NW: waves per workgroup; PD: chunks in flight ahead of the
// one being consumed; NC: chunks per straight-line block.
template <typename T, int D, int GT, int NL, int NW, int PD, int NC>
__global__ void __launch_bounds__(kWave * NW) partial_kernel(const PartialParams p) {
    using E = Elem<T>;
    constexpr int kThreads = kWave * NW;
    constexpr int EPL = E::kPerLoad;  // elements per lane per load
    constexpr int LPT = D / EPL;      // lanes per token row
    constexpr int TPL = kWave / LPT;  // tokens per load
    constexpr int CT = NL * TPL;      // tokens per chunk per wave
    static_assert(TPL >= 2 && TPL <= 8 && (TPL & (TPL - 1)) == 0, "unsupported row split");
    static_assert(NL <= 32, "live mask is 32 bits");

    extern __shared__ float smem[];
    float (*wave_state)[GT][D + 2] = reinterpret_cast<float (*)[GT][D + 2]>(smem);  // [NW][GT][D+2]
    __shared__ int is_last;

    const int split = blockIdx.x;
    const int kv_head = blockIdx.y / p.head_tiles;
    const int tile = blockIdx.y - kv_head * p.head_tiles;
    const int b = blockIdx.z;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int row = lane / LPT;
    const int col = lane % LPT;

    // Partition [tb, te) of sequence b; the end is clamped to the table capacity
    // (decode.cu:42-44). Wave shares are contiguous and cut on TPL multiples.
    const int page_size = 1 << p.page_shift;
    const int capacity = p.table_width << p.page_shift;
    const int32_t* pages = p.table + static_cast<int64_t>(b) * p.table_width;
    // The page-id window (lane i holds the id of logical page window + i) is
    // requested before the sequence length is known, in parallel with it: it
    // starts at this wave's first page for a full-length partition, which is
    // exact for every partition but a sequence's last (re-aimed below).
    const int64_t first = static_cast<int64_t>(split) * p.split_tokens;
    const int per_full = ((p.split_tokens + NW - 1) / NW + TPL - 1) / TPL * TPL;
    int window = static_cast<int>(min<int64_t>(first + static_cast<int64_t>(wave) * per_full, capacity - 1)) >>
                 p.page_shift;
    int window_ids = pages[min(window + lane, p.table_width - 1)];

    const int len = max(0, min(p.lengths[b], capacity));
    const int tb = static_cast<int>(min<int64_t>(first, len));
    const int te = static_cast<int>(min<int64_t>(first + p.split_tokens, len));
    int per = (te - tb + NW - 1) / NW;
    per = (per + TPL - 1) / TPL * TPL;
    const int wb = min(tb + wave * per, te);
    const int we = min(wb + per, te);

    const int member0 = tile * GT;  // first GQA member handled here
    const int heads_here = min(GT, p.group - member0);
    const int64_t q_row = static_cast<int64_t>(b) * p.query_heads + kv_head * p.group + member0;
    const T* q_base = static_cast<const T*>(p.q) + q_row * D;

    u32x4 qv[GT];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        qv[g] = u32x4{0u, 0u, 0u, 0u};
        if (g < heads_here) qv[g] = *reinterpret_cast<const u32x4*>(q_base + g * D + col * EPL);
    }

    float m[GT], l[GT], acc[GT][EPL];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        m[g] = kNoToken;
        l[g] = 0.0f;
#pragma unroll
        for (int j = 0; j < EPL; ++j) acc[g][j] = 0.0f;
    }

    const char* k_head = static_cast<const char*>(p.k) + static_cast<size_t>(kv_head) * D * sizeof(T);
    const char* v_head = static_cast<const char*>(p.v) + static_cast<size_t>(kv_head) * D * sizeof(T);
    // Groups with no live token are redirected to this sequence's q row: always
    // mapped, finite, and the same line for every lane.
    const char* park = reinterpret_cast<const char*>(q_base);
    const uint32_t lane_bytes = static_cast<uint32_t>(col) * 16u;
    int rb = wb, re = wb;  // token range of the current window segment

    // Issue the 2*NL loads of the chunk whose first aligned group starts at c0.
    // Page ids come from `window_ids` (lane i holds the id of logical page
    // window + i) through v_readlane, so no scalar load sits on the issue path.
    // Lanes whose token lies outside the wave's range read a token inside it
    // (same page), so every value that reaches the FMAs is live data.
    auto issue = [&](Chunk<NL>& ch, int c0, int window_ids, int window) {
        const char* kp[NL];
        const char* vp[NL];
        uint32_t off[NL];
        uint32_t live = 0;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int g = c0 + i * TPL;  // wave-uniform, multiple of TPL
            int lo = max(g, rb);
            int hi = min(g + TPL, re) - 1;
            if (lo > hi) lo = hi = re - 1;
            // All tokens of [lo, hi] share one page because TPL divides page_size.
            const int slot = min(max((lo >> p.page_shift) - window, 0), kWave - 1);
            const int page = __builtin_amdgcn_readlane(window_ids, slot);
            const bool ok = g < re && static_cast<uint32_t>(page) < static_cast<uint32_t>(p.physical_pages);
            live |= static_cast<uint32_t>(ok) << i;
            const int t = min(max(g + row, lo), hi);
            const uint64_t page_off = static_cast<uint64_t>(ok ? page : 0) * p.page_bytes;
            kp[i] = ok ? k_head + page_off : park;
            vp[i] = ok ? v_head + page_off : park;
            off[i] = ok ? static_cast<uint32_t>(t & (page_size - 1)) * p.token_bytes + lane_bytes : lane_bytes;
        }
        ch.live = live;
#pragma unroll
        for (int i = 0; i < NL; ++i) ch.k[i] = *reinterpret_cast<const u32x4*>(kp[i] + off[i]);
#pragma unroll
        for (int i = 0; i < NL; ++i) ch.v[i] = *reinterpret_cast<const u32x4*>(vp[i] + off[i]);
        // Keep the whole chunk's loads ahead of the following consume; left
        // alone, the scheduler sinks them into it to save registers and the
        // prefetch distance collapses.
        __builtin_amdgcn_sched_barrier(0);
    };

    // Fold one chunk into the per-row online-softmax state. The running max is
    // raised (and the accumulators rescaled) only when a chunk's max exceeds it
    // by more than kRescaleSlack, a wave-uniform and rare branch.
    auto consume = [&](const Chunk<NL>& ch, int c0) {
        float s[NL][GT];
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int t = c0 + i * TPL + row;
            // Bitwise '&' keeps this branch-free (a '&&' on the uniform bit
            // becomes a scalar branch per load).
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
                const float alpha = fast_exp2(m[g] - m_new);  // 0 after kNoToken, else <= 1
                m[g] = m_new;
                l[g] *= alpha;
#pragma unroll
                for (int j = 0; j < EPL; ++j) acc[g][j] *= alpha;
            }
        }
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            float sum = l[g];
#pragma unroll
            for (int i = 0; i < NL; ++i) {
                s[i][g] = fast_exp2(fmaf(s[i][g], p.scale_log2, -m[g]));  // 0 for masked tokens
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
                for (int j = 0; j < EPL; ++j) acc[g][j] = fmaf(s[i][g], vf[j], acc[g][j]);
        }
    };

    // The wave's range is walked in segments of at most 64 pages (one window of
    // page ids); partitions up to 63 pages per wave take a single segment.
    for (rb = wb; rb < we; rb = re) {
        if ((rb >> p.page_shift) != window) {
            window = rb >> p.page_shift;
            window_ids = pages[min(window + lane, p.table_width - 1)];
        }
        re = min(we, (window + kWave) << p.page_shift);
        // Blocks of NC chunks run as fully unrolled straight-line code with PD
        // chunks in flight ahead of the one being consumed; the PD + 1 buffers
        // rotate by compile-time index, so no register holding a pending load
        // is ever copied and every wait covers exactly one chunk. (Loads kept
        // in flight across a loop back-edge make the compiler wait for all of
        // them.) The pipeline fills and drains once per block.
        for (int s = rb & ~(TPL - 1); s < re; s += NC * CT) {
            Chunk<NL> buf[PD + 1];
#pragma unroll
            for (int n = 0; n < PD; ++n) issue(buf[n], s + n * CT, window_ids, window);
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                if (s + n * CT >= re) break;
                if (n + PD < NC) issue(buf[(n + PD) % (PD + 1)], s + (n + PD) * CT, window_ids, window);
                consume(buf[n % (PD + 1)], s + n * CT);
            }
        }
    }

    // Combine the TPL token-row streams of this wave (lanes LPT, 2*LPT, ... apart).
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
        for (int j = 0; j < EPL; ++j) {
            float a = acc[g][j] * f;
#pragma unroll
            for (int x = LPT; x < kWave; x <<= 1) a += __shfl_xor(a, x);
            acc[g][j] = a;
        }
        m[g] = mw;
        l[g] = lw;
    }
    if (lane < LPT) {
#pragma unroll
        for (int g = 0; g < GT; ++g) {
#pragma unroll
            for (int j = 0; j < EPL; ++j) wave_state[wave][g][col * EPL + j] = acc[g][j];
            if (lane == 0) {
                wave_state[wave][g][D] = m[g];
                wave_state[wave][g][D + 1] = l[g];
            }
        }
    }
    __syncthreads();

    // Combine the waves; one partition state per query head.
    for (int idx = threadIdx.x; idx < GT * D; idx += kThreads) {
        const int g = idx / D;
        const int d = idx - g * D;
        if (g >= heads_here) break;
        float mx = kNoToken;
#pragma unroll
        for (int w = 0; w < NW; ++w)
            if (wave_state[w][g][D + 1] > 0.0f) mx = fmaxf(mx, wave_state[w][g][D]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float lw = wave_state[w][g][D + 1];
            if (lw > 0.0f) {
                const float f = fast_exp2(wave_state[w][g][D] - mx);
                den = fmaf(f, lw, den);
                num = fmaf(f, wave_state[w][g][d], num);
            }
        }
        const int64_t part = (q_row + g) * p.splits + split;
        p.numerator[part * D + d] = num;
        if (d == 0) {
            p.stats[part * 2] = mx;
            p.stats[part * 2 + 1] = den;
        }
    }
    if (p.fuse == kFuseNone) return;

    // Fused merge: the last workgroup to finish a (sequence, KV head, tile) row
    // combines that row's partition states. Release: every thread's stores are
    // made device-visible before the arrival is counted.
    __threadfence();
    __syncthreads();
    const int64_t row_id = static_cast<int64_t>(b) * gridDim.y + blockIdx.y;
    if (threadIdx.x == 0) is_last = atomicAdd(&p.counters[row_id], 1) == p.splits - 1;
    __syncthreads();
    if (!is_last) return;
    __threadfence();  // acquire: observe the other workgroups' states
    const float2* st_base = reinterpret_cast<const float2*>(p.stats);
    if (p.fuse == kFuseShared) {
        // LDS-bounded: one weight per (head, partition), computed once by the
        // wave that owns the head.
        float* weight = smem;                         // [GT][splits]; wave states are dead now
        float* row_den = smem + GT * p.splits;        // [GT]
        for (int g = wave; g < heads_here; g += NW) {
            const float2* st = st_base + (q_row + g) * p.splits;
            float mx = kNoToken;
            for (int j = lane; j < p.splits; j += kWave) {
                const float2 s = load_state(st, j);
                mx = s.y > 0.0f ? fmaxf(mx, s.x) : mx;
            }
            mx = wave_max(mx);
            float den = 0.0f;
            for (int j = lane; j < p.splits; j += kWave) {
                const float2 s = load_state(st, j);
                const float f = s.y > 0.0f ? fast_exp2(s.x - mx) : 0.0f;
                weight[g * p.splits + j] = f;
                den = fmaf(f, s.y, den);
            }
            den = wave_sum(den);
            if (lane == 0) row_den[g] = den;
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < heads_here * D; idx += kThreads) {
            const int g = idx / D;
            const int d = idx - g * D;
            const float* num = p.numerator + (q_row + g) * p.splits * D + d;
            const float* w = weight + g * p.splits;
            float acc_d = 0.0f;
#pragma unroll kMergeUnroll
            for (int j = 0; j < p.splits; ++j) {
                const float n = num[static_cast<int64_t>(j) * D];
                acc_d = w[j] > 0.0f ? fmaf(w[j], n, acc_d) : acc_d;
            }
            const float den = row_den[g];
            p.out[(q_row + g) * D + d] = den > 0.0f ? acc_d / den : 0.0f;
        }
    } else {
        // Serial: every lane scans the row's states itself.
        for (int idx = threadIdx.x; idx < heads_here * D; idx += kThreads) {
            const int g = idx / D;
            const int d = idx - g * D;
            const float2* st = st_base + (q_row + g) * p.splits;
            float mx = kNoToken;
#pragma unroll kMergeUnroll
            for (int j = 0; j < p.splits; ++j) {
                const float2 s = load_state(st, j);
                mx = s.y > 0.0f ? fmaxf(mx, s.x) : mx;
            }
            const float* num = p.numerator + (q_row + g) * p.splits * D + d;
            float den = 0.0f, acc_d = 0.0f;
#pragma unroll kMergeUnroll
            for (int j = 0; j < p.splits; ++j) {
                const float2 s = load_state(st, j);
                const float n = num[static_cast<int64_t>(j) * D];
                const bool live = s.y > 0.0f;
                const float f = live ? fast_exp2(s.x - mx) : 0.0f;
                den = live ? fmaf(f, s.y, den) : den;
                acc_d = live ? fmaf(f, n, acc_d) : acc_d;
            }
            p.out[(q_row + g) * D + d] = den > 0.0f ? acc_d / den : 0.0f;
        }
    }
    if (threadIdx.x == 0) p.counters[row_id] = 0;  // ready for the next call
}

// ---------------------------------------------------------------------------
// Merge kernels: one workgroup per (sequence, query head) row, one lane per
// output dimension. A state with l == 0 is the identity (decode.cu:94-107).

// Serial: every lane scans all partition states itself (no LDS).
template <int D>
__global__ void __launch_bounds__(D) merge_serial_kernel(const float* __restrict__ numerator,
                                                         const float* __restrict__ stats,
                                                         float* __restrict__ out, int parts) {
    const int64_t row = blockIdx.x;
    const int d = threadIdx.x;
    const float2* st = reinterpret_cast<const float2*>(stats) + row * parts;
    float mx = kNoToken;
#pragma unroll kMergeUnroll
    for (int j = 0; j < parts; ++j) {
        const float2 s = load_state(st, j);
        mx = s.y > 0.0f ? fmaxf(mx, s.x) : mx;
    }
    const float* num = numerator + row * parts * D + d;
    float den = 0.0f, acc = 0.0f;
#pragma unroll kMergeUnroll
    for (int j = 0; j < parts; ++j) {
        const float2 s = load_state(st, j);
        const float n = num[static_cast<int64_t>(j) * D];
        const bool live = s.y > 0.0f;
        const float f = live ? fast_exp2(s.x - mx) : 0.0f;
        den = live ? fmaf(f, s.y, den) : den;
        acc = live ? fmaf(f, n, acc) : acc;
    }
    out[row * D + d] = den > 0.0f ? acc / den : 0.0f;
}

template <int D>
__global__ void __launch_bounds__(D) merge_shared_kernel(const float* __restrict__ numerator,
                                                         const float* __restrict__ stats,
                                                         float* __restrict__ out, int parts) {
    extern __shared__ float weight[];  // [parts]
    constexpr int kWaves = D / kWave;
    __shared__ float scratch[2][kWaves];
    const int64_t row = blockIdx.x;
    const int d = threadIdx.x;
    const int lane = d % kWave;
    const int wave = d / kWave;
    const float2* st = reinterpret_cast<const float2*>(stats) + row * parts;

    float mx = kNoToken;
    for (int j = d; j < parts; j += D) {
        const float2 s = load_state(st, j);
        mx = s.y > 0.0f ? fmaxf(mx, s.x) : mx;
    }
    mx = wave_max(mx);
    if (lane == 0) scratch[0][wave] = mx;
    __syncthreads();
    mx = scratch[0][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, scratch[0][w]);

    float den = 0.0f;
    for (int j = d; j < parts; j += D) {
        const float2 s = load_state(st, j);
        const float f = s.y > 0.0f ? fast_exp2(s.x - mx) : 0.0f;
        weight[j] = f;
        den = fmaf(f, s.y, den);
    }
    den = wave_sum(den);
    if (lane == 0) scratch[1][wave] = den;
    __syncthreads();
    den = scratch[1][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) den += scratch[1][w];

    const float* num = numerator + row * parts * D + d;
    float acc = 0.0f;
#pragma unroll kMergeUnroll
    for (int j = 0; j < parts; ++j) {
        // A state with weight 0 (empty partition) contributes nothing, whatever
        // its numerator holds.
        const float n = num[static_cast<int64_t>(j) * D];
        acc = weight[j] > 0.0f ? fmaf(weight[j], n, acc) : acc;
    }
    out[row * D + d] = den > 0.0f ? acc / den : 0.0f;
}

// ---------------------------------------------------------------------------
// Host side.

int check_common(const void* q, const void* k, const void* v, int dtype, const int32_t* table,
                 const int32_t* lengths, const float* numerator, const float* stats, int batch,
                 int query_heads, int kv_heads, int head_dim, int page_size, int table_width,
                 int physical_pages, int splits, int split_tokens) {
    if (!q || !k || !v || !table || !lengths || !numerator || !stats) return PD_ERR_NULL_POINTER;
    if (dtype != PD_DTYPE_F32 && dtype != PD_DTYPE_F16) return PD_ERR_DTYPE;
    if (batch < 1 || batch > 65535 || query_heads < 1 || query_heads > 65535) return PD_ERR_SHAPE;
    if (kv_heads < 1 || query_heads % kv_heads != 0) return PD_ERR_SHAPE;
    if (head_dim != 64 && head_dim != 128) return PD_ERR_SHAPE;
    if (page_size != 16 && page_size != 32) return PD_ERR_SHAPE;
    if (table_width < 1 || table_width > 65536 || physical_pages < 1) return PD_ERR_SHAPE;
    if (splits < 1 || splits > 65535 || split_tokens < 1 || split_tokens > (1 << 20)) return PD_ERR_SPLIT;
    return PD_OK;
}

int launch_status() { return hipGetLastError() == hipSuccess ? PD_OK : PD_ERR_LAUNCH; }

// Waves per partition workgroup and 16-byte loads of K (and of V) per lane per
// chunk, chunks in flight ahead of the one being consumed, and chunks per
// straight-line block.
#ifndef PD_PARTIAL_WAVES
#define PD_PARTIAL_WAVES 4
#endif
#ifndef PD_CHUNK_LOADS
#define PD_CHUNK_LOADS 1
#endif
#ifndef PD_PREFETCH
#define PD_PREFETCH 4
#endif
#ifndef PD_BLOCK_CHUNKS
#define PD_BLOCK_CHUNKS 16
#endif

template <typename T, int D, int GT>
int launch_partial(const PartialParams& prm, int batch, int kv_heads, hipStream_t stream) {
    constexpr int NW = PD_PARTIAL_WAVES;
    constexpr int NL = PD_CHUNK_LOADS;
    constexpr int PD = PD_PREFETCH;
    constexpr int NC = PD_BLOCK_CHUNKS;
    size_t floats = static_cast<size_t>(wave_state_floats<D, GT, NW>());
    if (prm.fuse == kFuseShared) floats = std::max(floats, static_cast<size_t>(GT) * (prm.splits + 1));
    const dim3 grid(prm.splits, kv_heads * prm.head_tiles, batch);
    hipLaunchKernelGGL((partial_kernel<T, D, GT, NL, NW, PD, NC>), grid, dim3(kWave * NW), floats * sizeof(float),
                       stream, prm);
    return launch_status();
}

// Head tile: the GQA group padded to 1, 2, 4 or 8 query heads; larger groups
// are cut into tiles of 8 (one workgroup per tile).
int head_tile(int group) { return group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 ? 4 : 8; }

template <typename T, int D>
int dispatch_group(PartialParams& prm, int batch, int kv_heads, hipStream_t stream) {
    const int gt = head_tile(prm.group);
    prm.head_tiles = (prm.group + gt - 1) / gt;
    switch (gt) {
        case 1: return launch_partial<T, D, 1>(prm, batch, kv_heads, stream);
        case 2: return launch_partial<T, D, 2>(prm, batch, kv_heads, stream);
        case 4: return launch_partial<T, D, 4>(prm, batch, kv_heads, stream);
        default: return launch_partial<T, D, 8>(prm, batch, kv_heads, stream);
    }
}

int run_partial(const void* q, const void* k, const void* v, int dtype, const int32_t* table,
                const int32_t* lengths, float* numerator, float* stats, float* out, int32_t* counters,
                int fuse, int batch, int query_heads, int kv_heads, int head_dim, int page_size,
                int table_width, int physical_pages, int splits, int split_tokens, hipStream_t stream) {
    const size_t elem = dtype == PD_DTYPE_F16 ? 2 : 4;
    PartialParams prm{};
    prm.q = q;
    prm.k = k;
    prm.v = v;
    prm.table = table;
    prm.lengths = lengths;
    prm.numerator = numerator;
    prm.stats = stats;
    prm.out = out;
    prm.counters = counters;
    prm.fuse = fuse;
    prm.query_heads = query_heads;
    prm.group = query_heads / kv_heads;
    prm.page_shift = page_size == 16 ? 4 : 5;
    prm.table_width = table_width;
    prm.physical_pages = physical_pages;
    prm.splits = splits;
    prm.split_tokens = split_tokens;
    prm.token_bytes = static_cast<uint32_t>(static_cast<size_t>(kv_heads) * head_dim * elem);
    prm.page_bytes = static_cast<uint64_t>(page_size) * prm.token_bytes;
    prm.scale_log2 = kLog2e / sqrtf(static_cast<float>(head_dim));
    if (dtype == PD_DTYPE_F16) {
        return head_dim == 64 ? dispatch_group<_Float16, 64>(prm, batch, kv_heads, stream)
                              : dispatch_group<_Float16, 128>(prm, batch, kv_heads, stream);
    }
    return head_dim == 64 ? dispatch_group<float, 64>(prm, batch, kv_heads, stream)
                          : dispatch_group<float, 128>(prm, batch, kv_heads, stream);
}

template <int D>
int launch_merge(const float* numerator, const float* stats, float* out, int rows, int parts,
                 int merge_mode, hipStream_t stream) {
    if (merge_mode == PD_MERGE_SHARED) {
        hipLaunchKernelGGL((merge_shared_kernel<D>), dim3(rows), dim3(D), parts * sizeof(float), stream,
                           numerator, stats, out, parts);
    } else {
        hipLaunchKernelGGL((merge_serial_kernel<D>), dim3(rows), dim3(D), 0, stream, numerator, stats,
                           out, parts);
    }
    return launch_status();
}

int check_merge(const float* numerator, const float* stats, const float* out, int batch,
                int query_heads, int head_dim, int splits, int merge_mode) {
    if (!numerator || !stats || !out) return PD_ERR_NULL_POINTER;
    if (batch < 1 || batch > 65535 || query_heads < 1 || query_heads > 65535) return PD_ERR_SHAPE;
    if (head_dim != 64 && head_dim != 128) return PD_ERR_SHAPE;
    if (splits < 1 || splits > 65535) return PD_ERR_SPLIT;
    if (merge_mode != PD_MERGE_SERIAL && merge_mode != PD_MERGE_SHARED) return PD_ERR_MERGE;
    if (merge_mode == PD_MERGE_SHARED && splits > PD_SHARED_MERGE_MAX_PARTS) return PD_ERR_MERGE;
    return PD_OK;
}

int run_merge(const float* numerator, const float* stats, float* out, int batch, int query_heads,
              int head_dim, int splits, int merge_mode, hipStream_t stream) {
    const int rows = batch * query_heads;
    return head_dim == 64 ? launch_merge<64>(numerator, stats, out, rows, splits, merge_mode, stream)
                          : launch_merge<128>(numerator, stats, out, rows, splits, merge_mode, stream);
}

}  // namespace

extern "C" {

int pd_decode_partial(const void* q, const void* k, const void* v, int dtype, const int32_t* table,
                      const int32_t* lengths, float* numerator, float* stats, int batch,
                      int query_heads, int kv_heads, int head_dim, int page_size, int table_width,
                      int physical_pages, int splits, int split_tokens, void* stream) {
    const int status = check_common(q, k, v, dtype, table, lengths, numerator, stats, batch, query_heads,
                                    kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                                    split_tokens);
    if (status != PD_OK) return status;
    return run_partial(q, k, v, dtype, table, lengths, numerator, stats, nullptr, nullptr, kFuseNone, batch,
                       query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                       split_tokens, static_cast<hipStream_t>(stream));
}

int pd_decode_merge(const float* numerator, const float* stats, float* out, int batch, int query_heads,
                    int head_dim, int splits, int merge_mode, void* stream) {
    const int status = check_merge(numerator, stats, out, batch, query_heads, head_dim, splits, merge_mode);
    if (status != PD_OK) return status;
    return run_merge(numerator, stats, out, batch, query_heads, head_dim, splits, merge_mode,
                     static_cast<hipStream_t>(stream));
}

int pd_decode(const void* q, const void* k, const void* v, int dtype, const int32_t* table,
              const int32_t* lengths, float* numerator, float* stats, float* out, int batch,
              int query_heads, int kv_heads, int head_dim, int page_size, int table_width,
              int physical_pages, int splits, int split_tokens, int merge_mode, void* stream) {
    int status = check_common(q, k, v, dtype, table, lengths, numerator, stats, batch, query_heads,
                              kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                              split_tokens);
    if (status == PD_OK)
        status = check_merge(numerator, stats, out, batch, query_heads, head_dim, splits, merge_mode);
    if (status != PD_OK) return status;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    status = run_partial(q, k, v, dtype, table, lengths, numerator, stats, nullptr, nullptr, kFuseNone, batch,
                         query_heads, kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                         split_tokens, s);
    if (status != PD_OK) return status;
    return run_merge(numerator, stats, out, batch, query_heads, head_dim, splits, merge_mode, s);
}

int pd_decode_fused(const void* q, const void* k, const void* v, int dtype, const int32_t* table,
                    const int32_t* lengths, float* numerator, float* stats, int32_t* counters, float* out,
                    int batch, int query_heads, int kv_heads, int head_dim, int page_size, int table_width,
                    int physical_pages, int splits, int split_tokens, int merge_mode, void* stream) {
    int status = check_common(q, k, v, dtype, table, lengths, numerator, stats, batch, query_heads,
                              kv_heads, head_dim, page_size, table_width, physical_pages, splits,
                              split_tokens);
    if (status == PD_OK)
        status = check_merge(numerator, stats, out, batch, query_heads, head_dim, splits, merge_mode);
    if (status == PD_OK && !counters) status = PD_ERR_NULL_POINTER;
    if (status == PD_OK && merge_mode == PD_MERGE_SHARED && splits > PD_FUSED_SHARED_MAX_PARTS)
        status = PD_ERR_MERGE;
    if (status != PD_OK) return status;
    return run_partial(q, k, v, dtype, table, lengths, numerator, stats, out, counters,
                       merge_mode == PD_MERGE_SHARED ? kFuseShared : kFuseSerial, batch, query_heads,
                       kv_heads, head_dim, page_size, table_width, physical_pages, splits, split_tokens,
                       static_cast<hipStream_t>(stream));
}

size_t pd_workspace_bytes(int batch, int query_heads, int head_dim, int splits) {
    if (batch <= 0 || query_heads <= 0 || head_dim <= 0 || splits <= 0) return 0;
    return static_cast<size_t>(batch) * query_heads * splits * (head_dim + 2) * sizeof(float);
}

const char* pd_status_string(int status) {
    switch (status) {
        case PD_OK: return "success";
        case PD_ERR_NULL_POINTER: return "a required pointer is null";
        case PD_ERR_SHAPE: return "a dimension is outside the supported range";
        case PD_ERR_DTYPE: return "unsupported dtype (float16 or float32 expected)";
        case PD_ERR_SPLIT: return "invalid split configuration";
        case PD_ERR_MERGE: return "unknown merge mode or shared merge requires at most 4096 partial states";
        case PD_ERR_LAUNCH: return "kernel launch failed";
        default: return "unknown status";
    }
}

int pd_abi_version(void) { return 2; }

}  // extern "C"
