// Split-K paged GQA decode attention for gfx950 (AMD Instinct MI355X).
//
// Implements the C ABI declared in include/paged_decode.h. Two launches per
// decode call, both on the caller's stream:
//
//  1. partial_kernel: one 256-thread workgroup per (partition, KV head [,
//     head tile], sequence). Each K/V row is loaded from HBM exactly once and
//     used by every query head of the GQA group, held in registers. The four
//     waves take contiguous quarters of the partition; inside a wave, a 16-byte
//     load covers TPL consecutive tokens (lanes [r*LPT, (r+1)*LPT) hold token
//     r's row), loads are double-buffered chunk by chunk, q.k is reduced with
//     DPP row operations, and each token row r keeps its own online-softmax
//     stream. Streams are combined within the wave by lane shuffles and across
//     waves through LDS, leaving one (m, l, n[D]) state per query head and
//     partition. Scores are kept in log2 units (scale * log2 e) and
//     exponentiated with v_exp_f32.
//  2. merge_serial_kernel or merge_shared_kernel: max-corrected combination of
//     the partition states of one (sequence, query head) row, one lane per
//     output dimension; the shared variant computes each partition's weight
//     once into LDS and is bounded to PD_SHARED_MERGE_MAX_PARTS partitions.
//
// Semantics follow reference src/paged_decode/csrc/decode.cu:26-168 (online
// softmax and merge algebra, empty rows -> 0, l > 0 merge guard, page-id guard)
// and docs/DESIGN.md:5-65; the decomposition and data paths are this file's own.

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "paged_decode.h"

namespace {

constexpr int kWave = 64;
constexpr int kPartialWaves = 4;
constexpr int kPartialThreads = kWave * kPartialWaves;
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

struct PartialParams {
    const void* q;
    const void* k;
    const void* v;
    const int32_t* table;
    const int32_t* lengths;
    float* numerator;  // [B, Hq, splits, D]
    float* stats;      // [B, Hq, splits, 2]
    int query_heads;
    int group;       // query heads per KV head
    int head_tiles;  // ceil(group / GT)
    int page_shift;  // log2(page_size)
    int table_width;
    int physical_pages;
    int splits;
    int split_tokens;
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

// T: element type; D: head dim; GT: query heads per tile (the GQA group, padded
// to a power of two, or a slice of it); NL: 16-byte loads per chunk per lane.
template <typename T, int D, int GT, int NL>
__global__ void __launch_bounds__(kPartialThreads) partial_kernel(const PartialParams p) {
    using E = Elem<T>;
    constexpr int EPL = E::kPerLoad;  // elements per lane per load
    constexpr int LPT = D / EPL;      // lanes per token row
    constexpr int TPL = kWave / LPT;  // tokens per load
    constexpr int CT = NL * TPL;      // tokens per chunk per wave
    static_assert(TPL >= 2 && TPL <= 8 && (TPL & (TPL - 1)) == 0, "unsupported row split");
    static_assert(NL <= 32, "live mask is 32 bits");

    __shared__ float wave_state[kPartialWaves][GT][D + 2];

    const int split = blockIdx.x;
    const int kv_head = blockIdx.y / p.head_tiles;
    const int tile = blockIdx.y - kv_head * p.head_tiles;
    const int b = blockIdx.z;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int row = lane / LPT;
    const int col = lane % LPT;

    // Partition [tb, te) of sequence b; the end is clamped to the table capacity
    // (decode.cu:42-44). Quarters are cut on TPL multiples.
    const int page_size = 1 << p.page_shift;
    const int capacity = p.table_width << p.page_shift;
    const int len = max(0, min(p.lengths[b], capacity));
    const int64_t first = static_cast<int64_t>(split) * p.split_tokens;
    const int tb = static_cast<int>(min<int64_t>(first, len));
    const int te = static_cast<int>(min<int64_t>(first + p.split_tokens, len));
    int per = (te - tb + kPartialWaves - 1) / kPartialWaves;
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

    const int32_t* pages = p.table + static_cast<int64_t>(b) * p.table_width;
    const char* k_head = static_cast<const char*>(p.k) + static_cast<size_t>(kv_head) * D * sizeof(T);
    const char* v_head = static_cast<const char*>(p.v) + static_cast<size_t>(kv_head) * D * sizeof(T);
    // Groups with no live token are redirected to this sequence's q row: always
    // mapped, finite, and the same line for every lane.
    const char* park = reinterpret_cast<const char*>(q_base);
    const uint32_t lane_bytes = static_cast<uint32_t>(col) * 16u;

    // Issue the 2*NL loads of the chunk whose first aligned group starts at c0.
    auto issue = [&](Chunk<NL>& ch, int c0) {
        const char* kp[NL];
        const char* vp[NL];
        uint32_t off[NL];
        uint32_t live = 0;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int g = c0 + i * TPL;  // wave-uniform, multiple of TPL
            int lo = max(g, wb);
            int hi = min(g + TPL, we) - 1;
            if (lo > hi) lo = hi = we - 1;
            // All tokens of [lo, hi] share one page because TPL divides page_size.
            const int page = pages[lo >> p.page_shift];
            const bool ok = g < we && static_cast<uint32_t>(page) < static_cast<uint32_t>(p.physical_pages);
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

    // Fold one chunk into the per-row online-softmax state.
    auto consume = [&](const Chunk<NL>& ch, int c0) {
        float s[NL][GT];
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int t = c0 + i * TPL + row;
            // Bitwise '&' keeps this branch-free (a '&&' on the uniform bit
            // becomes a scalar branch per load).
            const bool valid = (((ch.live >> i) & 1u) != 0u) & (t >= wb) & (t < we);
#pragma unroll
            for (int g = 0; g < GT; ++g) {
                const float d = group_sum<LPT>(E::dot(qv[g], ch.k[i]));
                s[i][g] = valid ? d * p.scale_log2 : -INFINITY;
            }
        }
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            float chunk_max = s[0][g];
#pragma unroll
            for (int i = 1; i < NL; ++i) chunk_max = fmaxf(chunk_max, s[i][g]);
            const float m_new = fmaxf(m[g], chunk_max);
            const float alpha = fast_exp2(m[g] - m_new);  // 1 while no token seen, 0 after the first
            m[g] = m_new;
            float sum = l[g] * alpha;
#pragma unroll
            for (int i = 0; i < NL; ++i) {
                s[i][g] = fast_exp2(s[i][g] - m_new);  // exp2(-inf) = 0 for masked tokens
                sum += s[i][g];
            }
            l[g] = sum;
#pragma unroll
            for (int j = 0; j < EPL; ++j) acc[g][j] *= alpha;
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

    if (wb < we) {
        const int g0 = wb & ~(TPL - 1);
        const int chunks = (we - g0 + CT - 1) / CT;
        Chunk<NL> a, c;
        issue(a, g0);
        // Ping-pong: the next chunk's loads are in flight while this one is
        // consumed. The steady loop and the tail issue unconditionally inside
        // straight-line blocks whose contents differ, so the wait counters
        // only ever cover the buffer being consumed.
        int n = 0;
        for (; n + 2 < chunks; n += 2) {
            issue(c, g0 + (n + 1) * CT);
            consume(a, g0 + n * CT);
            issue(a, g0 + (n + 2) * CT);
            consume(c, g0 + (n + 1) * CT);
        }
        if (n + 1 < chunks) {
            issue(c, g0 + (n + 1) * CT);
            consume(a, g0 + n * CT);
            consume(c, g0 + (n + 1) * CT);
        } else {
            consume(a, g0 + n * CT);
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

    // Combine the four waves; one partition state per query head.
    for (int idx = threadIdx.x; idx < GT * D; idx += kPartialThreads) {
        const int g = idx / D;
        const int d = idx - g * D;
        if (g >= heads_here) break;
        float mx = kNoToken;
#pragma unroll
        for (int w = 0; w < kPartialWaves; ++w)
            if (wave_state[w][g][D + 1] > 0.0f) mx = fmaxf(mx, wave_state[w][g][D]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int w = 0; w < kPartialWaves; ++w) {
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
}

// ---------------------------------------------------------------------------
// Merge kernels: one workgroup per (sequence, query head) row, one lane per
// output dimension. A state with l == 0 is the identity (decode.cu:94-107).

template <int D>
__global__ void __launch_bounds__(D) merge_serial_kernel(const float* __restrict__ numerator,
                                                         const float* __restrict__ stats,
                                                         float* __restrict__ out, int parts) {
    const int64_t row = blockIdx.x;
    const int d = threadIdx.x;
    const float* st = stats + row * parts * 2;
    float mx = kNoToken;
    for (int j = 0; j < parts; ++j)
        if (st[2 * j + 1] > 0.0f) mx = fmaxf(mx, st[2 * j]);
    const float* num = numerator + row * parts * D + d;
    float den = 0.0f, acc = 0.0f;
    for (int j = 0; j < parts; ++j) {
        const float lj = st[2 * j + 1];
        if (lj > 0.0f) {
            const float f = fast_exp2(st[2 * j] - mx);
            den = fmaf(f, lj, den);
            acc = fmaf(f, num[static_cast<int64_t>(j) * D], acc);
        }
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
    const float* st = stats + row * parts * 2;

    float mx = kNoToken;
    for (int j = d; j < parts; j += D)
        if (st[2 * j + 1] > 0.0f) mx = fmaxf(mx, st[2 * j]);
    mx = wave_max(mx);
    if (lane == 0) scratch[0][wave] = mx;
    __syncthreads();
    mx = scratch[0][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, scratch[0][w]);

    float den = 0.0f;
    for (int j = d; j < parts; j += D) {
        const float lj = st[2 * j + 1];
        const float f = lj > 0.0f ? fast_exp2(st[2 * j] - mx) : 0.0f;
        weight[j] = f;
        den = fmaf(f, lj, den);
    }
    den = wave_sum(den);
    if (lane == 0) scratch[1][wave] = den;
    __syncthreads();
    den = scratch[1][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) den += scratch[1][w];

    const float* num = numerator + row * parts * D + d;
    float acc = 0.0f;
    for (int j = 0; j < parts; ++j) acc = fmaf(weight[j], num[static_cast<int64_t>(j) * D], acc);
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

template <typename T, int D, int GT>
int launch_partial(const PartialParams& prm, int batch, int kv_heads, hipStream_t stream) {
    constexpr int NL = GT >= 8 ? 4 : 8;
    const dim3 grid(prm.splits, kv_heads * prm.head_tiles, batch);
    hipLaunchKernelGGL((partial_kernel<T, D, GT, NL>), grid, dim3(kPartialThreads), 0, stream, prm);
    return launch_status();
}

template <typename T, int D>
int dispatch_group(PartialParams& prm, int batch, int kv_heads, hipStream_t stream) {
    const int group = prm.group;
    if (group == 1) {
        prm.head_tiles = 1;
        return launch_partial<T, D, 1>(prm, batch, kv_heads, stream);
    }
    if (group == 2) {
        prm.head_tiles = 1;
        return launch_partial<T, D, 2>(prm, batch, kv_heads, stream);
    }
    if (group <= 4) {
        prm.head_tiles = 1;
        return launch_partial<T, D, 4>(prm, batch, kv_heads, stream);
    }
    prm.head_tiles = (group + 7) / 8;
    return launch_partial<T, D, 8>(prm, batch, kv_heads, stream);
}

int run_partial(const void* q, const void* k, const void* v, int dtype, const int32_t* table,
                const int32_t* lengths, float* numerator, float* stats, int batch, int query_heads,
                int kv_heads, int head_dim, int page_size, int table_width, int physical_pages,
                int splits, int split_tokens, hipStream_t stream) {
    const size_t elem = dtype == PD_DTYPE_F16 ? 2 : 4;
    PartialParams prm{};
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
    return run_partial(q, k, v, dtype, table, lengths, numerator, stats, batch, query_heads, kv_heads,
                       head_dim, page_size, table_width, physical_pages, splits, split_tokens,
                       static_cast<hipStream_t>(stream));
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
    status = run_partial(q, k, v, dtype, table, lengths, numerator, stats, batch, query_heads, kv_heads,
                         head_dim, page_size, table_width, physical_pages, splits, split_tokens, s);
    if (status != PD_OK) return status;
    return run_merge(numerator, stats, out, batch, query_heads, head_dim, splits, merge_mode, s);
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

int pd_abi_version(void) { return 1; }

}  // extern "C"
