// Partition kernels of the gfx950 decode library and their launchers, as
// templates: each partial_*.hip translation unit instantiates those of one q
// format and head dimension (decode.hip's run_partial picks the unit), so the
// library's many kernel instantiations compile in parallel.
#ifndef PAGED_DECODE_PARTITION_KERNELS_H
#define PAGED_DECODE_PARTITION_KERNELS_H

#include "device_common.h"

namespace pd {
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
// kRow: a whole-row workgroup (up to kRowMaxWaves waves) that folds its
// waves' states in LDS and writes the output rows instead of states.
template <typename T, int D, int GT, int NL, int PD, int NC, int kList, bool kRow = false>
__global__ void __launch_bounds__(kRow ? kWave * fp32_row_max_waves(GT) : kWave * 8)
    partial_kernel(const PartialParams p) {
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
    const BlockCoords bc = block_coords<kList>(blockIdx.x, blockIdx.y, blockIdx.z, p.grid_x, p.grid_y, p.xcd_shift,
                                                     p.xcd_main_rows, p.xcd_tail_shift);
    const PartitionRange pr = partition_range<kList>(p, bc);
    const int waves_wg = blockDim.x / kWave;
    const int32_t* pages = p.table + static_cast<int64_t>(pr.b) * p.table_width;
    int window = kRow ? row_speculative_page<TPL>(p, wave, waves_wg)
                      : speculative_page<TPL>(p, pr.first, pr.count, pr.qgroup, wave);
    int window_ids = pages[window_entry(p, window, lane)];
    const int len_raw = p.lengths[pr.b];
    const WaveWork w = kRow ? row_wave_work<GT, TPL>(p, pr.b, bc.heads, wave, waves_wg, len_raw)
                            : wave_work<GT, TPL>(p, pr.b, pr.first, pr.count, pr.qgroup, bc.heads, wave, len_raw);
    // Whole-row waves with an empty slice stay for the fold (empty state).
    if (!kRow && w.dead) {
        // Never read: the merge stops at the sequence's last live partition.
        // The speculative page-id window is consumed here (an empty asm
        // operand) so that its load is issued before this branch, alongside
        // the length's, rather than sunk into the live path after it.
        asm volatile("" ::"v"(window_ids));
        return;
    }
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
    if constexpr (kRow) {
        // Every wave leaves its state in its LDS slot -- m[8], l[8], then
        // acc[8][D] -- and after one barrier the workgroup forms each output
        // element of the tile's live heads as the merge does (max over the
        // states with l > 0, weights 2^(m - max), sum(weight * n) * v_scale /
        // sum(weight * l), or 0 for a row without tokens; decode.cu:94-107).
        extern __shared__ __attribute__((aligned(16))) float row_lds[];
        constexpr int kSlot = row_slot_bytes_fp32(D) / 4;
        float* slot = row_lds + wave * kSlot;
        if (lane == 0) {
#pragma unroll
            for (int g = 0; g < GT; ++g) {
                slot[g] = m[g];
                slot[8 + g] = l[g];
            }
        }
        if (lane < LPT) {
#pragma unroll
            for (int g = 0; g < GT; ++g)
#pragma unroll
                for (int e = 0; e < EPL; ++e) slot[16 + g * D + col * EPL + e] = acc[g][e];
        }
        __syncthreads();
        for (int o = threadIdx.x; o < w.heads_here * D; o += blockDim.x) {
            const int h = o / D;
            float mx = kNoToken;
            for (int s = 0; s < waves_wg; ++s) {
                const float* st = row_lds + s * kSlot;
                mx = st[8 + h] > 0.0f ? fmaxf(mx, st[h]) : mx;
            }
            float den = 0.0f, num = 0.0f;
            for (int s = 0; s < waves_wg; ++s) {
                const float* st = row_lds + s * kSlot;
                const float ls = st[8 + h];
                const float f = ls > 0.0f ? fast_exp2(st[h] - mx) : 0.0f;
                den = fmaf(f, ls, den);
                num = fmaf(f, st[16 + o], num);
            }
            p.out[w.q_row * D + o] = den > 0.0f ? num * p.v_scale / den : 0.0f;
        }
        return;
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
// kFold: what the workgroup stores -- 0 one state per wave; 1 one state per
// qw quarters of a partition (quarter combine); 2 the output rows of a whole
// row's states (whole-row launch, up to kRowMaxWaves waves: 1024 lanes).
template <typename QT, int KVF, int D, int GT, int PD, int NC, int kStream, int kFold, int kList>
__global__ void __launch_bounds__(kFold == 2 ? kWave * kRowMaxWaves : kWave * 8)
    partial_mfma_kernel(const PartialParams p) {
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
    // Dynamic LDS: the waves' K tiles, then the quarter-combine slots
    // ([waves / qw][qw - 1] CombineSlot<VH>, kFold 1) or one slot per wave
    // (kFold 2); sized by the launch.
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
    const BlockCoords bc = block_coords<kList>(blockIdx.x, blockIdx.y, blockIdx.z, p.grid_x, p.grid_y, p.xcd_shift,
                                                     p.xcd_main_rows, p.xcd_tail_shift);
    const PartitionRange pr = partition_range<kList>(p, bc);
    // A whole-row workgroup's wave runs slice `wave` of its row (one KV head,
    // one head tile); otherwise the wave index splits into (head, tile,
    // quarter) within the workgroup's partition.
    const int waves_wg = blockDim.x / kWave;
    // The item's page-table row (a shared-prefix item's: its members' leader,
    // which its shared pass reads for every member that maps the same pages).
    const int32_t* pages = p.table + static_cast<int64_t>(pr.row) * p.table_width;
    int window = kFold == 2 ? row_speculative_page<kTileTokens>(p, wave, waves_wg)
                            : speculative_page<kTileTokens>(p, pr.first, pr.count, pr.qgroup, wave);
    int window_ids = pages[window_entry(p, window, lane)];
    // Members of a shared-prefix item (work lists only): lane m < members
    // holds member m's sequence and length; the wave covers the longest
    // member's tokens, and tile column n belongs to member n / GT, which
    // masks it at its own length. Any other item is one member, all columns.
    const bool grouped = kList == kGridList && pr.members > 1;
    int member_b = pr.b;
    int member_len = 0;
    int len_raw;
    if (grouped) {
        const bool is_member = lane < pr.members;
        member_b = p.prefix_order[pr.member0 + (is_member ? lane : 0)];
        member_len = is_member ? p.lengths[member_b] : 0;
        int longest = member_len;
#pragma unroll
        for (int offset = 8; offset > 0; offset >>= 1) longest = max(longest, __shfl_xor(longest, offset));
        len_raw = __builtin_amdgcn_readfirstlane(longest);
    } else {
        len_raw = p.lengths[pr.b];
    }
    const WaveWork w = kFold == 2 ? row_wave_work<GT, kTileTokens>(p, pr.b, bc.heads, wave, waves_wg, len_raw)
                                  : wave_work<GT, kTileTokens>(p, pr.b, pr.first, pr.count, pr.qgroup, bc.heads, wave,
                                                               len_raw);
    // A whole-row workgroup's waves with an empty slice stay to contribute
    // the empty state to the fold.
    if (kFold != 2 && w.dead) {
        // Never read: the merge stops at the sequence's last live partition.
        // The speculative page-id window is consumed here (an empty asm
        // operand) so that its load is issued before this branch, alongside
        // the length's, rather than sunk into the live path after it.
        asm volatile("" ::"v"(window_ids));
        return;
    }
    const char* q_row = static_cast<const char*>(p.q) + w.q_row * D * 2;
    // Column n's member, its query head within the tile, and its first masked
    // token: for a single-member item, member 0, head n, no mask of its own.
    const int col_slots = grouped ? GT : 16;
    const int col_member = n / col_slots;
    const int col_head = n - col_member * col_slots;
    const bool col_live = col_member < pr.members && col_head < w.heads_here;
    const int64_t row_base = static_cast<int64_t>(w.kv_head) * p.group + static_cast<int64_t>(w.tile) * GT;
    // q row (batch x query-head index) of member m's tile head 0.
    auto member_row = [&](int m) {
        return grouped ? static_cast<int64_t>(__shfl(member_b, m)) * p.query_heads + row_base : w.q_row;
    };
    const int64_t col_row = member_row(col_member) + col_head;
    const int col_end = grouped ? min(max(__shfl(member_len, col_member), 0), p.reach) : 0x7FFFFFFF;

    // Page check of a shared-prefix item (prefix_span_pages): bit m of `own`
    // marks member m, whose table row differs from the leader's on a page
    // where it has tokens; it reads its own row in a later pass.
    uint32_t own = 0;
    if (grouped) {
        const int span = prefix_span_pages(p, w.wb, w.we);
        const int pairs = span * pr.members;
        uint32_t differs = 0;
        for (int base = 0; base < pairs; base += kWave) {
            const int pair = base + lane;
            const int m = pair < pairs ? prefix_pair_member(pair, span) : 0;
            const int page = prefix_pair_page(p, w.wb, pair < pairs ? pair : 0, span);
            const int mb = __shfl(member_b, m);
            const int m_end = min(min(max(__shfl(member_len, m), 0), p.reach), w.we);
            if (pair < pairs && (page << p.page_shift) < m_end &&
                p.table[static_cast<int64_t>(mb) * p.table_width + page] != pages[page])
                differs |= 1u << m;
        }
#pragma unroll
        for (int offset = 32; offset > 0; offset >>= 1) differs |= __shfl_xor(differs, offset);
        own = __builtin_amdgcn_readfirstlane(differs);
    }

    u32x4 qb[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        qb[s] = u32x4{0u, 0u, 0u, 0u};
        if (grouped) {
            if (col_live)
                qb[s] = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.q) +
                                                        (col_row * D + 32 * s + 8 * g) * 2);
        } else if (n < w.heads_here) {
            qb[s] = *reinterpret_cast<const u32x4*>(q_row + (n * D + 32 * s + 8 * g) * 2);
        }
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
    // The pass: its page-table row, its token end, and whether this lane's
    // column takes part (the shared pass: every member but those in `own`).
    const int32_t* pass_pages = pages;
    int pass_end = w.we;
    bool col_on = !grouped || ((own >> col_member) & 1u) == 0;

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
            const bool valid = (tl.live != 0u) & (t >= rb) & (t < re) & (t < col_end) & col_on;
            x[e] = valid ? sc[e] : -INFINITY;
            mx = fmaxf(mx, x[e]);
        }
        const float tile_max = max_over_lane_groups(mx) * p.scale_log2;
        if (__any((n < GT * pr.members) & (tile_max > m_head + kRescaleSlack))) {
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

    uint32_t pending = own;
    for (;;) {
        for (rb = w.wb; rb < pass_end; rb = re) {
            if ((rb >> p.page_shift) != window) {
                window = rb >> p.page_shift;
                window_ids = pass_pages[window_entry(p, window, lane)];
            }
            re = min(pass_end, (window + kWave) << p.page_shift);
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
        if (!grouped || pending == 0) break;
        // Next member with a row of its own: its row, up to its own end.
        const int m = __builtin_ctz(pending);
        pending &= pending - 1;
        pass_pages = p.table + static_cast<int64_t>(__builtin_amdgcn_readlane(member_b, m)) * p.table_width;
        pass_end = min(w.we, min(max(__builtin_amdgcn_readlane(member_len, m), 0), p.reach));
        col_on = col_member == m;
        window = -1;
    }

    // Lane (g, n) holds heads 4 g + i of dims n VH .. n VH + VH - 1; the
    // denominator of head n is summed over the four lane groups.
    float l_head = sum_over_lane_groups(l_part);
    if constexpr (kFold == 2) {
        // Every wave leaves its state in its slot; after one barrier the
        // workgroup forms each output element of the tile's live heads as the
        // merge does: the max over the states with l > 0, their weights
        // 2^(m - max), and sum(weight * n) * v_scale / sum(weight * l), or 0
        // for a row without tokens (decode.cu:94-107). Thread o covers
        // elements o, o + blockDim.x, ...: column n of dims n VH + j, head h,
        // with n fastest, so a slot's accumulators are read in lane order.
        CombineSlot<VH>* slots = reinterpret_cast<CombineSlot<VH>*>(combine_lds);
        CombineSlot<VH>* mine = slots + wave;
        if (lane < 16) {
            mine->m[n] = m_head;
            mine->l[n] = l_head;
        }
#pragma unroll
        for (int j = 0; j < VH; ++j) mine->acc[j][lane] = acc[j];
        __syncthreads();
        const int waves = waves_wg;
        for (int o = threadIdx.x; o < w.heads_here * D; o += blockDim.x) {
            const int col = o % 16;
            const int j = (o / 16) % VH;
            const int h = o / D;
            const int src_lane = 16 * (h / 4) + col;
            float mx = kNoToken;
            for (int s = 0; s < waves; ++s) mx = slots[s].l[h] > 0.0f ? fmaxf(mx, slots[s].m[h]) : mx;
            float den = 0.0f, num = 0.0f;
            for (int s = 0; s < waves; ++s) {
                const float ls = slots[s].l[h];
                const float f = ls > 0.0f ? fast_exp2(slots[s].m[h] - mx) : 0.0f;
                den = fmaf(f, ls, den);
                num = fmaf(f, slots[s].acc[j][src_lane][h % 4], num);
            }
            p.out[(w.q_row + h) * D + col * VH + j] = den > 0.0f ? num * p.v_scale / den : 0.0f;
        }
        return;
    }
    const int part = w.split * kQuarters + w.quarter;
    if (!grouped) store_empty_states(p, w, lane, extra_live_partitions(p, pr.first, pr.count, len_raw));
    // A member whose own length ends before the partition (shorter on the
    // device than its host bound) stores nothing, like a dead item: no state
    // past a sequence's end is written. Column h's end lives in lane h.
    const int64_t part_first = static_cast<int64_t>(w.split) * p.split_tokens;
    auto column_alive = [&](int h) { return !grouped || part_first < __shfl(col_end, h); };
    if constexpr (kFold == 1) {
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
            if (lane < 16 && col_live && part_first < col_end)
                *reinterpret_cast<float2*>(p.stats + stats_offset(p, col_row, part)) = make_float2(kNoToken, 0.0f);
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
    // acc[.][i] is tile column h = 4 g + i: member h / col_slots, head h % col_slots.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int h = 4 * g + i;
        const int m = h / col_slots;
        const int hm = h - m * col_slots;
        const int64_t row = member_row(m) + hm;
        const bool alive = column_alive(h);
        if (m < pr.members && hm < w.heads_here && alive) {
            f32x4* dst = reinterpret_cast<f32x4*>(p.numerator + numerator_offset(p, row, part, D) + n * VH);
#pragma unroll
            for (int j = 0; j < VH; j += 4)
                dst[j / 4] = f32x4{acc[j][i], acc[j + 1][i], acc[j + 2][i], acc[j + 3][i]} * p.v_scale;
        }
    }
    if (lane < 16 && col_live && part_first < col_end) {
        float2* st = reinterpret_cast<float2*>(p.stats + stats_offset(p, col_row, part));
        *st = make_float2(l_head > 0.0f ? m_head : kNoToken, l_head);
    }
}

inline int launch_status() { return hipGetLastError() == hipSuccess ? PD_OK : PD_ERR_LAUNCH; }

// FP32 kernel: 16-byte loads of K (and of V) per lane per chunk, chunks in
// flight ahead of the one being consumed, chunks per straight-line block.
constexpr int kFp32ChunkLoads = 1;
constexpr int kFp32Prefetch = 4;
constexpr int kFp32BlockChunks = 16;
// Whole-row FP32 launches give each wave a slice of a few chunks (16 tokens
// at most rows' sizes): a block of four keeps the straight-line code short.
constexpr int kFp32RowBlockChunks = 4;
// Matrix-core kernel: 16-token tiles issued ahead of the one being consumed,
// and tiles per straight-line block (with 2 and 2, each block's two tiles are
// requested together and consumed in order). Short blocks keep the kernel's
// code small: with 8 waves per CU running through cold straight-line code,
// instruction fetch is on the critical path (two-tile blocks measured 1 us
// faster per Llama-3-8B-shape call than eight-tile blocks, same loads).
constexpr int kMfmaPrefetch = 2;
constexpr int kMfmaBlock = 2;
// FP8 K/V tiles are half the bytes: a 64-token quarter's four tiles are all
// requested at once, in one block. Measured on MI355X (decode call, us), 2 and
// 2 -> 4 and 4: B1 L4096 10.7 -> 10.2, B16 L4096 32.5 -> 32.1, MQA B128 L1024
// D64 12.03 -> 11.90, Llama-3-8B B4 L4096 14.7 -> 14.7. Whole-row launches
// keep 2 and 2: at 1024 lanes their kernel has 128 VGPRs, and four tiles in
// flight spilled.
constexpr int kMfmaPrefetchFp8 = 4;
constexpr int kMfmaBlockFp8 = 4;

// Compute units of the current device, read once per device.
inline int device_compute_units() {
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

inline dim3 to_dim3(const Grid& g) { return dim3(g.x, g.y, g.z); }

// Launches the matrix-core kernel planned by plan_mfma (head tile GT, stream
// mode and quarter combine chosen there).
template <typename QT, int KVF, int D, int GT>
int launch_mfma(const PartialParams& prm, int kv_heads, hipStream_t stream) {
    static_assert(sizeof(CombineSlot<D / 16>) == 2 * 16 * 4 + (D / 16) * kWave * 16, "combine_slot_bytes");
    const dim3 grid = to_dim3(partial_grid(prm, kv_heads));
    const dim3 block(partial_threads(prm));
    const size_t lds = static_cast<size_t>(mfma_lds_bytes(prm, D, KVF == kKvNative ? 2 : 1));
    const int kind = grid_kind(prm);
    constexpr int kPD = KVF == kKvNative ? kMfmaPrefetch : kMfmaPrefetchFp8;
    constexpr int kNC = KVF == kKvNative ? kMfmaBlock : kMfmaBlockFp8;
    // Whole-row launches are rectangular (one workgroup per row).
#define PD_LAUNCH_MFMA(MODE, FOLD)                                                                                \
    do {                                                                                                          \
        if constexpr (FOLD == 2)                                                                                  \
            hipLaunchKernelGGL((partial_mfma_kernel<QT, KVF, D, GT, kMfmaPrefetch, kMfmaBlock, MODE, 2, kGridRect>), \
                               grid, block, lds, stream, prm);                                                    \
        else if (kind == kGridList)                                                                               \
            hipLaunchKernelGGL((partial_mfma_kernel<QT, KVF, D, GT, kPD, kNC, MODE, FOLD, kGridList>), grid,      \
                               block, lds, stream, prm);                                                          \
        else if (kind == kGridRectTails)                                                                          \
            hipLaunchKernelGGL((partial_mfma_kernel<QT, KVF, D, GT, kPD, kNC, MODE, FOLD, kGridRectTails>), grid, \
                               block, lds, stream, prm);                                                          \
        else                                                                                                      \
            hipLaunchKernelGGL((partial_mfma_kernel<QT, KVF, D, GT, kPD, kNC, MODE, FOLD, kGridRect>), grid,      \
                               block, lds, stream, prm);                                                          \
    } while (0)
#define PD_LAUNCH_MFMA_FOLDS(MODE)                      \
    do {                                                \
        if (prm.row_mode) PD_LAUNCH_MFMA(MODE, 2);      \
        else if (prm.combine) PD_LAUNCH_MFMA(MODE, 1);  \
        else PD_LAUNCH_MFMA(MODE, 0);                   \
    } while (0)
    if constexpr (KVF == kKvNative) {
        if (prm.stream_mode == 2) {
            PD_LAUNCH_MFMA_FOLDS(2);
            return launch_status();
        }
    }
    if (prm.stream_mode >= 1) PD_LAUNCH_MFMA_FOLDS(1);
    else PD_LAUNCH_MFMA_FOLDS(0);
#undef PD_LAUNCH_MFMA_FOLDS
#undef PD_LAUNCH_MFMA
    return launch_status();
}

template <int D, int GT>
int launch_fp32(const PartialParams& prm, int kv_heads, hipStream_t stream) {
    const dim3 grid = to_dim3(partial_grid(prm, kv_heads));
    const dim3 block(partial_threads(prm));
    constexpr int NL = kFp32ChunkLoads, PD = kFp32Prefetch, NC = kFp32BlockChunks;
    const int kind = grid_kind(prm);
    if (prm.row_mode)
        hipLaunchKernelGGL((partial_kernel<float, D, GT, NL, PD, kFp32RowBlockChunks, kGridRect, true>), grid, block,
                           static_cast<size_t>(prm.row_waves) * row_slot_bytes_fp32(D), stream, prm);
    else if (kind == kGridList)
        hipLaunchKernelGGL((partial_kernel<float, D, GT, NL, PD, NC, kGridList>), grid, block, 0, stream, prm);
    else if (kind == kGridRectTails)
        hipLaunchKernelGGL((partial_kernel<float, D, GT, NL, PD, NC, kGridRectTails>), grid, block, 0, stream, prm);
    else
        hipLaunchKernelGGL((partial_kernel<float, D, GT, NL, PD, NC, kGridRect>), grid, block, 0, stream, prm);
    return launch_status();
}

template <typename QT, int KVF, int D>
int dispatch_mfma(PartialParams& prm, int kv_heads, hipStream_t stream) {
    plan_mfma(prm, kv_heads, device_compute_units(), D, KVF == kKvNative ? 2 : 1);
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
    plan_fp32(prm, kv_heads, D);
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

// Launch the partition kernel of one (q format, head dimension), planned from
// prm (whose shape fields are set): one definition per partial_*.hip unit.
int dispatch_partial_f32_d64(PartialParams& prm, int kv_dtype, int kv_heads, hipStream_t stream);
int dispatch_partial_f32_d128(PartialParams& prm, int kv_dtype, int kv_heads, hipStream_t stream);
int dispatch_partial_f16_d64(PartialParams& prm, int kv_dtype, int kv_heads, hipStream_t stream);
int dispatch_partial_f16_d128(PartialParams& prm, int kv_dtype, int kv_heads, hipStream_t stream);
int dispatch_partial_bf16_d64(PartialParams& prm, int kv_dtype, int kv_heads, hipStream_t stream);
int dispatch_partial_bf16_d128(PartialParams& prm, int kv_dtype, int kv_heads, hipStream_t stream);

}  // namespace pd

#endif  // PAGED_DECODE_PARTITION_KERNELS_H
