/*
 * FP32 split-K paged GQA decode on the CPU -- TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/ as a second cross-check of the FP64 oracle and by bench.py's
 * CPU-baseline leg as the timed host implementation. The paged_decode package
 * never loads it.
 *
 * It restates the algorithm of reference src/paged_decode/csrc/decode.cu on
 * host cores, with the same observable semantics:
 *   - sequence end is clamped to min(length, table_width * page_size)
 *     (decode.cu:42-44);
 *   - tokens whose page id is outside [0, physical_pages) are skipped
 *     (decode.cu:56-58);
 *   - each partition keeps an online softmax (m, l, n) with
 *     m' = max(m, x), alpha = e^(m-m'), beta = e^(x-m') (decode.cu:61-74,
 *     docs/DESIGN.md:31-42);
 *   - the merge skips partitions with l == 0 and writes zeros for an empty
 *     row (decode.cu:94-107, docs/DESIGN.md:48-61).
 * Work is split over (sequence, KV head, partition) items so each K/V row is
 * converted once and used by all query heads of the GQA group.
 */
#include <float.h>
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { CPU_F32 = 0, CPU_F16 = 1 };

static void load_row(const void* base, int dtype, int64_t offset, int dim, float* dst) {
    if (dtype == CPU_F32) {
        memcpy(dst, (const float*)base + offset, (size_t)dim * sizeof(float));
        return;
    }
    const uint16_t* src = (const uint16_t*)base + offset;
    for (int d = 0; d < dim; d += 8) {
        __m128i packed = _mm_loadu_si128((const __m128i*)(src + d));
        _mm256_storeu_ps(dst + d, _mm256_cvtph_ps(packed));
    }
}

static float dot(const float* a, const float* b, int n) {
    float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
    for (int i = 0; i < n; ++i) acc += a[i] * b[i];
    return acc;
}

/* Returns 0 on success, 1 on invalid arguments, 2 on allocation failure. */
int pd_cpu_decode(const void* q, const void* k, const void* v, int dtype,
                  const int32_t* table, const int32_t* lengths, float* out,
                  int batch, int q_heads, int kv_heads, int head_dim, int page_size,
                  int table_width, int physical_pages, int split_tokens, int threads) {
    if (!q || !k || !v || !table || !lengths || !out) return 1;
    if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads) return 1;
    if (head_dim <= 0 || head_dim % 8 || page_size <= 0 || table_width <= 0) return 1;
    if (physical_pages <= 0 || split_tokens <= 0 || (dtype != CPU_F32 && dtype != CPU_F16)) return 1;
    if (threads <= 0) threads = 1;

    const int group = q_heads / kv_heads;
    const int64_t capacity = (int64_t)table_width * page_size;
    int64_t max_len = 0;
    for (int b = 0; b < batch; ++b) {
        int64_t len = lengths[b] < 0 ? 0 : lengths[b];
        if (len > capacity) len = capacity;
        if (len > max_len) max_len = len;
    }
    const int64_t splits = max_len == 0 ? 1 : (max_len + split_tokens - 1) / split_tokens;
    const int stride = head_dim + 2; /* n[D], m, l per partial */
    float* work = (float*)malloc((size_t)batch * q_heads * splits * stride * sizeof(float));
    if (!work) return 2;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const int64_t items = (int64_t)batch * kv_heads * splits;

#pragma omp parallel num_threads(threads)
    {
        float* key = (float*)malloc((size_t)head_dim * sizeof(float));
        float* val = (float*)malloc((size_t)head_dim * sizeof(float));
        float* query = (float*)malloc((size_t)group * head_dim * sizeof(float));
        float* state = (float*)malloc((size_t)group * stride * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (int64_t item = 0; item < items; ++item) {
            const int64_t split = item % splits;
            const int kvh = (int)((item / splits) % kv_heads);
            const int b = (int)(item / splits / kv_heads);
            int64_t len = lengths[b] < 0 ? 0 : lengths[b];
            if (len > capacity) len = capacity;
            const int64_t begin = split * split_tokens;
            const int64_t end = begin + split_tokens < len ? begin + split_tokens : len;
            for (int g = 0; g < group; ++g) {
                load_row(q, dtype, ((int64_t)b * q_heads + kvh * group + g) * head_dim, head_dim,
                         query + (size_t)g * head_dim);
                float* s = state + (size_t)g * stride;
                memset(s, 0, (size_t)head_dim * sizeof(float));
                s[head_dim] = -INFINITY;
                s[head_dim + 1] = 0.0f;
            }
            for (int64_t t = begin; t < end; ++t) {
                const int page = table[(int64_t)b * table_width + t / page_size];
                if (page < 0 || page >= physical_pages) continue;
                const int64_t offset =
                    (((int64_t)page * page_size + t % page_size) * kv_heads + kvh) * head_dim;
                load_row(k, dtype, offset, head_dim, key);
                load_row(v, dtype, offset, head_dim, val);
                for (int g = 0; g < group; ++g) {
                    float* s = state + (size_t)g * stride;
                    const float score = dot(query + (size_t)g * head_dim, key, head_dim) * scale;
                    const float m_new = fmaxf(s[head_dim], score);
                    const float alpha = expf(s[head_dim] - m_new);
                    const float beta = expf(score - m_new);
#pragma omp simd
                    for (int d = 0; d < head_dim; ++d) s[d] = s[d] * alpha + beta * val[d];
                    s[head_dim + 1] = s[head_dim + 1] * alpha + beta;
                    s[head_dim] = m_new;
                }
            }
            for (int g = 0; g < group; ++g) {
                const int h = kvh * group + g;
                memcpy(work + (((size_t)b * q_heads + h) * splits + split) * stride,
                       state + (size_t)g * stride, (size_t)stride * sizeof(float));
            }
        }
        free(key);
        free(val);
        free(query);
        free(state);

#pragma omp for schedule(static)
        for (int64_t row = 0; row < (int64_t)batch * q_heads; ++row) {
            const float* parts = work + (size_t)row * splits * stride;
            float maximum = -INFINITY;
            for (int64_t p = 0; p < splits; ++p)
                if (parts[p * stride + head_dim + 1] > 0.0f)
                    maximum = fmaxf(maximum, parts[p * stride + head_dim]);
            float denominator = 0.0f;
            float* o = out + (size_t)row * head_dim;
            memset(o, 0, (size_t)head_dim * sizeof(float));
            for (int64_t p = 0; p < splits; ++p) {
                const float* part = parts + p * stride;
                if (part[head_dim + 1] == 0.0f) continue;
                const float weight = expf(part[head_dim] - maximum);
                denominator += weight * part[head_dim + 1];
                for (int d = 0; d < head_dim; ++d) o[d] += weight * part[d];
            }
            if (denominator > 0.0f) {
                for (int d = 0; d < head_dim; ++d) o[d] /= denominator;
            } else {
                memset(o, 0, (size_t)head_dim * sizeof(float));
            }
        }
    }
    free(work);
    return 0;
}
