// CPU BASELINE (timed by bench.py's cpu_baseline leg; test infrastructure,
// never linked into the product): one decode step of every KV head as the
// reference's path computes it, written for the host's vector units and
// cores rather than as a checker:
//   - query-group sum and the fp32 FMA score chain of every cell
//     (compute_impl.cu:62-103), eight cells per AVX2 register over centroids
//     transposed once at set-up (each lane is one cell's chain in dimension
//     order, so the scores, and with them the selection, equal the oracle's
//     bit for bit);
//   - the mask (retrieval.py:357), top-nprobe + token rule
//     (retrieval.py:295-303) and page rule (wave_buffer_cpu_hotcold.cpp:
//     303-371), as the oracle states them;
//   - softmax attention in fp32 over [static rows | selected rows]
//     (copy_kernel.cuh:220-335, retrieval.py:439-447): each K/V row is read
//     once for all G query heads of its KV head; the rows are split into
//     chunks over the OpenMP threads, each chunk keeps its own running max,
//     denominator and output, and the chunks are merged per head.
// Built with its own vectorizing flags (Makefile: libcpudecode.so), not with
// the checker's -ffp-contract=off build.
#include <immintrin.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

namespace {

inline float bf16_to_f32(uint16_t b) {
    const uint32_t u = static_cast<uint32_t>(b) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// eight bf16 values -> eight floats
inline __m256 load_bf16x8(const uint16_t* p) {
    const __m128i u = _mm_loadu_si128(reinterpret_cast<const __m128i*>(p));
    return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(u), 16));
}

inline float hsum(__m256 v) {
    const __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    const __m128 t = _mm_add_ps(s, _mm_movehl_ps(s, s));
    return _mm_cvtss_f32(_mm_add_ss(t, _mm_shuffle_ps(t, t, 1)));
}

constexpr int kChunk = 512;    // rows per attention task
constexpr int kMaxD = 256;
constexpr int kMaxG = 16;

}  // namespace

extern "C" {

// Arguments:
//   q [H][G][D] bf16, centT [H][D][N] fp32 (merged, padded, transposed), sizes / masked /
//   offsets [H][N(+1)], lk / lv [H][L][D] bf16, sk / sv [H][S][D] bf16;
//   out [H][G][D] fp32; m [H] cells selected.  D a multiple of 8, <= 256;
//   G <= 16.
void cpu_decode_step_f32(const uint16_t* q, const float* centT, const int32_t* sizes, const uint8_t* masked,
                         const int32_t* offsets, int H, int G, int N, int D, const uint16_t* lk,
                         const uint16_t* lv, int64_t L, const uint16_t* sk, const uint16_t* sv, int64_t S,
                         int static_len, int nprobe, int max_tokens, int buffer_pages, int page_size,
                         float scale, float* out, int32_t* m_out) {
    if (D % 8 != 0 || D > kMaxD || G > kMaxG) return;
    std::vector<float> qs((size_t)H * D), sc((size_t)H * N);
    for (int h = 0; h < H; ++h)
        for (int d = 0; d < D; ++d) {
            float a = 0.0f;
            for (int g = 0; g < G; ++g) a += bf16_to_f32(q[((int64_t)h * G + g) * D + d]);
            qs[(size_t)h * D + d] = a;
        }
    // scores: lane j of a register is cell c0 + j's chain fma(q[d], c[d], s)
    const int nb = (N + 7) / 8;
#pragma omp parallel for schedule(static)
    for (int64_t hb = 0; hb < (int64_t)H * nb; ++hb) {
        const int h = (int)(hb / nb), c0 = (int)(hb % nb) * 8;
        const int nc = std::min(8, N - c0);
        const float* qh = qs.data() + (size_t)h * D;
        const float* cp = centT + (int64_t)h * D * N + c0;
        __m256 s = _mm256_setzero_ps();
        if (nc == 8) {
            for (int d = 0; d < D; ++d)
                s = _mm256_fmadd_ps(_mm256_set1_ps(qh[d]), _mm256_loadu_ps(cp + (int64_t)d * N), s);
        } else {
            alignas(32) float cv[8] = {};
            for (int d = 0; d < D; ++d) {
                for (int j = 0; j < nc; ++j) cv[j] = cp[(int64_t)d * N + j];
                s = _mm256_fmadd_ps(_mm256_set1_ps(qh[d]), _mm256_load_ps(cv), s);
            }
        }
        alignas(32) float r[8];
        _mm256_store_ps(r, s);
        for (int j = 0; j < nc; ++j) {
            const int64_t hc = (int64_t)h * N + c0 + j;
            sc[hc] = masked[hc] ? -std::numeric_limits<float>::infinity() : r[j];
        }
    }
    // selection (the oracle's rules)
    std::vector<std::vector<int64_t>> rows(H);
#pragma omp parallel for schedule(dynamic, 1)
    for (int h = 0; h < H; ++h) {
        const float* s = sc.data() + (size_t)h * N;
        const int32_t* sz = sizes + (int64_t)h * N;
        const int k = std::min(nprobe, N);
        std::vector<int32_t> idx(N);
        for (int c = 0; c < N; ++c) idx[c] = c;
        std::partial_sort(idx.begin(), idx.begin() + k, idx.end(), [&](int32_t a, int32_t b) {
            return s[a] > s[b] || (s[a] == s[b] && a < b);
        });
        int32_t cum = 0;
        int pages = 0, cnt = 0;
        std::vector<int64_t>& r = rows[h];
        for (int i = 0; i < static_len; ++i) r.push_back(-1 - i);
        for (int i = 0; i < k; ++i) {
            const int32_t c = idx[i], size = sz[c];
            cum += size;
            if (!(size > 0 && (cum - size) < max_tokens)) continue;
            pages += (size + page_size - 1) / page_size;
            if (pages > buffer_pages) break;
            ++cnt;
            for (int32_t t = offsets[(int64_t)h * (N + 1) + c]; t < offsets[(int64_t)h * (N + 1) + c + 1]; ++t)
                r.push_back(t);
        }
        m_out[h] = cnt;
    }
    // attention tasks: (head, chunk of kChunk rows)
    std::vector<int> task_head, task_lo;
    for (int h = 0; h < H; ++h)
        for (int64_t lo = 0; lo < (int64_t)rows[h].size(); lo += kChunk) {
            task_head.push_back(h);
            task_lo.push_back((int)lo);
        }
    const int ntask = (int)task_head.size();
    // per task: max [G], denominator [G], output [G][D]
    std::vector<float> pm((size_t)ntask * G), pl((size_t)ntask * G), po((size_t)ntask * G * D);
    const int nv = D / 8;
#pragma omp parallel for schedule(dynamic, 1)
    for (int ti = 0; ti < ntask; ++ti) {
        const int h = task_head[ti];
        const std::vector<int64_t>& r = rows[h];
        const int lo = task_lo[ti], n = (int)std::min<int64_t>(kChunk, (int64_t)r.size() - lo);
        auto row_ptr = [&](int64_t x, const uint16_t* list, const uint16_t* steady) {
            return x < 0 ? steady + ((int64_t)h * S + (-1 - x)) * D : list + ((int64_t)h * L + x) * D;
        };
        alignas(32) float qf[kMaxG][kMaxD];
        for (int g = 0; g < G; ++g)
            for (int d = 0; d < D; ++d) qf[g][d] = bf16_to_f32(q[((int64_t)h * G + g) * D + d]);
        alignas(32) float p[kMaxG][kChunk];
        float mx[kMaxG];
        for (int g = 0; g < G; ++g) mx[g] = -std::numeric_limits<float>::infinity();
        __m256 kr[kMaxD / 8];
        for (int i = 0; i < n; ++i) {
            const uint16_t* kp = row_ptr(r[lo + i], lk, sk);
            for (int j = 0; j < nv; ++j) kr[j] = load_bf16x8(kp + 8 * j);
            for (int g = 0; g < G; ++g) {
                __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
                int j = 0;
                for (; j + 1 < nv; j += 2) {
                    a0 = _mm256_fmadd_ps(_mm256_load_ps(&qf[g][8 * j]), kr[j], a0);
                    a1 = _mm256_fmadd_ps(_mm256_load_ps(&qf[g][8 * j + 8]), kr[j + 1], a1);
                }
                if (j < nv) a0 = _mm256_fmadd_ps(_mm256_load_ps(&qf[g][8 * j]), kr[j], a0);
                const float v = hsum(_mm256_add_ps(a0, a1)) * scale;
                p[g][i] = v;
                mx[g] = std::max(mx[g], v);
            }
        }
        float* o = po.data() + (size_t)ti * G * D;
        std::fill(o, o + (size_t)G * D, 0.0f);
        float den[kMaxG] = {};
        for (int i = 0; i < n; ++i) {
            const uint16_t* vp = row_ptr(r[lo + i], lv, sv);
            for (int j = 0; j < nv; ++j) kr[j] = load_bf16x8(vp + 8 * j);
            for (int g = 0; g < G; ++g) {
                const float w = std::exp(p[g][i] - mx[g]);
                den[g] += w;
                const __m256 wv = _mm256_set1_ps(w);
                float* og = o + (size_t)g * D;
                for (int j = 0; j < nv; ++j)
                    _mm256_storeu_ps(og + 8 * j, _mm256_fmadd_ps(wv, kr[j], _mm256_loadu_ps(og + 8 * j)));
            }
        }
        for (int g = 0; g < G; ++g) {
            pm[(size_t)ti * G + g] = mx[g];
            pl[(size_t)ti * G + g] = den[g];
        }
    }
    // merge the chunks of each head
#pragma omp parallel for schedule(static)
    for (int hg = 0; hg < H * G; ++hg) {
        const int h = hg / G, g = hg % G;
        float* oo = out + (int64_t)hg * D;
        std::fill(oo, oo + D, 0.0f);
        float M = -std::numeric_limits<float>::infinity();
        for (int ti = 0; ti < ntask; ++ti)
            if (task_head[ti] == h) M = std::max(M, pm[(size_t)ti * G + g]);
        float den = 0.0f;
        for (int ti = 0; ti < ntask; ++ti) {
            if (task_head[ti] != h) continue;
            const float f = std::exp(pm[(size_t)ti * G + g] - M);
            den += f * pl[(size_t)ti * G + g];
            const float* o = po.data() + ((size_t)ti * G + g) * D;
            for (int d = 0; d < D; ++d) oo[d] += f * o[d];
        }
        if (den > 0.0f)
            for (int d = 0; d < D; ++d) oo[d] /= den;
    }
}

}  // extern "C"
