// CPU oracle for the AdaptiveIMI retrieval-guided sparse-decode path.
//
// TEST INFRASTRUCTURE ONLY.  Nothing in the product (adaptiveimi_amd/) links,
// loads or calls this file; only tests/, __graft_entry__.smoke() and the
// cpu_baseline leg of bench.py do, and only as the checker / CPU baseline.
//
// Every function restates one step of the reference path and cites the
// reference file:line it follows (paths relative to the reference repo root).
// Floating-point order is reproduced exactly where the reference fixes it:
//   * the squared-L2 distance accumulates 8 FMA lanes (lane j sums dims
//     i = j mod 8 in ascending order), then adds lane results 0..7 left to
//     right (library/AdaptiveIMI/cpp_extensions/src/kmeans_core.cpp:22-44);
//   * the M-step sums each thread's static OpenMP chunk sequentially, then
//     adds the per-thread partials in thread order and multiplies by
//     1.0f/size (kmeans_core.cpp:265-312);
//   * the decode score is a sequential fp32 FMA chain over the 128 dims of
//     the merged centroid (cuda/compute_impl.cu:80-101).
// Build: see oracle/Makefile (g++ -O3 -ffp-contract=off; FMA via fmaf or the
// AVX2 fmadd intrinsic, both correctly rounded).

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <random>
#include <vector>
#include <omp.h>
#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#endif

namespace {

inline float bf16_bits_to_f32(uint16_t h) {
    uint32_t u = static_cast<uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// kmeans_core.cpp:22-44 — eight FMA lanes over dims j, j+8, ... then
// r0+r1+...+r7 left to right, then a plain tail (never used: dim % 8 == 0).
inline float l2_lanes8(const float* a, const float* b, int dim) {
    int i = 0;
#if defined(__AVX2__) && defined(__FMA__)
    __m256 acc = _mm256_setzero_ps();
    for (; i + 7 < dim; i += 8) {
        __m256 d = _mm256_sub_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i));
        acc = _mm256_fmadd_ps(d, d, acc);
    }
    alignas(32) float lane[8];
    _mm256_store_ps(lane, acc);
#else
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (; i + 7 < dim; i += 8) {
        for (int j = 0; j < 8; ++j) {
            float d = a[i + j] - b[i + j];
            lane[j] = std::fmaf(d, d, lane[j]);
        }
    }
#endif
    float total = lane[0];
    for (int j = 1; j < 8; ++j) total = total + lane[j];
    for (; i < dim; ++i) {
        float d = a[i] - b[i];
        total = total + d * d;
    }
    return total;
}

// libgomp schedule(static) without chunk: thread t of P gets a contiguous
// block; the first n % P threads get one extra iteration.
inline void static_chunk(int64_t n, int P, int t, int64_t& lo, int64_t& hi) {
    int64_t q = n / P, r = n % P;
    lo = t * q + std::min<int64_t>(t, r);
    hi = lo + q + (t < r ? 1 : 0);
}

}  // namespace

extern "C" {

int orc_version(void) { return 1; }

void orc_bf16_to_f32(const uint16_t* src, float* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = bf16_bits_to_f32(src[i]);
}

float orc_l2(const float* a, const float* b, int dim) { return l2_lanes8(a, b, dim); }

// E-step, kmeans_core.cpp:222-242: label = argmin over c ascending with a
// strict '<' (lowest index wins ties), starting from FLT_MAX / cluster 0.
// Also returns the per-point minimum distance; `inertia` is their sum in
// index order (the reference uses an OpenMP reduction whose order is not
// fixed; it only feeds the early-stop test).
float orc_estep(const float* data, int64_t n, int dim, const float* cent, int k,
                int32_t* labels, float* mind, int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float best = std::numeric_limits<float>::max();
        int32_t arg = 0;
        const float* x = data + i * dim;
        for (int c = 0; c < k; ++c) {
            float d = l2_lanes8(x, cent + (int64_t)c * dim, dim);
            if (d < best) {
                best = d;
                arg = c;
            }
        }
        labels[i] = arg;
        if (mind) mind[i] = best;
    }
    float inertia = 0.0f;
    if (mind)
        for (int64_t i = 0; i < n; ++i) inertia += mind[i];
    return inertia;
}

// Raw engine outputs (the first n after seeding): std::mt19937 and
// std::mt19937_64, the engines of kmeans_core.cpp:150 and :293.  They let the
// tests pin the engines against the outputs the C++ standard fixes
// ([rand.predef]: the 10000th output of a default-seeded engine).
void orc_mt32_outputs(uint32_t seed, int64_t n, uint32_t* out) {
    std::mt19937 rng(seed);
    for (int64_t i = 0; i < n; ++i) out[i] = static_cast<uint32_t>(rng());
}
void orc_mt64_outputs(uint64_t seed, int64_t n, uint64_t* out) {
    std::mt19937_64 rng(seed);
    for (int64_t i = 0; i < n; ++i) out[i] = rng();
}

// Uniform draws used by the empty-cluster reseed of iteration `iter`:
// std::mt19937(iter + 12345) and uniform_int_distribution<int32_t>(0, n-1),
// drawn once per empty cluster in ascending cluster order
// (kmeans_core.cpp:299-311).
void orc_reseed_draws(int iter, int64_t n, int count, int32_t* out) {
    std::mt19937 rng(static_cast<unsigned>(iter + 12345));
    std::uniform_int_distribution<int32_t> dist(0, static_cast<int32_t>(n - 1));
    for (int e = 0; e < count; ++e) out[e] = dist(rng);
}

// M-step, kmeans_core.cpp:265-312, for a run with `nthreads` OpenMP threads.
void orc_mstep(const float* data, int64_t n, int dim, const int32_t* labels, int k,
               int nthreads, int iter, float* cent) {
    const int P = std::max(1, nthreads);
    std::vector<std::vector<float>> part(P, std::vector<float>((size_t)k * dim, 0.0f));
    std::vector<std::vector<int32_t>> cnt(P, std::vector<int32_t>(k, 0));
    for (int t = 0; t < P; ++t) {
        int64_t lo, hi;
        static_chunk(n, P, t, lo, hi);
        float* acc = part[t].data();
        for (int64_t i = lo; i < hi; ++i) {
            int c = labels[i];
            cnt[t][c]++;
            const float* x = data + i * dim;
            for (int d = 0; d < dim; ++d) acc[(size_t)c * dim + d] += x[d];
        }
    }
    std::vector<float> total((size_t)k * dim, 0.0f);
    std::vector<int32_t> size(k, 0);
    for (int t = 0; t < P; ++t)
        for (int c = 0; c < k; ++c) {
            size[c] += cnt[t][c];
            for (int d = 0; d < dim; ++d) total[(size_t)c * dim + d] += part[t][(size_t)c * dim + d];
        }
    std::mt19937 rng(static_cast<unsigned>(iter + 12345));
    std::uniform_int_distribution<int32_t> dist(0, static_cast<int32_t>(n - 1));
    for (int c = 0; c < k; ++c) {
        if (size[c] > 0) {
            float inv = 1.0f / static_cast<float>(size[c]);
            for (int d = 0; d < dim; ++d) cent[(size_t)c * dim + d] = total[(size_t)c * dim + d] * inv;
        } else {
            int32_t s = dist(rng);
            std::memcpy(cent + (size_t)c * dim, data + (int64_t)s * dim, sizeof(float) * dim);
        }
    }
}

// k-means++ seeding, kmeans_core.cpp:138-186: mt19937_64(seed); first pick
// uniform_int_distribution<int32_t>(0, n-1); each later pick draws
// uniform_real_distribution<double>(0, sum) against the running double sum
// of per-point minimum distances (taking the first index whose running sum
// reaches the target).
void orc_kmeanspp_init(const float* data, int64_t n, int dim, int k, uint64_t seed, float* cent) {
    std::vector<float> mind(n, std::numeric_limits<float>::max());
    std::mt19937_64 rng(seed);
    std::uniform_int_distribution<int32_t> first(0, static_cast<int32_t>(n - 1));
    int32_t idx = first(rng);
    std::memcpy(cent, data + (int64_t)idx * dim, sizeof(float) * dim);
    for (int c = 1; c < k; ++c) {
        const float* prev = cent + (int64_t)(c - 1) * dim;
        for (int64_t i = 0; i < n; ++i) {
            float d = l2_lanes8(data + i * dim, prev, dim);
            if (d < mind[i]) mind[i] = d;
        }
        double total = 0.0;
        for (int64_t i = 0; i < n; ++i) total += mind[i];
        std::uniform_real_distribution<double> real(0.0, total);
        double target = real(rng);
        double run = 0.0;
        int64_t pick = 0;
        for (int64_t i = 0; i < n; ++i) {
            run += mind[i];
            if (run >= target) {
                pick = i;
                break;
            }
        }
        std::memcpy(cent + (int64_t)c * dim, data + pick * dim, sizeof(float) * dim);
    }
}

// Lloyd loop, kmeans_core.cpp:190-314: E-step, early-stop test, M-step.
// After a full run the labels come from the last E-step while the centroids
// have been moved by the last M-step; an early stop skips that M-step.
// `mstep_threads` is the reference's threads_per_phase (it fixes the M-step
// summation order); `estep_threads` only parallelises the oracle itself.
// Returns the number of E-steps executed.
int orc_lloyd_p(const float* data, int64_t n, int dim, int k, float* cent, int32_t* labels,
                int max_iters, float tol, int es_min_iter, float es_rel_tol, int mstep_threads,
                int estep_threads) {
    std::vector<float> mind(n);
    float prev = std::numeric_limits<float>::max();
    int iters = 0;
    for (int it = 0; it < max_iters; ++it) {
        ++iters;
        float inertia = orc_estep(data, n, dim, cent, k, labels, mind.data(), estep_threads);
        float change = std::fabs(prev - inertia);
        float rel = (prev > 0) ? change / prev : 0.0f;
        bool min_ok = iters >= std::max(1, es_min_iter);
        if (min_ok && (rel <= std::max(0.0f, es_rel_tol) || change <= std::max(0.0f, tol))) break;
        prev = inertia;
        orc_mstep(data, n, dim, labels, k, mstep_threads, it, cent);
    }
    return iters;
}

// IMI cell construction + stable counting sort, reorganize_core.cpp:18-85
// (2-way), 87-176 (4-way, mixed radix ((l1*k2+l2)*k3+l3)*k4+l4), 178-231
// (IVF, P == 1) and 234-311.
//   labels: [P][T] subspace labels; ks: [P] centroids per subspace.
// Outputs: final_labels[T] (compact id = rank of the global cell id among
// occupied cells), gids[n_active] (global id of each compact cell),
// offsets[n_active+1], perm[T] (CSR position -> original token index, token
// indices ascending inside a cell).  Returns n_active.
int32_t orc_compact_reorg(const int32_t* labels, const int32_t* ks, int P, int64_t T,
                          int32_t* final_labels, int32_t* gids, int32_t* offsets, int32_t* perm) {
    int64_t ncells = 1;
    for (int p = 0; p < P; ++p) ncells *= ks[p];
    std::vector<int64_t> g(T);
    for (int64_t t = 0; t < T; ++t) {
        int64_t v = 0;
        for (int p = 0; p < P; ++p) v = v * ks[p] + labels[(int64_t)p * T + t];
        g[t] = v;
    }
    std::vector<uint8_t> used(ncells, 0);
    for (int64_t t = 0; t < T; ++t) used[g[t]] = 1;
    std::vector<int32_t> g2c(ncells, -1);
    int32_t n_active = 0;
    for (int64_t c = 0; c < ncells; ++c)
        if (used[c]) {
            gids[n_active] = static_cast<int32_t>(c);
            g2c[c] = n_active++;
        }
    std::vector<int32_t> cnt(n_active, 0);
    for (int64_t t = 0; t < T; ++t) {
        final_labels[t] = g2c[g[t]];
        cnt[final_labels[t]]++;
    }
    offsets[0] = 0;
    for (int32_t c = 0; c < n_active; ++c) offsets[c + 1] = offsets[c] + cnt[c];
    std::vector<int32_t> wp(offsets, offsets + n_active);
    for (int64_t t = 0; t < T; ++t) perm[wp[final_labels[t]]++] = static_cast<int32_t>(t);
    return n_active;
}

// Query-group similarity, cuda/compute_impl.cu:62-103: qsum[d] = sum over the
// G grouped queries (g ascending, from 0.0f) of float(q); score[c] = fp32
// FMA chain over d = 0..D-1 of qsum[d] * C[c][d] starting from 0.0f.
void orc_scores(const uint16_t* q, const float* cent, int H, int G, int N, int D, float* out) {
    std::vector<float> qs(D);
    for (int h = 0; h < H; ++h) {
        for (int d = 0; d < D; ++d) {
            float a = 0.0f;
            for (int gg = 0; gg < G; ++gg) a += bf16_bits_to_f32(q[((int64_t)h * G + gg) * D + d]);
            qs[d] = a;
        }
        for (int c = 0; c < N; ++c) {
            const float* cp = cent + ((int64_t)h * N + c) * D;
            float s = 0.0f;
            for (int d = 0; d < D; ++d) s = std::fmaf(qs[d], cp[d], s);
            out[(int64_t)h * N + c] = s;
        }
    }
}

// Cluster selection for one step, per head:
//   retrieval.py:357 (masked cells -> -inf) and 295-303: topk(nprobe) with
//   ties broken by the lower compact id; inclusive int32 cumsum of sizes;
//   keep = size > 0 and (cumsum - size) < max_tokens;
//   wave_buffer_cpu_hotcold.cpp:303-371: walk the kept ids in rank order,
//   skip empty ones, add ceil(size/page) pages and stop at the first id whose
//   running page count exceeds buffer_pages.
// scores/sizes/masked: [H][N]; out sel: [H][nprobe] compact ids in rank order
// (-1 after the last), m[H] = number selected, tokens[H] = their size sum.
void orc_select(const float* scores, const int32_t* sizes, const uint8_t* masked, int H, int N,
                int nprobe, int max_tokens, int buffer_pages, int page_size, int32_t* sel,
                int32_t* m, int64_t* tokens) {
    std::vector<int32_t> idx(N);
    for (int h = 0; h < H; ++h) {
        const float* s = scores + (int64_t)h * N;
        const uint8_t* mk = masked + (int64_t)h * N;
        const int32_t* sz = sizes + (int64_t)h * N;
        auto key = [&](int32_t c) {
            return mk[c] ? -std::numeric_limits<float>::infinity() : s[c];
        };
        for (int c = 0; c < N; ++c) idx[c] = c;
        std::stable_sort(idx.begin(), idx.end(),
                         [&](int32_t a, int32_t b) { return key(a) > key(b); });
        int32_t* out = sel + (int64_t)h * nprobe;
        for (int r = 0; r < nprobe; ++r) out[r] = -1;
        int32_t cum = 0;
        int pages = 0;
        int32_t cnt = 0;
        int64_t tok = 0;
        for (int r = 0; r < nprobe && r < N; ++r) {
            int32_t c = idx[r];
            int32_t size = sz[c];
            cum += size;
            bool keep = size > 0 && (cum - size) < max_tokens;
            if (!keep) continue;
            pages += (size + page_size - 1) / page_size;
            if (pages > buffer_pages) break;
            out[cnt++] = c;
            tok += size;
        }
        m[h] = cnt;
        tokens[h] = tok;
    }
}

// Cluster of each new decode key in the async centroid update,
// async_update.py:125-127: similarities = keys_fp32 @ shadow^T (torch.bmm),
// cluster = torch.argmax (first index of the maximum).  The bmm summation
// order is the BLAS library's and is not pinned by the reference; this
// restatement fixes it to the sequential fp32 FMA chain over d, with -0
// counted as +0 so that equal values tie and the lowest row wins.
// keys [B][D], rows [N][D] fp32; out [B] row index.
void orc_update_assign(const float* keys, int B, const float* rows, int N, int D, int32_t* out) {
    for (int b = 0; b < B; ++b) {
        const float* x = keys + (int64_t)b * D;
        float best = 0.0f;
        int32_t arg = 0;
        for (int r = 0; r < N; ++r) {
            const float* c = rows + (int64_t)r * D;
            float s = 0.0f;
            for (int d = 0; d < D; ++d) s = std::fmaf(x[d], c[d], s);
            s = s + 0.0f;
            if (r == 0 || s > best) {
                best = s;
                arg = r;
            }
        }
        out[b] = arg;
    }
}

// Softmax decode attention in double precision (closed form of the
// unvendored weighted_flash_decoding called at retrieval.py:439-447):
// out[h*G+g] = sum_r softmax_r(scale * q.k_r) v_r over the rows listed in
// rows[h][0..nrows[h]) (indices into kv[h]).  K/V/q are bf16 bit patterns.
void orc_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t kv_head_stride,
                   const int64_t* rows, const int32_t* nrows, int64_t rows_stride, int H, int G, int D,
                   double scale, double* out) {
    for (int h = 0; h < H; ++h) {
        const int64_t* rl = rows + (int64_t)h * rows_stride;
        int nr = nrows[h];
        for (int g = 0; g < G; ++g) {
            const uint16_t* qp = q + ((int64_t)h * G + g) * D;
            std::vector<double> sc(nr);
            double mx = -std::numeric_limits<double>::infinity();
            for (int r = 0; r < nr; ++r) {
                const uint16_t* kp = k + (int64_t)h * kv_head_stride + rl[r] * D;
                double a = 0.0;
                for (int d = 0; d < D; ++d) a += (double)bf16_bits_to_f32(qp[d]) * (double)bf16_bits_to_f32(kp[d]);
                sc[r] = a * scale;
                mx = std::max(mx, sc[r]);
            }
            double* o = out + ((int64_t)h * G + g) * D;
            for (int d = 0; d < D; ++d) o[d] = 0.0;
            if (nr == 0) continue;
            double den = 0.0;
            for (int r = 0; r < nr; ++r) {
                double p = std::exp(sc[r] - mx);
                den += p;
                const uint16_t* vp = v + (int64_t)h * kv_head_stride + rl[r] * D;
                for (int d = 0; d < D; ++d) o[d] += p * (double)bf16_bits_to_f32(vp[d]);
            }
            for (int d = 0; d < D; ++d) o[d] /= den;
        }
    }
}

}  // extern "C"
