// Per-step cell scoring and budget-bounded selection on gfx950.
//
// Reference:
//   scoring    cuda/compute_impl.cu:62-103 (qsum over the G grouped queries,
//              then a sequential fp32 FMA chain over the 128 merged dims)
//   mask       cache_hub/adaptive_imi/retrieval.py:357
//   selection  retrieval.py:295-303 (topk(nprobe), inclusive int32 cumsum of
//              sizes, keep = size>0 & cumsum-size < max_tokens)
//   page rule  library/AdaptiveIMI/cpp_extensions/src/wave_buffer_cpu_hotcold.cpp
//              :303-371 (stop at the first kept cell whose running page count
//              exceeds buffer_pages)
//
// One 1024-thread workgroup per KV head works in global-cell space (cell id
// g = l0 * k1 + l1), so the decode step never touches the merged-centroid
// array: the 128-term chain is evaluated as the 64-term chain over C0[l0]
// (computed once per l0) continued over C1[l1], which is the same sequence
// of fused multiply-adds.  Ranking is by (score desc, cell id asc); compact
// ids are ranks of global ids, so this is the reference tie order.
//
// Selection without a full sort: m <= K' = min(nprobe, buffer_pages, cells)
// because every kept cell costs at least one page.  A linear-bucket
// histogram of the scores finds the bucket holding the K'-th best cell; the
// cells up to that bucket (or, if that is more than kCap cells, the exact
// top K' found by a radix select on the 64-bit (score, ~cell) key) are
// sorted in LDS and the three budget rules are applied in rank order.
#include "imi_common.hpp"

namespace imi {
namespace {

constexpr int kSelThreads = 1024;
constexpr int kMaxE = 16;      // cells per thread -> up to 16384 cells
constexpr int kBins = 2048;
constexpr int kCap = 4096;     // candidate capacity (power of two)

struct SelParams {
    const uint16_t* q;
    const float* cent;
    const int32_t* cnt;
    const int32_t* off;
    int H, G, D, P, kmax, DP;
    int k[4];
    int ncells;
    int nprobe, max_tokens, buffer_pages, page_size;
    int32_t* sel_cell;
    int32_t* sel_offset;
    int32_t* sel_count;
    int32_t* sel_prefix;
    int32_t* n_sel;
    int32_t* n_rows;
    int sel_cap;
    int32_t* row_loc;  // [H][max_rows] or null
    int max_rows;
};

// Block-wide inclusive scan of one int per thread (1024 threads).
__device__ __forceinline__ int block_incl_scan(int v, int* sh, int& total) {
    const int incl = wave_incl_scan(v);
    const int wave = threadIdx.x >> 6;
    if (lane_id() == 63) sh[wave] = incl;
    __syncthreads();
    if (threadIdx.x < 64) {
        const int x = threadIdx.x < 16 ? sh[threadIdx.x] : 0;
        const int s = wave_incl_scan(x);
        if (threadIdx.x < 16) sh[16 + threadIdx.x] = s - x;
        if (threadIdx.x == 15) sh[32] = s;
    }
    __syncthreads();
    const int r = sh[16 + wave] + incl;
    total = sh[32];
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint64_t cell_key(uint32_t okey, int g) {
    return (static_cast<uint64_t>(okey) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(g));
}

__global__ __launch_bounds__(kSelThreads) void select_kernel(SelParams a) {
    extern __shared__ float smem[];
    __shared__ float qs[128];
    __shared__ float p1[256];
    __shared__ int hist[kBins];
    __shared__ int sh[48];
    __shared__ int shv[8];
    __shared__ float shf[32];

    const int h = blockIdx.x;
    const int tid = threadIdx.x;
    const int k0 = a.k[0], k1 = a.k[1];
    const int DP = a.DP;
    float* cT = smem;  // [DP][k1] during scoring; reused for candidates
    uint64_t* ck = reinterpret_cast<uint64_t*>(smem);
    int* cs = reinterpret_cast<int*>(ck + kCap);

    // 1. grouped-query sum (compute_impl.cu:80-87)
    if (tid < a.D) {
        float acc = 0.0f;
        for (int g = 0; g < a.G; ++g) acc += bf16_to_f32(a.q[(static_cast<int64_t>(h) * a.G + g) * a.D + tid]);
        qs[tid] = acc;
    }
    const float* c0 = a.cent + (static_cast<int64_t>(h) * a.P + 0) * a.kmax * DP;
    const float* c1 = a.cent + (static_cast<int64_t>(h) * a.P + 1) * a.kmax * DP;
    for (int i = tid; i < k1 * DP; i += kSelThreads) {
        const int j = i / DP, d = i - (i / DP) * DP;
        cT[d * k1 + j] = c1[static_cast<int64_t>(j) * DP + d];
    }
    __syncthreads();
    // 2. chain over the first subspace, once per l0
    if (tid < k0) {
        float acc = 0.0f;
        const float* row = c0 + static_cast<int64_t>(tid) * DP;
        for (int d = 0; d < DP; ++d) acc = __builtin_fmaf(qs[d], row[d], acc);
        p1[tid] = acc;
    }
    __syncthreads();

    // 3. scores of occupied cells (cell g = e * 1024 + tid)
    const int E = (a.ncells + kSelThreads - 1) / kSelThreads;
    const int32_t* cnt = a.cnt + static_cast<int64_t>(h) * a.ncells;
    float sc[kMaxE];
    int sz[kMaxE];
    int nvalid = 0;
    float smax = -INFINITY, smin = INFINITY;
#pragma unroll
    for (int e = 0; e < kMaxE; ++e) {
        sz[e] = 0;
        sc[e] = 0.0f;
        const int g = e * kSelThreads + tid;
        if (e < E && g < a.ncells) {
            const int n = cnt[g];
            if (n > 0) {
                const int i = g / k1, j = g - (g / k1) * k1;
                float s = p1[i];
                for (int d = 0; d < DP; ++d) s = __builtin_fmaf(qs[DP + d], cT[d * k1 + j], s);
                sc[e] = s;
                sz[e] = n;
                ++nvalid;
                smax = fmaxf(smax, s);
                smin = fminf(smin, s);
            }
        }
    }
    // block reductions
    {
        const int w = tid >> 6;
        const int nv = wave_sum_i(nvalid);
        const float mx = wave_max(smax);
        const float mn = -wave_max(-smin);
        if (lane_id() == 0) {
            shv[0] = 0;
            sh[w] = nv;
            shf[w] = mx;
            shf[16 + w] = mn;
        }
    }
    __syncthreads();
    if (tid == 0) {
        int nv = 0;
        float mx = -INFINITY, mn = INFINITY;
        for (int w = 0; w < 16; ++w) {
            nv += sh[w];
            mx = fmaxf(mx, shf[w]);
            mn = fminf(mn, shf[16 + w]);
        }
        shv[1] = nv;
        shf[0] = mx;
        shf[1] = mn;
    }
    for (int i = tid; i < kBins; i += kSelThreads) hist[i] = 0;
    __syncthreads();
    const int n_valid = shv[1];
    const float gmax = shf[0], gmin = shf[1];
    int kp = a.nprobe < a.buffer_pages ? a.nprobe : a.buffer_pages;
    kp = kp < n_valid ? kp : n_valid;
    int32_t* prefix_out = a.sel_prefix + static_cast<int64_t>(h) * (a.sel_cap + 1);
    if (kp <= 0) {
        if (tid == 0) {
            a.n_sel[h] = 0;
            a.n_rows[h] = 0;
            prefix_out[0] = 0;
        }
        return;
    }

    // 4. linear buckets: higher score -> lower or equal bucket
    const float range = gmax - gmin;
    const float inv = range > 0.0f ? static_cast<float>(kBins) / range : 0.0f;
    int bin[kMaxE];
#pragma unroll
    for (int e = 0; e < kMaxE; ++e) {
        int b = 0;
        if (sz[e] > 0) {
            const float t = (gmax - sc[e]) * inv;
            b = t < static_cast<float>(kBins - 1) ? static_cast<int>(t) : kBins - 1;
            atomicAdd(&hist[b], 1);
        }
        bin[e] = b;
    }
    __syncthreads();
    // bucket holding the kp-th best cell
    {
        const int b0 = 2 * tid, b1 = 2 * tid + 1;
        const int h0 = hist[b0], h1 = hist[b1];
        int total;
        const int incl = block_incl_scan(h0 + h1, sh, total);
        const int excl = incl - h0 - h1;
        if (excl < kp && excl + h0 >= kp) {
            shv[2] = b0;
            shv[3] = excl;
            shv[4] = excl + h0;
        } else if (excl + h0 < kp && incl >= kp) {
            shv[2] = b1;
            shv[3] = excl + h0;
            shv[4] = incl;
        }
    }
    __syncthreads();
    const int bK = shv[2], c_lt = shv[3], c_le = shv[4];
    uint64_t tau = 0;  // candidates of bucket bK need key >= tau
    if (c_le > kCap) {
        // exact: the (kp - c_lt)-th largest 64-bit key inside bucket bK
        int remaining = kp - c_lt;
        uint64_t prefix = 0, mask = 0;
        for (int pass = 0; pass < 8; ++pass) {
            const int shift = 56 - 8 * pass;
            for (int i = tid; i < 256; i += kSelThreads) hist[i] = 0;
            __syncthreads();
#pragma unroll
            for (int e = 0; e < kMaxE; ++e) {
                if (sz[e] > 0 && bin[e] == bK) {
                    const uint64_t key = cell_key(order_key(sc[e]), e * kSelThreads + tid);
                    if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255], 1);
                }
            }
            __syncthreads();
            if (tid < 64) {
                // lane l owns digits 255-4l .. 252-4l (descending order)
                int v[4], s = 0;
                for (int u = 0; u < 4; ++u) {
                    v[u] = hist[255 - 4 * tid - u];
                    s += v[u];
                }
                const int incl = wave_incl_scan(s);
                int run = incl - s;
                for (int u = 0; u < 4; ++u) {
                    if (run < remaining && run + v[u] >= remaining) {
                        shv[5] = 255 - 4 * tid - u;
                        shv[6] = run;
                    }
                    run += v[u];
                }
            }
            __syncthreads();
            const int digit = shv[5];
            remaining -= shv[6];
            prefix |= static_cast<uint64_t>(digit) << shift;
            mask |= static_cast<uint64_t>(255) << shift;
            __syncthreads();
        }
        tau = prefix;
    }

    // 5. gather candidates
#pragma unroll
    for (int e = 0; e < kMaxE; ++e) {
        if (sz[e] > 0) {
            const int g = e * kSelThreads + tid;
            const uint64_t key = cell_key(order_key(sc[e]), g);
            bool take = bin[e] < bK || (bin[e] == bK && (c_le <= kCap || key >= tau));
            if (take) {
                const int slot = atomicAdd(&shv[0], 1);
                ck[slot] = key;
                cs[slot] = sz[e];
            }
        }
    }
    __syncthreads();
    const int C = shv[0];
    int NP = 1;
    while (NP < C) NP <<= 1;
    for (int i = C + tid; i < NP; i += kSelThreads) {
        ck[i] = 0;
        cs[i] = 0;
    }
    __syncthreads();
    // 6. bitonic sort, descending by key
    for (int kk = 2; kk <= NP; kk <<= 1) {
        for (int j = kk >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < NP; i += kSelThreads) {
                const int l = i ^ j;
                if (l > i) {
                    const uint64_t x = ck[i], y = ck[l];
                    const bool up = (i & kk) == 0;
                    if (up ? (x < y) : (x > y)) {
                        ck[i] = y;
                        ck[l] = x;
                        const int t = cs[i];
                        cs[i] = cs[l];
                        cs[l] = t;
                    }
                }
            }
            __syncthreads();
        }
    }

    // 7. budget rules in rank order (ranks 4*tid .. 4*tid+3)
    int s4[4], pg4[4];
    int tsum = 0, psum = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int r = 4 * tid + u;
        s4[u] = r < C ? cs[r] : 0;
        pg4[u] = (s4[u] + a.page_size - 1) / a.page_size;
        tsum += s4[u];
        psum += pg4[u];
    }
    int ttot, ptot;
    const int tincl = block_incl_scan(tsum, sh, ttot);
    const int pincl = block_incl_scan(psum, sh, ptot);
    int texcl = tincl - tsum, pexcl = pincl - psum;
    int kept = 0;
    int excl_tok[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int r = 4 * tid + u;
        excl_tok[u] = texcl;
        pexcl += pg4[u];
        const bool keep = r < C && r < a.nprobe && texcl < a.max_tokens && pexcl <= a.buffer_pages;
        kept += keep ? 1 : 0;
        texcl += s4[u];
    }
    int m;
    block_incl_scan(kept, sh, m);
    // outputs for ranks < m
    int32_t* out_cell = a.sel_cell + static_cast<int64_t>(h) * a.sel_cap;
    int32_t* out_off = a.sel_offset + static_cast<int64_t>(h) * a.sel_cap;
    int32_t* out_cnt = a.sel_count + static_cast<int64_t>(h) * a.sel_cap;
    const int32_t* offs = a.off + static_cast<int64_t>(h) * (a.ncells + 1);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int r = 4 * tid + u;
        if (r < m) {
            const int g = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(ck[r] & 0xFFFFFFFFull));
            const int o = offs[g];
            out_cell[r] = g;
            out_off[r] = o;
            out_cnt[r] = s4[u];
            prefix_out[r] = excl_tok[u];
            if (a.row_loc) {
                int32_t* rl = a.row_loc + static_cast<int64_t>(h) * a.max_rows + excl_tok[u];
                for (int i = 0; i < s4[u]; ++i) rl[i] = o + i;
            }
        }
        if (r == m - 1) {
            prefix_out[m] = excl_tok[u] + s4[u];
            a.n_sel[h] = m;
            a.n_rows[h] = excl_tok[u] + s4[u];
        }
    }
    if (m == 0 && tid == 0) {
        a.n_sel[h] = 0;
        a.n_rows[h] = 0;
        prefix_out[0] = 0;
    }
}

// fused_query_group_similarities over compact merged centroids
// (compute_impl.cu:62-103), optional -inf mask (retrieval.py:357).
__global__ __launch_bounds__(256) void similarity_kernel(const uint16_t* q, const float* cent, float* out,
                                                         int64_t out_stride, const uint8_t* mask, int G, int N,
                                                         int D) {
    __shared__ float qs[512];
    const int h = blockIdx.y;
    for (int d = threadIdx.x; d < D; d += 256) {
        float acc = 0.0f;
        for (int g = 0; g < G; ++g) acc += bf16_to_f32(q[(static_cast<int64_t>(h) * G + g) * D + d]);
        qs[d] = acc;
    }
    __syncthreads();
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= N) return;
    const float* row = cent + (static_cast<int64_t>(h) * N + c) * D;
    float s = 0.0f;
    for (int d = 0; d < D; ++d) s = __builtin_fmaf(qs[d], row[d], s);
    if (mask && mask[static_cast<int64_t>(h) * N + c]) s = -INFINITY;
    out[static_cast<int64_t>(h) * out_stride + c] = s;
}

}  // namespace

int select_validate(const imi_select_args* a, int64_t& ncells, int& kmax) {
    IMI_REQUIRE(a != nullptr, IMI_ERR_INVALID, "imi_select: null args");
    IMI_REQUIRE(a->query && a->centroids && a->cell_count && a->cell_offset, IMI_ERR_INVALID,
                "imi_select: null input pointer");
    IMI_REQUIRE(a->kv_heads > 0 && a->groups > 0, IMI_ERR_INVALID, "imi_select: empty shape");
    IMI_REQUIRE(a->dim == 128, IMI_ERR_UNSUPPORTED, "imi_select: head_dim must be 128");
    IMI_REQUIRE(a->parts == 2, IMI_ERR_UNSUPPORTED, "imi_select: only 2-way IMI is implemented (parts=%d)",
                a->parts);
    IMI_REQUIRE(a->page_size > 0 && a->nprobe > 0 && a->max_tokens > 0 && a->buffer_pages > 0, IMI_ERR_INVALID,
                "imi_select: budgets must be positive");
    kmax = a->k[0] > a->k[1] ? a->k[0] : a->k[1];
    IMI_REQUIRE(a->k[0] >= 1 && a->k[1] >= 1 && kmax <= 256, IMI_ERR_UNSUPPORTED, "imi_select: k outside [1,256]");
    ncells = static_cast<int64_t>(a->k[0]) * a->k[1];
    IMI_REQUIRE(ncells <= static_cast<int64_t>(kMaxE) * kSelThreads, IMI_ERR_UNSUPPORTED,
                "imi_select: %lld cells exceed %d", static_cast<long long>(ncells), kMaxE * kSelThreads);
    const int kprime = a->nprobe < a->buffer_pages ? a->nprobe : a->buffer_pages;
    IMI_REQUIRE(kprime <= kCap, IMI_ERR_UNSUPPORTED, "imi_select: min(nprobe, buffer_pages)=%d exceeds %d", kprime,
                kCap);
    IMI_REQUIRE(a->sel_cap >= kprime, IMI_ERR_INVALID, "imi_select: sel_cap %d < min(nprobe, buffer_pages) %d",
                a->sel_cap, kprime);
    const int dp = a->dim / a->parts;
    const size_t lds = static_cast<size_t>(dp) * a->k[1] * 4;
    IMI_REQUIRE(lds <= kCap * 12, IMI_ERR_UNSUPPORTED, "imi_select: k too large for the LDS layout");
    return IMI_OK;
}

int select_launch(const imi_select_args* a, int32_t* row_loc, int max_rows, hipStream_t stream) {
    int64_t ncells;
    int kmax;
    int rc = select_validate(a, ncells, kmax);
    if (rc) return rc;
    IMI_REQUIRE(a->sel_cell && a->sel_offset && a->sel_count && a->sel_prefix && a->n_selected && a->n_rows,
                IMI_ERR_INVALID, "imi_select: null output pointer");
    SelParams p;
    p.q = a->query;
    p.cent = a->centroids;
    p.cnt = a->cell_count;
    p.off = a->cell_offset;
    p.H = a->kv_heads;
    p.G = a->groups;
    p.D = a->dim;
    p.P = a->parts;
    p.kmax = kmax;
    p.DP = a->dim / a->parts;
    for (int i = 0; i < 4; ++i) p.k[i] = a->k[i];
    p.ncells = static_cast<int>(ncells);
    p.nprobe = a->nprobe;
    p.max_tokens = a->max_tokens;
    p.buffer_pages = a->buffer_pages;
    p.page_size = a->page_size;
    p.sel_cell = a->sel_cell;
    p.sel_offset = a->sel_offset;
    p.sel_count = a->sel_count;
    p.sel_prefix = a->sel_prefix;
    p.n_sel = a->n_selected;
    p.n_rows = a->n_rows;
    p.sel_cap = a->sel_cap;
    p.row_loc = row_loc;
    p.max_rows = max_rows;
    const size_t lds = kCap * 12;
    static bool attr_set = false;
    if (!attr_set) {
        IMI_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&select_kernel),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        attr_set = true;
    }
    hipLaunchKernelGGL(select_kernel, dim3(a->kv_heads), dim3(kSelThreads), lds, stream, p);
    IMI_LAUNCH_CHECK("select_kernel");
    return IMI_OK;
}

}  // namespace imi

using namespace imi;

extern "C" int imi_select(const imi_select_args* a, imi_stream_t stream) {
    clear_error();
    return select_launch(a, nullptr, 0, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int imi_fused_query_group_similarities(const uint16_t* query, const float* centroids, float* out,
                                                  int64_t out_stride, const uint8_t* mask, int32_t kv_heads,
                                                  int32_t groups, int32_t n_clusters, int32_t dim,
                                                  imi_stream_t stream) {
    clear_error();
    IMI_REQUIRE(query && centroids && out, IMI_ERR_INVALID, "fused_query_group_similarities: null pointer");
    IMI_REQUIRE(kv_heads > 0 && groups > 0 && n_clusters > 0, IMI_ERR_INVALID,
                "fused_query_group_similarities: empty shape");
    IMI_REQUIRE(dim > 0 && dim <= 512, IMI_ERR_UNSUPPORTED, "fused_query_group_similarities: dim %d unsupported", dim);
    IMI_REQUIRE(out_stride >= n_clusters, IMI_ERR_INVALID, "fused_query_group_similarities: out_stride too small");
    hipLaunchKernelGGL(similarity_kernel, dim3((n_clusters + 255) / 256, kv_heads), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), query, centroids, out, out_stride, mask, groups,
                       n_clusters, dim);
    IMI_LAUNCH_CHECK("similarity_kernel");
    return IMI_OK;
}
