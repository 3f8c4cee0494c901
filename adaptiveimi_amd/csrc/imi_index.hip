// IMI cell index on gfx950: stable cell order, CSR over global cells, compact
// metadata and the K/V row permutation.
//
// Reference: library/AdaptiveIMI/cpp_extensions/src/reorganize_core.cpp
//   build_compact_reorg_input   18-85 (2-way), 87-176 (4-way)
//   reorganize_single_head      234-311 (stable counting sort by compact cell,
//                               then the K/V row copy)
// and the padded metadata of pipeline_bindings.cpp:206-276 /
// indexing.py:108-174.
//
// The cell order is produced by an LSD sort with one stable counting pass per
// subspace label (last subspace first), which yields tokens ordered by
// (l0, l1, ..., token) = (global cell id, token): the reference's CSR order,
// because compact ids are ranks of global ids.  IVF (one subspace, the
// cluster label is the cell id; build_compact_reorg_input_ivf, 178-231) is
// the one-pass case.
#include "imi_common.hpp"
#include "imi_sort.hpp"

namespace imi {
namespace {

struct IxParams {
    const int32_t* labels;  // [H][P][T]
    int H, T, P, kmax;
    int k[4];
    int64_t ncells;
    int nblk;
    int32_t* hist;   // [H][kmax][nblk]
    int32_t* rank;   // [H][T]
    int32_t* cid;    // [H][ncells] compact id scratch
    int32_t* sums;   // [H][nchunk][2] per-chunk row and occupied totals
};

__host__ __device__ inline int bits_for(int n) {
    int b = 0;
    while ((1 << b) < n) ++b;
    return b;
}

constexpr int kIvfMaxK = 4096;   // IVF clusters per head

template <int NB>
__global__ __launch_bounds__(256) void ix_rank_kernel(IxParams a, int p, const int32_t* in) {
    __shared__ int wcnt[4 * NB];
    const int h = blockIdx.y, blk = blockIdx.x;
    const int pos = blk * 256 + threadIdx.x;
    const bool valid = pos < a.T;
    const int64_t hT = static_cast<int64_t>(h) * a.T;
    int digit = 0;
    if (valid) {
        const int item = in ? in[hT + pos] : pos;
        digit = a.labels[(static_cast<int64_t>(h) * a.P + p) * a.T + item];
    }
    const int r = block_digit_rank(digit, valid, a.k[p], bits_for(a.k[p]), wcnt,
                                   a.hist + static_cast<int64_t>(h) * a.kmax * a.nblk, a.nblk, blk);
    if (valid) a.rank[hT + pos] = r;
}

__global__ __launch_bounds__(1024) void ix_scan_kernel(IxParams a, int p) {
    __shared__ int sh[40];
    const int h = blockIdx.x;
    block_exclusive_scan_1024(a.hist + static_cast<int64_t>(h) * a.kmax * a.nblk,
                              static_cast<int64_t>(a.k[p]) * a.nblk, sh);
}

__global__ __launch_bounds__(256) void ix_scatter_kernel(IxParams a, int p, const int32_t* in, int32_t* out) {
    const int h = blockIdx.y, blk = blockIdx.x;
    const int pos = blk * 256 + threadIdx.x;
    if (pos >= a.T) return;
    const int64_t hT = static_cast<int64_t>(h) * a.T;
    const int item = in ? in[hT + pos] : pos;
    const int digit = a.labels[(static_cast<int64_t>(h) * a.P + p) * a.T + item];
    const int dst = a.hist[(static_cast<int64_t>(h) * a.kmax + digit) * a.nblk + blk] + a.rank[hT + pos];
    out[hT + dst] = item;
}

__device__ __forceinline__ int64_t cell_of(const IxParams& a, int h, int t) {
    int64_t g = 0;
    for (int p = 0; p < a.P; ++p) g = g * a.k[p] + a.labels[(static_cast<int64_t>(h) * a.P + p) * a.T + t];
    return g;
}

__global__ void ix_zero_kernel(int32_t* x, int64_t n) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        x[i] = 0;
}

// Cell counts over the tokens in cell order (perm = the stable cell sort):
// equal cells are contiguous, so each wave adds one count per run of equal
// cells (one atomic per run instead of one per token).
__global__ __launch_bounds__(256) void ix_count_kernel(IxParams a, const int32_t* perm, int32_t* count) {
    const int h = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int lane = lane_id();
    const int64_t c = i < a.T ? cell_of(a, h, perm[static_cast<int64_t>(h) * a.T + i]) : -1;
    const int64_t cp = __shfl(c, lane > 0 ? lane - 1 : 0);
    const uint64_t starts = __builtin_amdgcn_ballot_w64(lane == 0 || c != cp);
    if (c >= 0 && (lane == 0 || c != cp)) {
        const uint64_t after = lane < 63 ? starts >> (lane + 1) : 0ull;
        const int len = after ? __builtin_ctzll(after) + 1 : 64 - lane;
        atomicAdd(&count[static_cast<int64_t>(h) * a.ncells + c], len);
    }
}

constexpr int kOffCells = 8192;                 // cells per workgroup of the offset scan
constexpr int kOffPT = kOffCells / 256;         // 32 consecutive cells per thread

// Inclusive scan of two ints over a 256-thread block; totals in tx / ty.
__device__ __forceinline__ void block_scan2_256(int& x, int& y, int* sh, int& tx, int& ty) {
    const int ix = wave_incl_scan(x), iy = wave_incl_scan(y);
    const int w = threadIdx.x >> 6;
    if (lane_id() == 63) {
        sh[w] = ix;
        sh[4 + w] = iy;
    }
    __syncthreads();
    int bx = 0, by = 0;
    tx = 0;
    ty = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (j < w) {
            bx += sh[j];
            by += sh[4 + j];
        }
        tx += sh[j];
        ty += sh[4 + j];
    }
    x = bx + ix;
    y = by + iy;
    __syncthreads();
}

// Per chunk of kOffCells global cells: the row count and the occupied cells.
__global__ __launch_bounds__(256) void ix_chunk_sums_kernel(IxParams a, const int32_t* count, int32_t* sums,
                                                            int nchunk) {
    __shared__ int sh[8];
    const int h = blockIdx.y, chunk = blockIdx.x, tid = threadIdx.x;
    const int32_t* c = count + static_cast<int64_t>(h) * a.ncells;
    int t = 0, o = 0;
#pragma unroll 8
    for (int u = 0; u < kOffPT; ++u) {
        const int64_t g = static_cast<int64_t>(chunk) * kOffCells + u * 256 + tid;
        const int v = g < a.ncells ? c[g] : 0;
        t += v;
        o += v > 0 ? 1 : 0;
    }
    int tt, to;
    block_scan2_256(t, o, sh, tt, to);
    if (tid == 0) {
        sums[(static_cast<int64_t>(h) * nchunk + chunk) * 2 + 0] = tt;
        sums[(static_cast<int64_t>(h) * nchunk + chunk) * 2 + 1] = to;
    }
}

// offsets[h][g] = exclusive prefix of count (offsets[h][ncells] = T); when
// compact metadata is requested also cid[h][g] = exclusive prefix of the
// occupied flags and n_active[h].  One workgroup per chunk: its base is the
// sum of the chunk totals before it, then 32 consecutive cells per thread.
__global__ __launch_bounds__(256) void ix_offsets_kernel(IxParams a, const int32_t* count, int32_t* offset,
                                                         int32_t* n_active, const int32_t* sums, int nchunk) {
    __shared__ int sh[8];
    const int h = blockIdx.y, chunk = blockIdx.x, tid = threadIdx.x;
    const int32_t* c = count + static_cast<int64_t>(h) * a.ncells;
    int32_t* o = offset + static_cast<int64_t>(h) * (a.ncells + 1);
    const int64_t g0 = static_cast<int64_t>(chunk) * kOffCells + static_cast<int64_t>(tid) * kOffPT;
    int v[kOffPT];
    if (g0 + kOffPT <= a.ncells && (reinterpret_cast<uintptr_t>(c + g0) & 15) == 0) {
#pragma unroll
        for (int u = 0; u < kOffPT / 4; ++u) {
            const int4 q = reinterpret_cast<const int4*>(c + g0)[u];
            v[4 * u + 0] = q.x;
            v[4 * u + 1] = q.y;
            v[4 * u + 2] = q.z;
            v[4 * u + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int u = 0; u < kOffPT; ++u) v[u] = g0 + u < a.ncells ? c[g0 + u] : 0;
    }
    int bt = 0, bo = 0;
    for (int i = tid; i < chunk; i += 256) {
        bt += sums[(static_cast<int64_t>(h) * nchunk + i) * 2 + 0];
        bo += sums[(static_cast<int64_t>(h) * nchunk + i) * 2 + 1];
    }
    int btt, bot;
    block_scan2_256(bt, bo, sh, btt, bot);
    int lt = 0, lo = 0;
#pragma unroll
    for (int u = 0; u < kOffPT; ++u) {
        lt += v[u];
        lo += v[u] > 0 ? 1 : 0;
    }
    int et = lt, eo = lo, tt, to;
    block_scan2_256(et, eo, sh, tt, to);
    int rt = btt + et - lt, ro = bot + eo - lo;
    int32_t* id = a.cid ? a.cid + static_cast<int64_t>(h) * a.ncells : nullptr;
    int ov[kOffPT], iv[kOffPT];
#pragma unroll
    for (int u = 0; u < kOffPT; ++u) {
        ov[u] = rt;
        iv[u] = ro;
        rt += v[u];
        ro += v[u] > 0 ? 1 : 0;
    }
    // 16-byte stores where the row allows them (the offset rows start at
    // h * (ncells + 1), so their alignment varies with h)
    const bool o_vec = g0 + kOffPT <= a.ncells && (reinterpret_cast<uintptr_t>(o + g0) & 15) == 0;
    const bool i_vec = id && g0 + kOffPT <= a.ncells && (reinterpret_cast<uintptr_t>(id + g0) & 15) == 0;
#pragma unroll
    for (int u = 0; u < kOffPT / 4; ++u) {
        if (o_vec) reinterpret_cast<int4*>(o + g0)[u] = make_int4(ov[4 * u], ov[4 * u + 1], ov[4 * u + 2], ov[4 * u + 3]);
        if (i_vec) reinterpret_cast<int4*>(id + g0)[u] = make_int4(iv[4 * u], iv[4 * u + 1], iv[4 * u + 2], iv[4 * u + 3]);
    }
#pragma unroll
    for (int u = 0; u < kOffPT; ++u) {
        if (g0 + u >= a.ncells) continue;
        if (!o_vec) o[g0 + u] = ov[u];
        if (id && !i_vec) id[g0 + u] = iv[u];
    }
    if (chunk == nchunk - 1 && tid == 0) {
        o[a.ncells] = btt + tt;
        if (id) n_active[h] = bot + to;
    }
}

struct CompactOut {
    int n_c;
    const float* cent;  // [H][P][kmax][DP]
    int DP, D;
    int32_t* gid;
    int32_t* size;
    int32_t* offset;
    float* merged;
    uint8_t* mask;
};

// One thread per global cell: an occupied cell writes its compact slot.
__global__ __launch_bounds__(256) void ix_compact_fill_kernel(IxParams a, CompactOut o, const int32_t* count,
                                                              const int32_t* offset) {
    const int h = blockIdx.y;
    const int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (g >= a.ncells) return;
    const int cnt = count[static_cast<int64_t>(h) * a.ncells + g];
    if (cnt == 0) return;
    const int c = a.cid[static_cast<int64_t>(h) * a.ncells + g];
    const int64_t hc = static_cast<int64_t>(h) * o.n_c + c;
    o.gid[hc] = static_cast<int32_t>(g);
    o.size[hc] = cnt;
    o.offset[static_cast<int64_t>(h) * (o.n_c + 1) + c] = offset[static_cast<int64_t>(h) * (a.ncells + 1) + g];
    if (o.mask) o.mask[hc] = 0;
}

// One wave per occupied compact slot: merged centroid = [C_0[l0] | C_1[l1] | ...].
__global__ __launch_bounds__(256) void ix_compact_merged_kernel(IxParams a, CompactOut o, const int32_t* n_active) {
    const int h = blockIdx.y;
    const int c = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (c >= min(n_active[h], o.n_c)) return;
    const int64_t hc = static_cast<int64_t>(h) * o.n_c + c;
    int64_t rem = o.gid[hc];
    int lab[4] = {0, 0, 0, 0};
    for (int p = a.P - 1; p >= 0; --p) {
        lab[p] = static_cast<int>(rem % a.k[p]);
        rem /= a.k[p];
    }
    for (int d = lane_id(); d < o.D; d += 64) {
        const int p = d / o.DP;
        o.merged[hc * o.D + d] =
            o.cent[((static_cast<int64_t>(h) * a.P + p) * a.kmax + lab[p]) * o.DP + (d - p * o.DP)];
    }
}

// Padding slots c >= n_active (and the closing offset).
__global__ __launch_bounds__(256) void ix_compact_pad_kernel(IxParams a, CompactOut o, const int32_t* n_active) {
    const int h = blockIdx.y;
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int na = n_active[h];
    if (c == 0) o.offset[static_cast<int64_t>(h) * (o.n_c + 1) + o.n_c] = a.T;
    if (c >= o.n_c || c < na) return;
    const int64_t hc = static_cast<int64_t>(h) * o.n_c + c;
    o.gid[hc] = -1;
    o.size[hc] = 0;
    o.offset[static_cast<int64_t>(h) * (o.n_c + 1) + c] = a.T;
    if (o.mask) o.mask[hc] = 1;
    if (o.merged)
        for (int d = 0; d < o.D; ++d) o.merged[hc * o.D + d] = 0.0f;
}

// list[h][pos] = src[h][perm[h][pos]] for keys and values; 16 lanes per
// 256-byte row, 16 rows per wave with every load issued before any store.
// Loads and stores are non-temporal (each byte is touched once) and the
// loads unconditional (rows past T re-read token 0 and are not stored): 1.07
// GB per layer at configs[1] in ~150 us, against ~237 us with cached,
// predicated loads and stores.  (32 rows per wave, twice the loads in
// flight, ran at 3.1 TB/s even on the identity permutation.)
constexpr int kPermRowsPerWave = 16;
typedef unsigned int ix_u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void ix_permute_kernel(const uint16_t* keys, const uint16_t* values, int64_t hs,
                                                         int64_t ts, int T, const int32_t* perm, uint16_t* lk,
                                                         uint16_t* lv, int64_t list_rows) {
    const int h = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = lane_id();
    const int rg = lane >> 4, li = lane & 15;
    const int base = (blockIdx.x * 4 + wave) * kPermRowsPerWave;
    const int my = base + lane;
    const int tok = (lane < kPermRowsPerWave && my < T) ? perm[static_cast<int64_t>(h) * T + my] : 0;
    constexpr int IT = kPermRowsPerWave / 4;
    ix_u32x4_t kv[IT], vv[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int t = __shfl(tok, it * 4 + rg);
        const int64_t so = h * hs + static_cast<int64_t>(t) * ts + li * 8;
        kv[it] = __builtin_nontemporal_load(reinterpret_cast<const ix_u32x4_t*>(keys + so));
        vv[it] = __builtin_nontemporal_load(reinterpret_cast<const ix_u32x4_t*>(values + so));
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int pos = base + it * 4 + rg;
        if (pos < T) {
            const int64_t dofs = (static_cast<int64_t>(h) * list_rows + pos) * 128 + li * 8;
            __builtin_nontemporal_store(kv[it], reinterpret_cast<ix_u32x4_t*>(lk + dofs));
            __builtin_nontemporal_store(vv[it], reinterpret_cast<ix_u32x4_t*>(lv + dofs));
        }
    }
}

int validate(const imi_index_args* a, int& kmax, int64_t& ncells) {
    IMI_REQUIRE(a != nullptr, IMI_ERR_INVALID, "imi_build_index: null args");
    IMI_REQUIRE(a->keys && a->values && a->labels && a->cell_count && a->cell_offset && a->perm &&
                    a->list_keys && a->list_values,
                IMI_ERR_INVALID, "imi_build_index: null pointer argument");
    IMI_REQUIRE(a->kv_heads > 0 && a->n_tokens > 0, IMI_ERR_INVALID, "imi_build_index: empty input");
    IMI_REQUIRE(a->dim == 128, IMI_ERR_UNSUPPORTED, "imi_build_index: head_dim must be 128 (got %d)", a->dim);
    IMI_REQUIRE(a->parts == 1 || a->parts == 2 || a->parts == 4, IMI_ERR_UNSUPPORTED,
                "imi_build_index: parts must be 1 (IVF), 2 or 4");
    IMI_REQUIRE(a->list_rows >= a->n_tokens, IMI_ERR_INVALID, "imi_build_index: list_rows %lld < n_tokens %d",
                static_cast<long long>(a->list_rows), a->n_tokens);
    IMI_REQUIRE((a->token_stride % 8) == 0 && (a->head_stride % 8) == 0, IMI_ERR_INVALID,
                "imi_build_index: strides must be multiples of 8 elements");
    kmax = 0;
    ncells = 1;
    const int kcap = a->parts == 1 ? kIvfMaxK : kImiMaxK;
    for (int p = 0; p < a->parts; ++p) {
        IMI_REQUIRE(a->k[p] >= 1 && a->k[p] <= kcap, IMI_ERR_UNSUPPORTED, "imi_build_index: k[%d]=%d outside [1,%d]",
                    p, a->k[p], kcap);
        kmax = a->k[p] > kmax ? a->k[p] : kmax;
        ncells *= a->k[p];
    }
    IMI_REQUIRE(ncells <= (int64_t(1) << 26), IMI_ERR_UNSUPPORTED, "imi_build_index: %lld cells exceed 2^26",
                static_cast<long long>(ncells));
    const bool compact = a->compact_gid || a->compact_size || a->compact_offset || a->compact_centroids ||
                         a->compact_mask || a->n_active;
    if (compact) {
        IMI_REQUIRE(a->compact_gid && a->compact_size && a->compact_offset && a->n_active, IMI_ERR_INVALID,
                    "imi_build_index: compact gid, size, offset and n_active must be all set or all NULL");
        IMI_REQUIRE(!a->compact_centroids || a->centroids, IMI_ERR_INVALID,
                    "imi_build_index: merged compact centroids need the subspace centroids");
        const int64_t max_active = ncells < a->n_tokens ? ncells : a->n_tokens;
        IMI_REQUIRE(a->n_centroids >= max_active, IMI_ERR_INVALID,
                    "imi_build_index: n_centroids %d < possible occupied cells %lld", a->n_centroids,
                    static_cast<long long>(max_active));
    }
    return IMI_OK;
}

size_t workspace_bytes(const imi_index_args* a, int kmax, int64_t ncells, IxParams* p, int32_t** tmp) {
    const int nblk = (a->n_tokens + 255) / 256;
    Carver cv(a->workspace);
    IxParams q{};
    q.hist = cv.take<int32_t>(static_cast<size_t>(a->kv_heads) * kmax * nblk);
    q.rank = cv.take<int32_t>(static_cast<size_t>(a->kv_heads) * a->n_tokens);
    q.cid = cv.take<int32_t>(static_cast<size_t>(a->kv_heads) * ncells);
    q.sums = cv.take<int32_t>(static_cast<size_t>(a->kv_heads) * 2 * ((ncells + kOffCells - 1) / kOffCells));
    int32_t* t = cv.take<int32_t>(static_cast<size_t>(a->kv_heads) * a->n_tokens);
    if (p) *p = q;
    if (tmp) *tmp = t;
    return cv.used();
}

}  // namespace
}  // namespace imi

using namespace imi;

extern "C" int imi_index_workspace_size(const imi_index_args* a, size_t* bytes) {
    clear_error();
    int kmax;
    int64_t ncells;
    int rc = validate(a, kmax, ncells);
    if (rc) return rc;
    IMI_REQUIRE(bytes != nullptr, IMI_ERR_INVALID, "imi_index_workspace_size: null output");
    imi_index_args tmp = *a;
    tmp.workspace = nullptr;
    *bytes = workspace_bytes(&tmp, kmax, ncells, nullptr, nullptr);
    return IMI_OK;
}

extern "C" int imi_build_index(const imi_index_args* a, imi_stream_t stream_) {
    clear_error();
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    int kmax;
    int64_t ncells;
    int rc = validate(a, kmax, ncells);
    if (rc) return rc;
    imi_index_args tmp = *a;
    tmp.workspace = nullptr;
    const size_t need = workspace_bytes(&tmp, kmax, ncells, nullptr, nullptr);
    IMI_REQUIRE(a->workspace != nullptr && a->workspace_bytes >= need, IMI_ERR_WORKSPACE,
                "imi_build_index: workspace %zu bytes < %zu required", a->workspace_bytes, need);
    IxParams p;
    int32_t* scratch;
    workspace_bytes(a, kmax, ncells, &p, &scratch);
    p.labels = a->labels;
    p.H = a->kv_heads;
    p.T = a->n_tokens;
    p.P = a->parts;
    p.kmax = kmax;
    for (int i = 0; i < 4; ++i) p.k[i] = i < a->parts ? a->k[i] : 1;
    p.ncells = ncells;
    p.nblk = (a->n_tokens + 255) / 256;
    const bool compact = a->compact_gid != nullptr;
    if (!compact) p.cid = nullptr;

    // LSD passes: last subspace first; the final pass lands in a->perm.
    const int32_t* in = nullptr;
    for (int pass = 0; pass < a->parts; ++pass) {
        const int part = a->parts - 1 - pass;
        int32_t* out = ((a->parts - 1 - pass) % 2 == 0) ? a->perm : scratch;
        if (a->k[part] <= 256)
            hipLaunchKernelGGL(ix_rank_kernel<256>, dim3(p.nblk, p.H), dim3(256), 0, stream, p, part, in);
        else
            hipLaunchKernelGGL(ix_rank_kernel<kIvfMaxK>, dim3(p.nblk, p.H), dim3(256), 0, stream, p, part, in);
        IMI_LAUNCH_CHECK("ix_rank_kernel");
        hipLaunchKernelGGL(ix_scan_kernel, dim3(p.H), dim3(1024), 0, stream, p, part);
        IMI_LAUNCH_CHECK("ix_scan_kernel");
        hipLaunchKernelGGL(ix_scatter_kernel, dim3(p.nblk, p.H), dim3(256), 0, stream, p, part, in, out);
        IMI_LAUNCH_CHECK("ix_scatter_kernel");
        in = out;
    }

    const int64_t cells_total = ncells * p.H;
    hipLaunchKernelGGL(ix_zero_kernel, dim3(static_cast<unsigned>((cells_total + 255) / 256 < 65535 ? (cells_total + 255) / 256 : 65535)),
                       dim3(256), 0, stream, a->cell_count, cells_total);
    IMI_LAUNCH_CHECK("ix_zero_kernel");
    hipLaunchKernelGGL(ix_count_kernel, dim3(p.nblk, p.H), dim3(256), 0, stream, p, a->perm, a->cell_count);
    IMI_LAUNCH_CHECK("ix_count_kernel");
    const int nchunk = static_cast<int>((ncells + kOffCells - 1) / kOffCells);
    hipLaunchKernelGGL(ix_chunk_sums_kernel, dim3(nchunk, p.H), dim3(256), 0, stream, p, a->cell_count, p.sums,
                       nchunk);
    IMI_LAUNCH_CHECK("ix_chunk_sums_kernel");
    hipLaunchKernelGGL(ix_offsets_kernel, dim3(nchunk, p.H), dim3(256), 0, stream, p, a->cell_count, a->cell_offset,
                       a->n_active, p.sums, nchunk);
    IMI_LAUNCH_CHECK("ix_offsets_kernel");

    if (compact) {
        CompactOut o;
        o.n_c = a->n_centroids;
        o.cent = a->centroids;
        o.D = a->dim;
        o.DP = a->dim / a->parts;
        o.gid = a->compact_gid;
        o.size = a->compact_size;
        o.offset = a->compact_offset;
        o.merged = a->compact_centroids;
        o.mask = a->compact_mask;
        hipLaunchKernelGGL(ix_compact_fill_kernel, dim3(static_cast<unsigned>((ncells + 255) / 256), p.H), dim3(256),
                           0, stream, p, o, a->cell_count, a->cell_offset);
        IMI_LAUNCH_CHECK("ix_compact_fill_kernel");
        if (o.merged) {
            hipLaunchKernelGGL(ix_compact_merged_kernel, dim3((o.n_c + 3) / 4, p.H), dim3(256), 0, stream, p, o,
                               a->n_active);
            IMI_LAUNCH_CHECK("ix_compact_merged_kernel");
        }
        hipLaunchKernelGGL(ix_compact_pad_kernel, dim3((o.n_c + 256) / 256, p.H), dim3(256), 0, stream, p, o,
                           a->n_active);
        IMI_LAUNCH_CHECK("ix_compact_pad_kernel");
    }

    hipLaunchKernelGGL(ix_permute_kernel, dim3((a->n_tokens + 4 * kPermRowsPerWave - 1) / (4 * kPermRowsPerWave), p.H),
                       dim3(256), 0, stream, a->keys,
                       a->values, a->head_stride, a->token_stride, a->n_tokens, a->perm, a->list_keys,
                       a->list_values, a->list_rows);
    IMI_LAUNCH_CHECK("ix_permute_kernel");
    return IMI_OK;
}
