// Per-step cell scoring and budget-bounded selection for a 4-way IMI on gfx950.
//
// Reference: the same path as the 2-way selection (compute_impl.cu:62-103
// scores over the padded compact cells, retrieval.py:295-303 and 357,
// wave_buffer_cpu_hotcold.cpp:303-371), with n_centroids = k^4 + 1 cells
// (runtime.py:35-38).  With k = 32 that is 1,048,576 cells, most of them
// empty, so the work runs over the occupied (compact) cells that
// imi_build_index lists in ascending global id:
//
//   sel4_score_kernel   16 occupied cells per thread, 16384 per workgroup:
//                       qsum (g ascending) and the 128-term FMA chain over
//                       [C0[l0] | C1[l1] | C2[l2] | C3[l3]] (the merged
//                       centroid, never materialised), continued from
//                       prefixes shared per (l0, l1) and (l0, l1, l2); key =
//                       (score, ~gid) so that key order is the reference rank
//                       order.  Each workgroup then lists its candidates:
//                       all its cells when they are at most K', else the
//                       cells in the buckets up to the one holding its own
//                       K'-th best cell (1024 linear buckets over its range),
//                       a superset of its share of the head's K' best.
//   sel4_final_kernel   one workgroup per head over the head's candidates:
//                       2048 linear buckets over their range, the bucket of
//                       the K'-th best, the candidates at or above it in LDS
//                       grouped by bucket and ranked inside their bucket by
//                       counting the better keys (a bitonic sort for a
//                       bucket over 512; an exact radix select over all
//                       candidates when more than 8192 are at or above it),
//                       then the token and page budgets in rank order.
// K' = min(nprobe, buffer_pages, occupied cells), or nprobe in tile mode and
// with the delta append.

// Outputs have the 2-way layout (cells in rank order, CSR offset, count,
// exclusive row prefix, m, rows), so the attention kernel is shared.  Each
// score workgroup writes its candidates to its own region of the workspace
// with its count and key range, and the final kernel reads only those: no
// workspace bytes have to start at zero and no global atomics are used.
#include "imi_common.hpp"

namespace imi {

size_t tile_delta_bytes(const imi_select_args* a);
int tile_delta_launch(const imi_select_args* a, void* scratch, hipStream_t stream);

namespace {

constexpr int kBins4 = 2048;
constexpr int kCand4 = 8192;     // candidates ranked in LDS per head
constexpr int kSegMax = 512;     // largest bucket ranked by counting (larger: a full sort)
constexpr int kRingSet = 2048;   // ring-code set of the delta match (ring <= 1024 entries)
constexpr int kK4 = 64;          // centroids per subspace the kernels hold
constexpr int kDp4 = 32;         // subspace width (D = 128, 4 parts)
constexpr int kMaxG4 = 16;       // query heads per KV head
constexpr int kScoreThreads = 256;   // 2-way score kernel
constexpr int kScore4Threads = 1024; // 4-way score kernel
constexpr int kFinalThreads = 1024;
constexpr int kSelCap4 = kCand4;  // cells to rank (K') per head
constexpr int kExtHeads = 1024;  // KV heads one call handles
constexpr int kCPT = 16;         // occupied cells per thread in the 4-way score kernel
constexpr int kCS4 = 36;         // LDS row stride of a subspace centroid (16-byte aligned rows)
constexpr int kTripCap = 8192;   // (l0, l1, l2) prefixes a score workgroup keeps
constexpr int kCellsPerBlock = kScore4Threads * kCPT;
constexpr int kFastCand = 2048;  // screened pass: candidates a score workgroup scores exactly
constexpr size_t kFastLds = static_cast<size_t>(kFastCand) * 12 + 2 * kK4 * 4;   // their (x0, gid, cell), d3 and A
constexpr int kDenseScoreCells = kScoreThreads;   // 2-way score kernel: one global cell per thread
constexpr int kDenseK = kImiMaxK;                 // 2-way centroids per subspace (k0 * k1 <= kMaxSeg * 256 cells)
constexpr int kIvfMaxK = 4096;                    // IVF clusters per head
constexpr int kLocBins = 1024;   // buckets of a score workgroup's own candidate cut
constexpr int kFinalCPT = 16;    // candidates per thread the final kernel holds in registers
constexpr int kMaxSeg = 1024;    // score workgroups per head the final kernel reads (candidate segments)

// Position of candidate j of score workgroup s (= h * nbs + b) in the list.
// A workgroup's candidates start at a staggered offset of its region
// (region is a power of two), so that the workgroups' first candidates do
// not all fall on the same memory channels.
__host__ __device__ __forceinline__ int64_t cand_pos(int64_t s, int j, int region) {
    return s * region + ((static_cast<int64_t>(s) * 520 + j) & (region - 1));
}

struct Sel4 {
    void* tile_scr;          // scratch of the tile-mode delta append (null: none)
    const uint16_t* q;
    const float* cent;       // [H][4][kmax][32]
    int H, G, kmax;
    int k[4];
    const int32_t* gid;      // [H][cap]
    const int32_t* csize;    // [H][cap]
    const int32_t* coff;     // [H][cap + 1]
    const int32_t* nact;     // [H]
    int cap;                 // cells listed per head (keys [H][cap])
    int dense;               // 2-way and IVF: every global cell listed (cell index = id, n_active = cap, key 0 = empty)
    int nprobe, max_tokens, buffer_pages, page_size;
    const int32_t* head_max_tokens;    // [H] or null
    const int32_t* head_buffer_pages;  // [H] or null
    int tile_mode;
    int32_t* sel_cell;
    int32_t* sel_offset;
    int32_t* sel_count;
    int32_t* sel_prefix;
    int32_t* n_sel;
    int32_t* n_rows;
    int sel_cap;
    int32_t* wcnt;           // [H][nbs] candidates of each score workgroup
    int region;              // cells per score workgroup: workgroup b lists its candidates from b * region on
    uint64_t* cand;          // [H][nbs * region] candidate keys (any order inside a workgroup's region)
    int32_t* cidx;           // [H][nbs * region] their cell indices
    uint32_t* rpart;         // [H][nbs][2]: per score workgroup, max order key and max ~order key of its candidates
    int nbs;                 // score workgroups per head
    // online index maintenance: replaced centroids (by compact id) and the
    // delta ring
    const float* shadow;
    int shadow_rows;
    const int32_t* upd_slot;
    const int32_t* upd_row;
    const int32_t* ring_cell;
    const int32_t* ring_row;
    const int32_t* ring_n;
    int ring_cap;
    int exec_rows;
    int32_t* delta_rows;
    int32_t* n_delta;
    int fast4;               // the 4-way score kernel has LDS for its screened pass
};

__device__ __forceinline__ float key_score(uint64_t key) {
    const uint32_t o = static_cast<uint32_t>(key >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

__device__ __forceinline__ int bucket4(float s, float gmax, float inv) {
    const float t = (gmax - s) * inv;
    return t < static_cast<float>(kBins4 - 1) ? static_cast<int>(t) : kBins4 - 1;
}

// listed cells of head h, clamped to the array width
__device__ __forceinline__ int n_active(const Sel4& a, int h) {
    if (a.dense) return a.cap;
    const int na = a.nact[h];
    return na < 0 ? 0 : (na < a.cap ? na : a.cap);
}

// this head's budgets (ragged batches), bounded by the launch-wide ones
__device__ __forceinline__ int head_pages(const Sel4& a, int h) {
    return a.head_buffer_pages ? min(a.head_buffer_pages[h], a.buffer_pages) : a.buffer_pages;
}
__device__ __forceinline__ int head_tokens(const Sel4& a, int h) {
    return a.head_max_tokens ? min(a.head_max_tokens[h], a.max_tokens) : a.max_tokens;
}

// cells to rank: every kept cell costs a page except in tile mode, and the
// delta match needs the ranks the page cut drops
__device__ __forceinline__ int kprime(const Sel4& a, int h, int na) {
    const int bp = head_pages(a, h);
    int kp = (a.tile_mode || a.ring_cap > 0) ? a.nprobe : (a.nprobe < bp ? a.nprobe : bp);
    return kp < na ? kp : na;
}

// Cell-id digits: POW2 (every k a power of two, as when a runtime config
// sets k explicitly, e.g. 4 x 32; the adaptive k of
// layer_pipeline.cpp:177-228 usually is not, e.g. 7, 10, 11 or 13 for
// 32k-512k tokens) takes shifts and masks instead of integer divisions.
template <bool POW2>
__device__ __forceinline__ uint32_t kdiv(uint32_t g, uint32_t k) {
    return POW2 ? g >> __builtin_ctz(k) : g / k;
}
template <bool POW2>
__device__ __forceinline__ uint32_t kmod(uint32_t g, uint32_t k) {
    return POW2 ? g & (k - 1) : g % k;
}

// The candidates of one score workgroup (T threads, CPT keys per thread,
// key 0 = no cell, ci = cell index): all its cells when they are at most K',
// else the cells in the buckets up to the one holding its own K'-th best
// cell (kLocBins linear buckets over its range; the bucket index falls as
// the score rises, so these cells include every cell at or above that one,
// ties included: a superset of the workgroup's share of the head's K'
// best).  They go to the head's list at one atomic offset per workgroup, in
// any order, in this workgroup's own region of the list (no atomics: a
// contended device-scope atomic per workgroup cost several microseconds),
// with their count in wcnt; the workgroup's candidate range goes to rpart.
// lh: kLocBins ints of LDS, zero on entry.
template <int T, int CPT>
__device__ void emit_candidates(const Sel4& a, int h, int kp, const uint64_t (&kv)[CPT], const int (&ci)[CPT],
                                int* lh) {
    // Branch-free per-cell code throughout: the unrolled per-cell branches
    // of a first version made this routine several times slower (each
    // workgroup runs it once, so its code is fetched cold).
    constexpr int NW = T / 64;
    __shared__ uint32_t red[NW][3];
    __shared__ int s_bk;
    const int tid = threadIdx.x, w = tid >> 6;
    // valid cells and their range (order keys)
    int nv = 0;
    uint32_t kmax = 0, nkmin = 0;
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const bool valid = kv[u] != 0ull;
        const uint32_t ok = static_cast<uint32_t>(kv[u] >> 32);
        nv += valid ? 1 : 0;
        kmax = max(kmax, valid ? ok : 0u);
        nkmin = max(nkmin, valid ? ~ok : 0u);
    }
    nv = wave_sum_i(nv);
    kmax = wave_max_u32(kmax);
    nkmin = wave_max_u32(nkmin);
    if (lane_id() == 0) {
        red[w][0] = static_cast<uint32_t>(nv);
        red[w][1] = kmax;
        red[w][2] = nkmin;
    }
    if (tid == 0) s_bk = kp > 0 ? kLocBins : -1;   // every bucket: all cells are candidates; none
    __syncthreads();
    int nvb = 0;
    uint32_t bmax = 0, bnmin = 0;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        nvb += static_cast<int>(red[j][0]);
        bmax = max(bmax, red[j][1]);
        bnmin = max(bnmin, red[j][2]);
    }
    const float wmax = key_score(static_cast<uint64_t>(bmax) << 32);
    const float wmin = key_score(static_cast<uint64_t>(~bnmin) << 32);
    const float range = wmax - wmin;
    const float inv = range > 0.0f ? static_cast<float>(kLocBins) / range : 0.0f;
    int bu[CPT];   // bucket of each cell, kLocBins for no cell
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const float t = (wmax - key_score(kv[u])) * inv;
        const int b = t < static_cast<float>(kLocBins - 1) ? static_cast<int>(t) : kLocBins - 1;
        bu[u] = kv[u] != 0ull ? b : kLocBins;
    }
    if (nvb > kp && kp > 0) {   // workgroup-uniform
#pragma unroll
        for (int u = 0; u < CPT; ++u)
            if (bu[u] < kLocBins) atomicAdd(&lh[bu[u]], 1);   // (one shared slot for every empty cell serialised)
        __syncthreads();
        // the bucket holding the kp-th best: kLocBins / T buckets per thread
        constexpr int PB = kLocBins / T;
        int v[PB], loc = 0;
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            v[j] = lh[tid * PB + j];
            loc += v[j];
        }
        const int incl = wave_incl_scan(loc);
        __syncthreads();   // every histogram read is done: red is reused below
        if (lane_id() == 63) red[w][0] = static_cast<uint32_t>(incl);
        __syncthreads();
        int run = incl - loc;
        for (int j = 0; j < w; ++j) run += static_cast<int>(red[j][0]);
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            if (run < kp && run + v[j] >= kp) s_bk = tid * PB + j;
            run += v[j];
        }
        __syncthreads();
    }
    const int bk = s_bk < kLocBins ? s_bk : kLocBins - 1;   // bucket of the cut; -1: none
    // this workgroup's candidates, their offsets and range
    int cnt = 0;
    uint32_t cnmin = 0;
    uint32_t cmask = 0;   // bit u: cell u is a candidate
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const bool c = bu[u] <= bk;   // false for no cell (kLocBins) and for bk = -1
        cmask |= c ? 1u << u : 0u;
        cnt += c ? 1 : 0;
        cnmin = max(cnmin, c ? ~static_cast<uint32_t>(kv[u] >> 32) : 0u);
    }
    const int cincl = wave_incl_scan(cnt);
    cnmin = wave_max_u32(cnmin);
    __syncthreads();   // red is reused
    if (lane_id() == 63) red[w][0] = static_cast<uint32_t>(cincl);
    if (lane_id() == 0) red[w][2] = cnmin;
    __syncthreads();
    int before = cincl - cnt, tot = 0;
    uint32_t cmn = 0;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        before += j < w ? static_cast<int>(red[j][0]) : 0;
        tot += static_cast<int>(red[j][0]);
        cmn = max(cmn, red[j][2]);
    }
    if (tid == 0) {
        a.wcnt[static_cast<int64_t>(h) * a.nbs + blockIdx.x] = tot;
        a.rpart[(static_cast<int64_t>(h) * a.nbs + blockIdx.x) * 2 + 0] = tot > 0 ? bmax : 0u;
        a.rpart[(static_cast<int64_t>(h) * a.nbs + blockIdx.x) * 2 + 1] = tot > 0 ? cmn : 0u;
    }
    // tot <= T * CPT = region; a thread's candidates in cell order
    const int64_t sg = static_cast<int64_t>(h) * a.nbs + blockIdx.x;
#pragma unroll
    for (int u = 0; u < CPT; ++u)
        if (cmask & (1u << u)) {
            const int64_t pos = cand_pos(sg, before + __builtin_popcount(cmask & ((1u << u) - 1u)), a.region);
            a.cand[pos] = kv[u];
            a.cidx[pos] = ci[u];
        }
}

// Screened candidate cut of a 4-way score workgroup (no online update,
// K' <= 1024).  Each cell's score is the
// chain continued from its triple prefix x0 over C3[l3]; its approximation
// fl(x0 + d3[l3]), with d3 the same chain from zero, differs from it by at
// most gamma_66 (|x0| + A[l3]) (A = sum |q c| over the 32 terms; u = 2^-24,
// one rounding per fused multiply-add, the chains' errors plus the final
// add).  E = 2^-16 (max |x0| + max A) + 1e-30 bounds that with a 4x margin
// and covers subnormal results.  A threshold L with K' approximate scores at
// or above it (from the threads' largest approximate scores) has K' exact
// scores at or above L - E: the workgroup's K'-th best exact score is
// >= L - E, and each of its cells that can be among the head's K' best has
// an approximate score >= L - 2E.  Those cells (a few percent) get the exact chain and are
// listed with their keys; every other cell is skipped.  Returns false
// (workgroup-uniform) when the bound is not finite or more than kFastCand
// cells pass: the caller then scores every cell.
template <bool POW2>
__device__ bool screened_cut(const Sel4& a, int h, int kp, int c_first, int na, const uint32_t (&gv)[kCPT],
                             const float (&sv)[kCPT], uint32_t k3, float* fx0, uint32_t* fgid, int* fci,
                             const float* fd3, const float* fa3, uint32_t (*s_fw)[3], const float* qs,
                             const float* cs, int* lh) {
    constexpr int NW = kScore4Threads / 64;
    const int tid = threadIdx.x, w = tid >> 6, lane = lane_id();
    if (kp > kScore4Threads) return false;   // (per-head budgets beyond the host's bound)
    if (kp <= 0) {   // no cells to rank: no candidates
        if (tid == 0) {
            const int64_t sg = static_cast<int64_t>(h) * a.nbs + blockIdx.x;
            a.wcnt[sg] = 0;
            a.rpart[sg * 2 + 0] = 0u;
            a.rpart[sg * 2 + 1] = 0u;
        }
        return true;
    }
    uint32_t xmb = 0;   // non-negative floats (NaN above inf) as their bits
#pragma unroll
    for (int j = 0; j < NW; ++j) xmb = max(xmb, s_fw[j][0]);
    const float E = 0x1p-16f * (__uint_as_float(xmb) + fa3[0] * 1.0001f) + 1e-30f;   // fa3[0]: the largest A
    const bool ok = E < 1e30f;   // false for inf and NaN
    // Each thread's largest approximate key stands for one of its cells:
    // the smallest thread maximum L among the threads in the buckets that
    // reach K' (a 1024-bucket histogram of the thread maxima) has K' cells at
    // or above it, whatever the buckets' rounding.
    uint32_t tmax = 0;
    bool any = false;
    float ap[kCPT];   // approximate scores
#pragma unroll
    for (int u = 0; u < kCPT; ++u) {
        const bool in = c_first + u * kScore4Threads + tid < na;
        ap[u] = in ? sv[u] + fd3[kmod<POW2>(gv[u], k3)] : -INFINITY;
        if (in) tmax = max(tmax, order_key(ap[u]));
        any = any || in;
    }
    {
        const uint32_t hi = wave_max_u32(any ? tmax : 0u);
        const uint32_t nlo = wave_max_u32(any ? ~tmax : 0u);
        if (lane == 0) {
            s_fw[w][1] = hi;
            s_fw[w][2] = nlo;
        }
    }
    __syncthreads();
    uint32_t khi = 0, knlo = 0;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        khi = max(khi, s_fw[j][1]);
        knlo = max(knlo, s_fw[j][2]);
    }
    const float fhi = key_score(static_cast<uint64_t>(khi) << 32);
    const float flo = key_score(static_cast<uint64_t>(~knlo) << 32);
    const float span = fhi - flo;
    const float inv = span > 0.0f ? static_cast<float>(kLocBins) / span : 0.0f;
    int bt = kLocBins;   // no bucket
    if (any) {
        const float t = (fhi - key_score(static_cast<uint64_t>(tmax) << 32)) * inv;
        bt = t < static_cast<float>(kLocBins - 1) ? (t > 0.0f ? static_cast<int>(t) : 0) : kLocBins - 1;
        atomicAdd(&lh[bt], 1);
    }
    __syncthreads();
    {
        // bucket bk where the count reaches kp (one bucket per thread)
        constexpr int PB = kLocBins / kScore4Threads;
        static_assert(PB == 1, "one bucket per thread");
        const int v = lh[tid];
        const int incl = wave_incl_scan(v);
        if (lane == 63) s_fw[w][1] = static_cast<uint32_t>(incl);
        __syncthreads();
        int run = incl - v;
        for (int j = 0; j < w; ++j) run += static_cast<int>(s_fw[j][1]);
        if (run < kp && run + v >= kp) s_fw[0][2] = static_cast<uint32_t>(tid);   // one writer
        if (tid == kScore4Threads - 1 && run + v < kp) s_fw[0][2] = static_cast<uint32_t>(kLocBins);   // fewer than kp
        __syncthreads();
    }
    const int bk = static_cast<int>(s_fw[0][2]);
    uint32_t lmin = bt <= bk && any ? tmax : 0xFFFFFFFFu;
    lmin = ~wave_max_u32(~lmin);
    if (lane == 0) s_fw[w][1] = lmin;   // (the scan's totals were read before the last barrier)
    __syncthreads();
    uint32_t L = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < NW; ++j) L = min(L, s_fw[j][1]);
    if (bk >= kLocBins) L = 0u;   // fewer than kp thread maxima: every cell
    float thr = -INFINITY;        // L = 0: every cell passes
    if (L != 0u) {
        const float lf = key_score(static_cast<uint64_t>(L) << 32);
        thr = lf - (2.0f * E + fabsf(lf) * 0x1p-20f);   // the margin covers the subtraction's rounding
    }
    // the cells that pass, listed in LDS in thread order (a block scan of the
    // per-thread counts)
    uint32_t cm = 0;
    int cnt = 0;
#pragma unroll
    for (int u = 0; u < kCPT; ++u) {
        const bool c = c_first + u * kScore4Threads + tid < na && ap[u] >= thr;
        cm |= c ? 1u << u : 0u;
        cnt += c ? 1 : 0;
    }
    const int incl = wave_incl_scan(cnt);
    if (lane == 63) s_fw[w][2] = static_cast<uint32_t>(incl);
    __syncthreads();
    int before = incl - cnt, total = 0;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        before += j < w ? static_cast<int>(s_fw[j][2]) : 0;
        total += static_cast<int>(s_fw[j][2]);
    }
    if (!ok || total > kFastCand) return false;
#pragma unroll
    for (int u = 0; u < kCPT; ++u)
        if (cm & (1u << u)) {
            const int pos = before + __builtin_popcount(cm & ((1u << u) - 1u));
            fx0[pos] = sv[u];
            fgid[pos] = gv[u];
            fci[pos] = c_first + u * kScore4Threads + tid;
        }
    __syncthreads();
    const int64_t sg = static_cast<int64_t>(h) * a.nbs + blockIdx.x;
    uint32_t kmx = 0, knm = 0;
    for (int j = tid; j < total; j += kScore4Threads) {
        float x = fx0[j];
        const uint32_t g = fgid[j];
        const float* c3r = &cs[(3 * a.kmax + static_cast<int>(kmod<POW2>(g, k3))) * kCS4];
#pragma unroll 2
        for (int d4 = 0; d4 < kDp4 / 4; ++d4) {
            const float4 q4 = *reinterpret_cast<const float4*>(&qs[3 * kDp4 + 4 * d4]);
            const float4 c4 = *reinterpret_cast<const float4*>(&c3r[4 * d4]);
            x = __builtin_fmaf(q4.x, c4.x, x);
            x = __builtin_fmaf(q4.y, c4.y, x);
            x = __builtin_fmaf(q4.z, c4.z, x);
            x = __builtin_fmaf(q4.w, c4.w, x);
        }
        const uint32_t ok32 = order_key(x);
        const int64_t pos = cand_pos(sg, j, a.region);
        a.cand[pos] = (static_cast<uint64_t>(ok32) << 32) | (0xFFFFFFFFu - g);
        a.cidx[pos] = fci[j];
        kmx = max(kmx, ok32);
        knm = max(knm, ~ok32);
    }
    kmx = wave_max_u32(kmx);
    knm = wave_max_u32(knm);
    if (lane == 0) {
        s_fw[w][0] = kmx;
        s_fw[w][1] = knm;
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t m1 = 0, m2 = 0;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            m1 = max(m1, s_fw[j][0]);
            m2 = max(m2, s_fw[j][1]);
        }
        a.wcnt[sg] = total;
        a.rpart[sg * 2 + 0] = total > 0 ? m1 : 0u;
        a.rpart[sg * 2 + 1] = total > 0 ? m2 : 0u;
    }
    return true;
}

// Every cell of the workgroup as a candidate, scored exactly: the chain
// from sv (through C2) over C3[l3] (the screened cut's fallback).
template <bool POW2>
__device__ void dense_emit(const Sel4& a, int h, int c_first, int na, const uint32_t (&gv)[kCPT],
                           const float (&sv)[kCPT], uint32_t k3, uint32_t (*s_fw)[3], const float* qs,
                           const float* cs) {
    constexpr int NW = kScore4Threads / 64;
    const int tid = threadIdx.x, w = tid >> 6, lane = lane_id();
    const int64_t sg = static_cast<int64_t>(h) * a.nbs + blockIdx.x;
    float x[kCPT];
    int r3[kCPT];
#pragma unroll
    for (int u = 0; u < kCPT; ++u) {
        x[u] = sv[u];
        r3[u] = (3 * a.kmax + static_cast<int>(kmod<POW2>(gv[u], k3))) * kCS4;
    }
#pragma unroll 1
    for (int d4 = 0; d4 < kDp4 / 4; ++d4) {
        const float4 q4 = *reinterpret_cast<const float4*>(&qs[3 * kDp4 + 4 * d4]);
#pragma unroll
        for (int u = 0; u < kCPT; ++u) {
            const float4 c4 = *reinterpret_cast<const float4*>(&cs[r3[u] + 4 * d4]);
            x[u] = __builtin_fmaf(q4.x, c4.x, x[u]);
            x[u] = __builtin_fmaf(q4.y, c4.y, x[u]);
            x[u] = __builtin_fmaf(q4.z, c4.z, x[u]);
            x[u] = __builtin_fmaf(q4.w, c4.w, x[u]);
        }
    }
    uint32_t kmx = 0, knm = 0;
#pragma unroll
    for (int u = 0; u < kCPT; ++u) {
        const int loc = u * kScore4Threads + tid;
        if (c_first + loc < na) {
            const uint32_t o = order_key(x[u]);
            const int64_t pos = cand_pos(sg, loc, a.region);
            a.cand[pos] = (static_cast<uint64_t>(o) << 32) | (0xFFFFFFFFu - gv[u]);
            a.cidx[pos] = c_first + loc;
            kmx = max(kmx, o);
            knm = max(knm, ~o);
        }
    }
    kmx = wave_max_u32(kmx);
    knm = wave_max_u32(knm);
    __syncthreads();   // s_fw was read by every thread
    if (lane == 0) {
        s_fw[w][0] = kmx;
        s_fw[w][1] = knm;
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t m1 = 0, m2 = 0;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            m1 = max(m1, s_fw[j][0]);
            m2 = max(m2, s_fw[j][1]);
        }
        const int n = max(min(na - c_first, kCellsPerBlock), 0);
        a.wcnt[sg] = n;
        a.rpart[sg * 2 + 0] = n > 0 ? m1 : 0u;
        a.rpart[sg * 2 + 1] = n > 0 ? m2 : 0u;
    }
}

// ONLINE: replaced centroids / the delta ring (a separate instantiation).
template <bool ONLINE, bool POW2, bool FAST>
__global__ __launch_bounds__(kScore4Threads) void sel4_score_kernel(Sel4 a) {
    __shared__ __attribute__((aligned(16))) float qs[128];
    __shared__ int s_pair[2];
    __shared__ int s_trip[2];
    __shared__ int lh[kLocBins];   // the candidate cut's buckets
    // dynamic LDS, sized by the launch: C0..C3 rows [4][kmax][kCS4], the
    // chain over subspaces 0 and 1 per (l0, l1) pair this block uses
    // [k0 * k1], then the chain over subspaces 0..2 per (l0, l1, l2) [kTripCap]
    extern __shared__ __attribute__((aligned(16))) float s_dyn4[];
    float* cs = s_dyn4;                      // row r of subspace p at (p * kmax + r) * kCS4
    float* p01 = s_dyn4 + 4 * a.kmax * kCS4;
    const int pair_cap = a.k[0] * a.k[1];
    float* p012 = p01 + pair_cap;
    // screened pass (fast4): the candidates' chain prefix, global id and
    // cell index, and per l3 the chain over C3 from zero (d3) and the sum
    // of |q c| (A)
    float* fx0 = p012 + kTripCap;                                   // [kFastCand]
    uint32_t* fgid = reinterpret_cast<uint32_t*>(fx0 + kFastCand);  // [kFastCand]
    int* fci = reinterpret_cast<int*>(fgid + kFastCand);            // [kFastCand]
    float* fd3 = reinterpret_cast<float*>(fci + kFastCand);         // [kK4]
    float* fa3 = fd3 + kK4;                                         // [kK4]
    __shared__ uint32_t s_fw[kScore4Threads / 64][3];
    const int h = blockIdx.y, tid = threadIdx.x;
    // the block's cells (ascending global id): their ids, loaded with the
    // occupied-cell count (reads past it stay inside the [H][cap] arrays and
    // are masked once the count is known)
    uint32_t gv[kCPT];
#pragma unroll
    for (int u = 0; u < kCPT; ++u) {
        const int c = blockIdx.x * kCellsPerBlock + u * kScore4Threads + tid;
        gv[u] = c < a.cap ? static_cast<uint32_t>(a.gid[static_cast<int64_t>(h) * a.cap + c]) : 0u;
    }
    const int na = n_active(a, h);
#pragma unroll
    for (int u = 0; u < kCPT; ++u)
        if (static_cast<int>(blockIdx.x) * kCellsPerBlock + u * kScore4Threads + tid >= na) gv[u] = 0u;
    const int c_first = blockIdx.x * kCellsPerBlock;
    const int c_last = min(na, c_first + kCellsPerBlock) - 1;
    const uint32_t k23 = static_cast<uint32_t>(a.k[2]) * static_cast<uint32_t>(a.k[3]);
    const uint32_t k3 = static_cast<uint32_t>(a.k[3]), k2 = static_cast<uint32_t>(a.k[2]);
    // the range of (l0, l1) pairs and (l0, l1, l2) triples: from the first
    // cell (thread 0, u = 0) and the last one (its owner), both in registers
    if (c_first <= c_last) {
#pragma unroll
        for (int u = 0; u < kCPT; ++u) {
            const int c = c_first + u * kScore4Threads + tid;
            if (c == c_first) {
                s_pair[0] = static_cast<int>(kdiv<POW2>(gv[u], k23));
                s_trip[0] = static_cast<int>(kdiv<POW2>(gv[u], k3));
            }
            if (c == c_last) {
                s_pair[1] = static_cast<int>(kdiv<POW2>(gv[u], k23));
                s_trip[1] = static_cast<int>(kdiv<POW2>(gv[u], k3));
            }
        }
    }
    if (tid < 128) {
        // rows past G re-read row G - 1 (G >= 1) and are dropped from the
        // sum: unconditional loads, all in flight at once
        const uint16_t* qh = a.q + static_cast<int64_t>(h) * a.G * 128;
        uint16_t qv[kMaxG4];
        load_group_rows(qh, a.G, tid, qv);
        float acc = 0.0f;   // grouped-query sum, g ascending (compute_impl.cu:80-87)
#pragma unroll
        for (int g = 0; g < kMaxG4; ++g)
            if (g < a.G) acc += bf16_to_f32(qv[g]);
        qs[tid] = acc;
    }
    {
        // the four codebooks [4][kmax][32] as float4, every load in flight
        // at once, then to LDS at the padded row stride
        constexpr int kRowF4 = kDp4 / 4;
        const float4* cp = reinterpret_cast<const float4*>(a.cent + static_cast<int64_t>(h) * 4 * a.kmax * kDp4);
        const int n4 = 4 * a.kmax * kRowF4;
        float4 cv[4 * kK4 * kRowF4 / kScore4Threads];
#pragma unroll
        for (int u = 0; u < 4 * kK4 * kRowF4 / kScore4Threads; ++u) {
            const int i = tid + u * kScore4Threads;
            cv[u] = i < n4 ? cp[i] : make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4 * kK4 * kRowF4 / kScore4Threads; ++u) {
            const int i = tid + u * kScore4Threads;
            if (i < n4) *reinterpret_cast<float4*>(&cs[(i / kRowF4) * kCS4 + 4 * (i % kRowF4)]) = cv[u];
        }
    }
    for (int i = tid; i < kLocBins; i += kScore4Threads) lh[i] = 0;
    // no occupied cells here (a head with fewer than the grid covers): the
    // check waits for the count, so it comes after every load is issued
    if (c_first > c_last) {
        if (tid == 0) {
            const int64_t sg = static_cast<int64_t>(h) * a.nbs + blockIdx.x;
            a.wcnt[sg] = 0;
            a.rpart[sg * 2 + 0] = 0u;
            a.rpart[sg * 2 + 1] = 0u;
        }
        return;
    }
    __syncthreads();
    // The 128-term chain runs over C0[l0], C1[l1], C2[l2], C3[l3] in turn, so
    // its value after the first 64 terms depends on (l0, l1) only: computed
    // once per pair in the block's (contiguous) pair range, then continued per
    // cell over C2 and C3 -- the same multiply-adds in the same order.
    const int pa = c_first <= c_last ? s_pair[0] : 0;
    // (ids out of order or out of range would only give wrong scores: both ends are clamped)
    const int npair = c_first <= c_last ? min(max(s_pair[1] - s_pair[0] + 1, 0), pair_cap) : 0;
    for (int t = tid; t < npair; t += kScore4Threads) {
        const uint32_t pt = static_cast<uint32_t>(pa + t), k1 = static_cast<uint32_t>(a.k[1]);
        const int l0 = static_cast<int>(kdiv<POW2>(pt, k1)), l1 = static_cast<int>(kmod<POW2>(pt, k1));
        float s = 0.0f;
#pragma unroll
        for (int d4 = 0; d4 < kDp4 / 4; ++d4) {
            const float4 q4 = *reinterpret_cast<const float4*>(&qs[4 * d4]);
            const float4 c4 = *reinterpret_cast<const float4*>(&cs[l0 * kCS4 + 4 * d4]);
            s = __builtin_fmaf(q4.x, c4.x, s);
            s = __builtin_fmaf(q4.y, c4.y, s);
            s = __builtin_fmaf(q4.z, c4.z, s);
            s = __builtin_fmaf(q4.w, c4.w, s);
        }
#pragma unroll
        for (int d4 = 0; d4 < kDp4 / 4; ++d4) {
            const float4 q4 = *reinterpret_cast<const float4*>(&qs[kDp4 + 4 * d4]);
            const float4 c4 = *reinterpret_cast<const float4*>(&cs[(a.kmax + l1) * kCS4 + 4 * d4]);
            s = __builtin_fmaf(q4.x, c4.x, s);
            s = __builtin_fmaf(q4.y, c4.y, s);
            s = __builtin_fmaf(q4.z, c4.z, s);
            s = __builtin_fmaf(q4.w, c4.w, s);
        }
        p01[t] = s;
    }
    __syncthreads();
    // Every cell's chain continues from its pair prefix over C2[l2], then
    // C3[l3]; dims outer and the kCPT cells inner, so one broadcast read of
    // q feeds kCPT multiply-adds (each cell's chain keeps its order).  When
    // the block's (l0, l1, l2) range is short (dense heads), the chain
    // through C2 is also computed once per triple, and cells continue over
    // C3 only.
    float sv[kCPT];
    const int ta = c_first <= c_last ? s_trip[0] : 0;
    const int ntrip = c_first <= c_last ? s_trip[1] - s_trip[0] + 1 : 0;
    if (ntrip > 0 && ntrip <= kTripCap) {
        for (int t = tid; t < ntrip; t += kScore4Threads) {
            const int tg = ta + t;
            float x = p01[min(max(static_cast<int>(kdiv<POW2>(tg, k2)) - pa, 0), pair_cap - 1)];
            const float* c2r = &cs[(2 * a.kmax + static_cast<int>(kmod<POW2>(tg, k2))) * kCS4];
#pragma unroll
            for (int d4 = 0; d4 < kDp4 / 4; ++d4) {
                const float4 q4 = *reinterpret_cast<const float4*>(&qs[2 * kDp4 + 4 * d4]);
                const float4 c4 = *reinterpret_cast<const float4*>(&c2r[4 * d4]);
                x = __builtin_fmaf(q4.x, c4.x, x);
                x = __builtin_fmaf(q4.y, c4.y, x);
                x = __builtin_fmaf(q4.z, c4.z, x);
                x = __builtin_fmaf(q4.w, c4.w, x);
            }
            p012[t] = x;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kCPT; ++u)
            sv[u] = p012[min(max(static_cast<int>(kdiv<POW2>(gv[u], k3)) - ta, 0), kTripCap - 1)];
    } else {
        int r2[kCPT];   // LDS offsets of the rows C2[l2]
#pragma unroll
        for (int u = 0; u < kCPT; ++u) {
            r2[u] = (2 * a.kmax + static_cast<int>(kmod<POW2>(kdiv<POW2>(gv[u], k3), k2))) * kCS4;
            sv[u] = p01[min(max(static_cast<int>(kdiv<POW2>(gv[u], k23)) - pa, 0), pair_cap - 1)];
        }
#pragma unroll 1
        for (int d4 = 0; d4 < kDp4 / 4; ++d4) {
            const float4 q4 = *reinterpret_cast<const float4*>(&qs[2 * kDp4 + 4 * d4]);
#pragma unroll
            for (int u = 0; u < kCPT; ++u) {
                const float4 c4 = *reinterpret_cast<const float4*>(&cs[r2[u] + 4 * d4]);
                sv[u] = __builtin_fmaf(q4.x, c4.x, sv[u]);
                sv[u] = __builtin_fmaf(q4.y, c4.y, sv[u]);
                sv[u] = __builtin_fmaf(q4.z, c4.z, sv[u]);
                sv[u] = __builtin_fmaf(q4.w, c4.w, sv[u]);
            }
        }
    }
    if constexpr (FAST) {
        // sv: every cell's chain through C2.  The largest |prefix|, and per
        // l3 the chain over C3 from zero (d3) and the sum of |q c| (A), for
        // the screened cut; the cells it cannot settle are scored exactly.
        uint32_t xm = 0;   // fp32 bits of a non-negative value (NaN above inf)
#pragma unroll
        for (int u = 0; u < kCPT; ++u)
            if (c_first + u * kScore4Threads + tid < na) xm = max(xm, __float_as_uint(fabsf(sv[u])));
        xm = wave_max_u32(xm);
        if (lane_id() == 0) s_fw[tid >> 6][0] = xm;
        if (tid < 64) {   // wave 0: one l3 per lane (k3 <= 64), and the largest A
            float am = 0.0f;
            if (tid < static_cast<int>(k3)) {
                const float* c3r = &cs[(3 * a.kmax + tid) * kCS4];
                float d = 0.0f;
#pragma unroll 2
                for (int d4 = 0; d4 < kDp4 / 4; ++d4) {
                    const float4 q4 = *reinterpret_cast<const float4*>(&qs[3 * kDp4 + 4 * d4]);
                    const float4 c4 = *reinterpret_cast<const float4*>(&c3r[4 * d4]);
                    d = __builtin_fmaf(q4.x, c4.x, d);
                    d = __builtin_fmaf(q4.y, c4.y, d);
                    d = __builtin_fmaf(q4.z, c4.z, d);
                    d = __builtin_fmaf(q4.w, c4.w, d);
                    am += fabsf(q4.x * c4.x) + fabsf(q4.y * c4.y) + fabsf(q4.z * c4.z) + fabsf(q4.w * c4.w);
                }
                fd3[tid] = d;
            }
            const uint32_t amb = wave_max_u32(__float_as_uint(am));   // NaN above inf
            if (tid == 0) fa3[0] = __uint_as_float(amb);
        }
        __syncthreads();
        const int kp = kprime(a, h, na);
        if (!screened_cut<POW2>(a, h, kp, c_first, na, gv, sv, k3, fx0, fgid, fci, fd3, fa3, s_fw, qs, cs, lh))
            dense_emit<POW2>(a, h, c_first, na, gv, sv, k3, s_fw, qs, cs);
        return;
    }
    int r3[kCPT];   // LDS offsets of the rows C3[l3]
#pragma unroll
    for (int u = 0; u < kCPT; ++u) r3[u] = (3 * a.kmax + static_cast<int>(kmod<POW2>(gv[u], k3))) * kCS4;
#pragma unroll 1
    for (int d4 = 0; d4 < kDp4 / 4; ++d4) {
        const float4 q4 = *reinterpret_cast<const float4*>(&qs[3 * kDp4 + 4 * d4]);
#pragma unroll
        for (int u = 0; u < kCPT; ++u) {
            const float4 c4 = *reinterpret_cast<const float4*>(&cs[r3[u] + 4 * d4]);
            sv[u] = __builtin_fmaf(q4.x, c4.x, sv[u]);
            sv[u] = __builtin_fmaf(q4.y, c4.y, sv[u]);
            sv[u] = __builtin_fmaf(q4.z, c4.z, sv[u]);
            sv[u] = __builtin_fmaf(q4.w, c4.w, sv[u]);
        }
    }
    // replaced centroids (async_update.py:7-19): the override slots of the
    // thread's cells, then the shadow rows of the replaced ones, each set of
    // loads issued together (one round trip each; the second only when the
    // wave has a replaced cell)
    int srow[ONLINE ? kCPT : 1];
    uint32_t rmask = 0;
    if (ONLINE && a.upd_slot) {
#pragma unroll
        for (int u = 0; u < kCPT; ++u) {
            const int c = blockIdx.x * kCellsPerBlock + u * kScore4Threads + tid;
            srow[u] = a.upd_slot[static_cast<int64_t>(h) * a.cap + min(c, a.cap - 1)];
            if (c < na && srow[u] >= 0) rmask |= 1u << u;
        }
        if (__builtin_amdgcn_ballot_w64(rmask != 0) != 0ull) {
#pragma unroll
            for (int u = 0; u < kCPT; ++u) {
                const int us = min(max(srow[u], 0), a.shadow_rows - 1);
                srow[u] = min(max(a.upd_row[static_cast<int64_t>(h) * a.shadow_rows + us], 0), a.shadow_rows - 1);
            }
        }
    }
    uint64_t kv[kCPT];
    int ci[kCPT];
#pragma unroll
    for (int u = 0; u < kCPT; ++u) {
        const int c = blockIdx.x * kCellsPerBlock + u * kScore4Threads + tid;
        ci[u] = c;
        kv[u] = 0ull;
        if (c >= na) continue;
        float s = sv[u];
        if (ONLINE) {
            if (rmask & (1u << u)) {
                const float4* sr = reinterpret_cast<const float4*>(
                    a.shadow + (static_cast<int64_t>(h) * a.shadow_rows + srow[u]) * 128);
                s = 0.0f;
                for (int d4 = 0; d4 < 32; ++d4) {
                    const float4 v = sr[d4];
                    s = __builtin_fmaf(qs[4 * d4 + 0], v.x, s);
                    s = __builtin_fmaf(qs[4 * d4 + 1], v.y, s);
                    s = __builtin_fmaf(qs[4 * d4 + 2], v.z, s);
                    s = __builtin_fmaf(qs[4 * d4 + 3], v.w, s);
                }
            }
        }
        kv[u] = (static_cast<uint64_t>(order_key(s)) << 32) | (0xFFFFFFFFu - gv[u]);
    }
    emit_candidates<kScore4Threads, kCPT>(a, h, kprime(a, h, na), kv, ci, lh);
}

// 2-way IMI over every global cell g = l0 * k1 + l1 (the shapes beyond the
// one-kernel selection): the chain over C0[l0] once per l0 of the
// workgroup's 256-cell range (one thread per row), continued per cell over
// C1[l1] held in registers -- the same fused multiply-adds in the same order
// as the chain over the merged centroid (compute_impl.cu:80-101).  Key =
// (order key, ~g) of an occupied cell, 0 for an empty one (masked,
// retrieval.py:357); one score range per workgroup.  ONLINE: a cell whose
// merged centroid was replaced (async_update.py:7-19) is scored over its
// shadow row with the full 128-term chain.
template <bool ONLINE>
__global__ __launch_bounds__(kScoreThreads) void sel2_dense_score_kernel(Sel4 a) {
    __shared__ __attribute__((aligned(16))) float qs[128];
    __shared__ float p1[kScoreThreads + 2];
    __shared__ int lh[kLocBins];   // the candidate cut's buckets
    const int h = blockIdx.y, tid = threadIdx.x;
    const int k1 = a.k[1];
    const int ncells = a.cap;
    const int g0 = blockIdx.x * kDenseScoreCells;
    const int g = g0 + tid;
    const bool in = g < ncells;
    const int gl = min(g0 + kDenseScoreCells, ncells) - 1;
    const int r0 = g0 < ncells ? g0 / k1 : 0;
    const int nr = g0 < ncells ? gl / k1 - r0 + 1 : 0;
    // ---- loads, all issued before the first wait ----
    uint16_t qv[kMaxG4];
    if (tid < 128) {
        // rows past G re-read row G - 1 and are dropped from the sum
        const uint16_t* qh = a.q + static_cast<int64_t>(h) * a.G * 128;
        load_group_rows(qh, a.G, tid, qv);
    }
    const int l0 = in ? g / k1 : 0, l1 = in ? g - (g / k1) * k1 : 0;
    const float4* c0 = reinterpret_cast<const float4*>(a.cent + (static_cast<int64_t>(h) * 2 + 0) * a.kmax * 64);
    const float4* c1 = reinterpret_cast<const float4*>(a.cent + (static_cast<int64_t>(h) * 2 + 1) * a.kmax * 64);
    float4 r0v[16], r1v[16];
    const int myrow = tid < nr ? r0 + tid : 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        r0v[i] = tid < nr ? c0[myrow * 16 + i] : make_float4(0, 0, 0, 0);
        r1v[i] = c1[l1 * 16 + i];
    }
    const int cnt = in ? a.csize[static_cast<int64_t>(h) * ncells + g] : 0;
    int slot = -1;
    if (ONLINE && a.upd_slot && in) slot = a.upd_slot[static_cast<int64_t>(h) * ncells + g];
    if (tid < 128) {
        float acc = 0.0f;   // grouped-query sum, g ascending (compute_impl.cu:80-87)
#pragma unroll
        for (int j = 0; j < kMaxG4; ++j)
            if (j < a.G) acc += bf16_to_f32(qv[j]);
        qs[tid] = acc;
    }
    for (int i = tid; i < kLocBins; i += kScoreThreads) lh[i] = 0;
    __syncthreads();
    if (tid < nr) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 qq = *reinterpret_cast<const float4*>(qs + 4 * i);
            acc = __builtin_fmaf(qq.x, r0v[i].x, acc);
            acc = __builtin_fmaf(qq.y, r0v[i].y, acc);
            acc = __builtin_fmaf(qq.z, r0v[i].z, acc);
            acc = __builtin_fmaf(qq.w, r0v[i].w, acc);
        }
        p1[tid] = acc;
    }
    __syncthreads();
    float sc = p1[l0 - r0 >= 0 && l0 - r0 < nr ? l0 - r0 : 0];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 qq = *reinterpret_cast<const float4*>(qs + 64 + 4 * i);
        sc = __builtin_fmaf(qq.x, r1v[i].x, sc);
        sc = __builtin_fmaf(qq.y, r1v[i].y, sc);
        sc = __builtin_fmaf(qq.z, r1v[i].z, sc);
        sc = __builtin_fmaf(qq.w, r1v[i].w, sc);
    }
    if (ONLINE && slot >= 0) {
        const int row = min(max(a.upd_row[static_cast<int64_t>(h) * a.shadow_rows + min(slot, a.shadow_rows - 1)], 0),
                            a.shadow_rows - 1);
        const float4* sr = reinterpret_cast<const float4*>(a.shadow + (static_cast<int64_t>(h) * a.shadow_rows + row) * 128);
        float acc = 0.0f;
        for (int i = 0; i < 32; ++i) {
            const float4 v = sr[i];
            const float4 qq = *reinterpret_cast<const float4*>(qs + 4 * i);
            acc = __builtin_fmaf(qq.x, v.x, acc);
            acc = __builtin_fmaf(qq.y, v.y, acc);
            acc = __builtin_fmaf(qq.z, v.z, acc);
            acc = __builtin_fmaf(qq.w, v.w, acc);
        }
        sc = acc;
    }
    const uint64_t kv[1] = {in && cnt > 0 ? (static_cast<uint64_t>(order_key(sc)) << 32) |
                                                (0xFFFFFFFFu - static_cast<uint32_t>(g))
                                          : 0ull};
    const int ci[1] = {g};
    emit_candidates<kScoreThreads, 1>(a, h, kprime(a, h, ncells), kv, ci, lh);
}

// IVF (one 128-dim space): one cluster per thread, the 128-term chain of
// compute_impl.cu:80-101 over its centroid, keys as in
// sel2_dense_score_kernel (0 for an empty cluster).  ONLINE: a cluster
// whose centroid was replaced is scored over its shadow row instead.
template <bool ONLINE>
__global__ __launch_bounds__(kScoreThreads) void sel1_score_kernel(Sel4 a) {
    __shared__ __attribute__((aligned(16))) float qs[128];
    __shared__ int lh[kLocBins];   // the candidate cut's buckets
    const int h = blockIdx.y, tid = threadIdx.x;
    const int ncells = a.cap;
    const int g = blockIdx.x * kDenseScoreCells + tid;
    const bool in = g < ncells;
    // ---- loads, all issued before the first wait ----
    uint16_t qv[kMaxG4];
    if (tid < 128) {
        // rows past G re-read row G - 1 and are dropped from the sum
        const uint16_t* qh = a.q + static_cast<int64_t>(h) * a.G * 128;
        load_group_rows(qh, a.G, tid, qv);
    }
    int slot = -1;
    if (ONLINE && a.upd_slot && in) slot = a.upd_slot[static_cast<int64_t>(h) * ncells + g];
    const float4* cr =
        reinterpret_cast<const float4*>(a.cent + (static_cast<int64_t>(h) * a.kmax + (in ? g : 0)) * 128);
    if (ONLINE && slot >= 0) {
        const int row = min(max(a.upd_row[static_cast<int64_t>(h) * a.shadow_rows + min(slot, a.shadow_rows - 1)], 0),
                            a.shadow_rows - 1);
        cr = reinterpret_cast<const float4*>(a.shadow + (static_cast<int64_t>(h) * a.shadow_rows + row) * 128);
    }
    float4 r[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) r[i] = cr[i];
    const int cnt = in ? a.csize[static_cast<int64_t>(h) * ncells + g] : 0;
    if (tid < 128) {
        float acc = 0.0f;   // grouped-query sum, g ascending (compute_impl.cu:80-87)
#pragma unroll
        for (int j = 0; j < kMaxG4; ++j)
            if (j < a.G) acc += bf16_to_f32(qv[j]);
        qs[tid] = acc;
    }
    for (int i = tid; i < kLocBins; i += kScoreThreads) lh[i] = 0;
    __syncthreads();
    float sc = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const float4 qq = *reinterpret_cast<const float4*>(qs + 4 * i);
        sc = __builtin_fmaf(qq.x, r[i].x, sc);
        sc = __builtin_fmaf(qq.y, r[i].y, sc);
        sc = __builtin_fmaf(qq.z, r[i].z, sc);
        sc = __builtin_fmaf(qq.w, r[i].w, sc);
    }
    const uint64_t kv[1] = {in && cnt > 0 ? (static_cast<uint64_t>(order_key(sc)) << 32) |
                                                (0xFFFFFFFFu - static_cast<uint32_t>(g))
                                          : 0ull};
    const int ci[1] = {g};
    emit_candidates<kScoreThreads, 1>(a, h, kprime(a, h, ncells), kv, ci, lh);
}

__device__ __forceinline__ void block_scan2(int& x, int& y, int* sh, int& tx, int& ty) {
    const int ix = wave_incl_scan(x), iy = wave_incl_scan(y);
    const int w = threadIdx.x >> 6;
    if (lane_id() == 63) {
        sh[w] = ix;
        sh[16 + w] = iy;
    }
    __syncthreads();
    int bx = 0, by = 0;
    tx = 0;
    ty = 0;
    for (int j = 0; j < kFinalThreads / 64; ++j) {
        if (j < w) {
            bx += sh[j];
            by += sh[16 + j];
        }
        tx += sh[j];
        ty += sh[16 + j];
    }
    x = bx + ix;
    y = by + iy;
    __syncthreads();
}

// Bitonic sort, descending, of the first N entries of sk / si (N a power of
// two).  N <= kFinalThreads: one entry per thread, held in registers; the
// compare-exchange stages whose partner lies in the same wave (distance < 64)
// run on lane shuffles, only the longer ones go through LDS (two barriers
// each: 10 of the 55 stages at N = 1024).  Larger N: every stage in LDS.
__device__ void bitonic_desc(uint64_t* sk, int* si, int N) {
    const int tid = threadIdx.x;
    if (N <= kFinalThreads) {
        uint64_t x = tid < N ? sk[tid] : 0ull;
        int xi = tid < N ? si[tid] : -1;
        for (int kk = 2; kk <= N; kk <<= 1) {
            for (int j = kk >> 1; j > 0; j >>= 1) {
                uint64_t y;
                int yi;
                if (j >= 64) {
                    __syncthreads();
                    if (tid < N) {
                        sk[tid] = x;
                        si[tid] = xi;
                    }
                    __syncthreads();
                    const int p = tid ^ j;
                    y = p < N ? sk[p] : 0ull;
                    yi = p < N ? si[p] : -1;
                } else {
                    const uint32_t lo = static_cast<uint32_t>(__shfl_xor(static_cast<int>(x & 0xFFFFFFFFull), j));
                    const uint32_t hi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(x >> 32), j));
                    y = (static_cast<uint64_t>(hi) << 32) | lo;
                    yi = __shfl_xor(xi, j);
                }
                const bool desc = (tid & kk) == 0;
                const bool lower = (tid & j) == 0;
                if (lower == desc ? y > x : y < x) {   // the lower slot keeps the larger key when descending
                    x = y;
                    xi = yi;
                }
            }
        }
        __syncthreads();
        if (tid < N) {
            sk[tid] = x;
            si[tid] = xi;
        }
        __syncthreads();
        return;
    }
    for (int kk = 2; kk <= N; kk <<= 1) {
        for (int j = kk >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < N; i += kFinalThreads) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const bool desc = (i & kk) == 0;
                    const uint64_t x = sk[i], y = sk[ixj];
                    if ((x < y) == desc) {
                        sk[i] = y;
                        sk[ixj] = x;
                        const int t = si[i];
                        si[i] = si[ixj];
                        si[ixj] = t;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// Ring-code set of the delta match: open addressing over kRingSet slots
// (at most kFinalThreads codes, so at most half full); returns the slot.
__device__ __forceinline__ int ring_slot(int code) {
    return static_cast<int>((static_cast<uint32_t>(code) * 2654435761u) >> (32 - 11)) & (kRingSet - 1);
}
__device__ int ring_insert(int* t, int code) {
    int i = ring_slot(code);
    while (true) {
        const int prev = atomicCAS(&t[i], -1, code);
        if (prev == -1 || prev == code) return i;
        i = (i + 1) & (kRingSet - 1);
    }
}
__device__ int ring_find(const int* t, int code) {
    int i = ring_slot(code);
    while (true) {
        const int v = t[i];
        if (v == code) return i;
        if (v == -1) return -1;
        i = (i + 1) & (kRingSet - 1);
    }
}

constexpr int kRPT = kCand4 / kFinalThreads;   // ranks per thread of the budget rules

// Final LDS: candidate keys and cell indices (slot order), the slot of each
// rank, the bucket bases.
constexpr size_t kFinalLds = static_cast<size_t>(kCand4) * (8 + 4 + 4) + (kBins4 + 1) * 4;

// One workgroup per head: the candidates in rank order (within each bucket by
// counting the better keys of the same bucket; a bitonic sort when a bucket
// holds more than kSegMax; an exact radix select of the K'-th key when the
// candidates did not fit), then the token and page budgets in rank order and
// the outputs, then the delta match.
template <bool ONLINE>
__global__ __launch_bounds__(kFinalThreads) void sel4_final_kernel(Sel4 a) {
    extern __shared__ __attribute__((aligned(16))) uint64_t f_lds[];
    uint64_t* sk = f_lds;                                  // [kCand4]
    int* si = reinterpret_cast<int*>(sk + kCand4);        // [kCand4]
    int* ord = si + kCand4;                                // [kCand4] slot of rank r
    int* binbase = ord + kCand4;                           // [kBins4 + 1]
    __shared__ int sh[48];
    __shared__ int shk[kFinalThreads / 64];
    __shared__ int s_rows;
    __shared__ uint32_t h256[256];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int na = n_active(a, h);
    const int kp = kprime(a, h, na);
    int32_t* prefix_out = a.sel_prefix + static_cast<int64_t>(h) * (a.sel_cap + 1);
    // The head's candidates: score workgroup b listed wcnt[b] of them from
    // b * region on.  The counts and the range partials come in one round
    // trip; flat candidate i lies in the last segment whose start is <= i
    // (a binary search over the starts in LDS).  The first kFinalThreads *
    // kFinalCPT candidates are held in registers, the rest streamed in
    // batches.
    __shared__ int seg0[kMaxSeg + 1];
    const int64_t hb = static_cast<int64_t>(h) * a.nbs;
    int cw = tid < a.nbs ? min(max(a.wcnt[hb + tid], 0), a.region) : 0;
    uint32_t m1 = 0, m2 = 0;
    if (tid < a.nbs) {
        m1 = a.rpart[(hb + tid) * 2 + 0];
        m2 = a.rpart[(hb + tid) * 2 + 1];
    }
    // A score workgroup that listed at least kp candidates holds kp cells at
    // or above its lowest candidate, so the head's kp-th best key is at or
    // above the highest such lowest score, lb (order-key bits): a candidate
    // below lb cannot rank, and a workgroup whose best cell is below lb is
    // skipped whole.  The range of the candidates left starts at lb.
    uint32_t lb = (kp > 0 && cw >= kp) ? ~m2 : 0u;
    lb = wave_max_u32(lb);
    if (lane_id() == 0) shk[tid >> 6] = static_cast<int>(lb);
    __syncthreads();
    lb = 0u;
#pragma unroll
    for (int w = 0; w < kFinalThreads / 64; ++w) lb = max(lb, static_cast<uint32_t>(shk[w]));
    if (m1 < lb) {
        cw = 0;
        m1 = 0u;
        m2 = 0u;
    } else {
        m2 = min(m2, ~lb);
    }
    {
        const int incl = wave_incl_scan(cw);
        if (lane_id() == 63) sh[tid >> 6] = incl;
        __syncthreads();
        int before = incl - cw, tot = 0;
        for (int j = 0; j < kFinalThreads / 64; ++j) {
            before += j < (tid >> 6) ? sh[j] : 0;
            tot += sh[j];
        }
        seg0[tid] = before;
        if (tid == 0) seg0[kMaxSeg] = tot;
        __syncthreads();
    }
    const int n1 = seg0[kMaxSeg];
    // list position of candidate i < n1: the last segment start <= i, by a
    // binary search over the nbs starts (log2 nbs dependent LDS reads; the
    // starts past the last score workgroup all equal n1 > i, so the search
    // needs no bound test)
    const int top = a.nbs <= 1 ? 1 : 1 << (32 - __builtin_clz(a.nbs - 1));   // power of two >= nbs
    auto cand_at = [&](int i) {
        int lo = 0;
        for (int step = top >> 1; step > 0; step >>= 1) {
            const int mid = lo + step;
            lo = seg0[mid] <= i ? mid : lo;
        }
        return cand_pos(hb + lo, i - seg0[lo], a.region);
    };
    const uint64_t* candl = a.cand;
    const int32_t* cidxl = a.cidx;
    uint64_t ck[kFinalCPT];
    int cc[kFinalCPT];
#pragma unroll
    for (int u = 0; u < kFinalCPT; ++u) {
        const int i = tid + u * kFinalThreads;
        ck[u] = 0ull;
        cc[u] = 0;
        if (i < n1) {
            const int64_t at = cand_at(i);
            ck[u] = candl[at];
            cc[u] = cidxl[at];
        }
    }
#pragma unroll
    for (int u = 0; u < kFinalCPT; ++u)
        if (static_cast<uint32_t>(ck[u] >> 32) < lb) ck[u] = 0ull;
    m1 = wave_max_u32(m1);
    m2 = wave_max_u32(m2);
    int* hist = ord;             // [kBins4] bucket counts
    int* cur = ord + kBins4;     // [kBins4] gather cursors
    if (lane_id() == 0) {
        h256[2 * (tid >> 6)] = m1;
        h256[2 * (tid >> 6) + 1] = m2;
    }
    for (int i = tid; i < kBins4; i += kFinalThreads) {
        hist[i] = 0;
        cur[i] = 0;
    }
    __syncthreads();
    uint32_t r1 = 0, r2 = 0;
#pragma unroll
    for (int w = 0; w < kFinalThreads / 64; ++w) {
        r1 = max(r1, h256[2 * w]);
        r2 = max(r2, h256[2 * w + 1]);
    }
    const float gmax = key_score(static_cast<uint64_t>(r1) << 32);
    const float gmin = key_score(static_cast<uint64_t>(~r2) << 32);
    const float range = gmax - gmin;
    const float inv = range > 0.0f ? static_cast<float>(kBins4) / range : 0.0f;
    constexpr int kHeld = kFinalThreads * kFinalCPT;
    constexpr int kBatch = 8;
    // candidates past the held ones, kBatch loads per thread in flight
    auto stream_rest = [&](auto fn) {
        for (int base = kHeld; base < n1; base += kFinalThreads * kBatch) {
            uint64_t bk[kBatch];
            int bc[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int i = base + tid + u * kFinalThreads;
                bk[u] = 0ull;
                bc[u] = 0;
                if (i < n1) {
                    const int64_t at = cand_at(i);
                    bk[u] = candl[at];
                    bc[u] = cidxl[at];
                }
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (bk[u] != 0ull && static_cast<uint32_t>(bk[u] >> 32) >= lb) fn(bk[u], bc[u]);
        }
    };
    // histogram of the candidates over kBins4 linear buckets of their range
#pragma unroll
    for (int u = 0; u < kFinalCPT; ++u)
        if (ck[u] != 0ull) atomicAdd(&hist[bucket4(key_score(ck[u]), gmax, inv)], 1);
    stream_rest([&](uint64_t key, int) { atomicAdd(&hist[bucket4(key_score(key), gmax, inv)], 1); });
    __syncthreads();
    // bucket bK holding the kp-th best candidate (the last one when fewer),
    // and the first slot of every bucket
    int bK = kBins4 - 1;
    {
        constexpr int PER = kBins4 / kFinalThreads;
        int v[PER], loc = 0;
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            v[u] = hist[tid * PER + u];
            loc += v[u];
        }
        const int incl = wave_incl_scan(loc);
        const int w = tid >> 6;
        if (lane_id() == 63) sh[w] = incl;
        if (tid == 0) sh[32] = kBins4 - 1;
        __syncthreads();
        int run = incl - loc;
        for (int j = 0; j < w; ++j) run += sh[j];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            binbase[tid * PER + u] = run;
            if (run < kp && run + v[u] >= kp) sh[32] = tid * PER + u;
            run += v[u];
        }
        if (tid == kFinalThreads - 1) binbase[kBins4] = run;
        __syncthreads();
        bK = sh[32];
    }
    const int n_c = binbase[bK + 1];
    int n = 0;   // ranked candidates; ord[r] = slot of rank r
    if (kp > 0 && n_c <= kCand4) {
        n = n_c;
        // the candidates at or above bK into LDS, grouped by bucket
        auto place = [&](uint64_t key, int c) {
            const int b = bucket4(key_score(key), gmax, inv);
            if (b <= bK) {
                const int slot = binbase[b] + atomicAdd(&cur[b], 1);
                if (slot < kCand4) {   // only if the histogram disagreed with the keys
                    sk[slot] = key;
                    si[slot] = c;
                }
            }
        };
#pragma unroll
        for (int u = 0; u < kFinalCPT; ++u)
            if (ck[u] != 0ull) place(ck[u], cc[u]);
        stream_rest(place);
        int seg = 0;   // largest bucket among the candidates
        for (int b = tid; b <= bK; b += kFinalThreads) seg = max(seg, binbase[b + 1] - binbase[b]);
        seg = wave_max_i(seg);
        if (lane_id() == 0) shk[tid >> 6] = seg;
        __syncthreads();
        seg = 0;
        for (int w = 0; w < kFinalThreads / 64; ++w) seg = max(seg, shk[w]);
        if (seg <= kSegMax) {
            // rank of each candidate: its bucket's first slot plus the better
            // keys of its bucket (keys are unique)
            for (int i = tid; i < n; i += kFinalThreads) {
                const uint64_t key = sk[i];
                const int b = bucket4(key_score(key), gmax, inv);
                const int s0 = binbase[b], s1 = binbase[b + 1];
                int better = 0;
                for (int j = s0; j < s1; ++j) better += sk[j] > key ? 1 : 0;
                ord[min(s0 + better, kCand4 - 1)] = i;
            }
            __syncthreads();
        } else {
            int N = 1;
            while (N < n) N <<= 1;
            for (int i = n + tid; i < N; i += kFinalThreads) {
                sk[i] = 0ull;
                si[i] = -1;
            }
            __syncthreads();
            bitonic_desc(sk, si, N);
            for (int i = tid; i < n; i += kFinalThreads) ord[i] = i;
            __syncthreads();
        }
    } else if (kp > 0) {
        // Exact radix select of the kp-th largest candidate key (keys are
        // unique), then every key at or above it, sorted.
        uint64_t prefix = 0, mask = 0;
        int remaining = kp;
        for (int pass = 0; pass < 8; ++pass) {
            const int shift = 8 * (7 - pass);
            for (int i = tid; i < 256; i += kFinalThreads) h256[i] = 0;
            __syncthreads();
            for (int c = tid; c < n1; c += kFinalThreads) {
                const uint64_t key = candl[cand_at(c)];
                if (key != 0ull && (key & mask) == prefix) atomicAdd(&h256[(key >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (tid == 0) {
                int acc = 0;
                for (int d = 255; d >= 0; --d) {
                    const int hv = static_cast<int>(h256[d]);
                    if (acc + hv >= remaining) {
                        sh[40] = d;
                        sh[41] = remaining - acc;
                        break;
                    }
                    acc += hv;
                }
            }
            __syncthreads();
            prefix |= static_cast<uint64_t>(sh[40]) << shift;
            mask |= 255ull << shift;
            remaining = sh[41];
            __syncthreads();
        }
        if (tid == 0) sh[42] = 0;
        __syncthreads();
        for (int c = tid; c < n1; c += kFinalThreads) {
            const int64_t at = cand_at(c);
            const uint64_t key = candl[at];
            if (key != 0ull && key >= prefix) {
                const int slot = atomicAdd(&sh[42], 1);
                if (slot < kCand4) {   // exactly kp keys (keys are unique)
                    sk[slot] = key;
                    si[slot] = cidxl[at];
                }
            }
        }
        __syncthreads();
        n = min(sh[42], kCand4);   // == kp
        int N = 1;
        while (N < n) N <<= 1;
        for (int i = n + tid; i < N; i += kFinalThreads) {
            sk[i] = 0ull;
            si[i] = -1;
        }
        __syncthreads();
        bitonic_desc(sk, si, N);
        for (int i = tid; i < n; i += kFinalThreads) ord[i] = i;
        __syncthreads();
    }

    // budget rules in rank order over the best kp cells: ranks kRPT*tid + u
    const int C = n < kp ? n : kp;
    int s2[kRPT], pg2[kRPT], o2[kRPT];
    uint32_t g2[kRPT];
    int tsum = 0, psum = 0;
    if (C > 0) {
        // size and CSR offset of every rank in one round trip: branch-free
        // (ranks past C re-read rank C - 1 and are masked), so the kRPT
        // LDS lookups and loads overlap instead of running one by one
        int cr[kRPT];
#pragma unroll
        for (int u = 0; u < kRPT; ++u) {
            const int slot = min(max(ord[min(kRPT * tid + u, C - 1)], 0), kCand4 - 1);
            cr[u] = min(max(si[slot], 0), a.cap - 1);
            g2[u] = 0xFFFFFFFFu - static_cast<uint32_t>(sk[slot] & 0xFFFFFFFFull);
        }
#pragma unroll
        for (int u = 0; u < kRPT; ++u) {
            s2[u] = a.csize[static_cast<int64_t>(h) * a.cap + cr[u]];
            o2[u] = a.coff[static_cast<int64_t>(h) * (a.cap + 1) + cr[u]];
        }
#pragma unroll
        for (int u = 0; u < kRPT; ++u) {
            const bool in = kRPT * tid + u < C;
            s2[u] = in ? s2[u] : 0;
            o2[u] = in ? o2[u] : 0;
            g2[u] = in ? g2[u] : 0u;
        }
    } else {
#pragma unroll
        for (int u = 0; u < kRPT; ++u) {
            s2[u] = 0;
            o2[u] = 0;
            g2[u] = 0u;
        }
    }
#pragma unroll
    for (int u = 0; u < kRPT; ++u) {
        // pages = ceil(size / page_size); a power-of-two page size takes a shift
        pg2[u] = (a.page_size & (a.page_size - 1)) == 0 ? (s2[u] + a.page_size - 1) >> (__builtin_ctz(a.page_size))
                                                        : (s2[u] + a.page_size - 1) / a.page_size;
        if (a.tile_mode) pg2[u] = pg2[u] > head_pages(a, h) ? 1 : 0;   // cells that alone overflow
        tsum += s2[u];
        psum += pg2[u];
    }
    int ttot, ptot;
    int tincl = tsum, pincl = psum;
    block_scan2(tincl, pincl, sh, ttot, ptot);
    int texcl = tincl - tsum, pexcl = pincl - psum;
    int kept = 0, kept_tok = 0;
    int excl_tok[kRPT];
#pragma unroll
    for (int u = 0; u < kRPT; ++u) {
        const int r = kRPT * tid + u;
        excl_tok[u] = texcl;
        pexcl += pg2[u];
        const bool keep_tok = r < C && r < a.nprobe && texcl < head_tokens(a, h);
        const bool keep = keep_tok && pexcl <= (a.tile_mode ? 0 : head_pages(a, h));
        kept += keep ? 1 : 0;
        kept_tok += keep_tok ? 1 : 0;
        texcl += s2[u];
    }
    // the rules are monotone in rank, so the kept ranks are the first m (the
    // first m_tok before the page cut)
    {
        const int wk = wave_sum_i(kept);
        const int wt = ONLINE ? wave_sum_i(kept_tok) : 0;
        if (lane_id() == 0) {
            sh[32 + (tid >> 6)] = wk;
            if (ONLINE) shk[tid >> 6] = wt;
        }
    }
    __syncthreads();
    int m = 0, m_tok = 0;
    for (int w = 0; w < kFinalThreads / 64; ++w) {
        m += sh[32 + w];
        if (ONLINE) m_tok += shk[w];
    }
    int32_t* out_cell = a.sel_cell + static_cast<int64_t>(h) * a.sel_cap;
    int32_t* out_off = a.sel_offset + static_cast<int64_t>(h) * a.sel_cap;
    int32_t* out_cnt = a.sel_count + static_cast<int64_t>(h) * a.sel_cap;
#pragma unroll
    for (int u = 0; u < kRPT; ++u) {
        const int r = kRPT * tid + u;
        if (r < m) {
            out_cell[r] = static_cast<int32_t>(g2[u]);
            out_off[r] = o2[u];
            out_cnt[r] = s2[u];
            prefix_out[r] = excl_tok[u];
        }
        if (r == m - 1) {
            const int total = excl_tok[u] + s2[u];
            prefix_out[m] = total;
            a.n_sel[h] = m;
            a.n_rows[h] = total;
            if (ONLINE) s_rows = total;
        }
    }
    if (m == 0 && tid == 0) {
        a.n_sel[h] = 0;
        a.n_rows[h] = 0;
        prefix_out[0] = 0;
    }
    if (ONLINE && a.ring_cap > 0) {
        // Delta append (async_update.py:20-76): the ring entries whose cell
        // is one of the m_tok cells that pass nprobe and the token budget,
        // or the padding id when m_tok < nprobe, up to the execution-buffer
        // rows left.  The ring's cell codes go to a set; every kept-token
        // cell marks its code's slot.
        int* rtab = ord;
        int* rhit = ord + kRingSet;
        __syncthreads();   // ord fully read above
        const int rows_sel = m > 0 ? s_rows : 0;
        for (int i = tid; i < kRingSet; i += kFinalThreads) {
            rtab[i] = -1;
            rhit[i] = 0;
        }
        __syncthreads();
        const int nvalid = min(a.ring_n[h], a.ring_cap);
        int code = -3, rrow = 0, rs = -1;
        if (tid < nvalid) {
            code = a.ring_cell[static_cast<int64_t>(h) * a.ring_cap + tid];
            rrow = a.ring_row[static_cast<int64_t>(h) * a.ring_cap + tid];
            if (code >= 0) rs = ring_insert(rtab, code);
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kRPT; ++u) {
            const int r = kRPT * tid + u;
            if (r < m_tok) {
                const int f = ring_find(rtab, static_cast<int>(g2[u]));
                if (f >= 0) rhit[f] = 1;
            }
        }
        __syncthreads();
        const bool match = code >= 0 ? rhit[rs] != 0 : (code == -1 && m_tok < a.nprobe);
        int f = match ? 1 : 0, z = 0, tot, ztot;
        block_scan2(f, z, sh, tot, ztot);
        const int pos = f - (match ? 1 : 0);
        const int nd = min(tot, max(a.exec_rows - rows_sel, 0));
        if (match && pos < nd) a.delta_rows[static_cast<int64_t>(h) * a.ring_cap + pos] = rrow;
        if (tid == 0) a.n_delta[h] = nd;
    }
}

size_t sel4_workspace(const imi_select_args* a, Sel4* p) {
    Carver cv(a->workspace);
    const size_t H = a->kv_heads;
    const bool dense = a->parts <= 2;
    const int cap = a->parts == 1 ? a->k[0] : (dense ? a->k[0] * a->k[1] : a->compact_cap);
    const int region = dense ? kDenseScoreCells : kCellsPerBlock;
    const int nbs = (cap + region - 1) / region;
    // every score workgroup writes its count and range each call, and the
    // final kernel reads only those: nothing has to start at zero
    int32_t* wcnt = cv.take<int32_t>(H * static_cast<size_t>(nbs));
    uint32_t* rpart = cv.take<uint32_t>(H * static_cast<size_t>(nbs) * 2);
    uint64_t* cand = cv.take<uint64_t>(H * static_cast<size_t>(nbs) * region);
    int32_t* cidx = cv.take<int32_t>(H * static_cast<size_t>(nbs) * region);
    const size_t tb = tile_delta_bytes(a);
    char* tscr = tb > 0 ? cv.take<char>(tb) : nullptr;
    if (p) {
        p->tile_scr = tscr;
        p->wcnt = wcnt;
        p->region = region;
        p->rpart = rpart;
        p->nbs = nbs;
        p->cap = cap;
        p->dense = dense ? 1 : 0;
        p->cand = cand;
        p->cidx = cidx;
    }
    return cv.used();
}

}  // namespace

// The ranking pipeline: 4-way over the occupied cells, or (parts = 2) a 2-way
// IMI over every global cell beyond the one-kernel selection's bounds, or
// (parts = 1) the IVF clusters.
int select4_validate(const imi_select_args* a) {
    const bool dense = a->parts == 1 || a->parts == 2;
    IMI_REQUIRE(a->dim == 128 && (a->parts == 4 || dense), IMI_ERR_UNSUPPORTED,
                "imi_select: the ranking pipeline needs D=128 and parts 1, 2 or 4");
    IMI_REQUIRE(a->kv_heads <= kExtHeads, IMI_ERR_UNSUPPORTED, "imi_select: at most %d KV heads per call", kExtHeads);
    IMI_REQUIRE(a->groups >= 1 && a->groups <= kMaxG4, IMI_ERR_UNSUPPORTED,
                "imi_select: %d query heads per kv head exceed %d", a->groups, kMaxG4);
    int64_t cells_max;
    if (a->parts == 1) {
        IMI_REQUIRE(a->k[0] >= 1 && a->k[0] <= kIvfMaxK, IMI_ERR_UNSUPPORTED, "imi_select: IVF k=%d outside [1,%d]",
                    a->k[0], kIvfMaxK);
        cells_max = a->k[0];
    } else if (dense) {
        for (int p = 0; p < 2; ++p)
            IMI_REQUIRE(a->k[p] >= 1 && a->k[p] <= kDenseK, IMI_ERR_UNSUPPORTED,
                        "imi_select: 2-way k[%d]=%d outside [1,%d]", p, a->k[p], kDenseK);
        cells_max = static_cast<int64_t>(a->k[0]) * a->k[1];
    } else {
        for (int p = 0; p < 4; ++p)
            IMI_REQUIRE(a->k[p] >= 1 && a->k[p] <= kK4, IMI_ERR_UNSUPPORTED,
                        "imi_select: 4-way k[%d]=%d outside [1,%d]", p, a->k[p], kK4);
        IMI_REQUIRE(a->compact_gid && a->compact_size && a->compact_offset && a->n_active && a->compact_cap > 0,
                    IMI_ERR_INVALID, "imi_select: 4-way selection needs the compact cell arrays");
        cells_max = a->compact_cap;
    }
    IMI_REQUIRE((cells_max + (dense ? kDenseScoreCells : kCellsPerBlock) - 1) / (dense ? kDenseScoreCells : kCellsPerBlock) <=
                    kMaxSeg,
                IMI_ERR_UNSUPPORTED, "imi_select: %lld cells per head exceed the ranking pipeline's %d score workgroups",
                static_cast<long long>(cells_max), kMaxSeg);
    const bool rank_all = a->tile_mode || a->ring_cap > 0;
    const int kprime_max = rank_all ? a->nprobe : (a->nprobe < a->buffer_pages ? a->nprobe : a->buffer_pages);
    const int64_t kp_eff = kprime_max < cells_max ? kprime_max : cells_max;
    IMI_REQUIRE(kp_eff <= kSelCap4, IMI_ERR_UNSUPPORTED, "imi_select: %lld cells to rank exceed %d",
                static_cast<long long>(kp_eff), kSelCap4);
    IMI_REQUIRE(a->sel_cap >= kprime_max, IMI_ERR_INVALID, "imi_select: sel_cap %d < %d (%s)", a->sel_cap,
                kprime_max, rank_all ? "nprobe" : "min(nprobe, buffer_pages)");
    return IMI_OK;
}

// Bytes at the start of the workspace that a call expects zero: none (each
// call's score kernel writes every count and range its final kernel reads).
size_t select4_zero_bytes() { return 0; }

size_t select4_workspace_size(const imi_select_args* a) {
    imi_select_args t = *a;
    t.workspace = nullptr;
    return sel4_workspace(&t, nullptr);
}

int select4_launch(const imi_select_args* a, hipStream_t stream) {
    int rc = select4_validate(a);
    if (rc) return rc;
    IMI_REQUIRE(a->workspace && a->workspace_bytes >= select4_workspace_size(a), IMI_ERR_WORKSPACE,
                "imi_select: workspace %zu bytes < %zu required", a->workspace_bytes, select4_workspace_size(a));
    Sel4 p{};
    sel4_workspace(a, &p);
    p.q = a->query;
    p.cent = a->centroids;
    p.H = a->kv_heads;
    p.G = a->groups;
    p.kmax = 0;
    for (int i = 0; i < a->parts; ++i) {
        p.k[i] = a->k[i];
        p.kmax = a->k[i] > p.kmax ? a->k[i] : p.kmax;
    }
    const bool dense = p.dense != 0;
    p.gid = dense ? nullptr : a->compact_gid;
    p.csize = dense ? a->cell_count : a->compact_size;
    p.coff = dense ? a->cell_offset : a->compact_offset;
    p.nact = dense ? nullptr : a->n_active;
    p.nprobe = a->nprobe;
    p.max_tokens = a->max_tokens;
    p.buffer_pages = a->buffer_pages;
    p.page_size = a->page_size;
    p.head_max_tokens = a->head_max_tokens;
    p.head_buffer_pages = a->head_buffer_pages;
    p.tile_mode = a->tile_mode != 0;
    p.sel_cell = a->sel_cell;
    p.sel_offset = a->sel_offset;
    p.sel_count = a->sel_count;
    p.sel_prefix = a->sel_prefix;
    p.n_sel = a->n_selected;
    p.n_rows = a->n_rows;
    p.sel_cap = a->sel_cap;
    p.shadow = a->shadow;
    p.shadow_rows = a->shadow_rows;
    p.upd_slot = a->upd_slot;
    p.upd_row = a->upd_row;
    p.ring_cell = a->ring_cell;
    p.ring_row = a->ring_row;
    p.ring_n = a->ring_n;
    p.ring_cap = a->ring_cap;
    p.exec_rows = a->exec_rows;
    p.delta_rows = a->delta_rows;
    p.n_delta = a->n_delta;
    const bool tile_delta = a->tile_mode && a->ring_cap > 0;
    if (tile_delta) p.ring_cap = 0;   // the tile launches append the delta
    const bool online = p.upd_slot || p.ring_cap > 0;
    if (a->parts == 1) {
        if (p.upd_slot)
            hipLaunchKernelGGL(sel1_score_kernel<true>, dim3(p.nbs, a->kv_heads), dim3(kScoreThreads), 0, stream, p);
        else
            hipLaunchKernelGGL(sel1_score_kernel<false>, dim3(p.nbs, a->kv_heads), dim3(kScoreThreads), 0, stream, p);
        IMI_LAUNCH_CHECK("sel1_score_kernel");
    } else if (dense) {
        const dim3 grid_s(p.nbs, a->kv_heads);
        if (p.upd_slot)
            hipLaunchKernelGGL((sel2_dense_score_kernel<true>), grid_s, dim3(kScoreThreads), 0, stream, p);
        else
            hipLaunchKernelGGL((sel2_dense_score_kernel<false>), grid_s, dim3(kScoreThreads), 0, stream, p);
        IMI_LAUNCH_CHECK("sel2_dense_score_kernel");
    } else {
        const dim3 grid(p.nbs, a->kv_heads);
        // C0..C3 rows at the padded stride, the chain prefixes per (l0, l1) pair and per triple
        // (+ the screened pass's candidates and per-l3 tables: without the
        // online update and for K' <= 64 per wave)
        const bool rank_all = a->tile_mode || a->ring_cap > 0;
        const int kprime_max = rank_all ? a->nprobe : (a->nprobe < a->buffer_pages ? a->nprobe : a->buffer_pages);
        const bool fast = !online && kprime_max <= kScore4Threads;
        p.fast4 = fast ? 1 : 0;
        const size_t score_lds = (static_cast<size_t>(4) * p.kmax * kCS4 + static_cast<size_t>(a->k[0]) * a->k[1] +
                                  kTripCap) * sizeof(float) +
                                 (fast ? kFastLds : 0);
        bool pow2 = true;
        for (int i = 0; i < 4; ++i) pow2 = pow2 && (a->k[i] & (a->k[i] - 1)) == 0;
        static bool score_attr = false;
        if (!score_attr) {   // over 64 KB of LDS with k = 64 per subspace
            const int lds_max = static_cast<int>((4 * kK4 * kCS4 + kK4 * kK4 + kTripCap) * sizeof(float) + kFastLds);
            const void* fns[6] = {reinterpret_cast<const void*>(&sel4_score_kernel<true, true, false>),
                                  reinterpret_cast<const void*>(&sel4_score_kernel<true, false, false>),
                                  reinterpret_cast<const void*>(&sel4_score_kernel<false, true, false>),
                                  reinterpret_cast<const void*>(&sel4_score_kernel<false, false, false>),
                                  reinterpret_cast<const void*>(&sel4_score_kernel<false, true, true>),
                                  reinterpret_cast<const void*>(&sel4_score_kernel<false, false, true>)};
            for (const void* f : fns)
                IMI_HIP_CHECK(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds_max));
            score_attr = true;
        }
        const dim3 blk(kScore4Threads);
        if (online && pow2)
            hipLaunchKernelGGL((sel4_score_kernel<true, true, false>), grid, blk, score_lds, stream, p);
        else if (online)
            hipLaunchKernelGGL((sel4_score_kernel<true, false, false>), grid, blk, score_lds, stream, p);
        else if (fast && pow2)
            hipLaunchKernelGGL((sel4_score_kernel<false, true, true>), grid, blk, score_lds, stream, p);
        else if (fast)
            hipLaunchKernelGGL((sel4_score_kernel<false, false, true>), grid, blk, score_lds, stream, p);
        else if (pow2)
            hipLaunchKernelGGL((sel4_score_kernel<false, true, false>), grid, blk, score_lds, stream, p);
        else
            hipLaunchKernelGGL((sel4_score_kernel<false, false, false>), grid, blk, score_lds, stream, p);
        IMI_LAUNCH_CHECK("sel4_score_kernel");
    }
    static bool attr_set[2] = {false, false};
    if (!attr_set[online]) {
        IMI_HIP_CHECK(hipFuncSetAttribute(online ? reinterpret_cast<const void*>(&sel4_final_kernel<true>)
                                                 : reinterpret_cast<const void*>(&sel4_final_kernel<false>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kFinalLds)));
        attr_set[online] = true;
    }
    if (online)
        hipLaunchKernelGGL(sel4_final_kernel<true>, dim3(a->kv_heads), dim3(kFinalThreads), kFinalLds, stream, p);
    else
        hipLaunchKernelGGL(sel4_final_kernel<false>, dim3(a->kv_heads), dim3(kFinalThreads), kFinalLds, stream, p);
    IMI_LAUNCH_CHECK("sel4_final_kernel");
    if (tile_delta) return tile_delta_launch(a, p.tile_scr, stream);
    return IMI_OK;
}

}  // namespace imi
