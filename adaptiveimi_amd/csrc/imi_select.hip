// Per-step cell scoring and budget-bounded selection of a 2-way IMI on gfx950.
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
// Everything runs in global-cell space (cell g = l0 * k1 + l1), so that the
// decode step never touches the merged-centroid array: the 128-term chain is
// evaluated as the 64-term chain over C0[l0] continued over C1[l1], which is
// the same sequence of fused multiply-adds.  Two paths:
//   select_kernel      (k0, k1 <= 128, K' <= 2048) one 1024-thread workgroup
//                      per head scores every cell and ranks the candidates in
//                      one pass
//   otherwise          (k <= 256, K' <= 8192) the ranking pipeline of
//                      imi_select4.hip over every global cell: a score
//                      kernel of one cell per thread and many workgroups
//                      per head, a histogram, the candidates, the ranks and
//                      budgets in one workgroup per head.
// An IVF index (parts = 1) always takes the ranking pipeline.
#include "imi_common.hpp"

namespace imi {

namespace {

constexpr int kMaxGroups = 16;  // query heads per KV head
constexpr int kRingCap = 1024; // delta ring entries (4 per thread)

// ---------------------------------------------------------------- one-kernel path
// select_kernel: one 1024-thread workgroup per KV head scores, ranks and
// applies the budgets in one pass while k0, k1 <= 128 and K' <= 2048.
constexpr int kSelThreads = 1024;
constexpr int kBins = 2048;
constexpr int kCap = 2048;     // candidate capacity
constexpr int kOvr = 64;       // replaced centroids scored per pass
constexpr int kKeepWords = 512;  // bitmap of kept global cells (k0 * k1 <= 16384)

// Fields in the order the kernel first needs them: the first 64 bytes hold
// what the prologue's loads depend on (one kernel-argument cache line).
// (2-way IMI at D = 128: two subspaces of 64 dims, centroid rows
// [H][2][max(k0, k1)][64], k0 * k1 global cells).
struct SelParams {
    const uint16_t* q;
    const float* cent;
    const int32_t* cnt;
    const int32_t* off;
    const int32_t* head_max_tokens;    // [H] or null
    const int32_t* head_buffer_pages;  // [H] or null
    int k[2];                          // cells per subspace
    int G;
    int nprobe;
    // -- 64 bytes: budgets, the selection outputs and the online prologue
    int max_tokens, buffer_pages, page_size;
    int tile_mode;
    int sel_cap;
    int ring_cap;
    int exec_rows;
    int H;
    int32_t* sel_prefix;
    int32_t* n_sel;
    int32_t* n_rows;
    const int32_t* upd_slot;
    // -- 128 bytes
    int32_t* sel_cell;
    int32_t* sel_offset;
    int32_t* sel_count;
    // online index maintenance: replaced centroids and the delta ring
    const float* shadow;
    int shadow_rows;
    const int32_t* upd_row;
    const int32_t* upd_n;
    const int32_t* ring_cell;
    const int32_t* ring_row;
    const int32_t* ring_n;
    int32_t* delta_rows;
    int32_t* n_delta;
};
static_assert(offsetof(SelParams, max_tokens) == 64 && offsetof(SelParams, sel_cell) == 128,
              "prologue fields in the first 64 bytes, budgets and outputs in the next 64");

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

// Two block-wide inclusive scans at once (same three barriers as one).
__device__ __forceinline__ void block_incl_scan2(int& a, int& b, int* sh, int& ta, int& tb) {
    const int ia = wave_incl_scan(a), ib = wave_incl_scan(b);
    const int wave = threadIdx.x >> 6;
    if (lane_id() == 63) {
        sh[wave] = ia;
        sh[16 + wave] = ib;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int xa = threadIdx.x < 16 ? sh[threadIdx.x] : 0;
        const int xb = threadIdx.x < 16 ? sh[16 + threadIdx.x] : 0;
        const int va = wave_incl_scan(xa), vb = wave_incl_scan(xb);
        if (threadIdx.x < 16) {
            sh[32 + threadIdx.x] = va - xa;
            sh[48 + threadIdx.x] = vb - xb;
        }
        if (threadIdx.x == 15) {
            sh[64] = va;
            sh[65] = vb;
        }
    }
    __syncthreads();
    a = sh[32 + wave] + ia;
    b = sh[48 + wave] + ib;
    ta = sh[64];
    tb = sh[65];
    __syncthreads();
}

__device__ __forceinline__ uint64_t cell_key(uint32_t okey, int g) {
    return (static_cast<uint64_t>(okey) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(g));
}

__device__ __forceinline__ int cell_of_key(uint64_t key) {
    return static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(key & 0xFFFFFFFFull));
}

__device__ __forceinline__ int bucket_of(float s, float gmax, float inv) {
    const float t = (gmax - s) * inv;
    return t < static_cast<float>(kBins - 1) ? static_cast<int>(t) : kBins - 1;
}

// Delta append (async_update.py:20-76, called at retrieval.py:420): the
// ring entries (ring index order, the first rn valid) whose cell is in the
// reference's `selected` -- the m_tok cells that pass nprobe and the token
// budget (retrieval.py:295-303), set in the `keep` bitmap of global cell
// ids, plus the padding id when m_tok < nprobe -- up to the
// execution-buffer rows left after the selected rows.  rcode / rrow: this
// thread's ring entry (thread = ring index).  One barrier, which also
// publishes *rows_sel (written before the call by the thread that knows it).
__device__ void delta_match(const SelParams& a, int h, int m_tok, const int* rows_sel, bool have_rows,
                            const uint32_t* keep, int* wcnt, int rcode, int rrow, int rn) {
    const int tid = threadIdx.x, wave = tid >> 6;
    bool match = false;
    if (tid < rn)
        match = rcode >= 0 ? (rcode < a.k[0] * a.k[1] && ((keep[rcode >> 5] >> (rcode & 31)) & 1u) != 0)
                           : (rcode == -1 && m_tok < a.nprobe);
    const uint64_t bal = __builtin_amdgcn_ballot_w64(match);
    if (lane_id() == 0) wcnt[wave] = __builtin_popcountll(bal);
    __syncthreads();
    int before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kSelThreads / 64; ++w) {
        const int x = wcnt[w];
        tot += x;
        before += w < wave ? x : 0;
    }
    const int pos = before + __builtin_popcountll(bal & lanemask_lt());
    const int rsel = have_rows ? *rows_sel : 0;
    const int nd = min(tot, max(a.exec_rows - rsel, 0));
    if (match && pos < nd) a.delta_rows[static_cast<int64_t>(h) * a.ring_cap + pos] = rrow;
    if (tid == 0) a.n_delta[h] = nd;
}

// DP: subspace width (64 for 2-way IMI at D = 128); EPT: cells per thread;
// ONLINE: replaced centroids and the delta ring (a separate instantiation,
// so the plain kernel carries none of that code).
template <int DP, int EPT, bool ONLINE>
__global__ __launch_bounds__(kSelThreads) void select_kernel(SelParams a) {
    extern __shared__ uint64_t dyn[];
    __shared__ __attribute__((aligned(16))) float qs[128];
    __shared__ float p1[256];
    __shared__ int hist[kBins];         // bucket counts, then fill cursors
    __shared__ int binbase[kBins + 1];  // first candidate slot of each bucket
    __shared__ int sh[82];
    __shared__ int shv[8];
    __shared__ int shk[16];
    __shared__ int shk2[16];
    __shared__ uint32_t s_keep[ONLINE ? kKeepWords : 1];   // kept cells of the delta match
    __shared__ float shf[40];

    const int h = blockIdx.x;
    const int tid = threadIdx.x;
    const int k0 = a.k[0], k1 = a.k[1];
    const int ncells = k0 * k1, kmax = max(k0, k1);
    constexpr int D = 128;
    // LDS regions: centroids during scoring, candidates afterwards
    float* c1T = reinterpret_cast<float*>(dyn);          // [DP][k1 + 1]
    float* c0s = c1T + DP * (k1 + 1);                    // [k0][DP + 1]
    uint64_t* ck = dyn;                                  // [kCap] keys by bucket
    int* cs = reinterpret_cast<int*>(ck + kCap);         // [kCap] sizes
    int* co = cs + kCap;                                 // [kCap] CSR offsets
    int* sg = co + kCap;                                 // [kCap] cell id in rank order
    int* ss = sg + kCap;                                 // [kCap] size in rank order
    int* so = ss + kCap;                                 // [kCap] offset in rank order
    int* seg = so + kCap;                                // [kCap] segment (start | len << 16)

    // ---- loads, all issued before the first wait ----
    // Cell (i, j), g = i * k1 + j, lives in thread t = r * k1 + j with
    // i = r + R * e (R = 1024 / k1 rows of cells in flight): lanes run over j,
    // so one LDS read of C1[j][d] feeds EPT fused multiply-adds.
    const int R = kSelThreads / k1;
    const int jcell = tid % k1, rcell = tid / k1;
    const int32_t* cntp = a.cnt + static_cast<int64_t>(h) * ncells;
    const int32_t* offs = a.off + static_cast<int64_t>(h) * (ncells + 1);
    // with 8 or more cells per thread the CSR offsets are read at the end,
    // for the kept cells only (holding them would spill registers)
    constexpr bool LATE_OFF = EPT >= 8;
    int sz[EPT], co_[LATE_OFF ? 1 : EPT];
    // cell g = i * k1 + jcell = tid + R k1 e: a wave-uniform row base plus
    // the thread id, so each load takes the base in SGPRs and tid as a 32-bit
    // offset.  (Index arithmetic in VGPRs compiled to 64-bit multiply-adds
    // whose unused high operand could be a register still being loaded,
    // which put a wait for the earlier loads before every later one.)
    const int64_t gstride = static_cast<int64_t>(R) * k1;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int i = rcell + R * e;
        const bool in = rcell < R && i < k0;
        const int32_t* crow = cntp + gstride * e;
        sz[e] = in ? crow[static_cast<uint32_t>(tid)] : 0;
        if (!LATE_OFF) co_[e] = in ? (offs + gstride * e)[static_cast<uint32_t>(tid)] : 0;
    }
    // this head's budgets (ragged batches), read with the other loads
    const int hmt_raw = a.head_max_tokens ? vec_load_i32(a.head_max_tokens, h) : INT_MAX;
    const int hbp_raw = a.head_buffer_pages ? vec_load_i32(a.head_buffer_pages, h) : INT_MAX;
    // Online index maintenance (async_update.py): the override slot of each
    // of this thread's cells (-1: merged centroid unchanged), the shadow row
    // of each of the first kOvr slots (thread t stages float4 t & 31 of slot
    // t >> 5), and this thread's delta ring entry (thread = ring index).
    const bool upd = ONLINE && a.upd_slot != nullptr;
    // the counts stay in VGPRs until first use: a readfirstlane here would
    // wait for every load issued so far
    const int n_upd_v = upd ? vec_load_i32(a.upd_n, h) : 0;
    int us[EPT];
    int urow[2] = {0, 0};
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int i = rcell + R * e;
        const bool in = upd && rcell < R && i < k0;
        us[e] = in ? a.upd_slot[static_cast<int64_t>(h) * ncells + i * k1 + jcell] : -1;
    }
    if (upd) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int slot = (tid + u * kSelThreads) >> 5;   // shadow_rows >= 1 here
            const int v = a.upd_row[static_cast<int64_t>(h) * a.shadow_rows + min(slot, a.shadow_rows - 1)];
            urow[u] = slot < a.shadow_rows ? v : 0;
        }
    }
    const bool ring = ONLINE && a.ring_cap > 0;
    int rcode = -3, rrow = 0;
    const int rn_v = ring ? vec_load_i32(a.ring_n, h) : 0;
    if (ring && tid < a.ring_cap) {
        rcode = a.ring_cell[static_cast<int64_t>(h) * a.ring_cap + tid];
        rrow = a.ring_row[static_cast<int64_t>(h) * a.ring_cap + tid];
    }
    // C0 and C1 rows [k][DP] are read coalesced (float4 per thread) and
    // stored in LDS with padded strides (conflict-free word reads): C0
    // row-major [l0][DP + 1] for the per-l0 chain, C1 transposed
    // [d][k1 + 1] so that lanes over l1 read consecutive words.
    const float* c0 = a.cent + (static_cast<int64_t>(h) * 2 + 0) * kmax * DP;
    const float* c1 = a.cent + (static_cast<int64_t>(h) * 2 + 1) * kmax * DP;
    constexpr int kV4 = 128 * DP / 4 / kSelThreads;   // float4 per thread per subspace (k <= 128)
    float4 c0v[kV4], c1v[kV4];
#pragma unroll
    for (int u = 0; u < kV4; ++u) {
        const int i4 = tid + u * kSelThreads;          // float4 index: row i4 / (DP/4)
        c0v[u] = i4 * 4 < k0 * DP ? reinterpret_cast<const float4*>(c0)[i4] : make_float4(0, 0, 0, 0);
        c1v[u] = i4 * 4 < k1 * DP ? reinterpret_cast<const float4*>(c1)[i4] : make_float4(0, 0, 0, 0);
    }
    // the G query rows of this head: rows past G re-read row G - 1 (G >= 1)
    // and are dropped from the sum, so the loads are unconditional and all
    // in flight at once
    uint16_t qv[kMaxGroups];
    if (tid < D) {
        const uint16_t* qh = a.q + static_cast<int64_t>(h) * a.G * D;
        load_group_rows(qh, a.G, tid, qv);
    }
#pragma unroll
    for (int u = 0; u < kV4; ++u) {
        const int i4 = tid + u * kSelThreads;
        const int r = (i4 * 4) / DP, d = (i4 * 4) % DP;
        const float e0[4] = {c0v[u].x, c0v[u].y, c0v[u].z, c0v[u].w};
        const float e1[4] = {c1v[u].x, c1v[u].y, c1v[u].z, c1v[u].w};
        if (r < k0) {
#pragma unroll
            for (int x = 0; x < 4; ++x) c0s[r * (DP + 1) + d + x] = e0[x];
        }
        if (r < k1) {
#pragma unroll
            for (int x = 0; x < 4; ++x) c1T[(d + x) * (k1 + 1) + r] = e1[x];
        }
    }
    if (tid < D) {
        float acc = 0.0f;   // grouped-query sum, g ascending (compute_impl.cu:80-87)
#pragma unroll
        for (int g = 0; g < kMaxGroups; ++g)
            if (g < a.G) acc += bf16_to_f32(qv[g]);
        qs[tid] = acc;
    }
    for (int i = tid; i < kBins; i += kSelThreads) hist[i] = 0;
    if (ring)
        for (int i = tid; i < kKeepWords; i += kSelThreads) s_keep[i] = 0;
    if (tid == 0) shv[0] = 0;
    __syncthreads();
    // chain over the first subspace, once per l0
    if (tid < k0) {
        float acc = 0.0f;
#pragma unroll
        for (int d = 0; d < DP; ++d) acc = __builtin_fmaf(qs[d], c0s[tid * (DP + 1) + d], acc);
        p1[tid] = acc;
    }
    __syncthreads();

    // shadow rows of the first kOvr override slots, in flight during scoring
    float4 ovv[2] = {};
    if (upd) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int row = min(max(urow[u], 0), a.shadow_rows - 1);
            ovv[u] = reinterpret_cast<const float4*>(a.shadow + (static_cast<int64_t>(h) * a.shadow_rows + row) *
                                                     128)[(tid + u * kSelThreads) & 31];
        }
    }

    // ---- scores: the chain continues over the second subspace ----
    float sc[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int i = rcell + R * e;
        sc[e] = p1[i < k0 ? i : 0];
    }
    if (rcell < R) {
        if constexpr (EPT >= 8) {
            // 8+ fused multiply-adds per LDS read already: a rolled loop keeps
            // the centroid reads from being hoisted into spilled registers
#pragma unroll 1
            for (int d0 = 0; d0 < DP; d0 += 8) {
#pragma unroll
                for (int d = d0; d < d0 + 8; ++d) {
                    const float qd = qs[DP + d];
                    const float cv = c1T[d * (k1 + 1) + jcell];
#pragma unroll
                    for (int e = 0; e < EPT; ++e) sc[e] = __builtin_fmaf(qd, cv, sc[e]);
                }
            }
        } else {
#pragma unroll
            for (int d = 0; d < DP; ++d) {
                const float qd = qs[DP + d];
                const float cv = c1T[d * (k1 + 1) + jcell];
#pragma unroll
                for (int e = 0; e < EPT; ++e) sc[e] = __builtin_fmaf(qd, cv, sc[e]);
            }
        }
    }
    // cells whose centroid was replaced: the full 128-term chain over the
    // shadow row (compute_impl.cu:80-101 on the updated centroid), kOvr
    // slots per pass, staged in LDS after the C0 rows
    float* ovr = c0s + k0 * (DP + 1);   // [kOvr][129] replaced centroids staged in LDS
    float* ovs = ovr + kOvr * 129;      // [kOvr] their scores
    const int n_upd = __builtin_amdgcn_readfirstlane(n_upd_v);
    const int rn = min(__builtin_amdgcn_readfirstlane(rn_v), a.ring_cap);
    if (ONLINE && n_upd > kOvr) {
        // more than kOvr replaced cells: passes of kOvr slots before the range
        for (int base = 0; base < n_upd; base += kOvr) {
            if (base > 0) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int slot = base + ((tid + u * kSelThreads) >> 5);
                    const int row = slot < a.shadow_rows ? a.upd_row[static_cast<int64_t>(h) * a.shadow_rows + slot] : 0;
                    const int rc = min(max(row, 0), a.shadow_rows - 1);
                    ovv[u] = reinterpret_cast<const float4*>(
                        a.shadow + (static_cast<int64_t>(h) * a.shadow_rows + rc) * 128)[(tid + u * kSelThreads) & 31];
                }
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int i4 = tid + u * kSelThreads;
                float* dst = ovr + (i4 >> 5) * 129 + (i4 & 31) * 4;
                dst[0] = ovv[u].x;
                dst[1] = ovv[u].y;
                dst[2] = ovv[u].z;
                dst[3] = ovv[u].w;
            }
            __syncthreads();
            if (tid < kOvr && base + tid < n_upd) {
                float acc = 0.0f;
                for (int d = 0; d < 128; ++d) acc = __builtin_fmaf(qs[d], ovr[tid * 129 + d], acc);
                ovs[tid] = acc;
            }
            __syncthreads();
#pragma unroll
            for (int e = 0; e < EPT; ++e)
                if (us[e] >= base && us[e] < base + kOvr) sc[e] = ovs[us[e] - base];
            __syncthreads();
        }
    }
    // up to kOvr replaced cells: their rows (loaded during the scoring) go to
    // LDS now; wave 0 scores them between the two barriers of the range
    // reduction, whose range then covers both old and new scores
    const bool ovr_one = ONLINE && n_upd > 0 && n_upd <= kOvr;
    if (ovr_one) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int i4 = tid + u * kSelThreads;
            float* dst = ovr + (i4 >> 5) * 129 + (i4 & 31) * 4;
            dst[0] = ovv[u].x;
            dst[1] = ovv[u].y;
            dst[2] = ovv[u].z;
            dst[3] = ovv[u].w;
        }
    }
    int nvalid = 0;
    float smax = -INFINITY, smin = INFINITY;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
        if (sz[e] > 0) {
            ++nvalid;
            smax = fmaxf(smax, sc[e]);
            smin = fminf(smin, sc[e]);
        }
    {
        const int w = tid >> 6;
        const int nv = wave_sum_i(nvalid);
        const float mx = wave_max(smax);
        const float mn = -wave_max(-smin);
        if (lane_id() == 0) {
            sh[w] = nv;
            shf[w] = mx;
            shf[16 + w] = mn;
        }
    }
    __syncthreads();
    float ov_mx = -INFINITY, ov_mn = INFINITY;
    if (ovr_one && tid < 64) {
        if (tid < n_upd) {
            float acc = 0.0f;   // compute_impl.cu:80-101 over the replaced centroid
            for (int d = 0; d < 128; ++d) acc = __builtin_fmaf(qs[d], ovr[tid * 129 + d], acc);
            ovs[tid] = acc;
            ov_mx = ov_mn = acc;
        }
        ov_mx = wave_max(ov_mx);
        ov_mn = -wave_max(-ov_mn);
    }
    if (tid == 0) {
        int nv = 0;
        float mx = ov_mx, mn = ov_mn;
        for (int w = 0; w < 16; ++w) {
            nv += sh[w];
            mx = fmaxf(mx, shf[w]);
            mn = fminf(mn, shf[16 + w]);
        }
        shv[1] = nv;
        shf[32] = mx;
        shf[33] = mn;
    }
    __syncthreads();
    if (ovr_one) {
#pragma unroll
        for (int e = 0; e < EPT; ++e)
            if (us[e] >= 0 && us[e] < kOvr) sc[e] = ovs[us[e]];
    }
    const int n_valid = shv[1];
    const float gmax = shf[32], gmin = shf[33];
    // this head's budgets (ragged batches), bounded by the launch-wide ones
    const int max_tokens = min(__builtin_amdgcn_readfirstlane(hmt_raw), a.max_tokens);
    const int buffer_pages = min(__builtin_amdgcn_readfirstlane(hbp_raw), a.buffer_pages);
    // every kept cell costs a page, except in tile mode (no running page cut);
    // the delta match needs the ranks the page cut drops too
    int kp = (a.tile_mode || a.ring_cap > 0) ? a.nprobe : (a.nprobe < buffer_pages ? a.nprobe : buffer_pages);
    kp = kp < n_valid ? kp : n_valid;
    int32_t* prefix_out = a.sel_prefix + static_cast<int64_t>(h) * (a.sel_cap + 1);
    if (kp <= 0) {
        if (tid == 0) {
            a.n_sel[h] = 0;
            a.n_rows[h] = 0;
            prefix_out[0] = 0;
        }
        if (ring) delta_match(a, h, 0, nullptr, false, s_keep, shk, rcode, rrow, rn);
        return;
    }

    // ---- candidates: iterative linear-bucket refinement ----
    // st: 0 = dropped, 1 = in play, 2 = placed.  Each level buckets the
    // in-play scores linearly over their [lo, hi] (higher score -> lower or
    // equal bucket), places every bucket wholly above the one holding the
    // kp-th best cell and, when that bucket still does not fit in kCap
    // slots, refines inside it.  Placed cells form segments (one per bucket)
    // that are already in rank order relative to each other.
    int st[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) st[e] = sz[e] > 0 ? 1 : 0;
    int c_sel = 0;
    float lo = gmin, hi = gmax;
    for (int level = 0; level < 16; ++level) {
        const float range = hi - lo;
        const float inv = range > 0.0f ? static_cast<float>(kBins) / range : 0.0f;
#pragma unroll
        for (int e = 0; e < EPT; ++e)
            if (st[e] == 1) atomicAdd(&hist[bucket_of(sc[e], hi, inv)], 1);
        __syncthreads();
        const int need = kp - c_sel;
        {
            const int b0 = 2 * tid, b1 = 2 * tid + 1;
            const int h0 = hist[b0], h1 = hist[b1];
            int total;
            const int incl = block_incl_scan(h0 + h1, sh, total);
            const int excl = incl - h0 - h1;
            binbase[b0] = excl;
            binbase[b1] = excl + h0;
            if (tid == kSelThreads - 1) binbase[kBins] = incl;
            if (excl < need && excl + h0 >= need) {
                shv[2] = b0;
                shv[3] = excl;
                shv[4] = excl + h0;
            } else if (excl + h0 < need && incl >= need) {
                shv[2] = b1;
                shv[3] = excl + h0;
                shv[4] = incl;
            }
        }
        for (int i = tid; i < kBins; i += kSelThreads) hist[i] = 0;   // fill cursors
        __syncthreads();
        const int bK = shv[2], c_lt = shv[3], c_le = shv[4];
        const bool fits = c_sel + c_le <= kCap;
        const bool flat = !(range > 0.0f);
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
            if (st[e] != 1) continue;
            const int b = bucket_of(sc[e], hi, inv);
            if (b < bK || (fits && b == bK)) {
                const int g = (rcell + R * e) * k1 + jcell;
                const int slot = c_sel + binbase[b] + atomicAdd(&hist[b], 1);
                ck[slot] = cell_key(order_key(sc[e]), g);
                cs[slot] = sz[e];
                if (!LATE_OFF) co[slot] = co_[e];
                seg[slot] = (c_sel + binbase[b]) | ((binbase[b + 1] - binbase[b]) << 16);
                st[e] = 2;
            } else if (b > bK) {
                st[e] = 0;
            }
        }
        if (fits) {
            c_sel += c_le;
            break;
        }
        c_sel += c_lt;
        __syncthreads();
        for (int i = tid; i < kBins; i += kSelThreads) hist[i] = 0;
        if (flat) {
            // every cell still in play has the same score: the best are the
            // lowest cell ids, i.e. the first `need` in cell-id order
            const int keep = kp - c_sel;
            int base = 0;
#pragma unroll
            for (int e = 0; e < EPT; ++e) {
                const int f = st[e] == 1 ? 1 : 0;
                int tot;
                const int r = block_incl_scan(f, sh, tot) - f + base;
                if (f && r < keep) {
                    const int g = (rcell + R * e) * k1 + jcell;
                    const int slot = c_sel + r;
                    ck[slot] = cell_key(order_key(sc[e]), g);
                    cs[slot] = sz[e];
                    if (!LATE_OFF) co[slot] = co_[e];
                    seg[slot] = c_sel | (keep << 16);
                }
                base += tot;
            }
            c_sel += keep;
            break;
        }
        // next level: range of the cells still in play
        float mx = -INFINITY, mn = INFINITY;
#pragma unroll
        for (int e = 0; e < EPT; ++e)
            if (st[e] == 1) {
                mx = fmaxf(mx, sc[e]);
                mn = fminf(mn, sc[e]);
            }
        mx = wave_max(mx);
        mn = -wave_max(-mn);
        if (lane_id() == 0) {
            shf[tid >> 6] = mx;
            shf[16 + (tid >> 6)] = mn;
        }
        __syncthreads();
        hi = -INFINITY;
        lo = INFINITY;
        for (int w = 0; w < 16; ++w) {
            hi = fmaxf(hi, shf[w]);
            lo = fminf(lo, shf[16 + w]);
        }
        __syncthreads();
    }
    __syncthreads();
    const int C = c_sel;
    // rank inside each segment by counting larger keys (segments are short)
    for (int sl = tid; sl < C; sl += kSelThreads) {
        const uint64_t key = ck[sl];
        const int sg0 = seg[sl] & 0xFFFF, sgn = seg[sl] >> 16;
        int r = 0;
        for (int i = sg0; i < sg0 + sgn; ++i) r += ck[i] > key;
        const int pos = sg0 + r;
        sg[pos] = cell_of_key(key);
        ss[pos] = cs[sl];
        if (!LATE_OFF) so[pos] = co[sl];
    }
    __syncthreads();

    // ---- budget rules in rank order (ranks 2*tid, 2*tid+1) ----
    int s2[2], pg2[2];
    int tsum = 0, psum = 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int r = 2 * tid + u;
        s2[u] = r < C ? ss[r] : 0;
        // pages = ceil(size / page_size); a power-of-two page size (8 in every
        // configuration) takes a shift instead of an integer division
        pg2[u] = (a.page_size & (a.page_size - 1)) == 0 ? (s2[u] + a.page_size - 1) >> (__builtin_ctz(a.page_size))
                                                        : (s2[u] + a.page_size - 1) / a.page_size;
        // tile mode counts the cells that alone overflow the page budget
        if (a.tile_mode) pg2[u] = pg2[u] > buffer_pages ? 1 : 0;
        tsum += s2[u];
        psum += pg2[u];
    }
    int ttot, ptot;
    int tincl = tsum, pincl = psum;
    block_incl_scan2(tincl, pincl, sh, ttot, ptot);
    int texcl = tincl - tsum, pexcl = pincl - psum;
    int kept = 0, kept_tok = 0;
    int excl_tok[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int r = 2 * tid + u;
        excl_tok[u] = texcl;
        pexcl += pg2[u];
        const bool keep_tok = r < C && r < a.nprobe && texcl < max_tokens;
        const bool keep = keep_tok && pexcl <= (a.tile_mode ? 0 : buffer_pages);
        kept += keep ? 1 : 0;
        kept_tok += keep_tok ? 1 : 0;
        if (ring && keep_tok) {   // the kept cell set of the delta match
            const int g = sg[r];
            atomicOr(&s_keep[g >> 5], 1u << (g & 31));
        }
        texcl += s2[u];
    }
    // the rules are monotone in rank (prefixes only grow), so the kept ranks
    // are exactly the first m (the first m_tok before the page cut): count
    // them per wave, then over the 16 waves
    {
        const int wk = wave_sum_i(kept);
        const int wt = ring ? wave_sum_i(kept_tok) : 0;
        if (lane_id() == 0) {
            sh[66 + (tid >> 6)] = wk;
            if (ONLINE) shk[tid >> 6] = wt;
        }
    }
    __syncthreads();
    int m = 0, m_tok = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) m += sh[66 + w];
    if (ring) {
#pragma unroll
        for (int w = 0; w < 16; ++w) m_tok += shk[w];
    }
    int32_t* out_cell = a.sel_cell + static_cast<int64_t>(h) * a.sel_cap;
    int32_t* out_off = a.sel_offset + static_cast<int64_t>(h) * a.sel_cap;
    int32_t* out_cnt = a.sel_count + static_cast<int64_t>(h) * a.sel_cap;
    // late CSR offsets: both ranks' loads issued before either is stored
    // (ranks past m re-read rank m - 1)
    int offv[2] = {0, 0};
    if (LATE_OFF && m > 0) {
#pragma unroll
        for (int u = 0; u < 2; ++u) offv[u] = offs[sg[min(2 * tid + u, m - 1)]];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int r = 2 * tid + u;
        if (r < m) {
            out_cell[r] = sg[r];
            out_off[r] = LATE_OFF ? offv[u] : so[r];
            out_cnt[r] = s2[u];
            prefix_out[r] = excl_tok[u];
        }
        if (r == m - 1) {
            const int total = excl_tok[u] + s2[u];
            prefix_out[m] = total;
            a.n_sel[h] = m;
            a.n_rows[h] = total;
            if (ONLINE) shv[5] = total;
        }
    }
    if (m == 0 && tid == 0) {
        a.n_sel[h] = 0;
        a.n_rows[h] = 0;
        prefix_out[0] = 0;
    }
    if (ring) delta_match(a, h, m_tok, &shv[5], m > 0, s_keep, shk2, rcode, rrow, rn);
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

// ---- Tile mode with the delta append (retrieval.py:480-509) ----
//
// The reference attends tile after tile, each through its own execution
// buffer, and appends the delta entries that match a tile after that tile's
// rows (async_update.py:41-76).  Here every tile is attended in the one pass
// over the union of the tiles, so only the delta list has to follow the
// tiles: per tile t of head h, the valid ring entries (index order) whose
// cell is one of the tile's cells -- or the padding id, when the head took
// fewer cells into tile t than the head that took most, so that its row of
// the tile tensor is padded -- up to the buffer rows the tile's cells leave.
// Tiles are each head's greedy runs of its ranked cells that fit the page
// budget (_build_cluster_tiles, retrieval.py:30-112); the tile count of the
// call is the most any head has.  Two launches after the selection:
//   tile_ends_kernel   (one workgroup per head) the end rank of every tile
//   tile_delta_kernel  (one workgroup per head) the cross-head tile sizes
//                      where a padding entry exists, and the delta list
// A padding entry can match several tiles, and the reference then attends
// its row once per such tile; the list keeps every repeat up to ring_cap
// rows per head.
constexpr int kTileRanks = 8192;   // ranks the tiles of a head cover (>= any K')
constexpr int kTileSet = 2048;     // ring-code set (ring <= 1024 entries)

struct TileDeltaParams {
    int H, sel_cap;
    const int32_t* sel_cell;
    const int32_t* sel_count;
    const int32_t* sel_prefix;
    const int32_t* n_sel;
    int page_size, buffer_pages;
    const int32_t* head_buffer_pages;
    const int32_t* ring_cell;
    const int32_t* ring_row;
    const int32_t* ring_n;
    int ring_cap, exec_rows;
    int32_t* delta_rows;
    int32_t* n_delta;
    int32_t* tile_end;   // [H][sel_cap] scratch
    int32_t* n_tiles;    // [H] scratch
};

__device__ __forceinline__ int tile_block_max(int v, int* sh) {
    v = wave_max_i(v);
    if (lane_id() == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    int r = sh[0];
#pragma unroll
    for (int w = 1; w < 16; ++w) r = max(r, sh[w]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ int tile_block_min(int v, int* sh) {
    return -tile_block_max(-v, sh);
}

__global__ __launch_bounds__(1024) void tile_ends_kernel(TileDeltaParams a) {
    __shared__ int P[kTileRanks];          // inclusive page prefix over the ranks
    __shared__ uint16_t nxt[kTileRanks];   // end of the tile that starts at each rank
    __shared__ int sh[80];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int m = min(max(a.n_sel[h], 0), min(a.sel_cap, kTileRanks));
    const int B = a.head_buffer_pages ? min(a.head_buffer_pages[h], a.buffer_pages) : a.buffer_pages;
    const int32_t* cnt = a.sel_count + static_cast<int64_t>(h) * a.sel_cap;
    constexpr int RPT = kTileRanks / 1024;
    int pg[RPT], sum = 0;
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
        const int r = RPT * tid + u;
        const int sz = r < m ? cnt[r] : 0;
        pg[u] = sz > 0 ? max((sz + a.page_size - 1) / a.page_size, 1) : 0;
        sum += pg[u];
    }
    int incl = sum, dummy = 0, tot, dtot;
    block_incl_scan2(incl, dummy, sh, tot, dtot);
    int run = incl - sum;
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
        run += pg[u];
        P[RPT * tid + u] = run;
    }
    __syncthreads();
    // the tile that starts at rank s ends before the first rank whose
    // prefix exceeds the pages before s plus the budget (every rank below m
    // fits alone: the selection stops at the first cell that does not)
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
        const int s0 = RPT * tid + u;
        if (s0 < m) {
            const int lim = (s0 > 0 ? P[s0 - 1] : 0) + B;
            int lo = s0, hi = m;   // first e in [s0, m] with P[e] > lim (m: none)
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (P[mid] > lim) hi = mid;
                else lo = mid + 1;
            }
            nxt[s0] = static_cast<uint16_t>(max(lo, s0 + 1));
        }
    }
    __syncthreads();
    if (tid == 0) {
        int32_t* ends = a.tile_end + static_cast<int64_t>(h) * a.sel_cap;
        int t = 0;
        for (int s0 = 0; s0 < m; s0 = nxt[s0]) ends[t++] = nxt[s0];
        a.n_tiles[h] = t;
    }
}

__device__ __forceinline__ int tile_slot(int code) {
    return static_cast<int>((static_cast<uint32_t>(code) * 2654435761u) >> 21) & (kTileSet - 1);
}

__global__ __launch_bounds__(1024) void tile_delta_kernel(TileDeltaParams a) {
    __shared__ int te[kTileRanks];     // this head's tile ends
    __shared__ int rtab[kTileSet];     // ring-code set
    __shared__ int rtile[kTileSet];    // tile of each code (-1: in no tile)
    __shared__ int sh[80];
    const int h = blockIdx.x, tid = threadIdx.x, wave = tid >> 6;
    const int sc = a.sel_cap;
    const int m = min(max(a.n_sel[h], 0), min(sc, kTileRanks));
    const int nh = min(a.n_tiles[h], m);
    int nt = 0;
    for (int i = tid; i < a.H; i += 1024) nt = max(nt, a.n_tiles[i]);
    for (int t = tid; t < nh; t += 1024) te[t] = a.tile_end[static_cast<int64_t>(h) * sc + t];
    for (int i = tid; i < kTileSet; i += 1024) {
        rtab[i] = -1;
        rtile[i] = -1;
    }
    nt = tile_block_max(nt, sh);   // (its barriers also publish te and the cleared set)
    const int rn = min(max(a.ring_n[h], 0), a.ring_cap);
    int code = -3, rrow = 0, slot = -1;
    if (tid < rn) {
        code = a.ring_cell[static_cast<int64_t>(h) * a.ring_cap + tid];
        rrow = a.ring_row[static_cast<int64_t>(h) * a.ring_cap + tid];
    }
    if (code >= 0) {
        int i = tile_slot(code);
        while (true) {
            const int prev = atomicCAS(&rtab[i], -1, code);
            if (prev == -1 || prev == code) break;
            i = (i + 1) & (kTileSet - 1);
        }
        slot = i;
    }
    __syncthreads();
    // the tile of each ranked cell whose code the ring holds
    for (int r = tid; r < m; r += 1024) {
        const int c = a.sel_cell[static_cast<int64_t>(h) * sc + r];
        int i = tile_slot(c);
        while (rtab[i] != c && rtab[i] != -1) i = (i + 1) & (kTileSet - 1);
        if (rtab[i] == c) {
            int lo = 0, hi = nh - 1;   // the first tile that ends past r
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (te[mid] > r) hi = mid;
                else lo = mid + 1;
            }
            rtile[i] = lo;
        }
    }
    const bool padc = code == -1;
    const int npad = tile_block_max(padc ? 1 : 0, sh);   // any padding entry (its barriers publish rtile)
    const int my_t = slot >= 0 ? rtile[slot] : -1;
    const int32_t* pre = a.sel_prefix + static_cast<int64_t>(h) * (sc + 1);
    int base = 0;
    // every tile when a padding entry can match, else only the tiles holding matches
    int t = npad > 0 ? 0 : tile_block_min(my_t >= 0 ? my_t : INT_MAX, sh);
    while (t < nt) {
        const int s_t = t == 0 ? 0 : (t - 1 < nh ? te[t - 1] : m);
        const int e_t = t < nh ? te[t] : m;
        const int rows_t = e_t > s_t ? pre[e_t] - pre[s_t] : 0;
        bool pad = false;
        if (npad > 0) {   // padded row: another head took more cells into tile t
            int mt = 0;
            for (int i = tid; i < a.H; i += 1024) {
                const int ni = a.n_tiles[i];
                if (t < ni) {
                    const int32_t* ei = a.tile_end + static_cast<int64_t>(i) * sc;
                    mt = max(mt, ei[t] - (t > 0 ? ei[t - 1] : 0));
                }
            }
            mt = tile_block_max(mt, sh);
            pad = e_t - s_t < mt;
        }
        const bool match = my_t == t || (padc && pad);
        const uint64_t bal = __builtin_amdgcn_ballot_w64(match);
        if (lane_id() == 0) sh[wave] = __builtin_popcountll(bal);
        __syncthreads();
        int before = 0, cnt = 0;
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            cnt += sh[w];
            before += w < wave ? sh[w] : 0;
        }
        const int pos = before + __builtin_popcountll(bal & lanemask_lt());
        const int app = min(cnt, max(a.exec_rows - rows_t, 0));
        if (match && pos < app && base + pos < a.ring_cap)
            a.delta_rows[static_cast<int64_t>(h) * a.ring_cap + base + pos] = rrow;
        base += app;
        __syncthreads();   // sh is reused
        t = npad > 0 ? t + 1 : tile_block_min(my_t > t ? my_t : INT_MAX, sh);
    }
    if (tid == 0) a.n_delta[h] = min(base, a.ring_cap);
}

}  // namespace

int select4_validate(const imi_select_args* a);
size_t select4_workspace_size(const imi_select_args* a);
int select4_launch(const imi_select_args* a, hipStream_t stream);

// The one-kernel 2-way path applies while both codebooks fit 128 rows, a
// 1024-thread workgroup holds every cell (16 per thread) and K' fits its
// candidate buffer; larger shapes take the ranking pipeline of
// imi_select4.hip over every global cell.
bool sel2_one_kernel(const imi_select_args* a) {
    if (a->parts != 2) return false;
    const int k0 = a->k[0], k1 = a->k[1];
    const bool rank_all = a->tile_mode || a->ring_cap > 0;
    const int kprime = rank_all ? a->nprobe : (a->nprobe < a->buffer_pages ? a->nprobe : a->buffer_pages);
    return k0 <= 128 && k1 <= 128 && k0 <= 16 * (kSelThreads / k1) && kprime <= kCap;
}

int select_validate(const imi_select_args* a, int64_t& ncells, int& kmax) {
    IMI_REQUIRE(a != nullptr, IMI_ERR_INVALID, "imi_select: null args");
    IMI_REQUIRE(a->query && a->centroids && a->cell_count && a->cell_offset, IMI_ERR_INVALID,
                "imi_select: null input pointer");
    IMI_REQUIRE(a->kv_heads > 0 && a->groups > 0, IMI_ERR_INVALID, "imi_select: empty shape");
    IMI_REQUIRE(a->groups <= kMaxGroups, IMI_ERR_UNSUPPORTED, "imi_select: %d query heads per kv head exceed %d",
                a->groups, kMaxGroups);
    IMI_REQUIRE(a->dim == 128, IMI_ERR_UNSUPPORTED, "imi_select: head_dim must be 128");
    IMI_REQUIRE(a->parts == 1 || a->parts == 2 || a->parts == 4, IMI_ERR_UNSUPPORTED,
                "imi_select: parts must be 1 (IVF), 2 or 4 (got %d)", a->parts);
    if (a->ring_cap != 0) {
        IMI_REQUIRE(a->ring_cap > 0 && a->ring_cap <= kRingCap, IMI_ERR_UNSUPPORTED,
                    "imi_select: ring_cap %d outside [1, %d]", a->ring_cap, kRingCap);
        IMI_REQUIRE(a->ring_cell && a->ring_row && a->ring_n, IMI_ERR_INVALID, "imi_select: null delta ring");
        IMI_REQUIRE(a->exec_rows >= 0, IMI_ERR_INVALID, "imi_select: exec_rows must be >= 0");
    }
    if (a->upd_slot)
        IMI_REQUIRE(a->shadow && a->upd_row && a->upd_n && a->shadow_rows > 0, IMI_ERR_INVALID,
                    "imi_select: replaced centroids need shadow, shadow_rows, upd_row and upd_n");
    if (a->parts != 2) {
        IMI_REQUIRE(a->page_size > 0 && a->nprobe > 0 && a->max_tokens > 0 && a->buffer_pages > 0, IMI_ERR_INVALID,
                    "imi_select: budgets must be positive");
        kmax = 0;
        ncells = 1;
        for (int p = 0; p < a->parts; ++p) {
            kmax = a->k[p] > kmax ? a->k[p] : kmax;
            ncells *= a->k[p];
        }
        return select4_validate(a);
    }
    IMI_REQUIRE(a->page_size > 0 && a->nprobe > 0 && a->max_tokens > 0 && a->buffer_pages > 0, IMI_ERR_INVALID,
                "imi_select: budgets must be positive");
    kmax = a->k[0] > a->k[1] ? a->k[0] : a->k[1];
    IMI_REQUIRE(a->k[0] >= 1 && a->k[1] >= 1 && kmax <= kImiMaxK, IMI_ERR_UNSUPPORTED, "imi_select: k outside [1,%d]",
                kImiMaxK);
    ncells = static_cast<int64_t>(a->k[0]) * a->k[1];
    if (!sel2_one_kernel(a)) return select4_validate(a);
    const bool rank_all = a->tile_mode || a->ring_cap > 0;
    const int kprime = rank_all ? a->nprobe : (a->nprobe < a->buffer_pages ? a->nprobe : a->buffer_pages);
    IMI_REQUIRE(a->sel_cap >= kprime, IMI_ERR_INVALID, "imi_select: sel_cap %d < %d (%s)", a->sel_cap, kprime,
                rank_all ? "nprobe" : "min(nprobe, buffer_pages)");
    return IMI_OK;
}

namespace {

template <int EPT, bool ONLINE>
int launch_ept(const SelParams& p, int H, hipStream_t stream) {
    constexpr int DP = 64;
    const size_t cand = static_cast<size_t>(kCap) * (sizeof(uint64_t) + 6 * sizeof(int));
    size_t ct = (static_cast<size_t>(DP) * (p.k[1] + 1) + static_cast<size_t>(p.k[0]) * (DP + 1)) * sizeof(float);
    if (p.upd_slot) ct += static_cast<size_t>(kOvr) * 130 * sizeof(float);   // override rows + scores
    const size_t lds = cand > ct ? cand : ct;
    static bool attr_set = false;
    if (!attr_set) {
        IMI_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&select_kernel<DP, EPT, ONLINE>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024));
        attr_set = true;
    }
    hipLaunchKernelGGL((select_kernel<DP, EPT, ONLINE>), dim3(H), dim3(kSelThreads), lds, stream, p);
    IMI_LAUNCH_CHECK("select_kernel");
    return IMI_OK;
}

int select_one_kernel(const imi_select_args* a, hipStream_t stream) {
    SelParams p;
    p.q = a->query;
    p.cent = a->centroids;
    p.cnt = a->cell_count;
    p.off = a->cell_offset;
    p.H = a->kv_heads;
    p.G = a->groups;
    p.k[0] = a->k[0];
    p.k[1] = a->k[1];
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
    p.upd_n = a->upd_n;
    p.ring_cell = a->ring_cell;
    p.ring_row = a->ring_row;
    p.ring_n = a->ring_n;
    p.ring_cap = a->tile_mode ? 0 : a->ring_cap;   // tile mode: the tile launches append the delta
    p.exec_rows = a->exec_rows;
    p.delta_rows = a->delta_rows;
    p.n_delta = a->n_delta;
    const int rows_in_flight = kSelThreads / a->k[1];
    const int ept = (a->k[0] + rows_in_flight - 1) / rows_in_flight;
    if (p.upd_slot || p.ring_cap > 0) {
        if (ept <= 1) return launch_ept<1, true>(p, a->kv_heads, stream);
        if (ept <= 2) return launch_ept<2, true>(p, a->kv_heads, stream);
        if (ept <= 4) return launch_ept<4, true>(p, a->kv_heads, stream);
        if (ept <= 8) return launch_ept<8, true>(p, a->kv_heads, stream);
        return launch_ept<16, true>(p, a->kv_heads, stream);
    }
    if (ept <= 1) return launch_ept<1, false>(p, a->kv_heads, stream);
    if (ept <= 2) return launch_ept<2, false>(p, a->kv_heads, stream);
    if (ept <= 4) return launch_ept<4, false>(p, a->kv_heads, stream);
    if (ept <= 8) return launch_ept<8, false>(p, a->kv_heads, stream);
    return launch_ept<16, false>(p, a->kv_heads, stream);
}

}  // namespace

// Scratch of the tile-mode delta append: the tile ends of every head and
// their counts (tile mode with a delta ring only).
size_t tile_delta_bytes(const imi_select_args* a) {
    if (!(a->tile_mode && a->ring_cap > 0)) return 0;
    return (static_cast<size_t>(a->kv_heads) * (a->sel_cap + 1)) * sizeof(int32_t) + 256;
}

int tile_delta_launch(const imi_select_args* a, void* scratch, hipStream_t stream) {
    TileDeltaParams t{};
    t.H = a->kv_heads;
    t.sel_cap = a->sel_cap;
    t.sel_cell = a->sel_cell;
    t.sel_count = a->sel_count;
    t.sel_prefix = a->sel_prefix;
    t.n_sel = a->n_selected;
    t.page_size = a->page_size;
    t.buffer_pages = a->buffer_pages;
    t.head_buffer_pages = a->head_buffer_pages;
    t.ring_cell = a->ring_cell;
    t.ring_row = a->ring_row;
    t.ring_n = a->ring_n;
    t.ring_cap = a->ring_cap;
    t.exec_rows = a->exec_rows;
    t.delta_rows = a->delta_rows;
    t.n_delta = a->n_delta;
    const uintptr_t p0 = (reinterpret_cast<uintptr_t>(scratch) + 255) & ~static_cast<uintptr_t>(255);
    t.tile_end = reinterpret_cast<int32_t*>(p0);
    t.n_tiles = t.tile_end + static_cast<size_t>(a->kv_heads) * a->sel_cap;
    hipLaunchKernelGGL(tile_ends_kernel, dim3(a->kv_heads), dim3(1024), 0, stream, t);
    IMI_LAUNCH_CHECK("tile_ends_kernel");
    hipLaunchKernelGGL(tile_delta_kernel, dim3(a->kv_heads), dim3(1024), 0, stream, t);
    IMI_LAUNCH_CHECK("tile_delta_kernel");
    return IMI_OK;
}

// Workspace of a 2-way selection: for the one-kernel path only the tile-mode
// delta scratch, the ranking pipeline's otherwise.
size_t sel2_keys_bytes(const imi_select_args* a) {
    if (sel2_one_kernel(a)) return tile_delta_bytes(a);
    return select4_workspace_size(a);
}

int select_launch(const imi_select_args* a, hipStream_t stream) {
    int64_t ncells;
    int kmax;
    int rc = select_validate(a, ncells, kmax);
    if (rc) return rc;
    IMI_REQUIRE(a->sel_cell && a->sel_offset && a->sel_count && a->sel_prefix && a->n_selected && a->n_rows,
                IMI_ERR_INVALID, "imi_select: null output pointer");
    IMI_REQUIRE(a->ring_cap == 0 || (a->delta_rows && a->n_delta), IMI_ERR_INVALID,
                "imi_select: null delta output pointer");
    if (a->parts == 2 && sel2_one_kernel(a)) {
        if (a->tile_mode && a->ring_cap > 0)
            IMI_REQUIRE(a->workspace && a->workspace_bytes >= tile_delta_bytes(a), IMI_ERR_WORKSPACE,
                        "imi_select: workspace %zu bytes < %zu required", a->workspace_bytes, tile_delta_bytes(a));
        rc = select_one_kernel(a, stream);
        if (rc || !(a->tile_mode && a->ring_cap > 0)) return rc;
        return tile_delta_launch(a, a->workspace, stream);
    }
    return select4_launch(a, stream);
}

}  // namespace imi

using namespace imi;

extern "C" int imi_select_workspace_size(const imi_select_args* a, size_t* bytes) {
    clear_error();
    int64_t ncells;
    int kmax;
    int rc = select_validate(a, ncells, kmax);
    if (rc) return rc;
    IMI_REQUIRE(bytes != nullptr, IMI_ERR_INVALID, "imi_select_workspace_size: null output");
    *bytes = a->parts == 4 ? select4_workspace_size(a) : sel2_keys_bytes(a);
    return IMI_OK;
}

extern "C" int imi_select(const imi_select_args* a, imi_stream_t stream) {
    clear_error();
    return select_launch(a, reinterpret_cast<hipStream_t>(stream));
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
