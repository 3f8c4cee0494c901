// Fused gather + GQA sparse decode attention on gfx950 (HBM-bound).
//
// Reference: the execution-buffer gather concat_gather_copy
// (include/copy_kernel.cuh:220-335, launched by cuda/gather_copy.cu:100-213:
// rows = [static_len steady rows | miss pages | hit pages]) followed by the
// unvendored weighted_flash_decoding (retrieval.py:439-447).  Here the rows
// are read in place: the steady zone for the first static_len rows, then the
// CSR list rows of the selected cells (each workgroup stages the head's
// selection in LDS and binary-searches its rows) -- no execution buffer.
//
// Grid: H * nsplit workgroups of 8 waves, block b -> head b % H, split b / H,
// so with 8 KV heads each head's splits run on one XCD (dispatch is round
// robin over the 8 XCDs).  Each wave owns 16 or 32 consecutive rows; a row is
// read by 16 lanes x 16 bytes (fully coalesced 1 KiB per wave instruction for
// 4 rows).  q.k uses v_dot2_f32_bf16 and a 16-lane DPP reduction; softmax is
// online in base 2 with fp32 state; the 32 (wave, row-group) states of a
// workgroup merge in LDS into one partial, written with plain stores.  A
// second kernel merges each head's partials in split order (deterministic)
// and writes the bf16 output and the LSE: the kernel boundary makes the
// partials visible across XCDs without any device-scope fence.
#include "imi_common.hpp"

namespace imi {

int select_launch(const imi_select_args* a, hipStream_t stream);
int select_validate(const imi_select_args* a, int64_t& ncells, int& kmax);

namespace {

constexpr int kWaves = 8;            // waves per workgroup (512 threads)
constexpr int kMaxSplit = 1024;      // splits per head the merge kernel handles
constexpr int kSelCapMax = 2048;     // selected cells per head the gather indexes

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

struct AttnParams {
    const uint16_t* q;
    const uint16_t* sk;
    const uint16_t* sv;
    int64_t s_stride;
    int static_len;
    const uint16_t* lk;
    const uint16_t* lv;
    int64_t list_rows;
    const int32_t* sel_offset;  // [H][sel_cap]
    const int32_t* sel_prefix;  // [H][sel_cap + 1]
    const int32_t* n_selected;  // [H]
    int sel_cap;
    const int32_t* n_rows;      // [H]
    int H, nsplit;
    int rows_per_block;
    float scale_log2;        // scale * log2(e)
    float* part_acc;         // [H][nsplit][G][128]
    float* part_ml;          // [H][nsplit][G][2]
    uint16_t* out;           // [H*G][128]
    float* lse;              // [H*G] or null
};

__device__ __forceinline__ float dot8(const uint4& k, const uint32_t (&q)[4]) {
    float s = 0.0f;
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k.x), __builtin_bit_cast(bf16x2_t, q[0]), s, false);
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k.y), __builtin_bit_cast(bf16x2_t, q[1]), s, false);
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k.z), __builtin_bit_cast(bf16x2_t, q[2]), s, false);
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, k.w), __builtin_bit_cast(bf16x2_t, q[3]), s, false);
    return s;
}

__device__ __forceinline__ float bf16_at(const uint4& v, int u) {
    const uint32_t w = u < 2 ? v.x : u < 4 ? v.y : u < 6 ? v.z : v.w;
    return (u & 1) ? bf16_hi(w) : bf16_lo(w);
}

__device__ __forceinline__ float safe_exp2(float x) { return x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(x); }

// Weight exp2(m - M) of a state with running max m inside a merge whose max
// is M; an empty state (m = -inf) weighs 0 even when M is -inf too.
__device__ __forceinline__ float wexp(float m, float M) { return m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M); }

// One workgroup = 8 waves over rows [split * rows_per_block, +rows_per_block)
// of head h; each wave owns TILES * 16 consecutive rows, read as tiles of 4
// rows x 4 iterations (16 lanes x 16 bytes per row).  The workgroup writes
// one partial (max, sum, unnormalised output) with plain stores; merge_kernel
// combines the partials after the kernel boundary.
template <int G, int TILES>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void attention_kernel(AttnParams a) {
    constexpr int RW = TILES * 16;
    __shared__ float s_acc[kWaves][G][128];
    __shared__ float s_ml[kWaves][G][2];
    __shared__ int s_pre[kSelCapMax + 1];
    __shared__ int s_off[kSelCapMax];

    const int b = blockIdx.x;
    const int h = b % a.H;
    const int split = b / a.H;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int rg = lane >> 4, li = lane & 15;
    const int row0 = split * a.rows_per_block + wave * RW;

    // One round trip for everything the gather needs: q, the row and cell
    // counts, and the head's selection (CSR offset and row prefix per cell).
    uint32_t qp[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const uint4 v = *reinterpret_cast<const uint4*>(a.q + (static_cast<int64_t>(h) * G + g) * 128 + li * 8);
        qp[g][0] = v.x; qp[g][1] = v.y; qp[g][2] = v.z; qp[g][3] = v.w;
    }
    const int nrows = a.n_rows[h];
    const int m = a.n_selected[h];
    {
        const int32_t* pre = a.sel_prefix + static_cast<int64_t>(h) * (a.sel_cap + 1);
        const int32_t* off = a.sel_offset + static_cast<int64_t>(h) * a.sel_cap;
        for (int i = tid; i <= a.sel_cap; i += 64 * kWaves) {
            s_pre[i] = pre[i];
            if (i < a.sel_cap) s_off[i] = off[i];
        }
    }
    __syncthreads();
    // row location of lane < RW: cell r with pre[r] <= j < pre[r + 1]
    int myloc = 0;
    {
        const int j = row0 + lane - a.static_len;
        if (lane < RW && j >= 0 && j < nrows) {
            int lo = 0, hi = m;
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (s_pre[mid] <= j) lo = mid; else hi = mid;
            }
            myloc = s_off[lo] + (j - s_pre[lo]);
        }
    }
    const int N = a.static_len + nrows;
    float m_[G], l_[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m_[g] = -INFINITY;
        l_[g] = 0.0f;
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[g][u] = 0.0f;
    }
    const uint16_t* skh = a.sk + static_cast<int64_t>(h) * a.s_stride * 128;
    const uint16_t* svh = a.sv + static_cast<int64_t>(h) * a.s_stride * 128;
    const uint16_t* lkh = a.lk + static_cast<int64_t>(h) * a.list_rows * 128;
    const uint16_t* lvh = a.lv + static_cast<int64_t>(h) * a.list_rows * 128;

    if (row0 < N) {
        // Branch-free gather: rows past N read row 0 of the list (always in
        // bounds) and get a -inf score, so all 2 * 4 * TILES loads issue
        // back to back.
        uint4 kk[TILES][4], vv[TILES][4];
        bool ok[TILES][4];
#pragma unroll
        for (int t = 0; t < TILES; ++t)
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int j = t * 16 + it * 4 + rg;
                const int n = row0 + j;
                const int loc = __shfl(myloc, j);
                ok[t][it] = n < N;
                const bool st = n < a.static_len;
                const int64_t roff = (st ? static_cast<int64_t>(n) : static_cast<int64_t>(ok[t][it] ? loc : 0)) * 128;
                const uint16_t* kp = (st ? skh : lkh) + roff + li * 8;
                const uint16_t* vp = (st ? svh : lvh) + roff + li * 8;
                kk[t][it] = *reinterpret_cast<const uint4*>(kp);
                vv[t][it] = *reinterpret_cast<const uint4*>(vp);
            }
#pragma unroll
        for (int t = 0; t < TILES; ++t) {
            float s[4][G];
#pragma unroll
            for (int it = 0; it < 4; ++it)
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float d = row16_sum(dot8(kk[t][it], qp[g]));
                    s[it][g] = ok[t][it] ? d * a.scale_log2 : -INFINITY;
                }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float tm = fmaxf(fmaxf(s[0][g], s[1][g]), fmaxf(s[2][g], s[3][g]));
                const float mn = fmaxf(m_[g], tm);
                const float corr = wexp(m_[g], mn);
                float p[4];
#pragma unroll
                for (int it = 0; it < 4; ++it) p[it] = wexp(s[it][g], mn);   // 0 for rows past the end
                l_[g] = l_[g] * corr + ((p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    float x = acc[g][u] * corr;
#pragma unroll
                    for (int it = 0; it < 4; ++it) x = __builtin_fmaf(p[it], bf16_at(vv[t][it], u), x);
                    acc[g][u] = x;
                }
                m_[g] = mn;
            }
        }
    }
    // merge the four row groups of the wave (lanes li, li+16, li+32, li+48)
    // with the permlane swaps: first across rows 0<->1, 2<->3, then halves
#pragma unroll
    for (int step = 0; step < 2; ++step) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mo = step == 0 ? xor16(m_[g]) : xor32(m_[g]);
            const float lo = step == 0 ? xor16(l_[g]) : xor32(l_[g]);
            const float mn = fmaxf(m_[g], mo);
            const float wa = wexp(m_[g], mn), wb = wexp(mo, mn);
            l_[g] = l_[g] * wa + lo * wb;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float ao = step == 0 ? xor16(acc[g][u]) : xor32(acc[g][u]);
                acc[g][u] = acc[g][u] * wa + ao * wb;
            }
            m_[g] = mn;
        }
    }
    if (rg == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int u = 0; u < 8; ++u) s_acc[wave][g][li * 8 + u] = acc[g][u];
            if (li == 0) {
                s_ml[wave][g][0] = m_[g];
                s_ml[wave][g][1] = l_[g];
            }
        }
    }
    __syncthreads();
    // block partial (waves merged in order)
    const int64_t pbase = static_cast<int64_t>(h) * a.nsplit + split;
    for (int o = tid; o < G * 128; o += 64 * kWaves) {
        const int g = o >> 7, d = o & 127;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_ml[w][g][0]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float wt = wexp(s_ml[w][g][0], M);
            L += s_ml[w][g][1] * wt;
            A += s_acc[w][g][d] * wt;
        }
        a.part_acc[(pbase * G + g) * 128 + d] = A;
        if (d == 0) {
            a.part_ml[(pbase * G + g) * 2 + 0] = M;
            a.part_ml[(pbase * G + g) * 2 + 1] = L;
        }
    }
}

// Merge of the nsplit partials of one head for 64 outputs (query head
// g = chunk / 2, dims (chunk % 2) * 64 ..).  Each of the four waves sums a
// quarter of the splits (s = q, q + 4, ...); its first 16 loads are issued
// before wave 0 has derived the split weights, so the common case needs one
// round trip.  Quarters are added in a fixed order (deterministic).
__global__ __launch_bounds__(256) void merge_kernel(AttnParams a, int G) {
    __shared__ float s_w[kMaxSplit];
    __shared__ float s_red[4][64];
    __shared__ float s_ML[2];
    const int h = blockIdx.y, chunk = blockIdx.x;
    const int g = chunk >> 1;
    const int tid = threadIdx.x, q = tid >> 6, lane = tid & 63;
    const int o = chunk * 64 + lane;  // g * 128 + d
    const int ns = a.nsplit;
    const int64_t stride = static_cast<int64_t>(G) * 128;
    const float* pacc = a.part_acc + static_cast<int64_t>(h) * ns * stride + o;
    const float* pml = a.part_ml + (static_cast<int64_t>(h) * ns * G + g) * 2;
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int s = q + 4 * u;
        v[u] = s < ns ? pacc[s * stride] : 0.0f;
    }
    if (q == 0) {
        float M = -INFINITY;
        for (int s = lane; s < ns; s += 64) M = fmaxf(M, pml[static_cast<int64_t>(s) * G * 2]);
        M = wave_max(M);
        float L = 0.0f;
        for (int s = lane; s < ns; s += 64) {
            const float w = wexp(pml[static_cast<int64_t>(s) * G * 2], M);
            s_w[s] = w;
            L += pml[static_cast<int64_t>(s) * G * 2 + 1] * w;
        }
        L = wave_sum(L);
        if (lane == 0) {
            s_ML[0] = M;
            s_ML[1] = L;
        }
    }
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int s = q + 4 * u;
        if (s < ns) acc = __builtin_fmaf(v[u], s_w[s], acc);
    }
    for (int s0 = q + 64; s0 < ns; s0 += 64) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int s = s0 + 4 * u;
            v[u] = s < ns ? pacc[s * stride] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int s = s0 + 4 * u;
            if (s < ns) acc = __builtin_fmaf(v[u], s_w[s], acc);
        }
    }
    s_red[q][lane] = acc;
    __syncthreads();
    if (q == 0) {
        const float A = ((s_red[0][lane] + s_red[1][lane]) + s_red[2][lane]) + s_red[3][lane];
        const float L = s_ML[1];
        a.out[static_cast<int64_t>(h) * G * 128 + o] = f32_to_bf16(L > 0.0f ? A / L : 0.0f);
        if (a.lse && lane == 0 && (chunk & 1) == 0)
            a.lse[static_cast<int64_t>(h) * G + g] =
                L > 0.0f ? (s_ML[0] + log2f(L)) * 0.69314718055994530942f : -INFINITY;
    }
}

// Rows per wave: two tiles when the head has enough rows to give every CU
// about two workgroups, otherwise one.
int tiles_for(int rows, int H) {
    const int blocks_one_tile = (rows + kWaves * 16 - 1) / (kWaves * 16);
    return blocks_one_tile * H > 512 ? 2 : 1;
}

int nsplit_for(const imi_attention_args* a) {
    const int rows = a->static_len + a->max_rows;
    const int rb = kWaves * 16 * tiles_for(rows, a->kv_heads);
    return rows <= 0 ? 1 : (rows + rb - 1) / rb;
}

// Splits the workspace is sized for: any static_len up to steady_stride, so a
// workspace sized once stays valid while the steady zone grows.
int nsplit_bound(const imi_attention_args* a) {
    const int64_t srows = a->steady_stride > a->static_len ? a->steady_stride : a->static_len;
    const int rows = static_cast<int>(srows + a->max_rows);
    return rows <= 0 ? 1 : (rows + kWaves * 16 - 1) / (kWaves * 16);
}

size_t attn_workspace(const imi_attention_args* a, AttnParams* p) {
    const int nsplit = nsplit_bound(a);
    Carver cv(a->workspace);
    float* acc = cv.take<float>(static_cast<size_t>(a->kv_heads) * nsplit * a->groups * 128);
    float* ml = cv.take<float>(static_cast<size_t>(a->kv_heads) * nsplit * a->groups * 2);
    if (p) {
        p->part_acc = acc;
        p->part_ml = ml;
        p->nsplit = nsplit_for(a);
        const int rows = a->static_len + a->max_rows;
        p->rows_per_block = kWaves * 16 * tiles_for(rows, a->kv_heads);
    }
    return cv.used();
}

int attn_validate(const imi_attention_args* a, bool need_sel) {
    IMI_REQUIRE(a != nullptr, IMI_ERR_INVALID, "imi_sparse_attention: null args");
    IMI_REQUIRE(a->dim == 128, IMI_ERR_UNSUPPORTED, "imi_sparse_attention: head_dim must be 128");
    IMI_REQUIRE(a->groups == 1 || a->groups == 2 || a->groups == 4 || a->groups == 7 || a->groups == 8,
                IMI_ERR_UNSUPPORTED, "imi_sparse_attention: %d query heads per kv head unsupported", a->groups);
    IMI_REQUIRE(a->kv_heads > 0, IMI_ERR_INVALID, "imi_sparse_attention: kv_heads must be > 0");
    IMI_REQUIRE(a->query && a->out, IMI_ERR_INVALID, "imi_sparse_attention: null query/out");
    IMI_REQUIRE(a->static_len >= 0 && a->static_len <= a->steady_stride, IMI_ERR_INVALID,
                "imi_sparse_attention: static_len %d outside steady zone of %lld rows", a->static_len,
                static_cast<long long>(a->steady_stride));
    IMI_REQUIRE(a->static_len == 0 || (a->steady_keys && a->steady_values), IMI_ERR_INVALID,
                "imi_sparse_attention: null steady zone");
    IMI_REQUIRE(a->list_keys && a->list_values, IMI_ERR_INVALID, "imi_sparse_attention: null list");
    IMI_REQUIRE(a->max_rows >= 0, IMI_ERR_INVALID, "imi_sparse_attention: max_rows must be >= 0");
    if (need_sel)
        IMI_REQUIRE(a->n_rows != nullptr, IMI_ERR_INVALID, "imi_sparse_attention: null n_rows");
    IMI_REQUIRE(a->sel_cap >= 0 && a->sel_cap <= kSelCapMax, IMI_ERR_UNSUPPORTED,
                "imi_sparse_attention: sel_cap %d exceeds %d", a->sel_cap, kSelCapMax);
    IMI_REQUIRE(nsplit_bound(a) <= kMaxSplit, IMI_ERR_UNSUPPORTED,
                "imi_sparse_attention: %d rows need more than %d splits per head", a->static_len + a->max_rows,
                kMaxSplit);
    return IMI_OK;
}

template <int G>
void launch_g(const AttnParams& p, int blocks, hipStream_t stream) {
    if (p.rows_per_block == kWaves * 32)
        hipLaunchKernelGGL((attention_kernel<G, 2>), dim3(blocks), dim3(64 * kWaves), 0, stream, p);
    else
        hipLaunchKernelGGL((attention_kernel<G, 1>), dim3(blocks), dim3(64 * kWaves), 0, stream, p);
}

int attn_launch(const imi_attention_args* a, hipStream_t stream) {
    AttnParams p;
    attn_workspace(a, &p);
    p.q = a->query;
    p.sk = a->steady_keys;
    p.sv = a->steady_values;
    p.s_stride = a->steady_stride;
    p.static_len = a->static_len;
    p.lk = a->list_keys;
    p.lv = a->list_values;
    p.list_rows = a->list_rows;
    p.sel_offset = a->sel_offset;
    p.sel_prefix = a->sel_prefix;
    p.n_selected = a->n_selected;
    p.sel_cap = a->sel_cap;
    p.n_rows = a->n_rows;
    p.H = a->kv_heads;
    p.scale_log2 = a->scale * 1.44269504088896340736f;
    p.out = a->out;
    p.lse = a->out_lse;
    const int blocks = a->kv_heads * p.nsplit;
    switch (a->groups) {
        case 1: launch_g<1>(p, blocks, stream); break;
        case 2: launch_g<2>(p, blocks, stream); break;
        case 4: launch_g<4>(p, blocks, stream); break;
        case 7: launch_g<7>(p, blocks, stream); break;
        default: launch_g<8>(p, blocks, stream); break;
    }
    IMI_LAUNCH_CHECK("attention_kernel");
    hipLaunchKernelGGL(merge_kernel, dim3(2 * a->groups, a->kv_heads), dim3(256), 0, stream, p, a->groups);
    IMI_LAUNCH_CHECK("merge_kernel");
    return IMI_OK;
}

}  // namespace
}  // namespace imi

using namespace imi;

extern "C" int imi_attention_workspace_size(const imi_attention_args* a, size_t* bytes) {
    clear_error();
    int rc = attn_validate(a, false);
    if (rc) return rc;
    IMI_REQUIRE(bytes != nullptr, IMI_ERR_INVALID, "imi_attention_workspace_size: null output");
    imi_attention_args t = *a;
    t.workspace = nullptr;
    *bytes = attn_workspace(&t, nullptr);
    return IMI_OK;
}

extern "C" int imi_sparse_attention(const imi_attention_args* a, imi_stream_t stream_) {
    clear_error();
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    int rc = attn_validate(a, true);
    if (rc) return rc;
    IMI_REQUIRE(a->sel_offset && a->sel_prefix && a->n_selected, IMI_ERR_INVALID,
                "imi_sparse_attention: null selection arrays");
    size_t need;
    rc = imi_attention_workspace_size(a, &need);
    if (rc) return rc;
    IMI_REQUIRE(a->workspace && a->workspace_bytes >= need, IMI_ERR_WORKSPACE,
                "imi_sparse_attention: workspace %zu bytes < %zu required", a->workspace_bytes, need);
    return attn_launch(a, stream);
}

namespace {
struct DecodeLayout {
    int32_t *cell, *off, *cnt, *prefix, *nsel, *nrows;
    char* attn_ws;
    size_t attn_bytes;
    size_t total;
};

DecodeLayout decode_layout(const imi_decode_args* a, void* ws) {
    DecodeLayout L{};
    Carver cv(ws);
    const int H = a->sel.kv_heads, cap = a->sel.sel_cap;
    L.cell = cv.take<int32_t>(static_cast<size_t>(H) * cap);
    L.off = cv.take<int32_t>(static_cast<size_t>(H) * cap);
    L.cnt = cv.take<int32_t>(static_cast<size_t>(H) * cap);
    L.prefix = cv.take<int32_t>(static_cast<size_t>(H) * (cap + 1));
    L.nsel = cv.take<int32_t>(H);
    L.nrows = cv.take<int32_t>(H);
    imi_attention_args t = a->attn;
    t.workspace = nullptr;
    L.attn_bytes = attn_workspace(&t, nullptr);
    L.attn_ws = cv.take<char>(L.attn_bytes);
    L.total = cv.used();
    return L;
}

int decode_validate(const imi_decode_args* a) {
    IMI_REQUIRE(a != nullptr, IMI_ERR_INVALID, "imi_decode_step: null args");
    IMI_REQUIRE(a->sel.kv_heads == a->attn.kv_heads && a->sel.groups == a->attn.groups,
                IMI_ERR_INVALID, "imi_decode_step: selection and attention shapes differ");
    IMI_REQUIRE(a->attn.max_rows >= a->sel.buffer_pages * a->sel.page_size, IMI_ERR_INVALID,
                "imi_decode_step: max_rows %d < buffer_pages * page_size %d", a->attn.max_rows,
                a->sel.buffer_pages * a->sel.page_size);
    return attn_validate(&a->attn, false);
}
}  // namespace

extern "C" int imi_decode_workspace_size(const imi_decode_args* a, size_t* bytes) {
    clear_error();
    int rc = decode_validate(a);
    if (rc) return rc;
    IMI_REQUIRE(bytes != nullptr, IMI_ERR_INVALID, "imi_decode_workspace_size: null output");
    *bytes = decode_layout(a, nullptr).total;
    return IMI_OK;
}

extern "C" int imi_decode_step(const imi_decode_args* a, imi_stream_t stream_) {
    clear_error();
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    int rc = decode_validate(a);
    if (rc) return rc;
    const DecodeLayout need = decode_layout(a, nullptr);
    IMI_REQUIRE(a->attn.workspace && a->attn.workspace_bytes >= need.total, IMI_ERR_WORKSPACE,
                "imi_decode_step: workspace %zu bytes < %zu required", a->attn.workspace_bytes, need.total);
    const DecodeLayout L = decode_layout(a, a->attn.workspace);
    const int phases = (a->phases & 3) == 0 ? 3 : (a->phases & 3);
    imi_select_args s = a->sel;
    if (!s.sel_cell) s.sel_cell = L.cell;
    if (!s.sel_offset) s.sel_offset = L.off;
    if (!s.sel_count) s.sel_count = L.cnt;
    if (!s.sel_prefix) s.sel_prefix = L.prefix;
    if (!s.n_selected) s.n_selected = L.nsel;
    if (!s.n_rows) s.n_rows = L.nrows;
    if (phases & 1) {
        rc = select_launch(&s, stream);
        if (rc) return rc;
    } else {
        int64_t nc;
        int km;
        rc = select_validate(&s, nc, km);
        if (rc) return rc;
    }
    if (!(phases & 2)) return IMI_OK;
    imi_attention_args t = a->attn;
    t.sel_offset = s.sel_offset;
    t.sel_count = s.sel_count;
    t.sel_prefix = s.sel_prefix;
    t.n_selected = s.n_selected;
    t.n_rows = s.n_rows;
    t.sel_cap = s.sel_cap;
    t.workspace = L.attn_ws;
    t.workspace_bytes = L.attn_bytes;
    return attn_launch(&t, stream);
}
