// Fused gather + GQA sparse decode attention on gfx950 (HBM-bound).
//
// Reference: the execution-buffer gather concat_gather_copy
// (include/copy_kernel.cuh:220-335, launched by cuda/gather_copy.cu:100-213:
// rows = [static_len steady rows | miss pages | hit pages]) followed by the
// unvendored weighted_flash_decoding (retrieval.py:439-447).  Here the rows
// are read in place: the steady zone for the first static_len rows, then the
// CSR list rows of the selected cells (row_loc table written by the
// selection kernel) -- no execution buffer.
//
// Grid: H * nsplit workgroups of 4 waves, block b -> head b % H, split b / H,
// so with 8 KV heads each head's splits run on one XCD (dispatch is round
// robin over the 8 XCDs) and its partials stay in that XCD's L2.  Each wave
// owns 32 consecutive rows; a row is read by 16 lanes x 16 bytes (fully
// coalesced 1 KiB per wave instruction for 4 rows).  q.k uses v_dot2_f32_bf16
// and a 16-lane DPP reduction; softmax is online in base 2 with fp32 state;
// the 16 (wave, row-group) states merge in LDS into one partial per block.
// The last block of each head (device-scope counter) merges the nsplit
// partials in split order (deterministic) and writes bf16 output and LSE.
#include "imi_common.hpp"

namespace imi {

int select_launch(const imi_select_args* a, int32_t* row_loc, int max_rows, hipStream_t stream);
int select_validate(const imi_select_args* a, int64_t& ncells, int& kmax);

namespace {

constexpr int kWaves = 8;            // waves per workgroup (512 threads)
constexpr int kMaxSplitG = 8192;     // splits * groups the final merge can index

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
    const int32_t* row_loc;  // [H][max_rows]
    int max_rows;
    const int32_t* n_rows;   // [H]
    int H, nsplit;
    int rows_per_block;
    float scale_log2;        // scale * log2(e)
    float* part_acc;         // [H][nsplit][G][128]
    float* part_ml;          // [H][nsplit][G][2]
    int32_t* counter;        // [H]
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

// Agent-scope relaxed atomic store / load: encoded with the coherence bit, so
// other XCDs see the value without an L2 write-back / invalidate.
__device__ __forceinline__ void coherent_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// s_waitcnt vmcnt(0): this thread's stores have been acknowledged.
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Weight exp2(m - M) of a state with running max m inside a merge whose max
// is M; an empty state (m = -inf) weighs 0 even when M is -inf too.
__device__ __forceinline__ float wexp(float m, float M) { return m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M); }

// One workgroup = 8 waves over rows [split * rows_per_block, +rows_per_block)
// of head h; each wave owns TILES * 16 consecutive rows, read as tiles of 4
// rows x 4 iterations (16 lanes x 16 bytes per row).
template <int G, int TILES>
__global__ __launch_bounds__(512) void attention_kernel(AttnParams a) {
    constexpr int RW = TILES * 16;
    __shared__ float s_acc[kWaves][G][128];
    __shared__ float s_ml[kWaves][G][2];
    __shared__ float s_w[kMaxSplitG];
    __shared__ float s_ML[G][2];
    __shared__ float s_red[4][G * 128];
    __shared__ int s_last;

    const int b = blockIdx.x;
    const int h = b % a.H;
    const int split = b / a.H;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int rg = lane >> 4, li = lane & 15;
    const int N = a.static_len + a.n_rows[h];
    const int row0 = split * a.rows_per_block + wave * RW;

    // q and the row locations of this wave, loaded together up front
    uint32_t qp[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const uint4 v = *reinterpret_cast<const uint4*>(a.q + (static_cast<int64_t>(h) * G + g) * 128 + li * 8);
        qp[g][0] = v.x; qp[g][1] = v.y; qp[g][2] = v.z; qp[g][3] = v.w;
    }
    int myloc = 0;
    {
        const int n = row0 + lane;
        if (lane < RW && n < N && n >= a.static_len)
            myloc = a.row_loc[static_cast<int64_t>(h) * a.max_rows + (n - a.static_len)];
    }
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
#pragma unroll
    for (int o = 16; o <= 32; o <<= 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mo = __shfl_xor(m_[g], o);
            const float lo = __shfl_xor(l_[g], o);
            const float mn = fmaxf(m_[g], mo);
            const float wa = wexp(m_[g], mn), wb = wexp(mo, mn);
            l_[g] = l_[g] * wa + lo * wb;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float ao = __shfl_xor(acc[g][u], o);
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
    // block partial (waves merged in order), published with agent-coherent
    // stores (write-through past the XCD's L2) instead of a device fence
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
        coherent_store(a.part_acc + (pbase * G + g) * 128 + d, A);
        if (d == 0) {
            coherent_store(a.part_ml + (pbase * G + g) * 2 + 0, M);
            coherent_store(a.part_ml + (pbase * G + g) * 2 + 1, L);
        }
    }
    wait_stores();
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(&a.counter[h], 1) == a.nsplit - 1;
    __syncthreads();
    if (!s_last) return;

    // ---- final merge of head h's nsplit partials (deterministic order) ----
    const float* pml = a.part_ml + static_cast<int64_t>(h) * a.nsplit * G * 2;
    for (int i = tid; i < a.nsplit * G; i += 64 * kWaves) s_w[i] = coherent_load(pml + 2 * i);
    __syncthreads();
    if (wave < G) {
        const int g = wave;
        float M = -INFINITY;
        for (int s = lane; s < a.nsplit; s += 64) M = fmaxf(M, s_w[s * G + g]);
        M = wave_max(M);
        float L = 0.0f;
        for (int s = lane; s < a.nsplit; s += 64) L += coherent_load(pml + (s * G + g) * 2 + 1) * wexp(s_w[s * G + g], M);
        L = wave_sum(L);
        if (lane == 0) {
            s_ML[g][0] = M;
            s_ML[g][1] = L;
        }
    }
    __syncthreads();
    for (int i = tid; i < a.nsplit * G; i += 64 * kWaves) s_w[i] = wexp(s_w[i], s_ML[i % G][0]);
    __syncthreads();
    // thread -> 4 consecutive outputs x one quarter of the splits; loads of
    // 4 splits are issued together
    const float* pacc = a.part_acc + static_cast<int64_t>(h) * a.nsplit * G * 128;
    const int o4 = (tid & 127) * 4;  // output index (g * 128 + d), 4 at a time
    const int quarter = tid >> 7;    // 0..3
    for (int o = o4; o < G * 128; o += 512) {
        const int g = o >> 7;
        float A[4] = {0.f, 0.f, 0.f, 0.f};
        for (int s0 = quarter; s0 < a.nsplit; s0 += 16) {
            float v[4][4], w[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int s = s0 + 4 * u;
                const bool in = s < a.nsplit;
                w[u] = in ? s_w[s * G + g] : 0.0f;
#pragma unroll
                for (int x = 0; x < 4; ++x)
                    v[u][x] = in ? coherent_load(pacc + static_cast<int64_t>(s) * G * 128 + o + x) : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int x = 0; x < 4; ++x) A[x] = __builtin_fmaf(v[u][x], w[u], A[x]);
        }
#pragma unroll
        for (int x = 0; x < 4; ++x) s_red[quarter][o + x] = A[x];
    }
    __syncthreads();
    for (int o = tid; o < G * 128; o += 64 * kWaves) {
        const int g = o >> 7;
        const float A = ((s_red[0][o] + s_red[1][o]) + s_red[2][o]) + s_red[3][o];
        const float L = s_ML[g][1];
        a.out[static_cast<int64_t>(h) * G * 128 + o] = f32_to_bf16(L > 0.0f ? A / L : 0.0f);
        if (a.lse && (o & 127) == 0)
            a.lse[static_cast<int64_t>(h) * G + g] =
                L > 0.0f ? (s_ML[g][0] + log2f(L)) * 0.69314718055994530942f : -INFINITY;
    }
    if (tid == 0) a.counter[h] = 0;
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
    int32_t* cnt = cv.take<int32_t>(a->kv_heads);
    if (p) {
        p->part_acc = acc;
        p->part_ml = ml;
        p->counter = cnt;
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
    IMI_REQUIRE(nsplit_bound(a) * a->groups <= kMaxSplitG, IMI_ERR_UNSUPPORTED,
                "imi_sparse_attention: %d rows x %d groups exceed the split table", a->static_len + a->max_rows,
                a->groups);
    return IMI_OK;
}

template <int G>
void launch_g(const AttnParams& p, int blocks, hipStream_t stream) {
    if (p.rows_per_block == kWaves * 32)
        hipLaunchKernelGGL((attention_kernel<G, 2>), dim3(blocks), dim3(64 * kWaves), 0, stream, p);
    else
        hipLaunchKernelGGL((attention_kernel<G, 1>), dim3(blocks), dim3(64 * kWaves), 0, stream, p);
}

int attn_launch(const imi_attention_args* a, const int32_t* row_loc, hipStream_t stream) {
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
    p.row_loc = row_loc;
    p.max_rows = a->max_rows;
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
    return IMI_OK;
}

// Row-location table for a caller-supplied selection (imi_sparse_attention
// without imi_decode_step): one wave per selected cell.
__global__ __launch_bounds__(256) void expand_rows_kernel(const int32_t* sel_offset, const int32_t* sel_count,
                                                          const int32_t* sel_prefix, const int32_t* n_selected,
                                                          int sel_cap, int32_t* row_loc, int max_rows) {
    const int h = blockIdx.y;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= n_selected[h]) return;
    const int o = sel_offset[static_cast<int64_t>(h) * sel_cap + r];
    const int c = sel_count[static_cast<int64_t>(h) * sel_cap + r];
    const int base = sel_prefix[static_cast<int64_t>(h) * (sel_cap + 1) + r];
    for (int i = lane_id(); i < c; i += 64)
        if (base + i < max_rows) row_loc[static_cast<int64_t>(h) * max_rows + base + i] = o + i;
}

}  // namespace
}  // namespace imi

using namespace imi;

namespace {
size_t rowloc_bytes(const imi_attention_args* a) {
    return align_up(static_cast<size_t>(a->kv_heads) * (a->max_rows > 0 ? a->max_rows : 1) * sizeof(int32_t), 256);
}
}  // namespace

extern "C" int imi_attention_workspace_size(const imi_attention_args* a, size_t* bytes) {
    clear_error();
    int rc = attn_validate(a, false);
    if (rc) return rc;
    IMI_REQUIRE(bytes != nullptr, IMI_ERR_INVALID, "imi_attention_workspace_size: null output");
    imi_attention_args t = *a;
    t.workspace = nullptr;
    *bytes = rowloc_bytes(a) + attn_workspace(&t, nullptr);
    return IMI_OK;
}

extern "C" int imi_sparse_attention(const imi_attention_args* a, imi_stream_t stream_) {
    clear_error();
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    int rc = attn_validate(a, true);
    if (rc) return rc;
    IMI_REQUIRE(a->sel_offset && a->sel_count && a->sel_prefix && a->n_selected, IMI_ERR_INVALID,
                "imi_sparse_attention: null selection arrays");
    size_t need;
    rc = imi_attention_workspace_size(a, &need);
    if (rc) return rc;
    IMI_REQUIRE(a->workspace && a->workspace_bytes >= need, IMI_ERR_WORKSPACE,
                "imi_sparse_attention: workspace %zu bytes < %zu required", a->workspace_bytes, need);
    int32_t* row_loc = static_cast<int32_t*>(a->workspace);
    imi_attention_args t = *a;
    t.workspace = static_cast<char*>(a->workspace) + rowloc_bytes(a);
    if (a->sel_cap > 0) {
        hipLaunchKernelGGL(expand_rows_kernel, dim3((a->sel_cap + 3) / 4, a->kv_heads), dim3(256), 0, stream,
                           a->sel_offset, a->sel_count, a->sel_prefix, a->n_selected, a->sel_cap, row_loc,
                           a->max_rows);
        IMI_LAUNCH_CHECK("expand_rows_kernel");
    }
    return attn_launch(&t, row_loc, stream);
}

namespace {
struct DecodeLayout {
    int32_t *cell, *off, *cnt, *prefix, *nsel, *nrows, *row_loc;
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
    L.row_loc = cv.take<int32_t>(static_cast<size_t>(H) * (a->attn.max_rows > 0 ? a->attn.max_rows : 1));
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
        rc = select_launch(&s, L.row_loc, a->attn.max_rows, stream);
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
    return attn_launch(&t, L.row_loc, stream);
}
