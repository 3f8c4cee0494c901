// Fused gather + GQA sparse decode attention on gfx950 (HBM-bound).
//
// Reference: the execution-buffer gather concat_gather_copy
// (include/copy_kernel.cuh:220-335, launched by cuda/gather_copy.cu:100-213:
// rows = [static_len steady rows | miss pages | hit pages]) followed by the
// unvendored weighted_flash_decoding (retrieval.py:439-447).  Here the rows
// are read in place: the steady zone for the first static_len rows, then the
// CSR list rows of the selected cells (each workgroup stages the head's
// selection in LDS and each wave maps its rows to list rows with two ballot
// rounds and a flag count) -- no execution buffer.
//
// Grid: H * nsplit workgroups of 4 waves; workgroup b takes split b / H of
// head (b + b / H) % H, so consecutive workgroups (which the dispatcher deals
// round robin to the 8 XCDs) rotate over the heads and every XCD gets a
// share of every head's rows.  A wave owns NT tiles of 16 consecutive rows
// and keeps two tiles in flight ahead of the one it computes.  Rows are read
// whole (16 lanes x 16 bytes per 256-byte row) and staged through LDS, which
// hands K back in the MFMA operand layout and V transposed.
//
// Per tile, on the matrix cores:
//   S = K Q^T   4 x v_mfma_f32_16x16x32_bf16: A = the K tile read back from
//               LDS (lane -> token lane % 16, 8 dims), B = Q with column n holding
//               query n % G; lane l gets S[token 4(l/16)+i][query (l%16)%G].
//   O += P V    8 x v_mfma_f32_16x16x16_bf16: A = P, which is exactly the S
//               layout above (row = query slot, k = token) after exp2 and a
//               bf16 pack; B = V^T, read from a per-wave LDS copy of the V
//               tile with ds_read_b64_tr_b16 (4 tokens x 1 dim per lane).
// Softmax is online in base 2 with fp32 state per query slot; the rescale
// of O is skipped when no running max moved.  The waves of a workgroup merge
// in LDS into one partial (plain stores); a second kernel merges each
// head's partials in split order (deterministic) and writes the bf16 output
// and the LSE: the kernel boundary makes the partials visible across XCDs
// without any device-scope fence.
#include <mutex>

#include "imi_common.hpp"

namespace imi {

int select_launch(const imi_select_args* a, hipStream_t stream);
int select_validate(const imi_select_args* a, int64_t& ncells, int& kmax);
size_t select4_workspace_size(const imi_select_args* a);
size_t select4_zero_bytes();

namespace {

constexpr int kWaves = 4;            // waves per workgroup (256 threads)
constexpr int kMaxSplit = 4096;      // splits per head the merge kernel handles
constexpr int kSelCapMax = 2048;     // selected cells per head the gather indexes
constexpr int kDeltaMax = 1024;      // delta rows per head (the delta ring)
constexpr int kVStride = 144;        // u16 per LDS row of a wave's V tile (288 B)

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

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
    const int32_t* delta_rows;  // [H][delta_cap] steady rows after the selected rows, or null
    const int32_t* n_delta;     // [H]
    int delta_cap;
    int H, nsplit;
    int rows_per_block;
    float scale_log2;        // scale * log2(e)
    float* part_acc;         // [H][nsplit][G][128]
    float* part_ml;          // [H][nsplit][G][2]
    uint16_t* out;           // [H*G][128]
    float* lse;              // [H*G] or null
};

// Weight exp2(m - M) of a state with running max m inside a merge whose max
// is M; an empty state (m = -inf) weighs 0 even when M is -inf too.
__device__ __forceinline__ float wexp(float m, float M) { return m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M); }

// Orders this wave's LDS accesses around a hand-off between its own lanes
// (compiler-only: a wave executes its LDS instructions in order, but without
// the fences the compiler may reorder or forward them as if each lane ran
// alone).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Number of set bits of the 128-bit mask (lo, hi) at positions 0..i.
__device__ __forceinline__ int popc_upto(uint64_t lo, uint64_t hi, int i) {
    if (i < 64) return __builtin_popcountll(lo & (~0ull >> (63 - i)));
    return __builtin_popcountll(lo) + __builtin_popcountll(hi & (~0ull >> (127 - i)));
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

// One workgroup = 4 waves over rows [split * rows_per_block, +rows_per_block)
// of its head; the workgroup writes one partial (max, sum, unnormalised
// output) with plain stores and merge_kernel combines the partials after the
// kernel boundary.  Workgroups past the end of their head write nothing.
// DELTA: rows appended after the selected rows (a separate instantiation).
template <int G, int NT, bool DELTA>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2))) void attention_kernel(AttnParams a) {
    constexpr int RW = NT * 16;                       // rows per wave
    constexpr int NR = (RW + 63) / 64;                // row locations per lane
    static_assert(NR <= 2, "the row lookup covers windows of at most 128 rows");
    constexpr int SU = (kSelCapMax + 1 + 64 * kWaves - 1) / (64 * kWaves);
    constexpr int DU = kDeltaMax / (64 * kWaves);
    __shared__ float s_acc[kWaves][G][128];
    __shared__ float s_ml[kWaves][G][2];
    __shared__ int s_pre[kSelCapMax + 1];
    __shared__ int s_off[kSelCapMax];
    __shared__ int s_drow[DELTA ? kDeltaMax : 1];
    __shared__ int s_flag[kWaves][NR * 64];
    __shared__ __attribute__((aligned(16))) uint16_t s_v[kWaves][16 * kVStride];
    __shared__ __attribute__((aligned(16))) uint16_t s_k[kWaves][16 * kVStride];

    const int b = blockIdx.x;
    const int split = b / a.H;
    const int h = (b % a.H + split) % a.H;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lg = lane >> 4, ln = lane & 15;
    const int row0 = split * a.rows_per_block + wave * RW;

    // One round trip for everything the gather needs: q (as the MFMA B
    // operand: column ln = query ln % G, dims 32c + 8lg..), the row and cell
    // counts, and the head's selection (row prefix and CSR offset per cell).
    u32x4_t qb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        qb[c] = *reinterpret_cast<const u32x4_t*>(a.q + (static_cast<int64_t>(h) * G + ln % G) * 128 + c * 32 + lg * 8);
    const int nrows = a.n_rows[h];
    const int m = a.n_selected[h];
    const int nd = DELTA ? min(max(a.n_delta[h], 0), a.delta_cap) : 0;
    {
        const int32_t* pre = a.sel_prefix + static_cast<int64_t>(h) * (a.sel_cap + 1);
        const int32_t* off = a.sel_offset + static_cast<int64_t>(h) * a.sel_cap;
        int pv[SU], ov[SU];
#pragma unroll
        for (int u = 0; u < SU; ++u) {
            const int i = tid + u * 64 * kWaves;
            pv[u] = i <= a.sel_cap ? pre[i] : 0;
            ov[u] = i < a.sel_cap ? off[i] : 0;
        }
        int dv[DU];
#pragma unroll
        for (int u = 0; u < DU; ++u) {
            const int i = tid + u * 64 * kWaves;
            dv[u] = DELTA && i < a.delta_cap ? a.delta_rows[static_cast<int64_t>(h) * a.delta_cap + i] : 0;
        }
#pragma unroll
        for (int u = 0; u < SU; ++u) {
            const int i = tid + u * 64 * kWaves;
            if (i <= a.sel_cap) s_pre[i] = pv[u];
            if (i < a.sel_cap) s_off[i] = ov[u];
        }
        if (DELTA) {
#pragma unroll
            for (int u = 0; u < DU; ++u) s_drow[tid + u * 64 * kWaves] = dv[u];
        }
    }
    __syncthreads();
    // rows: [static_len steady rows | nrows list rows | nd delta rows (steady)]
    const int N = a.static_len + nrows + nd;
    if (split * a.rows_per_block >= N) return;   // the merge ignores this split

    // List row of window row i (rows row0 + i, i = lane + 64r): the wave
    // finds the cell c0 that holds its first list row j0 (two ballot rounds
    // over the staged prefix), flags the window offsets where the following
    // cells start, and counts the flags up to each row.  Selected cells hold
    // at least one row, so their starts are distinct; locations are clamped
    // to the list.  A delta row gets -1 - its steady row (clamped to the
    // steady zone).
    int loc[NR];
    {
        const int j0 = max(row0 - a.static_len, 0);
        int c0 = 0;
        if (m > 1) {
            const int step = (m + 63) >> 6;   // <= 32 cells per lane sample
            const int cs = lane * step;
            const uint64_t b1 = __builtin_amdgcn_ballot_w64(cs < m && s_pre[cs] <= j0);
            const int base = (63 - __builtin_clzll(b1 | 1ull)) * step;
            const int cc = base + lane;
            const uint64_t b2 = __builtin_amdgcn_ballot_w64(lane < step && cc < m && s_pre[cc] <= j0);
            c0 = base + (63 - __builtin_clzll(b2 | 1ull));
        }
        int* fl = s_flag[wave];
#pragma unroll
        for (int r = 0; r < NR; ++r) fl[lane + 64 * r] = 0;
        wave_lds_sync();
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int c = c0 + 1 + lane + 64 * r;
            if (c < m) {
                const int o = s_pre[c] - j0;
                if (o > 0 && o < NR * 64) fl[o] = 1;
            }
        }
        wave_lds_sync();
        uint64_t fm[2] = {0ull, 0ull};
#pragma unroll
        for (int r = 0; r < NR; ++r) fm[r] = __builtin_amdgcn_ballot_w64(fl[lane + 64 * r] != 0);
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int j = row0 + lane + 64 * r - a.static_len;
            int l = 0;
            if (j >= 0 && j < nrows) {
                const int c = c0 + popc_upto(fm[0], fm[1], j - j0);
                l = s_off[c] + (j - s_pre[c]);
                l = min(max(l, 0), static_cast<int>(a.list_rows) - 1);
            } else if (DELTA && j >= nrows && j < nrows + nd) {
                l = -1 - min(max(s_drow[j - nrows], 0), static_cast<int>(a.s_stride) - 1);
            }
            loc[r] = l;
        }
    }

    const uint16_t* skh = a.sk + static_cast<int64_t>(h) * a.s_stride * 128;
    const uint16_t* svh = a.sv + static_cast<int64_t>(h) * a.s_stride * 128;
    const uint16_t* lkh = a.lk + static_cast<int64_t>(h) * a.list_rows * 128;
    const uint16_t* lvh = a.lv + static_cast<int64_t>(h) * a.list_rows * 128;
    f32x4_t acc[8];   // acc[d][r] = O[query slot 4lg + r][dim 16d + ln]
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[d] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m_own = -INFINITY, l_own = 0.0f;   // softmax state of query slot ln
    uint16_t* sv = s_v[wave];
    uint16_t* sk = s_k[wave];

    if (row0 < N) {
        // Tile t, load it: rows t*16 + 4it + rg, 16 lanes x 16 bytes per row
        // (whole 256-byte rows per 16 lanes).  Rows past N read list row 0
        // (in bounds) and are masked below.
        const int rg = lane >> 4, li = lane & 15;
        u32x4_t kb[2][4], vb[2][4];
        auto load = [&](int t, int slot) {
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int jt = t * 16 + it * 4 + rg;
                const int n = row0 + jt;
                const int lr = __shfl(loc[(t * 16) >> 6], jt & 63);
                const bool st = n < a.static_len;
                const bool dl = DELTA && !st && n < N && lr < 0;   // delta row: steady row -1 - lr
                const int64_t roff =
                    (st ? static_cast<int64_t>(n) : static_cast<int64_t>(dl ? -1 - lr : (n < N ? lr : 0))) * 128;
                kb[slot][it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>((st || dl ? skh : lkh) + roff + li * 8));
                vb[slot][it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>((st || dl ? svh : lvh) + roff + li * 8));
            }
        };
        load(0, 0);
        if (NT > 1) load(1, 1);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int slot = t & 1;
            // K and V tiles -> LDS, row-major [token][dim]; K comes back in
            // the MFMA A layout (lane -> token ln, dims 32c + 8lg)
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                *reinterpret_cast<u32x4_t*>(sv + (4 * it + rg) * kVStride + li * 8) = vb[slot][it];
                *reinterpret_cast<u32x4_t*>(sk + (4 * it + rg) * kVStride + li * 8) = kb[slot][it];
            }
            wave_lds_sync();
            u32x4_t ka[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) ka[c] = *reinterpret_cast<const u32x4_t*>(sk + ln * kVStride + c * 32 + lg * 8);
            f32x4_t s4 = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < 4; ++c)
                s4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ka[c]),
                                                             __builtin_bit_cast(bf16x8_t, qb[c]), s4, 0, 0, 0);
            if (t + 2 < NT) load(t + 2, slot);
            float s[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                s[i] = (row0 + t * 16 + 4 * lg + i < N) ? s4[i] * a.scale_log2 : -INFINITY;
            float tm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
            tm = fmaxf(tm, xor16(tm));
            tm = fmaxf(tm, xor32(tm));
            const float mn = fmaxf(m_own, tm);
            const float corr = wexp(m_own, mn);
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = wexp(s[i], mn);   // 0 for masked rows
            l_own = l_own * corr + ((p[0] + p[1]) + (p[2] + p[3]));
            m_own = mn;
            if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
                // O row 4lg + r belongs to query slot 4lg + r: its factor sits
                // in lane 16lg + 4lg + r (any lane of that slot would do).
                float cr[4];
                if (4 % G == 0) {
                    cr[0] = dpp_f32<0x00>(corr);
                    cr[1] = dpp_f32<0x55>(corr);
                    cr[2] = dpp_f32<0xAA>(corr);
                    cr[3] = dpp_f32<0xFF>(corr);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) cr[r] = __shfl(corr, 16 * lg + 4 * lg + r);
                }
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                    acc[d][0] *= cr[0];
                    acc[d][1] *= cr[1];
                    acc[d][2] *= cr[2];
                    acc[d][3] *= cr[3];
                }
            }
            u32x2_t pa;
            pa.x = pack_bf16(p[0], p[1]);
            pa.y = pack_bf16(p[2], p[3]);
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                // lane (lg, ln) gets V[token 4lg + e][dim 16d + ln], e = 0..3
                const s16x4_t vt = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4_t*)(sv + (4 * lg + (ln >> 2)) * kVStride + d * 16 + 4 * (ln & 3)));
                acc[d] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, pa), vt, acc[d], 0,
                                                                   0, 0);
            }
            wave_lds_sync();
        }
    }
    // sum over the four lane groups (different tokens, shared max)
    l_own += xor16(l_own);
    l_own += xor32(l_own);
    // query g: O row g (lane group g / 4, register g % 4), state of slot g
#pragma unroll
    for (int g = 0; g < G; ++g)
        if (lg == g / 4) {
#pragma unroll
            for (int d = 0; d < 8; ++d) s_acc[wave][g][d * 16 + ln] = acc[d][g % 4];
        }
    if (lg == 0 && ln < G) {
        s_ml[wave][ln][0] = m_own;
        s_ml[wave][ln][1] = l_own;
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

// Merge of the partials of one head for 64 outputs (query head
// g = chunk / 2, dims (chunk % 2) * 64 ..).  Only splits that hold rows of
// the head (ceil((static_len + n_rows) / rows_per_block)) take part.  Every
// load of the first 64 splits (partial sums, and the max / sum pairs that
// wave 0 turns into split weights) is issued before the row count is known,
// so the common case needs one round trip.  Each of the four waves sums a
// quarter of the splits (s = q, q + 4, ...); quarters are added in a fixed
// order (deterministic).
__global__ __launch_bounds__(256) void merge_kernel(AttnParams a, int G) {
    __shared__ float s_w[kMaxSplit];
    __shared__ float s_red[4][64];
    __shared__ float s_ML[2];
    const int h = blockIdx.y, chunk = blockIdx.x;
    const int g = chunk >> 1;
    const int tid = threadIdx.x, q = tid >> 6, lane = tid & 63;
    const int o = chunk * 64 + lane;  // g * 128 + d
    const int nsm = a.nsplit;
    const int64_t stride = static_cast<int64_t>(G) * 128;
    const float* pacc = a.part_acc + static_cast<int64_t>(h) * nsm * stride + o;
    const float* pml = a.part_ml + (static_cast<int64_t>(h) * nsm * G + g) * 2;
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int s = q + 4 * u;
        v[u] = s < nsm ? pacc[s * stride] : 0.0f;
    }
    float pm = -INFINITY, pl = 0.0f;
    if (q == 0 && lane < nsm) {
        pm = pml[static_cast<int64_t>(lane) * G * 2];
        pl = pml[static_cast<int64_t>(lane) * G * 2 + 1];
    }
    const int rows = a.static_len + a.n_rows[h] + (a.delta_rows ? min(max(a.n_delta[h], 0), a.delta_cap) : 0);
    const int ns = min(nsm, (rows + a.rows_per_block - 1) / a.rows_per_block);
    if (q == 0) {
        float M = lane < ns ? pm : -INFINITY;
        for (int s = lane + 64; s < ns; s += 64) M = fmaxf(M, pml[static_cast<int64_t>(s) * G * 2]);
        M = wave_max(M);
        float w = lane < ns ? wexp(pm, M) : 0.0f;
        if (lane < nsm) s_w[lane] = w;
        float L = pl * w;
        for (int s = lane + 64; s < ns; s += 64) {
            const float ws = wexp(pml[static_cast<int64_t>(s) * G * 2], M);
            s_w[s] = ws;
            L += pml[static_cast<int64_t>(s) * G * 2 + 1] * ws;
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

// Rows the workspace and the tile size are fixed for: any static_len up to
// steady_stride, so one workspace (and one captured launch shape) stays valid
// while the steady zone grows.
int64_t rows_bound(const imi_attention_args* a) {
    const int64_t srows = a->steady_stride > a->static_len ? a->steady_stride : a->static_len;
    return srows + a->max_rows;
}

// Tiles per wave: the fewest (1..8) whose grid still fits on the CUs in one
// round, so that every CU streams and each workgroup's share is as short as
// possible (at 128k, H = 8: 7 tiles, 240 workgroups, 15.7 us vs 15.9 us with
// 8 tiles and 208 workgroups).  When no grid fits, the one (4..8 tiles, so
// that each wave's ramp stays amortised) whose busiest CU streams the fewest
// rows: workgroups per CU x rows per workgroup.
int tiles_per_wave(const imi_attention_args* a) {
    const int64_t rows = rows_bound(a);
    const int64_t cus = device_cus();
    for (int nt = 1; nt < 8; ++nt) {
        const int64_t rpb = 64 * nt;
        if (a->kv_heads * ((rows + rpb - 1) / rpb) <= cus) return nt;
    }
    int best = 8;
    int64_t best_load = INT64_MAX;
    for (int nt = 8; nt >= 4; --nt) {
        const int64_t rpb = 64 * nt;
        const int64_t wgs = a->kv_heads * ((rows + rpb - 1) / rpb);
        const int64_t load = (wgs + cus - 1) / cus * rpb;
        if (load < best_load) {
            best_load = load;
            best = nt;
        }
    }
    return best;
}

int nsplit_bound(const imi_attention_args* a) {
    const int64_t rpb = 64 * tiles_per_wave(a);
    const int64_t rows = rows_bound(a);
    return rows <= 0 ? 1 : static_cast<int>((rows + rpb - 1) / rpb);
}

size_t attn_workspace(const imi_attention_args* a, AttnParams* p) {
    const int nsplit = nsplit_bound(a);
    Carver cv(a->workspace);
    float* acc = cv.take<float>(static_cast<size_t>(a->kv_heads) * nsplit * a->groups * 128);
    float* ml = cv.take<float>(static_cast<size_t>(a->kv_heads) * nsplit * a->groups * 2);
    if (p) {
        p->part_acc = acc;
        p->part_ml = ml;
        p->nsplit = nsplit;
        p->rows_per_block = 64 * tiles_per_wave(a);
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
    if (a->delta_rows) {
        IMI_REQUIRE(a->delta_cap > 0 && a->delta_cap <= kDeltaMax, IMI_ERR_UNSUPPORTED,
                    "imi_sparse_attention: delta_cap %d outside [1, %d]", a->delta_cap, kDeltaMax);
        IMI_REQUIRE(a->steady_keys && a->steady_values && a->steady_stride > 0, IMI_ERR_INVALID,
                    "imi_sparse_attention: delta rows need the steady zone");
        IMI_REQUIRE(a->max_rows >= a->delta_cap, IMI_ERR_INVALID,
                    "imi_sparse_attention: max_rows %d must cover the %d delta rows", a->max_rows, a->delta_cap);
        if (need_sel)
            IMI_REQUIRE(a->n_delta != nullptr, IMI_ERR_INVALID, "imi_sparse_attention: null n_delta");
    }
    IMI_REQUIRE(a->sel_cap >= 0 && a->sel_cap <= kSelCapMax, IMI_ERR_UNSUPPORTED,
                "imi_sparse_attention: sel_cap %d exceeds %d", a->sel_cap, kSelCapMax);
    IMI_REQUIRE(nsplit_bound(a) <= kMaxSplit, IMI_ERR_UNSUPPORTED,
                "imi_sparse_attention: %d rows need more than %d splits per head", a->static_len + a->max_rows,
                kMaxSplit);
    return IMI_OK;
}

template <int G, bool DELTA>
void launch_gd(const AttnParams& p, int blocks, hipStream_t stream) {
#define IMI_ATT_CASE(N) \
    case N: hipLaunchKernelGGL((attention_kernel<G, N, DELTA>), dim3(blocks), dim3(64 * kWaves), 0, stream, p); break;
    switch (p.rows_per_block / 64) {
        IMI_ATT_CASE(8)
        IMI_ATT_CASE(7)
        IMI_ATT_CASE(6)
        IMI_ATT_CASE(5)
        IMI_ATT_CASE(4)
        IMI_ATT_CASE(3)
        IMI_ATT_CASE(2)
        default: hipLaunchKernelGGL((attention_kernel<G, 1, DELTA>), dim3(blocks), dim3(64 * kWaves), 0, stream, p); break;
    }
#undef IMI_ATT_CASE
}

template <int G>
void launch_g(const AttnParams& p, int blocks, hipStream_t stream) {
    if (p.delta_rows)
        launch_gd<G, true>(p, blocks, stream);
    else
        launch_gd<G, false>(p, blocks, stream);
}

// kernels: bit 0 the split pass, bit 1 the merge (which reads the partials
// the last split pass left in the workspace).
int attn_launch(const imi_attention_args* a, hipStream_t stream, int kernels = 3) {
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
    p.delta_rows = a->delta_rows;
    p.n_delta = a->n_delta;
    p.delta_cap = a->delta_cap;
    p.H = a->kv_heads;
    p.scale_log2 = a->scale * 1.44269504088896340736f;
    p.out = a->out;
    p.lse = a->out_lse;
    const int64_t rows = static_cast<int64_t>(a->static_len) + a->max_rows;
    const int splits = rows <= 0 ? 1 : static_cast<int>((rows + p.rows_per_block - 1) / p.rows_per_block);
    const int blocks = a->kv_heads * splits;
    if (kernels & 1) {
        switch (a->groups) {
            case 1: launch_g<1>(p, blocks, stream); break;
            case 2: launch_g<2>(p, blocks, stream); break;
            case 4: launch_g<4>(p, blocks, stream); break;
            case 7: launch_g<7>(p, blocks, stream); break;
            default: launch_g<8>(p, blocks, stream); break;
        }
        IMI_LAUNCH_CHECK("attention_kernel");
    }
    if (kernels & 2) {
        hipLaunchKernelGGL(merge_kernel, dim3(2 * a->groups, a->kv_heads), dim3(256), 0, stream, p, a->groups);
        IMI_LAUNCH_CHECK("merge_kernel");
    }
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
    int32_t *drows, *ndelta;   // delta append outputs (ring_cap > 0)
    char* sel_ws;            // 4-way selection scratch (empty for 2-way)
    size_t sel_bytes;
    char* attn_ws;
    size_t attn_bytes;
    char* zero_at;           // the words the kernels expect zero at the start of a call
    size_t zero_bytes;
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
    const int rc = a->sel.ring_cap > 0 ? a->sel.ring_cap : 0;
    L.drows = cv.take<int32_t>(static_cast<size_t>(H) * (rc > 0 ? rc : 1));
    L.ndelta = cv.take<int32_t>(H);
    L.sel_bytes = a->sel.parts == 4 ? select4_workspace_size(&a->sel) : 0;
    L.sel_ws = cv.take<char>(L.sel_bytes > 0 ? L.sel_bytes : 1);
    L.zero_bytes = a->sel.parts == 4 ? select4_zero_bytes() : 0;
    L.zero_at = L.sel_ws;
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
    // selected rows: at most buffer_pages pages, or in tile mode the token
    // budget plus one cell of at most buffer_pages pages; then the delta rows
    if (a->sel.ring_cap > 0)
        IMI_REQUIRE(a->sel.ring_cap <= kDeltaMax && a->attn.steady_keys && a->attn.steady_values &&
                        a->attn.steady_stride > 0,
                    IMI_ERR_INVALID, "imi_decode_step: the delta append needs ring_cap <= %d and the steady zone",
                    kDeltaMax);
    const int64_t need_rows = static_cast<int64_t>(a->sel.buffer_pages) * a->sel.page_size +
                              (a->sel.tile_mode ? static_cast<int64_t>(a->sel.max_tokens) : 0) +
                              (a->sel.ring_cap > 0 ? a->sel.ring_cap : 0);
    IMI_REQUIRE(a->attn.max_rows >= need_rows, IMI_ERR_INVALID, "imi_decode_step: max_rows %d < %lld selectable rows",
                a->attn.max_rows, static_cast<long long>(need_rows));
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

namespace {
// One decode step with its workspace at ws (already checked to be large enough).
int decode_run(const imi_decode_args* a, void* ws, hipStream_t stream) {
    int rc;
    const DecodeLayout L = decode_layout(a, ws);
    IMI_REQUIRE(a->phases >= 0 && a->phases < 16, IMI_ERR_INVALID, "imi_decode_step: phases %d outside [0, 15]",
                a->phases);
    const int phases = a->phases == 0 ? 3 : a->phases;
    const int kernels = ((phases & 2) ? 3 : 0) | ((phases & 4) ? 1 : 0) | ((phases & 8) ? 2 : 0);
    imi_select_args s = a->sel;
    if (!s.sel_cell) s.sel_cell = L.cell;
    if (!s.sel_offset) s.sel_offset = L.off;
    if (!s.sel_count) s.sel_count = L.cnt;
    if (!s.sel_prefix) s.sel_prefix = L.prefix;
    if (!s.n_selected) s.n_selected = L.nsel;
    if (!s.n_rows) s.n_rows = L.nrows;
    if (s.ring_cap > 0) {
        if (!s.delta_rows) s.delta_rows = L.drows;
        if (!s.n_delta) s.n_delta = L.ndelta;
    }
    if (s.parts == 4 && !s.workspace) {
        s.workspace = L.sel_ws;
        s.workspace_bytes = L.sel_bytes;
    }
    if (phases & 1) {
        rc = select_launch(&s, stream);
        if (rc) return rc;
    } else {
        int64_t nc;
        int km;
        rc = select_validate(&s, nc, km);
        if (rc) return rc;
    }
    if (!kernels) return IMI_OK;
    imi_attention_args t = a->attn;
    t.sel_offset = s.sel_offset;
    t.sel_count = s.sel_count;
    t.sel_prefix = s.sel_prefix;
    t.n_selected = s.n_selected;
    t.n_rows = s.n_rows;
    t.sel_cap = s.sel_cap;
    t.delta_rows = s.ring_cap > 0 ? s.delta_rows : nullptr;
    t.n_delta = s.ring_cap > 0 ? s.n_delta : nullptr;
    t.delta_cap = s.ring_cap > 0 ? s.ring_cap : 0;
    t.workspace = L.attn_ws;
    t.workspace_bytes = L.attn_bytes;
    return attn_launch(&t, stream, kernels);
}
}  // namespace

extern "C" int imi_decode_step(const imi_decode_args* a, imi_stream_t stream_) {
    clear_error();
    int rc = decode_validate(a);
    if (rc) return rc;
    const DecodeLayout need = decode_layout(a, nullptr);
    IMI_REQUIRE(a->attn.workspace && a->attn.workspace_bytes >= need.total, IMI_ERR_WORKSPACE,
                "imi_decode_step: workspace %zu bytes < %zu required", a->attn.workspace_bytes, need.total);
    return decode_run(a, a->attn.workspace, reinterpret_cast<hipStream_t>(stream_));
}

// ------------------------------------------------ decode without allocation
// imi_decode_step_noalloc keeps its workspace in this file-scope device
// array instead of a caller buffer.  Host code never passes the array's name
// to a kernel (on the host it is only a stand-in symbol): the device address
// comes from hipGetSymbolAddress, once per device, and is kept per device.
namespace {
constexpr size_t kScratchBytes = size_t(64) << 20;   // 64 MiB per device
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (resolved on the first
// call per device, with that device current).
int scratch_address(void** out) {
    int dev = 0;
    IMI_HIP_CHECK(hipGetDevice(&dev));
    IMI_REQUIRE(dev >= 0 && dev < kMaxDevices, IMI_ERR_UNSUPPORTED, "imi_decode_step_noalloc: device %d beyond %d",
                dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        IMI_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        IMI_REQUIRE(ptr != nullptr, IMI_ERR_HIP, "imi_decode_step_noalloc: no device address for the scratch array");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return IMI_OK;
}

// Zero fill with a kernel (no memset node when a caller captures the step).
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, size_t n) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256)
        p[i] = 0u;
}
}  // namespace

extern "C" int imi_decode_step_noalloc(const imi_decode_args* a, imi_stream_t stream_) {
    clear_error();
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    int rc = decode_validate(a);
    if (rc) return rc;
    const DecodeLayout need = decode_layout(a, nullptr);
    IMI_REQUIRE(need.total <= kScratchBytes, IMI_ERR_UNSUPPORTED,
                "imi_decode_step_noalloc: this shape needs %zu bytes of scratch, the static scratch holds %zu",
                need.total, kScratchBytes);
    void* ws = nullptr;
    rc = scratch_address(&ws);
    if (rc) return rc;
    // The array keeps whatever the previous call (of any shape) left in it:
    // clear the words this call's kernels expect to find zero.
    const DecodeLayout L = decode_layout(a, ws);
    if (L.zero_bytes > 0) {
        const size_t words = L.zero_bytes / 4;
        const unsigned blocks = static_cast<unsigned>(words < 256 * 256 ? (words + 255) / 256 : 256);
        hipLaunchKernelGGL(zero_words_kernel, dim3(blocks), dim3(256), 0, stream,
                           reinterpret_cast<uint32_t*>(L.zero_at), words);
        IMI_LAUNCH_CHECK("zero_words_kernel");
    }
    return decode_run(a, ws, stream);
}
