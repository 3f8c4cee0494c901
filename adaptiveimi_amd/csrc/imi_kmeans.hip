// Per-(head, subspace) Lloyd k-means on gfx950.
//
// Reference: library/AdaptiveIMI/cpp_extensions/src/kmeans_core.cpp
//   distance     22-44   (8 FMA lanes, lane sums left to right)
//   E-step       222-242 (argmin, strict '<': lowest index wins ties)
//   early stop   244-262
//   M-step       265-312 (members summed in ascending token order, times
//                          1.0f/size; empty cluster <- x[uniform draw])
//   executor     384-501 (one independent run per (head, subspace))
//
// IVF (KmeansExecutorIVF, 503-595) is the one-subspace case: P = 1, Dp = 128,
// k up to kIvfMaxK, kmeans++ with seed 42.
//
// Work layout: every kernel covers all H*P (head, subspace) segments at once.
// E-step (k <= 128): distances are screened on the matrix cores (bf16 MFMA
// with the centroids split into hi + lo bf16 parts, under a proven rounding
// bound) and only the centroids that can still win get the exact reference
// distance; k > 128 uses the exact distance to every centroid.  Both emit
// the block histogram of labels and each token's stable rank inside its
// block, so the M-step's member lists come from one scan + one scatter.  The
// M-step sums each cluster sequentially in ascending token order (the
// reference's order with one thread per subspace run): one workgroup per
// cluster, one wave running the chains while three waves stream the member
// rows through register rings and an LDS hand-off.
#include <limits>
#include <random>
#include <vector>

#include "imi_common.hpp"
#include "imi_sort.hpp"

namespace imi {
namespace {

struct KmParams {
    const uint16_t* keys;
    int64_t hs, ts;
    int H, T, P, kmax, DP;
    int k[4];
    float* cent;       // [seg][kmax][DP]
    int32_t* labels;   // [seg][T]
    float* mind;       // [seg][T] or null
    int32_t* hist;     // [seg][kmax][nblk] or null
    int32_t* rank;     // [seg][T]
    float* ipart;      // [seg][nblk]
    int32_t* sorted;   // [seg][T]
    int32_t* off;      // [seg][kmax + 1]
    int32_t* empties;  // [seg][kmax]
    float* prev;       // [seg]
    int32_t* done;     // [seg] or null
    int32_t* iters;    // [seg] or null
    void* ppstats;     // kmeans++ block statistics [seg][T / kPpRows] (init_mode 2)
    int nblk;
    int max_iters;
    float tol;
    int es_min;
    float es_rel;
    int exact;         // the E-step's distances are read (min distances or the early-stop inertia)
    // Block member lists (no km_scan / km_scatter pass): the E-step writes each
    // block's tokens in label order to `rank` ([seg][T], position blk * 256 +
    // the token's place in its block) and the block's row of label offsets to
    // loff ([seg][nblk][kmax + 1]: first place of each label, then the
    // block's token count); the M-step finds its members from its label's
    // pair of offsets in every row.  Null: the scanned member lists.
    int32_t* loff;
};

struct Draws {
    int32_t v[256];  // uniform draws for the empty clusters of one iteration
};

constexpr int kDraws = 256;      // empty-cluster draws one launch carries
constexpr int kLocalMaxBlk = 512;   // blocks (T <= 131072) of the block member lists
constexpr int kIvfMaxK = 4096;   // IVF clusters per head

__host__ __device__ inline int bits_for(int n) {
    int b = 0;
    while ((1 << b) < n) ++b;
    return b;
}

__global__ __launch_bounds__(64) void km_init_first_kernel(KmParams a) {
    const int c = blockIdx.x, seg = blockIdx.y;
    const int h = seg / a.P, p = seg % a.P;
    if (c >= a.k[p]) return;
    for (int d = threadIdx.x; d < a.DP; d += 64)
        a.cent[(static_cast<int64_t>(seg) * a.kmax + c) * a.DP + d] =
            bf16_to_f32(a.keys[h * a.hs + static_cast<int64_t>(c) * a.ts + p * a.DP + d]);
}

// Reference distance between the register-resident subvector x and centroid
// row cr (LDS): lane j accumulates dims j, j+8, ... with fused multiply-add,
// then the eight lane sums are added left to right.
template <int DP>
__device__ __forceinline__ float l2_lanes8(const float (&x)[DP], const float* cr) {
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < DP; i += 8) {
        const float4 c0 = *reinterpret_cast<const float4*>(cr + i);
        const float4 c1 = *reinterpret_cast<const float4*>(cr + i + 4);
        float d;
        d = x[i + 0] - c0.x; acc[0] = __builtin_fmaf(d, d, acc[0]);
        d = x[i + 1] - c0.y; acc[1] = __builtin_fmaf(d, d, acc[1]);
        d = x[i + 2] - c0.z; acc[2] = __builtin_fmaf(d, d, acc[2]);
        d = x[i + 3] - c0.w; acc[3] = __builtin_fmaf(d, d, acc[3]);
        d = x[i + 4] - c1.x; acc[4] = __builtin_fmaf(d, d, acc[4]);
        d = x[i + 5] - c1.y; acc[5] = __builtin_fmaf(d, d, acc[5]);
        d = x[i + 6] - c1.z; acc[6] = __builtin_fmaf(d, d, acc[6]);
        d = x[i + 7] - c1.w; acc[7] = __builtin_fmaf(d, d, acc[7]);
    }
    float t = acc[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) t = t + acc[j];
    return t;
}

// The same distance with the row still in its bf16 load registers (each
// 16-byte part holds dims i .. i+7 of lanes 0..7): no float copy of the row,
// for kernels that keep many rows in flight.
template <int DP, typename V>
__device__ __forceinline__ float l2_lanes8_bf16(const V (&v)[DP / 8], const float* cr) {
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < DP / 8; ++i) {
        const float4 c0 = *reinterpret_cast<const float4*>(cr + 8 * i);
        const float4 c1 = *reinterpret_cast<const float4*>(cr + 8 * i + 4);
        float d;
        d = bf16_lo(v[i].x) - c0.x; acc[0] = __builtin_fmaf(d, d, acc[0]);
        d = bf16_hi(v[i].x) - c0.y; acc[1] = __builtin_fmaf(d, d, acc[1]);
        d = bf16_lo(v[i].y) - c0.z; acc[2] = __builtin_fmaf(d, d, acc[2]);
        d = bf16_hi(v[i].y) - c0.w; acc[3] = __builtin_fmaf(d, d, acc[3]);
        d = bf16_lo(v[i].z) - c1.x; acc[4] = __builtin_fmaf(d, d, acc[4]);
        d = bf16_hi(v[i].z) - c1.y; acc[5] = __builtin_fmaf(d, d, acc[5]);
        d = bf16_lo(v[i].w) - c1.z; acc[6] = __builtin_fmaf(d, d, acc[6]);
        d = bf16_hi(v[i].w) - c1.w; acc[7] = __builtin_fmaf(d, d, acc[7]);
    }
    float t = acc[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) t = t + acc[j];
    return t;
}

// E-step over one block of 256 tokens of one segment.
template <int DP>
__global__ __launch_bounds__(256) void km_assign_kernel(KmParams a) {
    extern __shared__ float smem[];
    const int seg = blockIdx.y, blk = blockIdx.x;
    if (a.done && a.done[seg]) return;
    const int h = seg / a.P, p = seg % a.P;
    const int k = a.k[p];
    const int tid = threadIdx.x;
    float* cs = smem;                                   // [k][DP]
    int* wcnt = reinterpret_cast<int*>(smem + a.kmax * DP);  // [4][kmax]
    float* red = reinterpret_cast<float*>(wcnt + 4 * a.kmax);  // [4]

    const float* cg = a.cent + static_cast<int64_t>(seg) * a.kmax * DP;
    for (int i = tid; i < k * DP; i += 256) cs[i] = cg[i];

    const int t = blk * 256 + tid;
    const bool valid = t < a.T;
    float x[DP];
    if (valid) {
        const uint4* src = reinterpret_cast<const uint4*>(a.keys + h * a.hs + static_cast<int64_t>(t) * a.ts + p * DP);
#pragma unroll
        for (int i = 0; i < DP / 8; ++i) {
            const uint4 v = src[i];
            x[8 * i + 0] = bf16_lo(v.x); x[8 * i + 1] = bf16_hi(v.x);
            x[8 * i + 2] = bf16_lo(v.y); x[8 * i + 3] = bf16_hi(v.y);
            x[8 * i + 4] = bf16_lo(v.z); x[8 * i + 5] = bf16_hi(v.z);
            x[8 * i + 6] = bf16_lo(v.w); x[8 * i + 7] = bf16_hi(v.w);
        }
    } else {
#pragma unroll
        for (int i = 0; i < DP; ++i) x[i] = 0.0f;
    }
    __syncthreads();

    float best = 3.402823466e38f;  // FLT_MAX
    int arg = 0;
    for (int c = 0; c < k; ++c) {
        const float dist = l2_lanes8<DP>(x, cs + c * DP);
        if (dist < best) {
            best = dist;
            arg = c;
        }
    }
    if (valid) {
        a.labels[static_cast<int64_t>(seg) * a.T + t] = arg;
        if (a.mind) a.mind[static_cast<int64_t>(seg) * a.T + t] = best;
    }
    if (a.hist == nullptr) return;

    // inertia partial of this block (fixed reduction order)
    float part = wave_sum(valid ? best : 0.0f);
    if (lane_id() == 0) red[tid >> 6] = part;
    const int r = block_digit_rank(arg, valid, k, bits_for(k), wcnt,
                                   a.hist + static_cast<int64_t>(seg) * a.kmax * a.nblk, a.nblk, blk);
    if (valid) a.rank[static_cast<int64_t>(seg) * a.T + t] = r;
    if (tid == 0) a.ipart[static_cast<int64_t>(seg) * a.nblk + blk] = ((red[0] + red[1]) + red[2]) + red[3];
}

// E-step of the IVF index (Dp = 128, k up to kIvfMaxK): the centroids pass
// through LDS in tiles of kTileC rows; the exact reference distance to every
// centroid, c ascending, strict '<'.  Outputs as km_assign_kernel.
constexpr int kTileC = 64;

template <int DP>
size_t tiled_lds_bytes(int kmax) {
    return static_cast<size_t>(kTileC) * DP * sizeof(float) + 4 * static_cast<size_t>(kmax) * sizeof(int) + 64;
}

template <int DP>
__global__ __launch_bounds__(256) void km_assign_tiled_kernel(KmParams a) {
    extern __shared__ float smem[];
    const int seg = blockIdx.y, blk = blockIdx.x;
    if (a.done && a.done[seg]) return;
    const int h = seg / a.P, p = seg % a.P;
    const int k = a.k[p];
    const int tid = threadIdx.x;
    float* cs = smem;                                              // [kTileC][DP]
    int* wcnt = reinterpret_cast<int*>(smem + kTileC * DP);        // [4][kmax]
    float* red = reinterpret_cast<float*>(wcnt + 4 * a.kmax);      // [4]
    const float4* cg = reinterpret_cast<const float4*>(a.cent + static_cast<int64_t>(seg) * a.kmax * DP);

    const int t = blk * 256 + tid;
    const bool valid = t < a.T;
    float x[DP];
    {
        // past the end: row T - 1 again (a valid row; its label is not stored)
        const uint4* src = reinterpret_cast<const uint4*>(a.keys + h * a.hs +
                                                          static_cast<int64_t>(valid ? t : a.T - 1) * a.ts + p * DP);
#pragma unroll
        for (int i = 0; i < DP / 8; ++i) {
            const uint4 v = src[i];
            x[8 * i + 0] = bf16_lo(v.x); x[8 * i + 1] = bf16_hi(v.x);
            x[8 * i + 2] = bf16_lo(v.y); x[8 * i + 3] = bf16_hi(v.y);
            x[8 * i + 4] = bf16_lo(v.z); x[8 * i + 5] = bf16_hi(v.z);
            x[8 * i + 6] = bf16_lo(v.w); x[8 * i + 7] = bf16_hi(v.w);
        }
    }
    float best = 3.402823466e38f;  // FLT_MAX
    int arg = 0;
    for (int c0 = 0; c0 < k; c0 += kTileC) {
        const int nc = min(kTileC, k - c0);
        __syncthreads();   // the previous tile is read
        for (int i = tid; i < nc * (DP / 4); i += 256)
            reinterpret_cast<float4*>(cs)[i] = cg[static_cast<int64_t>(c0) * (DP / 4) + i];
        __syncthreads();
#pragma unroll 1
        for (int c = 0; c < nc; ++c) {
            const float dist = l2_lanes8<DP>(x, cs + c * DP);
            if (dist < best) {
                best = dist;
                arg = c0 + c;
            }
        }
    }
    if (valid) {
        a.labels[static_cast<int64_t>(seg) * a.T + t] = arg;
        if (a.mind) a.mind[static_cast<int64_t>(seg) * a.T + t] = best;
    }
    if (a.hist == nullptr) return;
    float part = wave_sum(valid ? best : 0.0f);
    if (lane_id() == 0) red[tid >> 6] = part;
    const int r = block_digit_rank(arg, valid, k, bits_for(k), wcnt,
                                   a.hist + static_cast<int64_t>(seg) * a.kmax * a.nblk, a.nblk, blk);
    if (valid) a.rank[static_cast<int64_t>(seg) * a.T + t] = r;
    if (tid == 0) a.ipart[static_cast<int64_t>(seg) * a.nblk + blk] = ((red[0] + red[1]) + red[2]) + red[3];
}

// E-step with matrix-core screening (k <= 128).  For token x and centroid
// c the distance is approximated as D~ = |x|^2 + |c|^2 - 2 x.c, with x.c on
// v_mfma_f32_16x16x32_bf16: x is bf16 already and c enters as two bf16
// parts (hi = bf16(c), lo = bf16(c - hi), |c - hi - lo| <= 2^-16 |c|).
// Rounding analysis (unit roundoff u = 2^-24, at most ~256 accumulations
// per dot product, reference distance = 8 FMA chains + 7 adds):
//   |D~ - D_ref| <= 2^-14.6 (|x|^2 + |c|^2) <= E = 2^-12 (|x|^2 + max|c|^2)
// (4x margin, plus 1e-30 for flushed subnormal products).  Any centroid
// that can win under the reference order satisfies D~(c) <= min D~ + 2E, so
// only those candidates get the exact reference distance (l2_lanes8, c
// ascending, strict '<'); usually there is one.  Non-finite or huge values
// (|x|^2 + max|c|^2 > 1e37) make every centroid a candidate, which is the
// plain exact E-step.  Outputs (labels, min distances, block ranks, label
// histogram, inertia partials) are those of km_assign_kernel.
typedef __attribute__((ext_vector_type(8))) __bf16 km_bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float km_f32x4_t;
typedef __attribute__((ext_vector_type(4))) unsigned int km_u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned int km_u32x2_t;
typedef __attribute__((ext_vector_type(4))) short km_s16x4_t;
typedef __attribute__((address_space(3))) km_s16x4_t km_lds_s16x4_t;

constexpr int kScreenMaxK = 128;
constexpr int kScreenQueue = 64;   // queued exact passes per 256-token block

__device__ __forceinline__ uint32_t xor16_u(uint32_t v) { return __float_as_uint(xor16(__uint_as_float(v))); }
__device__ __forceinline__ uint32_t xor32_u(uint32_t v) { return __float_as_uint(xor32(__uint_as_float(v))); }

// Intra-wave LDS hand-off (compiler ordering only; a wave's LDS instructions
// execute in order).
__device__ __forceinline__ void km_wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int DP>
size_t screen_lds_bytes(int kmax) {
    constexpr int KH = DP / 32;
    const size_t nct = (kmax + 15) / 16;
    return static_cast<size_t>(kmax) * (DP + 4) * 4 + nct * KH * 2 * 64 * 16 + nct * 16 * 4 + 256 * 2 * 8 +
           kScreenQueue * 8 + 4 * static_cast<size_t>(kmax) * 4 + 16 + (kScreenQueue + 1) * 4 +
           (kScreenQueue + 1) * 4;
}

// Row shift left by K inside a row of 16 lanes: lane i gets lane i + K's value.
template <int K>
__device__ __forceinline__ float dpp_row_shl(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + K, 0xF, 0xF, false));
}

// KT > 0: every segment has k = 16 KT centroids (whole tiles, no per-tile
// tests); KT = 0: any k <= MAXK.
template <int DP, int MAXK, int KT, bool EXACT>
__global__ __launch_bounds__(256, 4) void km_assign_screen_kernel(KmParams a, int chunks) {
    constexpr int KH = DP / 32;   // 32-dim K steps per subvector
    constexpr int NCT = KT > 0 ? KT : MAXK / 16;   // centroid tiles held per lane
    extern __shared__ float smem[];
    const int seg = blockIdx.y;
    if (a.done && a.done[seg]) return;
    const int h = seg / a.P, p = seg % a.P;
    const int k = KT > 0 ? 16 * KT : a.k[p];
    const int nct = KT > 0 ? KT : (k + 15) >> 4;
    const int nct_max = (a.kmax + 15) >> 4;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    constexpr int CS = DP + 4;
    float* cs = smem;                                                        // [kmax][DP + 4]
    km_u32x4_t* apk = reinterpret_cast<km_u32x4_t*>(cs + a.kmax * CS);      // [nct][KH][hi,lo][64 lanes]
    float* ccs = reinterpret_cast<float*>(apk + nct_max * KH * 2 * 64);     // [nct * 16]
    uint64_t* cmask = reinterpret_cast<uint64_t*>(ccs + nct_max * 16);      // [256][2] candidate bits
    uint64_t* qbest = cmask + 256 * 2;                                      // [kScreenQueue] (distance, centroid)
    int* wcnt = reinterpret_cast<int*>(qbest + kScreenQueue);               // [4][kmax]
    float* red = reinterpret_cast<float*>(wcnt + 4 * a.kmax);               // [4]
    int* qtok = reinterpret_cast<int*>(red + 4);                            // [kScreenQueue] queued tokens
    int* qcnt = qtok + kScreenQueue;                                        // queue length
    int* qoff = qcnt + 1;                                                   // [kScreenQueue + 1] first pair
    // the block rank's label offsets reuse the queue's slots, which are read
    // before its first barrier ([kmax] <= 2 * kScreenQueue ints, [4])
    int* lofs = reinterpret_cast<int*>(qbest);
    int* lwsum = qoff;

    const float* cg = a.cent + static_cast<int64_t>(seg) * a.kmax * DP;
    {
        // centroid rows -> LDS (padded rows), every float4 load issued first
        constexpr int PER = MAXK * DP / 4 / 256;
        float4 v[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i4 = tid + u * 256;
            v[u] = i4 * 4 < k * DP ? reinterpret_cast<const float4*>(cg)[i4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i = (tid + u * 256) * 4;
            if (i < k * DP) *reinterpret_cast<float4*>(cs + (i / DP) * CS + i % DP) = v[u];
        }
    }
    if (tid == 0) *qcnt = 0;
    __syncthreads();
    // A operands: lane l of tile ct holds centroid 16ct + l%16, dims
    // 32kh + 8(l/16) .. +7 (v_mfma_f32_16x16x32_bf16 A layout)
    for (int e = tid; e < nct * KH * 2 * 64; e += 256) {
        const int l = e & 63, part = (e >> 6) & 1, t2 = e >> 7;
        const int kh = t2 % KH, ct = t2 / KH;
        const int c = ct * 16 + (l & 15);
        const int d0 = kh * 32 + 8 * (l >> 4);
        uint32_t w[4] = {0u, 0u, 0u, 0u};
        if (c < k) {
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                const float v0 = cs[c * CS + d0 + i], v1 = cs[c * CS + d0 + i + 1];
                uint16_t b0 = f32_to_bf16(v0), b1 = f32_to_bf16(v1);
                if (part) {
                    b0 = f32_to_bf16(v0 - bf16_to_f32(b0));
                    b1 = f32_to_bf16(v1 - bf16_to_f32(b1));
                }
                w[i / 2] = static_cast<uint32_t>(b0) | (static_cast<uint32_t>(b1) << 16);
            }
        }
        apk[e] = km_u32x4_t{w[0], w[1], w[2], w[3]};
    }
    for (int c = tid; c < nct * 16; c += 256) {
        float sq = INFINITY;   // padding rows of A are zero: their e(c) is +inf
        if (c < k) {
            sq = 0.0f;
#pragma unroll
            for (int d = 0; d < DP; ++d) sq = __builtin_fmaf(cs[c * CS + d], cs[c * CS + d], sq);
        }
        ccs[c] = sq;
    }
    __syncthreads();
    float ccmax = 0.0f;
    for (int c = lane; c < k; c += 64) ccmax = fmaxf(ccmax, ccs[c]);
    ccmax = wave_max(ccmax);
    const int nwords = (nct + 1) >> 1;          // 32-bit candidate words in use
    // |c|^2 of the lane's accumulator rows (centroid 16 ct + 4 (lane / 16) + r)
    // in registers for up to 4 tiles, else read from LDS per use
    constexpr bool CCREG = NCT <= 4;
    float ccv[CCREG ? NCT : 1][4];
#pragma unroll
    for (int ct = 0; ct < (CCREG ? NCT : 1); ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) ccv[ct][r] = ct < nct ? -0.5f * ccs[ct * 16 + 4 * (lane >> 4) + r] : -INFINITY;

    const uint16_t* kb = a.keys + h * a.hs + p * DP;
    // 256-token blocks blockIdx.x * chunks .. +chunks-1 (the prologue above is
    // shared by all of them)
#pragma unroll 1
    for (int ci = 0; ci < chunks; ++ci) {
    const int blk = blockIdx.x * chunks + ci;
    if (blk >= a.nblk) break;
    if (ci > 0) __syncthreads();   // the previous block's LDS reads are done
    // the MFMA operands of the wave's four 16-token tiles are loaded up front
    // (lane l: token l%16, dims 32kh + 8(l/16) .. +7)
    const int tw0 = blk * 256 + wave * 64;
    const int t = blk * 256 + tid;
    const bool valid = t < a.T;
    // (tokens past T re-read token T - 1: the loads need no branches, and
    // those lanes' results are never stored)
    km_u32x4_t bqa[4][KH];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int tt = min(tw0 + 16 * j + (lane & 15), a.T - 1);
#pragma unroll
        for (int kh = 0; kh < KH; ++kh)
            bqa[j][kh] = *reinterpret_cast<const km_u32x4_t*>(kb + static_cast<int64_t>(tt) * a.ts + kh * 32 +
                                                              8 * (lane >> 4));
    }
    // the thread's own token row for the exact pass, loaded now as well
    km_u32x4_t xr[EXACT ? DP / 8 : 1];
    if constexpr (EXACT) {
        const int tc = min(t, a.T - 1);
#pragma unroll
        for (int i = 0; i < DP / 8; ++i)
            xr[i] = *reinterpret_cast<const km_u32x4_t*>(kb + static_cast<int64_t>(tc) * a.ts + 8 * i);
    }
    // screening: token tile j = tokens 16j .. 16j+15 of this wave's 64.
    // f(c) = x.c - |c|^2 / 2 = -e(c) / 2 with e(c) = |c|^2 - 2 x.c, which
    // orders the centroids like D~ = |x|^2 + e(c) (largest f first): the
    // matrix cores start each tile's accumulator at -|c|^2 / 2 (halving is
    // exact but for subnormals, which the absolute term of the bound covers).
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const km_u32x4_t* bq = bqa[j];
        // |x|^2 from the diagonal of x x^T (the same registers serve as A and
        // B): token t's entry sits in lane 16(t/4) + t, register t % 4
        float xs;
        {
            km_f32x4_t dg = km_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kh = 0; kh < KH; ++kh)
                dg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(km_bf16x8_t, bq[kh]),
                                                             __builtin_bit_cast(km_bf16x8_t, bq[kh]), dg, 0, 0, 0);
            const int tl = lane & 15, rr = tl & 3;
            const float own = rr == 0 ? dg[0] : rr == 1 ? dg[1] : rr == 2 ? dg[2] : dg[3];
            xs = __shfl(own, 16 * (tl >> 2) + tl);
        }
        float ev[NCT][4];
        float emax = -INFINITY;
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            if (KT > 0 || ct < nct) {
                km_f32x4_t acc;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[r] = CCREG ? ccv[CCREG ? ct : 0][r] : -0.5f * ccs[ct * 16 + 4 * (lane >> 4) + r];
#pragma unroll
                for (int kh = 0; kh < KH; ++kh) {
                    const km_u32x4_t ah = apk[((ct * KH + kh) * 2 + 0) * 64 + lane];
                    const km_u32x4_t al = apk[((ct * KH + kh) * 2 + 1) * 64 + lane];
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(km_bf16x8_t, ah),
                                                                  __builtin_bit_cast(km_bf16x8_t, bq[kh]), acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(km_bf16x8_t, al),
                                                                  __builtin_bit_cast(km_bf16x8_t, bq[kh]), acc, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    ev[ct][r] = acc[r];
                    emax = fmaxf(emax, acc[r]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) ev[ct][r] = -INFINITY;
            }
        }
        emax = fmaxf(emax, xor16(emax));
        emax = fmaxf(emax, xor32(emax));
        // candidates: e(c) <= min e + 2E, i.e. f(c) >= max f - E; non-finite
        // or huge magnitudes make every finite f a candidate (the exhaustive
        // E-step)
        const float mag = xs + ccmax;
        const float lim0 = emax - (0x1p-12f * mag + 1e-30f);
        const bool all = !(mag <= 1e37f) || !(lim0 > -INFINITY);
        const float lim = all ? -3.402823466e38f : lim0;
        uint32_t m[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            uint32_t nib = 0u;
#pragma unroll
            for (int r = 0; r < 4; ++r) nib |= ev[ct][r] >= lim ? (1u << r) : 0u;
            if (all) {
                // every real centroid: past 1e37 the screen's products and
                // norms can overflow to inf or NaN where a distance does not
                const int c0 = 16 * ct + 4 * (lane >> 4);
                nib = KT > 0 ? 0xFu : (c0 >= k ? 0u : (k - c0 >= 4 ? 0xFu : (1u << (k - c0)) - 1u));
            }
            m[ct >> 1] |= nib << ((ct & 1) * 16 + 4 * (lane >> 4));
        }
#pragma unroll
        for (int w = 0; w < MAXK / 32; ++w) {
            if (w < nwords) {
                m[w] |= xor16_u(m[w]);
                m[w] |= xor32_u(m[w]);
            }
        }
        if (lane < 16) {
            const int slot = wave * 64 + 16 * j + lane;
            cmask[slot * 2 + 0] = static_cast<uint64_t>(m[0]) | (static_cast<uint64_t>(m[1]) << 32);
            cmask[slot * 2 + 1] = static_cast<uint64_t>(m[2]) | (static_cast<uint64_t>(m[3]) << 32);
        }
    }
    km_wave_lds_sync();

    float best = 3.402823466e38f;  // FLT_MAX
    int arg = 0;
    if constexpr (EXACT) {
        // exact reference distance to every candidate of the thread's token
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            uint64_t mm = cmask[tid * 2 + w];
            while (mm) {
                const int c = 64 * w + __builtin_ctzll(mm);
                mm &= mm - 1;
                const float dist = l2_lanes8_bf16<DP>(xr, cs + c * CS);
                if (dist < best) {
                    best = dist;
                    arg = c;
                }
            }
        }
    } else {
        // No distance is read: a lone candidate is the reference's label (the
        // bound above).  Tokens with several candidates (a few percent, but
        // in most waves) queue up; their (token, candidate) distances are
        // spread over the block, 8 lanes per pair.
        const uint64_t m0 = cmask[tid * 2], m1 = cmask[tid * 2 + 1];
        arg = m0 ? __builtin_ctzll(m0) : (m1 ? 64 + __builtin_ctzll(m1) : 0);
        const bool multi = valid && __popcll(m0) + __popcll(m1) > 1;
        const uint64_t bal = __ballot(multi);
        int slot = 0;
        if (bal) {
            int base = 0;
            if (lane == 0) base = atomicAdd(qcnt, __popcll(bal));
            slot = __shfl(base, 0) + __popcll(bal & lanemask_lt());
        }
        if (multi && slot < kScreenQueue) qtok[slot] = tid;
        __syncthreads();
        const int nq = min(*qcnt, kScreenQueue);
        if (wave == 0) {
            // the pairs of queued token i are [qoff[i], qoff[i + 1])
            int n = 0;
            if (lane < nq) {
                const int tk = qtok[lane];
                n = __popcll(cmask[tk * 2]) + __popcll(cmask[tk * 2 + 1]);
                qbest[lane] = ~0ull;
            }
            const int incl = wave_incl_scan(n);
            if (lane < kScreenQueue) qoff[lane] = incl - n;
            if (lane == 63) qoff[kScreenQueue] = incl;
        }
        __syncthreads();
        {
            // Pair p on lanes 8 (p % 8) .. +7 of wave (p / 8) % 4: lane part j
            // sums dims j, j + 8, .. in ascending order (the reference's
            // lane j), the group adds the eight sums left to right on its
            // first lane (row shifts inside the 16-lane row), and an LDS
            // minimum over (distance bits, centroid) keeps the smallest
            // distance below FLT_MAX and, among equal ones, the lowest
            // centroid: the reference's strict < over ascending centroids.
            const int npairs = qoff[kScreenQueue];
            const int part = lane & 7;
#pragma unroll 1
            for (int p0 = 0; p0 < npairs; p0 += 32) {
                const int pr = p0 + wave * 8 + (lane >> 3);
                float acc = 0.0f;
                int qi = 0, c = 0;
                if (pr < npairs) {
                    for (int step = 32; step > 0; step >>= 1)
                        if (qi + step < nq && qoff[qi + step] <= pr) qi += step;
                    const int tk = qtok[qi];
                    int r = pr - qoff[qi];
                    const uint64_t w0 = cmask[tk * 2], w1 = cmask[tk * 2 + 1];
                    const int n0 = __popcll(w0);
                    uint64_t mm = r < n0 ? w0 : w1;
                    const int cb = r < n0 ? 0 : 64;
                    r = r < n0 ? r : r - n0;
                    for (int i = 0; i < r; ++i) mm &= mm - 1;
                    c = cb + __builtin_ctzll(mm);
                    const uint16_t* xr = kb + static_cast<int64_t>(blk * 256 + tk) * a.ts + part;
                    uint16_t xv[DP / 8];
#pragma unroll
                    for (int i = 0; i < DP / 8; ++i) xv[i] = xr[8 * i];
                    const float* cr = cs + c * CS + part;
#pragma unroll
                    for (int i = 0; i < DP / 8; ++i) {
                        const float d = bf16_to_f32(xv[i]) - cr[8 * i];
                        acc = __builtin_fmaf(d, d, acc);
                    }
                }
                float t = acc;
                t = t + dpp_row_shl<1>(acc);
                t = t + dpp_row_shl<2>(acc);
                t = t + dpp_row_shl<3>(acc);
                t = t + dpp_row_shl<4>(acc);
                t = t + dpp_row_shl<5>(acc);
                t = t + dpp_row_shl<6>(acc);
                t = t + dpp_row_shl<7>(acc);
                if (pr < npairs && part == 0 && t < 3.402823466e38f)
                    atomicMin(reinterpret_cast<unsigned long long*>(&qbest[qi]),
                              (static_cast<unsigned long long>(__float_as_uint(t)) << 32) | static_cast<uint32_t>(c));
            }
        }
        // past the queue's end a token runs its own exact pass (its row
        // re-read: it is in L2)
        auto exact_label = [&](int tk) {
            km_u32x4_t xq[DP / 8];
#pragma unroll
            for (int i = 0; i < DP / 8; ++i)
                xq[i] = *reinterpret_cast<const km_u32x4_t*>(kb + static_cast<int64_t>(blk * 256 + tk) * a.ts + 8 * i);
            float qb = 3.402823466e38f;
            int qa = 0;
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                uint64_t mm = cmask[tk * 2 + w];
                while (mm) {
                    const int c = 64 * w + __builtin_ctzll(mm);
                    mm &= mm - 1;
                    const float dist = l2_lanes8_bf16<DP>(xq, cs + c * CS);
                    if (dist < qb) {
                        qb = dist;
                        qa = c;
                    }
                }
            }
            return qa;
        };
        if (multi && slot >= kScreenQueue) arg = exact_label(tid);
        __syncthreads();
        if (multi && slot < kScreenQueue) {
            const uint64_t b = qbest[slot];   // no distance below FLT_MAX: label 0, as the reference's loop
            arg = b == ~0ull ? 0 : static_cast<int>(static_cast<uint32_t>(b));
        }
        if (tid == 0) *qcnt = 0;   // read by every thread before the barrier above
    }
    if (valid) {
        a.labels[static_cast<int64_t>(seg) * a.T + t] = arg;
        if (EXACT && a.mind) a.mind[static_cast<int64_t>(seg) * a.T + t] = best;
    }
    if (a.hist == nullptr) continue;

    float part = EXACT ? wave_sum(valid ? best : 0.0f) : 0.0f;
    if (lane_id() == 0) red[tid >> 6] = part;
    if (a.loff) {
        // block member lists: the token at its place in the block's label order
        const int pos = block_digit_pos(arg, valid, k, bits_for(k), wcnt, lofs, lwsum,
                                        a.loff + (static_cast<int64_t>(seg) * a.nblk + blk) * (a.kmax + 1));
        if (valid) a.rank[static_cast<int64_t>(seg) * a.T + blk * 256 + pos] = t;
    } else {
        const int r = block_digit_rank(arg, valid, k, bits_for(k), wcnt,
                                       a.hist + static_cast<int64_t>(seg) * a.kmax * a.nblk, a.nblk, blk);
        if (valid) a.rank[static_cast<int64_t>(seg) * a.T + t] = r;
    }
    if (tid == 0) a.ipart[static_cast<int64_t>(seg) * a.nblk + blk] = ((red[0] + red[1]) + red[2]) + red[3];
    }
}

// ---------------------------------------------------------------- kmeans++
// kmeans_plusplus_init_inplace (kmeans_core.cpp:138-186) for every (head,
// subspace) segment at once, two launches per pick.  The random draws do not
// depend on the data: the host replays std::mt19937_64(seed) for the first
// index (uniform_int_distribution<int32_t>(0, T-1)) and for one
// generate_canonical<double, 53> per pick, which is what
// uniform_real_distribution<double>(0, total) consumes; target = canon *
// total.  The reference sums the min distances sequentially in double (the
// total, then the running sum that picks the first index with cumsum >=
// target).  When every value is a multiple of the smallest value's ulp and
// the total stays below 2^53 such units (the exponent spread is checked per
// pick), no partial sum rounds, so the sequential doubles equal exact
// integer prefix sums, which any blocking of the rows reproduces; otherwise
// one thread replays the sequential loops.
//   km_pp_step_kernel  (launch c >= 1; blocks of kPpRows rows x segments):
//                      pick c - 1 (the first row, or found from launch
//                      c - 1's block statistics and minima), written by the
//                      segment's block 0; then each row's min distance to
//                      the picks 0..c-1, and the block's exponent range and
//                      its sum in units of its own smallest exponent
//   km_pp_pick_kernel  (one workgroup per segment): the last pick
// Every block finds the pick itself (a few KB of statistics and one block's
// minima), so no launch separates a pick from the next distance pass; the
// minima and statistics alternate between two buffers for that reason.
constexpr int kPpRPT = 4;                 // consecutive rows per thread
constexpr int kPpRows = 256 * kPpRPT;     // rows per distance block

struct PpBlock {                 // per (segment, block)
    unsigned long long units;    // sum of its values in units of 2^(emin - 150)
    int emin, emax;              // exponent range of its non-zero values (emin = INT_MAX: none)
};


// value m in units of 2^(emin_eff - 150) (m a multiple of that unit when the
// segment passes the exactness test; shifts past 63 only occur when it fails)
__device__ __forceinline__ unsigned long long pp_units(float m, int emin_eff) {
    const uint32_t u = __float_as_uint(m);
    const int e = static_cast<int>((u >> 23) & 0xFFu);
    const unsigned long long mant = static_cast<unsigned long long>(u & 0x7FFFFFu) | (e > 0 ? (1ull << 23) : 0ull);
    const int sh = (e > 0 ? e : 1) - emin_eff;
    return (mant == 0 || sh < 0 || sh > 63) ? 0ull : mant << sh;
}

__device__ __forceinline__ int pp_exp(float m) {
    const int e = static_cast<int>((__float_as_uint(m) >> 23) & 0xFFu);
    return e > 0 ? e : 1;
}

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ long long wave_incl_scan_ll(long long v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const long long y = __shfl_up(v, o);
        if (lane_id() >= o) v += y;
    }
    return v;
}

// 256-thread exclusive scan of one long long per thread; the total to all
__device__ __forceinline__ long long block_excl_scan_ll(long long v, long long* sh, long long& total) {
    const long long incl = wave_incl_scan_ll(v);
    const int w = threadIdx.x >> 6;
    if (lane_id() == 63) sh[w] = incl;
    __syncthreads();
    long long base = 0;
    total = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (j < w) base += sh[j];
        total += sh[j];
    }
    __syncthreads();
    return base + incl - v;
}

typedef unsigned int __attribute__((ext_vector_type(4))) pp_u32x4_t;

struct PpShared {
    int e[2][4];
    long long sc[4];
    int blk, sel;
    long long base;
};

// Row of pick c >= 1 of one segment (all 256 threads; the row to every
// thread) from the minima md and block statistics st the distance pass of
// pick c wrote: the segment's exponent range and, when every partial sum is
// exact in double, the block and then the row whose integer prefix sum
// reaches the target; otherwise thread 0 replays the reference's sequential
// double sums (kmeans_core.cpp:160-181).
__device__ int pp_pick_row(const float* md, const PpBlock* st, int nbp, int T, double canon, PpShared& sh) {
    const int tid = threadIdx.x;
    if (tid == 0) {
        sh.blk = nbp;
        sh.sel = T;
    }
    // this thread's consecutive blocks
    const int per = (nbp + 255) / 256;
    const int b0 = min(tid * per, nbp), b1 = min(b0 + per, nbp);
    int emin = 0x7FFFFFFF, emax = 0;
    for (int bb = b0; bb < b1; ++bb) {
        emin = min(emin, st[bb].emin);
        emax = max(emax, st[bb].emax);
    }
    const int w = tid >> 6;
    emin = wave_min_i(emin);
    emax = wave_max_i(emax);
    if (lane_id() == 0) {
        sh.e[0][w] = emin;
        sh.e[1][w] = emax;
    }
    __syncthreads();
    const int e_lo = min(min(sh.e[0][0], sh.e[0][1]), min(sh.e[0][2], sh.e[0][3]));
    const int e_hi = max(max(sh.e[1][0], sh.e[1][1]), max(sh.e[1][2], sh.e[1][3]));
    int logT = 0;
    while ((1ll << logT) < static_cast<long long>(T)) ++logT;
    const bool any = e_lo != 0x7FFFFFFF;
    const bool exact = !any || (e_hi - e_lo) + 24 + logT <= 53;
    if (exact) {
        const int emin_eff = any ? e_lo : 1;
        long long mine = 0;
        for (int bb = b0; bb < b1; ++bb)
            if (st[bb].emin != 0x7FFFFFFF)
                mine += static_cast<long long>(st[bb].units << (st[bb].emin - emin_eff));
        long long total_u;
        const long long base = block_excl_scan_ll(mine, sh.sc, total_u);
        const double scale = ldexp(1.0, emin_eff - 150);
        const double total = static_cast<double>(total_u) * scale;
        const double target = canon * total + 0.0;
        const double tu = target / scale;
        // the first block whose inclusive prefix reaches the target
        long long run = base;
        for (int bb = b0; bb < b1; ++bb) {
            const long long ub =
                st[bb].emin != 0x7FFFFFFF ? static_cast<long long>(st[bb].units << (st[bb].emin - emin_eff)) : 0;
            if (static_cast<double>(run + ub) >= tu) {
                atomicMin(&sh.blk, bb);
                break;
            }
            run += ub;
        }
        __syncthreads();
        const int blk = sh.blk;
        if (blk < nbp) {
            // the exclusive prefix of that block, from the thread that holds it
            if (blk >= b0 && blk < b1) {
                long long r = base;
                for (int bb = b0; bb < blk; ++bb)
                    if (st[bb].emin != 0x7FFFFFFF)
                        r += static_cast<long long>(st[bb].units << (st[bb].emin - emin_eff));
                sh.base = r;
            }
            __syncthreads();
            // rows of that block: kPpRPT consecutive rows per thread, as the distance pass
            const int r0 = blk * kPpRows + tid * kPpRPT;
            long long uj[kPpRPT];
            long long ut = 0;
#pragma unroll
            for (int j = 0; j < kPpRPT; ++j) {
                uj[j] = r0 + j < T ? static_cast<long long>(pp_units(md[r0 + j], emin_eff)) : 0;
                ut += uj[j];
            }
            long long tot;
            long long rr = sh.base + block_excl_scan_ll(ut, sh.sc, tot);
#pragma unroll
            for (int j = 0; j < kPpRPT; ++j) {
                rr += uj[j];
                if (r0 + j < T && static_cast<double>(rr) >= tu) {
                    atomicMin(&sh.sel, r0 + j);
                    break;
                }
            }
        }
    } else if (tid == 0) {
        double tw = 0.0;
        for (int i = 0; i < T; ++i) tw += static_cast<double>(md[i]);
        const double target = canon * tw + 0.0;
        double cs = 0.0;
        int pick = 0;
        for (int i = 0; i < T; ++i) {
            cs += static_cast<double>(md[i]);
            if (cs >= target) {
                pick = i;
                break;
            }
        }
        sh.sel = pick;
    }
    __syncthreads();
    return sh.sel < T ? sh.sel : 0;
}

struct PpStep {
    int c;                       // launch index: pick c - 1, distances to it
    int nbp;                     // blocks per segment
    int nsub;                    // blocks per workgroup
    int first[4];                // the first row, per subspace
    double canon[4];             // canon of pick c - 1 (c >= 2), per subspace
    const float* md_in;          // [seg][T] minima of launch c - 1
    float* md_out;               // [seg][T]
    const PpBlock* st_in;        // [seg][nbp] statistics of launch c - 1
    PpBlock* st_out;
};

template <int DP>
__global__ __launch_bounds__(256) void km_pp_step_kernel(KmParams a, PpStep ps) {
    __shared__ __attribute__((aligned(16))) float cur[DP];
    __shared__ int s_e[2][4];
    __shared__ long long s_u[4];
    __shared__ PpShared sh;
    // one round of 256 rows at a padded stride
    constexpr int CH = DP / 8;   // 16-byte chunks per row
    extern __shared__ __attribute__((aligned(16))) pp_u32x4_t s_rows[];   // [256][CH + 1]
    const int nb = ps.nbp, c = ps.c, nsub = ps.nsub;
    const int seg = blockIdx.y, wb = blockIdx.x, tid = threadIdx.x;
    const int h = seg / a.P, p = seg % a.P;
    if (c - 1 >= a.k[p]) return;
    const bool dist = c < a.k[p];   // false: pick c - 1 is the segment's last
    if (!dist && wb != 0) return;
    const int T = a.T;
    const float* mdi = ps.md_in + static_cast<int64_t>(seg) * T;
    float* mdo = ps.md_out + static_cast<int64_t>(seg) * T;
    const uint16_t* xb = a.keys + static_cast<int64_t>(h) * a.hs + p * DP;
    const int blk0 = wb * nsub, blk1 = min(blk0 + nsub, nb);
    // Block bk: rows bk * kPpRows + 256 j + tid (j < kPpRPT) for the thread;
    // each round of 256 rows is loaded coalesced (consecutive lanes read
    // consecutive 16-byte chunks, so one wave instruction covers whole rows)
    // and staged in LDS, from which each thread takes its own row.  The first
    // block's previous minima and first round do not depend on the pick:
    // they are loaded before it.
    float prev[kPpRPT];
    pp_u32x4_t ld[CH];
    if (dist) {
        const int r0 = blk0 * kPpRows;
#pragma unroll
        for (int j = 0; j < kPpRPT; ++j) {   // c == 1: no distances yet (FLT_MAX)
            const int r = r0 + 256 * j + tid;
            prev[j] = (c > 1 && r < T) ? mdi[r] : 3.402823466e38f;
        }
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int f = tid + 256 * k, row = f / CH, ch = f % CH;
            const int r = min(r0 + row, T - 1);
            ld[k] = reinterpret_cast<const pp_u32x4_t*>(xb + static_cast<int64_t>(r) * a.ts)[ch];
        }
    }
    const int sel = c == 1 ? ps.first[p]
                           : pp_pick_row(mdi, ps.st_in + static_cast<int64_t>(seg) * nb, nb, T, ps.canon[p], sh);
    if (tid < CH) {
        const pp_u32x4_t v = reinterpret_cast<const pp_u32x4_t*>(xb + static_cast<int64_t>(sel) * a.ts)[tid];
        const float4 f0 = make_float4(bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y));
        const float4 f1 = make_float4(bf16_lo(v.z), bf16_hi(v.z), bf16_lo(v.w), bf16_hi(v.w));
        reinterpret_cast<float4*>(cur)[2 * tid] = f0;
        reinterpret_cast<float4*>(cur)[2 * tid + 1] = f1;
        if (wb == 0) {
            float4* dst = reinterpret_cast<float4*>(a.cent + (static_cast<int64_t>(seg) * a.kmax + c - 1) * DP);
            dst[2 * tid] = f0;
            dst[2 * tid + 1] = f1;
        }
    }
    if (!dist) return;
    const int w = tid >> 6;
    for (int bk = blk0; bk < blk1; ++bk) {
        const int r0 = bk * kPpRows;
        if (bk > blk0) {
#pragma unroll
            for (int j = 0; j < kPpRPT; ++j) {
                const int r = r0 + 256 * j + tid;
                prev[j] = (c > 1 && r < T) ? mdi[r] : 3.402823466e38f;
            }
        }
        float m[kPpRPT];
        int emin = 0x7FFFFFFF, emax = 0;
#pragma unroll
        for (int j = 0; j < kPpRPT; ++j) {
            if (j > 0 || bk > blk0) {
#pragma unroll
                for (int k = 0; k < CH; ++k) {
                    const int f = tid + 256 * k, row = f / CH, ch = f % CH;
                    const int r = min(r0 + 256 * j + row, T - 1);
                    ld[k] = reinterpret_cast<const pp_u32x4_t*>(xb + static_cast<int64_t>(r) * a.ts)[ch];
                }
                __syncthreads();   // the previous round's rows are read
            }
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                const int f = tid + 256 * k, row = f / CH, ch = f % CH;
                s_rows[row * (CH + 1) + ch] = ld[k];
            }
            __syncthreads();   // (and cur, before the first round)
            pp_u32x4_t v[CH];
#pragma unroll
            for (int k = 0; k < CH; ++k) v[k] = s_rows[tid * (CH + 1) + k];
            const int r = r0 + 256 * j + tid;
            const float d = l2_lanes8_bf16<DP>(v, cur);
            float mm = prev[j];
            if (d < mm) mm = d;
            m[j] = r < T ? mm : 0.0f;
            if (r < T) mdo[r] = mm;
            if (m[j] > 0.0f) {
                emin = min(emin, pp_exp(m[j]));
                emax = max(emax, pp_exp(m[j]));
            }
        }
        emin = wave_min_i(emin);
        emax = wave_max_i(emax);
        if (lane_id() == 0) {
            s_e[0][w] = emin;
            s_e[1][w] = emax;
        }
        __syncthreads();
        const int be = min(min(s_e[0][0], s_e[0][1]), min(s_e[0][2], s_e[0][3]));
        const int bx = max(max(s_e[1][0], s_e[1][1]), max(s_e[1][2], s_e[1][3]));
        unsigned long long u = 0;
        if (be != 0x7FFFFFFF) {
#pragma unroll
            for (int j = 0; j < kPpRPT; ++j) u += pp_units(m[j], be);
        }
        const long long us = wave_incl_scan_ll(static_cast<long long>(u));
        if (lane_id() == 63) s_u[w] = us;
        __syncthreads();
        if (tid == 0) {
            PpBlock o;
            o.units = static_cast<unsigned long long>(((s_u[0] + s_u[1]) + s_u[2]) + s_u[3]);
            o.emin = be;
            o.emax = bx;
            ps.st_out[static_cast<int64_t>(seg) * nb + bk] = o;
        }
    }
}

// The last pick c of every segment with k == c + 1 (c == 0: the first row)
// from the minima and statistics of launch c.
template <int DP>
__global__ __launch_bounds__(256) void km_pp_pick_kernel(KmParams a, PpStep ps) {
    __shared__ PpShared sh;
    const int seg = blockIdx.x, tid = threadIdx.x;
    const int h = seg / a.P, p = seg % a.P;
    const int c = ps.c;
    if (c >= a.k[p]) return;
    const int T = a.T, nb = ps.nbp;
    const uint16_t* xb = a.keys + static_cast<int64_t>(h) * a.hs + p * DP;
    const int sel = c == 0 ? ps.first[p]
                           : pp_pick_row(ps.md_in + static_cast<int64_t>(seg) * T,
                                         ps.st_in + static_cast<int64_t>(seg) * nb, nb, T, ps.canon[p], sh);
    float* dst = a.cent + (static_cast<int64_t>(seg) * a.kmax + c) * DP;
    for (int d = tid; d < DP; d += 256) dst[d] = bf16_to_f32(xb[static_cast<int64_t>(sel) * a.ts + d]);
}

// Per segment: exclusive scan of the [label][block] counts, cluster offsets,
// empty-cluster ordinals, inertia (fixed reduction order) and the early-stop
// test of kmeans_core.cpp:244-262.  Up to 64 counts per thread (k * nblk <=
// 65536, 16-byte aligned) stay in registers: one read, one write, and the
// cluster offsets come from the threads that hold them; larger segments use
// the two-pass block scan.
constexpr int kScanRegInts = 64;

__global__ __launch_bounds__(1024) void km_scan_kernel(KmParams a, int it) {
    __shared__ int sh[40];
    __shared__ int soff[kIvfMaxK + 1];
    __shared__ float sred[16];
    __shared__ int stop;
    const int seg = blockIdx.x;
    if (a.done && a.done[seg]) return;
    const int p = seg % a.P;
    const int k = a.k[p];
    const int tid = threadIdx.x, wave = tid >> 6;
    int32_t* hist = a.hist + static_cast<int64_t>(seg) * a.kmax * a.nblk;
    const int n = k * a.nblk;
    const bool reg = n <= 1024 * kScanRegInts && (n & 3) == 0 && (reinterpret_cast<uintptr_t>(hist) & 15) == 0;
    // this thread's counts: a contiguous run of `per` (multiple of 4) ints
    int per = (n + 1023) / 1024;
    per = (per + 3) & ~3;
    const int lo = min(tid * per, n), hi = min(lo + per, n);
    typedef int __attribute__((ext_vector_type(4))) i32x4;
    i32x4 v[kScanRegInts / 4];
    if (reg) {
#pragma unroll
        for (int u = 0; u < kScanRegInts / 4; ++u)
            v[u] = lo + 4 * u < hi ? *reinterpret_cast<const i32x4*>(hist + lo + 4 * u) : i32x4{0, 0, 0, 0};
    }
    // inertia partials: contiguous chunk per thread, then waves in order
    const float* ip = a.ipart + static_cast<int64_t>(seg) * a.nblk;
    const int iper = (a.nblk + 1023) / 1024;
    float part = 0.0f;
    for (int b = tid * iper; b < (tid + 1) * iper && b < a.nblk; ++b) part += ip[b];
    part = wave_sum(part);
    if ((tid & 63) == 0) sred[wave] = part;
    int32_t* off = a.off + static_cast<int64_t>(seg) * (a.kmax + 1);
    if (reg) {
        int local = 0;
#pragma unroll
        for (int u = 0; u < kScanRegInts / 4; ++u) local += (v[u][0] + v[u][1]) + (v[u][2] + v[u][3]);
        const int incl = wave_incl_scan(local);
        if ((tid & 63) == 63) sh[wave] = incl;
        __syncthreads();
        if (tid < 64) {
            const int x = tid < 16 ? sh[tid] : 0;
            const int sc = wave_incl_scan(x);
            if (tid < 16) sh[16 + tid] = sc - x;
        }
        __syncthreads();
        const int run0 = sh[16 + wave] + incl - local;
        // cluster offsets: the label boundaries c * nblk inside [lo, hi)
        for (int c = (lo + a.nblk - 1) / a.nblk; c < k && c * a.nblk < hi; ++c) {
            const int at = c * a.nblk - lo;
            int sum = run0;
#pragma unroll
            for (int u = 0; u < kScanRegInts / 4; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) sum += 4 * u + e < at ? v[u][e] : 0;
            off[c] = sum;
            soff[c] = sum;
        }
        int run = run0;
#pragma unroll
        for (int u = 0; u < kScanRegInts / 4; ++u) {
            if (lo + 4 * u < hi) {
                i32x4 o;
                o[0] = run;
                run += v[u][0];
                o[1] = run;
                run += v[u][1];
                o[2] = run;
                run += v[u][2];
                o[3] = run;
                run += v[u][3];
                *reinterpret_cast<i32x4*>(hist + lo + 4 * u) = o;
            }
        }
    } else {
        block_exclusive_scan_1024(hist, static_cast<int64_t>(n), sh);
        for (int c = tid; c < k; c += 1024) {
            const int o = hist[static_cast<int64_t>(c) * a.nblk];
            off[c] = o;
            soff[c] = o;
        }
    }
    if (tid == 0) {
        off[k] = a.T;
        soff[k] = a.T;
    }
    __syncthreads();
    // empty-cluster ordinals: exclusive count of empty clusters before c,
    // 256 clusters at a time on the first four waves
    for (int c0 = 0, carry = 0; c0 < k; c0 += 256) {
        const int c = c0 + tid;
        int empty = 0, eincl = 0;
        if (wave < 4) {
            empty = c < k && soff[c + 1] == soff[c] ? 1 : 0;
            eincl = wave_incl_scan(empty);
            if ((tid & 63) == 63) sh[32 + wave] = eincl;
        }
        __syncthreads();
        if (wave < 4 && c < k) {
            int before = carry;
            for (int w = 0; w < wave; ++w) before += sh[32 + w];
            a.empties[static_cast<int64_t>(seg) * a.kmax + c] = before + eincl - empty;
        }
        carry += (sh[32] + sh[33]) + (sh[34] + sh[35]);
        __syncthreads();
    }
    if (tid == 0) {
        float inertia = 0.0f;
        for (int w = 0; w < 16; ++w) inertia += sred[w];
        if (a.iters) a.iters[seg] = it + 1;
        const float prev = a.prev[seg];
        const float change = fabsf(prev - inertia);
        const float rel = prev > 0.0f ? change / prev : 0.0f;
        const bool min_ok = (it + 1) >= (a.es_min > 1 ? a.es_min : 1);
        stop = min_ok && (rel <= fmaxf(0.0f, a.es_rel) || change <= fmaxf(0.0f, a.tol));
        if (!stop) a.prev[seg] = inertia;
    }
    __syncthreads();
    if (tid == 0 && stop && a.done) a.done[seg] = 1;
}

// Member lists: token t of block b goes to the scanned [label][block] offset
// plus its rank in the block.  Each thread takes one token of each of
// kScatterBlocks consecutive blocks, so all its loads are in flight together.
constexpr int kScatterBlocks = 4;

__global__ __launch_bounds__(256) void km_scatter_kernel(KmParams a) {
    const int seg = blockIdx.y;
    if (a.done && a.done[seg]) return;
    const int64_t so = static_cast<int64_t>(seg) * a.T;
    const int32_t* hist = a.hist + static_cast<int64_t>(seg) * a.kmax * a.nblk;
    int lab[kScatterBlocks], rnk[kScatterBlocks];
#pragma unroll
    for (int u = 0; u < kScatterBlocks; ++u) {
        const int t = (blockIdx.x * kScatterBlocks + u) * 256 + threadIdx.x;
        const bool in = t < a.T;
        lab[u] = in ? a.labels[so + t] : 0;
        rnk[u] = in ? a.rank[so + t] : 0;
    }
    int base[kScatterBlocks];
#pragma unroll
    for (int u = 0; u < kScatterBlocks; ++u) {
        const int blk = blockIdx.x * kScatterBlocks + u;
        base[u] = blk < a.nblk ? hist[static_cast<int64_t>(lab[u]) * a.nblk + blk] : 0;
    }
#pragma unroll
    for (int u = 0; u < kScatterBlocks; ++u) {
        const int t = (blockIdx.x * kScatterBlocks + u) * 256 + threadIdx.x;
        if (t < a.T) a.sorted[so + base[u] + rnk[u]] = t;
    }
}

// M-step, one workgroup per cluster: wave 0 keeps the chains (lane d =
// dimension d, members in ascending token order, one dependent fp32 add
// each) while waves 1..3 gather the member rows, so a large cluster streams
// with three waves' worth of loads in flight.  Batch b (64 rows) belongs to
// loader 1 + b % 3 as its local batch b / 3; round q hands batches 3q ..
// 3q+2 over through one of two sets of LDS slots (the loaders fill round
// q+1 while wave 0 sums round q), one barrier per round.  Each loader keeps
// NB local batches in flight in a register ring and loads the member ids 2 NB
// local batches ahead.
template <int DP>
__global__ __launch_bounds__(256) void km_update_block_kernel(KmParams a, Draws draws) {
    constexpr int PARTS = DP / 8;    // 16-byte parts per row
    constexpr int RPL = 64 / PARTS;  // rows per load instruction
    constexpr int LPB = PARTS;       // load instructions per 64-row batch
    constexpr int NL = 3;            // loader waves
    // local batches in flight per loader (register ring).  Two: every
    // workgroup fills its ring at the start, and with four the burst (~75 MB
    // at configs[1]) delayed the first rounds of the largest clusters, whose
    // chains set the kernel's length (79.9 -> 71.4 us per M-step).
    constexpr int NB = 2;
    constexpr int HALVES = DP > 64 ? DP / 64 : 1;   // dims per chain lane
    __shared__ km_u32x4_t ring[2 * NL][64 * PARTS];
    // block member lists: the label's exclusive prefix over the blocks, its
    // first place in each block, the waves' member counts
    __shared__ int s_pref[kLocalMaxBlk];
    __shared__ int s_lof[kLocalMaxBlk];
    __shared__ int s_wt[4];
    const int c = blockIdx.x, seg = blockIdx.y;
    const int h = seg / a.P, p = seg % a.P;
    if (c >= a.k[p]) return;
    if (a.done && a.done[seg]) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint16_t* kbase = a.keys + h * a.hs + p * DP;
    float* dst = a.cent + (static_cast<int64_t>(seg) * a.kmax + c) * DP;
    const bool local = a.loff != nullptr;
    int lo = 0, n = 0;
    if (local) {
        // this label's first place and count in every block (nblk <= 512:
        // two blocks per thread, their offset pairs loaded together), then
        // the prefix of the counts
        const int32_t* rows = a.loff + static_cast<int64_t>(seg) * a.nblk * (a.kmax + 1) + c;
        int cv[kLocalMaxBlk / 256], lv[kLocalMaxBlk / 256];
#pragma unroll
        for (int u = 0; u < kLocalMaxBlk / 256; ++u) {
            const int b = min(2 * tid + u, a.nblk - 1);
            lv[u] = rows[static_cast<int64_t>(b) * (a.kmax + 1)];
            cv[u] = rows[static_cast<int64_t>(b) * (a.kmax + 1) + 1];
        }
#pragma unroll
        for (int u = 0; u < kLocalMaxBlk / 256; ++u) cv[u] = 2 * tid + u < a.nblk ? cv[u] - lv[u] : 0;
        const int run = cv[0] + cv[1];
        const int incl = wave_incl_scan(run);
        if (lane == 63) s_wt[wave] = incl;
        __syncthreads();
        int before = incl - run;
        for (int w = 0; w < wave; ++w) before += s_wt[w];
        if (2 * tid < a.nblk) {
            s_pref[2 * tid] = before;
            s_lof[2 * tid] = lv[0];
        }
        if (2 * tid + 1 < a.nblk) {
            s_pref[2 * tid + 1] = before + cv[0];
            s_lof[2 * tid + 1] = lv[1];
        }
        __syncthreads();
        n = (s_wt[0] + s_wt[1]) + (s_wt[2] + s_wt[3]);
    } else {
        const int32_t* off = a.off + static_cast<int64_t>(seg) * (a.kmax + 1);
        lo = off[c];
        n = off[c + 1] - lo;
    }
    if (n == 0) {
        int e;
        if (local) {
            // the empty ordinal: labels below c whose block counts are all zero
            // (every thread sums one label's column, in parallel over labels)
            __shared__ int s_emp;
            if (tid == 0) s_emp = 0;
            __syncthreads();
            for (int c2 = tid; c2 < c; c2 += 256) {
                const int32_t* r2 = a.loff + static_cast<int64_t>(seg) * a.nblk * (a.kmax + 1) + c2;
                int sum = 0;
                for (int b = 0; b < a.nblk; ++b) sum += r2[static_cast<int64_t>(b) * (a.kmax + 1) + 1] - r2[static_cast<int64_t>(b) * (a.kmax + 1)];
                if (sum == 0) atomicAdd(&s_emp, 1);
            }
            __syncthreads();
            e = s_emp;
        } else {
            e = a.empties[static_cast<int64_t>(seg) * a.kmax + c];   // past this launch's draws: km_reseed_kernel
        }
        if (wave == 0 && e < kDraws) {
            const int tok = draws.v[e];
            for (int d = lane; d < DP; d += 64) dst[d] = bf16_to_f32(kbase[static_cast<int64_t>(tok) * a.ts + d]);
        }
        return;
    }
    const int nb = (n + 63) >> 6;              // 64-row batches
    const int rounds = (nb + NL - 1) / NL;     // = local batches of loader 1
    const int32_t* srt = a.sorted + static_cast<int64_t>(seg) * a.T + lo;
    const int32_t* lst = a.rank + static_cast<int64_t>(seg) * a.T;
    // member j: the block holding it (the last one whose prefix is <= j) and
    // its place there
    auto member = [&](int j) {
        if (!local) return srt[j];
        int b = 0;
#pragma unroll
        for (int step = kLocalMaxBlk / 2; step > 0; step >>= 1)
            b = (b + step < a.nblk && s_pref[b + step] <= j) ? b + step : b;
        return lst[b * 256 + s_lof[b] + (j - s_pref[b])];
    };
    // rounds padded to whole ring cycles: the loaders' loop body is then free
    // of branches, so the compiler's wait before each slot write counts the
    // loads issued since that batch's (a branch around a load makes it assume
    // the fewest, which waited for nearly every load and left one batch in
    // flight).  Padding rounds re-read the last member's row (L2-resident)
    // and are not summed.
    const int rounds_pad = (rounds + NB - 1) / NB * NB;
    if (wave > 0) {
        const int lw = wave - 1;
        const int part = lane % PARTS, rsub = lane / PARTS;
        // member ids of local batch q (global batch NL q + lw); past n the
        // last member again (a valid row, never summed: the chain adds only
        // the first n).  No select on the loaded id: one would make the
        // compiler wait for each id load right after issuing it.
#define KMB_ID(q) member(min((NL * (q) + lw) * 64 + lane, n - 1))
#define KMB_ROWS(idv, slot)                                                                            \
    _Pragma("unroll") for (int u = 0; u < LPB; ++u) {                                                \
        const int id_ = __shfl((idv), u * RPL + rsub);                                               \
        rr[slot][u] = *reinterpret_cast<const km_u32x4_t*>(kbase + static_cast<int64_t>(id_) * a.ts + part * 8); \
    }
        // rows of local batches 0 .. NB-1 in the register ring, ids of
        // NB .. 2NB-1 in the id ring; round q writes batch q, loads the rows
        // of q + NB and the ids of q + 2NB
        // (the prologue issues its loads in the loop's order -- slot j's rows,
        // then slot j's next ids -- so the waits inside the loop are the same
        // on entry and on the back edge)
        int idr[NB], id0[NB];
        km_u32x4_t rr[NB][LPB];
#pragma unroll
        for (int j = 0; j < NB; ++j) id0[j] = KMB_ID(j);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            KMB_ROWS(id0[j], j)
            idr[j] = KMB_ID(NB + j);
            __builtin_amdgcn_sched_barrier(0);   // keep this order (no reordering of the loads)
        }
#pragma unroll 1
        for (int q0 = 0; q0 < rounds_pad; q0 += NB) {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int q = q0 + j;
                km_u32x4_t* slot = ring[(q & 1) * NL + lw];
#pragma unroll
                for (int u = 0; u < LPB; ++u) slot[(u * RPL + rsub) * PARTS + part] = rr[j][u];
                KMB_ROWS(idr[j], j)
                idr[j] = KMB_ID(q + 2 * NB);
                __syncthreads();
            }
        }
#undef KMB_ID
#undef KMB_ROWS
    } else {
        float acc[HALVES];
#pragma unroll
        for (int hh = 0; hh < HALVES; ++hh) acc[hh] = 0.0f;
#pragma unroll 1
        for (int q = 0; q < rounds_pad; ++q) {
            __syncthreads();   // round q's slots are filled
            if (q >= rounds) continue;
            if (HALVES == 1 && NL * 64 * (q + 1) <= n) {
                // a full round (three batches of 64 members): the next batch's
                // reads are issued before the current batch's additions, and
                // the widening of value j + 1 is scheduled between the adds of
                // j - 1 and j, so no add waits on the instruction before it
                const int lg = lane >> 4, ln = lane & 15;
                const int boff = (ln >> 2) * DP + 16 * (lg % (DP / 16)) + 4 * (ln & 3);
                km_u32x2_t w[2][16];
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    w[0][i] = __builtin_bit_cast(
                        km_u32x2_t,
                        __builtin_amdgcn_ds_read_tr16_b64_v4i16((km_lds_s16x4_t*)(reinterpret_cast<const uint16_t*>(
                                                                    ring[(q & 1) * NL]) + boff + 4 * i * DP)));
#pragma unroll
                for (int lw = 0; lw < NL; ++lw) {
                    if (lw + 1 < NL) {
#pragma unroll
                        for (int i = 0; i < 16; ++i)
                            w[(lw + 1) & 1][i] = __builtin_bit_cast(
                                km_u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                (km_lds_s16x4_t*)(reinterpret_cast<const uint16_t*>(
                                                                      ring[(q & 1) * NL + lw + 1]) + boff + 4 * i * DP)));
                    }
                    float f[64];
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        f[4 * i] = __uint_as_float(w[lw & 1][i][0] << 16);
                        f[4 * i + 1] = __uint_as_float(w[lw & 1][i][0] & 0xFFFF0000u);
                        f[4 * i + 2] = __uint_as_float(w[lw & 1][i][1] << 16);
                        f[4 * i + 3] = __uint_as_float(w[lw & 1][i][1] & 0xFFFF0000u);
                    }
#pragma unroll
                    for (int j = 0; j < 64; ++j) acc[0] = acc[0] + f[j];
                }
                continue;
            }
#pragma unroll
            for (int lw = 0; lw < NL; ++lw) {
                const int b = NL * q + lw;
                if (b < nb) {
                    const uint16_t* rows = reinterpret_cast<const uint16_t*>(ring[(q & 1) * NL + lw]);
                    const int cnt = (n - 64 * b) < 64 ? (n - 64 * b) : 64;
                    if (cnt == 64) {
                        // transposing reads: 16-lane group g takes the 4 x 16
                        // block of members 4i..4i+3, dims 16 (g % (DP/16)) ..
                        // +15, so lane d holds dim d of four consecutive
                        // members per read (lanes >= DP read a copy and are
                        // not stored); all 16 reads in flight at once.  DP =
                        // 128: a second pass over dims 64..127.
                        const int lg = lane >> 4, ln = lane & 15;
#pragma unroll
                        for (int hh = 0; hh < HALVES; ++hh) {
                            const uint16_t* base =
                                rows + (ln >> 2) * DP + 64 * hh + 16 * (lg % (DP / 16)) + 4 * (ln & 3);
                            km_u32x2_t w[16];
#pragma unroll
                            for (int i = 0; i < 16; ++i)
                                w[i] = __builtin_bit_cast(
                                    km_u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                    (km_lds_s16x4_t*)(base + 4 * i * DP)));
#pragma unroll
                            for (int i = 0; i < 16; ++i) {
                                acc[hh] = acc[hh] + __uint_as_float(w[i][0] << 16);
                                acc[hh] = acc[hh] + __uint_as_float(w[i][0] & 0xFFFF0000u);
                                acc[hh] = acc[hh] + __uint_as_float(w[i][1] << 16);
                                acc[hh] = acc[hh] + __uint_as_float(w[i][1] & 0xFFFF0000u);
                            }
                        }
                    } else {
#pragma unroll
                        for (int hh = 0; hh < HALVES; ++hh)
                            if (64 * hh + lane < DP)
                                for (int r = 0; r < cnt; ++r)
                                    acc[hh] = acc[hh] + bf16_to_f32(rows[r * DP + 64 * hh + lane]);
                    }
                }
            }
        }
#pragma unroll
        for (int hh = 0; hh < HALVES; ++hh)
            if (64 * hh + lane < DP) dst[64 * hh + lane] = acc[hh] * (1.0f / static_cast<float>(n));
    }
}

// Empty clusters whose ordinal falls in [e0, e0 + kDraws): the draws of
// that slice (clusters beyond kDraws empty ones only occur when k > kDraws).
__global__ __launch_bounds__(64) void km_reseed_kernel(KmParams a, Draws draws, int e0) {
    const int c = blockIdx.x, seg = blockIdx.y;
    const int h = seg / a.P, p = seg % a.P;
    if (c >= a.k[p]) return;
    if (a.done && a.done[seg]) return;
    const int32_t* off = a.off + static_cast<int64_t>(seg) * (a.kmax + 1);
    if (off[c + 1] != off[c]) return;
    const int e = a.empties[static_cast<int64_t>(seg) * a.kmax + c] - e0;
    if (e < 0 || e >= kDraws) return;
    const uint16_t* row = a.keys + h * a.hs + p * a.DP + static_cast<int64_t>(draws.v[e]) * a.ts;
    float* dst = a.cent + (static_cast<int64_t>(seg) * a.kmax + c) * a.DP;
    for (int d = threadIdx.x; d < a.DP; d += 64) dst[d] = bf16_to_f32(row[d]);
}

__global__ void km_reset_kernel(KmParams a) {
    const int seg = blockIdx.x * blockDim.x + threadIdx.x;
    if (seg >= a.H * a.P) return;
    a.prev[seg] = 3.402823466e38f;
    if (a.done) a.done[seg] = 0;
    if (a.iters) a.iters[seg] = a.loff ? a.max_iters : 0;   // no km_scan counts them without early stop
}

int validate(const imi_kmeans_args* a, int& kmax, int& dp) {
    IMI_REQUIRE(a != nullptr, IMI_ERR_INVALID, "imi_kmeans: null args");
    IMI_REQUIRE(a->keys && a->centroids && a->labels, IMI_ERR_INVALID, "imi_kmeans: null pointer argument");
    IMI_REQUIRE(a->kv_heads > 0 && a->n_tokens > 0, IMI_ERR_INVALID, "imi_kmeans: empty input (H=%d T=%d)",
                a->kv_heads, a->n_tokens);
    IMI_REQUIRE(a->parts == 1 || a->parts == 2 || a->parts == 4, IMI_ERR_UNSUPPORTED,
                "imi_kmeans: parts must be 1 (IVF), 2 or 4 (got %d)", a->parts);
    IMI_REQUIRE(a->dim % a->parts == 0, IMI_ERR_INVALID, "imi_kmeans: dim %d not divisible by parts %d", a->dim,
                a->parts);
    dp = a->dim / a->parts;
    IMI_REQUIRE(dp == 32 || dp == 64 || (a->parts == 1 && dp == 128), IMI_ERR_UNSUPPORTED,
                "imi_kmeans: subspace width %d unsupported (32 or 64; 128 for IVF)", dp);
    IMI_REQUIRE(a->max_iters >= 1, IMI_ERR_INVALID, "imi_kmeans: max_iters must be >= 1");
    const int kcap = a->parts == 1 ? kIvfMaxK : kImiMaxK;
    kmax = 0;
    for (int p = 0; p < a->parts; ++p) {
        IMI_REQUIRE(a->k[p] >= 1 && a->k[p] <= kcap, IMI_ERR_UNSUPPORTED, "imi_kmeans: k[%d]=%d outside [1,%d]", p,
                    a->k[p], kcap);
        kmax = a->k[p] > kmax ? a->k[p] : kmax;
    }
    IMI_REQUIRE(a->init_mode >= 0 && a->init_mode <= 2, IMI_ERR_INVALID,
                "imi_kmeans: init_mode %d (0 first-k, 1 given, 2 kmeans++)", a->init_mode);
    if (a->init_mode == 0)
        IMI_REQUIRE(kmax <= a->n_tokens, IMI_ERR_INVALID,
                    "imi_kmeans: first-k initialisation needs n_tokens (%d) >= k (%d)", a->n_tokens, kmax);
    IMI_REQUIRE((a->token_stride % 8) == 0 && (a->head_stride % 8) == 0, IMI_ERR_INVALID,
                "imi_kmeans: strides must be multiples of 8 elements (16-byte rows)");
    IMI_REQUIRE((reinterpret_cast<uintptr_t>(a->keys) & 15) == 0, IMI_ERR_INVALID,
                "imi_kmeans: keys must be 16-byte aligned");
    return IMI_OK;
}

size_t workspace_bytes(const imi_kmeans_args* a, int kmax, KmParams* out) {
    const int segs = a->kv_heads * a->parts;
    const int nblk = (a->n_tokens + 255) / 256;
    Carver cv(a->workspace);
    KmParams p{};
    p.hist = cv.take<int32_t>(static_cast<size_t>(segs) * kmax * nblk);
    p.rank = cv.take<int32_t>(static_cast<size_t>(segs) * a->n_tokens);
    p.ipart = cv.take<float>(static_cast<size_t>(segs) * nblk);
    p.sorted = cv.take<int32_t>(static_cast<size_t>(segs) * a->n_tokens);
    p.off = cv.take<int32_t>(static_cast<size_t>(segs) * (kmax + 1));
    p.empties = cv.take<int32_t>(static_cast<size_t>(segs) * kmax);
    p.prev = cv.take<float>(segs);
    p.done = cv.take<int32_t>(segs);
    p.loff = cv.take<int32_t>(static_cast<size_t>(segs) * nblk * (kmax + 1));
    if (a->init_mode == 2) {
        const int nbp = (a->n_tokens + kPpRows - 1) / kPpRows;
        PpBlock* st = cv.take<PpBlock>(static_cast<size_t>(2) * segs * nbp);   // two launches' worth
        if (out) p.ppstats = st;
    }
    if (out) *out = p;
    return cv.used();
}

template <int DP, int MAXK, int KT, bool EXACT>
int launch_screen(const KmParams& p, int segs, hipStream_t stream) {
    const size_t lds = screen_lds_bytes<DP>(p.kmax);
    const void* fn = reinterpret_cast<const void*>(&km_assign_screen_kernel<DP, MAXK, KT, EXACT>);
    if (lds > 64 * 1024)
        IMI_HIP_CHECK(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    // as many workgroups as fit on the device at once, each over `chunks`
    // consecutive 256-token blocks
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, km_assign_screen_kernel<DP, MAXK, KT, EXACT>, 256,
                                                     lds) != hipSuccess ||
        per_cu <= 0)
        per_cu = 1;
    const int64_t want = static_cast<int64_t>(per_cu) * device_cus();
    const int chunks = static_cast<int>(std::max<int64_t>(1, (static_cast<int64_t>(p.nblk) * segs + want - 1) / want));
    const int gx = (p.nblk + chunks - 1) / chunks;
    hipLaunchKernelGGL((km_assign_screen_kernel<DP, MAXK, KT, EXACT>), dim3(gx, segs), dim3(256), lds, stream, p,
                       chunks);
    IMI_LAUNCH_CHECK("km_assign_screen_kernel");
    return IMI_OK;
}

// EXACT: the distances are read (min distances or the early-stop inertia)
template <int DP, int MAXK, int KT>
int run_screen(const KmParams& p, int segs, hipStream_t stream) {
    return p.exact ? launch_screen<DP, MAXK, KT, true>(p, segs, stream)
                   : launch_screen<DP, MAXK, KT, false>(p, segs, stream);
}

template <int DP>
int run_assign(const KmParams& p, int segs, hipStream_t stream) {
    if constexpr (DP == 128) {
        const size_t lds = tiled_lds_bytes<DP>(p.kmax);
        if (lds > 64 * 1024)
            IMI_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&km_assign_tiled_kernel<DP>),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        hipLaunchKernelGGL(km_assign_tiled_kernel<DP>, dim3(p.nblk, segs), dim3(256), lds, stream, p);
        IMI_LAUNCH_CHECK("km_assign_tiled_kernel");
        return IMI_OK;
    } else if (p.kmax <= kScreenMaxK) {
        bool same = true;   // every subspace has kmax centroids
        for (int q = 0; q < p.P; ++q) same = same && p.k[q] == p.kmax;
        if (same) {
            switch (p.kmax) {
                case 16: return run_screen<DP, 64, 1>(p, segs, stream);
                case 32: return run_screen<DP, 64, 2>(p, segs, stream);
                case 64: return run_screen<DP, 64, 4>(p, segs, stream);
                case 128: return run_screen<DP, kScreenMaxK, 8>(p, segs, stream);
                default: break;
            }
        }
        return p.kmax <= 64 ? run_screen<DP, 64, 0>(p, segs, stream) : run_screen<DP, kScreenMaxK, 0>(p, segs, stream);
    }
    const size_t lds = static_cast<size_t>(p.kmax) * DP * sizeof(float) + 4 * p.kmax * sizeof(int) + 64;
    if (lds > 64 * 1024) IMI_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&km_assign_kernel<DP>),
                                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                                           static_cast<int>(lds)));
    hipLaunchKernelGGL(km_assign_kernel<DP>, dim3(p.nblk, segs), dim3(256), lds, stream, p);
    IMI_LAUNCH_CHECK("km_assign_kernel");
    return IMI_OK;
}

}  // namespace
}  // namespace imi

using namespace imi;

extern "C" int imi_kmeans_workspace_size(const imi_kmeans_args* a, size_t* bytes) {
    clear_error();
    int kmax, dp;
    int rc = validate(a, kmax, dp);
    if (rc) return rc;
    IMI_REQUIRE(bytes != nullptr, IMI_ERR_INVALID, "imi_kmeans_workspace_size: null output");
    imi_kmeans_args tmp = *a;
    tmp.workspace = nullptr;
    *bytes = workspace_bytes(&tmp, kmax, nullptr);
    return IMI_OK;
}

extern "C" int imi_kmeans_execute(const imi_kmeans_args* a, imi_stream_t stream_) {
    clear_error();
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    int kmax, dp;
    int rc = validate(a, kmax, dp);
    if (rc) return rc;
    imi_kmeans_args tmp = *a;
    tmp.workspace = nullptr;
    const size_t need = workspace_bytes(&tmp, kmax, nullptr);
    IMI_REQUIRE(a->workspace != nullptr && a->workspace_bytes >= need, IMI_ERR_WORKSPACE,
                "imi_kmeans_execute: workspace %zu bytes < %zu required", a->workspace_bytes, need);

    KmParams p;
    workspace_bytes(a, kmax, &p);
    p.keys = a->keys;
    p.hs = a->head_stride;
    p.ts = a->token_stride;
    p.H = a->kv_heads;
    p.T = a->n_tokens;
    p.P = a->parts;
    p.kmax = kmax;
    p.DP = dp;
    for (int i = 0; i < 4; ++i) p.k[i] = i < a->parts ? a->k[i] : 0;
    p.cent = a->centroids;
    p.labels = a->labels;
    p.mind = nullptr;
    p.iters = a->iters_run;
    p.nblk = (a->n_tokens + 255) / 256;
    p.max_iters = a->max_iters;
    p.tol = a->tol;
    p.es_min = a->early_stop_min_iter;
    p.es_rel = a->early_stop_rel_tol;
    const int segs = a->kv_heads * a->parts;
    const bool early_stop = a->early_stop_min_iter <= a->max_iters;
    if (!early_stop) p.done = nullptr;  // no test can fire: skip the flag reads
    // Block member lists instead of km_scan + km_scatter: without early stop
    // (nothing reads the inertia), with the screened E-step (subspaces of at
    // most 64 dims, k <= 128) and at most kLocalMaxBlk blocks.
    const bool local = !early_stop && dp <= 64 && kmax <= kScreenMaxK && p.nblk <= kLocalMaxBlk;
    if (!local) p.loff = nullptr;

    hipLaunchKernelGGL(km_reset_kernel, dim3((segs + 63) / 64), dim3(64), 0, stream, p);
    IMI_LAUNCH_CHECK("km_reset_kernel");
    if (a->init_mode == 0) {
        hipLaunchKernelGGL(km_init_first_kernel, dim3(kmax, segs), dim3(64), 0, stream, p);
        IMI_LAUNCH_CHECK("km_init_first_kernel");
    } else if (a->init_mode == 2) {
        // kmeans++ seeds 42, 43, 44, 45 by subspace, the same for every head
        // (kmeans_core.cpp:459, 469; IVF: seed 42, kmeans_core.cpp:548-556);
        // every segment's pick c in one pair of launches
        PpStep ps{};
        std::vector<double> canon[4];
        for (int part = 0; part < a->parts; ++part) {
            std::mt19937_64 rng(static_cast<uint64_t>(42 + part));
            std::uniform_int_distribution<int32_t> first(0, a->n_tokens - 1);
            ps.first[part] = first(rng);
            canon[part].assign(a->k[part], 0.0);
            for (int c = 1; c < a->k[part]; ++c)
                canon[part][c] = std::generate_canonical<double, std::numeric_limits<double>::digits>(rng);
        }
        const int nbp = (a->n_tokens + kPpRows - 1) / kPpRows;
        ps.nbp = nbp;
        PpBlock* st = static_cast<PpBlock*>(p.ppstats);
        // minima and statistics alternate between two buffers (the member
        // lists' `rank` and `sorted`, free until the first E-step)
        float* md[2] = {reinterpret_cast<float*>(p.rank), reinterpret_cast<float*>(p.sorted)};
        PpBlock* sts[2] = {st, st + static_cast<size_t>(segs) * nbp};
        const size_t lds = static_cast<size_t>(256) * (dp / 8 + 1) * 16;
        if (dp == 128)   // 68 KB of LDS per workgroup
            IMI_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&km_pp_step_kernel<128>),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        // one resident round of workgroups, each over nsub consecutive blocks
        int per_cu = 0;
        const void* fn = dp == 128 ? reinterpret_cast<const void*>(&km_pp_step_kernel<128>)
                                   : (dp == 64 ? reinterpret_cast<const void*>(&km_pp_step_kernel<64>)
                                               : reinterpret_cast<const void*>(&km_pp_step_kernel<32>));
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, lds) != hipSuccess || per_cu <= 0)
            per_cu = 1;
        const int64_t want = static_cast<int64_t>(per_cu) * device_cus();
        ps.nsub = static_cast<int>(std::max<int64_t>(1, (static_cast<int64_t>(nbp) * segs + want - 1) / want));
        const int nbw = (nbp + ps.nsub - 1) / ps.nsub;
        // launch c (1 <= c < kmax): pick c - 1 and the distances to it
        for (int c = 1; c < kmax; ++c) {
            ps.c = c;
            for (int part = 0; part < a->parts; ++part)
                ps.canon[part] = c - 1 >= 1 && c - 1 < a->k[part] ? canon[part][c - 1] : 0.0;
            ps.md_in = md[(c - 1) & 1];
            ps.md_out = md[c & 1];
            ps.st_in = sts[(c - 1) & 1];
            ps.st_out = sts[c & 1];
            const dim3 grid(nbw, segs);
            if (dp == 128)
                hipLaunchKernelGGL(km_pp_step_kernel<128>, grid, dim3(256), lds, stream, p, ps);
            else if (dp == 64)
                hipLaunchKernelGGL(km_pp_step_kernel<64>, grid, dim3(256), lds, stream, p, ps);
            else
                hipLaunchKernelGGL(km_pp_step_kernel<32>, grid, dim3(256), lds, stream, p, ps);
            IMI_LAUNCH_CHECK("km_pp_step_kernel");
        }
        // the last pick of the segments with kmax centroids
        const int c = kmax - 1;
        ps.c = c;
        for (int part = 0; part < a->parts; ++part) ps.canon[part] = c >= 1 && c < a->k[part] ? canon[part][c] : 0.0;
        ps.md_in = md[c & 1];
        ps.st_in = sts[c & 1];
        ps.md_out = nullptr;
        ps.st_out = nullptr;
        if (dp == 128)
            hipLaunchKernelGGL(km_pp_pick_kernel<128>, dim3(segs), dim3(256), 0, stream, p, ps);
        else if (dp == 64)
            hipLaunchKernelGGL(km_pp_pick_kernel<64>, dim3(segs), dim3(256), 0, stream, p, ps);
        else
            hipLaunchKernelGGL(km_pp_pick_kernel<32>, dim3(segs), dim3(256), 0, stream, p, ps);
        IMI_LAUNCH_CHECK("km_pp_pick_kernel");
    }
    for (int it = 0; it < a->max_iters; ++it) {
        // the inertia of iteration it enters the stop tests of it and it + 1
        p.exact = early_stop && it + 2 >= std::max(a->early_stop_min_iter, 1) ? 1 : 0;
        rc = dp == 128 ? run_assign<128>(p, segs, stream)
                       : (dp == 64 ? run_assign<64>(p, segs, stream) : run_assign<32>(p, segs, stream));
        if (rc) return rc;
        if (!local) {
            hipLaunchKernelGGL(km_scan_kernel, dim3(segs), dim3(1024), 0, stream, p, it);
            IMI_LAUNCH_CHECK("km_scan_kernel");
            hipLaunchKernelGGL(km_scatter_kernel, dim3((p.nblk + kScatterBlocks - 1) / kScatterBlocks, segs),
                               dim3(256), 0, stream, p);
            IMI_LAUNCH_CHECK("km_scatter_kernel");
        }
        // Empty-cluster draws of this iteration: std::mt19937(it + 12345) with
        // uniform_int_distribution<int32_t>(0, T-1), one per empty cluster in
        // ascending cluster order (kmeans_core.cpp:299-311).
        Draws dr;
        std::mt19937 rng(static_cast<unsigned>(it + 12345));
        std::uniform_int_distribution<int32_t> dist(0, a->n_tokens - 1);
        for (int e = 0; e < std::min(kmax, kDraws); ++e) dr.v[e] = dist(rng);
        if (dp == 128)
            hipLaunchKernelGGL(km_update_block_kernel<128>, dim3(kmax, segs), dim3(256), 0, stream, p, dr);
        else if (dp == 64)
            hipLaunchKernelGGL(km_update_block_kernel<64>, dim3(kmax, segs), dim3(256), 0, stream, p, dr);
        else
            hipLaunchKernelGGL(km_update_block_kernel<32>, dim3(kmax, segs), dim3(256), 0, stream, p, dr);
        IMI_LAUNCH_CHECK("km_update_block_kernel");
        // the draws of empty ordinals kDraws and up (IVF, k > kDraws)
        for (int e0 = kDraws; e0 < kmax; e0 += kDraws) {
            for (int e = e0; e < std::min(kmax, e0 + kDraws); ++e) dr.v[e - e0] = dist(rng);
            hipLaunchKernelGGL(km_reseed_kernel, dim3(kmax, segs), dim3(64), 0, stream, p, dr, e0);
            IMI_LAUNCH_CHECK("km_reseed_kernel");
        }
    }
    return IMI_OK;
}

extern "C" int imi_kmeans_assign(const uint16_t* keys, int64_t head_stride, int64_t token_stride, int32_t kv_heads,
                                 int32_t n_tokens, int32_t dim, int32_t parts, const int32_t* k,
                                 const float* centroids, int32_t* labels, float* mind, imi_stream_t stream_) {
    clear_error();
    imi_kmeans_args a{};
    a.keys = keys;
    a.head_stride = head_stride;
    a.token_stride = token_stride;
    a.kv_heads = kv_heads;
    a.n_tokens = n_tokens;
    a.dim = dim;
    a.parts = parts;
    IMI_REQUIRE(k != nullptr, IMI_ERR_INVALID, "imi_kmeans_assign: null k");
    for (int i = 0; i < parts && i < 4; ++i) a.k[i] = k[i];
    a.max_iters = 1;
    a.init_mode = 1;
    a.centroids = const_cast<float*>(centroids);
    a.labels = labels;
    int kmax, dp;
    int rc = validate(&a, kmax, dp);
    if (rc) return rc;
    KmParams p{};
    p.keys = keys;
    p.hs = head_stride;
    p.ts = token_stride;
    p.H = kv_heads;
    p.T = n_tokens;
    p.P = parts;
    p.kmax = kmax;
    p.DP = dp;
    for (int i = 0; i < 4; ++i) p.k[i] = i < parts ? k[i] : 0;
    p.cent = const_cast<float*>(centroids);
    p.labels = labels;
    p.mind = mind;
    p.exact = mind != nullptr ? 1 : 0;
    p.nblk = (n_tokens + 255) / 256;
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (dp == 128) return run_assign<128>(p, kv_heads * parts, stream);
    return dp == 64 ? run_assign<64>(p, kv_heads * parts, stream) : run_assign<32>(p, kv_heads * parts, stream);
}
