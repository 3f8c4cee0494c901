// Online index maintenance on gfx950: the reference's async centroid update
// and delta ring (cache_hub/adaptive_imi/async_update.py:77-162, state set
// up at runtime.py:106-166).
//
// imi_update_assign, for a batch of decode keys (steady rows row0 ..):
//   upd_sim_kernel     grid (row chunks of 256, H, keys / 4): one compact row
//                      per thread, the dot product of four batch keys with it
//                      as sequential fp32 FMA chains over d (keys broadcast
//                      from LDS, the row streamed 32 dims at a time), then a
//                      workgroup arg-max per key packed as (order key of the
//                      value, ~row) so that the largest value and, among
//                      equal values, the lowest row wins (torch.argmax).
//   upd_assign_kernel  one workgroup per head: arg-max over the chunks, the
//                      delta counts and sums in batch order (each touched
//                      row read once, the keys added in order, written once)
//                      and the ring entries.
// imi_update_refresh, for the same batch:
//   upd_refresh_kernel one workgroup per head: every row the batch touched
//                      whose delta count reached the threshold gets the
//                      count-weighted mean (async_update.py:135-143), and an
//                      occupied row its override slot for imi_select.
#include "imi_common.hpp"

namespace imi {
namespace {

constexpr int kSimThreads = 256;   // compact rows per workgroup of upd_sim_kernel
constexpr int kKeyBlock = 4;       // batch keys per workgroup of upd_sim_kernel
constexpr int kMaxBatch = 64;      // keys one assign call takes
constexpr int kRingMax = 1024;     // delta ring capacity bound
constexpr int kD = 128;

struct UpdParams {
    const uint16_t* keys;   // steady zone [H][stride][D]
    int64_t stride;
    int row0, count, H;
    float* shadow;          // [H][n_rows][D]
    int n_rows, padding_id;
    const int32_t* n_active;
    const int32_t* gid;     // [H][n_rows]
    int32_t* cc;            // centroid counts [H][n_rows]
    int32_t* dc;            // delta counts [H][n_rows]
    float* ds;              // delta sums [H][n_rows][D]
    int threshold;
    int32_t* ring_id;
    int32_t* ring_cell;
    int32_t* ring_row;
    int32_t* ring_pos;
    int32_t* ring_n;
    int ring_cap;
    int32_t* upd_slot;      // [H][n_index]
    int32_t* upd_row;       // [H][n_rows]
    int32_t* upd_n;         // [H]
    int n_index, by_gid;
    uint64_t* part;         // [H][count][nchunk] packed arg-max per row chunk
    int nchunk;
};

__device__ __forceinline__ const uint16_t* key_row(const UpdParams& a, int h, int s) {
    return a.keys + (static_cast<int64_t>(h) * a.stride + a.row0 + s) * kD;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const int lo = __shfl_xor(static_cast<int>(v & 0xFFFFFFFFull), m);
    const int hi = __shfl_xor(static_cast<int>(v >> 32), m);
    return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

// Dot products of four batch keys (4 blockIdx.z .. +3) with one compact row
// per thread, and the arg-max of each key over the workgroup's 256 rows.
__global__ __launch_bounds__(kSimThreads) void upd_sim_kernel(UpdParams a) {
    __shared__ __attribute__((aligned(16))) float xs[kKeyBlock][kD];
    __shared__ uint64_t red[kSimThreads / 64][kKeyBlock];
    const int h = blockIdx.y, chunk = blockIdx.x, tid = threadIdx.x;
    const int kb = blockIdx.z * kKeyBlock;
    const int nk = min(kKeyBlock, a.count - kb);
    const int r = chunk * kSimThreads + tid;
    const bool live = r < a.n_rows;
    const float4* row = reinterpret_cast<const float4*>(a.shadow + (static_cast<int64_t>(h) * a.n_rows + (live ? r : 0)) * kD);
    // the block's keys (bf16 -> fp32 is exact), zero past the batch
    for (int i = tid; i < kKeyBlock * kD; i += kSimThreads) {
        const int j = i / kD, d = i % kD;
        xs[j][d] = j < nk ? bf16_to_f32(key_row(a, h, kb + j)[d]) : 0.0f;
    }
    float acc[kKeyBlock];
#pragma unroll
    for (int j = 0; j < kKeyBlock; ++j) acc[j] = 0.0f;
    float4 rv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) rv[u] = row[u];
    __syncthreads();
    // chain over d in order, the row read 32 dims (8 float4) at a time
#pragma unroll 1
    for (int dc = 0; dc < kD / 32; ++dc) {
        if (dc > 0) {
#pragma unroll
            for (int u = 0; u < 8; ++u) rv[u] = row[dc * 8 + u];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
#pragma unroll
            for (int j = 0; j < kKeyBlock; ++j) {
                const float4 x = *reinterpret_cast<const float4*>(&xs[j][dc * 32 + u * 4]);
                acc[j] = __builtin_fmaf(x.x, rv[u].x, acc[j]);
                acc[j] = __builtin_fmaf(x.y, rv[u].y, acc[j]);
                acc[j] = __builtin_fmaf(x.z, rv[u].z, acc[j]);
                acc[j] = __builtin_fmaf(x.w, rv[u].w, acc[j]);
            }
        }
    }
    // (value, ~row) keys: -0 counts as +0, rows past n_rows never win
    const int wave = tid >> 6;
#pragma unroll
    for (int j = 0; j < kKeyBlock; ++j) {
        const float v = acc[j] + 0.0f;
        uint64_t key = live ? (static_cast<uint64_t>(order_key(v)) << 32) |
                                  static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(r))
                            : 0ull;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const uint64_t o = shfl_xor_u64(key, m);
            key = o > key ? o : key;
        }
        if (lane_id() == 0) red[wave][j] = key;
    }
    __syncthreads();
    if (tid < nk) {
        uint64_t best = red[0][tid];
#pragma unroll
        for (int w = 1; w < kSimThreads / 64; ++w) best = red[w][tid] > best ? red[w][tid] : best;
        a.part[(static_cast<int64_t>(h) * a.count + kb + tid) * a.nchunk + chunk] = best;
    }
}

// First occurrence of each batch id, in batch order: grp[s] = index of the
// distinct id of key s, cells[i] = i-th distinct id, returns their number.
__device__ int group_ids(const int* ids, int count, int* grp, int* cells, int* sh) {
    const int tid = threadIdx.x;
    for (int s = tid; s < count; s += blockDim.x) {
        int f = s;
        for (int t = 0; t < s; ++t)
            if (ids[t] == ids[s]) {
                f = t;
                break;
            }
        grp[s] = f;   // first position for now
    }
    __syncthreads();
    if (tid == 0) {
        int n = 0;
        for (int s = 0; s < count; ++s) {
            if (grp[s] == s) {
                cells[n] = ids[s];
                grp[s] = n++;
            } else {
                grp[s] = grp[grp[s]];
            }
        }
        sh[0] = n;
    }
    __syncthreads();
    return sh[0];
}

// Batch ids, delta counts and sums (async_update.py:126-134) and the ring
// entries (146-161).  128 threads: thread d owns dimension d.
__global__ __launch_bounds__(kD) void upd_assign_kernel(UpdParams a) {
    __shared__ int ids[kMaxBatch];
    __shared__ int grp[kMaxBatch];
    __shared__ int cells[kMaxBatch];
    __shared__ int mult[kMaxBatch];
    __shared__ int sh[2];
    __shared__ float acc[kMaxBatch][kD + 1];
    __shared__ unsigned long long best[kMaxBatch];
    const int h = blockIdx.x, tid = threadIdx.x;
    if (tid < kMaxBatch) best[tid] = 0ull;
    __syncthreads();
    // arg-max over the chunks: every (key, chunk) partial loaded by some
    // thread, 8 loads in flight, combined with LDS atomics
    {
        const uint64_t* p = a.part + static_cast<int64_t>(h) * a.count * a.nchunk;
        const int total = a.count * a.nchunk;
        for (int i0 = tid; i0 < total; i0 += 8 * kD) {
            uint64_t v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = i0 + u * kD < total ? p[i0 + u * kD] : 0ull;
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (i0 + u * kD < total) atomicMax(&best[(i0 + u * kD) / a.nchunk], static_cast<unsigned long long>(v[u]));
        }
    }
    __syncthreads();
    for (int s = tid; s < a.count; s += kD)
        ids[s] = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(best[s] & 0xFFFFFFFFull));
    __syncthreads();
    const int nd = group_ids(ids, a.count, grp, cells, sh);
    const int64_t hrow = static_cast<int64_t>(h) * a.n_rows;
    // current sums of the touched rows (8 loads in flight), then the keys
    // added in batch order; thread d only touches column d
    for (int i0 = 0; i0 < nd; i0 += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = i0 + u < nd ? a.ds[(hrow + cells[i0 + u]) * kD + tid] : 0.0f;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (i0 + u < nd) acc[i0 + u][tid] = v[u];
    }
    if (tid < kMaxBatch) mult[tid] = 0;
    __syncthreads();
    for (int s0 = 0; s0 < a.count; s0 += 8) {
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = s0 + u < a.count ? bf16_to_f32(key_row(a, h, s0 + u)[tid]) : 0.0f;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (s0 + u < a.count) {
                const int g = grp[s0 + u];
                acc[g][tid] += x[u];
                if (tid == 0) mult[g] += 1;
            }
        }
    }
    __syncthreads();
    for (int i = 0; i < nd; ++i) a.ds[(hrow + cells[i]) * kD + tid] = acc[i][tid];
    if (tid < nd) a.dc[hrow + cells[tid]] += mult[tid];
    // ring entries at ring_pos, ring_pos + 1, ... (mod ring_cap)
    const int pos0 = a.ring_pos[h];
    const int na = a.n_active[h];
    for (int s = tid; s < a.count; s += kD) {
        const int c = ids[s];
        const int pos = (pos0 + s) % a.ring_cap;
        const int64_t e = static_cast<int64_t>(h) * a.ring_cap + pos;
        a.ring_id[e] = c;
        a.ring_cell[e] = c < na ? a.gid[hrow + c] : (c == a.padding_id ? -1 : -2);
        a.ring_row[e] = a.row0 + s;
    }
    if (tid == 0) {
        a.ring_pos[h] = (pos0 + a.count) % a.ring_cap;
        a.ring_n[h] = min(a.ring_n[h] + a.count, a.ring_cap);
    }
}

// Threshold update of the rows the last batch touched (async_update.py:
// 135-143): (shadow * count + sum) / max(count + delta, 1), multiply then add
// then divide, each rounded to fp32 as the reference's tensor ops are.  The
// touched rows' counts are read at once, the replaced rows 8 at a time (thread
// d owns dimension d), and override slots are handed out in first-touch order.
__global__ __launch_bounds__(kD) void upd_refresh_kernel(UpdParams a) {
    __shared__ int ids[kMaxBatch];
    __shared__ int grp[kMaxBatch];
    __shared__ int cells[kMaxBatch];
    __shared__ int sh[2];
    __shared__ int s_cnt[kMaxBatch], s_dlt[kMaxBatch], s_key[kMaxBatch], s_old[kMaxBatch];
    __shared__ int s_rep[kMaxBatch];
    __shared__ int s_nrep;
    const int h = blockIdx.x, tid = threadIdx.x;
    const int pos_end = a.ring_pos[h];
    const int un0 = a.upd_n[h];
    for (int s = tid; s < a.count; s += kD) {
        const int pos = ((pos_end - a.count + s) % a.ring_cap + a.ring_cap) % a.ring_cap;
        ids[s] = a.ring_id[static_cast<int64_t>(h) * a.ring_cap + pos];
    }
    __syncthreads();
    const int nd = group_ids(ids, a.count, grp, cells, sh);
    const int64_t hrow = static_cast<int64_t>(h) * a.n_rows;
    const int na = a.n_active[h];
    if (tid < nd) {
        const int c = cells[tid];
        const bool ok = c >= 0 && c < a.n_rows;   // a ring slot never written is skipped
        s_dlt[tid] = ok ? a.dc[hrow + c] : -1;
        s_cnt[tid] = ok ? a.cc[hrow + c] : 0;
        const int key = ok && c < na ? (a.by_gid ? a.gid[hrow + c] : c) : -1;
        s_key[tid] = key >= 0 && key < a.n_index ? key : -1;
        s_old[tid] = s_key[tid] >= 0 ? a.upd_slot[static_cast<int64_t>(h) * a.n_index + s_key[tid]] : 0;
    }
    __syncthreads();
    if (tid == 0) {
        int n = 0;
        for (int i = 0; i < nd; ++i)
            if (s_dlt[i] >= a.threshold) s_rep[n++] = i;
        s_nrep = n;
    }
    __syncthreads();
    const int nrep = s_nrep;
    for (int i0 = 0; i0 < nrep; i0 += 8) {
        float sv[8], dv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = i0 + u < nrep ? cells[s_rep[i0 + u]] : 0;
            sv[u] = i0 + u < nrep ? a.shadow[(hrow + c) * kD + tid] : 0.0f;
            dv[u] = i0 + u < nrep ? a.ds[(hrow + c) * kD + tid] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (i0 + u < nrep) {
                const int i = s_rep[i0 + u];
                const int c = cells[i];
                const int total = s_cnt[i] + s_dlt[i];
                const float num = __fadd_rn(__fmul_rn(sv[u], static_cast<float>(s_cnt[i])), dv[u]);
                a.shadow[(hrow + c) * kD + tid] = __fdiv_rn(num, static_cast<float>(total > 1 ? total : 1));
                a.ds[(hrow + c) * kD + tid] = 0.0f;
            }
        }
    }
    if (tid < nrep) {
        const int i = s_rep[tid];
        a.cc[hrow + cells[i]] = s_cnt[i] + s_dlt[i];
        a.dc[hrow + cells[i]] = 0;
    }
    if (tid == 0) {
        int n = un0;
        for (int r = 0; r < nrep; ++r) {
            const int i = s_rep[r];
            if (s_key[i] >= 0 && s_old[i] < 0 && n < a.n_rows) {
                a.upd_row[hrow + n] = cells[i];
                a.upd_slot[static_cast<int64_t>(h) * a.n_index + s_key[i]] = n;
                ++n;
            }
        }
        a.upd_n[h] = n;
    }
}

int update_validate(const imi_update_args* a, bool assign) {
    IMI_REQUIRE(a != nullptr, IMI_ERR_INVALID, "imi_update: null args");
    IMI_REQUIRE(a->dim == kD, IMI_ERR_UNSUPPORTED, "imi_update: head_dim must be 128");
    IMI_REQUIRE(a->kv_heads > 0 && a->n_rows > 0 && a->n_index > 0, IMI_ERR_INVALID, "imi_update: empty shape");
    IMI_REQUIRE(a->ring_cap >= 1 && a->ring_cap <= kRingMax, IMI_ERR_UNSUPPORTED,
                "imi_update: ring_cap %d outside [1, %d]", a->ring_cap, kRingMax);
    IMI_REQUIRE(a->count >= 1 && a->count <= kMaxBatch && a->count <= a->ring_cap, IMI_ERR_UNSUPPORTED,
                "imi_update: batch of %d keys outside [1, min(%d, ring_cap)]", a->count, kMaxBatch);
    IMI_REQUIRE(a->threshold >= 1, IMI_ERR_INVALID, "imi_update: threshold must be >= 1");
    IMI_REQUIRE(a->shadow && a->n_active && a->compact_gid && a->centroid_counts && a->delta_counts &&
                    a->delta_sums && a->ring_id && a->ring_cell && a->ring_row && a->ring_pos && a->ring_n &&
                    a->upd_slot && a->upd_row && a->upd_n,
                IMI_ERR_INVALID, "imi_update: null state pointer");
    if (assign) {
        IMI_REQUIRE(a->steady_keys != nullptr, IMI_ERR_INVALID, "imi_update_assign: null steady_keys");
        IMI_REQUIRE(a->row0 >= 0 && static_cast<int64_t>(a->row0) + a->count <= a->steady_stride, IMI_ERR_INVALID,
                    "imi_update_assign: rows [%d, %d) outside the steady zone of %lld rows", a->row0,
                    a->row0 + a->count, static_cast<long long>(a->steady_stride));
    }
    return IMI_OK;
}

size_t update_workspace(const imi_update_args* a, UpdParams* p) {
    Carver cv(a->workspace);
    const int nchunk = (a->n_rows + kSimThreads - 1) / kSimThreads;
    uint64_t* part = cv.take<uint64_t>(static_cast<size_t>(a->kv_heads) * a->count * nchunk);
    if (p) {
        p->part = part;
        p->nchunk = nchunk;
    }
    return cv.used();
}

void fill_params(const imi_update_args* a, UpdParams& p) {
    p.keys = a->steady_keys;
    p.stride = a->steady_stride;
    p.row0 = a->row0;
    p.count = a->count;
    p.H = a->kv_heads;
    p.shadow = a->shadow;
    p.n_rows = a->n_rows;
    p.padding_id = a->padding_id;
    p.n_active = a->n_active;
    p.gid = a->compact_gid;
    p.cc = a->centroid_counts;
    p.dc = a->delta_counts;
    p.ds = a->delta_sums;
    p.threshold = a->threshold;
    p.ring_id = a->ring_id;
    p.ring_cell = a->ring_cell;
    p.ring_row = a->ring_row;
    p.ring_pos = a->ring_pos;
    p.ring_n = a->ring_n;
    p.ring_cap = a->ring_cap;
    p.upd_slot = a->upd_slot;
    p.upd_row = a->upd_row;
    p.upd_n = a->upd_n;
    p.n_index = a->n_index;
    p.by_gid = a->index_by_gid != 0;
}

}  // namespace
}  // namespace imi

using namespace imi;

extern "C" int imi_update_workspace_size(const imi_update_args* a, size_t* bytes) {
    clear_error();
    int rc = update_validate(a, false);
    if (rc) return rc;
    IMI_REQUIRE(bytes != nullptr, IMI_ERR_INVALID, "imi_update_workspace_size: null output");
    imi_update_args t = *a;
    t.workspace = nullptr;
    *bytes = update_workspace(&t, nullptr);
    return IMI_OK;
}

extern "C" int imi_update_assign(const imi_update_args* a, imi_stream_t stream_) {
    clear_error();
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    int rc = update_validate(a, true);
    if (rc) return rc;
    imi_update_args t = *a;
    t.workspace = nullptr;
    const size_t need = update_workspace(&t, nullptr);
    IMI_REQUIRE(a->workspace && a->workspace_bytes >= need, IMI_ERR_WORKSPACE,
                "imi_update_assign: workspace %zu bytes < %zu required", a->workspace_bytes, need);
    UpdParams p{};
    fill_params(a, p);
    update_workspace(a, &p);
    hipLaunchKernelGGL(upd_sim_kernel, dim3(p.nchunk, a->kv_heads, (a->count + kKeyBlock - 1) / kKeyBlock),
                       dim3(kSimThreads), 0, stream, p);
    IMI_LAUNCH_CHECK("upd_sim_kernel");
    hipLaunchKernelGGL(upd_assign_kernel, dim3(a->kv_heads), dim3(kD), 0, stream, p);
    IMI_LAUNCH_CHECK("upd_assign_kernel");
    return IMI_OK;
}

extern "C" int imi_update_refresh(const imi_update_args* a, imi_stream_t stream_) {
    clear_error();
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    int rc = update_validate(a, false);
    if (rc) return rc;
    UpdParams p{};
    fill_params(a, p);
    hipLaunchKernelGGL(upd_refresh_kernel, dim3(a->kv_heads), dim3(kD), 0, stream, p);
    IMI_LAUNCH_CHECK("upd_refresh_kernel");
    return IMI_OK;
}
