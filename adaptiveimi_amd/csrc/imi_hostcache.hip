// Host tier: KV lists in pinned host memory, a GPU block cache per KV head.
//
// Reference: library/AdaptiveIMI/cpp_extensions/src/wave_buffer_cpu_hotcold.cpp
//   ClusterDescriptor / BufferManager   39-372 (hot / cold LRU of clusters,
//                                        block allocation, access, admission)
//   AdpIMI_Index::set_cluster_metadata  850-895
//   AdpIMI_Index::batch_access / update 897-949
// and the copies of include/copy_kernel.cuh (concat_gather_copy 220-335: the
// execution buffer is [static | miss pages | hit pages]; gather_copy_scatter
// 439-530: admitted pages from the buffer into the cache).
//
// The manager is plain host code, one per group (the reference spreads the
// groups over a thread pool; each group's decisions depend only on its own
// state).  The two kernels copy whole 256-byte rows, 16 lanes per row.  The
// steady rows are not copied (the attention reads them in place), so the
// buffer holds [miss | hit].
#include <algorithm>
#include <new>
#include <vector>

#include "imi_common.hpp"

struct imi_hostcache {
    // One cluster (cell) of one group.
    struct Cell {
        int start = 0;        // first list row
        int blocks = 0;       // ceil(size / block_size); 0 for an empty cell
        int last = 0;         // rows in the last block
        bool cached = false;
        bool hot = false;
        int prev = -1, next = -1;   // LRU links (in the hot or the cold list)
        std::vector<int> ids;       // cache block of each of its blocks
    };
    struct Group {
        std::vector<Cell> cells;
        std::vector<int> free_ids;  // free cache blocks, taken from the back
        int cold_head = -1, cold_tail = -1, hot_head = -1, hot_tail = -1;
        int hot_blocks = 0, cold_blocks = 0;
        std::vector<int> hit_keys, miss_keys;   // of the last access
        int64_t hit_blocks_last = 0, miss_blocks_last = 0;
    };
    int groups = 0, n_cells = 0, capacity = 0, block_size = 0, max_consider = 0, max_keys = 0;
    int hot_capacity = 1;
    std::vector<Group> g;

    void reset(Group& gr) const {
        gr.free_ids.resize(capacity);
        for (int i = 0; i < capacity; ++i) gr.free_ids[i] = i;
        gr.cold_head = gr.cold_tail = gr.hot_head = gr.hot_tail = -1;
        gr.hot_blocks = gr.cold_blocks = 0;
        gr.hit_keys.clear();
        gr.miss_keys.clear();
        gr.hit_blocks_last = gr.miss_blocks_last = 0;
        for (auto& c : gr.cells) {
            c.cached = c.hot = false;
            c.prev = c.next = -1;
        }
    }
    static void unlink(Group& gr, int k, int& head, int& tail) {
        Cell& c = gr.cells[k];
        if (c.prev >= 0) gr.cells[c.prev].next = c.next;
        else head = c.next;
        if (c.next >= 0) gr.cells[c.next].prev = c.prev;
        else tail = c.prev;
        c.prev = c.next = -1;
    }
    static void push_front(Group& gr, int k, int& head, int& tail) {
        Cell& c = gr.cells[k];
        c.prev = -1;
        c.next = head;
        if (head >= 0) gr.cells[head].prev = k;
        head = k;
        if (tail < 0) tail = k;
    }
    // A hit cluster moves to the front of the hot list (a cold one is
    // promoted when it fits the hot capacity, else refreshed in the cold
    // list); the hot tail spills to the front of the cold list.
    void touch_hit(Group& gr, int k) const {
        Cell& c = gr.cells[k];
        if (c.hot) {
            if (gr.hot_head != k) {
                unlink(gr, k, gr.hot_head, gr.hot_tail);
                push_front(gr, k, gr.hot_head, gr.hot_tail);
            }
            return;
        }
        if (c.blocks > hot_capacity) {
            if (gr.cold_head != k) {
                unlink(gr, k, gr.cold_head, gr.cold_tail);
                push_front(gr, k, gr.cold_head, gr.cold_tail);
            }
            return;
        }
        unlink(gr, k, gr.cold_head, gr.cold_tail);
        gr.cold_blocks -= c.blocks;
        c.hot = true;
        push_front(gr, k, gr.hot_head, gr.hot_tail);
        gr.hot_blocks += c.blocks;
        while (gr.hot_blocks > hot_capacity && gr.hot_tail >= 0) {
            const int d = gr.hot_tail;
            unlink(gr, d, gr.hot_head, gr.hot_tail);
            gr.cells[d].hot = false;
            gr.hot_blocks -= gr.cells[d].blocks;
            push_front(gr, d, gr.cold_head, gr.cold_tail);
            gr.cold_blocks += gr.cells[d].blocks;
        }
    }
    // Evicts the least recently used cluster: the cold tail, else the hot
    // tail; its blocks go back to the end of the free list.
    static void evict_one(Group& gr) {
        const int v = gr.cold_tail >= 0 ? gr.cold_tail : gr.hot_tail;
        if (v < 0) return;
        Cell& c = gr.cells[v];
        if (c.hot) {
            unlink(gr, v, gr.hot_head, gr.hot_tail);
            gr.hot_blocks -= c.blocks;
        } else {
            unlink(gr, v, gr.cold_head, gr.cold_tail);
            gr.cold_blocks -= c.blocks;
        }
        c.hot = false;
        gr.free_ids.insert(gr.free_ids.end(), c.ids.begin(), c.ids.begin() + c.blocks);
        c.cached = false;
    }
};

namespace imi {
namespace {

constexpr int kCopyThreads = 256;
constexpr int kCopyRows = 128;   // rows per workgroup (16 lanes per row, 16 rows per pass)

__device__ __forceinline__ void copy_row(const uint16_t* src, uint16_t* dst, int li) {
    *reinterpret_cast<uint4*>(dst + li * 8) = *reinterpret_cast<const uint4*>(src + li * 8);
}

// Last index i in [0, n) with pre[i] <= r (pre ascending, pre[0] = 0 <= r).
__device__ __forceinline__ int last_le(const int* pre, int n, int r) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pre[mid] <= r) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Rows [kCopyRows x, + kCopyRows) of group blockIdx.y's execution buffer
// [miss rows | hit rows]; workgroup 0 of the group also writes the one-cell
// selection over the buffer.
__global__ __launch_bounds__(kCopyThreads) void hc_gather_kernel(imi_hostcache_gather_args a) {
    extern __shared__ int hc_lds[];
    const int grp = blockIdx.y, tid = threadIdx.x;
    const int mb = a.max_blocks;
    int* mpre = hc_lds;        // [mb]
    int* hpre = hc_lds + mb;   // [mb]
    const int64_t lb = static_cast<int64_t>(grp) * mb;
    const int nm = min(max(a.miss_nums[grp], 0), mb), nh = min(max(a.hit_nums[grp], 0), mb);
    const int miss_rows = nm > 0 ? a.miss_prefix[lb + nm - 1] + a.miss_sizes[lb + nm - 1] : 0;
    const int hit_rows = nh > 0 ? a.hit_prefix[lb + nh - 1] + a.hit_sizes[lb + nh - 1] : 0;
    const int total = static_cast<int>(min(static_cast<int64_t>(miss_rows) + hit_rows, a.exec_rows));
    if (blockIdx.x == 0 && tid == 0) {
        const int64_t so = static_cast<int64_t>(grp) * a.sel_cap;
        const int64_t sp = static_cast<int64_t>(grp) * (a.sel_cap + 1);
        a.sel_offset[so] = 0;
        a.sel_count[so] = total;
        a.sel_prefix[sp] = 0;
        a.sel_prefix[sp + 1] = total;
        a.n_selected[grp] = total > 0 ? 1 : 0;
        a.n_rows[grp] = total;
    }
    const int r0 = blockIdx.x * kCopyRows;
    if (r0 >= total) return;   // uniform over the workgroup
    for (int i = tid; i < nm; i += kCopyThreads) mpre[i] = a.miss_prefix[lb + i];
    for (int i = tid; i < nh; i += kCopyThreads) hpre[i] = a.hit_prefix[lb + i];
    __syncthreads();
    const int li = tid & 15;
    const int64_t eb = static_cast<int64_t>(grp) * a.exec_rows;
    const int r1 = min(r0 + kCopyRows, total);
    for (int r = r0 + (tid >> 4); r < r1; r += kCopyThreads / 16) {
        const uint16_t *sk, *sv;
        if (r < miss_rows) {
            const int b = last_le(mpre, nm, r);
            const int64_t row = static_cast<int64_t>(grp) * a.list_rows + a.miss_ids[lb + b] + (r - mpre[b]);
            sk = a.host_keys + row * 128;
            sv = a.host_values + row * 128;
        } else {
            const int rh = r - miss_rows;
            const int b = last_le(hpre, nh, rh);
            const int64_t row = static_cast<int64_t>(grp) * a.cache_rows +
                                static_cast<int64_t>(a.hit_ids[lb + b]) * a.block_size + (rh - hpre[b]);
            sk = a.cache_keys + row * 128;
            sv = a.cache_values + row * 128;
        }
        copy_row(sk, a.exec_keys + (eb + r) * 128, li);
        copy_row(sv, a.exec_values + (eb + r) * 128, li);
    }
}

struct AdmitArgs {
    const uint16_t* ek;
    const uint16_t* ev;
    int64_t exec_rows;
    uint16_t* ck;
    uint16_t* cv;
    int64_t cache_rows;
    int block_size, max_blocks;
    const int32_t* ids;
    const int32_t* sizes;
    const int32_t* prefix;
    const int32_t* nums;
};

// Admitted block blockIdx.x of group blockIdx.y: its rows of the buffer's
// miss region to its cache block.
__global__ __launch_bounds__(kCopyThreads) void hc_admit_kernel(AdmitArgs a) {
    const int grp = blockIdx.y, u = blockIdx.x, tid = threadIdx.x;
    const int n = min(max(a.nums[grp], 0), a.max_blocks);
    if (u >= n) return;
    const int64_t lb = static_cast<int64_t>(grp) * a.max_blocks + u;
    const int rows = min(a.sizes[lb], a.block_size);
    const int64_t src0 = static_cast<int64_t>(grp) * a.exec_rows + a.prefix[lb];
    const int64_t dst0 = static_cast<int64_t>(grp) * a.cache_rows + static_cast<int64_t>(a.ids[lb]) * a.block_size;
    const int li = tid & 15;
    for (int r = tid >> 4; r < rows; r += kCopyThreads / 16) {
        copy_row(a.ek + (src0 + r) * 128, a.ck + (dst0 + r) * 128, li);
        copy_row(a.ev + (src0 + r) * 128, a.cv + (dst0 + r) * 128, li);
    }
}

}  // namespace
}  // namespace imi

using imi::set_error;

extern "C" {

int imi_hostcache_create(int32_t groups, int32_t n_cells, int32_t capacity, int32_t block_size,
                         int32_t max_consider_blocks, int32_t max_keys, double hot_ratio, imi_hostcache** out) {
    imi::clear_error();
    IMI_REQUIRE(out != nullptr, IMI_ERR_INVALID, "imi_hostcache_create: null out");
    *out = nullptr;
    IMI_REQUIRE(groups > 0 && n_cells > 0 && capacity > 0 && block_size > 0 && max_consider_blocks > 0 &&
                    max_keys > 0,
                IMI_ERR_INVALID, "imi_hostcache_create: sizes must be positive");
    auto* c = new (std::nothrow) imi_hostcache();
    IMI_REQUIRE(c != nullptr, IMI_ERR_INVALID, "imi_hostcache_create: out of host memory");
    c->groups = groups;
    c->n_cells = n_cells;
    c->capacity = capacity;
    c->block_size = block_size;
    c->max_consider = max_consider_blocks;
    c->max_keys = max_keys;
    // hot share of the capacity (wave_buffer_cpu_hotcold.cpp:75-95):
    // default 0.3, at most 1, truncated, at least one block
    double ratio = hot_ratio > 0.0 ? hot_ratio : 0.3;
    if (ratio > 1.0) ratio = 1.0;
    int target = static_cast<int>(capacity * ratio);
    if (target <= 0) target = std::min(capacity, 1);
    c->hot_capacity = target;
    c->g.resize(groups);
    for (auto& gr : c->g) {
        gr.cells.resize(n_cells);
        gr.hit_keys.reserve(max_keys);
        gr.miss_keys.reserve(max_keys);
        c->reset(gr);
    }
    *out = c;
    return IMI_OK;
}

void imi_hostcache_destroy(imi_hostcache* c) { delete c; }

int imi_hostcache_set_metadata(imi_hostcache* c, const int32_t* sizes, const int32_t* offsets) {
    imi::clear_error();
    IMI_REQUIRE(c && sizes && offsets, IMI_ERR_INVALID, "imi_hostcache_set_metadata: null argument");
    for (int gi = 0; gi < c->groups; ++gi) {
        auto& gr = c->g[gi];
        const int32_t* sz = sizes + static_cast<int64_t>(gi) * c->n_cells;
        const int32_t* of = offsets + static_cast<int64_t>(gi) * (c->n_cells + 1);
        for (int i = 0; i < c->n_cells; ++i) {
            auto& cell = gr.cells[i];
            const int n = sz[i];
            IMI_REQUIRE(n >= 0, IMI_ERR_INVALID, "imi_hostcache_set_metadata: negative size");
            cell.start = of[i];
            cell.blocks = n > 0 ? (n + c->block_size - 1) / c->block_size : 0;
            cell.last = n > 0 ? (n % c->block_size == 0 ? c->block_size : n % c->block_size) : 0;
            if (static_cast<int>(cell.ids.size()) < cell.blocks) cell.ids.resize(cell.blocks);
        }
        c->reset(gr);
    }
    return IMI_OK;
}

int imi_hostcache_access(imi_hostcache* c, const int64_t* keys, int32_t n_keys, int32_t* hit_ids,
                         int32_t* hit_sizes, int32_t* hit_prefix, int32_t* hit_nums, int32_t* miss_ids,
                         int32_t* miss_sizes, int32_t* miss_prefix, int32_t* miss_nums) {
    imi::clear_error();
    IMI_REQUIRE(c && keys && hit_ids && hit_sizes && hit_prefix && hit_nums && miss_ids && miss_sizes &&
                    miss_prefix && miss_nums,
                IMI_ERR_INVALID, "imi_hostcache_access: null argument");
    IMI_REQUIRE(n_keys >= 0 && n_keys <= c->max_keys, IMI_ERR_INVALID,
                "imi_hostcache_access: %d keys outside [0, %d]", n_keys, c->max_keys);
    // every key of every group is checked before any output or cache state
    // changes; a rejected call also forgets the previous access's hit and
    // miss lists, so that an update after it admits and touches nothing
    for (int64_t i = 0; i < static_cast<int64_t>(c->groups) * n_keys; ++i) {
        if (keys[i] >= 0 && keys[i] < c->n_cells) continue;
        for (auto& gr : c->g) {
            gr.hit_keys.clear();
            gr.miss_keys.clear();
        }
        IMI_REQUIRE(false, IMI_ERR_INVALID, "imi_hostcache_access: cell %lld outside [0, %d) (group %lld)",
                    static_cast<long long>(keys[i]), c->n_cells, static_cast<long long>(i / n_keys));
    }
    const int mb = c->max_consider;
    for (int gi = 0; gi < c->groups; ++gi) {
        auto& gr = c->g[gi];
        const int64_t* k = keys + static_cast<int64_t>(gi) * n_keys;
        int32_t *hid = hit_ids + static_cast<int64_t>(gi) * mb, *hsz = hit_sizes + static_cast<int64_t>(gi) * mb,
                *hpr = hit_prefix + static_cast<int64_t>(gi) * mb;
        int32_t *mid = miss_ids + static_cast<int64_t>(gi) * mb, *msz = miss_sizes + static_cast<int64_t>(gi) * mb,
                *mpr = miss_prefix + static_cast<int64_t>(gi) * mb;
        gr.hit_keys.clear();
        gr.miss_keys.clear();
        int nh = 0, nm = 0, hrow = 0, mrow = 0, consider = 0;
        for (int i = 0; i < n_keys; ++i) {
            const int64_t key = k[i];
            auto& cell = gr.cells[key];
            if (cell.blocks == 0 || cell.last == 0) continue;
            consider += cell.blocks;
            if (consider > mb) break;   // the buffer page rule
            if (!cell.cached) {
                gr.miss_keys.push_back(static_cast<int>(key));
                for (int j = 0; j < cell.blocks; ++j) {
                    const int span = j + 1 == cell.blocks ? cell.last : c->block_size;
                    mid[nm] = cell.start + j * c->block_size;
                    msz[nm] = span;
                    mpr[nm] = mrow;
                    mrow += span;
                    ++nm;
                }
            } else {
                gr.hit_keys.push_back(static_cast<int>(key));
                for (int j = 0; j < cell.blocks; ++j) {
                    const int span = j + 1 == cell.blocks ? cell.last : c->block_size;
                    hid[nh] = cell.ids[j];
                    hsz[nh] = span;
                    hpr[nh] = hrow;
                    hrow += span;
                    ++nh;
                }
            }
        }
        hit_nums[gi] = nh;
        miss_nums[gi] = nm;
        gr.hit_blocks_last = nh;
        gr.miss_blocks_last = nm;
    }
    return IMI_OK;
}

int imi_hostcache_update(imi_hostcache* c, int32_t* update_ids, int32_t* update_sizes, int32_t* update_prefix,
                         int32_t* update_nums) {
    imi::clear_error();
    IMI_REQUIRE(c && update_ids && update_sizes && update_prefix && update_nums, IMI_ERR_INVALID,
                "imi_hostcache_update: null argument");
    const int mb = c->max_consider;
    for (int gi = 0; gi < c->groups; ++gi) {
        auto& gr = c->g[gi];
        int32_t *uid = update_ids + static_cast<int64_t>(gi) * mb, *usz = update_sizes + static_cast<int64_t>(gi) * mb,
                *upr = update_prefix + static_cast<int64_t>(gi) * mb;
        // hits, last to first, to the front of the hot list
        for (int i = static_cast<int>(gr.hit_keys.size()) - 1; i >= 0; --i) {
            const int key = gr.hit_keys[i];
            if (gr.cells[key].blocks == 0 || gr.cells[key].last == 0) continue;
            c->touch_hit(gr, key);
        }
        // the prefix of the misses (rank order) that fits the capacity
        int admit = 0, need = 0;
        for (const int key : gr.miss_keys) {
            if (need + gr.cells[key].blocks > c->capacity) break;
            ++admit;
            need += gr.cells[key].blocks;
        }
        int nu = 0, row = 0;
        if (admit > 0) {
            while (static_cast<int>(gr.free_ids.size()) < need) imi_hostcache::evict_one(gr);
            for (int i = 0; i < admit; ++i) {
                const int key = gr.miss_keys[i];
                auto& cell = gr.cells[key];
                if (static_cast<int>(gr.free_ids.size()) < cell.blocks) continue;
                cell.cached = true;
                cell.hot = false;
                const size_t base = gr.free_ids.size() - cell.blocks;
                for (int j = 0; j < cell.blocks; ++j) {
                    const int id = gr.free_ids[base + cell.blocks - 1 - j];   // the back of the free list first
                    const int span = j + 1 == cell.blocks ? cell.last : c->block_size;
                    cell.ids[j] = id;
                    uid[nu] = id;
                    usz[nu] = span;
                    upr[nu] = row;
                    row += span;
                    ++nu;
                }
                gr.free_ids.resize(base);
                imi_hostcache::push_front(gr, key, gr.cold_head, gr.cold_tail);
                gr.cold_blocks += cell.blocks;
            }
        }
        update_nums[gi] = nu;
        gr.hit_keys.clear();
        gr.miss_keys.clear();
    }
    return IMI_OK;
}

int imi_hostcache_stats(const imi_hostcache* c, int64_t* hit_blocks, int64_t* miss_blocks) {
    imi::clear_error();
    IMI_REQUIRE(c && hit_blocks && miss_blocks, IMI_ERR_INVALID, "imi_hostcache_stats: null argument");
    int64_t h = 0, m = 0;
    for (const auto& gr : c->g) {
        h += gr.hit_blocks_last;
        m += gr.miss_blocks_last;
    }
    *hit_blocks = h;
    *miss_blocks = m;
    return IMI_OK;
}

int imi_hostcache_gather(const imi_hostcache_gather_args* a, imi_stream_t stream) {
    imi::clear_error();
    IMI_REQUIRE(a != nullptr, IMI_ERR_INVALID, "imi_hostcache_gather: null args");
    IMI_REQUIRE(a->host_keys && a->host_values && a->cache_keys && a->cache_values && a->exec_keys &&
                    a->exec_values && a->hit_ids && a->hit_sizes && a->hit_prefix && a->hit_nums && a->miss_ids &&
                    a->miss_sizes && a->miss_prefix && a->miss_nums && a->sel_offset && a->sel_count &&
                    a->sel_prefix && a->n_selected && a->n_rows,
                IMI_ERR_INVALID, "imi_hostcache_gather: null pointer argument");
    IMI_REQUIRE(a->groups > 0 && a->max_blocks > 0 && a->block_size > 0 && a->sel_cap >= 1, IMI_ERR_INVALID,
                "imi_hostcache_gather: empty shape");
    IMI_REQUIRE(a->exec_rows >= static_cast<int64_t>(a->max_blocks) * a->block_size, IMI_ERR_INVALID,
                "imi_hostcache_gather: exec_rows %lld < max_blocks * block_size", static_cast<long long>(a->exec_rows));
    IMI_REQUIRE(a->cache_rows > 0 && a->cache_rows % a->block_size == 0 && a->list_rows > 0, IMI_ERR_INVALID,
                "imi_hostcache_gather: cache_rows must be a positive multiple of block_size");
    IMI_REQUIRE(a->groups <= 65535 && a->max_blocks <= 16384, IMI_ERR_UNSUPPORTED,
                "imi_hostcache_gather: %d groups / %d blocks per group exceed the grid", a->groups, a->max_blocks);
    const int64_t nx = (a->exec_rows + imi::kCopyRows - 1) / imi::kCopyRows;
    const size_t lds = static_cast<size_t>(2) * a->max_blocks * sizeof(int);
    if (lds > 64 * 1024)
        IMI_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&imi::hc_gather_kernel),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    hipLaunchKernelGGL(imi::hc_gather_kernel, dim3(static_cast<unsigned>(nx), a->groups), dim3(imi::kCopyThreads),
                       lds, reinterpret_cast<hipStream_t>(stream), *a);
    IMI_LAUNCH_CHECK("hc_gather_kernel");
    return IMI_OK;
}

int imi_hostcache_admit(const uint16_t* exec_keys, const uint16_t* exec_values, int64_t exec_rows,
                        uint16_t* cache_keys, uint16_t* cache_values, int64_t cache_rows, int32_t block_size,
                        int32_t groups, int32_t max_blocks, const int32_t* update_ids, const int32_t* update_sizes,
                        const int32_t* update_prefix, const int32_t* update_nums, imi_stream_t stream) {
    imi::clear_error();
    IMI_REQUIRE(exec_keys && exec_values && cache_keys && cache_values && update_ids && update_sizes &&
                    update_prefix && update_nums,
                IMI_ERR_INVALID, "imi_hostcache_admit: null pointer argument");
    IMI_REQUIRE(groups > 0 && max_blocks > 0 && block_size > 0 && exec_rows > 0 && cache_rows > 0, IMI_ERR_INVALID,
                "imi_hostcache_admit: empty shape");
    IMI_REQUIRE(groups <= 65535, IMI_ERR_UNSUPPORTED, "imi_hostcache_admit: %d groups exceed the grid", groups);
    imi::AdmitArgs p{exec_keys, exec_values, exec_rows, cache_keys, cache_values, cache_rows, block_size,
                     max_blocks, update_ids, update_sizes, update_prefix, update_nums};
    hipLaunchKernelGGL(imi::hc_admit_kernel, dim3(max_blocks, groups), dim3(imi::kCopyThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), p);
    IMI_LAUNCH_CHECK("hc_admit_kernel");
    return IMI_OK;
}

int imi_host_device_pointer(const void* host, void** device) {
    imi::clear_error();
    IMI_REQUIRE(host && device, IMI_ERR_INVALID, "imi_host_device_pointer: null argument");
    IMI_HIP_CHECK(hipHostGetDevicePointer(device, const_cast<void*>(host), 0));
    return IMI_OK;
}

}  // extern "C"
