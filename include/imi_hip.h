/*
 * imi_hip.h — C ABI of the MI355X (gfx950) AdaptiveIMI sparse-decode path.
 *
 * Plain pointers and sizes only.  Every pointer named "device" is HIP device
 * memory owned by the caller; the library keeps no pointer after a call
 * returns.  Every entry point enqueues work on the caller's stream and returns
 * without a host synchronisation; a non-zero return is an error whose text
 * imi_last_error() gives (thread-local), with nothing enqueued.
 *
 * Layout conventions (H = kv heads, T = indexed tokens, D = head_dim = 128,
 * P = subspace parts, Dp = D / P, G = query heads per kv head):
 *   keys/values  bf16 bit patterns, element (h, t, d) at
 *                base[h * head_stride + t * token_stride + d]
 *   centroids    fp32 [H][P][kmax][Dp]   (subspace centroids)
 *   labels       int32 [H][P][T]          (subspace labels)
 *   cell index   global cell id g = ((l0 * k1 + l1) * k2 + l2) * k3 + l3
 *                (mixed radix, reorganize_core.cpp:33-35, 112-118); IVF
 *                (P = 1, Dp = D): g = the cluster label
 *   cell_count / cell_offset   int32 [H][ncells] / [H][ncells + 1]: CSR over
 *                global cell ids (empty cells have count 0)
 *   list_keys / list_values    bf16 [H][list_stride_rows][D]: rows in CSR order
 *   perm         int32 [H][T]: CSR position -> original token index
 */
#ifndef IMI_HIP_H_
#define IMI_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* imi_stream_t; /* == hipStream_t */

enum {
    IMI_OK = 0,
    IMI_ERR_INVALID = 1,     /* bad argument / shape */
    IMI_ERR_HIP = 2,         /* HIP runtime error */
    IMI_ERR_UNSUPPORTED = 3, /* shape outside what the kernels implement */
    IMI_ERR_WORKSPACE = 4    /* workspace too small */
};

/* Thread-local text of the last error (empty string when none). */
const char* imi_last_error(void);
/* ABI version of this library (bumped on any signature change). */
int imi_version(void);

/* ------------------------------------------------------------------ k-means
 * Replaces the CPU k-means of the index build:
 *   kmeans_execute / kmeans_execute_4 / kmeans_execute_ivf
 *     (library/AdaptiveIMI/cpp_extensions/src/kmeans_core.cpp:822-1174),
 *   KmeansExecutor::execute (kmeans_core.cpp:384-501),
 *   lloyd_iteration (kmeans_core.cpp:190-314).
 * Assignments use the reference distance order exactly (8 FMA lanes then a
 * left-to-right lane sum, strict '<' so ties go to the lower centroid); the
 * M-step sums each cluster's members in ascending token order and multiplies
 * by 1.0f/size (the reference with one thread per (head, subspace), which is
 * what it runs on hosts with fewer than 32 cores); empty clusters are
 * re-seeded from std::mt19937(iter + 12345) exactly as the reference does.
 */
typedef struct {
    const uint16_t* keys;     /* device, bf16 bits, see layout above */
    int64_t head_stride;      /* elements between heads */
    int64_t token_stride;     /* elements between tokens */
    int32_t kv_heads;         /* H */
    int32_t n_tokens;         /* T */
    int32_t dim;              /* D (128) */
    int32_t parts;            /* P: 2 or 4 (IMI subspaces), or 1 (IVF: one
                                 128-dim space, kmeans_core.cpp:503-595) */
    int32_t k[4];             /* centroids per subspace, each in [1, 512]
                                 (IVF: [1, 4096]) */
    int32_t max_iters;        /* >= 1 */
    float tol;                /* absolute inertia tolerance */
    int32_t early_stop_min_iter; /* early stop disabled when > max_iters */
    float early_stop_rel_tol;
    int32_t init_mode;        /* 0: first k rows of each subspace;
                                 1: centroids already hold the initial values;
                                 2: kmeans++ (kmeans_core.cpp:138-186, seeds
                                    42 + subspace, same for every head) */
    float* centroids;         /* device [H][P][kmax][Dp] in/out */
    int32_t* labels;          /* device [H][P][T] out (last E-step) */
    int32_t* iters_run;       /* device [H][P] out (E-steps executed), may be NULL */
    void* workspace;          /* device, >= imi_kmeans_workspace_size() bytes */
    size_t workspace_bytes;
} imi_kmeans_args;

int imi_kmeans_workspace_size(const imi_kmeans_args* a, size_t* bytes);
int imi_kmeans_execute(const imi_kmeans_args* a, imi_stream_t stream);

/* One assignment pass with given centroids (the E-step of
 * kmeans_core.cpp:222-242), for parity checks with injected centroids.
 * mind (optional) receives each token's minimum distance. */
int imi_kmeans_assign(const uint16_t* keys, int64_t head_stride, int64_t token_stride, int32_t kv_heads,
                      int32_t n_tokens, int32_t dim, int32_t parts, const int32_t* k, const float* centroids,
                      int32_t* labels, float* mind, imi_stream_t stream);

/* ------------------------------------------------------------ cell index
 * Replaces reorganize_from_kmeans / _4 (reorganize_core.cpp:313-394,
 * 477-569) with build_compact_reorg_input (18-176) and reorganize_single_head
 * (234-311): stable order of tokens by (cell, token), CSR over global cells,
 * compact metadata padded to n_centroids (pipeline_bindings.cpp:206-276,
 * indexing.py:108-174) and the K/V row permutation into the list.
 */
typedef struct {
    const uint16_t* keys;     /* device bf16, layout above */
    const uint16_t* values;   /* device bf16, same strides as keys */
    int64_t head_stride;
    int64_t token_stride;
    int32_t kv_heads, n_tokens, dim, parts;
    int32_t k[4];
    const float* centroids;   /* device [H][P][kmax][Dp] (from imi_kmeans_execute) */
    const int32_t* labels;    /* device [H][P][T] */
    /* outputs (device) */
    int32_t* cell_count;      /* [H][ncells] */
    int32_t* cell_offset;     /* [H][ncells + 1] */
    int32_t* perm;            /* [H][T] */
    uint16_t* list_keys;      /* [H][list_rows][D] */
    uint16_t* list_values;    /* [H][list_rows][D] */
    int64_t list_rows;        /* >= T */
    /* compact metadata (optional: all NULL to skip) */
    int32_t n_centroids;      /* padded slot count (>= occupied cells + 0) */
    int32_t* n_active;        /* [H] occupied cells */
    int32_t* compact_gid;     /* [H][n_centroids], -1 for padding slots */
    int32_t* compact_size;    /* [H][n_centroids] */
    int32_t* compact_offset;  /* [H][n_centroids + 1] */
    float* compact_centroids; /* [H][n_centroids][D] merged, zero padding (may be NULL) */
    uint8_t* compact_mask;    /* [H][n_centroids] 1 = masked (padding) (may be NULL) */
    void* workspace;
    size_t workspace_bytes;
} imi_index_args;

int imi_index_workspace_size(const imi_index_args* a, size_t* bytes);
int imi_build_index(const imi_index_args* a, imi_stream_t stream);

/* ------------------------------------------------------ decode: scoring
 * fused_query_group_similarities (src/gpu_bindings.cpp:21-43,
 * cuda/compute_impl.cu:62-103): scores[h][c] = fp32 FMA chain over d of
 * qsum[h][d] * centroids[h][c][d], qsum = sum over the G grouped queries.
 * query: bf16 [H][G][D]; centroids fp32 [H][N][D]; out fp32 [H][out_stride].
 * mask (optional, [H][N], 1 = masked) writes -inf (retrieval.py:357).
 */
int imi_fused_query_group_similarities(const uint16_t* query, const float* centroids, float* out,
                                       int64_t out_stride, const uint8_t* mask, int32_t kv_heads,
                                       int32_t groups, int32_t n_clusters, int32_t dim, imi_stream_t stream);

/* -------------------------------------------------- decode: selection
 * _select_clusters (retrieval.py:295-303) after the -inf mask (357), plus
 * the page-budget truncation of BufferManager::batch_access
 * (wave_buffer_cpu_hotcold.cpp:303-371), computed without a host round trip:
 * per head, cells ranked by (score desc, cell id asc) over occupied cells;
 * the first m kept where m = min(nprobe, rank at which the exclusive token
 * prefix reaches max_tokens, rank at which the page count exceeds
 * buffer_pages).  Scores follow compute_impl.cu:80-101 bit for bit (the
 * 128-term chain is split at the subspace boundary, which leaves the
 * arithmetic unchanged).
 */
typedef struct {
    const uint16_t* query;    /* device bf16 [H][G][D] (q heads h*G..h*G+G-1) */
    const float* centroids;   /* device [H][P][kmax][Dp] */
    const int32_t* cell_count;  /* device [H][ncells] */
    const int32_t* cell_offset; /* device [H][ncells + 1] */
    int32_t kv_heads, groups, dim, parts;   /* groups (G): 1..16 */
    int32_t k[4];
    int32_t nprobe, max_tokens, buffer_pages, page_size;
    /* outputs (device) */
    int32_t* sel_cell;        /* [H][sel_cap] global cell ids in rank order */
    int32_t* sel_offset;      /* [H][sel_cap] CSR row of each selected cell */
    int32_t* sel_count;       /* [H][sel_cap] rows of each selected cell */
    int32_t* sel_prefix;      /* [H][sel_cap + 1] exclusive row prefix */
    int32_t* n_selected;      /* [H] m */
    int32_t* n_rows;          /* [H] selected rows (sum of sel_count) */
    int32_t sel_cap;          /* >= min(nprobe, buffer_pages) */
    /* 4-way IMI (parts == 4) only: occupied cells in ascending global id,
     * the compact outputs of imi_build_index, and a workspace zero-filled
     * before its first use (calls of any shape may then share it; calls
     * that overlap in time may not).  At most 1024 KV heads. */
    const int32_t* compact_gid;     /* [H][compact_cap] */
    const int32_t* compact_size;    /* [H][compact_cap] */
    const int32_t* compact_offset;  /* [H][compact_cap + 1] */
    const int32_t* n_active;        /* [H] */
    int32_t compact_cap;
    void* workspace;
    size_t workspace_bytes;         /* >= imi_select_workspace_size() */
    /* Ragged batches (the heads of several sequences in one call, no
     * counterpart in the batch-1 reference): per-head token and page budgets,
     * device int32 [H], or NULL for max_tokens / buffer_pages on every head.
     * Each per-head value is clamped to its scalar, so the scalars must be
     * the largest budgets (they size sel_cap and the attention's max_rows). */
    const int32_t* head_max_tokens;
    const int32_t* head_buffer_pages;
    /* Tile mode (IMI_MAX_TILES != 0 in the reference; retrieval.py:30-112,
     * 452-527): the cells kept by nprobe and the token budget are not cut by
     * the running page total -- the reference attends them tile by tile
     * (each tile at most buffer_pages pages, outputs merged by LSE) -- and a
     * head stops at its first cell that alone needs more than buffer_pages
     * pages.  Selected rows then reach max_tokens - 1 + buffer_pages *
     * page_size, and sel_cap must cover nprobe.  0 = off. */
    int32_t tile_mode;
    /* Online index maintenance (imi_update_*; async_update.py:7-19): cells
     * whose merged centroid was replaced are scored over their shadow row
     * (the same 128-term chain).  upd_slot NULL = no replaced centroids. */
    const float* shadow;            /* [H][shadow_rows][D] */
    int32_t shadow_rows;
    const int32_t* upd_slot;        /* [H][ncells] (2-way) or [H][compact_cap] (4-way) */
    const int32_t* upd_row;         /* [H][shadow_rows] */
    const int32_t* upd_n;           /* [H] */
    /* Delta append (async_update.py:20-76): ring entries whose cell is in the
     * reference's `selected` (the cells that pass nprobe and the token
     * budget, before the page cut, plus the padding id when fewer than
     * nprobe pass) are appended after the selected rows, in ring index
     * order, up to exec_rows - n_rows.  With tile_mode (retrieval.py:
     * 480-509) the append follows the tiles: per tile, the entries of the
     * tile's cells -- and the padding entries where the head's row of the
     * tile is padded, i.e. it took fewer cells into the tile than the head
     * that took most -- up to exec_rows minus the rows of the tile's cells;
     * a padding entry can then repeat, and delta_rows keeps the first
     * ring_cap rows.  ring_cap 0 = off; sel_cap must then cover nprobe. */
    const int32_t* ring_cell;       /* [H][ring_cap] match code (imi_update_args) */
    const int32_t* ring_row;        /* [H][ring_cap] steady row of each entry */
    const int32_t* ring_n;          /* [H] valid entries (ring index 0 ..) */
    int32_t ring_cap;               /* <= 1024 */
    int32_t exec_rows;              /* execution-buffer rows after the static rows */
    int32_t* delta_rows;            /* out [H][ring_cap] steady rows appended */
    int32_t* n_delta;               /* out [H] */
} imi_select_args;

/* Workspace imi_select needs (0 for 2-way IMI within the one-kernel
 * selection, except tile mode with the delta append: its tile scratch). */
int imi_select_workspace_size(const imi_select_args* a, size_t* bytes);
int imi_select(const imi_select_args* a, imi_stream_t stream);

/* ------------------------------------------ decode: gather + attention
 * Replaces concat_gather_copy (include/copy_kernel.cuh:220-335, launched by
 * cuda/gather_copy.cu:100-213) and the unvendored weighted_flash_decoding
 * called at retrieval.py:439-447: for kv head h and each of its G query
 * heads, softmax(scale * q.k) v over [the first static_len rows of the steady
 * zone | the rows of the selected cells], read in place from the list (no
 * execution buffer).  fp32 accumulation, bf16 output [H*G][D].
 */
typedef struct {
    const uint16_t* query;        /* device bf16 [H][G][D] */
    const uint16_t* steady_keys;  /* device bf16 [H][steady_stride][D] */
    const uint16_t* steady_values;
    int64_t steady_stride;        /* rows per head in the steady zone */
    int32_t static_len;           /* rows attended from the steady zone */
    const uint16_t* list_keys;    /* device bf16 [H][list_rows][D] */
    const uint16_t* list_values;
    int64_t list_rows;
    const int32_t* sel_offset;    /* from imi_select; every selected cell */
    const int32_t* sel_count;     /*   holds at least one row (imi_select */
    const int32_t* sel_prefix;    /*   keeps no empty cell) */
    const int32_t* n_selected;
    const int32_t* n_rows;
    int32_t sel_cap;
    int32_t max_rows;             /* bound on n_rows (buffer_pages * page_size) */
    int32_t kv_heads, groups, dim;   /* groups (G): 1..8 or 16 */
    float scale;                  /* softmax scale (1/sqrt(D)) */
    uint16_t* out;                /* device bf16 [H*G][D] */
    float* out_lse;               /* device fp32 [H*G] natural-log LSE, may be NULL */
    void* workspace;              /* zero-filled before first use */
    size_t workspace_bytes;       /* >= imi_attention_workspace_size() */
    /* Delta rows (imi_select delta append): steady-zone rows attended after
     * the selected rows, or NULL.  max_rows must then also cover delta_cap. */
    const int32_t* delta_rows;    /* [H][delta_cap] */
    const int32_t* n_delta;       /* [H] */
    int32_t delta_cap;
    /* Optional HOST array [H] (read during the call, not kept), NULL if
     * absent: a bound on each head's attended rows (static + selected +
     * delta), e.g. buffer_pages[h] * page_size + steady_stride in a ragged
     * batch.  When the bounds differ, the split pass gives each run of equal
     * bounds a number of workgroups per head proportional to its bound (at
     * most 4 runs; more fall back to equal shares).  No counterpart in the
     * reference (its decode batch is one sequence). */
    const int32_t* head_rows_bound;
    /* Optional expected attended rows per head (0 = unknown), e.g. the
     * page rule over cells of the index's mean size.  A decode step takes
     * the fixed-window split pass only when the hint is at least half the
     * row bound: with far fewer rows, a few windows would hold them all.
     * Never a bound and never read by the kernels.  No counterpart in the
     * reference. */
    int32_t rows_hint;
} imi_attention_args;

int imi_attention_workspace_size(const imi_attention_args* a, size_t* bytes);
int imi_sparse_attention(const imi_attention_args* a, imi_stream_t stream);

/* --------------------------------------------- online index maintenance
 * The reference's async centroid update and delta append
 * (cache_hub/adaptive_imi/async_update.py:77-162, state from
 * runtime.py:106-166), split in two calls on the caller's stream:
 *
 * imi_update_assign  (async_update.py:119-134, 146-161) for the batch of
 *   `count` decode keys at steady rows [row0, row0 + count): each key's
 *   cluster is the first compact row with the largest dot product over the
 *   shadow (torch.argmax of keys_fp32 @ shadow^T; the dot products here are
 *   sequential fp32 FMA chains over d, -0 counted as +0); delta_counts +=
 *   1 and delta_sums += key per key in batch order; the keys enter the delta
 *   ring (ring_id = compact row, ring_cell = match code, ring_row = steady
 *   row) at ring_pos, which advances modulo ring_cap; ring_n saturates at
 *   ring_cap.
 * imi_update_refresh (async_update.py:135-143) for the same batch: every
 *   row the batch touched whose delta count reached `threshold` becomes
 *   (shadow * centroid_count + delta_sum) / (centroid_count + delta_count),
 *   its centroid count takes the sum and its delta state is cleared; an
 *   occupied row (< n_active) so replaced gets an override slot that
 *   imi_select reads.  The reference copies the shadow into the scored
 *   centroids when its side stream has finished (async_update.py:7-19);
 *   callers make that deterministic by calling refresh before the next
 *   step's selection (and before the next assign).
 *
 * Match codes (ring_cell): the global cell id of an occupied row; -1 for
 * the reference padding id (padding_id, which `selected` holds wherever a
 * rank was not kept); -2 for any other empty slot (never selected).
 */
typedef struct {
    const uint16_t* steady_keys;   /* device bf16 [H][steady_stride][D] */
    int64_t steady_stride;
    int32_t row0;                  /* steady row of the batch's first key */
    int32_t count;                 /* keys in the batch, 1 .. ring_cap */
    int32_t kv_heads, dim;         /* D = 128 */
    float* shadow;                 /* device [H][n_rows][D] merged centroids by compact id */
    int32_t n_rows;                /* compact rows held (>= n_active + 1) */
    int32_t padding_id;            /* reference padding cluster id (n_centroids - 1) */
    const int32_t* n_active;       /* device [H] */
    const int32_t* compact_gid;    /* device [H][n_rows] global cell id per compact row */
    int32_t* centroid_counts;      /* device [H][n_rows] */
    int32_t* delta_counts;         /* device [H][n_rows] */
    float* delta_sums;             /* device [H][n_rows][D] */
    int32_t threshold;             /* >= 1 */
    int32_t* ring_id;              /* device [H][ring_cap] compact row (delta_cluster_ids) */
    int32_t* ring_cell;            /* device [H][ring_cap] match code */
    int32_t* ring_row;             /* device [H][ring_cap] steady row */
    int32_t* ring_pos;             /* device [H] next write position */
    int32_t* ring_n;               /* device [H] valid entries */
    int32_t ring_cap;              /* 1 .. 1024 (delta_tokens) */
    int32_t* upd_slot;             /* device [H][n_index] override slot or -1 */
    int32_t* upd_row;              /* device [H][n_rows] shadow row of each slot */
    int32_t* upd_n;                /* device [H] slots in use */
    int32_t n_index;               /* ncells (2-way, by global id) or n_rows (4-way, by compact id) */
    int32_t index_by_gid;          /* 1: upd_slot is indexed by global cell id (2-way selection) */
    void* workspace;               /* device, >= imi_update_workspace_size() bytes */
    size_t workspace_bytes;
} imi_update_args;

int imi_update_workspace_size(const imi_update_args* a, size_t* bytes);
int imi_update_assign(const imi_update_args* a, imi_stream_t stream);
int imi_update_refresh(const imi_update_args* a, imi_stream_t stream);

/* One decode step of one layer (retrieval.py:320-602, tile mode off):
 * imi_select followed by the gather + attention kernel on the same stream;
 * with sel.ring_cap > 0 the matched delta-ring tokens are attended after the
 * selected rows (attn.max_rows must also cover ring_cap).
 * The selection outputs and the split partials live in attn.workspace,
 * which must be zero-filled before its first use; every call leaves it
 * reusable.  Calls that share a workspace must not overlap.
 * phases (bits): 1 = selection, 2 = attention (split pass + merge),
 * 4 = split pass only, 8 = merge only; 0 = 3 = the whole step.  A phase
 * run alone reads what the previous call left in the workspace (the
 * selection, the split partials), e.g. to time one kernel. */
typedef struct {
    imi_select_args sel;          /* output pointers may be NULL: workspace used */
    imi_attention_args attn;      /* sel_* fields are filled in by the call */
    int32_t phases;
} imi_decode_args;

int imi_decode_workspace_size(const imi_decode_args* a, size_t* bytes);
int imi_decode_step(const imi_decode_args* a, imi_stream_t stream);

/* imi_decode_step without any allocation and without a caller workspace:
 * no counterpart in the reference.  It is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops).  The
 * workspace lives in a static device array of 64 MiB per device, held until
 * the process ends (its address is resolved once per device on the first
 * call); a shape whose workspace (imi_decode_workspace_size) exceeds it is
 * rejected with IMI_ERR_UNSUPPORTED.  attn.workspace / workspace_bytes are
 * ignored.  Every call on a device shares that device's array, so calls
 * that overlap in time on one device (two streams, two threads) race; calls
 * in stream order are fine.  Each call first clears the words its kernels
 * expect zero.  No hipMalloc / hipFree is called. */
int imi_decode_step_noalloc(const imi_decode_args* a, imi_stream_t stream);

/* ------------------------------------------------------------- host tier --
 * KV lists in pinned host memory with a GPU block cache per KV head, for
 * shapes whose lists exceed HBM.
 *
 * imi_hostcache_* is host code (no GPU call): one block-cache manager per
 * group (KV head) with the hot / cold LRU policy of the reference's
 * BufferManager (library/AdaptiveIMI/cpp_extensions/src/
 * wave_buffer_cpu_hotcold.cpp:54-372): `capacity` cache blocks of
 * `block_size` rows, a hot list of at most max(1, int(capacity * hot_ratio))
 * blocks (hot_ratio <= 0 means the reference default 0.3; > 1 counts as 1),
 * and at most `max_consider_blocks` blocks per access (the buffer page
 * rule).  Replaces AdpIMI_Index::set_cluster_metadata (:850-895),
 * batch_access (:897-929, BufferManager::batch_access :295-371) and
 * batch_update (:931-949, BufferManager::batch_update :216-293); lists are
 * [groups][max_consider_blocks] int32 host arrays, counts [groups]. */
typedef struct imi_hostcache imi_hostcache;

int imi_hostcache_create(int32_t groups, int32_t n_cells, int32_t capacity, int32_t block_size,
                         int32_t max_consider_blocks, int32_t max_keys, double hot_ratio, imi_hostcache** out);
void imi_hostcache_destroy(imi_hostcache* c);
/* Cluster sizes [groups][n_cells] and CSR offsets [groups][n_cells + 1]
 * (host int32); resets every group's cache to empty. */
int imi_hostcache_set_metadata(imi_hostcache* c, const int32_t* sizes, const int32_t* offsets);
/* keys: [groups][n_keys] host int64 cell ids in rank order (cells of size 0,
 * e.g. the padding cell, are skipped).  hit_*: cache block id, rows, row
 * prefix (exclusive, within the hit region); miss_*: first list row, rows,
 * row prefix within the miss region. */
int imi_hostcache_access(imi_hostcache* c, const int64_t* keys, int32_t n_keys, int32_t* hit_ids,
                         int32_t* hit_sizes, int32_t* hit_prefix, int32_t* hit_nums, int32_t* miss_ids,
                         int32_t* miss_sizes, int32_t* miss_prefix, int32_t* miss_nums);
/* After an access: admits the missed clusters that fit (in rank order),
 * evicting from the cold then hot tail; update_ids = the cache block each
 * admitted block goes to, update_sizes its rows, update_prefix its first
 * row in the miss region of the execution buffer. */
int imi_hostcache_update(imi_hostcache* c, int32_t* update_ids, int32_t* update_sizes, int32_t* update_prefix,
                         int32_t* update_nums);
/* Totals over the last access: hit and miss blocks. */
int imi_hostcache_stats(const imi_hostcache* c, int64_t* hit_blocks, int64_t* miss_blocks);

/* GPU side.  Execution buffer exec_* [groups][exec_rows][128] bf16 = the
 * miss rows (read from the pinned host lists host_* [groups][list_rows][128]
 * through their device mapping, see imi_host_device_pointer) then the hit
 * rows (from cache_* [groups][capacity * block_size][128]); the lists are
 * device copies of the access outputs.  Also writes a one-cell selection
 * per group over the buffer (sel_offset = 0, sel_count = sel_prefix[1] =
 * n_rows = rows, n_selected = rows > 0), so imi_sparse_attention with
 * list = exec, list_rows = exec_rows attends [steady | miss | hit] rows as
 * the reference's concat_gather_copy (include/copy_kernel.cuh:220-335)
 * orders them. */
typedef struct {
    const uint16_t* host_keys;   /* device address of pinned host memory */
    const uint16_t* host_values;
    int64_t list_rows;
    const uint16_t* cache_keys;  /* device [groups][capacity * block_size][128] */
    const uint16_t* cache_values;
    int64_t cache_rows;          /* capacity * block_size */
    uint16_t* exec_keys;         /* device [groups][exec_rows][128] */
    uint16_t* exec_values;
    int64_t exec_rows;           /* >= max_consider_blocks * block_size */
    int32_t groups, max_blocks;  /* list width (max_consider_blocks) */
    int32_t block_size;          /* rows per cache block */
    const int32_t* hit_ids;      /* device copies of the access lists */
    const int32_t* hit_sizes;
    const int32_t* hit_prefix;
    const int32_t* hit_nums;
    const int32_t* miss_ids;
    const int32_t* miss_sizes;
    const int32_t* miss_prefix;
    const int32_t* miss_nums;
    int32_t* sel_offset;         /* [groups][sel_cap] outputs: the one-cell */
    int32_t* sel_count;          /*   selection over the buffer */
    int32_t* sel_prefix;         /* [groups][sel_cap + 1] */
    int32_t* n_selected;         /* [groups] */
    int32_t* n_rows;             /* [groups] */
    int32_t sel_cap;
} imi_hostcache_gather_args;

int imi_hostcache_gather(const imi_hostcache_gather_args* a, imi_stream_t stream);
/* Cache admission (the reference's gather_copy_scatter,
 * include/copy_kernel.cuh:439-530): rows [update_prefix[u], + update_sizes[u])
 * of the buffer's miss region go to cache block update_ids[u]. */
int imi_hostcache_admit(const uint16_t* exec_keys, const uint16_t* exec_values, int64_t exec_rows,
                        uint16_t* cache_keys, uint16_t* cache_values, int64_t cache_rows, int32_t block_size,
                        int32_t groups, int32_t max_blocks, const int32_t* update_ids, const int32_t* update_sizes,
                        const int32_t* update_prefix, const int32_t* update_nums, imi_stream_t stream);
/* Device address of pinned host memory allocated by hipHostMalloc (torch
 * pin_memory=True); no counterpart in the reference (CUDA's unified
 * addressing hands the host pointer to the kernel). */
int imi_host_device_pointer(const void* host, void** device);

#ifdef __cplusplus
}
#endif
#endif /* IMI_HIP_H_ */
