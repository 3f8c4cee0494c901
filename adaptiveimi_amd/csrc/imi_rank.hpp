// Exact budget-bounded ranking of one KV head's cells inside one workgroup of
// 256 threads (gfx950).  Shared by the standalone selection kernel and the
// fused selection + attention kernel, so that both rank with the same code.
//
// Reference rules (per KV head):
//   retrieval.py:295-303  topk(nprobe) of the scores (ties: lowest cell id),
//                         inclusive int32 cumsum of the sizes, keep = size > 0
//                         & cumsum - size < max_tokens
//   retrieval.py:357      empty / padding cells masked to -inf (never kept)
//   wave_buffer_cpu_hotcold.cpp:303-371  stop at the first kept cell whose
//                         running page count exceeds buffer_pages
//   retrieval.py:30-112   tile mode: no running page cut; stop at the first
//                         cell that alone needs more than buffer_pages pages
//
// Input: each thread holds E items (key, cell id, size, CSR offset); a key is
// the order key of the cell's fp32 score (order_key), 0 for an empty item.
// Cell order is (key desc, cell id asc).  Because every kept cell costs at
// least one page, the kept cells are among the first K' = min(nprobe,
// buffer_pages, occupied) of that order (K' = nprobe in tile mode and for the
// delta match, which needs the cells the page cut drops too).  A linear-bucket
// histogram of the scores, refined inside the bucket that holds the K'-th
// cell when needed, puts the cells up to that bucket into LDS in bucket order
// (at most CAP of them); ranks inside each bucket segment come from counting
// larger keys, and block scans give the token and page prefixes.
#pragma once

#include "imi_common.hpp"

namespace imi {
namespace rank {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kBins = 2048;

// LDS words (int) the ranking uses for candidate capacity CAP and NB
// histogram bins.  Layout:
//   [0, 2 NB + 8)            hist[NB] | base[NB + 1] (pad); after the sort:
//                            the exclusive token prefix sp[CAP + 1]
//   [.., + 2 CAP)            ck (uint64 keys); after the sort: sg[CAP] (cell
//                            id) | ss[CAP] (size)
//   next CAP                 cs (size by slot)
//   next CAP                 co (CSR offset by slot)
//   next CAP                 seg (start | len << 16); after the sort: so[CAP]
//   next 192                 small scratch (reductions and scans)
template <int CAP, int NB = kBins>
struct Layout {
    static constexpr int kHist = 0;
    static constexpr int kBase = NB;
    static constexpr int kCk = ((2 * NB + 8 > CAP + 1 ? 2 * NB + 8 : CAP + 1) + 7) / 8 * 8;
    static constexpr int kCs = kCk + 2 * CAP;
    static constexpr int kCo = kCs + CAP;
    static constexpr int kSeg = kCo + CAP;
    static constexpr int kSmall = kSeg + CAP;
    static constexpr int kWords = kSmall + 192;
    static_assert(CAP + 1 <= kCk, "the token prefix reuses the histogram words");
    static_assert(NB % 256 == 0, "bins per thread");
    static_assert(CAP <= 32768, "segment fields are 16 bits");
};

struct Budget {
    int nprobe;
    int max_tokens;
    int buffer_pages;
    int page_size;
    int tile_mode;
    int rank_all;   // K' = nprobe (tile mode, delta match)
};

struct Result {
    int m;        // kept cells (ranks 0 .. m-1)
    int m_tok;    // cells that pass nprobe and the token budget (before the page cut)
    int n_rows;   // rows of the kept cells
    int C;        // ranked candidates (>= min(K', occupied))
};

// Item orders: BLOCKED, thread t's item e is cell (e >> 2) * 1024 + 4 t +
// (e & 3) (four consecutive cells per 1024-cell block, one 16-byte load per
// thread); SLOTS, thread t's item e is slot e * 256 + t of a list whose slot
// order is cell-id order; CONTIG, thread t's item e is the (E t + e)-th item
// of a list in cell-id order.
enum Order { BLOCKED = 0, SLOTS = 1, CONTIG = 2 };

__device__ __forceinline__ int item_cell(int e, int t) { return (e >> 2) * (4 * kThreads) + 4 * t + (e & 3); }

__device__ __forceinline__ float key_to_score(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

__device__ __forceinline__ uint64_t cand_key(uint32_t okey, int g) {
    return (static_cast<uint64_t>(okey) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(g));
}

__device__ __forceinline__ int cand_cell(uint64_t key) {
    return static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(key & 0xFFFFFFFFull));
}

template <int NB = kBins>
__device__ __forceinline__ int bucket_of(float s, float hi, float inv) {
    const float t = (hi - s) * inv;
    return t < static_cast<float>(NB - 1) ? static_cast<int>(t) : NB - 1;
}

// Block-wide exclusive scan of one int per thread; *total gets the sum.  One
// barrier: sm (kWaves words) must not be written again before another
// barrier.
__device__ __forceinline__ int block_excl_scan(int v, int* sm, int* total) {
    const int incl = wave_incl_scan(v);
    const int wave = threadIdx.x >> 6;
    if (lane_id() == 63) sm[wave] = incl;
    __syncthreads();
    int before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const int x = sm[w];
        before += w < wave ? x : 0;
        tot += x;
    }
    *total = tot;
    return before + incl - v;
}

// Two exclusive scans at once (one barrier; sm: 2 kWaves words).
__device__ __forceinline__ void block_excl_scan2(int& a, int& b, int* sm, int& ta, int& tb) {
    const int ia = wave_incl_scan(a), ib = wave_incl_scan(b);
    const int wave = threadIdx.x >> 6;
    if (lane_id() == 63) {
        sm[wave] = ia;
        sm[kWaves + wave] = ib;
    }
    __syncthreads();
    int ba = 0, bb = 0;
    ta = tb = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const int xa = sm[w], xb = sm[kWaves + w];
        ba += w < wave ? xa : 0;
        bb += w < wave ? xb : 0;
        ta += xa;
        tb += xb;
    }
    a = ba + ia - a;
    b = bb + ib - b;
}

// Sum of an int, max and min of a float over the block (one barrier; sm:
// 3 kWaves words).
__device__ __forceinline__ void block_sum_max_min(int& n, float& mx, float& mn, int* sm) {
    const int wn = wave_sum_i(n);
    const float wx = wave_max(mx), wm = -wave_max(-mn);
    const int wave = threadIdx.x >> 6;
    float* smf = reinterpret_cast<float*>(sm);
    if (lane_id() == 0) {
        sm[wave] = wn;
        smf[kWaves + wave] = wx;
        smf[2 * kWaves + wave] = wm;
    }
    __syncthreads();
    n = 0;
    mx = -INFINITY;
    mn = INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        n += sm[w];
        mx = fmaxf(mx, smf[kWaves + w]);
        mn = fminf(mn, smf[2 * kWaves + w]);
    }
}

// Ranks the items (see the file comment).  e_live: items e >= e_live are
// empty on every thread (a uniform bound that lets the loops skip them).
// gid is read only in the SLOTS order (the others imply the cell id).
// cnt_g / off_g: the head's cell sizes and CSR offsets in global memory, read
// for the placed candidates instead of cnt / off when LATE (many items per
// thread: fewer registers).  On return (after a barrier) the LDS holds, for
// ranks r < C: sg[r] cell id, ss[r] size, so[r] CSR offset; sp[r] the
// exclusive token prefix for r <= m.
template <int E, int CAP, bool LATE, int ORDER, int NB = kBins>
__device__ Result rank_cells(const uint32_t (&key)[E], const int (&gid)[E], const int (&cnt)[E], const int (&off)[E],
                             int e_live, const int32_t* cnt_g, const int32_t* off_g, const Budget& bud, int* lds) {
    using Lay = Layout<CAP, NB>;
    int* hist = lds + Lay::kHist;
    int* base = lds + Lay::kBase;
    uint64_t* ck = reinterpret_cast<uint64_t*>(lds + Lay::kCk);
    int* cs = lds + Lay::kCs;
    int* co = lds + Lay::kCo;
    int* seg = lds + Lay::kSeg;
    int* sm = lds + Lay::kSmall;   // [0, 16) reductions, [16, 32) level results, [32, 160) scans (8 alternating slots)
    const int tid = threadIdx.x;

    // ---- occupied items and their score range ----
    int n_valid = 0;
    float gmax = -INFINITY, gmin = INFINITY;
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (e < e_live && key[e] != 0u) {
            ++n_valid;
            const float s = key_to_score(key[e]);
            gmax = fmaxf(gmax, s);
            gmin = fminf(gmin, s);
        }
    for (int i = tid; i < NB; i += kThreads) hist[i] = 0;
    block_sum_max_min(n_valid, gmax, gmin, sm);

    int kp = bud.rank_all ? bud.nprobe : min(bud.nprobe, bud.buffer_pages);
    kp = min(kp, n_valid);
    Result res{0, 0, 0, 0};
    if (kp <= 0) {
        __syncthreads();
        if (tid == 0) lds[0] = 0;   // sp[0]
        __syncthreads();
        return res;
    }

    // ---- candidates: iterative linear-bucket refinement ----
    // st bit e: 1 = still in play.  Each level buckets the in-play scores
    // linearly over [lo, hi] (a higher score goes to a lower or equal
    // bucket), places every bucket wholly above the one holding the kp-th
    // best cell and, when that bucket does not fit in the remaining slots,
    // refines inside it.  Placed cells form segments (one per bucket) that
    // are already in rank order relative to each other.
    uint64_t st = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) st |= (e < e_live && key[e] != 0u ? 1ull : 0ull) << e;
    int c_sel = 0;
    float lo = gmin, hi = gmax;
    int scan_slot = 0;
    for (int level = 0; level < 16; ++level) {
        const float range = hi - lo;
        const float inv = range > 0.0f ? static_cast<float>(NB) / range : 0.0f;
        int bk[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            bk[e] = -1;
            if (e < e_live && ((st >> e) & 1ull)) bk[e] = bucket_of<NB>(key_to_score(key[e]), hi, inv);
        }
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (bk[e] >= 0) atomicAdd(&hist[bk[e]], 1);
        __syncthreads();
        const int need = kp - c_sel;
        {
            // NB / 256 bins per thread: serial prefix, then one block scan
            constexpr int BPT = NB / kThreads;
            int hv[BPT];
            int tsum = 0;
#pragma unroll
            for (int i = 0; i < BPT; ++i) {
                hv[i] = hist[tid * BPT + i];
                tsum += hv[i];
            }
            int total;
            int run = block_excl_scan(tsum, sm + 32 + 16 * (scan_slot++ & 7), &total);
#pragma unroll
            for (int i = 0; i < BPT; ++i) {
                const int b = tid * BPT + i;
                base[b] = run;
                if (run < need && run + hv[i] >= need) {
                    sm[16] = b;
                    sm[17] = run;
                    sm[18] = run + hv[i];
                }
                run += hv[i];
            }
            if (tid == kThreads - 1) base[NB] = run;
        }
        __syncthreads();
        for (int i = tid; i < NB; i += kThreads) hist[i] = 0;   // fill cursors
        const int bK = sm[16], c_lt = sm[17], c_le = sm[18];
        const bool fits = c_sel + c_le <= CAP;
        const bool flat = !(range > 0.0f);
        __syncthreads();
        int slot[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int b = bk[e];
            slot[e] = -1;
            if (b >= 0 && (b < bK || (fits && b == bK))) slot[e] = atomicAdd(&hist[b], 1);
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int b = bk[e];
            if (b < 0) continue;
            if (slot[e] >= 0) {
                const int g = ORDER == BLOCKED ? item_cell(e, tid) : ORDER == CONTIG ? E * tid + e : gid[e];
                const int s = c_sel + base[b] + slot[e];
                ck[s] = cand_key(key[e], g);
                cs[s] = LATE ? cnt_g[g] : cnt[e];
                co[s] = LATE ? off_g[g] : off[e];
                seg[s] = (c_sel + base[b]) | ((base[b + 1] - base[b]) << 16);
                st &= ~(1ull << e);
            } else if (b > bK) {
                st &= ~(1ull << e);
            }
        }
        if (fits) {
            c_sel += c_le;
            break;
        }
        c_sel += c_lt;
        __syncthreads();
        for (int i = tid; i < NB; i += kThreads) hist[i] = 0;
        if (flat) {
            // every cell still in play has the same score: the best are the
            // lowest cell ids, i.e. the first `keep` in cell-id order
            const int keep = kp - c_sel;
            int done = 0;
            // groups of items in cell-id order, GW items per group and thread
            constexpr int NG = ORDER == BLOCKED ? E / 4 : ORDER == SLOTS ? E : 1;
            constexpr int GW = ORDER == BLOCKED ? 4 : ORDER == SLOTS ? 1 : E;
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                int f = 0;
#pragma unroll
                for (int u = 0; u < GW; ++u) f += (st >> (GW * j + u)) & 1ull ? 1 : 0;
                int tot;
                int r = block_excl_scan(f, sm + 32 + 16 * (scan_slot++ & 7), &tot) + done;
#pragma unroll
                for (int u = 0; u < GW; ++u) {
                    const int e = GW * j + u;
                    if (((st >> e) & 1ull) == 0) continue;
                    if (r < keep) {
                        const int g = ORDER == BLOCKED ? item_cell(e, tid) : ORDER == CONTIG ? E * tid + e : gid[e];
                        const int s = c_sel + r;
                        ck[s] = cand_key(key[e], g);
                        cs[s] = LATE ? cnt_g[g] : cnt[e];
                        co[s] = LATE ? off_g[g] : off[e];
                        seg[s] = c_sel | (keep << 16);
                    }
                    ++r;
                }
                done += tot;
            }
            c_sel += keep;
            break;
        }
        // next level: the range of the cells still in play
        int dummy = 0;
        float mx = -INFINITY, mn = INFINITY;
#pragma unroll
        for (int e = 0; e < E; ++e)
            if ((st >> e) & 1ull) {
                const float s = key_to_score(key[e]);
                mx = fmaxf(mx, s);
                mn = fminf(mn, s);
            }
        block_sum_max_min(dummy, mx, mn, sm + 32 + 16 * (scan_slot++ & 7));
        hi = mx;
        lo = mn;
    }
    __syncthreads();
    const int C = c_sel;

    // ---- rank inside each segment by counting larger keys (segments are
    // short); values go through registers so that the sorted arrays can
    // reuse the key and segment words ----
    constexpr int SPT = CAP / kThreads;
    const int s_live = (C + kThreads - 1) / kThreads;   // slots in use per thread (uniform bound)
    int pg[SPT], pz[SPT], po[SPT], pp[SPT];
#pragma unroll
    for (int u = 0; u < SPT; ++u) {
        const int sl = tid + u * kThreads;
        pp[u] = -1;
        if (u < s_live && sl < C) {
            const uint64_t kk = ck[sl];
            const int sgv = seg[sl];
            const int s0 = sgv & 0xFFFF, sn = sgv >> 16;
            int r = 0;
            for (int i = s0; i < s0 + sn; ++i) r += ck[i] > kk;
            pp[u] = s0 + r;
            pg[u] = cand_cell(kk);
            pz[u] = cs[sl];
            po[u] = co[sl];
        }
    }
    __syncthreads();
    int* sg = lds + Lay::kCk;
    int* ss = lds + Lay::kCk + CAP;
    int* so = lds + Lay::kSeg;
    int* sp = lds + Lay::kHist;
#pragma unroll
    for (int u = 0; u < SPT; ++u)
        if (pp[u] >= 0) {
            sg[pp[u]] = pg[u];
            ss[pp[u]] = pz[u];
            so[pp[u]] = po[u];
        }
    __syncthreads();

    // ---- budget rules in rank order: thread t owns ranks [SPT t, SPT t + SPT) ----
    const int pshift = (bud.page_size & (bud.page_size - 1)) == 0 ? __builtin_ctz(bud.page_size) : -1;
    int tz[SPT], tp[SPT];
    int tsum = 0, psum = 0;
    const bool mine = tid * SPT < C;
#pragma unroll
    for (int u = 0; u < SPT; ++u) {
        const int r = tid * SPT + u;
        tz[u] = (mine && r < C) ? ss[r] : 0;
        // pages = ceil(size / page_size); tile mode counts the cells that
        // alone overflow the page budget
        int p = pshift >= 0 ? (tz[u] + bud.page_size - 1) >> pshift : (tz[u] + bud.page_size - 1) / bud.page_size;
        if (bud.tile_mode) p = p > bud.buffer_pages ? 1 : 0;
        tp[u] = p;
        tsum += tz[u];
        psum += p;
    }
    int ttot, ptot;
    int texcl = tsum, pexcl = psum;
    block_excl_scan2(texcl, pexcl, sm + 32 + 16 * (scan_slot++ & 7), ttot, ptot);
    int kept = 0, kept_tok = 0, kept_rows = 0;
#pragma unroll
    for (int u = 0; u < SPT; ++u) {
        const int r = tid * SPT + u;
        pexcl += tp[u];
        const bool keep_tok = r < C && r < bud.nprobe && texcl < bud.max_tokens;
        const bool keep = keep_tok && pexcl <= (bud.tile_mode ? 0 : bud.buffer_pages);
        kept += keep ? 1 : 0;
        kept_tok += keep_tok ? 1 : 0;
        kept_rows += keep ? tz[u] : 0;
        if (mine && r < C) sp[r] = texcl;
        texcl += tz[u];
    }
    // the rules are monotone in rank (prefixes only grow), so the kept ranks
    // are exactly the first m (the first m_tok before the page cut) and the
    // row total is the sum of their sizes
    {
        const int wk = wave_sum_i(kept), wt = wave_sum_i(kept_tok), wr = wave_sum_i(kept_rows);
        int* sr = sm + 32 + 16 * (scan_slot++ & 7);
        if (lane_id() == 0) {
            sr[tid >> 6] = wk;
            sr[kWaves + (tid >> 6)] = wt;
            sm[20 + (tid >> 6)] = wr;
        }
        __syncthreads();
        int m = 0, mt = 0, nr = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            m += sr[w];
            mt += sr[kWaves + w];
            nr += sm[20 + w];
        }
        res.m = m;
        res.m_tok = mt;
        res.n_rows = nr;
    }
    res.C = C;
    if (tid == 0) sp[res.m] = res.n_rows;
    __syncthreads();
    return res;
}

// Delta append (async_update.py:20-76, called at retrieval.py:420): the ring
// entries (ring index order, the first rn valid) whose cell is in the
// reference's `selected` -- the m_tok cells that pass nprobe and the token
// budget (retrieval.py:295-303), set in `keep` (a bitmap over global cell
// ids), plus the padding id (match code -1) when m_tok < nprobe -- up to
// exec_left rows.  Thread t holds ring entries 4t .. 4t + 3.  Writes the
// matched steady rows to drow[0 .. nd) in ring order and returns nd.
__device__ __forceinline__ int ring_match(const int (&rcode)[4], const int (&rrow)[4], int rn, int ncells, int m_tok,
                                          int nprobe, int exec_left, const uint32_t* keep, int* drow, int* sm) {
    bool match[4];
    int f = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = 4 * threadIdx.x + u;
        const int c = rcode[u];
        match[u] = i < rn && (c >= 0 ? (c < ncells && ((keep[c >> 5] >> (c & 31)) & 1u) != 0)
                                     : (c == -1 && m_tok < nprobe));
        f += match[u] ? 1 : 0;
    }
    int tot;
    int pos = block_excl_scan(f, sm, &tot);
    const int nd = min(tot, max(exec_left, 0));
#pragma unroll
    for (int u = 0; u < 4; ++u)
        if (match[u]) {
            if (pos < nd) drow[pos] = rrow[u];
            ++pos;
        }
    return nd;
}

}  // namespace rank
}  // namespace imi
