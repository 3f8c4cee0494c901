// Fused gather + GQA sparse decode attention on gfx950 (HBM-bound).
//
// Reference: the execution-buffer gather concat_gather_copy
// (include/copy_kernel.cuh:220-335, launched by cuda/gather_copy.cu:100-213:
// rows = [static_len steady rows | miss pages | hit pages]) followed by the
// unvendored weighted_flash_decoding (retrieval.py:439-447).  Here the rows
// are read in place -- the steady zone for the first static_len rows, the
// CSR list rows of the selected cells, then the matched delta-ring rows
// (steady rows) -- with no execution buffer.
//
// Grid: workgroups of 4 waves in up to four runs of heads; run r covers
// heads [h_r, h_r + n_r) with S_r splits each, and its workgroup l (counted
// from the run's first) takes split l / n_r of head h_r + l % n_r, so
// consecutive workgroups (which the dispatcher deals round robin to the 8
// XCDs) rotate over the heads.  One run covers every head unless the host
// passes per-head row bounds (ragged batches), where each run of
// equal-bound heads gets splits in proportion to its bound.  The run table
// sits in the first kernel-argument line.  Split s covers rows
// [R s / S, R (s + 1) / S) of its head's R attended rows, so the work follows
// the rows each head actually selected, not a bound.
//
// Prologue: one round trip brings q, the head's row / cell / delta counts,
// the first kStageCap cells of its selection (row prefix and CSR offset per
// cell) and its delta rows into registers, then LDS.  Each wave builds the
// row table of its quarter: a 64-ary ballot search finds the cell of its
// first selected row, the start of every later non-empty cell inside its
// rows is flagged with its rank, an inclusive max-scan gives each row its
// cell, and row -> list row (or -1 - steady row) goes to LDS.  The staged
// selection shares its LDS with the K / V tiles: a workgroup barrier after
// the tables separates the last read of the one from the first write of the
// other.  The short form (at most kFastCap selected cells and 64 NR rows
// per wave, NR = 2 or 4: the decode configurations at up to 128k tokens)
// keeps each lane's NR row locations in registers (the tile loads fetch
// them with a lane shuffle) and stages the selection apart from the tiles,
// so no workgroup barrier separates the lookup from the first loads.  Kernel
// arguments are ordered so that the prologue's loads depend on one 64-byte
// argument line, and the per-head counts are read with vector loads that
// leave with the others (one memory round trip before the lookup).
//
// Streaming: a wave owns a quarter of the workgroup's rows in tiles of 16
// and keeps two tiles in flight ahead of the one it computes.  Rows are read
// whole (16 lanes x 16 bytes per 256-byte row) and staged through LDS, which
// hands K back in the MFMA operand layout and V transposed.  Per tile:
//   S = K Q^T   4 x v_mfma_f32_16x16x32_bf16: A = the K tile read back from
//               LDS (lane -> token lane % 16, 8 dims), B = Q with column n holding
//               query n % G; lane l gets S[token 4(l/16)+i][query (l%16)%G].
//   O += P V    8 x v_mfma_f32_16x16x16_bf16: A = P, which is exactly the S
//               layout above (row = query slot, k = token) after exp2 and a
//               bf16 pack; B = V^T, read from a per-wave LDS copy of the V
//               tile with ds_read_b64_tr_b16 (4 tokens x 1 dim per lane).
// Softmax is online in base 2 with fp32 state per query slot; the rescale
// of O is skipped when no running max moved.  The waves of a workgroup merge
// in LDS into one partial (plain stores); merge_kernel combines each head's S
// partials in split order (deterministic) and writes the bf16 output and the
// LSE: the kernel boundary makes the partials visible across XCDs without any
// device-scope fence.
#include <climits>
#include <mutex>
#include <type_traits>

#include "imi_common.hpp"

namespace imi {

int select_launch(const imi_select_args* a, hipStream_t stream);
int select_validate(const imi_select_args* a, int64_t& ncells, int& kmax);
size_t select4_zero_bytes();
size_t sel2_keys_bytes(const imi_select_args* a);
size_t select4_workspace_size(const imi_select_args* a);

namespace {

constexpr int kWaves = 4;            // waves per workgroup (256 threads)
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxSplit = 4096;      // splits per head the merge kernel handles
constexpr int kLocCap = 2048;        // attended rows per workgroup (row lookup in LDS)
constexpr int kDeltaMax = 1024;      // delta rows per head (the delta ring)
constexpr int kVStride = 144;        // u16 per LDS row of a wave's K / V tile (288 B)
constexpr int kPF = 2;               // K / V tiles in flight per wave
constexpr int kStageCap = 2048;      // selected cells staged in the prologue's first round trip
constexpr int kStageMax = 16384;     // selected cells per head (row prefix + offset staged in LDS)
constexpr int kStageMax16 = 12288;   // the same for 16 query heads per KV head (larger wave partials)
// query heads per KV head with their own kernels (the 16 columns of the
// matrix-core tile hold query n mod G in column n, so any G <= 16 fits)
constexpr bool groups_supported(int g) { return (g >= 1 && g <= 8) || g == 16; }
constexpr int stage_max(int g) { return g > 8 ? kStageMax16 : kStageMax; }
// The short form (NR > 0): at most kFastCap selected cells (three entries
// per thread in one round trip) and kWaves * 64 * NR rows per workgroup, so
// that each lane keeps the locations of NR of its wave's rows in registers.
constexpr int kFastCap = 767;
constexpr int kFastPad = kFastCap + 1;   // words of each staged array (the prefix has cap + 1 entries)
constexpr int kFastNRMax = 4;            // row locations per lane (256 rows per wave)
constexpr int kMaxRuns = 4;              // runs of heads with their own split count (ragged batches)
constexpr int fast_rows(int nr) { return kWaves * 64 * nr; }

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __attribute__((address_space(1))) const u32x4_t g_u32x4_t;   // global (not flat) loads

// Fields in the order the kernel first needs them: the first 128 bytes (two
// scalar-cache lines, fetched together) hold everything the prologue's loads
// depend on, the next 64 what the row lookup and the first tile loads need.
//
// The split pass runs in runs of heads with a split count each: one run of
// all heads, or up to kMaxRuns for a ragged batch.  Run r = (first workgroup
// (= its first partial), first head, splits | heads << 16, floor(2^32 /
// heads) + 1 or 0 for one head); unused runs hold (INT_MAX, H, 0, 0).
// Workgroup b of run r takes split local / nh of head h0 + (local % nh +
// split) % nh, local = b - first (consecutive workgroups, which the
// dispatcher deals round robin to the XCDs, rotate over the run's heads);
// its partial is first + (h - h0) * splits + split.
struct DecParams {
    int4 run[kMaxRuns];
    // -- 64 bytes
    const uint16_t* q;
    const int32_t* g_prefix;   // [H][g_cap + 1]
    const int32_t* g_offset;   // [H][g_cap]
    const int32_t* g_nsel;     // [H]
    const int32_t* g_nrows;    // [H]
    const int32_t* g_drows;    // [H][g_dcap] or null
    const int32_t* g_ndelta;   // [H]
    int g_cap;                 // selection capacity per head
    int g_dcap;
    // -- 128 bytes: what the row lookup and the first loads need
    int H;
    int static_len;
    int s_stride;              // steady rows per head (< 2^31, checked by the host)
    int list_rows;             // list rows per head (< 2^31, checked by the host)
    const uint16_t* sk;
    const uint16_t* sv;
    const uint16_t* lk;
    const uint16_t* lv;
    float scale_log2;          // scale * log2(e)
    int o_base;                // LDS word of the staged offsets (after the prefix)
    int stage_words;           // LDS words shared by the staged selection and the K / V tiles
    int nr;                    // the short form's row locations per lane (0: the general form)
    // -- 192 bytes
    int total;                 // workgroups of the split pass (= partials)
    float* part_acc;           // [total][G][128]
    float* part_ml;            // [total][G][2]
    uint16_t* out;             // [H*G][128]
    float* lse;                // [H*G] or null
    int fixed_nt;              // tiles per wave of the fixed-grid split pass, 0: row-balanced
};
static_assert(offsetof(DecParams, q) == 64 && offsetof(DecParams, H) == 128 && offsetof(DecParams, total) == 192,
              "prologue fields in the first 128 bytes, lookup and load fields in the next 64");

// floor(R s / S) for R < 2^32 and 0 <= s <= S <= kMaxSplit.  R s < 2^44 is
// exact in fp64 and the rounded quotient is within 2^-8 / S of R s / S,
// whose distance to the next integer above is 0 or at least 1 / S: the
// truncation is exact or one below, which the check corrects.
__device__ __forceinline__ int64_t split_floor(uint32_t R, int s, int S, double inv_S) {
    const uint64_t n = static_cast<uint64_t>(R) * static_cast<uint32_t>(s);
    uint64_t q = static_cast<uint64_t>(static_cast<double>(n) * inv_S);
    if ((q + 1) * static_cast<uint64_t>(S) <= n) ++q;
    return static_cast<int64_t>(q);
}

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

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

// Inclusive max-scan across the 64 lanes (row shifts, then row broadcasts;
// lanes without a source keep INT_MIN, the identity).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_imin(int v) {
    return __builtin_amdgcn_update_dpp(INT_MIN, v, CTRL, ROW_MASK, 0xF, false);
}
__device__ __forceinline__ int wave_incl_max_scan(int v) {
    v = max(v, dpp_imin<0x111>(v));
    v = max(v, dpp_imin<0x112>(v));
    v = max(v, dpp_imin<0x114>(v));
    v = max(v, dpp_imin<0x118>(v));
    v = max(v, dpp_imin<0x142, 0xA>(v));
    v = max(v, dpp_imin<0x143, 0xC>(v));
    return v;
}

// LDS: [staged selection | K and V tiles] (stage_words), then the wave
// partials, the row lookup and the delta rows; the short form keeps the
// staged selection apart, after those.
constexpr int kTileU16 = kWaves * 16 * kVStride;   // one of the K / V tiles of all waves
constexpr int kTileWords = kTileU16;               // both tiles, in 32-bit words
template <int G>
constexpr int tail_words() {
    return kWaves * G * 128 + kWaves * G * 2 + kLocCap + kDeltaMax;
}
template <int G>
constexpr int fast_words() {
    return kTileWords + tail_words<G>() + 2 * kFastPad;
}

// One workgroup = 4 waves over its split of head h's rows [static | selected
// | delta]; writes one partial (max, sum, unnormalised output).  The head's
// selection (row prefix and CSR offset per cell, at most kStageCap cells in
// the first round trip) is staged in LDS together with q and the row counts.
// NR > 0, the short form (at most kFastCap cells, fast_rows(NR) rows per
// workgroup): each lane holds the locations of NR of its wave's rows in
// registers, and the staged selection does not share LDS with the tiles, so
// no workgroup barrier separates the row lookup from the first loads.
template <int G, int NR>
__global__ __launch_bounds__(kThreads) void attention_kernel(DecParams a) {
    constexpr bool FAST = NR > 0;
    static_assert(NR == 0 || NR == 2 || NR == 4, "two or four row locations per lane");
    extern __shared__ __attribute__((aligned(16))) int lds[];
    uint16_t* s_k = reinterpret_cast<uint16_t*>(lds);   // the tiles reuse the staged selection's words
    uint16_t* s_v = s_k + kTileU16;
    float* s_acc = reinterpret_cast<float*>(lds + (FAST ? kTileWords : a.stage_words));   // [4][G][128]
    float* s_ml = s_acc + kWaves * G * 128;                                 // [4][G][2]
    int* s_loc = reinterpret_cast<int*>(s_ml + kWaves * G * 2);             // [kLocCap]
    int* s_drow = s_loc + kLocCap;                                          // [kDeltaMax]
    int* P = FAST ? s_drow + kDeltaMax : lds;       // [g_cap + 1] row prefix of the selected cells
    int* O = FAST ? P + kFastPad : lds + a.o_base;  // [g_cap] CSR offset of each selected cell

    // this workgroup's run, head and split (divisions by the run's head
    // count as multiply-highs, exact for workgroups x heads < 2^32, which the
    // host checks)
    // (selects only, no branch and no indexed load).  The empty asm takes a
    // field of each of the first three argument lines, so that the lines are
    // fetched at once rather than one after another as the code needs them.
    asm volatile("" ::"s"(a.run[0].x), "s"(a.q), "s"(a.H));
    // (component by component: a select of whole int4 values went through
    // scratch memory)
    const uint32_t b = blockIdx.x;
    int rx = a.run[0].x, ry = a.run[0].y, rz = a.run[0].z, rw = a.run[0].w;
#pragma unroll
    for (int i = 1; i < kMaxRuns; ++i) {
        const bool in = a.run[i].x <= static_cast<int>(b);
        rx = in ? a.run[i].x : rx;
        ry = in ? a.run[i].y : ry;
        rz = in ? a.run[i].z : rz;
        rw = in ? a.run[i].w : rw;
    }
    const int nh = rz >> 16, S_h = max(rz & 0xFFFF, 1);
    const uint32_t local = b - static_cast<uint32_t>(rx);
    const uint32_t mg = static_cast<uint32_t>(rw);
    const int split = mg ? static_cast<int>(__umulhi(local, mg)) : static_cast<int>(local);
    int hl = static_cast<int>(local - static_cast<uint32_t>(split) * nh) +
             (split - static_cast<int>(__umulhi(static_cast<uint32_t>(split), mg)) * nh);
    hl = hl >= nh ? hl - nh : hl;
    hl = mg ? hl : 0;
    const int h = ry + hl;
    const int64_t pbase = rx + static_cast<int64_t>(hl) * S_h;   // partial of split 0 of this head
    const double inv_S = 1.0 / static_cast<double>(S_h);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lg = lane >> 4, ln = lane & 15;

    // ---- one round trip: q (as the MFMA B operand: column ln = query
    // ln % G, dims 32c + 8lg ..), the row and cell counts, the first
    // kStageCap cells of the selection and the delta rows ----
    u32x4_t qb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        qb[c] = *reinterpret_cast<const u32x4_t*>(a.q + (static_cast<int64_t>(h) * G + ln % G) * 128 + c * 32 + lg * 8);
    const int32_t* pre = a.g_prefix + static_cast<int64_t>(h) * (a.g_cap + 1);
    const int32_t* offg = a.g_offset + static_cast<int64_t>(h) * a.g_cap;
    // the counts travel with the vector loads below (one round trip for all)
    const int m_raw = vec_load_i32(a.g_nsel, h);
    const int nrows_raw = vec_load_i32(a.g_nrows, h);
    const int nd_raw = a.g_drows ? vec_load_i32(a.g_ndelta, h) : 0;
    constexpr int SU = FAST ? kFastPad / kThreads : (kStageCap + kThreads) / kThreads;   // entries per thread
    static_assert(!FAST || SU * kThreads == kFastPad, "the short form stages the prefix in SU loads per thread");
    int pv[SU], ov[SU];
    const int c1 = min(a.g_cap, FAST ? kFastCap : kStageCap);
#pragma unroll
    for (int u = 0; u < SU; ++u) {
        const int i = tid + u * kThreads;
        pv[u] = i <= c1 ? pre[i] : 0;
        ov[u] = i < c1 ? offg[i] : 0;
    }
    int dv[kDeltaMax / kThreads];
#pragma unroll
    for (int u = 0; u < kDeltaMax / kThreads; ++u) {
        const int i = tid + u * kThreads;
        dv[u] = (a.g_drows && i < a.g_dcap) ? a.g_drows[static_cast<int64_t>(h) * a.g_dcap + i] : 0;
    }
#pragma unroll
    for (int u = 0; u < SU; ++u) {
        const int i = tid + u * kThreads;
        if (i <= c1) P[i] = pv[u];
        if (i < c1) O[i] = ov[u];
    }
#pragma unroll
    for (int u = 0; u < kDeltaMax / kThreads; ++u) s_drow[tid + u * kThreads] = dv[u];
    const int m = min(max(__builtin_amdgcn_readfirstlane(m_raw), 0), a.g_cap);
    const int nrows = max(__builtin_amdgcn_readfirstlane(nrows_raw), 0);
    const int nd = min(max(__builtin_amdgcn_readfirstlane(nd_raw), 0), a.g_dcap);
    if constexpr (!FAST) {
        // selections above kStageCap cells: the rest in further round trips
        for (int i = kStageCap + 1 + tid; i <= m; i += kThreads) P[i] = pre[i];
        for (int i = kStageCap + tid; i < m; i += kThreads) O[i] = offg[i];
    }
    __syncthreads();
    const int sl = a.static_len;
    // split boundaries floor(R s / S) (R < 2^32)
    const uint32_t R = static_cast<uint32_t>(sl) + static_cast<uint32_t>(nrows) + static_cast<uint32_t>(nd);
    const int64_t r0 = split_floor(R, split, S_h, inv_S);
    const int64_t r1e = split_floor(R, split + 1, S_h, inv_S);
    const int64_t r1 = min(r1e, r0 + (FAST ? fast_rows(NR) : kLocCap));   // the host sizes S so that this never cuts

    // ---- row lookup: s_loc[i] for rows r0 + i of this split.  Each wave
    // fills the entries of its own quarter: a steady
    // row gets -1 - its row, a delta row -1 - its ring row, a selected row j
    // the list row O[c] + j - P[c] of the cell c holding it.  The cell of the
    // wave's first selected row comes from a 64-ary search over the staged
    // prefix (ballots); the start of every later non-empty cell inside the
    // wave's rows is flagged with its rank and an inclusive max-scan gives
    // every row its cell.  List rows are clamped to the list, steady rows to
    // the steady zone. ----
    const int nr = static_cast<int>(r1 - r0);
    const int wb = nr * wave / kWaves, we = nr * (wave + 1) / kWaves;
    const int wn = we - wb;   // <= kLocCap / 4 = 512 (FAST: 64 NR)
    const int lmax = max(a.list_rows - 1, 0);
    const int smax = a.s_stride - 1;
    // FAST: locations of rows wb + lane + 64 r (r < NR), same encoding (rows
    // past the wave's end: list row 0, never used)
    constexpr int NRL = NR > 0 ? NR : 1;
    int loc[NRL];
#pragma unroll
    for (int r = 0; r < NRL; ++r) loc[r] = 0;
    if constexpr (FAST) {
        const int64_t w0 = r0 + wb;
        const int pa = static_cast<int>(min(max(sl - w0, int64_t(0)), int64_t(wn)));
        const int pb = static_cast<int>(min(max(sl + nrows - w0, int64_t(0)), int64_t(wn)));
#pragma unroll
        for (int r = 0; r < NR; ++r) {   // steady or delta rows
            const int i = lane + 64 * r;
            if (i < pa) {
                loc[r] = -1 - static_cast<int>(w0 + i);
            } else if (i >= pb && i < wn) {
                const int d = static_cast<int>(w0 + i - sl - nrows);
                loc[r] = -1 - min(max(s_drow[min(d, kDeltaMax - 1)], 0), smax);
            }
        }
        if (pb > pa) {
            int* fl = s_loc + wave * 64 * NR;   // cell that starts at each position, else INT_MIN
#pragma unroll
            for (int r = 0; r < NR; ++r) fl[lane + 64 * r] = INT_MIN;
            const int jlo = static_cast<int>(w0 + pa - sl), jhi = jlo + (pb - pa);
            // c0 = the last cell with P[c] <= jlo (P[0] = 0 <= jlo): two
            // ballot rounds, m <= kFastCap < 64 * 64
            const int step = (m + 63) >> 6;
            const uint64_t b1 = __builtin_amdgcn_ballot_w64(lane * step < m && P[lane * step] <= jlo);
            const int base = (63 - __builtin_clzll(b1 | 1ull)) * step;
            const uint64_t b2 = __builtin_amdgcn_ballot_w64(lane < step && base + lane < m && P[base + lane] <= jlo);
            const int c0 = base + (63 - __builtin_clzll(b2 | 1ull));
            wave_lds_sync();   // the INT_MIN fill precedes the flags
            // later non-empty cells start above jlo: flag those that start below jhi
            for (int cb = c0 + 1; cb < m; cb += 64) {
                const int c = cb + lane;
                const int pc = c < m ? P[c] : INT_MAX;
                const int pn = c < m ? P[c + 1] : 0;
                if (pc < jhi && pn > pc) fl[pa + (pc - jlo)] = c;
                if (__builtin_amdgcn_readlane(pc, 63) >= jhi) break;
            }
            wave_lds_sync();
            int carry = c0;   // the cell of the positions before this lane's
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const int sc = max(wave_incl_max_scan(fl[lane + 64 * r]), carry);
                carry = __builtin_amdgcn_readlane(sc, 63);
                const int i = lane + 64 * r;
                if (i >= pa && i < pb) {
                    const int j = jlo + (i - pa);
                    loc[r] = min(max(O[sc] + (j - P[sc]), 0), lmax);
                }
            }
        }
    } else {
        const int64_t w0 = r0 + wb;   // first row of this wave
        // positions [0, pa) steady, [pa, pb) selected, [pb, wn) delta
        const int pa = static_cast<int>(min(max(sl - w0, int64_t(0)), int64_t(wn)));
        const int pb = static_cast<int>(min(max(sl + nrows - w0, int64_t(0)), int64_t(wn)));
        for (int i = lane; i < wn; i += 64) {
            int v = INT_MIN;
            if (i < pa) {
                v = -1 - static_cast<int>(w0 + i);
            } else if (i >= pb) {
                const int d = static_cast<int>(w0 + i - sl - nrows);
                v = -1 - min(max(s_drow[min(d, kDeltaMax - 1)], 0), smax);
            }
            s_loc[wb + i] = v;
        }
        if (pb > pa) {
            const int jlo = static_cast<int>(w0 + pa - sl), jhi = jlo + (pb - pa);
            // c0 = the last cell with P[c] <= jlo (P[0] = 0 <= jlo)
            int lo = 0, len = m;
            while (len > 1) {
                const int step = (len + 63) >> 6;
                const bool ok = lane * step < len && P[lo + lane * step] <= jlo;
                const int k = 63 - __builtin_clzll(__builtin_amdgcn_ballot_w64(ok) | 1ull);
                lo += k * step;
                len = min(step, len - k * step);
            }
            wave_lds_sync();   // the fill above precedes the flags
            if (lane == 0) s_loc[wb + pa] = lo;
            // later cells start above jlo: flag those that start below jhi
            for (int cb = lo + 1; cb < m; cb += 64) {
                const int c = cb + lane;
                const int pc = c < m ? P[c] : INT_MAX;
                const int pn = c < m ? P[c + 1] : 0;
                if (pc < jhi && pn > pc) s_loc[wb + pa + (pc - jlo)] = c;
                if (__builtin_amdgcn_readlane(pc, 63) >= jhi) break;
            }
            wave_lds_sync();
            // `per` consecutive selected positions per lane
            const int per = (pb - pa + 63) >> 6;   // <= 8
            const int q0 = pa + lane * per;
            int v[8];
            int run = INT_MIN;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                v[u] = (u < per && q0 + u < pb) ? s_loc[wb + q0 + u] : INT_MIN;
                run = max(run, v[u]);
            }
            // exclusive max over the lanes below (wave_shr:1 of the inclusive scan)
            int c = __builtin_amdgcn_update_dpp(INT_MIN, wave_incl_max_scan(run), 0x138, 0xF, 0xF, false);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                c = max(c, v[u]);
                if (u < per && q0 + u < pb) {
                    const int cc = max(c, 0);
                    const int j = jlo + (q0 + u - pa);
                    s_loc[wb + q0 + u] = min(max(O[cc] + (j - P[cc]), 0), lmax);
                }
            }
        }
    }
    // every wave is done with the staged selection before any wave writes
    // its K / V tiles over it
    if constexpr (!FAST) __syncthreads();

    // ---- stream this wave's quarter of the rows ----
    const uint16_t* skh = a.sk + static_cast<int64_t>(h) * a.s_stride * 128;
    const uint16_t* svh = a.sv + static_cast<int64_t>(h) * a.s_stride * 128;
    const uint16_t* lkh = a.lk + static_cast<int64_t>(h) * a.list_rows * 128;
    const uint16_t* lvh = a.lv + static_cast<int64_t>(h) * a.list_rows * 128;
    f32x4_t acc[8];   // acc[d][r] = O[query slot 4lg + r][dim 16d + ln]
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[d] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m_own = -INFINITY, l_own = 0.0f;   // softmax state of query slot ln
    uint16_t* sv = s_v + wave * 16 * kVStride;
    uint16_t* sk = s_k + wave * 16 * kVStride;
    const int nt = (wn + 15) >> 4;
    if (nt > 0) {
        // Tile t: rows wb + t*16 + 4it + rg, 16 lanes x 16 bytes per row.
        // Rows past the wave's end read list row 0 (in bounds) and are masked.
        const int rg = lane >> 4, li = lane & 15;
        u32x4_t kb[kPF][4], vb[kPF][4];
        auto load = [&](int t, auto slot_c) {
            constexpr int SLOT = decltype(slot_c)::value;
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int jt = t * 16 + it * 4 + rg;
                int lr;
                if constexpr (FAST) {
                    // row jt sits in lane jt % 64 of loc[t / 4] (t / 4 is
                    // wave-uniform); every lane takes part in the shuffle
                    int src = loc[0];
#pragma unroll
                    for (int r = 1; r < NR; ++r) src = (t >> 2) == r ? loc[r] : src;
                    const int v = __shfl(src, jt & 63);
                    lr = jt < wn ? v : 0;
                } else {
                    lr = jt < wn ? s_loc[wb + jt] : 0;
                }
                const bool steady = lr < 0;
                const int64_t roff = static_cast<int64_t>(steady ? -1 - lr : lr) * 128;
                kb[SLOT][it] = __builtin_nontemporal_load((g_u32x4_t*)((steady ? skh : lkh) + roff + li * 8));
                vb[SLOT][it] = __builtin_nontemporal_load((g_u32x4_t*)((steady ? svh : lvh) + roff + li * 8));
            }
        };
        auto body = [&](int t, auto slot_c, auto prefetch_c) {
            constexpr int SLOT = decltype(slot_c)::value;
            // K and V tiles -> LDS, row-major [token][dim]; K comes back in the
            // MFMA A layout (lane -> token ln, dims 32c + 8lg)
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                *reinterpret_cast<u32x4_t*>(sv + (4 * it + rg) * kVStride + li * 8) = vb[SLOT][it];
                *reinterpret_cast<u32x4_t*>(sk + (4 * it + rg) * kVStride + li * 8) = kb[SLOT][it];
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
            if constexpr (decltype(prefetch_c)::value) load(t + kPF, slot_c);
            float s[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) s[i] = (t * 16 + 4 * lg + i < wn) ? s4[i] * a.scale_log2 : -INFINITY;
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
        };
        // Groups of kPF tiles, every load and body unconditional (so that the
        // waits before each tile count exactly the loads issued after it):
        // the tiles past nt in the last group are masked and read list row 0.
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using S2 = std::integral_constant<int, 2>;
        using S3 = std::integral_constant<int, 3>;
        using Pf = std::true_type;
        using NoPf = std::false_type;
        auto group = [&](int t0, auto pf) {
            body(t0, S0{}, pf);
            body(t0 + 1, S1{}, pf);
            if constexpr (kPF == 4) {
                body(t0 + 2, S2{}, pf);
                body(t0 + 3, S3{}, pf);
            }
        };
        static_assert(kPF == 2 || kPF == 4, "two or four tile slots");
        load(0, S0{});
        load(1, S1{});
        if constexpr (kPF == 4) {
            load(2, S2{});
            load(3, S3{});
        }
        const int ng = (nt + kPF - 1) / kPF;
        for (int g = 0; g + 1 < ng; ++g) group(g * kPF, Pf{});
        group((ng - 1) * kPF, NoPf{});
    }
    // sum over the four lane groups (different tokens, shared max)
    l_own += xor16(l_own);
    l_own += xor32(l_own);
    // query g: O row g (lane group g / 4, register g % 4), state of slot g
#pragma unroll
    for (int g = 0; g < G; ++g)
        if (lg == g / 4) {
#pragma unroll
            for (int d = 0; d < 8; ++d) s_acc[(wave * G + g) * 128 + d * 16 + ln] = acc[d][g % 4];
        }
    if (lg == 0 && ln < G) {
        s_ml[(wave * G + ln) * 2 + 0] = m_own;
        s_ml[(wave * G + ln) * 2 + 1] = l_own;
    }
    __syncthreads();
    // workgroup partial (waves merged in order); an empty split writes an
    // empty state (max -inf, sum 0), which the merge weighs 0
    const int64_t pidx = pbase + split;
    for (int o = tid; o < G * 128; o += kThreads) {
        const int g = o >> 7, d = o & 127;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_ml[(w * G + g) * 2]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float wt = wexp(s_ml[(w * G + g) * 2], M);
            L += s_ml[(w * G + g) * 2 + 1] * wt;
            A += s_acc[(w * G + g) * 128 + d] * wt;
        }
        a.part_acc[(pidx * G + g) * 128 + d] = A;
        if (d == 0) {
            a.part_ml[(pidx * G + g) * 2 + 0] = M;
            a.part_ml[(pidx * G + g) * 2 + 1] = L;
        }
    }
}

// Merge of the S partials of one head for 64 outputs (query head g = chunk
// / 2, dims (chunk % 2) * 64 ..).  Every load of the first 64 splits
// (partial sums, and the max / sum pairs that wave 0 turns into split
// weights) is issued at once; each of the four waves sums a quarter of the
// splits (s = q, q + 4, ...) and the quarters are added in a fixed order
// (deterministic).
__global__ __launch_bounds__(256) void merge_kernel(DecParams a, int G) {
    __shared__ float s_w[kMaxSplit];
    __shared__ float s_red[4][64];
    __shared__ float s_ML[2];
    const int h = blockIdx.y, chunk = blockIdx.x;
    const int g = chunk >> 1;
    const int tid = threadIdx.x, q = tid >> 6, lane = tid & 63;
    const int o = chunk * 64 + lane;  // g * 128 + d
    // this head's run: its splits and first partial (component selects)
    int rx = a.run[0].x, ry = a.run[0].y, rz = a.run[0].z;
#pragma unroll
    for (int i = 1; i < kMaxRuns; ++i) {
        const bool in = a.run[i].y <= h && a.run[i].x != INT_MAX;
        rx = in ? a.run[i].x : rx;
        ry = in ? a.run[i].y : ry;
        rz = in ? a.run[i].z : rz;
    }
    const int ns = max(rz & 0xFFFF, 1);
    const int64_t first = rx + static_cast<int64_t>(h - ry) * ns;
    const int64_t stride = static_cast<int64_t>(G) * 128;
    const float* pacc = a.part_acc + first * stride + o;
    const float* pml = a.part_ml + (first * G + g) * 2;
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int s = q + 4 * u;
        v[u] = s < ns ? pacc[s * stride] : 0.0f;
    }
    if (q == 0) {
        float pm = -INFINITY, pl = 0.0f;
        if (lane < ns) {
            pm = pml[static_cast<int64_t>(lane) * G * 2];
            pl = pml[static_cast<int64_t>(lane) * G * 2 + 1];
        }
        float M = pm;
        for (int s = lane + 64; s < ns; s += 64) M = fmaxf(M, pml[static_cast<int64_t>(s) * G * 2]);
        M = wave_max(M);
        const float w = lane < ns ? wexp(pm, M) : 0.0f;
        if (lane < ns) s_w[lane] = w;
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
    float accv = 0.0f;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int s = q + 4 * u;
        if (s < ns) accv = __builtin_fmaf(v[u], s_w[s], accv);
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
            if (s < ns) accv = __builtin_fmaf(v[u], s_w[s], accv);
        }
    }
    s_red[q][lane] = accv;
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


// The merge for heads of at most SMAX (32 or 64) splits: one wave per (head,
// query head, 64 dims), no LDS and no barrier.  Lane s holds split s's (max,
// sum), the split weights come from one wave max and one wave sum, and each
// lane (one output dim) adds its partials in split order with the weights
// read lane by lane (deterministic).  Loads and adds are unconditional:
// splits past the head's count re-read its last partial and weigh 0.
constexpr int kMergeWaveSplits = 64;

template <int SMAX>
__global__ __launch_bounds__(64) void merge_wave_kernel(DecParams a, int G) {
    const int h = blockIdx.y, chunk = blockIdx.x;
    const int g = chunk >> 1;
    const int lane = threadIdx.x;
    const int o = chunk * 64 + lane;   // g * 128 + d
    int rx = a.run[0].x, ry = a.run[0].y, rz = a.run[0].z;
#pragma unroll
    for (int i = 1; i < kMaxRuns; ++i) {
        const bool in = a.run[i].y <= h && a.run[i].x != INT_MAX;
        rx = in ? a.run[i].x : rx;
        ry = in ? a.run[i].y : ry;
        rz = in ? a.run[i].z : rz;
    }
    const int ns = min(max(rz & 0xFFFF, 1), SMAX);
    const int64_t first = rx + static_cast<int64_t>(h - ry) * ns;
    const int64_t stride = static_cast<int64_t>(G) * 128;
    const float* pacc = a.part_acc + first * stride + o;
    const float* pml = a.part_ml + (first * G + g) * 2;
    float v[SMAX];
#pragma unroll
    for (int s = 0; s < SMAX; ++s) v[s] = pacc[min(s, ns - 1) * stride];
    const int sl = min(lane, ns - 1);
    const float pm0 = pml[static_cast<int64_t>(sl) * G * 2];
    const float pl0 = pml[static_cast<int64_t>(sl) * G * 2 + 1];
    const float pm = lane < ns ? pm0 : -INFINITY;
    const float M = wave_max(pm);
    const float w = wexp(pm, M);   // 0 past ns and for empty splits
    const float L = wave_sum(lane < ns ? pl0 * w : 0.0f);
    float A = 0.0f;
#pragma unroll
    for (int s = 0; s < SMAX; ++s) A = __builtin_fmaf(v[s], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), s)), A);
    a.out[static_cast<int64_t>(h) * G * 128 + o] = f32_to_bf16(L > 0.0f ? A / L : 0.0f);
    if (a.lse && lane == 0 && (chunk & 1) == 0)
        a.lse[static_cast<int64_t>(h) * G + g] = L > 0.0f ? (M + log2f(L)) * 0.69314718055994530942f : -INFINITY;
}

// ------------------------------------------------- fixed-grid split pass
// The decode step's split pass when every head has the same row bound and at
// most kFixedCap selected cells (the selection of imi_select: every cell
// holds at least one row): workgroup b takes split b / H of head
// (b % H + split) % H and the rows [split * 64 NT, + 64 NT) of that head's
// [static | selected | delta] rows, NT tiles of 16 rows per wave, the tile
// loop unrolled at compile time.  The head's selection is staged in LDS in
// one round trip; each wave finds the cell of its first row with two ballot
// rounds over the staged prefix, flags the window offsets where the next
// cells start and counts the flags up to each row.  A split past the head's
// rows writes an empty partial (max -inf, sum 0), which the merge weighs 0.
// At configs[1] this form runs the split pass in 12.4 us against 13.3 us for
// the row-balanced form (whose per-split ranges follow the rows each head
// actually selected, for ragged batches and larger shapes).
constexpr int kFixedCap = 2048;   // selected cells per head the fixed grid stages

__device__ __forceinline__ int popc_upto(uint64_t lo, uint64_t hi, int i) {   // set bits at positions 0..i
    if (i < 64) return __builtin_popcountll(lo & (~0ull >> (63 - i)));
    return __builtin_popcountll(lo) + __builtin_popcountll(hi & (~0ull >> (127 - i)));
}

template <int G, int NT, bool DELTA>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void fixed_attention_kernel(
    DecParams a) {
    constexpr int RW = NT * 16;                 // rows per wave
    constexpr int NRL = (RW + 63) / 64;         // row locations per lane
    static_assert(NRL <= 2, "the row lookup covers windows of at most 128 rows");
    constexpr int SU = (kFixedCap + kThreads) / kThreads;
    constexpr int DU = kDeltaMax / kThreads;
    __shared__ float s_acc[kWaves][G][128];
    __shared__ float s_ml[kWaves][G][2];
    __shared__ int s_pre[kFixedCap + 1];
    __shared__ int s_off[kFixedCap];
    __shared__ int s_drow[DELTA ? kDeltaMax : 1];
    __shared__ int s_flag[kWaves][NRL * 64];
    __shared__ __attribute__((aligned(16))) uint16_t s_v[kWaves][16 * kVStride];
    __shared__ __attribute__((aligned(16))) uint16_t s_k[kWaves][16 * kVStride];

    const int b = blockIdx.x;
    const int H = a.H, S = a.run[0].z & 0xFFFF;
    const int split = b / H;
    const int h = (b % H + split) % H;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lg = lane >> 4, ln = lane & 15;
    const int row0 = split * (64 * NT) + wave * RW;

    // one round trip: q (as the MFMA B operand: column ln = query ln % G,
    // dims 32c + 8lg ..), the row and cell counts, the head's selection (row
    // prefix and CSR offset per cell) and its delta rows
    u32x4_t qb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        qb[c] = *reinterpret_cast<const u32x4_t*>(a.q + (static_cast<int64_t>(h) * G + ln % G) * 128 + c * 32 + lg * 8);
    const int nrows_raw = vec_load_i32(a.g_nrows, h);
    const int m_raw = vec_load_i32(a.g_nsel, h);
    const int nd_raw = DELTA ? vec_load_i32(a.g_ndelta, h) : 0;
    {
        const int32_t* pre = a.g_prefix + static_cast<int64_t>(h) * (a.g_cap + 1);
        const int32_t* off = a.g_offset + static_cast<int64_t>(h) * a.g_cap;
        int pv[SU], ov[SU];
#pragma unroll
        for (int u = 0; u < SU; ++u) {
            const int i = tid + u * kThreads;
            pv[u] = i <= a.g_cap ? pre[i] : 0;
            ov[u] = i < a.g_cap ? off[i] : 0;
        }
        int dv[DELTA ? DU : 1];
        if constexpr (DELTA) {
#pragma unroll
            for (int u = 0; u < DU; ++u) {
                const int i = tid + u * kThreads;
                dv[u] = i < a.g_dcap ? a.g_drows[static_cast<int64_t>(h) * a.g_dcap + i] : 0;
            }
        }
#pragma unroll
        for (int u = 0; u < SU; ++u) {
            const int i = tid + u * kThreads;
            if (i <= a.g_cap) s_pre[i] = pv[u];
            if (i < a.g_cap) s_off[i] = ov[u];
        }
        if constexpr (DELTA) {
#pragma unroll
            for (int u = 0; u < DU; ++u) s_drow[tid + u * kThreads] = dv[u];
        }
    }
    __syncthreads();
    const int nrows = max(__builtin_amdgcn_readfirstlane(nrows_raw), 0);
    const int m = min(max(__builtin_amdgcn_readfirstlane(m_raw), 0), a.g_cap);
    const int nd = DELTA ? min(max(__builtin_amdgcn_readfirstlane(nd_raw), 0), a.g_dcap) : 0;
    const int sl = a.static_len;
    // rows: [static_len steady rows | nrows list rows | nd delta rows (steady)]
    const int N = sl + nrows + nd;
    const int64_t pidx = static_cast<int64_t>(h) * S + split;
    if (split * (64 * NT) >= N) {   // no rows in this split: an empty partial
        for (int o = tid; o < G * 128; o += kThreads) a.part_acc[pidx * G * 128 + o] = 0.0f;
        if (tid < G) {
            a.part_ml[(pidx * G + tid) * 2 + 0] = -INFINITY;
            a.part_ml[(pidx * G + tid) * 2 + 1] = 0.0f;
        }
        return;
    }

    // list row of window row i (rows row0 + i, i = lane + 64 r): the cell c0
    // holding the wave's first list row j0 comes from two ballot rounds over
    // the staged prefix, the window offsets where the following cells start
    // are flagged, and the flags are counted up to each row.  Locations are
    // clamped to the list; a delta row gets -1 - its steady row (clamped to
    // the steady zone).
    int loc[NRL];
    {
        const int j0 = max(row0 - sl, 0);
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
        for (int r = 0; r < NRL; ++r) fl[lane + 64 * r] = 0;
        wave_lds_sync();
#pragma unroll
        for (int r = 0; r < NRL; ++r) {
            const int c = c0 + 1 + lane + 64 * r;
            if (c < m) {
                const int o = s_pre[c] - j0;
                if (o > 0 && o < NRL * 64) fl[o] = 1;
            }
        }
        wave_lds_sync();
        uint64_t fm[2] = {0ull, 0ull};
#pragma unroll
        for (int r = 0; r < NRL; ++r) fm[r] = __builtin_amdgcn_ballot_w64(fl[lane + 64 * r] != 0);
        const int lmax = max(a.list_rows - 1, 0);
#pragma unroll
        for (int r = 0; r < NRL; ++r) {
            const int j = row0 + lane + 64 * r - sl;
            int l = 0;
            if (j >= 0 && j < nrows) {
                const int c = c0 + popc_upto(fm[0], fm[1], j - j0);
                l = min(max(s_off[c] + (j - s_pre[c]), 0), lmax);
            } else if (DELTA && j >= nrows && j < nrows + nd) {
                l = -1 - min(max(s_drow[j - nrows], 0), a.s_stride - 1);
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
        // tile t: rows t*16 + 4it + rg, 16 lanes x 16 bytes per row; rows past
        // N read list row 0 (in bounds) and are masked below
        const int rg = lane >> 4, li = lane & 15;
        u32x4_t kb[2][4], vb[2][4];
        auto load = [&](int t, int slot) {
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int jt = t * 16 + it * 4 + rg;
                const int n = row0 + jt;
                const int lr = __shfl(loc[(t * 16) >> 6], jt & 63);
                const bool st = n < sl;
                const bool dl = DELTA && !st && n < N && lr < 0;   // delta row: steady row -1 - lr
                const int64_t roff =
                    (st ? static_cast<int64_t>(n) : static_cast<int64_t>(dl ? -1 - lr : (n < N ? lr : 0))) * 128;
                kb[slot][it] = __builtin_nontemporal_load((g_u32x4_t*)((st || dl ? skh : lkh) + roff + li * 8));
                vb[slot][it] = __builtin_nontemporal_load((g_u32x4_t*)((st || dl ? svh : lvh) + roff + li * 8));
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
            for (int i = 0; i < 4; ++i) s[i] = (row0 + t * 16 + 4 * lg + i < N) ? s4[i] * a.scale_log2 : -INFINITY;
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
                // in lane 16lg + 4lg + r (any lane of that slot would do)
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
    // workgroup partial (waves merged in order)
    for (int o = tid; o < G * 128; o += kThreads) {
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
        a.part_acc[(pidx * G + g) * 128 + d] = A;
        if (d == 0) {
            a.part_ml[(pidx * G + g) * 2 + 0] = M;
            a.part_ml[(pidx * G + g) * 2 + 1] = L;
        }
    }
}

// Rows one split may hold for any call of this shape: any static_len up to
// steady_stride (so one workspace and one captured launch shape stay valid
// while the steady zone grows), the selected rows, the delta rows.
int64_t rows_bound(const imi_attention_args* a) {
    const int64_t srows = a->steady_stride > a->static_len ? a->steady_stride : a->static_len;
    return srows + a->max_rows;
}

// About one workgroup per CU in all.
int64_t splits_one_round(const imi_attention_args* a) {
    const int64_t s = (device_cus() + a->kv_heads - 1) / a->kv_heads;
    return s < 1 ? 1 : s;
}

// The short form when the selection fits its staging and one round of
// workgroups keeps every split within fast_rows(NR) rows: the row
// locations per lane, or 0 for the general form.
int attn_nr(const imi_attention_args* a) {
    if (a->sel_cap > kFastCap) return 0;
    for (int nr = 2; nr <= kFastNRMax; nr += 2)
        if (rows_bound(a) <= splits_one_round(a) * fast_rows(nr)) return nr;
    return 0;
}

// Splits per head: about one workgroup per CU in all, and enough that no
// split holds more than kLocCap rows.
int splits_per_head(const imi_attention_args* a) {
    int64_t s = splits_one_round(a);
    const int64_t need = (rows_bound(a) + kLocCap - 1) / kLocCap;
    if (s < need) s = need;
    return static_cast<int>(s);
}

uint32_t div_magic(int n) {   // floor(2^32 / n) + 1, or 0 for n = 1 (quotient = dividend)
    return n > 1 ? static_cast<uint32_t>((uint64_t(1) << 32) / static_cast<uint64_t>(n) + 1) : 0u;
}

// Workgroups of the split pass.  Equal splits per head (S > 0), or, with
// per-head row bounds that form 2..kMaxRuns runs of equal bounds (a ragged
// batch), splits proportional to each run's bound.
struct SplitPlan {
    int S = 0;
    int total = 0;   // workgroups = partials
    int nr = 0;      // the short form's row locations per lane
    int fixed_nt = 0;   // tiles per wave of the fixed grid (0: row-balanced)
    int4 run[kMaxRuns];
};

// Tiles per wave of the fixed-grid split pass: the fewest in [4, 8] whose
// grid (64 NT rows per workgroup) fits the CUs in one round, or 0.  Only for
// selections made by imi_select (fixed_ok: every selected cell holds a row)
// with one row bound for every head.
int fixed_tiles(const imi_attention_args* a, bool fixed_ok) {
    if (!fixed_ok || a->sel_cap > kFixedCap) return 0;
    if (a->head_rows_bound)
        for (int h = 1; h < a->kv_heads; ++h)
            if (a->head_rows_bound[h] != a->head_rows_bound[0]) return 0;
    const int64_t rb = rows_bound(a);
    if (a->rows_hint > 0 && 2 * static_cast<int64_t>(a->rows_hint) < rb) return 0;   // mostly empty windows
    for (int nt = 4; nt <= 8; ++nt)
        if (static_cast<int64_t>(a->kv_heads) * ((rb + 64 * nt - 1) / (64 * nt)) <= device_cus()) return nt;
    return 0;
}

SplitPlan split_plan(const imi_attention_args* a, bool fixed_ok = false) {
    SplitPlan P;
    const int H = a->kv_heads;
    const int64_t rb = rows_bound(a);
    for (int r = 0; r < kMaxRuns; ++r) P.run[r] = make_int4(INT_MAX, H, 0, 0);
    if ((P.fixed_nt = fixed_tiles(a, fixed_ok)) > 0) {
        P.S = static_cast<int>((rb + 64 * P.fixed_nt - 1) / (64 * P.fixed_nt));
        P.total = H * P.S;
        P.run[0] = make_int4(0, 0, P.S | (H << 16), static_cast<int>(div_magic(H)));
        return P;
    }
    if (a->head_rows_bound && H > 1) {
        int nruns = 0;
        int h0[kMaxRuns];
        int64_t B[kMaxRuns];
        bool ok = true;
        for (int h = 0; h < H && ok; ++h) {
            int64_t bh = a->head_rows_bound[h];
            bh = bh < 1 ? 1 : (bh > rb ? rb : bh);   // never above the launch-wide bound
            if (h == 0 || bh != B[nruns - 1]) {
                if (nruns == kMaxRuns) {
                    ok = false;
                } else {
                    h0[nruns] = h;
                    B[nruns] = bh;
                    ++nruns;
                }
            }
        }
        if (ok && nruns > 1) {
            int64_t tot = 0;
            for (int r = 0; r < nruns; ++r) tot += B[r] * ((r + 1 < nruns ? h0[r + 1] : H) - h0[r]);
            const int64_t T = device_cus() > H ? device_cus() : H;
            int64_t wg = 0, per = 0;
            for (int r = 0; r < nruns; ++r) {
                const int nh = (r + 1 < nruns ? h0[r + 1] : H) - h0[r];
                int64_t S = T * B[r] / tot;
                const int64_t need = (B[r] + kLocCap - 1) / kLocCap;
                S = S < need ? need : S;
                S = S < 1 ? 1 : (S > kMaxSplit ? kMaxSplit : S);
                P.run[r] = make_int4(static_cast<int>(wg), h0[r], static_cast<int>(S) | (nh << 16),
                                     static_cast<int>(div_magic(nh)));
                wg += nh * S;
                const int64_t rows = (B[r] + S - 1) / S;
                per = rows > per ? rows : per;
            }
            P.S = 0;
            P.total = static_cast<int>(wg);
            if (a->sel_cap <= kFastCap)
                for (int nr = 2; nr <= kFastNRMax && P.nr == 0; nr += 2)
                    if (per <= fast_rows(nr)) P.nr = nr;
            return P;
        }
    }
    P.S = splits_per_head(a);
    P.total = H * P.S;
    P.nr = attn_nr(a);
    P.run[0] = make_int4(0, 0, P.S | (H << 16), static_cast<int>(div_magic(H)));
    return P;
}

size_t attn_workspace(const imi_attention_args* a, DecParams* p, bool fixed_ok = false) {
    const SplitPlan P = split_plan(a, fixed_ok);
    Carver cv(a->workspace);
    float* acc = cv.take<float>(static_cast<size_t>(P.total) * a->groups * 128);
    float* ml = cv.take<float>(static_cast<size_t>(P.total) * a->groups * 2);
    if (p) {
        p->part_acc = acc;
        p->part_ml = ml;
        p->total = P.total;
        p->nr = P.nr;
        p->fixed_nt = P.fixed_nt;
        for (int r = 0; r < kMaxRuns; ++r) p->run[r] = P.run[r];
    }
    return cv.used();
}

int attn_validate(const imi_attention_args* a, bool need_sel) {
    IMI_REQUIRE(a != nullptr, IMI_ERR_INVALID, "imi_sparse_attention: null args");
    IMI_REQUIRE(a->dim == 128, IMI_ERR_UNSUPPORTED, "imi_sparse_attention: head_dim must be 128");
    IMI_REQUIRE(groups_supported(a->groups), IMI_ERR_UNSUPPORTED,
                "imi_sparse_attention: %d query heads per kv head unsupported (1..8 or 16)", a->groups);
    IMI_REQUIRE(a->kv_heads > 0, IMI_ERR_INVALID, "imi_sparse_attention: kv_heads must be > 0");
    IMI_REQUIRE(a->kv_heads < 32768, IMI_ERR_UNSUPPORTED, "imi_sparse_attention: %d kv heads exceed 32767", a->kv_heads);
    IMI_REQUIRE(a->query && a->out, IMI_ERR_INVALID, "imi_sparse_attention: null query/out");
    IMI_REQUIRE(a->static_len >= 0 && a->static_len <= a->steady_stride, IMI_ERR_INVALID,
                "imi_sparse_attention: static_len %d outside steady zone of %lld rows", a->static_len,
                static_cast<long long>(a->steady_stride));
    IMI_REQUIRE(a->static_len == 0 || (a->steady_keys && a->steady_values), IMI_ERR_INVALID,
                "imi_sparse_attention: null steady zone");
    IMI_REQUIRE(a->list_keys && a->list_values && a->list_rows > 0, IMI_ERR_INVALID,
                "imi_sparse_attention: null or empty list");
    IMI_REQUIRE(a->list_rows < (int64_t(1) << 31) && a->steady_stride < (int64_t(1) << 31), IMI_ERR_UNSUPPORTED,
                "imi_sparse_attention: list_rows / steady_stride must be below 2^31");
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
    IMI_REQUIRE(a->sel_cap >= 0, IMI_ERR_INVALID, "imi_sparse_attention: sel_cap must be >= 0");
    IMI_REQUIRE(a->sel_cap <= stage_max(a->groups), IMI_ERR_UNSUPPORTED, "imi_sparse_attention: sel_cap %d above %d",
                a->sel_cap, stage_max(a->groups));
    IMI_REQUIRE(splits_per_head(a) <= kMaxSplit, IMI_ERR_UNSUPPORTED,
                "imi_sparse_attention: %lld rows need more than %d splits per head",
                static_cast<long long>(rows_bound(a)), kMaxSplit);
    // the kernel splits its workgroup index by a 32-bit multiply-high
    IMI_REQUIRE(static_cast<uint64_t>(split_plan(a).total) * a->kv_heads < (uint64_t(1) << 32), IMI_ERR_UNSUPPORTED,
                "imi_sparse_attention: %d kv heads x %d workgroups too large", a->kv_heads, split_plan(a).total);
    return IMI_OK;
}

void fill_common(const imi_attention_args* a, DecParams* p) {
    p->q = a->query;
    p->sk = a->steady_keys ? a->steady_keys : a->list_keys;   // never read when static_len = 0 and no delta rows
    p->sv = a->steady_values ? a->steady_values : a->list_values;
    p->s_stride = a->steady_keys ? static_cast<int>(a->steady_stride) : 1;
    p->static_len = a->static_len;
    p->lk = a->list_keys;
    p->lv = a->list_values;
    p->list_rows = static_cast<int>(a->list_rows);
    p->H = a->kv_heads;
    p->scale_log2 = a->scale * 1.44269504088896340736f;
    p->out = a->out;
    p->lse = a->out_lse;
}

// Words of the staged selection's region: the row prefix (cap + 1, padded
// to 4 words) and the offsets, or the two K / V tiles if those are larger.
int stage_obase(int cap) { return (cap + 1 + 3) & ~3; }
int stage_words(int cap) {
    const int w = stage_obase(cap) + ((cap + 3) & ~3);
    return w > kTileWords ? w : kTileWords;
}

template <int G>
int launch_att(const DecParams& p, hipStream_t stream) {
    static bool attr_set = false;
    if (!attr_set) {
        constexpr size_t lds_max = static_cast<size_t>(2 * (stage_max(G) + 4) + tail_words<G>()) * 4;
        constexpr size_t lds_fast = static_cast<size_t>(fast_words<G>()) * 4;
        static_assert(lds_max <= 160 * 1024 && lds_fast <= 160 * 1024, "LDS of one workgroup");
        IMI_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_kernel<G, 0>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_max)));
        IMI_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_kernel<G, 2>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_fast)));
        IMI_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_kernel<G, 4>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_fast)));
        attr_set = true;
    }
    const size_t lds_fast = static_cast<size_t>(fast_words<G>()) * 4;
    if (p.fixed_nt > 0) {
        const bool delta = p.g_drows != nullptr;
        auto go = [&](auto kern) { hipLaunchKernelGGL(kern, dim3(p.total), dim3(kThreads), 0, stream, p); };
        switch (p.fixed_nt * 2 + (delta ? 1 : 0)) {
            case 8: go(fixed_attention_kernel<G, 4, false>); break;
            case 9: go(fixed_attention_kernel<G, 4, true>); break;
            case 10: go(fixed_attention_kernel<G, 5, false>); break;
            case 11: go(fixed_attention_kernel<G, 5, true>); break;
            case 12: go(fixed_attention_kernel<G, 6, false>); break;
            case 13: go(fixed_attention_kernel<G, 6, true>); break;
            case 14: go(fixed_attention_kernel<G, 7, false>); break;
            case 15: go(fixed_attention_kernel<G, 7, true>); break;
            case 16: go(fixed_attention_kernel<G, 8, false>); break;
            default: go(fixed_attention_kernel<G, 8, true>); break;
        }
    } else if (p.nr == 2) {
        hipLaunchKernelGGL((attention_kernel<G, 2>), dim3(p.total), dim3(kThreads), lds_fast, stream, p);
    } else if (p.nr == 4) {
        hipLaunchKernelGGL((attention_kernel<G, 4>), dim3(p.total), dim3(kThreads), lds_fast, stream, p);
    } else {
        const size_t lds = static_cast<size_t>(p.stage_words + tail_words<G>()) * 4;
        hipLaunchKernelGGL((attention_kernel<G, 0>), dim3(p.total), dim3(kThreads), lds, stream, p);
    }
    IMI_LAUNCH_CHECK("attention_kernel");
    return IMI_OK;
}

// kernels: bit 0 the split pass, bit 1 the merge (which reads the partials
// the last split pass left in the workspace).
int attn_run(const DecParams& p, int groups, hipStream_t stream, int kernels) {
    int rc = IMI_OK;
    if (kernels & 1) {
        switch (groups) {
            case 1: rc = launch_att<1>(p, stream); break;
            case 2: rc = launch_att<2>(p, stream); break;
            case 3: rc = launch_att<3>(p, stream); break;
            case 4: rc = launch_att<4>(p, stream); break;
            case 5: rc = launch_att<5>(p, stream); break;
            case 6: rc = launch_att<6>(p, stream); break;
            case 7: rc = launch_att<7>(p, stream); break;
            case 8: rc = launch_att<8>(p, stream); break;
            default: rc = launch_att<16>(p, stream); break;   // groups_supported: 16
        }
        if (rc) return rc;
    }
    if (kernels & 2) {
        int smax = 0;   // the most splits of any head
        for (int r = 0; r < kMaxRuns; ++r)
            if (p.run[r].x != INT_MAX) smax = std::max(smax, p.run[r].z & 0xFFFF);
        if (smax <= 32) {
            hipLaunchKernelGGL(merge_wave_kernel<32>, dim3(2 * groups, p.H), dim3(64), 0, stream, p, groups);
            IMI_LAUNCH_CHECK("merge_wave_kernel");
        } else if (smax <= kMergeWaveSplits) {
            hipLaunchKernelGGL(merge_wave_kernel<kMergeWaveSplits>, dim3(2 * groups, p.H), dim3(64), 0, stream, p,
                               groups);
            IMI_LAUNCH_CHECK("merge_wave_kernel");
        } else {
            hipLaunchKernelGGL(merge_kernel, dim3(2 * groups, p.H), dim3(256), 0, stream, p, groups);
            IMI_LAUNCH_CHECK("merge_kernel");
        }
    }
    return IMI_OK;
}

// Attention over a selection held in global memory (fixed_ok: made by
// imi_select, so every selected cell holds a row).
int attn_launch_given(const imi_attention_args* a, hipStream_t stream, int kernels, bool fixed_ok = false) {
    DecParams p{};
    attn_workspace(a, &p, fixed_ok);
    fill_common(a, &p);
    p.g_prefix = a->sel_prefix;
    p.g_offset = a->sel_offset;
    p.g_nsel = a->n_selected;
    p.g_nrows = a->n_rows;
    p.g_cap = a->sel_cap;
    p.g_drows = a->delta_rows;
    p.g_ndelta = a->n_delta;
    p.g_dcap = a->delta_cap;
    p.o_base = stage_obase(a->sel_cap);
    p.stage_words = stage_words(a->sel_cap);
    return attn_run(p, a->groups, stream, kernels);
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
    return attn_launch_given(a, stream, 3);
}

namespace {
struct DecodeLayout {
    int32_t *cell, *off, *cnt, *prefix, *nsel, *nrows;
    int32_t *drows, *ndelta;   // delta append outputs (ring_cap > 0)
    char* sel_ws;              // 4-way selection scratch (empty for 2-way)
    size_t sel_bytes;
    char* attn_ws;
    size_t attn_bytes;
    char* zero_at;             // the words the kernels expect zero at the start of a call
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
    // the ranking pipeline's workspace (4-way, and 2-way beyond the one-kernel selection)
    L.sel_bytes = a->sel.parts == 4 ? select4_workspace_size(&a->sel) : sel2_keys_bytes(&a->sel);
    L.sel_ws = cv.take<char>(L.sel_bytes > 0 ? L.sel_bytes : 1);
    L.zero_bytes = L.sel_bytes > 0 ? select4_zero_bytes() : 0;
    L.zero_at = L.sel_ws;
    imi_attention_args t = a->attn;
    t.workspace = nullptr;
    L.attn_bytes = attn_workspace(&t, nullptr, true);
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
    IMI_REQUIRE(a->sel.sel_cap <= stage_max(a->sel.groups), IMI_ERR_UNSUPPORTED,
                "imi_decode_step: sel_cap %d above %d", a->sel.sel_cap, stage_max(a->sel.groups));
    int64_t nc;
    int km;
    int rc = select_validate(&a->sel, nc, km);
    if (rc) return rc;
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
// One decode step with its workspace at ws (already checked to be large
// enough): imi_select's kernels -> attention_kernel (given selection) ->
// merge_kernel.  phases (bits): 1 the selection, 4 attention_kernel, 8
// merge_kernel, 2 both of those.
int decode_run(const imi_decode_args* a, void* ws, hipStream_t stream) {
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
    s.workspace = L.sel_ws;
    s.workspace_bytes = L.sel_bytes;
    if (phases & 1) {
        const int rc = select_launch(&s, stream);
        if (rc) return rc;
    }
    if (!kernels) return IMI_OK;
    imi_attention_args t = a->attn;
    t.workspace = L.attn_ws;
    t.workspace_bytes = L.attn_bytes;
    t.sel_offset = s.sel_offset;
    t.sel_count = s.sel_count;
    t.sel_prefix = s.sel_prefix;
    t.n_selected = s.n_selected;
    t.n_rows = s.n_rows;
    t.sel_cap = s.sel_cap;
    t.delta_rows = s.ring_cap > 0 ? s.delta_rows : nullptr;
    t.n_delta = s.ring_cap > 0 ? s.n_delta : nullptr;
    t.delta_cap = s.ring_cap > 0 ? s.ring_cap : 0;
    return attn_launch_given(&t, stream, kernels, true);
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
