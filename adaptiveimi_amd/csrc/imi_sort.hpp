// Device building blocks of the stable counting sorts used by the index
// build: a per-block (256 items) histogram with each item's stable rank among
// equal digits of its block, an exclusive scan of the [digit][block] counts,
// and the scatter.  Used for the k-means member lists (digit = subspace label)
// and for the LSD cell sort (one pass per subspace label), which together
// reproduce the reference's ascending-token counting sort
// (reorganize_core.cpp:287-295).
#pragma once

#include "imi_common.hpp"

namespace imi {

constexpr int kSortBlock = 256;  // items per histogram block (4 waves)

// Block-wide ranks.  `digit` < nbins (nbins <= 256), `valid` false for lanes
// past the end.  Writes hist[digit * nblk + blockIdx.x] (count of each digit
// in this block, every digit < nbins written) and returns the item's rank
// among earlier items of the block with the same digit.  `wcnt` is LDS of
// 4 * nbins ints.  Must be called by all 256 threads.
__device__ __forceinline__ int block_digit_rank(int digit, bool valid, int nbins, int nbits, int* wcnt,
                                                int32_t* hist, int nblk, int blk) {
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    for (int i = tid; i < 4 * nbins; i += kSortBlock) wcnt[i] = 0;
    __syncthreads();
    const uint64_t active = __ballot(valid);
    const uint64_t peers = match_peers(static_cast<uint32_t>(digit), nbits, active);
    const int in_wave = __popcll(peers & lanemask_lt());
    if (valid && in_wave == 0) wcnt[wave * nbins + digit] = __popcll(peers);
    __syncthreads();
    for (int c = tid; c < nbins; c += kSortBlock) {
        int run = 0;
        for (int w = 0; w < 4; ++w) {
            const int t = wcnt[w * nbins + c];
            wcnt[w * nbins + c] = run;
            run += t;
        }
        if (hist) hist[static_cast<int64_t>(c) * nblk + blk] = run;
    }
    __syncthreads();
    return valid ? wcnt[wave * nbins + digit] + in_wave : 0;
}

// The same ranks as positions in the block's digit-sorted order: the item's
// rank plus the count of smaller digits in the block (lofs, LDS of nbins
// ints).  The block's row of digit offsets goes to loff_row[0 .. nbins - 1]
// and its item count to loff_row[nbins] (one contiguous store per block).
// nbins <= 256; `wsum` is LDS of 4 ints.
__device__ __forceinline__ int block_digit_pos(int digit, bool valid, int nbins, int nbits, int* wcnt, int* lofs,
                                               int* wsum, int32_t* loff_row) {
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    for (int i = tid; i < 4 * nbins; i += kSortBlock) wcnt[i] = 0;
    __syncthreads();
    const uint64_t active = __ballot(valid);
    const uint64_t peers = match_peers(static_cast<uint32_t>(digit), nbits, active);
    const int in_wave = __popcll(peers & lanemask_lt());
    if (valid && in_wave == 0) wcnt[wave * nbins + digit] = __popcll(peers);
    __syncthreads();
    int run = 0;   // digit tid's count in this block
    if (tid < nbins) {
        for (int w = 0; w < 4; ++w) {
            const int t = wcnt[w * nbins + tid];
            wcnt[w * nbins + tid] = run;
            run += t;
        }
    }
    if (nbins <= 64) {   // one wave holds every digit: no cross-wave step
        if (wave == 0) {
            const int incl = wave_incl_scan(run);
            if (tid < nbins) {
                lofs[tid] = incl - run;
                loff_row[tid] = incl - run;
            }
            if (tid == 63) loff_row[nbins] = incl;
        }
    } else {
        const int incl = wave_incl_scan(run);
        if ((tid & 63) == 63) wsum[wave] = incl;
        __syncthreads();
        int before = incl - run;
        for (int w = 0; w < wave; ++w) before += wsum[w];
        if (tid < nbins) {
            lofs[tid] = before;
            loff_row[tid] = before;
        }
        if (tid == 255) loff_row[nbins] = before + run;
    }
    __syncthreads();
    return valid ? lofs[digit] + wcnt[wave * nbins + digit] + in_wave : 0;
}

// Exclusive scan, in place, of n ints by one 1024-thread block.  `sh` is LDS
// of at least 33 ints.  Returns the total on every thread.  Each thread owns a
// contiguous chunk; when n is a multiple of 4 and data 16-byte aligned the
// chunks are whole int4s read 8 at a time (8 loads in flight per thread).
typedef int __attribute__((ext_vector_type(4))) scan_i32x4_t;

__device__ __forceinline__ int block_exclusive_scan_1024(int32_t* data, int64_t n, int* sh) {
    const int tid = threadIdx.x;
    const bool vec = (n % 4) == 0 && (reinterpret_cast<uintptr_t>(data) & 15) == 0;
    int64_t per = (n + 1023) / 1024;
    if (vec) per = (per + 3) & ~static_cast<int64_t>(3);
    const int64_t lo = tid * per < n ? tid * per : n;
    const int64_t hi = lo + per < n ? lo + per : n;
    int local = 0;
    if (vec) {
        for (int64_t i = lo; i < hi; i += 32) {
            scan_i32x4_t v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = i + 4 * u < hi ? *reinterpret_cast<const scan_i32x4_t*>(data + i + 4 * u)
                                      : scan_i32x4_t{0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < 8; ++u) local += (v[u][0] + v[u][1]) + (v[u][2] + v[u][3]);
        }
    } else {
        for (int64_t i = lo; i < hi; ++i) local += data[i];
    }
    const int incl = wave_incl_scan(local);
    const int wave = tid >> 6;
    if (lane_id() == 63) sh[wave] = incl;
    __syncthreads();
    if (tid < 64) {
        int v = tid < 16 ? sh[tid] : 0;
        int s = wave_incl_scan(v);
        if (tid < 16) sh[16 + tid] = s - v;
        if (tid == 15) sh[32] = s;
    }
    __syncthreads();
    int run = sh[16 + wave] + incl - local;
    if (vec) {
        for (int64_t i = lo; i < hi; i += 32) {
            scan_i32x4_t v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = i + 4 * u < hi ? *reinterpret_cast<const scan_i32x4_t*>(data + i + 4 * u)
                                      : scan_i32x4_t{0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (i + 4 * u < hi) {
                    scan_i32x4_t o;
                    o[0] = run;
                    run += v[u][0];
                    o[1] = run;
                    run += v[u][1];
                    o[2] = run;
                    run += v[u][2];
                    o[3] = run;
                    run += v[u][3];
                    *reinterpret_cast<scan_i32x4_t*>(data + i + 4 * u) = o;
                }
            }
        }
    } else {
        for (int64_t i = lo; i < hi; ++i) {
            const int v = data[i];
            data[i] = run;
            run += v;
        }
    }
    const int total = sh[32];
    __syncthreads();
    return total;
}

}  // namespace imi
