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

// Exclusive scan, in place, of n ints by one 1024-thread block.  `sh` is LDS
// of at least 32 ints.  Returns the total on every thread.
__device__ __forceinline__ int block_exclusive_scan_1024(int32_t* data, int64_t n, int* sh) {
    const int tid = threadIdx.x;
    const int64_t per = (n + 1023) / 1024;
    const int64_t lo = tid * per;
    const int64_t hi = lo + per < n ? lo + per : n;
    int local = 0;
    for (int64_t i = lo; i < hi; ++i) local += data[i];
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
    for (int64_t i = lo; i < hi; ++i) {
        const int v = data[i];
        data[i] = run;
        run += v;
    }
    const int total = sh[32];
    __syncthreads();
    return total;
}

}  // namespace imi
