// Shared helpers of the gfx950 AdaptiveIMI kernels: error reporting through
// the C ABI, bf16 handling, wave64 cross-lane primitives.
#pragma once

#include <hip/hip_runtime.h>

#include <climits>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <type_traits>

#include "imi_hip.h"

namespace imi {

// ---------------------------------------------------------------- errors --
void set_error(const char* fmt, ...);
void clear_error();

#define IMI_REQUIRE(cond, code, ...)      \
    do {                                  \
        if (!(cond)) {                    \
            ::imi::set_error(__VA_ARGS__); \
            return (code);                \
        }                                 \
    } while (0)

#define IMI_HIP_CHECK(expr)                                                              \
    do {                                                                                 \
        hipError_t e_ = (expr);                                                          \
        if (e_ != hipSuccess) {                                                          \
            ::imi::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, \
                             __LINE__);                                                  \
            return IMI_ERR_HIP;                                                          \
        }                                                                                \
    } while (0)

#define IMI_LAUNCH_CHECK(name)                                                             \
    do {                                                                                   \
        hipError_t e_ = hipGetLastError();                                                 \
        if (e_ != hipSuccess) {                                                            \
            ::imi::set_error("launch of %s failed: %s", name, hipGetErrorString(e_));      \
            return IMI_ERR_HIP;                                                            \
        }                                                                                  \
    } while (0)

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Carves aligned sub-buffers out of one caller-provided workspace.
struct Carver {
    char* base;
    size_t off = 0;
    explicit Carver(void* b) : base(static_cast<char*>(b)) {}
    template <typename T>
    T* take(size_t count) {
        off = align_up(off, 256);
        T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
        off += count * sizeof(T);
        return p;
    }
    size_t used() const { return align_up(off, 256); }
};

// ------------------------------------------------------------------ bf16 --
__device__ __forceinline__ float bf16_lo(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t packed) { return __uint_as_float(packed & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return static_cast<uint16_t>((u >> 16) | 0x40);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// Element `col` of the G (<= 16) query rows of one KV head (row stride 128):
// rows past G re-read row G - 1, so the loads carry no per-row test and are
// all in flight at once; the upper eight only when G > 8 (a uniform branch).
__device__ __forceinline__ void load_group_rows(const uint16_t* qh, int G, int col, uint16_t (&qv)[16]) {
#pragma unroll
    for (int g = 0; g < 8; ++g) qv[g] = qh[min(g, G - 1) * 128 + col];
    if (G > 8) {
#pragma unroll
        for (int g = 8; g < 16; ++g) qv[g] = qh[min(g, G - 1) * 128 + col];
    } else {
#pragma unroll
        for (int g = 8; g < 16; ++g) qv[g] = 0;
    }
}

// fp32 -> uint32 whose unsigned order equals the float order (NaN-free input).
__device__ __forceinline__ uint32_t order_key(float f) {
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Compute units of the current device (queried once per device).
inline int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

// Centroids per subspace of a 2-way or 4-way IMI: the k-means E-step holds
// k x 64 fp32 rows in LDS (132 KB at 512), the 2-way ranking pipeline scores
// k * k <= 1024 x 256 cells per head.  512 covers the reference's adaptive k
// (layer_pipeline.cpp:177-228) up to 4M tokens.
constexpr int kImiMaxK = 512;

// ------------------------------------------------- LDS set of cell ids --
// Open-addressing set of non-negative ints in a kSetSize-int LDS table
// (empty = -1), filled at most half: inserts and lookups always end.
constexpr int kSetBits = 12;
constexpr int kSetSize = 1 << kSetBits;

__device__ __forceinline__ uint32_t set_slot(int key) {
    return (static_cast<uint32_t>(key) * 2654435761u) >> (32 - kSetBits);
}

__device__ __forceinline__ void set_insert(int* t, int key) {
    uint32_t i = set_slot(key);
    while (true) {
        const int prev = atomicCAS(&t[i], -1, key);
        if (prev == -1 || prev == key) return;
        i = (i + 1) & (kSetSize - 1);
    }
}

__device__ __forceinline__ bool set_find(const int* t, int key) {
    uint32_t i = set_slot(key);
    while (true) {
        const int v = t[i];
        if (v == key) return true;
        if (v == -1) return false;
        i = (i + 1) & (kSetSize - 1);
    }
}

// ----------------------------------------------------------- wave helpers --
constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

__device__ __forceinline__ uint64_t lanemask_lt() {
    const int l = lane_id();
    return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// Lanes of the wave (among `active`) whose `key` (first `bits` bits) equals
// this lane's key.
__device__ __forceinline__ uint64_t match_peers(uint32_t key, int bits, uint64_t active) {
    uint64_t peers = active;
    for (int b = 0; b < bits; ++b) {
        const uint64_t m = __ballot((key >> b) & 1u);
        peers &= ((key >> b) & 1u) ? m : ~m;
    }
    return peers;
}

// DPP row operations (rows of 16 lanes).  Control codes of the GFX9 DPP
// encoding: quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E, row_half_mirror =
// 0x141, row_mirror = 0x140.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of each DPP row; every lane of the row gets the sum.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    return v;
}

// Lane exchanges across the halves / rows of the wave with the gfx950
// permlane swaps (VALU, no LDS crossbar): value of lane ^ 32 and lane ^ 16.
__device__ __forceinline__ float xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(lane_id() < 32 ? r[1] : r[0]);
}
__device__ __forceinline__ float xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(((lane_id() >> 4) & 1) == 0 ? r[1] : r[0]);
}

// DPP controls used below: row_shr:n = 0x110 + n, row_bcast:15 = 0x142,
// row_bcast:31 = 0x143.  update_dpp(0, v, ...) returns 0 in lanes whose
// source is outside the row (or whose row is masked off).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xF, false);
}

// Inclusive prefix sum across the 64 lanes (row scans, then row carries).
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += dpp_i<0x111>(v);
    v += dpp_i<0x112>(v);
    v += dpp_i<0x114>(v);
    v += dpp_i<0x118>(v);
    v += dpp_i<0x142, 0xA>(v);
    v += dpp_i<0x143, 0xC>(v);
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
    return __builtin_amdgcn_readlane(wave_incl_scan(v), 63);
}

// Butterfly reductions (every lane gets the result; fixed order, so the
// result is the same on every call).
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    v += xor16(v);
    v += xor32(v);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    v = fmaxf(v, xor16(v));
    v = fmaxf(v, xor32(v));
    return v;
}

__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o));
    return v;
}

// Unsigned max over the 64 lanes on DPP row operations (no LDS round trips):
// row shifts and row broadcasts give lane 63 the maximum, which every lane
// then reads.  Lanes without a source contribute 0, the identity.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    auto sh = [](uint32_t x, auto ctrl_c, auto mask_c) {
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), decltype(ctrl_c)::value,
                                                                 decltype(mask_c)::value, 0xF, false));
    };
    using F = std::integral_constant<int, 0xF>;
    v = max(v, sh(v, std::integral_constant<int, 0x111>{}, F{}));
    v = max(v, sh(v, std::integral_constant<int, 0x112>{}, F{}));
    v = max(v, sh(v, std::integral_constant<int, 0x114>{}, F{}));
    v = max(v, sh(v, std::integral_constant<int, 0x118>{}, F{}));
    v = max(v, sh(v, std::integral_constant<int, 0x142>{}, std::integral_constant<int, 0xA>{}));
    v = max(v, sh(v, std::integral_constant<int, 0x143>{}, std::integral_constant<int, 0xC>{}));
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// p[i] through a vector load.  A load at a wave-uniform address becomes a
// scalar load, which the compiler may place after the wait for the vector
// loads issued before it -- one more memory round trip at a kernel's start.
// The zero offset below comes from a VGPR the compiler cannot see through,
// so the load is a vector load scheduled with the others; readfirstlane
// makes the value uniform again where it is used.
__device__ __forceinline__ int vec_load_i32(const int32_t* p, int64_t i) {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return p[i + z];
}

}  // namespace imi
