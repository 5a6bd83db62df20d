// Shared device/host helpers for the gfx950 HELLO hot-path kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/helloot_hip.h"

namespace hm {

// ------------------------------------------------------------------------------------------------
// Error reporting: thread-local message behind hm_last_error().
// ------------------------------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

// Per-kernel HIP-event timing (hm_profile_enable); no-ops unless enabled.
bool profiling();
void prof_begin(hipStream_t st, const char* name);
void prof_end(hipStream_t st);
void prof_count(const char* name, int64_t count);  // adds to a name's count (queued rescans, ...)
// while alive, this thread's launches record no timing events and no counts
struct ProfileOff {
    ProfileOff();
    ~ProfileOff();
};

#define HM_CHECK_ARG(cond, ...)                                  \
    do {                                                         \
        if (!(cond)) return ::hm::fail(HM_EINVAL, __VA_ARGS__);  \
    } while (0)

#define HM_HIP(expr)                                                                              \
    do {                                                                                          \
        hipError_t hm_err_ = (expr);                                                              \
        if (hm_err_ != hipSuccess)                                                                \
            return ::hm::fail(HM_EHIP, "%s failed: %s", #expr, hipGetErrorString(hm_err_));     \
    } while (0)

#define HM_LAUNCH_CHECK(name)                                                                     \
    do {                                                                                          \
        hipError_t hm_err_ = hipGetLastError();                                                   \
        if (hm_err_ != hipSuccess)                                                                \
            return ::hm::fail(HM_EHIP, "%s launch failed: %s", name, hipGetErrorString(hm_err_)); \
    } while (0)

// Bump allocator over the caller's workspace (256-byte aligned slices).
struct Arena {
    char* base;
    size_t size;
    size_t used = 0;
    Arena(void* b, size_t s) : base(static_cast<char*>(b)), size(s) {}
    template <class T>
    T* take(size_t count) {
        size_t bytes = (count * sizeof(T) + 255) & ~size_t(255);
        if (base == nullptr || used + bytes > size) return nullptr;
        T* p = reinterpret_cast<T*>(base + used);
        used += bytes;
        return p;
    }
};

// Size calculator matching Arena::take.
struct Sizer {
    size_t used = 0;
    template <class T>
    T* take(size_t count) {
        used += (count * sizeof(T) + 255) & ~size_t(255);
        return nullptr;
    }
};

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// ------------------------------------------------------------------------------------------------
// Candidate ordering: better(a, b) = a.v > b.v || (a.v == b.v && a.i < b.i) with valid indices winning
// ties against missing (-1) ones; NaN never compares better (pricing.cu:38-51).
// ------------------------------------------------------------------------------------------------
__host__ __device__ inline bool better(double av, int ai, double bv, int bi) {
    return av > bv || (av == bv && ai >= 0 && (bi < 0 || ai < bi));
}

// Sorted insertion into a k-slot list (descending, tie rule above). k is a compile-time bound.
template <int K>
__device__ inline void put_sorted(double (&v)[K], int (&id)[K], int k, double value, int index) {
    if (!better(value, index, v[k - 1], id[k - 1])) return;
    double cv = value;
    int ci = index;
#pragma unroll
    for (int s = 0; s < K; ++s) {
        if (s < k && better(cv, ci, v[s], id[s])) {
            double tv = v[s];
            int ti = id[s];
            v[s] = cv;
            id[s] = ci;
            cv = tv;
            ci = ti;
        }
    }
}

// ------------------------------------------------------------------------------------------------
// dot64: fp64 dot product of two fp32 rows in the fixed "64-lane" order -- lane l accumulates features
// k = l, l+64, l+128, ... sequentially, then a pairwise tree with halving stride (32, 16, ..., 1).
// fp32*fp32 products are exact in fp64, so FMA contraction cannot change any bit.
// ------------------------------------------------------------------------------------------------

// Wave-cooperative form: every lane of a full 64-lane wave calls it; lane 0 (and, by commutativity,
// every lane holding the same partial pattern) returns the exact tree result.
__device__ inline double wave_tree_sum(double v) {
    // shfl_down with halving stride: lane l (< s) adds lane l+s, matching the oracle's tree.
    v = v + __shfl_down(v, 32, 64);
    v = v + __shfl_down(v, 16, 64);
    v = v + __shfl_down(v, 8, 64);
    v = v + __shfl_down(v, 4, 64);
    v = v + __shfl_down(v, 2, 64);
    v = v + __shfl_down(v, 1, 64);
    return __shfl(v, 0, 64);
}

__device__ inline double wave_dot64(const float* __restrict__ x, const float* __restrict__ y, int d, int lane) {
    double acc = 0.0;
    for (int k = lane; k < d; k += 64) acc = acc + (double)x[k] * (double)y[k];
    return wave_tree_sum(acc);
}

// Single-lane form of the same order: 64 register partials, used where one lane owns one pair.
__device__ inline double lane_dot64(const float* __restrict__ x, const float* __restrict__ y, int d) {
    double acc[64];
#pragma unroll
    for (int l = 0; l < 64; ++l) acc[l] = 0.0;
    int base = 0;
    for (; base + 64 <= d; base += 64) {
#pragma unroll
        for (int l = 0; l < 64; ++l) acc[l] = acc[l] + (double)x[base + l] * (double)y[base + l];
    }
#pragma unroll
    for (int l = 0; l < 64; ++l)
        if (base + l < d) acc[l] = acc[l] + (double)x[base + l] * (double)y[base + l];
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
#pragma unroll
        for (int l = 0; l < s; ++l) acc[l] = acc[l] + acc[l + s];
    }
    return acc[0];
}

// Monotone float <-> uint key (for atomicMax on floats of either sign).
__device__ inline unsigned int float_key(float f) {
    unsigned int u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ inline float key_float(unsigned int k) {
    unsigned int u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}
__device__ inline unsigned long long double_key(double f) {
    unsigned long long u = (unsigned long long)__double_as_longlong(f);
    return (u & 0x8000000000000000ull) ? ~u : (u | 0x8000000000000000ull);
}
__device__ inline double key_double(unsigned long long k) {
    unsigned long long u = (k & 0x8000000000000000ull) ? (k & 0x7fffffffffffffffull) : ~k;
    return __longlong_as_double((long long)u);
}

}  // namespace hm
