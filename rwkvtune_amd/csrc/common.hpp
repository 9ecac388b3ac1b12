// Shared device helpers for the gfx950 WKV7 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define RWKV7_HEAD 64  // head size N; the reference hard-codes it too (model.py:507-508)

typedef uint16_t bf16_t;  // raw bfloat16 bits
typedef _Float16 f16_t;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Scalar conversions (round-to-nearest-even, like at::BFloat16 / at::Half).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(bf16_t x) {
    return __uint_as_float(((uint32_t)x) << 16);
}

__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)0x7fc0;  // NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (bf16_t)(u >> 16);
}

// Streaming access to the recurrent state: each (slot, head) state is read once
// and written once per step, and a step's pool (hundreds of MB) does not fit the
// last-level cache, so loads and stores carry the non-temporal hint.  On MI355X
// this moves the decode step from ~64% to ~74% of HBM peak (measured).
__device__ __forceinline__ f32x4 stream_load(const f32x4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void stream_store(f32x4* p, f32x4 v) { __builtin_nontemporal_store(v, p); }

// Orders LDS writes before LDS reads of other lanes of the same wave (wave-scope
// release / acquire around a wave barrier); enough where a wave only exchanges
// data through its own LDS slice.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename IO> struct io_traits;

template <> struct io_traits<float> {
    static __device__ __forceinline__ float to_f32(float x) { return x; }
    static __device__ __forceinline__ float from_f32(float x) { return x; }
    // 4 consecutive elements starting at p (16-byte aligned)
    static __device__ __forceinline__ f32x4 load4(const float* p) {
        return *reinterpret_cast<const f32x4*>(p);
    }
};

template <> struct io_traits<bf16_t> {
    static __device__ __forceinline__ float to_f32(bf16_t x) { return bf16_to_f32(x); }
    static __device__ __forceinline__ bf16_t from_f32(float x) { return f32_to_bf16(x); }
    static __device__ __forceinline__ f32x4 load4(const bf16_t* p) {
        uint2 u = *reinterpret_cast<const uint2*>(p);
        f32x4 o;
        o.x = __uint_as_float(u.x << 16);
        o.y = __uint_as_float(u.x & 0xffff0000u);
        o.z = __uint_as_float(u.y << 16);
        o.w = __uint_as_float(u.y & 0xffff0000u);
        return o;
    }
};

template <> struct io_traits<f16_t> {
    static __device__ __forceinline__ float to_f32(f16_t x) { return (float)x; }
    static __device__ __forceinline__ f16_t from_f32(float x) { return (f16_t)x; }
    static __device__ __forceinline__ f32x4 load4(const f16_t* p) {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        h4 h = *reinterpret_cast<const h4*>(p);
        f32x4 o;
        o.x = (float)h.x; o.y = (float)h.y; o.z = (float)h.z; o.w = (float)h.w;
        return o;
    }
};

// ---------------------------------------------------------------------------
// DPP lane exchanges inside a 16-lane row.  All of these read from a lane of
// the same row, so every source lane is valid.
//   row_mirror       lane c <- lane 15-c   (= c ^ 15)
//   row_half_mirror  lane c <- lane 7-c within each 8  (= c ^ 7)
//   quad_perm 2301   lane c <- c ^ 2
//   quad_perm 1032   lane c <- c ^ 1
// ---------------------------------------------------------------------------
__device__ __forceinline__ float dpp_xor15(float x) {
    return __builtin_amdgcn_update_dpp(0.0f, x, 0x140, 0xf, 0xf, false);
}
__device__ __forceinline__ float dpp_xor7(float x) {
    return __builtin_amdgcn_update_dpp(0.0f, x, 0x141, 0xf, 0xf, false);
}
__device__ __forceinline__ float dpp_xor2(float x) {
    return __builtin_amdgcn_update_dpp(0.0f, x, 0x4e, 0xf, 0xf, false);
}
__device__ __forceinline__ float dpp_xor1(float x) {
    return __builtin_amdgcn_update_dpp(0.0f, x, 0xb1, 0xf, 0xf, false);
}
// Sum of n float4 planes p[0], p[stride], ..., p[(n-1) stride] in plane order.
// n = 1..8 run unrolled, every load issued before the first add (a loop with a
// run-time count waits for each load before issuing the next).
template <int N>
__device__ __forceinline__ f32x4 sum_planes_n(const float* p, int64_t stride) {
    f32x4 t[N];
#pragma unroll
    for (int q = 0; q < N; ++q) t[q] = *reinterpret_cast<const f32x4*>(p + q * stride);
    f32x4 v = t[0];
#pragma unroll
    for (int q = 1; q < N; ++q) v += t[q];
    return v;
}
__device__ __forceinline__ f32x4 sum_planes(const float* p, int64_t stride, int n) {
    switch (n) {
    case 1: return sum_planes_n<1>(p, stride);
    case 2: return sum_planes_n<2>(p, stride);
    case 3: return sum_planes_n<3>(p, stride);
    case 4: return sum_planes_n<4>(p, stride);
    case 5: return sum_planes_n<5>(p, stride);
    case 6: return sum_planes_n<6>(p, stride);
    case 7: return sum_planes_n<7>(p, stride);
    case 8: return sum_planes_n<8>(p, stride);
    default: {
        f32x4 v = *reinterpret_cast<const f32x4*>(p);
        for (int q = 1; q < n; ++q) v += *reinterpret_cast<const f32x4*>(p + q * stride);
        return v;
    }
    }
}

// Value of lane l ^ 16 / l ^ 32 (l = lane in the wave) by gfx950's
// v_permlane16_swap / v_permlane32_swap with both operands x: the first swaps
// odd 16-lane rows of its first operand with even rows of its second, so the
// partner is the first result in odd rows and the second in even rows; the
// second does the same for the upper and lower 32 lanes.
__device__ __forceinline__ float lane_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// Sum over the 16 lanes of a DPP row, returned in every lane of the row (the
// partners c^1, c^2, c^7, c^15 double the covered lanes at each step).
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_xor1(v);
    v += dpp_xor2(v);
    v += dpp_xor7(v);
    v += dpp_xor15(v);
    return v;
}

__device__ __forceinline__ float fast_dot4(f32x4 a, f32x4 b) {
    return fmaf(a.x, b.x, fmaf(a.y, b.y, fmaf(a.z, b.z, a.w * b.w)));
}
