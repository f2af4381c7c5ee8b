// Shared host/device helpers for the gfx950 H3 hot-path kernels: the
// NineToothedTensor view, host-side validation, and the bf16 rounding
// primitives every kernel uses.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <limits>

#include "../../include/h3mi355x.h"

namespace h3 {

// ------------------------------------------------------------------ host side

constexpr int kInvalid = static_cast<int>(hipErrorInvalidValue);

// Longest query or key sequence the attention launchers accept: the kernels
// count queries and keys in 32-bit integers and round them up to whole tiles
// (at most 256), which must not overflow.
constexpr int64_t kMaxSeqLen = std::numeric_limits<int32_t>::max() - 1024;

// A validated, fixed-rank copy of a NineToothedTensor: the launchers read the
// caller's shape/stride arrays exactly once, here.
template <int N>
struct View {
    char *data = nullptr;
    int64_t shape[N] = {};
    int64_t stride[N] = {};
    int64_t numel() const {
        int64_t n = 1;
        for (int i = 0; i < N; ++i) n *= shape[i];
        return n;
    }
};

// Copies `t` into `v` and checks what every tensor argument must satisfy:
// shape/stride arrays present, sizes representable, data present unless the
// tensor is empty. `elem` is the element size in bytes.
template <int N>
inline bool load_view(const NineToothedTensor &t, int elem, View<N> &v) {
    if (t.shape == nullptr || t.strides == nullptr) return false;
    for (int i = 0; i < N; ++i) {
        if (t.shape[i] > static_cast<uint64_t>(std::numeric_limits<int32_t>::max())) return false;
        v.shape[i] = static_cast<int64_t>(t.shape[i]);
        v.stride[i] = t.strides[i];
    }
    v.data = static_cast<char *>(t.data);
    if (v.numel() != 0 && v.data == nullptr) return false;
    // The furthest element reachable must have a representable byte offset.
    __int128 span = 0;
    for (int i = 0; i < N; ++i) {
        if (v.shape[i] == 0) return true;
        __int128 s = static_cast<__int128>(v.stride[i]) * (v.shape[i] - 1);
        span += s < 0 ? -s : s;
    }
    return span * elem < (static_cast<__int128>(1) << 62);
}

// Reads a NineToothed scalar ({&double, NULL, NULL}).
inline bool load_scalar(const NineToothedTensor &t, double &out) {
    if (t.data == nullptr) return false;
    out = *static_cast<const double *>(t.data);
    return true;
}

template <int N>
inline bool same_shape(const View<N> &a, const View<N> &b) {
    for (int i = 0; i < N; ++i)
        if (a.shape[i] != b.shape[i]) return false;
    return true;
}

// True when the innermost dimension is unit-stride and every row start is
// 16-byte aligned, so the row can be streamed with 16-byte vector accesses.
template <int N>
inline bool rows_vec16(const View<N> &v, int elem) {
    if (v.shape[N - 1] > 1 && v.stride[N - 1] != 1) return false;
    if ((reinterpret_cast<uintptr_t>(v.data) & 15) != 0) return false;
    if ((v.shape[N - 1] * elem) % 16 != 0) return false;
    for (int i = 0; i < N - 1; ++i)
        if (v.shape[i] > 1 && (v.stride[i] * elem) % 16 != 0) return false;
    return true;
}

// True when every element offset of the view is a non-negative value below
// 2^31 and every stride and extent is below 2^24, so that kernels may form the
// offsets in 32-bit arithmetic with 24-bit multiplies (v_mul_u32_u24, full
// rate, exact while both factors are below 2^24 and the product below 2^32).
template <int N>
inline bool offsets_fit_int32(const View<N> &v) {
    int64_t span = 0;
    for (int i = 0; i < N; ++i) {
        if (v.shape[i] == 0) return true;
        if (v.stride[i] < 0 || v.stride[i] >= (int64_t{1} << 24) || v.shape[i] >= (int64_t{1} << 24)) return false;
        span += v.stride[i] * (v.shape[i] - 1);
    }
    return span < (int64_t{1} << 31);
}

// Division by a divisor fixed at launch, for dividends n < 2^31: q = floor(n / d)
// = (n * m) >> shift with m = ceil(2^(31 + s) / d), s = ceil(log2 d). The error
// of m is below 1, so n * m / 2^(31 + s) exceeds n / d by less than
// n / 2^(31 + s) < 2^-s <= 1 / d, which never reaches the next integer.
// The device forms it as mulhi(2n, m) >> s: mulhi(2n, m) = floor(n m / 2^31)
// (2n < 2^32), and flooring twice is flooring once by the product.
struct FastDiv {
    uint32_t d, m, shift;
};

inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t s = 0;
    while ((uint64_t{1} << s) < d) ++s;
    const uint64_t m = ((uint64_t{1} << (31 + s)) + d - 1) / d;
    return {d, static_cast<uint32_t>(m), 31 + s};
}

__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv &f) {
    return __umulhi(n << 1, f.m) >> (f.shift - 31);
}

// True when a byte view has unit inner stride and every row start (and the
// base) is 8-byte aligned, so each 8 consecutive bytes can go as one store.
template <int N>
inline bool rows_vec8_bytes(const View<N> &v) {
    if (v.shape[N - 1] > 1 && v.stride[N - 1] != 1) return false;
    if ((reinterpret_cast<uintptr_t>(v.data) & 7) != 0 || v.shape[N - 1] % 8 != 0) return false;
    for (int i = 0; i < N - 1; ++i)
        if (v.shape[i] > 1 && v.stride[i] % 8 != 0) return false;
    return true;
}

inline hipStream_t as_stream(NineToothedStream s) { return static_cast<hipStream_t>(s); }

// Launch epilogue shared by all launchers: the launch status of the kernel.
inline int launch_status() { return static_cast<int>(hipGetLastError()); }

// ---------------------------------------------------------------- device side

typedef uint16_t bf16_t;  // raw bf16 bits
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf2f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
// Low / high bf16 of a packed dword, widened to fp32 (exact).
__device__ __forceinline__ float lo2f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi2f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round two fp32 values to bf16 (round-to-nearest-even, v_cvt_pk_bf16_f32) and
// pack them, `a` in the low half.
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    f32x2_t f = {a, b};
    bf16x2_t h = __builtin_convertvector(f, bf16x2_t);
    return __builtin_bit_cast(uint32_t, h);
}

// fp32 -> bf16 -> fp32, i.e. the value `.to(bfloat16)` leaves behind, in one
// instruction: the packed conversion of (0, a) puts bf16(a) in the high half
// over a zero low half, which read as fp32 is exactly bf16(a).
__device__ __forceinline__ float rbf(float a) { return __uint_as_float(pack2(0.0f, a)); }

// The same for a pair (two conversions: one conversion of the pair would need
// a shift and a mask to widen its halves, three instructions for two values).
__device__ __forceinline__ void rbf2(float &a, float &b) {
    a = rbf(a);
    b = rbf(b);
}

// 1/sqrt(v) with two IEEE roundings (correctly rounded sqrt, then correctly
// rounded division): the value torch computes for rsqrt on the CPU.
__device__ __forceinline__ float rsqrt_ieee(float v) { return __fdiv_rn(1.0f, __fsqrt_rn(v)); }

struct U4 {
    uint32_t x, y, z, w;
};
__device__ __forceinline__ U4 ld16(const void *p) {
    uint4 v = *static_cast<const uint4 *>(p);
    return {v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ void st16(void *p, const U4 &v) {
    *static_cast<uint4 *>(p) = make_uint4(v.x, v.y, v.z, v.w);
}
// Non-temporal 16-byte accesses for data touched once (streamed rows): the
// lines are not kept in the caches, leaving them to the reused operands.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ U4 ld16_stream(const void *p) {
    const u32x4_t v = __builtin_nontemporal_load(static_cast<const u32x4_t *>(p));
    return {v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ void st16_stream(void *p, const U4 &v) {
    const u32x4_t w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, static_cast<u32x4_t *>(p));
}
// Hides a packed group from the optimizer (an empty asm that may "change" its
// registers), so values widened from it earlier are not kept alive in place of
// widening it again: four packed registers instead of eight floats.
__device__ __forceinline__ void keep_packed(U4 &v) {
    asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}
__device__ __forceinline__ void u4_to_f8(const U4 &v, float f[8]) {
    f[0] = lo2f(v.x); f[1] = hi2f(v.x); f[2] = lo2f(v.y); f[3] = hi2f(v.y);
    f[4] = lo2f(v.z); f[5] = hi2f(v.z); f[6] = lo2f(v.w); f[7] = hi2f(v.w);
}
__device__ __forceinline__ U4 f8_to_u4(const float f[8]) {
    return {pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7])};
}

// sat() of the e4m3 codes: clamps to [-448, 448] and keeps NaN, so a NaN value
// gets the NaN code (as a NaN does in the bf16 ops). fminf / fmaxf would
// return the bound for a NaN, a finite code that hides it.
__device__ __forceinline__ float sat_e4m3(float v) {
    constexpr float kMax = 448.0f;
    return v > kMax ? kMax : (v < -kMax ? -kMax : v);
}

// The e4m3 code scale of a head whose values are bounded by `bound` (its amax,
// or a proven bound): codes = e4m3(sat((x * pre) * inv)).
//   - 448 / bound finite: pre = 1, inv = fp32(448 / bound), so the code is the
//     one rounding of x * (448 / bound).
//   - 448 / bound overflows (0 < bound < 448 / FLT_MAX ~ 1.3e-36: bf16
//     subnormals and the smallest normals): pre = 2^64, inv = fp32(448 /
//     (bound * 2^64)). Both scalings by 2^64 are exact (|x| <= bound, and
//     bound * 2^64 >= 2^-85 stays normal), so x * 448 / bound is still formed
//     with one division and one product, and inv is finite.
//   - bound = 0 (an all-zero head): pre = 1, inv = 0, every code 0.
__device__ __forceinline__ void e4m3_code_scale(float bound, float &pre, float &inv) {
    constexpr float kMax = 448.0f, kTwo64 = 18446744073709551616.0f;
    pre = 1.0f;
    inv = 0.0f;
    if (bound > 0.0f) {
        inv = kMax / bound;
        if (inv > 3.40282347e38f) {  // +inf
            pre = kTwo64;
            inv = kMax / (bound * kTwo64);
        }
    }
}

}  // namespace h3
