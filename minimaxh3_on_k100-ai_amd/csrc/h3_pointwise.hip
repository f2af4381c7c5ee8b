// gfx950 kernels for the H3 DiT pointwise ops around attention: SwiGLU,
// RMSNorm (+AdaLN), gated residual (+RMSNorm+AdaLN), RoPE, q/k RMSNorm+RoPE and
// the RoPE table. Each op reproduces the reference's per-step bf16 rounding
// (tools/h3_pointwise.py) and is a single pass over HBM.
//
// Every kernel has two load/store paths sharing one arithmetic body: a 16-byte
// vector path (unit inner stride, 16-byte aligned rows) and a generic path that
// reads the same 8-element groups element by element with arbitrary strides.
// The fp32 sum of squares in the RMS family is accumulated in one fixed order
// that depends only on the row width W (not on the path):
//   - W8 = ceil(W / 8) groups of 8 consecutive elements;
//   - W8 <= 64: lane g owns group g (L = next power of two >= W8 lanes per row);
//     W8 > 64: 256 threads, thread t owns groups t, t+256, t+512, ...;
//   - each thread adds its elements left to right (group by group, element by
//     element) into one fp32 partial, starting from +0;
//   - partials are folded pairwise within each 64-lane wave (lane i += lane
//     i^off for off = L/2 ... 1), then across the 4 waves as (w0+w2)+(w1+w3).
#include "h3_common.hpp"

namespace h3 {
namespace {

constexpr int kThreads = 256;

// A row-major 3-D view [B, S, W] reduced to what kernels need.
struct Rows {
    char *p;
    int64_t sb, ss, sw;  // element strides
};

template <int N>
Rows rows_of(const View<N> &v) {
    static_assert(N == 3, "3-D views only");
    return {v.data, v.stride[0], v.stride[1], v.stride[2]};
}

__device__ __forceinline__ const bf16_t *row_ptr(const Rows &t, int64_t b, int64_t s) {
    return reinterpret_cast<const bf16_t *>(t.p) + b * t.sb + s * t.ss;
}
__device__ __forceinline__ bf16_t *row_ptr_w(const Rows &t, int64_t b, int64_t s) {
    return reinterpret_cast<bf16_t *>(t.p) + b * t.sb + s * t.ss;
}

// Loads the 8-element group starting at column c0 of a row: 16-byte vector on
// the VEC path, element-wise (zero past W) otherwise.
template <bool VEC>
__device__ __forceinline__ void load8(const bf16_t *row, int64_t sw, int c0, int W, float f[8]) {
    if constexpr (VEC) {
        u4_to_f8(ld16(row + c0), f);
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = (c0 + e < W) ? bf2f(row[(c0 + e) * sw]) : 0.0f;
    }
}

template <bool VEC>
__device__ __forceinline__ void store8(bf16_t *row, int64_t sw, int c0, int W, const float f[8]) {
    if constexpr (VEC) {
        st16(row + c0, f8_to_u4(f));
    } else {
        const U4 v = f8_to_u4(f);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (c0 + e < W) row[(c0 + e) * sw] = static_cast<bf16_t>(w[e >> 1] >> (16 * (e & 1)));
    }
}

// Pairwise fold of one fp32 value over groups of L lanes (L a power of two <= 64).
template <int L>
__device__ __forceinline__ float fold_lanes(float v) {
#pragma unroll
    for (int off = L / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, L);
    return v;
}

// ============================================================ RMS family

enum RmsMode { kRms = 0, kRmsModulate = 1, kGatedRmsModulate = 2 };

struct RmsArgs {
    Rows x, gate, y, scale, shift, residual, out;
    const bf16_t *w;
    int64_t w_stride;
    int64_t rows, S;
    int W;
    float eps_bf;  // eps already rounded fp64 -> fp32 -> bf16
};

// The per-row epilogue shared by every path: value -> normalized -> weighted
// (-> modulated). `r` is the bf16 reciprocal, widened.
template <int MODE>
__device__ __forceinline__ void rms_epilogue(float f[8], float r, const float w[8], const float sc[8],
                                             const float sh[8]) {
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        float n0 = f[e] * r, n1 = f[e + 1] * r;
        rbf2(n0, n1);  // normalized = bf16(value * reciprocal)
        float a0 = n0 * w[e], a1 = n1 * w[e + 1];
        if constexpr (MODE == kRms) {
            f[e] = a0;  // rounded by the store
            f[e + 1] = a1;
        } else {
            rbf2(a0, a1);  // weighted = bf16(normalized * weight)
            float k0 = 1.0f + sc[e], k1 = 1.0f + sc[e + 1];
            rbf2(k0, k1);  // factor = bf16(1 + scale)
            float p0 = a0 * k0, p1 = a1 * k1;
            rbf2(p0, p1);  // product = bf16(weighted * factor)
            f[e] = p0 + sh[e];  // out = bf16(product + shift), rounded by the store
            f[e + 1] = p1 + sh[e + 1];
        }
    }
}

// One row per group of L lanes (L <= 64, one 8-element group per lane), or
// one row per 256-thread block (L == 256, VPT groups per thread).
template <int L, int VPT, bool VEC, int MODE>
__global__ __launch_bounds__(kThreads) void rms_rows_kernel(RmsArgs a) {
    constexpr int kRowsPerBlock = L >= kThreads ? 1 : kThreads / L;
    const int lane = threadIdx.x % (L >= kThreads ? kThreads : L);
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / (L >= kThreads ? kThreads : L);
    const bool row_ok = row < a.rows;
    const int64_t b = row_ok ? row / a.S : 0;
    const int64_t s = row_ok ? row % a.S : 0;
    const int W = a.W;
    const int W8 = (W + 7) / 8;

    float v[VPT][8];
    float partial = 0.0f;
    const bf16_t *xr = row_ptr(a.x, b, s);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int g = lane + j * (L >= kThreads ? kThreads : L);
        const bool ok = row_ok && g < W8;
        if (ok) {
            load8<VEC>(xr, a.x.sw, g * 8, W, v[j]);
            if constexpr (MODE == kGatedRmsModulate) {
                float gt[8], yy[8];
                load8<VEC>(row_ptr(a.gate, b, s), a.gate.sw, g * 8, W, gt);
                load8<VEC>(row_ptr(a.y, b, s), a.y.sw, g * 8, W, yy);
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    float p0 = gt[e] * yy[e], p1 = gt[e + 1] * yy[e + 1];
                    rbf2(p0, p1);  // product = bf16(gate * y)
                    float h0 = v[j][e] + p0, h1 = v[j][e + 1] + p1;
                    rbf2(h0, h1);  // residual = bf16(x + product)
                    v[j][e] = h0;
                    v[j][e + 1] = h1;
                }
                if constexpr (!VEC) {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (g * 8 + e >= W) v[j][e] = 0.0f;
                }
                store8<VEC>(row_ptr_w(a.residual, b, s), a.residual.sw, g * 8, W, v[j]);
            }
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                float q0 = v[j][e] * v[j][e], q1 = v[j][e + 1] * v[j][e + 1];
                rbf2(q0, q1);  // squared = bf16(value * value)
                partial += q0;
                partial += q1;
            }
        }
    }

    // Fold the partials in the fixed order.
    float total;
    if constexpr (L >= kThreads) {
        __shared__ float red[kThreads / 64];
        const float wsum = fold_lanes<64>(partial);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = wsum;
        __syncthreads();
        total = (red[0] + red[2]) + (red[1] + red[3]);
    } else {
        total = fold_lanes<L>(partial);
    }
    if (!row_ok) return;

    const float mean = rbf(__fdiv_rn(total, static_cast<float>(W)));  // bf16(sum / W)
    const float var = rbf(mean + a.eps_bf);                           // bf16(mean + eps)
    const float r = rbf(rsqrt_ieee(var));                             // bf16(rsqrt(var))

    bf16_t *outr = row_ptr_w(a.out, b, s);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int g = lane + j * (L >= kThreads ? kThreads : L);
        if (g >= W8) continue;
        float w[8], sc[8], sh[8];
        if constexpr (VEC) {
            u4_to_f8(ld16(a.w + g * 8), w);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) w[e] = (g * 8 + e < W) ? bf2f(a.w[(g * 8 + e) * a.w_stride]) : 0.0f;
        }
        if constexpr (MODE != kRms) {
            load8<VEC>(row_ptr(a.scale, b, s), a.scale.sw, g * 8, W, sc);
            load8<VEC>(row_ptr(a.shift, b, s), a.shift.sw, g * 8, W, sh);
        }
        rms_epilogue<MODE>(v[j], r, w, sc, sh);
        store8<VEC>(outr, a.out.sw, g * 8, W, v[j]);
    }
}

template <int MODE, bool VEC>
int launch_rms_vec(const RmsArgs &a, hipStream_t stream) {
    const int W8 = (a.W + 7) / 8;
    auto grid_small = [&](int L) { return static_cast<unsigned>((a.rows + (kThreads / L) - 1) / (kThreads / L)); };
    if (W8 <= 64) {
        int L = 1;
        while (L < W8) L <<= 1;
        switch (L) {
#define H3_RMS_SMALL(LL)                                                                          \
    case LL:                                                                                     \
        rms_rows_kernel<LL, 1, VEC, MODE><<<grid_small(LL), kThreads, 0, stream>>>(a);            \
        break;
            H3_RMS_SMALL(1) H3_RMS_SMALL(2) H3_RMS_SMALL(4) H3_RMS_SMALL(8) H3_RMS_SMALL(16)
            H3_RMS_SMALL(32) H3_RMS_SMALL(64)
#undef H3_RMS_SMALL
        }
        return launch_status();
    }
    const int vpt = (W8 + kThreads - 1) / kThreads;
    const unsigned grid = static_cast<unsigned>(a.rows);
#define H3_RMS_BIG(V)                                                                     \
    if (vpt <= V) {                                                                      \
        rms_rows_kernel<kThreads, V, VEC, MODE><<<grid, kThreads, 0, stream>>>(a);        \
        return launch_status();                                                          \
    }
    H3_RMS_BIG(1) H3_RMS_BIG(2) H3_RMS_BIG(3) H3_RMS_BIG(4) H3_RMS_BIG(6) H3_RMS_BIG(8)
    H3_RMS_BIG(12) H3_RMS_BIG(16)
#undef H3_RMS_BIG
    return kInvalid;  // W > 32768: outside the supported widths
}

// Host-side fp32 -> bf16 round-to-nearest-even, NaN kept quiet.
float host_round_bf16(double eps) {
    float f = static_cast<float>(eps);
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        u = (u | 0x00400000u) & 0xffff0000u;
    } else {
        u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
    }
    __builtin_memcpy(&f, &u, 4);
    return f;
}

int rms_family(int mode, hipStream_t stream, const NineToothedTensor &x_t, const NineToothedTensor *gate_t,
               const NineToothedTensor *y_t, const NineToothedTensor &w_t, const NineToothedTensor &eps_t,
               const NineToothedTensor *scale_t, const NineToothedTensor *shift_t,
               const NineToothedTensor *residual_t, const NineToothedTensor &out_t, int required_width) {
    View<3> x, out, gate, y, scale, shift, residual;
    View<1> w;
    double eps;
    if (!load_view(x_t, 2, x) || !load_view(out_t, 2, out) || !load_view(w_t, 2, w) || !load_scalar(eps_t, eps))
        return kInvalid;
    if (!same_shape(x, out) || w.shape[0] != x.shape[2]) return kInvalid;
    if (required_width > 0 && x.shape[2] != required_width) return kInvalid;
    if (x.shape[2] > 32768) return kInvalid;
    bool vec = rows_vec16(x, 2) && rows_vec16(out, 2) && rows_vec16(w, 2);
    if (mode == kGatedRmsModulate) {
        if (!load_view(*gate_t, 2, gate) || !load_view(*y_t, 2, y) || !load_view(*residual_t, 2, residual))
            return kInvalid;
        if (!same_shape(x, gate) || !same_shape(x, y) || !same_shape(x, residual)) return kInvalid;
        vec = vec && rows_vec16(gate, 2) && rows_vec16(y, 2) && rows_vec16(residual, 2);
    }
    if (mode != kRms) {
        if (!load_view(*scale_t, 2, scale) || !load_view(*shift_t, 2, shift)) return kInvalid;
        if (!same_shape(x, scale) || !same_shape(x, shift)) return kInvalid;
        vec = vec && rows_vec16(scale, 2) && rows_vec16(shift, 2);
    }
    RmsArgs a{};
    a.x = rows_of(x);
    a.out = rows_of(out);
    a.gate = mode == kGatedRmsModulate ? rows_of(gate) : a.x;
    a.y = mode == kGatedRmsModulate ? rows_of(y) : a.x;
    a.residual = mode == kGatedRmsModulate ? rows_of(residual) : a.out;
    a.scale = mode != kRms ? rows_of(scale) : a.x;
    a.shift = mode != kRms ? rows_of(shift) : a.x;
    a.w = reinterpret_cast<const bf16_t *>(w.data);
    a.w_stride = w.stride[0];
    a.rows = x.shape[0] * x.shape[1];
    a.S = x.shape[1];
    a.W = static_cast<int>(x.shape[2]);
    a.eps_bf = host_round_bf16(eps);
    if (a.rows == 0 || a.W == 0) return 0;
    if (a.rows > static_cast<int64_t>(std::numeric_limits<int32_t>::max())) return kInvalid;
    switch (mode) {
        case kRms: return vec ? launch_rms_vec<kRms, true>(a, stream) : launch_rms_vec<kRms, false>(a, stream);
        case kRmsModulate:
            return vec ? launch_rms_vec<kRmsModulate, true>(a, stream) : launch_rms_vec<kRmsModulate, false>(a, stream);
        default:
            return vec ? launch_rms_vec<kGatedRmsModulate, true>(a, stream)
                       : launch_rms_vec<kGatedRmsModulate, false>(a, stream);
    }
}

// ============================================================ elementwise

// Column-chunked row streaming: block (row, chunk) handles 8-element groups
// chunk*256*U + t + 256*u. Loads are issued before any store.
constexpr int kEwUnroll = 4;

struct EwArgs {
    Rows a, b, c, out;  // op inputs (c unused by SwiGLU) and output
    int64_t rows, S;
    int W, chunks;
};

// out = bf16(x + bf16(gate * y)) (tools/h3_pointwise.py:121-124)
struct GatedResidualOp {
    static constexpr int kInputs = 3;
    __device__ static void apply(const float x[8], const float g[8], const float y[8], float o[8]) {
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            float p0 = g[e] * y[e], p1 = g[e + 1] * y[e + 1];
            rbf2(p0, p1);
            o[e] = x[e] + p0;
            o[e + 1] = x[e + 1] + p1;
        }
    }
};

// out = bf16(up * bf16(g / (1 + exp(-g)))) (tools/h3_pointwise.py:18-22)
struct SwigluOp {
    static constexpr int kInputs = 2;
    __device__ static void apply(const float up[8], const float g[8], const float *, float o[8]) {
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            float a0 = __fdiv_rn(g[e], 1.0f + expf(-g[e]));
            float a1 = __fdiv_rn(g[e + 1], 1.0f + expf(-g[e + 1]));
            rbf2(a0, a1);
            o[e] = up[e] * a0;
            o[e + 1] = up[e + 1] * a1;
        }
    }
};

template <class Op, bool VEC>
__global__ __launch_bounds__(kThreads) void ew_kernel(EwArgs a) {
    const int64_t row = blockIdx.x / a.chunks;
    const int chunk = blockIdx.x % a.chunks;
    const int64_t b = row / a.S, s = row % a.S;
    const int W8 = (a.W + 7) / 8;
    const bf16_t *pa = row_ptr(a.a, b, s);
    const bf16_t *pb = row_ptr(a.b, b, s);
    const bf16_t *pc = Op::kInputs > 2 ? row_ptr(a.c, b, s) : nullptr;
    bf16_t *po = row_ptr_w(a.out, b, s);
    float va[kEwUnroll][8], vb[kEwUnroll][8], vc[kEwUnroll][8];
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) {
        const int g = chunk * kThreads * kEwUnroll + u * kThreads + threadIdx.x;
        if (g < W8) {
            load8<VEC>(pa, a.a.sw, g * 8, a.W, va[u]);
            load8<VEC>(pb, a.b.sw, g * 8, a.W, vb[u]);
            if constexpr (Op::kInputs > 2) load8<VEC>(pc, a.c.sw, g * 8, a.W, vc[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) {
        const int g = chunk * kThreads * kEwUnroll + u * kThreads + threadIdx.x;
        if (g < W8) {
            float o[8];
            Op::apply(va[u], vb[u], vc[u], o);
            store8<VEC>(po, a.out.sw, g * 8, a.W, o);
        }
    }
}

template <class Op>
int launch_ew(hipStream_t stream, const View<3> *in, const View<3> &out) {
    for (int i = 0; i < Op::kInputs; ++i)
        if (!same_shape(in[i], out)) return kInvalid;
    bool vec = rows_vec16(out, 2);
    for (int i = 0; i < Op::kInputs; ++i) vec = vec && rows_vec16(in[i], 2);
    EwArgs a{};
    a.a = rows_of(in[0]);
    a.b = rows_of(in[1]);
    a.c = Op::kInputs > 2 ? rows_of(in[2]) : a.a;
    a.out = rows_of(out);
    a.rows = out.shape[0] * out.shape[1];
    a.S = out.shape[1];
    a.W = static_cast<int>(out.shape[2]);
    if (a.rows == 0 || a.W == 0) return 0;
    const int W8 = (a.W + 7) / 8;
    a.chunks = (W8 + kThreads * kEwUnroll - 1) / (kThreads * kEwUnroll);
    const int64_t grid = a.rows * a.chunks;
    if (grid > static_cast<int64_t>(std::numeric_limits<int32_t>::max())) return kInvalid;
    if (vec)
        ew_kernel<Op, true><<<static_cast<unsigned>(grid), kThreads, 0, stream>>>(a);
    else
        ew_kernel<Op, false><<<static_cast<unsigned>(grid), kThreads, 0, stream>>>(a);
    return launch_status();
}

// ============================================================ RoPE family

// 128-channel head rows, 16 lanes per row, lane j owns channels 8j..8j+7.
struct HeadRows {
    char *p;
    int64_t s0, s1, s2, s3;  // element strides of [T, P, Hs, 128] (or [S, H, 1, 128])
};

struct RopeArgs {
    HeadRows x, out;
    const bf16_t *cos, *sin;
    int64_t cs0, cs1, ss0, ss1;  // element strides of the [T, n] cos and sin tables
    int64_t rows, P, Hs;
    const bf16_t *w;  // [128] RMS weight (norm kernels only)
    int64_t w_stride;
    float eps_bf;
};

__device__ __forceinline__ int64_t head_offset(const HeadRows &h, int64_t t, int64_t p, int64_t hh) {
    return t * h.s0 + p * h.s1 + hh * h.s2;
}

template <bool VEC>
__device__ __forceinline__ void load_head8(const HeadRows &h, int64_t off, int lane, float f[8]) {
    const bf16_t *row = reinterpret_cast<const bf16_t *>(h.p) + off;
    if constexpr (VEC) {
        u4_to_f8(ld16(row + lane * 8), f);
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = bf2f(row[(lane * 8 + e) * h.s3]);
    }
}

template <bool VEC>
__device__ __forceinline__ void store_head8(const HeadRows &h, int64_t off, int lane, const float f[8]) {
    bf16_t *row = reinterpret_cast<bf16_t *>(h.p) + off;
    if constexpr (VEC) {
        st16(row + lane * 8, f8_to_u4(f));
    } else {
        const U4 v = f8_to_u4(f);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) row[(lane * 8 + e) * h.s3] = static_cast<bf16_t>(w[e >> 1] >> (16 * (e & 1)));
    }
}

// RMSNorm over the 128 channels held by a 16-lane row group (the same fixed
// order as the rms family at W = 128), then weight: returns bf16 values in f.
template <bool VEC>
__device__ __forceinline__ void head_rms(float f[8], int lane, const RopeArgs &a) {
    float partial = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        float q0 = f[e] * f[e], q1 = f[e + 1] * f[e + 1];
        rbf2(q0, q1);
        partial += q0;
        partial += q1;
    }
    const float total = fold_lanes<16>(partial);
    const float mean = rbf(__fdiv_rn(total, 128.0f));
    const float var = rbf(mean + a.eps_bf);
    const float r = rbf(rsqrt_ieee(var));
    float w[8];
    if constexpr (VEC) {
        u4_to_f8(ld16(a.w + lane * 8), w);
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) w[e] = bf2f(a.w[(lane * 8 + e) * a.w_stride]);
    }
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        float n0 = f[e] * r, n1 = f[e + 1] * r;
        rbf2(n0, n1);  // bf16(value * reciprocal)
        n0 *= w[e];
        n1 *= w[e + 1];
        rbf2(n0, n1);  // bf16(normalized * weight)
        f[e] = n0;
        f[e + 1] = n1;
    }
}

// Rotate-half RoPE on channels 0..95 (pairs i, i+48), 96..127 pass through,
// cos/sin [T, 48] (tools/h3_pointwise.py:199-214). Lanes 0-5 hold the first
// halves, lanes 6-11 the second halves, lanes 12-15 the pass-through.
template <bool VEC>
__device__ __forceinline__ void rope_rotate_half(float f[8], int lane, int64_t t, const RopeArgs &a) {
    float partner[8];
    const int src = lane < 6 ? lane + 6 : (lane < 12 ? lane - 6 : lane);
#pragma unroll
    for (int e = 0; e < 8; ++e) partner[e] = __shfl(f[e], src, 16);
    if (lane >= 12) return;
    const int c0 = (lane < 6 ? lane : lane - 6) * 8;
    float c[8], s[8];
    const bf16_t *cr = a.cos + t * a.cs0;
    const bf16_t *sr = a.sin + t * a.ss0;
    if constexpr (VEC) {
        u4_to_f8(ld16(cr + c0), c);
        u4_to_f8(ld16(sr + c0), s);
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            c[e] = bf2f(cr[(c0 + e) * a.cs1]);
            s[e] = bf2f(sr[(c0 + e) * a.ss1]);
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float av = lane < 6 ? f[e] : partner[e];  // first half a
        const float bv = lane < 6 ? partner[e] : f[e];  // second half b
        float t0, t1;
        if (lane < 6) {
            t0 = av * c[e];     // ac = bf16(a c)
            t1 = -bv * s[e];    // bs = bf16(-b s)
        } else {
            t0 = bv * c[e];     // bc = bf16(b c)
            t1 = av * s[e];     // as = bf16(a s)
        }
        rbf2(t0, t1);
        f[e] = t0 + t1;  // y = bf16(. + .), rounded by the store
    }
}

// Interleaved-pair RoPE on all 128 channels: pair i = (2i, 2i+1), cos/sin
// [T, 64]; lane j owns pairs 4j..4j+3.
template <bool VEC>
__device__ __forceinline__ void rope_interleaved(float f[8], int lane, int64_t t, const RopeArgs &a) {
    float c[4], s[4];
    const bf16_t *cr = a.cos + t * a.cs0 + lane * 4 * a.cs1;
    const bf16_t *sr = a.sin + t * a.ss0 + lane * 4 * a.ss1;
    if constexpr (VEC) {
        const uint2 cv = *reinterpret_cast<const uint2 *>(cr);
        const uint2 sv = *reinterpret_cast<const uint2 *>(sr);
        c[0] = lo2f(cv.x); c[1] = hi2f(cv.x); c[2] = lo2f(cv.y); c[3] = hi2f(cv.y);
        s[0] = lo2f(sv.x); s[1] = hi2f(sv.x); s[2] = lo2f(sv.y); s[3] = hi2f(sv.y);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[i] = bf2f(cr[i * a.cs1]);
            s[i] = bf2f(sr[i * a.ss1]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float av = f[2 * i], bv = f[2 * i + 1];
        float ac = av * c[i], bs = -bv * s[i];
        rbf2(ac, bs);
        float bc = bv * c[i], as = av * s[i];
        rbf2(bc, as);
        f[2 * i] = ac + bs;
        f[2 * i + 1] = bc + as;
    }
}

enum RopeMode { kRopeOnly = 0, kNormRope = 1, kNormRopeInterleaved = 2 };

template <bool VEC, int MODE>
__global__ __launch_bounds__(kThreads) void head_rows_kernel(RopeArgs a) {
    const int lane = threadIdx.x & 15;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / 16) + (threadIdx.x >> 4);
    const bool ok = row < a.rows;
    const int64_t r = ok ? row : 0;
    const int64_t t = r / (a.P * a.Hs);
    const int64_t rem = r % (a.P * a.Hs);
    const int64_t p = rem / a.Hs, hh = rem % a.Hs;
    float f[8];
    load_head8<VEC>(a.x, head_offset(a.x, t, p, hh), lane, f);
    if constexpr (MODE != kRopeOnly) head_rms<VEC>(f, lane, a);
    if constexpr (MODE == kNormRopeInterleaved) {
        rope_interleaved<VEC>(f, lane, t, a);
    } else {
        rope_rotate_half<VEC>(f, lane, t, a);
    }
    if (ok) store_head8<VEC>(a.out, head_offset(a.out, t, p, hh), lane, f);
}

template <int MODE>
int launch_head_rows(hipStream_t stream, const View<4> &x, const View<4> &out, const View<2> &cos,
                     const View<2> &sin, const View<1> *w, double eps) {
    const int64_t table_width = MODE == kNormRopeInterleaved ? 64 : 48;
    if (!same_shape(x, out) || x.shape[3] != 128) return kInvalid;
    if (cos.shape[0] != x.shape[0] || cos.shape[1] != table_width || !same_shape(cos, sin)) return kInvalid;
    if (w != nullptr && w->shape[0] != 128) return kInvalid;
    bool vec = rows_vec16(x, 2) && rows_vec16(out, 2) && rows_vec16(cos, 2) && rows_vec16(sin, 2);
    if (w != nullptr) vec = vec && rows_vec16(*w, 2);
    RopeArgs a{};
    a.x = {x.data, x.stride[0], x.stride[1], x.stride[2], x.stride[3]};
    a.out = {out.data, out.stride[0], out.stride[1], out.stride[2], out.stride[3]};
    a.cos = reinterpret_cast<const bf16_t *>(cos.data);
    a.sin = reinterpret_cast<const bf16_t *>(sin.data);
    a.cs0 = cos.stride[0];
    a.cs1 = cos.stride[1];
    a.ss0 = sin.stride[0];
    a.ss1 = sin.stride[1];
    a.P = x.shape[1];
    a.Hs = x.shape[2];
    a.rows = x.shape[0] * x.shape[1] * x.shape[2];
    if (w != nullptr) {
        a.w = reinterpret_cast<const bf16_t *>(w->data);
        a.w_stride = w->stride[0];
    }
    a.eps_bf = host_round_bf16(eps);
    if (a.rows == 0) return 0;
    const int64_t grid = (a.rows + kThreads / 16 - 1) / (kThreads / 16);
    if (grid > static_cast<int64_t>(std::numeric_limits<int32_t>::max())) return kInvalid;
    if (vec)
        head_rows_kernel<true, MODE><<<static_cast<unsigned>(grid), kThreads, 0, stream>>>(a);
    else
        head_rows_kernel<false, MODE><<<static_cast<unsigned>(grid), kThreads, 0, stream>>>(a);
    return launch_status();
}

// ============================================================ RoPE table

// cos/sin[t, a*16 + k] = bf16(cos/sin(fp32(position[t, a]) * (1 / power[k])))
// (tools/h3_pointwise.py:416-427). One thread per (t, a, k).
__global__ __launch_bounds__(kThreads) void rope_cache_kernel(const double *pos, int64_t ps0, int64_t ps1,
                                                              const float *power, int64_t pw_s, bf16_t *cos,
                                                              bf16_t *sin, int64_t cs0, int64_t cs1, int64_t ss0,
                                                              int64_t ss1, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    const int64_t t = i / 48;
    const int c = static_cast<int>(i % 48);
    const int axis = c / 16, k = c % 16;
    const float inverse = __fdiv_rn(1.0f, power[k * pw_s]);
    const float x = static_cast<float>(pos[t * ps0 + axis * ps1]);
    const float angle = x * inverse;
    cos[t * cs0 + c * cs1] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(cosf(angle)));
    sin[t * ss0 + c * ss1] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(sinf(angle)));
}

}  // namespace
}  // namespace h3

using namespace h3;

extern "C" {

NineToothedResult launch_h3_swiglu_exact(NineToothedStream stream, NineToothedTensor up, NineToothedTensor gate,
                                         NineToothedTensor out) {
    View<3> in[2], o;
    if (!load_view(up, 2, in[0]) || !load_view(gate, 2, in[1]) || !load_view(out, 2, o)) return kInvalid;
    return launch_ew<SwigluOp>(as_stream(stream), in, o);
}

NineToothedResult launch_h3_gated_residual_exact(NineToothedStream stream, NineToothedTensor x,
                                                 NineToothedTensor gate, NineToothedTensor y,
                                                 NineToothedTensor out) {
    View<3> in[3], o;
    if (!load_view(x, 2, in[0]) || !load_view(gate, 2, in[1]) || !load_view(y, 2, in[2]) || !load_view(out, 2, o))
        return kInvalid;
    return launch_ew<GatedResidualOp>(as_stream(stream), in, o);
}

NineToothedResult launch_h3_rms_exact(NineToothedStream stream, NineToothedTensor x, NineToothedTensor weight,
                                      NineToothedTensor eps, NineToothedTensor out) {
    return rms_family(kRms, as_stream(stream), x, nullptr, nullptr, weight, eps, nullptr, nullptr, nullptr, out, 0);
}

NineToothedResult launch_h3_rms_exact_128(NineToothedStream stream, NineToothedTensor x, NineToothedTensor weight,
                                          NineToothedTensor eps, NineToothedTensor out) {
    return rms_family(kRms, as_stream(stream), x, nullptr, nullptr, weight, eps, nullptr, nullptr, nullptr, out, 128);
}

NineToothedResult launch_h3_rms_exact_5376(NineToothedStream stream, NineToothedTensor x, NineToothedTensor weight,
                                           NineToothedTensor eps, NineToothedTensor out) {
    return rms_family(kRms, as_stream(stream), x, nullptr, nullptr, weight, eps, nullptr, nullptr, nullptr, out,
                      5376);
}

NineToothedResult launch_h3_rms_modulate_exact(NineToothedStream stream, NineToothedTensor x,
                                               NineToothedTensor weight, NineToothedTensor eps,
                                               NineToothedTensor scale, NineToothedTensor shift,
                                               NineToothedTensor out) {
    return rms_family(kRmsModulate, as_stream(stream), x, nullptr, nullptr, weight, eps, &scale, &shift, nullptr,
                      out, 0);
}

NineToothedResult launch_h3_gated_residual_rms_modulate_exact(
    NineToothedStream stream, NineToothedTensor x, NineToothedTensor gate, NineToothedTensor y,
    NineToothedTensor weight, NineToothedTensor eps, NineToothedTensor scale, NineToothedTensor shift,
    NineToothedTensor residual, NineToothedTensor out) {
    return rms_family(kGatedRmsModulate, as_stream(stream), x, &gate, &y, weight, eps, &scale, &shift, &residual,
                      out, 0);
}

NineToothedResult launch_h3_rope_exact(NineToothedStream stream, NineToothedTensor x0, NineToothedTensor x1,
                                       NineToothedTensor xp, NineToothedTensor cos, NineToothedTensor sin,
                                       NineToothedTensor y0, NineToothedTensor y1, NineToothedTensor yp) {
    // The three views of each side must be one tensor (the reference's
    // callers alias them, patches/InfiniCore.patch:1131).
    if (x0.data != x1.data || x0.data != xp.data || y0.data != y1.data || y0.data != yp.data) return kInvalid;
    View<3> x3, o3;
    View<2> c, s;
    if (!load_view(x0, 2, x3) || !load_view(y0, 2, o3) || !load_view(cos, 2, c) || !load_view(sin, 2, s))
        return kInvalid;
    // [S, H, 128] as [S, H, 1, 128]
    View<4> x, o;
    x.data = x3.data;
    o.data = o3.data;
    for (int i = 0; i < 2; ++i) {
        x.shape[i] = x3.shape[i];
        x.stride[i] = x3.stride[i];
        o.shape[i] = o3.shape[i];
        o.stride[i] = o3.stride[i];
    }
    x.shape[2] = o.shape[2] = 1;
    x.stride[2] = o.stride[2] = 0;
    x.shape[3] = x3.shape[2];
    x.stride[3] = x3.stride[2];
    o.shape[3] = o3.shape[2];
    o.stride[3] = o3.stride[2];
    return launch_head_rows<kRopeOnly>(as_stream(stream), x, o, c, s, nullptr, 0.0);
}

NineToothedResult launch_h3_qk_norm_rope(NineToothedStream stream, NineToothedTensor x0, NineToothedTensor x1,
                                         NineToothedTensor xp, NineToothedTensor w0, NineToothedTensor w1,
                                         NineToothedTensor wp, NineToothedTensor eps, NineToothedTensor cos,
                                         NineToothedTensor sin, NineToothedTensor y0, NineToothedTensor y1,
                                         NineToothedTensor yp) {
    if (x0.data != x1.data || x0.data != xp.data || y0.data != y1.data || y0.data != yp.data ||
        w0.data != w1.data || w0.data != wp.data)
        return kInvalid;
    View<4> x, o;
    View<2> c, s;
    View<1> w;
    double e;
    if (!load_view(x0, 2, x) || !load_view(y0, 2, o) || !load_view(cos, 2, c) || !load_view(sin, 2, s) ||
        !load_view(w0, 2, w) || !load_scalar(eps, e))
        return kInvalid;
    return launch_head_rows<kNormRope>(as_stream(stream), x, o, c, s, &w, e);
}

NineToothedResult launch_h3_qk_norm_rope_interleaved(NineToothedStream stream, NineToothedTensor x,
                                                     NineToothedTensor weight, NineToothedTensor eps,
                                                     NineToothedTensor cos, NineToothedTensor sin,
                                                     NineToothedTensor out) {
    View<4> xv, o;
    View<2> c, s;
    View<1> w;
    double e;
    if (!load_view(x, 2, xv) || !load_view(out, 2, o) || !load_view(cos, 2, c) || !load_view(sin, 2, s) ||
        !load_view(weight, 2, w) || !load_scalar(eps, e))
        return kInvalid;
    return launch_head_rows<kNormRopeInterleaved>(as_stream(stream), xv, o, c, s, &w, e);
}

NineToothedResult launch_h3_rope_cache(NineToothedStream stream, NineToothedTensor position,
                                       NineToothedTensor power, NineToothedTensor cos, NineToothedTensor sin) {
    View<2> pos, c, s;
    View<1> pw;
    if (!load_view(position, 8, pos) || !load_view(power, 4, pw) || !load_view(cos, 2, c) || !load_view(sin, 2, s))
        return kInvalid;
    if (pos.shape[1] != 3 || pw.shape[0] != 16 || c.shape[0] != pos.shape[0] || c.shape[1] != 48 ||
        !same_shape(c, s))
        return kInvalid;
    const int64_t n = pos.shape[0] * 48;
    if (n == 0) return 0;
    const int64_t grid = (n + kThreads - 1) / kThreads;
    if (grid > static_cast<int64_t>(std::numeric_limits<int32_t>::max())) return kInvalid;
    rope_cache_kernel<<<static_cast<unsigned>(grid), kThreads, 0, as_stream(stream)>>>(
        reinterpret_cast<const double *>(pos.data), pos.stride[0], pos.stride[1],
        reinterpret_cast<const float *>(pw.data), pw.stride[0], reinterpret_cast<bf16_t *>(c.data),
        reinterpret_cast<bf16_t *>(s.data), c.stride[0], c.stride[1], s.stride[0], s.stride[1], n);
    return launch_status();
}

}  // extern "C"
