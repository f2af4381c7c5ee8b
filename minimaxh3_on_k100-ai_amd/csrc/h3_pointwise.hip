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
#include <atomic>

#include "h3_common.hpp"
#include "h3_internal.hpp"

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

// Loads the 8-element group starting at column c0 of a row as packed bf16: a
// 16-byte vector on the VEC path (non-temporal when STREAM, for data read
// once), element by element (zero past W) otherwise.
template <bool VEC, bool STREAM = false>
__device__ __forceinline__ U4 load_group(const bf16_t *row, int64_t sw, int c0, int W) {
    if constexpr (VEC) {
        if constexpr (STREAM) {
            return ld16_stream(row + c0);
        } else {
            return ld16(row + c0);
        }
    } else {
        // Element loads from clamped (valid) indices, zeroed past W by a select.
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const int i0 = c0 + e < W ? c0 + e : W - 1, i1 = c0 + e + 1 < W ? c0 + e + 1 : W - 1;
            const uint32_t lo = row[i0 * sw], hi = row[i1 * sw];
            w[e / 2] = (c0 + e < W ? lo : 0u) | ((c0 + e + 1 < W ? hi : 0u) << 16);
        }
        return {w[0], w[1], w[2], w[3]};
    }
}

template <bool VEC, bool STREAM = false>
__device__ __forceinline__ void store_group(bf16_t *row, int64_t sw, int c0, int W, const U4 &v) {
    if constexpr (VEC) {
        if constexpr (STREAM) {
            st16_stream(row + c0, v);
        } else {
            st16(row + c0, v);
        }
    } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (c0 + e < W) row[(c0 + e) * sw] = static_cast<bf16_t>(w[e >> 1] >> (16 * (e & 1)));
    }
}

template <bool VEC, bool STREAM = false>
__device__ __forceinline__ void load8(const bf16_t *row, int64_t sw, int c0, int W, float f[8]) {
    u4_to_f8(load_group<VEC, STREAM>(row, sw, c0, W), f);
}

template <bool VEC, bool STREAM = false>
__device__ __forceinline__ void store8(bf16_t *row, int64_t sw, int c0, int W, const float f[8]) {
    store_group<VEC, STREAM>(row, sw, c0, W, f8_to_u4(f));
}

// The value of lane (i - N) mod 16 of lane i's 16-lane row (DPP row_ror:N).
template <int N>
__device__ __forceinline__ float row_ror(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, false));
}

// Pairwise fold of one fp32 value over groups of L lanes (L a power of two <=
// 64): stage `off` = L/2, ..., 2, 1 adds lane i ^ off to lane i (the xor
// butterfly). For L >= 16 the stages run without LDS: off = 32 and 16 through
// v_permlane32_swap / v_permlane16_swap (the pair's sum, in either order, is
// v[i] + v[i ^ off] exactly), off = 8 through row_ror:8 (which is i ^ 8 within
// a row), and off = 4, 2, 1 through row_ror:off, which equals i ^ off because
// after the stage above the values repeat with period 2 off within the row.
template <int L>
__device__ __forceinline__ float fold_lanes(float v) {
    if constexpr (L >= 16) {
        if constexpr (L == 64) {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            v = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        if constexpr (L >= 32) {
            const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            v = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        v += row_ror<8>(v);
        v += row_ror<4>(v);
        v += row_ror<2>(v);
        v += row_ror<1>(v);
    } else {
#pragma unroll
        for (int off = L / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, L);
    }
    return v;
}

// ============================================================ RMS family

enum RmsMode { kRms = 0, kRmsModulate = 1, kGatedRmsModulate = 2 };

// Per-token modulation rows: token (b, s) takes row p[b * sb + s * ss] of
// [count, W] tables (scale, shift, gate). p == nullptr: the modulation views
// are [B, S, W] like x and token (b, s) takes their row (b, s).
struct ModIndex {
    const int64_t *p;
    int64_t sb, ss, count;
};

// A value every lane of the wave holds, moved to scalar registers so that
// branches on it are uniform.
__device__ __forceinline__ int64_t uniform64(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// The coordinates of token (b, s)'s modulation row in the modulation views:
// (b, s) itself, or (index[b, s], 0) in the tables (a table is a Rows view with
// its row stride in sb), the index clamped into [0, count) so that no value
// of it reads outside the tables.
__device__ __forceinline__ int64_t index_row(const ModIndex &ix, int64_t b, int64_t s) {
    const int64_t m = ix.p[b * ix.sb + s * ix.ss];
    return m < 0 ? 0 : (m < ix.count ? m : ix.count - 1);
}
__device__ __forceinline__ void mod_coords(const ModIndex &ix, int64_t b, int64_t s, int64_t &mb, int64_t &ms) {
    if (ix.p == nullptr) {
        mb = b;
        ms = s;
    } else {
        mb = index_row(ix, b, s);
        ms = 0;
    }
}

struct RmsArgs {
    Rows x, gate, y, scale, shift, residual, out;
    const bf16_t *w;
    int64_t w_stride;
    int64_t rows, S;
    int W;
    float eps_bf;  // eps already rounded fp64 -> fp32 -> bf16
    bool staged;   // weight, scale, shift and gate are the same for every s of a batch entry
    ModIndex index;  // gate, scale and shift rows per token (indexed entry points)
    FastDiv by_s;    // row -> (b, s): division by S (rows < 2^31)
};

// bf16(1 + scale) of a group: the modulation factor, packed.
__device__ __forceinline__ U4 factor_of(const U4 &scv) {
    float sc[8];
    u4_to_f8(scv, sc);
#pragma unroll
    for (int e = 0; e < 8; ++e) sc[e] += 1.0f;
    return f8_to_u4(sc);
}

// The per-row epilogue shared by every path: value -> normalized -> weighted
// (-> modulated). `r` is the bf16 reciprocal, widened; `k` the factor
// bf16(1 + scale).
template <int MODE>
__device__ __forceinline__ void rms_epilogue(float f[8], float r, const float w[8], const float k[8],
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
            float p0 = a0 * k[e], p1 = a1 * k[e + 1];
            rbf2(p0, p1);  // product = bf16(weighted * factor)
            f[e] = p0 + sh[e];  // out = bf16(product + shift), rounded by the store
            f[e + 1] = p1 + sh[e + 1];
        }
    }
}

// Launch shape of rms_staged_kernel: waves per block and about how many blocks.
constexpr int kStagedThreads = 512;
constexpr int kStagedBlocks = 512;
// rms_stream_kernel (the gated mode): blocks in all (two per CU, as many as the
// staged vectors leave room for), rows in flight per block. Measured at
// S = 8192, C = 7168 against rms_staged_kernel: the gated mode streams faster
// (x and y per row need twice the registers), the others do not.
constexpr int kStreamBlocks = 512;
constexpr int kStreamDepth = 2;

// Loads are issued for every lane from a valid address, and only the arithmetic
// and the stores are guarded: a load under a per-lane branch is waited for
// before the branch closes, which would serialize a wave's loads. Groups past
// the row read its last group (already in flight for another lane) and rows
// past the end read the last row.
__device__ __forceinline__ int clamp_group(int g, int W8) { return g < W8 ? g : W8 - 1; }

// Phase 1 of one group: from the raw x (and, gated, gate and y) groups to the
// value the row is normalized from (gated: the residual bf16(x + bf16(gate y)),
// which the caller stores). When `valid`, its squares are added to `partial`
// left to right; otherwise `partial` is unchanged.
template <int MODE>
__device__ __forceinline__ U4 rms_phase1(const U4 &xv, const U4 &gv, const U4 &yv, bool valid, float &partial) {
    float f[8];
    u4_to_f8(xv, f);
    U4 v = xv;
    if constexpr (MODE == kGatedRmsModulate) {
        float gt[8], yy[8];
        u4_to_f8(gv, gt);
        u4_to_f8(yv, yy);
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            float p0 = gt[e] * yy[e], p1 = gt[e + 1] * yy[e + 1];
            rbf2(p0, p1);  // product = bf16(gate * y)
            float h0 = f[e] + p0, h1 = f[e + 1] + p1;
            rbf2(h0, h1);  // residual = bf16(x + product)
            f[e] = h0;
            f[e + 1] = h1;
        }
        v = f8_to_u4(f);  // exact: the values are bf16
    }
    float sum = partial;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        float q0 = f[e] * f[e], q1 = f[e + 1] * f[e + 1];
        rbf2(q0, q1);  // squared = bf16(value * value)
        sum += q0;
        sum += q1;
    }
    partial = valid ? sum : partial;
    return v;
}

// bf16 reciprocal RMS of a row from its fp32 sum of squares.
__device__ __forceinline__ float rms_reciprocal(float total, int W, float eps_bf) {
    const float mean = rbf(__fdiv_rn(total, static_cast<float>(W)));  // bf16(sum / W)
    const float var = rbf(mean + eps_bf);                             // bf16(mean + eps)
    return rbf(rsqrt_ieee(var));                                      // bf16(rsqrt(var))
}

// Phase 2 of one group: normalize, weight, modulate (kv = bf16(1 + scale)).
template <int MODE>
__device__ __forceinline__ U4 rms_phase2(const U4 &v, float r, const U4 &wv, const U4 &kv, const U4 &shv) {
    float f[8], w[8], k[8], sh[8];
    u4_to_f8(v, f);
    u4_to_f8(wv, w);
    if constexpr (MODE != kRms) {
        u4_to_f8(kv, k);
        u4_to_f8(shv, sh);
    }
    rms_epilogue<MODE>(f, r, w, k, sh);
    return f8_to_u4(f);
}

// Rows of W8 <= 64 groups: a group of L lanes per row (L = next power of two
// >= W8, lane g owns group g) and R rows per lane group. Every load of the
// block (x, gate, y, weight, scale, shift) is issued before the first store.
template <int L, int R, bool VEC, int MODE>
__global__ __launch_bounds__(kThreads) void rms_lanes_kernel(RmsArgs a) {
    constexpr int kGroups = kThreads / L;
    const int lane = threadIdx.x % L;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kGroups * R + threadIdx.x / L;
    const int W8 = (a.W + 7) / 8;
    const int c0 = clamp_group(lane, W8) * 8;
    int64_t b[R], s[R];
    bool ok[R];
    U4 xv[R], gv[R], yv[R], scv[R], shv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = base + r * kGroups;
        ok[r] = row < a.rows && lane < W8;
        const int64_t rr = row < a.rows ? row : a.rows - 1;
        b[r] = rr / a.S;
        s[r] = rr % a.S;
        xv[r] = load_group<VEC, true>(row_ptr(a.x, b[r], s[r]), a.x.sw, c0, a.W);
        if constexpr (MODE == kGatedRmsModulate)
            yv[r] = load_group<VEC, true>(row_ptr(a.y, b[r], s[r]), a.y.sw, c0, a.W);
        if constexpr (MODE != kRms) {
            int64_t mb, ms;
            mod_coords(a.index, b[r], s[r], mb, ms);
            if constexpr (MODE == kGatedRmsModulate)
                gv[r] = load_group<VEC>(row_ptr(a.gate, mb, ms), a.gate.sw, c0, a.W);
            scv[r] = load_group<VEC>(row_ptr(a.scale, mb, ms), a.scale.sw, c0, a.W);
            shv[r] = load_group<VEC>(row_ptr(a.shift, mb, ms), a.shift.sw, c0, a.W);
        }
    }
    const U4 wv = load_group<VEC>(a.w, a.w_stride, c0, a.W);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float partial = 0.0f;
        const U4 v = rms_phase1<MODE>(xv[r], gv[r], yv[r], ok[r], partial);
        if constexpr (MODE == kGatedRmsModulate)
            if (ok[r]) store_group<VEC, true>(row_ptr_w(a.residual, b[r], s[r]), a.residual.sw, c0, a.W, v);
        const float rcp = rms_reciprocal(fold_lanes<L>(partial), a.W, a.eps_bf);
        const U4 o = rms_phase2<MODE>(v, rcp, wv, factor_of(scv[r]), shv[r]);
        if (ok[r]) store_group<VEC, true>(row_ptr_w(a.out, b[r], s[r]), a.out.sw, c0, a.W, o);
    }
}

// Rows of 64 < W8 <= 64 * G groups with per-row modulation (or a generic
// layout): one row per wave. Lane l takes groups l + 64k (k < G) and keeps four
// partial sums, one for each of the threads l + 64w (w = k mod 4) of the
// 256-thread order, which it reproduces exactly. Weight, scale and shift come
// in batches of four groups, each batch's loads issued before the previous
// batch's stores.
template <int G, bool VEC, int MODE>
__global__ __launch_bounds__(kThreads) void rms_wave_kernel(RmsArgs a) {
    constexpr int kChunk = 4;
    constexpr int kChunks = (G + kChunk - 1) / kChunk;
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= a.rows) return;  // whole waves only; no block-level synchronization below
    const int64_t b = row / a.S, s = row % a.S;
    int64_t mb, ms;
    mod_coords(a.index, b, s, mb, ms);
    const int W8 = (a.W + 7) / 8;
    U4 v[G], gv[G], yv[G];
#pragma unroll
    for (int k = 0; k < G; ++k) {
        const int c0 = clamp_group(lane + 64 * k, W8) * 8;
        v[k] = load_group<VEC, true>(row_ptr(a.x, b, s), a.x.sw, c0, a.W);
        if constexpr (MODE == kGatedRmsModulate) {
            gv[k] = load_group<VEC>(row_ptr(a.gate, mb, ms), a.gate.sw, c0, a.W);
            yv[k] = load_group<VEC, true>(row_ptr(a.y, b, s), a.y.sw, c0, a.W);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // the row's loads stay together, ahead of its arithmetic
    U4 wv[2][kChunk], scv[2][kChunk], shv[2][kChunk];
    auto load_chunk = [&](int c) {
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            const int c0 = clamp_group(lane + 64 * (c * kChunk + j), W8) * 8;
            wv[c & 1][j] = load_group<VEC>(a.w, a.w_stride, c0, a.W);
            if constexpr (MODE != kRms) {
                scv[c & 1][j] = load_group<VEC>(row_ptr(a.scale, mb, ms), a.scale.sw, c0, a.W);
                shv[c & 1][j] = load_group<VEC>(row_ptr(a.shift, mb, ms), a.shift.sw, c0, a.W);
            }
        }
    };
    load_chunk(0);
    float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < G; ++k) {
        const int g = lane + 64 * k;
        v[k] = rms_phase1<MODE>(v[k], gv[k], yv[k], g < W8, part[k & 3]);
        if constexpr (MODE == kGatedRmsModulate)
            if (g < W8) store_group<VEC, true>(row_ptr_w(a.residual, b, s), a.residual.sw, g * 8, a.W, v[k]);
        keep_packed(v[k]);
    }
    const float total = (fold_lanes<64>(part[0]) + fold_lanes<64>(part[2])) +
                        (fold_lanes<64>(part[1]) + fold_lanes<64>(part[3]));
    const float r = rms_reciprocal(total, a.W, a.eps_bf);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        if (c + 1 < kChunks) load_chunk(c + 1);
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            const int k = c * kChunk + j, g = lane + 64 * k;
            if (k < G) {
                const U4 o = rms_phase2<MODE>(v[k], r, wv[c & 1][j], factor_of(scv[c & 1][j]), shv[c & 1][j]);
                if (g < W8) store_group<VEC, true>(row_ptr_w(a.out, b, s), a.out.sw, g * 8, a.W, o);
            }
        }
    }
}

// Stages the row-invariant vectors of batch entry b in LDS: weight,
// bf16(1 + scale), shift and (gated) gate, W8 groups each.
template <int MODE, int THREADS>
__device__ __forceinline__ void stage_vectors(const RmsArgs &a, int64_t b, int W8, U4 *staged) {
    for (int g = threadIdx.x; g < W8; g += THREADS) {
        staged[g] = ld16(a.w + g * 8);
        if constexpr (MODE != kRms) {
            staged[W8 + g] = factor_of(ld16(row_ptr(a.scale, b, 0) + g * 8));
            staged[2 * W8 + g] = ld16(row_ptr(a.shift, b, 0) + g * 8);
        }
        if constexpr (MODE == kGatedRmsModulate) staged[3 * W8 + g] = ld16(row_ptr(a.gate, b, 0) + g * 8);
    }
    __syncthreads();
}

// Rows whose weight, modulation and gate vectors are the same for every s of
// a batch entry b (broadcast over S, or S = 1), W8 <= 64 * G: the block stages
// those vectors in LDS once, and each wave streams whole rows of b through
// registers in the order of rms_wave_kernel, the rows grid-strided so that
// the rows in flight are close together in memory. After a row's own loads the
// only global accesses are its stores.
//
// EXACT: W8 = 64 G, so no group is clamped or masked; the row's addresses are
// then one base and constant offsets, the kernel is held to 80 VGPRs (at
// G = 14 it fits them without spilling), and three
// 512-thread blocks share a CU (24 waves, 6144 rows in flight over the chip):
// measured 46.5 against 49.5 us for the clamped form at two blocks per CU
// (RMSNorm + AdaLN at [8192, 7168]). The EXACT kernel over 2 or 4 blocks per CU
// measured 51 us; 16-byte aligned LDS reads of the staged rows (ds_read_b128
// instead of ds_read2_b32 pairs) made it spill 284 bytes and cost 2.4x.
template <int G, int MODE, int THREADS, bool EXACT>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(EXACT ? 6 : 1)))
void rms_staged_kernel(RmsArgs a) {
    static_assert(MODE != kGatedRmsModulate, "the gated mode runs as rms_stream_kernel");
    extern __shared__ U4 staged[];
    const int W8 = (a.W + 7) / 8;
    const int64_t b = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int64_t step = static_cast<int64_t>(gridDim.x) * (THREADS / 64);
    auto group = [&](int g) { return EXACT ? g : clamp_group(g, W8); };
    U4 v[G], yv[G];
    auto load_row = [&](int64_t s) {
#pragma unroll
        for (int k = 0; k < G; ++k) {
            const int c0 = group(lane + 64 * k) * 8;
            v[k] = ld16_stream(row_ptr(a.x, b, s) + c0);
            if constexpr (MODE == kGatedRmsModulate) yv[k] = ld16_stream(row_ptr(a.y, b, s) + c0);
        }
        // The row's loads stay together, ahead of its arithmetic (EXACT's
        // constant offsets keep them together without the barrier, in fewer
        // registers).
        if constexpr (!EXACT) __builtin_amdgcn_sched_barrier(0);
    };
    int64_t s = static_cast<int64_t>(blockIdx.x) * (THREADS / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // The first row's loads go out before the vectors are staged (a wave
    // without rows re-reads the last one and stores nothing).
    load_row(s < a.S ? s : a.S - 1);
    stage_vectors<MODE, THREADS>(a, b, W8, staged);
    const U4 *lw = staged, *lk = staged + W8, *lsh = staged + 2 * W8, *lg = staged + 3 * W8;
    for (bool first = true; s < a.S; s += step, first = false) {
        if (!first) load_row(s);
        float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < G; ++k) {
            const int g = lane + 64 * k, gc = group(g);
            U4 gv{};
            if constexpr (MODE == kGatedRmsModulate) gv = lg[gc];
            v[k] = rms_phase1<MODE>(v[k], gv, yv[k], EXACT || g < W8, part[k & 3]);
            if constexpr (MODE == kGatedRmsModulate)
                if (EXACT || g < W8) st16_stream(row_ptr_w(a.residual, b, s) + g * 8, v[k]);
            keep_packed(v[k]);
        }
        const float total = (fold_lanes<64>(part[0]) + fold_lanes<64>(part[2])) +
                            (fold_lanes<64>(part[1]) + fold_lanes<64>(part[3]));
        const float r = rms_reciprocal(total, a.W, a.eps_bf);
#pragma unroll
        for (int k = 0; k < G; ++k) {
            const int g = lane + 64 * k, gc = group(g);
            U4 kv{}, shv{};
            if constexpr (MODE != kRms) {
                kv = lk[gc];
                shv = lsh[gc];
            }
            const U4 o = rms_phase2<MODE>(v[k], r, lw[gc], kv, shv);
            if (EXACT || g < W8) st16_stream(row_ptr_w(a.out, b, s) + g * 8, o);
        }
    }
}

// RMSNorm + AdaLN with per-token modulation rows (ModIndex), W8 <= 64 * G:
// rms_staged_kernel's order and register use over all B * S rows. A block
// takes groups of kWaves consecutive rows, one per wave, the groups
// grid-strided. The weight is staged once. Lane j < kWaves of every wave
// splits row j of the group into (b, s) with the launch-time division by S and
// loads that row's index (lanes past kWaves repeat them), before the wave's
// own row is loaded, so the index arrives first. One ballot tells every wave
// whether the group's kWaves indices name one table row -- nearly every group,
// the indices coming in long runs -- and each wave takes its own (b, s) and
// index from lane `wave`. All waves therefore take the same branches: a group
// of one table row stages that row's factor and shift in LDS unless they are
// there already; a group across a run boundary reads each row's factor and
// shift from the tables (L2) instead. The launch bound keeps two blocks
// resident per CU up to G = 14 (W = 7168).
//
// EXACT: W8 = 64 G, so no group is clamped or masked.
template <int G, int THREADS, bool EXACT>
__global__ __launch_bounds__(THREADS, G <= 14 ? 4 : 3) void rms_modulate_indexed_kernel(RmsArgs a) {
    constexpr int kWaves = THREADS / 64;
    static_assert((kWaves & (kWaves - 1)) == 0 && kWaves <= 64, "a power-of-two number of waves");
    extern __shared__ U4 staged[];
    const int W8 = (a.W + 7) / 8;
    U4 *lw = staged, *lk = staged + W8, *lsh = staged + 2 * W8;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t step = static_cast<int64_t>(gridDim.x) * kWaves;
    const int64_t last = a.rows - 1;
    const uint32_t S32 = static_cast<uint32_t>(a.S);
    U4 v[G];
    auto load_row = [&](int64_t b, int64_t s) {
#pragma unroll
        for (int k = 0; k < G; ++k)
            v[k] = ld16_stream(row_ptr(a.x, b, s) + (EXACT ? lane + 64 * k : clamp_group(lane + 64 * k, W8)) * 8);
        // The row's loads stay together, ahead of its arithmetic (EXACT's
        // constant offsets keep them together without the barrier).
        if constexpr (!EXACT) __builtin_amdgcn_sched_barrier(0);
    };
    int64_t in_lds = -1;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * kWaves; base < a.rows; base += step) {
        // same trip count in every wave
        const bool ok = base + wave < a.rows;
        // Row j of the group in lane j (rows past the end repeat the last
        // row): (b, s) and its index; no load sits under a branch.
        const int64_t rj64 = base + (lane & (kWaves - 1));
        const uint32_t rj = static_cast<uint32_t>(rj64 < last ? rj64 : last);
        const uint32_t bj = fast_div(rj, a.by_s), sj = rj - bj * S32;
        const int64_t mj = index_row(a.index, bj, sj);
        const int64_t b = __builtin_amdgcn_readlane(static_cast<int>(bj), wave);
        const int64_t s = __builtin_amdgcn_readlane(static_cast<int>(sj), wave);
        load_row(b, s);
        const int64_t m0 = uniform64(mj);
        const bool same = __builtin_amdgcn_ballot_w64(mj != m0) == 0;
        const int64_t mine = static_cast<int64_t>(
            (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(mj >> 32), wave)))
             << 32) |
            static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(mj), wave)));
        // Staging: the weight with the first group, the group's table row when
        // it changes. The loads go out while the row's own are in flight.
        const bool first = base == static_cast<int64_t>(blockIdx.x) * kWaves;
        const bool restage = same && m0 != in_lds;
        if (first || restage) {
            if (!first) __syncthreads();  // the earlier groups' reads of the staged rows are done
            for (int g = threadIdx.x; g < W8; g += THREADS) {
                if (first) lw[g] = ld16(a.w + g * 8);
                if (restage) {
                    lk[g] = factor_of(ld16(row_ptr(a.scale, m0, 0) + g * 8));
                    lsh[g] = ld16(row_ptr(a.shift, m0, 0) + g * 8);
                }
            }
            __syncthreads();
            in_lds = restage ? m0 : in_lds;
        }
        float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < G; ++k) {
            const U4 unused{};
            v[k] = rms_phase1<kRmsModulate>(v[k], unused, unused, EXACT || lane + 64 * k < W8, part[k & 3]);
            keep_packed(v[k]);
        }
        const float total = (fold_lanes<64>(part[0]) + fold_lanes<64>(part[2])) +
                            (fold_lanes<64>(part[1]) + fold_lanes<64>(part[3]));
        const float r = rms_reciprocal(total, a.W, a.eps_bf);
        if (same) {
#pragma unroll
            for (int k = 0; k < G; ++k) {
                const int g = lane + 64 * k, gc = EXACT ? g : clamp_group(g, W8);
                const U4 o = rms_phase2<kRmsModulate>(v[k], r, lw[gc], lk[gc], lsh[gc]);
                if (ok && (EXACT || g < W8)) st16_stream(row_ptr_w(a.out, b, s) + g * 8, o);
            }
        } else {
#pragma unroll
            for (int k = 0; k < G; ++k) {
                const int g = lane + 64 * k, gc = EXACT ? g : clamp_group(g, W8);
                const U4 kv = factor_of(ld16(row_ptr(a.scale, mine, 0) + gc * 8));
                const U4 shv = ld16(row_ptr(a.shift, mine, 0) + gc * 8);
                const U4 o = rms_phase2<kRmsModulate>(v[k], r, lw[gc], kv, shv);
                if (ok && (EXACT || g < W8)) st16_stream(row_ptr_w(a.out, b, s) + g * 8, o);
                __builtin_amdgcn_sched_barrier(0);  // one group's table loads at a time (registers)
            }
        }
    }
}

// Rows whose weight, modulation and gate vectors are the same for every s of
// a batch entry b: one row at a time per 256-thread block, thread t owning
// groups t, t + 256, ... (the fixed order itself). The block stages the
// vectors in LDS once, then walks the rows of entry b grid-strided with a ring
// of DEPTH rows in registers (the loads of the next DEPTH - 1 rows are in
// flight while a row is reduced and written), so the blocks stream a sliding
// window of rows. The four wave partials meet in LDS (double-buffered by row
// parity, one barrier per row).
//
// INDEXED: every token names its modulation row (ModIndex). The blocks walk
// all B * S rows grid-strided; a row's index is loaded with its data (one
// value for the whole block), and the block stages that row of the tables
// whenever it differs from the one in LDS -- once per run of equal indices a
// block meets, since a block's rows are in token order.
template <int VPT, int MODE, int DEPTH, bool INDEXED>
__global__ __launch_bounds__(kThreads) void rms_stream_kernel(RmsArgs a) {
    extern __shared__ U4 staged[];
    __shared__ float red[2][kThreads / 64];
    const int W8 = (a.W + 7) / 8;
    const int64_t count = INDEXED ? a.rows : a.S;  // rows this block's grid walks
    const int64_t b0 = INDEXED ? 0 : blockIdx.y;
    if constexpr (!INDEXED) stage_vectors<MODE, kThreads>(a, b0, W8, staged);
    const U4 *lw = staged, *lk = staged + W8, *lsh = staged + 2 * W8, *lg = staged + 3 * W8;
    const int64_t step = gridDim.x;
    U4 xr[DEPTH][VPT], yr[DEPTH][VPT];
    int64_t mr[DEPTH];     // INDEXED: the modulation row of each row in the ring
    int64_t in_lds = -1;   // INDEXED: the modulation row staged in LDS
    // Rows past the end (block-uniform) re-read the last row; only stores are guarded.
    auto load_row = [&](int64_t i, U4 (&xv)[VPT], U4 (&yv)[VPT], int64_t &m) {
        const int64_t ic = i < count ? i : count - 1;
        const int64_t b = INDEXED ? ic / a.S : b0, s = INDEXED ? ic % a.S : ic;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int c0 = clamp_group(threadIdx.x + j * kThreads, W8) * 8;
            xv[j] = ld16_stream(row_ptr(a.x, b, s) + c0);
            if constexpr (MODE == kGatedRmsModulate) yv[j] = ld16_stream(row_ptr(a.y, b, s) + c0);
        }
        if constexpr (INDEXED) {
            int64_t ms;
            mod_coords(a.index, b, s, m, ms);
        }
    };
    auto finish_row = [&](int64_t i, int parity, U4 (&xv)[VPT], U4 (&yv)[VPT], int64_t m) {
        const bool ok = i < count;
        const int64_t b = INDEXED ? i / a.S : b0, s = INDEXED ? i % a.S : i;
        if constexpr (INDEXED) {
            m = uniform64(m);  // every thread loaded the same index
            if (m != in_lds) {
                __syncthreads();  // the previous row's reads of the staged vectors are done
                stage_vectors<MODE, kThreads>(a, m, W8, staged);
                in_lds = m;
            }
        }
        float partial = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int g = threadIdx.x + j * kThreads, gc = clamp_group(g, W8);
            U4 gv{};
            if constexpr (MODE == kGatedRmsModulate) gv = lg[gc];
            xv[j] = rms_phase1<MODE>(xv[j], gv, yv[j], g < W8, partial);
            if constexpr (MODE == kGatedRmsModulate)
                if (ok && g < W8) st16_stream(row_ptr_w(a.residual, b, s) + g * 8, xv[j]);
            keep_packed(xv[j]);
        }
        const float wsum = fold_lanes<64>(partial);
        if ((threadIdx.x & 63) == 0) red[parity][threadIdx.x >> 6] = wsum;
        __syncthreads();
        const float *t = red[parity];
        const float r = rms_reciprocal((t[0] + t[2]) + (t[1] + t[3]), a.W, a.eps_bf);
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int g = threadIdx.x + j * kThreads, gc = clamp_group(g, W8);
            U4 kv{}, shv{};
            if constexpr (MODE != kRms) {
                kv = lk[gc];
                shv = lsh[gc];
            }
            const U4 o = rms_phase2<MODE>(xv[j], r, lw[gc], kv, shv);
            if (ok && g < W8) st16_stream(row_ptr_w(a.out, b, s) + g * 8, o);
        }
    };
    const int64_t first = blockIdx.x;
#pragma unroll
    for (int d = 0; d < DEPTH - 1; ++d) load_row(first + d * step, xr[d], yr[d], mr[d]);
    int parity = 0;
    for (int64_t base = first; base < count; base += DEPTH * step) {  // same trip count in every wave
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int64_t i = base + d * step;
            const int nd = (d + DEPTH - 1) % DEPTH;
            load_row(i + (DEPTH - 1) * step, xr[nd], yr[nd], mr[nd]);
            finish_row(i, parity, xr[d], yr[d], mr[d]);
            parity ^= 1;
        }
    }
}

// Rows of W8 > 1024 groups: one row per 256-thread block, VPT groups per
// thread (thread t owns groups t, t + 256, ...), the four wave partials
// combined as (w0 + w2) + (w1 + w3).
template <int VPT, bool VEC, int MODE>
__global__ __launch_bounds__(kThreads) void rms_block_kernel(RmsArgs a) {
    const int64_t row = blockIdx.x;
    const int64_t b = row / a.S, s = row % a.S;
    int64_t mb, ms;
    mod_coords(a.index, b, s, mb, ms);
    const int W8 = (a.W + 7) / 8;
    U4 v[VPT], gv[VPT], yv[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c0 = clamp_group(threadIdx.x + j * kThreads, W8) * 8;
        v[j] = load_group<VEC, true>(row_ptr(a.x, b, s), a.x.sw, c0, a.W);
        if constexpr (MODE == kGatedRmsModulate) {
            gv[j] = load_group<VEC>(row_ptr(a.gate, mb, ms), a.gate.sw, c0, a.W);
            yv[j] = load_group<VEC, true>(row_ptr(a.y, b, s), a.y.sw, c0, a.W);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // the row's loads stay together, ahead of its arithmetic
    float partial = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int g = threadIdx.x + j * kThreads;
        v[j] = rms_phase1<MODE>(v[j], gv[j], yv[j], g < W8, partial);
        if constexpr (MODE == kGatedRmsModulate)
            if (g < W8) store_group<VEC, true>(row_ptr_w(a.residual, b, s), a.residual.sw, g * 8, a.W, v[j]);
        keep_packed(v[j]);
    }
    __shared__ float red[kThreads / 64];
    const float wsum = fold_lanes<64>(partial);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = wsum;
    __syncthreads();
    const float r = rms_reciprocal((red[0] + red[2]) + (red[1] + red[3]), a.W, a.eps_bf);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int g = threadIdx.x + j * kThreads, c0 = clamp_group(g, W8) * 8;
        const U4 wv = load_group<VEC>(a.w, a.w_stride, c0, a.W);
        U4 scv{}, shv{};
        if constexpr (MODE != kRms) {
            scv = load_group<VEC>(row_ptr(a.scale, mb, ms), a.scale.sw, c0, a.W);
            shv = load_group<VEC>(row_ptr(a.shift, mb, ms), a.shift.sw, c0, a.W);
        }
        const U4 o = rms_phase2<MODE>(v[j], r, wv, factor_of(scv), shv);
        if (g < W8) store_group<VEC, true>(row_ptr_w(a.out, b, s), a.out.sw, g * 8, a.W, o);
    }
}

template <int MODE, bool VEC>
int launch_rms_vec(const RmsArgs &a, hipStream_t stream) {
    const int W8 = (a.W + 7) / 8;
    if (W8 <= 64) {
        int L = 1;
        while (L < W8) L <<= 1;
        // Four rows per lane group when that still leaves >= 1024 blocks.
        const int64_t rows_per_block4 = static_cast<int64_t>(kThreads / L) * 4;
        const bool four = (a.rows + rows_per_block4 - 1) / rows_per_block4 >= 1024;
        const int64_t per_block = four ? rows_per_block4 : kThreads / L;
        const unsigned grid = static_cast<unsigned>((a.rows + per_block - 1) / per_block);
        switch (L) {
#define H3_RMS_LANES(LL)                                                                  \
    case LL:                                                                             \
        if (four)                                                                        \
            rms_lanes_kernel<LL, 4, VEC, MODE><<<grid, kThreads, 0, stream>>>(a);        \
        else                                                                             \
            rms_lanes_kernel<LL, 1, VEC, MODE><<<grid, kThreads, 0, stream>>>(a);        \
        break;
            H3_RMS_LANES(1) H3_RMS_LANES(2) H3_RMS_LANES(4) H3_RMS_LANES(8) H3_RMS_LANES(16)
            H3_RMS_LANES(32) H3_RMS_LANES(64)
#undef H3_RMS_LANES
        }
        return launch_status();
    }
    const int need = (W8 + 63) / 64;
    // Staged vectors: 1 (weight), 3 (+ factor, shift) or 4 (+ gate) rows of W8
    // groups in LDS, within the 64 KiB a workgroup may allocate.
    const int arrays = MODE == kRms ? 1 : (MODE == kRmsModulate ? 3 : 4);
    const size_t lds = static_cast<size_t>(arrays) * W8 * sizeof(U4);
    if constexpr (VEC && MODE != kRms) {
        // Per-token modulation rows: rms_stream_kernel over all rows, restaging
        // the tables' row at each change of index.
        const int vpt = (W8 + kThreads - 1) / kThreads;
        if (MODE == kRmsModulate && a.index.p != nullptr && lds <= 65536 && need <= 16) {
            constexpr int kWaves = kStagedThreads / 64;
            const int64_t groups = (a.rows + kWaves - 1) / kWaves;
            const bool exact = W8 % 64 == 0;
            const unsigned grid = static_cast<unsigned>(groups < kStagedBlocks ? groups : kStagedBlocks);
#define H3_RMS_MOD_INDEXED(GG)                                                                                    \
    if (need <= GG) {                                                                                            \
        if (exact && W8 == 64 * GG)                                                                              \
            rms_modulate_indexed_kernel<GG, kStagedThreads, true><<<grid, kStagedThreads, lds, stream>>>(a);    \
        else                                                                                                     \
            rms_modulate_indexed_kernel<GG, kStagedThreads, false><<<grid, kStagedThreads, lds, stream>>>(a);   \
        return launch_status();                                                                                  \
    }
            H3_RMS_MOD_INDEXED(2) H3_RMS_MOD_INDEXED(3) H3_RMS_MOD_INDEXED(4) H3_RMS_MOD_INDEXED(6)
            H3_RMS_MOD_INDEXED(8) H3_RMS_MOD_INDEXED(10) H3_RMS_MOD_INDEXED(12) H3_RMS_MOD_INDEXED(14)
            H3_RMS_MOD_INDEXED(16)
#undef H3_RMS_MOD_INDEXED
        }
        if (a.index.p != nullptr && lds <= 65536 && vpt <= 4) {
            const unsigned grid = static_cast<unsigned>(a.rows < kStreamBlocks ? a.rows : kStreamBlocks);
#define H3_RMS_STREAM_INDEXED(V)                                                            \
    if (vpt <= V) {                                                                        \
        rms_stream_kernel<V, MODE, kStreamDepth, true><<<grid, kThreads, lds, stream>>>(a); \
        return launch_status();                                                            \
    }
            H3_RMS_STREAM_INDEXED(1) H3_RMS_STREAM_INDEXED(2) H3_RMS_STREAM_INDEXED(3) H3_RMS_STREAM_INDEXED(4)
#undef H3_RMS_STREAM_INDEXED
        }
    }
    if (VEC && a.staged && lds <= 65536) {
        if constexpr (VEC) {
            const unsigned batch = static_cast<unsigned>(a.rows / a.S);
            if constexpr (MODE == kGatedRmsModulate) {
                const int64_t per_entry = (kStreamBlocks + batch - 1) / batch;
                const dim3 grid(static_cast<unsigned>(a.S < per_entry ? a.S : per_entry), batch);
                const int vpt = (W8 + kThreads - 1) / kThreads;
#define H3_RMS_STREAM(V)                                                                    \
    if (vpt <= V) {                                                                        \
        rms_stream_kernel<V, MODE, kStreamDepth, false><<<grid, kThreads, lds, stream>>>(a); \
        return launch_status();                                                            \
    }
                H3_RMS_STREAM(1) H3_RMS_STREAM(2) H3_RMS_STREAM(3) H3_RMS_STREAM(4)
#undef H3_RMS_STREAM
            } else if (need <= 16) {
                constexpr int kWaves = kStagedThreads / 64;
                // EXACT (W8 = 64 G): three blocks per CU; otherwise about two.
                const bool exact = W8 % 64 == 0;
                int cus = exact ? stream_device_cus(stream) : 0;
                const int64_t blocks = exact && cus > 0 ? 3 * static_cast<int64_t>(cus) : kStagedBlocks;
                const int64_t per_entry = (blocks + batch - 1) / batch;
                const int64_t needed = (a.S + kWaves - 1) / kWaves;
                const dim3 grid(static_cast<unsigned>(needed < per_entry ? needed : per_entry), batch);
#define H3_RMS_STAGED(GG)                                                                               \
    if (need <= GG) {                                                                                  \
        if (exact && W8 == 64 * GG)                                                                    \
            rms_staged_kernel<GG, MODE, kStagedThreads, true><<<grid, kStagedThreads, lds, stream>>>(a);  \
        else                                                                                           \
            rms_staged_kernel<GG, MODE, kStagedThreads, false><<<grid, kStagedThreads, lds, stream>>>(a); \
        return launch_status();                                                                        \
    }
                H3_RMS_STAGED(2) H3_RMS_STAGED(3) H3_RMS_STAGED(4) H3_RMS_STAGED(6) H3_RMS_STAGED(8)
                H3_RMS_STAGED(10) H3_RMS_STAGED(12) H3_RMS_STAGED(14) H3_RMS_STAGED(16)
#undef H3_RMS_STAGED
            }
        }
    }
    if (need <= 16) {
        const unsigned grid = static_cast<unsigned>((a.rows + kThreads / 64 - 1) / (kThreads / 64));
#define H3_RMS_WAVE(GG)                                                            \
    if (need <= GG) {                                                             \
        rms_wave_kernel<GG, VEC, MODE><<<grid, kThreads, 0, stream>>>(a);         \
        return launch_status();                                                   \
    }
        H3_RMS_WAVE(2) H3_RMS_WAVE(3) H3_RMS_WAVE(4) H3_RMS_WAVE(6) H3_RMS_WAVE(8) H3_RMS_WAVE(10)
        H3_RMS_WAVE(12) H3_RMS_WAVE(14) H3_RMS_WAVE(16)
#undef H3_RMS_WAVE
    }
    const int vpt = (W8 + kThreads - 1) / kThreads;
    const unsigned grid = static_cast<unsigned>(a.rows);
#define H3_RMS_BLOCK(V)                                                                \
    if (vpt <= V) {                                                                   \
        rms_block_kernel<V, VEC, MODE><<<grid, kThreads, 0, stream>>>(a);             \
        return launch_status();                                                       \
    }
    H3_RMS_BLOCK(6) H3_RMS_BLOCK(8) H3_RMS_BLOCK(12) H3_RMS_BLOCK(16)
#undef H3_RMS_BLOCK
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

// A modulation operand (scale, shift, gate) as the kernels address it: a
// [B, S, W] view shaped like x, or, with a per-token index, a [R, W] table
// whose row r is addressed as (r, 0) (Rows with the row stride in sb). `vec`
// drops to false when the operand cannot be read with 16-byte vectors;
// `invariant` when its rows differ within a batch entry (views only);
// `table_rows` takes R from the first table and checks the others against it.
bool load_modulation(const NineToothedTensor &t, const View<3> &x, bool indexed, Rows &r, bool &vec,
                     bool &invariant, int64_t &table_rows) {
    if (!indexed) {
        View<3> v;
        if (!load_view(t, 2, v) || !same_shape(x, v)) return false;
        r = rows_of(v);
        vec = vec && rows_vec16(v, 2);
        invariant = invariant && (v.shape[1] == 1 || v.stride[1] == 0);
        return true;
    }
    View<2> v;
    if (!load_view(t, 2, v) || v.shape[1] != x.shape[2]) return false;
    if (table_rows < 0) table_rows = v.shape[0];
    if (v.shape[0] != table_rows) return false;
    r = {v.data, v.stride[0], 0, v.stride[1]};
    vec = vec && rows_vec16(v, 2);
    return true;
}

// The RMS family's launcher. `index_t` (indexed entry points only): int64
// [B, S], token (b, s)'s row of the [R, W] gate / scale / shift tables.
int rms_family(int mode, hipStream_t stream, const NineToothedTensor &x_t, const NineToothedTensor *gate_t,
               const NineToothedTensor *y_t, const NineToothedTensor &w_t, const NineToothedTensor &eps_t,
               const NineToothedTensor *scale_t, const NineToothedTensor *shift_t,
               const NineToothedTensor *residual_t, const NineToothedTensor &out_t, int required_width,
               const NineToothedTensor *index_t = nullptr) {
    View<3> x, out, y, residual;
    View<1> w;
    double eps;
    if (!load_view(x_t, 2, x) || !load_view(out_t, 2, out) || !load_view(w_t, 2, w) || !load_scalar(eps_t, eps))
        return kInvalid;
    if (!same_shape(x, out) || w.shape[0] != x.shape[2]) return kInvalid;
    if (required_width > 0 && x.shape[2] != required_width) return kInvalid;
    if (x.shape[2] > 32768) return kInvalid;
    bool vec = rows_vec16(x, 2) && rows_vec16(out, 2) && rows_vec16(w, 2);
    RmsArgs a{};
    const bool indexed = index_t != nullptr;
    bool invariant = true;  // every modulation operand is the same for all s of a batch entry
    int64_t table_rows = -1;
    if (mode == kGatedRmsModulate) {
        if (!load_view(*y_t, 2, y) || !load_view(*residual_t, 2, residual)) return kInvalid;
        if (!same_shape(x, y) || !same_shape(x, residual)) return kInvalid;
        vec = vec && rows_vec16(y, 2) && rows_vec16(residual, 2);
        if (!load_modulation(*gate_t, x, indexed, a.gate, vec, invariant, table_rows)) return kInvalid;
    }
    if (mode != kRms) {
        if (!load_modulation(*scale_t, x, indexed, a.scale, vec, invariant, table_rows) ||
            !load_modulation(*shift_t, x, indexed, a.shift, vec, invariant, table_rows))
            return kInvalid;
    }
    if (indexed) {
        View<2> ix;
        if (mode == kRms || !load_view(*index_t, 8, ix)) return kInvalid;
        if (ix.shape[0] != x.shape[0] || ix.shape[1] != x.shape[1]) return kInvalid;
        if (table_rows == 0 && x.numel() != 0) return kInvalid;  // no row for the tokens to take
        a.index = {reinterpret_cast<const int64_t *>(ix.data), ix.stride[0], ix.stride[1], table_rows};
    }
    a.x = rows_of(x);
    a.out = rows_of(out);
    if (mode != kGatedRmsModulate) a.gate = a.x;
    a.y = mode == kGatedRmsModulate ? rows_of(y) : a.x;
    a.residual = mode == kGatedRmsModulate ? rows_of(residual) : a.out;
    if (mode == kRms) a.scale = a.shift = a.x;
    a.w = reinterpret_cast<const bf16_t *>(w.data);
    a.w_stride = w.stride[0];
    a.rows = x.shape[0] * x.shape[1];
    a.S = x.shape[1];
    a.by_s = make_fastdiv(static_cast<uint32_t>(a.S > 0 ? a.S : 1));
    a.W = static_cast<int>(x.shape[2]);
    a.eps_bf = host_round_bf16(eps);
    // Row-invariant within a batch entry: broadcast over S (stride 0) or S = 1.
    a.staged = !indexed && x.shape[0] <= 65535 && invariant;
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
// chunk*256*U + t + 256*u with U = Op::kUnroll (measured best per op: more
// waves beat more loads per wave). Loads are issued before any store.

struct EwArgs {
    Rows a, b, c, out;  // op inputs (c unused by SwiGLU) and output
    int64_t rows, S;
    int W, chunks;
    ModIndex index;  // IDX kernels: token (b, s) reads row index[b, s] of the table `b`
};

// out = bf16(x + bf16(gate * y)) (tools/h3_pointwise.py:121-124)
struct GatedResidualOp {
    static constexpr int kInputs = 3;
    static constexpr unsigned kStream = 0b101;  // x, y streamed; gate (an AdaLN row, reused) cached
    static constexpr int kUnroll = 1;
    static constexpr bool kIndexable = true;  // the gate may be a table row per token
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

// silu(g) = g / (1 + exp(-g)) in fp32, for |g| < 64, with the same values as
// __fdiv_rn(g, 1 + expf(-g)) after the bf16 rounding that follows it. The
// exponential is a Cody-Waite range reduction (Cody and Waite, 1980):
// exp(x) = 2^n 2^t with n = rint(x log2 e) and t the remainder, log2 e split
// into its fp32 value and the residual (constants fixed by the mathematics);
// no overflow or underflow handling is needed for |g| < 64. The quotient is
// q0 = g rcp(d) plus one residual correction. Every bf16 g with |g| < 64 takes
// this path in the exhaustive swiglu test, whose bf16 results are bitwise the
// oracle's.
__device__ __forceinline__ float silu_fast(float g) {
    constexpr float kNegLog2e = -0x1.715476p+0f;        // -log2(e), fp32
    constexpr float kNegLog2eLow = -0x1.4ae0bep-26f;    // -(log2(e) - 0x1.715476p+0)
    const float ph = g * kNegLog2e;
    const float n = __builtin_rintf(ph);
    float pl = __builtin_fmaf(g, kNegLog2e, -ph);
    pl = __builtin_fmaf(g, kNegLog2eLow, pl);
    const float e = __builtin_ldexpf(__builtin_amdgcn_exp2f((ph - n) + pl), static_cast<int>(n));
    const float d = 1.0f + e;
    const float y = __builtin_amdgcn_rcpf(d);
    const float q0 = g * y;
    // d >= 1 and the quotient never underflows to zero, so it has the sign of
    // g; the copy keeps g = -0 at -0 (the correction would add +0 to it).
    return __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q0, d, g), y, q0), g);
}

// out = bf16(up * bf16(g / (1 + exp(-g)))) (tools/h3_pointwise.py:18-22)
struct SwigluOp {
    static constexpr int kInputs = 2;
    static constexpr unsigned kStream = 0b11;  // up and gate both streamed
    static constexpr int kUnroll = 2;
    static constexpr bool kIndexable = false;
    __device__ static void apply(const float up[8], const float g[8], const float *, float o[8]) {
        bool fast = true;
#pragma unroll
        for (int e = 0; e < 8; ++e) fast = fast && __builtin_fabsf(g[e]) < 64.0f;
        float a[8];
        if (fast) {
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = silu_fast(g[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = __fdiv_rn(g[e], 1.0f + expf(-g[e]));
        }
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            rbf2(a[e], a[e + 1]);
            o[e] = up[e] * a[e];
            o[e + 1] = up[e + 1] * a[e + 1];
        }
    }
};

template <class Op, bool VEC, bool IDX, int TB>
__global__ __launch_bounds__(TB) void ew_kernel(EwArgs a) {
    const int64_t row = blockIdx.x / a.chunks;
    const int chunk = blockIdx.x % a.chunks;
    const int64_t b = row / a.S, s = row % a.S;
    const int W8 = (a.W + 7) / 8;
    int64_t mb = b, ms = s;
    if constexpr (IDX) mod_coords(a.index, b, s, mb, ms);
    const bf16_t *pa = row_ptr(a.a, b, s);
    const bf16_t *pb = row_ptr(a.b, mb, ms);
    const bf16_t *pc = Op::kInputs > 2 ? row_ptr(a.c, b, s) : nullptr;
    bf16_t *po = row_ptr_w(a.out, b, s);
    float va[Op::kUnroll][8], vb[Op::kUnroll][8], vc[Op::kUnroll][8];
    // Loads from clamped groups for every lane (see clamp_group); only the
    // stores are guarded.
#pragma unroll
    for (int u = 0; u < Op::kUnroll; ++u) {
        const int c0 = clamp_group(chunk * TB * Op::kUnroll + u * TB + threadIdx.x, W8) * 8;
        load8<VEC, (Op::kStream & 1) != 0>(pa, a.a.sw, c0, a.W, va[u]);
        load8<VEC, (Op::kStream & 2) != 0>(pb, a.b.sw, c0, a.W, vb[u]);
        if constexpr (Op::kInputs > 2) load8<VEC, (Op::kStream & 4) != 0>(pc, a.c.sw, c0, a.W, vc[u]);
    }
#pragma unroll
    for (int u = 0; u < Op::kUnroll; ++u) {
        const int g = chunk * TB * Op::kUnroll + u * TB + threadIdx.x;
        if (g < W8) {
            float o[8];
            Op::apply(va[u], vb[u], vc[u], o);
            store8<VEC, true>(po, a.out.sw, g * 8, a.W, o);
        }
    }
}

// Launches Op over [B, S, W] views. With `index` (int64 [B, S]), input 1 is a
// [R, W] table and token (b, s) reads its row index[b, s].
template <class Op>
int launch_ew(hipStream_t stream, const NineToothedTensor *in_t, const NineToothedTensor &out_t,
              const NineToothedTensor *index_t = nullptr) {
    View<3> in[Op::kInputs], out;
    if (!load_view(out_t, 2, out)) return kInvalid;
    bool vec = rows_vec16(out, 2);
    EwArgs a{};
    Rows rows[Op::kInputs];
    for (int i = 0; i < Op::kInputs; ++i) {
        if (i == 1 && index_t != nullptr) {
            View<2> table;
            View<2> ix;
            if (!load_view(in_t[i], 2, table) || table.shape[1] != out.shape[2]) return kInvalid;
            if (!load_view(*index_t, 8, ix) || ix.shape[0] != out.shape[0] || ix.shape[1] != out.shape[1])
                return kInvalid;
            if (table.shape[0] == 0 && out.numel() != 0) return kInvalid;  // no row for the tokens to take
            rows[i] = {table.data, table.stride[0], 0, table.stride[1]};
            vec = vec && rows_vec16(table, 2);
            a.index = {reinterpret_cast<const int64_t *>(ix.data), ix.stride[0], ix.stride[1], table.shape[0]};
            continue;
        }
        if (!load_view(in_t[i], 2, in[i]) || !same_shape(in[i], out)) return kInvalid;
        rows[i] = rows_of(in[i]);
        vec = vec && rows_vec16(in[i], 2);
    }
    a.a = rows[0];
    a.b = rows[1];
    a.c = Op::kInputs > 2 ? rows[Op::kInputs - 1] : a.a;
    a.out = rows_of(out);
    a.rows = out.shape[0] * out.shape[1];
    a.S = out.shape[1];
    a.W = static_cast<int>(out.shape[2]);
    if (a.rows == 0 || a.W == 0) return 0;
    const int W8 = (a.W + 7) / 8;
    // One group per thread (the gated residual): blocks of 128 threads where
    // they tile a row exactly and 256 do not (W = 7168: 7 blocks of 128 per
    // row instead of 4 of 256, the last half idle), measured 55.9 against
    // 59.6 us at [8192, 7168]. SwiGLU's two groups per thread keep 256
    // (128 measured 1.6% slower at W = 18432).
    const bool half = vec && Op::kUnroll == 1 && W8 % kThreads != 0 && W8 % (kThreads / 2) == 0;
    const int tb = half ? kThreads / 2 : kThreads;
    a.chunks = (W8 + tb * Op::kUnroll - 1) / (tb * Op::kUnroll);
    const int64_t grid = a.rows * a.chunks;
    if (grid > static_cast<int64_t>(std::numeric_limits<int32_t>::max())) return kInvalid;
    const unsigned g = static_cast<unsigned>(grid);
    if (index_t != nullptr) {
        if constexpr (Op::kIndexable) {
            if (half)
                ew_kernel<Op, true, true, kThreads / 2><<<g, kThreads / 2, 0, stream>>>(a);
            else if (vec)
                ew_kernel<Op, true, true, kThreads><<<g, kThreads, 0, stream>>>(a);
            else
                ew_kernel<Op, false, true, kThreads><<<g, kThreads, 0, stream>>>(a);
        } else {
            return kInvalid;
        }
    } else if (half) {
        ew_kernel<Op, true, false, kThreads / 2><<<g, kThreads / 2, 0, stream>>>(a);
    } else if (vec) {
        ew_kernel<Op, true, false, kThreads><<<g, kThreads, 0, stream>>>(a);
    } else {
        ew_kernel<Op, false, false, kThreads><<<g, kThreads, 0, stream>>>(a);
    }
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
    HeadRows x2, out2;  // a second tensor at the same (t, p, h) rows (q and k in one launch)
    const bf16_t *cos, *sin;
    int64_t cs0, cs1, ss0, ss1;  // element strides of the [T, n] cos and sin tables
    int64_t rows, P, Hs;
    FastDiv by_ph, by_h;  // row -> (t, p, h): divisions by P * Hs and by Hs
    const bf16_t *w;  // [128] RMS weight (norm kernels only)
    int64_t w_stride;
    const bf16_t *w2;  // the second tensor's weight
    int64_t w2_stride;
    float eps_bf;
};

enum RopeMode { kRopeOnly = 0, kNormRope = 1, kNormRopeInterleaved = 2 };

// i * stride in the 32-bit offset path: the host has checked that every
// index, stride and the divisors P * Hs and Hs are below 2^24 and every offset
// below 2^31 (offsets_fit_int32), so the full-rate 24-bit multiply is exact.
__device__ __forceinline__ uint32_t mul24(uint32_t i, int64_t stride) {
    return __umul24(i, static_cast<uint32_t>(stride));
}

// Element offset of head row (t, p, hh); OFF32: the 32-bit offset path above.
template <bool OFF32>
__device__ __forceinline__ int64_t head_offset(const HeadRows &h, uint32_t t, uint32_t p, uint32_t hh) {
    if constexpr (OFF32) {
        return static_cast<int64_t>(mul24(t, h.s0) + mul24(p, h.s1) + mul24(hh, h.s2));
    } else {
        return static_cast<int64_t>(t) * h.s0 + static_cast<int64_t>(p) * h.s1 + static_cast<int64_t>(hh) * h.s2;
    }
}

// Row r of the [T, P, Hs] row space -> (t, p, hh), r < 2^31; OFF32: the
// quotient-times-divisor products have 24-bit factors (checked on the host).
template <bool OFF32>
__device__ __forceinline__ void split_row(uint32_t r, const FastDiv &by_ph, const FastDiv &by_h, uint32_t &t,
                                          uint32_t &p, uint32_t &hh) {
    t = fast_div(r, by_ph);
    const uint32_t rem = r - (OFF32 ? __umul24(t, by_ph.d) : t * by_ph.d);
    p = fast_div(rem, by_h);
    hh = rem - (OFF32 ? __umul24(p, by_h.d) : p * by_h.d);
}

template <bool VEC>
__device__ __forceinline__ U4 load_head(const HeadRows &h, int64_t off, int lane) {
    return load_group<VEC, true>(reinterpret_cast<const bf16_t *>(h.p) + off, h.s3, lane * 8, 128);
}

template <bool VEC>
__device__ __forceinline__ void store_head(const HeadRows &h, int64_t off, int lane, const float f[8]) {
    store_group<VEC, true>(reinterpret_cast<bf16_t *>(h.p) + off, h.s3, lane * 8, 128, f8_to_u4(f));
}

// The cos/sin entries a lane needs for one row, loaded ahead of the arithmetic:
// rotate-half, 8 entries of [T, 48] at column (lane mod 6) * 8 (lanes 0-11);
// interleaved, 4 entries of [T, 64] at column 4 * lane (in c.x, c.y).
struct RopeTab {
    U4 c, s;
};

template <bool VEC, int MODE, bool OFF32>
__device__ __forceinline__ RopeTab load_tab(const RopeArgs &a, uint32_t t, int lane) {
    RopeTab tab{};
    const bf16_t *cr = a.cos + (OFF32 ? static_cast<int64_t>(mul24(t, a.cs0)) : static_cast<int64_t>(t) * a.cs0);
    const bf16_t *sr = a.sin + (OFF32 ? static_cast<int64_t>(mul24(t, a.ss0)) : static_cast<int64_t>(t) * a.ss0);
    if constexpr (MODE == kNormRopeInterleaved) {
        const int c0 = lane * 4;
        if constexpr (VEC) {
            const uint2 cv = *reinterpret_cast<const uint2 *>(cr + c0);
            const uint2 sv = *reinterpret_cast<const uint2 *>(sr + c0);
            tab.c = {cv.x, cv.y, 0u, 0u};
            tab.s = {sv.x, sv.y, 0u, 0u};
        } else {
            tab.c.x = cr[c0 * a.cs1] | (static_cast<uint32_t>(cr[(c0 + 1) * a.cs1]) << 16);
            tab.c.y = cr[(c0 + 2) * a.cs1] | (static_cast<uint32_t>(cr[(c0 + 3) * a.cs1]) << 16);
            tab.s.x = sr[c0 * a.ss1] | (static_cast<uint32_t>(sr[(c0 + 1) * a.ss1]) << 16);
            tab.s.y = sr[(c0 + 2) * a.ss1] | (static_cast<uint32_t>(sr[(c0 + 3) * a.ss1]) << 16);
        }
    } else {
        // Lanes 12-15 (pass-through channels) load a column they do not use,
        // so that no load sits under a per-lane branch.
        const int c0 = (lane < 6 ? lane : (lane < 12 ? lane - 6 : 0)) * 8;
        tab.c = load_group<VEC>(cr, a.cs1, c0, 48);
        tab.s = load_group<VEC>(sr, a.ss1, c0, 48);
    }
    return tab;
}

// The reciprocal of a head row, bf16(1 / sqrt(var)) with IEEE sqrt and
// division, for a var that is itself a bf16 value: with var = 1.m x 2^(2k + p),
// sqrt and 1/x commute exactly with the power-of-two scaling (normal range), so
// the result is T[p][m] x 2^-k where T holds the 256 values for p = 0, 1 and the
// 7-bit mantissa m. The block builds T in LDS with the IEEE sequence itself;
// zero, subnormal, infinite and NaN var take that sequence directly.
constexpr int kRsqrtTable = 256;

__device__ __forceinline__ void build_rsqrt_table(bf16_t *tab) {
    for (int i = threadIdx.x; i < kRsqrtTable; i += blockDim.x) {
        const float var = __uint_as_float((static_cast<uint32_t>(127 + (i >> 7)) << 23) | (static_cast<uint32_t>(i & 127) << 16));
        tab[i] = static_cast<bf16_t>(__float_as_uint(rbf(rsqrt_ieee(var))) >> 16);
    }
}

__device__ __forceinline__ float rsqrt_bf16(float var, const bf16_t *tab) {
    const uint32_t b = __float_as_uint(var);
    const int e = static_cast<int>((b >> 23) & 255u);
    if (e == 0 || e == 255) return rbf(rsqrt_ieee(var));
    const int ee = e - 127, p = ee & 1;
    return __builtin_ldexpf(bf2f(tab[(p << 7) | ((b >> 16) & 127u)]), -((ee - p) >> 1));
}

// RMSNorm over the 128 channels held by a 16-lane row group (the same fixed
// order as the rms family at W = 128), then weight: returns bf16 values in f.
// `tab`: the block's reciprocal table (build_rsqrt_table), or null for the IEEE
// sequence in every lane.
__device__ __forceinline__ void head_rms(float f[8], const float w[8], float eps_bf, const bf16_t *tab = nullptr) {
    float partial = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        float q0 = f[e] * f[e], q1 = f[e + 1] * f[e + 1];
        rbf2(q0, q1);
        partial += q0;
        partial += q1;
    }
    float r;
    if (tab != nullptr) {
        const float mean = rbf(fold_lanes<16>(partial) * 0.0078125f);  // bf16(sum / 128): exact scaling
        r = rsqrt_bf16(rbf(mean + eps_bf), tab);
    } else {
        r = rms_reciprocal(fold_lanes<16>(partial), 128, eps_bf);
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
__device__ __forceinline__ void rope_rotate_half(float f[8], int lane, const RopeTab &tab) {
    float partner[8];
    const int src = lane < 6 ? lane + 6 : (lane < 12 ? lane - 6 : lane);
#pragma unroll
    for (int e = 0; e < 8; ++e) partner[e] = __shfl(f[e], src, 16);
    if (lane >= 12) return;
    float c[8], s[8];
    u4_to_f8(tab.c, c);
    u4_to_f8(tab.s, s);
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
__device__ __forceinline__ void rope_interleaved(float f[8], const RopeTab &tab) {
    const float c[4] = {lo2f(tab.c.x), hi2f(tab.c.x), lo2f(tab.c.y), hi2f(tab.c.y)};
    const float s[4] = {lo2f(tab.s.x), hi2f(tab.s.x), lo2f(tab.s.y), hi2f(tab.s.y)};
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

// R rows per 16-lane group: every row's x and table loads are issued before
// the arithmetic of the first.
template <bool VEC, int MODE, int R, bool OFF32>
__global__ __launch_bounds__(kThreads) void head_rows_kernel(RopeArgs a) {
    constexpr int kGroups = kThreads / 16;
    const int lane = threadIdx.x & 15;
    const uint32_t base = blockIdx.x * kGroups * R + (threadIdx.x >> 4);  // rows < 2^31 (host check)
    bool ok[R];
    int64_t out_off[R];
    U4 xv[R];
    RopeTab tab[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = base + r * kGroups;
        ok[r] = row < a.rows;
        uint32_t t, p, hh;
        split_row<OFF32>(ok[r] ? row : 0u, a.by_ph, a.by_h, t, p, hh);
        out_off[r] = head_offset<OFF32>(a.out, t, p, hh);
        xv[r] = load_head<VEC>(a.x, head_offset<OFF32>(a.x, t, p, hh), lane);
        tab[r] = load_tab<VEC, MODE, OFF32>(a, t, lane);
    }
    float w[8];
    if constexpr (MODE != kRopeOnly) u4_to_f8(load_group<VEC>(a.w, a.w_stride, lane * 8, 128), w);
    __shared__ bf16_t rs_tab[kRsqrtTable];
    if constexpr (MODE != kRopeOnly) {
        build_rsqrt_table(rs_tab);  // while the rows are in flight
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float f[8];
        u4_to_f8(xv[r], f);
        if constexpr (MODE != kRopeOnly) head_rms(f, w, a.eps_bf, rs_tab);
        if constexpr (MODE == kNormRopeInterleaved) {
            rope_interleaved(f, tab[r]);
        } else {
            rope_rotate_half(f, lane, tab[r]);
        }
        if (ok[r]) store_head<VEC>(a.out, out_off[r], lane, f);
    }
}

// The rows of head_rows_kernel walked in batches of R rows per 16-lane group,
// grid-strided, the next batch's x and table loads issued before the current
// batch's arithmetic (two register sets used in turn; the loop condition is
// uniform over the block, so no load sits under a per-lane branch). NT = 2:
// the group also takes the row at the same (t, p, h) of the second tensor
// (x2 -> out2, weight w2) against the same table entries.
template <bool VEC, int MODE, int R, bool OFF32, int NT = 1>
__global__ __launch_bounds__(kThreads) void head_rows_loop_kernel(RopeArgs a) {
    static_assert(NT == 1 || NT == 2, "one or two tensors");
    constexpr int kGroups = kThreads / 16;
    const int lane = threadIdx.x & 15;
    const uint32_t stride = gridDim.x * kGroups * R;
    const uint32_t group = threadIdx.x >> 4;
    struct Batch {
        bool ok[R];
        int64_t out_off[R][NT];
        U4 xv[R][NT];
        RopeTab tab[R];
    };
    auto load = [&](uint32_t block_base, Batch &bt) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = block_base + group + r * kGroups;
            bt.ok[r] = row < a.rows;
            uint32_t t, p, hh;
            split_row<OFF32>(bt.ok[r] ? row : 0u, a.by_ph, a.by_h, t, p, hh);
            bt.out_off[r][0] = head_offset<OFF32>(a.out, t, p, hh);
            bt.xv[r][0] = load_head<VEC>(a.x, head_offset<OFF32>(a.x, t, p, hh), lane);
            if constexpr (NT == 2) {
                bt.out_off[r][NT - 1] = head_offset<OFF32>(a.out2, t, p, hh);
                bt.xv[r][NT - 1] = load_head<VEC>(a.x2, head_offset<OFF32>(a.x2, t, p, hh), lane);
            }
            bt.tab[r] = load_tab<VEC, MODE, OFF32>(a, t, lane);
        }
    };
    float w[NT][8];
    if constexpr (MODE != kRopeOnly) {
        u4_to_f8(load_group<VEC>(a.w, a.w_stride, lane * 8, 128), w[0]);
        if constexpr (NT == 2) u4_to_f8(load_group<VEC>(a.w2, a.w2_stride, lane * 8, 128), w[NT - 1]);
    }
    __shared__ bf16_t rs_tab[kRsqrtTable];
    auto finish = [&](Batch &bt) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                float f[8];
                u4_to_f8(bt.xv[r][n], f);
                if constexpr (MODE != kRopeOnly) head_rms(f, w[n], a.eps_bf, rs_tab);
                if constexpr (MODE == kNormRopeInterleaved) {
                    rope_interleaved(f, bt.tab[r]);
                } else {
                    rope_rotate_half(f, lane, bt.tab[r]);
                }
                if (bt.ok[r]) store_head<VEC>(n == 0 ? a.out : a.out2, bt.out_off[r][n], lane, f);
            }
    };
    Batch A, B;
    uint32_t base = blockIdx.x * kGroups * R;
    load(base, A);
    if constexpr (MODE != kRopeOnly) {
        build_rsqrt_table(rs_tab);  // while the first batch is in flight
        __syncthreads();
    }
    while (true) {
        load(base + stride, B);
        finish(A);
        base += stride;
        if (base >= a.rows) break;
        load(base + stride, A);
        finish(B);
        base += stride;
        if (base >= a.rows) break;
    }
}

// Launch shape of head_rows_loop_kernel (the 16-byte, 32-bit-offset case):
// blocks, and rows per 16-lane group per batch. Measured on [8192, 1, 14, 128]
// against one batch per block: 14.8 against 16.3 us (rotate-half), 13.6
// against 14.2 us (interleaved); 4096 blocks against 2048: 24.1-25.0 against
// 25.6-27.8 us for q and k in one launch, 13.8-14.1 against 13.9-14.5 us
// (interleaved) and 14.4-15.0 against 15.1-16.3 us (rotate-half) per tensor.
constexpr int kHeadLoopBlocks = 4096;
constexpr int kHeadLoopRows = 1;

// x2 / out2 / w2 (optional, all or none): a second tensor of x's shape taken
// in the same launch (one pass over both when the rows are 16-byte aligned and
// the offsets fit 32 bits; otherwise one launch per tensor).
template <int MODE>
int launch_head_rows(hipStream_t stream, const View<4> &x, const View<4> &out, const View<2> &cos,
                     const View<2> &sin, const View<1> *w, double eps, const View<4> *x2 = nullptr,
                     const View<4> *out2 = nullptr, const View<1> *w2 = nullptr) {
    const int64_t table_width = MODE == kNormRopeInterleaved ? 64 : 48;
    if (!same_shape(x, out) || x.shape[3] != 128) return kInvalid;
    if (cos.shape[0] != x.shape[0] || cos.shape[1] != table_width || !same_shape(cos, sin)) return kInvalid;
    if (w != nullptr && w->shape[0] != 128) return kInvalid;
    const bool pair = x2 != nullptr;
    if (pair && (out2 == nullptr || (w == nullptr) != (w2 == nullptr) || !same_shape(*x2, x) ||
                 !same_shape(*out2, x) || (w2 != nullptr && w2->shape[0] != 128)))
        return kInvalid;
    bool vec = rows_vec16(x, 2) && rows_vec16(out, 2) && rows_vec16(cos, 2) && rows_vec16(sin, 2);
    if (w != nullptr) vec = vec && rows_vec16(*w, 2);
    if (pair) {
        const bool vec2 = vec && rows_vec16(*x2, 2) && rows_vec16(*out2, 2) && (w2 == nullptr || rows_vec16(*w2, 2));
        const bool off2 = offsets_fit_int32(x) && offsets_fit_int32(out) && offsets_fit_int32(*x2) &&
                          offsets_fit_int32(*out2) && offsets_fit_int32(cos) && offsets_fit_int32(sin) &&
                          x.shape[1] * x.shape[2] < (int64_t{1} << 24);
        if (!(vec2 && off2 && kHeadLoopBlocks > 0)) {
            const int st = launch_head_rows<MODE>(stream, x, out, cos, sin, w, eps);
            return st != 0 ? st : launch_head_rows<MODE>(stream, *x2, *out2, cos, sin, w2, eps);
        }
    }
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
    if (a.rows >= (int64_t{1} << 31) - kThreads * 4) return kInvalid;
    a.by_ph = make_fastdiv(static_cast<uint32_t>(a.P * a.Hs > 0 ? a.P * a.Hs : 1));
    a.by_h = make_fastdiv(static_cast<uint32_t>(a.Hs > 0 ? a.Hs : 1));
    const bool off32 = offsets_fit_int32(x) && offsets_fit_int32(out) && offsets_fit_int32(cos) &&
                       offsets_fit_int32(sin) && a.P * a.Hs < (int64_t{1} << 24);
    if (w != nullptr) {
        a.w = reinterpret_cast<const bf16_t *>(w->data);
        a.w_stride = w->stride[0];
    }
    if (pair) {
        a.x2 = {x2->data, x2->stride[0], x2->stride[1], x2->stride[2], x2->stride[3]};
        a.out2 = {out2->data, out2->stride[0], out2->stride[1], out2->stride[2], out2->stride[3]};
        if (w2 != nullptr) {
            a.w2 = reinterpret_cast<const bf16_t *>(w2->data);
            a.w2_stride = w2->stride[0];
        }
    }
    a.eps_bf = host_round_bf16(eps);
    if (a.rows == 0) return 0;
    // Four rows per lane group when that still leaves >= 1024 blocks.
    constexpr int64_t kPerBlock = kThreads / 16;
    const bool four = (a.rows + 4 * kPerBlock - 1) / (4 * kPerBlock) >= 1024;
    const int64_t per_block = four ? 4 * kPerBlock : kPerBlock;
    const int64_t grid = (a.rows + per_block - 1) / per_block;
    if (grid > static_cast<int64_t>(std::numeric_limits<int32_t>::max())) return kInvalid;
    const unsigned g = static_cast<unsigned>(grid);
    if (kHeadLoopBlocks > 0 && vec && off32) {
        constexpr int64_t kBatch = kPerBlock * kHeadLoopRows;
        const int64_t needed = (a.rows + kBatch - 1) / kBatch;
        const unsigned gl = static_cast<unsigned>(needed < kHeadLoopBlocks ? needed : kHeadLoopBlocks);
        if (pair)
            head_rows_loop_kernel<true, MODE, kHeadLoopRows, true, 2><<<gl, kThreads, 0, stream>>>(a);
        else
            head_rows_loop_kernel<true, MODE, kHeadLoopRows, true><<<gl, kThreads, 0, stream>>>(a);
        return launch_status();
    }
#define H3_HEAD_ROWS(V, R, O) \
    if (vec == V && (four ? 4 : 1) == R && off32 == O) head_rows_kernel<V, MODE, R, O><<<g, kThreads, 0, stream>>>(a);
    H3_HEAD_ROWS(true, 4, true) H3_HEAD_ROWS(true, 1, true) H3_HEAD_ROWS(true, 4, false)
    H3_HEAD_ROWS(true, 1, false) H3_HEAD_ROWS(false, 4, true) H3_HEAD_ROWS(false, 1, true)
    H3_HEAD_ROWS(false, 4, false) H3_HEAD_ROWS(false, 1, false)
#undef H3_HEAD_ROWS
    return launch_status();
}

// ============================================================ q/k/v send pack

// One launch over the q, k and v head rows of a head group as InfiniLM's
// sequence-parallel attention produces them (patches/InfiniLM.patch:1071-1110):
// q and k get the per-head RMSNorm + rotate-half RoPE of head_rows_kernel, with
// the cos/sin rows gathered from the RoPE cache through the token positions
// (the gather_rows of :1077-1080, fused), and v is copied; every input and
// output is a [T, P, Hs, 128] view with any strides (the by-rank views of the
// fused projection, :1093-1097, and the permuted send buffers, :1100-1102).
struct QkvArgs {
    HeadRows q, k, v, q_out, k_out, v_out;
    const bf16_t *wq, *wk;
    int64_t wq_stride, wk_stride;
    const bf16_t *cos, *sin;
    int64_t cs0, cs1, ss0, ss1;
    const int64_t *pos;
    int64_t pos_stride, table_rows;
    int64_t rows, P, Hs;  // rows = T * P * Hs per tensor
    FastDiv by_ph, by_h;
    float eps_bf;
    float *q_descale, *k_descale;  // FP8: fp32 [P * Hs] each
    uint32_t *v_amax;              // VAMAX: [P * Hs, H3_AMAX_SLOTS] |v| maxima as fp32 bits
    char *q_out_lo, *k_out_lo;     // TWO: the lo codes, with q_out's / k_out's strides
    bool v_pinned;                 // VAMAX: v blocks pinned to heads, at most H3_AMAX_SLOTS per head
};

// The fp8 epilogue's scale. An RMSNorm'd 128-vector n has sum(n^2) = 128, so
// every element and every rotated pair (a, b) has |.| <= sqrt(128); the
// weight scales that by at most max|w| and the RoPE rotation preserves pair
// norms. The bf16 roundings on the way (reciprocal, normalized, weighted, the
// two products and the sum) add at most about 9 half-ulps of 2^-8, under 2%:
// |y| <= sqrt(128) * 1.03125 * max|w| =: bound for every output. Codes are
// e4m3(bf16(y) * 448 / bound) with saturation at +-448 as a guard; descale =
// bound / 448 for every head.
constexpr float kQkFp8BoundPerWeight = 11.667261889577f;  // fp32(sqrt(128) * 1.03125)
constexpr float kE4M3Max = 448.0f;

// The scaled values of eight outputs (already bf16): y = sat((f * pre) * inv),
// the scale of e4m3_code_scale. pre is 1 except for a bound below about
// 1.3e-36, and f * 1 = f exactly, so a launch with pre = 1 (every block of it
// the same) skips that product. sat() is applied only when some |y| exceeds
// 448 (a cos/sin table that is not a rotation can exceed the weight bound);
// otherwise it changes nothing: values within +-448 are kept, and a NaN --
// which fmaxf passes over -- stays NaN either way.
__device__ __forceinline__ void e4m3_scaled8(const float f[8], float pre, float inv, float y[8]) {
    if (pre == 1.0f) {
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = f[e] * inv;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = (f[e] * pre) * inv;
    }
    float m = fabsf(y[0]);
#pragma unroll
    for (int e = 1; e < 8; ++e) m = fmaxf(m, fabsf(y[e]));
    if (m > 448.0f) {
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = sat_e4m3(y[e]);
    }
}

// Eight scaled values (e4m3_scaled8) as e4m3fn codes.
__device__ __forceinline__ uint2 e4m3x8(const float y[8]) {
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], lo, true);
    int hi = __builtin_amdgcn_cvt_pk_fp8_f32(y[4], y[5], 0, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(y[6], y[7], hi, true);
    return make_uint2(static_cast<uint32_t>(lo), static_cast<uint32_t>(hi));
}

// The lo term of the two-term split of eight scaled values y with codes hi =
// e4m3x8(y): e4m3(16 (y - hi)). y - hi is exact in fp32 (hi is y rounded to 4
// significant bits, or 0) and |16 (y - hi)| <= 256, so the saturation of the
// quantiser's formula, e4m3(sat(16 (y - hi))), never acts and is left out.
// 16 hi comes straight from the scaled conversion (v_cvt_scalef32_pk_f32_fp8
// with scale 16 equals the plain conversion times 16 for all 65,536 code
// pairs, measured on the hardware), and 16 (y - hi) = fma(y, 16, -16 hi): the
// exact value is representable, so the one rounding of the fma leaves it.
constexpr float kLoTermShift = 16.0f;
__device__ __forceinline__ uint2 e4m3x8_lo(const float y[8], uint2 hi) {
    float r[8];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int w = static_cast<int>(half == 0 ? hi.x : hi.y);
        const f32x2_t h01 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, kLoTermShift, false);
        const f32x2_t h23 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, kLoTermShift, true);
        const float h16[4] = {h01[0], h01[1], h23[0], h23[1]};
#pragma unroll
        for (int e = 0; e < 4; ++e) r[4 * half + e] = __builtin_fmaf(y[4 * half + e], kLoTermShift, -h16[e]);
    }
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(r[0], r[1], 0, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(r[2], r[3], lo, true);
    int hi2 = __builtin_amdgcn_cvt_pk_fp8_f32(r[4], r[5], 0, false);
    hi2 = __builtin_amdgcn_cvt_pk_fp8_f32(r[6], r[7], hi2, true);
    return make_uint2(static_cast<uint32_t>(lo), static_cast<uint32_t>(hi2));
}

__device__ __forceinline__ HeadRows pick3(int kind, const HeadRows &a, const HeadRows &b, const HeadRows &c) {
    // Field by field, so that the choice stays in scalar registers.
    return {kind == 0 ? a.p : (kind == 1 ? b.p : c.p), kind == 0 ? a.s0 : (kind == 1 ? b.s0 : c.s0),
            kind == 0 ? a.s1 : (kind == 1 ? b.s1 : c.s1), kind == 0 ? a.s2 : (kind == 1 ? b.s2 : c.s2),
            kind == 0 ? a.s3 : (kind == 1 ? b.s3 : c.s3)};
}

// The v blocks' per-head maximum of |v| (VAMAX): each block folds its rows'
// |v| into an LDS maximum per head, then into slot (block % H3_AMAX_SLOTS) of
// the head with one atomic max per head, so about blocks / H3_AMAX_SLOTS
// atomics meet at any one address. The head's amax is the maximum over its
// slots. Maxima are compared as the bits of |v| (ordered like the values for
// non-NaN bf16). Heads per launch are limited to what the LDS array holds.
constexpr int kVamaxHeads = 1024;
static_assert(kVamaxHeads == H3_NOALLOC_MAX_HEADS, "the no-alloc slot array holds the LDS fold's heads");

// Block b handles tensor b % 3 (0 q, 1 k, 2 v): batches of R rows per 16-lane
// group, the batches of that tensor grid-strided over the blocks of its kind,
// the next batch's loads issued before the current batch's arithmetic (two
// register sets used in turn; the loop condition is uniform over the block).
// Every load (x, position, table, weight) is issued for every block kind from
// valid addresses; the kind only selects the arithmetic.
// FP8: q and k leave as e4m3 codes (uint8 outputs, 8 codes per lane) scaled
// by the weight bound above; v stays a bf16 copy.
// TWO (FP8 only): q and k also leave their lo codes (two-term split) at the
// same offsets of q_out_lo / k_out_lo.
// PIN (VAMAX only): the launch pins its v blocks to heads (v_pinned), so the
// q/k loop below carries none of the v blocks' maximum bookkeeping: 78
// VGPRs instead of 93 for the two-term pack, 6 waves per SIMD instead of 5
// (46.2 -> 43.3 us at [8192, 1, 14, 128]).
template <bool VEC, int R, bool OFF32, bool FP8, bool VAMAX = false, bool TWO = false, bool PIN = false>
__global__ __launch_bounds__(kThreads) void qkv_pack_kernel(QkvArgs a) {
    static_assert(!TWO || FP8, "the two-term split is of the fp8 codes");
    static_assert(!PIN || VAMAX, "pinning is of the v blocks' maximum");
    constexpr bool kLoopAmax = VAMAX && !PIN;  // the v maxima folded in the loop below
    constexpr int kGroups = kThreads / 16;
    const int kind = static_cast<int>(blockIdx.x % 3);
    const uint32_t tile0 = blockIdx.x / 3, tiles = gridDim.x / 3;  // gridDim.x is a multiple of 3
    const int lane = threadIdx.x & 15;
    const uint32_t group = threadIdx.x >> 4;
    const HeadRows in = pick3(kind, a.q, a.k, a.v), out = pick3(kind, a.q_out, a.k_out, a.v_out);
    if constexpr (VAMAX) {
        // V blocks pinned to heads (v_pinned: at least one v block per head):
        // v block j copies the rows of head hp = j % (P Hs) only, the head's
        // 16-row batches grid-strided over its n blocks (n <= H3_AMAX_SLOTS),
        // so every lane keeps one running maximum of |v| in a register. The block folds it once at the end and stores it, as the
        // k-th block of its head (k = j / (P Hs) < n), into slot k of the head,
        // and zeros into slots k + n, k + 2n, ...: every slot of every head
        // has exactly one writer, so the slots need no clearing and no atomics.
        // The pinned blocks of all heads run together, so the reads still
        // cover whole token rows at any moment.
        const uint32_t heads = static_cast<uint32_t>(a.P * a.Hs);
        if (kind == 2 && (PIN || a.v_pinned)) {
            const uint32_t hp = tile0 % heads, first = tile0 / heads;
            // The head's v blocks: those of index j = hp + k (P Hs), at most
            // H3_AMAX_SLOTS of them (the others have no rows).
            const uint32_t all = (tiles - hp + heads - 1) / heads;
            const uint32_t step = all < H3_AMAX_SLOTS ? all : H3_AMAX_SLOTS;
            if (first >= step) return;
            const uint32_t T = static_cast<uint32_t>(a.rows / heads);
            const uint32_t pp = hp / static_cast<uint32_t>(a.Hs), hh = hp - pp * static_cast<uint32_t>(a.Hs);
            constexpr uint32_t kBatch = kGroups * R;
            const uint32_t nb = (T + kBatch - 1) / kBatch;
            struct VBatch {
                bool ok[R];
                int64_t out_off[R];
                U4 xv[R];
            };
            // A row past the head's end re-reads its last token (the head's own
            // values, so the maximum stays exact) and is not stored.
            auto vload = [&](uint32_t i, VBatch &bt) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint32_t t = i * kBatch + group + r * kGroups;
                    bt.ok[r] = t < T;
                    const uint32_t tc = t < T ? t : T - 1;
                    bt.out_off[r] = head_offset<OFF32>(out, tc, pp, hh);
                    bt.xv[r] = load_head<VEC>(in, head_offset<OFF32>(in, tc, pp, hh), lane);
                }
            };
            uint32_t vm = 0;
            auto vfinish = [&](VBatch &bt) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    if (bt.ok[r])
                        store_group<VEC, true>(reinterpret_cast<bf16_t *>(out.p) + bt.out_off[r], out.s3, lane * 8,
                                               128, bt.xv[r]);
                    const uint32_t w[4] = {bt.xv[r].x, bt.xv[r].y, bt.xv[r].z, bt.xv[r].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t lo = (w[e] << 16) & 0x7fffffffu, hi = w[e] & 0x7fff0000u;
                        vm = lo > vm ? lo : vm;
                        vm = hi > vm ? hi : vm;
                    }
                }
            };
            if (first < nb) {
                VBatch A, B;
                uint32_t i = first;
                vload(i, A);
                while (true) {
                    vload(i + step < nb ? i + step : i, B);
                    vfinish(A);
                    i += step;
                    if (i >= nb) break;
                    vload(i + step < nb ? i + step : i, A);
                    vfinish(B);
                    i += step;
                    if (i >= nb) break;
                }
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                const uint32_t o = __shfl_xor(vm, off, 64);
                vm = o > vm ? o : vm;
            }
            __shared__ uint32_t wave_vm[kThreads / 64];
            if ((threadIdx.x & 63) == 0) wave_vm[threadIdx.x >> 6] = vm;
            __syncthreads();
            uint32_t m = wave_vm[0];
#pragma unroll
            for (int w2 = 1; w2 < kThreads / 64; ++w2) m = wave_vm[w2] > m ? wave_vm[w2] : m;
            uint32_t *slots = a.v_amax + static_cast<uint64_t>(hp) * H3_AMAX_SLOTS;
            for (uint32_t j = first + threadIdx.x * step; j < H3_AMAX_SLOTS; j += kThreads * step)
                slots[j] = j == first ? m : 0u;
            return;
        }
    }
    RopeArgs ta{};
    ta.cos = a.cos;
    ta.sin = a.sin;
    ta.cs0 = a.cs0;
    ta.cs1 = a.cs1;
    ta.ss0 = a.ss0;
    ta.ss1 = a.ss1;
    struct Batch {
        bool ok[R];
        int64_t out_off[R];
        U4 xv[R];
        RopeTab tab[R];
        uint32_t head[R];  // VAMAX: p * Hs + h
    };
    auto load = [&](uint32_t tile, Batch &bt) {
        uint32_t t[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = tile * kGroups * R + group + r * kGroups;
            bt.ok[r] = row < a.rows;
            uint32_t p, hh;
            split_row<OFF32>(bt.ok[r] ? row : 0u, a.by_ph, a.by_h, t[r], p, hh);
            if constexpr (kLoopAmax) bt.head[r] = p * static_cast<uint32_t>(a.Hs) + hh;
            bt.out_off[r] = head_offset<OFF32>(out, t[r], p, hh);
            bt.xv[r] = load_head<VEC>(in, head_offset<OFF32>(in, t[r], p, hh), lane);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t m = a.pos[OFF32 ? static_cast<int64_t>(mul24(t[r], a.pos_stride))
                                           : static_cast<int64_t>(t[r]) * a.pos_stride];
            const uint32_t row = static_cast<uint32_t>(m < 0 ? 0 : (m < a.table_rows ? m : a.table_rows - 1));
            bt.tab[r] = load_tab<VEC, kNormRope, OFF32>(ta, row, lane);
        }
    };
    float w[8];
    u4_to_f8(load_group<VEC>(kind == 0 ? a.wq : a.wk, kind == 0 ? a.wq_stride : a.wk_stride, lane * 8, 128), w);
    __shared__ bf16_t rs_tab[kRsqrtTable];
    float pre = 1.0f, inv = 0.0f;
    if constexpr (FP8) {
        float mw = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) mw = fmaxf(mw, fabsf(w[e]));
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) mw = fmaxf(mw, __shfl_xor(mw, off, 16));
        const float bound = kQkFp8BoundPerWeight * mw;
        e4m3_code_scale(bound, pre, inv);
        if (kind < 2 && tile0 == 0) {  // the first block of q and of k writes the descales
            float *descale = kind == 0 ? a.q_descale : a.k_descale;
            for (int64_t h = threadIdx.x; h < a.P * a.Hs; h += kThreads)
                descale[h] = bound > 0.0f ? bound / kE4M3Max : 1.0f;
        }
    }
    __shared__ uint32_t vmax[kLoopAmax ? kVamaxHeads : 1];
    auto finish = [&](Batch &bt) {
        if (kind == 2) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (bt.ok[r])
                    store_group<VEC, true>(reinterpret_cast<bf16_t *>(out.p) + bt.out_off[r], out.s3, lane * 8, 128,
                                           bt.xv[r]);
                if constexpr (kLoopAmax) {
                    // A row past the end re-read row 0 (head 0's): its values
                    // are head 0's, so the maximum stays exact.
                    const uint32_t w[4] = {bt.xv[r].x, bt.xv[r].y, bt.xv[r].z, bt.xv[r].w};
                    uint32_t m = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t lo = (w[e] << 16) & 0x7fffffffu, hi = w[e] & 0x7fff0000u;
                        m = lo > m ? lo : m;
                        m = hi > m ? hi : m;
                    }
#pragma unroll
                    for (int off = 8; off >= 1; off >>= 1) {
                        const uint32_t o = __shfl_xor(m, off, 16);
                        m = o > m ? o : m;
                    }
                    if (lane == 0) atomicMax(&vmax[bt.head[r]], m);
                }
            }
            return;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float f[8];
            u4_to_f8(bt.xv[r], f);
            head_rms(f, w, a.eps_bf, rs_tab);
            rope_rotate_half(f, lane, bt.tab[r]);
            if constexpr (FP8) {
#pragma unroll
                for (int e = 0; e < 8; e += 2) rbf2(f[e], f[e + 1]);  // the bf16 output, then its codes
                float y[8];
                e4m3_scaled8(f, pre, inv, y);
                const uint2 codes = e4m3x8(y);
                uint2 lo_codes = {0u, 0u};
                if constexpr (TWO) lo_codes = e4m3x8_lo(y, codes);
                if (bt.ok[r]) {
#pragma unroll
                    for (int term = 0; term < (TWO ? 2 : 1); ++term) {
                        const uint2 cw = term == 0 ? codes : lo_codes;
                        uint8_t *row = reinterpret_cast<uint8_t *>(
                                           term == 0 ? out.p : (kind == 0 ? a.q_out_lo : a.k_out_lo)) +
                                       bt.out_off[r];
                        if constexpr (VEC) {
                            // Streamed like the bf16 rows: a non-temporal 8-byte store.
                            typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
                            const u32x2_t cv = {cw.x, cw.y};
                            __builtin_nontemporal_store(cv, reinterpret_cast<u32x2_t *>(row + lane * 8));
                        } else {
#pragma unroll
                            for (int e = 0; e < 8; ++e)
                                row[(lane * 8 + e) * out.s3] =
                                    static_cast<uint8_t>((e < 4 ? cw.x : cw.y) >> (8 * (e & 3)));
                        }
                    }
                }
            } else {
                if (bt.ok[r]) store_head<VEC>(out, bt.out_off[r], lane, f);
            }
        }
    };
    const uint32_t batches = static_cast<uint32_t>((a.rows + kGroups * R - 1) / (kGroups * R));
    const uint32_t heads = static_cast<uint32_t>(a.P * a.Hs);
    Batch A, B;
    uint32_t tile = tile0;
    load(tile, A);
    if (kind < 2) {  // uniform over the block: q and k blocks normalise
        build_rsqrt_table(rs_tab);  // while the first batch is in flight
        __syncthreads();
    } else if constexpr (kLoopAmax) {
        for (uint32_t h = threadIdx.x; h < heads; h += kThreads) vmax[h] = 0u;
        __syncthreads();
    }
    while (true) {
        load(tile + tiles, B);
        finish(A);
        tile += tiles;
        if (tile >= batches) break;
        load(tile + tiles, A);
        finish(B);
        tile += tiles;
        if (tile >= batches) break;
    }
    if constexpr (kLoopAmax) {
        if (kind == 2) {
            __syncthreads();
            uint32_t *slots = a.v_amax + tile0 % H3_AMAX_SLOTS;
            for (uint32_t h = threadIdx.x; h < heads; h += kThreads) {
                const uint32_t m = vmax[h];
                if (m != 0u) atomicMax(slots + static_cast<uint64_t>(h) * H3_AMAX_SLOTS, m);
            }
        }
    }
}

// Clears n 32-bit words (a fill kernel rather than a memset, so that a
// captured graph replays it like any other node).
__global__ void clear_words_kernel(uint32_t *p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// Launch shape of qkv_pack_kernel: blocks per tensor and rows per 16-lane
// group per batch. Measured on [8192, 1, 14, 128]: 38.8 us, against 40.3
// (1024 blocks), 40.5 (4096) and 45-50 (one batch per block, 1-4 rows).
constexpr int64_t kQkvBlocks = 2048;
constexpr int kQkvRows = 1;

// fp8 (q_descale, k_descale non-null): out[0] and out[1] are uint8 e4m3 code
// views, the descales fp32 [P * Hs] (contiguous). v_amax (fp8 only, may be
// null): the [P * Hs, H3_AMAX_SLOTS] slots of V's per-head maxima, cleared
// here and then filled by the v blocks. check_only: the checks alone (0 or
// kInvalid), no HIP call.
// out_lo (fp8 only, may be null): the q and k lo codes of the two-term
// split, each with its hi output's shape and strides.
int launch_qkv_pack(hipStream_t stream, const View<4> *in, const View<4> *out, const View<1> &wq,
                    const View<1> &wk, double eps, const View<2> &cos, const View<2> &sin,
                    const View<1> &pos, const View<1> *q_descale = nullptr, const View<1> *k_descale = nullptr,
                    const View<2> *v_amax = nullptr, bool check_only = false, const View<4> *out_lo = nullptr) {
    const bool fp8 = q_descale != nullptr;
    const bool vamax = v_amax != nullptr;
    const bool two = out_lo != nullptr;
    if (two) {
        if (!fp8 || !vamax) return kInvalid;  // built with the V-amax fold only
        for (int i = 0; i < 2; ++i) {
            if (!same_shape(out_lo[i], out[i])) return kInvalid;
            for (int d = 0; d < 4; ++d)
                if (out[i].shape[d] > 1 && out_lo[i].stride[d] != out[i].stride[d]) return kInvalid;
            if ((reinterpret_cast<uintptr_t>(out_lo[i].data) & 7) != (reinterpret_cast<uintptr_t>(out[i].data) & 7))
                return kInvalid;
        }
    }
    for (int i = 0; i < 3; ++i)
        if (!same_shape(in[i], in[0]) || !same_shape(out[i], in[0])) return kInvalid;
    if (in[0].shape[3] != 128 || wq.shape[0] != 128 || wk.shape[0] != 128) return kInvalid;
    if (cos.shape[1] != 48 || !same_shape(cos, sin) || pos.shape[0] != in[0].shape[0]) return kInvalid;
    const int64_t rows = in[0].shape[0] * in[0].shape[1] * in[0].shape[2];
    if (rows != 0 && cos.shape[0] == 0) return kInvalid;  // no table row for the tokens to take
    bool vec = rows_vec16(cos, 2) && rows_vec16(sin, 2) && rows_vec16(wq, 2) && rows_vec16(wk, 2);
    for (int i = 0; i < 3; ++i) vec = vec && rows_vec16(in[i], 2);
    // bf16 rows: 16-byte vectors; fp8 code rows (128 B): 8-byte vectors per lane.
    for (int i = 0; i < 3; ++i) vec = vec && (fp8 && i < 2 ? rows_vec8_bytes(out[i]) : rows_vec16(out[i], 2));
    if (fp8) {
        const int64_t heads = in[0].shape[1] * in[0].shape[2];
        for (const View<1> *d : {q_descale, k_descale})
            if (d->shape[0] != heads || (heads > 1 && d->stride[0] != 1)) return kInvalid;
        if (vamax && (heads > kVamaxHeads || v_amax->shape[0] != heads || v_amax->shape[1] != H3_AMAX_SLOTS ||
                      v_amax->stride[1] != 1 || (heads > 1 && v_amax->stride[0] != H3_AMAX_SLOTS)))
            return kInvalid;
    }
    auto head_rows = [](const View<4> &v) {
        return HeadRows{v.data, v.stride[0], v.stride[1], v.stride[2], v.stride[3]};
    };
    QkvArgs a{};
    a.q = head_rows(in[0]);
    a.k = head_rows(in[1]);
    a.v = head_rows(in[2]);
    a.q_out = head_rows(out[0]);
    a.k_out = head_rows(out[1]);
    a.v_out = head_rows(out[2]);
    a.wq = reinterpret_cast<const bf16_t *>(wq.data);
    a.wk = reinterpret_cast<const bf16_t *>(wk.data);
    a.wq_stride = wq.stride[0];
    a.wk_stride = wk.stride[0];
    a.cos = reinterpret_cast<const bf16_t *>(cos.data);
    a.sin = reinterpret_cast<const bf16_t *>(sin.data);
    a.cs0 = cos.stride[0];
    a.cs1 = cos.stride[1];
    a.ss0 = sin.stride[0];
    a.ss1 = sin.stride[1];
    a.pos = reinterpret_cast<const int64_t *>(pos.data);
    a.pos_stride = pos.stride[0];
    a.table_rows = cos.shape[0];
    a.rows = rows;
    a.P = in[0].shape[1];
    a.Hs = in[0].shape[2];
    a.eps_bf = host_round_bf16(eps);
    if (fp8) {
        a.q_descale = reinterpret_cast<float *>(q_descale->data);
        a.k_descale = reinterpret_cast<float *>(k_descale->data);
    }
    if (vamax) a.v_amax = reinterpret_cast<uint32_t *>(v_amax->data);
    if (two) {
        a.q_out_lo = out_lo[0].data;
        a.k_out_lo = out_lo[1].data;
    }
    if (rows >= (int64_t{1} << 31) - kThreads * 4) return kInvalid;
    if (check_only) return 0;
    // kQkvBlocks blocks per tensor at most, one batch of kThreads / 16 rows each
    // per turn.
    constexpr int64_t kBatch = kThreads / 16 * kQkvRows;
    const int64_t batches = (rows + kBatch - 1) / kBatch;
    const int64_t tiles = batches < kQkvBlocks ? batches : kQkvBlocks;
    const int64_t heads = a.P * a.Hs;
    a.v_pinned = vamax && heads > 0 && tiles >= heads;
    if (vamax && !a.v_pinned) {  // the slots start at 0 (an empty V has amax 0)
        const int64_t n = heads * H3_AMAX_SLOTS;
        if (n > 0) clear_words_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, stream>>>(a.v_amax, n);
    }
    if (rows == 0) return vamax ? launch_status() : 0;
    a.by_ph = make_fastdiv(static_cast<uint32_t>(a.P * a.Hs));
    a.by_h = make_fastdiv(static_cast<uint32_t>(a.Hs));
    bool off32 = offsets_fit_int32(cos) && offsets_fit_int32(sin) && offsets_fit_int32(pos) &&
                 a.P * a.Hs < (int64_t{1} << 24);
    for (int i = 0; i < 3; ++i) off32 = off32 && offsets_fit_int32(in[i]) && offsets_fit_int32(out[i]);
    const unsigned g = static_cast<unsigned>(3 * tiles);
#define H3_QKV(V, O, F) \
    if (vec == V && off32 == O && fp8 == F && !vamax && !two) \
        qkv_pack_kernel<V, kQkvRows, O, F><<<g, kThreads, 0, stream>>>(a);
    H3_QKV(true, true, false) H3_QKV(true, false, false) H3_QKV(false, true, false) H3_QKV(false, false, false)
    H3_QKV(true, true, true) H3_QKV(true, false, true) H3_QKV(false, true, true) H3_QKV(false, false, true)
    // With V's maximum (one- or two-term codes): the pinned instantiation when
    // the launch pins its v blocks to heads.
#define H3_QKVA(V, O, T) \
    if (vec == V && off32 == O && (vamax || two) && two == T) { \
        if (a.v_pinned) \
            qkv_pack_kernel<V, kQkvRows, O, true, true, T, true><<<g, kThreads, 0, stream>>>(a); \
        else \
            qkv_pack_kernel<V, kQkvRows, O, true, true, T><<<g, kThreads, 0, stream>>>(a); \
    }
    H3_QKVA(true, true, false) H3_QKVA(true, false, false) H3_QKVA(false, true, false) H3_QKVA(false, false, false)
    H3_QKVA(true, true, true) H3_QKVA(true, false, true) H3_QKVA(false, true, true) H3_QKVA(false, false, true)
#undef H3_QKVA
#undef H3_QKV
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

// V's amax slots of launch_h3_qkv_norm_rope_pack_fp8_noalloc, which allocates
// nothing: one H3_AMAX_SLOTS-word row per head for up to kVamaxHeads heads
// (256 KiB on every device the library runs on, held until the process ends).
// Host code never passes `scratch` itself to a kernel: on the host the name
// stands for a shadow variable, not a device address. scratch_slots() looks
// up the device address once per device (hipGetSymbolAddress, with that
// device current) and every launch takes that address.
static __device__ __align__(256) uint32_t scratch[kVamaxHeads * H3_AMAX_SLOTS];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<uintptr_t> scratch_address[kMaxDevices];  // 0 until looked up

// The device address of `scratch` on the device that `stream` belongs to.
int scratch_slots(hipStream_t stream, uint32_t *&slots) {
    int dev = 0;
    hipError_t e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) return static_cast<int>(e);
    if (dev < 0 || dev >= kMaxDevices) return kInvalid;
    uintptr_t addr = scratch_address[dev].load(std::memory_order_acquire);
    if (addr == 0) {
        int current = 0;
        if ((e = hipGetDevice(&current)) != hipSuccess) return static_cast<int>(e);
        if (current != dev && (e = hipSetDevice(dev)) != hipSuccess) return static_cast<int>(e);
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (current != dev) {
            const hipError_t back = hipSetDevice(current);
            if (e == hipSuccess) e = back;
        }
        if (e != hipSuccess) return static_cast<int>(e);
        if (p == nullptr) return kInvalid;
        addr = reinterpret_cast<uintptr_t>(p);
        scratch_address[dev].store(addr, std::memory_order_release);
    }
    slots = reinterpret_cast<uint32_t *>(addr);
    return 0;
}

}  // namespace
}  // namespace h3

using namespace h3;

extern "C" {

NineToothedResult launch_h3_swiglu_exact(NineToothedStream stream, NineToothedTensor up, NineToothedTensor gate,
                                         NineToothedTensor out) {
    const NineToothedTensor in[2] = {up, gate};
    return launch_ew<SwigluOp>(as_stream(stream), in, out);
}

NineToothedResult launch_h3_gated_residual_exact(NineToothedStream stream, NineToothedTensor x,
                                                 NineToothedTensor gate, NineToothedTensor y,
                                                 NineToothedTensor out) {
    const NineToothedTensor in[3] = {x, gate, y};
    return launch_ew<GatedResidualOp>(as_stream(stream), in, out);
}

NineToothedResult launch_h3_gated_residual_indexed(NineToothedStream stream, NineToothedTensor x,
                                                   NineToothedTensor gate, NineToothedTensor y,
                                                   NineToothedTensor index, NineToothedTensor out) {
    const NineToothedTensor in[3] = {x, gate, y};
    return launch_ew<GatedResidualOp>(as_stream(stream), in, out, &index);
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

NineToothedResult launch_h3_rms_modulate_indexed(NineToothedStream stream, NineToothedTensor x,
                                                 NineToothedTensor weight, NineToothedTensor eps,
                                                 NineToothedTensor scale, NineToothedTensor shift,
                                                 NineToothedTensor index, NineToothedTensor out) {
    return rms_family(kRmsModulate, as_stream(stream), x, nullptr, nullptr, weight, eps, &scale, &shift, nullptr,
                      out, 0, &index);
}

NineToothedResult launch_h3_gated_residual_rms_modulate_indexed(
    NineToothedStream stream, NineToothedTensor x, NineToothedTensor gate, NineToothedTensor y,
    NineToothedTensor weight, NineToothedTensor eps, NineToothedTensor scale, NineToothedTensor shift,
    NineToothedTensor index, NineToothedTensor residual, NineToothedTensor out) {
    return rms_family(kGatedRmsModulate, as_stream(stream), x, &gate, &y, weight, eps, &scale, &shift, &residual,
                      out, 0, &index);
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

NineToothedResult launch_h3_qk_norm_rope_interleaved_qk(NineToothedStream stream, NineToothedTensor q,
                                                        NineToothedTensor k, NineToothedTensor q_weight,
                                                        NineToothedTensor k_weight, NineToothedTensor eps,
                                                        NineToothedTensor cos, NineToothedTensor sin,
                                                        NineToothedTensor q_out, NineToothedTensor k_out) {
    View<4> qv, kv, qo, ko;
    View<2> c, s;
    View<1> wq, wk;
    double e;
    if (!load_view(q, 2, qv) || !load_view(k, 2, kv) || !load_view(q_out, 2, qo) || !load_view(k_out, 2, ko) ||
        !load_view(cos, 2, c) || !load_view(sin, 2, s) || !load_view(q_weight, 2, wq) ||
        !load_view(k_weight, 2, wk) || !load_scalar(eps, e))
        return kInvalid;
    return launch_head_rows<kNormRopeInterleaved>(as_stream(stream), qv, qo, c, s, &wq, e, &kv, &ko, &wk);
}

NineToothedResult launch_h3_qkv_norm_rope_pack(NineToothedStream stream, NineToothedTensor q,
                                               NineToothedTensor k, NineToothedTensor v,
                                               NineToothedTensor q_weight, NineToothedTensor k_weight,
                                               NineToothedTensor eps, NineToothedTensor cos,
                                               NineToothedTensor sin, NineToothedTensor positions,
                                               NineToothedTensor q_out, NineToothedTensor k_out,
                                               NineToothedTensor v_out) {
    View<4> in[3], out[3];
    View<1> wq, wk, pos;
    View<2> c, sn;
    double e;
    const NineToothedTensor ins[3] = {q, k, v}, outs[3] = {q_out, k_out, v_out};
    for (int i = 0; i < 3; ++i)
        if (!load_view(ins[i], 2, in[i]) || !load_view(outs[i], 2, out[i])) return kInvalid;
    if (!load_view(q_weight, 2, wq) || !load_view(k_weight, 2, wk) || !load_scalar(eps, e) ||
        !load_view(cos, 2, c) || !load_view(sin, 2, sn) || !load_view(positions, 8, pos))
        return kInvalid;
    return launch_qkv_pack(as_stream(stream), in, out, wq, wk, e, c, sn, pos);
}

NineToothedResult launch_h3_qkv_norm_rope_pack_fp8(NineToothedStream stream, NineToothedTensor q,
                                                   NineToothedTensor k, NineToothedTensor v,
                                                   NineToothedTensor q_weight, NineToothedTensor k_weight,
                                                   NineToothedTensor eps, NineToothedTensor cos,
                                                   NineToothedTensor sin, NineToothedTensor positions,
                                                   NineToothedTensor q8, NineToothedTensor k8,
                                                   NineToothedTensor v_out, NineToothedTensor q_descale,
                                                   NineToothedTensor k_descale) {
    View<4> in[3], out[3];
    View<1> wq, wk, pos, qd, kd;
    View<2> c, sn;
    double e;
    const NineToothedTensor ins[3] = {q, k, v};
    for (int i = 0; i < 3; ++i)
        if (!load_view(ins[i], 2, in[i])) return kInvalid;
    if (!load_view(q8, 1, out[0]) || !load_view(k8, 1, out[1]) || !load_view(v_out, 2, out[2])) return kInvalid;
    if (!load_view(q_weight, 2, wq) || !load_view(k_weight, 2, wk) || !load_scalar(eps, e) ||
        !load_view(cos, 2, c) || !load_view(sin, 2, sn) || !load_view(positions, 8, pos) ||
        !load_view(q_descale, 4, qd) || !load_view(k_descale, 4, kd))
        return kInvalid;
    return launch_qkv_pack(as_stream(stream), in, out, wq, wk, e, c, sn, pos, &qd, &kd);
}

NineToothedResult launch_h3_qkv_norm_rope_pack_fp8_vamax(
    NineToothedStream stream, NineToothedTensor q, NineToothedTensor k, NineToothedTensor v,
    NineToothedTensor q_weight, NineToothedTensor k_weight, NineToothedTensor eps, NineToothedTensor cos,
    NineToothedTensor sin, NineToothedTensor positions, NineToothedTensor q8, NineToothedTensor k8,
    NineToothedTensor v_out, NineToothedTensor q_descale, NineToothedTensor k_descale, NineToothedTensor v_amax) {
    View<4> in[3], out[3];
    View<1> wq, wk, pos, qd, kd;
    View<2> c, sn, va;
    double e;
    const NineToothedTensor ins[3] = {q, k, v};
    for (int i = 0; i < 3; ++i)
        if (!load_view(ins[i], 2, in[i])) return kInvalid;
    if (!load_view(q8, 1, out[0]) || !load_view(k8, 1, out[1]) || !load_view(v_out, 2, out[2])) return kInvalid;
    if (!load_view(q_weight, 2, wq) || !load_view(k_weight, 2, wk) || !load_scalar(eps, e) ||
        !load_view(cos, 2, c) || !load_view(sin, 2, sn) || !load_view(positions, 8, pos) ||
        !load_view(q_descale, 4, qd) || !load_view(k_descale, 4, kd) || !load_view(v_amax, 4, va))
        return kInvalid;
    return launch_qkv_pack(as_stream(stream), in, out, wq, wk, e, c, sn, pos, &qd, &kd, &va);
}

NineToothedResult launch_h3_qkv_norm_rope_pack_fp8x2_vamax(
    NineToothedStream stream, NineToothedTensor q, NineToothedTensor k, NineToothedTensor v,
    NineToothedTensor q_weight, NineToothedTensor k_weight, NineToothedTensor eps, NineToothedTensor cos,
    NineToothedTensor sin, NineToothedTensor positions, NineToothedTensor q8, NineToothedTensor q8_lo,
    NineToothedTensor k8, NineToothedTensor k8_lo, NineToothedTensor v_out, NineToothedTensor q_descale,
    NineToothedTensor k_descale, NineToothedTensor v_amax) {
    View<4> in[3], out[3], lo[2];
    View<1> wq, wk, pos, qd, kd;
    View<2> c, sn, va;
    double e;
    const NineToothedTensor ins[3] = {q, k, v};
    for (int i = 0; i < 3; ++i)
        if (!load_view(ins[i], 2, in[i])) return kInvalid;
    if (!load_view(q8, 1, out[0]) || !load_view(k8, 1, out[1]) || !load_view(v_out, 2, out[2]) ||
        !load_view(q8_lo, 1, lo[0]) || !load_view(k8_lo, 1, lo[1]))
        return kInvalid;
    if (!load_view(q_weight, 2, wq) || !load_view(k_weight, 2, wk) || !load_scalar(eps, e) ||
        !load_view(cos, 2, c) || !load_view(sin, 2, sn) || !load_view(positions, 8, pos) ||
        !load_view(q_descale, 4, qd) || !load_view(k_descale, 4, kd) || !load_view(v_amax, 4, va))
        return kInvalid;
    return launch_qkv_pack(as_stream(stream), in, out, wq, wk, e, c, sn, pos, &qd, &kd, &va, false, lo);
}

NineToothedResult launch_h3_qkv_norm_rope_pack_fp8_noalloc(
    NineToothedStream stream, NineToothedTensor q, NineToothedTensor k, NineToothedTensor v,
    NineToothedTensor q_weight, NineToothedTensor k_weight, NineToothedTensor eps, NineToothedTensor cos,
    NineToothedTensor sin, NineToothedTensor positions, NineToothedTensor q8, NineToothedTensor k8,
    NineToothedTensor v_out, NineToothedTensor q_descale, NineToothedTensor k_descale, NineToothedTensor v8,
    NineToothedTensor v_descale) {
    View<4> in[3], out[3];
    View<1> wq, wk, pos, qd, kd;
    View<2> c, sn;
    double e;
    const NineToothedTensor ins[3] = {q, k, v};
    for (int i = 0; i < 3; ++i)
        if (!load_view(ins[i], 2, in[i])) return kInvalid;
    if (!load_view(q8, 1, out[0]) || !load_view(k8, 1, out[1]) || !load_view(v_out, 2, out[2])) return kInvalid;
    if (!load_view(q_weight, 2, wq) || !load_view(k_weight, 2, wk) || !load_scalar(eps, e) ||
        !load_view(cos, 2, c) || !load_view(sin, 2, sn) || !load_view(positions, 8, pos) ||
        !load_view(q_descale, 4, qd) || !load_view(k_descale, 4, kd))
        return kInvalid;
    // One rank's heads (P = 1), at most as many as the scratch slots hold.
    const int64_t T = out[2].shape[0], heads = out[2].shape[2];
    if (out[2].shape[1] != 1 || heads > kVamaxHeads) return kInvalid;
    hipStream_t st = as_stream(stream);
    // Every check of both steps before the first HIP call: the pack's, then the
    // quantiser's on v_out read as [1, Hs, T, 128].
    if (launch_qkv_pack(st, in, out, wq, wk, e, c, sn, pos, &qd, &kd, nullptr, true) != 0) return kInvalid;
    uint64_t xshape[4] = {1, static_cast<uint64_t>(heads), static_cast<uint64_t>(T), 128};
    int64_t xstride[4] = {0, out[2].stride[2], out[2].stride[0], out[2].stride[3]};
    const NineToothedTensor x{v_out.data, xshape, xstride};
    if (check_quantize_fp8_per_head(x, v8, v_descale) != 0) return kInvalid;
    uint32_t *slots = nullptr;
    const int rc = scratch_slots(st, slots);
    if (rc != 0) return rc;
    View<2> sv;
    sv.data = reinterpret_cast<char *>(slots);
    sv.shape[0] = heads;
    sv.shape[1] = H3_AMAX_SLOTS;
    sv.stride[0] = H3_AMAX_SLOTS;
    sv.stride[1] = 1;
    const int packed = launch_qkv_pack(st, in, out, wq, wk, e, c, sn, pos, &qd, &kd, &sv);
    if (packed != 0) return packed;
    uint64_t sshape[2] = {static_cast<uint64_t>(heads), H3_AMAX_SLOTS};
    int64_t sstride[2] = {H3_AMAX_SLOTS, 1};
    return launch_h3_quantize_fp8_per_head_slots(stream, x, NineToothedTensor{slots, sshape, sstride}, v8, v_descale);
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
