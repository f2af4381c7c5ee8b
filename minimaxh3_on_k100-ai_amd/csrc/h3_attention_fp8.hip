// fp8 (OCP e4m3fn) attention for gfx950: per-head quantisation of Q/K/V and a
// flash-attention forward whose P.V product (and, in the all-fp8 recipe, the
// Q K^T product) runs on v_mfma_scale_f32_32x32x64_f8f6f4 (unit scales).
// No counterpart in the reference, which has no fp8 path; the numerics follow
// its bf16 kernel (tools/h3_attention.py:25-41) with these changes:
//   - x8 = e4m3(x * 448 / amax_h), descale_h = amax_h / 448 per head;
//   - logits = (q8 . k8) * q_descale * k_descale * scale * log2(e) (all-fp8), or
//     the bf16 logits of the bf16 kernel (fp8 P.V variant);
//   - P = exp2(logit - running max) is requantised per 64-key tile as
//     e4m3(448 * P) (P <= 1, so the fixed factor uses the whole range); 448 P
//     is formed directly as exp2(logit - (running max - log2 448)), and
//     o = acc * v_descale / denominator -- the same quantities as
//     o = acc * v_descale / (448 l). The denominator sums the fp32 448 P in
//     the bf16-logit and the two-term variants; in the one-term all-fp8
//     recipe it sums the quantised e4m3(448 P) -- the weights the numerator
//     uses -- on the MFMA.
//
// Work decomposition as in the bf16 kernel: 512-thread workgroups (8 waves,
// two per SIMD), 32 queries per wave, 64-key tiles in double-buffered LDS,
// S^T = K Q^T so each lane owns one query row of the softmax.
//
// Key order. K row for MFMA row m of 32-key block ks is
//   key(ks, m) = 32*bit2(m) + 16*ks + 4*(m >> 3) + (m & 3),
// which makes accumulator register i of block ks in a lane of half h hold key
// 32h + 16ks + i: each lane's 32 scores are the contiguous keys [32h, 32h+32)
// of the tile, i.e. exactly the 32 k-slots of its half in the 64-deep fp8 P.V
// MFMA. The V operand is then V^T[d][32h .. 32h+32): 32 contiguous bytes of
// the V^T tile, which the quantiser provides by writing V8 S-contiguous.
//
// LDS tiles carry no padding; 16-byte chunks are XOR-swizzled per row so the
// rows read by one 16-lane ds_read_b128 pass fall in distinct banks.
#include <type_traits>

#include "h3_common.hpp"
#include "h3_internal.hpp"

namespace h3 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));

constexpr int kD = 128;
constexpr int kWaves = 8;
constexpr int kThreadsWG = 64 * kWaves;
constexpr int kBM = 32 * kWaves;
constexpr int kBN = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kE4M3Max = 448.0f;
constexpr float kLog2E4M3Max = 8.80735492205760410744f;  // log2(448)
constexpr int kE4M3OnesX4 = 0x38383838;                   // four e4m3fn 1.0 codes
constexpr int kScale1 = 127;  // E8M0 exponent of 1.0 for the scaled MFMA
// Two-term Q and K: the lo term's codes count 2^-4 of the hi term's units,
// which the scaled MFMA applies as the E8M0 block scale 2^-4.
constexpr float kLoTermShift = 16.0f;
constexpr int kScaleLo = 123;

// ------------------------------------------------------------------ swizzles

// K tile of QK_FP8 (fp8, 128 B rows = 8 chunks): position of chunk c of row r.
__device__ __forceinline__ int kswz8(int r, int c) { return c ^ (((r >> 1) & 3) | (((r >> 5) & 1) << 2)); }
// K tile of bf16 logits (256 B rows = 16 chunks).
__device__ __forceinline__ int kswz16(int r, int c) { return c ^ ((r & 7) | (((r >> 5) & 1) << 3)); }
// V^T tile (64 B rows = 4 chunks).
__device__ __forceinline__ int vswz(int d, int c) { return c ^ ((d >> 2) & 3); }

// K row feeding MFMA row m of 32-key block ks (see header).
__device__ __forceinline__ int key_of_row(int ks, int m) {
    return 32 * ((m >> 2) & 1) + 16 * ks + 4 * (m >> 3) + (m & 3);
}

__device__ __forceinline__ int xcd_remap(int x, int total) {
    const int per = total / 8, rem = total % 8;
    const int xcd = x % 8, slot = x / 8;
    return xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

struct Fp8Args {
    const uint8_t *q8, *k8;  // all-fp8 recipe
    const uint8_t *q8lo, *k8lo;  // two-term Q and K: the lo codes (q8's / k8's strides)
    const bf16_t *q, *k;     // bf16-logit variant
    const uint8_t *v8;       // S-contiguous (element (b, h, s, d) at b*vs0 + h*vs1 + s + d*vs3)
    bf16_t *o;
    const float *q_descale, *k_descale, *v_descale;
    int64_t qs[3], ks[3], vs0, vs1, vs3, os[3];
    int B, H, Sq, Sk, qblocks;
    float c;  // scale * log2(e)
    int k_bytes, v_bytes;  // buffer-load path: byte extent of one head's K rows / V^T rows
};

// The dword-3 word of a raw buffer descriptor on gfx9 (CDNA): no format
// conversion, bounds checked against num_records in bytes.
constexpr int kBufferWord3 = 0x00020000;

// ------------------------------------------------------------------ tiles

// K tile, global -> LDS (through registers): 64 rows of 128 (fp8) or 256 (bf16)
// bytes; rows past `valid` are zero.
// TWO (fp8 only): reg[1] holds the same chunk of the lo codes' tile.
template <bool QK_FP8, bool TWO>
__device__ __forceinline__ void load_k(const Fp8Args &a, int b, int h, int key0, int valid, u32x4_t (&reg)[2]) {
    const int t = threadIdx.x;
    constexpr int kChunks = QK_FP8 ? 8 : 16;
    constexpr int kPerThread = kBN * kChunks / kThreadsWG;  // 1 or 2
    static_assert(!TWO || kPerThread == 1, "the lo tile takes the second register");
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        const int idx = t + i * kThreadsWG;
        const int r = idx / kChunks, c = idx % kChunks;
        if (r < valid) {
            const int64_t off = b * a.ks[0] + h * a.ks[1] + static_cast<int64_t>(key0 + r) * a.ks[2];
            const uint8_t *row = QK_FP8 ? a.k8 + off : reinterpret_cast<const uint8_t *>(a.k + off);
            reg[i] = *reinterpret_cast<const u32x4_t *>(row + 16 * c);
            if constexpr (TWO) reg[1] = *reinterpret_cast<const u32x4_t *>(a.k8lo + off + 16 * c);
        } else {
            reg[i] = u32x4_t{0u, 0u, 0u, 0u};
            if constexpr (TWO) reg[1] = u32x4_t{0u, 0u, 0u, 0u};
        }
    }
}

// A full K tile: the loads of load_k without the row test, so the main loop
// issues them unconditionally (a load under a branch is waited for before the
// branch closes).
template <bool QK_FP8, bool TWO>
__device__ __forceinline__ void load_k_full(const Fp8Args &a, int b, int h, int key0, u32x4_t (&reg)[2]) {
    const int t = threadIdx.x;
    constexpr int kChunks = QK_FP8 ? 8 : 16;
    constexpr int kPerThread = kBN * kChunks / kThreadsWG;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        const int idx = t + i * kThreadsWG;
        const int r = idx / kChunks, c = idx % kChunks;
        const int64_t off = b * a.ks[0] + h * a.ks[1] + static_cast<int64_t>(key0 + r) * a.ks[2];
        const uint8_t *row = QK_FP8 ? a.k8 + off : reinterpret_cast<const uint8_t *>(a.k + off);
        reg[i] = *reinterpret_cast<const u32x4_t *>(row + 16 * c);
        if constexpr (TWO) reg[1] = *reinterpret_cast<const u32x4_t *>(a.k8lo + off + 16 * c);
    }
}

// TWO: the lo tile follows the hi tile (kBN 128-byte rows further on).
template <bool QK_FP8, bool TWO>
__device__ __forceinline__ void store_k(uint8_t *lds, const u32x4_t (&reg)[2]) {
    const int t = threadIdx.x;
    constexpr int kChunks = QK_FP8 ? 8 : 16;
    constexpr int kPerThread = kBN * kChunks / kThreadsWG;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        const int idx = t + i * kThreadsWG;
        const int r = idx / kChunks, c = idx % kChunks;
        const int pos = QK_FP8 ? kswz8(r, c) : kswz16(r, c);
        *reinterpret_cast<u32x4_t *>(lds + r * (16 * kChunks) + 16 * pos) = reg[i];
        if constexpr (TWO) *reinterpret_cast<u32x4_t *>(lds + kBN * 128 + r * 128 + 16 * pos) = reg[1];
    }
}

// V^T tile: 128 rows (dims) of 64 key bytes; keys past `valid` are zero.
__device__ __forceinline__ void load_v(const Fp8Args &a, int b, int h, int key0, int valid, u32x4_t &reg) {
    const int t = threadIdx.x;
    const int d = t / 4, c = t % 4;
    const uint8_t *row = a.v8 + b * a.vs0 + h * a.vs1 + static_cast<int64_t>(d) * a.vs3 + key0 + 16 * c;
    if (16 * c + 16 <= valid) {
        reg = *reinterpret_cast<const u32x4_t *>(row);
    } else {
        uint8_t bytes[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) bytes[e] = (16 * c + e < valid) ? row[e] : 0;
        reg = *reinterpret_cast<const u32x4_t *>(bytes);
    }
}

// A full V^T tile: every 16-byte chunk is inside the 64 keys.
__device__ __forceinline__ void load_v_full(const Fp8Args &a, int b, int h, int key0, u32x4_t &reg) {
    const int t = threadIdx.x;
    const int d = t / 4, c = t % 4;
    reg = *reinterpret_cast<const u32x4_t *>(a.v8 + b * a.vs0 + h * a.vs1 + static_cast<int64_t>(d) * a.vs3 + key0 + 16 * c);
}

__device__ __forceinline__ void store_v(uint8_t *lds, const u32x4_t &reg) {
    const int t = threadIdx.x;
    const int d = t / 4, c = t % 4;
    *reinterpret_cast<u32x4_t *>(lds + d * 64 + 16 * vswz(d, c)) = reg;
}

// One full K tile and V^T tile straight from HBM into LDS (the buffer path):
// wave w's K load i and its V^T load write 64 16-byte slots each at the
// wave's LDS base + 16 lane; `kvoff` / `vvoff` (per thread, fixed for the
// kernel) pick the source chunk each slot holds, `ksoff` / `vsoff` are the
// tile's uniform byte offsets. The loads complete asynchronously: the caller
// waits on vmcnt before the barrier that publishes the tiles.
// (Plain overloads for one and two K loads per thread: the buffer resource
// type cannot be substituted into a template in the host pass.)
__device__ __forceinline__ void dma_k_load(__amdgpu_buffer_rsrc_t krs, int voff, int soff, uint8_t *kn, int slot0) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (__attribute__((address_space(3))) void *)(kn + 16 * slot0), 16, voff,
                                             soff, 0, 0);
}
__device__ __forceinline__ void dma_tile_pair(__amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                              const int (&kvoff)[1], int vvoff, int ksoff, int vsoff, uint8_t *kn,
                                              uint8_t *vn) {
    const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    dma_k_load(krs, kvoff[0], ksoff, kn, 64 * w);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (__attribute__((address_space(3))) void *)(vn + 16 * 64 * w), 16,
                                             vvoff, vsoff, 0, 0);
}
// Two-term K: the hi and lo tiles (descriptors krs, krs_lo, the same
// offsets), the lo tile at the hi tile's end.
__device__ __forceinline__ void dma_tile_two(__amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t krs_lo,
                                             __amdgpu_buffer_rsrc_t vrs, const int (&kvoff)[1], int vvoff, int ksoff,
                                             int vsoff, uint8_t *kn, uint8_t *vn) {
    const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    dma_k_load(krs, kvoff[0], ksoff, kn, 64 * w);
    dma_k_load(krs_lo, kvoff[0], ksoff, kn, kThreadsWG + 64 * w);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (__attribute__((address_space(3))) void *)(vn + 16 * 64 * w), 16,
                                             vvoff, vsoff, 0, 0);
}
__device__ __forceinline__ void dma_tile_pair(__amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                              const int (&kvoff)[2], int vvoff, int ksoff, int vsoff, uint8_t *kn,
                                              uint8_t *vn) {
    const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    dma_k_load(krs, kvoff[0], ksoff, kn, 64 * w);
    dma_k_load(krs, kvoff[1], ksoff, kn, kThreadsWG + 64 * w);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (__attribute__((address_space(3))) void *)(vn + 16 * 64 * w), 16,
                                             vvoff, vsoff, 0, 0);
}

// ------------------------------------------------------------------ kernel

// BUF: the main loop's full K and V^T tiles through buffer loads, each
// thread's byte offsets fixed for the kernel and the tile's offset uniform (the
// host checks that one head's rows fit a 31-bit byte range).
// TWO (QK_FP8 only): Q and K each as hi + lo e4m3 codes (lo in 2^-4 of hi's
// units): the logits accumulate hi.hi + 2^-4 (lo.hi + hi.lo) on one
// accumulator, the 2^-4 applied as the MFMA's block scale of the lo operand.
template <bool QK_FP8, bool NEG, bool BUF, bool TWO = false>
__global__ __launch_bounds__(kThreadsWG) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_fp8_kernel(
    Fp8Args a) {
    static_assert(!TWO || QK_FP8, "the two-term split is of fp8 Q and K");
    // The one-term all-fp8 recipe forms its denominator on the MFMA (its VALU is
    // the scarcer unit); the others sum the fp32 448 P on the VALU (the
    // two-term recipe's MFMA work is three Q K^T products already: measured
    // 2.5% faster with the VALU sum).
    constexpr bool kDenOnMfma = QK_FP8 && !TWO;
    constexpr int kKBytes = kBN * (QK_FP8 ? 128 : 256) * (TWO ? 2 : 1);
    // Two buffers per operand as separate arrays: the loads into one buffer
    // then provably do not alias the reads of the other.
    __shared__ __attribute__((aligned(1024))) uint8_t lds_k0[kKBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t lds_k1[kKBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t lds_v0[kD * kBN];
    __shared__ __attribute__((aligned(1024))) uint8_t lds_v1[kD * kBN];

    const int total = a.B * a.H * a.qblocks;
    const int logical = xcd_remap(blockIdx.x, total);
    const int qb = logical % a.qblocks;
    const int bh = logical / a.qblocks;
    const int b = bh / a.H, h = bh % a.H;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int l32 = lane & 31;
    const int half = lane >> 5;

    const float c = QK_FP8 ? a.c * a.q_descale[h] * a.k_descale[h] : a.c;
    const float out_scale = a.v_descale[h];  // the denominator sums 448 P

    // Q^T operands (this lane's query row).
    const int query = qb * kBM + wave * 32 + l32;
    const int qrow_i = query < a.Sq ? query : a.Sq - 1;
    i32x8_t q8reg[2], q8lo[2];
    bf16x8_t qbreg[8];
    if constexpr (QK_FP8) {
        const int64_t qoff = b * a.qs[0] + h * a.qs[1] + static_cast<int64_t>(qrow_i) * a.qs[2] + 32 * half;
#pragma unroll
        for (int term = 0; term < (TWO ? 2 : 1); ++term) {
            const uint8_t *qrow = (term == 0 ? a.q8 : a.q8lo) + qoff;
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const uint4 lo = *reinterpret_cast<const uint4 *>(qrow + 64 * kk);
                const uint4 hi = *reinterpret_cast<const uint4 *>(qrow + 64 * kk + 16);
                const i32x8_t v{static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z),
                                static_cast<int>(lo.w), static_cast<int>(hi.x), static_cast<int>(hi.y),
                                static_cast<int>(hi.z), static_cast<int>(hi.w)};
                if (term == 0)
                    q8reg[kk] = v;
                else
                    q8lo[kk] = v;
            }
        }
    } else {
        const bf16_t *qrow = a.q + b * a.qs[0] + h * a.qs[1] + static_cast<int64_t>(qrow_i) * a.qs[2] + 8 * half;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
            qbreg[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(qrow + 16 * kk));
    }

    f32x16_t acc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[db][i] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    // One-term all-fp8: the denominator on the MFMA. V^T's rows are replaced by
    // e4m3 ones, so every accumulator register of a lane gathers its query's
    // sum of the quantised 448 P over the keys so far; element 0 is the one the
    // rescale keeps up to date. The bf16-logit variant keeps the fp32 sum (no
    // VGPRs to spare), and so does the two-term one (kDenOnMfma).
    f32x16_t lacc;
#pragma unroll
    for (int i = 0; i < 16; ++i) lacc[i] = 0.0f;
    const i32x8_t ones{kE4M3OnesX4, kE4M3OnesX4, kE4M3OnesX4, kE4M3OnesX4,
                       kE4M3OnesX4, kE4M3OnesX4, kE4M3OnesX4, kE4M3OnesX4};

    const int ntiles = (a.Sk + kBN - 1) / kBN;
    {
        u32x4_t kr[2], vr;
        const int valid = a.Sk < kBN ? a.Sk : kBN;
        load_k<QK_FP8, TWO>(a, b, h, 0, valid, kr);
        load_v(a, b, h, 0, valid, vr);
        store_k<QK_FP8, TWO>(lds_k0, kr);
        store_v(lds_v0, vr);
    }
    __syncthreads();

    // One tile of keys from the LDS tiles (kt, vt): S^T = K Q^T, online softmax, O^T
    // += V^T P^T. MASKED: keys >= valid are excluded (the last, partial tile).
    auto attend = [&](auto masked_tag, const uint8_t *kt, const uint8_t *vt, int valid) __attribute__((always_inline)) {
        constexpr bool MASKED = decltype(masked_tag)::value;

        // ---- S^T = K Q^T: s[ks][i] = logit of key 32*half + 16*ks + i
        f32x16_t s[2];
        const f32x16_t zero = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int r = key_of_row(ks, l32);
            if constexpr (QK_FP8) {
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const int c0 = 4 * kk + 2 * half;  // 16-byte chunk of dims 64kk + 32half
                    i32x8_t kop[2];
#pragma unroll
                    for (int term = 0; term < (TWO ? 2 : 1); ++term) {
                        const uint8_t *krow = kt + term * (kBN * 128) + r * 128;
                        const uint4 lo = *reinterpret_cast<const uint4 *>(krow + 16 * kswz8(r, c0));
                        const uint4 hi = *reinterpret_cast<const uint4 *>(krow + 16 * kswz8(r, c0 + 1));
                        kop[term] = i32x8_t{static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z),
                                            static_cast<int>(lo.w), static_cast<int>(hi.x), static_cast<int>(hi.y),
                                            static_cast<int>(hi.z), static_cast<int>(hi.w)};
                    }
                    s[ks] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kop[0], q8reg[kk], kk == 0 ? zero : s[ks],
                                                                            0, 0, 0, kScale1, 0, kScale1);
                    if constexpr (TWO) {
                        s[ks] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kop[1], q8reg[kk], s[ks], 0, 0, 0,
                                                                                kScaleLo, 0, kScale1);
                        s[ks] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kop[0], q8lo[kk], s[ks], 0, 0, 0,
                                                                                kScale1, 0, kScaleLo);
                    }
                }
            } else {
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    const int c0 = 2 * kk + half;  // 16-byte chunk of dims 16kk + 8half
                    const bf16x8_t kop =
                        __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(kt + r * 256 + 16 * kswz16(r, c0)));
                    s[ks] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop, qbreg[kk], kk == 0 ? zero : s[ks], 0, 0, 0);
                }
            }
        }

        // Bounded K operand window: a few LDS reads ahead of the MFMAs,
        // so the operands do not all occupy registers at once.
        if constexpr (TWO) {  // 16 reads, 12 MFMAs
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
        } else if constexpr (QK_FP8) {
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        } else {
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
            for (int i = 0; i < 14; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }

        // ---- online softmax (this lane's query)
        if constexpr (MASKED) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (32 * half + 16 * ks + i >= valid) s[ks][i] = NEG ? INFINITY : -INFINITY;
        }
        float mx = s[0][0];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = NEG ? fminf(mx, s[ks][i]) : fmaxf(mx, s[ks][i]);
        {
            auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
            const float o0 = __uint_as_float(sw[0]), o1 = __uint_as_float(sw[1]);
            mx = NEG ? fminf(o0, o1) : fmaxf(o0, o1);
        }
        const float m_tile = mx * c;
        const bool grow = m_tile > m_run;
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float m_new = grow ? m_tile : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            if constexpr (kDenOnMfma)
                lacc[0] *= alpha;
            else
                l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[db][i] *= alpha;
        }
        // 448 P directly: exp2(logit - (m - log2 448)), one subtraction per
        // tile instead of a multiplication per score; the denominator then
        // sums 448 P and the epilogue divides by it as it stands.
        const float m_bias = m_run - kLog2E4M3Max;
        float rowsum = 0.0f;
        int pk[8];  // 32 e4m3 codes of 448 * P, key order 32*half + j
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[ks][i], c, -m_bias));
                if (MASKED && 32 * half + 16 * ks + i >= valid) p = 0.0f;
                s[ks][i] = p;
                if constexpr (!kDenOnMfma) rowsum += p;
            }
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                int v = __builtin_amdgcn_cvt_pk_fp8_f32(s[ks][4 * w], s[ks][4 * w + 1], 0, false);
                v = __builtin_amdgcn_cvt_pk_fp8_f32(s[ks][4 * w + 2], s[ks][4 * w + 3], v, true);
                pk[4 * ks + w] = v;
            }
        }
        const i32x8_t pop{pk[0], pk[1], pk[2], pk[3], pk[4], pk[5], pk[6], pk[7]};
        if constexpr (kDenOnMfma) {
            lacc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ones, pop, lacc, 0, 0, 0, kScale1, 0, kScale1);
        } else {
            auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(rowsum), __float_as_uint(rowsum), false, false);
            rowsum = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
            l_run += rowsum;
        }

        // ---- O^T += V^T P^T, one 64-key MFMA per 32 dims
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const int d = 32 * db + l32;
            const uint4 lo = *reinterpret_cast<const uint4 *>(vt + d * 64 + 16 * vswz(d, 2 * half));
            const uint4 hi = *reinterpret_cast<const uint4 *>(vt + d * 64 + 16 * vswz(d, 2 * half + 1));
            const i32x8_t vop{static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z),
                              static_cast<int>(lo.w), static_cast<int>(hi.x), static_cast<int>(hi.y),
                              static_cast<int>(hi.z), static_cast<int>(hi.w)};
            acc[db] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vop, pop, acc[db], 0, 0, 0, kScale1, 0, kScale1);
        }
        // Bounded V^T operand window.
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    };
    using Full = std::integral_constant<bool, false>;
    using Partial = std::integral_constant<bool, true>;
    const int full = a.Sk / kBN;  // tiles 0 .. full-1 hold 64 keys
    int tile = 0;
    // Buffer descriptors of this head's K rows and V^T rows (range 0 when unused).
    constexpr int kKChunks = QK_FP8 ? 8 : 16;
    constexpr int kKPerThread = kBN * kKChunks / kThreadsWG;
    const int64_t k_row_bytes = a.ks[2] * (QK_FP8 ? 1 : 2);
    const uint8_t *khead = QK_FP8 ? a.k8 + b * a.ks[0] + h * a.ks[1]
                                  : reinterpret_cast<const uint8_t *>(a.k + b * a.ks[0] + h * a.ks[1]);
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(khead),
                                                                         static_cast<short>(0), a.k_bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(a.v8 + b * a.vs0 + h * a.vs1), static_cast<short>(0), a.v_bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t krs_lo = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(TWO ? a.k8lo + b * a.ks[0] + h * a.ks[1] : khead), static_cast<short>(0), a.k_bytes,
        kBufferWord3);
    // Per-thread byte offsets of the buffer path, fixed for the kernel: wave w's
    // load i writes tile slots 64 (8 i + w) .. +63, 16 bytes per lane, at the
    // wave's LDS base + 16 lane (the direct-to-LDS form of the buffer load);
    // slot s of the K tile is chunk position s % chunks of row s / chunks, so
    // the lane loads the chunk the swizzle puts there (the swizzle is an XOR,
    // its own inverse). Likewise slot s of the V^T tile is position s % 4 of
    // dim row s / 4.
    int kvoff[kKPerThread], vvoff;  // TWO: the lo tile's loads take the hi tile's offsets
#pragma unroll
    for (int i = 0; i < kKPerThread; ++i) {
        const int slot = static_cast<int>(threadIdx.x) + i * kThreadsWG;
        const int r = slot / kKChunks, pos = slot % kKChunks;
        kvoff[i] = r * static_cast<int>(k_row_bytes) + 16 * (QK_FP8 ? kswz8(r, pos) : kswz16(r, pos));
    }
    {
        const int d = static_cast<int>(threadIdx.x) / 4, pos = static_cast<int>(threadIdx.x) % 4;
        vvoff = d * static_cast<int>(a.vs3) + 16 * vswz(d, pos);
    }
    // One full tile from (kc, vc) while the next, also full, goes into (kn, vn).
    auto step = [&](int t, const uint8_t *kc, const uint8_t *vc, uint8_t *kn, uint8_t *vn) {
        if constexpr (BUF) {
            if constexpr (TWO)
                dma_tile_two(krs, krs_lo, vrs, kvoff, vvoff, (t + 1) * kBN * static_cast<int>(k_row_bytes),
                             (t + 1) * kBN, kn, vn);
            else
                dma_tile_pair(krs, vrs, kvoff, vvoff, (t + 1) * kBN * static_cast<int>(k_row_bytes), (t + 1) * kBN,
                              kn, vn);
            attend(Full{}, kc, vc, kBN);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else {
            u32x4_t kr[2], vr;
            load_k_full<QK_FP8, TWO>(a, b, h, (t + 1) * kBN, kr);
            load_v_full(a, b, h, (t + 1) * kBN, vr);
            attend(Full{}, kc, vc, kBN);
            store_k<QK_FP8, TWO>(kn, kr);
            store_v(vn, vr);
        }
        __syncthreads();
    };
    // Main loop: the next tile is full, so its loads need no masks or branches;
    // the buffers alternate, two tiles per iteration.
    const int nmain = full > 1 ? full - 1 : 0;  // tiles 0 .. full-2 (their successors are full)
    for (int t = 0; t < nmain; t += 2) {
        step(t, lds_k0, lds_v0, lds_k1, lds_v1);
        if (t + 1 < nmain) step(t + 1, lds_k1, lds_v1, lds_k0, lds_v0);
    }
    tile = nmain;
    // The last full tile (if any) and the partial tile (if any).
    for (; tile < ntiles; ++tile) {
        const bool odd = tile & 1;
        const uint8_t *kc = odd ? lds_k1 : lds_k0;
        const uint8_t *vc = odd ? lds_v1 : lds_v0;
        uint8_t *kn = odd ? lds_k0 : lds_k1;
        uint8_t *vn = odd ? lds_v0 : lds_v1;
        const int key0 = tile * kBN;
        const int valid = a.Sk - key0 < kBN ? a.Sk - key0 : kBN;
        const bool has_next = tile + 1 < ntiles;
        u32x4_t kr[2], vr;
        if (has_next) {
            const int nvalid = a.Sk - key0 - kBN < kBN ? a.Sk - key0 - kBN : kBN;
            load_k<QK_FP8, TWO>(a, b, h, key0 + kBN, nvalid, kr);
            load_v(a, b, h, key0 + kBN, nvalid, vr);
        }
        if (valid < kBN)
            attend(Partial{}, kc, vc, valid);
        else
            attend(Full{}, kc, vc, kBN);
        if (has_next) {
            store_k<QK_FP8, TWO>(kn, kr);
            store_v(vn, vr);
            __syncthreads();
        }
    }

    if (query >= a.Sq) return;
    const float inv = out_scale / (kDenOnMfma ? lacc[0] : l_run);
    bf16_t *orow = a.o + b * a.os[0] + h * a.os[1] + static_cast<int64_t>(query) * a.os[2];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint2 w;
            w.x = pack2(acc[db][4 * g + 0] * inv, acc[db][4 * g + 1] * inv);
            w.y = pack2(acc[db][4 * g + 2] * inv, acc[db][4 * g + 3] * inv);
            *reinterpret_cast<uint2 *>(orow + 32 * db + 8 * g + 4 * half) = w;
        }
}

// ------------------------------------------------------------------ quantiser

// descale[h] <- 0 (amax accumulator, as uint bits of a non-negative float).
__global__ void zero_kernel(float *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

// Blocks of amax_kernel over all heads: about one resident block per slot of
// the chip. Each block folds its maxima into one atomicMax per head, so the
// same-address device-scope atomics (serialised at the memory side) number
// about kAmaxBlocks instead of one per 256 rows.
constexpr int kAmaxBlocks = 2048;
// Rows per thread per chunk of amax_kernel; a chunk is 16 * kAmaxRows rows.
constexpr int kAmaxRows = 16;

// amax[h] = max |x[:, h, :, :]| over the B * S rows of head h. Block j handles
// head j % H and the chunks j / H, j / H + G, ... (G blocks per head;
// heads vary fastest, so the blocks running together read whole token rows).
// 16 threads per 128-element row; a thread's kAmaxRows row loads per chunk are issued
// before its first comparison (rows past the end re-read the last row, so no
// load sits under a branch); row r splits into (b, s) by the launch-time
// division by S (B * S < 2^31, checked on the host).
__global__ __launch_bounds__(256) void amax_kernel(const bf16_t *x, int64_t s0, int64_t s1, int64_t s2, uint32_t rows,
                                                   uint32_t chunks, int H, uint32_t G, FastDiv by_s, float *amax) {
    constexpr int kRows = kAmaxRows;
    const int h = static_cast<int>(blockIdx.x % static_cast<uint32_t>(H));
    const bf16_t *xh = x + h * s1 + 8 * (threadIdx.x % 16);
    uint32_t m = 0;
    for (uint32_t chunk = blockIdx.x / static_cast<uint32_t>(H); chunk < chunks; chunk += G) {
        const uint32_t r0 = chunk * (16u * kRows) + threadIdx.x / 16;
        U4 v[kRows];
#pragma unroll
        for (int i = 0; i < kRows; ++i) {
            const uint32_t r = r0 + 16u * i < rows ? r0 + 16u * i : rows - 1;
            const uint32_t b = fast_div(r, by_s), ss = r - b * by_s.d;
            v[i] = ld16(xh + static_cast<int64_t>(b) * s0 + static_cast<int64_t>(ss) * s2);
        }
#pragma unroll
        for (int i = 0; i < kRows; ++i) {
            const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = (w[e] << 16) & 0x7fffffffu, hi = w[e] & 0x7fff0000u;
                m = lo > m ? lo : m;
                m = hi > m ? hi : m;
            }
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    __shared__ uint32_t wave_max[4];
    if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x / 64] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t a = wave_max[0] > wave_max[1] ? wave_max[0] : wave_max[1];
        const uint32_t b = wave_max[2] > wave_max[3] ? wave_max[2] : wave_max[3];
        atomicMax(reinterpret_cast<unsigned int *>(amax) + h, a > b ? a : b);
    }
}

// Four values as e4m3fn codes: e4m3(sat((f * pre) * inv)), the scale of
// e4m3_code_scale (pre = 1 except for a head whose amax is below ~1.3e-36).
__device__ __forceinline__ uint32_t quant4(const float f[4], float pre, float inv) {
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = sat_e4m3((f[e] * pre) * inv);
    int v = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
    v = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], v, true);
    return static_cast<uint32_t>(v);
}

// The lo term of a two-term split of four values: with y = sat((f * pre) *
// inv) and hi = e4m3(y) (the codes of quant4), lo = e4m3(sat(16 (y - hi))).
// y - hi is exact in fp32 (hi is y rounded to 4 significant bits, or 0) and
// |16 (y - hi)| <= 256, so the saturation never acts.
__device__ __forceinline__ uint32_t quant4_lo(const float f[4], float pre, float inv, uint32_t hi) {
    float y[4], r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = sat_e4m3((f[e] * pre) * inv);
    const f32x2_t h01 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(hi), false);
    const f32x2_t h23 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(hi), true);
    const float h[4] = {h01[0], h01[1], h23[0], h23[1]};
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = sat_e4m3((y[e] - h[e]) * kLoTermShift);
    int v = __builtin_amdgcn_cvt_pk_fp8_f32(r[0], r[1], 0, false);
    v = __builtin_amdgcn_cvt_pk_fp8_f32(r[2], r[3], v, true);
    return static_cast<uint32_t>(v);
}

// x8 = e4m3(x * 448 / amax_h). D-contiguous output: 16 dims per thread.
// (row, chunk) index i < 2^31 (checked on the host), split by the launch-time
// divisions by S and H. TWO: also the lo term of the two-term split into
// y_lo (the same strides as y).
template <bool TWO>
__global__ __launch_bounds__(256) void quant_rows_kernel(const bf16_t *x, int64_t s0, int64_t s1, int64_t s2,
                                                         uint8_t *y, int64_t t0, int64_t t1, int64_t t2, uint32_t n,
                                                         FastDiv by_s, FastDiv by_h, const float *amax,
                                                         uint8_t *y_lo) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;  // (row, 16-dim chunk)
    if (i >= n) return;
    const int chunk = static_cast<int>(i & 7u);
    const uint32_t row = i >> 3;
    const uint32_t bh = fast_div(row, by_s);
    const int64_t ss = row - bh * by_s.d;
    const uint32_t bbu = fast_div(bh, by_h);
    const int hh = static_cast<int>(bh - bbu * by_h.d);
    const int64_t bb = bbu;
    float pre, inv;
    e4m3_code_scale(amax[hh], pre, inv);
    const bf16_t *src = x + bb * s0 + hh * s1 + ss * s2 + 16 * chunk;
    float f[16];
    u4_to_f8(ld16(src), f);
    u4_to_f8(ld16(src + 8), f + 8);
    uint4 out;
    out.x = quant4(f, pre, inv);
    out.y = quant4(f + 4, pre, inv);
    out.z = quant4(f + 8, pre, inv);
    out.w = quant4(f + 12, pre, inv);
    *reinterpret_cast<uint4 *>(y + bb * t0 + hh * t1 + ss * t2 + 16 * chunk) = out;
    if constexpr (TWO) {
        uint4 lo;
        lo.x = quant4_lo(f, pre, inv, out.x);
        lo.y = quant4_lo(f + 4, pre, inv, out.y);
        lo.z = quant4_lo(f + 8, pre, inv, out.z);
        lo.w = quant4_lo(f + 12, pre, inv, out.w);
        *reinterpret_cast<uint4 *>(y_lo + bb * t0 + hh * t1 + ss * t2 + 16 * chunk) = lo;
    }
}

// 4 x 4 byte transpose: out[e] byte k = in[k] byte e. __builtin_amdgcn_perm(a,
// b, sel) picks result byte i by selector byte i from {b bytes 0-3 as 0-3,
// a bytes 0-3 as 4-7}.
__device__ __forceinline__ void transpose_bytes4(const uint32_t in[4], uint32_t out[4]) {
    const uint32_t p01 = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);  // in0.b0 in1.b0 in0.b1 in1.b1
    const uint32_t q01 = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);  // in0.b2 in1.b2 in0.b3 in1.b3
    const uint32_t p23 = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);
    const uint32_t q23 = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);
    out[0] = __builtin_amdgcn_perm(p23, p01, 0x05040100u);
    out[1] = __builtin_amdgcn_perm(p23, p01, 0x07060302u);
    out[2] = __builtin_amdgcn_perm(q23, q01, 0x05040100u);
    out[3] = __builtin_amdgcn_perm(q23, q01, 0x07060302u);
}

// x8 = e4m3(x * 448 / amax_h) written S-contiguous (V^T layout): a 128-token x
// 128-dim tile per block. Thread t quantises dims 8c..8c+7 (c = t % 16) of
// tokens 4g..4g+3 and 64+4g..64+4g+3 (g = t / 16); each group of 4 tokens is
// byte-transposed in registers into one 4-token word per dim and stored to the
// LDS tile (128-byte rows, 16-byte pieces XOR-swizzled by (d / 8) % 8); the
// tile leaves as 16-byte pieces, 8 per 128-byte output row. Token rows past
// S re-read row S - 1 and are not stored.
// SLOTS: the head's amax is the maximum over its H3_AMAX_SLOTS producer slots
// (fp32 bits of |x|, `slots` with row stride slot_stride), read by every
// block; the head's first block (batch 0, tile 0) writes descale[h] = amax /
// 448 (1 for 0), so the quantisation is this one launch. Otherwise `amax`
// holds the per-head amax and a finalize pass writes the descales.
template <bool SLOTS>
__global__ __launch_bounds__(256) void quant_transposed_kernel(const bf16_t *x, int64_t s0, int64_t s1, int64_t s2,
                                                               uint8_t *y, int64_t t0, int64_t t1, int64_t t3, int H,
                                                               int S, int stiles, const float *amax,
                                                               const uint32_t *slots, int64_t slot_stride,
                                                               float *descale) {
    constexpr int kTok = 128;
    __shared__ __align__(16) uint8_t tile[kD * kTok];
    const int st = blockIdx.x % stiles;
    const int bh = blockIdx.x / stiles;
    const int hh = bh % H, bb = bh / H;
    const int s_base = st * kTok;
    // The scale's load first, then the tile's loads, so that both are in
    // flight before the slot reduction waits for the first.
    uint32_t m = 0;
    float a = 0.0f;
    if constexpr (SLOTS) {
        static_assert(H3_AMAX_SLOTS == 64, "one slot per lane");
        m = slots[hh * slot_stride + (threadIdx.x & 63)];
    } else {
        a = amax[hh];
    }
    const int c = threadIdx.x % 16, g = threadIdx.x / 16;
    const bf16_t *src = x + bb * s0 + hh * s1 + 8 * c;
    U4 v[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int s = min(s_base + 64 * j + 4 * g + k, S - 1);
            v[j][k] = ld16(src + static_cast<int64_t>(s) * s2);
        }
    if constexpr (SLOTS) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const uint32_t o = __shfl_xor(m, off, 64);
            m = o > m ? o : m;
        }
        a = __uint_as_float(m);
        if (bh < H && st == 0 && threadIdx.x == 0) descale[hh] = a > 0.0f ? a / kE4M3Max : 1.0f;
    }
    float pre, inv;
    e4m3_code_scale(a, pre, inv);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float f[8];
            u4_to_f8(v[j][k], f);
            lo[k] = quant4(f, pre, inv);
            hi[k] = quant4(f + 4, pre, inv);
        }
        uint32_t w[8];
        transpose_bytes4(lo, w);
        transpose_bytes4(hi, w + 4);
        const int piece = 4 * j + g / 4;  // 16-byte piece of the 128-token row
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int d = 8 * c + e;
            *reinterpret_cast<uint32_t *>(tile + d * kTok + 16 * (piece ^ (c & 7)) + 4 * (g % 4)) = w[e];
        }
    }
    __syncthreads();
    uint8_t *dst = y + bb * t0 + hh * t1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int p = threadIdx.x + 256 * i;
        const int d = p / 8, q = p % 8;
        const uint4 out = *reinterpret_cast<const uint4 *>(tile + d * kTok + 16 * (q ^ ((d / 8) & 7)));
        const int s = s_base + 16 * q;
        uint8_t *row = dst + static_cast<int64_t>(d) * t3 + s;
        if (s + 16 <= S) {
            *reinterpret_cast<uint4 *>(row) = out;
        } else if (s < S) {
            const uint32_t ww[4] = {out.x, out.y, out.z, out.w};
            for (int e = 0; e < S - s; ++e) row[e] = static_cast<uint8_t>(ww[e / 4] >> (8 * (e % 4)));
        }
    }
}

// amax[h] = the maximum over the head's H3_AMAX_SLOTS slots (fp32 bits of |x|,
// compared as integers like amax_kernel's). One 64-lane wave per head.
__global__ __launch_bounds__(64) void reduce_slots_kernel(const uint32_t *slots, int64_t head_stride,
                                                          float *amax) {
    static_assert(H3_AMAX_SLOTS == 64, "one slot per lane");
    uint32_t m = slots[blockIdx.x * head_stride + threadIdx.x];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    if (threadIdx.x == 0) amax[blockIdx.x] = __uint_as_float(m);
}

// descale[h] = amax_h / 448 (1 for an all-zero head).
__global__ void finalize_kernel(float *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = p[i] > 0.0f ? p[i] / kE4M3Max : 1.0f;
}

template <bool QK_FP8, bool TWO = false>
int launch_fp8(hipStream_t stream, const Fp8Args &a0) {
    Fp8Args a = a0;
    a.qblocks = (a.Sq + kBM - 1) / kBM;
    const int64_t grid = static_cast<int64_t>(a.B) * a.H * a.qblocks;
    if (grid > static_cast<int64_t>(std::numeric_limits<int32_t>::max())) return kInvalid;
    // Buffer loads when one head's K rows (non-overlapping) and V^T rows (each
    // at least Sk bytes apart) fit a 31-bit byte range.
    const int64_t esize = QK_FP8 ? 1 : 2, k_row = a.ks[2] * esize;
    const int64_t k_ext = k_row >= kD * esize ? (static_cast<int64_t>(a.Sk) - 1) * k_row + kD * esize : -1;
    const int64_t v_ext = a.vs3 >= a.Sk ? (kD - 1) * a.vs3 + a.Sk : -1;
    const bool buf = k_ext > 0 && v_ext > 0 && k_ext < (int64_t{1} << 31) && v_ext < (int64_t{1} << 31);
    a.k_bytes = buf ? static_cast<int>(k_ext) : 0;
    a.v_bytes = buf ? static_cast<int>(v_ext) : 0;
    const unsigned g = static_cast<unsigned>(grid);
    if (a.c < 0.0f) {
        if (buf)
            attention_fp8_kernel<QK_FP8, true, true, TWO><<<g, kThreadsWG, 0, stream>>>(a);
        else
            attention_fp8_kernel<QK_FP8, true, false, TWO><<<g, kThreadsWG, 0, stream>>>(a);
    } else {
        if (buf)
            attention_fp8_kernel<QK_FP8, false, true, TWO><<<g, kThreadsWG, 0, stream>>>(a);
        else
            attention_fp8_kernel<QK_FP8, false, false, TWO><<<g, kThreadsWG, 0, stream>>>(a);
    }
    return launch_status();
}

// Shared host checks: o [B, H, Sq, 128] bf16 (D unit-stride, 16-byte rows);
// v8 [B, H, Sk, 128] with unit stride on S; descales [H] contiguous.
int check_common(const View<4> &qshape, const View<4> &kshape, const View<4> &v8, const View<4> &o,
                 const View<1> *descales[], int ndescale, Fp8Args &a) {
    if (!same_shape(qshape, o) || !same_shape(kshape, v8)) return kInvalid;
    if (qshape.shape[0] != kshape.shape[0] || qshape.shape[1] != kshape.shape[1] || qshape.shape[3] != kD ||
        kshape.shape[3] != kD)
        return kInvalid;
    if (qshape.shape[2] > kMaxSeqLen || kshape.shape[2] > kMaxSeqLen) return kInvalid;
    if (!rows_vec16(o, 2)) return kInvalid;
    if (v8.shape[2] > 1 && v8.stride[2] != 1) return kInvalid;
    if ((reinterpret_cast<uintptr_t>(v8.data) & 15) != 0 || (v8.stride[3] % 16) != 0 ||
        (v8.shape[0] > 1 && v8.stride[0] % 16 != 0) || (v8.shape[1] > 1 && v8.stride[1] % 16 != 0))
        return kInvalid;
    for (int i = 0; i < ndescale; ++i) {
        const View<1> &d = *descales[i];
        if (d.shape[0] != qshape.shape[1] || (d.shape[0] > 1 && d.stride[0] != 1)) return kInvalid;
    }
    a.v8 = reinterpret_cast<const uint8_t *>(v8.data);
    a.vs0 = v8.stride[0];
    a.vs1 = v8.stride[1];
    a.vs3 = v8.stride[3];
    a.o = reinterpret_cast<bf16_t *>(o.data);
    for (int i = 0; i < 3; ++i) a.os[i] = o.stride[i];
    a.B = static_cast<int>(qshape.shape[0]);
    a.H = static_cast<int>(qshape.shape[1]);
    a.Sq = static_cast<int>(qshape.shape[2]);
    a.Sk = static_cast<int>(kshape.shape[2]);
    return 0;
}

// The quantiser chain on the caller's stream: the per-head amax into
// `descale` (amax_kernel after a clear, or reduce_slots_kernel from a
// producer's slots), the code pass, then descale = amax / 448 in place. Every
// check comes before the first launch, so a rejected call leaves `descale`
// untouched. check_only: the checks alone (0 or kInvalid), no HIP call.
// x8_lo (may be null): the lo codes of the two-term split, D-contiguous with
// x8's strides (x8 then D-contiguous too; not with amax_slots).
int launch_quantize(NineToothedStream stream, const NineToothedTensor &x, const NineToothedTensor &x8,
                    const NineToothedTensor &descale, const NineToothedTensor *amax_slots,
                    bool check_only = false, const NineToothedTensor *x8_lo = nullptr) {
    View<4> xv, yv, lv;
    View<1> dv;
    View<2> sv;
    if (!load_view(x, 2, xv) || !load_view(x8, 1, yv) || !load_view(descale, 4, dv)) return kInvalid;
    if (amax_slots != nullptr && !load_view(*amax_slots, 4, sv)) return kInvalid;
    if (x8_lo != nullptr) {
        if (amax_slots != nullptr || !load_view(*x8_lo, 1, lv) || !same_shape(lv, yv) || !rows_vec16(lv, 1) ||
            !rows_vec16(yv, 1))
            return kInvalid;
        for (int i = 0; i < 4; ++i)
            if (lv.shape[i] > 1 && lv.stride[i] != yv.stride[i]) return kInvalid;
    }
    if (!same_shape(xv, yv) || xv.shape[3] != kD || dv.shape[0] != xv.shape[1]) return kInvalid;
    if (dv.shape[0] > 1 && dv.stride[0] != 1) return kInvalid;
    // Slots are contiguous per head: H3_AMAX_SLOTS words, heads H3_AMAX_SLOTS apart.
    if (amax_slots != nullptr && (sv.shape[0] != xv.shape[1] || sv.shape[1] != H3_AMAX_SLOTS || sv.stride[1] != 1 ||
                                  (sv.shape[0] > 1 && sv.stride[0] != H3_AMAX_SLOTS)))
        return kInvalid;
    if (!rows_vec16(xv, 2)) return kInvalid;
    const int B = static_cast<int>(xv.shape[0]), H = static_cast<int>(xv.shape[1]), S = static_cast<int>(xv.shape[2]);
    if (H == 0) return 0;
    const bool d_contig = rows_vec16(yv, 1);
    const bool s_contig = (S <= 1 || yv.stride[2] == 1) && (reinterpret_cast<uintptr_t>(yv.data) & 15) == 0 &&
                          yv.stride[3] % 16 == 0 && (B <= 1 || yv.stride[0] % 16 == 0) &&
                          (H <= 1 || yv.stride[1] % 16 == 0);
    if (!d_contig && !s_contig) return kInvalid;
    const int64_t rows = static_cast<int64_t>(B) * S;
    const int64_t n = rows * H * 8;  // (row, 16-dim chunk) pairs of quant_rows_kernel
    if (n >= (int64_t{1} << 31)) return kInvalid;
    if (check_only) return 0;
    hipStream_t st = as_stream(stream);
    float *amax = reinterpret_cast<float *>(dv.data);
    const uint32_t *slots = amax_slots != nullptr ? reinterpret_cast<const uint32_t *>(sv.data) : nullptr;
    if (slots != nullptr && s_contig && !d_contig && rows > 0) {
        // One launch: the V^T code pass reduces the slots and writes the descales.
        const int stiles = (S + 127) / 128;
        quant_transposed_kernel<true><<<static_cast<unsigned>(static_cast<int64_t>(B) * H * stiles), 256, 0, st>>>(
            reinterpret_cast<const bf16_t *>(xv.data), xv.stride[0], xv.stride[1], xv.stride[2],
            reinterpret_cast<uint8_t *>(yv.data), yv.stride[0], yv.stride[1], yv.stride[3], H, S, stiles, nullptr,
            slots, sv.stride[0], amax);
        return launch_status();
    }
    if (slots != nullptr)
        reduce_slots_kernel<<<H, 64, 0, st>>>(slots, sv.stride[0], amax);
    else
        zero_kernel<<<(H + 255) / 256, 256, 0, st>>>(amax, H);
    if (rows > 0) {
        const FastDiv by_s = make_fastdiv(static_cast<uint32_t>(S)), by_h = make_fastdiv(static_cast<uint32_t>(H));
        if (amax_slots == nullptr) {
            const int64_t chunks = (rows + 16 * kAmaxRows - 1) / (16 * kAmaxRows);
            const int64_t per = (chunks * H + kAmaxBlocks - 1) / kAmaxBlocks;  // chunks per block
            const int64_t G = (chunks + per - 1) / per;                  // blocks per head
            amax_kernel<<<static_cast<unsigned>(G * H), 256, 0, st>>>(
                reinterpret_cast<const bf16_t *>(xv.data), xv.stride[0], xv.stride[1], xv.stride[2],
                static_cast<uint32_t>(rows), static_cast<uint32_t>(chunks), H, static_cast<uint32_t>(G), by_s, amax);
        }
        if (x8_lo != nullptr) {
            quant_rows_kernel<true><<<static_cast<unsigned>((n + 255) / 256), 256, 0, st>>>(
                reinterpret_cast<const bf16_t *>(xv.data), xv.stride[0], xv.stride[1], xv.stride[2],
                reinterpret_cast<uint8_t *>(yv.data), yv.stride[0], yv.stride[1], yv.stride[2],
                static_cast<uint32_t>(n), by_s, by_h, amax, reinterpret_cast<uint8_t *>(lv.data));
        } else if (d_contig) {
            quant_rows_kernel<false><<<static_cast<unsigned>((n + 255) / 256), 256, 0, st>>>(
                reinterpret_cast<const bf16_t *>(xv.data), xv.stride[0], xv.stride[1], xv.stride[2],
                reinterpret_cast<uint8_t *>(yv.data), yv.stride[0], yv.stride[1], yv.stride[2],
                static_cast<uint32_t>(n), by_s, by_h, amax, nullptr);
        } else {
            const int stiles = (S + 127) / 128;
            quant_transposed_kernel<false><<<static_cast<unsigned>(static_cast<int64_t>(B) * H * stiles), 256, 0, st>>>(
                reinterpret_cast<const bf16_t *>(xv.data), xv.stride[0], xv.stride[1], xv.stride[2],
                reinterpret_cast<uint8_t *>(yv.data), yv.stride[0], yv.stride[1], yv.stride[3], H, S, stiles, amax,
                nullptr, 0, nullptr);
        }
    }
    finalize_kernel<<<(H + 255) / 256, 256, 0, st>>>(amax, H);
    return launch_status();
}

}  // namespace

int check_quantize_fp8_per_head(const NineToothedTensor &x, const NineToothedTensor &x8,
                                const NineToothedTensor &descale) {
    return launch_quantize(nullptr, x, x8, descale, nullptr, true);
}

}  // namespace h3

using namespace h3;

extern "C" {

NineToothedResult launch_h3_quantize_fp8_per_head(NineToothedStream stream, NineToothedTensor x,
                                                  NineToothedTensor x8, NineToothedTensor descale) {
    return launch_quantize(stream, x, x8, descale, nullptr);
}

NineToothedResult launch_h3_quantize_fp8_two_term(NineToothedStream stream, NineToothedTensor x,
                                                   NineToothedTensor x8, NineToothedTensor x8_lo,
                                                   NineToothedTensor descale) {
    return launch_quantize(stream, x, x8, descale, nullptr, false, &x8_lo);
}

NineToothedResult launch_h3_quantize_fp8_per_head_slots(NineToothedStream stream, NineToothedTensor x,
                                                        NineToothedTensor amax_slots, NineToothedTensor x8,
                                                        NineToothedTensor descale) {
    return launch_quantize(stream, x, x8, descale, &amax_slots);
}

NineToothedResult launch_h3_full_attention_fp8(NineToothedStream stream, NineToothedTensor q8, NineToothedTensor k8,
                                               NineToothedTensor v8, NineToothedTensor q_descale,
                                               NineToothedTensor k_descale, NineToothedTensor v_descale,
                                               NineToothedTensor scale, NineToothedTensor o) {
    View<4> qv, kv, vv, ov;
    View<1> qd, kd, vd;
    double sc;
    if (!load_view(q8, 1, qv) || !load_view(k8, 1, kv) || !load_view(v8, 1, vv) || !load_view(o, 2, ov) ||
        !load_view(q_descale, 4, qd) || !load_view(k_descale, 4, kd) || !load_view(v_descale, 4, vd) ||
        !load_scalar(scale, sc))
        return kInvalid;
    Fp8Args a{};
    const View<1> *ds[3] = {&qd, &kd, &vd};
    if (check_common(qv, kv, vv, ov, ds, 3, a) != 0) return kInvalid;
    if (!rows_vec16(qv, 1) || !rows_vec16(kv, 1)) return kInvalid;
    if (qv.shape[0] == 0 || qv.shape[1] == 0 || qv.shape[2] == 0) return 0;
    if (kv.shape[2] == 0) return kInvalid;
    a.q8 = reinterpret_cast<const uint8_t *>(qv.data);
    a.k8 = reinterpret_cast<const uint8_t *>(kv.data);
    for (int i = 0; i < 3; ++i) {
        a.qs[i] = qv.stride[i];
        a.ks[i] = kv.stride[i];
    }
    a.q_descale = reinterpret_cast<const float *>(qd.data);
    a.k_descale = reinterpret_cast<const float *>(kd.data);
    a.v_descale = reinterpret_cast<const float *>(vd.data);
    a.c = static_cast<float>(static_cast<float>(sc) * kLog2e);
    return launch_fp8<true>(as_stream(stream), a);
}

NineToothedResult launch_h3_full_attention_fp8x2(NineToothedStream stream, NineToothedTensor q8,
                                                 NineToothedTensor q8_lo, NineToothedTensor k8,
                                                 NineToothedTensor k8_lo, NineToothedTensor v8,
                                                 NineToothedTensor q_descale, NineToothedTensor k_descale,
                                                 NineToothedTensor v_descale, NineToothedTensor scale,
                                                 NineToothedTensor o) {
    View<4> qv, qlv, kv, klv, vv, ov;
    View<1> qd, kd, vd;
    double sc;
    if (!load_view(q8, 1, qv) || !load_view(q8_lo, 1, qlv) || !load_view(k8, 1, kv) || !load_view(k8_lo, 1, klv) ||
        !load_view(v8, 1, vv) || !load_view(o, 2, ov) || !load_view(q_descale, 4, qd) ||
        !load_view(k_descale, 4, kd) || !load_view(v_descale, 4, vd) || !load_scalar(scale, sc))
        return kInvalid;
    Fp8Args a{};
    const View<1> *ds[3] = {&qd, &kd, &vd};
    if (check_common(qv, kv, vv, ov, ds, 3, a) != 0) return kInvalid;
    // The lo codes share the hi codes' shape and strides.
    if (!same_shape(qv, qlv) || !same_shape(kv, klv)) return kInvalid;
    for (int i = 0; i < 4; ++i)
        if ((qv.shape[i] > 1 && qlv.stride[i] != qv.stride[i]) || (kv.shape[i] > 1 && klv.stride[i] != kv.stride[i]))
            return kInvalid;
    if (!rows_vec16(qv, 1) || !rows_vec16(kv, 1) || !rows_vec16(qlv, 1) || !rows_vec16(klv, 1)) return kInvalid;
    if (qv.shape[0] == 0 || qv.shape[1] == 0 || qv.shape[2] == 0) return 0;
    if (kv.shape[2] == 0) return kInvalid;
    a.q8 = reinterpret_cast<const uint8_t *>(qv.data);
    a.k8 = reinterpret_cast<const uint8_t *>(kv.data);
    a.q8lo = reinterpret_cast<const uint8_t *>(qlv.data);
    a.k8lo = reinterpret_cast<const uint8_t *>(klv.data);
    for (int i = 0; i < 3; ++i) {
        a.qs[i] = qv.stride[i];
        a.ks[i] = kv.stride[i];
    }
    a.q_descale = reinterpret_cast<const float *>(qd.data);
    a.k_descale = reinterpret_cast<const float *>(kd.data);
    a.v_descale = reinterpret_cast<const float *>(vd.data);
    a.c = static_cast<float>(static_cast<float>(sc) * kLog2e);
    return launch_fp8<true, true>(as_stream(stream), a);
}

NineToothedResult launch_h3_full_attention_fp8pv(NineToothedStream stream, NineToothedTensor q, NineToothedTensor k,
                                                 NineToothedTensor v8, NineToothedTensor v_descale,
                                                 NineToothedTensor scale, NineToothedTensor o) {
    View<4> qv, kv, vv, ov;
    View<1> vd;
    double sc;
    if (!load_view(q, 2, qv) || !load_view(k, 2, kv) || !load_view(v8, 1, vv) || !load_view(o, 2, ov) ||
        !load_view(v_descale, 4, vd) || !load_scalar(scale, sc))
        return kInvalid;
    Fp8Args a{};
    const View<1> *ds[1] = {&vd};
    if (check_common(qv, kv, vv, ov, ds, 1, a) != 0) return kInvalid;
    if (!rows_vec16(qv, 2) || !rows_vec16(kv, 2)) return kInvalid;
    if (qv.shape[0] == 0 || qv.shape[1] == 0 || qv.shape[2] == 0) return 0;
    if (kv.shape[2] == 0) return kInvalid;
    a.q = reinterpret_cast<const bf16_t *>(qv.data);
    a.k = reinterpret_cast<const bf16_t *>(kv.data);
    for (int i = 0; i < 3; ++i) {
        a.qs[i] = qv.stride[i];
        a.ks[i] = kv.stride[i];
    }
    a.v_descale = reinterpret_cast<const float *>(vd.data);
    a.c = static_cast<float>(static_cast<float>(sc) * kLog2e);
    return launch_fp8<false>(as_stream(stream), a);
}

}  // extern "C"
