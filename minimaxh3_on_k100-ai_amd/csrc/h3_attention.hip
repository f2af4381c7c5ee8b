// Non-causal full attention forward for gfx950 (CDNA4), bf16 in/out, fp32
// softmax state: the MI355X counterpart of the reference's NineToothed kernel
// (tools/h3_attention.py:25-41, `fp32_qk` numerics).
//
// Work decomposition (both kernels below)
//   - one 512-thread workgroup (8 waves, two per SIMD) per (batch, head,
//     256-query block); the workgroup order is remapped so the blocks
//     dispatched to one XCD are consecutive (same head) and share that XCD's
//     L2 for the K/V stream;
//   - each wave owns 32 queries and keeps its Q^T operands in registers for
//     the whole key loop; all of a wave's state (Q, scores, O accumulators)
//     lives in arch VGPRs (at most the 256 a wave gets at two waves per SIMD),
//     so the softmax never shuttles values through AGPRs;
//   - K/V tiles of 64 keys go from HBM straight into double-buffered LDS
//     (buffer loads with the LDS destination), in rows of 256 bytes whose
//     16-byte chunks are XOR-swizzled so every operand read is bank-conflict
//     free (below); the next tile's loads run during the current tile's work;
//   - one workgroup fills a CU, so a launch runs in rounds of one workgroup
//     per CU. When the last round would be about 2/3 to 3/4 full, it runs
//     instead as a full round of 192-query units (attention16_small_kernel).
//     When it is otherwise partly filled and a workspace is given, the units
//     of that round are split along the keys into pieces that fill whole
//     rounds (SPLIT); each piece leaves its unnormalised O, reference maximum
//     and denominator in the workspace and a merge kernel combines them (the
//     same algebra as the online rescale).
//
// attention16_kernel (D = 128 on the buffer path: the configurations) runs on
// v_mfma_f32_16x16x32_bf16 and keeps one reference maximum per unit (its
// layout and numerics are described above it). attention_fwd_kernel runs on
// v_mfma_f32_32x32x16_bf16 with the exact online rescale and serves D = 72
// and K/V views outside the buffer path:
//
// MFMA formulation (v_mfma_f32_32x32x16_bf16; A row = lane % 32, B column =
// lane % 32, accumulator register i of lane l holds row 8*(i/4) + 4*(l/32) + i%4)
//   - S^T = K Q^T: A = 32 keys x 16 dims of K from LDS, B = Q^T from registers.
//     Each lane therefore accumulates the scores of ONE query (its column), so
//     the softmax max/sum are per-lane plus one exchange with lane l^32.
//   - The A operand reads K row pi(m) for MFMA row m, pi swapping bits 2 and 3.
//     With that, accumulator register i of lane l holds key
//     16*(i/8) + 8*(l/32) + i%8 of its 32-key block, which is exactly the
//     B-operand layout (k = 8*(l/32) + j) of the next product:
//   - O^T += V^T P^T: A = 32 dims x 16 keys of V^T, read from the row-major V
//     tile with ds_read_b64_tr_b16; B = the bf16-rounded P^T registers. The
//     O^T accumulators of a lane again belong to its own query, so the online
//     rescale is a per-lane scalar.
// Numerics follow the reference: fp32 logits scaled by scale*log2(e), exp2
// online softmax, bf16 P in the P.V product, fp32 P in the denominator, fp32
// accumulation, o = acc / denominator rounded to bf16.
#include <atomic>
#include <type_traits>

#include "h3_common.hpp"
#include "h3_internal.hpp"

namespace h3 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

constexpr int kD = 128;           // head dim
constexpr int kWaves = 8;                     // waves per workgroup (2 per SIMD)
constexpr int kQS = 1;                        // 32-query MFMA blocks per wave
constexpr int kThreadsWG = 64 * kWaves;
constexpr int kBM = 32 * kQS * kWaves;        // queries per workgroup
constexpr int kBN = 64;           // keys per tile
// LDS tiles: 64 rows of 256 bytes (16 chunks of 8 dims), unpadded, so that a
// wave's 64-lane buffer-to-LDS load fills 4 whole rows. The 16-byte chunk c of
// row r sits at slot c ^ swz(r), against 64 banks x 4 bytes:
//   K: swz(r) = r & 15 -> the 16 rows one 16-lane ds_read_b128 pass reads (same
//      chunk) land on 16 distinct slots, every bank once;
//   V: swz(r) = 4 (r & 3) -> each 32-lane ds_read_b64_tr_b16 pass reads 4 rows
//      x 4 chunks, 16 distinct slots, every bank once.
constexpr int kRow = kD;
constexpr int kTileElems = kBN * kRow;
constexpr int kLoadRows = kBN * 16 / kThreadsWG;  // 16-byte chunks per thread per tile
static_assert(kBN * 16 % kThreadsWG == 0, "a tile is an exact number of chunks per thread");
static_assert(kLoadRows * 64 / 16 * kWaves == kBN, "each wave's loads fill whole rows");
__device__ __forceinline__ int swz_k(int row) { return row & 15; }
// The 16-dim k-steps of Q K^T and the 32-dim blocks of O^T a DIM-wide head
// needs (dims past DIM are zero in Q, K and V): 8 and 4 at DIM = 128, 5 and 3
// at DIM = 72.
template <int DIM>
constexpr int kk_steps() { return (DIM + 15) / 16; }
template <int DIM>
constexpr int dim_blocks() { return (DIM + 31) / 32; }
__device__ __forceinline__ int swz_v(int row) { return 4 * (row & 3); }
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
    const bf16_t *q, *k, *v;
    bf16_t *o;
    int64_t qs[3], ks[3], vs[3], os[3];  // element strides of B, H, S
    int64_t qd, kd, vd, od;               // element strides of D (1 except on the element-strided path)
    int B, H, Sq, Sk;
    int qblocks;                          // ceil(Sq / kBM)
    float c;                              // scale * log2(e)
    int k_bytes, v_bytes;                 // buffer-load path: byte extent of one head's K / V rows
    bool prescale;                        // q enters the product as bf16(c q) and the logits are not rescaled
    // SPLIT kernels: workgroups [0, n_full) run whole units (b, h, 256-query
    // block) 0 .. n_full-1; workgroup n_full + j runs piece p of tail unit
    // n_full + u, (p, u) = (lp / n_tail, lp % n_tail) for lp the XCD-remapped
    // j: key tiles [p T / split, (p + 1) T / split) of the unit's T tiles.
    int n_full, n_tail, split;
    float *ws;                            // the partials (layout at kWsSlotAcc)
    // SMALL kernels: workgroups [0, n_big) run 256-query units and workgroups
    // [n_big, n_big + n_small) 192-query units, each range XCD-remapped on its
    // own, so the 192-query units make up the last round. A head (b H + h)
    // starts with its 256-query units and ends with its 192-query ones: heads
    // 0 .. sm_k-1 hold sm_big0 and sm_small0 of them, head sm_k sm_big1 and
    // sm_small1, the others qblocks 256-query units. Units are numbered head
    // by head within each range.
    int n_big, n_small, sm_k, sm_big0, sm_small0, sm_big1, sm_small1;
};

constexpr int kSmallBM = 192;  // queries of a SMALL launch's last-round units

struct SmallUnit {
    int bh, q0;  // head (b H + h) and first query
    bool small;  // a 192-query unit
};

// The unit of SMALL workgroup x.
__device__ __forceinline__ SmallUnit small_plan_unit(const AttnArgs &a, int x);

// Workspace of the SPLIT kernels, per piece slot (u split + p): the
// unnormalised O as [256 queries][128 dims] floats, then, after all slots'
// O, the reference maximum and the denominator as [256 queries][2] floats.
constexpr int kWsSlotAcc = kBM * kD;
constexpr int kWsSlotMl = kBM * 2;
constexpr int64_t kWsSlotBytes = static_cast<int64_t>(kWsSlotAcc + kWsSlotMl) * 4;
constexpr int kMaxSplit = 8;

// The dword-3 word of a raw buffer descriptor on gfx9 (CDNA): no format
// conversion, bounds checked against num_records in bytes.
constexpr int kBufferWord3 = 0x00020000;
// A per-lane buffer offset past any descriptor range here (ranges and tile
// offsets stay below 2^31, so offset + tile offset cannot wrap).
constexpr int kBeyondRange = 0x40000000;

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4 &v) { return __builtin_bit_cast(bf16x8_t, v); }

// Maps the hardware workgroup id to a logical one so that each XCD (ids
// dispatched round-robin over 8 XCDs) receives a contiguous logical range.
__device__ __forceinline__ int xcd_remap(int x, int total) {
    const int per = total / 8, rem = total % 8;
    const int xcd = x % 8, slot = x / 8;
    return xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

__device__ __forceinline__ SmallUnit small_plan_unit(const AttnArgs &a, int x) {
    if (x < a.n_big) {
        int i = xcd_remap(x, a.n_big);
        const int c0 = a.sm_k * a.sm_big0;
        if (i < c0) return {i / a.sm_big0, (i % a.sm_big0) * kBM, false};
        i -= c0;
        if (i < a.sm_big1) return {a.sm_k, i * kBM, false};
        i -= a.sm_big1;
        return {a.sm_k + 1 + i / a.qblocks, (i % a.qblocks) * kBM, false};
    }
    int i = xcd_remap(x - a.n_big, a.n_small);
    const int c0 = a.sm_k * a.sm_small0;
    if (i < c0) return {i / a.sm_small0, a.sm_big0 * kBM + (i % a.sm_small0) * kSmallBM, true};
    i -= c0;
    return {a.sm_k, a.sm_big1 * kBM + i * kSmallBM, true};
}

// Thread t's share of a 64-key tile: wave w's i-th load (i < kLoadRows) fills
// tile rows 4 (kLoadRows w + i) .. +3, one row per 16 lanes; lane l fills slot
// l % 16 of its row, which holds the row's chunk (l % 16) ^ swz(row).
__device__ __forceinline__ int tile_row(int i) {
    return 4 * (kLoadRows * static_cast<int>(threadIdx.x >> 6) + i) + static_cast<int>(threadIdx.x & 63) / 16;
}
template <bool IS_K>
__device__ __forceinline__ int tile_chunk(int row) {
    return static_cast<int>(threadIdx.x & 15) ^ (IS_K ? swz_k(row) : swz_v(row));
}

// Global -> registers for one 64-key tile (the pointer path). Rows past
// `valid` re-read row valid-1: every load is issued unconditionally (a load
// under a branch is waited for before the branch closes), and the softmax
// masks those keys (their scores become -inf and their probabilities exactly
// 0, which leaves the finite V rows without effect). DIM < 128: chunks past
// DIM / 8 read the row's last chunk and are replaced by zeros.
//
// GEN (the element-strided path): the row's 8 elements are read one by one
// with the head-dim stride d_stride, from any 2-byte aligned address.
template <bool IS_K, int DIM, bool GEN = false>
__device__ __forceinline__ void load_tile(const bf16_t *base, int64_t s_stride, int key0, int valid,
                                          u32x4_t (&reg)[kLoadRows], int64_t d_stride = 1) {
#pragma unroll
    for (int r = 0; r < kLoadRows; ++r) {
        const int row0 = tile_row(r);
        const int row = row0 < valid ? row0 : valid - 1;
        const int chunk = tile_chunk<IS_K>(row0), cc = chunk < DIM / 8 ? chunk : DIM / 8 - 1;
        const bf16_t *src = base + static_cast<int64_t>(key0 + row) * s_stride;
        u32x4_t v;
        if constexpr (GEN) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2)
                w[e / 2] = static_cast<uint32_t>(src[(cc * 8 + e) * d_stride]) |
                           (static_cast<uint32_t>(src[(cc * 8 + e + 1) * d_stride]) << 16);
            v = u32x4_t{w[0], w[1], w[2], w[3]};
        } else {
            v = *reinterpret_cast<const u32x4_t *>(src + cc * 8);
        }
        reg[r] = chunk < DIM / 8 ? v : u32x4_t{0u, 0u, 0u, 0u};
    }
}

// Eight consecutive head-dim elements of a row from d0 on, as packed bf16:
// a 16-byte load, or (GEN) element loads with the head-dim stride.
template <bool GEN>
__device__ __forceinline__ uint4 load_row8(const bf16_t *row, int d0, int64_t d_stride) {
    if constexpr (GEN) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2)
            w[e / 2] = static_cast<uint32_t>(row[(d0 + e) * d_stride]) |
                       (static_cast<uint32_t>(row[(d0 + e + 1) * d_stride]) << 16);
        return make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        return *reinterpret_cast<const uint4 *>(row + d0);
    }
}

// Registers -> the LDS tile: load r of wave w is one contiguous 1 KiB run.
__device__ __forceinline__ void store_tile(bf16_t *lds, const u32x4_t (&reg)[kLoadRows]) {
#pragma unroll
    for (int r = 0; r < kLoadRows; ++r)
        *reinterpret_cast<u32x4_t *>(lds + 4 * kRow * (kLoadRows * static_cast<int>(threadIdx.x >> 6) + r) +
                                     8 * static_cast<int>(threadIdx.x & 63)) = reg[r];
}

// Global -> LDS directly (the buffer path): each buffer load writes lane l's
// 16 bytes at the wave's LDS base + 16 l, with per-thread byte offsets fixed
// for the kernel (voff) plus the tile's uniform byte offset (soff). Rows past
// the head's last key fall outside the descriptor's range and read as zero
// (their scores are masked), so no address is clamped per tile. The loads
// complete asynchronously: the caller waits on vmcnt before the barrier that
// publishes the tile.
__device__ __forceinline__ void dma_tile(__amdgpu_buffer_rsrc_t rs, const int (&voff)[kLoadRows], int soff,
                                         bf16_t *lds) {
    const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
#pragma unroll
    for (int r = 0; r < kLoadRows; ++r)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (__attribute__((address_space(3))) void *)(lds + 4 * kRow * (kLoadRows * w + r)), 16, voff[r], soff, 0,
            0);
}

// One 64-key tile: S^T = K Q^T, online softmax, O^T += V^T P^T. MASK marks the
// last, partial tile (keys >= valid are excluded).
// kidx: element index of this lane's K operand chunk for k-step 0 (k-step kk
// is kidx ^ 16 kk); vidx: of its V^T operand for dim block 0 (block db is
// vidx ^ 32 db).
template <bool MASK, bool NEG, int DIM>
__device__ __forceinline__ void attend_tile(const bf16_t *kt, const bf16_t *vt, int valid, const bf16x8_t (&qreg)[kQS][8],
                                            f32x16_t (&acc)[4][kQS], float (&m_run)[kQS], float (&l_run)[kQS], float c,
                                            int kidx, int half, int vidx) {
    f32x16_t s[2][kQS];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int qs = 0; qs < kQS; ++qs)
#pragma unroll
            for (int i = 0; i < 16; ++i) s[ks][qs][i] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < kk_steps<DIM>(); ++kk) {
            const bf16x8_t kop = as_bf16x8(*reinterpret_cast<const uint4 *>(kt + 32 * ks * kRow + (kidx ^ (16 * kk))));
#pragma unroll
            for (int qs = 0; qs < kQS; ++qs)
                s[ks][qs] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop, qreg[qs][kk], s[ks][qs], 0, 0, 0);
        }
    }
    // Rolling window of K operand reads: two reads ahead of the MFMAs, so only
    // a few operands occupy VGPRs at any time.
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int i = 0; i < 2 * kk_steps<DIM>() - 2; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, kQS, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * kQS, 0);

    bf16x8_t pop[kQS][4];  // P^T operands: query block x 16-key step
#pragma unroll
    for (int qs = 0; qs < kQS; ++qs) {
        if constexpr (MASK) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = 32 * ks + 16 * (i / 8) + 8 * half + (i % 8);
                    if (key >= valid) s[ks][qs][i] = NEG ? INFINITY : -INFINITY;
                }
        }
        float mx = s[0][qs][0];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = NEG ? fminf(mx, s[ks][qs][i]) : fmaxf(mx, s[ks][qs][i]);
        {
            auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
            const float o0 = __uint_as_float(sw[0]), o1 = __uint_as_float(sw[1]);
            mx = NEG ? fminf(o0, o1) : fmaxf(o0, o1);
        }
        const float m_tile = mx * c;  // this tile's row maximum in logit units
        // Exact running max as in the reference; the accumulators are only
        // touched when some row's max grew (alpha == 1 exactly otherwise).
        const bool grow = m_tile > m_run[qs];
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float m_new = grow ? m_tile : m_run[qs];
            const float alpha = __builtin_amdgcn_exp2f(m_run[qs] - m_new);
            m_run[qs] = m_new;
            l_run[qs] *= alpha;
#pragma unroll
            for (int db = 0; db < dim_blocks<DIM>(); ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[db][qs][i] *= alpha;
        }
        const float m_use = m_run[qs];
        float rowsum = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[ks][qs][i], c, -m_use));
                if constexpr (MASK) {
                    const int key = 32 * ks + 16 * (i / 8) + 8 * half + (i % 8);
                    if (key >= valid) p = 0.0f;
                }
                s[ks][qs][i] = p;
                rowsum += p;
            }
        }
        {
            auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(rowsum), __float_as_uint(rowsum), false, false);
            rowsum = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        l_run[qs] += rowsum;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int ks = t >> 1, base = 8 * (t & 1);
            uint4 packed;
            packed.x = pack2(s[ks][qs][base + 0], s[ks][qs][base + 1]);
            packed.y = pack2(s[ks][qs][base + 2], s[ks][qs][base + 3]);
            packed.z = pack2(s[ks][qs][base + 4], s[ks][qs][base + 5]);
            packed.w = pack2(s[ks][qs][base + 6], s[ks][qs][base + 7]);
            pop[qs][t] = as_bf16x8(packed);
        }
    }

#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int db = 0; db < dim_blocks<DIM>(); ++db) {
            const bf16_t *vp = vt + 16 * t * kRow + (vidx ^ (32 * db));
            const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(vp));
            const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(vp + 4 * kRow));
            const uint2 lo2 = __builtin_bit_cast(uint2, lo), hi2 = __builtin_bit_cast(uint2, hi);
            const bf16x8_t vop = as_bf16x8(make_uint4(lo2.x, lo2.y, hi2.x, hi2.y));
#pragma unroll
            for (int qs = 0; qs < kQS; ++qs)
                acc[db][qs] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop, pop[qs][t], acc[db][qs], 0, 0, 0);
        }
    }
    // Rolling window of V^T operand reads (two ds_read_b64_tr_b16 per MFMA
    // operand), two operands ahead of the MFMAs.
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 4 * dim_blocks<DIM>() - 2; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, kQS, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * kQS, 0);
}

// BUF: K and V tiles through buffer loads (the host checks that one head's
// rows fit a 31-bit byte range and that rows do not overlap). DIM: the head
// dim, 128 or 72. The tiles keep the 128-dim row layout; dims past DIM are
// zero in Q, K and V, so the dot products and the first DIM output dims are
// those of the DIM-wide head. Only the k-steps and dim blocks that hold a dim
// below DIM are computed (72: 5 k-steps, dims 0..79, and 3 blocks, dims
// 0..95; 22 MFMAs per tile and wave against 32), and only dims below DIM are
// stored.
//
// GEN: the element-strided path for views the 16-byte accesses cannot take (a
// head-dim stride other than 1, or rows that are not 16-byte aligned): Q, K,
// V and O move element by element with their strides (pointer path only);
// the arithmetic is unchanged.
template <bool NEG, bool BUF, int DIM, bool GEN = false>
__global__ __launch_bounds__(kThreadsWG) __attribute__((amdgpu_waves_per_eu(kWaves / 4, kWaves / 4))) void attention_fwd_kernel(AttnArgs a) {
    static_assert(!GEN || !BUF, "the element-strided path loads through registers");
    // Two buffers per operand as separate arrays: the loads into one buffer
    // then provably do not alias the reads of the other, so the compiler's
    // wait for the loads is not placed before those reads.
    __shared__ __attribute__((aligned(1024))) bf16_t lds_k0[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t lds_k1[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t lds_v0[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t lds_v1[kTileElems];

    const int logical = xcd_remap(blockIdx.x, a.B * a.H * a.qblocks);
    const int qb = logical % a.qblocks;
    const int bh = logical / a.qblocks;
    const int b = bh / a.H, h = bh % a.H;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int l32 = lane & 31;
    const int half = lane >> 5;

    const bf16_t *qbase = a.q + b * a.qs[0] + h * a.qs[1];
    const bf16_t *kbase = a.k + b * a.ks[0] + h * a.ks[1];
    const bf16_t *vbase = a.v + b * a.vs[0] + h * a.vs[1];
    bf16_t *obase = a.o + b * a.os[0] + h * a.os[1];

    // Q^T operands: query block qs (0/1) of this wave, k-step kk covers dims
    // 16kk + 8*half .. +8.
    const int q_first = qb * kBM + wave * 32 * kQS;
    bf16x8_t qreg[kQS][8];
#pragma unroll
    for (int qs = 0; qs < kQS; ++qs) {
        int query = q_first + qs * 32 + l32;
        query = query < a.Sq ? query : a.Sq - 1;
        const bf16_t *qrow = qbase + static_cast<int64_t>(query) * a.qs[2];
#pragma unroll
        for (int kk = 0; kk < kk_steps<DIM>(); ++kk) {
            // This lane's 8 dims; past the head dim, a valid chunk is read and zeroed.
            const int d0 = 16 * kk + 8 * half;
            const uint4 u = load_row8<GEN>(qrow, d0 < DIM ? d0 : DIM - 8, a.qd);
            qreg[qs][kk] = as_bf16x8(d0 < DIM ? u : make_uint4(0u, 0u, 0u, 0u));
        }
        if (a.prescale) {  // bf16(fp32(c) * fp32(q)) (tools/h3_attention.py:88)
#pragma unroll
            for (int kk = 0; kk < kk_steps<DIM>(); ++kk) {
                const uint4 u = __builtin_bit_cast(uint4, qreg[qs][kk]);
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
                uint32_t o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = pack2(lo2f(w[e]) * a.c, hi2f(w[e]) * a.c);
                qreg[qs][kk] = as_bf16x8(make_uint4(o[0], o[1], o[2], o[3]));
            }
        }
    }

    f32x16_t acc[4][kQS];  // O^T: dim block db (32 dims) x query block qs
#pragma unroll
    for (int db = 0; db < dim_blocks<DIM>(); ++db)
#pragma unroll
        for (int qs = 0; qs < kQS; ++qs)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[db][qs][i] = 0.0f;
    float m_run[kQS];  // running max of the logits
    float l_run[kQS];
#pragma unroll
    for (int qs = 0; qs < kQS; ++qs) {
        m_run[qs] = -INFINITY;
        l_run[qs] = 0.0f;  // running denominator
    }

    u32x4_t kreg[kLoadRows], vreg[kLoadRows];
    // Descriptors of this head's K and V rows (range 0 on the pointer path, never used there).
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t *>(kbase), static_cast<short>(0), a.k_bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t *>(vbase), static_cast<short>(0), a.v_bytes, kBufferWord3);
    int kvoff[kLoadRows], vvoff[kLoadRows];
    const int kstep = static_cast<int>(a.ks[2]) * 2 * kBN, vstep = static_cast<int>(a.vs[2]) * 2 * kBN;
    if constexpr (BUF) {
#pragma unroll
        for (int r = 0; r < kLoadRows; ++r) {
            const int row = tile_row(r);
            const int kc = 8 * tile_chunk<true>(row), vc = 8 * tile_chunk<false>(row);
            // Chunks past the head dim point past the descriptor's range (which
            // is below 2^31 with every tile offset) and read as zero.
            kvoff[r] = kc < DIM ? (row * static_cast<int>(a.ks[2]) + kc) * 2 : kBeyondRange;
            vvoff[r] = vc < DIM ? (row * static_cast<int>(a.vs[2]) + vc) * 2 : kBeyondRange;
        }
        dma_tile(krs, kvoff, 0, lds_k0);
        dma_tile(vrs, vvoff, 0, lds_v0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
        load_tile<true, DIM, GEN>(kbase, a.ks[2], 0, a.Sk < kBN ? a.Sk : kBN, kreg, a.kd);
        load_tile<false, DIM, GEN>(vbase, a.vs[2], 0, a.Sk < kBN ? a.Sk : kBN, vreg, a.vd);
        store_tile(lds_k0, kreg);
        store_tile(lds_v0, vreg);
    }
    __syncthreads();

    // This lane's K operand: row pi(l32) of each 32-key block (MFMA row m reads
    // K row pi(m), bits 2 and 3 swapped), chunk 2 kk + half at slot
    // (2 kk + half) ^ swz_k(row), i.e. element index kidx ^ 16 kk.
    const int krow = (l32 & ~12) | ((l32 & 4) << 1) | ((l32 & 8) >> 1);
    const int kidx = krow * kRow + 8 * (half ^ swz_k(krow));
    // ds_read_b64_tr_b16 addressing for the V^T operand: within each 16-lane
    // group, lane s points at row (s/4) and dims 4*(s%4) of its 4x16 block;
    // dims 32 db + col sit at element (32 db + col) ^ 8 swz_v(row) of the row.
    const int g16 = lane >> 4, s16 = lane & 15;
    const int v_row_off = 8 * (g16 >> 1) + (s16 >> 2);
    const int v_col_off = 16 * (g16 & 1) + 4 * (s16 & 3);
    const int vidx = v_row_off * kRow + (v_col_off ^ (8 * swz_v(v_row_off)));

    // The logits' factor: c, or 1 when c is already in bf16(c q).
    const float c_loop = a.prescale ? 1.0f : a.c;
    // One full tile from (kc, vc) while the next is loaded into (kn, vn).
    auto step = [&](int tile, const bf16_t *kc, const bf16_t *vc, bf16_t *kn, bf16_t *vn) {
        const int next0 = (tile + 1) * kBN;
        const bool has_next = next0 < a.Sk;
        if constexpr (BUF) {
            // After the last tile the loads fall past the rows and write zeros (unused).
            dma_tile(krs, kvoff, (tile + 1) * kstep, kn);
            dma_tile(vrs, vvoff, (tile + 1) * vstep, vn);
        } else {
            // After the last tile the loads re-read the last row (unused), so
            // they need no branch either.
            const int n0 = has_next ? next0 : a.Sk - 1;
            const int nvalid = a.Sk - n0 < kBN ? a.Sk - n0 : kBN;
            load_tile<true, DIM, GEN>(kbase, a.ks[2], n0, nvalid, kreg, a.kd);
            load_tile<false, DIM, GEN>(vbase, a.vs[2], n0, nvalid, vreg, a.vd);
        }
        attend_tile<false, NEG, DIM>(kc, vc, kBN, qreg, acc, m_run, l_run, c_loop, kidx, half, vidx);
        if constexpr (BUF) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else if (has_next) {
            store_tile(kn, kreg);
            store_tile(vn, vreg);
        }
        __syncthreads();
    };
    // Full tiles in the loop, two per iteration (the buffers alternate); a
    // partial last tile (Sk % 64 != 0) after it.
    const int full = a.Sk / kBN;
    for (int tile = 0; tile < full; tile += 2) {
        step(tile, lds_k0, lds_v0, lds_k1, lds_v1);
        if (tile + 1 < full) step(tile + 1, lds_k1, lds_v1, lds_k0, lds_v0);
    }
    if (full * kBN < a.Sk) {
        if (full & 1)
            attend_tile<true, NEG, DIM>(lds_k1, lds_v1, a.Sk - full * kBN, qreg, acc, m_run, l_run, c_loop, kidx, half, vidx);
        else
            attend_tile<true, NEG, DIM>(lds_k0, lds_v0, a.Sk - full * kBN, qreg, acc, m_run, l_run, c_loop, kidx, half, vidx);
    }

    // ---- o = acc / denominator, bf16; lane owns one query, dims
    // 32db + 8g + 4*half + 0..3 for g = 0..3.
#pragma unroll
    for (int qs = 0; qs < kQS; ++qs) {
        const int query = q_first + qs * 32 + l32;
        if (query >= a.Sq) continue;
        const float inv = __fdiv_rn(1.0f, l_run[qs]);
        bf16_t *orow = obase + static_cast<int64_t>(query) * a.os[2];
#pragma unroll
        for (int db = 0; db < dim_blocks<DIM>(); ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                uint2 w;
                w.x = pack2(acc[db][qs][4 * g + 0] * inv, acc[db][qs][4 * g + 1] * inv);
                w.y = pack2(acc[db][qs][4 * g + 2] * inv, acc[db][qs][4 * g + 3] * inv);
                const int d0 = 32 * db + 8 * g + 4 * half;
                if (d0 < DIM) {
                    if constexpr (GEN) {
                        orow[d0 * a.od] = static_cast<bf16_t>(w.x);
                        orow[(d0 + 1) * a.od] = static_cast<bf16_t>(w.x >> 16);
                        orow[(d0 + 2) * a.od] = static_cast<bf16_t>(w.y);
                        orow[(d0 + 3) * a.od] = static_cast<bf16_t>(w.y >> 16);
                    } else {
                        *reinterpret_cast<uint2 *>(orow + d0) = w;
                    }
                }
            }
    }
}

// ============================================================ attention16_kernel
//
// The D = 128 kernel on the buffer path, on v_mfma_f32_16x16x32_bf16: under
// power the part sustains about 14% more flops with this product than with
// 32x32x16 (launch_h3_calibration_mfma_16x16x32).
//
// Layout (A row and B column = lane % 16, the 32-deep k split over the four
// 16-lane groups; accumulator register i of lane l holds row 4 (l / 16) + i,
// column l % 16):
//   - each wave's 32 queries are two 16-query blocks qb. S^T = K Q^T (A = 16
//     keys x 32 dims of K from LDS, B = Q^T from registers) leaves in lane l
//     the logits of query 16 qb + l % 16 against keys 16 kb + 4 (l / 16) + i
//     (kb, i = 0..3): 16 per block, a query's 64 keys spread over the four
//     16-lane groups;
//   - P^T, the B operand of O^T += V^T P^T, takes each 32-key half h in the
//     order the lane holds it (element j of lane l is key 32 h + 16 (j / 4) +
//     4 (l / 16) + j % 4), and the V^T operand reads the same key order with
//     two ds_read_b64_tr_b16 (4 consecutive keys each); a lane's O^T
//     accumulators again belong to its own queries.
//
// The softmax's maximum. The reference normalises by the running maximum of
// the logits, rescaling O and the denominator whenever a tile raises it. Here
// a unit (or key piece) takes the maximum of its FIRST tile as the reference
// m and keeps it: each later tile's p = exp2(c s - m) is computed against that
// m, with no per-tile maximum, cross-lane fold, rescale or branch in the loop,
// so each tile is one scheduling block. o = (sum p v) / (sum p) is the same
// quantity for any m. A later logit far above the first tile's maximum makes
// p large; if that overflows anywhere (p, the denominator or an accumulator
// not finite), the workgroup recomputes the unit with the running-maximum
// rescale, so a result is finite wherever the reference's is.
//
// The denominator sums the same bf16-rounded p that weight V (the reference
// sums p in fp32 before that rounding). Against a running maximum the largest
// p of a row is exactly 1 and loses nothing to bf16; against a fixed m it is
// any number, and a row that one key dominates would carry that key's bf16
// rounding (up to 2^-9) into o if the denominator did not share it (at
// |o| ~ 8 that flips the bf16 rounding of o: 0.03 from the fp32 result on the
// peaky configuration). With the shared weights o is an exact convex
// combination of the V rows under the rounded weights. The sum runs on the
// matrix core, as a product of a ones operand with P^T accumulated across
// the tiles (4 products per tile and wave beside the 64 of Q K^T and P V):
// the VALU sum it replaces, v_dot2c_f32_bf16 against (1, 1), issues about
// four times slower than an fp32 add and cost 2-3% of the kernel's time.

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// V tile swizzle of this kernel: chunk c of row r at slot c ^ 2 (r & 7), so
// the 8 consecutive rows x 2 chunks one half-wave's ds_read_b64_tr_b16 reads
// land on 16 distinct slots.
__device__ __forceinline__ int swz_v16(int row) { return 2 * (row & 7); }

// Max (NEG: min) over the four 16-lane groups that hold a query's keys: lanes
// l, l ^ 16, l ^ 32, l ^ 48, combined as ((x0 . x1) . (x2 . x3)) in every one
// of them.
template <bool NEG>
__device__ __forceinline__ float fold_groups_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = NEG ? fminf(__uint_as_float(a[0]), __uint_as_float(a[1])) : fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return NEG ? fminf(__uint_as_float(b[0]), __uint_as_float(b[1])) : fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// S^T of one 64-key tile for NQB 16-query blocks. kidx: this lane's K operand
// element for k-step 0 (row 16 kb + l % 16 of the tile, chunk 4 ks + l / 16;
// k-step ks reads kidx ^ 32 ks). Each K operand feeds every query block.
template <int NQB>
__device__ __forceinline__ void qk_tile16(const bf16_t *kt, const bf16x8_t (&qreg)[NQB][4], int kidx,
                                          f32x4_t (&s)[NQB][4]) {
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) s[qb][kb][i] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const bf16x8_t kop = as_bf16x8(*reinterpret_cast<const uint4 *>(kt + 16 * kb * kRow + (kidx ^ (32 * ks))));
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb)
                s[qb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qreg[qb][ks], s[qb][kb], 0, 0, 0);
        }
    // Rolling window of K operand reads, four ahead of the MFMAs (measured
    // +0.8% over three ahead, which was +1.3% over two; five ahead, or a
    // deeper V^T window, lose).
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, NQB, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4 * NQB, 0);
}

// P = bf16(exp2(c s - m)) (keys >= valid: 0 when MASK), the denominator
// l += sum of P, and O^T += V^T P^T.
// vidx: this lane's V^T operand address for dim block 0 of the lower 4 keys
// (row 4 (l / 16) + (l % 16) / 4, dims 4 (l % 4) of the block; block db reads
// vidx ^ 16 db, the upper 4 keys 16 rows further, half h 32 rows further).
template <bool MASK, int NQB>
__device__ __forceinline__ void pv_tile16(const bf16_t *vt, int vidx, const f32x4_t (&s)[NQB][4], const float (&m)[NQB],
                                          f32x4_t (&l)[NQB], float c, int valid, int g, f32x4_t (&acc)[NQB][8]) {
    bf16x8_t pop[NQB][2];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        float p[4][4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][kb][i], c, -m[qb]));
                if constexpr (MASK) {
                    if (16 * kb + 4 * g + i >= valid) e = 0.0f;
                }
                p[kb][i] = e;
            }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint4 packed;
            packed.x = pack2(p[2 * h][0], p[2 * h][1]);
            packed.y = pack2(p[2 * h][2], p[2 * h][3]);
            packed.z = pack2(p[2 * h + 1][0], p[2 * h + 1][1]);
            packed.w = pack2(p[2 * h + 1][2], p[2 * h + 1][3]);
            pop[qb][h] = as_bf16x8(packed);
        }
    }
    // The denominator on the matrix core: ones x P^T adds the 32 keys of each
    // half to every row of l (each lane then holds its query's whole sum).
    {
        const bf16x8_t ones = as_bf16x8(make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u));
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) l[qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pop[qb][h], l[qb], 0, 0, 0);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            const bf16_t *vp = vt + 32 * h * kRow + (vidx ^ (16 * db));
            const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(vp));
            const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(vp + 16 * kRow));
            const uint2 lo2 = __builtin_bit_cast(uint2, lo), hi2 = __builtin_bit_cast(uint2, hi);
            const bf16x8_t vop = as_bf16x8(make_uint4(lo2.x, lo2.y, hi2.x, hi2.y));
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb)
                acc[qb][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[qb][h], acc[qb][db], 0, 0, 0);
        }
    // Rolling window of V^T operand reads (two per operand), two operands ahead.
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 14; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, NQB, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * NQB, 0);
}

// A tile with the running-maximum rescale: the tile's maximum, and when it
// raises the running maximum m of some query, O and the denominator scaled by
// exp2(m_old - m_new) first (the reference's order). From m = -inf, l = 0,
// O = 0 it sets the reference maximum of the first tile.
template <bool MASK, bool NEG, int NQB>
__device__ __forceinline__ void exact_tile16(const bf16_t *kt, const bf16_t *vt, int valid,
                                             const bf16x8_t (&qreg)[NQB][4], int kidx, int vidx, int g, float c,
                                             float (&m)[NQB], f32x4_t (&l)[NQB], f32x4_t (&acc)[NQB][8]) {
    static_assert(NQB == 1 || NQB == 2, "one or two query blocks per wave");
    f32x4_t s[NQB][4];
    qk_tile16(kt, qreg, kidx, s);
    float mt[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        if constexpr (MASK) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (16 * kb + 4 * g + i >= valid) s[qb][kb][i] = NEG ? INFINITY : -INFINITY;
        }
        float mx = s[qb][0][0];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = NEG ? fminf(mx, s[qb][kb][i]) : fmaxf(mx, s[qb][kb][i]);
        mt[qb] = fold_groups_max<NEG>(mx) * c;
    }
    if constexpr (NQB == 2) {
        const bool grow0 = mt[0] > m[0], grow1 = mt[1] > m[1];
        if (__builtin_amdgcn_ballot_w64(grow0 || grow1)) {
            const float n0 = grow0 ? mt[0] : m[0], n1 = grow1 ? mt[1] : m[1];
            const float a0 = __builtin_amdgcn_exp2f(m[0] - n0), a1 = __builtin_amdgcn_exp2f(m[1] - n1);
            m[0] = n0;
            m[1] = n1;
            l[0] *= a0;
            l[1] *= a1;
#pragma unroll
            for (int db = 0; db < 8; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc[0][db][i] *= a0;
                    acc[1][db][i] *= a1;
                }
        }
    } else {
        const bool grow0 = mt[0] > m[0];
        if (__builtin_amdgcn_ballot_w64(grow0)) {
            const float n0 = grow0 ? mt[0] : m[0];
            const float a0 = __builtin_amdgcn_exp2f(m[0] - n0);
            m[0] = n0;
            l[0] *= a0;
#pragma unroll
            for (int db = 0; db < 8; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[0][db][i] *= a0;
        }
    }
    pv_tile16<MASK>(vt, vidx, s, m, l, c, valid, g, acc);
}

// A tile against the fixed reference maximum m.
template <bool MASK, int NQB>
__device__ __forceinline__ void ref_tile16(const bf16_t *kt, const bf16_t *vt, int valid,
                                           const bf16x8_t (&qreg)[NQB][4], int kidx, int vidx, int g, float c,
                                           const float (&m)[NQB], f32x4_t (&l)[NQB], f32x4_t (&acc)[NQB][8]) {
    f32x4_t s[NQB][4];
    qk_tile16(kt, qreg, kidx, s);
    pv_tile16<MASK>(vt, vidx, s, m, l, c, valid, g, acc);
}

// A query's denominator: every row of its l accumulator holds the whole sum.
__device__ __forceinline__ float den_total(const f32x4_t &l) { return l[0]; }

// The Q^T operands of query block qb (k-step ks: dims 32 ks + 8 g .. +8 of
// query q_first + 16 qb + l16, clamped to the last query), prescaled to
// bf16(fp32(c) * fp32(q)) for the prescale numerics (tools/h3_attention.py:88).
__device__ __forceinline__ void load_q16(const AttnArgs &a, const bf16_t *qbase, int q_first, int qb, int l16, int g,
                                         bf16x8_t (&qr)[4]) {
    int query = q_first + 16 * qb + l16;
    query = query < a.Sq ? query : a.Sq - 1;
    const bf16_t *qrow = qbase + static_cast<int64_t>(query) * a.qs[2];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qr[ks] = as_bf16x8(*reinterpret_cast<const uint4 *>(qrow + 32 * ks + 8 * g));
    if (a.prescale) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const uint4 u = __builtin_bit_cast(uint4, qr[ks]);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = pack2(lo2f(w[e]) * a.c, hi2f(w[e]) * a.c);
            qr[ks] = as_bf16x8(make_uint4(o[0], o[1], o[2], o[3]));
        }
    }
}

// SPLIT: the key-split launch (see AttnArgs); a piece leaves its unnormalised
// O, reference maximum and denominator in the workspace for the merge.
template <bool NEG, bool SPLIT>
__global__ __launch_bounds__(kThreadsWG) __attribute__((amdgpu_waves_per_eu(kWaves / 4, kWaves / 4))) void attention16_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(1024))) bf16_t lds_k0[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t lds_k1[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t lds_v0[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t lds_v1[kTileElems];
    __shared__ int wave_overflow[kWaves];

    int logical, piece = -1;  // piece >= 0: a key piece of a tail unit
    if constexpr (SPLIT) {
        const int x = static_cast<int>(blockIdx.x);
        if (x < a.n_full) {
            logical = xcd_remap(x, a.n_full);
        } else {
            const int lp = xcd_remap(x - a.n_full, a.n_tail * a.split);
            piece = lp / a.n_tail;
            logical = a.n_full + lp % a.n_tail;
        }
    } else {
        logical = xcd_remap(blockIdx.x, a.B * a.H * a.qblocks);
    }
    const int qbk = logical % a.qblocks;
    const int bh = logical / a.qblocks;
    const int b = bh / a.H, h = bh % a.H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const bf16_t *qbase = a.q + b * a.qs[0] + h * a.qs[1];
    const bf16_t *kbase = a.k + b * a.ks[0] + h * a.ks[1];
    const bf16_t *vbase = a.v + b * a.vs[0] + h * a.vs[1];
    bf16_t *obase = a.o + b * a.os[0] + h * a.os[1];

    // Q^T operands: query block qb, k-step ks holds dims 32 ks + 8 g .. +8 of
    // query 16 qb + l16 of this wave's 32.
    const int q_first = qbk * kBM + wave * 32;
    bf16x8_t qreg[2][4];
    load_q16(a, qbase, q_first, 0, l16, g, qreg[0]);
    load_q16(a, qbase, q_first, 1, l16, g, qreg[1]);

    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t *>(kbase), static_cast<short>(0), a.k_bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t *>(vbase), static_cast<short>(0), a.v_bytes, kBufferWord3);
    int kvoff[kLoadRows], vvoff[kLoadRows];
    const int kstep = static_cast<int>(a.ks[2]) * 2 * kBN, vstep = static_cast<int>(a.vs[2]) * 2 * kBN;
#pragma unroll
    for (int r = 0; r < kLoadRows; ++r) {
        const int row = tile_row(r);
        kvoff[r] = (row * static_cast<int>(a.ks[2]) + 8 * (static_cast<int>(threadIdx.x & 15) ^ swz_k(row))) * 2;
        vvoff[r] = (row * static_cast<int>(a.vs[2]) + 8 * (static_cast<int>(threadIdx.x & 15) ^ swz_v16(row))) * 2;
    }
    const int kidx = l16 * kRow + 8 * (g ^ l16);
    const int vrow = 4 * g + (l16 >> 2);
    const int vidx = vrow * kRow + (16 * (vrow & 7) + 8 * ((l16 >> 1) & 1) + 4 * (l16 & 1));
    const float c = a.prescale ? 1.0f : a.c;  // the logits' factor (1 when c is in bf16(c q))

    // Key tiles [t0, t_end) are full; a partial tile (Sk % 64 keys) follows
    // when it belongs to this unit or piece.
    const int T = (a.Sk + kBN - 1) / kBN, full = a.Sk / kBN;
    int t0 = 0, t_end = full;
    bool partial = full < T;
    if constexpr (SPLIT) {
        if (piece >= 0) {
            t0 = piece * T / a.split;
            const int t1 = (piece + 1) * T / a.split;
            t_end = t1 < full ? t1 : full;
            partial = t1 > full;
        }
    }
    const int valid_last = a.Sk - full * kBN;

    f32x4_t acc[2][8];
    float m[2];
    f32x4_t l[2];
    // One pass over the unit's tiles for the query blocks of qq (one or two;
    // their maxima, denominator chains and accumulators in mm, ll, aa): the
    // first tile exact (it sets the reference maxima), the rest against them
    // (EXACT: all with the online rescale).
    auto pass = [&](auto exact_tag, const auto &qq, auto &mm, auto &ll, auto &aa) __attribute__((always_inline)) {
        constexpr bool EXACT = decltype(exact_tag)::value;
        constexpr int NQ = sizeof(mm) / sizeof(float);
#pragma unroll
        for (int qb = 0; qb < NQ; ++qb) {
            mm[qb] = -INFINITY;
            ll[qb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int db = 0; db < 8; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) aa[qb][db][i] = 0.0f;
        }
        dma_tile(krs, kvoff, t0 * kstep, lds_k0);
        dma_tile(vrs, vvoff, t0 * vstep, lds_v0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        // Tile `tile` from (kc, vc) while tile + 1 is loaded into (kn, vn);
        // past the head's last key the loads read zeros (unused).
        auto step = [&](auto first_tag, int tile, const bf16_t *kc, const bf16_t *vc, bf16_t *kn, bf16_t *vn)
                        __attribute__((always_inline)) {
            dma_tile(krs, kvoff, (tile + 1) * kstep, kn);
            dma_tile(vrs, vvoff, (tile + 1) * vstep, vn);
            if constexpr (EXACT || decltype(first_tag)::value)
                exact_tile16<false, NEG>(kc, vc, kBN, qq, kidx, vidx, g, c, mm, ll, aa);
            else
                ref_tile16<false>(kc, vc, kBN, qq, kidx, vidx, g, c, mm, ll, aa);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        };
        if (t_end > t0) {
            step(std::true_type{}, t0, lds_k0, lds_v0, lds_k1, lds_v1);
            int t = t0 + 1;
            for (; t + 1 < t_end; t += 2) {
                step(std::false_type{}, t, lds_k1, lds_v1, lds_k0, lds_v0);
                step(std::false_type{}, t + 1, lds_k0, lds_v0, lds_k1, lds_v1);
            }
            if (t < t_end) step(std::false_type{}, t, lds_k1, lds_v1, lds_k0, lds_v0);
            if (partial) {  // tile t_end, in buffer (t_end - t0) & 1
                const bool odd = (t_end - t0) & 1;
                const bf16_t *kc = odd ? lds_k1 : lds_k0;
                const bf16_t *vc = odd ? lds_v1 : lds_v0;
                if constexpr (EXACT)
                    exact_tile16<true, NEG>(kc, vc, valid_last, qq, kidx, vidx, g, c, mm, ll, aa);
                else
                    ref_tile16<true>(kc, vc, valid_last, qq, kidx, vidx, g, c, mm, ll, aa);
            }
        } else if (partial) {  // the partial tile is the only one
            exact_tile16<true, NEG>(lds_k0, lds_v0, valid_last, qq, kidx, vidx, g, c, mm, ll, aa);
        }
    };
    pass(std::false_type{}, qreg, m, l, acc);
    // Overflow against the reference maxima: redo the unit with the running
    // maximum. The test covers the denominator (finite weights can sum to
    // +inf) and every accumulator. A key piece is held to
    // FLT_MAX / kMaxSplit, so that the merge's sums over up to kMaxSplit
    // pieces, each weighted by at most 1, stay finite. Every wave has passed
    // its last LDS read of the pass before the barrier.
    float lt[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) lt[qb] = den_total(l[qb]);
    const float limit = piece >= 0 ? __FLT_MAX__ / kMaxSplit : INFINITY;
    // x < limit is false for NaN, so NaN counts as overflow too.
    bool finite = lt[0] < limit && lt[1] < limit;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int db = 0; db < 8; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) finite = finite && fabsf(acc[qb][db][i]) < limit;
    const bool wave_bad = __builtin_amdgcn_ballot_w64(!finite) != 0;
    if (lane == 0) wave_overflow[wave] = wave_bad ? 1 : 0;
    __syncthreads();
    int any_bad = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) any_bad |= wave_overflow[w];
    if (any_bad) {
        // The fallback takes one query block at a time, with its Q operands
        // loaded again, so that it holds half the state of the pass above
        // (the kernel's register peak otherwise).
        auto redo = [&](auto qb_tag) __attribute__((always_inline)) {
            constexpr int qb = decltype(qb_tag)::value;
            bf16x8_t q1[1][4];
            load_q16(a, qbase, q_first, qb, l16, g, q1[0]);
            pass(std::true_type{}, q1, *reinterpret_cast<float(*)[1]>(&m[qb]), *reinterpret_cast<f32x4_t(*)[1]>(&l[qb]),
                 *reinterpret_cast<f32x4_t(*)[1][8]>(&acc[qb]));
            lt[qb] = den_total(l[qb]);
        };
        redo(std::integral_constant<int, 0>{});
        __syncthreads();  // every wave past its last LDS read
        redo(std::integral_constant<int, 1>{});
    }
    if constexpr (SPLIT) {
        if (piece >= 0) {  // a piece: O, m and l of its 256 queries go to the workspace
            const int64_t slot = static_cast<int64_t>(logical - a.n_full) * a.split + piece;
            float *pa = a.ws + slot * kWsSlotAcc;
            float *pm = a.ws + static_cast<int64_t>(a.n_tail) * a.split * kWsSlotAcc + slot * kWsSlotMl;
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
                const int r = wave * 32 + 16 * qb + l16;
#pragma unroll
                for (int db = 0; db < 8; ++db)
                    *reinterpret_cast<float4 *>(pa + r * kD + 16 * db + 4 * g) =
                        float4{acc[qb][db][0], acc[qb][db][1], acc[qb][db][2], acc[qb][db][3]};
                if (g == 0) *reinterpret_cast<float2 *>(pm + 2 * r) = float2{m[qb], lt[qb]};
            }
            return;
        }
    }
    // o = acc / denominator, bf16: lane l holds dims 16 db + 4 g .. +4 of
    // query 16 qb + l16.
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int query = q_first + 16 * qb + l16;
        if (query >= a.Sq) continue;
        const float inv = __fdiv_rn(1.0f, lt[qb]);
        bf16_t *orow = obase + static_cast<int64_t>(query) * a.os[2];
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            uint2 w;
            w.x = pack2(acc[qb][db][0] * inv, acc[qb][db][1] * inv);
            w.y = pack2(acc[qb][db][2] * inv, acc[qb][db][3] * inv);
            *reinterpret_cast<uint2 *>(orow + 16 * db + 4 * g) = w;
        }
    }
}

// attention16_kernel for the launch whose last round is 192-query units (see
// AttnArgs, SMALL kernels). In such a unit waves 0-3 take 32 queries each and
// waves 4-7 16 each, so every SIMD (waves w and w + 4) carries 48 queries, 3/4
// of a 256-query unit; the arithmetic of a query is attention16_kernel's. (A
// kernel of its own: folding this plan into attention16_kernel changed that
// kernel's code enough to raise its HBM traffic at S = 73,984 by 3-30%.)
template <bool NEG>
__global__ __launch_bounds__(kThreadsWG) __attribute__((amdgpu_waves_per_eu(kWaves / 4, kWaves / 4))) void attention16_small_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(1024))) bf16_t lds_k0[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t lds_k1[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t lds_v0[kTileElems];
    __shared__ __attribute__((aligned(1024))) bf16_t lds_v1[kTileElems];
    __shared__ int wave_overflow[kWaves];

    const SmallUnit u = small_plan_unit(a, static_cast<int>(blockIdx.x));
    const int b = u.bh / a.H, h = u.bh % a.H;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // a scalar: the branch below is on it
    const int l16 = lane & 15, g = lane >> 4;
    const bf16_t *qbase = a.q + b * a.qs[0] + h * a.qs[1];
    const bf16_t *kbase = a.k + b * a.ks[0] + h * a.ks[1];
    const bf16_t *vbase = a.v + b * a.vs[0] + h * a.vs[1];
    bf16_t *obase = a.o + b * a.os[0] + h * a.os[1];

    // This wave's queries: NQB blocks of 16 from q_first (waves 4-7 of a
    // 192-query unit: one block each, after the 128 queries of waves 0-3).
    const int q_first = u.small && wave >= 4 ? u.q0 + 128 + 16 * (wave - 4) : u.q0 + 32 * wave;
    auto run = [&](auto nqb_tag) __attribute__((always_inline)) {
        constexpr int NQB = decltype(nqb_tag)::value;
        // Q^T operands: query block qb, k-step ks holds dims 32 ks + 8 g .. +8 of
        // query 16 qb + l16 of this wave's queries.
        bf16x8_t qreg[NQB][4];
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) load_q16(a, qbase, q_first, qb, l16, g, qreg[qb]);

        const __amdgpu_buffer_rsrc_t krs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t *>(kbase), static_cast<short>(0), a.k_bytes, kBufferWord3);
        const __amdgpu_buffer_rsrc_t vrs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t *>(vbase), static_cast<short>(0), a.v_bytes, kBufferWord3);
        int kvoff[kLoadRows], vvoff[kLoadRows];
        const int kstep = static_cast<int>(a.ks[2]) * 2 * kBN, vstep = static_cast<int>(a.vs[2]) * 2 * kBN;
#pragma unroll
        for (int r = 0; r < kLoadRows; ++r) {
            const int row = tile_row(r);
            kvoff[r] = (row * static_cast<int>(a.ks[2]) + 8 * (static_cast<int>(threadIdx.x & 15) ^ swz_k(row))) * 2;
            vvoff[r] = (row * static_cast<int>(a.vs[2]) + 8 * (static_cast<int>(threadIdx.x & 15) ^ swz_v16(row))) * 2;
        }
        const int kidx = l16 * kRow + 8 * (g ^ l16);
        const int vrow = 4 * g + (l16 >> 2);
        const int vidx = vrow * kRow + (16 * (vrow & 7) + 8 * ((l16 >> 1) & 1) + 4 * (l16 & 1));
        const float c = a.prescale ? 1.0f : a.c;  // the logits' factor (1 when c is in bf16(c q))

        // Key tiles [0, full) are full; a partial tile (Sk % 64 keys) follows.
        const int T = (a.Sk + kBN - 1) / kBN, full = a.Sk / kBN;
        constexpr int t0 = 0;
        const int t_end = full;
        const bool partial = full < T;
        const int valid_last = a.Sk - full * kBN;

        f32x4_t acc[NQB][8];
        float m[NQB];
        f32x4_t l[NQB];
        // One pass over the unit's tiles for the query blocks of qq (see
        // attention16_kernel).
        auto pass = [&](auto exact_tag, const auto &qq, auto &mm, auto &ll, auto &aa) __attribute__((always_inline)) {
            constexpr bool EXACT = decltype(exact_tag)::value;
            constexpr int NQ = sizeof(mm) / sizeof(float);
#pragma unroll
            for (int qb = 0; qb < NQ; ++qb) {
                mm[qb] = -INFINITY;
                ll[qb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int db = 0; db < 8; ++db)
#pragma unroll
                    for (int i = 0; i < 4; ++i) aa[qb][db][i] = 0.0f;
            }
            dma_tile(krs, kvoff, t0 * kstep, lds_k0);
            dma_tile(vrs, vvoff, t0 * vstep, lds_v0);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            // Tile `tile` from (kc, vc) while tile + 1 is loaded into (kn, vn);
            // past the head's last key the loads read zeros (unused).
            auto step = [&](auto first_tag, int tile, const bf16_t *kc, const bf16_t *vc, bf16_t *kn, bf16_t *vn)
                            __attribute__((always_inline)) {
                dma_tile(krs, kvoff, (tile + 1) * kstep, kn);
                dma_tile(vrs, vvoff, (tile + 1) * vstep, vn);
                if constexpr (EXACT || decltype(first_tag)::value)
                    exact_tile16<false, NEG>(kc, vc, kBN, qq, kidx, vidx, g, c, mm, ll, aa);
                else
                    ref_tile16<false>(kc, vc, kBN, qq, kidx, vidx, g, c, mm, ll, aa);
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
            };
            if (t_end > t0) {
                step(std::true_type{}, t0, lds_k0, lds_v0, lds_k1, lds_v1);
                int t = t0 + 1;
                for (; t + 1 < t_end; t += 2) {
                    step(std::false_type{}, t, lds_k1, lds_v1, lds_k0, lds_v0);
                    step(std::false_type{}, t + 1, lds_k0, lds_v0, lds_k1, lds_v1);
                }
                if (t < t_end) step(std::false_type{}, t, lds_k1, lds_v1, lds_k0, lds_v0);
                if (partial) {  // tile t_end, in buffer (t_end - t0) & 1
                    const bool odd = (t_end - t0) & 1;
                    const bf16_t *kc = odd ? lds_k1 : lds_k0;
                    const bf16_t *vc = odd ? lds_v1 : lds_v0;
                    if constexpr (EXACT)
                        exact_tile16<true, NEG>(kc, vc, valid_last, qq, kidx, vidx, g, c, mm, ll, aa);
                    else
                        ref_tile16<true>(kc, vc, valid_last, qq, kidx, vidx, g, c, mm, ll, aa);
                }
            } else if (partial) {  // the partial tile is the only one
                exact_tile16<true, NEG>(lds_k0, lds_v0, valid_last, qq, kidx, vidx, g, c, mm, ll, aa);
            }
        };
        pass(std::false_type{}, qreg, m, l, acc);
        // Overflow against the reference maxima: redo the unit with the running
        // maximum (as attention16_kernel does).
        float lt[NQB];
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) lt[qb] = den_total(l[qb]);
        constexpr float limit = INFINITY;
        // x < limit is false for NaN, so NaN counts as overflow too.
        bool finite = true;
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) finite = finite && lt[qb] < limit;
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
            for (int db = 0; db < 8; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) finite = finite && fabsf(acc[qb][db][i]) < limit;
        const bool wave_bad = __builtin_amdgcn_ballot_w64(!finite) != 0;
        if (lane == 0) wave_overflow[wave] = wave_bad ? 1 : 0;
        __syncthreads();
        int any_bad = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) any_bad |= wave_overflow[w];
        if (any_bad) {
            // One query block at a time, as attention16_kernel does. Every
            // wave runs two passes, so that all reach the same barriers: a
            // wave of one block computes it twice (the same result).
            auto redo = [&](auto qb_tag) __attribute__((always_inline)) {
                constexpr int qb = decltype(qb_tag)::value;
                bf16x8_t q1[1][4];
                load_q16(a, qbase, q_first, qb, l16, g, q1[0]);
                pass(std::true_type{}, q1, *reinterpret_cast<float(*)[1]>(&m[qb]),
                     *reinterpret_cast<f32x4_t(*)[1]>(&l[qb]), *reinterpret_cast<f32x4_t(*)[1][8]>(&acc[qb]));
                lt[qb] = den_total(l[qb]);
            };
            redo(std::integral_constant<int, 0>{});
            __syncthreads();  // every wave past its last LDS read
            redo(std::integral_constant<int, NQB - 1>{});
        }
        // o = acc / denominator, bf16: lane l holds dims 16 db + 4 g .. +4 of
        // query 16 qb + l16.
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            const int query = q_first + 16 * qb + l16;
            if (query >= a.Sq) continue;
            const float inv = __fdiv_rn(1.0f, lt[qb]);
            bf16_t *orow = obase + static_cast<int64_t>(query) * a.os[2];
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                uint2 w;
                w.x = pack2(acc[qb][db][0] * inv, acc[qb][db][1] * inv);
                w.y = pack2(acc[qb][db][2] * inv, acc[qb][db][3] * inv);
                *reinterpret_cast<uint2 *>(orow + 16 * db + 4 * g) = w;
            }
        }
    };
    if (u.small && wave >= 4)
        run(std::integral_constant<int, 1>{});
    else
        run(std::integral_constant<int, 2>{});
}

// Combines the SPLIT pieces of the tail units: a 256-thread block per (tail
// unit, 8 queries), a thread per (query, 4 dims), all SPLIT pieces' loads
// issued together. With M = max_p m_p and w_p = 2^(m_p - M):
// o = bf16((sum_p w_p acc_p) / (sum_p w_p l_p)), sums in piece order.
template <int SPLIT>
__global__ __launch_bounds__(256) void attention_merge_kernel(AttnArgs a) {
    const int u = static_cast<int>(blockIdx.x) / (kBM / 8);
    const int r = (static_cast<int>(blockIdx.x) % (kBM / 8)) * 8 + static_cast<int>(threadIdx.x) / 32;
    const int d4 = static_cast<int>(threadIdx.x) % 32;
    const int unit = a.n_full + u;
    const int qb = unit % a.qblocks, bh = unit / a.qblocks;
    const int b = bh / a.H, h = bh % a.H;
    const int query = qb * kBM + r;
    if (query >= a.Sq) return;  // no barrier below
    const int64_t slot0 = static_cast<int64_t>(u) * SPLIT;
    const float *ml = a.ws + static_cast<int64_t>(a.n_tail) * SPLIT * kWsSlotAcc;
    float2 st[SPLIT];
    float4 part[SPLIT];
#pragma unroll
    for (int p = 0; p < SPLIT; ++p) {
        st[p] = *reinterpret_cast<const float2 *>(ml + (slot0 + p) * kWsSlotMl + 2 * r);
        part[p] = *reinterpret_cast<const float4 *>(a.ws + (slot0 + p) * kWsSlotAcc + r * kD + 4 * d4);
    }
    float m_all = st[0].x;
#pragma unroll
    for (int p = 1; p < SPLIT; ++p) m_all = fmaxf(m_all, st[p].x);
    float4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
    float den = 0.0f;
#pragma unroll
    for (int p = 0; p < SPLIT; ++p) {
        const float w = __builtin_amdgcn_exp2f(st[p].x - m_all);
        den += st[p].y * w;
        sum.x += w * part[p].x;
        sum.y += w * part[p].y;
        sum.z += w * part[p].z;
        sum.w += w * part[p].w;
    }
    const float inv = __fdiv_rn(1.0f, den);
    bf16_t *orow = a.o + b * a.os[0] + h * a.os[1] + static_cast<int64_t>(query) * a.os[2];
    uint2 o;
    o.x = pack2(sum.x * inv, sum.y * inv);
    o.y = pack2(sum.z * inv, sum.w * inv);
    *reinterpret_cast<uint2 *>(orow + 4 * d4) = o;
}

}  // namespace

// CUs of a device, looked up once per device.
constexpr int kMaxDevices = 64;
std::atomic<int> cu_count[kMaxDevices];

int device_cus(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return 0;
    int n = cu_count[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cu_count[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

int stream_device_cus(hipStream_t stream) {
    int dev = 0;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess) return 0;
    return device_cus(dev);
}

}  // namespace h3

using namespace h3;

namespace {

// The key split of the last round. Units of work (one workgroup each, one
// workgroup per CU) run in rounds of n_cu. The launch is power-bound: a round
// with only a fraction f of the CUs busy runs at a higher clock, and takes
// about max(f, kRoundFloor) of a full round's time (the loaded clock, ~2.0 GHz,
// is 0.82 of the 2.4 GHz peak; measured: at S = 12,288, H = 14 splitting the
// 5/8-full last round saves 3.4%, at S = 8192, H = 14 splitting the 3/4-full
// one saves nothing). Splitting the r units of the last round into s key pieces
// replaces that round by rounds of ceil(T / s) tiles (at least 8 per piece),
// plus the merge (130 KiB of partials per piece read back at ~3.5 TB/s and
// ~5 us of launch and latency, against ~1.8 us per tile-step). The split is
// taken when the model saves at least 3%.
struct SplitPlan {
    int n_full = 0, n_tail = 0, split = 1;
};

constexpr double kRoundFloor = 0.85;

double round_time(int64_t busy, int n_cu) {
    const double f = static_cast<double>(busy) / n_cu;
    return f > kRoundFloor ? f : kRoundFloor;
}

SplitPlan plan_split(int64_t units, int64_t tiles, int n_cu) {
    SplitPlan plan;
    plan.n_full = static_cast<int>(units);
    if (n_cu <= 0 || units <= 0 || units % n_cu == 0) return plan;
    const int64_t rounds = units / n_cu, r = units % n_cu;
    const double unsplit = static_cast<double>(rounds) + round_time(r, n_cu);  // in unit-times
    double best = unsplit;
    for (int s = 2; s <= kMaxSplit && tiles >= 8 * s; ++s) {
        const int64_t pieces = r * s;
        const double piece = static_cast<double>((tiles + s - 1) / s) / static_cast<double>(tiles);
        const double merge = (static_cast<double>(pieces) * kWsSlotBytes / 3.5e12 + 5e-6) / (tiles * 1.8e-6);
        const double t = static_cast<double>(rounds) +
                         piece * (static_cast<double>(pieces / n_cu) + (pieces % n_cu ? round_time(pieces % n_cu, n_cu) : 0.0)) +
                         merge;
        if (t < best) {
            best = t;
            plan.split = s;
        }
    }
    if (plan.split == 1 || best > 0.97 * unsplit) return SplitPlan{static_cast<int>(units), 0, 1};
    plan.n_full = static_cast<int>(rounds * n_cu);
    plan.n_tail = static_cast<int>(r);
    return plan;
}

// A last round of t 256-query units (t / n_cu at most 3/4) run instead as
// 4t/3 units of 192 queries: each CU of that round carries 3/4 of a unit, and
// the round fills the CUs. Three of every four 256-query units of a head's
// tail become four 192-query units (the same queries); the plan spreads those
// conversions over as few heads as it can (each head gives at most a third of
// its units). Taken when Sq is a multiple of 256, t is a multiple of 3 and the
// new round keeps at least kRoundFloor of the CUs busy, so it costs 3/4 of a
// round where the unsplit tail costs max(t / n_cu, kRoundFloor). No workspace;
// each query's arithmetic is that of the unsplit launch.
struct SmallPlan {
    bool use = false;
    int n_big = 0, n_small = 0, k = 0, big0 = 0, small0 = 0, big1 = 0, small1 = 0;
};

SmallPlan plan_small(int64_t heads, int64_t Sq, int n_cu) {
    SmallPlan p;
    if (n_cu <= 0 || heads <= 0 || Sq <= 0 || Sq % kBM != 0) return p;
    const int64_t per_head = Sq / kBM, units = heads * per_head;
    const int64_t rounds = units / n_cu, tail = units % n_cu;
    if (rounds < 1 || tail == 0 || tail % 3 != 0) return p;
    const int64_t n_small = 4 * tail / 3;
    if (n_small > n_cu || static_cast<double>(n_small) < kRoundFloor * n_cu) return p;
    const int64_t conversions = tail / 3, per_head_max = per_head / 3;
    if (per_head_max == 0 || conversions > heads * per_head_max) return p;
    const int64_t rem = conversions % per_head_max;
    p.use = true;
    p.n_big = static_cast<int>(rounds * n_cu);
    p.n_small = static_cast<int>(n_small);
    p.k = static_cast<int>(conversions / per_head_max);
    p.big0 = static_cast<int>(per_head - 3 * per_head_max);
    p.small0 = static_cast<int>(4 * per_head_max);
    p.big1 = static_cast<int>(per_head - 3 * rem);
    p.small1 = static_cast<int>(4 * rem);
    return p;
}


// The launcher of both numerics: fp32_qk (logits scaled by c = scale log2 e in
// fp32) and bf16_prescale (q rounded to bf16(c q) before the product).
// workspace (fp32_qk, D = 128, may be null): bytes for the key split of the
// last round; too small for the planned split (empty included), the launch
// runs unsplit.
int launch_attention(NineToothedStream stream, NineToothedTensor q, NineToothedTensor k, NineToothedTensor v,
                     NineToothedTensor scale, NineToothedTensor o, bool prescale, int64_t dim,
                     const NineToothedTensor *workspace = nullptr) {
    View<4> qv, kv, vv, ov;
    View<1> wv;
    double sc;
    if (!load_view(q, 2, qv) || !load_view(k, 2, kv) || !load_view(v, 2, vv) || !load_view(o, 2, ov) ||
        !load_scalar(scale, sc))
        return kInvalid;
    if (workspace != nullptr &&
        (!load_view(*workspace, 1, wv) || (wv.shape[0] > 1 && wv.stride[0] != 1) ||
         (reinterpret_cast<uintptr_t>(wv.data) & 255) != 0))
        return kInvalid;
    // Contract of the reference operator (patches/InfiniCore.patch:1366-1376):
    // same B/H/D, q and o alike, k and v alike, Sq and Sk free; D = `dim`
    // (128, or 72 for the vision launcher).
    if (!same_shape(qv, ov) || !same_shape(kv, vv)) return kInvalid;
    if (qv.shape[0] != kv.shape[0] || qv.shape[1] != kv.shape[1] || qv.shape[3] != kv.shape[3]) return kInvalid;
    if (qv.shape[3] != dim) return kInvalid;
    // Views the 16-byte accesses cannot take run on the element-strided path
    // (the reference's launcher likewise dispatches such views to its generic
    // stride variant, patches/ninetoothed.patch:131-169).
    const bool gen = !rows_vec16(qv, 2) || !rows_vec16(kv, 2) || !rows_vec16(vv, 2) || !rows_vec16(ov, 2);
    if ((reinterpret_cast<uintptr_t>(qv.data) | reinterpret_cast<uintptr_t>(kv.data) |
         reinterpret_cast<uintptr_t>(vv.data) | reinterpret_cast<uintptr_t>(ov.data)) & 1)
        return kInvalid;  // bf16 elements are 2-byte aligned
    if (qv.shape[0] == 0 || qv.shape[1] == 0 || qv.shape[2] == 0) return 0;
    if (kv.shape[2] == 0) return kInvalid;  // softmax over no keys is undefined
    if (qv.shape[2] > kMaxSeqLen || kv.shape[2] > kMaxSeqLen) return kInvalid;
    AttnArgs a{};
    a.q = reinterpret_cast<const bf16_t *>(qv.data);
    a.k = reinterpret_cast<const bf16_t *>(kv.data);
    a.v = reinterpret_cast<const bf16_t *>(vv.data);
    a.o = reinterpret_cast<bf16_t *>(ov.data);
    for (int i = 0; i < 3; ++i) {
        a.qs[i] = qv.stride[i];
        a.ks[i] = kv.stride[i];
        a.vs[i] = vv.stride[i];
        a.os[i] = ov.stride[i];
    }
    a.qd = qv.stride[3];
    a.kd = kv.stride[3];
    a.vd = vv.stride[3];
    a.od = ov.stride[3];
    a.B = static_cast<int>(qv.shape[0]);
    a.H = static_cast<int>(qv.shape[1]);
    a.Sq = static_cast<int>(qv.shape[2]);
    a.Sk = static_cast<int>(kv.shape[2]);
    a.qblocks = (a.Sq + kBM - 1) / kBM;
    const int64_t grid = static_cast<int64_t>(a.B) * a.H * a.qblocks;
    if (grid > static_cast<int64_t>(std::numeric_limits<int32_t>::max())) return kInvalid;
    a.c = static_cast<float>(static_cast<float>(sc) * kLog2e);
    a.prescale = prescale;
    // Buffer loads when one head's K / V rows (plus one tile of key offsets
    // past the end, which the last iteration's unused loads reach) fit a
    // 31-bit byte range and rows do not overlap.
    auto extent = [&](int64_t stride) -> int64_t {
        return stride >= dim ? (static_cast<int64_t>(a.Sk) - 1) * stride * 2 + dim * 2 : -1;
    };
    const int64_t k_ext = extent(a.ks[2]), v_ext = extent(a.vs[2]);
    const int64_t reach = (static_cast<int64_t>(a.Sk) + 2 * kBN) * 2 *
                          (a.ks[2] > a.vs[2] ? a.ks[2] : a.vs[2]);
    const bool buf = !gen && k_ext > 0 && v_ext > 0 && reach < (int64_t{1} << 30);
    a.k_bytes = buf ? static_cast<int>(k_ext) : 0;
    a.v_bytes = buf ? static_cast<int>(v_ext) : 0;
    const unsigned g = static_cast<unsigned>(grid);
    hipStream_t st = as_stream(stream);
    const bool neg = a.c < 0.0f && !prescale;  // the loop's max runs over c * s
    int n_cu = 0;
    if (buf && dim == kD) {
        int dev = 0;
        const hipError_t e = hipStreamGetDevice(st, &dev);
        if (e != hipSuccess) return static_cast<int>(e);
        n_cu = device_cus(dev);
        const SmallPlan sp = plan_small(static_cast<int64_t>(a.B) * a.H, a.Sq, n_cu);
        if (sp.use) {
            a.n_big = sp.n_big;
            a.n_small = sp.n_small;
            a.sm_k = sp.k;
            a.sm_big0 = sp.big0;
            a.sm_small0 = sp.small0;
            a.sm_big1 = sp.big1;
            a.sm_small1 = sp.small1;
            const unsigned gs = static_cast<unsigned>(sp.n_big + sp.n_small);
            if (neg)
                attention16_small_kernel<true><<<gs, kThreadsWG, 0, st>>>(a);
            else
                attention16_small_kernel<false><<<gs, kThreadsWG, 0, st>>>(a);
            return launch_status();
        }
    }
    if (workspace != nullptr && buf && dim == kD && !prescale && wv.shape[0] > 0) {
        const SplitPlan plan = plan_split(grid, (a.Sk + kBN - 1) / kBN, n_cu);
        const int64_t pieces = static_cast<int64_t>(plan.n_tail) * plan.split;
        if (plan.split > 1 && wv.shape[0] >= pieces * kWsSlotBytes) {
            a.n_full = plan.n_full;
            a.n_tail = plan.n_tail;
            a.split = plan.split;
            a.ws = reinterpret_cast<float *>(wv.data);
            const unsigned gs = static_cast<unsigned>(plan.n_full + pieces);
            if (neg)
                attention16_kernel<true, true><<<gs, kThreadsWG, 0, st>>>(a);
            else
                attention16_kernel<false, true><<<gs, kThreadsWG, 0, st>>>(a);
            const unsigned gm = static_cast<unsigned>(plan.n_tail * (kBM / 8));
            switch (plan.split) {
#define H3_MERGE(S) \
    case S: attention_merge_kernel<S><<<gm, 256, 0, st>>>(a); break;
                H3_MERGE(2) H3_MERGE(3) H3_MERGE(4) H3_MERGE(5) H3_MERGE(6) H3_MERGE(7) H3_MERGE(8)
#undef H3_MERGE
                default: return kInvalid;
            }
            return launch_status();
        }
    }
    if (buf && dim == kD) {
        if (neg)
            attention16_kernel<true, false><<<g, kThreadsWG, 0, st>>>(a);
        else
            attention16_kernel<false, false><<<g, kThreadsWG, 0, st>>>(a);
        return launch_status();
    }
#define H3_ATTN(N, B, D, G) \
    if (neg == N && buf == B && dim == D && gen == G) attention_fwd_kernel<N, B, D, G><<<g, kThreadsWG, 0, st>>>(a);
    H3_ATTN(false, false, 128, false) H3_ATTN(true, false, 128, false)
    H3_ATTN(false, true, 72, false) H3_ATTN(false, false, 72, false) H3_ATTN(true, true, 72, false)
    H3_ATTN(true, false, 72, false)
    H3_ATTN(false, false, 128, true) H3_ATTN(true, false, 128, true) H3_ATTN(false, false, 72, true)
    H3_ATTN(true, false, 72, true)
#undef H3_ATTN
    return launch_status();
}

}  // namespace

extern "C" NineToothedResult launch_h3_full_attention(NineToothedStream stream, NineToothedTensor q,
                                                      NineToothedTensor k, NineToothedTensor v,
                                                      NineToothedTensor scale, NineToothedTensor o) {
    return launch_attention(stream, q, k, v, scale, o, false, kD);
}

extern "C" NineToothedResult launch_h3_full_attention_ws(NineToothedStream stream, NineToothedTensor q,
                                                         NineToothedTensor k, NineToothedTensor v,
                                                         NineToothedTensor scale, NineToothedTensor o,
                                                         NineToothedTensor workspace) {
    return launch_attention(stream, q, k, v, scale, o, false, kD, &workspace);
}

extern "C" int64_t h3_full_attention_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Sk) {
    if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0 || Sq > kMaxSeqLen || Sk > kMaxSeqLen) return 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -1;
    const int64_t units = B * H * ((Sq + kBM - 1) / kBM);
    if (units > std::numeric_limits<int32_t>::max()) return 0;
    if (plan_small(B * H, Sq, device_cus(dev)).use) return 0;  // the 192-query last round needs none
    const SplitPlan plan = plan_split(units, (Sk + kBN - 1) / kBN, device_cus(dev));
    return plan.split > 1 ? static_cast<int64_t>(plan.n_tail) * plan.split * kWsSlotBytes : 0;
}

extern "C" NineToothedResult launch_h3_vision_attention_72(NineToothedStream stream, NineToothedTensor q,
                                                           NineToothedTensor k, NineToothedTensor v,
                                                           NineToothedTensor scale, NineToothedTensor o) {
    return launch_attention(stream, q, k, v, scale, o, false, 72);
}

extern "C" NineToothedResult launch_h3_full_attention_bf16_prescale(NineToothedStream stream, NineToothedTensor q,
                                                                    NineToothedTensor k, NineToothedTensor v,
                                                                    NineToothedTensor scale, NineToothedTensor o) {
    return launch_attention(stream, q, k, v, scale, o, true, kD);
}
