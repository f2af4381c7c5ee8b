/*
 * h3mi355x.h -- C ABI of the MI355X (gfx950) MiniMax-H3 DiT hot-path library
 * (libh3mi355x.so).
 *
 * The struct ABI and the entry points mirror the NineToothed HIP-AOT launchers
 * the reference links into InfiniCore:
 *   - `NineToothedTensor {data, shape, strides}` with strides in ELEMENTS and
 *     scalars passed as `{&double, NULL, NULL}`: the reference fills it at
 *     patches/InfiniCore.patch:1062-1073 (View<N>) and :1086 (eps scalar).
 *   - `NineToothedResult launch_<kernel>(NineToothedStream stream, NineToothedTensor ...)`
 *     with one tensor per kernel parameter in the kernel's declaration order:
 *     emitted at patches/ninetoothed.patch:138-146 and :259-260.
 *   - Return 0 on success, a hipError_t value otherwise; a launch whose grid
 *     would be empty returns 0 without touching the device
 *     (patches/ninetoothed.patch:304-307). Every launcher validates shapes,
 *     strides and alignment on the host before any HIP call and returns
 *     hipErrorInvalidValue (1) when they do not fit.
 *   - The launchers allocate nothing; every buffer is owned by the caller.
 *     They are reentrant and enqueue on the caller's stream (NULL = the
 *     default stream).
 *
 * Element types are fixed per entry point (the NineToothed tensor carries no
 * dtype): bf16 unless stated otherwise.
 */
#ifndef H3MI355X_H
#define H3MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *NineToothedStream;  /* hipStream_t */
typedef int NineToothedResult;    /* hipError_t */

typedef struct NineToothedTensor {
    void *data;
    uint64_t *shape;
    int64_t *strides;
} NineToothedTensor;

/* ---------------------------------------------------------------- attention */

/* Non-causal full attention forward, O = softmax(Q K^T * scale) V.
 * q, o: [B, H, Sq, 128]; k, v: [B, H, Sk, 128]; any strides (in elements, on
 * every dimension) with 2-byte aligned elements. Views with unit head-dim
 * stride and 16-byte aligned rows take the 16-byte tile path; any other view
 * runs on an element-strided path with the same arithmetic. Sq may differ from
 * Sk (keys past Sk are masked). scale: fp64 scalar. fp32 logits scaled by
 * scale * log2(e), exp2, bf16 P for the P.V product. The softmax's
 * stabilising maximum is each query's maximum over the first key tile, kept
 * for the later tiles (a workgroup recomputes its queries with the running
 * maximum when anything overflows against it), and the denominator sums the
 * same bf16-rounded P that weights V; the reference instead rescales at every
 * new running maximum and sums P in fp32 before rounding (both orders stay
 * within the operator's tolerance). Queries run in units of 256 per
 * workgroup; a launch whose last round of units would leave a quarter of the
 * CUs idle runs that round as units of 192 queries (same per-query
 * arithmetic). Allocates nothing.
 * Replaces launch_h3_full_attention (tools/h3_attention.py:25-41,104-121;
 * called at patches/InfiniCore.patch:1421-1422 with the [B,S,H,D] -> [B,H,S,D]
 * stride swap of :1403-1411). */
NineToothedResult launch_h3_full_attention(NineToothedStream stream, NineToothedTensor q,
                                           NineToothedTensor k, NineToothedTensor v,
                                           NineToothedTensor scale, NineToothedTensor o);

/* launch_h3_full_attention with a caller-provided workspace (uint8, 1-D,
 * contiguous, 256-byte aligned). One workgroup of 256 queries fills a CU, so
 * the launch runs in rounds of one unit per CU; when its last round is only
 * partly filled, the units of that round are split along the keys into pieces
 * that fill whole rounds, and a merge kernel combines their partial softmax
 * states (same algebra as the online rescale; results within the operator's
 * tolerance of the unsplit kernel, deterministic). The split is planned from
 * the shapes and the device's CU count and needs
 * h3_full_attention_workspace_bytes(B, H, Sq, Sk) bytes; a smaller workspace
 * (an empty one included) runs the unsplit kernel. No counterpart in the
 * reference: for callers that can pass scratch memory (the Python face
 * allocates it from torch's caching allocator). */
NineToothedResult launch_h3_full_attention_ws(NineToothedStream stream, NineToothedTensor q,
                                              NineToothedTensor k, NineToothedTensor v,
                                              NineToothedTensor scale, NineToothedTensor o,
                                              NineToothedTensor workspace);

/* Workspace bytes launch_h3_full_attention_ws uses for these shapes on the
 * current device: 0 when the last round is full or splitting it saves under
 * 3% of the launch, -1 on a HIP error. */
int64_t h3_full_attention_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Sk);

/* The same operator built for head dim 72 (the Qwen vision tower's heads):
 * q, o: [B, H, Sq, 72]; k, v: [B, H, Sk, 72]; views and masking as
 * launch_h3_full_attention, fp32_qk numerics in the reference's own order
 * (a running maximum with rescaling, fp32 denominator). Returns an error for any other
 * head dim, as launch_h3_full_attention does for a head dim other than 128.
 * Replaces launch_h3_vision_attention_72 (scripts/build_h3_attention.py:23-24,
 * tools/h3_attention.py:104-121 with head_dim=72; called at
 * patches/InfiniCore.patch:1421-1423 when q's head dim is 72, allowed by
 * :1376 under H3_QWEN_NINETOOTHED=1). */
NineToothedResult launch_h3_vision_attention_72(NineToothedStream stream, NineToothedTensor q,
                                                NineToothedTensor k, NineToothedTensor v,
                                                NineToothedTensor scale, NineToothedTensor o);

/* The `bf16_prescale` numerics of the same operator: q enters the product as
 * bf16(fp32(scale * log2(e)) * q) and the logits are used as they come
 * (tools/h3_attention.py:87-101, selected by make_attention(numerics=
 * "bf16_prescale"), :114). Same arguments and layouts as
 * launch_h3_full_attention. The reference's AOT build names this launcher
 * after its kernel_name (patches/ninetoothed.patch:138-146); this is the name
 * the library exports for it. */
NineToothedResult launch_h3_full_attention_bf16_prescale(NineToothedStream stream, NineToothedTensor q,
                                                         NineToothedTensor k, NineToothedTensor v,
                                                         NineToothedTensor scale, NineToothedTensor o);

/* Per-head fp8 (OCP e4m3fn) quantisation for the fp8 attention variants.
 * x: bf16 [B, H, S, 128] (any strides on B/H/S, unit stride on D, 16-byte
 * aligned rows); x8: uint8 storage of e4m3fn codes, same shape, either
 * D-contiguous (16-byte rows) or S-contiguous (the V^T layout the attention
 * kernels read V in; its D stride a multiple of 16); descale: fp32 [H]
 * (contiguous), receives amax_h / 448, the factor that maps x8 back to x.
 * A head with amax 0 gets descale 1 and all-zero codes. Codes are
 * e4m3fn(x * fp32(448 / amax_h)), one correctly rounded fp32 division,
 * saturated at +-448. B * H * S * 8 < 2^31 (otherwise the invalid-argument
 * result). The kernel chain clears, then accumulates, the amax in `descale`
 * itself (no workspace).
 * No counterpart in the reference (it has no fp8 path); its callers are the
 * fp8 attention users below. */
NineToothedResult launch_h3_quantize_fp8_per_head(NineToothedStream stream, NineToothedTensor x,
                                                  NineToothedTensor x8, NineToothedTensor descale);

/* Slots per head of a precomputed per-head amax (launch_h3_qkv_norm_rope_pack_fp8_vamax
 * writes them; launch_h3_quantize_fp8_per_head_slots reads them): the head's
 * amax is the maximum over its H3_AMAX_SLOTS slots. */
#define H3_AMAX_SLOTS 64

/* launch_h3_quantize_fp8_per_head with the per-head amax already folded into
 * slots by the producer, so only the code pass reads x: amax_slots: fp32
 * [H, H3_AMAX_SLOTS] (contiguous) holding maxima of |x| (the maximum over a
 * head's slots is its amax); x, x8, descale and the codes as for
 * launch_h3_quantize_fp8_per_head (bitwise the same codes and descales for
 * the same amax). amax_slots is only read.
 * No counterpart in the reference; its callers are the fp8 attention users
 * that quantise V after launch_h3_qkv_norm_rope_pack_fp8_vamax. */
NineToothedResult launch_h3_quantize_fp8_per_head_slots(NineToothedStream stream, NineToothedTensor x,
                                                        NineToothedTensor amax_slots, NineToothedTensor x8,
                                                        NineToothedTensor descale);

/* Two-term per-head e4m3fn split of x [B, H, S, 128] (bf16, 16-byte rows):
 * with y = sat(x * 448 / amax_h) in the code scale of
 * launch_h3_quantize_fp8_per_head, x8 = e4m3(y) (the same codes) and x8_lo =
 * e4m3(16 (y - x8)), exact residuals, so x ~= (x8 + x8_lo / 16) * descale[h]
 * (about 8 significant bits where one e4m3 term has 4). x8, x8_lo: uint8
 * [B, H, S, 128], D-contiguous, one set of strides for both; descale fp32
 * [H] = amax / 448 (the lo term's is descale / 16). Checks as
 * launch_h3_quantize_fp8_per_head, before any launch. No counterpart in the
 * reference; it feeds launch_h3_full_attention_fp8x2. */
NineToothedResult launch_h3_quantize_fp8_two_term(NineToothedStream stream, NineToothedTensor x,
                                                   NineToothedTensor x8, NineToothedTensor x8_lo,
                                                   NineToothedTensor descale);

/* fp8 (OCP e4m3fn) non-causal attention with per-head descales: the all-fp8
 * recipe. q8, k8: uint8 e4m3fn [B, H, S, 128] (unit stride on D, 16-byte
 * aligned rows); v8: uint8 e4m3fn [B, H, Sk, 128] with unit stride on S (see
 * the quantiser); q_descale, k_descale, v_descale: fp32 [H]; scale: fp64;
 * o: bf16 [B, H, Sq, 128]. Logits = (q8 . k8) q_descale k_descale scale in
 * fp32 on the fp8 MFMA; P is requantised per 64-key tile to e4m3(448 P)
 * (P <= 1 after the running-max shift); the fp32 P.V accumulator is scaled by
 * v_descale / 448 and divided by the denominator, the fp32 sum of the same
 * quantised weights e4m3(448 P) / 448.
 * No counterpart in the reference (fp8 attention is a new feature); same
 * callers as launch_h3_full_attention. */
NineToothedResult launch_h3_full_attention_fp8(NineToothedStream stream, NineToothedTensor q8,
                                               NineToothedTensor k8, NineToothedTensor v8,
                                               NineToothedTensor q_descale, NineToothedTensor k_descale,
                                               NineToothedTensor v_descale, NineToothedTensor scale,
                                               NineToothedTensor o);

/* fp8 attention with two-term Q and K (launch_h3_quantize_fp8_two_term): q8,
 * q8_lo and k8, k8_lo as q8, k8 of launch_h3_full_attention_fp8, each lo
 * tensor with its hi tensor's strides; v8 and the descales (of the hi terms)
 * as there. Logits = (q8.k8 + (q8.k8_lo + q8_lo.k8) / 16) q_descale
 * k_descale scale in fp32 on the fp8 MFMA, the lo operands' 1/16 applied as
 * the MFMA's E8M0 block scale, so the three products share one accumulator;
 * P and the output as launch_h3_full_attention_fp8, but the denominator is the
 * fp32 sum of the unquantised 448 P / 448 (summed on the VALU). It keeps
 * Q, K and V in e4m3 on the fp8 MFMA and meets the fp8 configuration's
 * relative RMS 5e-2 where the one-term recipe does not. No counterpart in the
 * reference; same callers as launch_h3_full_attention. */
NineToothedResult launch_h3_full_attention_fp8x2(NineToothedStream stream, NineToothedTensor q8,
                                                 NineToothedTensor q8_lo, NineToothedTensor k8,
                                                 NineToothedTensor k8_lo, NineToothedTensor v8,
                                                 NineToothedTensor q_descale, NineToothedTensor k_descale,
                                                 NineToothedTensor v_descale, NineToothedTensor scale,
                                                 NineToothedTensor o);

/* fp8 P.V with bf16 logits: q, k bf16 [B, H, S, 128] as for
 * launch_h3_full_attention, v8 and v_descale as for
 * launch_h3_full_attention_fp8. Keeps the Q K^T product (whose e4m3 error
 * grows with the logit magnitude) in bf16 and runs only P.V on the fp8 MFMA.
 * No counterpart in the reference; same callers as launch_h3_full_attention. */
NineToothedResult launch_h3_full_attention_fp8pv(NineToothedStream stream, NineToothedTensor q,
                                                 NineToothedTensor k, NineToothedTensor v8,
                                                 NineToothedTensor v_descale, NineToothedTensor scale,
                                                 NineToothedTensor o);

/* ---------------------------------------------------------------- pointwise */

/* out = bf16(up * bf16(g / (1 + exp(-g)))), g = fp32(gate). [B, S, F], any
 * strides. Replaces launch_h3_swiglu_exact (tools/h3_pointwise.py:9-34; called
 * at patches/InfiniCore.patch:1101). */
NineToothedResult launch_h3_swiglu_exact(NineToothedStream stream, NineToothedTensor up,
                                         NineToothedTensor gate, NineToothedTensor out);

/* RMSNorm with every intermediate rounded to bf16 (tools/h3_pointwise.py:46-57):
 * x, out [B, S, W]; weight [W]; eps fp64 scalar. The _128 and _5376 entry
 * points are the reference's width-specialised launchers
 * (tools/h3_pointwise.py:60-70; called at patches/InfiniCore.patch:1087-1089)
 * and require that width; launch_h3_rms_exact accepts any width. */
NineToothedResult launch_h3_rms_exact(NineToothedStream stream, NineToothedTensor x,
                                      NineToothedTensor weight, NineToothedTensor eps,
                                      NineToothedTensor out);
NineToothedResult launch_h3_rms_exact_128(NineToothedStream stream, NineToothedTensor x,
                                          NineToothedTensor weight, NineToothedTensor eps,
                                          NineToothedTensor out);
NineToothedResult launch_h3_rms_exact_5376(NineToothedStream stream, NineToothedTensor x,
                                           NineToothedTensor weight, NineToothedTensor eps,
                                           NineToothedTensor out);

/* RMSNorm + AdaLN: out = bf16(bf16(bf16(rms(x) * w) * bf16(1 + scale)) + shift).
 * x, scale, shift, out [B, S, W] (scale/shift may broadcast with stride 0);
 * weight [W]; eps fp64. Replaces launch_h3_rms_modulate_exact
 * (tools/h3_pointwise.py:73-108; called at patches/InfiniCore.patch:1117-1118),
 * width-generic. */
NineToothedResult launch_h3_rms_modulate_exact(NineToothedStream stream, NineToothedTensor x,
                                               NineToothedTensor weight, NineToothedTensor eps,
                                               NineToothedTensor scale, NineToothedTensor shift,
                                               NineToothedTensor out);

/* 3-axis NeoX RoPE on channels 0..95 of [S, H, 128] (rotate-half pairs i,
 * i+48; channels 96..127 pass through); cos/sin [S, 48] indexed by dim 0.
 * x0/x1/xp and y0/y1/yp are the same views passed three times, as the
 * reference's callers do. Replaces launch_h3_rope_exact
 * (tools/h3_pointwise.py:184-231; called at patches/InfiniCore.patch:1131). */
NineToothedResult launch_h3_rope_exact(NineToothedStream stream, NineToothedTensor x0,
                                       NineToothedTensor x1, NineToothedTensor xp,
                                       NineToothedTensor cos, NineToothedTensor sin,
                                       NineToothedTensor y0, NineToothedTensor y1,
                                       NineToothedTensor yp);

/* out = bf16(x + bf16(gate * y)), [B, S, W], any strides (gate typically
 * broadcast). Replaces launch_h3_gated_residual_exact
 * (tools/h3_pointwise.py:112-136; called at patches/InfiniCore.patch:1144). */
NineToothedResult launch_h3_gated_residual_exact(NineToothedStream stream, NineToothedTensor x,
                                                 NineToothedTensor gate, NineToothedTensor y,
                                                 NineToothedTensor out);

/* residual = bf16(x + bf16(gate * y)); out = rms_modulate(residual).
 * Replaces launch_h3_gated_residual_rms_modulate_exact
 * (tools/h3_pointwise.py:139-182; called at patches/InfiniCore.patch:1161-1163),
 * width-generic. */
NineToothedResult launch_h3_gated_residual_rms_modulate_exact(
    NineToothedStream stream, NineToothedTensor x, NineToothedTensor gate, NineToothedTensor y,
    NineToothedTensor weight, NineToothedTensor eps, NineToothedTensor scale,
    NineToothedTensor shift, NineToothedTensor residual, NineToothedTensor out);

/* ------------------------------------------- per-token AdaLN rows (indexed) */

/* The three AdaLN ops of a DiT block over all tokens in ONE launch each, every
 * token taking its own row of the modulation tables. The reference runs them
 * once per run-length segment of its AdaLN indices, on stride-0 broadcast
 * views of the segment's modulation row, after copying the indices to the
 * host to build the segments (patches/InfiniLM.patch:1353-1397 per-segment
 * launches, :1765-1793 segment construction); these entry points read the
 * per-token indices on the device instead, with no host round trip, and give
 * the same bits as the per-segment launches.
 *
 * Common arguments:
 *   - x, y, out, residual: bf16 [B, S, W] as for the non-indexed entry points;
 *   - scale, shift, gate: bf16 tables [R, W] (any row stride, e.g. column
 *     blocks of the [R, 6 * W] modulation matrix: shift_msa 0, scale_msa 1,
 *     gate_msa 2, shift_mlp 3, scale_mlp 4, gate_mlp 5, as at
 *     patches/InfiniLM.patch:1375); all tables of one call have the same R >= 1;
 *   - index: int64 [B, S] (any strides), token (b, s) uses row index[b, s] of
 *     every table. Indices must lie in [0, R); the kernels clamp any other
 *     value into that range so that no index reads outside the tables (the
 *     reference's host-side narrow rejects them: callers that need the error
 *     check the range before the launch).
 * No single-launch counterpart in the reference; callers are the DiT block's
 * AdaLN sites named above. */

/* launch_h3_rms_modulate_exact with scale/shift rows index[b, s] of the tables. */
NineToothedResult launch_h3_rms_modulate_indexed(NineToothedStream stream, NineToothedTensor x,
                                                 NineToothedTensor weight, NineToothedTensor eps,
                                                 NineToothedTensor scale, NineToothedTensor shift,
                                                 NineToothedTensor index, NineToothedTensor out);

/* launch_h3_gated_residual_rms_modulate_exact with gate/scale/shift rows
 * index[b, s] of the tables. */
NineToothedResult launch_h3_gated_residual_rms_modulate_indexed(
    NineToothedStream stream, NineToothedTensor x, NineToothedTensor gate, NineToothedTensor y,
    NineToothedTensor weight, NineToothedTensor eps, NineToothedTensor scale,
    NineToothedTensor shift, NineToothedTensor index, NineToothedTensor residual,
    NineToothedTensor out);

/* launch_h3_gated_residual_exact with the gate row index[b, s] of the table. */
NineToothedResult launch_h3_gated_residual_indexed(NineToothedStream stream, NineToothedTensor x,
                                                   NineToothedTensor gate, NineToothedTensor y,
                                                   NineToothedTensor index, NineToothedTensor out);

/* ----------------------------------------------------------------- q/k + RoPE */

/* Per-(token, head) RMSNorm over 128 channels (weight [128]) then the
 * rotate-half RoPE of launch_h3_rope_exact, on x [T, P, Hs, 128] (any strides)
 * written to out [T, P, Hs, 128] (any strides, e.g. a permuted all-to-all send
 * buffer); cos/sin [T, 48]. Views repeated as in the reference.
 * Replaces launch_h3_qk_norm_rope (tools/h3_pointwise.py:234-294,370-402;
 * called at patches/InfiniCore.patch:1180-1182). */
NineToothedResult launch_h3_qk_norm_rope(NineToothedStream stream, NineToothedTensor x0,
                                         NineToothedTensor x1, NineToothedTensor xp,
                                         NineToothedTensor w0, NineToothedTensor w1,
                                         NineToothedTensor wp, NineToothedTensor eps,
                                         NineToothedTensor cos, NineToothedTensor sin,
                                         NineToothedTensor y0, NineToothedTensor y1,
                                         NineToothedTensor yp);

/* The q, k and v head rows of one head group in ONE launch, in the layout of
 * the reference's sequence-parallel attention (patches/InfiniLM.patch:1071-1110):
 * q and k get launch_h3_qk_norm_rope's per-head RMSNorm + rotate-half RoPE,
 * with their cos/sin rows gathered from the RoPE cache through the token
 * positions, and v is copied.
 *   q, k, v: bf16 [T, P, Hs, 128], any strides (the by-rank views of the fused
 *     [T, 3, P * Hs, 128] projection, :1093-1097);
 *   q_out, k_out, v_out: bf16 [T, P, Hs, 128], any strides (the permuted
 *     [P, T, Hs, 128] all-to-all send buffers, :1098-1102);
 *   q_weight, k_weight: bf16 [128]; eps: fp64 scalar;
 *   cos, sin: bf16 [N, 48], the halves of the [N, 96] RoPE cache;
 *   positions: int64 [T], token t's row of the cache (a value outside
 *     [0, N) is clamped into it; the kernel never reads outside the cache).
 * Per-step bf16 rounding as launch_h3_qk_norm_rope; v is copied bit for bit.
 * Replaces, per head group, the gather_rows of the cache (:1077-1080), the two
 * launch_h3_qk_norm_rope calls (:1098-1102, via patches/InfiniCore.patch:1180-1182)
 * and the v send-block copy (:1063-1069,1104). */
NineToothedResult launch_h3_qkv_norm_rope_pack(NineToothedStream stream, NineToothedTensor q,
                                               NineToothedTensor k, NineToothedTensor v,
                                               NineToothedTensor q_weight, NineToothedTensor k_weight,
                                               NineToothedTensor eps, NineToothedTensor cos,
                                               NineToothedTensor sin, NineToothedTensor positions,
                                               NineToothedTensor q_out, NineToothedTensor k_out,
                                               NineToothedTensor v_out);

/* launch_h3_qkv_norm_rope_pack with an fp8 epilogue for q and k, the producer
 * of launch_h3_full_attention_fp8's q8 / k8: q8, k8 are uint8 e4m3fn codes
 * [T, P, Hs, 128] (any strides; 8-byte aligned rows for the vector path),
 * codes = e4m3fn(sat(bf16(y) * 448 / bound)) where y is the value
 * launch_h3_qkv_norm_rope_pack writes and bound = fp32(sqrt(128) * 1.03125) *
 * max|weight|, an upper bound of |y| that RMSNorm + RoPE guarantee for any
 * input, so no absmax pass over the data is needed; q_descale, k_descale:
 * fp32 [P * Hs] (contiguous), every head receives bound / 448 (1 for a zero
 * weight). v_out: bf16 as before (V's scale depends on its data: quantise it
 * with launch_h3_quantize_fp8_per_head).
 * No counterpart in the reference (it has no fp8 path); callers are the fp8
 * attention users, at the same site as launch_h3_qkv_norm_rope_pack. */
NineToothedResult launch_h3_qkv_norm_rope_pack_fp8(NineToothedStream stream, NineToothedTensor q,
                                                   NineToothedTensor k, NineToothedTensor v,
                                                   NineToothedTensor q_weight, NineToothedTensor k_weight,
                                                   NineToothedTensor eps, NineToothedTensor cos,
                                                   NineToothedTensor sin, NineToothedTensor positions,
                                                   NineToothedTensor q8, NineToothedTensor k8,
                                                   NineToothedTensor v_out, NineToothedTensor q_descale,
                                                   NineToothedTensor k_descale);

/* launch_h3_qkv_norm_rope_pack_fp8 that also folds V's per-head amax while
 * copying v, so that V's quantisation (launch_h3_quantize_fp8_per_head_slots)
 * needs only its code pass: v_amax: fp32 [P * Hs, H3_AMAX_SLOTS]
 * (contiguous), cleared by the launch and then filled with maxima of |v| per
 * head (head index p * Hs + h; the maximum over a head's slots is the amax of
 * that head's rows in this launch). P * Hs <= 1024. With several ranks, the
 * receiving rank's amax of a head is the maximum of the senders' slots.
 * Everything else as launch_h3_qkv_norm_rope_pack_fp8. Reference site of the
 * v copy: patches/InfiniLM.patch:1063-1069,1104. */
NineToothedResult launch_h3_qkv_norm_rope_pack_fp8_vamax(
    NineToothedStream stream, NineToothedTensor q, NineToothedTensor k, NineToothedTensor v,
    NineToothedTensor q_weight, NineToothedTensor k_weight, NineToothedTensor eps, NineToothedTensor cos,
    NineToothedTensor sin, NineToothedTensor positions, NineToothedTensor q8, NineToothedTensor k8,
    NineToothedTensor v_out, NineToothedTensor q_descale, NineToothedTensor k_descale, NineToothedTensor v_amax);

/* launch_h3_qkv_norm_rope_pack_fp8_vamax with q and k as two-term e4m3 codes
 * for launch_h3_full_attention_fp8x2: q8, k8 the one-term codes (the weight
 * bound's scale, bitwise those of launch_h3_qkv_norm_rope_pack_fp8) and
 * q8_lo, k8_lo = e4m3(16 (y - code)) for y the bf16 output in code units, each
 * lo tensor with its hi tensor's shape and strides; q_descale, k_descale the
 * hi terms' (the lo terms' are 1/16 of them). So the fp8 configuration's
 * Q and K need no quantiser pass after the pack. No counterpart in the
 * reference; the v copy it extends is patches/InfiniLM.patch:1063-1069,1104. */
NineToothedResult launch_h3_qkv_norm_rope_pack_fp8x2_vamax(
    NineToothedStream stream, NineToothedTensor q, NineToothedTensor k, NineToothedTensor v,
    NineToothedTensor q_weight, NineToothedTensor k_weight, NineToothedTensor eps, NineToothedTensor cos,
    NineToothedTensor sin, NineToothedTensor positions, NineToothedTensor q8, NineToothedTensor q8_lo,
    NineToothedTensor k8, NineToothedTensor k8_lo, NineToothedTensor v_out, NineToothedTensor q_descale,
    NineToothedTensor k_descale, NineToothedTensor v_amax);

/* Maximum heads of launch_h3_qkv_norm_rope_pack_fp8_noalloc (the rows of its
 * static slot array). */
#define H3_NOALLOC_MAX_HEADS 1024

/* launch_h3_qkv_norm_rope_pack_fp8_vamax followed by
 * launch_h3_quantize_fp8_per_head_slots of v_out, with V's amax slots in a
 * static device array of the library instead of a caller's buffer, so that
 * the call allocates nothing and takes no workspace: for one rank (P = 1,
 * q/k/v/q8/k8/v_out [T, 1, Hs, 128]), Hs <= H3_NOALLOC_MAX_HEADS. v8: uint8
 * e4m3fn [1, Hs, T, 128] (any layout the quantiser takes; the fp8 attention
 * reads V S-contiguous), v_descale: fp32 [Hs]; v_out is quantised as the
 * [1, Hs, T, 128] view of its rows. Everything else as
 * launch_h3_qkv_norm_rope_pack_fp8_vamax, and q8, k8, v_out, the descales and
 * v8 are bitwise those of the two-call sequence. Every argument of both steps
 * is checked before the first HIP call; P != 1 or Hs > H3_NOALLOC_MAX_HEADS
 * returns hipErrorInvalidValue. The slot array (256 KiB per device, kept
 * until the process ends) is shared by every call on a device: calls that
 * overlap on one device (other streams, other threads) race; calls on one
 * stream do not. No counterpart in the reference: it is for callers that
 * cannot allocate device memory or pass a workspace (code under HIP graph
 * capture, fixed serving loops). */
NineToothedResult launch_h3_qkv_norm_rope_pack_fp8_noalloc(
    NineToothedStream stream, NineToothedTensor q, NineToothedTensor k, NineToothedTensor v,
    NineToothedTensor q_weight, NineToothedTensor k_weight, NineToothedTensor eps, NineToothedTensor cos,
    NineToothedTensor sin, NineToothedTensor positions, NineToothedTensor q8, NineToothedTensor k8,
    NineToothedTensor v_out, NineToothedTensor q_descale, NineToothedTensor k_descale, NineToothedTensor v8,
    NineToothedTensor v_descale);

/* The same RMSNorm followed by an interleaved-pair RoPE over all 128
 * channels: pair i = channels (2i, 2i+1), angle table cos/sin [T, 64]
 * (rotary channels split 32/48/48 over the t/h/w axes). Per-step bf16
 * rounding as launch_h3_qk_norm_rope. No counterpart in the reference (its
 * table is rotate-half over 96 channels, tools/h3_pointwise.py:184-214); it
 * serves callers whose RoPE uses the interleaved 32/48/48 layout. */
NineToothedResult launch_h3_qk_norm_rope_interleaved(NineToothedStream stream, NineToothedTensor x,
                                                     NineToothedTensor weight, NineToothedTensor eps,
                                                     NineToothedTensor cos, NineToothedTensor sin,
                                                     NineToothedTensor out);

/* launch_h3_qk_norm_rope_interleaved for q and k in ONE pass: for each
 * (t, p, h), the q row (weight q_weight) and the k row (weight k_weight) are
 * taken by one lane group against the same cos/sin [T, 64] entries, so the
 * table is read once for both. q, k, q_out, k_out: bf16 [T, P, Hs, 128], any
 * strides, all of one shape; results bitwise equal to two calls of
 * launch_h3_qk_norm_rope_interleaved. No counterpart in the reference: it is
 * the q+k form of the fused QK-RMSNorm + 3D RoPE workload (q and k
 * [1, 8192, 14, 128], 32/48/48 interleaved rotary channels). */
NineToothedResult launch_h3_qk_norm_rope_interleaved_qk(NineToothedStream stream, NineToothedTensor q,
                                                        NineToothedTensor k, NineToothedTensor q_weight,
                                                        NineToothedTensor k_weight, NineToothedTensor eps,
                                                        NineToothedTensor cos, NineToothedTensor sin,
                                                        NineToothedTensor q_out, NineToothedTensor k_out);

/* H3's RoPE table: cos/sin[t, a*16 + k] = bf16(cos/sin(fp32(position[t, a]) *
 * (1 / power[k]))), position fp64 [T, 3], power fp32 [16], cos/sin bf16
 * [T, 48] views (the halves of a [T, 96] cache). Replaces launch_h3_rope_cache
 * (tools/h3_pointwise.py:405-442; called at patches/InfiniCore.patch:1197). */
NineToothedResult launch_h3_rope_cache(NineToothedStream stream, NineToothedTensor position,
                                       NineToothedTensor power, NineToothedTensor cos,
                                       NineToothedTensor sin);

/* ------------------------------------------------------------ measurement */

/* The HBM ceilings of the pointwise ops' access patterns, for judging their
 * achieved GB/s: out0 = in0 xor in1 and out1 = in1 (in1 / out1 may be empty
 * tensors: one input / one output), bitwise. launch_h3_calibration_stream: 1-D
 * uint8 [n] views (n a multiple of 16, 16-byte aligned, contiguous), one flat
 * non-temporal pass, two 16-byte chunks per thread. launch_h3_calibration_row_copy:
 * 2-D uint8 [rows, row_bytes] (row_bytes 14 KiB or 36 KiB, contiguous rows),
 * one wave per row with every load of the row issued before its first store,
 * the pattern of the RMS family. No counterpart in the reference; the caller
 * is bench.py, which times each op beside the copy of its bytes. */
NineToothedResult launch_h3_calibration_stream(NineToothedStream stream, NineToothedTensor in0,
                                               NineToothedTensor in1, NineToothedTensor out0,
                                               NineToothedTensor out1);
NineToothedResult launch_h3_calibration_row_copy(NineToothedStream stream, NineToothedTensor in0,
                                                 NineToothedTensor in1, NineToothedTensor out0,
                                                 NineToothedTensor out1);

/* The bf16 MFMA rate the part sustains, against which the attention kernels
 * are judged beside the published peak: out fp32 [blocks, 512] (contiguous);
 * each of the 512 threads of each of the blocks runs `iterations` (fp64
 * scalar, 0..1e7) rounds of 16 v_mfma_f32_32x32x16_bf16 (4 independent chains,
 * 32768 flop each per wave) on operands bf16 [512, 64] (contiguous, 16-byte
 * aligned: thread t's 4 A and 4 B fragments of 8 values at row t), and writes
 * the sum of its accumulators. All-ones operands give 4096 * iterations per
 * thread. No counterpart in the reference (measurement only). */
NineToothedResult launch_h3_calibration_mfma(NineToothedStream stream, NineToothedTensor operands,
                                             NineToothedTensor out, NineToothedTensor iterations);

/* launch_h3_calibration_mfma with v_mfma_f32_16x16x32_bf16: each round is 32
 * products of 16384 flop per wave over 8 independent chains (the same flops
 * per round), same arguments and checks; all-ones operands again give
 * 4096 * iterations per thread. No counterpart in the reference (measurement
 * only). */
NineToothedResult launch_h3_calibration_mfma_16x16x32(NineToothedStream stream, NineToothedTensor operands,
                                                      NineToothedTensor out, NineToothedTensor iterations);

/* The fp8 MFMA rate, for the fp8 attention kernels: launch_h3_calibration_mfma
 * with v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 A and B, unit block scales),
 * 16 products of 131072 flop per wave and round over 4 chains, on operands
 * uint8 [512, 256] (e4m3 codes, contiguous, 16-byte aligned: thread t's 4 A
 * and 4 B fragments of 32 codes at row t); out and iterations as there.
 * All-ones operands (code 0x38) give 16384 * iterations per thread. No
 * counterpart in the reference (measurement only). */
NineToothedResult launch_h3_calibration_mfma_fp8(NineToothedStream stream, NineToothedTensor operands,
                                                 NineToothedTensor out, NineToothedTensor iterations);

#ifdef __cplusplus
}
#endif

#endif /* H3MI355X_H */
