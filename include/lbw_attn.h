/*
 * lbw_attn.h -- C-ABI of liblbw_attn.so: Sage-style quantized DiT attention for MI355X (gfx950).
 *
 * Replaces, for the plain self-attention call of the LingBot-World DiT, the native boundary the reference
 * binds through SageAttention 2.2's pybind functions:
 *   - lingbot/layers/attention.py:31-36    sageattn(q, k, v, tensor_layout="NHD", ...)
 *   - lingbot/layers/sage_preq.py:116      per_warp_int8_cuda(q, k, km, BLKQ=128, WARPQ=32, BLKK=64)
 *   - lingbot/layers/sage_preq.py:121-124  V scale + fp8 V quantisation (_v_scale, _quant_v)
 *   - lingbot/layers/sage_preq.py:126-127  sm89_compile.qk_int8_sv_f8_accum_f16_fuse_v_scale_attn_inst_buf(...)
 *   - experiments/modules/sage_kvq.py:78-111  write_chunk / requant_all / attend over a pre-quantised cache
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers owned by the caller; nothing is allocated, freed or synchronised here,
 *     so every call can be recorded into a HIP graph. `stream` is a hipStream_t (0 = default stream).
 *   - Sizes and strides are int64 element counts. bf16 tensors are passed as raw 16-bit words.
 *   - The head dimension is 128 and must be contiguous (stride 1).
 *   - Return value: LBW_OK (0) or one of the LBW_E* codes below; lbw_status_string() names it.
 *
 * Quantised ring cache (one per layer; `layers` of them back to back, slot capacity `cap` tokens, a multiple
 * of 64; BH = batch * heads; nb = cap / 64):
 *   k8      int8  [layers][slots][BH][cap][128]       K - mean, per 64-token block int8
 *   k_scale fp32  [layers][slots][BH][nb]             amax / 127 of each 64-token block
 *   km      fp32  [layers][slots][BH][128]            per-(head, channel) chunk mean (a bf16 value)
 *   v8      uint8 [layers][slots][BH][nb][128][64]    e4m3 V, per 64-key block: [channel][position]
 *   v8lo    uint8 [layers][slots][BH][nb][128][48]    optional residual plane: bf6 (OCP e3m2) codes of y - hi,
 *                                                      y = V / 2^e, hi = e4m3(y); per block [channel][48 bytes]
 *   v_scale uint8 [layers][slots][BH][nb][256]        E8M0 V scales of each 64-key block: one power of two 2^e per
 *                                                      (key group, channel) with amax / 2^e in (224, 448] (amax over
 *                                                      the group's 32 keys, floored at 1e-7), so y is exact; byte
 *                                                      (32 g + c % 32) * 4 + c / 32 = 127 + e of channel c, group g
 * Key k of a block is in group k / 32 (its 32-key half).
 * With the residual plane, V = (hi + lo) * 2^e to about 7 significant bits instead of 4 (|y - hi| <= 16 fits bf6
 * unscaled). A residual row holds the 32 codes of each key group g (positions 16g .. 16g + 15, then 32 + 16g ..
 * 47 + 16g: the keys 32g .. 32g + 31) as 24 bytes (code k of the group at bits 6k .. 6k + 5): group 0's bytes 0-15,
 * group 1's bytes 0-15, then the groups' bytes 16-23, group 1's first in channels whose bit 4 is set. A NaN or an
 * infinity in V gives hi a NaN code and lo a code of magnitude 28.
 * Position p of a 64-key V block holds key 32*((p&31)>>4) + 8*((p>>2)&3) + 4*(p>>5) + (p&3).
 *
 * Quantised Q (per call): q8 int8 [BH][Lp][128], q_scale fp32 [BH][Lp/32], Lp = Lq rounded up to 256;
 * bias fp32 [n_seg][BH][Lp] holds q . km of each attended chunk (only read when n_seg > 1).
 */
#ifndef LBW_ATTN_H
#define LBW_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  LBW_OK = 0,
  LBW_E_NULL = 1,        /* a required pointer is null */
  LBW_E_SHAPE = 2,       /* a size is out of range or inconsistent */
  LBW_E_ALIGN = 3,       /* a pointer or stride breaks the 16-byte alignment the kernels load with */
  LBW_E_DEVICE = 4,      /* the current device is not gfx950 */
  LBW_E_LAUNCH = 5,      /* the kernel launch failed */
  LBW_E_SEGMENTS = 6,    /* the attended-chunk table is invalid */
  LBW_E_SCRATCH = 7      /* the problem needs more scratch than lbw_attn_fwd_noalloc's fixed array holds */
};

#define LBW_HEAD_DIM 128
#define LBW_MAX_SEGMENTS 8

/* The 16-bit input formats of lbw_kv_requant and lbw_quant_q (their `dtype` argument). */
#define LBW_DTYPE_BF16 0
#define LBW_DTYPE_FP16 1

/* Name of a status code. */
const char* lbw_status_string(int status);

/* Library version (major * 10000 + minor * 100 + patch). */
int lbw_version(void);

/* Bytes of scratch `lbw_kv_requant` needs for `layers` chunks of `len` tokens and `bh` batch*heads. */
int64_t lbw_kv_requant_workspace_bytes(int64_t layers, int64_t bh, int64_t len);

/*
 * Quantise K and V chunks of `len` tokens (bf16, or fp16 with dtype LBW_DTYPE_FP16: 16-bit words either way) into
 * slot `slot` of `layers` consecutive layer caches: the per-(head, channel) K mean (rounded to the inputs' own
 * format, as the reference's k.mean of such a tensor), K - mean as int8 per 64-token block, V as e4m3 with one scale
 * per (64-key block, key group, channel), plus the residual plane when v8lo is not null. Replaces sage_kvq.requant_all + write_chunk (experiments/modules/sage_kvq.py:78-98)
 * and Sage's per_warp_int8 K part / per_channel_fp8 (lingbot/layers/sage_preq.py:115-124).
 * k/v element (layer l, batch b, token t, head h, channel d) sits at l*s_layer + b*s_batch + t*s_tok
 * + h*s_head + d. `workspace` holds lbw_kv_requant_workspace_bytes() bytes, 16-byte aligned; its
 * contents need not be preserved between calls, and calls that share a workspace must not overlap. Tokens in [len, ceil64(len)) of the slot are written
 * as zero; blocks past ceil64(len) are left untouched (the attention never reads them).
 */
int lbw_kv_requant(const uint16_t* k, const uint16_t* v, int dtype,
                   int64_t layers, int64_t batch, int64_t len, int64_t heads,
                   int64_t k_s_layer, int64_t k_s_batch, int64_t k_s_tok, int64_t k_s_head,
                   int64_t v_s_layer, int64_t v_s_batch, int64_t v_s_tok, int64_t v_s_head,
                   int8_t* k8, float* k_scale, float* km, uint8_t* v8, uint8_t* v8lo, uint8_t* v_scale,
                   int64_t slots, int64_t cap, int64_t slot,
                   void* workspace, void* stream);

/*
 * Quantise Q [batch][lq][heads][128] (bf16, or fp16 with dtype LBW_DTYPE_FP16; strides s_batch, s_tok, s_head) to
 * int8 with one scale per
 * 32 rows (Sage per_warp_int8 Q part with BLKQ=128, WARPQ=32: lingbot/layers/sage_preq.py:116,
 * experiments/modules/sage_kvq.py:104). When n_seg > 1 it also writes bias[c][bh][row] = q . km of chunk
 * seg_slot[c] of the (layer-offset) cache `km` with `slots` slots; km is then 16-byte aligned. seg_slot is a
 * host array.
 */
int lbw_quant_q(const uint16_t* q, int dtype, int64_t batch, int64_t lq, int64_t heads,
                int64_t s_batch, int64_t s_tok, int64_t s_head,
                int8_t* q8, float* q_scale,
                const float* km, int64_t slots, int n_seg, const int32_t* seg_slot, float* bias,
                void* stream);

/*
 * The self-attention prologue of a DiT block for Q, fused with its quantisation: q [batch][lq][heads * 128] bf16
 * projection rows (strides s_batch, s_tok; channels contiguous) -> RMSNorm over all heads * 128 channels times
 * norm_weight (bf16, heads * 128) with eps -> 3-axis rotary embedding -> the outputs of lbw_quant_q on that roped Q
 * (q8, q_scale and, when n_seg > 1, bias; same layouts and conditions), plus the roped bf16 Q itself in q_out
 * [batch][lq][heads][128] (strides o_s_*) when q_out is not null. Replaces norm_q + causal_rope_apply + the Q
 * quantisation (lingbot/models/lingbot_world/transformer.py:201-211 with lingbot/layers/sage_preq.py:116).
 * rope: float64 (cos, sin) table [rope_rows][64][2] (the model's freqs, transformer.py:553-556), 16-byte aligned;
 * token t takes frame row start_frame + t / (grid_h grid_w) for pairs 0..21, row (t / grid_w) % grid_h for pairs
 * 22..42 and row t % grid_w for pairs 43..63 (causal_rope_freqs, transformer.py:53-77). heads <= 16.
 */
int lbw_norm_rope_quant_q(const uint16_t* q, int64_t batch, int64_t lq, int64_t heads,
                          int64_t s_batch, int64_t s_tok, const uint16_t* norm_weight, float eps,
                          const double* rope, int64_t rope_rows, int64_t grid_h, int64_t grid_w,
                          int64_t start_frame, int8_t* q8, float* q_scale,
                          const float* km, int64_t slots, int n_seg, const int32_t* seg_slot, float* bias,
                          uint16_t* q_out, int64_t o_s_batch, int64_t o_s_tok, int64_t o_s_head, void* stream);

/*
 * The same prologue for K, fused with the chunk's re-quant: k [batch][len][heads * 128] bf16 projection rows ->
 * RMSNorm (norm_weight, eps) -> rotary embedding (rope table and grid as above) -> the roped bf16 K in k_out
 * [batch][len][heads][128] (strides o_s_*), and the ring slot exactly as lbw_kv_requant (one layer) writes it from
 * that roped K and v [batch][len][heads][128] (strides v_s_*). The K statistics are taken while the roped rows
 * are in registers, so the roped K is read back once (by the quantiser) instead of twice. `workspace` holds
 * lbw_kv_requant_workspace_bytes(1, batch * heads, len) bytes. Replaces norm_k + causal_rope_apply + kvc.write +
 * the K/V quantisation (transformer.py:202-218; experiments/modules/sage_kvq.py:78-98).
 */
int lbw_norm_rope_kv_requant(const uint16_t* k, const uint16_t* v, int64_t batch, int64_t len, int64_t heads,
                             int64_t k_s_batch, int64_t k_s_tok, int64_t v_s_batch, int64_t v_s_tok,
                             int64_t v_s_head, const uint16_t* norm_weight, float eps,
                             const double* rope, int64_t rope_rows, int64_t grid_h, int64_t grid_w,
                             int64_t start_frame, uint16_t* k_out, int64_t o_s_batch, int64_t o_s_tok,
                             int64_t o_s_head, int8_t* k8, float* k_scale, float* km, uint8_t* v8, uint8_t* v8lo,
                             uint8_t* v_scale, int64_t slots, int64_t cap, int64_t slot, void* workspace,
                             void* stream);

/*
 * The cross-attention context in the layout lbw_cross_attn_fwd reads: k, v [batch][lk][heads][128] bf16 (strides
 * *_s_batch, *_s_tok, *_s_head) -> k_prep [batch * heads][Lkp][128] and vt_prep [batch * heads][128][Lkp] (V
 * transposed; within each 16-key group the keys are stored in the order 0-3, 8-11, 4-7, 12-15), Lkp = ceil64(lk),
 * padding keys zero. The reference computes the cross-attention K / V once per
 * generation and keeps them (crossattn_cache, lingbot/models/lingbot_world/transformer.py:251-266); this is the
 * one-time step that goes with it.
 */
int lbw_cross_prepare(const uint16_t* k, const uint16_t* v, int64_t batch, int64_t lk, int64_t heads,
                      int64_t k_s_batch, int64_t k_s_tok, int64_t k_s_head,
                      int64_t v_s_batch, int64_t v_s_tok, int64_t v_s_head,
                      uint16_t* k_prep, uint16_t* vt_prep, void* stream);

/*
 * Cross-attention, bf16 in / bf16 out with fp32 accumulation: q [batch][lq][heads][128] (strides q_s_*) against a
 * context prepared by lbw_cross_prepare (lk keys), softmax(q k^T * sm_scale) v into out (strides o_s_*). k_lens:
 * null, or a host array of `batch` key counts (1 .. lk) -- the varlen key lengths of the reference's flash call.
 * batch <= 64. Replaces flash_attention(q, k, v, k_lens) of the cross-attention (transformer.py:272; the paper's
 * FlashAttention, reference/wan/modules/attention.py:23-129).
 */
int lbw_cross_attn_fwd(const uint16_t* q, int64_t batch, int64_t lq, int64_t heads,
                       int64_t q_s_batch, int64_t q_s_tok, int64_t q_s_head,
                       const uint16_t* k_prep, const uint16_t* vt_prep, int64_t lk, const int32_t* k_lens,
                       uint16_t* out, int64_t o_s_batch, int64_t o_s_tok, int64_t o_s_head,
                       float sm_scale, void* stream);

/*
 * Rowwise FP8 quantisation of x [rows][cols] (bf16, or fp32 when x_is_fp32; row stride s_row elements, cols a
 * multiple of 16): scale[row] = max(amax(|x[row]|) / 448, 1e-12) and x8[row][col] = e4m3(x / scale), round to
 * nearest even, rows packed (cols bytes apart). The quantisation of lingbot/layers/linear.py:15-26 (FP8Linear):
 * once per output row for a weight, per token for the activations of every call.
 */
int lbw_quant_rows_fp8(const void* x, int x_is_fp32, int64_t rows, int64_t cols, int64_t s_row,
                       uint8_t* x8, float* scale, void* stream);

/*
 * The feed-forward activation and the next linear's activation quantisation in one pass: y = GELU(x) in its tanh
 * form, rounded to bf16 (nn.GELU(approximate='tanh') on bf16 x, the activation between the two linears of
 * lingbot/models/lingbot_world/transformer.py:313-315), then x8 / scale exactly as lbw_quant_rows_fp8 gives them
 * for that bf16 y. x bf16 [rows][cols] (row stride s_row elements, cols a multiple of 16). GELU is evaluated as
 * x / (1 + e^(-2u)) with the hardware exp2 and reciprocal: within a few fp32 ulps of the exact value, so y differs
 * from the correctly rounded bf16 GELU only for values within that distance of a bf16 rounding boundary. Replaces
 * the GELU + activation quantisation of lingbot/layers/linear.py:15-26 that a compiled reference fuses.
 */
int lbw_quant_rows_fp8_gelu(const uint16_t* x, int64_t rows, int64_t cols, int64_t s_row, uint8_t* x8,
                            float* scale, void* stream);

/*
 * MXFP8 quantisation of x [rows][cols] (bf16, or fp32 when x_is_fp32; row stride s_row; cols a multiple of 32):
 * per 32 consecutive values, scale = 2^e, e = ceil(log2(max(amax, 2^-126) / 448)) (exact, floored at -127),
 * x8 = e4m3(x / scale) and scale_e8m0 = e + 127, rows packed (x8 [rows_pad][cols], scale_e8m0
 * [rows_pad][cols / 32]); rows rows .. rows_pad - 1 are written as zeros with scale byte 127. The quantisation of
 * lingbot/layers/linear.py:42-50 (MXFP8Linear), for a GEMM whose row count is padded to its tile.
 */
int lbw_quant_mx_fp8(const void* x, int x_is_fp32, int64_t rows, int64_t rows_pad, int64_t cols, int64_t s_row,
                     uint8_t* x8, uint8_t* scale_e8m0, void* stream);

/*
 * Quantized attention of Q (from lbw_quant_q) over the chunks seg_slot[0..n_seg) of one layer's cache
 * (pointers already offset to that layer): chunk c is read over tokens [first, first + seg_len[c]) of its slot,
 * first = seg_first[c] (seg_first null: every chunk from token 0), 1 <= seg_len[c] <= cap - first. The keys of a
 * chunk's first and last 64-token blocks outside that range are masked, so a window may start and end anywhere
 * in a chunk (the token window of lingbot/layers/kv_cache.py:23-81). Writes bf16
 * out [batch][lq][heads][128] with strides o_s_batch, o_s_tok, o_s_head. S = q8 . k8 in int32 on the
 * int8 MFMA, online softmax in the exp2 domain, P in e4m3 on the fp8 MFMA with V's E8M0 block scales applied by
 * the MFMA itself (when v8lo is not null, a second product of the residual plane with bf6(P / 16) on the 6-bit
 * MFMA, at twice the fp8 rate, scaled back by 2^4), fp32
 * accumulation, 1 / row sum applied at the end (the row sum adds the e4m3 P the products apply, formed on the
 * matrix core; the reference sums the unrounded P). Replaces the fused Sage kernel call (lingbot/layers/sage_preq.py:
 * 126-127; experiments/modules/sage_kvq.py:107-110). seg_slot / seg_len are host arrays. `workspace` holds
 * lbw_attn_workspace_bytes() bytes (16-byte aligned); two kernels run: the attention over a persistent grid
 * and a merge of the query tiles whose keys were split between workgroups.
 */
int lbw_attn_fwd(const int8_t* q8, const float* q_scale, const float* bias,
                 int64_t batch, int64_t lq, int64_t heads,
                 const int8_t* k8, const float* k_scale, const uint8_t* v8, const uint8_t* v8lo,
                 const uint8_t* v_scale, int64_t slots, int64_t cap, int n_seg, const int32_t* seg_slot,
                 const int32_t* seg_len, const int32_t* seg_first,
                 uint16_t* out, int64_t o_s_batch, int64_t o_s_tok, int64_t o_s_head,
                 float sm_scale, void* workspace, void* stream);

/* Bytes of scratch lbw_attn_fwd needs on the current device (partial results of query tiles whose key range
 * is split between workgroups); independent of the problem size. Calls that share a workspace must not overlap
 * (calls on different streams need workspaces of their own). */
int64_t lbw_attn_workspace_bytes(void);

/*
 * lbw_attn_fwd without the workspace argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). Has no counterpart in the reference.
 * Same arguments (less `workspace`), kernels and results as lbw_attn_fwd; the split-tile partials go to a fixed
 * array inside the library, one per GPU, of lbw_attn_noalloc_scratch_bytes() = 68,157,440 bytes (the workspace
 * of a device with up to 256 CUs; LBW_E_SCRATCH on a larger one), held until the process ends. Allocates, frees
 * and synchronises nothing. The first call on a device looks up that device's array (hipGetSymbolAddress): make
 * it outside graph capture. Every call on one GPU shares its array, so calls that overlap on one GPU (on other
 * streams or host threads) race on it.
 */
int lbw_attn_fwd_noalloc(const int8_t* q8, const float* q_scale, const float* bias,
                         int64_t batch, int64_t lq, int64_t heads,
                         const int8_t* k8, const float* k_scale, const uint8_t* v8, const uint8_t* v8lo,
                         const uint8_t* v_scale, int64_t slots, int64_t cap, int n_seg, const int32_t* seg_slot,
                         const int32_t* seg_len, const int32_t* seg_first,
                         uint16_t* out, int64_t o_s_batch, int64_t o_s_tok, int64_t o_s_head,
                         float sm_scale, void* stream);

/* Size of lbw_attn_fwd_noalloc's per-GPU scratch array, in bytes. */
int64_t lbw_attn_noalloc_scratch_bytes(void);

/* Persistent workgroups per XCD that lbw_attn_fwd launches on the current device (one per CU). Query tiles
 * are dealt to XCDs in 8 contiguous ranges and, within one, whole tiles go round-robin to these workgroups
 * while each gets one; the remaining tiles' key blocks are cut into equal contiguous pieces, one per
 * workgroup. Exposed so a checker can reproduce the pieces (each piece rounds P against its own running max). */
int lbw_attn_workgroups_per_xcd(void);

/*
 * Debug: lbw_attn_fwd (same arguments, same results in `out`) run by a checking build of the attention kernel
 * that also writes, for every key block it processes, the raw words of its QK^T accumulator: the int8 MFMA's
 * int32 sums started from S_MAGIC = 0x3E22F983 (the bits of 1 / (2 pi)), as the attention's softmax reads them,
 * before any key mask. logits is int32 [BH][Lp][nb * 64] (Lp = lq rounded up to 256; nb = the sum over chunks of
 * ceil((seg_first[c] % 64 + seg_len[c]) / 64), their blocks in call order): element [bh][i][64 j + t] is
 * S_MAGIC + sum_d q8[bh][i][d] * k8[slot][bh][64 b + t][d] for key t of the slot block b that is block j. The
 * same stages, direct-to-LDS loads, XOR swizzle, fragment reads and accumulator start as lbw_attn_fwd, so the
 * int32 logits the attention uses can be checked bit for bit; read as a float, word w is exactly
 * 1/(2 pi) + (w - S_MAGIC) * 2^-26. Has no reference counterpart.
 */
int lbw_qk_logits_i32(const int8_t* q8, const float* q_scale, const float* bias,
                      int64_t batch, int64_t lq, int64_t heads,
                      const int8_t* k8, const float* k_scale, const uint8_t* v8, const uint8_t* v8lo,
                      const uint8_t* v_scale, int64_t slots, int64_t cap, int n_seg, const int32_t* seg_slot,
                      const int32_t* seg_len, const int32_t* seg_first,
                      uint16_t* out, int64_t o_s_batch, int64_t o_s_tok, int64_t o_s_head,
                      float sm_scale, int32_t* logits, void* workspace, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LBW_ATTN_H */
