// Self-attention prologue of the causal DiT (gfx950): RMSNorm and the 3-axis rotary embedding of the q / k
// projections, fused with the quantisation that consumes them.
//
//   norm_rope_q_kernel:  q projection -> RMSNorm (times its weight) -> rope -> int8 Q per 32-row group with its
//                        scale, the per-chunk logit bias q . km_c, and (optionally) the roped bf16 Q.
//   norm_rope_k_kernel:  k projection -> RMSNorm -> rope -> the roped bf16 K, plus, per 32-token half of each
//                        64-token block, the fp32 column sums of the roped K: the partials the re-quant's own
//                        statistics pass would write, in its order, so its finaliser and quantiser finish the job
//                        (the quantiser reads V and quantises it with K).
//
// A workgroup has one wave per head and takes 32 token rows. Lane (rq, g) = (lane >> 4, lane & 15)
// of wave h holds channels 8 g .. 8 g + 7 of head h in rows 4 (rq + 4 s) + j, s = 0, 1, j = 0..3 (four
// consecutive rows per (lane, s): the statistics pass's summation unit), read as 16-byte loads that cover 4 rows
// x 256 contiguous bytes per instruction.
//
// Row arithmetic (fixed so the CPU restatement reproduces it bit for bit):
//   sum of squares, fp64: per lane a = x0^2 + .. + x7^2 left to right; pairwise over the 16 lanes of the head
//   (xor 1, 2, 4, 8); the heads left to right through LDS. r = fp32(1 / sqrt(fp32(total / C) + eps)).
//   y = bf16(x * r), n = bf16(y * weight); rope in fp64 (products and sums rounded one at a time), then
//   fp64 -> fp32 -> bf16.
#include "lbw_common.h"

#pragma clang fp contract(off)

namespace lbw {

constexpr int RP = D / 2;                 // rotary pairs per head
constexpr int RS0 = RP - 2 * (RP / 3);    // frame pairs (22)
constexpr int RS1 = RS0 + RP / 3;         // the height pairs end here (43); the width pairs follow
constexpr int PR = 32;                    // token rows per pass
constexpr int PRO_MAX_HEADS = 16;         // one wave per head: at most 1024 threads

struct ProArgs {
  int64_t len, heads, bh;
  int64_t x_sb, x_st;          // projection strides (elements): batch, token; its heads * 128 channels contiguous
  int64_t o_sb, o_st, o_sh;    // roped output strides
  int64_t frame_tokens, gw, start_frame;
  int64_t lp, nb;              // Q rows padded to the attention tile (Q); 64-token blocks of the chunk (K)
  float eps;
  int n_seg;
  int seg_slot[LBW_MAX_SEGMENTS];
};

// (cos, sin) of rows row0 .. row0 + 31 into LDS, [row][pair]; rows past len get (1, 0).
__device__ __forceinline__ void stage_rope(double2* s_cs, const double2* __restrict__ tab, const ProArgs& a,
                                           int64_t row0) {
  for (int i = threadIdx.x; i < PR * RP; i += blockDim.x) {
    const int r = i / RP, j = i % RP;
    const int64_t t = row0 + r;
    double2 cs = make_double2(1.0, 0.0);
    if (t < a.len) {   // 32-bit index arithmetic: the host bounds len and the table below 2^31
      const uint32_t tt = (uint32_t)t, ft = (uint32_t)a.frame_tokens, gw = (uint32_t)a.gw;
      const uint32_t f = tt / ft, rem = tt - f * ft;
      const uint32_t row = j < RS0 ? (uint32_t)a.start_frame + f : (j < RS1 ? rem / gw : rem % gw);
      cs = tab[row * RP + j];
    }
    s_cs[i] = cs;
  }
}

// The chunk means of the workgroup's heads (batch b) into LDS, [chunk][head][channel]: loaded with the rows and
// the rope table, so the logit bias at the end waits for no global load.
__device__ __forceinline__ void stage_means(float4* s_km, const float* __restrict__ km, const ProArgs& a, int64_t b) {
  const int per_chunk = (int)a.heads * (D / 4);
  for (int i = threadIdx.x; i < a.n_seg * per_chunk; i += blockDim.x) {
    const int c = i / per_chunk, r = i - c * per_chunk, hh = r / (D / 4), u = r - hh * (D / 4);
    s_km[(c * PRO_MAX_HEADS + hh) * (D / 4) + u] =
        *(const float4*)(km + ((int64_t)a.seg_slot[c] * a.bh + b * a.heads + hh) * D + 4 * u);
  }
}

// Two bf16 (low half first) <-> two fp32. The rounding is v_cvt_pk_bf16_f32 (round to nearest even, the same
// bits as the integer rounding of the other kernels for every finite value), one instruction for two values.
typedef __bf16 pbf2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t bf_pair(float lo, float hi) {
  const pbf2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// The wave's rows of one projection (src already offset to the batch), kept as packed bf16: x[s][j][q] = channels
// 8 g + 2 q, 8 g + 2 q + 1 of row 4 (rq + 4 s) + j; rows past len are 0. Issued before the rope table is staged,
// so the two sets of loads are in flight together. norm_rope_rows below needs s_cs staged; its barriers order
// the staging before the reads.
__device__ __forceinline__ void load_rows(uint32_t (&x)[2][4][4], const uint16_t* __restrict__ src,
                                          const ProArgs& a, int64_t row0) {
  const int lane = threadIdx.x & 63, h = threadIdx.x >> 6, rq = lane >> 4, g = lane & 15;
  const uint16_t* p = src + h * D + g * 8;
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = row0 + 4 * (rq + 4 * s) + j;
      const v4i v = t < a.len ? *(const v4i*)(p + (uint32_t)t * (uint32_t)a.x_st) : v4i{0, 0, 0, 0};
#pragma unroll
      for (int q = 0; q < 4; ++q) x[s][j][q] = (uint32_t)v[q];
    }
}

// x (from load_rows; rows row0 .. row0 + 31) normalised, weighted and roped in place. Rows past the chunk get
// the scale 0, so they stay exact zeros for any eps (with eps = 0, 1 / sqrt(0 + eps) would make them NaN and
// spoil the group's Q scale and the half block's column sums).
__device__ __forceinline__ void norm_rope_rows(uint32_t (&x)[2][4][4], const uint16_t* __restrict__ w,
                                               const ProArgs& a, int64_t row0, double* s_ss, float* s_r,
                                               const double2* s_cs) {
  const int lane = threadIdx.x & 63, h = threadIdx.x >> 6, rq = lane >> 4, g = lane & 15;
  double ss[2][4];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      double acc = 0.0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const double x0 = (double)bf_lo(x[s][j][q]), x1 = (double)bf_hi(x[s][j][q]);
        acc = acc + x0 * x0;
        acc = acc + x1 * x1;
      }
      ss[s][j] = acc;
    }
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) ss[s][j] = row16_sum(ss[s][j]);
  if (g == 0)
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) s_ss[(4 * (rq + 4 * s) + j) * PRO_MAX_HEADS + h] = ss[s][j];
  __syncthreads();
  if (threadIdx.x < PR) {   // one thread per row: the heads' partials in order, and the row's scale
    double tot = 0.0;
    for (int hh = 0; hh < a.heads; ++hh) tot = tot + s_ss[threadIdx.x * PRO_MAX_HEADS + hh];
    const float ms = (float)(tot / (double)(a.heads * D));
    s_r[threadIdx.x] = row0 + threadIdx.x < a.len ? (float)(1.0 / sqrt((double)(ms + a.eps))) : 0.f;
  }
  __syncthreads();
  const v4i wv = *(const v4i*)(w + h * D + g * 8);
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 4 * (rq + 4 * s) + j;
      const float r = s_r[row];
      const double2* cs = s_cs + row * RP + g * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t u = x[s][j][q], wq = (uint32_t)wv[q];
        const uint32_t y = bf_pair(bf_lo(u) * r, bf_hi(u) * r);                     // bf16(x r)
        const uint32_t nn = bf_pair(bf_lo(y) * bf_lo(wq), bf_hi(y) * bf_hi(wq));    // bf16(y w)
        const float n0 = bf_lo(nn), n1 = bf_hi(nn);
        const double2 c = cs[q];
        const double re = (double)n0 * c.x - (double)n1 * c.y;
        const double im = (double)n0 * c.y + (double)n1 * c.x;
        x[s][j][q] = bf_pair((float)re, (float)im);
      }
      // one row at a time: hoisting every row's 16 table reads ahead of the arithmetic would hold 128 registers
      __builtin_amdgcn_sched_barrier(0);
    }
}

// Workgroup (32-row group, batch): one wave per head. MAXT: 768 for up to 12 heads (168 registers a lane), else
// 1024 (128 registers; spills).
template <int MAXT>
__global__ __launch_bounds__(MAXT) void norm_rope_q_kernel(const uint16_t* __restrict__ q,
                                                           const uint16_t* __restrict__ w,
                                                           const double2* __restrict__ tab, ProArgs a,
                                                           int8_t* __restrict__ q8, float* __restrict__ q_scale,
                                                           const float* __restrict__ km, float* __restrict__ bias,
                                                           uint16_t* __restrict__ q_out) {
  __shared__ double2 s_cs[PR * RP];
  __shared__ double s_ss[PR * PRO_MAX_HEADS];
  __shared__ float s_r[PR];
  __shared__ float4 s_km[LBW_MAX_SEGMENTS * PRO_MAX_HEADS * (D / 4)];
  const int grp = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, h = threadIdx.x >> 6, rq = lane >> 4, g = lane & 15;
  const int64_t row0 = (int64_t)grp * PR;
  const int64_t bh = (int64_t)b * a.heads + h;
  uint32_t x[2][4][4];
  load_rows(x, q + b * a.x_sb, a, row0);
  stage_rope(s_cs, tab, a, row0);
  if (a.n_seg > 1) stage_means(s_km, km, a, b);   // norm_rope_rows' barriers order the staging before the reads
  norm_rope_rows(x, w, a, row0, s_ss, s_r, s_cs);
  float amax = 0.f;
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) amax = fmaxf(amax, fmaxf(fabsf(bf_lo(x[s][j][c])), fabsf(bf_hi(x[s][j][c]))));
  amax = fmaxf(wave_max(amax), AMAX_FLOOR);
  const float recip = __fdiv_rn(127.f, amax);
  if (lane == 0) q_scale[bh * (a.lp / QG) + grp] = __fdiv_rn(amax, 127.f);
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = row0 + 4 * (rq + 4 * s) + j;
      uint32_t wd[2];
#pragma unroll
      for (int hw = 0; hw < 2; ++hw) {
        const uint32_t u0 = x[s][j][2 * hw], u1 = x[s][j][2 * hw + 1];
        wd[hw] = ((uint32_t)quant_i8(bf_lo(u0), recip) & 0xFFu) | (((uint32_t)quant_i8(bf_hi(u0), recip) & 0xFFu) << 8) |
                 (((uint32_t)quant_i8(bf_lo(u1), recip) & 0xFFu) << 16) |
                 (((uint32_t)quant_i8(bf_hi(u1), recip) & 0xFFu) << 24);
      }
      *(uint2*)(q8 + (bh * a.lp + t) * D + g * 8) = make_uint2(wd[0], wd[1]);
      if (q_out && t < a.len)
        *(v4i*)(q_out + b * a.o_sb + h * a.o_sh + g * 8 + (uint32_t)t * (uint32_t)a.o_st) =
            v4i{(int)x[s][j][0], (int)x[s][j][1], (int)x[s][j][2], (int)x[s][j][3]};
    }
  for (int c = 0; a.n_seg > 1 && c < a.n_seg; ++c) {
    const float4* m = s_km + (c * PRO_MAX_HEADS + h) * (D / 4) + 2 * g;
    const float4 m0 = m[0], m1 = m[1];
    const float mv[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc = fmaf(bf_lo(x[s][j][q]), mv[2 * q], acc);
          acc = fmaf(bf_hi(x[s][j][q]), mv[2 * q + 1], acc);
        }
        acc = row16_sum(acc);
        if (g == 0) bias[((int64_t)c * a.bh + bh) * a.lp + row0 + 4 * (rq + 4 * s) + j] = acc;
      }
  }
}

// Workgroup (32-token half of a 64-token block, batch): one wave per head. Writes that half's column sums of K.
template <int MAXT>
__global__ __launch_bounds__(MAXT) void norm_rope_k_kernel(const uint16_t* __restrict__ k,
                                                           const uint16_t* __restrict__ w,
                                                           const double2* __restrict__ tab, ProArgs a,
                                                           uint16_t* __restrict__ k_out,
                                                           float* __restrict__ part_sum) {
  __shared__ double2 s_cs[PR * RP];
  __shared__ double s_ss[PR * PRO_MAX_HEADS];
  __shared__ float s_r[PR];
  __shared__ float4 s_S[MAXT / 64][8][D / 4];   // per head: the 4-row column sums, [row group][channel]
  const int half = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, h = threadIdx.x >> 6, rq = lane >> 4, g = lane & 15;
  const int64_t row0 = (int64_t)half * PR;
  uint32_t x[2][4][4];
  load_rows(x, k + b * a.x_sb, a, row0);
  stage_rope(s_cs, tab, a, row0);
  // partials [batch * heads][blocks][2 halves][128]: half index = blockIdx.x
  const int64_t o = (((int64_t)b * a.heads + h) * a.nb * 2 + half) * D + g * 8;
  norm_rope_rows(x, w, a, row0, s_ss, s_r, s_cs);
  uint16_t* ko = k_out + b * a.o_sb + h * a.o_sh + g * 8;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    float S[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float t0 = 0.f, t1 = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        t0 = t0 + bf_lo(x[s][j][q]);
        t1 = t1 + bf_hi(x[s][j][q]);
      }
      S[2 * q] = t0;
      S[2 * q + 1] = t1;
    }
    s_S[h][rq + 4 * s][2 * g] = make_float4(S[0], S[1], S[2], S[3]);
    s_S[h][rq + 4 * s][2 * g + 1] = make_float4(S[4], S[5], S[6], S[7]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = row0 + 4 * (rq + 4 * s) + j;
      if (t < a.len)
        *(v4i*)(ko + (uint32_t)t * (uint32_t)a.o_st) =
            v4i{(int)x[s][j][0], (int)x[s][j][1], (int)x[s][j][2], (int)x[s][j][3]};
    }
  }
  __syncthreads();
  // the half's column sum over its 4-row sums in row order; lane (rq, g) takes channels 8 g + 2 rq, + 1
  const float* col = (const float*)&s_S[h][0][0] + 8 * g + 2 * rq;
  float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    acc0 = acc0 + col[r * D];
    acc1 = acc1 + col[r * D + 1];
  }
  part_sum[o + 2 * rq] = acc0;
  part_sum[o + 2 * rq + 1] = acc1;
}

// Shared argument checks of the two entry points; fills the rope / norm part of `a`.
static int prologue_args(ProArgs& a, int64_t batch, int64_t len, int64_t heads, const uint16_t* x,
                         int64_t s_batch, int64_t s_tok, const uint16_t* weight, float eps, const double* rope,
                         int64_t rope_rows, int64_t grid_h, int64_t grid_w, int64_t start_frame) {
  if (!x || !weight || !rope) return LBW_E_NULL;
  if (batch <= 0 || len <= 0 || heads <= 0 || heads > PRO_MAX_HEADS || batch > 65535) return LBW_E_SHAPE;
  if (grid_h <= 0 || grid_w <= 0 || start_frame < 0 || rope_rows <= 0) return LBW_E_SHAPE;
  const int64_t frame_tokens = grid_h * grid_w;
  if (grid_h > rope_rows || grid_w > rope_rows || start_frame + (len - 1) / frame_tokens >= rope_rows)
    return LBW_E_SHAPE;   // every rotation row the chunk needs is in the table
  if (len >= ((int64_t)1 << 30) || rope_rows * RP >= ((int64_t)1 << 31)) return LBW_E_SHAPE;
  if (!(eps >= 0.f) || eps > 1.f) return LBW_E_SHAPE;
  if (s_batch % 8 || s_tok % 8) return LBW_E_ALIGN;
  if (s_tok < 0 || (len + KB) * s_tok >= ((int64_t)1 << 31)) return LBW_E_SHAPE;   // 32-bit row offsets
  if (((uintptr_t)x | (uintptr_t)weight | (uintptr_t)rope) & 15) return LBW_E_ALIGN;
  a.len = len; a.heads = heads; a.bh = batch * heads;
  a.x_sb = s_batch; a.x_st = s_tok;
  a.o_sb = a.o_st = a.o_sh = 0;
  a.frame_tokens = frame_tokens; a.gw = grid_w; a.start_frame = start_frame;
  a.lp = 0; a.nb = 0;
  a.eps = eps;
  a.n_seg = 0;
  for (int c = 0; c < LBW_MAX_SEGMENTS; ++c) a.seg_slot[c] = 0;
  return LBW_OK;
}

}  // namespace lbw

using namespace lbw;

extern "C" int lbw_norm_rope_quant_q(const uint16_t* q, int64_t batch, int64_t lq, int64_t heads,
                                     int64_t s_batch, int64_t s_tok, const uint16_t* norm_weight, float eps,
                                     const double* rope, int64_t rope_rows, int64_t grid_h, int64_t grid_w,
                                     int64_t start_frame, int8_t* q8, float* q_scale, const float* km,
                                     int64_t slots, int n_seg, const int32_t* seg_slot, float* bias,
                                     uint16_t* q_out, int64_t o_s_batch, int64_t o_s_tok, int64_t o_s_head,
                                     void* stream) {
  ProArgs a;
  if (const int st = prologue_args(a, batch, lq, heads, q, s_batch, s_tok, norm_weight, eps, rope, rope_rows,
                                   grid_h, grid_w, start_frame))
    return st;
  if (!q8 || !q_scale) return LBW_E_NULL;
  if (n_seg < 0 || n_seg > LBW_MAX_SEGMENTS) return LBW_E_SEGMENTS;
  if (((uintptr_t)q8 | (uintptr_t)q_scale) & 7) return LBW_E_ALIGN;
  if (q_out) {
    if (o_s_batch % 8 || o_s_tok % 8 || o_s_head % 8 || ((uintptr_t)q_out & 15)) return LBW_E_ALIGN;
    if (o_s_tok < 0 || (lq + KB) * o_s_tok >= ((int64_t)1 << 31)) return LBW_E_SHAPE;
    a.o_sb = o_s_batch; a.o_st = o_s_tok; a.o_sh = o_s_head;
  }
  a.lp = (lq + QT - 1) / QT * QT;
  if (a.lp / PR > 0x7fffffff) return LBW_E_SHAPE;
  a.n_seg = n_seg;
  if (n_seg > 1) {
    if (!km || !bias || !seg_slot) return LBW_E_NULL;
    if ((uintptr_t)km & 15) return LBW_E_ALIGN;   // read as float4
    for (int c = 0; c < n_seg; ++c) {
      if (seg_slot[c] < 0 || seg_slot[c] >= slots) return LBW_E_SEGMENTS;
      a.seg_slot[c] = seg_slot[c];
    }
  }
  if (const int dv = check_device()) return dv;
  const dim3 grid((unsigned)(a.lp / PR), (unsigned)batch), block(64 * (unsigned)heads);
  if (heads <= 12)
    hipLaunchKernelGGL(norm_rope_q_kernel<768>, grid, block, 0, (hipStream_t)stream, q, norm_weight,
                       (const double2*)rope, a, q8, q_scale, km, bias, q_out);
  else
    hipLaunchKernelGGL(norm_rope_q_kernel<1024>, grid, block, 0, (hipStream_t)stream, q, norm_weight,
                       (const double2*)rope, a, q8, q_scale, km, bias, q_out);
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return LBW_OK;
}

extern "C" int lbw_norm_rope_kv_requant(const uint16_t* k, const uint16_t* v, int64_t batch, int64_t len,
                                        int64_t heads, int64_t k_s_batch, int64_t k_s_tok, int64_t v_s_batch,
                                        int64_t v_s_tok, int64_t v_s_head, const uint16_t* norm_weight, float eps,
                                        const double* rope, int64_t rope_rows, int64_t grid_h, int64_t grid_w,
                                        int64_t start_frame, uint16_t* k_out, int64_t o_s_batch,
                                        int64_t o_s_tok, int64_t o_s_head, int8_t* k8, float* k_scale,
                                        float* km, uint8_t* v8, uint8_t* v8lo, uint8_t* v_scale, int64_t slots,
                                        int64_t cap, int64_t slot, void* workspace, void* stream) {
  ProArgs a;
  if (const int st = prologue_args(a, batch, len, heads, k, k_s_batch, k_s_tok, norm_weight, eps, rope, rope_rows,
                                   grid_h, grid_w, start_frame))
    return st;
  if (!v || !k_out || !workspace) return LBW_E_NULL;
  if (v_s_batch % 8 || v_s_tok % 8 || v_s_head % 8 || o_s_batch % 8 || o_s_tok % 8 || o_s_head % 8)
    return LBW_E_ALIGN;
  if (((uintptr_t)v | (uintptr_t)k_out | (uintptr_t)workspace) & 15) return LBW_E_ALIGN;
  if (v_s_tok < 0 || o_s_tok < 0 || (len + KB) * v_s_tok >= ((int64_t)1 << 31) ||
      (len + KB) * o_s_tok >= ((int64_t)1 << 31))
    return LBW_E_SHAPE;
  a.o_sb = o_s_batch; a.o_st = o_s_tok; a.o_sh = o_s_head;
  a.nb = (len + KB - 1) / KB;
  if (a.nb > 0x7fffffff) return LBW_E_SHAPE;
  // the re-quant's own checks (shape, slot, ring pointers) run before anything is launched
  if (const int st = kv_requant_check(1, batch, len, heads, k8, k_scale, km, v8, v8lo, v_scale, slots, cap, slot))
    return st;
  if (const int dv = check_device()) return dv;
  float* part_sum = (float*)workspace;
  const dim3 grid((unsigned)(2 * a.nb), (unsigned)batch), block(64 * (unsigned)heads);
  if (heads <= 12)
    hipLaunchKernelGGL(norm_rope_k_kernel<768>, grid, block, 0, (hipStream_t)stream, k, norm_weight,
                       (const double2*)rope, a, k_out, part_sum);
  else
    hipLaunchKernelGGL(norm_rope_k_kernel<1024>, grid, block, 0, (hipStream_t)stream, k, norm_weight,
                       (const double2*)rope, a, k_out, part_sum);
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return kv_requant_launch(false, false, k_out, v, 1, batch, len, heads, 0, o_s_batch, o_s_tok, o_s_head, 0, v_s_batch,
                           v_s_tok, v_s_head, k8, k_scale, km, v8, v8lo, v_scale, slots, cap, slot, workspace,
                           stream);
}
