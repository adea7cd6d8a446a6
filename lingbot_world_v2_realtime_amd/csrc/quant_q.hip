// Q -> int8 with one fp32 scale per 32 rows, plus the per-chunk logit bias q . km (gfx950).
#include "lbw_common.h"

namespace lbw {

struct QArgs {
  int64_t lq, lp, heads, bh;
  int64_t sb, st, sh;
  int64_t slots;
  int n_seg;
  int seg_slot[LBW_MAX_SEGMENTS];
};

// One wave per (32-row group, batch*head), four waves (four batch*heads) per workgroup. Lane (rq, g) =
// (lane >> 4, lane & 15) holds channels 8 g .. 8 g + 7 of rows 4 (rq + 4 s) + j, s = 0, 1, j = 0..3, so each
// 16-byte load instruction reads 4 rows x 256 contiguous bytes. The logit bias of a row is its 16 lanes' 8-term
// dot products with the chunk mean, summed pairwise (xor 1, 2, 4, 8).
// F16: q is fp16 (else bf16).
constexpr int QQ_WAVES = 4;
template <bool F16>
__global__ __launch_bounds__(64 * QQ_WAVES) void quant_q_kernel(const uint16_t* __restrict__ q, QArgs a,
                                                               int8_t* __restrict__ q8, float* __restrict__ q_scale,
                                                               const float* __restrict__ km,
                                                               float* __restrict__ bias) {
  const int grp = blockIdx.x;
  const int lane = threadIdx.x & 63, rq = lane >> 4, g = lane & 15;
  const int64_t bh = (int64_t)blockIdx.y * QQ_WAVES + (threadIdx.x >> 6);
  if (bh >= a.bh) return;   // wave-uniform; the kernel has no barrier
  const int64_t b = bh / a.heads, h = bh % a.heads;
  const int64_t row0 = (int64_t)grp * QG;
  const uint16_t* qp = q + b * a.sb + h * a.sh + g * 8;
  uint32_t x[2][4][4];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = row0 + 4 * (rq + 4 * s) + j;
      const v4i v = t < a.lq ? *(const v4i*)(qp + t * a.st) : v4i{0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < 4; ++c) x[s][j][c] = (uint32_t)v[c];
    }
  float amax = 0.f;
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        amax = fmaxf(amax, fmaxf(fabsf(lo16<F16>(x[s][j][c])), fabsf(hi16<F16>(x[s][j][c]))));
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
        wd[hw] = ((uint32_t)quant_i8(lo16<F16>(u0), recip) & 0xFFu) |
                 (((uint32_t)quant_i8(hi16<F16>(u0), recip) & 0xFFu) << 8) |
                 (((uint32_t)quant_i8(lo16<F16>(u1), recip) & 0xFFu) << 16) |
                 (((uint32_t)quant_i8(hi16<F16>(u1), recip) & 0xFFu) << 24);
      }
      *(uint2*)(q8 + (bh * a.lp + t) * D + g * 8) = make_uint2(wd[0], wd[1]);
    }
  for (int c = 0; a.n_seg > 1 && c < a.n_seg; ++c) {
    const float* m = km + ((int64_t)a.seg_slot[c] * a.bh + bh) * D + g * 8;
    const float4 m0 = *(const float4*)m, m1 = *(const float4*)(m + 4);
    const float mv[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc = fmaf(lo16<F16>(x[s][j][e]), mv[2 * e], acc);
          acc = fmaf(hi16<F16>(x[s][j][e]), mv[2 * e + 1], acc);
        }
        acc = row16_sum(acc);
        if (g == 0) bias[((int64_t)c * a.bh + bh) * a.lp + row0 + 4 * (rq + 4 * s) + j] = acc;
      }
  }
}

}  // namespace lbw

using namespace lbw;

extern "C" int lbw_quant_q(const uint16_t* q, int dtype, int64_t batch, int64_t lq, int64_t heads, int64_t s_batch,
                           int64_t s_tok, int64_t s_head, int8_t* q8, float* q_scale, const float* km,
                           int64_t slots, int n_seg, const int32_t* seg_slot, float* bias, void* stream) {
  if (!q || !q8 || !q_scale) return LBW_E_NULL;
  if (dtype != LBW_DTYPE_BF16 && dtype != LBW_DTYPE_FP16) return LBW_E_SHAPE;
  if (batch <= 0 || heads <= 0 || lq <= 0 || batch * heads > 65535) return LBW_E_SHAPE;
  if (n_seg < 0 || n_seg > LBW_MAX_SEGMENTS) return LBW_E_SEGMENTS;
  if (s_batch % 8 || s_tok % 8 || s_head % 8) return LBW_E_ALIGN;
  if (((uintptr_t)q | (uintptr_t)q8) & 15) return LBW_E_ALIGN;
  QArgs a;
  a.lq = lq;
  a.lp = (lq + QT - 1) / QT * QT;
  a.heads = heads;
  a.bh = batch * heads;
  a.sb = s_batch; a.st = s_tok; a.sh = s_head;
  a.slots = slots;
  a.n_seg = n_seg;
  for (int c = 0; c < LBW_MAX_SEGMENTS; ++c) a.seg_slot[c] = 0;
  if (n_seg > 1) {
    if (!km || !bias || !seg_slot) return LBW_E_NULL;
    if ((uintptr_t)km & 15) return LBW_E_ALIGN;   // read as float4
    for (int c = 0; c < n_seg; ++c) {
      if (seg_slot[c] < 0 || seg_slot[c] >= slots) return LBW_E_SEGMENTS;
      a.seg_slot[c] = seg_slot[c];
    }
  }
  if (a.lp / QG > 0x7fffffff) return LBW_E_SHAPE;
  if (const int dv = check_device()) return dv;
  const dim3 grid((unsigned)(a.lp / QG), (unsigned)((a.bh + QQ_WAVES - 1) / QQ_WAVES));
  if (dtype == LBW_DTYPE_FP16)
    hipLaunchKernelGGL(quant_q_kernel<true>, grid, dim3(64 * QQ_WAVES), 0, (hipStream_t)stream, q, a, q8, q_scale, km,
                       bias);
  else
    hipLaunchKernelGGL(quant_q_kernel<false>, grid, dim3(64 * QQ_WAVES), 0, (hipStream_t)stream, q, a, q8, q_scale,
                       km, bias);
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return LBW_OK;
}
