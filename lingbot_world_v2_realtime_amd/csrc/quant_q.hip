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

// One wave per (32-row group, batch*head): lane = 2 * row + half, each lane owns 64 channels of one row.
__global__ __launch_bounds__(64) void quant_q_kernel(const uint16_t* __restrict__ q, QArgs a,
                                                     int8_t* __restrict__ q8, float* __restrict__ q_scale,
                                                     const float* __restrict__ km, float* __restrict__ bias) {
  __shared__ __align__(16) float s_km[LBW_MAX_SEGMENTS][D];   // the chunks' K means for the logit bias
  const int grp = blockIdx.x, bh = blockIdx.y;
  const int lane = threadIdx.x, r = lane >> 1, half = lane & 1;
  const int64_t row = (int64_t)grp * QG + r;
  const int64_t b = bh / a.heads, h = bh % a.heads;
  const bool ok = row < a.lq;
  const uint16_t* qp = q + b * a.sb + row * a.st + h * a.sh + half * 64;
  // the K means go through LDS once per row group: read from global memory inside the dot products below,
  // every lane would wait on 16 dependent loads per chunk
  if (a.n_seg > 1) {
    for (int i = lane; i < a.n_seg * (D / 4); i += 64) {
      const int c = i / (D / 4), k4 = i % (D / 4);
      *(float4*)&s_km[c][4 * k4] = *(const float4*)(km + ((int64_t)a.seg_slot[c] * a.bh + bh) * D + 4 * k4);
    }
  }
  float x[64];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const v4i w = ok ? *(const v4i*)(qp + 8 * i) : v4i{0, 0, 0, 0};
    unpack8(w, x + 8 * i);
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 64; ++i) amax = fmaxf(amax, fabsf(x[i]));
  amax = fmaxf(wave_max(amax), AMAX_FLOOR);
  const float recip = __fdiv_rn(127.f, amax);
  if (lane == 0) q_scale[(int64_t)bh * (a.lp / QG) + grp] = __fdiv_rn(amax, 127.f);
  int8_t* out = q8 + ((int64_t)bh * a.lp + row) * D + half * 64;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t u = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) u |= ((uint32_t)quant_i8(x[16 * i + 4 * j + c], recip) & 0xFFu) << (8 * c);
      w[j] = (int)u;
    }
    *(v4i*)(out + 16 * i) = v4i{w[0], w[1], w[2], w[3]};
  }
  if (a.n_seg > 1) {
    __syncthreads();   // s_km is filled (one wave: orders the LDS writes before the reads)
    for (int c = 0; c < a.n_seg; ++c) {
      const float* m = &s_km[c][half * 64];
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 64; ++i) acc = fmaf(x[i], m[i], acc);
      acc += __shfl_xor(acc, 1);
      if (half == 0) bias[((int64_t)c * a.bh + bh) * a.lp + row] = acc;
    }
  }
}

}  // namespace lbw

using namespace lbw;

extern "C" int lbw_quant_q(const uint16_t* q, int64_t batch, int64_t lq, int64_t heads, int64_t s_batch,
                           int64_t s_tok, int64_t s_head, int8_t* q8, float* q_scale, const float* km,
                           int64_t slots, int n_seg, const int32_t* seg_slot, float* bias, void* stream) {
  if (!q || !q8 || !q_scale) return LBW_E_NULL;
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
  hipLaunchKernelGGL(quant_q_kernel, dim3((unsigned)(a.lp / QG), (unsigned)a.bh), dim3(64), 0,
                     (hipStream_t)stream, q, a, q8, q_scale, km, bias);
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return LBW_OK;
}
