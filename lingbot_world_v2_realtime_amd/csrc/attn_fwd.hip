// Quantized attention forward for gfx950: int8 QK^T on v_mfma_i32_32x32x32_i8, online softmax in the exp2
// domain, e4m3 P times e4m3 V on v_mfma_f32_32x32x64_f8f6f4, fp32 accumulation.
//
// Work decomposition: one workgroup of 4 waves per (128-query tile, batch*head); wave w owns queries
// 32w .. 32w+31 of the tile. Each wave computes S^T = K Q^T (keys on the MFMA M axis, queries on N), so a
// lane holds one query and 16 keys of each 32x32 S tile: the row max and row sum are in-lane plus one
// exchange with lane ^ 32, and the S tile's register layout is directly the B operand (P^T) of the PV
// product O^T = V^T P^T once the fp8 V block stores its keys in the matching position order.
//
// K / V tiles of 64 keys (8 KB each) stream through LDS, double buffered; the next tile's global loads are
// in flight while the current one is computed. The int32 accumulator starts at the bits of 1.5 * 2^23, so
// its result reads directly as the float 12582912 + S (|S| <= 2^21) and the int -> float conversion is free.
#include "lbw_common.h"

namespace lbw {

struct SegTable {
  int n;
  int slot[LBW_MAX_SEGMENTS];
  int len[LBW_MAX_SEGMENTS];
};

struct AttnArgs {
  int64_t lq, lp, bh, heads, cap, nbc;
  int64_t o_sb, o_st, o_sh;
  float sl2;   // sm_scale * log2(e)
  SegTable seg;
};

constexpr int TILE_BYTES = KB * D;   // 8 KB: one 64-key K tile, or one 64-key fp8 V block

// LDS byte offset of 16-byte chunk `ch` (0..7) of K row `row` (0..63): rows of 128 bytes, chunk index
// xor-swizzled with the row so the 32 rows an MFMA A-operand read touches spread over the banks.
__device__ __forceinline__ int k_lds_off(int row, int ch) { return row * 128 + ((ch ^ (row & 7)) << 4); }
// LDS byte offset of 16-byte chunk `ch` (0..3) of V row (channel) `row` (0..127): rows of 64 bytes.
__device__ __forceinline__ int v_lds_off(int row, int ch) { return TILE_BYTES + row * 64 + ((ch ^ ((row >> 1) & 3)) << 4); }

// S^T tile pair for 64 keys x 32 queries of this wave: acc[mt] covers keys 32 mt .. 32 mt + 31.
__device__ __forceinline__ void qk_tile(const uint8_t* sk, const v4i* qf, int lq, int g, v16i* acc, int init) {
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    v16i c;
#pragma unroll
    for (int i = 0; i < 16; ++i) c[i] = init;
    const int row = 32 * mt + lq;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const v4i kf = *(const v4i*)(sk + k_lds_off(row, 4 * g + kk));
      c = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf[kk], c, 0, 0, 0);
    }
    acc[mt] = c;
  }
}

__global__ __launch_bounds__(256) void attn_fwd_kernel(const int8_t* __restrict__ q8,
                                                       const float* __restrict__ q_scale,
                                                       const float* __restrict__ bias,
                                                       const int8_t* __restrict__ k8,
                                                       const float* __restrict__ k_scale,
                                                       const uint8_t* __restrict__ v8,
                                                       const float* __restrict__ v_scale,
                                                       uint16_t* __restrict__ out, AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][2 * TILE_BYTES];
  const int tile = blockIdx.x, bh = blockIdx.y;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63, lq = lane & 31, g = lane >> 5;
  const int64_t q0 = (int64_t)tile * QT + w * 32;

  // Q^T B-operand fragments: lane (query lq, half g) holds channels 64 g .. 64 g + 63.
  v4i qf[4];
  {
    const int8_t* qrow = q8 + ((int64_t)bh * a.lp + q0 + lq) * D + 64 * g;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[kk] = *(const v4i*)(qrow + 16 * kk);
  }
  const float qs = q_scale[(int64_t)bh * (a.lp / QG) + (q0 >> 5)];

  v16f o[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[mt][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  v4i pk0, pk1, pv0, pv1;
  auto gload = [&](int c, int blk) {
    const int64_t sbh = (int64_t)a.seg.slot[c] * a.bh + bh;
    const int8_t* kp = k8 + (sbh * a.cap + (int64_t)blk * KB) * D;
    const uint8_t* vp = v8 + (sbh * a.nbc + blk) * TILE_BYTES;
    pk0 = *(const v4i*)(kp + t * 16);
    pk1 = *(const v4i*)(kp + 4096 + t * 16);
    pv0 = *(const v4i*)(vp + t * 16);
    pv1 = *(const v4i*)(vp + 4096 + t * 16);
  };
  auto lstore = [&](uint8_t* s) {
    {
      const int id0 = t, id1 = t + 256;
      *(v4i*)(s + k_lds_off(id0 >> 3, id0 & 7)) = pk0;
      *(v4i*)(s + k_lds_off(id1 >> 3, id1 & 7)) = pk1;
      *(v4i*)(s + v_lds_off(id0 >> 2, id0 & 3)) = pv0;
      *(v4i*)(s + v_lds_off(id1 >> 2, id1 & 3)) = pv1;
    }
  };

  int c = 0, blk = 0, buf = 0;
  const bool multi = a.seg.n > 1;
  float beta = multi ? bias[(int64_t)bh * a.lp + q0 + lq] * a.sl2 : 0.f;
  gload(0, 0);
  lstore(smem[0]);
  __syncthreads();

  for (;;) {
    int cn = c, bn = blk + 1;
    if (bn * KB >= a.seg.len[c]) { cn = c + 1; bn = 0; }
    const bool more = cn < a.seg.n;
    if (more) gload(cn, bn);

    const uint8_t* sk = smem[buf];
    v16i acc[2];
    qk_tile(sk, qf, lq, g, acc, S_MAGIC);

    const int64_t sbh = (int64_t)a.seg.slot[c] * a.bh + bh;
    const float cb = qs * k_scale[sbh * a.nbc + blk] * a.sl2;
    float f[32];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) f[16 * mt + i] = __int_as_float(acc[mt][i]);
    const int valid = a.seg.len[c] - blk * KB;   // keys of this block that exist (>= 1)
    if (valid < KB) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = 32 * mt + 8 * (i >> 2) + 4 * g + (i & 3);
          if (key >= valid) f[16 * mt + i] = -INFINITY;
        }
    }
    float mx = f[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) mx = fmaxf(mx, f[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_blk = (mx - S_MAGIC_F) * cb + beta;
    const float m_new = fmaxf(m_run, m_blk);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[mt][i] *= alpha;
    const float kc = (beta - m_new + P_OFFSET) - S_MAGIC_F * cb;
    float p[32];
    float ls = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      p[i] = __builtin_amdgcn_exp2f(fmaf(f[i], cb, kc));
      ls += p[i];
    }
    l_run += ls;
    // P^T B operand: byte 16 mt' + 4 i + j of this lane = p[16 mt' + 4 i + j] (keys 32 mt' + 8 i + 4 g + j).
    v8i pb;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      int wd = __builtin_amdgcn_cvt_pk_fp8_f32(p[4 * r], p[4 * r + 1], 0, false);
      wd = __builtin_amdgcn_cvt_pk_fp8_f32(p[4 * r + 2], p[4 * r + 3], wd, true);
      pb[r] = wd;
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int row = 32 * mt + lq;
      const v4i lo = *(const v4i*)(sk + v_lds_off(row, 2 * g));
      const v4i hi = *(const v4i*)(sk + v_lds_off(row, 2 * g + 1));
      const v8i vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      o[mt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pb, o[mt], 0, 0, 0, 0, 0, 0);
    }

    if (more) lstore(smem[buf ^ 1]);
    __syncthreads();
    if (!more) break;
    if (cn != c) {
      // next chunk: its own V scale (rescale the accumulator per channel) and its own logit bias
      const float* vs_old = v_scale + sbh * D;
      const float* vs_new = v_scale + ((int64_t)a.seg.slot[cn] * a.bh + bh) * D;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int ch = 32 * mt + 8 * (i >> 2) + 4 * g + (i & 3);
          o[mt][i] *= vs_old[ch] / vs_new[ch];
        }
      beta = bias[((int64_t)cn * a.bh + bh) * a.lp + q0 + lq] * a.sl2;
    }
    c = cn;
    blk = bn;
    buf ^= 1;
  }

  // epilogue: O = o * v_scale / l, bf16, lane (query lq) writes channels 32 mt + 8 i + 4 g + (0..3)
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv_l = 1.f / l_tot;
  const int64_t qrow = q0 + lq;
  if (qrow < a.lq) {
    const int64_t b = bh / a.heads, h = bh % a.heads;
    uint16_t* op = out + b * a.o_sb + qrow * a.o_st + h * a.o_sh;
    const float* vs = v_scale + ((int64_t)a.seg.slot[c] * a.bh + bh) * D;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ch = 32 * mt + 8 * i + 4 * g;
        uint32_t w0 = f32_to_bf16_bits(o[mt][4 * i] * vs[ch] * inv_l) |
                      ((uint32_t)f32_to_bf16_bits(o[mt][4 * i + 1] * vs[ch + 1] * inv_l) << 16);
        uint32_t w1 = f32_to_bf16_bits(o[mt][4 * i + 2] * vs[ch + 2] * inv_l) |
                      ((uint32_t)f32_to_bf16_bits(o[mt][4 * i + 3] * vs[ch + 3] * inv_l) << 16);
        *(uint2*)(op + ch) = make_uint2(w0, w1);
      }
  }
}

// Debug: S = q8 . k8^T in int32 for one slot, through the same LDS tile layout and MFMA as the attention.
__global__ __launch_bounds__(256) void qk_logits_kernel(const int8_t* __restrict__ q8,
                                                        const int8_t* __restrict__ k8, int64_t lp,
                                                        int64_t cap, int64_t bh_count, int64_t slot,
                                                        int32_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * TILE_BYTES];
  const int tile = blockIdx.x, blk = blockIdx.y, bh = blockIdx.z;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63, lq = lane & 31, g = lane >> 5;
  const int64_t q0 = (int64_t)tile * QT + w * 32;
  v4i qf[4];
  const int8_t* qrow = q8 + ((int64_t)bh * lp + q0 + lq) * D + 64 * g;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) qf[kk] = *(const v4i*)(qrow + 16 * kk);
  const int8_t* kp = k8 + ((slot * bh_count + bh) * cap + (int64_t)blk * KB) * D;
  const int id0 = t, id1 = t + 256;
  *(v4i*)(smem + k_lds_off(id0 >> 3, id0 & 7)) = *(const v4i*)(kp + id0 * 16);
  *(v4i*)(smem + k_lds_off(id1 >> 3, id1 & 7)) = *(const v4i*)(kp + id1 * 16);
  __syncthreads();
  v16i acc[2];
  qk_tile(smem, qf, lq, g, acc, 0);
  int32_t* op = out + ((int64_t)bh * lp + q0 + lq) * cap + (int64_t)blk * KB;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) op[32 * mt + 8 * (i >> 2) + 4 * g + (i & 3)] = acc[mt][i];
}

}  // namespace lbw

using namespace lbw;

extern "C" int lbw_attn_fwd(const int8_t* q8, const float* q_scale, const float* bias, int64_t batch,
                            int64_t lq, int64_t heads, const int8_t* k8, const float* k_scale,
                            const uint8_t* v8, const float* v_scale, int64_t slots, int64_t cap, int n_seg,
                            const int32_t* seg_slot, const int32_t* seg_len, uint16_t* out,
                            int64_t o_s_batch, int64_t o_s_tok, int64_t o_s_head, float sm_scale,
                            void* stream) {
  if (!q8 || !q_scale || !k8 || !k_scale || !v8 || !v_scale || !out || !seg_slot || !seg_len) return LBW_E_NULL;
  if (batch <= 0 || heads <= 0 || lq <= 0 || slots <= 0 || cap <= 0 || cap % KB) return LBW_E_SHAPE;
  if (batch * heads > 65535 || !(sm_scale > 0.f)) return LBW_E_SHAPE;
  if (n_seg < 1 || n_seg > LBW_MAX_SEGMENTS) return LBW_E_SEGMENTS;
  if (n_seg > 1 && !bias) return LBW_E_NULL;
  if (o_s_batch % 4 || o_s_tok % 4 || o_s_head % 4) return LBW_E_ALIGN;
  if (((uintptr_t)q8 | (uintptr_t)k8 | (uintptr_t)v8) & 15 || ((uintptr_t)out & 7)) return LBW_E_ALIGN;
  AttnArgs a;
  a.lq = lq;
  a.lp = (lq + QT - 1) / QT * QT;
  a.bh = batch * heads;
  a.heads = heads;
  a.cap = cap;
  a.nbc = cap / KB;
  a.o_sb = o_s_batch; a.o_st = o_s_tok; a.o_sh = o_s_head;
  a.sl2 = sm_scale * 1.4426950408889634f;
  a.seg.n = n_seg;
  for (int c = 0; c < LBW_MAX_SEGMENTS; ++c) { a.seg.slot[c] = 0; a.seg.len[c] = 0; }
  for (int c = 0; c < n_seg; ++c) {
    if (seg_slot[c] < 0 || seg_slot[c] >= slots || seg_len[c] < 1 || seg_len[c] > cap) return LBW_E_SEGMENTS;
    a.seg.slot[c] = seg_slot[c];
    a.seg.len[c] = seg_len[c];
  }
  hipLaunchKernelGGL(attn_fwd_kernel, dim3((unsigned)(a.lp / QT), (unsigned)a.bh), dim3(256), 0,
                     (hipStream_t)stream, q8, q_scale, bias, k8, k_scale, v8, v_scale, out, a);
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return LBW_OK;
}

extern "C" int lbw_qk_logits_i32(const int8_t* q8, int64_t bh, int64_t lq, const int8_t* k8, int64_t slots,
                                 int64_t cap, int64_t slot, int32_t* out, void* stream) {
  if (!q8 || !k8 || !out) return LBW_E_NULL;
  if (bh <= 0 || bh > 65535 || lq <= 0 || cap <= 0 || cap % KB || slot < 0 || slot >= slots) return LBW_E_SHAPE;
  if (((uintptr_t)q8 | (uintptr_t)k8) & 15) return LBW_E_ALIGN;
  const int64_t lp = (lq + QT - 1) / QT * QT;
  hipLaunchKernelGGL(qk_logits_kernel, dim3((unsigned)(lp / QT), (unsigned)(cap / KB), (unsigned)bh), dim3(256),
                     0, (hipStream_t)stream, q8, k8, lp, cap, bh, slot, out);
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return LBW_OK;
}
