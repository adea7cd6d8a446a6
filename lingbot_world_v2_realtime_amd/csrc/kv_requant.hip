// K/V re-quant of finished chunks into the quantised ring cache (gfx950).
//
// Three launches:
//   1. kv_stats:    per 64-token block (grid: block, batch*head, layer): fp32 column sums of K for each 32-token
//                   half, and all of V's quantisation -- V is read once. A block's V scales are powers of two, one per
//                   (key group, channel): group g is the block's 32-token half g, the K-block g of the attention's
//                   64-deep fp8 PV MFMA, whose per-lane E8M0 block scale then applies the scale. 2^e takes the
//                   group's amax into (224, 448]; y = V * 2^-e (exact) -> e4m3
//                   hi = rn(y) and, when a second plane is given, the bf6 (e3m2) residual lo = rn(y - hi) over the
//                   same positions (|y - hi| <= 16 fits bf6 unscaled), packed 48 bytes per channel row (the two
//                   scale groups' 24 bytes as 16 + 16 + 8 + 8, the 8-byte tails swapped in channels with bit 4
//                   set), and the block's 256-byte E8M0 table (byte (32 g + c % 32) * 4 + c / 32 = 127 + e of
//                   channel c, group g: the attention lane that scales channel c's row for group g reads dword
//                   32 g + c % 32 and selects byte c / 32).
//   2. kv_finalize: per (batch*head, layer, 16 channels), the half-block sums added into blocks and 4-block
//                   super-blocks in parallel, the super-blocks left to right, then the mean in the inputs' format.
//   3. kv_quant:    K - mean -> int8 per 64-token block (reads K a second time); with V (a caller that wrote the
//                   K partials itself and never read V) also V as in pass 1.
// The column-sum order is fixed (see the oracle's chunk_mean): s = x[4q] + x[4q+1] + x[4q+2] + x[4q+3] per
// thread, q = 0..7 and q = 8..15 left to right per half-block, the two halves added, the blocks of each 4-block
// super-block left to right, then the super-blocks left to right, so the mean is the same bits on every run and
// on the CPU. (The halves let a producer that sees 32 tokens at a time write the partials itself.)
#include <algorithm>
#include <type_traits>

#include "lbw_common.h"

namespace lbw {

struct ReqArgs {
  int64_t len, heads, bh, slots, cap, slot, nb, nbc;  // nb: blocks of len, nbc: blocks of cap
  int64_t k_sl, k_sb, k_st, k_sh;
  int64_t v_sl, v_sb, v_st, v_sh;
};

constexpr int REQ_SUPER = 4;   // blocks per super-block of the mean's defined order
constexpr int FIN_U = 8;       // super-block sums per lane the finaliser holds in LDS at a time

// V of one 64-token block, quantised by the block's 256 threads. Thread t = (cg, kq) = (t & 15, t >> 4) holds
// channels 8 cg .. + 8 of keys 4 kq .. 4 kq + 3, all of group kq >> 3 (waves 0-1: group 0, waves 2-3: group 1), so
// its e4m3 bytes of one channel are 4 adjacent positions (one dword) of the permuted layout. Steps separated by
// workgroup barriers.
struct VBlockLds {
  // [channel][16 dwords], dword xor-swizzled by channel >> 3: the hi plane's 4 e4m3 bytes of a position quad, and
  // the residual plane's 4 bf6 codes of it in the low 24 bits
  uint32_t tile[2][D * 16];
  float gmax[4][D];           // per wave: max |V| of each channel over the wave's 16 keys
  float rec[2][D];            // 2^-e of [group][channel]
  uint32_t table[64];         // the block's E8M0 scale table, stored out as 64 dwords
};

// Step 1: the thread's 4 x 8 values, and the wave's per-group column maxima into LDS.
template <bool F16>
__device__ __forceinline__ void vblock_max(const v4i* vw, float (&vf)[4][8], VBlockLds& s) {
  const int t = threadIdx.x, lane = t & 63, cg = t & 15;
  float m[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) m[c] = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    unpack8t<F16>(vw[j], vf[j]);
#pragma unroll
    for (int c = 0; c < 8; ++c) m[c] = fmaxf(m[c], fabsf(vf[j][c]));
  }
  // the wave's four key quads of these channels: lanes cg + 16 i
#pragma unroll
  for (int c = 0; c < 8; ++c) m[c] = max_xor32(max_xor16(m[c]));
  if (lane < 16) {
    float* gm = &s.gmax[t >> 6][cg * 8];
    *(float4*)gm = make_float4(m[0], m[1], m[2], m[3]);
    *(float4*)(gm + 4) = make_float4(m[4], m[5], m[6], m[7]);
  }
}

// Step 2: thread t forms the scale of table byte t (group t >> 7, channel 32 (t & 3) + ((t >> 2) & 31)), kept in
// LDS until step 4 stores the table: the power of two 2^e with amax / 2^e in (224, 448]. amax = f * 2^x with f in
// [0.5, 1) (a normal float after the floor): e = x - 9 when f <= 0.875 (mantissa bits <= 0x600000), else x - 8;
// x = biased exponent - 126.
__device__ __forceinline__ void vblock_scale(VBlockLds& s) {
  const int t = threadIdx.x, g = t >> 7, ch = 32 * (t & 3) + ((t >> 2) & 31);
  float mx = fmaxf(s.gmax[2 * g][ch], s.gmax[2 * g + 1][ch]);   // the group's two waves
  mx = fmaxf(mx, AMAX_FLOOR);
  const uint32_t mb = __float_as_uint(mx);
  const int e = (int)(mb >> 23) - ((mb & 0x7FFFFFu) <= 0x600000u ? 135 : 134);
  s.rec[g][ch] = __uint_as_float((uint32_t)(127 - e) << 23);
  ((uint8_t*)s.table)[t] = (uint8_t)(127 + e);
}

// Step 3: e4m3 bytes into the transposed LDS tile, and with `two` the residual plane's bf6 codes beside them.
__device__ __forceinline__ void vblock_quant(const float (&vf)[4][8], bool two, VBlockLds& s) {
  const int t = threadIdx.x, cg = t & 15, kq = t >> 4;
  float rec[8];
  {
    const float* rp = &s.rec[kq >> 3][cg * 8];
    const float4 r0 = *(const float4*)rp, r1 = *(const float4*)(rp + 4);
    rec[0] = r0.x; rec[1] = r0.y; rec[2] = r0.z; rec[3] = r0.w;
    rec[4] = r1.x; rec[5] = r1.y; rec[6] = r1.z; rec[7] = r1.w;
  }
  uint32_t vb[8];   // per channel: 4 e4m3 bytes of keys 4kq .. 4kq+3
  float y[4][8];
  int pk[4][4];     // e4m3 bytes of (key j, channels 2 i, 2 i + 1)
#pragma unroll
  for (int c = 0; c < 8; ++c) vb[c] = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int c = 0; c < 8; c += 2) {
      // |V| * 2^-e <= 448 by the choice of e, and the product is exact (a power-of-two factor), so no clamp: a NaN
      // or an infinity becomes an e4m3 NaN (as the reference's per-channel quantiser makes its channel NaN)
      y[j][c] = __fmul_rn(vf[j][c], rec[c]);
      y[j][c + 1] = __fmul_rn(vf[j][c + 1], rec[c + 1]);
      pk[j][c >> 1] = __builtin_amdgcn_cvt_pk_fp8_f32(y[j][c], y[j][c + 1], 0, false);
      vb[c] |= ((uint32_t)pk[j][c >> 1] & 0xFFu) << (8 * j);
      vb[c + 1] |= (((uint32_t)pk[j][c >> 1] >> 8) & 0xFFu) << (8 * j);
    }
  // row = channel, dword = position / 4
  const int pdw = v_pos_of_key(kq * 4) >> 2;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int ch = cg * 8 + c;
    s.tile[0][ch * 16 + (pdw ^ (ch >> 3))] = vb[c];
  }
  if (two) {
    // Residual plane: y - hi is exact in fp32 and |y - hi| <= 16 lies inside bf6's range. One conversion of the
    // 32 residuals, sources ordered so that code 4 c + j is the residual of (channel c, key j): channel c's 4
    // codes are then bits 24 c .. 24 c + 23 of the result, the packed form of its 4 adjacent positions.
    v16f s0, s1;
#pragma unroll
    for (int i = 0; i < 4; ++i)   // channels 2 i (byte 0 of the e4m3 pairs) and 2 i + 1 (byte 1)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        s0[4 * i + m] = __fsub_rn(y[2 * m][2 * i], __builtin_amdgcn_cvt_f32_fp8(pk[2 * m][i], 0));
        s1[4 * i + m] = __fsub_rn(y[2 * m + 1][2 * i], __builtin_amdgcn_cvt_f32_fp8(pk[2 * m + 1][i], 0));
        s0[4 * i + 2 + m] = __fsub_rn(y[2 * m][2 * i + 1], __builtin_amdgcn_cvt_f32_fp8(pk[2 * m][i], 1));
        s1[4 * i + 2 + m] = __fsub_rn(y[2 * m + 1][2 * i + 1], __builtin_amdgcn_cvt_f32_fp8(pk[2 * m + 1][i], 1));
      }
    const v6i r = cvt_bf6_x32(s0, s1, 1.f);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int bit = 24 * c, dw = bit >> 5, sh = bit & 31;
      const uint32_t w0 = (uint32_t)r[dw], w1 = sh > 8 ? (uint32_t)r[dw + 1] : 0u;
      const uint32_t vl = (sh > 8 ? __builtin_amdgcn_alignbit(w1, w0, sh) : w0 >> sh) & 0xFFFFFFu;
      const int ch = cg * 8 + c;
      s.tile[1][ch * 16 + (pdw ^ (ch >> 3))] = vl;
    }
  }
}

// Step 4: the tiles out. hi plane: each store instruction 1 KB contiguous per wave, store s of thread t writing
// bytes 4096 s + 16 t .. + 15 of the 8 KB tile (channel 64 s + t / 4, dwords 4 (t % 4) .. + 3 of its row). Residual
// plane: thread t packs the 24 bytes of channel t / 2, scale group g = t % 2 (8 position quads of 3 bytes: positions
// 16 g .. 16 g + 15, then 32 + 16 g .. 47 + 16 g, the 32 codes one lane of the 6-bit PV operand holds, since such a
// lane holds a whole K-block) and writes their first 16 at 16 g of the 48-byte row and the last 8 at 32 + 8 g, or
// 40 - 8 g in channels with bit 4 set; a wave writes 1.5 KB of contiguous rows. Threads 0-63 also write the scale
// table, a dword each.
__device__ __forceinline__ void vblock_store(const VBlockLds& s, uint8_t* __restrict__ v8, uint8_t* __restrict__ v8lo,
                                             uint8_t* __restrict__ v_scale, int64_t tile) {
  const int t = threadIdx.x, dw = 4 * (t & 3);
  if (t < 64) ((uint32_t*)(v_scale + tile * 256))[t] = s.table[t];
  {
    uint8_t* vout = v8 + tile * (D * KB) + 16 * t;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int ch = 64 * half + (t >> 2);
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = s.tile[0][ch * 16 + ((dw + i) ^ (ch >> 3))];
      store_once(vout + 4096 * half, v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]});
    }
  }
  if (v8lo) {
    const int ch = t >> 1, g = t & 1;
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = s.tile[1][ch * 16 + ((4 * g + i + (i & 4)) ^ (ch >> 3))];   // quads of group g
    uint8_t* row = v8lo + tile * V_LO_TILE + ch * V_LO_ROW;
    store_once(row + 16 * g, v4i{(int)(w[0] | (w[1] << 24)), (int)((w[1] >> 8) | (w[2] << 16)),
                                 (int)((w[2] >> 16) | (w[3] << 8)), (int)(w[4] | (w[5] << 24))});
    store_once(row + 32 + 8 * (g ^ ((ch >> 4) & 1)), v2i{(int)((w[5] >> 8) | (w[6] << 16)),
                                                         (int)((w[6] >> 16) | (w[7] << 8))});
  }
}

// Thread (cg, q) = (t & 15, t >> 4) sums channels 8 cg .. + 8 over tokens 4 q .. 4 q + 3 of the block and holds the
// same channels and tokens of V. F16: the inputs are fp16 (else bf16).
template <bool F16>
__global__ __launch_bounds__(256) void kv_stats_kernel(const uint16_t* __restrict__ k,
                                                       const uint16_t* __restrict__ v, ReqArgs a,
                                                       float* __restrict__ part_sum, uint8_t* __restrict__ v8,
                                                       uint8_t* __restrict__ v8lo, uint8_t* __restrict__ v_scale) {
  __shared__ float s_sum[16][D];
  __shared__ VBlockLds s_v;
  const int blk = blockIdx.x, bh = blockIdx.y, layer = blockIdx.z;
  const int t = threadIdx.x, cg = t & 15, q = t >> 4;
  const int64_t b = bh / a.heads, h = bh % a.heads;
  const uint16_t* kp = k + layer * a.k_sl + b * a.k_sb + h * a.k_sh + cg * 8;
  const uint16_t* vp = v + layer * a.v_sl + b * a.v_sb + h * a.v_sh + cg * 8;
  v4i kw[4], vw[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t tok = (int64_t)blk * KB + 4 * q + j;
    const bool ok = tok < a.len;
    // V is read once (non-temporal); K is read again by the quantiser, so its lines may stay in the caches
    // (plain loads here: -0.7 % for a 30-layer call against non-temporal ones)
    kw[j] = ok ? *(const v4i*)(kp + tok * a.k_st) : v4i{0, 0, 0, 0};
    vw[j] = ok ? load_once(vp + tok * a.v_st) : v4i{0, 0, 0, 0};
  }
  float s[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) s[c] = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float kf[8];
    unpack8t<F16>(kw[j], kf);
#pragma unroll
    for (int c = 0; c < 8; ++c) s[c] = __fadd_rn(s[c], kf[c]);
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) s_sum[q][cg * 8 + c] = s[c];
  float vf[4][8];
  vblock_max<F16>(vw, vf, s_v);
  __syncthreads();
  {   // thread t: half t >> 7 of the block, channel t & 127
    const int c = t & (D - 1), r0 = (t >> 7) * 8;
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) acc = __fadd_rn(acc, s_sum[r0 + r][c]);
    part_sum[((((int64_t)layer * a.bh + bh) * a.nb + blk) * 2 + (t >> 7)) * D + c] = acc;
  }
  const int64_t tile = (((int64_t)layer * a.slots + a.slot) * a.bh + bh) * a.nbc + blk;
  vblock_scale(s_v);
  __syncthreads();
  vblock_quant(vf, v8lo != nullptr, s_v);
  __syncthreads();
  vblock_store(s_v, v8, v8lo, v_scale, tile);
}

// One workgroup per (batch*head, layer, group of 16 channels). Thread (j, c) = (t >> 4, t & 15) forms the
// super-block sums U[u] = B[4u] + .. + B[4u+3] of channel 16 cgrp + c for u = j, j + 16, .. (all of them at
// once, in parallel); then one thread per channel sums the U left to right.
constexpr int FIN_CH = 16;                 // channels per finaliser workgroup
constexpr int FIN_J = 256 / FIN_CH;        // super-block lanes per channel
template <bool F16>
__global__ __launch_bounds__(256) void kv_finalize_kernel(ReqArgs a, const float* __restrict__ part_sum,
                                                          float* __restrict__ km) {
  __shared__ float buf[FIN_U * FIN_J * FIN_CH];
  const int bh = blockIdx.x, layer = blockIdx.y, cgrp = blockIdx.z;
  const int t = threadIdx.x, c = t & (FIN_CH - 1), j = t / FIN_CH, ch = cgrp * FIN_CH + c;
  const int64_t grp = (int64_t)layer * a.bh + bh;
  const float* bsum = part_sum + grp * a.nb * 2 * D + ch;   // [block][half][channel]
  const int nsup = (int)((a.nb + REQ_SUPER - 1) / REQ_SUPER);
  float tot = 0.f;
  for (int u0 = 0; u0 < nsup; u0 += FIN_U * FIN_J) {
    const int nu = min(FIN_U * FIN_J, nsup - u0);
    for (int uu = j; uu < nu; uu += FIN_J) {
      const int b0 = (u0 + uu) * REQ_SUPER;
      float us = 0.f;   // absent blocks add +0, which leaves the sum unchanged
#pragma unroll
      for (int i = 0; i < REQ_SUPER; ++i) {
        const bool ok = b0 + i < a.nb;
        const int64_t o = (int64_t)(b0 + i) * 2 * D;
        us = __fadd_rn(us, ok ? __fadd_rn(bsum[o], bsum[o + D]) : 0.f);
      }
      buf[uu * FIN_CH + c] = us;
    }
    __syncthreads();
    if (j == 0)
      for (int uu = 0; uu < nu; ++uu) tot = __fadd_rn(tot, buf[uu * FIN_CH + c]);
    __syncthreads();
  }
  if (j == 0) {
    const int64_t so = (((int64_t)layer * a.slots + a.slot) * a.bh + bh) * D + ch;
    km[so] = round16<F16>(__fdiv_rn(tot, (float)a.len));   // the mean in the inputs' own format
  }
}

// Thread t owns channels 8*(t & 15) .. +8 and the 4 consecutive keys 4*(t >> 4) .. +4 of the block. Layers go last
// to first: the statistics pass read the last layers most recently, so the first re-reads can still find them in
// the memory-side cache. WITH_V: V of the block is quantised here too.
template <bool F16, bool WITH_V>
__global__ __launch_bounds__(256) void kv_quant_kernel(const uint16_t* __restrict__ k,
                                                       const uint16_t* __restrict__ v, ReqArgs a,
                                                       int8_t* __restrict__ k8, float* __restrict__ k_scale,
                                                       const float* __restrict__ km, uint8_t* __restrict__ v8,
                                                       uint8_t* __restrict__ v8lo, uint8_t* __restrict__ v_scale) {
  __shared__ float s_red[4];
  __shared__ std::conditional_t<WITH_V, VBlockLds, int> s_v;   // (no V tile without V)
  const int blk = blockIdx.x, bh = blockIdx.y, layer = gridDim.z - 1 - blockIdx.z;
  const int t = threadIdx.x, cg = t & 15, kq = t >> 4;
  const int64_t b = bh / a.heads, h = bh % a.heads;
  const uint16_t* kp = k + layer * a.k_sl + b * a.k_sb + h * a.k_sh + cg * 8;
  const int64_t slot_bh = ((int64_t)layer * a.slots + a.slot) * a.bh + bh;
  float mean[8];
  {
    const float* kmp = km + slot_bh * D + cg * 8;
#pragma unroll
    for (int c = 0; c < 8; ++c) mean[c] = kmp[c];
  }
  v4i vw[4];
  if constexpr (WITH_V) {
    const uint16_t* vp = v + layer * a.v_sl + b * a.v_sb + h * a.v_sh + cg * 8;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t tok = (int64_t)blk * KB + kq * 4 + j;
      vw[j] = tok < a.len ? *(const v4i*)(vp + tok * a.v_st) : v4i{0, 0, 0, 0};
    }
  }
  float x[4][8];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t tok = (int64_t)blk * KB + kq * 4 + j;
    const bool ok = tok < a.len;
    v4i kw = ok ? *(const v4i*)(kp + tok * a.k_st) : v4i{0, 0, 0, 0};
    float kf[8];
    unpack8t<F16>(kw, kf);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      x[j][c] = ok ? __fsub_rn(kf[c], mean[c]) : 0.f;
      amax = fmaxf(amax, fabsf(x[j][c]));
    }
  }
  // block amax over 64 tokens x 128 channels
  amax = wave_max(amax);
  if ((t & 63) == 0) s_red[t >> 6] = amax;
  float vf[4][8];
  if constexpr (WITH_V) vblock_max<F16>(vw, vf, s_v);
  __syncthreads();
  const int64_t tile = slot_bh * a.nbc + blk;
  if constexpr (WITH_V) vblock_scale(s_v);
  amax = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  amax = fmaxf(amax, AMAX_FLOOR);
  const float recip = __fdiv_rn(127.f, amax);
  if (t == 0) k_scale[tile] = __fdiv_rn(amax, 127.f);
  int8_t* kout = k8 + (slot_bh * a.cap + (int64_t)blk * KB) * D + cg * 8;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      lo |= ((uint32_t)quant_i8(x[j][c], recip) & 0xFFu) << (8 * c);
      hi |= ((uint32_t)quant_i8(x[j][c + 4], recip) & 0xFFu) << (8 * c);
    }
    store_once(kout + (kq * 4 + j) * D, v2i{(int)lo, (int)hi});
  }
  if constexpr (WITH_V) {
    __syncthreads();
    vblock_quant(vf, v8lo != nullptr, s_v);
    __syncthreads();
    vblock_store(s_v, v8, v8lo, v_scale, tile);
  }
}

int kv_requant_check(int64_t layers, int64_t batch, int64_t len, int64_t heads, const int8_t* k8,
                     const float* k_scale, const float* km, const uint8_t* v8, const uint8_t* v8lo,
                     const uint8_t* v_scale, int64_t slots, int64_t cap, int64_t slot) {
  if (!k8 || !k_scale || !km || !v8 || !v_scale) return LBW_E_NULL;
  if (layers <= 0 || batch <= 0 || heads <= 0 || len <= 0 || slots <= 0 || cap <= 0) return LBW_E_SHAPE;
  if (cap % KB != 0 || len > cap || slot < 0 || slot >= slots) return LBW_E_SHAPE;
  if (layers > 65535 || batch * heads > 65535 || cap / KB > (int64_t)1 << 30) return LBW_E_SHAPE;
  if (((uintptr_t)k8 | (uintptr_t)v8 | (uintptr_t)v8lo) & 15 || (uintptr_t)v_scale & 3) return LBW_E_ALIGN;
  return LBW_OK;
}

int kv_requant_launch(bool with_stats, bool f16, const uint16_t* k, const uint16_t* v, int64_t layers, int64_t batch,
                      int64_t len, int64_t heads, int64_t k_s_layer, int64_t k_s_batch, int64_t k_s_tok,
                      int64_t k_s_head, int64_t v_s_layer, int64_t v_s_batch, int64_t v_s_tok, int64_t v_s_head,
                      int8_t* k8, float* k_scale, float* km, uint8_t* v8, uint8_t* v8lo, uint8_t* v_scale,
                      int64_t slots, int64_t cap, int64_t slot, void* workspace, void* stream) {
  if (!k || !v || !workspace) return LBW_E_NULL;
  if (const int st = kv_requant_check(layers, batch, len, heads, k8, k_scale, km, v8, v8lo, v_scale, slots, cap,
                                      slot))
    return st;
  const int64_t strides[8] = {k_s_layer, k_s_batch, k_s_tok, k_s_head, v_s_layer, v_s_batch, v_s_tok, v_s_head};
  for (int64_t s : strides)
    if (s % 8 != 0) return LBW_E_ALIGN;
  if (((uintptr_t)k | (uintptr_t)v | (uintptr_t)workspace) & 15) return LBW_E_ALIGN;
  ReqArgs a;
  a.len = len; a.heads = heads; a.bh = batch * heads; a.slots = slots; a.cap = cap; a.slot = slot;
  a.nb = (len + KB - 1) / KB;
  a.nbc = cap / KB;
  a.k_sl = k_s_layer; a.k_sb = k_s_batch; a.k_st = k_s_tok; a.k_sh = k_s_head;
  a.v_sl = v_s_layer; a.v_sb = v_s_batch; a.v_st = v_s_tok; a.v_sh = v_s_head;
  float* part_sum = (float*)workspace;
  if (const int dv = check_device()) return dv;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)a.nb, (unsigned)a.bh, (unsigned)layers);
  const dim3 fgrid((unsigned)a.bh, (unsigned)layers, D / FIN_CH);
  // with the statistics pass, V is quantised there and the last pass is K only; without it, the last pass does both
  if (f16) {
    if (with_stats)
      hipLaunchKernelGGL(kv_stats_kernel<true>, grid, dim3(256), 0, st, k, v, a, part_sum, v8, v8lo, v_scale);
    hipLaunchKernelGGL(kv_finalize_kernel<true>, fgrid, dim3(256), 0, st, a, part_sum, km);
    if (with_stats)
      hipLaunchKernelGGL((kv_quant_kernel<true, false>), grid, dim3(256), 0, st, k, v, a, k8, k_scale, km, v8, v8lo,
                         v_scale);
    else
      hipLaunchKernelGGL((kv_quant_kernel<true, true>), grid, dim3(256), 0, st, k, v, a, k8, k_scale, km, v8, v8lo,
                         v_scale);
  } else {
    if (with_stats)
      hipLaunchKernelGGL(kv_stats_kernel<false>, grid, dim3(256), 0, st, k, v, a, part_sum, v8, v8lo, v_scale);
    hipLaunchKernelGGL(kv_finalize_kernel<false>, fgrid, dim3(256), 0, st, a, part_sum, km);
    if (with_stats)
      hipLaunchKernelGGL((kv_quant_kernel<false, false>), grid, dim3(256), 0, st, k, v, a, k8, k_scale, km, v8, v8lo,
                         v_scale);
    else
      hipLaunchKernelGGL((kv_quant_kernel<false, true>), grid, dim3(256), 0, st, k, v, a, k8, k_scale, km, v8, v8lo,
                         v_scale);
  }
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return LBW_OK;
}

}  // namespace lbw

using namespace lbw;

extern "C" int64_t lbw_kv_requant_workspace_bytes(int64_t layers, int64_t bh, int64_t len) {
  if (layers <= 0 || bh <= 0 || len <= 0) return 0;
  const int64_t nb = (len + KB - 1) / KB;
  return 2 * layers * bh * nb * D * (int64_t)sizeof(float);
}

extern "C" int lbw_kv_requant(const uint16_t* k, const uint16_t* v, int dtype, int64_t layers, int64_t batch,
                              int64_t len, int64_t heads, int64_t k_s_layer, int64_t k_s_batch,
                              int64_t k_s_tok, int64_t k_s_head, int64_t v_s_layer, int64_t v_s_batch,
                              int64_t v_s_tok, int64_t v_s_head, int8_t* k8, float* k_scale, float* km,
                              uint8_t* v8, uint8_t* v8lo, uint8_t* v_scale, int64_t slots, int64_t cap,
                              int64_t slot, void* workspace, void* stream) {
  if (dtype != LBW_DTYPE_BF16 && dtype != LBW_DTYPE_FP16) return LBW_E_SHAPE;
  return kv_requant_launch(true, dtype == LBW_DTYPE_FP16, k, v, layers, batch, len, heads, k_s_layer, k_s_batch,
                           k_s_tok, k_s_head,
                           v_s_layer, v_s_batch, v_s_tok, v_s_head, k8, k_scale, km, v8, v8lo, v_scale, slots,
                           cap, slot, workspace, stream);
}
