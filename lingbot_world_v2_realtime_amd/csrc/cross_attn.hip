// Cross-attention of the DiT blocks against the text context (gfx950): bf16 flash attention with fp32
// accumulation, for a short key sequence (the 512 context tokens) that every layer and pass re-reads.
//
//   cross_prepare_kernel: the context's K and V, [B, Lk, H, 128] bf16, into the layout the attention reads:
//                         K [BH][Lkp][128] and V transposed, [BH][128][Lkp], keys zero-padded to Lkp = ceil64(Lk).
//                         Done once per generation (the reference caches the cross-attention K / V the same way).
//   cross_attn_kernel:    one workgroup per (128-query tile, batch * head), 4 waves x 32 queries, three workgroups
//                         a CU (168 registers, 48 KB of LDS each), so the DiT's 576 tiles run in one round on 768
//                         slots. Per 32-key tile (three LDS stages, filled by direct global -> LDS loads two tiles
//                         ahead): S^T = K Q^T on v_mfma_f32_32x32x16_bf16 (lane = query, 16 keys per lane), an
//                         online softmax in the exp2 domain (one FMA and one exp2 per score, the key mask only on
//                         a ragged last tile), P^T in bf16 straight from the S^T registers into the B operand of
//                         O^T += V^T P^T (the keys of the two products are permuted alike, so P needs no exchange
//                         between lanes), then O / l.
#include <type_traits>

#include "lbw_common.h"

namespace lbw {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

constexpr int XQ = 128;                     // queries per workgroup
constexpr int XK = 32;                      // keys per attention tile
constexpr int XKT = XK / 32;                // 32-key S^T products per tile
constexpr int XNC = XK / 8;                 // 16-byte chunks per V^T row of a tile
constexpr int XSTAGES = XK == 32 ? 3 : 2;   // LDS stages: tile t + XSTAGES - 1 loads while tile t is read
constexpr int XOCC = XK == 32 ? 3 : 2;      // workgroups per CU (registers and LDS sized for it)
constexpr int XPK = 64;                     // the prepared context pads its keys to a multiple of this
constexpr int XWAVES = 4;
constexpr int XT = XWAVES * 64;    // threads
constexpr int XMAX_BATCH = 64;

struct XArgs {
  int64_t lq, lk, lkp, heads, bh;
  int64_t q_sb, q_st, q_sh;
  int64_t o_sb, o_st, o_sh;
  float sl2;   // sm_scale * log2(e)
  int klen[XMAX_BATCH];   // valid keys per batch entry (1 .. lk)
};

// Key held at position p of a 32-key span of a prepared V^T row: inside each 16-key group the middle two quarters
// are swapped (positions 4-7 hold keys 8-11, positions 8-11 keys 4-7).
__device__ __forceinline__ int vt_key(int p) {
  const int qd = (p >> 2) & 3;
  return (p & ~15) + ((qd == 1 ? 2 : qd == 2 ? 1 : qd) << 2) + (p & 3);
}

// Workgroup (64-key padding tile, batch * head): K rows copied, V transposed through LDS; keys past lk are zero.
__global__ __launch_bounds__(256) void cross_prepare_kernel(const uint16_t* __restrict__ k,
                                                            const uint16_t* __restrict__ v, int64_t lk,
                                                            int64_t lkp, int64_t heads, int64_t k_sb,
                                                            int64_t k_st, int64_t k_sh, int64_t v_sb,
                                                            int64_t v_st, int64_t v_sh, uint16_t* __restrict__ kp,
                                                            uint16_t* __restrict__ vt) {
  __shared__ uint16_t s_v[XPK][D + 2];
  const int tile = blockIdx.x, bh = blockIdx.y, t = threadIdx.x;
  const int64_t b = bh / heads, h = bh % heads;
  // thread t: key 4 (t >> 4) .. + 3, channels 8 (t & 15) .. + 7
  const int c8 = (t & 15) * 8;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int kk = 4 * (t >> 4) + j;
    const int64_t key = (int64_t)tile * XPK + kk;
    v4i kw = {0, 0, 0, 0}, vw = {0, 0, 0, 0};
    if (key < lk) {
      kw = *(const v4i*)(k + b * k_sb + key * k_st + h * k_sh + c8);
      vw = *(const v4i*)(v + b * v_sb + key * v_st + h * v_sh + c8);
    }
    *(v4i*)(kp + ((int64_t)bh * lkp + key) * D + c8) = kw;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      s_v[kk][c8 + 2 * q] = (uint16_t)((uint32_t)vw[q] & 0xFFFFu);
      s_v[kk][c8 + 2 * q + 1] = (uint16_t)((uint32_t)vw[q] >> 16);
    }
  }
  __syncthreads();
  // thread t: channel t >> 1, keys 32 (t & 1) .. + 31 -> 64 contiguous bytes of V^T, each 16-key group stored
  // in the order 0-3, 8-11, 4-7, 12-15 (vt_key): the 8 keys a PV fragment lane takes are one 16-byte chunk
  const int ch = t >> 1, k0 = (t & 1) * 32;
  uint32_t w[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int kk = k0 + vt_key(2 * i);   // stored positions 2 i, 2 i + 1 hold consecutive keys
    w[i] = (uint32_t)s_v[kk][ch] | ((uint32_t)s_v[kk + 1][ch] << 16);
  }
  uint16_t* dst = vt + ((int64_t)bh * D + ch) * lkp + (int64_t)tile * XPK + k0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    *(v4i*)(dst + 8 * i) = v4i{(int)w[4 * i], (int)w[4 * i + 1], (int)w[4 * i + 2], (int)w[4 * i + 3]};
}

__device__ __forceinline__ bf8 as_bf8(const v4i x) { return __builtin_bit_cast(bf8, x); }

typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
// two fp32 -> packed bf16, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const bf2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Global -> LDS copy of 16 bytes per lane (lane i lands at M0 + 16 i) from a wave-uniform base plus a 32-bit
// per-lane byte offset (the global instruction's scalar-base form: no 64-bit address per lane), as inline asm:
// the compiler's builtin is modelled as a FLAT access that may touch LDS, which would make every LDS wait drain
// all reads in flight.
__device__ __forceinline__ void xdma16(const void* base, uint32_t off, uint8_t* lds) {
  uint32_t keep;
  const uint32_t dst = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)lds;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\t"
               "s_mov_b32 m0, %0"
               : "=&s"(keep) : "v"(off), "s"(base), "s"(dst) : "memory");
}

// LDS tiles, XOR-swizzled by row so the fragment reads spread over the banks:
//   K   [XK keys][256 B]: 16-byte chunk c of row r sits at position c ^ (r & 15)
//   V^T [128 channels][2 XK B]: chunk c of row r sits at position c ^ vswz(r), so the 16 rows a fragment read
//       serves at a time cover 16 distinct (row offset, position) bank groups
constexpr int XK_TILE = XK * D * 2;
constexpr int XV_TILE = D * XK * 2;
constexpr int XSTAGE = XK_TILE + XV_TILE;
static_assert(XSTAGES * XSTAGE * XOCC <= 163840, "LDS");
__device__ __forceinline__ int vswz(int r) { return (r >> (XNC == 4 ? 2 : 1)) & (XNC - 1); }

// s_waitcnt on vmcnt only (lgkmcnt and expcnt at their maxima): vmcnt(n) for n = 0 .. 15
__device__ __forceinline__ void xwait_vm(int n) {
  switch (n) {
    case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
    case 8: __builtin_amdgcn_s_waitcnt(0x0F78); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
  }
}

template <int N>
using ic = std::integral_constant<int, N>;

__global__ __launch_bounds__(XT, XOCC) void cross_attn_kernel(const uint16_t* __restrict__ q,
                                                              const uint16_t* __restrict__ kp,
                                                              const uint16_t* __restrict__ vt, XArgs a,
                                                              uint16_t* __restrict__ out) {
  __shared__ __align__(16) uint8_t xlds[XSTAGES * XSTAGE];
  const int qt = blockIdx.x, bh = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63, lq = lane & 31, hf = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t b = bh / a.heads, h = bh % a.heads;
  const int klen = a.klen[b];
  const int ntile = (klen + XK - 1) / XK;
  const uint8_t* kbase = (const uint8_t*)(kp + (int64_t)bh * a.lkp * D);
  const uint8_t* vbase = (const uint8_t*)(vt + (int64_t)bh * D * a.lkp);
  const int64_t vrow_bytes = a.lkp * 2;

  // Q rows, whole: lane -> row 4 j + lane / 16 of the wave's 32, 16-byte chunk lane & 15 (rows past lq are zero);
  // through LDS into the Q^T B operand below
  const int c16 = lane & 15;
  v4i qraw[8];
  {
    const uint16_t* qb = q + b * a.q_sb + h * a.q_sh + c16 * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t row = (int64_t)qt * XQ + 32 * w + 4 * j + (lane >> 4);
      qraw[j] = row < a.lq ? *(const v4i*)(qb + row * a.q_st) : v4i{0, 0, 0, 0};
    }
  }

  // DMA: wave w moves K rows (XK / 4) w .. + XK / 4 and V^T rows 32 w .. 32 w + 31 of a tile, 1 KB per
  // instruction, XK / 16 of each a wave per tile; byte offsets from the tile's scalar base below 2^31
  constexpr int NDMA = XK / 16;
  constexpr int VROWS = 1024 / (2 * XK);   // V^T rows per 1 KB
  uint32_t koff[NDMA], voff[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int r = (XK / 4) * w + 4 * i + (lane >> 4), p = lane & 15;
    koff[i] = (uint32_t)(r * (D * 2) + ((p ^ (r & 15)) << 4));
    const int rv = 32 * w + VROWS * i + lane / XNC, pv = lane % XNC;
    voff[i] = (uint32_t)(rv * vrow_bytes + ((pv ^ vswz(rv)) << 4));
  }
  auto issue = [&](int tl, int stg) {
    uint8_t* sk = xlds + stg * XSTAGE;
    uint8_t* sv = sk + XK_TILE;
    const uint8_t* kt_base = kbase + (int64_t)tl * XK_TILE;
    const uint8_t* vt_base = vbase + (int64_t)tl * (XK * 2);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      xdma16(kt_base, koff[i], sk + ((XK / 4) * w + 4 * i) * 256);
      xdma16(vt_base, voff[i], sv + (32 * w + VROWS * i) * (2 * XK));
    }
  };

  // fragment read offsets inside a stage: K chunk 2 st + hf of row lq; V^T chunk 4 kt + 2 u + hf of row lq
  // (the rows of further products follow at fixed distances)
  int kro[8], vro[XKT][2];
#pragma unroll
  for (int st = 0; st < 8; ++st) kro[st] = lq * 256 + (((2 * st + hf) ^ (lq & 15)) << 4);
#pragma unroll
  for (int kt = 0; kt < XKT; ++kt)
#pragma unroll
    for (int u = 0; u < 2; ++u) vro[kt][u] = XK_TILE + lq * (2 * XK) + (((4 * kt + 2 * u + hf) ^ vswz(lq)) << 4);

  v16f o[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[mt][i] = 0.f;
  float m_ref = -INFINITY, l_run = 0.f;

  issue(0, 0);   // tile 0's K / V travel with the Q rows
  // Q^T B operand: lane (lq, hf) holds query 32 w + lq of the tile, channels 16 st + 8 hf .. + 8. The rows pass
  // through the LDS after stage 0 (256-byte rows, chunk c at position c ^ (row & 15)), 8 KB a wave.
  static_assert(XSTAGE + XWAVES * 32 * 256 <= XSTAGES * XSTAGE, "Q staging");
  bf8 qf[8];
  {
    uint8_t* sq = xlds + XSTAGE + w * 32 * 256;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = 4 * j + (lane >> 4);
      *(v4i*)(sq + r * 256 + ((c16 ^ (r & 15)) << 4)) = qraw[j];
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the wave's rows are in LDS (it reads only its own)
#pragma unroll
    for (int st = 0; st < 8; ++st) qf[st] = as_bf8(*(const v4i*)(sq + lq * 256 + (((2 * st + hf) ^ (lq & 15)) << 4)));
    asm volatile("" : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]), "+v"(qf[4]), "+v"(qf[5]), "+v"(qf[6]),
                 "+v"(qf[7]));
  }
  __syncthreads();   // every wave holds its fragments: the staging area is free for the next tiles' DMA
#pragma unroll
  for (int i = 1; i < XSTAGES - 1; ++i)
    if (i < ntile) issue(i, i);

  // The tiles go in pairs: both tiles' scores, one running-max update and O rescale for the 64 keys, then each
  // tile's P V. Tile t sits in stage t % 3; a pair's first DMA (tile t0 + 2) goes into the stage of tile t0 - 1,
  // its second (tile t0 + 3) into the first tile's stage once every wave's P V of it is done. Stages are
  // constants, so every LDS address is a register plus an immediate.
  static_assert(XK == 32 && XSTAGES == 3, "the pair schedule assumes three stages of 32 keys");
  // S^T of the tile in stage S: lane (lq, hf) value i is key 8 (i >> 2) + 4 hf + (i & 3) of the tile
  auto qk = [&](auto stage) {
    constexpr int S = decltype(stage)::value;
    const uint8_t* sb = xlds + S * XSTAGE;
    v16f sc;
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] = 0.f;
#pragma unroll
    for (int st = 0; st < 8; ++st)
      sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf8(*(const v4i*)(sb + kro[st])), qf[st], sc, 0, 0, 0);
    return sc;
  };
  auto mask = [&](v16f& sc, int tl) {   // the ragged last tile: keys past klen drop out
    if ((tl + 1) * XK > klen) {
      const int kb = tl * XK + 4 * hf;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (kb + 8 * (i >> 2) + (i & 3) >= klen) sc[i] = -INFINITY;
    }
  };
  // P^T fragment u: values i = 8 u .. 8 u + 7 = keys 16 u + {4 hf + 0..3, 8 + 4 hf + 0..3}; P = exp2(s sl2 - m)
  // <= 1, on v_exp_f32 itself (exp2f adds a compare, a select and a v_ldexp per value to keep results below
  // 2^-126 exact; weights that small do not matter next to the row's largest, exactly 1). Returns the sum of P.
  auto probs = [&](const v16f& sc, float nm, v4i (&pf)[2]) {
    float ps[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) p[j] = __builtin_amdgcn_exp2f(fmaf(sc[8 * u + j], a.sl2, nm));
      ps[u] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
      pf[u] = v4i{(int)pack_bf16(p[0], p[1]), (int)pack_bf16(p[2], p[3]), (int)pack_bf16(p[4], p[5]),
                  (int)pack_bf16(p[6], p[7])};
    }
    return ps[0] + ps[1];
  };
  // O^T += V^T P^T: A = V^T row 32 mt + lq, the lane's 8 keys of u: one 16-byte chunk (the prepared V^T stores
  // each 16-key group in the fragment order)
  auto pv = [&](auto stage, const v4i (&pf)[2]) {
    constexpr int S = decltype(stage)::value;
    const uint8_t* sb = xlds + S * XSTAGE;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const v4i vf = *(const v4i*)(sb + mt * 32 * (2 * XK) + vro[0][u]);
        o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf8(vf), as_bf8(pf[u]), o[mt], 0, 0, 0);
      }
  };
  auto pair = [&](int t0, auto sa, auto sb) {
    constexpr int SA = decltype(sa)::value, SB = decltype(sb)::value, SC = 3 - SA - SB;
    const bool two = t0 + 1 < ntile;   // workgroup-uniform
    xwait_vm(0);       // this wave's pieces of tiles t0 and t0 + 1 have landed
    __syncthreads();   // ... and every wave's; every wave is done with tile t0 - 1's stage
    if (t0 + 2 < ntile) issue(t0 + 2, SC);
    v16f s0 = qk(ic<SA>{}), s1;
    if (two) {
      s1 = qk(ic<SB>{});
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) s1[i] = -INFINITY;
    }
    __builtin_amdgcn_sched_barrier(0);   // the phases stay apart: reads hoisted across them cost registers
    mask(s0, t0);
    if (two) mask(s1, t0 + 1);
    float m3[6];
#pragma unroll
    for (int i = 0; i < 5; ++i) m3[i] = fmaxf(fmaxf(s0[3 * i], s0[3 * i + 1]), s0[3 * i + 2]);
    m3[5] = fmaxf(s0[15], s1[15]);
    float mx = fmaxf(fmaxf(m3[0], m3[1]), fmaxf(m3[2], m3[3]));
    mx = fmaxf(mx, fmaxf(m3[4], m3[5]));
#pragma unroll
    for (int i = 0; i < 5; ++i) mx = fmaxf(mx, fmaxf(fmaxf(s1[3 * i], s1[3 * i + 1]), s1[3 * i + 2]));
    mx = max_xor32(mx) * a.sl2;   // exp2 domain; finite: every tile holds a valid key
    // the exact running max: the row's largest P is exactly 1, which keeps its bf16 rounding error at zero (a
    // reference max that moves only by steps measured 19 % more mean error on a peaked softmax)
    const float m_new = fmaxf(m_ref, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_ref - m_new);   // m_ref = -inf at the first tile: 0
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[mt][i] *= alpha;
    m_ref = m_new;
    v4i pf0[2], pf1[2];
    float lt = probs(s0, -m_ref, pf0);
    if (two) lt += probs(s1, -m_ref, pf1);
    l_run = fmaf(l_run, alpha, lt);
    __builtin_amdgcn_sched_barrier(0);
    pv(ic<SA>{}, pf0);
    __syncthreads();   // every wave is done with tile t0's stage
    if (t0 + 3 < ntile) issue(t0 + 3, SA);
    if (two) pv(ic<SB>{}, pf1);
  };
  for (int t0 = 0; t0 < ntile; t0 += 6) {
    pair(t0, ic<0>{}, ic<1>{});
    if (t0 + 2 < ntile) pair(t0 + 2, ic<2>{}, ic<0>{});
    if (t0 + 4 < ntile) pair(t0 + 4, ic<1>{}, ic<2>{});
  }
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
    l_run = __uint_as_float(r[0]) + __uint_as_float(r[1]);   // both halves of the query's keys
  }
  // O / l through LDS (rows of 272 bytes: the 16 rows a 16-lane group writes start 16 bytes apart in the banks),
  // then out as whole rows: each store instruction writes 4 rows x 256 contiguous bytes
  const float inv_l = 1.f / l_run;
  constexpr int OROW = D * 2 + 16;
  static_assert(XWAVES * 32 * OROW <= XSTAGES * XSTAGE, "O staging");
  __syncthreads();   // every wave is done with the stages
  uint8_t* so = xlds + w * 32 * OROW;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i)   // channels 32 mt + 8 i + 4 hf + 0..3
      *(uint2*)(so + lq * OROW + (32 * mt + 8 * i + 4 * hf) * 2) =
          make_uint2(pack_bf16(o[mt][4 * i] * inv_l, o[mt][4 * i + 1] * inv_l),
                     pack_bf16(o[mt][4 * i + 2] * inv_l, o[mt][4 * i + 3] * inv_l));
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's rows are in LDS (each wave reads only its own)
  uint16_t* ob = out + b * a.o_sb + h * a.o_sh + c16 * 8;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = 4 * j + (lane >> 4);
    const int64_t row = (int64_t)qt * XQ + 32 * w + r;
    const v4i x = *(const v4i*)(so + r * OROW + c16 * 16);
    if (row < a.lq) *(v4i*)(ob + row * a.o_st) = x;
  }
}

}  // namespace lbw

using namespace lbw;

extern "C" int lbw_cross_prepare(const uint16_t* k, const uint16_t* v, int64_t batch, int64_t lk, int64_t heads,
                                 int64_t k_s_batch, int64_t k_s_tok, int64_t k_s_head, int64_t v_s_batch,
                                 int64_t v_s_tok, int64_t v_s_head, uint16_t* k_prep, uint16_t* vt_prep,
                                 void* stream) {
  if (!k || !v || !k_prep || !vt_prep) return LBW_E_NULL;
  if (batch <= 0 || lk <= 0 || heads <= 0 || batch * heads > 65535 || lk > (1 << 20)) return LBW_E_SHAPE;
  const int64_t strides[6] = {k_s_batch, k_s_tok, k_s_head, v_s_batch, v_s_tok, v_s_head};
  for (int64_t s : strides)
    if (s % 8 != 0) return LBW_E_ALIGN;
  if (((uintptr_t)k | (uintptr_t)v | (uintptr_t)k_prep | (uintptr_t)vt_prep) & 15) return LBW_E_ALIGN;
  if (const int dv = check_device()) return dv;
  const int64_t lkp = (lk + XPK - 1) / XPK * XPK;
  hipLaunchKernelGGL(cross_prepare_kernel, dim3((unsigned)(lkp / XPK), (unsigned)(batch * heads)), dim3(256), 0,
                     (hipStream_t)stream, k, v, lk, lkp, heads, k_s_batch, k_s_tok, k_s_head, v_s_batch, v_s_tok,
                     v_s_head, k_prep, vt_prep);
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return LBW_OK;
}

extern "C" int lbw_cross_attn_fwd(const uint16_t* q, int64_t batch, int64_t lq, int64_t heads, int64_t q_s_batch,
                                  int64_t q_s_tok, int64_t q_s_head, const uint16_t* k_prep,
                                  const uint16_t* vt_prep, int64_t lk, const int32_t* k_lens, uint16_t* out,
                                  int64_t o_s_batch, int64_t o_s_tok, int64_t o_s_head, float sm_scale,
                                  void* stream) {
  if (!q || !k_prep || !vt_prep || !out) return LBW_E_NULL;
  if (batch <= 0 || lq <= 0 || heads <= 0 || lk <= 0 || batch > XMAX_BATCH || batch * heads > 65535 ||
      lk > (1 << 20))
    return LBW_E_SHAPE;
  if (!(sm_scale > 0.f) || !(sm_scale < INFINITY)) return LBW_E_SHAPE;
  const int64_t strides[6] = {q_s_batch, q_s_tok, q_s_head, o_s_batch, o_s_tok, o_s_head};
  for (int64_t s : strides)
    if (s % 8 != 0) return LBW_E_ALIGN;
  if (((uintptr_t)q | (uintptr_t)k_prep | (uintptr_t)vt_prep | (uintptr_t)out) & 15) return LBW_E_ALIGN;
  XArgs a;
  a.lq = lq; a.lk = lk; a.lkp = (lk + XPK - 1) / XPK * XPK; a.heads = heads; a.bh = batch * heads;
  a.q_sb = q_s_batch; a.q_st = q_s_tok; a.q_sh = q_s_head;
  a.o_sb = o_s_batch; a.o_st = o_s_tok; a.o_sh = o_s_head;
  a.sl2 = sm_scale * 1.4426950408889634f;
  for (int i = 0; i < XMAX_BATCH; ++i) a.klen[i] = (int)lk;
  if (k_lens) {   // the varlen key lengths of the reference's flash call, a host array; each 1 .. lk
    for (int i = 0; i < batch; ++i) {
      if (k_lens[i] < 1 || k_lens[i] > lk) return LBW_E_SHAPE;
      a.klen[i] = k_lens[i];
    }
  }
  if ((lq + XQ - 1) / XQ > 0x7fffffff) return LBW_E_SHAPE;
  if (const int dv = check_device()) return dv;
  hipLaunchKernelGGL(cross_attn_kernel, dim3((unsigned)((lq + XQ - 1) / XQ), (unsigned)(batch * heads)), dim3(XT),
                     0, (hipStream_t)stream, q, k_prep, vt_prep, a, out);
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return LBW_OK;
}
