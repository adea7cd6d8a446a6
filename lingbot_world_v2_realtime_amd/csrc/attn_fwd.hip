// Quantized attention forward for gfx950: int8 QK^T on v_mfma_i32_32x32x32_i8, online softmax in the exp2
// domain, e4m3 P times e4m3 V on v_mfma_scale_f32_32x32x64_f8f6f4 and, for V's optional residual plane, bf6(P / 16)
// times the bf6 residual on the same instruction with both operands 6-bit (twice the fp8 rate), fp32 accumulation.
//
// Tile: 8 waves x 32 queries = 256 queries of one batch*head. Each wave computes S^T = K Q^T (keys on the MFMA
// M axis, queries on N), so a lane holds one query and 16 keys of each 32x32 S tile: the row max is in-lane
// plus one exchange with lane ^ 32 (v_permlane32_swap), and the S tile's register layout is directly the B
// operand (P^T) of the PV product O^T = V^T P^T because the fp8 V block stores its keys in that order. The row
// sum of the rounded P is one more matrix product per block (a ones operand times the same P^T).
// The int32 accumulator starts at the bits of 1 / (2 pi) (an inline constant of the MFMA), so its result reads
// directly as the float 1/(2 pi) + S * 2^-26 (|S| <= 2^21, one binade): the int -> float conversion is free, and
// the logit scale carries the factor 2^26. The two 4-wave halves of the workgroup run
// phase-shifted (one half's MFMAs under the other half's softmax); K / V blocks of 64 keys reach LDS by direct
// global -> LDS loads several blocks ahead (see attend_range).
//
// Scheduling: a persistent grid of `gx` workgroups per XCD (workgroup g runs on XCD g % 8). The query tiles
// (head-major, so one head's tiles are contiguous) are split into 8 contiguous ranges, one per XCD, so each
// XCD's L2 holds the K/V of ~1.5 heads. Within an XCD, whole tiles are dealt round-robin while every workgroup
// gets one; the remaining tiles' (tile, key block) units are cut into equal contiguous pieces, one per
// workgroup. A piece that is not a whole tile leaves an unnormalised partial (O, running max, row sum) in the
// workspace, and attn_merge_kernel combines the pieces of each split tile.
#include <atomic>
#include <type_traits>

#include "lbw_common.h"

namespace lbw {

constexpr int XCDS = 8;
constexpr int XCDS_MAX = 8;
constexpr int TILE_BYTES = KB * D;   // 8 KB: one 64-key K tile or one 64-key fp8 V block

struct AttnArgs {
  int64_t lq, lp, bh, heads, cap, nbc;
  int64_t o_sb, o_st, o_sh;
  float sl2;                       // sm_scale * log2(e)
  int n_seg, nb, q_tiles, n_tiles, gx;
  int seg_slot[LBW_MAX_SEGMENTS];
  int seg_fb[LBW_MAX_SEGMENTS];         // the slot block holding the chunk's first attended key
  int seg_lead[LBW_MAX_SEGMENTS];       // keys of that block before the first attended one (masked)
  int seg_span[LBW_MAX_SEGMENTS];       // keys from the start of block seg_fb to the last attended key
  int seg_blk0[LBW_MAX_SEGMENTS + 1];   // first tile-relative block of each chunk; [n_seg] = nb
  int split0[XCDS_MAX + 1];             // split tiles of XCDs before x (prefix), for the merge grid
};

// Range of tiles of XCD x and its data-parallel / split phases.
struct XcdPlan {
  int t_lo, t_hi, ts;   // tiles [t_lo, t_hi); tiles from ts on are split into pieces
  int64_t units;        // (t_hi - ts) * nb
};

__device__ __forceinline__ XcdPlan xcd_plan(const AttnArgs& a, int x) {
  XcdPlan p;
  p.t_lo = (int)((int64_t)x * a.n_tiles / XCDS);
  p.t_hi = (int)((int64_t)(x + 1) * a.n_tiles / XCDS);
  const int rounds = (p.t_hi - p.t_lo) / a.gx;
  p.ts = p.t_lo + rounds * a.gx;
  p.units = (int64_t)(p.t_hi - p.ts) * a.nb;
  return p;
}

constexpr int S_MASKED = (int)0xFF800000;      // bits of -inf: the int max ignores it, exp2 gives 0
constexpr int E8M0_ONE = 0x7F7F7F7F;           // MFMA block scale 1.0 in every byte
constexpr int E8M0_P16 = 0x83838383;           // 2^4: the residual product's P operand is bf6(P / 16)

// max of a value over the two lane halves (lanes l and l ^ 32 hold the same query)
__device__ __forceinline__ int halves_max_i(int x) {
  auto r = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
  return max((int)r[0], (int)r[1]);
}

// max of 32 ints as a tree of 3-input maxes (v_max3_i32)
__device__ __forceinline__ int max32i(const int* f) {
  int a[11];
#pragma unroll
  for (int i = 0; i < 10; ++i) a[i] = max(max(f[3 * i], f[3 * i + 1]), f[3 * i + 2]);
  a[10] = max(f[30], f[31]);
  const int b0 = max(max(a[0], a[1]), a[2]), b1 = max(max(a[3], a[4]), a[5]);
  const int b2 = max(max(a[6], a[7]), a[8]), b3 = max(a[9], a[10]);
  return max(max(b0, b1), max(b2, b3));
}

// Row sums on the matrix core: one v_mfma_scale_f32_16x16x128_f8f6f4 per block multiplies a ones operand with the
// packed P^T (the 32 x 32 x 64 B operand of the P V products, read as the 16 x 16 x 128 B operand). There, lane l
// holds column l % 16 and lane group l / 16 of K; the groups hold queries 0-15 / 16-31 (key half 0) and 0-15 /
// 16-31 (key half 1). A row m takes ones from groups {0, 2} when m & 4 == 0 and from groups {1, 3} otherwise, so
// the four rows 4 (l / 16) .. + 3 that lane l receives all hold the full key sum of the lane's own query l % 32.
// The ones are e4m3 (0x38): the operand must have P's format, whose K order within a lane it then shares.
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int E4M3_ONES = 0x38383838;
__device__ __forceinline__ v8i rowsum_ones(int lane) {
  const int o = (((lane & 4) != 0) == (((lane >> 4) & 1) != 0)) ? E4M3_ONES : 0;
  const v8i r = {o, o, o, o, o, o, o, o};
  return r;
}

struct Piece {      // online-softmax state of one wave after a range of key blocks
  v16f o[4];        // O^T accumulator, in true V units (the PV MFMAs apply V's block scales)
  float m, l;       // reference max (log2 domain, bias included) and row sum of the rounded P
};

// ---- 8-wave ping-pong attention --------------------------------------------------------------------------
// A workgroup is 8 waves x 32 queries = a 256-query tile. Waves 0-3 (group A) and 4-7 (group B) share the SIMDs
// (one wave of each per SIMD) and run the same per-block program with a phase offset of one barrier: while one
// group issues its MFMAs (S = K Q^T of block j, then P V of block j - 1) the other computes the softmax of its
// block, so the matrix cores and the vector ALUs work at the same time. In its MFMA phase every wave streams
// one piece of each tile of block j + LEAD into LDS with direct global -> LDS loads, through NSTAGE stages;
// group A waits for its pieces at the end of a softmax phase, group B at the end of an MFMA phase (in the fast
// form of the pass both groups wait at both points), so each block has landed before the barrier that opens its
// first MFMA phase. Stage layout (22 KB; the block's scales go to records of their own, below):
// K tile 64 rows x 128 B, V tile 128 channels x 64 B, V residual tile 128 channels x 48 B (bf6 codes, the row layout
// of the re-quant). K and V 16-byte chunks are XOR-swizzled by row (K: chunk ^ ((row >> 1) & 7), V: chunk ^
// ((row >> 2) & 3)) so that the fragment reads of the MFMA operands hit 16 distinct bank groups per 16 lanes, and
// every 1 KB of those tiles is one contiguous DMA of 64 lanes x 16 B. The residual rows need no swizzle: at their
// 48-byte stride the 16-byte reads of 16 consecutive channels cover the 64 banks once, and their 8-byte tails,
// stored swapped in channels with bit 4 set, do the same for 32 channels; each wave moves 768 B (48 lanes x 16 B).
constexpr int AT_WAVES = 8;
constexpr int AT_THREADS = 64 * AT_WAVES;
constexpr int NSTAGE = 6;
constexpr int LEAD = 4;                        // NSTAGE - LEAD >= 2: a stage is free one phase before its reload
constexpr int ST_K = 0, ST_V = 8192, ST_VLO = 16384, ST_BYTES = ST_VLO + V_LO_TILE;
constexpr int VLO_PIECE = V_LO_TILE / AT_WAVES;   // 768 B of the residual tile per wave
static_assert(ST_BYTES % 1024 == 0 && VLO_PIECE == 48 * 16, "stage layout");
static_assert(QT == 32 * AT_WAVES, "query tile");
// Scales of the block in each stage ([stage][wave w][36 B]): wave w's record holds dwords 8 w .. 8 w + 7 of the
// block's V scale table, then the block's K scale (each wave its own copy). Table dword l is the E8M0 block scales
// lane l gives the PV MFMAs (byte mt: channel 32 mt + l % 32, keys 32 (l / 32) .. + 31 of the block -- the MFMA's
// K-block l / 32, bytes 16 (l / 32) .. + 15 of every lane's operand). One 9-lane load per wave and block fills a
// record, with the block's tiles.
constexpr int SC_WAVE = 36, SC_STAGE = AT_WAVES * SC_WAVE;
constexpr int TAB_SC = NSTAGE * ST_BYTES;
// Per-piece chunk table, so a chunk switch inside the loop reads LDS instead of global memory (waiting for a
// global load would also wait for every global -> LDS load in flight):
//   bias  [chunk c][query]    q . mean_k(c) * sm_scale * log2(e) of the tile's queries
constexpr int TAB_BIAS = TAB_SC + NSTAGE * SC_STAGE;
constexpr int AT_LDS = TAB_BIAS + LBW_MAX_SEGMENTS * QT * 4;   // 157376 of the 163840 bytes of a CU
static_assert(AT_LDS <= 163840, "LDS");

// Workgroup barrier that also stops the compiler from moving memory accesses across it. No wait is implied:
// the global -> LDS loads a phase depends on are waited for explicitly by the waves that issued them.
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// s_waitcnt on vmcnt only (lgkmcnt and expcnt at their maxima); vmcnt bits 5:4 sit in bits 15:14.
constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }
__device__ __forceinline__ void wait_vm(int n) {
  switch (n) {   // the counts the block loop uses: multiples of 3 or 4 DMA instructions per block, up to 4 blocks
    case 3: __builtin_amdgcn_s_waitcnt(vmcnt_imm(3)); break;
    case 4: __builtin_amdgcn_s_waitcnt(vmcnt_imm(4)); break;
    case 6: __builtin_amdgcn_s_waitcnt(vmcnt_imm(6)); break;
    case 8: __builtin_amdgcn_s_waitcnt(vmcnt_imm(8)); break;
    case 9: __builtin_amdgcn_s_waitcnt(vmcnt_imm(9)); break;
    case 12: __builtin_amdgcn_s_waitcnt(vmcnt_imm(12)); break;
    case 16: __builtin_amdgcn_s_waitcnt(vmcnt_imm(16)); break;
    default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;   // 0, and anything else: wait for everything
  }
}

// Global -> LDS loads (M0 = the wave's LDS destination; lane i writes M0 + i * size). Written as inline asm on
// purpose: the compiler models the builtin as a FLAT access that may touch LDS, and while one may be pending
// it cannot count LDS reads individually, so every LDS wait in the block loop became lgkmcnt(0), draining all
// fragment reads in flight before each MFMA pair. Hidden from the compiler, the DMA is waited for only by the
// explicit vmcnt waits below (in-order retirement keeps the compiler's own vmcnt waits correct, at worst
// stricter). The s_nop covers the M0-write -> LDS-DMA hazard. M0 is a reserved register the compiler does not
// let inline asm clobber, so the asm saves and restores it.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// The first int8 MFMA of a QK^T accumulation, its accumulator operand the inline constant whose bits are S_MAGIC
// (written as asm: the builtin folds only a zero accumulator into the instruction, any other constant tile is moved
// into 16 registers first). The result then reads as the float S_MAGIC_F + s * 2^-26.
__device__ __forceinline__ v16i mfma_i8_from_magic(v4i a, v4i b) {
  static_assert(S_MAGIC == 0x3E22F983, "the asm below encodes this value");
  v16i d;
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, 0x3e22f983" : "=&v"(d) : "v"(a), "v"(b));
  return d;
}

// A block's loads in one asm, M0 saved once and restored once around them: the K and V tiles, 16 bytes per lane,
// and (with TWO) the V-residual tile, 16 bytes per lane of lanes 0-47 (EXEC narrowed), each a wave-uniform base plus
// a 32-bit per-lane byte offset (the global instruction's scalar-base form: no 64-bit address per lane to form);
// then the wave's scale record by lanes 0-8 from 64-bit per-lane addresses (`sp`: lanes 0-7 this wave's 32 bytes of
// the V scale table, lane 8 the K scale), lane i writing M0 + 4 i. EXEC is restored before the asm ends, so no
// branch.
template <bool TWO>
__device__ __forceinline__ void dma_block(const void* kb, uint32_t koff, const void* vb, const void* vlb, uint32_t voff,
                                          uint32_t vloff, uint64_t sp, uint8_t* lk, uint8_t* lv, uint8_t* lvl,
                                          uint8_t* lsc) {
  uint32_t keep;
  uint64_t ex;
  if (TWO)
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %6\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, %3\n\t"
                 "s_mov_b32 m0, %7\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %4, %5\n\t"
                 "s_mov_b64 %1, exec\n\ts_mov_b32 exec_hi, 0xffff\n\t"
                 "s_mov_b32 m0, %9\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %12, %8\n\t"
                 "s_mov_b64 exec, 0x1ff\n\t"
                 "s_mov_b32 m0, %11\n\ts_nop 0\n\tglobal_load_lds_dword %10, off\n\t"
                 "s_mov_b64 exec, %1\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(keep), "=&s"(ex)
                 : "v"(koff), "s"(kb), "v"(voff), "s"(vb), "s"(lds_addr(lk)), "s"(lds_addr(lv)), "s"(vlb),
                   "s"(lds_addr(lvl)), "v"(sp), "s"(lds_addr(lsc)), "v"(vloff)
                 : "memory");
  else
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %6\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, %3\n\t"
                 "s_mov_b32 m0, %7\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %4, %5\n\t"
                 "s_mov_b64 %1, exec\n\ts_mov_b64 exec, 0x1ff\n\t"
                 "s_mov_b32 m0, %9\n\ts_nop 0\n\tglobal_load_lds_dword %8, off\n\t"
                 "s_mov_b64 exec, %1\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(keep), "=&s"(ex)
                 : "v"(koff), "s"(kb), "v"(voff), "s"(vb), "s"(lds_addr(lk)), "s"(lds_addr(lv)), "v"(sp),
                   "s"(lds_addr(lsc))
                 : "memory");
}

// PV MFMA f of a block: O^T tile f & 3 += V^T fragment times P^T, with V's E8M0 block scales from byte f & 3 of vsc
// (the byte select is an immediate of the instruction). f < 4: the e4m3 hi plane times the e4m3 P, unscaled.
// f >= 4: the residual plane, bf6 x bf6 (both operands 6-bit, so the product runs at twice the fp8 rate: 6 of the
// 8 operand registers are read), times bf6(P / 16) with the B scale 2^4 (a constant operand, so no per-block
// arithmetic on vsc).
template <int F>
__device__ __forceinline__ void pv_mfma(v16f (&o)[4], const v8i& vf, const v8i& pb, const v8i& pb6, int vsc) {
  if constexpr (F < 4)
    o[F & 3] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pb, o[F & 3], 0, 0, F & 3, vsc, 0, E8M0_ONE);
  else
    o[F & 3] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pb6, o[F & 3], 3, 3, F & 3, vsc, 0, E8M0_P16);
}

// Key blocks [j0, j1) of one tile for this wave's 32 queries (first query q0). TWO: V has a residual plane.
// LOGITS (a checking build): each block's raw QK^T accumulator words, S_MAGIC + S, also go to
// logits[bh][q0 + row][64 j + key] (int32 [BH][Lp][nb * 64]) right after the QK MFMAs, before any mask.
template <bool TWO, bool LOGITS>
__device__ __forceinline__ void attend_range(const AttnArgs& a, const int8_t* __restrict__ q8,
                                             const float* __restrict__ q_scale, const float* __restrict__ bias,
                                             const int8_t* __restrict__ k8, const float* __restrict__ k_scale,
                                             const uint8_t* __restrict__ v8, const uint8_t* __restrict__ v8lo,
                                             const uint8_t* __restrict__ v_scale, uint8_t* lds, int bh, int64_t q0,
                                             int j0, int j1, Piece& st, int32_t* __restrict__ logits) {
  constexpr int NPB = TWO ? 4 : 3;   // DMA instructions per block of each wave (tiles, then the scale record)
  const int t = threadIdx.x, lane = t & 63, lq = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);   // wave-uniform, so the loader's control stays scalar
  const bool grp_a = w < 4;
  const int n = j1 - j0;
  v4i qf[4];
  {
    const int8_t* qrow = q8 + ((int64_t)bh * a.lp + q0 + lq) * D + 64 * g;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[kk] = *(const v4i*)(qrow + 16 * kk);
  }
  // the logit scale per unit of the accumulator's float reading (2^-26 per integer step; exact power-of-2 factor)
  const float qs_sl2 = q_scale[(int64_t)bh * (a.lp / QG) + (q0 >> 5)] * a.sl2 * S_MAGIC_INV_ULP;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) st.o[mt][i] = 0.f;
  float m_ref = -INFINITY;
  v4f l_run = {0.f, 0.f, 0.f, 0.f};      // row sum of the rounded P (all four words equal)
  const v8i ones = rowsum_ones(lane);
  const bool multi = a.n_seg > 1;

  // fragment read offsets in a stage (K: chunk 4g + kk of row 32 mt + lq; V: chunks 2g, 2g + 1 of row 32 mt + lq;
  // V residual: half g's 16-byte piece and its 8-byte tail in row 32 mt + lq). The tails of odd mt have a base
  // register of their own: the fragments mt, mt + 1 are read together, and two 8-byte reads from one base would be
  // merged into one two-address read, whose 4-register result then takes moves to form each fragment's 6
  // contiguous operand registers.
  int kro[4], vro[2], lro[3];
  {
    const int s1 = (lq >> 1) & 7, s2 = (lq >> 2) & 3;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) kro[kk] = lq * 128 + (((4 * g + kk) ^ s1) << 4);
#pragma unroll
    for (int h = 0; h < 2; ++h) vro[h] = ST_V + lq * 64 + (((2 * g + h) ^ s2) << 4);
    lro[0] = ST_VLO + lq * V_LO_ROW + 16 * g;
    lro[1] = ST_VLO + lq * V_LO_ROW + 32 + 8 * (g ^ ((lq >> 4) & 1));
    lro[2] = lro[1] + 32 * V_LO_ROW;
    asm volatile("" : "+v"(lro[2]));   // opaque: not folded back into lro[1] + offset
  }

  // loader: wave w moves 1 KB piece w of each 8 KB tile (K, V) and 768 B piece w of the 6 KB V residual tile
  int koff, voff;
  const int vloff = VLO_PIECE * w + 16 * lane;   // lanes 0-47 load
  {
    const int kr = 8 * w + (lane >> 3), vr = 16 * w + (lane >> 2);
    koff = kr * 128 + (((lane & 7) ^ ((kr >> 1) & 7)) << 4);
    voff = vr * 64 + (((lane & 3) ^ ((vr >> 2) & 3)) << 4);
  }
  // chunk lengths are only read when a cursor enters a chunk: an indexed read of the arguments is a memory load,
  // and waiting for it would also wait for every global -> LDS load in flight
  int lc = 0;
  while (j0 >= a.seg_blk0[lc + 1]) ++lc;
  int lrem = a.seg_blk0[lc + 1] - j0;   // blocks the loader has left in chunk lc
  const int lb = j0 - a.seg_blk0[lc];
  const int8_t* kbase;
  const uint8_t* vbase;
  const uint8_t* vlbase;
  // this lane's scale dword of the block (lanes 0-7: V scale table bytes 32 w + 4 lane ..; lane 8: the K scale; the
  // other lanes load nothing) and its step to the next block of a chunk
  uint64_t sptr;
  const uint32_t sstep = lane < 8 ? 256u : 4u;
  auto seek = [&](int cc, int bb) {   // block bb of chunk cc's range, i.e. slot block seg_fb[cc] + bb
    const int64_t sbh = (int64_t)a.seg_slot[cc] * a.bh + bh;
    const int64_t blk = (int64_t)bb + a.seg_fb[cc];
    kbase = k8 + (sbh * a.cap + blk * KB) * D;
    vbase = v8 + (sbh * a.nbc + blk) * TILE_BYTES;
    if (TWO) vlbase = v8lo + (sbh * a.nbc + blk) * V_LO_TILE;
    sptr = lane < 8 ? (uint64_t)(uintptr_t)(v_scale + (sbh * a.nbc + blk) * 256 + w * 32 + 4 * lane)
                    : (uint64_t)(uintptr_t)(k_scale + sbh * a.nbc + blk);
  };
  seek(lc, lb);
  auto issue = [&](int stage) {
    uint8_t* sb = lds + stage * ST_BYTES;
    dma_block<TWO>(kbase, (uint32_t)koff, vbase, TWO ? (const void*)vlbase : nullptr, (uint32_t)voff,
                   (uint32_t)vloff, sptr, sb + ST_K + w * 1024, sb + ST_V + w * 1024, sb + ST_VLO + w * VLO_PIECE,
                   lds + TAB_SC + stage * SC_STAGE + w * SC_WAVE);
  };
  auto advance = [&](auto fast) {   // fast: the next block is in the same chunk (lrem >= 2)
    if (!decltype(fast)::value && --lrem == 0) {   // the fast form's steps are taken off lrem after the run
      ++lc;
      if (lc < a.n_seg) {
        seek(lc, 0);
        lrem = a.seg_blk0[lc + 1] - a.seg_blk0[lc];
      }
    } else {
      kbase += TILE_BYTES;
      vbase += TILE_BYTES;
      if (TWO) vlbase += V_LO_TILE;
      sptr += sstep;
    }
  };

  // compute cursor: chunk c of the block in the softmax and the blocks it has left
  int c = 0;
  while (j0 >= a.seg_blk0[c + 1]) ++c;
  int crem = a.seg_blk0[c + 1] - j0;                   // blocks left in chunk c, this one included
  int last_valid = a.seg_span[c] - (a.seg_blk0[c + 1] - a.seg_blk0[c] - 1) * KB;   // keys in its last block
  int lead = j0 == a.seg_blk0[c] ? a.seg_lead[c] : 0;  // leading keys of this block outside chunk c's range
  int c_prev = c;
  int jd = j0;                                         // LOGITS: tile-relative block of the softmax phase

  // chunk table: its global loads go out before the first blocks' DMA, so waiting for them waits for nothing
  // else. The previous piece's readers are done: it ended with a workgroup barrier.
  float* const bias_tab = (float*)(lds + TAB_BIAS) + 32 * w + lq;   // this lane's query; [c * QT]
  float tb[LBW_MAX_SEGMENTS];
  if (multi) {
#pragma unroll
    for (int cc = 0; cc < LBW_MAX_SEGMENTS; ++cc)
      if (cc < a.n_seg) tb[cc] = bias[((int64_t)cc * a.bh + bh) * a.lp + q0 + lq];
  }

  const int npre = n < LEAD ? n : LEAD;
  for (int i = 0; i < npre; ++i) {
    issue(i);
    advance(std::false_type{});
  }
  float beta = 0.f;
  if (multi) {
    wait_vm(NPB * npre);   // the table loads (older than every DMA) have landed
#pragma unroll
    for (int cc = 0; cc < LBW_MAX_SEGMENTS; ++cc)
      if (cc < a.n_seg) bias_tab[cc * QT] = tb[cc] * a.sl2;
    beta = tb[0];
#pragma unroll
    for (int cc = 1; cc < LBW_MAX_SEGMENTS; ++cc)
      if (cc == c) beta = tb[cc];
    beta *= a.sl2;
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the table writes are done before the barrier below
  }
  // per-row values that change only with m_ref or beta: the rescale threshold and the exponent's offset
  float thr = m_ref + RESCALE_SLACK;
  float tk = beta - m_ref + (P_OFFSET - RESCALE_SLACK);
  wait_vm(NPB * (npre - 1));   // every wave's piece of the first block has landed
  int ldstage = npre % NSTAGE;
  phase_barrier();
  if (!grp_a) phase_barrier();   // group B runs one phase behind

  v8i pb = {0, 0, 0, 0, 0, 0, 0, 0};    // P^T as e4m3 bytes
  v8i pb6 = {0, 0, 0, 0, 0, 0, 0, 0};   // the same keys as bf6(P / 16) codes (TWO; registers 6 and 7 unused)
  int stage = 0, pstage = 0;
  int it = 0;
  // One pass: the MFMA phase of block it and the softmax phase of block it. The fast form assumes what holds for
  // most passes: the loader's block it + LEAD exists and lies in the loader's current chunk, and block it is
  // neither the first nor the last block of its chunk (so no new logit bias, no key mask, no chunk step). It
  // returns true after the last MFMA phase (it == n).
  auto pass = [&](auto fast) -> bool {
    constexpr bool FAST = decltype(fast)::value;
    // ---- MFMA phase: S of block it, P V of block it - 1 ----
    // (wave priorities stay equal: raising this phase's cost 0.3 % of kernel time, raising the softmax phase's 0.2 %)
    // LDS reads run ahead of the MFMAs that consume them: all eight K fragments and the first two V fragments
    // are requested before the first QK MFMA, and each later pair of V fragments before the MFMA pair ahead of
    // its consumers. The scheduling fences keep the compiler from sinking the reads next to their uses, which
    // would expose the LDS latency once per MFMA.
    v16i acc[2];
    const uint8_t* sk = lds + stage * ST_BYTES;
    const uint8_t* sv = lds + pstage * ST_BYTES;
    constexpr int NVF = TWO ? 8 : 4;   // V fragments (one per PV MFMA): hi plane mt 0..3, then lo plane mt 0..3
    auto vfrag = [&](int f) {
      if (f >= 4) {   // 32 bf6 codes: 16 + 8 bytes (operand registers 6 and 7 are not read)
        const int off = (f & 3) * 32 * V_LO_ROW;
        const v4i a = *(const v4i*)(sv + lro[0] + off);
        const v2i b = *(const v2i*)(sv + ((f & 1) ? lro[2] + (off - 32 * V_LO_ROW) : lro[1] + off));
        const v8i r = {a[0], a[1], a[2], a[3], b[0], b[1], 0, 0};
        return r;
      }
      const int off = (f & 3) * 2048;
      const v4i lo = *(const v4i*)(sv + vro[0] + off);
      const v4i hi = *(const v4i*)(sv + vro[1] + off);
      const v8i r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      return r;
    };
    // V's block scales: this lane's dword of block it - 1's table (read below); byte mt scales the rows of O^T
    // tile mt (A operand row l % 32 in K-block l / 32).
    int vsc;
    auto pv = [&](int f, const v8i& vf) {   // f is a constant once the loop below is unrolled
      switch (f) {
        case 0: pv_mfma<0>(st.o, vf, pb, pb6, vsc); break;
        case 1: pv_mfma<1>(st.o, vf, pb, pb6, vsc); break;
        case 2: pv_mfma<2>(st.o, vf, pb, pb6, vsc); break;
        case 3: pv_mfma<3>(st.o, vf, pb, pb6, vsc); break;
        case 4: pv_mfma<4>(st.o, vf, pb, pb6, vsc); break;
        case 5: pv_mfma<5>(st.o, vf, pb, pb6, vsc); break;
        case 6: pv_mfma<6>(st.o, vf, pb, pb6, vsc); break;
        default: pv_mfma<7>(st.o, vf, pb, pb6, vsc); break;
      }
    };
    // Both halves run on every pass, so the LDS waits need no control-flow joins: at it == n the QK MFMAs read
    // a stage nothing uses (its int32 results are dropped), and at it == 0 P is all zeros, so the PV MFMAs add
    // exactly 0 (stage 0 holds block 0, whose fp8 V values are finite).
    constexpr bool do_qk = true, do_pv = true;
    // Nothing is outstanding on the LDS / scalar counter here in the common case; saying so lets the waits
    // below count individual LDS reads (a scalar load that might still be pending forces every wait to zero).
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0), vmcnt and expcnt unconstrained
    v4i kf[8];
    v8i vq[2];
    if (do_qk) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        kf[2 * kk] = *(const v4i*)(sk + kro[kk]);
        kf[2 * kk + 1] = *(const v4i*)(sk + kro[kk] + 4096);
      }
    }
    // the K scale of block it, for its softmax in the next phase (this wave's copy landed with its pieces)
    const float ks = *(const float*)(lds + TAB_SC + stage * SC_STAGE + w * SC_WAVE + 32);
    vsc = *(const int*)(lds + TAB_SC + pstage * SC_STAGE + (lane >> 3) * SC_WAVE + 4 * (lane & 7));
    if (do_pv) {
      vq[0] = vfrag(0);
      vq[1] = vfrag(1);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (do_qk) {
      acc[0] = mfma_i8_from_magic(kf[0], qf[0]);
      acc[1] = mfma_i8_from_magic(kf[1], qf[0]);
    }
    __builtin_amdgcn_sched_barrier(0);
    // DMA of block it + LEAD into the stage of block it - 2 (both groups finished it a phase ago): in the MFMA
    // phase, where the wave mostly waits for the matrix core (the softmax phase slows down with it), and after
    // the first two QK MFMAs, so the matrix core starts at once and the issue hides under their execution
    // (-1 to -2 % against issuing it before them, same-box A/B)
    if (FAST || it + LEAD < n) {
      issue(ldstage);
      advance(fast);
      ldstage = ldstage + 1 == NSTAGE ? 0 : ldstage + 1;
    }
    __builtin_amdgcn_sched_barrier(0);
    if (do_qk) {
#pragma unroll
      for (int kk = 1; kk < 4; ++kk) {
        acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[2 * kk], qf[kk], acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[2 * kk + 1], qf[kk], acc[1], 0, 0, 0);
      }
      // MFMAs are pure register operations: without this the compiler sinks them below the phase barrier,
      // next to their first use in the softmax, and the two halves' MFMA and softmax phases no longer alternate
      asm volatile("" : "+v"(acc[0]), "+v"(acc[1]));
    }
    if (do_pv) {
#pragma unroll
      for (int f = 0; f < NVF; f += 2) {
        v8i nx[2];
        if (f + 2 < NVF) {
          nx[0] = vfrag(f + 2);
          nx[1] = vfrag(f + 3);
        }
        __builtin_amdgcn_sched_barrier(0);
        pv(f, vq[0]);
        pv(f + 1, vq[1]);
        __builtin_amdgcn_sched_barrier(0);
        if (f + 2 < NVF) {
          vq[0] = nx[0];
          vq[1] = nx[1];
        }
      }
      // the row sums of block it - 1's rounded P, after the P V products (at the phase start, ahead of the QK
      // products, it delayed them: the matrix core would not start the first QK product any earlier)
      l_run = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ones, pb, l_run, 0, 0, 0, E8M0_ONE, 0, E8M0_ONE);
      asm volatile("" : "+v"(st.o[0]), "+v"(st.o[1]), "+v"(st.o[2]), "+v"(st.o[3]), "+v"(l_run));   // as for acc
    }
    if (!FAST && it == n) return true;
    // B's pieces of block it + 1 have landed before A starts on it (it + 2 .. it + LEAD in flight). The fast
    // form waits in both groups (no branch): A's pieces of block it + 1 were issued LEAD - 1 passes ago, and A
    // needs them by the end of this pass anyway.
    if (FAST || !grp_a) {
      if (FAST || it + LEAD < n) {   // steady state as one constant wait (a general count is a chain of branches)
        wait_vm(NPB * (LEAD - 1));
      } else {
        const int ahead = n - 1 - (it + 1);
        wait_vm(ahead > 0 ? NPB * ahead : 0);
      }
    }
    phase_barrier();

    // ---- softmax phase for block it (chunk c) ----
    if (!FAST && c != c_prev) {
      // a new chunk (c_prev == c - 1: every chunk has a block): its logit bias from the piece's LDS table (O is in
      // true V units, so it carries over unchanged)
      beta = bias_tab[c * QT];
      tk = beta - m_ref + (P_OFFSET - RESCALE_SLACK);
      c_prev = c;
    }
    const float cb = qs_sl2 * ks;
    int si[32];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) si[16 * mt + i] = acc[mt][i];
    if constexpr (LOGITS) {   // the raw accumulator words of block jd, then nothing left in flight but the DMA
      int32_t* lrow = logits + ((int64_t)bh * a.lp + q0 + lq) * ((int64_t)a.nb * KB) + (int64_t)jd * KB + 4 * g;
#pragma unroll
      for (int i = 0; i < 32; ++i) lrow[32 * (i >> 4) + 8 * ((i >> 2) & 3) + (i & 3)] = si[i];
      wait_vm(0);
      ++jd;
    }
    const int valid = FAST || crem != 1 ? KB : last_valid;   // keys of this block that exist (>= 1)
    if (!FAST && (valid < KB || lead > 0)) {
      // key 32 mt + 8 (i >> 2) + 4 g + (i & 3) is past the end iff its lane-independent part reaches vt, and
      // before the chunk's first attended key iff that part is below lt
      const int vt = valid - 4 * g, lt = lead - 4 * g;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int kk = 32 * (i >> 4) + 8 * ((i >> 2) & 3) + (i & 3);
        if (kk >= vt || kk < lt) si[i] = S_MASKED;
      }
    }
    if (!FAST) lead = 0;
    // reference max: moves only when this block's max exceeds it by more than RESCALE_SLACK
    const int mx = halves_max_i(max32i(si));
    const float m_blk = (__int_as_float(mx) - S_MAGIC_F) * cb + beta;
    const bool moved = m_blk > thr;
    if (__builtin_expect(__any(moved), 0)) {   // wave-uniform and rare
      const float m_new = moved ? m_blk : m_ref;
      const float alpha = __builtin_amdgcn_exp2f(m_ref - m_new);
      l_run *= alpha;   // the row sums through block it - 1, like O
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) st.o[mt][i] *= alpha;
      m_ref = m_new;
      thr = m_ref + RESCALE_SLACK;
      tk = beta - m_ref + (P_OFFSET - RESCALE_SLACK);
    }
    const float kc = tk - S_MAGIC_F * cb;
    // p_i = exp2(S_i * cb + kc), i = 0..31, held as pe[k] = p_2k and po[k] = p_2k+1: the operand order of the bf6
    // conversion below, so neither packing needs a register move.
    v16f pe, po;
#pragma unroll
    for (int k2 = 0; k2 < 16; ++k2) {
      pe[k2] = __builtin_amdgcn_exp2f(fmaf(__int_as_float(si[2 * k2]), cb, kc));
      po[k2] = __builtin_amdgcn_exp2f(fmaf(__int_as_float(si[2 * k2 + 1]), cb, kc));
    }
    // P^T B operand: byte 16 mt' + 4 i + j of this lane = p_(16 mt' + 4 i + j) (keys 32 mt' + 8 i + 4 g + j).
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      // both halves of the word are written, so the previous word serves as the "old" operand (no zeroing move)
      int wd = __builtin_amdgcn_cvt_pk_fp8_f32(pe[2 * r], po[2 * r], pb[r], false);
      wd = __builtin_amdgcn_cvt_pk_fp8_f32(pe[2 * r + 1], po[2 * r + 1], wd, true);
      pb[r] = wd;
    }
    if constexpr (TWO) {
      // The residual product's operand, bf6(p / 16): code c of this lane is first the key of byte c of pb. A lane
      // of the 6-bit operand holds one whole K-block (lane half g: K-block g, the keys of V scale group g), where an
      // fp8 lane holds 16 values of each: so the lower half's codes 16-31 (dwords 3-5) and the upper half's codes
      // 0-15 (dwords 0-2) trade places across the halves. Lane half g then holds positions 16 g .. 16 g + 15 and
      // 32 + 16 g .. 47 + 16 g, in the code order of the residual plane's rows.
      const v6i c6 = cvt_bf6_x32(pe, po, P_LO_SCALE);
#pragma unroll
      for (int r = 0; r < 3; ++r) {
        const auto sw = __builtin_amdgcn_permlane32_swap((unsigned)c6[r], (unsigned)c6[r + 3], false, false);
        pb6[r] = (int)sw[0];
        pb6[r + 3] = (int)sw[1];
      }
    }
    // next block of the compute cursor
    if (!FAST && --crem == 0 && c + 1 < a.n_seg) {   // the fast form's steps are taken off crem after the run
      ++c;
      crem = a.seg_blk0[c + 1] - a.seg_blk0[c];
      last_valid = a.seg_span[c] - (crem - 1) * KB;
      lead = a.seg_lead[c];
    }
    if (FAST || grp_a) {   // A's pieces of block it + 1 have landed (blocks up to it + LEAD may still be in flight)
      if (FAST || it + LEAD < n) {   // steady state as one constant wait (a general count is a chain of branches)
        wait_vm(NPB * (LEAD - 1));
      } else {
        const int ahead = n - 1 - (it + 1);
        wait_vm(ahead > 0 ? NPB * ahead : 0);
      }
    }
    phase_barrier();
    pstage = stage;
    stage = stage + 1 == NSTAGE ? 0 : stage + 1;
    if (!FAST) ++it;
    return false;
  };
  for (;;) {
    // passes from here on that take the fast form: the loader stays in its chunk for f more blocks, block it is
    // not its chunk's first (c == c_prev) nor a block with masked leading keys, none of the f blocks is its
    // chunk's last, and block it + f - 1 + LEAD still exists
    int f = (lrem < crem ? lrem : crem) - 1;
    if (n - LEAD - it < f) f = n - LEAD - it;
    if (c != c_prev || lead > 0) f = 0;
    if (f > 0) {
      for (int i = 0; i < f; ++i) pass(std::true_type{});
      it += f;
      lrem -= f;
      crem -= f;
    }
    if (pass(std::false_type{})) break;
  }
  if (grp_a) phase_barrier();   // matches group B's extra barrier at the start
  phase_barrier();               // every wave is done with the stages before they are refilled
  st.m = m_ref;
  st.l = l_run[0];
}

// Whole tile: O = o / l as bf16; lane (query lq) writes channels 32 mt + 8 i + 4 g + (0..3).
__device__ __forceinline__ void store_out(const AttnArgs& a, const Piece& st, uint16_t* __restrict__ out, int bh,
                                          int64_t q0) {
  const int lane = threadIdx.x & 63, lq = lane & 31, g = lane >> 5;
  const int64_t qrow = q0 + lq;
  if (qrow >= a.lq) return;
  const float inv_l = 1.f / st.l;
  const int64_t b = bh / a.heads, h = bh % a.heads;
  uint16_t* op = out + b * a.o_sb + qrow * a.o_st + h * a.o_sh;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = 32 * mt + 8 * i + 4 * g;
      const uint32_t w0 = f32_to_bf16_bits(st.o[mt][4 * i] * inv_l) |
                          ((uint32_t)f32_to_bf16_bits(st.o[mt][4 * i + 1] * inv_l) << 16);
      const uint32_t w1 = f32_to_bf16_bits(st.o[mt][4 * i + 2] * inv_l) |
                          ((uint32_t)f32_to_bf16_bits(st.o[mt][4 * i + 3] * inv_l) << 16);
      *(uint2*)(op + ch) = make_uint2(w0, w1);
    }
}

// Part of a tile: o (unnormalised) and (m, l) per row into workspace slot (g, slot).
__device__ __forceinline__ void store_part(const Piece& st, float* __restrict__ o_part, float* __restrict__ ml_part,
                                           int64_t slot_idx, int w) {
  const int lane = threadIdx.x & 63, lq = lane & 31, g = lane >> 5;
  const int row = w * 32 + lq;
  float* op = o_part + (slot_idx * QT + row) * D;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = 32 * mt + 8 * i + 4 * g;
      *(float4*)(op + ch) = make_float4(st.o[mt][4 * i], st.o[mt][4 * i + 1], st.o[mt][4 * i + 2],
                                        st.o[mt][4 * i + 3]);
    }
  if (g == 0) *(float2*)(ml_part + (slot_idx * QT + row) * 2) = make_float2(st.m, st.l);
}

template <bool TWO, bool LOGITS>
__global__ __launch_bounds__(AT_THREADS, 1) void attn_fwd_kernel(const int8_t* __restrict__ q8,
                                                                 const float* __restrict__ q_scale,
                                                                 const float* __restrict__ bias,
                                                                 const int8_t* __restrict__ k8,
                                                                 const float* __restrict__ k_scale,
                                                                 const uint8_t* __restrict__ v8,
                                                                 const uint8_t* __restrict__ v8lo,
                                                                 const uint8_t* __restrict__ v_scale,
                                                                 uint16_t* __restrict__ out, float* __restrict__ o_part,
                                                                 float* __restrict__ ml_part, int32_t* __restrict__ logits,
                                                                 AttnArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[AT_LDS];
  const int gid = blockIdx.x, x = gid % XCDS, i = gid / XCDS;
  const int w = threadIdx.x >> 6;
  const XcdPlan p = xcd_plan(a, x);
  Piece st;
  // whole tiles, dealt round-robin among this XCD's workgroups
  for (int tile = p.t_lo + i; tile < p.ts; tile += a.gx) {
    const int bh = tile / a.q_tiles;
    const int64_t q0 = (int64_t)(tile % a.q_tiles) * QT + w * 32;
    attend_range<TWO, LOGITS>(a, q8, q_scale, bias, k8, k_scale, v8, v8lo, v_scale, lds, bh, q0, 0, a.nb, st, logits);
    store_out(a, st, out, bh, q0);
  }
  // this workgroup's piece of the split tiles
  if (p.units == 0) return;
  const int64_t u0 = (int64_t)i * p.units / a.gx, u1 = (int64_t)(i + 1) * p.units / a.gx;
  const int first_tile = p.ts + (int)(u0 / a.nb);
  for (int64_t u = u0; u < u1;) {
    const int tile = p.ts + (int)(u / a.nb);
    const int j0 = (int)(u % a.nb);
    const int j1 = (int)((u1 - u + j0 < a.nb) ? (u1 - u + j0) : a.nb);
    const int bh = tile / a.q_tiles;
    const int64_t q0 = (int64_t)(tile % a.q_tiles) * QT + w * 32;
    attend_range<TWO, LOGITS>(a, q8, q_scale, bias, k8, k_scale, v8, v8lo, v_scale, lds, bh, q0, j0, j1, st, logits);
    if (j0 == 0 && j1 == a.nb) {
      store_out(a, st, out, bh, q0);
    } else {
      store_part(st, o_part, ml_part, (int64_t)gid * 2 + (tile == first_tile ? 0 : 1), w);
    }
    u += j1 - j0;
  }
}

// Combine the pieces of each split tile: O = sum 2^(m_i - M) o_i / sum 2^(m_i - M) l_i
// (experiments/bench_attn/splitkv/README.md:62). Grid: (split tile, 16-row slab) -- only split tiles are
// launched; 256 threads = 16 rows x 16 lanes, each lane 8 consecutive channels, so a row's 512-byte partial is
// read by 16 consecutive lanes.
constexpr int MERGE_ROWS = 16;
__global__ __launch_bounds__(256) void attn_merge_kernel(const float* __restrict__ o_part,
                                                         const float* __restrict__ ml_part,
                                                         uint16_t* __restrict__ out, AttnArgs a) {
  const int st = blockIdx.x / (QT / MERGE_ROWS), slab = blockIdx.x % (QT / MERGE_ROWS);
  int x = 0;
  while (x + 1 < XCDS && st >= a.split0[x + 1]) ++x;
  const XcdPlan p = xcd_plan(a, x);
  const int tile = p.ts + (st - a.split0[x]);
  const int64_t ua = (int64_t)(tile - p.ts) * a.nb, ub = ua + a.nb;
  // workgroups of this XCD whose unit range meets [ua, ub): owner(u) = floor(((u + 1) gx - 1) / units)
  const int i_a = (int)(((ua + 1) * a.gx - 1) / p.units);
  const int i_b = (int)((ub * a.gx - 1) / p.units);
  // workgroup i's units are [floor(i units / gx), floor((i + 1) units / gx)): stepped from i_a with the quotient
  // and remainder of units / gx, so the loops below divide nothing (64-bit divisions are long instruction
  // sequences, and this kernel is short)
  const int64_t uq = p.units / a.gx;
  const int ur = (int)(p.units % a.gx);
  const int64_t lo_a = (int64_t)i_a * uq + (int64_t)i_a * ur / a.gx;
  const int rem_a = (int)((int64_t)i_a * ur % a.gx);
  const int64_t hi_a = lo_a + uq + (rem_a + ur >= a.gx ? 1 : 0);
  if (i_a == i_b && lo_a <= ua && hi_a >= ub) return;   // written whole by one workgroup
  const int t = threadIdx.x, row = slab * MERGE_ROWS + (t >> 4), c0 = (t & 15) * 8;
  const int64_t q = (int64_t)(tile % a.q_tiles) * QT + row;
  if (q >= a.lq) return;
  // a piece of workgroup ii that meets this tile is in its partial slot 0 when the tile is the first of
  // the workgroup's range, i.e. when the piece starts inside the tile, else in slot 1
  // The loads do not depend on whether workgroup ii's range meets the tile (every slot index stays inside the
  // workspace, ii < gx), so they are issued unconditionally and unrolled to keep several in flight; a slot of a
  // workgroup with no units here is read but not used (select, not multiply: it may hold anything).
  float mmax = -INFINITY;
  {
    int64_t lo = lo_a;
    int rem = rem_a;
#pragma unroll 8
    for (int ii = i_a; ii <= i_b; ++ii) {
      const bool carry = rem + ur >= a.gx;
      const int64_t hi = lo + uq + (carry ? 1 : 0);
      rem += ur - (carry ? a.gx : 0);
      const int64_t slot = (int64_t)(ii * XCDS + x) * 2 + (lo >= ua ? 0 : 1);
      const float m = ml_part[(slot * QT + row) * 2];
      if (hi > lo && hi > ua && lo < ub) mmax = fmaxf(mmax, m);   // units of this tile
      lo = hi;
    }
  }
  float acc[8], den = 0.f;
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = 0.f;
  int64_t lo = lo_a;
  int rem = rem_a;
#pragma unroll 8
  for (int ii = i_a; ii <= i_b; ++ii) {
    const bool carry = rem + ur >= a.gx;
    const int64_t hi = lo + uq + (carry ? 1 : 0);
    rem += ur - (carry ? a.gx : 0);
    const int64_t plo = lo;
    lo = hi;
    const int64_t slot = (int64_t)(ii * XCDS + x) * 2 + (plo >= ua ? 0 : 1);
    const float2 ml = *(const float2*)(ml_part + (slot * QT + row) * 2);
    const float* op = o_part + (slot * QT + row) * D + c0;
    const float4 v0 = *(const float4*)op, v1 = *(const float4*)(op + 4);
    if (hi > plo && hi > ua && plo < ub) {
      const float wgt = __builtin_amdgcn_exp2f(ml.x - mmax);
      den += wgt * ml.y;
      acc[0] += wgt * v0.x; acc[1] += wgt * v0.y; acc[2] += wgt * v0.z; acc[3] += wgt * v0.w;
      acc[4] += wgt * v1.x; acc[5] += wgt * v1.y; acc[6] += wgt * v1.z; acc[7] += wgt * v1.w;
    }
  }
  const float inv = 1.f / den;
  const int bh = tile / a.q_tiles;
  const int64_t b = bh / a.heads, h = bh % a.heads;
  uint16_t* dst = out + b * a.o_sb + q * a.o_st + h * a.o_sh + c0;
  uint32_t w[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    w[c] = f32_to_bf16_bits(acc[2 * c] * inv) | ((uint32_t)f32_to_bf16_bits(acc[2 * c + 1] * inv) << 16);
  *(uint2*)dst = make_uint2(w[0], w[1]);        // the output contract guarantees 8-byte alignment
  *(uint2*)(dst + 4) = make_uint2(w[2], w[3]);
}

// Persistent workgroups per XCD: one per CU (a workgroup is 8 waves, two per SIMD, and uses AT_LDS bytes of the
// CU's 160 KB of LDS). Cached per device ordinal; atomic, since entry points may run on several host threads.
static int attn_wgs_per_xcd() {
  static std::atomic<int> cached[64];   // 0 unknown (static storage: zero-initialised)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 32;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    v = (cus + XCDS - 1) / XCDS;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

}  // namespace lbw

using namespace lbw;

extern "C" int lbw_attn_workgroups_per_xcd(void) { return attn_wgs_per_xcd(); }

extern "C" int64_t lbw_attn_workspace_bytes(void) {
  const int64_t gx = attn_wgs_per_xcd();
  return (int64_t)XCDS * gx * 2 * QT * (D + 2) * (int64_t)sizeof(float);
}

// The checks and launches of lbw_attn_fwd; with `logits` not null the checking build of the kernel also writes
// every block's raw QK^T accumulator words there.
static int attn_launch(const int8_t* q8, const float* q_scale, const float* bias, int64_t batch, int64_t lq,
                       int64_t heads, const int8_t* k8, const float* k_scale, const uint8_t* v8, const uint8_t* v8lo,
                       const uint8_t* v_scale, int64_t slots, int64_t cap, int n_seg, const int32_t* seg_slot,
                       const int32_t* seg_len, const int32_t* seg_first, uint16_t* out, int64_t o_s_batch,
                       int64_t o_s_tok, int64_t o_s_head, float sm_scale, int32_t* logits, void* workspace,
                       void* stream) {
  if (!q8 || !q_scale || !k8 || !k_scale || !v8 || !v_scale || !out || !seg_slot || !seg_len || !workspace)
    return LBW_E_NULL;
  if (batch <= 0 || heads <= 0 || lq <= 0 || slots <= 0 || cap <= 0 || cap % KB) return LBW_E_SHAPE;
  if (batch * heads > 65535 || !(sm_scale > 0.f) || lq > ((int64_t)1 << 30)) return LBW_E_SHAPE;
  if (n_seg < 1 || n_seg > LBW_MAX_SEGMENTS) return LBW_E_SEGMENTS;
  if (n_seg > 1 && !bias) return LBW_E_NULL;
  if (o_s_batch % 4 || o_s_tok % 4 || o_s_head % 4) return LBW_E_ALIGN;
  if (((uintptr_t)q8 | (uintptr_t)k8 | (uintptr_t)v8 | (uintptr_t)v8lo | (uintptr_t)workspace) & 15 ||
      ((uintptr_t)out & 7) || (((uintptr_t)logits | (uintptr_t)v_scale) & 3))
    return LBW_E_ALIGN;
  AttnArgs a;
  a.lq = lq;
  a.lp = (lq + QT - 1) / QT * QT;
  a.bh = batch * heads;
  a.heads = heads;
  a.cap = cap;
  a.nbc = cap / KB;
  a.o_sb = o_s_batch; a.o_st = o_s_tok; a.o_sh = o_s_head;
  a.sl2 = sm_scale * 1.4426950408889634f;
  a.n_seg = n_seg;
  int nb = 0;
  for (int c = 0; c <= LBW_MAX_SEGMENTS; ++c) a.seg_blk0[c] = 0;
  for (int c = 0; c < LBW_MAX_SEGMENTS; ++c) a.seg_slot[c] = a.seg_fb[c] = a.seg_lead[c] = a.seg_span[c] = 0;
  for (int c = 0; c < n_seg; ++c) {
    const int first = seg_first ? seg_first[c] : 0;
    if (seg_slot[c] < 0 || seg_slot[c] >= slots || seg_len[c] < 1 || first < 0 || seg_len[c] > cap - first)
      return LBW_E_SEGMENTS;
    a.seg_slot[c] = seg_slot[c];
    a.seg_fb[c] = first / KB;
    a.seg_lead[c] = first % KB;
    a.seg_span[c] = first % KB + seg_len[c];
    a.seg_blk0[c] = nb;
    nb += (a.seg_span[c] + KB - 1) / KB;
  }
  for (int c = n_seg; c <= LBW_MAX_SEGMENTS; ++c) a.seg_blk0[c] = nb;
  a.nb = nb;
  a.q_tiles = (int)(a.lp / QT);
  if ((int64_t)a.q_tiles * a.bh > 0x7fffffff / 2) return LBW_E_SHAPE;
  a.n_tiles = (int)(a.q_tiles * a.bh);
  if (const int dv = check_device()) return dv;
  a.gx = attn_wgs_per_xcd();
  a.split0[0] = 0;
  for (int x = 0; x < XCDS; ++x) {   // tiles past the whole-tile rounds of each XCD are split (xcd_plan)
    const int t_lo = (int)((int64_t)x * a.n_tiles / XCDS), t_hi = (int)((int64_t)(x + 1) * a.n_tiles / XCDS);
    a.split0[x + 1] = a.split0[x] + (t_hi - t_lo) % a.gx;
  }
  float* o_part = (float*)workspace;
  float* ml_part = o_part + (int64_t)XCDS * a.gx * 2 * QT * D;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)(XCDS * a.gx)), block(AT_THREADS);
  if (v8lo && logits)
    hipLaunchKernelGGL((attn_fwd_kernel<true, true>), grid, block, 0, st, q8, q_scale, bias, k8, k_scale, v8, v8lo,
                       v_scale, out, o_part, ml_part, logits, a);
  else if (v8lo)
    hipLaunchKernelGGL((attn_fwd_kernel<true, false>), grid, block, 0, st, q8, q_scale, bias, k8, k_scale, v8, v8lo,
                       v_scale, out, o_part, ml_part, logits, a);
  else if (logits)
    hipLaunchKernelGGL((attn_fwd_kernel<false, true>), grid, block, 0, st, q8, q_scale, bias, k8, k_scale, v8, v8lo,
                       v_scale, out, o_part, ml_part, logits, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<false, false>), grid, block, 0, st, q8, q_scale, bias, k8, k_scale, v8, v8lo,
                       v_scale, out, o_part, ml_part, logits, a);
  if (a.split0[XCDS] > 0)
    hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)(a.split0[XCDS] * (QT / MERGE_ROWS))), dim3(256), 0, st,
                       o_part, ml_part, out, a);
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return LBW_OK;
}

extern "C" int lbw_attn_fwd(const int8_t* q8, const float* q_scale, const float* bias, int64_t batch,
                            int64_t lq, int64_t heads, const int8_t* k8, const float* k_scale,
                            const uint8_t* v8, const uint8_t* v8lo, const uint8_t* v_scale, int64_t slots,
                            int64_t cap, int n_seg, const int32_t* seg_slot, const int32_t* seg_len,
                            const int32_t* seg_first, uint16_t* out, int64_t o_s_batch, int64_t o_s_tok,
                            int64_t o_s_head, float sm_scale, void* workspace, void* stream) {
  return attn_launch(q8, q_scale, bias, batch, lq, heads, k8, k_scale, v8, v8lo, v_scale, slots, cap, n_seg, seg_slot,
                     seg_len, seg_first, out, o_s_batch, o_s_tok, o_s_head, sm_scale, nullptr, workspace, stream);
}

extern "C" int lbw_qk_logits_i32(const int8_t* q8, const float* q_scale, const float* bias, int64_t batch,
                                 int64_t lq, int64_t heads, const int8_t* k8, const float* k_scale,
                                 const uint8_t* v8, const uint8_t* v8lo, const uint8_t* v_scale, int64_t slots,
                                 int64_t cap, int n_seg, const int32_t* seg_slot, const int32_t* seg_len,
                                 const int32_t* seg_first, uint16_t* out, int64_t o_s_batch, int64_t o_s_tok,
                                 int64_t o_s_head, float sm_scale, int32_t* logits, void* workspace, void* stream) {
  if (!logits) return LBW_E_NULL;
  return attn_launch(q8, q_scale, bias, batch, lq, heads, k8, k_scale, v8, v8lo, v_scale, slots, cap, n_seg, seg_slot,
                     seg_len, seg_first, out, o_s_batch, o_s_tok, o_s_head, sm_scale, logits, workspace, stream);
}

// ---- the entry point that allocates nothing -----------------------------------------------------------------
// The split-tile partials of lbw_attn_fwd_noalloc live in this file-scope array instead of a caller workspace:
// one copy per GPU, held until the process ends. Its size is the attention workspace at 32 workgroups per XCD
// (256 CUs). In host code `scratch` names a host-side stand-in, never the device memory: the device address of a
// GPU's copy comes from hipGetSymbolAddress on that GPU, once, and only that address is passed to kernels.
constexpr int SCRATCH_WGS_PER_XCD = 32;
constexpr int64_t ATTN_SCRATCH_BYTES = (int64_t)XCDS * SCRATCH_WGS_PER_XCD * 2 * QT * (D + 2) * (int64_t)sizeof(float);
static __device__ __align__(256) uint8_t scratch[ATTN_SCRATCH_BYTES];

// Device address of this GPU's `scratch` (the current device's), looked up on the first call on each device and
// kept per device ordinal; null if the lookup fails.
static void* scratch_on_current_device() {
  static std::atomic<void*> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  void* p = cached[dev].load(std::memory_order_acquire);
  if (!p) {
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    cached[dev].store(p, std::memory_order_release);
  }
  return p;
}

extern "C" int64_t lbw_attn_noalloc_scratch_bytes(void) { return ATTN_SCRATCH_BYTES; }

extern "C" int lbw_attn_fwd_noalloc(const int8_t* q8, const float* q_scale, const float* bias, int64_t batch,
                                    int64_t lq, int64_t heads, const int8_t* k8, const float* k_scale,
                                    const uint8_t* v8, const uint8_t* v8lo, const uint8_t* v_scale, int64_t slots,
                                    int64_t cap, int n_seg, const int32_t* seg_slot, const int32_t* seg_len,
                                    const int32_t* seg_first, uint16_t* out, int64_t o_s_batch, int64_t o_s_tok,
                                    int64_t o_s_head, float sm_scale, void* stream) {
  if (const int dv = check_device()) return dv;
  if (lbw_attn_workspace_bytes() > ATTN_SCRATCH_BYTES) return LBW_E_SCRATCH;   // more CUs than the array covers
  void* ws = scratch_on_current_device();
  if (!ws) return LBW_E_DEVICE;
  return attn_launch(q8, q_scale, bias, batch, lq, heads, k8, k_scale, v8, v8lo, v_scale, slots, cap, n_seg, seg_slot,
                     seg_len, seg_first, out, o_s_batch, o_s_tok, o_s_head, sm_scale, nullptr, ws, stream);
}
