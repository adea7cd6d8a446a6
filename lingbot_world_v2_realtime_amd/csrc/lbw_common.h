// Shared device helpers of the gfx950 quantized attention kernels.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <climits>

#include "../../include/lbw_attn.h"

namespace lbw {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int D = LBW_HEAD_DIM;   // head dim
constexpr int KB = 64;            // keys per K scale block / V block
constexpr int QG = 32;            // query rows per Q scale
constexpr int QT = 256;           // Lq is padded to whole tiles of this many rows (the attention tile)
constexpr float V_MAX = 448.f;
// The optional second V plane holds the residual y - e4m3(y) of y = V / 2^e as bf6 (OCP e3m2) codes, the 32 of a key
// group in 24 bytes, rows of 48 bytes per channel and block; the attention multiplies it by bf6(P / P_LO_SCALE).
constexpr int V_LO_ROW = 48;
constexpr int V_LO_TILE = D * V_LO_ROW;      // 6 KB: the residual plane of one 64-key block
constexpr float P_LO_SCALE = 16.f;
constexpr float AMAX_FLOOR = 1e-7f;
constexpr float P_OFFSET = 8.807f;           // log2(448): P = exp2(s - m + P_OFFSET) <= 448
// A row's reference max m moves only when a block's max exceeds it by more than RESCALE_SLACK (log2 units);
// P = exp2(s - m + P_OFFSET - RESCALE_SLACK) then stays <= 448 and the O rescale is rare.
constexpr float RESCALE_SLACK = 2.f;
// The QK^T accumulator starts at the bits of S_MAGIC_F = 0x1.45f306p-3 (1 / (2 pi), an inline constant of the MFMA's
// accumulator operand), whose binade [1/8, 1/4) has ulp 2^-26 and room for 2292099 steps down and 6096509 up: for an
// int8 logit |s| <= 128 * 128 * 128 = 2^21, float(S_MAGIC + s) == S_MAGIC_F + s * 2^-26 exactly.
constexpr int S_MAGIC = 0x3E22F983;
constexpr float S_MAGIC_F = 0x1.45f306p-3f;
constexpr float S_MAGIC_INV_ULP = 67108864.f;   // 2^26

// Loads of data that is read once: the non-temporal hint streams it through the caches without keeping it
// (measured on MI355X: 7.0-7.3 TB/s for a 1.1 GB read against 6.3-6.4 TB/s with plain loads).
__device__ __forceinline__ v4i load_once(const void* p) { return __builtin_nontemporal_load((const v4i*)p); }
// Stores of results the next kernels do not read soon (measured: no change for a 30-layer re-quant, -4 % for a
// one-layer one; non-temporal loads in the re-quant's second pass cost +5 %, so it keeps plain loads).
typedef int v2i __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void store_once(void* p, v2i v) { __builtin_nontemporal_store(v, (v2i*)p); }
__device__ __forceinline__ void store_once(void* p, v4i v) { __builtin_nontemporal_store(v, (v4i*)p); }

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// 32 floats -> 32 bf6 codes (192 bits, code k at bits 6 k .. 6 k + 5): code 2 k is a[k] / scale and code 2 k + 1 is
// b[k] / scale, rounded to nearest even, magnitudes above 28 saturating (a NaN gives 28 with its sign). Inline asm
// with an early-clobber result: the builtin's result register range was allowed to overlap its sources, which the
// instruction does not support (it overwrote sources it had yet to read).
typedef int v6i __attribute__((ext_vector_type(6)));
__device__ __forceinline__ v6i cvt_bf6_x32(const v16f& a, const v16f& b, float scale) {
  v6i r;
  asm("v_cvt_scalef32_2xpk16_bf6_f32 %0, %1, %2, %3" : "=&v"(r) : "v"(a), "v"(b), "v"(scale));
  return r;
}

// fp32 -> nearest bf16 (ties to even) as fp32; finite inputs.
__device__ __forceinline__ float bf16_round(float x) {
  uint32_t u = __float_as_uint(x);
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  return __uint_as_float(u);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  u = u + 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Unpack 8 bf16 held in a 16-byte vector to fp32.
__device__ __forceinline__ void unpack8(const v4i w, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t u = (uint32_t)w[i];
    f[2 * i] = __uint_as_float(u << 16);
    f[2 * i + 1] = __uint_as_float(u & 0xFFFF0000u);
  }
}

// The 16-bit input formats of the quantisers: bf16, or IEEE fp16 (LBW_DTYPE_FP16).
template <bool F16>
__device__ __forceinline__ float lo16(uint32_t u) {   // the low 16-bit value of a word, exactly, as fp32
  if constexpr (F16) return __half2float(__ushort_as_half((unsigned short)(u & 0xFFFFu)));
  else return __uint_as_float(u << 16);
}
template <bool F16>
__device__ __forceinline__ float hi16(uint32_t u) {   // the high one
  if constexpr (F16) return __half2float(__ushort_as_half((unsigned short)(u >> 16)));
  else return __uint_as_float(u & 0xFFFF0000u);
}
template <bool F16>
__device__ __forceinline__ void unpack8t(const v4i w, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = lo16<F16>((uint32_t)w[i]);
    f[2 * i + 1] = hi16<F16>((uint32_t)w[i]);
  }
}
// fp32 -> the nearest value of the 16-bit format (ties to even), as fp32; finite inputs
template <bool F16>
__device__ __forceinline__ float round16(float x) {
  if constexpr (F16) return __half2float(__float2half_rn(x));
  else return bf16_round(x);
}

// round(x * recip) to int8 with saturation; explicit roundings so no FMA contraction can occur.
__device__ __forceinline__ int quant_i8(float x, float recip) {
  float r = rintf(__fmul_rn(x, recip));
  r = fminf(fmaxf(r, -128.f), 127.f);
  return (int)r;
}

// Cross-lane reads by DPP, within rows of 16 lanes: a VALU operand modifier, with no LDS round trip (a shuffle
// through ds_bpermute costs an LDS instruction and its latency per step). Every source lane used here is inside
// the row, so the row / bank masks keep all lanes.
constexpr int DPP_XOR1 = 0xB1;          // quad_perm [1, 0, 3, 2]: lane ^ 1
constexpr int DPP_XOR2 = 0x4E;          // quad_perm [2, 3, 0, 1]: lane ^ 2
constexpr int DPP_HALF_MIRROR = 0x141;  // lane 7 - i within each 8 lanes
constexpr int DPP_MIRROR = 0x140;       // lane 15 - i within each 16 lanes

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp(float x) { return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(x))); }
template <int CTRL>
__device__ __forceinline__ double dpp(double x) {
  const uint64_t u = (uint64_t)__double_as_longlong(x);
  const uint64_t lo = dpp_u32<CTRL>((uint32_t)u), hi = dpp_u32<CTRL>((uint32_t)(u >> 32));
  return __longlong_as_double((long long)(lo | (hi << 32)));
}

// Sum over each row of 16 lanes, every lane receiving the value of the xor butterfly s += s[lane ^ o] for
// o = 1, 2, 4, 8 in that order, bit for bit: after the first two steps the four lanes of a quad hold the same
// bits (each addition is commutative), so the half-row mirror reads what lane ^ 4 holds; after the third, the
// eight lanes of a half-row do, so the row mirror reads what lane ^ 8 holds.
template <typename T>
__device__ __forceinline__ T row16_sum(T s) {
  s = s + dpp<DPP_XOR1>(s);
  s = s + dpp<DPP_XOR2>(s);
  s = s + dpp<DPP_HALF_MIRROR>(s);
  s = s + dpp<DPP_MIRROR>(s);
  return s;
}

// max over lanes l and l ^ 16 (v_permlane16_swap), and over l and l ^ 32 (v_permlane32_swap)
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// max over the wave's 64 lanes (exact in any order), in every lane
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp<DPP_XOR1>(x));
  x = fmaxf(x, dpp<DPP_XOR2>(x));
  x = fmaxf(x, dpp<DPP_HALF_MIRROR>(x));
  x = fmaxf(x, dpp<DPP_MIRROR>(x));
  return max_xor32(max_xor16(x));
}

// LBW_OK when the current device is a gfx950, else LBW_E_DEVICE (defined in lbw_abi.hip).
int check_device();

// The K/V re-quant's argument checks of the ring side, and its launches (kv_requant.hip). With with_stats false
// the statistics pass is skipped: the caller has written the column sums of K of each 32-token half of each 64-token
// block ([layers][batch * heads][blocks][2][128] fp32) at the start of the workspace, and V is quantised in the last
// pass with K.
int kv_requant_check(int64_t layers, int64_t batch, int64_t len, int64_t heads, const int8_t* k8,
                     const float* k_scale, const float* km, const uint8_t* v8, const uint8_t* v8lo,
                     const uint8_t* v_scale, int64_t slots, int64_t cap, int64_t slot);
int kv_requant_launch(bool with_stats, bool f16, const uint16_t* k, const uint16_t* v, int64_t layers, int64_t batch,
                      int64_t len, int64_t heads, int64_t k_s_layer, int64_t k_s_batch, int64_t k_s_tok,
                      int64_t k_s_head, int64_t v_s_layer, int64_t v_s_batch, int64_t v_s_tok, int64_t v_s_head,
                      int8_t* k8, float* k_scale, float* km, uint8_t* v8, uint8_t* v8lo, uint8_t* v_scale,
                      int64_t slots, int64_t cap, int64_t slot, void* workspace, void* stream);

// Position of key k (0..63) inside a 64-key fp8 V block.
__device__ __forceinline__ int v_pos_of_key(int k) {
  return 32 * ((k >> 2) & 1) + 16 * ((k >> 5) & 1) + 4 * ((k >> 3) & 3) + (k & 3);
}

}  // namespace lbw
