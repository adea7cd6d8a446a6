// Rowwise FP8 quantisation for the FP8 linear layers (gfx950): per row, scale = max(amax / 448, 1e-12) and
// e4m3(x / scale) with round-to-nearest-even, the scheme of the reference's FP8Linear for its weights (once, per
// output row) and its activations (every call, per token). The GEMM itself is a plain rowwise-scaled FP8 GEMM
// (hipBLASLt); this kernel is the part around it that runs on every call.
//
// Many rows of up to 4096 values: one wave per row (a one-wave workgroup), the row's amax within the wave (no
// barrier): 5.7 against 6.4 us for 6032 x 1536 bf16 on MI355X. Otherwise one workgroup per row, 256 threads, more
// loads in flight per row (2.05 against 2.4 us for 333 x 1536); rows of up to 16384 values stay in registers
// between the amax and the quantisation (one read), longer ones are read twice (the second read from the cache).
// 16-byte loads.
#include "lbw_common.h"

#pragma clang fp contract(off)

namespace lbw {

constexpr float FP8_MAX = 448.f;
constexpr float FP8_SCALE_FLOOR = 1e-12f;

template <typename T>
struct Row8;

template <>
struct Row8<uint16_t> {   // bf16: 8 values = 16 bytes
  static __device__ __forceinline__ void load(const uint16_t* p, float* f) { unpack8(*(const v4i*)p, f); }
};

template <>
struct Row8<float> {      // fp32: 8 values = 32 bytes
  static __device__ __forceinline__ void load(const float* p, float* f) {
    const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  }
};

// GELU in its tanh form (nn.GELU(approximate='tanh'), the feed-forward activation of the DiT blocks,
// lingbot/models/lingbot_world/transformer.py:313-315): 0.5 x (1 + tanh(u)) with u = sqrt(2 / pi) (x + 0.044715 x^3),
// evaluated as the identical x / (1 + e^(-2u)) on the hardware exp2 and reciprocal, then rounded to bf16 (the
// module's output type; round to nearest even). The fp32 value is within a few ulps of the exact one, so the bf16
// result is the correctly rounded GELU except for values that close to a bf16 rounding boundary. Large negative x:
// e^(-2u) overflows to inf and the result is -0 (the exact value underflows); +-inf give inf / NaN and a NaN stays
// NaN, as the tanh form does.
__device__ __forceinline__ float gelu_tanh_bf16(float x) {
  constexpr float NEG2_SQRT2PI_LOG2E = -2.f * 0.7978845608028654f * 1.4426950408889634f;
  const float a = fmaf(0.044715f * x, x, 1.f);                 // 1 + 0.044715 x^2
  const float e = __builtin_amdgcn_exp2f(NEG2_SQRT2PI_LOG2E * x * a);
  const float g = x * __builtin_amdgcn_rcpf(1.f + e);
  return (float)(__bf16)g;
}

template <bool GELU, typename T>
__device__ __forceinline__ void load8(const T* p, float* f) {
  Row8<T>::load(p, f);
  if constexpr (GELU) {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = gelu_tanh_bf16(f[e]);
  }
}

// x / sc rounded to nearest, from the row's reciprocal r = RN(1 / sc): q = RN(x r) is within an ulp of x / sc, the
// remainder x - q sc is exact under an FMA, and RN(q + rem r) is the correctly rounded quotient (Markstein's
// correction step); the sign comes from x, so a zero quotient keeps it. Equal to IEEE division wherever
// |x / sc| >= 2^-12 (a smaller quotient is +-0 in e4m3 either way): tests/test_fp8_division.py checks every bf16 x
// against 2048 scales and 2e7 random fp32 pairs (2e9 pairs and 2e4 scales checked once as well). Three
// instructions against ~10 for the division.
__device__ __forceinline__ float div_sc(float x, float sc, float r) {
  const float q = x * r;
  return __builtin_copysignf(fmaf(fmaf(-q, sc, x), r, q), x);
}

// e4m3 of 8 values divided by the row scale, as 8 bytes. For a finite scale, |x / scale| <= 448 (1 + 2^-23) by
// construction (|x| <= amax, scale >= amax / 448 up to its rounding), which the round-to-nearest cast takes to 448,
// so no clamp is needed, and a NaN quotient stays NaN as the reference's cast makes it. A row holding an infinity
// has scale = inf and r = 0: the quotient is then x * 0, +-0 for finite x and NaN for an infinite one, as IEEE
// division by infinity gives (the correction step would turn 0 * inf into NaN); a NaN row has scale NaN and every
// quotient NaN. (The row-uniform branch costs nothing.)
__device__ __forceinline__ uint2 quant8(const float* f, float sc, float r) {
  uint32_t w[2];
  const bool finite = sc < INFINITY;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = finite ? div_sc(f[4 * h + e], sc, r) : f[4 * h + e] * r;
    int pk = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
    pk = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], pk, true);
    w[h] = (uint32_t)pk;
  }
  return make_uint2(w[0], w[1]);
}

// |x| as bits: for non-negative floats the unsigned integer order is the float order, with every NaN above +inf,
// so an integer max over these is an amax that propagates NaN (as torch's amax does; fmaxf would drop it)
__device__ __forceinline__ uint32_t abs_bits(float x) { return __float_as_uint(x) & 0x7FFFFFFFu; }

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = max(x, dpp_u32<DPP_XOR1>(x));
  x = max(x, dpp_u32<DPP_XOR2>(x));
  x = max(x, dpp_u32<DPP_HALF_MIRROR>(x));
  x = max(x, dpp_u32<DPP_MIRROR>(x));
  auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = max((uint32_t)r[0], (uint32_t)r[1]);
  r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return max((uint32_t)r[0], (uint32_t)r[1]);
}

// the row's amax (as abs_bits, over the workgroup, in every thread) -> its scale, written by thread 0:
// max(amax / 448, 1e-12), NaN for a row holding a NaN and inf for one holding an infinity (the reference's clamp
// keeps both)
__device__ __forceinline__ float row_scale(uint32_t amax_bits, uint32_t* s_red, float* scale, int64_t row) {
  const int t = threadIdx.x;
  amax_bits = wave_max_u32(amax_bits);
  if ((t & 63) == 0) s_red[t >> 6] = amax_bits;
  __syncthreads();
  const float amax = __uint_as_float(max(max(s_red[0], s_red[1]), max(s_red[2], s_red[3])));
  const float q = __fdiv_rn(amax, FP8_MAX);
  const float sc = q < FP8_SCALE_FLOOR ? FP8_SCALE_FLOOR : q;
  if (t == 0) scale[row] = sc;
  return sc;
}

// Rows of at most NCH * 512 values, a one-wave workgroup each: lane l holds 8-value chunks l, l + 64, ... in
// registers. The same amax, scale and quotients as the workgroup-per-row kernels.
template <typename T, int NCH, bool GELU>
__global__ __launch_bounds__(64) void quant_rows_fp8_wave_kernel(const T* __restrict__ x, int64_t cols, int64_t s_row,
                                                                 uint8_t* __restrict__ x8, float* __restrict__ scale) {
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  const T* xr = x + row * s_row;
  float f[NCH][8];
  uint32_t amax = 0;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int64_t c = 8 * (int64_t)(lane + 64 * i);
    if (c < cols) {
      load8<GELU>(xr + c, f[i]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) f[i][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = max(amax, abs_bits(f[i][e]));
  }
  const float q = __fdiv_rn(__uint_as_float(wave_max_u32(amax)), FP8_MAX);
  const float sc = q < FP8_SCALE_FLOOR ? FP8_SCALE_FLOOR : q;
  if (lane == 0) scale[row] = sc;
  const float r = __fdiv_rn(1.f, sc);
  uint8_t* outr = x8 + row * cols;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int64_t c = 8 * (int64_t)(lane + 64 * i);
    if (c < cols) *(uint2*)(outr + c) = quant8(f[i], sc, r);
  }
}

// Rows of at most NCH * 2048 values: thread t holds 8-value chunks t, t + 256, ... in registers.
template <typename T, int NCH, bool GELU>
__global__ __launch_bounds__(256) void quant_rows_fp8_kernel(const T* __restrict__ x, int64_t cols, int64_t s_row,
                                                             uint8_t* __restrict__ x8, float* __restrict__ scale) {
  __shared__ uint32_t s_red[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * s_row;
  const int t = threadIdx.x;
  float f[NCH][8];
  uint32_t amax = 0;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int64_t c = 8 * (int64_t)(t + 256 * i);
    if (c < cols) {
      load8<GELU>(xr + c, f[i]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) f[i][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = max(amax, abs_bits(f[i][e]));
  }
  const float sc = row_scale(amax, s_red, scale, row);
  const float r = __fdiv_rn(1.f, sc);
  uint8_t* outr = x8 + row * cols;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int64_t c = 8 * (int64_t)(t + 256 * i);
    if (c < cols) *(uint2*)(outr + c) = quant8(f[i], sc, r);
  }
}

// Longer rows: the amax pass and the quantise pass each read the row.
template <typename T, bool GELU>
__global__ __launch_bounds__(256) void quant_rows_fp8_long_kernel(const T* __restrict__ x, int64_t cols,
                                                                  int64_t s_row, uint8_t* __restrict__ x8,
                                                                  float* __restrict__ scale) {
  __shared__ uint32_t s_red[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * s_row;
  const int t = threadIdx.x;
  uint32_t amax = 0;
  for (int64_t c = 8 * (int64_t)t; c < cols; c += 8 * 256) {
    float f[8];
    load8<GELU>(xr + c, f);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = max(amax, abs_bits(f[e]));
  }
  const float sc = row_scale(amax, s_red, scale, row);
  const float r = __fdiv_rn(1.f, sc);
  uint8_t* outr = x8 + row * cols;
  for (int64_t c = 8 * (int64_t)t; c < cols; c += 8 * 256) {
    float f[8];
    load8<GELU>(xr + c, f);
    *(uint2*)(outr + c) = quant8(f, sc, r);
  }
}

template <typename T, bool GELU>
static void launch_quant_rows(const T* x, int64_t rows, int64_t cols, int64_t s_row, uint8_t* x8, float* scale,
                              hipStream_t stream) {
  const dim3 grid((unsigned)rows), block(256);
  if (cols <= 4096 && rows >= 2048) {
    const dim3 wblock(64);
    const int64_t wch = (cols + 511) / 512;
    if (wch <= 1)
      hipLaunchKernelGGL((quant_rows_fp8_wave_kernel<T, 1, GELU>), grid, wblock, 0, stream, x, cols, s_row, x8, scale);
    else if (wch <= 2)
      hipLaunchKernelGGL((quant_rows_fp8_wave_kernel<T, 2, GELU>), grid, wblock, 0, stream, x, cols, s_row, x8, scale);
    else if (wch <= 3)
      hipLaunchKernelGGL((quant_rows_fp8_wave_kernel<T, 3, GELU>), grid, wblock, 0, stream, x, cols, s_row, x8, scale);
    else if (wch <= 4)
      hipLaunchKernelGGL((quant_rows_fp8_wave_kernel<T, 4, GELU>), grid, wblock, 0, stream, x, cols, s_row, x8, scale);
    else
      hipLaunchKernelGGL((quant_rows_fp8_wave_kernel<T, 8, GELU>), grid, wblock, 0, stream, x, cols, s_row, x8, scale);
    return;
  }
  const int64_t nch = (cols + 2047) / 2048;
  if (nch <= 1)
    hipLaunchKernelGGL((quant_rows_fp8_kernel<T, 1, GELU>), grid, block, 0, stream, x, cols, s_row, x8, scale);
  else if (nch <= 2)
    hipLaunchKernelGGL((quant_rows_fp8_kernel<T, 2, GELU>), grid, block, 0, stream, x, cols, s_row, x8, scale);
  else if (nch <= 4)
    hipLaunchKernelGGL((quant_rows_fp8_kernel<T, 4, GELU>), grid, block, 0, stream, x, cols, s_row, x8, scale);
  else if (nch <= 5)
    hipLaunchKernelGGL((quant_rows_fp8_kernel<T, 5, GELU>), grid, block, 0, stream, x, cols, s_row, x8, scale);
  else if (nch <= 8)
    hipLaunchKernelGGL((quant_rows_fp8_kernel<T, 8, GELU>), grid, block, 0, stream, x, cols, s_row, x8, scale);
  else
    hipLaunchKernelGGL((quant_rows_fp8_long_kernel<T, GELU>), grid, block, 0, stream, x, cols, s_row, x8, scale);
}

// MXFP8 (the reference's MXFP8Linear, lingbot/layers/linear.py:42-50): per 32 consecutive values of a row,
// scale = 2^e with e = ceil(log2(max(amax, 2^-126) / 448)) taken exactly from the bits of the fp32 quotient
// (floored at -127, E8M0's smallest), values e4m3(x / scale) (exact division by a power of two, then round to
// nearest even), and the E8M0 byte e + 127. A group holding a NaN or an infinity gets what the reference's formula
// gives it: the E8M0 NaN byte 255 and x / amax (all NaN for a NaN group; +-0, and NaN for the infinity, for an
// infinite one). One thread per 32-value group; rows from `rows` up to `rows_pad` are written as zeros with scale
// byte 127 (2^0), so the GEMM can take a row count padded to its tile.
template <typename T>
__global__ __launch_bounds__(256) void quant_mx_fp8_kernel(const T* __restrict__ x, int64_t rows, int64_t rows_pad,
                                                           int64_t cols, int64_t s_row, uint8_t* __restrict__ x8,
                                                           uint8_t* __restrict__ e8) {
  const int64_t groups = cols / 32;
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= rows_pad * groups) return;
  const int64_t row = id / groups, grp = id - row * groups;
  uint8_t* out = x8 + row * cols + grp * 32;
  if (row >= rows) {
#pragma unroll
    for (int i = 0; i < 2; ++i) *(v4i*)(out + 16 * i) = v4i{0, 0, 0, 0};
    e8[id] = 127;
    return;
  }
  float f[32];
  const T* xr = x + row * s_row + grp * 32;
#pragma unroll
  for (int i = 0; i < 4; ++i) Row8<T>::load(xr + 8 * i, f + 8 * i);
  uint32_t abits = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) abits = max(abits, abs_bits(f[i]));
  const bool finite = abits < 0x7F800000u;
  const float amax = fmaxf(__uint_as_float(finite ? abits : 0u), 0x1p-126f);
  const float qv = __fdiv_rn(amax, FP8_MAX);
  // exact ceil(log2(qv)) of a positive float: the exponent of its top bit, plus one unless qv is a power of two
  const uint32_t qb = __float_as_uint(qv);
  int e;
  if ((qb >> 23) == 0) {   // subnormal quotient: value = m * 2^-149
    const uint32_t m = qb & 0x7FFFFFu;
    const int top = 31 - __builtin_clz(m);
    e = top - 149 + ((m & (m - 1)) ? 1 : 0);
  } else {
    e = (int)(qb >> 23) - 127 + ((qb & 0x7FFFFFu) ? 1 : 0);
  }
  e = e < -127 ? -127 : e;
  // 1 / 2^e as a float (2^-e, e in [-127, 127]); x * 2^-e is exact for every finite x here, and |x| 2^-e <= 448
  // (2^e >= amax / 448), so the cast needs no clamp. Non-finite group: 1 / amax (0 or NaN).
  const float inv = !finite ? __uint_as_float(abits == 0x7F800000u ? 0u : abits)
                            : e >= -126 ? __uint_as_float((uint32_t)(127 - e) << 23) : 0x1p127f;
  e8[id] = finite ? (uint8_t)(e + 127) : (uint8_t)255;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int b0 = 16 * i + 4 * k;
      int pk = __builtin_amdgcn_cvt_pk_fp8_f32(f[b0] * inv, f[b0 + 1] * inv, 0, false);
      pk = __builtin_amdgcn_cvt_pk_fp8_f32(f[b0 + 2] * inv, f[b0 + 3] * inv, pk, true);
      w[k] = (uint32_t)pk;
    }
    *(v4i*)(out + 16 * i) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  }
}

}  // namespace lbw

using namespace lbw;

extern "C" int lbw_quant_rows_fp8(const void* x, int x_is_fp32, int64_t rows, int64_t cols, int64_t s_row,
                                  uint8_t* x8, float* scale, void* stream) {
  if (!x || !x8 || !scale) return LBW_E_NULL;
  if (rows <= 0 || cols <= 0 || rows > 0x7fffffff || cols % 16 != 0) return LBW_E_SHAPE;
  if (s_row < cols) return LBW_E_SHAPE;
  if (s_row % 8 != 0 || ((uintptr_t)x & 15) || ((uintptr_t)x8 & 7)) return LBW_E_ALIGN;
  if (const int dv = check_device()) return dv;
  if (x_is_fp32)
    launch_quant_rows<float, false>((const float*)x, rows, cols, s_row, x8, scale, (hipStream_t)stream);
  else
    launch_quant_rows<uint16_t, false>((const uint16_t*)x, rows, cols, s_row, x8, scale, (hipStream_t)stream);
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return LBW_OK;
}

extern "C" int lbw_quant_rows_fp8_gelu(const uint16_t* x, int64_t rows, int64_t cols, int64_t s_row, uint8_t* x8,
                                       float* scale, void* stream) {
  if (!x || !x8 || !scale) return LBW_E_NULL;
  if (rows <= 0 || cols <= 0 || rows > 0x7fffffff || cols % 16 != 0) return LBW_E_SHAPE;
  if (s_row < cols) return LBW_E_SHAPE;
  if (s_row % 8 != 0 || ((uintptr_t)x & 15) || ((uintptr_t)x8 & 7)) return LBW_E_ALIGN;
  if (const int dv = check_device()) return dv;
  launch_quant_rows<uint16_t, true>(x, rows, cols, s_row, x8, scale, (hipStream_t)stream);
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return LBW_OK;
}

extern "C" int lbw_quant_mx_fp8(const void* x, int x_is_fp32, int64_t rows, int64_t rows_pad, int64_t cols,
                                int64_t s_row, uint8_t* x8, uint8_t* scale_e8m0, void* stream) {
  if (!x || !x8 || !scale_e8m0) return LBW_E_NULL;
  if (rows <= 0 || rows_pad < rows || cols <= 0 || cols % 32 != 0 || s_row < cols) return LBW_E_SHAPE;
  if (rows_pad > ((int64_t)1 << 31) || rows_pad * (cols / 32) > ((int64_t)1 << 38)) return LBW_E_SHAPE;
  if (s_row % 8 != 0 || ((uintptr_t)x & 15) || ((uintptr_t)x8 & 15)) return LBW_E_ALIGN;
  if (const int dv = check_device()) return dv;
  const int64_t n = rows_pad * (cols / 32);
  const dim3 grid((unsigned)((n + 255) / 256));
  if (x_is_fp32)
    hipLaunchKernelGGL(quant_mx_fp8_kernel<float>, grid, dim3(256), 0, (hipStream_t)stream, (const float*)x, rows,
                       rows_pad, cols, s_row, x8, scale_e8m0);
  else
    hipLaunchKernelGGL(quant_mx_fp8_kernel<uint16_t>, grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t*)x,
                       rows, rows_pad, cols, s_row, x8, scale_e8m0);
  if (hipGetLastError() != hipSuccess) return LBW_E_LAUNCH;
  return LBW_OK;
}
