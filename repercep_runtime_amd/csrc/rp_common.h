// Shared device helpers for the gfx950 FP8 attention path.
//
// Everything here is written for CDNA4 (gfx950): wave64, OCP e4m3fn FP8
// (bias 7, max 448, S.1111.111 = NaN), the f8f6f4 MFMA family, 160 KiB LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/repercep_fp8.h"

namespace rp {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;
constexpr float kE4m3Max = 448.0f;
// 0.95 * 448 evaluated in double is 425.59999999999997; torch applies the
// scalar divisor as the nearest fp32 value, 425.6f.
constexpr float kScaleDivisor = 425.6f;

// ------------------------------------------------------------------ bf16
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 bits, round to nearest even; NaN stays NaN (quieted).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16_bits(f)); }

// ------------------------------------------------------------------ fp16
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
// fp32 -> fp16 -> fp32, round to nearest even with fp16 subnormals kept
// (v_cvt_f16_f32 under the default mode), overflow to inf, NaN stays NaN.
// The empty asm makes the operand an opaque, already rounded fp32 value:
// otherwise the compiler fuses a preceding multiply into the conversion
// (v_fma_mixlo_f16, one rounding), where the reference rounds the fp32
// product first and then converts.
__device__ __forceinline__ float f16_round(float f) {
  asm("" : "+v"(f));
  return (float)(_Float16)f;
}
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  asm("" : "+v"(lo), "+v"(hi));
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
}

// Quantizer input element types (RP_DTYPE_* of the C interface).
constexpr int kInBf16 = 0, kInF16 = 1;

template <int DT>
__device__ __forceinline__ float in_to_f32(uint32_t bits16) {
  if constexpr (DT == kInF16) return f16_to_f32(bits16);
  else return bf16_to_f32(bits16);
}

// -------------------------------------------------------------- e4m3fn
// Two fp32 -> two e4m3fn codes in bits [16*hi, 16*hi+16) of `old`, using the
// gfx950 hardware conversion (round to nearest even).
template <bool kHi>
__device__ __forceinline__ int cvt_pk_e4m3(float a, float b, int old) {
  return __builtin_amdgcn_cvt_pk_fp8_f32(a, b, old, kHi);
}

// Four fp32 -> one dword of codes, element 0 in the low byte.
__device__ __forceinline__ uint32_t pack4_e4m3(float a, float b, float c, float d) {
  // The low-half conversion as asm with a write-only destination: the
  // builtin keeps the destination's high half, which would cost a register
  // initialisation per dword although the high-half conversion below
  // overwrites it.
  int r;
  asm("v_cvt_pk_fp8_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  r = cvt_pk_e4m3<true>(c, d, r);
  return (uint32_t)r;
}

// Reference clamp: Tensor.clamp(-448, 448) propagates NaN.  The IEEE
// 754-2019 minimum and maximum (v_minimum3_f32, v_maximum3_f32 on gfx950)
// propagate it themselves: two instructions instead of a min, a max, a
// compare and a select (the NaN's sign and payload may change; its e4m3
// code is a NaN code either way).
__device__ __forceinline__ float clamp_e4m3(float v) {
  return __builtin_elementwise_maximum(__builtin_elementwise_minimum(v, kE4m3Max), -kE4m3Max);
}

// Four 16-bit inputs (two packed pairs, element 0 in the low half of
// lo_pair) -> one dword of e4m3fn codes: the quantizer's
// clamp(x * qm, +-448) cast (qm = fp32 1 / dequant).  Shared by the
// quantizer and the attention kernels that quantize their own Q rows, so
// both produce the same codes.
template <int DT>
__device__ __forceinline__ uint32_t quant4(uint32_t lo_pair, uint32_t hi_pair, float qm) {
  const float a = clamp_e4m3(in_to_f32<DT>(lo_pair & 0xffffu) * qm);
  const float b = clamp_e4m3(in_to_f32<DT>(lo_pair >> 16) * qm);
  const float c = clamp_e4m3(in_to_f32<DT>(hi_pair & 0xffffu) * qm);
  const float d = clamp_e4m3(in_to_f32<DT>(hi_pair >> 16) * qm);
  return pack4_e4m3(a, b, c, d);
}

// ---------------------------------------------------------- reductions
template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

// v + (v of the lane N places further round this lane's 16-lane row), by a
// DPP row rotation (no LDS round trip).  Sums over a 16-lane row in the
// order of the xor butterfly (xor 8, 4, 2, 1) come out bit for bit when the
// rotations go 8, 4, 2, 1: after the xor-8 step lanes 8 apart hold equal
// values, so lane i + 4 (mod 16) holds the value of lane i ^ 4, and so on
// down; every lane adds the same two operands in the same order.
template <int N>
__device__ __forceinline__ float add_row_ror(float v) {
  static_assert(N >= 1 && N <= 15, "row rotation");
  const int r = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x120 + N, 0xf, 0xf, false);
  return v + __int_as_float(r);
}

__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b) { return a > b ? a : b; }

// Two independent 16-bit unsigned maxima in one dword (v_pk_max_u16).
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                                __builtin_bit_cast(u16x2, b)));
}

// Max of n uint32 values at v, by one workgroup of NT threads; the result is
// valid in thread 0.  Each thread keeps eight independent loads in flight
// (a per-tensor scale reduces ~10^4 block maxima: one load at a time, that is
// a chain of ~50 memory latencies per thread).
template <int NT>
__device__ __forceinline__ uint32_t block_max_u32(const uint32_t* v, int64_t n) {
  uint32_t m = 0;
  for (int64_t i0 = threadIdx.x; i0 < n; i0 += 8 * NT) {
    uint32_t x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t i = i0 + (int64_t)u * NT;
      x[u] = i < n ? v[i] : 0u;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) m = umax32(m, x[u]);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = umax32(m, (uint32_t)__shfl_xor((int)m, o, 64));
  __shared__ uint32_t wmax[NT / 64];
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x / 64] = m;
  __syncthreads();
  uint32_t r = wmax[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) r = umax32(r, wmax[w]);
  return r;
}

// Dequant scale from the bf16 bit pattern of a group's |x| maximum, as the
// reference computes it: clamp in bf16 against bf16(1e-6), divide by 425.6
// in fp32, round the quotient to bf16.  Division is IEEE (this file is never
// built with fast-math).
__device__ __forceinline__ float dequant_from_amax_bits(uint32_t amax_bits) {
  const float lo = __uint_as_float(0x3586u << 16);  // bf16(1e-6) = 9.98377799987793e-07
  float a = bf16_to_f32(amax_bits);
  if (!(a != a) && a < lo) a = lo;
  return bf16_round(a / kScaleDivisor);
}

// The same for fp16 input.  On the GPU torch evaluates `half_tensor / 425.6`
// as a multiply by the fp32 reciprocal of the scalar (its true-divide kernel
// takes a * (1/b) when b is a CPU scalar), and that differs from a division
// for two fp16 maxima; for bf16 the two forms agree on every value.  Amax
// values below ~1.3e-5 give a zero fp16 scale, as in the reference.
__device__ __forceinline__ float dequant_from_amax_bits_f16(uint32_t amax_bits) {
  const float lo = 17.0f * 0x1p-24f;                // fp16(1e-6) = 1.0132789611816406e-06
  constexpr float inv = 1.0f / kScaleDivisor;       // RN(1 / 425.6f)
  float a = f16_to_f32(amax_bits);
  if (!(a != a) && a < lo) a = lo;
  return f16_round(a * inv);
}

template <int DT>
__device__ __forceinline__ float dequant_from_amax(uint32_t amax_bits) {
  if constexpr (DT == kInF16) return dequant_from_amax_bits_f16(amax_bits);
  else return dequant_from_amax_bits(amax_bits);
}

}  // namespace rp

// Thread-local last-error message shared by all entry points.
extern "C" void rp_set_error(const char* fmt, ...);
