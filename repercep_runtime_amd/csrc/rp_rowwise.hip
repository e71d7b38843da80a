// Row-wise FP8 quantization for gfx950, and the row kernels of the unfused
// FP8 attention built on it.
//
// Semantics follow _rowwise_quantize of the reference's unfused FP8
// attention (src/repercep/attention/fp8_scaled_mm.py:107-133) with the OCP
// e4m3fn constants (FP8_MAX 448, target 0.95 * 448 -> 425.6f as torch applies
// the Python scalar), the same adaptation the OCP siblings of the per-(b,h)
// quantizer make (kernels/triton_kernels/fp8_flash_attn_hopper.py:374-398).
// For each row of `cols` elements, in the input dtype (bf16 or fp16):
//   amax    = max |x| over the row, clamped below at dtype(1e-6)
//   qmul    = dtype(dtype(1 / amax) * 425.6f)  -- torch's `target / amax` is
//             amax.reciprocal() * target: two roundings to the dtype
//   dequant = dtype(amax / 425.6)                -- as the per-(b,h) scale
//   codes   = e4m3fn(clamp(fp32(x) * qmul, -448, 448)), round to nearest even
// so a row's largest element maps to ~425.6, like the per-(b,h) path, but
// through a 16-bit multiplier instead of the fp32 reciprocal of the scale.
//
// Kernels:
// * rowwise_quant_kernel<DT, TPR>: rows of at most 2048 elements; TPR
//   consecutive lanes hold one row (<= 4 16-byte vectors each), reduce its
//   maximum with a butterfly and write its codes: one read, one write.
// * rowwise_quant_long_kernel<DT>: longer rows, one workgroup per row, the
//   row read twice (the second read mostly from L2).
// * transpose16_kernel: a 16-bit (R, C) -> (C, R) transpose through LDS, for
//   V^T, whose rows (one per head-dim index) the P.V product quantizes.
// * softmax_rowquant_kernel: one workgroup per row of raw scores:
//   s = bf16(raw * scale), the causal mask, P = softmax(s) rounded to bf16
//   as torch's bf16 softmax returns it, and P's row-wise codes and scale.
//   Three passes over the row (max, sum, output); the row maximum of P is
//   bf16(1 / sum) -- exp(0) = 1 at the row's largest score, and rounding is
//   monotone -- so P's scale is known before its codes are written.

#include "rp_common.h"

namespace rp {
namespace {

constexpr int kRThreads = 256;
typedef unsigned int u32x4r __attribute__((ext_vector_type(4)));

// qmul and dequant of a row from the bit pattern of its |x| maximum.
template <int DT>
__device__ __forceinline__ void rowwise_scales(uint32_t amax_bits, float* qmul, float* dequant) {
  if constexpr (DT == kInF16) {
    const float lo = 17.0f * 0x1p-24f;  // fp16(1e-6)
    float a = f16_to_f32(amax_bits);
    if (!(a != a) && a < lo) a = lo;
    const float r = f16_round(1.0f / a);
    *qmul = f16_round(r * kScaleDivisor);
    *dequant = f16_round(a * (1.0f / kScaleDivisor));
  } else {
    const float lo = __uint_as_float(0x3586u << 16);  // bf16(1e-6)
    float a = bf16_to_f32(amax_bits);
    if (!(a != a) && a < lo) a = lo;
    const float r = bf16_round(1.0f / a);
    *qmul = bf16_round(r * kScaleDivisor);
    *dequant = bf16_round(a / kScaleDivisor);
  }
}

__device__ __forceinline__ uint32_t pk_umax16r(uint32_t a, uint32_t b) {
  const uint32_t lo = umax32(a & 0xffffu, b & 0xffffu);
  const uint32_t hi = umax32(a >> 16, b >> 16);
  return lo | (hi << 16);
}

// Eight inputs (one 16-byte vector) -> eight codes.
template <int DT>
__device__ __forceinline__ uint2 quant8(const u32x4r& v, float qm) {
  uint2 o;
  const float a0 = clamp_e4m3(in_to_f32<DT>(v[0] & 0xffffu) * qm);
  const float a1 = clamp_e4m3(in_to_f32<DT>(v[0] >> 16) * qm);
  const float a2 = clamp_e4m3(in_to_f32<DT>(v[1] & 0xffffu) * qm);
  const float a3 = clamp_e4m3(in_to_f32<DT>(v[1] >> 16) * qm);
  const float a4 = clamp_e4m3(in_to_f32<DT>(v[2] & 0xffffu) * qm);
  const float a5 = clamp_e4m3(in_to_f32<DT>(v[2] >> 16) * qm);
  const float a6 = clamp_e4m3(in_to_f32<DT>(v[3] & 0xffffu) * qm);
  const float a7 = clamp_e4m3(in_to_f32<DT>(v[3] >> 16) * qm);
  o.x = pack4_e4m3(a0, a1, a2, a3);
  o.y = pack4_e4m3(a4, a5, a6, a7);
  return o;
}

__device__ __forceinline__ uint32_t absmax8(const u32x4r& v) {
  uint32_t m = pk_umax16r(v[0] & 0x7fff7fffu, v[1] & 0x7fff7fffu);
  m = pk_umax16r(m, pk_umax16r(v[2] & 0x7fff7fffu, v[3] & 0x7fff7fffu));
  return umax32(m & 0xffffu, m >> 16);
}

// Rows of at most 4 * 8 * TPR elements: TPR lanes per row (TPR divides 64).
template <int DT, int TPR>
__global__ __launch_bounds__(kRThreads) void rowwise_quant_kernel(const uint16_t* x, int64_t rows,
                                                                  int64_t cols, int64_t ldx,
                                                                  float* dequant, uint8_t* codes,
                                                                  int64_t ldq) {
  constexpr int RPB = kRThreads / TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const int t = threadIdx.x % TPR;
  const int nv = (int)(cols >> 3);
  const bool live = row < rows;
  const u32x4r* src = reinterpret_cast<const u32x4r*>(x + (live ? row : 0) * ldx);
  u32x4r v[4];
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int vi = t + i * TPR;
    v[i] = (live && vi < nv) ? src[vi] : u32x4r{0u, 0u, 0u, 0u};
    m = umax32(m, absmax8(v[i]));
  }
#pragma unroll
  for (int o = TPR / 2; o >= 1; o >>= 1) m = umax32(m, (uint32_t)__shfl_xor((int)m, o, kWave));
  if (!live) return;
  float qm, dq;
  rowwise_scales<DT>(m, &qm, &dq);
  uint8_t* dst = codes + row * ldq;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int vi = t + i * TPR;
    if (vi < nv) *reinterpret_cast<uint2*>(dst + 8 * vi) = quant8<DT>(v[i], qm);
  }
  if (t == 0) dequant[row] = dq;
}

// Rows longer than 2048 elements: one workgroup per row.
template <int DT>
__global__ __launch_bounds__(kRThreads) void rowwise_quant_long_kernel(const uint16_t* x,
                                                                       int64_t cols, int64_t ldx,
                                                                       float* dequant,
                                                                       uint8_t* codes,
                                                                       int64_t ldq) {
  const int64_t row = blockIdx.x;
  const int64_t nv = cols >> 3;
  const u32x4r* src = reinterpret_cast<const u32x4r*>(x + row * ldx);
  uint32_t m = 0;
  for (int64_t vi = threadIdx.x; vi < nv; vi += kRThreads) m = umax32(m, absmax8(src[vi]));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = umax32(m, (uint32_t)__shfl_xor((int)m, o, kWave));
  __shared__ uint32_t wmax[kRThreads / kWave];
  if ((threadIdx.x & (kWave - 1)) == 0) wmax[threadIdx.x / kWave] = m;
  __syncthreads();
  m = umax32(umax32(wmax[0], wmax[1]), umax32(wmax[2], wmax[3]));
  float qm, dq;
  rowwise_scales<DT>(m, &qm, &dq);
  uint8_t* dst = codes + row * ldq;
  for (int64_t vi = threadIdx.x; vi < nv; vi += kRThreads)
    *reinterpret_cast<uint2*>(dst + 8 * vi) = quant8<DT>(src[vi], qm);
  if (threadIdx.x == 0) dequant[row] = dq;
}

// 16-bit transpose of each of `batch` (R, C) matrices: dst (C, R), row
// strides lds / ldd elements, batch strides bs / bd.  64 x 64 tiles.
__global__ __launch_bounds__(kRThreads) void transpose16_kernel(const uint16_t* src, uint16_t* dst,
                                                                int64_t R, int64_t C, int64_t lds,
                                                                int64_t ldd, int64_t bs,
                                                                int64_t bd) {
  __shared__ uint16_t tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  src += (int64_t)blockIdx.z * bs;
  dst += (int64_t)blockIdx.z * bd;
  for (int i = threadIdx.x; i < 64 * 64; i += kRThreads) {
    const int r = i >> 6, c = i & 63;
    if (r0 + r < R && c0 + c < C) tile[r][c] = src[(r0 + r) * lds + c0 + c];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += kRThreads) {
    const int c = i >> 6, r = i & 63;
    if (r0 + r < R && c0 + c < C) dst[(c0 + c) * ldd + r0 + r] = tile[r][c];
  }
}

// max that propagates NaN, as torch's softmax does
__device__ __forceinline__ float nmax(float a, float b) {
  return (a != a) ? a : ((b != b) ? b : fmaxf(a, b));
}

// Block-wide reductions of one value per thread (256 threads).
__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = nmax(v, __shfl_xor(v, o, kWave));
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  return nmax(nmax(red[0], red[1]), nmax(red[2], red[3]));
}
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// s = bf16(raw * scale), -inf past the row's causal limit
__device__ __forceinline__ float score(uint32_t raw_bits, float scale, int64_t j, int64_t lim) {
  const float s = bf16_round(bf16_to_f32(raw_bits) * scale);
  return j <= lim ? s : -__builtin_inff();
}

// One workgroup per row r of `rows` raw score rows (bf16, `cols` each, row
// stride lds); query index q = r % sq gives the causal limit (keys j <= q).
__global__ __launch_bounds__(kRThreads) void softmax_rowquant_kernel(const uint16_t* scores,
                                                                     int64_t cols, int64_t lds,
                                                                     int64_t sq, int causal,
                                                                     float scale, float* dequant,
                                                                     uint8_t* codes, int64_t ldq) {
  __shared__ float red[kRThreads / kWave];
  const int64_t row = blockIdx.x;
  const int64_t lim = causal ? row % sq : cols;
  const uint16_t* src = scores + row * lds;
  const int64_t npair = cols >> 1;
  const uint32_t* s2 = reinterpret_cast<const uint32_t*>(src);
  float m = -__builtin_inff();
  for (int64_t i = threadIdx.x; i < npair; i += kRThreads) {
    const uint32_t w = s2[i];
    m = nmax(m, nmax(score(w & 0xffffu, scale, 2 * i, lim), score(w >> 16, scale, 2 * i + 1, lim)));
  }
  m = block_max(m, red);
  float sum = 0.0f;
  for (int64_t i = threadIdx.x; i < npair; i += kRThreads) {
    const uint32_t w = s2[i];
    sum += expf(score(w & 0xffffu, scale, 2 * i, lim) - m);
    sum += expf(score(w >> 16, scale, 2 * i + 1, lim) - m);
  }
  sum = block_sum(sum, red);
  // P's row maximum is bf16(1 / sum): its scales, then its codes
  float qm, dq;
  rowwise_scales<kInBf16>(f32_to_bf16_bits(1.0f / sum), &qm, &dq);
  uint8_t* dst = codes + row * ldq;
  for (int64_t i = threadIdx.x; i < npair; i += kRThreads) {
    const uint32_t w = s2[i];
    const float p0 = bf16_round(expf(score(w & 0xffffu, scale, 2 * i, lim) - m) / sum);
    const float p1 = bf16_round(expf(score(w >> 16, scale, 2 * i + 1, lim) - m) / sum);
    int pk;
    asm("v_cvt_pk_fp8_f32 %0, %1, %2" : "=v"(pk) : "v"(clamp_e4m3(p0 * qm)), "v"(clamp_e4m3(p1 * qm)));
    *reinterpret_cast<uint16_t*>(dst + 2 * i) = (uint16_t)pk;
  }
  if (threadIdx.x == 0) dequant[row] = dq;
}

int rw_check(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    rp_set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return RP_ERR_LAUNCH;
  }
  return RP_OK;
}

template <int DT>
int launch_rowwise(const uint16_t* x, int64_t rows, int64_t cols, int64_t ldx, float* dq,
                   uint8_t* codes, int64_t ldq, hipStream_t st) {
  const int64_t nv = cols / 8;
  if (nv > 256) {
    if (rows > 0x7fffffff) {
      rp_set_error("rowwise_quantize: too many rows");
      return RP_ERR_UNSUPPORTED;
    }
    hipLaunchKernelGGL(rowwise_quant_long_kernel<DT>, dim3((unsigned)rows), dim3(kRThreads), 0,
                       st, x, cols, ldx, dq, codes, ldq);
    return rw_check("rowwise_quant_long");
  }
  // lanes per row: the smallest power of two with at most 4 vectors each
  int tpr = 8;
  while (tpr < 64 && (nv + tpr - 1) / tpr > 4) tpr *= 2;
  const int64_t rpb = kRThreads / tpr;
  const int64_t blocks = (rows + rpb - 1) / rpb;
  if (blocks > 0x7fffffff) {
    rp_set_error("rowwise_quantize: too many rows");
    return RP_ERR_UNSUPPORTED;
  }
  const dim3 g((unsigned)blocks), b(kRThreads);
  switch (tpr) {
    case 8: hipLaunchKernelGGL((rowwise_quant_kernel<DT, 8>), g, b, 0, st, x, rows, cols, ldx, dq, codes, ldq); break;
    case 16: hipLaunchKernelGGL((rowwise_quant_kernel<DT, 16>), g, b, 0, st, x, rows, cols, ldx, dq, codes, ldq); break;
    case 32: hipLaunchKernelGGL((rowwise_quant_kernel<DT, 32>), g, b, 0, st, x, rows, cols, ldx, dq, codes, ldq); break;
    default: hipLaunchKernelGGL((rowwise_quant_kernel<DT, 64>), g, b, 0, st, x, rows, cols, ldx, dq, codes, ldq); break;
  }
  return rw_check("rowwise_quant");
}

}  // namespace
}  // namespace rp

using namespace rp;

extern "C" int rp_fp8_rowwise_quantize(const void* x, int x_dtype, int64_t rows, int64_t cols,
                                       int64_t ldx, float* dequant_out, uint8_t* codes,
                                       int64_t ldq, void* stream) {
  if (!x || !dequant_out || !codes) {
    rp_set_error("rowwise_quantize: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (x_dtype != RP_DTYPE_BF16 && x_dtype != RP_DTYPE_F16) {
    rp_set_error("rowwise_quantize: unknown input dtype %d", x_dtype);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (rows <= 0 || cols <= 0 || ldx < cols || ldq < cols) {
    rp_set_error("rowwise_quantize: bad sizes rows=%lld cols=%lld ldx=%lld ldq=%lld",
                 (long long)rows, (long long)cols, (long long)ldx, (long long)ldq);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (cols % 8 != 0 || ldx % 8 != 0 || ldq % 8 != 0 ||
      reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(codes) % 8 != 0) {
    rp_set_error("rowwise_quantize: needs cols, ldx, ldq multiples of 8, x 16-byte and codes "
                 "8-byte aligned");
    return RP_ERR_UNSUPPORTED;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  if (x_dtype == RP_DTYPE_F16)
    return launch_rowwise<kInF16>(xp, rows, cols, ldx, dequant_out, codes, ldq, st);
  return launch_rowwise<kInBf16>(xp, rows, cols, ldx, dequant_out, codes, ldq, st);
}

extern "C" int rp_transpose16(const void* src, void* dst, int64_t batch, int64_t R, int64_t C,
                              int64_t lds, int64_t ldd, int64_t bs, int64_t bd, void* stream) {
  if (!src || !dst || batch <= 0 || R <= 0 || C <= 0 || lds < C || ldd < R) {
    rp_set_error("transpose16: bad arguments");
    return RP_ERR_INVALID_ARGUMENT;
  }
  const dim3 grid((unsigned)((C + 63) / 64), (unsigned)((R + 63) / 64), (unsigned)batch);
  if ((R + 63) / 64 > 65535 || batch > 65535 || (C + 63) / 64 > 0x7fffffff) {
    rp_set_error("transpose16: matrix or batch too large");
    return RP_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL(transpose16_kernel, grid, dim3(kRThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), R, C, lds, ldd,
                     bs, bd);
  return rw_check("transpose16");
}

extern "C" int rp_fp8_softmax_rowwise_quantize(const void* scores, int64_t rows, int64_t cols,
                                               int64_t lds, int64_t sq, int causal, float scale,
                                               float* dequant_out, uint8_t* codes, int64_t ldq,
                                               void* stream) {
  if (!scores || !dequant_out || !codes) {
    rp_set_error("softmax_rowwise_quantize: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (rows <= 0 || cols <= 0 || lds < cols || ldq < cols || sq <= 0 || !(scale == scale)) {
    rp_set_error("softmax_rowwise_quantize: bad arguments");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (cols % 2 != 0 || lds % 2 != 0 || ldq % 2 != 0 ||
      reinterpret_cast<uintptr_t>(scores) % 4 != 0 || reinterpret_cast<uintptr_t>(codes) % 2 != 0) {
    rp_set_error("softmax_rowwise_quantize: needs even cols, lds, ldq and aligned rows");
    return RP_ERR_UNSUPPORTED;
  }
  if (rows > 0x7fffffff) {
    rp_set_error("softmax_rowwise_quantize: too many rows");
    return RP_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL(softmax_rowquant_kernel, dim3((unsigned)rows), dim3(kRThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(scores), cols,
                     lds, sq, causal ? 1 : 0, scale, dequant_out, codes, ldq);
  return rw_check("softmax_rowquant");
}
