// FP8 scaled GEMM for gfx950: C (M, N) bf16 = bf16(fp32(A8 . B8) * a_scale*b_scale).
//
// Semantics follow kernels/hip/fp8_attn/fp8_gemm.hip:79-156 of the reference
// (fp32 accumulation, the product of the two scales applied once to the
// accumulator, round-to-nearest-even bf16 output), on OCP e4m3fn operands.
// The reference kernel is one wave per 16x16 tile with strided operand
// gathers and no LDS; this one is an LDS-staged, double-buffered block GEMM
// on v_mfma_f32_16x16x128_f8f6f4:
//
// * Both operands are K-contiguous rows (A8 (M, K), B8 transposed (N, K)),
//   so every MFMA operand is 32 contiguous bytes per lane.
// * The MFMA computes C^T tiles (A operand = rows of B^T, B operand = rows of
//   A): the accumulator then gives each lane 4 consecutive output columns
//   of one row, stored as one 8-byte write.
// * Workgroup = 4 waves in a 2 x 2 grid over a BM x BN block tile; each
//   K step of 128 stages BM + BN rows of 128 bytes in LDS (XOR-swizzled
//   16-byte chunks) while the next step is fetched into registers.
// * Workgroups are remapped so those resident on one XCD cover a compact
//   patch of C and share operand rows in that XCD's L2.

#include "rp_common.h"

namespace rp {
namespace {

constexpr int kGThreads = 256;
constexpr int kKStep = 128;

struct GemmArgs {
  const uint8_t* a;
  const uint8_t* bt;
  uint16_t* c;
  int64_t M, N, K, lda, ldb, ldc;
  float a_scale, b_scale;
  const float* a_dev;
  const float* b_dev;
  int tiles_m, tiles_n;
};

__device__ __forceinline__ f32x4 mfma_16x16x128(const i32x8& a, const i32x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ i32x8 cat8(const i32x4& lo, const i32x4& hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// BM x BN block tile, waves arranged 2 x 2, each wave (BM/2) x (BN/2).
template <int BM, int BN>
struct GGeo {
  static constexpr int WM = BM / 2, WN = BN / 2;
  static constexpr int TM = WM / 16, TN = WN / 16;   // 16x16 tiles per wave
  static constexpr int A_BYTES = BM * kKStep;
  static constexpr int B_BYTES = BN * kKStep;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int A_LOADS = A_BYTES / 16 / kGThreads;
  static constexpr int B_LOADS = B_BYTES / 16 / kGThreads;
};

template <int BM, int BN>
__device__ __forceinline__ void gemm_load(const GemmArgs& g, int64_t m0, int64_t n0, int64_t k0,
                                          int tid, i32x4 (&sa)[GGeo<BM, BN>::A_LOADS],
                                          i32x4 (&sb)[GGeo<BM, BN>::B_LOADS]) {
  using G = GGeo<BM, BN>;
#pragma unroll
  for (int n = 0; n < G::A_LOADS; ++n) {
    const int ci = tid + kGThreads * n;
    const int r = ci >> 3, c = ci & 7;
    const int64_t row = min(m0 + r, g.M - 1);
    const int64_t k = k0 + c * 16;
    sa[n] = k < g.K ? *reinterpret_cast<const i32x4*>(g.a + row * g.lda + k)
                    : i32x4{0, 0, 0, 0};
  }
#pragma unroll
  for (int n = 0; n < G::B_LOADS; ++n) {
    const int ci = tid + kGThreads * n;
    const int r = ci >> 3, c = ci & 7;
    const int64_t row = min(n0 + r, g.N - 1);
    const int64_t k = k0 + c * 16;
    sb[n] = k < g.K ? *reinterpret_cast<const i32x4*>(g.bt + row * g.ldb + k)
                    : i32x4{0, 0, 0, 0};
  }
}

template <int BM, int BN>
__device__ __forceinline__ void gemm_store(uint8_t* st, int tid,
                                           const i32x4 (&sa)[GGeo<BM, BN>::A_LOADS],
                                           const i32x4 (&sb)[GGeo<BM, BN>::B_LOADS]) {
  using G = GGeo<BM, BN>;
  uint8_t* bl = st + G::A_BYTES;
#pragma unroll
  for (int n = 0; n < G::A_LOADS; ++n) {
    const int ci = tid + kGThreads * n;
    const int r = ci >> 3, c = ci & 7;
    *reinterpret_cast<i32x4*>(st + r * kKStep + ((c ^ (r & 7)) << 4)) = sa[n];
  }
#pragma unroll
  for (int n = 0; n < G::B_LOADS; ++n) {
    const int ci = tid + kGThreads * n;
    const int r = ci >> 3, c = ci & 7;
    *reinterpret_cast<i32x4*>(bl + r * kKStep + ((c ^ (r & 7)) << 4)) = sb[n];
  }
}

__device__ __forceinline__ i32x8 lds_operand(const uint8_t* tile, int row, int lg) {
  const int sw = row & 7;
  const uint8_t* p = tile + row * kKStep;
  return cat8(*reinterpret_cast<const i32x4*>(p + (((2 * lg) ^ sw) << 4)),
              *reinterpret_cast<const i32x4*>(p + (((2 * lg + 1) ^ sw) << 4)));
}

template <int BM, int BN>
__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
void gemm_kernel(GemmArgs g) {
  using G = GGeo<BM, BN>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * G::STAGE];

  // XCD-aware remap, then column-major walk over 8-tile-tall bands of C so
  // consecutive workgroups reuse the same B^T rows.
  const int nwork = g.tiles_m * g.tiles_n;
  const int w = blockIdx.x;
  const int per = nwork >> 3, rem = nwork & 7;
  const int xcd = w & 7;
  const int L = xcd * per + min(xcd, rem) + (w >> 3);
  constexpr int kBand = 8;
  const int band_tiles = kBand * g.tiles_n;
  const int band = L / band_tiles;
  const int in_band = L - band * band_tiles;
  const int band_h = min(kBand, g.tiles_m - band * kBand);
  const int tm = band * kBand + in_band % band_h;
  const int tn = in_band / band_h;
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t n0 = (int64_t)tn * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;

  f32x4 acc[G::TN][G::TM];
#pragma unroll
  for (int j = 0; j < G::TN; ++j)
#pragma unroll
    for (int i = 0; i < G::TM; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  i32x4 sa[G::A_LOADS];
  i32x4 sb[G::B_LOADS];
  const int nk = (int)((g.K + kKStep - 1) / kKStep);
  gemm_load<BM, BN>(g, m0, n0, 0, tid, sa, sb);
  gemm_store<BM, BN>(smem, tid, sa, sb);
  __syncthreads();

  for (int kk = 0; kk < nk; ++kk) {
    const int st = kk & 1;
    const bool more = kk + 1 < nk;
    if (more) gemm_load<BM, BN>(g, m0, n0, (int64_t)(kk + 1) * kKStep, tid, sa, sb);
    const uint8_t* al = smem + st * G::STAGE;
    const uint8_t* bl = al + G::A_BYTES;
    i32x8 bop[G::TN];
#pragma unroll
    for (int j = 0; j < G::TN; ++j) bop[j] = lds_operand(bl, wn * G::WN + 16 * j + li, lg);
#pragma unroll
    for (int i = 0; i < G::TM; ++i) {
      const i32x8 aop = lds_operand(al, wm * G::WM + 16 * i + li, lg);
#pragma unroll
      for (int j = 0; j < G::TN; ++j) acc[j][i] = mfma_16x16x128(bop[j], aop, acc[j][i]);
    }
    if (more) gemm_store<BM, BN>(smem + (st ^ 1) * G::STAGE, tid, sa, sb);
    __syncthreads();
  }

  const float scale = (g.a_dev ? *g.a_dev : g.a_scale) * (g.b_dev ? *g.b_dev : g.b_scale);
#pragma unroll
  for (int i = 0; i < G::TM; ++i) {
    const int64_t m = m0 + wm * G::WM + 16 * i + li;
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < G::TN; ++j) {
      const int64_t n = n0 + wn * G::WN + 16 * j + 4 * lg;
      if (n >= g.N) continue;
      const f32x4 v = acc[j][i];
      uint2 pk;
      pk.x = f32_to_bf16_bits(v[0] * scale) | (f32_to_bf16_bits(v[1] * scale) << 16);
      pk.y = f32_to_bf16_bits(v[2] * scale) | (f32_to_bf16_bits(v[3] * scale) << 16);
      *reinterpret_cast<uint2*>(g.c + m * g.ldc + n) = pk;
    }
  }
}

// 64 x 64 byte-tile transpose through LDS.
__global__ __launch_bounds__(256) void transpose_u8_kernel(const uint8_t* src, uint8_t* dst,
                                                           int64_t R, int64_t C, int64_t lds,
                                                           int64_t ldd) {
  __shared__ uint8_t tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int r = i >> 6, c = i & 63;
    if (r0 + r < R && c0 + c < C) tile[r][c] = src[(r0 + r) * lds + c0 + c];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int c = i >> 6, r = i & 63;
    if (r0 + r < R && c0 + c < C) dst[(c0 + c) * ldd + r0 + r] = tile[r][c];
  }
}

template <int BM, int BN>
int launch_gemm(GemmArgs g, hipStream_t st) {
  g.tiles_m = (int)((g.M + BM - 1) / BM);
  g.tiles_n = (int)((g.N + BN - 1) / BN);
  const int64_t nwork = (int64_t)g.tiles_m * g.tiles_n;
  if (nwork > 0x7fffffff) {
    rp_set_error("gemm: grid too large");
    return RP_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL((gemm_kernel<BM, BN>), dim3((unsigned)nwork), dim3(kGThreads), 0, st, g);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    rp_set_error("gemm: launch failed: %s", hipGetErrorString(e));
    return RP_ERR_LAUNCH;
  }
  return RP_OK;
}

}  // namespace
}  // namespace rp

using namespace rp;

extern "C" int rp_fp8_gemm(const uint8_t* a8, const uint8_t* bt8, void* c, int64_t M, int64_t N,
                           int64_t K, int64_t lda, int64_t ldb, int64_t ldc, float a_scale,
                           float b_scale, const float* a_scale_dev, const float* b_scale_dev,
                           void* stream) {
  if (!a8 || !bt8 || !c) {
    rp_set_error("gemm: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (M <= 0 || N <= 0 || K <= 0 || lda < K || ldb < K || ldc < N) {
    rp_set_error("gemm: bad sizes M=%lld N=%lld K=%lld lda=%lld ldb=%lld ldc=%lld",
                 (long long)M, (long long)N, (long long)K, (long long)lda, (long long)ldb,
                 (long long)ldc);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (K % 16 != 0 || lda % 16 != 0 || ldb % 16 != 0 || N % 4 != 0 || ldc % 4 != 0) {
    rp_set_error("gemm: needs K, lda, ldb multiples of 16 and N, ldc multiples of 4");
    return RP_ERR_UNSUPPORTED;
  }
  if ((reinterpret_cast<uintptr_t>(a8) | reinterpret_cast<uintptr_t>(bt8)) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(c) % 8 != 0) {
    rp_set_error("gemm: operands must be 16-byte aligned and C 8-byte aligned");
    return RP_ERR_UNSUPPORTED;
  }
  GemmArgs g{};
  g.a = a8; g.bt = bt8; g.c = static_cast<uint16_t*>(c);
  g.M = M; g.N = N; g.K = K; g.lda = lda; g.ldb = ldb; g.ldc = ldc;
  g.a_scale = a_scale; g.b_scale = b_scale; g.a_dev = a_scale_dev; g.b_dev = b_scale_dev;
  return launch_gemm<256, 128>(g, static_cast<hipStream_t>(stream));
}

extern "C" int rp_fp8_transpose(const uint8_t* src, uint8_t* dst, int64_t R, int64_t C,
                                int64_t lds, int64_t ldd, void* stream) {
  if (!src || !dst || R <= 0 || C <= 0 || lds < C || ldd < R) {
    rp_set_error("transpose: bad arguments");
    return RP_ERR_INVALID_ARGUMENT;
  }
  dim3 grid((unsigned)((C + 63) / 64), (unsigned)((R + 63) / 64));
  if (grid.y > 65535) {
    rp_set_error("transpose: R too large");
    return RP_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL(transpose_u8_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     src, dst, R, C, lds, ldd);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    rp_set_error("transpose: launch failed: %s", hipGetErrorString(e));
    return RP_ERR_LAUNCH;
  }
  return RP_OK;
}
