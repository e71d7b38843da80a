// FP8 scaled GEMM for gfx950: C (M, N) bf16 = bf16(fp32(A8 . B8) * a_scale*b_scale).
//
// Semantics follow kernels/hip/fp8_attn/fp8_gemm.hip:79-156 of the reference
// (fp32 accumulation, the product of the two scales applied once to the
// accumulator, round-to-nearest-even bf16 output), on OCP e4m3fn operands.
// The reference kernel is one wave per 16x16 tile with strided operand
// gathers and no LDS.  Here every MFMA operand is 32 K-contiguous bytes per
// lane, and the MFMA computes C^T tiles (A operand = rows of B^T, B operand
// = rows of A): the accumulator gives each lane 4 consecutive output columns
// of one row, stored as one 8-byte write.  B comes in either layout:
// transposed, (N, K) rows (RP_B_NK: K-contiguous like A), or as the
// reference takes it, (K, N) row-major (RP_B_KN).  A (K, N) slice is staged
// in LDS as it lies in memory -- K rows of N bytes -- and the B^T operand is
// read from it with ds_read_b64_tr_b8, the gfx950 LDS transpose read (see
// kn_operand), so neither layout costs a transpose pass.  Two kernels:
//
// * gemm256_kernel (K a multiple of 64, the production shapes): 256 x 256
//   block tiles on v_mfma_f32_32x32x64_f8f6f4, four waves of 128 x 128 with
//   their accumulators in AGPRs, operands streamed by direct-to-LDS loads
//   through a ring of five 32 KiB slots (the A and B^T halves of 128-byte K
//   slices), each slice loaded two slices ahead of its use.
// * gemm_kernel (any K multiple of 16, any (K, N) B): 256 x 128 block tiles
//   on v_mfma_f32_16x16x128_f8f6f4, operands staged through VGPRs into a
//   double-buffered, XOR-swizzled LDS tile, K tail zero-filled; a (K, N) B
//   is gathered byte by byte (the fallback for shapes the large-tile kernel
//   does not take).
//
// Both remap workgroups so that those resident on one XCD cover a compact
// patch of C and share operand rows in that XCD's L2.

#include <type_traits>

#include "rp_common.h"

namespace rp {
namespace {

constexpr int kGThreads = 256;
constexpr int kKStep = 128;

struct GemmArgs {
  const uint8_t* a;
  const uint8_t* bt;
  uint16_t* c;
  const uint16_t* bias;   // bf16 [N] added in the epilogue, or null
  int64_t M, N, K, lda, ldb, ldc;
  float a_scale, b_scale;
  const float* a_dev;
  const float* b_dev;
  int tiles_m, tiles_n;
  int b_kn;   // 1: B is (K, N) row-major, row stride ldb (RP_B_KN)
  // row-wise scales (rp_fp8_gemm_rowwise): C = bf16((acc * row_scale[m]) *
  // col_scale[n]) instead of the per-tensor scales; null otherwise
  const float* row_scale;
  const float* col_scale;
  // batched launches (blockIdx.y = batch): strides of A and B (bytes), C
  // (elements) and the two scale vectors (elements)
  int64_t bsa, bsb, bsc, bsr, bss;
  // rp_fp8_linear_balanced (one batch): the last pool_r tiles of every
  // XCD's share of gemm256_kernel's tiles are handed out through this
  // counter, zeroed before the launch; null: every tile in place
  unsigned* item_counter;
  int pool_r;
};

// The batch a workgroup works on: offsets every operand pointer (one batch
// unless blockIdx.y > 0).
__device__ __forceinline__ void gemm_batch(GemmArgs& g) {
  const int64_t z = blockIdx.y;
  g.a += z * g.bsa;
  g.bt += z * g.bsb;
  g.c += z * g.bsc;
  if (g.row_scale) g.row_scale += z * g.bsr;
  if (g.col_scale) g.col_scale += z * g.bss;
}

// Row-wise epilogue values: fp32(fp32(acc * row scale) * column scale), then
// the bias as in epi4.
__device__ __forceinline__ void epi4_rows(bool has_bias, uint2 bb, float sm, const float4& sn,
                                          float v0, float v1, float v2, float v3, float (&o)[4]) {
  o[0] = v0 * sm; o[1] = v1 * sm; o[2] = v2 * sm; o[3] = v3 * sm;
  asm("" : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]));
  o[0] *= sn.x; o[1] *= sn.y; o[2] *= sn.z; o[3] *= sn.w;
  if (has_bias) {
    asm("" : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]));
    o[0] += bf16_to_f32(bb.x & 0xffffu);
    o[1] += bf16_to_f32(bb.x >> 16);
    o[2] += bf16_to_f32(bb.y & 0xffffu);
    o[3] += bf16_to_f32(bb.y >> 16);
  }
}

// Bias values of the 4 columns n..n+3 (bf16 pairs), or zeros past N.  Every
// thread loads its columns before the first output store: the bias and C are
// both bf16 pointers, so a load after a store would have to wait for it.
__device__ __forceinline__ uint2 bias4(const GemmArgs& g, int64_t n) {
  return n < g.N ? *reinterpret_cast<const uint2*>(g.bias + n) : make_uint2(0u, 0u);
}

// Epilogue value: t = fp32(acc * scale), then fp32(t + bias[n]) when there
// is a bias -- two roundings (the empty asm keeps the compiler from fusing
// them into one FMA), the fp32 result a bf16 nn.Linear rounds once.
__device__ __forceinline__ void epi4(bool has_bias, uint2 bb, float scale, float v0, float v1,
                                     float v2, float v3, float (&o)[4]) {
  o[0] = v0 * scale; o[1] = v1 * scale; o[2] = v2 * scale; o[3] = v3 * scale;
  if (has_bias) {
    asm("" : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]));
    o[0] += bf16_to_f32(bb.x & 0xffffu);
    o[1] += bf16_to_f32(bb.x >> 16);
    o[2] += bf16_to_f32(bb.y & 0xffffu);
    o[3] += bf16_to_f32(bb.y >> 16);
  }
}

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

// Chunk ci of a B^T tile: row r (an N row of the tile), 16-byte K granule c.
// For a (K, N) B the 128 rows of a chunk group are consecutive lanes, so the
// byte gathers of one wave read consecutive N columns of each K row.
template <int BN, bool KN>
__device__ __forceinline__ void b_chunk(int ci, int& r, int& c) {
  if constexpr (KN) {
    r = ci % BN;
    c = ci / BN;
  } else {
    r = ci >> 3;
    c = ci & 7;
  }
}

template <int BM, int BN, bool KN>
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
    int r, c;
    b_chunk<BN, KN>(ci, r, c);
    const int64_t row = min(n0 + r, g.N - 1);
    const int64_t k = k0 + c * 16;
    if constexpr (KN) {
      // column `row` of B, K rows k .. k+15 (zero past K), one byte each
      uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (k + e < g.K) w[e >> 2] |= (uint32_t)g.bt[(k + e) * g.ldb + row] << (8 * (e & 3));
      sb[n] = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    } else {
      sb[n] = k < g.K ? *reinterpret_cast<const i32x4*>(g.bt + row * g.ldb + k)
                      : i32x4{0, 0, 0, 0};
    }
  }
}

template <int BM, int BN, bool KN>
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
    int r, c;
    b_chunk<BN, KN>(ci, r, c);
    *reinterpret_cast<i32x4*>(bl + r * kKStep + ((c ^ (r & 7)) << 4)) = sb[n];
  }
}

__device__ __forceinline__ i32x8 lds_operand(const uint8_t* tile, int row, int lg) {
  const int sw = row & 7;
  const uint8_t* p = tile + row * kKStep;
  return cat8(*reinterpret_cast<const i32x4*>(p + (((2 * lg) ^ sw) << 4)),
              *reinterpret_cast<const i32x4*>(p + (((2 * lg + 1) ^ sw) << 4)));
}

template <int BM, int BN, bool KN>
__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
void gemm_kernel(GemmArgs g) {
  using G = GGeo<BM, BN>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * G::STAGE];

  gemm_batch(g);
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
  gemm_load<BM, BN, KN>(g, m0, n0, 0, tid, sa, sb);
  gemm_store<BM, BN, KN>(smem, tid, sa, sb);
  __syncthreads();

  for (int kk = 0; kk < nk; ++kk) {
    const int st = kk & 1;
    const bool more = kk + 1 < nk;
    if (more) gemm_load<BM, BN, KN>(g, m0, n0, (int64_t)(kk + 1) * kKStep, tid, sa, sb);
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
    if (more) gemm_store<BM, BN, KN>(smem + (st ^ 1) * G::STAGE, tid, sa, sb);
    __syncthreads();
  }

  const float scale = g.row_scale ? 1.0f
                    : (g.a_dev ? *g.a_dev : g.a_scale) * (g.b_dev ? *g.b_dev : g.b_scale);
  const bool has_bias = g.bias != nullptr;
  uint2 bb[G::TN];
#pragma unroll
  for (int j = 0; j < G::TN; ++j)
    bb[j] = has_bias ? bias4(g, n0 + wn * G::WN + 16 * j + 4 * lg) : make_uint2(0u, 0u);
#pragma unroll
  for (int i = 0; i < G::TM; ++i) {
    const int64_t m = m0 + wm * G::WM + 16 * i + li;
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < G::TN; ++j) {
      const int64_t n = n0 + wn * G::WN + 16 * j + 4 * lg;
      if (n >= g.N) continue;
      const f32x4 v = acc[j][i];
      float o[4];
      if (g.row_scale)
        epi4_rows(has_bias, bb[j], g.row_scale[m], *reinterpret_cast<const float4*>(g.col_scale + n),
                  v[0], v[1], v[2], v[3], o);
      else
        epi4(has_bias, bb[j], scale, v[0], v[1], v[2], v[3], o);
      uint2 pk;
      pk.x = f32_to_bf16_bits(o[0]) | (f32_to_bf16_bits(o[1]) << 16);
      pk.y = f32_to_bf16_bits(o[2]) | (f32_to_bf16_bits(o[3]) << 16);
      *reinterpret_cast<uint2*>(g.c + m * g.ldc + n) = pk;
    }
  }
}


// ------------------------------------------------------------- large tiles
// The kernel for K a multiple of 64: 256 x 256 block tiles on
// v_mfma_f32_32x32x64_f8f6f4, four waves (one per SIMD) of 128 x 128 each,
// accumulators in AGPRs.  Operands reach LDS by global_load_lds_dwordx4 (no
// VGPR staging) in K slices of 128 bytes -- eight lanes read one row's whole
// cache line -- through a ring of five 32 KiB slots, each holding the A or
// the B^T part of one slice: while slice k is multiplied, slice k+1 lands and
// slice k+2 loads, its A part during the first half of slice k and its B^T
// part during the second, so the loads leave at an even rate (issuing a
// whole slice at once measured 4% slower).  One wait and barrier per slice;
// all but the last three slices run a branch-free copy of the sub-step.
// Each slice is two MFMA depths (sub-slices of 64 bytes); operands are
// double-buffered in registers a sub-slice ahead.  LDS rows are unpadded;
// the eight 16-byte granules of a row are XOR-swizzled by (row >> 1) & 7, so
// the 16-lane ds_read_b128 groups are conflict-free.  The MFMA computes C^T
// tiles (A operand = rows of B^T, B operand = rows of A); the epilogue
// re-stages the bf16 tile through LDS so that each output row leaves as one
// 256-byte run.
constexpr int kG2Threads = 256;
constexpr int kG2Tile = 256;                        // BM = BN
constexpr int kG2K = 128;                           // K bytes per slice (two MFMA depths)
constexpr int kG2Sub = 64;                          // K bytes per MFMA (a sub-slice)
constexpr int kG2Pitch = kG2K;                      // LDS row pitch (no pad)
constexpr int kG2Half = kG2Tile * kG2Pitch;         // A (or B^T) part of a stage
constexpr int kG2Slots = 5;                         // LDS ring of slice halves (A or B^T)
constexpr int kG2Loads = 2 * kG2Half / 1024 / 4;    // 1 KiB loads per wave per slice
constexpr int kG2ALoads = kG2Half / 1024 / 4;       // of which A
static_assert(kG2Half % 4096 == 0, "A and B^T parts split evenly over the waves");
static_assert(kG2Slots * kG2Half <= 160 * 1024, "LDS");

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 16 bytes global -> LDS: lane i reads base + voff_i and lands at
// lds_block + 16*i.  base (64-bit) and lds_block are wave-uniform and go in
// SGPRs ("saddr" form: no per-lane 64-bit address arithmetic per load).
// Inline asm keeps the load out of the compiler's waitcnt bookkeeping,
// which would otherwise order every later ds_read behind it; the kernel
// waits for its loads explicitly (vmcnt) before the barrier that precedes
// their first read.  Nothing else in this kernel uses M0.  (The buffer-
// resource form of this load measured 4-8% slower at the Wan FFN shape.)
__device__ __forceinline__ void g2_gload_lds16_s(const void* base, uint32_t voff,
                                                 uint32_t lds_block) {
  // readfirstlane states the uniformity where the compiler cannot prove it
  // (and folds away where it can).  It returns int: each half is widened
  // through uint32_t, since a sign-extended low word would corrupt the
  // high half of the address.
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
  const uint32_t m0v = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_block);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(reinterpret_cast<const void*>(sb)), "s"(m0v)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(N): all but this wave's N most recent loads have landed.
template <int N>
__device__ __forceinline__ void g2_wait_vmem() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__device__ __forceinline__ f32x16 mfma_32x32x64(const i32x8& a, const i32x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ i32x8 g2_op(const uint8_t* p, int h0, int h1) {
  return cat8(*reinterpret_cast<const i32x4*>(p + h0), *reinterpret_cast<const i32x4*>(p + h1));
}

// two fp32 -> packed bf16 with v_cvt_pk_bf16_f32 (round to nearest even)
__device__ __forceinline__ uint32_t g2_pack_bf16(float lo, float hi) {
  // as one vector conversion: value by value, the compiler converts each
  // alone and packs them with an extra or
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

struct G2Ops {
  i32x8 a[4], b[4];
};

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b8: each group of 16 lanes reads an 8 x 16 byte block --
// lane i supplies the address of bytes 8(i%2) .. 8(i%2)+7 of row i/2 -- and
// lane i receives column i of it: byte j from row j.  (Measured on gfx950:
// lane l, byte j <- lane 16(l/16) + 2j + (l%16)/8, byte l%8.)
__device__ __forceinline__ i32x2 lds_tr8(uint32_t lds_addr) {
  typedef __attribute__((address_space(3))) i32x2* lds_i32x2_p;
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2_p)(uintptr_t)lds_addr);
}

// B^T operand from a (K, N) slice in LDS (RP_B_KN).  Slice rows are K (256
// bytes of N each); the 16 N granules of row r sit at slots g ^ 2(r & 7).
// Lane l needs N column n = l % 32 of its 32-row block and K bytes
// 32(l / 32) .. +31 of the sub-slice: four transpose reads of 8 K rows each.
// Lane i of a 16-lane group points at row k8 + i/2 (k8 a multiple of 8, so
// r & 7 = i/2), granule g of columns 16((l / 16) % 2) .. +15 of the block, byte
// 8(i % 2): `base` carries the per-lane part, the rest is immediate.  The
// slots g ^ {0, 2, .., 14} of one group's eight rows and g+1 ^ {...} of its
// neighbour cover all sixteen 16-byte bank groups once: conflict-free.
__device__ __forceinline__ i32x8 kn_operand(uint32_t base) {
  const i32x2 r0 = lds_tr8(base), r1 = lds_tr8(base + 8 * kG2Tile);
  const i32x2 r2 = lds_tr8(base + 16 * kG2Tile), r3 = lds_tr8(base + 24 * kG2Tile);
  return i32x8{r0.x, r0.y, r1.x, r1.y, r2.x, r2.y, r3.x, r3.y};
}

// Epilogue modes of gemm256_kernel, fixed at compile time: per-tensor
// scales; per-tensor scales and a bias; row-wise scales (bias optional).
constexpr int kEpiPlain = 0, kEpiBias = 1, kEpiRows = 2;

template <bool KN, int EPI>
__global__ __launch_bounds__(kG2Threads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm256_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kG2Slots * kG2Half];
  const uint32_t smem_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)smem;

  gemm_batch(g);
  // XCD-aware remap, then a column-major walk over 4-tile-tall bands of C:
  // the 32 workgroups resident on one XCD cover a 4 x 8 patch and share
  // its A and B^T rows in that XCD's L2 (4-tall measured best of 1, 2, 4,
  // 8 and 16 at the C4 shape).
  const int nwork = g.tiles_m * g.tiles_n;
  const int w = blockIdx.x;
  const int per = nwork >> 3, rem = nwork & 7;
  const int xcd = w & 7;
  int L = xcd * per + min(xcd, rem) + (w >> 3);
  if (g.item_counter != nullptr) {
    // XCDs run at different speeds: every XCD runs its share of tiles but
    // the last pool_r (pool_r + 1 for the first rem shares) in place, and
    // the tiles so left go, in share order, to whichever XCD asks first
    const int in_place = per - g.pool_r;
    if ((w >> 3) >= in_place) {
      // the operand ring is full: its first bytes pass the item on, read by
      // every thread before the first loads can land there
      int* const item = reinterpret_cast<int*>(smem);
      if (threadIdx.x == 0) *item = (int)atomicAdd(g.item_counter, 1u);
      __syncthreads();
      const int p = *item;
      __syncthreads();
      if (p >= 8 * g.pool_r + rem) return;   // every tile is taken
      const int big = rem * (g.pool_r + 1);    // pooled tiles of the larger shares
      const int x = p < big ? p / (g.pool_r + 1) : rem + (p - big) / g.pool_r;
      const int j = p < big ? p - x * (g.pool_r + 1) : (p - big) - (x - rem) * g.pool_r;
      L = x * per + min(x, rem) + in_place + j;
    }
  }
  constexpr int kBand = 4;
  const int band_tiles = kBand * g.tiles_n;
  const int band = L / band_tiles;
  const int in_band = L - band * band_tiles;
  const int band_h = min(kBand, g.tiles_m - band * kBand);
  const int tm = band * kBand + in_band % band_h;
  const int tn = in_band / band_h;
  const int64_t m0 = (int64_t)tm * kG2Tile;
  const int64_t n0 = (int64_t)tn * kG2Tile;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31, lg = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;

  // This lane's direct-to-LDS loads: load n fills KiB block (n % 8) * 4 +
  // wave of a slot; loads 0..7 the A part, 8..15 the B^T part.
  // A and (N, K) B^T: eight consecutive lanes read one row's 128-byte K slice
  // (a whole cache line); LDS granule `slot` of row r holds K granule
  // slot ^ ((r >> 1) & 7).  Rows past M or N re-read the last row (their
  // results are not stored).
  // (K, N) B: sixteen consecutive lanes read one K row's 256 N bytes of the
  // tile; LDS granule `slot` of row r holds N granule slot ^ 2(r & 7), and
  // granules past N re-read the last one inside N (N % 16 == 0).
  const uint8_t* abase = g.a + m0 * g.lda;
  const uint8_t* bbase = KN ? g.bt + n0 : g.bt + n0 * g.ldb;
  uint32_t gofs[kG2Loads];
#pragma unroll
  for (int n = 0; n < kG2Loads; ++n) {
    const int blk = n * 4 + wave;
    const bool is_a = n < kG2ALoads;
    const int p = (is_a ? blk : blk - kG2Half / 1024) * kWave + lane;
    if (KN && !is_a) {
      const int row = p >> 4, slot = p & 15;
      const int last = (int)min((g.N - n0) >> 4, (int64_t)16) - 1;
      const int gran = min(slot ^ (2 * (row & 7)), last);
      gofs[n] = (uint32_t)((int64_t)row * g.ldb + gran * 16);
      continue;
    }
    const int row = p >> 3, slot = p & 7;
    const int s16 = (slot ^ ((row >> 1) & 7)) * 16;
    if (is_a) {
      const int64_t r = min(m0 + row, g.M - 1) - m0;
      gofs[n] = (uint32_t)(r * g.lda + s16);
    } else {
      const int64_t r = min(n0 + row, g.N - 1) - n0;
      gofs[n] = (uint32_t)(r * g.ldb + s16);
    }
  }
  // K in 64-byte sub-slices; slices are pairs of them.  With K % 128 == 64
  // the last slice is a half: the lanes that would fill its second sub-slice
  // re-read in-bounds bytes of the first (K granules 0..3 of the row for A
  // and B^T, K rows 0..63 for a (K, N) B), and that sub-slice is never used.
  const int nsub = (int)(g.K / kG2Sub);
  const int nslice = (nsub + 1) >> 1;
  const int half_tail = nsub & 1;
  // bit 2 of this lane's K granule is (slot bit 2) ^ (block parity), and a
  // block's parity is the wave's: the same for all of its loads
  const uint32_t tail_back = (uint32_t)(((lane >> 2) ^ wave) & 1) * 64;
  // (K, N) B: loads n >= kG2ALoads + 4 fill K rows 64..127 of the slice
  const uint32_t tail_back_kn = (uint32_t)(64 * g.ldb);
  // load n of slice kk into `slot` (FULL: kk is not a half tail slice)
  auto issue = [&](int n, int kk, int slot, auto full_c) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full_c)::value;
    uint32_t off = gofs[n];
    const bool is_a = n < kG2ALoads;
    if (!FULL && half_tail && kk == nslice - 1) {
      if (KN && !is_a) off -= n >= kG2ALoads + 4 ? tail_back_kn : 0u;
      else off -= tail_back;
    }
    const uint8_t* src = is_a ? abase + (int64_t)kk * kG2K
                              : bbase + (int64_t)kk * kG2K * (KN ? g.ldb : 1);
    g2_gload_lds16_s(src, off,
                     smem_lds + (uint32_t)(slot * kG2Half + ((n % kG2ALoads) * 4 + wave) * 1024));
  };

  // Per-lane operand offsets inside a slot: row lq of each 32-row block,
  // K granules 4h + 2lg and 4h + 2lg + 1 of sub-slice h at their swizzled
  // slots (the swizzle term (row >> 1) & 7 depends on lq only, as block
  // bases are multiples of 32 rows).  Sixteen consecutive lanes then hit
  // sixteen distinct 16-byte bank groups.
  const int swz = (lq >> 1) & 7;
  const int h00 = ((2 * lg) ^ swz) * 16, h01 = ((2 * lg + 1) ^ swz) * 16;
  const int h10 = ((4 + 2 * lg) ^ swz) * 16, h11 = ((4 + 2 * lg + 1) ^ swz) * 16;
  const int a_off = (wm * 128 + lq) * kG2Pitch;
  const int b_off = (wn * 128 + lq) * kG2Pitch;
  // (K, N) B: per-lane LDS offsets of the four B^T operands' transpose reads
  // (see kn_operand); sub-slice h adds 64 K rows, an immediate
  uint32_t kn_off[4];
  {
    const int i = lane & 15;
    const int row = 32 * lg + (i >> 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gr = 8 * wn + 2 * j + ((lane >> 4) & 1);
      kn_off[j] = (uint32_t)(row * kG2Tile + ((gr ^ (i & 14)) << 4) + 8 * (i & 1));
    }
  }
  auto b_op = [&](const uint8_t* st, int j, int h, int c0, int c1) __attribute__((always_inline)) {
    if constexpr (KN) {
      const uint32_t st_lds = smem_lds + (uint32_t)(st - smem);
      return kn_operand(st_lds + kn_off[j] + (uint32_t)(64 * h * kG2Tile));
    } else {
      return g2_op(st + b_off + 32 * j * kG2Pitch, c0, c1);
    }
  };
  auto wrap = [](int x) { return x >= kG2Slots ? x - kG2Slots : x; };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  // Slice kk's A part sits in slot 2kk % 5 and its B^T part in slot
  // (2kk + 1) % 5.  prologue: slices 0 and 1 in flight, wait for slice 0,
  // read sub-slice 0
#pragma unroll
  for (int n = 0; n < kG2Loads; ++n) issue(n, 0, n < kG2ALoads ? 0 : 1, std::false_type{});
  if (nslice > 1) {
#pragma unroll
    for (int n = 0; n < kG2Loads; ++n) issue(n, 1, n < kG2ALoads ? 2 : 3, std::false_type{});
    g2_wait_vmem<kG2Loads>();
  } else {
    g2_wait_vmem<0>();
  }
  __syncthreads();
  G2Ops o0, o1;
#pragma unroll
  for (int i = 0; i < 4; ++i) o0.a[i] = g2_op(smem + a_off + 32 * i * kG2Pitch, h00, h01);
#pragma unroll
  for (int j = 0; j < 4; ++j) o0.b[j] = b_op(smem + kG2Half, j, 0, h00, h01);

  // Sub-step (kk, H): 16 MFMAs on `cur` (sub-slice 2kk + H) with the operand
  // reads of the next sub-slice into `nxt` and eight loads of slice kk + 2
  // spread between them: its A part in (kk, 0), into the slot of slice
  // kk - 1's B^T part, and its B^T part in (kk, 1), into the slot of slice
  // kk's A part -- an even stream of loads, each with two to three
  // sub-steps to land.  Sub-step (kk, 1) begins with the slice's one wait
  // and barrier: slice kk + 1 (read from here on) has landed, and every wave
  // has finished reading slice kk.
  // STEADY sub-steps (kk + 2 < nslice - 1) load a full slice and read a
  // next sub-slice unconditionally: no branches between their MFMAs.
  // The next sub-slice's operands are read in the first eight steps, and a
  // scheduling fence after every step keeps that order: the barrier's fence
  // waits for every LDS read the wave has in flight, and with one wave per
  // SIMD that wait idles the matrix core.  (Left to the scheduler, the reads
  // went out in a burst just before the barrier and twelve of the
  // sub-step's MFMAs after it: C4 3.83 ms against 3.69-3.70 ms fenced,
  // alternating on one box.)
  int sa = 0;   // slot of slice kk's A part
  auto sub = [&](int kk, auto Hc, auto Sc, G2Ops& cur, G2Ops& nxt) __attribute__((always_inline)) {
    constexpr int H = decltype(Hc)::value;
    constexpr bool STEADY = decltype(Sc)::value;
    const int u = 2 * kk + H;
    const bool more = STEADY || u + 1 < nsub;
    const bool load = STEADY || kk + 2 < nslice;
    if (H == 1) {
      // in flight behind slice kk + 1: the A part of slice kk + 2
      if (more) {
        if (load) g2_wait_vmem<kG2ALoads>();
        else g2_wait_vmem<0>();
      }
      __syncthreads();
    }
    // the next sub-slice: (kk, 1) when H == 0, else (kk + 1, 0)
    const uint8_t* sta = smem + (H == 0 ? sa : wrap(sa + 2)) * kG2Half;
    const uint8_t* stb = smem + (H == 0 ? wrap(sa + 1) : wrap(sa + 3)) * kG2Half;
    const int lslot = H == 0 ? wrap(sa + 4) : sa;
    const int r0 = H == 0 ? h10 : h00, r1 = H == 0 ? h11 : h01;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int i = t >> 2, j = t & 3;
      acc[i][j] = mfma_32x32x64(cur.b[j], cur.a[i], acc[i][j]);
      if ((t & 1) == 1 && load)
        issue(H * kG2ALoads + (t >> 1), kk + 2, lslot, std::integral_constant<bool, STEADY>{});
      if (t < 8 && more) {
        const int v = t >> 1;
        if ((t & 1) == 0) nxt.a[v] = g2_op(sta + a_off + 32 * v * kG2Pitch, r0, r1);
        else nxt.b[v] = b_op(stb, v, H == 0 ? 1 : 0, r0, r1);
      }
      if constexpr (STEADY) __builtin_amdgcn_sched_barrier(0);
    }
    if (H == 1) sa = wrap(sa + 2);
  };
  const int nfull = nsub >> 1;
  const int nsteady = max(0, nslice - 3);
  using H0 = std::integral_constant<int, 0>;
  using H1 = std::integral_constant<int, 1>;
  int kk = 0;
  for (; kk < nsteady; ++kk) {
    sub(kk, H0{}, std::true_type{}, o0, o1);
    sub(kk, H1{}, std::true_type{}, o1, o0);
  }
  for (; kk < nfull; ++kk) {
    sub(kk, H0{}, std::false_type{}, o0, o1);
    sub(kk, H1{}, std::false_type{}, o1, o0);
  }
  if (half_tail) sub(nfull, H0{}, std::false_type{}, o0, o1);

  // epilogue: C[m][n] = bf16(acc * a_scale * b_scale), or with row-wise
  // scales bf16((acc * row_scale[m]) * col_scale[n]).  The bf16 tile goes
  // through LDS so that every store writes whole rows: each wave puts its
  // 128 x 128 part (32 KiB) in its own LDS region, row r at 256 r, 8-byte
  // slot s (columns 4s .. 4s+3) at slot s ^ (r & 31) -- the 32 rows of one
  // write instruction then cover all 64 banks -- and reads it back 16 bytes
  // per lane, 16 lanes per row (16 distinct granules), so each row leaves
  // as one 256-byte run instead of sixteen 16-byte pieces.  The stores are
  // non-temporal: C is not read again, and the L2 keeps the operand rows
  // that other tiles still need.  The mode (EPI) is a template parameter
  // and a tile wholly inside C skips every bound check, so the staging is
  // straight-line code and the store loop reads eight rows from LDS before
  // it stores them (a read, its wait and its store per row took ~4x as
  // long).
  constexpr bool ROWS = EPI == kEpiRows;
  const float scale = ROWS ? 1.0f
                    : (g.a_dev ? *g.a_dev : g.a_scale) * (g.b_dev ? *g.b_dev : g.b_scale);
  const bool has_bias = EPI == kEpiBias || (ROWS && g.bias != nullptr);
  constexpr int kCPitch = 128 * 2;                  // bytes per row of a wave's C part
  static_assert(4 * 128 * kCPitch <= kG2Slots * kG2Half, "C staging fits the slots");
  uint8_t* ct = smem + wave * 128 * kCPitch;
  float sm[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + wm * 128 + 32 * i + lq;
    sm[i] = ROWS && m < g.M ? g.row_scale[m] : 1.0f;
  }
  __syncthreads();   // every wave has finished reading the operand slots
  // (no global store precedes these loads of bias and column scales)
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t n = n0 + wn * 128 + 32 * j + 8 * q + 4 * lg;
      // columns past N are never stored; with a bias or column scales
      // their (out-of-range) values are not read either
      if (EPI != kEpiPlain && n >= g.N) continue;
      const uint2 bb = has_bias ? bias4(g, n) : make_uint2(0u, 0u);
      const float4 sn = ROWS ? *reinterpret_cast<const float4*>(g.col_scale + n)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // rows past M are written here but never stored
        const f32x16& v = acc[i][j];
        float o[4];
        if constexpr (ROWS)
          epi4_rows(has_bias, bb, sm[i], sn, v[4 * q + 0], v[4 * q + 1], v[4 * q + 2],
                    v[4 * q + 3], o);
        else
          epi4(EPI == kEpiBias, bb, scale, v[4 * q + 0], v[4 * q + 1], v[4 * q + 2],
               v[4 * q + 3], o);
        uint2 pk;
        pk.x = g2_pack_bf16(o[0], o[1]);
        pk.y = g2_pack_bf16(o[2], o[3]);
        const int cs = ((8 * j + 2 * q + lg) ^ lq);
        *reinterpret_cast<uint2*>(ct + (32 * i + lq) * kCPitch + cs * 8) = pk;
      }
    }
  __syncthreads();
  // 16-byte stores need C, its row stride and batch stride 16-byte aligned;
  // otherwise each run is stored as 8-byte halves
  const bool c16 = reinterpret_cast<uintptr_t>(g.c) % 16 == 0 && g.ldc % 8 == 0;
  const int c = lane & 15;
  const bool odd = (lane >> 4) & 1;   // the parity of every row this lane reads
  const int64_t n = n0 + wn * 128 + 8 * c;
  // row r of the wave's part: logical slots 2c, 2c+1 sit in granule
  // c ^ ((r & 31) >> 1), swapped when r is odd
  auto stage_row = [&](int r) __attribute__((always_inline)) {
    const int cg = (c ^ ((r & 31) >> 1));
    const uint4 t = *reinterpret_cast<const uint4*>(ct + r * kCPitch + cg * 16);
    return odd ? u32x4{t.z, t.w, t.x, t.y} : u32x4{t.x, t.y, t.z, t.w};
  };
  uint16_t* const cw = g.c + (m0 + wm * 128) * g.ldc + n;
  if (c16 && m0 + 256 <= g.M && n0 + 256 <= g.N) {
    // a tile inside C: eight rows read, then eight whole-row stores
#pragma unroll
    for (int k8 = 0; k8 < 32; k8 += 8) {
      u32x4 t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = stage_row(4 * (k8 + u) + (lane >> 4));
#pragma unroll
      for (int u = 0; u < 8; ++u)
        __builtin_nontemporal_store(
            t[u], reinterpret_cast<u32x4*>(cw + (int64_t)(4 * (k8 + u) + (lane >> 4)) * g.ldc));
    }
    return;
  }
#pragma unroll 4
  for (int k = 0; k < 32; ++k) {
    const int r = 4 * k + (lane >> 4);
    const int64_t m = m0 + wm * 128 + r;
    const u32x4 t = stage_row(r);
    if (m >= g.M || n >= g.N) continue;
    uint16_t* dst = g.c + m * g.ldc + n;
    if (c16 && n + 8 <= g.N) {
      __builtin_nontemporal_store(t, reinterpret_cast<u32x4*>(dst));
    } else {
      // n + 4 <= N (N % 4 == 0)
      __builtin_nontemporal_store(u32x2{t.x, t.y}, reinterpret_cast<u32x2*>(dst));
      if (n + 8 <= g.N)
        __builtin_nontemporal_store(u32x2{t.z, t.w}, reinterpret_cast<u32x2*>(dst + 4));
    }
  }
}

template <bool KN>
void launch_g256(const GemmArgs& g, dim3 grid, hipStream_t st) {
  if (g.row_scale)
    hipLaunchKernelGGL((gemm256_kernel<KN, kEpiRows>), grid, dim3(kG2Threads), 0, st, g);
  else if (g.bias)
    hipLaunchKernelGGL((gemm256_kernel<KN, kEpiBias>), grid, dim3(kG2Threads), 0, st, g);
  else
    hipLaunchKernelGGL((gemm256_kernel<KN, kEpiPlain>), grid, dim3(kG2Threads), 0, st, g);
}

__global__ void gemm_zero_counter_kernel(unsigned* c) { *c = 0u; }

// Tiles per XCD share handed out through the counter of a balanced launch.
// At C4 (15,984 tiles, ~62 per CU), alternating on one box: static shares
// 4.04-4.07 ms ((K, N) B) and 3.97-3.99 ms ((N, K)); 32 pooled per share
// 4.01-4.02 / 3.93; 64 3.98-3.99 / 3.90-3.91; 128 the same as 64.
constexpr int kGemmPoolPerXcd = 64;

int launch_gemm256(GemmArgs g, int64_t batch, hipStream_t st) {
  g.tiles_m = (int)((g.M + kG2Tile - 1) / kG2Tile);
  g.tiles_n = (int)((g.N + kG2Tile - 1) / kG2Tile);
  const int64_t nwork = (int64_t)g.tiles_m * g.tiles_n;
  if (nwork > 0x3fffffff) {
    rp_set_error("gemm: grid too large");
    return RP_ERR_UNSUPPORTED;
  }
  int64_t nwg = nwork;
  const int64_t per = nwork >> 3;
  g.pool_r = g.item_counter != nullptr && batch == 1 ? (int)min((int64_t)kGemmPoolPerXcd, per) : 0;
  if (g.pool_r == 0) {
    g.item_counter = nullptr;
  } else {
    // the tiles left by every share, run by twice as many workgroups, the
    // same number on every XCD
    const int64_t pooled = 8 * (int64_t)g.pool_r + (nwork & 7);
    nwg = 8 * (per - g.pool_r) + (2 * pooled + 7) / 8 * 8;
    hipLaunchKernelGGL(gemm_zero_counter_kernel, dim3(1), dim3(1), 0, st, g.item_counter);
  }
  const dim3 grid((unsigned)nwg, (unsigned)batch);
  if (g.b_kn)
    launch_g256<true>(g, grid, st);
  else
    launch_g256<false>(g, grid, st);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    rp_set_error("gemm: launch failed: %s", hipGetErrorString(e));
    return RP_ERR_LAUNCH;
  }
  return RP_OK;
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
int launch_gemm(GemmArgs g, int64_t batch, hipStream_t st) {
  g.tiles_m = (int)((g.M + BM - 1) / BM);
  g.tiles_n = (int)((g.N + BN - 1) / BN);
  const int64_t nwork = (int64_t)g.tiles_m * g.tiles_n;
  if (nwork > 0x7fffffff) {
    rp_set_error("gemm: grid too large");
    return RP_ERR_UNSUPPORTED;
  }
  const dim3 grid((unsigned)nwork, (unsigned)batch);
  if (g.b_kn)
    hipLaunchKernelGGL((gemm_kernel<BM, BN, true>), grid, dim3(kGThreads), 0, st, g);
  else
    hipLaunchKernelGGL((gemm_kernel<BM, BN, false>), grid, dim3(kGThreads), 0, st, g);
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

// Row-wise scales and batching of rp_fp8_gemm_rowwise (none for the others).
struct RowwiseBatch {
  const float* row_scale = nullptr;
  const float* col_scale = nullptr;
  int64_t batch = 1, bsa = 0, bsb = 0, bsc = 0, bsr = 0, bss = 0;
};

static int gemm_run(const uint8_t* a8, const uint8_t* b8, int b_layout, const void* bias,
                    void* c, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                    int64_t ldc, float a_scale, float b_scale, const float* a_scale_dev,
                    const float* b_scale_dev, void* stream, const RowwiseBatch& rb = {},
                    unsigned* item_counter = nullptr) {
  if (!a8 || !b8 || !c) {
    rp_set_error("gemm: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (b_layout != RP_B_NK && b_layout != RP_B_KN) {
    rp_set_error("gemm: unknown B layout %d", b_layout);
    return RP_ERR_INVALID_ARGUMENT;
  }
  const bool kn = b_layout == RP_B_KN;
  if (M <= 0 || N <= 0 || K <= 0 || lda < K || ldb < (kn ? N : K) || ldc < N) {
    rp_set_error("gemm: bad sizes M=%lld N=%lld K=%lld lda=%lld ldb=%lld ldc=%lld (B %s)",
                 (long long)M, (long long)N, (long long)K, (long long)lda, (long long)ldb,
                 (long long)ldc, kn ? "(K, N)" : "(N, K)");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (K % 16 != 0 || lda % 16 != 0 || N % 4 != 0 || ldc % 4 != 0 || (!kn && ldb % 16 != 0)) {
    rp_set_error("gemm: needs K, lda multiples of 16, N, ldc multiples of 4, and for an (N, K) "
                 "B, ldb a multiple of 16");
    return RP_ERR_UNSUPPORTED;
  }
  if (reinterpret_cast<uintptr_t>(a8) % 16 != 0 ||
      (!kn && reinterpret_cast<uintptr_t>(b8) % 16 != 0) ||
      reinterpret_cast<uintptr_t>(c) % 8 != 0) {
    rp_set_error("gemm: A (and an (N, K) B) must be 16-byte aligned and C 8-byte aligned");
    return RP_ERR_UNSUPPORTED;
  }
  if (bias != nullptr && reinterpret_cast<uintptr_t>(bias) % 8 != 0) {
    rp_set_error("gemm: bias must be 8-byte aligned");
    return RP_ERR_UNSUPPORTED;
  }
  if (rb.batch < 1 || rb.batch > 65535) {
    rp_set_error("gemm: batch count %lld outside 1..65535", (long long)rb.batch);
    return RP_ERR_UNSUPPORTED;
  }
  if ((rb.row_scale == nullptr) != (rb.col_scale == nullptr) ||
      reinterpret_cast<uintptr_t>(rb.col_scale) % 16 != 0 || rb.bss % 4 != 0) {
    rp_set_error("gemm: row-wise scales need both vectors, the column scales 16-byte aligned "
                 "per batch");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (rb.batch > 1 && (rb.bsc % 4 != 0 || rb.bsa % 16 != 0 || (!kn && rb.bsb % 16 != 0) ||
                       (kn && rb.bsb % 16 != 0))) {
    rp_set_error("gemm: batch strides of A and B must be multiples of 16 bytes, of C of 4 "
                 "elements");
    return RP_ERR_UNSUPPORTED;
  }
  GemmArgs g{};
  g.row_scale = rb.row_scale; g.col_scale = rb.col_scale;
  g.bsa = rb.bsa; g.bsb = rb.bsb; g.bsc = rb.bsc; g.bsr = rb.bsr; g.bss = rb.bss;
  g.a = a8; g.bt = b8; g.c = static_cast<uint16_t*>(c);
  g.bias = static_cast<const uint16_t*>(bias);
  g.M = M; g.N = N; g.K = K; g.lda = lda; g.ldb = ldb; g.ldc = ldc;
  g.a_scale = a_scale; g.b_scale = b_scale; g.a_dev = a_scale_dev; g.b_dev = b_scale_dev;
  g.b_kn = kn ? 1 : 0;
  g.item_counter = item_counter;
  // The large-tile kernel reads whole 64-byte K sub-slices and keeps tile
  // offsets in 32 bits; from a (K, N) B it loads whole 16-byte N granules.
  const bool big = K % kG2Sub == 0 && lda * (int64_t)kG2Tile < (int64_t)1 << 32 &&
                   (kn ? (N % 16 == 0 && ldb % 16 == 0 && reinterpret_cast<uintptr_t>(b8) % 16 == 0 &&
                          ldb * (int64_t)kG2K < (int64_t)1 << 32)
                       : ldb * (int64_t)kG2Tile < (int64_t)1 << 32);
  if (big) return launch_gemm256(g, rb.batch, static_cast<hipStream_t>(stream));
  return launch_gemm<256, 128>(g, rb.batch, static_cast<hipStream_t>(stream));
}

extern "C" int rp_fp8_gemm(const uint8_t* a8, const uint8_t* b8, int b_layout, void* c, int64_t M,
                           int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                           float a_scale, float b_scale, const float* a_scale_dev,
                           const float* b_scale_dev, void* stream) {
  return gemm_run(a8, b8, b_layout, nullptr, c, M, N, K, lda, ldb, ldc, a_scale, b_scale,
                  a_scale_dev, b_scale_dev, stream);
}

extern "C" int rp_fp8_linear(const uint8_t* a8, const uint8_t* b8, int b_layout, const void* bias,
                             void* c, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                             int64_t ldc, float a_scale, float b_scale, const float* a_scale_dev,
                             const float* b_scale_dev, void* stream) {
  return gemm_run(a8, b8, b_layout, bias, c, M, N, K, lda, ldb, ldc, a_scale, b_scale,
                  a_scale_dev, b_scale_dev, stream);
}

extern "C" int rp_fp8_linear_balanced(const uint8_t* a8, const uint8_t* b8, int b_layout,
                                      const void* bias, void* c, int64_t M, int64_t N, int64_t K,
                                      int64_t lda, int64_t ldb, int64_t ldc, float a_scale,
                                      float b_scale, const float* a_scale_dev,
                                      const float* b_scale_dev, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  if (workspace == nullptr || workspace_bytes < RP_GEMM_BALANCED_WORKSPACE_BYTES ||
      reinterpret_cast<uintptr_t>(workspace) % 256 != 0) {
    rp_set_error("gemm: the balanced launch needs a 256-byte aligned workspace of %u bytes",
                 (unsigned)RP_GEMM_BALANCED_WORKSPACE_BYTES);
    return RP_ERR_WORKSPACE;
  }
  return gemm_run(a8, b8, b_layout, bias, c, M, N, K, lda, ldb, ldc, a_scale, b_scale,
                  a_scale_dev, b_scale_dev, stream, RowwiseBatch{},
                  static_cast<unsigned*>(workspace));
}

extern "C" int rp_fp8_gemm_rowwise(const uint8_t* a8, const uint8_t* b8, int b_layout, void* c,
                                   int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                   int64_t ldc, const float* row_scale, const float* col_scale,
                                   int64_t batch, int64_t bsa, int64_t bsb, int64_t bsc,
                                   int64_t bs_row, int64_t bs_col, void* stream) {
  if (row_scale == nullptr || col_scale == nullptr) {
    rp_set_error("gemm_rowwise: null scale vector");
    return RP_ERR_INVALID_ARGUMENT;
  }
  RowwiseBatch rb;
  rb.row_scale = row_scale; rb.col_scale = col_scale;
  rb.batch = batch; rb.bsa = bsa; rb.bsb = bsb; rb.bsc = bsc; rb.bsr = bs_row; rb.bss = bs_col;
  return gemm_run(a8, b8, b_layout, nullptr, c, M, N, K, lda, ldb, ldc, 1.0f, 1.0f, nullptr,
                  nullptr, stream, rb);
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
