// Per-group amax scaling and BF16/FP16 -> OCP e4m3fn quantization for gfx950.
//
// Behaviour follows the reference quantizer
// (kernels/triton_kernels/fp8_flash_attn_hopper.py:374-398; gfx942 sibling
// kernels/triton_kernels/fp8_flash_attn.py:425-448), whose scale arithmetic
// runs in the input dtype:
//   bf16: dequant = bf16(max(amax|x|, bf16(1e-6)) / 425.6)          per group
//   fp16: dequant = fp16(max(amax|x|, fp16(1e-6)) * RN(1/425.6))    per group
//   code  = e4m3fn(clamp(float(x) * (1/dequant), +-448))  round to nearest even
// The reference runs this as six torch ops over fp32 temporaries (about
// 33 B of HBM traffic per element).  Here it is two streaming passes plus a
// tiny per-group finalize: 2 B/element to find the maximum, 2 B read + 1 B
// written to quantize -- 5 B/element, the algorithmic minimum.
//
// Pass 1 (amax_flat / amax_partial): each 256-thread block reduces a
//   32 KiB slab of one group with packed 16-bit integer max over |x| bit
//   patterns (exact and order-free; NaN patterns sort above +inf, so NaN
//   propagates like torch.amax) and writes one partial per block -- no
//   atomics, no memset.  The _flat kernels serve contiguous tensors and issue
//   all eight of a thread's 16-byte loads before using any.
// Pass 2 (scale_finalize): one block per group folds its partials and forms
//   the dequant scale.
// Pass 3 (quant_flat / quant_apply / apply_t): re-reads x, multiplies by the correctly rounded
//   fp32 reciprocal and converts with the gfx950 v_cvt_pk_fp8_f32.
//   apply_t writes V transposed per head (D rows of ld codes), which is the
//   layout the attention kernel's P.V MFMA reads K-contiguous.
//
// This translation unit must not be compiled with fast-math: the scale
// division and the reciprocal have to be IEEE correctly rounded.

#include "rp_common.h"

#include <stdarg.h>
#include <stdio.h>

#include <mutex>

namespace rp {
namespace {

constexpr int kQThreads = 256;
constexpr int64_t kElemsPerBlock = 16384;  // 32 KiB of bf16 per block per pass

struct QParams {
  const uint16_t* x;
  int64_t B, H, S, D;
  int64_t sb, sh, ss;
  int64_t rows_per_group;  // rows (one row = D elements) in one group
  int64_t ngroups;
  int64_t rpb;             // rows per block
  int64_t nbg;             // blocks per group
  int vpr_log2;            // log2(D / 8): vectors of 8 elements per row
};

// Walks global rows r = bh*S + s of the (B, H, S, D) view.
struct RowCursor {
  int64_t s, bh, base;
  __device__ void init(int64_t r, const QParams& p) {
    bh = r / p.S;
    s = r - bh * p.S;
    base = (bh / p.H) * p.sb + (bh % p.H) * p.sh;
  }
  __device__ void advance(int64_t step, const QParams& p) {
    s += step;
    while (s >= p.S) {
      s -= p.S;
      ++bh;
      base = (bh / p.H) * p.sb + (bh % p.H) * p.sh;
    }
  }
};

__device__ __forceinline__ uint32_t pk_umax16(uint32_t a, uint32_t b) {
  // two independent 16-bit unsigned maxima in one dword
  uint32_t lo = umax32(a & 0xffffu, b & 0xffffu);
  uint32_t hi = umax32(a >> 16, b >> 16);
  return lo | (hi << 16);
}

__device__ __forceinline__ void amax_partial_body(int64_t blk_id, QParams p, uint32_t* partial) {
  const int64_t blk = blk_id;
  const int64_t g = blk / p.nbg;
  const int64_t j = blk - g * p.nbg;
  const int64_t first = j * p.rpb;
  const int64_t nrows = min(p.rpb, p.rows_per_group - first);
  const int vpr_mask = (1 << p.vpr_log2) - 1;
  const int col = threadIdx.x & vpr_mask;
  const int64_t roff = threadIdx.x >> p.vpr_log2;
  const int64_t step = kQThreads >> p.vpr_log2;

  uint32_t m = 0;
  if (roff < nrows) {
    RowCursor cur;
    cur.init(g * p.rows_per_group + first + roff, p);
    for (int64_t r = roff; r < nrows; r += step) {
      const uint4 v = *reinterpret_cast<const uint4*>(p.x + cur.base + cur.s * p.ss + col * 8);
      m = pk_umax16(m, v.x & 0x7fff7fffu);
      m = pk_umax16(m, v.y & 0x7fff7fffu);
      m = pk_umax16(m, v.z & 0x7fff7fffu);
      m = pk_umax16(m, v.w & 0x7fff7fffu);
      cur.advance(step, p);
    }
  }
  uint32_t m16 = umax32(m & 0xffffu, m >> 16);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m16 = umax32(m16, (uint32_t)shfl_xor((int)m16, o));
  __shared__ uint32_t wmax[kQThreads / kWave];
  if ((threadIdx.x & (kWave - 1)) == 0) wmax[threadIdx.x / kWave] = m16;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = wmax[0];
#pragma unroll
    for (int w = 1; w < kQThreads / kWave; ++w) r = umax32(r, wmax[w]);
    partial[blk] = r;
  }
}

__global__ __launch_bounds__(kQThreads) void amax_partial_kernel(QParams p, uint32_t* partial) {
  amax_partial_body(blockIdx.x, p, partial);
}

template <int DT>
__device__ __forceinline__ void scale_finalize_body(int64_t blk_id, const uint32_t* partial,
                                                                   int64_t nbg, float* dequant) {
  const int64_t g = blk_id;
  const uint32_t r = block_max_u32<kQThreads>(partial + g * nbg, nbg);
  if (threadIdx.x == 0) dequant[g] = dequant_from_amax<DT>(r);
}

template <int DT>
__global__ __launch_bounds__(kQThreads) void scale_finalize_kernel(const uint32_t* partial,
                                                                   int64_t nbg, float* dequant) {
  scale_finalize_body<DT>(blockIdx.x, partial, nbg, dequant);
}

template <int DT>
__device__ __forceinline__ uint32_t quant4(uint32_t lo_pair, uint32_t hi_pair, float qm) {
  const float a = clamp_e4m3(in_to_f32<DT>(lo_pair & 0xffffu) * qm);
  const float b = clamp_e4m3(in_to_f32<DT>(lo_pair >> 16) * qm);
  const float c = clamp_e4m3(in_to_f32<DT>(hi_pair & 0xffffu) * qm);
  const float d = clamp_e4m3(in_to_f32<DT>(hi_pair >> 16) * qm);
  return pack4_e4m3(a, b, c, d);
}


// Contiguous (B, H, S, D) input: group g is the flat element range
// [g*gsize, (g+1)*gsize).  Each block takes kElemsPerBlock elements of one
// group; each thread issues all of its kFlatLoads 16-byte loads before using
// any of them, so every wave keeps 8 loads in flight.
constexpr int kFlatLoads = kElemsPerBlock / 8 / kQThreads;  // 16-byte loads per thread
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void amax_flat_body(int64_t blk_id, const uint16_t* x, int64_t gsize,
                                                              int64_t nbg, uint32_t* partial) {
  const int64_t blk = blk_id;
  const int64_t g = blk / nbg;
  const int64_t j = blk - g * nbg;
  const int64_t start = g * gsize + j * kElemsPerBlock;
  const int64_t n8 = (min((int64_t)kElemsPerBlock, gsize - j * kElemsPerBlock)) / 8;
  const u32x4* src = reinterpret_cast<const u32x4*>(x + start);
  u32x4 v[kFlatLoads];
#pragma unroll
  for (int i = 0; i < kFlatLoads; ++i) {
    const int64_t idx = (int64_t)i * kQThreads + threadIdx.x;
    v[i] = idx < n8 ? __builtin_nontemporal_load(src + idx) : u32x4{0u, 0u, 0u, 0u};
  }
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < kFlatLoads; ++i) {
    m = pk_umax16(m, v[i][0] & 0x7fff7fffu);
    m = pk_umax16(m, v[i][1] & 0x7fff7fffu);
    m = pk_umax16(m, v[i][2] & 0x7fff7fffu);
    m = pk_umax16(m, v[i][3] & 0x7fff7fffu);
  }
  uint32_t m16 = umax32(m & 0xffffu, m >> 16);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m16 = umax32(m16, (uint32_t)shfl_xor((int)m16, o));
  __shared__ uint32_t wmax[kQThreads / kWave];
  if ((threadIdx.x & (kWave - 1)) == 0) wmax[threadIdx.x / kWave] = m16;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = wmax[0];
#pragma unroll
    for (int w = 1; w < kQThreads / kWave; ++w) r = umax32(r, wmax[w]);
    partial[blk] = r;
  }
}

__global__ __launch_bounds__(kQThreads) void amax_flat_kernel(const uint16_t* x, int64_t gsize,
                                                              int64_t nbg, uint32_t* partial) {
  amax_flat_body(blockIdx.x, x, gsize, nbg, partial);
}

template <int DT>
__device__ __forceinline__ void quant_flat_body(int64_t blk_id, const uint16_t* x, int64_t gsize,
                                                               int64_t nbg, const float* dequant,
                                                               int per_bh, uint8_t* codes) {
  const int64_t blk = blk_id;
  const int64_t g = blk / nbg;
  const int64_t j = blk - g * nbg;
  const int64_t start = g * gsize + j * kElemsPerBlock;
  const int64_t n8 = (min((int64_t)kElemsPerBlock, gsize - j * kElemsPerBlock)) / 8;
  const u32x4* src = reinterpret_cast<const u32x4*>(x + start);
  uint2* dst = reinterpret_cast<uint2*>(codes + start);
  const float qm = 1.0f / dequant[per_bh ? g : 0];
  u32x4 v[kFlatLoads];
#pragma unroll
  for (int i = 0; i < kFlatLoads; ++i) {
    const int64_t idx = (int64_t)i * kQThreads + threadIdx.x;
    v[i] = idx < n8 ? __builtin_nontemporal_load(src + idx) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int i = 0; i < kFlatLoads; ++i) {
    const int64_t idx = (int64_t)i * kQThreads + threadIdx.x;
    if (idx < n8) {
      uint2 o;
      o.x = quant4<DT>(v[i][0], v[i][1], qm);
      o.y = quant4<DT>(v[i][2], v[i][3], qm);
      dst[idx] = o;
    }
  }
}

template <int DT>
__global__ __launch_bounds__(kQThreads) void quant_flat_kernel(const uint16_t* x, int64_t gsize,
                                                               int64_t nbg, const float* dequant,
                                                               int per_bh, uint8_t* codes) {
  quant_flat_body<DT>(blockIdx.x, x, gsize, nbg, dequant, per_bh, codes);
}

// BHSD output: codes[r*D + d] for global row r = bh*S + s.
template <int DT>
__device__ __forceinline__ void quant_apply_body(int64_t blk_id, QParams p, const float* dequant,
                                                                int per_bh, uint8_t* codes) {
  const int64_t blk = blk_id;
  const int64_t g = blk / p.nbg;
  const int64_t j = blk - g * p.nbg;
  const int64_t first = j * p.rpb;
  const int64_t nrows = min(p.rpb, p.rows_per_group - first);
  const int vpr_mask = (1 << p.vpr_log2) - 1;
  const int col = threadIdx.x & vpr_mask;
  const int64_t roff = threadIdx.x >> p.vpr_log2;
  const int64_t step = kQThreads >> p.vpr_log2;
  if (roff >= nrows) return;

  RowCursor cur;
  const int64_t r0 = g * p.rows_per_group + first + roff;
  cur.init(r0, p);
  // group of the first row; a block never straddles groups
  const float qm = 1.0f / dequant[per_bh ? cur.bh : 0];
  int64_t r = r0;
  for (int64_t k = roff; k < nrows; k += step) {
    const uint4 v = *reinterpret_cast<const uint4*>(p.x + cur.base + cur.s * p.ss + col * 8);
    uint2 o;
    o.x = quant4<DT>(v.x, v.y, qm);
    o.y = quant4<DT>(v.z, v.w, qm);
    *reinterpret_cast<uint2*>(codes + r * p.D + col * 8) = o;
    cur.advance(step, p);
    r += step;
  }
}

template <int DT>
__global__ __launch_bounds__(kQThreads) void quant_apply_kernel(QParams p, const float* dequant,
                                                                int per_bh, uint8_t* codes) {
  quant_apply_body<DT>(blockIdx.x, p, dequant, per_bh, codes);
}

// BHDS output: per head, codes[(bh*D + d)*ld + s]; columns [S, ld) zeroed.
// Tile: 128 rows (s) x 64 columns (d), or 32 for the last block of a head
// dim that is an odd multiple of 32.  Thread t loads column chunk t & 7 (8
// elements) of rows 4*(t >> 3) + i, so the eight lanes of a chunk group
// read one row's 128 bytes (a whole line per 8 lanes), transposes its 4x8
// codes in registers and writes 8 dwords [d][s..s+3] into LDS; the tile
// then leaves as 64 rows of 128 contiguous codes.  In LDS, dword q of row d
// sits at q ^ 8((d >> 3) & 3): the 64 lanes of a write instruction (rows of
// one parity: 32 banks) land two to a bank, the minimum.
template <int DT>
__global__ __launch_bounds__(kQThreads) void quant_apply_t_kernel(QParams p, const float* dequant,
                                                                  int per_bh, uint8_t* codes,
                                                                  int64_t ld) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[64 * 128];
  const int64_t s0 = (int64_t)blockIdx.x * 128;
  const int64_t d0 = (int64_t)blockIdx.y * 64;
  const int dcols = (int)min((int64_t)64, p.D - d0);  // 64 or 32
  const int64_t bh = blockIdx.z;
  const float qm = 1.0f / dequant[per_bh ? bh : 0];
  const int64_t base = (bh / p.H) * p.sb + (bh % p.H) * p.sh + d0;
  const int q = threadIdx.x >> 3;   // row quad: rows 4q .. 4q+3 of the tile
  const int c = threadIdx.x & 7;    // column chunk: columns 8c .. 8c+7

  uint32_t w[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t s = s0 + 4 * q + i;
    if (s < p.S && c * 8 < dcols) {
      const uint4 v = *reinterpret_cast<const uint4*>(p.x + base + s * p.ss + c * 8);
      w[i][0] = quant4<DT>(v.x, v.y, qm);
      w[i][1] = quant4<DT>(v.z, v.w, qm);
    } else {
      w[i][0] = 0u;
      w[i][1] = 0u;
    }
  }
  // 4x4 byte transposes: rows i (s) x columns e (d) -> dword per column.
  const int qs = 4 * (q ^ (8 * (c & 3)));   // byte offset of this quad's dword in its row
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t t0 = __builtin_amdgcn_perm(w[1][h], w[0][h], 0x05010400u);
    const uint32_t t1 = __builtin_amdgcn_perm(w[1][h], w[0][h], 0x07030602u);
    const uint32_t t2 = __builtin_amdgcn_perm(w[3][h], w[2][h], 0x05010400u);
    const uint32_t t3 = __builtin_amdgcn_perm(w[3][h], w[2][h], 0x07030602u);
    const uint32_t col0 = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
    const uint32_t col1 = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    const uint32_t col2 = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
    const uint32_t col3 = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
    const int d = c * 8 + h * 4;
    *reinterpret_cast<uint32_t*>(&tile[(d + 0) * 128 + qs]) = col0;
    *reinterpret_cast<uint32_t*>(&tile[(d + 1) * 128 + qs]) = col1;
    *reinterpret_cast<uint32_t*>(&tile[(d + 2) * 128 + qs]) = col2;
    *reinterpret_cast<uint32_t*>(&tile[(d + 3) * 128 + qs]) = col3;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int dr = (threadIdx.x >> 3) + 32 * k;
    if (dr >= dcols) break;
    const int ch = threadIdx.x & 7;
    // physical 16-byte chunk ch of row dr holds the codes of s chunk
    // ch ^ 2((dr >> 3) & 3)
    const int sch = ch ^ (2 * ((dr >> 3) & 3));
    const uint4 v = *reinterpret_cast<const uint4*>(&tile[dr * 128 + ch * 16]);
    *reinterpret_cast<uint4*>(codes + (bh * p.D + d0 + dr) * ld + s0 + sch * 16) = v;
  }
}

// Multi-tensor launches (the Q, K and V of one attention call): blockIdx.y
// selects the job, blockIdx.x is the block inside it, and blocks past a
// job's own count return at once.  One launch per pass instead of three.
struct QJob {
  QParams p;          // the tensor's plan
  int flat;           // contiguous: the flat kernels
  int per_bh;
  int64_t gsize;      // elements per group (flat)
  int64_t nblocks;    // ngroups * nbg
  uint32_t* partial;  // this job's partial maxima
  float* dequant;     // this job's scales
  uint8_t* codes;     // BHSD codes (apply jobs)
};
struct QJobs3 {
  QJob j0, j1, j2;
};

// the job of this block (a select, not a dynamic index into the kernel
// arguments, which would copy them to scratch)
__device__ __forceinline__ const QJob& job_of(const QJobs3& jobs) {
  return blockIdx.y == 0 ? jobs.j0 : blockIdx.y == 1 ? jobs.j1 : jobs.j2;
}

__global__ __launch_bounds__(kQThreads) void amax_multi_kernel(QJobs3 jobs) {
  const QJob& jb = job_of(jobs);
  if ((int64_t)blockIdx.x >= jb.nblocks) return;
  if (jb.flat) amax_flat_body(blockIdx.x, jb.p.x, jb.gsize, jb.p.nbg, jb.partial);
  else amax_partial_body(blockIdx.x, jb.p, jb.partial);
}

template <int DT>
__global__ __launch_bounds__(kQThreads) void finalize_multi_kernel(QJobs3 jobs) {
  const QJob& jb = job_of(jobs);
  if ((int64_t)blockIdx.x >= jb.p.ngroups) return;
  scale_finalize_body<DT>(blockIdx.x, jb.partial, jb.p.nbg, jb.dequant);
}

template <int DT>
__global__ __launch_bounds__(kQThreads) void apply_multi_kernel(QJobs3 jobs) {
  const QJob& jb = job_of(jobs);
  if ((int64_t)blockIdx.x >= jb.nblocks) return;
  if (jb.flat)
    quant_flat_body<DT>(blockIdx.x, jb.p.x, jb.gsize, jb.p.nbg, jb.dequant, jb.per_bh, jb.codes);
  else
    quant_apply_body<DT>(blockIdx.x, jb.p, jb.dequant, jb.per_bh, jb.codes);
}

__global__ void selftest_e4m3_kernel(const float* x, uint8_t* out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = clamp_e4m3(x[i]);
  out[i] = (uint8_t)(cvt_pk_e4m3<false>(v, 0.0f, 0) & 0xff);
}

template <int DT>
__global__ void selftest_scale_kernel(const uint16_t* amax_bits, float* dequant, float* qmul,
                                      int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float dq = dequant_from_amax<DT>(amax_bits[i]);
  dequant[i] = dq;
  qmul[i] = 1.0f / dq;
}

// ------------------------------------------------------------------ host
struct Plan {
  QParams p;
  int dt;         // RP_DTYPE_* of x
  int per_bh;
  size_t ws_bytes;
  bool flat;      // contiguous input: the flat kernels apply
  int64_t gsize;  // elements per group when flat
};

bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }
int ilog2(int64_t v) {
  int r = 0;
  while ((int64_t(1) << r) < v) ++r;
  return r;
}

int make_plan(const void* x, int x_dtype, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
              int64_t sh, int64_t ss, int granularity, Plan* out) {
  if (x_dtype != RP_DTYPE_BF16 && x_dtype != RP_DTYPE_F16) {
    rp_set_error("quantize: unknown input dtype %d", x_dtype);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (B <= 0 || H <= 0 || S <= 0 || D <= 0) {
    rp_set_error("quantize: non-positive shape (%lld, %lld, %lld, %lld)", (long long)B,
                 (long long)H, (long long)S, (long long)D);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (granularity != RP_SCALE_PER_BH && granularity != RP_SCALE_PER_TENSOR) {
    rp_set_error("quantize: unknown granularity %d", granularity);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (D % 8 != 0) {
    rp_set_error("quantize: D=%lld must be a multiple of 8", (long long)D);
    return RP_ERR_UNSUPPORTED;
  }
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0 || (ss % 8) != 0 || (sh % 8) != 0 ||
      (sb % 8) != 0) {
    rp_set_error("quantize: input pointer and strides must be 16-byte aligned");
    return RP_ERR_UNSUPPORTED;
  }
  QParams p{};
  p.x = static_cast<const uint16_t*>(x);
  const bool contiguous = (ss == D) && (sh == S * D) && (sb == H * S * D);
  if (contiguous) {
    // A contiguous tensor is re-viewed as rows of 8 elements: every group is
    // then a contiguous run of rows and the per-thread walk is one vector.
    const int64_t rows_per_bh = S * D / 8;
    p.B = B; p.H = H; p.S = rows_per_bh; p.D = 8;
    p.sb = H * S * D; p.sh = S * D; p.ss = 8;
  } else {
    if (!is_pow2(D) || D > 2048) {
      rp_set_error("quantize: strided input needs a power-of-two D <= 2048 (got %lld)",
                   (long long)D);
      return RP_ERR_UNSUPPORTED;
    }
    p.B = B; p.H = H; p.S = S; p.D = D; p.sb = sb; p.sh = sh; p.ss = ss;
  }
  const int64_t total_rows = p.B * p.H * p.S;
  p.ngroups = granularity == RP_SCALE_PER_BH ? B * H : 1;
  p.rows_per_group = total_rows / p.ngroups;
  p.rpb = kElemsPerBlock / p.D;
  p.nbg = (p.rows_per_group + p.rpb - 1) / p.rpb;
  p.vpr_log2 = ilog2(p.D / 8);
  out->p = p;
  out->dt = x_dtype;
  out->per_bh = granularity == RP_SCALE_PER_BH;
  out->flat = contiguous;
  out->gsize = B * H * S * D / p.ngroups;
  out->ws_bytes = (size_t)(p.ngroups * p.nbg) * sizeof(uint32_t);
  return RP_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    rp_set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return RP_ERR_LAUNCH;
  }
  return RP_OK;
}

int launch_scale(const Plan& pl, float* dequant_out, void* ws, size_t ws_bytes, hipStream_t st) {
  if (ws == nullptr || ws_bytes < pl.ws_bytes) {
    rp_set_error("scale: workspace of %zu bytes needed, got %zu", pl.ws_bytes, ws_bytes);
    return RP_ERR_WORKSPACE;
  }
  uint32_t* partial = static_cast<uint32_t*>(ws);
  const int64_t nblocks = pl.p.ngroups * pl.p.nbg;
  if (pl.flat)
    hipLaunchKernelGGL(amax_flat_kernel, dim3((unsigned)nblocks), dim3(kQThreads), 0, st, pl.p.x,
                       pl.gsize, pl.p.nbg, partial);
  else
    hipLaunchKernelGGL(amax_partial_kernel, dim3((unsigned)nblocks), dim3(kQThreads), 0, st,
                       pl.p, partial);
  int rc = check_launch("amax_partial");
  if (rc) return rc;
  if (pl.dt == RP_DTYPE_F16)
    hipLaunchKernelGGL(scale_finalize_kernel<kInF16>, dim3((unsigned)pl.p.ngroups),
                       dim3(kQThreads), 0, st, partial, pl.p.nbg, dequant_out);
  else
    hipLaunchKernelGGL(scale_finalize_kernel<kInBf16>, dim3((unsigned)pl.p.ngroups),
                       dim3(kQThreads), 0, st, partial, pl.p.nbg, dequant_out);
  return check_launch("scale_finalize");
}

template <int DT>
int launch_apply_t(const Plan& pl, const void* x, int64_t B, int64_t H, int64_t S, int64_t D,
                   int64_t sb, int64_t sh, int64_t ss, const float* dequant, uint8_t* codes,
                   int layout, int64_t ld, hipStream_t st) {
  if (layout == RP_LAYOUT_BHSD) {
    const int64_t nblocks = pl.p.ngroups * pl.p.nbg;
    if (pl.flat)
      hipLaunchKernelGGL(quant_flat_kernel<DT>, dim3((unsigned)nblocks), dim3(kQThreads), 0, st,
                         pl.p.x, pl.gsize, pl.p.nbg, dequant, pl.per_bh, codes);
    else
      hipLaunchKernelGGL(quant_apply_kernel<DT>, dim3((unsigned)nblocks), dim3(kQThreads), 0, st,
                         pl.p, dequant, pl.per_bh, codes);
    return check_launch("quant_apply");
  }
  if (layout != RP_LAYOUT_BHDS) {
    rp_set_error("quantize: unknown layout %d", layout);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (D % 32 != 0 || ld < S || ld % 128 != 0) {
    rp_set_error("quantize(BHDS): needs D %% 32 == 0 and ld >= S with ld %% 128 == 0 "
                 "(D=%lld S=%lld ld=%lld)", (long long)D, (long long)S, (long long)ld);
    return RP_ERR_UNSUPPORTED;
  }
  QParams q{};
  q.x = static_cast<const uint16_t*>(x);
  q.B = B; q.H = H; q.S = S; q.D = D; q.sb = sb; q.sh = sh; q.ss = ss;
  if (B * H > 65535) {
    rp_set_error("quantize(BHDS): B*H=%lld exceeds the grid limit", (long long)(B * H));
    return RP_ERR_UNSUPPORTED;
  }
  dim3 grid((unsigned)(ld / 128), (unsigned)((D + 63) / 64), (unsigned)(B * H));
  hipLaunchKernelGGL(quant_apply_t_kernel<DT>, grid, dim3(kQThreads), 0, st, q, dequant,
                     pl.per_bh, codes, ld);
  return check_launch("quant_apply_t");
}

int launch_apply(const Plan& pl, const void* x, int64_t B, int64_t H, int64_t S, int64_t D,
                 int64_t sb, int64_t sh, int64_t ss, const float* dequant, uint8_t* codes,
                 int layout, int64_t ld, hipStream_t st) {
  if (pl.dt == RP_DTYPE_F16)
    return launch_apply_t<kInF16>(pl, x, B, H, S, D, sb, sh, ss, dequant, codes, layout, ld, st);
  return launch_apply_t<kInBf16>(pl, x, B, H, S, D, sb, sh, ss, dequant, codes, layout, ld, st);
}

}  // namespace
}  // namespace rp

using namespace rp;

extern "C" size_t rp_fp8_quant_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D,
                                               int granularity) {
  // Assumes a contiguous input; the strided plan never needs more rows per
  // group, and its rows hold at least as many elements.
  Plan pl;
  const void* dummy = reinterpret_cast<const void*>(uintptr_t(256));
  if (make_plan(dummy, RP_DTYPE_BF16, B, H, S, D, H * S * D, S * D, D, granularity, &pl) != RP_OK)
    return 0;
  Plan pl2;
  size_t strided = 0;
  if (make_plan(dummy, RP_DTYPE_BF16, B, H, S, D, H * S * D + 8, S * D + 8, D, granularity,
                &pl2) == RP_OK)
    strided = pl2.ws_bytes;
  return pl.ws_bytes > strided ? pl.ws_bytes : strided;
}

extern "C" int rp_fp8_scale(const void* x, int x_dtype, int64_t B, int64_t H, int64_t S,
                            int64_t D, int64_t sb, int64_t sh, int64_t ss, int granularity,
                            float* dequant_out, void* workspace, size_t workspace_bytes,
                            void* stream) {
  if (x == nullptr || dequant_out == nullptr) {
    rp_set_error("scale: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  Plan pl;
  int rc = make_plan(x, x_dtype, B, H, S, D, sb, sh, ss, granularity, &pl);
  if (rc) return rc;
  return launch_scale(pl, dequant_out, workspace, workspace_bytes,
                      static_cast<hipStream_t>(stream));
}

extern "C" int rp_fp8_quantize(const void* x, int x_dtype, int64_t B, int64_t H, int64_t S,
                               int64_t D, int64_t sb, int64_t sh, int64_t ss, int granularity,
                               const float* dequant, uint8_t* codes, int layout, int64_t ld,
                               void* stream) {
  if (x == nullptr || dequant == nullptr || codes == nullptr) {
    rp_set_error("quantize: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  Plan pl;
  int rc = make_plan(x, x_dtype, B, H, S, D, sb, sh, ss, granularity, &pl);
  if (rc) return rc;
  return launch_apply(pl, x, B, H, S, D, sb, sh, ss, dequant, codes, layout, ld,
                      static_cast<hipStream_t>(stream));
}

extern "C" int rp_fp8_scale_quantize(const void* x, int x_dtype, int64_t B, int64_t H, int64_t S,
                                     int64_t D, int64_t sb, int64_t sh, int64_t ss,
                                     int granularity, float* dequant_out, uint8_t* codes,
                                     int layout, int64_t ld, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  if (x == nullptr || dequant_out == nullptr || codes == nullptr) {
    rp_set_error("scale_quantize: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  Plan pl;
  int rc = make_plan(x, x_dtype, B, H, S, D, sb, sh, ss, granularity, &pl);
  if (rc) return rc;
  if (layout == RP_LAYOUT_BHDS && (D % 32 != 0 || ld < S || ld % 128 != 0)) {
    rp_set_error("scale_quantize(BHDS): needs D %% 32 == 0 and ld >= S with ld %% 128 == 0");
    return RP_ERR_UNSUPPORTED;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  rc = launch_scale(pl, dequant_out, workspace, workspace_bytes, st);
  if (rc) return rc;
  return launch_apply(pl, x, B, H, S, D, sb, sh, ss, dequant_out, codes, layout, ld, st);
}

static size_t align256(size_t n) { return (n + 255) / 256 * 256; }

extern "C" size_t rp_fp8_quant_qkv_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Skv,
                                                   int64_t D, int granularity) {
  const size_t q = rp_fp8_quant_workspace_bytes(B, H, Sq, D, granularity);
  const size_t kv = rp_fp8_quant_workspace_bytes(B, H, Skv, D, granularity);
  if (q == 0 || kv == 0) return 0;
  return align256(q) + align256(kv) + kv;
}

// Validates one Q/K/V quantizer call and returns the scratch bytes it needs
// (the three tensors' partial maxima side by side, each run 256-byte aligned).
static int qkv_plan(const void* q, const void* k, const void* v, int x_dtype, int64_t B,
                    int64_t H, int64_t Sq, int64_t Skv, int64_t D, int64_t qsb, int64_t qsh,
                    int64_t qss, int64_t ksb, int64_t ksh, int64_t kss, int64_t vsb, int64_t vsh,
                    int64_t vss, int granularity, const float* dequant_out, const uint8_t* q8,
                    const uint8_t* k8, const uint8_t* vt8, int64_t ldv, Plan* pq, Plan* pk,
                    Plan* pv, size_t* off_k, size_t* off_v, size_t* need) {
  if (q == nullptr || k == nullptr || v == nullptr || dequant_out == nullptr || q8 == nullptr ||
      k8 == nullptr || vt8 == nullptr) {
    rp_set_error("scale_quantize_qkv: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  int rc = make_plan(q, x_dtype, B, H, Sq, D, qsb, qsh, qss, granularity, pq);
  if (rc) return rc;
  if ((rc = make_plan(k, x_dtype, B, H, Skv, D, ksb, ksh, kss, granularity, pk))) return rc;
  if ((rc = make_plan(v, x_dtype, B, H, Skv, D, vsb, vsh, vss, granularity, pv))) return rc;
  if (D % 32 != 0 || ldv < Skv || ldv % 128 != 0) {
    rp_set_error("scale_quantize_qkv: V^T needs D %% 32 == 0 and ldv >= Skv with ldv %% 128 == 0");
    return RP_ERR_UNSUPPORTED;
  }
  if (B * H > 65535) {
    rp_set_error("scale_quantize_qkv: B*H=%lld exceeds the grid limit", (long long)(B * H));
    return RP_ERR_UNSUPPORTED;
  }
  *off_k = align256(pq->ws_bytes);
  *off_v = *off_k + align256(pk->ws_bytes);
  *need = *off_v + pv->ws_bytes;
  return RP_OK;
}

// The four launches of one Q/K/V quantizer call, partial maxima in `ws`.
static int qkv_launch(const Plan& pq, const Plan& pk, const Plan& pv, const void* v,
                      int x_dtype, int64_t B, int64_t H, int64_t Skv, int64_t D, int64_t vsb,
                      int64_t vsh, int64_t vss, float* dequant_out, uint8_t* q8, uint8_t* k8,
                      uint8_t* vt8, int64_t ldv, uint8_t* ws, size_t off_k, size_t off_v,
                      void* stream) {
  int rc;
  const int64_t ng = pq.p.ngroups;
  auto job = [&](const Plan& pl, size_t off, float* dq, uint8_t* codes) {
    QJob jb{};
    jb.p = pl.p;
    jb.flat = pl.flat;
    jb.per_bh = pl.per_bh;
    jb.gsize = pl.gsize;
    jb.nblocks = pl.p.ngroups * pl.p.nbg;
    jb.partial = reinterpret_cast<uint32_t*>(ws + off);
    jb.dequant = dq;
    jb.codes = codes;
    return jb;
  };
  QJobs3 jobs;
  jobs.j0 = job(pq, 0, dequant_out, q8);
  jobs.j1 = job(pk, off_k, dequant_out + ng, k8);
  jobs.j2 = job(pv, off_v, dequant_out + 2 * ng, nullptr);
  const int64_t amax_blocks = max(jobs.j0.nblocks, max(jobs.j1.nblocks, jobs.j2.nblocks));
  const int64_t apply_blocks = max(jobs.j0.nblocks, jobs.j1.nblocks);
  if (amax_blocks > 0x7fffffff) {
    rp_set_error("scale_quantize_qkv: grid too large");
    return RP_ERR_UNSUPPORTED;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(amax_multi_kernel, dim3((unsigned)amax_blocks, 3), dim3(kQThreads), 0, st,
                     jobs);
  if ((rc = check_launch("amax_multi"))) return rc;
  if (x_dtype == RP_DTYPE_F16) {
    hipLaunchKernelGGL(finalize_multi_kernel<kInF16>, dim3((unsigned)ng, 3), dim3(kQThreads), 0,
                       st, jobs);
    hipLaunchKernelGGL(apply_multi_kernel<kInF16>, dim3((unsigned)apply_blocks, 2),
                       dim3(kQThreads), 0, st, jobs);
  } else {
    hipLaunchKernelGGL(finalize_multi_kernel<kInBf16>, dim3((unsigned)ng, 3), dim3(kQThreads), 0,
                       st, jobs);
    hipLaunchKernelGGL(apply_multi_kernel<kInBf16>, dim3((unsigned)apply_blocks, 2),
                       dim3(kQThreads), 0, st, jobs);
  }
  if ((rc = check_launch("apply_multi"))) return rc;
  // V^T: its own grid shape
  return launch_apply(pv, v, B, H, Skv, D, vsb, vsh, vss, dequant_out + 2 * ng, vt8,
                      RP_LAYOUT_BHDS, ldv, st);
}

extern "C" int rp_fp8_scale_quantize_qkv(const void* q, const void* k, const void* v, int x_dtype,
                                         int64_t B, int64_t H, int64_t Sq, int64_t Skv, int64_t D,
                                         int64_t qsb, int64_t qsh, int64_t qss, int64_t ksb,
                                         int64_t ksh, int64_t kss, int64_t vsb, int64_t vsh,
                                         int64_t vss, int granularity, float* dequant_out,
                                         uint8_t* q8, uint8_t* k8, uint8_t* vt8, int64_t ldv,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  Plan pq, pk, pv;
  size_t off_k, off_v, need;
  int rc = qkv_plan(q, k, v, x_dtype, B, H, Sq, Skv, D, qsb, qsh, qss, ksb, ksh, kss, vsb, vsh,
                    vss, granularity, dequant_out, q8, k8, vt8, ldv, &pq, &pk, &pv, &off_k,
                    &off_v, &need);
  if (rc) return rc;
  if (workspace == nullptr || workspace_bytes < need ||
      reinterpret_cast<uintptr_t>(workspace) % 256 != 0) {
    rp_set_error("scale_quantize_qkv: workspace of %zu bytes (256-byte aligned) needed, got %zu",
                 need, workspace_bytes);
    return RP_ERR_WORKSPACE;
  }
  return qkv_launch(pq, pk, pv, v, x_dtype, B, H, Skv, D, vsb, vsh, vss, dequant_out, q8, k8,
                    vt8, ldv, static_cast<uint8_t*>(workspace), off_k, off_v, stream);
}

// ------------------------------------------------ allocation-free variant
// The partial maxima of rp_fp8_scale_quantize_qkv_noalloc live in this
// file-scope device array: each GPU the library runs on holds its own copy
// until the process ends.  Host code never passes the symbol itself to a
// kernel (on the host it names a stand-in, not device memory); it passes the
// device address hipGetSymbolAddress returns for the device in use, looked
// up once per device.  Every partial is written by the amax pass before the
// finalize pass reads it, so nothing needs clearing between calls.
static __device__ __align__(256) uint8_t scratch[RP_QKV_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// Device address of `scratch` on the device that runs `stream`, looked up on
// the first call for that device (with that device current).
int scratch_for_stream(hipStream_t st, uint8_t** out) {
  int dev = -1;
  hipError_t e = st != nullptr ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    rp_set_error("scale_quantize_qkv_noalloc: cannot tell the stream's device (%s)",
                 hipGetErrorString(e));
    return RP_ERR_INVALID_ARGUMENT;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    if ((e = hipGetDevice(&cur)) != hipSuccess) {
      rp_set_error("scale_quantize_qkv_noalloc: hipGetDevice: %s", hipGetErrorString(e));
      return RP_ERR_LAUNCH;
    }
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) {
      rp_set_error("scale_quantize_qkv_noalloc: hipSetDevice(%d): %s", dev, hipGetErrorString(e));
      return RP_ERR_LAUNCH;
    }
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || ptr == nullptr) {
      rp_set_error("scale_quantize_qkv_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                   dev, hipGetErrorString(e));
      return RP_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = static_cast<uint8_t*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return RP_OK;
}
}  // namespace

extern "C" int rp_fp8_scale_quantize_qkv_noalloc(const void* q, const void* k, const void* v,
                                                 int x_dtype, int64_t B, int64_t H, int64_t Sq,
                                                 int64_t Skv, int64_t D, int64_t qsb, int64_t qsh,
                                                 int64_t qss, int64_t ksb, int64_t ksh,
                                                 int64_t kss, int64_t vsb, int64_t vsh,
                                                 int64_t vss, int granularity, float* dequant_out,
                                                 uint8_t* q8, uint8_t* k8, uint8_t* vt8,
                                                 int64_t ldv, void* stream) {
  Plan pq, pk, pv;
  size_t off_k, off_v, need;
  int rc = qkv_plan(q, k, v, x_dtype, B, H, Sq, Skv, D, qsb, qsh, qss, ksb, ksh, kss, vsb, vsh,
                    vss, granularity, dequant_out, q8, k8, vt8, ldv, &pq, &pk, &pv, &off_k,
                    &off_v, &need);
  if (rc) return rc;
  if (need > RP_QKV_NOALLOC_SCRATCH_BYTES) {
    rp_set_error("scale_quantize_qkv_noalloc: these shapes need %zu bytes of scratch, more than "
                 "the %u this entry point holds; use rp_fp8_scale_quantize_qkv with a workspace",
                 need, (unsigned)RP_QKV_NOALLOC_SCRATCH_BYTES);
    return RP_ERR_WORKSPACE;
  }
  uint8_t* ws = nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if ((rc = scratch_for_stream(st, &ws))) return rc;
  return qkv_launch(pq, pk, pv, v, x_dtype, B, H, Skv, D, vsb, vsh, vss, dequant_out, q8, k8,
                    vt8, ldv, ws, off_k, off_v, stream);
}

extern "C" int rp_selftest_e4m3(const float* x, uint8_t* out, int64_t n, void* stream) {
  if (x == nullptr || out == nullptr || n < 0) {
    rp_set_error("selftest_e4m3: bad arguments");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (n == 0) return RP_OK;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(selftest_e4m3_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, out, n);
  return check_launch("selftest_e4m3");
}

extern "C" int rp_selftest_scale(const uint16_t* amax_bits, int x_dtype, float* dequant,
                                 float* qmul, int64_t n, void* stream) {
  if (amax_bits == nullptr || dequant == nullptr || qmul == nullptr || n < 0 ||
      (x_dtype != RP_DTYPE_BF16 && x_dtype != RP_DTYPE_F16)) {
    rp_set_error("selftest_scale: bad arguments");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (n == 0) return RP_OK;
  const int64_t blocks = (n + 255) / 256;
  if (x_dtype == RP_DTYPE_F16)
    hipLaunchKernelGGL(selftest_scale_kernel<kInF16>, dim3((unsigned)blocks), dim3(256), 0,
                       static_cast<hipStream_t>(stream), amax_bits, dequant, qmul, n);
  else
    hipLaunchKernelGGL(selftest_scale_kernel<kInBf16>, dim3((unsigned)blocks), dim3(256), 0,
                       static_cast<hipStream_t>(stream), amax_bits, dequant, qmul, n);
  return check_launch("selftest_scale");
}
