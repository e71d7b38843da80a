// Device bodies and the host-side plan of the amax quantizer (rp_quant.hip),
// shared with the fused QK-norm prologue (rp_prologue.hip), whose Q/K/V
// entry point runs V's passes inside the prologue's own launches.  Each
// body takes its block index as an argument, so one launch can hand its
// blocks to several tensors.  Everything here has internal linkage: each
// translation unit that includes it compiles its own copy.
#pragma once

#include "rp_common.h"

namespace rp {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

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
      // non-temporal (C3 Q/K/V on permuted views 0.979 -> 0.941 ms per call)
      const u32x4 vv = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(p.x + cur.base + cur.s * p.ss + col * 8));
      const uint4 v = make_uint4(vv[0], vv[1], vv[2], vv[3]);
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

template <int DT>
__device__ __forceinline__ void scale_finalize_body(int64_t blk_id, const uint32_t* partial,
                                                                   int64_t nbg, float* dequant) {
  const int64_t g = blk_id;
  const uint32_t r = block_max_u32<kQThreads>(partial + g * nbg, nbg);
  if (threadIdx.x == 0) dequant[g] = dequant_from_amax<DT>(r);
}



// Contiguous (B, H, S, D) input: group g is the flat element range
// [g*gsize, (g+1)*gsize).  Each block takes kElemsPerBlock elements of one
// group; each thread issues all of its kFlatLoads 16-byte loads before using
// any of them, so every wave keeps 8 loads in flight.
constexpr int kFlatLoads = kElemsPerBlock / 8 / kQThreads;  // 16-byte loads per thread

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


template <int DT>
__device__ __forceinline__ void quant_flat_core(int64_t blk_id, const uint16_t* x, int64_t gsize,
                                                int64_t nbg, float qm, uint8_t* codes) {
  const int64_t blk = blk_id;
  const int64_t g = blk / nbg;
  const int64_t j = blk - g * nbg;
  const int64_t start = g * gsize + j * kElemsPerBlock;
  const int64_t n8 = (min((int64_t)kElemsPerBlock, gsize - j * kElemsPerBlock)) / 8;
  const u32x4* src = reinterpret_cast<const u32x4*>(x + start);
  uint2* dst = reinterpret_cast<uint2*>(codes + start);
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
      // non-temporal, like every code store of the quantizers: the codes are
      // read once, by the next kernel (C3 Q/K/V call 0.960 -> 0.917 ms with
      // the three quantizer stores non-temporal, C2 0.618 -> 0.585 ms)
      __builtin_nontemporal_store(u32x2{o.x, o.y}, reinterpret_cast<u32x2*>(dst + idx));
    }
  }
}

template <int DT>
__device__ __forceinline__ void quant_flat_body(int64_t blk_id, const uint16_t* x, int64_t gsize,
                                                int64_t nbg, const float* dequant, int per_bh,
                                                uint8_t* codes) {
  const float qm = 1.0f / dequant[per_bh ? blk_id / nbg : 0];
  quant_flat_core<DT>(blk_id, x, gsize, nbg, qm, codes);
}


// BHSD output: codes[r*D + d] for global row r = bh*S + s.
template <int DT>
__device__ __forceinline__ void quant_apply_core(int64_t blk_id, QParams p, float qm,
                                                 uint8_t* codes) {
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
  int64_t r = r0;
  for (int64_t k = roff; k < nrows; k += step) {
    // non-temporal: x is read for the last time, the codes are read once
    // (C3 Q/K/V on permuted (B, S, H, D) views 1.026 -> 0.978 ms per call)
    const u32x4 v = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(p.x + cur.base + cur.s * p.ss + col * 8));
    __builtin_nontemporal_store(u32x2{quant4<DT>(v[0], v[1], qm), quant4<DT>(v[2], v[3], qm)},
                                reinterpret_cast<u32x2*>(codes + r * p.D + col * 8));
    cur.advance(step, p);
    r += step;
  }
}

// (a block never straddles groups; with per-(b, h) groups group g is head g)
template <int DT>
__device__ __forceinline__ void quant_apply_body(int64_t blk_id, QParams p, const float* dequant,
                                                 int per_bh, uint8_t* codes) {
  const float qm = 1.0f / dequant[per_bh ? blk_id / p.nbg : 0];
  quant_apply_core<DT>(blk_id, p, qm, codes);
}

// BHDS output: per head, codes[(bh*D + d)*ld + s]; columns [S, ld) zeroed.
// Tile: 128 rows (s) x 64 columns (d), or 32 for the last block of a head
// dim that is an odd multiple of 32.  Thread t loads column chunk t & 7 (8
// elements) of rows 4*(t >> 3) + i, so the eight lanes of a chunk group
// read one row's 128 bytes (a whole line per 8 lanes), transposes its 4x8
// codes in registers and writes 8 dwords [d][s..s+3] into LDS; the tile
// then leaves as 64 rows of 128 contiguous codes.  In LDS, dword q of row d
// sits at q ^ 8((d >> 3) & 3): the 64 lanes of a write instruction (rows of
// one parity: 32 banks) land two to a bank, the minimum.  The block takes
// s tile s_blk (128 rows) and d tile d_blk (64 columns) of head bh; `tile`
// is the block's 8 KiB of LDS, free again once every thread has returned.
constexpr int kTileBytes = 64 * 128;

// First half of a V^T tile: the codes of this thread's four rows (s) and
// eight columns (d), in registers.  NT: non-temporal loads (V is read for
// the last time).  Measured: the C3 Q/K/V call 0.979 -> 0.961 ms with them;
// in the fused Q/K-norm + V apply, whose Q/K half already loads
// non-temporally, plain loads are faster (0.618 against 0.631 ms at C2).
template <int DT, bool NT>
__device__ __forceinline__ void apply_t_load(const QParams& p, float qm, int64_t s_blk,
                                             int64_t d_blk, int64_t bh, uint32_t (&w)[4][2]) {
  const int64_t s0 = s_blk * 128;
  const int64_t d0 = d_blk * 64;
  const int dcols = (int)min((int64_t)64, p.D - d0);  // 64 or 32
  const int64_t base = (bh / p.H) * p.sb + (bh % p.H) * p.sh + d0;
  const int q = threadIdx.x >> 3;   // row quad: rows 4q .. 4q+3 of the tile
  const int c = threadIdx.x & 7;    // column chunk: columns 8c .. 8c+7
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t s = s0 + 4 * q + i;
    if (s < p.S && c * 8 < dcols) {
      const u32x4* src = reinterpret_cast<const u32x4*>(p.x + base + s * p.ss + c * 8);
      const u32x4 v = NT ? __builtin_nontemporal_load(src) : *src;
      w[i][0] = quant4<DT>(v[0], v[1], qm);
      w[i][1] = quant4<DT>(v[2], v[3], qm);
    } else {
      w[i][0] = 0u;
      w[i][1] = 0u;
    }
  }
}

// Second half: transpose the codes through `tile` and store the tile's rows.
__device__ __forceinline__ void apply_t_store(const QParams& p, const uint32_t (&w)[4][2],
                                              uint8_t* codes, int64_t ld, int64_t s_blk,
                                              int64_t d_blk, int64_t bh, uint8_t* tile) {
  const int64_t s0 = s_blk * 128;
  const int64_t d0 = d_blk * 64;
  const int dcols = (int)min((int64_t)64, p.D - d0);
  const int q = threadIdx.x >> 3;
  const int c = threadIdx.x & 7;
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
    __builtin_nontemporal_store(
        u32x4{v.x, v.y, v.z, v.w},
        reinterpret_cast<u32x4*>(codes + (bh * p.D + d0 + dr) * ld + s0 + sch * 16));
  }
}

template <int DT, bool NT>
__device__ __forceinline__ void apply_t_body(const QParams& p, const float* dequant, int per_bh,
                                             uint8_t* codes, int64_t ld, int64_t s_blk,
                                             int64_t d_blk, int64_t bh, uint8_t* tile) {
  const float qm = 1.0f / dequant[per_bh ? bh : 0];
  uint32_t w[4][2];
  apply_t_load<DT, NT>(p, qm, s_blk, d_blk, bh, w);
  apply_t_store(p, w, codes, ld, s_blk, d_blk, bh, tile);
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
}  // namespace
}  // namespace rp
