// Fused QK-norm (+ rotary embedding) + amax scaling + e4m3fn quantization.
//
// The step right before the FP8 path in the Cosmos/Wan attention processors
// (reference docs/walkthroughs/02-architecture.md:114-123) is
//     q = norm_q(q); k = norm_k(k)                 RMSNorm over the head dim
//     q, k = apply_rotary_emb(q, rope), ...(k)     optional
// followed by the quantizer of rp_quant.hip.  As separate passes that is one
// extra read and write of Q and K (4 B/element) per op.  Here the normalised
// (and rotated) row is recomputed inside both quantizer passes from the raw
// input, so the whole prologue moves 5 B/element, like the plain quantizer.
//
// Per row of D elements, in the operation order of torch's RMSNorm with
// weight w (diffusers' RMSNorm: fp32 math, result cast to the weight dtype
// before the weight multiply) and of diffusers' apply_rotary_emb(use_real):
//   ss   = sum over d of x_d^2        fp32; each 8-element chunk sums its
//                                     squares in order, then a butterfly
//                                     over the row's D/8 chunks (chunk q
//                                     with chunk q ^ k, k = D/16 ... 1)
//   r    = 1 / sqrt(ss * (1/D) + eps) IEEE sqrt and divide (two roundings)
//   n_d  = bf16(x_d * r)              then, with a weight, bf16(n_d * w_d)
//   y_d  = bf16(n_d * cos_d + rot(n)_d * sin_d)      three fp32 roundings
//          rot(n) = (-n[D/2:], n[:D/2]) for RP_ROPE_HALF,
//                   (-n_1, n_0, -n_3, n_2, ...) for RP_ROPE_INTERLEAVED
// and y is then scaled and quantized exactly as rp_fp8_scale_quantize does
// (dequant = bf16(max(amax|y|, bf16(1e-6)) / 425.6), code = e4m3fn RNE of
// clamp(y * RN(1/dequant), +-448)).  No step is contracted into an FMA
// (`#pragma clang fp contract(off)`), so every rounding above happens.
//
// rp_fp8_rmsnorm_scale_quantize runs one tensor in three launches (amax,
// finalize, apply); rp_fp8_rmsnorm_scale_quantize_qkv runs Q and K through
// this prologue and V through the plain quantizer's bodies (rp_quant_dev.h)
// in three launches for all three tensors.

#include "rp_quant_dev.h"

namespace rp {
namespace {

constexpr int kPThreads = 256;
constexpr int64_t kPElemsPerBlock = 16384;

struct PParams {
  const uint16_t* x;
  int64_t B, H, S, D;
  int64_t sb, sh, ss;
  const uint16_t* weight;  // bf16 [D] or null
  float eps;
  const float* cosv;       // fp32 [S, D] or null
  const float* sinv;
  float* rinv;             // [B*H*S] 1/sqrt(mean(x^2) + eps) of each row
  int64_t rows_per_group;  // S (per (b, h)) or B*H*S (per tensor)
  int64_t rpb;             // rows per block
  int64_t nbg;             // blocks per group
};

// fp32 -> nearest-even bf16 value, held in fp32 (v_cvt_pk_bf16_f32)
__device__ __forceinline__ float bf16r(float f) { return (float)(__bf16)f; }

// The normalised (and rotated) 8 elements [8c, 8c+8) of U rows at xrow[u]
// (positions s[u], global rows row[u]), each exactly a bf16 value held in
// fp32.  All D/8 threads of a row call this together (the sum of squares
// and the half rotation cross threads).  The U rows go through each step
// side by side, so their dependent chains (squares, butterfly, sqrt,
// divide) overlap.  Without rotary tables the amax pass (STORE) writes
// each row's r = 1/sqrt(mean(x^2) + eps) to p.rinv and the apply pass
// (LOAD) reads it back instead of repeating the chain -- the same fp32
// value, so both passes normalise identically.  With tables the apply pass
// recomputes r: reading it back measured 4% slower there (0.595 against
// 0.57 ms at (1, 32, 56320, 128)), while it saves 7% without them.
// The rotary layout is a template parameter: with it as a runtime branch,
// hipcc 7.2 merged the two layouts' code so that the interleaved path
// skipped its own sign flips (rotated with stale registers).
// Sum of the two lanes of a quad xor K apart (DPP quad_perm, no LDS trip).
template <int K>
__device__ __forceinline__ float add_quad_xor(float v) {
  static_assert(K == 1 || K == 2, "quad lanes");
  constexpr int sel = K == 1 ? 0xB1 : 0x4E;   // (1, 0, 3, 2) or (2, 3, 0, 1)
  const int r = __builtin_amdgcn_mov_dpp(__float_as_int(v), sel, 0xf, 0xf, false);
  return v + __int_as_float(r);
}

// The first steps of prologue_rows: this thread's EPT elements of each row
// as fp32 and each row's r = 1/sqrt(mean(x^2) + eps).  TPR = D/EPT threads
// share a row; thread c holds the row's 16-byte chunks c + TPR*m (m < EPT/8)
// at x[u][8m .. 8m+7].  The sum of squares keeps one order whatever EPT is:
// each chunk sums its 8 squares in order, then the chunk sums combine as a
// butterfly over the D/8 chunks (chunk q with chunk q ^ k, k = D/16 ... 1).
// The levels k >= TPR pair chunks of one thread; the others pair lanes.
// With PMAX, pmax[u] also gets the two 16-bit maxima of |x| over the
// thread's elements of row u, from the packed input bits.
template <int D, int U, int EPT, bool LOAD, bool STORE, bool PMAX = false>
__device__ __forceinline__ void load_norm(const PParams& p, const uint16_t* const (&xrow)[U],
                                          const int64_t (&row)[U], int c, float (&x)[U][EPT],
                                          float (&r)[U], uint32_t* pmax = nullptr) {
#pragma clang fp contract(off)
  constexpr int TPR = D / EPT;
  constexpr int NC = EPT / 8;
  static_assert(EPT % 8 == 0 && TPR >= 1 && TPR * EPT == D, "row split");
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int m = 0; m < NC; ++m) {
      // non-temporal: each pass reads x once (0.625 -> 0.618 ms per C2 Q/K/V call)
      const u32x4 v = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(xrow[u] + 8 * (c + TPR * m)));
      const uint32_t w4[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[u][8 * m + 2 * i] = bf16_to_f32(w4[i] & 0xffffu);
        x[u][8 * m + 2 * i + 1] = bf16_to_f32(w4[i] >> 16);
        if constexpr (PMAX) pmax[u] = pk_max_u16(m == 0 && i == 0 ? 0u : pmax[u], w4[i] & 0x7fff7fffu);
      }
    }
  if constexpr (LOAD) {
#pragma unroll
    for (int u = 0; u < U; ++u) r[u] = p.rinv[row[u]];
  } else {
    float ss[U][NC];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int m = 0; m < NC; ++m) {
        ss[u][m] = x[u][8 * m] * x[u][8 * m];
#pragma unroll
        for (int i = 1; i < 8; ++i) ss[u][m] = ss[u][m] + x[u][8 * m + i] * x[u][8 * m + i];
      }
    // levels k = D/16 ... TPR: chunks c + TPR*m and c + TPR*(m + k/TPR)
#pragma unroll
    for (int b = NC / 2; b >= 1; b >>= 1)
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int m = 0; m < b; ++m) ss[u][m] = ss[u][m] + ss[u][m + b];
    if constexpr (TPR == 16 && D == 128) {
      // a row is one 16-lane DPP row: the butterfly by row rotations
#pragma unroll
      for (int u = 0; u < U; ++u) {
        ss[u][0] = add_row_ror<8>(ss[u][0]);
        ss[u][0] = add_row_ror<4>(ss[u][0]);
        ss[u][0] = add_row_ror<2>(ss[u][0]);
        ss[u][0] = add_row_ror<1>(ss[u][0]);
      }
    } else if constexpr (TPR <= 4) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if constexpr (TPR == 4) ss[u][0] = add_quad_xor<2>(ss[u][0]);
        if constexpr (TPR >= 2) ss[u][0] = add_quad_xor<1>(ss[u][0]);
      }
    } else {
#pragma unroll
      for (int o = TPR / 2; o >= 1; o >>= 1)
#pragma unroll
        for (int u = 0; u < U; ++u) ss[u][0] = ss[u][0] + shfl_xor(ss[u][0], o);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      r[u] = 1.0f / __builtin_sqrtf(ss[u][0] * (1.0f / D) + p.eps);
      if (STORE && c == 0) p.rinv[row[u]] = r[u];
    }
  }
}

template <int D, int ROPE, int U, int EPT, bool LOAD, bool STORE>
__device__ __forceinline__ void prologue_rows(const PParams& p, const uint16_t* const (&xrow)[U],
                                              const int64_t (&s)[U], const int64_t (&row)[U],
                                              int c, float (&y)[U][EPT]) {
#pragma clang fp contract(off)
  static_assert(ROPE == RP_ROPE_NONE || EPT == 8, "rotary rows: 8 elements per thread");
  constexpr int TPR = D / EPT;
  float x[U][EPT], r[U];
  load_norm<D, U, EPT, LOAD, STORE>(p, xrow, row, c, x, r);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int i = 0; i < EPT; ++i) y[u][i] = bf16r(x[u][i] * r[u]);
  if (p.weight != nullptr) {
#pragma unroll
    for (int m = 0; m < EPT / 8; ++m) {
      const uint4 wv = *reinterpret_cast<const uint4*>(p.weight + 8 * (c + TPR * m));
      const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float& lo = y[u][8 * m + 2 * i];
          float& hi = y[u][8 * m + 2 * i + 1];
          lo = bf16r(lo * bf16_to_f32(ww[i] & 0xffffu));
          hi = bf16r(hi * bf16_to_f32(ww[i] >> 16));
        }
    }
  }
  if constexpr (ROPE == RP_ROPE_NONE) return;
  else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float rot[8];
      if constexpr (ROPE == RP_ROPE_HALF) {
        // partner elements d +- D/2 live in thread c ^ (D/16)
        const bool lo = c < D / 16;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float o = shfl_xor(y[u][i], D / 16);
          rot[i] = lo ? -o : o;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          rot[i] = -y[u][i + 1];
          rot[i + 1] = y[u][i];
        }
      }
      const float4* cp = reinterpret_cast<const float4*>(p.cosv + s[u] * D + 8 * c);
      const float4* sp = reinterpret_cast<const float4*>(p.sinv + s[u] * D + 8 * c);
      const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
      const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
      const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float a = y[u][i] * cs[i];
        const float b = rot[i] * sn[i];
        y[u][i] = bf16r(a + b);
      }
    }
  }
}

// (b, h, s) of a row, advanced without divisions.
struct PCursor {
  int64_t b, h, s;
  __device__ __forceinline__ void advance(int64_t n, const PParams& p) {
    s += n;
    while (s >= p.S) {
      s -= p.S;
      if (++h == p.H) { h = 0; ++b; }
    }
  }
};

// Rows per thread and loop step: the rows of one step run side by side.
// Measured at (1, 32, 56320, 128): without rotary tables 1/2/4 rows take
// 0.296/0.246/0.251 ms; with tables (16 more fp32 values per row) one row
// is fastest (0.57 ms, 0.63 with two).
template <int ROPE>
constexpr int kPRowsPerStep = ROPE == RP_ROPE_NONE ? 2 : 1;
// Elements per thread and rows per step of the amax pass without rotary
// tables.  Every thread of a row computes the row's inverse norm (IEEE sqrt
// and divide, the butterfly), so fewer threads per row spread that over more
// elements: 8 elements per thread took 14 VALU instructions per element.
// Measured at C2 (1, 32, 56320, 128), Q/K/V in one call: 8/16/32 elements
// per thread with two rows per step 0.628/0.626/0.622 ms, 32 with one row
// 0.624 ms.
template <int ROPE>
constexpr int kAmaxEpt = ROPE == RP_ROPE_NONE ? 32 : 8;
template <int ROPE>
constexpr int kAmaxRows = kPRowsPerStep<ROPE>;

// Whether the apply pass reads each row's inverse norm back from the amax pass.
template <int ROPE>
constexpr bool kStoreNorm = ROPE == RP_ROPE_NONE;

// Row iteration shared by both passes: block blk covers rows
// [first, first + nrows) of group g; with TPR = D/EPT threads per row,
// thread t works on row offsets t / TPR + j * STEP and is thread c = t % TPR
// of each of them.  Each loop step hands
// fn U rows, STEP apart; a row past the block's range is
// replaced by the step's first row (read, never used: ok[u] is false).
template <int D, int U, int EPT, typename F>
__device__ __forceinline__ void for_rows(const PParams& p, int64_t blk, F&& fn) {
  constexpr int TPR = D / EPT;
  constexpr int STEP = kPThreads / TPR;
  const int64_t g = blk / p.nbg;
  const int64_t first = (blk - g * p.nbg) * p.rpb;
  const int64_t nrows = min(p.rpb, p.rows_per_group - first);
  const int c = threadIdx.x % TPR;
  int64_t k = threadIdx.x / TPR;
  if (k >= nrows) return;
  // Fast path: the block's rows all lie in one (b, h), so a thread's rows
  // are STEP apart in s and their addresses advance by a fixed stride.
  {
    const int64_t rb = g * p.rows_per_group + first;   // the block's first row
    const int64_t bhb = rb / p.S;
    const int64_t sb0 = rb - bhb * p.S;
    if (sb0 + nrows <= p.S) {
      const int64_t bb = bhb / p.H;
      const uint16_t* xp = p.x + bb * p.sb + (bhb - bb * p.H) * p.sh + (sb0 + k) * p.ss;
      const int64_t dstep = (int64_t)STEP * p.ss;
      for (; k < nrows; k += U * STEP, xp += U * dstep) {
        int64_t rr[U], bh[U], sv[U];
        const uint16_t* xr[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          ok[u] = k + u * STEP < nrows;
          // a row past the range repeats the step's first row (never used)
          const int64_t du = ok[u] ? u * STEP : 0;
          rr[u] = rb + k + du;
          bh[u] = bhb;
          sv[u] = sb0 + k + du;
          xr[u] = xp + (ok[u] ? u * dstep : 0);
        }
        fn(rr, bh, sv, xr, ok, c);
      }
      return;
    }
  }
  int64_t r = g * p.rows_per_group + first + k;  // global row bh*S + s
  PCursor cur;
  {
    const int64_t bh = r / p.S;
    cur.s = r - bh * p.S;
    cur.b = bh / p.H;
    cur.h = bh - cur.b * p.H;
  }
  for (; k < nrows; k += U * STEP, r += U * STEP) {
    int64_t rr[U], bh[U], sv[U];
    const uint16_t* xr[U];
    bool ok[U];
    PCursor cu = cur;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (u > 0) cu.advance(STEP, p);
      ok[u] = k + u * STEP < nrows;
      const PCursor& q = ok[u] ? cu : cur;
      rr[u] = ok[u] ? r + u * STEP : r;
      bh[u] = q.b * p.H + q.h;
      sv[u] = q.s;
      xr[u] = p.x + q.b * p.sb + q.h * p.sh + q.s * p.ss;
    }
    fn(rr, bh, sv, xr, ok, c);
    cur.advance(U * STEP, p);
  }
}

template <int D, int ROPE>
__device__ __forceinline__ void prologue_amax_body(const PParams& p, int64_t blk,
                                                   uint32_t* partial) {
  constexpr int U = kAmaxRows<ROPE>;
  constexpr int EPT = kAmaxEpt<ROPE>;
  uint32_t m = 0;
  if (ROPE == RP_ROPE_NONE && p.weight == nullptr) {
    // y = bf16(x * r) is only needed for its maximum, and for r >= 0 that is
    // bf16(max |x| * r): the product and the rounding are monotonic in |x|.
    // So each thread takes the maximum of its |x| from the packed input bits
    // (two per packed 16-bit max, no unpacking) and multiplies once per row;
    // the block's maximum over its threads is then the row's.  The one
    // exception is r = inf (eps = 0 and every square underflowing to 0),
    // where 0 * r is NaN while max|x| * r is not: such a row takes the
    // maximum over its products.  A row past the range repeats a row of the
    // range (the same maximum), so it needs no mask.
    for_rows<D, U, EPT>(p, blk, [&](const int64_t (&r)[U], const int64_t (&)[U],
                                    const int64_t (&)[U], const uint16_t* const (&xrow)[U],
                                    const bool (&)[U], int c) {
#pragma clang fp contract(off)
      float x[U][EPT], rn[U];
      uint32_t pm[U];
      load_norm<D, U, EPT, false, kStoreNorm<ROPE>, true>(p, xrow, r, c, x, rn, pm);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        // the bf16 conversion of y in every other path (v_cvt_pk_bf16_f32)
        auto bits = [](float f) { return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f); };
        const float ax = bf16_to_f32(umax32(pm[u] & 0xffffu, pm[u] >> 16));
        m = umax32(m, bits(ax * rn[u]) & 0x7fffu);
        if (rn[u] == __builtin_inff()) {
#pragma unroll
          for (int i = 0; i < EPT; ++i) m = umax32(m, bits(x[u][i] * rn[u]) & 0x7fffu);
        }
      }
    });
  } else {
    for_rows<D, U, EPT>(p, blk, [&](const int64_t (&r)[U], const int64_t (&)[U],
                                    const int64_t (&s)[U], const uint16_t* const (&xrow)[U],
                                    const bool (&ok)[U], int c) {
      float y[U][EPT];
      prologue_rows<D, ROPE, U, EPT, false, kStoreNorm<ROPE>>(p, xrow, s, r, c, y);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < EPT; ++i)
          m = umax32(m, ok[u] ? (__float_as_uint(y[u][i]) >> 16) & 0x7fffu : 0u);
    });
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = umax32(m, (uint32_t)shfl_xor((int)m, o));
  __shared__ uint32_t wmax[kPThreads / kWave];
  if ((threadIdx.x & (kWave - 1)) == 0) wmax[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = wmax[0];
#pragma unroll
    for (int w = 1; w < kPThreads / kWave; ++w) r = umax32(r, wmax[w]);
    partial[blk] = r;
  }
}

template <int D, int ROPE>
__global__ __launch_bounds__(kPThreads) void prologue_amax_kernel(PParams p, uint32_t* partial) {
  prologue_amax_body<D, ROPE>(p, blockIdx.x, partial);
}

__global__ __launch_bounds__(kPThreads) void prologue_finalize_kernel(const uint32_t* partial,
                                                                      int64_t nbg,
                                                                      float* dequant) {
  const int64_t g = blockIdx.x;
  const uint32_t r = block_max_u32<kPThreads>(partial + g * nbg, nbg);
  if (threadIdx.x == 0) dequant[g] = dequant_from_amax_bits(r);
}

template <int D, int ROPE>
__device__ __forceinline__ void prologue_quant_body(const PParams& p, int64_t blk,
                                                    const float* dequant, int per_bh,
                                                    uint8_t* codes) {
  constexpr int U = kPRowsPerStep<ROPE>;
  for_rows<D, U, 8>(p, blk, [&](const int64_t (&r)[U], const int64_t (&bh)[U],
                                const int64_t (&s)[U], const uint16_t* const (&xrow)[U],
                                const bool (&ok)[U], int c) {
    float y[U][8];
    prologue_rows<D, ROPE, U, 8, kStoreNorm<ROPE>, false>(p, xrow, s, r, c, y);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!ok[u]) continue;
      const float qm = 1.0f / dequant[per_bh ? bh[u] : 0];
      uint2 o;
      o.x = pack4_e4m3(clamp_e4m3(y[u][0] * qm), clamp_e4m3(y[u][1] * qm),
                       clamp_e4m3(y[u][2] * qm), clamp_e4m3(y[u][3] * qm));
      o.y = pack4_e4m3(clamp_e4m3(y[u][4] * qm), clamp_e4m3(y[u][5] * qm),
                       clamp_e4m3(y[u][6] * qm), clamp_e4m3(y[u][7] * qm));
      __builtin_nontemporal_store(u32x2{o.x, o.y},
                                  reinterpret_cast<u32x2*>(codes + r[u] * D + 8 * c));
    }
  });
}

template <int D, int ROPE>
__global__ __launch_bounds__(kPThreads) void prologue_quant_kernel(PParams p,
                                                                   const float* dequant,
                                                                   int per_bh, uint8_t* codes) {
  prologue_quant_body<D, ROPE>(p, blockIdx.x, dequant, per_bh, codes);
}

// ---- Q and K through the prologue, V through the plain quantizer, together:
// three launches for the three tensors instead of nine.  Block i of the amax
// and apply launches works for tensor i % 3, so the amax pass's VALU-bound
// norm blocks share each CU with V's HBM-bound blocks instead of running
// before or after them; a tensor with fewer blocks than the others leaves
// its surplus blocks to return at once.
struct NormQKV {
  PParams q, k;
  QParams v;                 // V's amax plan (rows of 8 elements when contiguous)
  QParams vt;                // V as (B, H, Skv, D) with its strides (transposed apply)
  int vflat;                 // contiguous V: the flat amax body
  int per_bh;
  int64_t vgsize;            // elements per group of contiguous V
  int64_t nq, nk, nv, nvt;   // blocks: Q and K (both passes), V amax, V^T apply
  int64_t vt_tiles;          // 128-column tiles per head of V^T (ldv / 128)
  int64_t ldv;
  int64_t ngroups;
  uint32_t *pq, *pk, *pv;    // partial maxima
  float* dequant;            // Q's, K's and V's scales, ngroups each
  uint8_t *q8, *k8, *vt8;
};

template <int D, int ROPE>
__global__ __launch_bounds__(kPThreads) void qkv_norm_amax_kernel(NormQKV a) {
  const int t = blockIdx.x % 3;
  const int64_t b = blockIdx.x / 3;
  if (t == 0) {
    if (b < a.nq) prologue_amax_body<D, ROPE>(a.q, b, a.pq);
  } else if (t == 1) {
    if (b < a.nk) prologue_amax_body<D, ROPE>(a.k, b, a.pk);
  } else if (b < a.nv) {
    if (a.vflat) amax_flat_body(b, a.v.x, a.vgsize, a.v.nbg, a.pv);
    else amax_partial_body(b, a.v, a.pv);
  }
}

__global__ __launch_bounds__(kPThreads) void qkv_norm_finalize_kernel(NormQKV a) {
  const int t = blockIdx.y;
  const uint32_t* partial = t == 0 ? a.pq : t == 1 ? a.pk : a.pv;
  const int64_t nbg = t == 0 ? a.q.nbg : t == 1 ? a.k.nbg : a.v.nbg;
  scale_finalize_body<kInBf16>(blockIdx.x, partial, nbg, a.dequant + t * a.ngroups);
}

template <int D, int ROPE>
__global__ __launch_bounds__(kPThreads) void qkv_norm_apply_kernel(NormQKV a) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kTileBytes];
  const int t = blockIdx.x % 3;
  const int64_t b = blockIdx.x / 3;
  if (t == 0) {
    if (b < a.nq) prologue_quant_body<D, ROPE>(a.q, b, a.dequant, a.per_bh, a.q8);
  } else if (t == 1) {
    if (b < a.nk) prologue_quant_body<D, ROPE>(a.k, b, a.dequant + a.ngroups, a.per_bh, a.k8);
  } else if (b < a.nvt) {
    // 128 rows of one head of V: its D/64 column tiles one after the other
    const int64_t bh = b / a.vt_tiles;
    const int64_t sblk = b - bh * a.vt_tiles;
#pragma unroll
    for (int db = 0; db < D / 64; ++db) {
      if (db > 0) __syncthreads();  // every thread has read the previous tile back
      apply_t_body<kInBf16, false>(a.vt, a.dequant + 2 * a.ngroups, a.per_bh, a.vt8, a.ldv,
                                   sblk, db, bh, tile);
    }
  }
}

int launch_check(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    rp_set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return RP_ERR_LAUNCH;
  }
  return RP_OK;
}

template <int D, int ROPE>
int run_prologue(const PParams& p, int64_t ngroups, float* dequant, uint8_t* codes, int per_bh,
                 uint32_t* partial, hipStream_t st) {
  const unsigned blocks = (unsigned)(ngroups * p.nbg);
  hipLaunchKernelGGL((prologue_amax_kernel<D, ROPE>), dim3(blocks), dim3(kPThreads), 0, st, p,
                     partial);
  int rc = launch_check("rmsnorm_quantize(amax)");
  if (rc) return rc;
  hipLaunchKernelGGL(prologue_finalize_kernel, dim3((unsigned)ngroups), dim3(kPThreads), 0, st,
                     partial, p.nbg, dequant);
  rc = launch_check("rmsnorm_quantize(finalize)");
  if (rc) return rc;
  hipLaunchKernelGGL((prologue_quant_kernel<D, ROPE>), dim3(blocks), dim3(kPThreads), 0, st, p,
                     dequant, per_bh, codes);
  return launch_check("rmsnorm_quantize(apply)");
}

template <int D, int ROPE>
int run_norm_qkv(const NormQKV& a, hipStream_t st) {
  const int64_t amax_blocks = 3 * max(max(a.nq, a.nk), a.nv);
  const int64_t apply_blocks = 3 * max(max(a.nq, a.nk), a.nvt);
  hipLaunchKernelGGL((qkv_norm_amax_kernel<D, ROPE>), dim3((unsigned)amax_blocks),
                     dim3(kPThreads), 0, st, a);
  int rc = launch_check("rmsnorm_quantize_qkv(amax)");
  if (rc) return rc;
  hipLaunchKernelGGL(qkv_norm_finalize_kernel, dim3((unsigned)a.ngroups, 3), dim3(kPThreads), 0,
                     st, a);
  rc = launch_check("rmsnorm_quantize_qkv(finalize)");
  if (rc) return rc;
  hipLaunchKernelGGL((qkv_norm_apply_kernel<D, ROPE>), dim3((unsigned)apply_blocks),
                     dim3(kPThreads), 0, st, a);
  return launch_check("rmsnorm_quantize_qkv(apply)");
}

// Bytes of one tensor's partial maxima and of its rows' inverse norms.
struct PSizes {
  size_t partials, rinv;
};
bool prologue_sizes(int64_t B, int64_t H, int64_t S, int64_t D, int granularity, PSizes* out) {
  if (B <= 0 || H <= 0 || S <= 0 || (D != 64 && D != 128)) return false;
  if (granularity != RP_SCALE_PER_BH && granularity != RP_SCALE_PER_TENSOR) return false;
  const int64_t ngroups = granularity == RP_SCALE_PER_BH ? B * H : 1;
  const int64_t rows = B * H * S / ngroups;
  const int64_t rpb = kPElemsPerBlock / D;
  out->partials = (size_t)(ngroups * ((rows + rpb - 1) / rpb)) * sizeof(uint32_t);
  out->rinv = (size_t)(B * H * S) * sizeof(float);
  return true;
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Checks one tensor's prologue arguments (`who` prefixes each error) and
// fills its plan, all but p.rinv.
int make_pparams(const char* who, const void* x, int64_t B, int64_t H, int64_t S, int64_t D,
                 int64_t sb, int64_t sh, int64_t ss, const void* weight, float eps,
                 const float* rope_cos, const float* rope_sin, int rope_mode, int granularity,
                 const void* codes, PParams* out) {
  if (x == nullptr || codes == nullptr) {
    rp_set_error("%s: null pointer", who);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (B <= 0 || H <= 0 || S <= 0) {
    rp_set_error("%s: non-positive shape B=%lld H=%lld S=%lld", who, (long long)B, (long long)H,
                 (long long)S);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (D != 64 && D != 128) {
    rp_set_error("%s: head dim %lld not in {64, 128}", who, (long long)D);
    return RP_ERR_UNSUPPORTED;
  }
  if (granularity != RP_SCALE_PER_BH && granularity != RP_SCALE_PER_TENSOR) {
    rp_set_error("%s: unknown granularity %d", who, granularity);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (rope_mode != RP_ROPE_NONE && rope_mode != RP_ROPE_HALF && rope_mode != RP_ROPE_INTERLEAVED) {
    rp_set_error("%s: unknown rope_mode %d", who, rope_mode);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (rope_mode != RP_ROPE_NONE && (rope_cos == nullptr || rope_sin == nullptr)) {
    rp_set_error("%s: rope_mode %d needs cos and sin tables", who, rope_mode);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (!(eps >= 0.0f) || eps == __builtin_inff()) {
    rp_set_error("%s: eps=%g must be finite and >= 0", who, (double)eps);
    return RP_ERR_INVALID_ARGUMENT;
  }
  const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                          (uintptr_t)(sb * 2) | (uintptr_t)(sh * 2) | (uintptr_t)(ss * 2) |
                          reinterpret_cast<uintptr_t>(rope_cos) |
                          reinterpret_cast<uintptr_t>(rope_sin) |
                          reinterpret_cast<uintptr_t>(codes);
  if (align % 16 != 0) {
    rp_set_error("%s: x, weight, strides, tables and codes must be 16-byte aligned", who);
    return RP_ERR_UNSUPPORTED;
  }
  const int64_t ngroups = granularity == RP_SCALE_PER_BH ? B * H : 1;
  PParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.B = B; p.H = H; p.S = S; p.D = D; p.sb = sb; p.sh = sh; p.ss = ss;
  p.weight = static_cast<const uint16_t*>(weight);
  p.eps = eps;
  p.cosv = rope_mode != RP_ROPE_NONE ? rope_cos : nullptr;
  p.sinv = rope_mode != RP_ROPE_NONE ? rope_sin : nullptr;
  p.rows_per_group = B * H * S / ngroups;
  p.rpb = kPElemsPerBlock / D;
  p.nbg = (p.rows_per_group + p.rpb - 1) / p.rpb;
  if (3 * ngroups * p.nbg > 0x7fffffffLL) {
    rp_set_error("%s: grid too large", who);
    return RP_ERR_UNSUPPORTED;
  }
  *out = p;
  return RP_OK;
}

template <typename F>
int with_layout(int64_t D, int rope_mode, F&& f) {
  auto by_rope = [&](auto d_c) {
    if (rope_mode == RP_ROPE_HALF)
      return f(d_c, std::integral_constant<int, RP_ROPE_HALF>{});
    if (rope_mode == RP_ROPE_INTERLEAVED)
      return f(d_c, std::integral_constant<int, RP_ROPE_INTERLEAVED>{});
    return f(d_c, std::integral_constant<int, RP_ROPE_NONE>{});
  };
  if (D == 128) return by_rope(std::integral_constant<int, 128>{});
  return by_rope(std::integral_constant<int, 64>{});
}

}  // namespace
}  // namespace rp

using namespace rp;

extern "C" size_t rp_fp8_rmsnorm_quant_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D,
                                                       int granularity) {
  PSizes z;
  if (!prologue_sizes(B, H, S, D, granularity, &z)) return 0;
  // per-block partial maxima, then one fp32 inverse norm per row
  return align256(z.partials) + z.rinv;
}

extern "C" int rp_fp8_rmsnorm_scale_quantize(const void* x, int64_t B, int64_t H, int64_t S,
                                             int64_t D, int64_t sb, int64_t sh, int64_t ss,
                                             const void* weight, float eps, const float* rope_cos,
                                             const float* rope_sin, int rope_mode,
                                             int granularity, float* dequant_out, uint8_t* codes,
                                             void* workspace, size_t workspace_bytes,
                                             void* stream) {
  const char* who = "rmsnorm_quantize";
  if (dequant_out == nullptr) {
    rp_set_error("%s: null pointer", who);
    return RP_ERR_INVALID_ARGUMENT;
  }
  PParams p;
  int rc = make_pparams(who, x, B, H, S, D, sb, sh, ss, weight, eps, rope_cos, rope_sin,
                        rope_mode, granularity, codes, &p);
  if (rc) return rc;
  const size_t need = rp_fp8_rmsnorm_quant_workspace_bytes(B, H, S, D, granularity);
  if (workspace == nullptr || workspace_bytes < need) {
    rp_set_error("%s: workspace of %zu bytes needed, got %zu", who, need, workspace_bytes);
    return RP_ERR_WORKSPACE;
  }
  const int64_t ngroups = granularity == RP_SCALE_PER_BH ? B * H : 1;
  uint32_t* partial = static_cast<uint32_t*>(workspace);
  const size_t partial_bytes = (size_t)(ngroups * p.nbg) * sizeof(uint32_t);
  p.rinv = reinterpret_cast<float*>(static_cast<char*>(workspace) + align256(partial_bytes));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int per_bh = granularity == RP_SCALE_PER_BH;
  return with_layout(D, rope_mode, [&](auto d_c, auto r_c) {
    return run_prologue<decltype(d_c)::value, decltype(r_c)::value>(p, ngroups, dequant_out,
                                                                     codes, per_bh, partial, st);
  });
}

extern "C" size_t rp_fp8_rmsnorm_quant_qkv_workspace_bytes(int64_t B, int64_t H, int64_t Sq,
                                                           int64_t Skv, int64_t D,
                                                           int granularity) {
  PSizes zq, zk;
  if (!prologue_sizes(B, H, Sq, D, granularity, &zq) ||
      !prologue_sizes(B, H, Skv, D, granularity, &zk))
    return 0;
  Plan pv;
  if (make_plan(reinterpret_cast<const void*>(256), RP_DTYPE_BF16, B, H, Skv, D, H * Skv * D,
                Skv * D, D, granularity, &pv) != RP_OK)
    return 0;
  // Q's, K's and V's partial maxima, then Q's and K's inverse norms
  return align256(zq.partials) + align256(zk.partials) + align256(pv.ws_bytes) +
         align256(zq.rinv) + zk.rinv;
}

extern "C" int rp_fp8_rmsnorm_scale_quantize_qkv(
    const void* q, const void* k, const void* v, int64_t B, int64_t H, int64_t Sq, int64_t Skv,
    int64_t D, int64_t qsb, int64_t qsh, int64_t qss, int64_t ksb, int64_t ksh, int64_t kss,
    int64_t vsb, int64_t vsh, int64_t vss, const void* q_weight, const void* k_weight, float eps,
    const float* q_cos, const float* q_sin, const float* k_cos, const float* k_sin,
    int rope_mode, int granularity, float* dequant_out, uint8_t* q8, uint8_t* k8, uint8_t* vt8,
    int64_t ldv, void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "rmsnorm_quantize_qkv";
  if (v == nullptr || vt8 == nullptr || dequant_out == nullptr) {
    rp_set_error("%s: null pointer", who);
    return RP_ERR_INVALID_ARGUMENT;
  }
  NormQKV a{};
  int rc = make_pparams(who, q, B, H, Sq, D, qsb, qsh, qss, q_weight, eps, q_cos, q_sin,
                        rope_mode, granularity, q8, &a.q);
  if (rc) return rc;
  if ((rc = make_pparams(who, k, B, H, Skv, D, ksb, ksh, kss, k_weight, eps, k_cos, k_sin,
                         rope_mode, granularity, k8, &a.k)))
    return rc;
  Plan pv;
  if ((rc = make_plan(v, RP_DTYPE_BF16, B, H, Skv, D, vsb, vsh, vss, granularity, &pv))) return rc;
  if (ldv < Skv || ldv % 128 != 0) {
    rp_set_error("%s: V^T needs ldv >= Skv with ldv %% 128 == 0 (Skv=%lld ldv=%lld)", who,
                 (long long)Skv, (long long)ldv);
    return RP_ERR_UNSUPPORTED;
  }
  if ((reinterpret_cast<uintptr_t>(vt8) & 15u) != 0) {
    rp_set_error("%s: vt8 must be 16-byte aligned", who);
    return RP_ERR_UNSUPPORTED;
  }
  const size_t need = rp_fp8_rmsnorm_quant_qkv_workspace_bytes(B, H, Sq, Skv, D, granularity);
  if (workspace == nullptr || workspace_bytes < need ||
      reinterpret_cast<uintptr_t>(workspace) % 256 != 0) {
    rp_set_error("%s: workspace of %zu bytes (256-byte aligned) needed, got %zu", who, need,
                 workspace_bytes);
    return RP_ERR_WORKSPACE;
  }
  const int64_t ngroups = granularity == RP_SCALE_PER_BH ? B * H : 1;
  a.v = pv.p;
  a.vt = QParams{};
  a.vt.x = static_cast<const uint16_t*>(v);
  a.vt.B = B; a.vt.H = H; a.vt.S = Skv; a.vt.D = D;
  a.vt.sb = vsb; a.vt.sh = vsh; a.vt.ss = vss;
  a.vflat = pv.flat;
  a.per_bh = granularity == RP_SCALE_PER_BH;
  a.vgsize = pv.gsize;
  a.nq = ngroups * a.q.nbg;
  a.nk = ngroups * a.k.nbg;
  a.nv = pv.p.ngroups * pv.p.nbg;
  a.vt_tiles = ldv / 128;
  a.nvt = B * H * a.vt_tiles;
  a.ldv = ldv;
  a.ngroups = ngroups;
  if (3 * max(max(a.nq, a.nk), max(a.nv, a.nvt)) > 0x7fffffffLL) {
    rp_set_error("%s: grid too large", who);
    return RP_ERR_UNSUPPORTED;
  }
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  size_t off = 0;
  a.pq = reinterpret_cast<uint32_t*>(ws + off);
  off += align256((size_t)a.nq * sizeof(uint32_t));
  a.pk = reinterpret_cast<uint32_t*>(ws + off);
  off += align256((size_t)a.nk * sizeof(uint32_t));
  a.pv = reinterpret_cast<uint32_t*>(ws + off);
  off += align256(pv.ws_bytes);
  a.q.rinv = reinterpret_cast<float*>(ws + off);
  off += align256((size_t)(B * H * Sq) * sizeof(float));
  a.k.rinv = reinterpret_cast<float*>(ws + off);
  a.dequant = dequant_out;
  a.q8 = q8;
  a.k8 = k8;
  a.vt8 = vt8;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_layout(D, rope_mode, [&](auto d_c, auto r_c) {
    return run_norm_qkv<decltype(d_c)::value, decltype(r_c)::value>(a, st);
  });
}
