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
//   ss   = sum over d of x_d^2        fp32; each thread sums its 8 elements
//                                     in order, then a butterfly over the
//                                     row's D/8 threads (xor D/16 ... 1)
//   r    = 1 / sqrt(ss * (1/D) + eps) IEEE sqrt and divide (two roundings)
//   n_d  = bf16(x_d * r)              then, with a weight, bf16(n_d * w_d)
//   y_d  = bf16(n_d * cos_d + rot(n)_d * sin_d)      three fp32 roundings
//          rot(n) = (-n[D/2:], n[:D/2]) for RP_ROPE_HALF,
//                   (-n_1, n_0, -n_3, n_2, ...) for RP_ROPE_INTERLEAVED
// and y is then scaled and quantized exactly as rp_fp8_scale_quantize does
// (dequant = bf16(max(amax|y|, bf16(1e-6)) / 425.6), code = e4m3fn RNE of
// clamp(y * RN(1/dequant), +-448)).  No step is contracted into an FMA
// (`#pragma clang fp contract(off)`), so every rounding above happens.

#include "rp_common.h"

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
// The first steps of prologue_rows: the 8 elements of each row as fp32 and
// each row's r = 1/sqrt(mean(x^2) + eps).
template <int D, int U, bool LOAD, bool STORE>
__device__ __forceinline__ void load_norm(const PParams& p, const uint16_t* const (&xrow)[U],
                                          const int64_t (&row)[U], int c, float (&x)[U][8],
                                          float (&r)[U]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint4 v = *reinterpret_cast<const uint4*>(xrow[u] + 8 * c);
    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[u][2 * i] = bf16_to_f32(w4[i] & 0xffffu);
      x[u][2 * i + 1] = bf16_to_f32(w4[i] >> 16);
    }
  }
  if constexpr (LOAD) {
#pragma unroll
    for (int u = 0; u < U; ++u) r[u] = p.rinv[row[u]];
  } else {
    float ss[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ss[u] = x[u][0] * x[u][0];
#pragma unroll
      for (int i = 1; i < 8; ++i) ss[u] = ss[u] + x[u][i] * x[u][i];
    }
    if constexpr (D == 128) {
      // a row is one 16-lane DPP row: the butterfly by row rotations
#pragma unroll
      for (int u = 0; u < U; ++u) {
        ss[u] = add_row_ror<8>(ss[u]);
        ss[u] = add_row_ror<4>(ss[u]);
        ss[u] = add_row_ror<2>(ss[u]);
        ss[u] = add_row_ror<1>(ss[u]);
      }
    } else {
#pragma unroll
      for (int o = D / 16; o >= 1; o >>= 1)
#pragma unroll
        for (int u = 0; u < U; ++u) ss[u] = ss[u] + shfl_xor(ss[u], o);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      r[u] = 1.0f / __builtin_sqrtf(ss[u] * (1.0f / D) + p.eps);
      if (STORE && c == 0) p.rinv[row[u]] = r[u];
    }
  }
}

template <int D, int ROPE, int U, bool LOAD, bool STORE>
__device__ __forceinline__ void prologue_rows(const PParams& p, const uint16_t* const (&xrow)[U],
                                              const int64_t (&s)[U], const int64_t (&row)[U],
                                              int c, float (&y)[U][8]) {
#pragma clang fp contract(off)
  float x[U][8], r[U];
  load_norm<D, U, LOAD, STORE>(p, xrow, row, c, x, r);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int i = 0; i < 8; ++i) y[u][i] = bf16r(x[u][i] * r[u]);
  if (p.weight != nullptr) {
    const uint4 wv = *reinterpret_cast<const uint4*>(p.weight + 8 * c);
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        y[u][2 * i] = bf16r(y[u][2 * i] * bf16_to_f32(ww[i] & 0xffffu));
        y[u][2 * i + 1] = bf16r(y[u][2 * i + 1] * bf16_to_f32(ww[i] >> 16));
      }
  }
  if constexpr (ROPE == RP_ROPE_NONE) return;
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

// Whether the apply pass reads each row's inverse norm back from the amax pass.
template <int ROPE>
constexpr bool kStoreNorm = ROPE == RP_ROPE_NONE;

// Row iteration shared by both passes: block blk covers rows
// [first, first + nrows) of group g; thread t works on row offsets
// t / (D/8) + j * STEP and 8-element chunk t % (D/8).  Each loop step hands
// fn U rows, STEP apart; a row past the block's range is
// replaced by the step's first row (read, never used: ok[u] is false).
template <int D, int U, typename F>
__device__ __forceinline__ void for_rows(const PParams& p, F&& fn) {
  constexpr int TPR = D / 8;
  constexpr int STEP = kPThreads / TPR;
  const int64_t blk = blockIdx.x;
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
__global__ __launch_bounds__(kPThreads) void prologue_amax_kernel(PParams p, uint32_t* partial) {
  constexpr int U = kPRowsPerStep<ROPE>;
  uint32_t m = 0;
  if (ROPE == RP_ROPE_NONE && p.weight == nullptr) {
    // y = bf16(x * r) is only needed for its maximum: take it from the
    // packed bf16 pairs, two per packed 16-bit max.  A row past the range
    // repeats a row of the range (the same maximum), so it needs no mask.
    uint32_t m2 = 0;
    for_rows<D, U>(p, [&](const int64_t (&r)[U], const int64_t (&)[U], const int64_t (&)[U],
                       const uint16_t* const (&xrow)[U], const bool (&)[U], int c) {
#pragma clang fp contract(off)
      float x[U][8], rn[U];
      load_norm<D, U, false, kStoreNorm<ROPE>>(p, xrow, r, c, x, rn);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < 8; i += 2)
          m2 = pk_max_u16(m2, pk_bf16(x[u][i] * rn[u], x[u][i + 1] * rn[u]) & 0x7fff7fffu);
    });
    m = umax32(m2 & 0xffffu, m2 >> 16);
  } else {
    for_rows<D, U>(p, [&](const int64_t (&r)[U], const int64_t (&)[U], const int64_t (&s)[U],
                       const uint16_t* const (&xrow)[U], const bool (&ok)[U], int c) {
      float y[U][8];
      prologue_rows<D, ROPE, U, false, kStoreNorm<ROPE>>(p, xrow, s, r, c, y);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i)
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
    partial[blockIdx.x] = r;
  }
}

__global__ __launch_bounds__(kPThreads) void prologue_finalize_kernel(const uint32_t* partial,
                                                                      int64_t nbg,
                                                                      float* dequant) {
  const int64_t g = blockIdx.x;
  const uint32_t r = block_max_u32<kPThreads>(partial + g * nbg, nbg);
  if (threadIdx.x == 0) dequant[g] = dequant_from_amax_bits(r);
}

template <int D, int ROPE>
__global__ __launch_bounds__(kPThreads) void prologue_quant_kernel(PParams p,
                                                                   const float* dequant,
                                                                   int per_bh, uint8_t* codes) {
  constexpr int U = kPRowsPerStep<ROPE>;
  for_rows<D, U>(p, [&](const int64_t (&r)[U], const int64_t (&bh)[U], const int64_t (&s)[U],
                     const uint16_t* const (&xrow)[U], const bool (&ok)[U], int c) {
    float y[U][8];
    prologue_rows<D, ROPE, U, kStoreNorm<ROPE>, false>(p, xrow, s, r, c, y);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!ok[u]) continue;
      const float qm = 1.0f / dequant[per_bh ? bh[u] : 0];
      uint2 o;
      o.x = pack4_e4m3(clamp_e4m3(y[u][0] * qm), clamp_e4m3(y[u][1] * qm),
                       clamp_e4m3(y[u][2] * qm), clamp_e4m3(y[u][3] * qm));
      o.y = pack4_e4m3(clamp_e4m3(y[u][4] * qm), clamp_e4m3(y[u][5] * qm),
                       clamp_e4m3(y[u][6] * qm), clamp_e4m3(y[u][7] * qm));
      *reinterpret_cast<uint2*>(codes + r[u] * D + 8 * c) = o;
    }
  });
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

}  // namespace
}  // namespace rp

using namespace rp;

extern "C" size_t rp_fp8_rmsnorm_quant_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D,
                                                       int granularity) {
  if (B <= 0 || H <= 0 || S <= 0 || (D != 64 && D != 128)) return 0;
  if (granularity != RP_SCALE_PER_BH && granularity != RP_SCALE_PER_TENSOR) return 0;
  const int64_t ngroups = granularity == RP_SCALE_PER_BH ? B * H : 1;
  const int64_t rows = B * H * S / ngroups;
  const int64_t rpb = kPElemsPerBlock / D;
  // per-block partial maxima, then one fp32 inverse norm per row
  const size_t partials = (size_t)(ngroups * ((rows + rpb - 1) / rpb)) * sizeof(uint32_t);
  return (partials + 255) / 256 * 256 + (size_t)(B * H * S) * sizeof(float);
}

extern "C" int rp_fp8_rmsnorm_scale_quantize(const void* x, int64_t B, int64_t H, int64_t S,
                                             int64_t D, int64_t sb, int64_t sh, int64_t ss,
                                             const void* weight, float eps, const float* rope_cos,
                                             const float* rope_sin, int rope_mode,
                                             int granularity, float* dequant_out, uint8_t* codes,
                                             void* workspace, size_t workspace_bytes,
                                             void* stream) {
  if (x == nullptr || dequant_out == nullptr || codes == nullptr) {
    rp_set_error("rmsnorm_quantize: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (B <= 0 || H <= 0 || S <= 0) {
    rp_set_error("rmsnorm_quantize: non-positive shape B=%lld H=%lld S=%lld", (long long)B,
                 (long long)H, (long long)S);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (D != 64 && D != 128) {
    rp_set_error("rmsnorm_quantize: head dim %lld not in {64, 128}", (long long)D);
    return RP_ERR_UNSUPPORTED;
  }
  if (granularity != RP_SCALE_PER_BH && granularity != RP_SCALE_PER_TENSOR) {
    rp_set_error("rmsnorm_quantize: unknown granularity %d", granularity);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (rope_mode != RP_ROPE_NONE && rope_mode != RP_ROPE_HALF && rope_mode != RP_ROPE_INTERLEAVED) {
    rp_set_error("rmsnorm_quantize: unknown rope_mode %d", rope_mode);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (rope_mode != RP_ROPE_NONE && (rope_cos == nullptr || rope_sin == nullptr)) {
    rp_set_error("rmsnorm_quantize: rope_mode %d needs cos and sin tables", rope_mode);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (!(eps >= 0.0f) || eps == __builtin_inff()) {
    rp_set_error("rmsnorm_quantize: eps=%g must be finite and >= 0", (double)eps);
    return RP_ERR_INVALID_ARGUMENT;
  }
  const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                          (uintptr_t)(sb * 2) | (uintptr_t)(sh * 2) | (uintptr_t)(ss * 2) |
                          reinterpret_cast<uintptr_t>(rope_cos) |
                          reinterpret_cast<uintptr_t>(rope_sin) |
                          reinterpret_cast<uintptr_t>(codes);
  if (align % 16 != 0) {
    rp_set_error("rmsnorm_quantize: x, weight, strides, tables and codes must be 16-byte aligned");
    return RP_ERR_UNSUPPORTED;
  }
  const size_t need = rp_fp8_rmsnorm_quant_workspace_bytes(B, H, S, D, granularity);
  if (workspace == nullptr || workspace_bytes < need) {
    rp_set_error("rmsnorm_quantize: workspace of %zu bytes needed, got %zu", need,
                 workspace_bytes);
    return RP_ERR_WORKSPACE;
  }
  const int64_t ngroups = granularity == RP_SCALE_PER_BH ? B * H : 1;
  PParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.B = B; p.H = H; p.S = S; p.D = D; p.sb = sb; p.sh = sh; p.ss = ss;
  p.weight = static_cast<const uint16_t*>(weight);
  p.eps = eps;
  p.cosv = rope_cos; p.sinv = rope_sin;
  p.rows_per_group = B * H * S / ngroups;
  p.rpb = kPElemsPerBlock / D;
  p.nbg = (p.rows_per_group + p.rpb - 1) / p.rpb;
  if (ngroups * p.nbg > 0x7fffffffLL) {
    rp_set_error("rmsnorm_quantize: grid too large");
    return RP_ERR_UNSUPPORTED;
  }
  uint32_t* partial = static_cast<uint32_t*>(workspace);
  const size_t partial_bytes = (size_t)(ngroups * p.nbg) * sizeof(uint32_t);
  p.rinv = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                    (partial_bytes + 255) / 256 * 256);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int per_bh = granularity == RP_SCALE_PER_BH;
  auto run = [&](auto d_c) {
    constexpr int DD = decltype(d_c)::value;
    if (rope_mode == RP_ROPE_HALF)
      return run_prologue<DD, RP_ROPE_HALF>(p, ngroups, dequant_out, codes, per_bh, partial, st);
    if (rope_mode == RP_ROPE_INTERLEAVED)
      return run_prologue<DD, RP_ROPE_INTERLEAVED>(p, ngroups, dequant_out, codes, per_bh,
                                                   partial, st);
    return run_prologue<DD, RP_ROPE_NONE>(p, ngroups, dequant_out, codes, per_bh, partial, st);
  };
  if (D == 128) return run(std::integral_constant<int, 128>{});
  return run(std::integral_constant<int, 64>{});
}
