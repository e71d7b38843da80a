/*
 * CPU oracle for the FP8 attention hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker.  Nothing in the product path
 * (repercep_runtime_amd/) links or calls it.
 *
 * It restates, in plain C, the numerics of miteshs/repercep-runtime's FP8
 * path for the OCP e4m3fn format (the gfx950 format):
 *
 *   quantizer   kernels/triton_kernels/fp8_flash_attn_hopper.py:374-398
 *               (identical formula to the gfx942 one at
 *               kernels/triton_kernels/fp8_flash_attn.py:425-448, with
 *               FP8_MAX = 448 instead of 240)
 *   attention   kernels/triton_kernels/fp8_flash_attn.py:294-391 (kernel body)
 *               with the OCP P cast of fp8_flash_attn_hopper.py:322
 *   GEMM        kernels/hip/fp8_attn/fp8_gemm.hip:79-156 (epilogue: one fp32
 *               scale a_scale*b_scale applied to the fp32 accumulator, then
 *               a round-to-nearest-even cast to bf16)
 *
 * The e4m3fn encoder is written from the format definition (1 sign bit,
 * 4 exponent bits with bias 7, 3 mantissa bits, no infinities, S.1111.111
 * is NaN, largest finite 448) with round-to-nearest-even, which is the
 * rounding torch applies in Tensor.to(torch.float8_e4m3fn).  The tests pin
 * it against torch's own cast.
 *
 * Build: oracle/build_oracle.py (gcc -O2 -fopenmp -ffp-contract=off).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define E4M3_MAX 448.0f
/* Python evaluates 0.95 * 448 as 425.59999999999997; torch turns the
 * scalar into the fp32 value nearest to it, 425.6f. */
#define SCALE_DIVISOR 425.6f
/* torch.clamp(min=1e-6) on a bf16 tensor compares against bf16(1e-6). */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---------------------------------------------------------------- formats */

/* fp32 -> bf16 bits, round to nearest even (NaN stays NaN, quieted). */
uint16_t or_bf16_bits(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float or_bf16_to_f32(uint16_t b) { return u2f(((uint32_t)b) << 16); }

float or_bf16_round(float x) { return or_bf16_to_f32(or_bf16_bits(x)); }

/* fp32 -> OCP e4m3fn, round to nearest even, no saturation: magnitudes that
 * do not round to a finite e4m3 value (>= 464 after rounding, i.e. the
 * S.1111.111 pattern or beyond) become NaN, as torch's cast does. */
uint8_t or_e4m3fn_encode(float x) {
    uint32_t u = f2u(x);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint8_t)(sign | 0x7f);       /* NaN */
    float v = u2f(a);
    if (v >= 480.0f) return (uint8_t)(sign | 0x7f);          /* out of range */
    uint32_t code;
    if (v < 0.015625f) {
        /* Subnormal range of e4m3 (below 2^-6): quantum 2^-9.  v * 512 is
         * exact (power-of-two scaling of a number far from the fp32 limits);
         * rintf rounds half to even under the default rounding mode. */
        code = (uint32_t)rintf(v * 512.0f);   /* 0..8; 8 is the smallest normal */
    } else {
        uint32_t exp32 = a >> 23;              /* biased fp32 exponent */
        uint32_t mant = a & 0x7fffffu;
        uint32_t keep = mant >> 20;            /* top 3 mantissa bits */
        uint32_t rest = mant & 0xfffffu;       /* 20 discarded bits */
        uint32_t up = (rest > 0x80000u) || (rest == 0x80000u && (keep & 1u));
        code = ((exp32 - 127u + 7u) << 3) + keep + up;   /* carry ripples into exp */
    }
    if (code >= 0x7fu) return (uint8_t)(sign | 0x7f);
    return (uint8_t)(sign | code);
}

float or_e4m3fn_decode(uint8_t c) {
    uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
    float mag;
    if (e == 0xfu && m == 7u) return NAN;
    if (e == 0) mag = (float)m * (1.0f / 512.0f);
    else mag = ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
    return (c & 0x80u) ? -mag : mag;
}

void or_e4m3fn_encode_array(const float* x, int64_t n, uint8_t* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = or_e4m3fn_encode(x[i]);
}

/* --------------------------------------------------------------- quantizer */

/* amax of |x| over a bf16 array, as bf16 bits.  |x| bit patterns order as
 * unsigned integers exactly like their values, with NaN patterns above
 * +inf, so an integer max propagates NaN the way torch.amax does. */
uint16_t or_amax_bf16(const uint16_t* x, int64_t n) {
    uint16_t best = 0;
#pragma omp parallel for reduction(max : best) schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        uint16_t a = (uint16_t)(x[i] & 0x7fffu);
        if (a > best) best = a;
    }
    return best;
}

/* Strided variant: rows of `cols` contiguous bf16 elements, `nrows` rows
 * separated by `row_stride` elements. */
uint16_t or_amax_bf16_rows(const uint16_t* x, int64_t nrows, int64_t cols, int64_t row_stride) {
    uint16_t best = 0;
#pragma omp parallel for reduction(max : best) schedule(static)
    for (int64_t r = 0; r < nrows; ++r) {
        const uint16_t* p = x + r * row_stride;
        for (int64_t c = 0; c < cols; ++c) {
            uint16_t a = (uint16_t)(p[c] & 0x7fffu);
            if (a > best) best = a;
        }
    }
    return best;
}

/* dequant = (amax.clamp(min=1e-6) / (0.95 * FP8_MAX)).to(float32) where
 * amax is a bf16 tensor: the clamp happens in bf16, the division in fp32 and
 * its result is rounded to bf16 (the tensor's dtype) before widening.
 * fp8_flash_attn_hopper.py:383-385. */
float or_dequant_from_amax(uint16_t amax_bits) {
    float lo = or_bf16_round(1e-6f);
    float a = or_bf16_to_f32(amax_bits);
    if (!(a != a) && a < lo) a = lo;      /* clamp keeps NaN */
    return or_bf16_round(a / SCALE_DIVISOR);
}

/* codes = (x.float() * (1.0 / dequant)).clamp(-448, 448).to(float8_e4m3fn)
 * fp8_flash_attn_hopper.py:396-398.  1.0/dequant is one correctly rounded
 * fp32 reciprocal; the product is one fp32 multiply. */
static inline uint8_t quant_one(uint16_t xb, float qmul) {
    float v = or_bf16_to_f32(xb) * qmul;
    if (!(v != v)) {
        if (v > E4M3_MAX) v = E4M3_MAX;
        if (v < -E4M3_MAX) v = -E4M3_MAX;
    }
    return or_e4m3fn_encode(v);
}

float or_qmul_from_dequant(float dequant) { return 1.0f / dequant; }

void or_quantize_bf16(const uint16_t* x, int64_t n, float dequant, uint8_t* codes) {
    float qmul = 1.0f / dequant;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) codes[i] = quant_one(x[i], qmul);
}

void or_quantize_bf16_rows(const uint16_t* x, int64_t nrows, int64_t cols, int64_t row_stride,
                           float dequant, uint8_t* codes) {
    float qmul = 1.0f / dequant;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < nrows; ++r)
        for (int64_t c = 0; c < cols; ++c)
            codes[r * cols + c] = quant_one(x[r * row_stride + c], qmul);
}

/* -------------------------------------------------------- QK-norm prologue */

/* RMSNorm over D of bf16 rows, unit weight, no rotation: the C form of
 * oracle/prologue.py rmsnorm_rope(weight=None, rope=NONE), which restates the
 * processors' norm_q / norm_k (reference docs/walkthroughs/02-architecture.md:
 * 114-123) in the summation order the gfx950 prologue commits to:
 *   ss_c = x_8c^2 + ... + x_8c+7^2 in order, per 8-element chunk c;
 *   ss_c = ss_c + ss_(c^o) for o = D/16, ..., 1 (every chunk at once);
 *   r = 1 / sqrt(ss_0 * fp32(1/D) + eps);  y = bf16(x * r).
 * Every step is one correctly rounded fp32 operation (built without
 * contraction).  D is a multiple of 16, at most 512.  x and y: nrows x D. */
void or_rmsnorm_bf16_rows(const uint16_t* x, int64_t nrows, int D, float eps, uint16_t* y) {
    const float inv_d = (float)(1.0 / (double)D);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < nrows; ++r) {
        const uint16_t* xr = x + r * D;
        float ss[64], nxt[64];
        const int nc = D / 8;
        for (int c = 0; c < nc; ++c) {
            float acc = 0.0f;
            for (int i = 0; i < 8; ++i) {
                const float v = or_bf16_to_f32(xr[8 * c + i]);
                const float sq = v * v;
                acc = i == 0 ? sq : acc + sq;
            }
            ss[c] = acc;
        }
        for (int o = nc / 2; o >= 1; o /= 2) {
            for (int c = 0; c < nc; ++c) nxt[c] = ss[c] + ss[c ^ o];
            for (int c = 0; c < nc; ++c) ss[c] = nxt[c];
        }
        const float mean = ss[0] * inv_d;
        const float rn = 1.0f / sqrtf(mean + eps);
        for (int d = 0; d < D; ++d) y[r * D + d] = or_bf16_bits(or_bf16_to_f32(xr[d]) * rn);
    }
}

/* --------------------------------------------------------------- attention */

/* Mask modes: 0 none, 1 causal (kv <= q, fp8_flash_attn.py:350-352),
 * 2 shared-prefix candidates: kv < prefix is visible to every query; a query
 * at row q belongs to candidate q / suffix and sees suffix key
 * j = kv - prefix when j / suffix == q / suffix and j <= q. */
static inline int visible(int mask, int q, int kv, int prefix, int suffix) {
    if (mask == 1) return kv <= q;
    if (mask == 2) {
        if (kv < prefix) return 1;
        int j = kv - prefix;
        return (j / suffix == q / suffix) && (j <= q);
    }
    return 1;
}

/*
 * Tile-exact emulation of the FA-2 FP8 kernel for one (b, h) slice.
 * q8: (Sq, D) codes, k8/v8: (Skv, D) codes, all row-major.
 * For each listed query row, walks the key axis in tiles of block_n and
 * applies the reference's online-softmax update:
 *
 *   qk      = fp32(Q8 . K8^T) * qk_scale          qk_scale = sm*qs*ks  (:329, :346-347)
 *   masked  -> -inf                                 (:350-356)
 *   m_new   = max(m, rowmax(qk))                    (:359)
 *   alpha   = exp(m - m_new); p = exp(qk - m_new)   (:360-361)
 *   l       = l*alpha + sum(p)                      (:362, fp32 p, unquantized)
 *   acc    *= alpha                                 (:365)
 *   p8      = e4m3fn(p * 448)                       (hopper :322)
 *   acc    += fp32(p8 . V8) * (vs / 448)            (:376-380)
 *   out     = acc / l                               (:385)
 *
 * Dot products are accumulated exactly (double) and rounded to fp32 once,
 * standing in for the fp32 MFMA accumulator whose internal order is not
 * observable.  `pquant` = 0 replaces the P cast by the identity (used by
 * the tests to compare against an exact softmax).  Output is fp32.
 */
void or_attn_rows(const uint8_t* q8, const uint8_t* k8, const uint8_t* v8,
                  int Sq, int Skv, int D,
                  float q_scale, float k_scale, float v_scale, float sm_scale,
                  int block_n, int mask, int prefix, int suffix, int pquant,
                  const int32_t* rows, int nrows, float* out) {
    float lut[256];
    for (int c = 0; c < 256; ++c) lut[c] = or_e4m3fn_decode((uint8_t)c);
    const float qk_scale = (sm_scale * q_scale) * k_scale;
    const float pv_scale = v_scale / E4M3_MAX;
    (void)Sq;
#pragma omp parallel
    {
        float qv[512];
        float acc[512];
        double pv[512];
        float s[1024];
        float p[1024];
#pragma omp for schedule(dynamic, 1)
        for (int ri = 0; ri < nrows; ++ri) {
            int q = rows[ri];
            for (int d = 0; d < D; ++d) qv[d] = lut[q8[(int64_t)q * D + d]];
            for (int d = 0; d < D; ++d) acc[d] = 0.0f;
            float m = -INFINITY, l = 0.0f;
            for (int n0 = 0; n0 < Skv; n0 += block_n) {
                int nb = block_n;
                float mx = -INFINITY;
                for (int j = 0; j < nb; ++j) {
                    int kv = n0 + j;
                    float sj;
                    if (kv >= Skv || !visible(mask, q, kv, prefix, suffix)) {
                        sj = -INFINITY;
                    } else {
                        const uint8_t* kr = k8 + (int64_t)kv * D;
                        double dot = 0.0;
                        for (int d = 0; d < D; ++d) dot += (double)qv[d] * (double)lut[kr[d]];
                        sj = (float)dot * qk_scale;
                    }
                    s[j] = sj;
                    if (sj > mx) mx = sj;
                }
                float m_new = m > mx ? m : mx;
                float alpha = expf(m - m_new);
                double psum = 0.0;
                for (int j = 0; j < nb; ++j) {
                    p[j] = expf(s[j] - m_new);
                    psum += p[j];
                }
                l = l * alpha + (float)psum;
                for (int d = 0; d < D; ++d) { acc[d] = acc[d] * alpha; pv[d] = 0.0; }
                for (int j = 0; j < nb; ++j) {
                    int kv = n0 + j;
                    if (kv >= Skv) continue;          /* masked-load zeros (:369-370) */
                    float pj = pquant ? lut[or_e4m3fn_encode(p[j] * E4M3_MAX)] : p[j] * E4M3_MAX;
                    const uint8_t* vr = v8 + (int64_t)kv * D;
                    for (int d = 0; d < D; ++d) pv[d] += (double)pj * (double)lut[vr[d]];
                }
                for (int d = 0; d < D; ++d) acc[d] = acc[d] + (float)pv[d] * pv_scale;
                m = m_new;
            }
            for (int d = 0; d < D; ++d) out[(int64_t)ri * D + d] = acc[d] / l;
        }
    }
}

/* -------------------------------------------------------------------- GEMM */

/* C[m, n] = bf16( fp32(sum_k A8[m,k] * B8[k,n]) * (a_scale * b_scale) ).
 * a8: (M, K) row-major, bt8: (N, K) row-major (B transposed).  Only the
 * listed rows of C are produced (c: nrows x N, bf16 bits). */
void or_gemm_rows(const uint8_t* a8, const uint8_t* bt8, int M, int N, int K,
                  float a_scale, float b_scale, const int32_t* rows, int nrows, uint16_t* c) {
    float lut[256];
    for (int i = 0; i < 256; ++i) lut[i] = or_e4m3fn_decode((uint8_t)i);
    const float scale = a_scale * b_scale;
    (void)M;
#pragma omp parallel
    {
        float arow[16384];
#pragma omp for schedule(dynamic, 1)
        for (int ri = 0; ri < nrows; ++ri) {
            int m = rows[ri];
            for (int k = 0; k < K; ++k) arow[k] = lut[a8[(int64_t)m * K + k]];
            for (int n = 0; n < N; ++n) {
                const uint8_t* br = bt8 + (int64_t)n * K;
                double acc = 0.0;
                for (int k = 0; k < K; ++k) acc += (double)arow[k] * (double)lut[br[k]];
                c[(int64_t)ri * N + n] = or_bf16_bits((float)acc * scale);
            }
        }
    }
}

int or_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
