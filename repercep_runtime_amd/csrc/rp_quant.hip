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

#include "rp_quant_dev.h"

#include <stdarg.h>
#include <stdio.h>

#include <mutex>

namespace rp {
namespace {

__global__ __launch_bounds__(kQThreads) void amax_partial_kernel(QParams p, uint32_t* partial) {
  amax_partial_body(blockIdx.x, p, partial);
}

template <int DT>
__global__ __launch_bounds__(kQThreads) void scale_finalize_kernel(const uint32_t* partial,
                                                                   int64_t nbg, float* dequant) {
  scale_finalize_body<DT>(blockIdx.x, partial, nbg, dequant);
}

__global__ __launch_bounds__(kQThreads) void amax_flat_kernel(const uint16_t* x, int64_t gsize,
                                                              int64_t nbg, uint32_t* partial) {
  amax_flat_body(blockIdx.x, x, gsize, nbg, partial);
}

template <int DT>
__global__ __launch_bounds__(kQThreads) void quant_flat_kernel(const uint16_t* x, int64_t gsize,
                                                               int64_t nbg, const float* dequant,
                                                               int per_bh, uint8_t* codes) {
  quant_flat_body<DT>(blockIdx.x, x, gsize, nbg, dequant, per_bh, codes);
}

template <int DT>
__global__ __launch_bounds__(kQThreads) void quant_apply_kernel(QParams p, const float* dequant,
                                                                int per_bh, uint8_t* codes) {
  quant_apply_body<DT>(blockIdx.x, p, dequant, per_bh, codes);
}

template <int DT>
__global__ __launch_bounds__(kQThreads) void quant_apply_t_kernel(QParams p, const float* dequant,
                                                                  int per_bh, uint8_t* codes,
                                                                  int64_t ld) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kTileBytes];
  apply_t_body<DT, true>(p, dequant, per_bh, codes, ld, blockIdx.x, blockIdx.y, blockIdx.z,
                         tile);
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

// Calls whose groups have at most kFoldMaxPartials amax partials (small
// tensors: C1, C5): every apply block folds its own group's partials into
// the scale -- a few hundred bytes from L2, the same max and the same
// rounding as the finalize kernel -- and the first block of each group
// writes it, so the scales need no launch of their own, and V^T's tiles
// (blockIdx.y == 2) run in the same launch: two launches per call instead
// of four, which is what bounds calls this small.  Without Q's codes (an
// attention launch that quantizes Q itself) only K and V need to be small:
// job 0 has no codes, and its first ngroups blocks fold Q's partials into
// Q's scales, however many there are (the finalize kernel's work, one block
// per group).
constexpr int64_t kFoldMaxPartials = 256;

template <int DT>
__global__ __launch_bounds__(kQThreads) void apply_fold_multi_kernel(QJobs3 jobs, QParams vt,
                                                                     int64_t ld,
                                                                     int64_t vt_stiles,
                                                                     int64_t vt_dtiles,
                                                                     uint8_t* vt8) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kTileBytes];
  const QJob& jb = job_of(jobs);
  const int64_t blk = blockIdx.x;
  if (blockIdx.y < 2) {
    if (jb.codes == nullptr) {   // Q's scales only
      if (blk >= jb.p.ngroups) return;
      const float dq = dequant_from_amax<DT>(
          block_max_u32<kQThreads>(jb.partial + blk * jb.p.nbg, jb.p.nbg));
      if (threadIdx.x == 0) jb.dequant[blk] = dq;
      return;
    }
    if (blk >= jb.nblocks) return;
    const int64_t g = blk / jb.p.nbg;
    const float dq =
        dequant_from_amax<DT>(block_max_u32<kQThreads>(jb.partial + g * jb.p.nbg, jb.p.nbg));
    if (blk == g * jb.p.nbg && threadIdx.x == 0) jb.dequant[g] = dq;
    if (jb.flat)
      quant_flat_core<DT>(blk, jb.p.x, jb.gsize, jb.p.nbg, 1.0f / dq, jb.codes);
    else
      quant_apply_core<DT>(blk, jb.p, 1.0f / dq, jb.codes);
  } else {
    // V^T tile (s tile sb, d tile db) of head bh
    if (blk >= vt_stiles * vt_dtiles * vt.B * vt.H) return;
    const int64_t sb = blk % vt_stiles, rest = blk / vt_stiles;
    const int64_t db = rest % vt_dtiles, bh = rest / vt_dtiles;
    const int64_t g = jb.per_bh ? bh : 0;
    const float dq =
        dequant_from_amax<DT>(block_max_u32<kQThreads>(jb.partial + g * jb.p.nbg, jb.p.nbg));
    if (sb == 0 && db == 0 && bh == g && threadIdx.x == 0) jb.dequant[g] = dq;
    uint32_t w[4][2];
    apply_t_load<DT, true>(vt, 1.0f / dq, sb, db, bh, w);
    apply_t_store(vt, w, vt8, ld, sb, db, bh, tile);
  }
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
  // q8 may be null: Q's scale only (an attention launch that quantizes its
  // own Q rows from the input, rp_fp8_attn_fwd_q16)
  if (q == nullptr || k == nullptr || v == nullptr || dequant_out == nullptr ||
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
  const int64_t vt_stiles = ldv / 128, vt_dtiles = (D + 63) / 64;
  const int64_t vt_blocks = vt_stiles * vt_dtiles * B * H;
  // (with Q's codes, Q's own apply blocks write its scale; without them,
  // job 0's first blocks do, from any number of partials)
  const int64_t fold_blocks =
      max(q8 != nullptr ? apply_blocks : max(jobs.j1.nblocks, ng), vt_blocks);
  if ((q8 == nullptr || pq.p.nbg <= kFoldMaxPartials) &&
      max(pk.p.nbg, pv.p.nbg) <= kFoldMaxPartials && fold_blocks <= 0x7fffffff) {
    QParams vt{};
    vt.x = static_cast<const uint16_t*>(v);
    vt.B = B; vt.H = H; vt.S = Skv; vt.D = D; vt.sb = vsb; vt.sh = vsh; vt.ss = vss;
    const dim3 grid((unsigned)fold_blocks, 3);
    if (x_dtype == RP_DTYPE_F16)
      hipLaunchKernelGGL(apply_fold_multi_kernel<kInF16>, grid, dim3(kQThreads), 0, st, jobs, vt,
                         ldv, vt_stiles, vt_dtiles, vt8);
    else
      hipLaunchKernelGGL(apply_fold_multi_kernel<kInBf16>, grid, dim3(kQThreads), 0, st, jobs,
                         vt, ldv, vt_stiles, vt_dtiles, vt8);
    return check_launch("apply_fold_multi");
  }
  // the Q and K codes (blockIdx.y 0 and 1), or K's alone (as job 0) when q8
  // is null
  QJobs3 apply_jobs = jobs;
  int n_apply = 2;
  int64_t blocks = apply_blocks;
  if (q8 == nullptr) {
    apply_jobs.j0 = jobs.j1;
    n_apply = 1;
    blocks = jobs.j1.nblocks;
  }
  if (x_dtype == RP_DTYPE_F16) {
    hipLaunchKernelGGL(finalize_multi_kernel<kInF16>, dim3((unsigned)ng, 3), dim3(kQThreads), 0,
                       st, jobs);
    hipLaunchKernelGGL(apply_multi_kernel<kInF16>, dim3((unsigned)blocks, n_apply),
                       dim3(kQThreads), 0, st, apply_jobs);
  } else {
    hipLaunchKernelGGL(finalize_multi_kernel<kInBf16>, dim3((unsigned)ng, 3), dim3(kQThreads), 0,
                       st, jobs);
    hipLaunchKernelGGL(apply_multi_kernel<kInBf16>, dim3((unsigned)blocks, n_apply),
                       dim3(kQThreads), 0, st, apply_jobs);
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
// the first call for that device (with that device current).  The lookup may
// load the code object, which a stream under graph capture must not see:
// a first call on a device made while `stream` is capturing is refused, so
// one call outside capture has to come first on every device.
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
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if ((e = hipStreamIsCapturing(st, &cap)) != hipSuccess || cap != hipStreamCaptureStatusNone) {
      rp_set_error("scale_quantize_qkv_noalloc: the first call on device %d must be made "
                   "outside graph capture (it looks up the scratch address)%s%s", dev,
                   e != hipSuccess ? ": " : "", e != hipSuccess ? hipGetErrorString(e) : "");
      return RP_ERR_INVALID_ARGUMENT;
    }
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
    // give the caller back its current device; a failed restore is an error
    // even when the lookup worked (the caller's later calls would run on the
    // wrong device)
    const hipError_t er = cur != dev ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess || ptr == nullptr) {
      rp_set_error("scale_quantize_qkv_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                   dev, hipGetErrorString(e));
      return RP_ERR_LAUNCH;
    }
    if (er != hipSuccess) {
      rp_set_error("scale_quantize_qkv_noalloc: restoring device %d: %s", cur,
                   hipGetErrorString(er));
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
