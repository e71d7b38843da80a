/*
 * repercep_fp8.h -- C ABI of the MI355X (gfx950) FP8 attention hot path.
 *
 * One shared library, librepercep_fp8.so, built from the .hip sources in
 * repercep_runtime_amd/csrc.  Plain pointers and sizes only: device
 * pointers come from any HIP allocator, streams are hipStream_t passed as
 * void* (NULL = the legacy default stream).  Every call is stream-ordered and
 * asynchronous, allocates nothing, and returns an int status (RP_OK = 0);
 * rp_last_error() gives a message for the calling thread's last failure.
 *
 * Number formats: FP8 codes are OCP e4m3fn bytes (bias 7, max 448,
 * 0x7f/0xff = NaN, no infinities) -- the format gfx950 MFMAs consume.  Scales
 * are *dequant* scales (fp32 multiplier that maps a code back to the input
 * magnitude), one per group, exactly as the reference's _per_bh_scale
 * returns them.
 *
 * Reference: miteshs/repercep-runtime.  Each entry point names the interface
 * it replaces (file:line under the reference tree).
 */
#ifndef REPERCEP_FP8_H
#define REPERCEP_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------- status */
#define RP_OK 0
#define RP_ERR_INVALID_ARGUMENT 1 /* null pointer, bad size/stride/enum        */
#define RP_ERR_UNSUPPORTED 2      /* shape outside the compiled kernel set      */
#define RP_ERR_WORKSPACE 3        /* workspace missing or too small             */
#define RP_ERR_LAUNCH 4           /* the HIP runtime rejected a kernel launch   */

/* Scale granularity (a group shares one amax/dequant scale). */
#define RP_SCALE_PER_BH 0     /* one group per (batch, head): the reference's  */
#define RP_SCALE_PER_TENSOR 1 /* one group for the whole tensor                */

/* Layout of quantized codes written by rp_fp8_quantize*. */
#define RP_LAYOUT_BHSD 0 /* (B, H, S, D) contiguous                              */
#define RP_LAYOUT_BHDS 1 /* per (b, h): D rows of `ld` codes (S transposed), the */
                         /* tail [S, ld) zero-filled; V operand of attention     */

/* Output element type of rp_fp8_attn_fwd. */
#define RP_OUT_BF16 0
#define RP_OUT_F32 1
#define RP_OUT_F16 2

/* Input element type of the quantizer entry points (x_dtype). */
#define RP_DTYPE_BF16 0
#define RP_DTYPE_F16 1

/* Mask kinds of rp_fp8_attn_fwd. */
/* rotary-embedding layouts of rp_fp8_rmsnorm_scale_quantize, as diffusers'
 * apply_rotary_emb(use_real=True) pairs elements */
#define RP_ROPE_NONE 0
#define RP_ROPE_HALF 1        /* d pairs with d +- D/2 (use_real_unbind_dim=-2) */
#define RP_ROPE_INTERLEAVED 2 /* 2k pairs with 2k+1   (use_real_unbind_dim=-1) */

#define RP_MASK_NONE 0
#define RP_MASK_CAUSAL 1        /* key kv visible to query q iff kv <= q          */
#define RP_MASK_SHARED_PREFIX 2 /* keys [0, prefix) visible to all queries; query */
                                /* q sees suffix key j = kv - prefix iff          */
                                /* j / suffix == q / suffix and j <= q            */

/* 3: rp_fp8_gemm / rp_fp8_linear take b_layout (RP_B_KN or RP_B_NK). */
int rp_abi_version(void);
const char* rp_status_string(int status);
const char* rp_last_error(void);

/* ---------------------------------------------------------- quantize
 * Input x: bf16 or fp16 (x_dtype RP_DTYPE_*) viewed as (B, H, S, D) with
 * element strides sb, sh, ss for the first three axes and unit stride along
 * D.  D must be a multiple of 8.
 *
 * rp_fp8_quant_workspace_bytes: device scratch the two-pass quantizer needs
 * (per-block partial maxima plus per-group multipliers).
 */
size_t rp_fp8_quant_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D, int granularity);

/* Per-group dequant scales, computed in the input dtype as the reference's
 * torch expression evaluates on the GPU:
 *   bf16: dequant = bf16(max(amax|x|, bf16(1e-6)) / 425.6)
 *   fp16: dequant = fp16(max(amax|x|, fp16(1e-6)) * fp32(1 / 425.6))
 * Replaces _per_bh_scale, kernels/triton_kernels/fp8_flash_attn_hopper.py:374-385
 * (OCP sibling of kernels/triton_kernels/fp8_flash_attn.py:425-436).
 * dequant_out: float[B*H] (RP_SCALE_PER_BH) or float[1] (RP_SCALE_PER_TENSOR). */
int rp_fp8_scale(const void* x, int x_dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                 int64_t sb, int64_t sh, int64_t ss, int granularity,
                 float* dequant_out, void* workspace, size_t workspace_bytes, void* stream);

/* Codes = e4m3fn(clamp(x * (1 / dequant), -448, 448)), round to nearest even,
 * given the per-group dequant scales.
 * Replaces _quantize, kernels/triton_kernels/fp8_flash_attn_hopper.py:388-398
 * (OCP sibling of kernels/triton_kernels/fp8_flash_attn.py:439-448) and the
 * .contiguous() that follows it (fp8_flash_attn.py:526-528).
 * layout RP_LAYOUT_BHSD: codes (B, H, S, D) contiguous, ld ignored.
 * layout RP_LAYOUT_BHDS: codes (B, H, D, ld), ld >= S and ld % 128 == 0,
 *                        D % 32 == 0; columns [S, ld) are written as 0. */
int rp_fp8_quantize(const void* x, int x_dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                    int64_t sb, int64_t sh, int64_t ss, int granularity,
                    const float* dequant, uint8_t* codes, int layout, int64_t ld,
                    void* stream);

/* rp_fp8_scale followed by rp_fp8_quantize in one stream-ordered call
 * (the pair _per_bh_scale + _quantize at fp8_flash_attn.py:522-528). */
int rp_fp8_scale_quantize(const void* x, int x_dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                          int64_t sb, int64_t sh, int64_t ss, int granularity,
                          float* dequant_out, uint8_t* codes, int layout, int64_t ld,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Q, K and V of one attention call in one call: the scales and codes of
 * rp_fp8_scale_quantize for q and k ((B, H, S, D) codes) and for v (V^T,
 * (B, H, D, ldv)), from four kernel launches (amax of all three, their
 * scales, q and k codes, V^T codes) instead of nine -- launches bound small
 * calls.  dequant_out: float[3 * G], G = B*H (RP_SCALE_PER_BH) or 1, in the
 * order q, k, v.  workspace: rp_fp8_quant_qkv_workspace_bytes, 256-byte
 * aligned.  Replaces the three _per_bh_scale + _quantize pairs at
 * kernels/triton_kernels/fp8_flash_attn.py:522-528 with one host call.
 * q8 may be NULL: Q's scale is computed and no Q codes are written, for an
 * attention launch that quantizes Q itself (rp_fp8_attn_fwd_q16). */
size_t rp_fp8_quant_qkv_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Skv,
                                        int64_t D, int granularity);
int rp_fp8_scale_quantize_qkv(const void* q, const void* k, const void* v, int x_dtype,
                              int64_t B, int64_t H, int64_t Sq, int64_t Skv, int64_t D,
                              int64_t qsb, int64_t qsh, int64_t qss, int64_t ksb, int64_t ksh,
                              int64_t kss, int64_t vsb, int64_t vsh, int64_t vss,
                              int granularity, float* dequant_out, uint8_t* q8, uint8_t* k8,
                              uint8_t* vt8, int64_t ldv, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Allocation-free variant of rp_fp8_scale_quantize_qkv.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory --
 * code under HIP graph capture, serving loops and harnesses that forbid
 * hipMalloc.  Same arguments, scales and codes as rp_fp8_scale_quantize_qkv,
 * without the workspace: the partial maxima go to a static device array of
 * RP_QKV_NOALLOC_SCRATCH_BYTES that each GPU holds until the process ends
 * (the library allocates nothing, here or on any later call).  Shapes whose
 * rp_fp8_quant_qkv_workspace_bytes exceeds that size are refused with
 * RP_ERR_WORKSPACE (at 16384 elements per partial, 1 MiB covers e.g. three
 * 1.4e9-element tensors per tensor-scale, fewer with many small heads).
 * Every call on one GPU shares that GPU's array: calls that may overlap on
 * one GPU (two streams, two host threads) race and must be serialised by
 * the caller; calls in one stream are ordered.  The first call on each GPU
 * looks up the array's device address and must be made outside graph
 * capture (under capture it returns RP_ERR_INVALID_ARGUMENT); later calls
 * may be captured and replayed. */
#define RP_QKV_NOALLOC_SCRATCH_BYTES (1u << 20)
int rp_fp8_scale_quantize_qkv_noalloc(const void* q, const void* k, const void* v, int x_dtype,
                                      int64_t B, int64_t H, int64_t Sq, int64_t Skv, int64_t D,
                                      int64_t qsb, int64_t qsh, int64_t qss, int64_t ksb,
                                      int64_t ksh, int64_t kss, int64_t vsb, int64_t vsh,
                                      int64_t vss, int granularity, float* dequant_out,
                                      uint8_t* q8, uint8_t* k8, uint8_t* vt8, int64_t ldv,
                                      void* stream);

/* ------------------------------------------------------- row-wise FP8
 * Per-row scales: each of `rows` rows of `cols` contiguous elements (bf16 or
 * fp16, row stride ldx elements) gets its own amax over the row and
 *   dequant_out[r] = dtype(max(amax, dtype(1e-6)) / 425.6)
 *   codes[r, :]    = e4m3fn(clamp(x * dtype(dtype(1 / amax) * 425.6), -448, 448))
 * (RNE; codes rows of stride ldq bytes).  Replaces _rowwise_quantize,
 * src/repercep/attention/fp8_scaled_mm.py:107-133 (amax over the last axis;
 * `target / amax` evaluates as amax.reciprocal() * target, two roundings to
 * the input dtype), with the OCP e4m3fn constants (448, 0.95 * 448) as the
 * OCP siblings of the per-(b,h) quantizer use them.  cols, ldx, ldq
 * multiples of 8; x 16-byte and codes 8-byte aligned. */
int rp_fp8_rowwise_quantize(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ldx,
                            float* dequant_out, uint8_t* codes, int64_t ldq, void* stream);

/* 16-bit transpose of `batch` (R, C) matrices: dst_z (C, R) <- src_z (R, C),
 * row strides lds / ldd and batch strides bs / bd in elements.  The
 * reference's v.transpose(-1, -2).contiguous() ahead of V's row-wise
 * quantization (src/repercep/attention/fp8_scaled_mm.py:167-168). */
int rp_transpose16(const void* src, void* dst, int64_t batch, int64_t R, int64_t C, int64_t lds,
                   int64_t ldd, int64_t bs, int64_t bd, void* stream);

/* Softmax of raw bf16 scores and P's row-wise quantization in one pass per
 * row: for row r (query q = r % sq) of `cols` raw scores (row stride lds),
 *   s_j = bf16(raw_j * scale), -inf for j > q when causal
 *   p_j = bf16(exp(s_j - max s) / sum_k exp(s_k - max s))   (fp32 math)
 *   dequant_out[r], codes[r, :] = the row-wise quantization of p (as above)
 * Replaces `scores_raw * scale`, the causal masked_fill, torch.softmax in
 * bf16 and _rowwise_quantize(p) of src/repercep/attention/fp8_scaled_mm.py:
 * 159-171.  cols, lds, ldq even; scores 4-byte aligned. */
int rp_fp8_softmax_rowwise_quantize(const void* scores, int64_t rows, int64_t cols, int64_t lds,
                                    int64_t sq, int causal, float scale, float* dequant_out,
                                    uint8_t* codes, int64_t ldq, void* stream);

/* --------------------------------------------------------- attention
 * FP8 flash-attention forward, FA-2 online softmax in fp32, both dot
 * products on gfx950 e4m3 MFMAs, P re-quantized as e4m3fn(p * 448).
 * Replaces the launch of _fp8_flash_attn_fwd_impl,
 * kernels/triton_kernels/fp8_flash_attn.py:251-391 (launch :604-644) plus the
 * fp32->input-dtype cast at :645 (written directly as bf16 or fp16 here,
 * one round to nearest even of the fp32 result, as that cast does).
 *   q8  : (B, H, Sq, D)  codes, contiguous
 *   k8  : (B, H, Skv, D) codes, contiguous
 *   vt8 : (B, H, D, ldv) codes, V transposed per head (RP_LAYOUT_BHDS),
 *         ldv % 128 == 0, ldv >= Skv, columns [Skv, ldv) zero
 *   q/k/v_scale : dequant scales, element bh*scale_stride for head bh = b*H+h
 *         (scale_stride 1: per (b, h); 0: per tensor)
 *   sm_scale : softmax temperature (the reference default is 1/sqrt(D)),
 *         finite and >= 0
 *   out : (B, H, Sq, D) logical, element (b,h,s,d) at
 *         out + b*osb + h*osh + s*oss + d (elements of out_dtype)
 *   D in {32, 64, 128, 256} (the reference's compiled set,
 *   fp8_flash_attn.py:516); mask per RP_MASK_*; Sq, Skv >= 1. */
int rp_fp8_attn_fwd(const uint8_t* q8, const uint8_t* k8, const uint8_t* vt8, int64_t ldv,
                    const float* q_scale, const float* k_scale, const float* v_scale,
                    int scale_stride, float sm_scale, void* out, int out_dtype,
                    int64_t osb, int64_t osh, int64_t oss,
                    int B, int H, int Sq, int Skv, int D,
                    int mask, int prefix_len, int suffix_len, void* stream);

/* Short-query variant of rp_fp8_attn_fwd: a workgroup of eight waves takes
 * block_m (32, 64 or 128) query rows of one head and gives each 32-row group
 * 256 / block_m waves, each a run of the key tiles
 * (rp_fp8_attn_wsplit_plan); the workgroup merges the runs of its rows in
 * LDS and writes the output (one launch, no workspace).  Where the 256-row
 * blocks of rp_fp8_attn_fwd leave most of the GPU idle (few heads, short
 * Sq: C1, the shared-prefix decode) it runs up to eight times the
 * workgroups over a fraction of the keys each.  Numerically it is the
 * one-range rp_fp8_attn_fwd, not a key split: a wave starts its running
 * max from the maxima of the tiles before its run (exchanged in LDS), so
 * every tile's P is quantized against the reference's running max
 * (fp8_flash_attn.py:334-380); the result differs from rp_fp8_attn_fwd only
 * by fp32 rounding.  The reference's autotune grid has BLOCK_M 64 and 128
 * too (fp8_flash_attn.py:177-186).  D in {64, 128} (RP_ERR_UNSUPPORTED
 * otherwise); other arguments as rp_fp8_attn_fwd. */
int rp_fp8_attn_fwd_wsplit(const uint8_t* q8, const uint8_t* k8, const uint8_t* vt8, int64_t ldv,
                           const float* q_scale, const float* k_scale, const float* v_scale,
                           int scale_stride, float sm_scale, void* out, int out_dtype,
                           int64_t osb, int64_t osh, int64_t oss,
                           int B, int H, int Sq, int Skv, int D,
                           int mask, int prefix_len, int suffix_len, int block_m, void* stream);

/* Key tiles per wave and waves with tiles per 32-row query group that
 * rp_fp8_attn_fwd_wsplit runs for Skv keys at block_m; exposed for tests.
 * RP_ERR_INVALID_ARGUMENT for Skv <= 0 or another block_m. */
int rp_fp8_attn_wsplit_plan(int Skv, int block_m, int* split_tiles, int* n_splits);

/* The launch plan rp_fp8_attn_fwd / rp_fp8_attn_fwd_split use for a shape:
 * the number of consecutive query blocks (256 rows each) one workgroup
 * runs.  Above 1, the kernel streams a workgroup's blocks through one tile
 * pipeline (short unmasked key ranges, head dim <= 128, one key split).
 * No counterpart in the reference (its Triton launch has one program per
 * query block); exposed for tests and profiling.  0 on invalid sizes. */
int rp_fp8_attn_blocks_per_workgroup(int B, int H, int Sq, int Skv, int D, int mask,
                                     int kv_splits);

/* Whether rp_fp8_attn_fwd (and the balanced entry, which then runs it)
 * runs a shape with the head's whole K and V^T resident in LDS: unmasked,
 * one key split, head dim 64 or 128, at most 512 (D = 128) or 1024 (D = 64)
 * keys, and a multi-block plan above 1.  A persistent grid, one workgroup
 * per CU, takes runs of 32-row query tasks; each wave computes a task's
 * whole attention against the resident tiles in the reference's tile order
 * (the same one-range result as the other launches, to fp32 rounding).
 * No counterpart in the reference; exposed for tests and profiling.  1 or
 * 0. */
int rp_fp8_attn_resident_kv(int B, int H, int Sq, int Skv, int D, int mask, int kv_splits);

/* rp_fp8_attn_fwd_balanced (kv_splits 0) or rp_fp8_attn_fwd_split
 * (kv_splits >= 1) with Q as its 16-bit input instead of codes: q is the
 * bf16 or fp16 (q_dtype RP_DTYPE_*) tensor (B, H, Sq, D) with element strides
 * qsb, qsh, qss (16-byte aligned, unit stride on D), q_scale its dequant
 * scale(s) as rp_fp8_scale_quantize_qkv computes them (there with q8 =
 * NULL), and each workgroup quantizes the Q rows it reads with the
 * quantizer's arithmetic -- the codes, and so the output, are those of the
 * separate quantizer and rp_fp8_attn_fwd*, bit for bit.  bf16 rows skip the
 * clamp to +-448, which Q's own scale never reaches (|x / scale| <= 426.67);
 * with a smaller scale, elements past 464 * scale become NaN codes.  No
 * counterpart in the reference, whose wrapper writes Q's codes and reads them back
 * (fp8_flash_attn.py:526-528, 604-644): this saves 3 of Q's 6 bytes per
 * element of HBM traffic.  Head dims 64, 128 and 256; the multi-block launch
 * of short key ranges that do not fit LDS takes codes only
 * (RP_ERR_UNSUPPORTED; rp_fp8_attn_q16_supported tells beforehand).
 * Workspace as the entry point kv_splits selects. */
int rp_fp8_attn_q16_supported(int B, int H, int Sq, int Skv, int D, int mask, int kv_splits,
                              void* stream);
int rp_fp8_attn_fwd_q16(const void* q, int q_dtype, int64_t qsb, int64_t qsh, int64_t qss,
                        const uint8_t* k8, const uint8_t* vt8, int64_t ldv,
                        const float* q_scale, const float* k_scale, const float* v_scale,
                        int scale_stride, float sm_scale, void* out, int out_dtype,
                        int64_t osb, int64_t osh, int64_t oss, int B, int H, int Sq, int Skv,
                        int D, int mask, int prefix_len, int suffix_len, int kv_splits,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Key-split variant of rp_fp8_attn_fwd: the key range is cut into
 * `kv_splits` contiguous parts of whole 128-key tiles (fewer when Skv has
 * fewer tiles), each run by its own workgroups with its own running max, and
 * a second kernel merges the parts.  It raises the parallelism of short or
 * few-head problems, which otherwise occupy a fraction of the GPU.  The
 * reference has no such entry point; it stands for the tile configuration its
 * wrapper resolves per shape (fp8_flash_attn.py:461-477, BLOCK_M/BLOCK_N),
 * and like BLOCK_N there it moves P's quantization grid within the FP8
 * tolerance.  kv_splits == 1 is rp_fp8_attn_fwd (workspace may be NULL).
 *   workspace : >= rp_fp8_attn_workspace_bytes(B, H, Sq, D, kv_splits)
 *               bytes of device memory, 256-byte aligned; not shared by calls
 *               that may overlap. */
size_t rp_fp8_attn_workspace_bytes(int B, int H, int Sq, int D, int kv_splits);
int rp_fp8_attn_fwd_split(const uint8_t* q8, const uint8_t* k8, const uint8_t* vt8, int64_t ldv,
                          const float* q_scale, const float* k_scale, const float* v_scale,
                          int scale_stride, float sm_scale, void* out, int out_dtype,
                          int64_t osb, int64_t osh, int64_t oss,
                          int B, int H, int Sq, int Skv, int D,
                          int mask, int prefix_len, int suffix_len, int kv_splits,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Balanced variant of rp_fp8_attn_fwd: the launch configuration the
 * wrapper resolves for grids of two or more rounds (the role of the
 * reference's per-shape config resolution, fp8_flash_attn.py:461-477, here
 * KV_SPLITS = 0).  A launch of one 256-query block per workgroup runs in
 * rounds of one workgroup per CU, so a last partial round costs about a
 * whole one.  For unmasked shapes whose blocks do not fill whole rounds, the
 * largest number of query blocks per head that does runs over the whole key
 * range, and the keys of the remaining blocks are split 2, 4 or 8 ways; both
 * kinds of workgroup run in one launch, and rp_fp8_attn_fwd_split's merge
 * follows.  The split items and the last unsplit items of every XCD's share
 * are handed out through a counter in the workspace (zeroed by the call's
 * own first kernel), so the XCDs that run faster take more of them; calls
 * that may overlap must not share a workspace.  E.g. (1, 40, 75600, 75600, 128) on
 * 256 CUs runs 288 blocks per head unsplit and the last 8 split 4 ways.  Rows
 * of the unsplit blocks are rp_fp8_attn_fwd's bit for bit; rows of the split
 * ones are what rp_fp8_attn_fwd_split computes for them.  Shapes with
 * nothing to split run rp_fp8_attn_fwd.  rp_fp8_attn_balanced_plan reports the
 * plan for `cus` CUs (main_blocks: query blocks per head run unsplit;
 * splits: key splits of the rest, 1 = a plain launch);
 * rp_fp8_attn_balanced_workspace_bytes the workspace for the CU count of the
 * stream's device (0: none needed). */
int rp_fp8_attn_balanced_plan(int B, int H, int Sq, int Skv, int D, int mask, int cus,
                              int* main_blocks, int* splits);
size_t rp_fp8_attn_balanced_workspace_bytes(int B, int H, int Sq, int Skv, int D, int mask,
                                            void* stream);
int rp_fp8_attn_fwd_balanced(const uint8_t* q8, const uint8_t* k8, const uint8_t* vt8,
                             int64_t ldv, const float* q_scale, const float* k_scale,
                             const float* v_scale, int scale_stride, float sm_scale, void* out,
                             int out_dtype, int64_t osb, int64_t osh, int64_t oss,
                             int B, int H, int Sq, int Skv, int D,
                             int mask, int prefix_len, int suffix_len,
                             void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------- fused QK-norm prologue
 * rp_fp8_scale_quantize of y instead of x, where per row of D elements
 *   n = RMSNorm(x) = bf16(x * (1 / sqrt(mean(x^2) + eps)))   fp32 math
 *   n = bf16(n * weight)                          when weight (bf16 [D]) != NULL
 *   y = bf16(n * cos + rot(n) * sin)              when rope_mode != RP_ROPE_NONE,
 *                                                 cos/sin fp32 [S, D] row s
 * computed inside both quantizer passes, so Q and K are read twice and
 * written once as codes -- the normalised tensor never reaches HBM.
 * Replaces the attention processors' norm_q/norm_k + apply_rotary_emb
 * ahead of the FP8 path (reference docs/walkthroughs/02-architecture.md:
 * 114-123), the rank-4 item of the path's next steps.  codes are BHSD
 * contiguous; D in {64, 128}; x, strides*2, weight, tables and codes
 * 16-byte aligned; the sum of squares runs in the order the header of
 * rp_prologue.hip states.  The workspace holds the amax pass's partial
 * maxima and each row's fp32 inverse norm, which the apply pass reads back
 * (4 bytes per row); it must not be shared by calls that may overlap. */
size_t rp_fp8_rmsnorm_quant_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D,
                                            int granularity);
int rp_fp8_rmsnorm_scale_quantize(const void* x, int64_t B, int64_t H, int64_t S, int64_t D,
                                  int64_t sb, int64_t sh, int64_t ss, const void* weight,
                                  float eps, const float* rope_cos, const float* rope_sin,
                                  int rope_mode, int granularity, float* dequant_out,
                                  uint8_t* codes, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* One attention call's three quantizers with the QK-norm prologue: Q and K
 * as rp_fp8_rmsnorm_scale_quantize (each with its own weight, NULL for
 * none, and its own cos/sin tables, Q's [Sq, D] and K's [Skv, D]; one
 * rope_mode for both), V as rp_fp8_scale_quantize into transposed codes
 * (RP_LAYOUT_BHDS, row stride ldv >= Skv, ldv % 128 == 0).  The same
 * scales and codes as those three calls, bit for bit, from three kernel
 * launches instead of nine.  Replaces, like the single-tensor call, the
 * processor's norm_q/norm_k ahead of the FP8 path (reference docs/
 * walkthroughs/02-architecture.md:114-123) together with the path's own
 * quantizer of V (kernels/triton_kernels/fp8_flash_attn.py:526-528).
 * bf16 inputs with a unit stride on D, D in {64, 128}; dequant_out holds
 * Q's, K's, then V's scales (ngroups each: B*H per head, 1 per tensor).
 * The workspace (256-byte aligned) must not be shared by calls that may
 * overlap. */
size_t rp_fp8_rmsnorm_quant_qkv_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Skv,
                                                int64_t D, int granularity);
int rp_fp8_rmsnorm_scale_quantize_qkv(const void* q, const void* k, const void* v, int64_t B,
                                      int64_t H, int64_t Sq, int64_t Skv, int64_t D, int64_t qsb,
                                      int64_t qsh, int64_t qss, int64_t ksb, int64_t ksh,
                                      int64_t kss, int64_t vsb, int64_t vsh, int64_t vss,
                                      const void* q_weight, const void* k_weight, float eps,
                                      const float* q_cos, const float* q_sin, const float* k_cos,
                                      const float* k_sin, int rope_mode, int granularity,
                                      float* dequant_out, uint8_t* q8, uint8_t* k8, uint8_t* vt8,
                                      int64_t ldv, void* workspace, size_t workspace_bytes,
                                      void* stream);

/* --------------------------------------------------------------- GEMM
 * C (M, N) bf16 = bf16( fp32(A8 . B8) * (a_scale * b_scale) ).
 * Replaces fp8_gemm_launch, kernels/hip/fp8_attn/fp8_gemm.hip:162-179
 * (kernel :79-156).  A8 (M, K) row-major, row stride lda; C row stride ldc.
 * B8 in either layout (b_layout):
 *   RP_B_KN  (K, N) row-major, row stride ldb >= N -- the reference's B
 *            (binding.cpp:25-57 passes B as (K, N) contiguous), staged into
 *            LDS as it lies and transposed by the LDS reads: no extra pass
 *   RP_B_NK  B transposed, (N, K) rows of stride ldb >= K: the nn.Linear
 *            weight layout
 * a_scale_dev / b_scale_dev: optional device pointers to the fp32 scales
 * (e.g. produced by rp_fp8_scale with RP_SCALE_PER_TENSOR); when non-NULL
 * they are used instead of the host values, avoiding a device->host read.
 * K, lda multiples of 16; N, ldc multiples of 4; a8 16-byte aligned, c
 * 8-byte aligned; RP_B_NK also needs ldb % 16 == 0 and b8 16-byte aligned.
 * Fastest path: K % 64 == 0 (and for RP_B_KN, N and ldb multiples of 16,
 * b8 16-byte aligned); other shapes run a general kernel. */
#define RP_B_NK 0
#define RP_B_KN 1
int rp_fp8_gemm(const uint8_t* a8, const uint8_t* b8, int b_layout, void* c,
                int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                float a_scale, float b_scale, const float* a_scale_dev,
                const float* b_scale_dev, void* stream);

/* rp_fp8_gemm with a bias: C = bf16(fp32(fp32(A8 . B8) * a_scale * b_scale)
 * + bias[n]), bias bf16 [N] (8-byte aligned), the product and the sum each
 * rounded to fp32 -- the epilogue of a bf16 nn.Linear.  A NULL bias makes
 * it rp_fp8_gemm.  No counterpart in the reference GEMM
 * (kernels/hip/fp8_attn/fp8_gemm.hip has no bias); it serves the FP8 linear
 * layers that replace nn.Linear in the module-swap pattern of
 * src/repercep/runtime/quantize.py:135-179. */
int rp_fp8_linear(const uint8_t* a8, const uint8_t* b8, int b_layout, const void* bias, void* c,
                  int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                  float a_scale, float b_scale, const float* a_scale_dev,
                  const float* b_scale_dev, void* stream);

/* rp_fp8_linear (bias may be NULL: rp_fp8_gemm) with the work balanced
 * across the GPU's XCDs, which run the same tiles at different speeds (at
 * C4 the mean 256 x 256 tile took 63-68 us depending on the XCD, so equal
 * static shares ended 0.25 ms apart).  Every XCD runs its share of tiles
 * but the last few in place; the tiles so left are handed out, in share
 * order, through a counter in `workspace` to whichever XCD asks first.  The
 * outputs equal rp_fp8_linear's bit for bit.  workspace: at least
 * RP_GEMM_BALANCED_WORKSPACE_BYTES, 256-byte aligned, zeroed by the call's
 * own first kernel, not shared by calls that may overlap.  No counterpart
 * in the reference (its GEMM launch takes no workspace); for callers that
 * can pass one, e.g. the FP8 linear layers. */
#define RP_GEMM_BALANCED_WORKSPACE_BYTES 256u
int rp_fp8_linear_balanced(const uint8_t* a8, const uint8_t* b8, int b_layout, const void* bias,
                           void* c, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                           int64_t ldc, float a_scale, float b_scale, const float* a_scale_dev,
                           const float* b_scale_dev, void* workspace, size_t workspace_bytes,
                           void* stream);

/* rp_fp8_gemm with row-wise scales, batched: for each batch z < `batch`,
 *   C_z (M, N) = bf16( fp32(fp32(A8_z . B8_z) * row_scale_z[m]) * col_scale_z[n] )
 * with A8_z = a8 + z*bsa, B8_z = b8 + z*bsb (bytes), C_z = c + z*bsc,
 * row_scale_z = row_scale + z*bs_row, col_scale_z = col_scale + z*bs_col
 * (elements).  Replaces the two torch._scaled_grouped_mm calls of the
 * reference's unfused FP8 attention (src/repercep/attention/
 * fp8_scaled_mm.py:149-157 and :172-178: scale_a per row of A, scale_b per
 * column of the product, a (BH, M, K) x (BH, N, K)^T batch).  Same size
 * rules as rp_fp8_gemm; col_scale_z 16-byte aligned; batch <= 65535; batch
 * strides of A and B multiples of 16, of C of 4. */
int rp_fp8_gemm_rowwise(const uint8_t* a8, const uint8_t* b8, int b_layout, void* c, int64_t M,
                        int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                        const float* row_scale, const float* col_scale, int64_t batch,
                        int64_t bsa, int64_t bsb, int64_t bsc, int64_t bs_row, int64_t bs_col,
                        void* stream);

/* FP8 byte transpose: dst (C, R) <- src (R, C); row strides lds, ldd.  No
 * counterpart in the reference; turns a (K, N) weight into the (N, K)
 * nn.Linear layout once, for layers stored that way. */
int rp_fp8_transpose(const uint8_t* src, uint8_t* dst, int64_t R, int64_t C,
                     int64_t lds, int64_t ldd, void* stream);

/* ---------------------------------------------------------- self-test
 * Device routines exposed so the tests can pin them exhaustively against
 * the CPU oracle.  They run the same device functions the kernels above use.
 * rp_selftest_e4m3: out[i] = e4m3fn code of clamp(x[i], -448, 448).
 * rp_selftest_scale: dequant[i] / qmul[i] from bf16 or fp16 (x_dtype) amax
 * bit patterns. */
int rp_selftest_e4m3(const float* x, uint8_t* out, int64_t n, void* stream);
int rp_selftest_scale(const uint16_t* amax_bits, int x_dtype, float* dequant, float* qmul, int64_t n,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* REPERCEP_FP8_H */
