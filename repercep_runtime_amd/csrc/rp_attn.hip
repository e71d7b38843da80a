// FP8 flash-attention forward for gfx950 (CDNA4).
//
// Semantics follow the reference kernel body
// kernels/triton_kernels/fp8_flash_attn.py:294-391 (OCP P cast as in
// fp8_flash_attn_hopper.py:322): FA-2 online softmax in fp32, both dot
// products on e4m3 operands, P re-quantized with the fixed scale 448, the
// row sum taken over the unquantized fp32 P, dequant factors folded into the
// softmax temperature and the final normalisation.
//
// Mapping onto CDNA4
// ------------------
// * Matrix core: v_mfma_f32_32x32x64_f8f6f4 (e4m3 x e4m3, fp32 acc).  For
//   one tile, lane l holds row/column l%32 of an operand and k-slots
//   [32*(l/32), +32) (32 bytes); the accumulator gives lane l column l%32 and
//   rows 8*(r/4) + 4*(l/32) + r%4 for its 16 registers r.
// * S^T = K . Q^T instead of S = Q . K^T: the accumulator then holds one
//   query per lane (column l%32) and keys down the rows -- exactly the
//   B-operand layout of the P.V product, so P never leaves registers.  The
//   K operand rows are gathered in a permuted order,
//       row rho of key tile h  <-  key 64(h/2) + 32((rho/4)%2) + 16(h%2)
//                                      + 4(rho/8) + rho%4,
//   so that, for key tiles 2m and 2m+1, lane group g holds keys
//   64m + 32g + [0, 32) in register order: the 32 bytes it feeds the
//   O^T += V^T . P^T MFMA over those 64 keys.
// * O^T = V^T . P^T: V^T is the A operand, read as 32 contiguous bytes per
//   lane from the per-head transposed V (layout RP_LAYOUT_BHDS written by
//   the quantizer).  The O^T accumulator again holds one query per lane, so
//   the online-softmax rescale (acc *= alpha) is lane-local.  One 32x32
//   operand feeds 32 queries, so each wave reads every K and V^T byte of a
//   tile from LDS once for its 32 query rows.
// * Row statistics: each lane keeps the running max and a partial row sum
//   for its query over its 64 keys of the tile; the two lanes sharing a
//   query (l, l^32) combine the max every tile and the sums once at the end.
// * Softmax in base 2: exp(x) = exp2(x*log2e); log2e and all dequant
//   factors are folded into one multiplier and log2(448) into the row
//   offset, so each score costs one FMA + one v_exp_f32 to become the
//   e4m3-ready value p*448.  The rescale of O is skipped for a tile when no
//   row of the wave raised its maximum (alpha == 1 exactly).
// * Workgroup of 8 waves x 32 query rows, two waves per SIMD (<= 256 VGPRs
//   each), in two groups of four that alternate between an MFMA phase and a
//   softmax phase at every workgroup barrier, so that on each SIMD one
//   wave's MFMAs overlap the other wave's softmax.  A single wave issues
//   VALU instructions at about one per 5 cycles (v_exp_f32 and
//   v_cvt_pk_fp8_f32 one per 9), so the softmax phase, not the matrix core,
//   sets the pace.  The MFMA phase therefore keeps its own VALU work small
//   and tucked between its MFMAs, runs at raised wave priority, and reads
//   its LDS operands two MFMAs ahead.
// * K tiles of 128 keys are double-buffered and V^T tiles triple-buffered
//   in LDS, loaded by the four waves of group 0 with global_load_lds_dwordx4
//   (no VGPR staging; SGPR tile base + fixed per-lane offsets); each LDS row
//   carries one 16-byte pad granule so every 16-lane ds_read_b128 group hits
//   16 distinct bank groups.
// * Grid: one workgroup per (head, query block), remapped so that the
//   workgroups resident on one XCD (dispatch is round-robin over the 8
//   XCDs) work on the same head and share its K/V through that XCD's L2.
//   The balanced launch (tail_plan) adds key-split workgroups for the query
//   blocks past the last whole round; they and the last unsplit items of
//   every XCD's share are pooled behind a counter, so faster XCDs take more
//   of them.  Short key ranges run several query blocks per workgroup
//   (multi_block_plan).

#include "rp_common.h"

#include <utility>

namespace rp {
namespace {

constexpr int kBlockN = 128;  // keys per tile = K depth of the P.V MFMA
constexpr int kBlockM = 32 * 8;  // query rows per workgroup
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLog2PMax = 8.807354922057604f;  // log2(448)

struct AttnArgs {
  const uint8_t* q;
  // Q as its bf16 or fp16 input (q_dt: kInBf16 / kInF16), (B, H, Sq, D) with
  // element strides qsb, qsh, qss, instead of codes in q: the kernel
  // quantizes its own Q rows with the quantizer's arithmetic (quant4, qm =
  // 1 / q scale), so the codes are the quantizer's.  Null when q holds codes.
  const uint16_t* q16;
  int64_t qsb, qsh, qss;
  int q_dt;
  const uint8_t* k;
  const uint8_t* vt;
  const float* qs;
  const float* ks;
  const float* vs;
  void* out;
  int64_t osb, osh, oss;
  int64_t ldv;
  float sm_scale;
  int scale_stride;
  int B, H, Sq, Skv;
  int mask, prefix, suffix;
  int D;          // head dim: row length of Q and K, rows of V^T per head
  int dv_halves;  // 2: each query block runs as two workgroups, one per half
                  // of V^T / O (head dim 256), both computing the same S
  // multi-block launches: each workgroup runs qb_per_wg consecutive query
  // blocks of one head (wg_per_bh workgroups per head)
  int qb_per_wg, wg_per_bh;
  int n_qblocks;
  int n_work;
  // key splits: split j covers keys [j*split_tiles*128, (j+1)*split_tiles*128)
  // and writes partial results (running max, row sum, unnormalised O) to
  // ws_ml / ws_acc, which attn_combine_kernel merges
  int kv_splits, split_tiles;
  float* ws_ml;   // [split][B*H][ws_rows] x {m, l}
  float* ws_acc;  // [split][B*H][ws_rows][D]
  // Key-split partial rows are indexed from the first row of query block
  // qb_begin, ws_rows rows per (split, head).  A mixed launch (the balanced
  // launch) runs query blocks [0, qb_begin) of every head over the whole key
  // range into the output (n_main workgroups, a multiple of 8) and blocks
  // [qb_begin, n_qblocks) key-split into the workspace.
  int qb_begin;
  int ws_rows;
  int n_main;
  // A mixed launch hands its key-split items out through this counter
  // (zeroed before the launch) to n_grid - n_main workgroups, more than the
  // n_work - n_main items: the XCDs that finish their unsplit share first
  // take more of them, and workgroups that find none left return at once.
  unsigned* item_counter;
  int n_grid;
  int pool_r;   // unsplit items per XCD share that go to the pool
};

// Output kinds of the attention kernel.
constexpr int kOutBf16 = 0, kOutF32 = 1, kOutSplit = 2, kOutF16 = 3;

__device__ __forceinline__ f32x16 mfma_32x32x64(const i32x8& a, const i32x8& b, const f32x16& c) {
  // cbsz = blgp = 0: both operands OCP e4m3; scale operands 0 select the
  // unscaled instruction.
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ i32x8 cat8(const i32x4& lo, const i32x4& hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// v_max3_f32 straight from asm: the builtin form makes the compiler quiet
// every MFMA result (v_max_f32 x, x, x) first, which doubles the VALU cost of
// the row max.  Scores are never signalling NaNs.
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Tile geometry for QK depth DK (the head dim) and PV width DV (the O^T rows
// one workgroup produces: DK, or half of it when a head of 256 is split over
// two workgroups).
template <int DK, int DV, int NW>
struct Geo {
  static constexpr int THREADS = NW * kWave;
  static constexpr int KSTEPS = DK >= 64 ? DK / 64 : 1;  // 64-deep MFMA steps over DK
  static constexpr int KROW = 64 * KSTEPS;               // K bytes per LDS row (>= DK)
  static constexpr int KVALID = DK / 16;                 // granules of a K row in HBM
  static constexpr int ETILES = DV / 32;                 // 32-row tiles of O^T
  // LDS pitches carry one 16-byte pad granule per row: the granule count per
  // row (5, 9 or 17) is odd, so 16 consecutive rows start in 16 distinct
  // 16-byte bank groups and every operand read is conflict-free without
  // swizzling.  With DK = 32 the upper half of each K row is padding too.
  static constexpr int K_PITCH = KROW + 16;
  static constexpr int V_PITCH = kBlockN + 16;
  static constexpr int K_GRAN = K_PITCH / 16;   // granules per K row
  static constexpr int V_GRAN = V_PITCH / 16;
  static constexpr int K_BYTES = kBlockN * K_PITCH;
  static constexpr int K_BLKS = kBlockN * K_GRAN / 64;   // wave instructions per K tile
  static constexpr int V_BLKS = (DV * V_GRAN + 63) / 64;
  static constexpr int V_BYTES = V_BLKS * 1024;          // DV rows, rounded up to a KiB
  static constexpr int K_STAGES = 2;               // ping-pong layout:
  static constexpr int V_STAGES = 3;               // V^T lives one step longer
  static constexpr int LDS_BYTES = K_STAGES * K_BYTES + V_STAGES * V_BYTES;
  static_assert(DK == 32 || DK == 64 || DK == 128 || DK == 256, "head dim");
  static_assert(DV % 32 == 0 && DV <= 128 && DV <= DK, "PV width");
  static_assert(K_BLKS * 64 == kBlockN * K_GRAN, "whole KiB K blocks");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS");
};

// Key (row inside the 128-key tile) that row rho of the S^T A operand of key
// tile h carries.
__device__ __forceinline__ int key_of(int h, int rho) {
  return 64 * (h >> 1) + 32 * ((rho >> 2) & 1) + 16 * (h & 1) + ((rho >> 3) << 2) + (rho & 3);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) void* gbl_ptr_t;

// 16 bytes global -> LDS without passing through VGPRs.  `lds_block` (an LDS
// byte address) must be wave-uniform: lane i lands at lds_block + 16*i.
//
// Written as inline asm on purpose.  The compiler books an LDS DMA as an
// outstanding LDS event that can complete out of order, and then guards
// every later ds_read with lgkmcnt(0) -- which serialises the operand reads
// of the MFMA phase.  Hidden from it, the loads are waited for by the
// explicit vmcnt(0) + workgroup barrier that precede every first read of a
// tile.  M0 carries the LDS destination; nothing else in this kernel uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void gload_lds16(const void* src, uint32_t lds_block) {
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_block);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(base)
               : "memory", "m0");
}
// The same load with a wave-uniform 64-bit base in SGPRs and a 32-bit
// per-lane offset ("saddr" form): no per-lane address arithmetic.
__device__ __forceinline__ void gload_lds16_s(const void* base, uint32_t voff, uint32_t lds_block) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_block);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(base), "s"(m0v)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Combine a lane's value with lane l^32's (the other half of the wave)
// through v_permlane32_swap -- a VALU op, no LDS round trip.
__device__ __forceinline__ float xhalf_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max3f(__uint_as_float(r[0]), __uint_as_float(r[1]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Direct-to-LDS loads of one (K, V^T) tile.  Each wave instruction fills one
// contiguous KiB (64 granules) of LDS; granule p of a block is row p / GRAN,
// slot p % GRAN.  K rows are stored in S^T A-operand order (LDS row 32h + rho
// holds key_of(h, rho)); V^T rows are d.  Pad slots re-load the row's first
// granule (valid memory; with DK = 32 the K pad slots are read, times the
// zero upper half of Q, so they must hold finite codes, which the row's own
// codes are).  V^T rows past DV in the last, rounded-up block re-load row
// DV-1 and are never read.  The tile's K_BLKS + V_BLKS blocks, K first, are
// dealt round-robin to the NL loading waves; a wave left one block short
// repeats its own previous block (same source, same destination).
template <int DK, int DV, int NL>
struct TileLoads {
  using G = Geo<DK, DV, 8>;
  static constexpr int T = G::K_BLKS + G::V_BLKS;
  static constexpr int N = (T + NL - 1) / NL;
  uint32_t off[N];  // K: key*D + granule; V^T: d*ldv + granule (bytes, per lane)
  int key[N];       // K: key inside the tile, for the tail clamp
  int blk[N];       // block index (wave-uniform)
};

template <int DK, int DV, int NL>
__device__ __forceinline__ TileLoads<DK, DV, NL> tile_loads(int64_t ldv, int wave, int lane) {
  using G = Geo<DK, DV, 8>;
  using TL = TileLoads<DK, DV, NL>;
  TL o;
#pragma unroll
  for (int n = 0; n < TL::N; ++n) {
    int b = n * NL + wave;
    if (b >= TL::T) b -= NL;
    o.blk[n] = b;
    if (b < G::K_BLKS) {
      const int p = b * kWave + lane;
      const int row = p / G::K_GRAN, slot = p % G::K_GRAN;
      const int key = key_of(row >> 5, row & 31);
      o.key[n] = key;
      o.off[n] = (uint32_t)(key * DK + (slot < G::KVALID ? slot : 0) * 16);
    } else {
      const int p = (b - G::K_BLKS) * kWave + lane;
      const int d = min(p / G::V_GRAN, DV - 1), slot = p % G::V_GRAN;
      o.key[n] = 0;
      o.off[n] = (uint32_t)(d * ldv + (slot < kBlockN / 16 ? slot : 0) * 16);
    }
  }
  return o;
}

// Where the loads of one tile go.  A tile holds keys [kbeg, kbeg + 128).
// The last tile, when Skv is not a multiple of 128, is shifted back to end
// at key Skv-1 (kbeg = Skv - 128; the keys it repeats from before its start
// are masked), so that every load stays inside K without per-lane clamps.
// Only a tile of a key range shorter than 128 (Skv < 128) cannot shift: its
// rows past Skv re-read key Skv-1 (CLAMP loads) and are masked.
struct TileDst {
  const uint8_t* kt;  // K rows of the tile in HBM
  const uint8_t* vt;  // V^T columns of the tile in HBM
  int klim;           // last valid key inside the tile, CLAMP loads only
  uint32_t kst, vst;  // LDS stages
};

// Issue load slot n of the tile.  Called with a constant n (unrolled
// loops), so whether the slot is a K or a V^T block folds at compile time,
// except for the one slot shared by both, where a wave-uniform select picks
// it: no branches.
template <int DK, int DV, int NL, bool CLAMP>
__device__ __forceinline__ void issue_slot(int n, const TileLoads<DK, DV, NL>& L,
                                           const TileDst& t) {
  using G = Geo<DK, DV, 8>;
  const bool any_k = n * NL < G::K_BLKS;
  const bool any_v =
      n * NL + NL - 1 >= G::K_BLKS || (n + 1) * NL > TileLoads<DK, DV, NL>::T;
  const int b = L.blk[n];
  const uint32_t kdst = t.kst + (uint32_t)b * 1024u;
  const uint32_t vdst = t.vst + (uint32_t)(b - G::K_BLKS) * 1024u;
  if constexpr (CLAMP) {
    const uint8_t* ksrc = t.kt + (L.off[n] - (uint32_t)(max(L.key[n] - t.klim, 0) * DK));
    const uint8_t* vsrc = t.vt + L.off[n];
    if (any_k && !any_v) {
      gload_lds16(ksrc, kdst);
    } else if (!any_k) {
      gload_lds16(vsrc, vdst);
    } else {
      const bool is_k = b < G::K_BLKS;
      gload_lds16(is_k ? ksrc : vsrc, is_k ? kdst : vdst);
    }
  } else {
    if (any_k && !any_v) {
      gload_lds16_s(t.kt, L.off[n], kdst);
    } else if (!any_k) {
      gload_lds16_s(t.vt, L.off[n], vdst);
    } else {
      const bool is_k = b < G::K_BLKS;
      gload_lds16_s(is_k ? t.kt : t.vt, L.off[n], is_k ? kdst : vdst);
    }
  }
}

__device__ __forceinline__ void wait_vmem_all() {
  // s_waitcnt vmcnt(0): direct-to-LDS loads have landed
  __builtin_amdgcn_s_waitcnt(0x0F70);
}
// s_waitcnt vmcnt(N): all but this wave's N most recent vector memory
// operations have completed
template <int N>
__device__ __forceinline__ void wait_vmem_n() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// One v_cvt_pk_bf16_f32 (round to nearest even): the pair as one vector
// conversion.  Converted one value at a time, the compiler emitted a
// conversion per value plus a shift and an or to pack them.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// 32 consecutive 16-bit Q elements (64 bytes at p, 16-byte aligned) in four
// loads, and their e4m3 codes (element 0 in the low byte, as the quantizer
// stores them)
struct QRaw32 {
  i32x4 w[4];
};
__device__ __forceinline__ QRaw32 qraw_load(const uint16_t* p) {
  const i32x4* s = reinterpret_cast<const i32x4*>(p);
  return QRaw32{{s[0], s[1], s[2], s[3]}};
}
//
// bf16 rows skip the quantizer's clamp to +-448.  The attention launches
// take Q's scale as the quantizer computed it from Q itself, bf16(max(amax,
// 1e-6) / 425.6), and for every finite bf16 amax fl(amax * qm) <= 426.67
// (the largest, at amax = 1.043e-6), so |x * qm| never reaches 448 and the
// clamp never binds: the codes are the quantizer's.  A NaN or infinite
// element makes the scale non-finite and every code of the group NaN or 0
// either way.  This saves two of the 4.5 instructions per element.  fp16
// scales can round to subnormals or 0 (977 fp16 amax values give
// |amax * qm| > 448), so fp16 rows keep the clamp.
__device__ __forceinline__ uint32_t quant4_bf16_own_scale(uint32_t lo_pair, uint32_t hi_pair,
                                                          float qm) {
  return pack4_e4m3(bf16_to_f32(lo_pair & 0xffffu) * qm, bf16_to_f32(lo_pair >> 16) * qm,
                    bf16_to_f32(hi_pair & 0xffffu) * qm, bf16_to_f32(hi_pair >> 16) * qm);
}
__device__ __forceinline__ i32x8 qraw_codes(const QRaw32& r, float qm, int dt) {
  i32x8 c;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t x = (uint32_t)r.w[m][0], y = (uint32_t)r.w[m][1];
    const uint32_t z = (uint32_t)r.w[m][2], t = (uint32_t)r.w[m][3];
    if (dt == kInF16) {
      c[2 * m] = (int)quant4<kInF16>(x, y, qm);
      c[2 * m + 1] = (int)quant4<kInF16>(z, t, qm);
    } else {
      c[2 * m] = (int)quant4_bf16_own_scale(x, y, qm);
      c[2 * m + 1] = (int)quant4_bf16_own_scale(z, t, qm);
    }
  }
  return c;
}

// Two LDS reads (32 bytes per lane) of one MFMA operand.
__device__ __forceinline__ i32x8 lds_op(uint32_t lds_addr) {
  typedef const i32x4 __attribute__((address_space(3)))* lds_i32x4_p;
  const lds_i32x4_p p = (lds_i32x4_p)(uintptr_t)lds_addr;
  const i32x4 lo = p[0], hi = p[1];
  return cat8(lo, hi);
}

// One MFMA phase: S^T = K(i) . Q^T, then O^T += V^T(i-1) . P^T(i-1), as one
// stream of MFMAs whose operands are read from LDS through a ring of kRing
// register sets, kRing-1 MFMAs ahead of their use.  Consecutive MFMAs write
// different accumulators, so none waits for its predecessor's result.
//
// Between the MFMAs the wave issues the phase's other work, which would
// otherwise wait for the stream to drain:
//   during S^T:  the loads of tile i+1 (LOADS) and O^T *= alpha(i-1), the
//                rescale owed since the previous phase's row max (skipped
//                when no row of the wave raised its max);
//   during PV:   partial row maxima of S^T(i) (MAX), 64 / NP scores per step.
constexpr int kRing = 3;

template <int DK, int DV, bool LOADS, bool MAX>
__device__ __forceinline__ void mfma_phase(uint32_t kl, uint32_t vl,
                                           const i32x8 (&qop)[Geo<DK, DV, 8>::KSTEPS],
                                           const i32x8 (&pop)[2], f32x16 (&s)[4],
                                           f32x16 (&acc)[DV / 32], float alpha_prev,
                                           float (&mh)[8], const TileLoads<DK, DV, 4>& L,
                                           const TileDst& dst) {
  using G = Geo<DK, DV, 8>;
  constexpr int NS = 4 * G::KSTEPS;   // S^T steps: ks outer, key tile hh inner
  constexpr int NP = 2 * G::ETILES;   // PV steps: k-half m outer, d tile e inner
  constexpr int N = NS + NP;
  constexpr int NLD = TileLoads<DK, DV, 4>::N;
  constexpr int MX = 64 / NP;              // scores per partial max
  auto addr = [&](int t) -> uint32_t {
    if (t < NS) {
      const int hh = t & 3, ks = t >> 2;
      return kl + 32 * hh * G::K_PITCH + 64 * ks;
    }
    const int u = t - NS, e = u % G::ETILES, m = u / G::ETILES;
    return vl + 32 * e * G::V_PITCH + 64 * m;
  };
  // O^T *= alpha(i-1), unless no lane of the wave raised its max (the vote
  // is one SGPR branch per S^T step): the multiplies are spread between the
  // S^T MFMAs, which do not read O^T, so they run in the MFMAs' shadow and
  // finish before the first P.V MFMA.  (Done up front, they delayed that
  // MFMA stream by their own issue time: 1.4% slower at the Wan shape.)
  constexpr int RPS = G::ETILES * 16 / NS;   // rescale multiplies per S^T step
  static_assert(RPS * NS == G::ETILES * 16, "rescale spread");
  const bool rescale = __any(alpha_prev != 1.0f);
  i32x8 ring[kRing];
#pragma unroll
  for (int t = 0; t < kRing - 1; ++t) ring[t] = lds_op(addr(t));
#pragma unroll
  for (int t = 0; t < N; ++t) {
    if (t + kRing - 1 < N) ring[(t + kRing - 1) % kRing] = lds_op(addr(t + kRing - 1));
    const i32x8 op = ring[t % kRing];
    if (t < NS) {
      const int hh = t & 3, ks = t >> 2;
      // the first k-step starts from the inline constant 0
      s[hh] = mfma_32x32x64(op, qop[ks], ks == 0 ? f32x16{} : s[hh]);
      if constexpr (LOADS) {
#pragma unroll
        for (int n = t * NLD / NS; n < (t + 1) * NLD / NS; ++n)
          issue_slot<DK, DV, 4, false>(n, L, dst);
      }
      if (rescale) {
#pragma unroll
        for (int v = t * RPS; v < (t + 1) * RPS; ++v) acc[v / 16][v % 16] *= alpha_prev;
      }
    } else {
      const int u = t - NS, e = u % G::ETILES, m = u / G::ETILES;
      acc[e] = mfma_32x32x64(op, pop[m], acc[e]);
      if constexpr (MAX) {
        const int f0 = u * MX;
        float x = max3f(s[f0 >> 4][f0 & 15], s[(f0 + 1) >> 4][(f0 + 1) & 15],
                        s[(f0 + 2) >> 4][(f0 + 2) & 15]);
#pragma unroll
        for (int j = 3; j + 1 < MX; j += 2)
          x = max3f(x, s[(f0 + j) >> 4][(f0 + j) & 15], s[(f0 + j + 1) >> 4][(f0 + j + 1) & 15]);
        if constexpr (MX % 2 == 0) x = max3f(x, s[(f0 + MX - 1) >> 4][(f0 + MX - 1) & 15], x);
        mh[u] = x;
      }
    }
    // Fence each step: the machine scheduler would otherwise sink the
    // operand reads next to their MFMAs and pull VALU work next to the
    // MFMA that produces its input, stalling the wave.
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Eight waves per workgroup in two groups of four; waves w and w+4 share a
// SIMD.  The groups run half a step out of phase ("ping-pong"), separated by
// workgroup barriers, so that on every SIMD one wave issues MFMAs while the
// other runs the softmax:
//
//   slot 2i   : group 0  MFMA(i)        group 1  SOFTMAX(i-1)
//   slot 2i+1 : group 0  SOFTMAX(i)     group 1  MFMA(i)
//
//   MFMA(i)    = O^T *= alpha(i-1), then S^T(i) = K(i) . Q^T and
//                O^T += V^T(i-1) . P^T(i-1), with the running max and
//                alpha(i) of tile i taken between and after those MFMAs
//   SOFTMAX(i) = P(i) = e4m3(p * 448) and the row sums
//
// One softmax wave keeps the SIMD's VALU nearly saturated, and the
// arbiter favours the older wave (group 0), so group 1's MFMA phase, whose
// few VALU instructions gate a whole stream of MFMAs, would wait behind
// group 0's softmax.  Group 1 therefore raises its priority for its MFMA
// phase (s_setprio); group 0's MFMA phase already wins by age.
//
// Numbering the workgroup barriers from the prologue's (0), group 0 runs
// MFMA(j) between barriers 2j and 2j+1 and group 1 between 2j+1 and 2j+2.
// Tile j (K(j), V^T(j)) overwrites K(j-2) and V^T(j-3), whose last reads end
// at barrier 2j-2, and is first read right after barrier 2j; so group 0's
// waves issue tile j after barrier 2j-2 and wait for it (s_waitcnt vmcnt(0))
// before barrier 2j.  Only group 0 loads: the slot in which a group issues
// loads costs its SIMD VALU time, and in this slot the MFMA group, not the
// softmax group, has VALU time to spare.
template <int DK, int DV, int OUT, bool WINDOW, bool MULTI, bool STAGE = false,
          bool MIXED = false>
__global__ __launch_bounds__(512, 1)
void attn_fwd_kernel(AttnArgs a) {
  constexpr int NW = 8;
  using G = Geo<DK, DV, NW>;
  constexpr int D = DK;
  static_assert(!MULTI || (OUT != kOutSplit && !WINDOW && DV == DK), "multi-block launches");
  static_assert(!STAGE || (MULTI && DK == 128 && (OUT == kOutBf16 || OUT == kOutF16)),
                "staged output stores");
  static_assert(!MIXED || (OUT != kOutSplit && !WINDOW && !MULTI), "mixed launches");
  constexpr int QROWS = 32;
  constexpr int BLOCK_M = QROWS * NW;
  // multi-block launches stage the next query block's Q in LDS: two buffers
  // of BLOCK_M rows (the block being switched to, and the one after)
  constexpr int Q_BYTES = MULTI ? BLOCK_M * DK : 0;
  constexpr int Q_LOADS = Q_BYTES / 1024 / 4;   // per loading wave
  // K and V^T stages.  (Three and four, loading each tile one step earlier,
  // measured 6% slower at the Wan shape: the tile loads' latency is hidden.)
  constexpr int KST = 2, VST = 3;
  constexpr int NLD = TileLoads<DK, DV, 4>::N;
  constexpr int LDS_TILES = KST * G::K_BYTES + VST * G::V_BYTES;
  static_assert(LDS_TILES + 2 * Q_BYTES <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[LDS_TILES + 2 * Q_BYTES];
  uint8_t* const kbuf = smem;                        // KST x K_BYTES
  uint8_t* const vbuf = smem + KST * G::K_BYTES;     // VST x V_BYTES
  // the same two regions as LDS byte addresses, for the direct-to-LDS loads
  const uint32_t kbuf_lds = (uint32_t)(uintptr_t)(lds_ptr_t)smem;
  const uint32_t vbuf_lds = kbuf_lds + KST * G::K_BYTES;
  const uint32_t qbuf_lds = kbuf_lds + LDS_TILES;   // multi-block launches only

  // ---- work item (XCD-aware remap of the linear workgroup id: XCD x runs
  // the x-th contiguous share of the items, k-th item at its k-th dispatch)
  const int w = blockIdx.x;
  const int xcd = w & 7, k_x = w >> 3;
  // a mixed launch's XCDs each run their share of the unsplit items first,
  // then their share of the key-split ones, which fill the launch's end
  const int pm = MIXED ? a.n_main >> 3 : 0;      // unsplit items per XCD
  const int ps = MIXED ? pm - a.pool_r : 0;       // of which taken in place
  bool part = OUT == kOutSplit;
  const int nw = MIXED ? a.n_work - a.n_main : a.n_work;   // split items
  const int per = nw >> 3, rem = nw & 7;
  int L2 = MIXED ? xcd * pm + k_x : xcd * per + min(xcd, rem) + k_x;
  if constexpr (MIXED) {
    if (k_x >= ps) {
      // the next pooled item, whichever XCD asks: first the last pool_r
      // unsplit items of every XCD's share, then the key-split items
      __shared__ int item;
      if (threadIdx.x == 0) item = (int)atomicAdd(a.item_counter, 1u);
      __syncthreads();
      const int it = item;
      if (it >= 8 * a.pool_r + nw) return;   // every item is taken
      part = it >= 8 * a.pool_r;
      // consecutive pooled items share K/V: the unsplit ones share by share
      // (one head's consecutive query blocks), the split ones by head and key
      // range.  (Interleaving the shares read 13.4 GB of HBM per C3 launch
      // against 8.8 GB this way, in the same time.)
      if (!part) {
        L2 = (it / a.pool_r) * pm + ps + it % a.pool_r;
      } else {
        const int r = it - 8 * a.pool_r;
        const int nq_s = a.n_qblocks - a.qb_begin;            // split blocks per head
        const int per_h = nq_s * a.kv_splits * (DV < DK ? 2 : 1);
        const int hh = r / per_h, rr = r - hh * per_h;
        const int hv = DV < DK ? rr & 1 : 0, r2 = DV < DK ? rr >> 1 : rr;
        const int sp = r2 / nq_s, ql = r2 - sp * nq_s;
        L2 = hh * per_h + ((ql * a.kv_splits + sp) << (DV < DK ? 1 : 0)) + hv;
      }
    }
  }
  // the two halves of a split query block are neighbours: same XCD, same
  // K tiles in its L2
  const int half = DV < DK ? L2 & 1 : 0;
  const int L = DV < DK ? L2 >> 1 : L2;
  const int dv_off = half * DV;  // first O column / V^T row of this workgroup
  // the items' query blocks [first_qb, first_qb + nqb) and key splits
  const int first_qb = MIXED && !part ? 0 : a.qb_begin;
  const int nqb = MIXED ? (part ? a.n_qblocks - a.qb_begin : a.qb_begin) : a.n_qblocks;
  const int nsplit = MIXED && !part ? 1 : a.kv_splits;
  const int per_bh = MULTI ? a.wg_per_bh : nqb * nsplit;
  const int bh = L / per_bh;
  const int qb = MULTI ? (L - bh * per_bh) * a.qb_per_wg
                       : (L - bh * per_bh) / nsplit + first_qb;
  const int split = MULTI ? 0 : L - bh * per_bh - (qb - first_qb) * nsplit;
  const int nblk = MULTI ? min(a.qb_per_wg, a.n_qblocks - qb) : 1;  // query blocks
  const int b = bh / a.H, h = bh - b * a.H;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int group = wave >> 2;
  const int lq = lane & 31;  // query column / operand row inside a 32x32 tile
  const int lg = lane >> 5;  // k-slot group (32 bytes)

  // this workgroup's current query block, this wave's and this lane's first
  // query in it (they advance at block boundaries of a multi-block launch)
  int q_block0 = qb * BLOCK_M;
  int q_wave0 = q_block0 + wave * QROWS;
  int q = q_wave0 + lq;

  const uint8_t* qh = a.q + (int64_t)bh * a.Sq * D;
  const uint8_t* kh = a.k + (int64_t)bh * a.Skv * D;
  const uint8_t* vh = a.vt + ((int64_t)bh * D + dv_off) * a.ldv;

  const float q_scale = a.qs[bh * a.scale_stride];
  const float k_scale = a.ks[bh * a.scale_stride];
  const float v_scale = a.vs[bh * a.scale_stride];
  // exp2 domain: s2 = dot * c2 with c2 = sm_scale*q_scale*k_scale*log2(e).
  // A zero product (sm_scale = 0) becomes the smallest normal float: the
  // reference scales the scores before masking them (fp8_flash_attn.py:
  // 341-356), so every visible score is 0 and every masked one -inf, while
  // here the masked raw score -inf times 0 would be NaN.  With c2 = FLT_MIN a
  // visible score lands within 1e-30 of 0, which exp2 and the running max
  // cannot tell from 0 (p = 448, alpha = 1 exactly), and -inf stays -inf.
  const float c2_raw = ((a.sm_scale * q_scale) * k_scale) * kLog2e;
  const float c2 = c2_raw == 0.0f ? 1.17549435e-38f : c2_raw;

  // ---- key range [kv_begin, kv_end): this workgroup's split; causal blocks
  // past the block's last query are skipped
  const int kv_begin = split * a.split_tiles * kBlockN;
  const int kv_end = MIXED && !part ? a.Skv : min(a.Skv, kv_begin + a.split_tiles * kBlockN);
  int n_kb = (kv_end - kv_begin + kBlockN - 1) / kBlockN;
  if (a.mask == RP_MASK_CAUSAL) {
    const int q_last = min(q_block0 + BLOCK_M, a.Sq) - 1;
    n_kb = q_last < kv_begin ? 0 : min(n_kb, (q_last - kv_begin) / kBlockN + 1);
  }
  if constexpr (OUT == kOutSplit) {
    if (n_kb == 0) {  // a causal split wholly past this block's queries
      const int q0 = q_block0 + tid;
      if (tid < BLOCK_M && q0 < a.Sq) {
        const int64_t row =
            ((int64_t)split * a.B * a.H + bh) * a.ws_rows + (q0 - a.qb_begin * BLOCK_M);
        if (half == 0) {
          a.ws_ml[2 * row] = -__builtin_inff();
          a.ws_ml[2 * row + 1] = 0.0f;
        }
        for (int d = 0; d < DV; d += 4)
          *reinterpret_cast<float4*>(a.ws_acc + row * D + dv_off + d) =
              make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
      return;
    }
  }

  // Group 0's four waves issue every tile (see the schedule below); their
  // per-lane load offsets are fixed for the whole kernel.
  const TileLoads<DK, DV, 4> tl = tile_loads<DK, DV, 4>(a.ldv, wave & 3, lane);
  // first key of tile j of the range (see TileDst)
  auto tile_begin = [&](int j) {
    const int kv0 = kv_begin + j * kBlockN;
    return (kv0 + kBlockN > a.Skv && a.Skv >= kBlockN) ? a.Skv - kBlockN : kv0;
  };
  // loads of tile `src` into the LDS stages of tile `stage`
  auto tile_dst = [&](int src, int stage) {
    TileDst t;
    const int kbeg = tile_begin(src);
    t.kt = kh + (int64_t)kbeg * D;
    t.vt = vh + kbeg;
    t.klim = a.Skv - 1 - kbeg;
    t.kst = kbuf_lds + (stage % KST) * G::K_BYTES;
    t.vst = vbuf_lds + (stage % VST) * G::V_BYTES;
    return t;
  };
  if (group == 0) {
    const TileDst t0 = tile_dst(0, 0);
#pragma unroll
    for (int n = 0; n < NLD; ++n) issue_slot<DK, DV, 4, true>(n, tl, t0);
  }
  // V^T stage VST-1 is read (times P = 0) by the first MFMA phase before
  // tile VST-1 lands there: clear it so that no stale NaN code can reach the
  // accumulator.
  for (int o = tid * 16; o < G::V_BYTES; o += G::THREADS * 16)
    *reinterpret_cast<i32x4*>(vbuf + (VST - 1) * G::V_BYTES + o) = i32x4{0, 0, 0, 0};

  // ---- Q^T operand (B operand of S^T), resident for the whole kernel
  auto load_q = [&](i32x8 (&dst)[G::KSTEPS], int qrow) {
    if constexpr (!MULTI && DK >= 64) {
      if (a.q16 != nullptr) {
        // Q from its 16-bit input: this lane's 32-element runs 32 lg + 64 ks
        // of row qrow, quantized here
        const uint16_t* src = a.q16 + (int64_t)b * a.qsb + (int64_t)h * a.qsh +
                              (int64_t)min(qrow, a.Sq - 1) * a.qss + 32 * lg;
        const float qm = 1.0f / q_scale;
        QRaw32 raw[G::KSTEPS];
#pragma unroll
        for (int ks = 0; ks < G::KSTEPS; ++ks) raw[ks] = qraw_load(src + 64 * ks);
#pragma unroll
        for (int ks = 0; ks < G::KSTEPS; ++ks) dst[ks] = qraw_codes(raw[ks], qm, a.q_dt);
        return;
      }
    }
    if constexpr (DK < 64) {
      // one 64-deep step over a 32-byte row: k-slot group 1 is zero padding
      const i32x4* src = reinterpret_cast<const i32x4*>(qh + (int64_t)min(qrow, a.Sq - 1) * D);
      dst[0] = lg == 0 ? cat8(src[0], src[1]) : i32x8{};
    } else {
      const i32x4* src =
          reinterpret_cast<const i32x4*>(qh + (int64_t)min(qrow, a.Sq - 1) * D + 32 * lg);
#pragma unroll
      for (int ks = 0; ks < G::KSTEPS; ++ks) dst[ks] = cat8(src[4 * ks], src[4 * ks + 1]);
    }
  };
  i32x8 qop[G::KSTEPS];
  load_q(qop, q);
  // Multi-block launches: the loading waves fetch block k+1's Q into LDS
  // buffer (k+1) % 2 while block k runs (direct-to-LDS, like the tiles; one
  // KiB of rows per instruction, rows past Sq re-read row Sq-1), and every
  // wave reads its Q^T operand from there at the switch.
  auto issue_q = [&](int blk_next) __attribute__((always_inline)) {
    const int row0 = (qb + blk_next) * BLOCK_M;   // < Sq: blk_next < nblk
    const uint8_t* base = qh + (int64_t)row0 * D;
    const uint32_t dst = qbuf_lds + (uint32_t)((blk_next & 1) * Q_BYTES);
#pragma unroll
    for (int n = 0; n < Q_LOADS; ++n) {
      const int p = ((n * 4 + (wave & 3)) * 1024 + 16 * lane);   // byte in the buffer
      const int row = min(row0 + p / D, a.Sq - 1) - row0;
      gload_lds16_s(base, (uint32_t)(row * D + p % D), dst + (uint32_t)((n * 4 + (wave & 3)) * 1024));
    }
  };
  auto read_q = [&](int blk) __attribute__((always_inline)) {
    const uint32_t src = qbuf_lds + (uint32_t)((blk & 1) * Q_BYTES) + (uint32_t)((wave * QROWS + lq) * D);
    if constexpr (DK < 64) {
      qop[0] = lg == 0 ? lds_op(src) : i32x8{};
    } else {
#pragma unroll
      for (int ks = 0; ks < G::KSTEPS; ++ks) qop[ks] = lds_op(src + 32 * lg + 64 * ks);
    }
  };

  // per-lane LDS byte offsets of the operand reads (inside one stage): row
  // lq of each 32-row operand block, k-slot group lg; the rest is immediate
  const int k_base = lq * G::K_PITCH + 32 * lg;
  const int v_base = lq * G::V_PITCH + 32 * lg;

  f32x16 acc[G::ETILES];
#pragma unroll
  for (int e = 0; e < G::ETILES; ++e) acc[e] = f32x16{};
  float m_run = -__builtin_inff(), l_run = 0.0f;
  f32x16 s[4];
  i32x8 pop[2] = {i32x8{}, i32x8{}};

  wait_vmem_all();
  __syncthreads();
  if (group == 1) __syncthreads();  // group 1 starts half a step behind

  // out = acc * v_scale / l for query row qrow (acc carries P*448, l sums
  // P*448); every lane takes part (the row sum combines lane pairs).
  // STAGE (multi-block launches, D = 128, 16-bit output, two or more key
  // tiles per block): the rows go out through Q buffer sbuf, whose
  // block has been read by every wave and which no load refills before the
  // next block switch.  Each wave stages its 32 rows in a 4 KiB share, 64
  // columns at a time: row r (128 bytes) at 128 r, 16-byte chunk c at
  // granule c ^ ((r >> 1) & 7) -- the 16 lanes of a write group cover the 16
  // bank groups -- then reads them back eight lanes to a row, so every
  // store instruction writes whole 128-byte lines (the unstaged stores write
  // 32-byte pieces, which the L2 has to merge).
  auto store_out = [&](int qrow, float l_lane, int sbuf) __attribute__((always_inline)) {
    const float l = xhalf_sum(l_lane);
    const float inv = v_scale / l;
    uint2 pend = make_uint2(0u, 0u);
    if (STAGE || qrow < a.Sq) {
      const int64_t obase =
          (int64_t)b * a.osb + (int64_t)h * a.osh + (int64_t)qrow * a.oss + dv_off;
      // the wave's first row of the block, and its staging share.  The
      // staging addresses derive from `ln`, opaque to the compiler here, so
      // that they are computed at the store and not hoisted out of the tile
      // loop (where they would hold registers through every phase).
      const int row0 = __builtin_amdgcn_readfirstlane(qrow - lq);
      int ln = lane;
      asm volatile("" : "+v"(ln));
      uint8_t* const st = smem + LDS_TILES + sbuf * Q_BYTES + wave * 4096;
#pragma unroll
      for (int e = 0; e < G::ETILES; ++e) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 32 * e + 8 * i + 4 * lg;
          const float o0 = acc[e][4 * i + 0] * inv, o1 = acc[e][4 * i + 1] * inv;
          const float o2 = acc[e][4 * i + 2] * inv, o3 = acc[e][4 * i + 3] * inv;
          if constexpr (OUT == kOutF32) {
            *reinterpret_cast<float4*>(static_cast<float*>(a.out) + obase + d) =
                make_float4(o0, o1, o2, o3);
          } else {
            uint2 pk;
            if constexpr (OUT == kOutF16) {
              pk.x = pack_f16x2(o0, o1);
              pk.y = pack_f16x2(o2, o3);
            } else {
              pk.x = pack_bf16x2(o0, o1);
              pk.y = pack_bf16x2(o2, o3);
            }
            // Chunk c = 4e + i (columns 8c .. 8c+7) of this row is split
            // over the lane pair (l, l+32): columns 8c..8c+3 here when
            // lg = 0, 8c+4..8c+7 when lg = 1.  For the chunk pair (c, c+1),
            // i even, swapping chunk c+1's low half of the lower lane with
            // chunk c's high half of the upper lane leaves lane lg = 0 with
            // all of chunk c and lane lg = 1 with all of chunk c+1: one
            // 16-byte store each, the pair writing 32 contiguous bytes.
            if (i % 2 == 0) {
              pend = pk;
            } else {
              // pend: chunk c (= 4e + i - 1) part, pk: chunk c+1 part
              const auto x = __builtin_amdgcn_permlane32_swap(pend.x, pk.x, false, false);
              const auto y = __builtin_amdgcn_permlane32_swap(pend.y, pk.y, false, false);
              const uint4 v = make_uint4(x[0], y[0], x[1], y[1]);
              const int c = 4 * e + i - 1 + lg;   // the chunk this lane now holds
              if constexpr (STAGE) {
                const int cl = c & 7;               // chunk within the 64 staged columns
                const int lr = ln & 31;             // = lq, the row this lane holds
                *reinterpret_cast<uint4*>(st + lr * 128 + ((cl ^ ((lr >> 1) & 7)) << 4)) = v;
              } else {
                *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.out) + obase + 8 * c) = v;
              }
            }
          }
        }
        if constexpr (STAGE) {
          if ((e & 1) == 1) {
            // 64 columns (chunks 8(e/2) .. +7) of the wave's 32 rows staged
            __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the writes are done
            __builtin_amdgcn_wave_barrier();
            const int cl = ln & 7;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const int r = 8 * k + (ln >> 3);
              const uint4 v =
                  *reinterpret_cast<const uint4*>(st + r * 128 + ((cl ^ ((r >> 1) & 7)) << 4));
              const int qr = row0 + r;
              if (qr < a.Sq) {
                const int64_t ob = (int64_t)b * a.osb + (int64_t)h * a.osh +
                                   (int64_t)qr * a.oss + dv_off + 8 * (8 * (e >> 1) + cl);
                *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.out) + ob) = v;
              }
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);   // the reads are done before the next writes
            __builtin_amdgcn_wave_barrier();
          }
        }
      }
    }
  };

  // Tiles of the workgroup, in stream order: n_kb per query block.  A
  // multi-block launch runs its blocks as one stream: at the first tile of a
  // block the wave switches to that block's Q^T (loaded one block ahead) and
  // restarts the running max at -inf, so alpha of that tile is exp2(-inf) = 0
  // and clears O^T and l; the finished block's output is stored first, at
  // the start of the following softmax phase, when its last PV is done.
  const int T = MULTI ? nblk * n_kb : n_kb;
  float l_done = 0.0f;   // multi-block: row sum of the block awaiting its store

  // The two groups run separate copies of the loop, so that each MFMA phase
  // is one branch-free block: group 0 issues the tile loads, group 1 none.
  auto run = [&](auto loads_c) {
    constexpr bool LOADS = decltype(loads_c)::value;
    // alpha: rescale of tile i's row statistics, applied to l in SOFTMAX(i)
    // and to O^T in MFMA(i+1), before PV(i) accumulates
    float alpha = 1.0f, moff = 0.0f;
    for (int i = 0; i <= T; ++i) {
      // ================= MFMA(i) =================
      const int j = MULTI ? i % n_kb : i;  // tile of the current query block
      const int blk = MULTI ? i / n_kb : 0;  // query block of the workgroup
      if constexpr (MULTI) {
        // the loading group stores the finished block here, ahead of this
        // phase's tile loads (its counted waits then never cover stores)
        if (LOADS && i >= 2 && (i - 1) % n_kb == 0 && i - 1 < T)
          store_out(q - BLOCK_M, l_done, blk & 1);
        if (j == 0 && i > 0 && i < T) {
          read_q(blk);
          m_run = -__builtin_inff();
          q_block0 += BLOCK_M;
          q_wave0 += BLOCK_M;
          q += BLOCK_M;
        }
      }
      if (!LOADS) __builtin_amdgcn_s_setprio(1);  // the MFMA phase issues first on its SIMD
      // Tile j is issued by group 0 during MFMA(j-1), after workgroup barrier
      // 2j-2, and waited for at the end of SOFTMAX(j-1), before barrier 2j
      // (the prologue's barrier is number 0).  Every MFMA phase runs both
      // products: in the first one P is zero and V^T stage 2 holds zeros
      // (cleared in the prologue), in the last one the S^T result is unused.
      const int kv0 = kv_begin + j * kBlockN;
      const bool tail = kv0 + kBlockN > a.Skv;
      // operand base addresses of this phase's K and V^T stages; opaque to
      // the compiler, so every read is one register plus an immediate
      uint32_t kl = kbuf_lds + (i % KST) * G::K_BYTES + k_base;
      uint32_t vl = vbuf_lds + ((i + VST - 1) % VST) * G::V_BYTES + v_base;
      asm("" : "+v"(kl), "+v"(vl));
      // group 0 issues tile i+1; past the last tile it re-reads the last one
      // into the stages tile i+1 would use, which are free (see above)
      const TileDst nxt = tile_dst(min(i + 1, T - 1) % n_kb, i + 1);
      // Without a window mask the row max is taken between the PV MFMAs, over
      // the raw scores: rows past Skv duplicate key Skv-1, and the keys a
      // shifted last tile repeats were in the tile before, so the raw max is
      // the max over the tile's visible keys.  It is not when a shifted tile
      // opens a key split (its repeats belong to the previous split), nor
      // under a window mask: such a tile takes its max after the phase, from
      // the masked scores.
      float mh[8];
      mfma_phase<DK, DV, LOADS, !WINDOW>(kl, vl, qop, pop, s, acc, alpha, mh, tl, nxt);
      // the next block's Q, after the tile loads (so a counted wait can leave
      // it in flight)
      const bool q_issued = MULTI && LOADS && j == 0 && blk + 1 < nblk;
      if constexpr (MULTI && LOADS) {
        if (q_issued) issue_q(blk + 1);
      }
      if (i < T) {
        bool masked = tail;
        if (a.mask == RP_MASK_CAUSAL) masked |= kv0 + kBlockN - 1 > q_wave0;
        if (a.mask == RP_MASK_SHARED_PREFIX) masked |= kv0 + kBlockN > a.prefix;
        if (masked) {
          // every supported mask is "kv < pre_end, or lo <= kv <= hi" with a
          // per-query window; bitwise predicates, one select per score
          const float ninf = -__builtin_inff();
          int lo = 0, hi = a.Skv - 1;
          if (a.mask == RP_MASK_CAUSAL) hi = min(q, hi);
          if (a.mask == RP_MASK_SHARED_PREFIX) {
            lo = a.prefix + q - q % a.suffix;
            hi = min(a.prefix + q, hi);
          }
          const int pre_end = a.mask == RP_MASK_SHARED_PREFIX ? min(a.prefix, a.Skv) : 0;
          // keys before kv0 are the shifted last tile's repeats
          const int kvl = tile_begin(j) + 32 * lg;
          const int lo_t = lo - kvl, hi_t = hi - kvl, pe_t = pre_end - kvl, new_t = kv0 - kvl;
  #pragma unroll
          for (int hh = 0; hh < 4; ++hh)
  #pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int o = 64 * (hh >> 1) + 16 * (hh & 1) + r;  // key - kvl
              const int vis = (o >= new_t) & (((o >= lo_t) & (o <= hi_t)) | (o < pe_t));
              s[hh][r] = vis ? s[hh][r] : ninf;
            }
        }
        float mx;
        if (!WINDOW && !(j == 0 && tile_begin(0) != kv0)) {
          constexpr int NP = 2 * G::ETILES;   // partial maxima mh[0 .. NP)
          if constexpr (NP == 2) {
            mx = max3f(mh[0], mh[1], mh[1]);
          } else {
            mx = max3f(mh[0], mh[1], mh[2]);
  #pragma unroll
            for (int j = 3; j + 1 < NP; j += 2) mx = max3f(mx, mh[j], mh[j + 1]);
            if constexpr (NP % 2 == 0) mx = max3f(mx, mh[NP - 1], mh[NP - 1]);
          }
        } else {
          float mt[4];
  #pragma unroll
          for (int hh = 0; hh < 4; ++hh) {
            float x = max3f(s[hh][0], s[hh][1], s[hh][2]);
  #pragma unroll
            for (int r = 3; r < 15; r += 2) x = max3f(x, s[hh][r], s[hh][r + 1]);
            mt[hh] = max3f(x, s[hh][15], s[hh][15]);
          }
          mx = max3f(mt[0], mt[1], max3f(mt[2], mt[3], mt[3]));
        }
        mx = xhalf_max(mx);
        const float m_new = max3f(m_run, mx * c2, mx * c2);
        const float m_use = (m_new == -__builtin_inff()) ? 0.0f : m_new;
        alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        m_run = m_new;
        moff = m_use - kLog2PMax;
      }
      if (!LOADS) __builtin_amdgcn_s_setprio(0);
      __syncthreads();

      // ================= SOFTMAX(i) =================
      if constexpr (MULTI) {
        if (j == 0 && i > 0 && i < T) {
          l_done = l_run;   // the finished block's row sum, before this tile's update
          if (!LOADS) store_out(q - BLOCK_M, l_done, blk & 1);
        }
      }
      if (i < T) {
        float ps[4] = {-0.0f, -0.0f, -0.0f, -0.0f};  // x + -0 == x: no first add
  #pragma unroll
        for (int m = 0; m < 2; ++m) {
          int pw[8];
  #pragma unroll
          for (int wd = 0; wd < 8; ++wd) {
            const int hh = 2 * m + (wd >> 2);
            const int r = 4 * (wd & 3);
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hh][r + 0], c2, -moff));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hh][r + 1], c2, -moff));
            const float p2 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hh][r + 2], c2, -moff));
            const float p3 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hh][r + 3], c2, -moff));
            ps[wd & 3] += (p0 + p1) + (p2 + p3);
            pw[wd] = (int)pack4_e4m3(p0, p1, p2, p3);
          }
          pop[m] = i32x8{pw[0], pw[1], pw[2], pw[3], pw[4], pw[5], pw[6], pw[7]};
        }
        l_run = l_run * alpha + ((ps[0] + ps[1]) + (ps[2] + ps[3]));
      }
      if constexpr (LOADS) {
        // tile i+1 must have landed; Q loads issued in this phase may stay
        // in flight unless the next tile opens the block that reads them
        if (MULTI && q_issued && j + 1 < n_kb) wait_vmem_n<Q_LOADS>();
        else wait_vmem_all();
      }
      __syncthreads();
    }
  };
  if (group == 0) {
    run(std::true_type{});
    __syncthreads();  // balance group 1's extra opening barrier
  } else {
    run(std::false_type{});
  }

  // ---- epilogue: the (last) query block's output, or a split's partials
  if constexpr (OUT == kOutSplit || MIXED) {
    if (part) {
      const float l = xhalf_sum(l_run);
      // partial result of this key split, relative to its own running max
      if (q < a.Sq) {
        const int64_t row =
            ((int64_t)split * a.B * a.H + bh) * a.ws_rows + (q - a.qb_begin * BLOCK_M);
        float* dst = a.ws_acc + row * D + dv_off;
#pragma unroll
        for (int e = 0; e < G::ETILES; ++e)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            *reinterpret_cast<float4*>(dst + 32 * e + 8 * i + 4 * lg) =
                make_float4(acc[e][4 * i], acc[e][4 * i + 1], acc[e][4 * i + 2], acc[e][4 * i + 3]);
        if (lg == 0 && half == 0)
          *reinterpret_cast<float2*>(a.ws_ml + 2 * row) = make_float2(m_run, l);
      }
      return;
    }
  }
  if constexpr (OUT != kOutSplit) store_out(q, l_run, (nblk - 1) & 1);
}

// Merge the key splits of one query row: with m_j, l_j, O_j the running
// max, row sum and unnormalised output of split j (O_j and l_j relative to
// m_j, in the exp2 domain), out = sum_j w_j O_j * v_scale / sum_j w_j l_j,
// w_j = exp2(m_j - max_j m_j).  Splits that saw no visible key (l_j = 0)
// are left out.  One thread per four head-dim elements of a row.  OUT is
// kOutBf16, kOutF32 or kOutF16.
template <int D, int OUT>
__global__ __launch_bounds__(256)
void attn_combine_kernel(AttnArgs a) {
  constexpr int CH = D / 4;
  const int64_t rows = (int64_t)a.B * a.H * a.ws_rows;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = t / CH;
  if (row >= rows) return;
  const int d = (int)(t - row * CH) * 4;
  const float2* ml = reinterpret_cast<const float2*>(a.ws_ml);
  float mmax = -__builtin_inff();
#pragma unroll 8
  for (int j = 0; j < a.kv_splits; ++j) {
    const float2 v = ml[row + j * rows];
    if (v.y != 0.0f) mmax = fmaxf(mmax, v.x);
  }
  float l = 0.0f;
  float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 8
  for (int j = 0; j < a.kv_splits; ++j) {
    const float2 v = ml[row + j * rows];
    const float4 x = *reinterpret_cast<const float4*>(a.ws_acc + (row + j * rows) * D + d);
    // a split that saw no key of this row has l = 0 and O = 0: weight 0
    const float w = v.y != 0.0f ? __builtin_amdgcn_exp2f(v.x - mmax) : 0.0f;
    l += w * v.y;
    o.x += w * x.x; o.y += w * x.y; o.z += w * x.z; o.w += w * x.w;
  }
  const int bh = (int)(row / a.ws_rows);
  const int q = (int)(row - (int64_t)bh * a.ws_rows) + a.qb_begin * kBlockM;
  const int b = bh / a.H, h = bh - b * a.H;
  const float inv = a.vs[bh * a.scale_stride] / l;
  const int64_t obase = (int64_t)b * a.osb + (int64_t)h * a.osh + (int64_t)q * a.oss + d;
  if constexpr (OUT == kOutF32) {
    *reinterpret_cast<float4*>(static_cast<float*>(a.out) + obase) =
        make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
  } else {
    uint2 pk;
    if constexpr (OUT == kOutF16) {
      pk.x = pack_f16x2(o.x * inv, o.y * inv);
      pk.y = pack_f16x2(o.z * inv, o.w * inv);
    } else {
      pk.x = pack_bf16x2(o.x * inv, o.y * inv);
      pk.y = pack_bf16x2(o.z * inv, o.w * inv);
    }
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + obase) = pk;
  }
}

// O^T rows one workgroup produces for head dim D
template <int D>
constexpr int kPVWidth = D > 128 ? 128 : D;

template <int D, int OUT>
void launch_fwd(const AttnArgs& a, hipStream_t st) {
  constexpr int DV = kPVWidth<D>;
  const dim3 grid(a.n_work), block(512);
  if constexpr (OUT != kOutSplit && DV == D) {
    if (a.qb_per_wg > 1) {
      // staged output stores need a block's Q buffer idle from its switch
      // to the next one: two or more key tiles per block
      if constexpr (D == 128 && OUT != kOutF32) {
        if (a.Skv > kBlockN) {
          hipLaunchKernelGGL((attn_fwd_kernel<D, DV, OUT, false, true, true>), grid, block, 0, st, a);
          return;
        }
      }
      hipLaunchKernelGGL((attn_fwd_kernel<D, DV, OUT, false, true>), grid, block, 0, st, a);
      return;
    }
  }
  if (a.mask != RP_MASK_NONE)
    hipLaunchKernelGGL((attn_fwd_kernel<D, DV, OUT, true, false>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<D, DV, OUT, false, false>), grid, block, 0, st, a);
}

// The balanced launch: the unsplit query blocks into the output, the rest
// key-split into the workspace (attn_combine_kernel merges them after).
// The XCDs of one GPU run the same workgroups at different speeds (measured
// at C3, per-XCD mean time of an unsplit workgroup: 1.12 to 1.19 ms, the
// same XCDs slow on every launch of a box), so equal static shares end
// up to 3 ms apart.  A mixed launch therefore pools the key-split items and
// the last kPoolPerXcd unsplit items of every XCD's share behind one
// counter: C3 balanced 54.6 -> 54.0 ms with the split items pooled, 53.4 ms
// with 32 unsplit items per XCD as well (64: the same), alternating on one
// box.
constexpr int kPoolPerXcd = 32;

__global__ void attn_zero_counter_kernel(unsigned* c) { *c = 0u; }

template <int D, int OUT>
void launch_fwd_mixed(const AttnArgs& a, hipStream_t st) {
  constexpr int DV = kPVWidth<D>;
  hipLaunchKernelGGL(attn_zero_counter_kernel, dim3(1), dim3(1), 0, st, a.item_counter);
  hipLaunchKernelGGL((attn_fwd_kernel<D, DV, OUT, false, false, false, true>), dim3(a.n_grid),
                     dim3(512), 0, st, a);
}

// Multi-block launches pay off where a workgroup's fixed cost (Q load,
// first-tile latency, pipeline fill and drain, output store, all serialised
// with one workgroup per CU) is large against its key tiles: short,
// unmasked key ranges.  Costs in units of one key tile's time: a workgroup's
// fixed cost is ~7 tiles (measured: a Skv sweep at the Wan query shape
// extrapolates to 0.51 ms at Skv = 0 against 0.074 ms per 128 keys over 46
// rounds of workgroups), and a block switch inside a multi-block workgroup
// costs about one to two tiles (measured on the same sweep; the plans do not
// change between the two).  Returns the query blocks per workgroup (1: off)
// that minimises rounds-of-256-workgroups x workgroup time.
constexpr int kMultiMaxTiles = 32;  // key tiles per block up to which it applies
constexpr int kCUs = 256;
constexpr int64_t kFixedTiles = 7, kSwitchTiles = 1;
inline int multi_block_plan(const AttnArgs& a, int D) {
  const int n_kb = (a.Skv + kBlockN - 1) / kBlockN;
  const int64_t heads = (int64_t)a.B * a.H;
  if (a.mask != RP_MASK_NONE || a.kv_splits != 1 || D > 128 || n_kb > kMultiMaxTiles ||
      a.qb_begin != 0)
    return 1;
  auto rounds = [&](int64_t wgs) { return (wgs + kCUs - 1) / kCUs; };
  int best = 1;
  int64_t best_cost = rounds(heads * a.n_qblocks) * (n_kb + kFixedTiles);
  for (int per = 2; per <= a.n_qblocks; ++per) {
    const int64_t wgs = heads * ((a.n_qblocks + per - 1) / per);
    const int64_t cost = rounds(wgs) * (per * (n_kb + kSwitchTiles) + kFixedTiles);
    if (cost < best_cost) {
      best = per;
      best_cost = cost;
    }
  }
  return best;
}

// Key tiles per split and the number of non-empty splits for a request of
// `kv_splits`.
inline void split_plan(int Skv, int kv_splits, int* split_tiles, int* n_splits) {
  const int n_kb = (Skv + kBlockN - 1) / kBlockN;
  const int want = max(1, min(kv_splits, n_kb));
  *split_tiles = (n_kb + want - 1) / want;
  *n_splits = (n_kb + *split_tiles - 1) / *split_tiles;
}

// Balanced launches.  A launch of W workgroups, one per CU, runs in
// ceil(W / CUs) rounds of equal length (measured at the Wan shape: 45, 46
// and 47 rounds take 48.7, 49.9 and 51.2 ms), so a last partial round costs
// a whole one.  For an unmasked launch of one query block per workgroup the
// plan keeps the largest number of query blocks per head whose workgroups
// fill whole rounds, and splits the keys of the remaining blocks s ways
// (s = 2, 4 or 8), so that their workgroups, each about 1/s of a whole one,
// fill the last rounds; attn_combine_kernel merges their partial results.
// C3 self (40 heads x 296 blocks on 256 CUs): 288 blocks per head in 45
// rounds, the last 8 split 4 ways in 1.25 round-equivalents, against 47.
// Both kinds of workgroup run in one launch, the split ones last: they also
// fill the uneven end of the unsplit rounds, which a second launch would
// wait for, and they are pooled with the last unsplit items of every XCD's
// share (kPoolPerXcd).
struct TailPlan {
  int main_blocks;   // query blocks per head run unsplit
  int splits;        // key splits of the remaining blocks (1: a plain launch)
};
inline TailPlan tail_plan(int B, int H, int Sq, int Skv, int D, int mask, int cus) {
  const int nq = (Sq + kBlockM - 1) / kBlockM;
  TailPlan t{nq, 1};
  if (mask != RP_MASK_NONE || cus <= 0 || B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0) return t;
  AttnArgs a{};
  a.B = B; a.H = H; a.Sq = Sq; a.Skv = Skv; a.mask = mask; a.kv_splits = 1; a.n_qblocks = nq;
  if (multi_block_plan(a, D) > 1) return t;
  const int n_kb = (Skv + kBlockN - 1) / kBlockN;
  const int64_t per_block = (int64_t)B * H * (D == 256 ? 2 : 1);   // workgroups per block row
  int64_t g = per_block, c = cus;
  while (c) { const int64_t r = g % c; g = c; c = r; }             // gcd(per_block, cus)
  const int64_t step = cus / g;      // blocks per head that fill whole rounds
  const int64_t m = (nq / step) * step;
  // the unsplit workgroups spread evenly over the 8 XCDs
  if (m == nq || m == 0 || (per_block * m) % 8 != 0) return t;
  const int64_t tail = per_block * (nq - m);
  auto rounds = [&](int64_t w, int s) { return (double)((w + cus - 1) / cus) / s; };
  double best = rounds(tail, 1);
  int best_s = 1;
  for (int sp = 2; sp <= 8 && 2 * sp <= n_kb; sp *= 2) {
    // ~0.05 of a round for the partial results and the merge
    const double cost = rounds(tail * sp, sp) + 0.05;
    if (cost < best) {
      best = cost;
      best_s = sp;
    }
  }
  if (best_s > 1) t = TailPlan{(int)m, best_s};
  return t;
}

// CUs of the stream's device (its current device for a null stream); 0 when
// the runtime cannot tell.
inline int stream_cus(void* stream) {
  int dev = 0, v = 0;
  const hipError_t e = stream ? hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev)
                              : hipGetDevice(&dev);
  if (e != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return v;
}

// kOutBf16 / kOutF32 / kOutF16 for an RP_OUT_* value
inline int out_kind(int out_dtype) {
  return out_dtype == RP_OUT_F32 ? kOutF32 : out_dtype == RP_OUT_F16 ? kOutF16 : kOutBf16;
}

inline bool kvres_applies(const AttnArgs& a, int D);
template <int D>
int launch_kvres(const AttnArgs& base, int out_dtype, hipStream_t st, int cus);

template <int D>
int launch_attn(const AttnArgs& base, int out_dtype, hipStream_t st) {
  const int kind = out_kind(out_dtype);
  AttnArgs a = base;
  a.n_qblocks = (a.Sq + kBlockM - 1) / kBlockM;
  a.D = D;
  a.dv_halves = D / kPVWidth<D>;
  a.qb_per_wg = multi_block_plan(a, D);
  a.wg_per_bh = (a.n_qblocks + a.qb_per_wg - 1) / a.qb_per_wg;
  // a key range resident in LDS runs the persistent resident-K/V kernel
  if constexpr (D == 64 || D == 128) {
    if (kvres_applies(a, D)) return launch_kvres<D>(a, out_dtype, st, stream_cus(st));
  }
  if (a.q16 != nullptr && a.qb_per_wg > 1) {
    rp_set_error("attn: the multi-block launch of this shape takes Q as codes only");
    return RP_ERR_UNSUPPORTED;
  }
  // a mixed launch: blocks [0, qb_begin) unsplit, the rest key-split
  const bool mixed = a.qb_begin > 0;
  const int64_t heads = (int64_t)a.B * a.H * a.dv_halves;
  const int64_t work =
      a.qb_per_wg > 1 ? (int64_t)a.wg_per_bh * a.B * a.H
      : mixed ? heads * (a.qb_begin + (int64_t)(a.n_qblocks - a.qb_begin) * a.kv_splits)
              : heads * a.n_qblocks * a.kv_splits;
  if (work > 0x7fffffff || (int64_t)a.B * a.H * a.Sq * (D / 4) > 0x7fffffffLL * 256) {
    rp_set_error("attn: grid too large");
    return RP_ERR_UNSUPPORTED;
  }
  a.n_work = (int)work;
  a.n_main = mixed ? (int)(heads * a.qb_begin) : 0;
  if (mixed && (a.n_main % 8 != 0 || a.kv_splits < 2 || a.mask != RP_MASK_NONE ||
                a.item_counter == nullptr)) {
    rp_set_error("attn: mixed launch needs unsplit workgroups in multiples of 8, key splits, "
                 "no mask and an item counter");
    return RP_ERR_UNSUPPORTED;
  }
  // pooled items: the last pool_r unsplit items of each XCD's share and the
  // split items, run by twice as many workgroups, the same number per XCD
  a.pool_r = mixed ? min(kPoolPerXcd, a.n_main / 8) : 0;
  const int64_t pooled = 8 * (int64_t)a.pool_r + (work - a.n_main);
  const int64_t grid = mixed ? a.n_main - 8 * a.pool_r + (2 * pooled + 7) / 8 * 8 : work;
  if (grid > 0x7fffffff) {
    rp_set_error("attn: grid too large");
    return RP_ERR_UNSUPPORTED;
  }
  a.n_grid = (int)grid;
  if (a.kv_splits == 1) {
    if (kind == kOutF32)
      launch_fwd<D, kOutF32>(a, st);
    else if (kind == kOutF16)
      launch_fwd<D, kOutF16>(a, st);
    else
      launch_fwd<D, kOutBf16>(a, st);
  } else {
    if (!mixed)
      launch_fwd<D, kOutSplit>(a, st);
    else if (kind == kOutF32)
      launch_fwd_mixed<D, kOutF32>(a, st);
    else if (kind == kOutF16)
      launch_fwd_mixed<D, kOutF16>(a, st);
    else
      launch_fwd_mixed<D, kOutBf16>(a, st);
    const int64_t threads = (int64_t)a.B * a.H * a.ws_rows * (D / 4);
    const dim3 cgrid((unsigned)((threads + 255) / 256)), cblock(256);
    if (kind == kOutF32)
      hipLaunchKernelGGL((attn_combine_kernel<D, kOutF32>), cgrid, cblock, 0, st, a);
    else if (kind == kOutF16)
      hipLaunchKernelGGL((attn_combine_kernel<D, kOutF16>), cgrid, cblock, 0, st, a);
    else
      hipLaunchKernelGGL((attn_combine_kernel<D, kOutBf16>), cgrid, cblock, 0, st, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    rp_set_error("attn: launch failed: %s", hipGetErrorString(e));
    return RP_ERR_LAUNCH;
  }
  return RP_OK;
}

// ---------------------------------------------------------------------------
// Short query ranges: keys split across the waves of one workgroup.
//
// A workgroup of eight waves takes QG groups of 32 query rows of one head
// (BLOCK_M = 32 QG) and gives each group 8 / QG waves, one run of key tiles
// each: wave s covers the tiles [s * split_tiles, (s + 1) * split_tiles) of
// the key range (split_plan).  A wave loads its operands straight from
// global memory into registers (K rows in the permuted S^T order, V^T rows
// of the transposed V) -- no barrier in the tile loop -- and
// runs the per-tile arithmetic of attn_fwd_kernel (S^T = K . Q^T, base-2
// online softmax, P = e4m3(p * 448), O^T += V^T . P^T).  Its K tile, then
// its V^T tile, pass through a region of LDS of its own, filled by
// direct-to-LDS loads of whole KiB (eight 128-byte rows per instruction) in
// attn_fwd_kernel's padded operand layout and read back as MFMA operands:
// loaded straight into the operand registers, every 16-byte piece of a wave
// instruction lies in another row, and the C5 tile loads took 4 us.
//
// The waves of a query group reproduce the one-range algorithm, not a key
// split: P of tile t is quantized against the running max of tiles 0..t,
// as in the reference's loop (fp8_flash_attn.py:334-380).  Each wave first
// takes the row maxima of its own tiles and leaves them in LDS; after a
// workgroup barrier it starts its running max from the maximum over the
// tiles of the waves before it, which is the reference's running max at its
// first tile.  With one tile per wave the scores stay in registers across
// the barrier; with more, the wave computes its S^T tiles once for their
// maxima and again for P.  Wave s then holds tile run s's row sum l_s and
// unnormalised O^T_s relative to its final running max m_s, and the
// workgroup merges them in LDS: out = sum_s w_s O_s * v_scale /
// sum_s w_s l_s with w_s = exp2(m_s - m), m = max_s m_s.  That is the
// reference's l and acc with the rescale factors of the later tiles
// multiplied out, up to fp32 rounding.  One launch, no workspace.  Where the
// 256-row kernel runs a few dozen workgroups through their whole key range
// one tile after another (C1: 32 workgroups x 8 tiles), this one runs eight
// times as many, each wave over a fraction of the tiles.
constexpr int kWsWaves = 8;

template <int D, int QG>
struct WsGeo {
  using T = Geo<D, D, 8>;                       // attn_fwd_kernel's tile layout in LDS
  static constexpr int SPLITS = kWsWaves / QG;  // tile runs (waves) per query group
  static constexpr int KSTEPS = D / 64;
  static constexpr int ETILES = D / 32;
  static constexpr int OPITCH = D + 4;          // fp32 per staged O row: an odd granule count
  static constexpr int ROWS = 32 * QG;          // query rows per workgroup
  static constexpr int CPT = ROWS * D / 512;    // output columns per merging thread
  // a wave's LDS region: its K tile, then its V^T tile, then its O^T rows
  static constexpr int REGION = (T::K_BLKS > T::V_BLKS ? T::K_BLKS : T::V_BLKS) * 1024;
  static constexpr int LDS_BYTES = kWsWaves * (REGION + 32 * 12);
  static_assert(D == 64 || D == 128, "head dim");
  static_assert(QG == 1 || QG == 2 || QG == 4, "query groups");
  static_assert(CPT % 4 == 0, "whole float4 columns");
  static_assert(32 * OPITCH * 4 <= REGION, "O^T rows fit the region");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS");
};

// x, or -inf unless O lies in [i0, i0 + w] (O - i0 <= w, unsigned): one
// subtract, compare and select per score.  Written as asm so that each
// compare's lane mask is consumed at once -- as C the compiler computes all
// 64 compares of a tile first and spills their masks; O, the score's key
// offset, is an immediate.
template <int O>
__device__ __forceinline__ float mask1(float x, int i0, unsigned w, float ninf) {
  int t;
  asm("v_sub_u32 %1, %3, %4\n\tv_cmp_le_u32 vcc, %1, %5\n\tv_cndmask_b32 %0, %2, %0, vcc"
      : "+v"(x), "=&v"(t)
      : "v"(ninf), "n"(O), "v"(i0), "v"(w)
      : "vcc");
  return x;
}
// the same for the union of [i0, i0 + w] and [j0, j0 + u]
template <int O>
__device__ __forceinline__ float mask2(float x, int i0, unsigned w, int j0, unsigned u,
                                       float ninf) {
  int t;
  uint64_t m;
  asm("v_sub_u32 %1, %4, %5\n\tv_cmp_le_u32 vcc, %1, %6\n\t"
      "v_sub_u32 %1, %4, %7\n\tv_cmp_le_u32 %2, %1, %8\n\t"
      "s_or_b64 vcc, vcc, %2\n\tv_cndmask_b32 %0, %3, %0, vcc"
      : "+v"(x), "=&v"(t), "=&s"(m)
      : "v"(ninf), "n"(O), "v"(i0), "v"(w), "v"(j0), "v"(u)
      : "vcc");
  return x;
}
// f(integral_constant<int, t>) for t = 0 .. 63, the scores of a lane in
// register order (block t / 16, register t % 16)
template <typename F, int... T>
__device__ __forceinline__ void each_score(F&& f, std::integer_sequence<int, T...>) {
  (f(std::integral_constant<int, T>{}), ...);
}

__device__ __forceinline__ i32x8 gload32(const uint8_t* p) {
  const i32x4* s = reinterpret_cast<const i32x4*>(p);
  return cat8(s[0], s[1]);
}


template <int D, int QG, int OUT>
__global__ __launch_bounds__(512, 1)
void attn_wsplit_kernel(AttnArgs a) {
  using G = WsGeo<D, QG>;
  using GT = typename G::T;
  __shared__ __attribute__((aligned(1024))) uint8_t s_stage[kWsWaves * G::REGION];
  __shared__ float2 s_ml[kWsWaves * 32];
  __shared__ float s_tm[kWsWaves * 32];   // row max of each wave's tiles (exp2 domain)

  // work item: (head, block of ROWS query rows); the XCD-aware remap of
  // attn_fwd_kernel puts one head's blocks on one XCD (its K/V in one L2)
  const int w = blockIdx.x;
  const int xcd = w & 7, k_x = w >> 3;
  const int per = a.n_work >> 3, rem = a.n_work & 7;
  const int L = xcd * per + min(xcd, rem) + k_x;
  const int bh = L / a.n_qblocks, qb = L - bh * a.n_qblocks;
  const int b = bh / a.H, h = bh - b * a.H;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qg = wave % QG, sp = wave / QG;   // query group, tile run
  const int lq = lane & 31, lg = lane >> 5;
  const int q_wave0 = qb * G::ROWS + qg * 32;
  const int q = q_wave0 + lq;
  const int q_last = min(q_wave0 + 31, a.Sq - 1);

  const uint8_t* qh = a.q + (int64_t)bh * a.Sq * D;
  const uint8_t* kh = a.k + (int64_t)bh * a.Skv * D;
  const uint8_t* vh = a.vt + (int64_t)bh * D * a.ldv;
  const float q_scale = a.qs[bh * a.scale_stride];
  const float k_scale = a.ks[bh * a.scale_stride];
  const float v_scale = a.vs[bh * a.scale_stride];
  // the exp2-domain score factor, as in attn_fwd_kernel
  const float c2_raw = ((a.sm_scale * q_scale) * k_scale) * kLog2e;
  const float c2 = c2_raw == 0.0f ? 1.17549435e-38f : c2_raw;

  // this wave's tiles; under a mask, the tiles past every key its rows can
  // see hold nothing visible and are skipped (their scores would all be
  // -inf: they move neither the running max nor l nor O)
  const int n_kb = (a.Skv + kBlockN - 1) / kBlockN;
  const int t_begin = sp * a.split_tiles;
  int t_end = min(n_kb, t_begin + a.split_tiles);
  if (a.mask == RP_MASK_CAUSAL) t_end = min(t_end, q_last / kBlockN + 1);
  if (a.mask == RP_MASK_SHARED_PREFIX)
    t_end = min(t_end, (a.prefix + q_last) / kBlockN + 1);

  i32x8 qop[G::KSTEPS];
  {
    const uint8_t* src = qh + (int64_t)min(q, a.Sq - 1) * D + 32 * lg;
#pragma unroll
    for (int ks = 0; ks < G::KSTEPS; ++ks) qop[ks] = gload32(src + 64 * ks);
  }

  // first key of tile j: the last tile of a ragged key range is shifted back
  // to end at key Skv - 1, its repeats masked (attn_fwd_kernel's
  // tile_begin); a range shorter than one tile re-reads key Skv - 1
  auto tile_begin = [&](int j) {
    const int kv0 = j * kBlockN;
    return (kv0 + kBlockN > a.Skv && a.Skv >= kBlockN) ? a.Skv - kBlockN : kv0;
  };
  // this wave's LDS region (byte address for the direct-to-LDS loads)
  uint8_t* const region = s_stage + wave * G::REGION;
  const uint32_t region_lds = (uint32_t)(uintptr_t)(lds_ptr_t)region;
  // K tile from key kbeg into the region: LDS row 32 hh + rho holds key
  // key_of(hh, rho), each row one pad granule longer (the pad re-loads the
  // row's first granule; rows past Skv re-read key Skv - 1)
  // (rolled loops: unrolled, the per-lane addresses of all blocks stay live
  // and spill at D = 128)
  auto stage_k = [&](int kbeg) __attribute__((always_inline)) {
#pragma unroll 1
    for (int b = 0; b < GT::K_BLKS; ++b) {
      const int p = b * kWave + lane;
      const int row = p / GT::K_GRAN, slot = p % GT::K_GRAN;
      const int key = min(kbeg + key_of(row >> 5, row & 31), a.Skv - 1);
      gload_lds16(kh + (int64_t)key * D + (slot < GT::KVALID ? slot : 0) * 16,
                  region_lds + (uint32_t)b * 1024u);
    }
  };
  // V^T columns [kbeg, kbeg + 128) into the region: LDS row d holds V^T row
  // d (rows past D in the last, rounded-up KiB re-load row D - 1)
  auto stage_v = [&](int kbeg) __attribute__((always_inline)) {
#pragma unroll 1
    for (int b = 0; b < GT::V_BLKS; ++b) {
      const int p = b * kWave + lane;
      const int d = min(p / GT::V_GRAN, D - 1), slot = p % GT::V_GRAN;
      gload_lds16(vh + (int64_t)d * a.ldv + kbeg + (slot < kBlockN / 16 ? slot : 0) * 16,
                  region_lds + (uint32_t)b * 1024u);
    }
  };
  // the staged V^T tile as PV operands (its loads waited for)
  auto read_v = [&](i32x8 (&vop)[G::ETILES][2]) __attribute__((always_inline)) {
    const uint32_t vb = region_lds + (uint32_t)(lq * GT::V_PITCH + 32 * lg);
#pragma unroll
    for (int e = 0; e < G::ETILES; ++e)
#pragma unroll
      for (int m = 0; m < 2; ++m) vop[e][m] = lds_op(vb + 32 * e * GT::V_PITCH + 64 * m);
  };
  // V^T of tile j into registers, once the K operands have left the region
  auto fetch_v = [&](i32x8 (&vop)[G::ETILES][2], int kbeg) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the region's K reads are done
    stage_v(kbeg);
    wait_vmem_all();
    read_v(vop);
  };
  // S^T of tile j with the mask applied; returns the row max of the raw
  // dot products over the visible keys (-inf if none), combined over the
  // lane pair that shares the row.  With `stage_v_too` the tile's V^T loads
  // go out into the region right after the K operands are read from it.
  auto scores = [&](int j, f32x16 (&s)[4], bool stage_v_too)
      __attribute__((always_inline)) -> float {
    const int kv0 = j * kBlockN;
    const int kbeg = tile_begin(j);
    stage_k(kbeg);
    wait_vmem_all();
    i32x8 kop[4][G::KSTEPS];
    {
      const uint32_t kb = region_lds + (uint32_t)(lq * GT::K_PITCH + 32 * lg);
#pragma unroll
      for (int hh = 0; hh < 4; ++hh)
#pragma unroll
        for (int ks = 0; ks < G::KSTEPS; ++ks)
          kop[hh][ks] = lds_op(kb + 32 * hh * GT::K_PITCH + 64 * ks);
    }
    if (stage_v_too) {
      __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): K is out of the region
      stage_v(kbeg);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < G::KSTEPS; ++ks)
#pragma unroll
      for (int hh = 0; hh < 4; ++hh)
        s[hh] = mfma_32x32x64(kop[hh][ks], qop[ks], ks == 0 ? f32x16{} : s[hh]);
    __builtin_amdgcn_sched_barrier(0);
    bool masked = kv0 + kBlockN > a.Skv;
    if (a.mask == RP_MASK_CAUSAL) masked |= kv0 + kBlockN - 1 > q_wave0;
    if (a.mask == RP_MASK_SHARED_PREFIX) masked |= kv0 + kBlockN > a.prefix;
    if (masked) {
      const float ninf = -__builtin_inff();
      int lo = 0, hi = a.Skv - 1;
      if (a.mask == RP_MASK_CAUSAL) hi = min(q, hi);
      if (a.mask == RP_MASK_SHARED_PREFIX) {
        lo = a.prefix + q - q % a.suffix;
        hi = min(a.prefix + q, hi);
      }
      const int pre_end = a.mask == RP_MASK_SHARED_PREFIX ? min(a.prefix, a.Skv) : 0;
      const int kvl = kbeg + 32 * lg;
      const int lo_t = lo - kvl, hi_t = hi - kvl, pe_t = pre_end - kvl, new_t = kv0 - kvl;
      // the visible keys of a lane, o = key - kvl: the window [lo, hi] and
      // the shared prefix [0, pre_end), both from the tile's first new key
      // on; each interval [i0, i0 + w] is one unsigned compare per score
      // (o - i0 <= w), an empty one starts past every o
      auto interval = [](int i0, int i1, int& start, unsigned& width) {
        start = i1 >= i0 ? i0 : (1 << 20);
        width = i1 >= i0 ? (unsigned)(i1 - i0) : 0u;
      };
      int w0, p0;
      unsigned ww, pw;
      interval(max(lo_t, new_t), hi_t, w0, ww);
      // score t of the lane: block hh = t / 16, register r = t % 16, key
      // offset o = 64 (hh / 2) + 16 (hh % 2) + r
      if (pre_end <= kv0) {   // no prefix key in the tile (wave-uniform)
        each_score([&](auto tc) __attribute__((always_inline)) {
          constexpr int t = decltype(tc)::value, hh = t / 16, r = t % 16;
          s[hh][r] = mask1<64 * (hh >> 1) + 16 * (hh & 1) + r>(s[hh][r], w0, ww, ninf);
        }, std::make_integer_sequence<int, 64>{});
      } else {
        interval(new_t, pe_t - 1, p0, pw);
        each_score([&](auto tc) __attribute__((always_inline)) {
          constexpr int t = decltype(tc)::value, hh = t / 16, r = t % 16;
          s[hh][r] = mask2<64 * (hh >> 1) + 16 * (hh & 1) + r>(s[hh][r], w0, ww, p0, pw, ninf);
        }, std::make_integer_sequence<int, 64>{});
      }
    }
    float mt[4];
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      float x = max3f(s[hh][0], s[hh][1], s[hh][2]);
#pragma unroll
      for (int r = 3; r < 15; r += 2) x = max3f(x, s[hh][r], s[hh][r + 1]);
      mt[hh] = max3f(x, s[hh][15], s[hh][15]);
    }
    return xhalf_max(max3f(mt[0], mt[1], max3f(mt[2], mt[3], mt[3])));
  };

  f32x16 acc[G::ETILES];
  float m_run, l_run = 0.0f;
  // P of a tile from its scores and raw max, the running max and the rescale
  // of l and O^T (attn_fwd_kernel's softmax phase and P.V products); FIRST:
  // O^T and l start here, from the first P.V product
  auto consume = [&](f32x16 (&s)[4], float mx, const i32x8 (&vop)[G::ETILES][2],
                     auto first_c) __attribute__((always_inline)) {
    constexpr bool FIRST = decltype(first_c)::value;
    const float m_new = max3f(m_run, mx * c2, mx * c2);
    const float m_use = (m_new == -__builtin_inff()) ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    const float moff = m_use - kLog2PMax;
    i32x8 pop[2];
    float ps[4] = {-0.0f, -0.0f, -0.0f, -0.0f};
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      int pw[8];
#pragma unroll
      for (int wd = 0; wd < 8; ++wd) {
        const int hh = 2 * m + (wd >> 2);
        const int r = 4 * (wd & 3);
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hh][r + 0], c2, -moff));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hh][r + 1], c2, -moff));
        const float p2 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hh][r + 2], c2, -moff));
        const float p3 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hh][r + 3], c2, -moff));
        ps[wd & 3] += (p0 + p1) + (p2 + p3);
        pw[wd] = (int)pack4_e4m3(p0, p1, p2, p3);
      }
      pop[m] = i32x8{pw[0], pw[1], pw[2], pw[3], pw[4], pw[5], pw[6], pw[7]};
    }
    const float psum = (ps[0] + ps[1]) + (ps[2] + ps[3]);
    if constexpr (FIRST) {
      l_run = psum;
    } else {
      l_run = l_run * alpha + psum;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int e = 0; e < G::ETILES; ++e)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[e][r] *= alpha;
      }
    }
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int e = 0; e < G::ETILES; ++e)
        acc[e] = mfma_32x32x64(vop[e][m], pop[m], FIRST && m == 0 ? f32x16{} : acc[e]);
  };
  // running max at this wave's first tile: the max over the tiles of the
  // waves before it in its query group
  auto prefix_max = [&]() {
    float m = -__builtin_inff();
    for (int s2 = 0; s2 < sp; ++s2) m = fmaxf(m, s_tm[(s2 * QG + qg) * 32 + lq]);
    return m;
  };

  const bool has_tiles = t_begin < t_end;
  if (a.split_tiles == 1) {
    // one tile per wave: its scores stay in registers across the barrier
    f32x16 s[4];
    i32x8 vop[G::ETILES][2];
    float mx = -__builtin_inff();
    if (has_tiles) mx = scores(t_begin, s, true);
    if (lg == 0) s_tm[wave * 32 + lq] = mx * c2;
    __syncthreads();
    m_run = prefix_max();
    if (has_tiles) {
      wait_vmem_all();   // the V^T tile staged before the barrier
      read_v(vop);
      consume(s, mx, vop, std::true_type{});
    }
  } else {
    // several tiles per wave: their maxima first, then P and O^T
    float wm = -__builtin_inff();
    for (int j = t_begin; j < t_end; ++j) {
      f32x16 s[4];
      wm = fmaxf(wm, scores(j, s, false));
    }
    if (lg == 0) s_tm[wave * 32 + lq] = wm * c2;
    __syncthreads();
    m_run = prefix_max();
    if (has_tiles) {
      f32x16 s[4];
      i32x8 vop[G::ETILES][2];
      float mx = scores(t_begin, s, false);
      fetch_v(vop, tile_begin(t_begin));
      consume(s, mx, vop, std::true_type{});
      for (int j = t_begin + 1; j < t_end; ++j) {
        mx = scores(j, s, false);
        fetch_v(vop, tile_begin(j));
        consume(s, mx, vop, std::false_type{});
      }
    }
  }
  if (!has_tiles) {
#pragma unroll
    for (int e = 0; e < G::ETILES; ++e) acc[e] = f32x16{};
  }

  // ---- each wave's state into LDS: (m, l) per row, O^T as rows of fp32 in
  // its own region (its V^T reads, earlier LDS operations of the same wave,
  // are done first); waves past the plan's run count write nothing
  if (sp < a.kv_splits) {
    const float l_split = xhalf_sum(l_run);
    if (lg == 0) s_ml[wave * 32 + lq] = make_float2(m_run, l_split);
    float* const o_w = reinterpret_cast<float*>(region) + lq * G::OPITCH;
#pragma unroll
    for (int e = 0; e < G::ETILES; ++e)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4*>(o_w + 32 * e + 8 * i + 4 * lg) =
            make_float4(acc[e][4 * i], acc[e][4 * i + 1], acc[e][4 * i + 2], acc[e][4 * i + 3]);
  }
  __syncthreads();

  // ---- merge: out = sum_s w_s O_s * v_scale / sum_s w_s l_s with
  // w_s = exp2(m_s - max_s m_s) over the waves that saw a key of the row
  // (attn_combine_kernel's formula, runs in ascending order)
  constexpr int TPR = D / G::CPT;             // merging threads per row
  const int r = tid / TPR, c0 = (tid % TPR) * G::CPT;
  const int rg = r >> 5, rl = r & 31;
  const int nsp = a.kv_splits;   // <= SPLITS
  float mmax = -__builtin_inff();
#pragma unroll
  for (int s2 = 0; s2 < G::SPLITS; ++s2) {
    if (s2 >= nsp) break;
    const float2 v = s_ml[(s2 * QG + rg) * 32 + rl];
    if (v.y != 0.0f) mmax = fmaxf(mmax, v.x);
  }
  float l = 0.0f;
  float o[G::CPT];
#pragma unroll
  for (int c = 0; c < G::CPT; ++c) o[c] = 0.0f;
#pragma unroll
  for (int s2 = 0; s2 < G::SPLITS; ++s2) {
    if (s2 >= nsp) break;
    const int ws = s2 * QG + rg;
    const float2 v = s_ml[ws * 32 + rl];
    const float wgt = v.y != 0.0f ? __builtin_amdgcn_exp2f(v.x - mmax) : 0.0f;
    l += wgt * v.y;
    const float* src = reinterpret_cast<const float*>(s_stage + ws * G::REGION) +
                       rl * G::OPITCH + c0;
#pragma unroll
    for (int c = 0; c < G::CPT; c += 4) {
      const float4 x = *reinterpret_cast<const float4*>(src + c);
      o[c] += wgt * x.x; o[c + 1] += wgt * x.y; o[c + 2] += wgt * x.z; o[c + 3] += wgt * x.w;
    }
  }
  const int qrow = qb * G::ROWS + r;
  if (qrow < a.Sq) {
    const float inv = v_scale / l;
    const int64_t obase = (int64_t)b * a.osb + (int64_t)h * a.osh + (int64_t)qrow * a.oss + c0;
#pragma unroll
    for (int c = 0; c < G::CPT; c += 4) {
      const float o0 = o[c] * inv, o1 = o[c + 1] * inv, o2 = o[c + 2] * inv, o3 = o[c + 3] * inv;
      if constexpr (OUT == kOutF32) {
        *reinterpret_cast<float4*>(static_cast<float*>(a.out) + obase + c) =
            make_float4(o0, o1, o2, o3);
      } else {
        uint2 pk;
        if constexpr (OUT == kOutF16) {
          pk.x = pack_f16x2(o0, o1);
          pk.y = pack_f16x2(o2, o3);
        } else {
          pk.x = pack_bf16x2(o0, o1);
          pk.y = pack_bf16x2(o2, o3);
        }
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + obase + c) = pk;
      }
    }
  }
}

template <int D, int QG>
int launch_wsplit(const AttnArgs& base, int out_dtype, hipStream_t st) {
  using G = WsGeo<D, QG>;
  AttnArgs a = base;
  a.D = D;
  a.n_qblocks = (a.Sq + G::ROWS - 1) / G::ROWS;
  int split_tiles = 0, n_splits = 1;
  split_plan(a.Skv, G::SPLITS, &split_tiles, &n_splits);
  a.split_tiles = split_tiles;
  a.kv_splits = n_splits;
  const int64_t work = (int64_t)a.B * a.H * a.n_qblocks;
  if (work > 0x7fffffff) {
    rp_set_error("attn: grid too large");
    return RP_ERR_UNSUPPORTED;
  }
  a.n_work = (int)work;
  const dim3 grid(a.n_work), block(512);
  const int kind = out_kind(out_dtype);
  if (kind == kOutF32)
    hipLaunchKernelGGL((attn_wsplit_kernel<D, QG, kOutF32>), grid, block, 0, st, a);
  else if (kind == kOutF16)
    hipLaunchKernelGGL((attn_wsplit_kernel<D, QG, kOutF16>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((attn_wsplit_kernel<D, QG, kOutBf16>), grid, block, 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    rp_set_error("attn: launch failed: %s", hipGetErrorString(e));
    return RP_ERR_LAUNCH;
  }
  return RP_OK;
}

template <int D>
int launch_wsplit_rows(const AttnArgs& a, int block_m, int out_dtype, hipStream_t st) {
  switch (block_m) {
    case 32: return launch_wsplit<D, 1>(a, out_dtype, st);
    case 64: return launch_wsplit<D, 2>(a, out_dtype, st);
    default: return launch_wsplit<D, 4>(a, out_dtype, st);
  }
}

// ---------------------------------------------------------------------------
// Short key ranges against many queries (cross-attention: C3's 512 text
// keys): the head's whole K and V^T resident in LDS.
//
// One workgroup per CU, persistent: it takes a contiguous run of the
// launch's tasks -- 32 query rows of one head each, head-major -- loads the
// K and V^T of each head it meets into LDS once (K rows in the S^T operand
// order of attn_fwd_kernel, tile after tile; V^T rows d), and its eight
// waves then take the head's tasks in turn.  A task is one wave's whole
// attention for its 32 rows: Q^T into registers, then tile after tile S^T
// = K . Q^T, the base-2 online softmax, P = e4m3(p * 448) and O^T += V^T .
// P^T with the operands read from LDS, and the rows' output stored -- the
// one-range arithmetic of attn_fwd_kernel with the tiles in the reference's
// order (a ragged last tile masks its keys past Skv).  No barrier runs
// inside a head's tasks, and each wave pipelines its own steps: the next
// tile's S^T MFMAs go out between the halves of the current tile's softmax
// (see the loop).  At C3 cross (40 heads x 75,600 queries x 512 keys) this
// takes 0.52-0.53 ms against the multi-block launch's 0.58 ms; the same
// kernel with the main kernel's barrier ping-pong took 0.567 ms, and
// starting the two waves of a SIMD up to 1,500 cycles apart changed nothing.
template <int D>
struct KvGeo {
  static constexpr int KSTEPS = D / 64;
  static constexpr int ETILES = D / 32;
  static constexpr int K_PITCH = D + 16;         // an odd number of 16-byte granules
  static constexpr int K_GRAN = K_PITCH / 16;
  static constexpr int MAX_TILES = D == 128 ? 4 : 8;
  static constexpr int K_BYTES = MAX_TILES * kBlockN * K_PITCH;
  static constexpr int V_BYTES = D * (MAX_TILES * kBlockN + 16);
  static_assert(D == 64 || D == 128, "head dim");
  static_assert(K_BYTES + V_BYTES <= 156 * 1024, "LDS");
};

// The output rows of one wave's 32 queries from its O^T fragments: row
// q0 + lq gets acc * inv, written through the output strides.  The lane pair
// (l, l + 32) holding a row swaps halves of adjacent 8-column chunks so that
// each 16-bit store writes 16 contiguous bytes (attn_fwd_kernel's store).
template <int DV, int OUT>
__device__ __forceinline__ void store_o_rows(const AttnArgs& a, const f32x16 (&acc)[DV / 32],
                                             float inv, int b, int h, int q, int lg) {
  const bool ok = q < a.Sq;
  const int64_t obase = (int64_t)b * a.osb + (int64_t)h * a.osh + (int64_t)q * a.oss;
  uint2 pend = make_uint2(0u, 0u);
#pragma unroll
  for (int e = 0; e < DV / 32; ++e) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 32 * e + 8 * i + 4 * lg;
      const float o0 = acc[e][4 * i + 0] * inv, o1 = acc[e][4 * i + 1] * inv;
      const float o2 = acc[e][4 * i + 2] * inv, o3 = acc[e][4 * i + 3] * inv;
      if constexpr (OUT == kOutF32) {
        if (ok)
          *reinterpret_cast<float4*>(static_cast<float*>(a.out) + obase + d) =
              make_float4(o0, o1, o2, o3);
      } else {
        uint2 pk;
        if constexpr (OUT == kOutF16) {
          pk.x = pack_f16x2(o0, o1);
          pk.y = pack_f16x2(o2, o3);
        } else {
          pk.x = pack_bf16x2(o0, o1);
          pk.y = pack_bf16x2(o2, o3);
        }
        if (i % 2 == 0) {
          pend = pk;
        } else {
          const auto x = __builtin_amdgcn_permlane32_swap(pend.x, pk.x, false, false);
          const auto y = __builtin_amdgcn_permlane32_swap(pend.y, pk.y, false, false);
          const int c = 4 * e + i - 1 + lg;   // the 8-column chunk this lane now holds
          if (ok)
            *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.out) + obase + 8 * c) =
                make_uint4(x[0], y[0], x[1], y[1]);
        }
      }
    }
  }
}

template <int D, int OUT, bool Q16>
__global__ __launch_bounds__(512, 1)
void attn_kvres_kernel(AttnArgs a) {
  using G = KvGeo<D>;
  __shared__ __attribute__((aligned(16))) uint8_t s_kv[G::K_BYTES + G::V_BYTES];
  uint8_t* const kl = s_kv;                 // K: tile j row 32 hh + rho = key 128 j + key_of(hh, rho)
  uint8_t* const vl = s_kv + G::K_BYTES;    // V^T: row d at d * VP
  const uint32_t kl_lds = (uint32_t)(uintptr_t)(lds_ptr_t)kl;
  const uint32_t vl_lds = (uint32_t)(uintptr_t)(lds_ptr_t)vl;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31, lg = lane >> 5;
  const int n_kb = (a.Skv + kBlockN - 1) / kBlockN;   // <= MAX_TILES (host-checked)
  const int VP = n_kb * kBlockN + 16;                  // V^T LDS pitch: odd granule count
  const int VG = VP / 16;
  const int nq = (a.Sq + 31) / 32;                      // 32-row tasks per head
  const int64_t ntask = (int64_t)a.B * a.H * nq;
  const int64_t t0 = ntask * blockIdx.x / gridDim.x;
  const int64_t t1 = ntask * (blockIdx.x + 1) / gridDim.x;
  const float ninf = -__builtin_inff();

  for (int64_t seg = t0; seg < t1;) {
    const int bh = (int)(seg / nq);
    const int64_t seg_end = min(t1, (int64_t)(bh + 1) * nq);
    const int b = bh / a.H, h = bh - b * a.H;
    const uint8_t* qh = a.q + (int64_t)bh * a.Sq * D;
    const uint8_t* kh = a.k + (int64_t)bh * a.Skv * D;
    const uint8_t* vh = a.vt + (int64_t)bh * D * a.ldv;
    // ---- the head's K and V^T into LDS (keys past Skv re-read key Skv - 1,
    // V^T columns past Skv are the zero tail of the ldv row; pad granules
    // re-read a row's first granule)
    const int kg = n_kb * kBlockN * G::K_GRAN;
    for (int g = tid; g < kg; g += 512) {
      const int row = g / G::K_GRAN, slot = g - row * G::K_GRAN;
      const int j = row >> 7, rho = row & 127;
      const int key = min(j * kBlockN + key_of(rho >> 5, rho & 31), a.Skv - 1);
      const i32x4 v = *reinterpret_cast<const i32x4*>(kh + (int64_t)key * D +
                                                      (slot < D / 16 ? slot : 0) * 16);
      *reinterpret_cast<i32x4*>(kl + row * G::K_PITCH + slot * 16) = v;
    }
    for (int g = tid; g < D * VG; g += 512) {
      const int d = g / VG, slot = g - d * VG;
      const i32x4 v = *reinterpret_cast<const i32x4*>(vh + (int64_t)d * a.ldv +
                                                      (slot < VG - 1 ? slot : 0) * 16);
      *reinterpret_cast<i32x4*>(vl + d * VP + slot * 16) = v;
    }
    const float q_scale = a.qs[bh * a.scale_stride];
    const float k_scale = a.ks[bh * a.scale_stride];
    const float v_scale = a.vs[bh * a.scale_stride];
    const float c2_raw = ((a.sm_scale * q_scale) * k_scale) * kLog2e;
    const float c2 = c2_raw == 0.0f ? 1.17549435e-38f : c2_raw;
    __syncthreads();

    // ---- the head's tasks, wave by wave, as one stream of (task, tile)
    // steps.  Step i computes tile j = i % n_kb of the wave's task i / n_kb:
    // its row max, then P in two halves (score blocks 0-1, then 2-3), then
    // one block of MFMAs: step i + 1's S^T into the consumed score
    // registers, then step i's P.V.  The wave waits on MFMA results only
    // where the next max needs them.  The block runs at raised wave priority,
    // so that its MFMAs go out ahead of the other wave's softmax on the SIMD
    // and run under it.  (Step i + 1's first S^T pair issued between the
    // halves, into the registers the first half had consumed, measured 2.5%
    // slower at C3 cross: the waves' MFMA and VALU stretches overlapped
    // less.)  A task's Q^T is loaded one task ahead.
    auto load_q = [&](i32x8 (&dst)[G::KSTEPS], int64_t task) __attribute__((always_inline)) {
      const int qr = min((int)(task - (int64_t)bh * nq) * 32 + lq, a.Sq - 1);
      const uint8_t* src = qh + (int64_t)qr * D + 32 * lg;
#pragma unroll
      for (int ks = 0; ks < G::KSTEPS; ++ks) dst[ks] = gload32(src + 64 * ks);
    };
    // Q16: a task's Q rows from their 16-bit input, loaded one task ahead
    // as they lie and quantized (quant4, the quantizer's arithmetic) when
    // the task starts
    const float qm = 1.0f / q_scale;
    auto load_qraw = [&](QRaw32 (&dst)[G::KSTEPS], int64_t task) __attribute__((always_inline)) {
      const int qr = min((int)(task - (int64_t)bh * nq) * 32 + lq, a.Sq - 1);
      const uint16_t* src = a.q16 + (int64_t)b * a.qsb + (int64_t)h * a.qsh +
                            (int64_t)qr * a.qss + 32 * lg;
#pragma unroll
      for (int ks = 0; ks < G::KSTEPS; ++ks) dst[ks] = qraw_load(src + 64 * ks);
    };
    auto qcodes = [&](i32x8 (&dst)[G::KSTEPS], const QRaw32 (&raw)[G::KSTEPS])
        __attribute__((always_inline)) {
#pragma unroll
      for (int ks = 0; ks < G::KSTEPS; ++ks) dst[ks] = qraw_codes(raw[ks], qm, a.q_dt);
    };
    const int64_t first = seg + wave;   // the wave's tasks: first, first + 8, ...
    const int ntw = first < seg_end ? (int)((seg_end - first + kWsWaves - 1) / kWsWaves) : 0;
    const int nsteps = ntw * n_kb;
    const uint32_t kb = kl_lds + (uint32_t)(lq * G::K_PITCH + 32 * lg);
    const uint32_t vb = vl_lds + (uint32_t)(lq * VP + 32 * lg);
    f32x16 s[4], acc[G::ETILES];
    i32x8 qop[G::KSTEPS], qnext[G::KSTEPS];
    QRaw32 qnraw[Q16 ? G::KSTEPS : 1];
    // S^T MFMAs of tile jj, score blocks h0 and h0 + 1, against Q^T qq
    auto s_pair = [&](int jj, int h0, const i32x8 (&qq)[G::KSTEPS]) __attribute__((always_inline)) {
      i32x8 kop[2][G::KSTEPS];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int ks = 0; ks < G::KSTEPS; ++ks)
          kop[u][ks] = lds_op(kb + (uint32_t)((jj * kBlockN + 32 * (h0 + u)) * G::K_PITCH + 64 * ks));
#pragma unroll
      for (int ks = 0; ks < G::KSTEPS; ++ks)
#pragma unroll
        for (int u = 0; u < 2; ++u)
          s[h0 + u] = mfma_32x32x64(kop[u][ks], qq[ks], ks == 0 ? f32x16{} : s[h0 + u]);
    };
    if (nsteps > 0) {
      // the next task's Q^T; the last task's "next" re-reads its own rows
      if constexpr (Q16) {
        load_qraw(qnraw, first);
        qcodes(qop, qnraw);
        load_qraw(qnraw, ntw > 1 ? first + kWsWaves : first);
      } else {
        load_q(qop, first);
        load_q(qnext, ntw > 1 ? first + kWsWaves : first);
      }
      s_pair(0, 0, qop);
      s_pair(0, 2, qop);
    }
    float m_run = -__builtin_inff(), l_run = 0.0f;
    for (int i = 0; i < nsteps; ++i) {
      const int t = i / n_kb, j = i - t * n_kb;
      const bool ends_task = j == n_kb - 1;
      const int jn = ends_task ? 0 : j + 1;    // tile of step i + 1
      if (j == 0) m_run = -__builtin_inff();
      // keys past Skv in a ragged last tile
      if (j * kBlockN + kBlockN > a.Skv) {
        // visible key offsets o = key - (128 j + 32 lg): [0, last]
        const int last = a.Skv - 1 - j * kBlockN - 32 * lg;
        const int i0 = last >= 0 ? 0 : (1 << 20);
        const unsigned wd = last >= 0 ? (unsigned)last : 0u;
        each_score([&](auto tc) __attribute__((always_inline)) {
          constexpr int tt = decltype(tc)::value, hh = tt / 16, r = tt % 16;
          s[hh][r] = mask1<64 * (hh >> 1) + 16 * (hh & 1) + r>(s[hh][r], i0, wd, ninf);
        }, std::make_integer_sequence<int, 64>{});
      }
      float mt[4];
#pragma unroll
      for (int hh = 0; hh < 4; ++hh) {
        float x = max3f(s[hh][0], s[hh][1], s[hh][2]);
#pragma unroll
        for (int r = 3; r < 15; r += 2) x = max3f(x, s[hh][r], s[hh][r + 1]);
        mt[hh] = max3f(x, s[hh][15], s[hh][15]);
      }
      const float mx = xhalf_max(max3f(mt[0], mt[1], max3f(mt[2], mt[3], mt[3])));
      const float m_new = max3f(m_run, mx * c2, mx * c2);
      const float m_use = (m_new == -__builtin_inff()) ? 0.0f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      m_run = m_new;
      const float moff = m_use - kLog2PMax;
      i32x8 pop[2];
      float ps[4] = {-0.0f, -0.0f, -0.0f, -0.0f};
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        int pw[8];
#pragma unroll
        for (int wd = 0; wd < 8; ++wd) {
          const int hh = 2 * m + (wd >> 2);
          const int r = 4 * (wd & 3);
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hh][r + 0], c2, -moff));
          const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hh][r + 1], c2, -moff));
          const float p2 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hh][r + 2], c2, -moff));
          const float p3 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hh][r + 3], c2, -moff));
          ps[wd & 3] += (p0 + p1) + (p2 + p3);
          pw[wd] = (int)pack4_e4m3(p0, p1, p2, p3);
        }
        pop[m] = i32x8{pw[0], pw[1], pw[2], pw[3], pw[4], pw[5], pw[6], pw[7]};
        // qop is step i + 1's Q^T: at a task's last tile it takes the next
        // task's rows before step i + 1's S^T goes out
        if (m == 0 && ends_task) {
          if constexpr (Q16) {
            qcodes(qop, qnraw);
            load_qraw(qnraw, first + (int64_t)min(t + 2, ntw - 1) * kWsWaves);
          } else {
#pragma unroll
            for (int ks = 0; ks < G::KSTEPS; ++ks) qop[ks] = qnext[ks];
            load_q(qnext, first + (int64_t)min(t + 2, ntw - 1) * kWsWaves);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      const float psum = (ps[0] + ps[1]) + (ps[2] + ps[3]);
      // the scores are consumed: step i + 1's S^T into them (issued after
      // the last step too, on valid operands, and never read: a conditional
      // issue would keep the consumed scores live)
      __builtin_amdgcn_s_setprio(1);
      s_pair(jn, 0, qop);
      s_pair(jn, 2, qop);
      __builtin_amdgcn_sched_barrier(0);
      // P.V: V^T operands read through a ring two MFMAs ahead (all eight at
      // once would hold 64 registers); the first tile of a task starts O^T
      // from the product, the others rescale it first
      constexpr int NP = 2 * G::ETILES;
      auto vaddr = [&](int u) {
        return vb + (uint32_t)(32 * (u % G::ETILES) * VP + j * kBlockN + 64 * (u / G::ETILES));
      };
      auto pv = [&](auto first_c) __attribute__((always_inline)) {
        constexpr bool FIRST = decltype(first_c)::value;
        i32x8 ring[3];
        ring[0] = lds_op(vaddr(0));
        ring[1] = lds_op(vaddr(1));
#pragma unroll
        for (int u = 0; u < NP; ++u) {
          if (u + 2 < NP) ring[(u + 2) % 3] = lds_op(vaddr(u + 2));
          const int e = u % G::ETILES, m = u / G::ETILES;
          acc[e] = mfma_32x32x64(ring[u % 3], pop[m], FIRST && m == 0 ? f32x16{} : acc[e]);
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      if (j == 0) {
        l_run = psum;
        pv(std::true_type{});
      } else {
        l_run = l_run * alpha + psum;
        if (__any(alpha != 1.0f)) {
#pragma unroll
          for (int e = 0; e < G::ETILES; ++e)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[e][r] *= alpha;
        }
        pv(std::false_type{});
      }
      __builtin_amdgcn_s_setprio(0);
      if (ends_task) {
        const int64_t task = first + (int64_t)t * kWsWaves;
        const int q = (int)(task - (int64_t)bh * nq) * 32 + lq;
        store_o_rows<D, OUT>(a, acc, v_scale / xhalf_sum(l_run), b, h, q, lg);
      }
    }
    seg = seg_end;
    __syncthreads();   // every wave is done with this head's K/V^T
  }
}

// Whether the plain launch runs attn_kvres_kernel: unmasked, one key range,
// head dim 64 or 128, the key range resident in LDS, and a shape whose
// 256-row blocks would otherwise stream through multi-block workgroups.
inline bool kvres_applies(const AttnArgs& a, int D) {
  if (a.mask != RP_MASK_NONE || a.kv_splits != 1 || a.qb_begin != 0) return false;
  if (D != 64 && D != 128) return false;
  const int n_kb = (a.Skv + kBlockN - 1) / kBlockN;
  if (n_kb > (D == 128 ? KvGeo<128>::MAX_TILES : KvGeo<64>::MAX_TILES)) return false;
  return multi_block_plan(a, D) > 1;
}

template <int D>
int launch_kvres(const AttnArgs& base, int out_dtype, hipStream_t st, int cus) {
  AttnArgs a = base;
  a.D = D;
  const int64_t ntask = (int64_t)a.B * a.H * ((a.Sq + 31) / 32);
  const int64_t want = cus > 0 ? cus : kCUs;
  const int grid = (int)(ntask < want ? ntask : want);
  const int kind = out_kind(out_dtype);
  if (a.q16 != nullptr) {
    if (kind == kOutF32)
      hipLaunchKernelGGL((attn_kvres_kernel<D, kOutF32, true>), dim3(grid), dim3(512), 0, st, a);
    else if (kind == kOutF16)
      hipLaunchKernelGGL((attn_kvres_kernel<D, kOutF16, true>), dim3(grid), dim3(512), 0, st, a);
    else
      hipLaunchKernelGGL((attn_kvres_kernel<D, kOutBf16, true>), dim3(grid), dim3(512), 0, st, a);
  } else if (kind == kOutF32) {
    hipLaunchKernelGGL((attn_kvres_kernel<D, kOutF32, false>), dim3(grid), dim3(512), 0, st, a);
  } else if (kind == kOutF16) {
    hipLaunchKernelGGL((attn_kvres_kernel<D, kOutF16, false>), dim3(grid), dim3(512), 0, st, a);
  } else {
    hipLaunchKernelGGL((attn_kvres_kernel<D, kOutBf16, false>), dim3(grid), dim3(512), 0, st, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    rp_set_error("attn: launch failed: %s", hipGetErrorString(e));
    return RP_ERR_LAUNCH;
  }
  return RP_OK;
}

}  // namespace
}  // namespace rp

using namespace rp;

namespace {

// Argument checks shared by the attention entry points; fills `a`.
int attn_setup(AttnArgs& a, const uint8_t* q8, const uint8_t* k8, const uint8_t* vt8, int64_t ldv,
               const float* q_scale, const float* k_scale, const float* v_scale,
               int scale_stride, float sm_scale, void* out, int out_dtype, int64_t osb,
               int64_t osh, int64_t oss, int B, int H, int Sq, int Skv, int D, int mask,
               int prefix_len, int suffix_len) {
  if (!q8 || !k8 || !vt8 || !q_scale || !k_scale || !v_scale || !out) {
    rp_set_error("attn: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0) {
    rp_set_error("attn: non-positive shape B=%d H=%d Sq=%d Skv=%d", B, H, Sq, Skv);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (D != 32 && D != 64 && D != 128 && D != 256) {
    rp_set_error("attn: head dim %d not in {32, 64, 128, 256}", D);
    return RP_ERR_UNSUPPORTED;
  }
  if (ldv < Skv || ldv % kBlockN != 0) {
    rp_set_error("attn: ldv=%lld must be a multiple of %d and >= Skv=%d", (long long)ldv,
                 kBlockN, Skv);
    return RP_ERR_INVALID_ARGUMENT;
  }
  // the row max is taken over the raw dot products and scaled afterwards,
  // which is the max of the scaled scores only for a non-negative factor
  if (!(sm_scale >= 0.0f) || sm_scale == __builtin_inff()) {
    rp_set_error("attn: sm_scale=%g must be finite and >= 0", (double)sm_scale);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (scale_stride != 0 && scale_stride != 1) {
    rp_set_error("attn: scale_stride must be 0 or 1");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (out_dtype != RP_OUT_BF16 && out_dtype != RP_OUT_F32 && out_dtype != RP_OUT_F16) {
    rp_set_error("attn: unknown out_dtype %d", out_dtype);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (mask != RP_MASK_NONE && mask != RP_MASK_CAUSAL && mask != RP_MASK_SHARED_PREFIX) {
    rp_set_error("attn: unknown mask %d", mask);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (mask == RP_MASK_SHARED_PREFIX && (prefix_len < 0 || suffix_len <= 0)) {
    rp_set_error("attn: shared-prefix mask needs prefix_len >= 0 and suffix_len > 0");
    return RP_ERR_INVALID_ARGUMENT;
  }
  const int elem = out_dtype == RP_OUT_F32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(out) % 16) != 0 || (osb * elem) % 16 != 0 ||
      (osh * elem) % 16 != 0 || (oss * elem) % 16 != 0) {
    rp_set_error("attn: out pointer and strides must be 16-byte aligned");
    return RP_ERR_UNSUPPORTED;
  }
  if ((reinterpret_cast<uintptr_t>(q8) | reinterpret_cast<uintptr_t>(k8) |
       reinterpret_cast<uintptr_t>(vt8)) % 16 != 0) {
    rp_set_error("attn: q8/k8/vt8 must be 16-byte aligned");
    return RP_ERR_UNSUPPORTED;
  }
  a = AttnArgs{};
  a.q = q8; a.k = k8; a.vt = vt8;
  a.qs = q_scale; a.ks = k_scale; a.vs = v_scale;
  a.out = out; a.osb = osb; a.osh = osh; a.oss = oss;
  a.ldv = ldv; a.sm_scale = sm_scale; a.scale_stride = scale_stride;
  a.B = B; a.H = H; a.Sq = Sq; a.Skv = Skv;
  a.mask = mask; a.prefix = prefix_len; a.suffix = suffix_len > 0 ? suffix_len : 1;
  a.kv_splits = 1;
  a.split_tiles = (Skv + kBlockN - 1) / kBlockN;
  a.qb_begin = 0;
  a.ws_rows = Sq;
  a.n_main = 0;
  return RP_OK;
}

int attn_run(const AttnArgs& a, int D, int out_dtype, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (D) {
    case 32: return launch_attn<32>(a, out_dtype, st);
    case 64: return launch_attn<64>(a, out_dtype, st);
    case 128: return launch_attn<128>(a, out_dtype, st);
    default: return launch_attn<256>(a, out_dtype, st);
  }
}

}  // namespace

extern "C" int rp_fp8_attn_fwd(const uint8_t* q8, const uint8_t* k8, const uint8_t* vt8,
                               int64_t ldv, const float* q_scale, const float* k_scale,
                               const float* v_scale, int scale_stride, float sm_scale, void* out,
                               int out_dtype, int64_t osb, int64_t osh, int64_t oss, int B, int H,
                               int Sq, int Skv, int D, int mask, int prefix_len, int suffix_len,
                               void* stream) {
  AttnArgs a;
  const int rc = attn_setup(a, q8, k8, vt8, ldv, q_scale, k_scale, v_scale, scale_stride,
                            sm_scale, out, out_dtype, osb, osh, oss, B, H, Sq, Skv, D, mask,
                            prefix_len, suffix_len);
  return rc != RP_OK ? rc : attn_run(a, D, out_dtype, stream);
}

extern "C" int rp_fp8_attn_fwd_wsplit(const uint8_t* q8, const uint8_t* k8, const uint8_t* vt8,
                                      int64_t ldv, const float* q_scale, const float* k_scale,
                                      const float* v_scale, int scale_stride, float sm_scale,
                                      void* out, int out_dtype, int64_t osb, int64_t osh,
                                      int64_t oss, int B, int H, int Sq, int Skv, int D, int mask,
                                      int prefix_len, int suffix_len, int block_m, void* stream) {
  AttnArgs a;
  const int rc = attn_setup(a, q8, k8, vt8, ldv, q_scale, k_scale, v_scale, scale_stride,
                            sm_scale, out, out_dtype, osb, osh, oss, B, H, Sq, Skv, D, mask,
                            prefix_len, suffix_len);
  if (rc != RP_OK) return rc;
  if (block_m != 32 && block_m != 64 && block_m != 128) {
    rp_set_error("attn wave-split: block_m=%d not in {32, 64, 128}", block_m);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (D != 64 && D != 128) {
    rp_set_error("attn wave-split: head dim %d not in {64, 128}", D);
    return RP_ERR_UNSUPPORTED;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  return D == 64 ? launch_wsplit_rows<64>(a, block_m, out_dtype, st)
                 : launch_wsplit_rows<128>(a, block_m, out_dtype, st);
}

extern "C" int rp_fp8_attn_wsplit_plan(int Skv, int block_m, int* split_tiles, int* n_splits) {
  if (!split_tiles || !n_splits || Skv <= 0 ||
      (block_m != 32 && block_m != 64 && block_m != 128)) {
    rp_set_error("attn wave-split plan: bad arguments");
    return RP_ERR_INVALID_ARGUMENT;
  }
  split_plan(Skv, kWsWaves * 32 / block_m, split_tiles, n_splits);
  return RP_OK;
}

extern "C" int rp_fp8_attn_blocks_per_workgroup(int B, int H, int Sq, int Skv, int D, int mask,
                                               int kv_splits) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0 || kv_splits < 1) return 0;
  AttnArgs a{};
  a.B = B; a.H = H; a.Sq = Sq; a.Skv = Skv; a.mask = mask;
  int split_tiles = 0, n_splits = 1;
  split_plan(Skv, kv_splits, &split_tiles, &n_splits);
  a.kv_splits = n_splits;
  a.n_qblocks = (Sq + kBlockM - 1) / kBlockM;
  return multi_block_plan(a, D);
}

extern "C" int rp_fp8_attn_resident_kv(int B, int H, int Sq, int Skv, int D, int mask,
                                       int kv_splits) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0 || kv_splits < 1) return 0;
  AttnArgs a{};
  a.B = B; a.H = H; a.Sq = Sq; a.Skv = Skv; a.mask = mask;
  int split_tiles = 0, n_splits = 1;
  split_plan(Skv, kv_splits, &split_tiles, &n_splits);
  a.kv_splits = n_splits;
  a.n_qblocks = (Sq + kBlockM - 1) / kBlockM;
  return kvres_applies(a, D) ? 1 : 0;
}

extern "C" size_t rp_fp8_attn_workspace_bytes(int B, int H, int Sq, int D, int kv_splits) {
  if (B <= 0 || H <= 0 || Sq <= 0 || D <= 0 || kv_splits <= 1) return 0;
  const size_t rows = (size_t)kv_splits * B * H * Sq;
  const size_t ml = (rows * 2 * sizeof(float) + 255) / 256 * 256;
  return ml + rows * (size_t)D * sizeof(float);
}

// The key-split launch on set-up arguments (rp_fp8_attn_fwd_split).
static int run_split(AttnArgs& a, int B, int H, int Sq, int Skv, int D, int out_dtype,
                     int kv_splits, void* workspace, size_t workspace_bytes, void* stream) {
  if (kv_splits < 1) {
    rp_set_error("attn: kv_splits=%d must be >= 1", kv_splits);
    return RP_ERR_INVALID_ARGUMENT;
  }
  int split_tiles = 0, n_splits = 1;
  split_plan(Skv, kv_splits, &split_tiles, &n_splits);
  if (n_splits > 1) {
    const size_t need = rp_fp8_attn_workspace_bytes(B, H, Sq, D, n_splits);
    if (!workspace || workspace_bytes < need ||
        reinterpret_cast<uintptr_t>(workspace) % 256 != 0) {
      rp_set_error("attn: workspace of %zu bytes (256-byte aligned) needed for %d key splits",
                   need, n_splits);
      return RP_ERR_INVALID_ARGUMENT;
    }
    const size_t rows = (size_t)n_splits * B * H * Sq;
    a.kv_splits = n_splits;
    a.split_tiles = split_tiles;
    a.ws_ml = static_cast<float*>(workspace);
    a.ws_acc = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                        (rows * 2 * sizeof(float) + 255) / 256 * 256);
  }
  return attn_run(a, D, out_dtype, stream);
}

extern "C" int rp_fp8_attn_fwd_split(const uint8_t* q8, const uint8_t* k8, const uint8_t* vt8,
                                     int64_t ldv, const float* q_scale, const float* k_scale,
                                     const float* v_scale, int scale_stride, float sm_scale,
                                     void* out, int out_dtype, int64_t osb, int64_t osh,
                                     int64_t oss, int B, int H, int Sq, int Skv, int D, int mask,
                                     int prefix_len, int suffix_len, int kv_splits,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  AttnArgs a;
  int rc = attn_setup(a, q8, k8, vt8, ldv, q_scale, k_scale, v_scale, scale_stride, sm_scale,
                      out, out_dtype, osb, osh, oss, B, H, Sq, Skv, D, mask, prefix_len,
                      suffix_len);
  if (rc != RP_OK) return rc;
  return run_split(a, B, H, Sq, Skv, D, out_dtype, kv_splits, workspace, workspace_bytes, stream);
}

extern "C" int rp_fp8_attn_balanced_plan(int B, int H, int Sq, int Skv, int D, int mask, int cus,
                                         int* main_blocks, int* splits) {
  if (!main_blocks || !splits) {
    rp_set_error("attn: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  const TailPlan t = tail_plan(B, H, Sq, Skv, D, mask, cus);
  *main_blocks = t.main_blocks;
  *splits = t.splits;
  return RP_OK;
}

// Workspace of rp_fp8_attn_fwd_balanced: the key-split partial results of
// the rows past the unsplit blocks, then 256 bytes for the launch's item
// counter.
static size_t balanced_partials_bytes(const TailPlan& t, int B, int H, int Sq, int Skv, int D) {
  int split_tiles = 0, n_splits = 1;
  split_plan(Skv, t.splits, &split_tiles, &n_splits);
  const size_t n = rp_fp8_attn_workspace_bytes(B, H, Sq - t.main_blocks * kBlockM, D, n_splits);
  return (n + 255) / 256 * 256;
}
static size_t balanced_ws_bytes(const TailPlan& t, int B, int H, int Sq, int Skv, int D) {
  if (t.splits <= 1) return 0;
  return balanced_partials_bytes(t, B, H, Sq, Skv, D) + 256;
}

extern "C" size_t rp_fp8_attn_balanced_workspace_bytes(int B, int H, int Sq, int Skv, int D,
                                                       int mask, void* stream) {
  if (D != 32 && D != 64 && D != 128 && D != 256) return 0;
  return balanced_ws_bytes(tail_plan(B, H, Sq, Skv, D, mask, stream_cus(stream)), B, H, Sq, Skv,
                           D);
}

// The balanced launch on set-up arguments (rp_fp8_attn_fwd_balanced).
static int run_balanced(AttnArgs& a, int B, int H, int Sq, int Skv, int D, int mask,
                        int out_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  const TailPlan t = tail_plan(B, H, Sq, Skv, D, mask, stream_cus(stream));
  if (t.splits <= 1) return attn_run(a, D, out_dtype, stream);
  const size_t need = balanced_ws_bytes(t, B, H, Sq, Skv, D);
  if (!workspace || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 256 != 0) {
    rp_set_error("attn: workspace of %zu bytes (256-byte aligned) needed for the balanced launch "
                 "(rp_fp8_attn_balanced_workspace_bytes)", need);
    return RP_ERR_INVALID_ARGUMENT;
  }
  // one launch: query blocks [0, main_blocks) of every head unsplit, then
  // rows [main_blocks * 256, Sq) of every head key-split; the merge after
  int split_tiles = 0, n_splits = 1;
  split_plan(Skv, t.splits, &split_tiles, &n_splits);
  a.qb_begin = t.main_blocks;
  a.ws_rows = Sq - t.main_blocks * kBlockM;
  a.kv_splits = n_splits;
  a.split_tiles = split_tiles;
  const size_t rows = (size_t)n_splits * B * H * a.ws_rows;
  a.ws_ml = static_cast<float*>(workspace);
  a.ws_acc = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                      (rows * 2 * sizeof(float) + 255) / 256 * 256);
  a.item_counter = reinterpret_cast<unsigned*>(static_cast<char*>(workspace) +
                                               balanced_partials_bytes(t, B, H, Sq, Skv, D));
  return attn_run(a, D, out_dtype, stream);
}

extern "C" int rp_fp8_attn_fwd_balanced(const uint8_t* q8, const uint8_t* k8, const uint8_t* vt8,
                                        int64_t ldv, const float* q_scale, const float* k_scale,
                                        const float* v_scale, int scale_stride, float sm_scale,
                                        void* out, int out_dtype, int64_t osb, int64_t osh,
                                        int64_t oss, int B, int H, int Sq, int Skv, int D,
                                        int mask, int prefix_len, int suffix_len, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  AttnArgs a;
  int rc = attn_setup(a, q8, k8, vt8, ldv, q_scale, k_scale, v_scale, scale_stride, sm_scale,
                      out, out_dtype, osb, osh, oss, B, H, Sq, Skv, D, mask, prefix_len,
                      suffix_len);
  if (rc != RP_OK) return rc;
  return run_balanced(a, B, H, Sq, Skv, D, mask, out_dtype, workspace, workspace_bytes, stream);
}

// Whether the launch a shape resolves to (kv_splits 0: the balanced launch;
// 1: one key range; more: key splits) quantizes Q itself: every launch but
// the multi-block one (short key ranges that are not resident in LDS) and
// the head dim 32 layout.
static bool q16_launch_ok(int B, int H, int Sq, int Skv, int D, int mask, int kv_splits,
                          int cus) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0 || kv_splits < 0) return false;
  if (D != 64 && D != 128 && D != 256) return false;
  int splits = kv_splits;
  if (kv_splits == 0) {
    const TailPlan t = tail_plan(B, H, Sq, Skv, D, mask, cus);
    if (t.splits > 1) return true;    // the mixed launch: one query block per workgroup
    splits = 1;
  }
  AttnArgs a{};
  a.B = B; a.H = H; a.Sq = Sq; a.Skv = Skv; a.mask = mask;
  int split_tiles = 0, n_splits = 1;
  split_plan(Skv, splits, &split_tiles, &n_splits);
  a.kv_splits = n_splits;
  a.n_qblocks = (Sq + kBlockM - 1) / kBlockM;
  if (kvres_applies(a, D)) return true;
  return multi_block_plan(a, D) <= 1;
}

extern "C" int rp_fp8_attn_q16_supported(int B, int H, int Sq, int Skv, int D, int mask,
                                         int kv_splits, void* stream) {
  return q16_launch_ok(B, H, Sq, Skv, D, mask, kv_splits, stream_cus(stream)) ? 1 : 0;
}

extern "C" int rp_fp8_attn_fwd_q16(const void* q, int q_dtype, int64_t qsb, int64_t qsh,
                                   int64_t qss, const uint8_t* k8, const uint8_t* vt8,
                                   int64_t ldv, const float* q_scale, const float* k_scale,
                                   const float* v_scale, int scale_stride, float sm_scale,
                                   void* out, int out_dtype, int64_t osb, int64_t osh,
                                   int64_t oss, int B, int H, int Sq, int Skv, int D, int mask,
                                   int prefix_len, int suffix_len, int kv_splits,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  if (q == nullptr) {
    rp_set_error("attn: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (q_dtype != RP_DTYPE_BF16 && q_dtype != RP_DTYPE_F16) {
    rp_set_error("attn: unknown q_dtype %d", q_dtype);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if ((reinterpret_cast<uintptr_t>(q) % 16) != 0 || qsb % 8 != 0 || qsh % 8 != 0 ||
      qss % 8 != 0) {
    rp_set_error("attn: q and its strides must be 16-byte aligned");
    return RP_ERR_UNSUPPORTED;
  }
  AttnArgs a;
  // q passes the null and alignment checks in place of the codes
  int rc = attn_setup(a, static_cast<const uint8_t*>(q), k8, vt8, ldv, q_scale, k_scale,
                      v_scale, scale_stride, sm_scale, out, out_dtype, osb, osh, oss, B, H, Sq,
                      Skv, D, mask, prefix_len, suffix_len);
  if (rc != RP_OK) return rc;
  if (!q16_launch_ok(B, H, Sq, Skv, D, mask, kv_splits, stream_cus(stream))) {
    rp_set_error("attn: this shape's launch takes Q as codes only "
                 "(rp_fp8_attn_q16_supported)");
    return RP_ERR_UNSUPPORTED;
  }
  a.q = nullptr;
  a.q16 = static_cast<const uint16_t*>(q);
  a.qsb = qsb; a.qsh = qsh; a.qss = qss;
  a.q_dt = q_dtype == RP_DTYPE_F16 ? kInF16 : kInBf16;
  if (kv_splits == 0)
    return run_balanced(a, B, H, Sq, Skv, D, mask, out_dtype, workspace, workspace_bytes, stream);
  return run_split(a, B, H, Sq, Skv, D, out_dtype, kv_splits, workspace, workspace_bytes, stream);
}
