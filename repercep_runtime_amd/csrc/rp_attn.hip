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
// * Matrix core: v_mfma_f32_16x16x128_f8f6f4 (e4m3 x e4m3, fp32 acc).  For
//   one 16x16 tile, lane l holds row/column l%16 of an operand and k-slots
//   [32*(l/16), +32) (32 bytes); the accumulator holds rows 4*(l/16)+r,
//   column l%16, r = 0..3.
// * S^T = K . Q^T instead of S = Q . K^T: the accumulator of S^T puts one
//   query per lane (column l%16) and keys down the rows, which is exactly
//   the B-operand layout the P.V product needs, so P never leaves
//   registers and never round-trips through LDS.  The K operand rows are
//   gathered in a permuted order (row 4g+r of tile t is key 32g+4t+r) so
//   that lane group g ends up owning keys [32g, 32g+32) of the 128-key
//   block in ascending byte order.
// * O^T = V^T . P^T: V^T is the A operand, read as 32 contiguous bytes per
//   lane from the per-head transposed V (layout RP_LAYOUT_BHDS written by
//   the quantizer).  The O^T accumulator again holds one query per lane, so
//   the online-softmax rescale (acc *= alpha) is lane-local.
// * Row statistics: each lane keeps the running max m and a partial row
//   sum for its query over its 32 keys; the max is combined across the 4
//   lanes sharing a query (xor 16, xor 32) each tile, the sums once at the
//   end.
// * Softmax in base 2: exp(x) = exp2(x*log2e); log2e and all dequant
//   factors are folded into one multiplier, and log2(448) into the row
//   offset, so each score costs one FMA + one v_exp_f32 to become the
//   e4m3-ready value p*448.  The rescale of O is skipped for a tile when no
//   row of the wave raised its maximum (alpha == 1 exactly).
// * 4 waves per workgroup, each wave owns QT*16 query rows; K/V tiles of
//   128 keys are double-buffered in LDS (XOR-swizzled 16-byte chunks so the
//   operand reads are bank-conflict free) and prefetched from HBM one tile
//   ahead through registers.
// * Grid: one workgroup per (head, query block), remapped so that the
//   workgroups resident on one XCD (dispatch is round-robin over the 8
//   XCDs) work on the same head and share its K/V through that XCD's L2.

#include "rp_common.h"

#include <stdlib.h>
#include <string.h>

namespace rp {
namespace {

constexpr int kBlockN = 128;  // keys per tile = K depth of the P.V MFMA
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLog2PMax = 8.807354922057604f;  // log2(448)

struct AttnArgs {
  const uint8_t* q;
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
  int n_qblocks;
  int n_work;
};

__device__ __forceinline__ f32x4 mfma_16x16x128(const i32x8& a, const i32x8& b, const f32x4& c) {
  // cbsz = blgp = 0: both operands OCP e4m3; scale operands 0 select the
  // unscaled instruction.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ i32x8 cat8(const i32x4& lo, const i32x4& hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ float max3f(float a, float b, float c) {
  return __builtin_fmaxf(a, __builtin_fmaxf(b, c));
}

template <int D, int NW>
struct Geo {
  static constexpr int THREADS = NW * kWave;
  static constexpr int KCH = D / 16;                 // 16-byte chunks per K row
  static constexpr int ETILES = D / 16;              // 16-row tiles of O^T
  static constexpr int K_BYTES = kBlockN * D;
  static constexpr int V_BYTES = D * kBlockN;
  static constexpr int STAGE = K_BYTES + V_BYTES;
  static constexpr int K_LOADS = K_BYTES / 16 / THREADS;
  static constexpr int V_LOADS = V_BYTES / 16 / THREADS;
  static_assert(D == 64 || D == 128, "head dim");
  static_assert(K_LOADS * 16 * THREADS == K_BYTES, "K tile split");
  static_assert(V_LOADS * 16 * THREADS == V_BYTES, "V tile split");
};

// Chunk swizzles (16-byte granules) for the two LDS tiles.
template <int D>
__device__ __forceinline__ int k_swz(int r) {
  return ((r & 3) | ((r >> 3) & 4)) & (D / 16 - 1);
}
__device__ __forceinline__ int v_swz(int d) { return d & 7; }

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) void* gbl_ptr_t;

// 16 bytes global -> LDS without passing through VGPRs.  `lds_block` must be
// wave-uniform: lane i lands at lds_block + 16*i.
__device__ __forceinline__ void gload_lds16(const void* src, void* lds_block) {
  __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)lds_block, 16, 0, 0);
}

// Per-thread byte offsets of the direct-to-LDS loads of one (K, V^T) tile,
// relative to the tile's first key.  Each wave instruction fills one
// contiguous KiB of LDS, so the XOR swizzle is applied on the global side:
// the lane that lands on physical chunk `phys` of row r fetches logical chunk
// phys ^ swz(r).
template <int D, int NW>
struct TileOffsets {
  uint32_t k[Geo<D, NW>::K_LOADS];  // relative to kh + kv0*D
  uint32_t v[Geo<D, NW>::V_LOADS];  // relative to vh + kv0
  int k_row[Geo<D, NW>::K_LOADS];   // key row of each K load inside the tile
};

template <int D, int NW>
__device__ __forceinline__ TileOffsets<D, NW> tile_offsets(int64_t ldv, int wave, int lane) {
  using G = Geo<D, NW>;
  TileOffsets<D, NW> o;
#pragma unroll
  for (int n = 0; n < G::K_LOADS; ++n) {
    const int p = (n * NW + wave) * kWave + lane;
    const int r = p / G::KCH, phys = p % G::KCH;
    o.k_row[n] = r;
    o.k[n] = (uint32_t)(r * D + ((phys ^ k_swz<D>(r)) << 4));
  }
#pragma unroll
  for (int n = 0; n < G::V_LOADS; ++n) {
    const int p = (n * NW + wave) * kWave + lane;
    const int d = p >> 3, phys = p & 7;
    o.v[n] = (uint32_t)(d * ldv + ((phys ^ v_swz(d)) << 4));
  }
  return o;
}

// Issue tile `kb` into one LDS stage.  K rows past Skv (last tile only)
// re-read the last key -- their scores are masked; V^T is zero-padded to ldv.
template <int D, int NW>
__device__ __forceinline__ void issue_tile(const AttnArgs& a, const uint8_t* kh, const uint8_t* vh,
                                           const TileOffsets<D, NW>& o, int kb, uint8_t* stage,
                                           int wave) {
  using G = Geo<D, NW>;
  const int kv0 = kb * kBlockN;
  const uint8_t* kt = kh + (int64_t)kv0 * D;
  const bool tail = kv0 + kBlockN > a.Skv;
#pragma unroll
  for (int n = 0; n < G::K_LOADS; ++n) {
    uint32_t off = o.k[n];
    if (tail && kv0 + o.k_row[n] >= a.Skv)
      off = off - (uint32_t)((kv0 + o.k_row[n] - (a.Skv - 1)) * D);
    gload_lds16(kt + off, stage + (n * NW + wave) * 1024);
  }
  const uint8_t* vt = vh + kv0;
  uint8_t* vst = stage + G::K_BYTES;
#pragma unroll
  for (int n = 0; n < G::V_LOADS; ++n) gload_lds16(vt + o.v[n], vst + (n * NW + wave) * 1024);
}

__device__ __forceinline__ void wait_vmem_all() {
  // s_waitcnt vmcnt(0): direct-to-LDS loads have landed
  __builtin_amdgcn_s_waitcnt(0x0F70);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const __bf16 a = (__bf16)lo, b = (__bf16)hi;  // v_cvt_pk_bf16_f32, round to nearest even
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// NW waves per workgroup, each owning QT 16-row query tiles; launch bounds
// ask for two waves per SIMD (256 VGPRs each) so one wave's MFMAs overlap
// the other's softmax.
template <int D, int QT, int NW, bool OUT_F32>
__global__ __launch_bounds__(NW * kWave, 8 / NW)
void attn_fwd_kernel(AttnArgs a) {
  using G = Geo<D, NW>;
  constexpr int QROWS = 16 * QT;
  constexpr int BLOCK_M = QROWS * NW;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * G::STAGE];

  // ---- work item (XCD-aware remap of the linear workgroup id)
  const int w = blockIdx.x;
  const int per = a.n_work >> 3, rem = a.n_work & 7;
  const int xcd = w & 7;
  const int L = xcd * per + min(xcd, rem) + (w >> 3);
  const int bh = L / a.n_qblocks;
  const int qb = L - bh * a.n_qblocks;
  const int b = bh / a.H, h = bh - b * a.H;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int li = lane & 15;  // row/column inside a 16x16 tile
  const int lg = lane >> 4;  // k-slot group (32 bytes)

  const int q_block0 = qb * BLOCK_M;
  const int q_wave0 = q_block0 + wave * QROWS;

  const uint8_t* qh = a.q + (int64_t)bh * a.Sq * D;
  const uint8_t* kh = a.k + (int64_t)bh * a.Skv * D;
  const uint8_t* vh = a.vt + (int64_t)bh * D * a.ldv;

  const float q_scale = a.qs[bh * a.scale_stride];
  const float k_scale = a.ks[bh * a.scale_stride];
  const float v_scale = a.vs[bh * a.scale_stride];
  // exp2 domain: s2 = dot * c2 with c2 = sm_scale*q_scale*k_scale*log2(e)
  const float c2 = ((a.sm_scale * q_scale) * k_scale) * kLog2e;

  // ---- key range: causal blocks past the block's last query are skipped
  int n_kb = (a.Skv + kBlockN - 1) / kBlockN;
  if (a.mask == RP_MASK_CAUSAL) {
    const int q_last = min(q_block0 + BLOCK_M, a.Sq) - 1;
    n_kb = min(n_kb, q_last / kBlockN + 1);
  }

  const TileOffsets<D, NW> toff = tile_offsets<D, NW>(a.ldv, wave, lane);
  issue_tile<D, NW>(a, kh, vh, toff, 0, smem, wave);

  // ---- Q^T operand (B operand of S^T), resident for the whole kernel
  i32x8 qop[QT];
#pragma unroll
  for (int u = 0; u < QT; ++u) {
    const int qrow = min(q_wave0 + 16 * u + li, a.Sq - 1);
    if (32 * lg < D) {
      const i32x4* src = reinterpret_cast<const i32x4*>(qh + (int64_t)qrow * D + 32 * lg);
      qop[u] = cat8(src[0], src[1]);
    } else {
      qop[u] = i32x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }

  // ---- online softmax state (per lane: query q_wave0 + 16u + li)
  f32x4 acc[QT][G::ETILES];
  float m_run[QT], l_run[QT];
#pragma unroll
  for (int u = 0; u < QT; ++u) {
    m_run[u] = -__builtin_inff();
    l_run[u] = 0.0f;
#pragma unroll
    for (int e = 0; e < G::ETILES; ++e) acc[u][e] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // K operand row of tile t for this lane: 32*(li>>2) + 4t + (li&3).  Its
  // swizzle reads bits 0-1 and 5 of the row, which 4t (t < 8) never changes.
  const int k_row0 = 32 * (li >> 2) + (li & 3);
  const int k_sw = k_swz<D>(k_row0);
  const bool k_has = 32 * lg < D;
  const int k_off0 = k_row0 * D + (((2 * lg) ^ k_sw) << 4);
  const int k_off1 = k_row0 * D + (((2 * lg + 1) ^ k_sw) << 4);

  wait_vmem_all();
  __syncthreads();

  for (int kb = 0; kb < n_kb; ++kb) {
    const int st = kb & 1;
    if (kb + 1 < n_kb) issue_tile<D, NW>(a, kh, vh, toff, kb + 1, smem + (st ^ 1) * G::STAGE, wave);

    const uint8_t* kl = smem + st * G::STAGE;
    const uint8_t* vl = kl + G::K_BYTES;
    const int kv0 = kb * kBlockN;

    const bool tail = kv0 + kBlockN > a.Skv;
    bool need_mask = tail;
    if (a.mask == RP_MASK_CAUSAL) need_mask |= kv0 + kBlockN - 1 > q_wave0;
    if (a.mask == RP_MASK_SHARED_PREFIX) need_mask |= kv0 + kBlockN > a.prefix;
    const int kvl = kv0 + 32 * lg;  // key of (t, r) is kvl + 4t + r
    const int pre_end = a.mask == RP_MASK_SHARED_PREFIX ? min(a.prefix, a.Skv) : 0;

    i32x8 pop[QT];
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      // ---- S^T tile column block u: s[t][r] = score(query u, key kvl + 4t + r)
      f32x4 s[8];
      // Re-read K per query tile u rather than keeping 8 K operands (64 VGPRs)
      // live across u: the empty asm hides that the address is unchanged.
      // (a 32-bit LDS offset, so the loads stay ds_read_b128)
      int kbu = st * G::STAGE;
      asm volatile("" : "+v"(kbu));
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        i32x8 kop = i32x8{0, 0, 0, 0, 0, 0, 0, 0};
        if (k_has)
          kop = cat8(*reinterpret_cast<const i32x4*>(smem + kbu + k_off0 + 4 * t * D),
                     *reinterpret_cast<const i32x4*>(smem + kbu + k_off1 + 4 * t * D));
        s[t] = mfma_16x16x128(kop, qop[u], f32x4{0.f, 0.f, 0.f, 0.f});
      }
      // Pipeline the scheduler to "2 LDS reads, 1 MFMA" so only a couple of
      // K operands are in flight (each holds 8 VGPRs).
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      }

      // ---- masking: every supported mask is "kv < pre_end, or lo <= kv <= hi"
      // with a per-query window; bitwise predicates, one select per score.
      if (need_mask) {
        const float ninf = -__builtin_inff();
        const int q = q_wave0 + 16 * u + li;
        int lo = 0, hi = a.Skv - 1;
        if (a.mask == RP_MASK_CAUSAL) hi = min(q, hi);
        if (a.mask == RP_MASK_SHARED_PREFIX) {
          lo = a.prefix + q - q % a.suffix;
          hi = min(a.prefix + q, hi);
        }
        const int lo_t = lo - kvl, hi_t = hi - kvl, pe_t = pre_end - kvl;
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int o = 4 * t + r;
            const int vis = ((o >= lo_t) & (o <= hi_t)) | (o < pe_t);
            s[t][r] = vis ? s[t][r] : ninf;
          }
      }

      // ---- online softmax for this lane's query
      float mx = max3f(s[0][0], s[0][1], s[0][2]);
      mx = max3f(mx, s[0][3], s[1][0]);
      mx = max3f(mx, s[1][1], s[1][2]);
      mx = max3f(mx, s[1][3], s[2][0]);
#pragma unroll
      for (int t = 2; t < 8; ++t) {
        if (t > 2) mx = max3f(mx, s[t][0], s[t][1]);
        else mx = __builtin_fmaxf(mx, s[t][1]);
        mx = max3f(mx, s[t][2], s[t][3]);
      }
      mx = __builtin_fmaxf(mx, shfl_xor(mx, 16));
      mx = __builtin_fmaxf(mx, shfl_xor(mx, 32));
      const float m_new = __builtin_fmaxf(m_run[u], mx * c2);
      const float m_use = (m_new == -__builtin_inff()) ? 0.0f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run[u] - m_use);
      m_run[u] = m_new;
      const float moff = m_use - kLog2PMax;
      float ps0 = 0.0f, ps1 = 0.0f;
      int pw[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][0], c2, -moff));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][1], c2, -moff));
        const float p2 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][2], c2, -moff));
        const float p3 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][3], c2, -moff));
        ps0 += p0 + p1;
        ps1 += p2 + p3;
        pw[t] = (int)pack4_e4m3(p0, p1, p2, p3);
      }
      l_run[u] = l_run[u] * alpha + (ps0 + ps1);
      pop[u] = i32x8{pw[0], pw[1], pw[2], pw[3], pw[4], pw[5], pw[6], pw[7]};
      // Materialise P for this query tile here: without this the optimiser
      // sinks every tile's exp/pack into the P.V phase and keeps all S live.
      asm volatile("" : "+v"(pop[u]));
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int e = 0; e < G::ETILES; ++e) acc[u][e] *= alpha;
      }
    }

    // ---- O^T += V^T . P^T  (each V^T operand read once, used for every u)
#pragma unroll
    for (int e = 0; e < G::ETILES; ++e) {
      const int d = 16 * e + li;
      const int sw = v_swz(d);
      const uint8_t* row = vl + d * kBlockN;
      const i32x8 vop = cat8(*reinterpret_cast<const i32x4*>(row + (((2 * lg) ^ sw) << 4)),
                             *reinterpret_cast<const i32x4*>(row + (((2 * lg + 1) ^ sw) << 4)));
#pragma unroll
      for (int u = 0; u < QT; ++u) acc[u][e] = mfma_16x16x128(vop, pop[u], acc[u][e]);
    }
#pragma unroll
    for (int e = 0; e < G::ETILES; ++e) {
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);   // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, QT, 1);  // MFMA
    }

    wait_vmem_all();
    __syncthreads();
  }

  // ---- epilogue: out = acc * v_scale / l  (acc carries P*448, l sums P*448)
#pragma unroll
  for (int u = 0; u < QT; ++u) {
    float l = l_run[u];
    l += shfl_xor(l, 16);
    l += shfl_xor(l, 32);
    const float inv = v_scale / l;
    const int q = q_wave0 + 16 * u + li;
    if (q < a.Sq) {
      const int64_t obase = (int64_t)b * a.osb + (int64_t)h * a.osh + (int64_t)q * a.oss;
#pragma unroll
      for (int e = 0; e < G::ETILES; ++e) {
        const int d = 16 * e + 4 * lg;
        const float o0 = acc[u][e][0] * inv, o1 = acc[u][e][1] * inv;
        const float o2 = acc[u][e][2] * inv, o3 = acc[u][e][3] * inv;
        if constexpr (OUT_F32) {
          *reinterpret_cast<float4*>(static_cast<float*>(a.out) + obase + d) =
              make_float4(o0, o1, o2, o3);
        } else {
          uint2 pk;
          pk.x = pack_bf16x2(o0, o1);
          pk.y = pack_bf16x2(o2, o3);
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + obase + d) = pk;
        }
      }
    }
  }
}

template <int D, int QT, int NW>
int launch_attn(const AttnArgs& base, bool out_f32, hipStream_t st) {
  AttnArgs a = base;
  constexpr int BLOCK_M = 16 * QT * NW;
  a.n_qblocks = (a.Sq + BLOCK_M - 1) / BLOCK_M;
  const int64_t work = (int64_t)a.n_qblocks * a.B * a.H;
  if (work > 0x7fffffff) {
    rp_set_error("attn: grid too large");
    return RP_ERR_UNSUPPORTED;
  }
  a.n_work = (int)work;
  if (out_f32)
    hipLaunchKernelGGL((attn_fwd_kernel<D, QT, NW, true>), dim3(a.n_work), dim3(NW * kWave), 0, st,
                       a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<D, QT, NW, false>), dim3(a.n_work), dim3(NW * kWave), 0,
                       st, a);
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

extern "C" int rp_fp8_attn_fwd(const uint8_t* q8, const uint8_t* k8, const uint8_t* vt8,
                               int64_t ldv, const float* q_scale, const float* k_scale,
                               const float* v_scale, int scale_stride, float sm_scale, void* out,
                               int out_dtype, int64_t osb, int64_t osh, int64_t oss, int B, int H,
                               int Sq, int Skv, int D, int mask, int prefix_len, int suffix_len,
                               void* stream) {
  if (!q8 || !k8 || !vt8 || !q_scale || !k_scale || !v_scale || !out) {
    rp_set_error("attn: null pointer");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0) {
    rp_set_error("attn: non-positive shape B=%d H=%d Sq=%d Skv=%d", B, H, Sq, Skv);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (D != 64 && D != 128) {
    rp_set_error("attn: head dim %d not in {64, 128}", D);
    return RP_ERR_UNSUPPORTED;
  }
  if (ldv < Skv || ldv % kBlockN != 0) {
    rp_set_error("attn: ldv=%lld must be a multiple of %d and >= Skv=%d", (long long)ldv,
                 kBlockN, Skv);
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (scale_stride != 0 && scale_stride != 1) {
    rp_set_error("attn: scale_stride must be 0 or 1");
    return RP_ERR_INVALID_ARGUMENT;
  }
  if (out_dtype != RP_OUT_BF16 && out_dtype != RP_OUT_F32) {
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
  AttnArgs a{};
  a.q = q8; a.k = k8; a.vt = vt8;
  a.qs = q_scale; a.ks = k_scale; a.vs = v_scale;
  a.out = out; a.osb = osb; a.osh = osh; a.oss = oss;
  a.ldv = ldv; a.sm_scale = sm_scale; a.scale_stride = scale_stride;
  a.B = B; a.H = H; a.Sq = Sq; a.Skv = Skv;
  a.mask = mask; a.prefix = prefix_len; a.suffix = suffix_len > 0 ? suffix_len : 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool f32 = out_dtype == RP_OUT_F32;
  const char* cfg = getenv("RP_ATTN_CFG");  // tuning hook: "qt,nw"
  if (cfg && D == 128) {
    if (!strcmp(cfg, "2,4")) return launch_attn<128, 2, 4>(a, f32, st);
    if (!strcmp(cfg, "2,8")) return launch_attn<128, 2, 8>(a, f32, st);
  }
  if (D == 128) return launch_attn<128, 2, 8>(a, f32, st);
  return launch_attn<64, 2, 8>(a, f32, st);
}
