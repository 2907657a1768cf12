// Flash attention forward for gfx950 (CDNA4): bf16 in/out, fp32 online softmax,
// v_mfma_f32_32x32x16_bf16 matrix cores.
//
// Computes O = softmax(Q K^T * scale + key_bias [+ causal]) V per (batch, head),
// the operator `F.scaled_dot_product_attention` performs on the RLDX-1 hot path:
//   * MSAT joint attention, non-causal, additive key-padding mask
//     (rldx/model/modules/action_model/blocks.py:548-585, :836-869);
//   * VLM GQA prefill, causal, query head h reads KV head h / (Hq/Hkv), with the
//     Qwen3-VL q_norm + rotate-half RoPE optionally fused into the Q load
//     (rldx/model/modules/backbone/modeling_qwen3_vl.py:139-176, :356-490;
//     rldx/inference/backbone/llm/engine/kernels/fused_llm_attention.py:379-770).
//
// Design (short sequences: 608 / 1280 tokens, batch 1)
//   * A workgroup has 4 waves = QW query sub-blocks of 32 queries x KW key
//     groups.  KW = 2 (64-query workgroups) doubles the number of workgroups for
//     the short sequences of this path so the grid reaches the 256 CUs; the two
//     key groups walk interleaved key tiles and are merged through LDS at the end.
//   * K and V^T tiles are staged in LDS with coalesced 16-byte loads (global ->
//     VGPR -> LDS, double-buffered: one barrier per tile, the next tile's loads in
//     flight during the current tile's math) and shared by the QW waves of the
//     key group.  Loads use clamped addresses, never per-lane predication, so the
//     compiler keeps exact vmcnt waits.
//   * S^T = K Q^T: A = K rows from LDS, B = Q^T kept in VGPRs for the whole
//     kernel.  Each lane owns one query column, so the online-softmax max / sum /
//     rescale are lane-local (one xor-32 exchange per tile for the max).
//   * O^T = V^T P^T: B = P^T is the exp'd score accumulator packed to bf16 (the
//     accumulator row order permutes the key index inside each group of 16); A
//     = V^T from a pre-transposed copy of V whose keys are stored in that same
//     permuted order, so every operand is one 16-byte LDS read.  The V^T copy is
//     made once per V (by the producing kernel, or by `vt_transpose_kernel`
//     here), not once per query block.
//   * Softmax in the exp2 domain with the scale folded into one FMA; tiles with
//     no masked key skip all masking; the O / l rescale is lazy (the reference
//     max moves only when a tile max exceeds it by more than 2^8), exact up to
//     rounding because softmax is shift-invariant.
//   * P is rounded to bf16 before the P.V product, the same rounding point as
//     the eager CPU flash-attention kernel.
#include "rldx_amd.h"
#include "rldx_common.h"

namespace rldx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazyThreshold = 8.0f;  // log2 units: rescale only when the max grows by > 2^8
constexpr int kXcds = 8;                // MI355X: 8 XCDs x 32 CUs, one L2 per XCD

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* vt;  // V^T, keys permuted within groups of 16, zero-padded to a multiple of 32
  uint16_t* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t vt_sb, vt_sh, vt_sd;
  int64_t o_sb, o_sh, o_ss;
  const float* key_bias;  // [batch, sk] additive (natural-log units) or nullptr
  int64_t kb_sb;
  int hq, hkv, group, sq, sk;
  int num_q_blocks;
  float scale_log2;  // softmax scale * log2(e)
  // fused Q RMSNorm + rotate-half RoPE (Qwen3-VL), used when kQNorm
  const uint16_t* q_norm_w;  // [D] bf16
  const uint16_t* cos;       // [sq, D] bf16
  const uint16_t* sin;       // [sq, D] bf16 (pre-signed if sin_signed)
  int64_t cs_ss;             // row stride of cos/sin
  float eps;
  int sin_signed;
};

__device__ __forceinline__ float bf(uint16_t b) { return bf16_bits_to_f32(b); }

template <int D>
__device__ __forceinline__ void qnorm_rope_operands(bf16x8 (&qreg)[D / 16], const AttnArgs& a, int pos, bool valid) {
  // Lane holds d = 16*ks + 8*g + i (g = lane half).  Row sum: own D/2 values + lane ^ 32.
  // The rotate-half partner of d is d +- D/2, i.e. ks +- D/32 in the same lane.
  constexpr int KS = D / 16;
  const int g = (threadIdx.x & 63) >> 5;
  float x[KS][8];
  float ss = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const u32x4 raw = __builtin_bit_cast(u32x4, qreg[ks]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w = raw[i >> 1];
      x[ks][i] = bf(static_cast<uint16_t>((i & 1) ? (w >> 16) : (w & 0xffffu)));
      ss += x[ks][i] * x[ks][i];
    }
  }
  ss += __shfl_xor(ss, 32, 64);
  float y[KS][8];
  {
#pragma clang fp contract(off)
    const float rinv = 1.0f / __builtin_sqrtf(ss * (1.0f / D) + a.eps);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int d = ks * 16 + g * 8 + i;
        y[ks][i] = round_bf16(bf(a.q_norm_w[d]) * round_bf16(x[ks][i] * rinv));
      }
  }
  const uint16_t* cr = a.cos + static_cast<int64_t>(valid ? pos : 0) * a.cs_ss + g * 8;
  const uint16_t* sr = a.sin + static_cast<int64_t>(valid ? pos : 0) * a.cs_ss + g * 8;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int pks = ks < KS / 2 ? ks + KS / 2 : ks - KS / 2;
    const u32x4 craw = *reinterpret_cast<const u32x4*>(cr + ks * 16);
    const u32x4 sraw = *reinterpret_cast<const u32x4*>(sr + ks * 16);
    u32x4 outraw;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      uint32_t packed = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma clang fp contract(off)
        const int ii = i + h;
        const uint32_t cw = craw[ii >> 1], sw = sraw[ii >> 1];
        const float cv = bf(static_cast<uint16_t>(h ? (cw >> 16) : (cw & 0xffffu)));
        const float sv = bf(static_cast<uint16_t>(h ? (sw >> 16) : (sw & 0xffffu)));
        const float part = y[pks][ii];
        const float rot = (a.sin_signed || ks >= KS / 2) ? part : -part;
        const float t1 = round_bf16(y[ks][ii] * cv);
        const float t2 = round_bf16(rot * sv);
        packed |= static_cast<uint32_t>(f32_to_bf16_bits(t1 + t2)) << (16 * h);
      }
      outraw[i >> 1] = packed;
    }
    qreg[ks] = __builtin_bit_cast(bf16x8, outraw);
  }
}

template <int D, int KW, bool kCausal, bool kBias, bool kQNorm>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(AttnArgs a) {
  constexpr int QW = 4 / KW;             // query sub-blocks (waves) per key group
  constexpr int BMW = 32 * QW;           // queries per workgroup
  constexpr int BNT = KW == 1 ? 64 : 32; // keys per tile
  constexpr int KB = BNT / 32;           // 32-key blocks of S^T per tile
  constexpr int PSTEPS = BNT / 16;       // 16-key MFMA steps of O^T per tile
  constexpr int KSTEPS = D / 16;         // MFMA k-steps over head_dim for S^T
  constexpr int DBLK = D / 32;           // 32-row blocks of O^T
  constexpr int KPITCH = D + 8;          // LDS row pitch of K (elements): conflict-free 16-byte reads
  constexpr int VPITCH = BNT + 8;        // LDS row pitch of V^T (elements)
  constexpr int GT = 256 / KW;           // threads per key group
  constexpr int KCH = D / 8;             // 16-byte chunks per K row
  constexpr int VCH = BNT / 8;           // 16-byte chunks per V^T row
  constexpr int KL = BNT * KCH / GT;     // K chunks per thread per tile
  constexpr int VL = D * VCH / GT;       // V^T chunks per thread per tile
  static_assert(KL >= 1 && VL >= 1 && KL * GT == BNT * KCH && VL * GT == D * VCH, "tile shape");
  constexpr int K_ELEMS = BNT * KPITCH;
  constexpr int V_ELEMS = D * VPITCH;
  constexpr int BUF_BYTES = (K_ELEMS + V_ELEMS) * 2 + BNT * 4;  // one buffer of one key group
  constexpr int MERGE = DBLK * 16 + 2;                           // floats per lane in the merge
  constexpr int MERGE_BYTES = KW > 1 ? QW * 64 * MERGE * 4 : 0;
  constexpr int TILE_BYTES = KW * 2 * BUF_BYTES;
  constexpr int LDS_BYTES = TILE_BYTES > MERGE_BYTES ? TILE_BYTES : MERGE_BYTES;
  __shared__ __attribute__((aligned(16))) unsigned char smem[LDS_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int kg = wave / QW;  // key group of this wave
  const int qw = wave % QW;  // query sub-block of this wave
  const int gt = tid - kg * GT;

  // XCD-aware work mapping.  Workgroups are dispatched round-robin over the 8
  // XCDs (workgroup i runs on XCD i % 8), each with its own L2.  Work items are
  // ordered (batch, head, query block) — heads sharing a KV head are adjacent —
  // and cut into 8 contiguous ranges, one per XCD, so the K/V of a head is
  // fetched into a single L2 and reused there by all of its query blocks.
  int qb, h, b;
  {
    const int total = static_cast<int>(gridDim.x);
    const int i = static_cast<int>(blockIdx.x);
    const int per = total / kXcds, rem = total % kXcds;
    const int xcd = i % kXcds, k = i / kXcds;
    const int p = xcd < rem ? xcd * (per + 1) + k : rem * (per + 1) + (xcd - rem) * per + k;
    const int nqb = a.num_q_blocks;
    const int qi = p % nqb;
    qb = kCausal ? nqb - 1 - qi : qi;  // causal: longest query blocks first on each XCD
    h = (p / nqb) % a.hq;
    b = p / (nqb * a.hq);
  }
  const int hk = h / a.group;

  const uint16_t* kbase = a.k + b * a.k_sb + hk * a.k_sh;
  const uint16_t* vtbase = a.vt + b * a.vt_sb + hk * a.vt_sh;
  const float* bias = kBias ? a.key_bias + b * a.kb_sb : nullptr;

  // ---- Q^T operand: lane holds query l32 of this wave's sub-block, d-chunk (2*ks + g) ----
  // Global loads use clamped, always-valid addresses (no per-lane predication), so the
  // loop stays branch-free around its loads and vmcnt accounting stays precise.
  const int q_first = qb * BMW + qw * 32;
  const int q_idx = q_first + l32;
  const bool q_valid = q_idx < a.sq;
  bf16x8 qreg[KSTEPS];
  {
    const uint16_t* qrow = a.q + b * a.q_sb + h * a.q_sh + static_cast<int64_t>(min(q_idx, a.sq - 1)) * a.q_ss + g * 8;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
      qreg[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(qrow + ks * 16));
    if constexpr (kQNorm) qnorm_rope_operands<D>(qreg, a, q_idx, q_valid);
  }

  const int k_end = kCausal ? min(a.sk, min(a.sq, qb * BMW + BMW)) : a.sk;
  const int ntiles = (k_end + BNT - 1) / BNT;
  const int iters = (ntiles + KW - 1) / KW;  // tiles per key group (group kg takes tiles kg, kg+KW, ...)
  const int last_key = a.sk - 1;

  // ---- global -> register staging of one tile of this key group (coalesced 16-byte loads) ----
  u32x4 kreg[KL], vreg[VL];
  float breg = 0.f;
  auto fetch = [&](int t) {
    const int k0 = t * BNT;
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const int c = i * GT + gt;
      const int key = min(k0 + c / KCH, last_key);  // keys past the end are masked in the softmax
      kreg[i] = *reinterpret_cast<const u32x4*>(kbase + static_cast<int64_t>(key) * a.k_ss + (c % KCH) * 8);
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int c = i * GT + gt;
      vreg[i] = *reinterpret_cast<const u32x4*>(vtbase + static_cast<int64_t>(c / VCH) * a.vt_sd + k0 + (c % VCH) * 8);
    }
    if constexpr (kBias) breg = bias[min(k0 + (gt % BNT), last_key)] * kLog2e;
  };
  auto stash = [&](int buf) {
    unsigned char* base = smem + (kg * 2 + buf) * BUF_BYTES;
    uint16_t* Ks = reinterpret_cast<uint16_t*>(base);
    uint16_t* Vs = Ks + K_ELEMS;
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const int c = i * GT + gt;
      *reinterpret_cast<u32x4*>(&Ks[(c / KCH) * KPITCH + (c % KCH) * 8]) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int c = i * GT + gt;
      *reinterpret_cast<u32x4*>(&Vs[(c / VCH) * VPITCH + (c % VCH) * 8]) = vreg[i];
    }
    if (kBias && gt < BNT) reinterpret_cast<float*>(Vs + V_ELEMS)[gt] = breg;
  };

  floatx16 oacc[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) oacc[i] = floatx16{};
  float m_ref = -__builtin_inff();  // reference max (log2 units) used for exp
  float l_part = 0.f;
  const float c = a.scale_log2;

  // prologue: tile kg -> LDS buffer 0, tile kg+KW -> registers
  const int t_last = ntiles > 0 ? ntiles - 1 : 0;
  fetch(min(kg, t_last));
  stash(0);
  __syncthreads();
  fetch(min(kg + KW, t_last));

  for (int it = 0; it < iters; ++it) {
    const int t = it * KW + kg;
    const int buf = it & 1;
    const int k0 = t * BNT;
    // a wave with no tile (ragged split) or whose queries all precede the tile has nothing to do
    const bool active = (t < ntiles) && !(kCausal && k0 > q_first + 31);
    if (active) {
      const uint16_t* Ks = reinterpret_cast<const uint16_t*>(smem + (kg * 2 + buf) * BUF_BYTES);
      const uint16_t* Vs = Ks + K_ELEMS;
      const float* bs = reinterpret_cast<const float*>(Vs + V_ELEMS);
      // ---- S^T = K Q^T ----
      floatx16 sacc[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const uint16_t* krow = &Ks[(kb * 32 + l32) * KPITCH + g * 8];
        floatx16 sa = floatx16{}, sb = floatx16{};
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ks += 2) {
          sa = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(krow + ks * 16)), qreg[ks], sa, 0, 0, 0);
          sb = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(krow + ks * 16 + 16)), qreg[ks + 1], sb, 0,
              0, 0);
        }
        sacc[kb] = sa + sb;
      }
      // ---- softmax (log2 domain, lane = one query) ----
      bool edge = (k0 + BNT > a.sk) || (kCausal && k0 + BNT - 1 > q_first);
      if (kBias) edge = edge || __any(bs[lane % BNT] != 0.f);
      float mt = -__builtin_inff();
      if (!edge) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int j = 0; j < 16; ++j) mt = fmaxf(mt, sacc[kb][j]);
        mt *= c;
      } else {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int kl = kb * 32 + 8 * (j >> 2) + 4 * g + (j & 3);
            const int key = k0 + kl;
            float s = kBias ? __builtin_fmaf(sacc[kb][j], c, bs[kl]) : sacc[kb][j] * c;
            bool ok = key < a.sk;
            if (kCausal) ok = ok && (key <= q_idx);
            s = ok ? s : -__builtin_inff();
            sacc[kb][j] = s;
            mt = fmaxf(mt, s);
          }
      }
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      const bool need = mt > m_ref + kLazyThreshold;
      if (__any(need)) {
        const float new_ref = need ? mt : m_ref;
        const float alpha = (m_ref == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(m_ref - new_ref);
        m_ref = new_ref;
        l_part *= alpha;
#pragma unroll
        for (int db = 0; db < DBLK; ++db) oacc[db] *= alpha;
      }
      const float m_use = (m_ref == -__builtin_inff()) ? 0.f : m_ref;
      float psum = 0.f;
      if (!edge) {
        const float nm = -m_use;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][j], c, nm));
            sacc[kb][j] = p;
            psum += p;
          }
      } else {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const float p = __builtin_amdgcn_exp2f(sacc[kb][j] - m_use);
            sacc[kb][j] = p;
            psum += p;
          }
      }
      l_part += psum;
      // ---- O^T += V^T P^T, 16-key steps ----
#pragma unroll
      for (int s = 0; s < PSTEPS; ++s) {
        floatx8 pv;
#pragma unroll
        for (int i = 0; i < 8; ++i) pv[i] = sacc[s >> 1][(s & 1) * 8 + i];
        const bf16x8 pop = __builtin_convertvector(pv, bf16x8);
#pragma unroll
        for (int db = 0; db < DBLK; ++db) {
          const u32x4 vv = *reinterpret_cast<const u32x4*>(&Vs[(db * 32 + l32) * VPITCH + s * 16 + g * 8]);
          oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vv), pop, oacc[db], 0, 0, 0);
        }
      }
    }
    // next tile of this group: registers -> the other LDS buffer, then prefetch the one after
    if (it + 1 < iters) {
      stash(buf ^ 1);
      __syncthreads();
      fetch(min(t + 2 * KW, t_last));
    }
  }

  // ---- merge key groups through LDS (group 1 hands its partial state to group 0) ----
  if constexpr (KW > 1) {
    __syncthreads();
    float* mb = reinterpret_cast<float*>(smem) + qw * (64 * MERGE);
    if (kg == 1) {
#pragma unroll
      for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) mb[(db * 16 + j) * 64 + lane] = oacc[db][j];
      mb[(DBLK * 16) * 64 + lane] = m_ref;
      mb[(DBLK * 16 + 1) * 64 + lane] = l_part;
    }
    __syncthreads();
    if (kg != 0) return;
    const float m1 = mb[(DBLK * 16) * 64 + lane];
    const float l1 = mb[(DBLK * 16 + 1) * 64 + lane];
    const float m = fmaxf(m_ref, m1);
    const float a0 = (m_ref == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(m_ref - m);
    const float a1 = (m1 == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(m1 - m);
    l_part = l_part * a0 + l1 * a1;
#pragma unroll
    for (int db = 0; db < DBLK; ++db)
#pragma unroll
      for (int j = 0; j < 16; ++j) oacc[db][j] = oacc[db][j] * a0 + mb[(db * 16 + j) * 64 + lane] * a1;
  }

  // ---- normalise and store: lane holds query l32, d = 32db + 8jj + 4g + (0..3) ----
  const float l_tot = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (q_valid) {
    uint16_t* orow = a.o + b * a.o_sb + h * a.o_sh + static_cast<int64_t>(q_idx) * a.o_ss;
#pragma unroll
    for (int db = 0; db < DBLK; ++db) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int d = db * 32 + jj * 8 + g * 4;
        uint2 w;
        w.x = static_cast<uint32_t>(f32_to_bf16_bits(oacc[db][jj * 4 + 0] * inv)) |
              (static_cast<uint32_t>(f32_to_bf16_bits(oacc[db][jj * 4 + 1] * inv)) << 16);
        w.y = static_cast<uint32_t>(f32_to_bf16_bits(oacc[db][jj * 4 + 2] * inv)) |
              (static_cast<uint32_t>(f32_to_bf16_bits(oacc[db][jj * 4 + 3] * inv)) << 16);
        *reinterpret_cast<uint2*>(orow + d) = w;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// V [B, H, Sk, D] -> V^T [B, H, D, Skp] with keys permuted inside each group of
// 16 (the P^T accumulator order) and zero padding up to Skp (multiple of 64).
// One workgroup per (32-key block, head, batch), transposed through LDS.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void vt_transpose_kernel(const uint16_t* __restrict__ v, int64_t v_sb, int64_t v_sh,
                                                           int64_t v_ss, uint16_t* __restrict__ vt, int64_t vt_sb,
                                                           int64_t vt_sh, int64_t vt_sd, int sk) {
  constexpr int PITCH = D + 8;
  constexpr int CH = D / 8;  // 16-byte chunks per V row
  __shared__ __attribute__((aligned(16))) uint16_t tile[32 * PITCH];
  const int k0 = blockIdx.x * 32;
  const uint16_t* src = v + blockIdx.z * v_sb + blockIdx.y * v_sh;
  uint16_t* dst = vt + blockIdx.z * vt_sb + blockIdx.y * vt_sh + k0;
  for (int c = threadIdx.x; c < 32 * CH; c += 256) {
    const int r = c / CH, col = (c % CH) * 8;
    const int key = k0 + r;
    u32x4 val = key < sk ? *reinterpret_cast<const u32x4*>(src + static_cast<int64_t>(key) * v_ss + col)
                         : u32x4{0, 0, 0, 0};
    *reinterpret_cast<u32x4*>(&tile[r * PITCH + col]) = val;
  }
  __syncthreads();
  for (int c = threadIdx.x; c < D * 4; c += 256) {
    const int d = c >> 2, q = c & 3;  // output row d, 8-position chunk q of the 32-key block
    u32x4 out;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      uint32_t w = 0;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int p = q * 8 + i + hh;            // position in the block
        const int gp = (p & 15) >> 3, ip = p & 7;  // lane half / element inside the 16-group
        const int key = (p & ~15) + (ip < 4 ? 4 * gp + ip : 8 + 4 * gp + (ip - 4));
        w |= static_cast<uint32_t>(tile[key * PITCH + d]) << (16 * hh);
      }
      out[i >> 1] = w;
    }
    *reinterpret_cast<u32x4*>(dst + static_cast<int64_t>(d) * vt_sd + q * 8) = out;
  }
}

template <int D, int KW, bool kQNorm>
hipError_t launch_attn_d(const AttnArgs& a, int batch, bool causal, bool has_bias, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>(a.num_q_blocks) * a.hq * batch);
  dim3 block(256);
  if (causal) {
    if (has_bias)
      hipLaunchKernelGGL((attn_fwd_kernel<D, KW, true, true, kQNorm>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((attn_fwd_kernel<D, KW, true, false, kQNorm>), grid, block, 0, stream, a);
  } else {
    if (has_bias)
      hipLaunchKernelGGL((attn_fwd_kernel<D, KW, false, true, kQNorm>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((attn_fwd_kernel<D, KW, false, false, kQNorm>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

// Two key groups (64-query workgroups) unless one group already gives >= 2
// workgroups per CU (then 128-query workgroups keep K/V reuse per LDS tile high).
int choose_kw(int64_t sq, int64_t heads_x_batch) {
  return ((sq + 127) / 128) * heads_x_batch >= 512 ? 1 : 2;
}

template <bool kQNorm>
hipError_t launch_attn(AttnArgs a, int64_t head_dim, int batch, bool causal, bool has_bias, hipStream_t stream) {
  const int kw = choose_kw(a.sq, static_cast<int64_t>(a.hq) * batch);
  const int bm = kw == 1 ? 128 : 64;
  a.num_q_blocks = (a.sq + bm - 1) / bm;
  if (head_dim == 128)
    return kw == 1 ? launch_attn_d<128, 1, kQNorm>(a, batch, causal, has_bias, stream)
                   : launch_attn_d<128, 2, kQNorm>(a, batch, causal, has_bias, stream);
  return kw == 1 ? launch_attn_d<64, 1, kQNorm>(a, batch, causal, has_bias, stream)
                 : launch_attn_d<64, 2, kQNorm>(a, batch, causal, has_bias, stream);
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int64_t round_up64(int64_t x) { return (x + 63) / 64 * 64; }

// Shared validation of the q/k/o side; V^T validated by the callers.
hipError_t check_qko(const void* q, const void* k, void* o, int64_t batch, int64_t q_heads, int64_t kv_heads,
                     int64_t seq_q, int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
                     const int64_t* k_strides, const int64_t* o_strides) {
  if (head_dim != 64 && head_dim != 128) return hipErrorInvalidValue;
  if (batch < 0 || q_heads < 0 || kv_heads <= 0 || seq_q < 0 || seq_k < 0) return hipErrorInvalidValue;
  if (q_heads % kv_heads != 0) return hipErrorInvalidValue;
  if (!q_strides || !k_strides || !o_strides) return hipErrorInvalidValue;
  if (batch == 0 || q_heads == 0 || seq_q == 0) return hipSuccess;
  if (seq_k == 0) return hipErrorInvalidValue;  // softmax over an empty key set is undefined
  if (!q || !k || !o) return hipErrorInvalidValue;
  if (!a16(q) || !a16(k) || reinterpret_cast<uintptr_t>(o) % 8) return hipErrorInvalidValue;
  for (int i = 0; i < 3; ++i)
    if (q_strides[i] % 8 || k_strides[i] % 8 || o_strides[i] % 4) return hipErrorInvalidValue;
  if (seq_q > (1 << 24) || seq_k > (1 << 30) || q_heads > 65535 || batch > 65535) return hipErrorInvalidValue;
  if (((seq_q + 31) / 32) * q_heads * batch > (int64_t{1} << 31) - 1) return hipErrorInvalidValue;  // 1-D grid
  return hipSuccess;
}

void fill_qko(AttnArgs& a, const void* q, const void* k, void* o, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
              int64_t seq_k, const int64_t* qs, const int64_t* ks, const int64_t* os, const float* key_bias,
              int64_t kb_sb, float scale) {
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.o = static_cast<uint16_t*>(o);
  a.q_sb = qs[0]; a.q_sh = qs[1]; a.q_ss = qs[2];
  a.k_sb = ks[0]; a.k_sh = ks[1]; a.k_ss = ks[2];
  a.o_sb = os[0]; a.o_sh = os[1]; a.o_ss = os[2];
  a.key_bias = key_bias;
  a.kb_sb = kb_sb;
  a.hq = static_cast<int>(q_heads);
  a.hkv = static_cast<int>(kv_heads);
  a.group = static_cast<int>(q_heads / kv_heads);
  a.sq = static_cast<int>(seq_q);
  a.sk = static_cast<int>(seq_k);
  a.scale_log2 = scale * kLog2e;
}

}  // namespace
}  // namespace rldx

using namespace rldx;

extern "C" int64_t rldx_attention_workspace_bytes(int64_t batch, int64_t kv_heads, int64_t seq_k, int64_t head_dim) {
  if (batch < 0 || kv_heads < 0 || seq_k < 0 || head_dim < 0) return -1;
  return batch * kv_heads * head_dim * round_up64(seq_k) * 2;
}

extern "C" hipError_t rldx_v_transpose_bf16(const void* v, const int64_t* v_strides, void* vt,
                                            const int64_t* vt_strides, int64_t batch, int64_t kv_heads,
                                            int64_t seq_k, int64_t head_dim, hipStream_t stream) {
  if (head_dim != 64 && head_dim != 128) return hipErrorInvalidValue;
  if (batch < 0 || kv_heads < 0 || seq_k < 0 || !v_strides || !vt_strides) return hipErrorInvalidValue;
  if (batch == 0 || kv_heads == 0 || seq_k == 0) return hipSuccess;
  if (!v || !vt || !a16(v) || !a16(vt)) return hipErrorInvalidValue;
  for (int i = 0; i < 3; ++i)
    if (v_strides[i] % 8 || vt_strides[i] % 8) return hipErrorInvalidValue;
  if (vt_strides[2] < round_up64(seq_k) || batch > 65535 || kv_heads > 65535) return hipErrorInvalidValue;
  dim3 grid(static_cast<unsigned>(round_up64(seq_k) / 32), static_cast<unsigned>(kv_heads),
            static_cast<unsigned>(batch));
  if (head_dim == 128)
    hipLaunchKernelGGL(vt_transpose_kernel<128>, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(v),
                       v_strides[0], v_strides[1], v_strides[2], static_cast<uint16_t*>(vt), vt_strides[0],
                       vt_strides[1], vt_strides[2], static_cast<int>(seq_k));
  else
    hipLaunchKernelGGL(vt_transpose_kernel<64>, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(v),
                       v_strides[0], v_strides[1], v_strides[2], static_cast<uint16_t*>(vt), vt_strides[0],
                       vt_strides[1], vt_strides[2], static_cast<int>(seq_k));
  return hipGetLastError();
}

extern "C" hipError_t rldx_attention_vt_fwd_bf16(const void* q, const void* k, const void* vt, void* o,
                                                 int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                                                 int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
                                                 const int64_t* k_strides, const int64_t* vt_strides,
                                                 const int64_t* o_strides, const float* key_bias,
                                                 int64_t key_bias_batch_stride, float scale, int32_t causal,
                                                 hipStream_t stream) {
  hipError_t e = check_qko(q, k, o, batch, q_heads, kv_heads, seq_q, seq_k, head_dim, q_strides, k_strides,
                           o_strides);
  if (e != hipSuccess || batch == 0 || q_heads == 0 || seq_q == 0) return e;
  if (!vt || !vt_strides || !a16(vt)) return hipErrorInvalidValue;
  for (int i = 0; i < 3; ++i)
    if (vt_strides[i] % 8) return hipErrorInvalidValue;
  if (vt_strides[2] < round_up64(seq_k)) return hipErrorInvalidValue;
  AttnArgs a{};
  fill_qko(a, q, k, o, q_heads, kv_heads, seq_q, seq_k, q_strides, k_strides, o_strides, key_bias,
           key_bias_batch_stride, scale);
  a.vt = static_cast<const uint16_t*>(vt);
  a.vt_sb = vt_strides[0]; a.vt_sh = vt_strides[1]; a.vt_sd = vt_strides[2];
  return launch_attn<false>(a, head_dim, static_cast<int>(batch), causal != 0, key_bias != nullptr, stream);
}

extern "C" hipError_t rldx_attention_fwd_bf16(const void* q, const void* k, const void* v, void* o, int64_t batch,
                                              int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k,
                                              int64_t head_dim, const int64_t* q_strides,
                                              const int64_t* k_strides, const int64_t* v_strides,
                                              const int64_t* o_strides, const float* key_bias,
                                              int64_t key_bias_batch_stride, float scale, int32_t causal,
                                              void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  hipError_t e = check_qko(q, k, o, batch, q_heads, kv_heads, seq_q, seq_k, head_dim, q_strides, k_strides,
                           o_strides);
  if (e != hipSuccess || batch == 0 || q_heads == 0 || seq_q == 0) return e;
  if (!v || !v_strides || !a16(v)) return hipErrorInvalidValue;
  for (int i = 0; i < 3; ++i)
    if (v_strides[i] % 8) return hipErrorInvalidValue;
  const int64_t need = rldx_attention_workspace_bytes(batch, kv_heads, seq_k, head_dim);
  if (!workspace || workspace_bytes < need || !a16(workspace)) return hipErrorInvalidValue;
  const int64_t skp = round_up64(seq_k);
  const int64_t vts[3] = {kv_heads * head_dim * skp, head_dim * skp, skp};
  e = rldx_v_transpose_bf16(v, v_strides, workspace, vts, batch, kv_heads, seq_k, head_dim, stream);
  if (e != hipSuccess) return e;
  return rldx_attention_vt_fwd_bf16(q, k, workspace, o, batch, q_heads, kv_heads, seq_q, seq_k, head_dim, q_strides,
                                    k_strides, vts, o_strides, key_bias, key_bias_batch_stride, scale, causal,
                                    stream);
}

extern "C" int64_t rldx_llm_fused_attention_workspace_bytes(int64_t seq, int64_t kv_heads, int64_t head_dim) {
  if (seq < 0 || kv_heads < 0 || head_dim < 0) return -1;
  // normalised K [seq, Hkv, D] followed by V^T [Hkv, D, round_up64(seq)]
  return seq * kv_heads * head_dim * 2 + kv_heads * head_dim * round_up64(seq) * 2;
}

extern "C" hipError_t rldx_llm_fused_attention_bf16(const void* qkv, int64_t qkv_row_stride, const void* q_norm_w,
                                                    const void* k_norm_w, const void* cos, const void* sin,
                                                    int64_t cos_row_stride, int32_t sin_is_signed, void* out,
                                                    int64_t out_row_stride, int64_t seq, int64_t q_heads,
                                                    int64_t kv_heads, int64_t head_dim, float eps, void* workspace,
                                                    int64_t workspace_bytes, hipStream_t stream) {
  if (head_dim != 64 && head_dim != 128) return hipErrorInvalidValue;
  if (seq < 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0) return hipErrorInvalidValue;
  if (seq == 0) return hipSuccess;
  if (!qkv || !q_norm_w || !k_norm_w || !cos || !sin || !out || !workspace) return hipErrorInvalidValue;
  if (qkv_row_stride < (q_heads + 2 * kv_heads) * head_dim || qkv_row_stride % 8 || out_row_stride % 8 ||
      out_row_stride < q_heads * head_dim || cos_row_stride < head_dim || cos_row_stride % 8)
    return hipErrorInvalidValue;
  if (workspace_bytes < rldx_llm_fused_attention_workspace_bytes(seq, kv_heads, head_dim))
    return hipErrorInvalidValue;
  if (!a16(qkv) || !a16(out) || !a16(cos) || !a16(sin) || !a16(workspace)) return hipErrorInvalidValue;
  if (seq > (1 << 30) || q_heads > 65535) return hipErrorInvalidValue;
  const uint16_t* base = static_cast<const uint16_t*>(qkv);
  uint16_t* kws = static_cast<uint16_t*>(workspace);  // normalised K, [seq, kv_heads, D]
  uint16_t* vtws = kws + seq * kv_heads * head_dim;    // V^T, [kv_heads, D, round_up64(seq)]
  const int64_t skp = round_up64(seq);
  // 1) K: RMSNorm + rotate-half RoPE into the workspace (Q is done inside the attention kernel)
  const int64_t k_strides[3] = {0, qkv_row_stride, head_dim};
  const int64_t ko_strides[3] = {0, kv_heads * head_dim, head_dim};
  const int64_t zero3[3] = {0, 0, 0};
  const int64_t cs[2] = {0, cos_row_stride};
  hipError_t e = rldx_qk_rmsnorm_rope_half_bf16(nullptr, base + q_heads * head_dim, nullptr, k_norm_w, cos, sin,
                                                nullptr, kws, 1, seq, 0, kv_heads, head_dim, zero3, k_strides, zero3,
                                                ko_strides, cs, eps, sin_is_signed ? RLDX_ROPE_SIN_SIGNED : 0, stream);
  if (e != hipSuccess) return e;
  // 2) V^T of the packed V columns
  const int64_t v_strides[3] = {0, head_dim, qkv_row_stride};
  const int64_t vt_strides[3] = {0, head_dim * skp, skp};
  e = rldx_v_transpose_bf16(base + (q_heads + kv_heads) * head_dim, v_strides, vtws, vt_strides, 1, kv_heads, seq,
                            head_dim, stream);
  if (e != hipSuccess) return e;
  // 3) causal GQA attention, Q normalised in the prologue
  AttnArgs a{};
  const int64_t q_strides[3] = {0, head_dim, qkv_row_stride};
  const int64_t kk_strides[3] = {0, head_dim, kv_heads * head_dim};
  const int64_t o_strides[3] = {0, head_dim, out_row_stride};
  fill_qko(a, base, kws, out, q_heads, kv_heads, seq, seq, q_strides, kk_strides, o_strides, nullptr, 0,
           1.0f / __builtin_sqrtf(static_cast<float>(head_dim)));
  a.vt = vtws;
  a.vt_sb = 0; a.vt_sh = head_dim * skp; a.vt_sd = skp;
  a.q_norm_w = static_cast<const uint16_t*>(q_norm_w);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.cs_ss = cos_row_stride;
  a.eps = eps;
  a.sin_signed = sin_is_signed ? 1 : 0;
  return launch_attn<true>(a, head_dim, 1, true, false, stream);
}
