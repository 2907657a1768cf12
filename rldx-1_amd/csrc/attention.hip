// Flash attention forward for gfx950 (CDNA4): bf16 in/out, fp32 online softmax,
// v_mfma_f32_32x32x16_bf16 matrix cores, K / V^T tiles staged in LDS.
//
// Computes O = softmax(Q K^T * scale + key_bias [+ causal]) V per (batch, head),
// the operator `F.scaled_dot_product_attention` performs on the RLDX-1 hot path:
//   * MSAT joint attention, non-causal, additive key-padding mask
//     (rldx/model/modules/action_model/blocks.py:548-585, :836-869);
//   * VLM GQA prefill, causal, query head h reads KV head h / (Hq/Hkv)
//     (rldx/model/modules/backbone/modeling_qwen3_vl.py:139-176, :404-490).
//
// Work decomposition
//   grid = (query blocks of 128, query heads, batch); 4 waves per group,
//   each wave owns 32 queries.  Keys are walked in tiles of 64.
//   The score tile is computed transposed, S^T = K Q^T (A = K from LDS,
//   B = Q^T kept in VGPRs for the whole kernel), so every lane owns exactly one
//   query column: the running max / sum / rescale of the online softmax are
//   lane-local, with one xor-32 exchange per tile for the max.
//   O is accumulated transposed too, O^T = V^T P^T: P^T leaves the score
//   accumulators already in B-operand order after a bf16 pack (the K-index
//   permutation this implies is mirrored in the V^T LDS layout), and the
//   per-query rescale stays lane-local.
//   P is rounded to bf16 before the P.V product, the same rounding the eager
//   CPU flash-attention kernel applies.
#include "rldx_amd.h"
#include "rldx_common.h"

namespace rldx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128;  // queries per workgroup
constexpr int BN = 64;   // keys per tile
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  const float* key_bias;  // [batch, sk] additive (natural-log units) or nullptr
  int64_t kb_sb;
  int hq, hkv, group, sq, sk;
  int num_q_blocks;
  float scale_log2;  // softmax scale * log2(e)
};

// Position of key k (0..15) inside a 16-key group of the V^T LDS tile, chosen
// so that lane half g of the P^T operand finds its 8 keys {4g..4g+3, 8+4g..8+4g+3}
// contiguous at positions 8g..8g+7.
__device__ __forceinline__ int vt_pos16(int k) {
  const int a = k >> 2;
  const int base = (a == 0) ? 0 : (a == 1) ? 8 : (a == 2) ? 4 : 12;
  return base + (k & 3);
}

template <int D, bool kCausal, bool kBias>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(AttnArgs a) {
  constexpr int KSTEPS = D / 16;     // MFMA k-steps over head_dim for S
  constexpr int DBLK = D / 32;       // 32-row blocks of O^T
  constexpr int KPITCH = D + 8;      // LDS row pitch of K (elements)
  constexpr int VPITCH = BN + 8;     // LDS row pitch of V^T (elements)
  constexpr int KCH = D / 8;         // 16-byte chunks per K/V row
  constexpr int KLOADS = BN * KCH / 256;   // 16-byte K loads per thread per tile
  constexpr int KPT = BN * D / (256 * 8);  // keys per thread in the V transpose (D/32)
  static_assert(KLOADS >= 1 && KPT >= 1, "tile shape");

  __shared__ __attribute__((aligned(16))) uint16_t Ks[BN * KPITCH];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[D * VPITCH];
  __shared__ float bias_s[BN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int g = lane >> 5;

  const int qb = kCausal ? (a.num_q_blocks - 1 - static_cast<int>(blockIdx.x)) : static_cast<int>(blockIdx.x);
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int hk = h / a.group;

  const uint16_t* qbase = a.q + b * a.q_sb + h * a.q_sh;
  const uint16_t* kbase = a.k + b * a.k_sb + hk * a.k_sh;
  const uint16_t* vbase = a.v + b * a.v_sb + hk * a.v_sh;
  uint16_t* obase = a.o + b * a.o_sb + h * a.o_sh;
  const float* bias = kBias ? a.key_bias + b * a.kb_sb : nullptr;

  // ---- Q^T operand: lane holds query (l32) and d-chunk (2*ks + g) ----
  const int q_idx = qb * BM + wave * 32 + l32;
  const bool q_valid = q_idx < a.sq;
  bf16x8 qreg[KSTEPS];
  {
    const uint16_t* qrow = qbase + static_cast<int64_t>(q_valid ? q_idx : 0) * a.q_ss;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      u32x4 raw = q_valid ? *reinterpret_cast<const u32x4*>(qrow + ks * 16 + g * 8) : u32x4{0, 0, 0, 0};
      qreg[ks] = __builtin_bit_cast(bf16x8, raw);
    }
  }

  // ---- key range ----
  int k_end = a.sk;
  if (kCausal) {
    const int last_q = min(a.sq, (qb + 1) * BM) - 1;
    k_end = min(a.sk, last_q + 1);
  }
  const int ntiles = (k_end + BN - 1) / BN;

  // ---- global -> register prefetch of one K/V tile ----
  u32x4 kreg[KLOADS];
  u32x4 vreg[KPT];
  float breg = 0.f;
  const int v_dc = tid % KCH;  // d chunk for V (8 values)
  const int v_kc = tid / KCH;  // key chunk for V (KPT keys)
  auto prefetch = [&](int t) {
    const int k0 = t * BN;
#pragma unroll
    for (int i = 0; i < KLOADS; ++i) {
      const int c = i * 256 + tid;
      const int row = c / KCH, col = (c % KCH) * 8;
      const int key = k0 + row;
      kreg[i] = key < a.sk ? *reinterpret_cast<const u32x4*>(kbase + static_cast<int64_t>(key) * a.k_ss + col)
                           : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int key = k0 + v_kc * KPT + i;
      vreg[i] = key < a.sk ? *reinterpret_cast<const u32x4*>(vbase + static_cast<int64_t>(key) * a.v_ss + v_dc * 8)
                           : u32x4{0, 0, 0, 0};
    }
    if (kBias && tid < BN) {
      const int key = k0 + tid;
      breg = key < a.sk ? bias[key] : 0.f;
    }
  };

  floatx16 oacc[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) oacc[i] = floatx16{};
  float m_run = -__builtin_inff();
  float l_part = 0.f;

  if (ntiles > 0) prefetch(0);

  for (int t = 0; t < ntiles; ++t) {
    const int k0 = t * BN;
    __syncthreads();
    // ---- registers -> LDS: K row-major, V transposed into the permuted key order ----
#pragma unroll
    for (int i = 0; i < KLOADS; ++i) {
      const int c = i * 256 + tid;
      const int row = c / KCH, col = (c % KCH) * 8;
      *reinterpret_cast<u32x4*>(&Ks[row * KPITCH + col]) = kreg[i];
    }
    {
      const uint16_t* ve[KPT];
#pragma unroll
      for (int i = 0; i < KPT; ++i) ve[i] = reinterpret_cast<const uint16_t*>(&vreg[i]);
      const int key0 = v_kc * KPT;                 // first key of this thread (multiple of KPT)
      const int pos = (key0 & ~15) + vt_pos16(key0 & 15);  // KPT consecutive keys stay consecutive
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint16_t* dst = &Vt[(v_dc * 8 + e) * VPITCH + pos];
        if constexpr (KPT == 4) {
          uint2 w;
          w.x = static_cast<uint32_t>(ve[0][e]) | (static_cast<uint32_t>(ve[1][e]) << 16);
          w.y = static_cast<uint32_t>(ve[2][e]) | (static_cast<uint32_t>(ve[3][e]) << 16);
          *reinterpret_cast<uint2*>(dst) = w;
        } else {
          static_assert(KPT == 2, "KPT");
          *reinterpret_cast<uint32_t*>(dst) =
              static_cast<uint32_t>(ve[0][e]) | (static_cast<uint32_t>(ve[1][e]) << 16);
        }
      }
    }
    if (kBias && tid < BN) bias_s[tid] = breg * kLog2e;
    __syncthreads();
    if (t + 1 < ntiles) prefetch(t + 1);

    // ---- S^T = K Q^T for the 64-key tile: two 32x32 blocks ----
    floatx16 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sacc[kb] = floatx16{};
      const uint16_t* krow = &Ks[(kb * 32 + l32) * KPITCH + g * 8];
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        bf16x8 kop = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(krow + ks * 16));
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop, qreg[ks], sacc[kb], 0, 0, 0);
      }
    }

    // ---- scale, mask, online softmax (lane-local: one query per lane) ----
    float mloc = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int kl = kb * 32 + 8 * (j >> 2) + 4 * g + (j & 3);  // key within tile
        const int key = k0 + kl;
        float s = sacc[kb][j] * a.scale_log2;
        if (kBias) s += bias_s[kl];
        bool ok = key < a.sk;
        if (kCausal) ok = ok && (key <= q_idx);
        s = ok ? s : -__builtin_inff();
        sacc[kb][j] = s;
        mloc = fmaxf(mloc, s);
      }
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float m_new = fmaxf(m_run, mloc);
    const float m_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float p = __builtin_amdgcn_exp2f(sacc[kb][j] - m_use);
        sacc[kb][j] = p;
        psum += p;
      }
    }
    l_part = l_part * alpha + psum;
#pragma unroll
    for (int db = 0; db < DBLK; ++db) oacc[db] *= alpha;

    // ---- O^T += V^T P^T, four 16-key steps ----
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int kb = s >> 1;
      const int j0 = (s & 1) * 8;
      floatx8 pv;
#pragma unroll
      for (int i = 0; i < 8; ++i) pv[i] = sacc[kb][j0 + i];
      const bf16x8 pop = __builtin_convertvector(pv, bf16x8);
#pragma unroll
      for (int db = 0; db < DBLK; ++db) {
        const uint16_t* vrow = &Vt[(db * 32 + l32) * VPITCH + s * 16 + g * 8];
        bf16x8 vop = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(vrow));
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop, pop, oacc[db], 0, 0, 0);
      }
    }
  }

  // ---- normalise and store: lane holds query l32, d = 32db + 8jj + 4g + (0..3) ----
  const float l_tot = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (q_valid) {
    uint16_t* orow = obase + static_cast<int64_t>(q_idx) * a.o_ss;
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

template <int D>
hipError_t launch_attn(const AttnArgs& a, int batch, bool causal, bool has_bias, hipStream_t stream) {
  dim3 grid(a.num_q_blocks, a.hq, batch);
  dim3 block(256);
  if (causal) {
    if (has_bias)
      hipLaunchKernelGGL((attn_fwd_kernel<D, true, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((attn_fwd_kernel<D, true, false>), grid, block, 0, stream, a);
  } else {
    if (has_bias)
      hipLaunchKernelGGL((attn_fwd_kernel<D, false, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((attn_fwd_kernel<D, false, false>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace rldx

using namespace rldx;

extern "C" hipError_t rldx_attention_fwd_bf16(const void* q, const void* k, const void* v, void* o, int64_t batch,
                                              int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k,
                                              int64_t head_dim, const int64_t* q_strides,
                                              const int64_t* k_strides, const int64_t* v_strides,
                                              const int64_t* o_strides, const float* key_bias,
                                              int64_t key_bias_batch_stride, float scale, int32_t causal,
                                              hipStream_t stream) {
  if (head_dim != 64 && head_dim != 128) return hipErrorInvalidValue;
  if (batch < 0 || q_heads < 0 || kv_heads <= 0 || seq_q < 0 || seq_k < 0) return hipErrorInvalidValue;
  if (q_heads % kv_heads != 0) return hipErrorInvalidValue;
  if (!q_strides || !k_strides || !v_strides || !o_strides) return hipErrorInvalidValue;
  if (batch == 0 || q_heads == 0 || seq_q == 0) return hipSuccess;
  if (!q || !k || !v || !o) return hipErrorInvalidValue;
  if (!a16(q) || !a16(k) || !a16(v) || !(reinterpret_cast<uintptr_t>(o) % 8 == 0)) return hipErrorInvalidValue;
  for (int i = 0; i < 3; ++i) {
    if (q_strides[i] % 8 || k_strides[i] % 8 || v_strides[i] % 8 || o_strides[i] % 4) return hipErrorInvalidValue;
  }
  if (seq_q > (1 << 30) || seq_k > (1 << 30) || q_heads > 65535 || batch > 65535) return hipErrorInvalidValue;
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<uint16_t*>(o);
  a.q_sb = q_strides[0]; a.q_sh = q_strides[1]; a.q_ss = q_strides[2];
  a.k_sb = k_strides[0]; a.k_sh = k_strides[1]; a.k_ss = k_strides[2];
  a.v_sb = v_strides[0]; a.v_sh = v_strides[1]; a.v_ss = v_strides[2];
  a.o_sb = o_strides[0]; a.o_sh = o_strides[1]; a.o_ss = o_strides[2];
  a.key_bias = key_bias;
  a.kb_sb = key_bias_batch_stride;
  a.hq = static_cast<int>(q_heads);
  a.hkv = static_cast<int>(kv_heads);
  a.group = static_cast<int>(q_heads / kv_heads);
  a.sq = static_cast<int>(seq_q);
  a.sk = static_cast<int>(seq_k);
  a.num_q_blocks = static_cast<int>((seq_q + BM - 1) / BM);
  a.scale_log2 = scale * kLog2e;
  const bool has_bias = key_bias != nullptr;
  if (head_dim == 128) return launch_attn<128>(a, static_cast<int>(batch), causal != 0, has_bias, stream);
  return launch_attn<64>(a, static_cast<int>(batch), causal != 0, has_bias, stream);
}
