// Residual-add + norm row epilogues for gfx950: the block-boundary operators
//   ds::grouped_res_ln      out   = LN(res + proj + bias)                 fp32 sum, one rounding
//   ds::vl_epilogue_ln      new   = ((res + proj_bias) + w3_bias) + w3    bf16 rounding after each add
//                           ln    = LN(new)
//   ss::fused_epilogue_ln   new   = hidden + residual (bf16); ln = LN(new)   (or ln = LN(hidden))
//   rldx_backbone::fused_epilogue_add{2,3}_rmsnorm
//                           new   = (hidden + residual) [+ deepstack]     bf16 rounding after each add
//                           normed = bf16(w * bf16(new * rsqrt(mean(new^2) + eps)))
// LN is LayerNorm without affine: mean and biased variance in fp32 (two passes
// over the row in registers), (x - mean) * (1 / sqrt(var + eps)), one rounding.
//
// Reference kernels: rldx/inference/action_model/double_stream/engine/kernels/
// grouped_res_ln.py:40-148 and vl_epilogue_ln.py:31-125,
// rldx/inference/action_model/single_stream/engine/kernels/ss_epilogue_ln.py:33-143,
// rldx/inference/backbone/llm/engine/kernels/fused_add2_rmsnorm.py:29-83 and
// fused_add3_rmsnorm.py:31-83.  The RMSNorm ops follow the eager arithmetic their
// op files promise (op_fused_epilogue_add2_rmsnorm.py:7-10: the sum is rounded
// to bf16 before the norm, Qwen3VLTextRMSNorm, modeling_qwen3_vl.py:366-371);
// the reference's Triton kernel normalises the unrounded fp32 sum instead, a
// difference of at most one bf16 rounding per element.
//
// Memory-bound and small at the block-boundary shapes (rows of 1536 or 4096
// bf16, a few dozen to a few hundred rows): one workgroup per row so that even
// 18 rows spread over 18 CUs, the whole row in registers, every addend's loads
// in flight together, so every input byte is read once and every output byte
// written once.  All of a row's loads happen before any of its stores (the
// cross-wave reduction is a barrier), so an output may alias an input of the
// same row layout (in-place residual update).  Rows whose width is not a
// multiple of 8 (or unaligned) take a three-pass scalar kernel.
#include "rldx_amd.h"
#include "rldx_common.h"

namespace rldx {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxTerms = 4;
enum { kSumF32 = 0, kSumBf16 = 1 };
enum { kNormLayer = 0, kNormRms = 1 };

struct AddNormGroup {
  const uint16_t* term[kMaxTerms];  // addends, summed in this order
  int64_t term_ld[kMaxTerms];       // row stride in elements; 0 = one vector broadcast over rows
  int nterms;
  const uint16_t* weight;           // RMSNorm weight [dim] (kNormRms)
  uint16_t* sum_out;                // bf16 sum, or nullptr
  int64_t sum_ld;
  uint16_t* norm_out;
  int64_t norm_ld;
  int rows, dim;
  int blocks;                       // workgroups of this group (set by the launcher)
};

struct AddNormArgs {
  AddNormGroup g[2];
  float eps;
};

// One workgroup per row (64-256 threads, whole waves): thread tid holds the
// 8-column chunks tid + nthr j, j < CPT, of the row (dim a multiple of 8,
// 16-byte aligned rows).  Every addend's loads are issued before any
// arithmetic (one memory round trip per row); the row sums are reduced over the
// waves through LDS in a fixed order (deterministic).
template <int CPT, int kSum, int kNorm>
__global__ __launch_bounds__(256) void add_norm_rows_kernel(AddNormArgs a) {
#pragma clang fp contract(off)
  const int blk = static_cast<int>(blockIdx.x);
  const int gi = blk >= a.g[0].blocks ? 1 : 0;
  const AddNormGroup& G = a.g[gi];
  const int row = blk - (gi ? a.g[0].blocks : 0);
  const int tid = static_cast<int>(threadIdx.x), nthr = static_cast<int>(blockDim.x);
  const int lane = tid & 63, wave = tid >> 6, nwaves = nthr >> 6;
  const int dim = G.dim;
  auto col_of = [&](int j) { return 8 * (tid + nthr * j); };

  u32x4 raw[kMaxTerms][CPT];
#pragma unroll
  for (int t = 0; t < kMaxTerms; ++t) {
    if (t < G.nterms) {
      const uint16_t* tp = G.term[t] + static_cast<int64_t>(row) * G.term_ld[t];
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        const int col = col_of(j);
        raw[t][j] = col < dim ? *reinterpret_cast<const u32x4*>(tp + col) : u32x4{0, 0, 0, 0};
      }
    }
  }
  // bf16 sums round each pair of columns with one v_cvt_pk_bf16_f32 (round to
  // nearest even, the rounding of f32_to_bf16_bits for every non-NaN value)
  float v[CPT][8];
#pragma unroll
  for (int j = 0; j < CPT; ++j)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[j][2 * k] = bf16x2_lo(raw[0][j][k]);
      v[j][2 * k + 1] = bf16x2_hi(raw[0][j][k]);
    }
#pragma unroll
  for (int t = 1; t < kMaxTerms; ++t) {
    if (t >= G.nterms) break;
#pragma unroll
    for (int j = 0; j < CPT; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float x0 = v[j][2 * k] + bf16x2_lo(raw[t][j][k]);
        float x1 = v[j][2 * k + 1] + bf16x2_hi(raw[t][j][k]);
        if constexpr (kSum == kSumBf16) {
          const uint32_t r = pack_bf16x2(x0, x1);
          x0 = bf16x2_lo(r);
          x1 = bf16x2_hi(r);
        }
        v[j][2 * k] = x0;
        v[j][2 * k + 1] = x1;
      }
  }

  __shared__ float red[2][4];
  auto row_sum = [&](float x, int slot) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    if (lane == 0) red[slot][wave] = x;
    __syncthreads();
    float s = red[slot][0];
    for (int w = 1; w < nwaves; ++w) s += red[slot][w];
    return s;
  };

  // ---- statistics (out-of-row slots hold 0) ----
  float mean = 0.f, scale;
  if constexpr (kNorm == kNormLayer) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < CPT; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) s += v[j][i];
    mean = row_sum(s, 0) / static_cast<float>(dim);
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < CPT; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = col_of(j) < dim ? v[j][i] - mean : 0.f;
        q += d * d;
      }
    scale = 1.0f / __builtin_sqrtf(row_sum(q, 1) / static_cast<float>(dim) + a.eps);  // 1 / std
  } else {
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < CPT; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) q += v[j][i] * v[j][i];
    scale = 1.0f / __builtin_sqrtf(row_sum(q, 0) / static_cast<float>(dim) + a.eps);  // 1 / rms
  }
  // LN: (x - mean) / std; RMS: bf16(w * bf16(x / rms)) (bf16 tensor product)
  auto normed = [&](float x, float w) {
    if constexpr (kNorm == kNormLayer)
      return (x - mean) * scale;
    else
      return w * bf16x2_lo(pack_bf16x2(x * scale, 0.f));
  };

  // ---- stores ----
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int col = col_of(j);
    if (col >= dim) continue;
    u32x4 w = {0, 0, 0, 0};
    if constexpr (kNorm == kNormRms) w = *reinterpret_cast<const u32x4*>(G.weight + col);
    u32x4 sv, nv;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      sv[k] = pack_bf16x2(v[j][2 * k], v[j][2 * k + 1]);
      nv[k] = pack_bf16x2(normed(v[j][2 * k], bf16x2_lo(w[k])), normed(v[j][2 * k + 1], bf16x2_hi(w[k])));
    }
    if (G.sum_out) *reinterpret_cast<u32x4*>(G.sum_out + static_cast<int64_t>(row) * G.sum_ld + col) = sv;
    *reinterpret_cast<u32x4*>(G.norm_out + static_cast<int64_t>(row) * G.norm_ld + col) = nv;
  }
}

// Any dim / alignment: one wave per row, three passes over the row with the
// sum recomputed from the inputs each time (they stay in L1/L2): mean (LN),
// second moment, then normalise and store.  Stores happen only in the last pass,
// element by element after that element's inputs are read by the same lane, so
// exact aliasing of an output with an input stays safe.
template <int kSum, int kNorm>
__global__ __launch_bounds__(256) void add_norm_rows_scalar_kernel(AddNormArgs a) {
#pragma clang fp contract(off)
  const int blk = static_cast<int>(blockIdx.x);
  const int gi = blk >= a.g[0].blocks ? 1 : 0;
  const AddNormGroup& G = a.g[gi];
  const int row = (blk - (gi ? a.g[0].blocks : 0)) * 4 + (static_cast<int>(threadIdx.x) >> 6);
  if (row >= G.rows) return;
  const int lane = threadIdx.x & 63;
  const int dim = G.dim;
  auto sum_at = [&](int col) {
    float x = 0.f;
    for (int t = 0; t < G.nterms; ++t) {
      const float y = bf16_bits_to_f32(G.term[t][static_cast<int64_t>(row) * G.term_ld[t] + col]);
      if (t == 0)
        x = y;
      else if constexpr (kSum == kSumBf16)
        x = round_bf16(x + y);
      else
        x = x + y;
    }
    return x;
  };
  float mean = 0.f;
  if constexpr (kNorm == kNormLayer) {
    float s = 0.f;
    for (int col = lane; col < dim; col += 64) s += sum_at(col);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    mean = s / static_cast<float>(dim);
  }
  float q = 0.f;
  for (int col = lane; col < dim; col += 64) {
    const float d = sum_at(col) - mean;
    q += d * d;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) q += __shfl_xor(q, o, 64);
  const float scale = 1.0f / __builtin_sqrtf(q / static_cast<float>(dim) + a.eps);
  for (int col = lane; col < dim; col += 64) {
    const float x = sum_at(col);
    float n;
    if constexpr (kNorm == kNormLayer)
      n = (x - mean) * scale;
    else
      n = bf16_bits_to_f32(G.weight[col]) * round_bf16(x * scale);
    if (G.sum_out) G.sum_out[static_cast<int64_t>(row) * G.sum_ld + col] = f32_to_bf16_bits(x);
    G.norm_out[static_cast<int64_t>(row) * G.norm_ld + col] = f32_to_bf16_bits(n);
  }
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool group_vec_ok(const AddNormGroup& G) {
  if (G.dim % 8) return false;
  for (int t = 0; t < G.nterms; ++t)
    if (!a16(G.term[t]) || G.term_ld[t] % 8) return false;
  if (G.weight && !a16(G.weight)) return false;
  if (G.sum_out && (!a16(G.sum_out) || G.sum_ld % 8)) return false;
  return a16(G.norm_out) && G.norm_ld % 8 == 0;
}

template <int kSum, int kNorm>
hipError_t launch_kernel(AddNormArgs& a, int ngroups, bool vec, int max_dim, hipStream_t stream) {
  // vector kernel: one workgroup per row; scalar kernel: one wave per row, 4 rows per workgroup
  int64_t blocks = 0;
  for (int i = 0; i < ngroups; ++i) {
    a.g[i].blocks = vec ? a.g[i].rows : (a.g[i].rows + 3) / 4;
    blocks += a.g[i].blocks;
  }
  if (ngroups == 1) a.g[0].blocks = static_cast<int>(blocks);
  if (blocks > (int64_t{1} << 31) - 1) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(blocks));
  if (!vec) {
    hipLaunchKernelGGL((add_norm_rows_scalar_kernel<kSum, kNorm>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
  }
  const int chunks = max_dim / 8;
  const int cpt = (chunks + 255) / 256;                     // chunks per thread
  const int threads = ((chunks + cpt - 1) / cpt + 63) / 64 * 64;
  const dim3 block(static_cast<unsigned>(threads));
  if (cpt <= 1)
    hipLaunchKernelGGL((add_norm_rows_kernel<1, kSum, kNorm>), grid, block, 0, stream, a);
  else if (cpt <= 2)
    hipLaunchKernelGGL((add_norm_rows_kernel<2, kSum, kNorm>), grid, block, 0, stream, a);
  else if (cpt <= 3)
    hipLaunchKernelGGL((add_norm_rows_kernel<3, kSum, kNorm>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((add_norm_rows_kernel<4, kSum, kNorm>), grid, block, 0, stream, a);
  return hipGetLastError();
}

constexpr int64_t kMaxDim = 8192;

// Validates and launches up to two groups in one launch.
hipError_t launch_add_norm(AddNormGroup* gs, int n, int sum_mode, int norm, float eps, hipStream_t stream) {
  if (!(eps >= 0.f)) return hipErrorInvalidValue;
  AddNormArgs a{};
  a.eps = eps;
  int k = 0, max_dim = 0;
  bool vec = true;
  for (int i = 0; i < n; ++i) {
    AddNormGroup& G = gs[i];
    if (G.rows < 0 || G.dim < 0) return hipErrorInvalidValue;
    if (G.rows == 0) continue;
    if (G.dim == 0 || G.dim > kMaxDim || !G.norm_out) return hipErrorInvalidValue;
    if (G.nterms < 1 || G.nterms > kMaxTerms) return hipErrorInvalidValue;
    for (int t = 0; t < G.nterms; ++t)
      if (!G.term[t]) return hipErrorInvalidValue;
    if (norm == kNormRms && !G.weight) return hipErrorInvalidValue;
    vec = vec && group_vec_ok(G);
    max_dim = G.dim > max_dim ? G.dim : max_dim;
    a.g[k++] = G;
  }
  if (k == 0) return hipSuccess;
  if (sum_mode == kSumF32) {
    if (norm != kNormLayer) return hipErrorInvalidValue;
    return launch_kernel<kSumF32, kNormLayer>(a, k, vec, max_dim, stream);
  }
  if (norm == kNormLayer) return launch_kernel<kSumBf16, kNormLayer>(a, k, vec, max_dim, stream);
  return launch_kernel<kSumBf16, kNormRms>(a, k, vec, max_dim, stream);
}

bool rows_ok(int64_t m, int64_t dim) {
  return m >= 0 && dim >= 0 && m <= (int64_t{1} << 30) && dim <= kMaxDim;
}

AddNormGroup make_group(int64_t m, int64_t dim) {
  AddNormGroup G{};
  G.rows = static_cast<int>(m);
  G.dim = static_cast<int>(dim);
  return G;
}

void add_term(AddNormGroup& G, const void* p, int64_t ld) {
  G.term[G.nterms] = static_cast<const uint16_t*>(p);
  G.term_ld[G.nterms] = ld;
  ++G.nterms;
}

}  // namespace
}  // namespace rldx

using namespace rldx;

extern "C" hipError_t rldx_grouped_res_ln_bf16(const void* sa_res, const void* sa_bias, const void* sa_proj,
                                               void* sa_out, const void* vl_res, const void* vl_bias,
                                               const void* vl_proj, void* vl_out, int64_t m_sa, int64_t m_vl,
                                               int64_t sa_dim, int64_t vl_dim, float eps, hipStream_t stream) {
  if (!rows_ok(m_sa, sa_dim) || !rows_ok(m_vl, vl_dim)) return hipErrorInvalidValue;
  AddNormGroup g[2] = {make_group(m_sa, sa_dim), make_group(m_vl, vl_dim)};
  add_term(g[0], sa_res, sa_dim);
  add_term(g[0], sa_proj, sa_dim);
  add_term(g[0], sa_bias, 0);
  g[0].norm_out = static_cast<uint16_t*>(sa_out);
  g[0].norm_ld = sa_dim;
  add_term(g[1], vl_res, vl_dim);
  add_term(g[1], vl_proj, vl_dim);
  add_term(g[1], vl_bias, 0);
  g[1].norm_out = static_cast<uint16_t*>(vl_out);
  g[1].norm_ld = vl_dim;
  return launch_add_norm(g, 2, kSumF32, kNormLayer, eps, stream);
}

extern "C" hipError_t rldx_vl_epilogue_ln_bf16(const void* vl_res, const void* proj_bias, const void* w3_bias,
                                               const void* w3_out, void* new_vl, void* ln_vl, int64_t m,
                                               int64_t dim, float eps, hipStream_t stream) {
  if (!rows_ok(m, dim)) return hipErrorInvalidValue;
  AddNormGroup g = make_group(m, dim);
  add_term(g, vl_res, dim);
  add_term(g, proj_bias, 0);
  add_term(g, w3_bias, 0);
  add_term(g, w3_out, dim);
  if (m > 0 && !new_vl) return hipErrorInvalidValue;
  g.sum_out = static_cast<uint16_t*>(new_vl);
  g.sum_ld = dim;
  g.norm_out = static_cast<uint16_t*>(ln_vl);
  g.norm_ld = dim;
  return launch_add_norm(&g, 1, kSumBf16, kNormLayer, eps, stream);
}

extern "C" hipError_t rldx_ss_epilogue_ln_bf16(const void* hidden, const void* residual, void* new_hidden,
                                               void* ln_out, int64_t m, int64_t dim, float eps,
                                               hipStream_t stream) {
  if (!rows_ok(m, dim)) return hipErrorInvalidValue;
  AddNormGroup g = make_group(m, dim);
  add_term(g, hidden, dim);
  if (residual) {
    add_term(g, residual, dim);
    if (m > 0 && !new_hidden) return hipErrorInvalidValue;
    g.sum_out = static_cast<uint16_t*>(new_hidden);
    g.sum_ld = dim;
  }
  g.norm_out = static_cast<uint16_t*>(ln_out);
  g.norm_ld = dim;
  return launch_add_norm(&g, 1, kSumBf16, kNormLayer, eps, stream);
}

extern "C" hipError_t rldx_add_rmsnorm_bf16(const void* hidden, const void* residual, const void* deepstack,
                                            const void* weight, void* new_hidden, void* normed, int64_t m,
                                            int64_t dim, float eps, hipStream_t stream) {
  if (!rows_ok(m, dim)) return hipErrorInvalidValue;
  AddNormGroup g = make_group(m, dim);
  add_term(g, hidden, dim);
  add_term(g, residual, dim);
  if (deepstack) add_term(g, deepstack, dim);
  if (m > 0 && !new_hidden) return hipErrorInvalidValue;
  g.weight = static_cast<const uint16_t*>(weight);
  g.sum_out = static_cast<uint16_t*>(new_hidden);
  g.sum_ld = dim;
  g.norm_out = static_cast<uint16_t*>(normed);
  g.norm_ld = dim;
  return launch_add_norm(&g, 1, kSumBf16, kNormRms, eps, stream);
}
