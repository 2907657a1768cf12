// SwiGLU for gfx950: y[r, j] = bf16( bf16(silu(gate[r, j])) * up[r, j] ),
// gate = x[r, 0:n_half], up = x[r, n_half:2*n_half]  (the `x12.chunk(2, -1)`
// split of rldx/model/modules/action_model/ops.py:157-161).
//
// Memory-bound: every thread moves 16 B of gate, 16 B of up and writes 16 B of
// y (8 elements) with 128-bit global loads/stores.  Work is a flat list of
// 8-element chunks over all groups, walked with a grid-stride loop, so any row
// count fills all 256 CUs.
//
// Optional per-column bias (the `ds::grouped_swiglu` form,
// rldx/inference/action_model/double_stream/engine/ops/op_grouped_swiglu.py:12-49)
// is added with eager bf16 rounding: bf16(x + b) before silu / product.
#include "rldx_amd.h"
#include "rldx_common.h"

namespace rldx {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct SwigluGroup {
  const uint16_t* x;     // [rows, >= 2*n_half] bf16, row stride ldx elements
  const uint16_t* bias;  // [2*n_half] bf16 or nullptr
  uint16_t* y;           // [rows, >= n_half] bf16, row stride ldy elements
  int64_t ldx, ldy;
  int64_t rows, n_half;
  int64_t chunks_per_row;  // n_half / 8
  int64_t chunk_begin;     // first flat chunk index of this group
};

struct SwigluArgs {
  SwigluGroup g[3];
  int num_groups;
  int64_t total_chunks;
};

__device__ __forceinline__ uint32_t swiglu_pair(uint32_t g2, uint32_t u2) {
  uint16_t lo = swiglu_bf16_bits(static_cast<uint16_t>(g2 & 0xffffu), static_cast<uint16_t>(u2 & 0xffffu));
  uint16_t hi = swiglu_bf16_bits(static_cast<uint16_t>(g2 >> 16), static_cast<uint16_t>(u2 >> 16));
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

__device__ __forceinline__ uint32_t add_bias_pair(uint32_t x2, uint32_t b2) {
  uint16_t lo = f32_to_bf16_bits(bf16_bits_to_f32(static_cast<uint16_t>(x2 & 0xffffu)) +
                                 bf16_bits_to_f32(static_cast<uint16_t>(b2 & 0xffffu)));
  uint16_t hi = f32_to_bf16_bits(bf16_bits_to_f32(static_cast<uint16_t>(x2 >> 16)) +
                                 bf16_bits_to_f32(static_cast<uint16_t>(b2 >> 16)));
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

template <bool kHasBias>
__global__ __launch_bounds__(256) void swiglu_vec8_kernel(SwigluArgs args) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; c < args.total_chunks;
       c += stride) {
    int gi = 0;
    if (args.num_groups > 1 && c >= args.g[1].chunk_begin) gi = 1;
    if (args.num_groups > 2 && c >= args.g[2].chunk_begin) gi = 2;
    const SwigluGroup& G = args.g[gi];
    const int64_t local = c - G.chunk_begin;
    const int64_t r = local / G.chunks_per_row;
    const int64_t j = (local - r * G.chunks_per_row) * 8;
    const u32x4* gp = reinterpret_cast<const u32x4*>(G.x + r * G.ldx + j);
    const u32x4* up = reinterpret_cast<const u32x4*>(G.x + r * G.ldx + G.n_half + j);
    u32x4 gv = __builtin_nontemporal_load(gp);
    u32x4 uv = __builtin_nontemporal_load(up);
    if constexpr (kHasBias) {
      u32x4 bg = *reinterpret_cast<const u32x4*>(G.bias + j);
      u32x4 bu = *reinterpret_cast<const u32x4*>(G.bias + G.n_half + j);
      gv.x = add_bias_pair(gv.x, bg.x); gv.y = add_bias_pair(gv.y, bg.y);
      gv.z = add_bias_pair(gv.z, bg.z); gv.w = add_bias_pair(gv.w, bg.w);
      uv.x = add_bias_pair(uv.x, bu.x); uv.y = add_bias_pair(uv.y, bu.y);
      uv.z = add_bias_pair(uv.z, bu.z); uv.w = add_bias_pair(uv.w, bu.w);
    }
    u32x4 out;
    out.x = swiglu_pair(gv.x, uv.x);
    out.y = swiglu_pair(gv.y, uv.y);
    out.z = swiglu_pair(gv.z, uv.z);
    out.w = swiglu_pair(gv.w, uv.w);
    __builtin_nontemporal_store(out, reinterpret_cast<u32x4*>(G.y + r * G.ldy + j));
  }
}

// Scalar fallback for shapes/strides the 128-bit path cannot take
// (n_half not a multiple of 8, or rows not 16-byte aligned).
template <bool kHasBias>
__global__ __launch_bounds__(256) void swiglu_scalar_kernel(SwigluGroup G) {
  const int64_t total = G.rows * G.n_half;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / G.n_half;
    const int64_t j = i - r * G.n_half;
    uint16_t g = G.x[r * G.ldx + j];
    uint16_t u = G.x[r * G.ldx + G.n_half + j];
    if constexpr (kHasBias) {
      g = f32_to_bf16_bits(bf16_bits_to_f32(g) + bf16_bits_to_f32(G.bias[j]));
      u = f32_to_bf16_bits(bf16_bits_to_f32(u) + bf16_bits_to_f32(G.bias[G.n_half + j]));
    }
    G.y[r * G.ldy + j] = swiglu_bf16_bits(g, u);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool vec_ok(const SwigluGroup& G) {
  return (G.n_half % 8 == 0) && (G.ldx % 8 == 0) && (G.ldy % 8 == 0) && aligned16(G.x) && aligned16(G.y) &&
         (G.bias == nullptr || aligned16(G.bias));
}

int grid_for(int64_t work_items) {
  // 256 CUs x 8 resident 256-thread groups; the grid-stride loop covers the rest.
  const int64_t max_blocks = 256 * 8;
  int64_t b = (work_items + 255) / 256;
  if (b > max_blocks) b = max_blocks;
  if (b < 1) b = 1;
  return static_cast<int>(b);
}

hipError_t launch_groups(SwigluGroup* gs, int n, hipStream_t stream) {
  bool has_bias = gs[0].bias != nullptr;
  bool all_vec = true;
  for (int i = 0; i < n; ++i) {
    if ((gs[i].bias != nullptr) != has_bias) return hipErrorInvalidValue;
    all_vec = all_vec && vec_ok(gs[i]);
  }
  if (all_vec) {
    SwigluArgs a{};
    int64_t begin = 0;
    int k = 0;
    for (int i = 0; i < n; ++i) {
      if (gs[i].rows == 0 || gs[i].n_half == 0) continue;
      a.g[k] = gs[i];
      a.g[k].chunks_per_row = gs[i].n_half / 8;
      a.g[k].chunk_begin = begin;
      begin += gs[i].rows * a.g[k].chunks_per_row;
      ++k;
    }
    if (k == 0) return hipSuccess;
    a.num_groups = k;
    a.total_chunks = begin;
    const int grid = grid_for(begin);
    if (has_bias)
      hipLaunchKernelGGL(swiglu_vec8_kernel<true>, dim3(grid), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL(swiglu_vec8_kernel<false>, dim3(grid), dim3(256), 0, stream, a);
    return hipGetLastError();
  }
  for (int i = 0; i < n; ++i) {
    if (gs[i].rows == 0 || gs[i].n_half == 0) continue;
    const int grid = grid_for(gs[i].rows * gs[i].n_half);
    if (has_bias)
      hipLaunchKernelGGL(swiglu_scalar_kernel<true>, dim3(grid), dim3(256), 0, stream, gs[i]);
    else
      hipLaunchKernelGGL(swiglu_scalar_kernel<false>, dim3(grid), dim3(256), 0, stream, gs[i]);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

bool group_valid(const void* x, const void* y, int64_t ldx, int64_t ldy, int64_t rows, int64_t n_half) {
  if (rows < 0 || n_half < 0) return false;
  if (rows == 0 || n_half == 0) return true;
  if (x == nullptr || y == nullptr) return false;
  if (ldx < 2 * n_half || ldy < n_half) return false;
  return true;
}

}  // namespace
}  // namespace rldx

using namespace rldx;

extern "C" hipError_t rldx_swiglu_bf16(const void* x, int64_t ldx, const void* bias, void* y, int64_t ldy,
                                       int64_t rows, int64_t n_half, hipStream_t stream) {
  if (!group_valid(x, y, ldx, ldy, rows, n_half)) return hipErrorInvalidValue;
  SwigluGroup g{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y),
                ldx, ldy, rows, n_half, 0, 0};
  return launch_groups(&g, 1, stream);
}

extern "C" hipError_t rldx_grouped_swiglu_bf16(const void* sa_x, const void* sa_bias, const void* vl_x,
                                               const void* vl_bias, void* sa_y, void* vl_y, int64_t m_sa,
                                               int64_t m_vl, int64_t n_half_sa, int64_t n_half_vl,
                                               hipStream_t stream) {
  if (!group_valid(sa_x, sa_y, 2 * n_half_sa, n_half_sa, m_sa, n_half_sa)) return hipErrorInvalidValue;
  if (!group_valid(vl_x, vl_y, 2 * n_half_vl, n_half_vl, m_vl, n_half_vl)) return hipErrorInvalidValue;
  if ((sa_bias == nullptr) != (vl_bias == nullptr)) return hipErrorInvalidValue;
  SwigluGroup g[2] = {
      {static_cast<const uint16_t*>(sa_x), static_cast<const uint16_t*>(sa_bias), static_cast<uint16_t*>(sa_y),
       2 * n_half_sa, n_half_sa, m_sa, n_half_sa, 0, 0},
      {static_cast<const uint16_t*>(vl_x), static_cast<const uint16_t*>(vl_bias), static_cast<uint16_t*>(vl_y),
       2 * n_half_vl, n_half_vl, m_vl, n_half_vl, 0, 0},
  };
  return launch_groups(g, 2, stream);
}

// Host execution of the exact device element function, used by the CPU test
// suite to verify the silu/SwiGLU rounding exhaustively over all bf16 inputs.
extern "C" int rldx_host_swiglu_bf16(const uint16_t* g, const uint16_t* u, uint16_t* y, int64_t n) {
  if (n < 0 || (n > 0 && (g == nullptr || u == nullptr || y == nullptr))) return 1;
  for (int64_t i = 0; i < n; ++i) y[i] = swiglu_bf16_bits(g[i], u[i]);
  return 0;
}
