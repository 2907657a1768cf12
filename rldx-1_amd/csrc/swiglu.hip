// SwiGLU for gfx950: y[r, j] = bf16( bf16(silu(gate[r, j])) * up[r, j] ),
// gate = x[r, 0:n_half], up = x[r, n_half:2*n_half]  (the `x12.chunk(2, -1)`
// split of rldx/model/modules/action_model/ops.py:157-161).
//
// Memory-bound once silu is cheap: the vectorised kernel evaluates silu with
// the hardware exp2 / reciprocal (swiglu_bf16x2, about 15 VALU operations per
// element instead of about 60 for the IEEE-division form, which made the
// kernel VALU-bound), bit-identical to the exact element function.  Every
// thread moves 16 B of gate, 16 B of up and writes 16 B of y (8 elements) with
// 128-bit global loads/stores, two chunks per thread with all four loads issued
// before any arithmetic; one workgroup per 512 chunks of a group, so any row
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
};

// One group of the vectorised kernel: rows of n_half elements cut into
// 8-element chunks; workgroups [block_begin, block_begin + blocks) cover it.
struct VecGroup {
  const uint16_t* x;
  const uint16_t* bias;
  uint16_t* y;
  int64_t ldx, ldy, n_half;
  uint32_t chunks;        // rows * n_half / 8 (< 2^31)
  uint32_t cpr;           // chunks per row
  DivMagic div;           // division by cpr
  uint32_t block_begin;   // first workgroup; 0xffffffff for an unused slot
};

struct VecArgs {
  VecGroup g[3];
};

constexpr int kVecThreads = 256;
constexpr int kVecChunks = 2;  // 8-element chunks per thread, all loads issued before any math

// Two elements per 32-bit word: (lo, hi) bf16 halves.
__device__ __forceinline__ uint32_t swiglu_pair(uint32_t g2, uint32_t u2) {
  return swiglu_bf16x2(bf16x2_lo(g2), bf16x2_hi(g2), bf16x2_lo(u2), bf16x2_hi(u2));
}

__device__ __forceinline__ uint32_t add_bias_pair(uint32_t x2, uint32_t b2) {
  return pack_bf16x2(bf16x2_lo(x2) + bf16x2_lo(b2), bf16x2_hi(x2) + bf16x2_hi(b2));
}

// The group is uniform per workgroup (scalar selection); within a group the
// chunk index is 32-bit and the row comes from the invariant-divisor multiply.
// Chunk loads past the end of a group are clamped to its last chunk (in
// bounds) and their stores skipped.
template <bool kHasBias>
__global__ __launch_bounds__(kVecThreads) void swiglu_vec8_kernel(VecArgs a) {
  const uint32_t blk = blockIdx.x;
  const int gi = (blk >= a.g[1].block_begin) + (blk >= a.g[2].block_begin);
  const VecGroup& G = a.g[gi];
  const uint32_t c0 = (blk - G.block_begin) * (kVecThreads * kVecChunks) + threadIdx.x;
  u32x4 gv[kVecChunks], uv[kVecChunks], bg[kVecChunks], bu[kVecChunks];
  int64_t yoff[kVecChunks];
#pragma unroll
  for (int i = 0; i < kVecChunks; ++i) {
    const uint32_t c = min(c0 + i * kVecThreads, G.chunks - 1);
    const uint32_t r = div_u32(c, G.div);
    const int64_t j = static_cast<int64_t>(c - r * G.cpr) * 8;
    const uint16_t* xr = G.x + r * G.ldx + j;
    gv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xr));
    uv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xr + G.n_half));
    if constexpr (kHasBias) {
      bg[i] = *reinterpret_cast<const u32x4*>(G.bias + j);
      bu[i] = *reinterpret_cast<const u32x4*>(G.bias + G.n_half + j);
    }
    yoff[i] = r * G.ldy + j;
  }
#pragma unroll
  for (int i = 0; i < kVecChunks; ++i) {
    u32x4 gx = gv[i], ux = uv[i];
    if constexpr (kHasBias) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        gx[w] = add_bias_pair(gx[w], bg[i][w]);
        ux[w] = add_bias_pair(ux[w], bu[i][w]);
      }
    }
    u32x4 out;
#pragma unroll
    for (int w = 0; w < 4; ++w) out[w] = swiglu_pair(gx[w], ux[w]);
    if (c0 + i * kVecThreads < G.chunks)
      __builtin_nontemporal_store(out, reinterpret_cast<u32x4*>(G.y + yoff[i]));
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
         (G.bias == nullptr || aligned16(G.bias)) && G.rows * (G.n_half / 8) < (int64_t{1} << 31);
}

int grid_for(int64_t work_items) {
  // Scalar kernel: 256 CUs x 8 resident 256-thread groups; a grid-stride loop covers the rest.
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
    VecArgs a{};
    for (auto& v : a.g) v.block_begin = 0xffffffffu;
    int64_t blocks = 0;
    int k = 0;
    for (int i = 0; i < n; ++i) {
      if (gs[i].rows == 0 || gs[i].n_half == 0) continue;
      VecGroup& v = a.g[k++];
      v.x = gs[i].x;
      v.bias = gs[i].bias;
      v.y = gs[i].y;
      v.ldx = gs[i].ldx;
      v.ldy = gs[i].ldy;
      v.n_half = gs[i].n_half;
      v.cpr = static_cast<uint32_t>(gs[i].n_half / 8);
      v.chunks = static_cast<uint32_t>(gs[i].rows * v.cpr);
      v.div = div_magic(v.cpr);
      v.block_begin = static_cast<uint32_t>(blocks);
      blocks += (v.chunks + kVecThreads * kVecChunks - 1) / (kVecThreads * kVecChunks);
    }
    if (k == 0) return hipSuccess;
    if (blocks >= 0xffffffffll) return hipErrorInvalidValue;
    if (has_bias)
      hipLaunchKernelGGL(swiglu_vec8_kernel<true>, dim3(static_cast<uint32_t>(blocks)), dim3(kVecThreads), 0,
                         stream, a);
    else
      hipLaunchKernelGGL(swiglu_vec8_kernel<false>, dim3(static_cast<uint32_t>(blocks)), dim3(kVecThreads), 0,
                         stream, a);
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
                ldx, ldy, rows, n_half};
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
       2 * n_half_sa, n_half_sa, m_sa, n_half_sa},
      {static_cast<const uint16_t*>(vl_x), static_cast<const uint16_t*>(vl_bias), static_cast<uint16_t*>(vl_y),
       2 * n_half_vl, n_half_vl, m_vl, n_half_vl},
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
