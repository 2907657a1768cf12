// Model-level primitives of the reference's eager modules, for callers that
// use the modules directly rather than the fused chains:
//   * RMSNorm (rldx/model/modules/norms.py:7-22): y = (w * (x * rsqrt(mean(x^2)
//     + eps))).to(x.dtype) -- fp32 arithmetic, one rounding at the end, w fp32
//     (the module's parameter) or bf16 (a model cast to bf16, promoted to fp32
//     by the product).
//   * Interleaved RoPE, apply_rotary_emb (rldx/model/modules/action_model/
//     ops.py:48-67): pairs (x[2i], x[2i+1]) times freqs_cis[n][i] = (cos, sin)
//     as complex numbers in fp32, rounded once to the input type.
// Both are HBM-bound elementwise / row kernels: 16-byte loads and stores, the
// row reduction over the lanes that hold the row (xor shuffles), no LDS.
#include "rldx_amd.h"
#include "rldx_common.h"

namespace rldx {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16-byte chunk <-> V fp32 values (V = 8 for bf16, 4 for fp32)
template <typename T>
struct Chunk;
template <>
struct Chunk<uint16_t> {
  static constexpr int V = 8;
  static __device__ __forceinline__ void unpack(const u32x4& r, float* v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16x2_lo(r[i]);
      v[2 * i + 1] = bf16x2_hi(r[i]);
    }
  }
  static __device__ __forceinline__ u32x4 pack(const float* v) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    return r;
  }
};
template <>
struct Chunk<float> {
  static constexpr int V = 4;
  static __device__ __forceinline__ void unpack(const u32x4& r, float* v) {
    // through a scalar: __builtin_bit_cast of a vector element lvalue compiles
    // to a cast of the vector's first element
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t u = r[i];
      v[i] = __builtin_bit_cast(float, u);
    }
  }
  static __device__ __forceinline__ u32x4 pack(const float* v) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = __builtin_bit_cast(uint32_t, v[i]);
    return r;
  }
};

struct RmsArgs {
  const void* x;
  void* out;
  const void* w;
  int64_t x_ld, o_ld;  // row strides (elements)
  int rows, dim;
  int w_f32;           // weight dtype: fp32 (1) or bf16 (0)
  float eps;
};

// LPR lanes per row (consecutive, aligned), each holding CPL 16-byte chunks:
// lane j of a row has columns V (j + LPR c) .. + V - 1.
template <typename T, int LPR, int CPL>
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(RmsArgs a) {
#pragma clang fp contract(off)
  using C = Chunk<T>;
  constexpr int V = C::V;
  const int gid = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  const int row = gid / LPR, j = gid % LPR;
  const bool valid = row < a.rows;  // the whole row group agrees
  const T* xr = static_cast<const T*>(a.x) + static_cast<int64_t>(valid ? row : 0) * a.x_ld;
  float v[CPL][V];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = V * (j + LPR * c);
    const u32x4 raw = valid && col < a.dim ? *reinterpret_cast<const u32x4*>(xr + col) : u32x4{0, 0, 0, 0};
    C::unpack(raw, v[c]);
#pragma unroll
    for (int i = 0; i < V; ++i) ss += v[c][i] * v[c][i];
  }
#pragma unroll
  for (int m = LPR / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
  const float r = 1.0f / __builtin_sqrtf(ss / static_cast<float>(a.dim) + a.eps);
  if (!valid) return;
  T* orow = static_cast<T*>(a.out) + static_cast<int64_t>(row) * a.o_ld;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = V * (j + LPR * c);
    if (col >= a.dim) continue;
    float w[V];
    if (a.w_f32) {
      const f32x4* wp = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.w) + col);
#pragma unroll
      for (int q = 0; q < V / 4; ++q) {
        const f32x4 t = wp[q];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[4 * q + i] = t[i];
      }
    } else {
      const uint16_t* wb = static_cast<const uint16_t*>(a.w) + col;
#pragma unroll
      for (int i = 0; i < V; ++i) w[i] = bf16_bits_to_f32(wb[i]);
    }
    float y[V];
#pragma unroll
    for (int i = 0; i < V; ++i) y[i] = w[i] * (v[c][i] * r);
    *reinterpret_cast<u32x4*>(orow + col) = C::pack(y);
  }
}

template <typename T, int LPR, int CPL>
void launch_rms(const RmsArgs& a, hipStream_t stream) {
  const int64_t threads = static_cast<int64_t>(a.rows) * LPR;
  hipLaunchKernelGGL((rms_norm_rows_kernel<T, LPR, CPL>), dim3(static_cast<unsigned>((threads + 255) / 256)),
                     dim3(256), 0, stream, a);
}

template <typename T>
hipError_t rms_entry(const void* x, int64_t x_ld, const void* w, int32_t w_is_f32, void* out, int64_t o_ld,
                     int64_t rows, int64_t dim, float eps, hipStream_t stream) {
  constexpr int V = Chunk<T>::V;
  if (rows < 0 || dim < 0 || !(eps >= 0.f)) return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  if (dim == 0 || dim % V || dim > 64 * 16 * V || !x || !out || !w) return hipErrorInvalidValue;
  if (x_ld < dim || o_ld < dim || x_ld % V || o_ld % V) return hipErrorInvalidValue;
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                       (w_is_f32 ? reinterpret_cast<uintptr_t>(w) : 0);
  if (al % 16 || reinterpret_cast<uintptr_t>(w) % 2) return hipErrorInvalidValue;
  if (rows * 64 > (int64_t{1} << 31) - 256) return hipErrorInvalidValue;
  RmsArgs a{x, out, w, x_ld, o_ld, static_cast<int>(rows), static_cast<int>(dim), w_is_f32 ? 1 : 0, eps};
  const int64_t chunks = dim / V;
  if (chunks <= 8) launch_rms<T, 8, 1>(a, stream);
  else if (chunks <= 16) launch_rms<T, 16, 1>(a, stream);
  else if (chunks <= 32) launch_rms<T, 32, 1>(a, stream);
  else if (chunks <= 64) launch_rms<T, 64, 1>(a, stream);
  else if (chunks <= 128) launch_rms<T, 64, 2>(a, stream);
  else if (chunks <= 256) launch_rms<T, 64, 4>(a, stream);
  else if (chunks <= 512) launch_rms<T, 64, 8>(a, stream);
  else launch_rms<T, 64, 16>(a, stream);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Interleaved RoPE
// ---------------------------------------------------------------------------
struct RopeTensor {
  const void* in;
  void* out;
  int64_t sb, sh, sn;     // input strides (elements) over (B, H, N)
  int64_t ob, oh, on;     // output strides
  int heads;
};

struct RopeArgs {
  RopeTensor t[2];        // q, k
  const float* freqs;     // (cos, sin) pairs: [B or 1][N][D / 2] complex64
  int64_t f_sb, f_sn;     // strides in pairs (f_sb 0: one table for every batch entry)
  int batch, seq, head_dim;
  int64_t q_chunks;       // 16-byte chunks of q (B * Hq * N * D / V); k's follow
  DivMagic cpr_div;       // chunks per row (D / V)
  DivMagic seq_div;
  DivMagic hq_div, hk_div;
};

template <typename T>
__global__ __launch_bounds__(256) void rope_interleaved_kernel(RopeArgs a, int64_t total) {
#pragma clang fp contract(off)
  using C = Chunk<T>;
  constexpr int V = C::V;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= total) return;
  const bool is_k = gid >= a.q_chunks;
  const RopeTensor& t = a.t[is_k ? 1 : 0];
  const uint32_t idx = static_cast<uint32_t>(is_k ? gid - a.q_chunks : gid);
  const uint32_t row = div_u32(idx, a.cpr_div);
  const int c = static_cast<int>(idx - row * static_cast<uint32_t>(a.head_dim / V));
  const uint32_t bh = div_u32(row, a.seq_div);
  const int n = static_cast<int>(row - bh * static_cast<uint32_t>(a.seq));
  const uint32_t b = div_u32(bh, is_k ? a.hk_div : a.hq_div);
  const int h = static_cast<int>(bh - b * static_cast<uint32_t>(t.heads));
  const T* src = static_cast<const T*>(t.in) + b * t.sb + h * t.sh + n * t.sn + c * V;
  const float* f = a.freqs + 2 * (b * a.f_sb + n * a.f_sn + c * (V / 2));
  float x[V], fr[V];
  C::unpack(*reinterpret_cast<const u32x4*>(src), x);
#pragma unroll
  for (int q = 0; q < V / 4; ++q) {
    const f32x4 p = reinterpret_cast<const f32x4*>(f)[q];
#pragma unroll
    for (int i = 0; i < 4; ++i) fr[4 * q + i] = p[i];
  }
  float y[V];
#pragma unroll
  for (int p = 0; p < V / 2; ++p) {
    const float re = x[2 * p], im = x[2 * p + 1], cs = fr[2 * p], sn = fr[2 * p + 1];
    y[2 * p] = re * cs - im * sn;
    y[2 * p + 1] = im * cs + re * sn;
  }
  T* dst = static_cast<T*>(t.out) + b * t.ob + h * t.oh + n * t.on + c * V;
  *reinterpret_cast<u32x4*>(dst) = C::pack(y);
}

template <typename T>
hipError_t rope_entry(const void* xq, const int64_t* q_strides, void* q_out, const int64_t* q_out_strides,
                      const void* xk, const int64_t* k_strides, void* k_out, const int64_t* k_out_strides,
                      int64_t batch, int64_t q_heads, int64_t k_heads, int64_t seq, int64_t head_dim,
                      const float* freqs, const int64_t* freqs_strides, hipStream_t stream) {
  constexpr int V = Chunk<T>::V;
  if (batch < 0 || q_heads < 0 || k_heads < 0 || seq < 0 || head_dim <= 0 || head_dim % V) return hipErrorInvalidValue;
  if (batch == 0 || seq == 0 || q_heads + k_heads == 0) return hipSuccess;
  if (!freqs || !freqs_strides || reinterpret_cast<uintptr_t>(freqs) % 16) return hipErrorInvalidValue;
  if (freqs_strides[0] < 0 || freqs_strides[1] < 0 || freqs_strides[0] % 2 || freqs_strides[1] % 2)
    return hipErrorInvalidValue;  // whole 16-byte pair groups
  if (seq > 1 && freqs_strides[1] < head_dim / 2) return hipErrorInvalidValue;
  RopeArgs a{};
  const void* ins[2] = {xq, xk};
  void* outs[2] = {q_out, k_out};
  const int64_t* ist[2] = {q_strides, k_strides};
  const int64_t* ost[2] = {q_out_strides, k_out_strides};
  const int64_t heads[2] = {q_heads, k_heads};
  for (int i = 0; i < 2; ++i) {
    if (heads[i] == 0) continue;
    if (!ins[i] || !outs[i] || !ist[i] || !ost[i]) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(ins[i]) | reinterpret_cast<uintptr_t>(outs[i])) % 16) return hipErrorInvalidValue;
    for (int d = 0; d < 3; ++d)
      if (ist[i][d] % V || ost[i][d] % V || ist[i][d] < 0 || ost[i][d] < 0) return hipErrorInvalidValue;
    a.t[i] = RopeTensor{ins[i], outs[i], ist[i][0], ist[i][1], ist[i][2], ost[i][0], ost[i][1], ost[i][2],
                        static_cast<int>(heads[i])};
  }
  const int64_t cpr = head_dim / V;
  a.q_chunks = batch * q_heads * seq * cpr;
  const int64_t total = a.q_chunks + batch * k_heads * seq * cpr;
  if (a.q_chunks >= (int64_t{1} << 31) || total - a.q_chunks >= (int64_t{1} << 31) || seq > (1 << 30) ||
      q_heads > (1 << 20) || k_heads > (1 << 20))
    return hipErrorInvalidValue;
  a.freqs = freqs;
  a.f_sb = freqs_strides[0];
  a.f_sn = freqs_strides[1];
  a.batch = static_cast<int>(batch);
  a.seq = static_cast<int>(seq);
  a.head_dim = static_cast<int>(head_dim);
  a.cpr_div = div_magic(static_cast<uint32_t>(cpr));
  a.seq_div = div_magic(static_cast<uint32_t>(seq));
  a.hq_div = div_magic(static_cast<uint32_t>(q_heads > 0 ? q_heads : 1));
  a.hk_div = div_magic(static_cast<uint32_t>(k_heads > 0 ? k_heads : 1));
  hipLaunchKernelGGL(rope_interleaved_kernel<T>, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                     stream, a, total);
  return hipGetLastError();
}

}  // namespace
}  // namespace rldx

using namespace rldx;

extern "C" hipError_t rldx_rms_norm_bf16(const void* x, int64_t x_row_stride, const void* weight, int32_t weight_is_f32,
                                         void* out, int64_t out_row_stride, int64_t rows, int64_t dim, float eps,
                                         hipStream_t stream) {
  return rms_entry<uint16_t>(x, x_row_stride, weight, weight_is_f32, out, out_row_stride, rows, dim, eps, stream);
}

extern "C" hipError_t rldx_rms_norm_f32(const float* x, int64_t x_row_stride, const void* weight,
                                        int32_t weight_is_f32, float* out, int64_t out_row_stride, int64_t rows,
                                        int64_t dim, float eps, hipStream_t stream) {
  return rms_entry<float>(x, x_row_stride, weight, weight_is_f32, out, out_row_stride, rows, dim, eps, stream);
}

extern "C" hipError_t rldx_rope_interleaved_bf16(const void* xq, const int64_t* q_strides, void* q_out,
                                                 const int64_t* q_out_strides, const void* xk,
                                                 const int64_t* k_strides, void* k_out, const int64_t* k_out_strides,
                                                 int64_t batch, int64_t q_heads, int64_t k_heads, int64_t seq,
                                                 int64_t head_dim, const float* freqs, const int64_t* freqs_strides,
                                                 hipStream_t stream) {
  return rope_entry<uint16_t>(xq, q_strides, q_out, q_out_strides, xk, k_strides, k_out, k_out_strides, batch,
                              q_heads, k_heads, seq, head_dim, freqs, freqs_strides, stream);
}

extern "C" hipError_t rldx_rope_interleaved_f32(const float* xq, const int64_t* q_strides, float* q_out,
                                                const int64_t* q_out_strides, const float* xk,
                                                const int64_t* k_strides, float* k_out, const int64_t* k_out_strides,
                                                int64_t batch, int64_t q_heads, int64_t k_heads, int64_t seq,
                                                int64_t head_dim, const float* freqs, const int64_t* freqs_strides,
                                                hipStream_t stream) {
  return rope_entry<float>(xq, q_strides, q_out, q_out_strides, xk, k_strides, k_out, k_out_strides, batch, q_heads,
                           k_heads, seq, head_dim, freqs, freqs_strides, stream);
}
