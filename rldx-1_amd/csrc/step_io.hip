// The flow-matching loop's action encoder and decoder around the MSAT blocks,
// one launch each per denoising iteration (the eager chain is eleven launches:
// addmm, two adds and three operand packs before the blocks; unpack,
// layer_norm, addmm, mul and add after them):
//   * encode + pack: the action rows x = bf16(bf16(bf16(act W_in^T + b_in) +
//     temb) + pos) (addmm, add, add of the eager loop), written in the grouped
//     GEMM's packed activation order with the LayerNorm statistics a folding
//     GEMM reads, and up to three more row-major matrices (the cognition and
//     physics inputs) packed with their statistics by the same launch;
//   * decode + Euler: act = bf16(act + bf16(dt * bf16(LN(x) W_out^T + b_out)))
//     with LN(x) = bf16((x - mean) * rsqrt(var + eps)) (no affine) of the packed
//     action rows.
// The small linears (action_dim 32) are dot products in fp32 on the vector
// units; the statistics are summed in the order rows_pack_kernel uses, so they
// are the bits that packing the same bf16 rows with rldx_act_pack_stats_bf16
// gives.  The action rows take one workgroup each (a thread per 8 columns: the
// dot products of a row spread over 192 threads instead of 64 lanes).
#include "rldx_amd.h"
#include "rldx_common.h"

namespace rldx {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kEncMats = 4;   // the encoded rows + up to 3 packed matrices
constexpr int kMaxAdim = 64;  // action_dim bound (registers of one act row)

__device__ __forceinline__ float bfv(uint16_t b) { return bf16_bits_to_f32(b); }

struct EncArgs {
  const uint16_t* act;   // [n, adim]
  const uint16_t* w_in;  // [k, adim]
  const uint16_t* b_in;  // [k]
  const uint16_t* temb;  // [k]
  const uint16_t* pos;   // [n, k]
  int adim;
  // matrix 0: the encoded rows (x == nullptr); 1..: row-major inputs
  const uint16_t* x[kEncMats];
  int64_t ldx[kEncMats];
  uint16_t* out[kEncMats];
  float* stats[kEncMats];
  int m[kEncMats];
  int begin[kEncMats + 1];
  int count, k;
};

// Workgroups [0, m[0]) encode one action row each: thread t computes the 8
// columns 8 t .. 8 t + 7 (k / 8 <= 256 threads), the row's statistics summed
// per wave and then over the waves.  The workgroups after them pack the other
// matrices, one wave per row (4 rows per workgroup, lane j holding columns
// 8 (j + 64 c) .. +7), as rows_pack_kernel does.
template <int CPL>
__global__ __launch_bounds__(256) void encode_pack_kernel(EncArgs a) {
  const int k = a.k;
  const int lane = threadIdx.x & 63;
  if (a.x[0] == nullptr && static_cast<int>(blockIdx.x) < a.m[0]) {
    // statistics chain: thread t = lane + 64 c holds the chunk that lane `lane`
    // of rows_pack_kernel holds as its c-th; the per-lane sums are carried from
    // wave to wave in that order, then reduced over the lanes as there
    __shared__ float chain[2][64];
    const int row = blockIdx.x, t = threadIdx.x, wv = t >> 6, col = 8 * t;
    const bool live = col < k;
    float v[8];
    if (live) {
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = 0.f;
      const uint16_t* ap = a.act + static_cast<int64_t>(row) * a.adim;
      for (int q = 0; q < a.adim / 8; ++q) {  // 8 inputs at a time: act chunk (broadcast) x 8 weight rows
        const u32x4 av = *reinterpret_cast<const u32x4*>(ap + 8 * q);
        float ar[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ar[2 * e] = bf16x2_lo(av[e]);
          ar[2 * e + 1] = bf16x2_hi(av[e]);
        }
        u32x4 wq[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          wq[i] = *reinterpret_cast<const u32x4*>(a.w_in + static_cast<int64_t>(col + i) * a.adim + 8 * q);
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            y[i] = __builtin_fmaf(ar[2 * e], bf16x2_lo(wq[i][e]), y[i]);
            y[i] = __builtin_fmaf(ar[2 * e + 1], bf16x2_hi(wq[i][e]), y[i]);
          }
      }
      const u32x4 bi = *reinterpret_cast<const u32x4*>(a.b_in + col);
      const u32x4 te = *reinterpret_cast<const u32x4*>(a.temb + col);
      const u32x4 po = *reinterpret_cast<const u32x4*>(a.pos + static_cast<int64_t>(row) * k + col);
      u32x4 raw;
      // addmm (bias in fp32, one rounding), then the two bf16 adds
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t x = pack_bf16x2(y[2 * e] + bf16x2_lo(bi[e]), y[2 * e + 1] + bf16x2_hi(bi[e]));
        x = pack_bf16x2(bf16x2_lo(x) + bf16x2_lo(te[e]), bf16x2_hi(x) + bf16x2_hi(te[e]));
        x = pack_bf16x2(bf16x2_lo(x) + bf16x2_lo(po[e]), bf16x2_hi(x) + bf16x2_hi(po[e]));
        raw[e] = x;
        v[2 * e] = bf16x2_lo(x);
        v[2 * e + 1] = bf16x2_hi(x);
      }
      *reinterpret_cast<u32x4*>(a.out[0] + packed_act_offset(row, col, k)) = raw;
    }
    for (int c = 0; c < 4; ++c) {  // (k <= 2048: at most 4 chunks per lane)
      if (wv == c) {
        float s1 = c == 0 ? 0.f : chain[0][lane], s2 = c == 0 ? 0.f : chain[1][lane];
        if (live) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            s1 += v[i];
            s2 += v[i] * v[i];
          }
        }
        chain[0][lane] = s1;
        chain[1][lane] = s2;
      }
      __syncthreads();
    }
    if (wv == 0) {
      float s1 = chain[0][lane], s2 = chain[1][lane];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        s1 += __shfl_xor(s1, o, 64);
        s2 += __shfl_xor(s2, o, 64);
      }
      // statistics [k / 64][m][2]: the row's sums in slot 0, zeros in the others
      const int m = a.m[0];
      f32x2* st = reinterpret_cast<f32x2*>(a.stats[0]) + row;
      if (lane < k / 64) st[static_cast<int64_t>(lane) * m] = lane == 0 ? f32x2{s1, s2} : f32x2{0.f, 0.f};
    }
    return;
  }
  int mi = a.x[0] == nullptr ? 1 : 0;
#pragma unroll
  for (int i = 1; i < kEncMats; ++i)
    if (i < a.count && static_cast<int>(blockIdx.x) >= a.begin[i]) mi = i;
  const int row = (static_cast<int>(blockIdx.x) - a.begin[mi]) * 4 + (threadIdx.x >> 6);
  const int m = a.m[mi];
  if (row >= m) return;
  float v[CPL][8];
  u32x4 raw[CPL];
  const uint16_t* xr = a.x[mi] + static_cast<int64_t>(row) * a.ldx[mi];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = 8 * (lane + 64 * c);
    raw[c] = col < k ? *reinterpret_cast<const u32x4*>(xr + col) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[c][2 * i] = bf16x2_lo(raw[c][i]);
      v[c][2 * i + 1] = bf16x2_hi(raw[c][i]);
    }
  }
  uint16_t* out = a.out[mi];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = 8 * (lane + 64 * c);
    if (col < k) {
      *reinterpret_cast<u32x4*>(out + packed_act_offset(row, col, k)) = raw[c];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        s1 += v[c][i];
        s2 += v[c][i] * v[c][i];
      }
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    s1 += __shfl_xor(s1, o, 64);
    s2 += __shfl_xor(s2, o, 64);
  }
  // statistics [k / 64][m][2]: the row's sums in slot 0, zeros in the others
  f32x2* st = reinterpret_cast<f32x2*>(a.stats[mi]) + row;
  for (int j = lane; j < k / 64; j += 64) st[static_cast<int64_t>(j) * m] = j == 0 ? f32x2{s1, s2} : f32x2{0.f, 0.f};
}

struct DecArgs {
  const uint16_t* x;  // packed [m, k]
  const uint16_t* w_out;  // [adim, k]
  const uint16_t* b_out;  // [adim]
  uint16_t* act;          // [m, adim], updated in place
  int m, k, adim;
  float eps, dt;
};

// One workgroup per row; thread t holds columns 8 t .. 8 t + 7 (k <= 2048).
__global__ __launch_bounds__(256) void decode_euler_kernel(DecArgs a) {
  __shared__ float red[4][kMaxAdim + 2];
  const int row = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int k = a.k;
  const bool live = 8 * t < k;
  float v[8];
  {
    const u32x4 r = live ? *reinterpret_cast<const u32x4*>(a.x + packed_act_offset(row, 8 * t, k)) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16x2_lo(r[i]);
      v[2 * i + 1] = bf16x2_hi(r[i]);
    }
  }
  // mean, then the biased variance about it (two passes, fp32)
  auto block_sum = [&](float s, int slot) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) red[wv][slot] = s;
    __syncthreads();
    const float r = red[0][slot] + red[1][slot] + red[2][slot] + red[3][slot];
    __syncthreads();
    return r;
  };
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += v[i];
  const float mean = block_sum(s, 0) / static_cast<float>(k);
  float q = 0.f;
  if (live) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float d = v[i] - mean;
      q += d * d;
    }
  }
  const float var = block_sum(q, 1) / static_cast<float>(k);
  const float rstd = 1.0f / __builtin_sqrtf(var + a.eps);
  float h[8];
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    const uint32_t p = pack_bf16x2((v[i] - mean) * rstd, (v[i + 1] - mean) * rstd);
    h[i] = live ? bf16x2_lo(p) : 0.f;
    h[i + 1] = live ? bf16x2_hi(p) : 0.f;
  }
  // vel[j] = sum_c h[c] W_out[j][c]: each thread's 8 columns of 8 outputs at a
  // time (their weight chunks loaded together), then the wave sums, then the
  // sum over the waves
  for (int j0 = 0; j0 < a.adim; j0 += 8) {
    u32x4 w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      w[j] = live ? *reinterpret_cast<const u32x4*>(a.w_out + static_cast<int64_t>(j0 + j) * k + 8 * t)
                  : u32x4{0, 0, 0, 0};
    float p[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        p[j] = __builtin_fmaf(h[2 * e], bf16x2_lo(w[j][e]), p[j]);
        p[j] = __builtin_fmaf(h[2 * e + 1], bf16x2_hi(w[j][e]), p[j]);
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
      for (int j = 0; j < 8; ++j) p[j] += __shfl_xor(p[j], o, 64);
    if (lane == 0)
#pragma unroll
      for (int j = 0; j < 8; ++j) red[wv][2 + j0 + j] = p[j];
  }
  __syncthreads();
  if (t < a.adim) {
    const float y = red[0][2 + t] + red[1][2 + t] + red[2][2 + t] + red[3][2 + t];
    uint16_t* ap = a.act + static_cast<int64_t>(row) * a.adim + t;
    // addmm (bias in fp32, one rounding), vel * dt, act + vel: each rounded to bf16
    const float vel = round_bf16(y + bfv(a.b_out[t]));
    const float step = round_bf16(vel * a.dt);
    *ap = f32_to_bf16_bits(bfv(*ap) + step);
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace rldx

using namespace rldx;

extern "C" hipError_t rldx_action_encode_pack_bf16(const void* act, int64_t n, int64_t action_dim, const void* w_in,
                                                   const void* b_in, const void* temb, const void* pos,
                                                   int64_t hidden, void* packed, float* stats,
                                                   const rldx_rows_t* rows, float* const* rows_stats,
                                                   int32_t num_rows, hipStream_t stream) {
  if (n < 0 || hidden <= 0 || hidden % 64 || hidden > 2048) return hipErrorInvalidValue;
  if (action_dim <= 0 || action_dim % 8 || action_dim > kMaxAdim) return hipErrorInvalidValue;
  if (num_rows < 0 || num_rows > kEncMats - 1 || (num_rows > 0 && (!rows || !rows_stats))) return hipErrorInvalidValue;
  EncArgs a{};
  a.k = static_cast<int>(hidden);
  a.adim = static_cast<int>(action_dim);
  int cnt = 0, blocks = 0;
  if (n > 0) {
    if (!act || !w_in || !b_in || !temb || !pos || !packed || !stats) return hipErrorInvalidValue;
    if (!al16(act) || !al16(w_in) || !al16(b_in) || !al16(temb) || !al16(pos) || !al16(packed) ||
        reinterpret_cast<uintptr_t>(stats) % 8)
      return hipErrorInvalidValue;
    if (n > (1 << 24)) return hipErrorInvalidValue;
    a.act = static_cast<const uint16_t*>(act);
    a.w_in = static_cast<const uint16_t*>(w_in);
    a.b_in = static_cast<const uint16_t*>(b_in);
    a.temb = static_cast<const uint16_t*>(temb);
    a.pos = static_cast<const uint16_t*>(pos);
    a.x[0] = nullptr;
    a.out[0] = static_cast<uint16_t*>(packed);
    a.stats[0] = stats;
    a.m[0] = static_cast<int>(n);
    a.begin[0] = 0;
    blocks = static_cast<int>(n);  // one workgroup per action row
    cnt = 1;
  }
  for (int i = 0; i < num_rows; ++i) {
    const rldx_rows_t& r = rows[i];
    if (r.m < 0 || r.k != hidden) return hipErrorInvalidValue;
    if (r.m == 0) continue;
    if (!r.x || !r.packed || !al16(r.x) || !al16(r.packed) || r.ldx < r.k || r.ldx % 8) return hipErrorInvalidValue;
    if (!rows_stats[i] || reinterpret_cast<uintptr_t>(rows_stats[i]) % 8) return hipErrorInvalidValue;
    if (r.m > (1 << 24)) return hipErrorInvalidValue;
    a.x[cnt] = static_cast<const uint16_t*>(r.x);
    a.ldx[cnt] = r.ldx;
    a.out[cnt] = static_cast<uint16_t*>(r.packed);
    a.stats[cnt] = rows_stats[i];
    a.m[cnt] = static_cast<int>(r.m);
    a.begin[cnt] = blocks;
    blocks += static_cast<int>((r.m + 3) / 4);
    ++cnt;
  }
  if (cnt == 0) return hipSuccess;
  a.count = cnt;
  a.begin[cnt] = blocks;
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  if (hidden <= 512)
    hipLaunchKernelGGL(encode_pack_kernel<1>, grid, block, 0, stream, a);
  else if (hidden <= 1024)
    hipLaunchKernelGGL(encode_pack_kernel<2>, grid, block, 0, stream, a);
  else if (hidden <= 1536)
    hipLaunchKernelGGL(encode_pack_kernel<3>, grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL(encode_pack_kernel<4>, grid, block, 0, stream, a);
  return hipGetLastError();
}

extern "C" hipError_t rldx_action_decode_euler_bf16(const void* packed, int64_t n, int64_t hidden, float eps,
                                                    const void* w_out, const void* b_out, int64_t action_dim,
                                                    float dt, void* act, hipStream_t stream) {
  if (n < 0 || hidden <= 0 || hidden % 64 || hidden > 2048) return hipErrorInvalidValue;
  if (action_dim <= 0 || action_dim % 8 || action_dim > kMaxAdim) return hipErrorInvalidValue;
  if (!(eps >= 0.f) || !(dt == dt)) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  if (!packed || !w_out || !b_out || !act || !al16(packed) || !al16(w_out) || !al16(act) ||
      reinterpret_cast<uintptr_t>(b_out) % 2)
    return hipErrorInvalidValue;
  if (n > (1 << 24)) return hipErrorInvalidValue;
  DecArgs a{static_cast<const uint16_t*>(packed), static_cast<const uint16_t*>(w_out),
            static_cast<const uint16_t*>(b_out), static_cast<uint16_t*>(act), static_cast<int>(n),
            static_cast<int>(hidden), static_cast<int>(action_dim), eps, dt};
  hipLaunchKernelGGL(decode_euler_kernel, dim3(static_cast<unsigned>(n)), dim3(256), 0, stream, a);
  return hipGetLastError();
}
