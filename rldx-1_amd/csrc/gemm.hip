// Grouped bf16 GEMM for the linears of an MSAT block on gfx950 (CDNA4):
//   y_s = x_s W_s^T + b_s  for up to 3 streams s in one launch, fp32 accumulation
// on v_mfma_f32_32x32x16_bf16, with the block's epilogues fused:
//   bias            out = bf16(y)                                (nn.Linear)
//   residual        out = bf16(res + bf16(y))                    (x_s += Proj_s(o_s), x_s += W3_s(...))
//   SwiGLU          out = swiglu(bf16(y_gate), bf16(y_up))       (W12_s followed by SwiGLU),
//                   row-major or in the packed activation order (the next GEMM's A)
// The rounding points are those of the eager chain (addmm to bf16, then the
// bf16 add / SwiGLU), rldx/model/modules/action_model/blocks.py:705-891 and
// rldx/model/modules/action_model/ops.py:137-161.  The SwiGLU epilogue replaces
// _fused_mlp_swiglu_kernel behind ss::fused_mlp_swiglu
// (rldx/inference/action_model/single_stream/engine/kernels/fused_mlp_swiglu.py:199-267).
//
// Design
//   * Weights are static, so they are packed once (pack_weight_kernel) into the
//     MFMA B-operand order: 1 KB chunk (nb, kb) holds W[32 nb + l%32][16 kb +
//     8 (l/32) + i] for lane l, element i, and the chunks of one 32-column block
//     are contiguous along K.  Every weight load is one coalesced 16-byte load
//     per lane; a wave streams its K range of a column block front to back.
//   * A workgroup computes a (32*MB rows) x (32*NB columns) tile; its 4 waves
//     split K into quarters (no operand is loaded twice inside a workgroup) and
//     the partial accumulators are reduced through LDS in a fixed order, so the
//     result is deterministic.
//   * Activations are read in the same packed operand order (chunk (mb, kb) =
//     rows 32 mb.., k 16 kb..), written so by their producers (the LayerNorm
//     pack kernel below, the attention kernel's packed output, the SwiGLU
//     epilogue): a row-major A costs 32 cache lines per load instruction and
//     measured 2-4x slower.
//   * Operands go straight from memory into VGPRs, double-buffered U k-steps
//     deep: the next stage's loads are in flight during the current stage's
//     MFMAs.  The activations (a few hundred KB) stay in L2; the weights stream
//     from HBM once per workgroup row.
//   * MB = 4 (128-row tiles) for the 512-token cognition stream, whose GEMMs are
//     MFMA-bound; MB = 2 for the 64 / 32-token action and physics streams, whose
//     GEMMs are weight-streaming (HBM-bound).  Work items are mapped XCD-aware:
//     the m-tiles of one column block run on one XCD and share its L2.
#include "rldx_amd.h"
#include "rldx_common.h"

namespace rldx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kXcds = 8;
constexpr int kWaves = 4;
constexpr int kBufWord3 = 0x00020000;  // gfx9 raw buffer descriptor, word 3 (untyped dword data)

enum { kEpiBias = 0, kEpiResidual = 1, kEpiSwiglu = 2, kEpiSwigluPacked = 3 };


__device__ __forceinline__ float bf(uint16_t b) { return bf16_bits_to_f32(b); }

// W [n, k] (row stride ldw) -> packed 1 KB chunks (nb, kb), nb-major.  With
// swiglu_pairs, packed block 2p holds W rows 32p.. (gate) and block 2p+1 rows
// n/2 + 32p.. (up), so one workgroup tile holds matching gate / up columns.
__global__ __launch_bounds__(256) void pack_weight_kernel(const uint16_t* __restrict__ w, int64_t ldw, int n, int k,
                                                          int swiglu_pairs, uint16_t* __restrict__ out) {
  const int kbs = k / 16;
  const int64_t chunk = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (chunk >= static_cast<int64_t>(n / 32) * kbs) return;
  const int lane = threadIdx.x & 63;
  const int nb = static_cast<int>(chunk / kbs), kb = static_cast<int>(chunk % kbs);
  const int row = swiglu_pairs ? (nb & 1) * (n / 2) + 32 * (nb >> 1) + (lane & 31) : 32 * nb + (lane & 31);
  const u32x4 v = *reinterpret_cast<const u32x4*>(w + static_cast<int64_t>(row) * ldw + 16 * kb + 8 * (lane >> 5));
  *reinterpret_cast<u32x4*>(out + chunk * 512 + lane * 8) = v;
}

struct Group {
  const uint16_t* a;  // packed activations
  int m;
  const uint16_t* w;
  const uint16_t* bias;
  uint16_t* out;
  int64_t ldo;
  const uint16_t* res;
  int64_t ldr;
};

struct GemmArgs {
  Group g[3];
  int num_groups;
  int n, k;           // n = rows of W (2 * N_half with the SwiGLU epilogue)
  int m_tiles[3];
  int item_end[3];    // cumulative work items per group
};

template <int MB, int NB, int U, int EPI>
__global__ __launch_bounds__(256, 1) void gemm_kernel(GemmArgs a) {
  static_assert((EPI != kEpiSwiglu && EPI != kEpiSwigluPacked) || NB % 2 == 0, "SwiGLU tiles pair gate / up blocks");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;

  // XCD-aware work mapping (workgroup i runs on XCD i % 8): consecutive items —
  // the m-tiles of one column block — land on one XCD.
  int item;
  {
    const int total = static_cast<int>(gridDim.x);
    const int i = static_cast<int>(blockIdx.x);
    const int per = total / kXcds, rem = total % kXcds;
    const int xcd = i % kXcds, kk = i / kXcds;
    item = xcd < rem ? xcd * (per + 1) + kk : rem * (per + 1) + (xcd - rem) * per + kk;
  }
  int gi = 0;
  if (a.num_groups > 1 && item >= a.item_end[0]) gi = 1;
  if (a.num_groups > 2 && item >= a.item_end[1]) gi = 2;
  const Group& G = a.g[gi];
  const int local = item - (gi ? a.item_end[gi - 1] : 0);
  const int mt = local % a.m_tiles[gi], nt = local / a.m_tiles[gi];
  const int ksteps = a.k / 16;
  const int kw = ksteps / kWaves;  // k-steps of this wave
  const int kb0 = wave * kw;

  // Buffer descriptors: per-lane 32-bit offsets, the k-stage offset in an SGPR
  // and the k-step within a stage as an immediate, so a load costs no VALU.
  const int mblocks = (G.m + 31) / 32;
  const __amdgpu_buffer_rsrc_t ar =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(G.a), 0, mblocks * ksteps * 1024, kBufWord3);
  int aoff[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)  // m-blocks past the end re-read the last one (rows never stored)
    aoff[mb] = (min(mt * MB + mb, mblocks - 1) * ksteps + kb0) * 1024 + lane * 16;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(G.w + static_cast<int64_t>(nt * NB) * ksteps * 512), 0, NB * ksteps * 1024, kBufWord3);
  const int woff = lane * 16;

  floatx16 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = floatx16{};

  u32x4 wa[U][NB], xa[U][MB], wb[U][NB], xb[U][MB];
  // Workgroups start their K walk at different stages (rotated by column tile):
  // the activation chunks are shared by every column tile, and workgroups that
  // walk K in lockstep request the same chunk at the same time, all from one
  // L2 channel.  The summation order stays fixed per tile.
  const int stages = kw / U;
  const int rot = nt % stages;
  auto load = [&](u32x4(&w)[U][NB], u32x4(&x)[U][MB], int st) {  // st: stage in walk order
    int sr = st + rot;
    if (sr >= stages) sr -= stages;
    const int kb = sr * U;  // first k-step of the stage, wave-relative
    const int ks = kb0 + kb;
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        w[u][nb] = __builtin_amdgcn_raw_buffer_load_b128(wr, woff + u * 1024, (nb * ksteps + ks) * 1024, 0);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) x[u][mb] = __builtin_amdgcn_raw_buffer_load_b128(ar, aoff[mb] + u * 1024, kb * 1024, 0);
    }
  };
  auto mma = [&](u32x4(&w)[U][NB], u32x4(&x)[U][MB]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x[u][mb]),
                                                                __builtin_bit_cast(bf16x8, w[u][nb]), acc[mb][nb], 0,
                                                                0, 0);
  };
  // Stages of U k-steps, double-buffered.  The scheduling barriers keep each
  // stage's loads ahead of the previous stage's MFMAs (the scheduler would
  // otherwise sink them next to their uses).  A load past the last stage
  // re-reads the last stage (in bounds, never used).
  load(wa, xa, 0);

  // Epilogue operands, fetched behind the first stage so their latency hides
  // under the K loop: the bias of the output columns this wave finalises, and
  // the residual chunks of this thread's 16-byte stores (each chunk is read and
  // written by the same thread, so the residual may alias the output).
  constexpr bool kSwiglu = EPI == kEpiSwiglu || EPI == kEpiSwigluPacked;
  constexpr int TR = MB * 32;                      // tile rows
  constexpr int TC = kSwiglu ? NB * 16 : NB * 32;  // tile output columns
  constexpr int BLK = MB * NB;
  // epilogue work units per wave: 32x32 blocks, or for SwiGLU (gate, up) block
  // pairs split into their 4 row quarters (the SwiGLU math is the costly part)
  constexpr int UNITS = kSwiglu ? (BLK / 2) * 4 : BLK;
  constexpr int PER_WAVE = (UNITS + kWaves - 1) / kWaves;
  constexpr int NCHUNK = (TR * TC / 8 + 255) / 256;  // 16-byte output chunks per thread
  // (raw bf16 bits: converting here would make the loads' results needed, and
  // with in-order load counters wait for the first stage too)
  uint16_t pb0[PER_WAVE], pb1[PER_WAVE];
#pragma unroll
  for (int j = 0; j < PER_WAVE; ++j) {
    const int id = wave + j * kWaves;
    pb0[j] = pb1[j] = 0;
    if constexpr (kSwiglu) {
      if (G.bias && id < UNITS) {
        const int col = 32 * (nt * (NB / 2) + (id / 4) % (NB / 2)) + l32;
        pb0[j] = G.bias[col];
        pb1[j] = G.bias[a.n / 2 + col];
      }
    } else {
      if (G.bias && id < BLK) pb0[j] = G.bias[32 * (nt * NB + id % NB) + l32];
    }
  }
  u32x4 pres[NCHUNK];
  if constexpr (EPI == kEpiResidual) {
#pragma unroll
    for (int j = 0; j < NCHUNK; ++j) {
      const int t = static_cast<int>(threadIdx.x) + 256 * j;
      const int row = mt * TR + t / (TC / 8), col = nt * TC + 8 * (t % (TC / 8));
      pres[j] = (t < TR * TC / 8 && row < G.m)
                    ? *reinterpret_cast<const u32x4*>(G.res + static_cast<int64_t>(row) * G.ldr + col)
                    : u32x4{0, 0, 0, 0};
    }
  }

  int st = 0;
  for (; st + 2 <= stages; st += 2) {
    load(wb, xb, min(st + 1, stages - 1));
    __builtin_amdgcn_sched_barrier(0);
    mma(wa, xa);
    __builtin_amdgcn_sched_barrier(0);
    load(wa, xa, min(st + 2, stages - 1));
    __builtin_amdgcn_sched_barrier(0);
    mma(wb, xb);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (st < stages) mma(wa, xa);

  // ---- reduce the 4 waves' partial tiles through LDS, in wave order ----
  __shared__ floatx4 red[kWaves * BLK * 4 * 64];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        red[((wave * BLK + mb * NB + nb) * 4 + q4) * 64 + lane] =
            floatx4{acc[mb][nb][4 * q4], acc[mb][nb][4 * q4 + 1], acc[mb][nb][4 * q4 + 2], acc[mb][nb][4 * q4 + 3]};
  __syncthreads();
  auto reduced = [&](int blk, int q4) {
    floatx4 s = red[(blk * 4 + q4) * 64 + lane];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) s += red[((w * BLK + blk) * 4 + q4) * 64 + lane];
    return s;
  };
  // ---- epilogue: bias / SwiGLU on the reduced sums -> bf16 tile in LDS ->
  // 16-byte, row-contiguous stores (a 2-byte store per accumulator element
  // scatters every store instruction over 2-8 segments; measured to cost more
  // than the whole K loop) ----
  constexpr int OP = TC + 8;                       // LDS row pitch in elements (16-byte multiple)
  __shared__ __attribute__((aligned(16))) uint16_t otile[TR * OP];
  if constexpr (kSwiglu) {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int u = wave + j * kWaves;
      if (u >= UNITS) break;
      const int pi = u / 4, q4 = u % 4;
      const int mb = pi / (NB / 2), pp = pi % (NB / 2);
      const float bg = bf(pb0[j]), bu = bf(pb1[j]);
      const floatx4 sg = reduced(mb * NB + 2 * pp, q4), su = reduced(mb * NB + 2 * pp + 1, q4);
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        const uint32_t gp = pack_bf16x2(sg[e] + bg, sg[e + 1] + bg);
        const uint32_t up = pack_bf16x2(su[e] + bu, su[e + 1] + bu);
        const uint32_t y = swiglu_bf16x2(bf16x2_lo(gp), bf16x2_hi(gp), bf16x2_lo(up), bf16x2_hi(up));
        otile[(32 * mb + 8 * q4 + 4 * g + e) * OP + 32 * pp + l32] = static_cast<uint16_t>(y);
        otile[(32 * mb + 8 * q4 + 4 * g + e + 1) * OP + 32 * pp + l32] = static_cast<uint16_t>(y >> 16);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int blk = wave + j * kWaves;
      if (blk >= BLK) break;
      const int mb = blk / NB, nb = blk % NB;
      const float bias = bf(pb0[j]);
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const floatx4 s = reduced(blk, q4);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          otile[(32 * mb + 8 * q4 + 4 * g + e) * OP + 32 * nb + l32] = f32_to_bf16_bits(s[e] + bias);
      }
    }
  }
  __syncthreads();
  const int row0 = mt * TR, col0 = nt * TC;
#pragma unroll
  for (int j = 0; j < NCHUNK; ++j) {
    const int t = static_cast<int>(threadIdx.x) + 256 * j;
    const int r = t / (TC / 8), c = 8 * (t % (TC / 8));
    const int row = row0 + r, col = col0 + c;
    if (t >= TR * TC / 8 || row >= G.m) continue;
    u32x4 v = *reinterpret_cast<const u32x4*>(&otile[r * OP + c]);
    if constexpr (EPI == kEpiResidual) {
      const u32x4 rv = pres[j];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = f32_to_bf16_bits(bf(static_cast<uint16_t>(rv[i] & 0xffffu)) + bf(static_cast<uint16_t>(v[i] & 0xffffu)));
        const uint32_t hi = f32_to_bf16_bits(bf(static_cast<uint16_t>(rv[i] >> 16)) + bf(static_cast<uint16_t>(v[i] >> 16)));
        v[i] = lo | (hi << 16);
      }
    }
    if constexpr (EPI == kEpiSwigluPacked)
      *reinterpret_cast<u32x4*>(G.out + packed_act_offset(row, col, a.n / 2)) = v;
    else
      *reinterpret_cast<u32x4*>(G.out + static_cast<int64_t>(row) * G.ldo + col) = v;
  }
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int MB, int NB, int U>
hipError_t launch_groups(const rldx_gemm_group_t* gs, const int* idx, int count, int64_t n, int64_t k, int epi,
                         hipStream_t stream) {
  if (count == 0) return hipSuccess;
  GemmArgs a{};
  a.num_groups = count;
  a.n = static_cast<int>(n);
  a.k = static_cast<int>(k);
  const int n_tiles = static_cast<int>(n / (32 * NB));
  int64_t items = 0;
  for (int j = 0; j < count; ++j) {
    const rldx_gemm_group_t& s = gs[idx[j]];
    a.g[j] = Group{static_cast<const uint16_t*>(s.a_packed), static_cast<int>(s.m),
                   static_cast<const uint16_t*>(s.w_packed), static_cast<const uint16_t*>(s.bias),
                   static_cast<uint16_t*>(s.out), s.ldo, static_cast<const uint16_t*>(s.residual), s.ldr};
    a.m_tiles[j] = static_cast<int>((s.m + 32 * MB - 1) / (32 * MB));
    items += static_cast<int64_t>(a.m_tiles[j]) * n_tiles;
    if (items > (int64_t{1} << 31) - 1) return hipErrorInvalidValue;
    a.item_end[j] = static_cast<int>(items);
  }
  const dim3 grid(static_cast<unsigned>(items)), block(256);
  if (epi == kEpiBias)
    hipLaunchKernelGGL((gemm_kernel<MB, NB, U, kEpiBias>), grid, block, 0, stream, a);
  else if (epi == kEpiResidual)
    hipLaunchKernelGGL((gemm_kernel<MB, NB, U, kEpiResidual>), grid, block, 0, stream, a);
  else if constexpr (NB % 2 == 0) {
    if (epi == kEpiSwiglu)
      hipLaunchKernelGGL((gemm_kernel<MB, NB, U, kEpiSwiglu>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((gemm_kernel<MB, NB, U, kEpiSwigluPacked>), grid, block, 0, stream, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Row-major activations -> packed operand order, optionally through a
// LayerNorm without affine parameters (the MSAT block pre-norm,
// rldx/model/modules/action_model/blocks.py:705-891 with nn.LayerNorm(dim,
// elementwise_affine=False, eps)): y = (x - mean) * rsqrt(var + eps), mean and
// biased variance in fp32 (two passes over the row held in registers), rounded
// once to bf16 — F.layer_norm's arithmetic on bf16 input.
// One wave per row; lane j holds columns 8 (j + 64 c) .. +7.
// ---------------------------------------------------------------------------
template <int CPL>
__global__ __launch_bounds__(256) void rows_pack_kernel(const uint16_t* __restrict__ x, int64_t ldx, int m, int k,
                                                        float eps, int normalize, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= m) return;
  const uint16_t* xr = x + static_cast<int64_t>(row) * ldx;
  u32x4 raw[CPL];
  float v[CPL][8];
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = 8 * (lane + 64 * c);
    raw[c] = col < k ? *reinterpret_cast<const u32x4*>(xr + col) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[c][i] = bf(static_cast<uint16_t>((i & 1) ? (raw[c][i >> 1] >> 16) : (raw[c][i >> 1] & 0xffffu)));
      sum += v[c][i];
    }
  }
  if (normalize) {
#pragma clang fp contract(off)
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
    const float mean = sum / static_cast<float>(k);
    float sq = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c)
      if (8 * (lane + 64 * c) < k)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float d = v[c][i] - mean;
          sq += d * d;
        }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sq += __shfl_xor(sq, o, 64);
    const float rstd = 1.0f / __builtin_sqrtf(sq / static_cast<float>(k) + eps);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        const uint32_t lo = f32_to_bf16_bits((v[c][i] - mean) * rstd);
        const uint32_t hi = f32_to_bf16_bits((v[c][i + 1] - mean) * rstd);
        raw[c][i >> 1] = lo | (hi << 16);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = 8 * (lane + 64 * c);
    if (col < k) *reinterpret_cast<u32x4*>(out + packed_act_offset(row, col, k)) = raw[c];
  }
}

hipError_t rows_pack(const void* x, int64_t ldx, int64_t m, int64_t k, float eps, bool normalize, void* packed,
                     hipStream_t stream) {
  if (m < 0 || k < 0) return hipErrorInvalidValue;
  if (m == 0 || k == 0) return hipSuccess;
  if (!x || !packed || !a16(x) || !a16(packed) || ldx < k || ldx % 8 || k % 16) return hipErrorInvalidValue;
  if (m > (int64_t{1} << 30)) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>((m + 3) / 4)), block(256);
  const auto* xp = static_cast<const uint16_t*>(x);
  auto* op = static_cast<uint16_t*>(packed);
  const int mi = static_cast<int>(m), ki = static_cast<int>(k), nz = normalize ? 1 : 0;
  if (k <= 512)
    hipLaunchKernelGGL(rows_pack_kernel<1>, grid, block, 0, stream, xp, ldx, mi, ki, eps, nz, op);
  else if (k <= 1024)
    hipLaunchKernelGGL(rows_pack_kernel<2>, grid, block, 0, stream, xp, ldx, mi, ki, eps, nz, op);
  else if (k <= 2048)
    hipLaunchKernelGGL(rows_pack_kernel<4>, grid, block, 0, stream, xp, ldx, mi, ki, eps, nz, op);
  else if (k <= 4096)
    hipLaunchKernelGGL(rows_pack_kernel<8>, grid, block, 0, stream, xp, ldx, mi, ki, eps, nz, op);
  else if (k <= 8192)
    hipLaunchKernelGGL(rows_pack_kernel<16>, grid, block, 0, stream, xp, ldx, mi, ki, eps, nz, op);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace
}  // namespace rldx

using namespace rldx;

extern "C" hipError_t rldx_gemm_pack_weight_bf16(const void* w, int64_t ldw, int64_t n, int64_t k,
                                                 int32_t swiglu_pairs, void* packed, hipStream_t stream) {
  if (n < 0 || k < 0) return hipErrorInvalidValue;
  if (n == 0 || k == 0) return hipSuccess;
  if (!w || !packed || !a16(w) || !a16(packed) || ldw < k || ldw % 8) return hipErrorInvalidValue;
  if (n % (swiglu_pairs ? 64 : 32) != 0 || k % 16 != 0) return hipErrorInvalidValue;
  const int64_t chunks = n / 32 * (k / 16);
  if (n > (int64_t{1} << 30) || k > (int64_t{1} << 30) || (chunks + 3) / 4 > (int64_t{1} << 31) - 1)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(pack_weight_kernel, dim3(static_cast<unsigned>((chunks + 3) / 4)), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(w), ldw, static_cast<int>(n), static_cast<int>(k),
                     swiglu_pairs ? 1 : 0, static_cast<uint16_t*>(packed));
  return hipGetLastError();
}

extern "C" hipError_t rldx_grouped_gemm_bf16(const rldx_gemm_group_t* groups, int32_t num_groups, int64_t n,
                                             int64_t k, int32_t epilogue, hipStream_t stream) {
  if (!groups || num_groups < 1 || num_groups > 3) return hipErrorInvalidValue;
  if (epilogue < kEpiBias || epilogue > kEpiSwigluPacked) return hipErrorInvalidValue;
  // k: whole stages of 8 k-steps per wave; n: whole 64-column tiles
  if (n <= 0 || k <= 0 || n % 64 != 0 || k % (kWaves * 16 * 8) != 0) return hipErrorInvalidValue;
  if (n > (1 << 30) || k > (1 << 30)) return hipErrorInvalidValue;
  const bool swiglu = epilogue == kEpiSwiglu || epilogue == kEpiSwigluPacked;
  const int64_t n_out = swiglu ? n / 2 : n;
  int order[3], cnt = 0;
  for (int i = 0; i < num_groups; ++i) {
    const rldx_gemm_group_t& s = groups[i];
    if (s.m < 0 || s.m > (1 << 24)) return hipErrorInvalidValue;
    if (s.m == 0) continue;
    if (!s.a_packed || !s.w_packed || !s.out || !a16(s.a_packed) || !a16(s.w_packed)) return hipErrorInvalidValue;
    // packed operands are addressed with 32-bit byte offsets
    if ((s.m + 31) / 32 * 32 * k * 2 > (int64_t{1} << 31) - 1 || n * k * 2 > (int64_t{1} << 31) - 1)
      return hipErrorInvalidValue;
    // the epilogue stores (and reads the residual) in 16-byte pieces
    if (!a16(s.out) || (s.bias && reinterpret_cast<uintptr_t>(s.bias) % 2)) return hipErrorInvalidValue;
    if (epilogue != kEpiSwigluPacked && (s.ldo < n_out || s.ldo % 8)) return hipErrorInvalidValue;
    if (epilogue == kEpiResidual && (!s.residual || !a16(s.residual) || s.ldr < n_out || s.ldr % 8))
      return hipErrorInvalidValue;
    order[cnt++] = i;
  }
  // One launch for all groups, smallest first: the weight-streaming tiles of
  // the short streams are dispatched first and overlap the MFMA-bound tiles of
  // the long one.  64 x 64 tiles: measured best for the MSAT shapes (enough
  // workgroups to fill 256 CUs twice over, two workgroups per CU).
  for (int i = 1; i < cnt; ++i)
    for (int j = i; j > 0 && groups[order[j]].m < groups[order[j - 1]].m; --j) {
      const int t = order[j];
      order[j] = order[j - 1];
      order[j - 1] = t;
    }
  return launch_groups<2, 2, 4>(groups, order, cnt, n, k, epilogue, stream);
}

extern "C" int64_t rldx_act_packed_elems(int64_t m, int64_t k) {
  if (m < 0 || k < 0) return -1;
  return (m + 31) / 32 * 32 * k;
}

extern "C" hipError_t rldx_act_pack_bf16(const void* x, int64_t ldx, int64_t m, int64_t k, void* packed,
                                         hipStream_t stream) {
  return rows_pack(x, ldx, m, k, 0.f, false, packed, stream);
}

extern "C" hipError_t rldx_layernorm_pack_bf16(const void* x, int64_t ldx, int64_t m, int64_t k, float eps,
                                               void* packed, hipStream_t stream) {
  return rows_pack(x, ldx, m, k, eps, true, packed, stream);
}
