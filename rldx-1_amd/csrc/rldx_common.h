// Shared device/host helpers for the rldx_amd HIP kernels (gfx950 / CDNA4).
//
// Everything here is written for one target: AMD CDNA4, wave64.  The numeric
// helpers are __host__ __device__ so that the very same IEEE operation
// sequence can be executed on the CPU (exhaustive self-checks) and on the GPU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define RLDX_HD __host__ __device__ __forceinline__

namespace rldx {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// bf16 <-> fp32 (bit-level, round-to-nearest-even, NaN quieted).  PyTorch's
// c10::BFloat16 conversion uses the same rule, so rounding here is identical to
// what eager bf16 tensors do after every op.
// ---------------------------------------------------------------------------
RLDX_HD float bf16_bits_to_f32(uint16_t b) {
  uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

RLDX_HD uint16_t f32_to_bf16_bits(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

RLDX_HD float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// ---------------------------------------------------------------------------
// exp(a) with |error| < 1 ulp on the range where silu needs it.
//
// Cody-Waite reduction a = n*ln2 + r (|r| <= ~0.347), degree-7 Taylor
// polynomial evaluated by Horner with explicit fmaf, exact scaling by 2^n via
// ldexpf.  Truncation error r^8/8! < 5.3e-9 relative; the final fma rounds
// once, so the total stays below one ulp.  All steps are explicit IEEE
// operations (no contraction is left to the compiler), so host and device
// produce identical bits.
// ---------------------------------------------------------------------------
RLDX_HD float exp_f32_1ulp(float a) {
#pragma clang fp contract(off)
  if (a > 88.72283935546875f) return __builtin_inff();
  if (a < -104.0f) return 0.0f;
  const float kLog2e = 1.44269502162933349609375f;
  const float kLn2Hi = 0.693145751953125f;           // 0x3f317200: 12 significant bits
  const float kLn2Lo = 1.428606765330187045e-06f;    // ln2 - kLn2Hi
  float n = __builtin_rintf(a * kLog2e);
  float r = __builtin_fmaf(-n, kLn2Hi, a);
  r = __builtin_fmaf(-n, kLn2Lo, r);
  float p = 1.98412698412698412526e-4f;              // 1/5040
  p = __builtin_fmaf(p, r, 1.38888888888888894189e-3f);  // 1/720
  p = __builtin_fmaf(p, r, 8.33333333333333321769e-3f);  // 1/120
  p = __builtin_fmaf(p, r, 4.16666666666666643537e-2f);  // 1/24
  p = __builtin_fmaf(p, r, 1.66666666666666657415e-1f);  // 1/6
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, static_cast<int>(n));
}

// silu(x) = x / (1 + exp(-x)) in fp32, the formula PyTorch's silu kernel uses
// for reduced-precision inputs (opmath float).  IEEE division (HIP's default
// correctly-rounded fp32 divide).
RLDX_HD float silu_f32(float x) {
#pragma clang fp contract(off)
  float e = exp_f32_1ulp(-x);
  float d = 1.0f + e;
  return x / d;
}

// Eager bf16 SwiGLU element: y = bf16( bf16(silu(g)) * u ), two roundings,
// exactly as `F.silu(x1) * x2` on bf16 tensors.  The product of two bf16
// values is exact in fp32, so the only rounding-sensitive step is silu.
RLDX_HD uint16_t swiglu_bf16_bits(uint16_t g, uint16_t u) {
#pragma clang fp contract(off)
  float s = round_bf16(silu_f32(bf16_bits_to_f32(g)));
  return f32_to_bf16_bits(s * bf16_bits_to_f32(u));
}

// ---------------------------------------------------------------------------
// Device SwiGLU with the hardware exp2 / reciprocal, bit-identical to
// swiglu_bf16_bits.
//
// Only the bf16 rounding of silu reaches the output, so silu may be evaluated
// by any method whose fp32 value rounds like silu_f32's.  The fast form is
// x * rcp(1 + exp2(-x log2e)) with v_exp_f32 and v_rcp_f32 (1 ulp each);
// log2e = kL2eHi + lo, kL2eHi holding 16 significant bits so that x * kL2eHi
// is exact for the 8-bit significand of a bf16 x, and exp2(-x lo) is applied
// to first order (|x lo ln2| < 4e-4 for |x| <= 80).  Over every bf16 x with
// |x| <= 80 the fast value lies within 5 ulps of silu_f32's, with either
// hardware op off by one ulp in either direction.  Where it lies within
// kSiluFastMargin ulps of a bf16 rounding midpoint (low 16 bits 0x8000), or
// x is outside [-80, 80] (inf and NaN included), silu_f32 is evaluated
// instead; elsewhere no midpoint separates the two values and both round to
// the same bf16.  About 1 element in 2000 takes the exact branch.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// (lo, hi) -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
// Cache-policy immediate of a buffer load / store at device scope: SC1 = 1,
// SC0 = 0 (the instruction's own access is coherent across the XCDs' L2s).
constexpr int kCpolDevice = 16;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ float bf16x2_lo(uint32_t p) { return __builtin_bit_cast(float, p << 16); }
__device__ __forceinline__ float bf16x2_hi(uint32_t p) { return __builtin_bit_cast(float, p & 0xffff0000u); }

constexpr uint32_t kSiluFastMargin = 16;

__device__ __forceinline__ float silu_bf16_input(float x) {
#pragma clang fp contract(off)
  const float kL2eHi = 1.44268798828125f;            // log2(e) to 16 significant bits
  const float kL2eLoLn2 = 4.888495368504664e-06f;    // (log2(e) - kL2eHi) * ln(2)
  const float e1 = __builtin_amdgcn_exp2f(x * -kL2eHi);
  const float e = __builtin_fmaf(e1, x * -kL2eLoLn2, e1);
  float s = x * __builtin_amdgcn_rcpf(1.0f + e);
  const uint32_t b = __builtin_bit_cast(uint32_t, s);
  const bool near_mid = static_cast<uint16_t>(b + (kSiluFastMargin - 0x8000u)) <= 2 * kSiluFastMargin;
  if (__builtin_expect(near_mid || !(__builtin_fabsf(x) <= 80.0f), 0)) s = silu_f32(x);
  return s;
}

// Two SwiGLU elements: g0, g1, u0, u1 are bf16 values held as fp32; returns
// the packed bf16 pair bf16(bf16(silu(g)) * u), as swiglu_bf16_bits.
__device__ __forceinline__ uint32_t swiglu_bf16x2(float g0, float g1, float u0, float u1) {
#pragma clang fp contract(off)
  const uint32_t s = pack_bf16x2(silu_bf16_input(g0), silu_bf16_input(g1));
  return pack_bf16x2(bf16x2_lo(s) * u0, bf16x2_hi(s) * u1);
}

// Unsigned 32-bit division by an invariant divisor d >= 1 (Granlund and
// Montgomery, "Division by invariant integers using multiplication", PLDI
// 1994, figure 4.1): q = (t + ((n - t) >> sh1)) >> sh2 with t = mulhi(m, n),
// exact for every 32-bit n.
struct DivMagic {
  uint32_t m, sh1, sh2;
};

inline DivMagic div_magic(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t{1} << l) < d) ++l;
  DivMagic r;
  r.m = static_cast<uint32_t>((uint64_t{1} << 32) * ((uint64_t{1} << l) - d) / d + 1);
  r.sh1 = l < 1 ? l : 1;
  r.sh2 = l < 1 ? 0 : l - 1;
  return r;
}

__device__ __forceinline__ uint32_t div_u32(uint32_t n, const DivMagic& dm) {
  const uint32_t t = __umulhi(dm.m, n);
  return (t + ((n - t) >> dm.sh1)) >> dm.sh2;
}

// Element offset of A[row][col] in the packed activation order (the A operand
// of the grouped GEMM) of a matrix with k columns: 1 KB chunk (row / 32,
// col / 16), lane row % 32 + 32 * (col / 8 % 2), element col % 8.
RLDX_HD int64_t packed_act_offset(int64_t row, int64_t col, int64_t k) {
  return ((row >> 5) * (k >> 4) + (col >> 4)) * 512 + ((row & 31) + 32 * ((col >> 3) & 1)) * 8 + (col & 7);
}

// Host-side launcher shared between translation units (rmsnorm_rope.hip).
hipError_t gqa_k_norm_rope_kv_pack(const uint16_t* k, const uint16_t* v, int64_t row_stride, const uint16_t* k_w,
                                   const uint16_t* cos, const uint16_t* sin, int64_t cos_row_stride, bool sin_signed,
                                   int64_t seq, int64_t kv_heads, int64_t head_dim, float eps, uint16_t* kvp,
                                   int64_t kvp_sh, hipStream_t stream);

// Element offset of K[key][d0 .. d0+7] (d0 % 8 == 0) inside the packed K/V
// tiles of one head (32 keys per tile, 128 * D bytes, K chunks then V chunks):
// tile key / 32, 1 KB chunk d0 / 16, lane key % 32 + 32 * (d0 / 8 % 2).
RLDX_HD int64_t packed_k_offset(int64_t key, int d0, int D) {
  const int lane = static_cast<int>(key & 31) + 32 * ((d0 >> 3) & 1);
  return (key >> 5) * (64 * D) + ((d0 >> 4) * 64 + lane) * 8;
}

// Memory-side-cache warm-up carried by extra workgroups of a launch: up to
// three byte ranges, `end` the cumulative counts of their whole 128-byte lines.
struct WarmRanges {
  const uint32_t* ptr[3];
  int64_t end[3];
  int64_t per_wg;  // lines per warm-up workgroup
};

// Warm-up workgroup w (of `nthreads` threads) reads one dword of each of its
// lines: plain loads (they allocate in the memory-side cache on the way;
// non-temporal loads measured no warm-up), 8 per thread in flight, the results
// folded into a register that an empty asm statement consumes (no stores, no
// LDS, no barrier).
__device__ __forceinline__ void warm_lines(const WarmRanges& wr, int w, int nthreads) {
  const int64_t l0 = w * wr.per_wg, l1 = min(l0 + wr.per_wg, wr.end[2]);
  uint32_t acc = 0;
  for (int64_t base = l0 + static_cast<int>(threadIdx.x); base < l1; base += 8 * nthreads) {
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t l = base + j * nthreads;
      const int r = l < wr.end[0] ? 0 : l < wr.end[1] ? 1 : 2;
      const int64_t rb = r == 0 ? 0 : wr.end[r - 1];
      v[j] = l < l1 ? wr.ptr[r][(l - rb) * 32] : 0u;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= v[j];
  }
  asm volatile("" ::"v"(acc));
}

// Host: validates up to three ranges (4-byte aligned, non-negative lengths) and
// fills `wr` (per_wg left 0); returns false on a bad argument.
inline bool warm_ranges(const void* const* ptrs, const int64_t* bytes, int32_t count, WarmRanges& wr) {
  wr = WarmRanges{};
  if (count < 0 || count > 3 || (count > 0 && (!ptrs || !bytes))) return false;
  int64_t lines = 0;
  for (int i = 0; i < count; ++i) {
    if (bytes[i] < 0 || (bytes[i] > 0 && (!ptrs[i] || reinterpret_cast<uintptr_t>(ptrs[i]) % 4))) return false;
    wr.ptr[i] = static_cast<const uint32_t*>(ptrs[i]);
    lines += bytes[i] / 128;
    wr.end[i] = lines;
  }
  for (int i = count; i < 3; ++i) {
    wr.ptr[i] = wr.ptr[0];
    wr.end[i] = lines;
  }
  return lines <= (int64_t{1} << 40);
}

}  // namespace rldx
