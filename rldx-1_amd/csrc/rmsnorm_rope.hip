// Fused per-head RMSNorm + rotary embedding for gfx950.
//
// Two conventions live on the RLDX-1 inference path and both are here:
//
//  * rotate-half (Qwen3-VL text attention):
//      y   = w * to_dtype(x * rsqrt(mean(x^2) + eps))
//      out = y*cos + rotate_half(y)*sin,  rotate_half(y) = cat(-y[D/2:], y[:D/2])
//    rldx/model/modules/backbone/modeling_qwen3_vl.py:118-122 (rotate_half),
//    :356-371 (Qwen3VLTextRMSNorm), :377-401 (apply_rotary_pos_emb).
//
//  * interleaved (MSAT joint attention, Llama/complex style), per stream:
//      y   = to_bf16( float(w) * (x * rsqrt(mean(x^2) + eps)) )    (one rounding)
//      (y[2i] + i*y[2i+1]) * (cos_i + i*sin_i), fp32, rounded once to bf16
//    rldx/model/modules/norms.py:18-22 (RMSNorm), action_model/ops.py:48-67
//    (apply_rotary_emb); fused form of the per-stream QKV gather in
//    rldx/inference/action_model/double_stream/engine/kernels/rmsnorm_rope_ds.py:11-231
//    and rmsnorm_rope_ds_3way.py:22-386.
//
// Layout: one row (token, head) of D elements is owned by a group of
// D*sizeof(T)/16 lanes, each holding 16 contiguous bytes (128-bit loads and
// stores).  The sum of squares is reduced with xor-shuffles inside the group;
// the rotate-half partner d +- D/2 lives in lane (i ^ group/2), one shuffle;
// interleaved pairs (2i, 2i+1) are adjacent inside a lane, no shuffle at all.
#include "rldx_amd.h"
#include "rldx_common.h"

namespace rldx {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Vec16;
template <>
struct Vec16<float> {
  static constexpr int N = 4;
};
template <>
struct Vec16<uint16_t> {
  static constexpr int N = 8;
};

template <typename T>
__device__ __forceinline__ float load_elem(const T* p, int i);
template <>
__device__ __forceinline__ float load_elem<float>(const float* p, int i) { return p[i]; }
template <>
__device__ __forceinline__ float load_elem<uint16_t>(const uint16_t* p, int i) { return bf16_bits_to_f32(p[i]); }

__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, kWave); }

// ---------------------------------------------------------------------------
// rotate-half (Qwen) variant
// ---------------------------------------------------------------------------
struct HalfArgs {
  const void* q;
  const void* k;
  const void* q_w;
  const void* k_w;
  const void* cos;
  const void* sin;
  void* q_out;
  void* k_out;
  int64_t batch, seq, hq, hk;
  int64_t q_sb, q_ss, q_sh;    // input strides (elements)
  int64_t k_sb, k_ss, k_sh;
  int64_t qo_sb, qo_ss, qo_sh; // output strides
  int64_t ko_sb, ko_ss, ko_sh;
  int64_t c_sb, c_ss;          // cos/sin strides ([B or 1, S, D])
  float eps;
  int sin_signed;              // sin table already carries the rotate_half sign
  int no_norm;                 // RoPE only (apply_rotary_pos_emb): no RMSNorm, no weights
  int64_t total_rows;          // batch * seq * (hq + hk); total_rows * D / V < 2^31
  DivMagic per_tok_div;        // division by hq + hk
  DivMagic seq_div;            // division by seq
  // Packed K/V mode (kernel template PK; bf16, batch 1, K heads only, R == 1):
  // K rows go into the attention kernels' packed K/V tiles of head h at
  // kvp + h * kvp_sh, and workgroups [norm_blocks, norm_blocks + hk * kv_tiles)
  // pack the V tiles from v (row stride v_ss, head stride v_sh) and zero the K
  // rows of the padding keys.
  uint16_t* kvp;
  int64_t kvp_sh, norm_blocks, kv_tiles;
  const uint16_t* v;
  int64_t v_ss, v_sh;
};

// One 32-key tile of the packed K/V layout (32 keys, 128 * D bytes: K operand
// chunks, then V operand chunks) at dst: V rows k0 .. k0 + 31 (vrow(m) points at
// V[m][0 .. D), keys >= m_total read as zeros) go to the V chunks; the K rows of
// keys >= m_total are zeroed (the K rows of real keys are written by the norm
// role).  V chunk 2 db + s2, lane l, element i holds
// V[k0 + 16 s2 + 8 (i / 4) + 4 (l / 32) + i % 4][32 db + l % 32].
template <int D, class RowFn>
__device__ void kv_tile_pack(RowFn vrow, int64_t m_total, int64_t k0, uint16_t* dst) {
  constexpr int PITCH = D + 8;
  constexpr int CH = D / 8;    // 16-byte chunks per V row
  constexpr int NCH = D / 16;  // 1 KB chunks per part of a tile
  __shared__ __attribute__((aligned(16))) uint16_t tile[32 * PITCH];
  for (int c = threadIdx.x; c < 32 * CH; c += blockDim.x) {
    const int r = c / CH, col = (c % CH) * 8;
    const int64_t m = k0 + r;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (m < m_total) val = *reinterpret_cast<const uint4*>(vrow(m) + col);
    *reinterpret_cast<uint4*>(&tile[r * PITCH + col]) = val;
  }
  for (int idx = threadIdx.x; idx < NCH * 64; idx += blockDim.x)
    if (k0 + (idx & 31) >= m_total) *reinterpret_cast<uint4*>(dst + idx * 8) = make_uint4(0, 0, 0, 0);
  __syncthreads();
  for (int idx = threadIdx.x; idx < NCH * 64; idx += blockDim.x) {
    const int cc = idx >> 6, l = idx & 63;
    const int d = 32 * (cc >> 1) + (l & 31);
    const int rb = 16 * (cc & 1) + 4 * (l >> 5);
    uint4 out;
    uint32_t* ow = reinterpret_cast<uint32_t*>(&out);
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const int r0 = rb + 8 * (i >> 2) + (i & 3);
      ow[i >> 1] = static_cast<uint32_t>(tile[r0 * PITCH + d]) | (static_cast<uint32_t>(tile[(r0 + 1) * PITCH + d]) << 16);
    }
    *reinterpret_cast<uint4*>(dst + NCH * 512 + idx * 8) = out;
  }
}

// One thread: V consecutive elements of R heads of one token (the R heads
// share the token's cos / sin and, within q or within k, the norm weight, so
// those are loaded once for R rows).  R divides both hq and hk.
// NTL / NTS (large launches): non-temporal loads of the rows / stores of the
// results (read once, written once; the memory-side cache keeps what the
// rest of the launch reuses: cos / sin and the norm weights).
template <typename T, int D, int R, bool PK = false, bool NTL = false, bool NTS = false>
__global__ __launch_bounds__(256) void rmsnorm_rope_half_kernel(HalfArgs a) {
  constexpr int V = Vec16<T>::N;   // elements per lane
  constexpr int LPR = D / V;       // lanes per row
  static_assert(LPR >= 2 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "unsupported head_dim");
  static_assert(!PK || (sizeof(T) == 2 && R == 1), "packed K/V mode: bf16, one head per thread");
  if constexpr (PK) {
    if (static_cast<int64_t>(blockIdx.x) >= a.norm_blocks) {  // a V tile (whole workgroups take this branch)
      const int64_t vb = static_cast<int64_t>(blockIdx.x) - a.norm_blocks;
      const int64_t h = vb / a.kv_tiles, t = vb - h * a.kv_tiles;
      const uint16_t* vh = a.v + h * a.v_sh;
      kv_tile_pack<D>([&](int64_t m) { return vh + m * a.v_ss; }, a.seq, t * 32, a.kvp + h * a.kvp_sh + t * (64 * D));
      return;
    }
  }
  // 32-bit index math with invariant-divisor multiplies (a 64-bit division by
  // a run-time value costs ~130 instructions, more than the rows' arithmetic)
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  const int lane_in_row = static_cast<int>(tid % LPR);
  const uint32_t item = tid / LPR;  // (token, group of R heads)
  const bool valid = item < a.total_rows / R;
  const uint32_t r = valid ? item * R : 0u;  // first row of the group

  const uint32_t per_tok = static_cast<uint32_t>(a.hq + a.hk);
  const uint32_t tok = div_u32(r, a.per_tok_div);
  const int64_t hh = r - tok * per_tok;
  const uint32_t b32 = div_u32(tok, a.seq_div);
  const int64_t b = b32;
  const int64_t s = tok - b32 * static_cast<uint32_t>(a.seq);
  const bool is_q = hh < a.hq;  // the whole group: R divides hq
  const int64_t h = is_q ? hh : hh - a.hq;

  const T* src = is_q ? static_cast<const T*>(a.q) + b * a.q_sb + s * a.q_ss + h * a.q_sh
                      : static_cast<const T*>(a.k) + b * a.k_sb + s * a.k_ss + h * a.k_sh;
  const int64_t src_h = is_q ? a.q_sh : a.k_sh;
  T* dst = is_q ? static_cast<T*>(a.q_out) + b * a.qo_sb + s * a.qo_ss + h * a.qo_sh
                : static_cast<T*>(a.k_out) + b * a.ko_sb + s * a.ko_ss + h * a.ko_sh;
  const int64_t dst_h = is_q ? a.qo_sh : a.ko_sh;
  const T* w = static_cast<const T*>(is_q ? a.q_w : a.k_w);
  const T* cs = static_cast<const T*>(a.cos) + b * a.c_sb + s * a.c_ss;
  const T* sn = static_cast<const T*>(a.sin) + b * a.c_sb + s * a.c_ss;
  const int d0 = lane_in_row * V;

  // every load of the thread is issued before any arithmetic
  uint4 raw[R];
#pragma unroll
  for (int j = 0; j < R; ++j)
    raw[j] = !valid ? make_uint4(0, 0, 0, 0)
             : NTL ? __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + j * src_h + d0)))
                   : *reinterpret_cast<const uint4*>(src + j * src_h + d0);
  const uint4 wraw = a.no_norm ? make_uint4(0, 0, 0, 0) : *reinterpret_cast<const uint4*>(w + d0);
  const uint4 craw = *reinterpret_cast<const uint4*>(cs + d0);
  const uint4 sraw = *reinterpret_cast<const uint4*>(sn + d0);
  const T* we = reinterpret_cast<const T*>(&wraw);
  const T* ce = reinterpret_cast<const T*>(&craw);
  const T* se = reinterpret_cast<const T*>(&sraw);
  const bool first_half = lane_in_row < LPR / 2;

#pragma unroll
  for (int j = 0; j < R; ++j) {
    float x[V];
    const T* e = reinterpret_cast<const T*>(&raw[j]);
#pragma unroll
    for (int i = 0; i < V; ++i) x[i] = load_elem<T>(e, i);
    float y[V];
    if (a.no_norm) {  // (uniform) RoPE of the input as it is
#pragma unroll
      for (int i = 0; i < V; ++i) y[i] = x[i];
    } else {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < V; ++i) ss += x[i] * x[i];
#pragma unroll
      for (int m = LPR / 2; m >= 1; m >>= 1) ss += shfl_xor_f(ss, m);
      {
#pragma clang fp contract(off)
        const float rinv = 1.0f / __builtin_sqrtf(ss * (1.0f / D) + a.eps);
#pragma unroll
        for (int i = 0; i < V; ++i) {
          float xn = x[i] * rinv;
          if constexpr (sizeof(T) == 2) {
            // w * bf16(xn): bf16 x bf16 product, rounded to bf16.
            y[i] = round_bf16(load_elem<T>(we, i) * round_bf16(xn));
          } else {
            y[i] = load_elem<T>(we, i) * xn;
          }
        }
      }
    }
    // rotate_half partner: element d +- D/2 sits in lane (lane_in_row ^ LPR/2).
    float part[V];
#pragma unroll
    for (int i = 0; i < V; ++i) part[i] = shfl_xor_f(y[i], LPR / 2);

    uint4 outraw;
    T* o = reinterpret_cast<T*>(&outraw);
    {
#pragma clang fp contract(off)
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float rot = (first_half && !a.sin_signed) ? -part[i] : part[i];
        const float c = load_elem<T>(ce, i);
        const float sv = load_elem<T>(se, i);
        if constexpr (sizeof(T) == 2) {
          const float t1 = round_bf16(y[i] * c);
          const float t2 = round_bf16(rot * sv);
          o[i] = f32_to_bf16_bits(t1 + t2);
        } else {
          const float t1 = y[i] * c;
          const float t2 = rot * sv;
          o[i] = t1 + t2;
        }
      }
    }
    if constexpr (PK) {
      if (valid) *reinterpret_cast<uint4*>(a.kvp + h * a.kvp_sh + packed_k_offset(s, d0, D)) = outraw;
    } else {
      if (valid) {
        if constexpr (NTS)
          __builtin_nontemporal_store(__builtin_bit_cast(u32x4, outraw), reinterpret_cast<u32x4*>(dst + j * dst_h + d0));
        else
          *reinterpret_cast<uint4*>(dst + j * dst_h + d0) = outraw;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MSAT multi-stream interleaved variant
// ---------------------------------------------------------------------------
struct MsatStream {
  const uint16_t* qkv;   // [n, >= 3*H*D] bf16 packed Q|K|V
  int64_t ld;            // row stride (elements)
  int64_t n;             // rows
  int64_t m_begin;       // first row in the joint sequence
  const uint16_t* q_w;   // [D] bf16
  const uint16_t* k_w;   // [D] bf16
  const float* cos;      // [n, D/2] fp32 or nullptr (no rotary on this stream)
  const float* sin;
  int64_t rope_ld;       // row stride of cos/sin (elements)
  int64_t b_step;        // elements from one batch entry's rows to the next's
};

typedef float floatx4 __attribute__((ext_vector_type(4)));

struct MsatArgs {
  MsatStream s[3];
  int num_streams;
  int64_t heads;
  int64_t m_total;
  uint16_t* q_out;  // (B, H, M, D) with strides
  uint16_t* k_out;
  uint16_t* v_out;
  int64_t o_sb, o_sh, o_sm;  // output strides (batch, head, row) in elements, shared by q/k/v
  float eps;
  int64_t total_items;  // rows of D handled by the norm/copy role: 3*H*M, or 2*H*M with kvp
  // optional packed K/V tiles of the attention kernels (32 keys per tile, 128*D
  // bytes, K operand chunks then V operand chunks, keys >= M zero): K rows are
  // scattered into them by the norm role; V and the K padding are written by
  // workgroups [qk_blocks, qk_blocks + H * kv_tiles)
  uint16_t* kvp;
  int64_t kvp_sb, kvp_sh;  // batch / head strides in elements
  int64_t qk_blocks;
  int64_t kv_tiles;  // 32-token tiles per head
  // 32-bit index math of the norm role (host-checked: its threads < 2^31)
  uint32_t per_kind;  // m_total * heads
  DivMagic dm_kind, dm_heads;
};

template <int D>
__device__ void msat_kv_pack_block(const MsatArgs& a, int64_t vb, int64_t b) {
  const int64_t h = vb / a.kv_tiles;
  const int64_t t = vb - h * a.kv_tiles;
  const int64_t inner = a.heads * D;
  auto vrow = [&](int64_t m) {
    int si = 0;
    if (a.num_streams > 1 && m >= a.s[1].m_begin) si = 1;
    if (a.num_streams > 2 && m >= a.s[2].m_begin) si = 2;
    const MsatStream& S = a.s[si];
    return S.qkv + b * S.b_step + (m - S.m_begin) * S.ld + 2 * inner + h * D;
  };
  kv_tile_pack<D>(vrow, a.m_total, t * 32, a.kvp + b * a.kvp_sb + h * a.kvp_sh + t * (64 * D));
}

template <int D>
__global__ __launch_bounds__(256) void msat_qkv_norm_rope_kernel(MsatArgs a) {
  constexpr int V = 8;
  constexpr int LPR = D / V;
  static_assert(LPR >= 2 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "unsupported head_dim");
  const int64_t b = blockIdx.y;  // batch entry
  if (a.kvp != nullptr && static_cast<int64_t>(blockIdx.x) >= a.qk_blocks) {
    msat_kv_pack_block<D>(a, static_cast<int64_t>(blockIdx.x) - a.qk_blocks, b);
    return;
  }
  // 32-bit index math with invariant-divisor multiplies (a 64-bit division by
  // the run-time row / head counts costs a few hundred instructions per thread)
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  const int lane_in_row = static_cast<int>(tid % LPR);
  const uint32_t item = tid / LPR;
  const bool valid = item < static_cast<uint64_t>(a.total_items);
  const uint32_t it = valid ? item : 0;
  // item -> (which, m, h); h fastest so a wave walks consecutive heads of one token.
  const uint32_t which = div_u32(it, a.dm_kind);  // 0=q 1=k 2=v
  const uint32_t rem = it - which * a.per_kind;
  const uint32_t m = div_u32(rem, a.dm_heads);
  const uint32_t h = rem - m * static_cast<uint32_t>(a.heads);
  int si = 0;
  if (a.num_streams > 1 && m >= a.s[1].m_begin) si = 1;
  if (a.num_streams > 2 && m >= a.s[2].m_begin) si = 2;
  const MsatStream& S = a.s[si];
  const int64_t row = static_cast<int64_t>(m) - S.m_begin;
  const int64_t inner = a.heads * D;
  const int d0 = lane_in_row * V;
  const uint16_t* src = S.qkv + b * S.b_step + row * S.ld + which * inner + static_cast<int64_t>(h) * D + d0;
  uint16_t* dst = (a.kvp != nullptr && which == 1)
                      ? a.kvp + b * a.kvp_sb + h * a.kvp_sh + packed_k_offset(m, d0, D)
                      : (which == 0 ? a.q_out : which == 1 ? a.k_out : a.v_out) + b * a.o_sb + h * a.o_sh +
                            m * a.o_sm + d0;

  uint4 raw = valid ? *reinterpret_cast<const uint4*>(src) : make_uint4(0, 0, 0, 0);
  if (which == 2) {  // V passthrough (uniform per row group, but shuffles below need all lanes)
    if (valid) *reinterpret_cast<uint4*>(dst) = raw;
  }
  const uint32_t* e = reinterpret_cast<const uint32_t*>(&raw);
  float x[V];
#pragma unroll
  for (int i = 0; i < V / 2; ++i) {
    x[2 * i] = bf16x2_lo(e[i]);
    x[2 * i + 1] = bf16x2_hi(e[i]);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) ss += x[i] * x[i];
#pragma unroll
  for (int mm = LPR / 2; mm >= 1; mm >>= 1) ss += shfl_xor_f(ss, mm);
  if (which == 2 || !valid) return;

  const uint4 wraw = *reinterpret_cast<const uint4*>((which == 0 ? S.q_w : S.k_w) + d0);
  const uint32_t* wv = reinterpret_cast<const uint32_t*>(&wraw);
  float y[V];
  {
#pragma clang fp contract(off)
    const float rinv = 1.0f / __builtin_sqrtf(ss * (1.0f / D) + a.eps);
#pragma unroll
    for (int i = 0; i < V / 2; ++i) {
      // y = bf16(w * (x * rinv)) (one rounding, RNE)
      const uint32_t yp = pack_bf16x2(bf16x2_lo(wv[i]) * (x[2 * i] * rinv), bf16x2_hi(wv[i]) * (x[2 * i + 1] * rinv));
      y[2 * i] = bf16x2_lo(yp);
      y[2 * i + 1] = bf16x2_hi(yp);
    }
  }
  uint4 outraw;
  uint32_t* o = reinterpret_cast<uint32_t*>(&outraw);
  if (S.cos != nullptr) {
#pragma clang fp contract(off)
    const floatx4 c = *reinterpret_cast<const floatx4*>(S.cos + row * S.rope_ld + d0 / 2);
    const floatx4 sn = *reinterpret_cast<const floatx4*>(S.sin + row * S.rope_ld + d0 / 2);
#pragma unroll
    for (int p = 0; p < V / 2; ++p) {
      const float re = y[2 * p], im = y[2 * p + 1];
      const float ore = re * c[p] - im * sn[p];
      const float oim = re * sn[p] + im * c[p];
      o[p] = pack_bf16x2(ore, oim);
    }
  } else {
#pragma unroll
    for (int p = 0; p < V / 2; ++p) o[p] = pack_bf16x2(y[2 * p], y[2 * p + 1]);
  }
  *reinterpret_cast<uint4*>(dst) = outraw;
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename T, int D>
hipError_t launch_half_d(const HalfArgs& a, hipStream_t stream) {
  constexpr int V = Vec16<T>::N;
  // Small launches are latency-bound: one head per thread, the most
  // parallelism.  Large launches (measured on MI355X, fp32 q / k [1, S, 16, 64],
  // outputs bit-identical in every variant):
  //  * rows that fit the 256 MB memory-side cache (16K tokens, 134 MB in):
  //    4 heads per thread (fewer loads per element) and non-temporal stores,
  //    46.3 -> 41.1 us (0.84 of 8 TB/s; a plain torch.neg of the same bytes
  //    40.6 us); non-temporal loads there lose (47 us: the rows of a repeated
  //    call are served from that cache);
  //  * larger rows (64K tokens, 537 MB in): 2 heads per thread, non-temporal
  //    loads and stores, 199.6 -> 174.3 us (0.79; torch.neg 180 us); 4 heads
  //    184 us, 8 heads 187 us, 1 head 198 us.
  const bool large = a.total_rows * (D / V) >= (int64_t{1} << 21);
  const bool past_cache = a.total_rows * D * static_cast<int64_t>(sizeof(T)) > (int64_t{256} << 20);
  const bool by2 = a.hq % 2 == 0 && a.hk % 2 == 0, by4 = a.hq % 4 == 0 && a.hk % 4 == 0;
  const int R = !large ? 1 : past_cache ? (by2 ? 2 : 1) : by4 ? 4 : by2 ? 2 : 1;
  const int64_t threads = a.total_rows / R * (D / V);
  const int grid = static_cast<int>((threads + 255) / 256);
  if (grid == 0) return hipSuccess;
  if (!large)
    hipLaunchKernelGGL((rmsnorm_rope_half_kernel<T, D, 1>), dim3(grid), dim3(256), 0, stream, a);
  else if (past_cache && R == 2)
    hipLaunchKernelGGL((rmsnorm_rope_half_kernel<T, D, 2, false, true, true>), dim3(grid), dim3(256), 0, stream, a);
  else if (past_cache)
    hipLaunchKernelGGL((rmsnorm_rope_half_kernel<T, D, 1, false, true, true>), dim3(grid), dim3(256), 0, stream, a);
  else if (R == 4)
    hipLaunchKernelGGL((rmsnorm_rope_half_kernel<T, D, 4, false, false, true>), dim3(grid), dim3(256), 0, stream, a);
  else if (R == 2)
    hipLaunchKernelGGL((rmsnorm_rope_half_kernel<T, D, 2, false, false, true>), dim3(grid), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((rmsnorm_rope_half_kernel<T, D, 1, false, false, true>), dim3(grid), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_half(const HalfArgs& a, int64_t head_dim, hipStream_t stream) {
  if (head_dim == 64) return launch_half_d<T, 64>(a, stream);
  if (head_dim == 128) return launch_half_d<T, 128>(a, stream);
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t half_entry(const void* q, const void* k, const void* q_w, const void* k_w, const void* cos,
                      const void* sin, void* q_out, void* k_out, int64_t batch, int64_t seq, int64_t hq,
                      int64_t hk, int64_t head_dim, const int64_t* q_strides, const int64_t* k_strides,
                      const int64_t* qo_strides, const int64_t* ko_strides, const int64_t* cs_strides, float eps,
                      int32_t flags, hipStream_t stream) {
  if (head_dim != 64 && head_dim != 128) return hipErrorInvalidValue;
  if (batch < 0 || seq < 0 || hq < 0 || hk < 0) return hipErrorInvalidValue;
  if (!q_strides || !k_strides || !qo_strides || !ko_strides || !cs_strides) return hipErrorInvalidValue;
  if (batch == 0 || seq == 0 || hq + hk == 0) return hipSuccess;
  if (!cos || !sin) return hipErrorInvalidValue;
  if (flags & ~(RLDX_ROPE_SIN_SIGNED | RLDX_ROPE_NO_NORM)) return hipErrorInvalidValue;
  const bool no_norm = (flags & RLDX_ROPE_NO_NORM) != 0;
  if (hq > 0 && (!q || (!q_w && !no_norm) || !q_out)) return hipErrorInvalidValue;
  if (hk > 0 && (!k || (!k_w && !no_norm) || !k_out)) return hipErrorInvalidValue;
  const int V = Vec16<T>::N;
  const void* ptrs[] = {q, k, q_out, k_out, cos, sin, q_w, k_w};
  for (const void* p : ptrs)
    if (p && !al16(p)) return hipErrorInvalidValue;
  const int64_t* all[] = {q_strides, k_strides, qo_strides, ko_strides};
  for (const int64_t* st : all)
    for (int i = 0; i < 3; ++i)
      if (st[i] % V != 0) return hipErrorInvalidValue;
  if (cs_strides[0] % V != 0 || cs_strides[1] % V != 0) return hipErrorInvalidValue;
  const int64_t rows = batch * seq * (hq + hk);
  if (rows * (head_dim / V) >= (int64_t{1} << 31) - 256) return hipErrorInvalidValue;
  HalfArgs a{q, k, q_w, k_w, cos, sin, q_out, k_out, batch, seq, hq, hk,
             q_strides[0], q_strides[1], q_strides[2], k_strides[0], k_strides[1], k_strides[2],
             qo_strides[0], qo_strides[1], qo_strides[2], ko_strides[0], ko_strides[1], ko_strides[2],
             cs_strides[0], cs_strides[1], eps, (flags & RLDX_ROPE_SIN_SIGNED) ? 1 : 0, no_norm ? 1 : 0,
             rows, div_magic(static_cast<uint32_t>(hq + hk)), div_magic(static_cast<uint32_t>(seq))};
  return launch_half<T>(a, head_dim, stream);
}

}  // namespace

// K of a GQA prefill (rows [seq] of stride row_stride, head h at k + h * D):
// RMSNorm + rotate-half RoPE straight into the packed K/V tiles, and the V tiles
// (v + h * D) packed by further workgroups of the same launch.  Arguments are
// validated by the caller (rldx_llm_fused_attention_bf16).
hipError_t gqa_k_norm_rope_kv_pack(const uint16_t* k, const uint16_t* v, int64_t row_stride, const uint16_t* k_w,
                                   const uint16_t* cos, const uint16_t* sin, int64_t cos_row_stride, bool sin_signed,
                                   int64_t seq, int64_t kv_heads, int64_t head_dim, float eps, uint16_t* kvp,
                                   int64_t kvp_sh, hipStream_t stream) {
  const int64_t rows = seq * kv_heads;
  if (rows * (head_dim / 8) >= (int64_t{1} << 31) - 256 || kv_heads > 65535) return hipErrorInvalidValue;
  HalfArgs a{};
  a.k = k;
  a.k_w = k_w;
  a.cos = cos;
  a.sin = sin;
  a.batch = 1;
  a.seq = seq;
  a.hq = 0;
  a.hk = kv_heads;
  a.k_ss = row_stride;
  a.k_sh = head_dim;
  a.c_ss = cos_row_stride;
  a.eps = eps;
  a.sin_signed = sin_signed ? 1 : 0;
  a.total_rows = rows;
  a.per_tok_div = div_magic(static_cast<uint32_t>(kv_heads));
  a.seq_div = div_magic(static_cast<uint32_t>(seq));
  a.kvp = kvp;
  a.kvp_sh = kvp_sh;
  a.kv_tiles = (seq + 31) / 32;
  a.v = v;
  a.v_ss = row_stride;
  a.v_sh = head_dim;
  a.norm_blocks = (rows * (head_dim / 8) + 255) / 256;
  const int64_t grid = a.norm_blocks + kv_heads * a.kv_tiles;
  if (grid > (int64_t{1} << 31) - 1) return hipErrorInvalidValue;
  if (head_dim == 64)
    hipLaunchKernelGGL((rmsnorm_rope_half_kernel<uint16_t, 64, 1, true>), dim3(static_cast<unsigned>(grid)), dim3(256),
                       0, stream, a);
  else if (head_dim == 128)
    hipLaunchKernelGGL((rmsnorm_rope_half_kernel<uint16_t, 128, 1, true>), dim3(static_cast<unsigned>(grid)),
                       dim3(256), 0, stream, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace rldx

using namespace rldx;

extern "C" hipError_t rldx_qk_rmsnorm_rope_half_f32(
    const float* q, const float* k, const float* q_w, const float* k_w, const float* cos, const float* sin,
    float* q_out, float* k_out, int64_t batch, int64_t seq, int64_t q_heads, int64_t k_heads, int64_t head_dim,
    const int64_t* q_strides, const int64_t* k_strides, const int64_t* q_out_strides,
    const int64_t* k_out_strides, const int64_t* cos_strides, float eps, int32_t flags, hipStream_t stream) {
  return half_entry<float>(q, k, q_w, k_w, cos, sin, q_out, k_out, batch, seq, q_heads, k_heads, head_dim,
                           q_strides, k_strides, q_out_strides, k_out_strides, cos_strides, eps, flags, stream);
}

extern "C" hipError_t rldx_qk_rmsnorm_rope_half_bf16(
    const void* q, const void* k, const void* q_w, const void* k_w, const void* cos, const void* sin,
    void* q_out, void* k_out, int64_t batch, int64_t seq, int64_t q_heads, int64_t k_heads, int64_t head_dim,
    const int64_t* q_strides, const int64_t* k_strides, const int64_t* q_out_strides,
    const int64_t* k_out_strides, const int64_t* cos_strides, float eps, int32_t flags, hipStream_t stream) {
  return half_entry<uint16_t>(q, k, q_w, k_w, cos, sin, q_out, k_out, batch, seq, q_heads, k_heads, head_dim,
                              q_strides, k_strides, q_out_strides, k_out_strides, cos_strides, eps, flags, stream);
}

namespace {
hipError_t msat_qkv(const rldx_msat_stream_t* streams, int32_t num_streams, int64_t batch,
                    const int64_t* batch_rows, int64_t heads, int64_t head_dim, void* q_out, void* k_out,
                    void* v_out, int64_t out_batch_stride, int64_t out_head_stride, int64_t out_row_stride,
                    void* kv_packed, int64_t kv_packed_batch_stride, int64_t kv_packed_head_stride, float eps,
                    hipStream_t stream) {
  if (streams == nullptr || num_streams < 1 || num_streams > 3) return hipErrorInvalidValue;
  if (batch < 0 || batch > 65535 || (batch > 1 && !batch_rows)) return hipErrorInvalidValue;
  if (out_batch_stride % 8 || kv_packed_batch_stride % 8) return hipErrorInvalidValue;
  if (batch == 0) return hipSuccess;
  if (head_dim != 64 && head_dim != 128) return hipErrorInvalidValue;
  if (heads <= 0 || !q_out) return hipErrorInvalidValue;
  if (!kv_packed && (!k_out || !v_out)) return hipErrorInvalidValue;
  if (!al16(q_out) || out_head_stride % 8 || out_row_stride % 8) return hipErrorInvalidValue;
  if (!kv_packed && (!al16(k_out) || !al16(v_out))) return hipErrorInvalidValue;
  if (kv_packed && (!al16(kv_packed) || kv_packed_head_stride % 8)) return hipErrorInvalidValue;
  MsatArgs a{};
  int64_t m = 0;
  int k = 0;
  for (int i = 0; i < num_streams; ++i) {
    const rldx_msat_stream_t& s = streams[i];
    if (s.rows < 0 || (batch > 1 && batch_rows[i] < 0)) return hipErrorInvalidValue;
    if (s.rows == 0) continue;
    if (!s.qkv || !s.q_norm_w || !s.k_norm_w || !al16(s.qkv) || !al16(s.q_norm_w) || !al16(s.k_norm_w))
      return hipErrorInvalidValue;
    if (s.qkv_row_stride < 3 * heads * head_dim || s.qkv_row_stride % 8) return hipErrorInvalidValue;
    if ((s.rope_cos == nullptr) != (s.rope_sin == nullptr)) return hipErrorInvalidValue;
    if (s.rope_cos && (!al16(s.rope_cos) || !al16(s.rope_sin) || s.rope_row_stride < head_dim / 2 ||
                       s.rope_row_stride % 4))
      return hipErrorInvalidValue;
    a.s[k] = MsatStream{static_cast<const uint16_t*>(s.qkv), s.qkv_row_stride, s.rows, m,
                        static_cast<const uint16_t*>(s.q_norm_w), static_cast<const uint16_t*>(s.k_norm_w),
                        s.rope_cos, s.rope_sin, s.rope_row_stride,
                        batch > 1 ? batch_rows[i] * s.qkv_row_stride : 0};
    m += s.rows;
    ++k;
  }
  if (k == 0) return hipSuccess;
  a.num_streams = k;
  a.heads = heads;
  a.m_total = m;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.k_out = static_cast<uint16_t*>(k_out);
  a.v_out = static_cast<uint16_t*>(v_out);
  a.o_sb = out_batch_stride;
  a.o_sh = out_head_stride;
  a.o_sm = out_row_stride;
  a.eps = eps;
  a.total_items = (kv_packed ? 2 : 3) * heads * m;
  const int64_t threads = a.total_items * (head_dim / 8);
  a.qk_blocks = (threads + 255) / 256;
  if (a.qk_blocks * 256 + heads * ((m + 31) / 32) * 256 > (int64_t{1} << 31) - 1) return hipErrorInvalidValue;
  a.per_kind = static_cast<uint32_t>(m * heads);
  a.dm_kind = div_magic(a.per_kind);
  a.dm_heads = div_magic(static_cast<uint32_t>(heads));
  a.kvp = static_cast<uint16_t*>(kv_packed);
  a.kvp_sb = kv_packed_batch_stride;
  a.kvp_sh = kv_packed_head_stride;
  a.kv_tiles = (m + 31) / 32;
  if (kv_packed && kv_packed_head_stride < a.kv_tiles * 64 * head_dim) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(a.qk_blocks + (kv_packed ? heads * a.kv_tiles : 0)),
                  static_cast<unsigned>(batch));
  if (head_dim == 64)
    hipLaunchKernelGGL(msat_qkv_norm_rope_kernel<64>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(msat_qkv_norm_rope_kernel<128>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}
}  // namespace

extern "C" hipError_t rldx_msat_qkv_norm_rope_bf16(const rldx_msat_stream_t* streams, int32_t num_streams,
                                                   int64_t heads, int64_t head_dim, void* q_out, void* k_out,
                                                   void* v_out, int64_t out_head_stride, int64_t out_row_stride,
                                                   void* kv_packed, int64_t kv_packed_head_stride, float eps,
                                                   hipStream_t stream) {
  return msat_qkv(streams, num_streams, 1, nullptr, heads, head_dim, q_out, k_out, v_out, 0, out_head_stride,
                  out_row_stride, kv_packed, 0, kv_packed_head_stride, eps, stream);
}

extern "C" hipError_t rldx_msat_qkv_norm_rope_batch_bf16(const rldx_msat_stream_t* streams, int32_t num_streams,
                                                         int64_t batch, const int64_t* stream_batch_rows,
                                                         int64_t heads, int64_t head_dim, void* q_out, void* k_out,
                                                         void* v_out, int64_t out_batch_stride,
                                                         int64_t out_head_stride, int64_t out_row_stride,
                                                         void* kv_packed, int64_t kv_packed_batch_stride,
                                                         int64_t kv_packed_head_stride, float eps,
                                                         hipStream_t stream) {
  return msat_qkv(streams, num_streams, batch, stream_batch_rows, heads, head_dim, q_out, k_out, v_out,
                  out_batch_stride, out_head_stride, out_row_stride, kv_packed, kv_packed_batch_stride,
                  kv_packed_head_stride, eps, stream);
}
