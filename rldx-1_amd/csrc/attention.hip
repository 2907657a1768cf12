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
//   * K and V are read in a packed tile layout (below) in which every MFMA
//     operand of a 32-key tile is one contiguous 1 KB block: lane l reads the
//     16 bytes at l*16.  Operands therefore go straight from global memory into
//     VGPRs with fully coalesced buffer loads (scalar tile offset, constant
//     immediate offsets) — no LDS staging, no swizzle arithmetic, no barrier in
//     the main loop.  The packed copy is written once per K/V by the producing
//     kernel (the MSAT QKV kernel, or `kv_pack_kernel` here), not once per
//     query block.
//   * A workgroup = 32*NSUB queries of one head and 4 waves that split the key
//     range (wave w walks tiles w, w+4, ...); the 4 partial softmax states are
//     merged through LDS at the end.  NSUB = 2 would double the reuse of every
//     loaded K/V operand; the launcher uses NSUB = 1, which fits in 256 VGPRs and
//     68 KB of LDS, so two workgroups share a CU and hide each other's latency.
//   * S^T = K Q^T: A = K operand, B = Q^T kept in VGPRs.  Each lane owns one
//     query column, so the online-softmax max / sum / rescale are lane-local.
//   * O^T = V^T P^T: B = P^T is the exp'd score accumulator packed to bf16; the
//     V part of a packed tile stores the keys in the accumulator's row order.
//   * The next tile's K operands are loaded as soon as the S MFMAs have read the
//     current ones, its V operands as soon as the P.V MFMAs have.
//   * Workgroups are mapped XCD-aware: the query blocks of a head run on one XCD
//     and share its L2.
//   * Softmax in the exp2 domain with the scale folded into one FMA; tiles with
//     no masked key skip all masking; the O / l rescale is lazy (the reference
//     max moves only when a tile max exceeds it by more than 2^8), exact up to
//     rounding because softmax is shift-invariant; the two lanes of a query only
//     exchange their maxima (v_permlane32_swap) when a rescale is due.
//   * P is rounded to bf16 before the P.V product, the same rounding point as
//     the eager CPU flash-attention kernel.
//
// Packed K/V tile t (keys 32t .. 32t+31) of one (batch, kv head), D = head_dim,
// 128*D bytes, tiles of a head contiguous:
//   K part, bytes [0, 64 D):     1 KB chunk ks (0 <= ks < D/16), lane l, element i
//                                = K[32t + (l & 31)][16 ks + 8 (l >> 5) + i]
//   V part, bytes [64 D, 128 D): 1 KB chunk 2 db + s2 (0 <= db < D/32, s2 < 2),
//                                lane l, element i
//                                = V[32t + 16 s2 + 8 (i >> 2) + 4 (l >> 5) + (i & 3)][32 db + (l & 31)]
//   keys >= Sk hold zeros.
#include <algorithm>
#include <mutex>

#include "rldx_amd.h"
#include "rldx_common.h"

namespace rldx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazyThreshold = 8.0f;  // log2 units: rescale only when the max grows by > 2^8
constexpr int kXcds = 8;                // MI355X: 8 XCDs x 32 CUs, one L2 per XCD
constexpr int kTileKeys = 32;
constexpr int kBufWord3 = 0x00020000;   // gfx9 raw buffer descriptor, word 3 (untyped dword data)

__host__ __device__ constexpr int64_t kv_tile_elems(int64_t d) { return 64 * d; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kBufWord3);
}

// max(x of this lane, x of lane ^ 32)
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  return fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(r[0])),
               __builtin_bit_cast(float, static_cast<uint32_t>(r[1])));
}

// x of this lane + x of lane ^ 32
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  return __builtin_bit_cast(float, static_cast<uint32_t>(r[0])) +
         __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}

// The 16 bias values of a lane's S^T accumulator rows: keys key0 + 8*qq + c,
// qq, c in 0..3, with key0 = tile start + 4 * (lane half).
__device__ __forceinline__ void load_bias(floatx4 (&out)[4], __amdgpu_buffer_rsrc_t r, int key0) {
#pragma unroll
  for (int qq = 0; qq < 4; ++qq)
#pragma unroll
    for (int cc = 0; cc < 4; ++cc)
      out[qq][cc] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, key0 * 4 + 32 * qq + 4 * cc, 0, 0));
}

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* kv;  // packed K/V tiles
  uint16_t* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t kv_sb, kv_sh;  // element strides of the packed tiles per batch / kv head
  int64_t o_sb, o_sh, o_ss;
  int64_t o_packed_k;  // > 0: O written as the packed activations of [sq, hq * D] (batch 1)
  // packed O by row segments (o_nseg > 0, any batch): query row r of batch entry
  // b with o_seg_off[s] <= r < o_seg_off[s] + o_seg_rows[s] goes to packed row
  // o_seg_base[s] + b o_seg_rows[s] + r - o_seg_off[s]; rows outside every
  // segment are not stored
  int o_nseg;
  int o_seg_off[3], o_seg_rows[3], o_seg_base[3];
  const float* key_bias;  // [batch, sk] additive (natural-log units) or nullptr
  int64_t kb_sb;
  int hq, hkv, group, sq, sk;
  int num_q_blocks;
  float scale_log2;  // softmax scale * log2(e), > 0
  // fused Q RMSNorm + rotate-half RoPE (Qwen3-VL), used when kQNorm
  const uint16_t* q_norm_w;  // [D] bf16
  const uint16_t* cos;       // [sq, D] bf16
  const uint16_t* sin;       // [sq, D] bf16 (pre-signed if sin_signed)
  int64_t cs_ss;             // row stride of cos/sin
  float eps;
  int sin_signed;
  // variable-length sequences (kVarlen): query / key rows of sequence s are
  // [cu_seqlens[s], cu_seqlens[s+1]) of q / o; its packed K/V tiles start at
  // tile slot seq_slot_base(s) of each head
  const int32_t* cu_seqlens;
  int num_seqs;
  int total_rows;
  int d_store;  // output columns written per head (<= D)
  // the first n_work workgroups compute attention; those after them read the
  // lines of `warm` (rldx_attention_packed_fwd_warm_bf16)
  int n_work;
  WarmRanges warm;
};


// Sequence s of a variable-length batch (rows [c_s, c_{s+1}) with
// c_s = clamp(cu_seqlens[s], 0, rows)) owns the 32-row slots
// [base_s, base_s + ceil(len_s / 32)) with base_s = floor((c_s + 31 s) / 32).
// base_{s+1} - base_s >= ceil(len_s / 32), so the slot ranges of the
// sequences do not overlap, and every slot is below
// floor((rows + 31 num_seqs) / 32) whatever the cu_seqlens values are: no
// scan of cu_seqlens is needed to place a sequence, and a slot finds its
// sequence with one load per lane (up to 63 sequences) or a binary search.
struct SeqSlot {
  int start, len, base;
};

__host__ __device__ constexpr int64_t seq_slot_count(int64_t rows, int64_t num_seqs) {
  return (rows + 31 * num_seqs) / 32;
}

__device__ __forceinline__ int clamp_row(int32_t c, int rows) { return c < 0 ? 0 : (c > rows ? rows : c); }

// Called with the whole wave active.
__device__ __forceinline__ SeqSlot find_seq_slot(const int32_t* cu, int num_seqs, int rows, int slot) {
  if (num_seqs <= 63) {
    // one load per lane: lane s holds c_s (lanes past num_seqs repeat c_num_seqs);
    // the sequence is the last s < num_seqs with base_s <= slot
    const int lane = static_cast<int>(threadIdx.x & 63);
    const int c = clamp_row(cu[min(lane, num_seqs)], rows);
    const int64_t base = (static_cast<int64_t>(c) + 31 * static_cast<int64_t>(lane)) / 32;
    const uint64_t cand = __ballot(lane < num_seqs && base <= slot);
    const int s = cand ? 63 - __builtin_clzll(cand) : 0;
    const int c0 = __builtin_amdgcn_readlane(c, s), c1 = __builtin_amdgcn_readlane(c, s + 1);
    return SeqSlot{c0, c1 > c0 ? c1 - c0 : 0,
                   static_cast<int>((static_cast<int64_t>(c0) + 31 * static_cast<int64_t>(s)) / 32)};
  }
  int lo = 0, hi = num_seqs - 1;  // last s with base_s <= slot (0 when there is none)
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    const int64_t base = (static_cast<int64_t>(clamp_row(cu[mid], rows)) + 31 * static_cast<int64_t>(mid)) / 32;
    if (base <= slot) lo = mid;
    else hi = mid - 1;
  }
  const int c0 = clamp_row(cu[lo], rows), c1 = clamp_row(cu[lo + 1], rows);
  return SeqSlot{c0, c1 > c0 ? c1 - c0 : 0,
                 static_cast<int>((static_cast<int64_t>(c0) + 31 * static_cast<int64_t>(lo)) / 32)};
}

__device__ __forceinline__ float bf(uint16_t b) { return bf16_bits_to_f32(b); }

// Q RMSNorm (Qwen3VLTextRMSNorm: y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))))
// + rotate-half RoPE (bf16(bf16(y * cos) + bf16(rot(y) * sin))) of the
// workgroup's 32 query rows, done once per workgroup: wave w < KS/2 computes
// column chunks w and w + KS/2 (a rotate-half pair, so no other chunk is
// needed) and writes them to `qsh`; after the barrier every wave loads its Q
// operands from there.  Lane holds d = 16*ks + 8*g + i (g = lane half); the
// row sum of squares is over the lane's own D/2 values + those of lane ^ 32.
// Roundings to bf16 use v_cvt_pk_bf16_f32 (round to nearest even).  The chunk
// index is a template parameter: a run-time index into the register array
// would compile to select chains over every chunk.
template <int D, int K0>
__device__ __forceinline__ void qnorm_rope_pair(const bf16x8 (&qreg)[D / 16], const AttnArgs& a, int pos, bool valid,
                                                u32x4* qsh) {
#pragma clang fp contract(off)
  constexpr int KS = D / 16, K1 = K0 + KS / 2;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 5;
  const uint16_t* cr = a.cos + static_cast<int64_t>(valid ? pos : 0) * a.cs_ss + g * 8;
  const uint16_t* sr = a.sin + static_cast<int64_t>(valid ? pos : 0) * a.cs_ss + g * 8;
  const u32x4 w0 = *reinterpret_cast<const u32x4*>(a.q_norm_w + K0 * 16 + g * 8);
  const u32x4 w1 = *reinterpret_cast<const u32x4*>(a.q_norm_w + K1 * 16 + g * 8);
  const u32x4 c0 = *reinterpret_cast<const u32x4*>(cr + K0 * 16), c1 = *reinterpret_cast<const u32x4*>(cr + K1 * 16);
  const u32x4 s0 = *reinterpret_cast<const u32x4*>(sr + K0 * 16), s1 = *reinterpret_cast<const u32x4*>(sr + K1 * 16);
  float ss = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const u32x4 raw = __builtin_bit_cast(u32x4, qreg[ks]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = bf16x2_lo(raw[j]), hi = bf16x2_hi(raw[j]);
      ss += lo * lo;
      ss += hi * hi;
    }
  }
  ss = pair_sum(ss);
  const float rinv = 1.0f / __builtin_sqrtf(ss * (1.0f / D) + a.eps);
  const u32x4 x0 = __builtin_bit_cast(u32x4, qreg[K0]), x1 = __builtin_bit_cast(u32x4, qreg[K1]);
  u32x4 o0, o1;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // y = bf16(w * bf16(x * rinv)) for the two elements of word j of both chunks
    const uint32_t n0 = pack_bf16x2(bf16x2_lo(x0[j]) * rinv, bf16x2_hi(x0[j]) * rinv);
    const uint32_t n1 = pack_bf16x2(bf16x2_lo(x1[j]) * rinv, bf16x2_hi(x1[j]) * rinv);
    const uint32_t y0 = pack_bf16x2(bf16x2_lo(w0[j]) * bf16x2_lo(n0), bf16x2_hi(w0[j]) * bf16x2_hi(n0));
    const uint32_t y1 = pack_bf16x2(bf16x2_lo(w1[j]) * bf16x2_lo(n1), bf16x2_hi(w1[j]) * bf16x2_hi(n1));
    const float y0l = bf16x2_lo(y0), y0h = bf16x2_hi(y0), y1l = bf16x2_lo(y1), y1h = bf16x2_hi(y1);
    // chunk K0 (first half): partner -y1 (+y1 with a pre-signed sin); chunk K1: partner +y0
    const float r0l = a.sin_signed ? y1l : -y1l, r0h = a.sin_signed ? y1h : -y1h;
    const uint32_t t0 = pack_bf16x2(y0l * bf16x2_lo(c0[j]), y0h * bf16x2_hi(c0[j]));
    const uint32_t u0 = pack_bf16x2(r0l * bf16x2_lo(s0[j]), r0h * bf16x2_hi(s0[j]));
    const uint32_t t1 = pack_bf16x2(y1l * bf16x2_lo(c1[j]), y1h * bf16x2_hi(c1[j]));
    const uint32_t u1 = pack_bf16x2(y0l * bf16x2_lo(s1[j]), y0h * bf16x2_hi(s1[j]));
    o0[j] = pack_bf16x2(bf16x2_lo(t0) + bf16x2_lo(u0), bf16x2_hi(t0) + bf16x2_hi(u0));
    o1[j] = pack_bf16x2(bf16x2_lo(t1) + bf16x2_lo(u1), bf16x2_hi(t1) + bf16x2_hi(u1));
  }
  qsh[K0 * 64 + lane] = o0;
  qsh[K1 * 64 + lane] = o1;
}

template <int D>
__device__ __forceinline__ void qnorm_rope_shared(bf16x8 (&qreg)[D / 16], const AttnArgs& a, int pos, bool valid,
                                                  int wave, u32x4* qsh) {
  constexpr int KS = D / 16;
  static_assert(KS / 2 <= 4, "one rotate-half chunk pair per wave");
  if (wave == 0) qnorm_rope_pair<D, 0>(qreg, a, pos, valid, qsh);
  else if (wave == 1) qnorm_rope_pair<D, 1>(qreg, a, pos, valid, qsh);
  else if constexpr (KS / 2 > 2) {
    if (wave == 2) qnorm_rope_pair<D, 2>(qreg, a, pos, valid, qsh);
    else if (wave == 3) qnorm_rope_pair<D, 3>(qreg, a, pos, valid, qsh);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qreg[ks] = __builtin_bit_cast(bf16x8, qsh[ks * 64 + lane]);
}

// Non-negative integer quotient a / b of wave-uniform operands, b >= 1.  For
// a < 2^22 a float estimate is within 1 of the quotient (v_rcp_f32 is within
// 1 ulp, the product rounds once more), so one correction step each way makes
// it exact; larger a take the integer division.  The work decode of the
// attention kernel needs four of these: the integer divisions by run-time
// values cost ~0.45 us per workgroup.
__device__ __forceinline__ int div_small(int a, int b) {
  if (a >= (1 << 22)) return a / b;
  int q = static_cast<int>(static_cast<float>(a) * __builtin_amdgcn_rcpf(static_cast<float>(b)));
  const int r = a - q * b;
  if (r >= b) ++q;
  else if (r < 0) --q;
  return q;
}

// Wait until at most N of this wave's vector-memory loads are in flight, then
// barrier.  Inline assembly: the compiler does not track the loads that write
// LDS directly (buffer_load ... lds).
template <int N>
__device__ __forceinline__ void vm_wait_barrier() {
  static_assert(N == 4 || N == 6 || N == 8, "vmcnt immediate: the V loads of the first tile");
  if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (N == 6) asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int D, int NSUB, bool kCausal, bool kBias, bool kQNorm, bool kVarlen = false>
__global__ __launch_bounds__(256, 1) void attn_fwd_kernel(AttnArgs a) {
  static_assert(NSUB == 1, "32-query workgroups");
  static_assert(!kVarlen || (!kCausal && !kBias && !kQNorm),
                "variable-length mode: no mask, no fused Q normalisation");
  constexpr int NW = 4;           // waves per workgroup; each walks its own key tiles
  constexpr int BN = kTileKeys;   // keys per tile
  constexpr int KSTEPS = D / 16;  // MFMA k-steps over head_dim for S^T
  constexpr int DBLK = D / 32;    // 32-row blocks of O^T
  constexpr int TILE_BYTES = 128 * D;
  constexpr int VPART = 64 * D;
  constexpr int G4 = DBLK * 4 + 1;  // float4 groups per lane in the merge: O + (m, l)
  __shared__ floatx4 merge[NW * G4 * 64];
  __shared__ u32x4 qsh[KSTEPS * 64];  // the workgroup's Q operands, loaded once and read by every wave
  if (static_cast<int>(blockIdx.x) >= a.n_work) {  // warm-up workgroups (no barrier, no LDS)
    warm_lines(a.warm, static_cast<int>(blockIdx.x) - a.n_work, 256);
    return;
  }

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;

  // XCD-aware work mapping.  Workgroups are dispatched round-robin over the 8
  // XCDs (workgroup i runs on XCD i % 8), each with its own L2.  Work items are
  // ordered (batch, head, query block) — heads sharing a KV head are adjacent —
  // and cut into 8 contiguous ranges, one per XCD, so the K/V of a head is
  // fetched into a single L2 and reused there by all of its query blocks.
  int qb, h, b;
  {
    const int total = a.n_work;
    const int i = static_cast<int>(blockIdx.x);
    const int per = total / kXcds, rem = total % kXcds;
    const int xcd = i % kXcds, k = i / kXcds;
    const int p = xcd < rem ? xcd * (per + 1) + k : rem * (per + 1) + (xcd - rem) * per + k;
    const int nqb = a.num_q_blocks;
    const int ph = __builtin_amdgcn_readfirstlane(div_small(p, nqb));  // batch * hq + head
    const int qi = p - ph * nqb;
    qb = kCausal ? nqb - 1 - qi : qi;  // causal: longest query blocks first on each XCD
    b = __builtin_amdgcn_readfirstlane(div_small(ph, a.hq));
    h = ph - b * a.hq;
  }
  // Query / key range of the workgroup: the whole batch entry, or (kVarlen)
  // the sequence that owns 32-row slot qb; an unused slot exits here, before
  // any barrier.
  int sq = a.sq, sk = a.sk;
  int64_t row0 = 0, tile0 = 0;
  if constexpr (kVarlen) {
    const SeqSlot ss = find_seq_slot(a.cu_seqlens, a.num_seqs, a.total_rows, qb);
    const int lq = qb - ss.base;
    if (lq < 0 || lq >= (ss.len + BN - 1) / BN) return;
    qb = lq;
    sq = sk = ss.len;
    row0 = ss.start;
    tile0 = ss.base;
  }
  const int hk = __builtin_amdgcn_readfirstlane(div_small(h, a.group));
  const int q_first = qb * 32;
  const int q_idx = q_first + l32;  // this lane's query
  const int k_end = kCausal ? min(sk, min(sq, q_first + 32)) : sk;
  const int ntiles = (k_end + BN - 1) / BN;  // >= 1: q_first < sq and sk >= 1
  const int head_tiles = (sk + BN - 1) / BN;
  const int my_tiles = (ntiles - wave + NW - 1) / NW;  // tiles wave, wave + 4, ... (0 when ntiles <= wave)

  // Every K/V load below stays inside this head's (sequence's) packed tiles:
  // tile indices are clamped to [0, ntiles), and ntiles <= head_tiles.
  const __amdgpu_buffer_rsrc_t kvr =
      make_rsrc(a.kv + b * a.kv_sb + hk * a.kv_sh + tile0 * kv_tile_elems(D), head_tiles * TILE_BYTES);
  const int voff = lane * 16;
  auto tile_off = [&](int i) { return min(wave + NW * i, ntiles - 1) * TILE_BYTES; };  // the wave's i-th tile
  // Bias: lane reads the 16 keys of its accumulator rows (4 runs of 4 keys); a
  // dword past sk is out of the descriptor's range and reads as 0.
  __amdgpu_buffer_rsrc_t bsr;
  if constexpr (kBias) bsr = make_rsrc(a.key_bias + b * a.kb_sb, a.sk * 4);

  // ---- loads, in the order they are needed: K of the first tile, the bias
  // scan, Q, V of the first tile ----
  u32x4 kop[KSTEPS], vop[2 * DBLK];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) kop[ks] = __builtin_amdgcn_raw_buffer_load_b128(kvr, voff + ks * 1024, tile_off(0), 0);
  // Per-wave bias flags: bit i of `wbias` is set when the wave's i-th tile has
  // a bias entry that is not +0 / -0 (a key-padding mask is zero almost
  // everywhere).  Only flagged tiles load and add the bias; the scan covers a
  // wave's first 2 * kScanLoads tiles, later tiles are always treated as
  // flagged.
  constexpr int kScanLoads = 16;
  uint64_t wbias = 0;
  float bscan[kScanLoads];
  if constexpr (kBias) {
#pragma unroll
    for (int r = 0; r < kScanLoads; ++r) {
      bscan[r] = 0.f;
      if (2 * r < my_tiles)  // lanes 0-31: tile slot 2r, lanes 32-63: slot 2r + 1
        bscan[r] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(bsr, ((wave + NW * (2 * r + g)) * BN + l32) * 4, 0, 0));
    }
  }
  // Q^T operands: lane holds query l32, d-chunk (2 ks + g).  Without the fused
  // norm the workgroup loads them once: wave w copies chunks w, w + 4, ...
  // straight into LDS (buffer_load ... lds), then every wave reads all of them.
  bf16x8 qreg[KSTEPS];
  const uint16_t* qbase = a.q + b * a.q_sb + h * a.q_sh + row0 * a.q_ss;
  if constexpr (kQNorm) {
    const uint16_t* qrow = qbase + min(q_idx, sq - 1) * a.q_ss + g * 8;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
      qreg[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(qrow + ks * 16));
  } else {
    // byte extent of the head's rows and this lane's row offset: below 2^31 (checked by the launcher)
    const __amdgpu_buffer_rsrc_t qr =
        make_rsrc(qbase, static_cast<int>((static_cast<int64_t>(sq - 1) * a.q_ss + D) * 2));
    const int qoff = static_cast<int>((static_cast<int64_t>(min(q_idx, sq - 1)) * a.q_ss + g * 8) * 2);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
      if (ks % NW == wave)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(qr, (__attribute__((address_space(3))) void*)(qsh + ks * 64), 16,
                                                 qoff, ks * 32, 0, 0);
  }
#pragma unroll
  for (int cc = 0; cc < 2 * DBLK; ++cc)
    vop[cc] = __builtin_amdgcn_raw_buffer_load_b128(kvr, voff + VPART + cc * 1024, tile_off(0), 0);
  if constexpr (kQNorm) {
    qnorm_rope_shared<D>(qreg, a, q_idx, q_idx < sq, wave, qsh);
  } else {
    vm_wait_barrier<2 * DBLK>();  // this wave's Q chunks are in LDS (only V still in flight); every wave's after the barrier
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) qreg[ks] = __builtin_bit_cast(bf16x8, qsh[ks * 64 + lane]);
  }

  // bias flags (NaN != 0 is true: a NaN bias is applied, not skipped)
  auto flagged = [&](int i) { return i >= 64 || ((wbias >> i) & 1ull); };
  auto load_bias_of = [&](floatx4 (&dst)[4], int i) { load_bias(dst, bsr, (wave + NW * i) * BN + 4 * g); };
  if constexpr (kBias) {
#pragma unroll
    for (int r = 0; r < kScanLoads; ++r) {
      const uint64_t bal = __ballot(bscan[r] != 0.f);
      if (bal & 0xffffffffull) wbias |= 1ull << (2 * r);
      if (bal >> 32) wbias |= 1ull << (2 * r + 1);
    }
    if (my_tiles > 2 * kScanLoads) wbias |= ~0ull << (2 * kScanLoads);
  }

  floatx16 oacc[DBLK];
#pragma unroll
  for (int db = 0; db < DBLK; ++db) oacc[db] = floatx16{};
  float m_ref = -__builtin_inff();  // reference max (log2 units) used for exp
  float l_part = 0.f;               // this lane's share of the row sum
  const float c = a.scale_log2;
  const float kb = kLog2e / c;  // a natural-log bias in raw-score units (the score is scaled by c later)

  // ---- softmax helpers (log2 domain; lane = one query, 16 of the tile's keys) ----
  // Masking of the wave's i-th tile on its raw scores: keys past sk, the causal
  // future and -inf biases become -inf, other biases are added (flagged tiles).
  floatx4 bn[4] = {};  // the bias of the next flagged tile, loaded one tile ahead
  auto mask_tile = [&](floatx16& s, int i) {
    const int k0 = (wave + NW * i) * BN;
    const bool btile = kBias && flagged(i);
    if ((k0 + BN > sk) || (kCausal && k0 + BN - 1 > q_first) || btile) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = k0 + 8 * (e >> 2) + 4 * g + (e & 3);
        float sv = s[e];
        if constexpr (kBias) {
          if (btile) sv += bn[e >> 2][e & 3] * kb;
        }
        bool ok = key < sk;
        if constexpr (kCausal) ok = ok && (key <= q_idx);
        s[e] = ok ? sv : -__builtin_inff();
      }
    }
  };
  // Lazy rescale: the reference max moves only when a tile max exceeds it by
  // more than 2^8 (softmax is shift-invariant).  Both lanes of a query see the
  // same pair maximum, so they keep the same reference.
  auto update_max = [&](const floatx16& s) {
    float mt = s[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) mt = fmaxf(mt, s[e]);
    mt *= c;
    if (__any(mt > m_ref + kLazyThreshold)) {
      const float mq = pair_max(mt);
      const float new_ref = mq > m_ref + kLazyThreshold ? mq : m_ref;
      const float alpha = (m_ref == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(m_ref - new_ref);
      m_ref = new_ref;
      l_part *= alpha;
#pragma unroll
      for (int db = 0; db < DBLK; ++db) oacc[db] *= alpha;
    }
  };
  // P = exp2(s c - m) packed to bf16, its row sum; meanwhile the S^T MFMAs of
  // a later tile (K operands `kk`) are issued between the exponentials, so the
  // matrix pipe works during the softmax.
  bf16x8 pop[2];
  auto exp_pack_and_score = [&](floatx16& s, floatx16& snew) {
    const float nm = (m_ref == -__builtin_inff()) ? 0.f : -m_ref;
    float psum = 0.f;
    snew = floatx16{};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(s[e], c, nm));
      s[e] = pe;
      psum += pe;
#pragma unroll
      for (int ks = e * KSTEPS / 16; ks < (e + 1) * KSTEPS / 16; ++ks)  // KSTEPS MFMAs spread over the 16 exps
        snew = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kop[ks]), qreg[ks], snew, 0, 0, 0);
    }
    l_part += psum;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      floatx8 pv;
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = s[s2 * 8 + e];
      pop[s2] = __builtin_convertvector(pv, bf16x8);
    }
  };
  auto pv_mma = [&]() {  // O^T += V^T P^T, two 16-key steps
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int db = 0; db < DBLK; ++db)
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vop[db * 2 + s2]), pop[s2],
                                                           oacc[db], 0, 0, 0);
  };

  // ---- main loop, software-pipelined over the wave's tiles t_i = wave + 4 i.
  // Per iteration i: P(t_i) V(t_i) on the matrix pipe while the VALU masks and
  // takes the max of S(t_i+1); then the exponentials of S(t_i+1) with the
  // S(t_i+2) MFMAs issued between them.  K operands are loaded once their
  // tile's S MFMAs are issued, V operands once their P.V MFMAs are. ----
  if (my_tiles > 0) {
    floatx16 sa, sb;
    sa = floatx16{};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
      sa = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kop[ks]), qreg[ks], sa, 0, 0, 0);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) kop[ks] = __builtin_amdgcn_raw_buffer_load_b128(kvr, voff + ks * 1024, tile_off(1), 0);
    if constexpr (kBias) {
      if (flagged(0)) load_bias_of(bn, 0);
    }
    mask_tile(sa, 0);
    if constexpr (kBias) {
      if (my_tiles > 1 && flagged(1)) load_bias_of(bn, 1);
    }
    update_max(sa);
    exp_pack_and_score(sa, sb);  // P(t_0); S(t_1)
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) kop[ks] = __builtin_amdgcn_raw_buffer_load_b128(kvr, voff + ks * 1024, tile_off(2), 0);
    // iteration i: pop = P(t_i), vop = V(t_i), s_next = S(t_i+1), kop = K(t_i+2)
    auto body = [&](int i, floatx16& s_next, floatx16& s_out) {
      pv_mma();
#pragma unroll
      for (int cc = 0; cc < 2 * DBLK; ++cc)
        vop[cc] = __builtin_amdgcn_raw_buffer_load_b128(kvr, voff + VPART + cc * 1024, tile_off(i + 1), 0);
      if (i + 1 < my_tiles) {
        mask_tile(s_next, i + 1);
        if constexpr (kBias) {
          if (i + 2 < my_tiles && flagged(i + 2)) load_bias_of(bn, i + 2);
        }
        update_max(s_next);
        exp_pack_and_score(s_next, s_out);  // P(t_i+1); S(t_i+2)
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
          kop[ks] = __builtin_amdgcn_raw_buffer_load_b128(kvr, voff + ks * 1024, tile_off(i + 3), 0);
      }
    };
    for (int i = 0; i < my_tiles; i += 2) {
      body(i, sb, sa);
      if (i + 1 >= my_tiles) break;
      body(i + 1, sa, sb);
    }
  }

  // ---- merge the 4 waves' partial states; wave w finalises d-blocks w, w+4, ... ----
  // LDS layout: [wave][float4 group][lane] -> 16-byte, conflict-free accesses.
  {
    floatx4* mine = merge + wave * (G4 * 64);
#pragma unroll
    for (int db = 0; db < DBLK; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        mine[(db * 4 + q4) * 64 + lane] =
            floatx4{oacc[db][q4 * 4], oacc[db][q4 * 4 + 1], oacc[db][q4 * 4 + 2], oacc[db][q4 * 4 + 3]};
    mine[(DBLK * 4) * 64 + lane] = floatx4{m_ref, l_part, 0.f, 0.f};
  }
  __syncthreads();
  {
    // every LDS read of this lane is issued before the arithmetic that uses it
    floatx4 ml[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) ml[w] = merge[w * (G4 * 64) + (DBLK * 4) * 64 + lane];
    constexpr int DPW = (DBLK + NW - 1) / NW;  // d-blocks finalised per wave
    floatx4 part[DPW][4][NW];
#pragma unroll
    for (int r = 0; r < DPW; ++r) {
      const int db = wave + r * NW;
      if (db < DBLK) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
          for (int w = 0; w < NW; ++w) part[r][q4][w] = merge[w * (G4 * 64) + (db * 4 + q4) * 64 + lane];
      }
    }
    float wgt[NW];
    float m = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < NW; ++w) m = fmaxf(m, ml[w][0]);
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      wgt[w] = (ml[w][0] == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(ml[w][0] - m);
      l += ml[w][1] * wgt[w];
    }
    l = pair_sum(l);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    // packed row of this lane's query (o_packed_k > 0); constant indices into
    // the segment arrays, so they stay scalar kernel arguments
    int prow = q_idx;
    bool stored = q_idx < sq;
    if (a.o_nseg > 0) {
      const bool s1 = a.o_nseg > 1 && q_idx >= a.o_seg_off[1], s2 = a.o_nseg > 2 && q_idx >= a.o_seg_off[2];
      const int off = s2 ? a.o_seg_off[2] : s1 ? a.o_seg_off[1] : a.o_seg_off[0];
      const int rows = s2 ? a.o_seg_rows[2] : s1 ? a.o_seg_rows[1] : a.o_seg_rows[0];
      const int base = s2 ? a.o_seg_base[2] : s1 ? a.o_seg_base[1] : a.o_seg_base[0];
      stored = stored && q_idx >= off && q_idx - off < rows;
      prow = base + b * rows + (q_idx - off);
    }
    if (stored) {
      uint16_t* orow = a.o + b * a.o_sb + h * a.o_sh + (row0 + q_idx) * a.o_ss;
#pragma unroll
      for (int r = 0; r < DPW; ++r) {
        const int db = wave + r * NW;
        if (db >= DBLK) break;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          floatx4 acc = part[r][q4][0] * wgt[0];
#pragma unroll
          for (int w = 1; w < NW; ++w) acc += part[r][q4][w] * wgt[w];
          acc *= inv;
          const int d = db * 32 + q4 * 8 + g * 4;
          if (kVarlen && d >= a.d_store) continue;  // zero padding columns of a head_dim < D
          uint2 wv;
          wv.x = pack_bf16x2(acc[0], acc[1]);
          wv.y = pack_bf16x2(acc[2], acc[3]);
          if (a.o_packed_k > 0)  // 4 consecutive columns stay inside one 8-element run
            *reinterpret_cast<uint2*>(a.o + packed_act_offset(prow, static_cast<int64_t>(h) * D + d, a.o_packed_k)) = wv;
          else
            *reinterpret_cast<uint2*>(orow + d) = wv;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// K [B, H, Sk, D], V [B, H, Sk, D] (strided) -> packed K/V tiles (layout at the
// top of this file).  One workgroup per (32-key tile, head, batch); V is
// transposed through LDS.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void kv_pack_kernel(const uint16_t* __restrict__ k, int64_t k_sb, int64_t k_sh,
                                                      int64_t k_ss, const uint16_t* __restrict__ v, int64_t v_sb,
                                                      int64_t v_sh, int64_t v_ss, uint16_t* __restrict__ kvp,
                                                      int64_t p_sb, int64_t p_sh, int sk) {
  constexpr int PITCH = D + 8;
  constexpr int CH = D / 8;      // 16-byte chunks per V row
  constexpr int NCH = D / 16;    // 1 KB chunks per part
  __shared__ __attribute__((aligned(16))) uint16_t tile[32 * PITCH];
  const int k0 = blockIdx.x * kTileKeys;
  const uint16_t* ksrc = k + blockIdx.z * k_sb + blockIdx.y * k_sh;
  const uint16_t* vsrc = v + blockIdx.z * v_sb + blockIdx.y * v_sh;
  uint16_t* dst = kvp + blockIdx.z * p_sb + blockIdx.y * p_sh + static_cast<int64_t>(blockIdx.x) * kv_tile_elems(D);
  for (int cidx = threadIdx.x; cidx < 32 * CH; cidx += 256) {
    const int r = cidx / CH, col = (cidx % CH) * 8;
    const int key = k0 + r;
    const u32x4 val = key < sk ? *reinterpret_cast<const u32x4*>(vsrc + static_cast<int64_t>(key) * v_ss + col)
                               : u32x4{0, 0, 0, 0};
    *reinterpret_cast<u32x4*>(&tile[r * PITCH + col]) = val;
  }
  // K part: straight 16-byte copies into operand order
  for (int idx = threadIdx.x; idx < NCH * 64; idx += 256) {
    const int ks = idx >> 6, l = idx & 63;
    const int key = k0 + (l & 31);
    const u32x4 val = key < sk ? *reinterpret_cast<const u32x4*>(ksrc + static_cast<int64_t>(key) * k_ss + 16 * ks +
                                                                 8 * (l >> 5))
                               : u32x4{0, 0, 0, 0};
    *reinterpret_cast<u32x4*>(dst + idx * 8) = val;
  }
  __syncthreads();
  // V part: gather 8 keys of one column per lane
  for (int idx = threadIdx.x; idx < NCH * 64; idx += 256) {
    const int cc = idx >> 6, l = idx & 63;
    const int db = cc >> 1, s2 = cc & 1;
    const int d = 32 * db + (l & 31);
    u32x4 out;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const int r0 = 16 * s2 + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
      out[i >> 1] = static_cast<uint32_t>(tile[r0 * PITCH + d]) | (static_cast<uint32_t>(tile[(r0 + 1) * PITCH + d]) << 16);
    }
    *reinterpret_cast<u32x4*>(dst + NCH * 512 + idx * 8) = out;
  }
}

// ---------------------------------------------------------------------------
// Vision attention front end (Qwen3-VL ViT blocks, variable-length images).
// Fused QKV rows [rows, 3 * H * hd] -> (1) rotate-half RoPE'd Q rows, zero
// padded to DP columns, [H][rows][DP]; (2) the packed K/V tiles (D = DP, layout
// at the top of this file) of every (head, sequence), K RoPE'd, keys and
// columns past the sequence / hd zero.  Tile lt of sequence s sits in slot
// base_s + lt of its head (SeqSlot).  One workgroup per (slot, head); an unused
// slot exits at once.
// RoPE (fused_vision_attention.py:47-80, :117-139), fp32, each product rounded:
//   y[d] = bf16(x[d] * cos[d] + x[d +- hd/2] * sin_baked[d]),
// the sign of rotate_half's first half folded into sin_baked
// (custom_vision_encoder_chain.py:101-108).
// ---------------------------------------------------------------------------
struct VitArgs {
  const uint16_t* qkv;  // [rows, 3 * heads * hd]
  const float* cos;     // [rows, hd]
  const float* sin;     // [rows, hd], baked sign
  const int32_t* cu_seqlens;
  uint16_t* qpad;       // [heads][rows][DP]
  uint16_t* kvp;        // [heads][slots] packed tiles
  int64_t kv_sh;        // elements per head of kvp
  int num_seqs, rows, heads, hd;
};

__device__ __forceinline__ uint2 vit_rope4(uint2 x, uint2 p, floatx4 c, floatx4 s) {
#pragma clang fp contract(off)
  const float y0 = bf16x2_lo(x.x) * c[0] + bf16x2_lo(p.x) * s[0];
  const float y1 = bf16x2_hi(x.x) * c[1] + bf16x2_hi(p.x) * s[1];
  const float y2 = bf16x2_lo(x.y) * c[2] + bf16x2_lo(p.y) * s[2];
  const float y3 = bf16x2_hi(x.y) * c[3] + bf16x2_hi(p.y) * s[3];
  return uint2{pack_bf16x2(y0, y1), pack_bf16x2(y2, y3)};
}

template <int DP>
__global__ __launch_bounds__(256) void vit_pack_kernel(VitArgs v) {
  constexpr int PITCH = DP + 8;  // 16-byte aligned LDS rows
  constexpr int G = DP / 4;      // 4-column groups per padded row
  static_assert((32 * G) % 256 == 0, "whole groups per thread");
  constexpr int NCH = DP / 16;   // 1 KB chunks per K / V part
  __shared__ __attribute__((aligned(16))) uint16_t tq[32 * PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t tk[32 * PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t tv[32 * PITCH];
  const int slot = static_cast<int>(blockIdx.x), h = static_cast<int>(blockIdx.y);
  const SeqSlot ss = find_seq_slot(v.cu_seqlens, v.num_seqs, v.rows, slot);
  const int lt = slot - ss.base;
  if (lt < 0 || lt >= (ss.len + 31) / 32) return;
  const int r0 = ss.start + 32 * lt;           // first row of the tile
  const int nrows = min(32, ss.len - 32 * lt);  // rows of the sequence in it
  const int hd = v.hd, half = hd >> 1;
  const int64_t qkv_ss = 3LL * v.heads * hd;
  const uint16_t* qsrc = v.qkv + static_cast<int64_t>(h) * hd;
  const uint16_t* ksrc = qsrc + static_cast<int64_t>(v.heads) * hd;
  const uint16_t* vsrc = ksrc + static_cast<int64_t>(v.heads) * hd;
  // Every read uses a row clamped into the sequence's rows of the tile and a
  // column group clamped below hd (so the unrolled loads are unconditional and
  // issue back to back); groups outside are replaced by zeros afterwards.
  // 4-column groups never straddle hd or hd / 2 (hd % 8 == 0).
  constexpr int NU = 32 * G / 256;  // groups per thread
  uint2 xq[NU], pq[NU], xk[NU], pk[NU], xv[NU];
  floatx4 cs[NU], sn[NU];
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const int u = threadIdx.x + 256 * i;
    const int64_t row = r0 + min(u / G, nrows - 1);
    const int d4 = min((u % G) * 4, hd - 4);
    const int pd = d4 < half ? d4 + half : d4 - half;
    const uint16_t* qr = qsrc + row * qkv_ss;
    const uint16_t* kr = ksrc + row * qkv_ss;
    xq[i] = *reinterpret_cast<const uint2*>(qr + d4);
    pq[i] = *reinterpret_cast<const uint2*>(qr + pd);
    xk[i] = *reinterpret_cast<const uint2*>(kr + d4);
    pk[i] = *reinterpret_cast<const uint2*>(kr + pd);
    xv[i] = *reinterpret_cast<const uint2*>(vsrc + row * qkv_ss + d4);
    cs[i] = *reinterpret_cast<const floatx4*>(v.cos + row * hd + d4);
    sn[i] = *reinterpret_cast<const floatx4*>(v.sin + row * hd + d4);
  }
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const int u = threadIdx.x + 256 * i;
    const int r = u / G, d4 = (u % G) * 4;
    const bool in = r < nrows && d4 < hd;
    const uint2 z{0, 0};
    *reinterpret_cast<uint2*>(&tq[r * PITCH + d4]) = in ? vit_rope4(xq[i], pq[i], cs[i], sn[i]) : z;
    *reinterpret_cast<uint2*>(&tk[r * PITCH + d4]) = in ? vit_rope4(xk[i], pk[i], cs[i], sn[i]) : z;
    *reinterpret_cast<uint2*>(&tv[r * PITCH + d4]) = in ? xv[i] : z;
  }
  __syncthreads();
  // Q rows of the sequence -> qpad (DP columns, the padding included)
  uint16_t* qdst = v.qpad + (static_cast<int64_t>(h) * v.rows + r0) * DP;
  for (int c = threadIdx.x; c < nrows * (DP / 8); c += 256) {
    const int r = c / (DP / 8), col = (c % (DP / 8)) * 8;
    *reinterpret_cast<u32x4*>(qdst + r * DP + col) = *reinterpret_cast<const u32x4*>(&tq[r * PITCH + col]);
  }
  uint16_t* dst = v.kvp + static_cast<int64_t>(h) * v.kv_sh + static_cast<int64_t>(slot) * kv_tile_elems(DP);
  // K part: chunk ks, lane l = key (l & 31), columns 16 ks + 8 (l >> 5) .. + 7
  for (int idx = threadIdx.x; idx < NCH * 64; idx += 256) {
    const int ks = idx >> 6, l = idx & 63;
    *reinterpret_cast<u32x4*>(dst + idx * 8) =
        *reinterpret_cast<const u32x4*>(&tk[(l & 31) * PITCH + 16 * ks + 8 * (l >> 5)]);
  }
  // V part: 8 keys of one column per lane
  for (int idx = threadIdx.x; idx < NCH * 64; idx += 256) {
    const int cc = idx >> 6, l = idx & 63;
    const int db = cc >> 1, s2 = cc & 1;
    const int d = 32 * db + (l & 31);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const int rr = 16 * s2 + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
      o[i >> 1] = static_cast<uint32_t>(tv[rr * PITCH + d]) | (static_cast<uint32_t>(tv[(rr + 1) * PITCH + d]) << 16);
    }
    *reinterpret_cast<u32x4*>(dst + NCH * 512 + idx * 8) = o;
  }
}

// ---------------------------------------------------------------------------
// TransformerMemory attention (mem::fused_attention): bf16 rotate-half RoPE on
// Q and K + softmax(Q K^T / sqrt(D)) V with the block-causal mask
// (query i sees key j iff j / B <= i / B), fused QKV rows [M, 3 H D].
// The problem is tiny (M = 4 timesteps x 16 cognition tokens, 16 heads x 256)
// and latency-bound, so a workgroup (32 queries of one head, 8 waves) stages
// its RoPE'd Q, then chunks of 64 RoPE'd keys and the transposed V chunk in
// LDS, each thread issuing all of its loads before the first use; every wave
// computes the full score tile S^T = K Q^T (lane = query column) and its own
// d-blocks of O^T = V^T P^T, so no cross-wave merge is needed.  Online softmax
// in the exp2 domain across key tiles.
// RoPE (fused_memory_attention.py:84-108, :124-138; memory.py:52-57), every
// step rounded to bf16:  y = bf16(bf16(x * cos) + bf16(x[d +- D/2] * signed_sin)).
// ---------------------------------------------------------------------------
struct MemArgs {
  const uint16_t* qkv;         // [M, 3 * heads * D]
  const uint16_t* cos;         // [M, D] bf16
  const uint16_t* signed_sin;  // [M, D] bf16, first half negated
  uint16_t* out;               // [M, heads * D]
  int m, heads;
  int64_t block;               // block_attn_size >= 1
  float scale_log2;            // log2(e) / sqrt(D)
};

__device__ __forceinline__ uint32_t mem_rope_bf16x2(uint32_t x, uint32_t p, uint32_t c, uint32_t s) {
#pragma clang fp contract(off)
  const uint32_t t = pack_bf16x2(bf16x2_lo(x) * bf16x2_lo(c), bf16x2_hi(x) * bf16x2_hi(c));
  const uint32_t u = pack_bf16x2(bf16x2_lo(p) * bf16x2_lo(s), bf16x2_hi(p) * bf16x2_hi(s));
  return pack_bf16x2(bf16x2_lo(t) + bf16x2_lo(u), bf16x2_hi(t) + bf16x2_hi(u));
}

// Operands of the RoPE of one 8-column chunk (self, rotate-half partner, cos,
// signed sin), loaded together so that a thread's loads are all in flight
// before the first use.
struct RopeIn {
  u32x4 x, p, c, s;
};

// Chunk c8 of row `row` of the head's Q (col0 = h D) or K (col0 = (H + h) D) columns.
template <int D>
__device__ __forceinline__ RopeIn mem_rope_load(const MemArgs& a, int64_t row, int64_t col0, int c8) {
  constexpr int HALF8 = D / 16;  // rotate-half partner: 8-column chunks are D/16 apart
  const int64_t ld = 3LL * a.heads * D;
  const int pc = c8 < HALF8 ? c8 + HALF8 : c8 - HALF8;
  const uint16_t* r = a.qkv + row * ld + col0;
  RopeIn in;
  in.x = *reinterpret_cast<const u32x4*>(r + 8 * c8);
  in.p = *reinterpret_cast<const u32x4*>(r + 8 * pc);
  in.c = *reinterpret_cast<const u32x4*>(a.cos + row * D + 8 * c8);
  in.s = *reinterpret_cast<const u32x4*>(a.signed_sin + row * D + 8 * c8);
  return in;
}

__device__ __forceinline__ u32x4 mem_rope_apply(const RopeIn& in) {
  u32x4 y;
#pragma unroll
  for (int j = 0; j < 4; ++j) y[j] = mem_rope_bf16x2(in.x[j], in.p[j], in.c[j], in.s[j]);
  return y;
}

template <int D>
__global__ __launch_bounds__(512) void mem_attn_kernel(MemArgs a) {
  constexpr int NT = 512;              // 8 waves
  constexpr int NW = NT / 64;
  constexpr int KSTEPS = D / 16;
  constexpr int DBLK = D / 32;
  constexpr int DPW = (DBLK + NW - 1) / NW;  // d-blocks of O per wave (wave w: w, w + 8, ...)
  constexpr int CH = D / 8;            // 8-column chunks per row
  constexpr int QP = D + 8;            // LDS pitch of Q / K rows (elements)
  constexpr int KC = 64;               // keys per staged chunk
  constexpr int VP = KC + 4;           // LDS pitch of transposed V rows (elements; conflict-free b64 reads)
  constexpr int QU = (32 * CH + NT - 1) / NT;        // Q chunks per thread
  constexpr int KU = (KC * CH + NT - 1) / NT;        // K chunks per thread
  constexpr int VU = ((KC / 2) * CH + NT - 1) / NT;  // V key-pair chunks per thread
  __shared__ __attribute__((aligned(16))) uint16_t qs[32 * QP];
  __shared__ __attribute__((aligned(16))) uint16_t ks[KC * QP];
  __shared__ __attribute__((aligned(16))) uint16_t vt[D * VP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const int h = static_cast<int>(blockIdx.y);
  const int q0 = static_cast<int>(blockIdx.x) * 32;
  const int m = a.m;
  const int64_t qcol = static_cast<int64_t>(h) * D, kcol = static_cast<int64_t>(a.heads + h) * D,
                vcol = static_cast<int64_t>(2 * a.heads + h) * D;
  const int64_t ld = 3LL * a.heads * D;
  // keys visible to the block's last row (all rows of the block see keys below it only)
  const int64_t q_last = min(q0 + 31, m - 1);
  const int k_end = static_cast<int>(min<int64_t>(m, (q_last / a.block + 1) * a.block));
  // this lane's query and its key limit: keys j < lim are visible
  const int qi = min(q0 + l32, m - 1);
  const int lim = static_cast<int>(min<int64_t>(m, (qi / a.block + 1) * a.block));

  // Staging.  Every global load reads a row clamped into [0, limit) (so it is
  // unconditional and the unrolled loads issue back to back); rows past the
  // limit are replaced by zeros afterwards.
  RopeIn qin[QU];
#pragma unroll
  for (int i = 0; i < QU; ++i) {
    const int u = min(tid + NT * i, 32 * CH - 1);
    qin[i] = mem_rope_load<D>(a, min(q0 + u / CH, m - 1), qcol, u % CH);
  }
  RopeIn kin[KU];
  u32x4 va[VU], vb[VU];
  auto load_kv = [&](int c0) {
#pragma unroll
    for (int i = 0; i < KU; ++i) {
      const int u = min(tid + NT * i, KC * CH - 1);
      kin[i] = mem_rope_load<D>(a, min(c0 + u / CH, k_end - 1), kcol, u % CH);
    }
#pragma unroll
    for (int i = 0; i < VU; ++i) {
      const int u = min(tid + NT * i, (KC / 2) * CH - 1);
      const int j0 = c0 + 2 * (u % (KC / 2)), c8 = u / (KC / 2);
      va[i] = *reinterpret_cast<const u32x4*>(a.qkv + static_cast<int64_t>(min(j0, k_end - 1)) * ld + vcol + 8 * c8);
      vb[i] = *reinterpret_cast<const u32x4*>(a.qkv + static_cast<int64_t>(min(j0 + 1, k_end - 1)) * ld + vcol +
                                              8 * c8);
    }
  };
  auto store_kv = [&](int c0) {
    // K chunk, RoPE'd, row-major (rows >= k_end zero)
#pragma unroll
    for (int i = 0; i < KU; ++i) {
      const int u = tid + NT * i;
      if (u < KC * CH) {
        const int r = u / CH, c8 = u % CH;
        const u32x4 y = c0 + r < k_end ? mem_rope_apply(kin[i]) : u32x4{0, 0, 0, 0};
        *reinterpret_cast<u32x4*>(&ks[r * QP + 8 * c8]) = y;
      }
    }
    // V chunk, transposed: vt[d][key], two keys per 32-bit LDS write (keys >= k_end zero)
#pragma unroll
    for (int i = 0; i < VU; ++i) {
      const int u = tid + NT * i;
      if (u < (KC / 2) * CH) {
        const int p = u % (KC / 2), c8 = u / (KC / 2);
        const int j0 = c0 + 2 * p;
        const u32x4 v0 = j0 < k_end ? va[i] : u32x4{0, 0, 0, 0};
        const u32x4 v1 = j0 + 1 < k_end ? vb[i] : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t e0 = (v0[e >> 1] >> (16 * (e & 1))) & 0xffffu;
          const uint32_t e1 = (v1[e >> 1] >> (16 * (e & 1))) & 0xffffu;
          *reinterpret_cast<uint32_t*>(&vt[(8 * c8 + e) * VP + 2 * p]) = e0 | (e1 << 16);
        }
      }
    }
  };
  load_kv(0);
  // RoPE'd Q rows (rows past m zero)
#pragma unroll
  for (int i = 0; i < QU; ++i) {
    const int u = tid + NT * i;
    if (u < 32 * CH) {
      const int r = u / CH, c8 = u % CH;
      const u32x4 y = q0 + r < m ? mem_rope_apply(qin[i]) : u32x4{0, 0, 0, 0};
      *reinterpret_cast<u32x4*>(&qs[r * QP + 8 * c8]) = y;
    }
  }
  store_kv(0);
  __syncthreads();
  bf16x8 qreg[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk)
    qreg[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&qs[l32 * QP + 16 * kk + 8 * g]));

  floatx16 oacc[DPW];
#pragma unroll
  for (int r = 0; r < DPW; ++r) oacc[r] = floatx16{};
  float m_run = -__builtin_inff(), l_part = 0.f;
  const float c = a.scale_log2;

  for (int c0 = 0; c0 < k_end; c0 += KC) {
    if (c0 > 0) {  // next 64-key chunk (M > 64)
      __syncthreads();  // the previous chunk's K / V reads are done
      load_kv(c0);
      store_kv(c0);
      __syncthreads();
    }
    const int ntile = min(KC, k_end - c0 + 31) / 32;  // tiles of this chunk holding keys < k_end
    for (int t = 0; t < ntile; ++t) {
      // ---- S^T = K Q^T ----
      floatx16 sacc = floatx16{};
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) {
        const u32x4 kop = *reinterpret_cast<const u32x4*>(&ks[(32 * t + l32) * QP + 16 * kk + 8 * g]);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kop), qreg[kk], sacc, 0, 0, 0);
      }
      // ---- online softmax (log2 domain); lane = query l32, keys 8 (e/4) + 4 g + e%4 of the tile ----
      const int kb = c0 + 32 * t + 4 * g;
      float mt = -__builtin_inff();
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = kb + 8 * (e >> 2) + (e & 3);
        const float sv = key < lim ? sacc[e] * c : -__builtin_inff();
        sacc[e] = sv;
        mt = fmaxf(mt, sv);
      }
      const float m_new = fmaxf(m_run, pair_max(mt));  // finite: key 0 of tile 0 is visible to every row
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_part *= alpha;
#pragma unroll
      for (int r = 0; r < DPW; ++r) oacc[r] *= alpha;
      float psum = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pe = __builtin_amdgcn_exp2f(sacc[e] - m_new);
        sacc[e] = pe;
        psum += pe;
      }
      l_part += psum;
      // ---- O^T += V^T P^T over this wave's d-blocks ----
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        floatx8 pv;
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[e] = sacc[s2 * 8 + e];
        const bf16x8 pop = __builtin_convertvector(pv, bf16x8);
#pragma unroll
        for (int r = 0; r < DPW; ++r) {
          const int db = wave + NW * r;
          if (db < DBLK) {
            // keys 16 s2 + 8 (i / 4) + 4 g + i % 4 of the tile for element i: two runs of 4
            const uint16_t* vrow = &vt[(32 * db + l32) * VP + 32 * t + 16 * s2 + 4 * g];
            const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
            const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 8);
            const u32x4 vop{lo.x, lo.y, hi.x, hi.y};
            oacc[r] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vop), pop, oacc[r], 0, 0, 0);
          }
        }
      }
    }
  }

  // ---- normalise and store this wave's columns of the 32 rows ----
  const float l = pair_sum(l_part);
  const float inv = 1.0f / l;
  if (q0 + l32 < m) {
    uint16_t* orow = a.out + static_cast<int64_t>(q0 + l32) * a.heads * D + qcol;
#pragma unroll
    for (int r = 0; r < DPW; ++r) {
      const int db = wave + NW * r;
      if (db >= DBLK) break;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = db * 32 + q4 * 8 + g * 4;
        uint2 wv;
        wv.x = pack_bf16x2(oacc[r][q4 * 4] * inv, oacc[r][q4 * 4 + 1] * inv);
        wv.y = pack_bf16x2(oacc[r][q4 * 4 + 2] * inv, oacc[r][q4 * 4 + 3] * inv);
        *reinterpret_cast<uint2*>(orow + d) = wv;
      }
    }
  }
}

// head_dim -> padded K/V tile width (a multiple of 32 the attention kernel is
// built for), 0 when unsupported
constexpr int vit_padded_dim(int64_t hd) {
  return (hd < 8 || hd > 128 || hd % 8) ? 0 : (hd <= 64 ? 64 : (hd <= 96 ? 96 : 128));
}

template <int DP>
hipError_t launch_vit(const VitArgs& v, AttnArgs a, int64_t slots, hipStream_t stream) {
  hipLaunchKernelGGL(vit_pack_kernel<DP>, dim3(static_cast<unsigned>(slots), static_cast<unsigned>(v.heads)),
                     dim3(256), 0, stream, v);
  a.num_q_blocks = static_cast<int>(slots);
  a.n_work = static_cast<int>(slots * v.heads);
  hipLaunchKernelGGL((attn_fwd_kernel<DP, 1, false, false, false, true>),
                     dim3(static_cast<unsigned>(slots * v.heads)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int D, int NSUB, bool kQNorm>
void launch_attn_d(AttnArgs a, int batch, bool causal, bool has_bias, hipStream_t stream) {
  a.n_work = a.num_q_blocks * a.hq * batch;
  // warm-up workgroups: about 1024 lines (128 KB) each, at most 256
  int n_pf = 0;
  if (a.warm.end[2] > 0) {
    n_pf = static_cast<int>(std::min<int64_t>(256, (a.warm.end[2] + 1023) / 1024));
    a.warm.per_wg = (a.warm.end[2] + n_pf - 1) / n_pf;
  }
  dim3 grid(static_cast<unsigned>(a.n_work + n_pf));
  dim3 block(256);
  if (causal) {
    if (has_bias)
      hipLaunchKernelGGL((attn_fwd_kernel<D, NSUB, true, true, kQNorm>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((attn_fwd_kernel<D, NSUB, true, false, kQNorm>), grid, block, 0, stream, a);
  } else {
    if (has_bias)
      hipLaunchKernelGGL((attn_fwd_kernel<D, NSUB, false, true, kQNorm>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((attn_fwd_kernel<D, NSUB, false, false, kQNorm>), grid, block, 0, stream, a);
  }
}

template <bool kQNorm>
hipError_t launch_attn(AttnArgs a, int64_t head_dim, int batch, bool causal, bool has_bias, hipStream_t stream) {
  // 32 queries per workgroup: at 608-2560 tokens the kernel is latency-bound, and
  // twice the workgroups (two per CU, two waves per SIMD) beat the doubled K/V
  // operand reuse of 64-query workgroups (measured on MI355X: 12 x 608 masked
  // 9.6 vs 14.4 us, 28/4 x 1280 causal 29.5 vs 39.6 us).
  constexpr int NSUB = 1;
  a.num_q_blocks = (a.sq + 32 * NSUB - 1) / (32 * NSUB);
  if (head_dim == 128)
    launch_attn_d<128, NSUB, kQNorm>(a, batch, causal, has_bias, stream);
  else
    launch_attn_d<64, NSUB, kQNorm>(a, batch, causal, has_bias, stream);
  return hipGetLastError();
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int64_t tiles_of(int64_t sk) { return (sk + kTileKeys - 1) / kTileKeys; }

// Shared validation of the q/o side and the sizes.
hipError_t check_qo(const void* q, void* o, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                    int64_t seq_k, int64_t head_dim, const int64_t* q_strides, const int64_t* o_strides,
                    float scale) {
  if (head_dim != 64 && head_dim != 128) return hipErrorInvalidValue;
  if (batch < 0 || q_heads < 0 || kv_heads <= 0 || seq_q < 0 || seq_k < 0) return hipErrorInvalidValue;
  if (q_heads % kv_heads != 0) return hipErrorInvalidValue;
  if (!q_strides || !o_strides) return hipErrorInvalidValue;
  if (!(scale > 0.f) || scale == __builtin_inff()) return hipErrorInvalidValue;
  if (batch == 0 || q_heads == 0 || seq_q == 0) return hipSuccess;
  if (seq_k == 0) return hipErrorInvalidValue;  // softmax over an empty key set is undefined
  if (!q || !o) return hipErrorInvalidValue;
  if (!a16(q) || reinterpret_cast<uintptr_t>(o) % 8) return hipErrorInvalidValue;
  for (int i = 0; i < 3; ++i)
    if (q_strides[i] % 8 || o_strides[i] % 4) return hipErrorInvalidValue;
  // per-head packed tiles and per-head query rows are addressed with 32-bit byte offsets
  if (seq_q > (1 << 24) || tiles_of(seq_k) * 128 * head_dim > (int64_t{1} << 31) - 1 || q_heads > 65535 ||
      batch > 65535 || ((seq_q - 1) * q_strides[2] + head_dim) * 2 > (int64_t{1} << 31) - 1)
    return hipErrorInvalidValue;
  if (((seq_q + 31) / 32) * q_heads * batch > (int64_t{1} << 31) - 1) return hipErrorInvalidValue;  // 1-D grid
  return hipSuccess;
}

void fill_qo(AttnArgs& a, const void* q, void* o, int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k,
             const int64_t* qs, const int64_t* os, const float* key_bias, int64_t kb_sb, float scale) {
  a.q = static_cast<const uint16_t*>(q);
  a.o = static_cast<uint16_t*>(o);
  a.q_sb = qs[0]; a.q_sh = qs[1]; a.q_ss = qs[2];
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

extern "C" int64_t rldx_attention_kv_packed_elems(int64_t seq_k, int64_t head_dim) {
  if (seq_k < 0 || head_dim < 0) return -1;
  return tiles_of(seq_k) * kv_tile_elems(head_dim);
}

extern "C" int64_t rldx_attention_workspace_bytes(int64_t batch, int64_t kv_heads, int64_t seq_k, int64_t head_dim) {
  if (batch < 0 || kv_heads < 0 || seq_k < 0 || head_dim < 0) return -1;
  return batch * kv_heads * rldx_attention_kv_packed_elems(seq_k, head_dim) * 2;
}

extern "C" hipError_t rldx_attention_kv_pack_bf16(const void* k, const int64_t* k_strides, const void* v,
                                                  const int64_t* v_strides, void* kv_packed,
                                                  const int64_t* packed_strides, int64_t batch, int64_t kv_heads,
                                                  int64_t seq_k, int64_t head_dim, hipStream_t stream) {
  if (head_dim != 64 && head_dim != 128) return hipErrorInvalidValue;
  if (batch < 0 || kv_heads < 0 || seq_k < 0 || !k_strides || !v_strides || !packed_strides)
    return hipErrorInvalidValue;
  if (batch == 0 || kv_heads == 0 || seq_k == 0) return hipSuccess;
  if (!k || !v || !kv_packed || !a16(k) || !a16(v) || !a16(kv_packed)) return hipErrorInvalidValue;
  for (int i = 0; i < 3; ++i)
    if (k_strides[i] % 8 || v_strides[i] % 8) return hipErrorInvalidValue;
  const int64_t head_elems = rldx_attention_kv_packed_elems(seq_k, head_dim);
  if (packed_strides[0] % 8 || packed_strides[1] % 8 || packed_strides[1] < head_elems ||
      (batch > 1 && packed_strides[0] < kv_heads * packed_strides[1]))
    return hipErrorInvalidValue;
  if (batch > 65535 || kv_heads > 65535 || tiles_of(seq_k) > (int64_t{1} << 31) - 1) return hipErrorInvalidValue;
  dim3 grid(static_cast<unsigned>(tiles_of(seq_k)), static_cast<unsigned>(kv_heads), static_cast<unsigned>(batch));
  if (head_dim == 128)
    hipLaunchKernelGGL(kv_pack_kernel<128>, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(k), k_strides[0],
                       k_strides[1], k_strides[2], static_cast<const uint16_t*>(v), v_strides[0], v_strides[1],
                       v_strides[2], static_cast<uint16_t*>(kv_packed), packed_strides[0], packed_strides[1],
                       static_cast<int>(seq_k));
  else
    hipLaunchKernelGGL(kv_pack_kernel<64>, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(k), k_strides[0],
                       k_strides[1], k_strides[2], static_cast<const uint16_t*>(v), v_strides[0], v_strides[1],
                       v_strides[2], static_cast<uint16_t*>(kv_packed), packed_strides[0], packed_strides[1],
                       static_cast<int>(seq_k));
  return hipGetLastError();
}

namespace {
// The packed-K/V attention; warm: up to three byte ranges whose 128-byte lines
// extra workgroups of the launch read (see AttnArgs::n_work).
// Row segments of a packed O (num_segments x {first query row, rows stored,
// first packed row}): ascending, disjoint, inside [0, seq_q), every packed row
// below 2^31.
bool segments_ok(const int64_t* seg, int32_t n, int64_t batch, int64_t seq_q) {
  if (!seg || n < 1 || n > 3) return false;
  int64_t end = 0;
  for (int s = 0; s < n; ++s) {
    const int64_t off = seg[3 * s], rows = seg[3 * s + 1], base = seg[3 * s + 2];
    if (off < end || rows < 0 || base < 0 || off + rows > seq_q) return false;
    if (base + batch * rows > (int64_t{1} << 31) - 1) return false;
    end = off + rows;
  }
  return true;
}

hipError_t attention_packed(const void* q, const void* kv_packed, const int64_t* packed_strides, void* o,
                            int32_t out_packed, const int64_t* segments, int32_t num_segments, int64_t batch,
                            int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t head_dim,
                            const int64_t* q_strides, const int64_t* o_strides, const float* key_bias,
                            int64_t key_bias_batch_stride, float scale, int32_t causal, const void* const* warm_ptrs,
                            const int64_t* warm_bytes, int32_t warm_count, hipStream_t stream) {
  const int64_t zero3[3] = {0, 0, 0};
  if (num_segments && (!out_packed || !segments_ok(segments, num_segments, batch, seq_q)))
    return hipErrorInvalidValue;
  if (out_packed) {
    // 1: O is the packed [seq_q, q_heads*head_dim] matrix; > 1: O is the
    // column range of a packed matrix out_packed columns wide that starts at
    // the 16-column chunk `o`; a batch needs the row segments
    if ((batch > 1 && !num_segments) || reinterpret_cast<uintptr_t>(o) % 16) return hipErrorInvalidValue;
    if (out_packed < 0 || (out_packed > 1 && (out_packed % 16 || out_packed < q_heads * head_dim)))
      return hipErrorInvalidValue;
    o_strides = zero3;
  }
  hipError_t e = check_qo(q, o, batch, q_heads, kv_heads, seq_q, seq_k, head_dim, q_strides, o_strides, scale);
  if (e != hipSuccess || batch == 0 || q_heads == 0 || seq_q == 0) return e;
  if (!kv_packed || !packed_strides || !a16(kv_packed)) return hipErrorInvalidValue;
  if (packed_strides[0] % 8 || packed_strides[1] % 8 ||
      packed_strides[1] < rldx_attention_kv_packed_elems(seq_k, head_dim) ||
      (batch > 1 && packed_strides[0] < kv_heads * packed_strides[1]))
    return hipErrorInvalidValue;
  if (key_bias && reinterpret_cast<uintptr_t>(key_bias) % 4) return hipErrorInvalidValue;
  AttnArgs a{};
  fill_qo(a, q, o, q_heads, kv_heads, seq_q, seq_k, q_strides, o_strides, key_bias, key_bias_batch_stride, scale);
  a.o_packed_k = out_packed > 1 ? out_packed : (out_packed ? q_heads * head_dim : 0);
  a.o_nseg = num_segments;
  for (int s = 0; s < num_segments; ++s) {
    a.o_seg_off[s] = static_cast<int>(segments[3 * s]);
    a.o_seg_rows[s] = static_cast<int>(segments[3 * s + 1]);
    a.o_seg_base[s] = static_cast<int>(segments[3 * s + 2]);
  }
  a.kv = static_cast<const uint16_t*>(kv_packed);
  a.kv_sb = packed_strides[0];
  a.kv_sh = packed_strides[1];
  if (!warm_ranges(warm_ptrs, warm_bytes, warm_count, a.warm)) return hipErrorInvalidValue;
  return launch_attn<false>(a, head_dim, static_cast<int>(batch), causal != 0, key_bias != nullptr, stream);
}
}  // namespace

extern "C" hipError_t rldx_attention_packed_fwd_bf16(const void* q, const void* kv_packed,
                                                     const int64_t* packed_strides, void* o, int32_t out_packed,
                                                     int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                                                     int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
                                                     const int64_t* o_strides, const float* key_bias,
                                                     int64_t key_bias_batch_stride, float scale, int32_t causal,
                                                     hipStream_t stream) {
  return attention_packed(q, kv_packed, packed_strides, o, out_packed, nullptr, 0, batch, q_heads, kv_heads, seq_q,
                          seq_k, head_dim, q_strides, o_strides, key_bias, key_bias_batch_stride, scale, causal,
                          nullptr, nullptr, 0, stream);
}

extern "C" hipError_t rldx_attention_packed_segments_fwd_bf16(
    const void* q, const void* kv_packed, const int64_t* packed_strides, void* o, int32_t out_packed,
    const int64_t* segments, int32_t num_segments, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
    int64_t seq_k, int64_t head_dim, const int64_t* q_strides, const float* key_bias, int64_t key_bias_batch_stride,
    float scale, int32_t causal, hipStream_t stream) {
  if (!out_packed || num_segments < 1) return hipErrorInvalidValue;
  return attention_packed(q, kv_packed, packed_strides, o, out_packed, segments, num_segments, batch, q_heads,
                          kv_heads, seq_q, seq_k, head_dim, q_strides, nullptr, key_bias, key_bias_batch_stride,
                          scale, causal, nullptr, nullptr, 0, stream);
}

extern "C" hipError_t rldx_attention_packed_fwd_warm_bf16(
    const void* q, const void* kv_packed, const int64_t* packed_strides, void* o, int32_t out_packed, int64_t batch,
    int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
    const int64_t* o_strides, const float* key_bias, int64_t key_bias_batch_stride, float scale, int32_t causal,
    const void* const* warm_ptrs, const int64_t* warm_bytes, int32_t warm_count, hipStream_t stream) {
  WarmRanges check;
  if (!warm_ranges(warm_ptrs, warm_bytes, warm_count, check)) return hipErrorInvalidValue;
  return attention_packed(q, kv_packed, packed_strides, o, out_packed, nullptr, 0, batch, q_heads, kv_heads, seq_q,
                          seq_k, head_dim, q_strides, o_strides, key_bias, key_bias_batch_stride, scale, causal,
                          warm_ptrs, warm_bytes, warm_count, stream);
}

extern "C" hipError_t rldx_attention_fwd_bf16(const void* q, const void* k, const void* v, void* o, int64_t batch,
                                              int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k,
                                              int64_t head_dim, const int64_t* q_strides,
                                              const int64_t* k_strides, const int64_t* v_strides,
                                              const int64_t* o_strides, const float* key_bias,
                                              int64_t key_bias_batch_stride, float scale, int32_t causal,
                                              void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  hipError_t e = check_qo(q, o, batch, q_heads, kv_heads, seq_q, seq_k, head_dim, q_strides, o_strides, scale);
  if (e != hipSuccess || batch == 0 || q_heads == 0 || seq_q == 0) return e;
  if (!k || !v || !k_strides || !v_strides) return hipErrorInvalidValue;
  const int64_t need = rldx_attention_workspace_bytes(batch, kv_heads, seq_k, head_dim);
  if (!workspace || workspace_bytes < need || !a16(workspace)) return hipErrorInvalidValue;
  const int64_t head_elems = rldx_attention_kv_packed_elems(seq_k, head_dim);
  const int64_t ps[2] = {kv_heads * head_elems, head_elems};
  e = rldx_attention_kv_pack_bf16(k, k_strides, v, v_strides, workspace, ps, batch, kv_heads, seq_k, head_dim,
                                  stream);
  if (e != hipSuccess) return e;
  return rldx_attention_packed_fwd_bf16(q, workspace, ps, o, 0, batch, q_heads, kv_heads, seq_q, seq_k, head_dim,
                                        q_strides, o_strides, key_bias, key_bias_batch_stride, scale, causal, stream);
}

extern "C" int64_t rldx_llm_fused_attention_workspace_bytes(int64_t seq, int64_t kv_heads, int64_t head_dim) {
  if (seq < 0 || kv_heads < 0 || head_dim < 0) return -1;
  // the packed K/V tiles of the Hkv heads
  return kv_heads * rldx_attention_kv_packed_elems(seq, head_dim) * 2;
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
  if (!a16(qkv) || !a16(out) || !a16(cos) || !a16(sin) || !a16(workspace) || !a16(q_norm_w) || !a16(k_norm_w))
    return hipErrorInvalidValue;
  if (seq > (1 << 24) || q_heads > 65535) return hipErrorInvalidValue;
  const uint16_t* base = static_cast<const uint16_t*>(qkv);
  uint16_t* kvp = static_cast<uint16_t*>(workspace);  // packed K/V tiles
  const int64_t head_elems = rldx_attention_kv_packed_elems(seq, head_dim);
  // 1) K: RMSNorm + rotate-half RoPE straight into the packed tiles, V packed by
  //    the same launch (Q is done inside the attention kernel)
  hipError_t e = gqa_k_norm_rope_kv_pack(base + q_heads * head_dim, base + (q_heads + kv_heads) * head_dim,
                                         qkv_row_stride, static_cast<const uint16_t*>(k_norm_w),
                                         static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin),
                                         cos_row_stride, sin_is_signed != 0, seq, kv_heads, head_dim, eps, kvp,
                                         head_elems, stream);
  if (e != hipSuccess) return e;
  // 2) causal GQA attention, Q normalised in the prologue
  AttnArgs a{};
  const int64_t q_strides[3] = {0, head_dim, qkv_row_stride};
  const int64_t o_strides[3] = {0, head_dim, out_row_stride};
  fill_qo(a, base, out, q_heads, kv_heads, seq, seq, q_strides, o_strides, nullptr, 0,
          1.0f / __builtin_sqrtf(static_cast<float>(head_dim)));
  a.kv = kvp;
  a.kv_sb = 0;
  a.kv_sh = head_elems;
  a.q_norm_w = static_cast<const uint16_t*>(q_norm_w);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.cs_ss = cos_row_stride;
  a.eps = eps;
  a.sin_signed = sin_is_signed ? 1 : 0;
  return launch_attn<true>(a, head_dim, 1, true, false, stream);
}

// ---------------------------------------------------------------------------
// rldx_backbone::fused_attention without allocation: the packed K/V tiles live
// in a file-scope device array instead of a caller workspace.  Each GPU holds
// its own copy of the array (RLDX_LLM_ATTN_NOALLOC_MAX_BYTES) until the
// process ends; host code reaches it only through the per-device address that
// hipGetSymbolAddress returns (the array's name is a host-side stand-in).
//
// Calls on one GPU are serialised on the device: each call's stream waits for
// the event recorded after the previous call's launches (on whatever stream
// that was), and records it again after its own; a process-wide mutex makes
// wait + launches + record one step, so host threads cannot interleave them.
// A stream under hipGraph capture skips the event (the graph's replays are
// ordered by the stream they are launched on).  The address and the event are
// set up once per device, on the first call there.
// ---------------------------------------------------------------------------
namespace {
static __device__ __align__(256) unsigned char scratch[RLDX_LLM_ATTN_NOALLOC_MAX_BYTES];

constexpr int kMaxDevices = 64;
struct ScratchSlot {
  void* ptr = nullptr;
  hipEvent_t done = nullptr;  // recorded after the last call's launches on this device
};
std::mutex g_scratch_mutex;  // held for the whole of a call
ScratchSlot g_scratch[kMaxDevices];

// The current device's slot, set up on the first call there (caller holds the mutex).
hipError_t scratch_on_current_device(ScratchSlot** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  ScratchSlot& s = g_scratch[dev];
  if (s.ptr == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return e;
    s.done = ev;
    s.ptr = p;
  }
  *out = &s;
  return hipSuccess;
}
}  // namespace

extern "C" hipError_t rldx_llm_fused_attention_noalloc_bf16(const void* qkv, int64_t qkv_row_stride,
                                                            const void* q_norm_w, const void* k_norm_w,
                                                            const void* cos, const void* sin, int64_t cos_row_stride,
                                                            int32_t sin_is_signed, void* out, int64_t out_row_stride,
                                                            int64_t seq, int64_t q_heads, int64_t kv_heads,
                                                            int64_t head_dim, float eps, hipStream_t stream) {
  const int64_t need = rldx_llm_fused_attention_workspace_bytes(seq, kv_heads, head_dim);
  if (need < 0 || need > RLDX_LLM_ATTN_NOALLOC_MAX_BYTES) return hipErrorInvalidValue;  // beyond the scratch array
  if (seq == 0) return rldx_llm_fused_attention_bf16(qkv, qkv_row_stride, q_norm_w, k_norm_w, cos, sin,
                                                     cos_row_stride, sin_is_signed, out, out_row_stride, seq, q_heads,
                                                     kv_heads, head_dim, eps, nullptr, 0, stream);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  ScratchSlot* slot = nullptr;
  hipError_t e = scratch_on_current_device(&slot);
  if (e != hipSuccess) return e;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(stream, &cap);
  if (e != hipSuccess) return e;
  const bool ordered = cap == hipStreamCaptureStatusNone;
  if (ordered) {  // wait for the previous call on this device, whichever stream it used
    e = hipStreamWaitEvent(stream, slot->done, 0);
    if (e != hipSuccess) return e;
  }
  e = rldx_llm_fused_attention_bf16(qkv, qkv_row_stride, q_norm_w, k_norm_w, cos, sin, cos_row_stride, sin_is_signed,
                                    out, out_row_stride, seq, q_heads, kv_heads, head_dim, eps, slot->ptr,
                                    RLDX_LLM_ATTN_NOALLOC_MAX_BYTES, stream);
  if (e != hipSuccess || !ordered) return e;
  return hipEventRecord(slot->done, stream);
}

extern "C" int64_t rldx_vision_attention_workspace_bytes(int64_t total_tokens, int64_t num_seqs, int64_t num_heads,
                                                          int64_t head_dim) {
  const int dp = vit_padded_dim(head_dim);
  if (total_tokens < 0 || num_seqs < 0 || num_heads < 0 || dp == 0) return -1;
  // padded Q [H][rows][DP] (rounded up to 256 bytes), then the packed K/V slots of the H heads
  const int64_t q_bytes = (num_heads * total_tokens * dp * 2 + 255) / 256 * 256;
  return q_bytes + num_heads * seq_slot_count(total_tokens, num_seqs) * kv_tile_elems(dp) * 2;
}

extern "C" hipError_t rldx_vision_attention_bf16(const void* qkv, const float* rope_cos, const float* rope_sin,
                                                 const int32_t* cu_seqlens, int64_t num_seqs, void* out,
                                                 int64_t total_tokens, int64_t num_heads, int64_t head_dim,
                                                 float scaling, void* workspace, int64_t workspace_bytes,
                                                 hipStream_t stream) {
  const int dp = vit_padded_dim(head_dim);
  if (dp == 0 || total_tokens < 0 || num_heads <= 0 || num_seqs <= 0) return hipErrorInvalidValue;
  if (!(scaling > 0.f) || scaling == __builtin_inff()) return hipErrorInvalidValue;
  if (total_tokens == 0) return hipSuccess;
  if (!qkv || !rope_cos || !rope_sin || !cu_seqlens || !out || !workspace) return hipErrorInvalidValue;
  if (!a16(qkv) || !a16(rope_cos) || !a16(rope_sin) || !a16(workspace) || reinterpret_cast<uintptr_t>(out) % 8 ||
      reinterpret_cast<uintptr_t>(cu_seqlens) % 4)
    return hipErrorInvalidValue;
  if (total_tokens > (1 << 24) || num_seqs > (1 << 24) || num_heads > 65535) return hipErrorInvalidValue;
  if (total_tokens * dp * 2 > (int64_t{1} << 31) - 1) return hipErrorInvalidValue;  // 32-bit row offsets of Q
  const int64_t slots = seq_slot_count(total_tokens, num_seqs);
  // 1-D attention grid, 32-bit byte offsets inside a head's packed tiles
  if (slots * num_heads > (int64_t{1} << 31) - 1 || slots * kv_tile_elems(dp) * 2 > (int64_t{1} << 31) - 1)
    return hipErrorInvalidValue;
  if (workspace_bytes < rldx_vision_attention_workspace_bytes(total_tokens, num_seqs, num_heads, head_dim))
    return hipErrorInvalidValue;
  const int64_t q_bytes = (num_heads * total_tokens * dp * 2 + 255) / 256 * 256;
  VitArgs v{};
  v.qkv = static_cast<const uint16_t*>(qkv);
  v.cos = rope_cos;
  v.sin = rope_sin;
  v.cu_seqlens = cu_seqlens;
  v.qpad = static_cast<uint16_t*>(workspace);
  v.kvp = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + q_bytes);
  v.kv_sh = slots * kv_tile_elems(dp);
  v.num_seqs = static_cast<int>(num_seqs);
  v.rows = static_cast<int>(total_tokens);
  v.heads = static_cast<int>(num_heads);
  v.hd = static_cast<int>(head_dim);
  AttnArgs a{};
  a.q = v.qpad;
  a.q_sh = total_tokens * dp;
  a.q_ss = dp;
  a.kv = v.kvp;
  a.kv_sh = v.kv_sh;
  a.o = static_cast<uint16_t*>(out);
  a.o_sh = head_dim;
  a.o_ss = num_heads * head_dim;
  a.hq = a.hkv = v.heads;
  a.group = 1;
  a.scale_log2 = scaling * kLog2e;
  a.cu_seqlens = cu_seqlens;
  a.num_seqs = v.num_seqs;
  a.total_rows = v.rows;
  a.d_store = v.hd;
  if (dp == 64) return launch_vit<64>(v, a, slots, stream);
  if (dp == 96) return launch_vit<96>(v, a, slots, stream);
  return launch_vit<128>(v, a, slots, stream);
}

extern "C" hipError_t rldx_memory_attention_bf16(const void* qkv, const void* cos, const void* signed_sin, void* out,
                                                 int64_t tokens, int64_t num_heads, int64_t head_dim,
                                                 int64_t block_attn_size, hipStream_t stream) {
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return hipErrorInvalidValue;
  if (tokens < 0 || num_heads <= 0 || block_attn_size <= 0) return hipErrorInvalidValue;
  if (tokens == 0) return hipSuccess;
  if (!qkv || !cos || !signed_sin || !out) return hipErrorInvalidValue;
  if (!a16(qkv) || !a16(cos) || !a16(signed_sin) || reinterpret_cast<uintptr_t>(out) % 8) return hipErrorInvalidValue;
  if (tokens > (1 << 24) || num_heads > 65535) return hipErrorInvalidValue;
  MemArgs a{};
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.cos = static_cast<const uint16_t*>(cos);
  a.signed_sin = static_cast<const uint16_t*>(signed_sin);
  a.out = static_cast<uint16_t*>(out);
  a.m = static_cast<int>(tokens);
  a.heads = static_cast<int>(num_heads);
  a.block = block_attn_size;
  a.scale_log2 = kLog2e / __builtin_sqrtf(static_cast<float>(head_dim));
  const dim3 grid(static_cast<unsigned>((tokens + 31) / 32), static_cast<unsigned>(num_heads));
  if (head_dim == 64)
    hipLaunchKernelGGL(mem_attn_kernel<64>, grid, dim3(512), 0, stream, a);
  else if (head_dim == 128)
    hipLaunchKernelGGL(mem_attn_kernel<128>, grid, dim3(512), 0, stream, a);
  else
    hipLaunchKernelGGL(mem_attn_kernel<256>, grid, dim3(512), 0, stream, a);
  return hipGetLastError();
}
