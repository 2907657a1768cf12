// Grouped bf16 GEMM for the linears of an MSAT block on gfx950 (CDNA4):
//   y_s = x_s W_s^T + b_s  for up to 3 streams s in one launch, fp32 accumulation
// on v_mfma_f32_32x32x16_bf16, with the block's epilogues fused:
//   bias            out = bf16(y)                                (nn.Linear)
//   residual        out = bf16(res + bf16(y))                    (x_s += Proj_s(o_s), x_s += W3_s(...))
//   SwiGLU          out = swiglu(bf16(y_gate), bf16(y_up))       (W12_s followed by SwiGLU),
//                   row-major or in the packed activation order (the next GEMM's A)
//   residual, packed   the residual epilogue on a residual stream held in the
//                   packed activation order (read and written in place)
// and optionally the block's pre-LayerNorm (no affine) folded in: with the row
// sums s_n = sum_k W[n][k], LN(x) W^T = rstd (x W^T - mean s), so the GEMM
// takes the un-normalised rows x as its A operand and applies
// y = rstd acc - (rstd mean) s_n before the epilogue.  The row statistics come
// from the producer of x: the residual epilogue (or the activation-pack
// kernel) writes, per 64-column slot and row, the sum and the sum of squares
// of the bf16 values it stores ([k / 64][m][2], slot-major, so that a wave's
// loads of one slot for 64 consecutive rows are contiguous); the consumer
// loads its rows' slots before its K loop and sums them outside it.  No LayerNorm-pack launch and no
// normalised copy of x; the result differs from the eager chain only by the
// bf16 rounding of LN(x) it skips.
// The rounding points are those of the eager chain (addmm to bf16, then the
// bf16 add / SwiGLU), rldx/model/modules/action_model/blocks.py:705-891 and
// rldx/model/modules/action_model/ops.py:137-161.  The SwiGLU epilogue replaces
// _fused_mlp_swiglu_kernel behind ss::fused_mlp_swiglu
// (rldx/inference/action_model/single_stream/engine/kernels/fused_mlp_swiglu.py:199-267).
//
// Design (the limits it is built around, measured on MI355X: a CU's vector
// memory path delivers ~48 B/clk from L2, ~32 TB/s over the chip; ds_read_b128
// ~228 B/clk per CU, ds_write_b128 only ~74 B/clk)
//   * Operands are stored in the MFMA operand order: 1 KB chunks, one wave-wide
//     16-byte load per chunk.  Weights are packed once (pack_weight_kernel):
//     chunk (nb, kb) holds W[32 nb + l%32][16 kb + 8 (l/32) + i] for lane l,
//     element i, the chunks of one 32-column block contiguous along K.
//     Activations arrive packed the same way from their producers (the
//     LayerNorm-pack kernel, the attention kernel, the SwiGLU epilogue).
//   * A workgroup of 8 waves computes a (32 MB) x (32 NB) tile.  Per k-step the
//     tile's MB + NB chunks are loaded once, straight into LDS (buffer_load ...
//     lds: no VGPR staging, no ds_write), into a ring of NSLOT stages of two
//     k-steps; every wave reads the chunks of its m-block and n-blocks with
//     ds_read_b128 one stage ahead.  Sharing operands through LDS is what cuts
//     the L2 -> CU traffic: a 128 x 128 tile moves half the bytes per flop of a
//     64 x 64 one.
//   * Tile shapes: 128 x 128 (waves 4 x 2, 32 x 64 each) for long streams with
//     enough tiles; 64 x 64 (waves 2 x 2 in two K-groups) and 32 x 64 (waves
//     1 x 2 in four K-groups) for the short streams and the N = 1536 GEMMs.
//     K-groups take alternate stages; their partial tiles are summed in a
//     fixed order, so results are deterministic.
//   * Stage pipeline per wave: issue the loads of stage s + NSLOT - 1, MFMAs of
//     the first k-step of stage s, wait for stage s + 1 and barrier, read stage
//     s + 1 from LDS, MFMAs of the second k-step (they cover the read latency).
//   * MFMAs take (W chunk, A chunk), so each accumulator holds a transposed
//     block: lane l32 = row, (q4, g, e) = 4 consecutive columns.  Epilogue:
//     fp32 tiles in LDS, then every thread reduces the K-groups for 8
//     consecutive columns of a row, applies the epilogue and stores 16 bytes.
//   * Launch: workgroup b runs on XCD b % 8.  Each stream's workgroups start at
//     a multiple of 8 and give each XCD a contiguous run of tiles (the m-tiles
//     of a column block share its weight panel in that XCD's L2).  Streams are
//     launched heaviest first; two workgroups fit on a CU (<= 72 KB LDS,
//     <= 128 VGPRs), so the short streams' weight streaming runs beside the
//     long stream's tiles.
#include "rldx_amd.h"
#include "rldx_common.h"

namespace rldx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kXcds = 8;
constexpr int kThreads = 512;          // 8 waves per workgroup
constexpr int kBufWord3 = 0x00020000;  // gfx9 raw buffer descriptor, word 3 (untyped dword data)

enum {
  kEpiBias = 0,
  kEpiResidual = 1,
  kEpiSwiglu = 2,
  kEpiSwigluPacked = 3,
  kEpiBiasPacked = 4,
  kEpiResidualPacked = 5,
  kEpiQkv = 16,   // internal: rldx_grouped_gemm_qkv_norm_rope_bf16, head_dim 128
  kEpiQkv64 = 17  // the same, head_dim 64 (two heads per 128-column tile)
};
constexpr bool qkv_epi(int epi) { return epi == kEpiQkv || epi == kEpiQkv64; }
constexpr bool packed_out(int epi) {
  return epi == kEpiSwigluPacked || epi == kEpiBiasPacked || epi == kEpiResidualPacked;
}
constexpr bool residual_epi(int epi) { return epi == kEpiResidual || epi == kEpiResidualPacked; }
enum { kTile128 = 0, kTile64 = 1, kTile32 = 2, kTile64x128 = 3, kTile32x128 = 4 };

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

// Tile configuration: MB x NB blocks of 32 x 32; each wave covers one m-block
// and BNW n-blocks; the 8 waves form KG K-groups (stage s of group g covers
// k-steps (s KG + g) U .. + U - 1); NSLOT stages of the LDS ring.
template <int MB_, int NB_, int BNW_, int NSLOT_>
struct TileCfg {
  static constexpr int MB = MB_, NB = NB_, BNW = BNW_, NSLOT = NSLOT_;
  static constexpr int U = 2;                       // k-steps per stage
  static constexpr int WN = NB / BNW;               // waves along n
  static constexpr int WPG = MB * WN;               // waves per K-group
  static constexpr int KG = 8 / WPG;                // K-groups
  static constexpr int CH = MB + NB;                // 1 KB chunks per k-step
  static constexpr int ND = U * CH / WPG;           // chunks each wave loads per stage
  static constexpr int RING = KG * NSLOT * U * CH;  // ring size in chunks
  static constexpr int TP = 32 * NB + 4;            // fp32 tile pitch (rows shift 4 banks)
  static constexpr int TILE = 32 * MB * TP;         // floats per K-group tile
  static_assert(WPG * KG == 8 && (U * CH) % WPG == 0, "tile configuration");
  static_assert(NB % 2 == 0, "SwiGLU tiles pair gate / up blocks");
};
using Cfg128 = TileCfg<4, 4, 2, 4>;
using Cfg64 = TileCfg<2, 2, 1, 4>;
using Cfg32 = TileCfg<1, 2, 1, 3>;
// Whole 128-column heads for the QKV epilogue on streams too short for 128 x
// 128 tiles: 64 x 128 (waves 2 x 2, two K-groups) and 32 x 128 (waves 1 x 2,
// four K-groups) -- the K-groups of 64 x 64 and 32 x 64, so the sums are the
// same as theirs, bit for bit.
using Cfg64x128 = TileCfg<2, 4, 2, 3>;
using Cfg32x128 = TileCfg<1, 4, 2, 2>;
// Deep rings for launches of at most one workgroup per CU: one workgroup alone
// on a CU is latency-bound with the rings above (~48 KB of loads in flight,
// about half of what a CU can stream); these keep ~80-96 KB in flight.  Deeper
// rings (8 / 8 / 6 slots, 112-120 KB) measured slower: every workgroup issues
// its first NSLOT - 1 stages at once, and that initial burst of weight reads
// delays the first stage longer than the extra depth gains in the loop.
using Cfg128D = TileCfg<4, 4, 2, 6>;
using Cfg64D = TileCfg<2, 2, 1, 6>;
using Cfg32D = TileCfg<1, 2, 1, 5>;
using Cfg64x128D = TileCfg<2, 4, 2, 6>;
using Cfg32x128D = TileCfg<1, 4, 2, 3>;

constexpr int cmax(int a, int b) { return a > b ? a : b; }
// The ring during the K loop; afterwards the fp32 tiles of the K-groups and,
// behind them, the LayerNorm-fold partial row statistics (Σx, Σx² over the
// slots of each thread: 512 pairs).
template <class C>
constexpr int ln_stats_off() { return C::KG * C::TILE; }  // floats
// The register epilogue of tiles with one K-group and gate / up n-block pairs
// keeps its LayerNorm partial pairs (512 threads) and row factors past the ring.
template <class C>
constexpr int reg_ln_bytes() { return C::KG == 1 && C::BNW == 2 ? C::RING * 1024 + (2 * 512 + 2 * 32 * C::MB) * 4 : 0; }
template <class C>
constexpr int lds_bytes() { return cmax(cmax(C::RING * 1024, (ln_stats_off<C>() + 2 * 512) * 4), reg_ln_bytes<C>()); }
// LayerNorm statistics [k / 64][m][2]: thread t of a tile of R rows sums slots
// [q SPL, (q + 1) SPL) of row t % R (q = t / R, SPL = ceil(slots R / 512)),
// at most kLnSlotsMax (k <= 2048 at 128-row tiles).
constexpr int kLnSlotsMax = 8;
// The last kLdsTail bytes of a kernel's LDS: the SwiGLU tiles' W row sums
// (gate and up of at most 64 output columns, fp32, stored at the prologue for
// the LayerNorm fold of the epilogue; kernels without WIDE tiles, whose rings
// leave room behind them), the biases of the same columns (fp32, for the
// register epilogue of the packed SwiGLU tiles), then 16 bytes holding the
// split-K arrival flag, used by every kernel (in a WIDE kernel inside its ring
// area, past its epilogue).
constexpr int kWsumStash = 2 * 64 * 4;
constexpr int kBiasStash = 2 * 64 * 4;
constexpr int kLdsTail = kWsumStash + kBiasStash + 16;
template <class C>
constexpr int epi_bytes() { return (ln_stats_off<C>() + 2 * 512) * 4; }  // fp32 tiles + row statistics
constexpr int kLdsBytes =
    cmax(lds_bytes<Cfg128>(), cmax(lds_bytes<Cfg64>(), lds_bytes<Cfg32>())) + kLdsTail;
static_assert(kLdsBytes <= 80 * 1024, "two workgroups per CU");
constexpr int kLdsDeep = cmax(lds_bytes<Cfg128D>(), cmax(lds_bytes<Cfg64D>(), lds_bytes<Cfg32D>())) + kLdsTail;
static_assert(kLdsDeep <= 160 * 1024 && kLdsDeep >= kLdsBytes, "one workgroup per CU");
constexpr int kLdsQkv = cmax(lds_bytes<Cfg128>(), cmax(lds_bytes<Cfg64x128>(), lds_bytes<Cfg32x128>()));
constexpr int kLdsQkvDeep = cmax(lds_bytes<Cfg128D>(), cmax(lds_bytes<Cfg64x128D>(), lds_bytes<Cfg32x128D>()));
static_assert(kLdsQkv <= 80 * 1024 && kLdsQkvDeep <= 160 * 1024, "QKV epilogue tiles");
static_assert(kLdsQkv - 16 >= cmax(epi_bytes<Cfg128>(), cmax(epi_bytes<Cfg64x128>(), epi_bytes<Cfg32x128>())) &&
                  kLdsQkvDeep - 16 >=
                      cmax(epi_bytes<Cfg128D>(), cmax(epi_bytes<Cfg64x128D>(), epi_bytes<Cfg32x128D>())),
              "the split-K flag of a WIDE kernel lies past its epilogue tiles");

struct Group {
  const uint16_t* a;  // packed activations
  const uint16_t* w;  // packed weight
  const uint16_t* bias;
  uint16_t* out;
  const uint16_t* res;
  int64_t ldo, ldr;
  int m, cfg, m_tiles, items;  // items = tiles x splits
  int n, k;                     // this group's W [n, k] (n = 2 N_half with the SwiGLU epilogues)
  int wg_begin, per_xcd;        // first workgroup (multiple of 8); items per XCD
  int splits, ls_per;           // K splits across workgroups; K-group stages per split
  float* part;                  // split partials [tile][split][PER][512 threads][V]
  unsigned* cnt;                // per-tile arrival counters (zero between launches)
  // QKV epilogue: first row of the stream in the joint sequence, its Q / K
  // RMSNorm weights [128] and fp32 RoPE tables [m, 64] (row stride rope_ld) or null
  int m_begin, rope_ld;
  const uint16_t *qn_w, *kn_w;
  const float *cos, *sin;
  // LayerNorm fold: fp32 row sums of W [n] (original row order) and the
  // statistics of the A rows [m][k / 64][2] (both set, or both null)
  const float* wsum;
  const float* lnstats;
  // residual epilogues: statistics of the output rows [m][n / 64][2], or null
  float* stats_out;
};

// Outputs of the QKV epilogue: Q (H, M, 128) with strides (q_sh, q_sm), and the
// packed K/V tiles of the attention kernel, head h at kvp + h * kvp_sh.
struct QkvOut {
  uint16_t* q;
  uint16_t* kvp;
  int64_t q_sh, q_sm, kvp_sh;
  int inner;  // heads * head_dim (a multiple of 128): columns of each of Q, K, V
  float eps;
};

struct GemmArgs {
  Group g[3];
  int num_groups;
  int n, k;  // the first group's n, k (every group's with a uniform call); n = rows of W (2 N_half with SwiGLU)
  QkvOut qkv;
  int spread;    // != 0: the splits of a tile on different XCDs (RLDX_GEMM_SPLITS_ACROSS_XCDS)
  float ln_eps;  // LayerNorm fold (kernels instantiated with LN)
};

// y' = rstd y - (rstd mean) s: the LayerNorm fold of one accumulator (one
// fused multiply-add, so every epilogue computes the same bits)
__device__ __forceinline__ float ln_fold(float y, float rs, float rm, float s) {
  return __builtin_fmaf(rs, y, -(rm * s));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const uint16_t* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p), 0, bytes, kBufWord3);
}

// Wait until at most N of this wave's loads are in flight, then barrier.  Inline
// assembly: a release fence would also wait for every LDS-bound load.
template <int N>
__device__ __forceinline__ void wait_barrier() {
  static_assert(N == 0 || N == 3 || N == 4 || N == 5 || N == 8 || N == 9 || N == 12, "vmcnt immediate");  // (NSLOT - 2) * ND
  if constexpr (N == 12) asm volatile("s_waitcnt vmcnt(12) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (N == 9) asm volatile("s_waitcnt vmcnt(9) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (N == 5) asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (N == 3) asm volatile("s_waitcnt vmcnt(3) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// K (the kernel's WIDE) only keeps the tile specializations of the wide and
// narrow kernels apart: the host compilation pass rejects a second caller of a
// specialization whose body holds the 16-byte LDS-load builtin.  DP: the
// kernel is a deep-ring instantiation (one workgroup per CU).  TR: the MFMAs
// take (A chunk, W chunk), so each accumulator holds its block untransposed
// (the V tiles of the QKV epilogue, whose lanes then hold packed V chunks).
template <class C, int EPI, bool K, bool LN, bool DP, bool TR = false>
__device__ __forceinline__ void gemm_tile(const GemmArgs& a, const Group& G, int item, u32x4* lds, float* wsl) {
  constexpr bool kSwiglu = EPI == kEpiSwiglu || EPI == kEpiSwigluPacked;
  constexpr int MB = C::MB, NB = C::NB, BNW = C::BNW, U = C::U, CH = C::CH, NSLOT = C::NSLOT;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int grp = wv / C::WPG, wl = wv % C::WPG;
  const int wm = wl / C::WN, wn = wl % C::WN;
  const int l32 = lane & 31, g = lane >> 5;
  const int tile = item / G.splits, split = item % G.splits;
  const int mt = tile % G.m_tiles, nt = tile / G.m_tiles;
  const int ksteps = G.k / 16;
  const int lstages = G.ls_per;         // K-group stages of this split
  const int st0 = split * G.ls_per;     // its first stage
  const int mblocks = (G.m + 31) / 32, nblocks = G.n / 32;

  // The chunks this wave loads per stage: q = wl + j WPG, k-step q / CH, chunk
  // q % CH (m-blocks first, then n-blocks; blocks past the edge re-read the
  // last one: rows / columns that are never stored).
  __amdgpu_buffer_rsrc_t rs[C::ND];
  int qoff[C::ND];
#pragma unroll
  for (int j = 0; j < C::ND; ++j) {
    const int q = wl + j * C::WPG, u = q / CH, c = q % CH;
    if (c < MB) {
      rs[j] = rsrc(G.a, mblocks * ksteps * 1024);
      qoff[j] = (min(mt * MB + c, mblocks - 1) * ksteps + u) * 1024;
    } else {
      rs[j] = rsrc(G.w, nblocks * ksteps * 1024);
      qoff[j] = (min(nt * NB + c - MB, nblocks - 1) * ksteps + u) * 1024;
    }
  }
  u32x4* ring = lds + grp * NSLOT * U * CH * 64;
  auto dma = [&](int st, int slot) {
    const int ks = ((st0 + min(st, lstages - 1)) * C::KG + grp) * U * 1024;
#pragma unroll
    for (int j = 0; j < C::ND; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs[j], (__attribute__((address_space(3))) void*)(ring + (slot * U * CH + wl + j * C::WPG) * 64), 16,
          lane * 16, qoff[j] + ks, 0, 0);
  };
  u32x4 xa[2][U], xw[2][U][BNW];
  auto lread = [&](int b, int slot) {
    const u32x4* s = ring + slot * U * CH * 64 + lane;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xa[b][u] = s[(u * CH + wm) * 64];
#pragma unroll
      for (int bb = 0; bb < BNW; ++bb) xw[b][u][bb] = s[(u * CH + MB + wn * BNW + bb) * 64];
    }
  };
  floatx16 acc[BNW];
#pragma unroll
  for (int bb = 0; bb < BNW; ++bb) acc[bb] = floatx16{};
  auto mma = [&](int b, int u) {
#pragma unroll
    for (int bb = 0; bb < BNW; ++bb) {
      if constexpr (TR)
        acc[bb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, xa[b][u]),
                                                          __builtin_bit_cast(bf16x8, xw[b][u][bb]), acc[bb], 0, 0, 0);
      else
        acc[bb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, xw[b][u][bb]),
                                                          __builtin_bit_cast(bf16x8, xa[b][u]), acc[bb], 0, 0, 0);
    }
  };

  // ---- epilogue operands, loaded before the K loop (in flight beside the ring
  // prologue instead of exposed at the end of the loop) ----
  constexpr int R = 32 * MB;                       // tile rows
  constexpr int OC = kSwiglu ? 16 * NB : 32 * NB;  // tile output columns
  constexpr int CPR = OC / 8;                      // 16-byte output chunks per row
  constexpr int PER = (R * CPR + kThreads - 1) / kThreads;
  static_assert(kThreads % CPR == 0, "a thread keeps its column chunk");
  const int n_out = kSwiglu ? G.n / 2 : G.n;
  const int cc = 8 * (static_cast<int>(threadIdx.x) % CPR);
  const int col = nt * OC + cc;  // global output column of this thread's chunks
  const bool col_ok = col < n_out;
  // residual chunks (each is read and written by this thread, so it may alias the output)
  // Register epilogue of the packed residual epilogue on 64 x 64 tiles (two
  // K-groups of 2 x 2 waves, one n-block per wave) in the deep kernels: each
  // K-group finishes half of the tile's 8-column chunks (see there).
  constexpr bool kRegRes = EPI == kEpiResidualPacked && C::MB == 2 && C::NB == 2 && BNW == 1 && C::KG == 2 && DP;
  const bool reg_res = kRegRes && G.splits == 1;
  u32x4 pres[PER];
  if constexpr (residual_epi(EPI)) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      pres[i] = u32x4{0, 0, 0, 0};
      if (reg_res) continue;
      const int t = static_cast<int>(threadIdx.x) + kThreads * i;
      const int row = mt * R + t / CPR;
      const int64_t off = EPI == kEpiResidualPacked ? packed_act_offset(row, col, G.ldr)
                                                    : static_cast<int64_t>(row) * G.ldr + col;
      pres[i] = (t < R * CPR && row < G.m && col_ok) ? *reinterpret_cast<const u32x4*>(G.res + off)
                                                     : u32x4{0, 0, 0, 0};
    }
  }
  // biases of this thread's columns (gate and up for SwiGLU) as bf16 bits, packed
  // in pairs once loaded (at the prologue's wait).  No branch around the loads,
  // so all of them are in flight together: they go through a descriptor bounded
  // to the bias (a missing bias is an empty one: every read returns zero), and a
  // chunk past the output columns reads column 0's and is zeroed when packed.
  // Register epilogue (packed SwiGLU tiles of one K-group whose waves each hold
  // a gate / up n-block pair, no split-K): every lane finishes the outputs of
  // its own accumulators, so the fp32 tile never goes through LDS.  Its lanes
  // need the biases (and W row sums) of their accumulator columns, not of a
  // thread's output chunk: threads t < 2 OC load the bias of one column and
  // store it at the prologue's wait, as the row sums are.
  constexpr bool kRegEpi = EPI == kEpiSwigluPacked && C::KG == 1 && BNW == 2 && !K;
  const bool reg_epi = kRegEpi && G.splits == 1;
  // Register epilogue of the QKV epilogue (head_dim 128, one K-group, each
  // wave two n-blocks of a head; deep-ring kernels, whose 256 VGPRs hold its
  // operands): Q and K tiles (see there), and V tiles, which the launch runs
  // with TR accumulators.
  constexpr bool kRegQkv = EPI == kEpiQkv && C::KG == 1 && BNW == 2 && DP && !TR;
  const bool reg_qkv = kRegQkv && nt * OC / a.qkv.inner < 2;
  static_assert(!TR || (EPI == kEpiQkv && C::KG == 1 && BNW == 2 && DP), "TR: V tiles of the deep QKV launch");
  uint16_t braw[16];
  {
    const __amdgpu_buffer_rsrc_t brs = rsrc(G.bias, G.bias ? G.n * 2 : 0);
    const int bcol = col_ok ? col : 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) braw[i] = 0;
    if (!reg_epi && !reg_qkv && !reg_res) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        braw[i] = static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(brs, (bcol + i) * 2, 0, 0));
        braw[8 + i] = kSwiglu ? static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(brs, (G.n / 2 + bcol + i) * 2, 0, 0))
                              : uint16_t{0};
      }
    }
  }
  [[maybe_unused]] float bsv = 0.f;  // register epilogue: the bias of column t % OC (gate for t < OC, else up)
  if constexpr (kRegEpi) {
    const int t = static_cast<int>(threadIdx.x);
    const __amdgpu_buffer_rsrc_t brs = rsrc(G.bias, G.bias ? G.n * 2 : 0);
    const int bc = nt * OC + t % OC;
    if (reg_epi && t < 2 * OC && bc < n_out)
      bsv = bf(static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(brs, ((t < OC ? 0 : G.n / 2) + bc) * 2, 0, 0)));
  }
  uint32_t bpk[8];
  // LayerNorm fold: W row sums of this thread's columns (gate and up for SwiGLU).
  // The SwiGLU tiles keep theirs in LDS through the K loop (16 more live
  // registers would spill at two workgroups per CU): thread t < 2 OC loads one
  // with the prologue's loads and stores it at wsl[t] (gate sums, then up sums)
  // once the prologue's wait has passed; the epilogue reads them from there.
  // WIDE SwiGLU tiles, whose rings leave no room for it, load theirs after the
  // K loop.
  [[maybe_unused]] float wg[8], wu[8];
  [[maybe_unused]] float wsv = 0.f;
  constexpr bool kStash = LN && kSwiglu && !K;  // (WIDE rings fill their LDS)
  if constexpr (kStash) {
    const int t = static_cast<int>(threadIdx.x);
    if (t < 2 * OC && nt * OC + t % OC < n_out) wsv = G.wsum[(t < OC ? 0 : G.n / 2) + nt * OC + t % OC];
  }
  auto load_wsum_stash = [&]() {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      wg[i] = wsl[cc + i];
      wu[i] = wsl[OC + cc + i];
    }
  };
  auto load_wsum = [&]() {
    const floatx4 z = {0.f, 0.f, 0.f, 0.f};
    const floatx4* ws = reinterpret_cast<const floatx4*>(G.wsum + col);
    const floatx4 g0 = col_ok ? ws[0] : z, g1 = col_ok ? ws[1] : z;
    floatx4 u0 = z, u1 = z;
    if constexpr (kSwiglu) {
      const floatx4* wu4 = reinterpret_cast<const floatx4*>(G.wsum + G.n / 2 + col);
      u0 = col_ok ? wu4[0] : z;
      u1 = col_ok ? wu4[1] : z;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wg[i] = g0[i];
      wg[4 + i] = g1[i];
      wu[i] = u0[i];
      wu[4 + i] = u1[i];
    }
  };
  if constexpr (LN && !kSwiglu) load_wsum();
  // QKV epilogue: the Q or K RMSNorm weights of this thread's 8 columns of the
  // head; on a V tile the bias (and W row sum) of the one tile column the thread
  // packs (the same column on every pass of its V loop, see there)
  [[maybe_unused]] u32x4 qk_w = {0, 0, 0, 0};
  [[maybe_unused]] float v_bias = 0.f, v_wsum = 0.f;
  if constexpr (qkv_epi(EPI)) {
    constexpr int D = EPI == kEpiQkv ? 128 : 64;
    const int which = nt * OC / a.qkv.inner;
    if (which < 2) {
      if (!reg_qkv) qk_w = *reinterpret_cast<const u32x4*>((which == 0 ? G.qn_w : G.kn_w) + cc % D);
    } else if constexpr (!TR) {
      constexpr int NCH = D / 16;
      const int t = static_cast<int>(threadIdx.x);
      const int hh = t / (NCH * 64) % (OC / D), idx = t % (NCH * 64);
      const int d = hh * D + 32 * ((idx >> 6) >> 1) + (idx & 31);
      const __amdgpu_buffer_rsrc_t vbr = rsrc(G.bias, G.bias ? G.n * 2 : 0);  // no bias: reads zero
      v_bias = bf(static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(vbr, (nt * OC + d) * 2, 0, 0)));
      if constexpr (LN) v_wsum = G.wsum[nt * OC + d];
    }
  }
  // register QKV epilogue operands, loaded with the prologue's loads: for a Q
  // or K tile the biases and W row sums of the lane's 32 accumulator columns
  // and the norm weights of the 4 whole 8-column chunks it stores; for a V
  // tile (TR) the bias and W row sum of the lane's 2 columns
  [[maybe_unused]] uint32_t rq_b[2][4][2];
  [[maybe_unused]] floatx4 rq_ws[2][4];
  [[maybe_unused]] u32x4 rq_w[2][2];
  [[maybe_unused]] float rv_b[2] = {0.f, 0.f}, rv_ws[2] = {0.f, 0.f};
  if constexpr (kRegQkv) {
    if (reg_qkv) {
      const __amdgpu_buffer_rsrc_t brs = rsrc(G.bias, G.bias ? G.n * 2 : 0);  // no bias: reads zero
      const uint16_t* nw = nt * OC / a.qkv.inner == 0 ? G.qn_w : G.kn_w;
#pragma unroll
      for (int bb = 0; bb < 2; ++bb)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int c0 = nt * OC + 32 * (2 * wn + bb) + 8 * q4 + 4 * g;
          rq_b[bb][q4][0] = __builtin_amdgcn_raw_buffer_load_b32(brs, c0 * 2, 0, 0);
          rq_b[bb][q4][1] = __builtin_amdgcn_raw_buffer_load_b32(brs, c0 * 2 + 4, 0, 0);
          if constexpr (LN) rq_ws[bb][q4] = *reinterpret_cast<const floatx4*>(G.wsum + c0);
        }
#pragma unroll
      for (int bb = 0; bb < 2; ++bb)
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) rq_w[bb][pp] = *reinterpret_cast<const u32x4*>(nw + 64 * wn + 32 * bb + 16 * pp + 8 * g);
    }
  }
  if constexpr (TR) {
    const __amdgpu_buffer_rsrc_t brs = rsrc(G.bias, G.bias ? G.n * 2 : 0);
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      const int c0 = nt * OC + 32 * (2 * wn + bb) + l32;
      rv_b[bb] = bf(static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(brs, c0 * 2, 0, 0)));
      if constexpr (LN) rv_ws[bb] = G.wsum[c0];
    }
  }
  // register residual epilogue operands: the biases of the lane's columns in
  // the two chunks its K-group finishes, and the residual chunk it stores
  [[maybe_unused]] uint32_t rr_b[2][2];
  [[maybe_unused]] u32x4 rr_res = {0, 0, 0, 0};
  if constexpr (kRegRes) {
    if (reg_res) {
      const __amdgpu_buffer_rsrc_t brs = rsrc(G.bias, G.bias ? G.n * 2 : 0);  // no bias, or past n: reads zero
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c0 = nt * OC + 32 * wn + 8 * (2 * grp + j) + 4 * g;
        rr_b[j][0] = __builtin_amdgcn_raw_buffer_load_b32(brs, c0 * 2, 0, 0);
        rr_b[j][1] = __builtin_amdgcn_raw_buffer_load_b32(brs, c0 * 2 + 4, 0, 0);
      }
      const int row = mt * R + 32 * wm + l32, ocol = nt * OC + 32 * wn + 8 * (2 * grp + g);
      if (row < G.m && ocol < n_out) rr_res = *reinterpret_cast<const u32x4*>(G.res + packed_act_offset(row, ocol, G.ldr));
    }
  }
  // LayerNorm fold: this thread's slots of its row, loaded before the ring
  // (consecutive threads: consecutive rows of one slot, contiguous), summed at
  // the prologue's wait, where they are complete (older than every ring load)
  constexpr int RT = 32 * MB;  // tile rows
  [[maybe_unused]] f32x2_t lv[kLnSlotsMax];
  [[maybe_unused]] float lp1 = 0.f, lp2 = 0.f;
  const int ln_slots = G.k / 64, ln_spl = (ln_slots * RT + kThreads - 1) / kThreads;
  const int ln_q = static_cast<int>(threadIdx.x) / RT;
  if constexpr (LN) {
    const int row = min(mt * RT + static_cast<int>(threadIdx.x) % RT, G.m - 1);
    const f32x2_t* src = reinterpret_cast<const f32x2_t*>(G.lnstats) + row;
#pragma unroll
    for (int j = 0; j < kLnSlotsMax; ++j)
      lv[j] = src[static_cast<int64_t>(min(ln_q * ln_spl + j, ln_slots - 1)) * G.m];
  }
#pragma unroll
  for (int s = 0; s < NSLOT - 1; ++s) dma(s, s);
  // Register epilogue with the LayerNorm fold: the row factors are reduced here,
  // beside the ring fill, in LDS past the ring (the partial pairs of the
  // kThreads threads, then the R rows' factors), the same sums in the same order
  // as the store phase's reduction below; the prologue's barrier publishes them,
  // so the epilogue needs no barrier at all.
  float* const lnp = reinterpret_cast<float*>(lds) + C::RING * 256;
  constexpr bool kRegAny = kRegEpi || kRegQkv || TR;
  const bool reg_any = reg_epi || reg_qkv || TR;
  static_assert(!kRegAny || (kThreads == 512 && C::RING * 1024 + (2 * kThreads + 2 * R) * 4 <= reg_ln_bytes<C>()),
                "LayerNorm factors of the register epilogue past the ring");
  // the register Q / K epilogue's cross-wave exchange (8 waves x 64 lanes x 16 B) lies past the factors
  static_assert(!kRegQkv || C::RING * 1024 + (2 * kThreads + 2 * R) * 4 + 8 * 64 * 16 <= kLdsQkvDeep - 16,
                "QKV register epilogue exchange past the ring");
  if constexpr (kRegAny && LN) {
    if (reg_any) {
      float q1 = 0.f, q2 = 0.f;
#pragma unroll
      for (int j = 0; j < kLnSlotsMax; ++j)
        if (j < ln_spl && ln_q * ln_spl + j < ln_slots) {
          q1 += lv[j][0];
          q2 += lv[j][1];
        }
      lnp[2 * threadIdx.x] = q1;
      lnp[2 * threadIdx.x + 1] = q2;
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // (the ring loads stay in flight)
      const int r = static_cast<int>(threadIdx.x);
      if (r < R) {
        float s1 = lnp[2 * r], s2 = lnp[2 * r + 1];
#pragma unroll
        for (int pq = 1; pq < kThreads / R; ++pq) {
          s1 += lnp[(pq * R + r) * 2];
          s2 += lnp[(pq * R + r) * 2 + 1];
        }
        const float inv_k = 1.0f / static_cast<float>(G.k);
        const float mean = s1 * inv_k;
        const float var = __builtin_fmaxf(__builtin_fmaf(-mean, mean, s2 * inv_k), 0.f);
        const float rsd = __builtin_amdgcn_rsqf(var + a.ln_eps);
        lnp[2 * kThreads + 2 * r] = rsd;
        lnp[2 * kThreads + 2 * r + 1] = rsd * mean;
      }
    }
  }
  wait_barrier<(NSLOT - 2) * C::ND>();
  if constexpr (LN) {
#pragma unroll
    for (int j = 0; j < kLnSlotsMax; ++j)
      if (j < ln_spl && ln_q * ln_spl + j < ln_slots) {
        lp1 += lv[j][0];
        lp2 += lv[j][1];
      }
  }
  if constexpr (kStash) {  // read back after the K loop, whose barriers publish it
    if (static_cast<int>(threadIdx.x) < 2 * OC) wsl[threadIdx.x] = wsv;
  }
  if constexpr (kRegEpi) {
    if (reg_epi && static_cast<int>(threadIdx.x) < 2 * OC) wsl[kWsumStash / 4 + threadIdx.x] = bsv;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
    bpk[i] = col_ok ? static_cast<uint32_t>(braw[2 * i]) | (static_cast<uint32_t>(braw[2 * i + 1]) << 16) : 0u;
  lread(0, 0);
  int slot_next = 1, slot_dma = NSLOT - 1;  // ring slots of stages st + 1, st + NSLOT - 1
  for (int st = 0; st < lstages; st += 2) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      if (st + r >= lstages) break;
      dma(st + r + NSLOT - 1, slot_dma);  // past the last stage: re-loads it into a free slot
      __builtin_amdgcn_sched_barrier(0);
      mma(r, 0);
      __builtin_amdgcn_sched_barrier(0);
      wait_barrier<(NSLOT - 2) * C::ND>();  // stage st + r + 1 is in LDS
      __builtin_amdgcn_sched_barrier(0);
      lread(r ^ 1, slot_next);  // past the last stage: read, never used
      __builtin_amdgcn_sched_barrier(0);
      mma(r, 1);
      __builtin_amdgcn_sched_barrier(0);
      slot_next = slot_next + 1 == NSLOT ? 0 : slot_next + 1;
      slot_dma = slot_dma + 1 == NSLOT ? 0 : slot_dma + 1;
    }
  }

  if constexpr (kRegEpi) {
    if (reg_epi) {
      // Straight after the K loop: no operand of this epilogue is in the ring
      // (the stashes and the LayerNorm factors lie past it, written before the
      // prologue's barrier), so no wave waits for another.
      // Lane (l32, g) of wave (wm, wn) holds, for tile row 32 wm + l32, the gate
      // (acc[0]) and up (acc[1]) sums of the wave's output columns
      // 8 q4 + 4 g + c (element 4 q4 + c): the sums the fp32 tile would hand to
      // the store phase below, finished with the same arithmetic.
      const int r = 32 * wm + l32, row = mt * R + r;
      float rs = 0.f, rm = 0.f;
      if constexpr (LN) {
        rs = lnp[2 * kThreads + 2 * r];
        rm = lnp[2 * kThreads + 2 * r + 1];
      }
      const float* bst = wsl + kWsumStash / 4;  // biases: gate [0, OC), up [OC, 2 OC); W row sums likewise at wsl
      uint32_t od[4][2];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int oc = 32 * wn + 8 * q4 + 4 * g;
        const floatx4 bgv = *reinterpret_cast<const floatx4*>(bst + oc);
        const floatx4 buv = *reinterpret_cast<const floatx4*>(bst + OC + oc);
        float yg[4], yu[4];
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
          yg[c4] = acc[0][4 * q4 + c4];
          yu[c4] = acc[1][4 * q4 + c4];
        }
        if constexpr (LN) {
          const floatx4 wgv = *reinterpret_cast<const floatx4*>(wsl + oc);
          const floatx4 wuv = *reinterpret_cast<const floatx4*>(wsl + OC + oc);
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) {
            yg[c4] = ln_fold(yg[c4], rs, rm, wgv[c4]);
            yu[c4] = ln_fold(yu[c4], rs, rm, wuv[c4]);
          }
        }
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const uint32_t gp = pack_bf16x2(yg[2 * p] + bgv[2 * p], yg[2 * p + 1] + bgv[2 * p + 1]);
          const uint32_t up = pack_bf16x2(yu[2 * p] + buv[2 * p], yu[2 * p + 1] + buv[2 * p + 1]);
          od[q4][p] = swiglu_bf16x2(bf16x2_lo(gp), bf16x2_hi(gp), bf16x2_lo(up), bf16x2_hi(up));
        }
      }
      // 16-byte output chunks: chunk c8 (8 columns) of the wave's 32 is split
      // over the lanes l32 and l32 + 32 (lane half g holds its columns
      // 4 g .. 4 g + 3); the two swap halves so that lane half g stores chunk
      // 2 pp + g whole, pp = 0, 1.
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const uint32_t w0 = g == 0 ? od[2 * pp + 1][0] : od[2 * pp][0];
        const uint32_t w1 = g == 0 ? od[2 * pp + 1][1] : od[2 * pp][1];
        const uint32_t x0 = static_cast<uint32_t>(__shfl_xor(static_cast<int>(w0), 32, 64));
        const uint32_t x1 = static_cast<uint32_t>(__shfl_xor(static_cast<int>(w1), 32, 64));
        const u32x4 o = g == 0 ? u32x4{od[2 * pp][0], od[2 * pp][1], x0, x1}
                               : u32x4{x0, x1, od[2 * pp + 1][0], od[2 * pp + 1][1]};
        const int ocol = nt * OC + 32 * wn + 8 * (2 * pp + g);
        if (row < G.m && ocol < n_out) *reinterpret_cast<u32x4*>(G.out + packed_act_offset(row, ocol, G.ldo)) = o;
      }
      // the ring's re-loads past the last stage write LDS: none may still be in
      // flight when the workgroup ends and its LDS is released
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      return;
    }
  }
  if constexpr (kRegRes) {
    if (reg_res) {
      // Lane (l32, g) of wave (wm, wn) in K-group hg holds that group's partial
      // sums for tile row 32 wm + l32 and columns 32 wn + 8 q4 + 4 g + c
      // (element 4 q4 + c).  K-group hg finishes chunks q4 = 2 hg, 2 hg + 1 of
      // the wave's 32 columns: it hands the other group its partials of the
      // other two chunks (through LDS past the ring; the ring's last re-loads may
      // still be in flight), adds the other group's partials of its own two, and
      // then runs the store phase's arithmetic: bias, a swap of halves with lane
      // l ^ 32 so that it stores chunk 2 hg + g whole, the residual, and the row
      // statistics with the store phase's butterfly over the row's 8 chunks
      // (chunk 4 wn + 2 hg + g: ^4 is the group's other wave, ^2 the other
      // group, both through LDS, ^1 lane l ^ 32).
      static_assert(C::RING * 1024 + 8 * 64 * (32 + 8) <= kLdsDeep - kLdsTail, "residual exchange past the ring");
      const int hg = grp;
      floatx4* const xp = reinterpret_cast<floatx4*>(lnp);  // [8 waves][64 lanes][2 float4]
      const floatx4 lo4 = floatx4{acc[0][0], acc[0][1], acc[0][2], acc[0][3]};
      const floatx4 lo8 = floatx4{acc[0][4], acc[0][5], acc[0][6], acc[0][7]};
      const floatx4 hi4 = floatx4{acc[0][8], acc[0][9], acc[0][10], acc[0][11]};
      const floatx4 hi8 = floatx4{acc[0][12], acc[0][13], acc[0][14], acc[0][15]};
      xp[(wv * 64 + lane) * 2] = hg == 0 ? hi4 : lo4;  // the other group's chunks
      xp[(wv * 64 + lane) * 2 + 1] = hg == 0 ? hi8 : lo8;
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const int po = ((wv ^ 4) * 64 + lane) * 2;  // the same wave of the other group
      const floatx4 p0 = xp[po], p1 = xp[po + 1];
      const floatx4 m0 = hg == 0 ? lo4 : hi4, m1 = hg == 0 ? lo8 : hi8;
      // sums in K-group order (group 0's partial first)
      const floatx4 s0 = hg == 0 ? m0 + p0 : p0 + m0, s1v = hg == 0 ? m1 + p1 : p1 + m1;
      uint32_t od[2][2];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        od[0][p] = pack_bf16x2(s0[2 * p] + bf16x2_lo(rr_b[0][p]), s0[2 * p + 1] + bf16x2_hi(rr_b[0][p]));
        od[1][p] = pack_bf16x2(s1v[2 * p] + bf16x2_lo(rr_b[1][p]), s1v[2 * p + 1] + bf16x2_hi(rr_b[1][p]));
      }
      const uint32_t w0 = g == 0 ? od[1][0] : od[0][0], w1 = g == 0 ? od[1][1] : od[0][1];
      const uint32_t x0 = static_cast<uint32_t>(__shfl_xor(static_cast<int>(w0), 32, 64));
      const uint32_t x1 = static_cast<uint32_t>(__shfl_xor(static_cast<int>(w1), 32, 64));
      const u32x4 yv = g == 0 ? u32x4{od[0][0], od[0][1], x0, x1} : u32x4{x0, x1, od[1][0], od[1][1]};
      const int row = mt * R + 32 * wm + l32, ocol = nt * OC + 32 * wn + 8 * (2 * hg + g);
      const bool ok = row < G.m && ocol < n_out;
      u32x4 o = {0, 0, 0, 0};
      if (ok) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = pack_bf16x2(bf16x2_lo(rr_res[e]) + bf16x2_lo(yv[e]), bf16x2_hi(rr_res[e]) + bf16x2_hi(yv[e]));
        *reinterpret_cast<u32x4*>(G.out + packed_act_offset(row, ocol, G.ldo)) = o;
      }
      if (G.stats_out) {
        float t1 = 0.f, t2 = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = bf16x2_lo(o[e]), hi = bf16x2_hi(o[e]);
          t1 += lo + hi;
          t2 += lo * lo + hi * hi;
        }
        f32x2_t* const xs = reinterpret_cast<f32x2_t*>(lnp + 8 * 64 * 8);  // [8 waves][64 lanes], past the partials
        xs[wv * 64 + lane] = f32x2_t{t1, t2};
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const f32x2_t a4 = xs[(wv ^ 1) * 64 + lane], a2 = xs[(wv ^ 4) * 64 + lane], a6 = xs[(wv ^ 5) * 64 + lane];
        float u1 = t1 + a4[0], u2 = t2 + a4[1];                 // chunks c, c ^ 4
        const float v1 = a2[0] + a6[0], v2 = a2[1] + a6[1];     // chunks c ^ 2, c ^ 6
        u1 = u1 + v1;
        u2 = u2 + v2;
        u1 += __shfl_xor(u1, 32, 64);
        u2 += __shfl_xor(u2, 32, 64);
        if (wn == 0 && hg == 0 && g == 0 && row < G.m)
          *(reinterpret_cast<f32x2_t*>(G.stats_out) + static_cast<int64_t>(nt * (OC / 64)) * G.m + row) = f32x2_t{u1, u2};
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // (the ring's re-loads write LDS)
      return;
    }
  }
  // RoPE tables of the register Q / K epilogue's chunks (streams with RoPE),
  // loaded after the K loop rather than held through it
  [[maybe_unused]] floatx4 rq_c[2][2], rq_s[2][2];
  if constexpr (kRegQkv) {
    if (reg_qkv && G.cos != nullptr) {
      const int64_t rr = min(mt * 32 * MB + 32 * wm + l32, G.m - 1);
#pragma unroll
      for (int bb = 0; bb < 2; ++bb)
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
          const int cd = 64 * wn + 32 * bb + 16 * pp + 8 * g;
          rq_c[bb][pp] = *reinterpret_cast<const floatx4*>(G.cos + rr * G.rope_ld + cd / 2);
          rq_s[bb][pp] = *reinterpret_cast<const floatx4*>(G.sin + rr * G.rope_ld + cd / 2);
        }
    }
  }

  if constexpr (kRegQkv || TR) {
    // The QKV epilogue's register paths, straight after the K loop (their
    // operands lie past the ring, published by the loop's barriers): see the
    // store phase below for the arithmetic they reproduce.
    constexpr int D = 128;
    const QkvOut& O = a.qkv;
    const int n0 = nt * OC;
    const int which = n0 / O.inner;  // uniform per tile
    const int h0 = (n0 - which * O.inner) / D;
    if constexpr (kRegQkv) {
      if (reg_qkv) {
        // Lane (l32, g) of wave (wm, wn) holds, for tile row 32 wm + l32, the
        // sums of head columns 64 wn + 32 bb + 8 q4 + 4 g + c (acc[bb], element
        // 4 q4 + c): halves of the head's 8-column chunks 8 wn + 4 bb + q4.  The
        // arithmetic is the store phase's below: x = bf16(fold(acc) + bias); the
        // chunks made whole by a swap of halves with lane l ^ 32 (lane half g
        // keeps chunks 8 wn + 4 bb + 2 pp + g); each chunk's sum of squares in
        // column order; then the same butterfly over the row's 16 chunks, level
        // by level: chunk ^ 8 is the other wave of the row (through LDS), ^ 4
        // and ^ 2 are in the lane, ^ 1 is lane l ^ 32.
        static_assert(D == 128 && OC == 128, "one head of 128 columns per tile");
        const int r = 32 * wm + l32, row = mt * R + r;
        float rs = 0.f, rm = 0.f;
        if constexpr (LN) {
          rs = lnp[2 * kThreads + 2 * r];
          rm = lnp[2 * kThreads + 2 * r + 1];
        }
        uint32_t xp[2][4][2];
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
              float x0 = acc[bb][4 * q4 + 2 * p], x1 = acc[bb][4 * q4 + 2 * p + 1];
              if constexpr (LN) {
                x0 = ln_fold(x0, rs, rm, rq_ws[bb][q4][2 * p]);
                x1 = ln_fold(x1, rs, rm, rq_ws[bb][q4][2 * p + 1]);
              }
              xp[bb][q4][p] = pack_bf16x2(x0 + bf16x2_lo(rq_b[bb][q4][p]), x1 + bf16x2_hi(rq_b[bb][q4][p]));
            }
        u32x4 xc[2][2];
        float ss[2][2];
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
          for (int pp = 0; pp < 2; ++pp) {
            const uint32_t w0 = g == 0 ? xp[bb][2 * pp + 1][0] : xp[bb][2 * pp][0];
            const uint32_t w1 = g == 0 ? xp[bb][2 * pp + 1][1] : xp[bb][2 * pp][1];
            const uint32_t o0 = static_cast<uint32_t>(__shfl_xor(static_cast<int>(w0), 32, 64));
            const uint32_t o1 = static_cast<uint32_t>(__shfl_xor(static_cast<int>(w1), 32, 64));
            xc[bb][pp] = g == 0 ? u32x4{xp[bb][2 * pp][0], xp[bb][2 * pp][1], o0, o1}
                                : u32x4{o0, o1, xp[bb][2 * pp + 1][0], xp[bb][2 * pp + 1][1]};
            float s2 = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float lo = bf16x2_lo(xc[bb][pp][e]), hi = bf16x2_hi(xc[bb][pp][e]);
              s2 += lo * lo;
              s2 += hi * hi;
            }
            ss[bb][pp] = s2;
          }
        floatx4* const exch = reinterpret_cast<floatx4*>(lnp + 2 * kThreads + 2 * R);  // [8 waves][64 lanes], past the ring
        exch[wv * 64 + lane] = floatx4{ss[0][0], ss[0][1], ss[1][0], ss[1][1]};
        __syncthreads();
        const floatx4 ps = exch[(wv ^ 1) * 64 + lane];  // the row's other wave: wn ^ 1
        const float t00 = ss[0][0] + ps[0], t01 = ss[0][1] + ps[1], t10 = ss[1][0] + ps[2], t11 = ss[1][1] + ps[3];
        const float u0 = t00 + t10, u1 = t01 + t11;
        const float v = u0 + u1;
        const float sum = v + __shfl_xor(v, 32, 64);
        uint16_t* kvh = O.kvp + h0 * O.kvp_sh;
        const int64_t key = static_cast<int64_t>(G.m_begin) + row;
        {
#pragma clang fp contract(off)
          const float rinv = 1.0f / __builtin_sqrtf(sum * (1.0f / D) + O.eps);
#pragma unroll
          for (int bb = 0; bb < 2; ++bb)
#pragma unroll
            for (int pp = 0; pp < 2; ++pp) {
              const int cd = 64 * wn + 32 * bb + 16 * pp + 8 * g;
              float y[8];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float xl = bf16x2_lo(xc[bb][pp][e]), xh = bf16x2_hi(xc[bb][pp][e]);
                const uint32_t yp = pack_bf16x2(bf16x2_lo(rq_w[bb][pp][e]) * (xl * rinv),
                                                bf16x2_hi(rq_w[bb][pp][e]) * (xh * rinv));
                y[2 * e] = bf16x2_lo(yp);
                y[2 * e + 1] = bf16x2_hi(yp);
              }
              u32x4 o;
              if (G.cos != nullptr) {
                const floatx4 c = rq_c[bb][pp], sn = rq_s[bb][pp];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                  const float re = y[2 * p], im = y[2 * p + 1];
                  o[p] = pack_bf16x2(re * c[p] - im * sn[p], re * sn[p] + im * c[p]);
                }
              } else {
#pragma unroll
                for (int p = 0; p < 4; ++p) o[p] = pack_bf16x2(y[2 * p], y[2 * p + 1]);
              }
              if (row < G.m) {
                if (which == 0)
                  *reinterpret_cast<u32x4*>(O.q + h0 * O.q_sh + key * O.q_sm + cd) = o;
                else
                  *reinterpret_cast<u32x4*>(kvh + packed_k_offset(key, cd, D)) = o;
              } else if (which == 1 && (row & ~31) < G.m) {
                *reinterpret_cast<u32x4*>(kvh + packed_k_offset(key, cd, D)) = u32x4{0, 0, 0, 0};
              }
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // (the ring's re-loads write LDS)
        return;
      }
    }
    if constexpr (TR) {
      // V tile with untransposed accumulators: lane (l32, g) of wave (wm, wn)
      // holds head column d = 32 db + l32 (db = 2 wn + bb) of keys
      // 32 wm + 8 q + 4 g + c (acc[bb], element 4 q + c) -- element e of packed
      // V chunk 2 db + s2 is acc[bb][8 s2 + e], the lane's own.  The store
      // phase's arithmetic below, without the fp32 tile.
      constexpr int NCH = D / 16;
      const int row0 = mt * R + 32 * wm;  // first stream row of the wave's 32-key tile
      if (row0 < G.m) {
        uint16_t* kvt = O.kvp + h0 * O.kvp_sh + ((G.m_begin + row0) >> 5) * (64 * D) + NCH * 512;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          float rs[8], rm[8];  // LayerNorm factors of the chunk's keys 32 wm + 16 s2 + 8 (e / 4) + 4 g + e % 4
          if constexpr (LN) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int rr = 32 * wm + 16 * s2 + 8 * (e >> 2) + 4 * g + (e & 3);
              rs[e] = lnp[2 * kThreads + 2 * rr];
              rm[e] = lnp[2 * kThreads + 2 * rr + 1];
            }
          }
#pragma unroll
          for (int bb = 0; bb < 2; ++bb) {
            u32x4 o;
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) {
              float lo = acc[bb][8 * s2 + 2 * e2], hi = acc[bb][8 * s2 + 2 * e2 + 1];
              if constexpr (LN) {
                lo = ln_fold(lo, rs[2 * e2], rm[2 * e2], rv_ws[bb]);
                hi = ln_fold(hi, rs[2 * e2 + 1], rm[2 * e2 + 1], rv_ws[bb]);
              }
              const int k0 = row0 + 16 * s2 + 8 * (e2 >> 1) + 4 * g + 2 * (e2 & 1);
              o[e2] = pack_bf16x2(k0 < G.m ? lo + rv_b[bb] : 0.f, k0 + 1 < G.m ? hi + rv_b[bb] : 0.f);
            }
            *reinterpret_cast<u32x4*>(kvt + ((2 * (2 * wn + bb) + s2) * 64 + lane) * 8) = o;
          }
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // (the ring's re-loads write LDS)
      return;
    }
  }
  float bg[8], bu[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bg[2 * i] = bf16x2_lo(bpk[i]);
    bg[2 * i + 1] = bf16x2_hi(bpk[i]);
    bu[2 * i] = bf16x2_lo(bpk[4 + i]);
    bu[2 * i + 1] = bf16x2_hi(bpk[4 + i]);
  }
  if constexpr (kStash) load_wsum_stash();
  else if constexpr (LN && kSwiglu) load_wsum();
  wait_barrier<0>();  // the ring's last reads and loads are done; LDS becomes the fp32 tiles
  float* tiles = reinterpret_cast<float*>(lds);
  if (!reg_epi && !reg_qkv && !TR) {
    float* t = tiles + grp * C::TILE;
#pragma unroll
    for (int bb = 0; bb < BNW; ++bb)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        *reinterpret_cast<floatx4*>(&t[(32 * wm + l32) * C::TP + 32 * (wn * BNW + bb) + 8 * q4 + 4 * g]) =
            floatx4{acc[bb][4 * q4], acc[bb][4 * q4 + 1], acc[bb][4 * q4 + 2], acc[bb][4 * q4 + 3]};
  }
  float* const lnst = tiles + ln_stats_off<C>();  // [kThreads / R][R][2]: thread t = q R + r's Σx, Σx²
  if constexpr (LN) {
    lnst[2 * threadIdx.x] = lp1;
    lnst[2 * threadIdx.x + 1] = lp2;
  }
  wait_barrier<0>();
  // LayerNorm fold factors of tile row r: rstd and rstd * mean, with mean and
  // the biased variance E[x^2] - mean^2 (clamped at 0) in fp32 and rstd from
  // v_rsq_f32 (the fold is not bit-compatible with the eager pre-norm anyway).
  // Thread r < R computes its row's pair once and leaves it at lnst[2 r], so
  // every later use is two LDS reads (the V tiles of the QKV epilogue use each
  // row's pair 64 times per workgroup).
  if constexpr (LN) {
    float rs = 0.f, rm = 0.f;
    const int r = static_cast<int>(threadIdx.x);
    if (r < R) {
      float s1 = lnst[2 * r], s2 = lnst[2 * r + 1];
#pragma unroll
      for (int p = 1; p < kThreads / R; ++p) {
        s1 += lnst[(p * R + r) * 2];
        s2 += lnst[(p * R + r) * 2 + 1];
      }
      const float inv_k = 1.0f / static_cast<float>(G.k);
      const float mean = s1 * inv_k;
      const float var = __builtin_fmaxf(__builtin_fmaf(-mean, mean, s2 * inv_k), 0.f);
      rs = __builtin_amdgcn_rsqf(var + a.ln_eps);
      rm = rs * mean;
    }
    __syncthreads();  // every partial sum is read before the pairs overwrite them
    if (r < R) {
      lnst[2 * r] = rs;
      lnst[2 * r + 1] = rm;
    }
    __syncthreads();
  }
  auto ln_row = [&](int r, float& rs, float& rm) {
    rs = lnst[2 * r];
    rm = lnst[2 * r + 1];
  };
  // 8 consecutive fp32 sums (K-groups in order) of tile row r from tile column tc
  auto sum8 = [&](int r, int tc, float (&v)[8]) {
    floatx4 lo = *reinterpret_cast<const floatx4*>(&tiles[r * C::TP + tc]);
    floatx4 hi = *reinterpret_cast<const floatx4*>(&tiles[r * C::TP + tc + 4]);
#pragma unroll
    for (int kg = 1; kg < C::KG; ++kg) {
      lo += *reinterpret_cast<const floatx4*>(&tiles[kg * C::TILE + r * C::TP + tc]);
      hi += *reinterpret_cast<const floatx4*>(&tiles[kg * C::TILE + r * C::TP + tc + 4]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = lo[i];
      v[4 + i] = hi[i];
    }
  };
  if constexpr (qkv_epi(EPI)) {
    // The tile's 128 columns are one head (head_dim 128) or two (64) of Q, K or
    // V (columns n0.. of [Q | K | V]).  Q / K rows: x = bf16(acc + bias), then
    // the per-head RMSNorm y = bf16(w * (x * rsqrt(mean(x^2) + eps))) and, on
    // streams with tables, the interleaved RoPE rounded once:
    // msat_qkv_norm_rope_kernel's arithmetic with its partition of a head's row
    // (D / 8 lanes of 8 columns, butterfly sum over them), so the result is the
    // same bit for bit as this GEMM's bias epilogue followed by that kernel.  Q
    // goes to (H, M, D); K rows to their lanes of the packed tiles.  V is read
    // down the fp32 tile's columns (8 keys of one column per 16-byte chunk)
    // straight into the packed V chunks.  Keys of the stream's last 32-key tile
    // past its rows are written as zeros (padding keys of the attention).
    static_assert(OC == 128 && R * CPR == PER * kThreads, "QKV tiles are 128 columns of whole heads");
    constexpr int D = EPI == kEpiQkv ? 128 : 64;
    constexpr int HPT = OC / D;  // heads per tile
    const QkvOut& O = a.qkv;
    const int n0 = nt * OC;
    const int which = n0 / O.inner;  // uniform per tile
    const int h0 = (n0 - which * O.inner) / D;
    if (which == 2) {
      constexpr int NCH = D / 16;  // 1 KB chunks per K or V part of a head's 32-key tile
      static_assert(kThreads % (HPT * NCH * 64) == 0, "a thread's V column (hh, idx) is the same on every pass");
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int s = static_cast<int>(threadIdx.x) + kThreads * i;
        const int kt = s / (HPT * NCH * 64), hh = s / (NCH * 64) % HPT, idx = s % (NCH * 64);
        const int cx = idx >> 6, l = idx & 63;
        // chunk cx = 2 db + s2, lane l, element e: V[16 s2 + 8 (e / 4) + 4 (l / 32) + e % 4][32 db + l % 32]
        const int d = hh * D + 32 * (cx >> 1) + (l & 31);  // tile column
        const int rb = 32 * kt + 16 * (cx & 1) + 4 * (l >> 5);
        const int row0 = mt * R + 32 * kt;  // first stream row of this 32-key tile
        if (row0 >= G.m) continue;
        const float bd = v_bias;  // loaded in the prologue for this column d
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = rb + 8 * (e >> 1) + 2 * (e & 1);
          float lo = tiles[r * C::TP + d], hi = tiles[(r + 1) * C::TP + d];
#pragma unroll
          for (int kg = 1; kg < C::KG; ++kg) {
            lo += tiles[kg * C::TILE + r * C::TP + d];
            hi += tiles[kg * C::TILE + (r + 1) * C::TP + d];
          }
          if constexpr (LN) {
            const float sd = v_wsum;
            float rs, rm;
            ln_row(r, rs, rm);
            lo = ln_fold(lo, rs, rm, sd);
            ln_row(r + 1, rs, rm);
            hi = ln_fold(hi, rs, rm, sd);
          }
          o[e] = pack_bf16x2(mt * R + r < G.m ? lo + bd : 0.f, mt * R + r + 1 < G.m ? hi + bd : 0.f);
        }
        uint16_t* kvh = O.kvp + (h0 + hh) * O.kvp_sh;
        *reinterpret_cast<u32x4*>(kvh + ((G.m_begin + row0) >> 5) * (64 * D) + NCH * 512 + idx * 8) = o;
      }
      return;
    }
    const int c8 = cc;               // columns n0 + c8 = col
    const int cd = c8 % D;           // their columns within head h0 + c8 / D
    uint16_t* kvh = O.kvp + (h0 + c8 / D) * O.kvp_sh;
    const int h = h0 + c8 / D;
    const float* bq = bg;            // their biases
    const u32x4 wraw = qk_w;         // the Q or K norm weights of those columns
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int r = (static_cast<int>(threadIdx.x) + kThreads * i) / CPR, row = mt * R + r;
      float x[8];
      sum8(r, c8, x);
      if constexpr (LN) {
        float rs, rm;
        ln_row(r, rs, rm);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = ln_fold(x[e], rs, rm, wg[e]);  // (columns n0 + c8 = col)
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t xp = pack_bf16x2(x[2 * e] + bq[2 * e], x[2 * e + 1] + bq[2 * e + 1]);
        x[2 * e] = bf16x2_lo(xp);
        x[2 * e + 1] = bf16x2_hi(xp);
      }
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
#pragma unroll
      for (int mm = D / 16; mm >= 1; mm >>= 1) ss += __shfl_xor(ss, mm, 64);  // the D / 8 lanes of the head's row
      u32x4 o;
      {
#pragma clang fp contract(off)
        const float rinv = 1.0f / __builtin_sqrtf(ss * (1.0f / D) + O.eps);
        float y[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t yp = pack_bf16x2(bf16x2_lo(wraw[e]) * (x[2 * e] * rinv), bf16x2_hi(wraw[e]) * (x[2 * e + 1] * rinv));
          y[2 * e] = bf16x2_lo(yp);
          y[2 * e + 1] = bf16x2_hi(yp);
        }
        if (G.cos != nullptr) {
          const int64_t rr = min(row, G.m - 1);
          const floatx4 c = *reinterpret_cast<const floatx4*>(G.cos + rr * G.rope_ld + cd / 2);
          const floatx4 sn = *reinterpret_cast<const floatx4*>(G.sin + rr * G.rope_ld + cd / 2);
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const float re = y[2 * p], im = y[2 * p + 1];
            o[p] = pack_bf16x2(re * c[p] - im * sn[p], re * sn[p] + im * c[p]);
          }
        } else {
#pragma unroll
          for (int p = 0; p < 4; ++p) o[p] = pack_bf16x2(y[2 * p], y[2 * p + 1]);
        }
      }
      const int64_t key = static_cast<int64_t>(G.m_begin) + row;
      if (row < G.m) {
        if (which == 0)
          *reinterpret_cast<u32x4*>(O.q + h * O.q_sh + key * O.q_sm + cd) = o;
        else
          *reinterpret_cast<u32x4*>(kvh + packed_k_offset(key, cd, D)) = o;
      } else if (which == 1 && (row & ~31) < G.m) {
        *reinterpret_cast<u32x4*>(kvh + packed_k_offset(key, cd, D)) = u32x4{0, 0, 0, 0};
      }
    }
    return;
  }
  // fp32 sums of this thread's chunks: 8 columns, or 8 gate + 8 up columns
  constexpr int V = kSwiglu ? 16 : 8;
  const int tc = kSwiglu ? 64 * (cc / 32) + cc % 32 : cc;
  float y[PER][V];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int r = (static_cast<int>(threadIdx.x) + kThreads * i) / CPR;
    float lo[8];
    sum8(r < R ? r : 0, tc, lo);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[i][e] = lo[e];
    if constexpr (kSwiglu) {
      float hi[8];
      sum8(r < R ? r : 0, tc + 32, hi);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[i][8 + e] = hi[e];
    }
    if constexpr (LN) {  // (the host allows the fold only without split-K)
      float rs, rm;
      ln_row(r < R ? r : 0, rs, rm);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        y[i][e] = ln_fold(y[i][e], rs, rm, wg[e]);
        if constexpr (kSwiglu) y[i][8 + e] = ln_fold(y[i][8 + e], rs, rm, wu[e]);
      }
    }
  }
  // the residual epilogue's output chunk i: bf16(residual + bf16(y + bias))
  [[maybe_unused]] auto residual_out = [&](int i) {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = pack_bf16x2(y[i][2 * e] + bg[2 * e], y[i][2 * e + 1] + bg[2 * e + 1]);
      o[e] = pack_bf16x2(bf16x2_lo(pres[i][e]) + bf16x2_lo(o[e]), bf16x2_hi(pres[i][e]) + bf16x2_hi(o[e]));
    }
    return o;
  };
  auto store_out = [&](int row, const u32x4& o) {
    if constexpr (packed_out(EPI))  // ldo = width of the packed matrix the output columns belong to
      *reinterpret_cast<u32x4*>(G.out + packed_act_offset(row, col, G.ldo)) = o;
    else
      *reinterpret_cast<u32x4*>(G.out + static_cast<int64_t>(row) * G.ldo + col) = o;
  };
  if (G.splits > 1) {
    // Split-K.  Each split stores its fp32 partial with device-scope stores
    // (SC1: written through to the device coherence point, not held in this
    // XCD's L2), waits until they are complete, then counts in with a
    // device-scope atomic; the last to arrive reads the other partials with
    // device-scope loads (SC1: not served from a possibly stale L1 / L2), sums
    // all of them in split order (the same order whichever split arrives last),
    // applies the epilogue and re-arms the counter.  This holds wherever the
    // splits run; the launch normally gives every XCD whole tiles, so the
    // splits of a tile share one L2 (RLDX_GEMM_SPLITS_ACROSS_XCDS places them
    // on different XCDs, for tests).
    const int part_bytes = G.items * PER * kThreads * V * 4;  // < 2^31 (host check)
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(G.part, 0, part_bytes, kBufWord3);
    auto slot = [&](int sp, int i) { return (((tile * G.splits + sp) * PER + i) * kThreads + threadIdx.x) * V * 4; };
#pragma unroll
    for (int i = 0; i < PER; ++i)
#pragma unroll
      for (int e = 0; e < V; e += 4)
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4, floatx4{y[i][e], y[i][e + 1], y[i][e + 2], y[i][e + 3]}), prs,
            slot(split, i) + 4 * e, 0, kCpolDevice);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    int* last = reinterpret_cast<int*>(wsl + (kWsumStash + kBiasStash) / 4);  // the LDS tail: past the stashes and every epilogue tile
    if (threadIdx.x == 0)
      *last = __hip_atomic_fetch_add(G.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              static_cast<unsigned>(G.splits - 1);
    __syncthreads();
    if (!*last) return;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      float sum[V];
#pragma unroll
      for (int e = 0; e < V; ++e) sum[e] = 0.f;
      for (int sp = 0; sp < G.splits; ++sp) {
#pragma unroll
        for (int e = 0; e < V; e += 4) {
          const floatx4 v =
              sp == split ? floatx4{y[i][e], y[i][e + 1], y[i][e + 2], y[i][e + 3]}
                          : __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(prs, slot(sp, i) + 4 * e,
                                                                                              0, kCpolDevice));
#pragma unroll
          for (int f = 0; f < 4; ++f) sum[e + f] += v[f];
        }
      }
#pragma unroll
      for (int e = 0; e < V; ++e) y[i][e] = sum[e];
    }
    if (threadIdx.x == 0) __hip_atomic_store(G.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int t = static_cast<int>(threadIdx.x) + kThreads * i;
    const int r = t / CPR, row = mt * R + r;
    const bool ok = t < R * CPR && row < G.m && col_ok;
    if constexpr (residual_epi(EPI)) {
      // row statistics of the stored values for a LayerNorm-folding consumer:
      // Σx, Σx² over this tile's columns of the row (its CPR threads are
      // consecutive lanes), in slot nt OC / 64 of [n / 64][m][2] (a 128-column
      // tile writes its sums in the first of its two slots and zeros in the other)
      if (G.stats_out) {
        u32x4 o = ok ? residual_out(i) : u32x4{0, 0, 0, 0};
        if (ok) store_out(row, o);
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = bf16x2_lo(o[e]), hi = bf16x2_hi(o[e]);
          s1 += lo + hi;
          s2 += lo * lo + hi * hi;
        }
#pragma unroll
        for (int mm = CPR / 2; mm >= 1; mm >>= 1) {
          s1 += __shfl_xor(s1, mm, 64);
          s2 += __shfl_xor(s2, mm, 64);
        }
        if (ok && t % CPR == 0) {
          f32x2_t* st = reinterpret_cast<f32x2_t*>(G.stats_out) + static_cast<int64_t>(nt * (OC / 64)) * G.m + row;
          *st = f32x2_t{s1, s2};
          if constexpr (OC == 128)
            if (2 * nt + 1 < G.n / 64) st[G.m] = f32x2_t{0.f, 0.f};
        }
        continue;
      }
    }
    if (!ok) continue;
    u32x4 o;
    if constexpr (kSwiglu) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t gp = pack_bf16x2(y[i][2 * e] + bg[2 * e], y[i][2 * e + 1] + bg[2 * e + 1]);
        const uint32_t up = pack_bf16x2(y[i][8 + 2 * e] + bu[2 * e], y[i][8 + 2 * e + 1] + bu[2 * e + 1]);
        o[e] = swiglu_bf16x2(bf16x2_lo(gp), bf16x2_hi(gp), bf16x2_lo(up), bf16x2_hi(up));
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(y[i][2 * e] + bg[2 * e], y[i][2 * e + 1] + bg[2 * e + 1]);
      if constexpr (residual_epi(EPI)) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = pack_bf16x2(bf16x2_lo(pres[i][e]) + bf16x2_lo(o[e]), bf16x2_hi(pres[i][e]) + bf16x2_hi(o[e]));
      }
    }
    store_out(row, o);
  }
}

// WIDE: the plan uses 128 x 128, 64 x 128 and 32 x 128 tiles (always with the
// QKV epilogue; on request for the others).
// Second launch bound: minimum waves per SIMD (2 per workgroup of 8 waves):
// the two-workgroups-per-CU kernels keep to 128 VGPRs.
template <int EPI, bool DEEP, bool WIDE, bool LN>
__global__ __launch_bounds__(kThreads, DEEP ? 2 : 4) void gemm_kernel(GemmArgs a) {
  constexpr int kLds = WIDE ? (DEEP ? kLdsQkvDeep : kLdsQkv) : (DEEP ? kLdsDeep : kLdsBytes);
  __shared__ __attribute__((aligned(16))) u32x4 lds[kLds / 16];
  float* const wsl = reinterpret_cast<float*>(lds) + (kLds - kLdsTail) / 4;
  const int b = static_cast<int>(blockIdx.x);
  int gi = 0;
  if (a.num_groups > 1 && b >= a.g[1].wg_begin) gi = 1;
  if (a.num_groups > 2 && b >= a.g[2].wg_begin) gi = 2;
  const Group& G = a.g[gi];
  const int r = b - G.wg_begin;
  // XCD r % 8 takes a contiguous run of tiles; spread: consecutive items (the
  // splits of a tile) on consecutive workgroups, i.e. on different XCDs
  const int item = a.spread ? r : (r % kXcds) * G.per_xcd + r / kXcds;
  if (item >= G.items) return;
  if constexpr (WIDE && DEEP) {  // 128-column tiles (whole heads for the QKV epilogue)
    if (G.cfg == kTile128) {
      if constexpr (EPI == kEpiQkv) {
        // V tiles (the last third of [Q | K | V]) with untransposed accumulators
        const int nt = item / G.splits / G.m_tiles;
        if (nt * 128 / a.qkv.inner == 2)
          gemm_tile<Cfg128D, EPI, WIDE, LN, DEEP, true>(a, G, item, lds, wsl);
        else
          gemm_tile<Cfg128D, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
      } else {
        gemm_tile<Cfg128D, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
      }
    } else if (G.cfg == kTile64x128)
      gemm_tile<Cfg64x128D, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
    else
      gemm_tile<Cfg32x128D, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
  } else if constexpr (WIDE) {
    if (G.cfg == kTile128)
      gemm_tile<Cfg128, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
    else if (G.cfg == kTile64x128)
      gemm_tile<Cfg64x128, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
    else
      gemm_tile<Cfg32x128, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
  } else if constexpr (DEEP) {
    if (G.cfg == kTile128)
      gemm_tile<Cfg128D, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
    else if (G.cfg == kTile64)
      gemm_tile<Cfg64D, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
    else
      gemm_tile<Cfg32D, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
  } else {
    if (G.cfg == kTile128)
      gemm_tile<Cfg128, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
    else if (G.cfg == kTile64)
      gemm_tile<Cfg64, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
    else
      gemm_tile<Cfg32, EPI, WIDE, LN, DEEP>(a, G, item, lds, wsl);
  }
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <class C>
void tiles_of(int64_t m, int64_t n, int& m_tiles, int& n_tiles) {
  m_tiles = static_cast<int>((m + 32 * C::MB - 1) / (32 * C::MB));
  n_tiles = static_cast<int>((n / 32 + C::NB - 1) / C::NB);
}

// L2 -> CU bytes a workgroup of configuration cfg moves for one tile.
int64_t tile_bytes(int cfg, int64_t k) {
  const int ch = cfg == kTile128      ? Cfg128::CH
                 : cfg == kTile64     ? Cfg64::CH
                 : cfg == kTile64x128 ? Cfg64x128::CH
                 : cfg == kTile32x128 ? Cfg32x128::CH
                                      : Cfg32::CH;
  return ch * k * 64;  // ch chunks of 1 KB per 16 columns of K
}

template <class C>
void cfg_dims(int epi, int& kg, int& per, int& v) {
  const bool swiglu = epi == kEpiSwiglu || epi == kEpiSwigluPacked;
  const int cpr = (swiglu ? 16 * C::NB : 32 * C::NB) / 8;
  kg = C::KG;
  per = (32 * C::MB * cpr + kThreads - 1) / kThreads;
  v = swiglu ? 16 : 8;
}

constexpr int64_t kWsAlign = 256;
int64_t align_up(int64_t x) { return (x + kWsAlign - 1) / kWsAlign * kWsAlign; }
// Every plan keeps its tile counters in the first kCounterBytes of the
// workspace and its partials after them: calls with different shapes can share
// one workspace without one call's partials landing on another call's counters
// (which must read zero when a launch starts).
constexpr int64_t kCounterBytes = 65536;

// Validates the call and fills the launch arguments.  split_k > 1 splits the K
// range of every group over that many workgroups (the largest power of two
// <= split_k that divides its stages);
// *ws_bytes receives the workspace the plan needs (counters, then fp32 partials).
// The QKV epilogue (kEpiQkv) takes each group's norm weights and RoPE tables
// from norms[i] (the caller has checked them) and never splits.
// w_row_sums (LayerNorm fold): one fp32 row-sum vector per group, all present;
// only for the bias, packed-SwiGLU and QKV epilogues, without split-K.
hipError_t plan(const rldx_gemm_group_t* groups, int32_t num_groups, int64_t n, int64_t k, int32_t epilogue,
                int split_k, GemmArgs& args, int64_t* ws_bytes, int64_t* cnt_off, int64_t* part_off,
                const rldx_msat_stream_t* norms = nullptr, bool wide_tiles = false,
                const float* const* w_row_sums = nullptr, const float* const* ln_stats = nullptr,
                float* const* stats_out = nullptr, const int64_t* group_n = nullptr,
                const int64_t* group_k = nullptr, const int32_t* group_splits = nullptr) {
  if (!groups || num_groups < 1 || num_groups > 3) return hipErrorInvalidValue;
  // per-group shapes (rldx_grouped_gemm_mixed_bf16): every group its own n, k and split
  if ((group_n == nullptr) != (group_k == nullptr)) return hipErrorInvalidValue;
  if (group_n) {
    n = group_n[0];
    k = group_k[0];
    for (int i = 0; i < num_groups; ++i) {
      if (group_n[i] <= 0 || group_k[i] <= 0) return hipErrorInvalidValue;
      if (group_splits && (group_splits[i] < 1 || group_splits[i] > 64)) return hipErrorInvalidValue;
    }
  }
  auto gn = [&](int i) { return group_n ? group_n[i] : n; };
  auto gk = [&](int i) { return group_k ? group_k[i] : k; };
  if (!(epilogue >= kEpiBias && epilogue <= kEpiResidualPacked) && !qkv_epi(epilogue)) return hipErrorInvalidValue;
  const bool qkv = qkv_epi(epilogue);
  // LayerNorm fold: W row sums and A-row statistics for every group; k <= 2048
  // (a thread of a 128-row tile sums at most kLnSlotsMax slots)
  if ((w_row_sums == nullptr) != (ln_stats == nullptr)) return hipErrorInvalidValue;
  if (w_row_sums) {
    if (split_k > 1 || !(epilogue == kEpiBias || epilogue == kEpiSwigluPacked || qkv)) return hipErrorInvalidValue;
    for (int i = 0; i < num_groups; ++i)
      if (gk(i) > 64 * 4 * kLnSlotsMax) return hipErrorInvalidValue;
    for (int i = 0; i < num_groups; ++i)  // (an empty group reads nothing)
      if (groups[i].m != 0 && (!w_row_sums[i] || reinterpret_cast<uintptr_t>(w_row_sums[i]) % 4 || !ln_stats[i] ||
                               reinterpret_cast<uintptr_t>(ln_stats[i]) % 8))
        return hipErrorInvalidValue;
  }
  if (stats_out) {
    if (!residual_epi(epilogue)) return hipErrorInvalidValue;
    for (int i = 0; i < num_groups; ++i)
      if (groups[i].m != 0 && (!stats_out[i] || reinterpret_cast<uintptr_t>(stats_out[i]) % 8))
        return hipErrorInvalidValue;
  }
  const bool wide = qkv || wide_tiles;
  if (qkv && (norms == nullptr || split_k > 1 || group_splits)) return hipErrorInvalidValue;
  if (qkv && group_n)  // per-group K only: every group writes the same [Q | K | V] columns
    for (int i = 0; i < num_groups; ++i)
      if (group_n[i] != group_n[0]) return hipErrorInvalidValue;
  const bool swiglu = epilogue == kEpiSwiglu || epilogue == kEpiSwigluPacked;
  // k: whole stages of every K-group split (4 K-groups x 2 k-steps); n: whole 64-column blocks
  for (int i = 0; i < num_groups; ++i)
    if (gn(i) <= 0 || gk(i) <= 0 || gn(i) % 64 != 0 || gk(i) % 128 != 0 || gn(i) > (1 << 30) || gk(i) > (1 << 30))
      return hipErrorInvalidValue;
  args = GemmArgs{};
  args.n = static_cast<int>(n);
  args.k = static_cast<int>(k);
  int cnt = 0;
  int64_t m_begin = 0;  // joint-sequence row of the group (QKV epilogue)
  for (int i = 0; i < num_groups; ++i) {
    const int64_t n = gn(i), k = gk(i);  // this group's shape
    const int64_t n_out = swiglu ? n / 2 : n;
    const int ksteps = static_cast<int>(k / 16);
    const rldx_gemm_group_t& s = groups[i];
    if (s.m < 0 || s.m > (1 << 24)) return hipErrorInvalidValue;
    if (s.m == 0) continue;
    if (!s.a_packed || !s.w_packed || (!qkv && !s.out) || !a16(s.a_packed) || !a16(s.w_packed))
      return hipErrorInvalidValue;
    // packed operands are addressed with 32-bit byte offsets
    if ((s.m + 31) / 32 * 32 * k * 2 > (int64_t{1} << 31) - 1 || n * k * 2 > (int64_t{1} << 31) - 1)
      return hipErrorInvalidValue;
    // the epilogue stores (and reads the residual) in 16-byte pieces
    if ((!qkv && !a16(s.out)) || (s.bias && reinterpret_cast<uintptr_t>(s.bias) % 2)) return hipErrorInvalidValue;
    if (!qkv && !packed_out(epilogue) && (s.ldo < n_out || s.ldo % 8)) return hipErrorInvalidValue;
    // packed output: ldo 0 (= n_out) or the width of a wider packed matrix whose
    // 16-column chunk at `out` starts the output columns
    if (packed_out(epilogue) && (s.ldo < 0 || s.ldo % 16 || (s.ldo > 0 && s.ldo < n_out) || s.ldo > (1 << 30)))
      return hipErrorInvalidValue;
    if (epilogue == kEpiResidual && (!s.residual || !a16(s.residual) || s.ldr < n_out || s.ldr % 8))
      return hipErrorInvalidValue;
    // packed residual: ldr 0 (= n_out) or the width of the packed matrix, as ldo
    if (epilogue == kEpiResidualPacked &&
        (!s.residual || !a16(s.residual) || s.ldr < 0 || s.ldr % 16 || (s.ldr > 0 && s.ldr < n_out) ||
         s.ldr > (1 << 30)))
      return hipErrorInvalidValue;
    // Tile shape: 128 x 128 where the stream has rows and tiles enough to
    // occupy the chip (half the L2 traffic per flop of 64 x 64), else 64 x 64,
    // or 32 x 64 for streams of at most 32 rows.
    // Wide plans (the QKV epilogue needs whole 128-column heads): 64 x 128 and
    // 32 x 128 in place of 64 x 64 and 32 x 64, with the same K-groups (so the
    // same sums, bit for bit).
    int mt, nt, cfg, kg;
    tiles_of<Cfg128>(s.m, n, mt, nt);
    if (s.m >= 256 && static_cast<int64_t>(mt) * nt >= 128) {
      cfg = kTile128;
      kg = Cfg128::KG;
    } else if (wide && s.m > 32) {
      cfg = kTile64x128;
      kg = Cfg64x128::KG;
      tiles_of<Cfg64x128>(s.m, n, mt, nt);
    } else if (wide) {
      cfg = kTile32x128;
      kg = Cfg32x128::KG;
      tiles_of<Cfg32x128>(s.m, n, mt, nt);
    } else if (s.m > 32) {
      cfg = kTile64;
      kg = Cfg64::KG;
      tiles_of<Cfg64>(s.m, n, mt, nt);
    } else {
      cfg = kTile32;
      kg = Cfg32::KG;
      tiles_of<Cfg32>(s.m, n, mt, nt);
    }
    const int64_t tiles = static_cast<int64_t>(mt) * nt;
    if (tiles > (int64_t{1} << 24)) return hipErrorInvalidValue;
    const int lstages = ksteps / (2 * kg);
    const int want = group_splits ? group_splits[i] : split_k;
    int sp = 1;
    while (sp * 2 <= want && lstages % (sp * 2) == 0) sp *= 2;
    Group& G = args.g[cnt++];
    G = Group{static_cast<const uint16_t*>(s.a_packed), static_cast<const uint16_t*>(s.w_packed),
              static_cast<const uint16_t*>(s.bias), static_cast<uint16_t*>(s.out),
              static_cast<const uint16_t*>(s.residual), packed_out(epilogue) && s.ldo == 0 ? n_out : s.ldo,
              epilogue == kEpiResidualPacked && s.ldr == 0 ? n_out : s.ldr,
              static_cast<int>(s.m), cfg, mt,
              static_cast<int>(tiles * sp), static_cast<int>(n), static_cast<int>(k), 0, 0, sp, lstages / sp,
              nullptr, nullptr};
    G.wsum = w_row_sums ? w_row_sums[i] : nullptr;
    G.lnstats = ln_stats ? ln_stats[i] : nullptr;
    G.stats_out = stats_out ? stats_out[i] : nullptr;
    if (qkv) {
      G.m_begin = static_cast<int>(m_begin);
      G.qn_w = static_cast<const uint16_t*>(norms[i].q_norm_w);
      G.kn_w = static_cast<const uint16_t*>(norms[i].k_norm_w);
      G.cos = norms[i].rope_cos;
      G.sin = norms[i].rope_sin;
      G.rope_ld = static_cast<int>(norms[i].rope_row_stride);
    }
    m_begin += qkv ? (s.m + 31) / 32 * 32 : s.m;  // QKV: each stream starts a 32-key tile
  }
  args.num_groups = cnt;
  if (cnt == 0) return hipSuccess;
  // heaviest workgroups first (they take the first slot of every CU; the short
  // streams' workgroups fill the second)
  for (int i = 1; i < cnt; ++i)
    for (int j = i; j > 0 && tile_bytes(args.g[j].cfg, args.g[j].k) / args.g[j].splits >
                                 tile_bytes(args.g[j - 1].cfg, args.g[j - 1].k) / args.g[j - 1].splits;
         --j) {
      const Group t = args.g[j];
      args.g[j] = args.g[j - 1];
      args.g[j - 1] = t;
    }
  int64_t wgs = 0, ws = kCounterBytes, counters = 0;
  for (int i = 0; i < cnt; ++i) {
    Group& G = args.g[i];
    G.wg_begin = static_cast<int>(wgs);
    // whole tiles per XCD: the splits of a tile meet in one L2
    G.per_xcd = (G.items / G.splits + kXcds - 1) / kXcds * G.splits;
    wgs += static_cast<int64_t>(G.per_xcd) * kXcds;
    if (wgs > (int64_t{1} << 31) - 1) return hipErrorInvalidValue;
    cnt_off[i] = part_off[i] = -1;
    if (G.splits > 1) {
      int kgd, per, v;
      if (G.cfg == kTile64x128)
        cfg_dims<Cfg64x128>(epilogue, kgd, per, v);
      else if (G.cfg == kTile32x128)
        cfg_dims<Cfg32x128>(epilogue, kgd, per, v);
      else if (G.cfg == kTile128)
        cfg_dims<Cfg128>(epilogue, kgd, per, v);
      else if (G.cfg == kTile64)
        cfg_dims<Cfg64>(epilogue, kgd, per, v);
      else
        cfg_dims<Cfg32>(epilogue, kgd, per, v);
      cnt_off[i] = counters * 4;
      counters += G.items / G.splits;
      part_off[i] = ws;
      const int64_t pb = static_cast<int64_t>(G.items) * per * kThreads * v * 4;
      if (pb > (int64_t{1} << 31) - 1) return hipErrorInvalidValue;  // 32-bit buffer offsets
      ws = align_up(ws + pb);
    }
  }
  if (counters * 4 > kCounterBytes) return hipErrorInvalidValue;
  *ws_bytes = counters ? ws : 0;
  return hipSuccess;
}

template <int EPI, bool LN>
void launch_epi(const GemmArgs& args, dim3 grid, hipStream_t stream, bool deep, bool wide) {
  const dim3 block(kThreads);
  if (deep && wide)
    hipLaunchKernelGGL((gemm_kernel<EPI, true, true, LN>), grid, block, 0, stream, args);
  else if (deep)
    hipLaunchKernelGGL((gemm_kernel<EPI, true, false, LN>), grid, block, 0, stream, args);
  else if (wide)
    hipLaunchKernelGGL((gemm_kernel<EPI, false, true, LN>), grid, block, 0, stream, args);
  else
    hipLaunchKernelGGL((gemm_kernel<EPI, false, false, LN>), grid, block, 0, stream, args);
}

template <int EPI, bool LN>
void launch_qkv(const GemmArgs& args, dim3 grid, hipStream_t stream, bool deep) {
  if (deep)
    hipLaunchKernelGGL((gemm_kernel<EPI, true, true, LN>), grid, dim3(kThreads), 0, stream, args);
  else
    hipLaunchKernelGGL((gemm_kernel<EPI, false, true, LN>), grid, dim3(kThreads), 0, stream, args);
}

// ln: the groups carry W row sums (LayerNorm fold; plan() admits it for the
// bias, packed-SwiGLU and QKV epilogues only)
hipError_t launch(const GemmArgs& args, int epilogue, hipStream_t stream, bool wide = false, bool ln = false) {
  if (args.num_groups == 0) return hipSuccess;
  const Group& last = args.g[args.num_groups - 1];
  const int wgs = last.wg_begin + last.per_xcd * kXcds;
  const dim3 grid(static_cast<unsigned>(wgs));
  // at most one workgroup per CU (256 CUs): the deep-ring kernel
  const bool deep = wgs <= 256;
  if (ln) {
    if (epilogue == kEpiQkv)
      launch_qkv<kEpiQkv, true>(args, grid, stream, deep);
    else if (epilogue == kEpiQkv64)
      launch_qkv<kEpiQkv64, true>(args, grid, stream, deep);
    else if (epilogue == kEpiBias)
      launch_epi<kEpiBias, true>(args, grid, stream, deep, wide);
    else if (epilogue == kEpiSwigluPacked)
      launch_epi<kEpiSwigluPacked, true>(args, grid, stream, deep, wide);
    else
      return hipErrorInvalidValue;
    return hipGetLastError();
  }
  switch (epilogue) {
    case kEpiQkv: launch_qkv<kEpiQkv, false>(args, grid, stream, deep); break;
    case kEpiQkv64: launch_qkv<kEpiQkv64, false>(args, grid, stream, deep); break;
    case kEpiBias: launch_epi<kEpiBias, false>(args, grid, stream, deep, wide); break;
    case kEpiResidual: launch_epi<kEpiResidual, false>(args, grid, stream, deep, wide); break;
    case kEpiSwiglu: launch_epi<kEpiSwiglu, false>(args, grid, stream, deep, wide); break;
    case kEpiSwigluPacked: launch_epi<kEpiSwigluPacked, false>(args, grid, stream, deep, wide); break;
    case kEpiBiasPacked: launch_epi<kEpiBiasPacked, false>(args, grid, stream, deep, wide); break;
    case kEpiResidualPacked: launch_epi<kEpiResidualPacked, false>(args, grid, stream, deep, wide); break;
    default: return hipErrorInvalidValue;
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
// stats (optional, not with normalize): the row's Σx, Σx² for a LayerNorm-
// folding GEMM, in slot 0 of [k / 64][m][2], zeros in the other slots.
// Up to kRowsMax matrices per launch (the streams of a block): workgroups
// [begin[i], begin[i + 1]) take matrix i, 4 rows each.
constexpr int kRowsMax = 4;
struct RowsArgs {
  const uint16_t* x[kRowsMax];
  uint16_t* out[kRowsMax];
  float* stats[kRowsMax];
  int64_t ldx[kRowsMax];
  int m[kRowsMax], k[kRowsMax];
  int begin[kRowsMax + 1];
  int count, normalize;
  float eps;
};

template <int CPL>
__global__ __launch_bounds__(256) void rows_pack_kernel(RowsArgs a) {
  int mi = 0;
#pragma unroll
  for (int i = 1; i < kRowsMax; ++i)
    if (i < a.count && static_cast<int>(blockIdx.x) >= a.begin[i]) mi = i;
  const int m = a.m[mi], k = a.k[mi];
  float* __restrict__ stats = a.stats[mi];
  uint16_t* __restrict__ out = a.out[mi];
  const int lane = threadIdx.x & 63;
  const int row = (static_cast<int>(blockIdx.x) - a.begin[mi]) * 4 + (threadIdx.x >> 6);
  if (row >= m) return;
  const uint16_t* xr = a.x[mi] + static_cast<int64_t>(row) * a.ldx[mi];
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
  if (a.normalize) {
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
    const float rstd = 1.0f / __builtin_sqrtf(sq / static_cast<float>(k) + a.eps);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
#pragma unroll
      for (int i = 0; i < 8; i += 2)  // one RNE rounding per element (v_cvt_pk_bf16_f32)
        raw[c][i >> 1] = pack_bf16x2((v[c][i] - mean) * rstd, (v[c][i + 1] - mean) * rstd);
    }
  }
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = 8 * (lane + 64 * c);
    if (col < k) *reinterpret_cast<u32x4*>(out + packed_act_offset(row, col, k)) = raw[c];
  }
  if (stats != nullptr) {  // (wave-uniform)
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c)
      if (8 * (lane + 64 * c) < k)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          s1 += v[c][i];
          s2 += v[c][i] * v[c][i];
        }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      s1 += __shfl_xor(s1, o, 64);
      s2 += __shfl_xor(s2, o, 64);
    }
    const int slots = k / 64;
    f32x2_t* st = reinterpret_cast<f32x2_t*>(stats) + row;
    for (int j = lane; j < slots; j += 64) st[static_cast<int64_t>(j) * m] = j == 0 ? f32x2_t{s1, s2} : f32x2_t{0.f, 0.f};
  }
}

// Checks and launches up to kRowsMax matrices in one launch; the register
// width (CPL chunks of 8 columns per lane) is the widest matrix's.
hipError_t rows_pack_many(const rldx_rows_t* rows, int count, float eps, bool normalize, hipStream_t stream,
                          float* const* stats = nullptr) {
  if (!rows || count < 1 || count > kRowsMax) return hipErrorInvalidValue;
  RowsArgs a{};
  int n = 0, blocks = 0;
  int64_t kmax = 0;
  for (int i = 0; i < count; ++i) {
    const rldx_rows_t& r = rows[i];
    float* st = stats ? stats[i] : nullptr;
    if (r.m < 0 || r.k < 0) return hipErrorInvalidValue;
    if (r.m == 0 || r.k == 0) continue;
    if (!r.x || !r.packed || !a16(r.x) || !a16(r.packed) || r.ldx < r.k || r.ldx % 8 || r.k % 16 || r.k > 8192)
      return hipErrorInvalidValue;
    if (stats && (!st || normalize || r.k % 64 || reinterpret_cast<uintptr_t>(st) % 8)) return hipErrorInvalidValue;
    if (r.m > (int64_t{1} << 28)) return hipErrorInvalidValue;
    a.x[n] = static_cast<const uint16_t*>(r.x);
    a.out[n] = static_cast<uint16_t*>(r.packed);
    a.stats[n] = st;
    a.ldx[n] = r.ldx;
    a.m[n] = static_cast<int>(r.m);
    a.k[n] = static_cast<int>(r.k);
    a.begin[n] = blocks;
    blocks += static_cast<int>((r.m + 3) / 4);
    kmax = r.k > kmax ? r.k : kmax;
    ++n;
  }
  if (n == 0) return hipSuccess;
  a.begin[n] = blocks;
  a.count = n;
  a.normalize = normalize ? 1 : 0;
  a.eps = eps;
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  if (kmax <= 512)
    hipLaunchKernelGGL(rows_pack_kernel<1>, grid, block, 0, stream, a);
  else if (kmax <= 1024)
    hipLaunchKernelGGL(rows_pack_kernel<2>, grid, block, 0, stream, a);
  else if (kmax <= 2048)
    hipLaunchKernelGGL(rows_pack_kernel<4>, grid, block, 0, stream, a);
  else if (kmax <= 4096)
    hipLaunchKernelGGL(rows_pack_kernel<8>, grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL(rows_pack_kernel<16>, grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t rows_pack(const void* x, int64_t ldx, int64_t m, int64_t k, float eps, bool normalize, void* packed,
                     hipStream_t stream, float* stats = nullptr) {
  if (m < 0 || k < 0) return hipErrorInvalidValue;
  if (m == 0 || k == 0) return hipSuccess;
  if (stats && (normalize || k % 64 || reinterpret_cast<uintptr_t>(stats) % 8)) return hipErrorInvalidValue;
  if (m > (int64_t{1} << 28)) return hipErrorInvalidValue;
  const rldx_rows_t r{x, ldx, m, k, packed};
  float* const st[1] = {stats};
  return rows_pack_many(&r, 1, eps, normalize, stream, stats ? st : nullptr);
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
  GemmArgs args;
  int64_t ws, co[3], po[3];
  if (qkv_epi(epilogue)) return hipErrorInvalidValue;  // rldx_grouped_gemm_qkv_norm_rope_bf16
  const hipError_t e = plan(groups, num_groups, n, k, epilogue, 1, args, &ws, co, po);
  if (e != hipSuccess) return e;
  return launch(args, epilogue, stream);
}

extern "C" int64_t rldx_grouped_gemm_workspace_bytes(const rldx_gemm_group_t* groups, int32_t num_groups, int64_t n,
                                                     int64_t k, int32_t epilogue, int32_t split_k) {
  GemmArgs args;
  int64_t ws, co[3], po[3];
  if (qkv_epi(epilogue) || plan(groups, num_groups, n, k, epilogue, split_k, args, &ws, co, po) != hipSuccess)
    return -1;
  return ws;
}

namespace {
hipError_t gemm_ws(const rldx_gemm_group_t* groups, int32_t num_groups, int64_t n, int64_t k, int32_t epilogue,
                   int32_t split_k, int32_t flags, void* workspace, int64_t workspace_bytes, hipStream_t stream,
                   float* const* stats_out = nullptr, const int64_t* group_n = nullptr,
                   const int64_t* group_k = nullptr, const int32_t* group_splits = nullptr) {
  GemmArgs args;
  int64_t ws, co[3], po[3];
  if (qkv_epi(epilogue) || (flags & ~(RLDX_GEMM_WIDE_TILES | RLDX_GEMM_SPLITS_ACROSS_XCDS)))
    return hipErrorInvalidValue;
  const bool wide = (flags & RLDX_GEMM_WIDE_TILES) != 0;
  const hipError_t e = plan(groups, num_groups, n, k, epilogue, split_k, args, &ws, co, po, nullptr, wide, nullptr,
                            nullptr, stats_out, group_n, group_k, group_splits);
  if (e != hipSuccess) return e;
  args.spread = (flags & RLDX_GEMM_SPLITS_ACROSS_XCDS) != 0;
  if (ws > 0) {
    if (!workspace || workspace_bytes < ws || reinterpret_cast<uintptr_t>(workspace) % kWsAlign)
      return hipErrorInvalidValue;
    char* base = static_cast<char*>(workspace);
    for (int i = 0; i < args.num_groups; ++i)
      if (args.g[i].splits > 1) {
        args.g[i].cnt = reinterpret_cast<unsigned*>(base + co[i]);
        args.g[i].part = reinterpret_cast<float*>(base + po[i]);
      }
  }
  return launch(args, epilogue, stream, wide);
}
}  // namespace

extern "C" hipError_t rldx_grouped_gemm_ws_bf16(const rldx_gemm_group_t* groups, int32_t num_groups, int64_t n,
                                                int64_t k, int32_t epilogue, int32_t split_k, void* workspace,
                                                int64_t workspace_bytes, hipStream_t stream) {
  return gemm_ws(groups, num_groups, n, k, epilogue, split_k, 0, workspace, workspace_bytes, stream);
}

extern "C" hipError_t rldx_grouped_gemm_ex_bf16(const rldx_gemm_group_t* groups, int32_t num_groups, int64_t n,
                                                int64_t k, int32_t epilogue, int32_t split_k, int32_t flags,
                                                void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  return gemm_ws(groups, num_groups, n, k, epilogue, split_k, flags, workspace, workspace_bytes, stream);
}

extern "C" int64_t rldx_grouped_gemm_ex_workspace_bytes(const rldx_gemm_group_t* groups, int32_t num_groups,
                                                        int64_t n, int64_t k, int32_t epilogue, int32_t split_k,
                                                        int32_t flags) {
  GemmArgs args;
  int64_t ws, co[3], po[3];
  if (qkv_epi(epilogue) || (flags & ~(RLDX_GEMM_WIDE_TILES | RLDX_GEMM_SPLITS_ACROSS_XCDS)) ||
      plan(groups, num_groups, n, k, epilogue, split_k, args, &ws, co, po, nullptr,
           (flags & RLDX_GEMM_WIDE_TILES) != 0) != hipSuccess)
    return -1;
  return ws;
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

extern "C" hipError_t rldx_layernorm_pack_many_bf16(const rldx_rows_t* rows, int32_t count, float eps,
                                                    hipStream_t stream) {
  return rows_pack_many(rows, count, eps, true, stream);
}

extern "C" hipError_t rldx_act_pack_stats_bf16(const void* x, int64_t ldx, int64_t m, int64_t k, void* packed,
                                               float* ln_stats, hipStream_t stream) {
  if (!ln_stats) return hipErrorInvalidValue;
  return rows_pack(x, ldx, m, k, 0.f, false, packed, stream, ln_stats);
}

extern "C" hipError_t rldx_grouped_gemm_stats_bf16(const rldx_gemm_group_t* groups, float* const* ln_stats_out,
                                                   int32_t num_groups, int64_t n, int64_t k, int32_t epilogue,
                                                   int32_t split_k, int32_t flags, void* workspace,
                                                   int64_t workspace_bytes, hipStream_t stream) {
  if (!ln_stats_out) return hipErrorInvalidValue;
  return gemm_ws(groups, num_groups, n, k, epilogue, split_k, flags, workspace, workspace_bytes, stream,
                 ln_stats_out);
}

extern "C" hipError_t rldx_grouped_gemm_mixed_bf16(const rldx_gemm_group_t* groups, const int64_t* n,
                                                   const int64_t* k, const int32_t* split_k, float* const* ln_stats_out,
                                                   int32_t num_groups, int32_t epilogue, int32_t flags,
                                                   void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  if (!n || !k) return hipErrorInvalidValue;
  return gemm_ws(groups, num_groups, 0, 0, epilogue, 1, flags, workspace, workspace_bytes, stream, ln_stats_out, n, k,
                 split_k);
}

extern "C" int64_t rldx_grouped_gemm_mixed_workspace_bytes(const rldx_gemm_group_t* groups, const int64_t* n,
                                                           const int64_t* k, const int32_t* split_k,
                                                           int32_t num_groups, int32_t epilogue, int32_t flags) {
  GemmArgs args;
  int64_t ws, co[3], po[3];
  if (!n || !k || qkv_epi(epilogue) || (flags & ~(RLDX_GEMM_WIDE_TILES | RLDX_GEMM_SPLITS_ACROSS_XCDS)) ||
      plan(groups, num_groups, 0, 0, epilogue, 1, args, &ws, co, po, nullptr, (flags & RLDX_GEMM_WIDE_TILES) != 0,
           nullptr, nullptr, nullptr, n, k, split_k) != hipSuccess)
    return -1;
  return ws;
}

namespace {
hipError_t gemm_qkv(const rldx_gemm_group_t* groups, const rldx_msat_stream_t* norms, int32_t num_groups,
                    int64_t heads, int64_t head_dim, int64_t k, void* q_out, int64_t q_head_stride,
                    int64_t q_row_stride, void* kv_packed, int64_t kv_packed_head_stride, float eps,
                    const float* const* w_row_sums, const float* const* ln_stats, float ln_eps, hipStream_t stream,
                    const int64_t* group_k = nullptr) {
  if (!groups || !norms || num_groups < 1 || num_groups > 3) return hipErrorInvalidValue;
  // 128-column tiles of whole heads: head_dim 128, or 64 with an even head count
  if (!(head_dim == 128 || (head_dim == 64 && heads % 2 == 0)) || heads <= 0 || heads > 4096)
    return hipErrorInvalidValue;
  if (!q_out || !kv_packed || !a16(q_out) || !a16(kv_packed)) return hipErrorInvalidValue;
  if (q_head_stride < 0 || q_row_stride < 0 || q_head_stride % 8 || q_row_stride % 8 || kv_packed_head_stride % 8)
    return hipErrorInvalidValue;
  // joint rows: each stream starts a 32-key tile of the packed K/V (the rows of
  // a stream that is not the last are padded to a multiple of 32 with zero keys)
  int64_t m = 0;
  for (int i = 0; i < num_groups; ++i) {
    const rldx_gemm_group_t& g = groups[i];
    const rldx_msat_stream_t& s = norms[i];
    if (g.m < 0 || s.rows != g.m) return hipErrorInvalidValue;
    if (g.m == 0) continue;
    m = (m + 31) / 32 * 32;
    if (!s.q_norm_w || !s.k_norm_w || !a16(s.q_norm_w) || !a16(s.k_norm_w)) return hipErrorInvalidValue;
    if ((s.rope_cos == nullptr) != (s.rope_sin == nullptr)) return hipErrorInvalidValue;
    if (s.rope_cos && (!a16(s.rope_cos) || !a16(s.rope_sin) || s.rope_row_stride < head_dim / 2 ||
                       s.rope_row_stride % 4 || s.rope_row_stride > (1 << 24)))
      return hipErrorInvalidValue;
    m += g.m;
  }
  if (m == 0) return hipSuccess;
  if (kv_packed_head_stride < (m + 31) / 32 * 64 * head_dim) return hipErrorInvalidValue;
  if (w_row_sums && !(ln_eps >= 0.f)) return hipErrorInvalidValue;
  GemmArgs args;
  int64_t ws, co[3], po[3];
  const int epi = head_dim == 128 ? kEpiQkv : kEpiQkv64;
  const int64_t n = 3 * heads * head_dim;
  const int64_t ns[3] = {n, n, n};
  const hipError_t e = plan(groups, num_groups, n, k, epi, 1, args, &ws, co, po, norms, false, w_row_sums, ln_stats,
                            nullptr, group_k ? ns : nullptr, group_k);
  if (e != hipSuccess) return e;
  args.qkv = QkvOut{static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(kv_packed), q_head_stride, q_row_stride,
                    kv_packed_head_stride, static_cast<int>(heads * head_dim), eps};
  args.ln_eps = ln_eps;
  return launch(args, epi, stream, true, w_row_sums != nullptr);
}
}  // namespace

extern "C" hipError_t rldx_grouped_gemm_qkv_norm_rope_mixed_bf16(const rldx_gemm_group_t* groups,
                                                                 const rldx_msat_stream_t* norms, int32_t num_groups,
                                                                 int64_t heads, int64_t head_dim, const int64_t* k,
                                                                 void* q_out, int64_t q_head_stride,
                                                                 int64_t q_row_stride, void* kv_packed,
                                                                 int64_t kv_packed_head_stride, float eps,
                                                                 hipStream_t stream) {
  if (!k || num_groups < 1 || num_groups > 3) return hipErrorInvalidValue;
  return gemm_qkv(groups, norms, num_groups, heads, head_dim, k[0], q_out, q_head_stride, q_row_stride, kv_packed,
                  kv_packed_head_stride, eps, nullptr, nullptr, 0.f, stream, k);
}

extern "C" hipError_t rldx_grouped_gemm_qkv_norm_rope_bf16(const rldx_gemm_group_t* groups,
                                                           const rldx_msat_stream_t* norms, int32_t num_groups,
                                                           int64_t heads, int64_t head_dim, int64_t k, void* q_out,
                                                           int64_t q_head_stride, int64_t q_row_stride,
                                                           void* kv_packed, int64_t kv_packed_head_stride, float eps,
                                                           hipStream_t stream) {
  return gemm_qkv(groups, norms, num_groups, heads, head_dim, k, q_out, q_head_stride, q_row_stride, kv_packed,
                  kv_packed_head_stride, eps, nullptr, nullptr, 0.f, stream);
}

extern "C" hipError_t rldx_grouped_gemm_qkv_norm_rope_ln_bf16(
    const rldx_gemm_group_t* groups, const rldx_msat_stream_t* norms, const float* const* w_row_sums,
    const float* const* ln_stats, int32_t num_groups, int64_t heads, int64_t head_dim, int64_t k, void* q_out,
    int64_t q_head_stride, int64_t q_row_stride, void* kv_packed, int64_t kv_packed_head_stride, float eps,
    float ln_eps, hipStream_t stream) {
  if (!w_row_sums || !ln_stats) return hipErrorInvalidValue;
  return gemm_qkv(groups, norms, num_groups, heads, head_dim, k, q_out, q_head_stride, q_row_stride, kv_packed,
                  kv_packed_head_stride, eps, w_row_sums, ln_stats, ln_eps, stream);
}

extern "C" hipError_t rldx_grouped_gemm_ln_bf16(const rldx_gemm_group_t* groups, const float* const* w_row_sums,
                                                const float* const* ln_stats, int32_t num_groups, int64_t n,
                                                int64_t k, int32_t epilogue, int32_t flags, float ln_eps,
                                                hipStream_t stream) {
  GemmArgs args;
  int64_t ws, co[3], po[3];
  if (!w_row_sums || !ln_stats || !(ln_eps >= 0.f) || qkv_epi(epilogue) || (flags & ~RLDX_GEMM_WIDE_TILES))
    return hipErrorInvalidValue;
  const bool wide = (flags & RLDX_GEMM_WIDE_TILES) != 0;
  const hipError_t e = plan(groups, num_groups, n, k, epilogue, 1, args, &ws, co, po, nullptr, wide, w_row_sums,
                            ln_stats);
  if (e != hipSuccess) return e;
  args.ln_eps = ln_eps;
  return launch(args, epilogue, stream, wide, true);
}
