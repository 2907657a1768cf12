/*
 * rldx_amd — C ABI of the MI355X (gfx950) kernels for RLDX-1's real-time
 * inference hot path: fused SwiGLU, fused QK-RMSNorm + RoPE (rotate-half and
 * interleaved), and flash attention (MSAT joint attention, GQA causal prefill).
 *
 * Conventions shared by every entry point
 *   - All tensor pointers are DEVICE pointers owned by the caller.  bf16 data is
 *     passed as raw 16-bit words (uint16_t storage, IEEE bfloat16 bits).
 *   - Strides are in ELEMENTS; the innermost (head_dim / feature) dimension is
 *     contiguous.  Vector paths need 16-byte aligned rows; the functions
 *     validate and return hipErrorInvalidValue instead of guessing.
 *   - No entry point allocates, synchronises the host or keeps mutable state:
 *     each only enqueues kernels on `stream`, so all of them are reentrant and
 *     can be captured into a hipGraph.
 *   - Errors: argument validation -> hipErrorInvalidValue (nothing enqueued);
 *     otherwise the result of hipGetLastError() after the launch.
 *
 * Reference interfaces replaced (paths relative to the RLDX-1 repository):
 *   see the comment above each function.
 */
#ifndef RLDX_AMD_H_
#define RLDX_AMD_H_

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* SwiGLU                                                                   */
/* ------------------------------------------------------------------------ */

/*
 * y[r, j] = bf16( bf16(silu(g)) * u ),  g = x[r, j] (+ bias[j]),
 *                                        u = x[r, n_half + j] (+ bias[n_half + j])
 * for r < rows, j < n_half.  Matches eager `F.silu(x1) * x2` bit for bit
 * (two bf16 roundings); with `bias` (nullable, [2*n_half] bf16) each half is
 * first rounded as bf16(x + b).
 *
 * Replaces: SwiGLUFFN.forward activation (rldx/model/modules/action_model/ops.py:157-161),
 *   SS-block / LLM-chain `F.silu(x1) * x2`
 *   (rldx/inference/action_model/single_stream/engine/custom_single_stream_chain.py:54-55,
 *    rldx/inference/backbone/llm/engine/custom_llm_chain.py:133-135).
 */
hipError_t rldx_swiglu_bf16(const void* x, int64_t ldx, const void* bias, void* y, int64_t ldy, int64_t rows,
                            int64_t n_half, hipStream_t stream);

/*
 * Two SwiGLU groups (SA and VL) in ONE launch; x rows are contiguous
 * [m, 2*n_half], outputs [m, n_half].  Biases are both given or both null.
 *
 * Replaces: fused_grouped_swiglu(sa_w12_out, sa_bias, vl_w12_out, vl_bias, ...)
 *   (rldx/inference/action_model/double_stream/engine/kernels/grouped_swiglu.py:212-257)
 *   behind ds::grouped_swiglu (.../double_stream/engine/ops/op_grouped_swiglu.py:12-49).
 */
hipError_t rldx_grouped_swiglu_bf16(const void* sa_x, const void* sa_bias, const void* vl_x, const void* vl_bias,
                                    void* sa_y, void* vl_y, int64_t m_sa, int64_t m_vl, int64_t n_half_sa,
                                    int64_t n_half_vl, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* QK-RMSNorm + rotate-half RoPE (Qwen3-VL convention)                       */
/* ------------------------------------------------------------------------ */

/* flags bit: `sin` is the pre-signed table of prepare_signed_sin
 * (rldx/inference/backbone/llm/engine/kernels/fused_llm_attention.py:787-796),
 * i.e. its first half already carries rotate_half's minus sign. */
#define RLDX_ROPE_SIN_SIGNED 1
/* flags bit: RoPE only -- no RMSNorm, q_w / k_w unused (may be NULL):
 * apply_rotary_pos_emb alone (rldx/model/modules/backbone/modeling_qwen3_vl.py:377-401). */
#define RLDX_ROPE_NO_NORM 2

/*
 * q' = apply_rotary_pos_emb(q_norm(q)), k' likewise, for q [B, S, Hq, D] and
 * k [B, S, Hk, D] with strides {batch, seq, head} (3 int64 each; D contiguous).
 * cos/sin are [B or 1, S, D] tables (strides {batch, seq}; batch stride 0
 * broadcasts) built on the host.  head_dim 64 or 128.  eps as in the model.
 * fp32 variant: every step in fp32.  bf16 variant: eager bf16 rounding order
 * (bf16(x*rsqrt) -> bf16(w*.) -> bf16(y*cos), bf16(rot*sin) -> bf16(sum)).
 * q_heads or k_heads may be 0 (then q/q_w/q_out, resp. k/k_w/k_out, may be NULL).
 * Tensors, norm weights and tables are 16-byte aligned, strides multiples of
 * 16 bytes; (q_heads + k_heads) * B * S * D / 4 (fp32) or / 8 (bf16) < 2^31.
 * flags: RLDX_ROPE_SIN_SIGNED and / or RLDX_ROPE_NO_NORM (then q' = q cos +
 * rotate_half(q) sin in the input type, eager rounding), or 0.
 *
 * Replaces: Qwen3VLTextRMSNorm.forward + apply_rotary_pos_emb
 *   (rldx/model/modules/backbone/modeling_qwen3_vl.py:356-371, :377-401),
 *   the QK prologue of fused_llm_attention (.../backbone/llm/engine/kernels/fused_llm_attention.py:617-647).
 */
hipError_t rldx_qk_rmsnorm_rope_half_f32(const float* q, const float* k, const float* q_w, const float* k_w,
                                         const float* cos, const float* sin, float* q_out, float* k_out,
                                         int64_t batch, int64_t seq, int64_t q_heads, int64_t k_heads,
                                         int64_t head_dim, const int64_t* q_strides, const int64_t* k_strides,
                                         const int64_t* q_out_strides, const int64_t* k_out_strides,
                                         const int64_t* cos_strides, float eps, int32_t flags,
                                         hipStream_t stream);

hipError_t rldx_qk_rmsnorm_rope_half_bf16(const void* q, const void* k, const void* q_w, const void* k_w,
                                          const void* cos, const void* sin, void* q_out, void* k_out,
                                          int64_t batch, int64_t seq, int64_t q_heads, int64_t k_heads,
                                          int64_t head_dim, const int64_t* q_strides, const int64_t* k_strides,
                                          const int64_t* q_out_strides, const int64_t* k_out_strides,
                                          const int64_t* cos_strides, float eps, int32_t flags,
                                          hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* MSAT multi-stream QKV gather + QK-RMSNorm + interleaved RoPE             */
/* ------------------------------------------------------------------------ */

/* One stream of the joint sequence (VL / SA / P), in joint-sequence order. */
typedef struct rldx_msat_stream {
  const void* qkv;         /* [rows, >= 3*H*D] bf16, packed Q | K | V columns        */
  int64_t qkv_row_stride;  /* elements                                                */
  int64_t rows;            /* tokens in this stream                                   */
  const void* q_norm_w;    /* [D] bf16 RMSNorm weight of this stream's Q              */
  const void* k_norm_w;    /* [D] bf16                                                */
  const float* rope_cos;   /* [rows, D/2] fp32 cos table, or NULL: no rotary          */
  const float* rope_sin;   /* [rows, D/2] fp32 sin table (NULL iff rope_cos is NULL)  */
  int64_t rope_row_stride; /* elements                                                */
} rldx_msat_stream_t;

/*
 * For 1..3 streams concatenated in order (M = sum of rows), writes Q, K, V of
 * layout (H, M, D) at q_out/k_out/v_out with strides {out_head_stride,
 * out_row_stride}:
 *   Q/K = to_bf16(w * (x * rsqrt(mean(x^2) + eps)))       (one rounding)
 *   then, on streams with tables, the interleaved complex rotation in fp32,
 *   rounded once; V is copied.
 * If kv_packed is non-NULL, K and V are written instead (k_out / v_out may be
 * NULL) as the packed K/V tiles rldx_attention_packed_fwd_bf16 reads, head h at
 * kv_packed + h * kv_packed_head_stride (elements, >=
 * rldx_attention_kv_packed_elems(M, D)), padding keys zero — in the same launch.
 *
 * Replaces: rmsnorm_rope_kernel (ds) / rmsnorm_rope_kernel_3way
 *   (rldx/inference/action_model/double_stream/engine/kernels/rmsnorm_rope_ds.py:11-231,
 *    rmsnorm_rope_ds_3way.py:22-386), their ss counterparts
 *   (.../single_stream/engine/kernels/rmsnorm_rope_ss.py:11-192, rmsnorm_rope_ss_3way.py:17-343),
 *   with the eager semantics of RMSNorm (rldx/model/modules/norms.py:18-22) and
 *   apply_rotary_emb (rldx/model/modules/action_model/ops.py:48-67).
 */
hipError_t rldx_msat_qkv_norm_rope_bf16(const rldx_msat_stream_t* streams, int32_t num_streams, int64_t heads,
                                        int64_t head_dim, void* q_out, void* k_out, void* v_out,
                                        int64_t out_head_stride, int64_t out_row_stride, void* kv_packed,
                                        int64_t kv_packed_head_stride, float eps, hipStream_t stream);

/*
 * rldx_msat_qkv_norm_rope_bf16 for a batch of `batch` joint sequences in one
 * launch (0..65535): sequence b reads stream i's rows from
 * streams[i].qkv + b * stream_batch_rows[i] * qkv_row_stride (rows per
 * sequence: streams[i].rows; robot after robot, as the GEMMs stack a stream's
 * rows for a batch) and writes its Q / K / V at b * out_batch_stride, or its
 * packed K/V tiles at kv_packed + b * kv_packed_batch_stride (elements).  The
 * rows a sequence reads may run into the next one's (padding rows whose keys
 * the attention masks); every row read must lie inside the caller's buffer.
 * Each sequence's outputs are those of rldx_msat_qkv_norm_rope_bf16 on its rows,
 * bit for bit.
 * Replaces: the kernels above, called per sample for a batch of robots
 *   (custom_action_model_chain.py:85; the reference's chained ops take one).
 */
hipError_t rldx_msat_qkv_norm_rope_batch_bf16(const rldx_msat_stream_t* streams, int32_t num_streams, int64_t batch,
                                              const int64_t* stream_batch_rows, int64_t heads, int64_t head_dim,
                                              void* q_out, void* k_out, void* v_out, int64_t out_batch_stride,
                                              int64_t out_head_stride, int64_t out_row_stride, void* kv_packed,
                                              int64_t kv_packed_batch_stride, int64_t kv_packed_head_stride,
                                              float eps, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* Attention                                                                */
/* ------------------------------------------------------------------------ */

/*
 * Packed K/V tiles read by the attention kernels.  For each (batch, kv head),
 * ceil(Sk / 32) tiles of 32 keys, 128*D bytes each, contiguous; inside tile t
 * (element offsets, D = head_dim, lane l in 0..63, i in 0..7):
 *   K part: (ks*64 + l)*8 + i            = K[32t + l%32][16 ks + 8 (l/32) + i],  ks < D/16
 *   V part: 32 D + ((2 db + s2)*64 + l)*8 + i
 *                                        = V[32t + 16 s2 + 8 (i/4) + 4 (l/32) + i%4][32 db + l%32],
 *                                          db < D/32, s2 < 2
 * Keys >= Sk hold zeros.  Each 1 KB chunk is one wave's MFMA operand for one
 * v_mfma_f32_32x32x16_bf16 (K for S^T = K Q^T, V^T for O^T = V^T P^T, keys in
 * the row order of the P^T accumulator), so the attention kernel loads every
 * operand with one coalesced 16-byte load per lane.
 */

/* Elements (bf16) of the packed tiles of one (batch, kv head). */
int64_t rldx_attention_kv_packed_elems(int64_t seq_k, int64_t head_dim);

/* Bytes of workspace rldx_attention_fwd_bf16 needs (its packed K/V copy). */
int64_t rldx_attention_workspace_bytes(int64_t batch, int64_t kv_heads, int64_t seq_k, int64_t head_dim);

/*
 * K, V [B, Hkv, Sk, D] (strides {batch, head, seq}, D contiguous) -> packed
 * tiles, packed_strides {batch, head} in elements (head stride >=
 * rldx_attention_kv_packed_elems).
 * No reference counterpart: layout preparation for the attention kernels.
 */
hipError_t rldx_attention_kv_pack_bf16(const void* k, const int64_t* k_strides, const void* v,
                                       const int64_t* v_strides, void* kv_packed, const int64_t* packed_strides,
                                       int64_t batch, int64_t kv_heads, int64_t seq_k, int64_t head_dim,
                                       hipStream_t stream);

/*
 * O = softmax(Q K^T * scale + key_bias[b, key] (+ causal)) V, bf16 in/out,
 * fp32 softmax.  Q [B, Hq, Sq, D], K/V [B, Hkv, Sk, D], O [B, Hq, Sq, D] given
 * by strides {batch, head, seq} (3 int64 each, D contiguous; any permutation of
 * the outer dims works, e.g. token-major [S, H, D]).  Query head h reads KV
 * head h / (Hq / Hkv) (GQA; Hq % Hkv == 0).  key_bias is an optional fp32
 * [B, Sk] additive mask (0 / -inf for key padding), row stride
 * key_bias_batch_stride.  causal != 0: key j visible to query i iff j <= i
 * (top-left aligned, as SDPA's is_causal).  head_dim 64 or 128; scale > 0.
 * Two launches: K, V -> packed tiles in `workspace` (>=
 * rldx_attention_workspace_bytes, 16-byte aligned, caller-owned), then the
 * attention kernel.  seq_k must be >= 1 when seq_q >= 1.
 *
 * Replaces: F.scaled_dot_product_attention inside ds::fused_attention_2way /
 *   _3way and ss::fused_attention_2way / _3way
 *   (rldx/inference/action_model/double_stream/engine/ops/op_fused_attention.py:77-82,
 *    op_fused_attention_3way.py:111-116), eager joint attention
 *   (rldx/model/modules/action_model/blocks.py:577-579, :866), and the causal
 *   GQA core of fused_llm_attention_direct_kernel
 *   (rldx/inference/backbone/llm/engine/kernels/fused_llm_attention.py:379-770).
 */
hipError_t rldx_attention_fwd_bf16(const void* q, const void* k, const void* v, void* o, int64_t batch,
                                   int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k,
                                   int64_t head_dim, const int64_t* q_strides, const int64_t* k_strides,
                                   const int64_t* v_strides, const int64_t* o_strides, const float* key_bias,
                                   int64_t key_bias_batch_stride, float scale, int32_t causal, void* workspace,
                                   int64_t workspace_bytes, hipStream_t stream);

/*
 * Same operator with K and V already packed (packed_strides {batch, head}),
 * one launch.  Used on the MSAT path, where rldx_msat_qkv_norm_rope_bf16 writes
 * the packed tiles directly.  out_packed == 1 (batch 1): O is written as the
 * [seq_q, q_heads*head_dim] matrix in the packed activation order the grouped
 * GEMM reads (o_strides ignored, o 16-byte aligned, rldx_act_packed_elems
 * elements); out_packed > 1 (a multiple of 16, >= q_heads*head_dim): O is
 * written as columns [0, q_heads*head_dim) relative to `o` of a packed matrix
 * out_packed columns wide, `o` pointing at the 16-column chunk where they start
 * (the attention half of a concatenated GEMM operand).
 */
hipError_t rldx_attention_packed_fwd_bf16(const void* q, const void* kv_packed, const int64_t* packed_strides,
                                          void* o, int32_t out_packed, int64_t batch, int64_t q_heads,
                                          int64_t kv_heads, int64_t seq_q,
                                          int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
                                          const int64_t* o_strides, const float* key_bias,
                                          int64_t key_bias_batch_stride, float scale, int32_t causal,
                                          hipStream_t stream);

/*
 * rldx_attention_packed_fwd_bf16 with O written to a packed activation matrix
 * (out_packed as there, o_strides unused) by row segments, for a batch of
 * joint sequences whose streams the GEMMs hold stream by stream (every batch
 * entry's rows of one stream contiguous).  segments: num_segments (1..3) rows
 * {first query row, rows stored, first packed row}, ascending and disjoint
 * inside [0, seq_q): query row r of batch entry b with off <= r < off + rows
 * goes to packed row base + b * rows + (r - off); query rows outside every
 * segment (padding rows of a stream) are not stored.  Any batch >= 1; every
 * packed row below 2^31.  The attention itself is that of
 * rldx_attention_packed_fwd_bf16, bit for bit.
 * Replaces: the joint attention of the double / single-stream blocks with the
 *   [VL | SA | P] output split back into the streams
 *   (rldx/inference/action_model/double_stream/engine/ops/op_fused_attention_3way.py:13-138,
 *   custom_double_stream_chain.py:57-96), for a batch of B robots
 *   (custom_action_model_chain.py:85; the reference's chained ops take one).
 */
hipError_t rldx_attention_packed_segments_fwd_bf16(const void* q, const void* kv_packed,
                                                   const int64_t* packed_strides, void* o, int32_t out_packed,
                                                   const int64_t* segments, int32_t num_segments, int64_t batch,
                                                   int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k,
                                                   int64_t head_dim, const int64_t* q_strides, const float* key_bias,
                                                   int64_t key_bias_batch_stride, float scale, int32_t causal,
                                                   hipStream_t stream);

/*
 * rldx_attention_packed_fwd_bf16 plus a memory-side-cache warm-up: warm_count
 * (0..3) byte ranges warm_ptrs[i] (4-byte aligned), warm_bytes[i] long, whose
 * whole 128-byte lines further workgroups of the same launch read (one dword
 * each, results discarded) while the attention workgroups run.  For a chain of
 * launches that graph replay runs one after another: the joint attention of a
 * block is latency-bound and leaves HBM mostly idle, and the weight panels of a
 * later linear of the block read during it are then served from the
 * memory-side cache when that linear runs (the MSAT step warms its W3 panels
 * here).  The attention result is bit-identical to rldx_attention_packed_fwd_bf16.
 * Replaces: the joint attention of the double-stream blocks, as above
 *   (rldx/model/modules/action_model/blocks.py:866; the warm-up has no counterpart there).
 */
hipError_t rldx_attention_packed_fwd_warm_bf16(const void* q, const void* kv_packed, const int64_t* packed_strides,
                                               void* o, int32_t out_packed, int64_t batch, int64_t q_heads,
                                               int64_t kv_heads, int64_t seq_q, int64_t seq_k, int64_t head_dim,
                                               const int64_t* q_strides, const int64_t* o_strides,
                                               const float* key_bias, int64_t key_bias_batch_stride, float scale,
                                               int32_t causal, const void* const* warm_ptrs,
                                               const int64_t* warm_bytes, int32_t warm_count, hipStream_t stream);

/*
 * The complete rldx_backbone::fused_attention operator: packed QKV
 * (seq, >= (Hq + 2*Hkv)*D) bf16 -> out (seq, Hq*D) bf16 with q_norm/k_norm
 * (Qwen3VLTextRMSNorm, eps) + rotate-half RoPE (cos / sin tables [seq, D] bf16,
 * row stride cos_row_stride; sin pre-signed iff sin_is_signed) + causal GQA
 * attention, scale 1/sqrt(D).  Two launches: K normalisation + RoPE written
 * straight into the packed K/V tiles, with the V tiles packed by the same launch,
 * in `workspace` (>= rldx_llm_fused_attention_workspace_bytes(seq, Hkv, D) bytes,
 * 16-byte aligned, caller-owned), then attention with the Q normalisation fused
 * into its prologue.  qkv, out, cos, sin, q_norm_w and k_norm_w are 16-byte aligned.
 *
 * Replaces: fused_llm_attention.forward(qkv, q_norm_w, q_norm_w_rot, k_norm_w,
 *   k_norm_w_rot, cos, signed_sin, num_heads, num_kv_heads, head_dim, out)
 *   (rldx/inference/backbone/llm/engine/kernels/fused_llm_attention.py:1005-1057)
 *   behind rldx_backbone::fused_attention (.../llm/engine/ops/op_fused_llm_attention.py:13-45).
 *   The rotated norm weights of the reference are not needed: the kernel reads
 *   the rotate-half partner directly.
 */
hipError_t rldx_llm_fused_attention_bf16(const void* qkv, int64_t qkv_row_stride, const void* q_norm_w,
                                         const void* k_norm_w, const void* cos, const void* sin,
                                         int64_t cos_row_stride, int32_t sin_is_signed, void* out,
                                         int64_t out_row_stride, int64_t seq, int64_t q_heads, int64_t kv_heads,
                                         int64_t head_dim, float eps, void* workspace, int64_t workspace_bytes,
                                         hipStream_t stream);

/* Workspace bytes rldx_llm_fused_attention_bf16 needs (the packed K/V tiles). */
int64_t rldx_llm_fused_attention_workspace_bytes(int64_t seq, int64_t kv_heads, int64_t head_dim);

/* Scratch bytes of the allocation-free variant below, per GPU (16 MiB: e.g. 8 KV
 * heads x 4096 tokens at head_dim 128). */
#define RLDX_LLM_ATTN_NOALLOC_MAX_BYTES (16 << 20)

/*
 * rldx_llm_fused_attention_bf16 without a workspace argument: it allocates
 * nothing.  No counterpart in the reference: for callers that cannot allocate
 * device memory (code under hipGraph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The packed K/V tiles go to a file-scope device array
 * of RLDX_LLM_ATTN_NOALLOC_MAX_BYTES that each GPU the library runs on holds
 * until the process ends (its address is resolved once per device, on the
 * first call there, with that device current).  Calls whose
 * rldx_llm_fused_attention_workspace_bytes(seq, kv_heads, head_dim) exceeds it
 * return hipErrorInvalidValue with nothing enqueued.  Every call on a GPU shares
 * that GPU's array, so the library serialises them on the device: each call's
 * stream first waits for an event recorded after the previous call on that GPU
 * (whatever stream it used), and records it after its own launches; a mutex
 * makes this atomic across host threads.  The event is created once per
 * device, on the first call there, beside the address lookup.  A stream under
 * hipGraph capture skips the event: replays of a captured call are ordered
 * only by the stream they are launched on, so a caller that replays such a
 * graph beside other calls on the same GPU must order them itself.  Same
 * results as rldx_llm_fused_attention_bf16 (the same kernels).
 */
hipError_t rldx_llm_fused_attention_noalloc_bf16(const void* qkv, int64_t qkv_row_stride, const void* q_norm_w,
                                                 const void* k_norm_w, const void* cos, const void* sin,
                                                 int64_t cos_row_stride, int32_t sin_is_signed, void* out,
                                                 int64_t out_row_stride, int64_t seq, int64_t q_heads,
                                                 int64_t kv_heads, int64_t head_dim, float eps, hipStream_t stream);

/*
 * The rldx_backbone::vision_attention operator (Qwen3-VL ViT blocks): fused
 * QKV rows (total_tokens, 3*num_heads*head_dim) bf16, contiguous -> out
 * (total_tokens, num_heads*head_dim) bf16, contiguous.  Per head, the Q and K
 * columns get rotate-half RoPE in fp32 with the baked tables rope_cos /
 * rope_sin (total_tokens, head_dim) fp32, contiguous (sin's first half already
 * negated):  y[d] = bf16(x[d] * cos[d] + x[d +- head_dim/2] * sin[d]);  then
 * non-causal softmax(Q K^T * scaling) V over each sequence
 * [cu_seqlens[s], cu_seqlens[s+1]) (cu_seqlens: num_seqs + 1 int32 in device
 * memory, ascending, cu_seqlens[num_seqs] <= total_tokens), fp32 scores and
 * softmax, P rounded to bf16 before P.V.  Rows outside every sequence are not
 * written.  Sequences may have any lengths; the launch depends only on
 * total_tokens and num_seqs, never on the cu_seqlens values (graph
 * capturable); out-of-range cu_seqlens values are clamped to [0, total_tokens]
 * on the device.  head_dim % 8 == 0, 8 <= head_dim <= 128 (computed at 64,
 * 96 or 128 columns with zero padding).  qkv, rope_cos, rope_sin, workspace
 * 16-byte aligned, out 8-byte aligned.  Two launches: RoPE + K/V packing into
 * `workspace` (>= rldx_vision_attention_workspace_bytes bytes, caller-owned;
 * layout: RoPE'd Q [num_heads][total_tokens][64|96|128] bf16 at offset 0,
 * then the packed K/V tiles), then the attention kernel.
 *
 * Replaces: fused_vision_attention.forward(qkv, rope_cos, rope_sin, cu_seqlens,
 *   scaling, num_heads, head_dim)
 *   (rldx/inference/backbone/vision_encoder/engine/kernels/fused_vision_attention.py:622-645)
 *   behind rldx_backbone::vision_attention
 *   (.../vision_encoder/engine/ops/op_fused_vision_attention.py:14-42).  The
 *   reference sizes its grid for equal-length sequences (M // num_seqs, :490);
 *   here every sequence is covered whatever its length.
 */
hipError_t rldx_vision_attention_bf16(const void* qkv, const float* rope_cos, const float* rope_sin,
                                      const int32_t* cu_seqlens, int64_t num_seqs, void* out, int64_t total_tokens,
                                      int64_t num_heads, int64_t head_dim, float scaling, void* workspace,
                                      int64_t workspace_bytes, hipStream_t stream);

/*
 * The mem::fused_attention operator (TransformerMemory layers): fused QKV rows
 * (tokens, 3*num_heads*head_dim) bf16, contiguous -> out (tokens,
 * num_heads*head_dim) bf16, contiguous.  Q and K get rotate-half RoPE in bf16
 * arithmetic, each step rounded to bf16 as the eager module does:
 *   y[d] = bf16(bf16(x[d] * cos[d]) + bf16(x[d +- head_dim/2] * signed_sin[d]))
 * (cos / signed_sin (tokens, head_dim) bf16, contiguous, sin's first half
 * negated); then softmax(Q K^T / sqrt(head_dim)) V with the block-causal mask:
 * query i sees key j iff j / block_attn_size <= i / block_attn_size.  fp32
 * scores and softmax, P rounded to bf16 before P.V.  head_dim 64, 128 or 256;
 * block_attn_size >= 1.  qkv, cos, signed_sin 16-byte aligned, out 8-byte
 * aligned.  One launch, no workspace.
 *
 * Replaces: fused_memory_attention.forward(qkv, cos, signed_sin, num_heads,
 *   head_dim, block_attn_size)
 *   (rldx/inference/memory/engine/kernels/fused_memory_attention.py:220-264)
 *   behind mem::fused_attention (.../memory/engine/ops/op_fused_memory_attention.py:12-36).
 */
hipError_t rldx_memory_attention_bf16(const void* qkv, const void* cos, const void* signed_sin, void* out,
                                      int64_t tokens, int64_t num_heads, int64_t head_dim, int64_t block_attn_size,
                                      hipStream_t stream);

/* Workspace bytes rldx_vision_attention_bf16 needs; -1 for an unsupported head_dim. */
int64_t rldx_vision_attention_workspace_bytes(int64_t total_tokens, int64_t num_seqs, int64_t num_heads,
                                              int64_t head_dim);

/* ------------------------------------------------------------------------ */
/* Grouped GEMM of the MSAT block linears                                   */
/* ------------------------------------------------------------------------ */

/*
 * Packs a weight W [n, k] bf16 (row stride ldw elements, k contiguous) into
 * the MFMA operand order rldx_grouped_gemm_bf16 reads (n*k elements): 1 KB
 * chunk (nb, kb), nb-major, holds W[32 nb + l%32][16 kb + 8 (l/32) + i] at
 * element (nb*(k/16) + kb)*512 + l*8 + i.  With swiglu_pairs != 0, W = [gate;
 * up] (n = 2*N_half) and packed block 2p holds gate rows 32p.., block 2p+1 up
 * rows N_half + 32p.. .  n % 32 == 0 (% 64 with swiglu_pairs), k % 16 == 0.
 * No reference counterpart: one-time weight preparation.
 */
hipError_t rldx_gemm_pack_weight_bf16(const void* w, int64_t ldw, int64_t n, int64_t k, int32_t swiglu_pairs,
                                      void* packed, hipStream_t stream);

/*
 * Packed activation order read by rldx_grouped_gemm_bf16 for its A operand:
 * A [m, k] stored as 1 KB chunks (mb, kb), mb-major, chunk (mb, kb) at element
 * (mb*(k/16) + kb)*512 holding A[32 mb + l%32][16 kb + 8 (l/32) + i] at l*8 + i.
 * Rows are padded to a multiple of 32 (padding never reaches an output).
 */
int64_t rldx_act_packed_elems(int64_t m, int64_t k);

/* Row-major x [m, k] (row stride ldx) -> packed activation order.  k % 16 == 0. */
hipError_t rldx_act_pack_bf16(const void* x, int64_t ldx, int64_t m, int64_t k, void* packed, hipStream_t stream);

/*
 * LayerNorm without affine parameters, y = (x - mean) * rsqrt(var + eps) per
 * row (fp32 statistics, one rounding), written in the packed activation order.
 * k % 16 == 0, k <= 8192.
 * Replaces: the pre-norms of an MSAT block, nn.LayerNorm(dim, elementwise_affine=False)
 *   (rldx/model/modules/action_model/blocks.py:705-891; rldx/model/modules/action_model/msat.py:883-893).
 */
hipError_t rldx_layernorm_pack_bf16(const void* x, int64_t ldx, int64_t m, int64_t k, float eps, void* packed,
                                    hipStream_t stream);

/* One row-major bf16 matrix x [m, k] (row stride ldx elements) and its packed
 * activation buffer (rldx_act_packed_elems(m, k) elements). */
typedef struct {
  const void* x;
  int64_t ldx, m, k;
  void* packed;
} rldx_rows_t;

/*
 * rldx_layernorm_pack_bf16 over up to 4 matrices in one launch (each its own m,
 * k <= 8192 and eps shared): the pre-norms of the streams of one block, which
 * the reference applies one after the other.  Each output is bit-identical to
 * rldx_layernorm_pack_bf16 on that matrix alone.
 * Replaces: sa_norm1 / vl_norm1 / p_norm1 and the *_norm2_mlp pre-norms of the
 *   double-stream blocks (rldx/model/modules/action_model/blocks.py:508-520, 599-604, 804-818, 882-888).
 */
hipError_t rldx_layernorm_pack_many_bf16(const rldx_rows_t* rows, int32_t count, float eps, hipStream_t stream);

/*
 * The action encoder side of one flow-matching iteration of the action step,
 * one launch: the n action rows x = bf16(bf16(bf16(act W_in^T + b_in) + temb)
 * + pos) (act [n, action_dim], W_in [hidden, action_dim], b_in / temb [hidden],
 * pos [n, hidden], all bf16 row-major; the dot products in fp32) written in the
 * packed activation order at `packed` with their LayerNorm statistics
 * ([hidden / 64][n][2] fp32, the row's sum and sum of squares in slot 0, zeros
 * in the others, as rldx_act_pack_stats_bf16 writes them), and up to 3 more
 * row-major matrices rows[i] (k == hidden) packed with statistics rows_stats[i]
 * in the same launch.  action_dim % 8 == 0 and <= 64; hidden % 64 == 0 and
 * <= 2048; 16-byte aligned tensors.
 * Replaces: the action encoder + baked position embedding before the MSAT and
 *   the MSAT's input packing in the action chain's denoising loop
 *   (rldx/inference/action_model/engine/custom_action_model_chain.py:138-141; the
 *   synthetic action step's encoder is one Linear).
 */
hipError_t rldx_action_encode_pack_bf16(const void* act, int64_t n, int64_t action_dim, const void* w_in,
                                        const void* b_in, const void* temb, const void* pos, int64_t hidden,
                                        void* packed, float* stats, const rldx_rows_t* rows,
                                        float* const* rows_stats, int32_t num_rows, hipStream_t stream);

/*
 * The action decoder side of the iteration and its Euler update, one launch:
 * act = bf16(act + bf16(dt * bf16(LN(x) W_out^T + b_out))) for the n rows x of
 * a packed activation matrix [n, hidden] (LN without affine parameters:
 * bf16((x - mean) / sqrt(var + eps)), biased variance, fp32), W_out
 * [action_dim, hidden], b_out [action_dim], act [n, action_dim] updated in
 * place.  Limits as rldx_action_encode_pack_bf16.
 * Replaces: the action decoder and the Euler step of the denoising loop
 *   (rldx/inference/action_model/engine/custom_action_model_chain.py:166-169; the
 *   synthetic action step's decoder is LayerNorm + one Linear).
 */
hipError_t rldx_action_decode_euler_bf16(const void* packed, int64_t n, int64_t hidden, float eps, const void* w_out,
                                         const void* b_out, int64_t action_dim, float dt, void* act,
                                         hipStream_t stream);

/* One stream of a grouped GEMM. */
typedef struct rldx_gemm_group {
  const void* a_packed;  /* [m, k] bf16 activations in the packed activation order */
  int64_t m;             /* rows (0: group skipped)                              */
  const void* w_packed;  /* packed weight [n, k] of this stream                  */
  const void* bias;      /* [n] bf16 or NULL ([gate; up] order for SwiGLU)       */
  void* out;             /* [m, n] bf16 ([m, n/2] for SwiGLU), row stride ldo;   */
                         /* packed activation order for the *_PACKED epilogues: */
  int64_t ldo;           /* then ldo = 0 (a packed [m, n_out] matrix) or the     */
                         /* width (% 16) of a wider packed matrix whose 16-col  */
                         /* chunk at `out` is the first output column           */
  const void* residual;  /* [m, n] bf16, row stride ldr (RESIDUAL epilogue; may  */
  int64_t ldr;           /* alias out); RESIDUAL_PACKED: packed order, ldr as ldo */
} rldx_gemm_group_t;

#define RLDX_GEMM_EPI_BIAS 0     /* out = bf16(a W^T + bias)                      */
#define RLDX_GEMM_EPI_RESIDUAL 1 /* out = bf16(residual + bf16(a W^T + bias))     */
#define RLDX_GEMM_EPI_SWIGLU 2   /* out = swiglu(bf16(gate), bf16(up)), n/2 cols  */
#define RLDX_GEMM_EPI_SWIGLU_PACKED 3 /* same, out in the packed activation order */
#define RLDX_GEMM_EPI_BIAS_PACKED 4   /* out = bf16(a W^T + bias), packed order     */
#define RLDX_GEMM_EPI_RESIDUAL_PACKED 5 /* RESIDUAL with out and residual in the  */
                                        /* packed activation order (in place)      */

/*
 * y_s = a_s W_s^T (+ bias_s) with the epilogue above, for 1..3 groups that
 * share n and k (the three streams of an MSAT block), fp32 accumulation.
 * n % 64 == 0, k % 128 == 0.  One launch; per group 128 x 128 tiles (at least
 * 256 rows and 128 tiles), 64 x 64 tiles (more than 32 rows) or 32 x 64 tiles.
 * Deterministic (fixed summation order for a given shape).
 * Replaces: the per-stream nn.Linear calls of an MSAT block
 *   (rldx/model/modules/action_model/blocks.py:705-891), and
 *   fused_mlp_swiglu(x, weight, bias) behind ss::fused_mlp_swiglu
 *   (rldx/inference/action_model/single_stream/engine/kernels/fused_mlp_swiglu.py:199-267)
 *   with the SwiGLU epilogue.
 */
hipError_t rldx_grouped_gemm_bf16(const rldx_gemm_group_t* groups, int32_t num_groups, int64_t n, int64_t k,
                                  int32_t epilogue, hipStream_t stream);

/*
 * Workspace bytes rldx_grouped_gemm_ws_bf16 needs for these groups, shapes and
 * split_k (0 when nothing is split), or -1 if the call would be rejected.
 */
int64_t rldx_grouped_gemm_workspace_bytes(const rldx_gemm_group_t* groups, int32_t num_groups, int64_t n, int64_t k,
                                          int32_t epilogue, int32_t split_k);

/*
 * rldx_grouped_gemm_bf16 with split-K across workgroups: every group has its K
 * range split over S workgroups, S the largest power of two <= split_k that
 * divides the group's stages (split_k <= 1: no split).  Each split streams its
 * part of the operands; the partial tiles are summed in split
 * order by the last workgroup to finish the tile, so results do not depend on
 * timing (they differ from the unsplit sum by fp32 rounding only).  The splits
 * exchange partials with device-scope stores, loads and counter atomics, so the
 * hand-off holds on whichever XCDs they run; the launch places the splits of a
 * tile on one XCD, where the exchange stays close to that XCD's L2.
 * workspace: device memory, 256-byte aligned, at least
 * rldx_grouped_gemm_workspace_bytes(...) bytes, zero-filled before its first
 * use; each launch leaves it ready for the next, whatever its shapes (the first
 * 64 KB hold tile counters, at most 16384 split tiles per launch; partials
 * follow).  Launches that share a workspace must not overlap in time.  Too
 * small, missing or misaligned: hipErrorInvalidValue.
 * Replaces: the split_k argument of fused_mlp_swiglu(x, weight, bias, split_k)
 *   (rldx/inference/action_model/single_stream/engine/ops/op_fused_mlp_swiglu.py:13-43)
 *   and the per-stream nn.Linear calls of an MSAT block, as rldx_grouped_gemm_bf16.
 */
hipError_t rldx_grouped_gemm_ws_bf16(const rldx_gemm_group_t* groups, int32_t num_groups, int64_t n, int64_t k,
                                     int32_t epilogue, int32_t split_k, void* workspace, int64_t workspace_bytes,
                                     hipStream_t stream);

#define RLDX_GEMM_WIDE_TILES 1 /* 64 x 128 / 32 x 128 tiles for streams below the 128 x 128 threshold */
#define RLDX_GEMM_SPLITS_ACROSS_XCDS 2 /* the splits of a tile on different XCDs (tests of the split hand-off) */

/*
 * rldx_grouped_gemm_ws_bf16 with flags: RLDX_GEMM_WIDE_TILES gives the streams
 * that would take 64 x 64 or 32 x 64 tiles 64 x 128 or 32 x 128 tiles instead
 * (half the workgroups, each streaming a 128-column weight panel).  The K-groups
 * are those of the narrow tiles, so the results are the same bit for bit; which
 * is faster depends on the shape (wide: 64 x 22016 x 4096 SwiGLU 47.9 -> 42.2 us,
 * 64 x 4096 x 11008 split 4: 23.9 -> 31.1 us on MI355X).
 * RLDX_GEMM_SPLITS_ACROSS_XCDS places the splits of each tile on consecutive
 * workgroups (different XCDs) instead of on one XCD: the same results bit for
 * bit, for tests of the cross-XCD hand-off.  Other flag bits are rejected.  rldx_grouped_gemm_ex_workspace_bytes is the matching workspace query.
 * Replaces: as rldx_grouped_gemm_bf16.
 */
hipError_t rldx_grouped_gemm_ex_bf16(const rldx_gemm_group_t* groups, int32_t num_groups, int64_t n, int64_t k,
                                     int32_t epilogue, int32_t split_k, int32_t flags, void* workspace,
                                     int64_t workspace_bytes, hipStream_t stream);
int64_t rldx_grouped_gemm_ex_workspace_bytes(const rldx_gemm_group_t* groups, int32_t num_groups, int64_t n,
                                             int64_t k, int32_t epilogue, int32_t split_k, int32_t flags);

/*
 * The QKV linears of an MSAT block with the QK-RMSNorm + RoPE + K/V tiling of
 * rldx_msat_qkv_norm_rope_bf16 in the GEMM's epilogue (one launch instead of
 * two): for 1..3 groups in joint-sequence order, y_s = a_s W_s^T + bias_s with
 * W_s [3 * heads * head_dim, k] packed, y = [Q | K | V] per row; groups[i].out /
 * ldo / residual are unused.  norms[i] gives stream i's Q / K norm weights and
 * RoPE tables (its qkv / qkv_row_stride are unused; rows == groups[i].m).  Q is
 * written as (H, M, head_dim) at q_out with strides {q_head_stride, q_row_stride},
 * K and V as the packed K/V tiles at kv_packed + h * kv_packed_head_stride
 * (padding keys zero).  Each non-empty group starts a 32-key tile of the joint
 * sequence (M = its padded rows): a group before the last with rows % 32 != 0 is
 * followed by zero padding keys, and its padding Q rows are not written;
 * head_dim == 128, or 64 with an even head count (a 128-column tile then holds
 * two heads); k % 128 == 0.  Results are
 * bit-identical to rldx_grouped_gemm_bf16 (RLDX_GEMM_EPI_BIAS) followed by
 * rldx_msat_qkv_norm_rope_bf16 with kv_packed.
 * Replaces: the QKV nn.Linear calls of an MSAT block followed by its
 *   QK-RMSNorm + RoPE kernel (rldx/model/modules/action_model/blocks.py:525-537;
 *   rldx/inference/action_model/double_stream/engine/kernels/rmsnorm_rope_ds_3way.py:22-386).
 */
hipError_t rldx_grouped_gemm_qkv_norm_rope_bf16(const rldx_gemm_group_t* groups, const rldx_msat_stream_t* norms,
                                                int32_t num_groups, int64_t heads, int64_t head_dim, int64_t k,
                                                void* q_out, int64_t q_head_stride, int64_t q_row_stride,
                                                void* kv_packed, int64_t kv_packed_head_stride, float eps,
                                                hipStream_t stream);

/*
 * rldx_grouped_gemm_qkv_norm_rope_bf16 with a K per group (k[i], each a
 * multiple of 128; the same [Q | K | V] columns for every group): the QKV
 * linears of streams of different widths in one launch (the VL (4096) and SA
 * (1536) streams of an RLDX-1 double-stream block have this shape, head_dim
 * 64; the RLDX-1 chain keeps its split-K QKV launch plus
 * rldx_msat_qkv_norm_rope_bf16 there, which measured as fast: the fused
 * epilogue does not split K).  Bit-identical to the per-group GEMMs followed by
 * rldx_msat_qkv_norm_rope_bf16.
 * Replaces: the per-stream QKV nn.Linear calls of DoubleStreamBlock.forward and
 *   its QK-RMSNorm + RoPE (rldx/model/modules/action_model/blocks.py:508-537;
 *   rldx/inference/action_model/double_stream/engine/kernels/rmsnorm_rope_ds_3way.py:22-386).
 */
hipError_t rldx_grouped_gemm_qkv_norm_rope_mixed_bf16(const rldx_gemm_group_t* groups,
                                                      const rldx_msat_stream_t* norms, int32_t num_groups,
                                                      int64_t heads, int64_t head_dim, const int64_t* k, void* q_out,
                                                      int64_t q_head_stride, int64_t q_row_stride, void* kv_packed,
                                                      int64_t kv_packed_head_stride, float eps, hipStream_t stream);

/*
 * LayerNorm statistics of activation rows, for a GEMM with the pre-LayerNorm
 * folded in: fp32 [k / 64][rows][2] (slot-major: slot j of row r at
 * (j * rows + r) * 2), slot j of a row holding (sum, sum of squares) of some of
 * the row's k values, the slots of a row together covering each value once (the
 * producers below write the sums of columns [64 j, 64 j + 64), or of 128
 * columns in one slot and zeros in the next, or the whole row in slot 0 and
 * zeros elsewhere).
 */

/*
 * rldx_act_pack_bf16 that also writes the rows' LayerNorm statistics
 * (slot 0: the row's sums; the other slots zero).  k % 64 == 0; ln_stats 8-byte
 * aligned.
 * Replaces: the activation side of the pre-norm nn.LayerNorm of an MSAT block
 *   (rldx/model/modules/action_model/blocks.py:804, :882), for the folded GEMMs.
 */
hipError_t rldx_act_pack_stats_bf16(const void* x, int64_t ldx, int64_t m, int64_t k, void* packed, float* ln_stats,
                                    hipStream_t stream);

/*
 * rldx_grouped_gemm_ex_bf16 with the RESIDUAL or RESIDUAL_PACKED epilogue that
 * also writes the LayerNorm statistics of the rows it stores (the updated
 * residual stream): ln_stats_out[i] is group i's [n / 64][m][2] (8-byte aligned).
 * The statistics are of the bf16 values stored.  Deterministic.
 * Replaces: the residual additions of an MSAT block (blocks.py:870-889) together
 *   with the statistics half of the next pre-norm.
 */
hipError_t rldx_grouped_gemm_stats_bf16(const rldx_gemm_group_t* groups, float* const* ln_stats_out,
                                        int32_t num_groups, int64_t n, int64_t k, int32_t epilogue, int32_t split_k,
                                        int32_t flags, void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * The grouped GEMM with a shape per group: groups[i] multiplies by its own
 * W [n[i], k[i]] (each n a multiple of 64, each k of 128) and splits its K
 * range over split_k[i] workgroups (NULL: no split; as in
 * rldx_grouped_gemm_ws_bf16, the largest power of two <= split_k[i] that
 * divides its stages), all in one launch with one epilogue (not the QKV one).
 * For the linears of a block whose streams have different widths (the SA and
 * VL streams of an RLDX-1 double-stream block): the short stream's tiles run
 * beside the long one's instead of in a launch of their own.  ln_stats_out:
 * as in rldx_grouped_gemm_stats_bf16, or NULL.  Workspace from
 * rldx_grouped_gemm_mixed_workspace_bytes (-1: invalid call).  Each group's
 * result is bit-identical to the same group launched alone with the same split.
 * Replaces: the per-stream linears of DoubleStreamBlock.forward
 *   (rldx/model/modules/action_model/blocks.py:500-609; custom_double_stream_chain.py:57-96).
 */
hipError_t rldx_grouped_gemm_mixed_bf16(const rldx_gemm_group_t* groups, const int64_t* n, const int64_t* k,
                                        const int32_t* split_k, float* const* ln_stats_out, int32_t num_groups,
                                        int32_t epilogue, int32_t flags, void* workspace, int64_t workspace_bytes,
                                        hipStream_t stream);
int64_t rldx_grouped_gemm_mixed_workspace_bytes(const rldx_gemm_group_t* groups, const int64_t* n, const int64_t* k,
                                                const int32_t* split_k, int32_t num_groups, int32_t epilogue,
                                                int32_t flags);

/*
 * The pre-LayerNorm of an MSAT block folded into the grouped GEMM that consumes
 * it: y_s = LN(a_s) W_s^T + bias_s with LN the LayerNorm over the k columns
 * without affine parameters (eps ln_eps), from the un-normalised rows a_s
 * (packed activation order, e.g. a residual stream kept packed by
 * RLDX_GEMM_EPI_RESIDUAL_PACKED) and their statistics ln_stats[i] ([k / 64][m][2]
 * as above, from rldx_grouped_gemm_stats_bf16 or rldx_act_pack_stats_bf16).
 * w_row_sums[i] is group i's fp32 vector s[j] = sum_k W[j][k] over the n rows of
 * W in their original order ([gate; up] for SwiGLU).  The kernel computes
 * mean = sum / k and the biased variance sumsq / k - mean^2 (fp32, clamped at 0)
 * per row, rstd = rsqrt(var + eps) (the hardware reciprocal square root), and
 * rstd * (a W^T) - rstd * mean * s before the epilogue.
 * Epilogues: BIAS and SWIGLU_PACKED (flags: RLDX_GEMM_WIDE_TILES); no split-K;
 * k <= 2048.  Against LN(a) rounded to bf16 and then multiplied, the result skips
 * that one rounding of the normalised rows (about 0.1 % of |y| per element); it
 * is not bit-identical to rldx_layernorm_pack_bf16 followed by
 * rldx_grouped_gemm_bf16.
 * Replaces: the pre-norm nn.LayerNorm(dim, elementwise_affine=False) and the
 *   nn.Linear calls it feeds in an MSAT block
 *   (rldx/model/modules/action_model/blocks.py:804, :882 with :806-826, :886-888).
 */
hipError_t rldx_grouped_gemm_ln_bf16(const rldx_gemm_group_t* groups, const float* const* w_row_sums,
                                     const float* const* ln_stats, int32_t num_groups, int64_t n, int64_t k,
                                     int32_t epilogue, int32_t flags, float ln_eps, hipStream_t stream);

/*
 * rldx_grouped_gemm_qkv_norm_rope_bf16 with the pre-LayerNorm folded in, as
 * rldx_grouped_gemm_ln_bf16 (w_row_sums per group over the 3 * heads * 128 rows
 * of [W_q; W_k; W_v], ln_stats of the A rows, ln_eps the LayerNorm's eps; eps
 * stays the QK-RMSNorm's).
 * Replaces: the pre-norm + QKV nn.Linear + QK-RMSNorm + RoPE of an MSAT block
 *   (rldx/model/modules/action_model/blocks.py:804-834).
 */
hipError_t rldx_grouped_gemm_qkv_norm_rope_ln_bf16(const rldx_gemm_group_t* groups, const rldx_msat_stream_t* norms,
                                                   const float* const* w_row_sums, const float* const* ln_stats,
                                                   int32_t num_groups, int64_t heads, int64_t head_dim, int64_t k,
                                                   void* q_out, int64_t q_head_stride, int64_t q_row_stride,
                                                   void* kv_packed, int64_t kv_packed_head_stride, float eps,
                                                   float ln_eps, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* Host-side diagnostics (no reference counterpart)                         */
/* ------------------------------------------------------------------------ */

/*
 * Runs the SwiGLU element function the GPU kernels use, on the CPU, for n
 * (gate, up) bf16 pairs.  Exists so that the CPU test suite can verify the
 * silu/product rounding exhaustively over all 65536 bf16 inputs without a GPU.
 * Not used by any product path.  Returns 0 on success.
 */
int rldx_host_swiglu_bf16(const uint16_t* g, const uint16_t* u, uint16_t* y, int64_t n);

/* ------------------------------------------------------------------------- */
/* Residual-add + norm epilogues at block boundaries.  Rows are contiguous     */
/* (row stride = dim), bf16; dim <= 8192.  Outputs may alias inputs exactly   */
/* (same pointer, same layout), e.g. an in-place residual update.  The fast   */
/* path needs dim % 8 == 0 and 16-byte aligned rows; other shapes take a      */
/* slower scalar path.                                                        */
/* ------------------------------------------------------------------------- */

/*
 * Per stream s in {sa, vl}: out_s = LayerNorm(res_s + proj_s + bias_s) without
 * affine; the three-term sum is kept in fp32 (no intermediate rounding), fp32
 * statistics, one rounding.  bias_s is a [dim_s] vector broadcast over rows.
 * Replaces: ds::grouped_res_ln / fused_grouped_res_ln
 *   (rldx/inference/action_model/double_stream/engine/ops/op_grouped_res_ln.py:13-45,
 *    rldx/inference/action_model/double_stream/engine/kernels/grouped_res_ln.py:40-211).
 */
hipError_t rldx_grouped_res_ln_bf16(const void* sa_res, const void* sa_bias, const void* sa_proj, void* sa_out,
                                    const void* vl_res, const void* vl_bias, const void* vl_proj, void* vl_out,
                                    int64_t m_sa, int64_t m_vl, int64_t sa_dim, int64_t vl_dim, float eps,
                                    hipStream_t stream);

/*
 * new_vl = ((vl_res + proj_bias) + w3_bias) + w3_out, each add rounded to bf16
 * (eager bf16 tensor adds); ln_vl = LayerNorm(new_vl) without affine.
 * proj_bias, w3_bias: [dim] vectors broadcast over rows.
 * Replaces: ds::vl_epilogue_ln / fused_vl_epilogue_ln
 *   (rldx/inference/action_model/double_stream/engine/ops/op_vl_epilogue_ln.py:13-45,
 *    rldx/inference/action_model/double_stream/engine/kernels/vl_epilogue_ln.py:31-183).
 */
hipError_t rldx_vl_epilogue_ln_bf16(const void* vl_res, const void* proj_bias, const void* w3_bias,
                                    const void* w3_out, void* new_vl, void* ln_vl, int64_t m, int64_t dim,
                                    float eps, hipStream_t stream);

/*
 * With residual: new_hidden = bf16(hidden + residual), ln_out = LayerNorm(new_hidden).
 * residual == NULL: ln_out = LayerNorm(hidden) and new_hidden is not written
 * (the hidden state is already final).  LayerNorm without affine.
 * Replaces: ss::fused_epilogue_ln / fused_ss_epilogue_ln
 *   (rldx/inference/action_model/single_stream/engine/ops/op_fused_epilogue_ln.py:11-35,
 *    rldx/inference/action_model/single_stream/engine/kernels/ss_epilogue_ln.py:33-205).
 */
hipError_t rldx_ss_epilogue_ln_bf16(const void* hidden, const void* residual, void* new_hidden, void* ln_out,
                                    int64_t m, int64_t dim, float eps, hipStream_t stream);

/*
 * new_hidden = bf16(hidden + residual), then bf16(new_hidden + deepstack) when
 * deepstack != NULL; normed = bf16(weight * bf16(new_hidden * rsqrt(mean(new_hidden^2) + eps)))
 * (Qwen3VLTextRMSNorm on the rounded sum, the eager arithmetic).
 * Replaces: rldx_backbone::fused_epilogue_add2_rmsnorm and ::fused_epilogue_add3_rmsnorm
 *   (rldx/inference/backbone/llm/engine/ops/op_fused_epilogue_add2_rmsnorm.py:20-45,
 *    op_fused_epilogue_add3_rmsnorm.py:20-47; kernels/fused_add2_rmsnorm.py:29-115,
 *    kernels/fused_add3_rmsnorm.py:31-83).
 */
hipError_t rldx_add_rmsnorm_bf16(const void* hidden, const void* residual, const void* deepstack,
                                 const void* weight, void* new_hidden, void* normed, int64_t m, int64_t dim,
                                 float eps, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* Model-level primitives of the eager modules                               */
/* ------------------------------------------------------------------------ */

/*
 * RMSNorm with one rounding: out = (w * (x * rsqrt(mean(x^2) + eps))).to(x's
 * dtype), fp32 arithmetic, over rows of `dim` values (row strides in
 * elements).  weight [dim] is fp32 (weight_is_f32 = 1, the module's parameter)
 * or bf16 (0, a model cast to bf16; promoted to fp32 by the product).  dim a
 * multiple of 8 (bf16) / 4 (fp32) up to 8192 / 4096; x, out (and an fp32
 * weight) 16-byte aligned.
 * Replaces: RMSNorm.forward (rldx/model/modules/norms.py:7-22), the module the
 *   MSAT's create_qk_norm_layers and the memory module instantiate.
 */
hipError_t rldx_rms_norm_bf16(const void* x, int64_t x_row_stride, const void* weight, int32_t weight_is_f32,
                              void* out, int64_t out_row_stride, int64_t rows, int64_t dim, float eps,
                              hipStream_t stream);
hipError_t rldx_rms_norm_f32(const float* x, int64_t x_row_stride, const void* weight, int32_t weight_is_f32,
                             float* out, int64_t out_row_stride, int64_t rows, int64_t dim, float eps,
                             hipStream_t stream);

/*
 * Interleaved (complex) RoPE of q [B, Hq, N, D] and k [B, Hk, N, D] (strides
 * {batch, head, seq} in elements, D contiguous; outputs likewise): pair
 * (x[2i], x[2i+1]) times freqs[b][n][i] = (cos, sin) as complex numbers in
 * fp32, rounded once to the input type.  freqs: complex64 as fp32 pairs,
 * strides {batch, seq} in pairs (batch stride 0: one table for every batch
 * entry), 16-byte aligned, even strides.  D a multiple of 8 (bf16) / 4
 * (fp32).  q_heads or k_heads may be 0.
 * Replaces: apply_rotary_emb (rldx/model/modules/action_model/ops.py:48-67)
 *   with reshape_for_broadcast (:28-45).
 */
hipError_t rldx_rope_interleaved_bf16(const void* xq, const int64_t* q_strides, void* q_out,
                                      const int64_t* q_out_strides, const void* xk, const int64_t* k_strides,
                                      void* k_out, const int64_t* k_out_strides, int64_t batch, int64_t q_heads,
                                      int64_t k_heads, int64_t seq, int64_t head_dim, const float* freqs,
                                      const int64_t* freqs_strides, hipStream_t stream);
hipError_t rldx_rope_interleaved_f32(const float* xq, const int64_t* q_strides, float* q_out,
                                     const int64_t* q_out_strides, const float* xk, const int64_t* k_strides,
                                     float* k_out, const int64_t* k_out_strides, int64_t batch, int64_t q_heads,
                                     int64_t k_heads, int64_t seq, int64_t head_dim, const float* freqs,
                                     const int64_t* freqs_strides, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* Measurement                                                              */
/* ------------------------------------------------------------------------ */

/*
 * Reads `bytes` (a multiple of 16) of device memory at `data` (16-byte
 * aligned) with 16-byte vector loads and discards them: the benchmark's
 * measured read ceiling.  `sink` holds at least rldx_read_probe_sink_words()
 * 32-bit words of device memory the kernel may write (it almost never does).
 * No counterpart in the reference: a measurement helper of this library.
 */
int64_t rldx_read_probe_sink_words(void);
hipError_t rldx_read_probe(const void* data, int64_t bytes, void* sink, int64_t sink_words, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RLDX_AMD_H_ */
