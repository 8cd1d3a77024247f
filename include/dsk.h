/*
 * dsk.h — C ABI of libdsk.so, the gfx950 (MI355X) implementation of the
 * DeepSeek-V2-Lite fused MoE layer and its MLA helper kernels.
 *
 * Every entry point:
 *   - takes raw device pointers, explicit sizes/row strides and the HIP stream
 *     as its LAST argument (a hipStream_t passed as void*; NULL = default stream);
 *   - never allocates or frees device memory: outputs and workspaces are
 *     allocated by the caller (workspace sizes come from the *_workspace_size
 *     queries);
 *   - returns 0 on success, or a nonzero DSK_ERR_* code, in which case
 *     dsk_last_error() returns a thread-local message. Launch errors are
 *     checked with hipGetLastError() after every kernel launch.
 *   - never synchronises with the host: expert offsets stay on the device and
 *     the GEMM tile schedulers read them there.
 *
 * bf16 tensors are passed as dsk_bf16 (raw 16-bit storage, round-to-nearest-even).
 * Each declaration cites the reference interface it replaces
 * (sahan974/DeepSeek-V2-Lite-CUDA, file:line).
 */
#ifndef DSK_H_
#define DSK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t dsk_bf16;

enum {
  DSK_OK = 0,
  DSK_ERR_INVALID_ARG = 1,   /* shape / size / limit violation            */
  DSK_ERR_NULL_PTR = 2,      /* a required pointer is NULL                 */
  DSK_ERR_ALIGNMENT = 3,     /* pointer or stride not 16-byte aligned      */
  DSK_ERR_LAUNCH = 4,        /* hipGetLastError() reported a launch error  */
  DSK_ERR_WORKSPACE = 5      /* workspace too small                        */
};

/* Expert weight layouts accepted by dsk_moe_fused_forward. */
#define DSK_LAYOUT_ROW_MAJOR 0
#define DSK_LAYOUT_TILED 1

/* Element types of optional operands (the attention mask). */
#define DSK_DTYPE_BF16 0
#define DSK_DTYPE_F32 1

/* Limits mirrored from the reference routing kernel (routing.cu:32-33). */
#define DSK_MAX_EXPERTS 64
#define DSK_MAX_TOP_K 6

/* Thread-local message describing the last failed call on this thread. */
const char* dsk_last_error(void);
/* ABI version of this library (bumped on any signature change). */
int dsk_abi_version(void);

/* ------------------------------------------------------------ gate logits --
 * logits[t, e] = sum_k x[t, k] * gate_weight[e, k] (+ bias[e] if bias is not
 * NULL), bf16 inputs, fp32 accumulation and output. Replaces the fp32
 * F.linear(x.float(), gate.weight.float()) of the reference orchestrator
 * (moe_fused.py:131) and of MoEGate.forward (moe.py:35-37); same products,
 * summation order fixed by this kernel (results differ from torch's only by
 * fp32 rounding). The optional bias is a per-expert routing bias added to the
 * logits (the Zipf-skewed router of BASELINE config 2 is such a bias).
 * x: bf16 [T, H] row stride ld_x; gate_weight: bf16 [E, H], row-major
 * (DSK_LAYOUT_ROW_MAJOR) or fragment-tiled like the expert weights of
 * dsk_moe_fused_forward (DSK_LAYOUT_TILED, E % 32 == 0);
 * logits: fp32 [T, E] row stride ld_logits. E <= 64, H % 16 == 0. */
int dsk_moe_gate_logits(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* gate_weight,
                        const float* bias, float* logits, int64_t ld_logits,
                        int num_tokens, int num_experts, int hidden,
                        int weight_layout, void* stream);

/* ---------------------------------------------------------------- routing --
 * Softmax over E expert logits + top-K (ties -> lower expert index, emitted in
 * descending-weight order) + per-expert counts.
 * Replaces launch_moe_routing (include/moe/routing.h:27-36, routing.cu:230-260)
 * and moe_routing_forward (routing.cu:266-301). logits: fp32 [T, E] with row
 * stride ld_logits (elements); topk_idx int32 [T,K]; topk_w fp32 [T,K];
 * expert_counts int32 [E]. E <= 64, K <= 6, K <= E. */
size_t dsk_moe_routing_workspace_size(int num_tokens, int num_experts);
int dsk_moe_routing(const float* logits, int64_t ld_logits, int32_t* topk_idx,
                    float* topk_w, int32_t* expert_counts, int num_tokens,
                    int num_experts, int top_k, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------- scan --
 * expert_offsets[0] = 0, expert_offsets[e+1] = expert_offsets[e] + counts[e];
 * expert_offsets[E] = total. Computed on the device (no host round trip).
 * Replaces launch_moe_scan (include/moe/scan.h:31-36, scan.cu:33-75) and
 * moe_scan_forward (scan.cu:86-130). */
int dsk_moe_scan(const int32_t* expert_counts, int32_t* expert_offsets,
                 int num_experts, void* stream);

/* --------------------------------------------------------------- dispatch --
 * Deterministic, stable dispatch: slot s in [offsets[e], offsets[e+1]) holds
 * the tokens routed to expert e in ascending token order.
 *   token_map[s] = t, dispatched_weights[s] = topk_w[t,k], dispatched[s,:] = x[t,:]
 * x: bf16 [T, H] with row stride ld_x (H % 8 == 0, 16-byte aligned rows).
 * dispatched may be NULL (index-only dispatch). Entries whose expert index is
 * outside [0,E) or whose slot falls outside [0, T*K) are skipped.
 * Replaces launch_moe_dispatch (include/moe/dispatch.h:44-57,
 * dispatch.cu:106-139) and moe_dispatch_forward (dispatch.cu:156-218) in
 * function, not argument for argument: this entry adds ld_x, num_experts and a
 * sized workspace (instead of the caller-zeroed expert_cursor), takes the
 * output `dispatched` after the three inputs rather than second, and returns a
 * status. The Python op `moe_dispatch` keeps the reference's argument order
 * (bindings.cu); a C caller of launch_moe_dispatch must reorder. */
size_t dsk_moe_dispatch_workspace_size(int num_tokens, int num_experts,
                                       int top_k);
int dsk_moe_dispatch(const dsk_bf16* x, int64_t ld_x, const int32_t* topk_idx,
                     const float* topk_w, const int32_t* expert_offsets,
                     dsk_bf16* dispatched, int32_t* token_map,
                     float* dispatched_weights, int num_tokens, int hidden,
                     int num_experts, int top_k, void* workspace,
                     size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- combine --
 * out[t,:] = bf16( sum over slots s with token_map[s]==t, in ascending s, of
 *                  dispatched_weights[s] * float(expert_out[s,:]) ), fp32
 * accumulation, one rounding, no float atomics. Tokens with no slot -> 0.
 * Replaces launch_moe_combine (include/moe/combine.h:41-49, combine.cu:80-93)
 * and moe_combine_forward (combine.cu:107-176) in function, not argument for
 * argument: the output `out` comes after token_map and dispatched_weights
 * rather than second, num_tokens and a workspace are added, `out` needs no
 * zero-filling by the caller, and a status is returned. The Python op
 * `moe_combine` keeps the reference's argument order (bindings.cu); a C caller
 * of launch_moe_combine must reorder. */
size_t dsk_moe_combine_workspace_size(int total_slots, int num_tokens);
int dsk_moe_combine(const dsk_bf16* expert_out, const int32_t* token_map,
                    const float* dispatched_weights, dsk_bf16* out,
                    int total_slots, int num_tokens, int hidden,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ----------------------------------------------------------------- swiglu --
 * out[s, j] = bf16( silu(in[s, j]) * in[s, I + j] ), fp32 math.
 * Replaces launch_swiglu (include/moe/swiglu.h:26-32, swiglu.cu:114-130). */
int dsk_swiglu(const dsk_bf16* in, dsk_bf16* out, int rows,
               int intermediate, void* stream);

/* ------------------------------------------------------------ grouped GEMM --
 * gemm1: out[s, :] = dispatched[s, :] @ packed_w1[e]^T for s in
 * [offsets[e], offsets[e+1]); rows outside [offsets[0], offsets[E]) are zero.
 * packed_w1: [E, N, H] (N = 2*I, gate rows then up rows); out [S, N].
 * Offsets are read on the device and clamped to [0, S].
 * Replaces launch_moe_gemm1 (include/moe/gemm1.h:25-34, gemm1.cu:84-155) and
 * moe_gemm1_forward (gemm1.cu:167-227). */
int dsk_moe_gemm1(const dsk_bf16* dispatched, const dsk_bf16* packed_w1,
                  dsk_bf16* out, const int32_t* expert_offsets,
                  int total_slots, int num_experts, int hidden, int n_out,
                  void* stream);

/* gemm1 + SwiGLU fused in the epilogue: out[s, j] = silu(g) * u with
 * g = x.W1[e][j], u = x.W1[e][I + j] (fp32 accumulators, one rounding).
 * out: [S, I]. No reference counterpart as one op: it is moe_gemm1 followed by
 * swiglu (moe_fused.py:103-106). */
int dsk_moe_gemm1_swiglu(const dsk_bf16* dispatched,
                         const dsk_bf16* packed_w1, dsk_bf16* out,
                         const int32_t* expert_offsets, int total_slots,
                         int num_experts, int hidden, int intermediate,
                         void* stream);

/* gemm2: out[s, :] = swiglu_out[s, :] @ w2[e]^T; w2: [E, H, I]; out [S, H].
 * Replaces launch_moe_gemm2 (include/moe/gemm2.h:25-34, gemm2.cu:75-124) and
 * moe_gemm2_forward (gemm2.cu:136-195). */
int dsk_moe_gemm2(const dsk_bf16* swiglu_out, const dsk_bf16* w2,
                  dsk_bf16* out, const int32_t* expert_offsets,
                  int total_slots, int num_experts, int intermediate,
                  int hidden, void* stream);

/* Dense linear out[M, N] = x[M, K] @ w[N, K]^T (bf16 in/out, fp32 accumulate),
 * x row stride ld_x, out row stride ld_out (elements, multiples of 8).
 * kv_upproj is this op with K = kv_lora_rank (512), N = 4096.
 * Replaces launch_kv_upproj (include/mla/kv_upproj.h:31-39,
 * kv_upproj.cu:77-119) and kv_upproj_forward (kv_upproj.cu:133-178). */
int dsk_linear(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* w,
               dsk_bf16* out, int64_t ld_out, int M, int K, int N,
               void* stream);
int dsk_kv_upproj(const dsk_bf16* normed_kv, int64_t ld_in,
                  const dsk_bf16* weight, dsk_bf16* out, int rows,
                  int kv_lora_rank, int out_dim, void* stream);
/* dsk_linear with the weight in either layout: DSK_LAYOUT_ROW_MAJOR is
 * dsk_linear; DSK_LAYOUT_TILED takes the weight [N, K] in the fragment-tiled
 * order of the fused layer's expert weights (N % 32 == 0), which the one-wave-
 * per-SIMD GEMM streams straight into registers when K % 128 == 0 and the
 * output rows are 16-byte aligned. Serves the same projections as dsk_linear
 * (mla.py:252-261 q_proj / kv_a_proj_with_mqa / kv_b_proj / o_proj, and the
 * kv_upproj op's GEMM) with a prepacked weight. */
int dsk_linear_ex(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* w,
                  int weight_layout, dsk_bf16* out, int64_t ld_out, int M,
                  int K, int N, void* stream);

/* ------------------------------------- RMSNorm carried by projection epilogues --
 * The latent RMSNorm of the MLA projection block (mla.py:318-346: kv_a ->
 * RMSNorm(512) -> kv_b) moved into the two projections' epilogues, so the
 * normalised latent is never written or read:
 *   dsk_linear_rowsq:    out = x @ w^T (as dsk_linear_ex, tiled w), and for
 *     every output row m the sum of squares of its bf16 outputs in columns
 *     [col_begin, col_end) (256-aligned), as one fp32 partial per 256 columns:
 *     row_sumsq[p * ld_rowsq + m], p < (col_end - col_begin) / 256.
 *   dsk_linear_rowscale: out[m, :] = r_m * (x @ w^T)[m, :] with
 *     r_m = rsqrt(sum_{p < n_parts} row_sumsq[p * ld_rowsq + m] / n_cols + eps),
 *     n_parts 1 or 2 (up to 512 normalised columns).
 * With x the raw latent (a strided view of kv_a's output) and w = kv_b's
 * weight times the norm weight per input column, dsk_linear_rowscale is
 * kv_b(RMSNorm(x)) to fp32 rounding (one bf16 rounding instead of the
 * reference's two). Tiled weights only; K % 128 == 0; 16-byte aligned output
 * rows. The reference has no counterpart: it runs rms_norm (rms_norm.cu) and
 * kv_upproj (kv_upproj.cu) as separate passes. */
int dsk_linear_rowsq(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* w_tiled,
                     dsk_bf16* out, int64_t ld_out, int M, int K, int N,
                     float* row_sumsq, int64_t ld_rowsq, int col_begin,
                     int col_end, void* stream);
int dsk_linear_rowscale(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* w_tiled,
                        dsk_bf16* out, int64_t ld_out, int M, int K, int N,
                        const float* row_sumsq, int64_t ld_rowsq, int n_parts,
                        int n_cols, float eps, void* stream);

/* --------------------------------------------------------------- rms_norm --
 * y = w * x * rsqrt(mean(x^2) + eps), fp32 math, one rounding of the output.
 * bf16 in/out with fp32 weight: replaces launch_rms_norm
 * (include/mla/rms_norm.h:26-34, rms_norm.cu:126-144) and rms_norm_forward
 * (rms_norm.cu:158-192). Row strides allow normalising a strided view (e.g. the
 * 512-wide latent inside the 576-wide kv_a output) without a copy.
 * The _f32 variant is fp32 in/out (the 1e-5 path of RMSNorm, mla.py:53-64). */
int dsk_rms_norm(const dsk_bf16* in, int64_t ld_in, const float* weight,
                 dsk_bf16* out, int64_t ld_out, int rows, int hidden,
                 float eps, void* stream);
int dsk_rms_norm_f32(const float* in, int64_t ld_in, const float* weight,
                     float* out, int64_t ld_out, int rows, int hidden,
                     float eps, void* stream);

/* ------------------------------------------------------------------- rope --
 * Interleaved-to-half rotary embedding (mla.py:176-206, rope.cu:61-95):
 *   out[k]      = x[2k]   * cos[k]      - x[2k+1] * sin[k]
 *   out[k+d/2]  = x[2k+1] * cos[k+d/2]  + x[2k]   * sin[k+d/2]
 * x viewed as [B, Hh, S, d] with element strides (sb, sh, ss), last dim
 * contiguous; cos/sin are the pre-indexed tables [B, 1, S, d] with strides
 * (cb, cs), broadcast over heads (no materialised copy). out is contiguous
 * [B, Hh, S, d]. d must be a multiple of 8 and <= 256.
 * Replaces launch_rope (include/mla/rope.h:30-38, rope.cu:101-119) and
 * rope_forward (rope.cu:139-207); dsk_rope_qk does q and k in one launch. */
int dsk_rope(const dsk_bf16* x, int64_t sb, int64_t sh, int64_t ss,
             const dsk_bf16* cos_t, const dsk_bf16* sin_t, int64_t cb,
             int64_t cs, dsk_bf16* out, int B, int Hh, int S, int d,
             void* stream);
int dsk_rope_qk(const dsk_bf16* q, int64_t qsb, int64_t qsh, int64_t qss,
                const dsk_bf16* k, int64_t ksb, int64_t ksh, int64_t kss,
                const dsk_bf16* cos_t, const dsk_bf16* sin_t, int64_t cb,
                int64_t cs, dsk_bf16* q_out, dsk_bf16* k_out, int B, int Hq,
                int Hk, int S, int d, void* stream);

/* ----------------------------------------------------- two-output linear --
 * x[M, K] @ w^T with w fragment-tiled [N/32, K/16, 64, 8], output columns
 * [0, n_split) to out0 (row pitch ld_out0) and [n_split, N) to out1 (row pitch
 * ld_out1, column n at out1[m * ld_out1 + n - n_split]); n_split % 64 == 0.
 * For M <= 64 this is one launch of the small-group kernel, which picks the
 * destination per 64-column workgroup; larger M runs as two launches over the
 * weight's two row-block ranges. Lets the absorbed-MLA decode step run q_proj
 * and kv_a_proj (mla.py:318-334) as one launch with kv_a's rows written
 * straight into the latent cache; the reference has no counterpart (it runs
 * the two projections as separate torch GEMMs and copies into its cache,
 * mla_cache.py:104-147). */
int dsk_linear_split(const dsk_bf16* x, int64_t ld_x, const dsk_bf16* w_tiled,
                     dsk_bf16* out0, int64_t ld_out0, dsk_bf16* out1, int64_t ld_out1,
                     int M, int K, int N, int n_split, void* stream);

/* ------------------------------------------------------- few-row linear --
 * out[b][m][n] = sum_k x[b][m][k] * w[b][n][k] for M <= 4 token rows, with w
 * fragment-tiled [batch, N/32, K/16, 64, 8] (K % 128 == 0, N % 32 == 0), fp32
 * sums rounded once to bf16. Entry b of x starts x_batch_stride elements
 * after entry b-1, rows ld_x apart; entry b of w starts w_batch_stride
 * elements after entry b-1 (0: one weight for every entry); outputs
 * n < n_split go to out0 (row pitch ld_out0, entry stride out0_batch_stride),
 * the others to out1 at column n - n_split (n_split = N: out1 unused).
 * Vector-ALU dot products over 8 weight
 * rows per lane group, so a one-token projection of N rows runs as N/8 lane
 * groups instead of N/32 workgroups: the q/kv_a, per-head and o projections of
 * a one-token absorbed-MLA decode step. The reference has no counterpart (it
 * runs its projections as torch GEMMs and has no decode step). */
int dsk_linear_rows(const dsk_bf16* x, int64_t ld_x, int64_t x_batch_stride,
                    const dsk_bf16* w_tiled, int64_t w_batch_stride, dsk_bf16* out0,
                    int64_t ld_out0, int64_t out0_batch_stride, dsk_bf16* out1,
                    int64_t ld_out1, int64_t out1_batch_stride, int n_split, int batch,
                    int M, int K, int N, void* stream);

/* --------------------------------------------------------- batched linear --
 * out[b] = x[b] @ w[b]^T for b < batch, with M <= 64 rows per entry (the
 * weight-streaming small-group kernel; one launch for all entries). Entry b of
 * x starts x_batch_stride elements after entry b-1 and has rows ld_x apart;
 * out likewise with out_batch_stride and ld_out; w is fragment-tiled
 * [batch, N/32, K/16, 64, 8]. Runs the per-head products of absorbed MLA
 * decode (q_nope[h] -> q_abs[h] and o_lat[h] -> o[h], 16 entries) on strided
 * views, replacing a transpose copy and a torch batched product each; the
 * reference has no counterpart (it up-projects K and V instead). */
int dsk_linear_batched(const dsk_bf16* x, int64_t ld_x, int64_t x_batch_stride,
                       const dsk_bf16* w_tiled, dsk_bf16* out, int64_t ld_out,
                       int64_t out_batch_stride, int batch, int M, int K, int N,
                       void* stream);

/* ------------------------------------------------------ attention softmax --
 * In place over bf16 attention scores [rows, kv_len] (row stride ld): the
 * eager sequence of DeepSeekMLA.forward (mla.py:366-381) in one pass,
 *   p = bf16(softmax_fp32(bf16(score * scale) + causal_mask)),
 * with key j of query i masked when causal and j > i + kv_len - q_len (the row's
 * query index is row % q_len). Masked probabilities are written as 0 and their
 * scores are not read. Any kv_len >= 1: rows of up to 4096 keys are held in
 * registers, longer ones take two passes. ld % 8 == 0 and ld >= kv_len rounded
 * up to 8; keys kv_len.. up to that multiple of 8 are written as 0 (a 16-byte
 * padded score buffer then multiplies zero-padded V rows exactly). A fully
 * masked row gives NaN, as torch's softmax does. The reference has no kernel for
 * this: it replaces four torch passes over the scores (scale, mask, fp32
 * softmax, cast) of the decoder layer's attention core. */
int dsk_attn_softmax(dsk_bf16* scores, int64_t ld, int64_t rows, int kv_len,
                     int q_len, float scale, int causal, void* stream);

/* dsk_attn_softmax with the additive attention_mask of DeepSeekMLA.forward
 * (mla.py:295-315,374: `attn_weights + attention_mask`, [bsz, 1, q_len, kv_len],
 * -inf where masked) in place of (or besides) the causal mask. Rows are
 * (batch, head, query) with the query fastest and `heads` heads per batch
 * entry; the mask element of key j is at
 *   mask[b * mask_sb + h * mask_sh + i * mask_sq + j]   (element strides),
 * so a head stride of 0 broadcasts one mask over the heads. mask_dtype
 * DSK_DTYPE_BF16 adds in bf16 (the sum rounded, as a bf16 + bf16 tensor add),
 * DSK_DTYPE_F32 in fp32 (as torch promotes bf16 + fp32). */
int dsk_attn_softmax_masked(dsk_bf16* scores, int64_t ld, int64_t rows, int kv_len,
                            int q_len, int heads, float scale, int causal,
                            const void* mask, int mask_dtype, int64_t mask_sb,
                            int64_t mask_sh, int64_t mask_sq, void* stream);

/* --------------------------------------------------- attention operand pack --
 * Packs the operands of the full-sequence attention of DeepSeekMLA.forward
 * (mla.py:354-366: query_states and key_states assembled from the nope and
 * rotated rope parts, key_states.transpose(2, 3), value_states) in one pass:
 *   q_out[b, h, s, 0:128]   = q[t, h*192 + 0:128]           (t = b * seq + s)
 *   q_out[b, h, s, 128:192] = rope(q[t, h*192 + 128:192])
 *   k_t[b, h, 0:128, s]     = kv[t, h*256 + 0:128]
 *   k_t[b, h, 128:192, s]   = rope(k_pe[t, 0:64])          (every head)
 *   v_out[b, h, s, :]       = kv[t, h*256 + 128:256]
 * q, kv and k_pe are token rows (row strides ld_q, ld_kv, ld_kpe: the q_proj,
 * kv_b_proj and kv_a_proj outputs as they leave the projections); rope is that
 * of dsk_rope with the bf16 tables cos/sin [seq, 64] (row stride ld_cs) for
 * positions 0..seq-1. Outputs are contiguous. Head dims nope 128, rope 64,
 * v 128; seq % 8 == 0. The reference has no kernel for this: it replaces the
 * reference's head-major assembly copies and the transposed read of K. */
int dsk_mla_attn_pack(const dsk_bf16* q, int64_t ld_q, const dsk_bf16* kv,
                      int64_t ld_kv, const dsk_bf16* k_pe, int64_t ld_kpe,
                      const dsk_bf16* cos_t, const dsk_bf16* sin_t, int64_t ld_cs,
                      dsk_bf16* q_out, dsk_bf16* k_t, dsk_bf16* v_out, int batch,
                      int seq, int heads, int nope, int rope, int v_dim, void* stream);

/* dsk_mla_attn_pack for position_ids and any sequence length (mla.py:295-352:
 * apply_rotary_pos_emb indexes the tables by position_ids [bsz, seq]): the
 * tables of batch entry b start at cos_t + b * cs_batch_stride (0: one table
 * for every entry, row s for position s), and K^T rows and V are padded to
 * seq_pad positions (seq <= seq_pad, seq_pad % 8 == 0, seq_pad - seq < 8):
 *   k_t [b, h, 192, seq_pad], v_out [b, h, seq_pad, 128], q_out [b, h, seq, 192],
 * the padding columns of K^T and rows of V written as 0. With seq % 8 != 0 the
 * products Q.K^T and P.V then run on 16-byte aligned rows and the padding
 * adds exact zeros. */
int dsk_mla_attn_pack_ex(const dsk_bf16* q, int64_t ld_q, const dsk_bf16* kv,
                         int64_t ld_kv, const dsk_bf16* k_pe, int64_t ld_kpe,
                         const dsk_bf16* cos_t, const dsk_bf16* sin_t, int64_t ld_cs,
                         int64_t cs_batch_stride, dsk_bf16* q_out, dsk_bf16* k_t,
                         dsk_bf16* v_out, int batch, int seq, int seq_pad, int heads,
                         int nope, int rope, int v_dim, void* stream);

/* ----------------------------------------------- latent-cache decode attention --
 * Absorbed multi-head latent attention of new tokens over the latent KV cache
 * of LatentKVCache (src/kernels/mla_cache.py:29-219), which holds per token the
 * raw compressed latent x (pre-RMSNorm, 512) and the raw shared RoPE key
 * (pre-RoPE, 64). Query token t = b * q_len + i sits at cache position
 * kv_len - q_len + i; for each head h < 16 and key j <= that position:
 *   s_j     = scale * (q_abs[t,h] . (r_j x_j) + rope(q_pe[t,h]) . rope(k_pe_j))
 *   o[t,h]  = sum_j softmax(s)_j r_j x_j        (fp32, stored as bf16)
 * with r_j = rsqrt(mean(x_j^2) + eps) and rope as in dsk_rope (angles of the
 * row's position in cos/sin [positions, 64], which must cover kv_len rows).
 * k_rope holds rope(k_pe_j), the rotated keys in dsk_rope's output layout:
 * rows j < rope_len are read from it; rows rope_len <= j < kv_len are rotated
 * here from k_pe and written to it (each key is rotated once, by the call
 * after its append). q_abs[t,h] (512) is (W_UK[h] * norm_weight)^T
 * q_nope[t,h]; the caller applies (W_UV[h] * norm_weight) and o_proj to o.
 * Element strides: q_abs at t * qa_tok + h * qa_head, q_pe (raw, pre-RoPE) at
 * t * qp_tok + h * qp_head, cache token j of sequence b at b * ld_batch +
 * j * ld_tok in latent, k_pe and k_rope (the three may interleave in one row,
 * LatentKVCache's 640-wide rows), o at t * o_tok + h * o_head. This is the
 * attention of DeepSeekMLA.forward (mla.py:318-384) over the cached prefix
 * plus the new tokens; the reference has no kernel for it (it recomputes K and
 * V for the whole sequence). */
size_t dsk_mla_decode_workspace_size(int batch, int q_len, int kv_len);
int dsk_mla_decode_attention(const dsk_bf16* q_abs, int64_t qa_tok,
                             int64_t qa_head, const dsk_bf16* q_pe,
                             int64_t qp_tok, int64_t qp_head,
                             const dsk_bf16* latent, const dsk_bf16* k_pe,
                             dsk_bf16* k_rope, int rope_len,
                             int64_t ld_tok, int64_t ld_batch,
                             const dsk_bf16* cos_tab, const dsk_bf16* sin_tab,
                             float eps, float scale, int batch, int q_len,
                             int kv_len, dsk_bf16* o_latent, int64_t o_tok,
                             int64_t o_head, void* workspace, size_t bytes,
                             void* stream);

/* ------------------------------------------------------- fused MoE layer --
 * The whole DeepSeekMoE forward (moe.py:77-109) on the device:
 *   route -> stable permutation -> grouped GEMM1+SwiGLU -> grouped GEMM2 ->
 *   deterministic combine (+ shared expert), with no host synchronisation.
 * logits: fp32 [T, E] (gate GEMM output, as moe_fused.py:131 computes it);
 * x: bf16 [T, H]; w1: bf16 [G, 2I, H] and w2: bf16 [G, H, I] where
 * G = E + n_shared_groups, stored as selected by weight_layout:
 *   DSK_LAYOUT_ROW_MAJOR  nn.Linear order, each group [N, K] K-contiguous
 *                         (the reference prepack, expert_prepack.py:105-130);
 *   DSK_LAYOUT_TILED      MFMA-fragment order: a group's [N, K] matrix is cut
 *                         into 32-row x 16-column fragments, fragment (rb, ks)
 *                         at element (rb * K/16 + ks) * 512, and inside it
 *                         element (r, k) at ((k / 8) * 32 + r) * 8 + k % 8.
 *                         Each 1 KB fragment is then one coalesced 64-lane
 *                         load (decode streams the weights at full HBM rate).
 * Groups E.. are the shared expert split into
 * n_shared_groups slices of width I (every token routes to them with weight
 * 1.0). out: bf16 [T, H]. The replaced reference caller is
 * _route_dispatch_combine (moe_fused.py:118-154), which omits shared experts.
 * Optional debug outputs (may be NULL): topk_idx [T,K], topk_w [T,K],
 * expert_offsets [E+1]. Optional instrumentation (may be NULL): stage_events
 * points to 5 hipEvent_t recorded on `stream` before routing, after the
 * permutation, after GEMM1+SwiGLU, after GEMM2 and after the combine. */
size_t dsk_moe_fused_workspace_size(int num_tokens, int num_experts,
                                    int top_k, int n_shared_groups,
                                    int hidden, int intermediate);
int dsk_moe_fused_forward(const float* logits, const dsk_bf16* x,
                          const dsk_bf16* w1, const dsk_bf16* w2,
                          dsk_bf16* out, int num_tokens, int num_experts,
                          int top_k, int n_shared_groups, int hidden,
                          int intermediate, int weight_layout, int32_t* topk_idx_out,
                          float* topk_w_out, int32_t* expert_offsets_out,
                          void* workspace, size_t workspace_bytes,
                          void* const* stage_events, void* stream);

/* The same layer from the hidden states, gate included: the router logits
 * x @ gate_weight^T (+ gate_bias) are computed in fp32 from bf16 inputs (as
 * dsk_moe_gate_logits), as partial sums over K slices that the route kernel
 * adds in a fixed order, then the layer runs as dsk_moe_fused_forward.
 * Replaces the whole FusedMoELayer.forward of the reference
 * (moe_fused.py:197-216) including its fp32 gate linear (moe_fused.py:131).
 * gate_weight: bf16 [E, H], in the layout weight_layout names for w1/w2
 * (tiled needs E % 32 == 0); gate_bias: optional fp32 [E]. stage_events[0]
 * is recorded before the gate. */
size_t dsk_moe_layer_workspace_size(int num_tokens, int num_experts,
                                    int top_k, int n_shared_groups,
                                    int hidden, int intermediate);
int dsk_moe_layer_forward(const dsk_bf16* x, const dsk_bf16* gate_weight,
                          const float* gate_bias, const dsk_bf16* w1,
                          const dsk_bf16* w2, dsk_bf16* out, int num_tokens,
                          int num_experts, int top_k, int n_shared_groups,
                          int hidden, int intermediate, int weight_layout,
                          int32_t* topk_idx_out, float* topk_w_out,
                          int32_t* expert_offsets_out, void* workspace,
                          size_t workspace_bytes, void* const* stage_events,
                          void* stream);

/* ------------------------------------------ allocation-free fused MoE layer --
 * dsk_moe_layer_forward without the workspace argument: the scratch it needs
 * (routing planes, permutation, the [S, I] and [S, H] intermediates) lives in
 * a static per-GPU device array of DSK_NOALLOC_SCRATCH_BYTES inside this
 * library, so the call itself allocates nothing. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Limit: layers whose dsk_moe_layer_workspace_size exceeds
 * DSK_NOALLOC_SCRATCH_BYTES are rejected with DSK_ERR_WORKSPACE (at the
 * DeepSeek-V2-Lite shapes E=64, K=6, 2 shared groups, H=2048, I=1408 that
 * admits T <= 128, the decode sizes). The stream must belong to the current
 * device. The first call on a device must be eager (not under stream capture):
 * it resolves the array's device address and creates the device's in-flight
 * event; later calls may be captured into a HIP graph. Every call on one GPU
 * shares that GPU's array (no state is carried from one call to the next), so
 * calls that overlap on one GPU would race: an eager call on another stream
 * while the previous eager call is still running is refused with
 * DSK_ERR_INVALID_ARG; captured calls are not tracked, and replays of graphs
 * holding them must be serialised by the caller. Arguments otherwise as for
 * dsk_moe_layer_forward. */
#define DSK_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int dsk_moe_layer_forward_noalloc(const dsk_bf16* x, const dsk_bf16* gate_weight,
                                  const float* gate_bias, const dsk_bf16* w1,
                                  const dsk_bf16* w2, dsk_bf16* out, int num_tokens,
                                  int num_experts, int top_k, int n_shared_groups,
                                  int hidden, int intermediate, int weight_layout,
                                  int32_t* topk_idx_out, float* topk_w_out,
                                  int32_t* expert_offsets_out,
                                  void* const* stage_events, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSK_H_ */
