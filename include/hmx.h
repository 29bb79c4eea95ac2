/*
 * hmx.h — C ABI of libhmx.so, the MI355X (gfx950) linear-recurrent mixer kernels.
 *
 * Conventions shared by every entry point
 *  - All pointers are device pointers unless stated otherwise; sizes and
 *    strides are in ELEMENTS of the tensor they describe.
 *  - Optional tensors are passed as NULL.
 *  - `stream` is a hipStream_t (NULL = default stream).  Work is enqueued only:
 *    the library never allocates, frees or synchronises, and keeps no global
 *    mutable state, so calls are re-entrant and graph-capturable.
 *  - Return value: HMX_OK, or an HMX_E* code with a message available from
 *    hmx_last_error() (thread-local).
 *  - Dtype codes: HMX_F32, HMX_BF16, HMX_F16; index tensors are int32.
 *
 * The reference has no native code: each entry point replaces one Python op
 * (and the Triton kernels under it) of awslabs/hybrid-model-factory, cited
 * below as path:line relative to the reference repository root.
 */
#ifndef HMX_H_
#define HMX_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HMX_ABI_VERSION 13  /* 2: optional hmx_gated_norm output epilogue in the GDN ops;
                              3: q/k/v token strides in the GDN and GKA ops; slot-indexed
                              state pools and has_initial_state in the GDN, GKA and SSD
                              prefills;
                              4: grouped x heads (HX) and C groups (GC) in the SSD ops;
                              5: nblock_total in hmx_gka_chunk_fwd and its workspace size;
                              6: host segment planner hmx_plan_segments(_bounds);
                              7: gates from raw projections (hmx_gate_proj) in the GDN and
                                 GKA prefill / decode entry points;
                              8: N in hmx_gdn_train_bwd_workspace_bytes (the exact-run
                                 buffers are sized by the runs beyond each sequence's
                                 first);
                              9: hmx_gdn_chunk_workspace_bytes adds the per-walk fp16
                                 range flags (any bf16 magnitude is supported);
                              10: the same in hmx_ssd_chunk_workspace_bytes (nonzero for
                                  one segment per sequence too);
                              11: hmx_causal_conv1d_update_spec (speculative multi-token
                                  conv update);
                              12: hmx_causal_conv1d_fwd_blocks and
                                  hmx_causal_conv1d_update_blocks (prefix-cache block
                                  arguments);
                              13: hmx_ssd_chunk_bwd (the SSD scan's backward) */

enum hmx_status {
  HMX_OK = 0,
  HMX_EINVAL = 1,       /* bad argument: maps to ValueError on the Python side */
  HMX_EUNSUPPORTED = 2, /* unsupported shape/dtype: maps to NotImplementedError */
  HMX_EHIP = 3          /* HIP launch/runtime error: maps to RuntimeError */
};

enum hmx_dtype { HMX_F32 = 0, HMX_BF16 = 1, HMX_F16 = 2 };

int hmx_abi_version(void);

/* Optional output epilogue of the mixer ops: the gated RMSNorm of
 * hmx_rms_norm_gated (norm before gate) applied to every output row (one head's V
 * values) before it is stored, so out = o / sqrt(mean(o^2) + eps) * weight *
 * silu(gate), with o as the op would have returned it.  It fuses the layers'
 * o_norm(core_attn_out, z) (vllm-inference/src/primed_vllm/primed_gdn_layer.py:626,
 * primed_gka_layer.py:949) into the op; no reference counterpart as one call. */
typedef struct hmx_gated_norm {
  const void* gate;           /* [tokens, H, V] in the op's q/k/v dtype, or NULL */
  int64_t gate_token_stride;  /* elements between tokens (multiple of 8) */
  int64_t gate_head_stride;   /* elements between heads (multiple of 8); V contiguous */
  const void* weight;         /* [V] */
  int32_t weight_dtype;
  float eps;
} hmx_gated_norm;
const char* hmx_last_error(void);

/*
 * Gates computed from the layer's raw projections inside the mixer kernels' loads,
 * in place of a separate gating launch and its [tokens, H] gate tensors.  It fuses
 * vllm-inference/src/primed_vllm/gdn/ops/fused_gdn_gating.py:79-125 (with the
 * layer's beta *= 2 for negative eigenvalues, primed_gdn_layer.py:798-802) and
 * primed_gka_layer.py:224-358 (with the layer's alpha post-processing,
 * primed_gka_layer.py:1138-1153) into hmx_gdn_chunk_fwd, hmx_gdn_recurrent_fwd,
 * hmx_gka_chunk_fwd and hmx_gka_decode_fwd.  Per token t (the op's flattened
 * token index) and head h, each gate is rounded to in_dtype as the reference
 * stores it before the kernel reads it:
 *   g     = -exp(A_log[h]) * softplus(a[t,h] + dt_bias[h])   (softplus with
 *           softplus_beta / softplus_threshold as the reference); 0 when A_log is
 *           NULL (the GKA layer without a forgetting gate)
 *   beta  = sigmoid(b[t,h]), then * beta_scale (rounded again); none when b is NULL
 *   alpha = sigmoid(alpha_in[t,h]), then + alpha_add (rounded again), or 0 when
 *           alpha_zero (GKA only)
 *   gk    = g when gk_from_g, else none (GKA only)
 * An op given gates ignores its g / gk / beta / alpha pointers.
 */
typedef struct hmx_gate_proj {
  const void* A_log; int32_t A_log_dtype;            /* [H] or NULL */
  const void* dt_bias; int32_t dt_bias_dtype;        /* [H] */
  const void* a; int64_t a_token_stride, a_head_stride;            /* [tokens, H] */
  const void* b; int64_t b_token_stride, b_head_stride;            /* [tokens, H] or NULL */
  const void* alpha_in; int64_t alpha_token_stride, alpha_head_stride;  /* GKA [tokens, H] */
  int32_t in_dtype;                                  /* dtype of a, b, alpha_in */
  float softplus_beta, softplus_threshold;           /* 1, 20 in the layers */
  float beta_scale;                                  /* 1, or 2 for negative eigenvalues */
  float alpha_add;                                   /* GKA: 0.5, or 0 */
  int32_t alpha_zero;                                /* GKA: alpha = 0 (num_iter == 0) */
  int32_t gk_from_g;                                 /* GKA: gk = g (use_forgetting_gate_kk) */
} hmx_gate_proj;


/*
 * GDN gating: g = -exp(A_log) * softplus(a + dt_bias), beta_out = sigmoid(b).
 * softplus(x) = log(1 + exp(sp_beta*x)) / sp_beta, or x when sp_beta*x > threshold.
 * a, b: [num_tokens, num_heads] with arbitrary strides (the split of a fused
 * projection); A_log, dt_bias: [num_heads]; g, beta_out: contiguous
 * [num_tokens, num_heads] in out_dtype.
 * Replaces: fused_gdn_gating
 *   vllm-inference/src/primed_vllm/gdn/ops/fused_gdn_gating.py:79-125 (kernel :10-76).
 */
int hmx_gdn_gating(const void* A_log, int32_t A_log_dtype,
                   const void* a, int64_t a_stride0, int64_t a_stride1,
                   const void* b, int64_t b_stride0, int64_t b_stride1,
                   int32_t ab_dtype,
                   const void* dt_bias, int32_t dt_bias_dtype,
                   void* g, void* beta_out, int32_t out_dtype,
                   int64_t num_tokens, int32_t num_heads,
                   float sp_beta, float threshold, void* stream);

/*
 * GDN fused recurrent (decode) forward, GQA-native, slot-indexed state pool.
 *  q [B*T, H, K]; k [B*T, HKV, K]; v [B*T, HKV, V] (qkv_dtype): rows *_token_stride
 *    elements apart (multiples of 4; 16-byte aligned bases), heads contiguous in a
 *    row - the column slices of a fused projection pass without a copy
 *  g [B*T, H] (g_dtype); beta [B*T, H] or [B*T, H, V] when beta_headwise
 *  o [B*T, H, V] (qkv_dtype)
 *  h0, ht: state tensors of state_dtype, rows of [H, K, V] with row strides
 *    h0_row_stride / ht_row_stride (elements).  h0 may be NULL (zero state).
 *  Sequences: cu_seqlens [N+1] (varlen, B == 1) or N = B sequences of T tokens.
 *  Initial state of sequence n: row ssm_state_indices[n*idx_stride + c] with
 *    c = num_accepted_tokens[n]-1 (or 0), or row bos_n without indices.
 *  Final state: row ssm_state_indices[n*idx_stride] when inplace, else row bos_n
 *    (fused_recurrent_gqa.py:137-139 stores the non-inplace state at the sequence's bos).
 *  Zero-length sequences and negative slot indices are skipped.
 *  Supported: K in {64,128,256}; V a multiple of 32, <= 256.
 * Replaces: fused_recurrent_gated_delta_rule_gqa
 *   vllm-inference/src/primed_vllm/gdn/ops/fused_recurrent_gqa.py:227-277
 *   (wrapper :157-224, kernel :25-154).
 */
int hmx_gdn_recurrent_fwd(const void* q, int64_t q_token_stride, const void* k,
                          int64_t k_token_stride, const void* v, int64_t v_token_stride,
                          int32_t qkv_dtype,
                          const void* g, int32_t g_dtype,
                          const void* beta, int32_t beta_dtype, int32_t beta_headwise,
                          void* o,
                          const void* h0, int64_t h0_row_stride,
                          void* ht, int64_t ht_row_stride, int32_t state_dtype,
                          const int32_t* cu_seqlens,
                          const int32_t* ssm_state_indices, int64_t idx_stride,
                          const int32_t* num_accepted_tokens,
                          int64_t B, int64_t T, int64_t N,
                          int32_t H, int32_t HKV, int32_t K, int32_t V,
                          float scale, int32_t use_qk_l2norm, int32_t inplace_final_state,
                          const hmx_gated_norm* o_norm, const hmx_gate_proj* gates, void* stream);

/*
 * Segment planner (host code: host pointers, no GPU access, no allocation the
 * caller sees).  Builds the seg_table of hmx_gdn_chunk_fwd (op HMX_PLAN_GDN),
 * hmx_gka_chunk_fwd (HMX_PLAN_GKA) and hmx_ssd_chunk_fwd (HMX_PLAN_SSD) from the
 * sequence bounds, so a C/C++ caller drives the prefills without Python.  It
 * replaces the reference's per-call varlen bookkeeping, the cu_seqlens ->
 * chunk indices/offsets of vLLM's fla prepare_chunk_indices/_offsets
 * (vllm-inference/src/primed_vllm/gka/ops/chebyshev_prefill_gqa.py:133-134, :299;
 * inside each fla op that gdn/ops/chunk_gqa.py:63-81 passes cu_seqlens to); here
 * it runs on host offsets (vLLM's query_start_loc_cpu), so the prefill needs no
 * device-to-host copy.
 *  cu_seqlens: host int64 [nseq+1] offsets over the B*T tokens (non-decreasing
 *    from 0, ending <= B*T), or NULL for B sequences of T tokens (nseq == B).
 *  cu_count: compute units of the device the prefill runs on
 *    (hipDeviceAttributeMultiprocessorCount); the segment counts fill
 *    2 * cu_count / H workgroup slots (one or two waves).
 *  segment_chunks: > 0 cuts every sequence into equal segments of at most that
 *    many chunks (32 tokens for GDN, 64 for GKA and SSD) instead.
 *  table: host int32 [max_rows][8] rows (n, bos, eos, c_start, c_end, seg_idx,
 *    first_seg, nseg), or NULL to query *nrows only.
 *  nrows: rows of the plan (every sequence, even empty, has >= 1).
 *  nblock_total (may be NULL): the chunks of all sequences (hmx_gka_chunk_fwd's
 *    nblock_total for HMX_PLAN_GKA).
 * HMX_EINVAL for malformed offsets or a table with fewer than *nrows rows.
 */
enum hmx_plan_op { HMX_PLAN_GDN = 0, HMX_PLAN_GKA = 1, HMX_PLAN_SSD = 2 };
int hmx_plan_segments(int32_t op, const int64_t* cu_seqlens, int32_t nseq, int32_t B, int64_t T,
                      int32_t H, int32_t cu_count, int32_t segment_chunks, int32_t* table,
                      int32_t max_rows, int32_t* nrows, int32_t* nblock_total);
/* The same from explicit (bos, eos) token ranges: host int64 [nseq][2], each
 * within [0, tokens] (sequences need not be adjacent: the SSD scan's seq_idx
 * runs). */
int hmx_plan_segments_bounds(int32_t op, const int64_t* bos_eos, int32_t nseq, int64_t tokens,
                             int32_t H, int32_t cu_count, int32_t segment_chunks, int32_t* table,
                             int32_t max_rows, int32_t* nrows, int32_t* nblock_total);

/*
 * GDN chunked prefill forward, GQA-native, varlen via a segment table (the kernel
 * walks 32-token chunks; the result is the chunked recurrence at any chunk size).
 *  q [T_total, H, 128]; k, v [T_total, HKV, 128] (bf16; T_total = B*T): rows
 *    *_token_stride elements apart (multiples of 8; 16-byte aligned bases), heads
 *    contiguous in a row - the column slices of a fused projection pass as views
 *  g, beta [T_total, H] (f32/bf16/f16); o [T_total, H, 128] (bf16, contiguous)
 *  h0 / ht: the initial / end states, each a base of [H, 128, 128] slots
 *    state_slot_stride elements apart in state_dtype (f32 or bf16), or NULL (zero
 *    start / no end state).  Sequence n uses slot state_indices[n] (n when
 *    state_indices is NULL); a negative slot starts from zero and writes no end
 *    state; has_initial_state[n] == 0 (when not NULL) starts from zero.  With
 *    state_indices h0 and ht may be the same pool (read and written in place:
 *    the end states of sequences split into segments are staged in the workspace
 *    and copied into their slots by a last launch).
 *  seg_table: int32 [nseg_total][8] rows (n, bos, eos, c_start, c_end, seg_idx,
 *    first_seg, nseg) - the chunks [c_start, c_end) of sequence n (tokens
 *    [bos, eos)) form segment seg_idx of nseg; rows sorted by sequence, every
 *    sequence (even empty) has >= 1 segment.  Built by hmx_plan_segments.
 *  max_warm_chunks / decay_threshold: a segment's start state is recomputed
 *    from zero over at most max_warm_chunks preceding chunks when the dropped
 *    history is bounded below exp(-decay_threshold); otherwise the exact
 *    segment scan runs.
 *  workspace: device scratch of hmx_gdn_chunk_workspace_bytes(...) bytes.
 *  Any finite bf16 v and f32/bf16 initial state is supported: a walk whose fp16
 *  operands would leave fp16's range is detected and walked again with every
 *  operand scaled by a power of two (exact), with keys of norm <= 1 (in-kernel L2
 *  normalisation guarantees it), beta in [0, 2] and g <= 0.
 *  o_norm: NULL, or the output gated RMSNorm applied in the op's epilogue.
 * Replaces: chunk_gated_delta_rule_gqa
 *   vllm-inference/src/primed_vllm/gdn/ops/chunk_gqa.py:15-83 (and its kernels
 *   wy_fast_gqa.py:19-112, chunk_delta_h_gqa.py:29-215, chunk_o_gqa.py:30-114).
 */
int hmx_gdn_chunk_fwd(const void* q, int64_t q_token_stride, const void* k,
                      int64_t k_token_stride, const void* v, int64_t v_token_stride,
                      int32_t qkv_dtype, const void* g, int32_t g_dtype, const void* beta,
                      int32_t beta_dtype, void* o, const void* h0, void* ht,
                      int64_t state_slot_stride, int32_t state_dtype,
                      const int32_t* state_indices, const uint8_t* has_initial_state,
                      const int32_t* seg_table, int32_t nseg_total, int32_t N,
                      int32_t H, int32_t HKV, int32_t K, int32_t V, float scale,
                      int32_t use_qk_l2norm, int32_t max_warm_chunks, float decay_threshold,
                      void* workspace, size_t workspace_bytes, const hmx_gated_norm* o_norm,
                      const hmx_gate_proj* gates, void* stream);

/*
 * hmx_gdn_chunk_fwd without a workspace argument: the workspace is a static device
 * array of HMX_GDN_CHUNK_SCRATCH_BYTES per device, and the call allocates nothing
 * (no hipMalloc / hipFree, no allocating library routine).  Arguments and results
 * as hmx_gdn_chunk_fwd.  Returns HMX_EINVAL when the segment table needs more
 * workspace than the array holds (hmx_gdn_chunk_workspace_bytes > the limit).
 * The array's address is looked up once per device, on the first call with that
 * device current; later calls on the device reuse it.  The array has a code object
 * of its own, loaded by that first lookup: a process reserves it only on devices
 * where it calls this entry point.  The stream must belong to
 * the current device.  Calls that overlap on one device share the array and race:
 * serialise them (one stream, or events).
 * No counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid it).
 */
#define HMX_GDN_CHUNK_SCRATCH_BYTES (64u << 20)
int hmx_gdn_chunk_fwd_noalloc(const void* q, int64_t q_token_stride, const void* k,
                              int64_t k_token_stride, const void* v, int64_t v_token_stride,
                              int32_t qkv_dtype, const void* g, int32_t g_dtype,
                              const void* beta, int32_t beta_dtype, void* o, const void* h0,
                              void* ht, int64_t state_slot_stride, int32_t state_dtype,
                              const int32_t* state_indices, const uint8_t* has_initial_state,
                              const int32_t* seg_table, int32_t nseg_total, int32_t N,
                              int32_t H, int32_t HKV, int32_t K, int32_t V, float scale,
                              int32_t use_qk_l2norm, int32_t max_warm_chunks,
                              float decay_threshold, const hmx_gated_norm* o_norm, const hmx_gate_proj* gates, void* stream);

/* Workspace bytes hmx_gdn_chunk_fwd needs for a given segment table (host-only
 * arithmetic); pooled != 0 when the call passes state_indices.  Companion of
 * hmx_gdn_chunk_fwd; no reference counterpart (the reference allocates its
 * intermediates inside the op, chunk_gqa.py:63-81). */
size_t hmx_gdn_chunk_workspace_bytes(int32_t nseg_total, int32_t N, int32_t H, int32_t pooled);

/*
 * Training forward of the chunked gated delta rule: hmx_gdn_chunk_fwd with H query
 * and key/value heads (k, v already expanded, one token stride), fp32 h0 / ht
 * [N][H][128][128] (either may be null), no state pool, and in addition the state
 * entering every 32-token block written to block_states, fp16 [nblock_total][H]
 * [128][128], block b = cu_blocks[n] + (block index within sequence n); cu_blocks
 * is int32 [N+1].  The backward reads these states.
 * Replaces: the state recomputation of fla's chunk_gated_delta_rule backward
 *   (chunk_gated_delta_rule_fwd_h), called by the training layer at
 *   training/src/hmf/model/hybrid_zoo/layers/gated_deltanet/gdn.py:462-476.
 */
int hmx_gdn_train_fwd(const void* q, int64_t q_token_stride, const void* k, const void* v,
                      int64_t kv_token_stride, const void* g, int32_t g_dtype, const void* beta,
                      int32_t beta_dtype, void* o, const float* h0, float* ht,
                      const int32_t* seg_table, int32_t nseg_total, int32_t N, int32_t H,
                      float scale, int32_t use_qk_l2norm, int32_t max_warm_chunks,
                      float decay_threshold, void* workspace, size_t workspace_bytes,
                      void* block_states, const int32_t* cu_blocks, void* stream);

/*
 * Backward of the chunked gated delta rule for dout [tokens][H][128] bf16 (token
 * stride dout_token_stride) and, optionally, dht (the gradient of the final states,
 * fp32 [N][H][128][128]).  block_states: hmx_gdn_train_fwd's; block_table int32
 * [nblock_total][4] = (first token, tokens (1-32), sequence, block index within
 * the sequence); cu_blocks [N+1].  chain_segments int32 [nchain_segments][3] =
 * (sequence, first block, end block) cuts every sequence's blocks into runs that
 * one workgroup each walks backward.  Required order (not checked here; the Python
 * wrapper checks it on the host): rows grouped by ascending sequence 0..N-1, every
 * sequence with at least one row (one empty row (n, b, b) for a sequence without
 * tokens), and each sequence's rows tiling its blocks [cu_blocks[n], cu_blocks[n+1])
 * in ascending order with no gap or overlap; another order gives wrong gradients
 * for heads on the exact combine, with no error.  A run that ends before its sequence
 * starts from zero after a warm-up of up to max_warm_blocks following blocks whose
 * gates bring the dropped history under e^-decay_threshold; a head with a run that
 * finds no such warm-up takes every run's exact start from a combine over the runs
 * (each run's chain from zero and its transposed transition product).  Writes dq,
 * dk, dv [tokens][H][128] bf16 (rows
 * of the blocks' tokens only), dg and dbeta [tokens][H] fp32, and dh0 (the
 * gradient of the initial states, fp32 [N][H][128][128]) when not null.
 * workspace: hmx_gdn_train_bwd_workspace_bytes(nblock_total, nchain_segments, N, H) bytes.
 * Replaces: the backward of fla's chunk_gated_delta_rule (un-vendored; the training
 *   layer's call at training/src/hmf/model/hybrid_zoo/layers/gated_deltanet/gdn.py:
 *   462-476, whose torch fallback is the recurrence of
 *   .../qwen3_5_moe_hmf/modeling_qwen3_5_moe_hmf.py:330-407 under autograd).
 */
int hmx_gdn_train_bwd(const void* q, int64_t q_token_stride, const void* k, const void* v,
                      int64_t kv_token_stride, const void* g, int32_t g_dtype, const void* beta,
                      int32_t beta_dtype, const void* dout, int64_t dout_token_stride,
                      const float* dht, const void* block_states, const int32_t* block_table,
                      const int32_t* cu_blocks, int32_t nblock_total, int32_t N,
                      const int32_t* chain_segments, int32_t nchain_segments,
                      int32_t max_warm_blocks, float decay_threshold, int32_t H, float scale,
                      int32_t use_qk_l2norm, void* dq, void* dk, void* dv, float* dg,
                      float* dbeta, float* dh0, void* workspace, size_t workspace_bytes,
                      void* stream);
size_t hmx_gdn_train_bwd_workspace_bytes(int32_t nblock_total, int32_t nchain_segments, int32_t N,
                                         int32_t H);

/*
 * GKA gating: g = -exp(A_log) * softplus(a + dt_bias), alpha = sigmoid(alpha_in),
 * beta_out = sigmoid(b) when b is not NULL.  [num_tokens, num_heads] inputs with
 * arbitrary strides; contiguous outputs in out_dtype.
 * Replaces: fused_gka_gating
 *   vllm-inference/src/primed_vllm/primed_gka_layer.py:303-358 (kernel :224-300).
 */
int hmx_gka_gating(const void* A_log, int32_t A_log_dtype,
                   const void* a, int64_t a_stride0, int64_t a_stride1,
                   const void* alpha_in, int64_t alpha_in_stride0, int64_t alpha_in_stride1,
                   const void* b, int64_t b_stride0, int64_t b_stride1, int32_t in_dtype,
                   const void* dt_bias, int32_t dt_bias_dtype,
                   void* g, void* alpha, void* beta_out, int32_t out_dtype,
                   int64_t num_tokens, int32_t num_heads, float sp_beta, float threshold,
                   void* stream);

/*
 * GKA decode step (first token of each sequence), in place on slot-indexed pools.
 *  q [B*T, H, 128]; k, v [B*T, HKV, 128] (qkv_dtype); alpha [B*T, H];
 *  q/k/v rows *_token_stride elements apart (multiples of 4; 16-byte aligned bases),
 *  heads contiguous in a row (column slices of a fused projection pass as views)
 *  gk, beta [B*T, H] or NULL; o [B*T, H, 128] (qkv_dtype; first token per sequence)
 *  h_kk_in/out fp32 rows of [H, 128, 128] (row strides in elements; in == out for
 *  the in-place update); h_kv_in/out rows of [H, 128, 128] in h_kv_dtype (f32/bf16).
 *  State row of sequence n: ssm_state_indices[n*idx_stride], or n without indices.
 *  num_iter Chebyshev steps; ridge_ratio; scale (the GLA scale).
 * Replaces: chebyshev_iteration_gqa / gka_chebyshev_gla_decode
 *   vllm-inference/src/primed_vllm/gka/ops/chebyshev_iteration_gqa.py:173-238 (kernel :22-170),
 *   vllm-inference/src/primed_vllm/gka/gka_forward.py:248-326.
 */
int hmx_gka_decode_fwd(const void* q, int64_t q_token_stride, const void* k,
                       int64_t k_token_stride, const void* v, int64_t v_token_stride,
                       int32_t qkv_dtype,
                       const void* alpha, int32_t alpha_dtype,
                       const void* gk, int32_t gk_dtype, const void* beta, int32_t beta_dtype,
                       void* o,
                       const float* h_kk_in, int64_t h_kk_in_row_stride,
                       float* h_kk_out, int64_t h_kk_out_row_stride,
                       const void* h_kv_in, int64_t h_kv_in_row_stride,
                       void* h_kv_out, int64_t h_kv_out_row_stride, int32_t h_kv_dtype,
                       const int32_t* cu_seqlens, const int32_t* ssm_state_indices,
                       int64_t idx_stride, int64_t B, int64_t T, int64_t N,
                       int32_t H, int32_t HKV, int32_t D, int32_t V,
                       int32_t num_iter, float ridge_ratio, float scale,
                       const hmx_gated_norm* o_norm, const hmx_gate_proj* gates, void* stream);

/*
 * GKA chunked prefill forward (Chebyshev ridge solve + beta^2 GLA), GQA-native,
 * varlen via the segment table layout of hmx_gdn_chunk_fwd over 64-token blocks
 * (c_start / c_end count blocks of 64 tokens from the sequence start);
 * nblock_total = the sum over rows of c_end - c_start.  q [T_total, H, 128]; k, v [T_total, HKV, 128] bf16 (raw: q and k are
 * L2-normalised inside, without eps), rows *_token_stride elements apart
 * (multiples of 8; 16-byte aligned bases), heads contiguous in a row; alpha, g
 * [T_total, H]; gk, beta [T_total, H] or NULL; o [T_total, H, 128] bf16
 * (contiguous).  use_qk_l2norm = 0 uses q and k as given (the training form, whose
 * layer normalises them and applies beta to k and v).
 * States: h_kk0 / h_kk_final (and h_kv0 / h_kv_final) are bases of [H, 128, 128]
 * slots h_kk_slot_stride (h_kv_slot_stride) elements apart in h_kk_dtype
 * (h_kv_dtype), f32 or bf16, or NULL (zero start / no end state).  Sequence n
 * uses slot state_indices[n] (n when NULL); a negative slot starts from zero and
 * writes nothing; has_initial_state[n] == 0 (when not NULL) starts from zero.
 * Initial and final bases may be the same pool (updated in place).  h_kk is not
 * tracked when num_iter == 0: its end state is then not written, except that a
 * sequence with has_initial_state[n] == 0 clears its h_kk slot (as the layer's
 * update does, primed_gka_layer.py:1262-1265, :1296-1299).
 * workspace: hmx_gka_chunk_workspace_bytes(...) bytes of device scratch.
 * Replaces: gka_chebyshev_gla_prefill
 *   vllm-inference/src/primed_vllm/gka/gka_forward.py:161-242 (and its kernels
 *   ops/chebyshev_prefill_gqa.py:28-316, ops/chunk_simple_gla_gqa.py:33-190,
 *   ops/chunk_o_gqa.py:25-171) and, with use_qk_l2norm = 0 and beta = NULL, the
 *   training forms gka_chebyshev_gla / torch_decoding_one_step
 *   (training/src/hmf/model/hybrid_zoo/layers/gated_kalmanet/ops/chebyshev/
 *   gka_chebyshev_solve.py:107-164, :324-397).
 */
int hmx_gka_chunk_fwd(const void* q, int64_t q_token_stride, const void* k,
                      int64_t k_token_stride, const void* v, int64_t v_token_stride,
                      int32_t qkv_dtype, const void* alpha, int32_t alpha_dtype, const void* g,
                      int32_t g_dtype, const void* gk, int32_t gk_dtype, const void* beta,
                      int32_t beta_dtype, void* o,
                      const void* h_kk0, void* h_kk_final, int64_t h_kk_slot_stride,
                      int32_t h_kk_dtype, const void* h_kv0, void* h_kv_final,
                      int64_t h_kv_slot_stride, int32_t h_kv_dtype,
                      const int32_t* state_indices, const uint8_t* has_initial_state,
                      const int32_t* seg_table, int32_t nseg_total, int32_t nblock_total,
                      int32_t N, int32_t H, int32_t HKV, int32_t D, int32_t V,
                      int32_t num_iter, float ridge_ratio, float scale, int32_t use_qk_l2norm,
                      void* workspace, size_t workspace_bytes,
                      const hmx_gated_norm* o_norm, const hmx_gate_proj* gates, void* stream);

/* Workspace bytes hmx_gka_chunk_fwd needs (host-only arithmetic).  Companion of
 * hmx_gka_chunk_fwd; no reference counterpart (the reference allocates its
 * chunk states inside the op, chebyshev_prefill_gqa.py:137). */
size_t hmx_gka_chunk_workspace_bytes(int32_t nseg_total, int32_t nblock_total, int32_t N,
                                     int32_t H);

/* The training layer's Chebyshev solve, forward and backward.
 *
 * hmx_gka_cheb_fwd: per token x_t = the Chebyshev recurrence for
 * (H_t + r |H_t|_F I) x = q_t, H_t = e^{gk_t} H_{t-1} + k_t k_t^T from zero, for
 * N sequences of tokens given by seg_table (as hmx_gka_chunk_fwd's, HMX_PLAN_GKA).
 * k, q: [tokens][H][D] rows at their token strides, bf16, D = 128; gk [tokens][H]
 * f32/bf16/f16 or NULL (no decay).  Writes x [tokens][H][D] bf16 (contiguous),
 * fro = |H_t|_F [tokens][H] f32 and h_kk_final [N][H][D][D] f32.  The workspace
 * (hmx_gka_chunk_workspace_bytes) keeps the block-start states for the backward.
 * Replaces: ChebyshevIteration.forward
 *   training/src/hmf/model/hybrid_zoo/layers/gated_kalmanet/ops/chebyshev/
 *   chebyshev_iteration.py:569-604 (chebyshev_iteration_forward_triton :462-557
 *   and its kernels :167-460, chunk_fwd_h of fla for h_kk).
 */
int hmx_gka_cheb_fwd(const void* k, int64_t k_token_stride, const void* q,
                     int64_t q_token_stride, int32_t qk_dtype, const void* gk, int32_t gk_dtype,
                     void* x, float* fro, float* h_kk_final, const int32_t* seg_table,
                     int32_t nseg_total, int32_t nblock_total, int32_t N, int32_t H, int32_t D,
                     int32_t num_iter, float ridge_ratio, void* workspace,
                     size_t workspace_bytes, void* stream);

/* hmx_gka_cheb_bwd: the backward of hmx_gka_cheb_fwd on the same k, gk, seg_table
 * and forward workspace (unchanged since the forward), its x and fro, and dx
 * ([tokens][H][D] bf16 rows at dx_token_stride).  Writes dq, dk [tokens][H][D] bf16
 * (contiguous) and, with gk, dgk [tokens][H] f32: dq solves for dx with the saved
 * |H_t|_F; dk, dgk follow from dL/dH_t = -dq_t x_t^T, minus
 * r (dq_t . x_t) H_t / |H_t|_F when bp_lambda.  bwd_workspace:
 * hmx_gka_cheb_bwd_workspace_bytes(nblock_total, H, tokens) bytes.
 * Replaces: ChebyshevIteration.backward
 *   training/.../ops/chebyshev/chebyshev_iteration.py:606-688 (with
 *   chunk_dk_backward.py:372-445, chunk_dk_backward_gating.py:287-373,
 *   chunk_dh_kk_to_dk_backward.py:96-135, chunk_dh_kk_to_dk_gating_backward.py:146-198 and
 *   chunk_bwd_dh of fla).
 */
int hmx_gka_cheb_bwd(const void* k, int64_t k_token_stride, const void* x, const void* dx,
                     int64_t dx_token_stride, int32_t dtype, const void* gk, int32_t gk_dtype,
                     const float* fro, void* dq, void* dk, float* dgk,
                     const int32_t* seg_table, int32_t nseg_total, int32_t nblock_total,
                     int32_t N, int32_t H, int32_t D, int64_t tokens, int32_t num_iter,
                     float ridge_ratio, int32_t bp_lambda, void* fwd_workspace,
                     size_t fwd_workspace_bytes, void* bwd_workspace, size_t bwd_workspace_bytes,
                     void* stream);
size_t hmx_gka_cheb_bwd_workspace_bytes(int32_t nblock_total, int32_t H, int64_t tokens);

/* hmx_gka_train_fwd: the training GKA forward in one pass: the Chebyshev solve
 * (as hmx_gka_cheb_fwd), the blend u = q + alpha (x - q) and the GLA readout
 * o_t = scale S_t^T u_t, S_t = e^{g_t} S_{t-1} + k_t v_t^T from zero.  q, k, v
 * [tokens][H][D] bf16 contiguous (k, v at H heads, beta applied by the caller);
 * alpha, g [tokens][H] (f32/bf16/f16), gk [tokens][H] or NULL.  Writes o
 * [tokens][H][D] bf16, h_kv_final [N][H][D][D] f32 and, when num_iter > 0, x
 * [tokens][H][D] bf16, fro [tokens][H] f32 and h_kk_final [N][H][D][D] f32 for the
 * backward.  The workspace (hmx_gka_chunk_workspace_bytes) keeps the block-start
 * states for the backward.
 * Replaces: gka_chebyshev_gla
 *   training/.../ops/chebyshev/gka_chebyshev_solve.py:107-164 (ChebyshevIteration,
 *   the blend, and fla's chunk_simple_gla).
 */
int hmx_gka_train_fwd(const void* q, const void* k, const void* v, int32_t dtype,
                      const void* alpha, int32_t alpha_dtype, const void* g, int32_t g_dtype,
                      const void* gk, int32_t gk_dtype, void* o, void* x, float* fro,
                      float* h_kk_final, float* h_kv_final, const int32_t* seg_table,
                      int32_t nseg_total, int32_t nblock_total, int32_t N, int32_t H, int32_t D,
                      int32_t num_iter, float ridge_ratio, float scale, void* workspace,
                      size_t workspace_bytes, void* stream);

/* hmx_gka_train_bwd: the backward of hmx_gka_train_fwd (same inputs, its x, fro and
 * workspace) for dout [tokens][H][D] bf16: writes dq, dk, dv [tokens][H][D] bf16, dg
 * [tokens][H] f32 and, when num_iter > 0, dalpha and (with gk) dgk [tokens][H] f32.
 * The GLA readout's backward gives du, dk, dv, dg; dx = alpha du feeds the solve's
 * backward (as hmx_gka_cheb_bwd) whose dq and dk are added.  Gradients of the
 * final states are not taken.  bwd_workspace:
 * hmx_gka_train_bwd_workspace_bytes(nblock_total, H, tokens) bytes.
 * Replaces: the backward of gka_chebyshev_gla (ChebyshevIteration.backward,
 *   chebyshev_iteration.py:606-688, torch's autograd of the blend at
 *   gka_chebyshev_solve.py:156, and fla's chunk_simple_gla backward).
 */
int hmx_gka_train_bwd(const void* q, const void* k, const void* v, int32_t dtype,
                      const void* alpha, int32_t alpha_dtype, const void* g, int32_t g_dtype,
                      const void* gk, int32_t gk_dtype, const void* x, const float* fro,
                      const void* dout, void* dq, void* dk, void* dv, float* dalpha,
                      float* dg, float* dgk, const int32_t* seg_table, int32_t nseg_total,
                      int32_t nblock_total, int32_t N, int32_t H, int32_t D, int64_t tokens,
                      int32_t num_iter, float ridge_ratio, float scale, int32_t bp_lambda,
                      void* fwd_workspace, size_t fwd_workspace_bytes, void* bwd_workspace,
                      size_t bwd_workspace_bytes, void* stream);
size_t hmx_gka_train_bwd_workspace_bytes(int32_t nblock_total, int32_t H, int64_t tokens);

/*
 * Mamba2 SSD chunk scan forward, bf16 x/B/C/z/y, fp32 states, varlen via a
 * segment table of rows (n, bos, eos, c_start, c_end, seg_idx, first_seg, nseg)
 * over 64-token chunks (bos/eos index the flattened token axis).
 *  z, y [tokens, H, P], x [tokens, HX, P]: element strides (token, head), last
 *  dim contiguous; B [tokens, G, N], C [tokens, GC, N] with strides (token,
 *  group); head h reads x head h/(H/HX), B group h/(H/G), C group h/(H/GC) (HX,
 *  G, GC divide H; HX = GC = H with G = ngroups is the reference's layout, the
 *  primed Mamba2 layer's repeat_kv'd x and B are HX = G = d_xb/headdim read in
 *  place, primed_mamba2_layer.py:800-835); dt [tokens, H]
 *  (f32/bf16/f16) with strides; A [H] fp32 (= -exp(A_log)); D [H, P] fp32 or
 *  NULL; dt_bias [H] fp32 or NULL; z NULL for no gate.  dt' =
 *  clamp(softplus(dt + dt_bias) if dt_softplus else dt + dt_bias, dt_min, dt_max).
 *  h0 / h_final: the initial / end states, each a base of [H, P, N] slots
 *  state_slot_stride elements apart in state_dtype (f32 or bf16), or NULL (zero
 *  start / no end state).  Sequence n uses slot state_indices[n] (n when NULL);
 *  a negative slot starts from zero and writes nothing; has_initial_state[n] == 0
 *  (when not NULL) starts from zero.  h0 and h_final may be the same pool
 *  (updated in place).  P, N in {64, 128}; token/head strides multiples of 8
 *  elements.
 * workspace: hmx_ssd_chunk_workspace_bytes(...) bytes of device scratch.
 * Any finite bf16 x, B, C and f32/bf16 initial state is supported: a walk whose
 *  fp16 operands would leave fp16's range is detected and walked again with bf16
 *  operands (hi + lo pairs for the computed ones).
 * Replaces: mamba_chunk_scan_combined (mamba_ssm 2.3.0; call site
 *   training/src/hmf/model/hybrid_zoo/layers/mamba/mamba2.py:555-580) and
 *   mamba_chunk_scan_combined_varlen (vLLM 0.15.1; call site
 *   vllm-inference/src/primed_vllm/primed_mamba2_layer.py:844-863).
 */
int hmx_ssd_chunk_fwd(const void* x, int64_t x_ts, int64_t x_hs,
                      const void* B, int64_t b_ts, int64_t b_gs,
                      const void* C, int64_t c_ts, int64_t c_gs, int32_t xbc_dtype,
                      const void* dt, int32_t dt_dtype, int64_t dt_ts, int64_t dt_hs,
                      const float* A, const float* D, const float* dt_bias,
                      const void* z, int64_t z_ts, int64_t z_hs,
                      void* y, int64_t y_ts, int64_t y_hs,
                      const void* h0, void* h_final, int64_t state_slot_stride,
                      int32_t state_dtype, const int32_t* state_indices,
                      const uint8_t* has_initial_state,
                      const int32_t* seg_table, int32_t nseg_total, int32_t nseq,
                      int32_t H, int32_t HX, int32_t G, int32_t GC, int32_t P, int32_t N,
                      int32_t dt_softplus, float dt_min, float dt_max,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes hmx_ssd_chunk_fwd needs (host-only arithmetic).  Companion of
 * hmx_ssd_chunk_fwd; no reference counterpart (mamba_ssm allocates its chunk
 * states inside the op). */
size_t hmx_ssd_chunk_workspace_bytes(int32_t nseg_total, int32_t nseq, int32_t H,
                                     int32_t P, int32_t N);

/*
 * Mamba2 SSD chunk scan backward: the gradients of hmx_ssd_chunk_fwd's output y
 * (and end states) with respect to x, dt, A, B, C, D, z, dt_bias and the start
 * states.  The sequences are cut into chunks of at most 64 tokens, one row each of
 * seg_table (n, bos, eos, 0, 1, index in the sequence, first row, rows; a
 * sequence's rows consecutive); seq_table [nseq][2] = (first row, rows).  The
 * chunk start states are formed here (from h0), not taken from the forward.
 *  Inputs as in hmx_ssd_chunk_fwd (bf16 x [tokens, HX, P], B [tokens, G, N],
 *  C [tokens, GC, N], z and dy [tokens, H, P], dt [tokens, H] f32/bf16/f16, fp32 A,
 *  D [H, P], dt_bias).  h0: fp32 [nseq, H, P, N] start states or NULL (zero);
 *  d_final: fp32 [nseq, H, P, N] gradient of the end states, or NULL.
 *  Outputs, contiguous: dx [tokens, HX, P], dB [tokens, G, N], dC [tokens, GC, N]
 *  in grad_dtype (HMX_F32, or HMX_BF16 when none accumulates: HX = H and G = H or
 *  G = GC); dx accumulates when HX < H and dB when G < H and G != GC (then fp32,
 *  zero-filled by the caller); dz bf16 [tokens, H, P] (when z is
 *  given); ddt fp32 [tokens, H] (gradient of the raw dt); dA fp32 [H], dD fp32
 *  [H, P] (or NULL), ddt_bias fp32 [H] (or NULL), all zero-filled by the caller
 *  (they accumulate); dh0 fp32 [nseq, H, P, N] or NULL.  P, N in {64, 128}; z only
 *  with P = 64.
 * workspace: hmx_ssd_chunk_bwd_workspace_bytes(nrows, H, P, N) bytes.
 * Replaces: the backward of mamba_chunk_scan_combined (mamba_ssm 2.3.0, which the
 *   training layer calls under autograd: training/src/hmf/model/hybrid_zoo/
 *   layers/mamba/mamba2.py:555-580).
 */
int hmx_ssd_chunk_bwd(const void* x, int64_t x_ts, int64_t x_hs,
                      const void* B, int64_t b_ts, int64_t b_gs,
                      const void* C, int64_t c_ts, int64_t c_gs, int32_t xbc_dtype,
                      const void* dt, int32_t dt_dtype, int64_t dt_ts, int64_t dt_hs,
                      const float* A, const float* D, const float* dt_bias,
                      const void* z, int64_t z_ts, int64_t z_hs,
                      const void* dy, int64_t dy_ts, int64_t dy_hs,
                      const float* h0, const float* d_final,
                      const int32_t* seg_table, int32_t nrows, const int32_t* seq_table,
                      int32_t nseq, int32_t H, int32_t HX, int32_t G, int32_t GC, int32_t P,
                      int32_t N, int32_t dt_softplus, float dt_min, float dt_max,
                      void* dx, void* dB, void* dC, int32_t grad_dtype, void* dz,
                      float* ddt, float* dA,
                      float* dD, float* ddt_bias, float* dh0,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes hmx_ssd_chunk_bwd needs (host-only arithmetic).  Companion of
 * hmx_ssd_chunk_bwd; no reference counterpart. */
size_t hmx_ssd_chunk_bwd_workspace_bytes(int32_t nrows, int32_t H, int32_t P, int32_t N);

/*
 * Mamba2 single-token state update, in place on a slot-indexed state pool.
 *  state [slots, H, P, N] (f32 or bf16; slot_stride in elements, the rest
 *  contiguous); dt, z, out [batch, H, P], x [batch, HX, P] with element strides
 *  (batch, head, p); A fp32 [H, P, N] with strides (a_ps == a_ns == 0: one value
 *  per head); B [batch, G, N], C [batch, GC, N] with strides (batch, group), N
 *  contiguous; head h reads x head h/(H/HX), B group h/(H/G), C group h/(H/GC)
 *  (HX, G, GC divide H; HX = GC = H is the reference's layout); D, dt_bias fp32
 *  [H, P] with strides, or NULL.  Source slot state_batch_indices[i] (or i),
 *  skipped when equal to pad_slot_id; written to dst_state_batch_indices[i] when
 *  given.  P, N in {64, 128}.
 * Replaces: selective_state_update (mamba_ssm / vLLM; call sites
 *   training/src/hmf/model/hybrid_zoo/layers/mamba/mamba2.py:776-800,
 *   vllm-inference/src/primed_vllm/primed_mamba2_layer.py:1000-1021).
 */
int hmx_ssd_state_update(void* state, int32_t state_dtype, int64_t slot_stride,
                         const void* x, int32_t x_dtype, int64_t x_bs, int64_t x_hs, int64_t x_ps,
                         const void* dt, int32_t dt_dtype, int64_t dt_bs, int64_t dt_hs,
                         int64_t dt_ps, const float* A, int64_t a_hs, int64_t a_ps, int64_t a_ns,
                         const void* B, int32_t b_dtype, int64_t b_bs, int64_t b_gs,
                         const void* C, int32_t c_dtype, int64_t c_bs, int64_t c_gs,
                         const float* D, int64_t d_hs, int64_t d_ps,
                         const float* dt_bias, int64_t db_hs, int64_t db_ps,
                         const void* z, int32_t z_dtype, int64_t z_bs, int64_t z_hs, int64_t z_ps,
                         void* out, int32_t out_dtype, int64_t o_bs, int64_t o_hs, int64_t o_ps,
                         const int32_t* state_batch_indices,
                         const int32_t* dst_state_batch_indices, int32_t pad_slot_id,
                         int32_t batch, int32_t H, int32_t HX, int32_t G, int32_t GC,
                         int32_t P, int32_t N, int32_t dt_softplus, void* stream);

/*
 * Gated RMSNorm over rows of D elements (the GDN / GKA output norm):
 *   norm_before_gate != 0:  out = x / sqrt(mean(x^2) + eps) * weight * silu(z)
 *   norm_before_gate == 0:  u = x * silu(z); out = u / sqrt(mean(u^2) + eps) * weight
 * z may be NULL (plain RMSNorm).  x, z, out share `dtype` (16-byte aligned rows,
 * element row strides); weight [D] in weight_dtype.  fp32 arithmetic, one rounding
 * to dtype.  D in {64, 128, 256}.
 * Replaces: RMSNormGated(head_v_dim, group_size=None, norm_before_gate=True)
 *   (vLLM, un-vendored), constructed at
 *   vllm-inference/src/primed_vllm/primed_gdn_layer.py:443-450 and
 *   primed_gka_layer.py:736-743, called at primed_gdn_layer.py:626 and
 *   primed_gka_layer.py:949; fla FusedRMSNormGated in the training layers
 *   (training/.../layers/gated_deltanet/gdn.py:201, layers/gated_kalmanet/gka.py:233).
 */
int hmx_rms_norm_gated(const void* x, int64_t x_row_stride, const void* z,
                       int64_t z_row_stride, int32_t dtype, const void* weight,
                       int32_t weight_dtype, void* out, int64_t out_row_stride, int64_t rows,
                       int32_t D, float eps, int32_t norm_before_gate, void* stream);

/*
 * Short causal depthwise conv1d, prefill over concatenated sequences:
 *   out[t, c] = act(bias[c] + sum_i weight[c, i] x[t - (width-1) + i, c])
 * act = silu (activation 1) or none (0); width in 2..4.  x / out [total_tokens, dim]
 * rows (element token strides, channels contiguous, 16-byte aligned), sequence b =
 * tokens [query_start_loc[b], query_start_loc[b+1]) (non-decreasing from 0; the
 * kernels clamp them to [0, total_tokens]); tokens from query_start_loc[batch] to
 * total_tokens get output 0.  Positions before a sequence's first token read its conv
 * state (when conv_states is not NULL and has_initial_state[b] != 0, or
 * has_initial_state is NULL), zeros otherwise; afterwards the state holds the
 * sequence's last state_len inputs.  conv_states: rows [slots, state_len, dim] in x's
 * dtype, channels contiguous (element slot / row strides; the layers' cache tensor
 * self_kv_cache[0], primed_gdn_layer.py:669, which they hand to vLLM as its
 * [slots, dim, state_len] transpose), slot cache_indices[b] (or b), skipped (output 0)
 * when equal to pad_slot_id; state_len in [width-1, 8].  weight [dim, width] and bias
 * [dim] (or NULL) in their dtypes.
 * Replaces: causal_conv1d_fn (vLLM, un-vendored; called at
 *   vllm-inference/src/primed_vllm/primed_gdn_layer.py:747-757, :763-773; torch form
 *   training/.../qwen3_5_moe_hmf/modeling_qwen3_5_moe_hmf.py:306-321).
 */
int hmx_causal_conv1d_fwd(const void* x, int64_t x_token_stride, void* out,
                          int64_t out_token_stride, int32_t dtype, const void* weight,
                          int32_t weight_dtype, int32_t width, const void* bias,
                          int32_t bias_dtype, void* conv_states, int64_t state_slot_stride,
                          int64_t state_row_stride, int32_t state_len,
                          const int32_t* query_start_loc, int32_t batch, int64_t total_tokens,
                          const int32_t* cache_indices, const uint8_t* has_initial_state,
                          int32_t dim, int32_t activation, int32_t pad_slot_id, void* stream);

/*
 * Short causal depthwise conv1d, one decode token per sequence: x / out [batch, dim]
 * rows; the window is the last width-1 rows of conv_state[conv_state_indices[b]]
 * (or b) followed by x[b]; the state then shifts by one row with x[b] appended.
 * Padded entries (slot == pad_slot_id) write 0 and leave the pool alone.
 * Replaces: causal_conv1d_update (vLLM, un-vendored; called at
 *   vllm-inference/src/primed_vllm/primed_gdn_layer.py:735-743, :775-785); the
 *   speculative multi-token form is hmx_causal_conv1d_update_spec.
 */
int hmx_causal_conv1d_update(const void* x, int64_t x_token_stride, void* out,
                             int64_t out_token_stride, int32_t dtype, const void* weight,
                             int32_t weight_dtype, int32_t width, const void* bias,
                             int32_t bias_dtype, void* conv_state, int64_t state_slot_stride,
                             int64_t state_row_stride, int32_t state_len,
                             const int32_t* conv_state_indices, int32_t batch, int32_t dim,
                             int32_t activation, int32_t pad_slot_id, void* stream);

/*
 * The speculative multi-token form: sequence b's tokens are rows
 * query_start_loc[b] .. query_start_loc[b+1]-1 of x / out (offsets clamped to
 * [0, total_tokens]; at most state_len - width + 2 of them are processed), against slot
 * conv_state_indices[b] (or b).  With a = num_accepted_tokens[b] (the previous
 * step's accepted tokens, clamped to [1, state_len - width + 2]) the window before
 * the first token is state rows a-1 .. a+width-3; afterwards the slot holds rows
 * a .. a+state_len-n-1 followed by the n new inputs, so the next step's window
 * again ends at its last accepted input.  Padded entries (slot == pad_slot_id)
 * write 0 and leave the pool alone.
 * Replaces: causal_conv1d_update with num_accepted_tokens / query_start_loc / max_query_len
 *   (vLLM, un-vendored; called at
 *   vllm-inference/src/primed_vllm/primed_gdn_layer.py:700-712,
 *   primed_gka_layer.py:1029-1040).  vLLM's state rows are not vendored here: the
 *   row arithmetic above is pinned by the invariant that a speculative step followed
 *   by a step accepting a tokens computes the plain causal convolution over the
 *   accepted inputs.
 */
int hmx_causal_conv1d_update_spec(const void* x, int64_t x_token_stride, void* out,
                                  int64_t out_token_stride, int32_t dtype, const void* weight,
                                  int32_t weight_dtype, int32_t width, const void* bias,
                                  int32_t bias_dtype, void* conv_state, int64_t state_slot_stride,
                                  int64_t state_row_stride, int32_t state_len,
                                  const int32_t* conv_state_indices,
                                  const int32_t* num_accepted_tokens,
                                  const int32_t* query_start_loc, int32_t batch,
                                  int64_t total_tokens, int32_t dim, int32_t activation,
                                  int32_t pad_slot_id, void* stream);

/*
 * hmx_causal_conv1d_fwd with prefix caching (vLLM's block arguments, as the Mamba2
 * layer passes them with mamba_cache_mode "all"): cache_indices is a
 * [batch, cache_indices_cols] table (row stride cache_indices_row_stride elements)
 * of one slot per block of block_size tokens.  Sequence b continues
 * num_computed_tokens[b] computed tokens; it reads its initial state (where
 * has_initial_state[b] != 0) from column initial_state_idx[b]; every block k from
 * block_idx_first_scheduled_token[b] to block_idx_last_scheduled_token[b] - 1 ends in
 * this step, and column k receives the state at its end (the last state_len inputs
 * before absolute position (k + 1) * block_size); column
 * block_idx_last_scheduled_token[b] receives the state after the sequence's last
 * token.  Columns are clamped into the table; a written slot equal to pad_slot_id is
 * skipped, and a sequence whose last column's slot is pad_slot_id gets output 0 and
 * touches no state.  Outputs are those of hmx_causal_conv1d_fwd.
 * Replaces: causal_conv1d_fn with block_idx_first_scheduled_token /
 *   block_idx_last_scheduled_token / initial_state_idx / num_computed_tokens /
 *   block_size_to_align (vLLM, un-vendored; called at
 *   vllm-inference/src/primed_vllm/primed_mamba2_layer.py:770-793).  The block
 *   positions follow the layer's own use of the same metadata for the SSD states
 *   (:864-933: block k's state is the state after its last token).
 */
int hmx_causal_conv1d_fwd_blocks(const void* x, int64_t x_token_stride, void* out,
                                 int64_t out_token_stride, int32_t dtype, const void* weight,
                                 int32_t weight_dtype, int32_t width, const void* bias,
                                 int32_t bias_dtype, void* conv_states, int64_t state_slot_stride,
                                 int64_t state_row_stride, int32_t state_len,
                                 const int32_t* query_start_loc, int32_t batch,
                                 int64_t total_tokens, const int32_t* cache_indices,
                                 int64_t cache_indices_row_stride, int32_t cache_indices_cols,
                                 const uint8_t* has_initial_state,
                                 const int32_t* initial_state_idx,
                                 const int32_t* block_idx_first_scheduled_token,
                                 const int32_t* block_idx_last_scheduled_token,
                                 const int32_t* num_computed_tokens, int32_t block_size,
                                 int32_t dim, int32_t activation, int32_t pad_slot_id,
                                 void* stream);

/*
 * hmx_causal_conv1d_update with prefix caching: conv_state_indices is a
 * [batch, indices_cols] table (row stride indices_row_stride); the window is read from
 * the slot at column initial_state_idx[b] and the shifted state written to the slot at
 * column block_idx_last_scheduled_token[b] (the same slot when both columns agree).
 * An entry whose read or written slot is pad_slot_id writes 0 and touches no state.
 * Replaces: causal_conv1d_update with block_idx_last_scheduled_token /
 *   initial_state_idx (vLLM, un-vendored; called at
 *   vllm-inference/src/primed_vllm/primed_mamba2_layer.py:964-973).
 */
int hmx_causal_conv1d_update_blocks(const void* x, int64_t x_token_stride, void* out,
                                    int64_t out_token_stride, int32_t dtype, const void* weight,
                                    int32_t weight_dtype, int32_t width, const void* bias,
                                    int32_t bias_dtype, void* conv_state,
                                    int64_t state_slot_stride, int64_t state_row_stride,
                                    int32_t state_len, const int32_t* conv_state_indices,
                                    int64_t indices_row_stride, int32_t indices_cols,
                                    const int32_t* initial_state_idx,
                                    const int32_t* block_idx_last_scheduled_token, int32_t batch,
                                    int32_t dim, int32_t activation, int32_t pad_slot_id,
                                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HMX_H_ */
