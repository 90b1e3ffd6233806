/*
 * ccq_hip.h -- C ABI of the MI355X (gfx950) CCQ library, libccq_hip.so.
 *
 * All pointers are device pointers allocated by the caller; every call is
 * asynchronous on the given HIP stream (hipStream_t passed as void*, NULL =
 * default stream) and returns 0 on success or a negative status
 * (CCQ_ERR_*); ccq_last_error() describes the last failure of the calling
 * host thread.  No entry point allocates device memory or keeps state between
 * calls (apart from the opt-in kernel timing at the end of this header); buffers a
 * backward pass needs from its forward ("saved") and scratch
 * space ("workspace") are caller-provided, sized by the *_bytes() queries.
 *
 * The cleaning and GDN chunk entry points size their buffers (the *_bytes() queries) and shape
 * their launches by the CU count of the device that is current; they return CCQ_ERR_DEVICE when the
 * stream belongs to another device.  Make the stream's device current for the queries and calls.
 *
 * Layouts follow the reference (token-major, head-interleaved):
 *   q, k [tokens, H, K] bf16; v, o [tokens, H, V] bf16; per-token scalars
 *   [tokens, H] fp32; tokens = B*T (dense) or the packed length (varlen:
 *   B == 1 and cu_seqlens int64 [N+1]).  Per-sequence states are fp32:
 *   covariance [N, H, K, K], key sum [N, H, K], backbone state [N, H, K, V].
 */
#ifndef CCQ_HIP_H
#define CCQ_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CCQ_OK 0
#define CCQ_ERR_SHAPE (-1)     /* unsupported or inconsistent sizes */
#define CCQ_ERR_NULL (-2)      /* a required pointer is NULL */
#define CCQ_ERR_ALIGN (-3)     /* a pointer is not 16-byte aligned */
#define CCQ_ERR_HIP (-4)       /* a HIP runtime error (see ccq_last_error) */
#define CCQ_ERR_DEVICE (-5)    /* the stream belongs to a device other than the current one */

int ccq_abi_version(void);
const char* ccq_last_error(void);

/*
 * Fused covariance read + cleaning, forward.
 * Replaces the reference's FusedCCQCleanRead.forward -> _fused_read_fwd
 * (ccq/ops/common/fused_read.py:480-491, :379-403), i.e. fla chunk_fwd_h(v=k)
 * + _cumk_chunk_prefix + _ccq_fused_read_fwd_kernel, and the stock
 * _ccq_compute_z_and_sum_kk + _CCQCleanQ forward (clean.py:751-771, :696-715).
 *
 *   q_clean_t = q_t - lambda_t (h_t^T q_t / pos_t - (m_t . q_t) m_t / pos_t^2)
 *   h_t = h0 + sum_{j<=t} k_j k_j^T, m_t = m0 + sum_{j<=t} k_j, pos_t = max(t + 1 + position_offset, 1)
 *
 * lambda: fp32 [tokens, H] (the reference's lambda after _reshape_lambda_3d,
 *   clean.py:314-325).  Alternatively gate_w [H, K] / gate_b [H] (fp32) compute
 *   lambda_t = sigmoid(gate_w[h] . q_t + gate_b[h]) in the kernel (lambda is then
 *   ignored and written to lambda_out if non-NULL) -- the per-head form of the
 *   reference layer's erase_lambda_proj (ccq/gdn/layer.py:174, 292).
 * h0, m0: initial states (nullable); m0 is ignored unless subtract_mean.
 * saved: ccq_clean_saved_bytes() bytes, written here and read by ccq_clean_bwd
 *   (segment states; varlen block/segment indexes).  varlen = (cu_seqlens != NULL).
 * Outputs: q_clean bf16 and/or q_clean_f32 (at least one), h_final, m_final (nullable).
 * K in {32, 64, 128, 256}.
 */
size_t ccq_clean_saved_bytes(int64_t tokens, int B, int T, int N, int H, int K, int varlen);
int ccq_clean_fwd(const void* q, const void* k, const float* lambda, const float* gate_w, const float* gate_b,
                  float* lambda_out, const float* h0, const float* m0, const int64_t* cu_seqlens, void* saved,
                  void* q_clean, float* q_clean_f32, float* h_final, float* m_final, int B, int T, int H, int K,
                  int N, int position_offset, int subtract_mean, void* stream);

/*
 * Cleaning backward.  Replaces FusedCCQCleanRead.backward -> _fused_read_bwd
 * (fused_read.py:496-514, :406-460: chunk_bwd_dh, _ccq_fused_read_bwd_kernel,
 * the dlambda tile sum :443, _chunk_carry + _ccq_add_carry_kernel) and
 * _CCQCleanQ.backward (clean.py:720-748).
 *
 * Inputs as in the forward, plus `saved` from it.  lambda: the lambda the forward used
 * (the gate's lambda_out in the fused-gate form).  dq_clean: upstream gradient, fp32
 * (dq_clean_f32) or bf16 (dq_clean).  dk_extra: optional fp32 [tokens, H, K] added into dk
 * (another use of k).  dh_final / dm_final: gradients into the final states (nullable).
 * Outputs: dq, dk (bf16 and/or fp32 variants, at least one of each); dlambda fp32
 *   [tokens, H] (nullable), or with gate_w/gate_b: dgate_w [H, K], dgate_b [H] and the
 *   gate's path folded into dq; dh0, dm0 (nullable; h0 is treated as symmetric, as the
 *   reference does).  workspace: ccq_clean_bwd_workspace_bytes() bytes.
 */
size_t ccq_clean_bwd_workspace_bytes(int64_t tokens, int B, int T, int N, int H, int K, int varlen, int gate);
int ccq_clean_bwd(const void* q, const void* k, const float* lambda, const float* gate_w, const float* gate_b,
                  const float* dq_clean_f32, const void* dq_clean, const float* dk_extra, const float* h0,
                  const float* m0, const int64_t* cu_seqlens, const void* saved, const float* dh_final,
                  const float* dm_final, void* dq, float* dq_f32, void* dk, float* dk_f32, float* dlambda,
                  float* dgate_w, float* dgate_b, float* dh0, float* dm0, void* workspace, int B, int T, int H,
                  int K, int N, int position_offset, int subtract_mean, void* stream);

/*
 * Cleaning given a precomputed covariance read z = C_t^T q_t (the reference's stock `chunk` path):
 * replaces _CCQCleanQ (ccq/ops/common/clean.py:691-748; forward _ccq_clean_q_triton_fwd :341-384,
 * backward _ccq_clean_q_bwd_triton :633-688 with _rev_cumsum_time :190-217).
 *   q_clean_t = q_t - lambda_t (z_t/pos_t - (m_t . q_t) m_t/pos_t^2),  m_t = m0 + sum_{j<=t} k_j
 * q, k, z, q_clean bf16 [tokens, H, K]; lambda fp32 [tokens, H]; m0, m_final fp32 [N, H, K]
 * (nullable).  num_blocks / chunk_index / chunk_offsets: 64-token blocks, as for ccq_gdn_fwd.
 * saved: ccq_clean_z_saved_bytes() bytes (key-sum prefix per block), read by the backward.
 * Backward: dq_clean bf16 (or dq_clean_f32), dm_final (nullable; used with subtract_mean) ->
 * dq, dk, dz bf16, dlambda fp32 [tokens, H] (nullable), dm0 fp32 [N, H, K] (nullable).
 * K in {32, 64, 128, 256}.
 */
size_t ccq_clean_z_saved_bytes(int num_blocks, int H, int K);
size_t ccq_clean_z_bwd_workspace_bytes(int num_blocks, int H, int K);
int ccq_clean_z_fwd(const void* q, const void* k, const void* z, const float* lambda, const float* m0,
                    const int64_t* cu_seqlens, const int* chunk_index, const int* chunk_offsets, int num_blocks,
                    void* saved, void* q_clean, float* m_final, int B, int T, int H, int K, int N, int position_offset,
                    int subtract_mean, void* stream);
int ccq_clean_z_bwd(const void* q, const void* k, const void* z, const float* lambda, const int64_t* cu_seqlens,
                    const int* chunk_index, const int* chunk_offsets, int num_blocks, const void* saved,
                    const void* dq_clean, const float* dq_clean_f32, const float* dm_final, void* dq, void* dk,
                    void* dz, float* dlambda, float* dm0, void* workspace, int B, int T, int H, int K, int N,
                    int position_offset, int subtract_mean, void* stream);

/*
 * Varlen chunk index: chunk_offsets int32 [N+1] and chunk_index int32 [capacity, 2]
 * ((sequence, chunk) per 64-token chunk, -1 past the end), capacity >= tokens/64 + N.
 * Replaces fla prepare_chunk_indices / prepare_chunk_offsets (fused_read.py:36, :349-352).
 */
int ccq_chunk_index(const int64_t* cu_seqlens, int N, int* chunk_offsets, int* chunk_index, int capacity,
                    void* stream);

/* Bytes of the forward-to-backward buffer and of the backward workspace of the GDN chunk path. */
size_t ccq_gdn_saved_bytes(int64_t tokens, int num_chunks, int H, int K, int V);
size_t ccq_gdn_bwd_workspace_bytes(int64_t tokens, int num_chunks, int H, int K, int V);

/*
 * Gated delta rule, chunk form (64-token chunks), forward.
 * Replaces fla chunk_gated_delta_rule as called by the reference
 * (ccq/ops/ccq_gdn/fused_chunk.py:54-58, chunk.py:132-142):
 *   S <- exp(g_t) S; u = beta_t (v_t - S^T k_t); S <- S + k_t u^T; o_t = S^T (scale q_t)
 * q: bf16 (q) or fp32 (q_f32: the cleaned query kept in fp32); g fp32 [tokens, H]
 * (log decay, nullable = 0); beta fp32 [tokens, H]; initial_state fp32 [N, H, K, V]
 * (nullable).  num_chunks = B * ceil(T/64) (dense) or the capacity used for
 * ccq_chunk_index (varlen, with chunk_index / chunk_offsets).
 * Outputs: o bf16, final_state fp32 (nullable), saved (ccq_gdn_saved_bytes).
 * K in {64, 128, 256}; V a multiple of 64.
 */
int ccq_gdn_fwd(const void* q, const float* q_f32, const void* k, const void* v, const float* g, const float* beta,
                const float* initial_state, const int64_t* cu_seqlens, const int* chunk_index,
                const int* chunk_offsets, int num_chunks, void* o, float* final_state, void* saved, int B, int T,
                int H, int K, int V, int N, float scale, void* stream);

/*
 * Gated delta rule backward (same inputs and saved buffer as the forward).
 * d_o bf16 [tokens, H, V], d_final_state fp32 (nullable).
 * Outputs: dq_f32, dk_f32 fp32 [tokens, H, K]; dv bf16; dbeta, dg fp32 [tokens, H];
 * d_initial_state fp32 [N, H, K, V] (nullable).
 */
int ccq_gdn_bwd(const void* q, const float* q_f32, const void* k, const void* v, const float* g, const float* beta,
                const int64_t* cu_seqlens, const int* chunk_index, const int* chunk_offsets, int num_chunks,
                const void* saved, const void* d_o, const float* d_final_state, void* workspace, float* dq_f32,
                float* dk_f32, void* dv, float* dbeta, float* dg, float* d_initial_state, int B, int T, int H, int K,
                int V, int N, float scale, void* stream);

/* Bytes of the forward-to-backward buffer and of the backward workspace of the GLA chunk path. */
size_t ccq_gla_saved_bytes(int64_t tokens, int num_chunks, int H, int K, int V);
size_t ccq_gla_bwd_workspace_bytes(int64_t tokens, int num_chunks, int H, int K, int V);

/*
 * Gated linear attention, chunk form (64-token chunks), forward.
 * Replaces fla chunk_gla as called by the reference (ccq/ops/ccq_gla/fused_chunk.py:42-45,
 * ccq/ops/ccq_gla/chunk.py:53-58):
 *   S <- diag(exp(gk_t)) S + k_t v_t^T;  o_t = S^T (scale q_t)
 * q: bf16 (q) or fp32 (q_f32: the cleaned query kept in fp32); gk fp32 [tokens, H, K] per-channel
 * log decay (nullable = no decay); initial_state fp32 [N, H, K, V] (nullable).  num_chunks,
 * chunk_index, chunk_offsets as for ccq_gdn_fwd.  Outputs: o bf16, final_state fp32 (nullable),
 * saved (ccq_gla_saved_bytes).  K in {64, 128, 256}; V a multiple of 64 (<= 1024).  Exact while
 * the log decay summed over any 16 consecutive tokens stays above -80.
 */
int ccq_gla_fwd(const void* q, const float* q_f32, const void* k, const void* v, const float* gk,
                const float* initial_state, const int64_t* cu_seqlens, const int* chunk_index,
                const int* chunk_offsets, int num_chunks, void* o, float* final_state, void* saved, int B, int T,
                int H, int K, int V, int N, float scale, void* stream);

/*
 * GLA backward (same inputs and saved buffer as the forward).  d_o bf16 [tokens, H, V];
 * d_final_state fp32 (nullable) -- with dgk it needs the forward's final_state.
 * Outputs: dq_f32, dk_f32 fp32 [tokens, H, K]; dv bf16 and/or dv_f32 fp32 [tokens, H, V] (at least
 * one); dgk fp32 [tokens, H, K] (nullable); d_initial_state fp32 [N, H, K, V] (nullable).
 */
int ccq_gla_bwd(const void* q, const float* q_f32, const void* k, const void* v, const float* gk,
                const int64_t* cu_seqlens, const int* chunk_index, const int* chunk_offsets, int num_chunks,
                const void* saved, const void* d_o, const float* d_final_state, const float* final_state,
                void* workspace, float* dq_f32, float* dk_f32, void* dv, float* dv_f32, float* dgk,
                float* d_initial_state, int B, int T, int H, int K, int V, int N, float scale, void* stream);

/*
 * Recurrent (decode) step: a few tokens per sequence against cached states, inference only.
 * Replaces the reference's fused_recurrent_ccq_gdn (ccq/ops/ccq_gdn/fused_recurrent.py:18-75:
 * fused_ccq_clean(use_chunk=False) = fla fused_recurrent_gla(v=k, h0=C) + _CCQCleanQ, then fla
 * fused_recurrent_gated_delta_rule(h0=S)) and fused_recurrent_ccq_gla
 * (ccq/ops/ccq_gla/fused_recurrent.py:9-51, backbone fla fused_recurrent_gla(gk)).  Per token:
 *   q, k <- l2norm (if use_l2norm; results rounded to bf16); C += k k^T; m += k; z = C^T q;
 *   q_clean = q - lambda (z/pos - (m.q) m/pos^2), pos = max(t + 1 + position_offset, 1);
 *   GDN: S <- e^g diag(e^gk) S diag(e^gv); u = beta (v - S^T k); S += k u^T (gk fp32 [tokens, H, K]
 *   and gv fp32 [tokens, H, V] optional, as fla's fused_recurrent_gated_delta_rule takes them from
 *   the reference, ccq/ops/ccq_gdn/fused_recurrent.py:66-74).  GLA: S <- diag(e^gk) S + k v^T.
 *   o = S^T (scale q_clean)  (bf16 [tokens, H, V]).
 * state/cov_state/mean_state: cached fp32 S [N, H, K, V], C [N, H, K, K], m [N, H, K] (nullable =
 * zero); the *_out buffers receive the updated states (nullable = not written).  state_out and
 * cov_state_out may alias their inputs (in-place cache update); mean_state_out may not.
 * lambda fp32 [tokens, H] or gate_w/gate_b as in ccq_clean_fwd.  enable_ccq = 0 (GDN only) skips
 * the cleaning and the C/m states.  workspace: ccq_decode_workspace_bytes().
 * K in {32, 64, 128, 256}; V a multiple of 64 (<= 1024).  q, k, v, o, the workspace, state,
 * cov_state, their outputs and gv must be 16-byte aligned (CCQ_ERR_ALIGN otherwise): the kernels move
 * state slices and gv as 16-byte pieces of four columns.
 */
size_t ccq_decode_workspace_bytes(int64_t tokens, int H, int K);
int ccq_gdn_decode(const void* q, const void* k, const void* v, const float* lambda, const float* gate_w,
                   const float* gate_b, const float* g, const float* beta, const float* gk, const float* gv,
                   const float* state, const float* cov_state,
                   const float* mean_state, const int64_t* cu_seqlens, void* o, float* state_out,
                   float* cov_state_out, float* mean_state_out, void* workspace, int B, int T, int H, int K, int V,
                   int N, int position_offset, int subtract_mean, int use_l2norm, int enable_ccq, float scale,
                   void* stream);
/*
 * ccq_gdn_decode without a workspace argument, for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  Same arguments, results and kernels as ccq_gdn_decode; its scratch is a fixed
 * per-device array of CCQ_DECODE_SCRATCH_BYTES (8 bytes per token x head x key channel: B*T*H*K
 * up to 1 Mi elements, e.g. 1,024 tokens of 4 heads at K = 256), and a larger call returns
 * CCQ_ERR_SHAPE.  It calls no allocator.  Calls on one GPU share that array: calls that overlap
 * in time on one GPU (different streams or host threads) race; calls in one stream are ordered.
 */
#define CCQ_DECODE_SCRATCH_BYTES ((size_t)8 << 20)
int ccq_gdn_decode_noalloc(const void* q, const void* k, const void* v, const float* lambda, const float* gate_w,
                           const float* gate_b, const float* g, const float* beta, const float* gk, const float* gv,
                           const float* state,
                           const float* cov_state, const float* mean_state, const int64_t* cu_seqlens, void* o,
                           float* state_out, float* cov_state_out, float* mean_state_out, int B, int T, int H, int K,
                           int V, int N, int position_offset, int subtract_mean, int use_l2norm, int enable_ccq,
                           float scale, void* stream);
/*
 * GLA backbone options of the recurrent op (fla fused_recurrent_gla as the reference calls it,
 * ccq/ops/ccq_gla/fused_recurrent.py:41-49): gk fp32 [tokens, H, K] and gv fp32 [tokens, H, V] log
 * decays of the state's rows and columns (nullable), S <- diag(e^gk) S diag(e^gv) + k v^T; reverse
 * != 0 runs the backbone recurrence from each sequence's last token to its first (the cleaning runs
 * forwards, as in the reference).
 */
int ccq_gla_decode(const void* q, const void* k, const void* v, const float* lambda, const float* gate_w,
                   const float* gate_b, const float* gk, const float* gv, const float* state, const float* cov_state,
                   const float* mean_state, const int64_t* cu_seqlens, void* o, float* state_out,
                   float* cov_state_out, float* mean_state_out, void* workspace, int B, int T, int H, int K, int V,
                   int N, int position_offset, int subtract_mean, int use_l2norm, int reverse, float scale,
                   void* stream);

/*
 * Decode step for a captured (HIP-graph) generation loop: ccq_gdn_decode / ccq_gla_decode on B
 * sequences of T new tokens each, with the cached states S, C, m updated in place and the position
 * offset read from device memory (`position`, one int) and advanced by T after the step, so one
 * captured graph can be replayed token after token.  Replaces the same reference calls as
 * ccq_gdn_decode, as the reference layers make them once per generated token with the cache tuple
 * (S, C, m, position_offset) (ccq/gdn/layer.py:318-336, 397; ccq/gla/layer.py); the position lives
 * on the device here because a captured launch cannot take a new host value per replay.
 * workspace: ccq_decode_step_workspace_bytes(B, T, H, K) (the decode workspace plus the new key
 * sum, copied over mean_state by the step's second kernel).  Launches two kernels, no allocation
 * and no memset.
 */
size_t ccq_decode_step_workspace_bytes(int B, int T, int H, int K);
/*
 * Decode linear map y = x W^T (+ residual) for at most 16 token rows: the projections of a decode
 * step (the reference layer's nn.Linear q/k/v/a/b/g projections and o_proj, ccq/gdn/layer.py:
 * 286-316, 408, at one token per sequence), where the weight is read once and is nearly all the
 * bytes.  x bf16 [M, K] (row stride ldx, a multiple of 8, 16-byte aligned), weight bf16 [N, K]
 * (16-byte aligned), residual bf16 [M, N] with row stride ldr (nullable), y bf16 [M, N] with row
 * stride ldy.  fp32 accumulation rounded to bf16, then the residual added in fp32 and rounded again
 * (the roundings of residual + linear(x) on bf16 tensors).  With norm_weight (bf16 [K], 16-byte
 * aligned; nullable) each row of x first becomes bf16(x * norm_weight / sqrt(mean(x^2) + norm_eps)),
 * the rounding of a bf16 nn.RMSNorm ahead of the projection (a pre-norm block's norm, folded in).
 * M <= 16, K a multiple of 32 in [32, 4096].  One kernel, no allocation, graph-capturable.
 */
int ccq_decode_linear(const void* x, int64_t ldx, const void* weight, const void* residual, int64_t ldr, void* y,
                      int64_t ldy, int M, int K, int N, const void* norm_weight, float norm_eps, void* stream);
/*
 * A gated MLP's up projection in the same form: weight bf16 [2N, K] (the gate rows, then the up rows),
 * y bf16 [M, N] = silu(gate) * up with gate, up = (x weight^T).chunk(2, -1) -- the bf16 roundings of
 * those torch ops (each projection, silu, the product) made in the kernel's epilogue, so the
 * [M, 2N] projection never leaves the chip.  No counterpart in the reference's operators (its MLP is
 * fla's); for a decode step's MLP, which the C4 harness runs around the layers.
 */
int ccq_decode_linear_glu(const void* x, int64_t ldx, const void* weight, void* y, int64_t ldy, int M, int K, int N,
                          const void* norm_weight, float norm_eps, void* stream);
/*
 * ccq_decode_linear (without the norm) with the contraction split over `splits` workgroups per 16
 * output columns (1 <= splits <= min(8, K/32)): for the narrow projections of a decode step (N about
 * 1024: o_proj, an MLP's down projection), which otherwise run as N/16 workgroups, too few to keep
 * the weight's bytes in flight.  Each workgroup leaves an fp32 partial tile in the workspace; the
 * last of a column block's workgroups to arrive (an atomic count) adds the tiles in split order, so
 * the result is the same whichever finishes last, and rounds as ccq_decode_linear does.  workspace:
 * ccq_decode_linear_split_workspace_bytes(N, splits) bytes, 16-byte aligned, zero before the first
 * call (its counters; every call leaves them zero); calls that overlap on one workspace race.
 * No counterpart in the reference (its projections are nn.Linear: ccq/gdn/layer.py:408).
 */
/*
 * The output projection of a gated-norm layer with the norm folded in: y = (gnorm(x, gate) W^T)
 * (+ residual), gnorm(x, g) = bf16(x r norm_weight[k mod dv] silu(g)) per head of dv columns with
 * r = 1 / sqrt(mean over the head of x^2 + norm_eps) -- the arithmetic of
 * ccq_gated_rmsnorm_fwd_strided, so that this equals that norm followed by ccq_decode_linear_split
 * (up to the order of the head's sum of squares, which can move a rare normed element by one bf16
 * unit), without the norm's launch and the normed rows' round trip.  The contraction is split per
 * head (K / dv workgroups per 16 output columns, each forming its head's sum from its own operands);
 * workspace: ccq_decode_linear_split_workspace_bytes(N, K / dv) bytes as for
 * ccq_decode_linear_split (zero before the first call, left zero; not needed for one head).
 * gate: bf16 rows (row stride ldg >= K, a multiple of 8) in x's head layout; norm_weight fp32 [dv]
 * (nullable: ones); dv a multiple of 32, K / dv <= 8.  Follows FusedRMSNormGated + o_proj
 * (ccq/gdn/layer.py:402-408).
 */
int ccq_decode_linear_gnorm(const void* x, int64_t ldx, const void* gate, int64_t ldg, const float* norm_weight,
                            int dv, float norm_eps, const void* weight, const void* residual, int64_t ldr, void* y,
                            int64_t ldy, int M, int K, int N, void* workspace, void* stream);
/*
 * Greedy step of a generate loop (the argmax that HF greedy decoding takes of the last position's
 * logits, ccq/generation.py:17-50 feeding the token back): ids[m * ldi] = argmax over n of
 * logits[m * ldl + n] (int64; the first index of the maximum, a NaN larger than any number -- as
 * torch.argmax), and x[m * ldx + :D] = table[ids[m] * D + :D] (zeros for an id >= rows), the
 * embedding rows of the picked tokens: the next decode step's input.  logits bf16, ldl >= N (rows
 * 16-byte aligned are read in 16-byte pieces); table bf16 [rows, D]; x bf16.  One launch, no
 * allocation.
 */
int ccq_greedy_embed(const void* logits, int64_t ldl, int M, int N, const void* table, int64_t rows, int D,
                     int64_t* ids, int64_t ldi, void* x, int64_t ldx, void* stream);
size_t ccq_decode_linear_split_workspace_bytes(int N, int splits);
int ccq_decode_linear_split(const void* x, int64_t ldx, const void* weight, const void* residual, int64_t ldr, void* y,
                            int64_t ldy, int M, int K, int N, int splits, void* workspace, void* stream);
/*
 * The CCQ-GDN layer's per-token prologue in one launch, ahead of ccq_gdn_decode_step: what the
 * reference layer computes between its input projections and fused_recurrent_ccq_gdn
 * (ccq/gdn/layer.py:266-316) -- the q, k, v short convolutions + SiLU with their caches (fla
 * ShortConvolution), lambda = sigmoid(erase_lambda_proj(q)) on the un-normalised activation,
 * beta = sigmoid(b_proj x) (x 2 with allow_neg_eigval), g = -exp(A_log) softplus(a_proj x + dt_bias)
 * and the per-head L2 normalisation of q and k -- with the same bf16 roundings as that sequence of
 * bf16 operations.  xq, xk, xv, xa, xb: bf16 rows of the q (H*K), k (H*K), v (H*V), a (H) and b (H)
 * projections of token r = b*T + t at element offset r*ldx (ldx % 8 == 0, q/k/v rows 16-byte
 * aligned); wq/wk/wv bf16 [D, W] convolution weights, bq/bk/bv bf16 [D] biases (nullable); cq/ck/cv
 * bf16 [B, D, W-1] caches (each sequence's previous W-1 inputs), updated in place; lam_w bf16
 * [H, H*K], lam_b bf16 [H] (nullable), A_log, dt_bias bf16 [H].  Outputs: q, k bf16 [B, T, H, K], v
 * bf16 [B, T, H, V], lam, g, beta fp32 [B, T, H] -- the decode step's inputs with use_l2norm = 0
 * (lam may be NULL for a layer without cleaning: then lam_w and lam_b are not read).
 * H <= 32; K a power of two in [8, 512]; H*K <= 2048; V % 8 == 0; W in [1, 8]; the convolution
 * weights, biases, caches and lam_w 16-byte aligned.  No allocation; one kernel (a workgroup per
 * sequence and slice: the q channels with the gates, then up to 2048 k or v channels each).
 */
int ccq_gdn_decode_prologue(const void* xq, const void* xk, const void* xv, const void* xa, const void* xb,
                            int64_t ldx, const void* wq, const void* wk, const void* wv, const void* bq,
                            const void* bk, const void* bv, void* cq, void* ck, void* cv, const void* lam_w,
                            const void* lam_b, const void* A_log, const void* dt_bias, void* q, void* k, void* v,
                            float* lam, float* g, float* beta, int B, int T, int H, int K, int V, int W,
                            int allow_neg_eigval, float eps, void* stream);
/*
 * A CCQ-GDN layer's input projections for a decode step with the per-channel part of its decode
 * prologue in the epilogue (ccq_decode_linear's projection and optional folded RMSNorm, then): the
 * q, k and v column blocks (at off_q, off_k: Dq columns; off_v: Dv) leave as
 * bf16(SiLU(short convolution)) over each sequence's last 4 inputs (bf16 projection values; earlier
 * tokens of the call from their rows, older ones from the caches cq, ck, cv bf16 [B, D, 3], which
 * the call's last token advances), and the a and b columns (off_a, off_b: H each) also give
 * g = -exp(A_log) softplus(a + dt_bias) and beta = sigmoid(b) (x 2 with allow_neg_eigval) in fp32
 * [M, H] -- the roundings of ccq_gdn_decode_prologue, whose per-head L2 normalisation and lambda
 * gate ccq_gdn_layer_decode_step then applies.  Other columns (the output gate) are the projection.
 * M = B T rows (T tokens per sequence, M <= 16); convolution width 4 (taps bf16 [D, 4], biases
 * [D] nullable).  Follows ccq/gdn/layer.py:266-316 with ccq_gdn_decode_prologue.
 */
int ccq_gdn_decode_in_proj(const void* x, int64_t ldx, const void* weight, void* y, int64_t ldy, int M, int K, int N,
                           const void* norm_weight, float norm_eps, int off_q, int off_k, int off_v, int off_a,
                           int off_b, int H, int Dq, int Dv, int T, const void* wq, const void* wk, const void* wv,
                           const void* bq, const void* bk, const void* bv, void* cq, void* ck, void* cv,
                           const void* A_log, const void* dt_bias, float* g, float* beta, int allow_neg_eigval,
                           void* stream);
/*
 * ccq_gdn_decode_step over the rows ccq_gdn_decode_in_proj leaves: q and k (H K each, at off_q /
 * off_k of each token's row of x, row stride ldx) are L2-normalised per head here (l2_eps) and
 * lambda = sigmoid(lam_w q + lam_b) over the whole q activation (lam_w bf16 [H, H K], lam_b [H]
 * nullable), v is read in place (off_v), g and beta as given (fp32 [B T, H]).  States, position,
 * workspace (ccq_decode_step_workspace_bytes) and the output o bf16 [B, T, H, V] as
 * ccq_gdn_decode_step.  H K <= 2048; x and lam_w 16-byte aligned, ldx and off_q multiples of 8, the v
 * rows 8-byte aligned.  Two kernels, no allocation.
 */
int ccq_gdn_layer_decode_step(const void* x, int64_t ldx, int off_q, int off_k, int off_v, const void* lam_w,
                              const void* lam_b, const float* g, const float* beta, float* state, float* cov_state,
                              float* mean_state, int* position, void* o, void* workspace, int B, int T, int H, int K,
                              int V, int subtract_mean, int enable_ccq, float scale, float l2_eps, void* stream);
int ccq_gdn_decode_step(const void* q, const void* k, const void* v, const float* lambda, const float* gate_w,
                        const float* gate_b, const float* g, const float* beta, float* state, float* cov_state,
                        float* mean_state, int* position, void* o, void* workspace, int B, int T, int H, int K, int V,
                        int subtract_mean, int use_l2norm, int enable_ccq, float scale, void* stream);
int ccq_gla_decode_step(const void* q, const void* k, const void* v, const float* lambda, const float* gate_w,
                        const float* gate_b, const float* gk, float* state, float* cov_state, float* mean_state,
                        int* position, void* o, void* workspace, int B, int T, int H, int K, int V, int subtract_mean,
                        int use_l2norm, float scale, void* stream);

/*
 * Layer prologue: short causal depthwise convolution over time, y = act(bias + sum_w weight[:, w]
 * x[t - (W-1) + w]) with act = SiLU (activation != 0) or none, fused with the per-head L2
 * normalisation of y (y_norm, computed from y rounded to bf16).  Replaces the reference layers'
 * q/k/v ShortConvolution (fla, ccq/gdn/layer.py:266-284, ccq/gla/layer.py:211-229) followed by the
 * operators' l2norm of q and k (ccq/ops/ccq_gdn/fused_chunk.py:43-44): one pass over x instead of
 * conv, activation and normalisation round trips.  x, y, y_norm bf16 [tokens, D] (tokens = B*T;
 * varlen: B == 1 and cu_seqlens [N+1], each sequence restarts the window); weight fp32 [D, W]
 * (tap W-1 on the current token), bias fp32 [D] (nullable); cache_in / cache_out fp32 [N, D, W-1]
 * (the previous W-1 inputs of each sequence; nullable = zeros / not written).  y or y_norm may be
 * null (not written); y_norm needs rstd fp32 [tokens, D / head_dim] (kept for the backward).
 * D % 8 == 0; W in [1, 8]; head_dim a power of two in [8, 512] dividing D.
 * Backward: dy (gradient of y) and / or dy_norm (of y_norm) bf16 -> dx bf16, dweight fp32 [D, W],
 * dbias fp32 [D] (nullable); the cached inputs get no gradient.  workspace:
 * ccq_conv_bwd_workspace_bytes(tokens, D, W).
 */
size_t ccq_conv_bwd_workspace_bytes(int64_t tokens, int D, int W);
int ccq_conv_fwd(const void* x, const float* weight, const float* bias, const float* cache_in,
                 const int64_t* cu_seqlens, void* y, void* y_norm, float* rstd, float* cache_out, int B, int T, int N,
                 int D, int W, int head_dim, int activation, float eps, void* stream);
int ccq_conv_bwd(const void* x, const float* weight, const float* bias, const float* cache_in,
                 const int64_t* cu_seqlens, const void* dy, const void* dy_norm, const float* rstd, void* dx,
                 float* dweight, float* dbias, void* workspace, int B, int T, int N, int D, int W, int head_dim,
                 int activation, void* stream);

/*
 * Layer epilogue: gated RMSNorm y = x / sqrt(mean(x^2) + eps) * weight * silu(g) over rows of dv
 * (the reference's o_norm = fla FusedRMSNormGated, ccq/gdn/layer.py:402-404).  x, g, y, dy, dx,
 * dg bf16 [rows, dv]; weight fp32 [dv] (nullable = ones); rstd fp32 [rows] (written by the
 * forward, read by the backward); dweight fp32 [dv] (nullable) with workspace
 * ccq_gated_rmsnorm_bwd_workspace_bytes(rows, dv).  dv % 8 == 0, dv <= 512.
 */
size_t ccq_gated_rmsnorm_bwd_workspace_bytes(int64_t rows, int dv);
int ccq_gated_rmsnorm_fwd(const void* x, const void* g, const float* weight, void* y, float* rstd, int64_t rows,
                          int dv, float eps, void* stream);
int ccq_gated_rmsnorm_bwd(const void* x, const void* g, const float* weight, const float* rstd, const void* dy,
                          void* dx, void* dg, float* dweight, void* workspace, int64_t rows, int dv, void* stream);
/*
 * The same forward with the gate rows read in place from a wider tensor: gate row r (of dv) at
 * g + (r / g_group) * ldg + (r % g_group) * dv elements -- e.g. the output-gate columns of a decode
 * step's concatenated projection, g_group = heads, ldg = the projection's row width -- so no copy
 * makes them contiguous.  ldg >= g_group * dv and a multiple of 8; g 16-byte aligned.
 */
int ccq_gated_rmsnorm_fwd_strided(const void* x, const void* g, int64_t ldg, int g_group, const float* weight, void* y,
                                  float* rstd, int64_t rows, int dv, float eps, void* stream);

/*
 * Narrow linear map y = x W^T (+ b) with N <= 16 outputs per row, and its backward: the layers'
 * gate projections, nn.Linear in the reference -- erase_lambda_proj on q, a_proj and b_proj on the
 * hidden states (ccq/gdn/layer.py:174, 183-184, 292, 312, 316), the first factor of the low-rank
 * log gate and erase_lambda_proj (ccq/gla/layer.py:131, 162, 237-238).  x bf16 [rows, K] with row
 * stride ldx (a multiple of 8, >= K), weight bf16 [N, K], bias fp32 [N] (nullable), y bf16 [rows, N]
 * (fp32 accumulation, one rounding, as a bf16 GEMM).  Backward: dy bf16 [rows, N]; dx bf16
 * [rows, K] contiguous (nullable: not needed); dweight fp32 [N, K]; dbias fp32 [N] (nullable); the
 * workspace holds ccq_narrow_linear_bwd_workspace_bytes(rows, K, N) bytes.  1 <= N <= 16; K a
 * multiple of 32 in [32, 2016]; x, weight, dx, workspace 16-byte aligned.
 */
size_t ccq_narrow_linear_bwd_workspace_bytes(int64_t rows, int K, int N);
int ccq_narrow_linear_fwd(const void* x, int64_t ldx, const void* weight, const float* bias, void* y, int64_t rows,
                          int K, int N, void* stream);
int ccq_narrow_linear_bwd(const void* x, int64_t ldx, const void* weight, const void* dy, void* dx, float* dweight,
                          float* dbias, void* workspace, int64_t rows, int K, int N, void* stream);

/*
 * Row L2 normalisation y = x / sqrt(sum x^2 + eps) (bf16 rows of D <= 512) and its backward.
 * Replaces fla l2norm as called by the reference (ccq/ops/ccq_gdn/fused_chunk.py:43-44).
 * rstd fp32 [rows] is written by the forward and read by the backward.
 */
int ccq_l2norm_fwd(const void* x, void* y, float* rstd, int64_t rows, int D, float eps, void* stream);
int ccq_l2norm_bwd(const void* x, const float* rstd, const float* dy_f32, const void* dy, void* dx, int64_t rows,
                   int D, void* stream);

/*
 * Kernel timing (measurement facility; no counterpart in the reference).  While enabled, each
 * entry point records a HIP event pair around every launch of its kernels on the caller's
 * stream.  ccq_timing_read waits for the recorded events of `kernel` (names: conv_fwd, conv_bwd,
 * gnorm_fwd, gnorm_bwd, clean_fwd_sum, clean_fwd, clean_bwd_rows, clean_bwd_dq, clean_bwd_gsum,
 * clean_bwd_dk, clean_bwd_gate, gdn_prep, gdn_fwd_state, gdn_fwd_o, gdn_bwd_state, gdn_bwd_dqkw,
 * gdn_bwd_wy, gla_intra, gla_fwd_state, gla_fwd_o, gla_bwd_state, gla_bwd_dv, gla_bwd_dqk,
 * gla_bwd_gk, clean_z_fwd, clean_z_bwd, narrow_fwd, narrow_bwd) and returns the summed
 * milliseconds and the number of launches since the last ccq_timing_reset.  ccq_timing_select
 * restricts the events to the kernel of that name (NULL: every kernel), so that a timed loop carries
 * one event pair per step instead of one per kernel.
 */
int ccq_timing_enable(int on);
int ccq_timing_select(const char* kernel);
int ccq_timing_reset(void);
int ccq_timing_read(const char* kernel, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* CCQ_HIP_H */
