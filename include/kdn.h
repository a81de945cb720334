/*
 * kdn.h -- C ABI of the MI355X (gfx950) Kalman Delta Network scan library (libkdn_hip.so).
 *
 * Every entry point takes raw device pointers, plain sizes, and the hipStream_t to launch
 * on; it allocates no device memory (the caller passes outputs and workspaces, sized by the
 * *_size() queries) and returns 0 on success, KDN_ERR_ARG (-1) on a rejected argument,
 * or a positive hipError_t value from the launch.  Every entry point launches only on
 * `stream` and keeps no state between calls, with two exceptions that share one side stream:
 * kdn_mem_fwd called with its stage bits 0, 1 and 2 together and kdn_mem_bwd called with its
 * stage bits 0 and 1 together may use their overlapped schedules, which also launch on a stream
 * of the library's own and keep that stream, two events and a mutex per device for the life of
 * the process (their declarations below say when and how; calling the stages separately keeps to
 * `stream` alone).  kdn_iso_gain_fwd_noalloc keeps a fixed device array per GPU.  Tensors are
 * dense row-major:
 *   [B,T,H,D]  token-major with heads interleaved (the reference layout),
 *   bf16 arguments are raw uint16_t bit patterns.
 * Dtype flags (*_bf16) select bf16 (1) or fp32 (0) for arguments typed void*.
 * A pointer argument that a declaration does not call optional or nullable must address a device
 * buffer of the documented shape: the library checks sizes, flags and workspace lengths, not the
 * validity of such pointers.
 * g_cumsum is the base-2, chunk-local inclusive prefix of the per-channel log-gate; its
 * chunk length is kdn_mem_chunk_size() (64) for both variants, and it has exactly one
 * consumer (the memory scan), whose backward returns the gate cotangent in natural-log
 * coordinates, not reverse-summed (the frontends' backward performs that sum).
 *
 * The interface each entry point replaces is cited as reference-file:line
 * (ngocbh/kalman-delta-networks, lit_gpt/kdn_ops/).
 */
#ifndef KDN_H_
#define KDN_H_

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Returned for a rejected argument (shape, dtype flag, size, alignment or workspace too small). */
#define KDN_ERR_ARG (-1)
#define KDN_ERR_ARG_VALUE KDN_ERR_ARG /* earlier name, kept as an alias */

/* ---------------------------------------------------------------- iso frontend */
/* _iso_kdn_gate_precumsum_fwd (iso_kdn_chunk.py:1059-1113, kernel :739-813).
 * g_raw [B,T,H,K]; omega_r_raw [B,T,2H] with strides (orr_stride_b, orr_stride_t, 1).
 * Outputs g_cumsum [B,T,H,K] f32, a/omega/r [B,T,H] f32, mu [H] f32. */
int kdn_iso_gate_fwd(const void* g_raw, int g_raw_bf16, const void* omega_r_raw, int orr_bf16, int64_t orr_stride_b,
                     int64_t orr_stride_t, const float* omega_bias, const float* r_bias, const float* A_log,
                     const float* dt_bias, const float* mu_param, float omega_min, float r_min, int B, int T, int H,
                     int K, int chunk, float* g_cumsum, float* a, float* omega, float* r, float* mu,
                     hipStream_t stream);
size_t kdn_iso_gate_bwd_workspace_size(int B, int T, int H, int K, int chunk);
/* _iso_kdn_gate_precumsum_bwd (iso_kdn_chunk.py:1116-1314, kernel :816-1009).  Any cotangent
 * may be NULL (zero); any output may be NULL (not computed).  domega_r_raw is [B,T,2H] dense. */
int kdn_iso_gate_bwd(const void* g_raw, int g_raw_bf16, const void* omega_r_raw, int orr_bf16, int64_t orr_stride_b,
                     int64_t orr_stride_t, const float* omega_bias, const float* r_bias, const float* A_log,
                     const float* dt_bias, const float* mu_param, const float* dg_pre, const float* da,
                     const float* domega, const float* dr, const float* dmu, int B, int T, int H, int K, int chunk,
                     void* dg_raw, void* domega_r_raw, float* dA_log, float* ddt_bias, float* domega_bias,
                     float* dr_bias, float* dmu_param, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- iso gain */
/* Workspace of kdn_iso_gain_fwd / kdn_iso_gain_bwd (per-chunk maps and carries). */
size_t kdn_iso_gain_workspace_size(int B, int T, int H);
/* _iso_kdn_gain_forward (iso_kdn_chunk.py:1598-1664): beta [B,T,H]; p_prev (nullable) saves
 * the incoming covariance per token for the backward; final_precision [B,H] (nullable).  H <= 96.
 * initial_precision is [H] (prec_mode 0, the reference's only form) or [B,H] (prec_mode 1: the
 * final_precision of an earlier segment, for state continuation; the reference has no such mode). */
int kdn_iso_gain_fwd(const float* a, const float* omega, const float* r, const float* initial_precision,
                     int prec_mode, int B, int T, int H, float posterior_scale, float* beta, float* p_prev,
                     float* final_precision, void* workspace, size_t workspace_bytes, hipStream_t stream);
/* Allocation-free variant of kdn_iso_gain_fwd (same arguments and results, bit-identical), with no
 * counterpart in the reference.  For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): the map / carry workspace is a fixed
 * device array inside the library, KDN_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends, so
 * B * H * ceil(T / 64) * 20 bytes must not exceed it (else KDN_ERR_ARG; 4 MiB covers B*H*ceil(T/64) up
 * to 209,715, e.g. B = 182 at H = 18, T = 4096).  It calls no hipMalloc / hipFree.  The array belongs to
 * the current device, and `stream` must run on that device (else KDN_ERR_ARG).  Every call on one GPU
 * shares the array (each call writes all of the part it reads, so no clearing is needed): calls that
 * overlap in time on one GPU, e.g. on two streams, race and must be serialised by the caller.  The
 * first call on each device looks the array's address up (hipGetSymbolAddress) and must be made
 * outside HIP graph capture; later calls may be captured, and every replay of such a graph uses the
 * same array, so it too must not overlap another call on that GPU. */
#define KDN_NOALLOC_SCRATCH_BYTES (4u << 20)
int kdn_iso_gain_fwd_noalloc(const float* a, const float* omega, const float* r, const float* initial_precision,
                             int prec_mode, int B, int T, int H, float posterior_scale, float* beta, float* p_prev,
                             float* final_precision, hipStream_t stream);
/* _iso_kdn_gain_backward (iso_kdn_chunk.py:1817-1893); d_initial_precision is [H] summed over B
 * in a fixed order (deterministic) for prec_mode 0, [B,H] for prec_mode 1.  d_final_precision
 * (nullable; needs final_precision from the forward) is the cotangent of final_precision. */
int kdn_iso_gain_bwd(const float* a, const float* omega, const float* r, const float* initial_precision,
                     int prec_mode, const float* dbeta, const float* p_prev, const float* final_precision,
                     const float* d_final_precision, int B, int T, int H, float posterior_scale, float* da,
                     float* domega, float* dr, float* d_initial_precision, void* workspace, size_t workspace_bytes,
                     hipStream_t stream);

/* ---------------------------------------------------------------- fused iso front */
/* kdn_iso_gate_fwd -> kdn_iso_gain_fwd (and their backwards) as the iso layer composes them
 * (lit_gpt/iso_kdn.py:277-304 over iso_kdn_chunk.py:1317-1392, 1896-1962), chunk 64; no single
 * counterpart in the reference, whose two ops it replaces with the same results.  The gain's prior is
 * the gate's mu unless initial_precision is given ([H] for prec_mode 0, [B,H] for prec_mode 1).
 * Forward: the gate's kernel also writes each chunk's gain map; one gain kernel carries them.  a,
 * omega, r, mu are written (the backward reads them); p_prev and final_precision are nullable.
 * Backward: the gain's reverse chunk maps, then the gate's backward kernel runs the gain's backward
 * per chunk (the a/omega/r cotangents stay on chip).  dbeta is required, dg_pre and
 * d_final_precision (which needs final_precision) are nullable; any gradient output may be NULL.
 * dmu_param is zero when initial_precision is given; d_initial_precision has its shape.  Inputs the
 * vector kernels cannot take (K not tiling the workgroup, unaligned rows) run the two ops' kernels one
 * after the other, same results.  B * T == 0 is the caller's (the forward writes mu only). */
size_t kdn_iso_front_workspace_size(int B, int T, int H, int K);
int kdn_iso_front_fwd(const void* g_raw, int g_raw_bf16, const void* omega_r_raw, int orr_bf16, int64_t orr_stride_b,
                      int64_t orr_stride_t, const float* omega_bias, const float* r_bias, const float* A_log,
                      const float* dt_bias, const float* mu_param, float omega_min, float r_min,
                      const float* initial_precision, int prec_mode, int B, int T, int H, int K, float posterior_scale,
                      float* g_cumsum, float* a, float* omega, float* r, float* mu, float* beta, float* p_prev,
                      float* final_precision, void* workspace, size_t workspace_bytes, hipStream_t stream);
int kdn_iso_front_bwd(const void* g_raw, int g_raw_bf16, const void* omega_r_raw, int orr_bf16, int64_t orr_stride_b,
                      int64_t orr_stride_t, const float* omega_bias, const float* r_bias, const float* A_log,
                      const float* dt_bias, const float* mu_param, const float* initial_precision, int prec_mode,
                      const float* a, const float* omega, const float* r, const float* mu, const float* p_prev,
                      const float* final_precision, const float* dg_pre, const float* dbeta,
                      const float* d_final_precision, int B, int T, int H, int K, float posterior_scale, void* dg_raw,
                      void* domega_r_raw, float* dA_log, float* ddt_bias, float* domega_bias, float* dr_bias,
                      float* dmu_param, float* d_initial_precision, void* workspace, size_t workspace_bytes,
                      hipStream_t stream);

/* ---------------------------------------------------------------- row norms */
/* FLA l2norm_fwd / l2norm_bwd used inside _ChunkKDAPrecumsumFunction (iso_kdn_chunk.py:2203-2204,
 * 2229-2230): y = x * rsqrt(sum x^2 + eps), rstd [rows]. */
int kdn_l2norm_fwd(const void* x, int x_bf16, int64_t rows, int K, float eps, void* y, int y_bf16, float* rstd,
                   hipStream_t stream);
int kdn_l2norm_bwd(const void* x, int x_bf16, const float* rstd, const void* dy, int dy_bf16, int64_t rows, int K,
                   void* dx, hipStream_t stream);
/* _frozen_norm_launch_diag_norm_boundary_forward / _diag_kdn_norm_backward
 * (diag_kdn_chunk.py:358-368, 2079-2159): y = x / max(||x||, 1e-12); q_memory bf16, k_gain f32,
 * k_memory bf16, norms f32 [rows].  Backward sums the k_gain and k_memory cotangents. */
int kdn_diag_norm_fwd(const void* q_raw, const void* k_raw, int x_bf16, int64_t rows, int K, uint16_t* q_memory,
                      float* k_gain, uint16_t* k_memory, float* q_norm, float* k_norm, hipStream_t stream);
int kdn_diag_norm_bwd(const void* q_raw, const void* k_raw, int x_bf16, const float* q_norm, const float* k_norm,
                      const uint16_t* d_q_memory, const float* d_k_gain, const uint16_t* d_k_memory, int64_t rows,
                      int K, void* dq_raw, void* dk_raw, hipStream_t stream);

/* ---------------------------------------------------------------- diag frontend */
/* _diag_kdn_frontend_forward (diag_kdn_chunk.py:2218-2262, kernel :1866-1905). */
int kdn_diag_frontend_fwd(const uint16_t* retention_raw, const uint16_t* omega_raw, const uint16_t* r_raw,
                          const float* A_log, const float* dt_bias, const float* mu_param, int B, int T, int H, int K,
                          int chunk, float* g_cumsum, float* alpha, float* omega, float* r, float* mu,
                          hipStream_t stream);
size_t kdn_diag_frontend_bwd_workspace_size(int B, int T, int H, int K, int chunk);
/* _diag_kdn_frontend_backward (diag_kdn_chunk.py:2265-2423, kernels :1907-2016).  alpha is the
 * forward's output; the vectorised path (K % 8 == 0, 16-byte aligned) recomputes it bit-identically
 * from retention_raw instead of reading it. */
int kdn_diag_frontend_bwd(const uint16_t* retention_raw, const uint16_t* omega_raw, const uint16_t* r_raw,
                          const float* A_log, const float* dt_bias, const float* mu_param, const float* alpha,
                          const float* d_g_cumsum, const float* d_alpha, const float* d_omega, const float* d_r,
                          const float* d_mu, int B, int T, int H, int K, int chunk, uint16_t* d_retention_raw,
                          uint16_t* d_omega_raw, uint16_t* d_r_raw, float* dA_log, float* ddt_bias,
                          float* d_mu_param, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- diag gain */
size_t kdn_diag_gain_workspace_size(int B, int T, int H, int K);
/* _diag_kdn_gain_forward (diag_kdn_chunk.py:2499-2565, kernels :373-494).  initial_precision is
 * [H] (prec_mode 0) or [B,H,K] (prec_mode 1, state continuation).  p_prev [B,T,H,K] and
 * D [B,T,H] (nullable) are saved for the backward; final_precision [B,H,K] nullable. */
int kdn_diag_gain_fwd(const float* k, const float* alpha, const float* omega, const float* r,
                      const float* initial_precision, int prec_mode, int B, int T, int H, int K, float info_scale,
                      float* kappa, float* p_prev, float* D, float* final_precision, void* workspace,
                      size_t workspace_bytes, hipStream_t stream);
/* _diag_kdn_gain_backward (diag_kdn_chunk.py:2569-2683, kernels :496-700) with the fused
 * softplus VJPs of omega_raw and r_raw.  G_scratch is [B,T,H] f32.  d_final_precision
 * (nullable) is the cotangent of final_precision. */
int kdn_diag_gain_bwd(const float* k, const float* alpha, const float* omega, const float* r,
                      const float* initial_precision, int prec_mode, const float* dkappa, const float* p_prev,
                      const float* D, const float* final_precision, const float* d_final_precision,
                      const uint16_t* omega_raw, const uint16_t* r_raw, int B, int T, int H, int K, float info_scale,
                      float* dk, float* dalpha, uint16_t* domega_raw, uint16_t* dr_raw, float* d_initial_precision,
                      float* G_scratch, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- fused diag frontend + gain */
/* The front half of the layer composition (reference lit_gpt/diag_kdn.py:315-345): the gain key
 * k / max(||k||, 1e-12) of _diag_kdn_normalize (diag_kdn_chunk.py:2162-2168), the frontend
 * _diag_kdn_frontend_precumsum_paired (:2471-2495) and the gain _diag_kdn_gain (:2737-2791) in
 * one op whose passes recompute alpha, omega, r and the fp32 key per token instead of passing them
 * through memory.  k_raw [B,T,H,K] (bf16 or f32) with its row norms k_norm [B,T,H] (kdn_diag_norm_fwd
 * writes them; its k_gain output may then be null).  The prior precision is mu = 0.1 +
 * softplus(mu_param) [H] (mu_param non-null, initial_precision null, prec_mode 0) or an explicit
 * initial_precision [H] (prec_mode 0) or [B,H,K] (prec_mode 1).  Outputs g_cumsum and kappa
 * [B,T,H,K] f32; final_precision [B,H,K] nullable; saved (kdn_diag_front_saved_size bytes,
 * nullable for a forward-only call) keeps the precision entering every even token (per 16-token
 * tile, fp32, half of a [B,T,H,K] tensor), from which the backward re-derives the odd tokens'.  K in {64, 128}, chunk a multiple of 16, 16-byte aligned arrays. */
size_t kdn_diag_front_saved_size(int B, int T, int H, int K);
size_t kdn_diag_front_workspace_size(int B, int T, int H, int K);
int kdn_diag_front_fwd(const void* k_raw, int k_bf16, const float* k_norm, const uint16_t* retention_raw,
                       const uint16_t* omega_raw, const uint16_t* r_raw, const float* A_log, const float* dt_bias,
                       const float* mu_param, const float* initial_precision, int prec_mode, int B, int T, int H,
                       int K, int chunk, float info_scale, float* g_cumsum, float* kappa, float* final_precision,
                       float* saved, void* workspace, size_t workspace_bytes, hipStream_t stream);
/* Backward of kdn_diag_front_fwd: _diag_kdn_gain_backward (diag_kdn_chunk.py:2569-2683), the
 * frontend backward (:2265-2423) and the k part of _diag_kdn_norm_backward (:2079-2159), which
 * takes d_k_memory (bf16, nullable) so dk_raw (nullable) is the VJP of dk_gain + dk_memory.
 * d_retention_raw, d_omega_raw, d_r_raw are bf16 and required; dA_log, ddt_bias, d_mu_param
 * (with mu_param) and d_initial_precision (without) are nullable. */
int kdn_diag_front_bwd(const void* k_raw, int k_bf16, const float* k_norm, const uint16_t* retention_raw,
                       const uint16_t* omega_raw, const uint16_t* r_raw, const float* A_log, const float* dt_bias,
                       const float* mu_param, const float* initial_precision, int prec_mode, const float* saved,
                       const float* final_precision, const float* d_g_cumsum, const float* d_kappa,
                       const uint16_t* d_k_memory, const float* d_final_precision, int B, int T, int H, int K,
                       int chunk, float info_scale, void* dk_raw, uint16_t* d_retention_raw, uint16_t* d_omega_raw,
                       uint16_t* d_r_raw, float* dA_log, float* ddt_bias, float* d_mu_param,
                       float* d_initial_precision, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- memory scan */
int kdn_mem_chunk_size(void);
/* Chunk groups the serial state passes of kdn_mem_fwd / kdn_mem_bwd use at this shape (1: a single
 * serial pass; more: the two-level scan that fills the CUs when B*H is small), or KDN_ERR_ARG.  An
 * implementation detail of this library (the reference's state kernel is one serial pass,
 * diag_kdn_chunk.py:720-1229); callers need it only to size nothing -- the *_size() queries already
 * include the group buffers. */
int kdn_mem_state_groups(int B, int T, int H, int K, int V);
size_t kdn_mem_saved_size(int B, int T, int H, int K, int V);
size_t kdn_mem_bwd_workspace_size(int B, int T, int H, int K, int V);
/* Forward of the chunked memory scan: replaces _chunk_kda_fwd_precum (iso_kdn_chunk.py:2037-2086,
 * iso=1, kappa_or_beta = beta [B,T,H]) and _diag_kdn_memory_forward (diag_kdn_chunk.py:3224-3244,
 * iso=0, kappa_or_beta = kappa [B,T,H,K] f32).  q, k (normalised), v are bf16; o is bf16 or f32.
 * initial_state / final_state [B,H,K,V] f32 are nullable (state carry; the reference oracle's
 * initial_memory / output_final_state, iso_kdn_naive.py:376-440).  `saved` receives the
 * intermediates the backward consumes (kdn_mem_saved_size bytes).  `stages` selects kernels
 * (bit 0 intra-chunk WY build, bit 1 serial state pass, bit 2 readout o; -1 = all) so that a
 * caller can launch and time them one at a time; the stages must run in this order.  Bits 0, 1 and
 * 2 in one call with one chunk group (kdn_mem_state_groups == 1) take the overlapped schedule when B*H*V/64
 * leaves at least 32 CUs idle: the sequence runs in two chunk ranges, the second range's intra-chunk
 * build on the library's side stream beside the first range's state pass (made on the first such call
 * outside HIP graph capture; a captured call before that runs the stages in order on `stream`); the
 * side stream waits for `stream`'s earlier work and `stream` for the side build before the second
 * range's pass (an event each; under capture a fork and a join of the graph); the state crosses the
 * ranges in fp32 through `saved`, so every output is bit-identical to the stages in order.  Bits 1 and 2
 * in one call run the state pass with the readout fused.  Bit 3 (with stages >= 0) declares that
 * no backward follows (inference, as under torch.no_grad): the intermediates only the backward
 * reads are then not written, and `saved` is scratch for this call alone.  A caller that keeps no
 * `saved` from a training forward (the reference's policy: it re-runs recompute_w_u_fwd and the state
 * forward in its backward, iso_kdn_chunk.py:2101-2140, diag_kdn_chunk.py:3271-3277) rebuilds it for
 * kdn_mem_bwd with bit 0, then bit 1 alone (the state pass without the readout; o and final_state
 * may be null): the same kernels on the same inputs write the same intermediates.
 * q_rstd / k_rstd [B,T,H] f32 (both or neither, outputs): the in-op L2 norm of
 * _chunk_kda_precumsum_paired (iso_kdn_chunk.py:2203-2204).  Given, q and k are the raw bf16 inputs;
 * the scan consumes y = bf16(x / sqrt(sum x^2 + 1e-6)) per row, exactly what kdn_l2norm_fwd (eps 1e-6)
 * writes, and the rows' rstd are written here for kdn_mem_bwd. */
int kdn_mem_fwd(const uint16_t* q, const uint16_t* k, const float* kappa_or_beta, int iso, const uint16_t* v,
                const float* g_cumsum, int B, int T, int H, int K, int V, float scale, const float* initial_state,
                void* saved, size_t saved_bytes, float* final_state, void* o, int o_bf16, float* q_rstd,
                float* k_rstd, int stages, hipStream_t stream);
/* Backward: replaces _chunk_kda_bwd_precum (iso_kdn_chunk.py:2089-2187) and
 * _DiagKdnMemoryFunction.backward (diag_kdn_chunk.py:3258-3312).  dq, dk, dv bf16; dkappa
 * [B,T,H,K] f32 (diag) or dbeta [B,T,H] f32 (iso); dg [B,T,H,K] f32 in natural-log coordinates,
 * not reverse-summed.  d_final_state / d_initial_state nullable.
 * q_rstd / k_rstd [B,T,H] f32 (both or neither): the in-op L2 norm of _chunk_kda_precumsum_paired
 * (iso_kdn_chunk.py:2203-2204, 2229-2230), as kdn_mem_fwd wrote them.  Given, q and k are the raw bf16
 * inputs x the forward took, the kernels form the operand y = bf16(x rstd) again, and dq, dk are
 * returned for x: the norm's backward dx = rstd (dy - y (y . dy)) is applied to the fp32 dy in the
 * kernel (kdn_l2norm_bwd takes the bf16-rounded dy instead; the two agree to bf16 rounding).
 * `stages`: bit 0 reverse state pass, bit 1 the chunk-parallel backward, bits 2 and 3 the exact
 * path's solves and gradients for the chunks outside the factored range (-1 = all, in this order).
 * Bits 2 and 3 in one call run as one launch (each such chunk's solves, gradients and, with q_rstd, the
 * norm's backward of its rows in one workgroup), bit-identical to a call with bit 2 and then one with
 * bit 3.
 * Bits 0 and 1 in one call, with one chunk group (kdn_mem_state_groups == 1), at least 16 chunks
 * and at least 32 CUs the pass leaves idle (the overlapped schedule): the reverse pass runs in two
 * segments, and chunk-backward work of the first segment's chunks runs beside the second on a
 * stream of the library's own.  That stream (non-blocking, default priority) and two events that
 * order it against `stream` are created per device on the first such call made outside HIP graph
 * capture, and kept until the process ends; a first call inside a capture takes the serial
 * schedule.  The side stream's launch starts with a one-wave kernel that waits 3 us on the
 * device's constant wall clock (a bounded wait, no memory access), so that the pass's second
 * segment is dispatched onto the CUs the first segment frees before the side work takes them.
 * Under capture the side stream forks from and joins the capturing stream.  The call returns with
 * `stream` ordered after both streams' work, and the results are bit-identical to separate calls
 * (bit 0, then bit 1), which launch on `stream` alone.  Calls on one device serialise their
 * enqueue on a library mutex. */
int kdn_mem_bwd(const uint16_t* q, const uint16_t* k, const float* kappa_or_beta, int iso, const float* g_cumsum,
                int B, int T, int H, int K, int V, float scale, const void* d_o, int do_bf16,
                const float* d_final_state, const void* saved, size_t saved_bytes, void* workspace,
                size_t workspace_bytes, uint16_t* dq, uint16_t* dk, float* dkappa, float* dbeta, uint16_t* dv,
                float* dg, float* d_initial_state, const float* q_rstd, const float* k_rstd, int stages,
                hipStream_t stream);
/* One token of the memory recurrence with a carried state (decode).  The reference has no step
 * kernel (it refuses caching for KDN layers, model.py:104,184); this is the tokenwise recurrence
 * of iso_kdn_naive.py:308-332 / diag_kdn_naive.py:479-500 on the scan's state layout:
 * S = 2^g (.) S; delta = v - S^T k; S += kappa delta^T; o = scale S^T q.  q, k [B,H,K] and
 * v [B,H,V] share a dtype (qkv_bf16: bf16, else f32); g [B,H,K] f32 is the token's base-2 log
 * decay (kdn_mem_fwd's g_cumsum at T = 1).  iso = 1: kappa_or_beta is beta [B,H] and q, k are
 * L2-normalised inside (x rsqrt(sum x^2 + 1e-6)), kappa = beta k_hat; iso = 0: kappa [B,H,K]
 * f32 and q, k are used as given.  state [B,H,K,V] f32 is read and overwritten in place;
 * o [B,H,V] (o_bf16: bf16, else f32).  K, V in {64, 128}; state 16-byte aligned. */
int kdn_mem_step(const void* q, const void* k, const float* kappa_or_beta, int iso, const void* v, int qkv_bf16,
                 const float* g, int B, int H, int K, int V, float scale, float* state, void* o, int o_bf16,
                 hipStream_t stream);
/* One token of the whole Kalman step with a carried state (decode): the single-token gain of
 * _iso_kdn_gain_forward / _diag_kdn_gain_forward (iso_kdn_naive.py:200-251, diag_kdn_naive.py:
 * 217-276) from the carried precision, then kdn_mem_step's memory update, in one launch.  No
 * counterpart in the reference (it refuses caching for KDN layers, model.py:104,184).
 * iso = 1: gain_a = a [B,H] (mean alpha^2), omega, r [B,H], precision [B,H], unit keys as on the
 * production path: z = a/c + omega, beta = z / (r + z), c' = (r + s z) / (r z), s = info_scale / K.
 * iso = 0: gain_a = alpha [B,H,K] (the gain's unclamped alpha), omega [B,H,K], r [B,H],
 * k_gain [B,H,K] f32 (nullable: k), precision [B,H,K]: p_hat = alpha^2 / c + omega,
 * kappa = p_hat k_gain / (r + sum p_hat k_gain^2), c' = (1 + s k_gain^2 p_hat / r) / p_hat,
 * s = info_scale.  precision_out must not alias precision_in.  Other arguments as kdn_mem_step. */
int kdn_kalman_step(const void* q, const void* k, const void* v, int qkv_bf16, const float* g, const float* gain_a,
                    const float* omega, const float* r, const float* k_gain, const float* precision_in,
                    float* precision_out, int iso, int B, int H, int K, int V, float scale, float info_scale,
                    float* state, void* o, int o_bf16, hipStream_t stream);
/* Decode projections: y[m, :] = W x[m, :] (+ bias) for M <= 8 rows, the one-token-per-sequence
 * form of the layers' nn.Linear products (the reference runs every projection as a torch GEMM,
 * e.g. iso_kdn.py:277-312, model.py:415-464; this is no port of one).  W [N,K] bf16 row-major,
 * bias [N] bf16 (nullable), fp32 accumulation; x [M,K] bf16 (x_bf16) or f32 with row stride
 * x_row_stride elements, y [M,N] in x's dtype with row stride y_row_stride.  K % 8 == 0; W and
 * the rows of x 16-byte aligned.  gated != 0 fuses the SwiGLU gate of model.py:467-470 (the packed
 * decode form): W [2N,K] = [w1; w2], bias [2N], y[m, n] = silu(w1 x + b1)[n] * (w2 x + b2)[n]. */
int kdn_gemv(const void* x, int x_bf16, int64_t x_row_stride, const uint16_t* W, const uint16_t* bias, int M, int N,
             int K, int gated, void* y, int64_t y_row_stride, hipStream_t stream);

/* ---------------------------------------------------------------- language-model loss */
/* Fused cross-entropy forward, one row of logits per token.  Replaces cross_entropy_fwd_kernel
 * (lit_gpt/fused_cross_entropy.py:29-100) as launched by CrossEntropyLoss.forward (:156-260).
 * logits [n_rows, n_cols] with row stride logits_row_stride elements, logits_dtype 0 f32, 1 bf16,
 * 2 f16; labels [n_rows] int64 (labels_i64) or int32.  Per row: lse = log sum exp(logit_scale x)
 * (read from lse when precomputed_lse, which needs smoothing 0 and logit_scale 1); loss = lse -
 * (1 - smoothing) x_label - smoothing sum(x) / total_classes + lse_square_scale lse^2 (z_loss, the
 * last term); 0 on rows whose label is ignore_index; a label outside this slice's classes
 * [class_start_idx, class_start_idx + n_cols) keeps only the smoothing term.  split != 0 is the
 * vocabulary-split mode: lse is this slice's, the loss leaves out lse and the z-loss, and z_losses
 * is not written (nullable).  losses, lse, z_losses [n_rows] f32. */
int kdn_xent_fwd(const void* logits, int logits_dtype, int64_t logits_row_stride, const void* labels, int labels_i64,
                 int n_rows, int n_cols, float smoothing, float logit_scale, float lse_square_scale,
                 int64_t ignore_index, int64_t total_classes, int64_t class_start_idx, int split,
                 int precomputed_lse, float* losses, float* lse, float* z_losses, hipStream_t stream);
/* Fused cross-entropy backward.  Replaces cross_entropy_bwd_kernel (fused_cross_entropy.py:103-150)
 * as launched by CrossEntropyLoss.backward (:262-294): dlogits[r, c] = dlosses[r] logit_scale
 * (p (1 + 2 lse_square_scale lse) - [c == label](1 - smoothing) - smoothing / total_classes),
 * p = exp(logit_scale x - lse[r]); 0 on ignored rows.  dlogits has logits' dtype and may be logits
 * itself (in-place backward, same row stride); dlosses [n_rows] f32 with stride dlosses_stride. */
int kdn_xent_bwd(void* dlogits, int64_t dlogits_row_stride, const float* dlosses, int64_t dlosses_stride,
                 const void* logits, int logits_dtype, int64_t logits_row_stride, const float* lse,
                 const void* labels, int labels_i64, int n_rows, int n_cols, float smoothing, float logit_scale,
                 float lse_square_scale, int64_t ignore_index, int64_t total_classes, int64_t class_start_idx,
                 hipStream_t stream);

/* ---------------------------------------------------------------- layer frontends */
/* Depthwise causal short convolution with SiLU, fixed length, width W = 4, no bias:
 * y[b,t,d] = silu(sum_j w[d,j] x[b,t-3+j,d]), x before t = 0 is 0, computed in f32 and rounded to
 * x's dtype.  Replaces FLA causal_conv1d(x, weight, activation="silu") as called by
 * lit_gpt/diag_kdn.py:75-96 and per q|k|v group by qkv_causal_conv1d (iso_kdn_chunk.py:47-478,
 * forward kernel :56-120).  x [B,T,D] and y [B,T,D] have unit channel stride and the given batch /
 * time strides (elements; multiples of 8, so packed q|k|v views need no copy); weight [D,W] dense.
 * D % 8 == 0. */
int kdn_short_conv_fwd(const void* x, int x_bf16, int64_t x_stride_b, int64_t x_stride_t, const void* weight,
                       int w_bf16, int B, int T, int D, int W, void* y, int64_t y_stride_b, int64_t y_stride_t,
                       hipStream_t stream);
/* One token of the short convolution from carried inputs (decoding; no reference counterpart: the
 * reference refuses caching, model.py:104,184).  x [B,1,D] with batch stride x_stride_b, tail [B,3,D]
 * (the 3 earlier inputs, x's dtype, row stride D, batch stride tail_stride_b), y [B,1,D]:
 * y = silu(sum_j w[d,j] [tail_0, tail_1, tail_2, x]_j), equal to kdn_short_conv_fwd over the 4 rows;
 * then the tail is advanced in place to [tail_1, tail_2, x].  x, tail, y, weight 16-byte aligned. */
int kdn_short_conv_step(const void* x, int x_bf16, int64_t x_stride_b, void* tail, int64_t tail_stride_b,
                        const void* weight, int w_bf16, int B, int D, void* y, int64_t y_stride_b,
                        hipStream_t stream);
/* Workspace of kdn_short_conv_bwd when dweight is requested: f32 partials per (b, 64-token block). */
size_t kdn_short_conv_bwd_workspace_size(int B, int T, int D);
/* Backward (iso_kdn_chunk.py:127-254, 379-437): g = dy * silu'(y) with the preactivation y recomputed
 * (rounded to x's dtype when round_preactivation, as the reference's raw_y buffer is),
 * dx[t] = sum_j w[j] g[t+3-j], dweight[d,j] = sum_{b,t} g[t] x[t-3+j] summed in a fixed order and
 * stored in weight's dtype.  dy has x's dtype and may be NULL (zero); dx / dweight may be NULL. */
int kdn_short_conv_bwd(const void* x, int x_bf16, int64_t x_stride_b, int64_t x_stride_t, const void* weight,
                       int w_bf16, const void* dy, int64_t dy_stride_b, int64_t dy_stride_t, int B, int T, int D,
                       int W, int round_preactivation, void* dx, int64_t dx_stride_b, int64_t dx_stride_t,
                       void* dweight, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* RMS norm over wide dense rows (the model's block norm FusedRMSNorm, reference
 * lit_gpt/rmsnorm.py:1182-1216, no residual / dropout): y = x rsqrt(mean(x^2) + eps) * weight, f32 math,
 * y in x's dtype, rstd [rows] f32 (nullable).  D % 8 == 0, D <= 8192. */
int kdn_rms_norm_fwd(const void* x, int x_bf16, const void* weight, int w_bf16, int64_t rows, int D, float eps,
                     void* y, float* rstd, hipStream_t stream);
/* Workspace of kdn_rms_norm_bwd when dweight is requested (f32 partials). */
size_t kdn_rms_norm_bwd_workspace_size(int64_t rows, int D);
/* Backward: dx (x's dtype), dweight (weight's dtype, fixed-order sum); dy has x's dtype. */
int kdn_rms_norm_bwd(const void* x, int x_bf16, const void* weight, int w_bf16, const float* rstd, const void* dy,
                     int64_t rows, int D, void* dx, void* dweight, void* workspace, size_t workspace_bytes,
                     hipStream_t stream);

/* Gated RMS norm over the last dimension D of dense rows:
 * y = x rsqrt(mean(x^2) + eps) * weight * act(g), act = sigmoid (activation 0) or g sigmoid(g)
 * (activation 1, "swish"); f32 math, y in x's dtype, rstd [rows] f32 saved (nullable).
 * Replaces FLA FusedRMSNormGated as the layers' o_norm (lit_gpt/iso_kdn.py:192-196,305-312;
 * lit_gpt/diag_kdn.py:216-219,346).  D % 8 == 0, D / 8 a power of two <= 64. */
int kdn_rms_norm_gated_fwd(const void* x, int x_bf16, const void* g, int g_bf16, const void* weight, int w_bf16,
                           int64_t rows, int D, float eps, int activation, void* y, float* rstd, hipStream_t stream);
/* Workspace of kdn_rms_norm_gated_bwd when dweight is requested: f32 per-block partials. */
size_t kdn_rms_norm_gated_bwd_workspace_size(int64_t rows, int D);
/* Backward: dx (x's dtype), dg (g's dtype), dweight (weight's dtype, summed over rows in a fixed
 * order); dy has x's dtype; any output may be NULL. */
int kdn_rms_norm_gated_bwd(const void* x, int x_bf16, const void* g, int g_bf16, const void* weight, int w_bf16,
                           const float* rstd, const void* dy, int64_t rows, int D, int activation, void* dx,
                           void* dg, void* dweight, void* workspace, size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KDN_H_ */
