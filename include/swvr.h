/*
 * swvr.h — C ABI of the MI355X (gfx950) softmax-weighted embedding readout.
 *
 *   S   = logit_scale * h @ W^T + bias          h [N,K], W [V,K], bias [V] (optional)
 *   O   = softmax(S) @ E                          E [V,D]            -> O   [N,D] fp32
 *   LSE = logsumexp(S)                                                -> lse [N]   fp32
 *
 * and the gradients of (O, LSE) with respect to h, W, E and bias.
 *
 * The two compute entry points replace the bodies of the reference's custom ops
 *   swvr::chunked_fwd   swvr/chunked.py:157-161  (-> _forward,  swvr/chunked.py:82-105)
 *   swvr::chunked_bwd   swvr/chunked.py:170-178  (-> _backward, swvr/chunked.py:108-151)
 * The Python autograd.Function of the package calls them through ctypes; see
 * swvr_amd/_lib.py for the binding.
 *
 * Conventions
 *  - Every pointer is a device pointer on the current HIP device.  The caller
 *    allocates every output and the workspace; the library never allocates.
 *  - Work is enqueued on `stream` (a hipStream_t passed as void*); no call
 *    synchronises the host, except swvr_timing_collect.
 *  - Row-major operands with unit stride in the last dimension.  h, W and E
 *    have row strides ldh, ldw, lde (in elements).  K, ldh and ldw must be
 *    multiples of 8 and h, W 16-byte aligned (the host pads odd K with zero
 *    columns); K is at most 2^21.  D and lde are unrestricted.
 *  - The operand dtype (SWVR_BF16, SWVR_F16, SWVR_F32) is the compute dtype of
 *    the matrix products: the reference's `cdt` (swvr/api.py:8-11).  Products
 *    accumulate in fp32; scores, softmax state, O and LSE are fp32.
 *  - Return value: SWVR_OK, or a negative SWVR_E* code; swvr_last_error()
 *    then holds a message (thread-local).
 */
#ifndef SWVR_H_
#define SWVR_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SWVR_ABI_VERSION 1

/* dtype tags */
#define SWVR_BF16 0
#define SWVR_F16 1
#define SWVR_F32 2

/* status codes */
#define SWVR_OK 0
#define SWVR_EINVAL (-1)      /* bad shape, stride, alignment or pointer  */
#define SWVR_EDTYPE (-2)      /* unsupported dtype or D for this dtype    */
#define SWVR_EHIP (-3)        /* a HIP runtime call failed                */
#define SWVR_EWORKSPACE (-4)  /* workspace too small                      */

/* Version of this ABI (SWVR_ABI_VERSION).  No reference counterpart. */
int swvr_abi_version(void);

/* Message for the last failed call on this thread ("" if none).
 * No reference counterpart (the reference raises Python exceptions,
 * swvr/api.py:14-22). */
const char* swvr_last_error(void);

/* Largest embedding width D supported for a dtype: SWVR_MAX_D for bf16, f16
 * and f32, 0 for an unknown tag.  The reference has no cap (above 256 its
 * fused kernels hand over to its torch path, swvr/triton_kernels.py:27,
 * 121-123); here a forward with D above 256 (128 for f32) runs in passes over
 * slices of E's columns, and the backward streams E and gO in D-slices.  The
 * e4m3 entry points take D <= 128. */
#define SWVR_MAX_D 65536
int64_t swvr_max_d(int dtype);

/* Workspace bytes swvr_fwd needs for this shape. */
size_t swvr_fwd_workspace_size(int dtype, int64_t N, int64_t K, int64_t V, int64_t D);

/* Forward: O [N,D] (row stride D) and lse [N], both fp32.
 * Replaces swvr::chunked_fwd (swvr/chunked.py:157-161, 82-105).  bias may be
 * NULL; it is fp32 [V] and may hold -inf (masked vocabulary).  A row whose
 * scores are all -inf gets O = NaN and lse = -inf, as the reference does. */
int swvr_fwd(int dtype, int64_t N, int64_t K, int64_t V, int64_t D,
             const void* h, int64_t ldh, const void* W, int64_t ldw,
             const void* E, int64_t lde, const float* bias, float logit_scale,
             float* O, float* lse, void* workspace, size_t workspace_bytes,
             void* stream);

/* swvr_fwd with h and W stored in their own dtypes: h_dtype / w_dtype is the
 * compute dtype, or SWVR_F32 under a 2-byte compute dtype.  fp32 rows are
 * rounded to the compute dtype as they are packed, so autocast with fp32
 * weights needs no separate cast of W or h (the reference casts
 * W[v0:v1].to(cdt) per chunk, swvr/chunked.py:92,123,146).  The alignment
 * contract is the same, in elements.  Workspace: swvr_fwd_workspace_size. */
int swvr_fwd_mixed(int dtype, int h_dtype, int w_dtype, int64_t N, int64_t K, int64_t V, int64_t D,
                   const void* h, int64_t ldh, const void* W, int64_t ldw,
                   const void* E, int64_t lde, const float* bias, float logit_scale,
                   float* O, float* lse, void* workspace, size_t workspace_bytes, void* stream);

/* swvr_fwd_mixed for a weighted loss (swvr/api.py:53-66, which multiplies each
 * token's loss by weight[n]): only the tokens with weight[n] != 0 (fp32 [N]; a
 * NaN weight counts as non-zero) are computed; the O rows and lse of the others
 * are written as 0.  Their loss term weight[n] * (mean_d (O - target)^2 +
 * z * lse^2) is then 0 * finite = 0, as the reference's is, except where the
 * reference's is 0 * NaN; those rows are computed too:
 *   - a zero-weight token whose h row holds an infinity or a NaN;
 *   - every token, when W, E or the bias holds a NaN or +inf, every bias entry
 *     is -inf, V = 0, or logit_scale is not finite.
 * (A zero-weight token whose fp32 scores overflow from finite inputs is the one
 * case left: its reference loss is NaN, here 0 * finite.)  O and lse of the
 * computed tokens equal swvr_fwd_mixed's to fp32 rounding (the vocabulary is
 * split differently over the fewer tokens).  No reference counterpart: the
 * reference computes every token's readout before weighting the loss.
 * Workspace: swvr_fwd_active_workspace_size. */
size_t swvr_fwd_active_workspace_size(int dtype, int64_t N, int64_t K, int64_t V, int64_t D);
int swvr_fwd_active(int dtype, int h_dtype, int w_dtype, int64_t N, int64_t K, int64_t V, int64_t D,
                    const void* h, int64_t ldh, const void* W, int64_t ldw,
                    const void* E, int64_t lde, const float* bias, float logit_scale,
                    const float* weight, float* O, float* lse,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Vocabulary-parallel forward, one shard.  With W, E and bias holding V rows of
 * the vocabulary (a shard), writes the shard's softmax partials, fp32:
 *   m[n]     = max_v S[n,v]
 *   l[n]     = sum_v exp(S[n,v] - m[n])
 *   acc[n,:] = sum_v exp(S[n,v] - m[n]) E[v,:]      (row stride D, unnormalised)
 * with m = -inf, l = 0, acc = 0 for a row whose shard scores are all -inf.
 * Each rank of a vocabulary-parallel job runs it on its shard, the partials are
 * all-gathered (N (D + 2) floats per shard) and swvr_combine merges them; the
 * backward then runs swvr_bwd on each shard with the merged O and lse and sums
 * gh over the shards.  Workspace: swvr_fwd_workspace_size of the shard.
 * No reference counterpart: it is the shard-local half of the reference's
 * online softmax (swvr/chunked.py:82-105). */
int swvr_fwd_partial(int dtype, int64_t N, int64_t K, int64_t V, int64_t D,
                     const void* h, int64_t ldh, const void* W, int64_t ldw,
                     const void* E, int64_t lde, const float* bias, float logit_scale,
                     float* m, float* l, float* acc, void* workspace, size_t workspace_bytes,
                     void* stream);

/* Merge S shards' partials in shard order (deterministic): m, l are [S][N],
 * acc is [S][N][D] (each shard's swvr_fwd_partial output, stacked), into
 * O [N,D] and lse [N], as swvr_fwd would give for the whole vocabulary:
 * O = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M), lse = M + log(sum),
 * M = max_s m_s (the -inf guard of swvr/chunked.py:98-99 included).
 * No reference counterpart (the vocabulary-parallel combine). */
int swvr_combine(int64_t S, int64_t N, int64_t D, const float* m, const float* l,
                 const float* acc, float* O, float* lse, void* stream);

/* Workspace bytes swvr_bwd needs.  `chunk` is the vocabulary staging chunk
 * (the reference's chunk_size, swvr/chunked.py:120): the backward stages
 * dS for `chunk` vocabulary rows at a time, so this is O(N * chunk). */
size_t swvr_bwd_workspace_size(int dtype, int64_t N, int64_t K, int64_t V, int64_t D,
                               int64_t chunk, int need_gh);

/* Backward.  Replaces swvr::chunked_bwd (swvr/chunked.py:170-178, 108-151).
 * Inputs: the forward's operands, O [N,D] fp32 (row stride D), lse [N] fp32,
 * gO [N,D] fp32 (row stride D) and glse [N] fp32.
 * Outputs (any may be NULL = gradient not needed, chunked.py:197-198):
 *   gh [N,K] (row stride K) in gh_dtype, gW [V,K] (row stride K) in gW_dtype,
 *   gE [V,D] (row stride D) in gE_dtype, gb [V] fp32.
 * Gradients are deterministic: no atomics, fixed reduction order. */
int swvr_bwd(int dtype, int64_t N, int64_t K, int64_t V, int64_t D,
             const void* h, int64_t ldh, const void* W, int64_t ldw,
             const void* E, int64_t lde, const float* bias, float logit_scale,
             const float* O, const float* lse, const float* gO, const float* glse,
             int64_t chunk,
             void* gh, int gh_dtype, void* gW, int gW_dtype, void* gE, int gE_dtype,
             float* gb, void* workspace, size_t workspace_bytes, void* stream);

/* swvr_bwd with h and W stored in their own dtypes, as swvr_fwd_mixed.  With
 * an fp32 W the workspace also holds two chunks' rows of W in the compute
 * dtype (the dh product reads W rows): size it with
 * swvr_bwd_workspace_size_mixed. */
size_t swvr_bwd_workspace_size_mixed(int dtype, int w_dtype, int64_t N, int64_t K, int64_t V, int64_t D,
                                     int64_t chunk, int need_gh);
int swvr_bwd_mixed(int dtype, int h_dtype, int w_dtype, int64_t N, int64_t K, int64_t V, int64_t D,
                   const void* h, int64_t ldh, const void* W, int64_t ldw,
                   const void* E, int64_t lde, const float* bias, float logit_scale,
                   const float* O, const float* lse, const float* gO, const float* glse,
                   int64_t chunk,
                   void* gh, int gh_dtype, void* gW, int gW_dtype, void* gE, int gE_dtype,
                   float* gb, void* workspace, size_t workspace_bytes, void* stream);

/* The readout in fp64 (no reference counterpart as an entry point: the
 * reference computes fp64 inputs in fp64 on its torch path and returns fp64
 * O / lse, swvr/chunked.py:26-27, 62-63).  Same quantities as swvr_fwd /
 * swvr_bwd with every operand, bias, output and gradient fp64 and every
 * stride in elements (no alignment or K-multiple rules; K < 2^22).  The
 * vocabulary is processed `chunk` rows at a time, as the reference's chunk
 * size: the workspace is O(N * chunk).  Gradients are deterministic. */
size_t swvr_fwd_f64_workspace_size(int64_t N, int64_t V, int64_t D, int64_t chunk);
int swvr_fwd_f64(int64_t N, int64_t K, int64_t V, int64_t D, const double* h, int64_t ldh, const double* W,
                 int64_t ldw, const double* E, int64_t lde, const double* bias, double logit_scale, int64_t chunk,
                 double* O, double* lse, void* workspace, size_t workspace_bytes, void* stream);
size_t swvr_bwd_f64_workspace_size(int64_t N, int64_t V, int64_t D, int64_t chunk);
int swvr_bwd_f64(int64_t N, int64_t K, int64_t V, int64_t D, const double* h, int64_t ldh, const double* W,
                 int64_t ldw, const double* E, int64_t lde, const double* bias, double logit_scale, const double* O,
                 const double* lse, const double* gO, const double* glse, int64_t chunk, double* gh, double* gW,
                 double* gE, double* gb, void* workspace, size_t workspace_bytes, void* stream);

/* Tiling the backward uses for this shape (no reference counterpart; for
 * tests and tuning).  Writes up to n_out of: [0] BM, the token block of the
 * scores kernel; [1] BV, its vocabulary tile; [2] G, the token groups a
 * vocabulary tile's token blocks are split over (one workgroup per group, so a
 * workgroup walks ceil(active token blocks / G) blocks); [3] C, the vocabulary
 * rows per chunk; [4] the number of chunks; [5] DP, the padded embedding
 * width; [6] the scores kernel: 1 the narrow-embedding kernel (side tiles
 * carried by its K ring), 2 the wide-embedding kernel (gO and E streamed as
 * D-slices; dE formed by the gradient GEMM launch), 0 the general one.
 * Returns the number of fields (7) or a negative SWVR_E* code. */
int swvr_bwd_tiling(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, int64_t chunk,
                    int64_t* out, int n_out);

/* Forward with h and W in OCP e4m3 (fp8; opt-in, outside the reference's
 * precision policy, which has no fp8 path).  h [N][ldh] and W [V][ldw] hold
 * e4m3 bytes: h = h_scale[0] * h_e4m3 and W[v] = w_scale[v] * W_e4m3[v]
 * (fp32 scales on the device: one for h, one per vocabulary row of W).  The
 * scores S = logit_scale * h_scale * w_scale[v] * (h_e4m3 . W_e4m3[v]) + bias
 * accumulate in fp32; P is rounded to bf16 for P.E as in the bf16 forward; E
 * is bf16 [V][lde]; O and lse are fp32.  K, ldh and ldw are multiples of 16
 * (bytes), h and W 16-byte aligned; D <= 128.  Its backward, which
 * recomputes the same scores, is swvr_bwd_fp8. */
size_t swvr_fwd_fp8_workspace_size(int64_t N, int64_t K, int64_t V, int64_t D);
int swvr_fwd_fp8(int64_t N, int64_t K, int64_t V, int64_t D, const void* h, int64_t ldh, const float* h_scale,
                 const void* W, int64_t ldw, const float* w_scale, const void* E, int64_t lde, const float* bias,
                 float logit_scale, float* O, float* lse, void* workspace, size_t workspace_bytes, void* stream);

/* Backward of the e4m3 forward (opt-in; no reference counterpart): swvr_bwd
 * for bf16 h, W and E, with the scores recomputed from the e4m3 operands the
 * forward used (hq [N][ldhq], Wq [V][ldwq], K8 bytes per row, and their
 * scales), so P is the forward's.  The gradient products use the bf16 h and W:
 * gh = s dS W, gW = s dS^T h, as swvr_bwd.  K8 >= K, K8, ldhq and ldwq
 * multiples of 16; D <= 128. */
size_t swvr_bwd_fp8_workspace_size(int64_t N, int64_t K, int64_t K8, int64_t V, int64_t D, int64_t chunk,
                                   int need_gh);
int swvr_bwd_fp8(int64_t N, int64_t K, int64_t V, int64_t D, const void* h, int64_t ldh, const void* W, int64_t ldw,
                 const void* E, int64_t lde, const float* bias, float logit_scale, const void* hq, int64_t K8,
                 int64_t ldhq, const float* h_scale, const void* Wq, int64_t ldwq, const float* w_scale,
                 const float* O, const float* lse, const float* gO, const float* glse, int64_t chunk, void* gh,
                 int gh_dtype, void* gW, int gW_dtype, void* gE, int gE_dtype, float* gb, void* workspace,
                 size_t workspace_bytes, void* stream);

/* OCP e4m3 quantisation of h or W for swvr_fwd_fp8 (no reference
 * counterpart).  x is [R][ld] in x_dtype (SWVR_BF16, SWVR_F16, SWVR_F32);
 * out receives [R][ldo] e4m3 bytes (16-byte aligned, ldo a multiple of 16),
 * columns K .. Kp-1 zero.  per_row != 0: scale[r] = max(amax of row r, 1e-30)
 * * fl(1/448) (W); per_row == 0: one scale[0] from the amax of the whole
 * matrix (h), which needs swvr_quantize_e4m3_workspace_size(R, 0) bytes of
 * workspace.  out = x / scale rounded to nearest even: the same bytes and
 * scales as torch's (x / (amax.clamp_min(1e-30) / 448)).to(float8_e4m3fn). */
size_t swvr_quantize_e4m3_workspace_size(int64_t R, int per_row);
int swvr_quantize_e4m3(int64_t R, int64_t K, int64_t Kp, const void* x, int64_t ld, int x_dtype, int per_row,
                       void* out, int64_t ldo, float* scale, void* workspace, size_t workspace_bytes, void* stream);

/* MSE readout loss over the forward's outputs, the loss of
 * softmax_readout_mse (replaces swvr/api.py:53-66, which the reference
 * evaluates as a chain of torch ops):
 *   per_tok[n] = w[n] * (mean_d (O[n,d] - target[n,d])^2 + z_loss_weight * lse[n]^2)
 * reduction SWVR_REDUCE_NONE writes per_tok into out [N]; SWVR_REDUCE_SUM
 * writes sum_n per_tok[n] into out [1]; SWVR_REDUCE_MEAN writes that sum
 * divided by sum_n w[n] (by N without weights).  The sum is taken in a fixed
 * order, so it is the same on every run.  scale [1] (SUM / MEAN only;
 * nullable) receives c, the factor the sum is multiplied by (1, 1/sum w or
 * 1/N).  gO [N][D] and glse [N] (both or neither) receive the derivatives of
 * the loss divided by c (and by the incoming gradient):
 *   gO[n,d] = w[n] * (2/D) * (O[n,d] - target[n,d]),  glse[n] = w[n] * 2 z lse[n].
 * O is dense fp32 [N][D]; target is [N][ldt] in target_dtype (SWVR_BF16,
 * SWVR_F16 or SWVR_F32), unit column stride; weight is fp32 [N] or NULL.
 * The workspace holds the per-workgroup partial sums
 * (swvr_mse_loss_workspace_size; 0 bytes for SWVR_REDUCE_NONE is enough). */
#define SWVR_REDUCE_NONE 0
#define SWVR_REDUCE_SUM 1
#define SWVR_REDUCE_MEAN 2
size_t swvr_mse_loss_workspace_size(int64_t N);
int swvr_mse_loss(int64_t N, int64_t D, const float* O, const float* lse, const void* target, int target_dtype,
                  int64_t ldt, const float* weight, float z_loss_weight, int reduction, float* out, float* scale,
                  float* gO, float* glse, void* workspace, size_t workspace_bytes, void* stream);

/* swvr_mse_loss without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving or
 * training loops, harnesses that forbid hipMalloc).  No reference
 * counterpart.  The per-workgroup partial sums go to a fixed array in device
 * memory that each GPU the library runs on holds until the process ends
 * (8 * ceil(N / 16) bytes used, 2 MiB in all; the array of the stream's
 * device, the current device's for the null stream), so N is at most
 * SWVR_MSE_NOALLOC_MAX_N; larger N returns SWVR_EINVAL.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (several streams or
 * threads at once) race and must be serialised by the caller.  Each call
 * writes every partial it reads, so nothing needs clearing between calls.
 * Arguments and results are those of swvr_mse_loss, bit for bit. */
#define SWVR_MSE_NOALLOC_MAX_N (1 << 22)
int swvr_mse_loss_noalloc(int64_t N, int64_t D, const float* O, const float* lse, const void* target,
                          int target_dtype, int64_t ldt, const float* weight, float z_loss_weight, int reduction,
                          float* out, float* scale, float* gO, float* glse, void* stream);

/* Matrix-core throughput probe (measurement only; no reference counterpart):
 * `workgroups` workgroups of 8 waves, each wave `iters` steps of a 4 x 2 grid
 * of 32x32x16 bf16 MFMAs (2^18 flops per wave-step) on operands from
 * mode 0: random values in registers, 1: zeros in registers, 2: random values
 * read from LDS every step (6 x 16 bytes per lane per 8 MFMAs, the hot loops'
 * pattern), 3 / 4: as 2 with 4 / 3 reads per 8 MFMAs, 5: as 2 in the hot loops' software-pipelined
 * order, 6: A from LDS (4 reads per 8 MFMAs) and B loaded from an L2-resident device array into
 * registers 8 steps ahead (iters rounded up to a multiple of 8), 7: as 5 with a workgroup barrier
 * and 32 KB of direct-to-LDS stage loads every 2 steps, the hot loops' whole step (iters rounded up
 * to a multiple of 2), 8: as 7 with the barrier and 64 KB of stage loads every 4 steps (two slices
 * per stage; iters rounded up to a multiple of 4).  out receives workgroups * 512 floats (the
 * accumulator sums).
 * Timed, it measures the rate the chip sustains for such data. */
int swvr_probe_mfma(int64_t workgroups, int64_t iters, int mode, float* out, void* stream);

/* Instrumentation (no reference counterpart).  While enabled, every kernel
 * launch is bracketed by a pair of HIP events on its stream.
 * swvr_timing_collect synchronises those events, writes per-kernel-kind total
 * milliseconds and launch counts for up to max_kinds kinds, clears the record
 * and returns the number of kinds.  swvr_kernel_name(kind) names a kind. */
int swvr_timing_enable(int on);
int swvr_timing_collect(double* total_ms, int64_t* launches, int max_kinds);
const char* swvr_kernel_name(int kind);

#ifdef __cplusplus
}
#endif

#endif /* SWVR_H_ */
