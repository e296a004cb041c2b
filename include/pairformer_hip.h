/* C ABI of the MI355X (gfx950) PairFormer hot-path kernels: libpairformer_hip.so.
 *
 * Conventions
 *  - Every pointer is a device pointer (except where noted). Tensors are dense,
 *    row-major, 16-byte aligned.
 *  - dtype codes: PF_F32 = 0, PF_BF16 = 1. "zdtype" is the activation (residual
 *    stream) dtype, "cdtype" the GEMM operand dtype (MFMA inputs; accumulation is
 *    always fp32). Supported pairs: (F32, F32), (F32, BF16), (BF16, BF16).
 *  - LayerNorm affine parameters are always fp32. Weight arguments are in cdtype
 *    (cast once by the caller with pf_cast or a pack routine).
 *  - `stream` is a hipStream_t (pass torch.cuda.current_stream().cuda_stream).
 *    All work is enqueued on it; nothing synchronises the host.
 *  - The library never allocates device memory: scratch space is passed in as
 *    `workspace`, sized by the matching *_workspace_bytes query. The one exception is
 *    pf_single_attn_fwd_noalloc, whose scratch is a static device array of the library.
 *  - Every entry point returns a PF_* status; on failure pf_last_error()
 *    returns a thread-local message. No C++ exception crosses this boundary.
 *
 * Each entry point cites the reference (DeepFoldProtein/deepfold3-dev,
 * src/deepfold3/model/...) interface it replaces.
 */
#ifndef PAIRFORMER_HIP_H
#define PAIRFORMER_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PF_ABI_VERSION 2

#define PF_F32 0
#define PF_BF16 1

#define PF_OK 0
#define PF_ERR_INVALID_ARG 1
#define PF_ERR_UNSUPPORTED 2
#define PF_ERR_WORKSPACE 3
#define PF_ERR_ALIGNMENT 4
#define PF_ERR_LAUNCH 5

/* ---- library ---------------------------------------------------------- */
int pf_version(void);
const char* pf_last_error(void);
int pf_last_error_code(void);

/* Kernel timer (no counterpart in the reference; the reference times kernels with CUDA
 * events in benchmarks/utils.py:58-120). pf_kernel_timer_start(name) selects one launch
 * site ("trimul_project", "trimul_contract", "trimul_output", "attn_project", "pb_transpose",
 * "tri_attn", "tri_attn_redo", "attn_out", "evo_attn", "pair_transition", "single_attn_core",
 * "layernorm", "ln_transpose"), waits for the device to finish what it has queued, records
 * a reference event, and resets the totals; every later call of that site is bracketed by
 * HIP events on its own stream (without the system-scope fence) and timed from the first
 * event's end timestamp to the second's, both read against the reference event (an event's
 * start timestamp can precede the end of work queued ahead of it). pf_kernel_timer_read waits
 * for the events and returns the summed duration and the number of site calls so far;
 * pf_kernel_timer_stop switches timing off. Host-side state, guarded by a mutex. */
int pf_kernel_timer_start(const char* kernel);
int pf_kernel_timer_read(double* total_ms, long* count);
int pf_kernel_timer_stop(void);

/* dst[i] = (dst dtype) src[i]. Used to cast weights once per module version. */
int pf_cast(const void* src, int src_dtype, void* dst, int dst_dtype, size_t n, void* stream);

/* out[i] = res[i] + x[i] in res's dtype (out may alias res).
 * Replaces the eval branch of dropout_add_rowwise / dropout_add_columnwise
 * (triton/dropout_add.py:221-265, which return `residual + x` when not training). */
int pf_add(const void* res, int res_dtype, const void* x, int x_dtype, void* out, size_t n, void* stream);

/* ---- training-mode dropout-add (mask shared along one axis) ------------
 * Replaces the training branch of dropout_add_rowwise / dropout_add_columnwise
 * (triton/dropout_add.py:57-135 kernels, :137-201 autograd function, :221-265 wrappers).
 * The activation is [B, R, Cc, D] (D contiguous, D % 4 == 0). rowwise != 0 shares the mask
 * along R (one entry per (b, c, d), index b*Cc*D + c*D + d); rowwise == 0 shares it along Cc
 * (one entry per (b, r, d), index b*R*D + r*D + d). Mask entry i is 1/(1-p) when u_i >= p and
 * 0 otherwise, u_i = (word i%4 of Philox4x32-10(counter = i/4, key = seed) >> 8) * 2^-24; the
 * mask is never stored (the backward regenerates it from the seed). 0 <= p < 1.
 * pf_dropout_add_fwd: out = res + x * m in res's dtype (fp32 arithmetic, x*m and the add
 * rounded separately; out may alias res). pf_dropout_bwd: grad_x = grad_out * m in x's dtype
 * (the residual's gradient is grad_out itself). pf_dropout_mask writes the n mask entries
 * (0 or 1/(1-p), fp32) of a seed, for checking and for callers that want the mask. Pointers:
 * fp32 16-byte aligned, bf16 8-byte aligned. */
int pf_dropout_mask(float* mask, long n, float p, unsigned long long seed, void* stream);
int pf_dropout_add_fwd(const void* res, int res_dtype, const void* x, int x_dtype, void* out, long B, long R,
                       long Cc, long D, int rowwise, float p, unsigned long long seed, void* stream);
int pf_dropout_bwd(const void* grad_out, int grad_dtype, void* grad_x, int x_dtype, long B, long R, long Cc, long D,
                   int rowwise, float p, unsigned long long seed, void* stream);

/* RMSNormScaler + residual add (branch_scaler.py:38-50 with primitives.py:79-87, applied at
 * evoformer.py:298-335): out [M, C] = res + scale * x / sqrt(mean_c x^2 + eps) per row (eps
 * 1e-6 in the reference), fp32 arithmetic rounded once to res_dtype; out may alias res or x.
 * res NULL: out = scale * x / sqrt(mean_c x^2 + eps) (the scaled branch alone, in res_dtype). */
int pf_rms_residual_add(const void* res, int res_dtype, const void* x, int x_dtype, void* out, long M, int C,
                        float scale, float eps, void* stream);

/* ---- LayerNorm -------------------------------------------------------- */
/* out[r, :] = LN(x[r, :]) over C channels, fp32 statistics, output in x's dtype.
 * Replaces layer_norm / LayerNorm.forward (primitives.py:90-155). Tuned for C in
 * {128, 256, 384, 512}; other widths run a wave-per-row kernel. */
int pf_layernorm_fwd(const void* x, int dtype, const float* w, const float* b, float eps, void* out, long M, int C,
                     void* stream);
/* Backward of pf_layernorm_fwd (LayerNorm under autograd, primitives.py:90-115): for
 * dy = dL/dout [M, C] (x's dtype) writes dx (x's dtype) and the affine gradients dw, db [C]
 * fp32 (summed over rows in a fixed order). Statistics are recomputed from x.
 * C in {64, 128, 256, 384, 512}. */
size_t pf_layernorm_bwd_workspace_bytes(long M, int C);
int pf_layernorm_bwd(const void* x, const void* dy, int dtype, const float* w, float eps, void* dx, float* dw,
                     float* db, long M, int C, void* workspace, size_t workspace_bytes, void* stream);
/* Mixed-dtype LayerNorm (no counterpart in the reference, whose autocast path runs the
 * fp32 LayerNorm and then casts its output to bf16 for the next GEMM, and the cotangent back):
 * pf_layernorm_fwd_mixed writes LN(x) in odtype; pf_layernorm_bwd_mixed takes dy in dydtype
 * and writes dx in x's dtype. Same kernels, arithmetic and C range as the single-dtype entry
 * points; the autocast training path's input LayerNorms use them. */
int pf_layernorm_fwd_mixed(const void* x, int xdtype, const float* w, const float* b, float eps, void* out,
                           int odtype, long M, int C, void* stream);
int pf_layernorm_bwd_mixed(const void* x, int xdtype, const void* dy, int dydtype, const float* w, float eps,
                           void* dx, float* dw, float* db, long M, int C, void* workspace, size_t workspace_bytes,
                           void* stream);
/* x [B,N1,N2,C] -> out [B,N2,N1,C] (do_transpose) or [B,N1,N2,C]: LN then permute(0,2,1,3).
 * Replaces FusedLayerNormTranspose(C, do_transpose)(x, w, b) (triton/layernorm_transpose.py:269-316). */
int pf_ln_transpose_fwd(const void* x, int dtype, const float* w, const float* b, float eps, void* out, int B, int N1,
                        int N2, int C, int do_transpose, void* stream);

/* ---- triangle multiplicative update ----------------------------------- */
/* Replaces fused_trimul(z, mask, outgoing, norm_in, w_gate, w_proj, norm_out,
 * w_out, w_out_gate) (triton/fused_trimul.py:332-366) and the stock
 * TriangleMulOutgoing/Incoming._compute (ops.py:412-473).
 *
 * pf_trimul_pack_weights: w_proj, w_gate are [2C, C] (wdtype) in the fused
 * kernel's *block order* (rows 0..C-1 feed a, C..2C-1 feed b; the module's
 * `_block_order`, ops.py:285-288: (even, odd) outgoing, (odd, even) incoming).
 * Writes the packed [4C, C] cdtype operand `packed` consumed by pf_trimul_fwd with the
 * same C and cdtype (the packed order follows the kernel that reads it).
 *
 * pf_trimul_fwd: z [B,N,N,C] (zdtype); mask [B,N,N] fp32; w_out, w_out_gate
 * [C,C] cdtype. Writes the update to `out` [B,N,N,C] (zdtype), or adds it into
 * `out` when accumulate != 0 (out == z gives the fused residual z += update).
 * workspace >= pf_trimul_workspace_bytes(B, N, C, cdtype). C = 64, 128 or 256 (128 in
 * bf16 runs the persistent kernels, the rest the generic tile kernels). */
size_t pf_trimul_workspace_bytes(int B, int N, int C, int cdtype);
int pf_trimul_pack_weights(const void* w_proj, const void* w_gate, int wdtype, void* packed, int C, int cdtype,
                           void* stream);
int pf_trimul_fwd(const void* z, const float* mask, const float* ln_in_w, const float* ln_in_b, float eps_in,
                  const void* w_packed, const float* ln_out_w, const float* ln_out_b, float eps_out,
                  const void* w_out, const void* w_out_gate, int B, int N, int C, int outgoing, int zdtype, int cdtype,
                  void* out, int accumulate, void* workspace, size_t workspace_bytes, void* stream);

/* Training: FusedTriMulFunction (triton/fused_trimul.py:285-330), the triangle multiply
 * after its input LayerNorm, with a backward.
 *
 * pf_trimul_train_pack_weights: as pf_trimul_pack_weights, in the layout the training
 * kernels read: rows cb (4 j + kind) + r, kind 0 a proj, 1 a gate, 2 b proj, 3 b gate, in
 * blocks of cb = 32 channels for bf16 at C = 128 (the persistent kernels), 16 otherwise.
 *
 * pf_trimul_train_fwd: x [B,N,N,C] (xdtype) is the input LayerNorm's output; writes the
 * update to `out` (xdtype) and keeps the planes P, Q and the contraction X, channel-major
 * [B*C][Np][Np] each (cdtype, Np = N rounded up to 128, zero at padding), in `planes`
 * (pf_trimul_workspace_bytes(B, N, C, cdtype) bytes) for the backward.
 *
 * pf_trimul_output_vjp (_output_vjp_kernel, fused_trimul.py:153-212): with g the update's
 * cotangent [B,N,N,C] (xdtype), X from `planes` and w_out_t, w_out_gate_t the transposed
 * [C,C] weights, writes gp = g s, gg = g p s (1 - s) and xln = LN_out(X), token-major
 * [B*N*N, C] (cdtype), dX the cotangent of X (channel-major like X, zero at padding),
 * gx = gg Wog [B*N*N, C] fp32 and the LN_out affine gradients [C] fp32 (summed in a fixed
 * order). The host then forms dP = dX Q, dQ = dX^T P and the weight gradients
 * (w_out: gp^T xln, w_out_gate: gg^T x). `workspace` holds per-block partial sums.
 *
 * pf_trimul_project_vjp (_project_vjp_kernel, fused_trimul.py:214-262): dplanes = [dP; dQ]
 * (two [B*C][Np][Np] cdtype sets), w_packed from pf_trimul_train_pack_weights and
 * w_packed_t its [C, 4C] transpose; writes G = (gp_a, gg_a, gp_b, gg_b) token-major
 * [B*N*N, 4C] in the packed row order and dx = gx_in + G W4 [B*N*N, C] (xdtype). G's
 * rows follow the kernel's walk over plane positions (line, t) at b N^2 + line N + t:
 * token order when outgoing; when incoming (line = column of z) x is also written in that
 * order to xw [B*N*N, C] (cdtype), so the packed weights' gradient is G^T x (outgoing) or
 * G^T xw (incoming). C = 64, 128 or 256.
 *
 * pf_planes_transpose: dst[g] = src[g]^T for G planes [Np][Np] (Np a multiple of 64), the
 * dX^T operand of dQ = dX^T P.
 *
 * pf_planes_contract: X[g] = A[g] B[g]^T for G planes [Np][Np] (k contiguous, Np a multiple of
 * 128), on the forward's contraction kernels (K2). The VJP of X = P Q^T takes its cotangents
 * from it with transposed planes: dP = contract(dX, Q^T), dQ = contract(dX^T, P^T) (the
 * reference's backward forms both inside triton/fused_trimul.py:262-330). */
int pf_trimul_train_pack_weights(const void* w_proj, const void* w_gate, int wdtype, void* packed, int C, int cdtype,
                                 void* stream);
int pf_trimul_train_fwd(const void* x, const float* mask, const void* w_packed, const float* ln_out_w,
                        const float* ln_out_b, float eps_out, const void* w_out, const void* w_out_gate, int B, int N,
                        int C, int outgoing, int xdtype, int cdtype, void* planes, size_t planes_bytes, void* out,
                        void* stream);
size_t pf_trimul_output_vjp_workspace_bytes(int B, int N, int C, int cdtype);
int pf_trimul_output_vjp(const void* g, const void* X, const void* x, const float* ln_out_w, const float* ln_out_b,
                         float eps_out, const void* w_out, const void* w_out_gate, const void* w_out_t,
                         const void* w_out_gate_t, int B, int N, int C, int xdtype, int cdtype, void* gp, void* gg,
                         void* xln, void* dX, float* gx, float* d_ln_out_w, float* d_ln_out_b, void* workspace,
                         size_t workspace_bytes, void* stream);
int pf_trimul_project_vjp(const void* dplanes, const void* x, const float* mask, const void* w_packed,
                          const void* w_packed_t, const float* gx_in, int B, int N, int C, int outgoing, int xdtype,
                          int cdtype, void* gpg, void* xw, void* dx, void* stream);
int pf_planes_transpose(const void* src, void* dst, int G, int Np, int dtype, void* stream);
int pf_planes_contract(const void* A, const void* B, void* X, int G, int Np, int dtype, void* stream);

/* Multi-head routed (MHR) triangle multiplication: _TriangleMulBase with num_heads > 0
 * (ops.py:179-345) and its _mhr_head_mix (ops.py:476-545), between the contraction X and
 * out_proj. The C channels are H = num_heads heads of d = C / H (1 <= H <= 32); head_norm
 * 0 "channel" (LayerNorm over C), 1 "head_rms" (RMSNorm over each head, no shift: ln_out_b
 * may be NULL), 2 "head_ln" (LayerNorm over each head), 3 "post_channel" (gates, then
 * LayerNorm over C; needs the router); ln_out_w / ln_out_b are norm_center's [C] affine
 * (viewed [H, d] by the head modes), eps_out its eps. w_router [H, C] fp32 is the router
 * (r = LN_in(z) Wr^T per position; gates g = H softmax_h(r) for router_kind 0, 2 sigmoid(r)
 * for 1), or NULL for g = 1. The other arguments are those of the entry point each
 * extends:
 *
 * pf_trimul_mhr_fwd:        pf_trimul_fwd with the mix in K3 (the generic K3 at every C).
 * pf_trimul_mhr_train_fwd:  pf_trimul_train_fwd with the mix.
 * pf_trimul_mhr_output_vjp: pf_trimul_output_vjp through the mix: xln is the mix's output
 *                           (out_proj's input), the affine gradients are norm_center's, and
 *                           with a router d_router_logits [B*N*N, H] fp32 receives the
 *                           logits' cotangent dr, and gx also takes the router's share dr Wr.
 * pf_trimul_mhr_router_wgrad: the router weight's gradient d_router [H, C] fp32 = dr^T x over
 *                           the M = B*N*N tokens of x [M, C] (xdtype, the input LayerNorm's
 *                           output), summed in a fixed order; workspace >=
 *                           pf_trimul_mhr_router_wgrad_workspace_bytes(M, C, H). */
int pf_trimul_mhr_fwd(const void* z, const float* mask, const float* ln_in_w, const float* ln_in_b, float eps_in,
                      const void* w_packed, const float* ln_out_w, const float* ln_out_b, float eps_out,
                      const void* w_out, const void* w_out_gate, int B, int N, int C, int outgoing, int zdtype,
                      int cdtype, void* out, int accumulate, void* workspace, size_t workspace_bytes, int num_heads,
                      int head_norm, const float* w_router, int router_kind, void* stream);
int pf_trimul_mhr_train_fwd(const void* x, const float* mask, const void* w_packed, const float* ln_out_w,
                            const float* ln_out_b, float eps_out, const void* w_out, const void* w_out_gate, int B,
                            int N, int C, int outgoing, int xdtype, int cdtype, void* planes, size_t planes_bytes,
                            void* out, int num_heads, int head_norm, const float* w_router, int router_kind,
                            void* stream);
int pf_trimul_mhr_output_vjp(const void* g, const void* X, const void* x, const float* ln_out_w,
                             const float* ln_out_b, float eps_out, const void* w_out, const void* w_out_gate,
                             const void* w_out_t, const void* w_out_gate_t, int B, int N, int C, int xdtype,
                             int cdtype, void* gp, void* gg, void* xln, void* dX, float* gx, float* d_ln_out_w,
                             float* d_ln_out_b, void* workspace, size_t workspace_bytes, int num_heads, int head_norm,
                             const float* w_router, int router_kind, float* d_router_logits, void* stream);
size_t pf_trimul_mhr_router_wgrad_workspace_bytes(long M, int C, int H);
int pf_trimul_mhr_router_wgrad(const float* d_router_logits, const void* x, int xdtype, long M, int C, int H,
                               float* d_router, void* workspace, size_t workspace_bytes, void* stream);


/* ---- triangle attention (starting / ending node) ------------------------ */
/* Whole-module GridSelfAttention forward: replaces GridSelfAttention.forward
 * (src/deepfold3/model/attention.py:167-269) with its kernel chain FusedPairBias
 * (triton/fused_pair_bias.py:348-416) -> LN(+transpose) (triton/layernorm_transpose.py:269-316)
 * -> q/k/v/g projections -> _EvoformerAttention.apply (triton/evo_attention.py:1198-1292)
 * -> gate -> out_proj, and the dropout_add that consumes its output (eval: a plain add).
 *
 * z [B,N,N,C] (zdtype); mask [B,N,N] fp32 (pair mask, 1 keep / 0 pad); LN params fp32;
 * w_qkvgb [4C+16, C] cdtype: rows to_q | to_k | to_v | to_g | pair_bias (H rows) | zeros;
 * w_out [C, C] cdtype. transpose=0: starting node (rows), 1: ending node (columns).
 * Writes the update to `out`, or adds it into `out` when accumulate != 0 (out == z is the
 * fused residual). Masking follows the reference's eager path: keys with mask 0 get
 * -1e9 added in fp32, so a fully masked line attends uniformly (mean of V); the Triton
 * kernel's zero-output rule for such lines is not used. Built: C=128, H=4 (head dim 32);
 * C=256, H=8 with bf16 GEMMs (a persistent projection kernel writes both four-head frames);
 * other C a multiple of 32 with 1-16 heads of dimension max(C/H, 16) <= 32 (composed).
 * key_mask: NULL, or the caller's assertion that every mask[b] is the outer product of its
 * binary diagonal (m[i][k] = m[i][i] m[k][k], m in {0, 1}: the trunk's seq_mask x seq_mask),
 * given as that diagonal's additive key mask key_mask [B,N] fp32 = 1e9 (m[k][k] - 1) (both
 * from pf_pair_mask_outer). The key mask is then added to the pair bias once and the flash
 * kernel runs without per-line key masks; the result is the same. A mask that is not of that
 * form gives wrong results with key_mask set. Read by the C=128 and the C=256 bf16 paths;
 * the composed paths for other widths take the per-line masks and ignore it. */
size_t pf_grid_attn_workspace_bytes(int B, int N, int C, int H, int cdtype);
int pf_grid_attn_fwd(const void* z, const float* mask, const float* ln_w, const float* ln_b, float eps,
                     const void* w_qkvgb, const void* w_out, int B, int N, int C, int H, int transpose, int zdtype,
                     int cdtype, void* out, int accumulate, const float* key_mask, void* workspace,
                     size_t workspace_bytes, void* stream);
/* Whether pair masks are outer products (no reference counterpart: it selects
 * pf_grid_attn_fwd's key_mask path; the pair mask of featurizer.py:520 is seq x seq).
 * Writes flag[0] (device int) = 1 if every mask[b] [N,N] fp32 equals the outer product of
 * its diagonal with values in {0, 1}, else 0, and key_mask [B,N] fp32 = 1e9 (m[b][k][k] - 1).
 * Stream-ordered; the caller reads the flag. */
int pf_pair_mask_outer(const float* mask, int B, int N, int* flag, float* key_mask, void* stream);

/* ---- transitions ------------------------------------------------------- */
/* Pair transition, factor 4: replaces FusedTransitionBlock / TransitionBlock.forward
 * (triton/fused_transition.py:34-83, primitives.py:193-251; FusedLayerNormLinear
 * triton/layernorm_linear.py:537-592 and FusedSwiGLU triton/swiglu.py:192-200 inside it).
 * Built: C=128 (any supported dtype pair), and C=256 with bf16 x and bf16 weights (the
 * hidden activations stay on chip; no fused single_to_pair at this width).
 * x [M, C] zdtype; w1 [2*factor*C, C], w2 [C, factor*C] cdtype. out = y or out += y.
 * Optional fused single_to_pair at C=128 (evoformer.py:322-328): when pair_logits != NULL,
 * the updated rows are normalised with (s2p_ln_w, s2p_ln_b) and projected by w_s2p [16, C]
 * into pair_logits [M/NN, 16, NN] fp32 (NN = N*N positions per batch item). */
int pf_pair_transition_fwd(const void* x, const float* ln_w, const float* ln_b, float eps, const void* w1,
                           const void* w2, long M, int C, int factor, int zdtype, int cdtype, void* out, int accumulate,
                           const float* s2p_ln_w, const float* s2p_ln_b, float s2p_eps, const void* w_s2p,
                           float* pair_logits, long NN, void* stream);
/* single_to_pair(single_to_pair_norm(z)).movedim(-1, -3) (evoformer.py:322-328):
 * z [M, C] -> pair_logits [M/NN, H, NN] fp32. Built: C=128, H=16. */
int pf_single_to_pair_fwd(const void* z, const float* ln_w, const float* ln_b, float eps, const void* w_s2p, long M,
                          int C, int H, long NN, int zdtype, int cdtype, float* pair_logits, void* stream);
/* Generic TransitionBlock.forward (primitives.py:193-251) for any C (the single
 * transition, C=384): LN -> w1 [2fC, C] -> SwiGLU (contiguous halves) -> w2 [C, fC]. */
size_t pf_transition_workspace_bytes(long M, int C, int factor, int cdtype);
int pf_transition_fwd(const void* x, const float* ln_w, const float* ln_b, float eps, const void* w1, const void* w2,
                      long M, int C, int factor, int zdtype, int cdtype, void* out, int accumulate, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Recycling embedding around the trunk (evoformer.py:520-526 for the pair,
 * :558-561 for the single track): out += prev_embedding(prev_embedding_layer_norm(prev)),
 * prev and out [M, C] zdtype (not aliased), w [C, C] cdtype (the LinearNoBias weight, rows =
 * output channels). C a multiple of 64. */
size_t pf_recycle_embed_workspace_bytes(long M, int C, int cdtype);
int pf_recycle_embed_fwd(const void* prev, const float* ln_w, const float* ln_b, float eps, const void* w, long M,
                         int C, int zdtype, int cdtype, void* out, void* workspace, size_t workspace_bytes,
                         void* stream);

/* ---- MSA stack (Evoformer block) ----------------------------------------- */
/* OuterProductMean.forward (ops.py:683-785): msa [B,S,N,Cm] (mdtype), msa_mask [B,S,N] fp32;
 * LN params fp32; w_ab [2 CH, Cm] cdtype (proj_a rows, then proj_b rows); w_out [Cz, CH*CH]
 * cdtype (out_w[e][f][c] at row c, column e CH + f); b_out [Cz] fp32. The [B,N,N,Cz] result
 * is written to `out` (zdtype == mdtype) or added into it (accumulate != 0). Cm a multiple
 * of 32, CH of 8, Cz of 16. */
size_t pf_outer_product_mean_workspace_bytes(int B, int S, int N, int Cm, int CH, int Cz, int cdtype);
int pf_outer_product_mean_fwd(const void* msa, const float* msa_mask, const float* ln_w, const float* ln_b, float eps,
                              const void* w_ab, const void* w_out, const float* b_out, int B, int S, int N, int Cm,
                              int CH, int Cz, int mdtype, int zdtype, int cdtype, void* out, int accumulate,
                              void* workspace, size_t workspace_bytes, void* stream);
/* MSAAttention.forward (attention.py:272-341), AF3's pair-weighted averaging: msa [B,S,N,Cm]
 * and pair [B,N,N,Cz] (both mdtype), msa_mask [B,S,N] fp32; LN params fp32 (norm, pair_norm);
 * w_logits [16, Cz] cdtype (pair_logits rows, zero-padded to 16); w_vg [2 Cm, Cm] cdtype
 * (to_v rows, then to_g rows); w_out [Cm, Cm]. H heads of Cm/H. The [B,S,N,Cm] update is
 * written to `out` (mdtype) or added into it. Cm and Cz multiples of 32, 1 <= H <= 16. */
size_t pf_msa_pair_avg_workspace_bytes(int B, int S, int N, int Cm, int Cz, int H, int cdtype);
int pf_msa_pair_avg_fwd(const void* msa, const float* msa_mask, const void* pair, const float* ln_w, const float* ln_b,
                        float eps, const float* pair_ln_w, const float* pair_ln_b, float pair_eps, const void* w_logits,
                        const void* w_vg, const void* w_out, int B, int S, int N, int Cm, int Cz, int H, int mdtype,
                        int cdtype, void* out, int accumulate, void* workspace, size_t workspace_bytes, void* stream);

/* ---- single attention with pair bias ----------------------------------- */
/* SingleAttention.forward (attention.py:344-452), pair_bias_gate off: s [B,N,C] zdtype;
 * seq_mask [B,N] fp32; pair_logits [B,H,N,N] fp32; w_qkvg [4C, C] cdtype rows
 * to_q | to_k | to_v | to_g; q_bias [C] fp32; w_out [C, C]. Head dim C/H must be 24. */
size_t pf_single_attn_workspace_bytes(int B, int N, int C, int H, int cdtype);
int pf_single_attn_fwd(const void* s, const float* seq_mask, const float* pair_logits, const float* ln_w,
                       const float* ln_b, float eps, const void* w_qkvg, const float* q_bias, const void* w_out, int B,
                       int N, int C, int H, int zdtype, int cdtype, void* out, int accumulate, void* workspace,
                       size_t workspace_bytes, void* stream);
/* Allocation-free variant of pf_single_attn_fwd. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments and results as pf_single_attn_fwd
 * without the workspace: the scratch lives in a library-owned static device array of
 * PF_NOALLOC_SCRATCH_BYTES per GPU, held from the library's load on that GPU until the
 * process ends. Sizes whose pf_single_attn_workspace_bytes exceeds it return
 * PF_ERR_WORKSPACE (bf16: about 5.6 KB per token, so B*N up to ~5900; fp32 ~2900). Every
 * call on one GPU uses the same array: calls that overlap on one GPU (two streams, two
 * threads) race. The call allocates and frees nothing. */
#define PF_NOALLOC_SCRATCH_BYTES (32u << 20)
int pf_single_attn_fwd_noalloc(const void* s, const float* seq_mask, const float* pair_logits, const float* ln_w,
                               const float* ln_b, float eps, const void* w_qkvg, const float* q_bias, const void* w_out,
                               int B, int N, int C, int H, int zdtype, int cdtype, void* out, int accumulate,
                               void* stream);

/* ---- kernel-level operators of the reference's Triton layer -------------- */
/* _EvoformerAttention.apply(Q, K, V, res_mask, pair_bias, pre_transposed=True)
 * (triton/evo_attention.py:1198-1292): q, k, v, out [B,S,H,N,D] (dtype), res_mask [B,S,N]
 * fp32 additive (0 / -1e9 or -inf; the contiguous view of [B,S,1,1,N]), pair_bias
 * [B,H,N,N] fp32 (the view of [B,1,H,N,N]). out = softmax(q k^T D^-1/2 + pair_bias +
 * res_mask) v. masked_rows_zero != 0 writes 0 for a line whose keys are all masked (the
 * Triton kernel's rule, evo_attention.py:307-318); 0 gives the eager path's uniform
 * average (attention.py:157-160). Built: H = 4, D = 32. */
size_t pf_evo_attn_workspace_bytes(int B, int S, int H, int N, int D, int dtype);
int pf_evo_attn_fwd(const void* q, const void* k, const void* v, const float* res_mask, const float* pair_bias, int B,
                    int S, int H, int N, int D, int dtype, int masked_rows_zero, void* out, void* workspace,
                    size_t workspace_bytes, void* stream);
/* Redo flags of the flash-attention kernel (no counterpart in the reference: a test and
 * debugging aid). The kernel first runs a fast pass whose softmax keeps no running
 * maximum; every wave checks its row sums and outputs and writes one int32 flag, and a
 * nonzero flag makes the exact pass (running maximum) recompute that wave's block of
 * lines. Once a pf_grid_attn_fwd / pf_evo_attn_fwd call with the same sizes has completed
 * on its stream, its workspace holds *count such flags starting at byte *offset. */
int pf_grid_attn_redo_flags(int B, int N, int C, int H, int cdtype, size_t* offset, size_t* count);
int pf_evo_attn_redo_flags(int B, int S, int H, int N, int D, int dtype, size_t* offset, size_t* count);
/* _EvoformerAttention.backward (triton/evo_attention.py:1295-1472; kernels :335-1195):
 * gradients of out = softmax(scale q k^T + pair_bias + res_mask) v for q, k, v, dout
 * [B,S,H,N,D] (dtype) and res_mask [B,S,N], pair_bias [B,H,N,N] fp32. zero_masked_rows != 0
 * is the reference kernel's masked-row rule (a line whose keys are all masked, max logit
 * < -1e8, has output 0 and gradient 0); 0 is the stock eager rule (attention.py:415-433 under
 * autograd: the -1e9-shifted logits of such a row round to one value, its softmax is uniform
 * and its gradients are that softmax's Jacobian; only a row with no finite logit gets 0).
 * The softmax Jacobian is formed centred on each row's argmax, dS = P (u - C) with
 * u = dP - dP_imax (docs/optimizations.md:417-483). Writes dq, dk, dv (dtype) and
 * dpair_bias [B,H,N,N] fp32 (summed over S). The row statistics are recomputed here: the
 * forward saves nothing. Any H; D = 32. */
size_t pf_evo_attn_bwd_workspace_bytes(int B, int S, int H, int N, int D, int dtype);
int pf_evo_attn_bwd(const void* q, const void* k, const void* v, const float* res_mask, const float* pair_bias,
                    const void* dout, int B, int S, int H, int N, int D, int dtype, float softmax_scale,
                    int zero_masked_rows, void* dq, void* dk, void* dv, float* dpair_bias, void* workspace,
                    size_t workspace_bytes, void* stream);
/* Strided forms of pf_evo_attn_fwd / pf_evo_attn_bwd (no counterpart in the reference, whose
 * module path makes the [B, S, H, N, D] operands contiguous before the kernel): q, k, v, out,
 * dout, dq, dk, dv are views given by element strides {batch, line, head, key} (long[4]; D
 * contiguous; every stride a multiple of 16 bytes, the key stride >= D). q, k, v share
 * qkv_strides and dq, dk, dv share grad_strides. GridSelfAttention's training path passes
 * views of its token-major [B, N, N, 3, H, D] projection (rows: line stride N 3HD, key stride
 * 3HD; columns the two swapped) and takes O and the gradients in the same token order, so no
 * operand is permuted or copied around the kernels. Same arithmetic as the dense entry points;
 * res_mask [B, S, N] and pair_bias [B, H, N, N] stay dense.
 * lse (optional, NULL to skip): the forward writes each row's log-sum-exp of the logits in
 * log2 units, fp32 [B, S, H, Np] with Np = N rounded up to 128 (rows q < N written; +inf for a
 * line whose keys are all masked), the reference kernel's saved softmax_lse
 * (evo_attention.py:1279-1290). Given to the backward, it replaces the backward's first pass
 * over the keys (the row maximum): dQ's single pass takes p = 2^(x - lse) and re-centres its
 * sums on the row's dominant key (p > 1/2) when that key is reached. The backward recomputes
 * the row sum itself, so its results do not depend on the forward's rounding of lse; it must
 * come from the forward on the same q, k, res_mask, pair_bias and the backward's scale must
 * be 32^-1/2. NULL keeps the two-pass backward. */
int pf_evo_attn_fwd_strided(const void* q, const void* k, const void* v, const long* qkv_strides,
                            const float* res_mask, const float* pair_bias, int B, int S, int H, int N, int D,
                            int dtype, int masked_rows_zero, void* out, const long* out_strides, float* lse,
                            void* workspace, size_t workspace_bytes, void* stream);
int pf_evo_attn_bwd_strided(const void* q, const void* k, const void* v, const long* qkv_strides,
                            const float* res_mask, const float* pair_bias, const void* dout, const long* dout_strides,
                            const float* lse, int B, int S, int H, int N, int D, int dtype, float softmax_scale,
                            void* dq, void* dk, void* dv, const long* grad_strides, float* dpair_bias,
                            void* workspace, size_t workspace_bytes, void* stream);
/* FusedPairBias(c, H)(z, ln_w, ln_b, proj_w, mask) (triton/fused_pair_bias.py:348-416):
 * z [B,N,N,C] -> out [B,H,N,N] in z's dtype; proj_w16 [16, C] fp32 (proj_w padded with zero
 * rows); mask [B,N] fp32 or NULL adds (1 - mask) * (-1e9) on the last axis. C = 128, H <= 16. */
int pf_pair_bias_fwd(const void* z, int zdtype, const float* ln_w, const float* ln_b, float eps,
                     const float* proj_w16, int H, const float* mask, void* out, int B, int N, int C, void* stream);
/* FusedLayerNormLinear(K, N)(X, ln_w, ln_b, W, bias) (triton/layernorm_linear.py:537-592):
 * out [M, N] (x's dtype) = LN(x [M, K]) W + bias, with W passed as w_nk [N, K] (cdtype; the
 * reference's [K, N] argument transposed once by the caller), bias fp32 [N] or NULL.
 * K a multiple of 32, N of 16. */
size_t pf_layernorm_linear_workspace_bytes(long M, int K, int cdtype);
int pf_layernorm_linear_fwd(const void* x, int xdtype, const float* ln_w, const float* ln_b, float eps,
                            const void* w_nk, const float* bias, long M, int K, int Nout, int cdtype, void* out,
                            void* workspace, size_t workspace_bytes, void* stream);
/* FusedSwiGLU()(x) (triton/swiglu.py:192-200): y [M, D] = silu(x[:, :D]) * x[:, D:], x [M, 2D]. */
int pf_swiglu_fwd(const void* x, int dtype, void* y, long M, int D, void* stream);
/* Backward of pf_swiglu_fwd (FusedSwiGLU's VJP, triton/swiglu.py:60-95): dx [M, 2D] from
 * x [M, 2D] and dy [M, D], all in dtype. */
int pf_swiglu_bwd(const void* x, const void* dy, int dtype, void* dx, long M, int D, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAIRFORMER_HIP_H */
