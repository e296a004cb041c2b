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
 *    `workspace`, sized by the matching *_workspace_bytes query.
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

#define PF_ABI_VERSION 1

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

/* dst[i] = (dst dtype) src[i]. Used to cast weights once per module version. */
int pf_cast(const void* src, int src_dtype, void* dst, int dst_dtype, size_t n, void* stream);

/* out[i] = res[i] + x[i] in res's dtype (out may alias res).
 * Replaces the eval branch of dropout_add_rowwise / dropout_add_columnwise
 * (triton/dropout_add.py:221-265, which return `residual + x` when not training). */
int pf_add(const void* res, int res_dtype, const void* x, int x_dtype, void* out, size_t n, void* stream);

/* ---- LayerNorm -------------------------------------------------------- */
/* out[r, :] = LN(x[r, :]) over C channels, fp32 statistics, output in x's dtype.
 * Replaces layer_norm / LayerNorm.forward (primitives.py:90-155). C in {128, 256, 384, 512}. */
int pf_layernorm_fwd(const void* x, int dtype, const float* w, const float* b, float eps, void* out, long M, int C,
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
 * Writes the packed [4C, C] cdtype operand `packed` consumed by pf_trimul_fwd.
 *
 * pf_trimul_fwd: z [B,N,N,C] (zdtype); mask [B,N,N] fp32; w_out, w_out_gate
 * [C,C] cdtype. Writes the update to `out` [B,N,N,C] (zdtype), or adds it into
 * `out` when accumulate != 0 (out == z gives the fused residual z += update).
 * workspace >= pf_trimul_workspace_bytes(B, N, C, cdtype). Only C = 128. */
size_t pf_trimul_workspace_bytes(int B, int N, int C, int cdtype);
int pf_trimul_pack_weights(const void* w_proj, const void* w_gate, int wdtype, void* packed, int C, int cdtype,
                           void* stream);
int pf_trimul_fwd(const void* z, const float* mask, const float* ln_in_w, const float* ln_in_b, float eps_in,
                  const void* w_packed, const float* ln_out_w, const float* ln_out_b, float eps_out,
                  const void* w_out, const void* w_out_gate, int B, int N, int C, int outgoing, int zdtype, int cdtype,
                  void* out, int accumulate, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAIRFORMER_HIP_H */
