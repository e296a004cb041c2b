// The MSA-stack operators of the Evoformer block (src/deepfold3/model/evoformer.py:100-175):
//
//   pf_outer_product_mean_fwd: OuterProductMean.forward (ops.py:683-785). x = LN(msa);
//     a, b = x W_a^T * m, x W_b^T * m; ab[i,j,e,f] = sum_s a[s,i,e] b[s,j,f] (one GEMM per batch
//     item with the sequences as k: [N CH][S] x [N CH][S]^T); act = ab . out_w + out_b (a second
//     GEMM with k = CH^2); result = act / (1e-3 + sum_s m[s,i] m[s,j]) (the counts are a third,
//     fp32 GEMM), stored into or added to the pair stream.
//   pf_msa_pair_avg_fwd: MSAAttention.forward (attention.py:272-341), AF3's pair-weighted
//     averaging. W[h,q,k] = softmax_k(LN(pair) W_h + 1e9 (colmask_k - 1)) in fp32, cast to the
//     operand dtype (colmask = max over sequences of the mask); every MSA row averages its
//     values v = to_v(LN(msa)) with W (one GEMM per batch item and head with the keys as k:
//     [N][Kp] x [S D][Kp]^T), gates with sigmoid(to_g(LN(msa))) and projects with out_proj,
//     stored into or added to the MSA stream.
//
// LayerNorms and the thin projections use the row kernels; the contractions use the batched
// NT GEMM (k zero-padded to its tile).
#include <algorithm>

#include "capi.h"
#include "common.h"
#include "gemm.h"
#include "rowops.h"

namespace {

size_t es_of(int dt) { return dt == PF_F32 ? 4 : 2; }
long pad_k(long k) { return (k + kBgemmK - 1) / kBgemmK * kBgemmK; }

// ------------------------------------------------------------------ outer product mean
struct OpmWs {
  size_t xn, ab, at, bt, mt, x, y, act, cnt, total;
};

OpmWs opm_layout(int B, int S, int N, int Cm, int CH, int Cz, int cdtype) {
  const size_t es = es_of(cdtype);
  const size_t Sp = pad_k(S);
  const size_t R = (size_t)B * S * N;
  OpmWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += pf::round_up(bytes, 256);
    return at;
  };
  w.xn = take(R * Cm * es);
  w.ab = take(R * 2 * CH * es);
  w.at = take((size_t)B * N * CH * Sp * es);
  w.bt = take((size_t)B * N * CH * Sp * es);
  w.mt = take((size_t)B * N * Sp * 4);
  w.x = take((size_t)B * N * CH * N * CH * es);
  w.y = take((size_t)B * N * N * CH * CH * es);
  w.act = take((size_t)B * N * N * Cz * 4);
  w.cnt = take((size_t)B * N * N * 4);
  w.total = off;
  return w;
}

// At[b][i CH + e][s] = a[b,s,i,e] m[b,s,i], Bt likewise with b; Mt[b][i][s] = m[b,s,i];
// sequences S..Sp-1 are zero. One thread per (b, i, s).
template <class TC>
__global__ __launch_bounds__(256) void opm_pack_kernel(const TC* __restrict__ ab, const float* __restrict__ mask,
                                                       TC* __restrict__ At, TC* __restrict__ Bt, float* __restrict__ Mt,
                                                       int B, int S, int N, int CH, int Sp) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)B * N * Sp) return;
  const int s = (int)(idx % Sp);
  const int i = (int)((idx / Sp) % N);
  const int b = (int)(idx / ((long)Sp * N));
  const float m = s < S ? mask[((size_t)b * S + s) * N + i] : 0.f;
  const TC* row = ab + (((size_t)b * S + (s < S ? s : 0)) * N + i) * 2 * CH;
  const size_t base = (((size_t)b * N + i) * CH) * Sp + s;
  for (int e = 0; e < CH; ++e) {
    At[base + (size_t)e * Sp] = from_f32<TC>(to_f32(row[e]) * m);
    Bt[base + (size_t)e * Sp] = from_f32<TC>(to_f32(row[CH + e]) * m);
  }
  Mt[((size_t)b * N + i) * Sp + s] = m;
}

// Y[b][i N + j][e CH + f] = X[b][i CH + e][j CH + f]; one thread per element of Y.
template <class TC>
__global__ __launch_bounds__(256) void opm_reorder_kernel(const TC* __restrict__ X, TC* __restrict__ Y, int B, int N,
                                                          int CH) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  const long ch2 = (long)CH * CH;
  if (idx >= (long)B * N * N * ch2) return;
  const int f = (int)(idx % CH);
  const int e = (int)((idx / CH) % CH);
  const long ij = idx / ch2;
  const int j = (int)(ij % N);
  const int i = (int)((ij / N) % N);
  const int b = (int)(ij / ((long)N * N));
  const long NC = (long)N * CH;
  Y[idx] = X[(size_t)b * NC * NC + ((size_t)i * CH + e) * NC + (size_t)j * CH + f];
}

// out[b,i,j,c] (+)= (act + out_b[c]) / (1e-3 + cnt[b,i,j]).
template <class TZ>
__global__ __launch_bounds__(256) void opm_epilogue_kernel(const float* __restrict__ act, const float* __restrict__ bias,
                                                           const float* __restrict__ cnt, TZ* __restrict__ out, long rows,
                                                           int Cz, int accumulate) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * Cz) return;
  const int c = (int)(idx % Cz);
  const float v = (act[idx] + bias[c]) / (1e-3f + cnt[idx / Cz]);
  out[idx] = from_f32<TZ>(accumulate ? to_f32(out[idx]) + v : v);
}

template <class TM, class TC, class TZ>
int opm_launch(const void* msa, const float* mask, const float* lnw, const float* lnb, float eps, const void* w_ab,
               const void* w_out, const float* b_out, int B, int S, int N, int Cm, int CH, int Cz, void* out,
               int accumulate, void* ws, hipStream_t s) {
  const int cd = sizeof(TC) == 4 ? PF_F32 : PF_BF16;
  const OpmWs L = opm_layout(B, S, N, Cm, CH, Cz, cd);
  const int Sp = (int)pad_k(S);
  char* base = reinterpret_cast<char*>(ws);
  TC* xn = reinterpret_cast<TC*>(base + L.xn);
  TC* ab = reinterpret_cast<TC*>(base + L.ab);
  TC* At = reinterpret_cast<TC*>(base + L.at);
  TC* Bt = reinterpret_cast<TC*>(base + L.bt);
  float* Mt = reinterpret_cast<float*>(base + L.mt);
  TC* X = reinterpret_cast<TC*>(base + L.x);
  TC* Y = reinterpret_cast<TC*>(base + L.y);
  float* act = reinterpret_cast<float*>(base + L.act);
  float* cnt = reinterpret_cast<float*>(base + L.cnt);
  const long R = (long)B * S * N;
  if (int e = ln_launch<TM, TC>(msa, lnw, lnb, eps, xn, R, Cm, s)) return e;
  if (int e = rowgemm_launch<TC, TC, EPI_STORE>(xn, w_ab, nullptr, 0, ab, R, 2 * CH, Cm, s)) return e;
  opm_pack_kernel<TC><<<(unsigned)(((long)B * N * Sp + 255) / 256), 256, 0, s>>>(ab, mask, At, Bt, Mt, B, S, N, CH, Sp);
  if (int e = pf::check_launch("opm_pack")) return e;
  const long NC = (long)N * CH;
  if (int e = bgemm_nt(At, Bt, X, (int)NC, (int)NC, Sp, Sp, Sp, NC, NC * Sp, NC * Sp, NC * NC, B, cd, cd, s)) return e;
  const long ny = (long)B * N * N * CH * CH;
  opm_reorder_kernel<TC><<<(unsigned)((ny + 255) / 256), 256, 0, s>>>(X, Y, B, N, CH);
  if (int e = pf::check_launch("opm_reorder")) return e;
  const long NN = (long)B * N * N;
  if (int e = bgemm_nt(Y, w_out, act, (int)NN, Cz, CH * CH, CH * CH, CH * CH, Cz, 0, 0, 0, 1, cd, PF_F32, s)) return e;
  if (int e = bgemm_nt(Mt, Mt, cnt, N, N, Sp, Sp, Sp, N, (long)N * Sp, (long)N * Sp, (long)N * N, B, PF_F32, PF_F32, s))
    return e;
  opm_epilogue_kernel<TZ><<<(unsigned)((NN * Cz + 255) / 256), 256, 0, s>>>(act, b_out, cnt, (TZ*)out, NN, Cz,
                                                                            accumulate);
  return pf::check_launch("opm_epilogue");
}

// ------------------------------------------------------------------ MSA pair-weighted averaging
struct PavWs {
  size_t pn, lg, cm, w, xm, vg, vt, va, og, total;
};

PavWs pav_layout(int B, int S, int N, int Cm, int Cz, int H, int cdtype) {
  const size_t es = es_of(cdtype);
  const size_t Kp = pad_k(N);
  const size_t R = (size_t)B * S * N;
  const size_t D = Cm / H;
  PavWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += pf::round_up(bytes, 256);
    return at;
  };
  w.pn = take((size_t)B * N * N * Cz * es);
  w.lg = take((size_t)B * N * N * 16 * 4);
  w.cm = take((size_t)B * N * 4);
  w.w = take((size_t)B * H * N * Kp * es);
  w.xm = take(R * Cm * es);
  w.vg = take(R * 2 * Cm * es);
  w.vt = take((size_t)B * H * S * D * Kp * es);
  w.va = take((size_t)B * H * N * S * D * es);
  w.og = take(R * Cm * es);
  w.total = off;
  return w;
}

// colmask[b][k] = max over sequences of mask[b][s][k]; one thread per (b, k).
__global__ __launch_bounds__(256) void pav_colmask_kernel(const float* __restrict__ mask, float* __restrict__ cm, int B,
                                                          int S, int N) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= B * N) return;
  const int b = idx / N, k = idx % N;
  float m = -INFINITY;
  for (int s = 0; s < S; ++s) m = fmaxf(m, mask[((size_t)b * S + s) * N + k]);
  cm[idx] = m;
}

// W[b][h][q][k] = softmax_k(lg[b,q,k][h] + 1e9 (cm[b,k] - 1)) in fp32, stored in the operand
// dtype; keys N..Kp-1 are zero. One wave per (b, h, q) row.
template <class TC>
__global__ __launch_bounds__(256) void pav_softmax_kernel(const float* __restrict__ lg, const float* __restrict__ cm,
                                                          TC* __restrict__ W, int B, int N, int H, int Kp) {
  const long row = (long)blockIdx.x * 4 + wave_id();
  if (row >= (long)B * H * N) return;
  const int l = lane_id();
  const int q = (int)(row % N);
  const int h = (int)((row / N) % H);
  const int b = (int)(row / ((long)N * H));
  const float* lb = lg + ((size_t)b * N + q) * N * 16 + h;
  const float* cb = cm + (size_t)b * N;
  auto logit = [&](int k) { return lb[(size_t)k * 16] + 1e9f * (cb[k] - 1.0f); };
  float mx = -INFINITY;
  for (int k = l; k < N; k += 64) mx = fmaxf(mx, logit(k));
  mx = group_max<64>(mx);
  float sum = 0.f;
  for (int k = l; k < N; k += 64) sum += expf(logit(k) - mx);
  sum = group_sum<64>(sum);
  const float inv = 1.0f / sum;
  TC* wr = W + (size_t)row * Kp;
  for (int k = l; k < Kp; k += 64) wr[k] = from_f32<TC>(k < N ? expf(logit(k) - mx) * inv : 0.f);
}

// Vt[b][h][s D + d][k] = v[b,s,k,h D + d] (the first Cm columns of vg), keys N..Kp-1 zero.
template <class TC>
__global__ __launch_bounds__(256) void pav_vt_kernel(const TC* __restrict__ vg, TC* __restrict__ Vt, int B, int S, int N,
                                                     int Cm, int H, int Kp) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  const int D = Cm / H;
  if (idx >= (long)B * H * S * D * Kp) return;
  const int k = (int)(idx % Kp);
  const long r = idx / Kp;  // (b, h, s, d)
  const int d = (int)(r % D);
  const int s = (int)((r / D) % S);
  const int h = (int)((r / ((long)D * S)) % H);
  const int b = (int)(r / ((long)D * S * H));
  Vt[idx] = k < N ? vg[(((size_t)b * S + s) * N + k) * 2 * Cm + h * D + d] : from_f32<TC>(0.f);
}

// og[b,s,q][h D + d] = va[b][h][q][s D + d] * sigmoid(g[b,s,q][h D + d]).
template <class TC>
__global__ __launch_bounds__(256) void pav_gate_kernel(const TC* __restrict__ va, const TC* __restrict__ vg,
                                                       TC* __restrict__ og, int B, int S, int N, int Cm, int H) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)B * S * N * Cm) return;
  const int D = Cm / H;
  const int c = (int)(idx % Cm);
  const long pos = idx / Cm;  // (b, s, q)
  const int q = (int)(pos % N);
  const int s = (int)((pos / N) % S);
  const int b = (int)(pos / ((long)N * S));
  const int h = c / D, d = c % D;
  const float v = to_f32(va[(((size_t)b * H + h) * N + q) * (size_t)S * D + (size_t)s * D + d]);
  og[idx] = from_f32<TC>(v * sigmoidf_(to_f32(vg[pos * 2 * Cm + Cm + c])));
}

template <class TM, class TC>
int pav_launch(const void* msa, const float* mask, const void* pair, const float* lnw, const float* lnb, float eps,
               const float* plnw, const float* plnb, float peps, const void* w_lg, const void* w_vg, const void* w_out,
               int B, int S, int N, int Cm, int Cz, int H, void* out, int accumulate, void* ws, hipStream_t s) {
  const int cd = sizeof(TC) == 4 ? PF_F32 : PF_BF16;
  const PavWs L = pav_layout(B, S, N, Cm, Cz, H, cd);
  const int Kp = (int)pad_k(N);
  const int D = Cm / H;
  char* base = reinterpret_cast<char*>(ws);
  TC* pn = reinterpret_cast<TC*>(base + L.pn);
  float* lg = reinterpret_cast<float*>(base + L.lg);
  float* cm = reinterpret_cast<float*>(base + L.cm);
  TC* W = reinterpret_cast<TC*>(base + L.w);
  TC* xm = reinterpret_cast<TC*>(base + L.xm);
  TC* vg = reinterpret_cast<TC*>(base + L.vg);
  TC* Vt = reinterpret_cast<TC*>(base + L.vt);
  TC* va = reinterpret_cast<TC*>(base + L.va);
  TC* og = reinterpret_cast<TC*>(base + L.og);
  const long P = (long)B * N * N;
  const long R = (long)B * S * N;
  if (int e = ln_launch<TM, TC>(pair, plnw, plnb, peps, pn, P, Cz, s)) return e;
  if (int e = rowgemm_launch<TC, float, EPI_STORE>(pn, w_lg, nullptr, 0, lg, P, 16, Cz, s)) return e;
  pav_colmask_kernel<<<(unsigned)((B * N + 255) / 256), 256, 0, s>>>(mask, cm, B, S, N);
  pav_softmax_kernel<TC><<<(unsigned)(((long)B * H * N + 3) / 4), 256, 0, s>>>(lg, cm, W, B, N, H, Kp);
  if (int e = pf::check_launch("pav_softmax")) return e;
  if (int e = ln_launch<TM, TC>(msa, lnw, lnb, eps, xm, R, Cm, s)) return e;
  if (int e = rowgemm_launch<TC, TC, EPI_STORE>(xm, w_vg, nullptr, 0, vg, R, 2 * Cm, Cm, s)) return e;
  const long nvt = (long)B * H * S * D * Kp;
  pav_vt_kernel<TC><<<(unsigned)((nvt + 255) / 256), 256, 0, s>>>(vg, Vt, B, S, N, Cm, H, Kp);
  if (int e = pf::check_launch("pav_vt")) return e;
  const long SD = (long)S * D;
  if (int e = bgemm_nt(W, Vt, va, N, (int)SD, Kp, Kp, Kp, SD, (long)N * Kp, SD * Kp, (long)N * SD, B * H, cd, cd, s))
    return e;
  pav_gate_kernel<TC><<<(unsigned)((R * Cm + 255) / 256), 256, 0, s>>>(va, vg, og, B, S, N, Cm, H);
  if (int e = pf::check_launch("pav_gate")) return e;
  if (accumulate) return rowgemm_launch<TC, TM, EPI_RESIDUAL>(og, w_out, nullptr, 0, out, R, Cm, Cm, s);
  return rowgemm_launch<TC, TM, EPI_STORE>(og, w_out, nullptr, 0, out, R, Cm, Cm, s);
}

bool dt_ok(int d) { return d == PF_F32 || d == PF_BF16; }

}  // namespace

extern "C" {

size_t pf_outer_product_mean_workspace_bytes(int B, int S, int N, int Cm, int CH, int Cz, int cdtype) {
  if (B <= 0 || S <= 0 || N <= 0 || Cm <= 0 || CH <= 0 || Cz <= 0) return 0;
  return opm_layout(B, S, N, Cm, CH, Cz, cdtype).total;
}

int pf_outer_product_mean_fwd(const void* msa, const float* msa_mask, const float* ln_w, const float* ln_b, float eps,
                              const void* w_ab, const void* w_out, const float* b_out, int B, int S, int N, int Cm,
                              int CH, int Cz, int mdtype, int zdtype, int cdtype, void* out, int accumulate,
                              void* workspace, size_t workspace_bytes, void* stream) {
  PF_REQUIRE(msa && msa_mask && ln_w && ln_b && w_ab && w_out && b_out && out && workspace, PF_ERR_INVALID_ARG,
             "pf_outer_product_mean_fwd: null pointer");
  PF_REQUIRE(B > 0 && S > 0 && N > 0, PF_ERR_INVALID_ARG, "pf_outer_product_mean_fwd: B=%d S=%d N=%d", B, S, N);
  PF_REQUIRE(Cm % 32 == 0 && (2 * CH) % 16 == 0 && (CH * CH) % kBgemmK == 0 && Cz % 16 == 0, PF_ERR_UNSUPPORTED,
             "pf_outer_product_mean_fwd: Cm=%d CH=%d Cz=%d (Cm a multiple of 32, CH of 8, Cz of 16)", Cm, CH, Cz);
  PF_REQUIRE(dt_ok(mdtype) && dt_ok(zdtype) && dt_ok(cdtype) && !(mdtype == PF_BF16 && cdtype == PF_F32) &&
                 zdtype == mdtype,
             PF_ERR_UNSUPPORTED, "pf_outer_product_mean_fwd: dtypes msa %d pair %d gemm %d", mdtype, zdtype, cdtype);
  PF_REQUIRE(workspace_bytes >= pf_outer_product_mean_workspace_bytes(B, S, N, Cm, CH, Cz, cdtype), PF_ERR_WORKSPACE,
             "pf_outer_product_mean_fwd: workspace %zu < %zu bytes", workspace_bytes,
             pf_outer_product_mean_workspace_bytes(B, S, N, Cm, CH, Cz, cdtype));
  hipStream_t s = pf::as_stream(stream);
  if (mdtype == PF_F32 && cdtype == PF_F32)
    return opm_launch<float, float, float>(msa, msa_mask, ln_w, ln_b, eps, w_ab, w_out, b_out, B, S, N, Cm, CH, Cz,
                                           out, accumulate, workspace, s);
  if (mdtype == PF_F32)
    return opm_launch<float, bf16, float>(msa, msa_mask, ln_w, ln_b, eps, w_ab, w_out, b_out, B, S, N, Cm, CH, Cz, out,
                                          accumulate, workspace, s);
  return opm_launch<bf16, bf16, bf16>(msa, msa_mask, ln_w, ln_b, eps, w_ab, w_out, b_out, B, S, N, Cm, CH, Cz, out,
                                      accumulate, workspace, s);
}

size_t pf_msa_pair_avg_workspace_bytes(int B, int S, int N, int Cm, int Cz, int H, int cdtype) {
  if (B <= 0 || S <= 0 || N <= 0 || Cm <= 0 || Cz <= 0 || H <= 0) return 0;
  return pav_layout(B, S, N, Cm, Cz, H, cdtype).total;
}

int pf_msa_pair_avg_fwd(const void* msa, const float* msa_mask, const void* pair, const float* ln_w, const float* ln_b,
                        float eps, const float* pair_ln_w, const float* pair_ln_b, float pair_eps, const void* w_logits,
                        const void* w_vg, const void* w_out, int B, int S, int N, int Cm, int Cz, int H, int mdtype,
                        int cdtype, void* out, int accumulate, void* workspace, size_t workspace_bytes, void* stream) {
  PF_REQUIRE(msa && msa_mask && pair && ln_w && ln_b && pair_ln_w && pair_ln_b && w_logits && w_vg && w_out && out &&
                 workspace,
             PF_ERR_INVALID_ARG, "pf_msa_pair_avg_fwd: null pointer");
  PF_REQUIRE(B > 0 && S > 0 && N > 0, PF_ERR_INVALID_ARG, "pf_msa_pair_avg_fwd: B=%d S=%d N=%d", B, S, N);
  PF_REQUIRE(H >= 1 && H <= 16 && Cm % 32 == 0 && Cm % H == 0 && Cz % 32 == 0, PF_ERR_UNSUPPORTED,
             "pf_msa_pair_avg_fwd: Cm=%d Cz=%d H=%d (Cm, Cz multiples of 32, 1-16 heads dividing Cm)", Cm, Cz, H);
  PF_REQUIRE(dt_ok(mdtype) && dt_ok(cdtype) && !(mdtype == PF_BF16 && cdtype == PF_F32), PF_ERR_UNSUPPORTED,
             "pf_msa_pair_avg_fwd: dtypes msa %d gemm %d", mdtype, cdtype);
  PF_REQUIRE(workspace_bytes >= pf_msa_pair_avg_workspace_bytes(B, S, N, Cm, Cz, H, cdtype), PF_ERR_WORKSPACE,
             "pf_msa_pair_avg_fwd: workspace %zu < %zu bytes", workspace_bytes,
             pf_msa_pair_avg_workspace_bytes(B, S, N, Cm, Cz, H, cdtype));
  hipStream_t s = pf::as_stream(stream);
  if (mdtype == PF_F32 && cdtype == PF_F32)
    return pav_launch<float, float>(msa, msa_mask, pair, ln_w, ln_b, eps, pair_ln_w, pair_ln_b, pair_eps, w_logits,
                                    w_vg, w_out, B, S, N, Cm, Cz, H, out, accumulate, workspace, s);
  if (mdtype == PF_F32)
    return pav_launch<float, bf16>(msa, msa_mask, pair, ln_w, ln_b, eps, pair_ln_w, pair_ln_b, pair_eps, w_logits,
                                   w_vg, w_out, B, S, N, Cm, Cz, H, out, accumulate, workspace, s);
  return pav_launch<bf16, bf16>(msa, msa_mask, pair, ln_w, ln_b, eps, pair_ln_w, pair_ln_b, pair_eps, w_logits, w_vg,
                                w_out, B, S, N, Cm, Cz, H, out, accumulate, workspace, s);
}

}  // extern "C"
