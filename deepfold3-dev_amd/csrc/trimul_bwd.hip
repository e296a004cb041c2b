// Backward of the triangle multiply after its input LayerNorm (FusedTriMulFunction.backward,
// src/deepfold3/model/triton/fused_trimul.py:298-330, VJP kernels :153-262).
//
// Forward (x = LN_in(z) given): a | b = sigmoid(x Wg^T) * (x Wp^T) * mask on channel-major
// planes P, Q; X = P Q^T per channel; out = sigmoid(x Wog^T) * (LN_out(X) Wo^T).
//
//   trimul_output_vjp:  per (line, 64 plane positions): recompute LN_out(X) and both output
//                       GEMMs, gp = g s, gg = g p s (1 - s); d(xln) = gp Wo, pulled through
//                       LN_out into dX (channel-major planes, zero at padding); the output
//                       gate's x cotangent gg Wog (fp32); gp, gg channel-major and xln
//                       token-major for the weight gradients; per-block partial sums of the
//                       LN_out affine gradients, reduced in a fixed order by
//                       trimul_ln_grad_reduce.
//   (host)              dP = dX Q, dQ = dX^T P, weight gradients: plain library GEMMs.
//   trimul_project_vjp: per (line, plane positions) as the forward K1: recompute both gated
//                       projections, G = (gp_a, gg_a, gp_b, gg_b) in the packed weight order,
//                       dx = gx + G W4 (W4 the packed [4C][C] weights), G channel-major.
//
// The LN_out pullback with xn the standardised X and u = d(xln) * ln_w is
// rstd (u - mean_c(u) - xn mean_c(u xn)) (fused_trimul.py:166-171).
#include <algorithm>
#include <type_traits>

#include "capi.h"
#include "common.h"
#include "mhr.h"

namespace {

// Positions per block: 64 where LDS allows (C * sizeof(TC) <= 256 bytes), fewer above.
template <class TC, int C>
constexpr int vjp_bm() {
  return std::min(64, 16384 / (C * (int)sizeof(TC)));
}
// Threads of the generic VJP blocks: 8 waves from 256 channels, so each wave's accumulators
// halve (with 4 waves the project VJP held 320 VGPRs per lane at C=256, one wave per SIMD).
template <int C>
constexpr int vjp_nt() { return C >= 256 ? 512 : 256; }

// ------------------------------------------------------------------ output VJP
// MHR = true: the multi-head routed mix `mx` (mhr.h) in place of LN_out; xln_out is then its
// output Y, the affine gradients are those of the mix's norm and dr [M][H] (fp32) receives the
// router logits' cotangent when mx has a router.
template <class TZ, class TC, int C, bool MHR = false, int HM = kMhrMaxHeads>
__global__ __launch_bounds__(vjp_nt<C>()) void trimul_output_vjp_kernel(
    const TZ* __restrict__ g, const TC* __restrict__ X, const TZ* __restrict__ x, const float* __restrict__ lnow,
    const float* __restrict__ lnob, float eps, const TC* __restrict__ Wo, const TC* __restrict__ Wog,
    const TC* __restrict__ WoT, const TC* __restrict__ WogT, int B, int N, int Np, TC* __restrict__ gp_out,
    TC* __restrict__ gg_out, TC* __restrict__ xln_out, TC* __restrict__ dX, float* __restrict__ gx,
    float* __restrict__ partial, MixSpec mx, float* __restrict__ dr) {
  constexpr int BM = vjp_bm<TC, C>();
  constexpr int NT = vjp_nt<C>();
  constexpr int RB = BM / 16;
  constexpr int CBW = C / 16 / (NT / 64);  // 16-channel blocks per wave
  constexpr int XLD = BM + lds_pad<TC>();
  constexpr int ALD = C + lds_pad<TC>();
  constexpr int SLD = C + 4;
  constexpr int NQ = NT / BM;  // threads per position in the per-position passes
  constexpr int CPQ = C / NQ;
  constexpr int VEC = 16 / sizeof(TC);
  static_assert(CPQ % VEC == 0, "per-thread channel run must be whole 16-byte chunks");
  constexpr int XS_BYTES = C * XLD * (int)sizeof(TC);
  constexpr int A_BYTES = BM * ALD * (int)sizeof(TC);
  constexpr int ST_BYTES = BM * SLD * 4;
  constexpr int R_BYTES = 2 * A_BYTES > ST_BYTES ? 2 * A_BYTES : ST_BYTES;
  __shared__ __attribute__((aligned(16))) char smem[XS_BYTES + R_BYTES];
  __shared__ float s_mean[BM], s_rstd[BM];
  constexpr int MXN = MHR ? BM * HM : 1;
  __shared__ float mx_gate[MXN], mx_sa[MXN], mx_sb[MXN], mx_pa[MXN], mx_pb[MXN], mx_dg[MXN];
  __shared__ float mx_w[MHR ? C : 1], mx_b[MHR ? C : 1];  // norm_center's affine, staged once
  TC* Xs = reinterpret_cast<TC*>(smem);                       // X [c][p], later dX
  TC* A1 = reinterpret_cast<TC*>(smem + XS_BYTES);            // xln, then gp
  TC* A2 = reinterpret_cast<TC*>(smem + XS_BYTES + A_BYTES);  // x, then gg
  float* stage = reinterpret_cast<float*>(smem + XS_BYTES);   // d(xln), fp32

  const int j0 = blockIdx.x * BM;
  const int i = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const size_t pe = (size_t)Np * Np;
  RouterFrags<TC, C> rf;
  if constexpr (MHR) {
    if (mx.wr != nullptr && wave_id() < RB) rf.load(mx, 0);
    for (int c = tid; c < C; c += NT) {
      mx_w[c] = lnow[c];
      mx_b[c] = lnob != nullptr ? lnob[c] : 0.f;
    }
  }
  auto tok = [&](int p) -> long {
    const int j = j0 + p;
    return (i < N && j < N) ? ((long)b * N + i) * N + j : -1;
  };

  // X tile, channel-major (rows of BM contiguous positions per channel)
  {
    constexpr int CPR = BM / VEC;
    const TC* Xb = X + (size_t)b * C * pe + (size_t)i * Np + j0;
    for (int idx = tid; idx < C * CPR; idx += NT) {
      const int c = idx / CPR;
      const int ch = idx % CPR;
      *reinterpret_cast<u32x4*>(Xs + c * XLD + ch * VEC) =
          *reinterpret_cast<const u32x4*>(Xb + (size_t)c * pe + ch * VEC);
    }
  }
  copy_tile_to_lds<TZ, TC, C, BM, NT>(
      [&](int p) -> const TZ* {
        const long t = tok(p);
        return t < 0 ? nullptr : x + t * C;
      },
      A2, ALD);
  __syncthreads();

  // LN_out statistics (fp32, two-pass) and xln = LN_out(X) into A1 [p][c] and to xln_out
  const int pq = tid / NQ;
  const int qq = tid % NQ;
  if constexpr (MHR) {
    mhr_gates<TC, C, BM, NT>(A2, ALD, mx, mx_gate, rf);
    mhr_stats<TC, C, BM, NT>(Xs, XLD, mx_gate, mx, eps, mx_sa, mx_sb, mx_pa);
    mhr_mix_write<TC, C, BM, NT>(Xs, XLD, mx_gate, mx_sa, mx_sb, mx, mx_w, mx_b, A1, ALD);
    __syncthreads();
    constexpr int CPR = C / VEC;
    for (int idx = tid; idx < BM * CPR; idx += NT) {
      const int p = idx / CPR;
      const int ch = (idx % CPR) * VEC;
      const long t = tok(p);
      if (t >= 0) *reinterpret_cast<u32x4*>(xln_out + t * C + ch) = *reinterpret_cast<const u32x4*>(A1 + p * ALD + ch);
    }
  } else {
    float xv[CPQ];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < CPQ; ++e) {
      xv[e] = to_f32(Xs[(qq * CPQ + e) * XLD + pq]);
      s += xv[e];
    }
    const float mean = group_sum<NQ>(s) * (1.0f / C);
    float v = 0.f;
#pragma unroll
    for (int e = 0; e < CPQ; ++e) {
      const float d = xv[e] - mean;
      v += d * d;
    }
    const float rstd = rsqrtf(group_sum<NQ>(v) * (1.0f / C) + eps);
    if (qq == 0) {
      s_mean[pq] = mean;
      s_rstd[pq] = rstd;
    }
    float y[CPQ];
#pragma unroll
    for (int e = 0; e < CPQ; ++e) {
      const int c = qq * CPQ + e;
      y[e] = (xv[e] - mean) * rstd * lnow[c] + lnob[c];
    }
    const long t = tok(pq);
#pragma unroll
    for (int e = 0; e < CPQ; e += VEC) {
      store_vec<TC, VEC>(A1 + pq * ALD + qq * CPQ + e, y + e);
      if (t >= 0) store_vec<TC, VEC>(xln_out + t * C + qq * CPQ + e, y + e);
    }
  }
  __syncthreads();

  // p = xln Wo^T, s = sigmoid(x Wog^T)
  const int w = wave_id();
  const int l = lane_id();
  int wrow0[CBW];
#pragma unroll
  for (int j = 0; j < CBW; ++j) wrow0[j] = (w * CBW + j) * 16;
  f32x4 accp[RB][CBW], accg[RB][CBW];
  zero_acc(accp);
  zero_acc(accg);
  gemm16_lds_x_w<TC, C, RB, CBW>(accp, A1, ALD, 0, Wo, C, wrow0);
  gemm16_lds_x_w<TC, C, RB, CBW>(accg, A2, ALD, 0, Wog, C, wrow0);
  __syncthreads();  // A1 / A2 are rewritten below

  // gp = g s, gg = g p s (1 - s), rounded to TC as the next GEMMs' operands
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int jb = 0; jb < CBW; ++jb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int p = rb * 16 + 4 * (l >> 4) + e;
        const int c = (w * CBW + jb) * 16 + (l & 15);
        const long t = tok(p);
        const float gv = t < 0 ? 0.f : to_f32(g[t * C + c]);
        const float sv = sigmoidf_(accg[rb][jb][e]);
        A1[p * ALD + c] = from_f32<TC>(gv * sv);
        A2[p * ALD + c] = from_f32<TC>(gv * accp[rb][jb][e] * sv * (1.f - sv));
      }
  __syncthreads();
  // gp, gg token-major [M][C] for the weight-gradient GEMMs: the tile's rows are contiguous
  {
    constexpr int CPR = C / VEC;
    for (int idx = tid; idx < BM * CPR; idx += NT) {
      const int p = idx / CPR;
      const int ch = (idx % CPR) * VEC;
      const long t = tok(p);
      if (t < 0) continue;
      *reinterpret_cast<u32x4*>(gp_out + t * C + ch) = *reinterpret_cast<const u32x4*>(A1 + p * ALD + ch);
      *reinterpret_cast<u32x4*>(gg_out + t * C + ch) = *reinterpret_cast<const u32x4*>(A2 + p * ALD + ch);
    }
  }

  // d(xln) = gp Wo, the output gate's x cotangent gg Wog
  f32x4 accd[RB][CBW], accx[RB][CBW];
  zero_acc(accd);
  zero_acc(accx);
  gemm16_lds_x_w<TC, C, RB, CBW>(accd, A1, ALD, 0, WoT, C, wrow0);
  gemm16_lds_x_w<TC, C, RB, CBW>(accx, A2, ALD, 0, WogT, C, wrow0);
  if constexpr (!MHR) {  // with the mix, gx also takes the router's share and leaves last
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int jb = 0; jb < CBW; ++jb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int p = rb * 16 + 4 * (l >> 4) + e;
          const int c = (w * CBW + jb) * 16 + (l & 15);
          const long t = tok(p);
          if (t >= 0) gx[t * C + c] = accx[rb][jb][e];
        }
  }
  __syncthreads();  // A1 / A2 dead: the fp32 stage takes their place
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int jb = 0; jb < CBW; ++jb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int p = rb * 16 + 4 * (l >> 4) + e;
        const int c = (w * CBW + jb) * 16 + (l & 15);
        stage[p * SLD + c] = accd[rb][jb][e];
      }
  __syncthreads();

  if constexpr (MHR) {
    // the mix's pullback; between its passes, the per-block partial sums of the affine
    // gradients (one thread per channel) while Xs still holds X
    const size_t blk = ((size_t)b * gridDim.y + i) * gridDim.x + blockIdx.x;
    mhr_mix_pullback<TC, C, BM, NT>(Xs, XLD, mx_gate, mx_sa, mx_sb, mx, mx_w, mx_b, stage, SLD, mx_dg, mx_pa, mx_pb,
                                    [&]() {
                                      mhr_affine_partials<TC, C, BM, NT>(Xs, XLD, mx_gate, mx_sa, mx_sb, mx, stage,
                                                                         SLD, partial + blk * 2 * C,
                                                                         partial + blk * 2 * C + C);
                                    });
    // the router logits' cotangent dr, and gx = gg Wog + dr Wr (x's share through the router)
    const int H = mx.heads;
    if (mx.wr != nullptr) {
      for (int pr = tid; pr < BM * H; pr += NT) {
        const int p = pr % BM, h = pr / BM;
        const float v = mhr_router_grad<BM>(mx_gate, mx_dg, mx, p, h);
        mx_pa[h * BM + p] = v;
        const long t = tok(p);
        if (t >= 0) dr[t * H + h] = v;
      }
      __syncthreads();
    }
#pragma unroll
    for (int jb = 0; jb < CBW; ++jb) {
      const int c = (w * CBW + jb) * 16 + (l & 15);
      float wc[HM];
#pragma unroll
      for (int h = 0; h < HM; ++h) wc[h] = (mx.wr != nullptr && h < H) ? mx.wr[(size_t)h * C + c] : 0.f;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int p = rb * 16 + 4 * (l >> 4) + e;
          float v = accx[rb][jb][e];
#pragma unroll
          for (int h = 0; h < HM; ++h)
            if (h < H) v += mx_pa[h * BM + p] * wc[h];
          const long t = tok(p);
          if (t >= 0) gx[t * C + c] = mx.wr != nullptr ? v : accx[rb][jb][e];
        }
    }
  } else {
  // Per-block partial sums of the LN_out affine gradients, one thread per channel.
  {
    const size_t blk = ((size_t)b * gridDim.y + i) * gridDim.x + blockIdx.x;
    for (int c = tid; c < C; c += NT) {
      float sw = 0.f, sb = 0.f;
      for (int p = 0; p < BM; ++p) {
        const float xn = (to_f32(Xs[c * XLD + p]) - s_mean[p]) * s_rstd[p];
        const float d = stage[p * SLD + c];
        sw += d * xn;
        sb += d;
      }
      partial[blk * 2 * C + c] = sw;
      partial[blk * 2 * C + C + c] = sb;
    }
  }
  __syncthreads();  // Xs is overwritten with dX below

  // LN_out pullback, in place over Xs: each thread owns (position pq, channels qq*CPQ..)
  {
    const float mean = s_mean[pq], rstd = s_rstd[pq];
    float u[CPQ], xn[CPQ];
    float su = 0.f, sux = 0.f;
#pragma unroll
    for (int e = 0; e < CPQ; ++e) {
      const int c = qq * CPQ + e;
      xn[e] = (to_f32(Xs[c * XLD + pq]) - mean) * rstd;
      u[e] = stage[pq * SLD + c] * lnow[c];
      su += u[e];
      sux += u[e] * xn[e];
    }
    su = group_sum<NQ>(su) * (1.0f / C);
    sux = group_sum<NQ>(sux) * (1.0f / C);
#pragma unroll
    for (int e = 0; e < CPQ; ++e) Xs[(qq * CPQ + e) * XLD + pq] = from_f32<TC>(rstd * (u[e] - su - xn[e] * sux));
  }
  }
  __syncthreads();
  {
    constexpr int CPR = BM / VEC;
    TC* Db = dX + (size_t)b * C * pe + (size_t)i * Np + j0;
    for (int idx = tid; idx < C * CPR; idx += NT) {
      const int c = idx / CPR;
      const int ch = idx % CPR;
      *reinterpret_cast<u32x4*>(Db + (size_t)c * pe + ch * VEC) =
          *reinterpret_cast<const u32x4*>(Xs + c * XLD + ch * VEC);
    }
  }
}

// Output VJP, persistent and weight-stationary (bf16 GEMMs, C = 128): the same steps as
// trimul_output_vjp_kernel, with one 512-thread block per CU walking 64-position tiles. Wave w
// takes the output columns 16 w .. +16 of all four GEMMs (xln Wo^T, x Wog^T, gp Wo, gg Wog);
// their B fragments (16x16x32 steps, lane: column l & 15, k = 32 s + 8 (l >> 4) ..) are rows of
// Wo, Wog, Wo^T, Wog^T and stay in registers for the whole kernel. The LN_out affine gradients
// accumulate per thread (channel tid & 127, positions 16 (tid >> 7) .. +16 of every tile) and
// leave as one partial sum per block.
struct OutputVjpWs {
  static constexpr int C = 128;
  static constexpr int BM = 64;
  static constexpr int NT = 512;
  static constexpr int XLD = BM + 8;  // X tile [c][p] (bf16)
  static constexpr int ALD = C + 8;   // xln / x, then gp / gg, [p][c] (bf16)
  static constexpr int SLD = C + 4;   // d(xln) [p][c] (fp32)
  static constexpr int NQ = NT / BM;  // threads per position in the per-position passes
  static constexpr int CPQ = C / NQ;
};

// acc[rb] (rows 16 rb .., columns of this wave) += A [64][C] (LDS, k contiguous) W, W's B
// fragments in registers.
PF_DEVICE void gemm_a_lds_w_regs(f32x4 (&acc)[4], const bf16* A, int lda, const bf16x8 (&wf)[4]) {
  const int l = lane_id();
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const bf16x8 af = *reinterpret_cast<const bf16x8*>(A + (16 * rb + (l & 15)) * lda + 32 * st + 8 * (l >> 4));
      acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wf[st], acc[rb], 0, 0, 0);
    }
}

template <class TZ>
__global__ __launch_bounds__(OutputVjpWs::NT) void trimul_output_vjp_ws_kernel(
    const TZ* __restrict__ g, const bf16* __restrict__ X, const TZ* __restrict__ x, const float* __restrict__ lnow,
    const float* __restrict__ lnob, float eps, const bf16* __restrict__ Wo, const bf16* __restrict__ Wog,
    const bf16* __restrict__ WoT, const bf16* __restrict__ WogT, int B, int N, int Np, bf16* __restrict__ gp_out,
    bf16* __restrict__ gg_out, bf16* __restrict__ xln_out, bf16* __restrict__ dX, float* __restrict__ gx,
    float* __restrict__ partial) {
  using Cfg = OutputVjpWs;
  constexpr int C = Cfg::C, BM = Cfg::BM, NT = Cfg::NT, XLD = Cfg::XLD, ALD = Cfg::ALD, SLD = Cfg::SLD;
  constexpr int NQ = Cfg::NQ, CPQ = Cfg::CPQ;
  constexpr int A_BYTES = BM * ALD * 2;
  constexpr int ST_BYTES = BM * SLD * 4;
  constexpr int R_BYTES = 2 * A_BYTES > ST_BYTES ? 2 * A_BYTES : ST_BYTES;
  __shared__ __attribute__((aligned(16))) bf16 Xs[C * XLD];  // X [c][p], later dX
  __shared__ __attribute__((aligned(16))) char rsm[R_BYTES];
  __shared__ float s_mean[BM], s_rstd[BM];
  __shared__ float s_lnw[C], s_lnb[C];
  __shared__ float red[2][NT];
  bf16* A1 = reinterpret_cast<bf16*>(rsm);            // xln, then gp
  bf16* A2 = reinterpret_cast<bf16*>(rsm + A_BYTES);  // x, then gg
  float* stage = reinterpret_cast<float*>(rsm);       // d(xln), fp32

  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const size_t pe = (size_t)Np * Np;
  const int tpl = Np / BM;
  const int ntiles = B * Np * tpl;  // every tile of the planes, padding included (< 2^31)
  const int G = gridDim.x;
  const int col = 16 * w + (l & 15);  // this lane's output column in all four GEMMs

  bf16x8 wo[4], wog[4], wot[4], wogt[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const int k = 32 * st + 8 * (l >> 4);
    wo[st] = *reinterpret_cast<const bf16x8*>(Wo + (size_t)col * C + k);
    wog[st] = *reinterpret_cast<const bf16x8*>(Wog + (size_t)col * C + k);
    wot[st] = *reinterpret_cast<const bf16x8*>(WoT + (size_t)col * C + k);
    wogt[st] = *reinterpret_cast<const bf16x8*>(WogT + (size_t)col * C + k);
  }
  const int pq = tid / NQ;
  const int qq = tid % NQ;
  if (tid < C) {
    s_lnw[tid] = lnow[tid];
    s_lnb[tid] = lnob[tid];
  }
  float pw = 0.f, pb = 0.f;  // LN_out affine partials of channel tid & 127

  for (int tile = blockIdx.x; tile < ntiles; tile += G) {
    const int b = tile / (Np * tpl);
    const int rem = tile - b * (Np * tpl);
    const int i = rem / tpl;
    const int j0 = (rem - i * tpl) * BM;
    const int nvalid = i < N ? max(0, min(BM, N - j0)) : 0;
    const long tok0 = ((long)b * N + i) * N + j0;  // position p is token tok0 + p (p < nvalid)
    if (nvalid == 0) {
      // padding only: dX is zero there (the contraction's cotangent GEMMs read it)
      bf16* Db = dX + (size_t)b * C * pe + (size_t)i * Np + j0;
#pragma unroll
      for (int it = 0; it < C * BM / 8 / NT; ++it) {
        const int idx = tid + it * NT;
        *reinterpret_cast<u32x4*>(Db + (size_t)(idx / (BM / 8)) * pe + (idx % (BM / 8)) * 8) = u32x4{0u, 0u, 0u, 0u};
      }
      continue;  // block-uniform
    }

    // X tile, channel-major (rows of 64 contiguous positions per channel); x rows
    {
      const bf16* Xb = X + (size_t)b * C * pe + (size_t)i * Np + j0;
#pragma unroll
      for (int it = 0; it < C * BM / 8 / NT; ++it) {
        const int idx = tid + it * NT;
        const int c = idx / (BM / 8);
        const int ch = (idx % (BM / 8)) * 8;
        *reinterpret_cast<u32x4*>(Xs + c * XLD + ch) = *reinterpret_cast<const u32x4*>(Xb + (size_t)c * pe + ch);
      }
    }
    copy_tile_to_lds<TZ, bf16, C, BM, NT>(
        [&](int p) -> const TZ* { return p < nvalid ? x + (tok0 + p) * C : nullptr; }, A2, ALD);
    __syncthreads();

    // LN_out statistics (fp32, two-pass) and xln = LN_out(X) into A1 and xln_out
    {
      float xv[CPQ];
      float sm = 0.f;
#pragma unroll
      for (int e = 0; e < CPQ; ++e) {
        xv[e] = to_f32(Xs[(qq * CPQ + e) * XLD + pq]);
        sm += xv[e];
      }
      const float mean = group_sum<NQ>(sm) * (1.0f / C);
      float v = 0.f;
#pragma unroll
      for (int e = 0; e < CPQ; ++e) {
        const float d = xv[e] - mean;
        v += d * d;
      }
      const float rstd = rsqrtf(group_sum<NQ>(v) * (1.0f / C) + eps);
      if (qq == 0) {
        s_mean[pq] = mean;
        s_rstd[pq] = rstd;
      }
      float y[CPQ];
#pragma unroll
      for (int e = 0; e < CPQ; ++e) y[e] = (xv[e] - mean) * rstd * s_lnw[qq * CPQ + e] + s_lnb[qq * CPQ + e];
#pragma unroll
      for (int e = 0; e < CPQ; e += 8) {
        store_vec<bf16, 8>(A1 + pq * ALD + qq * CPQ + e, y + e);
        if (pq < nvalid) store_vec<bf16, 8>(xln_out + (tok0 + pq) * C + qq * CPQ + e, y + e);
      }
    }
    __syncthreads();

    // p = xln Wo^T, s = sigmoid(x Wog^T)
    f32x4 accp[4] = {}, accg[4] = {};
    gemm_a_lds_w_regs(accp, A1, ALD, wo);
    gemm_a_lds_w_regs(accg, A2, ALD, wog);
    __syncthreads();  // A1 / A2 are rewritten below

    // gp = g s, gg = g p s (1 - s), rounded to bf16 as the next GEMMs' operands
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int p = 16 * rb + 4 * (l >> 4) + e;
        const float gv = p < nvalid ? to_f32(g[(tok0 + p) * C + col]) : 0.f;
        const float sv = sigmoidf_(accg[rb][e]);
        A1[p * ALD + col] = from_f32<bf16>(gv * sv);
        A2[p * ALD + col] = from_f32<bf16>(gv * accp[rb][e] * sv * (1.f - sv));
      }
    __syncthreads();
    // gp, gg token-major for the weight-gradient GEMMs
#pragma unroll
    for (int it = 0; it < BM * C / 8 / NT; ++it) {
      const int idx = tid + it * NT;
      const int p = idx / (C / 8);
      const int ch = (idx % (C / 8)) * 8;
      if (p < nvalid) {
        *reinterpret_cast<u32x4*>(gp_out + (tok0 + p) * C + ch) = *reinterpret_cast<const u32x4*>(A1 + p * ALD + ch);
        *reinterpret_cast<u32x4*>(gg_out + (tok0 + p) * C + ch) = *reinterpret_cast<const u32x4*>(A2 + p * ALD + ch);
      }
    }

    // d(xln) = gp Wo, the output gate's x cotangent gg Wog
    f32x4 accd[4] = {}, accx[4] = {};
    gemm_a_lds_w_regs(accd, A1, ALD, wot);
    gemm_a_lds_w_regs(accx, A2, ALD, wogt);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int p = 16 * rb + 4 * (l >> 4) + e;
        if (p < nvalid) gx[(tok0 + p) * C + col] = accx[rb][e];
      }
    __syncthreads();  // A1 / A2 dead: the fp32 stage takes their place
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int e = 0; e < 4; ++e) stage[(16 * rb + 4 * (l >> 4) + e) * SLD + col] = accd[rb][e];
    __syncthreads();

    // LN_out affine partials: channel tid & 127 over positions 16 (tid >> 7) .. +16 (positions
    // past N have d = 0)
    {
      const int c = tid & (C - 1);
      const int p0 = 16 * (tid >> 7);
#pragma unroll 4
      for (int p = p0; p < p0 + 16; ++p) {
        const float xn = (to_f32(Xs[c * XLD + p]) - s_mean[p]) * s_rstd[p];
        const float d = stage[p * SLD + c];
        pw += d * xn;
        pb += d;
      }
    }
    __syncthreads();  // Xs is overwritten with dX below

    // LN_out pullback, in place over Xs: each thread owns (position pq, channels qq*CPQ..)
    {
      const float mean = s_mean[pq], rstd = s_rstd[pq];
      float u[CPQ], xn[CPQ];
      float su = 0.f, sux = 0.f;
#pragma unroll
      for (int e = 0; e < CPQ; ++e) {
        const int c = qq * CPQ + e;
        xn[e] = (to_f32(Xs[c * XLD + pq]) - mean) * rstd;
        u[e] = stage[pq * SLD + c] * s_lnw[c];
        su += u[e];
        sux += u[e] * xn[e];
      }
      su = group_sum<NQ>(su) * (1.0f / C);
      sux = group_sum<NQ>(sux) * (1.0f / C);
#pragma unroll
      for (int e = 0; e < CPQ; ++e)
        Xs[(qq * CPQ + e) * XLD + pq] = from_f32<bf16>(rstd * (u[e] - su - xn[e] * sux));
    }
    __syncthreads();
    {
      bf16* Db = dX + (size_t)b * C * pe + (size_t)i * Np + j0;
#pragma unroll
      for (int it = 0; it < C * BM / 8 / NT; ++it) {
        const int idx = tid + it * NT;
        const int c = idx / (BM / 8);
        const int ch = (idx % (BM / 8)) * 8;
        *reinterpret_cast<u32x4*>(Db + (size_t)c * pe + ch) = *reinterpret_cast<const u32x4*>(Xs + c * XLD + ch);
      }
    }
    __syncthreads();  // Xs, A1 / A2 and the stage free for the next tile
  }
  // this block's partials: the four position quarters added in order
  red[0][tid] = pw;
  red[1][tid] = pb;
  __syncthreads();
  if (tid < C) {
    float sw = 0.f, sb = 0.f;
#pragma unroll
    for (int q = 0; q < NT / C; ++q) {
      sw += red[0][q * C + tid];
      sb += red[1][q * C + tid];
    }
    partial[(size_t)blockIdx.x * 2 * C + tid] = sw;
    partial[(size_t)blockIdx.x * 2 * C + C + tid] = sb;
  }
}

// out[k] = sum over blocks of partial[blk][k], k < 2C (w then b), in a fixed order.
__global__ __launch_bounds__(256) void trimul_ln_grad_reduce_kernel(const float* __restrict__ partial, long nblk,
                                                                    int C2, float* __restrict__ dw,
                                                                    float* __restrict__ db) {
  __shared__ float red[256];
  const int k = blockIdx.x;
  float s = 0.f;
  for (long blk = threadIdx.x; blk < nblk; blk += 256) s += partial[blk * C2 + k];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const int C = C2 / 2;
    if (k < C)
      dw[k] = red[0];
    else
      db[k - C] = red[0];
  }
}

// MHR router weight gradient dWr = dr^T x: block b takes tokens [b tpb, (b + 1) tpb); thread
// (phase ph, channel c), NT = C x phases, accumulates sum_t dr[t][h] x[t][c] over its phase's
// tokens for every head; the phases are summed through LDS and the block leaves its [H][C]
// partial, reduced over blocks by trimul_ln_grad_reduce_kernel.
template <class TX, int H>
__global__ __launch_bounds__(256) void mhr_router_wgrad_kernel(const float* __restrict__ dr, const TX* __restrict__ x,
                                                               long M, int C, long tpb, float* __restrict__ partial) {
  constexpr int CH = 64;  // tokens per staged chunk of dr
  __shared__ float drs[CH * H];
  __shared__ float red[256];
  const int tid = threadIdx.x;
  const int nph = 256 / C;  // C in {64, 128, 256}
  const int c = tid % C, ph = tid / C;
  const long t0 = (long)blockIdx.x * tpb;
  const long t1 = t0 + tpb < M ? t0 + tpb : M;
  float acc[H];
#pragma unroll
  for (int h = 0; h < H; ++h) acc[h] = 0.f;
  for (long tc = t0; tc < t1; tc += CH) {
    const int n = (int)(t1 - tc < CH ? t1 - tc : CH);
    __syncthreads();
    for (int i = tid; i < n * H; i += 256) drs[i] = dr[tc * H + i];
    __syncthreads();
#pragma unroll 4
    for (int tt = ph; tt < n; tt += nph) {
      const float xv = to_f32(x[(tc + tt) * C + c]);
#pragma unroll
      for (int h = 0; h < H; ++h) acc[h] += drs[tt * H + h] * xv;  // one address per wave: a broadcast
    }
  }
  // sum the phases (at most 4) through LDS, one head at a time
  float* out = partial + (size_t)blockIdx.x * H * C;
#pragma unroll
  for (int h = 0; h < H; ++h) {
    __syncthreads();
    red[tid] = acc[h];
    __syncthreads();
    if (ph == 0) {
      float v = 0.f;
      for (int q = 0; q < nph; ++q) v += red[q * C + c];
      out[h * C + c] = v;
    }
  }
}

// ------------------------------------------------------------------ project VJP
// Packed weights w4 [4C][C] as the forward K1 reads them (16-channel blocks, rows
// 64 j + 16 kind + r: a proj, a gate, b proj, b gate); w4t = w4^T [C][4C].
template <class TZ, class TC, int C>
__global__ __launch_bounds__(vjp_nt<C>()) void trimul_project_vjp_kernel(const TC* __restrict__ dplanes,
                                                                 const TZ* __restrict__ x,
                                                                 const float* __restrict__ mask,
                                                                 const TC* __restrict__ w4,
                                                                 const TC* __restrict__ w4t,
                                                                 const float* __restrict__ gx_in, int B, int N,
                                                                 int Np, int outgoing, TC* __restrict__ gpg,
                                                                 TC* __restrict__ xw, TZ* __restrict__ dx) {
  constexpr int BM = vjp_bm<TC, C>();
  constexpr int NT = vjp_nt<C>();
  constexpr int RB = BM / 16;
  constexpr int CBW = C / 16 / (NT / 64);
  constexpr int LDA = C + lds_pad<TC>();
  constexpr int SLD = BM + lds_pad<TC>();
  constexpr int GLD = 4 * C + lds_pad<TC>();
  constexpr int VEC = 16 / sizeof(TC);
  constexpr int A_BYTES = BM * LDA * (int)sizeof(TC);
  constexpr int S_BYTES = 2 * C * SLD * (int)sizeof(TC);
  constexpr int G_BYTES = BM * GLD * (int)sizeof(TC);
  constexpr int SMEM = (A_BYTES + S_BYTES) > G_BYTES ? (A_BYTES + S_BYTES) : G_BYTES;
  __shared__ __attribute__((aligned(16))) char smem[SMEM];
  __shared__ float mk[BM];
  TC* A = reinterpret_cast<TC*>(smem);
  TC* S = reinterpret_cast<TC*>(smem + A_BYTES);
  TC* G = reinterpret_cast<TC*>(smem);

  const int t0 = blockIdx.x * BM;
  const int line = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const size_t pe = (size_t)Np * Np;
  auto pos_of = [&](int p) -> long {
    const int t = t0 + p;
    if (line >= N || t >= N) return -1;
    return outgoing ? (long)line * N + t : (long)t * N + line;
  };
  auto tok = [&](int p) -> long {
    const long pos = pos_of(p);
    return pos < 0 ? -1 : (long)b * N * N + pos;
  };
  copy_tile_to_lds<TZ, TC, C, BM, NT>(
      [&](int p) -> const TZ* {
        const long t = tok(p);
        return t < 0 ? nullptr : x + t * C;
      },
      A, LDA);
  if (tid < BM) {
    const long t = tok(tid);
    mk[tid] = t < 0 ? 0.f : mask[t];
  }
  if (!outgoing) {
    __syncthreads();
    constexpr int CPR = C / VEC;
    for (int idx = tid; idx < BM * CPR; idx += NT) {
      const int p = idx / CPR;
      const int ch = (idx % CPR) * VEC;
      if (line >= N || t0 + p >= N) continue;
      *reinterpret_cast<u32x4*>(xw + (((size_t)b * N + line) * N + t0 + p) * C + ch) =
          *reinterpret_cast<const u32x4*>(A + p * LDA + ch);
    }
  }
  {
    // cotangents of this block's plane entries: rows (plane, channel) of BM positions
    constexpr int CPR = BM / VEC;
    for (int idx = tid; idx < 2 * C * CPR; idx += NT) {
      const int row = idx / CPR;
      const int ch = idx % CPR;
      const int plane = row / C;
      const int c = row % C;
      const TC* src = dplanes + ((size_t)plane * B * C + (size_t)b * C + c) * pe + (size_t)line * Np + t0 + ch * VEC;
      *reinterpret_cast<u32x4*>(S + row * SLD + ch * VEC) = *reinterpret_cast<const u32x4*>(src);
    }
  }
  __syncthreads();

  const int w = wave_id();
  const int l = lane_id();
  f32x4 acc[RB][4 * CBW];
  zero_acc(acc);
  int wrow0[4 * CBW];
#pragma unroll
  for (int j = 0; j < 4 * CBW; ++j) wrow0[j] = (w * CBW + j / 4) * 64 + (j % 4) * 16;
  gemm16_lds_x_w<TC, C, RB, 4 * CBW>(acc, A, LDA, 0, w4, C, wrow0);

  // G = (gp_a, gg_a, gp_b, gg_b) in place of (proj_a, gate_a, proj_b, gate_b)
#pragma unroll
  for (int cbi = 0; cbi < CBW; ++cbi) {
    const int ch = (w * CBW + cbi) * 16 + (l & 15);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p = rb * 16 + 4 * (l >> 4) + r;
        const float m = mk[p];
        const float ga = to_f32(S[ch * SLD + p]) * m;
        const float gb = to_f32(S[(C + ch) * SLD + p]) * m;
        const float pa = acc[rb][4 * cbi + 0][r], sa = sigmoidf_(acc[rb][4 * cbi + 1][r]);
        const float pb = acc[rb][4 * cbi + 2][r], sb = sigmoidf_(acc[rb][4 * cbi + 3][r]);
        acc[rb][4 * cbi + 0][r] = ga * sa;
        acc[rb][4 * cbi + 1][r] = ga * pa * sa * (1.f - sa);
        acc[rb][4 * cbi + 2][r] = gb * sb;
        acc[rb][4 * cbi + 3][r] = gb * pb * sb * (1.f - sb);
      }
  }
  __syncthreads();  // A and S dead: G takes their place
#pragma unroll
  for (int j = 0; j < 4 * CBW; ++j)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p = rb * 16 + 4 * (l >> 4) + r;
        G[p * GLD + wrow0[j] + (l & 15)] = from_f32<TC>(acc[rb][j][r]);
      }
  __syncthreads();
  // G token-major [M][4C] in this kernel's walk order (position (line, t) at row
  // b N^2 + line N + t): the tile's rows are contiguous. For the outgoing direction that is the
  // token order; for the incoming one x is written in the same order (xw, before the tile is
  // reused), so that the packed weights' gradient G^T xw needs no transposed copy.
  {
    constexpr int CPR = 4 * C / VEC;  // 16-byte pieces per G row
    for (int idx = tid; idx < BM * CPR; idx += NT) {
      const int p = idx / CPR;
      const int ch = (idx % CPR) * VEC;
      if (line >= N || t0 + p >= N) continue;
      *reinterpret_cast<u32x4*>(gpg + (((size_t)b * N + line) * N + t0 + p) * 4 * C + ch) =
          *reinterpret_cast<const u32x4*>(G + p * GLD + ch);
    }
  }

  // dx = gx + G W4 (k = 4C)
  f32x4 acc2[RB][CBW];
  zero_acc(acc2);
  int wrow1[CBW];
#pragma unroll
  for (int j = 0; j < CBW; ++j) wrow1[j] = (w * CBW + j) * 16;
  gemm16_lds_x_w<TC, 4 * C, RB, CBW>(acc2, G, GLD, 0, w4t, 4 * C, wrow1);
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int jb = 0; jb < CBW; ++jb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int p = rb * 16 + 4 * (l >> 4) + e;
        const int c = wrow1[jb] + (l & 15);
        const long t = tok(p);
        if (t >= 0) dx[t * C + c] = from_f32<TZ>(gx_in[t * C + c] + acc2[rb][jb][e]);
      }
}

// Project VJP, persistent and weight-stationary (bf16 GEMMs, C = 128; weights packed in
// 32-channel blocks, rows 128 j + 32 kind + r, as the persistent K1 reads them). One 512-thread
// block per CU walks 64-position tiles along the lines. Wave w holds in MFMA operand registers,
// for the whole kernel, the proj and gate rows of plane w >> 2 (a | b), channels 32 (w & 3) ..
// +32, as the A operand of acc^T [row][position] = W4 x^T (lane: row l & 31, 8 k per step), so
// these weights are read once per CU, not once per tile. For dx [position][c] = G W4, wave w
// takes the columns c = 16 w .. +16; their B fragments (16x16x32 steps, lane: column l & 15,
// rows 32 s + 8 (l >> 4) ..) are 16-byte pieces of the rows of W4^T, read from L2 four steps
// at a time (registers for all sixteen would cost the occupancy). Per tile: x rows -> LDS (bf16), each
// wave's cotangent rows (32 channels x 64 positions of dP or dQ) -> its private LDS stage,
// both loaded a tile ahead into registers; acc^T, G in registers, G rows -> the LDS G tile;
// then G leaves token-major (1 KB rows) and dx = gx_in + G W4 is formed from the G tile.
struct ProjectVjpWs {
  static constexpr int C = 128;
  static constexpr int BP = 64;         // positions per tile
  static constexpr int NW = 8;          // waves per block
  static constexpr int NT = 64 * NW;
  static constexpr int XLD = C + 8;     // x tile rows (bf16): 272 bytes, conflict-free 16-byte reads
  static constexpr int GLD = 4 * C + 8; // G tile rows (bf16): 1040 bytes
  static constexpr int SLD = BP + 8;    // cotangent stage rows (bf16): [32 channels][64 positions]
};

template <class TZ>
__global__ __launch_bounds__(ProjectVjpWs::NT) void trimul_project_vjp_ws_kernel(
    const bf16* __restrict__ dplanes, const TZ* __restrict__ x, const float* __restrict__ mask,
    const bf16* __restrict__ w4, const bf16* __restrict__ w4t, const float* __restrict__ gx_in, int B, int N,
    int Np, int outgoing, bf16* __restrict__ gpg, bf16* __restrict__ xw, TZ* __restrict__ dx) {
  using Cfg = ProjectVjpWs;
  constexpr int C = Cfg::C, BP = Cfg::BP, NT = Cfg::NT, XLD = Cfg::XLD, GLD = Cfg::GLD, SLD = Cfg::SLD;
  constexpr int XV = 16 / sizeof(TZ);       // x elements per 16-byte load
  constexpr int XL = BP * C / XV / NT;      // x loads per thread per tile
  __shared__ __attribute__((aligned(16))) bf16 xs[BP * XLD];
  __shared__ __attribute__((aligned(16))) float mks[BP];
  __shared__ __attribute__((aligned(16))) bf16 gs[BP * GLD];
  __shared__ __attribute__((aligned(16))) bf16 cst_all[Cfg::NW][32 * SLD];

  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const int hh = l >> 5;
  const int pl = w >> 2;  // plane: 0 a (dP), 1 b (dQ)
  const int cj = w & 3;   // 32-channel chunk
  bf16* cst = cst_all[w];
  const size_t pe = (size_t)Np * Np;
  const int tpl = (N + BP - 1) / BP;
  const int ntiles = B * N * tpl;  // < 2^31 (checked at launch)
  const int G = gridDim.x;

  // Weights, once. G operand: rows 128 cj + 32 (2 pl + kind) + (l & 31), k = 16 ks + 8 hh + e.
  bf16x8 wa[2][C / 16];
#pragma unroll
  for (int kind = 0; kind < 2; ++kind) {
    const bf16* r = w4 + (size_t)(128 * cj + 32 * (2 * pl + kind) + (l & 31)) * C + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < C / 16; ++ks) wa[kind][ks] = *reinterpret_cast<const bf16x8*>(r + 16 * ks);
  }
  // dx operand: row 16 w + (l & 15) of W4^T, k = 32 s + 8 (l >> 4) + e.
  const bf16* wbrow = w4t + (size_t)(16 * w + (l & 15)) * 4 * C + 8 * (l >> 4);

  auto tile_coords = [&](int tile, int& b, int& line, int& t0) {
    b = tile / (N * tpl);
    const int rem = tile - b * (N * tpl);
    line = rem / tpl;
    t0 = (rem - line * tpl) * BP;
  };
  auto tok = [&](int b, int line, int t) -> long {
    return (long)b * N * N + (outgoing ? (long)line * N + t : (long)t * N + line);
  };
  // Next tile's x rows (thread: XL 16-byte pieces), mask value (threads < BP) and this wave's
  // cotangent rows (lane: row 8 it + (l >> 3), 8 positions), in registers. Positions past N
  // read a clamped real row; their mask and G are zero and nothing is stored for them.
  u32x4 xr[XL], cr[4];
  float mr = 0.f;
  auto issue = [&](int tile) __attribute__((always_inline)) {
    int b, line, t0;
    tile_coords(tile, b, line, t0);
#pragma unroll
    for (int q = 0; q < XL; ++q) {
      const int idx = tid + q * NT;
      const int p = idx / (C / XV);
      const int ch = (idx % (C / XV)) * XV;
      xr[q] = *reinterpret_cast<const u32x4*>(x + tok(b, line, min(t0 + p, N - 1)) * C + ch);
    }
    if (tid < BP) mr = t0 + tid < N ? mask[tok(b, line, t0 + tid)] : 0.f;
    const bf16* cb = dplanes + ((size_t)(pl * B + b) * C + 32 * cj) * pe + (size_t)line * Np + t0 + 8 * (l & 7);
#pragma unroll
    for (int it = 0; it < 4; ++it) cr[it] = *reinterpret_cast<const u32x4*>(cb + (size_t)(8 * it + (l >> 3)) * pe);
  };
  auto stage = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < XL; ++q) {
      const int idx = tid + q * NT;
      const int p = idx / (C / XV);
      const int ch = (idx % (C / XV)) * XV;
      float v[XV];
      unpack16<TZ>(xr[q], v);
      store_vec<bf16, XV>(xs + p * XLD + ch, v);
    }
    if (tid < BP) mks[tid] = mr;
#pragma unroll
    for (int it = 0; it < 4; ++it)
      *reinterpret_cast<u32x4*>(cst + (8 * it + (l >> 3)) * SLD + 8 * (l & 7)) = cr[it];
  };

  int tile = blockIdx.x;
  if (tile < ntiles) issue(tile);
  for (; tile < ntiles; tile += G) {
    int b, line, t0;
    tile_coords(tile, b, line, t0);
    stage();
    if (tile + G < ntiles) issue(tile + G);
    __syncthreads();  // x tile, masks and stages of this tile

    // acc^T [row][position] per 32-position half, then G = (g s, g p s (1 - s)) into gs.
#pragma unroll 1
    for (int pt = 0; pt < 2; ++pt) {
      f32x16 acc[2] = {};
      const bf16* xrow = xs + (32 * pt + (l & 31)) * XLD + 8 * hh;
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        const bf16x8 xf = *reinterpret_cast<const bf16x8*>(xrow + 16 * ks);
        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa[0][ks], xf, acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa[1][ks], xf, acc[1], 0, 0, 0);
      }
      const int p = 32 * pt + (l & 31);
      const float m = mks[p];
      bf16* grow = gs + p * GLD + 128 * cj + 64 * pl;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float gp[4], gg[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * j + e;
          const float g = to_f32(cst[(8 * j + 4 * hh + e) * SLD + p]) * m;
          const float sg = sigmoidf_(acc[1][r]);
          gp[e] = g * sg;
          gg[e] = g * acc[0][r] * sg * (1.f - sg);
        }
        store_vec<bf16, 4>(grow + 8 * j + 4 * hh, gp);
        store_vec<bf16, 4>(grow + 32 + 8 * j + 4 * hh, gg);
      }
    }
    __syncthreads();  // G tile

    // G rows token-major (walk order), 1 KB each; x rows in walk order for the incoming
    // direction.
    const int nvalid = min(BP, N - t0);
    bf16* gdst = gpg + (((size_t)b * N + line) * N + t0) * 4 * C;
#pragma unroll
    for (int it = 0; it < BP * 4 * C / 8 / NT; ++it) {
      const int idx = tid + it * NT;
      const int p = idx / (4 * C / 8);
      const int ch = (idx % (4 * C / 8)) * 8;
      if (p < nvalid)
        *reinterpret_cast<u32x4*>(gdst + (size_t)p * 4 * C + ch) = *reinterpret_cast<const u32x4*>(gs + p * GLD + ch);
    }
    if (!outgoing) {
      bf16* xdst = xw + (((size_t)b * N + line) * N + t0) * C;
#pragma unroll
      for (int it = 0; it < BP * C / 8 / NT; ++it) {
        const int idx = tid + it * NT;
        const int p = idx / (C / 8);
        const int ch = (idx % (C / 8)) * 8;
        if (p < nvalid)
          *reinterpret_cast<u32x4*>(xdst + (size_t)p * C + ch) = *reinterpret_cast<const u32x4*>(xs + p * XLD + ch);
      }
    }

    // dx [position][16 w + (l & 15)] = gx_in + G W4 (k = 4C in 32-row steps)
    const int c = 16 * w + (l & 15);
    f32x4 acc2[BP / 16] = {};
#pragma unroll 1
    for (int s4 = 0; s4 < 4 * C / 32; s4 += 4) {
      bf16x8 wb[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) wb[u] = *reinterpret_cast<const bf16x8*>(wbrow + 32 * (s4 + u));
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int rb = 0; rb < BP / 16; ++rb) {
          const bf16x8 gf =
              *reinterpret_cast<const bf16x8*>(gs + (16 * rb + (l & 15)) * GLD + 32 * (s4 + u) + 8 * (l >> 4));
          acc2[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(gf, wb[u], acc2[rb], 0, 0, 0);
        }
    }
    // position p of the tile is token tbase + p tstr
    const long tbase = tok(b, line, t0);
    const long tstr = outgoing ? 1 : N;
    const float* gxt = gx_in + tbase * C + c;
    TZ* dxt = dx + tbase * C + c;
#pragma unroll
    for (int rb = 0; rb < BP / 16; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p = 16 * rb + 4 * (l >> 4) + r;
        if (p < nvalid) dxt[p * tstr * C] = from_f32<TZ>(gxt[p * tstr * C] + acc2[rb][r]);
      }
    __syncthreads();  // x tile, stages and G tile free for the next tile
  }
}

// dst[g] = src[g]^T for G planes of [Np][Np] (64 x 64 tiles through LDS).
template <class T>
__global__ __launch_bounds__(256) void plane_transpose_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                              int Np) {
  __shared__ T t[64][65];
  const size_t base = (size_t)blockIdx.z * Np * Np;
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int r = i / 64, c = i % 64;
    t[r][c] = src[base + (size_t)(r0 + r) * Np + c0 + c];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int r = i / 64, c = i % 64;
    dst[base + (size_t)(c0 + r) * Np + r0 + c] = t[c][r];
  }
}

template <class TC, int C>
size_t out_vjp_partials(int B, int N) {
  const int Np = pf::pad128(N);
  return (size_t)B * Np * (Np / vjp_bm<TC, C>()) * 2 * C * sizeof(float);
}

// mx.heads > 0 runs the MHR pullback (always the generic kernel); dr its router cotangent.
template <class TZ, class TC, int C>
int output_vjp_launch(const void* g, const void* X, const void* x, const float* lnow, const float* lnob, float eps,
                      const void* wo, const void* wog, const void* wot, const void* wogt, int B, int N, void* gp,
                      void* gg, void* xln, void* dX, float* gx, float* dlnw, float* dlnb, void* ws, hipStream_t s,
                      const MixSpec& mx, float* dr) {
  const int Np = pf::pad128(N);
  float* partial = static_cast<float*>(ws);
  if (mx.heads > 0) {
    constexpr int BM = vjp_bm<TC, C>();
    if (mx.heads <= kMhrHeadsSmall)
      trimul_output_vjp_kernel<TZ, TC, C, true, kMhrHeadsSmall><<<dim3(Np / BM, Np, B), vjp_nt<C>(), 0, s>>>(
          (const TZ*)g, (const TC*)X, (const TZ*)x, lnow, lnob, eps, (const TC*)wo, (const TC*)wog, (const TC*)wot,
          (const TC*)wogt, B, N, Np, (TC*)gp, (TC*)gg, (TC*)xln, (TC*)dX, gx, partial, mx, dr);
    else
      trimul_output_vjp_kernel<TZ, TC, C, true><<<dim3(Np / BM, Np, B), vjp_nt<C>(), 0, s>>>(
          (const TZ*)g, (const TC*)X, (const TZ*)x, lnow, lnob, eps, (const TC*)wo, (const TC*)wog, (const TC*)wot,
          (const TC*)wogt, B, N, Np, (TC*)gp, (TC*)gg, (TC*)xln, (TC*)dX, gx, partial, mx, dr);
    if (int e = pf::check_launch("trimul_output_vjp")) return e;
    const long nblk = (long)B * Np * (Np / BM);
    trimul_ln_grad_reduce_kernel<<<2 * C, 256, 0, s>>>(partial, nblk, 2 * C, dlnw, dlnb);
    return pf::check_launch("trimul_ln_grad_reduce");
  }
  if constexpr (sizeof(TC) == 2 && C == 128) {
    const long ntiles = (long)B * Np * (Np / OutputVjpWs::BM);
    PF_REQUIRE(ntiles < (1L << 31), PF_ERR_UNSUPPORTED, "trimul_output_vjp: B=%d N=%d too large", B, N);
    const int nblk = (int)std::min<long>(ntiles, pf::cu_count());
    trimul_output_vjp_ws_kernel<TZ><<<nblk, OutputVjpWs::NT, 0, s>>>(
        (const TZ*)g, (const bf16*)X, (const TZ*)x, lnow, lnob, eps, (const bf16*)wo, (const bf16*)wog,
        (const bf16*)wot, (const bf16*)wogt, B, N, Np, (bf16*)gp, (bf16*)gg, (bf16*)xln, (bf16*)dX, gx, partial);
    if (int e = pf::check_launch("trimul_output_vjp")) return e;
    trimul_ln_grad_reduce_kernel<<<2 * C, 256, 0, s>>>(partial, nblk, 2 * C, dlnw, dlnb);
    return pf::check_launch("trimul_ln_grad_reduce");
  }
  constexpr int BM = vjp_bm<TC, C>();
  const dim3 grid(Np / BM, Np, B);
  trimul_output_vjp_kernel<TZ, TC, C><<<grid, vjp_nt<C>(), 0, s>>>(
      (const TZ*)g, (const TC*)X, (const TZ*)x, lnow, lnob, eps, (const TC*)wo, (const TC*)wog, (const TC*)wot,
      (const TC*)wogt, B, N, Np, (TC*)gp, (TC*)gg, (TC*)xln, (TC*)dX, gx, partial, mx, dr);
  if (int e = pf::check_launch("trimul_output_vjp")) return e;
  const long nblk = (long)B * Np * (Np / BM);
  trimul_ln_grad_reduce_kernel<<<2 * C, 256, 0, s>>>(partial, nblk, 2 * C, dlnw, dlnb);
  return pf::check_launch("trimul_ln_grad_reduce");
}

template <class TZ, class TC, int C>
int project_vjp_launch(const void* dplanes, const void* x, const float* mask, const void* w4, const void* w4t,
                       const float* gx_in, int B, int N, int outgoing, void* gpg, void* xw, void* dx, hipStream_t s) {
  const int Np = pf::pad128(N);
  if constexpr (sizeof(TC) == 2 && C == 128) {
    const long ntiles = (long)B * N * ((N + ProjectVjpWs::BP - 1) / ProjectVjpWs::BP);
    PF_REQUIRE(ntiles < (1L << 31), PF_ERR_UNSUPPORTED, "trimul_project_vjp: B=%d N=%d too large", B, N);
    const int nblk = (int)std::min<long>(ntiles, pf::cu_count());
    trimul_project_vjp_ws_kernel<TZ><<<nblk, ProjectVjpWs::NT, 0, s>>>(
        (const bf16*)dplanes, (const TZ*)x, mask, (const bf16*)w4, (const bf16*)w4t, gx_in, B, N, Np, outgoing,
        (bf16*)gpg, (bf16*)xw, (TZ*)dx);
    return pf::check_launch("trimul_project_vjp");
  }
  constexpr int BM = vjp_bm<TC, C>();
  trimul_project_vjp_kernel<TZ, TC, C><<<dim3(Np / BM, Np, B), vjp_nt<C>(), 0, s>>>(
      (const TC*)dplanes, (const TZ*)x, mask, (const TC*)w4, (const TC*)w4t, gx_in, B, N, Np, outgoing, (TC*)gpg,
      (TC*)xw, (TZ*)dx);
  return pf::check_launch("trimul_project_vjp");
}

// Calls f(TZ{}, TC{}, std::integral_constant<int, C>{}) for the built (xdtype, cdtype, C).
template <class F>
int dispatch_vjp(int xdtype, int cdtype, int C, F&& f) {
  auto by_c = [&](auto tz, auto tc) {
    if (C == 64) return f(tz, tc, std::integral_constant<int, 64>{});
    if (C == 256) return f(tz, tc, std::integral_constant<int, 256>{});
    return f(tz, tc, std::integral_constant<int, 128>{});
  };
  if (xdtype == PF_F32 && cdtype == PF_F32) return by_c(float{}, float{});
  if (xdtype == PF_F32) return by_c(float{}, bf16{});
  return by_c(bf16{}, bf16{});
}

bool vjp_args_ok(int B, int N, int C, int xdtype, int cdtype) {
  return B > 0 && N > 0 && (C == 64 || C == 128 || C == 256) && (xdtype == PF_F32 || xdtype == PF_BF16) &&
         (cdtype == PF_F32 || cdtype == PF_BF16) && !(xdtype == PF_BF16 && cdtype == PF_F32) &&
         (long)pf::pad128(N) * B <= 65535;
}

}  // namespace

extern "C" {

size_t pf_trimul_output_vjp_workspace_bytes(int B, int N, int C, int cdtype) {
  if (B <= 0 || N <= 0 || (cdtype != PF_F32 && cdtype != PF_BF16)) return 0;
  auto pick = [&](auto tc) -> size_t {
    using TC = decltype(tc);
    if (C == 64) return out_vjp_partials<TC, 64>(B, N);
    if (C == 128) return out_vjp_partials<TC, 128>(B, N);
    if (C == 256) return out_vjp_partials<TC, 256>(B, N);
    return 0;
  };
  return cdtype == PF_F32 ? pick(float{}) : pick(bf16{});
}

static int output_vjp_impl(const char* fn, const void* g, const void* X, const void* x, const float* ln_out_w,
                           const float* ln_out_b, float eps_out, const void* w_out, const void* w_out_gate,
                           const void* w_out_t, const void* w_out_gate_t, int B, int N, int C, int xdtype, int cdtype,
                           void* gp, void* gg, void* xln, void* dX, float* gx, float* d_ln_out_w, float* d_ln_out_b,
                           void* workspace, size_t workspace_bytes, void* stream, const MixSpec& mx, float* dr) {
  PF_REQUIRE(g && X && x && ln_out_w && w_out && w_out_gate && w_out_t && w_out_gate_t && gp && gg &&
                 xln && dX && gx && d_ln_out_w && d_ln_out_b && workspace,
             PF_ERR_INVALID_ARG, "%s: null pointer", fn);
  PF_REQUIRE(vjp_args_ok(B, N, C, xdtype, cdtype), PF_ERR_UNSUPPORTED,
             "%s: B=%d N=%d C=%d xdtype=%d cdtype=%d", fn, B, N, C, xdtype, cdtype);
  PF_REQUIRE(pf::aligned16(g) && pf::aligned16(X) && pf::aligned16(x) && pf::aligned16(gp) && pf::aligned16(gg) &&
                 pf::aligned16(xln) && pf::aligned16(dX) && pf::aligned16(gx) && pf::aligned16(workspace),
             PF_ERR_ALIGNMENT, "%s: pointers must be 16-byte aligned", fn);
  const size_t need = pf_trimul_output_vjp_workspace_bytes(B, N, C, cdtype);
  PF_REQUIRE(workspace_bytes >= need, PF_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", fn, workspace_bytes,
             need);
  hipStream_t s = pf::as_stream(stream);
  return dispatch_vjp(xdtype, cdtype, C, [&](auto tz, auto tc, auto cc) {
    using TZ = decltype(tz);
    using TC = decltype(tc);
    constexpr int CC = decltype(cc)::value;
    return output_vjp_launch<TZ, TC, CC>(g, X, x, ln_out_w, ln_out_b, eps_out, w_out, w_out_gate, w_out_t,
                                         w_out_gate_t, B, N, gp, gg, xln, dX, gx, d_ln_out_w, d_ln_out_b, workspace,
                                         s, mx, dr);
  });
}

int pf_trimul_output_vjp(const void* g, const void* X, const void* x, const float* ln_out_w, const float* ln_out_b,
                         float eps_out, const void* w_out, const void* w_out_gate, const void* w_out_t,
                         const void* w_out_gate_t, int B, int N, int C, int xdtype, int cdtype, void* gp, void* gg,
                         void* xln, void* dX, float* gx, float* d_ln_out_w, float* d_ln_out_b, void* workspace,
                         size_t workspace_bytes, void* stream) {
  PF_REQUIRE(ln_out_b, PF_ERR_INVALID_ARG, "pf_trimul_output_vjp: null pointer");
  return output_vjp_impl("pf_trimul_output_vjp", g, X, x, ln_out_w, ln_out_b, eps_out, w_out, w_out_gate, w_out_t,
                         w_out_gate_t, B, N, C, xdtype, cdtype, gp, gg, xln, dX, gx, d_ln_out_w, d_ln_out_b,
                         workspace, workspace_bytes, stream, MixSpec{0, 0, 0, nullptr}, nullptr);
}

int pf_trimul_mhr_output_vjp(const void* g, const void* X, const void* x, const float* ln_out_w,
                             const float* ln_out_b, float eps_out, const void* w_out, const void* w_out_gate,
                             const void* w_out_t, const void* w_out_gate_t, int B, int N, int C, int xdtype,
                             int cdtype, void* gp, void* gg, void* xln, void* dX, float* gx, float* d_ln_out_w,
                             float* d_ln_out_b, void* workspace, size_t workspace_bytes, int num_heads, int head_norm,
                             const float* w_router, int router_kind, float* d_router_logits, void* stream) {
  MixSpec mx;
  if (int e = mix_spec("pf_trimul_mhr_output_vjp", C, num_heads, head_norm, w_router, router_kind, ln_out_b, mx))
    return e;
  PF_REQUIRE(w_router == nullptr || d_router_logits != nullptr, PF_ERR_INVALID_ARG,
             "pf_trimul_mhr_output_vjp: a router needs d_router_logits");
  return output_vjp_impl("pf_trimul_mhr_output_vjp", g, X, x, ln_out_w, ln_out_b, eps_out, w_out, w_out_gate,
                         w_out_t, w_out_gate_t, B, N, C, xdtype, cdtype, gp, gg, xln, dX, gx, d_ln_out_w, d_ln_out_b,
                         workspace, workspace_bytes, stream, mx, d_router_logits);
}

int pf_trimul_project_vjp(const void* dplanes, const void* x, const float* mask, const void* w_packed,
                          const void* w_packed_t, const float* gx_in, int B, int N, int C, int outgoing, int xdtype,
                          int cdtype, void* gpg, void* xw, void* dx, void* stream) {
  PF_REQUIRE(dplanes && x && mask && w_packed && w_packed_t && gx_in && gpg && dx && (outgoing || xw),
             PF_ERR_INVALID_ARG, "pf_trimul_project_vjp: null pointer");
  PF_REQUIRE(vjp_args_ok(B, N, C, xdtype, cdtype), PF_ERR_UNSUPPORTED,
             "pf_trimul_project_vjp: B=%d N=%d C=%d xdtype=%d cdtype=%d", B, N, C, xdtype, cdtype);
  PF_REQUIRE(pf::aligned16(dplanes) && pf::aligned16(x) && pf::aligned16(gpg) && pf::aligned16(dx) &&
                 pf::aligned16(w_packed) && pf::aligned16(w_packed_t),
             PF_ERR_ALIGNMENT, "pf_trimul_project_vjp: pointers must be 16-byte aligned");
  hipStream_t s = pf::as_stream(stream);
  return dispatch_vjp(xdtype, cdtype, C, [&](auto tz, auto tc, auto cc) {
    using TZ = decltype(tz);
    using TC = decltype(tc);
    constexpr int CC = decltype(cc)::value;
    return project_vjp_launch<TZ, TC, CC>(dplanes, x, mask, w_packed, w_packed_t, gx_in, B, N, outgoing, gpg, xw, dx,
                                          s);
  });
}

size_t pf_trimul_mhr_router_wgrad_workspace_bytes(long M, int C, int H) {
  if (M <= 0 || C <= 0 || H <= 0) return 0;
  const long nblk = std::min<long>(1024, (M + 255) / 256);
  return (size_t)nblk * H * C * sizeof(float);
}

int pf_trimul_mhr_router_wgrad(const float* d_router_logits, const void* x, int xdtype, long M, int C, int H,
                               float* d_router, void* workspace, size_t workspace_bytes, void* stream) {
  PF_REQUIRE(d_router_logits && x && d_router && workspace, PF_ERR_INVALID_ARG,
             "pf_trimul_mhr_router_wgrad: null pointer");
  PF_REQUIRE(M > 0 && (C == 64 || C == 128 || C == 256) && H >= 1 && H <= kMhrMaxHeads && C % H == 0,
             PF_ERR_INVALID_ARG, "pf_trimul_mhr_router_wgrad: M=%ld C=%d H=%d", M, C, H);
  PF_REQUIRE(xdtype == PF_F32 || xdtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_trimul_mhr_router_wgrad: xdtype %d",
             xdtype);
  const size_t need = pf_trimul_mhr_router_wgrad_workspace_bytes(M, C, H);
  PF_REQUIRE(workspace_bytes >= need, PF_ERR_WORKSPACE, "pf_trimul_mhr_router_wgrad: workspace %zu < %zu bytes",
             workspace_bytes, need);
  hipStream_t s = pf::as_stream(stream);
  const long nblk = std::min<long>(1024, (M + 255) / 256);
  const long tpb = (M + nblk - 1) / nblk;
  float* partial = static_cast<float*>(workspace);
  auto launch = [&](auto hc) {
    constexpr int HH = decltype(hc)::value;
    if (xdtype == PF_F32)
      mhr_router_wgrad_kernel<float, HH><<<(unsigned)nblk, 256, 0, s>>>(d_router_logits, (const float*)x, M, C, tpb,
                                                                        partial);
    else
      mhr_router_wgrad_kernel<bf16, HH><<<(unsigned)nblk, 256, 0, s>>>(d_router_logits, (const bf16*)x, M, C, tpb,
                                                                       partial);
  };
  // C is a power of two, so the heads dividing it are too
  switch (H) {
    case 1: launch(std::integral_constant<int, 1>{}); break;
    case 2: launch(std::integral_constant<int, 2>{}); break;
    case 4: launch(std::integral_constant<int, 4>{}); break;
    case 8: launch(std::integral_constant<int, 8>{}); break;
    case 16: launch(std::integral_constant<int, 16>{}); break;
    default: launch(std::integral_constant<int, 32>{}); break;
  }
  if (int e = pf::check_launch("mhr_router_wgrad")) return e;
  const int HC = H * C;  // even: the reduce writes columns [0, HC/2) and [HC/2, HC) through two pointers
  trimul_ln_grad_reduce_kernel<<<HC, 256, 0, s>>>(partial, nblk, HC, d_router, d_router + HC / 2);
  return pf::check_launch("mhr_router_wgrad_reduce");
}

int pf_planes_transpose(const void* src, void* dst, int G, int Np, int dtype, void* stream) {
  PF_REQUIRE(src && dst && src != dst, PF_ERR_INVALID_ARG, "pf_planes_transpose: null or aliased pointers");
  PF_REQUIRE(G > 0 && G <= 65535 && Np > 0 && Np % 64 == 0, PF_ERR_INVALID_ARG, "pf_planes_transpose: G=%d Np=%d", G,
             Np);
  PF_REQUIRE(dtype == PF_F32 || dtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_planes_transpose: dtype %d", dtype);
  hipStream_t s = pf::as_stream(stream);
  const dim3 grid((unsigned)(Np / 64), (unsigned)(Np / 64), (unsigned)G);
  if (dtype == PF_F32)
    plane_transpose_kernel<float><<<grid, 256, 0, s>>>((const float*)src, (float*)dst, Np);
  else
    plane_transpose_kernel<bf16><<<grid, 256, 0, s>>>((const bf16*)src, (bf16*)dst, Np);
  return pf::check_launch("pf_planes_transpose");
}

}  // extern "C"
