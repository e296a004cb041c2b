// Multi-head routed (MHR) head mix of the triangle multiply's output kernels
// (src/deepfold3/model/ops.py:476-545): between the contraction X [C] and out_proj, the C
// channels are H heads of d = C / H and
//
//   channel       Y = g_h * LN_C(X)                          (LayerNorm over all C, affine)
//   head_rms      Y = g_h * (X_c rstd_h) w_c                 (RMS over the head's d channels)
//   head_ln       Y = g_h * ((X_c - mu_h) rstd_h w_c + b_c)  (LayerNorm over the head)
//   post_channel  Y = LN_C(g_h * X)                          (gate first, LayerNorm after)
//
// with the router's gates g = H softmax_h(r) or 2 sigmoid(r), r = x Wr^T (x = LN_in(z), the
// router weight Wr [H][C] fp32), or g = 1 without a router. The norms take eps, fp32
// statistics, two passes (mean, then the centred sum of squares).
//
// Thread mapping: one thread per (position p, head h) pair, p = pair % BM, so consecutive
// threads read consecutive positions of a channel row of the channel-major X tile. The
// per-position statistics of the channel modes are reduced over heads through LDS in a fixed
// order. LDS arrays hold [kMhrMaxHeads][BM] floats, index h BM + p (consecutive lanes take
// consecutive positions: no bank conflicts); per-position values sit in row 0.
#pragma once

#include "capi.h"
#include "common.h"

namespace {

constexpr int kMhrMaxHeads = 32;
// Kernels instantiated for at most this many heads hold half the per-head LDS (at 256
// channels the output VJP then keeps two blocks per CU); more heads take the kMhrMaxHeads ones.
constexpr int kMhrHeadsSmall = 16;
enum MixMode { kMixChannel = 0, kMixHeadRms = 1, kMixHeadLn = 2, kMixPostChannel = 3 };

struct MixSpec {
  int heads;        // H, C % H == 0, 1 <= H <= kMhrMaxHeads
  int mode;         // MixMode
  int kind;         // router gates: 0 H softmax_h(r), 1 2 sigmoid(r)
  const float* wr;  // router weight [H][C] fp32, or nullptr (g = 1)
};

// The MHR arguments of the pf_trimul_mhr_* entry points, checked, as a MixSpec.
inline int mix_spec(const char* fn, int C, int num_heads, int head_norm, const float* w_router, int router_kind,
                    const float* ln_out_b, MixSpec& mx) {
  PF_REQUIRE(num_heads >= 1 && num_heads <= kMhrMaxHeads && C % num_heads == 0, PF_ERR_INVALID_ARG,
             "%s: num_heads=%d (1..%d, dividing C=%d)", fn, num_heads, kMhrMaxHeads, C);
  PF_REQUIRE(head_norm >= kMixChannel && head_norm <= kMixPostChannel, PF_ERR_INVALID_ARG,
             "%s: head_norm=%d (0 channel, 1 head_rms, 2 head_ln, 3 post_channel)", fn, head_norm);
  PF_REQUIRE(router_kind == 0 || router_kind == 1, PF_ERR_INVALID_ARG, "%s: router_kind=%d (0 softmax, 1 sigmoid)",
             fn, router_kind);
  PF_REQUIRE(head_norm != kMixPostChannel || w_router != nullptr, PF_ERR_INVALID_ARG,
             "%s: post_channel needs the router", fn);
  PF_REQUIRE(head_norm == kMixHeadRms || ln_out_b != nullptr, PF_ERR_INVALID_ARG,
             "%s: null ln_out_b (only head_rms has no shift)", fn);
  mx = MixSpec{num_heads, head_norm, router_kind, w_router};
  return PF_OK;
}

// B fragments of the router's first 16 rows (zero beyond H) for 16x16 MFMA steps over C,
// loaded into registers at kernel start so their latency hides behind the tile loads.
template <class TC, int C>
struct RouterFrags {
  using M = Mfma<TC>;
  static constexpr int KS = C / M::K16;
  typename M::Frag f[KS];
  PF_DEVICE void load(const MixSpec& mx, int hb) {
    const int l = lane_id();
    const int h = hb * 16 + (l & 15);
    const int kq = (l >> 4) * M::KPL;
    const bool live = mx.wr != nullptr && h < mx.heads;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      float wv[M::KPL];
#pragma unroll
      for (int e = 0; e < M::KPL; ++e) wv[e] = live ? mx.wr[(size_t)h * C + ks * M::K16 + kq + e] : 0.f;
      f[ks] = M::from_floats(wv);
    }
  }
};

// Router gates for the BM positions of the x tile (A [p][ald], TC): gate[p][h]. The logits
// r = A Wr^T run on MFMA (16x16 tiles: wave w takes row blocks w, w + waves, ..; Wr's rows
// are the B fragments, zero beyond H; rf holds those of rows 0..15), then one thread per
// position forms the gates.
template <class TC, int C, int BM, int NT>
PF_DEVICE void mhr_gates(const TC* A, int ald, const MixSpec& mx, float* gate, const RouterFrags<TC, C>& rf) {
  const int H = mx.heads;
  const int tid = threadIdx.x;
  if (mx.wr == nullptr) {
    for (int pr = tid; pr < BM * H; pr += NT) gate[pr] = 1.f;  // pr = h BM + p
    __syncthreads();
    return;
  }
  using M = Mfma<TC>;
  constexpr int RB = BM / 16;
  constexpr int NW = NT / 64;
  const int w = wave_id();
  const int l = lane_id();
  const int r = l & 15;
  const int kq = (l >> 4) * M::KPL;
  const int hb_n = (H + 15) / 16;
  for (int rb = w; rb < RB; rb += NW) {
    for (int hb = 0; hb < hb_n; ++hb) {
      RouterFrags<TC, C> more;
      if (hb > 0) more.load(mx, hb);
      const RouterFrags<TC, C>& use = hb > 0 ? more : rf;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < RouterFrags<TC, C>::KS; ++ks)
        M::mma16(acc, M::load(A + (rb * 16 + r) * ald + ks * M::K16 + kq), use.f[ks]);
      const int h = hb * 16 + r;
      if (h < H) {
#pragma unroll
        for (int e = 0; e < 4; ++e) gate[h * BM + rb * 16 + 4 * (l >> 4) + e] = acc[e];
      }
    }
  }
  __syncthreads();
  for (int p = tid; p < BM; p += NT) {
    float* gp = gate + p;  // head h at gp[h * BM]
    if (mx.kind == 0) {
      float m = gp[0];
      for (int h = 1; h < H; ++h) m = fmaxf(m, gp[h * BM]);
      float s = 0.f;
      for (int h = 0; h < H; ++h) {
        const float e = __expf(gp[h * BM] - m);
        gp[h * BM] = e;
        s += e;
      }
      const float k = (float)H / s;
      for (int h = 0; h < H; ++h) gp[h * BM] *= k;
    } else {
      for (int h = 0; h < H; ++h) gp[h * BM] = 2.f / (1.f + __expf(-gp[h * BM]));
    }
  }
  __syncthreads();
}

// Per-position statistics of v over all C channels for the channel modes: mean -> sa[p][0],
// rstd -> sb[p][0]. v_c = X_c (channel) or g_h X_c (post_channel).
template <class TC, int C, int BM, int NT>
PF_DEVICE void mhr_position_stats(const TC* Xs, int xld, const float* gate, bool gated, int H, float eps,
                                  float* sa, float* sb, float* part) {
  const int tid = threadIdx.x;
  const int d = C / H;
  for (int pr = tid; pr < BM * H; pr += NT) {
    const int p = pr % BM, h = pr / BM;
    const float g = gated ? gate[h * BM + p] : 1.f;
    const TC* x = Xs + h * d * xld + p;
    float s = 0.f;
#pragma unroll 8
    for (int c = 0; c < d; ++c) s += to_f32(x[c * xld]);
    part[h * BM + p] = g * s;
  }
  __syncthreads();
  for (int p = tid; p < BM; p += NT) {
    float s = 0.f;
    for (int h = 0; h < H; ++h) s += part[h * BM + p];
    sa[p] = s * (1.0f / C);
  }
  __syncthreads();
  for (int pr = tid; pr < BM * H; pr += NT) {
    const int p = pr % BM, h = pr / BM;
    const float g = gated ? gate[h * BM + p] : 1.f;
    const float mean = sa[p];
    const TC* x = Xs + h * d * xld + p;
    float v = 0.f;
#pragma unroll 8
    for (int c = 0; c < d; ++c) {
      const float t = g * to_f32(x[c * xld]) - mean;
      v += t * t;
    }
    part[h * BM + p] = v;
  }
  __syncthreads();
  for (int p = tid; p < BM; p += NT) {
    float v = 0.f;
    for (int h = 0; h < H; ++h) v += part[h * BM + p];
    sb[p] = rsqrtf(v * (1.0f / C) + eps);
  }
  __syncthreads();
}

// Statistics of every mode: (mean, rstd) per (p, h) in sa, sb for the head modes (mean 0 for
// head_rms), per position in sa[p][0], sb[p][0] for the channel modes.
template <class TC, int C, int BM, int NT>
PF_DEVICE void mhr_stats(const TC* Xs, int xld, const float* gate, const MixSpec& mx, float eps, float* sa,
                         float* sb, float* part) {
  const int H = mx.heads;
  if (mx.mode == kMixChannel || mx.mode == kMixPostChannel) {
    mhr_position_stats<TC, C, BM, NT>(Xs, xld, gate, mx.mode == kMixPostChannel, H, eps, sa, sb, part);
    return;
  }
  const int d = C / H;
  const float inv_d = 1.0f / (float)d;
  for (int pr = threadIdx.x; pr < BM * H; pr += NT) {
    const int p = pr % BM, h = pr / BM;
    const TC* x = Xs + h * d * xld + p;
    float mu = 0.f;
    if (mx.mode == kMixHeadLn) {
#pragma unroll 8
      for (int c = 0; c < d; ++c) mu += to_f32(x[c * xld]);
      mu *= inv_d;
    }
    float v = 0.f;
#pragma unroll 8
    for (int c = 0; c < d; ++c) {
      const float t = to_f32(x[c * xld]) - mu;
      v += t * t;
    }
    sa[h * BM + p] = mu;
    sb[h * BM + p] = rsqrtf(v * inv_d + eps);
  }
  __syncthreads();
}

// The normalised value of a channel of head h at position p is n = (gs x - mu) rs.
struct NormCoef {
  float gs, mu, rs;
};
template <int BM>
PF_DEVICE NormCoef mhr_coef(const float* gate, const float* sa, const float* sb, const MixSpec& mx, int p, int h) {
  if (mx.mode == kMixChannel) return {1.f, sa[p], sb[p]};
  if (mx.mode == kMixPostChannel) return {gate[h * BM + p], sa[p], sb[p]};
  return {1.f, sa[h * BM + p], sb[h * BM + p]};
}
PF_DEVICE float mhr_norm(const NormCoef& q, float x) { return (q.gs * x - q.mu) * q.rs; }

// Y [p][c] (TC, row-major, ld ald) from the channel-major X tile after mhr_gates and mhr_stats.
template <class TC, int C, int BM, int NT>
PF_DEVICE void mhr_mix_write(const TC* Xs, int xld, const float* gate, const float* sa, const float* sb,
                             const MixSpec& mx, const float* lnw, const float* lnb, TC* Y, int ald) {
  const int H = mx.heads, d = C / H;
  const bool has_bias = mx.mode != kMixHeadRms;
  for (int pr = threadIdx.x; pr < BM * H; pr += NT) {
    const int p = pr % BM, h = pr / BM;
    const float g = mx.mode == kMixPostChannel ? 1.f : gate[h * BM + p];
    const NormCoef q = mhr_coef<BM>(gate, sa, sb, mx, p, h);
    const TC* x = Xs + h * d * xld + p;
    TC* y = Y + p * ald + h * d;
#pragma unroll 8
    for (int c = 0; c < d; ++c) {
      const float t = mhr_norm(q, to_f32(x[c * xld])) * lnw[h * d + c] + (has_bias ? lnb[h * d + c] : 0.f);
      y[c] = from_f32<TC>(g * t);
    }
  }
}

// The affine gradients' per-block partial sums, one thread per channel: sw[c] = sum_p dT[p][c]
// n[p][c], sb[c] = sum_p dT[p][c] (dT [p][sld] the affine output's cotangent, X in Xs).
template <class TC, int C, int BM, int NT>
PF_DEVICE void mhr_affine_partials(const TC* Xs, int xld, const float* gate, const float* sa, const float* sb,
                                   const MixSpec& mx, const float* dT, int sld, float* out_w, float* out_b) {
  const int d = C / mx.heads;
  for (int c = threadIdx.x; c < C; c += NT) {
    const int h = c / d;
    float sw = 0.f, s0 = 0.f;
#pragma unroll 8
    for (int p = 0; p < BM; ++p) {
      const float n = mhr_norm(mhr_coef<BM>(gate, sa, sb, mx, p, h), to_f32(Xs[c * xld + p]));
      const float dv = dT[p * sld + c];
      sw += dv * n;
      s0 += dv;
    }
    out_w[c] = sw;
    out_b[c] = s0;
  }
}

// Pullback of the mix. On entry dY [p][sld] (fp32) holds d(Y); on exit it holds the cotangent
// of the affine output (d(Y) g_h for the modes that gate after the norm, d(Y) for
// post_channel), the cotangent of X replaces X in Xs, and dg [p][h] holds d(gate). The
// affine gradients (sum_p dY[p][c] n[p][c] and sum_p dY[p][c]) need X: `between` runs after
// the first barrier below, before Xs is rewritten.
template <class TC, int C, int BM, int NT, class Between>
PF_DEVICE void mhr_mix_pullback(TC* Xs, int xld, const float* gate, const float* sa, const float* sb,
                                const MixSpec& mx, const float* lnw, const float* lnb, float* dY, int sld,
                                float* dg, float* pa, float* pb, Between&& between) {
  const int H = mx.heads, d = C / H;
  const int tid = threadIdx.x;
  const bool post = mx.mode == kMixPostChannel;
  const bool has_bias = mx.mode != kMixHeadRms;
  // 1) gates after the norm: dT = dY g, dg = sum_head dY t (t the affine output)
  if (!post) {
    for (int pr = tid; pr < BM * H; pr += NT) {
      const int p = pr % BM, h = pr / BM;
      const float g = gate[h * BM + p];
      const NormCoef q = mhr_coef<BM>(gate, sa, sb, mx, p, h);
      const TC* x = Xs + h * d * xld + p;
      float* dy = dY + p * sld + h * d;
      float s = 0.f;
#pragma unroll 8
      for (int c = 0; c < d; ++c) {
        const float t = mhr_norm(q, to_f32(x[c * xld])) * lnw[h * d + c] + (has_bias ? lnb[h * d + c] : 0.f);
        const float v = dy[c];
        s += v * t;
        dy[c] = v * g;
      }
      dg[h * BM + p] = s;
    }
  }
  __syncthreads();
  between();
  __syncthreads();
  // 2) the norm's pullback, u = dT w: rstd (u - mean(u) - n mean(u n)) over the norm's group
  //    (the head, or all C), the mean(u) term absent for head_rms
  if (mx.mode == kMixHeadRms || mx.mode == kMixHeadLn) {
    const float inv_d = 1.0f / (float)d;
    for (int pr = tid; pr < BM * H; pr += NT) {
      const int p = pr % BM, h = pr / BM;
      const NormCoef q = mhr_coef<BM>(gate, sa, sb, mx, p, h);
      TC* x = Xs + h * d * xld + p;
      const float* dy = dY + p * sld + h * d;
      float su = 0.f, sun = 0.f;
#pragma unroll 8
      for (int c = 0; c < d; ++c) {
        const float u = dy[c] * lnw[h * d + c];
        su += u;
        sun += u * mhr_norm(q, to_f32(x[c * xld]));
      }
      su = mx.mode == kMixHeadLn ? su * inv_d : 0.f;
      sun *= inv_d;
#pragma unroll 8
      for (int c = 0; c < d; ++c) {
        const float u = dy[c] * lnw[h * d + c];
        x[c * xld] = from_f32<TC>(q.rs * (u - su - mhr_norm(q, to_f32(x[c * xld])) * sun));
      }
    }
    __syncthreads();
    return;
  }
  for (int pr = tid; pr < BM * H; pr += NT) {
    const int p = pr % BM, h = pr / BM;
    const NormCoef q = mhr_coef<BM>(gate, sa, sb, mx, p, h);
    const TC* x = Xs + h * d * xld + p;
    const float* dy = dY + p * sld + h * d;
    float su = 0.f, sun = 0.f;
#pragma unroll 8
    for (int c = 0; c < d; ++c) {
      const float u = dy[c] * lnw[h * d + c];
      su += u;
      sun += u * mhr_norm(q, to_f32(x[c * xld]));
    }
    pa[h * BM + p] = su;
    pb[h * BM + p] = sun;
  }
  __syncthreads();
  for (int p = tid; p < BM; p += NT) {
    float su = 0.f, sun = 0.f;
    for (int h = 0; h < H; ++h) {
      su += pa[h * BM + p];
      sun += pb[h * BM + p];
    }
    pa[p] = su * (1.0f / C);
    pb[p] = sun * (1.0f / C);
  }
  __syncthreads();
  for (int pr = tid; pr < BM * H; pr += NT) {
    const int p = pr % BM, h = pr / BM;
    const NormCoef q = mhr_coef<BM>(gate, sa, sb, mx, p, h);
    const float su = pa[p], sun = pb[p];
    TC* x = Xs + h * d * xld + p;
    const float* dy = dY + p * sld + h * d;
    float s = 0.f;
#pragma unroll 8
    for (int c = 0; c < d; ++c) {
      const float xv = to_f32(x[c * xld]);
      const float du = q.rs * (dy[c] * lnw[h * d + c] - su - mhr_norm(q, xv) * sun);  // d(v), v = gs X
      s += du * xv;
      x[c * xld] = from_f32<TC>(du * q.gs);
    }
    if (post) dg[h * BM + p] = s;
  }
  __syncthreads();
}

// d(router logits) from d(gate) at position p: softmax g = H softmax(r): dr_j = g_j (dg_j -
// sum_h g_h dg_h / H); sigmoid g = 2 sigmoid(r): dr = dg g (1 - g / 2).
template <int BM>
PF_DEVICE float mhr_router_grad(const float* gate, const float* dg, const MixSpec& mx, int p, int j) {
  const float* g = gate + p;  // head h at [h * BM]
  const float* dgp = dg + p;
  const float gj = g[j * BM];
  if (mx.kind == 0) {
    float s = 0.f;
    for (int h = 0; h < mx.heads; ++h) s += g[h * BM] * dgp[h * BM];
    return gj * (dgp[j * BM] - s / (float)mx.heads);
  }
  return dgp[j * BM] * gj * (1.f - 0.5f * gj);
}

}  // namespace
