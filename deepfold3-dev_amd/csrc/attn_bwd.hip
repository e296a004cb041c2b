// Backward of the pair-biased flash attention (_EvoformerAttention.backward,
// src/deepfold3/model/triton/evo_attention.py:1295-1472; kernels :335-1195), with the
// softmax Jacobian in centred form (docs/optimizations.md:417-483).
//
// Per line (b, s, h) with logits t_ij = scale q_i.k_j + bias[b,h,i,j] + mask[b,s,j]:
//   P_ij = exp(t_ij - LSE_i),  dP_ij = dO_i . v_j
//   dS_ij = P_ij (u_ij - C_i),  u_ij = dP_ij - dP_i,imax (0 at j = imax_i, by index),
//   C_i = sum_j P_ij u_ij,
// which equals P (dP - rowsum(P dP)) but never subtracts two O(1) numbers at the softmax
// argmax. Outputs: dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO, d_bias = sum_s dS.
// Masked rows: under the reference kernel's rule a line whose keys are all masked (max logit
// < -1e8) gets LSE = +inf, so P = 0 and every gradient of its rows is 0 (its forward writes 0).
// Under the stock eager rule (the dense entry point with zero_masked_rows = 0) such a row is
// an ordinary row: its -1e9-shifted logits round to one value, P is uniform, and the
// gradients are the softmax Jacobian's at that point, as autograd of the eager path gives;
// only a row with no finite logit is dead there. Such a row's logits sit near -1.44e9 (log2
// units), where fp32 values are 128 apart, so its log-sum-exp cannot be stored there: under
// the eager rule every logit is formed at full magnitude (so it rounds exactly as the eager
// path's does) and then shifted by its line's offset, the line's largest key mask when that
// is below the dead threshold (0 otherwise), which keeps every statistic small.
//
// Kernels, all on 32x32 MFMA tiles with D = 32:
//   attn_bwd_relayout: K, Q, dO, V copied once into MFMA fragment order, as themselves and
//                  (K, Q, dO) transposed for the products that contract over rows (dQ over
//                  keys, dK and dV over queries): every fragment load of a wave is then one
//                  contiguous 1 KB piece.
//   attn_bwd_dq:   query-major. Pass 1 over the keys finds each row's maximum logit and first
//                  argmax; pass 2 forms P, dP and the centred sums and the two products whose
//                  difference is dQ, and leaves (LSE, dP_imax, imax, C) per row in the
//                  workspace for the other kernels. Given the forward's row LSE, pass 1 is
//                  skipped: p = 2^(x - LSE) <= ~1 needs no maximum, and the centring key is
//                  the row's dominant one (p > 1/2, the first in key order; none if no key
//                  dominates, then the sums stay centred on 0), found in pass 2 itself; the
//                  sums taken before it are moved onto it once (A += (ref - dP_k) B,
//                  C W += (ref - dP_k) W).
//   attn_bwd_dkdv: key-major, loops over query tiles: dV^T += dO^T P, dK^T += Q^T dS.
//   attn_bwd_db:   one (query tile, key tile) of one (b, h), loops over a group of lines and
//                  sums dS in registers; the groups' partial sums are added in a fixed order,
//                  so the bias gradient needs no atomics and every output is bit-reproducible.
// dQ and dK/dV blocks take four lines of one (b, h) that share a double-buffered pair-bias
// tile in LDS (one barrier per step). Logits are kept in log2 units (x = t log2 e) so P is
// one v_exp_f32.
#include <algorithm>
#include <climits>

#include "capi.h"
#include "common.h"

namespace {

constexpr int kBD = 32;            // head dimension
constexpr int kNT = 256;           // four waves
constexpr int kLines = 4;          // lines of one (b, h) per block: they share the bias tile
constexpr int kSubDq = 1;          // 32-query sub-tiles per wave in the dQ kernel
constexpr int kSubKv = 1;          // 32-key sub-tiles per wave in the dK / dV kernel
// Dead-row threshold in log2 units: the zero masked-row rule (the reference tests t < -1e8),
// and the eager rule (only rows without a finite logit).
constexpr float kDeadLog2 = -1.0e8f * kLog2e;
constexpr float kDeadEager = -3.402823466e38f;

// Element strides of one [B][S][H][N][D] operand view (D contiguous): batch item, line, head
// and key (row); a dense operand has {S H N D, H N D, N D, D}.
struct Strides4 {
  long b, s, h, n;
};
PF_DEVICE long line_offset(const Strides4& st, long b, long s, long h) { return b * st.b + s * st.s + h * st.h; }

// Tile row that element e of step t of lane half h's A fragment reads, for a product that
// contracts over the 32 rows of a tile with the other operand from bfrag_from_acc (the
// accumulator's row order): bf16 step t of 2 reads rows 16t + 8(e>>2) + 4h + (e&3), fp32
// step t of 4 reads rows 8t + 4h + e.
template <class TC>
PF_DEVICE int frag_row(int t, int h, int e);
template <>
PF_DEVICE int frag_row<bf16>(int t, int h, int e) {
  return 16 * t + 8 * (e >> 2) + 4 * h + (e & 3);
}
template <>
PF_DEVICE int frag_row<float>(int t, int h, int e) {
  return 8 * t + 4 * h + e;
}

// A 32x32 accumulator (lane: column l&31, rows 8(r>>2) + 4h + (r&3)) as the B operand of a
// product that contracts over its rows: step t of 32 / K32.
template <class TC>
PF_DEVICE typename Mfma<TC>::Frag bfrag_from_acc(const f32x16& acc, int t);
template <>
PF_DEVICE bf16x8 bfrag_from_acc<bf16>(const f32x16& acc, int t) {
  bf16x8 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = (bf16)acc[8 * t + e];
  return f;
}
template <>
PF_DEVICE f32x4 bfrag_from_acc<float>(const f32x16& acc, int t) {
  return f32x4{acc[4 * t], acc[4 * t + 1], acc[4 * t + 2], acc[4 * t + 3]};
}

// Accumulator row r of lane half h.
PF_DEVICE int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// One 32-row tile of an operand in MFMA fragment order, [tile][step][lane][16 bytes], so that
// every fragment load of a wave is one contiguous 1 KB piece (a row-major tile spreads each
// step over all 16 of its cache lines). Two orders, written from the same LDS stage:
//   XR: the fragments of X itself, lane (h, c) of step t holding row c, elements
//       t K32 + h KPL ..: the operands of Q K^T, dO V^T (K, Q, dO, V);
//   XT: the A fragments of X^T, lane (h, c) holding element d = c of the rows frag_row(t, h, .):
//       the operands of the products that contract over rows, dQ over keys and dK, dV over
//       queries (K, Q, dO).
// Rows past N are zero. blockIdx.z: 0 K, 1 Q, 2 dO, 3 V (no XT).
template <class TC>
PF_DEVICE size_t frag_offset(size_t line, int Np, int tile, int step, int lane) {
  constexpr int STEPS = kBD / Mfma<TC>::K32;
  return (((line * (size_t)(Np / 32) + tile) * STEPS + step) * 64 + lane) * Mfma<TC>::KPL;
}

template <class TC>
__global__ __launch_bounds__(256) void attn_bwd_relayout_kernel(const TC* __restrict__ K, const TC* __restrict__ Q,
                                                                const TC* __restrict__ dO, const TC* __restrict__ V,
                                                                TC* __restrict__ KR, TC* __restrict__ QR,
                                                                TC* __restrict__ OR, TC* __restrict__ VR,
                                                                TC* __restrict__ KT, TC* __restrict__ QT,
                                                                TC* __restrict__ OT, int S, int H, int N, int Np,
                                                                Strides4 sx, Strides4 sdo) {
  using M = Mfma<TC>;
  constexpr int VEC = M::KPL;  // elements per 16-byte piece
  constexpr int STEPS = kBD / M::K32;
  constexpr int R = 64;          // rows per block: two tiles
  constexpr int LD = kBD + VEC;  // [row][d] with a 16-byte pad
  __shared__ __attribute__((aligned(16))) TC t[R * LD];
  const int z = blockIdx.z;
  const TC* X = z == 0 ? K : (z == 1 ? Q : (z == 2 ? dO : V));
  TC* XR = z == 0 ? KR : (z == 1 ? QR : (z == 2 ? OR : VR));
  TC* XT = z == 0 ? KT : (z == 1 ? QT : OT);
  const size_t line = blockIdx.y;
  const int n0 = blockIdx.x * R;
  const Strides4& st = z == 2 ? sdo : sx;
  const long lb = (long)(line / ((size_t)S * H)), ls = (long)((line / H) % S), lh = (long)(line % H);
  const TC* Xl = X + line_offset(st, lb, ls, lh);
  for (int i = threadIdx.x; i < R * (kBD / VEC); i += 256) {
    const int r = i / (kBD / VEC);
    const int d0 = (i % (kBD / VEC)) * VEC;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (n0 + r < N) v = *reinterpret_cast<const u32x4*>(Xl + (long)(n0 + r) * st.n + d0);
    *reinterpret_cast<u32x4*>(t + r * LD + d0) = v;
  }
  __syncthreads();
  // piece i = (tile jj, step st, lane): consecutive threads write consecutive 16 bytes
  const size_t base = frag_offset<TC>(line, Np, n0 / 32, 0, 0);
  for (int i = threadIdx.x; i < 2 * STEPS * 64; i += 256) {
    const int jj = i / (STEPS * 64);
    const int st = (i / 64) % STEPS;
    const int h = (i >> 5) & 1;
    const int c = i & 31;
    *reinterpret_cast<u32x4*>(XR + base + (size_t)i * VEC) =
        *reinterpret_cast<const u32x4*>(t + (32 * jj + c) * LD + st * M::K32 + h * VEC);
    if (z < 3) {
      TC e[VEC];
#pragma unroll
      for (int u = 0; u < VEC; ++u) e[u] = t[(32 * jj + frag_row<TC>(st, h, u)) * LD + c];
      u32x4 v;
      __builtin_memcpy(&v, e, 16);
      *reinterpret_cast<u32x4*>(XT + base + (size_t)i * VEC) = v;
    }
  }
}

// bias2 [B*H][Np][Np] = pair_bias * log2 e (0 at padding), mask2 [B*S][Np] = res_mask * log2 e
// (-inf past N): every later load is an aligned 16-byte load with no bounds test.
__global__ __launch_bounds__(256) void attn_bwd_prep_kernel(const float* __restrict__ bias,
                                                            const float* __restrict__ res_mask,
                                                            float* __restrict__ bias2, float* __restrict__ mask2,
                                                            int BH, int BS, int N, int Np) {
  const size_t pp = (size_t)Np * Np;
  const size_t nb = (size_t)BH * pp;
  const size_t nm = (size_t)BS * Np;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < nb + nm; i += (size_t)gridDim.x * 256) {
    if (i < nb) {
      const size_t bh = i / pp;
      const int r = (int)((i / Np) % Np);
      const int k = (int)(i % Np);
      bias2[i] = (r < N && k < N) ? bias[(bh * N + r) * N + k] * kLog2e : 0.f;
    } else {
      const size_t j = i - nb;
      const size_t bs = j / Np;
      const int k = (int)(j % Np);
      mask2[j] = k < N ? res_mask[bs * N + k] * kLog2e : -INFINITY;
    }
  }
}

// Per-line logit offset of the eager masked-row rule: the line's largest key mask (log2
// units) when it is below the dead threshold, else 0. One 64-lane block per line.
__global__ __launch_bounds__(64) void attn_bwd_lineoff_kernel(const float* __restrict__ mask2, float* __restrict__ off,
                                                             int N, int Np, float dead_below) {
  const float* m = mask2 + (size_t)blockIdx.x * Np;
  float mx = -INFINITY;
  for (int k = threadIdx.x; k < N; k += 64) mx = fmaxf(mx, m[k]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (threadIdx.x == 0) off[blockIdx.x] = (mx < dead_below && mx > -INFINITY) ? mx : 0.f;
}

// Logit in log2 units from the raw product s (times scale log2 e), the bias and the mask
// (both already times log2 e); every kernel forms it the same way.
PF_DEVICE float logit2(float s, float sl2, float b2, float m2) { return fmaf(s, sl2, b2 + m2); }

// Row statistics, one 16-byte record per (line, query): {LSE (log2), dP at the argmax, C, argmax}.
PF_DEVICE f32x4 stats_pack(float lse2, float ref, float cen, int imax) {
  return f32x4{lse2, ref, cen, __int_as_float(imax)};
}

// ------------------------------------------------------------------ dQ (+ row statistics)
// Block: four lines of one (b, h) sharing a double-buffered pair-bias tile in LDS, which
// also holds the four lines' key masks; each wave owns one line and kRows queries (kSub
// sub-tiles of 32, the columns of S^T = K Q^T). The next key tile's fragments, bias and
// masks are fetched while the current one computes.
//
// Pass 1 forms the logits only and keeps each row's maximum m and first argmax. The
// reference value dP_imax = dO_i . v_imax is then one gathered dot product, and pass 2 needs
// no rescaling: with p_j = exp2(x_j - m) and W = sum_j p_j it accumulates W, C W = sum_j p_j
// u_j and the two products A = sum_j p_j u_j k_j and B = sum_j p_j k_j, so that
// dQ = scale (A - C B) / W. Each term of A and of C B is O(1 - P_imax): nothing of order one
// is cancelled, as in the per-element form P (u - C).
template <class TC>
struct DqOps {
  typename Mfma<TC>::Frag k[kBD / Mfma<TC>::K32], v[kBD / Mfma<TC>::K32], kt[kBD / Mfma<TC>::K32];
};

// Dot product of two fragments (the same k slice of two rows), in fp32.
PF_DEVICE float frag_dot(const bf16x8& a, const bf16x8& b) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s = fmaf((float)a[e], (float)b[e], s);
  return s;
}
PF_DEVICE float frag_dot(const f32x4& a, const f32x4& b) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) s = fmaf(a[e], b[e], s);
  return s;
}

template <class TC, int kSub, bool kLse, bool kOff>
__global__ __launch_bounds__(kNT, sizeof(TC) == 2 ? 3 : 2) void attn_bwd_dq_kernel(const TC* __restrict__ QR, const TC* __restrict__ KR,
                                                             const TC* __restrict__ VR, const TC* __restrict__ OR,
                                                             const TC* __restrict__ V, const TC* __restrict__ KT,
                                                             const float* __restrict__ mask2,
                                                             const float* __restrict__ bias2, int S, int H, int N,
                                                             int Np, float scale, TC* __restrict__ dQ,
                                                             f32x4* __restrict__ st4, Strides4 sx, Strides4 sg,
                                                             const float* __restrict__ lse_in, float dead_below,
                                                             const float* __restrict__ lineoff) {
  using M = Mfma<TC>;
  constexpr int STEPS = kBD / M::K32;
  constexpr int kRows = 32 * kSub;
  constexpr int BLD = 36;  // bias stage [query][32 keys + 4]
  __shared__ __attribute__((aligned(16))) float bstage[2][kRows * BLD];
  __shared__ __attribute__((aligned(16))) float mstage[2][kLines * 32];  // [line][key]

  const int bh = blockIdx.z;
  const int b = bh / H;
  const int hd = bh % H;
  const int w = wave_id();
  const int l = lane_id();
  const int hh = l >> 5;
  const int c = l & 31;
  const int s = blockIdx.y * kLines + w;
  const bool active = s < S;  // inactive waves mirror the group's first line and skip the math
  const long sl = active ? s : (int)blockIdx.y * kLines;  // this wave's line (or the mirrored one)
  const long bs = (long)b * S + sl;
  const size_t line = (size_t)bs * H + hd;
  const TC* Vl = V + line_offset(sx, b, sl, hd);
  const float off = kOff ? lineoff[bs] : 0.f;  // eager rule: this line's logit offset
  // line whose key mask thread t < 128 stages (the four lines of the group, clamped)
  const float* m2s = mask2 + ((long)b * S + min((int)blockIdx.y * kLines + (int)(threadIdx.x >> 5), S - 1)) * Np;
  const float* b2l = bias2 + (size_t)bh * Np * Np;
  const int q0 = blockIdx.x * kRows;
  const float sl2 = scale * kLog2e;
  const int nkt = (N + 31) / 32;

  typename M::Frag qf[kSub][STEPS], of[kSub][STEPS];
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) {
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      qf[sub][t] = M::load(QR + frag_offset<TC>(line, Np, q0 / 32 + sub, t, l));
      of[sub][t] = M::load(OR + frag_offset<TC>(line, Np, q0 / 32 + sub, t, l));
    }
  }

  f32x4 pf[2];
  float pm = 0.f;
  constexpr int BU = kRows * 8 / kNT;  // 16-byte bias loads per thread per step
  auto bias_load = [&](int k0) {
#pragma unroll
    for (int u = 0; u < BU; ++u) {
      const int i = threadIdx.x + u * kNT;
      pf[u] = *reinterpret_cast<const f32x4*>(b2l + (size_t)(q0 + (i >> 3)) * Np + k0 + (i & 7) * 4);
    }
    if (threadIdx.x < kLines * 32) pm = m2s[k0 + (threadIdx.x & 31)];
  };
  auto bias_store = [&](int st) {
#pragma unroll
    for (int u = 0; u < BU; ++u) {
      const int i = threadIdx.x + u * kNT;
      *reinterpret_cast<f32x4*>(&bstage[st][(i >> 3) * BLD + (i & 7) * 4]) = pf[u];
    }
    if (threadIdx.x < kLines * 32) mstage[st][threadIdx.x] = pm;
  };
  // K (pass 1); V and K^T as well (pass 2)
  auto fetch = [&](int k0, DqOps<TC>& o, bool full) {
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      o.k[t] = M::load(KR + frag_offset<TC>(line, Np, k0 / 32, t, l));
      if (full) {
        o.v[t] = M::load(VR + frag_offset<TC>(line, Np, k0 / 32, t, l));
        o.kt[t] = M::load(KT + frag_offset<TC>(line, Np, k0 / 32, t, l));
      }
    }
  };
  // log2 logits from the raw scores for keys k0..k0+31 (rows) and sub-tile `sub` (columns)
  auto logits = [&](const f32x16& sa, int st, int sub, f32x16& x) {
    const float* brow = &bstage[st][(32 * sub + c) * BLD];
    const float* mrow2 = &mstage[st][w * 32];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 b4 = *reinterpret_cast<const f32x4*>(brow + 8 * j + 4 * hh);
      const f32x4 m4 = *reinterpret_cast<const f32x4*>(mrow2 + 8 * j + 4 * hh);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[4 * j + e] = logit2(sa[4 * j + e], sl2, b4[e], m4[e]);
        if constexpr (kOff) x[4 * j + e] -= off;
      }
    }
  };

  float mrow[kSub], ref[kSub];
  int imax[kSub];
  bool dead[kSub], found[kSub];
  if constexpr (kLse) {
    // The forward's LSE (log2 units, +inf for a dead row) as the exponent offset: p <= ~1.
#pragma unroll
    for (int sub = 0; sub < kSub; ++sub) {
      const int q = q0 + 32 * sub + c;
      const float lf = q < N ? lse_in[line * Np + q] : INFINITY;
      dead[sub] = !(lf >= dead_below && lf < INFINITY);
      mrow[sub] = dead[sub] ? INFINITY : lf;
      ref[sub] = 0.f;
      imax[sub] = -1;
      found[sub] = false;
    }
  } else {
    // Pass 1: maximum and first argmax over this lane's half of the keys (its accumulator
    // rows ascend in key order, tiles ascend, so a strict > keeps the first).
    float run_max[kSub];
    int imx[kSub];
  #pragma unroll
    for (int sub = 0; sub < kSub; ++sub) {
      run_max[sub] = -INFINITY;
      imx[sub] = 0;
    }
    {
      DqOps<TC> cur, nxt;
      fetch(0, cur, false);
      bias_load(0);
      bias_store(0);
      __syncthreads();
      for (int kt = 0; kt < nkt; ++kt) {
        const int k0 = kt * 32;
        const bool more = kt + 1 < nkt;
        if (more) {
          bias_load(k0 + 32);
          fetch(k0 + 32, nxt, false);
        }
        if (active) {
          f32x16 sa[kSub];
  #pragma unroll
          for (int sub = 0; sub < kSub; ++sub) {
            sa[sub] = f32x16{};
  #pragma unroll
            for (int t = 0; t < STEPS; ++t) M::mma32(sa[sub], cur.k[t], qf[sub][t]);
          }
  #pragma unroll
          for (int sub = 0; sub < kSub; ++sub) {
            f32x16 x;
            logits(sa[sub], kt & 1, sub, x);
            // tile maximum, then its first row (rows ascend in key order: scan downwards)
            float tmax = x[0];
  #pragma unroll
            for (int r = 1; r < 16; ++r) tmax = fmaxf(tmax, x[r]);
            int trow = 0;
  #pragma unroll
            for (int r = 15; r >= 0; --r) trow = x[r] == tmax ? acc_row(r, hh) : trow;
            if (tmax > run_max[sub]) {
              run_max[sub] = tmax;
              imx[sub] = k0 + trow;
            }
          }
        }
        if (more) bias_store((kt + 1) & 1);
        __syncthreads();
        cur = nxt;
      }
    }
    // Merge the two halves (larger maximum; the smaller index on a tie), then dP at the argmax.
#pragma unroll
    for (int sub = 0; sub < kSub; ++sub) {
      const float om = __shfl_xor(run_max[sub], 32, 64);
      const int oi = __shfl_xor(imx[sub], 32, 64);
      if (om > run_max[sub] || (om == run_max[sub] && oi < imx[sub])) {
        run_max[sub] = om;
        imx[sub] = oi;
      }
      const bool live = run_max[sub] >= dead_below;
      dead[sub] = !live || q0 + 32 * sub + c >= N;
      mrow[sub] = live ? run_max[sub] : 0.f;
      imax[sub] = dead[sub] ? -1 : imx[sub];
      const int iv = live ? imx[sub] : 0;  // < N: keys past N have logit -inf
      float part = 0.f;
  #pragma unroll
      for (int t = 0; t < STEPS; ++t)
        part += frag_dot(of[sub][t], M::load(Vl + (long)iv * sx.n + t * M::K32 + hh * M::KPL));
      part += __shfl_xor(part, 32, 64);
      ref[sub] = dead[sub] ? 0.f : part;
    }

  }

  // Pass 2: A^T [d x q] += K^T [d x keys] (p u)^T, B^T += K^T p^T, with W and C W per lane.
  f32x16 da[kSub], db[kSub];
  float Wp[kSub], Cp[kSub];
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) {
    da[sub] = db[sub] = f32x16{};
    Wp[sub] = Cp[sub] = 0.f;
  }
  {
    DqOps<TC> cur, nxt;
    fetch(0, cur, true);
    bias_load(0);
    bias_store(0);
    __syncthreads();
    for (int kt = 0; kt < nkt; ++kt) {
      const int k0 = kt * 32;
      const bool more = kt + 1 < nkt;
      if (more) {
        bias_load(k0 + 32);
        fetch(k0 + 32, nxt, true);
      }
      if (active) {
        f32x16 sa[kSub], dp[kSub];
#pragma unroll
        for (int sub = 0; sub < kSub; ++sub) {
          sa[sub] = dp[sub] = f32x16{};
#pragma unroll
          for (int t = 0; t < STEPS; ++t) {
            M::mma32(sa[sub], cur.k[t], qf[sub][t]);
            M::mma32(dp[sub], cur.v[t], of[sub][t]);
          }
        }
#pragma unroll
        for (int sub = 0; sub < kSub; ++sub) {
          f32x16 x;
          logits(sa[sub], kt & 1, sub, x);
          f32x16 p, pu;
#pragma unroll
          for (int r = 0; r < 16; ++r) p[r] = __builtin_amdgcn_exp2f(x[r] - mrow[sub]);
          if constexpr (kLse) {
            // The dominant key (p > 1/2: at most one per row up to rounding; the first in key
            // order) becomes the reference when it appears: the sums so far, taken about 0,
            // are re-centred once. A row without one keeps 0 (no term dominates D).
            float tmax = p[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) tmax = fmaxf(tmax, p[r]);
            if (__any(!found[sub] && tmax > 0.5f)) {
              int kk = INT_MAX;
              float dv = 0.f;
#pragma unroll
              for (int r = 15; r >= 0; --r)
                if (p[r] > 0.5f) {
                  kk = k0 + acc_row(r, hh);
                  dv = dp[sub][r];
                }
              const int ok = __shfl_xor(kk, 32, 64);
              const float odv = __shfl_xor(dv, 32, 64);
              if (ok < kk) {
                kk = ok;
                dv = odv;
              }
              if (!found[sub] && kk != INT_MAX) {
                const float d = ref[sub] - dv;
#pragma unroll
                for (int r = 0; r < 16; ++r) da[sub][r] += d * db[sub][r];
                Cp[sub] += d * Wp[sub];
                ref[sub] = dv;
                imax[sub] = kk;
                found[sub] = true;
              }
            }
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            // with the forward's LSE the reference is this pass's own dP at imax: u = 0 there
            const float u = kLse ? dp[sub][r] - ref[sub]
                                 : ((k0 + acc_row(r, hh) == imax[sub]) ? 0.f : dp[sub][r] - ref[sub]);
            pu[r] = p[r] * u;
            Wp[sub] += p[r];
            Cp[sub] += pu[r];
          }
#pragma unroll
          for (int t = 0; t < STEPS; ++t) {
            M::mma32(da[sub], cur.kt[t], bfrag_from_acc<TC>(pu, t));
            M::mma32(db[sub], cur.kt[t], bfrag_from_acc<TC>(p, t));
          }
        }
      }
      if (more) bias_store((kt + 1) & 1);
      __syncthreads();
      cur = nxt;
    }
  }
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) {
    const float Wt = Wp[sub] + __shfl_xor(Wp[sub], 32, 64);
    const float Ct = Cp[sub] + __shfl_xor(Cp[sub], 32, 64);
    const int q = q0 + 32 * sub + c;
    const float lse2 = dead[sub] ? INFINITY : mrow[sub] + __builtin_amdgcn_logf(Wt);
    const float cen = dead[sub] ? 0.f : Ct / Wt;
    if (active && hh == 0) st4[line * Np + q] = stats_pack(lse2, ref[sub], cen, imax[sub]);
    if (!active || q >= N) continue;
    const float f = dead[sub] ? 0.f : scale / Wt;
    TC* dst = dQ + line_offset(sg, b, sl, hd) + (long)q * sg.n;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (da[sub][4 * j + e] - cen * db[sub][4 * j + e]) * f;
      store_vec<TC, 4>(dst + 8 * j + 4 * hh, v);
    }
  }
}

// ------------------------------------------------------------------ dK, dV
// Block: four lines of one (b, h); each wave owns one line and kRows keys (the columns of
// S = Q K^T) and loops over 32-query tiles. A double-buffered LDS step holds the bias tile
// (transposed, [key][query], so a lane reads its key's rows as 16-byte vectors) and the four
// lines' row statistics. The Q / dO fragments of the next tile are loaded into the registers
// of the current ones as soon as S and dP are issued, and the Q^T / dO^T fragments of the
// current tile at the same point: both loads are covered by the tile's softmax work, and no
// register copies between tiles are needed.
template <class TC, int kSub, bool kOff>
__global__ __launch_bounds__(kNT, sizeof(TC) == 2 ? 3 : 2) void attn_bwd_dkdv_kernel(
    const TC* __restrict__ QR, const TC* __restrict__ KR, const TC* __restrict__ VR, const TC* __restrict__ OR,
    const TC* __restrict__ QT, const TC* __restrict__ OT, const float* __restrict__ mask2,
    const float* __restrict__ bias2, int S, int H, int N, int Np, float scale, const f32x4* __restrict__ st4,
    TC* __restrict__ dK, TC* __restrict__ dV, Strides4 sg, const float* __restrict__ lineoff) {
  using M = Mfma<TC>;
  constexpr int STEPS = kBD / M::K32;
  constexpr int EPS = 16 / STEPS;  // accumulator elements per B fragment step
  constexpr int kRows = 32 * kSub;
  constexpr int BLD = 36;  // bias stage [kRows keys][32 queries + 4]
  __shared__ __attribute__((aligned(16))) float bstage[2][kRows * BLD];
  __shared__ __attribute__((aligned(16))) f32x4 sstage[2][kLines * 32];

  const int bh = blockIdx.z;
  const int b = bh / H;
  const int hd = bh % H;
  const int w = wave_id();
  const int l = lane_id();
  const int hh = l >> 5;
  const int c = l & 31;
  const int s = blockIdx.y * kLines + w;
  const bool active = s < S;
  const long sl = active ? s : (int)blockIdx.y * kLines;
  const long bs = (long)b * S + sl;
  const size_t line = (size_t)bs * H + hd;
  const long lo = line_offset(sg, b, sl, hd);  // this line's dK / dV rows
  const float off = kOff ? lineoff[bs] : 0.f;  // eager rule: this line's logit offset
  const float* b2l = bias2 + (size_t)bh * Np * Np;
  const int kb0 = blockIdx.x * kRows;
  const float sl2 = scale * kLog2e;
  const int nqt = (N + 31) / 32;
  // line whose statistics thread t < 128 stages (the four lines of the group, clamped)
  const int sw = threadIdx.x >> 5;
  const size_t sline = ((size_t)b * S + min((int)blockIdx.y * kLines + sw, S - 1)) * H + hd;

  typename M::Frag kf[kSub][STEPS], vf[kSub][STEPS];
  float mk2[kSub];
  int key[kSub];
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) {
    key[sub] = kb0 + 32 * sub + c;
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      kf[sub][t] = M::load(KR + frag_offset<TC>(line, Np, kb0 / 32 + sub, t, l));
      vf[sub][t] = M::load(VR + frag_offset<TC>(line, Np, kb0 / 32 + sub, t, l));
    }
    mk2[sub] = mask2[bs * Np + key[sub]];
  }

  f32x4 pf[32 * 32 * kSub / 4 / kNT], ps;
  constexpr int BU = 32 * kRows / 4 / kNT;  // 16-byte bias loads per thread per step
  constexpr int KPR = kRows / 4;              // loads per bias row
  auto stage_load = [&](int q0) {
#pragma unroll
    for (int u = 0; u < BU; ++u) {
      const int i = threadIdx.x + u * kNT;  // 32 queries x kRows keys, four keys per load
      pf[u] = *reinterpret_cast<const f32x4*>(b2l + (size_t)(q0 + i / KPR) * Np + kb0 + (i % KPR) * 4);
    }
    if (threadIdx.x < kLines * 32) ps = st4[sline * Np + q0 + (threadIdx.x & 31)];
  };
  auto stage_store = [&](int st) {
#pragma unroll
    for (int u = 0; u < BU; ++u) {
      const int i = threadIdx.x + u * kNT;
      const int q = i / KPR;
      const int k = (i % KPR) * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) bstage[st][(k + e) * BLD + q] = pf[u][e];
    }
    if (threadIdx.x < kLines * 32) sstage[st][threadIdx.x] = ps;
  };
  typename M::Frag qa[STEPS], oa[STEPS];
  auto fetch_qo = [&](int q0) {
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      qa[t] = M::load(QR + frag_offset<TC>(line, Np, q0 / 32, t, l));
      oa[t] = M::load(OR + frag_offset<TC>(line, Np, q0 / 32, t, l));
    }
  };

  f32x16 dk[kSub], dv[kSub];
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) dk[sub] = dv[sub] = f32x16{};
  if (active) fetch_qo(0);
  stage_load(0);
  stage_store(0);
  __syncthreads();
  for (int qt = 0; qt < nqt; ++qt) {
    const int q0 = qt * 32;
    const bool more = qt + 1 < nqt;
    if (more) stage_load(q0 + 32);
    if (active) {
      f32x16 sa[kSub], dp[kSub];
#pragma unroll
      for (int sub = 0; sub < kSub; ++sub) {
        sa[sub] = dp[sub] = f32x16{};
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
          M::mma32(sa[sub], qa[t], kf[sub][t]);
          M::mma32(dp[sub], oa[t], vf[sub][t]);
        }
      }
      typename M::Frag qtf[STEPS], otf[STEPS];
#pragma unroll
      for (int t = 0; t < STEPS; ++t) {
        qtf[t] = M::load(QT + frag_offset<TC>(line, Np, q0 / 32, t, l));
        otf[t] = M::load(OT + frag_offset<TC>(line, Np, q0 / 32, t, l));
      }
      if (more) fetch_qo(q0 + 32);
      const float* bst = bstage[qt & 1];
      const f32x4* sst = &sstage[qt & 1][w * 32];
#pragma unroll
      for (int sub = 0; sub < kSub; ++sub) {
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
          f32x16 p, ds;  // elements EPS t .. EPS t + EPS - 1 are formed and used here
#pragma unroll
          for (int jj = 0; jj < EPS / 4; ++jj) {
            const int j = t * (EPS / 4) + jj;
            const f32x4 b4 = *reinterpret_cast<const f32x4*>(bst + (32 * sub + c) * BLD + 8 * j + 4 * hh);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int r = 4 * j + e;
              const f32x4 st = sst[8 * j + 4 * hh + e];  // {lse2, ref, cen, imax}
              float x = logit2(sa[sub][r], sl2, b4[e], mk2[sub]);
              if constexpr (kOff) x -= off;
              const float pv = __builtin_amdgcn_exp2f(x - st[0]);
              const float u = (key[sub] == __float_as_int(st[3])) ? 0.f : dp[sub][r] - st[1];
              p[r] = pv;
              ds[r] = pv * (u - st[2]);
            }
          }
          M::mma32(dv[sub], otf[t], bfrag_from_acc<TC>(p, t));
          M::mma32(dk[sub], qtf[t], bfrag_from_acc<TC>(ds, t));
        }
      }
    }
    if (more) stage_store((qt + 1) & 1);
    __syncthreads();
  }
  if (!active) return;
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) {
    if (key[sub] >= N) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float vk[4], vv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vk[e] = dk[sub][4 * j + e] * scale;
        vv[e] = dv[sub][4 * j + e];
      }
      store_vec<TC, 4>(dK + lo + (long)key[sub] * sg.n + 8 * j + 4 * hh, vk);
      store_vec<TC, 4>(dV + lo + (long)key[sub] * sg.n + 8 * j + 4 * hh, vv);
    }
  }
}

// ------------------------------------------------------------------ d_bias
// Block: 64 queries x 64 keys of one (b, h) and one group of lines; wave w takes query tile
// (w & 1) and key tile (w >> 1) and sums dS^T over its lines, fetching the next line's
// operands while it works on the current one. Groups write partial sums, added in a fixed
// order by attn_bwd_db_reduce (so the result does not depend on scheduling).
template <class TC>
struct DbOps {
  typename Mfma<TC>::Frag k[kBD / Mfma<TC>::K32], q[kBD / Mfma<TC>::K32], v[kBD / Mfma<TC>::K32],
      o[kBD / Mfma<TC>::K32];
  f32x4 st;
  f32x4 m[4];
  float off;
};

template <class TC, bool kOff>
__global__ __launch_bounds__(kNT, 3) void attn_bwd_db_kernel(const TC* __restrict__ QR, const TC* __restrict__ KR,
                                                          const TC* __restrict__ VR, const TC* __restrict__ OR,
                                                          const float* __restrict__ mask2,
                                                          const float* __restrict__ bias2, int S, int H, int N,
                                                          int Np, float scale, int groups,
                                                          const f32x4* __restrict__ st4, float* __restrict__ dbias,
                                                          const float* __restrict__ lineoff) {
  using M = Mfma<TC>;
  constexpr int STEPS = kBD / M::K32;
  const int bh = blockIdx.z / groups;
  const int grp = blockIdx.z % groups;
  const int b = bh / H;
  const int hd = bh % H;
  const int w = wave_id();
  const int l = lane_id();
  const int hh = l >> 5;
  const int c = l & 31;
  const int q = blockIdx.x * 64 + (w & 1) * 32 + c;
  const int k0 = blockIdx.y * 64 + (w >> 1) * 32;
  const float sl2 = scale * kLog2e;
  const int s_begin = (int)((long)S * grp / groups);
  const int s_end = (int)((long)S * (grp + 1) / groups);
  f32x4 b4[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    b4[j] = *reinterpret_cast<const f32x4*>(bias2 + ((size_t)bh * Np + q) * Np + k0 + 8 * j + 4 * hh);
  auto fetch = [&](int s, DbOps<TC>& op) {
    const long bs = (long)b * S + s;
    const size_t line = (size_t)bs * H + hd;
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      op.k[t] = M::load(KR + frag_offset<TC>(line, Np, k0 / 32, t, l));
      op.q[t] = M::load(QR + frag_offset<TC>(line, Np, q / 32, t, l));
      op.v[t] = M::load(VR + frag_offset<TC>(line, Np, k0 / 32, t, l));
      op.o[t] = M::load(OR + frag_offset<TC>(line, Np, q / 32, t, l));
    }
    op.st = st4[line * Np + q];
    op.off = kOff ? lineoff[bs] : 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) op.m[j] = *reinterpret_cast<const f32x4*>(mask2 + bs * Np + k0 + 8 * j + 4 * hh);
  };
  f32x16 acc = {};
  if (s_begin < s_end) {
    DbOps<TC> cur, nxt;
    fetch(s_begin, cur);
    for (int s = s_begin; s < s_end; ++s) {
      if (s + 1 < s_end) fetch(s + 1, nxt);
      f32x16 sa = {}, dp = {};
#pragma unroll
      for (int t = 0; t < STEPS; ++t) {
        M::mma32(sa, cur.k[t], cur.q[t]);
        M::mma32(dp, cur.v[t], cur.o[t]);
      }
      const int im = __float_as_int(cur.st[3]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * j + e;
          const int key = k0 + 8 * j + 4 * hh + e;
          float x = logit2(sa[r], sl2, b4[j][e], cur.m[j][e]);
          if constexpr (kOff) x -= cur.off;
          const float pv = __builtin_amdgcn_exp2f(x - cur.st[0]);
          const float u = key == im ? 0.f : dp[r] - cur.st[1];
          acc[r] += pv * (u - cur.st[2]);
        }
      cur = nxt;
    }
  }
  if (q < N) {
    float* prow = dbias + (((size_t)grp * (gridDim.z / groups) + bh) * N + q) * N;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k0 + acc_row(r, hh);
      if (key < N) prow[key] = acc[r];
    }
  }
}

// dbias[i] = sum_g partial[g][i], in group order.
__global__ __launch_bounds__(256) void attn_bwd_db_reduce_kernel(const float* __restrict__ partial, size_t n,
                                                                 int groups, float* __restrict__ dbias) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    float s = 0.f;
    for (int g = 0; g < groups; ++g) s += partial[(size_t)g * n + i];
    dbias[i] = s;
  }
}

// Line groups of the bias gradient: enough blocks to fill the chip (about 2048), at most 16.
int db_groups(int B, int H, int N, int S) {
  const long tiles = (long)B * H * ((N + 63) / 64) * ((N + 63) / 64);
  int g = 1;
  while (g < 16 && tiles * g < 2048 && g * 2 <= S) g *= 2;
  return g;
}

struct BwdWs {
  size_t st, bias2, mask2, off, kr, qr, orr, vr, kt, qt, ot, part, total;
  int groups;
};

BwdWs bwd_ws_layout(int B, int S, int H, int N, int es) {
  const size_t Np = (size_t)pf::pad128(N);
  const size_t lines = (size_t)B * S * H;
  BwdWs w;
  w.groups = db_groups(B, H, N, S);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = pf::round_up(off + bytes, 256);
    return o;
  };
  w.st = take(lines * Np * 16);
  w.bias2 = take((size_t)B * H * Np * Np * 4);
  w.mask2 = take((size_t)B * S * Np * 4);
  w.off = take((size_t)B * S * 4);
  w.kr = take(lines * kBD * Np * es);
  w.qr = take(lines * kBD * Np * es);
  w.orr = take(lines * kBD * Np * es);
  w.vr = take(lines * kBD * Np * es);
  w.kt = take(lines * kBD * Np * es);
  w.qt = take(lines * kBD * Np * es);
  w.ot = take(lines * kBD * Np * es);
  w.part = w.groups > 1 ? take((size_t)w.groups * B * H * N * N * 4) : 0;
  w.total = off;
  return w;
}

template <class TC>
int attn_bwd_launch(const void* q, const void* k, const void* v, const float* res_mask, const float* pair_bias,
                    const void* dout, int B, int S, int H, int N, float scale, void* dq, void* dk, void* dv,
                    float* dbias, void* ws, hipStream_t s, const Strides4& sx, const Strides4& sdo,
                    const Strides4& sg, const float* lse_in, bool zero_rows) {
  const BwdWs lay = bwd_ws_layout(B, S, H, N, (int)sizeof(TC));
  char* base = static_cast<char*>(ws);
  f32x4* st4 = reinterpret_cast<f32x4*>(base + lay.st);
  float* bias2 = reinterpret_cast<float*>(base + lay.bias2);
  float* mask2 = reinterpret_cast<float*>(base + lay.mask2);
  float* lineoff = reinterpret_cast<float*>(base + lay.off);
  TC* KR = reinterpret_cast<TC*>(base + lay.kr);
  TC* QR = reinterpret_cast<TC*>(base + lay.qr);
  TC* OR = reinterpret_cast<TC*>(base + lay.orr);
  TC* VR = reinterpret_cast<TC*>(base + lay.vr);
  TC* KT = reinterpret_cast<TC*>(base + lay.kt);
  TC* QT = reinterpret_cast<TC*>(base + lay.qt);
  TC* OT = reinterpret_cast<TC*>(base + lay.ot);
  const int Np = pf::pad128(N);
  const unsigned lines = (unsigned)((long)B * S * H);
  const TC *Q = static_cast<const TC*>(q), *K = static_cast<const TC*>(k), *V = static_cast<const TC*>(v),
           *dO = static_cast<const TC*>(dout);
  {
    const size_t n = (size_t)B * H * Np * Np + (size_t)B * S * Np;
    attn_bwd_prep_kernel<<<(unsigned)std::min<size_t>((n + 255) / 256, 8192), 256, 0, s>>>(
        pair_bias, res_mask, bias2, mask2, B * H, B * S, N, Np);
    if (int e = pf::check_launch("attn_bwd_prep")) return e;
  }
  attn_bwd_relayout_kernel<TC><<<dim3((unsigned)(Np / 64), lines, 4), 256, 0, s>>>(K, Q, dO, V, KR, QR, OR, VR, KT,
                                                                                   QT, OT, S, H, N, Np, sx, sdo);
  if (int e = pf::check_launch("attn_bwd_relayout")) return e;
  const unsigned lg = (unsigned)((S + kLines - 1) / kLines);
  const dim3 gdq((unsigned)(Np / (32 * kSubDq)), lg, (unsigned)(B * H));
  // The eager rule shifts each line's logits by its offset (the saved-LSE path is zero-rule only).
  const bool eager = !zero_rows;
  if (eager) {
    attn_bwd_lineoff_kernel<<<(unsigned)(B * S), 64, 0, s>>>(mask2, lineoff, N, Np, kDeadLog2);
    if (int e = pf::check_launch("attn_bwd_lineoff")) return e;
  }
  const float dead_below = zero_rows ? kDeadLog2 : kDeadEager;
  if (lse_in)
    attn_bwd_dq_kernel<TC, kSubDq, true, false><<<gdq, kNT, 0, s>>>(QR, KR, VR, OR, V, KT, mask2, bias2, S, H, N,
                                                                    Np, scale, static_cast<TC*>(dq), st4, sx, sg,
                                                                    lse_in, dead_below, nullptr);
  else if (eager)
    attn_bwd_dq_kernel<TC, kSubDq, false, true><<<gdq, kNT, 0, s>>>(QR, KR, VR, OR, V, KT, mask2, bias2, S, H, N,
                                                                    Np, scale, static_cast<TC*>(dq), st4, sx, sg,
                                                                    nullptr, dead_below, lineoff);
  else
    attn_bwd_dq_kernel<TC, kSubDq, false, false><<<gdq, kNT, 0, s>>>(QR, KR, VR, OR, V, KT, mask2, bias2, S, H, N,
                                                                     Np, scale, static_cast<TC*>(dq), st4, sx, sg,
                                                                     nullptr, dead_below, nullptr);
  if (int e = pf::check_launch("attn_bwd_dq")) return e;
  const dim3 gkv((unsigned)(Np / (32 * kSubKv)), lg, (unsigned)(B * H));
  if (eager)
    attn_bwd_dkdv_kernel<TC, kSubKv, true><<<gkv, kNT, 0, s>>>(QR, KR, VR, OR, QT, OT, mask2, bias2, S, H, N, Np,
                                                               scale, st4, static_cast<TC*>(dk),
                                                               static_cast<TC*>(dv), sg, lineoff);
  else
    attn_bwd_dkdv_kernel<TC, kSubKv, false><<<gkv, kNT, 0, s>>>(QR, KR, VR, OR, QT, OT, mask2, bias2, S, H, N, Np,
                                                                scale, st4, static_cast<TC*>(dk),
                                                                static_cast<TC*>(dv), sg, nullptr);
  if (int e = pf::check_launch("attn_bwd_dkdv")) return e;
  const unsigned nb = (unsigned)((N + 63) / 64);
  const int G = lay.groups;
  float* part = G > 1 ? reinterpret_cast<float*>(base + lay.part) : dbias;
  const dim3 gdb(nb, nb, (unsigned)(B * H * G));
  if (eager)
    attn_bwd_db_kernel<TC, true><<<gdb, kNT, 0, s>>>(QR, KR, VR, OR, mask2, bias2, S, H, N, Np, scale, G, st4, part,
                                                     lineoff);
  else
    attn_bwd_db_kernel<TC, false><<<gdb, kNT, 0, s>>>(QR, KR, VR, OR, mask2, bias2, S, H, N, Np, scale, G, st4, part,
                                                      nullptr);
  if (int e = pf::check_launch("attn_bwd_db")) return e;
  if (G > 1) {
    const size_t n = (size_t)B * H * N * N;
    attn_bwd_db_reduce_kernel<<<(unsigned)std::min<size_t>((n + 255) / 256, 4096), 256, 0, s>>>(part, n, G, dbias);
    if (int e = pf::check_launch("attn_bwd_db_reduce")) return e;
  }
  return PF_OK;
}

// Shared checks and dispatch of the dense and strided entry points.
int evo_attn_bwd_any(const char* fn, const void* q, const void* k, const void* v, const float* res_mask,
                     const float* pair_bias, const void* dout, int B, int S, int H, int N, int D, int dtype,
                     float softmax_scale, void* dq, void* dk, void* dv, float* dpair_bias, void* workspace,
                     size_t workspace_bytes, void* stream, const Strides4& sx, const Strides4& sdo,
                     const Strides4& sg, const float* lse_in, bool zero_rows) {
  PF_REQUIRE(q && k && v && res_mask && pair_bias && dout && dq && dk && dv && dpair_bias && workspace,
             PF_ERR_INVALID_ARG, "%s: null pointer", fn);
  PF_REQUIRE(B > 0 && S > 0 && H > 0 && N > 0, PF_ERR_INVALID_ARG, "%s: B=%d S=%d H=%d N=%d", fn, B, S, H, N);
  PF_REQUIRE((long)B * S * H <= 65535 && (long)B * H <= 65535 && (long)N * N < (1L << 31), PF_ERR_INVALID_ARG,
             "%s: B*S*H=%ld N=%d too large (grid rows are the B*S*H lines)", fn, (long)B * S * H, N);
  PF_REQUIRE(D == kBD, PF_ERR_UNSUPPORTED, "%s: D=%d (built: D=32)", fn, D);
  PF_REQUIRE(dtype == PF_F32 || dtype == PF_BF16, PF_ERR_UNSUPPORTED, "%s: dtype %d", fn, dtype);
  PF_REQUIRE(zero_rows || !lse_in, PF_ERR_UNSUPPORTED, "%s: the saved-LSE backward follows the zero masked-row rule",
             fn);
  const long vec = dtype == PF_F32 ? 4 : 8;  // elements per 16 bytes
  for (const Strides4* st : {&sx, &sdo, &sg})
    PF_REQUIRE(st->b % vec == 0 && st->s % vec == 0 && st->h % vec == 0 && st->n % vec == 0 && st->n >= kBD,
               PF_ERR_ALIGNMENT, "%s: strides must keep 16-byte aligned rows of D elements", fn);
  PF_REQUIRE(pf::aligned16(q) && pf::aligned16(k) && pf::aligned16(v) && pf::aligned16(dout) && pf::aligned16(dq) &&
                 pf::aligned16(dk) && pf::aligned16(dv) && pf::aligned16(workspace),
             PF_ERR_ALIGNMENT, "%s: operand pointers must be 16-byte aligned", fn);
  const size_t need = bwd_ws_layout(B, S, H, N, dtype == PF_F32 ? 4 : 2).total;
  PF_REQUIRE(workspace_bytes >= need, PF_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", fn, workspace_bytes, need);
  hipStream_t s = pf::as_stream(stream);
  if (dtype == PF_F32)
    return attn_bwd_launch<float>(q, k, v, res_mask, pair_bias, dout, B, S, H, N, softmax_scale, dq, dk, dv,
                                  dpair_bias, workspace, s, sx, sdo, sg, lse_in, zero_rows);
  return attn_bwd_launch<bf16>(q, k, v, res_mask, pair_bias, dout, B, S, H, N, softmax_scale, dq, dk, dv, dpair_bias,
                               workspace, s, sx, sdo, sg, lse_in, zero_rows);
}

}  // namespace

extern "C" {

size_t pf_evo_attn_bwd_workspace_bytes(int B, int S, int H, int N, int D, int dtype) {
  if (B <= 0 || S <= 0 || H <= 0 || N <= 0 || D != kBD || (dtype != PF_F32 && dtype != PF_BF16)) return 0;
  return bwd_ws_layout(B, S, H, N, dtype == PF_F32 ? 4 : 2).total;
}

int pf_evo_attn_bwd(const void* q, const void* k, const void* v, const float* res_mask, const float* pair_bias,
                    const void* dout, int B, int S, int H, int N, int D, int dtype, float softmax_scale,
                    int zero_masked_rows, void* dq, void* dk, void* dv, float* dpair_bias, void* workspace,
                    size_t workspace_bytes, void* stream) {
  const Strides4 dense{(long)S * H * N * D, (long)H * N * D, (long)N * D, D};
  return evo_attn_bwd_any("pf_evo_attn_bwd", q, k, v, res_mask, pair_bias, dout, B, S, H, N, D, dtype, softmax_scale,
                          dq, dk, dv, dpair_bias, workspace, workspace_bytes, stream, dense, dense, dense, nullptr,
                          zero_masked_rows != 0);
}

int pf_evo_attn_bwd_strided(const void* q, const void* k, const void* v, const long* qkv_strides,
                            const float* res_mask, const float* pair_bias, const void* dout, const long* dout_strides,
                            const float* lse, int B, int S, int H, int N, int D, int dtype, float softmax_scale,
                            void* dq, void* dk,
                            void* dv, const long* grad_strides, float* dpair_bias, void* workspace,
                            size_t workspace_bytes, void* stream) {
  PF_REQUIRE(qkv_strides && dout_strides && grad_strides, PF_ERR_INVALID_ARG, "pf_evo_attn_bwd_strided: null strides");
  const Strides4 sx{qkv_strides[0], qkv_strides[1], qkv_strides[2], qkv_strides[3]};
  const Strides4 sdo{dout_strides[0], dout_strides[1], dout_strides[2], dout_strides[3]};
  const Strides4 sg{grad_strides[0], grad_strides[1], grad_strides[2], grad_strides[3]};
  return evo_attn_bwd_any("pf_evo_attn_bwd_strided", q, k, v, res_mask, pair_bias, dout, B, S, H, N, D, dtype,
                          softmax_scale, dq, dk, dv, dpair_bias, workspace, workspace_bytes, stream, sx, sdo, sg,
                          lse, true);
}

}  // extern "C"
