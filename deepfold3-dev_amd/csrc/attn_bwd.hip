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
// A line whose keys are all masked (max logit < -1e8) gets LSE = +inf, so P = 0 and every
// gradient of its rows is 0: the reference kernel's masked-row rule (its forward writes 0).
//
// Kernels, all on 32x32 MFMA tiles with D = 32:
//   attn_bwd_transpose: K, Q, dO transposed to [d][row] once, so that the products that
//                  contract over rows (dQ over keys, dK and dV over queries) load their
//                  fragments straight from memory.
//   attn_bwd_dq:   query-major. Pass 1 over the keys builds (LSE, dP_imax, imax, C) per row
//                  online (running max with rescaling and re-centring); pass 2 forms dS and
//                  dQ. The row statistics go to the workspace for the other kernels.
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
// Zero masked-row rule threshold in log2 units (the reference tests t < -1e8).
constexpr float kDeadLog2 = -1.0e8f * kLog2e;

// An A fragment whose k order matches bfrag_from_acc (the accumulator's row order):
// bf16 step t of 2: element e is k = 16t + 8(e>>2) + 4h + (e&3); fp32 step t of 4:
// element e is k = 8t + 4h + e. `row` points at the A row in LDS, k contiguous.
template <class TC>
PF_DEVICE typename Mfma<TC>::Frag afrag_perm(const TC* row, int t, int h);
template <>
PF_DEVICE bf16x8 afrag_perm<bf16>(const bf16* row, int t, int h) {
  const bf16x4 lo = *reinterpret_cast<const bf16x4*>(row + 16 * t + 4 * h);
  const bf16x4 hi = *reinterpret_cast<const bf16x4*>(row + 16 * t + 8 + 4 * h);
  bf16x8 f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[e] = lo[e];
    f[4 + e] = hi[e];
  }
  return f;
}
template <>
PF_DEVICE f32x4 afrag_perm<float>(const float* row, int t, int h) {
  return *reinterpret_cast<const f32x4*>(row + 8 * t + 4 * h);
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

// XT [line][d][Np] = X [line][n][d] for n < N, 0 for N <= n < Np, for the three operands a
// contraction over rows needs with rows along the lanes' k slices (blockIdx.z: K, Q, dO).
template <class TC>
__global__ __launch_bounds__(256) void attn_bwd_transpose_kernel(const TC* __restrict__ K, const TC* __restrict__ Q,
                                                                 const TC* __restrict__ dO, TC* __restrict__ KT,
                                                                 TC* __restrict__ QT, TC* __restrict__ OT, int N,
                                                                 int Np) {
  constexpr int VEC = 16 / sizeof(TC);
  constexpr int R = 64;  // rows per block
  constexpr int LD = R + VEC;
  __shared__ __attribute__((aligned(16))) TC t[kBD * LD];  // [d][row]
  const TC* X = blockIdx.z == 0 ? K : (blockIdx.z == 1 ? Q : dO);
  TC* XT = blockIdx.z == 0 ? KT : (blockIdx.z == 1 ? QT : OT);
  const size_t line = blockIdx.y;
  const int n0 = blockIdx.x * R;
  const TC* Xl = X + line * N * kBD;
  for (int i = threadIdx.x; i < R * (kBD / VEC); i += 256) {
    const int r = i / (kBD / VEC);
    const int d0 = (i % (kBD / VEC)) * VEC;
    const int n = n0 + r;
    TC e[VEC];
    if (n < N) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(Xl + (size_t)n * kBD + d0);
      __builtin_memcpy(e, &v, 16);
    } else {
#pragma unroll
      for (int u = 0; u < VEC; ++u) e[u] = from_f32<TC>(0.f);
    }
#pragma unroll
    for (int u = 0; u < VEC; ++u) t[(d0 + u) * LD + r] = e[u];
  }
  __syncthreads();
  TC* XTl = XT + line * kBD * Np;
  for (int i = threadIdx.x; i < kBD * (R / VEC); i += 256) {
    const int d = i / (R / VEC);
    const int r0 = (i % (R / VEC)) * VEC;
    *reinterpret_cast<u32x4*>(XTl + (size_t)d * Np + n0 + r0) = *reinterpret_cast<const u32x4*>(t + d * LD + r0);
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

// Logit in log2 units from the raw product s (times scale log2 e), the bias and the mask
// (both already times log2 e); every kernel forms it the same way.
PF_DEVICE float logit2(float s, float sl2, float b2, float m2) { return fmaf(s, sl2, b2 + m2); }

// Row statistics, one 16-byte record per (line, query): {LSE (log2), dP at the argmax, C, argmax}.
PF_DEVICE f32x4 stats_pack(float lse2, float ref, float cen, int imax) {
  return f32x4{lse2, ref, cen, __int_as_float(imax)};
}

// ------------------------------------------------------------------ dQ (+ row statistics)
// Block: four lines of one (b, h) sharing a double-buffered pair-bias tile in LDS; each wave
// owns one line and kRows queries (kSub sub-tiles of 32, the columns of S^T = K Q^T). The
// next key tile's K / V / K^T fragments and mask are fetched while the current one computes.
template <class TC>
struct DqOps {
  typename Mfma<TC>::Frag k[kBD / Mfma<TC>::K32], v[kBD / Mfma<TC>::K32], kt[kBD / Mfma<TC>::K32];
  f32x4 m[4];
};

template <class TC, int kSub>
__global__ __launch_bounds__(kNT) void attn_bwd_dq_kernel(const TC* __restrict__ Q, const TC* __restrict__ K,
                                                          const TC* __restrict__ V, const TC* __restrict__ dO,
                                                          const TC* __restrict__ KT, const float* __restrict__ mask2,
                                                          const float* __restrict__ bias2, int S, int H, int N,
                                                          int Np, float scale, TC* __restrict__ dQ,
                                                          f32x4* __restrict__ st4) {
  using M = Mfma<TC>;
  constexpr int STEPS = kBD / M::K32;
  constexpr int kRows = 32 * kSub;
  constexpr int BLD = 36;  // bias stage [query][32 keys + 4]
  __shared__ __attribute__((aligned(16))) float bstage[2][kRows * BLD];

  const int bh = blockIdx.z;
  const int b = bh / H;
  const int hd = bh % H;
  const int w = wave_id();
  const int l = lane_id();
  const int hh = l >> 5;
  const int c = l & 31;
  const int s = blockIdx.y * kLines + w;
  const bool active = s < S;  // inactive waves mirror the group's first line and skip the math
  const long bs = (long)b * S + (active ? s : (int)blockIdx.y * kLines);
  const size_t line = (size_t)bs * H + hd;
  const size_t lo = line * N * kBD;
  const TC *Kl = K + lo, *Vl = V + lo;
  const TC* KTl = KT + line * kBD * Np;
  const float* m2l = mask2 + bs * Np;
  const float* b2l = bias2 + (size_t)bh * Np * Np;
  const int q0 = blockIdx.x * kRows;
  const float sl2 = scale * kLog2e;
  const int nkt = (N + 31) / 32;

  typename M::Frag qf[kSub][STEPS], of[kSub][STEPS];
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) {
    const int qc = min(q0 + 32 * sub + c, N - 1);
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      qf[sub][t] = M::load(Q + lo + (size_t)qc * kBD + t * M::K32 + hh * M::KPL);
      of[sub][t] = M::load(dO + lo + (size_t)qc * kBD + t * M::K32 + hh * M::KPL);
    }
  }

  f32x4 pf[2];
  constexpr int BU = kRows * 8 / kNT;  // 16-byte bias loads per thread per step
  auto bias_load = [&](int k0) {
#pragma unroll
    for (int u = 0; u < BU; ++u) {
      const int i = threadIdx.x + u * kNT;
      pf[u] = *reinterpret_cast<const f32x4*>(b2l + (size_t)(q0 + (i >> 3)) * Np + k0 + (i & 7) * 4);
    }
  };
  auto bias_store = [&](int st) {
#pragma unroll
    for (int u = 0; u < BU; ++u) {
      const int i = threadIdx.x + u * kNT;
      *reinterpret_cast<f32x4*>(&bstage[st][(i >> 3) * BLD + (i & 7) * 4]) = pf[u];
    }
  };
  auto fetch = [&](int k0, DqOps<TC>& o, bool with_kt) {
    const int kc = min(k0 + c, N - 1);
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      o.k[t] = M::load(Kl + (size_t)kc * kBD + t * M::K32 + hh * M::KPL);
      o.v[t] = M::load(Vl + (size_t)kc * kBD + t * M::K32 + hh * M::KPL);
      if (with_kt) o.kt[t] = afrag_perm<TC>(KTl + (size_t)c * Np + k0, t, hh);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) o.m[j] = *reinterpret_cast<const f32x4*>(m2l + k0 + 8 * j + 4 * hh);
  };
  // log2 logits x and dP^T for keys k0..k0+31 (rows) and this wave's queries (columns)
  auto tile = [&](const DqOps<TC>& o, int st, f32x16 (&x)[kSub], f32x16 (&dp)[kSub]) {
#pragma unroll
    for (int sub = 0; sub < kSub; ++sub) {
      f32x16 sa = {};
      dp[sub] = f32x16{};
#pragma unroll
      for (int t = 0; t < STEPS; ++t) {
        M::mma32(sa, o.k[t], qf[sub][t]);
        M::mma32(dp[sub], o.v[t], of[sub][t]);
      }
      const float* brow = &bstage[st][(32 * sub + c) * BLD];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(brow + 8 * j + 4 * hh);
#pragma unroll
        for (int e = 0; e < 4; ++e) x[sub][4 * j + e] = logit2(sa[4 * j + e], sl2, b4[e], o.m[j][e]);
      }
    }
  };

  // Pass 1: running max m, first argmax, dP there, and per-lane partial sums
  // W = sum exp2(x - m), Cp = sum exp2(x - m) (dP - ref) over this lane's keys.
  float run_max[kSub], refv[kSub], Wp[kSub], Cp[kSub];
  int imx[kSub];
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) {
    run_max[sub] = -INFINITY;
    refv[sub] = Wp[sub] = Cp[sub] = 0.f;
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
      if (kt + 1 < nkt) {
        bias_load(k0 + 32);
        fetch(k0 + 32, nxt, false);
      }
      if (active) {
        f32x16 x[kSub], dp[kSub];
        tile(cur, kt & 1, x, dp);
#pragma unroll
        for (int sub = 0; sub < kSub; ++sub) {
          float tmax = x[sub][0];
#pragma unroll
          for (int r = 1; r < 16; ++r) tmax = fmaxf(tmax, x[sub][r]);
          tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
          int targ = INT_MAX;
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (x[sub][r] == tmax) targ = min(targ, k0 + acc_row(r, hh));
          targ = min(targ, __shfl_xor(targ, 32, 64));
          float tref = 0.f;
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (k0 + acc_row(r, hh) == targ) tref = dp[sub][r];
          tref += __shfl_xor(tref, 32, 64);  // exactly one lane of the pair holds it
          const bool better = tmax > run_max[sub];
          const float m_new = better ? tmax : run_max[sub];
          if (m_new != -INFINITY) {
            const float alpha = __builtin_amdgcn_exp2f(run_max[sub] - m_new);
            Wp[sub] *= alpha;
            Cp[sub] *= alpha;
            if (better) {
              Cp[sub] += (refv[sub] - tref) * Wp[sub];  // re-centre the mass seen so far
              refv[sub] = tref;
              imx[sub] = targ;
            }
            float ws = 0.f, cs = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float p = x[sub][r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(x[sub][r] - m_new);
              ws += p;
              cs += p * (dp[sub][r] - refv[sub]);
            }
            Wp[sub] += ws;
            Cp[sub] += cs;
            run_max[sub] = m_new;
          }
        }
      }
      if (kt + 1 < nkt) bias_store((kt + 1) & 1);
      __syncthreads();
      cur = nxt;
    }
  }
  float lse2[kSub], cen[kSub], ref[kSub];
  int imax[kSub];
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) {
    const float Wt = Wp[sub] + __shfl_xor(Wp[sub], 32, 64);
    const float Ct = Cp[sub] + __shfl_xor(Cp[sub], 32, 64);
    const int q = q0 + 32 * sub + c;
    const bool dead = !(run_max[sub] >= kDeadLog2) || q >= N;
    lse2[sub] = dead ? INFINITY : run_max[sub] + __builtin_amdgcn_logf(Wt);
    cen[sub] = dead ? 0.f : Ct / Wt;
    ref[sub] = dead ? 0.f : refv[sub];
    imax[sub] = dead ? -1 : imx[sub];
    if (active && hh == 0) st4[line * Np + q] = stats_pack(lse2[sub], ref[sub], cen[sub], imax[sub]);
  }

  // Pass 2: dS^T, then dQ^T [d x q] += K^T [d x keys] dS^T [keys x q].
  f32x16 dq[kSub];
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) dq[sub] = f32x16{};
  {
    DqOps<TC> cur, nxt;
    fetch(0, cur, true);
    bias_load(0);
    bias_store(0);
    __syncthreads();
    for (int kt = 0; kt < nkt; ++kt) {
      const int k0 = kt * 32;
      if (kt + 1 < nkt) {
        bias_load(k0 + 32);
        fetch(k0 + 32, nxt, true);
      }
      if (active) {
        f32x16 x[kSub], dp[kSub];
        tile(cur, kt & 1, x, dp);
#pragma unroll
        for (int sub = 0; sub < kSub; ++sub) {
          f32x16 ds;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float p = __builtin_amdgcn_exp2f(x[sub][r] - lse2[sub]);
            const float u = (k0 + acc_row(r, hh) == imax[sub]) ? 0.f : dp[sub][r] - ref[sub];
            ds[r] = p * (u - cen[sub]);
          }
#pragma unroll
          for (int t = 0; t < STEPS; ++t) M::mma32(dq[sub], cur.kt[t], bfrag_from_acc<TC>(ds, t));
        }
      }
      if (kt + 1 < nkt) bias_store((kt + 1) & 1);
      __syncthreads();
      cur = nxt;
    }
  }
  if (!active) return;
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) {
    const int q = q0 + 32 * sub + c;
    if (q >= N) continue;
    TC* dst = dQ + lo + (size_t)q * kBD;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = dq[sub][4 * j + e] * scale;
      store_vec<TC, 4>(dst + 8 * j + 4 * hh, v);
    }
  }
}

// ------------------------------------------------------------------ dK, dV
// Block: four lines of one (b, h); each wave owns one line and kRows keys (the columns of
// S = Q K^T) and loops over 32-query tiles. A double-buffered LDS step holds the bias tile
// (transposed, [key][query], so a lane reads its key's rows as 16-byte vectors) and the four
// lines' row statistics; the next tile's Q / dO / Q^T / dO^T fragments are fetched while the
// current one computes.
template <class TC>
struct DkvOps {
  typename Mfma<TC>::Frag q[kBD / Mfma<TC>::K32], o[kBD / Mfma<TC>::K32], qt[kBD / Mfma<TC>::K32],
      ot[kBD / Mfma<TC>::K32];
};

template <class TC, int kSub>
__global__ __launch_bounds__(kNT) void attn_bwd_dkdv_kernel(
    const TC* __restrict__ Q, const TC* __restrict__ K, const TC* __restrict__ V, const TC* __restrict__ dO,
    const TC* __restrict__ QT, const TC* __restrict__ OT, const float* __restrict__ mask2,
    const float* __restrict__ bias2, int S, int H, int N, int Np, float scale, const f32x4* __restrict__ st4,
    TC* __restrict__ dK, TC* __restrict__ dV) {
  using M = Mfma<TC>;
  constexpr int STEPS = kBD / M::K32;
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
  const long bs = (long)b * S + (active ? s : (int)blockIdx.y * kLines);
  const size_t line = (size_t)bs * H + hd;
  const size_t lo = line * N * kBD;
  const TC *Ql = Q + lo, *Ol = dO + lo;
  const TC* QTl = QT + line * kBD * Np;
  const TC* OTl = OT + line * kBD * Np;
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
    const int kc = min(key[sub], N - 1);
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      kf[sub][t] = M::load(K + lo + (size_t)kc * kBD + t * M::K32 + hh * M::KPL);
      vf[sub][t] = M::load(V + lo + (size_t)kc * kBD + t * M::K32 + hh * M::KPL);
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
  auto fetch = [&](int q0, DkvOps<TC>& o) {
    const int qc = min(q0 + c, N - 1);
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      o.q[t] = M::load(Ql + (size_t)qc * kBD + t * M::K32 + hh * M::KPL);
      o.o[t] = M::load(Ol + (size_t)qc * kBD + t * M::K32 + hh * M::KPL);
      o.qt[t] = afrag_perm<TC>(QTl + (size_t)c * Np + q0, t, hh);
      o.ot[t] = afrag_perm<TC>(OTl + (size_t)c * Np + q0, t, hh);
    }
  };

  f32x16 dk[kSub], dv[kSub];
#pragma unroll
  for (int sub = 0; sub < kSub; ++sub) dk[sub] = dv[sub] = f32x16{};
  DkvOps<TC> cur, nxt;
  fetch(0, cur);
  stage_load(0);
  stage_store(0);
  __syncthreads();
  for (int qt = 0; qt < nqt; ++qt) {
    const int q0 = qt * 32;
    if (qt + 1 < nqt) {
      stage_load(q0 + 32);
      fetch(q0 + 32, nxt);
    }
    if (active) {
      const float* bst = bstage[qt & 1];
      const f32x4* sst = &sstage[qt & 1][w * 32];
#pragma unroll
      for (int sub = 0; sub < kSub; ++sub) {
        f32x16 sa = {}, dp = {};
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
          M::mma32(sa, cur.q[t], kf[sub][t]);
          M::mma32(dp, cur.o[t], vf[sub][t]);
        }
        f32x16 p, ds;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4 b4 = *reinterpret_cast<const f32x4*>(bst + (32 * sub + c) * BLD + 8 * j + 4 * hh);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * j + e;
            const f32x4 st = sst[8 * j + 4 * hh + e];  // {lse2, ref, cen, imax}
            const float pv = __builtin_amdgcn_exp2f(logit2(sa[r], sl2, b4[e], mk2[sub]) - st[0]);
            const float u = (key[sub] == __float_as_int(st[3])) ? 0.f : dp[r] - st[1];
            p[r] = pv;
            ds[r] = pv * (u - st[2]);
          }
        }
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
          M::mma32(dv[sub], cur.ot[t], bfrag_from_acc<TC>(p, t));
          M::mma32(dk[sub], cur.qt[t], bfrag_from_acc<TC>(ds, t));
        }
      }
    }
    if (qt + 1 < nqt) stage_store((qt + 1) & 1);
    __syncthreads();
    cur = nxt;
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
      store_vec<TC, 4>(dK + lo + (size_t)key[sub] * kBD + 8 * j + 4 * hh, vk);
      store_vec<TC, 4>(dV + lo + (size_t)key[sub] * kBD + 8 * j + 4 * hh, vv);
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
};

template <class TC>
__global__ __launch_bounds__(kNT) void attn_bwd_db_kernel(const TC* __restrict__ Q, const TC* __restrict__ K,
                                                          const TC* __restrict__ V, const TC* __restrict__ dO,
                                                          const float* __restrict__ mask2,
                                                          const float* __restrict__ bias2, int S, int H, int N,
                                                          int Np, float scale, int groups,
                                                          const f32x4* __restrict__ st4, float* __restrict__ dbias) {
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
  const int qc = min(q, N - 1);
  const int k0 = blockIdx.y * 64 + (w >> 1) * 32;
  const int kc = min(k0 + c, N - 1);
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
    const size_t lo = line * N * kBD;
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      const int dofs = t * M::K32 + hh * M::KPL;
      op.k[t] = M::load(K + lo + (size_t)kc * kBD + dofs);
      op.q[t] = M::load(Q + lo + (size_t)qc * kBD + dofs);
      op.v[t] = M::load(V + lo + (size_t)kc * kBD + dofs);
      op.o[t] = M::load(dO + lo + (size_t)qc * kBD + dofs);
    }
    op.st = st4[line * Np + q];
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
          const float pv = __builtin_amdgcn_exp2f(logit2(sa[r], sl2, b4[j][e], cur.m[j][e]) - cur.st[0]);
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
  size_t st, bias2, mask2, kt, qt, ot, part, total;
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
                    float* dbias, void* ws, hipStream_t s) {
  const BwdWs lay = bwd_ws_layout(B, S, H, N, (int)sizeof(TC));
  char* base = static_cast<char*>(ws);
  f32x4* st4 = reinterpret_cast<f32x4*>(base + lay.st);
  float* bias2 = reinterpret_cast<float*>(base + lay.bias2);
  float* mask2 = reinterpret_cast<float*>(base + lay.mask2);
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
  attn_bwd_transpose_kernel<TC><<<dim3((unsigned)(Np / 64), lines, 3), 256, 0, s>>>(K, Q, dO, KT, QT, OT, N, Np);
  if (int e = pf::check_launch("attn_bwd_transpose")) return e;
  const unsigned lg = (unsigned)((S + kLines - 1) / kLines);
  attn_bwd_dq_kernel<TC, kSubDq><<<dim3((unsigned)(Np / (32 * kSubDq)), lg, (unsigned)(B * H)), kNT, 0, s>>>(Q, K, V, dO, KT, mask2, bias2, S, H, N, Np, scale, static_cast<TC*>(dq),
                                            st4);
  if (int e = pf::check_launch("attn_bwd_dq")) return e;
  attn_bwd_dkdv_kernel<TC, kSubKv><<<dim3((unsigned)(Np / (32 * kSubKv)), lg, (unsigned)(B * H)), kNT, 0, s>>>(Q, K, V, dO, QT, OT, mask2, bias2, S, H, N, Np, scale, st4,
                                              static_cast<TC*>(dk), static_cast<TC*>(dv));
  if (int e = pf::check_launch("attn_bwd_dkdv")) return e;
  const unsigned nb = (unsigned)((N + 63) / 64);
  const int G = lay.groups;
  float* part = G > 1 ? reinterpret_cast<float*>(base + lay.part) : dbias;
  attn_bwd_db_kernel<TC><<<dim3(nb, nb, (unsigned)(B * H * G)), kNT, 0, s>>>(Q, K, V, dO, mask2, bias2, S, H, N, Np,
                                                                             scale, G, st4, part);
  if (int e = pf::check_launch("attn_bwd_db")) return e;
  if (G > 1) {
    const size_t n = (size_t)B * H * N * N;
    attn_bwd_db_reduce_kernel<<<(unsigned)std::min<size_t>((n + 255) / 256, 4096), 256, 0, s>>>(part, n, G, dbias);
    if (int e = pf::check_launch("attn_bwd_db_reduce")) return e;
  }
  return PF_OK;
}

}  // namespace

extern "C" {

size_t pf_evo_attn_bwd_workspace_bytes(int B, int S, int H, int N, int D, int dtype) {
  if (B <= 0 || S <= 0 || H <= 0 || N <= 0 || D != kBD || (dtype != PF_F32 && dtype != PF_BF16)) return 0;
  return bwd_ws_layout(B, S, H, N, dtype == PF_F32 ? 4 : 2).total;
}

int pf_evo_attn_bwd(const void* q, const void* k, const void* v, const float* res_mask, const float* pair_bias,
                    const void* dout, int B, int S, int H, int N, int D, int dtype, float softmax_scale, void* dq,
                    void* dk, void* dv, float* dpair_bias, void* workspace, size_t workspace_bytes, void* stream) {
  PF_REQUIRE(q && k && v && res_mask && pair_bias && dout && dq && dk && dv && dpair_bias && workspace,
             PF_ERR_INVALID_ARG, "pf_evo_attn_bwd: null pointer");
  PF_REQUIRE(B > 0 && S > 0 && H > 0 && N > 0, PF_ERR_INVALID_ARG, "pf_evo_attn_bwd: B=%d S=%d H=%d N=%d", B, S, H,
             N);
  PF_REQUIRE((long)B * S * H <= 65535 && (long)B * H <= 65535 && (long)N * N < (1L << 31), PF_ERR_INVALID_ARG,
             "pf_evo_attn_bwd: B*S*H=%ld N=%d too large (grid rows are the B*S*H lines)", (long)B * S * H, N);
  PF_REQUIRE(D == kBD, PF_ERR_UNSUPPORTED, "pf_evo_attn_bwd: D=%d (built: D=32)", D);
  PF_REQUIRE(dtype == PF_F32 || dtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_evo_attn_bwd: dtype %d", dtype);
  PF_REQUIRE(pf::aligned16(q) && pf::aligned16(k) && pf::aligned16(v) && pf::aligned16(dout) && pf::aligned16(dq) &&
                 pf::aligned16(dk) && pf::aligned16(dv) && pf::aligned16(workspace),
             PF_ERR_ALIGNMENT, "pf_evo_attn_bwd: operand pointers must be 16-byte aligned");
  const size_t need = bwd_ws_layout(B, S, H, N, dtype == PF_F32 ? 4 : 2).total;
  PF_REQUIRE(workspace_bytes >= need, PF_ERR_WORKSPACE, "pf_evo_attn_bwd: workspace %zu < %zu bytes",
             workspace_bytes, need);
  hipStream_t s = pf::as_stream(stream);
  if (dtype == PF_F32)
    return attn_bwd_launch<float>(q, k, v, res_mask, pair_bias, dout, B, S, H, N, softmax_scale, dq, dk, dv,
                                  dpair_bias, workspace, s);
  return attn_bwd_launch<bf16>(q, k, v, res_mask, pair_bias, dout, B, S, H, N, softmax_scale, dq, dk, dv, dpair_bias,
                               workspace, s);
}

}  // extern "C"
