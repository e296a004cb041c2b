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
// Three kernels, all 32x32 MFMA tiles with D = 32:
//   attn_bwd_dq:   query-major. Pass 1 over the keys builds (LSE, dP_imax, imax, C) per row
//                  online (running max with rescaling and re-centring); pass 2 forms dS and
//                  dQ. The row statistics go to the workspace for the other two kernels.
//   attn_bwd_dkdv: key-major, loops over query tiles: dV^T += dO^T P, dK^T += Q^T dS.
//   attn_bwd_db:   one (query tile, key tile) of one (b, h), loops over the S lines and
//                  sums dS in registers, so the bias gradient needs no atomics and every
//                  output is bit-reproducible.
// Logits are kept in log2 units (x = t log2 e) so P is one v_exp_f32.
#include <climits>

#include "capi.h"
#include "common.h"

namespace {

constexpr int kBD = 32;    // head dimension
constexpr int kTile = 32;  // rows of one wave tile
constexpr int kNT = 256;   // four waves
constexpr int kQBlock = 4 * kTile;
// Zero masked-row rule threshold in log2 units (the reference tests t < -1e8).
constexpr float kDeadLog2 = -1.0e8f * kLog2e;

template <class TC>
constexpr int tile_ld() { return kBD + lds_pad<TC>(); }

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
// product that contracts over its rows: step t of kTile / K32.
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

// Stage rows r0..r0+31 of two [N][32] operands (clamped to N-1) into LDS tiles [32][LD],
// and transposed ([d][row]) into T0 / T1 where given.
template <class TC>
PF_DEVICE void stage_pair(const TC* __restrict__ X0, const TC* __restrict__ X1, int r0, int N, TC* S0, TC* S1,
                          TC* T0, TC* T1) {
  constexpr int LD = tile_ld<TC>();
  constexpr int VEC = 16 / sizeof(TC);
  constexpr int CPR = kBD / VEC;
  constexpr int CHUNKS = kTile * CPR;
  for (int i = threadIdx.x; i < 2 * CHUNKS; i += kNT) {
    const int which = i / CHUNKS;
    const int j = i % CHUNKS;
    const int r = j / CPR;
    const int cc = (j % CPR) * VEC;
    const int row = min(r0 + r, N - 1);
    const u32x4 v = *reinterpret_cast<const u32x4*>((which ? X1 : X0) + (size_t)row * kBD + cc);
    *reinterpret_cast<u32x4*>((which ? S1 : S0) + r * LD + cc) = v;
    TC* T = which ? T1 : T0;
    if (T != nullptr) {
      TC e[VEC];
      __builtin_memcpy(e, &v, 16);
#pragma unroll
      for (int u = 0; u < VEC; ++u) T[(cc + u) * LD + r] = e[u];
    }
  }
}

struct RowStats {
  float lse2, ref, cen;
  int imax;
};

// ------------------------------------------------------------------ dQ (+ row statistics)
template <class TC>
__global__ __launch_bounds__(kNT) void attn_bwd_dq_kernel(const TC* __restrict__ Q, const TC* __restrict__ K,
                                                          const TC* __restrict__ V, const TC* __restrict__ dO,
                                                          const float* __restrict__ res_mask,
                                                          const float* __restrict__ bias, int S, int H, int N, int Ns,
                                                          float scale, TC* __restrict__ dQ, float* __restrict__ st_lse,
                                                          float* __restrict__ st_ref, float* __restrict__ st_cen,
                                                          int* __restrict__ st_imax) {
  using M = Mfma<TC>;
  constexpr int LD = tile_ld<TC>();
  constexpr int STEPS = kBD / M::K32;
  __shared__ __attribute__((aligned(16))) TC Ks[kTile * LD];
  __shared__ __attribute__((aligned(16))) TC Vs[kTile * LD];
  __shared__ __attribute__((aligned(16))) TC KTs[kBD * LD];
  __shared__ float ms[kTile];

  const long line = blockIdx.y;
  const long bs = line / H;
  const int hd = (int)(line % H);
  const int b = (int)(bs / S);
  const size_t lo = (size_t)line * N * kBD;
  const TC *Ql = Q + lo, *Kl = K + lo, *Vl = V + lo, *Ol = dO + lo;
  const float* maskl = res_mask + (size_t)bs * N;
  const float* biasl = bias + ((size_t)b * H + hd) * N * N;

  const int w = wave_id();
  const int l = lane_id();
  const int hh = l >> 5;
  const int c = l & 31;
  const int q = blockIdx.x * kQBlock + w * kTile + c;  // this lane's query (an S^T column)
  const int qc = min(q, N - 1);
  typename M::Frag qf[STEPS], of[STEPS];
#pragma unroll
  for (int t = 0; t < STEPS; ++t) {
    qf[t] = M::load(Ql + (size_t)qc * kBD + t * M::K32 + hh * M::KPL);
    of[t] = M::load(Ol + (size_t)qc * kBD + t * M::K32 + hh * M::KPL);
  }
  const float* brow = biasl + (size_t)qc * N;
  const int nkt = (N + kTile - 1) / kTile;

  // S^T = K Q^T and dP^T = V dO^T for keys k0..k0+31 (rows) x this wave's queries (columns),
  // turned into log2-unit logits x.
  auto tile = [&](int k0, float (&x)[16], f32x16& dp) {
    __syncthreads();
    stage_pair<TC>(Kl, Vl, k0, N, Ks, Vs, KTs, nullptr);
    if (threadIdx.x < kTile) {
      const int key = k0 + threadIdx.x;
      ms[threadIdx.x] = key < N ? maskl[key] : -INFINITY;
    }
    __syncthreads();
    f32x16 s = {};
    dp = f32x16{};
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      M::mma32(s, M::load(Ks + c * LD + t * M::K32 + hh * M::KPL), qf[t]);
      M::mma32(dp, M::load(Vs + c * LD + t * M::K32 + hh * M::KPL), of[t]);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = acc_row(r, hh);
      const int key = k0 + kr;
      const float bv = key < N ? brow[key] : 0.f;
      x[r] = (s[r] * scale + bv + ms[kr]) * kLog2e;
    }
  };

  // Pass 1: running max m, first argmax, dP at it, and per-lane partial sums
  // W = sum exp2(x - m), Cp = sum exp2(x - m) (dP - ref) over this lane's keys.
  float run_max = -INFINITY, refv = 0.f, Wp = 0.f, Cp = 0.f;
  int imx = 0;
  for (int kt = 0; kt < nkt; ++kt) {
    const int k0 = kt * kTile;
    float x[16];
    f32x16 dp;
    tile(k0, x, dp);
    float tmax = x[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) tmax = fmaxf(tmax, x[r]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    int targ = INT_MAX;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (x[r] == tmax) targ = min(targ, k0 + acc_row(r, hh));
    targ = min(targ, __shfl_xor(targ, 32, 64));
    float tref = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (k0 + acc_row(r, hh) == targ) tref = dp[r];
    tref += __shfl_xor(tref, 32, 64);  // exactly one lane of the pair holds it
    const bool better = tmax > run_max;
    const float m_new = better ? tmax : run_max;
    if (m_new != -INFINITY) {
      const float alpha = __builtin_amdgcn_exp2f(run_max - m_new);
      Wp *= alpha;
      Cp *= alpha;
      if (better) {
        Cp += (refv - tref) * Wp;  // re-centre the mass seen so far on the new argmax
        refv = tref;
        imx = targ;
      }
      float ws = 0.f, cs = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = x[r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(x[r] - m_new);
        ws += p;
        cs += p * (dp[r] - refv);
      }
      Wp += ws;
      Cp += cs;
      run_max = m_new;
    }
  }
  const float Wt = Wp + __shfl_xor(Wp, 32, 64);
  const float Ct = Cp + __shfl_xor(Cp, 32, 64);
  const bool dead = !(run_max >= kDeadLog2) || q >= N;
  RowStats st;
  st.lse2 = dead ? INFINITY : run_max + __builtin_amdgcn_logf(Wt);
  st.cen = dead ? 0.f : Ct / Wt;
  st.ref = dead ? 0.f : refv;
  st.imax = dead ? -1 : imx;
  if (hh == 0) {
    const size_t si = (size_t)line * Ns + q;
    st_lse[si] = st.lse2;
    st_ref[si] = st.ref;
    st_cen[si] = st.cen;
    st_imax[si] = st.imax;
  }

  // Pass 2: dS^T and dQ^T [d x q] += K^T [d x keys] dS^T [keys x q].
  f32x16 dq = {};
  for (int kt = 0; kt < nkt; ++kt) {
    const int k0 = kt * kTile;
    float x[16];
    f32x16 dp;
    tile(k0, x, dp);
    f32x16 ds;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = __builtin_amdgcn_exp2f(x[r] - st.lse2);
      const float u = (k0 + acc_row(r, hh) == st.imax) ? 0.f : dp[r] - st.ref;
      ds[r] = p * (u - st.cen);
    }
#pragma unroll
    for (int t = 0; t < STEPS; ++t) M::mma32(dq, afrag_perm<TC>(KTs + c * LD, t, hh), bfrag_from_acc<TC>(ds, t));
  }
  if (q < N) {
    TC* dst = dQ + lo + (size_t)q * kBD;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = dq[4 * j + e] * scale;
      store_vec<TC, 4>(dst + 8 * j + 4 * hh, v);
    }
  }
}

// ------------------------------------------------------------------ dK, dV
template <class TC>
__global__ __launch_bounds__(kNT) void attn_bwd_dkdv_kernel(
    const TC* __restrict__ Q, const TC* __restrict__ K, const TC* __restrict__ V, const TC* __restrict__ dO,
    const float* __restrict__ res_mask, const float* __restrict__ bias, int S, int H, int N, int Ns, float scale,
    const float* __restrict__ st_lse, const float* __restrict__ st_ref, const float* __restrict__ st_cen,
    const int* __restrict__ st_imax, TC* __restrict__ dK, TC* __restrict__ dV) {
  using M = Mfma<TC>;
  constexpr int LD = tile_ld<TC>();
  constexpr int STEPS = kBD / M::K32;
  __shared__ __attribute__((aligned(16))) TC Qs[kTile * LD];
  __shared__ __attribute__((aligned(16))) TC Os[kTile * LD];
  __shared__ __attribute__((aligned(16))) TC QTs[kBD * LD];
  __shared__ __attribute__((aligned(16))) TC OTs[kBD * LD];
  __shared__ __attribute__((aligned(16))) float sl[kTile], sr[kTile], sc[kTile];
  __shared__ __attribute__((aligned(16))) int si[kTile];

  const long line = blockIdx.y;
  const long bs = line / H;
  const int hd = (int)(line % H);
  const int b = (int)(bs / S);
  const size_t lo = (size_t)line * N * kBD;
  const TC *Ql = Q + lo, *Kl = K + lo, *Vl = V + lo, *Ol = dO + lo;
  const float* biasl = bias + ((size_t)b * H + hd) * N * N;
  const size_t so = (size_t)line * Ns;

  const int w = wave_id();
  const int l = lane_id();
  const int hh = l >> 5;
  const int c = l & 31;
  const int key = blockIdx.x * kQBlock + w * kTile + c;  // this lane's key (an S column)
  const int kc = min(key, N - 1);
  typename M::Frag kf[STEPS], vf[STEPS];
#pragma unroll
  for (int t = 0; t < STEPS; ++t) {
    kf[t] = M::load(Kl + (size_t)kc * kBD + t * M::K32 + hh * M::KPL);
    vf[t] = M::load(Vl + (size_t)kc * kBD + t * M::K32 + hh * M::KPL);
  }
  const float mk = key < N ? res_mask[(size_t)bs * N + key] : -INFINITY;
  const int nqt = (N + kTile - 1) / kTile;

  f32x16 dk = {}, dv = {};
  for (int qt = 0; qt < nqt; ++qt) {
    const int q0 = qt * kTile;
    __syncthreads();
    stage_pair<TC>(Ql, Ol, q0, N, Qs, Os, QTs, OTs);
    if (threadIdx.x < kTile) {
      const size_t i = so + q0 + threadIdx.x;
      sl[threadIdx.x] = st_lse[i];
      sr[threadIdx.x] = st_ref[i];
      sc[threadIdx.x] = st_cen[i];
      si[threadIdx.x] = st_imax[i];
    }
    __syncthreads();
    f32x16 s = {}, dp = {};
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      M::mma32(s, M::load(Qs + c * LD + t * M::K32 + hh * M::KPL), kf[t]);
      M::mma32(dp, M::load(Os + c * LD + t * M::K32 + hh * M::KPL), vf[t]);
    }
    f32x16 p, ds;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r0 = 8 * j + 4 * hh;  // rows r0..r0+3 of accumulator group j
      const f32x4 L4 = *reinterpret_cast<const f32x4*>(sl + r0);
      const f32x4 R4 = *reinterpret_cast<const f32x4*>(sr + r0);
      const f32x4 C4 = *reinterpret_cast<const f32x4*>(sc + r0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * j + e;
        const int qg = q0 + r0 + e;
        const float bv = (key < N && qg < N) ? biasl[(size_t)qg * N + key] : 0.f;
        const float x = (s[r] * scale + bv + mk) * kLog2e;
        const float pv = __builtin_amdgcn_exp2f(x - L4[e]);
        const float u = (key == si[r0 + e]) ? 0.f : dp[r] - R4[e];
        p[r] = pv;
        ds[r] = pv * (u - C4[e]);
      }
    }
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      M::mma32(dv, afrag_perm<TC>(OTs + c * LD, t, hh), bfrag_from_acc<TC>(p, t));
      M::mma32(dk, afrag_perm<TC>(QTs + c * LD, t, hh), bfrag_from_acc<TC>(ds, t));
    }
  }
  if (key < N) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float vk[4], vv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vk[e] = dk[4 * j + e] * scale;
        vv[e] = dv[4 * j + e];
      }
      store_vec<TC, 4>(dK + lo + (size_t)key * kBD + 8 * j + 4 * hh, vk);
      store_vec<TC, 4>(dV + lo + (size_t)key * kBD + 8 * j + 4 * hh, vv);
    }
  }
}

// ------------------------------------------------------------------ d_bias
// Block: 64 queries x 64 keys of one (b, h); wave w takes query tile (w & 1) and key tile
// (w >> 1) and sums dS^T over the S lines in its accumulator.
template <class TC>
__global__ __launch_bounds__(kNT) void attn_bwd_db_kernel(
    const TC* __restrict__ Q, const TC* __restrict__ K, const TC* __restrict__ V, const TC* __restrict__ dO,
    const float* __restrict__ res_mask, const float* __restrict__ bias, int S, int H, int N, int Ns, float scale,
    const float* __restrict__ st_lse, const float* __restrict__ st_ref, const float* __restrict__ st_cen,
    const int* __restrict__ st_imax, float* __restrict__ dbias) {
  using M = Mfma<TC>;
  constexpr int STEPS = kBD / M::K32;
  const int bh = blockIdx.z;
  const int b = bh / H;
  const int hd = bh % H;
  const int w = wave_id();
  const int l = lane_id();
  const int hh = l >> 5;
  const int c = l & 31;
  const int q = blockIdx.x * 64 + (w & 1) * kTile + c;
  const int qc = min(q, N - 1);
  const int k0 = blockIdx.y * 64 + (w >> 1) * kTile;
  const int kc = min(k0 + c, N - 1);
  const float* brow = bias + ((size_t)bh * N + qc) * N;
  float bv[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int key = k0 + acc_row(r, hh);
    bv[r] = key < N ? brow[key] : 0.f;
  }
  f32x16 acc = {};
  for (int s = 0; s < S; ++s) {
    const long bs = (long)b * S + s;
    const size_t line = (size_t)bs * H + hd;
    const size_t lo = line * N * kBD;
    f32x16 sa = {}, dp = {};
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      const int dofs = t * M::K32 + hh * M::KPL;
      M::mma32(sa, M::load(K + lo + (size_t)kc * kBD + dofs), M::load(Q + lo + (size_t)qc * kBD + dofs));
      M::mma32(dp, M::load(V + lo + (size_t)kc * kBD + dofs), M::load(dO + lo + (size_t)qc * kBD + dofs));
    }
    const size_t sidx = line * Ns + q;
    const float L2 = st_lse[sidx], Rf = st_ref[sidx], Cn = st_cen[sidx];
    const int im = st_imax[sidx];
    const float* mrow = res_mask + (size_t)bs * N;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k0 + acc_row(r, hh);
      const float mk = key < N ? mrow[key] : -INFINITY;
      const float x = (sa[r] * scale + bv[r] + mk) * kLog2e;
      const float pv = __builtin_amdgcn_exp2f(x - L2);
      const float u = key == im ? 0.f : dp[r] - Rf;
      acc[r] += pv * (u - Cn);
    }
  }
  if (q < N) {
    float* drow = dbias + ((size_t)bh * N + q) * N;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k0 + acc_row(r, hh);
      if (key < N) drow[key] = acc[r];
    }
  }
}

struct BwdWs {
  size_t lse, ref, cen, imax, total;
};

BwdWs bwd_ws_layout(int B, int S, int H, int N) {
  const size_t rows = (size_t)B * S * H * pf::pad128(N);
  BwdWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = pf::round_up(off + bytes, 256);
    return o;
  };
  w.lse = take(rows * 4);
  w.ref = take(rows * 4);
  w.cen = take(rows * 4);
  w.imax = take(rows * 4);
  w.total = off;
  return w;
}

template <class TC>
int attn_bwd_launch(const void* q, const void* k, const void* v, const float* res_mask, const float* pair_bias,
                    const void* dout, int B, int S, int H, int N, float scale, void* dq, void* dk, void* dv,
                    float* dbias, void* ws, hipStream_t s) {
  const BwdWs lay = bwd_ws_layout(B, S, H, N);
  char* base = static_cast<char*>(ws);
  float* lse = reinterpret_cast<float*>(base + lay.lse);
  float* ref = reinterpret_cast<float*>(base + lay.ref);
  float* cen = reinterpret_cast<float*>(base + lay.cen);
  int* imx = reinterpret_cast<int*>(base + lay.imax);
  const int Ns = pf::pad128(N);
  const unsigned lines = (unsigned)((long)B * S * H);
  const TC *Q = static_cast<const TC*>(q), *K = static_cast<const TC*>(k), *V = static_cast<const TC*>(v),
           *dO = static_cast<const TC*>(dout);
  const dim3 g1((unsigned)(Ns / kQBlock), lines);
  attn_bwd_dq_kernel<TC><<<g1, kNT, 0, s>>>(Q, K, V, dO, res_mask, pair_bias, S, H, N, Ns, scale,
                                             static_cast<TC*>(dq), lse, ref, cen, imx);
  if (int e = pf::check_launch("attn_bwd_dq")) return e;
  attn_bwd_dkdv_kernel<TC><<<g1, kNT, 0, s>>>(Q, K, V, dO, res_mask, pair_bias, S, H, N, Ns, scale, lse, ref, cen,
                                               imx, static_cast<TC*>(dk), static_cast<TC*>(dv));
  if (int e = pf::check_launch("attn_bwd_dkdv")) return e;
  const unsigned nb = (unsigned)((N + 63) / 64);
  attn_bwd_db_kernel<TC><<<dim3(nb, nb, (unsigned)(B * H)), kNT, 0, s>>>(Q, K, V, dO, res_mask, pair_bias, S, H, N,
                                                                         Ns, scale, lse, ref, cen, imx, dbias);
  return pf::check_launch("attn_bwd_db");
}

}  // namespace

extern "C" {

size_t pf_evo_attn_bwd_workspace_bytes(int B, int S, int H, int N, int D, int dtype) {
  if (B <= 0 || S <= 0 || H <= 0 || N <= 0 || D != kBD || (dtype != PF_F32 && dtype != PF_BF16)) return 0;
  return bwd_ws_layout(B, S, H, N).total;
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
  const size_t need = bwd_ws_layout(B, S, H, N).total;
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
