// Triangle attention (GridSelfAttention, starting and ending node) in three launches:
//
//   A1 attn_project:  x = LN(z); q, k, v, g = x W{q,k,v,g}^T; pb = x Wpb^T. Writes the
//                     attention-frame operands Q, K (token-major), Vt (key-contiguous,
//                     keys permuted inside 32-blocks), G = sigmoid(g), the pair bias PB and
//                     the additive key mask MA (both pre-multiplied by log2 e).
//   A2 tri_attn:      flash attention over keys with an online base-2 softmax; the
//                     N^3*H logits never leave registers. Writes O (normalised, ungated).
//   A3 attn_out:      out = (O * G) Wout^T, written to `out` or added into it (residual),
//                     transposed back for the ending-node (column) direction.
//
// Reference semantics: GridSelfAttention._compute_baseline / forward
// (src/deepfold3/model/attention.py:143-269): head_dim = max(C/H, 16) (:67), the pair bias
// comes from the un-transposed LN(z) (:204-209), logits = q k^T * d^-1/2 + pb + 1e9 (mask - 1)
// (:151-158) and softmax runs in fp32 (:160). A fully masked line therefore attends uniformly
// over all N keys (output = mean of V), which this kernel reproduces exactly: the additive
// -1e9 * log2(e) term swamps every logit by the same amount.
//
// Frames. "line" is the attention row: i for the starting node (row mode), j for the
// ending node (column mode). Keys and queries run along the other token index. The
// projection kernel walks z along a line in both modes (column mode reads z down a column),
// so every operand is written contiguously in the attention frame.
//
// MFMA layout (v_mfma_f32_32x32x16_bf16 / v_mfma_f32_32x32x2f32). A wave owns 32 queries
// per sub-block and computes S^T = K Q^T (keys are accumulator rows), so lane (q, h)
// (q = lane & 31, h = lane >> 5) holds the logits of query q for keys
// kappa(r, h) = 8 (r >> 2) + 4 h + (r & 3), r = 0..15. Those 16 probabilities are exactly
// the B operand lane (q, h) must supply for O^T += V^T P^T when the keys of a 32-block are
// stored in the order kappa (storage slot 16 h + r holds key kappa(r, h)): Vt, PB (row
// mode) and MA are written in that order, so P never goes through LDS.
#include "capi.h"
#include "common.h"

namespace {

constexpr int kHeads = 4;
constexpr int kHeadDim = 32;
constexpr int kC = 128;

// Storage slot -> key inside a 32-key block, and its inverse.
PF_DEVICE int slot_key(int slot) { return 8 * ((slot & 15) >> 2) + 4 * (slot >> 4) + (slot & 3); }
PF_DEVICE int key_slot(int key) { return 16 * ((key >> 2) & 1) + 4 * (key >> 3) + (key & 3); }

template <class TC>
constexpr int proj_bm() { return sizeof(TC) == 2 ? 64 : 32; }

// ------------------------------------------------------------------ A1
// w5 [4C + 16][C] (cdtype): rows q | k | v | g | pb (H rows) | zero padding.
template <class TZ, class TC>
struct ProjCfg {
  static constexpr int BM = proj_bm<TC>();
  static constexpr int ALD = kC + lds_pad<TC>();
  static constexpr int SLD = kC + lds_pad<TC>();
  static constexpr int A_BYTES = BM * ALD * (int)sizeof(TC);
  static constexpr int S_BYTES = 4 * BM * SLD * (int)sizeof(TC);
  static constexpr int SMEM = A_BYTES > S_BYTES ? A_BYTES : S_BYTES;
};

template <class TZ, class TC>
__global__ __launch_bounds__(256) void attn_project_kernel(const TZ* __restrict__ z, const float* __restrict__ mask,
                                                           const float* __restrict__ lnw, const float* __restrict__ lnb,
                                                           float eps, const TC* __restrict__ w5, TC* __restrict__ Q,
                                                           TC* __restrict__ K, TC* __restrict__ Vt,
                                                           TC* __restrict__ G, float* __restrict__ PB,
                                                           float* __restrict__ MA, int N, int Np, int transpose,
                                                           float qscale) {
  using Cfg = ProjCfg<TZ, TC>;
  constexpr int BM = Cfg::BM, ALD = Cfg::ALD, SLD = Cfg::SLD;
  constexpr int NT = 256;
  constexpr int RB = BM / 16;
  constexpr int VEC = 16 / sizeof(TC);
  __shared__ __attribute__((aligned(16))) char smem[Cfg::SMEM];
  __shared__ float pbs[BM][kHeads];
  __shared__ float mks[BM];
  TC* A = reinterpret_cast<TC*>(smem);

  const int t0 = blockIdx.x * BM;
  const int line = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const TZ* zb = z + (size_t)b * N * N * kC;
  auto pos_of = [&](int p) -> long {
    const int t = t0 + p;
    if (line >= N || t >= N) return -1;
    return transpose ? (long)t * N + line : (long)line * N + t;
  };
  auto rowptr = [&](int p) -> const TZ* {
    const long pos = pos_of(p);
    return pos < 0 ? nullptr : zb + pos * kC;
  };
  ln_tile_to_lds<TZ, TC, kC, BM, NT>(rowptr, lnw, lnb, eps, A, ALD);
  if (tid < BM) {
    const long pos = pos_of(tid);
    mks[tid] = pos < 0 ? 0.f : mask[(size_t)b * N * N + pos];
  }
  __syncthreads();

  // Wave w computes kind w (q, k, v, g) for all BM rows; the pair-bias block is split by
  // row blocks over the waves.
  f32x4 acc[RB][8];
  zero_acc(acc);
  int wrow0[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) wrow0[j] = w * kC + j * 16;
  gemm16_lds_x_w<TC, kC, RB, 8>(acc, A, ALD, 0, w5, kC, wrow0);
  f32x4 accb[1][1];
  zero_acc(accb);
  const bool has_pb_rows = w < RB;
  if (has_pb_rows) {
    int prow[1] = {4 * kC};
    gemm16_lds_x_w<TC, kC, 1, 1>(accb, A, ALD, w * 16, w5, kC, prow);
  }
  __syncthreads();  // A is dead: reuse as four per-kind stage tiles S[w] [BM][SLD]

  TC* S = reinterpret_cast<TC*>(smem) + w * BM * SLD;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int p = rb * 16 + 4 * (l >> 4) + e;
        const int c = j * 16 + (l & 15);
        float v = acc[rb][j][e];
        if (w == 0) v *= qscale;
        if (w == 3) v = sigmoidf_(v);
        S[p * SLD + c] = from_f32<TC>(v);
      }
  if (has_pb_rows && (l & 15) < kHeads) {
#pragma unroll
    for (int e = 0; e < 4; ++e) pbs[w * 16 + 4 * (l >> 4) + e][l & 15] = accb[0][0][e] * kLog2e;
  }
  __syncthreads();

  const size_t lineq = (size_t)b * Np + line;  // [b][line] index over the padded frame
  const bool line_ok = line < N;
  if (w <= 1) {
    // Q / K: [b][line][h][t][d]; per head BM x D contiguous.
    TC* dst = (w == 0 ? Q : K) + lineq * kHeads * Np * kHeadDim;
    constexpr int CPH = BM * kHeadDim / VEC;  // chunks per head
    for (int idx = l; idx < kHeads * CPH; idx += 64) {
      const int hh = idx / CPH;
      const int r = idx % CPH;
      const int p = r / (kHeadDim / VEC);
      const int d0 = (r % (kHeadDim / VEC)) * VEC;
      u32x4 v = *reinterpret_cast<const u32x4*>(S + p * SLD + hh * kHeadDim + d0);
      if (!line_ok || t0 + p >= N) v = u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(dst + ((size_t)hh * Np + t0 + p) * kHeadDim + d0) = v;
    }
  } else if (w == 2) {
    // Vt: [b][line][h][d][slot], keys permuted inside each 32-block.
    TC* dst = Vt + lineq * kHeads * kHeadDim * Np;
    constexpr int CPR = BM / VEC;  // chunks per (h, d) row
    for (int idx = l; idx < kC * CPR; idx += 64) {
      const int c = idx / CPR;
      const int s0 = (idx % CPR) * VEC;  // slot offset inside the tile (tile is 32-aligned)
      float v[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const int s = s0 + e;
        const int p = (s & ~31) + slot_key(s & 31);
        v[e] = (line_ok && t0 + p < N) ? to_f32(S[p * SLD + c]) : 0.f;
      }
      store_vec<TC, VEC>(dst + (size_t)c * Np + t0 + s0, v);
    }
  } else {
    // G = sigmoid(g): [b][line][t][C]
    TC* dst = G + lineq * Np * kC;
    constexpr int CPR = kC / VEC;
    for (int idx = l; idx < BM * CPR; idx += 64) {
      const int p = idx / CPR;
      const int c0 = (idx % CPR) * VEC;
      *reinterpret_cast<u32x4*>(dst + (size_t)(t0 + p) * kC + c0) =
          *reinterpret_cast<const u32x4*>(S + p * SLD + c0);
    }
  }
  // Pair bias and key mask (tiny): one thread per (head, position).
  for (int idx = tid; idx < kHeads * BM; idx += NT) {
    const int hh = idx / BM;
    const int p = idx % BM;
    const int t = t0 + p;
    const bool ok = line_ok && t < N;
    const float v = ok ? pbs[p][hh] : 0.f;
    if (transpose) {
      // key-major [b][h][key = line][query = t]
      PB[(((size_t)b * kHeads + hh) * Np + line) * Np + t] = v;
    } else {
      // query-major [b][h][query = line][slot(key = t)]
      PB[(((size_t)b * kHeads + hh) * Np + line) * Np + (t & ~31) + key_slot(t & 31)] = v;
    }
  }
  if (tid < BM) {
    const int t = t0 + tid;
    const float m = mks[tid];
    const float v = t < N ? (m - 1.0f) * 1e9f * kLog2e : -INFINITY;
    MA[lineq * Np + (t & ~31) + key_slot(t & 31)] = v;
  }
}

// ------------------------------------------------------------------ A2
// 16 operand values per lane (bf16: 32 bytes; fp32: 64 bytes).
template <class TC>
struct Frag16;
template <>
struct Frag16<bf16> {
  bf16x8 v[2];
  PF_DEVICE void load(const bf16* p) {
    v[0] = *reinterpret_cast<const bf16x8*>(p);
    v[1] = *reinterpret_cast<const bf16x8*>(p + 8);
  }
};
template <>
struct Frag16<float> {
  f32x4 v[4];
  PF_DEVICE void load(const float* p) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = *reinterpret_cast<const f32x4*>(p + 4 * i);
  }
};

// acc += A B over the 16 k values the two lane halves hold (bf16: 2 MFMAs, fp32: 16).
PF_DEVICE void mma32_16(f32x16& acc, const Frag16<bf16>& a, const Frag16<bf16>& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.v[0], b.v[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.v[1], b.v[1], acc, 0, 0, 0);
}
PF_DEVICE void mma32_16(f32x16& acc, const Frag16<float>& a, const Frag16<float>& b) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.v[i][e], b.v[i][e], acc, 0, 0, 0);
}

// P^T as a B operand from 16 fp32 probabilities.
PF_DEVICE Frag16<bf16> pack_p(const float (&p)[16], bf16) {
  Frag16<bf16> f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    f.v[0][e] = (bf16)p[e];
    f.v[1][e] = (bf16)p[8 + e];
  }
  return f;
}
PF_DEVICE Frag16<float> pack_p(const float (&p)[16], float) {
  Frag16<float> f;
#pragma unroll
  for (int i = 0; i < 4; ++i) f.v[i] = f32x4{p[4 * i], p[4 * i + 1], p[4 * i + 2], p[4 * i + 3]};
  return f;
}

constexpr int kQSub = 2;                 // 32-query sub-blocks per wave
constexpr int kQBlock = 32 * kQSub;      // queries per wave
constexpr int kLinesPerBlock = 4;        // one line per wave

template <class TC, bool BIAS_KEY_MAJOR>
__global__ __launch_bounds__(256, 2) void tri_attn_kernel(const TC* __restrict__ Q, const TC* __restrict__ K,
                                                          const TC* __restrict__ Vt, const float* __restrict__ PB,
                                                          const float* __restrict__ MA, TC* __restrict__ O, int B,
                                                          int N, int Np, int xcd_remap) {
  const int nqb = Np / kQBlock;
  const int nlg = (N + kLinesPerBlock - 1) / kLinesPerBlock;
  const int total = B * nlg * kHeads * nqb;
  int bid = blockIdx.x;
  if (xcd_remap) bid = (bid & 7) * (total >> 3) + (bid >> 3);
  // task order: q-block fastest, then line group, then head, then batch, so that one XCD
  // walks all q-blocks of a line group (K/V reuse) and many line groups of one head (bias reuse)
  const int qb = bid % nqb;
  int rest = bid / nqb;
  const int lg = rest % nlg;
  rest /= nlg;
  const int h = rest % kHeads;
  const int b = rest / kHeads;
  const int w = wave_id();
  const int l = lane_id();
  const int line = lg * kLinesPerBlock + w;
  if (b >= B || line >= N) return;

  const int lq = l & 31;
  const int hf = l >> 5;
  const size_t lineq = (size_t)b * Np + line;
  const TC* Qh = Q + (lineq * kHeads + h) * (size_t)Np * kHeadDim;
  const TC* Kh = K + (lineq * kHeads + h) * (size_t)Np * kHeadDim;
  const TC* Vh = Vt + (lineq * kHeads + h) * (size_t)kHeadDim * Np;
  const float* PBh = PB + ((size_t)b * kHeads + h) * (size_t)Np * Np;
  const float* MAl = MA + lineq * Np;
  const int q0 = qb * kQBlock;

  Frag16<TC> qf[kQSub];
#pragma unroll
  for (int s = 0; s < kQSub; ++s) qf[s].load(Qh + (size_t)(q0 + 32 * s + lq) * kHeadDim + 16 * hf);

  // Does this line mask any real key? (wave-uniform)
  bool masked = false;
  for (int k = l; k < N; k += 64) masked |= MAl[(k & ~31) + key_slot(k & 31)] != 0.f;
  masked = __any(masked);

  f32x16 o[kQSub];
  float mrun[kQSub], lrun[kQSub];
#pragma unroll
  for (int s = 0; s < kQSub; ++s) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[s][r] = 0.f;
    mrun[s] = -INFINITY;
    lrun[s] = 0.f;
  }

  const int nkb = (N + 31) / 32;
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * 32;
    Frag16<TC> kf, vf;
    kf.load(Kh + (size_t)(k0 + lq) * kHeadDim + 16 * hf);
    vf.load(Vh + (size_t)lq * Np + k0 + 16 * hf);
    float madd[16];
    if (masked) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 mv = *reinterpret_cast<const f32x4*>(MAl + k0 + 16 * hf + 4 * i);
        madd[4 * i] = mv[0]; madd[4 * i + 1] = mv[1]; madd[4 * i + 2] = mv[2]; madd[4 * i + 3] = mv[3];
      }
    } else if (k0 + 32 > N) {
      // padding keys of the last block still need -inf
#pragma unroll
      for (int r = 0; r < 16; ++r) madd[r] = (k0 + 8 * (r >> 2) + 4 * hf + (r & 3)) < N ? 0.f : -INFINITY;
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) madd[r] = 0.f;
    }
#pragma unroll
    for (int s = 0; s < kQSub; ++s) {
      const int q = q0 + 32 * s + lq;
      f32x16 sacc;
      if (BIAS_KEY_MAJOR) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] = PBh[(size_t)(k0 + 8 * (r >> 2) + 4 * hf + (r & 3)) * Np + q] + madd[r];
      } else {
        const float* pr = PBh + (size_t)q * Np + k0 + 16 * hf;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f32x4 bv = *reinterpret_cast<const f32x4*>(pr + 4 * i);
          sacc[4 * i] = bv[0] + madd[4 * i];
          sacc[4 * i + 1] = bv[1] + madd[4 * i + 1];
          sacc[4 * i + 2] = bv[2] + madd[4 * i + 2];
          sacc[4 * i + 3] = bv[3] + madd[4 * i + 3];
        }
      }
      mma32_16(sacc, kf, qf[s]);
      float mx = sacc[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sacc[r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(mrun[s], mx);
      const float alpha = __builtin_amdgcn_exp2f(mrun[s] - mnew);
      mrun[s] = mnew;
      float p[16];
      float ls = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = __builtin_amdgcn_exp2f(sacc[r] - mnew);
        ls += p[r];
      }
      lrun[s] = lrun[s] * alpha + ls;
#pragma unroll
      for (int r = 0; r < 16; ++r) o[s][r] *= alpha;
      mma32_16(o[s], vf, pack_p(p, TC{}));
    }
  }

  // O^T lane (q, hf) holds d = 8 (r >> 2) + 4 hf + (r & 3).
  TC* Ol = O + lineq * (size_t)Np * kC;
#pragma unroll
  for (int s = 0; s < kQSub; ++s) {
    const float lt = lrun[s] + __shfl_xor(lrun[s], 32, 64);
    const float inv = 1.0f / lt;
    const int q = q0 + 32 * s + lq;
    if (q >= N) continue;
    TC* dst = Ol + (size_t)q * kC + h * kHeadDim;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = o[s][4 * j + e] * inv;
      store_vec<TC, 4>(dst + 8 * j + 4 * hf, v);
    }
  }
}

// ------------------------------------------------------------------ A3
template <class TZ, class TC>
struct OutCfg {
  static constexpr int BM = proj_bm<TC>();
  static constexpr int ALD = kC + lds_pad<TC>();
  static constexpr int SLD = kC + 4;
  static constexpr int A_BYTES = BM * ALD * (int)sizeof(TC);
  static constexpr int S_BYTES = BM * SLD * 4;
  static constexpr int SMEM = A_BYTES > S_BYTES ? A_BYTES : S_BYTES;
};

template <class TZ, class TC>
__global__ __launch_bounds__(256) void attn_out_kernel(const TC* __restrict__ O, const TC* __restrict__ G,
                                                       const TC* __restrict__ Wo, TZ* __restrict__ out, int N, int Np,
                                                       int transpose, int accumulate) {
  using Cfg = OutCfg<TZ, TC>;
  constexpr int BM = Cfg::BM, ALD = Cfg::ALD, SLD = Cfg::SLD;
  constexpr int NT = 256;
  constexpr int RB = BM / 16;
  constexpr int CBW = kC / 16 / 4;
  constexpr int VEC = 16 / sizeof(TC);
  __shared__ __attribute__((aligned(16))) char smem[Cfg::SMEM];
  TC* A = reinterpret_cast<TC*>(smem);
  float* stage = reinterpret_cast<float*>(smem);

  const int t0 = blockIdx.x * BM;
  const int line = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const size_t lineq = (size_t)b * Np + line;
  {
    const TC* Ol = O + (lineq * Np + t0) * kC;
    const TC* Gl = G + (lineq * Np + t0) * kC;
    constexpr int CPR = kC / VEC;
    for (int idx = tid; idx < BM * CPR; idx += NT) {
      const int p = idx / CPR;
      const int c0 = (idx % CPR) * VEC;
      float ov[VEC], gv[VEC], y[VEC];
      if (t0 + p < N) {
        load16<TC>(Ol + (size_t)p * kC + c0, ov);
        load16<TC>(Gl + (size_t)p * kC + c0, gv);
#pragma unroll
        for (int e = 0; e < VEC; ++e) y[e] = ov[e] * gv[e];
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) y[e] = 0.f;
      }
      store_vec<TC, VEC>(A + p * ALD + c0, y);
    }
  }
  __syncthreads();
  const int w = wave_id();
  const int l = lane_id();
  f32x4 acc[RB][CBW];
  zero_acc(acc);
  int wrow0[CBW];
#pragma unroll
  for (int j = 0; j < CBW; ++j) wrow0[j] = (w * CBW + j) * 16;
  gemm16_lds_x_w<TC, kC, RB, CBW>(acc, A, ALD, 0, Wo, kC, wrow0);
  __syncthreads();
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < CBW; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        stage[(rb * 16 + 4 * (l >> 4) + e) * SLD + (w * CBW + j) * 16 + (l & 15)] = acc[rb][j][e];
  __syncthreads();
  TZ* ob = out + (size_t)b * N * N * kC;
  auto orow = [&](int p) -> TZ* {
    const int t = t0 + p;
    if (t >= N) return nullptr;
    return ob + (transpose ? (size_t)t * N + line : (size_t)line * N + t) * kC;
  };
  store_tile_from_lds<TZ, kC, BM, NT>(orow, stage, SLD, accumulate != 0);
}

// Offsets of the operand buffers inside the workspace (bytes, 256-aligned).
struct AttnWs {
  size_t q, k, v, g, o, pb, ma, total;
};

AttnWs attn_ws_layout(int B, int N, int cdtype) {
  const size_t Np = (size_t)pf::round_up((size_t)N, kQBlock);
  const size_t es = cdtype == PF_F32 ? 4 : 2;
  const size_t tok = (size_t)B * Np * Np * kC * es;  // one [B][Np][Np][C] operand
  AttnWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += pf::round_up(bytes, 256);
    return at;
  };
  w.q = take(tok);
  w.k = take(tok);
  w.v = take(tok);
  w.g = take(tok);
  w.o = take(tok);
  w.pb = take((size_t)B * kHeads * Np * Np * 4);
  w.ma = take((size_t)B * Np * Np * 4);
  w.total = off;
  return w;
}

template <class TZ, class TC>
int grid_attn_launch(const void* z, const float* mask, const float* lnw, const float* lnb, float eps, const void* w5,
                     const void* wo, int B, int N, int transpose, void* out, int accumulate, void* ws, hipStream_t s) {
  const int Np = (int)pf::round_up((size_t)N, kQBlock);
  const AttnWs L = attn_ws_layout(B, N, sizeof(TC) == 4 ? PF_F32 : PF_BF16);
  char* base = reinterpret_cast<char*>(ws);
  TC* Qb = reinterpret_cast<TC*>(base + L.q);
  TC* Kb = reinterpret_cast<TC*>(base + L.k);
  TC* Vb = reinterpret_cast<TC*>(base + L.v);
  TC* Gb = reinterpret_cast<TC*>(base + L.g);
  TC* Ob = reinterpret_cast<TC*>(base + L.o);
  float* PBb = reinterpret_cast<float*>(base + L.pb);
  float* MAb = reinterpret_cast<float*>(base + L.ma);
  const float qscale = (1.0f / sqrtf((float)kHeadDim)) * kLog2e;
  {
    constexpr int BM = proj_bm<TC>();
    dim3 grid(Np / BM, Np, B);
    pf::KernelTimer timer_attn_project("attn_project", s);
    attn_project_kernel<TZ, TC><<<grid, 256, 0, s>>>((const TZ*)z, mask, lnw, lnb, eps, (const TC*)w5, Qb, Kb, Vb,
                                                     Gb, PBb, MAb, N, Np, transpose, qscale);
    timer_attn_project.stop();
    if (int e = pf::check_launch("attn_project")) return e;
  }
  {
    const int nqb = Np / kQBlock;
    const int nlg = (N + kLinesPerBlock - 1) / kLinesPerBlock;
    const long total = (long)B * nlg * kHeads * nqb;
    const int remap = (total % 8 == 0) ? 1 : 0;
    dim3 grid((unsigned)total);
    pf::KernelTimer timer("tri_attn", s);
    if (transpose)
      tri_attn_kernel<TC, true><<<grid, 256, 0, s>>>(Qb, Kb, Vb, PBb, MAb, Ob, B, N, Np, remap);
    else
      tri_attn_kernel<TC, false><<<grid, 256, 0, s>>>(Qb, Kb, Vb, PBb, MAb, Ob, B, N, Np, remap);
    timer.stop();
    if (int e = pf::check_launch("tri_attn")) return e;
  }
  {
    constexpr int BM = proj_bm<TC>();
    dim3 grid((N + BM - 1) / BM, N, B);
    pf::KernelTimer timer_attn_out("attn_out", s);
    attn_out_kernel<TZ, TC><<<grid, 256, 0, s>>>(Ob, Gb, (const TC*)wo, (TZ*)out, N, Np, transpose, accumulate);
    timer_attn_out.stop();
    if (int e = pf::check_launch("attn_out")) return e;
  }
  return pf::ok();
}

}  // namespace

extern "C" {

size_t pf_grid_attn_workspace_bytes(int B, int N, int C, int H, int cdtype) {
  if (B <= 0 || N <= 0 || C != kC || H != kHeads) return 0;
  return attn_ws_layout(B, N, cdtype).total;
}

int pf_grid_attn_fwd(const void* z, const float* mask, const float* ln_w, const float* ln_b, float eps,
                     const void* w_qkvgb, const void* w_out, int B, int N, int C, int H, int transpose, int zdtype,
                     int cdtype, void* out, int accumulate, void* workspace, size_t workspace_bytes, void* stream) {
  PF_REQUIRE(z && mask && ln_w && ln_b && w_qkvgb && w_out && out && workspace, PF_ERR_INVALID_ARG,
             "pf_grid_attn_fwd: null pointer");
  PF_REQUIRE(B > 0 && N > 0, PF_ERR_INVALID_ARG, "pf_grid_attn_fwd: B=%d N=%d", B, N);
  PF_REQUIRE(C == kC && H == kHeads, PF_ERR_UNSUPPORTED, "pf_grid_attn_fwd: C=%d H=%d (built: C=128, H=4, d=32)", C,
             H);
  PF_REQUIRE(zdtype == PF_F32 || zdtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_grid_attn_fwd: zdtype %d", zdtype);
  PF_REQUIRE(cdtype == PF_F32 || cdtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_grid_attn_fwd: cdtype %d", cdtype);
  PF_REQUIRE(!(zdtype == PF_BF16 && cdtype == PF_F32), PF_ERR_UNSUPPORTED,
             "pf_grid_attn_fwd: bf16 activations with fp32 GEMMs is not a supported regime");
  PF_REQUIRE(pf::aligned16(z) && pf::aligned16(out) && pf::aligned16(workspace) && pf::aligned16(w_qkvgb) &&
                 pf::aligned16(w_out),
             PF_ERR_ALIGNMENT, "pf_grid_attn_fwd: pointers must be 16-byte aligned");
  PF_REQUIRE(workspace_bytes >= attn_ws_layout(B, N, cdtype).total, PF_ERR_WORKSPACE,
             "pf_grid_attn_fwd: workspace %zu < %zu bytes", workspace_bytes, attn_ws_layout(B, N, cdtype).total);
  hipStream_t s = pf::as_stream(stream);
  if (zdtype == PF_F32 && cdtype == PF_F32)
    return grid_attn_launch<float, float>(z, mask, ln_w, ln_b, eps, w_qkvgb, w_out, B, N, transpose, out, accumulate,
                                          workspace, s);
  if (zdtype == PF_F32)
    return grid_attn_launch<float, bf16>(z, mask, ln_w, ln_b, eps, w_qkvgb, w_out, B, N, transpose, out, accumulate,
                                         workspace, s);
  return grid_attn_launch<bf16, bf16>(z, mask, ln_w, ln_b, eps, w_qkvgb, w_out, B, N, transpose, out, accumulate,
                                      workspace, s);
}

}  // extern "C"
