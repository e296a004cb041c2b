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
// so every operand is written contiguously in the attention frame. The pair bias is
// stored query-major [h][q][key slot] in row mode and key-major [h][key][q] in column mode
// (again the order in which the projection produces it); the attention kernel stages it
// through LDS either way.
//
// MFMA layout (v_mfma_f32_32x32x16_bf16 / v_mfma_f32_32x32x2f32). A wave owns 32 queries
// per sub-block and computes S^T = K Q^T (keys are accumulator rows), so lane (q, h)
// (q = lane & 31, h = lane >> 5) holds the logits of query q for keys
// kappa(r, h) = 8 (r >> 2) + 4 h + (r & 3), r = 0..15. Those 16 probabilities are exactly
// the B operand lane (q, h) must supply for O^T += V^T P^T when the keys of a 32-block are
// stored in the order kappa (storage slot 16 h + r holds key kappa(r, h)): Vt, PB and MA
// use that order, so P never goes through LDS.
#include "capi.h"
#include "common.h"

namespace {

constexpr int kHeads = 4;
constexpr int kHeadDim = 32;
constexpr int kC = 128;
constexpr int kPad = 128;  // token padding of the attention frame
#ifndef PF_ATTN_QS
#define PF_ATTN_QS 2
#endif

// Storage slot -> key inside a 32-key block, and its inverse.
PF_DEVICE int slot_key(int slot) { return 8 * ((slot & 15) >> 2) + 4 * (slot >> 4) + (slot & 3); }
PF_DEVICE int key_slot(int key) { return 16 * ((key >> 2) & 1) + 4 * (key >> 3) + (key & 3); }

// ------------------------------------------------------------------ A1
// w5 [4C + 16][C] (cdtype): rows q | k | v | g | pb (H rows) | zero padding.
// Block: BM positions of one line; 4 waves in 2 x 2 (positions x channels), each 32x32
// MFMA tiles. The four 128-row weight chunks go through one LDS buffer, which doubles as
// the staging tile for the chunk's output.
template <class TZ, class TC>
__global__ __launch_bounds__(256) void attn_project_kernel(const TZ* __restrict__ z, const float* __restrict__ mask,
                                                           const float* __restrict__ lnw, const float* __restrict__ lnb,
                                                           float eps, const TC* __restrict__ w5, TC* __restrict__ Q,
                                                           TC* __restrict__ K, TC* __restrict__ Vt,
                                                           TC* __restrict__ G, float* __restrict__ PB,
                                                           float* __restrict__ MA, int N, int Np, int transpose,
                                                           float qscale) {
  constexpr int BM = block_rows<TC>();
  constexpr int LD = ld128<TC>();
  constexpr int NT = 256;
  constexpr int WM = BM / 2;  // positions per wave
  constexpr int PT = WM / 32;
  constexpr int VEC = 16 / sizeof(TC);
  __shared__ __attribute__((aligned(16))) TC X[BM * LD];
  __shared__ __attribute__((aligned(16))) TC WS[128 * LD];
  __shared__ float pbs[BM][kHeads];
  __shared__ float mks[BM];

  const int t0 = blockIdx.x * BM;
  const int line = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const int wr = w >> 1, wc = w & 1;
  const TZ* zb = z + (size_t)b * N * N * kC;
  auto pos_of = [&](int p) -> long {
    const int t = t0 + p;
    if (line >= N || t >= N) return -1;
    return transpose ? (long)t * N + line : (long)line * N + t;
  };
  Rows128<TC, 128, NT> wpf;
  wpf.load(w5, kC);
  ln_tile_to_lds<TZ, TC, kC, BM, NT>([&](int p) -> const TZ* {
    const long pos = pos_of(p);
    return pos < 0 ? nullptr : zb + pos * kC;
  }, lnw, lnb, eps, X, LD);
  if (tid < BM) {
    const long pos = pos_of(tid);
    mks[tid] = pos < 0 ? 0.f : mask[(size_t)b * N * N + pos];
  }
  const size_t lineq = (size_t)b * Np + line;  // [b][line] over the padded frame

#pragma unroll 1
  for (int kind = 0; kind < 4; ++kind) {
    __syncthreads();  // previous chunk's stage fully consumed
    wpf.store(WS, LD);
    __syncthreads();
    if (kind < 3) wpf.load(w5 + (size_t)(kind + 1) * 128 * kC, kC);
    if (kind != 2) {
      // position-major output: acc^T = W X^T, lane holds 4 consecutive channels
      f32x16 acc[2][PT];
      zero_acc32(acc);
      wave_mma32<TC, 2, PT, kC>(acc, WS, LD, wc * 64, X, LD, wr * WM);
      __syncthreads();  // WS becomes the stage [pos][ch]
#pragma unroll
      for (int ci = 0; ci < 2; ++ci)
#pragma unroll
        for (int pj = 0; pj < PT; ++pj)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float x = acc[ci][pj][4 * g4 + e];
              if (kind == 0) x *= qscale;
              if (kind == 3) x = sigmoidf_(x);
              v[e] = x;
            }
            const int ch = wc * 64 + 32 * ci + acc32_row(4 * g4);
            const int p = wr * WM + 32 * pj + (l & 31);
            store_vec<TC, 4>(WS + p * LD + ch, v);
          }
    } else {
      // channel-major output (Vt): acc = X W^T, lane holds 4 consecutive positions
      f32x16 acc[PT][2];
      zero_acc32(acc);
      wave_mma32<TC, PT, 2, kC>(acc, X, LD, wr * WM, WS, LD, wc * 64);
      __syncthreads();  // WS becomes the stage [ch][slot]
#pragma unroll
      for (int pi = 0; pi < PT; ++pi)
#pragma unroll
        for (int cj = 0; cj < 2; ++cj)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[pi][cj][4 * g4 + e];
            const int p = wr * WM + 32 * pi + acc32_row(4 * g4);
            const int ch = wc * 64 + 32 * cj + (l & 31);
            store_vec<TC, 4>(WS + ch * LD + (p & ~31) + key_slot(p & 31), v);
          }
    }
    __syncthreads();
    if (kind == 0 || kind == 1) {
      // Q / K: [b][line][h][t][d]; per head BM x D contiguous.
      TC* dst = (kind == 0 ? Q : K) + lineq * kHeads * Np * kHeadDim;
      constexpr int CPP = kHeadDim / VEC;  // chunks per (position, head)
#pragma unroll
      for (int it = 0; it < BM * kC / VEC / NT; ++it) {
        const int idx = tid + it * NT;
        const int hh = idx / (BM * CPP);
        const int r = idx % (BM * CPP);
        const int p = r / CPP;
        const int d0 = (r % CPP) * VEC;
        *reinterpret_cast<u32x4*>(dst + ((size_t)hh * Np + t0 + p) * kHeadDim + d0) =
            *reinterpret_cast<const u32x4*>(WS + p * LD + hh * kHeadDim + d0);
      }
    } else if (kind == 2) {
      // Vt: [b][line][h][d][slot]
      TC* dst = Vt + lineq * kHeads * kHeadDim * Np + t0;
      constexpr int CPR = BM / VEC;
#pragma unroll
      for (int it = 0; it < BM * kC / VEC / NT; ++it) {
        const int idx = tid + it * NT;
        const int c = idx / CPR;
        const int s0 = (idx % CPR) * VEC;
        *reinterpret_cast<u32x4*>(dst + (size_t)c * Np + s0) = *reinterpret_cast<const u32x4*>(WS + c * LD + s0);
      }
    } else {
      // G = sigmoid(g): [b][line][t][C]
      TC* dst = G + (lineq * Np + t0) * kC;
      constexpr int CPR = kC / VEC;
#pragma unroll
      for (int it = 0; it < BM * kC / VEC / NT; ++it) {
        const int idx = tid + it * NT;
        const int p = idx / CPR;
        const int c0 = (idx % CPR) * VEC;
        *reinterpret_cast<u32x4*>(dst + (size_t)p * kC + c0) = *reinterpret_cast<const u32x4*>(WS + p * LD + c0);
      }
    }
  }

  // Pair bias: one 16-column block (H real columns) over BM rows, BM/4 rows per wave.
  {
    constexpr int RB = BM / 4 / 16;
    f32x4 accb[RB][1];
    zero_acc(accb);
    int prow[1] = {4 * kC};
    gemm16_lds_x_w<TC, kC, RB, 1>(accb, X, LD, w * (BM / 4), w5, kC, prow);
    if ((l & 15) < kHeads) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int e = 0; e < 4; ++e) pbs[w * (BM / 4) + rb * 16 + 4 * (l >> 4) + e][l & 15] = accb[rb][0][e] * kLog2e;
    }
  }
  __syncthreads();
  const bool line_ok = line < N;
  for (int idx = tid; idx < kHeads * BM; idx += NT) {
    const int hh = idx / BM;
    const int p = idx % BM;
    const int t = t0 + p;
    const float v = (line_ok && t < N) ? pbs[p][hh] : 0.f;
    if (transpose)  // key-major [b][h][key = line][query = t]
      PB[(((size_t)b * kHeads + hh) * Np + line) * Np + t] = v;
    else  // query-major [b][h][query = line][slot(key = t)]
      PB[(((size_t)b * kHeads + hh) * Np + line) * Np + (t & ~31) + key_slot(t & 31)] = v;
  }
  if (tid < BM) {
    const int t = t0 + tid;
    const float v = t < N ? (mks[tid] - 1.0f) * 1e9f * kLog2e : -INFINITY;
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
PF_DEVICE Frag16<bf16> pack_p(const f32x16& p, bf16) {
  Frag16<bf16> f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    f.v[0][e] = (bf16)p[e];
    f.v[1][e] = (bf16)p[8 + e];
  }
  return f;
}
PF_DEVICE Frag16<float> pack_p(const f32x16& p, float) {
  Frag16<float> f;
#pragma unroll
  for (int i = 0; i < 4; ++i) f.v[i] = f32x4{p[4 * i], p[4 * i + 1], p[4 * i + 2], p[4 * i + 3]};
  return f;
}

template <class TC>
constexpr int attn_qsub() { return sizeof(TC) == 2 ? PF_ATTN_QS : 2; }  // 32-query sub-blocks per wave
#ifndef PF_ATTN_LPB
#define PF_ATTN_LPB 4
#endif
constexpr int kLinesPerBlock = PF_ATTN_LPB;                       // one line per wave
constexpr int kBiasLd = 36;                                       // LDS row of 32 slots + pad (floats)
// Online-softmax reference. Probabilities are exp2(s - ref) with a per-query reference
// that starts at 0 and is raised only when a key block's maximum exceeds it by more than
// kRaise (base-2 units), so p <= 2^kRaise and a row sum <= N 2^kRaise stay far inside the
// fp32 and bf16 exponent range; a first block whose maximum is below -kLower (a masked
// start) sets the reference to it. The normalised result does not depend on the
// reference, and while it is 0 -- the common case -- the per-logit subtraction is skipped.
constexpr float kRaise = 32.0f;
constexpr float kLower = 64.0f;

// Block: 4 waves = 4 consecutive lines, one head, QB = 32 * QS queries. The pair-bias tile
// (shared by the 4 lines) is staged through LDS, double-buffered; Q is staged through LDS
// once; K and V are per line and loaded straight into MFMA operand registers, one key
// block ahead.
// L lines per batch item (line stride Lp in the operand buffers). O_HEAD_MAJOR writes O as
// [b][line][h][q][d] with q < N (the reference kernel's layout) instead of the frame's
// [b][line][q][h d]; zero_masked_lines writes 0 for a line whose keys are all masked (the
// reference kernel's rule) instead of the eager path's uniform average.
template <class TC, bool BIAS_KEY_MAJOR, int QS, bool O_HEAD_MAJOR>
__global__ __launch_bounds__(64 * kLinesPerBlock, QS == 1 ? 4 : (QS == 2 ? 3 : 2)) void tri_attn_kernel(const TC* __restrict__ Q,
                                                                        const TC* __restrict__ K,
                                                                        const TC* __restrict__ Vt,
                                                                        const float* __restrict__ PB,
                                                                        const float* __restrict__ MA,
                                                                        TC* __restrict__ O, int B, int N, int Np,
                                                                        int L, int Lp, int zero_masked_lines,
                                                                        int xcd_remap) {
  constexpr int QB = 32 * QS;
  constexpr int NT = 64 * kLinesPerBlock;
  constexpr int QLD = kHeadDim + lds_pad<TC>();
  constexpr int QVEC = 16 / sizeof(TC);
  __shared__ __attribute__((aligned(16))) float bias_lds[2][QB * kBiasLd];
  __shared__ __attribute__((aligned(16))) TC q_lds[kLinesPerBlock][QB * QLD];
  __shared__ int same_mask[kLinesPerBlock];

  const int nqb = Np / QB;
  const int nlg = (L + kLinesPerBlock - 1) / kLinesPerBlock;
  const int total = B * nlg * kHeads * nqb;
  int bid = blockIdx.x;
  if (xcd_remap) bid = (bid & 7) * (total >> 3) + (bid >> 3);
  // q-block fastest, then line group, then head: one XCD walks all q-blocks of a line
  // group (K/V reuse in its L2) and many line groups of one head (bias reuse).
  const int qb = bid % nqb;
  int rest = bid / nqb;
  const int lg = rest % nlg;
  rest /= nlg;
  const int h = rest % kHeads;
  const int b = rest / kHeads;
  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const int line = lg * kLinesPerBlock + w;
  const bool active = line < L;  // inactive waves still stage the shared bias tiles

  const int lq = l & 31;
  const int hf = l >> 5;
  const size_t lineq = (size_t)b * Lp + line;
  const TC* Qh = Q + (lineq * kHeads + h) * (size_t)Np * kHeadDim;
  const TC* Kh = K + (lineq * kHeads + h) * (size_t)Np * kHeadDim;
  const TC* Vh = Vt + (lineq * kHeads + h) * (size_t)kHeadDim * Np;
  const float* PBh = PB + ((size_t)b * kHeads + h) * (size_t)Np * Np;
  const float* MAl = MA + lineq * Np;
  const int q0 = qb * QB;

  // Bias tile staging: QB queries x 32 key slots per key block. When every line of the
  // block has the same key mask (the common case: pair masks are seq x seq, so all
  // unpadded lines share one row), the mask row is added to the shared tile here once,
  // instead of per wave and per logit. MA0 is the first line's mask row.
  const float* MA0 = MA + ((size_t)b * Lp + lg * kLinesPerBlock) * Np;
  constexpr int BIAS_IT = QB * 32 / 4 / NT;
  f32x4 bpf[BIAS_IT];
  bool fold_mask = false;
  auto bias_load = [&](int k0) {
#pragma unroll
    for (int it = 0; it < BIAS_IT; ++it) {
      const int idx = tid + it * NT;
      if (BIAS_KEY_MAJOR) {  // lanes run over the 32 keys, so the transposing LDS writes hit 32 banks
        const int k = idx & 31;
        const int qq = (idx >> 5) * 4;
        bpf[it] = *reinterpret_cast<const f32x4*>(PBh + (size_t)(k0 + k) * Np + q0 + qq);
        if (fold_mask) {
          const float m = MA0[k0 + key_slot(k)];
#pragma unroll
          for (int e = 0; e < 4; ++e) bpf[it][e] += m;
        }
      } else {  // rows: QB queries of 32 slots
        const int qq = idx / 8;
        const int s0 = (idx % 8) * 4;
        bpf[it] = *reinterpret_cast<const f32x4*>(PBh + (size_t)(q0 + qq) * Np + k0 + s0);
        if (fold_mask) {
          const f32x4 m = *reinterpret_cast<const f32x4*>(MA0 + k0 + s0);
#pragma unroll
          for (int e = 0; e < 4; ++e) bpf[it][e] += m[e];
        }
      }
    }
  };
  auto bias_store = [&](int buf) {
    float* dst = bias_lds[buf];
#pragma unroll
    for (int it = 0; it < BIAS_IT; ++it) {
      const int idx = tid + it * NT;
      if (BIAS_KEY_MAJOR) {
        const int k = idx & 31;
        const int qq = (idx >> 5) * 4;
        const int s = key_slot(k);
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[(qq + e) * kBiasLd + s] = bpf[it][e];
      } else {
        const int qq = idx / 8;
        const int s0 = (idx % 8) * 4;
        *reinterpret_cast<f32x4*>(dst + qq * kBiasLd + s0) = bpf[it];
      }
    }
  };

  // Q of this wave's line -> LDS (rows of D elements, padded)
  TC* qw = q_lds[w];
  if (active) {
#pragma unroll
    for (int it = 0; it < QB * kHeadDim / QVEC / 64; ++it) {
      const int idx = l + it * 64;
      const int qq = idx / (kHeadDim / QVEC);
      const int d0 = (idx % (kHeadDim / QVEC)) * QVEC;
      *reinterpret_cast<u32x4*>(qw + qq * QLD + d0) =
          *reinterpret_cast<const u32x4*>(Qh + (size_t)(q0 + qq) * kHeadDim + d0);
    }
  }
  bool masked = false, same = true, all_masked = true;
  if (active) {
    for (int k = l; k < N; k += 64) {
      const int sl = (k & ~31) + key_slot(k & 31);
      const float m = MAl[sl];
      masked |= m != 0.f;
      same &= m == MA0[sl];
      all_masked &= m < -1e8f;
    }
  }
  masked = __any(masked);
  same = __all(same);
  all_masked = __all(all_masked);
  if (l == 0) same_mask[w] = same ? 1 : 0;
  __syncthreads();
  fold_mask = true;
#pragma unroll
  for (int i = 0; i < kLinesPerBlock; ++i) fold_mask = fold_mask && same_mask[i];
  if (fold_mask) masked = false;  // the tile carries the mask (and the padding keys' -inf)

  f32x16 o[QS];
  float mref[QS], lrun[QS];
#pragma unroll
  for (int s = 0; s < QS; ++s) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[s][r] = 0.f;
    mref[s] = 0.f;
    lrun[s] = 0.f;
  }

  const int nkb = (N + 31) / 32;
  Frag16<TC> kf, vf;
  if (active) {
    kf.load(Kh + (size_t)lq * kHeadDim + 16 * hf);
    vf.load(Vh + (size_t)lq * Np + 16 * hf);
  }
  bias_load(0);
  bias_store(0);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * 32;
    const bool more = kb + 1 < nkb;
    Frag16<TC> kn, vn;
    if (more) {
      bias_load(k0 + 32);
      if (active) {
        kn.load(Kh + (size_t)(k0 + 32 + lq) * kHeadDim + 16 * hf);
        vn.load(Vh + (size_t)lq * Np + k0 + 32 + 16 * hf);
      }
    }
    if (active) {
      // Additive key mask, applied after q k^T + pb as the reference orders the fp32 adds
      // (a fully masked line then rounds every logit to the same -1e9 log2 e). The MA slots
      // of padding keys hold -inf.
      const bool use_madd = masked || (!fold_mask && k0 + 32 > N);
      const float* mrow = MAl + k0 + 16 * hf;
      const float* bl = bias_lds[kb & 1];
#pragma unroll
      for (int s = 0; s < QS; ++s) {
        f32x16 sacc;
        const float* br = bl + (32 * s + lq) * kBiasLd + 16 * hf;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 bv = *reinterpret_cast<const f32x4*>(br + 4 * i);
#pragma unroll
          for (int e = 0; e < 4; ++e) sacc[4 * i + e] = bv[e];
        }
        Frag16<TC> qf;
        qf.load(qw + (32 * s + lq) * QLD + 16 * hf);
        mma32_16(sacc, kf, qf);  // log2-domain q k^T + pb
        if (use_madd) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const f32x4 mv = *reinterpret_cast<const f32x4*>(mrow + 4 * i);
#pragma unroll
            for (int e = 0; e < 4; ++e) sacc[4 * i + e] += mv[e];
          }
        }
        if (__any(mref[s] != 0.f)) {
#pragma unroll
          for (int r = 0; r < 16; ++r) sacc[r] -= mref[s];
        }
        float mx = fmaxf(fmaxf(sacc[0], sacc[1]), sacc[2]);
#pragma unroll
        for (int r = 3; r < 15; r += 2) mx = fmaxf(fmaxf(mx, sacc[r]), sacc[r + 1]);
        mx = fmaxf(mx, sacc[15]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const bool first = kb == 0;
        const bool shift = mx > kRaise || (first && mx < -kLower);
        if (__any(shift)) {
          const float delta = shift ? mx : 0.f;
          const float alpha = first ? 0.f : __builtin_amdgcn_exp2f(-delta);
          mref[s] += delta;
          lrun[s] *= alpha;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            o[s][r] *= alpha;
            sacc[r] -= delta;
          }
        }
        float ls = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          sacc[r] = __builtin_amdgcn_exp2f(sacc[r]);
          ls += sacc[r];
        }
        lrun[s] += ls;
        mma32_16(o[s], vf, pack_p(sacc, TC{}));
      }
    }
    if (more) {
      bias_store((kb + 1) & 1);
      kf = kn;
      vf = vn;
    }
    __syncthreads();
  }
  if (!active) return;

  // O^T lane (q, hf) holds d = 8 (r >> 2) + 4 hf + (r & 3).
  const bool write_zero = zero_masked_lines && all_masked;
#pragma unroll
  for (int s = 0; s < QS; ++s) {
    const float lt = lrun[s] + __shfl_xor(lrun[s], 32, 64);
    const float inv = write_zero ? 0.f : 1.0f / lt;
    const int q = q0 + 32 * s + lq;
    if (q >= N) continue;
    TC* dst = O_HEAD_MAJOR ? O + ((lineq * kHeads + h) * (size_t)N + q) * kHeadDim
                           : O + (lineq * (size_t)Np + q) * kC + h * kHeadDim;
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
// Block: BM positions of one line. A = O * G -> LDS; acc^T = Wout A^T; fp32 stage; the
// update is stored (or added) at the z position of each attention-frame position.
template <class TZ, class TC>
__global__ __launch_bounds__(256) void attn_out_kernel(const TC* __restrict__ O, const TC* __restrict__ G,
                                                       const TC* __restrict__ Wo, TZ* __restrict__ out, int N, int Np,
                                                       int transpose, int accumulate) {
  constexpr int BM = block_rows<TC>();
  constexpr int LD = ld128<TC>();
  constexpr int SLD = kC + 4;
  constexpr int NT = 256;
  constexpr int WM = BM / 2;
  constexpr int PT = WM / 32;
  constexpr int VEC = 16 / sizeof(TC);
  constexpr int A_BYTES = BM * LD * (int)sizeof(TC);
  constexpr int W_BYTES = 128 * LD * (int)sizeof(TC);
  constexpr int S_BYTES = BM * SLD * 4;
  static_assert(S_BYTES <= A_BYTES + W_BYTES, "stage must fit over the operand tiles");
  __shared__ __attribute__((aligned(16))) char smem[A_BYTES + W_BYTES];
  TC* A = reinterpret_cast<TC*>(smem);
  TC* Wl = reinterpret_cast<TC*>(smem + A_BYTES);
  float* stage = reinterpret_cast<float*>(smem);

  const int t0 = blockIdx.x * BM;
  const int line = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const int wr = w >> 1, wc = w & 1;
  const size_t lineq = (size_t)b * Np + line;
  {
    Rows128<TC, 128, NT> wl;
    wl.load(Wo, kC);
    const TC* Ol = O + (lineq * Np + t0) * kC;
    const TC* Gl = G + (lineq * Np + t0) * kC;
    constexpr int CPR = kC / VEC;
#pragma unroll
    for (int it = 0; it < BM * CPR / NT; ++it) {
      const int idx = tid + it * NT;
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
      store_vec<TC, VEC>(A + p * LD + c0, y);
    }
    wl.store(Wl, LD);
  }
  __syncthreads();
  f32x16 acc[2][PT];
  zero_acc32(acc);
  wave_mma32<TC, 2, PT, kC>(acc, Wl, LD, wc * 64, A, LD, wr * WM);
  __syncthreads();
#pragma unroll
  for (int ci = 0; ci < 2; ++ci)
#pragma unroll
    for (int pj = 0; pj < PT; ++pj)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int ch = wc * 64 + 32 * ci + acc32_row(4 * g4);
        const int p = wr * WM + 32 * pj + (l & 31);
        *reinterpret_cast<f32x4*>(stage + p * SLD + ch) =
            f32x4{acc[ci][pj][4 * g4], acc[ci][pj][4 * g4 + 1], acc[ci][pj][4 * g4 + 2], acc[ci][pj][4 * g4 + 3]};
      }
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
  const size_t Np = pf::round_up((size_t)N, kPad);
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
  const int Np = (int)pf::round_up((size_t)N, kPad);
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
  constexpr int BM = block_rows<TC>();
  {
    dim3 grid(Np / BM, Np, B);
    pf::KernelTimer timer("attn_project", s);
    attn_project_kernel<TZ, TC><<<grid, 256, 0, s>>>((const TZ*)z, mask, lnw, lnb, eps, (const TC*)w5, Qb, Kb, Vb,
                                                     Gb, PBb, MAb, N, Np, transpose, qscale);
    timer.stop();
    if (int e = pf::check_launch("attn_project")) return e;
  }
  {
    const int nqb = Np / (32 * attn_qsub<TC>());
    const int nlg = (N + kLinesPerBlock - 1) / kLinesPerBlock;
    const long total = (long)B * nlg * kHeads * nqb;
    const int remap = (total % 8 == 0) ? 1 : 0;
    dim3 grid((unsigned)total);
    pf::KernelTimer timer("tri_attn", s);
    constexpr int QS = attn_qsub<TC>();
    constexpr int NT = 64 * kLinesPerBlock;
    if (transpose)
      tri_attn_kernel<TC, true, QS, false><<<grid, NT, 0, s>>>(Qb, Kb, Vb, PBb, MAb, Ob, B, N, Np, N, Np, 0, remap);
    else
      tri_attn_kernel<TC, false, QS, false><<<grid, NT, 0, s>>>(Qb, Kb, Vb, PBb, MAb, Ob, B, N, Np, N, Np, 0, remap);
    timer.stop();
    if (int e = pf::check_launch("tri_attn")) return e;
  }
  {
    dim3 grid((N + BM - 1) / BM, N, B);
    pf::KernelTimer timer("attn_out", s);
    attn_out_kernel<TZ, TC><<<grid, 256, 0, s>>>(Ob, Gb, (const TC*)wo, (TZ*)out, N, Np, transpose, accumulate);
    timer.stop();
    if (int e = pf::check_launch("attn_out")) return e;
  }
  return pf::ok();
}

// ------------------------------------------------------------------ kernel-level op
// _EvoformerAttention.apply(Q, K, V, res_mask, pair_bias, pre_transposed=True)
// (triton/evo_attention.py:1198-1292): O = softmax(Q K^T d^-1/2 + pair_bias + res_mask) V
// per (batch, line, head) with Q, K, V, O as [B][S][H][N][D], res_mask additive [B][S][N],
// pair_bias [B][H][N][N] fp32. The operands are repacked into the attention frame (padded
// to Np, Q pre-scaled by d^-1/2 log2 e, V transposed with the key-slot order, bias and mask
// times log2 e) and run through the same flash kernel. -inf mask entries become -1e9.
template <class TC>
__global__ __launch_bounds__(256) void evo_pack_qk_kernel(const TC* __restrict__ q, const TC* __restrict__ k,
                                                          TC* __restrict__ Qw, TC* __restrict__ Kw, int N, int Np,
                                                          float qscale) {
  constexpr int VEC = 16 / sizeof(TC);
  constexpr int CPT = kHeadDim / VEC;  // chunks per token
  const size_t bsh = blockIdx.y;       // (b, s, h) flattened
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= Np * CPT) return;
  const int t = idx / CPT;
  const int d0 = (idx % CPT) * VEC;
  float vq[VEC], vk[VEC];
  if (t < N) {
    load16<TC>(q + (bsh * N + t) * kHeadDim + d0, vq);
    load16<TC>(k + (bsh * N + t) * kHeadDim + d0, vk);
#pragma unroll
    for (int e = 0; e < VEC; ++e) vq[e] *= qscale;
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) vq[e] = vk[e] = 0.f;
  }
  store_vec<TC, VEC>(Qw + (bsh * Np + t) * kHeadDim + d0, vq);
  store_vec<TC, VEC>(Kw + (bsh * Np + t) * kHeadDim + d0, vk);
}

// One block per (32-key block, b s h): V[t][d] -> Vt[d][slot].
template <class TC>
__global__ __launch_bounds__(256) void evo_pack_v_kernel(const TC* __restrict__ v, TC* __restrict__ Vt, int N,
                                                         int Np) {
  __shared__ float tile[32][kHeadDim + 1];
  const size_t bsh = blockIdx.y;
  const int k0 = blockIdx.x * 32;
  for (int i = threadIdx.x; i < 32 * kHeadDim; i += 256) {
    const int t = i / kHeadDim, d = i % kHeadDim;
    tile[t][d] = (k0 + t < N) ? to_f32(v[(bsh * N + k0 + t) * kHeadDim + d]) : 0.f;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 32 * kHeadDim; i += 256) {
    const int d = i / 32, slot = i % 32;
    Vt[(bsh * kHeadDim + d) * Np + k0 + slot] = from_f32<TC>(tile[slot_key(slot)][d]);
  }
}

__global__ __launch_bounds__(256) void evo_pack_bias_kernel(const float* __restrict__ pb, float* __restrict__ PB,
                                                            int N, int Np) {
  const size_t bh = blockIdx.y;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)Np * Np) return;
  const int qi = (int)(idx / Np);
  const int sl = (int)(idx % Np);
  const int kk = (sl & ~31) + slot_key(sl & 31);
  PB[bh * Np * Np + idx] = (qi < N && kk < N) ? pb[(bh * N + qi) * N + kk] * kLog2e : 0.f;
}

__global__ __launch_bounds__(256) void evo_pack_mask_kernel(const float* __restrict__ rm, float* __restrict__ MA,
                                                            int N, int Np) {
  const size_t bs = blockIdx.y;
  const int sl = blockIdx.x * 256 + threadIdx.x;
  if (sl >= Np) return;
  const int kk = (sl & ~31) + slot_key(sl & 31);
  float v = -INFINITY;
  if (kk < N) v = fmaxf(rm[bs * N + kk], -1e9f) * kLog2e;
  MA[bs * Np + sl] = v;
}

struct EvoWs {
  size_t q, k, v, pb, ma, total;
};

EvoWs evo_ws_layout(int B, int S, int N, int cdtype) {
  const size_t Np = pf::round_up((size_t)N, kPad);
  const size_t es = cdtype == PF_F32 ? 4 : 2;
  const size_t tok = (size_t)B * S * kHeads * Np * kHeadDim * es;
  EvoWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += pf::round_up(bytes, 256);
    return at;
  };
  w.q = take(tok);
  w.k = take(tok);
  w.v = take(tok);
  w.pb = take((size_t)B * kHeads * Np * Np * 4);
  w.ma = take((size_t)B * S * Np * 4);
  w.total = off;
  return w;
}

template <class TC>
int evo_attn_launch(const void* q, const void* k, const void* v, const float* res_mask, const float* pair_bias, int B,
                    int S, int N, int zero_rule, void* out, void* ws, hipStream_t s) {
  const int Np = (int)pf::round_up((size_t)N, kPad);
  const EvoWs L = evo_ws_layout(B, S, N, sizeof(TC) == 4 ? PF_F32 : PF_BF16);
  char* base = reinterpret_cast<char*>(ws);
  TC* Qw = reinterpret_cast<TC*>(base + L.q);
  TC* Kw = reinterpret_cast<TC*>(base + L.k);
  TC* Vw = reinterpret_cast<TC*>(base + L.v);
  float* PBw = reinterpret_cast<float*>(base + L.pb);
  float* MAw = reinterpret_cast<float*>(base + L.ma);
  const float qscale = (1.0f / sqrtf((float)kHeadDim)) * kLog2e;
  const unsigned bsh = (unsigned)(B * S * kHeads);
  constexpr int VEC = 16 / sizeof(TC);
  evo_pack_qk_kernel<TC><<<dim3((Np * (kHeadDim / VEC) + 255) / 256, bsh), 256, 0, s>>>(
      (const TC*)q, (const TC*)k, Qw, Kw, N, Np, qscale);
  evo_pack_v_kernel<TC><<<dim3(Np / 32, bsh), 256, 0, s>>>((const TC*)v, Vw, N, Np);
  evo_pack_bias_kernel<<<dim3((unsigned)(((long)Np * Np + 255) / 256), B * kHeads), 256, 0, s>>>(pair_bias, PBw,
                                                                                                   N, Np);
  evo_pack_mask_kernel<<<dim3((Np + 255) / 256, B * S), 256, 0, s>>>(res_mask, MAw, N, Np);
  if (int e = pf::check_launch("evo_attn pack")) return e;
  constexpr int QS = attn_qsub<TC>();
  constexpr int NT = 64 * kLinesPerBlock;
  const int nqb = Np / (32 * QS);
  const int nlg = (S + kLinesPerBlock - 1) / kLinesPerBlock;
  const long total = (long)B * nlg * kHeads * nqb;
  const int remap = (total % 8 == 0) ? 1 : 0;
  pf::KernelTimer timer("evo_attn", s);
  tri_attn_kernel<TC, false, QS, true><<<dim3((unsigned)total), NT, 0, s>>>(Qw, Kw, Vw, PBw, MAw, (TC*)out, B, N, Np,
                                                                            S, S, zero_rule, remap);
  timer.stop();
  return pf::check_launch("evo_attn");
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

size_t pf_evo_attn_workspace_bytes(int B, int S, int H, int N, int D, int dtype) {
  if (B <= 0 || S <= 0 || N <= 0 || H != kHeads || D != kHeadDim) return 0;
  return evo_ws_layout(B, S, N, dtype).total;
}

int pf_evo_attn_fwd(const void* q, const void* k, const void* v, const float* res_mask, const float* pair_bias, int B,
                    int S, int H, int N, int D, int dtype, int masked_rows_zero, void* out, void* workspace,
                    size_t workspace_bytes, void* stream) {
  PF_REQUIRE(q && k && v && res_mask && pair_bias && out && workspace, PF_ERR_INVALID_ARG,
             "pf_evo_attn_fwd: null pointer");
  PF_REQUIRE(B > 0 && S > 0 && N > 0, PF_ERR_INVALID_ARG, "pf_evo_attn_fwd: B=%d S=%d N=%d", B, S, N);
  PF_REQUIRE(H == kHeads && D == kHeadDim, PF_ERR_UNSUPPORTED, "pf_evo_attn_fwd: H=%d D=%d (built: H=4, D=32)", H,
             D);
  PF_REQUIRE(dtype == PF_F32 || dtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_evo_attn_fwd: dtype %d", dtype);
  PF_REQUIRE(pf::aligned16(q) && pf::aligned16(k) && pf::aligned16(v) && pf::aligned16(out) &&
                 pf::aligned16(workspace),
             PF_ERR_ALIGNMENT, "pf_evo_attn_fwd: pointers must be 16-byte aligned");
  PF_REQUIRE(workspace_bytes >= evo_ws_layout(B, S, N, dtype).total, PF_ERR_WORKSPACE,
             "pf_evo_attn_fwd: workspace %zu < %zu bytes", workspace_bytes, evo_ws_layout(B, S, N, dtype).total);
  hipStream_t s = pf::as_stream(stream);
  if (dtype == PF_F32)
    return evo_attn_launch<float>(q, k, v, res_mask, pair_bias, B, S, N, masked_rows_zero, out, workspace, s);
  return evo_attn_launch<bf16>(q, k, v, res_mask, pair_bias, B, S, N, masked_rows_zero, out, workspace, s);
}

}  // extern "C"
