// Triangle attention (GridSelfAttention, starting and ending node) in three launches:
//
//   A1 attn_project:  x = LN(z); q, k, v, g = x W{q,k,v,g}^T; pb = x Wpb^T. Writes the
//                     attention-frame operands Q, K (token-major), Vt (key-contiguous,
//                     keys permuted inside 32-blocks), G = sigmoid(g) (fp32 only; in bf16
//                     A3 computes the gate from the z rows it reads), the pair bias PB and
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
// ending node (column mode). Keys and queries run along the other token index. In bf16, K
// and Vt are stored as 2 KB key-block tiles in the flash kernel's fragment order (kv_chunk).
// The projection kernel walks z along a line in both modes (column mode reads z down a column),
// so every operand is written contiguously in the attention frame. The pair bias is
// written query-major [h][q][key slot] in row mode and key-major [h][key][q] in column mode
// (again the order in which the projection produces it); an in-place tile transpose turns
// the latter query-major, the layout the attention kernel streams into LDS.
//
// MFMA layout (v_mfma_f32_32x32x16_bf16 / v_mfma_f32_32x32x2f32). A wave owns 32 queries
// per sub-block and computes S^T = K Q^T (keys are accumulator rows), so lane (q, h)
// (q = lane & 31, h = lane >> 5) holds the logits of query q for keys
// kappa(r, h) = 8 (r >> 2) + 4 h + (r & 3), r = 0..15. Those 16 probabilities are exactly
// the B operand lane (q, h) must supply for O^T += V^T P^T when the keys of a 32-block are
// stored in the order kappa (storage slot 16 h + r holds key kappa(r, h)): Vt, PB and MA
// use that order, so P never goes through LDS.
#include <algorithm>

#include "capi.h"
#include "common.h"
#include "rowops.h"

namespace {

constexpr int kHeads = 4;
constexpr int kHeadDim = 32;
constexpr int kC = 128;
constexpr int kPad = 128;  // token padding of the attention frame
#ifndef PF_ATTN_QS
#define PF_ATTN_QS 2
#endif

// bf16 K and Vt tiles. Per (line, head) each 32-key block is one 2 KB tile of 128 chunks of
// 16 bytes: chunk 32 g + r holds row r, columns 8 c .. 8 c + 7 with g = 2 (c & 1) + (c >> 1)
// (K: row = key, column = d; Vt: row = d, column = key slot). Lane (r, hf) of the flash
// kernel needs columns 16 hf + 8 j .. +7 of row r for MFMA j, i.e. chunk 64 j + 32 hf + r =
// 64 j + lane: each of its two loads reads one contiguous kilobyte.
PF_DEVICE int kv_chunk(int row, int c) { return 32 * (2 * (c & 1) + (c >> 1)) + row; }

// For a pair mask that is the outer product of its binary diagonal (m[i][k] = m[i][i]
// m[k][k], the trunk's seq_mask x seq_mask) every line with m[i][i] = 1 masks the same keys,
// so their additive key mask km[b][k] = 1e9 (m[k][k] - 1) is added to the shared pair bias
// once and the flash kernel needs no per-line mask (a line with m[i][i] = 0 has every key
// masked and takes the closed form). In the log2 domain; padding keys (key >= N) get -inf.
PF_DEVICE float folded_key_mask(const float* km, int N, int key) {
  return key < N ? km[key] * kLog2e : -INFINITY;
}


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

// A1, persistent and weight-stationary (bf16 GEMMs). One 512-thread block per CU walks
// tiles of 64 positions along a frame line. Waves 0-5 own kind w >> 1 (q, k, v) and heads
// 2 (w & 1), +1: those 64 weight rows stay in MFMA A-operand registers for the whole
// kernel. Per tile: each wave LayerNorms 8 z rows into a double-buffered LDS tile (the next
// tile's rows are loaded while this tile's MFMAs run); waves 0-5 compute their rows'
// projections, stage the result in a private LDS region in the layout of the output
// (Q, K: [h][t][d] via acc^T[channel][position]; Vt: [h][d][slot] via acc[position][channel])
// and write it with 16-byte stores. Waves 6 and 7 project the pair bias of 32 positions
// each (16x16x32 MFMAs on the bias rows); wave 7 writes the line's additive mask slots.
// The gate projection is not made here: the output kernel computes it from z.
struct ProjectAttnWs {
  static constexpr int BP = 64;
  static constexpr int NW = 8;
  static constexpr int NT = 64 * NW;
  static constexpr int XLD = kC + 8;
  static constexpr int QLD = kHeadDim + 8;  // Q/K stage rows [t][d]
  static constexpr int VLD = BP + 8;        // Vt stage rows [d][slot]
  static constexpr int STAGE = 2 * BP * QLD;
};

template <class TZ>
__global__ __launch_bounds__(ProjectAttnWs::NT) void attn_project_ws_kernel(
    const TZ* __restrict__ z, const float* __restrict__ mask, const float* __restrict__ lnw,
    const float* __restrict__ lnb, float eps, const bf16* __restrict__ w5, bf16* __restrict__ Q,
    bf16* __restrict__ K, bf16* __restrict__ Vt, float* __restrict__ PB,
    float* __restrict__ MA, int B, int N, int Np, int transpose, float qscale) {
  using Cfg = ProjectAttnWs;
  constexpr int BP = Cfg::BP, NW = Cfg::NW, XLD = Cfg::XLD, QLD = Cfg::QLD, VLD = Cfg::VLD;
  constexpr int VEC = 16 / sizeof(TZ);
  constexpr int LPR = kC / VEC;
  constexpr int RPI = 64 / LPR;
  constexpr int RPW = BP / NW;
  constexpr int NLD = RPW / RPI;
  static_assert(2 * kHeadDim * VLD <= Cfg::STAGE, "stage size");
  __shared__ __attribute__((aligned(16))) bf16 xs[2][BP * XLD];
  __shared__ __attribute__((aligned(16))) bf16 stage_all[NW][Cfg::STAGE];

  const int w = wave_id();
  const int l = lane_id();
  const int kind = w >> 1;  // 0 q, 1 k, 2 v, 3: pair bias and mask
  const int h0 = 2 * (w & 1);
  bf16* stg = stage_all[w];
  const int tpl = Np / BP;
  const long ntiles = (long)B * Np * tpl;

  // Weights -> A operands: rows kind * 128 + 32 (h0 + hi) + (l & 31), k = 16 ks + 8 (l >> 5).
  bf16x8 wa[2][kC / 16];
#pragma unroll
  for (int hi = 0; hi < 2; ++hi) {
    const bf16* rp = w5 + (size_t)(min(kind, 2) * kC + 32 * (h0 + hi) + (l & 31)) * kC + 8 * (l >> 5);
#pragma unroll
    for (int ks = 0; ks < kC / 16; ++ks) wa[hi][ks] = *reinterpret_cast<const bf16x8*>(rp + 16 * ks);
  }
  // Pair-bias rows: 16x16x32 A operands (lane holds row l & 15, k = 32 ks + 8 (l >> 4)),
  // kept in LDS as [ks][lane] fragments, which leaves the registers for the LayerNorm
  // parameters (read from LDS per tile, their 32-byte-strided reads cost more bank-conflict
  // cycles than the rest of the kernel's LDS traffic together).
  __shared__ bf16x8 wbs[kC / 32][64];
  if (w == 0) {
    const bf16* rp = w5 + (size_t)(4 * kC + (l & 15)) * kC + 8 * (l >> 4);
#pragma unroll
    for (int ks = 0; ks < kC / 32; ++ks) wbs[ks][l] = *reinterpret_cast<const bf16x8*>(rp + 32 * ks);
  }
  const int chunk = l % LPR;
  float lw[VEC], lb[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    lw[e] = lnw[chunk * VEC + e];
    lb[e] = lnb[chunk * VEC + e];
  }
  __syncthreads();

  auto tile_coords = [&](long tile, int& b, int& line, int& t0) {
    b = (int)(tile / ((long)Np * tpl));
    const long rem = tile % ((long)Np * tpl);
    line = (int)(rem / tpl);
    t0 = (int)(rem % tpl) * BP;
  };
  u32x4 zr[NLD];
  bool zok[NLD];
  float mkn = 0.f;
  auto issue = [&](long tile) {
    int b, line, t0;
    tile_coords(tile, b, line, t0);
    const TZ* zb = z + (size_t)b * N * N * kC;
#pragma unroll
    for (int q = 0; q < NLD; ++q) {
      const int t = t0 + w * RPW + q * RPI + l / LPR;
      zok[q] = line < N && t < N;
      if (zok[q]) {
        const size_t pos = transpose ? (size_t)t * N + line : (size_t)line * N + t;
        zr[q] = *reinterpret_cast<const u32x4*>(zb + pos * kC + chunk * VEC);
      } else {
        zr[q] = u32x4{0u, 0u, 0u, 0u};
      }
    }
    if (w == 7) {
      const int t = t0 + l;
      const size_t pos = transpose ? (size_t)t * N + line : (size_t)line * N + t;
      mkn = (line < N && t < N) ? mask[(size_t)b * N * N + pos] : 0.f;
    }
  };

  long tile = blockIdx.x;
  if (tile < ntiles) issue(tile);
  int buf = 0;
  for (; tile < ntiles; tile += gridDim.x, buf ^= 1) {
    int b, line, t0;
    tile_coords(tile, b, line, t0);
    const size_t lineq = (size_t)b * Np + line;
    bf16* xb = xs[buf];
#pragma unroll
    for (int q = 0; q < NLD; ++q) {
      float v[VEC];
      unpack16<TZ>(zr[q], v);
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) sum += v[e];
      const float mean = row_group_sum<LPR>(sum) * (1.0f / kC);
      float sq = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float d = v[e] - mean;
        sq += d * d;
      }
      const float rstd = rsqrtf(row_group_sum<LPR>(sq) * (1.0f / kC) + eps);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float y = (v[e] - mean) * rstd * lw[e] + lb[e];
        v[e] = zok[q] ? y : 0.f;
      }
      store_vec<bf16, VEC>(xb + (w * RPW + q * RPI + l / LPR) * XLD + chunk * VEC, v);
    }
    const float mk = mkn;
    const long next = tile + gridDim.x;
    if (next < ntiles) issue(next);
    __syncthreads();  // xs[buf] holds the whole tile

    if (kind == 3) {
      // Pair bias of positions 32 (w - 6) + 16 sb + l (lanes 0-15 hold heads 0-3).
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const int pp = 32 * (w - 6) + 16 * sb;
        f32x4 pacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < kC / 32; ++ks) {
          const bf16x8 xf = *reinterpret_cast<const bf16x8*>(xb + (pp + (l & 15)) * XLD + 32 * ks + 8 * (l >> 4));
          pacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wbs[ks][l], xf, pacc, 0, 0, 0);
        }
        if (l < 16) {
          const int t = t0 + pp + l;
          const bool ok = line < N && t < N;
#pragma unroll
          for (int hh = 0; hh < kHeads; ++hh) {
            const float v = ok ? pacc[hh] * kLog2e : 0.f;
            float* dst = PB + (((size_t)b * kHeads + hh) * Np + line) * Np;
            if (transpose)  // key-major [b][h][key = line][query = t]
              dst[t] = v;
            else  // query-major [b][h][query = line][slot(key = t)]
              dst[(t & ~31) + key_slot(t & 31)] = v;
          }
        }
      }
      if (w == 7) {
        const int t = t0 + l;
        MA[lineq * Np + (t & ~31) + key_slot(t & 31)] = t < N ? (mk - 1.0f) * 1e9f * kLog2e : -INFINITY;
      }
      continue;  // block-uniform barriers only at the top of the loop
    }

    // acc[head][position tile]: acc^T [channel][position] (a lane holds 16 channels of one
    // position) for Q and K; acc [position][channel] for Vt, the operands swapped, so a lane
    // holds 4 consecutive positions of a channel -- 4 consecutive key slots of its stage.
    f32x16 acc[2][2];
    zero_acc32(acc);
    auto gemm = [&](auto positions_as_rows) __attribute__((always_inline)) {
#pragma unroll
      for (int ks = 0; ks < kC / 16; ++ks) {
        bf16x8 xf[2];
#pragma unroll
        for (int pt = 0; pt < 2; ++pt)
          xf[pt] = *reinterpret_cast<const bf16x8*>(xb + (32 * pt + (l & 31)) * XLD + 16 * ks + 8 * (l >> 5));
#pragma unroll
        for (int hi = 0; hi < 2; ++hi)
#pragma unroll
          for (int pt = 0; pt < 2; ++pt)
            acc[hi][pt] = decltype(positions_as_rows)::value
                              ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(xf[pt], wa[hi][ks], acc[hi][pt], 0, 0, 0)
                              : __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa[hi][ks], xf[pt], acc[hi][pt], 0, 0, 0);
      }
    };
    if (kind == 2)
      gemm(std::true_type{});
    else
      gemm(std::false_type{});

    // Epilogue: stage in the output layout, then 16-byte stores.
    if (kind <= 1) {  // Q (pre-scaled) or K: stage [hi][t][d]
      const float sc = kind == 0 ? qscale : 1.0f;
#pragma unroll
      for (int hi = 0; hi < 2; ++hi)
#pragma unroll
        for (int pt = 0; pt < 2; ++pt)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[hi][pt][4 * g4 + e] * sc;
            store_vec<bf16, 4>(stg + (hi * BP + 32 * pt + (l & 31)) * QLD + acc32_row(4 * g4), v);
          }
    } else {  // Vt: stage [hi][d][slot]; positions 8 g4 + 4 hf + e are slots 16 hf + 4 g4 + e
#pragma unroll
      for (int hi = 0; hi < 2; ++hi)
#pragma unroll
        for (int pt = 0; pt < 2; ++pt)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[hi][pt][4 * g4 + e];
            store_vec<bf16, 4>(stg + (hi * kHeadDim + (l & 31)) * VLD + 32 * pt + key_slot(acc32_row(4 * g4)), v);
          }
    }
    // The stage is private to this wave: LDS operations of one wave complete in order.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (kind == 0) {
      bf16* dst0 = Q + ((lineq * kHeads + h0) * Np + t0) * kHeadDim;
#pragma unroll
      for (int hi = 0; hi < 2; ++hi)
#pragma unroll
        for (int it = 0; it < BP * kHeadDim / 8 / 64; ++it) {
          const int p = it * 16 + (l >> 2);
          const int c = l & 3;
          *reinterpret_cast<u32x4*>(dst0 + ((size_t)hi * Np + p) * kHeadDim + 8 * c) =
              *reinterpret_cast<const u32x4*>(stg + (hi * BP + p) * QLD + 8 * c);
        }
    } else {
      // K / Vt key-block tiles (kv_chunk): lane-consecutive chunks, so each store
      // instruction writes one contiguous kilobyte. The tile's BP / 32 key blocks of head
      // h0 + hi follow each other in memory.
      bf16* dst0 = (kind == 1 ? K : Vt) + ((lineq * kHeads + h0) * Np + t0) * kHeadDim;
#pragma unroll
      for (int hi = 0; hi < 2; ++hi)
#pragma unroll
        for (int it = 0; it < BP * kHeadDim / 8 / 64; ++it) {
          const int g = it * 64 + l;  // chunk of this head's BP / 32 tiles
          const int kbl = g >> 7, grp = (g >> 5) & 3, r = g & 31;
          const int c = 2 * (grp & 1) + (grp >> 1);
          const bf16* src = kind == 1 ? stg + (hi * BP + 32 * kbl + r) * QLD + 8 * c
                                      : stg + (hi * kHeadDim + r) * VLD + 32 * kbl + 8 * c;
          *reinterpret_cast<u32x4*>(dst0 + (size_t)hi * Np * kHeadDim + 8 * g) =
              *reinterpret_cast<const u32x4*>(src);
        }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// ------------------------------------------------------------------ A2
template <class TC>
constexpr int attn_qsub() { return sizeof(TC) == 2 ? PF_ATTN_QS : 2; }  // 32-query sub-blocks per wave
#ifndef PF_ATTN_LPB
#define PF_ATTN_LPB 4
#endif
constexpr int kLinesPerBlock = PF_ATTN_LPB;                       // one line per wave
// Online-softmax reference. Probabilities are exp2(s - ref) with a per-query reference
// that starts at 0 and is raised only when a key block's maximum exceeds it by more than
// kRaise (base-2 units), so p <= 2^kRaise and a row sum <= N 2^kRaise stay far inside the
// fp32 and bf16 exponent range; a first block whose maximum is below -kLower (a masked
// start) sets the reference to it. The normalised result does not depend on the
// reference, and while it is 0 -- the common case -- the per-logit subtraction is skipped.
constexpr float kRaise = 32.0f;
constexpr float kLower = 64.0f;
constexpr int kBiasStages = 3;  // LDS ring of pair-bias tiles, filled two key blocks ahead

// Element strides of one [B][S][H][N][D] operand view of the kernel-level attention op (D
// contiguous): batch item, line, head, key. Zero strides mean the dense [b][line][h][q][d].
struct Strides4 {
  long b, s, h, n;
};

// XOR swizzle of the 16-byte chunks of a 128-byte bias row: the 16 lanes of a ds_read_b128
// (rows R..R+15, one logical chunk) land on 16 distinct bank groups.
PF_DEVICE int bias_swz(int row) { return (row >> 1) & 7; }

// Dynamic LDS of the flash kernel: the bias ring, kBiasStages tiles of QB x 32 fp32.
template <class TC>
constexpr size_t attn_bias_lds_bytes() { return (size_t)kBiasStages * 32 * attn_qsub<TC>() * 32 * 4; }

// Register sets for the K / V / mask-row prefetch ring: loads one key block ahead. (Two
// blocks ahead needs a third set, 16 more VGPRs, and costs the fourth wave per SIMD that
// hides the same latency better: 487 -> 463 us at N=768 with one ahead and four waves.)
template <class TC>
constexpr int attn_kv_sets() { return 2; }

// Mask operand: S^T += M 1^T, A = the line's additive key mask in k-column 0 (lanes of the
// low half, key row lane & 31), B = ones in k-column 0. Keys are MFMA rows in natural
// order, so lane l reads the mask slot key_slot(l & 31).
PF_DEVICE void mma_mask(f32x16& acc, float m, bf16) {
  const bool lo = (threadIdx.x & 32) == 0;
  bf16x8 a = {}, one = {};
  a[0] = lo ? (bf16)m : (bf16)0.f;
  one[0] = lo ? (bf16)1.f : (bf16)0.f;
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, one, acc, 0, 0, 0);
}
PF_DEVICE void mma_mask(f32x16& acc, float m, float) {
  const bool lo = (threadIdx.x & 32) == 0;
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(lo ? m : 0.f, lo ? 1.f : 0.f, acc, 0, 0, 0);
}

// K / Vt fragment loads. bf16: the 2 KB tile of a key block is stored fragment-native
// (kv_chunk), so the two 16-byte loads of a wave are each one contiguous 1 KB run
// (voff = 16 * lane, second load at +1 KB). fp32: rows of the plain layouts, 16 bytes apart.
template <class TC>
PF_DEVICE Frag16<TC> buf_frag16(__amdgpu_buffer_rsrc_t r, int voff, int soff);
template <>
PF_DEVICE Frag16<bf16> buf_frag16<bf16>(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  Frag16<bf16> f;
  f.v[0] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  f.v[1] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff + 1024, soff, 0));
  return f;
}
template <>
PF_DEVICE Frag16<float> buf_frag16<float>(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  Frag16<float> f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    f.v[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16 * i, soff, 0));
  return f;
}

// Block: 4 waves = 4 consecutive lines, one head, QB = 32 * QS queries. The pair-bias tile
// (query-major, shared by the 4 lines) streams through a 3-stage LDS ring filled by direct
// buffer-to-LDS loads two key blocks ahead; Q is staged through LDS once and its fragments
// are read from there at every key block (bf16: unpadded 64-byte rows with a 16-byte chunk
// swizzle, so a block takes 40 KB of LDS and four blocks fit a CU); K, V and the line's mask
// slot for the lane's key row are per line and go straight into registers one key block
// ahead, in two register sets the unrolled key loop alternates. The kernel fits 128 VGPRs:
// four waves per SIMD. All
// global loads are raw buffer loads: a scalar base per operand, a fixed per-lane offset and
// a scalar per-key-block offset, so the key loop does no vector address arithmetic.
// L lines per batch item (line stride Lp in the operand buffers). O_HEAD_MAJOR writes O as
// [b][line][h][q][d] with q < N (the reference kernel's layout) instead of the frame's
// [b][line][q][h d]; zero_masked_lines writes 0 for a line whose keys are all masked (the
// reference kernel's rule) instead of the eager path's uniform average. POST_SCALE
// multiplies the fp32 logit accumulator by `post_scale` after the q k^T products, so Q
// reaches the MFMAs as given (no re-rounding of a pre-scaled Q to bf16) and the bias and
// mask operands carry 1 / post_scale (the kernel-level op's fp32 post-scale).
//
// Two modes share this kernel. FAST keeps the softmax reference at 0 for the whole key loop:
// no running maximum, no rescaling, only exp2, the row sum and the P V products per logit
// (the logits of LayerNorm-ed projections are small, so 2^s stays far inside fp32/bf16
// range). A line whose keys are all masked takes the closed form of the eager rule (every
// real key weighs 1). The wave then checks its result -- row sums in [2^-90, 3e38], all
// outputs finite -- and writes a per-wave flag redo[blockIdx.x * 4 + wave]; a flagged block
// is recomputed by the exact mode (FAST = false with `redo` set), which runs the lazy
// running-maximum softmax below and skips every block whose flags are all 0.
template <class TC, int QS, bool O_HEAD_MAJOR, bool FAST, bool POST_SCALE = false, bool KMASK = true>
__global__ __launch_bounds__(64 * kLinesPerBlock, QS == 1 ? 4 : (QS == 2 ? 4 : 2)) void tri_attn_kernel(
    const TC* __restrict__ Q, const TC* __restrict__ K, const TC* __restrict__ Vt, const float* __restrict__ PB,
    const float* __restrict__ MA, TC* __restrict__ O, int B, int N, int Np, int L, int Lp, int zero_masked_lines,
    int xcd_remap, int* __restrict__ redo, float post_scale = 1.f, Strides4 ost = {},
    float* __restrict__ lse_out = nullptr) {
  constexpr int QB = 32 * QS;
  constexpr int NT = 64 * kLinesPerBlock;
  constexpr int QLD = kHeadDim + (sizeof(TC) == 2 ? 0 : lds_pad<TC>());
  constexpr int QVEC = 16 / sizeof(TC);
  auto qswz = [](int row) { return sizeof(TC) == 2 ? (row >> 2) & 3 : 0; };
  constexpr int TILE = QB * 32;                   // floats per bias stage: QB rows of 32 slots
  constexpr int DL = TILE * 4 / (NT * 16);        // direct loads per lane per stage
  static_assert(DL * NT * 16 == TILE * 4, "bias stage must split evenly over the block");
  constexpr int NSET = attn_kv_sets<TC>();
  // vmcnt budget: loads a lane issues per key block (bias stage + K + V [+ mask slot])
  constexpr int KV_LOADS = (sizeof(TC) == 2 ? 4 : 8) + (KMASK ? 1 : 0);
  // The bias ring is dynamic LDS (attn_bias_lds_bytes at launch): the stage a step reads
  // is never the one its direct loads fill, and the explicit vmcnt + barrier order them.
  extern __shared__ __attribute__((aligned(16))) float bias_lds[];
  __shared__ __attribute__((aligned(16))) TC q_lds[kLinesPerBlock][QB * QLD];

  if (!FAST && redo != nullptr) {
    int any = 0;
#pragma unroll
    for (int i = 0; i < kLinesPerBlock; ++i) any |= redo[(size_t)blockIdx.x * kLinesPerBlock + i];
    if (!any) return;  // block-uniform: every wave leaves before the first barrier
  }
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
  const int w = wave_id();
  const int l = lane_id();
  const int line = lg * kLinesPerBlock + w;
  const bool active = line < L;  // inactive waves still load their share of the bias tiles

  const int lq = l & 31;
  const int hf = l >> 5;
  const size_t lineq = (size_t)b * Lp + (active ? line : lg * kLinesPerBlock);
  const TC* Qh = Q + (lineq * kHeads + h) * (size_t)Np * kHeadDim;
  const TC* Kh = K + (lineq * kHeads + h) * (size_t)Np * kHeadDim;
  const TC* Vh = Vt + (lineq * kHeads + h) * (size_t)kHeadDim * Np;
  const float* PBh = PB + ((size_t)b * kHeads + h) * (size_t)Np * Np;
  const float* MAl = MA + lineq * Np;
  const int q0 = qb * QB;
  const int nkb = (N + 31) / 32;
  // Last key block a load may address. With the key mask applied here (KMASK), steps past
  // nkb reload block nkb - 1 and the mask sends them to -inf; without it (the mask is in
  // the bias, which is -inf at every padding key), such steps read the padding blocks up to
  // Np (K and V zero there), which add nothing.
  const int kb_last = KMASK ? nkb - 1 : Np / 32 - 1;

  const auto rk = buf_rsrc(Kh, (unsigned)(Np * kHeadDim * sizeof(TC)));
  const auto rv = buf_rsrc(Vh, (unsigned)(kHeadDim * Np * sizeof(TC)));
  const auto rm = buf_rsrc(MAl, (unsigned)(Np * sizeof(float)));
  const auto rb = buf_rsrc(PBh, (unsigned)((size_t)Np * Np * sizeof(float)));
  // bf16: K and Vt in 2 KB fragment-native key-block tiles; fp32: K [key][d], Vt [d][slot].
  constexpr bool kBlk = sizeof(TC) == 2;
  const int k_voff = kBlk ? 16 * l : (lq * kHeadDim + 16 * hf) * (int)sizeof(TC);
  const int v_voff = kBlk ? 16 * l : (lq * Np + 16 * hf) * (int)sizeof(TC);
  const int v_kstride = kBlk ? kHeadDim * (int)sizeof(TC) : (int)sizeof(TC);  // bytes per key
  const int m_voff = key_slot(lq) * 4;
  // Bias stage: DL loads per lane, each 8 rows x 128 B; lane l writes row 8 blk + l / 8 at
  // physical chunk l % 8 = logical chunk (l % 8) ^ swz(row).
  int b_voff[DL];
#pragma unroll
  for (int j = 0; j < DL; ++j) {
    const int row = (w * DL + j) * 8 + (l >> 3);
    b_voff[j] = ((q0 + row) * Np + 4 * ((l & 7) ^ bias_swz(row))) * 4;
  }

  // Past the last key block the last tile is loaded again into a stage nobody reads, so
  // every iteration issues the same number of loads (the vmcnt budget below relies on it).
  // Bias ring stage of key block kb. The key loop runs whole rounds of NSET blocks from 0,
  // so with NSET == kBiasStages the stage is the (compile-time) position u in the round.
  // (u: the block's position in its round, or any value congruent to kb mod NSET).
  auto stage_of = [&](int kb, int u) { return NSET == kBiasStages ? u % NSET : kb % kBiasStages; };
  auto bias_issue = [&](int kb, int u) {
    float* st = bias_lds + stage_of(kb, u) * TILE;
    const int soff = min(kb, kb_last) * 32 * 4;
#pragma unroll
    for (int j = 0; j < DL; ++j) buf_load_lds16(rb, st + (w * DL + j) * 8 * 32, b_voff[j], soff);
  };
  auto kv_load = [&](int kb, Frag16<TC>& kf, Frag16<TC>& vf, float& mf) {
    const int k0 = min(kb, kb_last) * 32;
    kf = buf_frag16<TC>(rk, k_voff, k0 * kHeadDim * (int)sizeof(TC));
    vf = buf_frag16<TC>(rv, v_voff, k0 * v_kstride);
    if constexpr (KMASK)
      mf = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rm, m_voff, k0 * 4, 0));
    else
      mf = 0.f;
  };

  // Q of this wave's line -> LDS (rows of D elements, padded)
  TC* qw = q_lds[w];
  if (active) {
#pragma unroll
    for (int it = 0; it < QB * kHeadDim / QVEC / 64; ++it) {
      const int idx = l + it * 64;
      const int qq = idx / (kHeadDim / QVEC);
      const int d0 = (idx % (kHeadDim / QVEC)) * QVEC;
      *reinterpret_cast<u32x4*>(qw + qq * QLD + QVEC * ((d0 / QVEC) ^ qswz(qq))) =
          *reinterpret_cast<const u32x4*>(Qh + (size_t)(q0 + qq) * kHeadDim + d0);
    }
  }
  // Scan of the line's mask slots: 16-byte loads, four per lane in flight before any is
  // used (a load-then-test loop made one memory round trip per 64 keys). Padding slots
  // (keys >= N, holding -inf) are skipped by their key index.
  bool all_masked = true;
  if (active) {
    for (int s0 = 4 * l; s0 < Np; s0 += 1024) {
      f32x4 m4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) m4[j] = *reinterpret_cast<const f32x4*>(MAl + min(s0 + 256 * j, Np - 4));
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int sl = s0 + 256 * j + e;
          if (sl < Np && (sl & ~31) + slot_key(sl & 31) < N) all_masked &= m4[j][e] < -1e8f;
        }
    }
  }
  all_masked = __all(all_masked);

  f32x16 o[QS];
  float mref[QS], lrun[QS];
#pragma unroll
  for (int s = 0; s < QS; ++s) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[s][r] = 0.f;
    mref[s] = 0.f;
    lrun[s] = 0.f;
  }
  // FAST: row sums of P per sub-block, two partial sums each (bf16: v_dot2 over the packed
  // probabilities the P V product consumes).
  float lsum[QS][2];
#pragma unroll
  for (int s = 0; s < QS; ++s) lsum[s][0] = lsum[s][1] = 0.f;

  __syncthreads();  // Q tiles

  // Every key-block step issues K/V/mask (NSET - 1 blocks ahead) and then one bias stage
  // (two blocks ahead); the prologue issues what steps -2 and -1 would have, so every
  // lane -- inactive waves load their group's first line -- keeps the same load order.
  // The scheduling barriers keep the prologue's loads in the in-loop order (K/V/mask, then
  // bias): the vmcnt budget counts them in that order, and so does the compiler's own wait
  // insertion, which otherwise waits on the newest loads inside the first step of every round.
  Frag16<TC> kr[NSET], vr[NSET];
  float mr[NSET];
  if (NSET == 3) kv_load(0, kr[0], vr[0], mr[0]);
  __builtin_amdgcn_sched_barrier(0);
  bias_issue(0, 0);
  __builtin_amdgcn_sched_barrier(0);
  kv_load(NSET - 2, kr[NSET - 2], vr[NSET - 2], mr[NSET - 2]);
  __builtin_amdgcn_sched_barrier(0);
  bias_issue(1, 1);
  __builtin_amdgcn_sched_barrier(0);

  // Start of step kb: this lane's loads of bias stage kb landed (and with them, in issue
  // order, the K/V of block kb): after them it issued one step's K/V/mask loads and one bias
  // stage. Then every wave's stage kb is visible, and stage (kb + 2) % 3 (read at kb - 1) is
  // free for the next fill.
  auto sync_issue = [&](int kb, int u, Frag16<TC>& kn, Frag16<TC>& vn, float& mn) {
    constexpr int after = KV_LOADS + DL;
    static_assert(after < 16, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt(after | (7 << 4) | (15 << 8));
    __builtin_amdgcn_s_barrier();
    kv_load(kb + NSET - 1, kn, vn, mn);
    bias_issue(kb + 2, u + 2);
  };

  // Key mask of block kb (padding keys past N: -inf). The mask MFMA runs for every key
  // block, masked or not: skipping it behind a wave-wide vote costs more in branching and
  // scheduling than the one 32x32x16 step it saves (460 -> 448 us at N=768, rows).
  auto key_mask = [&](int kb, float mf) { return kb < nkb ? mf : -INFINITY; };
  // S^T tiles of key block kb: bias from the LDS stage, key mask, then q k^T (log2 domain).
  auto logits = [&](int kb, int u, int s, const Frag16<TC>& kf, float mk, f32x16& sacc) {
    const float* bl = bias_lds + stage_of(kb, u) * TILE;
    const int R = 32 * s + lq;
    const float* br = bl + R * 32;
    if constexpr (sizeof(TC) == 2) {
      // bf16: the accumulator starts at the bias, then the key mask, then q k^T (two
      // 32x32x16 steps, so the products meet the bias's magnitude twice).
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 bv = *reinterpret_cast<const f32x4*>(br + 4 * ((4 * hf + i) ^ bias_swz(R)));
#pragma unroll
        for (int e = 0; e < 4; ++e) sacc[4 * i + e] = bv[e];
      }
      if constexpr (KMASK) mma_mask(sacc, mk, TC{});
      Frag16<TC> qf;
      qf.v[0] = *reinterpret_cast<const bf16x8*>(qw + R * QLD + 8 * ((2 * hf) ^ qswz(R)));
      qf.v[1] = *reinterpret_cast<const bf16x8*>(qw + R * QLD + 8 * ((2 * hf + 1) ^ qswz(R)));
      mma32_16(sacc, kf, qf);
    } else {
      // fp32: q k^T from a zero accumulator (sixteen 32x32x2 steps), then the bias, then
      // the key mask -- the eager order (q k^T scale + bias) + mask. Accumulating the
      // sixteen partial products onto a large bias would round each at its magnitude.
      Frag16<TC> qf;
      qf.load(qw + R * QLD + 16 * hf);
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
      mma32_16(sacc, kf, qf);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 bv = *reinterpret_cast<const f32x4*>(br + 4 * ((4 * hf + i) ^ bias_swz(R)));
#pragma unroll
        for (int e = 0; e < 4; ++e) sacc[4 * i + e] += bv[e];
      }
      if constexpr (KMASK) mma_mask(sacc, mk, TC{});
    }
    if constexpr (POST_SCALE) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] *= post_scale;
    }
  };

  // FAST step: p = 2^s, row sums, O^T += V^T P^T.
  // Sub-blocks one after the other: one S tile live at a time.
  auto compute_fast = [&](int kb, int u, const Frag16<TC>& kf, const Frag16<TC>& vf, float mf) {
    const float km = key_mask(kb, mf);
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      f32x16 sacc;
      logits(kb, u, s, kf, km, sacc);
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = __builtin_amdgcn_exp2f(sacc[r]);
      const Frag16<TC> pf = pack_p(sacc, TC{});
      if constexpr (sizeof(TC) == 2) {
        typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
        const bf16x2_t one2 = {(bf16)1.f, (bf16)1.f};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const bf16x2_t pr = {pf.v[j >> 2][2 * (j & 3)], pf.v[j >> 2][2 * (j & 3) + 1]};
          lsum[s][j & 1] = __builtin_amdgcn_fdot2_f32_bf16(pr, one2, lsum[s][j & 1], false);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) lsum[s][r & 1] += sacc[r];
      }
      mma32_16(o[s], vf, pf);
    }
  };

  // Exact step: lazy running maximum (see kRaise / kLower). The block maximum is taken
  // over the raw logits and the reference is subtracted once, after it has been updated:
  // a reference at the mask level (about -1.44e9, set by a first key block whose keys are
  // all masked) subtracted from a real logit would round it to a multiple of 128, so it
  // is never applied to a block that holds a real key -- that block's maximum exceeds it
  // by far more than kRaise and replaces it first (alpha = 2^-1.44e9 = 0 then clears the
  // masked keys' contributions).
  auto compute_exact = [&](int kb, int u, const Frag16<TC>& kf, const Frag16<TC>& vf, float mf) {
    f32x16 sacc[QS];
    const float km = key_mask(kb, mf);
#pragma unroll
    for (int s = 0; s < QS; ++s) logits(kb, u, s, kf, km, sacc[s]);
    float mx[QS];
    bool any_shift = false;
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      float m = fmaxf(fmaxf(sacc[s][0], sacc[s][1]), sacc[s][2]);
#pragma unroll
      for (int r = 3; r < 15; r += 2) m = fmaxf(fmaxf(m, sacc[s][r]), sacc[s][r + 1]);
      m = fmaxf(m, sacc[s][15]);
      mx[s] = max_xor32(m);
      any_shift |= mx[s] - mref[s] > kRaise || (kb == 0 && mx[s] < -kLower);
    }
    if (__any(any_shift)) {
#pragma unroll
      for (int s = 0; s < QS; ++s) {
        const bool shift = mx[s] - mref[s] > kRaise || (kb == 0 && mx[s] < -kLower);
        // kb == 0: nothing accumulated yet. Otherwise only raises reach here (mx - mref >
        // kRaise), so the rescale factor is 2^(mref - mx) < 2^-kRaise.
        const float alpha = !shift ? 1.f : (kb == 0 ? 0.f : __builtin_amdgcn_exp2f(mref[s] - mx[s]));
        if (shift) mref[s] = mx[s];
        lrun[s] *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) o[s][r] *= alpha;
      }
    }
    bool ref_set = false;
#pragma unroll
    for (int s = 0; s < QS; ++s) ref_set |= mref[s] != 0.f;
    if (__any(ref_set)) {
#pragma unroll
      for (int s = 0; s < QS; ++s)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[s][r] -= mref[s];
    }
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      float ls = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sacc[s][r] = __builtin_amdgcn_exp2f(sacc[s][r]);
        ls += sacc[s][r];
      }
      lrun[s] += ls;
    }
#pragma unroll
    for (int s = 0; s < QS; ++s) mma32_16(o[s], vf, pack_p(sacc[s], TC{}));
  };

  // Key loop unrolled over the register sets: key block kb uses set kb % NSET and refills
  // set (kb - 1) % NSET, consumed one block earlier. Only whole rounds of NSET blocks run
  // (no conditional step, so the compiler's wait counts stay exact): a step past the last
  // key block sees every key masked to -inf and adds nothing. The loop is entered
  // unconditionally (nkb >= 1): a zero-trip test in front of it lets the compiler sink the
  // prologue's K/V loads behind the bias loads, and the reordered counts then make it wait
  // on the next block's loads inside every first step.
#define PF_TRI_ATTN_KEY_LOOP(COMPUTE)                         \
  for (int kb0 = 0;;) {                                       \
    _Pragma("unroll") for (int u = 0; u < NSET; ++u) {        \
      const int nx = (u + NSET - 1) % NSET;                   \
      sync_issue(kb0 + u, u, kr[nx], vr[nx], mr[nx]);         \
      if (active) COMPUTE(kb0 + u, u, kr[u], vr[u], mr[u]);   \
    }                                                         \
    kb0 += NSET;                                              \
    if (kb0 >= nkb) break;                                    \
  }
  // Fully masked lines skip the key loop in both modes (closed form below), so the exact
  // mode reproduces the fast mode's result for them bit for bit.
  const bool live = active && !all_masked;  // wave-uniform
  if constexpr (FAST) {
    auto compute_live = [&](int kb, int u, const Frag16<TC>& kf, const Frag16<TC>& vf, float mf) {
      if (live) compute_fast(kb, u, kf, vf, mf);
    };
    PF_TRI_ATTN_KEY_LOOP(compute_live)
  } else {
    auto compute_live = [&](int kb, int u, const Frag16<TC>& kf, const Frag16<TC>& vf, float mf) {
      if (live) compute_exact(kb, u, kf, vf, mf);
    };
    PF_TRI_ATTN_KEY_LOOP(compute_live)
  }
#undef PF_TRI_ATTN_KEY_LOOP
  if (active && all_masked) {
    // Fully masked line: every logit carries the same -1e9 shift, so each real key
    // weighs 1 (the eager rule's uniform average); V is summed outside the bias ring.
    for (int kb = 0; kb < nkb; ++kb) {
      const int k0 = kb * 32;
      const Frag16<TC> vf = buf_frag16<TC>(rv, v_voff, k0 * v_kstride);
      f32x16 pr;
#pragma unroll
      for (int r = 0; r < 16; ++r) pr[r] = k0 + 8 * (r >> 2) + 4 * hf + (r & 3) < N ? 1.f : 0.f;
      float c = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) c += pr[r];
      const Frag16<TC> pf = pack_p(pr, TC{});
#pragma unroll
      for (int s = 0; s < QS; ++s) {
        lsum[s][0] += c;
        mma32_16(o[s], vf, pf);
      }
    }
  }
  // FAST: lrun is 0 here and lsum holds the row sums; exact: lsum is 0 except for a
  // fully masked line.
#pragma unroll
  for (int s = 0; s < QS; ++s) lrun[s] += lsum[s][0] + lsum[s][1];
  // The last steps loaded repeat tiles into LDS; none may land after the block's LDS is
  // handed to another block.
  __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
  if constexpr (FAST) {
    bool bad = false;
    if (active) {
#pragma unroll
      for (int s = 0; s < QS; ++s) {
        const float lt = lrun[s] + __shfl_xor(lrun[s], 32, 64);
        const bool real = q0 + 32 * s + lq < N;
        bad |= real && !(lt >= 0x1p-90f && lt <= 3.0e38f);
#pragma unroll
        for (int r = 0; r < 16; ++r) bad |= real && !__builtin_isfinite(o[s][r]);
      }
    }
    bad = __any(bad);
    if (l == 0) redo[(size_t)blockIdx.x * kLinesPerBlock + w] = bad ? 1 : 0;
    if (bad) return;
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
    if (lse_out != nullptr && hf == 0) {
      // log2-unit LSE of the row (the softmax reference plus log2 of the row sum); +inf for a
      // line whose keys are all masked or a row whose logits are all below -1e8 log2 e.
      float lse2 = mref[s] + __builtin_amdgcn_logf(lt);
      if (all_masked || !(lse2 >= -1.0e8f * kLog2e)) lse2 = INFINITY;
      lse_out[(((size_t)b * L + line) * kHeads + h) * Np + q] = lse2;
    }
    TC* dst;
    if constexpr (O_HEAD_MAJOR)
      dst = ost.n ? O + b * ost.b + line * ost.s + h * ost.h + q * ost.n
                  : O + ((lineq * kHeads + h) * (size_t)N + q) * kHeadDim;
    else
      dst = O + (lineq * (size_t)Np + q) * kC + h * kHeadDim;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = o[s][4 * j + e] * inv;
      store_vec<TC, 4>(dst + 8 * j + 4 * hf, v);
    }
  }
}

// Column mode: the projection kernel writes the pair bias key-major [h][key][q]; the flash
// kernel reads it query-major in key-slot order, out[q][slot] = in[slot_key(slot)][q]
// within each 32-block. 32 x 32 tile (I, J) of the output depends only on tile (J, I) of
// the input, so one block swaps a tile pair in place (I <= J; blockIdx.y = b h). With an
// outer-product key mask `km` [b][N] its folded value is added on the way.
__global__ __launch_bounds__(256) void pb_transpose_kernel(float* __restrict__ PB, int Np,
                                                           const float* __restrict__ km, int N) {
  __shared__ float ta[32][33], tb[32][33];
  const int nt = Np / 32;
  int p = blockIdx.x, I = 0;
  while (p >= nt - I) {
    p -= nt - I;
    ++I;
  }
  const int J = I + p;
  float* M = PB + (size_t)blockIdx.y * Np * Np;
  for (int i = threadIdx.x; i < 1024; i += 256) {
    const int r = i >> 5, c = i & 31;
    ta[r][c] = M[(size_t)(32 * I + r) * Np + 32 * J + c];
    tb[r][c] = M[(size_t)(32 * J + r) * Np + 32 * I + c];
  }
  __syncthreads();
  const float* kb = km ? km + (size_t)(blockIdx.y / kHeads) * N : nullptr;
  for (int i = threadIdx.x; i < 1024; i += 256) {
    const int q = i >> 5, sl = i & 31;
    float x = tb[slot_key(sl)][q], y = ta[slot_key(sl)][q];
    if (kb) {
      x += folded_key_mask(kb, N, 32 * J + slot_key(sl));
      y += folded_key_mask(kb, N, 32 * I + slot_key(sl));
    }
    M[(size_t)(32 * I + q) * Np + 32 * J + sl] = x;
    M[(size_t)(32 * J + q) * Np + 32 * I + sl] = y;
  }
}

// Row mode: the folded outer-product key mask km [b][N] added to the query-major pair bias
// [b][h][q][slot] (key = slot_key of the slot inside its 32-block), four slots per thread.
__global__ __launch_bounds__(256) void pb_fold_kernel(float* __restrict__ PB, const float* __restrict__ km, int N,
                                                      int Np) {
  const size_t bh = blockIdx.y;
  const float* kb = km + (bh / kHeads) * N;
  f32x4* M = reinterpret_cast<f32x4*>(PB + bh * Np * Np);
  const size_t n4 = (size_t)Np * Np / 4;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    const int slot0 = (int)((4 * i) % Np);
    f32x4 v = M[i];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int sl = slot0 + e;
      v[e] += folded_key_mask(kb, N, (sl & ~31) + slot_key(sl & 31));
    }
    M[i] = v;
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

// A3, persistent and weight-stationary (bf16 GEMMs), with the output gate. Blocks of 8
// waves (two per CU) walk tiles of 64 positions of a frame line. Thread (position p, part
// sp) loads channels 16 sp .. +16 of z at p; the 8 threads of a position LayerNorm the row
// (statistics over DPP lane groups) into an LDS tile. Wave w owns channels 16 w .. +16 of
// the gate and of the output projection (W_g and W_out rows as 16x16x32 MFMA A operands,
// resident in registers): g^T = W_g LN(z)^T, then a = O * sigmoid(g) -- O read straight in
// the accumulator layout -- into a second LDS tile, y^T = W_out a^T staged in fp32, and each
// thread adds the update to the z channels it loaded and stores them. The next tile's z and
// O are loaded during this tile's gate GEMM, and its LayerNorm runs before the residual.
// Computing the gate here, from the z rows the residual needs anyway, saves A1 writing it
// and this kernel reading it back.
struct OutAttnWs {
  static constexpr int BP = 64;
  static constexpr int NW = 8;
  static constexpr int NT = 64 * NW;
  static constexpr int ALD = kC + 8;  // bf16 operand rows [pos][ch]
  static constexpr int SLD = kC + 4;  // fp32 update rows [pos][ch]
};

template <class TZ>
__global__ __launch_bounds__(OutAttnWs::NT, 4) void attn_out_ws_kernel(
    const bf16* __restrict__ O, const bf16* __restrict__ Wg, const bf16* __restrict__ Wo, const TZ* z,
    const float* __restrict__ lnw, const float* __restrict__ lnb, float eps, TZ* out, int B, int N, int Np,
    int transpose, int accumulate, int res_is_z) {
  using Cfg = OutAttnWs;
  constexpr int BP = Cfg::BP, ALD = Cfg::ALD, SLD = Cfg::SLD;
  constexpr int ZV = 16 / sizeof(TZ);  // z elements per 16-byte load
  constexpr int ZL = 16 / ZV;          // 16-byte z loads per thread (16 channels)
  __shared__ __attribute__((aligned(16))) bf16 x_lds[BP * ALD];  // LN(z)
  __shared__ __attribute__((aligned(16))) bf16 a_lds[BP * ALD];  // O * sigmoid(g)
  __shared__ __attribute__((aligned(16))) float upd[BP * SLD];
  // LayerNorm weight | bias as [q][sp] groups of 4 channels (16 sp + 4 q ..): the 8 parts of
  // a position read 8 consecutive 16-byte groups.
  __shared__ f32x4 lnq[2][4][8];

  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const int tpl = (N + BP - 1) / BP;
  const long ntiles = (long)B * N * tpl;

  bf16x8 wg[kC / 32], wo[kC / 32];
#pragma unroll
  for (int ks = 0; ks < kC / 32; ++ks) {
    const size_t at = (size_t)(16 * w + (l & 15)) * kC + 32 * ks + 8 * (l >> 4);
    wg[ks] = *reinterpret_cast<const bf16x8*>(Wg + at);
    wo[ks] = *reinterpret_cast<const bf16x8*>(Wo + at);
  }
  if (tid < 64) {
    const int sp = tid & 7, q = (tid >> 3) & 3, wb = tid >> 5;
    const float* src = (wb ? lnb : lnw) + 16 * sp + 4 * q;
    lnq[wb][q][sp] = f32x4{src[0], src[1], src[2], src[3]};
  }
  // Thread (position p, part s) handles channels 16 s .. +16 of position p.
  const int p = tid >> 3, sp = tid & 7;
  // Accumulator lanes: channels 16 w + 4 (l >> 4) + e of position 16 pt + (l & 15).
  const int cq = 16 * w + 4 * (l >> 4);

  auto tile_coords = [&](long tile, int& b, int& line, int& t0) {
    b = (int)(tile / ((long)N * tpl));
    const long rem = tile % ((long)N * tpl);
    line = (int)(rem / tpl);
    t0 = (int)(rem % tpl) * BP;
  };
  auto zpos = [&](int b, int line, int t) -> size_t {
    return (size_t)b * N * N + (transpose ? (size_t)t * N + line : (size_t)line * N + t);
  };
  // O tiles lie inside the padded frame (t0 + 63 < Np); z rows past N read as zeros.
  u32x2 orr[4];
  u32x4 zr[ZL];
  auto issue = [&](long tile) {
    int b, line, t0;
    tile_coords(tile, b, line, t0);
    const bf16* Ol = O + (((size_t)b * Np + line) * Np + t0) * kC + cq;
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) orr[pt] = *reinterpret_cast<const u32x2*>(Ol + (size_t)(16 * pt + (l & 15)) * kC);
    const int t = t0 + p;
    if (t < N) {
      const TZ* zp = z + zpos(b, line, t) * kC + 16 * sp;
#pragma unroll
      for (int q = 0; q < ZL; ++q) zr[q] = *reinterpret_cast<const u32x4*>(zp + ZV * q);
    } else {
#pragma unroll
      for (int q = 0; q < ZL; ++q) zr[q] = u32x4{0u, 0u, 0u, 0u};
    }
  };

  // LayerNorm of a position's row (fp32 two-pass statistics over the 8 lanes of the
  // position) -> x_lds.
  auto layer_norm = [&](const u32x4 (&zz)[ZL]) __attribute__((always_inline)) {
    float zv[16];
#pragma unroll
    for (int q = 0; q < ZL; ++q) unpack16<TZ>(zz[q], *reinterpret_cast<float(*)[ZV]>(zv + ZV * q));
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) sum += zv[e];
    const float mean = dpp_sum8(sum) * (1.0f / kC);
    float sq = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float d = zv[e] - mean;
      sq += d * d;
    }
    const float rstd = rsqrtf(dpp_sum8(sq) * (1.0f / kC) + eps);
    float x[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 gw = lnq[0][q][sp], gb = lnq[1][q][sp];
#pragma unroll
      for (int e = 0; e < 4; ++e) x[4 * q + e] = (zv[4 * q + e] - mean) * rstd * gw[e] + gb[e];
    }
    store_vec<bf16, 8>(x_lds + p * ALD + 16 * sp, x);
    store_vec<bf16, 8>(x_lds + p * ALD + 16 * sp + 8, x + 8);
  };

  // Two barriers per tile: the next tile's LayerNorm runs between the output GEMM and the
  // residual, so one barrier publishes both it and the update. zc / oc: this tile's raw z
  // rows and O; zr / orr: the next tile's, loaded during this tile's gate GEMM.
  long tile = blockIdx.x;
  if (tile >= ntiles) return;  // block-uniform
  issue(tile);
  __syncthreads();  // LayerNorm parameters
  layer_norm(zr);
  u32x4 zc[ZL];
  u32x2 oc[4];
#pragma unroll
  for (int q = 0; q < ZL; ++q) zc[q] = zr[q];
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) oc[pt] = orr[pt];
  __syncthreads();  // x_lds complete
  for (;;) {
    int b, line, t0;
    tile_coords(tile, b, line, t0);
    const long next = tile + gridDim.x;
    if (next < ntiles) issue(next);

    // g^T = W_g LN(z)^T; a = O * sigmoid(g) -> a_lds [pos][ch].
    {
      f32x4 gacc[4];
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) gacc[pt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kC / 32; ++ks)
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) {
          const bf16x8 fx =
              *reinterpret_cast<const bf16x8*>(x_lds + (16 * pt + (l & 15)) * ALD + 32 * ks + 8 * (l >> 4));
          gacc[pt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wg[ks], fx, gacc[pt], 0, 0, 0);
        }
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) {
        const bf16x4 o4 = __builtin_bit_cast(bf16x4, oc[pt]);
        float a[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] = (float)o4[e] * sigmoidf_(gacc[pt][e]);
        store_vec<bf16, 4>(a_lds + (16 * pt + (l & 15)) * ALD + cq, a);
      }
    }
    __syncthreads();  // a_lds complete; x_lds and the previous tile's update no longer read

    f32x4 acc[4];
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) acc[pt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kC / 32; ++ks)
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) {
        const bf16x8 fa =
            *reinterpret_cast<const bf16x8*>(a_lds + (16 * pt + (l & 15)) * ALD + 32 * ks + 8 * (l >> 4));
        acc[pt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wo[ks], fa, acc[pt], 0, 0, 0);
      }
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) *reinterpret_cast<f32x4*>(upd + (16 * pt + (l & 15)) * SLD + cq) = acc[pt];
    if (next < ntiles) layer_norm(zr);
    __syncthreads();  // update and the next tile's x_lds complete; a_lds no longer read

    const int t = t0 + p;
    if (t < N) {
      TZ* op = out + zpos(b, line, t) * kC + 16 * sp;
      float zv[16];
      if (accumulate && !res_is_z) {  // residual stream other than z: read it here
#pragma unroll
        for (int q = 0; q < ZL; ++q) load16<TZ>(op + ZV * q, *reinterpret_cast<float(*)[ZV]>(zv + ZV * q));
      } else {
#pragma unroll
        for (int q = 0; q < ZL; ++q) unpack16<TZ>(zc[q], *reinterpret_cast<float(*)[ZV]>(zv + ZV * q));
      }
      float y[16];
#pragma unroll
      for (int e = 0; e < 16; e += 4) {
        const f32x4 u = *reinterpret_cast<const f32x4*>(upd + p * SLD + 16 * sp + e);
#pragma unroll
        for (int k = 0; k < 4; ++k) y[e + k] = accumulate ? zv[e + k] + u[k] : u[k];
      }
#pragma unroll
      for (int q = 0; q < ZL; ++q) store_vec<TZ, ZV>(op + ZV * q, y + ZV * q);
    }
    if (next >= ntiles) break;
    tile = next;
#pragma unroll
    for (int q = 0; q < ZL; ++q) zc[q] = zr[q];
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) oc[pt] = orr[pt];
  }
}

// Offsets of the operand buffers inside the workspace (bytes, 256-aligned).
struct AttnWs {
  size_t q, k, v, g, o, pb, ma, redo, total;
};

// Redo flags of the flash kernel: one int per wave, an upper bound over the query-block
// sizes (lines rounded up to whole blocks, 32-query blocks).
size_t redo_flag_bytes(int B, int L, int Np) {
  const size_t lines = pf::round_up((size_t)L, kLinesPerBlock);
  return (size_t)B * lines * kHeads * (Np / 32) * sizeof(int);
}

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
  w.g = cdtype == PF_F32 ? take(tok) : 0;  // the bf16 path computes the gate in the output kernel
  w.o = take(tok);
  w.pb = take((size_t)B * kHeads * Np * Np * 4);
  w.ma = take((size_t)B * Np * Np * 4);
  w.redo = take(redo_flag_bytes(B, N, (int)Np));
  w.total = off;
  return w;
}

template <class TZ, class TC>
int grid_attn_launch(const void* z, const float* mask, const float* lnw, const float* lnb, float eps, const void* w5,
                     const void* wo, int B, int N, int transpose, void* out, int accumulate, const float* key_mask,
                     void* ws, hipStream_t s) {
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
  int* redo = reinterpret_cast<int*>(base + L.redo);
  const float qscale = (1.0f / sqrtf((float)kHeadDim)) * kLog2e;
  constexpr int BM = block_rows<TC>();
  {
    dim3 grid(Np / BM, Np, B);
    pf::KernelTimer timer("attn_project", s);
    if constexpr (sizeof(TC) == 2) {
      const long ntiles = (long)B * Np * (Np / ProjectAttnWs::BP);
      const int nblk = (int)std::min<long>(ntiles, pf::cu_count());
      attn_project_ws_kernel<TZ><<<nblk, ProjectAttnWs::NT, 0, s>>>((const TZ*)z, mask, lnw, lnb, eps,
                                                                    (const bf16*)w5, Qb, Kb, Vb, PBb, MAb, B, N,
                                                                    Np, transpose, qscale);
      (void)grid;
    } else {
      attn_project_kernel<TZ, TC><<<grid, 256, 0, s>>>((const TZ*)z, mask, lnw, lnb, eps, (const TC*)w5, Qb, Kb,
                                                       Vb, Gb, PBb, MAb, N, Np, transpose, qscale);
    }
    timer.stop();
    if (int e = pf::check_launch("attn_project")) return e;
  }
  // Outer-product mask: its key mask goes into the pair bias (rows: a pass over the bias;
  // columns: inside the transpose).
  const bool mask_outer = key_mask != nullptr;
  if (mask_outer && !transpose) {
    const long n4 = (long)Np * Np / 4;
    const int gx = (int)std::min<long>((n4 + 255) / 256, (4L * pf::cu_count() + B * kHeads - 1) / (B * kHeads));
    pb_fold_kernel<<<dim3(std::max(gx, 1), B * kHeads), 256, 0, s>>>(PBb, key_mask, N, Np);
    if (int e = pf::check_launch("pb_fold")) return e;
  }
  if (transpose) {
    const int nt = Np / 32;
    pf::KernelTimer timer("pb_transpose", s);
    pb_transpose_kernel<<<dim3(nt * (nt + 1) / 2, B * kHeads), 256, 0, s>>>(PBb, Np, key_mask, N);
    timer.stop();
    if (int e = pf::check_launch("pb_transpose")) return e;
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
    // With an outer-product mask the key mask is in the bias: no per-line key-mask MFMA or
    // mask loads.
    if (mask_outer)
      tri_attn_kernel<TC, QS, false, true, false, false><<<grid, NT, attn_bias_lds_bytes<TC>(), s>>>(
          Qb, Kb, Vb, PBb, MAb, Ob, B, N, Np, N, Np, 0, remap, redo);
    else
      tri_attn_kernel<TC, QS, false, true><<<grid, NT, attn_bias_lds_bytes<TC>(), s>>>(
          Qb, Kb, Vb, PBb, MAb, Ob, B, N, Np, N, Np, 0, remap, redo);
    timer.stop();
    if (int e = pf::check_launch("tri_attn")) return e;
    pf::KernelTimer timer2("tri_attn_redo", s);
    if (mask_outer)
      tri_attn_kernel<TC, QS, false, false, false, false><<<grid, NT, attn_bias_lds_bytes<TC>(), s>>>(
          Qb, Kb, Vb, PBb, MAb, Ob, B, N, Np, N, Np, 0, remap, redo);
    else
      tri_attn_kernel<TC, QS, false, false><<<grid, NT, attn_bias_lds_bytes<TC>(), s>>>(
          Qb, Kb, Vb, PBb, MAb, Ob, B, N, Np, N, Np, 0, remap, redo);
    timer2.stop();
    if (int e = pf::check_launch("tri_attn_redo")) return e;
  }
  {
    dim3 grid((N + BM - 1) / BM, N, B);
    pf::KernelTimer timer("attn_out", s);
    if constexpr (sizeof(TC) == 2) {
      const long ntiles = (long)B * N * ((N + OutAttnWs::BP - 1) / OutAttnWs::BP);
      const int nblk = (int)std::min<long>(ntiles, 2L * pf::cu_count());
      // The gate rows are kind 3 of the packed projection weights.
      const bf16* wg = (const bf16*)w5 + (size_t)3 * kC * kC;
      attn_out_ws_kernel<TZ><<<nblk, OutAttnWs::NT, 0, s>>>(Ob, wg, (const bf16*)wo, (const TZ*)z, lnw, lnb, eps,
                                                            (TZ*)out, B, N, Np, transpose, accumulate,
                                                            out == z ? 1 : 0);
      (void)grid;
    } else {
      attn_out_kernel<TZ, TC><<<grid, 256, 0, s>>>(Ob, Gb, (const TC*)wo, (TZ*)out, N, Np, transpose, accumulate);
    }
    timer.stop();
    if (int e = pf::check_launch("attn_out")) return e;
  }
  return pf::ok();
}

// Whether every pair mask [b][N][N] is the outer product of its binary diagonal (the
// case folded_key_mask serves): the flag starts at 1 and any element that breaks
// m[i][k] = m[i][i] m[k][k] with m in {0, 1} clears it (every writer stores the same 0).
// The init pass also writes the additive key mask of the diagonal, km[b][k] = 1e9 (m[k][k] - 1).
__global__ __launch_bounds__(256) void mask_outer_init_kernel(const float* __restrict__ mask, int B, int N,
                                                              int* __restrict__ flag, float* __restrict__ km) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx == 0) flag[0] = 1;
  if (idx < B * N) {
    const int b = idx / N, k = idx % N;
    km[idx] = (mask[((size_t)b * N + k) * N + k] - 1.0f) * 1e9f;
  }
}

__global__ __launch_bounds__(256) void mask_outer_check_kernel(const float* __restrict__ mask, int B, int N,
                                                               int* __restrict__ flag) {
  const long total = (long)B * N * N;
  for (long idx = (long)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (long)gridDim.x * 256) {
    const long b = idx / ((long)N * N);
    const long rem = idx - b * N * N;
    const long i = rem / N, k = rem - i * N;
    const float* mb = mask + b * N * N;
    const float m = mb[idx - b * N * N];
    const float di = mb[i * N + i], dk = mb[k * N + k];
    const bool ok = (m == 0.f || m == 1.f) && m == di * dk;
    if (!ok) flag[0] = 0;
  }
}

// ------------------------------------------------------------------ kernel-level op
// _EvoformerAttention.apply(Q, K, V, res_mask, pair_bias, pre_transposed=True)
// (triton/evo_attention.py:1198-1292): O = softmax(Q K^T d^-1/2 + pair_bias + res_mask) V
// per (batch, line, head) with Q, K, V, O as [B][S][H][N][D], res_mask additive [B][S][N],
// pair_bias [B][H][N][N] fp32. The operands are repacked into the attention frame (padded
// to Np, V transposed with the key-slot order) and run through the same flash kernel. In
// bf16 the kernel applies the fp32 post-scale the reference kernel uses
// (evo_attention.py:100-109): Q is copied as given, the bias and mask are stored times
// d^1/2, and the kernel multiplies the fp32 logit accumulator by d^-1/2 log2 e after the
// q k^T products (a pre-scaled Q re-rounded to bf16 would perturb a logit by ~2^-9 of its
// size). In fp32, Q is pre-scaled by d^-1/2 log2 e (one fp32 rounding) and the bias and mask
// are stored times log2 e, which keeps large biases at their own fp32 precision.
// -inf mask entries become -1e9.
template <class TC>
__global__ __launch_bounds__(256) void evo_pack_qk_kernel(const TC* __restrict__ q, const TC* __restrict__ k,
                                                          TC* __restrict__ Qw, TC* __restrict__ Kw, int S, int N,
                                                          int Np, float qscale, Strides4 sx) {
  constexpr int VEC = 16 / sizeof(TC);
  constexpr int CPT = kHeadDim / VEC;  // chunks per token
  const size_t bsh = blockIdx.y;       // (b, s, h) flattened
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= Np * CPT) return;
  const int t = idx / CPT;
  const int d0 = (idx % CPT) * VEC;
  float vq[VEC], vk[VEC];
  if (t < N) {
    const long off = (long)(bsh / ((size_t)S * kHeads)) * sx.b + (long)((bsh / kHeads) % S) * sx.s +
                     (long)(bsh % kHeads) * sx.h + (long)t * sx.n + d0;
    load16<TC>(q + off, vq);
    load16<TC>(k + off, vk);
#pragma unroll
    for (int e = 0; e < VEC; ++e) vq[e] *= qscale;
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) vq[e] = vk[e] = 0.f;
  }
  store_vec<TC, VEC>(Qw + (bsh * Np + t) * kHeadDim + d0, vq);
  if constexpr (sizeof(TC) == 2)  // key-block tiles (kv_chunk)
    store_vec<TC, VEC>(Kw + (bsh * Np + (t & ~31)) * kHeadDim + 8 * kv_chunk(t & 31, d0 / 8), vk);
  else
    store_vec<TC, VEC>(Kw + (bsh * Np + t) * kHeadDim + d0, vk);
}

// One block per (32-key block, b s h): V[t][d] -> Vt[d][slot] (bf16: the key-block tile).
template <class TC>
__global__ __launch_bounds__(256) void evo_pack_v_kernel(const TC* __restrict__ v, TC* __restrict__ Vt, int S,
                                                         int N, int Np, Strides4 sx) {
  __shared__ float tile[32][kHeadDim + 1];
  const size_t bsh = blockIdx.y;
  const int k0 = blockIdx.x * 32;
  const TC* vl = v + (long)(bsh / ((size_t)S * kHeads)) * sx.b + (long)((bsh / kHeads) % S) * sx.s +
                 (long)(bsh % kHeads) * sx.h;
  for (int i = threadIdx.x; i < 32 * kHeadDim; i += 256) {
    const int t = i / kHeadDim, d = i % kHeadDim;
    tile[t][d] = (k0 + t < N) ? to_f32(vl[(long)(k0 + t) * sx.n + d]) : 0.f;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 32 * kHeadDim; i += 256) {
    const int d = i / 32, slot = i % 32;
    const TC v = from_f32<TC>(tile[slot_key(slot)][d]);
    if constexpr (sizeof(TC) == 2)
      Vt[(bsh * Np + k0) * kHeadDim + 8 * kv_chunk(d, slot / 8) + slot % 8] = v;
    else
      Vt[(bsh * kHeadDim + d) * Np + k0 + slot] = v;
  }
}

__global__ __launch_bounds__(256) void evo_pack_bias_kernel(const float* __restrict__ pb, float* __restrict__ PB,
                                                            int N, int Np, float scale) {
  const size_t bh = blockIdx.y;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)Np * Np) return;
  const int qi = (int)(idx / Np);
  const int sl = (int)(idx % Np);
  const int kk = (sl & ~31) + slot_key(sl & 31);
  PB[bh * Np * Np + idx] = (qi < N && kk < N) ? pb[(bh * N + qi) * N + kk] * scale : 0.f;
}

__global__ __launch_bounds__(256) void evo_pack_mask_kernel(const float* __restrict__ rm, float* __restrict__ MA,
                                                            int N, int Np, float scale) {
  const size_t bs = blockIdx.y;
  const int sl = blockIdx.x * 256 + threadIdx.x;
  if (sl >= Np) return;
  const int kk = (sl & ~31) + slot_key(sl & 31);
  float v = -INFINITY;
  if (kk < N) v = fmaxf(rm[bs * N + kk], -1e9f) * scale;
  MA[bs * Np + sl] = v;
}

struct EvoWs {
  size_t q, k, v, pb, ma, redo, total;
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
  w.redo = take(redo_flag_bytes(B, S, (int)Np));
  w.total = off;
  return w;
}

// softmax_scale multiplies q k^T (the reference's d^-1/2; a caller whose heads are zero-padded
// to 32 dimensions passes its own head dimension's).
template <class TC>
int evo_attn_launch(const void* q, const void* k, const void* v, const float* res_mask, const float* pair_bias, int B,
                    int S, int N, int zero_rule, void* out, void* ws, hipStream_t s,
                    float softmax_scale = 1.0f / sqrtf((float)kHeadDim), const Strides4* sx_in = nullptr,
                    const Strides4* so_in = nullptr, float* lse_out = nullptr) {
  const Strides4 sx = sx_in ? *sx_in
                            : Strides4{(long)S * kHeads * N * kHeadDim, (long)kHeads * N * kHeadDim,
                                       (long)N * kHeadDim, kHeadDim};
  const Strides4 so = so_in ? *so_in : Strides4{};
  const int Np = (int)pf::round_up((size_t)N, kPad);
  const EvoWs L = evo_ws_layout(B, S, N, sizeof(TC) == 4 ? PF_F32 : PF_BF16);
  char* base = reinterpret_cast<char*>(ws);
  TC* Qw = reinterpret_cast<TC*>(base + L.q);
  TC* Kw = reinterpret_cast<TC*>(base + L.k);
  TC* Vw = reinterpret_cast<TC*>(base + L.v);
  float* PBw = reinterpret_cast<float*>(base + L.pb);
  float* MAw = reinterpret_cast<float*>(base + L.ma);
  int* redo = reinterpret_cast<int*>(base + L.redo);
  // logit (log2 units): bf16 post * (q k^T + (bias + mask) d^1/2) with post = d^-1/2 log2 e;
  // fp32 (q d^-1/2 log2 e) k^T + (bias + mask) log2 e.
  constexpr bool kPost = sizeof(TC) == 2;
  const float qscale = kPost ? 1.f : softmax_scale * kLog2e;
  const float bscale = kPost ? 1.f / softmax_scale : kLog2e;
  const float post = softmax_scale * kLog2e;
  const unsigned bsh = (unsigned)(B * S * kHeads);
  constexpr int VEC = 16 / sizeof(TC);
  evo_pack_qk_kernel<TC><<<dim3((Np * (kHeadDim / VEC) + 255) / 256, bsh), 256, 0, s>>>(
      (const TC*)q, (const TC*)k, Qw, Kw, S, N, Np, qscale, sx);
  evo_pack_v_kernel<TC><<<dim3(Np / 32, bsh), 256, 0, s>>>((const TC*)v, Vw, S, N, Np, sx);
  evo_pack_bias_kernel<<<dim3((unsigned)(((long)Np * Np + 255) / 256), B * kHeads), 256, 0, s>>>(pair_bias, PBw,
                                                                                                   N, Np, bscale);
  evo_pack_mask_kernel<<<dim3((Np + 255) / 256, B * S), 256, 0, s>>>(res_mask, MAw, N, Np, bscale);
  if (int e = pf::check_launch("evo_attn pack")) return e;
  constexpr int QS = attn_qsub<TC>();
  constexpr int NT = 64 * kLinesPerBlock;
  const int nqb = Np / (32 * QS);
  const int nlg = (S + kLinesPerBlock - 1) / kLinesPerBlock;
  const long total = (long)B * nlg * kHeads * nqb;
  const int remap = (total % 8 == 0) ? 1 : 0;
  pf::KernelTimer timer("evo_attn", s);
  tri_attn_kernel<TC, QS, true, true, kPost><<<dim3((unsigned)total), NT, attn_bias_lds_bytes<TC>(), s>>>(
      Qw, Kw, Vw, PBw, MAw, (TC*)out, B, N, Np, S, S, zero_rule, remap, redo, post, so, lse_out);
  if (int e = pf::check_launch("evo_attn")) return e;
  tri_attn_kernel<TC, QS, true, false, kPost><<<dim3((unsigned)total), NT, attn_bias_lds_bytes<TC>(), s>>>(
      Qw, Kw, Vw, PBw, MAw, (TC*)out, B, N, Np, S, S, zero_rule, remap, redo, post, so, lse_out);
  timer.stop();
  return pf::check_launch("evo_attn redo");
}

// ------------------------------------------------------------------ generic channels / heads
// GridSelfAttention for (C, H) other than (128, 4): the template stack's 64 channels in 4
// heads of 16 and the 256-channel trunk's 8 heads of 32 (attention.py:56-269, head dim
// max(C / H, 16), at most 32 here). Composed from the row kernels and the flash kernel:
// LN(z) -> [q | k | v | g | pair bias] projection -> pack into groups of four heads, the head
// dimension zero-padded to 32 (the logits and outputs are those of the real dimensions),
// the line mask 1e9 (m - 1) and the pair bias [h][q][k] of the un-transposed positions ->
// the flash kernel per group with the real head dimension's softmax scale (eager masked-line
// rule) -> o * sigmoid(g) back in z order -> out_proj, stored or added into `out`.
struct GridGenWs {
  size_t xn, proj, q, k, v, pb, ma, o, og, evo, total;
};

int grid_gen_head_dim(int C, int H) { return std::max(C / H, 16); }

GridGenWs grid_gen_layout(int B, int N, int C, int H, int cdtype) {
  const size_t es = cdtype == PF_F32 ? 4 : 2;
  const int d = grid_gen_head_dim(C, H);
  const int H4 = (H + 3) / 4 * 4;
  const size_t M = (size_t)B * N * N;
  const size_t heads = (size_t)B * N * H4 * N * kHeadDim * es;  // [group][b][line][4][N][32]
  GridGenWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += pf::round_up(bytes, 256);
    return at;
  };
  w.xn = take(M * C * es);
  w.proj = take(M * (size_t)(4 * H * d + 16) * es);
  w.q = take(heads);
  w.k = take(heads);
  w.v = take(heads);
  w.pb = take((size_t)B * H4 * N * N * 4);
  w.ma = take((size_t)B * N * N * 4);
  w.o = take(heads);
  w.og = take(M * (size_t)H * d * es);
  w.evo = take(evo_ws_layout(B, N, N, cdtype).total);
  w.total = off;
  return w;
}

// One thread per (position, head, 8-wide chunk of the 32-wide padded head dimension): the
// chunk runs fastest, then the head (count padded to a multiple of four; padding heads and
// dimensions are zero), then the position, so the reads of a position's q / k / v columns
// and the 16-byte stores of a head row are contiguous across the wave. Position (b, x, y)
// of z: row mode line x, token y; column mode line y, token x. The pair bias is that of
// position (x, y) in both modes (attention.py:204-209).
template <class TC>
__global__ __launch_bounds__(256) void grid_gen_pack_kernel(const TC* __restrict__ proj, const float* __restrict__ mask,
                                                            TC* __restrict__ Q, TC* __restrict__ K, TC* __restrict__ V,
                                                            float* __restrict__ PB, float* __restrict__ MA, int B, int N,
                                                            int H, int H4, int d, int PW, int transpose) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  const long M = (long)B * N * N;
  if (idx >= M * H4 * 4) return;
  const int c = (int)(idx & 3);
  const int h = (int)((idx >> 2) % H4);
  const long pos = (idx >> 2) / H4;
  const int b = (int)(pos / ((long)N * N));
  const int x = (int)((pos / N) % N), y = (int)(pos % N);
  const int line = transpose ? y : x, tok = transpose ? x : y;
  const int g = h / 4, hh = h % 4;
  const size_t head = (((((size_t)g * B + b) * N + line) * 4 + hh) * N + tok) * kHeadDim + 8 * c;
  const TC* row = proj + pos * PW;
  const int HD = H * d;
  float q[8], k[8], v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int dd = 8 * c + e;
    const bool real = h < H && dd < d;
    q[e] = real ? to_f32(row[h * d + dd]) : 0.f;
    k[e] = real ? to_f32(row[HD + h * d + dd]) : 0.f;
    v[e] = real ? to_f32(row[2 * HD + h * d + dd]) : 0.f;
  }
  store_vec<TC, 8>(Q + head, q);
  store_vec<TC, 8>(K + head, k);
  store_vec<TC, 8>(V + head, v);
  if (c == 0) PB[(((size_t)g * B + b) * 4 + hh) * N * N + (size_t)x * N + y] = h < H ? to_f32(row[4 * HD + h]) : 0.f;
  if (c == 0 && h == 0) MA[((size_t)b * N + line) * N + tok] = (mask[pos] - 1.0f) * 1e9f;
}

// og[pos][h d + e] = o * sigmoid(g) for the real heads and dimensions, in z position order.
// VEC = 8 (head dimension a multiple of 8): one thread per 8-wide chunk, chunk fastest, with
// 16-byte stores; VEC = 1: one thread per element.
template <class TC, int VEC>
__global__ __launch_bounds__(256) void grid_gen_gate_kernel(const TC* __restrict__ O, const TC* __restrict__ proj,
                                                            TC* __restrict__ og, int B, int N, int H, int d, int PW,
                                                            int transpose) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  const int HD = H * d;
  const int nc = d / VEC;
  if (idx >= (long)B * N * N * H * nc) return;
  const int e0 = (int)(idx % nc) * VEC;
  const int h = (int)((idx / nc) % H);
  const long pos = idx / ((long)nc * H);
  const int b = (int)(pos / ((long)N * N));
  const int x = (int)((pos / N) % N), y = (int)(pos % N);
  const int line = transpose ? y : x, tok = transpose ? x : y;
  const size_t head = (((((size_t)(h / 4) * B + b) * N + line) * 4 + h % 4) * N + tok) * kHeadDim + e0;
  const TC* gr = proj + pos * PW + 3 * HD + h * d + e0;
  float r[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) r[e] = to_f32(O[head + e]) * sigmoidf_(to_f32(gr[e]));
  store_vec<TC, VEC>(og + pos * HD + h * d + e0, r);
}

// The pair bias and the line mask of the strided path: one thread per (position, head of the
// four-head groups), PB [g][b][hh][x][y] fp32 (zero for padding heads) and MA [b][line][tok].
template <class TC>
__global__ __launch_bounds__(256) void grid_gen_bias_kernel(const TC* __restrict__ proj, const float* __restrict__ mask,
                                                            float* __restrict__ PB, float* __restrict__ MA, int B, int N,
                                                            int H, int H4, int d, int PW, int transpose) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  const long M = (long)B * N * N;
  if (idx >= M * H4) return;
  const int h = (int)(idx % H4);
  const long pos = idx / H4;
  const int b = (int)(pos / ((long)N * N));
  const int x = (int)((pos / N) % N), y = (int)(pos % N);
  PB[(((size_t)(h / 4) * B + b) * 4 + h % 4) * N * N + (size_t)x * N + y] =
      h < H ? to_f32(proj[pos * PW + 4 * H * d + h]) : 0.f;
  if (h == 0) {
    const int line = transpose ? y : x, tok = transpose ? x : y;
    MA[((size_t)b * N + line) * N + tok] = (mask[pos] - 1.0f) * 1e9f;
  }
}

// og[pos][j] *= sigmoid(g[pos][j]) in place, g the columns from `goff` of rows of PW
// elements (the gate columns of the projection); 8 columns per thread (H d a multiple of 8).
template <class TC>
__global__ __launch_bounds__(256) void grid_gen_gate_inplace_kernel(TC* __restrict__ og, const TC* __restrict__ proj,
                                                                    long M, int HD, int PW, int goff) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  const int nc = HD / 8;
  if (idx >= M * nc) return;
  const long pos = idx / nc;
  const int j = (int)(idx % nc) * 8;
  TC* o = og + pos * HD + j;
  const TC* g = proj + pos * PW + goff + j;
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = to_f32(o[e]) * sigmoidf_(to_f32(g[e]));
  store_vec<TC, 8>(o, r);
}

// ------------------------------------------------------------------ 256 channels, 8 heads
// GridSelfAttention at 256 channels in 8 heads of 32 with bf16 GEMMs (the reference's
// production width, configs/stage0.yaml:54-56): one persistent projection kernel writes the
// flash kernel's frame for both four-head groups -- Q (pre-scaled by d^-1/2 log2 e), the K
// and Vt key-block tiles, the pair bias (log2 units; query-major in key-slot order for rows,
// key-major for columns, turned by pb_transpose) and the line mask -- plus the gate rows
// sigmoid(g) as G [pos][256] in z order; then per group the flash kernel (o into og's rows,
// strided), and the output GEMM on og * G (the gate applied as its operand tile loads). No
// LayerNorm round trip, no projection rows, no repacking.
//
// The projection: one 8-wave block per CU walks tiles of 128 tokens of one line (the z
// positions (line, t) for rows, (t, line) for columns). A position's LayerNormed 256
// channels are held in registers as the B operand for the whole tile (lanes l and l ^ 32);
// the packed rows of w_qkvgb (q | k | v | g, 256 each, then the 8 bias rows) stream through
// a two-stage LDS ring in 64-row chunks (32 KB, XOR-swizzled 16-byte pieces) by direct
// buffer->LDS loads one chunk ahead, 16 q/k/v/g chunks (two heads each) and one bias chunk.
// Wave w computes rows 32 (w & 1) .. of each chunk for tokens 32 (w >> 1) ..; the values
// go through a double-buffered LDS stage in the layout their destination needs (token-major
// for Q, K and G, d-major in key-slot order for Vt, head-major for the bias) and leave as
// 16-byte pieces one chunk later, while the next tile's z rows load under this tile's chunks.
struct GridProj256 {
  static constexpr int C = 256;
  static constexpr int H = 8;
  static constexpr int HD = 256;                  // H x 32
  static constexpr int WROWS = 4 * HD + 16;       // rows of w_qkvgb (8 bias rows, 8 zero rows)
  static constexpr int BP = 128;                  // tokens per tile
  static constexpr int NW = 8;
  static constexpr int NT = 64 * NW;
  static constexpr int CR = 64;                   // weight rows per chunk
  static constexpr int NCH = 4 * HD / CR + 1;     // 16 head chunks + the bias chunk
  static constexpr int ROWB = C * 2;              // 512-byte weight rows
  static constexpr int CHUNK = CR * ROWB;         // 32 KB
  static constexpr int NS = 2;                    // ring stages (one chunk ahead)
  static constexpr int DMA = CHUNK / 1024 / NW;   // direct loads per wave per chunk
  static constexpr int TLD = 40;                  // token-major stage rows: 32 d + pad (bf16)
  static constexpr int VLD = BP + 8;              // d-major stage rows (bf16)
  static constexpr int STAGE = 2 * BP * TLD * 2;  // bytes per stage buffer (largest layout)
  static_assert(2 * 32 * VLD * 2 <= STAGE && 8 * BP * 4 <= STAGE, "stage layouts");
};

// Byte offset of logical 16-byte piece c (0..31) of 512-byte weight row r: the piece index's
// low four bits XOR the row's, so 16 consecutive rows at one logical piece spread over the
// 16 bank groups.
PF_DEVICE int gp256_off(int r, int c) { return r * GridProj256::ROWB + 16 * (c ^ (r & 15)); }

// Frame of the 256-channel path inside the workspace: per group of four heads, Q, K and Vt
// [B][N lines][4][Np][32] bf16 and the pair bias [B][4][Np][Np] fp32; one line mask
// [B][N][Np]; the gate rows and og [B N N][256] bf16; the redo flags of both groups.
struct Grid256Ws {
  size_t q, k, v, pb, ma, g, og, redo, total;
  size_t gq, gpb, gredo;  // per-group strides (elements of Q / K / Vt, floats of PB, ints)
};

Grid256Ws grid256_layout(int B, int N) {
  const size_t Np = pf::round_up((size_t)N, kPad);
  const size_t M = (size_t)B * N * N;
  Grid256Ws w;
  w.gq = (size_t)B * N * 4 * Np * kHeadDim;
  w.gpb = (size_t)B * 4 * Np * Np;
  w.gredo = redo_flag_bytes(B, N, (int)Np) / sizeof(int);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += pf::round_up(bytes, 256);
    return at;
  };
  w.q = take(2 * w.gq * 2);
  w.k = take(2 * w.gq * 2);
  w.v = take(2 * w.gq * 2);
  w.pb = take(2 * w.gpb * 4);
  w.ma = take((size_t)B * N * Np * 4);
  w.g = take(M * GridProj256::HD * 2);
  w.og = take(M * GridProj256::HD * 2);
  w.redo = take(2 * w.gredo * sizeof(int));
  w.total = off;
  return w;
}

bool grid256_applies(int C, int H, int cdtype) { return C == GridProj256::C && H == GridProj256::H && cdtype == PF_BF16; }

template <class TZ>
__global__ __launch_bounds__(GridProj256::NT, 1) void grid_project256_kernel(
    const TZ* __restrict__ z, const float* __restrict__ mask, const float* __restrict__ lnw,
    const float* __restrict__ lnb, float eps, const bf16* __restrict__ w5, bf16* __restrict__ Q,
    bf16* __restrict__ K, bf16* __restrict__ Vt, float* __restrict__ PB, float* __restrict__ MA,
    bf16* __restrict__ G, int B, int N, int Np, int transpose, float qscale, size_t gq, size_t gpb) {
  using Cfg = GridProj256;
  constexpr int C = Cfg::C, BP = Cfg::BP, NCH = Cfg::NCH, NS = Cfg::NS, TLD = Cfg::TLD, VLD = Cfg::VLD;
  // The rows are loaded at the start of their tile: holding the next tile's rows through the
  // chunks (64 VGPRs) spills, and each spill reload waits for every load in flight.
  constexpr bool PREFETCH = false;
  constexpr int NPIECE = C / 16 * (int)sizeof(TZ) / 2;  // 16-byte loads of a lane's half row
  __shared__ __attribute__((aligned(16))) char ring[NS * Cfg::CHUNK];
  __shared__ __attribute__((aligned(16))) char stage[2][Cfg::STAGE];
  __shared__ float lnp[2 * C];

  const int w = wave_id();
  const int l = lane_id();
  const int lq = l & 31, hf = l >> 5;
  const int rb = w & 1;   // rows 32 rb .. of each chunk
  const int pb = w >> 1;  // tokens 32 pb ..
  const int NT1 = Np / BP;
  const long ntiles = (long)B * N * NT1;
  const size_t NN = (size_t)N * N;
  const long total = blockIdx.x < ntiles ? ((ntiles - 1 - blockIdx.x) / gridDim.x + 1) * NCH : 0;

  for (int i = threadIdx.x; i < C; i += Cfg::NT) {
    lnp[i] = lnw[i];
    lnp[C + i] = lnb[i];
  }

  const i32x4_t rw = buf_rsrc_words(w5, Cfg::WROWS * C * 2);
  auto issue_chunk = [&](long gg) {
    const int c = (int)(gg % NCH);
    char* st = ring + (gg % NS) * Cfg::CHUNK;
#pragma unroll
    for (int t = 0; t < Cfg::DMA; ++t) {
      const int ins = w * Cfg::DMA + t;  // two 512-byte rows per instruction
      const int row = 2 * ins + (l >> 5);
      const int lc = (l & 31) ^ (row & 15);
      // the bias chunk's rows past the packed weights repeat its last row (never used)
      const int src = min(c * Cfg::CR + row, Cfg::WROWS - 1);
      buf_load_lds16_async(rw, st + ins * 1024, (src * C + 8 * lc) * 2, 0);
    }
  };
  auto tile_pos = [&](long tl, int& b, int& line, int& t0) {
    b = (int)(tl / ((long)N * NT1));
    const long r = tl - (long)b * N * NT1;
    line = (int)(r / NT1);
    t0 = (int)(r - (long)line * NT1) * BP;
  };
  auto zpos = [&](int line, int t) { return transpose ? (size_t)t * N + line : (size_t)line * N + t; };
  // this lane's half row of tile tl: channels 16 ks + 8 hf .. +7, ks = 0..15 (zeros past N)
  u32x4 zr[NPIECE];
  auto load_half = [&](long tl) {
    int b, line, t0;
    tile_pos(tl, b, line, t0);
    const int t = t0 + 32 * pb + lq;
    const TZ* src = t < N ? z + ((size_t)b * NN + zpos(line, t)) * C + 8 * hf : nullptr;
#pragma unroll
    for (int ks = 0; ks < C / 16; ++ks) {
      if constexpr (sizeof(TZ) == 2) {
        zr[ks] = src ? *reinterpret_cast<const u32x4*>(src + 16 * ks) : u32x4{0u, 0u, 0u, 0u};
      } else {
        zr[2 * ks] = src ? *reinterpret_cast<const u32x4*>(src + 16 * ks) : u32x4{0u, 0u, 0u, 0u};
        zr[2 * ks + 1] = src ? *reinterpret_cast<const u32x4*>(src + 16 * ks + 4) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto get = [&](int ks, float (&v)[8]) {
    if constexpr (sizeof(TZ) == 2) {
      const bf16x8 t = __builtin_bit_cast(bf16x8, zr[ks]);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (float)t[e];
    } else {
      const f32x4 a = __builtin_bit_cast(f32x4, zr[2 * ks]), c4 = __builtin_bit_cast(f32x4, zr[2 * ks + 1]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = a[e];
        v[4 + e] = c4[e];
      }
    }
  };
  // Chunk gg's staged values -> their destination (tile b, line, t0). Chunk c < 16 holds
  // part c / 4 (q, k, v, g) of heads 2 (c % 4) + rb; chunk 16 the bias of the 8 heads.
  auto store_chunk = [&](long gg, int b, int line, int t0) {
    const int c = (int)(gg % NCH);
    const char* sb = stage[gg & 1];
    const int idx = threadIdx.x;
    if (c == NCH - 1) {
      // bias: 8 heads x 32 pieces of 4 floats; row `line` of [b][head][Np][Np] in both modes
      if (idx < 256) {
        const int h8 = idx >> 5, p4 = idx & 31;
        float* dst = PB + (h8 >> 2) * gpb + (((size_t)b * 4 + (h8 & 3)) * Np + line) * Np + t0 + 4 * p4;
        *reinterpret_cast<f32x4*>(dst) = *reinterpret_cast<const f32x4*>(sb + (h8 * BP + 4 * p4) * 4);
      }
      return;
    }
    const int part = c >> 2, hp = c & 3;
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const int pc = idx + 512 * k2;
      const int r2 = pc >> 9;  // rb of the staged rows
      const int head = 2 * hp + r2;
      const size_t bsh = ((size_t)b * N + line) * 4 + (head & 3);
      const size_t grp = (size_t)(head >> 2) * gq;
      if (part == 0 || part == 3) {
        const int tok = (pc >> 2) & (BP - 1), c4 = pc & 3;
        const u32x4 v = *reinterpret_cast<const u32x4*>(sb + ((r2 * BP + tok) * TLD + 8 * c4) * 2);
        if (part == 0) {
          *reinterpret_cast<u32x4*>(Q + grp + (bsh * Np + t0 + tok) * kHeadDim + 8 * c4) = v;
        } else if (t0 + tok < N) {
          *reinterpret_cast<u32x4*>(G + ((size_t)b * NN + zpos(line, t0 + tok)) * Cfg::HD + head * kHeadDim +
                                    8 * c4) = v;
        }
      } else {
        // key-block tiles: piece pi = 32 cc + row of block kb, cc = 2 (c8 & 1) + (c8 >> 1)
        const int kb = (pc >> 7) & 3, pi = pc & 127;
        const int row = pi & 31, cc = pi >> 5;
        const int c8 = ((cc & 1) << 1) | (cc >> 1);
        const size_t dst = grp + (bsh * Np + t0 + 32 * kb) * kHeadDim + 8 * pi;
        if (part == 1)  // K: 8 dims of token 32 kb + row
          *reinterpret_cast<u32x4*>(K + dst) =
              *reinterpret_cast<const u32x4*>(sb + ((r2 * BP + 32 * kb + row) * TLD + 8 * c8) * 2);
        else  // Vt: dim `row`, slots 8 c8 .. of block kb
          *reinterpret_cast<u32x4*>(Vt + dst) =
              *reinterpret_cast<const u32x4*>(sb + ((r2 * 32 + row) * VLD + 32 * kb + 8 * c8) * 2);
      }
    }
  };

  long g = 0;
  long tile = blockIdx.x;
  int sbb = 0, sline = 0, st0 = 0;  // tile of the chunk waiting in the stage
  if (total > 0) {
    if (PREFETCH) load_half(tile);
    issue_chunk(0);
  }
  __syncthreads();  // LN parameters

  for (; tile < ntiles; tile += gridDim.x) {
    int b, line, t0;
    tile_pos(tile, b, line, t0);
    const int tpos = t0 + 32 * pb + lq;
    const bool live = tpos < N;
    const float mk = live ? mask[(size_t)b * NN + zpos(line, tpos)] : 0.f;
    if (!PREFETCH) load_half(tile);  // fp32 rows: loaded per tile, dead after the LayerNorm
    // the line mask of this tile's keys (log2 units; -inf past N)
    if (rb == 0 && hf == 0)
      MA[((size_t)b * N + line) * Np + t0 + 32 * pb + key_slot(lq)] =
          live ? (mk - 1.0f) * 1e9f * kLog2e : -INFINITY;

    // ---- LN -> B operands xf[ks]: channels 16 ks + 8 hf .. +7
    bf16x8 xf[C / 16];
    {
      float s = 0.f;
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        float v[8];
        get(ks, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) s += v[e];
      }
      s += __shfl_xor(s, 32, 64);
      const float mean = s * (1.0f / C);
      float q = 0.f;
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        float v[8];
        get(ks, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = v[e] - mean;
          q += d * d;
        }
      }
      q += __shfl_xor(q, 32, 64);
      const float rstd = rsqrtf(q * (1.0f / C) + eps);
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        float v[8];
        get(ks, v);
        const float* pw = lnp + 16 * ks + 8 * hf;
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[ks][e] = (bf16)((v[e] - mean) * rstd * pw[e] + pw[C + e]);
      }
    }
    const bool more = tile + gridDim.x < ntiles;

#pragma unroll 1
    for (int c = 0; c < NCH; ++c, ++g) {
      // Chunk g's weights landed in every wave. Past the barrier, ring slot (g + 1) % NS (read
      // by chunk g - 1's MFMAs) takes chunk g + 1, and stage (g - 1) & 1 leaves for its
      // destination before chunk g + 1's barrier lets it be rewritten.
      __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
      lds_barrier();
      if (g > 0) store_chunk(g - 1, sbb, sline, st0);
      if (PREFETCH && c == 1 && more) load_half(tile + gridDim.x);  // zr is free after LN
      if (g + NS - 1 < total) issue_chunk(g + NS - 1);
      if (c < NCH - 1 || rb == 0) {  // the bias chunk's rows 32 .. are empty
        const char* st = ring + (g % NS) * Cfg::CHUNK;
        f32x16 acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
        for (int ks = 0; ks < C / 16; ++ks) {
          const bf16x8 wf = *reinterpret_cast<const bf16x8*>(st + gp256_off(32 * rb + lq, 2 * ks + hf));
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, xf[ks], acc, 0, 0, 0);
        }
        // acc[e]: chunk row 32 rb + 8 (e >> 2) + 4 hf + (e & 3), token 32 pb + lq
        char* sb = stage[g & 1];
        const int tok = 32 * pb + lq;
        const int part = c >> 2;
        if (c == NCH - 1) {
          // bias rows 0..7 (heads 4 hf + e): head-major, key-slot order for rows
          const int col = transpose ? tok : 32 * pb + key_slot(lq);
          float* bs = reinterpret_cast<float*>(sb);
#pragma unroll
          for (int e = 0; e < 4; ++e) bs[(4 * hf + e) * BP + col] = live ? acc[e] * kLog2e : 0.f;
        } else if (part == 2) {
          // Vt: [rb][d][slot] (zero past N)
          bf16* vs = reinterpret_cast<bf16*>(sb) + rb * 32 * VLD;
          const int slot = 32 * pb + key_slot(lq);
#pragma unroll
          for (int e = 0; e < 16; ++e) vs[(8 * (e >> 2) + 4 * hf + (e & 3)) * VLD + slot] = (bf16)(live ? acc[e] : 0.f);
        } else {
          // Q (scaled), K, sigmoid(G): [rb][token][d] (Q and K zero past N)
          const float sc = part == 0 ? qscale : 1.0f;
          const float keep = live ? sc : 0.f;
          bf16* ts = reinterpret_cast<bf16*>(sb) + (rb * BP + tok) * TLD;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            bf16x4 v4;
            if (part == 3) {
#pragma unroll
              for (int e = 0; e < 4; ++e) v4[e] = (bf16)sigmoidf_(acc[4 * j + e]);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) v4[e] = (bf16)(acc[4 * j + e] * keep);
            }
            *reinterpret_cast<bf16x4*>(ts + 8 * j + 4 * hf) = v4;
          }
        }
      }
      sbb = b;
      sline = line;
      st0 = t0;
    }
  }
  if (total > 0) {
    lds_barrier();
    store_chunk(g - 1, sbb, sline, st0);
  }
  __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // no direct load outlives the block
}

// Rows N .. Np - 1 of each pair-bias matrix (keys past N once column mode has transposed
// it; padding queries in row mode) get no tile: zero them so every bias value is finite.
__global__ __launch_bounds__(256) void pb_zero_pad_rows_kernel(float* __restrict__ PB, int N, int Np) {
  float* m = PB + (size_t)blockIdx.y * Np * Np + (size_t)N * Np;
  const long n4 = (long)(Np - N) * Np / 4;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += (long)gridDim.x * 256)
    reinterpret_cast<f32x4*>(m)[i] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// key_mask (optional): the folded key mask [B][N] of a pair mask that is the outer product of
// its diagonal; it is then added to the pair bias (rows: a pass over the bias; columns: inside
// the transpose) and the flash kernel runs without its per-line key-mask MFMA.
template <class TZ>
int grid_attn256_launch(const void* z, const float* mask, const float* lnw, const float* lnb, float eps,
                        const void* w5, const void* wo, int B, int N, int transpose, void* out, int accumulate,
                        const float* key_mask, void* ws, hipStream_t s) {
  using Cfg = GridProj256;
  const int Np = (int)pf::round_up((size_t)N, kPad);
  const Grid256Ws L = grid256_layout(B, N);
  char* base = reinterpret_cast<char*>(ws);
  bf16* Q = reinterpret_cast<bf16*>(base + L.q);
  bf16* K = reinterpret_cast<bf16*>(base + L.k);
  bf16* V = reinterpret_cast<bf16*>(base + L.v);
  float* PB = reinterpret_cast<float*>(base + L.pb);
  float* MA = reinterpret_cast<float*>(base + L.ma);
  bf16* G = reinterpret_cast<bf16*>(base + L.g);
  bf16* og = reinterpret_cast<bf16*>(base + L.og);
  int* redo = reinterpret_cast<int*>(base + L.redo);
  const long M = (long)B * N * N;
  const float qscale = (1.0f / sqrtf((float)kHeadDim)) * kLog2e;
  {
    const long ntiles = (long)B * N * (Np / Cfg::BP);
    const int nblk = (int)std::min<long>(ntiles, pf::cu_count());
    pf::KernelTimer timer("grid_project256", s);
    grid_project256_kernel<TZ><<<nblk, Cfg::NT, 0, s>>>((const TZ*)z, mask, lnw, lnb, eps, (const bf16*)w5, Q, K,
                                                        V, PB, MA, G, B, N, Np, transpose, qscale, L.gq, L.gpb);
    timer.stop();
    if (int e = pf::check_launch("grid_project256")) return e;
  }
  const int HD = Cfg::HD;
  const long NN = (long)N * N;
  // o of (b, line, head, token) at og[pos][head d + e]: pos = (line, token) for rows,
  // (token, line) for columns
  const Strides4 so = transpose ? Strides4{NN * HD, (long)HD, (long)kHeadDim, (long)N * HD}
                                : Strides4{NN * HD, (long)N * HD, (long)kHeadDim, (long)HD};
  constexpr int QS = attn_qsub<bf16>();
  constexpr int NT = 64 * kLinesPerBlock;
  const int nqb = Np / (32 * QS);
  const int nlg = (N + kLinesPerBlock - 1) / kLinesPerBlock;
  const long total = (long)B * nlg * kHeads * nqb;
  const int remap = (total % 8 == 0) ? 1 : 0;
  if (Np > N) {
    const long n4 = (long)(Np - N) * Np / 4;
    pb_zero_pad_rows_kernel<<<dim3((unsigned)std::min<long>((n4 + 255) / 256, 64), 2 * B * kHeads), 256, 0, s>>>(
        PB, N, Np);
    if (int e = pf::check_launch("pb_zero_pad_rows")) return e;
  }
  for (int gi = 0; gi < 2; ++gi) {
    bf16* Qg = Q + gi * L.gq;
    bf16* Kg = K + gi * L.gq;
    bf16* Vg = V + gi * L.gq;
    float* PBg = PB + gi * L.gpb;
    int* rg = redo + gi * L.gredo;
    bf16* Og = og + gi * 4 * kHeadDim;
    if (transpose) {
      const int nt = Np / 32;
      pb_transpose_kernel<<<dim3(nt * (nt + 1) / 2, B * kHeads), 256, 0, s>>>(PBg, Np, key_mask, N);
      if (int e = pf::check_launch("pb_transpose")) return e;
    } else if (key_mask != nullptr) {
      const long n4 = (long)Np * Np / 4;
      const int gx = (int)std::min<long>((n4 + 255) / 256, (4L * pf::cu_count() + B * kHeads - 1) / (B * kHeads));
      pb_fold_kernel<<<dim3(std::max(gx, 1), B * kHeads), 256, 0, s>>>(PBg, key_mask, N, Np);
      if (int e = pf::check_launch("pb_fold")) return e;
    }
    pf::KernelTimer timer("tri_attn", s);
    const dim3 grid((unsigned)total);
    constexpr size_t lds = attn_bias_lds_bytes<bf16>();
    if (key_mask != nullptr)
      tri_attn_kernel<bf16, QS, true, true, false, false><<<grid, NT, lds, s>>>(
          Qg, Kg, Vg, PBg, MA, Og, B, N, Np, N, N, 0, remap, rg, 1.f, so);
    else
      tri_attn_kernel<bf16, QS, true, true, false, true><<<grid, NT, lds, s>>>(
          Qg, Kg, Vg, PBg, MA, Og, B, N, Np, N, N, 0, remap, rg, 1.f, so);
    timer.stop();
    if (int e = pf::check_launch("tri_attn")) return e;
    if (key_mask != nullptr)
      tri_attn_kernel<bf16, QS, true, false, false, false><<<grid, NT, lds, s>>>(
          Qg, Kg, Vg, PBg, MA, Og, B, N, Np, N, N, 0, remap, rg, 1.f, so);
    else
      tri_attn_kernel<bf16, QS, true, false, false, true><<<grid, NT, lds, s>>>(
          Qg, Kg, Vg, PBg, MA, Og, B, N, Np, N, N, 0, remap, rg, 1.f, so);
    if (int e = pf::check_launch("tri_attn_redo")) return e;
  }
  // The gate (G holds sigmoid(g)) is applied as the output GEMM loads og, so og is not
  // rewritten (a gate pass over og and G cost 136 us per call; o * sigmoid(g) in the flash
  // kernel's epilogue cost that kernel 67 us per launch).
  return tile_gemm_rows_gated(og, G, wo, out, M, Cfg::C, HD, accumulate, sizeof(TZ) == 2 ? PF_BF16 : PF_F32, s);
}

template <class TZ, class TC>
int grid_attn_generic_launch(const void* z, const float* mask, const float* lnw, const float* lnb, float eps,
                             const void* w5, const void* wo, int B, int N, int C, int H, int transpose, void* out,
                             int accumulate, const float* key_mask, void* ws, hipStream_t s) {
  const int cd = sizeof(TC) == 4 ? PF_F32 : PF_BF16;
  if constexpr (sizeof(TC) == 2)
    if (grid256_applies(C, H, cd))
      return grid_attn256_launch<TZ>(z, mask, lnw, lnb, eps, w5, wo, B, N, transpose, out, accumulate, key_mask, ws,
                                     s);
  const GridGenWs L = grid_gen_layout(B, N, C, H, cd);
  const int d = grid_gen_head_dim(C, H);
  const int H4 = (H + 3) / 4 * 4;
  const int PW = 4 * H * d + 16;
  const long M = (long)B * N * N;
  char* base = reinterpret_cast<char*>(ws);
  TC* xn = reinterpret_cast<TC*>(base + L.xn);
  TC* proj = reinterpret_cast<TC*>(base + L.proj);
  TC* Q = reinterpret_cast<TC*>(base + L.q);
  TC* K = reinterpret_cast<TC*>(base + L.k);
  TC* V = reinterpret_cast<TC*>(base + L.v);
  float* PB = reinterpret_cast<float*>(base + L.pb);
  float* MA = reinterpret_cast<float*>(base + L.ma);
  TC* O = reinterpret_cast<TC*>(base + L.o);
  TC* og = reinterpret_cast<TC*>(base + L.og);
  if (int e = ln_launch<TZ, TC>(z, lnw, lnb, eps, xn, M, C, s)) return e;
  if (int e = rowgemm_launch<TC, TC, EPI_STORE>(xn, w5, nullptr, 0, proj, M, PW, C, s)) return e;
  if (d == kHeadDim && H % 4 == 0) {
    // Heads of the flash kernel's width in whole groups of four: the attention reads q, k, v
    // straight from the projection rows and writes o into og's rows (strided), so nothing
    // is repacked into a head-major layout and back. Element (b, line, head, token, e) of
    // q sits at proj[pos (b, x, y)][head d + e] with (x, y) = (line, token) for rows and
    // (token, line) for columns; o goes to og[pos][head d + e].
    grid_gen_bias_kernel<TC><<<(unsigned)((M * H4 + 255) / 256), 256, 0, s>>>(proj, mask, PB, MA, B, N, H, H4, d, PW,
                                                                               transpose);
    if (int e = pf::check_launch("grid_gen_bias")) return e;
    const int HD = H * d;
    const long NN = (long)N * N;
    const Strides4 sx = transpose ? Strides4{NN * PW, (long)PW, (long)d, (long)N * PW}
                                  : Strides4{NN * PW, (long)N * PW, (long)d, (long)PW};
    const Strides4 so = transpose ? Strides4{NN * HD, (long)HD, (long)d, (long)N * HD}
                                  : Strides4{NN * HD, (long)N * HD, (long)d, (long)HD};
    for (int g = 0; g < H / 4; ++g) {
      const size_t hoff = (size_t)g * 4 * d;
      if (int e = evo_attn_launch<TC>(proj + hoff, proj + HD + hoff, proj + 2 * HD + hoff, MA,
                                      PB + (size_t)g * B * 4 * N * N, B, N, N, 0, og + hoff, base + L.evo, s,
                                      1.0f / sqrtf((float)d), &sx, &so))
        return e;
    }
    grid_gen_gate_inplace_kernel<TC><<<(unsigned)((M * (HD / 8) + 255) / 256), 256, 0, s>>>(og, proj, M, HD, PW,
                                                                                          3 * HD);
    if (int e = pf::check_launch("grid_gen_gate")) return e;
    if (accumulate) return rowgemm_launch<TC, TZ, EPI_RESIDUAL>(og, wo, nullptr, 0, out, M, C, HD, s);
    return rowgemm_launch<TC, TZ, EPI_STORE>(og, wo, nullptr, 0, out, M, C, HD, s);
  }
  grid_gen_pack_kernel<TC><<<(unsigned)((M * H4 * 4 + 255) / 256), 256, 0, s>>>(proj, mask, Q, K, V, PB, MA, B, N, H,
                                                                                H4, d, PW, transpose);
  if (int e = pf::check_launch("grid_gen_pack")) return e;
  const size_t group = (size_t)B * N * 4 * N * kHeadDim;  // elements of one four-head group
  for (int g = 0; g < H4 / 4; ++g) {
    if (int e = evo_attn_launch<TC>(Q + g * group, K + g * group, V + g * group, MA, PB + (size_t)g * B * 4 * N * N,
                                    B, N, N, 0, O + g * group, base + L.evo, s, 1.0f / sqrtf((float)d)))
      return e;
  }
  if (d % 8 == 0)
    grid_gen_gate_kernel<TC, 8><<<(unsigned)((M * H * (d / 8) + 255) / 256), 256, 0, s>>>(O, proj, og, B, N, H, d, PW,
                                                                                        transpose);
  else
    grid_gen_gate_kernel<TC, 1><<<(unsigned)((M * H * d + 255) / 256), 256, 0, s>>>(O, proj, og, B, N, H, d, PW,
                                                                                  transpose);
  if (int e = pf::check_launch("grid_gen_gate")) return e;
  if (accumulate) return rowgemm_launch<TC, TZ, EPI_RESIDUAL>(og, wo, nullptr, 0, out, M, C, H * d, s);
  return rowgemm_launch<TC, TZ, EPI_STORE>(og, wo, nullptr, 0, out, M, C, H * d, s);
}

bool grid_gen_supported(int C, int H) {
  return H >= 1 && H <= 16 && C % 32 == 0 && C % H == 0 && grid_gen_head_dim(C, H) <= kHeadDim &&
         (grid_gen_head_dim(C, H) * H) % 16 == 0;
}


}  // namespace

extern "C" {

size_t pf_grid_attn_workspace_bytes(int B, int N, int C, int H, int cdtype) {
  if (B <= 0 || N <= 0) return 0;
  if (C == kC && H == kHeads) return attn_ws_layout(B, N, cdtype).total;
  if (grid256_applies(C, H, cdtype)) return grid256_layout(B, N).total;
  return grid_gen_supported(C, H) ? grid_gen_layout(B, N, C, H, cdtype).total : 0;
}

int pf_grid_attn_fwd(const void* z, const float* mask, const float* ln_w, const float* ln_b, float eps,
                     const void* w_qkvgb, const void* w_out, int B, int N, int C, int H, int transpose, int zdtype,
                     int cdtype, void* out, int accumulate, const float* key_mask, void* workspace,
                     size_t workspace_bytes, void* stream) {
  PF_REQUIRE(z && mask && ln_w && ln_b && w_qkvgb && w_out && out && workspace, PF_ERR_INVALID_ARG,
             "pf_grid_attn_fwd: null pointer");
  PF_REQUIRE(B > 0 && N > 0, PF_ERR_INVALID_ARG, "pf_grid_attn_fwd: B=%d N=%d", B, N);
  const bool fused = C == kC && H == kHeads;
  PF_REQUIRE(fused || grid_gen_supported(C, H), PF_ERR_UNSUPPORTED,
             "pf_grid_attn_fwd: C=%d H=%d (built: C=128 with 4 heads, or C a multiple of 32 with 1-16 heads of "
             "dimension max(C/H, 16) <= 32)",
             C, H);
  PF_REQUIRE(zdtype == PF_F32 || zdtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_grid_attn_fwd: zdtype %d", zdtype);
  PF_REQUIRE(cdtype == PF_F32 || cdtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_grid_attn_fwd: cdtype %d", cdtype);
  PF_REQUIRE(!(zdtype == PF_BF16 && cdtype == PF_F32), PF_ERR_UNSUPPORTED,
             "pf_grid_attn_fwd: bf16 activations with fp32 GEMMs is not a supported regime");
  PF_REQUIRE(pf::aligned16(z) && pf::aligned16(out) && pf::aligned16(workspace) && pf::aligned16(w_qkvgb) &&
                 pf::aligned16(w_out),
             PF_ERR_ALIGNMENT, "pf_grid_attn_fwd: pointers must be 16-byte aligned");
  PF_REQUIRE(workspace_bytes >= pf_grid_attn_workspace_bytes(B, N, C, H, cdtype), PF_ERR_WORKSPACE,
             "pf_grid_attn_fwd: workspace %zu < %zu bytes", workspace_bytes,
             pf_grid_attn_workspace_bytes(B, N, C, H, cdtype));
  hipStream_t s = pf::as_stream(stream);
  if (!fused) {  // key_mask: used by the 256-channel bf16 path only (the others take the per-line mask)
    const float* km = grid256_applies(C, H, cdtype) ? key_mask : nullptr;
    if (zdtype == PF_F32 && cdtype == PF_F32)
      return grid_attn_generic_launch<float, float>(z, mask, ln_w, ln_b, eps, w_qkvgb, w_out, B, N, C, H, transpose,
                                                    out, accumulate, km, workspace, s);
    if (zdtype == PF_F32)
      return grid_attn_generic_launch<float, bf16>(z, mask, ln_w, ln_b, eps, w_qkvgb, w_out, B, N, C, H, transpose,
                                                   out, accumulate, km, workspace, s);
    return grid_attn_generic_launch<bf16, bf16>(z, mask, ln_w, ln_b, eps, w_qkvgb, w_out, B, N, C, H, transpose, out,
                                                accumulate, km, workspace, s);
  }
  if (zdtype == PF_F32 && cdtype == PF_F32)
    return grid_attn_launch<float, float>(z, mask, ln_w, ln_b, eps, w_qkvgb, w_out, B, N, transpose, out, accumulate,
                                          key_mask, workspace, s);
  if (zdtype == PF_F32)
    return grid_attn_launch<float, bf16>(z, mask, ln_w, ln_b, eps, w_qkvgb, w_out, B, N, transpose, out, accumulate,
                                         key_mask, workspace, s);
  return grid_attn_launch<bf16, bf16>(z, mask, ln_w, ln_b, eps, w_qkvgb, w_out, B, N, transpose, out, accumulate,
                                      key_mask, workspace, s);
}

int pf_pair_mask_outer(const float* mask, int B, int N, int* flag, float* key_mask, void* stream) {
  PF_REQUIRE(mask && flag && key_mask, PF_ERR_INVALID_ARG, "pf_pair_mask_outer: null pointer");
  PF_REQUIRE(B > 0 && N > 0, PF_ERR_INVALID_ARG, "pf_pair_mask_outer: B=%d N=%d", B, N);
  hipStream_t s = pf::as_stream(stream);
  mask_outer_init_kernel<<<(unsigned)((B * N + 255) / 256), 256, 0, s>>>(mask, B, N, flag, key_mask);
  if (int e = pf::check_launch("mask_outer_init")) return e;
  const long total = (long)B * N * N;
  const int nblk = (int)std::min<long>((total + 255) / 256, 4L * pf::cu_count());
  mask_outer_check_kernel<<<nblk, 256, 0, s>>>(mask, B, N, flag);
  return pf::check_launch("mask_outer_check");
}

// Number of redo flags the fast flash pass writes: one per wave of its grid.
static size_t redo_flag_count(int B, int L, int Np, int cdtype) {
  const int QS = cdtype == PF_F32 ? attn_qsub<float>() : attn_qsub<bf16>();
  const size_t nlg = (size_t)(L + kLinesPerBlock - 1) / kLinesPerBlock;
  return (size_t)B * nlg * kHeads * (size_t)(Np / (32 * QS)) * kLinesPerBlock;
}

int pf_grid_attn_redo_flags(int B, int N, int C, int H, int cdtype, size_t* offset, size_t* count) {
  PF_REQUIRE(offset && count, PF_ERR_INVALID_ARG, "pf_grid_attn_redo_flags: null pointer");
  const bool fused = C == kC && H == kHeads;
  PF_REQUIRE(B > 0 && N > 0 && (fused || grid_gen_supported(C, H)) && (cdtype == PF_F32 || cdtype == PF_BF16),
             PF_ERR_UNSUPPORTED, "pf_grid_attn_redo_flags: B=%d N=%d C=%d H=%d cdtype=%d", B, N, C, H, cdtype);
  // generic channels: the flags of the last group of four heads (256 channels: both groups)
  *count = redo_flag_count(B, N, pf::pad128(N), cdtype);
  if (!fused && grid256_applies(C, H, cdtype)) {
    const Grid256Ws L = grid256_layout(B, N);
    *offset = L.redo + L.gredo * sizeof(int);
    return pf::ok();
  }
  *offset = fused ? attn_ws_layout(B, N, cdtype).redo
                  : grid_gen_layout(B, N, C, H, cdtype).evo + evo_ws_layout(B, N, N, cdtype).redo;
  return pf::ok();
}

int pf_evo_attn_redo_flags(int B, int S, int H, int N, int D, int dtype, size_t* offset, size_t* count) {
  PF_REQUIRE(offset && count, PF_ERR_INVALID_ARG, "pf_evo_attn_redo_flags: null pointer");
  PF_REQUIRE(B > 0 && S > 0 && N > 0 && H == kHeads && D == kHeadDim && (dtype == PF_F32 || dtype == PF_BF16),
             PF_ERR_UNSUPPORTED, "pf_evo_attn_redo_flags: B=%d S=%d N=%d H=%d D=%d dtype=%d", B, S, N, H, D, dtype);
  *offset = evo_ws_layout(B, S, N, dtype).redo;
  *count = redo_flag_count(B, S, pf::pad128(N), dtype);
  return pf::ok();
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

int pf_evo_attn_fwd_strided(const void* q, const void* k, const void* v, const long* qkv_strides,
                            const float* res_mask, const float* pair_bias, int B, int S, int H, int N, int D,
                            int dtype, int masked_rows_zero, void* out, const long* out_strides, float* lse_out,
                            void* workspace, size_t workspace_bytes, void* stream) {
  PF_REQUIRE(q && k && v && qkv_strides && res_mask && pair_bias && out && out_strides && workspace,
             PF_ERR_INVALID_ARG, "pf_evo_attn_fwd_strided: null pointer");
  PF_REQUIRE(B > 0 && S > 0 && N > 0, PF_ERR_INVALID_ARG, "pf_evo_attn_fwd_strided: B=%d S=%d N=%d", B, S, N);
  PF_REQUIRE(H == kHeads && D == kHeadDim, PF_ERR_UNSUPPORTED,
             "pf_evo_attn_fwd_strided: H=%d D=%d (built: H=4, D=32)", H, D);
  PF_REQUIRE(dtype == PF_F32 || dtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_evo_attn_fwd_strided: dtype %d", dtype);
  const Strides4 sx{qkv_strides[0], qkv_strides[1], qkv_strides[2], qkv_strides[3]};
  const Strides4 so{out_strides[0], out_strides[1], out_strides[2], out_strides[3]};
  const long vec = dtype == PF_F32 ? 4 : 8;  // elements per 16 bytes
  for (const Strides4* st : {&sx, &so})
    PF_REQUIRE(st->b % vec == 0 && st->s % vec == 0 && st->h % vec == 0 && st->n % vec == 0 && st->n >= kHeadDim,
               PF_ERR_ALIGNMENT, "pf_evo_attn_fwd_strided: strides must keep 16-byte aligned rows of D elements");
  PF_REQUIRE(pf::aligned16(q) && pf::aligned16(k) && pf::aligned16(v) && pf::aligned16(out) &&
                 pf::aligned16(workspace),
             PF_ERR_ALIGNMENT, "pf_evo_attn_fwd_strided: pointers must be 16-byte aligned");
  PF_REQUIRE(workspace_bytes >= evo_ws_layout(B, S, N, dtype).total, PF_ERR_WORKSPACE,
             "pf_evo_attn_fwd_strided: workspace %zu < %zu bytes", workspace_bytes,
             evo_ws_layout(B, S, N, dtype).total);
  hipStream_t s = pf::as_stream(stream);
  const float sc = 1.0f / sqrtf((float)kHeadDim);
  if (dtype == PF_F32)
    return evo_attn_launch<float>(q, k, v, res_mask, pair_bias, B, S, N, masked_rows_zero, out, workspace, s, sc, &sx,
                                  &so, lse_out);
  return evo_attn_launch<bf16>(q, k, v, res_mask, pair_bias, B, S, N, masked_rows_zero, out, workspace, s, sc, &sx,
                               &so, lse_out);
}

}  // extern "C"
