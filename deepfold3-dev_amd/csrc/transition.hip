// Pair transition (SwiGLU MLP) with an optional fused single_to_pair epilogue, and the
// standalone single_to_pair projection.
//
//   pair_transition: y = (silu(h_a) * h_b) W2^T with [h_a | h_b] = LN(x) W1^T, the halves
//                    contiguous (reference TransitionBlock, src/deepfold3/model/primitives.py:193-251;
//                    FusedTransitionBlock, triton/fused_transition.py:34-83). The hidden
//                    activations never leave the chip: the hidden dim is walked in chunks of
//                    128, each chunk's SwiGLU output goes through LDS straight into the second
//                    GEMM, whose accumulators stay in registers. out = y or out += y.
//   single_to_pair:  logits[b, h, i, j] = LN'(z[b, i, j]) Ws2p[h]^T (reference
//                    evoformer.py:322-328, `.movedim(-1, -3)` materialised). When fused into
//                    the transition, LN' reads the updated z (rounded to z's dtype first, as
//                    the reference computes it from the stored residual stream).
#include <algorithm>

#include "capi.h"
#include "common.h"

namespace {

constexpr int kC = 128;
constexpr int kHidden = 512;  // factor 4: W1 [1024][128], W2 [128][512]
constexpr int kS2pHeads = 16;

template <class TC>
constexpr int tr_bm() { return sizeof(TC) == 2 ? 64 : 32; }

template <class TZ, class TC>
struct TrCfg {
  static constexpr int BM = tr_bm<TC>();
  static constexpr int ALD = kC + lds_pad<TC>();
  static constexpr int A_BYTES = BM * ALD * (int)sizeof(TC);
  static constexpr int SLD = kC + 4;
  static constexpr int S_BYTES = BM * SLD * 4;
  // A | U | (stage aliases A+U once both are dead)
  static constexpr int SMEM1 = 2 * A_BYTES;
  static constexpr int SMEM = SMEM1 > S_BYTES ? SMEM1 : S_BYTES;
};

// LN'(rows) W^T for one 16-column block over BM rows held in an LDS tile A (already
// normalised), written as logits[b][h][pos] for h < H. Row block rb is done by wave rb.
template <class TC, int BM>
PF_DEVICE void s2p_store(const TC* A, int ALD, const TC* __restrict__ Ws, float* __restrict__ logits, long m0, long M,
                         long NN) {
  constexpr int RB = BM / 16;
  const int w = wave_id();
  const int l = lane_id();
  if (w >= RB) return;
  f32x4 acc[1][1];
  zero_acc(acc);
  int wrow[1] = {0};
  gemm16_lds_x_w<TC, kC, 1, 1>(acc, A, ALD, w * 16, Ws, kC, wrow);
  const int h = l & 15;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const long m = m0 + w * 16 + 4 * (l >> 4) + e;
    if (m >= M) continue;
    const long b = m / NN;
    const long pos = m % NN;
    logits[(b * kS2pHeads + h) * NN + pos] = acc[0][0][e];
  }
}

template <class TZ, class TC, bool S2P>
__global__ __launch_bounds__(256) void pair_transition_kernel(
    const TZ* __restrict__ x, TZ* __restrict__ out, const float* __restrict__ lnw, const float* __restrict__ lnb,
    float eps, const TC* __restrict__ W1, const TC* __restrict__ W2, long M, int accumulate,
    const float* __restrict__ s2p_w, const float* __restrict__ s2p_b, float s2p_eps, const TC* __restrict__ Ws2p,
    float* __restrict__ logits, long NN) {
  using Cfg = TrCfg<TZ, TC>;
  constexpr int BM = Cfg::BM, ALD = Cfg::ALD, SLD = Cfg::SLD;
  constexpr int NT = 256;
  constexpr int RB = BM / 16;
  __shared__ __attribute__((aligned(16))) char smem[Cfg::SMEM];
  TC* A = reinterpret_cast<TC*>(smem);
  TC* U = reinterpret_cast<TC*>(smem + Cfg::A_BYTES);
  float* stage = reinterpret_cast<float*>(smem);

  const long m0 = (long)blockIdx.x * BM;
  const int w = wave_id();
  const int l = lane_id();
  auto xrow = [&](int p) -> const TZ* {
    const long m = m0 + p;
    return m < M ? x + m * kC : nullptr;
  };
  ln_tile_to_lds<TZ, TC, kC, BM, NT>(xrow, lnw, lnb, eps, A, ALD);
  __syncthreads();

  f32x4 acc_o[RB][2];
  zero_acc(acc_o);
  const int orow[2] = {w * 32, w * 32 + 16};
#pragma unroll 1
  for (int ch = 0; ch < kHidden / 128; ++ch) {
    f32x4 acc_h[RB][4];
    zero_acc(acc_h);
    const int hrow[4] = {ch * 128 + w * 32, ch * 128 + w * 32 + 16, kHidden + ch * 128 + w * 32,
                         kHidden + ch * 128 + w * 32 + 16};
    gemm16_lds_x_w<TC, kC, RB, 4>(acc_h, A, ALD, 0, W1, kC, hrow);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int p = rb * 16 + 4 * (l >> 4) + e;
          const int c = w * 32 + j * 16 + (l & 15);
          U[p * ALD + c] = from_f32<TC>(siluf_(acc_h[rb][j][e]) * acc_h[rb][j + 2][e]);
        }
    __syncthreads();
    gemm16_lds_x_w<TC, 128, RB, 2>(acc_o, U, ALD, 0, W2 + ch * 128, kHidden, orow);
    __syncthreads();
  }

  // y -> fp32 stage [BM][SLD] (A and U are dead)
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        stage[(rb * 16 + 4 * (l >> 4) + e) * SLD + w * 32 + j * 16 + (l & 15)] = acc_o[rb][j][e];
  __syncthreads();
  {
    constexpr int VEC = 16 / sizeof(TZ);
    constexpr int LPP = kC / VEC;
    constexpr int PPI = NT / LPP;
    const int tid = threadIdx.x;
    const int sub = tid % LPP;
    const int pp = tid / LPP;
#pragma unroll
    for (int p0 = 0; p0 < BM; p0 += PPI) {
      const int p = p0 + pp;
      const long m = m0 + p;
      if (m >= M) continue;
      float v[VEC];
      if (accumulate) {
        load16<TZ>(out + m * kC + sub * VEC, v);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        v[e] = to_f32(from_f32<TZ>(v[e] + stage[p * SLD + sub * VEC + e]));
        if (S2P) stage[p * SLD + sub * VEC + e] = v[e];
      }
      store_vec<TZ, VEC>(out + m * kC + sub * VEC, v);
    }
  }
  if (S2P) {
    // stage now holds the updated residual (as stored); LN' it into a TC tile placed after
    // the stage, then project to the single-attention heads.
    __syncthreads();
    __shared__ __attribute__((aligned(16))) TC A2[BM * ALD];
    auto srow = [&](int p) -> const float* { return m0 + p < M ? stage + p * SLD : nullptr; };
    ln_tile_to_lds<float, TC, kC, BM, NT>(srow, s2p_w, s2p_b, s2p_eps, A2, ALD);
    __syncthreads();
    s2p_store<TC, BM>(A2, ALD, Ws2p, logits, m0, M, NN);
  }
}

// bf16 path: 128 positions per block, 8 waves, 32x32x16 MFMAs on LDS operands. The block
// walks the hidden dim in four chunks of 128: [h_a | h_b]^T = W1_chunk LN(x)^T (wave w:
// hidden tile w & 3, positions 64 (w >> 2) ..), u = silu(h_a) h_b -> LDS, then
// y^T += W2_chunk u^T (wave w: output tile w & 3). Weight chunks are prefetched into
// registers one phase ahead. LDS: x | u | two weight buffers (136 KiB, one block per CU).
template <class TZ, bool S2P>
__global__ __launch_bounds__(512) void pair_transition32_kernel(
    const TZ* __restrict__ x, TZ* __restrict__ out, const float* __restrict__ lnw, const float* __restrict__ lnb,
    float eps, const bf16* __restrict__ W1, const bf16* __restrict__ W2, long M, int accumulate,
    const float* __restrict__ s2p_w, const float* __restrict__ s2p_b, float s2p_eps, const bf16* __restrict__ Ws2p,
    float* __restrict__ logits, long NN) {
  constexpr int BM = 128;
  constexpr int LD = ld128<bf16>();
  constexpr int SLD = kC + 4;
  constexpr int NT = 512;
  constexpr int TILE = BM * LD * 2;
  static_assert(BM * SLD * 4 <= 2 * TILE, "stage must fit over x and u");
  __shared__ __attribute__((aligned(16))) char smem[4 * TILE];
  bf16* X = reinterpret_cast<bf16*>(smem);
  bf16* U = reinterpret_cast<bf16*>(smem + TILE);
  bf16* Wa = reinterpret_cast<bf16*>(smem + 2 * TILE);
  bf16* Wb = reinterpret_cast<bf16*>(smem + 3 * TILE);
  float* stage = reinterpret_cast<float*>(smem);

  const long m0 = (long)blockIdx.x * BM;
  const int w = wave_id();
  const int l = lane_id();
  const int ht = w & 3;          // hidden / output tile of 32
  const int pg = (w >> 2) * 64;  // first position of the wave's two position tiles

  Rows128<bf16, 128, NT> pfa, pfb;
  pfa.load(W1, kC);
  pfb.load(W1 + (size_t)kHidden * kC, kC);
  ln_tile_to_lds<TZ, bf16, kC, BM, NT>([&](int p) -> const TZ* {
    const long m = m0 + p;
    return m < M ? x + m * kC : nullptr;
  }, lnw, lnb, eps, X, LD);
  pfa.store(Wa, LD);
  pfb.store(Wb, LD);
  __syncthreads();

  f32x16 acc_o[1][2];
  zero_acc32(acc_o);
#pragma unroll 1
  for (int ch = 0; ch < kHidden / 128; ++ch) {
    Rows128<bf16, 128, NT> pf2;
    pf2.load(W2 + ch * 128, kHidden);
    {
      f32x16 acc_a[1][2], acc_b[1][2];
      zero_acc32(acc_a);
      zero_acc32(acc_b);
      wave_mma32<bf16, 1, 2, kC>(acc_a, Wa, LD, 32 * ht, X, LD, pg);
      wave_mma32<bf16, 1, 2, kC>(acc_b, Wb, LD, 32 * ht, X, LD, pg);
#pragma unroll
      for (int pj = 0; pj < 2; ++pj)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = siluf_(acc_a[0][pj][4 * g4 + e]) * acc_b[0][pj][4 * g4 + e];
          store_vec<bf16, 4>(U + (pg + 32 * pj + (l & 31)) * LD + 32 * ht + acc32_row(4 * g4), v);
        }
    }
    __syncthreads();  // u complete; the W1 buffers are free
    pf2.store(Wa, LD);
    if (ch + 1 < kHidden / 128) {
      pfa.load(W1 + (size_t)(ch + 1) * 128 * kC, kC);
      pfb.load(W1 + (size_t)(kHidden + (ch + 1) * 128) * kC, kC);
    }
    __syncthreads();
    wave_mma32<bf16, 1, 2, 128>(acc_o, Wa, LD, 32 * ht, U, LD, pg);
    __syncthreads();  // Wa and u free
    if (ch + 1 < kHidden / 128) {
      pfa.store(Wa, LD);
      pfb.store(Wb, LD);
      __syncthreads();
    }
  }

  // y -> fp32 stage [pos][ch] over x and u
#pragma unroll
  for (int pj = 0; pj < 2; ++pj)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4)
      *reinterpret_cast<f32x4*>(stage + (pg + 32 * pj + (l & 31)) * SLD + 32 * ht + acc32_row(4 * g4)) =
          f32x4{acc_o[0][pj][4 * g4], acc_o[0][pj][4 * g4 + 1], acc_o[0][pj][4 * g4 + 2], acc_o[0][pj][4 * g4 + 3]};
  __syncthreads();
  {
    constexpr int VEC = 16 / sizeof(TZ);
    constexpr int LPP = kC / VEC;
    constexpr int PPI = NT / LPP;
    const int tid = threadIdx.x;
    const int sub = tid % LPP;
    const int pp = tid / LPP;
#pragma unroll
    for (int p0 = 0; p0 < BM; p0 += PPI) {
      const int p = p0 + pp;
      const long m = m0 + p;
      if (m >= M) continue;
      float v[VEC];
      if (accumulate) {
        load16<TZ>(out + m * kC + sub * VEC, v);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        v[e] = to_f32(from_f32<TZ>(v[e] + stage[p * SLD + sub * VEC + e]));
        if (S2P) stage[p * SLD + sub * VEC + e] = v[e];
      }
      store_vec<TZ, VEC>(out + m * kC + sub * VEC, v);
    }
  }
  if (S2P) {
    __syncthreads();
    bf16* A2 = Wa;
    ln_tile_to_lds<float, bf16, kC, BM, NT>([&](int p) -> const float* {
      return m0 + p < M ? stage + p * SLD : nullptr;
    }, s2p_w, s2p_b, s2p_eps, A2, LD);
    __syncthreads();
    s2p_store<bf16, BM>(A2, LD, Ws2p, logits, m0, M, NN);
  }
}

// bf16 path, persistent and weight-streaming: one 8-wave block per CU (two waves per SIMD)
// walks tiles of 256 positions, 32 per wave (one MFMA column tile). Per tile each wave
// normalises its positions straight into registers as the B operands of W1 (fp32
// statistics; a position's 128 channels live in lanes l and l ^ 32). The hidden dim is
// walked in eight chunks of 64 (a rows 64 c .., b rows 512 + 64 c ..): the chunk's W1 rows
// (32 KiB) and W2 columns (16 KiB) are streamed into a double-buffered LDS ring by direct
// buffer-to-LDS loads one chunk ahead (16-byte chunks XOR-swizzled by row, so fragment
// reads are conflict-free); [h_a | h_b]^T = W1_c LN(x)^T on 32x32x16 MFMAs, u = silu(h_a) h_b
// goes through a per-wave LDS tile into y^T += W2_c u^T, whose accumulators stay in
// registers for the whole tile. Epilogue: the residual add and the stores straight from the
// accumulator layout (lane: one position, 4-channel groups), then the fused single_to_pair:
// LN' of the updated rows (statistics via the lane-pair swap) and its [128 -> 16]
// projection as 8 more MFMAs whose A operands (Ws2p, columns in the accumulator's channel
// order) are built once per block in LDS. The next tile's rows are loaded before the
// epilogue so their latency overlaps it.
struct TransWs {
  static constexpr int C = 128;
  static constexpr int HC = 64;                      // hidden units per chunk
  static constexpr int NCH = kHidden / HC;           // 8 chunks
  static constexpr int NW = 8;                       // waves per block (two per SIMD)
  static constexpr int NT = 64 * NW;
  static constexpr int PW = 32;                      // positions per wave
  static constexpr int BP = PW * NW;                 // positions per tile
  static constexpr int W1_BYTES = 2 * HC * C * 2;    // 128 rows x 256 B
  static constexpr int W2_BYTES = C * HC * 2;        // 128 rows x 128 B
  static constexpr int STAGE = W1_BYTES + W2_BYTES;  // 48 KiB
  static constexpr int U_BYTES = PW * HC * 2;        // per wave
  static constexpr int DMA1 = W1_BYTES / 1024 / NW;  // W1 direct loads per wave per chunk
  static constexpr int DMA2 = W2_BYTES / 1024 / NW;  // W2 direct loads per wave per chunk
  static constexpr int S2P_BYTES = 8 * 64 * 16;      // Ws2p A fragments [k-step][lane]
};

constexpr size_t tr_ws_lds_bytes() {
  return 2 * (size_t)TransWs::STAGE + (size_t)TransWs::NW * TransWs::U_BYTES + TransWs::S2P_BYTES +
         4 * TransWs::C * sizeof(float);
}

// XOR swizzle of the 16-byte chunks of LDS rows of 256 or 128 bytes. The LDS serves a
// ds_read_b128 16 lanes at a time from 64 banks (256 bytes), and the 16 lanes of a fragment
// read are 16 consecutive rows at one logical chunk: with 256-byte rows (r & 15) spreads them
// over the 16 bank groups; with 128-byte rows a row pair spans the banks once, so pairs take
// the XOR (r >> 1) & 7.
PF_DEVICE int swz(int r, int row_bytes) { return row_bytes == 256 ? (r & 15) : ((r >> 1) & 7); }
// Byte offset of logical 16-byte chunk c of row r.
PF_DEVICE int swz_off(int r, int c, int row_bytes) { return r * row_bytes + 16 * (c ^ swz(r, row_bytes)); }

// One position row of z as the raw 16-byte pieces the LayerNorm B operands need: channels
// 16 ks + 8 hf .. +7 for ks = 0..7 (bf16: 8 pieces, fp32: 16).
template <class TZ>
struct ZRow {
  static constexpr int NP = sizeof(TZ) == 2 ? 8 : 16;
  u32x4 v[NP];
  PF_DEVICE void load(const TZ* __restrict__ x, long m, long M, int hf) {
    if (m < M) {
      const TZ* row = x + m * TransWs::C + 8 * hf;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        if constexpr (sizeof(TZ) == 2) {
          v[ks] = *reinterpret_cast<const u32x4*>(row + 16 * ks);
        } else {
          v[2 * ks] = *reinterpret_cast<const u32x4*>(row + 16 * ks);
          v[2 * ks + 1] = *reinterpret_cast<const u32x4*>(row + 16 * ks + 4);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < NP; ++i) v[i] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  PF_DEVICE void get(int ks, float (&o)[8]) const {
    if constexpr (sizeof(TZ) == 2) {
      const bf16x8 t = __builtin_bit_cast(bf16x8, v[ks]);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (float)t[e];
    } else {
      const f32x4 a = __builtin_bit_cast(f32x4, v[2 * ks]), b = __builtin_bit_cast(f32x4, v[2 * ks + 1]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = a[e];
        o[4 + e] = b[e];
      }
    }
  }
};

template <class TZ, bool S2P>
__global__ __launch_bounds__(TransWs::NT, 1) void pair_transition_ws_kernel(
    const TZ* __restrict__ x, TZ* __restrict__ out, const float* __restrict__ lnw, const float* __restrict__ lnb,
    float eps, const bf16* __restrict__ W1, const bf16* __restrict__ W2, long M, int accumulate,
    const float* __restrict__ s2p_w, const float* __restrict__ s2p_b, float s2p_eps, const bf16* __restrict__ Ws2p,
    float* __restrict__ logits, long NN) {
  using Cfg = TransWs;
  constexpr int C = Cfg::C, HC = Cfg::HC, NCH = Cfg::NCH, PW = Cfg::PW, BP = Cfg::BP;
  __shared__ __attribute__((aligned(16))) char smem[tr_ws_lds_bytes()];
  char* stage0 = smem;                                      // [2][STAGE]
  char* ubase = smem + 2 * Cfg::STAGE;                      // [NW][U_BYTES]
  char* s2pa = ubase + Cfg::NW * Cfg::U_BYTES;              // [8][64] x 16 B
  float* lnp = reinterpret_cast<float*>(s2pa + Cfg::S2P_BYTES);  // lnw | lnb | s2p_w | s2p_b

  const int w = wave_id();
  const int l = lane_id();
  const int lq = l & 31, hf = l >> 5;
  char* ub = ubase + w * Cfg::U_BYTES;
  const long ntiles = (M + BP - 1) / BP;

  for (int i = threadIdx.x; i < C; i += Cfg::NT) {
    lnp[i] = lnw[i];
    lnp[C + i] = lnb[i];
    if (S2P) {
      lnp[2 * C + i] = s2p_w[i];
      lnp[3 * C + i] = s2p_b[i];
    }
  }
  if (S2P && w == 0) {
    // k-step ks takes channels 16 ks + 8 hf + e (the epilogue's lane-pair-swapped order);
    // rows >= 16 are zero.
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      bf16x8 a;
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = lq < kS2pHeads ? Ws2p[lq * C + 16 * ks + 8 * hf + e] : (bf16)0.f;
      *reinterpret_cast<bf16x8*>(s2pa + (ks * 64 + l) * 16) = a;
    }
  }

  // Weight chunk g (global chunk counter; weights of hidden chunk g % NCH) -> LDS stage g & 1.
  const auto r1 = buf_rsrc(W1, 2 * kHidden * C * 2);
  const auto r2 = buf_rsrc(W2, C * kHidden * 2);
  auto issue_chunk = [&](long g) {
    const int c = (int)(g % NCH);
    char* st = stage0 + (g & 1) * Cfg::STAGE;
#pragma unroll
    for (int t = 0; t < Cfg::DMA1; ++t) {
      const int ins = w * Cfg::DMA1 + t;  // 4 LDS rows of 256 B per instruction
      const int row = 4 * ins + (l >> 4);
      const int lc = (l & 15) ^ swz(row, 256);  // logical chunk this lane fetches
      const int grow = row < HC ? HC * c + row : kHidden + HC * c + (row - HC);
      buf_load_lds16(r1, st + ins * 1024, (grow * C + 8 * lc) * 2, 0);
    }
#pragma unroll
    for (int t = 0; t < Cfg::DMA2; ++t) {
      const int ins = w * Cfg::DMA2 + t;  // 8 LDS rows of 128 B per instruction
      const int row = 8 * ins + (l >> 3);
      const int lc = (l & 7) ^ swz(row, 128);
      buf_load_lds16(r2, st + Cfg::W1_BYTES + ins * 1024, (row * kHidden + HC * c + 8 * lc) * 2, 0);
    }
  };

  long g = 0;  // chunks consumed so far
  long tile = blockIdx.x;
  ZRow<TZ> zr;
  if (tile < ntiles) {
    issue_chunk(0);
    zr.load(x, tile * BP + w * PW + lq, M, hf);
  }
  __syncthreads();  // LN parameters, Ws2p fragments

  for (; tile < ntiles; tile += gridDim.x) {
    const long m = tile * BP + w * PW + lq;  // this lane's position
    const long tb0 = S2P ? (tile * BP) / NN : 0, tp0 = S2P ? tile * BP - tb0 * NN : 0;

    // ---- LN(x) -> B operands xf[ks]: lane (position lq, half hf) holds channels
    // 16 ks + 8 hf .. +7.
    bf16x8 xf[C / 16];
    {
      float s = 0.f;
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        float v[8];
        zr.get(ks, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) s += v[e];
      }
      s += __shfl_xor(s, 32, 64);
      const float mean = s * (1.0f / C);
      float q = 0.f;
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        float v[8];
        zr.get(ks, v);
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
        zr.get(ks, v);
        const float* pw = lnp + 16 * ks + 8 * hf;
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[ks][e] = (bf16)((v[e] - mean) * rstd * pw[e] + pw[C + e]);
      }
    }

    f32x16 y[4];  // y^T tiles [out rows 32 o ..][the wave's 32 positions]
#pragma unroll
    for (int o = 0; o < 4; ++o)
#pragma unroll
      for (int e = 0; e < 16; ++e) y[o][e] = 0.f;

#pragma unroll 1
    for (int c = 0; c < NCH; ++c, ++g) {
      // Chunk g landed (this lane's loads, then every wave's); stage (g + 1) & 1 was read
      // by chunk g - 1, which every wave has finished.
      __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
      __syncthreads();
      if (c + 1 < NCH || tile + gridDim.x < ntiles) issue_chunk(g + 1);
      const char* st = stage0 + (g & 1) * Cfg::STAGE;
      const char* w2s = st + Cfg::W1_BYTES;

#pragma unroll
      for (int i = 0; i < HC / 32; ++i) {
        f32x16 ha, hb;
#pragma unroll
        for (int e = 0; e < 16; ++e) ha[e] = hb[e] = 0.f;
#pragma unroll
        for (int ks = 0; ks < C / 16; ++ks) {
          const bf16x8 wa = *reinterpret_cast<const bf16x8*>(st + swz_off(32 * i + lq, 2 * ks + hf, 256));
          const bf16x8 wb = *reinterpret_cast<const bf16x8*>(st + swz_off(HC + 32 * i + lq, 2 * ks + hf, 256));
          ha = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa, xf[ks], ha, 0, 0, 0);
          hb = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wb, xf[ks], hb, 0, 0, 0);
        }
        // u[pos][hidden 32 i + 8 gq + 4 hf + e] = silu(h_a) h_b, 8-byte writes into the
        // wave's swizzled [32 pos][64 hidden] tile (128-byte rows).
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          bf16x4 u4;
#pragma unroll
          for (int e = 0; e < 4; ++e) u4[e] = (bf16)(siluf_(ha[4 * gq + e]) * hb[4 * gq + e]);
          *reinterpret_cast<bf16x4*>(ub + swz_off(lq, 4 * i + gq, 128) + 8 * hf) = u4;
        }
      }
      // The u tile is private to this wave, and one wave's LDS operations complete in order.
#pragma unroll
      for (int ks = 0; ks < HC / 16; ++ks) {
        const bf16x8 uf = *reinterpret_cast<const bf16x8*>(ub + swz_off(lq, 2 * ks + hf, 128));
#pragma unroll
        for (int o = 0; o < 4; ++o) {
          const bf16x8 wf = *reinterpret_cast<const bf16x8*>(w2s + swz_off(32 * o + lq, 2 * ks + hf, 128));
          y[o] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, uf, y[o], 0, 0, 0);
        }
      }
      __builtin_amdgcn_wave_barrier();  // u reads issued before the next chunk's writes
    }

    // ---- the residual operands, then the next tile's rows (their latency overlaps this
    // epilogue and the next tile's first chunk), all issued before any of them is used.
    // Loads complete in issue order: the rows issued first would hold up every wait on
    // the residual.
    // Lane (position lq, half hf) holds channels 32 o + 8 gq + 4 hf + e of y[o][4 gq + e].
    // Swapping the (gq = 2 p, gq = 2 p + 1) registers between lanes l and l + 32 leaves lane
    // hf with channels 32 o + 16 p + 8 hf + e, e = 0..7, in v[o][8 p + e]: 16-byte row
    // accesses, and the natural k order for the single_to_pair MFMAs.
    float v[4][16];
#pragma unroll
    for (int o = 0; o < 4; ++o)
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float a = y[o][8 * pp + e], b = y[o][8 * pp + 4 + e];
          permlane32_swap(a, b);
          v[o][8 * pp + e] = a;
          v[o][8 * pp + 4 + e] = b;
        }
    // Raw 16-byte pieces of the residual row, unpacked after the next tile's loads are
    // issued. Both groups of loads are unconditional (a position past M reads row M - 1,
    // never stored), so the compiler counts them exactly on every path.
    constexpr int RN = sizeof(TZ) == 2 ? 8 : 16;
    u32x4 rr[RN];
    {
      const TZ* row = out + min(m, M - 1) * C;
#pragma unroll
      for (int o = 0; o < 4; ++o)
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
          const TZ* src = row + 32 * o + 16 * pp + 8 * hf;
          if constexpr (sizeof(TZ) == 2) {
            rr[2 * o + pp] = *reinterpret_cast<const u32x4*>(src);
          } else {
            rr[2 * (2 * o + pp)] = *reinterpret_cast<const u32x4*>(src);
            rr[2 * (2 * o + pp) + 1] = *reinterpret_cast<const u32x4*>(src + 4);
          }
        }
    }
    zr.load(x, min((tile + gridDim.x) * BP + w * PW + lq, M - 1), M, hf);
    __builtin_amdgcn_sched_barrier(0);  // keep the row loads ahead of the residual's waits
    // the residual add runs for every lane (its loads are used outside the store's branch,
    // so the compiler keeps them where they are), only the stores are conditional
    {
      TZ* row = out + m * C;
#pragma unroll
      for (int o = 0; o < 4; ++o)
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
          float r8[8];
          if constexpr (sizeof(TZ) == 2) {
            const bf16x8 t = __builtin_bit_cast(bf16x8, rr[2 * o + pp]);
#pragma unroll
            for (int e = 0; e < 8; ++e) r8[e] = (float)t[e];
          } else {
            const f32x4 ra = __builtin_bit_cast(f32x4, rr[2 * (2 * o + pp)]);
            const f32x4 rb = __builtin_bit_cast(f32x4, rr[2 * (2 * o + pp) + 1]);
#pragma unroll
            for (int e = 0; e < 4; ++e) r8[e] = ra[e], r8[4 + e] = rb[e];
          }
#pragma unroll
          for (int e = 0; e < 8; ++e)
            v[o][8 * pp + e] = to_f32(from_f32<TZ>((accumulate ? r8[e] : 0.f) + v[o][8 * pp + e]));  // as stored
          if (m < M) {
            if constexpr (sizeof(TZ) == 2) {
              store_vec<bf16, 8>(row + 32 * o + 16 * pp + 8 * hf, &v[o][8 * pp]);
            } else {
              store_vec<float, 4>(row + 32 * o + 16 * pp + 8 * hf, &v[o][8 * pp]);
              store_vec<float, 4>(row + 32 * o + 16 * pp + 8 * hf + 4, &v[o][8 * pp + 4]);
            }
          }
        }
    }

    if constexpr (S2P) {
      // LN' of the updated row, then logits^T = Ws2p LN'^T on 32x32x16 MFMAs (heads 16..31
      // of the A operand are zero); k-step ks = 2 o + pp is channels 16 ks + 8 hf + e.
      float s = 0.f;
#pragma unroll
      for (int o = 0; o < 4; ++o)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += v[o][e];
      s += __shfl_xor(s, 32, 64);
      const float mean = s * (1.0f / C);
      float q = 0.f;
#pragma unroll
      for (int o = 0; o < 4; ++o)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float d = v[o][e] - mean;
          q += d * d;
        }
      q += __shfl_xor(q, 32, 64);
      const float rstd = rsqrtf(q * (1.0f / C) + s2p_eps);
      f32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        bf16x8 bfr;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int ch = 16 * ks + 8 * hf + e;
          bfr[e] = (bf16)((v[ks >> 1][8 * (ks & 1) + e] - mean) * rstd * lnp[2 * C + ch] + lnp[3 * C + ch]);
        }
        const bf16x8 afr = *reinterpret_cast<const bf16x8*>(s2pa + (ks * 64 + l) * 16);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afr, bfr, acc, 0, 0, 0);
      }
      // acc: lane (position, half hf) holds heads 8 gq + 4 hf + e; heads < 16 for gq < 2.
      // Batch item and in-plane position from the tile's (scalar) start.
      if (m < M) {
        long b = tb0, pos = tp0 + w * PW + lq;
        while (pos >= NN) {
          pos -= NN;
          ++b;
        }
#pragma unroll
        for (int gq = 0; gq < 2; ++gq)
#pragma unroll
          for (int e = 0; e < 4; ++e) logits[(b * kS2pHeads + 8 * gq + 4 * hf + e) * NN + pos] = acc[4 * gq + e];
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // no direct load outlives the block
}

// Pair transition at 256 channels (factor 4: W1 [2048][256], W2 [256][1024]) with bf16 GEMMs
// and a bf16 stream, persistent and weight-streaming: the hidden activations never leave the
// chip (the composed path wrote and re-read 2 KB of them per position). One 8-wave block per
// CU walks tiles of 128 positions; the hidden dim is walked in 32 chunks of 32 units. A
// chunk's W1 rows (a 0-15, b 0-15, a 16-31, b 16-31 of its units: 32 KB) and W2 columns
// (256 x 32: 16 KB) stream into a two-stage LDS ring by direct buffer->LDS loads one chunk
// ahead, swizzled so fragment reads are conflict-free. GEMM1: wave (rb = w & 1, pb = w >> 1)
// computes the 32 rows 32 rb .. (a and b of 16 units) for positions 32 pb .. from its
// LayerNormed rows held in registers; a unit's a and b land in one lane (accumulator rows r and
// r + 16), so u = silu(a) b is formed in registers and written to an LDS tile [128][32].
// GEMM2: wave w accumulates y^T rows 32 w .. (its 32 output channels) for all 128 positions
// in registers over the whole tile. Epilogue: lane-pair swaps give 16-byte row pieces for
// the residual add and the stores.
struct Trans256 {
  static constexpr int C = 256;
  static constexpr int HID = 4 * C;                 // 1024 hidden units
  static constexpr int HC = 32;                     // units per chunk
  static constexpr int NCH = HID / HC;              // 32 chunks per tile
  static constexpr int BP = 128;                    // positions per tile
  static constexpr int NW = 8;
  static constexpr int NT = 64 * NW;
  static constexpr int W1_BYTES = 2 * HC * C * 2;   // 64 rows x 512 B
  static constexpr int W2_BYTES = C * HC * 2;       // 256 rows x 64 B
  static constexpr int STAGE = W1_BYTES + W2_BYTES; // 48 KB
  static constexpr int DMA1 = W1_BYTES / 1024 / NW; // 4
  static constexpr int DMA2 = W2_BYTES / 1024 / NW; // 2
};

// Byte offsets in the chunk stage: W1 rows of 512 B (16-byte piece c XOR row & 15), W2 and
// the u tile rows of 64 B (piece c XOR (row >> 2) & 3: 16 consecutive rows at one logical
// piece cover the 16 bank groups).
PF_DEVICE int t256_w1(int r, int c) { return r * 512 + 16 * (c ^ (r & 15)); }
PF_DEVICE int t256_r64(int r, int c) { return r * 64 + 16 * (c ^ ((r >> 2) & 3)); }

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

__global__ __launch_bounds__(Trans256::NT, 1) void pair_transition256_kernel(
    const bf16* __restrict__ x, bf16* __restrict__ out, const float* __restrict__ lnw, const float* __restrict__ lnb,
    float eps, const bf16* __restrict__ W1, const bf16* __restrict__ W2, long M, int accumulate) {
  using Cfg = Trans256;
  constexpr int C = Cfg::C, HC = Cfg::HC, NCH = Cfg::NCH, BP = Cfg::BP;
  __shared__ __attribute__((aligned(16))) char ring[2 * Cfg::STAGE];
  __shared__ __attribute__((aligned(16))) char ut[BP * HC * 2];  // u [pos][unit], 64-byte rows
  __shared__ float lnp[2 * C];

  const int w = wave_id();
  const int l = lane_id();
  const int lq = l & 31, hf = l >> 5;
  const int rb = w & 1, pb = w >> 1;
  const long ntiles = (M + BP - 1) / BP;
  const long total = blockIdx.x < ntiles ? ((ntiles - 1 - blockIdx.x) / gridDim.x + 1) * NCH : 0;

  for (int i = threadIdx.x; i < C; i += Cfg::NT) {
    lnp[i] = lnw[i];
    lnp[C + i] = lnb[i];
  }
  const i32x4_t r1 = buf_rsrc_words(W1, 2 * Cfg::HID * C * 2);
  const i32x4_t r2 = buf_rsrc_words(W2, C * Cfg::HID * 2);
  auto issue_chunk = [&](long gg) {
    const int c = (int)(gg % NCH);
    char* st = ring + (gg & 1) * Cfg::STAGE;
#pragma unroll
    for (int t = 0; t < Cfg::DMA1; ++t) {
      const int ins = w * Cfg::DMA1 + t;  // two 512-byte rows per instruction
      const int row = 2 * ins + (l >> 5);
      const int lc = (l & 31) ^ (row & 15);
      const int blk = row >> 4;  // a (even) or b (odd) rows of units 16 (blk >> 1) ..
      const int src = (blk & 1) * Cfg::HID + HC * c + 16 * (blk >> 1) + (row & 15);
      buf_load_lds16_async(r1, st + ins * 1024, (src * C + 8 * lc) * 2, 0);
    }
#pragma unroll
    for (int t = 0; t < Cfg::DMA2; ++t) {
      const int ins = w * Cfg::DMA2 + t;  // sixteen 64-byte rows per instruction
      const int o = 16 * ins + (l >> 2);
      const int lc = (l & 3) ^ ((o >> 2) & 3);
      buf_load_lds16_async(r2, st + Cfg::W1_BYTES + ins * 1024, (o * Cfg::HID + HC * c + 8 * lc) * 2, 0);
    }
  };
  // this lane's half row for GEMM1: channels 16 ks + 8 hf .. +7 of position 32 pb + lq
  u32x4 zr[C / 16];
  auto load_half = [&](long tl) {
    const long m = min(tl * BP + 32 * pb + lq, M - 1);  // past M: row M - 1, never stored
    const bf16* src = x + m * C + 8 * hf;
#pragma unroll
    for (int ks = 0; ks < C / 16; ++ks) zr[ks] = *reinterpret_cast<const u32x4*>(src + 16 * ks);
  };

  long g = 0;
  long tile = blockIdx.x;
  if (total > 0) issue_chunk(0);
  __syncthreads();  // LN parameters

  for (; tile < ntiles; tile += gridDim.x) {
    load_half(tile);  // rows dead after the LayerNorm (no register set held across the chunks)
    // ---- LN -> B operands xf[ks]
    bf16x8 xf[C / 16];
    {
      float s = 0.f;
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        const bf16x8 t = __builtin_bit_cast(bf16x8, zr[ks]);
#pragma unroll
        for (int e = 0; e < 8; ++e) s += (float)t[e];
      }
      s += __shfl_xor(s, 32, 64);
      const float mean = s * (1.0f / C);
      float q = 0.f;
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        const bf16x8 t = __builtin_bit_cast(bf16x8, zr[ks]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = (float)t[e] - mean;
          q += d * d;
        }
      }
      q += __shfl_xor(q, 32, 64);
      const float rstd = rsqrtf(q * (1.0f / C) + eps);
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        const bf16x8 t = __builtin_bit_cast(bf16x8, zr[ks]);
        const float* pw = lnp + 16 * ks + 8 * hf;
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[ks][e] = (bf16)(((float)t[e] - mean) * rstd * pw[e] + pw[C + e]);
      }
    }
    f32x16 y[4];  // y^T [out rows 32 w ..][positions 32 p ..]
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int e = 0; e < 16; ++e) y[p][e] = 0.f;

#pragma unroll 1
    for (int c = 0; c < NCH; ++c, ++g) {
      // Chunk g landed in every wave; the previous chunk's GEMM2 (reads of ring slot
      // (g + 1) & 1 and of ut) is done in every wave.
      __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
      lds_barrier();
      if (g + 1 < total) issue_chunk(g + 1);
      const char* st = ring + (g & 1) * Cfg::STAGE;
      f32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        const bf16x8 wf = *reinterpret_cast<const bf16x8*>(st + t256_w1(32 * rb + lq, 2 * ks + hf));
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, xf[ks], acc, 0, 0, 0);
      }
      // acc[e] (e < 8): a of unit 16 rb + 8 (e >> 2) + 4 hf + (e & 3); acc[e + 8]: its b
      {
        const int pos = 32 * pb + lq;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const int u0 = 16 * rb + 8 * (e >> 2) + 4 * hf + (e & 3);
          bf16x2 v2;
          v2[0] = (bf16)(siluf_(acc[e]) * acc[e + 8]);
          v2[1] = (bf16)(siluf_(acc[e + 1]) * acc[e + 9]);
          *reinterpret_cast<bf16x2*>(ut + t256_r64(pos, u0 >> 3) + 2 * (u0 & 7)) = v2;
        }
      }
      lds_barrier();  // ut complete
      const char* w2s = st + Cfg::W1_BYTES;
#pragma unroll
      for (int ks = 0; ks < HC / 16; ++ks) {
        const bf16x8 af = *reinterpret_cast<const bf16x8*>(w2s + t256_r64(32 * w + lq, 2 * ks + hf));
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const bf16x8 uf = *reinterpret_cast<const bf16x8*>(ut + t256_r64(32 * p + lq, 2 * ks + hf));
          y[p] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, uf, y[p], 0, 0, 0);
        }
      }
    }

    // ---- epilogue: lane (position 32 p + lq, half hf) holds channels 32 w + 8 gq + 4 hf + e
    // of y[p][4 gq + e]; swapping (gq = 2 q, 2 q + 1) between lanes l and l + 32 leaves lane hf
    // with channels 32 w + 16 q + 8 hf + e in v[8 q + e]: 16-byte row pieces.
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      float v[16];
#pragma unroll
      for (int qq = 0; qq < 2; ++qq)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float a = y[p][8 * qq + e], b = y[p][8 * qq + 4 + e];
          permlane32_swap(a, b);
          v[8 * qq + e] = a;
          v[8 * qq + 4 + e] = b;
        }
      const long m = tile * BP + 32 * p + lq;
      const long mr = min(m, M - 1);
      u32x4 rr[2];
#pragma unroll
      for (int qq = 0; qq < 2; ++qq)
        rr[qq] = *reinterpret_cast<const u32x4*>(out + mr * C + 32 * w + 16 * qq + 8 * hf);
      if (m < M) {
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
          const bf16x8 t = __builtin_bit_cast(bf16x8, rr[qq]);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[8 * qq + e] += accumulate ? (float)t[e] : 0.f;
          store_vec<bf16, 8>(out + m * C + 32 * w + 16 * qq + 8 * hf, &v[8 * qq]);
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // no direct load outlives the block
}

// Standalone single_to_pair: LN'(z) Ws2p^T -> logits [B][16][N][N].
template <class TZ, class TC>
__global__ __launch_bounds__(256) void single_to_pair_kernel(const TZ* __restrict__ z, const float* __restrict__ lnw,
                                                             const float* __restrict__ lnb, float eps,
                                                             const TC* __restrict__ Ws, float* __restrict__ logits,
                                                             long M, long NN) {
  constexpr int BM = tr_bm<TC>();
  constexpr int ALD = kC + lds_pad<TC>();
  __shared__ __attribute__((aligned(16))) TC A[BM * ALD];
  const long m0 = (long)blockIdx.x * BM;
  auto zrow = [&](int p) -> const TZ* { return m0 + p < M ? z + (m0 + p) * kC : nullptr; };
  ln_tile_to_lds<TZ, TC, kC, BM, 256>(zrow, lnw, lnb, eps, A, ALD);
  __syncthreads();
  s2p_store<TC, BM>(A, ALD, Ws, logits, m0, M, NN);
}

// FusedPairBias (triton/fused_pair_bias.py:348-416): LN(z) proj_w^T -> [B][H][N][N] in z's
// dtype, plus (1 - mask[b][j]) * (-1e9) when a [B][N] mask is given. Computed in fp32 (the
// reference's projection runs at fp32 accuracy, fused_pair_bias.py:198): the LN tile is
// fp32 and the projection uses v_mfma_f32_16x16x4f32 against proj_w padded to 16 rows.
template <class TZ>
__global__ __launch_bounds__(256) void pair_bias_kernel(const TZ* __restrict__ z, const float* __restrict__ lnw,
                                                        const float* __restrict__ lnb, float eps,
                                                        const float* __restrict__ w16, const float* __restrict__ mask,
                                                        TZ* __restrict__ out, int H, long M, long NN, int N) {
  constexpr int BM = 32;
  constexpr int ALD = kC + lds_pad<float>();
  __shared__ __attribute__((aligned(16))) float A[BM * ALD];
  const long m0 = (long)blockIdx.x * BM;
  auto zrow = [&](int p) -> const TZ* { return m0 + p < M ? z + (m0 + p) * kC : nullptr; };
  ln_tile_to_lds<TZ, float, kC, BM, 256>(zrow, lnw, lnb, eps, A, ALD);
  __syncthreads();
  const int w = wave_id();
  const int l = lane_id();
  if (w >= BM / 16) return;
  f32x4 acc[1][1];
  zero_acc(acc);
  int wrow[1] = {0};
  gemm16_lds_x_w<float, kC, 1, 1>(acc, A, ALD, w * 16, w16, kC, wrow);
  const int h = l & 15;
  if (h >= H) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const long m = m0 + w * 16 + 4 * (l >> 4) + e;
    if (m >= M) continue;
    const long b = m / NN;
    const long pos = m % NN;
    float v = acc[0][0][e];
    if (mask) v += (1.0f - mask[b * N + pos % N]) * (-1e9f);
    out[(b * H + h) * NN + pos] = from_f32<TZ>(v);
  }
}

template <class TZ, class TC>
int transition_launch(const void* x, const float* lnw, const float* lnb, float eps, const void* w1, const void* w2,
                      long M, void* out, int accumulate, const float* s2p_w, const float* s2p_b, float s2p_eps,
                      const void* ws2p, float* logits, long NN, hipStream_t s) {
  pf::KernelTimer timer("pair_transition", s);
  if constexpr (sizeof(TC) == 2) {
    const long ntiles = (M + TransWs::BP - 1) / TransWs::BP;
    const unsigned nblk = (unsigned)std::min<long>(ntiles, pf::cu_count());
    if (logits)
      pair_transition_ws_kernel<TZ, true><<<nblk, TransWs::NT, 0, s>>>(
          (const TZ*)x, (TZ*)out, lnw, lnb, eps, (const bf16*)w1, (const bf16*)w2, M, accumulate, s2p_w, s2p_b,
          s2p_eps, (const bf16*)ws2p, logits, NN);
    else
      pair_transition_ws_kernel<TZ, false><<<nblk, TransWs::NT, 0, s>>>(
          (const TZ*)x, (TZ*)out, lnw, lnb, eps, (const bf16*)w1, (const bf16*)w2, M, accumulate, nullptr, nullptr,
          0.f, nullptr, nullptr, NN);
    timer.stop();
    return pf::check_launch("pair_transition");
  }
  constexpr int BM = tr_bm<TC>();
  dim3 grid((unsigned)((M + BM - 1) / BM));
  if (logits)
    pair_transition_kernel<TZ, TC, true><<<grid, 256, 0, s>>>((const TZ*)x, (TZ*)out, lnw, lnb, eps, (const TC*)w1,
                                                             (const TC*)w2, M, accumulate, s2p_w, s2p_b, s2p_eps,
                                                             (const TC*)ws2p, logits, NN);
  else
    pair_transition_kernel<TZ, TC, false><<<grid, 256, 0, s>>>((const TZ*)x, (TZ*)out, lnw, lnb, eps, (const TC*)w1,
                                                              (const TC*)w2, M, accumulate, nullptr, nullptr, 0.f,
                                                              nullptr, nullptr, NN);
  timer.stop();
  return pf::check_launch("pair_transition");
}

template <class TZ, class TC>
int s2p_launch(const void* z, const float* lnw, const float* lnb, float eps, const void* ws, float* logits, long M,
               long NN, hipStream_t s) {
  constexpr int BM = tr_bm<TC>();
  dim3 grid((unsigned)((M + BM - 1) / BM));
  single_to_pair_kernel<TZ, TC><<<grid, 256, 0, s>>>((const TZ*)z, lnw, lnb, eps, (const TC*)ws, logits, M, NN);
  return pf::check_launch("single_to_pair");
}

// single_to_pair for other channel counts (a multiple of 64; the 256-channel trunk): one wave
// per position, fp32 LayerNorm statistics, the normalised row rounded to the GEMM operand
// dtype (the reference's LN output under autocast), 16 fp32 dot products reduced over the wave.
template <class TZ, class TC>
__global__ __launch_bounds__(256) void single_to_pair_generic_kernel(const TZ* __restrict__ z,
                                                                     const float* __restrict__ lnw,
                                                                     const float* __restrict__ lnb, float eps,
                                                                     const TC* __restrict__ w, float* __restrict__ logits,
                                                                     long M, long NN, int C) {
  const long row = (long)blockIdx.x * 4 + wave_id();
  if (row >= M) return;
  const int l = lane_id();
  const TZ* x = z + row * C;
  float s = 0.f;
  for (int c = l; c < C; c += 64) s += to_f32(x[c]);
  const float mean = group_sum<64>(s) / C;
  float q = 0.f;
  for (int c = l; c < C; c += 64) {
    const float d = to_f32(x[c]) - mean;
    q += d * d;
  }
  const float rstd = rsqrtf(group_sum<64>(q) / C + eps);
  float acc[kS2pHeads];
#pragma unroll
  for (int h = 0; h < kS2pHeads; ++h) acc[h] = 0.f;
  for (int c = l; c < C; c += 64) {
    const float xn = to_f32(from_f32<TC>((to_f32(x[c]) - mean) * rstd * lnw[c] + lnb[c]));
#pragma unroll
    for (int h = 0; h < kS2pHeads; ++h) acc[h] += xn * to_f32(w[(size_t)h * C + c]);
  }
  float mine = 0.f;
#pragma unroll
  for (int h = 0; h < kS2pHeads; ++h) {
    const float t = group_sum<64>(acc[h]);
    if (l == h) mine = t;
  }
  if (l < kS2pHeads) logits[((row / NN) * kS2pHeads + l) * NN + row % NN] = mine;
}

// bf16 operands, C in {64, 256}: 16 positions per wave. The wave LayerNorms its rows with
// C / 8 lanes per row (16-byte loads), stores the normalised rows rounded to bf16 in its LDS
// tile, and one 16x16 MFMA block per 32 channels gives the 16 positions x 16 heads logits
// (W [16][C] fragments from L1).
template <class TZ, int C>
__global__ __launch_bounds__(256) void single_to_pair_mfma_kernel(const TZ* __restrict__ z,
                                                                  const float* __restrict__ lnw,
                                                                  const float* __restrict__ lnb, float eps,
                                                                  const bf16* __restrict__ w, float* __restrict__ logits,
                                                                  long M, long NN) {
  constexpr int LPR = C / 8;
  constexpr int RPP = 64 / LPR;  // rows per pass
  constexpr int NPASS = 16 / RPP;
  constexpr int NV = sizeof(TZ) == 2 ? 1 : 2;  // 16-byte loads per lane per pass
  constexpr int LDC = C + 8;
  static_assert(C % 64 == 0 && C <= 256, "64 to 256 channels");
  __shared__ __attribute__((aligned(16))) bf16 tile[4][16 * LDC];
  const int wv = wave_id();
  const int l = lane_id();
  bf16* t = tile[wv];
  const long r0 = ((long)blockIdx.x * 4 + wv) * 16;
  const int c0 = (l % LPR) * 8;
  // Every pass's row piece is requested before any is used (one memory round trip per
  // wave, not one per pass); the lane's LayerNorm parameters are read once.
  u32x4 raw[NPASS][NV];
#pragma unroll
  for (int pass = 0; pass < NPASS; ++pass) {
    const long row = min(r0 + pass * RPP + l / LPR, M - 1);
    const TZ* src = z + row * C + c0;
#pragma unroll
    for (int j = 0; j < NV; ++j) raw[pass][j] = *reinterpret_cast<const u32x4*>(src + 4 * j);
  }
  float lw[8], lbv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    lw[e] = lnw[c0 + e];
    lbv[e] = lnb[c0 + e];
  }
#pragma unroll
  for (int pass = 0; pass < NPASS; ++pass) {
    const int rr = pass * RPP + l / LPR;
    float v[8];
    if constexpr (sizeof(TZ) == 2) {
      const bf16x8 b8 = __builtin_bit_cast(bf16x8, raw[pass][0]);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (float)b8[e];
    } else {
      const f32x4 a = __builtin_bit_cast(f32x4, raw[pass][0]), b = __builtin_bit_cast(f32x4, raw[pass][NV - 1]);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = a[e], v[e + 4] = b[e];
    }
    float sm = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sm += v[e];
    const float mean = (LPR >= 16 ? row_group_sum<(LPR >= 32 ? 32 : 16)>(sm) : group_sum<LPR>(sm)) / C;
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = v[e] - mean;
      q += d * d;
    }
    const float rstd = rsqrtf((LPR >= 16 ? row_group_sum<(LPR >= 32 ? 32 : 16)>(q) : group_sum<LPR>(q)) / C + eps);
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = (v[e] - mean) * rstd * lw[e] + lbv[e];
    store_vec<bf16, 8>(t + rr * LDC + c0, y);
  }
  __syncthreads();  // the tile's rows are in LDS
  using MF = Mfma<bf16>;
  const int r = l & 15;
  const int kq = (l >> 4) * MF::KPL;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k0 = 0; k0 < C; k0 += MF::K16) {
    const MF::Frag af = MF::load(t + r * LDC + k0 + kq);
    const MF::Frag bf = MF::load(w + (size_t)r * C + k0 + kq);
    MF::mma16(acc, af, bf);
  }
  // acc[e]: position r0 + 4 (l >> 4) + e, head l & 15. The block's 64 positions go through
  // LDS so each head's run leaves as 16-byte stores (256 contiguous bytes per head) instead of
  // 4-byte stores scattered over the 16 head planes.
  __shared__ __attribute__((aligned(16))) float ot[kS2pHeads][64 + 4];
#pragma unroll
  for (int e = 0; e < 4; ++e) ot[r][16 * wv + 4 * (l >> 4) + e] = acc[e];
  __syncthreads();
  const long p0 = (long)blockIdx.x * 64;
  if (NN % 64 == 0 && p0 + 64 <= M) {
    // one batch item, 16-byte aligned runs
    const int h = threadIdx.x >> 4, pc = threadIdx.x & 15;
    *reinterpret_cast<f32x4*>(logits + ((p0 / NN) * kS2pHeads + h) * NN + p0 % NN + 4 * pc) =
        *reinterpret_cast<const f32x4*>(&ot[h][4 * pc]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = threadIdx.x + 256 * i;  // (head, position) = (k >> 6, k & 63)
      const long row = p0 + (k & 63);
      if (row < M) logits[((row / NN) * kS2pHeads + (k >> 6)) * NN + row % NN] = ot[k >> 6][k & 63];
    }
  }
}

template <class TZ, class TC>
int s2p_generic_launch(const void* z, const float* lnw, const float* lnb, float eps, const void* w, float* logits,
                       long M, long NN, int C, hipStream_t s) {
  if constexpr (sizeof(TC) == 2) {
    const bool al = pf::aligned16(z) && pf::aligned16(w);
    const unsigned grid = (unsigned)((M + 63) / 64);
    if (al && C == 256) {
      single_to_pair_mfma_kernel<TZ, 256><<<grid, 256, 0, s>>>((const TZ*)z, lnw, lnb, eps, (const bf16*)w, logits,
                                                               M, NN);
      return pf::check_launch("single_to_pair");
    }
    if (al && C == 64) {
      single_to_pair_mfma_kernel<TZ, 64><<<grid, 256, 0, s>>>((const TZ*)z, lnw, lnb, eps, (const bf16*)w, logits, M,
                                                              NN);
      return pf::check_launch("single_to_pair");
    }
  }
  single_to_pair_generic_kernel<TZ, TC><<<(unsigned)((M + 3) / 4), 256, 0, s>>>((const TZ*)z, lnw, lnb, eps,
                                                                                 (const TC*)w, logits, M, NN, C);
  return pf::check_launch("single_to_pair");
}

#define PF_DISPATCH_ZC(zd, cd, FN, ...)                                                        \
  ((zd) == PF_F32 && (cd) == PF_F32 ? FN<float, float>(__VA_ARGS__)                            \
   : (zd) == PF_F32                 ? FN<float, bf16>(__VA_ARGS__)                             \
                                    : FN<bf16, bf16>(__VA_ARGS__))

}  // namespace

extern "C" {

int pf_pair_transition_fwd(const void* x, const float* ln_w, const float* ln_b, float eps, const void* w1,
                           const void* w2, long M, int C, int factor, int zdtype, int cdtype, void* out, int accumulate,
                           const float* s2p_ln_w, const float* s2p_ln_b, float s2p_eps, const void* w_s2p,
                           float* pair_logits, long NN, void* stream) {
  PF_REQUIRE(x && ln_w && ln_b && w1 && w2 && out, PF_ERR_INVALID_ARG, "pf_pair_transition_fwd: null pointer");
  const bool c256 = C == Trans256::C && factor == 4 && zdtype == PF_BF16 && cdtype == PF_BF16 && !pair_logits;
  PF_REQUIRE((C == kC && factor == 4) || c256, PF_ERR_UNSUPPORTED,
             "pf_pair_transition_fwd: C=%d factor=%d (built: C=128, factor 4; C=256, factor 4 with bf16 z and GEMMs "
             "and no fused single_to_pair)",
             C, factor);
  PF_REQUIRE(M >= 0, PF_ERR_INVALID_ARG, "pf_pair_transition_fwd: M=%ld", M);
  PF_REQUIRE((zdtype == PF_F32 || zdtype == PF_BF16) && (cdtype == PF_F32 || cdtype == PF_BF16) &&
                 !(zdtype == PF_BF16 && cdtype == PF_F32),
             PF_ERR_UNSUPPORTED, "pf_pair_transition_fwd: dtype pair (%d, %d)", zdtype, cdtype);
  PF_REQUIRE(!pair_logits || (s2p_ln_w && s2p_ln_b && w_s2p && NN > 0 && M % NN == 0), PF_ERR_INVALID_ARG,
             "pf_pair_transition_fwd: fused single_to_pair needs its LN, weight and NN dividing M");
  PF_REQUIRE(pf::aligned16(x) && pf::aligned16(out) && pf::aligned16(w1) && pf::aligned16(w2), PF_ERR_ALIGNMENT,
             "pf_pair_transition_fwd: pointers must be 16-byte aligned");
  if (M == 0) return pf::ok();
  hipStream_t s = pf::as_stream(stream);
  if (c256) {
    const long ntiles = (M + Trans256::BP - 1) / Trans256::BP;
    const unsigned nblk = (unsigned)std::min<long>(ntiles, pf::cu_count());
    pf::KernelTimer timer("pair_transition", s);
    pair_transition256_kernel<<<nblk, Trans256::NT, 0, s>>>((const bf16*)x, (bf16*)out, ln_w, ln_b, eps,
                                                            (const bf16*)w1, (const bf16*)w2, M, accumulate);
    timer.stop();
    return pf::check_launch("pair_transition256");
  }
  return PF_DISPATCH_ZC(zdtype, cdtype, transition_launch, x, ln_w, ln_b, eps, w1, w2, M, out, accumulate, s2p_ln_w,
                        s2p_ln_b, s2p_eps, w_s2p, pair_logits, NN, s);
}

int pf_pair_bias_fwd(const void* z, int zdtype, const float* ln_w, const float* ln_b, float eps,
                     const float* proj_w16, int H, const float* mask, void* out, int B, int N, int C, void* stream) {
  PF_REQUIRE(z && ln_w && ln_b && proj_w16 && out, PF_ERR_INVALID_ARG, "pf_pair_bias_fwd: null pointer");
  PF_REQUIRE(C == kC && H >= 1 && H <= 16, PF_ERR_UNSUPPORTED, "pf_pair_bias_fwd: C=%d H=%d (built: C=128, H<=16)",
             C, H);
  PF_REQUIRE(B >= 0 && N >= 0, PF_ERR_INVALID_ARG, "pf_pair_bias_fwd: B=%d N=%d", B, N);
  PF_REQUIRE(zdtype == PF_F32 || zdtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_pair_bias_fwd: zdtype %d", zdtype);
  const long NN = (long)N * N, M = (long)B * NN;
  if (M == 0) return pf::ok();
  hipStream_t s = pf::as_stream(stream);
  dim3 grid((unsigned)((M + 31) / 32));
  if (zdtype == PF_F32)
    pair_bias_kernel<float><<<grid, 256, 0, s>>>((const float*)z, ln_w, ln_b, eps, proj_w16, mask, (float*)out, H, M,
                                                 NN, N);
  else
    pair_bias_kernel<bf16><<<grid, 256, 0, s>>>((const bf16*)z, ln_w, ln_b, eps, proj_w16, mask, (bf16*)out, H, M,
                                                NN, N);
  return pf::check_launch("pair_bias");
}

int pf_single_to_pair_fwd(const void* z, const float* ln_w, const float* ln_b, float eps, const void* w_s2p, long M,
                          int C, int H, long NN, int zdtype, int cdtype, float* pair_logits, void* stream) {
  PF_REQUIRE(z && ln_w && ln_b && w_s2p && pair_logits, PF_ERR_INVALID_ARG, "pf_single_to_pair_fwd: null pointer");
  PF_REQUIRE(H == kS2pHeads && (C == kC || (C > 0 && C % 64 == 0)), PF_ERR_UNSUPPORTED,
             "pf_single_to_pair_fwd: C=%d H=%d (built: H=16, C a multiple of 64)", C, H);
  PF_REQUIRE(NN > 0 && M >= 0 && M % NN == 0, PF_ERR_INVALID_ARG, "pf_single_to_pair_fwd: M=%ld NN=%ld", M, NN);
  PF_REQUIRE((zdtype == PF_F32 || zdtype == PF_BF16) && (cdtype == PF_F32 || cdtype == PF_BF16) &&
                 !(zdtype == PF_BF16 && cdtype == PF_F32),
             PF_ERR_UNSUPPORTED, "pf_single_to_pair_fwd: dtype pair (%d, %d)", zdtype, cdtype);
  if (M == 0) return pf::ok();
  hipStream_t s = pf::as_stream(stream);
  if (C != kC)
    return PF_DISPATCH_ZC(zdtype, cdtype, s2p_generic_launch, z, ln_w, ln_b, eps, w_s2p, pair_logits, M, NN, C, s);
  return PF_DISPATCH_ZC(zdtype, cdtype, s2p_launch, z, ln_w, ln_b, eps, w_s2p, pair_logits, M, NN, s);
}

}  // extern "C"
