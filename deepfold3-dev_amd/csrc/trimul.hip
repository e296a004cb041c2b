// Triangle multiplicative update (outgoing and incoming) in three launches:
//
//   K1 trimul_project:  x = LN_in(z); a, b = sigmoid(x Wg^T) * (x Wp^T) * mask,
//                       stored channel-major as planes P, Q [B*C][Np][Np].
//   K2 trimul_contract: X_c = P_c Q_c^T for every (batch, channel) plane.
//   K3 trimul_output:   update = sigmoid(LN_in(z) Wog^T) * (LN_out(X) Wo^T),
//                       written to `out` or added into it (fused residual).
//
// Reference semantics: TriangleMulOutgoing/Incoming (src/deepfold3/model/ops.py:412-473,
// einsums ops.py:58-98) and the channel-major fused_trimul (triton/fused_trimul.py:264-366).
//
// Layout trick: the outgoing contraction X_ij = sum_k a_ik b_jk is P Q^T with P = a
// stored [i][k] and Q = b stored [j][k]. For the incoming one, X_ij = sum_k a_kj b_ki,
// K1 walks z along columns and stores the planes transposed (P = b^T as [i][k],
// Q = a^T as [j][k]), so K2 is always the same k-contiguous "NT" GEMM.
#include <algorithm>
#include <type_traits>

#include "capi.h"
#include "common.h"
#include "mhr.h"

namespace {

template <class TC>
constexpr int trimul_bm() { return sizeof(TC) == 2 ? 64 : 32; }
// Threads of the generic K1 / K3 blocks: 8 waves from 256 channels (each wave's accumulators
// and LN_out columns halve; 4 waves hold 512 VGPRs per lane at C=256, one wave per SIMD).
template <int C>
constexpr int trimul_nt() { return C >= 256 ? 512 : 256; }

// ------------------------------------------------------------------ K1
// Packed weights w4 [4C][C]: for channel block j (16 channels), rows 64j + 16*kind + r,
// kind 0 = a projection, 1 = a gate, 2 = b projection, 3 = b gate (channel 16j + r).
// NORM = false takes z as already normalised (the training entry, whose input LayerNorm
// runs outside).
template <class TZ, class TC, int C, bool NORM = true>
__global__ __launch_bounds__(trimul_nt<C>()) void trimul_project_kernel(const TZ* __restrict__ z, const float* __restrict__ mask,
                                                             const float* __restrict__ lnw,
                                                             const float* __restrict__ lnb, float eps,
                                                             const TC* __restrict__ w4, TC* __restrict__ planes,
                                                             int B, int N, int Np, int outgoing) {
  constexpr int BM = trimul_bm<TC>();
  constexpr int NT = trimul_nt<C>();
  constexpr int LDA = C + lds_pad<TC>();
  constexpr int SLD = BM + lds_pad<TC>();
  constexpr int RB = BM / 16;
  constexpr int CBW = C / 16 / (NT / 64);  // channel blocks per wave
  constexpr int A_BYTES = BM * LDA * (int)sizeof(TC);
  constexpr int S_BYTES = 2 * C * SLD * (int)sizeof(TC);
  __shared__ __attribute__((aligned(16))) char smem[(A_BYTES > S_BYTES ? A_BYTES : S_BYTES)];
  __shared__ float mk[BM];
  TC* A = reinterpret_cast<TC*>(smem);
  TC* S = reinterpret_cast<TC*>(smem);

  const int t0 = blockIdx.x * BM;
  const int line = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const TZ* zb = z + (size_t)b * N * N * C;
  auto pos_of = [&](int p) -> long {
    const int t = t0 + p;
    if (line >= N || t >= N) return -1;
    return outgoing ? (long)line * N + t : (long)t * N + line;
  };
  auto rowptr = [&](int p) -> const TZ* {
    const long pos = pos_of(p);
    return pos < 0 ? nullptr : zb + pos * C;
  };
  if constexpr (NORM)
    ln_tile_to_lds<TZ, TC, C, BM, NT>(rowptr, lnw, lnb, eps, A, LDA);
  else
    copy_tile_to_lds<TZ, TC, C, BM, NT>(rowptr, A, LDA);
  if (tid < BM) {
    const long pos = pos_of(tid);
    mk[tid] = pos < 0 ? 0.f : mask[(size_t)b * N * N + pos];
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
  __syncthreads();  // A is dead; its LDS becomes the staging tile S [2][C][SLD]

#pragma unroll
  for (int cbi = 0; cbi < CBW; ++cbi) {
    const int ch = (w * CBW + cbi) * 16 + (l & 15);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float av[4], bv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p = rb * 16 + 4 * (l >> 4) + r;
        const float m = mk[p];
        av[r] = sigmoidf_(acc[rb][4 * cbi + 1][r]) * acc[rb][4 * cbi + 0][r] * m;
        bv[r] = sigmoidf_(acc[rb][4 * cbi + 3][r]) * acc[rb][4 * cbi + 2][r] * m;
      }
      const int p0 = rb * 16 + 4 * (l >> 4);
      store_vec<TC, 4>(S + ch * SLD + p0, av);
      store_vec<TC, 4>(S + (C + ch) * SLD + p0, bv);
    }
  }
  __syncthreads();

  // Rows (plane, channel) of BM contiguous tokens.
  constexpr int VEC = 16 / sizeof(TC);
  constexpr int CPR = BM / VEC;  // 16-byte chunks per row
  const size_t plane_elems = (size_t)Np * Np;
  for (int idx = tid; idx < 2 * C * CPR; idx += NT) {
    const int row = idx / CPR;
    const int chunk = idx % CPR;
    const int plane = row / C;
    const int ch = row % C;
    TC* dst = planes + ((size_t)plane * B * C + (size_t)b * C + ch) * plane_elems + (size_t)line * Np + t0 + chunk * VEC;
    *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(S + row * SLD + chunk * VEC);
  }
}

// ------------------------------------------------------------------ K2
// X[g] = P[g] Q[g]^T, all [Np][Np] with k contiguous. 128x128 tile per block,
// four waves in a 2x2 grid of 64x64, double-buffered LDS k-tiles.
template <class TC>
struct ContractCfg {
  static constexpr int BMN = 128;
  static constexpr int KT = sizeof(TC) == 2 ? 64 : 32;
  static constexpr int LDK = KT + lds_pad<TC>();
  static constexpr int TILE_ELEMS = BMN * LDK;
  static constexpr int STAGE_BYTES = 2 * TILE_ELEMS * (int)sizeof(TC);
  static constexpr int OUT_LD = BMN + lds_pad<TC>();
  static constexpr int OUT_BYTES = BMN * OUT_LD * (int)sizeof(TC);
  static constexpr int SMEM = (2 * STAGE_BYTES > OUT_BYTES) ? 2 * STAGE_BYTES : OUT_BYTES;
};

template <class TC>
__global__ __launch_bounds__(256) void trimul_contract_kernel(const TC* __restrict__ P, const TC* __restrict__ Q,
                                                              TC* __restrict__ X, int G, int Np, int xcd_remap) {
  using Cfg = ContractCfg<TC>;
  using M = Mfma<TC>;
  constexpr int BMN = Cfg::BMN, KT = Cfg::KT, LDK = Cfg::LDK;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  TC* lds = reinterpret_cast<TC*>(smem);

  const int tiles1 = Np / BMN;
  const int tiles = tiles1 * tiles1;
  // Block -> (plane, tile). Blocks are dispatched round-robin over the 8 XCDs; with
  // the remap, XCD x walks planes x, x+8, ... one plane's tiles at a time, so a plane's
  // operands are read from one L2.
  int bid = blockIdx.x;
  int g, tile;
  if (xcd_remap) {
    const int xcd = bid & 7;
    const int u = bid >> 3;
    g = xcd + 8 * (u / tiles);
    tile = u % tiles;
  } else {
    g = bid / tiles;
    tile = bid % tiles;
  }
  if (g >= G) return;
  const int i0 = (tile / tiles1) * BMN;
  const int j0 = (tile % tiles1) * BMN;
  const size_t pe = (size_t)Np * Np;
  const TC* Pg = P + (size_t)g * pe + (size_t)i0 * Np;
  const TC* Qg = Q + (size_t)g * pe + (size_t)j0 * Np;

  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const int wr = (w >> 1) * 64;  // wave's row offset in the tile
  const int wc = (w & 1) * 64;   // wave's column offset

  // Global -> LDS staging: each k-tile is 2 x BMN rows of KT elements.
  constexpr int VEC = 16 / sizeof(TC);
  constexpr int CPR = KT / VEC;                    // chunks per row
  constexpr int LOADS = 2 * BMN * CPR / 256;       // 16-byte loads per thread per stage
  static_assert((2 * BMN * CPR) % 256 == 0, "stage must split evenly");
  u32x4 reg[LOADS];
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < LOADS; ++q) {
      const int idx = tid + q * 256;
      const int row = idx / CPR;  // 0..2*BMN
      const int chunk = idx % CPR;
      const TC* src = row < BMN ? Pg + (size_t)row * Np : Qg + (size_t)(row - BMN) * Np;
      reg[q] = *reinterpret_cast<const u32x4*>(src + k0 + chunk * VEC);
    }
  };
  auto lstore = [&](int buf) {
    TC* base = lds + buf * 2 * Cfg::TILE_ELEMS;
#pragma unroll
    for (int q = 0; q < LOADS; ++q) {
      const int idx = tid + q * 256;
      const int row = idx / CPR;
      const int chunk = idx % CPR;
      *reinterpret_cast<u32x4*>(base + row * LDK + chunk * VEC) = reg[q];
    }
  };

  f32x4 acc[4][4];
  zero_acc(acc);
  const int nk = Np / KT;
  gload(0);
  lstore(0);
  __syncthreads();
  const int r = l & 15;
  const int kq = (l >> 4) * M::KPL;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * KT);
    const TC* As = lds + buf * 2 * Cfg::TILE_ELEMS;
    const TC* Bs = As + Cfg::TILE_ELEMS;
#pragma unroll
    for (int kk = 0; kk < KT; kk += M::K16) {
      typename M::Frag af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = M::load(As + (wr + i * 16 + r) * LDK + kk + kq);
#pragma unroll
      for (int j = 0; j < 4; ++j) bfr[j] = M::load(Bs + (wc + j * 16 + r) * LDK + kk + kq);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) M::mma16(acc[i][j], af[i], bfr[j]);
    }
    if (kt + 1 < nk) lstore(buf ^ 1);
    __syncthreads();
  }

  // Stage the 128x128 output tile in LDS, then store 16-byte row chunks.
  TC* O = lds;
  constexpr int OLD = Cfg::OUT_LD;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) O[(wr + i * 16 + 4 * (l >> 4) + e) * OLD + wc + j * 16 + r] = from_f32<TC>(acc[i][j][e]);
  __syncthreads();
  constexpr int OCPR = BMN / VEC;
  TC* Xg = X + (size_t)g * pe + (size_t)i0 * Np + j0;
  for (int idx = tid; idx < BMN * OCPR; idx += 256) {
    const int row = idx / OCPR;
    const int chunk = idx % OCPR;
    *reinterpret_cast<u32x4*>(Xg + (size_t)row * Np + chunk * VEC) =
        *reinterpret_cast<const u32x4*>(O + row * OLD + chunk * VEC);
  }
}

// 16-byte chunk swizzle of the contraction's LDS k-tiles (64 bf16 per row, unpadded): the
// chunk c of row R is stored at chunk c ^ ((R >> 1) & 7). LDS serves a 128-bit read for 16
// lanes at a time over 64 four-byte banks; the 16 lanes of a fragment read 16 consecutive
// rows at the same chunk, and the swizzle gives the 8 row pairs sharing a 256-byte bank
// window the 8 different chunk slots in it. A wave's direct load writes 1 KiB
// lane-linearly (8 rows x 128 bytes), so lane l of a direct load fills row 8 blk + l / 8 at
// physical chunk l % 8.
PF_DEVICE int k2_swz(int row) { return (row >> 1) & 7; }

// Persistent bf16 contraction on 256 (i) x BJ (j) tiles, BJ = 384 when Np is a multiple
// of 768 (each operand row block is then read twice (P) or three times (Q) instead of three
// times each) and BJ = 256 for the other multiples of 256 (N = 1024: 16 tiles per plane).
// One block per CU walks tiles (at N = 768, B C 6 tiles: three per CU). Eight waves in
// 2 x 4, each owning a 128 (i) x BJ/4 (j) block as 4 x BJ/128 tiles of
// v_mfma_f32_32x32x16_bf16 (BJ/2 fp32 accumulators per lane): per k-step 4 + BJ/128
// fragment reads feed BJ/32 MFMAs. k-tiles of 64 (whole 128-byte lines per row) flow
// through two LDS stages of (256 + BJ) x 128 bytes, filled by global_load_lds_dwordx4 one
// tile ahead, one barrier per tile, with the same 16-byte chunk swizzle as the 256 x 256
// kernel. The last k-step of a tile issues the next tile's first k-tile into stage 0, so
// its latency hides behind the last MFMAs and the output pass; the output tile leaves
// through stage 1 in four passes of 64 rows i (the k-tile count is even: stage 1 holds the
// last k-tile, whose readers the first pass's barrier waits for).
template <int BJ_>
struct ContractP {
  static constexpr int BI = 256;
  static constexpr int BJ = BJ_;
  static constexpr int JT = BJ / 128;                // 32-wide j tiles per wave
  static constexpr int KT = 64;
  static constexpr int NT = 512;
  static constexpr int PT = BI * KT;                 // elements of the P k-tile
  static constexpr int STAGE = (BI + BJ) * KT;       // P tile then Q tile
  static constexpr int BLKS = (BI + BJ) / 8;         // 1 KiB direct-load blocks per stage
  static constexpr int DMA = BLKS / (NT / 64);       // per wave
  static constexpr int OLD = BJ + 8;                 // output staging rows (bf16)
  static constexpr int OROWS = 64;                   // output rows per staging pass
  static constexpr int SMEM = 2 * STAGE * 2;         // bytes (BJ 384: 163840, 256: 131072)
  static_assert(OROWS * OLD <= STAGE, "output pass fits stage 1");
};
using Contract768 = ContractP<384>;
using Contract1024 = ContractP<256>;

template <int BJ_>
__global__ __launch_bounds__(512) void trimul_contract_persistent_kernel(const bf16* __restrict__ P,
                                                                         const bf16* __restrict__ Q,
                                                                         bf16* __restrict__ X, int G, int Np,
                                                                         int xcd_remap) {
  using Cfg = ContractP<BJ_>;
  constexpr int BI = Cfg::BI, BJ = Cfg::BJ, KT = Cfg::KT, DMA = Cfg::DMA, JT = Cfg::JT;
  static_assert(DMA * (Cfg::NT / 64) == Cfg::BLKS, "a stage splits evenly over the waves");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* lds = reinterpret_cast<bf16*>(smem);

  const int ti = Np / BI, tj = Np / BJ;
  const int tiles = ti * tj;
  const int total = G * tiles;
  const size_t pe = (size_t)Np * Np;
  // Virtual tile vt -> plane g and tile origin. With the XCD remap, XCD x (vt & 7: the grid
  // is a multiple of 8 and vt steps by it) walks planes x, x + 8, ...: a plane's operands
  // stay in one L2.
  auto coords = [&](int vt, int& g, int& i0, int& j0) {
    int tile;
    if (xcd_remap) {
      const int u = vt >> 3;
      g = (vt & 7) + 8 * (u / tiles);
      tile = u % tiles;
    } else {
      g = vt / tiles;
      tile = vt % tiles;
    }
    i0 = (tile / tj) * BI;
    j0 = (tile % tj) * BJ;
  };

  const int w = wave_id();
  const int l = lane_id();
  const int wi = (w >> 2) * 128;      // wave's rows i in the tile
  const int wj = (w & 3) * (BJ / 4);  // wave's columns j

  // Direct loads: a stage is BLKS blocks of 8 rows (P blocks 0..31, then the Q blocks); wave
  // w loads blocks DMA w .. DMA w + DMA - 1. Lane l writes row 8 blk + l / 8 at physical
  // chunk l % 8, i.e. logical chunk (l % 8) ^ swz(row). 32-bit per-lane offsets from a scalar
  // base per operand (raw buffer loads).
  // The per-lane offsets are recomputed at each issue (a few VALU operations): the
  // accumulators leave no registers to keep them in.
  auto issue = [&](__amdgpu_buffer_rsrc_t rsP, __amdgpu_buffer_rsrc_t rsQ, int kt, int stage) {
    bf16* st = lds + stage * Cfg::STAGE;
#pragma unroll
    for (int q = 0; q < DMA; ++q) {
      const int blk = DMA * w + q;  // compile-time split per wave is not possible: w is uniform
      const int row = (blk < BI / 8 ? blk : blk - BI / 8) * 8 + (l >> 3);
      const int voff = (row * Np + 8 * ((l & 7) ^ k2_swz(row))) * 2;
      buf_load_lds16(blk < BI / 8 ? rsP : rsQ, st + blk * 8 * KT, voff, kt * KT * 2);
    }
  };
  auto rsrc_P = [&](int g, int i0) { return buf_rsrc(P + (size_t)g * pe + (size_t)i0 * Np, (unsigned)(BI * Np * 2)); };
  auto rsrc_Q = [&](int g, int j0) { return buf_rsrc(Q + (size_t)g * pe + (size_t)j0 * Np, (unsigned)(BJ * Np * 2)); };

  const int nk = Np / KT;  // even (Np is a multiple of 256)
  const int r = l & 31;
  const int hf = l >> 5;
  const int sw = k2_swz(r);  // rows wi + 32 t + r and wj + 32 t + r share the swizzle of r
  const int tid = threadIdx.x;

  int vt = blockIdx.x;
  if (vt >= total) return;  // block-uniform
  int g, i0, j0;
  coords(vt, g, i0, j0);
  auto rsP = rsrc_P(g, i0);
  auto rsQ = rsrc_Q(g, j0);
  issue(rsP, rsQ, 0, 0);
  for (;;) {
    const int nvt = vt + (int)gridDim.x;
    const bool has_next = nvt < total;  // block-uniform
    int ng = g, ni0 = i0, nj0 = j0;
    if (has_next) coords(nvt, ng, ni0, nj0);
    const auto nrsP = rsrc_P(ng, ni0);
    const auto nrsQ = rsrc_Q(ng, nj0);

    f32x16 acc[JT][4];  // [j tile][i tile]
#pragma unroll
    for (int a = 0; a < JT; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;
    for (int kt = 0; kt < nk; ++kt) {
      // s_waitcnt vmcnt(0) (other counters untouched): this wave's loads of tile kt landed.
      __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
      // All waves' loads of tile kt visible; stage (kt + 1) & 1 no longer read.
      __builtin_amdgcn_s_barrier();
      if (kt + 1 < nk)
        issue(rsP, rsQ, kt + 1, (kt + 1) & 1);
      else if (has_next)
        issue(nrsP, nrsQ, 0, 0);
      const bf16* Ps = lds + (kt & 1) * Cfg::STAGE;
      const bf16* Qs = Ps + Cfg::PT;
#pragma unroll
      for (int kk = 0; kk < KT; kk += 16) {
        const int c8 = 8 * ((kk / 8 + hf) ^ sw);
        bf16x8 af[JT], bfr[4];
#pragma unroll
        for (int t = 0; t < JT; ++t) af[t] = *reinterpret_cast<const bf16x8*>(Qs + (wj + 32 * t + r) * KT + c8);
#pragma unroll
        for (int t = 0; t < 4; ++t) bfr[t] = *reinterpret_cast<const bf16x8*>(Ps + (wi + 32 * t + r) * KT + c8);
#pragma unroll
        for (int a = 0; a < JT; ++a)
#pragma unroll
          for (int cc = 0; cc < 4; ++cc)
            acc[a][cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a], bfr[cc], acc[a][cc], 0, 0, 0);
      }
    }

    // acc[a][c] element e: j = wj + 32 a + acc32_row(e), i = wi + 32 c + (lane & 31). Four
    // passes of 64 rows i through stage 1 ([i][j], (BJ + 8) x 2-byte rows), stored as whole
    // 2 BJ-byte rows; stage 0 is receiving the next tile's first k-tile meanwhile.
    bf16* Xg = X + (size_t)g * pe + (size_t)i0 * Np + j0;
    bf16* ost = lds + Cfg::STAGE;
    // The store offsets are the same for every tile; the empty asm keeps the compiler from
    // hoisting all 24 of them out of the tile loop (they would not fit in registers).
    int t2 = tid;
    asm volatile("" : "+v"(t2));
#pragma unroll
    for (int pass = 0; pass < BI / Cfg::OROWS; ++pass) {
      // Stage 1 (the last k-tile, or the previous pass) is no longer read. A bare barrier
      // after this wave's LDS operations: __syncthreads() would also wait for the next
      // tile's buffer-to-LDS loads into stage 0, which are meant to overlap this pass.
      lds_barrier();
      if (wi == (pass >> 1) * 128) {
#pragma unroll
        for (int a = 0; a < JT; ++a)
#pragma unroll
          for (int c2 = 0; c2 < 2; ++c2) {
            const int cc = 2 * (pass & 1) + c2;
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              float v[4] = {acc[a][cc][4 * g4], acc[a][cc][4 * g4 + 1], acc[a][cc][4 * g4 + 2],
                            acc[a][cc][4 * g4 + 3]};
              store_vec<bf16, 4>(ost + (32 * c2 + r) * Cfg::OLD + wj + 32 * a + acc32_row(4 * g4), v);
            }
          }
      }
      lds_barrier();
#pragma unroll
      for (int it = 0; it < Cfg::OROWS * BJ / 8 / Cfg::NT; ++it) {
        const int idx = t2 + it * Cfg::NT;
        const int row = idx / (BJ / 8), ch = idx % (BJ / 8);
        *reinterpret_cast<u32x4*>(Xg + (pass * Cfg::OROWS + row) * Np + 8 * ch) =
            *reinterpret_cast<const u32x4*>(ost + row * Cfg::OLD + 8 * ch);
      }
    }
    if (!has_next) break;
    vt = nvt;
    g = ng;
    i0 = ni0;
    j0 = nj0;
    rsP = nrsP;
    rsQ = nrsQ;
  }
  // No buffer-to-LDS load may land after the block's LDS is handed to another block.
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
}

// Dynamic-LDS limits are set on every launch (a cheap host call): the attribute belongs to
// the current device, and the library keeps no per-process flags.
int reserve_lds(const void* fn, int bytes, const char* what) {
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  PF_REQUIRE(e == hipSuccess, PF_ERR_LAUNCH, "%s: cannot reserve %d bytes of LDS: %s", what, bytes,
             hipGetErrorString(e));
  return PF_OK;
}

template <int BJ>
int contract_persistent_launch(const void* P, const void* Q, void* X, int G, int Np, int remap, hipStream_t s) {
  using Cfg = ContractP<BJ>;
  if (int e = reserve_lds((const void*)trimul_contract_persistent_kernel<BJ>, Cfg::SMEM, "trimul_contract")) return e;
  // Persistent: at most one block per CU, a multiple of 8 for the XCD remap.
  const long total = (long)G * (Np / Cfg::BI) * (Np / Cfg::BJ);
  PF_REQUIRE(total < (1L << 31), PF_ERR_UNSUPPORTED, "trimul_contract: B C = %d planes of Np = %d", G, Np);
  long nblk = std::min<long>(total, pf::cu_count());
  if (remap) nblk = std::max<long>(8, nblk & ~7L);
  pf::KernelTimer timer("trimul_contract", s);
  trimul_contract_persistent_kernel<BJ><<<dim3((unsigned)nblk), Cfg::NT, Cfg::SMEM, s>>>(
      (const bf16*)P, (const bf16*)Q, (bf16*)X, G, Np, remap);
  timer.stop();
  return pf::check_launch("trimul_contract");
}

template <class TC>
int contract_generic_launch(const void* P, const void* Q, void* X, int G, int Np, int remap, hipStream_t s) {
  using Cfg = ContractCfg<TC>;
  if (int e = reserve_lds((const void*)trimul_contract_kernel<TC>, Cfg::SMEM, "trimul_contract")) return e;
  const int tiles = (Np / Cfg::BMN) * (Np / Cfg::BMN);
  pf::KernelTimer timer("trimul_contract", s);
  trimul_contract_kernel<TC><<<dim3((unsigned)(G * tiles)), 256, Cfg::SMEM, s>>>((const TC*)P, (const TC*)Q,
                                                                                  (TC*)X, G, Np, remap);
  timer.stop();
  return pf::check_launch("trimul_contract");
}

// ------------------------------------------------------------------ K3
template <class TZ, class TC, int C>
struct OutputCfg {
  static constexpr int BM = trimul_bm<TC>();
  static constexpr int XLD = BM + lds_pad<TC>();  // Xs [C][XLD]
  static constexpr int ALD = C + lds_pad<TC>();   // A1, A2 [BM][ALD]
  static constexpr int SLD = C + 4;               // fp32 stage [BM][SLD]
  static constexpr int XS_BYTES = C * XLD * (int)sizeof(TC);
  static constexpr int A_BYTES = BM * ALD * (int)sizeof(TC);
  static constexpr int STAGE_BYTES = BM * SLD * 4;
  static constexpr int NQ = trimul_nt<C>() / BM;  // threads per position in the LN_out pass
};

// MHR = true replaces LN_out by the multi-head routed mix `mx` (mhr.h) of at most HM heads
// (the LDS its per-head values take); ln_out_b may then be null (head_rms).
template <class TZ, class TC, int C, bool NORM = true, bool MHR = false, int HM = kMhrMaxHeads>
__global__ __launch_bounds__(trimul_nt<C>()) void trimul_output_kernel(
    const TC* __restrict__ X, const TZ* __restrict__ z, TZ* __restrict__ out, const float* __restrict__ lniw,
    const float* __restrict__ lnib, float eps_in, const float* __restrict__ lnow, const float* __restrict__ lnob,
    float eps_out, const TC* __restrict__ Wo, const TC* __restrict__ Wog, int B, int N, int Np, int accumulate,
    MixSpec mx) {
  using Cfg = OutputCfg<TZ, TC, C>;
  constexpr int BM = Cfg::BM, XLD = Cfg::XLD, ALD = Cfg::ALD, SLD = Cfg::SLD, NQ = Cfg::NQ;
  constexpr int NT = trimul_nt<C>();
  constexpr int RB = BM / 16;
  constexpr int CBW = C / 16 / (NT / 64);
  constexpr int SMEM1 = Cfg::XS_BYTES + 2 * Cfg::A_BYTES;
  constexpr int SMEM = SMEM1 > Cfg::STAGE_BYTES ? SMEM1 : Cfg::STAGE_BYTES;
  constexpr int MXN = MHR ? BM * HM : 1;
  __shared__ __attribute__((aligned(16))) char smem[SMEM];
  __shared__ float red[NQ][BM];
  __shared__ float stat_mean[BM];
  __shared__ float mx_gate[MXN], mx_sa[MXN], mx_sb[MXN], mx_part[MXN];
  __shared__ float mx_w[MHR ? C : 1], mx_b[MHR ? C : 1];  // norm_center's affine, staged once
  TC* Xs = reinterpret_cast<TC*>(smem);
  TC* A1 = reinterpret_cast<TC*>(smem + Cfg::XS_BYTES);
  TC* A2 = reinterpret_cast<TC*>(smem + Cfg::XS_BYTES + Cfg::A_BYTES);
  float* stage = reinterpret_cast<float*>(smem);

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

  // 1) raw X tile, channel-major: Xs[c][p] = X[b*C + c][i][j0 + p]
  {
    constexpr int VEC = 16 / sizeof(TC);
    constexpr int CPR = BM / VEC;
    const TC* Xb = X + (size_t)b * C * pe + (size_t)i * Np + j0;
    for (int idx = tid; idx < C * CPR; idx += NT) {
      const int c = idx / CPR;
      const int chunk = idx % CPR;
      *reinterpret_cast<u32x4*>(Xs + c * XLD + chunk * VEC) =
          *reinterpret_cast<const u32x4*>(Xb + (size_t)c * pe + chunk * VEC);
    }
  }
  // 3) LN_in(z) tile (independent of Xs)
  const TZ* zb = z + (size_t)b * N * N * C;
  auto zrow = [&](int p) -> const TZ* {
    const int j = j0 + p;
    return j < N ? zb + ((size_t)i * N + j) * C : nullptr;
  };
  if constexpr (NORM)
    ln_tile_to_lds<TZ, TC, C, BM, NT>(zrow, lniw, lnib, eps_in, A2, ALD);
  else
    copy_tile_to_lds<TZ, TC, C, BM, NT>(zrow, A2, ALD);
  __syncthreads();

  // 2) LN_out (or the MHR mix) over channels of X, transposing into A1[p][c]
  if constexpr (MHR) {
    mhr_gates<TC, C, BM, NT>(A2, ALD, mx, mx_gate, rf);
    mhr_stats<TC, C, BM, NT>(Xs, XLD, mx_gate, mx, eps_out, mx_sa, mx_sb, mx_part);
    mhr_mix_write<TC, C, BM, NT>(Xs, XLD, mx_gate, mx_sa, mx_sb, mx, mx_w, mx_b, A1, ALD);
  } else {
    constexpr int CPQ = C / NQ;
    const int p = tid % BM;
    const int q = tid / BM;
    float xv[CPQ];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < CPQ; ++e) {
      xv[e] = to_f32(Xs[(q * CPQ + e) * XLD + p]);
      s += xv[e];
    }
    red[q][p] = s;
    __syncthreads();
    if (q == 0) {
      float t = 0.f;
#pragma unroll
      for (int k = 0; k < NQ; ++k) t += red[k][p];
      stat_mean[p] = t * (1.0f / C);
    }
    __syncthreads();
    const float mean = stat_mean[p];
    float v = 0.f;
#pragma unroll
    for (int e = 0; e < CPQ; ++e) {
      const float d = xv[e] - mean;
      v += d * d;
    }
    __syncthreads();  // everyone has read stat_mean and red
    red[q][p] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < NQ; ++k) t += red[k][p];
    const float rstd = rsqrtf(t * (1.0f / C) + eps_out);
    float y[CPQ];
#pragma unroll
    for (int e = 0; e < CPQ; ++e) {
      const int c = q * CPQ + e;
      y[e] = (xv[e] - mean) * rstd * lnow[c] + lnob[c];
    }
    constexpr int VEC = 16 / sizeof(TC);
#pragma unroll
    for (int e = 0; e < CPQ; e += VEC) store_vec<TC, VEC>(A1 + p * ALD + q * CPQ + e, y + e);
  }
  __syncthreads();

  // 4) p = A1 Wo^T, g = A2 Wog^T
  const int w = wave_id();
  const int l = lane_id();
  f32x4 accp[RB][CBW], accg[RB][CBW];
  zero_acc(accp);
  zero_acc(accg);
  int wrow0[CBW];
#pragma unroll
  for (int j = 0; j < CBW; ++j) wrow0[j] = (w * CBW + j) * 16;
  gemm16_lds_x_w<TC, C, RB, CBW>(accp, A1, ALD, 0, Wo, C, wrow0);
  gemm16_lds_x_w<TC, C, RB, CBW>(accg, A2, ALD, 0, Wog, C, wrow0);
  __syncthreads();  // A1/A2/Xs dead: reuse as the fp32 stage

  // 5) update = sigmoid(g) * p, staged [p][c] in fp32, then stored / accumulated
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < CBW; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int p = rb * 16 + 4 * (l >> 4) + e;
        const int c = (w * CBW + j) * 16 + (l & 15);
        stage[p * SLD + c] = sigmoidf_(accg[rb][j][e]) * accp[rb][j][e];
      }
  __syncthreads();
  TZ* ob = out + (size_t)b * N * N * C;
  auto orow = [&](int p) -> TZ* {
    const int j = j0 + p;
    return j < N ? ob + ((size_t)i * N + j) * C : nullptr;
  };
  store_tile_from_lds<TZ, C, BM, NT>(orow, stage, SLD, accumulate != 0);
}

// ------------------------------------------------------------------ bf16 K1 / K3 (32x32 tiles)
// The bf16 path runs K1 and K3 as 128- and 64-position block tiles on 32x32x16 MFMAs with
// the weights staged through LDS; the fp32 parity path keeps the 16x16 kernels above.
//
// K1: packed weights in 32-channel chunks, row 128 j + 32 kind + r (kind 0 a proj, 1 a gate,
// 2 b proj, 3 b gate; channel 32 j + r). Waves 2 x 2: positions x (a | b). Each wave's
// accumulator pair (proj, gate) holds the same (position, channel) elements, so the gate is
// applied in registers; the gated chunk is staged channel-major and written as 256-byte
// plane rows.
template <class TZ>
__global__ __launch_bounds__(256) void trimul_project32_kernel(const TZ* __restrict__ z, const float* __restrict__ mask,
                                                               const float* __restrict__ lnw,
                                                               const float* __restrict__ lnb, float eps,
                                                               const bf16* __restrict__ w4, bf16* __restrict__ planes,
                                                               int B, int N, int Np, int outgoing) {
  constexpr int C = 128;
  constexpr int BM = 128;
  constexpr int LD = ld128<bf16>();
  constexpr int NT = 256;
  constexpr int WM = 64;
  constexpr int PT = 2;
  constexpr int SLD = BM + 8;
  __shared__ __attribute__((aligned(16))) bf16 X[BM * LD];
  __shared__ __attribute__((aligned(16))) bf16 WS[128 * LD];
  __shared__ float mk[BM];

  const int t0 = blockIdx.x * BM;
  const int line = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const int wr = w >> 1, wc = w & 1;
  const TZ* zb = z + (size_t)b * N * N * C;
  auto pos_of = [&](int p) -> long {
    const int t = t0 + p;
    if (line >= N || t >= N) return -1;
    return outgoing ? (long)line * N + t : (long)t * N + line;
  };
  Rows128<bf16, 128, NT> wpf;
  wpf.load(w4, C);
  ln_tile_to_lds<TZ, bf16, C, BM, NT>([&](int p) -> const TZ* {
    const long pos = pos_of(p);
    return pos < 0 ? nullptr : zb + pos * C;
  }, lnw, lnb, eps, X, LD);
  if (tid < BM) {
    const long pos = pos_of(tid);
    mk[tid] = pos < 0 ? 0.f : mask[(size_t)b * N * N + pos];
  }
  const size_t pe = (size_t)Np * Np;
#pragma unroll 1
  for (int j = 0; j < C / 32; ++j) {
    __syncthreads();
    wpf.store(WS, LD);
    __syncthreads();
    if (j + 1 < C / 32) wpf.load(w4 + (size_t)(j + 1) * 128 * C, C);
    f32x16 acc[PT][2];
    zero_acc32(acc);
    wave_mma32<bf16, PT, 2, C>(acc, X, LD, wr * WM, WS, LD, wc * 64);
    __syncthreads();  // WS becomes the stage [plane * 32 + channel][position]
#pragma unroll
    for (int pi = 0; pi < PT; ++pi)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int p0 = wr * WM + 32 * pi + acc32_row(4 * g4);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = sigmoidf_(acc[pi][1][4 * g4 + e]) * acc[pi][0][4 * g4 + e] * mk[p0 + e];
        store_vec<bf16, 4>(WS + (wc * 32 + (l & 31)) * SLD + p0, v);
      }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 64 * BM / 8 / NT; ++it) {
      const int idx = tid + it * NT;
      const int row = idx / (BM / 8);
      const int chunk = idx % (BM / 8);
      const int plane = row / 32;
      const int ch = 32 * j + (row % 32);
      bf16* dst = planes + ((size_t)plane * B * C + (size_t)b * C + ch) * pe + (size_t)line * Np + t0 + chunk * 8;
      *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(WS + row * SLD + chunk * 8);
    }
  }
}

// K1, persistent and weight-stationary (bf16 GEMMs). One 512-thread block per CU walks
// tiles of 64 positions along a line. Wave w owns plane w >> 2 (a | b) and channels
// 32 (w & 3) .. +32: its proj and gate weight rows (2 x 32 rows x 128 k, packed as above)
// stay in MFMA operand registers for the whole kernel, so weights are read once per CU
// instead of once per tile. Every wave computes acc[position][channel] for proj and gate of
// the current tile (the same elements), gates and masks in registers -- a lane holds four
// consecutive positions of one channel -- stages its 32 x 64 result channel-major in a
// private LDS region with 8-byte stores and writes 128-byte plane rows.
// Every wave LayerNorms 8 rows of the NEXT tile (from z rows it loaded two tiles ahead) into
// the other half of a double-buffered LDS tile. The two waves that share a SIMD (w, w + 4)
// work out of phase: waves 4-7 LayerNorm first and then run their GEMMs, waves 0-3 run their
// GEMMs first and LayerNorm after, so each wave's MFMAs overlap the other's LayerNorm and
// gating VALU work. One barrier per tile publishes the next tile's LayerNorm. NORM = false
// (the training forward, whose input is already LayerNormed in autograd) only rounds the rows
// to bf16 in that step.
// K1 at 256 channels (bf16 GEMMs), persistent and weight-streaming: one 8-wave block per CU
// walks tiles of 128 plane positions (one line, 128 consecutive t). The packed weights
// (1024 rows x 256 k, 512 KB: too large to stay in registers as at 128 channels) stream
// through a double-buffered LDS ring in 64-row chunks (16 channels: a proj, a gate, b proj,
// b gate; 32 KB) by direct buffer->LDS loads one chunk ahead, 16-byte pieces XOR-swizzled by
// row so fragment reads are conflict-free. Wave w owns rows 32 (w & 1) .. of every chunk
// (the a or b pair of projection and gate) and positions 32 (w >> 1) ..: its 32 positions
// are LayerNormed straight into registers as the B operands for the whole tile (a
// position's 256 channels live in lanes l and l ^ 32), and the next tile's rows are loaded
// while this tile's chunks run. Per chunk a wave issues 16 32x32x16 MFMAs; the projection
// and gate rows of one channel land in one lane (accumulator rows r and r + 16), so the
// gating is in registers; the gated values go through a double-buffered LDS stage
// [a | b][16 channels][128 positions] and leave as 256-byte plane-row pieces one chunk later.
// One barrier per chunk. (Three stages, weights two chunks ahead with each wait counting the
// vector-memory operations issued after them, measured slower: 533 -> 600-609 us at N=768;
// so did 64 positions per wave, whose operands spill.)
struct Project256 {
  static constexpr int C = 256;
  static constexpr int BP = 128;                  // positions per tile
  static constexpr int NW = 8;
  static constexpr int NT = 64 * NW;
  static constexpr int CR = 64;                   // weight rows per chunk
  static constexpr int NCH = 4 * C / CR;          // 16 chunks per tile
  static constexpr int ROWB = C * 2;              // 512-byte weight rows
  static constexpr int CHUNK = CR * ROWB;         // 32 KB
  static constexpr int NSTAGE = 2;                // weight chunks issued one ahead
  static constexpr int DMA = CHUNK / 1024 / NW;   // direct loads per wave per chunk
  static constexpr int SLD = BP + 8;              // stage rows (bf16)
};

// Byte offset of logical 16-byte piece c (0..31) of 512-byte weight row r: the piece index's
// low four bits XOR the row's, so 16 consecutive rows at one logical piece spread over the
// 16 bank groups.
PF_DEVICE int p256_off(int r, int c) { return r * Project256::ROWB + 16 * (c ^ (r & 15)); }

template <class TZ, bool NORM = true>
__global__ __launch_bounds__(Project256::NT, 1) void trimul_project256_kernel(
    const TZ* __restrict__ z, const float* __restrict__ mask, const float* __restrict__ lnw,
    const float* __restrict__ lnb, float eps, const bf16* __restrict__ w4, bf16* __restrict__ planes, int B, int N,
    int Np, int outgoing) {
  using Cfg = Project256;
  constexpr int C = Cfg::C, BP = Cfg::BP, NCH = Cfg::NCH, SLD = Cfg::SLD, NS = Cfg::NSTAGE;
  // bf16 rows: the next tile's rows load during this tile's chunks (a second register set
  // would not fit fp32 rows)
  constexpr bool PREFETCH = sizeof(TZ) == 2;
  constexpr int NPIECE = C / 16 * (int)sizeof(TZ) / 2;  // 16-byte loads of a lane's half row
  __shared__ __attribute__((aligned(16))) char ring[NS * Cfg::CHUNK];
  __shared__ __attribute__((aligned(16))) bf16 stage[2][2][16][SLD];
  __shared__ float lnp[2 * C];

  const int w = wave_id();
  const int l = lane_id();
  const int lq = l & 31, hf = l >> 5;
  const int rb = w & 1;   // a (0) or b (1) rows of each chunk
  const int pb = w >> 1;  // positions 32 pb ..
  const int NT1 = Np / BP;
  const long ntiles = (long)B * Np * NT1;
  const size_t pe = (size_t)Np * Np;
  // chunks this block consumes: its tiles x NCH
  const long total = blockIdx.x < ntiles ? ((ntiles - 1 - blockIdx.x) / gridDim.x + 1) * NCH : 0;

  if (NORM)
    for (int i = threadIdx.x; i < C; i += Cfg::NT) {
      lnp[i] = lnw[i];
      lnp[C + i] = lnb[i];
    }

  const auto rw = buf_rsrc(w4, 4 * C * C * 2);
  auto issue_chunk = [&](long gg) {
    const int c = (int)(gg % NCH);
    char* st = ring + (gg % NS) * Cfg::CHUNK;
#pragma unroll
    for (int t = 0; t < Cfg::DMA; ++t) {
      const int ins = w * Cfg::DMA + t;  // two 512-byte rows per instruction
      const int row = 2 * ins + (l >> 5);
      const int lc = (l & 31) ^ (row & 15);
      buf_load_lds16(rw, st + ins * 1024, ((c * Cfg::CR + row) * C + 8 * lc) * 2, 0);
    }
  };
  auto tile_pos = [&](long tl, int& b, int& line, int& t0) {
    b = (int)(tl / ((long)Np * NT1));
    const long r = tl - (long)b * Np * NT1;
    line = (int)(r / NT1);
    t0 = (int)(r - (long)line * NT1) * BP;
  };
  // this lane's half row of tile tl: channels 16 ks + 8 hf .. +7, ks = 0..15 (zeros past N)
  u32x4 zr[NPIECE];
  auto load_half = [&](long tl) {
    int b, line, t0;
    tile_pos(tl, b, line, t0);
    const int t = t0 + 32 * pb + lq;
    const TZ* src = nullptr;
    if (line < N && t < N)
      src = z + ((size_t)b * N * N + (outgoing ? (long)line * N + t : (long)t * N + line)) * C + 8 * hf;
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
  // chunk gg's gated values (stage gg & 1, plane-row pieces) -> planes of tile (b, line, t0)
  auto store_chunk = [&](long gg, int b, int line, int t0) {
    const int idx = threadIdx.x;  // 2 planes x 16 channels x 16 pieces = 512 threads
    const int p2 = idx >> 8, ch = (idx >> 4) & 15, pc = idx & 15;
    const int c = (int)(gg % NCH);
    bf16* dst = planes + ((size_t)p2 * B * C + (size_t)b * C + 16 * c + ch) * pe + (size_t)line * Np + t0 + 8 * pc;
    *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(&stage[gg & 1][p2][ch][8 * pc]);
  };

  long g = 0;
  long tile = blockIdx.x;
  int sb = 0, sline = 0, st0 = 0;  // tile of the chunk waiting in the stage
  if (total > 0) {
    load_half(tile);
    for (int i = 0; i < NS - 1 && i < total; ++i) issue_chunk(i);
  }
  __syncthreads();  // LN parameters

  for (; tile < ntiles; tile += gridDim.x) {
    int b, line, t0;
    tile_pos(tile, b, line, t0);
    const int tpos = t0 + 32 * pb + lq;
    const bool live = line < N && tpos < N;
    const float mk =
        live ? mask[(size_t)b * N * N + (outgoing ? (long)line * N + tpos : (long)tpos * N + line)] : 0.f;
    if (!PREFETCH && tile != (long)blockIdx.x) load_half(tile);

    // ---- LN (or the given x) -> B operands xf[ks]: channels 16 ks + 8 hf .. +7
    bf16x8 xf[C / 16];
    if constexpr (NORM) {
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
    } else {
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        float v[8];
        get(ks, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[ks][e] = (bf16)v[e];
      }
    }
    const bool more = tile + gridDim.x < ntiles;

#pragma unroll 1
    for (int c = 0; c < NCH; ++c, ++g) {
      // Chunk g's weights landed in every wave. Past the barrier, ring slot (g + 1) % NS (read
      // by chunk g - 1's MFMAs) takes chunk g + 1, and stage (g - 1) & 1 leaves for the
      // planes before chunk g + 1's barrier lets it be rewritten.
      __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
      lds_barrier();
      if (g > 0) store_chunk(g - 1, sb, sline, st0);
      if (PREFETCH && c == 1 && more) load_half(tile + gridDim.x);  // zr is free after LN
      if (g + NS - 1 < total) issue_chunk(g + NS - 1);
      const char* st = ring + (g % NS) * Cfg::CHUNK;
      f32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        const bf16x8 wf = *reinterpret_cast<const bf16x8*>(st + p256_off(32 * rb + lq, 2 * ks + hf));
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, xf[ks], acc, 0, 0, 0);
      }
      // acc[e]: chunk row 32 rb + 8 (e >> 2) + 4 hf + (e & 3), position 32 pb + lq; rows
      // 0..15 of the pair are the projection of channel 16 c + row, rows 16..31 its gate
      bf16(*sg)[SLD] = stage[g & 1][rb];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int ch = 8 * (e >> 2) + 4 * hf + (e & 3);
        sg[ch][32 * pb + lq] = (bf16)(sigmoidf_(acc[e + 8]) * acc[e] * mk);
      }
      sb = b;
      sline = line;
      st0 = t0;
    }
  }
  if (total > 0) {
    lds_barrier();
    store_chunk(g - 1, sb, sline, st0);
  }
  __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // no direct load outlives the block
}

struct ProjectWs {
  static constexpr int C = 128;
  static constexpr int BP = 64;   // positions per tile
  static constexpr int NW = 8;    // waves per block
  static constexpr int NT = 64 * NW;
  static constexpr int XLD = C + 8;   // 272-byte rows: conflict-free 16-byte operand reads
  static constexpr int SLD = BP + 8;  // stage rows (bf16)
};

template <class TZ, bool NORM = true>
__global__ __launch_bounds__(ProjectWs::NT) void trimul_project_ws_kernel(
    const TZ* __restrict__ z, const float* __restrict__ mask, const float* __restrict__ lnw,
    const float* __restrict__ lnb, float eps, const bf16* __restrict__ w4, bf16* __restrict__ planes, int B, int N,
    int Np, int outgoing) {
  using Cfg = ProjectWs;
  constexpr int C = Cfg::C, BP = Cfg::BP, XLD = Cfg::XLD, SLD = Cfg::SLD;
  constexpr int VEC = 16 / sizeof(TZ);  // z elements per 16-byte load
  constexpr int LPR = C / VEC;          // lanes per z row
  constexpr int RPI = 64 / LPR;         // rows per wave-wide load
  constexpr int RPW = BP / Cfg::NW;     // z rows each wave normalises per tile
  constexpr int NLD = RPW / RPI;        // 16-byte loads per lane per tile
  __shared__ __attribute__((aligned(16))) bf16 xs[2][BP * XLD];
  __shared__ __attribute__((aligned(16))) float mks[2][BP];
  __shared__ __attribute__((aligned(16))) bf16 stage_all[Cfg::NW][32 * SLD];

  const int w = wave_id();
  const int l = lane_id();
  const int pl = w >> 2;  // 0: a (P), 1: b (Q); also 1 = LayerNorm before the GEMMs
  const int cj = w & 3;   // 32-channel chunk
  bf16* stg = stage_all[w];
  const int tpl = Np / BP;
  const int ntiles = B * Np * tpl;  // < 2^31 (checked at launch)
  const int G = gridDim.x;
  const size_t pe = (size_t)Np * Np;

  // Weights -> B operands: lane l holds column (channel) l & 31, k = 16 ks + 8 (l >> 5) + e.
  bf16x8 wp[C / 16], wg[C / 16];
  {
    const bf16* rp = w4 + (size_t)(128 * cj + 32 * (2 * pl) + (l & 31)) * C + 8 * (l >> 5);
    const bf16* rg = rp + (size_t)32 * C;
#pragma unroll
    for (int ks = 0; ks < C / 16; ++ks) {
      wp[ks] = *reinterpret_cast<const bf16x8*>(rp + 16 * ks);
      wg[ks] = *reinterpret_cast<const bf16x8*>(rg + 16 * ks);
    }
  }
  const int chunk = l % LPR;
  // LayerNorm parameters of this lane's channels, read once.
  float lw[VEC], lb[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    lw[e] = NORM ? lnw[chunk * VEC + e] : 1.f;
    lb[e] = NORM ? lnb[chunk * VEC + e] : 0.f;
  }

  auto tile_coords = [&](int tile, int& b, int& line, int& t0) {
    b = tile / (Np * tpl);
    const int rem = tile - b * (Np * tpl);
    line = rem / tpl;
    t0 = (rem - line * tpl) * BP;
  };
  // z rows and mask values of two tiles ahead, in two register sets. The
  // loads are unconditional (a padding row reads a clamped real row; its mask becomes 0 when
  // it is used), so the compiler's wait counts stay exact and the second set stays in flight.
  u32x4 zr[2][NLD];
  float mkn[2][NLD];
  unsigned okb[2];
  auto issue = [&](int tile, int set) __attribute__((always_inline)) {
    int b, line, t0;
    tile_coords(tile, b, line, t0);
    const TZ* zb = z + (size_t)b * N * N * C;
    const float* mb = mask + (size_t)b * N * N;
    const int lc = min(line, N - 1);
    unsigned ok = 0;
#pragma unroll
    for (int q = 0; q < NLD; ++q) {
      const int t = t0 + w * RPW + q * RPI + l / LPR;
      ok |= (line < N && t < N) ? 1u << q : 0u;
      const int tc = min(t, N - 1);
      const size_t pos = outgoing ? (size_t)lc * N + tc : (size_t)tc * N + lc;
      zr[set][q] = *reinterpret_cast<const u32x4*>(zb + pos * C + chunk * VEC);
      mkn[set][q] = mb[pos];
    }
    okb[set] = ok;
  };
  // LayerNorm (fp32 two-pass statistics) of this wave's rows of a tile -> xs[buf] in bf16.
  auto layer_norm = [&](int set, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < NLD; ++q) {
      float v[VEC];
      unpack16<TZ>(zr[set][q], v);
      if constexpr (NORM) {
        float sum = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) sum += v[e];
        const float mean = row_group_sum<LPR>(sum) * (1.0f / C);
        float sq = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float d = v[e] - mean;
          sq += d * d;
        }
        const float rstd = rsqrtf(row_group_sum<LPR>(sq) * (1.0f / C) + eps);
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = (v[e] - mean) * rstd * lw[e] + lb[e];
      }
      const int row = w * RPW + q * RPI + l / LPR;
      store_vec<bf16, VEC>(xs[buf] + row * XLD + chunk * VEC, v);
      if (chunk == 0) mks[buf][row] = (okb[set] >> q) & 1u ? mkn[set][q] : 0.f;
    }
  };
  // Step for tile `tile`: normalise the next tile (register set `set`) into
  // xs[buf] and refill the set with the tile after the one already in flight.
  // Every issue is unconditional (a tile past the end reloads the last tile, unused), so all
  // paths through the loop carry the same load counts.
  auto prepare_next = [&](int tile, int set, int buf) __attribute__((always_inline)) {
    if (tile + G < ntiles) layer_norm(set, buf);
    issue(min(tile + 3 * G, ntiles - 1), set);
  };
  auto compute = [&](int tile, int buf) __attribute__((always_inline)) {
    int b, line, t0;
    tile_coords(tile, b, line, t0);
    const bf16* xb = xs[buf];
    f32x16 acc[2][2];  // [proj | gate][position tile]
    zero_acc32(acc);
#pragma unroll
    for (int ks = 0; ks < C / 16; ++ks) {
      bf16x8 xf[2];
#pragma unroll
      for (int pt = 0; pt < 2; ++pt)
        xf[pt] = *reinterpret_cast<const bf16x8*>(xb + (32 * pt + (l & 31)) * XLD + 16 * ks + 8 * (l >> 5));
#pragma unroll
      for (int pt = 0; pt < 2; ++pt) {
        acc[0][pt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xf[pt], wp[ks], acc[0][pt], 0, 0, 0);
        acc[1][pt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xf[pt], wg[ks], acc[1][pt], 0, 0, 0);
      }
    }
    // Gate, mask, stage channel-major: lane (channel l & 31) holds positions
    // 32 pt + acc32_row(4 g + e), four consecutive per g.
#pragma unroll
    for (int pt = 0; pt < 2; ++pt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int p0 = 32 * pt + acc32_row(4 * g);
        const f32x4 m4 = *reinterpret_cast<const f32x4*>(&mks[buf][p0]);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = sigmoidf_(acc[1][pt][4 * g + e]) * acc[0][pt][4 * g + e] * m4[e];
        store_vec<bf16, 4>(stg + (l & 31) * SLD + p0, v);
      }
    // The stage is private to this wave: LDS operations of one wave complete in order.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    bf16* pb = planes + ((size_t)pl * B * C + (size_t)b * C + 32 * cj) * pe + (size_t)line * Np + t0;
#pragma unroll
    for (int it = 0; it < 32 * BP / 8 / 64; ++it) {
      const int row = it * 8 + (l >> 3);
      const int c8 = l & 7;
      *reinterpret_cast<u32x4*>(pb + (size_t)row * pe + 8 * c8) =
          *reinterpret_cast<const u32x4*>(stg + row * SLD + 8 * c8);
    }
    __builtin_amdgcn_wave_barrier();
  };

  // Prologue: every wave loads its rows of two tiles and normalises the first. The loop
  // runs two tiles per trip so the register sets and LDS halves are compile-time indices;
  // all barrier conditions are block-uniform. The weights and LayerNorm parameters are
  // waited for here, once: the two wave groups take different load paths into the loop, and
  // without this the compiler waits on every load in flight wherever it first reads them.
  __builtin_amdgcn_s_waitcnt(0);
  int tile = blockIdx.x;
  issue(min(tile, ntiles - 1), 0);
  issue(min(tile + G, ntiles - 1), 1);
  if (tile < ntiles) layer_norm(0, 0);
  issue(min(tile + 2 * G, ntiles - 1), 0);
  __syncthreads();
  for (; tile < ntiles; tile += 2 * G) {
    if (pl == 1) prepare_next(tile, 1, 1);
    compute(tile, 0);
    if (pl == 0) prepare_next(tile, 1, 1);
    __syncthreads();  // xs[1] holds tile + G; every wave is done with xs[0]
    if (tile + G >= ntiles) break;
    if (pl == 1) prepare_next(tile + G, 0, 0);
    compute(tile + G, 1);
    if (pl == 0) prepare_next(tile + G, 0, 0);
    __syncthreads();  // xs[0] holds tile + 2 G; every wave is done with xs[1]
  }
}

// K3, persistent and weight-stationary (bf16 GEMMs). One 512-thread block per CU walks
// tiles of 64 positions (i, j0 .. j0+63) of one row. Wave w owns output channels
// 32 (w & 3) .. +32 of positions 32 (w >> 2) .. +32: rows of out_proj and out_gate as
// 32x32x16 MFMA A operands, resident in registers; the two accumulators share a layout, so
// the gate applies in registers. Per tile: the X tile (channel-major, 128 x 64) goes to
// LDS and is normalised (LN_out) by a pass whose reads run along positions (no bank
// conflicts); the z tile is normalised (LN_in) from registers that also keep it for the
// residual; after the MFMAs each wave stages its fp32 update block-wide, and each wave then
// adds the update to the 8 z rows it loaded and writes them. The next tile's X and z are
// loaded during this tile's MFMAs.
struct OutputWs {
  static constexpr int C = 128;
  static constexpr int BP = 64;
  static constexpr int NW = 8;
  static constexpr int NT = 64 * NW;
  static constexpr int XLD = C + 8;   // bf16 operand rows [pos][ch]
  static constexpr int TLD = BP + 8;  // bf16 X tile rows [ch][pos]
  static constexpr int SLD = C + 4;   // fp32 update stage rows [pos][ch]
};

template <class TZ>
__global__ __launch_bounds__(OutputWs::NT) void trimul_output_ws_kernel(
    const bf16* __restrict__ X, const TZ* __restrict__ z, TZ* __restrict__ out, const float* __restrict__ lniw,
    const float* __restrict__ lnib, float eps_in, const float* __restrict__ lnow, const float* __restrict__ lnob,
    float eps_out, const bf16* __restrict__ Wo, const bf16* __restrict__ Wog, int B, int N, int Np, int accumulate) {
  using Cfg = OutputWs;
  constexpr int C = Cfg::C, BP = Cfg::BP, NW = Cfg::NW, NT = Cfg::NT, XLD = Cfg::XLD, TLD = Cfg::TLD,
                SLD = Cfg::SLD;
  constexpr int VEC = 16 / sizeof(TZ);  // z elements per 16-byte load
  constexpr int LPR = C / VEC;          // lanes per z row
  constexpr int RPI = 64 / LPR;         // z rows per wave-wide load
  constexpr int RPW = BP / NW;          // z rows per wave per tile
  constexpr int NLD = RPW / RPI;        // z loads per lane per tile
  constexpr int XLDS = C * BP / 8 / NT; // 16-byte X loads per lane per tile
  __shared__ __attribute__((aligned(16))) bf16 xt[C * TLD];   // X tile [ch][pos]
  __shared__ __attribute__((aligned(16))) bf16 xa[BP * XLD];  // LN_out(X) [pos][ch]
  __shared__ __attribute__((aligned(16))) bf16 xb[BP * XLD];  // LN_in(z) [pos][ch]
  __shared__ __attribute__((aligned(16))) float upd[BP * SLD];

  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const int pe = Np * Np;  // plane size (elements); Np <= 4096 keeps every offset below 2^31
  const int tpr = (N + BP - 1) / BP;
  const int ntiles = B * N * tpr;
  const int cw = w & 3, pw = w >> 2;

  // Weights: lane holds row 32 cw + (l & 31), k = 16 ks + 8 (l >> 5) + e.
  bf16x8 wo[C / 16], wg[C / 16];
#pragma unroll
  for (int ks = 0; ks < C / 16; ++ks) {
    const size_t r = (size_t)(32 * cw + (l & 31)) * C + 16 * ks + 8 * (l >> 5);
    wo[ks] = *reinterpret_cast<const bf16x8*>(Wo + r);
    wg[ks] = *reinterpret_cast<const bf16x8*>(Wog + r);
  }
  const int chunk = l % LPR;
  float liw[VEC], lib[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    liw[e] = lniw[chunk * VEC + e];
    lib[e] = lnib[chunk * VEC + e];
  }
  // LN_out: thread (position op = tid / 8, part os = tid % 8) normalises the channel pairs
  // 16 k + 2 os + {0, 1}, k = 0..7: the 64 lanes of one read instruction touch 32 distinct
  // dwords in 32 distinct banks (rows 2 os + 16 k, positions op).
  const int op = tid >> 3, os = tid & 7;
  auto och = [&](int c) { return 16 * (c >> 1) + 2 * os + (c & 1); };
  float low[16], lob[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    low[c] = lnow[och(c)];
    lob[c] = lnob[och(c)];
  }
  // Per-lane load offsets (elements): z rows of this lane, X rows (tid >> 3) + 64 q.
  int zoff[NLD];
#pragma unroll
  for (int q = 0; q < NLD; ++q) zoff[q] = (w * RPW + q * RPI + l / LPR) * C + chunk * VEC;
  const int xoff = (tid >> 3) * pe + 8 * (tid & 7);

  auto tile_coords = [&](int tile, int& b, int& i, int& j0) {
    b = tile / (N * tpr);
    const int rem = tile - b * (N * tpr);
    i = rem / tpr;
    j0 = (rem - i * tpr) * BP;
  };
  u32x4 zr[NLD], xr[XLDS];
  auto issue = [&](int tile) {
    int b, i, j0;
    tile_coords(tile, b, i, j0);
    const TZ* zb = z + (((size_t)b * N + i) * N + j0) * C;
#pragma unroll
    for (int q = 0; q < NLD; ++q) {
      const int j = j0 + w * RPW + q * RPI + l / LPR;
      zr[q] = j < N ? *reinterpret_cast<const u32x4*>(zb + zoff[q]) : u32x4{0u, 0u, 0u, 0u};
    }
    const bf16* Xb = X + (size_t)b * C * pe + (size_t)i * Np + j0;
#pragma unroll
    for (int q = 0; q < XLDS; ++q)
      xr[q] = *reinterpret_cast<const u32x4*>(Xb + (size_t)q * (NT / 8) * pe + xoff);
  };

  int tile = blockIdx.x;
  if (tile < ntiles) issue(tile);
  for (; tile < ntiles; tile += gridDim.x) {
    int b, i, j0;
    tile_coords(tile, b, i, j0);
    // X tile -> LDS [ch][pos]; LN_in(z rows) -> xb (raw z stays in zr for the residual).
#pragma unroll
    for (int q = 0; q < XLDS; ++q) {
      const int c = (tid >> 3) + q * (NT / 8);
      *reinterpret_cast<u32x4*>(xt + c * TLD + 8 * (tid & 7)) = xr[q];
    }
    float zv[NLD][VEC];
#pragma unroll
    for (int q = 0; q < NLD; ++q) {
      unpack16<TZ>(zr[q], zv[q]);
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) sum += zv[q][e];
      const float mean = row_group_sum<LPR>(sum) * (1.0f / C);
      float sq = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float d = zv[q][e] - mean;
        sq += d * d;
      }
      const float rstd = rsqrtf(row_group_sum<LPR>(sq) * (1.0f / C) + eps_in);
      float y[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) y[e] = (zv[q][e] - mean) * rstd * liw[e] + lib[e];
      store_vec<bf16, VEC>(xb + (w * RPW + q * RPI + l / LPR) * XLD + chunk * VEC, y);
    }
    const int next = tile + gridDim.x;
    if (next < ntiles) issue(next);
    __syncthreads();  // xt complete
    {
      float v[16];
      float sum = 0.f;
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        v[c] = (float)xt[och(c) * TLD + op];
        sum += v[c];
      }
      const float mean = dpp_sum8(sum) * (1.0f / C);
      float sq = 0.f;
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const float d = v[c] - mean;
        sq += d * d;
      }
      const float rstd = rsqrtf(dpp_sum8(sq) * (1.0f / C) + eps_out);
#pragma unroll
      for (int c = 0; c < 16; ++c) v[c] = (v[c] - mean) * rstd * low[c] + lob[c];
#pragma unroll
      for (int k = 0; k < 8; ++k) store_vec<bf16, 2>(xa + op * XLD + och(2 * k), v + 2 * k);
    }
    __syncthreads();  // xa, xb complete

    f32x16 ao, ag;
#pragma unroll
    for (int r = 0; r < 16; ++r) ao[r] = ag[r] = 0.f;
    const int brow = (32 * pw + (l & 31)) * XLD + 8 * (l >> 5);
#pragma unroll
    for (int ks = 0; ks < C / 16; ++ks) {
      const bf16x8 fa = *reinterpret_cast<const bf16x8*>(xa + brow + 16 * ks);
      const bf16x8 fb = *reinterpret_cast<const bf16x8*>(xb + brow + 16 * ks);
      ao = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wo[ks], fa, ao, 0, 0, 0);
      ag = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wg[ks], fb, ag, 0, 0, 0);
    }
    // update = sigmoid(gate) * out: lane holds channels 32 cw + acc32_row(r) of position
    // 32 pw + (l & 31).
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      f32x4 u;
#pragma unroll
      for (int e = 0; e < 4; ++e) u[e] = sigmoidf_(ag[4 * g4 + e]) * ao[4 * g4 + e];
      *reinterpret_cast<f32x4*>(upd + (32 * pw + (l & 31)) * SLD + 32 * cw + acc32_row(4 * g4)) = u;
    }
    __syncthreads();  // update tile complete
    TZ* ob = out + ((size_t)b * N + i) * N * C;
#pragma unroll
    for (int q = 0; q < NLD; ++q) {
      const int p = w * RPW + q * RPI + l / LPR;
      const int j = j0 + p;
      if (j >= N) continue;
      float y[VEC];
#pragma unroll
      for (int e = 0; e < VEC; e += 4) {
        const f32x4 u = *reinterpret_cast<const f32x4*>(upd + p * SLD + chunk * VEC + e);
#pragma unroll
        for (int k = 0; k < 4; ++k) y[e + k] = accumulate ? zv[q][e + k] + u[k] : u[k];
      }
      store_vec<TZ, VEC>(ob + (size_t)j * C + chunk * VEC, y);
    }
  }
}

// K3 at 256 channels, persistent and weight-stationary (bf16 GEMMs, bf16 z). One 512-thread
// block per CU walks tiles of 64 positions (i, j0 .. j0+63) of one row. Wave w owns output
// channels 32 w .. +32 for both position halves: its rows of out_proj and out_gate stay in
// registers for the whole launch as 32x32x16 MFMA A operands (128 VGPRs), so no weight
// bytes move per tile. Per tile: the X tile (channel-major, 256 x 64, loaded into registers
// one tile ahead) goes to LDS and is normalised (LN_out) by a pass whose reads run along
// positions; the z rows (also one tile ahead) are normalised (LN_in) from registers that
// keep them for the residual; each 32-position half then runs 32 MFMAs per wave, stages its
// fp32 update block-wide and adds it to the z rows of that half.
struct Output256 {
  static constexpr int C = 256;
  static constexpr int BP = 64;
  static constexpr int NW = 8;
  static constexpr int NT = 64 * NW;
  static constexpr int XLD = C + 8;   // bf16 operand rows [pos][ch]
  static constexpr int TLD = BP + 8;  // bf16 X tile rows [ch][pos]
  static constexpr int SLD = C + 4;   // fp32 update stage rows [pos][ch], one half tile
};

__global__ __launch_bounds__(Output256::NT, 1) void trimul_output256_kernel(
    const bf16* __restrict__ X, const bf16* __restrict__ z, bf16* __restrict__ out, const float* __restrict__ lniw,
    const float* __restrict__ lnib, float eps_in, const float* __restrict__ lnow, const float* __restrict__ lnob,
    float eps_out, const bf16* __restrict__ Wo, const bf16* __restrict__ Wog, int B, int N, int Np, int accumulate) {
  using Cfg = Output256;
  constexpr int C = Cfg::C, BP = Cfg::BP, NW = Cfg::NW, NT = Cfg::NT, XLD = Cfg::XLD, TLD = Cfg::TLD,
                SLD = Cfg::SLD;
  constexpr int VEC = 8;                 // z elements per 16-byte load
  constexpr int LPR = C / VEC;           // lanes per z row (32)
  constexpr int RPI = 64 / LPR;          // z rows per wave-wide load (2)
  constexpr int RPW = BP / NW;           // z rows per wave per tile (8)
  constexpr int NLD = RPW / RPI;         // z loads per lane per tile (4)
  constexpr int XLDS = C * BP / 8 / NT;  // 16-byte X loads per lane per tile (4)
  __shared__ __attribute__((aligned(16))) bf16 xt[C * TLD];   // X tile [ch][pos]
  __shared__ __attribute__((aligned(16))) bf16 xa[BP * XLD];  // LN_out(X) [pos][ch]
  __shared__ __attribute__((aligned(16))) bf16 xb[BP * XLD];  // LN_in(z) [pos][ch]
  __shared__ __attribute__((aligned(16))) float upd[32 * SLD];
  __shared__ float lno[2 * C];  // LN_out weight | bias
  __shared__ float lni[2 * C];  // LN_in weight | bias

  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const int lq = l & 31, hf = l >> 5;
  const int pe = Np * Np;  // plane size (elements); checked below 2^31 / C at launch
  const int tpr = (N + BP - 1) / BP;
  const int ntiles = B * N * tpr;

  // Weights: lane holds row 32 w + lq, k = 16 ks + 8 hf + e.
  bf16x8 wo[C / 16], wg[C / 16];
#pragma unroll
  for (int ks = 0; ks < C / 16; ++ks) {
    const size_t r = (size_t)(32 * w + lq) * C + 16 * ks + 8 * hf;
    wo[ks] = *reinterpret_cast<const bf16x8*>(Wo + r);
    wg[ks] = *reinterpret_cast<const bf16x8*>(Wog + r);
  }
  for (int i = tid; i < C; i += NT) {
    lno[i] = lnow[i];
    lno[C + i] = lnob[i];
    lni[i] = lniw[i];
    lni[C + i] = lnib[i];
  }
  const int chunk = l % LPR;
  // LN_out: thread (position op = tid / 8, part os = tid % 8) normalises the channel pairs
  // 16 k + 2 os + {0, 1}, k = 0..15: the 64 lanes of one read touch 32 distinct dwords in
  // 32 distinct banks (rows 2 os + 16 k, positions op).
  const int op = tid >> 3, os = tid & 7;
  auto och = [&](int c) { return 16 * (c >> 1) + 2 * os + (c & 1); };
  const int zoff0 = (w * RPW + l / LPR) * C + chunk * VEC;  // + q RPI C for load q
  const int xoff = (tid >> 3) * pe + 8 * (tid & 7);

  auto tile_coords = [&](int tile, int& b, int& i, int& j0) {
    b = tile / (N * tpr);
    const int rem = tile - b * (N * tpr);
    i = rem / tpr;
    j0 = (rem - i * tpr) * BP;
  };
  // The tile's loads and residual stores are buffer operations on a per-tile base with
  // 32-bit lane offsets: 64-bit per-lane addresses held across the tile spilled, and each
  // spill reload waited for the next tile's loads in flight. The z rows' buffer ends at
  // position N of the row, so rows past N load zeros and their stores are dropped.
  u32x4 zr[NLD], xr[XLDS];
  auto issue = [&](int tile) {
    int b, i, j0;
    tile_coords(tile, b, i, j0);
    const __amdgpu_buffer_rsrc_t zrs =
        buf_rsrc(z + (((size_t)b * N + i) * N + j0) * C, (unsigned)((N - j0) * C * 2));
#pragma unroll
    for (int q = 0; q < NLD; ++q)
      zr[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(zrs, (zoff0 + q * RPI * C) * 2, 0, 0));
    const __amdgpu_buffer_rsrc_t xrs = buf_rsrc(X + (size_t)b * C * pe, (unsigned)((size_t)C * pe * 2));
#pragma unroll
    for (int q = 0; q < XLDS; ++q)
      xr[q] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     xrs, (int)((unsigned)(i * Np + j0 + q * (NT / 8) * pe + xoff) * 2u), 0, 0));
  };

  // After the LN_out pass the X tile's LDS holds the raw z rows [pos][ch] for the residual.
  bf16* zs = xt;
  int tile = blockIdx.x;
  if (tile < ntiles) issue(tile);
  __syncthreads();  // LN parameters
  for (; tile < ntiles; tile += gridDim.x) {
    int b, i, j0;
    tile_coords(tile, b, i, j0);
    if (tile != (int)blockIdx.x) __syncthreads();  // the last residual pass is done with zs
    // X tile -> LDS [ch][pos]; LN_in(z rows) -> xb
#pragma unroll
    for (int q = 0; q < XLDS; ++q) {
      const int c = (tid >> 3) + q * (NT / 8);
      *reinterpret_cast<u32x4*>(xt + c * TLD + 8 * (tid & 7)) = xr[q];
    }
#pragma unroll
    for (int q = 0; q < NLD; ++q) {
      float zv[VEC];
      unpack16<bf16>(zr[q], zv);
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) sum += zv[e];
      const float mean = row_group_sum<LPR>(sum) * (1.0f / C);
      float sq = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float d = zv[e] - mean;
        sq += d * d;
      }
      const float rstd = rsqrtf(row_group_sum<LPR>(sq) * (1.0f / C) + eps_in);
      float y[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) y[e] = (zv[e] - mean) * rstd * lni[chunk * VEC + e] + lni[C + chunk * VEC + e];
      store_vec<bf16, VEC>(xb + (w * RPW + q * RPI + l / LPR) * XLD + chunk * VEC, y);
    }
    __syncthreads();  // xt complete
    {
      float v[32];
      float sum = 0.f;
#pragma unroll
      for (int c = 0; c < 32; ++c) {
        v[c] = (float)xt[och(c) * TLD + op];
        sum += v[c];
      }
      const float mean = dpp_sum8(sum) * (1.0f / C);
      float sq = 0.f;
#pragma unroll
      for (int c = 0; c < 32; ++c) {
        const float d = v[c] - mean;
        sq += d * d;
      }
      const float rstd = rsqrtf(dpp_sum8(sq) * (1.0f / C) + eps_out);
#pragma unroll
      for (int c = 0; c < 32; ++c) v[c] = (v[c] - mean) * rstd * lno[och(c)] + lno[C + och(c)];
#pragma unroll
      for (int k = 0; k < 16; ++k) store_vec<bf16, 2>(xa + op * XLD + och(2 * k), v + 2 * k);
    }
    __syncthreads();  // xa, xb complete; every wave is done with the X tile
    // raw z rows -> zs (each lane reads back only what it wrote), then the next tile's loads
#pragma unroll
    for (int q = 0; q < NLD; ++q)
      *reinterpret_cast<u32x4*>(zs + (w * RPW + q * RPI + l / LPR) * C + chunk * VEC) = zr[q];
    const int next = tile + gridDim.x;
    if (next < ntiles) issue(next);

    const __amdgpu_buffer_rsrc_t ors =
        buf_rsrc(out + (((size_t)b * N + i) * N + j0) * C, (unsigned)((N - j0) * C * 2));
#pragma unroll 1
    for (int pt = 0; pt < 2; ++pt) {
      f32x16 ao, ag;
#pragma unroll
      for (int r = 0; r < 16; ++r) ao[r] = ag[r] = 0.f;
      const int brow = (32 * pt + lq) * XLD + 8 * hf;
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        const bf16x8 fa = *reinterpret_cast<const bf16x8*>(xa + brow + 16 * ks);
        const bf16x8 fb = *reinterpret_cast<const bf16x8*>(xb + brow + 16 * ks);
        ao = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wo[ks], fa, ao, 0, 0, 0);
        ag = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wg[ks], fb, ag, 0, 0, 0);
      }
      if (pt == 1) __syncthreads();  // the first half's residual pass is done with upd
      // update = sigmoid(gate) * out: lane holds channels 32 w + acc32_row(r) of position
      // 32 pt + lq.
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        f32x4 u;
#pragma unroll
        for (int e = 0; e < 4; ++e) u[e] = sigmoidf_(ag[4 * g4 + e]) * ao[4 * g4 + e];
        *reinterpret_cast<f32x4*>(upd + lq * SLD + 32 * w + acc32_row(4 * g4)) = u;
      }
      __syncthreads();  // this half's update complete
      // waves 4 pt .. 4 pt + 3 hold the z rows of positions 32 pt ..
      if ((w >> 2) == pt) {
#pragma unroll
        for (int q = 0; q < NLD; ++q) {
          const int p = w * RPW + q * RPI + l / LPR;
          float zv[VEC], y[VEC];
          unpack16<bf16>(*reinterpret_cast<const u32x4*>(zs + p * C + chunk * VEC), zv);
#pragma unroll
          for (int e = 0; e < VEC; e += 4) {
            const f32x4 u = *reinterpret_cast<const f32x4*>(upd + (p - 32 * pt) * SLD + chunk * VEC + e);
#pragma unroll
            for (int k = 0; k < 4; ++k) y[e + k] = accumulate ? zv[e + k] + u[k] : u[k];
          }
          bf16x8 o8;
#pragma unroll
          for (int e = 0; e < VEC; ++e) o8[e] = (bf16)y[e];
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o8), ors, (p * C + chunk * VEC) * 2, 0, 0);
        }
      }
    }
  }
}


// K3 on 64 positions of one row i: X tile (channel-major) -> LN_out -> A1 [pos][ch];
// LN_in(z) -> A2; acc^T for g = Wog A2^T and p = Wo A1^T (wave w: channels 32 w, all 64
// positions), update = sigmoid(g) p through an fp32 stage, stored or added.
template <class TZ>
__global__ __launch_bounds__(256) void trimul_output32_kernel(
    const bf16* __restrict__ X, const TZ* __restrict__ z, TZ* __restrict__ out, const float* __restrict__ lniw,
    const float* __restrict__ lnib, float eps_in, const float* __restrict__ lnow, const float* __restrict__ lnob,
    float eps_out, const bf16* __restrict__ Wo, const bf16* __restrict__ Wog, int B, int N, int Np, int accumulate) {
  constexpr int C = 128;
  constexpr int BM = 64;
  constexpr int LD = ld128<bf16>();
  constexpr int XLD = BM + 8;
  constexpr int SLD = C + 4;
  constexpr int NT = 256;
  constexpr int NQ = NT / BM;
  constexpr int R0 = C * XLD * 2;  // Xs, later A2 and (with R1) the fp32 stage
  constexpr int R1 = BM * LD * 2;  // A1
  constexpr int R2 = 128 * LD * 2; // weights
  static_assert(BM * LD * 2 <= R0 && BM * SLD * 4 <= R0 + R1, "LDS aliasing");
  __shared__ __attribute__((aligned(16))) char smem[R0 + R1 + R2];
  __shared__ float red[NQ][BM];
  __shared__ float stat_mean[BM];
  bf16* Xs = reinterpret_cast<bf16*>(smem);
  bf16* A2 = reinterpret_cast<bf16*>(smem);
  float* stage = reinterpret_cast<float*>(smem);
  bf16* A1 = reinterpret_cast<bf16*>(smem + R0);
  bf16* WS = reinterpret_cast<bf16*>(smem + R0 + R1);

  const int j0 = blockIdx.x * BM;
  const int i = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const size_t pe = (size_t)Np * Np;

  Rows128<bf16, 128, NT> wpf;
  wpf.load(Wog, C);
  const TZ* zb = z + (size_t)b * N * N * C;
  LnTile<TZ, bf16, C, BM, NT> zt;
  zt.load([&](int p) -> const TZ* {
    const int j = j0 + p;
    return j < N ? zb + ((size_t)i * N + j) * C : nullptr;
  });
  {
    const bf16* Xb = X + (size_t)b * C * pe + (size_t)i * Np + j0;
#pragma unroll
    for (int it = 0; it < C * BM / 8 / NT; ++it) {
      const int idx = tid + it * NT;
      const int c = idx / (BM / 8);
      const int chunk = idx % (BM / 8);
      *reinterpret_cast<u32x4*>(Xs + c * XLD + chunk * 8) =
          *reinterpret_cast<const u32x4*>(Xb + (size_t)c * pe + chunk * 8);
    }
  }
  __syncthreads();
  {  // LN_out over the channels of each position, transposing into A1 [pos][ch]
    constexpr int CPQ = C / NQ;
    const int p = tid % BM;
    const int q = tid / BM;
    float xv[CPQ];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < CPQ; ++e) {
      xv[e] = (float)Xs[(q * CPQ + e) * XLD + p];
      s += xv[e];
    }
    red[q][p] = s;
    __syncthreads();
    if (q == 0) {
      float t = 0.f;
#pragma unroll
      for (int k = 0; k < NQ; ++k) t += red[k][p];
      stat_mean[p] = t * (1.0f / C);
    }
    __syncthreads();
    const float mean = stat_mean[p];
    float v = 0.f;
#pragma unroll
    for (int e = 0; e < CPQ; ++e) {
      const float d = xv[e] - mean;
      v += d * d;
    }
    __syncthreads();
    red[q][p] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < NQ; ++k) t += red[k][p];
    const float rstd = rsqrtf(t * (1.0f / C) + eps_out);
    float y[CPQ];
#pragma unroll
    for (int e = 0; e < CPQ; ++e) {
      const int c = q * CPQ + e;
      y[e] = (xv[e] - mean) * rstd * lnow[c] + lnob[c];
    }
#pragma unroll
    for (int e = 0; e < CPQ; e += 8) store_vec<bf16, 8>(A1 + p * LD + q * CPQ + e, y + e);
  }
  __syncthreads();  // Xs dead: A2 takes its place
  zt.store(lniw, lnib, eps_in, A2, LD);
  wpf.store(WS, LD);
  __syncthreads();
  wpf.load(Wo, C);
  f32x16 accg[1][2], accp[1][2];
  zero_acc32(accg);
  zero_acc32(accp);
  wave_mma32<bf16, 1, 2, C>(accg, WS, LD, 32 * w, A2, LD, 0);
  __syncthreads();
  wpf.store(WS, LD);
  __syncthreads();
  wave_mma32<bf16, 1, 2, C>(accp, WS, LD, 32 * w, A1, LD, 0);
  __syncthreads();  // A1, A2 dead: fp32 stage [pos][ch]
#pragma unroll
  for (int pj = 0; pj < 2; ++pj)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int ch = 32 * w + acc32_row(4 * g4);
      const int p = 32 * pj + (l & 31);
      f32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = sigmoidf_(accg[0][pj][4 * g4 + e]) * accp[0][pj][4 * g4 + e];
      *reinterpret_cast<f32x4*>(stage + p * SLD + ch) = v;
    }
  __syncthreads();
  TZ* ob = out + (size_t)b * N * N * C;
  auto orow = [&](int p) -> TZ* {
    const int j = j0 + p;
    return j < N ? ob + ((size_t)i * N + j) * C : nullptr;
  };
  store_tile_from_lds<TZ, C, BM, NT>(orow, stage, SLD, accumulate != 0);
}

// ------------------------------------------------------------------ weight packing
// w_proj, w_gate: [2C][C] in block order (rows 0..C-1 feed a, C..2C-1 feed b).
// CB: channels per block of the packed order -- 32 for the persistent bf16 K1 (C = 128, its
// 32x32 tiles), 16 for the generic K1 (every other dtype / channel count).
template <class TS, class TD>
__global__ void trimul_pack_kernel(const TS* __restrict__ wp, const TS* __restrict__ wg, TD* __restrict__ w4, int C,
                                   int CB) {
  const int n = 4 * C * C;
  for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += gridDim.x * blockDim.x) {
    const int row = idx / C;
    const int k = idx % C;
    const int j = row / (4 * CB);
    const int kind = (row % (4 * CB)) / CB;
    const int r = row % CB;
    const int ch = j * CB + r;
    const TS* src = (kind & 1) ? wg : wp;
    const int srow = (kind >= 2 ? C : 0) + ch;
    w4[idx] = from_f32<TD>(to_f32(src[(size_t)srow * C + k]));
  }
}

// C = 128 in bf16 runs the persistent weight-stationary K1/K3 and C = 256 with bf16 z the
// persistent weight-streaming K1; fp32 and the other channel counts (the template stack's 64)
// run the generic tile kernels, as does K3 at 256 channels.
// mx.heads > 0 runs the MHR mix in K3 (always the generic K3).
template <class TZ, class TC, int C>
int trimul_launch(const void* z, const float* mask, const float* lniw, const float* lnib, float eps_in,
                  const void* w4, const float* lnow, const float* lnob, float eps_out, const void* wo,
                  const void* wog, int B, int N, int outgoing, void* out, int accumulate, void* ws,
                  hipStream_t s, const MixSpec& mx) {
  constexpr bool kWs = sizeof(TC) == 2 && C == 128;
  const int Np = pf::pad128(N);
  const size_t pe = (size_t)Np * Np;
  TC* planes = reinterpret_cast<TC*>(ws);
  TC* P = planes;
  TC* Q = planes + (size_t)B * C * pe;
  TC* X = planes + (size_t)2 * B * C * pe;
  {
    constexpr int BM = kWs ? 128 : trimul_bm<TC>();
    dim3 grid(Np / BM, Np, B);
    pf::KernelTimer timer_trimul_project("trimul_project", s);
    if constexpr (kWs) {
      const long ntiles = (long)B * Np * (Np / ProjectWs::BP);
      PF_REQUIRE(ntiles < (1L << 31), PF_ERR_UNSUPPORTED, "trimul_project: B=%d N=%d (B Np Np/64 must stay below 2^31)",
                 B, N);
      const int nblk = (int)std::min<long>(ntiles, pf::cu_count());
      trimul_project_ws_kernel<TZ><<<nblk, ProjectWs::NT, 0, s>>>((const TZ*)z, mask, lniw, lnib, eps_in,
                                                                  (const bf16*)w4, (bf16*)planes, B, N, Np,
                                                                  outgoing);
      (void)grid;
    }
    else if constexpr (sizeof(TC) == 2 && C == 256 && sizeof(TZ) == 2) {  // (fp32 rows would spill)
      const long ntiles = (long)B * Np * (Np / Project256::BP);
      const int nblk = (int)std::min<long>(ntiles, pf::cu_count());
      trimul_project256_kernel<TZ><<<nblk, Project256::NT, 0, s>>>((const TZ*)z, mask, lniw, lnib, eps_in,
                                                                   (const bf16*)w4, (bf16*)planes, B, N, Np,
                                                                   outgoing);
      (void)grid;
    } else
      trimul_project_kernel<TZ, TC, C><<<grid, trimul_nt<C>(), 0, s>>>((const TZ*)z, mask, lniw, lnib, eps_in, (const TC*)w4,
                                                            planes, B, N, Np, outgoing);
    timer_trimul_project.stop();
    if (int e = pf::check_launch("trimul_project")) return e;
  }
  {
    const int G = B * C;
    const int remap = (G % 8 == 0) ? 1 : 0;
    int e = PF_OK;
    if constexpr (sizeof(TC) == 2) {
      if (Np % 768 == 0)
        e = contract_persistent_launch<384>(P, Q, X, G, Np, remap, s);
      else if (Np % 256 == 0)
        e = contract_persistent_launch<256>(P, Q, X, G, Np, remap, s);
      else
        e = contract_generic_launch<TC>(P, Q, X, G, Np, remap, s);
    } else {
      e = contract_generic_launch<TC>(P, Q, X, G, Np, remap, s);
    }
    if (e) return e;
  }
  if (mx.heads > 0) {
    constexpr int BM = trimul_bm<TC>();
    const dim3 grid((N + BM - 1) / BM, N, B);
    pf::KernelTimer timer_trimul_output("trimul_output", s);
    if (mx.heads <= kMhrHeadsSmall)
      trimul_output_kernel<TZ, TC, C, true, true, kMhrHeadsSmall><<<grid, trimul_nt<C>(), 0, s>>>(
          X, (const TZ*)z, (TZ*)out, lniw, lnib, eps_in, lnow, lnob, eps_out, (const TC*)wo, (const TC*)wog, B, N,
          Np, accumulate, mx);
    else
      trimul_output_kernel<TZ, TC, C, true, true><<<grid, trimul_nt<C>(), 0, s>>>(
          X, (const TZ*)z, (TZ*)out, lniw, lnib, eps_in, lnow, lnob, eps_out, (const TC*)wo, (const TC*)wog, B, N,
          Np, accumulate, mx);
    timer_trimul_output.stop();
    if (int e = pf::check_launch("trimul_output")) return e;
  } else {
    constexpr int BM = kWs ? 64 : trimul_bm<TC>();
    dim3 grid((N + BM - 1) / BM, N, B);
    pf::KernelTimer timer_trimul_output("trimul_output", s);
    if constexpr (kWs) {
      const long ntiles = (long)B * N * ((N + OutputWs::BP - 1) / OutputWs::BP);
      PF_REQUIRE(ntiles < (1L << 31) && (long)Np * Np * OutputWs::C < (1L << 31), PF_ERR_UNSUPPORTED,
                 "trimul_output: N=%d B=%d (B N ceil(N/64) and 128 Np^2 must stay below 2^31)", N, B);
      const int nblk = (int)std::min<long>(ntiles, pf::cu_count());
      trimul_output_ws_kernel<TZ><<<nblk, OutputWs::NT, 0, s>>>((const bf16*)X, (const TZ*)z, (TZ*)out, lniw, lnib,
                                                                eps_in, lnow, lnob, eps_out, (const bf16*)wo,
                                                                (const bf16*)wog, B, N, Np, accumulate);
      (void)grid;
    } else if constexpr (sizeof(TC) == 2 && C == 256 && sizeof(TZ) == 2) {
      const long ntiles = (long)B * N * ((N + Output256::BP - 1) / Output256::BP);
      PF_REQUIRE(ntiles < (1L << 31) && (long)Np * Np * Output256::C < (1L << 31), PF_ERR_UNSUPPORTED,
                 "trimul_output: N=%d B=%d (B N ceil(N/64) and 256 Np^2 must stay below 2^31)", N, B);
      const int nblk = (int)std::min<long>(ntiles, pf::cu_count());
      trimul_output256_kernel<<<nblk, Output256::NT, 0, s>>>((const bf16*)X, (const bf16*)z, (bf16*)out, lniw, lnib,
                                                             eps_in, lnow, lnob, eps_out, (const bf16*)wo,
                                                             (const bf16*)wog, B, N, Np, accumulate);
      (void)grid;
    } else
      trimul_output_kernel<TZ, TC, C><<<grid, trimul_nt<C>(), 0, s>>>(X, (const TZ*)z, (TZ*)out, lniw, lnib, eps_in, lnow,
                                                           lnob, eps_out, (const TC*)wo, (const TC*)wog, B, N, Np,
                                                           accumulate, mx);
    timer_trimul_output.stop();
    if (int e = pf::check_launch("trimul_output")) return e;
  }
  return pf::ok();
}

// Training forward (FusedTriMulFunction.forward): the generic K1 and K3 without the input
// LayerNorm, the planes P, Q and the contraction X left in `planes` for the backward.
template <class TZ, class TC, int C>
int trimul_train_launch(const void* x, const float* mask, const void* w4, const float* lnow, const float* lnob,
                        float eps_out, const void* wo, const void* wog, int B, int N, int outgoing, void* planes_ws,
                        void* out, hipStream_t s, const MixSpec& mx) {
  const int Np = pf::pad128(N);
  const size_t pe = (size_t)Np * Np;
  TC* planes = reinterpret_cast<TC*>(planes_ws);
  TC* P = planes;
  TC* Q = planes + (size_t)B * C * pe;
  TC* X = planes + (size_t)2 * B * C * pe;
  constexpr int BM = trimul_bm<TC>();
  if constexpr (sizeof(TC) == 2 && C == 128) {
    // the persistent K1 without its LayerNorm; weights packed in 32-channel blocks
    const long ntiles = (long)B * Np * (Np / ProjectWs::BP);
    PF_REQUIRE(ntiles < (1L << 31), PF_ERR_UNSUPPORTED, "trimul_train_project: B=%d N=%d (B Np Np/64 must stay below 2^31)",
               B, N);
    const int nblk = (int)std::min<long>(ntiles, pf::cu_count());
    trimul_project_ws_kernel<TZ, false><<<nblk, ProjectWs::NT, 0, s>>>((const TZ*)x, mask, nullptr, nullptr, 0.f,
                                                                       (const bf16*)w4, (bf16*)planes, B, N, Np,
                                                                       outgoing);
  } else if constexpr (sizeof(TC) == 2 && C == 256) {
    const long ntiles = (long)B * Np * (Np / Project256::BP);
    const int nblk = (int)std::min<long>(ntiles, pf::cu_count());
    trimul_project256_kernel<TZ, false><<<nblk, Project256::NT, 0, s>>>((const TZ*)x, mask, nullptr, nullptr, 0.f,
                                                                        (const bf16*)w4, (bf16*)planes, B, N, Np,
                                                                        outgoing);
  } else {
    trimul_project_kernel<TZ, TC, C, false><<<dim3(Np / BM, Np, B), trimul_nt<C>(), 0, s>>>(
        (const TZ*)x, mask, nullptr, nullptr, 0.f, (const TC*)w4, planes, B, N, Np, outgoing);
  }
  if (int e = pf::check_launch("trimul_train_project")) return e;
  const int G = B * C;
  const int remap = (G % 8 == 0) ? 1 : 0;
  int e = PF_OK;
  if constexpr (sizeof(TC) == 2) {
    if (Np % 768 == 0)
      e = contract_persistent_launch<384>(P, Q, X, G, Np, remap, s);
    else if (Np % 256 == 0)
      e = contract_persistent_launch<256>(P, Q, X, G, Np, remap, s);
    else
      e = contract_generic_launch<TC>(P, Q, X, G, Np, remap, s);
  } else {
    e = contract_generic_launch<TC>(P, Q, X, G, Np, remap, s);
  }
  if (e) return e;
  if (mx.heads > kMhrHeadsSmall)
    trimul_output_kernel<TZ, TC, C, false, true><<<dim3((N + BM - 1) / BM, N, B), trimul_nt<C>(), 0, s>>>(
        X, (const TZ*)x, (TZ*)out, nullptr, nullptr, 0.f, lnow, lnob, eps_out, (const TC*)wo, (const TC*)wog, B, N,
        Np, 0, mx);
  else if (mx.heads > 0)
    trimul_output_kernel<TZ, TC, C, false, true, kMhrHeadsSmall><<<dim3((N + BM - 1) / BM, N, B), trimul_nt<C>(), 0,
                                                                  s>>>(
        X, (const TZ*)x, (TZ*)out, nullptr, nullptr, 0.f, lnow, lnob, eps_out, (const TC*)wo, (const TC*)wog, B, N,
        Np, 0, mx);
  else
    trimul_output_kernel<TZ, TC, C, false><<<dim3((N + BM - 1) / BM, N, B), trimul_nt<C>(), 0, s>>>(
        X, (const TZ*)x, (TZ*)out, nullptr, nullptr, 0.f, lnow, lnob, eps_out, (const TC*)wo, (const TC*)wog, B, N,
        Np, 0, mx);
  return pf::check_launch("trimul_train_output");
}

}  // namespace

extern "C" {

size_t pf_trimul_workspace_bytes(int B, int N, int C, int cdtype) {
  if (B <= 0 || N <= 0 || C <= 0) return 0;
  const size_t Np = (size_t)pf::pad128(N);
  const size_t es = cdtype == PF_F32 ? 4 : 2;
  return 3 * (size_t)B * C * Np * Np * es;
}

int pf_trimul_pack_weights(const void* w_proj, const void* w_gate, int wdtype, void* packed, int C, int cdtype,
                           void* stream) {
  PF_REQUIRE(w_proj && w_gate && packed, PF_ERR_INVALID_ARG, "pf_trimul_pack_weights: null pointer");
  PF_REQUIRE(C == 64 || C == 128 || C == 256, PF_ERR_UNSUPPORTED, "pf_trimul_pack_weights: C=%d (built: 64, 128, 256)",
             C);
  const int cb = (cdtype == PF_BF16 && C == 128) ? 32 : 16;  // the K1 that will read them (trimul_launch)
  PF_REQUIRE((wdtype == PF_F32 || wdtype == PF_BF16) && (cdtype == PF_F32 || cdtype == PF_BF16), PF_ERR_UNSUPPORTED,
             "pf_trimul_pack_weights: bad dtype");
  hipStream_t s = pf::as_stream(stream);
  const int n = 4 * C * C;
  dim3 grid((n + 255) / 256);
  if (wdtype == PF_F32 && cdtype == PF_F32)
    trimul_pack_kernel<float, float><<<grid, 256, 0, s>>>((const float*)w_proj, (const float*)w_gate, (float*)packed, C, cb);
  else if (wdtype == PF_F32)
    trimul_pack_kernel<float, bf16><<<grid, 256, 0, s>>>((const float*)w_proj, (const float*)w_gate, (bf16*)packed, C, cb);
  else if (cdtype == PF_F32)
    trimul_pack_kernel<bf16, float><<<grid, 256, 0, s>>>((const bf16*)w_proj, (const bf16*)w_gate, (float*)packed, C, cb);
  else
    trimul_pack_kernel<bf16, bf16><<<grid, 256, 0, s>>>((const bf16*)w_proj, (const bf16*)w_gate, (bf16*)packed, C, cb);
  return pf::check_launch("pf_trimul_pack_weights");
}

static int trimul_fwd_impl(const char* fn, const void* z, const float* mask, const float* ln_in_w,
                           const float* ln_in_b, float eps_in, const void* w_packed, const float* ln_out_w,
                           const float* ln_out_b, float eps_out, const void* w_out, const void* w_out_gate, int B,
                           int N, int C, int outgoing, int zdtype, int cdtype, void* out, int accumulate,
                           void* workspace, size_t workspace_bytes, void* stream,
                           const MixSpec& mx) {
  PF_REQUIRE(z && mask && ln_in_w && ln_in_b && w_packed && ln_out_w && w_out && w_out_gate && out &&
                 workspace,
             PF_ERR_INVALID_ARG, "%s: null pointer", fn);
  PF_REQUIRE(B > 0 && N > 0, PF_ERR_INVALID_ARG, "%s: B=%d N=%d", fn, B, N);
  PF_REQUIRE(C == 64 || C == 128 || C == 256, PF_ERR_UNSUPPORTED, "%s: C=%d (built: 64, 128, 256)", fn, C);
  PF_REQUIRE(zdtype == PF_F32 || zdtype == PF_BF16, PF_ERR_UNSUPPORTED, "%s: zdtype %d", fn, zdtype);
  PF_REQUIRE(cdtype == PF_F32 || cdtype == PF_BF16, PF_ERR_UNSUPPORTED, "%s: cdtype %d", fn, cdtype);
  PF_REQUIRE(!(zdtype == PF_BF16 && cdtype == PF_F32), PF_ERR_UNSUPPORTED,
             "%s: bf16 activations with fp32 GEMMs is not a supported regime", fn);
  PF_REQUIRE(pf::aligned16(z) && pf::aligned16(out) && pf::aligned16(workspace) && pf::aligned16(w_packed) &&
                 pf::aligned16(w_out) && pf::aligned16(w_out_gate),
             PF_ERR_ALIGNMENT, "%s: pointers must be 16-byte aligned", fn);
  PF_REQUIRE(workspace_bytes >= pf_trimul_workspace_bytes(B, N, C, cdtype), PF_ERR_WORKSPACE,
             "%s: workspace %zu < %zu bytes", fn, workspace_bytes, pf_trimul_workspace_bytes(B, N, C, cdtype));
  hipStream_t s = pf::as_stream(stream);
  auto run = [&](auto cc) {
    constexpr int CC = decltype(cc)::value;
    if (zdtype == PF_F32 && cdtype == PF_F32)
      return trimul_launch<float, float, CC>(z, mask, ln_in_w, ln_in_b, eps_in, w_packed, ln_out_w, ln_out_b, eps_out,
                                             w_out, w_out_gate, B, N, outgoing, out, accumulate, workspace, s, mx);
    if (zdtype == PF_F32)
      return trimul_launch<float, bf16, CC>(z, mask, ln_in_w, ln_in_b, eps_in, w_packed, ln_out_w, ln_out_b, eps_out,
                                            w_out, w_out_gate, B, N, outgoing, out, accumulate, workspace, s, mx);
    return trimul_launch<bf16, bf16, CC>(z, mask, ln_in_w, ln_in_b, eps_in, w_packed, ln_out_w, ln_out_b, eps_out,
                                         w_out, w_out_gate, B, N, outgoing, out, accumulate, workspace, s, mx);
  };
  if (C == 64) return run(std::integral_constant<int, 64>{});
  if (C == 256) return run(std::integral_constant<int, 256>{});
  return run(std::integral_constant<int, 128>{});
}


int pf_trimul_fwd(const void* z, const float* mask, const float* ln_in_w, const float* ln_in_b, float eps_in,
                  const void* w_packed, const float* ln_out_w, const float* ln_out_b, float eps_out,
                  const void* w_out, const void* w_out_gate, int B, int N, int C, int outgoing, int zdtype, int cdtype,
                  void* out, int accumulate, void* workspace, size_t workspace_bytes, void* stream) {
  PF_REQUIRE(ln_out_b, PF_ERR_INVALID_ARG, "pf_trimul_fwd: null pointer");
  return trimul_fwd_impl("pf_trimul_fwd", z, mask, ln_in_w, ln_in_b, eps_in, w_packed, ln_out_w, ln_out_b, eps_out,
                         w_out, w_out_gate, B, N, C, outgoing, zdtype, cdtype, out, accumulate, workspace,
                         workspace_bytes, stream, MixSpec{0, 0, 0, nullptr});
}

int pf_trimul_mhr_fwd(const void* z, const float* mask, const float* ln_in_w, const float* ln_in_b, float eps_in,
                      const void* w_packed, const float* ln_out_w, const float* ln_out_b, float eps_out,
                      const void* w_out, const void* w_out_gate, int B, int N, int C, int outgoing, int zdtype,
                      int cdtype, void* out, int accumulate, void* workspace, size_t workspace_bytes, int num_heads,
                      int head_norm, const float* w_router, int router_kind, void* stream) {
  MixSpec mx;
  if (int e = mix_spec("pf_trimul_mhr_fwd", C, num_heads, head_norm, w_router, router_kind, ln_out_b, mx)) return e;
  return trimul_fwd_impl("pf_trimul_mhr_fwd", z, mask, ln_in_w, ln_in_b, eps_in, w_packed, ln_out_w, ln_out_b,
                         eps_out, w_out, w_out_gate, B, N, C, outgoing, zdtype, cdtype, out, accumulate, workspace,
                         workspace_bytes, stream, mx);
}

int pf_trimul_train_pack_weights(const void* w_proj, const void* w_gate, int wdtype, void* packed, int C, int cdtype,
                                 void* stream) {
  PF_REQUIRE(w_proj && w_gate && packed, PF_ERR_INVALID_ARG, "pf_trimul_train_pack_weights: null pointer");
  PF_REQUIRE(C == 64 || C == 128 || C == 256, PF_ERR_UNSUPPORTED,
             "pf_trimul_train_pack_weights: C=%d (built: 64, 128, 256)", C);
  PF_REQUIRE((wdtype == PF_F32 || wdtype == PF_BF16) && (cdtype == PF_F32 || cdtype == PF_BF16), PF_ERR_UNSUPPORTED,
             "pf_trimul_train_pack_weights: bad dtype");
  // the K1 and project VJP that read them: 32-channel blocks for bf16 C = 128 (persistent
  // kernels), 16 otherwise
  const int cb = (cdtype == PF_BF16 && C == 128) ? 32 : 16;
  hipStream_t s = pf::as_stream(stream);
  dim3 grid((4 * C * C + 255) / 256);
  if (wdtype == PF_F32 && cdtype == PF_F32)
    trimul_pack_kernel<float, float><<<grid, 256, 0, s>>>((const float*)w_proj, (const float*)w_gate, (float*)packed, C, cb);
  else if (wdtype == PF_F32)
    trimul_pack_kernel<float, bf16><<<grid, 256, 0, s>>>((const float*)w_proj, (const float*)w_gate, (bf16*)packed, C, cb);
  else if (cdtype == PF_F32)
    trimul_pack_kernel<bf16, float><<<grid, 256, 0, s>>>((const bf16*)w_proj, (const bf16*)w_gate, (float*)packed, C, cb);
  else
    trimul_pack_kernel<bf16, bf16><<<grid, 256, 0, s>>>((const bf16*)w_proj, (const bf16*)w_gate, (bf16*)packed, C, cb);
  return pf::check_launch("pf_trimul_train_pack_weights");
}

static int trimul_train_fwd_impl(const char* fn, const void* x, const float* mask, const void* w_packed,
                                 const float* ln_out_w, const float* ln_out_b, float eps_out, const void* w_out,
                                 const void* w_out_gate, int B, int N, int C, int outgoing, int xdtype, int cdtype,
                                 void* planes, size_t planes_bytes, void* out, void* stream, const MixSpec& mx) {
  PF_REQUIRE(x && mask && w_packed && ln_out_w && w_out && w_out_gate && planes && out,
             PF_ERR_INVALID_ARG, "%s: null pointer", fn);
  PF_REQUIRE(B > 0 && N > 0, PF_ERR_INVALID_ARG, "%s: B=%d N=%d", fn, B, N);
  PF_REQUIRE(C == 64 || C == 128 || C == 256, PF_ERR_UNSUPPORTED, "%s: C=%d (built: 64, 128, 256)", fn, C);
  PF_REQUIRE((xdtype == PF_F32 || xdtype == PF_BF16) && (cdtype == PF_F32 || cdtype == PF_BF16) &&
                 !(xdtype == PF_BF16 && cdtype == PF_F32),
             PF_ERR_UNSUPPORTED, "%s: xdtype %d cdtype %d", fn, xdtype, cdtype);
  PF_REQUIRE(pf::aligned16(x) && pf::aligned16(out) && pf::aligned16(planes) && pf::aligned16(w_packed) &&
                 pf::aligned16(w_out) && pf::aligned16(w_out_gate),
             PF_ERR_ALIGNMENT, "%s: pointers must be 16-byte aligned", fn);
  PF_REQUIRE(planes_bytes >= pf_trimul_workspace_bytes(B, N, C, cdtype), PF_ERR_WORKSPACE,
             "%s: planes buffer %zu < %zu bytes", fn, planes_bytes,
             pf_trimul_workspace_bytes(B, N, C, cdtype));
  hipStream_t s = pf::as_stream(stream);
  auto run = [&](auto cc) {
    constexpr int CC = decltype(cc)::value;
    if (xdtype == PF_F32 && cdtype == PF_F32)
      return trimul_train_launch<float, float, CC>(x, mask, w_packed, ln_out_w, ln_out_b, eps_out, w_out, w_out_gate,
                                                   B, N, outgoing, planes, out, s, mx);
    if (xdtype == PF_F32)
      return trimul_train_launch<float, bf16, CC>(x, mask, w_packed, ln_out_w, ln_out_b, eps_out, w_out, w_out_gate,
                                                  B, N, outgoing, planes, out, s, mx);
    return trimul_train_launch<bf16, bf16, CC>(x, mask, w_packed, ln_out_w, ln_out_b, eps_out, w_out, w_out_gate, B,
                                               N, outgoing, planes, out, s, mx);
  };
  if (C == 64) return run(std::integral_constant<int, 64>{});
  if (C == 256) return run(std::integral_constant<int, 256>{});
  return run(std::integral_constant<int, 128>{});
}

int pf_trimul_train_fwd(const void* x, const float* mask, const void* w_packed, const float* ln_out_w,
                        const float* ln_out_b, float eps_out, const void* w_out, const void* w_out_gate, int B, int N,
                        int C, int outgoing, int xdtype, int cdtype, void* planes, size_t planes_bytes, void* out,
                        void* stream) {
  PF_REQUIRE(ln_out_b, PF_ERR_INVALID_ARG, "pf_trimul_train_fwd: null pointer");
  return trimul_train_fwd_impl("pf_trimul_train_fwd", x, mask, w_packed, ln_out_w, ln_out_b, eps_out, w_out,
                               w_out_gate, B, N, C, outgoing, xdtype, cdtype, planes, planes_bytes, out, stream,
                               MixSpec{0, 0, 0, nullptr});
}

int pf_trimul_mhr_train_fwd(const void* x, const float* mask, const void* w_packed, const float* ln_out_w,
                            const float* ln_out_b, float eps_out, const void* w_out, const void* w_out_gate, int B,
                            int N, int C, int outgoing, int xdtype, int cdtype, void* planes, size_t planes_bytes,
                            void* out, int num_heads, int head_norm, const float* w_router, int router_kind,
                            void* stream) {
  MixSpec mx;
  if (int e = mix_spec("pf_trimul_mhr_train_fwd", C, num_heads, head_norm, w_router, router_kind, ln_out_b, mx))
    return e;
  return trimul_train_fwd_impl("pf_trimul_mhr_train_fwd", x, mask, w_packed, ln_out_w, ln_out_b, eps_out, w_out,
                               w_out_gate, B, N, C, outgoing, xdtype, cdtype, planes, planes_bytes, out, stream, mx);
}

int pf_planes_contract(const void* A, const void* Bm, void* X, int G, int Np, int dtype, void* stream) {
  PF_REQUIRE(A && Bm && X && X != A && X != Bm, PF_ERR_INVALID_ARG, "pf_planes_contract: null or aliased pointers");
  PF_REQUIRE(G > 0 && Np > 0 && Np % 128 == 0, PF_ERR_INVALID_ARG, "pf_planes_contract: G=%d Np=%d (a multiple of 128)",
             G, Np);
  PF_REQUIRE(dtype == PF_F32 || dtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_planes_contract: dtype %d", dtype);
  PF_REQUIRE(pf::aligned16(A) && pf::aligned16(Bm) && pf::aligned16(X), PF_ERR_ALIGNMENT,
             "pf_planes_contract: pointers must be 16-byte aligned");
  hipStream_t s = pf::as_stream(stream);
  const int remap = (G % 8 == 0) ? 1 : 0;
  if (dtype == PF_BF16) {
    if (Np % 768 == 0) return contract_persistent_launch<384>(A, Bm, X, G, Np, remap, s);
    if (Np % 256 == 0) return contract_persistent_launch<256>(A, Bm, X, G, Np, remap, s);
    return contract_generic_launch<bf16>(A, Bm, X, G, Np, remap, s);
  }
  return contract_generic_launch<float>(A, Bm, X, G, Np, remap, s);
}

}  // extern "C"
