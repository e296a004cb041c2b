// Batched NT GEMM on MFMA tiles (see gemm.h): 128 x 128 output tile per 256-thread block,
// four waves in a 2 x 2 grid of 64 x 64, k-tiles double-buffered through LDS. Rows past M or
// N load the last valid row (their results are not stored), so any M, N work; K is a
// multiple of the k-tile. Serves the generic paths (outer product mean, MSA pair-weighted
// averaging), where M, N and K follow the sequence and residue counts.
#include <algorithm>

#include "capi.h"
#include "common.h"
#include "gemm.h"

namespace {

template <class TC>
struct BgemmCfg {
  static constexpr int BMN = 128;
  static constexpr int KT = sizeof(TC) == 2 ? 64 : 32;
  static constexpr int LDK = KT + lds_pad<TC>();
  static constexpr int TILE_ELEMS = BMN * LDK;
  static constexpr int SMEM = 2 * 2 * TILE_ELEMS * (int)sizeof(TC);
};

template <class TC, class TO>
__global__ __launch_bounds__(256) void bgemm_nt_kernel(const TC* __restrict__ A, const TC* __restrict__ Bm,
                                                       TO* __restrict__ Cm, int M, int N, int K, long lda, long ldb,
                                                       long ldc, long sA, long sB, long sC) {
  using Cfg = BgemmCfg<TC>;
  using MF = Mfma<TC>;
  constexpr int BMN = Cfg::BMN, KT = Cfg::KT, LDK = Cfg::LDK;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  TC* lds = reinterpret_cast<TC*>(smem);

  const int tn = (N + BMN - 1) / BMN;
  const int i0 = (blockIdx.x / tn) * BMN;
  const int j0 = (blockIdx.x % tn) * BMN;
  const TC* Ab = A + (size_t)blockIdx.y * sA;
  const TC* Bb = Bm + (size_t)blockIdx.y * sB;
  TO* Cb = Cm + (size_t)blockIdx.y * sC;

  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const int wr = (w >> 1) * 64;
  const int wc = (w & 1) * 64;

  constexpr int VEC = 16 / sizeof(TC);
  constexpr int CPR = KT / VEC;
  constexpr int LOADS = 2 * BMN * CPR / 256;
  static_assert((2 * BMN * CPR) % 256 == 0, "stage must split evenly");
  u32x4 reg[LOADS];
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < LOADS; ++q) {
      const int idx = tid + q * 256;
      const int row = idx / CPR;
      const int chunk = idx % CPR;
      const TC* src = row < BMN ? Ab + (size_t)min(i0 + row, M - 1) * lda
                                : Bb + (size_t)min(j0 + row - BMN, N - 1) * ldb;
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
  const int nk = K / KT;
  gload(0);
  lstore(0);
  __syncthreads();
  const int r = l & 15;
  const int kq = (l >> 4) * MF::KPL;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * KT);
    const TC* As = lds + buf * 2 * Cfg::TILE_ELEMS;
    const TC* Bs = As + Cfg::TILE_ELEMS;
#pragma unroll
    for (int kk = 0; kk < KT; kk += MF::K16) {
      typename MF::Frag af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = MF::load(As + (wr + i * 16 + r) * LDK + kk + kq);
#pragma unroll
      for (int j = 0; j < 4; ++j) bfr[j] = MF::load(Bs + (wc + j * 16 + r) * LDK + kk + kq);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) MF::mma16(acc[i][j], af[i], bfr[j]);
    }
    if (kt + 1 < nk) lstore(buf ^ 1);
    __syncthreads();
  }
  // acc[i][j][e]: row wr + 16 i + 4 (l >> 4) + e, column wc + 16 j + (l & 15)
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = j0 + wc + j * 16 + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = i0 + wr + i * 16 + 4 * (l >> 4) + e;
        if (m < M && n < N) Cb[(size_t)m * ldc + n] = from_f32<TO>(acc[i][j][e]);
      }
    }
}

template <class TC, class TO>
int bgemm_launch(const void* A, const void* B, void* C, int M, int N, int K, long lda, long ldb, long ldc, long sA,
                 long sB, long sC, int batch, hipStream_t s) {
  using Cfg = BgemmCfg<TC>;
  const hipError_t e = hipFuncSetAttribute((const void*)bgemm_nt_kernel<TC, TO>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::SMEM);
  PF_REQUIRE(e == hipSuccess, PF_ERR_LAUNCH, "bgemm: cannot reserve %d bytes of LDS: %s", Cfg::SMEM,
             hipGetErrorString(e));
  const long tiles = (long)((M + Cfg::BMN - 1) / Cfg::BMN) * ((N + Cfg::BMN - 1) / Cfg::BMN);
  PF_REQUIRE(tiles < (1L << 31) && batch < 65536, PF_ERR_UNSUPPORTED, "bgemm: M=%d N=%d batch=%d", M, N, batch);
  bgemm_nt_kernel<TC, TO><<<dim3((unsigned)tiles, (unsigned)batch), 256, Cfg::SMEM, s>>>(
      (const TC*)A, (const TC*)B, (TO*)C, M, N, K, lda, ldb, ldc, sA, sB, sC);
  return pf::check_launch("bgemm");
}

// Row GEMM over many rows: out[m][n] = epi(sum_k A[m][k] W[n][k]) on the bgemm tiling
// (128 rows x 128 weight rows per block, 2 x 2 waves of 64 x 64, k-tiles through LDS), with
// the row GEMM's epilogues: EPI 0 store, 1 add into out (residual), 2 SwiGLU (W has 2 Nout
// rows; out column j = silu(h_j) h_{Nout + j}). SwiGLU tiles cover 64 output columns: the
// B tile's rows are, per wave column, 32 "a" rows then the 32 matching "b" rows, so a lane
// holds both factors of each output (accumulator blocks j and j + 2). A [M][K], W [*][K],
// out [M][Nout], all row-major with k or n contiguous. Blocks walk the weight tiles of one
// row tile consecutively (the A tile stays in L2).
// The many-row GEMM's tiles: k-tiles half the batched GEMM's (41 KB of LDS per block, three
// blocks per CU), so more blocks keep loads in flight over the short k loops (K = 128-1024).
template <class TC>
struct TileRowsCfg {
  static constexpr int BMN = 128;
  static constexpr int KT = sizeof(TC) == 2 ? 32 : 16;
  static constexpr int LDK = KT + lds_pad<TC>();
  static constexpr int TILE_ELEMS = BMN * LDK;
  static constexpr int SMEM = 2 * 2 * TILE_ELEMS * (int)sizeof(TC);
  static constexpr int OSMEM = BMN / 2 * (128 + 4) * 4;  // the fp32 output stage, half a tile
  static constexpr int LDS = SMEM > OSMEM ? SMEM : OSMEM;
};

// GATE: the A operand is A * gate elementwise (gate [M][K] like A, bf16 operands), each
// product rounded to the operand dtype as it enters the LDS tile.
template <class TC, class TO, int EPI, bool GATE = false>
__global__ __launch_bounds__(256) void tile_gemm_rows_kernel(const TC* __restrict__ A, const TC* __restrict__ W,
                                                             TO* __restrict__ out, long M, int Nout, int K,
                                                             int vec_out, const TC* __restrict__ gate = nullptr) {
  using Cfg = TileRowsCfg<TC>;
  using MF = Mfma<TC>;
  constexpr int BMN = Cfg::BMN, KT = Cfg::KT, LDK = Cfg::LDK;
  constexpr int OCT = EPI == 2 ? 64 : 128;  // output columns per tile
  extern __shared__ __attribute__((aligned(16))) char smem[];
  TC* lds = reinterpret_cast<TC*>(smem);

  const int tn = (Nout + OCT - 1) / OCT;
  // Blocks are dispatched round-robin over the 8 XCDs; when the grid splits evenly, XCD x
  // takes the x-th eighth of the tiles in order, so the column tiles of one row tile run on
  // one XCD one after another and the second reads A from that XCD's L2.
  const unsigned nb = gridDim.x;
  const unsigned bid = nb % 8 == 0 ? (blockIdx.x & 7) * (nb >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const long i0 = (long)(bid / tn) * BMN;
  const int oc0 = (int)(bid % tn) * OCT;
  const int tid = threadIdx.x;
  const int w = wave_id();
  const int l = lane_id();
  const int wr = (w >> 1) * 64;
  const int wc = (w & 1) * 64;

  // Weight row of B-tile row rr.
  auto wrow = [&](int rr) -> int {
    if constexpr (EPI == 2) {
      const int col = min(oc0 + (rr >> 6) * 32 + (rr & 31), Nout - 1);
      return (rr & 32) ? Nout + col : col;
    } else {
      return min(oc0 + rr, Nout - 1);
    }
  };

  constexpr int VEC = 16 / sizeof(TC);
  constexpr int CPR = KT / VEC;
  constexpr int LOADS = 2 * BMN * CPR / 256;
  static_assert((2 * BMN * CPR) % 256 == 0, "stage must split evenly");
  constexpr int ALOADS = BMN * CPR / 256;  // loads q < ALOADS are A rows, the rest W rows
  static_assert((BMN * CPR) % 256 == 0, "A rows must fill whole loads");
  static_assert(!GATE || sizeof(TC) == 2, "the gated operand is bf16");
  const TC* src_row[LOADS];
  int dst_off[LOADS];
#pragma unroll
  for (int q = 0; q < LOADS; ++q) {
    const int idx = tid + q * 256;
    const int row = idx / CPR;
    const int chunk = idx % CPR;
    src_row[q] = (row < BMN ? A + (size_t)min(i0 + row, M - 1) * K : W + (size_t)wrow(row - BMN) * K) + chunk * VEC;
    dst_off[q] = row * LDK + chunk * VEC;
  }
  u32x4 reg[LOADS];
  u32x4 greg[GATE ? ALOADS : 1];
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < LOADS; ++q) reg[q] = *reinterpret_cast<const u32x4*>(src_row[q] + k0);
    if constexpr (GATE) {
#pragma unroll
      for (int q = 0; q < ALOADS; ++q)
        greg[q] = *reinterpret_cast<const u32x4*>(src_row[q] - A + gate + k0);
    }
  };
  auto lstore = [&](int buf) {
    TC* base = lds + buf * 2 * Cfg::TILE_ELEMS;
    if constexpr (GATE) {
#pragma unroll
      for (int q = 0; q < ALOADS; ++q) {
        const bf16x8 a = __builtin_bit_cast(bf16x8, reg[q]);
        const bf16x8 g = __builtin_bit_cast(bf16x8, greg[q]);
        bf16x8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (bf16)((float)a[e] * (float)g[e]);
        reg[q] = __builtin_bit_cast(u32x4, v);
      }
    }
#pragma unroll
    for (int q = 0; q < LOADS; ++q) *reinterpret_cast<u32x4*>(base + dst_off[q]) = reg[q];
  };

  f32x4 acc[4][4];
  zero_acc(acc);
  const int nk = K / KT;
  gload(0);
  lstore(0);
  __syncthreads();
  const int r = l & 15;
  const int kq = (l >> 4) * MF::KPL;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * KT);
    const TC* As = lds + buf * 2 * Cfg::TILE_ELEMS;
    const TC* Bs = As + Cfg::TILE_ELEMS;
#pragma unroll
    for (int kk = 0; kk < KT; kk += MF::K16) {
      typename MF::Frag af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = MF::load(As + (wr + i * 16 + r) * LDK + kk + kq);
#pragma unroll
      for (int j = 0; j < 4; ++j) bfr[j] = MF::load(Bs + (wc + j * 16 + r) * LDK + kk + kq);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) MF::mma16(acc[i][j], af[i], bfr[j]);
    }
    if (kt + 1 < nk) lstore(buf ^ 1);
    __syncthreads();
  }
  // acc[i][j][e]: row wr + 16 i + 4 (l >> 4) + e, B-tile row wc + 16 j + (l & 15). The tile
  // (after the SwiGLU pairing) is staged in fp32 through the LDS the k loop used, half a
  // tile (64 rows: waves 0-1, then 2-3) at a time, and leaves as 16-byte row pieces (with the
  // residual read the same way); rounding as a direct store.
  constexpr int SLD = OCT + 4;
  constexpr int HR = BMN / 2;
  static_assert(HR * SLD * 4 <= Cfg::LDS, "the output stage must fit the block's LDS");
  float* st = reinterpret_cast<float*>(smem);
  constexpr int OV = 16 / sizeof(TO);  // outputs per 16-byte piece
  constexpr int PPR = OCT / OV;        // pieces per tile row
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    if ((wr >> 6) == half) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = i * 16 + 4 * (l >> 4) + e;  // within the half
          if constexpr (EPI == 2) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
              st[row * SLD + (wc >> 6) * 32 + j * 16 + r] = siluf_(acc[i][j][e]) * acc[i][j + 2][e];
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) st[row * SLD + wc + j * 16 + r] = acc[i][j][e];
          }
        }
    }
    __syncthreads();
    for (int idx = tid; idx < HR * PPR; idx += 256) {
      const int row = idx / PPR;
      const int c0 = (idx % PPR) * OV;
      const long m = i0 + half * HR + row;
      const int n0 = oc0 + c0;
      if (m >= M || n0 >= Nout) continue;
      TO* dst = out + m * Nout + n0;
      float v[OV];
#pragma unroll
      for (int e = 0; e < OV; ++e) v[e] = st[row * SLD + c0 + e];
      if (vec_out && n0 + OV <= Nout) {
        if constexpr (EPI == 1) {
          float rv[OV];
          load16<TO>(dst, rv);
#pragma unroll
          for (int e = 0; e < OV; ++e) v[e] += rv[e];
        }
        store_vec<TO, OV>(dst, v);
      } else {
        for (int e = 0; e < OV && n0 + e < Nout; ++e) {
          if constexpr (EPI == 1)
            dst[e] = from_f32<TO>(to_f32(dst[e]) + v[e]);
          else
            dst[e] = from_f32<TO>(v[e]);
        }
      }
    }
    if (half == 0) __syncthreads();
  }
}

template <class TC, class TO, int EPI, bool GATE = false>
int tile_gemm_rows_launch(const void* A, const void* W, void* out, long M, int Nout, int K, hipStream_t s,
                          const void* gate = nullptr) {
  using Cfg = TileRowsCfg<TC>;
  const void* fn = (const void*)tile_gemm_rows_kernel<TC, TO, EPI, GATE>;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::LDS);
  PF_REQUIRE(e == hipSuccess, PF_ERR_LAUNCH, "row gemm: cannot reserve %d bytes of LDS: %s", Cfg::LDS,
             hipGetErrorString(e));
  const long tn = (Nout + (EPI == 2 ? 64 : 128) - 1) / (EPI == 2 ? 64 : 128);
  const long blocks = (M + Cfg::BMN - 1) / Cfg::BMN * tn;
  PF_REQUIRE(blocks < (1L << 31), PF_ERR_UNSUPPORTED, "row gemm: M=%ld Nout=%d", M, Nout);
  const int vec_out = pf::aligned16(out) && Nout % (16 / (int)sizeof(TO)) == 0;
  tile_gemm_rows_kernel<TC, TO, EPI, GATE><<<dim3((unsigned)blocks), 256, Cfg::LDS, s>>>(
      (const TC*)A, (const TC*)W, (TO*)out, M, Nout, K, vec_out, (const TC*)gate);
  return pf::check_launch("row gemm");
}

template <class TC, class TO>
int tile_gemm_rows_epi(const void* A, const void* W, void* out, long M, int Nout, int K, int epi, hipStream_t s) {
  if (epi == 1) return tile_gemm_rows_launch<TC, TO, 1>(A, W, out, M, Nout, K, s);
  if (epi == 2) return tile_gemm_rows_launch<TC, TO, 2>(A, W, out, M, Nout, K, s);
  return tile_gemm_rows_launch<TC, TO, 0>(A, W, out, M, Nout, K, s);
}

}  // namespace

int tile_gemm_rows(const void* A, const void* W, void* out, long M, int Nout, int K, int epi, int tc_dtype,
                   int out_dtype, hipStream_t s) {
  const int kt = tc_dtype == PF_F32 ? TileRowsCfg<float>::KT : TileRowsCfg<bf16>::KT;
  PF_REQUIRE(M > 0 && Nout > 0 && K > 0 && K % kt == 0 && epi >= 0 && epi <= 2, PF_ERR_INVALID_ARG,
             "row gemm: M=%ld Nout=%d K=%d (a multiple of %d) epi=%d", M, Nout, K, kt, epi);
  if (tc_dtype == PF_F32) return tile_gemm_rows_epi<float, float>(A, W, out, M, Nout, K, epi, s);
  if (out_dtype == PF_F32) return tile_gemm_rows_epi<bf16, float>(A, W, out, M, Nout, K, epi, s);
  return tile_gemm_rows_epi<bf16, bf16>(A, W, out, M, Nout, K, epi, s);
}

int tile_gemm_rows_gated(const void* A, const void* gate, const void* W, void* out, long M, int Nout, int K,
                         int accumulate, int out_dtype, hipStream_t s) {
  constexpr int kt = TileRowsCfg<bf16>::KT;
  PF_REQUIRE(M > 0 && Nout > 0 && K > 0 && K % kt == 0, PF_ERR_INVALID_ARG,
             "gated row gemm: M=%ld Nout=%d K=%d (a multiple of %d)", M, Nout, K, kt);
  PF_REQUIRE(pf::aligned16(A) && pf::aligned16(gate) && pf::aligned16(W), PF_ERR_INVALID_ARG,
             "gated row gemm: operands must be 16-byte aligned");
  if (out_dtype == PF_F32)
    return accumulate ? tile_gemm_rows_launch<bf16, float, 1, true>(A, W, out, M, Nout, K, s, gate)
                      : tile_gemm_rows_launch<bf16, float, 0, true>(A, W, out, M, Nout, K, s, gate);
  return accumulate ? tile_gemm_rows_launch<bf16, bf16, 1, true>(A, W, out, M, Nout, K, s, gate)
                    : tile_gemm_rows_launch<bf16, bf16, 0, true>(A, W, out, M, Nout, K, s, gate);
}

int bgemm_nt(const void* A, const void* B, void* C, int M, int N, int K, long lda, long ldb, long ldc, long sA,
             long sB, long sC, int batch, int tc_dtype, int out_dtype, hipStream_t s) {
  PF_REQUIRE(M > 0 && N > 0 && K > 0 && K % kBgemmK == 0 && batch > 0, PF_ERR_INVALID_ARG,
             "bgemm: M=%d N=%d K=%d (a multiple of %d) batch=%d", M, N, K, kBgemmK, batch);
  if (tc_dtype == PF_F32) return bgemm_launch<float, float>(A, B, C, M, N, K, lda, ldb, ldc, sA, sB, sC, batch, s);
  if (out_dtype == PF_F32) return bgemm_launch<bf16, float>(A, B, C, M, N, K, lda, ldb, ldc, sA, sB, sC, batch, s);
  return bgemm_launch<bf16, bf16>(A, B, C, M, N, K, lda, ldb, ldc, sA, sB, sC, batch, s);
}
