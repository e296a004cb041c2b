// Row kernels shared by the single track and the generic-channel pair paths: LayerNorm
// of [M, C] rows into the GEMM operand dtype, and a row GEMM out = epi(A W^T [+ bias]) with
// store / residual-add / SwiGLU epilogues. Included into each translation unit (internal
// linkage), so each keeps its own instantiations.
#pragma once

#include "capi.h"
#include "common.h"
#include "gemm.h"

namespace {

// ------------------------------------------------------------------ LayerNorm rows -> TO
template <class TI, class TO>
__global__ __launch_bounds__(256) void ln_rows_kernel(const TI* __restrict__ x, const float* __restrict__ w,
                                                      const float* __restrict__ b, float eps, TO* __restrict__ out,
                                                      long M, int C) {
  const long row = (long)blockIdx.x * 4 + wave_id();
  if (row >= M) return;
  const int l = lane_id();
  const TI* src = x + row * C;
  float s = 0.f;
  for (int c = l; c < C; c += 64) s += to_f32(src[c]);
  const float mean = group_sum<64>(s) / C;
  float q = 0.f;
  for (int c = l; c < C; c += 64) {
    const float d = to_f32(src[c]) - mean;
    q += d * d;
  }
  const float rstd = rsqrtf(group_sum<64>(q) / C + eps);
  TO* dst = out + row * C;
  for (int c = l; c < C; c += 64) dst[c] = from_f32<TO>((to_f32(src[c]) - mean) * rstd * w[c] + b[c]);
}

// LayerNorm rows with 8 elements per lane (16-byte bf16 loads): C / 8 lanes per row, 64 / (C / 8)
// rows per wave, statistics by shuffles within the row's lanes. C in {64, 128, 256, 512}.
template <class TI, class TO, int C>
__global__ __launch_bounds__(256) void ln_rows_vec_kernel(const TI* __restrict__ x, const float* __restrict__ w,
                                                          const float* __restrict__ b, float eps, TO* __restrict__ out,
                                                          long M) {
  constexpr int LPR = C / 8;
  constexpr int RPW = 64 / LPR;
  static_assert(LPR >= 8 && LPR <= 64 && 64 % LPR == 0, "8 to 64 lanes per row");
  const int l = lane_id();
  const long row = ((long)blockIdx.x * 4 + wave_id()) * RPW + l / LPR;
  if (row >= M) return;  // whole row groups leave together: the shuffles stay within a group
  const int c0 = (l % LPR) * 8;
  const TI* src = x + row * C + c0;
  float v[8];
  if constexpr (sizeof(TI) == 2) {
    load16<TI>(src, v);
  } else {
    float a[4], bb[4];
    load16<TI>(src, a);
    load16<TI>(src + 4, bb);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = a[e], v[e + 4] = bb[e];
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s += v[e];
  const float mean = group_sum<LPR>(s) / C;
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float d = v[e] - mean;
    q += d * d;
  }
  const float rstd = rsqrtf(group_sum<LPR>(q) / C + eps);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = (v[e] - mean) * rstd * w[c0 + e] + b[c0 + e];
  TO* dst = out + row * C + c0;
  if constexpr (sizeof(TO) == 2) {
    store_vec<TO, 8>(dst, y);
  } else {
    store_vec<TO, 4>(dst, y);
    store_vec<TO, 4>(dst + 4, y + 4);
  }
}

// ------------------------------------------------------------------ row GEMM
enum { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2 };

// out = epi(A W^T [+ bias]); A [M][K], W [Nw][K] (TC, k contiguous). One block computes a
// (16 RB)-row x 64-column output tile, each wave one 16-column block over RB row blocks;
// the operands come straight from global memory (L2), four k-steps' loads in flight.
// RB = 2 when the 64-row grid would leave most CUs idle (the single track has N rows).
// EPI_SWIGLU: output column j is silu(h_j) * h_{F + j} with F = Nout (W has 2 Nout rows).
// bias (fp32, may be null) applies to the first nbias output columns (EPI_STORE only).
template <class TC, class TO, int EPI, int RB>
__global__ __launch_bounds__(256) void rowgemm_kernel(const TC* __restrict__ A, const TC* __restrict__ W,
                                                      const float* __restrict__ bias, int nbias, TO* __restrict__ out,
                                                      long M, int Nout, int K) {
  using MF = Mfma<TC>;
  const int w = wave_id();
  const int l = lane_id();
  const long m0 = (long)blockIdx.x * 16 * RB;
  const int n0 = blockIdx.y * 64 + w * 16;
  if (n0 >= Nout) return;
  const int r = l & 15;
  const int kq = (l >> 4) * MF::KPL;
  f32x4 acc[RB], acc2[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) acc[i] = acc2[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  const TC* arow[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    long m = m0 + i * 16 + r;
    if (m >= M) m = M - 1;
    arow[i] = A + m * K;
  }
  const TC* wrow = W + (size_t)(n0 + r) * K;
  const TC* wrow2 = W + (size_t)(Nout + n0 + r) * K;
  auto kstep = [&](int k0) __attribute__((always_inline)) {
    const typename MF::Frag bf = MF::load(wrow + k0 + kq);
    typename MF::Frag bf2;
    if (EPI == EPI_SWIGLU) bf2 = MF::load(wrow2 + k0 + kq);
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const typename MF::Frag af = MF::load(arow[i] + k0 + kq);
      MF::mma16(acc[i], af, bf);
      if (EPI == EPI_SWIGLU) MF::mma16(acc2[i], af, bf2);
    }
  };
  // Four k-steps per trip (their loads in flight together), then the remainder.
  int k0 = 0;
  for (; k0 + 4 * MF::K16 <= K; k0 += 4 * MF::K16) {
#pragma unroll
    for (int j = 0; j < 4; ++j) kstep(k0 + j * MF::K16);
  }
  for (; k0 < K; k0 += MF::K16) kstep(k0);
  const int n = n0 + r;
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const long m = m0 + i * 16 + 4 * (l >> 4) + e;
      if (m >= M) continue;
      float y = acc[i][e];
      TO* dst = out + m * Nout + n;
      if (EPI == EPI_SWIGLU) {
        y = siluf_(y) * acc2[i][e];
        *dst = from_f32<TO>(y);
      } else if (EPI == EPI_RESIDUAL) {
        *dst = from_f32<TO>(to_f32(*dst) + y);
      } else {
        if (bias && n < nbias) y += bias[n];
        *dst = from_f32<TO>(y);
      }
    }
}


template <class TI, class TO>
int ln_launch(const void* x, const float* w, const float* b, float eps, void* out, long M, int C, hipStream_t s) {
  if (pf::aligned16(x) && pf::aligned16(out) && (C == 64 || C == 128 || C == 256 || C == 512)) {
    const long rows_per_block = 4L * (64 / (C / 8));
    const unsigned grid = (unsigned)((M + rows_per_block - 1) / rows_per_block);
    switch (C) {
      case 64: ln_rows_vec_kernel<TI, TO, 64><<<grid, 256, 0, s>>>((const TI*)x, w, b, eps, (TO*)out, M); break;
      case 128: ln_rows_vec_kernel<TI, TO, 128><<<grid, 256, 0, s>>>((const TI*)x, w, b, eps, (TO*)out, M); break;
      case 256: ln_rows_vec_kernel<TI, TO, 256><<<grid, 256, 0, s>>>((const TI*)x, w, b, eps, (TO*)out, M); break;
      default: ln_rows_vec_kernel<TI, TO, 512><<<grid, 256, 0, s>>>((const TI*)x, w, b, eps, (TO*)out, M); break;
    }
    return pf::check_launch("ln_rows");
  }
  ln_rows_kernel<TI, TO><<<(unsigned)((M + 3) / 4), 256, 0, s>>>((const TI*)x, w, b, eps, (TO*)out, M, C);
  return pf::check_launch("ln_rows");
}

template <class TC, class TO, int EPI>
int rowgemm_launch(const void* A, const void* W, const float* bias, int nbias, void* out, long M, int Nout, int K,
                   hipStream_t s) {
  // Many rows (the pair paths at generic widths): the LDS-tiled GEMM with the same epilogue.
  constexpr int kt = sizeof(TC) == 2 ? 32 : 16;  // tile_gemm_rows' k-tile
  if (M >= kTileGemmMinRows && K % kt == 0 && (bias == nullptr || nbias == 0) && pf::aligned16(A) &&
      pf::aligned16(W))
    return tile_gemm_rows(A, W, out, M, Nout, K, EPI, sizeof(TC) == 2 ? PF_BF16 : PF_F32,
                          sizeof(TO) == 2 ? PF_BF16 : PF_F32, s);
  const long nb64 = ((M + 63) / 64) * ((Nout + 63) / 64);
  if (nb64 < 2L * pf::cu_count()) {  // few row blocks: 32-row tiles, twice the blocks
    dim3 grid((unsigned)((M + 31) / 32), (unsigned)((Nout + 63) / 64));
    rowgemm_kernel<TC, TO, EPI, 2><<<grid, 256, 0, s>>>((const TC*)A, (const TC*)W, bias, nbias, (TO*)out, M, Nout, K);
  } else {
    dim3 grid((unsigned)((M + 63) / 64), (unsigned)((Nout + 63) / 64));
    rowgemm_kernel<TC, TO, EPI, 4><<<grid, 256, 0, s>>>((const TC*)A, (const TC*)W, bias, nbias, (TO*)out, M, Nout, K);
  }
  return pf::check_launch("rowgemm");
}


}  // namespace
