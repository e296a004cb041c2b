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
    dim3 grid((unsigned)((M + 127) / 128));
    if (logits)
      pair_transition32_kernel<TZ, true><<<grid, 512, 0, s>>>((const TZ*)x, (TZ*)out, lnw, lnb, eps, (const bf16*)w1,
                                                             (const bf16*)w2, M, accumulate, s2p_w, s2p_b, s2p_eps,
                                                             (const bf16*)ws2p, logits, NN);
    else
      pair_transition32_kernel<TZ, false><<<grid, 512, 0, s>>>((const TZ*)x, (TZ*)out, lnw, lnb, eps,
                                                              (const bf16*)w1, (const bf16*)w2, M, accumulate,
                                                              nullptr, nullptr, 0.f, nullptr, nullptr, NN);
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
  PF_REQUIRE(C == kC && factor == 4, PF_ERR_UNSUPPORTED,
             "pf_pair_transition_fwd: C=%d factor=%d (built: C=128, factor 4)", C, factor);
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
  PF_REQUIRE(C == kC && H == kS2pHeads, PF_ERR_UNSUPPORTED, "pf_single_to_pair_fwd: C=%d H=%d (built: 128, 16)", C,
             H);
  PF_REQUIRE(NN > 0 && M >= 0 && M % NN == 0, PF_ERR_INVALID_ARG, "pf_single_to_pair_fwd: M=%ld NN=%ld", M, NN);
  PF_REQUIRE((zdtype == PF_F32 || zdtype == PF_BF16) && (cdtype == PF_F32 || cdtype == PF_BF16) &&
                 !(zdtype == PF_BF16 && cdtype == PF_F32),
             PF_ERR_UNSUPPORTED, "pf_single_to_pair_fwd: dtype pair (%d, %d)", zdtype, cdtype);
  if (M == 0) return pf::ok();
  hipStream_t s = pf::as_stream(stream);
  return PF_DISPATCH_ZC(zdtype, cdtype, s2p_launch, z, ln_w, ln_b, eps, w_s2p, pair_logits, M, NN, s);
}

}  // extern "C"
