// Row LayerNorm and LayerNorm + transpose (HBM-bound).
//
//   pf_layernorm_fwd:    out[r] = LN(x[r]) over the last dim; fp32 statistics, output in
//                        x's dtype (reference layer_norm, src/deepfold3/model/primitives.py:90-115).
//   pf_ln_transpose_fwd: x [B,N1,N2,C] -> out [B,N2,N1,C] = LN(x).permute(0,2,1,3)
//                        (reference FusedLayerNormTranspose, triton/layernorm_transpose.py:269-316).
//   pf_layernorm_fwd_mixed / pf_layernorm_bwd_mixed: the same with the output (forward) or
//                        the cotangent dy (backward) in a dtype of its own: the autocast training
//                        path's LayerNorm of an fp32 stream feeding bf16 GEMMs, without the casts.
//
// C = 128 (the pair representation): 16 lanes per row, 16 rows per wave (layernorm128_kernel).
// Other C: one wave per row; each lane owns C/128 chunks of two channels, so every load
// instruction of a wave reads one 256-byte (bf16) or 512-byte (fp32) contiguous run.
#include <type_traits>

#include "capi.h"
#include "common.h"
#include "rowops.h"

namespace {

template <class T>
struct Pair;
template <>
struct Pair<float> {
  using V = __attribute__((__vector_size__(2 * sizeof(float)))) float;
};
template <>
struct Pair<bf16> {
  using V = __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16;
};

// rows_per_wave rows per wave, each row C channels (C % 128 == 0).
template <class T, int C, class TY = T>
__global__ __launch_bounds__(256) void layernorm_rows_kernel(const T* __restrict__ x, const float* __restrict__ w,
                                                             const float* __restrict__ b, float eps,
                                                             TY* __restrict__ out, long M, int N1, int N2,
                                                             int transpose) {
  using V2 = typename Pair<T>::V;
  using VY = typename Pair<TY>::V;
  constexpr int CH = C / 128;  // two-channel chunks per lane
  const int l = lane_id();
  const long row = (long)blockIdx.x * 4 + wave_id();
  if (row >= M) return;
  const T* src = x + row * C;
  float v[CH][2];
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    V2 p = *reinterpret_cast<const V2*>(src + c * 128 + 2 * l);
    v[c][0] = to_f32(p[0]);
    v[c][1] = to_f32(p[1]);
    s += v[c][0] + v[c][1];
  }
  const float mean = group_sum<64>(s) * (1.0f / C);
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const float d0 = v[c][0] - mean, d1 = v[c][1] - mean;
    q += d0 * d0 + d1 * d1;
  }
  const float rstd = rsqrtf(group_sum<64>(q) * (1.0f / C) + eps);
  long orow = row;
  if (transpose) {
    // row = (bb * N1 + i) * N2 + j  ->  (bb * N2 + j) * N1 + i
    const long j = row % N2;
    const long t = row / N2;
    const long i = t % N1;
    const long bb = t / N1;
    orow = (bb * N2 + j) * N1 + i;
  }
  TY* dst = out + orow * C;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = c * 128 + 2 * l;
    VY o;
    o[0] = from_f32<TY>((v[c][0] - mean) * rstd * w[ch] + b[ch]);
    o[1] = from_f32<TY>((v[c][1] - mean) * rstd * w[ch + 1] + b[ch + 1]);
    *reinterpret_cast<VY*>(dst + ch) = o;
  }
}

// C = 128: 16 lanes per row, each owning 8 consecutive channels (one 16-byte load for
// bf16, two for fp32), four rows per wave instruction and 16 rows per wave, with all of a
// lane's loads issued before the first reduction (64 bytes in flight per lane for bf16
// where the one-wave-per-row kernel has 4). Row statistics are two-pass fp32 sums over the
// 16 lanes (DPP within the row of 16 lanes). Each output row is one contiguous 256- or
// 512-byte store, whether or not it is transposed.
template <class T, class TY = T>
__global__ __launch_bounds__(256) void layernorm128_kernel(const T* __restrict__ x, const float* __restrict__ w,
                                                           const float* __restrict__ b, float eps,
                                                           TY* __restrict__ out, long M, int N1, int N2,
                                                           int transpose) {
  constexpr int C = 128;
  constexpr int R = 4;                     // rows per lane group
  constexpr int LPR = 16;                  // lanes per row
  constexpr int VL = 16 / sizeof(T);       // channels per 16-byte load
  constexpr int NL = 8 / VL;               // loads per lane per row
  constexpr int VY = 16 / sizeof(TY);      // channels per 16-byte store
  const int l = lane_id();
  const int grp = l / LPR, q = l % LPR;
  const long row0 = ((long)blockIdx.x * 4 + wave_id()) * (R * 64 / LPR);
  float wv[8], bv[8];
#pragma unroll
  for (int e = 0; e < 8; e += 4) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(w + 8 * q + e);
    const f32x4 c = *reinterpret_cast<const f32x4*>(b + 8 * q + e);
#pragma unroll
    for (int k = 0; k < 4; ++k) wv[e + k] = a[k], bv[e + k] = c[k];
  }
  float v[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const long row = min(row0 + 4 * r + grp, M - 1);  // rows past M recompute row M - 1, unstored
#pragma unroll
    for (int h = 0; h < NL; ++h) {
      float t[VL];
      load16<T>(x + row * C + 8 * q + VL * h, t);
#pragma unroll
      for (int e = 0; e < VL; ++e) v[r][VL * h + e] = t[e];
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const long row = row0 + 4 * r + grp;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += v[r][e];
    const float mean = row_group_sum<LPR>(s) * (1.0f / C);
    float qs = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = v[r][e] - mean;
      qs += d * d;
    }
    const float rstd = rsqrtf(row_group_sum<LPR>(qs) * (1.0f / C) + eps);
    if (row >= M) continue;
    long orow = row;
    if (transpose) {  // (bb N1 + i) N2 + j -> (bb N2 + j) N1 + i
      const long j = row % N2, t = row / N2;
      orow = ((t / N1) * N2 + j) * N1 + t % N1;
    }
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (v[r][e] - mean) * rstd * wv[e] + bv[e];
#pragma unroll
    for (int h = 0; h < 8 / VY; ++h) store_vec<TY, VY>(out + orow * C + 8 * q + VY * h, o + VY * h);
  }
}

// ------------------------------------------------------------------ backward
// One wave per row, kLnbRows rows per block; each lane owns C / 64 consecutive channels.
// dx = rstd (g - mean(g) - xn mean(g xn)) with g = dy * w and xn the standardised x
// (statistics recomputed, fp32 two-pass as the forward); per-block partial sums of
// dy * xn (weight) and dy (bias), added in block order by ln_param_grad_reduce.
constexpr int kLnbRows = 64;

template <class T, int C, class TD = T>
__global__ __launch_bounds__(256) void layernorm_bwd_kernel(const T* __restrict__ x, const TD* __restrict__ dy,
                                                            const float* __restrict__ w, float eps, long M,
                                                            T* __restrict__ dx, float* __restrict__ partial) {
  constexpr int CPL = C / 64;  // channels per lane
  __shared__ float red[4][2 * C];
  const int wv = wave_id();
  const int l = lane_id();
  float wl[CPL], sw[CPL], sb[CPL];
#pragma unroll
  for (int e = 0; e < CPL; ++e) {
    wl[e] = w[l * CPL + e];
    sw[e] = sb[e] = 0.f;
  }
  for (int rr = wv; rr < kLnbRows; rr += 4) {
    const long r = (long)blockIdx.x * kLnbRows + rr;
    if (r >= M) break;
    float xv[CPL], gv[CPL], dv[CPL];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      xv[e] = to_f32(x[r * C + l * CPL + e]);
      dv[e] = to_f32(dy[r * C + l * CPL + e]);
      s += xv[e];
    }
    const float mean = group_sum<64>(s) * (1.0f / C);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      const float d = xv[e] - mean;
      q += d * d;
    }
    const float rstd = rsqrtf(group_sum<64>(q) * (1.0f / C) + eps);
    float sg = 0.f, sgx = 0.f;
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      xv[e] = (xv[e] - mean) * rstd;  // xn
      gv[e] = dv[e] * wl[e];
      sg += gv[e];
      sgx += gv[e] * xv[e];
      sw[e] += dv[e] * xv[e];
      sb[e] += dv[e];
    }
    sg = group_sum<64>(sg) * (1.0f / C);
    sgx = group_sum<64>(sgx) * (1.0f / C);
#pragma unroll
    for (int e = 0; e < CPL; ++e) dx[r * C + l * CPL + e] = from_f32<T>(rstd * (gv[e] - sg - xv[e] * sgx));
  }
#pragma unroll
  for (int e = 0; e < CPL; ++e) {
    red[wv][l * CPL + e] = sw[e];
    red[wv][C + l * CPL + e] = sb[e];
  }
  __syncthreads();
  for (int k = threadIdx.x; k < 2 * C; k += 256)
    partial[(size_t)blockIdx.x * 2 * C + k] = red[0][k] + red[1][k] + red[2][k] + red[3][k];
}

// out[k] = sum over blocks of partial[blk][k] (k < 2C: weight then bias), in block order.
__global__ __launch_bounds__(256) void ln_param_grad_reduce_kernel(const float* __restrict__ partial, long nblk,
                                                                   int C, float* __restrict__ dw,
                                                                   float* __restrict__ db) {
  __shared__ float red[256];
  const int k = blockIdx.x;
  float s = 0.f;
  for (long blk = threadIdx.x; blk < nblk; blk += 256) s += partial[blk * 2 * C + k];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (k < C)
      dw[k] = red[0];
    else
      db[k - C] = red[0];
  }
}

template <class T, class TD = T>
int ln_bwd_launch(const void* x, const void* dy, const float* w, float eps, long M, int C, void* dx, float* dw,
                  float* db, void* ws, hipStream_t s) {
  const long nblk = (M + kLnbRows - 1) / kLnbRows;
  float* partial = static_cast<float*>(ws);
  auto run = [&](auto cc) {
    constexpr int CC = decltype(cc)::value;
    layernorm_bwd_kernel<T, CC, TD><<<(unsigned)nblk, 256, 0, s>>>((const T*)x, (const TD*)dy, w, eps, M, (T*)dx,
                                                                    partial);
  };
  switch (C) {
    case 64: run(std::integral_constant<int, 64>{}); break;
    case 128: run(std::integral_constant<int, 128>{}); break;
    case 256: run(std::integral_constant<int, 256>{}); break;
    case 384: run(std::integral_constant<int, 384>{}); break;
    default: run(std::integral_constant<int, 512>{}); break;
  }
  if (int e = pf::check_launch("layernorm_bwd")) return e;
  ln_param_grad_reduce_kernel<<<2 * C, 256, 0, s>>>(partial, nblk, C, dw, db);
  return pf::check_launch("ln_param_grad_reduce");
}

template <class T, class TY = T>
int ln_dispatch(const void* x, const float* w, const float* b, float eps, void* out, long M, int C, int N1, int N2,
                int transpose, hipStream_t s) {
  dim3 grid((unsigned)((M + 3) / 4));
  pf::KernelTimer timer(transpose ? "ln_transpose" : "layernorm", s);
  switch (C) {
    case 128:
      layernorm128_kernel<T, TY><<<dim3((unsigned)((M + 63) / 64)), 256, 0, s>>>((const T*)x, w, b, eps, (TY*)out, M,
                                                                                N1, N2, transpose);
      break;
    case 256:
      layernorm_rows_kernel<T, 256, TY><<<grid, 256, 0, s>>>((const T*)x, w, b, eps, (TY*)out, M, N1, N2, transpose);
      break;
    case 384:
      layernorm_rows_kernel<T, 384, TY><<<grid, 256, 0, s>>>((const T*)x, w, b, eps, (TY*)out, M, N1, N2, transpose);
      break;
    case 512:
      layernorm_rows_kernel<T, 512, TY><<<grid, 256, 0, s>>>((const T*)x, w, b, eps, (TY*)out, M, N1, N2, transpose);
      break;
    default:
      if (!transpose && C > 0) return ln_launch<T, TY>(x, w, b, eps, out, M, C, s);  // any other width: wave per row
      pf::set_error(PF_ERR_UNSUPPORTED, "layernorm + transpose: C=%d (built: 128, 256, 384, 512)", C);
      return PF_ERR_UNSUPPORTED;
  }
  timer.stop();
  return pf::check_launch("layernorm");
}

}  // namespace

// out[m] = res[m] + scale * x[m] / sqrt(mean_c x[m][c]^2 + eps): the RMSNorm branch scaler
// (non-learnable unit-RMS rows) and the residual add in one pass; one wave per row, fp32
// arithmetic, one rounding to the residual's dtype. out may alias res or x (each element is read
// and written by the same lane).
template <class TR, class TX>
__global__ __launch_bounds__(256) void rms_residual_add_kernel(const TR* res, const TX* x, TR* out,
                                                               long M, int C, float scale, float eps) {
  const long row = (long)blockIdx.x * 4 + wave_id();
  if (row >= M) return;
  const int l = lane_id();
  const TX* xr = x + row * C;
  float q = 0.f;
  for (int c = l; c < C; c += 64) {
    const float v = to_f32(xr[c]);
    q += v * v;
  }
  const float r = scale * rsqrtf(group_sum<64>(q) / C + eps);
  TR* o = out + row * C;
  if (res == nullptr) {
    for (int c = l; c < C; c += 64) o[c] = from_f32<TR>(to_f32(xr[c]) * r);
    return;
  }
  const TR* rr = res + row * C;
  for (int c = l; c < C; c += 64) o[c] = from_f32<TR>(to_f32(rr[c]) + to_f32(xr[c]) * r);
}

extern "C" {

int pf_rms_residual_add(const void* res, int res_dtype, const void* x, int x_dtype, void* out, long M, int C,
                        float scale, float eps, void* stream) {
  PF_REQUIRE(x && out, PF_ERR_INVALID_ARG, "pf_rms_residual_add: null pointer");
  PF_REQUIRE(M >= 0 && C > 0, PF_ERR_INVALID_ARG, "pf_rms_residual_add: M=%ld C=%d", M, C);
  PF_REQUIRE((res_dtype == PF_F32 || res_dtype == PF_BF16) && (x_dtype == PF_F32 || x_dtype == PF_BF16),
             PF_ERR_UNSUPPORTED, "pf_rms_residual_add: dtypes (%d, %d)", res_dtype, x_dtype);
  if (M == 0) return pf::ok();
  hipStream_t s = pf::as_stream(stream);
  const unsigned grid = (unsigned)((M + 3) / 4);
  if (res_dtype == PF_F32 && x_dtype == PF_F32)
    rms_residual_add_kernel<float, float><<<grid, 256, 0, s>>>((const float*)res, (const float*)x, (float*)out, M, C,
                                                               scale, eps);
  else if (res_dtype == PF_F32)
    rms_residual_add_kernel<float, bf16><<<grid, 256, 0, s>>>((const float*)res, (const bf16*)x, (float*)out, M, C,
                                                              scale, eps);
  else if (x_dtype == PF_F32)
    rms_residual_add_kernel<bf16, float><<<grid, 256, 0, s>>>((const bf16*)res, (const float*)x, (bf16*)out, M, C,
                                                              scale, eps);
  else
    rms_residual_add_kernel<bf16, bf16><<<grid, 256, 0, s>>>((const bf16*)res, (const bf16*)x, (bf16*)out, M, C,
                                                             scale, eps);
  return pf::check_launch("pf_rms_residual_add");
}

int pf_layernorm_fwd(const void* x, int dtype, const float* w, const float* b, float eps, void* out, long M, int C,
                     void* stream) {
  PF_REQUIRE(x && w && b && out, PF_ERR_INVALID_ARG, "pf_layernorm_fwd: null pointer");
  PF_REQUIRE(M >= 0, PF_ERR_INVALID_ARG, "pf_layernorm_fwd: M=%ld", M);
  PF_REQUIRE(dtype == PF_F32 || dtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_layernorm_fwd: dtype %d", dtype);
  if (M == 0) return pf::ok();
  hipStream_t s = pf::as_stream(stream);
  if (dtype == PF_F32) return ln_dispatch<float>(x, w, b, eps, out, M, C, 1, 1, 0, s);
  return ln_dispatch<bf16>(x, w, b, eps, out, M, C, 1, 1, 0, s);
}

int pf_ln_transpose_fwd(const void* x, int dtype, const float* w, const float* b, float eps, void* out, int B, int N1,
                        int N2, int C, int do_transpose, void* stream) {
  PF_REQUIRE(x && w && b && out, PF_ERR_INVALID_ARG, "pf_ln_transpose_fwd: null pointer");
  PF_REQUIRE(B >= 0 && N1 >= 0 && N2 >= 0, PF_ERR_INVALID_ARG, "pf_ln_transpose_fwd: bad shape");
  PF_REQUIRE(dtype == PF_F32 || dtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_ln_transpose_fwd: dtype %d", dtype);
  PF_REQUIRE(x != out || !do_transpose, PF_ERR_INVALID_ARG, "pf_ln_transpose_fwd: cannot transpose in place");
  const long M = (long)B * N1 * N2;
  if (M == 0) return pf::ok();
  hipStream_t s = pf::as_stream(stream);
  if (dtype == PF_F32) return ln_dispatch<float>(x, w, b, eps, out, M, C, N1, N2, do_transpose, s);
  return ln_dispatch<bf16>(x, w, b, eps, out, M, C, N1, N2, do_transpose, s);
}

size_t pf_layernorm_bwd_workspace_bytes(long M, int C) {
  if (M <= 0 || C <= 0) return 0;
  return (size_t)((M + kLnbRows - 1) / kLnbRows) * 2 * C * sizeof(float);
}

int pf_layernorm_bwd(const void* x, const void* dy, int dtype, const float* w, float eps, void* dx, float* dw,
                     float* db, long M, int C, void* workspace, size_t workspace_bytes, void* stream) {
  PF_REQUIRE(x && dy && w && dx && dw && db, PF_ERR_INVALID_ARG, "pf_layernorm_bwd: null pointer");
  PF_REQUIRE(M > 0, PF_ERR_INVALID_ARG, "pf_layernorm_bwd: M=%ld", M);
  PF_REQUIRE(C == 64 || C == 128 || C == 256 || C == 384 || C == 512, PF_ERR_UNSUPPORTED,
             "pf_layernorm_bwd: C=%d (built: 64, 128, 256, 384, 512)", C);
  PF_REQUIRE(dtype == PF_F32 || dtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_layernorm_bwd: dtype %d", dtype);
  PF_REQUIRE(workspace && workspace_bytes >= pf_layernorm_bwd_workspace_bytes(M, C), PF_ERR_WORKSPACE,
             "pf_layernorm_bwd: workspace %zu < %zu bytes", workspace_bytes, pf_layernorm_bwd_workspace_bytes(M, C));
  hipStream_t s = pf::as_stream(stream);
  if (dtype == PF_F32) return ln_bwd_launch<float>(x, dy, w, eps, M, C, dx, dw, db, workspace, s);
  return ln_bwd_launch<bf16>(x, dy, w, eps, M, C, dx, dw, db, workspace, s);
}

int pf_layernorm_fwd_mixed(const void* x, int xdtype, const float* w, const float* b, float eps, void* out,
                           int odtype, long M, int C, void* stream) {
  PF_REQUIRE(x && w && b && out, PF_ERR_INVALID_ARG, "pf_layernorm_fwd_mixed: null pointer");
  PF_REQUIRE(M >= 0, PF_ERR_INVALID_ARG, "pf_layernorm_fwd_mixed: M=%ld", M);
  PF_REQUIRE((xdtype == PF_F32 || xdtype == PF_BF16) && (odtype == PF_F32 || odtype == PF_BF16), PF_ERR_UNSUPPORTED,
             "pf_layernorm_fwd_mixed: dtypes %d -> %d", xdtype, odtype);
  if (M == 0) return pf::ok();
  hipStream_t s = pf::as_stream(stream);
  if (xdtype == PF_F32)
    return odtype == PF_F32 ? ln_dispatch<float, float>(x, w, b, eps, out, M, C, 1, 1, 0, s)
                            : ln_dispatch<float, bf16>(x, w, b, eps, out, M, C, 1, 1, 0, s);
  return odtype == PF_F32 ? ln_dispatch<bf16, float>(x, w, b, eps, out, M, C, 1, 1, 0, s)
                          : ln_dispatch<bf16, bf16>(x, w, b, eps, out, M, C, 1, 1, 0, s);
}

int pf_layernorm_bwd_mixed(const void* x, int xdtype, const void* dy, int dydtype, const float* w, float eps,
                           void* dx, float* dw, float* db, long M, int C, void* workspace, size_t workspace_bytes,
                           void* stream) {
  PF_REQUIRE(x && dy && w && dx && dw && db, PF_ERR_INVALID_ARG, "pf_layernorm_bwd_mixed: null pointer");
  PF_REQUIRE(M > 0, PF_ERR_INVALID_ARG, "pf_layernorm_bwd_mixed: M=%ld", M);
  PF_REQUIRE(C == 64 || C == 128 || C == 256 || C == 384 || C == 512, PF_ERR_UNSUPPORTED,
             "pf_layernorm_bwd_mixed: C=%d (built: 64, 128, 256, 384, 512)", C);
  PF_REQUIRE((xdtype == PF_F32 || xdtype == PF_BF16) && (dydtype == PF_F32 || dydtype == PF_BF16), PF_ERR_UNSUPPORTED,
             "pf_layernorm_bwd_mixed: dtypes x %d dy %d", xdtype, dydtype);
  PF_REQUIRE(workspace && workspace_bytes >= pf_layernorm_bwd_workspace_bytes(M, C), PF_ERR_WORKSPACE,
             "pf_layernorm_bwd_mixed: workspace %zu < %zu bytes", workspace_bytes,
             pf_layernorm_bwd_workspace_bytes(M, C));
  hipStream_t s = pf::as_stream(stream);
  if (xdtype == PF_F32)
    return dydtype == PF_F32 ? ln_bwd_launch<float, float>(x, dy, w, eps, M, C, dx, dw, db, workspace, s)
                             : ln_bwd_launch<float, bf16>(x, dy, w, eps, M, C, dx, dw, db, workspace, s);
  return dydtype == PF_F32 ? ln_bwd_launch<bf16, float>(x, dy, w, eps, M, C, dx, dw, db, workspace, s)
                           : ln_bwd_launch<bf16, bf16>(x, dy, w, eps, M, C, dx, dw, db, workspace, s);
}

}  // extern "C"
