// Training-mode dropout fused with the residual add, with the mask shared along one axis
// (row- or column-shared, as dropout_add_rowwise / dropout_add_columnwise,
// src/deepfold3/model/triton/dropout_add.py:57-135, :221-265).
//
// For an activation [B, R, Cc, D] (pair: rows, columns, channels; MSA: sequences, residues,
// channels) a row-shared mask has one entry per (b, c, d), index b*Cc*D + c*D + d; a
// column-shared mask one per (b, r, d), index b*R*D + r*D + d. Entry i keeps its element
// when u_i >= p, where u_i is a uniform number in [0, 1) drawn from a counter-based
// generator: Philox4x32 with 10 rounds (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC 2011), key = the 64-bit seed, counter = (i / 4) as a
// 64-bit word in its first two lanes, and u_i = (word i % 4 of the output >> 8) * 2^-24.
// A kept element is scaled by 1 / (1 - p). The mask is never stored: the backward
// regenerates it from the seed. Arithmetic in fp32: out = res + x * m rounded once to the
// residual's dtype (x * m and the add are separate roundings, no fused multiply-add).
//
// Kernels are HBM-bound elementwise passes: each thread takes 4 consecutive channels, whose
// 4 mask entries are the 4 words of one Philox call (D % 4 == 0 keeps them in one call).
#include "capi.h"
#include "common.h"

namespace {

constexpr uint32_t kPhiloxM0 = 0xD2511F53u, kPhiloxM1 = 0xCD9E8D57u;
constexpr uint32_t kPhiloxW0 = 0x9E3779B9u, kPhiloxW1 = 0xBB67AE85u;

PF_DEVICE u32x4 philox4x32_10(uint64_t ctr, uint64_t seed) {
  uint32_t c0 = (uint32_t)ctr, c1 = (uint32_t)(ctr >> 32), c2 = 0u, c3 = 0u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t hi0 = __umulhi(kPhiloxM0, c0), lo0 = kPhiloxM0 * c0;
    const uint32_t hi1 = __umulhi(kPhiloxM1, c2), lo1 = kPhiloxM1 * c2;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
    k0 += kPhiloxW0;
    k1 += kPhiloxW1;
  }
  return u32x4{c0, c1, c2, c3};
}

// The 4 mask values (0 or scale) of entries 4q .. 4q+3.
PF_DEVICE void mask4(uint64_t q, uint64_t seed, float p, float scale, float (&m)[4]) {
  const u32x4 w = philox4x32_10(q, seed);
#pragma unroll
  for (int e = 0; e < 4; ++e) m[e] = (float)(w[e] >> 8) * 0x1.0p-24f >= p ? scale : 0.f;
}

// Mask index (of the first of 4 channels) of element group g (elements 4g .. 4g+3).
PF_DEVICE uint64_t mask_index(uint64_t e, uint64_t R, uint64_t Cc, uint64_t D, bool rowwise) {
  const uint64_t CD = Cc * D, RCD = R * CD;
  const uint64_t b = e / RCD, local = e - b * RCD;
  if (rowwise) return b * CD + local % CD;
  const uint64_t r = local / CD;
  return b * R * D + r * D + local % D;
}

template <class T>
PF_DEVICE void load4(const T* p, float (&v)[4]);
template <>
PF_DEVICE void load4<float>(const float* p, float (&v)[4]) {
  const f32x4 x = *reinterpret_cast<const f32x4*>(p);
  v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
}
template <>
PF_DEVICE void load4<bf16>(const bf16* p, float (&v)[4]) {
  const bf16x4 x = *reinterpret_cast<const bf16x4*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = (float)x[e];
}

// out = res + x * m (out may alias res).
template <class TR, class TX>
__global__ __launch_bounds__(256) void dropout_add_kernel(const TR* res, const TX* __restrict__ x, TR* out,
                                                          uint64_t groups, uint64_t R, uint64_t Cc, uint64_t D,
                                                          int rowwise, float p, float scale, uint64_t seed) {
  for (uint64_t g = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; g < groups;
       g += (uint64_t)gridDim.x * blockDim.x) {
#pragma clang fp contract(off)
    const uint64_t e = 4 * g;
    float m[4], r[4], v[4], o[4];
    mask4(mask_index(e, R, Cc, D, rowwise != 0) >> 2, seed, p, scale, m);
    load4<TR>(res + e, r);
    load4<TX>(x + e, v);
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = r[k] + v[k] * m[k];  // two roundings: contraction is off
    store_vec<TR, 4>(out + e, o);
  }
}

// gx = g * m, in x's dtype.
template <class TG, class TX>
__global__ __launch_bounds__(256) void dropout_bwd_kernel(const TG* __restrict__ g_out, TX* __restrict__ gx,
                                                          uint64_t groups, uint64_t R, uint64_t Cc, uint64_t D,
                                                          int rowwise, float p, float scale, uint64_t seed) {
  for (uint64_t g = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; g < groups;
       g += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t e = 4 * g;
    float m[4], v[4], o[4];
    mask4(mask_index(e, R, Cc, D, rowwise != 0) >> 2, seed, p, scale, m);
    load4<TG>(g_out + e, v);
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = v[k] * m[k];
    store_vec<TX, 4>(gx + e, o);
  }
}

__global__ __launch_bounds__(256) void dropout_mask_kernel(float* __restrict__ mask, uint64_t n, float p,
                                                           float scale, uint64_t seed) {
  for (uint64_t q = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; 4 * q < n;
       q += (uint64_t)gridDim.x * blockDim.x) {
    float m[4];
    mask4(q, seed, p, scale, m);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (4 * q + e < n) mask[4 * q + e] = m[e];
  }
}

unsigned grid_for_groups(uint64_t groups) {
  const uint64_t cap = (uint64_t)pf::cu_count() * 16;  // 16 blocks of 256 per CU, grid-stride
  uint64_t g = (groups + 255) / 256;
  return (unsigned)(g > cap ? cap : (g == 0 ? 1 : g));
}

// 4-element vectors: 16 bytes of fp32 or 8 bytes of bf16.
bool vec_aligned(const void* ptr, int dtype) {
  return ((uintptr_t)ptr & (dtype == PF_F32 ? 15u : 7u)) == 0;
}

int check_shape(const char* fn, long B, long R, long Cc, long D, float p) {
  PF_REQUIRE(B >= 0 && R >= 0 && Cc >= 0 && D > 0, PF_ERR_INVALID_ARG, "%s: negative or zero size", fn);
  PF_REQUIRE(D % 4 == 0, PF_ERR_UNSUPPORTED, "%s: D=%ld must be a multiple of 4", fn, D);
  PF_REQUIRE(p >= 0.f && p < 1.f, PF_ERR_INVALID_ARG, "%s: p=%g must be in [0, 1)", fn, (double)p);
  return PF_OK;
}

}  // namespace

extern "C" {

int pf_dropout_mask(float* mask, long n, float p, unsigned long long seed, void* stream) {
  PF_REQUIRE(mask != nullptr || n == 0, PF_ERR_INVALID_ARG, "pf_dropout_mask: null pointer");
  PF_REQUIRE(n >= 0, PF_ERR_INVALID_ARG, "pf_dropout_mask: n=%ld", n);
  PF_REQUIRE(p >= 0.f && p < 1.f, PF_ERR_INVALID_ARG, "pf_dropout_mask: p=%g must be in [0, 1)", (double)p);
  if (n == 0) return pf::ok();
  const uint64_t groups = ((uint64_t)n + 3) / 4;
  dropout_mask_kernel<<<grid_for_groups(groups), 256, 0, pf::as_stream(stream)>>>(mask, (uint64_t)n, p,
                                                                                  1.0f / (1.0f - p), seed);
  return pf::check_launch("pf_dropout_mask");
}

int pf_dropout_add_fwd(const void* res, int res_dtype, const void* x, int x_dtype, void* out, long B, long R,
                       long Cc, long D, int rowwise, float p, unsigned long long seed, void* stream) {
  const char* fn = "pf_dropout_add_fwd";
  PF_REQUIRE(res && x && out, PF_ERR_INVALID_ARG, "%s: null pointer", fn);
  PF_REQUIRE((res_dtype == PF_F32 || res_dtype == PF_BF16) && (x_dtype == PF_F32 || x_dtype == PF_BF16),
             PF_ERR_UNSUPPORTED, "%s: dtype codes must be PF_F32 or PF_BF16", fn);
  if (int st = check_shape(fn, B, R, Cc, D, p)) return st;
  const uint64_t groups = (uint64_t)B * R * Cc * D / 4;
  if (groups == 0) return pf::ok();
  PF_REQUIRE(vec_aligned(res, res_dtype) && vec_aligned(out, res_dtype) && vec_aligned(x, x_dtype),
             PF_ERR_ALIGNMENT, "%s: fp32 pointers must be 16-byte and bf16 pointers 8-byte aligned", fn);
  const float scale = 1.0f / (1.0f - p);
  hipStream_t s = pf::as_stream(stream);
  const unsigned g = grid_for_groups(groups);
  const uint64_t r = R, c = Cc, d = D;
  if (res_dtype == PF_F32 && x_dtype == PF_F32)
    dropout_add_kernel<float, float><<<g, 256, 0, s>>>((const float*)res, (const float*)x, (float*)out, groups, r,
                                                        c, d, rowwise, p, scale, seed);
  else if (res_dtype == PF_F32)
    dropout_add_kernel<float, bf16><<<g, 256, 0, s>>>((const float*)res, (const bf16*)x, (float*)out, groups, r, c,
                                                       d, rowwise, p, scale, seed);
  else if (x_dtype == PF_F32)
    dropout_add_kernel<bf16, float><<<g, 256, 0, s>>>((const bf16*)res, (const float*)x, (bf16*)out, groups, r, c,
                                                       d, rowwise, p, scale, seed);
  else
    dropout_add_kernel<bf16, bf16><<<g, 256, 0, s>>>((const bf16*)res, (const bf16*)x, (bf16*)out, groups, r, c, d,
                                                      rowwise, p, scale, seed);
  return pf::check_launch(fn);
}

int pf_dropout_bwd(const void* grad_out, int grad_dtype, void* grad_x, int x_dtype, long B, long R, long Cc, long D,
                   int rowwise, float p, unsigned long long seed, void* stream) {
  const char* fn = "pf_dropout_bwd";
  PF_REQUIRE(grad_out && grad_x, PF_ERR_INVALID_ARG, "%s: null pointer", fn);
  PF_REQUIRE((grad_dtype == PF_F32 || grad_dtype == PF_BF16) && (x_dtype == PF_F32 || x_dtype == PF_BF16),
             PF_ERR_UNSUPPORTED, "%s: dtype codes must be PF_F32 or PF_BF16", fn);
  if (int st = check_shape(fn, B, R, Cc, D, p)) return st;
  const uint64_t groups = (uint64_t)B * R * Cc * D / 4;
  if (groups == 0) return pf::ok();
  PF_REQUIRE(vec_aligned(grad_out, grad_dtype) && vec_aligned(grad_x, x_dtype), PF_ERR_ALIGNMENT,
             "%s: fp32 pointers must be 16-byte and bf16 pointers 8-byte aligned", fn);
  const float scale = 1.0f / (1.0f - p);
  hipStream_t s = pf::as_stream(stream);
  const unsigned g = grid_for_groups(groups);
  const uint64_t r = R, c = Cc, d = D;
  if (grad_dtype == PF_F32 && x_dtype == PF_F32)
    dropout_bwd_kernel<float, float><<<g, 256, 0, s>>>((const float*)grad_out, (float*)grad_x, groups, r, c, d,
                                                        rowwise, p, scale, seed);
  else if (grad_dtype == PF_F32)
    dropout_bwd_kernel<float, bf16><<<g, 256, 0, s>>>((const float*)grad_out, (bf16*)grad_x, groups, r, c, d,
                                                       rowwise, p, scale, seed);
  else if (x_dtype == PF_F32)
    dropout_bwd_kernel<bf16, float><<<g, 256, 0, s>>>((const bf16*)grad_out, (float*)grad_x, groups, r, c, d,
                                                       rowwise, p, scale, seed);
  else
    dropout_bwd_kernel<bf16, bf16><<<g, 256, 0, s>>>((const bf16*)grad_out, (bf16*)grad_x, groups, r, c, d,
                                                      rowwise, p, scale, seed);
  return pf::check_launch(fn);
}

}  // extern "C"
