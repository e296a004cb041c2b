// Shared device helpers for the PairFormer HIP kernels (gfx950 / CDNA4 only).
//
// Element types: activations are float or __bf16 ("TZ"); GEMM operands are
// float or __bf16 ("TC"). bf16 operands run on v_mfma_f32_16x16x32_bf16 /
// v_mfma_f32_32x32x16_bf16, fp32 operands on v_mfma_f32_16x16x4f32 /
// v_mfma_f32_32x32x2f32; all accumulate in fp32.
//
// Fragment convention: every lane owns 16 bytes of an operand (8 bf16 or
// 4 fp32). For the 16x16 tiles, lane l holds row/column (l & 15) and the KPL
// consecutive k values starting at (l >> 4) * KPL; for the 32x32 tiles, row
// (l & 31) and k from (l >> 5) * KPL. An fp32 fragment of 4 values feeds four
// k=4 (or k=2) MFMAs, one per element, so the k order inside a fragment is a
// permutation of the textbook one; A and B are always loaded with the same
// convention, so the contraction is unchanged.
//
// Accumulator layout (CDNA): 16x16 -> lane l holds column (l & 15), rows
// 4*(l>>4) + r, r = 0..3. 32x32 -> lane l holds column (l & 31), rows
// 8*(r>>2) + 4*(l>>5) + (r&3), r = 0..15.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;

#define PF_DEVICE __device__ __forceinline__

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- conversions
PF_DEVICE float to_f32(float x) { return x; }
PF_DEVICE float to_f32(bf16 x) { return (float)x; }
template <class T>
PF_DEVICE T from_f32(float x);
template <>
PF_DEVICE float from_f32<float>(float x) { return x; }
template <>
PF_DEVICE bf16 from_f32<bf16>(float x) { return (bf16)x; }

// 16-byte vector of T as an array of floats.
template <class T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
};

template <class T>
PF_DEVICE void load16(const T* p, float (&out)[16 / sizeof(T)]);
template <>
PF_DEVICE void load16<float>(const float* p, float (&out)[4]) {
  f32x4 v = *reinterpret_cast<const f32x4*>(p);
  out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
}
template <>
PF_DEVICE void load16<bf16>(const bf16* p, float (&out)[8]) {
  bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (float)v[e];
}

// 16 raw bytes (as loaded) -> floats.
template <class T>
PF_DEVICE void unpack16(const u32x4& r, float (&out)[16 / sizeof(T)]);
template <>
PF_DEVICE void unpack16<float>(const u32x4& r, float (&out)[4]) {
  const f32x4 v = __builtin_bit_cast(f32x4, r);
  out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
}
template <>
PF_DEVICE void unpack16<bf16>(const u32x4& r, float (&out)[8]) {
  const bf16x8 v = __builtin_bit_cast(bf16x8, r);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (float)v[e];
}

// Store VEC floats (VEC * sizeof(T) bytes: 4, 8 or 16) as T.
template <class T, int VEC>
PF_DEVICE void store_vec(T* p, const float* v) {
#pragma unroll
  for (int e = 0; e < VEC; ++e) p[e] = from_f32<T>(v[e]);
}
template <>
PF_DEVICE void store_vec<bf16, 8>(bf16* p, const float* v) {
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (bf16)v[e];
  *reinterpret_cast<bf16x8*>(p) = o;
}
template <>
PF_DEVICE void store_vec<bf16, 4>(bf16* p, const float* v) {
  bf16x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = (bf16)v[e];
  *reinterpret_cast<bf16x4*>(p) = o;
}
template <>
PF_DEVICE void store_vec<float, 4>(float* p, const float* v) {
  f32x4 o = {v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4*>(p) = o;
}

// ---------------------------------------------------------------- math
PF_DEVICE float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
PF_DEVICE float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
PF_DEVICE float sigmoidf_(float x) { return fast_rcp(1.0f + fast_exp(-x)); }
PF_DEVICE float siluf_(float x) { return x * sigmoidf_(x); }

// Sum over aligned groups of W lanes (W a power of two <= 64).
template <int W>
PF_DEVICE float group_sum(float v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <int W>
PF_DEVICE float group_max(float v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Row-local DPP move of a float (bound_ctrl off, all rows and banks).
template <int CTRL>
PF_DEVICE float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
// Sums over aligned groups of 8 / 16 lanes with DPP moves (no LDS round trip): quad_perm
// [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror (8), then row_mirror (16) -- after each
// step every lane holds the sum over twice as many lanes.
PF_DEVICE float dpp_sum8(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  return v;
}
PF_DEVICE float dpp_sum16(float v) {
  v = dpp_sum8(v);
  v += dpp_mov<0x140>(v);
  return v;
}
// Sum over aligned groups of W lanes, W in {16, 32}: DPP inside rows, one swizzle across.
template <int W>
PF_DEVICE float row_group_sum(float v) {
  static_assert(W == 16 || W == 32, "row groups of 16 or 32 lanes");
  v = dpp_sum16(v);
  if (W == 32) v += __shfl_xor(v, 16, 64);
  return v;
}

// v_permlane32_swap: lanes 32..63 of a trade values with lanes 0..31 of b. Inline assembly
// with both operands read-write (the compiler builtin returned wrong lanes once unrolled).
// The compiler cannot see hazards through inline assembly, so the operands first pass
// through an ordinary VALU add: the compiler gives that add the wait states an MFMA result
// needs before a VALU read, and the s_nop covers the VALU-write -> cross-lane-read hazard.
// (x + 0 turns -0 into +0; nothing downstream distinguishes them.)
PF_DEVICE void permlane32_swap(float& a, float& b) {
  a += 0.0f;
  b += 0.0f;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

PF_DEVICE int lane_id() { return threadIdx.x & 63; }
// Wave index inside the block, as a wave-uniform (scalar) value.
PF_DEVICE int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// ---------------------------------------------------------------- MFMA
template <class TC>
struct Mfma;

template <>
struct Mfma<bf16> {
  using Frag = bf16x8;
  static constexpr int KPL = 8;        // k values per lane per fragment
  static constexpr int K16 = 32;       // k covered by one 16x16 fragment step
  static constexpr int K32 = 16;       // k covered by one 32x32 fragment step
  PF_DEVICE static void mma16(f32x4& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  PF_DEVICE static void mma32(f32x16& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
  }
  PF_DEVICE static Frag load(const bf16* p) { return *reinterpret_cast<const Frag*>(p); }
  PF_DEVICE static Frag from_floats(const float* v) {
    Frag f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (bf16)v[e];
    return f;
  }
};

template <>
struct Mfma<float> {
  using Frag = f32x4;
  static constexpr int KPL = 4;
  static constexpr int K16 = 16;
  static constexpr int K32 = 8;
  PF_DEVICE static void mma16(f32x4& acc, const Frag& a, const Frag& b) {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], acc, 0, 0, 0);
  }
  PF_DEVICE static void mma32(f32x16& acc, const Frag& a, const Frag& b) {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], b[e], acc, 0, 0, 0);
  }
  PF_DEVICE static Frag load(const float* p) { return *reinterpret_cast<const Frag*>(p); }
  PF_DEVICE static Frag from_floats(const float* v) {
    Frag f = {v[0], v[1], v[2], v[3]};
    return f;
  }
};

// Row padding (elements) for LDS operand tiles: 16 bytes.
template <class T>
constexpr int lds_pad() { return 16 / sizeof(T); }

// acc[rb][cb] += A[rb*16 .. +16][0..K) * W[wrow(cb) .. +16][0..K)^T
// A: LDS tile, row stride lda (elements). W: global weight rows, k contiguous,
// row stride ldw; col block cb starts at weight row wrow0[cb].
template <class TC, int K, int RB, int CB>
PF_DEVICE void gemm16_lds_x_w(f32x4 (&acc)[RB][CB], const TC* A, int lda, int arow0, const TC* W, int ldw,
                              const int (&wrow0)[CB]) {
  using M = Mfma<TC>;
  const int l = lane_id();
  const int r = l & 15;
  const int kq = (l >> 4) * M::KPL;
#pragma unroll 2
  for (int k0 = 0; k0 < K; k0 += M::K16) {
    typename M::Frag bf[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c) bf[c] = M::load(W + (size_t)(wrow0[c] + r) * ldw + k0 + kq);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      typename M::Frag af = M::load(A + (arow0 + rb * 16 + r) * lda + k0 + kq);
#pragma unroll
      for (int c = 0; c < CB; ++c) M::mma16(acc[rb][c], af, bf[c]);
    }
  }
}

template <int RB, int CB>
PF_DEVICE void zero_acc(f32x4 (&acc)[RB][CB]) {
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// ---------------------------------------------------------------- LayerNorm tile
// LayerNorm BM positions of C channels each and write them (as TC) into an LDS
// tile lds[p * lda + c]. rowptr(p) returns the position's first element, or
// nullptr for a padding position (written as zeros). Statistics are fp32 and
// two-pass (mean, then mean of squared deviations), eps inside the rsqrt, as
// torch.nn.functional.layer_norm. NT threads take part.
template <class TZ, class TC, int C, int BM, int NT, class RowFn>
PF_DEVICE void ln_tile_to_lds(RowFn rowptr, const float* __restrict__ w, const float* __restrict__ b, float eps,
                              TC* lds, int lda) {
  constexpr int VEC = 16 / sizeof(TZ);
  constexpr int LPP = C / VEC;  // lanes per position
  static_assert(C % VEC == 0 && 64 % LPP == 0, "channel count must tile a wave");
  constexpr int PPI = NT / LPP;
  static_assert(BM % PPI == 0, "tile rows must be a multiple of positions per pass");
  const int tid = threadIdx.x;
  const int sub = tid % LPP;
  const int pp = tid / LPP;
  float wv[VEC], bv[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    wv[e] = w[sub * VEC + e];
    bv[e] = b[sub * VEC + e];
  }
#pragma unroll
  for (int p0 = 0; p0 < BM; p0 += PPI) {
    const int p = p0 + pp;
    const TZ* src = rowptr(p);
    float x[VEC];
    if (src) {
      load16<TZ>(src + sub * VEC, x);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[e] = 0.f;
    }
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) s += x[e];
    const float mean = group_sum<LPP>(s) * (1.0f / C);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float d = x[e] - mean;
      q += d * d;
    }
    const float rstd = rsqrtf(group_sum<LPP>(q) * (1.0f / C) + eps);
    float y[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) y[e] = src ? (x[e] - mean) * rstd * wv[e] + bv[e] : 0.f;
    store_vec<TC, VEC>(lds + p * lda + sub * VEC, y);
  }
}

// Copy BM rows of C TZ elements into an LDS tile as TC without normalising.
template <class TZ, class TC, int C, int BM, int NT, class RowFn>
PF_DEVICE void copy_tile_to_lds(RowFn rowptr, TC* lds, int lda) {
  constexpr int VEC = 16 / sizeof(TZ);
  constexpr int LPP = C / VEC;
  constexpr int PPI = NT / LPP;
  const int tid = threadIdx.x;
  const int sub = tid % LPP;
  const int pp = tid / LPP;
#pragma unroll
  for (int p0 = 0; p0 < BM; p0 += PPI) {
    const int p = p0 + pp;
    const TZ* src = rowptr(p);
    float x[VEC];
    if (src) {
      load16<TZ>(src + sub * VEC, x);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[e] = 0.f;
    }
    store_vec<TC, VEC>(lds + p * lda + sub * VEC, x);
  }
}

// dst(p)[c] = (accumulate ? dst(p)[c] : 0) + stage[p * lds_ld + c] for BM positions of
// C channels; stage holds fp32. rowptr(p) returns nullptr for positions to skip.
template <class TZ, int C, int BM, int NT, class RowFn>
PF_DEVICE void store_tile_from_lds(RowFn rowptr, const float* stage, int lds_ld, bool accumulate) {
  constexpr int VEC = 16 / sizeof(TZ);
  constexpr int LPP = C / VEC;
  constexpr int PPI = NT / LPP;
  const int tid = threadIdx.x;
  const int sub = tid % LPP;
  const int pp = tid / LPP;
#pragma unroll
  for (int p0 = 0; p0 < BM; p0 += PPI) {
    const int p = p0 + pp;
    TZ* dst = const_cast<TZ*>(rowptr(p));
    if (!dst) continue;
    float x[VEC];
    if (accumulate) {
      load16<TZ>(dst + sub * VEC, x);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) x[e] += stage[p * lds_ld + sub * VEC + e];
    store_vec<TZ, VEC>(dst + sub * VEC, x);
  }
}

// ---------------------------------------------------------------- 32x32 block tiles
// Block GEMMs for the K = 128 contractions of the pair stack. Operands sit in LDS with
// k contiguous and rows padded by 16 bytes; a wave computes 32x32 MFMA tiles, lane l
// holding row (l & 31) and the KPL k values from (l >> 5) * KPL of each fragment.

// Rows of positions per block tile: 128 with bf16 operands, 64 with fp32 (LDS budget).
template <class TC>
constexpr int block_rows() { return sizeof(TC) == 2 ? 128 : 64; }

// LDS row stride (elements) of a 128-wide operand tile.
template <class TC>
constexpr int ld128() { return 128 + lds_pad<TC>(); }

// R rows x 128 TC elements, global row stride ldg, staged through registers so the
// global loads can be issued early (load) and written to LDS later (store).
template <class TC, int R, int NT>
struct Rows128 {
  static constexpr int VEC = 16 / sizeof(TC);
  static constexpr int CPR = 128 / VEC;
  static constexpr int IT = R * CPR / NT;
  static_assert((R * CPR) % NT == 0, "tile must split evenly over the block");
  u32x4 v[IT];
  PF_DEVICE void load(const TC* __restrict__ g, long ldg) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int idx = (int)threadIdx.x + it * NT;
      v[it] = *reinterpret_cast<const u32x4*>(g + (long)(idx / CPR) * ldg + (idx % CPR) * VEC);
    }
  }
  PF_DEVICE void store(TC* lds, int ld) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int idx = (int)threadIdx.x + it * NT;
      *reinterpret_cast<u32x4*>(lds + (idx / CPR) * ld + (idx % CPR) * VEC) = v[it];
    }
  }
};

// acc[i][j] += A[arow0 + 32 i + .][0, K) * B[brow0 + 32 j + .][0, K)^T, A and B in LDS.
template <class TC, int MI, int NJ, int K>
PF_DEVICE void wave_mma32(f32x16 (&acc)[MI][NJ], const TC* A, int lda, int arow0, const TC* B, int ldb, int brow0) {
  using M = Mfma<TC>;
  const int l = lane_id();
  const int r = l & 31;
  const int kq = (l >> 5) * M::KPL;
  // Two k-steps in flight: enough to cover LDS latency without hoisting every fragment.
#pragma unroll 2
  for (int kk = 0; kk < K; kk += M::K32) {
    typename M::Frag a[MI], b[NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i) a[i] = M::load(A + (arow0 + 32 * i + r) * lda + kk + kq);
#pragma unroll
    for (int j = 0; j < NJ; ++j) b[j] = M::load(B + (brow0 + 32 * j + r) * ldb + kk + kq);
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) M::mma32(acc[i][j], a[i], b[j]);
  }
}

template <int MI, int NJ>
PF_DEVICE void zero_acc32(f32x16 (&acc)[MI][NJ]) {
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
}

// ---------------------------------------------------------------- buffer loads
// Buffer resource over `bytes` bytes at `p` (raw buffer loads: scalar base, 32-bit offsets;
// out-of-range reads return 0).
PF_DEVICE __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// 16 bytes per lane from a buffer straight into LDS: lane l lands at lds + 16 l (the LDS
// address is taken from the wave's first lane). The host compilation pass cannot type-check
// this builtin; kernels only run on the device.
PF_DEVICE void buf_load_lds16(__amdgpu_buffer_rsrc_t r, void* lds, int voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
#endif
}

// The same load issued through inline assembly, which the compiler does not see as a write
// to LDS: it then inserts no wait for it before later LDS accesses (its conservative
// aliasing would otherwise wait for every direct load in flight before any LDS read, which
// makes a chunk wait for the next chunk's loads before its own fragment reads). The caller
// orders every LDS access to the destination with explicit s_waitcnt vmcnt and barriers.
// `r_words` is the buffer resource as four dwords (buf_rsrc_words). m0 is reserved to the
// compiler, which does not honour the clobber (hence its warning): use this only in kernels
// in which the compiler itself keeps nothing in m0 (no buf_load_lds16 beside it); in the
// assembly of the kernels that use it, m0 is written by these statements only.
typedef int i32x4_t __attribute__((ext_vector_type(4)));
PF_DEVICE i32x4_t buf_rsrc_words(const void* p, unsigned bytes) {
  const unsigned long long a = (unsigned long long)p;
  return i32x4_t{(int)(unsigned)a, (int)(unsigned)(a >> 32) & 0xffff, (int)bytes, 0x00020000};
}
PF_DEVICE void buf_load_lds16_async(const i32x4_t& r_words, void* lds, int voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  const unsigned m0 =
      __builtin_amdgcn_readfirstlane((unsigned)(unsigned long long)(__attribute__((address_space(3))) char*)lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(r_words), "s"(soff)
               : "memory", "m0");
#endif
}

// Workgroup barrier after this wave's LDS operations (s_waitcnt lgkmcnt(0); s_barrier),
// without waiting for outstanding global or buffer-to-LDS loads (vmcnt), which
// __syncthreads() would. Only for LDS data written by ds_* instructions.
PF_DEVICE void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt at their maxima
  __builtin_amdgcn_s_barrier();
}

// ---------------------------------------------------------------- 16-value fragments
// Key order of a 32-key block in flash-attention operands. With S^T = K Q^T on a 32x32
// MFMA, lane (q, h) (q = lane & 31, h = lane >> 5) holds the logits of query q for keys
// kappa(r, h) = 8 (r >> 2) + 4 h + (r & 3), r = 0..15; storing key kappa(r, h) at slot
// 16 h + r makes those 16 probabilities the lane's B operand of O^T += V^T P^T directly.
PF_DEVICE int slot_key(int slot) { return 8 * ((slot & 15) >> 2) + 4 * (slot >> 4) + (slot & 3); }
PF_DEVICE int key_slot(int key) { return 16 * ((key >> 2) & 1) + 4 * (key >> 3) + (key & 3); }

// Flash-attention operands: a lane holds 16 consecutive k values (k from 16 (lane >> 5)),
// fed to two 32x32x16 bf16 MFMAs (or sixteen 32x32x2 fp32 MFMAs).
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

// max(x[l], x[l ^ 32]) over the wave's two 32-lane halves. v_permlane32_swap of x with
// itself leaves (x[l], x[l + 32]) in the low half and (x[l - 32], x[l]) in the high half:
// a VALU op, no LDS round trip.
PF_DEVICE float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Row (inside a 32x32 tile) of accumulator element e of this lane; its column is lane & 31.
// Elements 4g .. 4g+3 are four consecutive rows.
PF_DEVICE int acc32_row(int e) { return 8 * (e >> 2) + 4 * (lane_id() >> 5) + (e & 3); }

// Two-phase LayerNorm of BM rows: load() issues the global loads (so they can overlap
// other work), store() normalises into an LDS tile with the same math as ln_tile_to_lds.
template <class TZ, class TC, int C, int BM, int NT>
struct LnTile {
  static constexpr int VEC = 16 / sizeof(TZ);
  static constexpr int LPP = C / VEC;
  static constexpr int PPI = NT / LPP;
  static constexpr int PASSES = BM / PPI;
  static_assert(BM % PPI == 0 && 64 % LPP == 0, "tile must split evenly");
  u32x4 raw[PASSES];
  bool ok[PASSES];
  template <class RowFn>
  PF_DEVICE void load(RowFn rowptr) {
    const int sub = threadIdx.x % LPP;
    const int pp = threadIdx.x / LPP;
#pragma unroll
    for (int s = 0; s < PASSES; ++s) {
      const TZ* src = rowptr(s * PPI + pp);
      ok[s] = src != nullptr;
      raw[s] = ok[s] ? *reinterpret_cast<const u32x4*>(src + sub * VEC) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  PF_DEVICE void store(const float* __restrict__ w, const float* __restrict__ b, float eps, TC* lds, int lda) const {
    const int sub = threadIdx.x % LPP;
    const int pp = threadIdx.x / LPP;
    float wv[VEC], bv[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      wv[e] = w[sub * VEC + e];
      bv[e] = b[sub * VEC + e];
    }
#pragma unroll
    for (int s = 0; s < PASSES; ++s) {
      float x[VEC];
      unpack16<TZ>(raw[s], x);
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) sum += x[e];
      const float mean = group_sum<LPP>(sum) * (1.0f / C);
      float q = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float d = x[e] - mean;
        q += d * d;
      }
      const float rstd = rsqrtf(group_sum<LPP>(q) * (1.0f / C) + eps);
      float y[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) y[e] = ok[s] ? (x[e] - mean) * rstd * wv[e] + bv[e] : 0.f;
      store_vec<TC, VEC>(lds + (s * PPI + pp) * lda + sub * VEC, y);
    }
  }
};
