// Single-track kernels (tokens x 384): LayerNorm into the GEMM operand dtype, a row GEMM
// with bias / SwiGLU / residual epilogues, and the attention-with-pair-bias core.
//
//   pf_single_attn_fwd: SingleAttention.forward (src/deepfold3/model/attention.py:415-452):
//     xn = LN(s); q = xn Wq^T + bq; k, v, g = xn W^T; logits = (q d^-1/2) k^T + pair_logits
//     + 1e9 (mask - 1); softmax in fp32; o = w v; out = (o * sigmoid(g)) Wout^T.
//   pf_transition_fwd:  TransitionBlock.forward (primitives.py:193-251) for any C:
//     LN -> W1 (SwiGLU on contiguous halves) -> W2, out = y or out += y.
//
// The single track is ~0.4 % of a PairFormer block's FLOPs. The row GEMMs read their
// operands straight from global memory (they stay in L2); the attention core is a
// flash kernel on 32x32 MFMAs (V transposed once into key-slot order by a pack kernel,
// keys split over the four waves of a block and merged through LDS).
#include <algorithm>
#include <mutex>

#include "capi.h"
#include "common.h"
#include "rowops.h"

namespace {

// ------------------------------------------------------------------ attention core
constexpr int kSHeadDim = 24;

// Flash attention for the single track, head dim 24 padded to 32, on 32x32 MFMAs with the
// same frame as the triangle-attention kernel: a wave owns 32 queries of one (b, h) and
// computes S^T = K Q^T per 32-key block, so lane (q, h) = (lane & 31, lane >> 5) holds the
// logits of query q for the 16 keys kappa(r, h) (key_slot / slot_key), which are the P^T
// operand of O^T += V^T P^T once V^T is stored with keys in slot order.
//
// Pack: Vt [B][H][32][Np] (TC; slot order inside each 32-key block; d >= 24 and keys >= N
// are zero) and the additive key mask MA [B][Np] fp32 in slot order, log2 e * 1e9 (m - 1)
// for real keys (attention.py:429-430) and -inf for the padding keys.
template <class TC>
__global__ __launch_bounds__(256) void single_attn_pack_kernel(const TC* __restrict__ qkvg,
                                                               const float* __restrict__ seq_mask,
                                                               TC* __restrict__ Vt, float* __restrict__ MA, int B,
                                                               int N, int Np, int H) {
  const int HD = H * kSHeadDim;
  const long nvt = (long)B * H * 32 * Np;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < nvt; i += (long)gridDim.x * 256) {
    const int slot = (int)(i % Np);
    const long r = i / Np;
    const int d = (int)(r % 32);
    const int h = (int)((r / 32) % H);
    const int b = (int)(r / (32 * H));
    const int key = (slot & ~31) + slot_key(slot & 31);
    float v = 0.f;
    if (d < kSHeadDim && key < N) v = to_f32(qkvg[((size_t)b * N + key) * 4 * HD + 2 * HD + h * kSHeadDim + d]);
    Vt[i] = from_f32<TC>(v);
    if (i < (long)B * Np) {
      const int bb = (int)(i / Np);
      MA[i] = key < N ? kLog2e * (1e9f * (seq_mask[(size_t)bb * N + key] - 1.0f)) : -INFINITY;
    }
  }
}

// 16 values of a 24-wide head row as a Frag16 (lane half hf: d 16 hf .. 16 hf + 15; d >= 24
// is zero), each multiplied by `scale`.
template <class TC>
PF_DEVICE Frag16<TC> head_frag(const TC* row, int hf, float scale);
template <>
PF_DEVICE Frag16<bf16> head_frag<bf16>(const bf16* row, int hf, float scale) {
  Frag16<bf16> f;
  const bf16x8 a = *reinterpret_cast<const bf16x8*>(row + 16 * hf);
  const bf16x8 c = *reinterpret_cast<const bf16x8*>(row + 8);  // d 8..15 (used by hf = 0)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    f.v[0][e] = scale == 1.0f ? a[e] : (bf16)((float)a[e] * scale);
    f.v[1][e] = hf ? (bf16)0.f : (scale == 1.0f ? c[e] : (bf16)((float)c[e] * scale));
  }
  return f;
}
template <>
PF_DEVICE Frag16<float> head_frag<float>(const float* row, int hf, float scale) {
  Frag16<float> f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d0 = 16 * hf + 4 * i;
    if (d0 < kSHeadDim) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(row + d0);
      f.v[i] = f32x4{v[0] * scale, v[1] * scale, v[2] * scale, v[3] * scale};
    } else {
      f.v[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  return f;
}

// One block per (b, h, 32 queries); its four waves split the key blocks (wave w takes
// blocks w, w + 4, ...) and merge their partial softmax states through LDS at the end.
// qkvg [B*N][4*H*24] (TC): q | k | v | g (pre-sigmoid); pair_logits pl fp32 [B][H][N][N];
// og [B*N][H*24] = o * sigmoid(g). Softmax in fp32 with a running maximum (base 2); a fully
// masked query row sees every logit shifted by the same -1e9 and attends uniformly, as the
// reference's fp32 softmax does.
template <class TC>
__global__ __launch_bounds__(256) void single_attn_flash_kernel(const TC* __restrict__ qkvg, const TC* __restrict__ Vt,
                                                                const float* __restrict__ MA,
                                                                const float* __restrict__ pl, TC* __restrict__ og,
                                                                int B, int N, int Np, int H) {
  constexpr int D = kSHeadDim;
  __shared__ float part[3][18][64];  // waves 1..3: running max, sum and 16 output values per lane
  const int nqb = Np / 32;
  const int qb = blockIdx.x % nqb;
  const int h = (blockIdx.x / nqb) % H;
  const int b = blockIdx.x / (nqb * H);
  const int w = wave_id();
  const int l = lane_id();
  const int lq = l & 31, hf = l >> 5;
  const int HD = H * D;
  const size_t ld = 4 * (size_t)HD;
  const TC* base = qkvg + (size_t)b * N * ld;
  const int q = qb * 32 + lq;
  const int qc = min(q, N - 1);
  const Frag16<TC> qf = head_frag<TC>(base + qc * ld + h * D, hf, kLog2e / sqrtf((float)D));
  const float* plr = pl + (((size_t)b * H + h) * N + qc) * N;
  const TC* vt = Vt + (((size_t)b * H + h) * 32 + lq) * Np + 16 * hf;
  const float* ma = MA + (size_t)b * Np + 16 * hf;
  const bool vec_ok = (N & 3) == 0;

  // Operands of one key block: K and V^T fragments, and the bias + mask logits.
  struct Ops {
    Frag16<TC> kf, vf;
    f32x4 mk[4], pb[4];
  };
  auto load = [&](int kb, Ops& op) {
    const int k0 = kb * 32;
    op.kf = head_frag<TC>(base + min(k0 + lq, N - 1) * ld + HD + h * D, hf, 1.0f);
    op.vf.load(vt + k0);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      op.mk[g] = *reinterpret_cast<const f32x4*>(ma + k0 + 4 * g);
      const int kk = k0 + 8 * g + 4 * hf;  // keys kappa(4 g .. 4 g + 3, hf)
      if (vec_ok && kk < N) {
        op.pb[g] = *reinterpret_cast<const f32x4*>(plr + kk);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) op.pb[g][e] = kk + e < N ? plr[kk + e] : 0.f;
      }
    }
  };

  f32x16 o;
#pragma unroll
  for (int r = 0; r < 16; ++r) o[r] = 0.f;
  float mrun = -INFINITY, lrun = 0.f;
  const int nkb = Np / 32;
  Ops cur, nxt;
  if (w < nkb) load(w, cur);
  for (int kb = w; kb < nkb; kb += 4) {
    if (kb + 4 < nkb) load(kb + 4, nxt);
    f32x16 s;
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) s[4 * g + e] = fmaf(cur.pb[g][e], kLog2e, cur.mk[g][e]);
    mma32_16(s, cur.kf, qf);
    float m = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) m = fmaxf(m, s[r]);
    const float mnew = fmaxf(mrun, max_xor32(m));
    const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
    mrun = mnew;
    float ls = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = __builtin_amdgcn_exp2f(s[r] - mnew);
      ls += s[r];
      o[r] *= alpha;
    }
    lrun = lrun * alpha + ls;
    mma32_16(o, cur.vf, pack_p(s, TC{}));
    cur = nxt;
  }
  if (w > 0) {
    part[w - 1][0][l] = mrun;
    part[w - 1][1][l] = lrun;
#pragma unroll
    for (int r = 0; r < 16; ++r) part[w - 1][2 + r][l] = o[r];
  }
  __syncthreads();
  if (w > 0) return;
  // Merge: wave 0 always holds key block 0 (a finite maximum), so mt is finite; a wave
  // without key blocks has mrun = -inf and contributes 0.
  float mt = mrun;
#pragma unroll
  for (int v = 0; v < 3; ++v) mt = fmaxf(mt, part[v][0][l]);
  const float a0 = __builtin_amdgcn_exp2f(mrun - mt);
  lrun *= a0;
#pragma unroll
  for (int r = 0; r < 16; ++r) o[r] *= a0;
#pragma unroll
  for (int v = 0; v < 3; ++v) {
    const float av = __builtin_amdgcn_exp2f(part[v][0][l] - mt);
    lrun += av * part[v][1][l];
#pragma unroll
    for (int r = 0; r < 16; ++r) o[r] += av * part[v][2 + r][l];
  }
  if (q >= N) return;
  const float inv = 1.0f / (lrun + __shfl_xor(lrun, 32, 64));
  // O^T lane (q, hf) holds d = 8 (r >> 2) + 4 hf + (r & 3); d < 24 for r < 12.
  const TC* grow = base + q * ld + 3 * HD + h * D;
  TC* dst = og + ((size_t)b * N + q) * HD + h * D;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int d0 = 8 * j + 4 * hf;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = o[4 * j + e] * inv * sigmoidf_(to_f32(grow[d0 + e]));
    store_vec<TC, 4>(dst + d0, v);
  }
}

// y = silu(x[:, :D]) * x[:, D:] (FusedSwiGLU, triton/swiglu.py:30-58, :192-200).
template <class T>
__global__ __launch_bounds__(256) void swiglu_kernel(const T* __restrict__ x, T* __restrict__ y, long M, int D) {
  const long n = M * D;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const long r = i / D;
    const int c = (int)(i % D);
    const float a = to_f32(x[r * 2 * D + c]);
    const float bb = to_f32(x[r * 2 * D + D + c]);
    y[i] = from_f32<T>(siluf_(a) * bb);
  }
}

// Backward of swiglu_kernel: for y = silu(a) b, da = dy b silu'(a) with
// silu'(a) = s (1 + a (1 - s)), s = sigmoid(a), and db = dy silu(a); dx = [da | db].
template <class T>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                         T* __restrict__ dx, long M, int D) {
  const long n = M * D;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const long r = i / D;
    const int c = (int)(i % D);
    const float a = to_f32(x[r * 2 * D + c]);
    const float bb = to_f32(x[r * 2 * D + D + c]);
    const float g = to_f32(dy[i]);
    const float sg = sigmoidf_(a);
    dx[r * 2 * D + c] = from_f32<T>(g * bb * sg * (1.f + a * (1.f - sg)));
    dx[r * 2 * D + D + c] = from_f32<T>(g * a * sg);
  }
}

size_t es_of(int dt) { return dt == PF_F32 ? 4 : 2; }

template <class TZ, class TC>
int single_attn_launch(const void* s_in, const float* seq_mask, const float* pair_logits, const float* lnw,
                       const float* lnb, float eps, const void* wqkvg, const float* qbias, const void* wout, int B,
                       int N, int C, int H, void* out, int accumulate, void* ws, hipStream_t st) {
  const long M = (long)B * N;
  const int HD = H * kSHeadDim;
  char* p = reinterpret_cast<char*>(ws);
  TC* xn = reinterpret_cast<TC*>(p);
  p += pf::round_up((size_t)M * C * sizeof(TC), 256);
  TC* qkvg = reinterpret_cast<TC*>(p);
  p += pf::round_up((size_t)M * 4 * HD * sizeof(TC), 256);
  TC* og = reinterpret_cast<TC*>(p);
  if (int e = ln_launch<TZ, TC>(s_in, lnw, lnb, eps, xn, M, C, st)) return e;
  if (int e = rowgemm_launch<TC, TC, EPI_STORE>(xn, wqkvg, qbias, HD, qkvg, M, 4 * HD, C, st)) return e;
  {
    const int Np = (int)pf::round_up((size_t)N, 32);
    p += pf::round_up((size_t)M * HD * sizeof(TC), 256);
    TC* vt = reinterpret_cast<TC*>(p);
    p += pf::round_up((size_t)B * H * 32 * Np * sizeof(TC), 256);
    float* ma = reinterpret_cast<float*>(p);
    const long nvt = (long)B * H * 32 * Np;
    single_attn_pack_kernel<TC><<<(unsigned)std::min<long>((nvt + 255) / 256, 4096), 256, 0, st>>>(
        qkvg, seq_mask, vt, ma, B, N, Np, H);
    if (int e = pf::check_launch("single_attn_pack")) return e;
    const long blocks = (long)B * H * (Np / 32);
    pf::KernelTimer timer("single_attn_core", st);
    single_attn_flash_kernel<TC><<<(unsigned)blocks, 256, 0, st>>>(qkvg, vt, ma, pair_logits, og, B, N, Np, H);
    timer.stop();
    if (int e = pf::check_launch("single_attn_core")) return e;
  }
  if (accumulate) return rowgemm_launch<TC, TZ, EPI_RESIDUAL>(og, wout, nullptr, 0, out, M, C, HD, st);
  return rowgemm_launch<TC, TZ, EPI_STORE>(og, wout, nullptr, 0, out, M, C, HD, st);
}

// out += LN(prev) W^T: LayerNorm into the workspace, then the row GEMM whose epilogue adds
// into `out` (one rounding of the sum, as the reference's `pair + prev_embedding(...)`).
template <class TZ, class TC>
int recycle_embed_launch(const void* prev, const float* lnw, const float* lnb, float eps, const void* w, long M,
                         int C, void* out, void* ws, hipStream_t st) {
  if (int e = ln_launch<TZ, TC>(prev, lnw, lnb, eps, ws, M, C, st)) return e;
  return rowgemm_launch<TC, TZ, EPI_RESIDUAL>(ws, w, nullptr, 0, out, M, C, C, st);
}

template <class TZ, class TC>
int transition_generic_launch(const void* x, const float* lnw, const float* lnb, float eps, const void* w1,
                              const void* w2, long M, int C, int F, void* out, int accumulate, void* ws,
                              hipStream_t st) {
  char* p = reinterpret_cast<char*>(ws);
  TC* xn = reinterpret_cast<TC*>(p);
  p += pf::round_up((size_t)M * C * sizeof(TC), 256);
  TC* u = reinterpret_cast<TC*>(p);
  if (int e = ln_launch<TZ, TC>(x, lnw, lnb, eps, xn, M, C, st)) return e;
  if (int e = rowgemm_launch<TC, TC, EPI_SWIGLU>(xn, w1, nullptr, 0, u, M, F, C, st)) return e;
  if (accumulate) return rowgemm_launch<TC, TZ, EPI_RESIDUAL>(u, w2, nullptr, 0, out, M, C, F, st);
  return rowgemm_launch<TC, TZ, EPI_STORE>(u, w2, nullptr, 0, out, M, C, F, st);
}

#define PF_DISPATCH_ZC(zd, cd, FN, ...)                                                        \
  ((zd) == PF_F32 && (cd) == PF_F32 ? FN<float, float>(__VA_ARGS__)                            \
   : (zd) == PF_F32                 ? FN<float, bf16>(__VA_ARGS__)                             \
                                    : FN<bf16, bf16>(__VA_ARGS__))

bool dtype_pair_ok(int zd, int cd) {
  return (zd == PF_F32 || zd == PF_BF16) && (cd == PF_F32 || cd == PF_BF16) && !(zd == PF_BF16 && cd == PF_F32);
}

// Argument checks shared by pf_single_attn_fwd and its allocation-free variant.
int single_attn_check(const char* fn, const void* s, const float* seq_mask, const float* pair_logits,
                      const float* ln_w, const float* ln_b, const void* w_qkvg, const float* q_bias,
                      const void* w_out, int B, int N, int C, int H, int zdtype, int cdtype, const void* out) {
  PF_REQUIRE(s && seq_mask && pair_logits && ln_w && ln_b && w_qkvg && q_bias && w_out && out, PF_ERR_INVALID_ARG,
             "%s: null pointer", fn);
  PF_REQUIRE(B > 0 && N > 0, PF_ERR_INVALID_ARG, "%s: B=%d N=%d", fn, B, N);
  PF_REQUIRE(H > 0 && H * kSHeadDim == C && C % 32 == 0, PF_ERR_UNSUPPORTED,
             "%s: C=%d H=%d (built: head dim 24, C a multiple of 32)", fn, C, H);
  PF_REQUIRE(dtype_pair_ok(zdtype, cdtype), PF_ERR_UNSUPPORTED, "%s: dtype pair (%d, %d)", fn, zdtype, cdtype);
  return PF_OK;
}

// ---- scratch of the allocation-free entry point (pf_single_attn_fwd_noalloc)
// One array per GPU, created with the code object when the library's kernels load on that
// device and held until the process ends. In host code `scratch` names a host-side
// stand-in, not device memory: kernels only ever receive the per-device address that
// hipGetSymbolAddress returns for it (scratch_base below).
static __device__ __align__(256) unsigned char scratch[PF_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_base[kMaxDevices] = {};

// Address of `scratch` on the device that `stream` runs on, looked up once per device with
// that device current.
int scratch_base(hipStream_t stream, void** base) {
  int dev = -1;
  if (stream != nullptr) {
    PF_REQUIRE(hipStreamGetDevice(stream, &dev) == hipSuccess, PF_ERR_LAUNCH,
               "pf_single_attn_fwd_noalloc: hipStreamGetDevice failed");
  } else {
    PF_REQUIRE(hipGetDevice(&dev) == hipSuccess, PF_ERR_LAUNCH, "pf_single_attn_fwd_noalloc: hipGetDevice failed");
  }
  PF_REQUIRE(dev >= 0 && dev < kMaxDevices, PF_ERR_UNSUPPORTED, "pf_single_attn_fwd_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_base[dev] == nullptr) {
    int cur = -1;
    PF_REQUIRE(hipGetDevice(&cur) == hipSuccess, PF_ERR_LAUNCH, "pf_single_attn_fwd_noalloc: hipGetDevice failed");
    if (cur != dev)
      PF_REQUIRE(hipSetDevice(dev) == hipSuccess, PF_ERR_LAUNCH, "pf_single_attn_fwd_noalloc: hipSetDevice(%d)", dev);
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    PF_REQUIRE(e == hipSuccess && p != nullptr, PF_ERR_LAUNCH,
               "pf_single_attn_fwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_base[dev] = p;
  }
  *base = g_scratch_base[dev];
  return PF_OK;
}

}  // namespace

extern "C" {

size_t pf_single_attn_workspace_bytes(int B, int N, int C, int H, int cdtype) {
  if (B <= 0 || N <= 0 || C <= 0 || H <= 0) return 0;
  const size_t M = (size_t)B * N, es = es_of(cdtype), HD = (size_t)H * kSHeadDim;
  const size_t Np = pf::round_up((size_t)N, 32);
  return pf::round_up(M * C * es, 256) + pf::round_up(M * 4 * HD * es, 256) + pf::round_up(M * HD * es, 256) +
         pf::round_up((size_t)B * H * 32 * Np * es, 256) + pf::round_up((size_t)B * Np * 4, 256);
}

int pf_single_attn_fwd(const void* s, const float* seq_mask, const float* pair_logits, const float* ln_w,
                       const float* ln_b, float eps, const void* w_qkvg, const float* q_bias, const void* w_out, int B,
                       int N, int C, int H, int zdtype, int cdtype, void* out, int accumulate, void* workspace,
                       size_t workspace_bytes, void* stream) {
  if (int e = single_attn_check("pf_single_attn_fwd", s, seq_mask, pair_logits, ln_w, ln_b, w_qkvg, q_bias, w_out, B,
                                N, C, H, zdtype, cdtype, out))
    return e;
  PF_REQUIRE(workspace != nullptr, PF_ERR_INVALID_ARG, "pf_single_attn_fwd: null workspace");
  PF_REQUIRE(workspace_bytes >= pf_single_attn_workspace_bytes(B, N, C, H, cdtype), PF_ERR_WORKSPACE,
             "pf_single_attn_fwd: workspace %zu < %zu bytes", workspace_bytes,
             pf_single_attn_workspace_bytes(B, N, C, H, cdtype));
  hipStream_t st = pf::as_stream(stream);
  return PF_DISPATCH_ZC(zdtype, cdtype, single_attn_launch, s, seq_mask, pair_logits, ln_w, ln_b, eps, w_qkvg, q_bias,
                        w_out, B, N, C, H, out, accumulate, workspace, st);
}

int pf_single_attn_fwd_noalloc(const void* s, const float* seq_mask, const float* pair_logits, const float* ln_w,
                               const float* ln_b, float eps, const void* w_qkvg, const float* q_bias, const void* w_out,
                               int B, int N, int C, int H, int zdtype, int cdtype, void* out, int accumulate,
                               void* stream) {
  if (int e = single_attn_check("pf_single_attn_fwd_noalloc", s, seq_mask, pair_logits, ln_w, ln_b, w_qkvg, q_bias,
                                w_out, B, N, C, H, zdtype, cdtype, out))
    return e;
  const size_t need = pf_single_attn_workspace_bytes(B, N, C, H, cdtype);
  PF_REQUIRE(need <= PF_NOALLOC_SCRATCH_BYTES, PF_ERR_WORKSPACE,
             "pf_single_attn_fwd_noalloc: B=%d N=%d C=%d needs %zu bytes of scratch, more than the %u-byte static "
             "array; use pf_single_attn_fwd with a workspace",
             B, N, C, need, (unsigned)PF_NOALLOC_SCRATCH_BYTES);
  hipStream_t st = pf::as_stream(stream);
  void* base = nullptr;
  if (int e = scratch_base(st, &base)) return e;
  // Every byte of the scratch a call reads is written earlier in the same call (LayerNorm
  // rows, projections, the packed V^T and mask including their padding, the attention
  // output), so nothing is cleared.
  return PF_DISPATCH_ZC(zdtype, cdtype, single_attn_launch, s, seq_mask, pair_logits, ln_w, ln_b, eps, w_qkvg, q_bias,
                        w_out, B, N, C, H, out, accumulate, base, st);
}

int pf_swiglu_fwd(const void* x, int dtype, void* y, long M, int D, void* stream) {
  PF_REQUIRE(x && y, PF_ERR_INVALID_ARG, "pf_swiglu_fwd: null pointer");
  PF_REQUIRE(M >= 0 && D > 0, PF_ERR_INVALID_ARG, "pf_swiglu_fwd: M=%ld D=%d", M, D);
  PF_REQUIRE(dtype == PF_F32 || dtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_swiglu_fwd: dtype %d", dtype);
  if (M == 0) return pf::ok();
  hipStream_t s = pf::as_stream(stream);
  const long n = M * D;
  const unsigned g = (unsigned)((n + 255) / 256 > 65536 ? 65536 : (n + 255) / 256);
  if (dtype == PF_F32)
    swiglu_kernel<float><<<g, 256, 0, s>>>((const float*)x, (float*)y, M, D);
  else
    swiglu_kernel<bf16><<<g, 256, 0, s>>>((const bf16*)x, (bf16*)y, M, D);
  return pf::check_launch("swiglu");
}

int pf_swiglu_bwd(const void* x, const void* dy, int dtype, void* dx, long M, int D, void* stream) {
  PF_REQUIRE(x && dy && dx, PF_ERR_INVALID_ARG, "pf_swiglu_bwd: null pointer");
  PF_REQUIRE(M >= 0 && D > 0, PF_ERR_INVALID_ARG, "pf_swiglu_bwd: M=%ld D=%d", M, D);
  PF_REQUIRE(dtype == PF_F32 || dtype == PF_BF16, PF_ERR_UNSUPPORTED, "pf_swiglu_bwd: dtype %d", dtype);
  if (M == 0) return pf::ok();
  hipStream_t s = pf::as_stream(stream);
  const long n = M * D;
  const unsigned g = (unsigned)((n + 255) / 256 > 65536 ? 65536 : (n + 255) / 256);
  if (dtype == PF_F32)
    swiglu_bwd_kernel<float><<<g, 256, 0, s>>>((const float*)x, (const float*)dy, (float*)dx, M, D);
  else
    swiglu_bwd_kernel<bf16><<<g, 256, 0, s>>>((const bf16*)x, (const bf16*)dy, (bf16*)dx, M, D);
  return pf::check_launch("swiglu_bwd");
}

size_t pf_layernorm_linear_workspace_bytes(long M, int K, int cdtype) {
  if (M <= 0 || K <= 0) return 0;
  return pf::round_up((size_t)M * K * es_of(cdtype), 256);
}

int pf_layernorm_linear_fwd(const void* x, int xdtype, const float* ln_w, const float* ln_b, float eps,
                            const void* w_nk, const float* bias, long M, int K, int Nout, int cdtype, void* out,
                            void* workspace, size_t workspace_bytes, void* stream) {
  PF_REQUIRE(x && ln_w && ln_b && w_nk && out && workspace, PF_ERR_INVALID_ARG,
             "pf_layernorm_linear_fwd: null pointer");
  PF_REQUIRE(M >= 0 && K > 0 && Nout > 0, PF_ERR_INVALID_ARG, "pf_layernorm_linear_fwd: M=%ld K=%d N=%d", M, K, Nout);
  PF_REQUIRE(K % 32 == 0 && Nout % 16 == 0, PF_ERR_UNSUPPORTED,
             "pf_layernorm_linear_fwd: K=%d N=%d (K a multiple of 32, N of 16)", K, Nout);
  PF_REQUIRE(dtype_pair_ok(xdtype, cdtype), PF_ERR_UNSUPPORTED, "pf_layernorm_linear_fwd: dtype pair (%d, %d)",
             xdtype, cdtype);
  PF_REQUIRE(workspace_bytes >= pf_layernorm_linear_workspace_bytes(M, K, cdtype), PF_ERR_WORKSPACE,
             "pf_layernorm_linear_fwd: workspace too small");
  if (M == 0) return pf::ok();
  hipStream_t st = pf::as_stream(stream);
  if (cdtype == PF_F32) {
    if (int e = ln_launch<float, float>(x, ln_w, ln_b, eps, workspace, M, K, st)) return e;
    return rowgemm_launch<float, float, EPI_STORE>(workspace, w_nk, bias, bias ? Nout : 0, out, M, Nout, K, st);
  }
  if (xdtype == PF_F32) {
    if (int e = ln_launch<float, bf16>(x, ln_w, ln_b, eps, workspace, M, K, st)) return e;
    return rowgemm_launch<bf16, float, EPI_STORE>(workspace, w_nk, bias, bias ? Nout : 0, out, M, Nout, K, st);
  }
  if (int e = ln_launch<bf16, bf16>(x, ln_w, ln_b, eps, workspace, M, K, st)) return e;
  return rowgemm_launch<bf16, bf16, EPI_STORE>(workspace, w_nk, bias, bias ? Nout : 0, out, M, Nout, K, st);
}

size_t pf_transition_workspace_bytes(long M, int C, int factor, int cdtype) {
  if (M <= 0 || C <= 0 || factor <= 0) return 0;
  const size_t es = es_of(cdtype);
  return pf::round_up((size_t)M * C * es, 256) + pf::round_up((size_t)M * C * factor * es, 256);
}

int pf_transition_fwd(const void* x, const float* ln_w, const float* ln_b, float eps, const void* w1, const void* w2,
                      long M, int C, int factor, int zdtype, int cdtype, void* out, int accumulate, void* workspace,
                      size_t workspace_bytes, void* stream) {
  PF_REQUIRE(x && ln_w && ln_b && w1 && w2 && out && workspace, PF_ERR_INVALID_ARG, "pf_transition_fwd: null pointer");
  PF_REQUIRE(M >= 0 && C > 0 && factor > 0, PF_ERR_INVALID_ARG, "pf_transition_fwd: M=%ld C=%d factor=%d", M, C,
             factor);
  PF_REQUIRE(C % 32 == 0 && (C * factor) % 64 == 0, PF_ERR_UNSUPPORTED,
             "pf_transition_fwd: C=%d factor=%d (C must be a multiple of 32, C*factor of 64)", C, factor);
  PF_REQUIRE(dtype_pair_ok(zdtype, cdtype), PF_ERR_UNSUPPORTED, "pf_transition_fwd: dtype pair (%d, %d)", zdtype,
             cdtype);
  PF_REQUIRE(workspace_bytes >= pf_transition_workspace_bytes(M, C, factor, cdtype), PF_ERR_WORKSPACE,
             "pf_transition_fwd: workspace %zu < %zu bytes", workspace_bytes,
             pf_transition_workspace_bytes(M, C, factor, cdtype));
  if (M == 0) return pf::ok();
  hipStream_t st = pf::as_stream(stream);
  return PF_DISPATCH_ZC(zdtype, cdtype, transition_generic_launch, x, ln_w, ln_b, eps, w1, w2, M, C, C * factor, out,
                        accumulate, workspace, st);
}

size_t pf_recycle_embed_workspace_bytes(long M, int C, int cdtype) {
  if (M <= 0 || C <= 0) return 0;
  return pf::round_up((size_t)M * C * es_of(cdtype), 256);
}

int pf_recycle_embed_fwd(const void* prev, const float* ln_w, const float* ln_b, float eps, const void* w, long M,
                         int C, int zdtype, int cdtype, void* out, void* workspace, size_t workspace_bytes,
                         void* stream) {
  PF_REQUIRE(prev && ln_w && ln_b && w && out && workspace, PF_ERR_INVALID_ARG,
             "pf_recycle_embed_fwd: null pointer");
  PF_REQUIRE(M >= 0 && C > 0, PF_ERR_INVALID_ARG, "pf_recycle_embed_fwd: M=%ld C=%d", M, C);
  PF_REQUIRE(C % 64 == 0, PF_ERR_UNSUPPORTED, "pf_recycle_embed_fwd: C=%d (a multiple of 64)", C);
  PF_REQUIRE(dtype_pair_ok(zdtype, cdtype), PF_ERR_UNSUPPORTED, "pf_recycle_embed_fwd: dtype pair (%d, %d)", zdtype,
             cdtype);
  PF_REQUIRE(prev != out, PF_ERR_INVALID_ARG, "pf_recycle_embed_fwd: prev and out must not alias");
  PF_REQUIRE(workspace_bytes >= pf_recycle_embed_workspace_bytes(M, C, cdtype), PF_ERR_WORKSPACE,
             "pf_recycle_embed_fwd: workspace %zu < %zu bytes", workspace_bytes,
             pf_recycle_embed_workspace_bytes(M, C, cdtype));
  if (M == 0) return pf::ok();
  hipStream_t st = pf::as_stream(stream);
  return PF_DISPATCH_ZC(zdtype, cdtype, recycle_embed_launch, prev, ln_w, ln_b, eps, w, M, C, out, workspace, st);
}

}  // extern "C"
