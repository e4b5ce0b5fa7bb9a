// AdamW step of the MoE decoder's training step, many tensors per launch.
//
// Reference: abacus/optimizers/adamw.py:85-119.  For each parameter with a
// gradient, the reference runs separate tensor ops on the parameter's dtype,
// so every intermediate is rounded to that dtype:
//   p  = p * (1 - lr*wd)                       weight.mul_
//   m  = lerp(m, g, 1 - beta1)                 exp_avg.lerp_
//   v  = v * beta2;  v = v + (1 - beta2) g g   exp_avg_sq.mul_(...).addcmul_
//   d  = sqrt(v);  d = d / sqrt(bc2);  d = d + eps
//   p  = p + (-lr / bc1) * (m / d)             weight.addcdiv_
// with bc1 = 1 - beta1^step, bc2 = 1 - beta2^step.  One pass here reads p, g,
// m, v once and writes p, m, v once (14 bytes per bf16 element), computing
// the same sequence in fp32 with the same roundings in between.  The fp32
// forms are those of torch's device kernels, which the reference runs on a
// GPU (each compared with torch's own op on MI355X): lerp fma(w, b - a, a)
// for |w| < 0.5 (else b - (b - a)(1 - w)), addcmul fma(s, b c, a), addcdiv
// fma(s, b / c, a), division by a Python scalar as a product with its
// reciprocal (taken in double, then rounded to fp32), every other op on its own (no other contraction); division and
// square root correctly rounded; scalars are the reference's double-precision
// values rounded to fp32.
#include <algorithm>
#include <cmath>

#include "common.h"

namespace abacus {
namespace {

constexpr int kAdamwMaxTensors = 48;  // tensors per launch (kernel-argument space)
constexpr int kAdamwThreads = 256;
constexpr int kAdamwVecs = 2;          // 16-byte vectors per thread per block

struct AdamwArgs {
  void* p[kAdamwMaxTensors];
  const void* g[kAdamwMaxTensors];
  void* m[kAdamwMaxTensors];
  void* v[kAdamwMaxTensors];
  int64_t numel[kAdamwMaxTensors];
  float neg_step_size[kAdamwMaxTensors];  // -(lr / bc1)
  float inv_sqrt_bc2[kAdamwMaxTensors];   // float(1 / sqrt(bc2)), the reciprocal taken in double
  int block_start[kAdamwMaxTensors + 1];  // tensor i owns blocks [block_start[i], block_start[i+1])
  int n;
  float decay;  // 1 - lr * wd (1 when wd == 0)
  float w1;     // 1 - beta1
  float beta2;
  float a2;     // 1 - beta2
  float eps;
};

// Rounds x and y to T's precision: bf16 by one v_cvt_pk_bf16_f32 for both
// (round to nearest even, the same bits as f32_to_bf16); fp32 unchanged.
template <typename T>
__device__ inline void rnd2(float& x, float& y);
template <>
__device__ inline void rnd2<float>(float&, float&) {}
template <>
__device__ inline void rnd2<uint16_t>(float& x, float& y) {
  const uint32_t w = pack_bf16x2(x, y);
  x = lo_bf16(w);
  y = hi_bf16(w);
}

// Two elements through the reference's op sequence, each op's results rounded
// together (fused multiply-adds only where torch's device kernels have them).
template <typename T>
__device__ inline void adamw_pair(float (&p)[2], const float (&g)[2], float (&m)[2], float (&v)[2],
                                  const AdamwArgs& a, float nss, float isb) {
#pragma clang fp contract(off)
  float d[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) p[k] = p[k] * a.decay;
  rnd2<T>(p[0], p[1]);
#pragma unroll
  for (int k = 0; k < 2; ++k)
    m[k] = a.w1 < 0.5f ? __builtin_fmaf(a.w1, g[k] - m[k], m[k]) : g[k] - (g[k] - m[k]) * (1.0f - a.w1);
  rnd2<T>(m[0], m[1]);
#pragma unroll
  for (int k = 0; k < 2; ++k) v[k] = v[k] * a.beta2;
  rnd2<T>(v[0], v[1]);
#pragma unroll
  for (int k = 0; k < 2; ++k) v[k] = __builtin_fmaf(a.a2, g[k] * g[k], v[k]);
  rnd2<T>(v[0], v[1]);
  // sqrtf and / are correctly rounded (hipcc's default); __fsqrt_rn is not, on gfx950
#pragma unroll
  for (int k = 0; k < 2; ++k) d[k] = sqrtf(v[k]);
  rnd2<T>(d[0], d[1]);
#pragma unroll
  for (int k = 0; k < 2; ++k) d[k] = d[k] * isb;
  rnd2<T>(d[0], d[1]);
#pragma unroll
  for (int k = 0; k < 2; ++k) d[k] = d[k] + a.eps;
  rnd2<T>(d[0], d[1]);
#pragma unroll
  for (int k = 0; k < 2; ++k) p[k] = __builtin_fmaf(nss, m[k] / d[k], p[k]);
  rnd2<T>(p[0], p[1]);
}

// Element pairs of one 16-byte vector: bf16 packs a pair per 32-bit word
// (values already on the bf16 grid, so packing is exact); fp32 a pair per two.
template <typename T>
struct Pairs;
template <>
struct Pairs<uint16_t> {
  static constexpr int N = 4;
  __device__ static inline void get(const Vec16& x, int k, float (&o)[2]) {
    o[0] = lo_bf16(x.w[k]);
    o[1] = hi_bf16(x.w[k]);
  }
  __device__ static inline void put(Vec16& x, int k, const float (&o)[2]) { x.w[k] = pack_bf16x2(o[0], o[1]); }
};
template <>
struct Pairs<float> {
  static constexpr int N = 2;
  __device__ static inline void get(const Vec16& x, int k, float (&o)[2]) {
    o[0] = bits_f32(x.w[2 * k]);
    o[1] = bits_f32(x.w[2 * k + 1]);
  }
  __device__ static inline void put(Vec16& x, int k, const float (&o)[2]) {
    x.w[2 * k] = f32_bits(o[0]);
    x.w[2 * k + 1] = f32_bits(o[1]);
  }
};

// Elements per 16-byte vector and per block.
template <typename T>
struct AdamwGeo {
  static constexpr int EPV = 16 / sizeof(T);
  static constexpr int EPB = kAdamwThreads * kAdamwVecs * EPV;
};

// Nontemporal 16-byte loads and stores (ld16_stream, st16_stream): every byte
// is touched once per step, so keeping it out of the caches' working set helps
// the stream (3.19 -> 3.00 ms per step over the decoder's 1.2 G bf16
// parameters; nontemporal stores alone made no difference).

template <typename T>
__global__ __launch_bounds__(kAdamwThreads) void adamw_kernel(AdamwArgs a) {
  constexpr int EPV = AdamwGeo<T>::EPV, EPB = AdamwGeo<T>::EPB;
  using PR = Pairs<T>;
  // this block's tensor (block_start is ascending; n <= kAdamwMaxTensors)
  int i = 0;
  while (i + 1 < a.n && (int)blockIdx.x >= a.block_start[i + 1]) ++i;
  const int64_t n = a.numel[i];
  const int64_t base = (int64_t)((int)blockIdx.x - a.block_start[i]) * EPB;
  T* P = (T*)a.p[i];
  const T* G = (const T*)a.g[i];
  T* M = (T*)a.m[i];
  T* V = (T*)a.v[i];
  const float nss = a.neg_step_size[i], isb = a.inv_sqrt_bc2[i];

  Vec16 vp[kAdamwVecs], vg[kAdamwVecs], vm[kAdamwVecs], vv[kAdamwVecs];
#pragma unroll
  for (int u = 0; u < kAdamwVecs; ++u) {
    const int64_t e0 = base + ((int64_t)u * kAdamwThreads + threadIdx.x) * EPV;
    if (e0 + EPV <= n) {
      vp[u] = ld16_stream(P + e0);
      vg[u] = ld16_stream(G + e0);
      vm[u] = ld16_stream(M + e0);
      vv[u] = ld16_stream(V + e0);
    }
  }
#pragma unroll
  for (int u = 0; u < kAdamwVecs; ++u) {
    const int64_t e0 = base + ((int64_t)u * kAdamwThreads + threadIdx.x) * EPV;
    if (e0 + EPV <= n) {
      Vec16 op, om, ov;
#pragma unroll
      for (int k = 0; k < PR::N; ++k) {
        float p[2], g[2], m[2], v[2];
        PR::get(vp[u], k, p);
        PR::get(vg[u], k, g);
        PR::get(vm[u], k, m);
        PR::get(vv[u], k, v);
        adamw_pair<T>(p, g, m, v, a, nss, isb);
        PR::put(op, k, p);
        PR::put(om, k, m);
        PR::put(ov, k, v);
      }
      st16_stream(P + e0, op);
      st16_stream(M + e0, om);
      st16_stream(V + e0, ov);
    } else if (e0 < n) {
      // the tensor's last, partial vector, a pair at a time (an odd last element
      // is paired with a copy of itself that is not stored)
      for (int64_t e = e0; e < n; e += 2) {
        const int64_t f = e + 1 < n ? e + 1 : e;
        float p[2] = {to_f32<T>(P[e]), to_f32<T>(P[f])}, g[2] = {to_f32<T>(G[e]), to_f32<T>(G[f])};
        float m[2] = {to_f32<T>(M[e]), to_f32<T>(M[f])}, v[2] = {to_f32<T>(V[e]), to_f32<T>(V[f])};
        adamw_pair<T>(p, g, m, v, a, nss, isb);
        P[e] = from_f32<T>(p[0]);
        M[e] = from_f32<T>(m[0]);
        V[e] = from_f32<T>(v[0]);
        if (f != e) {
          P[f] = from_f32<T>(p[1]);
          M[f] = from_f32<T>(m[1]);
          V[f] = from_f32<T>(v[1]);
        }
      }
    }
  }
}

}  // namespace
}  // namespace abacus

using namespace abacus;

extern "C" int abacus_adamw_step(void* const* params, const void* const* grads, void* const* exp_avgs,
                                 void* const* exp_avg_sqs, const int64_t* numels, const int64_t* steps, int n,
                                 double lr, double beta1, double beta2, double eps, double weight_decay, int dtype,
                                 void* stream) {
  ABACUS_CHECK_ARG(dtype == kF32 || dtype == kBF16, "unsupported dtype code %d (0 = fp32, 1 = bf16)", dtype);
  ABACUS_CHECK_ARG(n >= 0, "n %d must be >= 0", n);
  ABACUS_CHECK_ARG(n == 0 || (params && grads && exp_avgs && exp_avg_sqs && numels && steps),
                   "adamw: null tensor arrays");
  ABACUS_CHECK_ARG(lr >= 0 && eps >= 0 && weight_decay >= 0 && beta1 >= 0 && beta1 < 1 && beta2 >= 0 && beta2 < 1,
                   "adamw: invalid hyperparameters");
  const int epb = dtype == kBF16 ? AdamwGeo<uint16_t>::EPB : AdamwGeo<float>::EPB;
  const hipStream_t s = (hipStream_t)stream;
  AdamwArgs a{};
  // scalars as the reference's Python floats give them to torch's fp32 math
  a.decay = weight_decay != 0 ? (float)(1.0 - lr * weight_decay) : 1.0f;
  a.w1 = (float)(1.0 - beta1);
  a.beta2 = (float)beta2;
  a.a2 = (float)(1.0 - beta2);
  a.eps = (float)eps;
  // every tensor is checked before anything is launched
  for (int t = 0; t < n; ++t) {
    ABACUS_CHECK_ARG(numels[t] >= 0, "adamw: tensor %d has %lld elements", t, (long long)numels[t]);
    ABACUS_CHECK_ARG(steps[t] >= 1, "adamw: tensor %d step %lld must be >= 1", t, (long long)steps[t]);
    if (numels[t] > 0) {
      const uintptr_t al =
          (uintptr_t)params[t] | (uintptr_t)grads[t] | (uintptr_t)exp_avgs[t] | (uintptr_t)exp_avg_sqs[t];
      ABACUS_CHECK_ARG(params[t] && grads[t] && exp_avgs[t] && exp_avg_sqs[t] && al % 16 == 0,
                       "adamw: tensor %d: null or not 16-byte aligned", t);
      ABACUS_CHECK_ARG((numels[t] + epb - 1) / epb < (1ll << 30), "adamw: tensor %d too large", t);
    }
  }
  for (int first = 0; first < n; first += kAdamwMaxTensors) {
    const int cnt = std::min(kAdamwMaxTensors, n - first);
    int64_t blocks = 0;
    a.n = cnt;
    for (int j = 0; j < cnt; ++j) {
      const int t = first + j;
      a.p[j] = params[t];
      a.g[j] = grads[t];
      a.m[j] = exp_avgs[t];
      a.v[j] = exp_avg_sqs[t];
      a.numel[j] = numels[t];
      const double step = (double)steps[t];
      const double bc1 = 1.0 - std::pow(beta1, step);
      const double bc2 = 1.0 - std::pow(beta2, step);
      a.neg_step_size[j] = (float)(-(lr / bc1));
      a.inv_sqrt_bc2[j] = (float)(1.0 / std::pow(bc2, 0.5));
      a.block_start[j] = (int)blocks;
      blocks += (numels[t] + epb - 1) / epb;
    }
    ABACUS_CHECK_ARG(blocks < (1ll << 31), "adamw: too many elements in one launch");
    a.block_start[cnt] = (int)blocks;
    if (blocks == 0) continue;
    if (dtype == kBF16)
      hipLaunchKernelGGL(adamw_kernel<uint16_t>, dim3((unsigned)blocks), dim3(kAdamwThreads), 0, s, a);
    else
      hipLaunchKernelGGL(adamw_kernel<float>, dim3((unsigned)blocks), dim3(kAdamwThreads), 0, s, a);
    ABACUS_CHECK_LAUNCH("adamw");
  }
  return 0;
}
