// Next-token cross-entropy of the MoE decoder, forward and backward.
//
// Reference: abacus/kernels/liger.py:12-47 (cross_entropy, called at
// trainer.py:81-85): mean over the rows whose target is not ignore_index of
// lse(x_i) - x_i[t_i], as torch.nn.functional.cross_entropy, or liger's fused
// kernel when --liger is set.  Here:
//   forward   one pass over each row: lse_i = log(sum_j exp(x_ij)) in fp32
//             (running max and rescaled sum, base 2), loss_i = lse_i - x_i[t_i]
//             (0 for ignored rows, NaN for a target outside [0, V) that is
//             not ignore_index: the loss shows it, and nothing waits on the host)
//   backward  one pass: dx_ij = g * scale * (exp(x_ij - lse_i) - [j == t_i]),
//             0 on ignored rows, rounded once to the logits' dtype (bf16 pairs by
//             one hardware conversion, round to nearest even); g is read
//             from device memory (the loss's incoming gradient), so nothing
//             waits on the host.
// A row is one wave's: no barriers, and each lane keeps kCeBatch 16-byte
// vectors of loads in flight.  Layout: (N, V) rows, contiguous.
#include <algorithm>
#include <climits>

#include "common.h"

namespace abacus {

namespace {

constexpr int kCeBatch = 4;        // vectors per lane in flight (8 was slower backward)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Logits are read once per pass: nontemporal loads and stores (ld16_stream,
// st16_stream) keep them out of the caches' working set.

// g * exp2(x * log2e - l2) for the 8 bf16 / 4 fp32 elements of a vector,
// stored in the logits' dtype (bf16 pairs by one hardware conversion).
template <typename T> struct CeVec;
template <> struct CeVec<uint16_t> {
  __device__ static inline Vec16 grad(const Vec16& v, float l2, float gs) {
    Vec16 o;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o.w[k] = pack_bf16x2(gs * exp2_fast(__builtin_fmaf(lo_bf16(v.w[k]), kLog2e, -l2)),
                           gs * exp2_fast(__builtin_fmaf(hi_bf16(v.w[k]), kLog2e, -l2)));
    return o;
  }
};
template <> struct CeVec<float> {
  __device__ static inline Vec16 grad(const Vec16& v, float l2, float gs) {
    Vec16 o;
#pragma unroll
    for (int k = 0; k < 4; ++k) o.w[k] = f32_bits(gs * exp2_fast(__builtin_fmaf(bits_f32(v.w[k]), kLog2e, -l2)));
    return o;
  }
};

// (m, s): running max (base-2 scaled units) and sum of exp2(y - m); merge o.
__device__ inline void lse_merge(float& m, float& s, float om, float os) {
  const float mn = fmaxf(m, om);
  if (mn == -__builtin_inff()) return;  // both empty
  s = s * exp2_fast(m - mn) + os * exp2_fast(om - mn);
  m = mn;
}

template <typename T, bool VECOK>
__global__ __launch_bounds__(256) void ce_fwd_kernel(const T* __restrict__ x, const int64_t* __restrict__ tgt,
                                                     int64_t N, int64_t V, int64_t ignore_index,
                                                     float* __restrict__ lse, float* __restrict__ loss) {
  constexpr int VEC = VecTraits<T>::kN;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const T* xr = x + row * V;
  float m = -__builtin_inff(), s = 0.f;
  if (VECOK) {
    const int64_t nvec = V / VEC;
    for (int64_t c0 = 0; c0 < nvec; c0 += 64 * kCeBatch) {
      Vec16 v[kCeBatch];
#pragma unroll
      for (int u = 0; u < kCeBatch; ++u) {
        const int64_t c = c0 + u * 64 + lane;
        v[u] = c < nvec ? ld16_stream(xr + c * VEC) : zero16();
      }
#pragma unroll
      for (int u = 0; u < kCeBatch; ++u) {
        if (c0 + u * 64 + lane >= nvec) continue;
        float xv[VEC], vm = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          xv[i] = VecTraits<T>::get(v[u], i);
          vm = fmaxf(vm, xv[i]);
        }
        const float mn = fmaxf(m, vm * kLog2e);  // running max, base-2 units
        if (mn == -__builtin_inff()) continue;   // nothing above -inf yet
        float vs = 0.f;
#pragma unroll
        for (int i = 0; i < VEC; ++i) vs += exp2_fast(__builtin_fmaf(xv[i], kLog2e, -mn));
        s = s * exp2_fast(m - mn) + vs;  // exp2(-inf) = 0 on the first vector
        m = mn;
      }
    }
  } else {
    for (int64_t j = lane; j < V; j += 64) {
      const float xj = to_f32<T>(xr[j]);
      const float mn = fmaxf(m, xj * kLog2e);
      if (mn == -__builtin_inff()) continue;
      s = s * exp2_fast(m - mn) + exp2_fast(__builtin_fmaf(xj, kLog2e, -mn));
      m = mn;
    }
  }
  // merge the 64 lanes' (m, s) in a fixed butterfly order
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float om = __shfl_xor(m, off, 64), os = __shfl_xor(s, off, 64);
    lse_merge(m, s, om, os);
  }
  if (lane == 0) {
    const float l = (m + __builtin_amdgcn_logf(s)) * kLn2;
    lse[row] = l;
    const int64_t t = tgt[row];
    // a target outside [0, V) that is not ignore_index makes the row's loss NaN (no logit read)
    loss[row] = t == ignore_index ? 0.f : ((t >= 0 && t < V) ? l - to_f32<T>(xr[t]) : __builtin_nanf(""));
  }
}

template <typename T, bool VECOK>
__global__ __launch_bounds__(256) void ce_bwd_kernel(const T* __restrict__ x, const int64_t* __restrict__ tgt,
                                                     const float* __restrict__ lse, const float* __restrict__ grad,
                                                     float scale, int64_t N, int64_t V, int64_t ignore_index,
                                                     T* __restrict__ dx) {
  constexpr int VEC = VecTraits<T>::kN;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const T* xr = x + row * V;
  T* dr = dx + row * V;
  const int64_t t = tgt[row];
  const bool on = t != ignore_index && t >= 0 && t < V;
  const float gs = on ? grad[0] * scale : 0.f;
  const float l = lse[row], l2 = l * kLog2e;
  if (VECOK) {
    const int64_t nvec = V / VEC;
    for (int64_t c0 = 0; c0 < nvec; c0 += 64 * kCeBatch) {
      Vec16 v[kCeBatch];
#pragma unroll
      for (int u = 0; u < kCeBatch; ++u) {
        const int64_t c = c0 + u * 64 + lane;
        v[u] = (on && c < nvec) ? ld16_stream(xr + c * VEC) : zero16();
      }
#pragma unroll
      for (int u = 0; u < kCeBatch; ++u) {
        const int64_t c = c0 + u * 64 + lane;
        if (c >= nvec) continue;
        Vec16 o = on ? CeVec<T>::grad(v[u], l2, gs) : zero16();
        if (on && t / VEC == c) {  // the target's vector: g * (p - 1) there
          const int i = (int)(t - c * VEC);
          const float p = exp2_fast(__builtin_fmaf(VecTraits<T>::get(v[u], i), kLog2e, -l2));
          VecTraits<T>::set(o, i, gs * (p - 1.f));
        }
        st16_stream(dr + c * VEC, o);
      }
    }
  } else {
    for (int64_t j = lane; j < V; j += 64) {
      const float p = on ? exp2_fast(__builtin_fmaf(to_f32<T>(xr[j]), kLog2e, -l2)) : 0.f;
      dr[j] = from_f32<T>(gs * (p - (j == t ? 1.f : 0.f)));
    }
  }
}

int check_ce(const void* x, const int64_t* tgt, int64_t N, int64_t V, int dtype) {
  ABACUS_CHECK_ARG(dtype == kBF16 || dtype == kF32, "cross_entropy: dtype code %d (fp32 or bf16)", dtype);
  ABACUS_CHECK_ARG(N >= 0 && V >= 1 && N <= (int64_t)INT_MAX * 4, "cross_entropy: bad shape (%lld, %lld)",
                   (long long)N, (long long)V);
  ABACUS_CHECK_ARG(N == 0 || (x && tgt), "cross_entropy: null pointer");
  return 0;
}

bool ce_vec_ok(const void* p, int64_t V, int dtype) {
  const int vec = dtype == kBF16 ? 8 : 4;
  return V % vec == 0 && (uintptr_t)p % 16 == 0;
}

}  // namespace
}  // namespace abacus

using namespace abacus;

extern "C" int abacus_cross_entropy_fwd(const void* logits_NV, const int64_t* targets_N, int64_t N, int64_t V,
                                        int64_t ignore_index, int dtype, float* lse_N, float* loss_N,
                                        void* stream) {
  if (check_ce(logits_NV, targets_N, N, V, dtype)) return 1;
  ABACUS_CHECK_ARG(N == 0 || (lse_N && loss_N), "cross_entropy: null pointer");
  if (N == 0) return 0;
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)((N + 3) / 4));
  const bool vec = ce_vec_ok(logits_NV, V, dtype);
#define ABACUS_CE_FWD(TT, VO)                                                                                \
  hipLaunchKernelGGL((ce_fwd_kernel<TT, VO>), grid, dim3(256), 0, s, (const TT*)logits_NV, targets_N, N, V, \
                     ignore_index, lse_N, loss_N)
  if (dtype == kBF16) {
    if (vec) ABACUS_CE_FWD(uint16_t, true);
    else ABACUS_CE_FWD(uint16_t, false);
  } else {
    if (vec) ABACUS_CE_FWD(float, true);
    else ABACUS_CE_FWD(float, false);
  }
#undef ABACUS_CE_FWD
  ABACUS_CHECK_LAUNCH("cross_entropy_fwd");
  return 0;
}

extern "C" int abacus_cross_entropy_bwd(const void* logits_NV, const int64_t* targets_N, const float* lse_N,
                                        const float* grad_loss, float scale, int64_t N, int64_t V,
                                        int64_t ignore_index, int dtype, void* dlogits_NV, void* stream) {
  if (check_ce(logits_NV, targets_N, N, V, dtype)) return 1;
  ABACUS_CHECK_ARG(N == 0 || (lse_N && grad_loss && dlogits_NV), "cross_entropy: null pointer");
  if (N == 0) return 0;
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)((N + 3) / 4));
  const bool vec = ce_vec_ok(logits_NV, V, dtype) && ce_vec_ok(dlogits_NV, V, dtype);
#define ABACUS_CE_BWD(TT, VO)                                                                                \
  hipLaunchKernelGGL((ce_bwd_kernel<TT, VO>), grid, dim3(256), 0, s, (const TT*)logits_NV, targets_N, lse_N, \
                     grad_loss, scale, N, V, ignore_index, (TT*)dlogits_NV)
  if (dtype == kBF16) {
    if (vec) ABACUS_CE_BWD(uint16_t, true);
    else ABACUS_CE_BWD(uint16_t, false);
  } else {
    if (vec) ABACUS_CE_BWD(float, true);
    else ABACUS_CE_BWD(float, false);
  }
#undef ABACUS_CE_BWD
  ABACUS_CHECK_LAUNCH("cross_entropy_bwd");
  return 0;
}
