// Switch-Transformer auxiliary loss (abacus/moe/load_balancing.py:8-41) on the GPU.
//
//   f_E  = (#tokens whose slot list contains e, each token once) / (T * K)
//   p_E  = sum_t probs[t, e] / T                                   (fp32)
//   loss = sum_e f_E * p_E * (coeff * E), returned in the probabilities' dtype
//   d loss / d probs[t, e] = ((g * coeff * E) * f_E[e]) / T        (g: the loss gradient)
//
// One HBM pass: block b reduces a fixed range of tokens to per-expert partial
// sums and counts in the workspace; a one-block finalize adds the partials in
// block order.  No atomics touch global memory, so every result is the same on
// every run.  Expert ids outside [0, E) are reported through a flag word (bit
// 0: negative, bit 1: >= E) for the host to raise on, as torch.one_hot does.
#include <hip/hip_runtime.h>

#include "common.h"

namespace abacus {
namespace {

constexpr int kLbThreads = 256;
constexpr int kLbTokensPerBlock = 2048;
constexpr int kLbMaxE = 4096;

int64_t lb_blocks(int64_t T) { return (T + kLbTokensPerBlock - 1) / kLbTokensPerBlock; }

// Workspace: psum[nb][E] fp32 | cnt[nb][E] int32 | bad[nb] int32
template <typename T>
__global__ __launch_bounds__(kLbThreads) void lb_partial_kernel(const T* __restrict__ probs, const int64_t* __restrict__ slots,
                                                                int64_t Tn, int E, int K, float* psum, int* cnt, int* bad) {
  __shared__ float part[kLbThreads];
  __shared__ int hist[kLbMaxE];
  __shared__ int flag;
  const int tid = threadIdx.x;
  const int64_t t0 = (int64_t)blockIdx.x * kLbTokensPerBlock;
  const int64_t t1 = t0 + kLbTokensPerBlock < Tn ? t0 + kLbTokensPerBlock : Tn;
  for (int e = tid; e < E; e += kLbThreads) hist[e] = 0;
  if (tid == 0) flag = 0;

  // column sums: G row groups of E threads (E <= 256), else each thread owns
  // columns tid, tid + 256, ...; rows in a fixed order either way
  if (E <= kLbThreads) {
    const int G = kLbThreads / E;
    const int g = tid / E, c = tid % E;
    float s = 0.f;
    if (g < G)
      for (int64_t t = t0 + g; t < t1; t += G) s += to_f32<T>(probs[t * E + c]);
    part[tid] = s;
  } else {
    for (int c = tid; c < E; c += kLbThreads) {
      float s = 0.f;
      for (int64_t t = t0; t < t1; ++t) s += to_f32<T>(probs[t * E + c]);
      psum[(int64_t)blockIdx.x * E + c] = s;
    }
  }
  __syncthreads();

  // distinct experts per token (load_balancing.py:36): slot k counts unless an
  // earlier slot of the same token named the same expert
  int my_bad = 0;
  for (int64_t t = t0 + tid; t < t1; t += kLbThreads) {
    const int64_t* row = slots + t * K;
    for (int k = 0; k < K; ++k) {
      const int64_t e = row[k];
      if (e < 0) { my_bad |= 1; continue; }
      if (e >= E) { my_bad |= 2; continue; }
      bool seen = false;
      for (int j = 0; j < k; ++j) seen |= row[j] == e;
      if (!seen) atomicAdd(&hist[e], 1);  // LDS integer atomics: order-independent
    }
  }
  if (my_bad) atomicOr(&flag, my_bad);
  if (E <= kLbThreads) {
    const int G = kLbThreads / E;
    if (tid < E) {
      float s = 0.f;
      for (int g = 0; g < G; ++g) s += part[g * E + tid];
      psum[(int64_t)blockIdx.x * E + tid] = s;
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += kLbThreads) cnt[(int64_t)blockIdx.x * E + e] = hist[e];
  if (tid == 0) bad[blockIdx.x] = flag;
}

template <typename T>
__global__ __launch_bounds__(kLbThreads) void lb_finalize_kernel(const float* psum, const int* cnt, const int* bad, int nb,
                                                                 int64_t Tn, int E, int K, float coeff_e, float* f_E,
                                                                 float* loss_f32, T* loss_out, int* bad_out) {
  __shared__ float prod[kLbThreads];
  __shared__ int flag;
  const int tid = threadIdx.x;
  if (tid == 0) flag = 0;
  __syncthreads();
  const float tk = (float)(Tn * K), tn = (float)Tn;
  float acc = 0.f;  // this thread's columns, in column order
  for (int c = tid; c < E; c += kLbThreads) {
    float p = 0.f;
    int n = 0;
    for (int b = 0; b < nb; ++b) {
      p += psum[(int64_t)b * E + c];
      n += cnt[(int64_t)b * E + c];
    }
    const float f = (float)n / tk;
    f_E[c] = f;
    acc += f * (p / tn);
  }
  prod[tid] = acc;
  int my_bad = 0;
  for (int b = tid; b < nb; b += kLbThreads) my_bad |= bad[b];
  if (my_bad) atomicOr(&flag, my_bad);
  __syncthreads();
  for (int w = kLbThreads / 2; w > 0; w >>= 1) {  // fixed-shape tree
    if (tid < w) prod[tid] += prod[tid + w];
    __syncthreads();
  }
  if (tid == 0) {
    const float loss = prod[0] * coeff_e;
    *loss_f32 = loss;
    *loss_out = from_f32<T>(loss);
    *bad_out = flag;
  }
}

template <typename T>
__global__ __launch_bounds__(kLbThreads) void lb_bwd_kernel(const T* __restrict__ grad_loss, const float* __restrict__ f_E,
                                                            int64_t n, int E, float coeff_e, float tn,
                                                            T* __restrict__ grad) {
  const float gc = to_f32<T>(grad_loss[0]) * coeff_e;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    grad[i] = from_f32<T>((gc * f_E[i % E]) / tn);
}

int check_lb(int64_t T, int64_t E, int64_t K, int dtype) {
  ABACUS_CHECK_ARG(dtype == kF32 || dtype == kBF16, "unsupported dtype code %d (0 = fp32, 1 = bf16)", dtype);
  ABACUS_CHECK_ARG(E >= 1 && E <= kLbMaxE, "n_experts %lld out of range [1, %d]", (long long)E, kLbMaxE);
  ABACUS_CHECK_ARG(T >= 0 && T < (1ll << 40), "tokens %lld out of range", (long long)T);
  ABACUS_CHECK_ARG(K >= 1 && K <= 1024, "expert slots per token %lld out of range [1, 1024]", (long long)K);
  return 0;
}

}  // namespace
}  // namespace abacus

using namespace abacus;

extern "C" {

int64_t abacus_moe_load_balancing_ws_bytes(int64_t T, int64_t E) {
  if (T < 0 || E < 1) return 0;
  const int64_t nb = lb_blocks(T);
  return nb * E * 8 + nb * 4 + 16;
}

int abacus_moe_load_balancing_fwd(const void* probs_TE, const int64_t* slots_TK, int64_t T, int64_t E, int64_t K,
                                  double coeff_e_d, int dtype, void* ws, float* f_E, float* loss_f32, void* loss_out,
                                  int32_t* bad_index, void* stream) {
  const float coeff_e = (float)coeff_e_d;

  if (check_lb(T, E, K, dtype)) return 1;
  ABACUS_CHECK_ARG(T > 0, "no tokens: the loss is zero and needs no launch");
  const int64_t nb = lb_blocks(T);
  ABACUS_CHECK_ARG(nb < (1ll << 31), "too many tokens");
  float* psum = (float*)ws;
  int* cnt = (int*)(psum + nb * E);
  int* bad = cnt + nb * E;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == kBF16) {
    hipLaunchKernelGGL(lb_partial_kernel<uint16_t>, dim3((unsigned)nb), dim3(kLbThreads), 0, s,
                       (const uint16_t*)probs_TE, slots_TK, T, (int)E, (int)K, psum, cnt, bad);
    ABACUS_CHECK_LAUNCH("load_balancing_fwd");
    hipLaunchKernelGGL(lb_finalize_kernel<uint16_t>, dim3(1), dim3(kLbThreads), 0, s, psum, cnt, bad, (int)nb, T,
                       (int)E, (int)K, coeff_e, f_E, loss_f32, (uint16_t*)loss_out, bad_index);
  } else {
    hipLaunchKernelGGL(lb_partial_kernel<float>, dim3((unsigned)nb), dim3(kLbThreads), 0, s, (const float*)probs_TE,
                       slots_TK, T, (int)E, (int)K, psum, cnt, bad);
    ABACUS_CHECK_LAUNCH("load_balancing_fwd");
    hipLaunchKernelGGL(lb_finalize_kernel<float>, dim3(1), dim3(kLbThreads), 0, s, psum, cnt, bad, (int)nb, T, (int)E,
                       (int)K, coeff_e, f_E, loss_f32, (float*)loss_out, bad_index);
  }
  ABACUS_CHECK_LAUNCH("load_balancing_fwd");
  return 0;
}

int abacus_moe_load_balancing_bwd(const void* grad_loss, const float* f_E, int64_t T, int64_t E, double coeff_e_d,
                                  int dtype, void* grad_probs_TE, void* stream) {
  const float coeff_e = (float)coeff_e_d;
  if (check_lb(T, E, 1, dtype)) return 1;
  const int64_t n = T * E;
  if (n == 0) return 0;
  const int64_t want = (n + kLbThreads - 1) / kLbThreads;
  const unsigned blocks = (unsigned)(want < 4096 ? want : 4096);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == kBF16)
    hipLaunchKernelGGL(lb_bwd_kernel<uint16_t>, dim3(blocks), dim3(kLbThreads), 0, s, (const uint16_t*)grad_loss, f_E,
                       n, (int)E, coeff_e, (float)T, (uint16_t*)grad_probs_TE);
  else
    hipLaunchKernelGGL(lb_bwd_kernel<float>, dim3(blocks), dim3(kLbThreads), 0, s, (const float*)grad_loss, f_E, n,
                       (int)E, coeff_e, (float)T, (float*)grad_probs_TE);
  ABACUS_CHECK_LAUNCH("load_balancing_bwd");
  return 0;
}

}  // extern "C"
