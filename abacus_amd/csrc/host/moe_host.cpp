// Host (CPU) build of the libabacus_moe C ABI, for tensors that live on the CPU.
//
// abacus_amd/moe.py calls these entry points for CPU tensors exactly as it calls
// the HIP library (libabacus_moe.so) for GPU tensors: the same names, arguments,
// buffer layouts and rounding steps (a bf16 value is rounded wherever the GPU
// kernels round it), so the module code and the reference's CPU tests
// (tests/test_moe.py, tests/test_moe_ep.py) run unchanged on CPU tensors.  The
// loops are plain C++ with OpenMP over independent rows, tokens or experts;
// every reduction runs in a fixed order, so results do not depend on the thread
// count.  `stream` and the workspace arguments are accepted and ignored: every
// call has finished when it returns.
//
// Reference ops replaced are the ones named in include/abacus_moe.h beside each
// declaration (abacus/moe/router.py:40-70, abacus/moe/moe.py:60-86,
// abacus/moe/load_balancing.py:8-41).
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "abacus_moe.h"

namespace {

enum { kF32 = ABACUS_F32, kBF16 = ABACUS_BF16 };
constexpr int kTokBlock = 16;  // tokens per histogram block (abacus_moe_hist_len)

thread_local char g_error[512] = "";

int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return 1;
}

#define HOST_CHECK(cond, ...) \
  do {                        \
    if (!(cond)) return fail(__VA_ARGS__); \
  } while (0)

// bf16 travels as its 16-bit pattern; rounding is round-to-nearest-even with
// NaN made quiet (the GPU kernels' conversion).
inline float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
inline uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
inline float bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }
inline uint16_t f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <typename T> inline float ld(const T* p, int64_t i);
template <> inline float ld<float>(const float* p, int64_t i) { return p[i]; }
template <> inline float ld<uint16_t>(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
template <typename T> inline void st(T* p, int64_t i, float v);
template <> inline void st<float>(float* p, int64_t i, float v) { p[i] = v; }
template <> inline void st<uint16_t>(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
template <typename T> inline float rnd(float v);
template <> inline float rnd<float>(float v) { return v; }
template <> inline float rnd<uint16_t>(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// sigmoid in fp64, rounded once to fp32 (the router's correctly rounded form)
inline float sigmoid_cr(float x) { return (float)(1.0 / (1.0 + exp(-(double)x))); }
inline float silu_f32(float x) { return x / (1.0f + expf(-x)); }
inline float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

int check_dtype(int dtype) {
  HOST_CHECK(dtype == kF32 || dtype == kBF16, "unsupported dtype code %d (0 = fp32, 1 = bf16)", dtype);
  return 0;
}
int e_pad(int64_t E) { return (int)((E + 15) / 16) * 16; }
int64_t elem(int dtype) { return dtype == kBF16 ? 2 : 4; }

int check_route(int64_t T, int64_t D, int64_t E, int64_t K, int dtype) {
  if (check_dtype(dtype)) return 1;
  HOST_CHECK(T >= 0 && T < (1ll << 31), "token count %lld out of range", (long long)T);
  HOST_CHECK(E >= 1 && E < (1ll << 20), "n_experts %lld out of range", (long long)E);
  HOST_CHECK(K >= 1 && K <= E, "top_k %lld: must be in [1, n_experts]", (long long)K);
  HOST_CHECK(D >= 1 && D < (1ll << 31), "dim %lld out of range", (long long)D);
  HOST_CHECK(T * K < (1ll << 31), "routed rows T*K = %lld exceed int32 indexing", (long long)(T * K));
  return 0;
}

int check_gemm(int64_t R, int64_t D, int64_t M, int64_t E, int dtype) {
  if (check_dtype(dtype)) return 1;
  HOST_CHECK(E >= 1 && E < (1ll << 20), "n_experts %lld out of range", (long long)E);
  HOST_CHECK(R >= 0 && R < (1ll << 31), "routed rows %lld out of range", (long long)R);
  HOST_CHECK(D >= 1 && D < (1ll << 31), "dim %lld out of range", (long long)D);
  HOST_CHECK(M >= 1 && M < (1ll << 31), "hidden_dim %lld out of range", (long long)M);
  return 0;
}

// Expert of each routed row from the expert offsets.
std::vector<int> row_experts(const int32_t* offsets, int64_t R, int64_t E) {
  std::vector<int> ex((size_t)R);
  for (int64_t e = 0; e < E; ++e)
    for (int64_t r = offsets[e]; r < offsets[e + 1] && r < R; ++r) ex[(size_t)r] = (int)e;
  return ex;
}

// Router weights transposed to (E_pad, D) rows, padding rows zero (the layout
// the GPU router leaves in its workspace for the un-permute backward).
template <typename T>
void transpose_router(const T* w, T* wt, int64_t D, int64_t E) {
  const int EP = e_pad(E);
  for (int e = 0; e < EP; ++e)
    for (int64_t d = 0; d < D; ++d) wt[(int64_t)e * D + d] = e < E ? w[d * E + e] : T(0);
}

template <typename T>
void router_fwd(const T* x, const T* w, const T* bias, int64_t Tn, int64_t D, int64_t E, int64_t K, float rho,
                T* logits, T* weights, int64_t* indices, int32_t* idx32, float* score, int32_t* hist, T* wt) {
  transpose_router(w, wt, D, E);
  const int64_t nb = (Tn + kTokBlock - 1) / kTokBlock;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t b = 0; b < nb; ++b) {
    std::vector<float> l((size_t)E), s((size_t)E), sel((size_t)E);
    std::vector<char> taken((size_t)E);
    std::vector<int32_t> cnt((size_t)E, 0);
    for (int64_t t = b * kTokBlock; t < std::min(Tn, (b + 1) * kTokBlock); ++t) {
      for (int64_t e = 0; e < E; ++e) {  // l[e] = x[t] . w[:, e], over d in order
        float acc = 0.f;
        for (int64_t d = 0; d < D; ++d) acc += ld(x, t * D + d) * ld(wt, e * D + d);
        l[(size_t)e] = acc;
      }
      for (int64_t e = 0; e < E; ++e) {
        const float lr = rnd<T>(l[(size_t)e]);
        st(logits, t * E + e, lr);
        s[(size_t)e] = rnd<T>(sigmoid_cr(lr));
        sel[(size_t)e] = rnd<T>(s[(size_t)e] + ld(bias, e));
        taken[(size_t)e] = 0;
      }
      // descending selection value, NaN above every number, ties to the lower expert
      std::vector<float> pk((size_t)K);
      std::vector<int> pe((size_t)K);
      float sum = 0.f;
      for (int64_t k = 0; k < K; ++k) {
        int best_e = -1;
        float best = 0.f;
        bool best_nan = false;
        for (int64_t e = 0; e < E; ++e) {
          if (taken[(size_t)e]) continue;
          const float v = sel[(size_t)e];
          const bool v_nan = v != v;
          if (best_e < 0 || (v_nan && !best_nan) || (!v_nan && !best_nan && v > best)) {
            best_e = (int)e;
            best = v;
            best_nan = v_nan;
          }
        }
        taken[(size_t)best_e] = 1;
        pe[(size_t)k] = best_e;
        pk[(size_t)k] = s[(size_t)best_e];
        sum += pk[(size_t)k];
        cnt[(size_t)best_e] += 1;
      }
      const float denom = rnd<T>(sum);
      for (int64_t k = 0; k < K; ++k) {
        const int64_t o = t * K + k;
        st(weights, o, rnd<T>(rnd<T>(pk[(size_t)k] / denom) * rho));
        indices[o] = pe[(size_t)k];
        idx32[o] = pe[(size_t)k];
        score[o] = pk[(size_t)k];
      }
    }
    for (int64_t e = 0; e < E; ++e) hist[b * E + e] = cnt[(size_t)e];
  }
}

// bias += round(speed * sign(R - E * count)), in the bias dtype (router.py:57-70)
template <typename T>
void bias_step(const int64_t* counts, int64_t E, int64_t R, float speed, T* bias) {
  for (int64_t e = 0; e < E; ++e) {
    const int64_t v = R - counts[e] * E;
    const float step = v > 0 ? 1.0f : (v < 0 ? -1.0f : 0.0f);
    st(bias, e, ld(bias, e) + rnd<T>(speed * step));
  }
}

template <typename T>
void gateup_fwd(const T* xp, const T* wg, const T* wu, const int32_t* offsets, int64_t R, int64_t D, int64_t M,
                int64_t E, T* G, T* U, T* H) {
  const std::vector<int> ex = row_experts(offsets, R, E);
#pragma omp parallel
  {
    std::vector<float> ag((size_t)M), au((size_t)M);
#pragma omp for schedule(static)
    for (int64_t r = 0; r < R; ++r) {
      const int64_t e = ex[(size_t)r];
      std::fill(ag.begin(), ag.end(), 0.f);
      std::fill(au.begin(), au.end(), 0.f);
      for (int64_t d = 0; d < D; ++d) {
        const float xv = ld(xp, r * D + d);
        const int64_t o = (e * D + d) * M;
        for (int64_t m = 0; m < M; ++m) {
          ag[(size_t)m] += xv * ld(wg, o + m);
          au[(size_t)m] += xv * ld(wu, o + m);
        }
      }
      for (int64_t m = 0; m < M; ++m) {
        const float g = rnd<T>(ag[(size_t)m]), u = rnd<T>(au[(size_t)m]);
        if (G) st(G, r * M + m, g);
        if (U) st(U, r * M + m, u);
        st(H, r * M + m, rnd<T>(silu_f32(g)) * u);  // H = round(round(silu(G)) * U)
      }
    }
  }
}

// C[r] = A[r] (K_) . B[e] (K_ x N): rows of a row-grouped product, rounded once
template <typename T>
void rows_times_expert(const T* A, const T* B, const int32_t* offsets, int64_t R, int64_t Kd, int64_t N, int64_t E,
                       T* C) {
  const std::vector<int> ex = row_experts(offsets, R, E);
#pragma omp parallel
  {
    std::vector<float> acc((size_t)N);
#pragma omp for schedule(static)
    for (int64_t r = 0; r < R; ++r) {
      const int64_t e = ex[(size_t)r];
      std::fill(acc.begin(), acc.end(), 0.f);
      for (int64_t k = 0; k < Kd; ++k) {
        const float a = ld(A, r * Kd + k);
        const int64_t o = (e * Kd + k) * N;
        for (int64_t n = 0; n < N; ++n) acc[(size_t)n] += a * ld(B, o + n);
      }
      for (int64_t n = 0; n < N; ++n) st(C, r * N + n, acc[(size_t)n]);
    }
  }
}

// dH = dY . Wd[e]^T, then the SwiGLU backward rounded as the forward rounds
template <typename T>
void down_dgrad(const T* dy, const T* wd, const T* G, const T* U, const int32_t* offsets, int64_t R, int64_t M,
                int64_t D, int64_t E, T* dG, T* dU) {
  const std::vector<int> ex = row_experts(offsets, R, E);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < R; ++r) {
    const int64_t e = ex[(size_t)r];
    for (int64_t m = 0; m < M; ++m) {
      float acc = 0.f;
      const int64_t o = (e * M + m) * D;
      for (int64_t d = 0; d < D; ++d) acc += ld(dy, r * D + d) * ld(wd, o + d);
      const float dh = rnd<T>(acc);
      const float g = ld(G, r * M + m), u = ld(U, r * M + m);
      const float sig = sigmoid_f32(g);
      const float act = rnd<T>(silu_f32(g));
      const float dact = rnd<T>(dh * u);
      st(dG, r * M + m, dact * sig * (1.0f + g * (1.0f - sig)));
      st(dU, r * M + m, dh * act);
    }
  }
}

// dXp = dG . Wg[e]^T + dU . Wu[e]^T over the concatenated reduction (gate half first)
template <typename T>
void gateup_dgrad(const T* dG, const T* dU, const T* wg, const T* wu, const int32_t* offsets, int64_t R, int64_t D,
                  int64_t M, int64_t E, T* dxp) {
  const std::vector<int> ex = row_experts(offsets, R, E);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < R; ++r) {
    const int64_t e = ex[(size_t)r];
    for (int64_t d = 0; d < D; ++d) {
      float acc = 0.f;
      const int64_t o = (e * D + d) * M;
      for (int64_t m = 0; m < M; ++m) acc += ld(dG, r * M + m) * ld(wg, o + m);
      for (int64_t m = 0; m < M; ++m) acc += ld(dU, r * M + m) * ld(wu, o + m);
      st(dxp, r * D + d, acc);
    }
  }
}

// C[e] (P x N) = A_e^T . B_e over expert e's rows (A: rows x P, B: rows x N); zero for empty experts
template <typename T>
void expert_wgrad(const T* A, const T* B, const int32_t* offsets, int64_t P, int64_t N, int64_t E, T* C) {
#pragma omp parallel
  {
    std::vector<float> acc((size_t)N);
#pragma omp for collapse(2) schedule(static)
    for (int64_t e = 0; e < E; ++e)
      for (int64_t p = 0; p < P; ++p) {
        std::fill(acc.begin(), acc.end(), 0.f);
        for (int64_t r = offsets[e]; r < offsets[e + 1]; ++r) {
          const float a = ld(A, r * P + p);
          for (int64_t n = 0; n < N; ++n) acc[(size_t)n] += a * ld(B, r * N + n);
        }
        for (int64_t n = 0; n < N; ++n) st(C, (e * P + p) * N + n, acc[(size_t)n]);
      }
  }
}

// A token's K slots ordered by expert (insertion order among equals), as the
// GPU gather-reduce kernels visit them.
inline void slots_by_expert(const int32_t* idx, int64_t t, int64_t K, std::vector<int>& order) {
  order.resize((size_t)K);
  for (int64_t k = 0; k < K; ++k) order[(size_t)k] = (int)k;
  std::stable_sort(order.begin(), order.end(),
                   [&](int a, int b) { return idx[t * K + a] < idx[t * K + b]; });
}

template <typename T>
void combine_fwd(const T* y, const T* weights, const int32_t* idx, const int32_t* pos, int64_t Tn, int64_t D,
                 int64_t K, T* out) {
#pragma omp parallel
  {
    std::vector<int> order;
    std::vector<float> acc((size_t)D);
#pragma omp for schedule(static)
    for (int64_t t = 0; t < Tn; ++t) {
      slots_by_expert(idx, t, K, order);
      std::fill(acc.begin(), acc.end(), 0.f);
      for (int k : order) {
        const float w = ld(weights, t * K + k);
        const int64_t p = pos[t * K + k];
        for (int64_t d = 0; d < D; ++d) acc[(size_t)d] += rnd<T>(ld(y, p * D + d) * w);
      }
      for (int64_t d = 0; d < D; ++d) st(out, t * D + d, acc[(size_t)d]);
    }
  }
}

// dL/dweights -> dL/dlogit for one token (router.py:45,49-51)
inline void gating_bwd(int64_t K, float rho, const float* dw, const float* w, const float* s, float denom,
                       float* dl) {
  float c = 0.f;
  for (int64_t k = 0; k < K; ++k) c += dw[k] * w[k];
  for (int64_t k = 0; k < K; ++k) dl[k] = (rho * dw[k] - c) / denom * s[k] * (1.0f - s[k]);
}

template <typename T>
void combine_bwd(const T* dout, const T* y, const T* weights, const float* score, const int32_t* pos, int64_t Tn,
                 int64_t D, int64_t K, float rho, T* dy, float* dlogit) {
#pragma omp parallel
  {
    std::vector<float> w((size_t)K), dw((size_t)K), sc((size_t)K), dl((size_t)K);
#pragma omp for schedule(static)
    for (int64_t t = 0; t < Tn; ++t) {
      float sum = 0.f;
      for (int64_t k = 0; k < K; ++k) {
        w[(size_t)k] = ld(weights, t * K + k);
        const int64_t p = pos[t * K + k];
        float dot = 0.f;
        for (int64_t d = 0; d < D; ++d) {
          const float g = ld(dout, t * D + d);
          dot += g * ld(y, p * D + d);
          st(dy, p * D + d, g * w[(size_t)k]);
        }
        dw[(size_t)k] = dot;
        sc[(size_t)k] = score[t * K + k];
        sum += sc[(size_t)k];
      }
      gating_bwd(K, rho, dw.data(), w.data(), sc.data(), rnd<T>(sum), dl.data());
      for (int64_t k = 0; k < K; ++k) dlogit[t * K + k] = dl[(size_t)k];
    }
  }
}

template <typename T>
void unpermute_bwd(const T* dxp, const float* dlogit, const int32_t* idx, const int32_t* pos, const T* wt,
                   int64_t Tn, int64_t D, int64_t K, T* dx) {
#pragma omp parallel
  {
    std::vector<int> order;
    std::vector<float> acc((size_t)D);
#pragma omp for schedule(static)
    for (int64_t t = 0; t < Tn; ++t) {
      slots_by_expert(idx, t, K, order);
      std::fill(acc.begin(), acc.end(), 0.f);
      for (int k : order) {
        const int64_t e = idx[t * K + k];
        const float dl = dlogit[t * K + k];
        for (int64_t d = 0; d < D; ++d) {
          if (dxp) acc[(size_t)d] += ld(dxp, (int64_t)pos[t * K + k] * D + d);
          acc[(size_t)d] += dl * ld(wt, e * D + d);
        }
      }
      for (int64_t d = 0; d < D; ++d) st(dx, t * D + d, acc[(size_t)d]);
    }
  }
}

// dW_DE[d][e] = sum_t x[t][d] * dlogit(t, e), tokens in order
template <typename T>
void router_wgrad(const T* x, const float* dlogit, const int32_t* idx, int64_t Tn, int64_t D, int64_t E, int64_t K,
                  T* dw) {
#pragma omp parallel
  {
    std::vector<float> acc((size_t)E);
#pragma omp for schedule(static)
    for (int64_t d = 0; d < D; ++d) {
      std::fill(acc.begin(), acc.end(), 0.f);
      for (int64_t t = 0; t < Tn; ++t) {
        const float xv = ld(x, t * D + d);
        for (int64_t k = 0; k < K; ++k) acc[(size_t)idx[t * K + k]] += xv * dlogit[t * K + k];
      }
      for (int64_t e = 0; e < E; ++e) st(dw, d * E + e, acc[(size_t)e]);
    }
  }
}

}  // namespace

#define TP(T, p) ((T*)(p))

extern "C" {

const char* abacus_moe_last_error(void) { return g_error; }
int abacus_moe_abi_version(void) { return 4; }

int64_t abacus_moe_hist_len(int64_t T, int64_t E) { return ((T + kTokBlock - 1) / kTokBlock) * E; }
int64_t abacus_moe_router_ws_bytes(int64_t D, int64_t E, int dtype) { return (int64_t)e_pad(E) * D * elem(dtype); }
int64_t abacus_moe_router_wgrad_ws_bytes(int64_t, int64_t, int64_t, int) { return 0; }
int64_t abacus_moe_down_fwd_ws_bytes(int64_t, int64_t, int64_t, int64_t, int) { return 0; }

int abacus_moe_router_fwd(const void* x_TD, const void* w_DE, const void* bias_E, int64_t T, int64_t D, int64_t E,
                          int64_t K, float route_scale, int dtype, void* logits_TE, void* weights_TK,
                          int64_t* indices_TK_i64, int32_t* idx_TK, float* score_TK, int32_t* hist, void* wt_ws,
                          void*) {
  if (check_route(T, D, E, K, dtype)) return 1;
  HOST_CHECK(wt_ws != nullptr, "router_fwd: router weight workspace is NULL");
  if (dtype == kBF16)
    router_fwd<uint16_t>(TP(const uint16_t, x_TD), TP(const uint16_t, w_DE), TP(const uint16_t, bias_E), T, D, E, K,
                         route_scale, TP(uint16_t, logits_TE), TP(uint16_t, weights_TK), indices_TK_i64, idx_TK,
                         score_TK, hist, TP(uint16_t, wt_ws));
  else
    router_fwd<float>(TP(const float, x_TD), TP(const float, w_DE), TP(const float, bias_E), T, D, E, K, route_scale,
                      TP(float, logits_TE), TP(float, weights_TK), indices_TK_i64, idx_TK, score_TK, hist,
                      TP(float, wt_ws));
  return 0;
}

int abacus_moe_route_scan(const int32_t* hist, int64_t T, int64_t E, int64_t K, void* bias_E, float speed, int dtype,
                          int32_t* base, int32_t* counts_E, int32_t* offsets_E1, void*) {
  if (check_dtype(dtype)) return 1;
  HOST_CHECK(E >= 1 && T >= 0 && T * K < (1ll << 31), "route_scan: bad sizes T=%lld E=%lld K=%lld", (long long)T,
             (long long)E, (long long)K);
  const int64_t nb = (T + kTokBlock - 1) / kTokBlock;
  std::vector<int64_t> cnt((size_t)E, 0);
  for (int64_t b = 0; b < nb; ++b)
    for (int64_t e = 0; e < E; ++e) cnt[(size_t)e] += hist[b * E + e];
  int64_t run = 0;
  for (int64_t e = 0; e < E; ++e) {
    counts_E[e] = (int32_t)cnt[(size_t)e];
    offsets_E1[e] = (int32_t)run;
    int64_t r = run;
    for (int64_t b = 0; b < nb; ++b) {
      base[b * E + e] = (int32_t)r;
      r += hist[b * E + e];
    }
    run += cnt[(size_t)e];
  }
  offsets_E1[E] = (int32_t)run;
  if (bias_E != nullptr) {
    if (dtype == kBF16) bias_step<uint16_t>(cnt.data(), E, T * K, speed, TP(uint16_t, bias_E));
    else bias_step<float>(cnt.data(), E, T * K, speed, TP(float, bias_E));
  }
  return 0;
}

int abacus_moe_permute_gather(const void* x_TD, const int32_t* idx_TK, const int32_t* base, int64_t T, int64_t D,
                              int64_t E, int64_t K, int dtype, int32_t* pos_TK, int32_t* perm_R, void* x_perm_RD,
                              void*) {
  if (check_route(T, D, E, K, dtype)) return 1;
  const int64_t nb = (T + kTokBlock - 1) / kTokBlock;
  const int64_t row_bytes = D * elem(dtype);
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < nb; ++b) {
    std::vector<int32_t> rank((size_t)E, 0);
    for (int64_t t = b * kTokBlock; t < std::min(T, (b + 1) * kTokBlock); ++t)
      for (int64_t k = 0; k < K; ++k) {
        const int64_t e = idx_TK[t * K + k];
        const int32_t p = base[b * E + e] + rank[(size_t)e]++;
        pos_TK[t * K + k] = p;
        perm_R[p] = (int32_t)t;
        memcpy((char*)x_perm_RD + p * row_bytes, (const char*)x_TD + t * row_bytes, (size_t)row_bytes);
      }
  }
  return 0;
}

int abacus_moe_dispatch(const int32_t* hist, const void* x_TD, const int32_t* idx_TK, int64_t T, int64_t D,
                        int64_t E, int64_t K, void* bias_E, float speed, int dtype, int32_t* counts_E,
                        int32_t* offsets_E1, int32_t* pos_TK, int32_t* perm_R, void* x_perm_RD, int32_t* base_ws,
                        void* stream) {
  if (abacus_moe_route_scan(hist, T, E, K, bias_E, speed, dtype, base_ws, counts_E, offsets_E1, stream)) return 1;
  return abacus_moe_permute_gather(x_TD, idx_TK, base_ws, T, D, E, K, dtype, pos_TK, perm_R, x_perm_RD, stream);
}

int abacus_moe_gateup_fwd(const void* x_perm_RD, const void* w_gate_EDM, const void* w_up_EDM,
                          const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M, int64_t E, int dtype,
                          void* gate_RM, void* up_RM, void* h_RM, void*) {
  if (check_gemm(R, D, M, E, dtype)) return 1;
  if (dtype == kBF16)
    gateup_fwd<uint16_t>(TP(const uint16_t, x_perm_RD), TP(const uint16_t, w_gate_EDM), TP(const uint16_t, w_up_EDM),
                         offsets_E1, R, D, M, E, TP(uint16_t, gate_RM), TP(uint16_t, up_RM), TP(uint16_t, h_RM));
  else
    gateup_fwd<float>(TP(const float, x_perm_RD), TP(const float, w_gate_EDM), TP(const float, w_up_EDM), offsets_E1,
                      R, D, M, E, TP(float, gate_RM), TP(float, up_RM), TP(float, h_RM));
  return 0;
}

int abacus_moe_down_fwd(const void* h_RM, const void* w_down_EMD, const int32_t* offsets_E1, int64_t R, int64_t M,
                        int64_t D, int64_t E, int dtype, void* y_RD, void*, int64_t, void*) {
  if (check_gemm(R, D, M, E, dtype)) return 1;
  if (dtype == kBF16)
    rows_times_expert<uint16_t>(TP(const uint16_t, h_RM), TP(const uint16_t, w_down_EMD), offsets_E1, R, M, D, E,
                                TP(uint16_t, y_RD));
  else
    rows_times_expert<float>(TP(const float, h_RM), TP(const float, w_down_EMD), offsets_E1, R, M, D, E,
                             TP(float, y_RD));
  return 0;
}

int abacus_moe_combine_fwd(const void* y_RD, const void* weights_TK, const int32_t* idx_TK, const int32_t* pos_TK,
                           int64_t T, int64_t D, int64_t K, int dtype, void* out_TD, void*) {
  if (check_route(T, D, K, K, dtype)) return 1;
  if (dtype == kBF16)
    combine_fwd<uint16_t>(TP(const uint16_t, y_RD), TP(const uint16_t, weights_TK), idx_TK, pos_TK, T, D, K,
                          TP(uint16_t, out_TD));
  else
    combine_fwd<float>(TP(const float, y_RD), TP(const float, weights_TK), idx_TK, pos_TK, T, D, K, TP(float, out_TD));
  return 0;
}

int abacus_moe_combine_bwd(const void* dout_TD, const void* y_RD, const void* weights_TK, const float* score_TK,
                           const int32_t* pos_TK, int64_t T, int64_t D, int64_t K, float route_scale, int dtype,
                           void* dy_RD, float* dlogit_TK, void*) {
  if (check_route(T, D, K, K, dtype)) return 1;
  if (dtype == kBF16)
    combine_bwd<uint16_t>(TP(const uint16_t, dout_TD), TP(const uint16_t, y_RD), TP(const uint16_t, weights_TK),
                          score_TK, pos_TK, T, D, K, route_scale, TP(uint16_t, dy_RD), dlogit_TK);
  else
    combine_bwd<float>(TP(const float, dout_TD), TP(const float, y_RD), TP(const float, weights_TK), score_TK, pos_TK,
                       T, D, K, route_scale, TP(float, dy_RD), dlogit_TK);
  return 0;
}

int abacus_moe_down_bwd_dgrad(const void* dy_RD, const void* w_down_EMD, const void* gate_RM, const void* up_RM,
                              const int32_t* offsets_E1, int64_t R, int64_t M, int64_t D, int64_t E, int dtype,
                              void* dgate_RM, void* dup_RM, void*) {
  if (check_gemm(R, D, M, E, dtype)) return 1;
  if (dtype == kBF16)
    down_dgrad<uint16_t>(TP(const uint16_t, dy_RD), TP(const uint16_t, w_down_EMD), TP(const uint16_t, gate_RM),
                         TP(const uint16_t, up_RM), offsets_E1, R, M, D, E, TP(uint16_t, dgate_RM),
                         TP(uint16_t, dup_RM));
  else
    down_dgrad<float>(TP(const float, dy_RD), TP(const float, w_down_EMD), TP(const float, gate_RM),
                      TP(const float, up_RM), offsets_E1, R, M, D, E, TP(float, dgate_RM), TP(float, dup_RM));
  return 0;
}

int abacus_moe_down_bwd_wgrad(const void* h_RM, const void* dy_RD, const int32_t* offsets_E1, int64_t R, int64_t M,
                              int64_t D, int64_t E, int dtype, void* dw_down_EMD, int32_t* tile_ctr, void*) {
  if (check_gemm(R, D, M, E, dtype)) return 1;
  HOST_CHECK(tile_ctr != nullptr, "tile_ctr workspace is NULL");
  if (dtype == kBF16)
    expert_wgrad<uint16_t>(TP(const uint16_t, h_RM), TP(const uint16_t, dy_RD), offsets_E1, M, D, E,
                           TP(uint16_t, dw_down_EMD));
  else
    expert_wgrad<float>(TP(const float, h_RM), TP(const float, dy_RD), offsets_E1, M, D, E, TP(float, dw_down_EMD));
  return 0;
}

int abacus_moe_down_bwd(const void* dy_RD, const void* w_down_EMD, const void* gate_RM, const void* up_RM,
                        const void* h_RM, const int32_t* offsets_E1, int64_t R, int64_t M, int64_t D, int64_t E,
                        int dtype, void* dgate_RM, void* dup_RM, void* dw_down_EMD, int32_t* tile_ctr, void* s) {
  if (abacus_moe_down_bwd_dgrad(dy_RD, w_down_EMD, gate_RM, up_RM, offsets_E1, R, M, D, E, dtype, dgate_RM, dup_RM,
                                s))
    return 1;
  return abacus_moe_down_bwd_wgrad(h_RM, dy_RD, offsets_E1, R, M, D, E, dtype, dw_down_EMD, tile_ctr, s);
}

int abacus_moe_gateup_bwd_dgrad(const void* dgate_RM, const void* dup_RM, const void* w_gate_EDM,
                                const void* w_up_EDM, const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M,
                                int64_t E, int dtype, void* dx_perm_RD, void*) {
  if (check_gemm(R, D, M, E, dtype)) return 1;
  if (dtype == kBF16)
    gateup_dgrad<uint16_t>(TP(const uint16_t, dgate_RM), TP(const uint16_t, dup_RM), TP(const uint16_t, w_gate_EDM),
                           TP(const uint16_t, w_up_EDM), offsets_E1, R, D, M, E, TP(uint16_t, dx_perm_RD));
  else
    gateup_dgrad<float>(TP(const float, dgate_RM), TP(const float, dup_RM), TP(const float, w_gate_EDM),
                        TP(const float, w_up_EDM), offsets_E1, R, D, M, E, TP(float, dx_perm_RD));
  return 0;
}

int abacus_moe_gateup_bwd_wgrad(const void* x_perm_RD, const void* dgate_RM, const void* dup_RM,
                                const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M, int64_t E, int dtype,
                                void* dw_gate_EDM, void* dw_up_EDM, int32_t* tile_ctr, void*) {
  if (check_gemm(R, D, M, E, dtype)) return 1;
  HOST_CHECK(tile_ctr != nullptr, "tile_ctr workspace is NULL");
  if (dtype == kBF16) {
    expert_wgrad<uint16_t>(TP(const uint16_t, x_perm_RD), TP(const uint16_t, dgate_RM), offsets_E1, D, M, E,
                           TP(uint16_t, dw_gate_EDM));
    expert_wgrad<uint16_t>(TP(const uint16_t, x_perm_RD), TP(const uint16_t, dup_RM), offsets_E1, D, M, E,
                           TP(uint16_t, dw_up_EDM));
  } else {
    expert_wgrad<float>(TP(const float, x_perm_RD), TP(const float, dgate_RM), offsets_E1, D, M, E,
                        TP(float, dw_gate_EDM));
    expert_wgrad<float>(TP(const float, x_perm_RD), TP(const float, dup_RM), offsets_E1, D, M, E,
                        TP(float, dw_up_EDM));
  }
  return 0;
}

int abacus_moe_gateup_bwd(const void* dgate_RM, const void* dup_RM, const void* w_gate_EDM, const void* w_up_EDM,
                          const void* x_perm_RD, const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M,
                          int64_t E, int dtype, void* dx_perm_RD, void* dw_gate_EDM, void* dw_up_EDM,
                          int32_t* tile_ctr, void* s) {
  if (abacus_moe_gateup_bwd_dgrad(dgate_RM, dup_RM, w_gate_EDM, w_up_EDM, offsets_E1, R, D, M, E, dtype, dx_perm_RD,
                                  s))
    return 1;
  return abacus_moe_gateup_bwd_wgrad(x_perm_RD, dgate_RM, dup_RM, offsets_E1, R, D, M, E, dtype, dw_gate_EDM,
                                     dw_up_EDM, tile_ctr, s);
}

int abacus_moe_unpermute_bwd(const void* dx_perm_RD, const float* dlogit_TK, const int32_t* idx_TK,
                             const int32_t* pos_TK, const void* w_DE, void* wt_ws, int64_t T, int64_t D, int64_t E,
                             int64_t K, int dtype, void* dx_TD, void*) {
  if (check_route(T, D, E, K, dtype)) return 1;
  HOST_CHECK(wt_ws != nullptr, "unpermute_bwd: router weight workspace is NULL");
  if (dtype == kBF16) {
    if (w_DE) transpose_router(TP(const uint16_t, w_DE), TP(uint16_t, wt_ws), D, E);
    unpermute_bwd<uint16_t>(TP(const uint16_t, dx_perm_RD), dlogit_TK, idx_TK, pos_TK, TP(const uint16_t, wt_ws), T,
                            D, K, TP(uint16_t, dx_TD));
  } else {
    if (w_DE) transpose_router(TP(const float, w_DE), TP(float, wt_ws), D, E);
    unpermute_bwd<float>(TP(const float, dx_perm_RD), dlogit_TK, idx_TK, pos_TK, TP(const float, wt_ws), T, D, K,
                         TP(float, dx_TD));
  }
  return 0;
}

int abacus_moe_router_wgrad(const void* x_TD, const float* dlogit_TK, const int32_t* idx_TK, int64_t T, int64_t D,
                            int64_t E, int64_t K, int dtype, float*, void* dw_DE, void*) {
  if (check_route(T, D, E, K, dtype)) return 1;
  if (dtype == kBF16)
    router_wgrad<uint16_t>(TP(const uint16_t, x_TD), dlogit_TK, idx_TK, T, D, E, K, TP(uint16_t, dw_DE));
  else
    router_wgrad<float>(TP(const float, x_TD), dlogit_TK, idx_TK, T, D, E, K, TP(float, dw_DE));
  return 0;
}

int abacus_moe_router_wgrad_noalloc(const void* x_TD, const float* dlogit_TK, const int32_t* idx_TK, int64_t T,
                                    int64_t D, int64_t E, int64_t K, int dtype, void* dw_DE, void* s) {
  return abacus_moe_router_wgrad(x_TD, dlogit_TK, idx_TK, T, D, E, K, dtype, nullptr, dw_DE, s);
}

int abacus_router_gating_bwd(const void* dweights_TK, const void* weights_TK, const float* score_TK, int64_t T,
                             int64_t K, float route_scale, int dtype, float* dlogit_TK, void*) {
  if (check_dtype(dtype)) return 1;
  HOST_CHECK(K >= 1 && T >= 0, "router_gating_bwd: bad sizes T=%lld K=%lld", (long long)T, (long long)K);
#pragma omp parallel
  {
    std::vector<float> dw((size_t)K), w((size_t)K), sc((size_t)K);
#pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      float sum = 0.f;
      for (int64_t k = 0; k < K; ++k) {
        const int64_t o = t * K + k;
        dw[(size_t)k] = dtype == kBF16 ? ld(TP(const uint16_t, dweights_TK), o) : ld(TP(const float, dweights_TK), o);
        w[(size_t)k] = dtype == kBF16 ? ld(TP(const uint16_t, weights_TK), o) : ld(TP(const float, weights_TK), o);
        sc[(size_t)k] = score_TK[o];
        sum += sc[(size_t)k];
      }
      const float denom = dtype == kBF16 ? rnd<uint16_t>(sum) : sum;
      gating_bwd(K, route_scale, dw.data(), w.data(), sc.data(), denom, dlogit_TK + t * K);
    }
  }
  return 0;
}

int abacus_router_update_bias(const int64_t* indices, int64_t N, int64_t E, float speed, int dtype, void* bias_E,
                              void*) {
  if (check_dtype(dtype)) return 1;
  HOST_CHECK(E >= 1 && N >= 0, "update_bias: bad sizes N=%lld E=%lld", (long long)N, (long long)E);
  std::vector<int64_t> cnt((size_t)E, 0);
  for (int64_t i = 0; i < N; ++i) {
    HOST_CHECK(indices[i] >= 0 && indices[i] < E, "update_bias: expert index %lld out of range [0, %lld)",
               (long long)indices[i], (long long)E);
    cnt[(size_t)indices[i]] += 1;
  }
  if (dtype == kBF16) bias_step<uint16_t>(cnt.data(), E, N, speed, TP(uint16_t, bias_E));
  else bias_step<float>(cnt.data(), E, N, speed, TP(float, bias_E));
  return 0;
}

int64_t abacus_moe_load_balancing_ws_bytes(int64_t, int64_t) { return 0; }

int abacus_moe_load_balancing_fwd(const void* probs_TE, const int64_t* slots_TK, int64_t T, int64_t E, int64_t K,
                                  float coeff_e, int dtype, void*, float* f_E, float* loss_f32, void* loss_out,
                                  int32_t* bad_index, void*) {
  if (check_dtype(dtype)) return 1;
  HOST_CHECK(E >= 1 && T > 0 && K >= 1, "load_balancing_fwd: bad sizes T=%lld E=%lld K=%lld", (long long)T,
             (long long)E, (long long)K);
  std::vector<int64_t> n((size_t)E, 0);
  int bad = 0;
  for (int64_t t = 0; t < T; ++t)
    for (int64_t k = 0; k < K; ++k) {
      const int64_t e = slots_TK[t * K + k];
      if (e < 0) { bad |= 1; continue; }
      if (e >= E) { bad |= 2; continue; }
      bool seen = false;
      for (int64_t j = 0; j < k; ++j) seen |= slots_TK[t * K + j] == e;
      if (!seen) n[(size_t)e] += 1;
    }
  const float tk = (float)(T * K), tn = (float)T;
  float acc = 0.f;
  for (int64_t e = 0; e < E; ++e) {
    float p = 0.f;
    for (int64_t t = 0; t < T; ++t)
      p += dtype == kBF16 ? ld(TP(const uint16_t, probs_TE), t * E + e) : ld(TP(const float, probs_TE), t * E + e);
    const float f = (float)n[(size_t)e] / tk;
    f_E[e] = f;
    acc += f * (p / tn);
  }
  const float loss = acc * coeff_e;
  *loss_f32 = loss;
  if (dtype == kBF16) *TP(uint16_t, loss_out) = f32_to_bf16(loss);
  else *TP(float, loss_out) = loss;
  *bad_index = bad;
  return 0;
}

int abacus_moe_load_balancing_bwd(const void* grad_loss, const float* f_E, int64_t T, int64_t E, float coeff_e,
                                  int dtype, void* grad_probs_TE, void*) {
  if (check_dtype(dtype)) return 1;
  const float g = dtype == kBF16 ? ld(TP(const uint16_t, grad_loss), 0) : ld(TP(const float, grad_loss), 0);
  const float gc = g * coeff_e, tn = (float)T;
  for (int64_t i = 0; i < T * E; ++i) {
    const float v = (gc * f_E[i % E]) / tn;
    if (dtype == kBF16) TP(uint16_t, grad_probs_TE)[i] = f32_to_bf16(v);
    else TP(float, grad_probs_TE)[i] = v;
  }
  return 0;
}

}  // extern "C"
