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

// fp16 (ABACUS_F16) travels as its 16-bit IEEE binary16 pattern in a struct of
// its own (bf16 is the bare uint16_t).  Conversions: binary16 -> fp32 exactly;
// fp32 -> binary16 rounds to nearest even, with subnormals, overflow to
// infinity and NaN made quiet, as torch's float-to-half cast.
struct half_t {
  uint16_t bits;
};
inline float half_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    const float v = (float)m * 5.9604644775390625e-08f;  // m * 2^-24, exact
    return sign ? -v : v;
  }
  if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
  return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}
inline uint16_t f32_to_half(float f) {
  const uint32_t x = f32_bits(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));  // NaN, quiet
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to infinity (|f| >= 65520)
  if (ax < 0x38800000u) {  // below the smallest normal (2^-14): multiples of 2^-24, nearest even
    const float scaled = bits_f32(ax) * 16777216.0f;  // exact
    return (uint16_t)(sign | (uint16_t)lrintf(scaled));
  }
  uint32_t r = ax - 0x38000000u;  // exponent rebiased from 127 to 15
  r += 0xfffu + ((r >> 13) & 1u);
  return (uint16_t)(sign | (r >> 13));
}

// Per storage type: the compute type A (fp64 computes in double, the others in
// fp32 as the GPU kernels do), loads widened to A, stores and roundings to T.
template <typename T> struct Acc { using type = float; };
template <> struct Acc<double> { using type = double; };
template <typename T> using acc_t = typename Acc<T>::type;

template <typename T> inline acc_t<T> ld(const T* p, int64_t i);
template <> inline float ld<float>(const float* p, int64_t i) { return p[i]; }
template <> inline float ld<uint16_t>(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
template <> inline float ld<half_t>(const half_t* p, int64_t i) { return half_to_f32(p[i].bits); }
template <> inline double ld<double>(const double* p, int64_t i) { return p[i]; }
template <typename T> inline void st(T* p, int64_t i, acc_t<T> v);
template <> inline void st<float>(float* p, int64_t i, float v) { p[i] = v; }
template <> inline void st<uint16_t>(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
template <> inline void st<half_t>(half_t* p, int64_t i, float v) { p[i].bits = f32_to_half(v); }
template <> inline void st<double>(double* p, int64_t i, double v) { p[i] = v; }
template <typename T> inline acc_t<T> rnd(acc_t<T> v);
template <> inline float rnd<float>(float v) { return v; }
template <> inline float rnd<uint16_t>(float v) { return bf16_to_f32(f32_to_bf16(v)); }
template <> inline float rnd<half_t>(float v) { return half_to_f32(f32_to_half(v)); }
template <> inline double rnd<double>(double v) { return v; }
// A zero of the storage type (the transposed router weight's padding rows).
template <typename T> inline T zero_of() { return T(0); }
template <> inline half_t zero_of<half_t>() { return half_t{0}; }

// The router's sigmoid: in fp64, rounded once to fp32 (correctly rounded) for
// the fp32-computing types; in fp64 for fp64.
inline float sigmoid_sel(float x) { return (float)(1.0 / (1.0 + exp(-(double)x))); }
inline double sigmoid_sel(double x) { return 1.0 / (1.0 + exp(-x)); }
inline float silu_a(float x) { return x / (1.0f + expf(-x)); }
inline double silu_a(double x) { return x / (1.0 + exp(-x)); }
inline float sigmoid_a(float x) { return 1.0f / (1.0f + expf(-x)); }
inline double sigmoid_a(double x) { return 1.0 / (1.0 + exp(-x)); }

enum { kF64 = ABACUS_F64, kF16 = ABACUS_F16 };

int check_dtype(int dtype) {
  HOST_CHECK(dtype == kF32 || dtype == kBF16 || dtype == kF64 || dtype == kF16,
             "unsupported dtype code %d (0 = fp32, 1 = bf16, 2 = fp64, 3 = fp16)", dtype);
  return 0;
}
int e_pad(int64_t E) { return (int)((E + 15) / 16) * 16; }
int64_t elem(int dtype) { return dtype == kF64 ? 8 : (dtype == kF32 ? 4 : 2); }

// f(T()) with T the storage type of `dtype` (checked before).
template <typename F>
void with_type(int dtype, F&& f) {
  switch (dtype) {
    case kBF16: f(uint16_t()); break;
    case kF64: f(double()); break;
    case kF16: f(half_t{0}); break;
    default: f(float()); break;
  }
}

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
    for (int64_t d = 0; d < D; ++d) wt[(int64_t)e * D + d] = e < E ? w[d * E + e] : zero_of<T>();
}

// score_TK is acc_t<T> (fp32, or fp64 for fp64); rho is cast to acc_t<T>, as a
// Python scalar meets a tensor of that dtype in torch.
template <typename T>
void router_fwd(const T* x, const T* w, const T* bias, int64_t Tn, int64_t D, int64_t E, int64_t K, double rho_in,
                T* logits, T* weights, int64_t* indices, int32_t* idx32, acc_t<T>* score, int32_t* hist, T* wt) {
  using A = acc_t<T>;
  const A rho = (A)rho_in;
  transpose_router(w, wt, D, E);
  const int64_t nb = (Tn + kTokBlock - 1) / kTokBlock;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t b = 0; b < nb; ++b) {
    std::vector<A> l((size_t)E), s((size_t)E), sel((size_t)E);
    std::vector<char> taken((size_t)E);
    std::vector<int32_t> cnt((size_t)E, 0);
    for (int64_t t = b * kTokBlock; t < std::min(Tn, (b + 1) * kTokBlock); ++t) {
      for (int64_t e = 0; e < E; ++e) {  // l[e] = x[t] . w[:, e], over d in order
        A acc = 0;
        for (int64_t d = 0; d < D; ++d) acc += ld(x, t * D + d) * ld(wt, e * D + d);
        l[(size_t)e] = acc;
      }
      for (int64_t e = 0; e < E; ++e) {
        const A lr = rnd<T>(l[(size_t)e]);
        st(logits, t * E + e, lr);
        s[(size_t)e] = rnd<T>(sigmoid_sel(lr));
        sel[(size_t)e] = rnd<T>(s[(size_t)e] + ld(bias, e));
        taken[(size_t)e] = 0;
      }
      // descending selection value, NaN above every number, ties to the lower expert
      std::vector<A> pk((size_t)K);
      std::vector<int> pe((size_t)K);
      A sum = 0;
      for (int64_t k = 0; k < K; ++k) {
        int best_e = -1;
        A best = 0;
        bool best_nan = false;
        for (int64_t e = 0; e < E; ++e) {
          if (taken[(size_t)e]) continue;
          const A v = sel[(size_t)e];
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
      const A denom = rnd<T>(sum);
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
void bias_step(const int64_t* counts, int64_t E, int64_t R, double speed_in, T* bias) {
  using A = acc_t<T>;
  const A speed = (A)speed_in;
  for (int64_t e = 0; e < E; ++e) {
    const int64_t v = R - counts[e] * E;
    const A step = v > 0 ? A(1) : (v < 0 ? A(-1) : A(0));
    st(bias, e, ld(bias, e) + rnd<T>(speed * step));
  }
}

template <typename T>
void gateup_fwd(const T* xp, const T* wg, const T* wu, const int32_t* offsets, int64_t R, int64_t D, int64_t M,
                int64_t E, T* G, T* U, T* H) {
  using A = acc_t<T>;
  const std::vector<int> ex = row_experts(offsets, R, E);
#pragma omp parallel
  {
    std::vector<A> ag((size_t)M), au((size_t)M);
#pragma omp for schedule(static)
    for (int64_t r = 0; r < R; ++r) {
      const int64_t e = ex[(size_t)r];
      std::fill(ag.begin(), ag.end(), A(0));
      std::fill(au.begin(), au.end(), A(0));
      for (int64_t d = 0; d < D; ++d) {
        const A xv = ld(xp, r * D + d);
        const int64_t o = (e * D + d) * M;
        for (int64_t m = 0; m < M; ++m) {
          ag[(size_t)m] += xv * ld(wg, o + m);
          au[(size_t)m] += xv * ld(wu, o + m);
        }
      }
      for (int64_t m = 0; m < M; ++m) {
        const A g = rnd<T>(ag[(size_t)m]), u = rnd<T>(au[(size_t)m]);
        if (G) st(G, r * M + m, g);
        if (U) st(U, r * M + m, u);
        st(H, r * M + m, rnd<T>(silu_a(g)) * u);  // H = round(round(silu(G)) * U)
      }
    }
  }
}

// C[r] = A[r] (K_) . B[e] (K_ x N): rows of a row-grouped product, rounded once
template <typename T>
void rows_times_expert(const T* Am, const T* B, const int32_t* offsets, int64_t R, int64_t Kd, int64_t N, int64_t E,
                       T* C) {
  using A = acc_t<T>;
  const std::vector<int> ex = row_experts(offsets, R, E);
#pragma omp parallel
  {
    std::vector<A> acc((size_t)N);
#pragma omp for schedule(static)
    for (int64_t r = 0; r < R; ++r) {
      const int64_t e = ex[(size_t)r];
      std::fill(acc.begin(), acc.end(), A(0));
      for (int64_t k = 0; k < Kd; ++k) {
        const A a = ld(Am, r * Kd + k);
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
  using A = acc_t<T>;
  const std::vector<int> ex = row_experts(offsets, R, E);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < R; ++r) {
    const int64_t e = ex[(size_t)r];
    for (int64_t m = 0; m < M; ++m) {
      A acc = 0;
      const int64_t o = (e * M + m) * D;
      for (int64_t d = 0; d < D; ++d) acc += ld(dy, r * D + d) * ld(wd, o + d);
      const A dh = rnd<T>(acc);
      const A g = ld(G, r * M + m), u = ld(U, r * M + m);
      const A sig = sigmoid_a(g);
      const A act = rnd<T>(silu_a(g));
      const A dact = rnd<T>(dh * u);
      st(dG, r * M + m, dact * sig * (A(1) + g * (A(1) - sig)));
      st(dU, r * M + m, dh * act);
    }
  }
}

// dXp = dG . Wg[e]^T + dU . Wu[e]^T over the concatenated reduction (gate half first)
template <typename T>
void gateup_dgrad(const T* dG, const T* dU, const T* wg, const T* wu, const int32_t* offsets, int64_t R, int64_t D,
                  int64_t M, int64_t E, T* dxp) {
  using A = acc_t<T>;
  const std::vector<int> ex = row_experts(offsets, R, E);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < R; ++r) {
    const int64_t e = ex[(size_t)r];
    for (int64_t d = 0; d < D; ++d) {
      A acc = 0;
      const int64_t o = (e * D + d) * M;
      for (int64_t m = 0; m < M; ++m) acc += ld(dG, r * M + m) * ld(wg, o + m);
      for (int64_t m = 0; m < M; ++m) acc += ld(dU, r * M + m) * ld(wu, o + m);
      st(dxp, r * D + d, acc);
    }
  }
}

// C[e] (P x N) = A_e^T . B_e over expert e's rows (A: rows x P, B: rows x N); zero for empty experts
template <typename T>
void expert_wgrad(const T* Am, const T* B, const int32_t* offsets, int64_t P, int64_t N, int64_t E, T* C) {
  using A = acc_t<T>;
#pragma omp parallel
  {
    std::vector<A> acc((size_t)N);
#pragma omp for collapse(2) schedule(static)
    for (int64_t e = 0; e < E; ++e)
      for (int64_t p = 0; p < P; ++p) {
        std::fill(acc.begin(), acc.end(), A(0));
        for (int64_t r = offsets[e]; r < offsets[e + 1]; ++r) {
          const A a = ld(Am, r * P + p);
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
  using A = acc_t<T>;
#pragma omp parallel
  {
    std::vector<int> order;
    std::vector<A> acc((size_t)D);
#pragma omp for schedule(static)
    for (int64_t t = 0; t < Tn; ++t) {
      slots_by_expert(idx, t, K, order);
      std::fill(acc.begin(), acc.end(), A(0));
      for (int k : order) {
        const A w = ld(weights, t * K + k);
        const int64_t p = pos[t * K + k];
        for (int64_t d = 0; d < D; ++d) acc[(size_t)d] += rnd<T>(ld(y, p * D + d) * w);
      }
      for (int64_t d = 0; d < D; ++d) st(out, t * D + d, acc[(size_t)d]);
    }
  }
}

// dL/dweights -> dL/dlogit for one token (router.py:45,49-51)
template <typename A>
inline void gating_bwd(int64_t K, A rho, const A* dw, const A* w, const A* s, A denom, A* dl) {
  A c = 0;
  for (int64_t k = 0; k < K; ++k) c += dw[k] * w[k];
  for (int64_t k = 0; k < K; ++k) dl[k] = (rho * dw[k] - c) / denom * s[k] * (A(1) - s[k]);
}

template <typename T>
void combine_bwd(const T* dout, const T* y, const T* weights, const acc_t<T>* score, const int32_t* pos, int64_t Tn,
                 int64_t D, int64_t K, double rho_in, T* dy, acc_t<T>* dlogit) {
  using A = acc_t<T>;
  const A rho = (A)rho_in;
#pragma omp parallel
  {
    std::vector<A> w((size_t)K), dw((size_t)K), sc((size_t)K), dl((size_t)K);
#pragma omp for schedule(static)
    for (int64_t t = 0; t < Tn; ++t) {
      A sum = 0;
      for (int64_t k = 0; k < K; ++k) {
        w[(size_t)k] = ld(weights, t * K + k);
        const int64_t p = pos[t * K + k];
        A dot = 0;
        for (int64_t d = 0; d < D; ++d) {
          const A g = ld(dout, t * D + d);
          dot += g * ld(y, p * D + d);
          st(dy, p * D + d, g * w[(size_t)k]);
        }
        dw[(size_t)k] = dot;
        sc[(size_t)k] = score[t * K + k];
        sum += sc[(size_t)k];
      }
      gating_bwd<A>(K, rho, dw.data(), w.data(), sc.data(), rnd<T>(sum), dl.data());
      for (int64_t k = 0; k < K; ++k) dlogit[t * K + k] = dl[(size_t)k];
    }
  }
}

template <typename T>
void unpermute_bwd(const T* dxp, const acc_t<T>* dlogit, const int32_t* idx, const int32_t* pos, const T* wt,
                   int64_t Tn, int64_t D, int64_t K, T* dx) {
  using A = acc_t<T>;
#pragma omp parallel
  {
    std::vector<int> order;
    std::vector<A> acc((size_t)D);
#pragma omp for schedule(static)
    for (int64_t t = 0; t < Tn; ++t) {
      slots_by_expert(idx, t, K, order);
      std::fill(acc.begin(), acc.end(), A(0));
      for (int k : order) {
        const int64_t e = idx[t * K + k];
        const A dl = dlogit[t * K + k];
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
void router_wgrad(const T* x, const acc_t<T>* dlogit, const int32_t* idx, int64_t Tn, int64_t D, int64_t E,
                  int64_t K, T* dw) {
  using A = acc_t<T>;
#pragma omp parallel
  {
    std::vector<A> acc((size_t)E);
#pragma omp for schedule(static)
    for (int64_t d = 0; d < D; ++d) {
      std::fill(acc.begin(), acc.end(), A(0));
      for (int64_t t = 0; t < Tn; ++t) {
        const A xv = ld(x, t * D + d);
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
int abacus_moe_abi_version(void) { return 5; }

int64_t abacus_moe_hist_len(int64_t T, int64_t E) { return ((T + kTokBlock - 1) / kTokBlock) * E; }
int64_t abacus_moe_router_ws_bytes(int64_t D, int64_t E, int dtype) { return (int64_t)e_pad(E) * D * elem(dtype); }
int64_t abacus_moe_router_wgrad_ws_bytes(int64_t, int64_t, int64_t, int) { return 0; }
int64_t abacus_moe_down_fwd_ws_bytes(int64_t, int64_t, int64_t, int64_t, int) { return 0; }

int abacus_moe_router_fwd(const void* x_TD, const void* w_DE, const void* bias_E, int64_t T, int64_t D, int64_t E,
                          int64_t K, double route_scale, int dtype, void* logits_TE, void* weights_TK,
                          int64_t* indices_TK_i64, int32_t* idx_TK, void* score_TK, int32_t* hist, void* wt_ws,
                          void*) {
  if (check_route(T, D, E, K, dtype)) return 1;
  HOST_CHECK(wt_ws != nullptr, "router_fwd: router weight workspace is NULL");
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    router_fwd<S>(TP(const S, x_TD), TP(const S, w_DE), TP(const S, bias_E), T, D, E, K, route_scale,
                  TP(S, logits_TE), TP(S, weights_TK), indices_TK_i64, idx_TK, TP(acc_t<S>, score_TK), hist,
                  TP(S, wt_ws));
  });
  return 0;
}

int abacus_moe_route_scan(const int32_t* hist, int64_t T, int64_t E, int64_t K, void* bias_E, double speed,
                          int dtype, int32_t* base, int32_t* counts_E, int32_t* offsets_E1, void*) {
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
  if (bias_E != nullptr)
    with_type(dtype, [&](auto z) {
      using S = decltype(z);
      bias_step<S>(cnt.data(), E, T * K, speed, TP(S, bias_E));
    });
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
                        int64_t E, int64_t K, void* bias_E, double speed, int dtype, int32_t* counts_E,
                        int32_t* offsets_E1, int32_t* pos_TK, int32_t* perm_R, void* x_perm_RD, int32_t* base_ws,
                        void* stream) {
  if (abacus_moe_route_scan(hist, T, E, K, bias_E, speed, dtype, base_ws, counts_E, offsets_E1, stream)) return 1;
  return abacus_moe_permute_gather(x_TD, idx_TK, base_ws, T, D, E, K, dtype, pos_TK, perm_R, x_perm_RD, stream);
}

int abacus_moe_gateup_fwd(const void* x_perm_RD, const void* w_gate_EDM, const void* w_up_EDM,
                          const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M, int64_t E, int dtype,
                          void* gate_RM, void* up_RM, void* h_RM, void*) {
  if (check_gemm(R, D, M, E, dtype)) return 1;
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    gateup_fwd<S>(TP(const S, x_perm_RD), TP(const S, w_gate_EDM), TP(const S, w_up_EDM), offsets_E1, R, D, M, E,
                  TP(S, gate_RM), TP(S, up_RM), TP(S, h_RM));
  });
  return 0;
}

int abacus_moe_down_fwd(const void* h_RM, const void* w_down_EMD, const int32_t* offsets_E1, int64_t R, int64_t M,
                        int64_t D, int64_t E, int dtype, void* y_RD, void*, int64_t, void*) {
  if (check_gemm(R, D, M, E, dtype)) return 1;
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    rows_times_expert<S>(TP(const S, h_RM), TP(const S, w_down_EMD), offsets_E1, R, M, D, E, TP(S, y_RD));
  });
  return 0;
}

int abacus_moe_combine_fwd(const void* y_RD, const void* weights_TK, const int32_t* idx_TK, const int32_t* pos_TK,
                           int64_t T, int64_t D, int64_t K, int dtype, void* out_TD, void*) {
  if (check_route(T, D, K, K, dtype)) return 1;
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    combine_fwd<S>(TP(const S, y_RD), TP(const S, weights_TK), idx_TK, pos_TK, T, D, K, TP(S, out_TD));
  });
  return 0;
}

int abacus_moe_combine_bwd(const void* dout_TD, const void* y_RD, const void* weights_TK, const void* score_TK,
                           const int32_t* pos_TK, int64_t T, int64_t D, int64_t K, double route_scale, int dtype,
                           void* dy_RD, void* dlogit_TK, void*) {
  if (check_route(T, D, K, K, dtype)) return 1;
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    combine_bwd<S>(TP(const S, dout_TD), TP(const S, y_RD), TP(const S, weights_TK), TP(const acc_t<S>, score_TK),
                   pos_TK, T, D, K, route_scale, TP(S, dy_RD), TP(acc_t<S>, dlogit_TK));
  });
  return 0;
}

int abacus_moe_down_bwd_dgrad(const void* dy_RD, const void* w_down_EMD, const void* gate_RM, const void* up_RM,
                              const int32_t* offsets_E1, int64_t R, int64_t M, int64_t D, int64_t E, int dtype,
                              void* dgate_RM, void* dup_RM, void*) {
  if (check_gemm(R, D, M, E, dtype)) return 1;
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    down_dgrad<S>(TP(const S, dy_RD), TP(const S, w_down_EMD), TP(const S, gate_RM), TP(const S, up_RM), offsets_E1,
                  R, M, D, E, TP(S, dgate_RM), TP(S, dup_RM));
  });
  return 0;
}

int abacus_moe_down_bwd_wgrad(const void* h_RM, const void* dy_RD, const int32_t* offsets_E1, int64_t R, int64_t M,
                              int64_t D, int64_t E, int dtype, void* dw_down_EMD, int32_t* tile_ctr, void*) {
  if (check_gemm(R, D, M, E, dtype)) return 1;
  HOST_CHECK(tile_ctr != nullptr, "tile_ctr workspace is NULL");
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    expert_wgrad<S>(TP(const S, h_RM), TP(const S, dy_RD), offsets_E1, M, D, E, TP(S, dw_down_EMD));
  });
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
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    gateup_dgrad<S>(TP(const S, dgate_RM), TP(const S, dup_RM), TP(const S, w_gate_EDM), TP(const S, w_up_EDM),
                    offsets_E1, R, D, M, E, TP(S, dx_perm_RD));
  });
  return 0;
}

int abacus_moe_gateup_bwd_wgrad(const void* x_perm_RD, const void* dgate_RM, const void* dup_RM,
                                const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M, int64_t E, int dtype,
                                void* dw_gate_EDM, void* dw_up_EDM, int32_t* tile_ctr, void*) {
  if (check_gemm(R, D, M, E, dtype)) return 1;
  HOST_CHECK(tile_ctr != nullptr, "tile_ctr workspace is NULL");
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    expert_wgrad<S>(TP(const S, x_perm_RD), TP(const S, dgate_RM), offsets_E1, D, M, E, TP(S, dw_gate_EDM));
    expert_wgrad<S>(TP(const S, x_perm_RD), TP(const S, dup_RM), offsets_E1, D, M, E, TP(S, dw_up_EDM));
  });
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

int abacus_moe_unpermute_bwd(const void* dx_perm_RD, const void* dlogit_TK, const int32_t* idx_TK,
                             const int32_t* pos_TK, const void* w_DE, void* wt_ws, int64_t T, int64_t D, int64_t E,
                             int64_t K, int dtype, void* dx_TD, void*) {
  if (check_route(T, D, E, K, dtype)) return 1;
  HOST_CHECK(wt_ws != nullptr, "unpermute_bwd: router weight workspace is NULL");
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    if (w_DE) transpose_router(TP(const S, w_DE), TP(S, wt_ws), D, E);
    unpermute_bwd<S>(TP(const S, dx_perm_RD), TP(const acc_t<S>, dlogit_TK), idx_TK, pos_TK, TP(const S, wt_ws), T, D,
                     K, TP(S, dx_TD));
  });
  return 0;
}

int abacus_moe_router_wgrad(const void* x_TD, const void* dlogit_TK, const int32_t* idx_TK, int64_t T, int64_t D,
                            int64_t E, int64_t K, int dtype, float*, void* dw_DE, void*) {
  if (check_route(T, D, E, K, dtype)) return 1;
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    router_wgrad<S>(TP(const S, x_TD), TP(const acc_t<S>, dlogit_TK), idx_TK, T, D, E, K, TP(S, dw_DE));
  });
  return 0;
}

int abacus_moe_router_wgrad_noalloc(const void* x_TD, const void* dlogit_TK, const int32_t* idx_TK, int64_t T,
                                    int64_t D, int64_t E, int64_t K, int dtype, void* dw_DE, void* s) {
  return abacus_moe_router_wgrad(x_TD, dlogit_TK, idx_TK, T, D, E, K, dtype, nullptr, dw_DE, s);
}

int abacus_router_gating_bwd(const void* dweights_TK, const void* weights_TK, const void* score_TK, int64_t T,
                             int64_t K, double route_scale, int dtype, void* dlogit_TK, void*) {
  if (check_dtype(dtype)) return 1;
  HOST_CHECK(K >= 1 && T >= 0, "router_gating_bwd: bad sizes T=%lld K=%lld", (long long)T, (long long)K);
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    using A = acc_t<S>;
    const A rho = (A)route_scale;
    const A* score = TP(const A, score_TK);
    A* dlogit = TP(A, dlogit_TK);
#pragma omp parallel
    {
      std::vector<A> dw((size_t)K), w((size_t)K), sc((size_t)K);
#pragma omp for schedule(static)
      for (int64_t t = 0; t < T; ++t) {
        A sum = 0;
        for (int64_t k = 0; k < K; ++k) {
          const int64_t o = t * K + k;
          dw[(size_t)k] = ld(TP(const S, dweights_TK), o);
          w[(size_t)k] = ld(TP(const S, weights_TK), o);
          sc[(size_t)k] = score[o];
          sum += sc[(size_t)k];
        }
        gating_bwd<A>(K, rho, dw.data(), w.data(), sc.data(), rnd<S>(sum), dlogit + t * K);
      }
    }
  });
  return 0;
}

int abacus_router_update_bias(const int64_t* indices, int64_t N, int64_t E, double speed, int dtype, void* bias_E,
                              void*) {
  if (check_dtype(dtype)) return 1;
  HOST_CHECK(E >= 1 && N >= 0, "update_bias: bad sizes N=%lld E=%lld", (long long)N, (long long)E);
  std::vector<int64_t> cnt((size_t)E, 0);
  for (int64_t i = 0; i < N; ++i) {
    HOST_CHECK(indices[i] >= 0 && indices[i] < E, "update_bias: expert index %lld out of range [0, %lld)",
               (long long)indices[i], (long long)E);
    cnt[(size_t)indices[i]] += 1;
  }
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    bias_step<S>(cnt.data(), E, N, speed, TP(S, bias_E));
  });
  return 0;
}

int64_t abacus_moe_load_balancing_ws_bytes(int64_t, int64_t) { return 0; }

// fp32 for every dtype, as load_balancing.py:30 casts the probabilities to
// float; the loss and the probabilities' gradient are rounded to the dtype.
int abacus_moe_load_balancing_fwd(const void* probs_TE, const int64_t* slots_TK, int64_t T, int64_t E, int64_t K,
                                  double coeff_d, int dtype, void*, float* f_E, float* loss_f32, void* loss_out,
                                  int32_t* bad_index, void*) {
  if (check_dtype(dtype)) return 1;
  HOST_CHECK(E >= 1 && T > 0 && K >= 1, "load_balancing_fwd: bad sizes T=%lld E=%lld K=%lld", (long long)T,
             (long long)E, (long long)K);
  const float coeff_e = (float)coeff_d;
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
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    const float tk = (float)(T * K), tn = (float)T;
    float acc = 0.f;
    for (int64_t e = 0; e < E; ++e) {
      float p = 0.f;
      for (int64_t t = 0; t < T; ++t) p += (float)ld(TP(const S, probs_TE), t * E + e);
      const float f = (float)n[(size_t)e] / tk;
      f_E[e] = f;
      acc += f * (p / tn);
    }
    const float loss = acc * coeff_e;
    *loss_f32 = loss;
    st(TP(S, loss_out), 0, (acc_t<S>)loss);
  });
  *bad_index = bad;
  return 0;
}

int abacus_moe_load_balancing_bwd(const void* grad_loss, const float* f_E, int64_t T, int64_t E, double coeff_d,
                                  int dtype, void* grad_probs_TE, void*) {
  if (check_dtype(dtype)) return 1;
  const float coeff_e = (float)coeff_d;
  with_type(dtype, [&](auto z) {
    using S = decltype(z);
    const float g = (float)ld(TP(const S, grad_loss), 0);
    const float gc = g * coeff_e, tn = (float)T;
    for (int64_t i = 0; i < T * E; ++i) st(TP(S, grad_probs_TE), i, (acc_t<S>)((gc * f_E[i % E]) / tn));
  });
  return 0;
}

}  // extern "C"
