// RMSNorm for the MoE decoder around the MoE layer, forward and backward.
//
// Reference: abacus/norm.py:26-31, y = gamma * x / sqrt(mean(x^2) + eps)
// over the last dimension, evaluated there op by op in the activation dtype
// (about five kernels forward and ten backward).  Here one pass reads each
// row once and writes it once, in fp32 with one rounding of each output:
//   forward   y = gamma * x * r,  r = 1 / sqrt(sum(x^2) / D + eps)   (r kept per row)
//   backward  dx = r * gamma * dy - x * r^3 * sum(gamma * dy * x) / D
//             dgamma = sum over rows of dy * x * r
// dgamma is reduced deterministically: each block adds its rows in a fixed
// order into one partial row, and a second kernel adds the block partials
// in block order.
//
// Layout: rows of D elements, contiguous.  A row is spread over LPR lanes of
// a wave (LPR a power of two dividing the row's 16-byte vectors), each lane
// holding VPL vectors; a wave covers 64 / LPR rows at a time.
//
// The attention's q and k norms can also apply the rotary embedding that
// follows them (rope.py:36-46): for the (b, l, h) rows of a (B, L, H, K)
// tensor, out = u * cos[l] + rotate_half(u) * sin[l] with u the normed row,
// rotate_half(u) = (-u2, u1).  The backward first takes the transposed
// rotation, du = g * cos + (g2 * sin2, -g1 * sin1) with g = dout, then the
// norm's backward.  A row then sits on LPR lanes holding one vector each, so
// element c's partner c +- K/2 is on lane li ^ (LPR / 2).
#include <algorithm>

#include "common.h"

namespace abacus {

namespace {

// Waves per block: 16, or 8 where the backward's per-wave dgamma sums (64
// lanes x elements per lane, fp32) would pass 128 KB of LDS.  Many waves per
// CU keep enough row loads in flight to cover the memory latency.
__host__ __device__ constexpr int norm_waves(int elems_per_lane) { return elems_per_lane <= 32 ? 16 : 8; }
constexpr int kNormMaxBlocks = 1024;   // forward grid cap
constexpr int kNormBwdBlocks = 256;    // backward grid cap (one dgamma partial row each)

template <typename T>
__device__ inline void unpack(const Vec16& v, float* f) {
#pragma unroll
  for (int i = 0; i < VecTraits<T>::kN; ++i) f[i] = VecTraits<T>::get(v, i);
}

template <typename T>
__device__ inline Vec16 pack(const float* f) {
  Vec16 v;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v.w[i] = (uint32_t)f32_to_bf16(f[2 * i]) | ((uint32_t)f32_to_bf16(f[2 * i + 1]) << 16);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v.w[i] = f32_bits(f[i]);
  }
  return v;
}

// Sum over the lpr lanes of one row (lanes li = lane % lpr of a group).
__device__ inline float row_sum(float v, int lpr) {
  for (int off = lpr >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <typename T, int VPL, bool ROPE>
__global__ __launch_bounds__(norm_waves(VPL * VecTraits<T>::kN) * 64) void rmsnorm_fwd_kernel(const T* __restrict__ x,
                                                                      const T* __restrict__ gamma, int64_t rows,
                                                                      int D, int lpr, float eps, T* __restrict__ y,
                                                                      float* __restrict__ rstd,
                                                                      const T* __restrict__ cosv,
                                                                      const T* __restrict__ sinv, int L, int H) {
  static_assert(!ROPE || VPL == 1, "the rotary pairs sit on partner lanes");
  constexpr int EPV = VecTraits<T>::kN;
  constexpr int W = norm_waves(VPL * EPV);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rpw = 64 / lpr, sub = lane / lpr, li = lane % lpr;
  const int64_t groups = (rows + rpw - 1) / rpw;
  Vec16 gv[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) gv[v] = ld16(gamma + (li + v * lpr) * EPV);
  for (int64_t g = (int64_t)blockIdx.x * W + wave; g < groups; g += (int64_t)gridDim.x * W) {
    const int64_t r = g * rpw + sub;
    const bool act = r < rows;
    Vec16 xv[VPL];
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      xv[v] = act ? ld16(x + r * D + (li + v * lpr) * EPV) : zero16();
      float f[EPV];
      unpack<T>(xv[v], f);
#pragma unroll
      for (int i = 0; i < EPV; ++i) ss += f[i] * f[i];
    }
    ss = row_sum(ss, lpr);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
    if (ROPE) {
      float f[EPV], gf[EPV], pf[EPV], cf[EPV], sf[EPV];
      unpack<T>(xv[0], f);
      unpack<T>(gv[0], gf);
#pragma unroll
      for (int i = 0; i < EPV; ++i) f[i] = gf[i] * f[i] * inv;
#pragma unroll
      for (int i = 0; i < EPV; ++i) pf[i] = __shfl_xor(f[i], lpr >> 1, 64);
      if (act) {
        const int64_t l = (r / H) % L;
        unpack<T>(ld16(cosv + l * D + li * EPV), cf);
        unpack<T>(ld16(sinv + l * D + li * EPV), sf);
        const float sgn = li < (lpr >> 1) ? -1.0f : 1.0f;  // rotate_half: (-u2, u1)
#pragma unroll
        for (int i = 0; i < EPV; ++i) f[i] = f[i] * cf[i] + sgn * pf[i] * sf[i];
        st16(y + r * D + li * EPV, pack<T>(f));
        if (li == 0) rstd[r] = inv;
      }
    } else if (act) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        float f[EPV], gf[EPV];
        unpack<T>(xv[v], f);
        unpack<T>(gv[v], gf);
#pragma unroll
        for (int i = 0; i < EPV; ++i) f[i] = gf[i] * f[i] * inv;
        st16(y + r * D + (li + v * lpr) * EPV, pack<T>(f));
      }
      if (li == 0) rstd[r] = inv;
    }
  }
}

template <typename T, int VPL, bool ROPE>
__global__ __launch_bounds__(norm_waves(VPL * VecTraits<T>::kN) * 64) void rmsnorm_bwd_kernel(const T* __restrict__ dy,
                                                                      const T* __restrict__ x,
                                                                      const T* __restrict__ gamma,
                                                                      const float* __restrict__ rstd, int64_t rows,
                                                                      int D, int lpr, T* __restrict__ dx,
                                                                      float* __restrict__ partial,
                                                                      const T* __restrict__ cosv,
                                                                      const T* __restrict__ sinv, int L, int H) {
  static_assert(!ROPE || VPL == 1, "the rotary pairs sit on partner lanes");
  constexpr int EPV = VecTraits<T>::kN;
  constexpr int NE = VPL * EPV;  // elements per lane
  constexpr int W = norm_waves(NE);
  __shared__ float red_s[W][64 * NE];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rpw = 64 / lpr, sub = lane / lpr, li = lane % lpr;
  const int64_t groups = (rows + rpw - 1) / rpw;
  float gf[NE], dg[NE];
#pragma unroll
  for (int v = 0; v < VPL; ++v) unpack<T>(ld16(gamma + (li + v * lpr) * EPV), gf + v * EPV);
#pragma unroll
  for (int i = 0; i < NE; ++i) dg[i] = 0.f;
  for (int64_t g = (int64_t)blockIdx.x * W + wave; g < groups; g += (int64_t)gridDim.x * W) {
    const int64_t r = g * rpw + sub;
    const bool act = r < rows;
    float xf[NE], df[NE];
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int64_t o = r * D + (li + v * lpr) * EPV;
      unpack<T>(act ? ld16(x + o) : zero16(), xf + v * EPV);
      unpack<T>(act ? ld16(dy + o) : zero16(), df + v * EPV);
    }
    const float inv = act ? rstd[r] : 0.f;
    if (ROPE) {
      // gradient of the normed row through the rotation
      float cf[EPV], sf[EPV], wv[EPV], pw[EPV];
      const int64_t l = act ? (r / H) % L : 0;
      unpack<T>(act ? ld16(cosv + l * D + li * EPV) : zero16(), cf);
      unpack<T>(act ? ld16(sinv + l * D + li * EPV) : zero16(), sf);
#pragma unroll
      for (int i = 0; i < EPV; ++i) wv[i] = df[i] * sf[i];
#pragma unroll
      for (int i = 0; i < EPV; ++i) pw[i] = __shfl_xor(wv[i], lpr >> 1, 64);
      const float sgn = li < (lpr >> 1) ? 1.0f : -1.0f;  // transposed rotate_half: (w2, -w1)
#pragma unroll
      for (int i = 0; i < EPV; ++i) df[i] = df[i] * cf[i] + sgn * pw[i];
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NE; ++i) s += gf[i] * df[i] * xf[i];
    s = row_sum(s, lpr);
    const float c = inv * inv * inv * s / (float)D;
#pragma unroll
    for (int i = 0; i < NE; ++i) dg[i] += df[i] * xf[i] * inv;
    if (act) {
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        float o[EPV];
#pragma unroll
        for (int i = 0; i < EPV; ++i) o[i] = inv * gf[v * EPV + i] * df[v * EPV + i] - xf[v * EPV + i] * c;
        st16(dx + r * D + (li + v * lpr) * EPV, pack<T>(o));
      }
    }
  }
  // dgamma: the rows' sums of one lane index li over the wave's row groups
  // (sub-rows added in sub order), then over the waves in wave order.
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    float v = dg[i];
    for (int off = lpr; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
    dg[i] = v;
  }
  if (sub == 0) {
#pragma unroll
    for (int i = 0; i < NE; ++i) red_s[wave][li * NE + i] = dg[i];
  }
  __syncthreads();
  // the block's partial row, element order (vector li + v lpr, element e)
  for (int col = threadIdx.x; col < D; col += blockDim.x) {
    const int vec = col / EPV, e = col % EPV;
    const int l = vec % lpr, v = vec / lpr;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) sum += red_s[w][l * NE + v * EPV + e];
    partial[(int64_t)blockIdx.x * D + col] = sum;
  }
}

// dgamma[d] = the sum of the block partials in a fixed order: 64 columns per
// block; wave w of 16 loads partial rows 16w .. 16w+15 of each 256 at once
// (the rows come from other XCDs' writes, one memory round trip away) and
// adds them pairwise; the 16 wave sums are added in wave order.
constexpr int kDgammaWaves = 16;
template <typename T>
__global__ __launch_bounds__(kDgammaWaves * 64) void rmsnorm_dgamma_kernel(const float* __restrict__ partial,
                                                                           int nblocks, int D,
                                                                           T* __restrict__ dgamma) {
  __shared__ float s_part[kDgammaWaves][64];
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + l;
  float total = 0.f;
  for (int r0 = 0; r0 < nblocks; r0 += kDgammaWaves * 16) {
    float a[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int b = r0 + 16 * w + u;
      a[u] = col < D && b < nblocks ? partial[(int64_t)b * D + col] : 0.f;
    }
#pragma unroll
    for (int h = 8; h >= 1; h >>= 1)
#pragma unroll
      for (int u = 0; u < h; ++u) a[u] += a[u + h];
    s_part[w][l] = a[0];
    __syncthreads();
    if (w == 0) {
      float t = 0.f;
#pragma unroll
      for (int v = 0; v < kDgammaWaves; ++v) t += s_part[v][l];
      total += t;
    }
    __syncthreads();
  }
  if (w == 0 && col < D) dgamma[col] = from_f32<T>(total);
}

// Lanes per row: the largest power of two up to 64 dividing the row's vectors.
int lanes_per_row(int64_t nvec) {
  int lpr = 64;
  while (lpr > 1 && nvec % lpr != 0) lpr >>= 1;
  return lpr;
}

int check_norm(int64_t rows, int64_t D, int dtype, int* lpr, int* vpl) {
  ABACUS_CHECK_ARG(dtype == kF32 || dtype == kBF16, "unsupported dtype code %d (0 = fp32, 1 = bf16)", dtype);
  const int epv = dtype == kBF16 ? 8 : 4;
  ABACUS_CHECK_ARG(rows >= 0, "rows %lld must be >= 0", (long long)rows);
  ABACUS_CHECK_ARG(D >= 1 && D % epv == 0, "dim %lld must be a positive multiple of %d", (long long)D, epv);
  const int64_t nvec = D / epv;
  *lpr = lanes_per_row(nvec);
  const int64_t v = nvec / *lpr;
  ABACUS_CHECK_ARG(v <= 8, "dim %lld too large for the fused RMSNorm (at most %d)", (long long)D, 64 * 8 * epv);
  *vpl = v <= 1 ? 1 : v <= 2 ? 2 : v <= 4 ? 4 : 8;
  ABACUS_CHECK_ARG(*vpl == v, "dim %lld: the row's 16-byte vectors must split evenly over its lanes", (long long)D);
  return 0;
}

int64_t norm_groups(int64_t rows, int lpr) { return (rows + 64 / lpr - 1) / (64 / lpr); }

}  // namespace

}  // namespace abacus

using namespace abacus;

namespace {

int norm_fwd(const void* x, const void* gamma, int64_t rows, int64_t D, float eps, int dtype, void* y, float* rstd,
             const void* cosv, const void* sinv, int64_t L, int64_t H, bool rope, void* stream) {
  int lpr, vpl;
  if (check_norm(rows, D, dtype, &lpr, &vpl)) return 1;
  if (rope) {
    ABACUS_CHECK_ARG(vpl == 1 && lpr >= 2 && L >= 1 && H >= 1,
                     "rmsnorm_rope: head_dim %lld must be 2..64 16-byte vectors, a power of two", (long long)D);
  }
  if (rows == 0) return 0;
  const int64_t groups = norm_groups(rows, lpr);
  const int W = norm_waves(vpl * (dtype == kBF16 ? 8 : 4));
  const unsigned grid = (unsigned)std::min<int64_t>(kNormMaxBlocks, (groups + W - 1) / W);
  hipStream_t s = (hipStream_t)stream;
#define ABACUS_NORM_FWD(TT, V, R)                                                                                 \
  hipLaunchKernelGGL((rmsnorm_fwd_kernel<TT, V, R>), dim3(grid), dim3(W * 64), 0, s, (const TT*)x,                \
                     (const TT*)gamma, rows, (int)D, lpr, eps, (TT*)y, rstd, (const TT*)cosv, (const TT*)sinv,   \
                     (int)L, (int)H)
  if (dtype == kBF16) {
    if (rope) ABACUS_NORM_FWD(uint16_t, 1, true);
    else if (vpl == 1) ABACUS_NORM_FWD(uint16_t, 1, false);
    else if (vpl == 2) ABACUS_NORM_FWD(uint16_t, 2, false);
    else if (vpl == 4) ABACUS_NORM_FWD(uint16_t, 4, false);
    else ABACUS_NORM_FWD(uint16_t, 8, false);
  } else {
    if (rope) ABACUS_NORM_FWD(float, 1, true);
    else if (vpl == 1) ABACUS_NORM_FWD(float, 1, false);
    else if (vpl == 2) ABACUS_NORM_FWD(float, 2, false);
    else if (vpl == 4) ABACUS_NORM_FWD(float, 4, false);
    else ABACUS_NORM_FWD(float, 8, false);
  }
#undef ABACUS_NORM_FWD
  ABACUS_CHECK_LAUNCH("rmsnorm_fwd");
  return 0;
}

int norm_bwd(const void* dy, const void* x, const void* gamma, const float* rstd, int64_t rows, int64_t D, int dtype,
             void* dx, void* dgamma, float* ws, int64_t ws_bytes, const void* cosv, const void* sinv, int64_t L,
             int64_t H, bool rope, void* stream) {
  int lpr, vpl;
  if (check_norm(rows, D, dtype, &lpr, &vpl)) return 1;
  if (rope) {
    ABACUS_CHECK_ARG(vpl == 1 && lpr >= 2 && L >= 1 && H >= 1,
                     "rmsnorm_rope: head_dim %lld must be 2..64 16-byte vectors, a power of two", (long long)D);
  }
  hipStream_t s = (hipStream_t)stream;
  const int64_t groups = norm_groups(rows, lpr);
  const int W = norm_waves(vpl * (dtype == kBF16 ? 8 : 4));
  const int nb = (int)std::max<int64_t>(1, std::min<int64_t>(kNormBwdBlocks, (groups + W - 1) / W));
  ABACUS_CHECK_ARG(rows == 0 || ws_bytes >= (int64_t)nb * D * 4, "rmsnorm_bwd: workspace of %lld bytes, need %lld",
                   (long long)ws_bytes, (long long)nb * D * 4);
  if (rows == 0) {
    // no rows: dgamma is zero
    if (dtype == kBF16)
      hipLaunchKernelGGL(rmsnorm_dgamma_kernel<uint16_t>, dim3((unsigned)((D + 63) / 64)), dim3(kDgammaWaves * 64), 0, s, ws, 0,
                         (int)D, (uint16_t*)dgamma);
    else
      hipLaunchKernelGGL(rmsnorm_dgamma_kernel<float>, dim3((unsigned)((D + 63) / 64)), dim3(kDgammaWaves * 64), 0, s, ws, 0,
                         (int)D, (float*)dgamma);
    ABACUS_CHECK_LAUNCH("rmsnorm_dgamma");
    return 0;
  }
#define ABACUS_NORM_BWD(TT, V, R)                                                                                  \
  hipLaunchKernelGGL((rmsnorm_bwd_kernel<TT, V, R>), dim3(nb), dim3(W * 64), 0, s, (const TT*)dy,                  \
                     (const TT*)x, (const TT*)gamma, rstd, rows, (int)D, lpr, (TT*)dx, ws, (const TT*)cosv,        \
                     (const TT*)sinv, (int)L, (int)H)
  if (dtype == kBF16) {
    if (rope) ABACUS_NORM_BWD(uint16_t, 1, true);
    else if (vpl == 1) ABACUS_NORM_BWD(uint16_t, 1, false);
    else if (vpl == 2) ABACUS_NORM_BWD(uint16_t, 2, false);
    else if (vpl == 4) ABACUS_NORM_BWD(uint16_t, 4, false);
    else ABACUS_NORM_BWD(uint16_t, 8, false);
  } else {
    if (rope) ABACUS_NORM_BWD(float, 1, true);
    else if (vpl == 1) ABACUS_NORM_BWD(float, 1, false);
    else if (vpl == 2) ABACUS_NORM_BWD(float, 2, false);
    else if (vpl == 4) ABACUS_NORM_BWD(float, 4, false);
    else ABACUS_NORM_BWD(float, 8, false);
  }
#undef ABACUS_NORM_BWD
  ABACUS_CHECK_LAUNCH("rmsnorm_bwd");
  if (dtype == kBF16)
    hipLaunchKernelGGL(rmsnorm_dgamma_kernel<uint16_t>, dim3((unsigned)((D + 63) / 64)), dim3(kDgammaWaves * 64), 0, s, ws, nb,
                       (int)D, (uint16_t*)dgamma);
  else
    hipLaunchKernelGGL(rmsnorm_dgamma_kernel<float>, dim3((unsigned)((D + 63) / 64)), dim3(kDgammaWaves * 64), 0, s, ws, nb,
                       (int)D, (float*)dgamma);
  ABACUS_CHECK_LAUNCH("rmsnorm_dgamma");
  return 0;
}

}  // namespace

extern "C" {

int64_t abacus_rmsnorm_bwd_ws_bytes(int64_t rows, int64_t D) {
  if (rows <= 0 || D <= 0) return 0;
  return (int64_t)kNormBwdBlocks * D * 4;
}

int abacus_rmsnorm_fwd(const void* x, const void* gamma, int64_t rows, int64_t D, float eps, int dtype, void* y,
                       float* rstd, void* stream) {
  return norm_fwd(x, gamma, rows, D, eps, dtype, y, rstd, nullptr, nullptr, 1, 1, false, stream);
}

int abacus_rmsnorm_bwd(const void* dy, const void* x, const void* gamma, const float* rstd, int64_t rows, int64_t D,
                       int dtype, void* dx, void* dgamma, float* ws, int64_t ws_bytes, void* stream) {
  return norm_bwd(dy, x, gamma, rstd, rows, D, dtype, dx, dgamma, ws, ws_bytes, nullptr, nullptr, 1, 1, false, stream);
}

int abacus_rmsnorm_rope_fwd(const void* x, const void* gamma, const void* cos_LK, const void* sin_LK, int64_t rows,
                            int64_t L, int64_t H, int64_t K, float eps, int dtype, void* y, float* rstd,
                            void* stream) {
  return norm_fwd(x, gamma, rows, K, eps, dtype, y, rstd, cos_LK, sin_LK, L, H, true, stream);
}

int abacus_rmsnorm_rope_bwd(const void* dy, const void* x, const void* gamma, const float* rstd, const void* cos_LK,
                            const void* sin_LK, int64_t rows, int64_t L, int64_t H, int64_t K, int dtype, void* dx,
                            void* dgamma, float* ws, int64_t ws_bytes, void* stream) {
  return norm_bwd(dy, x, gamma, rstd, rows, K, dtype, dx, dgamma, ws, ws_bytes, cos_LK, sin_LK, L, H, true, stream);
}

}  // extern "C"
