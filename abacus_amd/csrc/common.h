// Shared device/host helpers for the MI355X (gfx950) MoE kernels.
//
// Storage types: fp32 is `float`; bf16 is carried as its raw 16-bit pattern
// (`uint16_t`) so that every rounding step is explicit and reproducible.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "abacus_moe.h"

namespace abacus {

enum DType : int { kF32 = 0, kBF16 = 1 };

// ---------------------------------------------------------------------------
// Scalar conversions.  bf16 rounding is round-to-nearest-even on the fp32 bit
// pattern (the IEEE default, and what torch uses for fp32 -> bf16 casts).
// ---------------------------------------------------------------------------
__host__ __device__ inline uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

__host__ __device__ inline float bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

__host__ __device__ inline uint16_t f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Round an fp32 value to the storage precision of T and return it as fp32.
template <typename T> __host__ __device__ inline float round_to(float v);
template <> __host__ __device__ inline float round_to<float>(float v) { return v; }
template <> __host__ __device__ inline float round_to<uint16_t>(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// Two floats to packed bf16 in one v_cvt_pk_bf16_f32 (gfx950): round to
// nearest even, NaN made quiet -- bit-identical to f32_to_bf16 for every
// input; lo_bf16 / hi_bf16 widen the halves back to fp32.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ inline uint32_t pack_bf16x2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ inline float lo_bf16(uint32_t w) { return bits_f32(w << 16); }
__device__ inline float hi_bf16(uint32_t w) { return bits_f32(w & 0xffff0000u); }

// global_load_lds_dwordx4 issued through inline asm: the compiler does not
// model it, so it neither inserts vmcnt(0) before LDS reads of other stages
// nor before barriers; completion is tracked explicitly with wait_vmcnt<N>().
// M0 holds the (wave-uniform) LDS destination; lane l's 16 bytes land at
// M0 + 16 l.
// dma16_to takes the destination as a wave-uniform LDS byte address, so a
// caller that converts its LDS base once does the per-DMA address arithmetic
// in 32-bit scalar registers (a generic pointer costs a 64-bit add and a null
// check per conversion).
__device__ inline uint32_t lds_addr32(const void* lds_ptr) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)lds_ptr;
}
__device__ inline void dma16_to(const void* src, uint32_t lds_addr) {
  // M0 is reserved by the compiler: save and restore it around the DMA.
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(lds_addr)
      : "memory");
}
__device__ inline void dma16(const void* src, char* lds_dst) {
  dma16_to(src, __builtin_amdgcn_readfirstlane(lds_addr32(lds_dst)));
}

// Wait until at most N DMA instructions of this thread are outstanding
// (vmcnt), without waiting on LDS or export counters.
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | (((N >> 4) & 3) << 14));
}


template <typename T> __host__ __device__ inline float to_f32(T v);
template <> __host__ __device__ inline float to_f32<float>(float v) { return v; }
template <> __host__ __device__ inline float to_f32<uint16_t>(uint16_t v) { return bf16_to_f32(v); }

template <typename T> __host__ __device__ inline T from_f32(float v);
template <> __host__ __device__ inline float from_f32<float>(float v) { return v; }
template <> __host__ __device__ inline uint16_t from_f32<uint16_t>(float v) { return f32_to_bf16(v); }

// Logistic sigmoid evaluated in fp64 and rounded once to fp32: correctly
// rounded for every finite fp32 input (the fp64 result carries ~2^-52 relative
// error, far inside half an fp32 ulp except on a measure-zero set).
__device__ inline float sigmoid_f32_cr(float x) {
  double d = (double)x;
  return (float)(1.0 / (1.0 + exp(-d)));
}

// SiLU in fp32: x * sigmoid(x) written as x / (1 + e^-x).
__device__ inline float silu_f32(float x) { return x / (1.0f + expf(-x)); }
__device__ inline float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---------------------------------------------------------------------------
// 16-byte vectors: 8 bf16 or 4 fp32 per lane.
// ---------------------------------------------------------------------------
struct alignas(16) Vec16 {
  uint32_t w[4];
};

template <typename T> struct VecTraits;
template <> struct VecTraits<float> {
  static constexpr int kN = 4;  // elements per 16 bytes
  __device__ static inline float get(const Vec16& v, int i) { return bits_f32(v.w[i]); }
  __device__ static inline void set(Vec16& v, int i, float f) { v.w[i] = f32_bits(f); }
};
template <> struct VecTraits<uint16_t> {
  static constexpr int kN = 8;
  __device__ static inline float get(const Vec16& v, int i) {
    uint32_t w = v.w[i >> 1];
    return bf16_to_f32((uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu)));
  }
  __device__ static inline void set(Vec16& v, int i, float f) {
    uint32_t h = f32_to_bf16(f);
    uint32_t& w = v.w[i >> 1];
    w = (i & 1) ? ((w & 0x0000ffffu) | (h << 16)) : ((w & 0xffff0000u) | h);
  }
};

__device__ inline Vec16 ld16(const void* p) { return *reinterpret_cast<const Vec16*>(p); }
__device__ inline void st16(void* p, const Vec16& v) { *reinterpret_cast<Vec16*>(p) = v; }
// Nontemporal 16-byte loads and stores, for data a pass touches once: they keep
// it out of the caches' working set.
typedef unsigned int u32x4_nt_t __attribute__((ext_vector_type(4)));
__device__ inline Vec16 ld16_stream(const void* p) {
  const u32x4_nt_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt_t*>(p));
  Vec16 r;
  r.w[0] = v.x;
  r.w[1] = v.y;
  r.w[2] = v.z;
  r.w[3] = v.w;
  return r;
}
__device__ inline void st16_stream(void* p, const Vec16& x) {
  u32x4_nt_t v;
  v.x = x.w[0];
  v.y = x.w[1];
  v.z = x.w[2];
  v.w = x.w[3];
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_nt_t*>(p));
}
__device__ inline Vec16 zero16() {
  Vec16 v;
  v.w[0] = v.w[1] = v.w[2] = v.w[3] = 0u;
  return v;
}

// ---------------------------------------------------------------------------
// Wave-level helpers (wave64).
// ---------------------------------------------------------------------------
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace abacus

// ---------------------------------------------------------------------------
// Error plumbing for the C ABI: every entry point returns 0 on success or a
// nonzero code; the message for the last failure on this thread is available
// from abacus_moe_last_error().
// ---------------------------------------------------------------------------
namespace abacus {
void set_error(const char* fmt, ...);
}

#define ABACUS_CHECK_ARG(cond, ...)      \
  do {                                   \
    if (!(cond)) {                       \
      ::abacus::set_error(__VA_ARGS__);  \
      return 1;                          \
    }                                    \
  } while (0)

#define ABACUS_CHECK_LAUNCH(name)                                                   \
  do {                                                                              \
    hipError_t _e = hipGetLastError();                                              \
    if (_e != hipSuccess) {                                                         \
      ::abacus::set_error("%s: launch failed: %s", name, hipGetErrorString(_e));    \
      return 2;                                                                     \
    }                                                                               \
  } while (0)
